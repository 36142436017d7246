// Split-K causal GQA attention over a KV cache, for decode and short chunks.
//
// Semantics: reference MSL attention_f32_batched_f16_kv / attention_f32_batched
// (mps_backend.mm:2879-3008): query token t at position start+t attends cache
// keys 0..position of its KV head (kv_head = head / group), scale 1/sqrt(D),
// f32 query times f16 (or f32) cache, fp32 accumulation, out = o/den (0 if
// den == 0).  The optional gate applies the full-attention output gate
// out *= sigmoid(G) (qwen35_runtime.cpp:3347-3355) in the epilogue.
//
// Design (gfx950, wave64):
//  * A workgroup of 16 waves (1024 threads) owns (token, kv_head, key split) and
//    serves all G query heads of the GQA group, so each K/V row is fetched once
//    for G heads.  Splits are sized to put about one workgroup on every CU: the
//    whole KV stream is requested by the first load of each thread, which is
//    what saturates HBM for the few MB of one decode step.
//  * A key row (D elements) is spread over R = D / E lanes, each holding one
//    16-byte chunk (E elements); a wave takes 64 / R keys per round (2 for the
//    f16 D=256 cache), the workgroup 16 * 64 / R.  Rows are read through buffer
//    resources bounded to the split, so lanes past its end get zeros from the
//    range check without a memory access, every round issues the same loads
//    with no branch, and the next two rounds are always in flight.
//  * The query, pre-scaled into the log2 domain, sits in registers (a lane's G
//    heads x E dims) when that is at most 32 floats, else in LDS.  Dot products
//    reduce over a row's R lanes with DPP and the gfx950 permlane swaps; each
//    wave runs its own online softmax against a wave-uniform reference max that
//    moves only when a score exceeds it by 2^8 (lazy rescale), and stops after
//    its last round that holds a key.
//  * Waves merge (m, l, o[G][D]) through LDS with a log-sum-exp rescale.
//    Unsplit, the workgroup writes the (gated) output directly.  Split, it
//    stores its partial and a second, wide pass merges them: one workgroup per
//    16-dim slice of each query head issues all of its partial loads at once,
//    reduces with lane shuffles and LDS, divides by the denominator and applies
//    the gate.  The kernel boundary orders the partial stores before the merge,
//    which needs no atomics or cross-workgroup fences.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "context_internal.hpp"
#include "attention_decode_internal.hpp"
#include "device_common.hpp"

namespace kraken {
namespace {

using namespace decode;

constexpr int kMaxSplits = 256;  // merge pass: 64 subsets x 4 loads per thread

template <typename KV>
struct KvTraits;
template <>
struct KvTraits<half_t> {
  static constexpr int kPerChunk = 8;  // elements per 16-byte chunk
  __device__ static void to_float(const u32x4_t& raw, float* out) {
    const half2_t* h = reinterpret_cast<const half2_t*>(&raw);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = static_cast<float>(h[i].x);
      out[2 * i + 1] = static_cast<float>(h[i].y);
    }
  }
};
template <>
struct KvTraits<float> {
  static constexpr int kPerChunk = 4;
  __device__ static void to_float(const u32x4_t& raw, float* out) {
    out[0] = __uint_as_float(raw.x);
    out[1] = __uint_as_float(raw.y);
    out[2] = __uint_as_float(raw.z);
    out[3] = __uint_as_float(raw.w);
  }
};

// Lane geometry of a key row: a lane holds one 16-byte chunk of E elements
// (EL = E), R = D/E lanes span a row, a wave takes KW = 64/R keys per round, a
// workgroup of W = 16 waves takes KPR = W*KW.  (Two chunks per lane in 8-wave
// workgroups, and a four-deep prefetch ring, both measured slower on the C1
// and C4 shapes once the ragged grid keeps every XCD busy.)
template <int D, typename KV>
struct RowShape {
  static constexpr int E = KvTraits<KV>::kPerChunk;
  static constexpr int EL = E;
  static constexpr int R = D / EL;
  static constexpr int KW = 64 / R;
  static constexpr int W = 16;
  static constexpr int KPR = W * KW;
  static_assert(R >= 8 && R <= 64 && 64 % R == 0, "row must span 8..64 lanes");
};

// Sum over the R lanes of a row (aligned lane group); result in all of them.
template <int R>
__device__ __forceinline__ float row_sum(float x) {
  x = reduce8_sum(x);
  if constexpr (R >= 16) {
    x += dpp<kDppRowMirror>(x);
  }
  if constexpr (R >= 32) {
    x = xor16_sum(x);
  }
  if constexpr (R >= 64) {
    x = xor32_sum(x);
  }
  return x;
}

// Max over the KW key slots of a wave of a value that is uniform within each
// row's lane group; result wave-uniform.
template <int R>
__device__ __forceinline__ float slots_max(float x) {
  if constexpr (R <= 8) {
    x = fmaxf(x, dpp<kDppRowRor8>(x));
  }
  if constexpr (R <= 16) {
    x = xor16_max(x);
  }
  if constexpr (R <= 32) {
    x = xor32_max(x);
  }
  return x;
}

// Lane-wise sum over the KW key slots (lanes sharing lane % R).
template <int R>
__device__ __forceinline__ float slots_sum(float x) {
  if constexpr (R <= 8) {
    x += dpp<kDppRowRor8>(x);
  }
  if constexpr (R <= 16) {
    x = xor16_sum(x);
  }
  if constexpr (R <= 32) {
    x = xor32_sum(x);
  }
  return x;
}

__device__ __forceinline__ float uniform_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(uint32_t, x)));
}

template <int D, int G, typename KV>
__global__ __launch_bounds__((64 * RowShape<D, KV>::W)) void attention_decode_kernel(
  DecodeParams p) {
  constexpr int C = 1;  // 16-byte chunks per lane
  constexpr int P = 2;  // rounds in flight (ring depth)
  using T = KvTraits<KV>;
  using S = RowShape<D, KV>;
  constexpr int E = S::E;
  constexpr int EL = S::EL;
  constexpr int R = S::R;
  constexpr int KW = S::KW;
  constexpr int KPR = S::KPR;
  constexpr int kWaves = S::W;
  constexpr int kThreads = 64 * kWaves;
  // A lane's query slice (G heads x its EL dims) lives in registers when it
  // fits beside the accumulators; otherwise in LDS, read by all lanes that hold
  // the same dims.
  constexpr bool kQRegs = G * EL <= (C == 2 ? 64 : 32);
  constexpr int kQVec = G * D / 4;
  constexpr int kOutPerThread = (G * D + kThreads - 1) / kThreads;
  static_assert(kQVec <= kThreads, "query staging takes one float4 per thread");

  // LDS query: G*D floats plus one float4 of padding that threads past the end
  // write into, so the store needs no branch (a branch would let the compiler
  // sink the query load below the K/V loads and wait for all of them).
  __shared__ __attribute__((aligned(16))) float s_q[kQRegs ? 4 : G * D + 4];
  __shared__ float s_o[kWaves][G * D];
  __shared__ float s_m[kWaves][G];
  __shared__ float s_l[kWaves][G];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kslot = lane / R;
  const int c = lane % R;
  uint32_t split = blockIdx.x;
  uint32_t kvh = blockIdx.y;
  uint32_t token = blockIdx.z;
  const bool ragged = p.seq_positions != nullptr;
  if (ragged) {
    const uint2 item = p.work_items[blockIdx.x];
    if (item.x == 0xffffffffu) {
      return;  // past the last work item
    }
    token = item.x;
    kvh = item.y >> 16;
    split = item.y & 0xffffu;
  }
  const uint32_t n_keys = token_keys(p.seq_positions, p.start_position, token);
  const uint32_t key_begin = split * p.keys_per_split;
  if (key_begin >= n_keys) {
    return;  // empty split (whole workgroup): the merge reads only this token's splits
  }
  const uint32_t key_end = min(n_keys, key_begin + p.keys_per_split);
  const uint32_t count = key_end - key_begin;

  const size_t row_stride = (size_t)p.kv_heads * D;
  const uint64_t seq_elem = ragged ? p.seq_kv_offsets[token]
                                   : (uint64_t)p.layer * p.capacity_tokens * row_stride;
  const uint64_t first_elem = seq_elem + (uint64_t)kvh * D;
  const KV* kbase = static_cast<const KV*>(p.key_cache) + first_elem;
  const KV* vbase = static_cast<const KV*>(p.value_cache) + first_elem;

  // The query heads kvh*G .. kvh*G+G-1 (G*D contiguous floats) are loaded
  // before K/V: vector loads retire in issue order, so using the query waits
  // only for the query (measured faster than issuing K/V first).
  const float* qhead = p.query + ((size_t)token * p.heads + kvh * G) * D;
  float4 qraw[kQRegs ? G * EL / 4 : 1];
  if constexpr (kQRegs) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < EL; e += 4) {
        qraw[(g * EL + e) / 4] = *reinterpret_cast<const float4*>(qhead + g * D + c * EL + e);
      }
    }
  } else {
    qraw[0] = reinterpret_cast<const float4*>(qhead)[tid < kQVec ? tid : 0];
  }

  // K/V rows of the split through buffer resources based at its first row and
  // ending at its last: lanes and rounds past the end read zeros from the range
  // check with no memory access (and are masked out of the softmax).
  const uint32_t row_bytes = (uint32_t)(row_stride * sizeof(KV));
  uint32_t span_bytes = count * row_bytes;
  if (ragged) {
    // Device-side offsets are not checked on the host: the range also ends at
    // the pool's end, so a bad offset reads zeros instead of faulting.
    // An offset that is not a whole 16-byte chunk (misaligned rows) reads zeros too.
    const uint64_t split_elem = first_elem + (uint64_t)key_begin * row_stride;
    const uint64_t avail =
      split_elem < p.pool_elems ? (p.pool_elems - split_elem) * sizeof(KV) : 0u;
    span_bytes = (seq_elem * sizeof(KV)) % 16u != 0 ? 0u
                                                   : (uint32_t)min((uint64_t)span_bytes, avail);
  }
  const __amdgpu_buffer_rsrc_t krsrc =
    make_buffer_rsrc(kbase + (size_t)key_begin * row_stride, span_bytes);
  const __amdgpu_buffer_rsrc_t vrsrc =
    make_buffer_rsrc(vbase + (size_t)key_begin * row_stride, span_bytes);
  const uint32_t wave_first = (uint32_t)(wave * KW);  // wave's first key in a round
  const uint32_t lane_key = wave_first + (uint32_t)kslot;
  const uint32_t lane_off = lane_key * row_bytes + 16u * C * c;

  // A ring of P register sets (round r uses set r % P), each reloaded in place
  // right after its round computes, so the next P rounds are always in flight
  // and no loaded register is ever copied (a copy would have to wait for its
  // load).  The scheduling barriers pin the issue order (K then V, set by
  // set), which the wait counts in the loop below depend on.
  u32x4_t kset[P][C], vset[P][C];
  auto load_set = [&](uint32_t ki, u32x4_t* kreg, u32x4_t* vreg) {
    const uint32_t off = lane_off + ki * row_bytes;
#pragma unroll
    for (int j = 0; j < C; ++j) {
      kreg[j] = buffer_load_nt_b128(krsrc, off + 16u * j);
    }
#pragma unroll
    for (int j = 0; j < C; ++j) {
      vreg[j] = buffer_load_nt_b128(vrsrc, off + 16u * j);
    }
  };
#pragma unroll
  for (int i = 0; i < P; ++i) {
    __builtin_amdgcn_sched_barrier(0);
    load_set((uint32_t)i * KPR, kset[i], vset[i]);
  }
  __builtin_amdgcn_sched_barrier(0);

  // Query pre-scaled into the log2 domain.
  float qr[kQRegs ? G : 1][kQRegs ? EL : 1];
  if constexpr (kQRegs) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < EL; e += 4) {
        const float4 t = qraw[(g * EL + e) / 4];
        qr[g][e + 0] = t.x * p.scale_log2;
        qr[g][e + 1] = t.y * p.scale_log2;
        qr[g][e + 2] = t.z * p.scale_log2;
        qr[g][e + 3] = t.w * p.scale_log2;
      }
    }
  } else {
    reinterpret_cast<float4*>(s_q)[tid < kQVec ? tid : kQVec] =
      make_float4(qraw[0].x * p.scale_log2, qraw[0].y * p.scale_log2, qraw[0].z * p.scale_log2,
                  qraw[0].w * p.scale_log2);
    __syncthreads();
  }

  float m[G];  // wave-uniform reference max (log2 domain)
  float l[G];
  float lc[G];  // Kahan compensation of l (see kahan_add)
  float o[G][EL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.0f;
    lc[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < EL; ++e) {
      o[g][e] = 0.0f;
    }
  }

  // One round: keys [kr, kr + KPR) of the split (relative), this lane's key at
  // kr + lane_key.
  auto round = [&](uint32_t kr, const u32x4_t* kraw, const u32x4_t* vraw) {
    const bool valid = kr + lane_key < count;
    float kf[EL];
#pragma unroll
    for (int j = 0; j < C; ++j) {
      T::to_float(kraw[j], kf + j * E);
    }
    float sc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float acc = 0.0f;
      if constexpr (kQRegs) {
#pragma unroll
        for (int e = 0; e < EL; ++e) {
          acc = fmaf(qr[g][e], kf[e], acc);
        }
      } else {
        // An opaque zero in the LDS address keeps the compiler from hoisting
        // the loop-invariant query words into registers across rounds.
        int qz;
        __asm__ volatile("v_mov_b32 %0, 0" : "=v"(qz));
        const float* sq = s_q + qz + g * D + c * EL;
#pragma unroll
        for (int e = 0; e < EL; e += 4) {
          const float4 q4 = *reinterpret_cast<const float4*>(sq + e);
          acc = fmaf(q4.x, kf[e + 0], acc);
          acc = fmaf(q4.y, kf[e + 1], acc);
          acc = fmaf(q4.z, kf[e + 2], acc);
          acc = fmaf(q4.w, kf[e + 3], acc);
        }
      }
      // The cross-lane reduction runs for every lane (it cannot sit under a
      // divergent mask); invalid keys are masked afterwards.
      const float red = row_sum<R>(acc);
      sc[g] = valid ? red : -INFINITY;
    }
    float vf[EL];
#pragma unroll
    for (int j = 0; j < C; ++j) {
      T::to_float(vraw[j], vf + j * E);
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float bmax = uniform_f(slots_max<R>(sc[g]));
      if (bmax > m[g] + kRescaleSlack) {
        const float corr = fast_exp2(m[g] - bmax);  // 0 on the first valid round
        m[g] = bmax;
        l[g] *= corr;
        lc[g] *= corr;
#pragma unroll
        for (int e = 0; e < EL; ++e) {
          o[g][e] *= corr;
        }
      }
      const float pr = valid ? fast_exp2(sc[g] - m[g]) : 0.0f;
      kahan_add(l[g], lc[g], pr);
#pragma unroll
      for (int e = 0; e < EL; ++e) {
        o[g][e] = fmaf(pr, vf[e], o[g][e]);
      }
    }
  };

  // Each wave stops after its last round holding a key of the split.  Written
  // as an explicit two-step body: exits leave the loop directly, so the
  // compiler's wait counts stay exact (a round waits only for its own set).
  auto step = [&](uint32_t ki, u32x4_t* kreg, u32x4_t* vreg) {
    round(ki, kreg, vreg);
    load_set(ki + P * KPR, kreg, vreg);
  };
  for (uint32_t kr = 0; kr + wave_first < count; kr += 2 * KPR) {
    step(kr, kset[0], vset[0]);
    if (kr + KPR + wave_first >= count) {
      break;
    }
    step(kr + KPR, kset[1], vset[1]);
  }

  // Wave partial: the KW key slots share the wave's running max, so their
  // accumulators add lane-wise.
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float lw = slots_sum<R>(l[g] - lc[g]);
#pragma unroll
    for (int e = 0; e < EL; ++e) {
      o[g][e] = slots_sum<R>(o[g][e]);
    }
    if (lane == 0) {
      s_m[wave][g] = m[g];
      s_l[wave][g] = lw;
    }
    if (kslot == 0) {
#pragma unroll
      for (int e = 0; e < EL; e += 4) {
        *reinterpret_cast<float4*>(&s_o[wave][g * D + c * EL + e]) =
          make_float4(o[g][e], o[g][e + 1], o[g][e + 2], o[g][e + 3]);
      }
    }
  }
  __syncthreads();

  // Workgroup merge of the wave partials; thread handles outputs
  // idx = tid + k*kThreads of the G*D block.
  const size_t tk = (size_t)token * p.kv_heads + kvh;
  float* po = p.part_o + (tk * p.splits + split) * (size_t)(G * D);
  float* pml = p.part_ml + (tk * p.splits + split) * (size_t)(G * 2);
#pragma unroll
  for (int k = 0; k < kOutPerThread; ++k) {
    const int idx = tid + k * kThreads;
    if (idx >= G * D) {
      continue;
    }
    const int g = idx / D;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      mx = fmaxf(mx, s_m[w][g]);
    }
    float acc = 0.0f;
    float den = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float wt = s_m[w][g] == -INFINITY ? 0.0f : fast_exp2(s_m[w][g] - mx);
      acc = fmaf(wt, s_o[w][idx], acc);
      den = fmaf(wt, s_l[w][g], den);
    }
    if (p.splits == 1) {
      write_final<D, G>(p, token, kvh, idx, den, acc);
    } else {
      store_through(&po[idx], acc);
      if (idx % D == 0) {
        store_through(&pml[g * 2 + 0], mx);
        store_through(&pml[g * 2 + 1], den);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// MFMA variant: head_dim 256, f16 cache, G <= 4 query heads per KV head.
//
// The vector kernel above spends about 80 VALU operations per 16-byte K/V
// chunk (f16 -> f32 conversions, G dot-product FMAs and 32-lane reductions,
// G P*V FMAs).  With every SIMD busy it tops out near 5.2 TB/s on a large
// batched decode (VALU active 75% of the time, measured).  This kernel moves
// the arithmetic onto the matrix cores so that the stream is bound by memory.
//  * A workgroup of 4 waves owns one (token, kv_head, key split) work item, as
//    above; wave w takes the split's 16-key tiles w, w + 4, ...  Each wave
//    copies its tiles' K and V rows straight into two LDS stages of its own
//    (buffer_load ... lds), so the loop has no barriers and the compiler's wait
//    counts are not involved: the kernel awaits the copies itself.  The copies
//    carry the nontemporal hint: the KV stream is read once, and keeping it out
//    of the caches was measured at 8% faster attention and 13% faster for the
//    C4 block, whose GDN state then stays cached.
//  * S^T = K Q^T on v_mfma_f32_16x16x32_f16.  A = the tile's 16 key rows (k =
//    head dims, 16-byte LDS fragments), B = the G query heads as columns.  The
//    query, pre-scaled into the log2 domain, is held in the split fp16 form of
//    device_common.hpp (split_f16: hi, and lo scaled by 2^11, both normal f16
//    where it matters), with the hi and lo products in separate accumulators,
//    so K (exact in f16) times the query reproduces the f32 dot product to
//    about 2^-21 relative even where the matrix core flushes f16 denormals.
//  * The S^T accumulator (lane l: head l % 16, keys 4 (l / 16) + r) is already
//    the A operand of O += P V on v_mfma_f32_16x16x16_f16 (k = keys), with P
//    split the same way into a hi and a lo output accumulator.  V^T fragments
//    come from LDS through the transposing read ds_read_b64_tr_b16.
//  * Online softmax per head with the vector kernel's wave-uniform lazy
//    rescale; wave partials merge through LDS and splits in the same second
//    pass, in the same partial format.
// LDS rows are XOR-swizzled in 16-byte chunks (K: chunk ^ (row & 7); V: chunk ^
// 2 (row & 3)) so that both fragment reads are free of bank conflicts.
// ---------------------------------------------------------------------------
constexpr int kMWaves = 4;
constexpr int kMStages = 2;                       // tiles in flight per wave
constexpr int kMCopiesPerTile = kMTile;           // 1 KB copies per tile: 8 for K, 8 for V

template <int G>
__global__ __launch_bounds__(64 * kMWaves) void attention_decode_mfma_kernel(DecodeParams p) {
  static_assert(G == 1 || G == 2 || G == 4, "query heads per KV head (rows 0..3 of a tile)");
  // Per wave and stage: the K tile, then the V tile.  After the key loop the
  // region holds the wave partials for the merge.
  __shared__ __attribute__((aligned(16))) half_t s_kv[kMWaves][kMStages][2][kMTileHalfs];
  __shared__ float s_m[kMWaves][G];
  __shared__ float s_l[kMWaves][G];
  static_assert(sizeof(float) * kMWaves * G * kMD <= sizeof(s_kv), "merge area");
  float(*s_o)[G * kMD] = reinterpret_cast<float(*)[G * kMD]>(&s_kv[0][0][0][0]);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  uint32_t split = blockIdx.x;
  uint32_t kvh = blockIdx.y;
  uint32_t token = blockIdx.z;
  const bool ragged = p.seq_positions != nullptr;
  if (ragged) {
    const uint2 item = p.work_items[blockIdx.x];
    if (item.x == 0xffffffffu) {
      return;  // past the last work item
    }
    token = item.x;
    kvh = item.y >> 16;
    split = item.y & 0xffffu;
  }
  const uint32_t n_keys = token_keys(p.seq_positions, p.start_position, token);
  const uint32_t key_begin = split * p.keys_per_split;
  if (key_begin >= n_keys) {
    return;  // empty split (whole workgroup)
  }
  const uint32_t count = min(n_keys, key_begin + p.keys_per_split) - key_begin;

  const size_t row_stride = (size_t)p.kv_heads * kMD;
  const uint32_t row_bytes = (uint32_t)(row_stride * sizeof(half_t));
  const uint64_t seq_elem = ragged ? p.seq_kv_offsets[token]
                                   : (uint64_t)p.layer * p.capacity_tokens * row_stride;
  const uint64_t first_elem = seq_elem + (uint64_t)kvh * kMD;
  uint32_t span_bytes = count * row_bytes;
  if (ragged) {
    // Device-side offsets are not checked on the host: the range also ends at
    // the pool's end (and is empty for rows that are not whole 16-byte chunks),
    // so a bad offset reads zeros instead of faulting.
    const uint64_t split_elem = first_elem + (uint64_t)key_begin * row_stride;
    const uint64_t avail =
      split_elem < p.pool_elems ? (p.pool_elems - split_elem) * sizeof(half_t) : 0u;
    span_bytes = (seq_elem * sizeof(half_t)) % 16u != 0
                   ? 0u
                   : (uint32_t)min((uint64_t)span_bytes, avail);
  }
  const half_t* kbase =
    static_cast<const half_t*>(p.key_cache) + first_elem + (size_t)key_begin * row_stride;
  const half_t* vbase =
    static_cast<const half_t*>(p.value_cache) + first_elem + (size_t)key_begin * row_stride;
  const i32x4_t krs = rsrc_words(kbase, span_bytes);
  const i32x4_t vrs = rsrc_words(vbase, span_bytes);

  // Query fragments (B operand of S^T): lane (head r16, kq) holds dims
  // 32 s + 8 kq .. + 7 of step s, scaled into the log2 domain, as hi + lo.
  half8_t qhi[8], qlo[8];
  {
    const int g = r16 < G ? r16 : 0;
    const float qscale = r16 < G ? p.scale_log2 : 0.0f;
    const float* qh = p.query + ((size_t)token * p.heads + kvh * G + g) * kMD + 8 * kq;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const float4 a = *reinterpret_cast<const float4*>(qh + 32 * s);
      const float4 b = *reinterpret_cast<const float4*>(qh + 32 * s + 4);
      const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        half_t hi, lo;
        split_f16(v[j] * qscale, hi, lo);
        qhi[s][j] = hi;
        qlo[s][j] = lo;
      }
    }
  }

  // Copies tile t (keys 16 t .. 16 t + 15 of the split) of K and V into stage
  // st of this wave: 8 + 8 copies of 1 KB, copy c filling rows 2 c, 2 c + 1.
  // Rows at or past the split's end read as zeros (resource range check).
  const uint32_t copy_row = (uint32_t)(lane >> 5);
  const uint32_t chunk = (uint32_t)(lane & 31);
  auto issue_tile = [&](uint32_t t, int st) __attribute__((always_inline)) {
    half_t* kdst = &s_kv[wave][st][0][0];
    half_t* vdst = &s_kv[wave][st][1][0];
#pragma unroll
    for (int c = 0; c < kMTile / 2; ++c) {
      const uint32_t row = 2u * c + copy_row;
      const uint32_t base = (kMTile * t + row) * row_bytes;
      copy16_to_lds_nt(krs, base + 16u * (chunk ^ (row & 7u)), kdst + c * 2 * kMD);
      copy16_to_lds_nt(vrs, base + 16u * (chunk ^ (2u * (row & 3u))), vdst + c * 2 * kMD);
    }
  };

  float m[G];  // wave-uniform reference max per head (log2 domain)
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
  }
  // This lane's share of head r16's denominator, summed with Kahan's
  // compensation (lcomp): a long split adds thousands of small weights to a sum
  // near 1, where plain fp32 addition would drop a systematic part of each.
  float lpart = 0.0f;
  float lcomp = 0.0f;
  // O tile n: lane l holds dim 16 n + l % 16 of heads 4 (l / 16) + r; o from
  // the hi probabilities, olo from the lo ones (scaled by 2^11).
  float4v_t o[16], olo[16];
#pragma unroll
  for (int n = 0; n < 16; ++n) {
    o[n] = float4v_t{0.f, 0.f, 0.f, 0.f};
    olo[n] = float4v_t{0.f, 0.f, 0.f, 0.f};
  }

  const uint32_t ntiles = (count + kMTile - 1) / kMTile;
  issue_tile((uint32_t)wave, 0);
  issue_tile((uint32_t)wave + kMWaves, 1);
  int st = 0;
  for (uint32_t t = (uint32_t)wave; t < ntiles; t += kMWaves) {
    // Stage st holds tile t once only the other stage's copies are in flight.
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kMCopiesPerTile) : "memory");
    const half_t* ks = &s_kv[wave][st][0][0];
    const half_t* vs = &s_kv[wave][st][1][0];

    // S^T = K Q^T (keys x heads): the hi and the lo chain, then combined.
    float4v_t shi = {0.f, 0.f, 0.f, 0.f};
    float4v_t slo = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const half8_t kf = *reinterpret_cast<const half8_t*>(
        ks + r16 * kMD + 8 * ((4 * s + kq) ^ (r16 & 7)));
      shi = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qhi[s], shi, 0, 0, 0);
      slo = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qlo[s], slo, 0, 0, 0);
    }
    float4v_t sacc;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sacc[r] = fmaf(slo[r], kLoUnscale, shi[r]);
    }

    // Softmax: lane holds keys 16 t + 4 kq + r of head r16.
    float sc[4];
    bool valid[4];
    float cmax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      valid[r] = r16 < G && kMTile * t + 4u * kq + r < count;
      sc[r] = valid[r] ? sacc[r] : -INFINITY;
      cmax = fmaxf(cmax, sc[r]);
    }
    cmax = fmaxf(cmax, __shfl_xor(cmax, 16, 64));
    cmax = fmaxf(cmax, __shfl_xor(cmax, 32, 64));
    float corr_lane = 1.0f;
    float m_lane = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float bm = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                   __builtin_bit_cast(int, cmax), g));
      if (bm > m[g] + kRescaleSlack) {  // wave-uniform
        const float corr = fast_exp2(m[g] - bm);  // 0 on the head's first valid tile
        m[g] = bm;
#pragma unroll
        for (int n = 0; n < 16; ++n) {
          o[n][g] *= corr;  // head g is row g: register g of lanes 0..15
          olo[n][g] *= corr;
        }
        corr_lane = r16 == g ? corr : corr_lane;
      }
      m_lane = r16 == g ? m[g] : m_lane;
    }
    lpart *= corr_lane;
    lcomp *= corr_lane;
    half4_t phi, plo;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float pr = valid[r] ? fast_exp2(sc[r] - m_lane) : 0.0f;
      kahan_add(lpart, lcomp, pr);
      half_t h, l;
      split_f16(pr, h, l);
      phi[r] = h;
      plo[r] = l;
    }

    // O += P V: lane 4 e + q of group kq points at row 4 kq + e, columns
    // 16 n + 4 q .. + 3; the transposing read returns column 16 n + l % 16
    // of rows 4 kq .. 4 kq + 3.
    const int vrow = 4 * kq + (r16 >> 2);
    const int q = r16 & 3;
    const half_t* vrow_p = vs + vrow * kMD + 4 * (q & 1);
    const int vswz = 2 * (vrow & 3);
#pragma unroll
    for (int n = 0; n < 16; ++n) {
      const half4_t vf = read_tr16(vrow_p + 8 * ((2 * n + (q >> 1)) ^ vswz));
      o[n] = __builtin_amdgcn_mfma_f32_16x16x16f16(phi, vf, o[n], 0, 0, 0);
      olo[n] = __builtin_amdgcn_mfma_f32_16x16x16f16(plo, vf, olo[n], 0, 0, 0);
    }

    // Refill this stage with tile t + 8 once its LDS reads have returned.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    issue_tile(t + kMStages * kMWaves, st);
    st ^= 1;
  }
  // No copy may land in a stage after the stages are reused below.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Wave partial: head r16's denominator over the four lane groups.
  float lw = lpart - lcomp;
  lw += __shfl_xor(lw, 16, 64);
  lw += __shfl_xor(lw, 32, 64);
  __syncthreads();  // every wave is done with its stages
  if (lane < G) {
    s_l[wave][lane] = lw;
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      s_m[wave][g] = m[g];
    }
  }
  if (lane < 16) {
#pragma unroll
    for (int n = 0; n < 16; ++n) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        s_o[wave][g * kMD + 16 * n + lane] = fmaf(olo[n][g], kLoUnscale, o[n][g]);
      }
    }
  }
  __syncthreads();

  // Workgroup merge of the wave partials, as in the vector kernel.
  constexpr int kThreads = 64 * kMWaves;
  constexpr int kOutPerThread = G * kMD / kThreads;
  const size_t tk = (size_t)token * p.kv_heads + kvh;
  float* po = p.part_o + (tk * p.splits + split) * (size_t)(G * kMD);
  float* pml = p.part_ml + (tk * p.splits + split) * (size_t)(G * 2);
#pragma unroll
  for (int k = 0; k < kOutPerThread; ++k) {
    const int idx = tid + k * kThreads;
    const int g = idx / kMD;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kMWaves; ++w) {
      mx = fmaxf(mx, s_m[w][g]);
    }
    float acc = 0.0f;
    float den = 0.0f;
#pragma unroll
    for (int w = 0; w < kMWaves; ++w) {
      const float wt = s_m[w][g] == -INFINITY ? 0.0f : fast_exp2(s_m[w][g] - mx);
      acc = fmaf(wt, s_o[w][idx], acc);
      den = fmaf(wt, s_l[w][g], den);
    }
    if (p.splits == 1) {
      write_final<kMD, G>(p, token, kvh, idx, den, acc);
    } else {
      store_through(&po[idx], acc);
      if (idx % kMD == 0) {
        store_through(&pml[g * 2 + 0], mx);
        store_through(&pml[g * 2 + 1], den);
      }
    }
  }
}

// Split merge: one workgroup per (token, head, 16-dim slice).  256 threads =
// 4 float4 chunks x 64 split subsets; every thread issues all of its (<= 4)
// partial loads before using any.  The global max and the weighted sums are
// reduced across subsets with lane shuffles (lane bits 2..5) and then across
// the 4 waves through LDS.
constexpr int kMergeDims = 16;
constexpr int kMergeChunks = kMergeDims / 4;
static_assert(kMergeChunks == 4, "merge lane reductions run over lane bits 2..5");
constexpr int kMergeSubsets = 256 / kMergeChunks;
constexpr int kMergePerThread = kMaxSplits / kMergeSubsets;

// Number of splits holding partials for `token` (>= 1: every token has a key).
__device__ __forceinline__ uint32_t token_splits(const CombineArgs& p, uint32_t token) {
  if (p.keys_per_split == 0) {
    return p.splits;
  }
  const uint64_t keys = token_keys(p.positions, p.start_position, token);
  const uint64_t needed = (keys + p.keys_per_split - 1u) / p.keys_per_split;
  return (uint32_t)max((uint64_t)1, min((uint64_t)p.splits, needed));
}

// Reductions over lane bits 2..5 (the split subsets of one chunk): rotations by
// 4 and 8 within each 16-lane row, then the xor-16 and xor-32 exchanges.
__device__ __forceinline__ float merge_lanes_max(float x) {
  x = fmaxf(x, dpp<kDppRowRor4>(x));
  x = fmaxf(x, dpp<kDppRowRor8>(x));
  return xor32_max(xor16_max(x));
}

__device__ __forceinline__ float merge_lanes_sum(float x) {
  x += dpp<kDppRowRor4>(x);
  x += dpp<kDppRowRor8>(x);
  return xor32_sum(xor16_sum(x));
}

// Gate values of four output dims, loaded before the partials so that the
// two loads overlap; (1, 1, 1, 1) when ungated or not needed.
__device__ __forceinline__ float4 load_gate4(const float* gate, size_t out_index, bool needed) {
  if (gate == nullptr || !needed) {
    return make_float4(1.f, 1.f, 1.f, 1.f);
  }
  return *reinterpret_cast<const float4*>(gate + out_index);
}

__device__ __forceinline__ void store_gated4(const CombineArgs& p, size_t out_index, float4 r,
                                             float inv, float4 gv) {
  float out[4] = {r.x * inv, r.y * inv, r.z * inv, r.w * inv};
  if (p.gate != nullptr) {
    out[0] *= sigmoidf_acc(gv.x);
    out[1] *= sigmoidf_acc(gv.y);
    out[2] *= sigmoidf_acc(gv.z);
    out[3] *= sigmoidf_acc(gv.w);
  }
  // Nontemporal (C2 at P=0 27.2 -> 26.8 us, P=3072 47.7 -> 47.1 us: the flash
  // merge writes 8 MB that the next launch reads).
  __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, make_float4(out[0], out[1], out[2], out[3])),
                              reinterpret_cast<u32x4_t*>(p.output + out_index));
}

__global__ __launch_bounds__(256) void attention_merge(CombineArgs p) {
  __shared__ float s_mx[4];
  __shared__ float s_den[4][kMergeChunks];
  __shared__ float4 s_acc[4][kMergeChunks];
  const uint32_t group = p.heads / p.kv_heads;
  const uint32_t token = blockIdx.x;
  const uint32_t head = blockIdx.y;
  const uint32_t kvh = head / group;
  const uint32_t g = head % group;
  const uint32_t d0 = blockIdx.z * kMergeDims;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int chunk = tid % kMergeChunks;
  const int subset = tid / kMergeChunks;
  const size_t base = (size_t)token * p.kv_heads + kvh;
  const uint32_t nsp = token_splits(p, token);
  const size_t out_index = ((size_t)token * p.heads + head) * p.head_dim + d0 + chunk * 4;
  const float4 gv = load_gate4(p.gate, out_index, tid < kMergeChunks);

  float mv[kMergePerThread], lv[kMergePerThread];
  float4 ov[kMergePerThread];
  // Unconditional loads from clamped indices (masked below) keep every load in
  // flight at once.
#pragma unroll
  for (int j = 0; j < kMergePerThread; ++j) {
    const uint32_t s = min(subset + j * kMergeSubsets, nsp - 1u);
    const size_t unit = (base * p.splits + s) * group + g;
    mv[j] = p.partial_ml[unit * 2];
    lv[j] = p.partial_ml[unit * 2 + 1];
    ov[j] = *reinterpret_cast<const float4*>(p.partial_o + unit * p.head_dim + d0 + chunk * 4);
  }
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < kMergePerThread; ++j) {
    if (subset + j * kMergeSubsets >= nsp) {
      mv[j] = -INFINITY;
    }
    mx = fmaxf(mx, mv[j]);
  }
  mx = merge_lanes_max(mx);
  if (lane == 0) {
    s_mx[wave] = mx;
  }
  __syncthreads();
  const float gmx = fmaxf(fmaxf(s_mx[0], s_mx[1]), fmaxf(s_mx[2], s_mx[3]));
  float den = 0.0f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int j = 0; j < kMergePerThread; ++j) {
    const float w = mv[j] == -INFINITY ? 0.0f : fast_exp2(mv[j] - gmx);
    den = fmaf(w, lv[j], den);
    acc.x = fmaf(w, ov[j].x, acc.x);
    acc.y = fmaf(w, ov[j].y, acc.y);
    acc.z = fmaf(w, ov[j].z, acc.z);
    acc.w = fmaf(w, ov[j].w, acc.w);
  }
  den = merge_lanes_sum(den);
  acc.x = merge_lanes_sum(acc.x);
  acc.y = merge_lanes_sum(acc.y);
  acc.z = merge_lanes_sum(acc.z);
  acc.w = merge_lanes_sum(acc.w);
  if (lane < kMergeChunks) {
    s_den[wave][chunk] = den;
    s_acc[wave][chunk] = acc;
  }
  __syncthreads();
  if (tid >= kMergeChunks) {
    return;
  }
  float tden = 0.0f;
  float4 r = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    tden += s_den[w][chunk];
    r.x += s_acc[w][chunk].x;
    r.y += s_acc[w][chunk].y;
    r.z += s_acc[w][chunk].z;
    r.w += s_acc[w][chunk].w;
  }

  const float inv = tden == 0.0f ? 0.0f : 1.0f / tden;
  store_gated4(p, out_index, r, inv, gv);
}

// Ragged work list.  The dispatcher hands workgroup i to XCD i mod 8, so empty
// workgroups interleaved in a (split, kv_head, sequence) grid starve whole XCDs
// (a grid of alternating empty/full workgroups runs half the chip).  One
// workgroup writes the non-empty (sequence, kv_head, split) items densely, in
// sequence order, then marks the rest of the grid empty: consecutive items (the
// splits of one sequence) land on consecutive XCDs and the empty tail costs
// nothing.
__global__ __launch_bounds__(256) void ragged_plan_kernel(const uint32_t* positions,
                                                          uint32_t sequences, uint32_t kv_heads,
                                                          uint32_t keys_per_split,
                                                          uint32_t max_splits,
                                                          uint32_t grid_items, uint2* items) {
  __shared__ uint32_t s_scan[256];
  const uint32_t tid = threadIdx.x;
  const uint32_t per = (sequences + 255u) / 256u;
  const uint32_t b0 = min(sequences, tid * per);
  const uint32_t b1 = min(sequences, b0 + per);
  auto splits_of = [&](uint32_t b) {
    const uint64_t keys = (uint64_t)positions[b] + 1u;
    const uint64_t n = (keys + keys_per_split - 1u) / keys_per_split;
    return (uint32_t)min(n, (uint64_t)max_splits);
  };
  uint32_t local = 0;
  for (uint32_t b = b0; b < b1; ++b) {
    local += splits_of(b) * kv_heads;
  }
  s_scan[tid] = local;
  __syncthreads();
  // Inclusive scan over the 256 per-thread counts (Hillis-Steele).
  for (uint32_t off = 1; off < 256u; off <<= 1) {
    const uint32_t add = tid >= off ? s_scan[tid - off] : 0u;
    __syncthreads();
    s_scan[tid] += add;
    __syncthreads();
  }
  uint32_t next = s_scan[tid] - local;
  for (uint32_t b = b0; b < b1; ++b) {
    const uint32_t n = splits_of(b);
    for (uint32_t h = 0; h < kv_heads; ++h) {
      for (uint32_t sp = 0; sp < n; ++sp) {
        items[next++] = make_uint2(b, (h << 16) | sp);
      }
    }
  }
  for (uint32_t i = s_scan[255] + tid; i < grid_items; i += 256u) {
    items[i] = make_uint2(0xffffffffu, 0u);
  }
}

// Shapes outside the tuned templates: one wave per (token, head), 64 lanes over
// dims, online softmax over keys (the reference kernel's structure).
template <typename KV>
__global__ __launch_bounds__(64) void attention_generic(DecodeParams p, uint32_t head_dim,
                                                        uint32_t group) {
  const uint32_t token = blockIdx.x;
  const uint32_t head = blockIdx.y;
  const int lane = threadIdx.x;
  const uint32_t kvh = head / group;
  const uint32_t position = p.start_position + token;
  const size_t row_stride = (size_t)p.kv_heads * head_dim;
  const KV* kbase = static_cast<const KV*>(p.key_cache) +
                    (size_t)p.layer * p.capacity_tokens * row_stride + (size_t)kvh * head_dim;
  const KV* vbase = static_cast<const KV*>(p.value_cache) +
                    (size_t)p.layer * p.capacity_tokens * row_stride + (size_t)kvh * head_dim;
  const float* q = p.query + ((size_t)token * p.heads + head) * head_dim;
  float qv[4];
  float o[4];
  for (int i = 0; i < 4; ++i) {
    const uint32_t d = lane + 64u * i;
    qv[i] = d < head_dim ? q[d] * p.scale_log2 : 0.0f;
    o[i] = 0.0f;
  }
  float m = -INFINITY;
  float l = 0.0f;
  for (uint32_t key = 0; key <= position; ++key) {
    float acc = 0.0f;
    for (int i = 0; i < 4; ++i) {
      const uint32_t d = lane + 64u * i;
      if (d < head_dim) {
        acc += qv[i] * static_cast<float>(kbase[(size_t)key * row_stride + d]);
      }
    }
    const float s = wave_sum(acc);
    const float mn = fmaxf(m, s);
    const float corr = fast_exp2(m - mn);
    const float pr = fast_exp2(s - mn);
    l = l * corr + pr;
    for (int i = 0; i < 4; ++i) {
      const uint32_t d = lane + 64u * i;
      const float v = d < head_dim ? static_cast<float>(vbase[(size_t)key * row_stride + d]) : 0.0f;
      o[i] = o[i] * corr + pr * v;
    }
    m = mn;
  }
  const float inv = l == 0.0f ? 0.0f : 1.0f / l;
  for (int i = 0; i < 4; ++i) {
    const uint32_t d = lane + 64u * i;
    if (d < head_dim) {
      const size_t idx = ((size_t)token * p.heads + head) * head_dim + d;
      float r = o[i] * inv;
      if (p.gate != nullptr) {
        r *= sigmoidf_acc(p.gate[idx]);
      }
      p.output[idx] = r;
    }
  }
}

struct SplitPlan {
  uint32_t keys_per_split;
  uint32_t splits;
};

// Splits per (token, kv_head) so that the grid puts about one workgroup on each
// CU; a split may be any number of keys (a partial last round is masked).
// Ragged decode: a fixed split size, so sequences of any length divide into
// equal pieces of work (the grid covers the longest; empty splits exit).
constexpr uint64_t kRaggedKeysPerSplit = 1024;
constexpr uint64_t kSingleSplitKeys = 256;

SplitPlan plan_splits(const AttentionArgs& a, int cu_count) {
  const bool ragged = a.seq_positions != nullptr;
  // Keys of the longest query.
  const uint64_t max_keys =
    ragged ? (uint64_t)a.max_position + 1 : (uint64_t)a.start_position + a.tokens;
  const uint64_t units = (uint64_t)a.tokens * a.kv_heads;
  const uint64_t slots = (uint64_t)(cu_count > 0 ? cu_count : 256);
  uint64_t splits_target = slots / units;
  if (splits_target < 1) {
    splits_target = 1;
  }
  uint64_t kps = ragged ? kRaggedKeysPerSplit : (max_keys + splits_target - 1) / splits_target;
  // A short context is one split: its keys are a few loads per wave, and the
  // merge launch a split would need costs more than they do.
  if (!ragged && max_keys <= kSingleSplitKeys) {
    kps = max_keys;
  }
  if (const char* env = std::getenv("KRAKEN_DECODE_KEYS_PER_SPLIT")) {
    const long v = std::strtol(env, nullptr, 10);
    if (v > 0) {
      kps = (uint64_t)v;
    }
  }
  uint64_t splits = (max_keys + kps - 1) / kps;
  if (splits > kMaxSplits) {
    kps = (max_keys + kMaxSplits - 1) / kMaxSplits;
    splits = (max_keys + kps - 1) / kps;
  }
  return SplitPlan{(uint32_t)kps, (uint32_t)splits};
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

// The tuned kernel moves 16-byte chunks; shapes or pointers outside that contract
// take the generic kernel.
bool tuned_args(const AttentionArgs& a) {
  const uint32_t d = a.head_dim;
  const uint32_t g = a.heads / a.kv_heads;
  if (!aligned16(a.query) || !aligned16(a.key_cache) || !aligned16(a.value_cache) ||
      !aligned16(a.output)) {
    return false;
  }
  return (d == 256 || d == 128 || d == 64) && (g == 1 || g == 2 || g == 4 || g == 8);
}

size_t partial_bytes(const AttentionArgs& a, const SplitPlan& plan) {
  if (plan.splits <= 1) {
    return 0;
  }
  const size_t g = a.heads / a.kv_heads;
  const size_t units = (size_t)a.tokens * a.kv_heads;
  return units * plan.splits * g * (a.head_dim + 2) * sizeof(float);
}

// Ragged work list entries: one per (sequence, kv_head, split) of the grid.
size_t work_item_count(const AttentionArgs& a, const SplitPlan& plan) {
  return a.seq_positions != nullptr ? (size_t)a.tokens * a.kv_heads * plan.splits : 0;
}

size_t data_bytes(const AttentionArgs& a, const SplitPlan& plan) {
  // Partials, then the work list (8-byte items) at a 256-byte boundary.
  return (partial_bytes(a, plan) + 255u) / 256u * 256u + work_item_count(a, plan) * 8u;
}

// Kernel choice for head_dim 256 with an f16 cache and up to 4 query heads per
// KV head.  Splits of at least kMfmaMinKeys keys (the ragged batched decode)
// take the MFMA kernel with its direct-to-LDS copy pipeline; shorter splits of
// one sequence (batch-1 decode) take the short-split MFMA kernel, whose loads
// are all issued up front.  Other shapes take the vector kernel.
// KRAKEN_DECODE_KERNEL=vector, =mfma or =short forces one.
constexpr uint32_t kMfmaMinKeys = 512;

enum class DecodeKernel { vector, mfma, short_split };

DecodeKernel decode_kernel_choice(uint32_t keys_per_split, bool ragged) {
  const char* v = std::getenv("KRAKEN_DECODE_KERNEL");
  if (v != nullptr && std::strcmp(v, "vector") == 0) {
    return DecodeKernel::vector;
  }
  if (v != nullptr && std::strcmp(v, "mfma") == 0) {
    return DecodeKernel::mfma;
  }
  if (v != nullptr && std::strcmp(v, "short") == 0 && !ragged) {
    return DecodeKernel::short_split;
  }
  if (keys_per_split >= kMfmaMinKeys) {
    return DecodeKernel::mfma;
  }
  return ragged ? DecodeKernel::vector : DecodeKernel::short_split;
}

template <int D, int G, typename KV>
hipError_t launch_tuned(const DecodeParams& p, hipStream_t stream) {
  // Ragged: one workgroup per work-list entry (see ragged_plan_kernel).
  const dim3 grid = p.work_items != nullptr ? dim3(p.splits * p.kv_heads * p.tokens)
                                            : dim3(p.splits, p.kv_heads, p.tokens);
  DecodeKernel kind = DecodeKernel::vector;
  if constexpr (D == kMD && std::is_same_v<KV, half_t> && (G == 1 || G == 2 || G == 4)) {
    kind = decode_kernel_choice(p.keys_per_split, p.work_items != nullptr);
    if (kind == DecodeKernel::mfma) {
      attention_decode_mfma_kernel<G><<<grid, 64 * kMWaves, 0, stream>>>(p);
    } else if (kind == DecodeKernel::short_split) {
      const hipError_t es = launch_decode_short(p, G, grid, stream);
      if (es != hipSuccess) {
        return es;
      }
    }
  }
  if (kind == DecodeKernel::vector) {
    attention_decode_kernel<D, G, KV><<<grid, 64 * RowShape<D, KV>::W, 0, stream>>>(p);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.splits == 1) {
    return e;
  }
  CombineArgs c{};
  c.partial_o = p.part_o;
  c.partial_ml = p.part_ml;
  c.gate = p.gate;
  c.output = p.output;
  c.tokens = p.tokens;
  c.heads = p.heads;
  c.kv_heads = p.kv_heads;
  c.splits = p.splits;
  c.head_dim = D;
  c.positions = p.seq_positions;
  c.start_position = p.start_position;
  c.keys_per_split = p.keys_per_split;
  return launch_attention_combine(c, stream);
}

template <typename KV>
hipError_t dispatch_kv(const DecodeParams& p, uint32_t d, uint32_t g, bool tuned,
                       hipStream_t stream) {
  switch (tuned ? d : 0u) {
    case 256:
      if (g == 1) return launch_tuned<256, 1, KV>(p, stream);
      if (g == 2) return launch_tuned<256, 2, KV>(p, stream);
      if (g == 4) return launch_tuned<256, 4, KV>(p, stream);
      if (g == 8) return launch_tuned<256, 8, KV>(p, stream);
      break;
    case 128:
      if (g == 1) return launch_tuned<128, 1, KV>(p, stream);
      if (g == 2) return launch_tuned<128, 2, KV>(p, stream);
      if (g == 4) return launch_tuned<128, 4, KV>(p, stream);
      if (g == 8) return launch_tuned<128, 8, KV>(p, stream);
      break;
    case 64:
      if (g == 1) return launch_tuned<64, 1, KV>(p, stream);
      if (g == 2) return launch_tuned<64, 2, KV>(p, stream);
      if (g == 4) return launch_tuned<64, 4, KV>(p, stream);
      if (g == 8) return launch_tuned<64, 8, KV>(p, stream);
      break;
    default:
      break;
  }
  attention_generic<KV><<<dim3(p.tokens, p.heads), 64, 0, stream>>>(p, d, g);
  return hipGetLastError();
}

// Widens an f16 query for the decode kernels (exact: every f16 is an f32).
__global__ __launch_bounds__(256) void f16_to_f32_kernel(const half_t* in, float* out,
                                                         uint64_t count) {
  const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  if (i < count) {
    out[i] = static_cast<float>(in[i]);
  }
}

}  // namespace

// Few splits (chunked prefill): one thread per (token, head, 4 dims) with all of
// its <= S partial loads in flight (clamped indices, masked), no LDS.  With
// kF16 the partials are each split's o / l in f16 (the flash kernel's), scaled
// back by l before the same weighted sum.
template <int S, bool kF16>
__global__ __launch_bounds__(256) void attention_merge_narrow(CombineArgs p) {
  const uint32_t chunks = p.head_dim / 4;
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (size_t)p.tokens * p.heads * chunks) {
    return;
  }
  const uint32_t chunk = (uint32_t)(idx % chunks);
  const size_t th = idx / chunks;  // token * heads + head
  const uint32_t head = (uint32_t)(th % p.heads);
  const uint32_t token = (uint32_t)(th / p.heads);
  const uint32_t group = p.heads / p.kv_heads;
  const uint32_t kvh = head / group;
  const uint32_t g = head % group;
  const size_t base = (size_t)token * p.kv_heads + kvh;
  const uint32_t nsp = token_splits(p, token);
  const size_t out_index = th * p.head_dim + chunk * 4;
  const float4 gv = load_gate4(p.gate, out_index, true);
  float mv[S], lv[S];
  float4 ov[S];
#pragma unroll
  for (int j = 0; j < S; ++j) {
    const uint32_t s = min((uint32_t)j, nsp - 1u);
    const size_t unit = (base * p.splits + s) * group + g;
    mv[j] = p.partial_ml[unit * 2];
    lv[j] = p.partial_ml[unit * 2 + 1];
    if constexpr (kF16) {
      const half4_t h = *reinterpret_cast<const half4_t*>(
        reinterpret_cast<const half_t*>(p.partial_o) + unit * p.head_dim + chunk * 4);
      ov[j] = make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
    } else {
      ov[j] = *reinterpret_cast<const float4*>(p.partial_o + unit * p.head_dim + chunk * 4);
    }
  }
  if constexpr (kF16) {
#pragma unroll
    for (int j = 0; j < S; ++j) {
      ov[j] = make_float4(ov[j].x * lv[j], ov[j].y * lv[j], ov[j].z * lv[j], ov[j].w * lv[j]);
    }
  }
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < S; ++j) {
    if ((uint32_t)j >= nsp) {
      mv[j] = -INFINITY;
    }
    mx = fmaxf(mx, mv[j]);
  }
  float den = 0.0f;
  float4 r = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int j = 0; j < S; ++j) {
    const float w = mv[j] == -INFINITY ? 0.0f : fast_exp2(mv[j] - mx);
    den = fmaf(w, lv[j], den);
    r.x = fmaf(w, ov[j].x, r.x);
    r.y = fmaf(w, ov[j].y, r.y);
    r.z = fmaf(w, ov[j].z, r.z);
    r.w = fmaf(w, ov[j].w, r.w);
  }
  const float inv = den == 0.0f ? 0.0f : 1.0f / den;
  store_gated4(p, out_index, r, inv, gv);
}

// The f16 partials of the flash path: as attention_merge_narrow<S, true>, with
// eight dims per thread (one 16-byte load per split, two output stores), the
// same arithmetic per element.
template <int S>
__global__ __launch_bounds__(256) void attention_merge_narrow_f16x8(CombineArgs p) {
  const uint32_t chunks = p.head_dim / 8;
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (size_t)p.tokens * p.heads * chunks) {
    return;
  }
  const uint32_t chunk = (uint32_t)(idx % chunks);
  const size_t th = idx / chunks;  // token * heads + head
  const uint32_t head = (uint32_t)(th % p.heads);
  const uint32_t token = (uint32_t)(th / p.heads);
  const uint32_t group = p.heads / p.kv_heads;
  const uint32_t kvh = head / group;
  const uint32_t g = head % group;
  const size_t base = (size_t)token * p.kv_heads + kvh;
  const uint32_t nsp = token_splits(p, token);
  const size_t out_index = th * p.head_dim + chunk * 8;
  const float4 gv0 = load_gate4(p.gate, out_index, true);
  const float4 gv1 = load_gate4(p.gate, out_index + 4, true);
  float mv[S], lv[S];
  float4 ov0[S], ov1[S];
#pragma unroll
  for (int j = 0; j < S; ++j) {
    const uint32_t s = min((uint32_t)j, nsp - 1u);
    const size_t unit = (base * p.splits + s) * group + g;
    mv[j] = p.partial_ml[unit * 2];
    lv[j] = p.partial_ml[unit * 2 + 1];
    const half8_t h = *reinterpret_cast<const half8_t*>(
      reinterpret_cast<const half_t*>(p.partial_o) + unit * p.head_dim + chunk * 8);
    ov0[j] = make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
    ov1[j] = make_float4((float)h[4], (float)h[5], (float)h[6], (float)h[7]);
  }
#pragma unroll
  for (int j = 0; j < S; ++j) {
    ov0[j] = make_float4(ov0[j].x * lv[j], ov0[j].y * lv[j], ov0[j].z * lv[j], ov0[j].w * lv[j]);
    ov1[j] = make_float4(ov1[j].x * lv[j], ov1[j].y * lv[j], ov1[j].z * lv[j], ov1[j].w * lv[j]);
  }
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < S; ++j) {
    if ((uint32_t)j >= nsp) {
      mv[j] = -INFINITY;
    }
    mx = fmaxf(mx, mv[j]);
  }
  float den = 0.0f;
  float4 r0 = make_float4(0.f, 0.f, 0.f, 0.f);
  float4 r1 = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int j = 0; j < S; ++j) {
    const float w = mv[j] == -INFINITY ? 0.0f : fast_exp2(mv[j] - mx);
    den = fmaf(w, lv[j], den);
    r0.x = fmaf(w, ov0[j].x, r0.x);
    r0.y = fmaf(w, ov0[j].y, r0.y);
    r0.z = fmaf(w, ov0[j].z, r0.z);
    r0.w = fmaf(w, ov0[j].w, r0.w);
    r1.x = fmaf(w, ov1[j].x, r1.x);
    r1.y = fmaf(w, ov1[j].y, r1.y);
    r1.z = fmaf(w, ov1[j].z, r1.z);
    r1.w = fmaf(w, ov1[j].w, r1.w);
  }
  const float inv = den == 0.0f ? 0.0f : 1.0f / den;
  store_gated4(p, out_index, r0, inv, gv0);
  store_gated4(p, out_index + 4, r1, inv, gv1);
}

// Many tokens with more than 16 splits (ragged batched decode): the same
// per-thread layout as attention_merge_narrow, walking a token's splits in
// batches of 8 (all loads of a batch in flight) with an online log-sum-exp, so
// a token reads only its own splits' partials.  The wide merge's thousands of
// small workgroups cost more than the partials they read at this shape.
__global__ __launch_bounds__(256) void attention_merge_tokens(CombineArgs p) {
  constexpr int B = 8;
  const uint32_t chunks = p.head_dim / 4;
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (size_t)p.tokens * p.heads * chunks) {
    return;
  }
  const uint32_t chunk = (uint32_t)(idx % chunks);
  const size_t th = idx / chunks;  // token * heads + head
  const uint32_t head = (uint32_t)(th % p.heads);
  const uint32_t token = (uint32_t)(th / p.heads);
  const uint32_t group = p.heads / p.kv_heads;
  const uint32_t kvh = head / group;
  const uint32_t g = head % group;
  const size_t base = (size_t)token * p.kv_heads + kvh;
  const uint32_t nsp = token_splits(p, token);
  const size_t out_index = th * p.head_dim + chunk * 4;
  const float4 gv = load_gate4(p.gate, out_index, true);
  float mx = -INFINITY;
  float den = 0.0f;
  float4 r = make_float4(0.f, 0.f, 0.f, 0.f);
  for (uint32_t s0 = 0; s0 < nsp; s0 += B) {
    float mv[B], lv[B];
    float4 ov[B];
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const uint32_t s = min(s0 + j, nsp - 1u);
      const size_t unit = (base * p.splits + s) * group + g;
      mv[j] = p.partial_ml[unit * 2];
      lv[j] = p.partial_ml[unit * 2 + 1];
      ov[j] = *reinterpret_cast<const float4*>(p.partial_o + unit * p.head_dim + chunk * 4);
    }
    float bmx = mx;
#pragma unroll
    for (int j = 0; j < B; ++j) {
      if (s0 + j >= nsp) {
        mv[j] = -INFINITY;
      }
      bmx = fmaxf(bmx, mv[j]);
    }
    const float f = mx == -INFINITY ? 0.0f : fast_exp2(mx - bmx);
    den *= f;
    r.x *= f;
    r.y *= f;
    r.z *= f;
    r.w *= f;
    mx = bmx;
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const float w = mv[j] == -INFINITY ? 0.0f : fast_exp2(mv[j] - mx);
      den = fmaf(w, lv[j], den);
      r.x = fmaf(w, ov[j].x, r.x);
      r.y = fmaf(w, ov[j].y, r.y);
      r.z = fmaf(w, ov[j].z, r.z);
      r.w = fmaf(w, ov[j].w, r.w);
    }
  }
  const float inv = den == 0.0f ? 0.0f : 1.0f / den;
  store_gated4(p, out_index, r, inv, gv);
}

hipError_t launch_attention_combine(const CombineArgs& c, hipStream_t stream) {
  if (c.splits > kMaxSplits || c.head_dim % kMergeDims != 0) {
    return hipErrorInvalidValue;
  }
  if (c.partial_f16 != 0 && c.splits > 16) {
    return hipErrorInvalidValue;
  }
  if (c.splits <= 16) {
    const size_t threads = (size_t)c.tokens * c.heads * (c.head_dim / 4);
    const dim3 grid((uint32_t)((threads + 255) / 256));
    if (c.partial_f16 != 0 && c.head_dim % 8 == 0) {
      const size_t threads8 = (size_t)c.tokens * c.heads * (c.head_dim / 8);
      const dim3 grid8((uint32_t)((threads8 + 255) / 256));
      if (c.splits <= 4) {
        attention_merge_narrow_f16x8<4><<<grid8, 256, 0, stream>>>(c);
      } else if (c.splits <= 8) {
        attention_merge_narrow_f16x8<8><<<grid8, 256, 0, stream>>>(c);
      } else {
        attention_merge_narrow_f16x8<16><<<grid8, 256, 0, stream>>>(c);
      }
    } else if (c.partial_f16 != 0) {
      if (c.splits <= 4) {
        attention_merge_narrow<4, true><<<grid, 256, 0, stream>>>(c);
      } else if (c.splits <= 8) {
        attention_merge_narrow<8, true><<<grid, 256, 0, stream>>>(c);
      } else {
        attention_merge_narrow<16, true><<<grid, 256, 0, stream>>>(c);
      }
    } else if (c.splits <= 4) {
      attention_merge_narrow<4, false><<<grid, 256, 0, stream>>>(c);
    } else if (c.splits <= 8) {
      attention_merge_narrow<8, false><<<grid, 256, 0, stream>>>(c);
    } else {
      attention_merge_narrow<16, false><<<grid, 256, 0, stream>>>(c);
    }
    return hipGetLastError();
  }
  // Enough (token, head) rows to fill the chip with one thread per 4 dims:
  // walk each token's splits; otherwise spread one token's splits over a
  // workgroup per 16-dim slice.
  const size_t threads = (size_t)c.tokens * c.heads * (c.head_dim / 4);
  if (threads >= 256u * 64u) {
    attention_merge_tokens<<<dim3((uint32_t)((threads + 255) / 256)), 256, 0, stream>>>(c);
    return hipGetLastError();
  }
  const dim3 grid(c.tokens, c.heads, c.head_dim / kMergeDims);
  attention_merge<<<grid, 256, 0, stream>>>(c);
  return hipGetLastError();
}

// The tuned kernel's buffer offsets are 32-bit: a split's byte span plus the
// two prefetched steps past its end must stay below 2^31.
bool offsets_fit(const AttentionArgs& a, const SplitPlan& plan) {
  const uint64_t row_bytes = (uint64_t)a.kv_heads * a.head_dim * (a.kv_f16 ? 2u : 4u);
  // At most 128 keys per round (D=64, f16), two rounds ahead of the last one.
  return ((uint64_t)plan.keys_per_split + 3u * 128u) * row_bytes < (1ull << 31);
}

bool use_tuned(const AttentionArgs& a, const SplitPlan& plan) {
  return tuned_args(a) && offsets_fit(a, plan);
}

size_t attention_decode_workspace_bytes(const AttentionArgs& a, int cu_count) {
  const SplitPlan plan = plan_splits(a, cu_count);
  if (!use_tuned(a, plan)) {
    return 0;
  }
  return data_bytes(a, plan);
}

hipError_t launch_attention_decode(const AttentionArgs& a, int cu_count, void* workspace,
                                   size_t workspace_bytes, hipStream_t stream) {
  const uint32_t g = a.heads / a.kv_heads;
  DecodeParams p{};
  p.query = a.query;
  p.key_cache = a.key_cache;
  p.value_cache = a.value_cache;
  p.gate = a.gate;
  p.output = a.output;
  p.layer = a.layer;
  p.start_position = a.start_position;
  p.tokens = a.tokens;
  p.capacity_tokens = a.capacity_tokens;
  p.heads = a.heads;
  p.kv_heads = a.kv_heads;
  p.scale_log2 = (1.0f / sqrtf((float)a.head_dim)) * kLog2e;
  p.seq_kv_offsets = a.seq_kv_offsets;
  p.seq_positions = a.seq_positions;
  p.pool_elems = a.pool_elems;
  const SplitPlan plan = plan_splits(a, cu_count);
  const bool tuned = use_tuned(a, plan);
  if (a.seq_positions != nullptr && !tuned) {
    return hipErrorInvalidValue;  // ragged decode runs on the tuned kernel only
  }
  p.splits = 1;
  if (tuned) {
    p.keys_per_split = plan.keys_per_split;
    p.splits = plan.splits;
    if (plan.splits > 1) {
      if (workspace == nullptr || workspace_bytes < data_bytes(a, plan)) {
        return hipErrorInvalidValue;
      }
      const size_t units = (size_t)a.tokens * a.kv_heads;
      p.part_o = static_cast<float*>(workspace);
      p.part_ml = p.part_o + units * plan.splits * g * a.head_dim;
    }
    if (a.seq_positions != nullptr) {
      if (workspace == nullptr || workspace_bytes < data_bytes(a, plan)) {
        return hipErrorInvalidValue;
      }
      uint2* items = reinterpret_cast<uint2*>(static_cast<char*>(workspace) +
                                              (partial_bytes(a, plan) + 255u) / 256u * 256u);
      p.work_items = items;
      ragged_plan_kernel<<<1, 256, 0, stream>>>(a.seq_positions, a.tokens, a.kv_heads,
                                                plan.keys_per_split, plan.splits,
                                                (uint32_t)work_item_count(a, plan), items);
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess) {
        return e;
      }
    }
  }
  return a.kv_f16 ? dispatch_kv<half_t>(p, a.head_dim, g, tuned, stream)
                  : dispatch_kv<float>(p, a.head_dim, g, tuned, stream);
}

hipError_t launch_attention_prologue_decode(const PrologueArgs& a, uint32_t layer,
                                            uint32_t start_position, uint32_t capacity_tokens,
                                            float* output, hipStream_t stream) {
  // The contract of the folded kernel: what the two-launch form would run on
  // the short-split kernel with one split (no kernel or split-size override).
  const char* kernel_env = std::getenv("KRAKEN_DECODE_KERNEL");
  if (a.tokens != 1 || a.head_dim != kMD || a.kv_heads == 0 || a.heads % a.kv_heads != 0 ||
      (uint64_t)start_position + 1u > kSingleSplitKeys || start_position >= capacity_tokens ||
      std::getenv("KRAKEN_DECODE_KEYS_PER_SPLIT") != nullptr ||
      (kernel_env != nullptr && std::strcmp(kernel_env, "short") != 0) ||
      !aligned16(a.key_cache) || !aligned16(a.value_cache) || !aligned16(output)) {
    return hipErrorNotSupported;
  }
  const uint32_t g = a.heads / a.kv_heads;
  if (g != 1 && g != 2 && g != 4) {
    return hipErrorNotSupported;
  }
  DecodeParams p{};
  p.key_cache = a.key_cache;
  p.value_cache = a.value_cache;
  p.output = output;
  p.layer = layer;
  p.start_position = start_position;
  p.tokens = 1;
  p.capacity_tokens = capacity_tokens;
  p.heads = a.heads;
  p.kv_heads = a.kv_heads;
  p.keys_per_split = start_position + 1u;
  p.splits = 1;
  p.scale_log2 = (1.0f / sqrtf((float)a.head_dim)) * kLog2e;
  PrologueFold f{};
  f.q_gate = a.q_gate;
  f.key = a.key;
  f.value = a.value;
  f.q_norm = a.q_norm;
  f.k_norm = a.k_norm;
  f.rope = RopeArgs{a.positions, a.mrope_start, 1u, a.n_dims, a.s0, a.s1, a.s2, a.s3, a.theta};
  f.eps = a.eps;
  return launch_decode_short_prologue(p, f, g, stream);
}

hipError_t launch_f16_to_f32(const void* in, float* out, size_t count, hipStream_t stream) {
  if (count == 0) {
    return hipSuccess;
  }
  f16_to_f32_kernel<<<dim3((uint32_t)((count + 255u) / 256u)), 256, 0, stream>>>(
    static_cast<const half_t*>(in), out, (uint64_t)count);
  return hipGetLastError();
}

}  // namespace kraken
