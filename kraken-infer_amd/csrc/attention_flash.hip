// flash256: causal GQA chunked-prefill attention for head_dim 256 over an F16
// KV cache, on fp16 MFMA (v_mfma_f32_32x32x16_f16) with an fp32 online softmax.
//
// Semantics: reference MSL attention_f32_batched_flash256_f16_kv
// (mps_backend.mm:3398-3643) -- f32 query rounded to f16 (mps_backend.mm:3458-3461),
// S = Q K^T in fp32, mask key > position or key >= key_count, online softmax,
// O = P V with fp32 accumulation, out = O / l.  Deliberate difference: P enters
// the PV product as f16 (the reference keeps it f32); P is at most 2^8 (see the
// lazy rescale below), so the rounding stays inside the 2e-3 relative / 1e-3
// absolute contract.
//
// Layout of the work (gfx950, wave64):
//  * A workgroup takes one KV head, a tile of 32 query tokens and a key split;
//    its G waves are the G query heads of the GQA group, so K/V tiles staged in
//    LDS serve G x 32 query rows.  Two workgroups share a CU (each wave stays
//    within 256 registers, each workgroup within 80 KB of LDS), so one
//    workgroup's staging and softmax overlap the other's MFMAs.
//  * K/V are staged 64 keys at a time; each 64-key tile is consumed in two
//    32-key steps.  Per step a wave computes S^T = K Q^T (keys x queries, one
//    32x32 MFMA tile over 16 k-steps of 16 dims): lane l owns query column l%32.
//    The accumulator's registers are already the B operand of the next product:
//    O^T = V^T P^T (dims x queries, 8 tiles of 32 dims, 2 k-steps of 16 keys),
//    so P never moves between lanes.
//  * Lazy rescale: scores live in the log2 domain with the 1/sqrt(D) scale
//    folded into the exp2 argument; a query's reference max moves (and O, l are
//    rescaled) only when a step's max exceeds it by more than 8, so P <= 2^8.
//  * K is staged row-major (padded rows, conflict-free 16-byte fragment reads);
//    V is staged transposed (V^T[dim][key]) with 4-key quads XOR-swizzled by
//    dim / 8, which keeps both the transposing writes and the 8-byte fragment
//    reads free of (almost all) bank conflicts.
//  * Tiles wholly inside every query's causal window skip the masking.
//  * Key splits (when the grid would not fill the chip) write (m, l, O) partials
//    in the decode path's layout; the decode combine pass merges them.  The
//    workgroup order is XCD-aware: the dispatcher deals workgroup i to XCD i % 8,
//    so work items are renumbered to give each XCD a contiguous run of
//    (split, query tile) items that share K/V in its L2.
//
// MFMA 32x32x16 lane layout (gfx950): A[i][k]: lane l holds row i = l%32, k =
// 8*(l/32) + j (j < 8).  B[k][n]: lane l holds column n = l%32, same k.  C: lane l
// holds column n = l%32, rows 8*(r/4) + 4*(l/32) + r%4 for r < 16.  Any fixed
// relabelling of k that A and B share leaves the product unchanged; the kernel
// relabels k so that B = P^T comes straight from the S^T accumulator.
#include <hip/hip_runtime.h>

#include <cstdlib>

#include "context_internal.hpp"
#include "device_common.hpp"

namespace kraken {
namespace {

constexpr int kD = 256;
constexpr int kQTile = 32;       // query tokens per workgroup
constexpr int kKTile = 64;       // keys per LDS tile
constexpr int kKRow = kD + 8;    // padded K row (halfs)
constexpr int kVRow = kKTile + 4;  // padded V^T row (halfs)
constexpr float kRescaleSlack = 8.0f;  // log2 headroom before O is rescaled

struct FlashParams {
  const float* query;
  const half_t* key_cache;
  const half_t* value_cache;
  const float* gate;
  float* output;
  float* partial_o;   // [tokens][kv_heads][splits][G][D]
  float* partial_ml;  // [tokens][kv_heads][splits][G][2]
  uint32_t layer, start_position, tokens, capacity_tokens, heads, kv_heads;
  uint32_t key_count, keys_per_split, splits, q_tiles;
  float scale_log2;
};

__device__ __forceinline__ float sigmoid_acc(float x) { return 1.0f / (1.0f + expf(-x)); }

// Row of C (32x32 accumulator) held in register r by a lane in half h.
__device__ __forceinline__ int c_row(int r, int h) { return (r >> 2) * 8 + h * 4 + (r & 3); }

// Half offset of 4-key quad `q` of V^T row `d` (quads XOR-swizzled by d / 8).
__device__ __forceinline__ int vt_offset(int d, int q) {
  return d * kVRow + 4 * (q ^ ((d >> 3) & 15));
}

// Scheduling constraint for a run of N (LDS fragment read, MFMA) pairs: the
// first kLookahead reads, then one MFMA per read, then the last MFMAs.  Keeps
// kLookahead fragments in flight instead of all N (sched_group_barrier masks:
// 0x008 MFMA, 0x100 LDS read).
constexpr int kLookahead = 3;
template <int N>
__device__ __forceinline__ void pipeline_reads_and_mfma() {
#pragma unroll
  for (int i = 0; i < kLookahead; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
  }
#pragma unroll
  for (int i = 0; i < N - kLookahead; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
  }
#pragma unroll
  for (int i = 0; i < kLookahead; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
  }
}

template <int G>
__global__ __launch_bounds__(64 * G) __attribute__((amdgpu_waves_per_eu(2)))
void flash256_kernel(FlashParams p) {
  __shared__ __attribute__((aligned(16))) half_t s_k[kKTile * kKRow];
  __shared__ __attribute__((aligned(16))) half_t s_vt[kD * kVRow];

  constexpr int kThreads = 64 * G;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int h = lane >> 5;  // lane half
  const int n = lane & 31;  // query column owned by this lane

  // XCD-aware renumbering of the linear workgroup id (see header), then the
  // work item (kv head, split, query tile) with query tiles fastest and the
  // heaviest (latest) query tiles first within a split.
  const uint32_t total = p.q_tiles * p.kv_heads * p.splits;
  const uint32_t lin = blockIdx.x;
  const uint32_t per_xcd = total / 8u;
  const uint32_t rem = total % 8u;
  const uint32_t xcd = lin % 8u;
  const uint32_t slot = lin / 8u;
  const uint32_t item = xcd * per_xcd + min(xcd, rem) + slot;
  const uint32_t q_tile = p.q_tiles - 1u - item % p.q_tiles;
  const uint32_t split = (item / p.q_tiles) % p.splits;
  const uint32_t kvh = item / (p.q_tiles * p.splits);
  const uint32_t head = kvh * G + wave;
  const uint32_t t0 = q_tile * kQTile;
  const uint32_t token = t0 + n;
  const bool token_ok = token < p.tokens;
  const uint32_t position = p.start_position + token;
  const uint32_t first_position = p.start_position + t0;

  // Keys this workgroup may need: causal limit of its last token.
  uint32_t block_keys = p.start_position + min(p.tokens, t0 + kQTile);
  if (block_keys > p.key_count) {
    block_keys = p.key_count;
  }
  const uint32_t key_begin = split * p.keys_per_split;
  uint32_t key_end = key_begin + p.keys_per_split;
  if (key_end > block_keys) {
    key_end = block_keys;
  }

  // Q^T as the B operand of S^T = K Q^T: lane holds query n, dims 16*step + 8*h + j.
  half8_t qf[kD / 16];
  {
    const float* qrow = p.query + ((size_t)(token_ok ? token : 0) * p.heads + head) * kD;
#pragma unroll
    for (int step = 0; step < kD / 16; ++step) {
      const int d0 = step * 16 + h * 8;
      float4 a = token_ok ? *reinterpret_cast<const float4*>(qrow + d0) : make_float4(0, 0, 0, 0);
      float4 b = token_ok ? *reinterpret_cast<const float4*>(qrow + d0 + 4) : make_float4(0, 0, 0, 0);
      qf[step] = half8_t{(half_t)a.x, (half_t)a.y, (half_t)a.z, (half_t)a.w,
                         (half_t)b.x, (half_t)b.y, (half_t)b.z, (half_t)b.w};
    }
  }

  float16_t o[kD / 32];  // O^T tiles: dims 32*dt + c_row(r, h), query n
#pragma unroll
  for (int dt = 0; dt < kD / 32; ++dt) {
    o[dt] = float16_t{};
  }
  float m = -INFINITY;  // reference max (log2 domain, scaled) of query n
  float l = 0.0f;       // this lane's share of the denominator (relative to m)
  const float c = p.scale_log2;

  // V^T fragment reads: quad q = 8*half + 4*ks + h (+2 for the high four keys) of
  // row d = 32*dt + n.  Bits 2..3 of q ^ swizzle(d) depend only on the unrolled
  // (half, ks, dt), bits 0..1 only on the lane, so each read is a per-lane base
  // plus an immediate offset.
  const int vt_lo = n * kVRow + 4 * (h ^ (n >> 3));
  const int vt_hi = n * kVRow + 4 * ((h | 2) ^ (n >> 3));

  // K/V rows of this layer through range-checked buffer resources: rows at or
  // past key_end read as zeros without a memory access (the host keeps every
  // byte offset below 2^31).
  const uint32_t row_bytes = p.kv_heads * kD * 2u;
  const size_t layer_elems = (size_t)p.layer * p.capacity_tokens * p.kv_heads * kD;
  const __amdgpu_buffer_rsrc_t krsrc =
    make_buffer_rsrc(p.key_cache + layer_elems, key_end * row_bytes);
  const __amdgpu_buffer_rsrc_t vrsrc =
    make_buffer_rsrc(p.value_cache + layer_elems, key_end * row_bytes);
  const uint32_t head_bytes = kvh * kD * 2u;

  for (uint32_t kt = key_begin; kt < key_end; kt += kKTile) {
    // ---- stage K (row-major) and V^T into LDS ----
    // (Staging is only partly unrolled: Q and O already hold 192 registers.)
    __syncthreads();
#pragma unroll 2
    for (int idx = tid; idx < kKTile * (kD / 8); idx += kThreads) {
      const int key = idx / (kD / 8);
      const int ch = idx % (kD / 8);
      const u32x4_t v = __builtin_bit_cast(
        u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                   krsrc, (int)((kt + key) * row_bytes + head_bytes + ch * 16u), 0, 0));
      *reinterpret_cast<u32x4_t*>(&s_k[key * kKRow + ch * 8]) = v;
    }
#pragma unroll 1
    for (int idx = tid; idx < (kKTile / 4) * (kD / 8); idx += kThreads) {
      const int kq = idx / (kD / 8);  // key quad
      const int dq = idx % (kD / 8);  // dim octet
      half8_t rows[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t key = kt + kq * 4 + r;
        rows[r] = __builtin_bit_cast(
          half8_t, __builtin_amdgcn_raw_buffer_load_b128(
                     vrsrc, (int)(key * row_bytes + head_bytes + dq * 16u), 0, 0));
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const half4_t col = half4_t{rows[0][i], rows[1][i], rows[2][i], rows[3][i]};
        *reinterpret_cast<half4_t*>(&s_vt[vt_offset(dq * 8 + i, kq)]) = col;
      }
    }
    __syncthreads();

    // Whole tile inside every query's causal window and the split: no masking.
    const bool full = kt + kKTile <= key_end && kt + kKTile - 1u <= first_position;

#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const uint32_t kh0 = kt + half * 32;
      // ---- S^T = K Q^T for 32 keys x 32 queries ----
      float16_t s = float16_t{};
#pragma unroll
      for (int step = 0; step < kD / 16; ++step) {
        const half8_t a =
          *reinterpret_cast<const half8_t*>(&s_k[(half * 32 + n) * kKRow + step * 16 + h * 8]);
        s = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[step], s, 0, 0, 0);
      }
      // Pipeline the fragment reads kLookahead MFMAs ahead (register budget).
      pipeline_reads_and_mfma<kD / 16>();

      // ---- mask, lazy online softmax (log2 domain) ----
      if (!full) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const uint32_t key = kh0 + c_row(r, h);
          const bool valid = key < key_end && key <= position;
          s[r] = valid ? s[r] : -INFINITY;
        }
      }
      float mx = s[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) {
        mx = fmaxf(mx, s[r]);
      }
      mx = xor32_max(mx) * c;  // this step's max for query n (both lane halves)
      const bool need = mx > m + kRescaleSlack;
      if (__builtin_amdgcn_ballot_w64(need) != 0) {
        const float m_new = need ? mx : m;
        const float corr = need ? fast_exp2(m - m_new) : 1.0f;  // m = -inf -> 0
        l *= corr;
#pragma unroll
        for (int dt = 0; dt < kD / 32; ++dt) {
          o[dt] *= corr;
        }
        m = m_new;
      }
      // A query with no valid key yet keeps m = -inf; its scores are all -inf.
      const float neg_m = m == -INFINITY ? 0.0f : -m;
      half8_t pb[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pr = fast_exp2(fmaf(s[r], c, neg_m));
        l += pr;
        pb[r >> 3][r & 7] = (half_t)pr;
      }

      // ---- O^T += V^T P^T: k-step ks covers keys 16*ks .. 16*ks+15 of this step ----
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
        for (int dt = 0; dt < kD / 32; ++dt) {
          // == vt_offset(32*dt + n, 8*half + 4*ks + h (+2))
          const int imm = dt * 32 * kVRow + 16 * ((2 * half + ks) ^ (dt & 3));
          const half4_t lo = *reinterpret_cast<const half4_t*>(&s_vt[vt_lo + imm]);
          const half4_t hi = *reinterpret_cast<const half4_t*>(&s_vt[vt_hi + imm]);
          const half8_t a = half8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb[ks], o[dt], 0, 0, 0);
        }
      }
      pipeline_reads_and_mfma<2 * (kD / 32)>();
    }
  }

  l = xor32_sum(l);  // both lane halves hold keys of query n
  if (!token_ok) {
    return;
  }
  // ---- epilogue: lane owns query n; dims 32*dt + c_row(r, h) ----
  if (p.splits == 1) {
    const float inv = l == 0.0f ? 0.0f : 1.0f / l;
    float* orow = p.output + ((size_t)token * p.heads + head) * kD;
    const float* grow = p.gate != nullptr ? p.gate + ((size_t)token * p.heads + head) * kD : nullptr;
#pragma unroll
    for (int dt = 0; dt < kD / 32; ++dt) {
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = dt * 32 + r4 * 8 + h * 4;
        float4 v = make_float4(o[dt][r4 * 4 + 0] * inv, o[dt][r4 * 4 + 1] * inv,
                               o[dt][r4 * 4 + 2] * inv, o[dt][r4 * 4 + 3] * inv);
        if (grow != nullptr) {
          const float4 g = *reinterpret_cast<const float4*>(grow + d);
          v.x *= sigmoid_acc(g.x);
          v.y *= sigmoid_acc(g.y);
          v.z *= sigmoid_acc(g.z);
          v.w *= sigmoid_acc(g.w);
        }
        *reinterpret_cast<float4*>(orow + d) = v;
      }
    }
  } else {
    const size_t base = (((size_t)token * p.kv_heads + kvh) * p.splits + split) * G + wave;
    float* po = p.partial_o + base * kD;
#pragma unroll
    for (int dt = 0; dt < kD / 32; ++dt) {
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = dt * 32 + r4 * 8 + h * 4;
        *reinterpret_cast<float4*>(po + d) =
          make_float4(o[dt][r4 * 4 + 0], o[dt][r4 * 4 + 1], o[dt][r4 * 4 + 2], o[dt][r4 * 4 + 3]);
      }
    }
    if (h == 0) {
      p.partial_ml[base * 2 + 0] = m;
      p.partial_ml[base * 2 + 1] = l;
    }
  }
}

struct FlashPlan {
  uint32_t q_tiles, keys_per_split, splits;
};

FlashPlan plan_flash(const AttentionArgs& a, int cu_count) {
  FlashPlan plan{};
  plan.q_tiles = (a.tokens + kQTile - 1) / kQTile;
  const uint32_t key_count = a.start_position + a.tokens;
  const uint64_t units = (uint64_t)plan.q_tiles * a.kv_heads;
  // Two workgroups per CU.
  const uint64_t target = 2u * (uint64_t)(cu_count > 0 ? cu_count : 256);
  uint64_t splits = (target + units - 1) / units;
  if (const char* env = std::getenv("KRAKEN_FLASH_SPLITS")) {
    const long v = std::strtol(env, nullptr, 10);
    if (v > 0) {
      splits = (uint64_t)v;
    }
  }
  // Every split must hold at least two key tiles of the longest query tile.
  const uint64_t max_useful = (key_count + 2 * kKTile - 1) / (2 * kKTile);
  if (splits > max_useful) {
    splits = max_useful;
  }
  if (splits < 1) {
    splits = 1;
  }
  uint64_t kps = (key_count + splits - 1) / splits;
  kps = (kps + kKTile - 1) / kKTile * kKTile;
  plan.keys_per_split = (uint32_t)kps;
  plan.splits = (uint32_t)((key_count + kps - 1) / kps);
  return plan;
}

template <int G>
hipError_t launch_g(const FlashParams& p, hipStream_t stream) {
  const dim3 grid(p.q_tiles * p.kv_heads * p.splits);
  flash256_kernel<G><<<grid, 64 * G, 0, stream>>>(p);
  return hipGetLastError();
}

}  // namespace

bool flash_prefill_supported(const AttentionArgs& a) {
  const uint32_t g = a.heads / a.kv_heads;
  // Buffer offsets are 32-bit signed: every key row of the layer (plus one
  // 64-key tile of overrun) must lie below 2^31 bytes.
  const uint64_t row_bytes = (uint64_t)a.kv_heads * 256u * 2u;
  const uint64_t keys = (uint64_t)a.start_position + a.tokens + kKTile;
  return a.kv_f16 && a.head_dim == 256 && (g == 1 || g == 2 || g == 4 || g == 8) &&
         keys * row_bytes < (1ull << 31) &&
         ((uintptr_t)a.query & 15u) == 0 && ((uintptr_t)a.key_cache & 15u) == 0 &&
         ((uintptr_t)a.value_cache & 15u) == 0 && ((uintptr_t)a.output & 15u) == 0 &&
         (a.gate == nullptr || ((uintptr_t)a.gate & 15u) == 0);
}

size_t attention_flash_workspace_bytes(const AttentionArgs& a, int cu_count) {
  const FlashPlan plan = plan_flash(a, cu_count);
  if (plan.splits <= 1) {
    return 0;
  }
  const size_t units = (size_t)a.tokens * a.heads * plan.splits;
  return kCounterRegionBytes + units * (kD + 2) * sizeof(float);
}

hipError_t launch_attention_flash(const AttentionArgs& a, int cu_count, void* workspace,
                                  size_t workspace_bytes, hipStream_t stream) {
  const FlashPlan plan = plan_flash(a, cu_count);
  FlashParams p{};
  p.query = a.query;
  p.key_cache = static_cast<const half_t*>(a.key_cache);
  p.value_cache = static_cast<const half_t*>(a.value_cache);
  p.gate = a.gate;
  p.output = a.output;
  p.layer = a.layer;
  p.start_position = a.start_position;
  p.tokens = a.tokens;
  p.capacity_tokens = a.capacity_tokens;
  p.heads = a.heads;
  p.kv_heads = a.kv_heads;
  p.key_count = a.start_position + a.tokens;
  p.keys_per_split = plan.keys_per_split;
  p.splits = plan.splits;
  p.q_tiles = plan.q_tiles;
  p.scale_log2 = (1.0f / sqrtf(256.0f)) * kLog2e;
  if (plan.splits > 1) {
    const size_t units = (size_t)a.tokens * a.heads * plan.splits;
    if (workspace == nullptr ||
        workspace_bytes < kCounterRegionBytes + units * (kD + 2) * sizeof(float)) {
      return hipErrorInvalidValue;
    }
    // Partials follow the counter region, which they must never overlap.
    p.partial_o = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterRegionBytes);
    p.partial_ml = p.partial_o + units * kD;
  }
  const uint32_t g = a.heads / a.kv_heads;
  hipError_t e;
  switch (g) {
    case 1: e = launch_g<1>(p, stream); break;
    case 2: e = launch_g<2>(p, stream); break;
    case 4: e = launch_g<4>(p, stream); break;
    case 8: e = launch_g<8>(p, stream); break;
    default: return hipErrorInvalidValue;
  }
  if (e != hipSuccess || plan.splits == 1) {
    return e;
  }
  CombineArgs c{};
  c.partial_o = p.partial_o;
  c.partial_ml = p.partial_ml;
  c.gate = a.gate;
  c.output = a.output;
  c.tokens = a.tokens;
  c.heads = a.heads;
  c.kv_heads = a.kv_heads;
  c.splits = plan.splits;
  c.head_dim = kD;
  c.positions = nullptr;
  c.start_position = a.start_position;
  c.keys_per_split = plan.keys_per_split;
  return launch_attention_combine(c, stream);
}

}  // namespace kraken
