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
//  * A workgroup takes one KV head, up to four query heads of its GQA group
//    ("head slots"), a tile of 32 query tokens and a key split.  It has two
//    waves per head slot, so a CU runs one workgroup of 8 waves, two per SIMD.
//    Wave dh of a pair computes the scores of keys 32 dh .. 32 dh + 31 of every
//    64-key tile and accumulates output dims 128 dh .. 128 dh + 127 over all 64
//    keys: the pair swaps its tile maxima and its P halves through LDS.  The
//    split of O by dims keeps each wave within the 256 registers that two waves
//    per SIMD allow (Q 64 + O 64 + scores and P 32, with room for the fragment
//    read pipeline); both waves of a pair make the same softmax decisions from
//    the same maxima, so they share one reference max per query.
//  * K/V tiles are copied global -> LDS by the gfx950 direct-to-LDS buffer loads
//    (buffer_load_dwordx4 ... lds), double-buffered: the next tile's copy is in
//    flight while the current one is consumed, and no register holds staging
//    data.  Rows stay in their row-major layout (512 bytes per key); the 16-byte
//    chunks of each row are XOR-swizzled (K by row % 16, V by 4 * (row % 4)) by
//    choosing which global chunk each lane fetches, which keeps the fragment
//    reads below free of bank conflicts.
//  * Per tile a wave computes S^T = K Q^T for its 32 keys (keys x queries, one
//    32x32 MFMA tile over 16 k-steps of 16 dims; lane l owns query column l%32).
//    The accumulator's registers are already the B operand of the next product,
//    O^T = V^T P^T (dims x queries, 4 tiles of 32 dims, 4 k-steps of 16 keys): a
//    lane's P values are the B operand as they stand, and the partner's P comes
//    from the same lane of the partner, so P never moves between lanes.  The V^T
//    operand comes straight from the row-major V tile through the gfx950
//    transposing LDS read ds_read_b64_tr_b16.
//  * Lazy rescale: scores live in the log2 domain with the 1/sqrt(D) scale
//    folded into the exp2 argument; a query's reference max moves (and O, l are
//    rescaled) only when a tile's max exceeds it by more than 8, so P <= 2^8.
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
//
// ds_read_b64_tr_b16 (gfx950; lane layout checked on the device): within each
// group of 16 lanes, result lane l' gets element e (e < 4) = the 16-bit value at
// (address supplied by lane 4e + l'/4 of the group) + (l' % 4).  So if lane
// 4e + q points at row e, columns 4q..4q+3 of a 4 x 16 block, lane l' receives
// column l' of that block.
//
// buffer_load_dwordx4 ... lds (gfx950): lane l's 16 bytes are written to LDS at
// M0 + 16 l (M0 = the wave-uniform LDS pointer); an offset at or past the
// resource's byte count returns zeros without a memory access.
#include <hip/hip_runtime.h>

#include <cstdlib>

#include "context_internal.hpp"
#include "device_common.hpp"

namespace kraken {
namespace {

constexpr int kD = 256;
constexpr int kQTile = 32;             // query tokens per workgroup
constexpr int kKTile = 64;             // keys per LDS tile (two 32-key halves)
constexpr int kRowHalfs = kD;          // an LDS row is a whole 512-byte key row
constexpr int kTileHalfs = kKTile * kRowHalfs;  // 32 KB per K or V tile
constexpr float kRescaleSlack = 8.0f;  // log2 headroom before O is rescaled

typedef __attribute__((address_space(3))) void lds_void_t;
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t lds_short4_t;

// Transposing 8-byte LDS read (ds_read_b64_tr_b16) of four 16-bit values.
__device__ __forceinline__ half4_t read_tr16(const half_t* lds_address) {
  return __builtin_bit_cast(half4_t,
                            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)lds_address));
}

struct FlashParams {
  const float* query;
  const half_t* key_cache;
  const half_t* value_cache;
  const float* gate;
  float* output;
  float* partial_o;   // [tokens][kv_heads][splits][G][D]
  float* partial_ml;  // [tokens][kv_heads][splits][G][2]
  uint32_t layer, start_position, tokens, capacity_tokens, heads, kv_heads;
  uint32_t key_count, keys_per_split, splits, q_tiles, head_groups;
  float scale_log2;
};

__device__ __forceinline__ float sigmoid_acc(float x) { return 1.0f / (1.0f + expf(-x)); }

// Row of C (32x32 accumulator) held in register r by a lane in half h.
__device__ __forceinline__ int c_row(int r, int h) { return (r >> 2) * 8 + h * 4 + (r & 3); }

// Scheduling constraint for a run of N (LDS fragment reads, MFMA) groups: the
// first kLookahead groups of reads, then one MFMA per group, then the last
// MFMAs.  Keeps kLookahead fragments in flight instead of all N
// (sched_group_barrier masks: 0x008 MFMA, 0x100 LDS read).
template <int N, int kLookahead, int kReadsPerMfma>
__device__ __forceinline__ void pipeline_reads_and_mfma() {
#pragma unroll
  for (int i = 0; i < kLookahead; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x100, kReadsPerMfma, 0);
  }
#pragma unroll
  for (int i = 0; i < N - kLookahead; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, kReadsPerMfma, 0);
  }
#pragma unroll
  for (int i = 0; i < kLookahead; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
  }
}

typedef int i32x4_t __attribute__((ext_vector_type(4)));

// Buffer resource words (raw, stride 0) over `bytes` bytes from `base`, for the
// inline-asm copies below; base and size are made wave-uniform.
__device__ __forceinline__ i32x4_t rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4_t r;
  r[0] = (int)__builtin_amdgcn_readfirstlane((uint32_t)a);
  r[1] = (int)(__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) & 0xFFFFu);
  r[2] = (int)__builtin_amdgcn_readfirstlane(bytes);
  r[3] = 0x00020000;
  return r;
}

// One direct-to-LDS 16-byte-per-lane copy (buffer_load_dwordx4 ... lds) to the
// wave-uniform LDS address `lds`.  Issued as inline asm so that the compiler does
// not make every later LDS read wait for it (it cannot tell the copy's target
// from the stage being read); completion is awaited explicitly by
// wait_tile_copies() before the barrier that publishes a stage.  M0 is set in the
// same statement, with the one wait state the M0 -> LDS-DMA hazard needs.
__device__ __forceinline__ void copy16_to_lds(i32x4_t rsrc, uint32_t voffset, const half_t* lds) {
  const uint32_t m0 =
    __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_t*)lds);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(m0), "v"(voffset), "s"(rsrc)
               : "memory", "m0");
}

// Copies one 64-key K and V tile (keys kt..kt+63) into an LDS stage.  Row pair
// rp (rows 2 rp, 2 rp + 1: 1 KB) is one wave instruction; lane l fills physical
// chunk l % 32 of row 2 rp + l / 32 with the logical chunk that the row's
// swizzle puts there.
template <int W>
__device__ __forceinline__ void issue_tile_copy(i32x4_t krsrc, i32x4_t vrsrc, half_t* k_stage,
                                                half_t* v_stage, uint32_t kt, uint32_t row_bytes,
                                                uint32_t head_bytes, int wave, int lane) {
  const int p = lane & 31;
#pragma unroll
  for (int i = 0; i < (kKTile / 2) / W; ++i) {
    const int rp = i * W + wave;
    const int r = 2 * rp + (lane >> 5);
    const uint32_t row_off = (kt + r) * row_bytes + head_bytes;
    const int kc = p ^ (r & 15);
    const int vc = p ^ (4 * (r & 3));
    copy16_to_lds(krsrc, row_off + 16u * kc, k_stage + rp * 2 * kRowHalfs);
    copy16_to_lds(vrsrc, row_off + 16u * vc, v_stage + rp * 2 * kRowHalfs);
  }
}

__device__ __forceinline__ void wait_tile_copies() {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

template <int GW>
__global__ __launch_bounds__(128 * GW) __attribute__((amdgpu_waves_per_eu(2)))
void flash256_kernel(FlashParams p) {
  // Two stages of K and V tiles (128 KB); the pair exchange slots for tile maxima
  // (per query) and P (16 halves per lane).
  __shared__ __attribute__((aligned(16))) half_t s_tiles[2 * 2 * kTileHalfs];
  __shared__ float s_mx[GW][2][32];
  __shared__ __attribute__((aligned(16))) half8_t s_p[GW][2][64][2];

  constexpr int W = 2 * GW;  // waves
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int slot = wave % GW;    // head slot
  const int dh = wave / GW;      // key half for scores, dim half for O
  const int h = lane >> 5;       // lane half
  const int n = lane & 31;       // query column owned by this lane
  const uint32_t G = p.heads / p.kv_heads;

  // XCD-aware renumbering of the linear workgroup id (see header), then the
  // work item (kv head, head group, split, query tile) with query tiles fastest
  // and the heaviest (latest) query tiles first within a split.
  const uint32_t total = p.q_tiles * p.kv_heads * p.head_groups * p.splits;
  const uint32_t lin = blockIdx.x;
  const uint32_t per_xcd = total / 8u;
  const uint32_t rem = total % 8u;
  const uint32_t xcd = lin % 8u;
  const uint32_t item = xcd * per_xcd + min(xcd, rem) + lin / 8u;
  const uint32_t q_tile = p.q_tiles - 1u - item % p.q_tiles;
  const uint32_t split = (item / p.q_tiles) % p.splits;
  const uint32_t hg = (item / (p.q_tiles * p.splits)) % p.head_groups;
  const uint32_t kvh = item / (p.q_tiles * p.splits * p.head_groups);
  const uint32_t g_in_group = hg * GW + slot;
  const uint32_t head = kvh * G + g_in_group;
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
  if (key_begin >= key_end) {
    // No key of this split is visible to any query of the tile.  The merge reads
    // only the first ceil(keys / keys_per_split) splits of a token, which never
    // include this one, so nothing is written.
    return;
  }

  // K/V rows of this layer through range-checked buffer resources: rows at or
  // past key_end read as zeros without a memory access (the host keeps every
  // byte offset below 2^31).
  const uint32_t row_bytes = p.kv_heads * kD * 2u;
  const size_t layer_elems = (size_t)p.layer * p.capacity_tokens * p.kv_heads * kD;
  const i32x4_t krsrc = rsrc_words(p.key_cache + layer_elems, key_end * row_bytes);
  const i32x4_t vrsrc = rsrc_words(p.value_cache + layer_elems, key_end * row_bytes);
  const uint32_t head_bytes = kvh * kD * 2u;

  // The first tile's copy goes out before the query is loaded.
  issue_tile_copy<W>(krsrc, vrsrc, s_tiles, s_tiles + kTileHalfs, key_begin, row_bytes,
                     head_bytes, wave, lane);

  // Q^T as the B operand of S^T = K Q^T: lane holds query n, dims 16*step + 8*h + j.
  half8_t qf[kD / 16];
  {
    // Unconditional loads from a valid row (token 0 stands in for tokens past the
    // end), zeroed afterwards, so all 32 loads are in flight together.
    const float* qrow = p.query + ((size_t)(token_ok ? token : 0) * p.heads + head) * kD;
    const float qmask = token_ok ? 1.0f : 0.0f;
#pragma unroll
    for (int step = 0; step < kD / 16; ++step) {
      const int d0 = step * 16 + h * 8;
      const float4 a = *reinterpret_cast<const float4*>(qrow + d0);
      const float4 b = *reinterpret_cast<const float4*>(qrow + d0 + 4);
      qf[step] = half8_t{(half_t)(a.x * qmask), (half_t)(a.y * qmask), (half_t)(a.z * qmask),
                         (half_t)(a.w * qmask), (half_t)(b.x * qmask), (half_t)(b.y * qmask),
                         (half_t)(b.z * qmask), (half_t)(b.w * qmask)};
    }
  }

  constexpr int kDt = kD / 64;  // O^T tiles of 32 dims per wave (half of D)
  float16_t o[kDt];  // O^T tiles: dims 128*dh + 32*dt + c_row(r, h), query n
#pragma unroll
  for (int dt = 0; dt < kDt; ++dt) {
    o[dt] = float16_t{};
  }
  float m = -INFINITY;  // reference max (log2 domain, scaled) of query n
  float l = 0.0f;       // this lane's share (own keys) of the denominator, relative to m
  const float c = p.scale_log2;

  // K fragment reads: row dh*32 + n, logical chunk 2*step + h at physical chunk
  // (2*step + h) ^ (n % 16) = 2*step ^ u.
  const int u = h ^ (n & 15);
  const int k_row = (dh * 32 + n) * kRowHalfs;
  // V^T fragment reads (ds_read_b64_tr_b16): lane L = 16 g + 4 e + q of group g
  // (h = g / 2, 16-dim group gd = g % 2) supplies row 4h + e (+8 for the high
  // four keys, +16 per k-step, +32 for the second key half), dims
  // 128 dh + 32 dt + 16 gd + 4q, i.e. physical chunk (16 dh + 4 dt + 2 gd + q/2)
  // ^ 4e: 128 dh + 32 (dt ^ e) + 16 gd + 4q halfs.
  const int e = (lane >> 2) & 3;
  const int v_lane = (4 * h + e) * kRowHalfs + 128 * dh + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  int v_addr[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    v_addr[b] = v_lane + 32 * (b ^ e);
  }

  int stage = 0;
  for (uint32_t kt = key_begin; kt < key_end; kt += kKTile, stage ^= 1) {
    wait_tile_copies();
    __syncthreads();  // tile kt is in `stage`; every wave is done with the other stage
    if (kt + kKTile < key_end) {
      half_t* nk = s_tiles + (stage ^ 1) * 2 * kTileHalfs;
      issue_tile_copy<W>(krsrc, vrsrc, nk, nk + kTileHalfs, kt + kKTile, row_bytes, head_bytes,
                         wave, lane);
    }
    const half_t* ks_base = s_tiles + stage * 2 * kTileHalfs;
    const half_t* vs_base = ks_base + kTileHalfs;
    const uint32_t k0 = kt + dh * 32;  // first key of this wave's score half

    // ---- S^T = K Q^T for 32 keys x 32 queries ----
    float16_t s = float16_t{};
#pragma unroll
    for (int step = 0; step < kD / 16; ++step) {
      const half8_t a =
        *reinterpret_cast<const half8_t*>(&ks_base[k_row + 8 * ((2 * step) ^ u)]);
      s = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[step], s, 0, 0, 0);
    }
    pipeline_reads_and_mfma<kD / 16, 3, 1>();

    // ---- mask; tile max shared with the partner wave ----
    const bool full = k0 + 32 <= key_end && k0 + 31 <= first_position;
    if (!full) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const uint32_t key = k0 + c_row(r, h);
        const bool valid = key < key_end && key <= position;
        s[r] = valid ? s[r] : -INFINITY;
      }
    }
    float mx = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) {
      mx = fmaxf(mx, s[r]);
    }
    mx = xor32_max(mx);  // this wave's 32 keys, query n (both lane halves)
    if (h == 0) {
      s_mx[slot][dh][n] = mx;
    }
    __syncthreads();
    mx = fmaxf(s_mx[slot][0][n], s_mx[slot][1][n]) * c;  // the tile's max, same in both waves

    // ---- lazy online softmax (log2 domain) ----
    const bool need = mx > m + kRescaleSlack;
    if (__builtin_amdgcn_ballot_w64(need) != 0) {
      const float m_new = need ? mx : m;
      const float corr = need ? fast_exp2(m - m_new) : 1.0f;  // m = -inf -> 0
      l *= corr;
#pragma unroll
      for (int dt = 0; dt < kDt; ++dt) {
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
    s_p[slot][dh][lane][0] = pb[0];
    s_p[slot][dh][lane][1] = pb[1];
    __syncthreads();
    const half8_t po0 = s_p[slot][dh ^ 1][lane][0];
    const half8_t po1 = s_p[slot][dh ^ 1][lane][1];
    // P of keys 0..31 and 32..63 of the tile, as B operands (k-steps of 16 keys).
    half8_t pk[4];
    pk[0] = dh == 0 ? pb[0] : po0;
    pk[1] = dh == 0 ? pb[1] : po1;
    pk[2] = dh == 0 ? po0 : pb[0];
    pk[3] = dh == 0 ? po1 : pb[1];

    // ---- O^T += V^T P^T over the 64 keys (4 k-steps), this wave's 128 dims ----
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int dt = 0; dt < kDt; ++dt) {
        const half_t* vp = vs_base + v_addr[dt] + 16 * ks * kRowHalfs;
        const half4_t lo = read_tr16(vp);
        const half4_t hi = read_tr16(vp + 8 * kRowHalfs);
        const half8_t a = half8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pk[ks], o[dt], 0, 0, 0);
      }
    }
    pipeline_reads_and_mfma<4 * kDt, 2, 2>();
  }

  // ---- denominator: own keys (both lane halves) plus the partner's keys ----
  l = xor32_sum(l);
  __syncthreads();  // every wave is past its last read of s_mx
  if (h == 0) {
    s_mx[slot][dh][n] = l;
  }
  __syncthreads();
  l += s_mx[slot][dh ^ 1][n];
  if (!token_ok) {
    return;
  }
  // ---- epilogue: lane owns query n; dims 128*dh + 32*dt + c_row(r, h) ----
  if (p.splits == 1) {
    const float inv = l == 0.0f ? 0.0f : 1.0f / l;
    float* orow = p.output + ((size_t)token * p.heads + head) * kD;
    const float* grow = p.gate != nullptr ? p.gate + ((size_t)token * p.heads + head) * kD : nullptr;
#pragma unroll
    for (int dt = 0; dt < kDt; ++dt) {
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = dh * 128 + dt * 32 + r4 * 8 + h * 4;
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
    const size_t base = (((size_t)token * p.kv_heads + kvh) * p.splits + split) * G + g_in_group;
    float* po = p.partial_o + base * kD;
#pragma unroll
    for (int dt = 0; dt < kDt; ++dt) {
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = dh * 128 + dt * 32 + r4 * 8 + h * 4;
        *reinterpret_cast<float4*>(po + d) =
          make_float4(o[dt][r4 * 4 + 0], o[dt][r4 * 4 + 1], o[dt][r4 * 4 + 2], o[dt][r4 * 4 + 3]);
      }
    }
    if (h == 0 && dh == 0) {
      p.partial_ml[base * 2 + 0] = m;
      p.partial_ml[base * 2 + 1] = l;
    }
  }
}

struct FlashPlan {
  uint32_t q_tiles, head_groups, keys_per_split, splits;
};

constexpr uint32_t kMinKeysPerSplit = 8 * kKTile;

FlashPlan plan_flash(const AttentionArgs& a, int cu_count) {
  FlashPlan plan{};
  const uint32_t g = a.heads / a.kv_heads;
  plan.q_tiles = (a.tokens + kQTile - 1) / kQTile;
  plan.head_groups = g > 4 ? g / 4 : 1;
  const uint32_t key_count = a.start_position + a.tokens;
  const uint64_t units = (uint64_t)plan.q_tiles * a.kv_heads * plan.head_groups;
  // One workgroup (8 waves, 128 KB of LDS) per CU.
  const uint64_t target = (uint64_t)(cu_count > 0 ? cu_count : 256);
  uint64_t splits = (target + units - 1) / units;
  // A split should hold enough key tiles to amortise its query load and
  // partial write.
  const uint64_t max_useful = (key_count + kMinKeysPerSplit - 1) / kMinKeysPerSplit;
  if (splits > max_useful) {
    splits = max_useful;
  }
  if (const char* env = std::getenv("KRAKEN_FLASH_SPLITS")) {
    const long v = std::strtol(env, nullptr, 10);
    if (v > 0) {
      splits = (uint64_t)v;
    }
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

template <int GW>
hipError_t launch_g(const FlashParams& p, hipStream_t stream) {
  const dim3 grid(p.q_tiles * p.kv_heads * p.head_groups * p.splits);
  flash256_kernel<GW><<<grid, 128 * GW, 0, stream>>>(p);
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
  p.head_groups = plan.head_groups;
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
    case 4:
    case 8: e = launch_g<4>(p, stream); break;
    default: return hipErrorInvalidValue;
  }
  if (e != hipSuccess || plan.splits == 1) {
    return e;
  }
  CombineArgs cmb{};
  cmb.partial_o = p.partial_o;
  cmb.partial_ml = p.partial_ml;
  cmb.gate = a.gate;
  cmb.output = a.output;
  cmb.tokens = a.tokens;
  cmb.heads = a.heads;
  cmb.kv_heads = a.kv_heads;
  cmb.splits = plan.splits;
  cmb.head_dim = kD;
  cmb.positions = nullptr;
  cmb.start_position = a.start_position;
  cmb.keys_per_split = plan.keys_per_split;
  return launch_attention_combine(cmb, stream);
}

}  // namespace kraken
