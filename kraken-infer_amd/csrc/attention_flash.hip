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
//    ("head slots"), a tile of 32 query tokens and a key split: one wave per
//    head slot, one workgroup (128 KB of LDS) per CU, so each wave owns a SIMD
//    and its 512 registers (Q 64, O 128, two score tiles 64, P 16, fragment read
//    pipelines).
//  * K and V tiles (64 keys) are copied global -> LDS by the gfx950
//    direct-to-LDS buffer loads (buffer_load_dwordx4 ... lds), double buffered,
//    so no register holds staging data.  Rows stay row-major (512 bytes per
//    key); the 16-byte chunks of each row are XOR-swizzled (K by row % 16, V by
//    4 * (row % 4)) by choosing which global chunk each lane fetches, which
//    keeps the fragment reads below free of bank conflicts.  Two barriers per
//    tile publish the copies (K before the S^T region, V before PV).
//  * Software pipeline, one step per tile t: S^T of tile t+1 runs on the MFMA
//    pipe while the VALU does tile t's mask, max and exponentials (pinned
//    between the MFMAs; the compiler would otherwise sink them to their use),
//    and the copies of K(t+2) are spread over the same MFMAs; then
//    O += V^T P^T for tile t, with the copies of V(t+1) spread over its MFMAs.
//    With one wave per SIMD every instruction costs an
//    issue slot, so the loop keeps its non-MFMA instructions few: one buffer
//    resource per workgroup for K and one for V, M0 walked from copy to copy
//    (nothing else in the kernel touches M0; tests/test_isa_m0.py checks the
//    ISA), Q held in AGPRs (the MFMA reads its B operand there), which leaves
//    the architectural VGPRs to scores, P and the fragment rings without spills.
//  * The LDS fragment reads of both products run several MFMAs ahead through
//    explicit register rings so that LDS latency stays off the MFMA issue.  S^T per 32 keys
//    (keys x queries, one 32x32 MFMA tile over 16 k-steps of 16 dims; lane l
//    owns query column l%32).  The accumulator's registers are already the B
//    operand of O^T = V^T P^T (dims x queries, 8 tiles of 32 dims, 4 k-steps of
//    16 keys), so P never moves between lanes.  The V^T operand comes straight
//    from the row-major V tile through the transposing LDS read
//    ds_read_b64_tr_b16.
//  * Lazy rescale: scores live in the log2 domain with the 1/sqrt(D) scale
//    folded into the exp2 argument; a query's reference max moves (and O, l are
//    rescaled) only when a tile's max exceeds it by more than 8, so P <= 2^8.
//  * Tiles wholly inside every query's causal window skip the masking.
//  * Key splits (when the grid would not fill the chip) write (m, l, O / l) partials
//    in the decode path's layout; the decode combine pass merges them.  The
//    workgroup order is XCD-aware: the dispatcher deals workgroup i to XCD i % 8,
//    so work items are renumbered to give each XCD a contiguous run of
//    (query tile, split) items, all splits of a query tile together, which
//    then share the tile's query rows in that XCD's L2.
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
#include <type_traits>

#include "context_internal.hpp"
#include "device_common.hpp"

namespace kraken {
namespace {

constexpr int kD = 256;
constexpr int kQTile = 32;             // query tokens per workgroup
constexpr int kKTile = 64;             // keys per LDS tile (two 32-key halves)
constexpr int kRowHalfs = kD;          // an LDS row is a whole 512-byte key row
constexpr int kTileHalfs = kKTile * kRowHalfs;  // 32 KB per K or V tile
constexpr uint32_t kStageBytes = 2u * kTileHalfs;
constexpr float kRescaleSlack = 8.0f;  // log2 headroom before O is rescaled

struct FlashParams {
  const float* query;
  const half_t* query_f16;  // set: the query is f16 (read instead of query)
  const half_t* key_cache;
  const half_t* value_cache;
  const float* gate;
  float* output;
  half_t* partial_o;  // [tokens][kv_heads][splits][G][D]: each split's o / l in f16
  float* partial_ml;  // [tokens][kv_heads][splits][G][2]
  uint32_t layer, start_position, tokens, capacity_tokens, heads, kv_heads;
  uint32_t key_count, keys_per_split, splits, q_tiles, head_groups;
  float scale_log2;
};

__device__ __forceinline__ float sigmoid_acc(float x) { return 1.0f / (1.0f + expf(-x)); }

// Row of C (32x32 accumulator) held in register r by a lane in half h.
__device__ __forceinline__ int c_row(int r, int h) { return (r >> 2) * 8 + h * 4 + (r & 3); }

// Scheduling constraints (sched_group_barrier masks: 0x002 VALU, 0x008 MFMA,
// 0x100 LDS read, 0x400 transcendental).  A run of N MFMAs, each fed by
// kReadsPerMfma LDS fragment reads issued kLookahead MFMAs ahead, with up to
// kValuPerMfma VALU instructions placed after each MFMA.
template <int N, int kLookahead, int kReadsPerMfma, int kValuPerMfma>
__device__ __forceinline__ void pipeline_mfma() {
#pragma unroll
  for (int i = 0; i < kLookahead; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x100, kReadsPerMfma, 0);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if (i + kLookahead < N) {
      __builtin_amdgcn_sched_group_barrier(0x100, kReadsPerMfma, 0);
    }
    if (kValuPerMfma > 0) {
      __builtin_amdgcn_sched_group_barrier(0x402, kValuPerMfma, 0);
    }
  }
}

// Per-lane byte offsets of the tile copies (loop invariant): copy i of wave w
// fills rows 2 (i W + w) + l / 32 (l = lane) of the stage, physical chunk
// l % 32, from logical chunk (l % 32) ^ swizzle(row).  The row's swizzle
// depends on i only through i mod (8 / W) for K (row % 16) and i mod 2 for V
// (row % 4, only when W = 1), so kK and kV offsets per lane cover every copy;
// the row pair 2 i W and the tile's first row enter through the buffer base.
template <int W>
struct CopyOffsets {
  static constexpr int kK = 8 / W;
  static constexpr int kV = W == 1 ? 2 : 1;
  uint32_t k[kK];
  uint32_t v[kV];
};

template <int W>
__device__ __forceinline__ CopyOffsets<W> copy_offsets(uint32_t row_bytes, uint32_t head_bytes,
                                                       int wave, int lane) {
  CopyOffsets<W> c;
  const int p = lane & 31;
  const uint32_t row_in_copy = (uint32_t)(2 * wave + (lane >> 5));
#pragma unroll
  for (int j = 0; j < CopyOffsets<W>::kK; ++j) {
    const int r = 2 * (j * W + wave) + (lane >> 5);
    c.k[j] = row_in_copy * row_bytes + head_bytes + 16u * (uint32_t)(p ^ (r & 15));
  }
#pragma unroll
  for (int j = 0; j < CopyOffsets<W>::kV; ++j) {
    const int r = 2 * (j * W + wave) + (lane >> 5);
    c.v[j] = row_in_copy * row_bytes + head_bytes + 16u * (uint32_t)(p ^ (4 * (r & 3)));
  }
  return c;
}

// The K or V rows of one workgroup: a buffer resource over the layer's first
// key_end rows (rows at or past key_end read as zeros without a memory access;
// the host keeps every byte offset below 2^31), the row size and the LDS byte
// address of this wave's first copy slot in stage 0.
struct TileSource {
  i32x4_t rsrc;
  uint32_t row_bytes;
  uint32_t lds;
};

// One direct-to-LDS copy of 16 bytes per lane (as copy16_to_lds) with M0 given
// as a scalar byte address.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void copy16_to_lds_m0(i32x4_t rsrc, uint32_t voffset, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(m0), "v"(voffset), "s"(rsrc)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Copy i of the 64-key tile starting at key row `row` into the stage whose LDS
// byte address (plus this wave's slot) is `stage_lds`: two key rows per wave,
// rows row + 2 (i W + wave) + lane / 32.  Scalar arithmetic plus one vector add.
template <int W, bool kV>
__device__ __forceinline__ void issue_copy(const TileSource& src, const CopyOffsets<W>& off,
                                           uint32_t row, uint32_t stage_lds, int i) {
  const uint32_t row_off = (row + 2u * i * W) * src.row_bytes;
  const uint32_t voff =
    (kV ? off.v[i % CopyOffsets<W>::kV] : off.k[i % CopyOffsets<W>::kK]) + row_off;
  copy16_to_lds_m0(src.rsrc, voff, stage_lds + (uint32_t)(i * W * 2 * kRowHalfs * 2));
}

// Copy i of a tile with M0 already holding its LDS address: the copy, then M0
// moved on by kStep bytes (the next copy of the tile) or set to `next` (the
// first copy of the other tile).  Whatever the caller issues between two copies
// covers the one wait state an M0 write needs before an LDS-DMA load.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
template <int W, bool kV, int kStep>
__device__ __forceinline__ void issue_copy_seq(const TileSource& src, const CopyOffsets<W>& off,
                                               uint32_t row, int i, bool last, uint32_t next) {
  const uint32_t voff = (kV ? off.v[i % CopyOffsets<W>::kV] : off.k[i % CopyOffsets<W>::kK]) +
                        (row + 2u * i * W) * src.row_bytes;
  if (last) {
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds\n\ts_mov_b32 m0, %2"
                 :
                 : "v"(voff), "s"(src.rsrc), "s"(next)
                 : "memory", "m0");
  } else {
    // s_add_u32 also writes SCC.
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds\n\ts_add_u32 m0, m0, %2"
                 :
                 : "v"(voff), "s"(src.rsrc), "n"(kStep)
                 : "memory", "m0", "scc");
  }
}

__device__ __forceinline__ void set_m0(uint32_t v) {
  asm volatile("s_mov_b32 m0, %0" : : "s"(v) : "m0");
}
#pragma clang diagnostic pop

// Copies per wave of one K or V tile.
template <int W>
constexpr int kCopiesPerTile = (kKTile / 2) / W;

template <int W, bool kV>
__device__ __forceinline__ void issue_tile_copy(const TileSource& src, const CopyOffsets<W>& off,
                                                uint32_t row, uint32_t stage_lds) {
#pragma unroll
  for (int i = 0; i < kCopiesPerTile<W>; ++i) {
    issue_copy<W, kV>(src, off, row, stage_lds, i);
  }
}

// Wait until at most N of this wave's vector-memory loads are outstanding.  The
// loop issues no other vector-memory loads than the tile copies, and loads
// complete in issue order, so this waits for all but the newest N copies.
template <int N>
__device__ __forceinline__ void wait_copies_but() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit count");
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

template <int GW, bool kQF16>
__global__ __launch_bounds__(64 * GW) __attribute__((amdgpu_waves_per_eu(1, 1)))
void flash256_kernel(FlashParams p) {
  // K and V tiles, two stages each (128 KB).
  __shared__ __attribute__((aligned(16))) half_t s_k[2 * kTileHalfs];
  __shared__ __attribute__((aligned(16))) half_t s_v[2 * kTileHalfs];
  // Staging for the query rows of waves 0 and 1 (waves 2 and 3 stage theirs in
  // V's second stage, which no copy writes before the loop): 160 KB in all.
  __shared__ __attribute__((aligned(16))) half_t s_q[2 * kQTile * kRowHalfs];

  constexpr int W = GW;  // waves
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Head slot; readfirstlane makes it a scalar, so the copies' resources and
  // LDS destinations are scalar arithmetic.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5;       // lane half
  const int n = lane & 31;       // query column owned by this lane
  const uint32_t G = p.heads / p.kv_heads;

  // XCD-aware renumbering of the linear workgroup id (see header), then the
  // work item (kv head, head group, query tile, split), the heaviest (latest)
  // query tiles first and the splits of a query tile fastest: an XCD's run
  // holds all splits of its query tiles, so each query row is read into one L2
  // instead of four, and each K/V tile is read by fewer workgroups at a time.
  const uint32_t total = p.q_tiles * p.kv_heads * p.head_groups * p.splits;
  const uint32_t lin = blockIdx.x;
  const uint32_t per_xcd = total / 8u;
  const uint32_t rem = total % 8u;
  const uint32_t xcd = lin % 8u;
  const uint32_t item = xcd * per_xcd + min(xcd, rem) + lin / 8u;
  const uint32_t qs = item % (p.q_tiles * p.splits);
  uint32_t q_rank = qs / p.splits;
  if ((p.q_tiles & 3u) == 0u) {
    // Consecutive ranks (one XCD's run) take query tiles a quarter apart, so
    // every XCD gets early and late (light and heavy causal) tiles.
    q_rank = (q_rank & 3u) * (p.q_tiles >> 2) + (q_rank >> 2);
  }
  const uint32_t q_tile = p.q_tiles - 1u - q_rank;
  const uint32_t split = qs % p.splits;
  const uint32_t hg = (item / (p.q_tiles * p.splits)) % p.head_groups;
  const uint32_t kvh = item / (p.q_tiles * p.splits * p.head_groups);
  const uint32_t g_in_group = hg * GW + wave;
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
  const uint32_t ntiles = (key_end - key_begin + kKTile - 1) / kKTile;

  // K/V rows of this layer through range-checked buffer resources: rows at or
  // past key_end read as zeros without a memory access (the host keeps every
  // byte offset below 2^31).
  const uint32_t row_bytes = p.kv_heads * kD * 2u;
  const size_t layer_elems = (size_t)p.layer * p.capacity_tokens * p.kv_heads * kD;
  const half_t* k_layer = p.key_cache + layer_elems;
  const half_t* v_layer = p.value_cache + layer_elems;
  const CopyOffsets<W> coff = copy_offsets<W>(row_bytes, kvh * kD * 2u, wave, lane);
  const uint32_t slot_bytes = (uint32_t)wave * 2u * kRowHalfs * 2u;
  const TileSource ksrc{rsrc_words(k_layer, key_end * row_bytes), row_bytes,
                        (uint32_t)(uintptr_t)(lds_void_t*)s_k + slot_bytes};
  const TileSource vsrc{rsrc_words(v_layer, key_end * row_bytes), row_bytes,
                        (uint32_t)(uintptr_t)(lds_void_t*)s_v + slot_bytes};

  // K(0)'s copies go out before the query is loaded; K(1)'s and V(0)'s after
  // the query's loads, so that the first S^T waits only for K(0) and the
  // query (K(1) past key_end reads as zeros).
  issue_tile_copy<W, false>(ksrc, coff, key_begin, ksrc.lds);

  // Q^T as the B operand of S^T = K Q^T: lane holds query n, dims 16*step + 8*h + j.
  // A lane's fragment takes 32 bytes from each of 16 places in its query row,
  // so loading it straight from global memory would touch 32 rows per load
  // instruction.  Instead each load reads one whole 1 KB row (16 bytes per
  // lane), and the rows are turned around in LDS as f16, with their 16-byte
  // chunks XOR-swizzled by row % 16 like the K tiles so that the fragment
  // reads are free of bank conflicts.
  half8_t qf[kD / 16];
  half_t* const q_stage = wave < 2 ? s_q + wave * (kQTile * kRowHalfs)
                                   : s_v + kTileHalfs + (wave - 2) * (kQTile * kRowHalfs);
  auto read_query_fragments = [&]() {
#pragma unroll
    for (int step = 0; step < kD / 16; ++step) {
      const int chunk = (2 * step + h) ^ (n & 15);
      qf[step] = *reinterpret_cast<const half8_t*>(q_stage + n * kRowHalfs + chunk * 8);
    }
    // Q stays in AGPRs (an MFMA reads its B operand from either file), which
    // leaves the architectural VGPRs to the scores, P and the fragment rings.
#pragma unroll
    for (int step = 0; step < kD / 16; ++step) {
      asm volatile("" : "+a"(qf[step]));
    }
  };
  if constexpr (kQF16) {
    // An f16 query row is copied straight into LDS like a key row: copy i
    // brings rows 2 i and 2 i + 1 (lanes 0-31 and 32-63), lane l fetching
    // logical chunk (l % 32) ^ (row % 16) into physical chunk l % 32.  The
    // resource starts at the tile's first row of this head and ends after the
    // last token's row, so rows past the end read as zeros.
    const uint32_t q_row_bytes = p.heads * kD * 2u;
    const uint32_t rows_left = p.tokens - t0;
    const i32x4_t qsrc = rsrc_words(p.query_f16 + ((size_t)t0 * p.heads + head) * kD,
                                    (rows_left - 1u) * q_row_bytes + kD * 2u);
    const uint32_t q_lds = (uint32_t)(uintptr_t)(lds_void_t*)q_stage;
    const uint32_t q_lane = (uint32_t)(lane >> 5) * q_row_bytes;
#pragma unroll
    for (int i = 0; i < kQTile / 2; ++i) {
      const int r = 2 * i + (lane >> 5);
      const uint32_t voff = q_lane + 2u * (uint32_t)i * q_row_bytes +
                            16u * (uint32_t)((lane & 31) ^ (r & 15));
      copy16_to_lds_m0(qsrc, voff, q_lds + (uint32_t)i * 2u * kRowHalfs * 2u);
    }
  } else {
    half_t* stage = q_stage;
    // Unconditional loads from a valid row (token 0 stands in for tokens past the
    // end), zeroed afterwards, so all 32 loads are in flight together.
    {
      float4 rows[kQTile];
#pragma unroll
      for (int r = 0; r < kQTile; ++r) {
        const uint32_t tok = t0 + (uint32_t)r < p.tokens ? t0 + (uint32_t)r : 0u;
        const float* qrow = p.query + ((size_t)tok * p.heads + head) * kD;
        rows[r] = *reinterpret_cast<const float4*>(qrow + 4 * lane);
      }
#pragma unroll
      for (int r = 0; r < kQTile; ++r) {
        const float qmask = t0 + (uint32_t)r < p.tokens ? 1.0f : 0.0f;
        const half4_t hv = {(half_t)(rows[r].x * qmask), (half_t)(rows[r].y * qmask),
                            (half_t)(rows[r].z * qmask), (half_t)(rows[r].w * qmask)};
        const int chunk = (lane >> 1) ^ (r & 15);
        *reinterpret_cast<half4_t*>(stage + r * kRowHalfs + chunk * 8 + (lane & 1) * 4) = hv;
      }
    }
    read_query_fragments();
  }
  issue_tile_copy<W, false>(ksrc, coff, key_begin + kKTile, ksrc.lds + kStageBytes);
  issue_tile_copy<W, true>(vsrc, coff, key_begin, vsrc.lds);

  float16_t o[kD / 32];  // O^T tiles: dims 32*dt + c_row(r, h), query n
#pragma unroll
  for (int dt = 0; dt < kD / 32; ++dt) {
    o[dt] = float16_t{};
  }
  float m = -INFINITY;  // reference max (log2 domain, scaled) of query n
  float l = 0.0f;       // this lane's share of the denominator (relative to m)
  const float c = p.scale_log2;

  // K fragment reads: row 32*half + n, logical chunk 2*step + h at physical
  // chunk (2*step + h) ^ (row % 16) = 2*step ^ u.  For step s + 8 that is chunk
  // 16 + (2s ^ u), 256 bytes past step s's, so 8 byte offsets cover the 16
  // steps; they stay in registers (the empty asm hides their origin, so they
  // are not recomputed at each read) and stage, key half and the step's high
  // bit enter as immediates.
  const int u = h ^ (n & 15);
  uint32_t k_byte[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    k_byte[s] = 2u * (uint32_t)(n * kRowHalfs + 8 * ((2 * s) ^ u));
    asm volatile("" : "+v"(k_byte[s]));
  }
  // V^T fragment reads (ds_read_b64_tr_b16): lane L = 16 g + 4 e + q of group g
  // (h = g / 2, 16-dim group gd = g % 2) supplies row 16 ks + 4h + e (+8 for the
  // high four keys), dims 32 dt + 16 gd + 4q, i.e. physical chunk
  // (4 dt + 2 gd + q/2) ^ 4e: 32 (dt ^ e) + 16 gd + 4q halfs (dt < 4; +128 for
  // dt >= 4).
  const int e = (lane >> 2) & 3;
  const int v_lane = (4 * h + e) * kRowHalfs + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  uint32_t v_byte[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    v_byte[b] = 2u * (uint32_t)(v_lane + 32 * (b ^ e)) + kStageBytes;  // toggled at step 0
    asm volatile("" : "+v"(v_byte[b]));
  }
  // The offsets also carry the LDS stage (bit 15: stages are 32 KB apart and
  // s_k, s_v start stage 0), toggled once per step.
  auto kfrag = [&](int i) {  // read i: step i / 2, key half i % 2
    const int s = i >> 1;
    const char* p =
      reinterpret_cast<const char*>(s_k + (i & 1) * 32 * kRowHalfs + 128 * (s >> 3));
    return *reinterpret_cast<const half8_t*>(p + k_byte[s & 7]);
  };
  auto vfrag = [&](int i) {  // read i: k-step i / 8, dim tile i % 8
    const int ks = i >> 3;
    const int dt = i & 7;
    const char* p =
      reinterpret_cast<const char*>(s_v + 128 * (dt >> 2) + 16 * ks * kRowHalfs) + v_byte[dt & 3];
    const half_t* vp = reinterpret_cast<const half_t*>(p);
    const half4_t lo = read_tr16(vp);
    const half4_t hi = read_tr16(vp + 8 * kRowHalfs);
    return half8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  };

  constexpr int kRing = 4;   // K fragment reads in flight
  constexpr int kVRing = 4;  // V fragment read pairs in flight
  // S^T of tile 0 (no softmax to overlap yet).
  auto first_scores = [&](float16_t& s0, float16_t& s1) {
    s0 = float16_t{};
    s1 = float16_t{};
    half8_t ring[kRing];
#pragma unroll
    for (int i = 0; i < kRing; ++i) {
      ring[i] = kfrag(i);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < kD / 8; ++i) {
      const half8_t a = ring[i % kRing];
      if (i + kRing < kD / 8) {
        ring[i % kRing] = kfrag(i + kRing);
      }
      if (i & 1) {
        s1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[i >> 1], s1, 0, 0, 0);
      } else {
        s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[i >> 1], s0, 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Step t (software pipelined): S^T of tile t is in (c0, c1).  After the
  // barrier that publishes K of tile t+1, S^T of tile t+1 runs on the MFMA pipe
  // into (n0, n1) while the VALU does tile t's mask, max and exponentials and
  // the copies of K(t+2) go out; after a second barrier, which publishes V of
  // tile t, O += V^T P^T for tile t runs while the copies of V(t+1) go out and
  // the last exponentials finish.  Each copy burst thus has a whole region to
  // land, and a region's copies are spread over its 32 MFMAs (a CU's
  // vector-memory path takes a tile's 64 KB only at a few tens of bytes per
  // clock).  Stage parity par = t % 2: K(t+1) sits in stage par ^ 1, V(t) in
  // stage par.
  auto step = [&](auto has_next, uint32_t t, float16_t& c0, float16_t& c1, float16_t& n0,
                  float16_t& n1) __attribute__((always_inline)) {
    constexpr bool kNext = decltype(has_next)::value;
    const uint32_t par = t & 1u;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      k_byte[s] ^= kStageBytes;
    }
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      v_byte[b] ^= kStageBytes;
    }
    // Outstanding here: K(t+1)'s copies, then V(t)'s (none at t = 0: the
    // prologue waited for everything it issued).
    constexpr int kc = kCopiesPerTile<W>;
    wait_copies_but<kc>();
    __syncthreads();
    const uint32_t kt = key_begin + t * kKTile;
    half8_t ring[kRing];
    // K(t+2) past the last tile has key rows at or past key_end only: it writes
    // zeros to a stage nothing reads again.
    const uint32_t k_lds = ksrc.lds + par * kStageBytes;
    const uint32_t v_lds = vsrc.lds + (par ^ 1u) * kStageBytes;
    // M0 walks the copies' LDS addresses: K(t+2)'s in the S^T region, whose
    // last copy points M0 at V(t+1)'s, walked in the PV region.
    constexpr int kStep = W * 2 * kRowHalfs * 2;
    // Copy j of a region goes after MFMA j * 32 / kc + offset (offset < 32 / kc).
    auto copy_piece = [&](int i, auto is_v, int offset) {
      constexpr bool kIsV = decltype(is_v)::value;
#pragma unroll
      for (int j = 0; j < kc; ++j) {
        if (j * (kD / 8) / kc + offset == i) {
          if (kIsV) {
            issue_copy_seq<W, true, kStep>(vsrc, coff, kt + kKTile, j, false, 0u);
          } else {
            issue_copy_seq<W, false, kStep>(ksrc, coff, kt + 2 * kKTile, j, j == kc - 1, v_lds);
          }
        }
      }
    };
    using IsV = std::integral_constant<bool, true>;
    using IsK = std::integral_constant<bool, false>;
    if (kNext) {
      if (W == 1) {
        // 32 copies per region: issued together (spread, their scalar
        // resources would not fit beside the S^T region's registers).
        issue_tile_copy<W, false>(ksrc, coff, kt + 2 * kKTile, k_lds);
      } else {
        set_m0(k_lds);
      }
#pragma unroll
      for (int i = 0; i < kRing; ++i) {
        ring[i] = kfrag(i);
      }
    }
    // ---- mask of tile t (only tiles that reach past a query's window) ----
    const bool full = kt + kKTile <= key_end && kt + kKTile - 1u <= first_position;
    if (!full) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const uint32_t k0 = kt + c_row(r, h);
        const uint32_t k1 = k0 + 32;
        c0[r] = (k0 < key_end && k0 <= position) ? c0[r] : -INFINITY;
        c1[r] = (k1 < key_end && k1 <= position) ? c1[r] : -INFINITY;
      }
    }
    if (kNext) {
      n0 = float16_t{};
      n1 = float16_t{};
    }
    __builtin_amdgcn_sched_barrier(0);

    // Softmax pieces of tile t, placed after MFMA i of the S^T region.
    float mx = -INFINITY;
    float corr = 1.0f;
    float neg_m = 0.0f;
    bool need = false;
    half8_t pb[4];
    // Each piece ends in an empty asm on its results: without it the compiler
    // sinks the work next to its first use (the PV region) and nothing overlaps.
    // Exponentials j (< 16): the two scores of pb[j / 4] at 2 (j % 4), +1.
    auto exp_piece = [&](int j) {
      const int b = j >> 2;
      const int k = 2 * (j & 3);
      const int r = 8 * (b & 1) + k;
      const float s0 = b < 2 ? c0[r] : c1[r];
      const float s1 = b < 2 ? c0[r + 1] : c1[r + 1];
      const float p0 = fast_exp2(fmaf(s0, c, neg_m));
      const float p1 = fast_exp2(fmaf(s1, c, neg_m));
      // The denominator sums the f16 weights that PV multiplies (v_dot2_f32_f16).
      half2_t hp = half2_t{(half_t)p0, (half_t)p1};
      l = __builtin_amdgcn_fdot2(hp, half2_t{(half_t)1.0f, (half_t)1.0f}, l, false);
      asm volatile("" : "+v"(hp), "+v"(l));
      pb[b][k] = hp[0];
      pb[b][k + 1] = hp[1];
    };
    auto soft_piece = [&](int i) {
      if (i < 4) {
        // IEEE maximum (v_maximum3_f32): fmaxf would first quiet each MFMA
        // result; a NaN score (non-finite inputs) propagates either way.
#pragma unroll
        for (int r = 4 * i; r < 4 * i + 4; ++r) {
          mx = __builtin_elementwise_maximum(mx, __builtin_elementwise_maximum(c0[r], c1[r]));
        }
        asm volatile("" : "+v"(mx));
      } else if (i == 4) {
        {
          const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx),
                                                           false, false);
          mx = __builtin_elementwise_maximum(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
        }
        mx *= c;  // tile max for query n (both lane halves)
        // The reference max moves only when the tile's exceeds it by the slack.
        need = mx > m + kRescaleSlack;
        const float m_new = need ? mx : m;
        corr = need ? fast_exp2(m - m_new) : 1.0f;  // m = -inf -> 0
        m = m_new;
        l *= corr;
        // A query with no valid key yet keeps m = -inf; its scores are all -inf.
        neg_m = m == -INFINITY ? 0.0f : -m;
        asm volatile("" : "+v"(neg_m), "+v"(corr), "+v"(l), "+v"(m));
      } else if (i >= 6 && i < 30 && (i & 1) == 0) {
        exp_piece((i - 6) >> 1);
      }
    };
#pragma unroll
    for (int i = 0; i < kD / 8; ++i) {
      if (kNext) {
        const half8_t a = ring[i % kRing];
        if (i + kRing < kD / 8) {
          ring[i % kRing] = kfrag(i + kRing);
        }
        if (i & 1) {
          n1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[i >> 1], n1, 0, 0, 0);
        } else {
          n0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[i >> 1], n0, 0, 0, 0);
        }
        if (W > 1) {
          copy_piece(i, IsK{}, 0);
        }
      }
      soft_piece(i);
      __builtin_amdgcn_sched_barrier(0);
    }
    // ---- O^T += V^T P^T over the tile's 64 keys (4 k-steps of 16) ----
    // Outstanding: V(t)'s copies, then K(t+2)'s (none in the last step).
    wait_copies_but<kNext ? kc : 0>();
    __syncthreads();
    if (kNext && W == 1) {
      issue_tile_copy<W, true>(vsrc, coff, kt + kKTile, v_lds);
    }
    half8_t vring[kVRing];
#pragma unroll
    for (int i = 0; i < kVRing; ++i) {
      vring[i] = vfrag(i);
    }
    if (__builtin_amdgcn_ballot_w64(need) != 0) {
#pragma unroll
      for (int dt = 0; dt < kD / 32; ++dt) {
        o[dt] *= corr;
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 4 * (kD / 32); ++i) {
      const half8_t a = vring[i % kVRing];
      if (i + kVRing < 4 * (kD / 32)) {
        vring[i % kVRing] = vfrag(i + kVRing);
      }
      o[i & 7] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb[i >> 3], o[i & 7], 0, 0, 0);
      if ((i & 3) == 0 && i < 16) {
        exp_piece(12 + (i >> 2));  // pb[3], first read by MFMA 24
      }
      if (kNext && W > 1) {
        copy_piece(i, IsV{}, (kD / 8) / kc / 2);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Prologue: publish K(0) (its copies and the query loads were issued before
  // K(1)'s and V(0)'s, and loads complete in issue order) and compute S^T of
  // tile 0; step 0 waits for K(1) and V(0).  An f16 query's rows are in LDS
  // once its copies are done (this wave's own), and go to the registers here.
  float16_t ca, cb, na, nb;
  constexpr int kAfterK0 = 2 * kCopiesPerTile<W> <= 63 ? 2 * kCopiesPerTile<W> : kCopiesPerTile<W>;
  wait_copies_but<kAfterK0>();
  __syncthreads();
  if constexpr (kQF16) {
    read_query_fragments();
  }
  first_scores(ca, cb);
  using Next = std::integral_constant<bool, true>;
  using Last = std::integral_constant<bool, false>;
  for (uint32_t t = 0; t + 1 < ntiles; ++t) {
    step(Next{}, t, ca, cb, na, nb);
    ca = na;
    cb = nb;
  }
  step(Last{}, ntiles - 1, ca, cb, na, nb);

  l = xor32_sum(l);  // both lane halves hold keys of query n
  // ---- epilogue: lane owns query n; dims 32*dt + c_row(r, h) ----
  if (p.splits == 1) {
    if (!token_ok) {
      return;
    }
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
    // The split's o / l in f16 (its values are a weighted average of V rows,
    // so within V's range); the merge scales it back by l.  The wave's 32 rows
    // go through its 16 KB of K's LDS (free after the loop: the last step reads
    // only V) so that each store writes whole 512-byte rows.
    const float inv = l == 0.0f ? 0.0f : 1.0f / l;
    half_t* stage = s_k + wave * (kQTile * kD);
#pragma unroll
    for (int dt = 0; dt < kD / 32; ++dt) {
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int c = 4 * dt + r4;  // 16-byte chunk of the row; h picks its half
        const half4_t v = {static_cast<half_t>(o[dt][r4 * 4 + 0] * inv),
                           static_cast<half_t>(o[dt][r4 * 4 + 1] * inv),
                           static_cast<half_t>(o[dt][r4 * 4 + 2] * inv),
                           static_cast<half_t>(o[dt][r4 * 4 + 3] * inv)};
        *reinterpret_cast<half4_t*>(stage + n * kD + 8 * (c ^ n) + 4 * h) = v;
      }
    }
    if (h == 0 && token_ok) {
      const size_t base = (((size_t)token * p.kv_heads + kvh) * p.splits + split) * G + g_in_group;
      p.partial_ml[base * 2 + 0] = m;
      p.partial_ml[base * 2 + 1] = l;
    }
    const size_t row_units = (size_t)p.kv_heads * p.splits * G;  // units between tokens
    const size_t base0 = (((size_t)t0 * p.kv_heads + kvh) * p.splits + split) * G + g_in_group;
    const int chunk = lane & 31;
#pragma unroll
    for (int i = 0; i < kQTile / 2; ++i) {
      const int row = 2 * i + (lane >> 5);
      if (t0 + (uint32_t)row < p.tokens) {
        const u32x4_t val = *reinterpret_cast<const u32x4_t*>(stage + row * kD + 8 * (chunk ^ row));
        u32x4_t* dst = reinterpret_cast<u32x4_t*>(p.partial_o + (base0 + row * row_units) * kD) + chunk;
        *dst = val;
      }
    }
  }
}

struct FlashPlan {
  uint32_t q_tiles, head_groups, keys_per_split, splits;
};

// Smallest split worth its query load, partial write and merge: 4 key tiles
// (measured on C2 at P=0: 2 splits 37.4 us, 4 splits 29.8, 8 splits 43.2).
constexpr uint32_t kMinKeysPerSplit = 4 * kKTile;

FlashPlan plan_flash(const AttentionArgs& a, int cu_count) {
  FlashPlan plan{};
  const uint32_t g = a.heads / a.kv_heads;
  plan.q_tiles = (a.tokens + kQTile - 1) / kQTile;
  plan.head_groups = g > 4 ? g / 4 : 1;
  const uint32_t key_count = a.start_position + a.tokens;
  const uint64_t units = (uint64_t)plan.q_tiles * a.kv_heads * plan.head_groups;
  // One workgroup (one wave per SIMD, 128 KB of LDS) per CU.
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
  // The f16 partials' merge takes at most 16 splits.
  if (splits > 16) {
    splits = 16;
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
  if (p.query_f16 != nullptr) {
    flash256_kernel<GW, true><<<grid, 64 * GW, 0, stream>>>(p);
  } else {
    flash256_kernel<GW, false><<<grid, 64 * GW, 0, stream>>>(p);
  }
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

// Workspace: the f16 partial outputs, then (256-byte aligned) the f32 (m, l).
size_t partial_ml_offset(size_t units) { return (units * kD * sizeof(half_t) + 255u) / 256u * 256u; }

size_t attention_flash_workspace_bytes(const AttentionArgs& a, int cu_count) {
  const FlashPlan plan = plan_flash(a, cu_count);
  if (plan.splits <= 1) {
    return 0;
  }
  const size_t units = (size_t)a.tokens * a.heads * plan.splits;
  return partial_ml_offset(units) + units * 2 * sizeof(float);
}

hipError_t launch_attention_flash(const AttentionArgs& a, int cu_count, void* workspace,
                                  size_t workspace_bytes, hipStream_t stream) {
  const FlashPlan plan = plan_flash(a, cu_count);
  FlashParams p{};
  p.query = a.query;
  p.query_f16 = static_cast<const half_t*>(a.query_f16);
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
  // Work items are numbered with the splits of a query tile fastest, query
  // tiles a quarter apart interleaved.  Measured on C2 (T = 1024, 4 splits)
  // against query tiles fastest: P = 3072 45.7 -> 42.7 us, P = 7168 77 ->
  // 72.5 us, and, with the query copied into LDS and the eight-dim merge,
  // P = 1024 31.7-31.85 -> 30.3-31.5 us, P = 0 level (22.2-22.9 us).
  p.scale_log2 = (1.0f / sqrtf(256.0f)) * kLog2e;
  if (plan.splits > 1) {
    const size_t units = (size_t)a.tokens * a.heads * plan.splits;
    if (workspace == nullptr || plan.splits > 16 ||
        workspace_bytes < partial_ml_offset(units) + units * 2 * sizeof(float)) {
      return hipErrorInvalidValue;
    }
    p.partial_o = static_cast<half_t*>(workspace);
    p.partial_ml =
      reinterpret_cast<float*>(static_cast<char*>(workspace) + partial_ml_offset(units));
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
  cmb.partial_o = reinterpret_cast<const float*>(p.partial_o);
  cmb.partial_ml = p.partial_ml;
  cmb.partial_f16 = 1u;
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
