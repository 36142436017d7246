// Shared by the decode translation units (attention_decode.hip and
// attention_decode_short.hip): the kernel parameter block, the key count of a
// query token, the output epilogue and the head_dim-256 tile constants.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "attention_prologue_common.hpp"
#include "device_common.hpp"

namespace kraken {
namespace decode {

struct DecodeParams {
  const float* query;
  const void* key_cache;
  const void* value_cache;
  const float* gate;
  float* output;
  float* part_o;   // [tokens][kv_heads][splits][G][D]
  float* part_ml;  // [tokens][kv_heads][splits][G][2]
  uint32_t layer, start_position, tokens, capacity_tokens, heads, kv_heads;
  uint32_t keys_per_split, splits;
  float scale_log2;
  // Ragged multi-sequence mode (see AttentionArgs): per-token K/V element
  // offsets and positions, and the pools' element count.
  const uint64_t* seq_kv_offsets;
  const uint32_t* seq_positions;
  uint64_t pool_elems;
  // Ragged mode: dense work list, one item per workgroup (blockIdx.x):
  // {token, kv_head << 16 | split}, token 0xffffffff past the last item.
  const uint2* work_items;
};

// Keys of token t (positions table in ragged mode); at least 1 (a position of
// 2^32 - 1 saturates instead of wrapping to 0).
__device__ __forceinline__ uint32_t token_keys(const uint32_t* positions, uint32_t start,
                                               uint32_t token) {
  const uint64_t keys = positions != nullptr ? (uint64_t)positions[token] + 1u
                                             : (uint64_t)start + token + 1u;
  return (uint32_t)min(keys, (uint64_t)0xffffffffu);
}

__device__ __forceinline__ float sigmoidf_acc(float x) { return 1.0f / (1.0f + expf(-x)); }


template <int D, int G>
__device__ __forceinline__ void write_final(const DecodeParams& p, uint32_t token, uint32_t kvh,
                                            int idx, float den, float acc) {
  const int g = idx / D;
  const int d = idx % D;
  const size_t out_index = ((size_t)token * p.heads + kvh * G + g) * D + d;
  float r = den == 0.0f ? 0.0f : acc / den;
  if (p.gate != nullptr) {
    r *= sigmoidf_acc(p.gate[out_index]);
  }
  p.output[out_index] = r;
}

// Lazy rescale slack (log2 domain): a wave exponentiates against a reference
// max that moves only when a score exceeds it by more than this, so p <= 2^8
// (far from f32 overflow) and most rounds skip the rescale of o and l.  The
// result is exact either way: o and l always share the same reference.
constexpr float kRescaleSlack = 8.0f;

// Kahan-compensated running sum: sum + (-comp) carries what plain fp32
// addition would drop when many small terms join a larger sum (the softmax
// denominator of a long split).  The library is built without fast-math, so
// the compiler keeps the compensation's operation order.
__device__ __forceinline__ void kahan_add(float& sum, float& comp, float x) {
  const float y = x - comp;
  const float t = sum + y;
  comp = (t - sum) - y;
  sum = t;
}

constexpr int kMD = 256;
constexpr int kMTile = 16;                        // keys per tile
constexpr int kMTileHalfs = kMTile * kMD;         // 8 KB per K or V tile

typedef float float4v_t __attribute__((ext_vector_type(4)));

// The full-attention prologue folded into the short-split kernel for one
// decode token (one split per KV head): the raw joint projection row and K/V
// rows of the token, the q/k norm weights and the MRoPE arguments.  The kernel
// normalises and rotates its query heads and its K head, appends the K/V row
// (f16) at start_position of the cache and uses it in place of what it loaded
// for that row; the output gate is the second half of each q_gate head.
struct PrologueFold {
  const float* q_gate;  // [heads][2 D]
  const float* key;     // [kv_heads][D]
  const float* value;   // [kv_heads][D]
  const float* q_norm;  // [D]
  const float* k_norm;  // [D]
  RopeArgs rope;
  float eps;
};

// Launches the short-split MFMA kernel (attention_decode_short.hip) for
// head_dim 256, an f16 cache and G = heads / kv_heads in {1, 2, 4}, one
// workgroup per (split, kv_head, token) of `grid`.
hipError_t launch_decode_short(const DecodeParams& p, uint32_t group, dim3 grid,
                               hipStream_t stream);
// The same kernel with the prologue folded in: p.tokens == 1, p.splits == 1,
// p.keys_per_split == p.start_position + 1, p.query and p.gate unused; grid
// (1, kv_heads, 1).
hipError_t launch_decode_short_prologue(const DecodeParams& p, const PrologueFold& f,
                                        uint32_t group, hipStream_t stream);

}  // namespace decode
}  // namespace kraken
