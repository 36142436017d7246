// The full-attention prologue of run_qwen35_full_attention_layer_chunk
// (qwen35_runtime.cpp:3229-3326) as one kernel:
//   copy_f32_rows x2           split of the joint Q/gate projection
//   qk_norm_f32_f32_batched x2 RMSNorm of q (q_norm) and k (k_norm)
//   mrope_f32_in_place x2      MRoPE of q and k
//   copy_f32_rows_to_f16 x2    K and V rows appended to the F16 cache
// One wave per (token, head slot): slots 0 .. H-1 are query heads, then
// Hkv key heads, then Hkv value heads.  The arithmetic is that of
// rms_norm_heads_kernel and mrope_kernel (same element-to-lane layout, same
// reduction order, the angle in double), so the result equals the unfused
// chain's bit for bit.
#include <hip/hip_runtime.h>

#include "attention_prologue_common.hpp"
#include "context_internal.hpp"
#include "device_common.hpp"

namespace kraken {
namespace {

constexpr int kWaves = 4;

__global__ __launch_bounds__(256) void attention_prologue_kernel(PrologueArgs a) {
  const int lane = threadIdx.x & 63;
  const uint32_t slots = a.heads + 2u * a.kv_heads;
  const size_t item = (size_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (item >= (size_t)a.tokens * slots) {
    return;  // whole wave
  }
  const uint32_t t = (uint32_t)(item / slots);
  const uint32_t slot = (uint32_t)(item % slots);
  const uint32_t d_head = a.head_dim;
  const size_t kv_dim = (size_t)a.kv_heads * d_head;

  if (slot >= a.heads + a.kv_heads) {  // value head: f32 -> f16 append
    const uint32_t kh = slot - a.heads - a.kv_heads;
    const float* src = a.value + (size_t)t * kv_dim + (size_t)kh * d_head;
    half_t* dst = a.value_cache + a.cache_offset + (size_t)t * kv_dim + (size_t)kh * d_head;
    for (uint32_t d = lane; d < d_head; d += 64) {
      dst[d] = static_cast<half_t>(src[d]);
    }
    return;
  }

  const bool is_q = slot < a.heads;
  const uint32_t head = is_q ? slot : slot - a.heads;
  const float* src = is_q ? a.q_gate + ((size_t)t * a.heads + head) * 2u * d_head
                          : a.key + (size_t)t * kv_dim + (size_t)head * d_head;
  const float* weight = is_q ? a.q_norm : a.k_norm;
  const RopeArgs rope{a.positions, a.mrope_start, a.tokens, a.n_dims, a.s0, a.s1, a.s2, a.s3,
                      a.theta};
  float v[4], w[4], g[4];
  load_head(src, weight, d_head, lane, v, w);
  // The gate half of a q_gate head is copied out; its loads go out with the rest.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t d = lane + 64u * i;
    g[i] = is_q && d < d_head ? src[d_head + d] : 0.0f;
  }
  int32_t pos[4];
  rope_positions(rope, t, pos);
  double sn[4], cs[4];
  rope_angles(rope, pos, lane, sn, cs);
  float r[4];
  norm_rope(v, w, d_head, a.eps, a.n_dims, sn, cs, lane, r);

  if (is_q) {
    float* q_out = a.query_out + ((size_t)t * a.heads + head) * d_head;
    float* g_out = a.gate_out + ((size_t)t * a.heads + head) * d_head;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t d = lane + 64u * i;
      if (d < d_head) {
        q_out[d] = r[i];
        g_out[d] = g[i];
      }
    }
  } else {
    half_t* dst = a.key_cache + a.cache_offset + (size_t)t * kv_dim + (size_t)head * d_head;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t d = lane + 64u * i;
      if (d < d_head) {
        dst[d] = static_cast<half_t>(r[i]);
      }
    }
  }
}

}  // namespace

hipError_t launch_attention_prologue(const PrologueArgs& a, hipStream_t stream) {
  const size_t items = (size_t)a.tokens * (a.heads + 2u * a.kv_heads);
  const size_t blocks = (items + kWaves - 1) / kWaves;
  if (blocks == 0) {
    return hipSuccess;
  }
  attention_prologue_kernel<<<dim3((uint32_t)blocks), 256, 0, stream>>>(a);
  return hipGetLastError();
}

}  // namespace kraken
