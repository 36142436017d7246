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

  // RMSNorm: lane holds elements lane + 64 i (the layout of rms_norm_heads_kernel).
  float v[4];
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t d = lane + 64u * i;
    v[i] = d < d_head ? src[d] : 0.0f;
    sum = fmaf(v[i], v[i], sum);
  }
  sum = wave_sum(sum);
  const float scale = 1.0f / sqrtf(sum / (float)d_head + a.eps);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t d = lane + 64u * i;
    v[i] = d < d_head ? v[i] * scale * weight[d] : 0.0f;
  }

  // MRoPE on pairs (p, p + n_dims / 2), p < n_dims / 2.  Each lane fetches the
  // partner of each of its elements from the lane and register that hold it.
  const uint32_t half_dims = a.n_dims / 2u;
  const uint32_t sections = a.s0 + a.s1 + a.s2 + a.s3;
  float r[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t e = lane + 64u * i;
    const uint32_t p = e < half_dims ? e + half_dims : (e < a.n_dims ? e - half_dims : e);
    const int src_lane = (int)(p & 63u);
    const uint32_t src_reg = p >> 6;
    float partner = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float x = __shfl(v[j], src_lane, 64);
      partner = src_reg == (uint32_t)j ? x : partner;
    }
    r[i] = v[i];
    if (e < a.n_dims) {
      const uint32_t pair = e < half_dims ? e : e - half_dims;
      const uint32_t sector = pair % sections;
      uint32_t row = 3;
      if (sector < a.s0) {
        row = 0;
      } else if (sector < a.s0 + a.s1) {
        row = 1;
      } else if (sector < a.s0 + a.s1 + a.s2) {
        row = 2;
      }
      const int32_t pos = a.positions != nullptr
                            ? a.positions[t + (size_t)a.tokens * row]
                            : (int32_t)(a.mrope_start + t);
      const double freq = pow((double)a.theta, -(double)(2u * pair) / (double)a.n_dims);
      const double angle = (double)pos * freq;
      double sn, cs;
      sincos(angle, &sn, &cs);
      const double x0 = e < half_dims ? v[i] : partner;
      const double x1 = e < half_dims ? partner : v[i];
      r[i] = e < half_dims ? (float)(x0 * cs - x1 * sn) : (float)(x1 * cs + x0 * sn);
    }
  }

  if (is_q) {
    float* q_out = a.query_out + ((size_t)t * a.heads + head) * d_head;
    float* g_out = a.gate_out + ((size_t)t * a.heads + head) * d_head;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t d = lane + 64u * i;
      if (d < d_head) {
        q_out[d] = r[i];
        g_out[d] = src[d_head + d];
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
