// One head of the full-attention prologue (RMSNorm with a weight, then MRoPE),
// shared by the prologue kernel and the decode kernel that folds the prologue
// in, so both produce the same bits.  Semantics: qk_norm_f32_f32_batched then
// mrope_f32_in_place (mps_backend.mm:1991-2024, 2482-2527): the element-to-lane
// layout and reduction order of rms_norm_heads_kernel, the angle in double.
//
// A wave holds a head of d_head <= 256 values as elements lane + 64 i (i < 4).
// The loads (load_head, rope_positions) are separate from the arithmetic so a
// caller can issue them before other loads it wants in flight meanwhile.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "device_common.hpp"

namespace kraken {

struct RopeArgs {
  const int32_t* positions;  // [4][tokens], or null: mrope_start + t in every row
  uint32_t mrope_start, tokens, n_dims, s0, s1, s2, s3;
  float theta;
};

// The lane's elements of src and of the norm weight (0 past d_head).
__device__ __forceinline__ void load_head(const float* src, const float* weight,
                                          uint32_t d_head, int lane, float v[4], float w[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t d = lane + 64u * i;
    v[i] = d < d_head ? src[d] : 0.0f;
    w[i] = d < d_head ? weight[d] : 0.0f;
  }
}

// Token t's position in each of the four MRoPE rows.
__device__ __forceinline__ void rope_positions(const RopeArgs& a, uint32_t t, int32_t pos[4]) {
#pragma unroll
  for (int row = 0; row < 4; ++row) {
    pos[row] = a.positions != nullptr ? a.positions[t + (size_t)a.tokens * row]
                                      : (int32_t)(a.mrope_start + t);
  }
}

// sin and cos of the rotation angle of each of the lane's elements below
// n_dims (pair p = e mod n_dims / 2 in the section that p mod sum(sections)
// falls into; the rest are left unset).
__device__ __forceinline__ void rope_angles(const RopeArgs& a, const int32_t pos[4], int lane,
                                            double sn[4], double cs[4]) {
  const uint32_t half_dims = a.n_dims / 2u;
  const uint32_t sections = a.s0 + a.s1 + a.s2 + a.s3;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t e = lane + 64u * i;
    if (e < a.n_dims) {
      const uint32_t pair = e < half_dims ? e : e - half_dims;
      const uint32_t sector = pair % sections;
      int32_t p = pos[3];
      if (sector < a.s0) {
        p = pos[0];
      } else if (sector < a.s0 + a.s1) {
        p = pos[1];
      } else if (sector < a.s0 + a.s1 + a.s2) {
        p = pos[2];
      }
      const double freq = pow((double)a.theta, -(double)(2u * pair) / (double)a.n_dims);
      const double angle = (double)p * freq;
      sincos(angle, &sn[i], &cs[i]);
    }
  }
}

// r = MRoPE(v * rsqrt(mean(v^2) + eps) * w): elements past d_head are 0, those
// in [n_dims, d_head) only normalised.
__device__ __forceinline__ void norm_rope(const float v_in[4], const float w[4], uint32_t d_head,
                                          float eps, uint32_t n_dims, const double sn[4],
                                          const double cs[4], int lane, float r[4]) {
  float v[4];
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[i] = v_in[i];
    sum = fmaf(v[i], v[i], sum);
  }
  sum = wave_sum(sum);
  const float scale = 1.0f / sqrtf(sum / (float)d_head + eps);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t d = lane + 64u * i;
    v[i] = d < d_head ? v[i] * scale * w[i] : 0.0f;
  }

  // Pairs (p, p + n_dims / 2), p < n_dims / 2.  Each lane fetches the partner
  // of each of its elements from the lane and register that hold it.
  const uint32_t half_dims = n_dims / 2u;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t e = lane + 64u * i;
    const uint32_t p = e < half_dims ? e + half_dims : (e < n_dims ? e - half_dims : e);
    const int src_lane = (int)(p & 63u);
    const uint32_t src_reg = p >> 6;
    float partner = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float x = __shfl(v[j], src_lane, 64);
      partner = src_reg == (uint32_t)j ? x : partner;
    }
    r[i] = v[i];
    if (e < n_dims) {
      const double x0 = e < half_dims ? v[i] : partner;
      const double x1 = e < half_dims ? partner : v[i];
      r[i] = e < half_dims ? (float)(x0 * cs[i] - x1 * sn[i]) : (float)(x1 * cs[i] + x0 * sn[i]);
    }
    // The f32 result kept as such: a caller that rounds it to fp16 (the K
    // append) must not get the norm's last multiply and that rounding fused
    // into one v_fma_mix, which the separate qk_norm / mrope / copy ops (each
    // storing f32) cannot do.
    asm("" : "+v"(r[i]));
  }
}

}  // namespace kraken
