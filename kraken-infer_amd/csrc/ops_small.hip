// Prologue/epilogue operators of the Qwen3.5 attention path: per-head RMSNorm
// (plain and norm-gated), L2 norm, the q/k/v split with L2 norm, gate/beta
// prepare, MRoPE, strided row copies (f32, f32->f16 RNE, f16), elementwise
// sigmoid/softplus/silu and (row-)broadcast multiply/add.
//
// Semantics follow the reference MSL kernels cited on each kernel.  Row
// reductions use one wave per row with DPP reductions; everything else is
// grid-stride elementwise with 64-bit indexing.
#include <hip/hip_runtime.h>

#include "context_internal.hpp"
#include "device_common.hpp"

namespace kraken {
namespace {

constexpr int kRowsPerBlock = 4;  // one wave per row

__device__ __forceinline__ float sigmoid_acc(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float softplus_ref(float x) {
  // mps_backend.mm:2584-2585: x > 20 ? x : log(1 + e^x)
  return x > 20.0f ? x : log1pf(expf(x));
}

// qk_norm_f32_f32_batched (mps_backend.mm:1991-2024) and, with gate != null,
// qwen35_norm_gated_f32_in_place (mps_backend.mm:2026-2063):
// x <- x * rsqrt(mean(x^2) + eps) * w [* silu(gate)].  head_dim <= 256.
__global__ __launch_bounds__(256) void rms_norm_heads_kernel(float* values, const float* weight,
                                                             const float* gate, uint32_t rows,
                                                             uint32_t head_dim, float eps) {
  const uint32_t row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) {
    return;  // whole wave exits together
  }
  float* x = values + (size_t)row * head_dim;
  // The weights and the gate are loaded with the row, before the reduction,
  // so the scaling does not wait for a second round trip.
  float v[4], w[4], z[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t d = lane + 64u * i;
    v[i] = d < head_dim ? x[d] : 0.0f;
    w[i] = d < head_dim ? weight[d] : 0.0f;
    z[i] = d < head_dim && gate != nullptr ? gate[(size_t)row * head_dim + d] : 0.0f;
  }
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    sum = fmaf(v[i], v[i], sum);
  }
  sum = wave_sum(sum);
  const float scale = 1.0f / sqrtf(sum / (float)head_dim + eps);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t d = lane + 64u * i;
    if (d < head_dim) {
      float r = v[i] * scale * w[i];
      if (gate != nullptr) {
        r *= z[i] * sigmoid_acc(z[i]);
      }
      x[d] = r;
    }
  }
}

// l2_norm_f32_in_place (mps_backend.mm:2065-2095): x / max(||x||, eps).
__global__ __launch_bounds__(256) void l2_norm_kernel(float* values, uint32_t rows,
                                                      uint32_t row_size, float eps) {
  const uint32_t row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) {
    return;
  }
  float* x = values + (size_t)row * row_size;
  float sum = 0.0f;
  for (uint32_t d = lane; d < row_size; d += 64) {
    sum = fmaf(x[d], x[d], sum);
  }
  sum = wave_sum(sum);
  const float inv = 1.0f / fmaxf(sqrtf(sum), eps);
  for (uint32_t d = lane; d < row_size; d += 64) {
    x[d] *= inv;
  }
}

// split_qkv_l2_norm_f32_qwen35 (mps_backend.mm:2097-2153).  One wave per
// (token, part, head): parts 0/1 are q/k (L2-normalised), part 2 copies v.
__global__ __launch_bounds__(256) void split_qkv_l2_kernel(const float* source, float* query,
                                                           float* key, float* value,
                                                           uint32_t tokens, uint32_t key_heads,
                                                           uint32_t value_heads,
                                                           uint32_t head_dim, float eps) {
  const uint32_t heads_per_token = 2u * key_heads + value_heads;
  const uint32_t unit = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (unit >= tokens * heads_per_token) {
    return;
  }
  const uint32_t token = unit / heads_per_token;
  const uint32_t r = unit % heads_per_token;
  const uint32_t key_dim = key_heads * head_dim;
  const size_t channels = 2ull * key_dim + (size_t)value_heads * head_dim;
  const float* src = source + (size_t)token * channels;
  if (r >= 2u * key_heads) {
    const uint32_t h = r - 2u * key_heads;
    const float* s = src + 2ull * key_dim + (size_t)h * head_dim;
    float* dst = value + ((size_t)token * value_heads + h) * head_dim;
    for (uint32_t d = lane; d < head_dim; d += 64) {
      dst[d] = s[d];
    }
    return;
  }
  const uint32_t part = r / key_heads;
  const uint32_t h = r % key_heads;
  const float* s = src + (size_t)part * key_dim + (size_t)h * head_dim;
  float sum = 0.0f;
  for (uint32_t d = lane; d < head_dim; d += 64) {
    sum = fmaf(s[d], s[d], sum);
  }
  sum = wave_sum(sum);
  const float inv = 1.0f / fmaxf(sqrtf(sum), eps);
  float* dst = (part == 0 ? query : key) + ((size_t)token * key_heads + h) * head_dim;
  for (uint32_t d = lane; d < head_dim; d += 64) {
    dst[d] = s[d] * inv;
  }
}

// prepare_qwen35_gdn_gate_beta_f32 (mps_backend.mm:2588-2605).
__global__ void prepare_gate_beta_kernel(float* gate, float* beta, const float* bias,
                                         const float* scale, size_t total, uint32_t row_size) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const uint32_t c = (uint32_t)(i % row_size);
    gate[i] = softplus_ref(gate[i] + bias[c]) * scale[c];
    beta[i] = sigmoid_acc(beta[i]);
  }
}

// mrope_f32_in_place (mps_backend.mm:2482-2527).  Angles are formed and reduced
// in double: positions reach 1e4 and theta 1e7, where fp32 angles lose ~1e-3 rad.
__global__ void mrope_kernel(float* values, const int32_t* positions, uint32_t tokens,
                             uint32_t heads, uint32_t head_dim, uint32_t n_dims, uint32_t s0,
                             uint32_t s1, uint32_t s2, uint32_t s3, float theta) {
  const uint32_t half_dims = n_dims / 2u;
  const size_t total = (size_t)tokens * heads * half_dims;
  const uint32_t sections = s0 + s1 + s2 + s3;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const uint32_t pair = (uint32_t)(i % half_dims);
    const uint32_t head = (uint32_t)((i / half_dims) % heads);
    const uint32_t token = (uint32_t)(i / ((size_t)half_dims * heads));
    const uint32_t sector = pair % sections;
    uint32_t row = 3;
    if (sector < s0) {
      row = 0;
    } else if (sector < s0 + s1) {
      row = 1;
    } else if (sector < s0 + s1 + s2) {
      row = 2;
    }
    const double position = (double)positions[token + (size_t)tokens * row];
    const double freq = pow((double)theta, -(double)(2u * pair) / (double)n_dims);
    const double angle = position * freq;
    double sn, cs;
    sincos(angle, &sn, &cs);
    float* x = values + ((size_t)token * heads + head) * head_dim;
    const double x0 = x[pair];
    const double x1 = x[half_dims + pair];
    x[pair] = (float)(x0 * cs - x1 * sn);
    x[half_dims + pair] = (float)(x1 * cs + x0 * sn);
  }
}

template <typename Src, typename Dst>
__device__ __forceinline__ Dst convert(Src v) {
  return static_cast<Dst>(v);
}

// copy_f32_rows / copy_f32_rows_to_f16 / copy_f16_rows (mps_backend.mm:2627-2679).
template <typename Src, typename Dst>
__global__ void copy_rows_kernel(const Src* source, Dst* destination, size_t total,
                                 size_t row_size, size_t source_stride, size_t source_offset,
                                 size_t destination_stride, size_t destination_offset) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t row = i / row_size;
    const size_t col = i % row_size;
    destination[destination_offset + row * destination_stride + col] =
      convert<Src, Dst>(source[source_offset + row * source_stride + col]);
  }
}

// Ragged KV append (one new row per sequence): the f32 -> f16 row copy of
// copy_f32_rows_to_f16 (mps_backend.mm:2655-2666) with the destination row taken
// from per-sequence tables.  A row that would land outside the pool is skipped.
__global__ void append_kv_ragged_kernel(const float* key_rows, const float* value_rows,
                                        half_t* key_pool, half_t* value_pool,
                                        const uint64_t* seq_offsets,
                                        const uint32_t* seq_positions, uint64_t pool_elems,
                                        uint32_t sequences, uint32_t row_size) {
  const size_t total = (size_t)sequences * row_size;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t b = i / row_size;
    const size_t c = i % row_size;
    const uint64_t row0 = seq_offsets[b] + (uint64_t)seq_positions[b] * row_size;
    if (row0 > pool_elems || pool_elems - row0 < row_size) {
      continue;
    }
    key_pool[row0 + c] = static_cast<half_t>(key_rows[i]);
    value_pool[row0 + c] = static_cast<half_t>(value_rows[i]);
  }
}

// sigmoid/softplus/silu_f32_in_place (mps_backend.mm:2569-2618).
template <UnaryKind K>
__global__ void unary_kernel(float* values, size_t size) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < size;
       i += (size_t)gridDim.x * blockDim.x) {
    const float x = values[i];
    float r;
    if (K == UnaryKind::sigmoid) {
      r = sigmoid_acc(x);
    } else if (K == UnaryKind::softplus) {
      r = softplus_ref(x);
    } else {
      r = x * sigmoid_acc(x);
    }
    values[i] = r;
  }
}

// mul_f32_in_place / add_f32_row_in_place / mul_f32_row_in_place (mps_backend.mm:2539-2567).
// One workgroup per row of `size` values: output = input * rsqrt(mean(input^2)
// + eps) * weight (rms_norm_f32_f32_batched, mps_backend.mm:1890-1920).  Input and
// output may be the same buffer: every value is read before the row is written.
__global__ __launch_bounds__(256) void rms_norm_rows_kernel(const float* input,
                                                            const float* weight, float* output,
                                                            uint32_t size, float eps) {
  __shared__ float s_part[4];
  const float* x = input + (size_t)blockIdx.x * size;
  float* y = output + (size_t)blockIdx.x * size;
  // Rows of up to 256 * kHeld values stay in registers between the sum of
  // squares and the scaling (with the weights loaded beside them), instead of
  // being read a second time; the sum runs over the same elements in the same
  // order either way (whole-model prefill 5.77 -> 5.72 ms per 1024-token
  // chunk, 48 calls per chunk).
  constexpr uint32_t kHeld = 8;
  const bool held = size <= 256u * kHeld;
  float xv[kHeld], wv[kHeld];
  float sum = 0.0f;
  if (held) {
#pragma unroll
    for (uint32_t k = 0; k < kHeld; ++k) {
      const uint32_t i = threadIdx.x + 256u * k;
      xv[k] = i < size ? x[i] : 0.0f;
      wv[k] = i < size ? weight[i] : 0.0f;
    }
#pragma unroll
    for (uint32_t k = 0; k < kHeld; ++k) {
      if (threadIdx.x + 256u * k < size) {
        sum = fmaf(xv[k], xv[k], sum);
      }
    }
  } else {
    for (uint32_t i = threadIdx.x; i < size; i += 256u) {
      const float v = x[i];
      sum = fmaf(v, v, sum);
    }
  }
  sum = wave_sum(sum);
  if ((threadIdx.x & 63) == 0) {
    s_part[threadIdx.x >> 6] = sum;
  }
  __syncthreads();
  const float total = (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]);
  const float scale = 1.0f / sqrtf(total / (float)size + eps);
  if (held) {
#pragma unroll
    for (uint32_t k = 0; k < kHeld; ++k) {
      const uint32_t i = threadIdx.x + 256u * k;
      if (i < size) {
        y[i] = xv[k] * scale * wv[k];
      }
    }
  } else {
    for (uint32_t i = threadIdx.x; i < size; i += 256u) {
      y[i] = x[i] * scale * weight[i];
    }
  }
}

template <BinaryKind K>
__global__ void binary_kernel(float* target, const float* rhs, size_t size, size_t row_size) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < size;
       i += (size_t)gridDim.x * blockDim.x) {
    if (K == BinaryKind::mul) {
      target[i] *= rhs[i];
    } else if (K == BinaryKind::add_row) {
      target[i] += rhs[i % row_size];
    } else if (K == BinaryKind::mul_row) {
      target[i] *= rhs[i % row_size];
    } else if (K == BinaryKind::add) {
      target[i] += rhs[i];
    } else {
      // silu(gate) * up, as silu_mul_f32_in_place writes it (mps_backend.mm:2620-2629).
      // No contraction into the inlined expf (the K-quant GEMM's first pass
      // forms the same product and must get the same bits).
#pragma clang fp contract(off)
      const float g = target[i];
      target[i] = (g / (1.0f + expf(-g))) * rhs[i];
    }
  }
}

unsigned grid_for(size_t total, unsigned block = 256) {
  size_t blocks = (total + block - 1) / block;
  if (blocks < 1) {
    blocks = 1;
  }
  if (blocks > 65535) {
    blocks = 65535;
  }
  return (unsigned)blocks;
}

}  // namespace

hipError_t launch_rms_norm_rows(const float* input, const float* weight, float* output,
                                uint32_t rows, uint32_t size, float eps, hipStream_t stream) {
  rms_norm_rows_kernel<<<rows, 256, 0, stream>>>(input, weight, output, size, eps);
  return hipGetLastError();
}

hipError_t launch_rms_norm_heads(float* values, const float* weight, const float* gate,
                                 uint32_t tokens, uint32_t heads, uint32_t head_dim, float eps,
                                 hipStream_t stream) {
  const uint32_t rows = tokens * heads;
  const unsigned grid = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  rms_norm_heads_kernel<<<grid, 256, 0, stream>>>(values, weight, gate, rows, head_dim, eps);
  return hipGetLastError();
}

hipError_t launch_l2_norm(float* values, uint32_t rows, uint32_t row_size, float eps,
                          hipStream_t stream) {
  const unsigned grid = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  l2_norm_kernel<<<grid, 256, 0, stream>>>(values, rows, row_size, eps);
  return hipGetLastError();
}

hipError_t launch_split_qkv_l2(const float* source, float* q, float* k, float* v,
                               uint32_t tokens, uint32_t key_heads, uint32_t value_heads,
                               uint32_t head_dim, float eps, hipStream_t stream) {
  const uint64_t units = (uint64_t)tokens * (2u * key_heads + value_heads);
  const unsigned grid = (unsigned)((units + kRowsPerBlock - 1) / kRowsPerBlock);
  split_qkv_l2_kernel<<<grid, 256, 0, stream>>>(source, q, k, v, tokens, key_heads, value_heads,
                                                head_dim, eps);
  return hipGetLastError();
}

hipError_t launch_prepare_gate_beta(float* gate, float* beta, const float* bias,
                                    const float* scale, uint32_t rows, uint32_t row_size,
                                    hipStream_t stream) {
  const size_t total = (size_t)rows * row_size;
  prepare_gate_beta_kernel<<<grid_for(total), 256, 0, stream>>>(gate, beta, bias, scale, total,
                                                                 row_size);
  return hipGetLastError();
}

hipError_t launch_mrope(float* values, const int32_t* positions, uint32_t tokens,
                        uint32_t heads, uint32_t head_dim, uint32_t n_dims, uint32_t s0,
                        uint32_t s1, uint32_t s2, uint32_t s3, float theta,
                        hipStream_t stream) {
  if (s0 + s1 + s2 + s3 == 0 || n_dims < 2) {
    return hipSuccess;  // the reference kernel returns early (mps_backend.mm:2496-2498)
  }
  const size_t total = (size_t)tokens * heads * (n_dims / 2u);
  mrope_kernel<<<grid_for(total), 256, 0, stream>>>(values, positions, tokens, heads, head_dim,
                                                     n_dims, s0, s1, s2, s3, theta);
  return hipGetLastError();
}

hipError_t launch_copy_rows(CopyKind kind, const void* source, void* destination, size_t rows,
                            size_t row_size, size_t source_stride, size_t source_offset,
                            size_t destination_stride, size_t destination_offset,
                            hipStream_t stream) {
  const size_t total = rows * row_size;
  const unsigned grid = grid_for(total);
  switch (kind) {
    case CopyKind::f32:
      copy_rows_kernel<float, float><<<grid, 256, 0, stream>>>(
        static_cast<const float*>(source), static_cast<float*>(destination), total, row_size,
        source_stride, source_offset, destination_stride, destination_offset);
      break;
    case CopyKind::f32_to_f16:
      copy_rows_kernel<float, half_t><<<grid, 256, 0, stream>>>(
        static_cast<const float*>(source), static_cast<half_t*>(destination), total, row_size,
        source_stride, source_offset, destination_stride, destination_offset);
      break;
    case CopyKind::f16:
      copy_rows_kernel<half_t, half_t><<<grid, 256, 0, stream>>>(
        static_cast<const half_t*>(source), static_cast<half_t*>(destination), total, row_size,
        source_stride, source_offset, destination_stride, destination_offset);
      break;
  }
  return hipGetLastError();
}

hipError_t launch_append_kv_ragged(const float* key_rows, const float* value_rows,
                                   void* key_pool, void* value_pool,
                                   const uint64_t* seq_offsets, const uint32_t* seq_positions,
                                   uint64_t pool_elems, uint32_t sequences, uint32_t row_size,
                                   hipStream_t stream) {
  const size_t total = (size_t)sequences * row_size;
  append_kv_ragged_kernel<<<grid_for(total), 256, 0, stream>>>(
    key_rows, value_rows, static_cast<half_t*>(key_pool), static_cast<half_t*>(value_pool),
    seq_offsets, seq_positions, pool_elems, sequences, row_size);
  return hipGetLastError();
}

hipError_t launch_unary(UnaryKind kind, float* values, size_t size, hipStream_t stream) {
  const unsigned grid = grid_for(size);
  switch (kind) {
    case UnaryKind::sigmoid:
      unary_kernel<UnaryKind::sigmoid><<<grid, 256, 0, stream>>>(values, size);
      break;
    case UnaryKind::softplus:
      unary_kernel<UnaryKind::softplus><<<grid, 256, 0, stream>>>(values, size);
      break;
    case UnaryKind::silu:
      unary_kernel<UnaryKind::silu><<<grid, 256, 0, stream>>>(values, size);
      break;
  }
  return hipGetLastError();
}

hipError_t launch_binary(BinaryKind kind, float* target, const float* rhs, size_t size,
                         size_t row_size, hipStream_t stream) {
  const unsigned grid = grid_for(size);
  switch (kind) {
    case BinaryKind::mul:
      binary_kernel<BinaryKind::mul><<<grid, 256, 0, stream>>>(target, rhs, size, row_size);
      break;
    case BinaryKind::add_row:
      binary_kernel<BinaryKind::add_row><<<grid, 256, 0, stream>>>(target, rhs, size, row_size);
      break;
    case BinaryKind::mul_row:
      binary_kernel<BinaryKind::mul_row><<<grid, 256, 0, stream>>>(target, rhs, size, row_size);
      break;
    case BinaryKind::add:
      binary_kernel<BinaryKind::add><<<grid, 256, 0, stream>>>(target, rhs, size, row_size);
      break;
    case BinaryKind::silu_mul:
      binary_kernel<BinaryKind::silu_mul><<<grid, 256, 0, stream>>>(target, rhs, size, row_size);
      break;
  }
  return hipGetLastError();
}

}  // namespace kraken
