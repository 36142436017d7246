// Achievable-rate probes for the benchmark (no counterpart in the reference):
// a streaming HBM read and an fp16 MFMA loop, the two ceilings the hot-path
// kernels are judged against besides the published peaks.  Built as its own
// library (libkraken_hip_diag.so) on top of the public C ABI, so the boundary
// library exports only the reference's interface.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "kraken_hip_diag.h"

namespace kraken_diag {
namespace {

typedef _Float16 half_t;
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));

thread_local std::string g_last_error;

int fail(int code, const std::string& message) {
  g_last_error = message;
  return code;
}

// Context validity and the validation-only answer: a live context always has
// a stream, a validation-only one has none.
int stream_of(kraken_hip_context* ctx, hipStream_t* stream) {
  *stream = static_cast<hipStream_t>(kraken_hip_context_stream(ctx));
  if (*stream == nullptr) {
    return fail(KRAKEN_UNAVAILABLE, "validation-only context: arguments accepted");
  }
  return KRAKEN_OK;
}

int check_f32(const kraken_buffer& b, size_t values, const char* name) {
  if (b.data == nullptr) {
    return fail(KRAKEN_INVALID_ARGUMENT, std::string("HIP ") + name + " buffer is not initialized");
  }
  if (b.byte_size < values * sizeof(float)) {
    return fail(KRAKEN_INVALID_ARGUMENT, std::string("HIP ") + name + " buffer is too small");
  }
  return KRAKEN_OK;
}

int launched(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(KRAKEN_INTERNAL_ERROR, std::string(what) + hipGetErrorString(e));
  }
  return KRAKEN_OK;
}

constexpr int kReadThreads = 256;
constexpr uint32_t kReadBlocks = 256;
constexpr int kMfmaThreads = 256;

// Grid-stride nontemporal 16-byte loads, eight in flight per lane; one sum per
// lane goes to `sink` so that the loads are kept.
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kReadThreads) void diag_stream_read_kernel(const f32x4_t* __restrict__ x,
                                                                      size_t n4, float* sink) {
  constexpr int U = 8;
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + (U - 1) * stride < n4; i += U * stride) {
    f32x4_t v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      v[u] = __builtin_nontemporal_load(x + i + u * stride);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      acc += v[u];
    }
  }
  for (; i < n4; i += stride) {
    acc += __builtin_nontemporal_load(x + i);
  }
  sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = acc[0] + acc[1] + acc[2] + acc[3];
}

// One wave per SIMD; each wave issues `iterations` x 8 v_mfma_f32_32x32x16_f16
// on four independent accumulators (32,768 flops each).
__global__ __launch_bounds__(kMfmaThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void diag_mfma_f16_kernel(uint32_t iterations, float* sink) {
  const int lane = threadIdx.x & 63;
  const half8_t a = half8_t{(half_t)(lane * 0.001f), 1, 1, 1, 1, 1, 1, 1};
  const half8_t b = half8_t{1, 2, 3, 4, 5, 6, 7, (half_t)(blockIdx.x * 0.001f)};
  float16_t acc[4] = {};
  for (uint32_t it = 0; it < iterations; ++it) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      acc[j & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[j & 3], 0, 0, 0);
    }
  }
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s += acc[j][r];
    }
  }
  sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}


// What the f16 matrix cores do with an f16 denormal operand: one wave runs
// v_mfma_f32_16x16x32_f16 and v_mfma_f32_16x16x16_f16 with a single nonzero
// element x at (row 0, k 0) of A (B all ones), then at (k 0, col 0) of B (A all
// ones), for x in {2^-15, 2^-24 (denormals), 2^-14 (smallest normal)}, and
// writes C[0][0] (lane 0, register 0 in both output layouts), which is x if the
// operand survives and 0 if it is flushed.  sink[4 v + 2 i + o]: value v,
// instruction i (0: 16x16x32, 1: 16x16x16), operand o (0: A, 1: B).
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));
constexpr int kDenormalCases = 12;

__global__ __launch_bounds__(64) void diag_mfma_denormal_kernel(float* sink) {
  const int lane = threadIdx.x;
  const float values[3] = {0x1p-15f, 0x1p-24f, 0x1p-14f};
#pragma unroll
  for (int v = 0; v < 3; ++v) {
    const half_t x = static_cast<half_t>(values[v]);
    half8_t one8, pick8;
    half4_t one4, pick4;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      one8[j] = 1;
      pick8[j] = (lane == 0 && j == 0) ? x : half_t(0);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      one4[j] = 1;
      pick4[j] = (lane == 0 && j == 0) ? x : half_t(0);
    }
    const float4_t zero = {0.f, 0.f, 0.f, 0.f};
    const float4_t a32 = __builtin_amdgcn_mfma_f32_16x16x32_f16(pick8, one8, zero, 0, 0, 0);
    const float4_t b32 = __builtin_amdgcn_mfma_f32_16x16x32_f16(one8, pick8, zero, 0, 0, 0);
    const float4_t a16 = __builtin_amdgcn_mfma_f32_16x16x16f16(pick4, one4, zero, 0, 0, 0);
    const float4_t b16 = __builtin_amdgcn_mfma_f32_16x16x16f16(one4, pick4, zero, 0, 0, 0);
    if (lane == 0) {
      sink[4 * v + 0] = a32[0];
      sink[4 * v + 1] = b32[0];
      sink[4 * v + 2] = a16[0];
      sink[4 * v + 3] = b16[0];
    }
  }
}

}  // namespace
}  // namespace kraken_diag

using namespace kraken_diag;

extern "C" {

KRAKEN_API const char* kraken_hip_diag_last_error(void) { return g_last_error.c_str(); }

KRAKEN_API int kraken_hip_diag_stream_read(kraken_hip_context* ctx, kraken_buffer source,
                                           size_t bytes, kraken_buffer sink) {
  if (ctx == nullptr) {
    return fail(KRAKEN_UNAVAILABLE, "HIP context is not initialized");
  }
  if (bytes == 0 || bytes % 16 != 0) {
    return fail(KRAKEN_INVALID_ARGUMENT, "HIP stream read bytes must be a positive multiple of 16");
  }
  int s = check_f32(source, bytes / 4, "stream read source");
  if (s == KRAKEN_OK) {
    s = check_f32(sink, (size_t)kReadBlocks * kReadThreads, "stream read sink");
  }
  if (s != KRAKEN_OK) {
    return s;
  }
  if (((uintptr_t)source.data & 15u) != 0) {
    return fail(KRAKEN_INVALID_ARGUMENT, "HIP stream read source must be 16-byte aligned");
  }
  hipStream_t stream;
  if ((s = stream_of(ctx, &stream)) != KRAKEN_OK) {
    return s;
  }
  diag_stream_read_kernel<<<kReadBlocks, kReadThreads, 0, stream>>>(
    static_cast<const f32x4_t*>(source.data), bytes / 16, static_cast<float*>(sink.data));
  return launched("HIP stream read launch failed: ");
}

KRAKEN_API int kraken_hip_diag_mfma_f16(kraken_hip_context* ctx, uint32_t workgroups,
                                        uint32_t iterations, kraken_buffer sink) {
  if (ctx == nullptr) {
    return fail(KRAKEN_UNAVAILABLE, "HIP context is not initialized");
  }
  if (workgroups == 0 || iterations == 0) {
    return fail(KRAKEN_INVALID_ARGUMENT, "HIP MFMA loop workgroups and iterations must be positive");
  }
  int s = check_f32(sink, (size_t)workgroups * kMfmaThreads, "MFMA loop sink");
  if (s != KRAKEN_OK) {
    return s;
  }
  hipStream_t stream;
  if ((s = stream_of(ctx, &stream)) != KRAKEN_OK) {
    return s;
  }
  diag_mfma_f16_kernel<<<workgroups, kMfmaThreads, 0, stream>>>(iterations,
                                                               static_cast<float*>(sink.data));
  return launched("HIP MFMA loop launch failed: ");
}

KRAKEN_API int kraken_hip_diag_mfma_f16_denormals(kraken_hip_context* ctx, kraken_buffer sink) {
  if (ctx == nullptr) {
    return fail(KRAKEN_UNAVAILABLE, "HIP context is not initialized");
  }
  int s = check_f32(sink, kDenormalCases, "MFMA denormal probe sink");
  if (s != KRAKEN_OK) {
    return s;
  }
  hipStream_t stream;
  if ((s = stream_of(ctx, &stream)) != KRAKEN_OK) {
    return s;
  }
  diag_mfma_denormal_kernel<<<1, 64, 0, stream>>>(static_cast<float*>(sink.data));
  return launched("HIP MFMA denormal probe launch failed: ");
}

}  // extern "C"
