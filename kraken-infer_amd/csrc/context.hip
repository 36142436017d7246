// Context, stream batching, buffers and host copies of the C ABI.
//
// Mirrors the non-kernel half of toyllm::mps::MpsContext
// (mps_backend.hpp:76-115; mps_backend.mm:4312-4467, 5043-5085, 5763-5874) on a
// HIP stream: ops enqueue on the context's stream; outside begin/commit_graph an
// op waits for its own completion, inside one the batch waits once at commit.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <string>

#include "context_internal.hpp"
#include "device_common.hpp"

namespace kraken {
namespace {

thread_local std::string g_last_error;

std::string hip_message(hipError_t e) {
  return std::string(hipGetErrorName(e)) + ": " + hipGetErrorString(e);
}

__global__ void fill_zero_bytes(uint8_t* dst, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  // 16-byte body when aligned, byte tail otherwise.
  if (((uintptr_t)dst & 15u) == 0) {
    const size_t vec = n / 16;
    uint4* d16 = reinterpret_cast<uint4*>(dst);
    for (size_t j = i; j < vec; j += stride) {
      d16[j] = make_uint4(0, 0, 0, 0);
    }
    for (size_t j = vec * 16 + i; j < n; j += stride) {
      dst[j] = 0;
    }
  } else {
    for (size_t j = i; j < n; j += stride) {
      dst[j] = 0;
    }
  }
}

}  // namespace

int fail(int code, const std::string& message) {
  g_last_error = message;
  return code;
}

int check_context(const kraken_hip_context* ctx) {
  if (ctx == nullptr) {
    return unavailable("HIP context is not initialized");
  }
  return KRAKEN_OK;
}

int begin_launch(kraken_hip_context* ctx) {
  if (ctx->validation_only) {
    return unavailable("validation-only context: arguments accepted");
  }
  const hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) {
    return internal("HIP set device failed: " + hip_message(e));
  }
  return KRAKEN_OK;
}

int finish_launch(kraken_hip_context* ctx, const char* error_prefix) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return internal(std::string(error_prefix) + hip_message(e));
  }
  if (ctx->graph_active) {
    return KRAKEN_OK;
  }
  e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    return internal(std::string(error_prefix) + hip_message(e));
  }
  return KRAKEN_OK;
}

int ensure_workspace(kraken_hip_context* ctx, size_t bytes) {
  if (ctx->validation_only || bytes <= ctx->workspace_bytes) {
    return KRAKEN_OK;
  }
  // Round up to 1 MiB and at least double, so steady-state calls never
  // reallocate and the retired workspaces stay smaller than the live one.
  size_t rounded = (bytes + (1u << 20) - 1) & ~static_cast<size_t>((1u << 20) - 1);
  if (ctx->workspace_bytes > 0 && rounded < 2 * ctx->workspace_bytes) {
    rounded = 2 * ctx->workspace_bytes;
  }
  void* fresh = nullptr;
  const hipError_t e = hipMalloc(&fresh, rounded);
  if (e != hipSuccess) {
    return internal("HIP workspace allocation failed: " + hip_message(e));
  }
  // Kernels already enqueued, and graphs captured earlier, may still use the
  // old workspace: keep it until the context is destroyed.
  if (ctx->workspace != nullptr) {
    ctx->retired_workspaces.push_back(ctx->workspace);
  }
  ctx->workspace = fresh;
  ctx->workspace_bytes = rounded;
  return KRAKEN_OK;
}

int check_u32(size_t value, const char* name) {
  if (!fits_u32(value)) {
    return invalid(std::string("HIP ") + name + " exceeds uint32 range");
  }
  return KRAKEN_OK;
}

int validate_buffer(const kraken_buffer& buffer, size_t values, size_t element_bytes,
                    const char* name) {
  size_t bytes = 0;
  if (!checked_mul(values, element_bytes, bytes)) {
    return invalid(std::string("HIP ") + name + " byte count overflow");
  }
  if (buffer.data == nullptr) {
    return invalid(std::string("HIP ") + name + " buffer is not initialized");
  }
  if (buffer.byte_size < bytes) {
    return invalid(std::string("HIP ") + name + " buffer is too small");
  }
  return KRAKEN_OK;
}

int validate_f32_region(const kraken_buffer& b, size_t offset, size_t values,
                        const char* name) {
  if (b.data == nullptr) {
    return invalid(std::string("HIP ") + name + " buffer is not initialized");
  }
  size_t offset_bytes = 0;
  size_t bytes = 0;
  if (!checked_mul(offset, sizeof(float), offset_bytes) ||
      !checked_mul(values, sizeof(float), bytes)) {
    return invalid(std::string("HIP ") + name + " byte count overflow");
  }
  if (offset_bytes > b.byte_size || bytes > b.byte_size - offset_bytes) {
    return invalid(std::string("HIP ") + name + " buffer region is too small");
  }
  return KRAKEN_OK;
}

int strided_region_end(size_t offset, size_t rows, size_t stride, size_t row_size,
                       const char* name, size_t& end) {
  if (rows == 0 || row_size == 0) {
    return invalid(std::string("HIP ") + name + " rows and row size must be positive");
  }
  if (stride < row_size) {
    return invalid(std::string("HIP ") + name + " stride must be at least row size");
  }
  size_t last_row = 0;
  if (!checked_mul(rows - 1u, stride, last_row)) {
    return invalid(std::string("HIP ") + name + " row offset overflow");
  }
  size_t last_offset = 0;
  if (!checked_add(offset, last_row, last_offset)) {
    return invalid(std::string("HIP ") + name + " offset overflow");
  }
  if (!checked_add(last_offset, row_size, end)) {
    return invalid(std::string("HIP ") + name + " end offset overflow");
  }
  return KRAKEN_OK;
}

}  // namespace kraken

using namespace kraken;

namespace {

// commit_graph() as the reference's host copies call it first
// (mps_backend.mm:5786, 5818, 5847): ends an open batch and waits.
int commit_pending(kraken_hip_context* ctx) {
  if (ctx->validation_only) {
    ctx->graph_active = false;
    return KRAKEN_OK;
  }
  ctx->graph_active = false;
  const hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    return internal("HIP graph command failed: " + hip_message(e));
  }
  return KRAKEN_OK;
}

}  // namespace

extern "C" {

KRAKEN_API const char* kraken_hip_last_error(void) { return g_last_error.c_str(); }

KRAKEN_API int kraken_hip_context_create(kraken_hip_context** out_context) {
  if (out_context == nullptr) {
    return invalid("HIP context output pointer must not be null");
  }
  *out_context = nullptr;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count <= 0) {
    return unavailable("HIP backend: no HIP device is available" +
                       (e != hipSuccess ? " (" + hip_message(e) + ")" : std::string()));
  }
  int device = 0;
  e = hipGetDevice(&device);
  if (e != hipSuccess) {
    return unavailable("HIP backend: cannot query the current device: " + hip_message(e));
  }
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) {
    return unavailable("HIP backend: cannot query device properties: " + hip_message(e));
  }
  auto* ctx = new kraken_hip_context();
  ctx->device = device;
  ctx->cu_count = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
  // Default-priority, non-blocking stream: never synchronises with the null stream.
  e = hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete ctx;
    return unavailable("HIP backend: stream creation failed: " + hip_message(e));
  }
  ctx->stream = ctx->own_stream;
  const int scratch_status = resolve_no_alloc_scratch(device, &ctx->no_alloc_scratch);
  if (scratch_status != KRAKEN_OK) {
    (void)hipStreamDestroy(ctx->own_stream);
    delete ctx;
    return scratch_status;
  }
  *out_context = ctx;
  return KRAKEN_OK;
}

KRAKEN_API int kraken_hip_context_create_validation_only(kraken_hip_context** out_context) {
  if (out_context == nullptr) {
    return invalid("HIP context output pointer must not be null");
  }
  auto* ctx = new kraken_hip_context();
  ctx->validation_only = true;
  ctx->cu_count = 256;
  *out_context = ctx;
  return KRAKEN_OK;
}

KRAKEN_API void kraken_hip_context_destroy(kraken_hip_context* ctx) {
  if (ctx == nullptr) {
    return;
  }
  if (!ctx->validation_only) {
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->workspace != nullptr) {
      (void)hipFree(ctx->workspace);
    }
    for (void* w : ctx->retired_workspaces) {
      (void)hipFree(w);
    }
    if (ctx->own_stream != nullptr) {
      (void)hipStreamDestroy(ctx->own_stream);
    }
  }
  delete ctx;
}

KRAKEN_API int kraken_hip_context_set_stream(kraken_hip_context* ctx, void* hip_stream) {
  int s = check_context(ctx);
  if (s != KRAKEN_OK) {
    return s;
  }
  if (ctx->graph_active) {
    return invalid("HIP stream cannot change while a graph is active");
  }
  if (!ctx->validation_only) {
    // Work already enqueued on the old stream must finish before the switch.
    const hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
      return internal("HIP stream switch wait failed: " + hip_message(e));
    }
  }
  ctx->stream = hip_stream != nullptr ? static_cast<hipStream_t>(hip_stream) : ctx->own_stream;
  return KRAKEN_OK;
}

KRAKEN_API void* kraken_hip_context_stream(const kraken_hip_context* ctx) {
  return ctx == nullptr ? nullptr : static_cast<void*>(ctx->stream);
}

KRAKEN_API int kraken_hip_begin_graph(kraken_hip_context* ctx) {
  int s = check_context(ctx);
  if (s != KRAKEN_OK) {
    return s;
  }
  if (ctx->graph_active) {
    return invalid("HIP graph execution is already active");
  }
  ctx->graph_active = true;
  return KRAKEN_OK;
}

KRAKEN_API int kraken_hip_commit_graph(kraken_hip_context* ctx) {
  int s = check_context(ctx);
  if (s != KRAKEN_OK) {
    return s;
  }
  if (!ctx->graph_active) {
    return KRAKEN_OK;
  }
  return commit_pending(ctx);
}

KRAKEN_API void kraken_hip_abort_graph(kraken_hip_context* ctx) {
  if (ctx == nullptr) {
    return;
  }
  // Work already enqueued cannot be withdrawn from a HIP stream; it is waited for
  // so nothing is left pending once the batch is abandoned.
  if (ctx->graph_active && !ctx->validation_only) {
    (void)hipStreamSynchronize(ctx->stream);
  }
  ctx->graph_active = false;
}

KRAKEN_API int kraken_hip_make_buffer(kraken_hip_context* ctx, size_t byte_size,
                                      kraken_buffer* out_buffer) {
  int s = check_context(ctx);
  if (s != KRAKEN_OK) {
    return s;
  }
  if (out_buffer == nullptr) {
    return invalid("HIP buffer output pointer must not be null");
  }
  out_buffer->data = nullptr;
  out_buffer->byte_size = 0;
  if (byte_size == 0) {
    return invalid("HIP buffer size must be positive");
  }
  if (ctx->validation_only) {
    return unavailable("validation-only context: arguments accepted");
  }
  (void)hipSetDevice(ctx->device);
  void* p = nullptr;
  const hipError_t e = hipMalloc(&p, byte_size);
  if (e != hipSuccess) {
    return unavailable("HIP buffer allocation failed: " + hip_message(e));
  }
  out_buffer->data = p;
  out_buffer->byte_size = byte_size;
  return KRAKEN_OK;
}

KRAKEN_API int kraken_hip_free_buffer(kraken_hip_context* ctx, kraken_buffer* buffer) {
  int s = check_context(ctx);
  if (s != KRAKEN_OK) {
    return s;
  }
  if (buffer == nullptr || buffer->data == nullptr) {
    return KRAKEN_OK;
  }
  if (!ctx->validation_only) {
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    const hipError_t e = hipFree(buffer->data);
    if (e != hipSuccess) {
      return internal("HIP buffer free failed: " + hip_message(e));
    }
  }
  buffer->data = nullptr;
  buffer->byte_size = 0;
  return KRAKEN_OK;
}

KRAKEN_API int kraken_hip_copy_to_buffer_at(kraken_hip_context* ctx, kraken_buffer buffer,
                                            size_t destination_offset, const void* data,
                                            size_t byte_size) {
  int s = check_context(ctx);
  if (s != KRAKEN_OK) {
    return s;
  }
  if (buffer.data == nullptr) {
    return invalid("HIP buffer is not initialized");
  }
  if (data == nullptr) {
    return invalid("HIP copy source must not be null");
  }
  if (destination_offset > buffer.byte_size ||
      byte_size > buffer.byte_size - destination_offset) {
    return invalid("HIP copy size exceeds destination buffer size");
  }
  if ((s = commit_pending(ctx)) != KRAKEN_OK) {
    return s;
  }
  if ((s = begin_launch(ctx)) != KRAKEN_OK) {
    return s;
  }
  const hipError_t e =
    hipMemcpy(static_cast<uint8_t*>(buffer.data) + destination_offset, data, byte_size,
              hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    return internal("HIP copy to buffer failed: " + hip_message(e));
  }
  return KRAKEN_OK;
}

KRAKEN_API int kraken_hip_copy_to_buffer(kraken_hip_context* ctx, kraken_buffer buffer,
                                         const void* data, size_t byte_size) {
  return kraken_hip_copy_to_buffer_at(ctx, buffer, 0, data, byte_size);
}

KRAKEN_API int kraken_hip_copy_from_buffer_at(kraken_hip_context* ctx, kraken_buffer buffer,
                                              size_t source_offset, void* data,
                                              size_t byte_size) {
  int s = check_context(ctx);
  if (s != KRAKEN_OK) {
    return s;
  }
  if (buffer.data == nullptr) {
    return invalid("HIP buffer is not initialized");
  }
  if (data == nullptr) {
    return invalid("HIP copy destination must not be null");
  }
  if (source_offset > buffer.byte_size || byte_size > buffer.byte_size - source_offset) {
    return invalid("HIP copy size exceeds source buffer size");
  }
  if ((s = commit_pending(ctx)) != KRAKEN_OK) {
    return s;
  }
  if ((s = begin_launch(ctx)) != KRAKEN_OK) {
    return s;
  }
  const hipError_t e =
    hipMemcpy(data, static_cast<const uint8_t*>(buffer.data) + source_offset, byte_size,
              hipMemcpyDeviceToHost);
  if (e != hipSuccess) {
    return internal("HIP copy from buffer failed: " + hip_message(e));
  }
  return KRAKEN_OK;
}

KRAKEN_API int kraken_hip_copy_from_buffer(kraken_hip_context* ctx, kraken_buffer buffer,
                                           void* data, size_t byte_size) {
  return kraken_hip_copy_from_buffer_at(ctx, buffer, 0, data, byte_size);
}

KRAKEN_API int kraken_hip_copy_buffer_region(kraken_hip_context* ctx, kraken_buffer source,
                                             kraken_buffer destination, size_t source_offset,
                                             size_t destination_offset, size_t byte_size) {
  int s = check_context(ctx);
  if (s != KRAKEN_OK) {
    return s;
  }
  if (source.data == nullptr || destination.data == nullptr) {
    return invalid("HIP buffer is not initialized");
  }
  if (source_offset > source.byte_size || byte_size > source.byte_size - source_offset) {
    return invalid("HIP copy size exceeds source buffer size");
  }
  if (destination_offset > destination.byte_size ||
      byte_size > destination.byte_size - destination_offset) {
    return invalid("HIP copy size exceeds destination buffer size");
  }
  if ((s = commit_pending(ctx)) != KRAKEN_OK) {
    return s;
  }
  if ((s = begin_launch(ctx)) != KRAKEN_OK) {
    return s;
  }
  if (byte_size == 0) {
    return KRAKEN_OK;
  }
  const uint8_t* src = static_cast<const uint8_t*>(source.data) + source_offset;
  uint8_t* dst = static_cast<uint8_t*>(destination.data) + destination_offset;
  // Enqueued on the context's stream.  Overlapping ranges get memmove
  // semantics (mps_backend.mm:5855-5856) through the context workspace.
  const bool overlap = src < dst + byte_size && dst < src + byte_size;
  hipError_t e;
  if (overlap) {
    if ((s = ensure_workspace(ctx, byte_size)) != KRAKEN_OK) {
      return s;
    }
    e = hipMemcpyAsync(ctx->workspace, src, byte_size, hipMemcpyDeviceToDevice, ctx->stream);
    if (e == hipSuccess) {
      e = hipMemcpyAsync(dst, ctx->workspace, byte_size, hipMemcpyDeviceToDevice, ctx->stream);
    }
  } else {
    e = hipMemcpyAsync(dst, src, byte_size, hipMemcpyDeviceToDevice, ctx->stream);
  }
  if (e != hipSuccess) {
    return internal("HIP buffer region copy failed: " + hip_message(e));
  }
  return finish_launch(ctx, "HIP buffer region copy failed: ");
}

KRAKEN_API int kraken_hip_zero_buffer(kraken_hip_context* ctx, kraken_buffer buffer,
                                      size_t byte_size) {
  int s = check_context(ctx);
  if (s != KRAKEN_OK) {
    return s;
  }
  if (buffer.data == nullptr) {
    return invalid("HIP buffer is not initialized");
  }
  if (byte_size > buffer.byte_size) {
    return invalid("HIP zero size exceeds buffer size");
  }
  if ((s = begin_launch(ctx)) != KRAKEN_OK) {
    return s;
  }
  if (byte_size == 0) {
    return KRAKEN_OK;
  }
  // Enqueued on the stream (ordered with earlier ops), unlike the reference's
  // immediate CPU memset (mps_backend.mm:5861-5874).
  const size_t blocks = (byte_size / 16 + 255) / 256;
  const unsigned grid = static_cast<unsigned>(blocks < 1 ? 1 : (blocks > 4096 ? 4096 : blocks));
  fill_zero_bytes<<<grid, 256, 0, ctx->stream>>>(static_cast<uint8_t*>(buffer.data), byte_size);
  return finish_launch(ctx, "HIP zero buffer command failed: ");
}

}  // extern "C"
