// kraken_hip_copy_regions: up to KRAKEN_COPY_REGIONS_MAX byte ranges between
// two buffers in one launch (no counterpart in the reference).  The ranges
// travel as a kernel argument, so the launch needs no device table and no
// host-to-device upload.  Each workgroup copies one tile of kTileBytes of one
// range; 16-byte vector moves where source and destination are both 16-byte
// aligned at the tile start, bytes otherwise.
#include <hip/hip_runtime.h>

#include <string>

#include "context_internal.hpp"
#include "kraken_hip.h"

namespace kraken {
namespace {

constexpr int kCopyThreads = 256;
constexpr int kVecPerThread = 4;
constexpr size_t kTileBytes = (size_t)kCopyThreads * kVecPerThread * 16;  // 16 KiB

struct CopyRegionArgs {
  const unsigned char* source;
  unsigned char* destination;
  uint64_t source_offset[KRAKEN_COPY_REGIONS_MAX];
  uint64_t destination_offset[KRAKEN_COPY_REGIONS_MAX];
  uint64_t bytes[KRAKEN_COPY_REGIONS_MAX];
  uint32_t first_tile[KRAKEN_COPY_REGIONS_MAX + 1];  // prefix sums of tiles per range
  uint32_t count;
};

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kCopyThreads) void copy_regions_kernel(CopyRegionArgs a) {
  const uint32_t tile = blockIdx.x;
  uint32_t r = 0;
  while (r + 1 < a.count && a.first_tile[r + 1] <= tile) {
    ++r;
  }
  const uint64_t begin = (uint64_t)(tile - a.first_tile[r]) * kTileBytes;
  const uint64_t n = min((uint64_t)kTileBytes, a.bytes[r] - begin);
  const unsigned char* src = a.source + a.source_offset[r] + begin;
  unsigned char* dst = a.destination + a.destination_offset[r] + begin;
  const bool vec = (((uintptr_t)src | (uintptr_t)dst) & 15u) == 0;
  const uint64_t nv = vec ? n / 16 : 0;
  const u32x4_t* s4 = reinterpret_cast<const u32x4_t*>(src);
  u32x4_t* d4 = reinterpret_cast<u32x4_t*>(dst);
  if (nv == (uint64_t)kCopyThreads * kVecPerThread) {
    u32x4_t v[kVecPerThread];
#pragma unroll
    for (int u = 0; u < kVecPerThread; ++u) {
      v[u] = __builtin_nontemporal_load(s4 + u * kCopyThreads + threadIdx.x);
    }
#pragma unroll
    for (int u = 0; u < kVecPerThread; ++u) {
      __builtin_nontemporal_store(v[u], d4 + u * kCopyThreads + threadIdx.x);
    }
  } else {
    for (uint64_t i = threadIdx.x; i < nv; i += kCopyThreads) {
      d4[i] = s4[i];
    }
  }
  for (uint64_t i = nv * 16 + threadIdx.x; i < n; i += kCopyThreads) {
    dst[i] = src[i];
  }
}

}  // namespace
}  // namespace kraken

using namespace kraken;

extern "C" {

KRAKEN_API int kraken_hip_copy_regions(kraken_hip_context* ctx, kraken_buffer source,
                                       kraken_buffer destination,
                                       const kraken_copy_region* regions, size_t count) {
  KRAKEN_TRY(check_context(ctx));
  if (source.data == nullptr || destination.data == nullptr) {
    return invalid("HIP buffer is not initialized");
  }
  if (count > KRAKEN_COPY_REGIONS_MAX) {
    return invalid("HIP copy regions: at most " + std::to_string(KRAKEN_COPY_REGIONS_MAX) +
                   " regions per call");
  }
  if (count > 0 && regions == nullptr) {
    return invalid("HIP copy regions: region list is null");
  }
  CopyRegionArgs a{};
  a.source = static_cast<const unsigned char*>(source.data);
  a.destination = static_cast<unsigned char*>(destination.data);
  uint64_t tiles = 0;
  for (size_t i = 0; i < count; ++i) {
    const kraken_copy_region& g = regions[i];
    if (g.source_offset > source.byte_size || g.byte_size > source.byte_size - g.source_offset) {
      return invalid("HIP copy regions: region " + std::to_string(i) +
                     " exceeds source buffer size");
    }
    if (g.destination_offset > destination.byte_size ||
        g.byte_size > destination.byte_size - g.destination_offset) {
      return invalid("HIP copy regions: region " + std::to_string(i) +
                     " exceeds destination buffer size");
    }
    if (g.byte_size == 0) {
      continue;
    }
    a.source_offset[a.count] = g.source_offset;
    a.destination_offset[a.count] = g.destination_offset;
    a.bytes[a.count] = g.byte_size;
    a.first_tile[a.count] = (uint32_t)tiles;
    tiles += (g.byte_size + kTileBytes - 1) / kTileBytes;
    if (tiles > 0x7fffffffu) {
      return invalid("HIP copy regions: total size exceeds one launch");
    }
    ++a.count;
  }
  a.first_tile[a.count] = (uint32_t)tiles;
  KRAKEN_TRY(begin_launch(ctx));
  if (tiles == 0) {
    return KRAKEN_OK;
  }
  copy_regions_kernel<<<dim3((uint32_t)tiles), kCopyThreads, 0, ctx->stream>>>(a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return internal(std::string{"HIP copy regions launch failed: "} + hipGetErrorString(e));
  }
  return finish_launch(ctx, "HIP copy regions command failed: ");
}

}  // extern "C"
