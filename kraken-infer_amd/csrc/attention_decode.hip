// Split-K causal GQA attention over a KV cache, for decode and short chunks.
//
// Semantics: reference MSL attention_f32_batched_f16_kv / attention_f32_batched
// (mps_backend.mm:2879-3008): query token t at position start+t attends cache
// keys 0..position of its KV head (kv_head = head / group), scale 1/sqrt(D),
// f32 query times f16 (or f32) cache, fp32 accumulation, out = o/den (0 if
// den == 0).  The optional gate applies the full-attention output gate
// out *= sigmoid(G) (qwen35_runtime.cpp:3347-3355) in the epilogue.
//
// Design (gfx950, wave64):
//  * Pass 1 (attention_split): one workgroup of 4 waves per (token, kv_head,
//    key split).  The workgroup serves all G query heads of the GQA group, so
//    each K/V row is fetched once for G heads.  A wave takes 8 keys per step:
//    lane = 8*key_slot + chunk, each lane loads 16-byte chunks (chunk + 8*i) of
//    its key's K and V rows, so one load instruction moves 8 x 128 contiguous
//    bytes.  Dot products reduce over the 8 lanes of a key with DPP; the online
//    softmax runs in the log2 domain (q pre-scaled by log2(e)/sqrt(D)) with a
//    wave-uniform running max.  Waves merge through LDS; the workgroup writes
//    (m, l, o[G][D]) for its split, or the final (gated) output if unsplit.
//  * Pass 2 (attention_combine): one workgroup per (token, head) rescales and
//    sums the split partials, divides by the total denominator, applies the gate.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdlib>

#include "context_internal.hpp"
#include "device_common.hpp"

namespace kraken {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kKeysPerWaveStep = 8;
constexpr int kMaxSplits = 1024;

struct DecodeParams {
  const float* query;
  const void* key_cache;
  const void* value_cache;
  const float* gate;
  float* output;
  float* partial_o;   // [tokens][kv_heads][splits][G][D]
  float* partial_ml;  // [tokens][kv_heads][splits][G][2]
  uint32_t layer, start_position, tokens, capacity_tokens, heads, kv_heads;
  uint32_t keys_per_split, splits;
  float scale_log2;
};

template <typename KV>
struct KvTraits;
template <>
struct KvTraits<half_t> {
  static constexpr int kPerChunk = 8;  // elements per 16-byte chunk
  __device__ static void to_float(const u32x4_t& raw, float* out) {
    const half2_t* h = reinterpret_cast<const half2_t*>(&raw);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = static_cast<float>(h[i].x);
      out[2 * i + 1] = static_cast<float>(h[i].y);
    }
  }
};
template <>
struct KvTraits<float> {
  static constexpr int kPerChunk = 4;
  __device__ static void to_float(const u32x4_t& raw, float* out) {
    out[0] = __uint_as_float(raw.x);
    out[1] = __uint_as_float(raw.y);
    out[2] = __uint_as_float(raw.z);
    out[3] = __uint_as_float(raw.w);
  }
};

__device__ __forceinline__ float sigmoidf_acc(float x) { return 1.0f / (1.0f + expf(-x)); }

template <int D, int G, typename KV>
__global__ __launch_bounds__(kThreads) void attention_split(DecodeParams p) {
  using T = KvTraits<KV>;
  constexpr int E = T::kPerChunk;
  constexpr int kChunksPerRow = D / E;
  constexpr int kChunksPerLane = kChunksPerRow / 8;
  constexpr int kDimsPerLane = kChunksPerLane * E;  // == D / 8
  static_assert(kChunksPerRow % 8 == 0, "row must split into 8 lanes of 16B chunks");

  __shared__ float s_o[kWaves][2][G][D];
  __shared__ float s_m[kWaves][G];
  __shared__ float s_l[kWaves][G];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int slot = lane >> 3;
  const int c8 = lane & 7;
  const uint32_t split = blockIdx.x;
  const uint32_t kvh = blockIdx.y;
  const uint32_t token = blockIdx.z;
  const uint32_t position = p.start_position + token;
  const uint32_t n_keys = position + 1u;
  const uint32_t key_begin = split * p.keys_per_split;
  uint32_t key_end = key_begin + p.keys_per_split;
  if (key_end > n_keys) {
    key_end = n_keys;
  }

  // Query heads kvh*G .. kvh*G+G-1, pre-scaled into the log2 domain.
  float qv[G][kDimsPerLane];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float* qrow = p.query + ((size_t)token * p.heads + kvh * G + g) * D;
#pragma unroll
    for (int i = 0; i < kChunksPerLane; ++i) {
      const int d0 = (c8 + 8 * i) * E;
#pragma unroll
      for (int e = 0; e < E; e += 4) {
        const float4 v = *reinterpret_cast<const float4*>(qrow + d0 + e);
        qv[g][i * E + e + 0] = v.x * p.scale_log2;
        qv[g][i * E + e + 1] = v.y * p.scale_log2;
        qv[g][i * E + e + 2] = v.z * p.scale_log2;
        qv[g][i * E + e + 3] = v.w * p.scale_log2;
      }
    }
  }

  float m[G];
  float l[G];
  float o[G][kDimsPerLane];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.0f;
#pragma unroll
    for (int d = 0; d < kDimsPerLane; ++d) {
      o[g][d] = 0.0f;
    }
  }

  const size_t row_stride = (size_t)p.kv_heads * D;  // elements between consecutive keys
  const KV* kbase = static_cast<const KV*>(p.key_cache) +
                    ((size_t)p.layer * p.capacity_tokens) * row_stride + (size_t)kvh * D;
  const KV* vbase = static_cast<const KV*>(p.value_cache) +
                    ((size_t)p.layer * p.capacity_tokens) * row_stride + (size_t)kvh * D;

  for (uint32_t kb = key_begin + wave * kKeysPerWaveStep; kb < key_end;
       kb += kWaves * kKeysPerWaveStep) {
    const uint32_t key = kb + slot;
    const bool valid = key < key_end;
    u32x4_t kraw[kChunksPerLane];
    u32x4_t vraw[kChunksPerLane];
    if (valid) {
      const u32x4_t* krow = reinterpret_cast<const u32x4_t*>(kbase + (size_t)key * row_stride);
      const u32x4_t* vrow = reinterpret_cast<const u32x4_t*>(vbase + (size_t)key * row_stride);
#pragma unroll
      for (int i = 0; i < kChunksPerLane; ++i) {
        kraw[i] = __builtin_nontemporal_load(krow + c8 + 8 * i);
      }
#pragma unroll
      for (int i = 0; i < kChunksPerLane; ++i) {
        vraw[i] = __builtin_nontemporal_load(vrow + c8 + 8 * i);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kChunksPerLane; ++i) {
        kraw[i] = u32x4_t{0u, 0u, 0u, 0u};
        vraw[i] = u32x4_t{0u, 0u, 0u, 0u};
      }
    }
    float kf[kDimsPerLane];
#pragma unroll
    for (int i = 0; i < kChunksPerLane; ++i) {
      T::to_float(kraw[i], kf + i * E);
    }
    float s[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float acc = 0.0f;
#pragma unroll
      for (int d = 0; d < kDimsPerLane; ++d) {
        acc = fmaf(qv[g][d], kf[d], acc);
      }
      acc = reduce8_sum(acc);
      s[g] = valid ? acc : -INFINITY;
    }
    float vf[kDimsPerLane];
#pragma unroll
    for (int i = 0; i < kChunksPerLane; ++i) {
      T::to_float(vraw[i], vf + i * E);
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float step_max = halves_max(across8_max(s[g]));
      if (step_max > m[g]) {  // wave-uniform branch
        const float corr = fast_exp2(m[g] - step_max);
        l[g] *= corr;
#pragma unroll
        for (int d = 0; d < kDimsPerLane; ++d) {
          o[g][d] *= corr;
        }
        m[g] = step_max;
      }
      const float pr = valid ? fast_exp2(s[g] - m[g]) : 0.0f;
      l[g] += pr;
#pragma unroll
      for (int d = 0; d < kDimsPerLane; ++d) {
        o[g][d] = fmaf(pr, vf[d], o[g][d]);
      }
    }
  }

  // Merge the 8 key slots of the wave: slots 0..3 and 4..7 within each half via
  // DPP, the two halves through LDS.
#pragma unroll
  for (int g = 0; g < G; ++g) {
    // l is replicated over the 8 lanes of a slot; sum over slots.
    const float lw = halves_sum(across8_sum(l[g]));
#pragma unroll
    for (int d = 0; d < kDimsPerLane; ++d) {
      o[g][d] = across8_sum(o[g][d]);
    }
    if (lane == 0) {
      s_m[wave][g] = m[g];
      s_l[wave][g] = lw;
    }
    if ((lane & 31) < 8) {
      const int half = lane >> 5;
#pragma unroll
      for (int i = 0; i < kChunksPerLane; ++i) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
          s_o[wave][half][g][(c8 + 8 * i) * E + e] = o[g][i * E + e];
        }
      }
    }
  }
  __syncthreads();

  // Workgroup merge: thread handles (g, d) pairs.
  const size_t tk = (size_t)token * p.kv_heads + kvh;
  for (int idx = threadIdx.x; idx < G * D; idx += kThreads) {
    const int g = idx / D;
    const int d = idx % D;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      mx = fmaxf(mx, s_m[w][g]);
    }
    float acc = 0.0f;
    float den = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float wt = s_m[w][g] == -INFINITY ? 0.0f : fast_exp2(s_m[w][g] - mx);
      acc += wt * (s_o[w][0][g][d] + s_o[w][1][g][d]);
      den += wt * s_l[w][g];
    }
    if (p.splits == 1) {
      const uint32_t head = kvh * G + g;
      const size_t out_index = ((size_t)token * p.heads + head) * D + d;
      float r = den == 0.0f ? 0.0f : acc / den;
      if (p.gate != nullptr) {
        r *= sigmoidf_acc(p.gate[out_index]);
      }
      p.output[out_index] = r;
    } else {
      const size_t base = (tk * p.splits + split) * G;
      p.partial_o[(base + g) * D + d] = acc;
      if (d == 0) {
        p.partial_ml[(base + g) * 2 + 0] = mx;
        p.partial_ml[(base + g) * 2 + 1] = den;
      }
    }
  }
}

// Pass 2: one workgroup per (token, head).
template <int D>
__global__ __launch_bounds__(256) void attention_combine(CombineArgs p) {
  constexpr int kChunks = D / 4;             // float4 chunks per row
  constexpr int kSubsets = 256 / kChunks;    // split subsets summed in parallel
  __shared__ float s_w[kMaxSplits];
  __shared__ float s_red[256];
  __shared__ float4 s_acc[kSubsets][kChunks];

  const uint32_t group = p.heads / p.kv_heads;
  const uint32_t token = blockIdx.x;
  const uint32_t head = blockIdx.y;
  const uint32_t kvh = head / group;
  const uint32_t g = head % group;
  const size_t tk = (size_t)token * p.kv_heads + kvh;
  const int tid = threadIdx.x;

  // Global max over splits.
  float mx = -INFINITY;
  for (uint32_t s = tid; s < p.splits; s += 256) {
    mx = fmaxf(mx, p.partial_ml[((tk * p.splits + s) * group + g) * 2]);
  }
  s_red[tid] = mx;
  __syncthreads();
  for (int stride = 128; stride > 0; stride >>= 1) {
    if (tid < stride) {
      s_red[tid] = fmaxf(s_red[tid], s_red[tid + stride]);
    }
    __syncthreads();
  }
  mx = s_red[0];
  __syncthreads();
  float den = 0.0f;
  for (uint32_t s = tid; s < p.splits; s += 256) {
    const float* ml = p.partial_ml + ((tk * p.splits + s) * group + g) * 2;
    const float w = ml[0] == -INFINITY ? 0.0f : fast_exp2(ml[0] - mx);
    s_w[s] = w;
    den += w * ml[1];
  }
  s_red[tid] = den;
  __syncthreads();
  for (int stride = 128; stride > 0; stride >>= 1) {
    if (tid < stride) {
      s_red[tid] += s_red[tid + stride];
    }
    __syncthreads();
  }
  den = s_red[0];

  const int chunk = tid % kChunks;
  const int subset = tid / kChunks;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  const float4* po = reinterpret_cast<const float4*>(p.partial_o);
  for (uint32_t s = subset; s < p.splits; s += kSubsets) {
    const float w = s_w[s];
    if (w != 0.0f) {
      const float4 v = po[((tk * p.splits + s) * group + g) * kChunks + chunk];
      acc.x = fmaf(w, v.x, acc.x);
      acc.y = fmaf(w, v.y, acc.y);
      acc.z = fmaf(w, v.z, acc.z);
      acc.w = fmaf(w, v.w, acc.w);
    }
  }
  s_acc[subset][chunk] = acc;
  __syncthreads();
  if (tid < kChunks) {
    float4 r = s_acc[0][tid];
    for (int i = 1; i < kSubsets; ++i) {
      const float4 v = s_acc[i][tid];
      r.x += v.x;
      r.y += v.y;
      r.z += v.z;
      r.w += v.w;
    }
    const float inv = den == 0.0f ? 0.0f : 1.0f / den;
    const size_t out_index = ((size_t)token * p.heads + head) * D + tid * 4;
    float out[4] = {r.x * inv, r.y * inv, r.z * inv, r.w * inv};
    if (p.gate != nullptr) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        out[e] *= sigmoidf_acc(p.gate[out_index + e]);
      }
    }
    *reinterpret_cast<float4*>(p.output + out_index) = make_float4(out[0], out[1], out[2], out[3]);
  }
}

// Shapes outside the tuned templates: one wave per (token, head), 64 lanes over
// dims, online softmax over keys (the reference kernel's structure).
template <typename KV>
__global__ __launch_bounds__(64) void attention_generic(DecodeParams p, uint32_t head_dim,
                                                        uint32_t group) {
  const uint32_t token = blockIdx.x;
  const uint32_t head = blockIdx.y;
  const int lane = threadIdx.x;
  const uint32_t kvh = head / group;
  const uint32_t position = p.start_position + token;
  const size_t row_stride = (size_t)p.kv_heads * head_dim;
  const KV* kbase = static_cast<const KV*>(p.key_cache) +
                    (size_t)p.layer * p.capacity_tokens * row_stride + (size_t)kvh * head_dim;
  const KV* vbase = static_cast<const KV*>(p.value_cache) +
                    (size_t)p.layer * p.capacity_tokens * row_stride + (size_t)kvh * head_dim;
  const float* q = p.query + ((size_t)token * p.heads + head) * head_dim;
  float qv[4];
  float o[4];
  for (int i = 0; i < 4; ++i) {
    const uint32_t d = lane + 64u * i;
    qv[i] = d < head_dim ? q[d] * p.scale_log2 : 0.0f;
    o[i] = 0.0f;
  }
  float m = -INFINITY;
  float l = 0.0f;
  for (uint32_t key = 0; key <= position; ++key) {
    float acc = 0.0f;
    for (int i = 0; i < 4; ++i) {
      const uint32_t d = lane + 64u * i;
      if (d < head_dim) {
        acc += qv[i] * static_cast<float>(kbase[(size_t)key * row_stride + d]);
      }
    }
    const float s = wave_sum(acc);
    const float mn = fmaxf(m, s);
    const float corr = fast_exp2(m - mn);
    const float pr = fast_exp2(s - mn);
    l = l * corr + pr;
    for (int i = 0; i < 4; ++i) {
      const uint32_t d = lane + 64u * i;
      const float v = d < head_dim ? static_cast<float>(vbase[(size_t)key * row_stride + d]) : 0.0f;
      o[i] = o[i] * corr + pr * v;
    }
    m = mn;
  }
  const float inv = l == 0.0f ? 0.0f : 1.0f / l;
  for (int i = 0; i < 4; ++i) {
    const uint32_t d = lane + 64u * i;
    if (d < head_dim) {
      const size_t idx = ((size_t)token * p.heads + head) * head_dim + d;
      float r = o[i] * inv;
      if (p.gate != nullptr) {
        r *= sigmoidf_acc(p.gate[idx]);
      }
      p.output[idx] = r;
    }
  }
}

struct SplitPlan {
  uint32_t keys_per_split;
  uint32_t splits;
};

SplitPlan plan_splits(const AttentionArgs& a, int cu_count) {
  const uint64_t max_keys = (uint64_t)a.start_position + a.tokens;  // last query's keys
  const uint64_t units = (uint64_t)a.tokens * a.kv_heads;
  const uint64_t target_blocks = 2ull * (uint64_t)(cu_count > 0 ? cu_count : 256);
  uint64_t kps = (units * max_keys + target_blocks - 1) / target_blocks;
  const uint64_t step = kWaves * kKeysPerWaveStep;
  if (const char* env = std::getenv("KRAKEN_DECODE_KEYS_PER_SPLIT")) {
    const long v = std::strtol(env, nullptr, 10);
    if (v > 0) {
      kps = (uint64_t)v;
    }
  }
  kps = ((kps + step - 1) / step) * step;
  if (kps < step) {
    kps = step;
  }
  uint64_t splits = (max_keys + kps - 1) / kps;
  if (splits > kMaxSplits) {
    kps = ((max_keys + kMaxSplits - 1) / kMaxSplits + step - 1) / step * step;
    splits = (max_keys + kps - 1) / kps;
  }
  return SplitPlan{(uint32_t)kps, (uint32_t)splits};
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

// The tuned kernels move 16-byte chunks; shapes or pointers outside that contract
// take the generic kernel.
bool tuned_args(const AttentionArgs& a) {
  const uint32_t d = a.head_dim;
  const uint32_t g = a.heads / a.kv_heads;
  if (!aligned16(a.query) || !aligned16(a.key_cache) || !aligned16(a.value_cache) ||
      !aligned16(a.output)) {
    return false;
  }
  if (d == 256) {
    return g == 1 || g == 2 || g == 4;
  }
  if (d == 128 || d == 64) {
    return g == 1 || g == 2 || g == 4 || g == 8;
  }
  return false;
}

template <int D, int G, typename KV>
hipError_t launch_tuned(const DecodeParams& p, hipStream_t stream) {
  dim3 grid(p.splits, p.kv_heads, p.tokens);
  attention_split<D, G, KV><<<grid, kThreads, 0, stream>>>(p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.splits == 1) {
    return e;
  }
  CombineArgs c{};
  c.partial_o = p.partial_o;
  c.partial_ml = p.partial_ml;
  c.gate = p.gate;
  c.output = p.output;
  c.tokens = p.tokens;
  c.heads = p.heads;
  c.kv_heads = p.kv_heads;
  c.splits = p.splits;
  c.head_dim = D;
  return launch_attention_combine(c, stream);
}

template <typename KV>
hipError_t dispatch_kv(const DecodeParams& p, uint32_t d, uint32_t g, bool tuned,
                       hipStream_t stream) {
  switch (tuned ? d : 0u) {
    case 256:
      if (g == 1) return launch_tuned<256, 1, KV>(p, stream);
      if (g == 2) return launch_tuned<256, 2, KV>(p, stream);
      if (g == 4) return launch_tuned<256, 4, KV>(p, stream);
      break;
    case 128:
      if (g == 1) return launch_tuned<128, 1, KV>(p, stream);
      if (g == 2) return launch_tuned<128, 2, KV>(p, stream);
      if (g == 4) return launch_tuned<128, 4, KV>(p, stream);
      if (g == 8) return launch_tuned<128, 8, KV>(p, stream);
      break;
    case 64:
      if (g == 1) return launch_tuned<64, 1, KV>(p, stream);
      if (g == 2) return launch_tuned<64, 2, KV>(p, stream);
      if (g == 4) return launch_tuned<64, 4, KV>(p, stream);
      if (g == 8) return launch_tuned<64, 8, KV>(p, stream);
      break;
    default:
      break;
  }
  attention_generic<KV><<<dim3(p.tokens, p.heads), 64, 0, stream>>>(p, d, g);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_attention_combine(const CombineArgs& c, hipStream_t stream) {
  if (c.splits > kMaxSplits) {
    return hipErrorInvalidValue;
  }
  const dim3 grid(c.tokens, c.heads);
  switch (c.head_dim) {
    case 256: attention_combine<256><<<grid, 256, 0, stream>>>(c); break;
    case 128: attention_combine<128><<<grid, 256, 0, stream>>>(c); break;
    case 64: attention_combine<64><<<grid, 256, 0, stream>>>(c); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

size_t attention_decode_workspace_bytes(const AttentionArgs& a, int cu_count) {
  const uint32_t g = a.heads / a.kv_heads;
  if (!tuned_args(a)) {
    return 0;
  }
  const SplitPlan plan = plan_splits(a, cu_count);
  if (plan.splits <= 1) {
    return 0;
  }
  const size_t units = (size_t)a.tokens * a.kv_heads * plan.splits * g;
  return units * (a.head_dim + 2) * sizeof(float);
}

hipError_t launch_attention_decode(const AttentionArgs& a, int cu_count, void* workspace,
                                   size_t workspace_bytes, hipStream_t stream) {
  const uint32_t g = a.heads / a.kv_heads;
  DecodeParams p{};
  p.query = a.query;
  p.key_cache = a.key_cache;
  p.value_cache = a.value_cache;
  p.gate = a.gate;
  p.output = a.output;
  p.layer = a.layer;
  p.start_position = a.start_position;
  p.tokens = a.tokens;
  p.capacity_tokens = a.capacity_tokens;
  p.heads = a.heads;
  p.kv_heads = a.kv_heads;
  p.scale_log2 = (1.0f / sqrtf((float)a.head_dim)) * kLog2e;
  if (tuned_args(a)) {
    const SplitPlan plan = plan_splits(a, cu_count);
    p.keys_per_split = plan.keys_per_split;
    p.splits = plan.splits;
    if (plan.splits > 1) {
      const size_t units = (size_t)a.tokens * a.kv_heads * plan.splits * g;
      if (workspace == nullptr || workspace_bytes < units * (a.head_dim + 2) * sizeof(float)) {
        return hipErrorInvalidValue;
      }
      p.partial_o = static_cast<float*>(workspace);
      p.partial_ml = p.partial_o + units * a.head_dim;
    }
  } else {
    p.keys_per_split = 0;
    p.splits = 1;
  }
  const bool tuned = tuned_args(a);
  return a.kv_f16 ? dispatch_kv<half_t>(p, a.head_dim, g, tuned, stream)
                  : dispatch_kv<float>(p, a.head_dim, g, tuned, stream);
}

}  // namespace kraken
