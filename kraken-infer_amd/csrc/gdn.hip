// Gated-delta-net linear attention: recurrent core and the causal conv1d
// state machinery in front of it.
//
// Recurrence (reference MSL gated_delta_net_f32_batched_qwen35 /
// _batched_in_place, mps_backend.mm:2225-2374), per value head h
// (key_head = h % key_heads), per token, for every state row r (value dim) over
// columns c (key dim):
//     S[r,:] *= exp(g);  sk = S[r,:].k;  delta = (v[r] - sk) * beta;
//     S[r,:] += k * delta;  y[r] = (S[r,:].q) / sqrt(D)
// State rows are independent, so the kernel spreads the 16 x 128 rows of a
// layer over the whole chip: 32 lanes own one row (4 fp32 columns each for
// D=128) and keep it in registers for the whole chunk; dot products reduce over
// the 32 lanes with DPP + swizzle.  The next token's k/q/v/g/beta are fetched
// while the current token computes.  With `prepare` the kernel also forms
// g = softplus(alpha + dt_bias) * ssm_a and beta = sigmoid(beta_raw)
// (prepare_qwen35_gdn_gate_beta_f32, mps_backend.mm:2588-2605) on the fly.
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>

#include "context_internal.hpp"
#include "device_common.hpp"

namespace kraken {
namespace {

// KRAKEN_GDN_PREFILL selects the multi-token kernel for head_dim 128:
// "sequential" the LDS-staged recurrence, "generic" the generic recurrence
// kernel; unset, the chunked (WY) kernels of gdn_chunked.hip run.  Used to
// compare the three on the same inputs.
bool gdn_prefill_disabled() {
  const char* v = std::getenv("KRAKEN_GDN_PREFILL");
  return v != nullptr && std::strcmp(v, "generic") == 0;
}
// (The chunked path's own selection is gdn_chunked_supported.)

constexpr int kGdnRowsPerBlock = 8;  // 4 waves x 2 rows

struct GdnParams {
  const float* query;
  const float* key;
  const float* value;
  const float* gate;
  const float* beta;
  const float* dt_bias;
  const float* ssm_a;
  float* state;
  float* output;
  uint32_t tokens, key_heads, value_heads, head_dim;
  float scale;
  // Ragged decode (blockIdx.z = sequence, one token each): state of sequence b
  // at element seq_state_offsets[b] of a pool of pool_elems elements.
  const uint64_t* seq_state_offsets;
  uint64_t pool_elems;
};

__device__ __forceinline__ float softplus_ref(float x) {
  return x > 20.0f ? x : log1pf(expf(x));
}

template <int CPL, bool kPrepare>
__global__ __launch_bounds__(256) void gdn_recurrent_kernel(GdnParams p) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const uint32_t h = blockIdx.y;
  const uint32_t row = blockIdx.x * kGdnRowsPerBlock + wave * 2 + (lane >> 5);
  const uint32_t col0 = (uint32_t)(lane & 31) * CPL;
  const uint32_t D = p.head_dim;
  const bool row_ok = row < D;
  const uint32_t kh = h % p.key_heads;

  // Token rows [t_first, t_first + n_tokens) and the state they update.
  float* state = p.state;
  uint32_t t_first = 0;
  uint32_t n_tokens = p.tokens;
  if (p.seq_state_offsets != nullptr) {
    const uint32_t seq = blockIdx.z;
    const uint64_t off = p.seq_state_offsets[seq];
    if (off > p.pool_elems || p.pool_elems - off < (uint64_t)p.value_heads * D * D) {
      return;  // offset outside the pool: this sequence is skipped, nothing touched
    }
    state += off;
    t_first = seq;
    n_tokens = 1;
  }

  float s[CPL];
  float* srow = state + ((size_t)h * D + (row_ok ? row : 0)) * D;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    s[i] = (row_ok && col0 + i < D) ? srow[col0 + i] : 0.0f;
  }

  auto load_token = [&](uint32_t t, float* k, float* q, float& v, float& g, float& b) {
    const float* kp = p.key + ((size_t)t * p.key_heads + kh) * D;
    const float* qp = p.query + ((size_t)t * p.key_heads + kh) * D;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const bool ok = col0 + i < D;
      k[i] = ok ? kp[col0 + i] : 0.0f;
      q[i] = ok ? qp[col0 + i] : 0.0f;
    }
    v = row_ok ? p.value[((size_t)t * p.value_heads + h) * D + row] : 0.0f;
    const size_t gi = (size_t)t * p.value_heads + h;
    g = p.gate[gi];
    b = p.beta[gi];
  };

  float kc[CPL], qc[CPL], vc, gc, bc;
  const uint32_t t_end = t_first + n_tokens;
  load_token(t_first, kc, qc, vc, gc, bc);
  for (uint32_t t = t_first; t < t_end; ++t) {
    float kn[CPL], qn[CPL], vn = 0.0f, gn = 0.0f, bn = 0.0f;
    if (t + 1 < t_end) {
      load_token(t + 1, kn, qn, vn, gn, bn);
    }
    float g = gc;
    float b = bc;
    if (kPrepare) {
      g = softplus_ref(g + p.dt_bias[h]) * p.ssm_a[h];
      b = 1.0f / (1.0f + expf(-b));
    }
    const float decay = expf(g);
    float sk = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      s[i] *= decay;
      sk = fmaf(s[i], kc[i], sk);
    }
    sk = reduce32_sum(sk);
    const float delta = (vc - sk) * b;
    float y = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      s[i] = fmaf(kc[i], delta, s[i]);
      y = fmaf(s[i], qc[i], y);
    }
    y = reduce32_sum(y);
    if (row_ok && (lane & 31) == 0) {
      p.output[((size_t)t * p.value_heads + h) * D + row] = y * p.scale;
    }
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      kc[i] = kn[i];
      qc[i] = qn[i];
    }
    vc = vn;
    gc = gn;
    bc = bn;
  }
  if (row_ok) {
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      if (col0 + i < D) {
        srow[col0 + i] = s[i];
      }
    }
  }
}

// One token per state (decode: a single sequence with tokens == 1, or ragged
// decode with one token per sequence, blockIdx.z = sequence), head_dim 128.
// The recurrence step of gdn_recurrent_kernel for T = 1, laid out to stream the
// state: a 32-lane group owns RPL state rows (4 columns = one 16-byte vector per
// lane per row), a workgroup 8 groups = 8*RPL rows.  Shapes are exact (no
// bounds branches) and every load is a 16-byte vector issued before any math,
// so each lane has RPL*16 bytes of state in flight; the RPL row reductions
// interleave.  The host checks 16-byte alignment of q/k/v/state; ragged state
// offsets must be multiples of 4 elements (others are skipped like offsets
// outside the pool).
template <bool kPrepare, int RPL>
__global__ __launch_bounds__(256) void gdn_decode_kernel(GdnParams p) {
  static_assert(RPL == 1 || RPL == 2 || RPL == 4, "rows per group");
  constexpr uint32_t D = 128;
  constexpr int CPL = 4;
  const int lane = threadIdx.x & 63;
  const int grp = threadIdx.x >> 5;  // 8 groups of 32 lanes
  const uint32_t h = blockIdx.y;
  const uint32_t row0 = (blockIdx.x * 8u + grp) * RPL;
  const uint32_t col0 = (uint32_t)(lane & 31) * CPL;
  const uint32_t kh = h % p.key_heads;

  float* state = p.state;
  uint32_t t = 0;
  if (p.seq_state_offsets != nullptr) {
    const uint32_t seq = blockIdx.z;
    const uint64_t off = p.seq_state_offsets[seq];
    if ((off & 3u) != 0 || off > p.pool_elems ||
        p.pool_elems - off < (uint64_t)p.value_heads * D * D) {
      return;  // misaligned or outside the pool: this sequence is skipped, nothing touched
    }
    state += off;
    t = seq;
  }
  float* shead = state + (size_t)h * D * D;

  float4 s[RPL];
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    s[j] = *reinterpret_cast<const float4*>(shead + (size_t)(row0 + j) * D + col0);
  }
  const float4 k = *reinterpret_cast<const float4*>(p.key + ((size_t)t * p.key_heads + kh) * D +
                                                    col0);
  const float4 q = *reinterpret_cast<const float4*>(
    p.query + ((size_t)t * p.key_heads + kh) * D + col0);
  // The group's RPL values of v (rows row0 .. row0 + RPL - 1).
  float v[RPL];
  {
    const float* vrow = p.value + ((size_t)t * p.value_heads + h) * D + row0;
    if constexpr (RPL == 4) {
      const float4 v4 = *reinterpret_cast<const float4*>(vrow);
      v[0] = v4.x;
      v[1] = v4.y;
      v[2] = v4.z;
      v[3] = v4.w;
    } else {
#pragma unroll
      for (int j = 0; j < RPL; ++j) {
        v[j] = vrow[j];
      }
    }
  }
  const size_t gi = (size_t)t * p.value_heads + h;
  float g = p.gate[gi];
  float b = p.beta[gi];
  if (kPrepare) {
    g = softplus_ref(g + p.dt_bias[h]) * p.ssm_a[h];
    b = 1.0f / (1.0f + expf(-b));
  }
  const float decay = expf(g);

  float sk[RPL];
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    s[j].x *= decay;
    s[j].y *= decay;
    s[j].z *= decay;
    s[j].w *= decay;
    sk[j] = fmaf(s[j].x, k.x, fmaf(s[j].y, k.y, fmaf(s[j].z, k.z, s[j].w * k.w)));
  }
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    sk[j] = reduce32_sum(sk[j]);
  }
  float y[RPL];
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    const float delta = (v[j] - sk[j]) * b;
    s[j].x = fmaf(k.x, delta, s[j].x);
    s[j].y = fmaf(k.y, delta, s[j].y);
    s[j].z = fmaf(k.z, delta, s[j].z);
    s[j].w = fmaf(k.w, delta, s[j].w);
    y[j] = fmaf(s[j].x, q.x, fmaf(s[j].y, q.y, fmaf(s[j].z, q.z, s[j].w * q.w)));
  }
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    y[j] = reduce32_sum(y[j]);
  }
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    *reinterpret_cast<float4*>(shead + (size_t)(row0 + j) * D + col0) = s[j];
  }
  // Lane 0 of the group writes the RPL outputs (one 16-byte store for 4).
  if ((lane & 31) == 0) {
    float* yrow = p.output + ((size_t)t * p.value_heads + h) * D + row0;
    if constexpr (RPL == 4) {
      *reinterpret_cast<float4*>(yrow) =
        make_float4(y[0] * p.scale, y[1] * p.scale, y[2] * p.scale, y[3] * p.scale);
    } else {
#pragma unroll
      for (int j = 0; j < RPL; ++j) {
        yrow[j] = y[j] * p.scale;
      }
    }
  }
}

// Sum over the 32 lanes of each wave half, VALU only: DPP within each 16-lane
// row, then v_permlane16_swap across the two rows of the half.
__device__ __forceinline__ float half_sum32(float x) {
  x += dpp<kDppQuadXor1>(x);
  x += dpp<kDppQuadXor2>(x);
  x += dpp<kDppRowHalfMirror>(x);
  x += dpp<kDppRowMirror>(x);
  return xor16_sum(x);
}

// Multi-token (prefill) form of the recurrence for head_dim 128.  Same lane
// layout as gdn_recurrent_kernel (32 lanes own one state row, one 16-byte
// vector of 4 columns per lane; a workgroup = 4 waves = 8 rows of one head,
// 16 workgroups per head), but the per-token inputs come from LDS: the
// workgroup stages kGdnChunk tokens of k, q (the whole 128-wide rows), its 8
// values of v, and the per-token decay exp(g) and beta (prepared once per token
// here rather than per lane) into one of two LDS buffers while the other is
// consumed, so no token waits on global memory.  The per-token arithmetic is
// the reference's, in its order: S *= exp(g); sk = S.k; delta = (v - sk) beta;
// S += k delta; y = S.q / sqrt(D).  The host checks 16-byte alignment of
// q/k/v/state and value_heads * 128 % 4 == 0 (always true for D = 128).
constexpr int kGdnChunk = 64;

template <bool kPrepare>
__global__ __launch_bounds__(256) void gdn_prefill_kernel(GdnParams p) {
  constexpr uint32_t D = 128;
  constexpr int TC = kGdnChunk;
  constexpr int kRows = 8;
  __shared__ float4 s_k[2][TC][D / 4];
  __shared__ float4 s_q[2][TC][D / 4];
  __shared__ float s_v[2][TC][kRows];
  __shared__ float s_decay[2][TC];
  __shared__ float s_beta[2][TC];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int lrow = (tid >> 6) * 2 + (lane >> 5);  // local row 0..7
  const int c4 = lane & 31;                        // columns 4*c4 .. 4*c4+3
  const uint32_t h = blockIdx.y;
  const uint32_t row0 = blockIdx.x * kRows;
  const uint32_t row = row0 + lrow;
  const uint32_t kh = h % p.key_heads;
  const uint32_t tokens = p.tokens;
  const uint32_t chunks = (tokens + TC - 1) / TC;

  float* srow = p.state + ((size_t)h * D + row) * D + 4 * c4;
  float4 s = *reinterpret_cast<const float4*>(srow);

  // Staging registers for one chunk: thread tid carries k/q vectors
  // tid + 256 i (token (tid + 256 i) / 32, vector (tid + 256 i) % 32), v vector
  // tid < 128 (token tid / 2, rows 4 (tid % 2) ..), and g/beta of token tid - 128
  // for 128 <= tid < 192.
  float4 kr[TC * 32 / 256], qr[TC * 32 / 256], vr = make_float4(0, 0, 0, 0);
  float dr = 0.0f, br = 0.0f;
  auto load_chunk = [&](uint32_t c) {
    const uint32_t tb = c * TC;
    const uint32_t n = min((uint32_t)TC, tokens - tb);
#pragma unroll
    for (int i = 0; i < TC * 32 / 256; ++i) {
      const uint32_t idx = tid + 256u * i;
      const uint32_t t = idx >> 5;
      const uint32_t v4 = idx & 31u;
      const size_t off = ((size_t)(tb + t) * p.key_heads + kh) * D + 4 * v4;
      kr[i] = t < n ? *reinterpret_cast<const float4*>(p.key + off) : make_float4(0, 0, 0, 0);
      qr[i] = t < n ? *reinterpret_cast<const float4*>(p.query + off) : make_float4(0, 0, 0, 0);
    }
    if (tid < 2 * TC) {
      const uint32_t t = tid >> 1;
      if (t < n) {
        vr = *reinterpret_cast<const float4*>(
          p.value + ((size_t)(tb + t) * p.value_heads + h) * D + row0 + 4 * (tid & 1));
      }
    } else if (tid < 3 * TC) {
      const uint32_t t = tid - 2 * TC;
      if (t < n) {
        const size_t gi = (size_t)(tb + t) * p.value_heads + h;
        float g = p.gate[gi];
        float b = p.beta[gi];
        if (kPrepare) {
          g = softplus_ref(g + p.dt_bias[h]) * p.ssm_a[h];
          b = 1.0f / (1.0f + expf(-b));
        }
        dr = expf(g);
        br = b;
      }
    }
  };
  auto store_chunk = [&](int buf) {
#pragma unroll
    for (int i = 0; i < TC * 32 / 256; ++i) {
      const uint32_t idx = tid + 256u * i;
      s_k[buf][idx >> 5][idx & 31u] = kr[i];
      s_q[buf][idx >> 5][idx & 31u] = qr[i];
    }
    if (tid < 2 * TC) {
      *reinterpret_cast<float4*>(&s_v[buf][tid >> 1][4 * (tid & 1)]) = vr;
    } else if (tid < 3 * TC) {
      s_decay[buf][tid - 2 * TC] = dr;
      s_beta[buf][tid - 2 * TC] = br;
    }
  };

  load_chunk(0);
  store_chunk(0);
  __syncthreads();
  for (uint32_t c = 0; c < chunks; ++c) {
    const int buf = (int)(c & 1u);
    if (c + 1 < chunks) {
      load_chunk(c + 1);  // lands while this chunk computes
    }
    const uint32_t tb = c * TC;
    const int n = (int)min((uint32_t)TC, tokens - tb);
    float* out = p.output + ((size_t)tb * p.value_heads + h) * D + row;
    const size_t out_stride = (size_t)p.value_heads * D;
    float4 k = s_k[buf][0][c4];
    float4 q = s_q[buf][0][c4];
    float v = s_v[buf][0][lrow];
    float decay = s_decay[buf][0];
    float b = s_beta[buf][0];
    for (int t = 0; t < n; ++t) {
      // Next token's inputs (clamped at the chunk end) before this token's math.
      const int tn = t + 1 < n ? t + 1 : t;
      const float4 k_n = s_k[buf][tn][c4];
      const float4 q_n = s_q[buf][tn][c4];
      const float v_n = s_v[buf][tn][lrow];
      const float decay_n = s_decay[buf][tn];
      const float b_n = s_beta[buf][tn];

      s.x *= decay;
      s.y *= decay;
      s.z *= decay;
      s.w *= decay;
      float sk = fmaf(s.w, k.w, fmaf(s.z, k.z, fmaf(s.y, k.y, s.x * k.x)));
      sk = half_sum32(sk);
      const float delta = (v - sk) * b;
      s.x = fmaf(k.x, delta, s.x);
      s.y = fmaf(k.y, delta, s.y);
      s.z = fmaf(k.z, delta, s.z);
      s.w = fmaf(k.w, delta, s.w);
      float y = fmaf(s.w, q.w, fmaf(s.z, q.z, fmaf(s.y, q.y, s.x * q.x)));
      y = half_sum32(y);
      if (c4 == 0) {
        out[(size_t)t * out_stride] = y * p.scale;
      }
      k = k_n;
      q = q_n;
      v = v_n;
      decay = decay_n;
      b = b_n;
    }
    if (c + 1 < chunks) {
      store_chunk(buf ^ 1);  // buffer buf ^ 1 was last read before the previous barrier
    }
    __syncthreads();
  }
  *reinterpret_cast<float4*>(srow) = s;
}

template <bool kPrepare>
hipError_t launch_gdn_cpl(const GdnParams& p, hipStream_t stream) {
  const bool one_token = p.seq_state_offsets != nullptr || p.tokens == 1;
  const uint32_t cpl = (p.head_dim + 31) / 32;
  const bool aligned = ((uintptr_t)p.query | (uintptr_t)p.key | (uintptr_t)p.value |
                        (uintptr_t)p.state | (uintptr_t)p.output) % 16u == 0;
  if (!one_token && p.head_dim == 128 && aligned && !gdn_prefill_disabled()) {
    const dim3 grid(128 / 8, p.value_heads);
    gdn_prefill_kernel<kPrepare><<<grid, 256, 0, stream>>>(p);
    return hipGetLastError();
  }
  if (one_token && p.head_dim == 128 && aligned) {
    // Rows per 32-lane group: 4 when there are many states to stream (ragged
    // decode), 1 for few, so that a single sequence's 16 heads still spread
    // over 256 workgroups (8 rows each) instead of 64.
    const uint32_t sequences = p.seq_state_offsets != nullptr ? p.tokens : 1u;
    if ((uint64_t)sequences * p.value_heads * 4u >= 1024u) {
      constexpr int kRpl = 4;
      const dim3 grid(128 / (8 * kRpl), p.value_heads, sequences);
      gdn_decode_kernel<kPrepare, kRpl><<<grid, 256, 0, stream>>>(p);
    } else {
      constexpr int kRpl = 1;
      const dim3 grid(128 / (8 * kRpl), p.value_heads, sequences);
      gdn_decode_kernel<kPrepare, kRpl><<<grid, 256, 0, stream>>>(p);
    }
    return hipGetLastError();
  }
  const dim3 grid((p.head_dim + kGdnRowsPerBlock - 1) / kGdnRowsPerBlock, p.value_heads,
                  p.seq_state_offsets != nullptr ? p.tokens : 1u);
  if (cpl <= 1) {
    gdn_recurrent_kernel<1, kPrepare><<<grid, 256, 0, stream>>>(p);
  } else if (cpl <= 2) {
    gdn_recurrent_kernel<2, kPrepare><<<grid, 256, 0, stream>>>(p);
  } else if (cpl <= 4) {
    gdn_recurrent_kernel<4, kPrepare><<<grid, 256, 0, stream>>>(p);
  } else {
    gdn_recurrent_kernel<8, kPrepare><<<grid, 256, 0, stream>>>(p);
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------- conv ------

// build_ssm_conv_state_f32 (mps_backend.mm:2428-2457).  One block per 64
// channels: thread c < 64 owns channel c's state (old state -> conv_input head,
// new state <- last K-1 entries of [old state | chunk]); the whole block copies
// the chunk transposed into conv_input[c][K-1+t].
__global__ __launch_bounds__(256) void build_conv_state_kernel(float* state, const float* input,
                                                               float* conv_input,
                                                               uint32_t conv_kernel,
                                                               uint32_t channels,
                                                               uint32_t tokens) {
  const uint32_t width = conv_kernel - 1u;
  const size_t span = (size_t)width + tokens;
  const uint32_t c0 = blockIdx.x * 64u;
  const uint32_t lc = threadIdx.x & 63u;
  const uint32_t c = c0 + lc;
  const uint32_t tlane = threadIdx.x >> 6;
  if (tlane == 0 && c < channels) {
    for (uint32_t j = 0; j < width; ++j) {
      conv_input[c * span + j] = state[(size_t)c * width + j];
    }
  }
  if (c < channels) {
    for (uint32_t t = tlane; t < tokens; t += 4u) {
      conv_input[c * span + width + t] = input[(size_t)t * channels + c];
    }
  }
  __syncthreads();
  if (tlane == 0 && c < channels) {
    for (uint32_t j = 0; j < width; ++j) {
      state[(size_t)c * width + j] = conv_input[c * span + tokens + j];
    }
  }
}

// ssm_conv_f32 (mps_backend.mm:2376-2400).
__global__ void ssm_conv_kernel(const float* input, const float* weights, float* output,
                                uint32_t conv_kernel, uint32_t channels, uint32_t tokens,
                                uint32_t sequences) {
  const size_t span = (size_t)conv_kernel - 1u + tokens;
  const size_t total = (size_t)sequences * tokens * channels;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const uint32_t c = (uint32_t)(i % channels);
    const uint32_t t = (uint32_t)((i / channels) % tokens);
    const size_t s = i / ((size_t)channels * tokens);
    const float* x = input + (s * channels + c) * span + t;
    const float* w = weights + (size_t)c * conv_kernel;
    float acc = 0.0f;
    for (uint32_t j = 0; j < conv_kernel; ++j) {
      acc = fmaf(x[j], w[j], acc);
    }
    output[i] = acc;
  }
}

// ssm_conv1_f32_stateful (mps_backend.mm:2402-2426).
__global__ void conv1_stateful_kernel(float* state, const float* input, const float* weights,
                                      float* output, uint32_t conv_kernel, uint32_t channels) {
  const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= channels) {
    return;
  }
  const uint32_t width = conv_kernel - 1u;
  float* st = state + (size_t)c * width;
  const float* w = weights + (size_t)c * conv_kernel;
  const float x = input[c];
  float acc = 0.0f;
  for (uint32_t j = 0; j < width; ++j) {
    acc = fmaf(st[j], w[j], acc);
  }
  acc = fmaf(x, w[width], acc);
  for (uint32_t j = 0; j + 1u < width; ++j) {
    st[j] = st[j + 1u];
  }
  st[width - 1u] = x;
  output[c] = acc;
}

// Fused linear-attention prologue (qwen35_runtime.cpp:2746-2796): causal depthwise
// conv over [old state | chunk] + SiLU + split into q/k/v + L2 norm of q and k.
// Block = 4 waves = one head-slice of D channels (q head, k head or v head) for a
// tile of tokens; lane owns CPL channels.  Each wave walks TPW consecutive tokens
// with a register sliding window of the last K rows.
constexpr int kConvTokensPerWave = 4;

template <int CPL, int K>
__global__ __launch_bounds__(256) void conv_split_l2_kernel(
  const float* qkv, const float* conv_state, const float* weights, uint32_t tokens,
  uint32_t key_heads, uint32_t value_heads, uint32_t head_dim, float eps, float* query,
  float* key, float* value) {
  constexpr int W = K - 1;
  const uint32_t heads_total = 2u * key_heads + value_heads;
  const uint32_t unit = blockIdx.x % heads_total;  // which q/k/v head
  const uint32_t tile = blockIdx.x / heads_total;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const size_t channels = (size_t)heads_total * head_dim;
  const uint32_t cbase = unit * head_dim;  // first channel of this head-slice
  const uint32_t t_begin = (tile * 4u + wave) * kConvTokensPerWave;
  if (t_begin >= tokens) {
    return;
  }
  const uint32_t t_end = min(tokens, t_begin + kConvTokensPerWave);

  float w[CPL][K];
  float win[CPL][W];  // win[.][j] = x[t - W + j]
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const uint32_t d = lane + 64u * i;
    const bool ok = d < head_dim;
    const size_t c = cbase + d;
#pragma unroll
    for (int j = 0; j < K; ++j) {
      w[i][j] = ok ? weights[c * K + j] : 0.0f;
    }
    // Rows t_begin - W .. t_begin - 1 (conv state rows when negative).
#pragma unroll
    for (int j = 0; j < W; ++j) {
      float v = 0.0f;
      if (ok) {
        const int64_t r = (int64_t)t_begin - W + j;
        v = r >= 0 ? qkv[(size_t)r * channels + c] : conv_state[c * W + (W + r)];
      }
      win[i][j] = v;
    }
  }

  // The wave's rows, all loads in flight before the first output (rows past
  // the end read as zeros and are not used): whole-model prefill 5.77 -> 5.74
  // ms per 1024-token chunk.
  float xs[kConvTokensPerWave][CPL];
#pragma unroll
  for (int k = 0; k < kConvTokensPerWave; ++k) {
    const uint32_t t = t_begin + (uint32_t)k;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const uint32_t d = lane + 64u * i;
      xs[k][i] = d < head_dim && t < t_end ? qkv[(size_t)t * channels + cbase + d] : 0.0f;
    }
  }
  const bool is_v = unit >= 2u * key_heads;
#pragma unroll
  for (int k = 0; k < kConvTokensPerWave; ++k) {
    const uint32_t t = t_begin + (uint32_t)k;
    if (t >= t_end) {
      break;
    }
    float y[CPL];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const uint32_t d = lane + 64u * i;
      const bool ok = d < head_dim;
      const float xt = xs[k][i];
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < W; ++j) {
        acc = fmaf(win[i][j], w[i][j], acc);
      }
      acc = fmaf(xt, w[i][W], acc);
#pragma unroll
      for (int j = 0; j + 1 < W; ++j) {
        win[i][j] = win[i][j + 1];
      }
      win[i][W - 1] = xt;
      const float sl = acc / (1.0f + expf(-acc));  // SiLU
      y[i] = ok ? sl : 0.0f;
      ss = fmaf(y[i], y[i], ss);
    }
    if (is_v) {
      const uint32_t vh = unit - 2u * key_heads;
      float* dst = value + ((size_t)t * value_heads + vh) * head_dim;
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const uint32_t d = lane + 64u * i;
        if (d < head_dim) {
          dst[d] = y[i];
        }
      }
    } else {
      ss = wave_sum(ss);
      const float inv = 1.0f / fmaxf(sqrtf(ss), eps);
      const uint32_t part = unit / key_heads;
      const uint32_t kh = unit % key_heads;
      float* dst = (part == 0 ? query : key) + ((size_t)t * key_heads + kh) * head_dim;
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const uint32_t d = lane + 64u * i;
        if (d < head_dim) {
          dst[d] = y[i] * inv;
        }
      }
    }
  }
}

// New conv state after the chunk: last K-1 rows of [old state | chunk].  Runs
// after the conv kernel so no block reads a state row this one overwrites.
__global__ void conv_state_update_kernel(float* conv_state, const float* qkv,
                                         uint32_t conv_kernel, uint32_t tokens,
                                         uint32_t channels) {
  const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= channels) {
    return;
  }
  const uint32_t width = conv_kernel - 1u;
  float* state = conv_state + (size_t)c * width;
  // New entry j is row tokens - width + j of [old state | chunk]: a chunk row,
  // or old entry j + tokens.  Ascending j reads each old entry before it is
  // overwritten (j + tokens > j), so the shift needs no private copy.
  constexpr uint32_t kHeld = 8;
  if (tokens >= width && width <= kHeld) {
    // Chunk rows only: every load goes out before the first store.
    float v[kHeld];
#pragma unroll
    for (uint32_t j = 0; j < kHeld; ++j) {
      v[j] = j < width ? qkv[(size_t)(tokens - width + j) * channels + c] : 0.0f;
    }
#pragma unroll
    for (uint32_t j = 0; j < kHeld; ++j) {
      if (j < width) {
        state[j] = v[j];
      }
    }
    return;
  }
  for (uint32_t j = 0; j < width; ++j) {
    const int64_t r = (int64_t)tokens - (int64_t)width + j;
    state[j] = r >= 0 ? qkv[(size_t)r * channels + c] : state[j + tokens];
  }
}

// Ragged decode form of the fused prologue: one token per sequence, sequence b's
// conv state R_b [channels][K-1] at element seq_conv_offsets[b] of a pool.  One
// wave per (head-slice, sequence); lane owns CPL channels.  The state update is
// fused (each channel's state is read and rewritten by the one lane that owns it).
template <int CPL, int K>
__global__ __launch_bounds__(64) void conv_split_l2_ragged_kernel(
  const float* qkv, float* conv_pool, const uint64_t* seq_conv_offsets, uint64_t pool_elems,
  const float* weights, uint32_t key_heads, uint32_t value_heads, uint32_t head_dim, float eps,
  float* query, float* key, float* value) {
  constexpr int W = K - 1;
  const uint32_t heads_total = 2u * key_heads + value_heads;
  const uint32_t unit = blockIdx.x;  // which q/k/v head
  const uint32_t seq = blockIdx.y;
  const int lane = threadIdx.x;
  const size_t channels = (size_t)heads_total * head_dim;
  const uint64_t off = seq_conv_offsets[seq];
  if (off > pool_elems || pool_elems - off < channels * W) {
    return;  // offset outside the pool: this sequence is skipped, nothing touched
  }
  float* state = conv_pool + off;
  const uint32_t cbase = unit * head_dim;
  float y[CPL];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const uint32_t d = lane + 64u * i;
    const bool ok = d < head_dim;
    const size_t c = cbase + (ok ? d : 0u);
    float win[W];
#pragma unroll
    for (int j = 0; j < W; ++j) {
      win[j] = ok ? state[c * W + j] : 0.0f;
    }
    const float xt = ok ? qkv[(size_t)seq * channels + c] : 0.0f;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < W; ++j) {
      acc = fmaf(win[j], ok ? weights[c * K + j] : 0.0f, acc);
    }
    acc = fmaf(xt, ok ? weights[c * K + W] : 0.0f, acc);
    if (ok) {
#pragma unroll
      for (int j = 0; j + 1 < W; ++j) {
        state[c * W + j] = win[j + 1];
      }
      state[c * W + (W - 1)] = xt;
    }
    const float sl = acc / (1.0f + expf(-acc));  // SiLU
    y[i] = ok ? sl : 0.0f;
    ss = fmaf(y[i], y[i], ss);
  }
  if (unit >= 2u * key_heads) {
    float* dst = value + ((size_t)seq * value_heads + (unit - 2u * key_heads)) * head_dim;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const uint32_t d = lane + 64u * i;
      if (d < head_dim) {
        dst[d] = y[i];
      }
    }
    return;
  }
  ss = wave_sum(ss);
  const float inv = 1.0f / fmaxf(sqrtf(ss), eps);
  const uint32_t part = unit / key_heads;
  const uint32_t kh = unit % key_heads;
  float* dst = (part == 0 ? query : key) + ((size_t)seq * key_heads + kh) * head_dim;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const uint32_t d = lane + 64u * i;
    if (d < head_dim) {
      dst[d] = y[i] * inv;
    }
  }
}

// Ragged decode of a whole Qwen3.5 linear-attention core (the op sequence of
// run_qwen35_linear_layer_chunk between its projections, qwen35_runtime.cpp:
// 2740-3008, for one token per sequence) in one launch: one workgroup per
// (sequence, value head) runs, in order,
//  * the conv prologue of conv_split_l2_ragged_kernel for the head's q, k and v
//    channels (waves 0, 1, 2: one unit each, with that kernel's lane mapping
//    and reduction order) into LDS, updating the conv state;
//  * the gated delta rule of gdn_decode_kernel on the head's 128 x 128 state
//    (8 groups of 32 lanes, 16 rows each; the state loads are issued first, so
//    they are in flight during the conv);
//  * the norm-gated epilogue of rms_norm_heads_kernel (wave 0).
// Each step repeats the replaced kernel's arithmetic, so the result equals the
// three-kernel chain bit for bit.  key_heads == value_heads: every workgroup
// owns its q/k channels, and the conv-state update has one writer.  A sequence
// whose state or conv offset is misaligned or outside its pool is skipped
// (nothing is read or written for it).
template <bool kPrepare>
__global__ __launch_bounds__(256) void gdn_layer_ragged_kernel(GdnLayerArgs p) {
  constexpr uint32_t D = 128;
  constexpr int K = 4;
  constexpr int W = K - 1;
  constexpr int RPL = 16;  // state rows per 32-lane group
  constexpr int CPL = 2;   // conv channels per lane (D / 64)
  __shared__ float qs[D], ks[D], vs[D], ys[D];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int grp = tid >> 5;
  const uint32_t h = blockIdx.x;
  const uint32_t seq = blockIdx.y;
  const uint32_t H = p.heads;
  const size_t channels = (size_t)3 * H * D;
  const uint32_t row0 = (uint32_t)grp * RPL;
  const uint32_t col0 = (uint32_t)(lane & 31) * 4;

  // Everything that does not depend on the sequence's pool offsets (which are
  // themselves loads) goes out first: the epilogue's and the gate's inputs,
  // and the conv's input row and weights.
  const size_t gi = (size_t)seq * H + h;
  float g = p.gate[gi];
  float b = p.beta[gi];
  float dtb = 0.0f, sa = 0.0f;
  if (kPrepare) {
    dtb = p.dt_bias[h];
    sa = p.ssm_a[h];
  }
  float zz[2], nw[2];
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      zz[i] = p.z[gi * D + lane + 64 * i];
      nw[i] = p.norm_weight[lane + 64 * i];
    }
  }
  const uint32_t cbase = ((uint32_t)(wave < 3 ? wave : 0) * H + h) * D;
  float xt[CPL], cw[CPL][K];
  if (wave < 3) {
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const size_t c = cbase + lane + 64u * i;
      xt[i] = p.qkv[(size_t)seq * channels + c];
#pragma unroll
      for (int j = 0; j < K; ++j) {
        cw[i][j] = p.conv_weights[c * K + j];
      }
    }
  }

  const uint64_t soff = p.seq_state_offsets[seq];
  const uint64_t coff = p.seq_conv_offsets[seq];
  if ((soff & 3u) != 0 || soff > p.state_pool_elems ||
      p.state_pool_elems - soff < (uint64_t)H * D * D || coff > p.conv_pool_elems ||
      p.conv_pool_elems - coff < channels * W) {
    return;  // whole workgroup, before any barrier
  }
  float* shead = p.state_pool + soff + (size_t)h * D * D;
  float4 s[RPL];
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    s[j] = *reinterpret_cast<const float4*>(shead + (size_t)(row0 + j) * D + col0);
  }

  if (wave < 3) {
    // Unit wave * H + h: the q, k or v channels of this head.  Both channels'
    // windows are loaded before either is written back.
    float* state = p.conv_pool + coff;
    float win[CPL][W];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const size_t c = cbase + lane + 64u * i;
#pragma unroll
      for (int j = 0; j < W; ++j) {
        win[i][j] = state[c * W + j];
      }
    }
    float y[CPL];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const size_t c = cbase + lane + 64u * i;
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < W; ++j) {
        acc = fmaf(win[i][j], cw[i][j], acc);
      }
      acc = fmaf(xt[i], cw[i][W], acc);
#pragma unroll
      for (int j = 0; j + 1 < W; ++j) {
        state[c * W + j] = win[i][j + 1];
      }
      state[c * W + (W - 1)] = xt[i];
      y[i] = acc / (1.0f + expf(-acc));  // SiLU
      ss = fmaf(y[i], y[i], ss);
    }
    float* dst = wave == 0 ? qs : (wave == 1 ? ks : vs);
    float inv = 1.0f;
    if (wave < 2) {
      ss = wave_sum(ss);
      inv = 1.0f / fmaxf(sqrtf(ss), p.eps);
    }
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      dst[lane + 64 * i] = wave < 2 ? y[i] * inv : y[i];
    }
  }
  if (kPrepare) {
    g = softplus_ref(g + dtb) * sa;
    b = 1.0f / (1.0f + expf(-b));
  }
  const float decay = expf(g);
  __syncthreads();

  const float4 k = *reinterpret_cast<const float4*>(&ks[col0]);
  const float4 q = *reinterpret_cast<const float4*>(&qs[col0]);
  const float scale = 1.0f / sqrtf((float)D);
  float sk[RPL];
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    s[j].x *= decay;
    s[j].y *= decay;
    s[j].z *= decay;
    s[j].w *= decay;
    sk[j] = fmaf(s[j].x, k.x, fmaf(s[j].y, k.y, fmaf(s[j].z, k.z, s[j].w * k.w)));
  }
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    sk[j] = reduce32_sum(sk[j]);
  }
  float yv[RPL];
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    const float delta = (vs[row0 + j] - sk[j]) * b;
    s[j].x = fmaf(k.x, delta, s[j].x);
    s[j].y = fmaf(k.y, delta, s[j].y);
    s[j].z = fmaf(k.z, delta, s[j].z);
    s[j].w = fmaf(k.w, delta, s[j].w);
    yv[j] = fmaf(s[j].x, q.x, fmaf(s[j].y, q.y, fmaf(s[j].z, q.z, s[j].w * q.w)));
  }
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    yv[j] = reduce32_sum(yv[j]);
  }
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    *reinterpret_cast<float4*>(shead + (size_t)(row0 + j) * D + col0) = s[j];
  }
  if ((lane & 31) == 0) {
#pragma unroll
    for (int j = 0; j < RPL; ++j) {
      ys[row0 + j] = yv[j] * scale;
    }
  }
  __syncthreads();

  if (wave == 0) {
    // Norm-gated epilogue: y <- y * rsqrt(mean(y^2) + eps) * w * silu(z).
    float v[2];
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      v[i] = ys[lane + 64 * i];
      sum = fmaf(v[i], v[i], sum);
    }
    sum = wave_sum(sum);
    const float nscale = 1.0f / sqrtf(sum / (float)D + p.eps);
    const size_t rowoff = gi * D;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      float r = v[i] * nscale * nw[i];
      r *= zz[i] * (1.0f / (1.0f + expf(-zz[i])));
      p.output[rowoff + lane + 64 * i] = r;
    }
  }
}

// The gated delta rule of gdn_layer_ragged_kernel without its conv prologue
// and norm-gated epilogue, for a qkv whose conv and SiLU are already applied
// (the input projection's conv epilogue): workgroup (part, head, sequence)
// owns 8 * RPL state rows of the head.  Waves 0 and 1 L2-normalise the head's
// q and k with the conv prologue's lane mapping and reduction order, each
// 32-lane group updates its RPL rows as the one-kernel layer does, and the
// rows' y * scale go to output, so state and y equal the one-kernel layer's
// bit for bit.  The rows' norm_weight * silu(z) go to gate_factor: the
// output projection's input transform finishes the norm-gated epilogue with
// the head's RMS scale.  With the conv-state update done per channel by the
// input projection, no part waits for another: a single sequence's 16 heads
// spread over 128 (RPL 2) or 256 (RPL 1) workgroups instead of 16.
template <bool kPrepare, int RPL>
__global__ __launch_bounds__(256) void gdn_state_split_kernel(GdnLayerArgs p) {
  constexpr uint32_t D = 128;
  constexpr int CPL = 2;
  __shared__ float qs[D], ks[D];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int grp = tid >> 5;
  const uint32_t part = blockIdx.x;
  const uint32_t h = blockIdx.y;
  const uint32_t seq = blockIdx.z;
  const uint32_t H = p.heads;
  const size_t channels = (size_t)3 * H * D;
  const uint32_t row0 = part * (8u * RPL) + (uint32_t)grp * RPL;
  const uint32_t col0 = (uint32_t)(lane & 31) * 4;

  // The loads that do not depend on the sequence's state offset go out
  // before it is known (the offset is itself a load, and the state rows wait
  // for it): decode loop 0.69 -> 0.667 ms per token.
  const float* qkv = p.qkv + (size_t)seq * channels;
  float vv[RPL];
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    vv[j] = qkv[(size_t)(2u * H + h) * D + row0 + j];
  }
  const size_t gi = (size_t)seq * H + h;
  float g = p.gate[gi];
  float b = p.beta[gi];
  float dtb = 0.0f, sa = 0.0f;
  if (kPrepare) {
    dtb = p.dt_bias[h];
    sa = p.ssm_a[h];
  }
  float zv[RPL], nw[RPL];
  if ((lane & 31) == 0) {
#pragma unroll
    for (int j = 0; j < RPL; ++j) {
      zv[j] = p.z[gi * D + row0 + j];
      nw[j] = p.norm_weight[row0 + j];
    }
  }
  float y[CPL];
  if (wave < 2) {
    const float* src = qkv + (size_t)((uint32_t)wave * H + h) * D;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      y[i] = src[lane + 64 * i];
    }
  }

  const uint64_t soff = p.seq_state_offsets[seq];
  if ((soff & 3u) != 0 || soff > p.state_pool_elems ||
      p.state_pool_elems - soff < (uint64_t)H * D * D) {
    return;  // whole workgroup, before any barrier
  }
  float* shead = p.state_pool + soff + (size_t)h * D * D;
  float4 s[RPL];
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    s[j] = *reinterpret_cast<const float4*>(shead + (size_t)(row0 + j) * D + col0);
  }
  if (wave < 2) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      ss = fmaf(y[i], y[i], ss);
    }
    ss = wave_sum(ss);
    const float inv = 1.0f / fmaxf(sqrtf(ss), p.eps);
    float* dst = wave == 0 ? qs : ks;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      dst[lane + 64 * i] = y[i] * inv;
    }
  }
  if (kPrepare) {
    g = softplus_ref(g + dtb) * sa;
    b = 1.0f / (1.0f + expf(-b));
  }
  const float decay = expf(g);
  __syncthreads();

  const float4 k = *reinterpret_cast<const float4*>(&ks[col0]);
  const float4 q = *reinterpret_cast<const float4*>(&qs[col0]);
  const float scale = 1.0f / sqrtf((float)D);
  float sk[RPL];
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    s[j].x *= decay;
    s[j].y *= decay;
    s[j].z *= decay;
    s[j].w *= decay;
    sk[j] = fmaf(s[j].x, k.x, fmaf(s[j].y, k.y, fmaf(s[j].z, k.z, s[j].w * k.w)));
  }
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    sk[j] = reduce32_sum(sk[j]);
  }
  float yv[RPL];
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    const float delta = (vv[j] - sk[j]) * b;
    s[j].x = fmaf(k.x, delta, s[j].x);
    s[j].y = fmaf(k.y, delta, s[j].y);
    s[j].z = fmaf(k.z, delta, s[j].z);
    s[j].w = fmaf(k.w, delta, s[j].w);
    yv[j] = fmaf(s[j].x, q.x, fmaf(s[j].y, q.y, fmaf(s[j].z, q.z, s[j].w * q.w)));
  }
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    yv[j] = reduce32_sum(yv[j]);
  }
#pragma unroll
  for (int j = 0; j < RPL; ++j) {
    *reinterpret_cast<float4*>(shead + (size_t)(row0 + j) * D + col0) = s[j];
  }
  if ((lane & 31) == 0) {
#pragma unroll
    for (int j = 0; j < RPL; ++j) {
      p.output[gi * D + row0 + j] = yv[j] * scale;
      // The norm-gated epilogue's per-value factor, norm_weight * silu(z).
      const float zz = zv[j];
      p.gate_factor[gi * D + row0 + j] = nw[j] * (zz * (1.0f / (1.0f + expf(-zz))));
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

size_t gdn_workspace_bytes(const GdnArgs& a) {
  return gdn_chunked_supported(a) ? gdn_chunked_workspace_bytes(a) : 0;
}

hipError_t launch_gated_delta_net(const GdnArgs& a, int cu_count, void* workspace,
                                  size_t workspace_bytes, hipStream_t stream) {
  (void)cu_count;
  if (gdn_chunked_supported(a)) {
    const hipError_t e = launch_gdn_chunked(a, workspace, workspace_bytes, stream);
    if (e != hipSuccess || a.z == nullptr) {
      return e;
    }
    return launch_rms_norm_heads(a.output, a.norm_weight, a.z, a.tokens, a.value_heads,
                                 a.head_dim, a.eps, stream);
  }
  GdnParams p{};
  p.query = a.query;
  p.key = a.key;
  p.value = a.value;
  p.gate = a.gate;
  p.beta = a.beta;
  p.dt_bias = a.dt_bias;
  p.ssm_a = a.ssm_a;
  p.state = a.state;
  p.output = a.output;
  p.tokens = a.tokens;
  p.key_heads = a.key_heads;
  p.value_heads = a.value_heads;
  p.head_dim = a.head_dim;
  p.scale = 1.0f / sqrtf((float)a.head_dim);
  p.seq_state_offsets = a.seq_state_offsets;
  p.pool_elems = a.pool_elems;
  hipError_t e = a.dt_bias != nullptr ? launch_gdn_cpl<true>(p, stream)
                                      : launch_gdn_cpl<false>(p, stream);
  if (e != hipSuccess || a.z == nullptr) {
    return e;
  }
  // Norm-gated epilogue over each (token, head) row of y.
  return launch_rms_norm_heads(a.output, a.norm_weight, a.z, a.tokens, a.value_heads,
                               a.head_dim, a.eps, stream);
}

hipError_t launch_ssm_conv(const float* input, const float* kernel, float* output,
                           uint32_t conv_kernel, uint32_t channels, uint32_t tokens,
                           uint32_t sequences, hipStream_t stream) {
  const size_t total = (size_t)sequences * tokens * channels;
  ssm_conv_kernel<<<grid_for(total), 256, 0, stream>>>(input, kernel, output, conv_kernel,
                                                        channels, tokens, sequences);
  return hipGetLastError();
}

hipError_t launch_build_ssm_conv_state(float* state, const float* input, float* conv_input,
                                       uint32_t conv_kernel, uint32_t channels,
                                       uint32_t tokens, hipStream_t stream) {
  const unsigned grid = (channels + 63u) / 64u;
  build_conv_state_kernel<<<grid, 256, 0, stream>>>(state, input, conv_input, conv_kernel,
                                                    channels, tokens);
  return hipGetLastError();
}

hipError_t launch_ssm_conv1_stateful(float* state, const float* input, const float* kernel,
                                     float* output, uint32_t conv_kernel, uint32_t channels,
                                     hipStream_t stream) {
  conv1_stateful_kernel<<<(channels + 255u) / 256u, 256, 0, stream>>>(state, input, kernel,
                                                                      output, conv_kernel,
                                                                      channels);
  return hipGetLastError();
}

hipError_t launch_conv_split_l2(const float* qkv, float* conv_state, const float* weights,
                                uint32_t conv_kernel, uint32_t tokens, uint32_t key_heads,
                                uint32_t value_heads, uint32_t head_dim, float eps,
                                float* query, float* key, float* value, hipStream_t stream) {
  const uint32_t heads_total = 2u * key_heads + value_heads;
  const uint32_t tokens_per_block = 4u * kConvTokensPerWave;
  const uint32_t tiles = (tokens + tokens_per_block - 1) / tokens_per_block;
  const dim3 grid(heads_total * tiles);
  const uint32_t cpl = (head_dim + 63u) / 64u;
  const int kk = (int)conv_kernel;
#define KRAKEN_CONV_CASE(CPLV, KV)                                                        \
  if (cpl <= CPLV && kk == KV) {                                                          \
    conv_split_l2_kernel<CPLV, KV><<<grid, 256, 0, stream>>>(                            \
      qkv, conv_state, weights, tokens, key_heads, value_heads, head_dim, eps, query, key, \
      value);                                                                             \
  } else
#define KRAKEN_CONV_CPL(CPLV)                                                             \
  KRAKEN_CONV_CASE(CPLV, 2) KRAKEN_CONV_CASE(CPLV, 3) KRAKEN_CONV_CASE(CPLV, 4)          \
  KRAKEN_CONV_CASE(CPLV, 5) KRAKEN_CONV_CASE(CPLV, 6) KRAKEN_CONV_CASE(CPLV, 7)          \
  KRAKEN_CONV_CASE(CPLV, 8)
  KRAKEN_CONV_CPL(1) KRAKEN_CONV_CPL(2) KRAKEN_CONV_CPL(4) { return hipErrorInvalidValue; }
#undef KRAKEN_CONV_CPL
#undef KRAKEN_CONV_CASE
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return e;
  }
  const uint32_t channels = heads_total * head_dim;
  conv_state_update_kernel<<<(channels + 255u) / 256u, 256, 0, stream>>>(
    conv_state, qkv, conv_kernel, tokens, channels);
  return hipGetLastError();
}

hipError_t launch_conv_split_l2_ragged(const float* qkv, float* conv_pool,
                                       const uint64_t* seq_conv_offsets, uint64_t pool_elems,
                                       const float* weights, uint32_t conv_kernel,
                                       uint32_t sequences, uint32_t key_heads,
                                       uint32_t value_heads, uint32_t head_dim, float eps,
                                       float* query, float* key, float* value,
                                       hipStream_t stream) {
  const dim3 grid(2u * key_heads + value_heads, sequences);
  const uint32_t cpl = (head_dim + 63u) / 64u;
  const int kk = (int)conv_kernel;
#define KRAKEN_CONV_CASE(CPLV, KV)                                                           \
  if (cpl <= CPLV && kk == KV) {                                                             \
    conv_split_l2_ragged_kernel<CPLV, KV><<<grid, 64, 0, stream>>>(                          \
      qkv, conv_pool, seq_conv_offsets, pool_elems, weights, key_heads, value_heads, head_dim, \
      eps, query, key, value);                                                               \
  } else
#define KRAKEN_CONV_CPL(CPLV)                                                                \
  KRAKEN_CONV_CASE(CPLV, 2) KRAKEN_CONV_CASE(CPLV, 3) KRAKEN_CONV_CASE(CPLV, 4)             \
  KRAKEN_CONV_CASE(CPLV, 5) KRAKEN_CONV_CASE(CPLV, 6) KRAKEN_CONV_CASE(CPLV, 7)             \
  KRAKEN_CONV_CASE(CPLV, 8)
  KRAKEN_CONV_CPL(1) KRAKEN_CONV_CPL(2) KRAKEN_CONV_CPL(4) { return hipErrorInvalidValue; }
#undef KRAKEN_CONV_CPL
#undef KRAKEN_CONV_CASE
  return hipGetLastError();
}

bool gdn_layer_fused_supported(uint32_t head_dim, uint32_t conv_kernel, uint32_t key_heads,
                               uint32_t value_heads) {
  return head_dim == 128 && conv_kernel == 4 && key_heads == value_heads;
}

hipError_t launch_gdn_state_ragged(const GdnLayerArgs& a, hipStream_t stream) {
  // One row per 32-lane group (256 workgroups per sequence) while that is at
  // most a few thousand workgroups, else two.
  const bool one_row = (uint64_t)a.sequences * a.heads * 16u <= 4096u;
  const dim3 grid(one_row ? 16u : 8u, a.heads, a.sequences);
  if (a.dt_bias != nullptr) {
    if (one_row) {
      gdn_state_split_kernel<true, 1><<<grid, 256, 0, stream>>>(a);
    } else {
      gdn_state_split_kernel<true, 2><<<grid, 256, 0, stream>>>(a);
    }
  } else if (one_row) {
    gdn_state_split_kernel<false, 1><<<grid, 256, 0, stream>>>(a);
  } else {
    gdn_state_split_kernel<false, 2><<<grid, 256, 0, stream>>>(a);
  }
  return hipGetLastError();
}

hipError_t launch_gdn_layer_ragged(const GdnLayerArgs& a, hipStream_t stream) {
  const dim3 grid(a.heads, a.sequences);
  if (a.dt_bias != nullptr) {
    gdn_layer_ragged_kernel<true><<<grid, 256, 0, stream>>>(a);
  } else {
    gdn_layer_ragged_kernel<false><<<grid, 256, 0, stream>>>(a);
  }
  return hipGetLastError();
}

}  // namespace kraken
