// Chunked (WY / UT-transform) form of the gated-delta-net prefill for head_dim
// 128, on fp32 MFMA (v_mfma_f32_16x16x4f32).
//
// It computes exactly the recurrence of the reference MSL kernel
// gated_delta_net_f32_batched_qwen35 (mps_backend.mm:2307-2374), per value head
// h and state row r (value dim), per token t:
//     S *= exp(g_t);  sk = S.k_t;  delta_t = (v_t[r] - sk) beta_t;
//     S += k_t delta_t;  y_t[r] = (S.q_t) / sqrt(D)
// rearranged over chunks of C = 64 tokens.  With G_t the inclusive sum of g over
// the chunk, gamma_t = exp(G_t), and S_0 the state before the chunk:
//     delta = T (diag(beta) V - diag(beta gamma) K S_0^T)            (C x rows)
//           = U - W S_0^T,  U = T diag(beta) V,  W = T diag(beta gamma) K
//     T = (I + A)^-1,  A[t][j] = beta_t exp(G_t - G_j) (k_t . k_j)  for j < t
//     Y = scale (diag(gamma) Q S_0^T + M delta),
//         M[t][j] = exp(G_t - G_j) (q_t . k_j)  for j <= t
//     S_C = exp(G_C) S_0 + Ktil^T delta,  Ktil[t] = exp(G_C - G_t) k_t
// (G_C is G of the chunk's last token).  Unrolling the recurrence gives these
// identities term by term; they are checked against the sequential kernel and
// the CPU oracle by the tests.  All decay factors are <= 1.
//
// Two kernels:
//  * gdn_chunk_prep_kernel, one workgroup per (chunk, value head), all chunks
//    in parallel: stages K, Q, V of the chunk in LDS, forms G, the Gram
//    matrices K K^T and Q K^T (MFMA), A and M, inverts I + A (diagonal 16 x 16
//    blocks by substitution, off-diagonal blocks by block substitution), then
//    U, W (MFMA), Qtil = diag(gamma) Q and Ktil^T into a workspace block.
//  * gdn_chunk_scan_kernel, one workgroup per (16 state rows, value head),
//    sequential over the chunks: the 16 x 128 state slice lives in LDS; per
//    chunk it forms [W; Qtil] S_0^T (MFMA, the state as the B operand in
//    registers), delta, Y = Z + M delta, and S_C = gamma_C S_0 + Ktil^T delta.
// MFMA operand layout of v_mfma_f32_16x16x4f32 (checked on the device): A[i][k]
// in lane i + 16 k, B[k][j] in lane j + 16 k, D[i][j] in lane j + 16 (i / 4),
// register i % 4.  The k index is relabelled per lane group (lane / 16 = kq
// supplies the contiguous k range of its group), which A and B share.
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>

#include "context_internal.hpp"
#include "device_common.hpp"

namespace kraken {
namespace {

constexpr int kC = 64;         // tokens per chunk
constexpr int kDim = 128;      // head_dim
constexpr int kRowPad = kDim + 4;
constexpr int kCPad = kC + 4;
constexpr int kScanRows = 16;  // state rows per scan workgroup
// Workspace block per (chunk, value head), in floats.
constexpr size_t kOffW = 0;                     // W     [C][D]
constexpr size_t kOffQ = kOffW + kC * kDim;     // Qtil  [C][D]
constexpr size_t kOffU = kOffQ + kC * kDim;     // U     [C][D]
constexpr size_t kOffKT = kOffU + kC * kDim;    // Ktil^T [D][C]
constexpr size_t kOffM = kOffKT + kDim * kC;    // M     [C][C]
constexpr size_t kOffGammaC = kOffM + kC * kC;  // gamma_C
constexpr size_t kBlockFloats = kOffGammaC + 4;
// Chunks per prep/scan pair: bounds the workspace (per value head 9.4 MB).
constexpr uint32_t kSlabChunks = 64;

typedef float float4_v __attribute__((ext_vector_type(4)));

struct ChunkParams {
  const float* query;
  const float* key;
  const float* value;
  const float* gate;
  const float* beta;
  const float* dt_bias;
  const float* ssm_a;
  float* state;
  float* output;
  float* ws;
  uint32_t tokens, chunk0, chunks, key_heads, value_heads;
  float scale;
};

__device__ __forceinline__ float softplus_ref(float x) {
  return x > 20.0f ? x : log1pf(expf(x));
}

__device__ __forceinline__ float4_v mfma4(float a, float b, float4_v c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <bool kPrepare>
__global__ __launch_bounds__(256) void gdn_chunk_prep_kernel(ChunkParams p) {
  __shared__ __attribute__((aligned(16))) float Ks[kC][kRowPad];
  __shared__ __attribute__((aligned(16))) float Qs[kC][kRowPad];
  __shared__ __attribute__((aligned(16))) float Vs[kC][kRowPad];
  __shared__ __attribute__((aligned(16))) float As[kC][kCPad];
  __shared__ __attribute__((aligned(16))) float Ts[kC][kCPad];
  __shared__ __attribute__((aligned(16))) float Tmp[3][16][16];
  __shared__ float Gs[kC], Bs[kC], Gam[kC];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int li = lane & 15;  // MFMA row / column within a tile
  const int kq = lane >> 4;  // MFMA k group
  const uint32_t cl = blockIdx.x;
  const uint32_t c = p.chunk0 + cl;
  const uint32_t h = blockIdx.y;
  const uint32_t kh = h % p.key_heads;
  const uint32_t t0 = c * kC;
  const uint32_t n = min((uint32_t)kC, p.tokens - t0);
  float* blk = p.ws + ((size_t)cl * p.value_heads + h) * kBlockFloats;

  // ---- stage K, Q, V (rows past the chunk's tokens are zero) ----
  // Unconditional loads from a valid row (the chunk's first token stands in for
  // rows past its end), zeroed afterwards, so all of them are in flight at once.
#pragma unroll
  for (int it = 0; it < kC * (kDim / 4) / 256; ++it) {
    const int idx = tid + 256 * it;
    const int t = idx >> 5;
    const int c4 = (idx & 31) * 4;
    const bool ok = (uint32_t)t < n;
    const uint32_t tr = t0 + (ok ? t : 0);
    const size_t ko = ((size_t)tr * p.key_heads + kh) * kDim + c4;
    float4 kk = *reinterpret_cast<const float4*>(p.key + ko);
    float4 qq = *reinterpret_cast<const float4*>(p.query + ko);
    float4 vv = *reinterpret_cast<const float4*>(p.value + ((size_t)tr * p.value_heads + h) * kDim + c4);
    if (!ok) {
      kk = qq = vv = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    *reinterpret_cast<float4*>(&Ks[t][c4]) = kk;
    *reinterpret_cast<float4*>(&Qs[t][c4]) = qq;
    *reinterpret_cast<float4*>(&Vs[t][c4]) = vv;
  }
  for (int idx = tid; idx < kC * kCPad; idx += 256) {
    (&As[0][0])[idx] = 0.0f;
    (&Ts[0][0])[idx] = 0.0f;
  }
  if (tid < kC) {
    float g = 0.0f, b = 0.0f;
    if ((uint32_t)tid < n) {
      const size_t gi = (size_t)(t0 + tid) * p.value_heads + h;
      g = p.gate[gi];
      b = p.beta[gi];
      if (kPrepare) {
        g = softplus_ref(g + p.dt_bias[h]) * p.ssm_a[h];
        b = 1.0f / (1.0f + expf(-b));
      }
    }
    // Inclusive prefix sum of g over the chunk (one wave).
    float x = g;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float y = __shfl_up(x, off, 64);
      if (lane >= off) {
        x += y;
      }
    }
    Gs[tid] = x;
    Gam[tid] = expf(x);
    Bs[tid] = b;
  }
  __syncthreads();
  const float g_last = Gs[kC - 1];  // padded tokens carry g = 0

  // ---- Gram matrices: tiles (I, J), J <= I, of K K^T (A) and Q K^T (M) ----
  // Jobs 0..9: the ten lower tiles of K K^T, 10..19: of Q K^T.  A wave runs two
  // jobs per pass with independent accumulators (LDS reads of one overlap the
  // MFMAs of the other).
  auto gram_tile = [&](int job, int& I, int& J, bool& is_q) __attribute__((always_inline)) {
    is_q = job >= 10;
    int jj = is_q ? job - 10 : job;  // lower-triangular tile index
    I = 0;
    while (jj > I) {
      jj -= I + 1;
      ++I;
    }
    J = jj;
  };
  auto gram_store = [&](int I, int J, bool is_q, const float4_v& acc) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 16 * I + 4 * kq + r;
      const int j = 16 * J + li;
      const float decay = expf(Gs[t] - Gs[j]);
      if (is_q) {
        blk[kOffM + t * kC + j] = j <= t ? decay * acc[r] : 0.0f;
      } else {
        As[t][j] = j < t ? Bs[t] * decay * acc[r] : 0.0f;
      }
    }
  };
  for (int job = wave; job < 20; job += 8) {
    int I0, J0, I1, J1;
    bool q0, q1;
    gram_tile(job, I0, J0, q0);
    const bool two = job + 4 < 20;
    gram_tile(two ? job + 4 : job, I1, J1, q1);
    const float(*X0)[kRowPad] = q0 ? Qs : Ks;
    const float(*X1)[kRowPad] = q1 ? Qs : Ks;
    float4_v acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
#pragma unroll
    for (int s4 = 0; s4 < 8; ++s4) {
      const float4 a0 = *reinterpret_cast<const float4*>(&X0[16 * I0 + li][32 * kq + 4 * s4]);
      const float4 b0 = *reinterpret_cast<const float4*>(&Ks[16 * J0 + li][32 * kq + 4 * s4]);
      const float4 a1 = *reinterpret_cast<const float4*>(&X1[16 * I1 + li][32 * kq + 4 * s4]);
      const float4 b1 = *reinterpret_cast<const float4*>(&Ks[16 * J1 + li][32 * kq + 4 * s4]);
      acc0 = mfma4(a0.x, b0.x, acc0);
      acc1 = mfma4(a1.x, b1.x, acc1);
      acc0 = mfma4(a0.y, b0.y, acc0);
      acc1 = mfma4(a1.y, b1.y, acc1);
      acc0 = mfma4(a0.z, b0.z, acc0);
      acc1 = mfma4(a1.z, b1.z, acc1);
      acc0 = mfma4(a0.w, b0.w, acc0);
      acc1 = mfma4(a1.w, b1.w, acc1);
    }
    gram_store(I0, J0, q0, acc0);
    if (two) {
      gram_store(I1, J1, q1, acc1);
    }
  }
  // Upper tiles of M are zero.
  for (int idx = tid; idx < 6 * 256; idx += 256) {
    int u = idx >> 8;  // upper tile index: (I, J) with J > I
    const int e = idx & 255;
    int I = 0, J = 1;
    while (u > 0) {
      --u;
      if (++J == 4) {
        ++I;
        J = I + 1;
      }
    }
    blk[kOffM + (16 * I + (e >> 4)) * kC + 16 * J + (e & 15)] = 0.0f;
  }
  __syncthreads();

  // ---- T = (I + A)^-1: diagonal 16 x 16 blocks by substitution ----
  if (li == lane) {  // lanes 0..15 of each wave: column j of block `wave`
    const int b0 = 16 * wave;
    const int j = lane;
    float col[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      float acc = 0.0f;
#pragma unroll
      for (int m = 0; m < t; ++m) {
        acc = fmaf(As[b0 + t][b0 + m], col[m], acc);
      }
      col[t] = t < j ? 0.0f : (t == j ? 1.0f : -acc);
    }
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      Ts[b0 + t][b0 + j] = col[t];
    }
  }
  __syncthreads();
  // Off-diagonal blocks by block rows: T_IJ = -T_II sum_{K=J}^{I-1} A_IK T_KJ.
  for (int I = 1; I < 4; ++I) {
    for (int idx = tid; idx < I * 256; idx += 256) {
      const int J = idx >> 8;
      const int i = (idx >> 4) & 15;
      const int j = idx & 15;
      float acc = 0.0f;
      for (int K = J; K < I; ++K) {
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          acc = fmaf(As[16 * I + i][16 * K + k], Ts[16 * K + k][16 * J + j], acc);
        }
      }
      Tmp[J][i][j] = acc;
    }
    __syncthreads();
    for (int idx = tid; idx < I * 256; idx += 256) {
      const int J = idx >> 8;
      const int i = (idx >> 4) & 15;
      const int j = idx & 15;
      float acc = 0.0f;
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        acc = fmaf(Ts[16 * I + i][16 * I + k], Tmp[J][k][j], acc);
      }
      Ts[16 * I + i][16 * J + j] = -acc;
    }
    __syncthreads();
  }

  // ---- Qtil = diag(gamma) Q and Ktil^T = (diag(exp(G_C - G)) K)^T ----
  for (int idx = tid; idx < kC * (kDim / 4); idx += 256) {
    const int t = idx >> 5;
    const int c4 = (idx & 31) * 4;
    const float gm = Gam[t];
    float4 qq = *reinterpret_cast<const float4*>(&Qs[t][c4]);
    qq.x *= gm;
    qq.y *= gm;
    qq.z *= gm;
    qq.w *= gm;
    *reinterpret_cast<float4*>(blk + kOffQ + t * kDim + c4) = qq;
  }
  for (int idx = tid; idx < kDim * (kC / 4); idx += 256) {
    const int d = idx >> 4;
    const int t4 = (idx & 15) * 4;
    float4 v;
    v.x = expf(g_last - Gs[t4 + 0]) * Ks[t4 + 0][d];
    v.y = expf(g_last - Gs[t4 + 1]) * Ks[t4 + 1][d];
    v.z = expf(g_last - Gs[t4 + 2]) * Ks[t4 + 2][d];
    v.w = expf(g_last - Gs[t4 + 3]) * Ks[t4 + 3][d];
    *reinterpret_cast<float4*>(blk + kOffKT + d * kC + t4) = v;
  }
  if (tid == 0) {
    blk[kOffGammaC] = expf(g_last);
  }
  __syncthreads();
  // V <- diag(beta) V, K <- diag(beta gamma) K (in place; the Grams are done).
  for (int idx = tid; idx < kC * (kDim / 4); idx += 256) {
    const int t = idx >> 5;
    const int c4 = (idx & 31) * 4;
    const float bv = Bs[t];
    const float bk = Bs[t] * Gam[t];
    float4 vv = *reinterpret_cast<const float4*>(&Vs[t][c4]);
    float4 kk = *reinterpret_cast<const float4*>(&Ks[t][c4]);
    vv.x *= bv;
    vv.y *= bv;
    vv.z *= bv;
    vv.w *= bv;
    kk.x *= bk;
    kk.y *= bk;
    kk.z *= bk;
    kk.w *= bk;
    *reinterpret_cast<float4*>(&Vs[t][c4]) = vv;
    *reinterpret_cast<float4*>(&Ks[t][c4]) = kk;
  }
  __syncthreads();

  // ---- U = T V', W = T K' (C x D): 2 x 32 output tiles, four per pass ----
  for (int job0 = 4 * wave; job0 < 64; job0 += 16) {
    float4_v acc[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      acc[u] = float4_v{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      const int k0 = 16 * kq + 4 * s4;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int job = job0 + u;
        const bool is_w = job >= 32;
        const int tile = job & 31;
        const int R = tile >> 3;   // token row block
        const int Cb = tile & 7;   // dim column block
        const float(*X)[kRowPad] = is_w ? Ks : Vs;
        const float4 a = *reinterpret_cast<const float4*>(&Ts[16 * R + li][k0]);
        acc[u] = mfma4(a.x, X[k0 + 0][16 * Cb + li], acc[u]);
        acc[u] = mfma4(a.y, X[k0 + 1][16 * Cb + li], acc[u]);
        acc[u] = mfma4(a.z, X[k0 + 2][16 * Cb + li], acc[u]);
        acc[u] = mfma4(a.w, X[k0 + 3][16 * Cb + li], acc[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int job = job0 + u;
      const int tile = job & 31;
      float* dst = blk + (job >= 32 ? kOffW : kOffU);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        dst[(16 * (tile >> 3) + 4 * kq + r) * kDim + 16 * (tile & 7) + li] = acc[u][r];
      }
    }
  }
}

// Global operands of one scan chunk for one lane (see gdn_chunk_scan_kernel).
struct ScanOps {
  float4 x[2][8];   // [W; Qtil] rows of the wave's two tiles, 32 k values each
  float4 kt[2][4];  // Ktil^T rows of the wave's two state tiles, 16 tokens each
  float4 m[2][4];   // M rows of the wave's two output tiles (waves 2, 3)
  float u[2][4];    // U values of the wave's delta entries (waves 0, 1)
  float gamma_c;
};

__global__ __launch_bounds__(256) void gdn_chunk_scan_kernel(ChunkParams p) {
  __shared__ __attribute__((aligned(16))) float Sl[kScanRows][kRowPad];
  __shared__ __attribute__((aligned(16))) float dT[kScanRows][kCPad];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int li = lane & 15;
  const int kq = lane >> 4;
  const uint32_t row0 = blockIdx.x * kScanRows;
  const uint32_t h = blockIdx.y;
  float* shead = p.state + ((size_t)h * kDim + row0) * kDim;

  for (int idx = tid; idx < kScanRows * (kDim / 4); idx += 256) {
    const int r = idx >> 5;
    const int c4 = (idx & 31) * 4;
    *reinterpret_cast<float4*>(&Sl[r][c4]) =
      *reinterpret_cast<const float4*>(shead + (size_t)r * kDim + c4);
  }

  // Loads every global operand of chunk cl that this lane uses (issued one
  // chunk ahead, so the chunk loop never waits on memory).
  auto load_ops = [&](uint32_t cl, ScanOps& o) __attribute__((always_inline)) {
    const float* blk = p.ws + ((size_t)cl * p.value_heads + h) * kBlockFloats;
    const float* X = blk + (wave < 2 ? kOffW : kOffQ) + (size_t)(32 * (wave & 1)) * kDim;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const float* xr = X + (size_t)(16 * tt + li) * kDim + 32 * kq;
#pragma unroll
      for (int s4 = 0; s4 < 8; ++s4) {
        o.x[tt][s4] = *reinterpret_cast<const float4*>(xr + 4 * s4);
      }
      const float* kr = blk + kOffKT + (size_t)(32 * wave + 16 * tt + li) * kC + 16 * kq;
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        o.kt[tt][s4] = *reinterpret_cast<const float4*>(kr + 4 * s4);
      }
      if (wave >= 2) {
        const float* mr = blk + kOffM + (size_t)(32 * (wave - 2) + 16 * tt + li) * kC + 16 * kq;
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
          o.m[tt][s4] = *reinterpret_cast<const float4*>(mr + 4 * s4);
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = 32 * wave + 16 * tt + 4 * kq + r;
          o.u[tt][r] = blk[kOffU + (size_t)t * kDim + row0 + li];
        }
      }
    }
    o.gamma_c = blk[kOffGammaC];
  };

  auto chunk = [&](uint32_t cl, const ScanOps& o) __attribute__((always_inline)) {
    const uint32_t t0 = (p.chunk0 + cl) * kC;
    const uint32_t n = min((uint32_t)kC, p.tokens - t0);
    // State slice as the B operand: lane (j, kq) holds S[j][32 kq .. 32 kq + 31].
    float sb[32];
#pragma unroll
    for (int s4 = 0; s4 < 8; ++s4) {
      const float4 v = *reinterpret_cast<const float4*>(&Sl[li][32 * kq + 4 * s4]);
      sb[4 * s4 + 0] = v.x;
      sb[4 * s4 + 1] = v.y;
      sb[4 * s4 + 2] = v.z;
      sb[4 * s4 + 3] = v.w;
    }
    // [W; Qtil] S_0^T: waves 0, 1 take W rows 32 w .., waves 2, 3 Qtil rows.
    float4_v acc[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      acc[tt] = float4_v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s4 = 0; s4 < 8; ++s4) {
        const float4 a = o.x[tt][s4];
        acc[tt] = mfma4(a.x, sb[4 * s4 + 0], acc[tt]);
        acc[tt] = mfma4(a.y, sb[4 * s4 + 1], acc[tt]);
        acc[tt] = mfma4(a.z, sb[4 * s4 + 2], acc[tt]);
        acc[tt] = mfma4(a.w, sb[4 * s4 + 3], acc[tt]);
      }
    }
    if (wave < 2) {
      // delta = U - W S_0^T, stored transposed (rows j, tokens t).
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          dT[li][32 * wave + 16 * tt + 4 * kq + r] = o.u[tt][r] - acc[tt][r];
        }
      }
    }
    __syncthreads();
    if (wave >= 2) {
      // Y = scale (Qtil S_0^T + M delta) for tokens 32 (w - 2) ..
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int tb = 32 * (wave - 2) + 16 * tt;
        float4_v y = acc[tt];
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
          const float4 a = o.m[tt][s4];
          const float4 b = *reinterpret_cast<const float4*>(&dT[li][16 * kq + 4 * s4]);
          y = mfma4(a.x, b.x, y);
          y = mfma4(a.y, b.y, y);
          y = mfma4(a.z, b.z, y);
          y = mfma4(a.w, b.w, y);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t t = tb + 4 * kq + r;
          if (t < n) {
            p.output[((size_t)(t0 + t) * p.value_heads + h) * kDim + row0 + li] = y[r] * p.scale;
          }
        }
      }
    }
    // S_C^T rows (key dims) 32 w .. 32 w + 31 = gamma_C S_0^T + Ktil^T delta.
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int kb = 32 * wave + 16 * tt;
      float4_v s;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s[r] = o.gamma_c * Sl[li][kb + 4 * kq + r];
      }
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const float4 a = o.kt[tt][s4];
        const float4 b = *reinterpret_cast<const float4*>(&dT[li][16 * kq + 4 * s4]);
        s = mfma4(a.x, b.x, s);
        s = mfma4(a.y, b.y, s);
        s = mfma4(a.z, b.z, s);
        s = mfma4(a.w, b.w, s);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        Sl[li][kb + 4 * kq + r] = s[r];
      }
    }
    __syncthreads();
  };

  ScanOps ops_a, ops_b;
  load_ops(0, ops_a);
  __syncthreads();  // state slice staged
  // Two chunks per iteration with the operand sets swapped, so the next
  // chunk's loads are always in flight during the current chunk.
  for (uint32_t cl = 0; cl < p.chunks; cl += 2) {
    if (cl + 1 < p.chunks) {
      load_ops(cl + 1, ops_b);
    }
    chunk(cl, ops_a);
    if (cl + 1 < p.chunks) {
      if (cl + 2 < p.chunks) {
        load_ops(cl + 2, ops_a);
      }
      chunk(cl + 1, ops_b);
    }
  }

  for (int idx = tid; idx < kScanRows * (kDim / 4); idx += 256) {
    const int r = idx >> 5;
    const int c4 = (idx & 31) * 4;
    *reinterpret_cast<float4*>(shead + (size_t)r * kDim + c4) =
      *reinterpret_cast<const float4*>(&Sl[r][c4]);
  }
}

}  // namespace

bool gdn_chunked_supported(const GdnArgs& a) {
  const char* v = std::getenv("KRAKEN_GDN_PREFILL");
  if (v != nullptr && (std::strcmp(v, "generic") == 0 || std::strcmp(v, "sequential") == 0)) {
    return false;
  }
  const bool aligned = ((uintptr_t)a.query | (uintptr_t)a.key | (uintptr_t)a.value |
                        (uintptr_t)a.state | (uintptr_t)a.output) % 16u == 0;
  return a.seq_state_offsets == nullptr && a.head_dim == (uint32_t)kDim && aligned &&
         a.tokens >= (uint32_t)kC;
}

size_t gdn_chunked_workspace_bytes(const GdnArgs& a) {
  const uint32_t chunks = (a.tokens + kC - 1) / kC;
  const uint32_t slab = chunks < kSlabChunks ? chunks : kSlabChunks;
  return kCounterRegionBytes + (size_t)slab * a.value_heads * kBlockFloats * sizeof(float);
}

hipError_t launch_gdn_chunked(const GdnArgs& a, void* workspace, size_t workspace_bytes,
                              hipStream_t stream) {
  if (workspace == nullptr || workspace_bytes < gdn_chunked_workspace_bytes(a)) {
    return hipErrorInvalidValue;
  }
  ChunkParams p{};
  p.query = a.query;
  p.key = a.key;
  p.value = a.value;
  p.gate = a.gate;
  p.beta = a.beta;
  p.dt_bias = a.dt_bias;
  p.ssm_a = a.ssm_a;
  p.state = a.state;
  p.output = a.output;
  // Blocks follow the counter region, which they must never overlap.
  p.ws = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterRegionBytes);
  p.tokens = a.tokens;
  p.key_heads = a.key_heads;
  p.value_heads = a.value_heads;
  p.scale = 1.0f / sqrtf((float)kDim);
  const uint32_t chunks = (a.tokens + kC - 1) / kC;
  for (uint32_t c0 = 0; c0 < chunks; c0 += kSlabChunks) {
    p.chunk0 = c0;
    p.chunks = chunks - c0 < kSlabChunks ? chunks - c0 : kSlabChunks;
    const dim3 pgrid(p.chunks, a.value_heads);
    if (a.dt_bias != nullptr) {
      gdn_chunk_prep_kernel<true><<<pgrid, 256, 0, stream>>>(p);
    } else {
      gdn_chunk_prep_kernel<false><<<pgrid, 256, 0, stream>>>(p);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
      return e;
    }
    gdn_chunk_scan_kernel<<<dim3(kDim / kScanRows, a.value_heads), 256, 0, stream>>>(p);
    e = hipGetLastError();
    if (e != hipSuccess) {
      return e;
    }
  }
  return hipSuccess;
}

}  // namespace kraken
