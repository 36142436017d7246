// Chunked (WY / UT-transform) form of the gated-delta-net prefill for head_dim
// 128, on fp32 MFMA (v_mfma_f32_16x16x4f32), with the sequential scan's two
// products on fp16 MFMA in split (hi + lo) form, which keeps them to about
// 2^-20 of fp32.
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
// Three kernels:
//  * gdn_chunk_prep_kernel, one workgroup per (chunk, value head), all chunks
//    in parallel: stages K, Q, V of the chunk in LDS, forms G, the Gram
//    matrices K K^T and Q K^T (MFMA), A and M, inverts I + A (diagonal 16 x 16
//    blocks by substitution, off-diagonal blocks by block substitution), then
//    U, W (MFMA), gamma and Ktil^T into a workspace block.
//  * gdn_chunk_scan_kernel, one workgroup per (16 state rows, value head),
//    sequential over the chunks, holds only the recurrence: the 16 x 128 state
//    slice lives in LDS; per chunk it stores S_0 and forms delta = U - W S_0^T
//    (stored too) and S_C = gamma_C S_0 + Ktil^T delta (split fp16 MFMA).
//    Loader waves stream the next chunk's W and Ktil^T into LDS meanwhile.
//  * gdn_chunk_out_kernel, one workgroup per (chunk, value head, 64 state
//    rows), all in parallel: Y = scale (diag(gamma) Q S_0^T + M delta).
// Taking Y out of the sequential kernel matters because each of its
// workgroups reads the chunk's operands through one CU's load path (about
// 30 bytes per clock measured), which then bounds the chunk's latency.
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
constexpr size_t kOffW = 0;                     // W     [C][D] as f16 (hi | lo), see below
constexpr size_t kOffGam = kOffW + kC * kDim;   // gamma [C] (exp of the inclusive sum of g)
constexpr size_t kOffU = kOffGam + kC;          // U^T   [D][C]
constexpr size_t kOffKT = kOffU + kC * kDim;    // Ktil^T [D][C] as f16 (hi | lo)
constexpr size_t kOffM = kOffKT + kDim * kC;    // M     [C][C]
constexpr size_t kOffS0 = kOffM + kC * kC;     // S_0   [D][D] (state before the chunk)
constexpr size_t kOffDT = kOffS0 + kDim * kDim; // delta^T [D][C]
constexpr size_t kOffGammaC = kOffDT + kDim * kC;  // gamma_C
constexpr size_t kBlockFloats = kOffGammaC + 4;
// Chunks per prep/scan/out pass: bounds the workspace (per value head 15.6 MB).
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

// The scan's two per-chunk products run on fp16 MFMA in the split form of
// device_common.hpp (split_f16: x = hi + 2^-11 lo, about 2^-21 relative; a
// product sums hi hi + 2^-11 (hi lo + lo hi) in fp32, the dropped lo lo term is
// below 2^-20 of the product).  W and Ktil^T rows are stored by the prep kernel
// in this form: a row of n values is n hi halves then n lo halves, the same bytes
// as the fp32 row.
__device__ __forceinline__ void split4_f16(const float x[4], half4_t& hi, half4_t& lo) {
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    half_t h, l;
    split_f16(x[c], h, l);
    hi[c] = h;
    lo[c] = l;
  }
}

// hi hi into acc_h, the cross terms into acc_x (v_mfma_f32_16x16x32_f16).
__device__ __forceinline__ void mfma_split(half8_t a_hi, half8_t a_lo, half8_t b_hi, half8_t b_lo,
                                           float4_v& acc_h, float4_v& acc_x) {
  acc_h = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_hi, b_hi, acc_h, 0, 0, 0);
  acc_x = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_hi, b_lo, acc_x, 0, 0, 0);
  acc_x = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_lo, b_hi, acc_x, 0, 0, 0);
}

// Eight waves: the prep phases are latency-bound at one workgroup per CU (its
// LDS), so twice the waves hide more of each phase's latency and shorten the
// MFMA critical paths of the Gram and U/W phases.
constexpr int kPrepThreads = 512;
constexpr int kPrepWaves = kPrepThreads / 64;

template <bool kPrepare>
__global__ __launch_bounds__(kPrepThreads) void gdn_chunk_prep_kernel(ChunkParams p) {
  // Operands of the split fp16 products, staged once in split form (hi, lo):
  // K rows; Q rows for the Gram matrices, then (same space) K^T rows (key
  // dims) for W; V^T rows for U.  Rows are padded by 8 halves so that 16 rows
  // at one column start in distinct 4-bank groups.
  constexpr int kRowH = kDim + 8;  // halves per K / Q row
  constexpr int kColH = kC + 8;    // halves per K^T / V^T row
  __shared__ __attribute__((aligned(16))) half_t Kh[kC][kRowH];
  __shared__ __attribute__((aligned(16))) half_t Kl[kC][kRowH];
  __shared__ __attribute__((aligned(16))) half_t QKT[2 * kDim * kColH];
  __shared__ __attribute__((aligned(16))) half_t VTh[kDim][kColH];
  __shared__ __attribute__((aligned(16))) half_t VTl[kDim][kColH];
  static_assert(2 * kC * kRowH <= 2 * kDim * kColH, "Q fits the shared Q / K^T array");
  __shared__ __attribute__((aligned(16))) float As[kC][kCPad];
  __shared__ __attribute__((aligned(16))) float Ts[kC][kCPad];
  __shared__ float Gs[kC], Bs[kC], Gam[kC];
  __shared__ __attribute__((aligned(16))) float Dec[kC];  // exp(G_C - G_t)
  __shared__ __attribute__((aligned(16))) float Red[4][64][4];  // Gram partial sums

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
  half_t(*Qh)[kRowH] = reinterpret_cast<half_t(*)[kRowH]>(QKT);
  half_t(*Ql)[kRowH] = reinterpret_cast<half_t(*)[kRowH]>(QKT + kC * kRowH);
  half_t(*KTh)[kColH] = reinterpret_cast<half_t(*)[kColH]>(QKT);
  half_t(*KTl)[kColH] = reinterpret_cast<half_t(*)[kColH]>(QKT + kDim * kColH);

  // ---- stage K, Q, V^T (rows past the chunk's tokens are zero) ----
  // Unconditional loads from a valid row (the chunk's first token stands in for
  // rows past its end), zeroed afterwards, so all of them are in flight at once.
#pragma unroll
  for (int it = 0; it < kC * (kDim / 4) / kPrepThreads; ++it) {
    const int idx = tid + kPrepThreads * it;
    const int t = idx >> 5;
    const int c4 = (idx & 31) * 4;
    const bool ok = (uint32_t)t < n;
    const uint32_t tr = t0 + (ok ? t : 0);
    const size_t ko = ((size_t)tr * p.key_heads + kh) * kDim + c4;
    float4 kk = *reinterpret_cast<const float4*>(p.key + ko);
    float4 qq = *reinterpret_cast<const float4*>(p.query + ko);
    if (!ok) {
      kk = qq = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const float kx[4] = {kk.x, kk.y, kk.z, kk.w};
    const float qx[4] = {qq.x, qq.y, qq.z, qq.w};
    half4_t hi, lo;
    split4_f16(kx, hi, lo);
    *reinterpret_cast<half4_t*>(&Kh[t][c4]) = hi;
    *reinterpret_cast<half4_t*>(&Kl[t][c4]) = lo;
    split4_f16(qx, hi, lo);
    *reinterpret_cast<half4_t*>(&Qh[t][c4]) = hi;
    *reinterpret_cast<half4_t*>(&Ql[t][c4]) = lo;
  }
  // V transposed: four lanes read 64 contiguous bytes of a row, sixteen rows per
  // 64 lanes, so the transposed writes of a row go to 16 consecutive tokens.
#pragma unroll
  for (int it = 0; it < kC * (kDim / 4) / kPrepThreads; ++it) {
    const int idx = tid + kPrepThreads * it;
    const int t = (idx >> 2) & (kC - 1);
    const int c4 = 16 * (idx >> 8) + 4 * (idx & 3);
    const bool ok = (uint32_t)t < n;
    const uint32_t tr = t0 + (ok ? t : 0);
    float4 vv = *reinterpret_cast<const float4*>(p.value + ((size_t)tr * p.value_heads + h) * kDim + c4);
    if (!ok) {
      vv = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const float vx[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      half_t hi, lo;
      split_f16(vx[e], hi, lo);
      VTh[c4 + e][t] = hi;
      VTl[c4 + e][t] = lo;
    }
  }
  for (int idx = tid; idx < kC * kCPad; idx += kPrepThreads) {
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
  if (tid < kC) {
    Dec[tid] = expf(g_last - Gs[tid]);
  }

  // ---- Gram matrices: tiles (I, J), J <= I, of K K^T (A) and Q K^T (M) ----
  // Jobs 0..9: the ten lower tiles of K K^T, 10..19: of Q K^T.  Wave w runs
  // jobs w and w + 8 in one pass with independent accumulators (LDS reads of
  // one overlap the MFMAs of the other), then half of job 16 + w % 4.
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
  static_assert(kPrepWaves == 8, "job assignment");
  // X rows 16 I .. + 15 times K rows 16 J .. + 15 over k steps [s0, s1) of 32
  // key dims, split fp16 (lane (li, kq): dims 32 s + 8 kq .. + 7 of row li).
  auto gram_acc = [&](bool is_q, int I, int J, int s0, int s1, float4_v& ah, float4_v& ax)
                    __attribute__((always_inline)) {
    const half_t(*Xh)[kRowH] = is_q ? Qh : Kh;
    const half_t(*Xl)[kRowH] = is_q ? Ql : Kl;
#pragma unroll
    for (int st = s0; st < s1; ++st) {
      const int c = 32 * st + 8 * kq;
      mfma_split(*reinterpret_cast<const half8_t*>(&Xh[16 * I + li][c]),
                 *reinterpret_cast<const half8_t*>(&Xl[16 * I + li][c]),
                 *reinterpret_cast<const half8_t*>(&Kh[16 * J + li][c]),
                 *reinterpret_cast<const half8_t*>(&Kl[16 * J + li][c]), ah, ax);
    }
  };
  auto combine = [&](const float4_v& ah, const float4_v& ax) __attribute__((always_inline)) {
    return float4_v{ah[0] + kLoUnscale * ax[0], ah[1] + kLoUnscale * ax[1],
                    ah[2] + kLoUnscale * ax[2], ah[3] + kLoUnscale * ax[3]};
  };
  {
    // Jobs w and w + 8 (0..15) in one pass with independent accumulators.
    const int job = wave;
    int I0, J0, I1, J1;
    bool q0, q1;
    gram_tile(job, I0, J0, q0);
    gram_tile(job + 8, I1, J1, q1);
    float4_v h0 = {0.f, 0.f, 0.f, 0.f}, x0 = h0, h1 = h0, x1 = h0;
#pragma unroll
    for (int st = 0; st < kDim / 32; ++st) {
      gram_acc(q0, I0, J0, st, st + 1, h0, x0);
      gram_acc(q1, I1, J1, st, st + 1, h1, x1);
    }
    gram_store(I0, J0, q0, combine(h0, x0));
    gram_store(I1, J1, q1, combine(h1, x1));
  }
  {
    // Jobs 16..19: wave w takes job 16 + w % 4 over half the key dims
    // (w / 4); the second half's partial sums meet the first's in LDS.
    int I, J;
    bool q;
    gram_tile(16 + (wave & 3), I, J, q);
    const int s0 = 2 * (wave >> 2);
    float4_v ah = {0.f, 0.f, 0.f, 0.f}, ax = ah;
    gram_acc(q, I, J, s0, s0 + 2, ah, ax);
    float4_v acc = combine(ah, ax);
    if (wave >= 4) {
      *reinterpret_cast<float4*>(&Red[wave & 3][lane][0]) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    }
    __syncthreads();
    if (wave < 4) {
      const float4 o = *reinterpret_cast<const float4*>(&Red[wave][lane][0]);
      acc[0] += o.x;
      acc[1] += o.y;
      acc[2] += o.z;
      acc[3] += o.w;
      gram_store(I, J, q, acc);
    }
  }
  // Upper tiles of M are zero.
  for (int idx = tid; idx < 6 * 256; idx += kPrepThreads) {
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

  // ---- T = (I + A)^-1: diagonal 16 x 16 blocks by substitution; waves 4..7
  // meanwhile transpose K into K^T (Q is done with) and store
  // Ktil^T = (diag(exp(G_C - G)) K)^T ----
  // The transpose runs in four parts, one beside each inversion phase (the
  // diagonal blocks and the three off-diagonal block rows keep waves 4..7
  // idle); part `part` takes key dims 32 part .. 32 part + 31.
  auto transpose_part = [&](int part) __attribute__((always_inline)) {
    if (wave >= 4) {
      for (int idx = tid - 256; idx < 32 * (kC / 4); idx += 256) {
        const int d = 32 * part + (idx >> 4);
        const int t4 = (idx & 15) * 4;
        half4_t kh, kl;
        float kt[4];
        const float4 e = *reinterpret_cast<const float4*>(&Dec[t4]);
        const float ev[4] = {e.x, e.y, e.z, e.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          kh[i] = Kh[t4 + i][d];
          kl[i] = Kl[t4 + i][d];
          kt[i] = ev[i] * (static_cast<float>(kh[i]) + kLoUnscale * static_cast<float>(kl[i]));
        }
        *reinterpret_cast<half4_t*>(&KTh[d][t4]) = kh;
        *reinterpret_cast<half4_t*>(&KTl[d][t4]) = kl;
        half4_t hi, lo;
        split4_f16(kt, hi, lo);
        half_t* row = reinterpret_cast<half_t*>(blk + kOffKT) + d * (2 * kC);
        *reinterpret_cast<half4_t*>(row + t4) = hi;
        *reinterpret_cast<half4_t*>(row + kC + t4) = lo;
      }
    }
  };
  transpose_part(0);
  if (wave < 4 && li == lane) {  // lanes 0..15 of waves 0..3: column j of block `wave`
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
  // Off-diagonal blocks by block rows: T_IJ = -T_II sum_{K=J}^{I-1} A_IK T_KJ,
  // wave J computing T_IJ on MFMA.  The first product leaves lane (j, q) with
  // rows 4q .. 4q + 3 of column j; the second relabels k = 4 kq + s for
  // instruction s, so that accumulator register s is its B operand as is.
  for (int I = 1; I < 4; ++I) {
    transpose_part(I);
    if (wave < I) {
      const int J = wave;
      float4_v acc = {0.f, 0.f, 0.f, 0.f};
      for (int K = J; K < I; ++K) {
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
          acc = mfma4(As[16 * I + li][16 * K + 4 * s4 + kq], Ts[16 * K + 4 * s4 + kq][16 * J + li],
                      acc);
        }
      }
      float4_v t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        t = mfma4(Ts[16 * I + li][16 * I + 4 * kq + s4], acc[s4], t);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        Ts[16 * I + 4 * kq + r][16 * J + li] = -t[r];
      }
    }
    __syncthreads();
  }

  // ---- gamma (the output kernel forms diag(gamma) Q S_0^T) ----
  if (tid < kC) {
    blk[kOffGam + tid] = Gam[tid];
  }
  if (tid == 0) {
    blk[kOffGammaC] = expf(g_last);
  }
  // ---- U = T diag(beta) V, W = T diag(beta gamma) K (C x D): 2 x 32 output
  // tiles, four per pass (one token row block R, four dim column blocks), on
  // split fp16 MFMA.  The A operand, T's rows 16 R + li with column k scaled by
  // beta_k (or beta_k gamma_k), k = 32 s + 8 kq + e, is split once per pass;
  // the B operands are the staged split V^T and K^T rows. ----
  for (int job0 = 4 * wave; job0 < 64; job0 += 4 * kPrepWaves) {
    const bool is_w = job0 >= 32;
    const int R = (job0 & 31) >> 3;
    half8_t ah[kC / 32], al[kC / 32];
#pragma unroll
    for (int st = 0; st < kC / 32; ++st) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int k = 32 * st + 8 * kq + e;
        const float f = is_w ? Bs[k] * Gam[k] : Bs[k];
        half_t hi, lo;
        split_f16(Ts[16 * R + li][k] * f, hi, lo);
        ah[st][e] = hi;
        al[st][e] = lo;
      }
    }
    const half_t(*XTh)[kColH] = is_w ? KTh : VTh;
    const half_t(*XTl)[kColH] = is_w ? KTl : VTl;
    float4_v acc[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int Cb = (job0 + u) & 7;  // dim column block
      float4_v h = {0.f, 0.f, 0.f, 0.f}, x = h;
#pragma unroll
      for (int st = 0; st < kC / 32; ++st) {
        const int c = 32 * st + 8 * kq;
        mfma_split(ah[st], al[st], *reinterpret_cast<const half8_t*>(&XTh[16 * Cb + li][c]),
                   *reinterpret_cast<const half8_t*>(&XTl[16 * Cb + li][c]), h, x);
      }
      acc[u] = combine(h, x);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int job = job0 + u;
      const int R = (job & 31) >> 3;
      const int Cb = job & 7;
      if (job >= 32) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          half_t hi, lo;
          split_f16(acc[u][r], hi, lo);
          half_t* row = reinterpret_cast<half_t*>(blk + kOffW) + (16 * R + 4 * kq + r) * (2 * kDim);
          row[16 * Cb + li] = hi;
          row[kDim + 16 * Cb + li] = lo;
        }
      } else {  // U transposed: the four tokens of a lane are contiguous
        *reinterpret_cast<float4*>(blk + kOffU + (16 * Cb + li) * kC + 16 * R + 4 * kq) =
          make_float4(acc[u][0], acc[u][1], acc[u][2], acc[u][3]);
      }
    }
  }
}

// The scan's workgroup: four compute waves run the recurrence; four loader
// waves stream the next chunk's W and Ktil^T into the other LDS buffer with
// direct-to-LDS copies and store S_0 and delta.  The chunk is bound about
// equally by one CU's MFMA rate and by its load path (about 30 bytes per clock
// for the 64 KB of W and Ktil^T); with the loads issued by the compute waves,
// an in-order wave stalled on a load issues no MFMAs and the two add up.
constexpr int kScanThreads = 512;
constexpr int kScanCompute = 4;  // waves 0..3; 4..7 load

__global__ __launch_bounds__(kScanThreads) void gdn_chunk_scan_kernel(ChunkParams p) {
  // W and Ktil^T of the current and the next chunk.  Each row's 16-byte chunks
  // are XOR-swizzled by row % 16 (the copies pick which global chunk a lane
  // fetches), so the compute waves' reads of 16 rows at one column are free of
  // bank conflicts.
  __shared__ __attribute__((aligned(16))) float Wb[2][kC * kDim];
  __shared__ __attribute__((aligned(16))) float KTb[2][kDim * kC];
  __shared__ __attribute__((aligned(16))) float Sl[kScanRows][kRowPad];
  __shared__ __attribute__((aligned(16))) float dT[kScanRows][kCPad];
  // The state slice and delta^T again in split form (hi, lo) for the MFMA B
  // operands; rows padded by 8 halves so that 16 rows at one column start in
  // distinct 4-bank groups.
  __shared__ __attribute__((aligned(16))) half_t Sh[kScanRows][kDim + 8];
  __shared__ __attribute__((aligned(16))) half_t Slo[kScanRows][kDim + 8];
  __shared__ __attribute__((aligned(16))) half_t dTh[kScanRows][kC + 8];
  __shared__ __attribute__((aligned(16))) half_t dTl[kScanRows][kC + 8];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15;
  const int kq = lane >> 4;
  // Workgroup i runs on XCD i % 8.  The (head, row block) pairs are numbered
  // so that the eight row blocks of a head share an XCD and its L2, which then
  // fetches the head's chunk operands once instead of eight times.
  constexpr uint32_t kXcds = 8;
  static_assert(kDim / kScanRows == kXcds, "grid of value_heads * kXcds workgroups");
  const uint32_t q = (blockIdx.x % kXcds) * p.value_heads + blockIdx.x / kXcds;
  const uint32_t row0 = (q % (kDim / kScanRows)) * kScanRows;
  const uint32_t h = q / (kDim / kScanRows);
  float* shead = p.state + ((size_t)h * kDim + row0) * kDim;
  auto block = [&](uint32_t cl) { return p.ws + ((size_t)cl * p.value_heads + h) * kBlockFloats; };

  // ---- loader side: chunk cl's W and Ktil^T into buffer b ----
  // Copy i of W fills LDS rows 2i, 2i + 1 (lane / 32) at physical chunk
  // lane % 32; copy i of Ktil^T fills rows 4i .. 4i + 3 (lane / 16) at
  // physical chunk lane % 16.  Loader wave lw issues copies 8 lw .. 8 lw + 7
  // of each.
  auto load_chunk = [&](uint32_t cl, int b) {
    const int lw = wave - kScanCompute;
    const i32x4_t rs = rsrc_words(block(cl), (uint32_t)(kBlockFloats * 4));
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = 8 * lw + j;
      const int row = 2 * i + (lane >> 5);
      const int g = (lane & 31) ^ (row & 15);
      copy16_to_lds(rs, (uint32_t)(kOffW * 4 + row * 512 + g * 16),
                    reinterpret_cast<const half_t*>(&Wb[b][0]) + i * 512);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = 8 * lw + j;
      const int row = 4 * i + (lane >> 4);
      const int g = (lane & 15) ^ (row & 15);
      copy16_to_lds(rs, (uint32_t)(kOffKT * 4 + row * 256 + g * 16),
                    reinterpret_cast<const half_t*>(&KTb[b][0]) + i * 512);
    }
  };

  for (int idx = tid; idx < kScanRows * (kDim / 4); idx += kScanThreads) {
    const int r = idx >> 5;
    const int c4 = (idx & 31) * 4;
    const float4 v = *reinterpret_cast<const float4*>(shead + (size_t)r * kDim + c4);
    *reinterpret_cast<float4*>(&Sl[r][c4]) = v;
    const float x[4] = {v.x, v.y, v.z, v.w};
    half4_t hi, lo;
split4_f16(x, hi, lo);
    *reinterpret_cast<half4_t*>(&Sh[r][c4]) = hi;
    *reinterpret_cast<half4_t*>(&Slo[r][c4]) = lo;
  }
  if (wave >= kScanCompute) {
    load_chunk(0, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  __syncthreads();  // state slice and chunk 0's operands staged

  if (wave >= kScanCompute) {
    // Per chunk: S_0 out, the next chunk's copies, [barrier], delta out, the
    // copies awaited, [barrier].
    const int lt = tid - kScanCompute * 64;
    for (uint32_t cl = 0; cl < p.chunks; ++cl) {
      float* blk = block(cl);
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const int idx = lt + 256 * it;
        const int r = idx >> 5;
        const int c4 = (idx & 31) * 4;
        *reinterpret_cast<float4*>(blk + kOffS0 + (size_t)(row0 + r) * kDim + c4) =
          *reinterpret_cast<const float4*>(&Sl[r][c4]);
      }
      if (cl + 1 < p.chunks) {
        load_chunk(cl + 1, (int)((cl + 1) & 1u));
      }
      __syncthreads();  // B1: delta^T is in dT
      {
        const int r = lt >> 4;
        const int t4 = (lt & 15) * 4;
        *reinterpret_cast<float4*>(blk + kOffDT + (size_t)(row0 + r) * kC + t4) =
          *reinterpret_cast<const float4*>(&dT[r][t4]);
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();  // B2: S_C in Sl, the next chunk's operands landed
    }
    return;
  }

  // ---- compute side ----
  // U entries of the lane's four delta values and gamma_C, one chunk ahead.
  auto load_u = [&](uint32_t cl, float4& u, float& gamma_c) {
    const float* blk = block(cl);
    u = *reinterpret_cast<const float4*>(blk + kOffU + (size_t)(row0 + li) * kC + 16 * wave +
                                          4 * kq);
    gamma_c = blk[kOffGammaC];
  };
  float4 u, nu;
  float gamma_c, ngamma_c;
  load_u(0, u, gamma_c);
  for (uint32_t cl = 0; cl < p.chunks; ++cl) {
    const int b = (int)(cl & 1u);
    const char* wb = reinterpret_cast<const char*>(&Wb[b][0]);
    const char* kb = reinterpret_cast<const char*>(&KTb[b][0]);
    load_u(min(cl + 1, p.chunks - 1), nu, ngamma_c);
    // delta = U - W S_0^T for tokens 16 w .. 16 w + 15 on split fp16 MFMA
    // (v_mfma_f32_16x16x32_f16, k steps of 32 key dims): lane (li, kq) holds
    // A = W[16 w + li][32 s + 8 kq .. + 7] (hi at logical chunk 4 s + kq of the
    // row, lo at 16 + 4 s + kq; physical chunk = logical ^ li) and
    // B = S_0[li][32 s + 8 kq .. + 7].
    const int wrow = 16 * wave + li;
    float4_v acc_h = {0.f, 0.f, 0.f, 0.f};
    float4_v acc_x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < kDim / 32; ++st) {
      const half8_t a_hi =
        *reinterpret_cast<const half8_t*>(wb + wrow * 512 + 16 * ((4 * st + kq) ^ li));
      const half8_t a_lo =
        *reinterpret_cast<const half8_t*>(wb + wrow * 512 + 16 * ((16 + 4 * st + kq) ^ li));
      const half8_t b_hi = *reinterpret_cast<const half8_t*>(&Sh[li][32 * st + 8 * kq]);
      const half8_t b_lo = *reinterpret_cast<const half8_t*>(&Slo[li][32 * st + 8 * kq]);
      mfma_split(a_hi, a_lo, b_hi, b_lo, acc_h, acc_x);
    }
    // delta^T (rows j, tokens t): lane holds tokens 16 w + 4 kq + r of row li.
    // fp32 for the loader waves to store, split for the S_C product.
    {
      const float d[4] = {u.x - (acc_h[0] + kLoUnscale * acc_x[0]),
                          u.y - (acc_h[1] + kLoUnscale * acc_x[1]),
                          u.z - (acc_h[2] + kLoUnscale * acc_x[2]),
                          u.w - (acc_h[3] + kLoUnscale * acc_x[3])};
      *reinterpret_cast<float4*>(&dT[li][16 * wave + 4 * kq]) = make_float4(d[0], d[1], d[2], d[3]);
      half4_t hi, lo;
split4_f16(d, hi, lo);
      *reinterpret_cast<half4_t*>(&dTh[li][16 * wave + 4 * kq]) = hi;
      *reinterpret_cast<half4_t*>(&dTl[li][16 * wave + 4 * kq]) = lo;
    }
    __syncthreads();  // B1
    // S_C^T rows (key dims) 32 w .. 32 w + 31 = gamma_C S_0^T + Ktil^T delta,
    // k steps of 32 tokens: A = Ktil^T[32 w + 16 tt + li][32 s + 8 kq .. + 7]
    // (hi at logical chunk 4 s + kq, lo at 8 + 4 s + kq; physical = logical ^ li),
    // B = delta[32 s + 8 kq .. + 7][li].
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int kbase = 32 * wave + 16 * tt;
      const float4 s0 = *reinterpret_cast<const float4*>(&Sl[li][kbase + 4 * kq]);
      float4_v sh = {0.f, 0.f, 0.f, 0.f};
      float4_v sx = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < kC / 32; ++st) {
        const half8_t a_hi = *reinterpret_cast<const half8_t*>(kb + (kbase + li) * 256 +
                                                               16 * ((4 * st + kq) ^ li));
        const half8_t a_lo = *reinterpret_cast<const half8_t*>(kb + (kbase + li) * 256 +
                                                               16 * ((8 + 4 * st + kq) ^ li));
        const half8_t b_hi = *reinterpret_cast<const half8_t*>(&dTh[li][32 * st + 8 * kq]);
        const half8_t b_lo = *reinterpret_cast<const half8_t*>(&dTl[li][32 * st + 8 * kq]);
        mfma_split(a_hi, a_lo, b_hi, b_lo, sh, sx);
      }
      const float sc[4] = {fmaf(gamma_c, s0.x, sh[0] + kLoUnscale * sx[0]),
                           fmaf(gamma_c, s0.y, sh[1] + kLoUnscale * sx[1]),
                           fmaf(gamma_c, s0.z, sh[2] + kLoUnscale * sx[2]),
                           fmaf(gamma_c, s0.w, sh[3] + kLoUnscale * sx[3])};
      *reinterpret_cast<float4*>(&Sl[li][kbase + 4 * kq]) = make_float4(sc[0], sc[1], sc[2], sc[3]);
      half4_t hi, lo;
split4_f16(sc, hi, lo);
      *reinterpret_cast<half4_t*>(&Sh[li][kbase + 4 * kq]) = hi;
      *reinterpret_cast<half4_t*>(&Slo[li][kbase + 4 * kq]) = lo;
    }
    __syncthreads();  // B2
    u = nu;
    gamma_c = ngamma_c;
  }

  for (int idx = tid; idx < kScanRows * (kDim / 4); idx += kScanCompute * 64) {
    const int r = idx >> 5;
    const int c4 = (idx & 31) * 4;
    *reinterpret_cast<float4*>(shead + (size_t)r * kDim + c4) =
      *reinterpret_cast<const float4*>(&Sl[r][c4]);
  }
}

constexpr int kOutRows = 64;  // state rows per output workgroup

// Y = scale (Qtil S_0^T + M delta) for one (chunk, value head, 64 state rows).
// Wave w takes tokens 16 w .. 16 w + 15 against four 16-row tiles; S_0 and
// delta^T rows are staged in LDS (shared by the four waves), the Qtil and M
// rows of the wave's tokens are the A operands in registers.
__global__ __launch_bounds__(256) void gdn_chunk_out_kernel(ChunkParams p) {
  __shared__ __attribute__((aligned(16))) float S0s[kOutRows][kRowPad];
  __shared__ __attribute__((aligned(16))) float Ds[kOutRows][kCPad];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int li = lane & 15;
  const int kq = lane >> 4;
  // Workgroups i and i + 8 (same XCD) take the two row halves of one
  // (chunk, head) unit and share its Qtil and M through that XCD's L2.
  constexpr uint32_t kHalves = kDim / kOutRows;
  static_assert(kHalves == 2, "two row halves per unit");
  const uint32_t unit = (blockIdx.x / 16) * 8 + blockIdx.x % 8;
  const uint32_t half = (blockIdx.x / 8) % 2;
  if (unit >= p.chunks * p.value_heads) {
    return;  // grid padding (whole workgroup)
  }
  const uint32_t cl = unit / p.value_heads;
  const uint32_t h = unit % p.value_heads;
  const uint32_t r0 = half * kOutRows;
  const float* blk = p.ws + ((size_t)cl * p.value_heads + h) * kBlockFloats;

  const uint32_t t0 = (p.chunk0 + cl) * kC;
  const uint32_t n = min((uint32_t)kC, p.tokens - t0);
  // A operands first (global, in flight while S_0 and delta are staged): the
  // query rows of the wave's tokens (a token past the chunk's end reads the
  // first row; its outputs are dropped) and M.
  const uint32_t qt = 16 * wave + li;
  const float* qr = p.query +
                    ((size_t)(t0 + (qt < n ? qt : 0u)) * p.key_heads + h % p.key_heads) * kDim +
                    4 * kq;
  const float* mr = blk + kOffM + (size_t)(16 * wave + li) * kC + 4 * kq;
  float gam[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    gam[r] = blk[kOffGam + 16 * wave + 4 * kq + r];
  }
  float4 qa[8], ma[4];
#pragma unroll
  for (int s4 = 0; s4 < 8; ++s4) {
    qa[s4] = *reinterpret_cast<const float4*>(qr + 16 * s4);
  }
#pragma unroll
  for (int s4 = 0; s4 < 4; ++s4) {
    ma[s4] = *reinterpret_cast<const float4*>(mr + 16 * s4);
  }
#pragma unroll
  for (int it = 0; it < kOutRows * (kDim / 4) / 256; ++it) {
    const int idx = tid + 256 * it;
    const int r = idx >> 5;
    const int c4 = (idx & 31) * 4;
    *reinterpret_cast<float4*>(&S0s[r][c4]) =
      *reinterpret_cast<const float4*>(blk + kOffS0 + (size_t)(r0 + r) * kDim + c4);
  }
#pragma unroll
  for (int it = 0; it < kOutRows * (kC / 4) / 256; ++it) {
    const int idx = tid + 256 * it;
    const int r = idx >> 4;
    const int c4 = (idx & 15) * 4;
    *reinterpret_cast<float4*>(&Ds[r][c4]) =
      *reinterpret_cast<const float4*>(blk + kOffDT + (size_t)(r0 + r) * kC + c4);
  }
  __syncthreads();

  const size_t row_floats = (size_t)p.value_heads * kDim;
  // Rows at or past the chunk's last token fall outside the resource and are
  // dropped.
  const __amdgpu_buffer_rsrc_t out =
    make_buffer_rsrc(p.output + (size_t)t0 * row_floats, n * (uint32_t)row_floats * 4u);
#pragma unroll
  for (int nt = 0; nt < kOutRows / 16; ++nt) {
    const int j = 16 * nt + li;
    float4_v y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s4 = 0; s4 < 8; ++s4) {
      const float4 b = *reinterpret_cast<const float4*>(&S0s[j][16 * s4 + 4 * kq]);
      y = mfma4(qa[s4].x, b.x, y);
      y = mfma4(qa[s4].y, b.y, y);
      y = mfma4(qa[s4].z, b.z, y);
      y = mfma4(qa[s4].w, b.w, y);
    }
    // Row t of Q S_0^T times gamma_t (lane (j, kq) holds rows 4 kq + r).
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      y[r] *= gam[r];
    }
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      const float4 b = *reinterpret_cast<const float4*>(&Ds[j][16 * s4 + 4 * kq]);
      y = mfma4(ma[s4].x, b.x, y);
      y = mfma4(ma[s4].y, b.y, y);
      y = mfma4(ma[s4].z, b.z, y);
      y = mfma4(ma[s4].w, b.w, y);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t t = 16 * wave + 4 * kq + r;
      const uint32_t off = ((t * p.value_heads + h) * kDim + r0 + j) * 4u;
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y[r] * p.scale), out,
                                            (int)off, 0, 0);
    }
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
  return (size_t)slab * a.value_heads * kBlockFloats * sizeof(float);
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
  p.ws = static_cast<float*>(workspace);
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
      gdn_chunk_prep_kernel<true><<<pgrid, kPrepThreads, 0, stream>>>(p);
    } else {
      gdn_chunk_prep_kernel<false><<<pgrid, kPrepThreads, 0, stream>>>(p);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
      return e;
    }
    // One workgroup per (head, 16-row block); the kernel maps the linear index
    // (value_heads * 8 of them, a multiple of the XCD count) to the pair.
    gdn_chunk_scan_kernel<<<a.value_heads * (kDim / kScanRows), kScanThreads, 0, stream>>>(p);
    e = hipGetLastError();
    if (e != hipSuccess) {
      return e;
    }
    // Two workgroups per (chunk, head) unit, padded to a multiple of 16.
    const uint32_t units = p.chunks * a.value_heads;
    gdn_chunk_out_kernel<<<(units + 7) / 8 * 16, 256, 0, stream>>>(p);
    e = hipGetLastError();
    if (e != hipSuccess) {
      return e;
    }
  }
  return hipSuccess;
}

}  // namespace kraken
