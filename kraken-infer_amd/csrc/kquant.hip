// K-quant (GGUF Q4_K / Q5_K / Q6_K) projections, dequantization and device
// argmax for gfx950.
//
// Semantics (reference Metal kernels, mps_backend.mm):
//  * matvec / few-token matmul (q*_k_matvec :295-460, q*_k_matmul
//    :1268-1440): out[t][r] = sum_c w[r][c] x[t][c] in fp32, with w
//    dequantized in fp32 ((d*sc)*q - dmin*m for Q4_K/Q5_K, (d*sc)*(q-32) for
//    Q6_K);
//  * many-token matmul (q*_k_mul_mm_simd :1082-1266): weights and inputs
//    rounded to fp16, fp32 accumulation;
//  * get_row / get_rows (:1448-1540, 1693-1825): dequantized rows, zeros for
//    row ids outside the matrix;
//  * argmax_f32_i32 / argmax_prob_f32_i32 (:2681-2779) and the top1/argmax
//    matvecs (:466-740, 1546-1690): first index of the maximum (NaN never
//    wins), probability 1 / sum exp(v - max).
// Block layouts are spelled out in oracle/kquant_oracle.c's header.
//
// Design (wave64):
//  * Every kernel decodes weights in units of one 16-byte quant chunk per lane:
//    8 lanes cover a 256-value block, a lane's chunk holds 32 quants, 16 of
//    each of two sub-blocks (Q4_K/Q5_K) or quarter-halves (Q6_K).  Nibbles are
//    split four at a time with masks on 32-bit words and converted with the
//    byte-to-float conversions; the Q5_K and Q6_K high bits are merged into the
//    same words before conversion.
//  * GEMV (1..8 tokens): a row is spread over 8 * BC lanes (BC blocks at a
//    time), a 64-lane wave holds 64 / (8 BC) rows, so every lane issues one
//    16-byte load per block for the quants; the fp32 input stays in the CU's
//    L1.  Partial sums reduce over the row's lanes with DPP and lane swaps.
//  * Many tokens: the weights are dequantized to fp16 and the inputs rounded to
//    fp16 in two streaming passes, then an fp16 MFMA GEMM (v_mfma_f32_32x32x16_f16,
//    128 x 128 output tile per 4-wave workgroup, 64-deep K steps double-
//    buffered through LDS with XOR-swizzled 16-byte chunks) writes
//    [tokens][rows] in fp32; grids too small for the chip split K into fp32
//    partial planes summed by one more pass.
//  * argmax: per-workgroup (max, first index, sum of exp) candidates, merged by
//    one workgroup; sizes that fit one workgroup take a single launch.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>

#include "context_internal.hpp"
#include "device_common.hpp"

namespace kraken {
namespace {

template <int F>
struct KqFormat;
template <>
struct KqFormat<0> {  // Q4_K
  static constexpr uint32_t kBytes = 144;
};
template <>
struct KqFormat<1> {  // Q5_K
  static constexpr uint32_t kBytes = 176;
};
template <>
struct KqFormat<2> {  // Q6_K
  static constexpr uint32_t kBytes = 210;
};

// A value the compiler must treat as opaque: no instruction is emitted, but an
// expression cannot be fused across it (a multiply into an FMA, or an
// arithmetic result and its fp16 conversion into one v_fma_mix rounding).
__device__ __forceinline__ float rounded(float v) {
  asm("" : "+v"(v));
  return v;
}

__device__ __forceinline__ float half_bits_to_float(uint32_t bits) {
  return static_cast<float>(__builtin_bit_cast(half_t, (uint16_t)(bits & 0xFFFFu)));
}

__device__ __forceinline__ uint32_t byte_of(const u32x4_t& w, uint32_t k) {
  // A 64-bit half and a shift (a select chain over the four words can be
  // turned into an indexed stack copy of the vector).
  const uint64_t half = k < 8 ? (((uint64_t)w.y << 32) | w.x) : (((uint64_t)w.w << 32) | w.z);
  return (uint32_t)(half >> (8u * (k & 7u))) & 0xFFu;
}

// The 6-bit scale and min of sub-block j from the 12 scale bytes held in
// header bytes 4..15 (mps_backend.mm:284-293).
__device__ __forceinline__ void scale_min(const u32x4_t& hdr, uint32_t j, uint32_t& sc,
                                          uint32_t& m) {
  if (j < 4) {
    sc = byte_of(hdr, 4 + j) & 63u;
    m = byte_of(hdr, 8 + j) & 63u;
  } else {
    sc = (byte_of(hdr, 12 + j - 4) & 0xFu) | ((byte_of(hdr, 4 + j - 4) >> 6) << 4);
    m = (byte_of(hdr, 12 + j - 4) >> 4) | ((byte_of(hdr, 4 + j) >> 6) << 4);
  }
}

// Four bytes of a word as floats (the compiler selects v_cvt_f32_ubyte0..3).
__device__ __forceinline__ void bytes_to_float(uint32_t w, float* out) {
  out[0] = (float)(w & 0xFFu);
  out[1] = (float)((w >> 8) & 0xFFu);
  out[2] = (float)((w >> 16) & 0xFFu);
  out[3] = (float)(w >> 24);
}

// A 16-byte (or 4-byte, 2-byte) load, with the nontemporal hint when the data
// is read once (the GEMVs stream each weight once; the GEMM re-reads a weight
// tile for every token tile and keeps it cached).
template <bool kNt, typename T>
__device__ __forceinline__ T load_hint(const T* p) {
  if constexpr (kNt) {
    return __builtin_nontemporal_load(p);
  } else {
    return *p;
  }
}

// The 16 bytes at `offset` (even) from the 4-byte-aligned `base`, read as
// aligned dwords and shifted by the misalignment (0 or 2 bytes), so Q6_K's
// 210-byte blocks need no unaligned access.  An aligned chunk re-reads its
// last dword instead of the one after it, so no byte past the chunk is read.
template <bool kNt = true>
__device__ __forceinline__ u32x4_t load16_even(const uint8_t* base, uint64_t offset) {
  const uint32_t* p = reinterpret_cast<const uint32_t*>(base + (offset & ~(uint64_t)3));
  const uint32_t shift = (uint32_t)(offset & 3u);
  const uint32_t w0 = load_hint<kNt>(p);
  const uint32_t w1 = load_hint<kNt>(p + 1);
  const uint32_t w2 = load_hint<kNt>(p + 2);
  const uint32_t w3 = load_hint<kNt>(p + 3);
  const uint32_t w4 = load_hint<kNt>(p + (shift != 0u ? 4 : 3));
  u32x4_t r;
  r.x = __builtin_amdgcn_alignbyte(w1, w0, shift);
  r.y = __builtin_amdgcn_alignbyte(w2, w1, shift);
  r.z = __builtin_amdgcn_alignbyte(w3, w2, shift);
  r.w = __builtin_amdgcn_alignbyte(w4, w3, shift);
  return r;
}

// The bytes one lane needs of a block's chunk c, loaded before any math: for
// Q4_K/Q5_K the 16-byte header (d, dmin, the 12 scale bytes), the chunk's 16
// nibble bytes and (Q5_K) the 16 fifth-bit bytes of its half; for Q6_K the
// chunk's 16 low-nibble bytes, its 16 high-bit-pair bytes, the 16 scales and d.
struct RawChunk {
  u32x4_t a, b, c;
  uint32_t d;
};

template <int F, bool kNt>
__device__ __forceinline__ RawChunk load_raw(const uint8_t* block, uint32_t c) {
  RawChunk r;
  if constexpr (F == 2) {
    const uint64_t base = (uint64_t)(uintptr_t)block;
    const uint8_t* b0 = reinterpret_cast<const uint8_t*>(base & ~(uint64_t)3);
    const uint64_t mis = base & 3u;
    const uint32_t h = c >> 2;
    const uint32_t half = c & 1u;
    r.a = load16_even<kNt>(b0, mis + 16u * c);                      // ql
    r.b = load16_even<kNt>(b0, mis + 128u + 32u * h + 16u * half);  // qh
    r.c = load16_even<kNt>(b0, mis + 192u);                         // scales
    r.d = load_hint<kNt>(reinterpret_cast<const uint16_t*>(block + 208u));
  } else {
    const uint32_t qs_at = F == 1 ? 48u : 16u;
    r.a = load_hint<kNt>(reinterpret_cast<const u32x4_t*>(block));  // header
    r.b = load_hint<kNt>(reinterpret_cast<const u32x4_t*>(block + qs_at + 16u * c));
    r.c = u32x4_t{0u, 0u, 0u, 0u};
    if constexpr (F == 1) {
      r.c = load_hint<kNt>(reinterpret_cast<const u32x4_t*>(block + 16u + 16u * (c & 1u)));
    }
    r.d = 0u;
  }
  return r;
}

// One lane's share of a block: chunk c (0..7) holds 32 quants, dequantized
// into v0 (block positions p0 .. p0 + 15) and v1 (p1 .. p1 + 15).  With
// kExact the arithmetic is the reference's, operation for operation (no
// contraction), so dequantized rows are bit-identical to the oracle.  load()
// and compute() split decode() so that a kernel can issue the loads of its next
// chunks before it decodes the current ones.
template <int F, bool kExact>
struct ChunkDecoder {
  float v0[16], v1[16];
  uint32_t p0, p1;

  __device__ __forceinline__ void decode(const uint8_t* block, uint32_t c) {
    compute(load_raw<F, true>(block, c), c);
  }

  __device__ __forceinline__ void compute(const RawChunk& r, uint32_t c) {
    if constexpr (F == 2) {
      compute_q6(r, c);
    } else {
      compute_q45(r, c);
    }
  }

  __device__ __forceinline__ static float axpy(float a, float x, float b) {
    if constexpr (kExact) {
      // a * x - b with two roundings, as the reference writes it, and the
      // f32 result kept as such before any later fp16 conversion.
      return rounded(rounded(a * x) - b);
    } else {
      return fmaf(a, x, -b);
    }
  }

  __device__ __forceinline__ void compute_q45(const RawChunk& r, uint32_t c) {
    const u32x4_t& hdr = r.a;
    const u32x4_t& qs = r.b;
    const u32x4_t& qh = r.c;
    const uint32_t s = c >> 1;
    p0 = 64u * s + 16u * (c & 1u);
    p1 = p0 + 32u;
    uint32_t sc0, m0, sc1, m1;
    scale_min(hdr, 2u * s, sc0, m0);
    scale_min(hdr, 2u * s + 1u, sc1, m1);
    const float d = half_bits_to_float(hdr.x);
    const float dmin = half_bits_to_float(hdr.x >> 16);
    float ds0, ms0, ds1, ms1;
    if constexpr (kExact) {
      ds0 = rounded(d * (float)sc0);
      ms0 = rounded(dmin * (float)m0);
      ds1 = rounded(d * (float)sc1);
      ms1 = rounded(dmin * (float)m1);
    } else {
      ds0 = d * (float)sc0;
      ms0 = dmin * (float)m0;
      ds1 = d * (float)sc1;
      ms1 = dmin * (float)m1;
    }
    const uint32_t words[4] = {qs.x, qs.y, qs.z, qs.w};
    const uint32_t hwords[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t lo = words[k] & 0x0F0F0F0Fu;
      uint32_t hi = (words[k] >> 4) & 0x0F0F0F0Fu;
      if constexpr (F == 1) {
        lo |= ((hwords[k] >> (2u * s)) & 0x01010101u) << 4;
        hi |= ((hwords[k] >> (2u * s + 1u)) & 0x01010101u) << 4;
      }
      float ql[4], qhf[4];
      bytes_to_float(lo, ql);
      bytes_to_float(hi, qhf);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v0[4 * k + e] = axpy(ds0, ql[e], ms0);
        v1[4 * k + e] = axpy(ds1, qhf[e], ms1);
      }
    }
  }

  __device__ __forceinline__ void compute_q6(const RawChunk& r, uint32_t c) {
    const u32x4_t& ql = r.a;
    const u32x4_t& qh = r.b;
    const u32x4_t& sc = r.c;
    const uint32_t h = c >> 2;
    const uint32_t c4 = c & 3u;
    const uint32_t g = c4 >> 1;
    const uint32_t half = c4 & 1u;
    const float d = half_bits_to_float(r.d);
    const int s_lo = (int8_t)byte_of(sc, 8u * h + 2u * g + half);
    const int s_hi = (int8_t)byte_of(sc, 8u * h + 4u + 2u * g + half);
    float dl, dh;
    if constexpr (kExact) {
      dl = rounded(d * (float)s_lo);
      dh = rounded(d * (float)s_hi);
    } else {
      dl = d * (float)s_lo;
      dh = d * (float)s_hi;
    }
    p0 = 128u * h + 32u * g + 16u * half;
    p1 = p0 + 64u;
    const uint32_t words[4] = {ql.x, ql.y, ql.z, ql.w};
    const uint32_t hwords[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t lo = (words[k] & 0x0F0F0F0Fu) | (((hwords[k] >> (2u * g)) & 0x03030303u) << 4);
      const uint32_t hi =
        ((words[k] >> 4) & 0x0F0F0F0Fu) | (((hwords[k] >> (2u * g + 4u)) & 0x03030303u) << 4);
      float ql4[4], qh4[4];
      bytes_to_float(lo, ql4);
      bytes_to_float(hi, qh4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // (d * sc) * (q - 32); q - 32 is exact.
        if constexpr (kExact) {
          v0[4 * k + e] = rounded(dl * (ql4[e] - 32.0f));
          v1[4 * k + e] = rounded(dh * (qh4[e] - 32.0f));
        } else {
          v0[4 * k + e] = dl * (ql4[e] - 32.0f);
          v1[4 * k + e] = dh * (qh4[e] - 32.0f);
        }
      }
    }
  }
};

// Sum over an aligned group of R lanes (R = 8, 16, 32 or 64); result in all.
template <int R>
__device__ __forceinline__ float group_sum(float x) {
  x = reduce8_sum(x);
  if constexpr (R >= 16) {
    x += dpp<kDppRowMirror>(x);
  }
  if constexpr (R >= 32) {
    x = xor16_sum(x);
  }
  if constexpr (R >= 64) {
    x = xor32_sum(x);
  }
  return x;
}

struct GemvArgs {
  const uint8_t* weight;
  const float* input;  // [tokens][cols]
  float* output;       // [tokens][rows]
  uint32_t rows, cols, blocks_per_row, tokens;
  uint32_t token_base;  // first token of this launch's group
  uint32_t round_f16;   // weights rounded to fp16 before the products
};

// GEMV over a group of TG tokens (tokens past `tokens` are computed on token
// 0's input and not stored).  One wave per workgroup: rows spread over
// 64 / (8 BC) row slots.
template <int F, int BC, int TG>
__global__ __launch_bounds__(64) void kq_gemv_kernel(GemvArgs a) {
  constexpr int LR = 8 * BC;
  constexpr int RW = 64 / LR;
  const int lane = threadIdx.x;
  const uint32_t row_slot = (uint32_t)(lane / LR);
  const uint32_t row = blockIdx.x * RW + row_slot;
  const bool row_ok = row < a.rows;
  const uint32_t r = row_ok ? row : a.rows - 1u;
  const uint32_t bl = (uint32_t)((lane % LR) / 8);
  const uint32_t c = (uint32_t)(lane & 7);
  const uint8_t* row_ptr = a.weight + (uint64_t)r * a.blocks_per_row * KqFormat<F>::kBytes;
  const float* xin[TG];
#pragma unroll
  for (int t = 0; t < TG; ++t) {
    const uint32_t tok = a.token_base + t;
    xin[t] = a.input + (uint64_t)(tok < a.tokens ? tok : 0u) * a.cols;
  }
  float acc[TG];
#pragma unroll
  for (int t = 0; t < TG; ++t) {
    acc[t] = 0.0f;
  }
  for (uint32_t b = bl; b < a.blocks_per_row; b += BC) {
    ChunkDecoder<F, false> dec;
    dec.decode(row_ptr + (uint64_t)b * KqFormat<F>::kBytes, c);
    if (a.round_f16 != 0u) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        dec.v0[i] = static_cast<float>(static_cast<half_t>(rounded(dec.v0[i])));
        dec.v1[i] = static_cast<float>(static_cast<half_t>(rounded(dec.v1[i])));
      }
    }
#pragma unroll
    for (int t = 0; t < TG; ++t) {
      const float4* x0 = reinterpret_cast<const float4*>(xin[t] + 256u * b + dec.p0);
      const float4* x1 = reinterpret_cast<const float4*>(xin[t] + 256u * b + dec.p1);
      float s = acc[t];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 u = x0[q];
        const float4 v = x1[q];
        s = fmaf(dec.v0[4 * q + 0], u.x, s);
        s = fmaf(dec.v0[4 * q + 1], u.y, s);
        s = fmaf(dec.v0[4 * q + 2], u.z, s);
        s = fmaf(dec.v0[4 * q + 3], u.w, s);
        s = fmaf(dec.v1[4 * q + 0], v.x, s);
        s = fmaf(dec.v1[4 * q + 1], v.y, s);
        s = fmaf(dec.v1[4 * q + 2], v.z, s);
        s = fmaf(dec.v1[4 * q + 3], v.w, s);
      }
      acc[t] = s;
    }
  }
#pragma unroll
  for (int t = 0; t < TG; ++t) {
    const float total = group_sum<LR>(acc[t]);
    const uint32_t tok = a.token_base + t;
    if (row_ok && (lane % LR) == 0 && tok < a.tokens) {
      a.output[(uint64_t)tok * a.rows + row] = total;
    }
  }
}

// One-token GEMV with the decoder layer's neighbouring ops folded in (no
// counterpart kernel in the reference, which runs them as separate ops):
//   XF = 1: the input is RMSNorm(input) * norm_weight (rms_norm_f32_f32_batched,
//           mps_backend.mm:1890-1920), the scale computed by every workgroup
//           from the whole input row;
//   XF = 2: the input is silu(input) * up (silu_mul_f32_in_place, :2620-2629);
//   residual != nullptr: output = residual + W x (add_f32_in_place, :2529-2537);
//           output may be the residual buffer itself (each row's value is read
//           and written by the same lane).
struct FusedGemvArgs {
  const uint8_t* weight;
  const float* input;
  const float* norm_weight;
  const float* up;
  const float* residual;
  float* output;
  uint32_t rows, cols, blocks_per_row;
  float eps;
};

template <int F, int BC, int XF>
__global__ __launch_bounds__(64) void kq_gemv_fused_kernel(FusedGemvArgs a) {
  constexpr int LR = 8 * BC;
  constexpr int RW = 64 / LR;
  const int lane = threadIdx.x;
  const uint32_t row = blockIdx.x * RW + (uint32_t)(lane / LR);
  const bool row_ok = row < a.rows;
  const uint32_t r = row_ok ? row : a.rows - 1u;
  const uint32_t bl = (uint32_t)((lane % LR) / 8);
  const uint32_t c = (uint32_t)(lane & 7);
  const uint8_t* row_ptr = a.weight + (uint64_t)r * a.blocks_per_row * KqFormat<F>::kBytes;
  float scale = 1.0f;
  if constexpr (XF == 1) {
    // cols is a multiple of 256: every lane takes cols / 256 float4s.
    float ss = 0.0f;
    for (uint32_t i = 4u * (uint32_t)lane; i < a.cols; i += 256u) {
      const float4 v = *reinterpret_cast<const float4*>(a.input + i);
      ss = fmaf(v.x, v.x, ss);
      ss = fmaf(v.y, v.y, ss);
      ss = fmaf(v.z, v.z, ss);
      ss = fmaf(v.w, v.w, ss);
    }
    ss = wave_sum(ss);
    scale = 1.0f / sqrtf(ss / (float)a.cols + a.eps);
  }
  // The transformed input at k .. k + 3.
  auto xin = [&](uint32_t k) __attribute__((always_inline)) {
    float4 x = *reinterpret_cast<const float4*>(a.input + k);
    if constexpr (XF == 1) {
      const float4 w = *reinterpret_cast<const float4*>(a.norm_weight + k);
      x = make_float4(x.x * scale * w.x, x.y * scale * w.y, x.z * scale * w.z, x.w * scale * w.w);
    } else if constexpr (XF == 2) {
      const float4 u = *reinterpret_cast<const float4*>(a.up + k);
      x = make_float4((x.x / (1.0f + expf(-x.x))) * u.x, (x.y / (1.0f + expf(-x.y))) * u.y,
                      (x.z / (1.0f + expf(-x.z))) * u.z, (x.w / (1.0f + expf(-x.w))) * u.w);
    }
    return x;
  };
  float s = 0.0f;
  for (uint32_t b = bl; b < a.blocks_per_row; b += BC) {
    ChunkDecoder<F, false> dec;
    dec.decode(row_ptr + (uint64_t)b * KqFormat<F>::kBytes, c);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 u = xin(256u * b + dec.p0 + 4u * q);
      const float4 v = xin(256u * b + dec.p1 + 4u * q);
      s = fmaf(dec.v0[4 * q + 0], u.x, s);
      s = fmaf(dec.v0[4 * q + 1], u.y, s);
      s = fmaf(dec.v0[4 * q + 2], u.z, s);
      s = fmaf(dec.v0[4 * q + 3], u.w, s);
      s = fmaf(dec.v1[4 * q + 0], v.x, s);
      s = fmaf(dec.v1[4 * q + 1], v.y, s);
      s = fmaf(dec.v1[4 * q + 2], v.z, s);
      s = fmaf(dec.v1[4 * q + 3], v.w, s);
    }
  }
  const float total = group_sum<LR>(s);
  if (row_ok && (lane % LR) == 0) {
    a.output[row] = a.residual != nullptr ? a.residual[row] + total : total;
  }
}

// ---------------------------------------------------------------------------
// Input-stationary one-token GEMV (the decode path's matvecs, plain or with
// the fused RMSNorm / SwiGLU / residual of kq_gemv_fused_kernel).  A row's
// P = 8 * blocks_per_row quant chunks are spread over LR lanes (PPL chunks per
// lane), so each lane needs the same 32 * PPL input values for every row: the
// workgroup computes the (transformed) input once into registers and then
// streams rows, U of them per lane in flight, each contributing one 16-byte
// chunk load per lane.  Grid-stride over rows, so a few workgroups per CU serve
// any row count and the input transform is paid once per workgroup.
// ---------------------------------------------------------------------------

// Block positions of chunk c's two 16-value halves (the decoders' p0 and p1).
template <int F>
__device__ __forceinline__ void chunk_positions(uint32_t c, uint32_t& p0, uint32_t& p1) {
  if constexpr (F == 2) {
    p0 = 128u * (c >> 2) + 32u * ((c & 3u) >> 1) + 16u * (c & 1u);
    p1 = p0 + 64u;
  } else {
    p0 = 64u * (c >> 1) + 16u * (c & 1u);
    p1 = p0 + 32u;
  }
}

template <int F>
__device__ __forceinline__ RawChunk load_chunk(const uint8_t* block, uint32_t c) {
  return load_raw<F, true>(block, c);
}

// sum over the chunk's 32 values of w * x, x[0..15] at p0 and x[16..31] at p1;
// the weights as the GEMV computes them (fma(d * sc, q, -dmin * m), (d * sc) * (q - 32)).
template <int F>
__device__ __forceinline__ float chunk_dot(const RawChunk& r, uint32_t c, const float* x,
                                           float acc) {
  const uint32_t words[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
  if constexpr (F == 2) {
    const uint32_t g = (c & 3u) >> 1;
    const uint32_t h = c >> 2;
    const uint32_t half = c & 1u;
    const int s_lo = (int8_t)byte_of(r.c, 8u * h + 2u * g + half);
    const int s_hi = (int8_t)byte_of(r.c, 8u * h + 4u + 2u * g + half);
    const float d = half_bits_to_float(r.d);
    const float dl = d * (float)s_lo;
    const float dh = d * (float)s_hi;
    const uint32_t lw[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t lo = (lw[k] & 0x0F0F0F0Fu) | (((words[k] >> (2u * g)) & 0x03030303u) << 4);
      const uint32_t hi =
        ((lw[k] >> 4) & 0x0F0F0F0Fu) | (((words[k] >> (2u * g + 4u)) & 0x03030303u) << 4);
      float ql[4], qh[4];
      bytes_to_float(lo, ql);
      bytes_to_float(hi, qh);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc = fmaf(dl * (ql[e] - 32.0f), x[4 * k + e], acc);
        acc = fmaf(dh * (qh[e] - 32.0f), x[16 + 4 * k + e], acc);
      }
    }
  } else {
    const uint32_t sb = c >> 1;
    uint32_t sc0, m0, sc1, m1;
    scale_min(r.a, 2u * sb, sc0, m0);
    scale_min(r.a, 2u * sb + 1u, sc1, m1);
    const float d = half_bits_to_float(r.a.x);
    const float dmin = half_bits_to_float(r.a.x >> 16);
    const float ds0 = d * (float)sc0, ms0 = dmin * (float)m0;
    const float ds1 = d * (float)sc1, ms1 = dmin * (float)m1;
    const uint32_t hw[4] = {r.c.x, r.c.y, r.c.z, r.c.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t lo = words[k] & 0x0F0F0F0Fu;
      uint32_t hi = (words[k] >> 4) & 0x0F0F0F0Fu;
      if constexpr (F == 1) {
        lo |= ((hw[k] >> (2u * sb)) & 0x01010101u) << 4;
        hi |= ((hw[k] >> (2u * sb + 1u)) & 0x01010101u) << 4;
      }
      float ql[4], qh[4];
      bytes_to_float(lo, ql);
      bytes_to_float(hi, qh);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc = fmaf(fmaf(ds0, ql[e], -ms0), x[4 * k + e], acc);
        acc = fmaf(fmaf(ds1, qh[e], -ms1), x[16 + 4 * k + e], acc);
      }
    }
  }
  return acc;
}

// chunk_dot with each sub-block's affine part taken out of the sum: a
// sub-block of 16 weights w = a * q + b (a = d * scale; b = -dmin * min, or
// -32 * a for Q6_K) against inputs x gives a * sum(q x) + b * sum(x), and the
// input sums xs_lo (x[0..15]) and xs_hi (x[16..31]) are fixed for a lane
// across rows.  A weight then costs a byte conversion and one FMA; the
// rounding is that of two fp32 sums of 16 terms, well inside the GEMV's
// accumulation bound.
template <int F>
__device__ __forceinline__ float chunk_dot_split(const RawChunk& r, uint32_t c, const float* x,
                                                 float xs_lo, float xs_hi, float acc) {
  const uint32_t words[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
  float s_lo = 0.0f, s_hi = 0.0f;
  float a_lo, a_hi, b_lo, b_hi;
  if constexpr (F == 2) {
    const uint32_t g = (c & 3u) >> 1;
    const uint32_t h = c >> 2;
    const uint32_t half = c & 1u;
    const int sc_lo = (int8_t)byte_of(r.c, 8u * h + 2u * g + half);
    const int sc_hi = (int8_t)byte_of(r.c, 8u * h + 4u + 2u * g + half);
    const float d = half_bits_to_float(r.d);
    a_lo = d * (float)sc_lo;
    a_hi = d * (float)sc_hi;
    b_lo = -32.0f * a_lo;
    b_hi = -32.0f * a_hi;
    const uint32_t lw[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t lo = (lw[k] & 0x0F0F0F0Fu) | (((words[k] >> (2u * g)) & 0x03030303u) << 4);
      const uint32_t hi =
        ((lw[k] >> 4) & 0x0F0F0F0Fu) | (((words[k] >> (2u * g + 4u)) & 0x03030303u) << 4);
      float ql[4], qh[4];
      bytes_to_float(lo, ql);
      bytes_to_float(hi, qh);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s_lo = fmaf(ql[e], x[4 * k + e], s_lo);
        s_hi = fmaf(qh[e], x[16 + 4 * k + e], s_hi);
      }
    }
  } else {
    const uint32_t sb = c >> 1;
    uint32_t sc0, m0, sc1, m1;
    scale_min(r.a, 2u * sb, sc0, m0);
    scale_min(r.a, 2u * sb + 1u, sc1, m1);
    const float d = half_bits_to_float(r.a.x);
    const float dmin = half_bits_to_float(r.a.x >> 16);
    a_lo = d * (float)sc0;
    a_hi = d * (float)sc1;
    b_lo = -(dmin * (float)m0);
    b_hi = -(dmin * (float)m1);
    const uint32_t hw[4] = {r.c.x, r.c.y, r.c.z, r.c.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t lo = words[k] & 0x0F0F0F0Fu;
      uint32_t hi = (words[k] >> 4) & 0x0F0F0F0Fu;
      if constexpr (F == 1) {
        lo |= ((hw[k] >> (2u * sb)) & 0x01010101u) << 4;
        hi |= ((hw[k] >> (2u * sb + 1u)) & 0x01010101u) << 4;
      }
      float ql[4], qh[4];
      bytes_to_float(lo, ql);
      bytes_to_float(hi, qh);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s_lo = fmaf(ql[e], x[4 * k + e], s_lo);
        s_hi = fmaf(qh[e], x[16 + 4 * k + e], s_hi);
      }
    }
  }
  acc = fmaf(a_lo, s_lo, acc);
  acc = fmaf(b_lo, xs_lo, acc);
  acc = fmaf(a_hi, s_hi, acc);
  return fmaf(b_hi, xs_hi, acc);
}

constexpr int kXsWaves = 4;
constexpr int kXsMaxMatrices = 4;
constexpr int kXsMaxCols = 4096;  // 16 blocks per row

// Up to four weight matrices that read the same input (the projections of one
// normed hidden state): each has its format, rows, output and optional
// residual; the workgroups of matrix m are [wg_begin[m], wg_begin[m + 1]).
struct MultiGemvArgs {
  const uint8_t* weight[kXsMaxMatrices];
  float* output[kXsMaxMatrices];
  const float* residual[kXsMaxMatrices];
  uint32_t rows[kXsMaxMatrices];
  int32_t format[kXsMaxMatrices];
  uint32_t wg_begin[kXsMaxMatrices + 1];
  uint32_t count;
  const float* input;
  const float* norm_weight;  // input = RMSNorm(input) * norm_weight
  const float* up;           // input = silu(input) * up
  uint32_t cols, blocks_per_row;
  float eps;
  // Head-normed input (XF = 3): per head of 128 values, input *
  // rsqrt(mean(input^2) + eps) * gate_factor[c].
  const float* gate_factor;
  // Conv epilogue of matrix 0 (conv_pool set): row r is conv channel r of one
  // sequence, whose state [rows][3] sits at conv_pool + *conv_offset; the row's
  // value x becomes silu(sum_j state[r][j] w[r][j] + x w[r][3]) and the state
  // shifts in x (conv_weights [rows][4]).
  float* conv_pool;
  const uint64_t* conv_offset;
  uint64_t conv_pool_elems;
  const float* conv_weights;
};

// The depthwise conv of one channel (kernel 4) over its state window and the
// new value x, with SiLU, and the state shifted (the conv prologue's
// arithmetic in the gated delta net kernels).
struct ConvRow {
  float win[3], w[4];
};
__device__ __forceinline__ ConvRow conv_row_load(const float* state_row, const float* weights) {
  ConvRow c;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    c.win[j] = state_row[j];
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    c.w[j] = weights[j];
  }
  return c;
}
__device__ __forceinline__ float conv_row_apply(const ConvRow& c, float x, float* state_row) {
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    acc = fmaf(c.win[j], c.w[j], acc);
  }
  acc = fmaf(x, c.w[3], acc);
  state_row[0] = c.win[1];
  state_row[1] = c.win[2];
  state_row[2] = x;
  return acc / (1.0f + expf(-acc));
}

// The raw weight bytes one lane holds for its rows of one trip slot.  Q4_K and
// Q5_K (16-byte aligned blocks): the lane's own chunk loads.  Q6_K with
// staging (internal format 3): the wave's rows are one contiguous byte span,
// read as 16-byte aligned pieces (piece k = lane + 64 j) and taken apart in
// LDS, since the 210-byte blocks put a lane's fields at 2-byte alignment and
// loading them per lane takes sixteen dword loads over a few dozen cache lines.
// A wave's span holds RW * blocks_per_row <= 8 * PPL blocks (LR lanes per row,
// 8 chunks per block), so 2 * PPL pieces per lane cover it with the 15-byte
// lead: 16 * 64 * 2 * PPL bytes >= 8 * PPL * 210 + 15.
constexpr int kSpanPiecesMax = 4;
template <int PPL>
constexpr int kSpanPieces = 2 * PPL;
template <int F, int PPL>
struct LaneRaw {
  RawChunk c[PPL];
};
template <int PPL>
struct LaneRaw<3, PPL> {
  u32x4_t v[kSpanPieces<PPL>];
};

// The 16 bytes at byte offset o (even) of an LDS word array (as load16_even).
__device__ __forceinline__ u32x4_t lds_load16_even(const uint32_t* words, uint32_t o) {
  const uint32_t w = o >> 2;
  const uint32_t shift = o & 3u;
  const uint32_t w0 = words[w];
  const uint32_t w1 = words[w + 1];
  const uint32_t w2 = words[w + 2];
  const uint32_t w3 = words[w + 3];
  const uint32_t w4 = words[w + (shift != 0u ? 4 : 3)];
  u32x4_t r;
  r.x = __builtin_amdgcn_alignbyte(w1, w0, shift);
  r.y = __builtin_amdgcn_alignbyte(w2, w1, shift);
  r.z = __builtin_amdgcn_alignbyte(w3, w2, shift);
  r.w = __builtin_amdgcn_alignbyte(w4, w3, shift);
  return r;
}

// silu(x) * u with the hardware exp2 and reciprocal (about 2 ulp).
__device__ __forceinline__ float silu_mul_fast(float x, float u) {
  const float e = __builtin_amdgcn_exp2f(-x * 1.4426950408889634f);
  return x * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

// The rows of one matrix for one workgroup (local index wl of nwg).  kConv:
// the launch carries the conv epilogue of matrix 0 (a template option, so the
// other launches keep its registers).
template <int F, int LR, int PPL, int XF, int U, bool kConv>
__device__ __forceinline__ void xs_matrix(const MultiGemvArgs& a, int m, uint32_t wl,
                                          uint32_t nwg, float* s_x, float* s_red,
                                          u32x4_t* s_span) {
  constexpr int FB = F == 3 ? 2 : F;  // block format (3: Q6_K read as spans)
  constexpr bool kSpan = F == 3;
  constexpr int RW = 64 / LR;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const uint32_t li = (uint32_t)(lane % LR);
  const uint32_t slot = (uint32_t)(lane / LR);
  const uint32_t positions = 8u * a.blocks_per_row;
  const uint32_t rows = a.rows[m];
  const uint8_t* weight = a.weight[m];
  uint32_t pb[PPL], pc[PPL];
  bool pv[PPL];
#pragma unroll
  for (int i = 0; i < PPL; ++i) {
    const uint32_t pos = li + (uint32_t)LR * (uint32_t)i;
    pv[i] = pos < positions;
    const uint32_t pq = pv[i] ? pos : 0u;
    pb[i] = pq >> 3;
    pc[i] = pq & 7u;
  }
  const uint32_t row_bytes = a.blocks_per_row * KqFormat<FB>::kBytes;
  const uint32_t stride = nwg * (uint32_t)(kXsWaves * RW);
  // Span layout: the wave's RW rows from row `first` start `shift` bytes into
  // the 16-byte piece at span_base(first); pieces at or past the matrix end
  // (rows * row_bytes, a multiple of 16 for format 3) read as zeros.
  const uint64_t matrix_bytes = (uint64_t)rows * row_bytes;
  const uint32_t span_pieces = (15u + (uint32_t)RW * row_bytes + 15u) >> 4;
  auto load_rows = [&](uint32_t r0, LaneRaw<F, PPL> (&raw)[U]) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if constexpr (kSpan) {
        const uint64_t start = (uint64_t)(r0 + (uint32_t)u * stride) * row_bytes;
        const uint64_t base = start & ~(uint64_t)15;
#pragma unroll
        for (int j = 0; j < kSpanPieces<PPL>; ++j) {
          const uint32_t k = (uint32_t)lane + 64u * (uint32_t)j;
          const uint64_t at = base + 16u * k;
          raw[u].v[j] = u32x4_t{0u, 0u, 0u, 0u};
          if (k < span_pieces && at < matrix_bytes) {
            raw[u].v[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(weight + at));
          }
        }
      } else {
        const uint32_t row = r0 + (uint32_t)u * stride + slot;
        const uint32_t rr = row < rows ? row : rows - 1u;
        const uint8_t* rp = weight + (uint64_t)rr * row_bytes;
#pragma unroll
        for (int i = 0; i < PPL; ++i) {
          raw[u].c[i] = load_chunk<FB>(rp + pb[i] * KqFormat<FB>::kBytes, pc[i]);
        }
      }
    }
  };
  // This lane's chunk i of its row in trip slot (r0, u), from the lane's raw
  // bytes (format 3: through this wave's LDS span buffer).
  u32x4_t* span_lds = s_span + wave * (kSpanPiecesMax * 64);
  auto stage_span = [&](const LaneRaw<F, PPL>& raw) __attribute__((always_inline)) {
    if constexpr (kSpan) {
      // Every lane writes its pieces (another lane's chunk may lie in them).
#pragma unroll
      for (int j = 0; j < kSpanPieces<PPL>; ++j) {
        span_lds[lane + 64 * j] = raw.v[j];
      }
    }
  };
  auto chunk_of = [&](const LaneRaw<F, PPL>& raw, uint32_t r0, int u, int i)
      __attribute__((always_inline)) -> RawChunk {
    if constexpr (kSpan) {
      const uint32_t shift = (uint32_t)(((uint64_t)(r0 + (uint32_t)u * stride) * row_bytes) & 15u);
      const uint32_t o = shift + slot * row_bytes + pb[i] * KqFormat<2>::kBytes;
      const uint32_t c = pc[i];
      const uint32_t* words = reinterpret_cast<const uint32_t*>(span_lds);
      RawChunk r;
      r.a = lds_load16_even(words, o + 16u * c);                                  // ql
      r.b = lds_load16_even(words, o + 128u + 32u * (c >> 2) + 16u * (c & 1u));   // qh
      r.c = lds_load16_even(words, o + 192u);                                     // scales
      r.d = reinterpret_cast<const uint16_t*>(span_lds)[(o + 208u) >> 1];
      return r;
    } else {
      return raw.c[i];
    }
  };
  uint32_t r0 = (wl * kXsWaves + (uint32_t)wave) * RW;

  // The transformed input is computed once per workgroup into LDS (each
  // thread takes up to four float4s of it; the RMSNorm's sum of squares is a
  // workgroup sum), then each lane reads the 32 * PPL values its chunks need
  // (zeros at absent positions).  Reading it per row group from global memory
  // instead would move several times the weight bytes through the caches.
  // The input loads (and the norm weights or the up half) go out first and
  // the first rows' weight loads right behind them: loads complete in issue
  // order, so the transform then waits only for the input while the weights
  // stream in.
  constexpr int kVecPerThread = kXsMaxCols / 4 / (64 * kXsWaves);
  const uint32_t nvec = a.cols / 4u;
  float4 xv[kVecPerThread], yv[kVecPerThread];
#pragma unroll
  for (int k = 0; k < kVecPerThread; ++k) {
    const uint32_t vi = threadIdx.x + (uint32_t)(64 * kXsWaves * k);
    xv[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    yv[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (vi < nvec) {
      xv[k] = reinterpret_cast<const float4*>(a.input)[vi];
      if constexpr (XF == 1) {
        yv[k] = reinterpret_cast<const float4*>(a.norm_weight)[vi];
      } else if constexpr (XF == 2) {
        yv[k] = reinterpret_cast<const float4*>(a.up)[vi];
      } else if constexpr (XF == 3) {
        yv[k] = reinterpret_cast<const float4*>(a.gate_factor)[vi];
      }
    }
  }
  // Matrix 0 with the conv epilogue: this lane's first-trip rows' conv state
  // and weights load with the input (trip slots beyond U load when reached).
  const bool conv = kConv && m == 0;
  float* conv_state = nullptr;
  ConvRow crow[kConv ? U : 1];
  if (conv) {
    const uint64_t coff = *a.conv_offset;
    if (coff <= a.conv_pool_elems && a.conv_pool_elems - coff >= (uint64_t)rows * 3u) {
      conv_state = a.conv_pool + coff;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t row = r0 + (uint32_t)u * stride + slot;
        if (li == 0 && row < rows) {
          crow[u] = conv_row_load(conv_state + (size_t)row * 3u, a.conv_weights + (size_t)row * 4u);
        }
      }
    }
  }
  asm volatile("" ::: "memory");
  LaneRaw<F, PPL> cur[U];
  load_rows(r0 < rows ? r0 : 0u, cur);
  {
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < kVecPerThread; ++k) {
      float4 v = xv[k];
      if constexpr (XF == 2) {
        const float4 u = yv[k];
        v = make_float4(silu_mul_fast(v.x, u.x), silu_mul_fast(v.y, u.y),
                        silu_mul_fast(v.z, u.z), silu_mul_fast(v.w, u.w));
      }
      if constexpr (XF == 1) {
        ss = fmaf(v.x, v.x, ss);
        ss = fmaf(v.y, v.y, ss);
        ss = fmaf(v.z, v.z, ss);
        ss = fmaf(v.w, v.w, ss);
      }
      if constexpr (XF == 3) {
        // The head's 32 float4s are held by 32 consecutive lanes.
        float hs = fmaf(v.x, v.x, fmaf(v.y, v.y, fmaf(v.z, v.z, v.w * v.w)));
        hs = group_sum<32>(hs);
        const float hscale = 1.0f / sqrtf(hs / 128.0f + a.eps);
        const float4 g = yv[k];
        v = make_float4(v.x * hscale * g.x, v.y * hscale * g.y, v.z * hscale * g.z,
                        v.w * hscale * g.w);
      }
      xv[k] = v;
    }
    if constexpr (XF == 1) {
      ss = group_sum<64>(ss);
      if (lane == 0) {
        s_red[wave] = ss;
      }
      __syncthreads();
      ss = 0.0f;
#pragma unroll
      for (int w = 0; w < kXsWaves; ++w) {
        ss += s_red[w];
      }
      const float scale = 1.0f / sqrtf(ss / (float)a.cols + a.eps);
#pragma unroll
      for (int k = 0; k < kVecPerThread; ++k) {
        const float4 w = yv[k];
        xv[k] = make_float4(xv[k].x * scale * w.x, xv[k].y * scale * w.y,
                            xv[k].z * scale * w.z, xv[k].w * scale * w.w);
      }
    }
#pragma unroll
    for (int k = 0; k < kVecPerThread; ++k) {
      const uint32_t vi = threadIdx.x + (uint32_t)(64 * kXsWaves * k);
      if (vi < nvec) {
        reinterpret_cast<float4*>(s_x)[vi] = xv[k];
      }
    }
    __syncthreads();
  }
  float x[PPL][32];
#pragma unroll
  for (int i = 0; i < PPL; ++i) {
    uint32_t p0, p1;
    chunk_positions<FB>(pc[i], p0, p1);
#pragma unroll
    for (int half_i = 0; half_i < 2; ++half_i) {
      const uint32_t k0 = 256u * pb[i] + (half_i == 0 ? p0 : p1);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 v = *reinterpret_cast<const float4*>(s_x + k0 + 4u * q);
        const bool ok = pv[i];
        x[i][16 * half_i + 4 * q + 0] = ok ? v.x : 0.0f;
        x[i][16 * half_i + 4 * q + 1] = ok ? v.y : 0.0f;
        x[i][16 * half_i + 4 * q + 2] = ok ? v.z : 0.0f;
        x[i][16 * half_i + 4 * q + 3] = ok ? v.w : 0.0f;
      }
    }
  }
  float xs_lo[PPL], xs_hi[PPL];
#pragma unroll
  for (int i = 0; i < PPL; ++i) {
    xs_lo[i] = 0.0f;
    xs_hi[i] = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      xs_lo[i] += x[i][e];
      xs_hi[i] += x[i][16 + e];
    }
  }
  const float* residual = a.residual[m];
  float* output = a.output[m];
  // Every lane of the wave runs the same trips, so the row reductions see all
  // lanes; the next trip's loads are issued before this trip's math.
  for (; r0 < rows; r0 += (uint32_t)U * stride) {
    const uint32_t nr0 = r0 + (uint32_t)U * stride;
    LaneRaw<F, PPL> nxt[U];
    if (U > 1 && nr0 < rows) {
      load_rows(nr0, nxt);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t row = r0 + (uint32_t)u * stride + slot;
      stage_span(cur[u]);
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < PPL; ++i) {
        if (pv[i]) {
          acc = chunk_dot_split<FB>(chunk_of(cur[u], r0, u, i), pc[i], x[i], xs_lo[i], xs_hi[i],
                                    acc);
        }
      }
      const float total = group_sum<LR>(acc);
      if (li == 0 && row < rows) {
        float value = residual != nullptr ? residual[row] + total : total;
        if (conv) {
          if (conv_state == nullptr) {
            continue;  // offset outside the pool: the sequence is skipped
          }
          if (r0 != (wl * kXsWaves + (uint32_t)wave) * RW) {
            crow[u] = conv_row_load(conv_state + (size_t)row * 3u,
                                    a.conv_weights + (size_t)row * 4u);
          }
          value = conv_row_apply(crow[u], value, conv_state + (size_t)row * 3u);
        }
        output[row] = value;
      }
    }
    if (U > 1) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        cur[u] = nxt[u];
      }
    } else if (nr0 < rows) {
      load_rows(nr0, cur);
    }
  }
}

// Four workgroups per CU must be resident for the kXsMaxWorkgroups launches
// (one chunk per lane: at most 128 VGPRs, four waves per SIMD).
template <int LR, int PPL, int XF, int U, bool kConv = false>
__global__ __launch_bounds__(64 * kXsWaves)
__attribute__((amdgpu_waves_per_eu(PPL == 1 ? 4 : 1)))
void kq_gemv_xs_kernel(MultiGemvArgs a) {
  __shared__ __attribute__((aligned(16))) float s_x[kXsMaxCols];
  __shared__ float s_red[kXsWaves];
  __shared__ u32x4_t s_span[kXsWaves * kSpanPiecesMax * 64];
  int m = 0;
#pragma unroll
  for (int k = 1; k < kXsMaxMatrices; ++k) {
    m += (k < (int)a.count && blockIdx.x >= a.wg_begin[k]) ? 1 : 0;
  }
  const uint32_t wl = blockIdx.x - a.wg_begin[m];
  const uint32_t nwg = a.wg_begin[m + 1] - a.wg_begin[m];
  switch (a.format[m]) {
    case 0:
      xs_matrix<0, LR, PPL, XF, U, kConv>(a, m, wl, nwg, s_x, s_red, s_span);
      break;
    case 1:
      xs_matrix<1, LR, PPL, XF, U, kConv>(a, m, wl, nwg, s_x, s_red, s_span);
      break;
    case 2:
      xs_matrix<2, LR, PPL, XF, U, kConv>(a, m, wl, nwg, s_x, s_red, s_span);
      break;
    default:
      xs_matrix<3, LR, PPL, XF, U, kConv>(a, m, wl, nwg, s_x, s_red, s_span);
      break;
  }
}

// Dequantized rows (get_row / get_rows): one lane per 16-byte chunk, exact
// reference arithmetic.  Row ids outside [0, rows) give zeros.
template <int F>
__global__ __launch_bounds__(256) void kq_dequant_rows_kernel(const uint8_t* weight,
                                                              const int32_t* row_ids,
                                                              uint32_t fixed_row, uint32_t rows,
                                                              uint32_t tokens,
                                                              uint32_t blocks_per_row,
                                                              float* output) {
  const uint64_t id = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  const uint64_t per_token = (uint64_t)blocks_per_row * 8u;
  if (id >= per_token * tokens) {
    return;
  }
  const uint32_t token = (uint32_t)(id / per_token);
  const uint32_t within = (uint32_t)(id % per_token);
  const uint32_t b = within / 8u;
  const uint32_t c = within % 8u;
  float* out = output + (uint64_t)token * blocks_per_row * 256u + 256u * b;
  const int64_t row = row_ids != nullptr ? (int64_t)row_ids[token] : (int64_t)fixed_row;
  ChunkDecoder<F, true> dec;
  if (row < 0 || row >= (int64_t)rows) {
    // Positions of this chunk's values, without touching the weights.
    dec.p0 = F == 2 ? 128u * (c >> 2) + 32u * ((c & 3u) >> 1) + 16u * (c & 1u)
                    : 64u * (c >> 1) + 16u * (c & 1u);
    dec.p1 = dec.p0 + (F == 2 ? 64u : 32u);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      dec.v0[j] = 0.0f;
      dec.v1[j] = 0.0f;
    }
  } else {
    dec.decode(weight + ((uint64_t)row * blocks_per_row + b) * KqFormat<F>::kBytes, c);
  }
  float4* o0 = reinterpret_cast<float4*>(out + dec.p0);
  float4* o1 = reinterpret_cast<float4*>(out + dec.p1);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    o0[q] = make_float4(dec.v0[4 * q], dec.v0[4 * q + 1], dec.v0[4 * q + 2], dec.v0[4 * q + 3]);
    o1[q] = make_float4(dec.v1[4 * q], dec.v1[4 * q + 1], dec.v1[4 * q + 2], dec.v1[4 * q + 3]);
  }
}

// Eight f32 values rounded to fp16 (RNE), group i of in -> out.
__device__ __forceinline__ void f32_to_f16_8(const float* in, half_t* out, uint64_t i) {
  const float4 a = reinterpret_cast<const float4*>(in)[2 * i];
  const float4 b = reinterpret_cast<const float4*>(in)[2 * i + 1];
  const half8_t h = {static_cast<half_t>(a.x), static_cast<half_t>(a.y), static_cast<half_t>(a.z),
                     static_cast<half_t>(a.w), static_cast<half_t>(b.x), static_cast<half_t>(b.y),
                     static_cast<half_t>(b.z), static_cast<half_t>(b.w)};
  __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, h), reinterpret_cast<u32x4_t*>(out) + i);
}

// The same for silu(in) * up, with silu_mul_f32_in_place's arithmetic (the
// f32 product, then one rounding to fp16).
__device__ __forceinline__ void f32_swiglu_to_f16_8(const float* in, const float* up,
                                                    half_t* out, uint64_t i) {
  // No contraction into the inlined expf: the same bits as binary_kernel's
  // silu_mul wherever either is inlined.
#pragma clang fp contract(off)
  const float4 a = reinterpret_cast<const float4*>(in)[2 * i];
  const float4 b = reinterpret_cast<const float4*>(in)[2 * i + 1];
  const float4 ua = reinterpret_cast<const float4*>(up)[2 * i];
  const float4 ub = reinterpret_cast<const float4*>(up)[2 * i + 1];
  const float g[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  const float u[8] = {ua.x, ua.y, ua.z, ua.w, ub.x, ub.y, ub.z, ub.w};
  half8_t h;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    // The f32 product kept as such: the compiler would otherwise fuse the
    // multiply and the fp16 conversion into one v_fma_mix (one rounding).
    h[j] = static_cast<half_t>(rounded((g[j] / (1.0f + expf(-g[j]))) * u[j]));
  }
  __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, h), reinterpret_cast<u32x4_t*>(out) + i);
}

// The two-pass GEMM's first pass, one launch: workgroups [0, convert_blocks)
// round the f32 inputs to fp16 (n8 groups of eight), the rest dequantize the
// weights and round them to fp16 (RNE), [rows][cols].
template <int F, int kCpt>
__global__ __launch_bounds__(256) void kq_dequant_f16_kernel(const uint8_t* weight, uint32_t rows,
                                                             uint32_t blocks_per_row,
                                                             half_t* out, const float* xin,
                                                             half_t* x16, uint64_t n8,
                                                             uint32_t convert_blocks,
                                                             const float* up) {
  if (blockIdx.x < convert_blocks) {
    // kCpt groups of eight per thread, the workgroup's 256 * kCpt groups contiguous.
#pragma unroll
    for (int j = 0; j < kCpt; ++j) {
      const uint64_t i = (uint64_t)blockIdx.x * (256u * kCpt) + 256u * j + threadIdx.x;
      if (i < n8) {
        if (up != nullptr) {
          f32_swiglu_to_f16_8(xin, up, x16, i);
        } else {
          f32_to_f16_8(xin, x16, i);
        }
      }
    }
    return;
  }
  // The workgroup's 32 blocks are decoded into LDS and written out as one
  // contiguous 16 KB run: a lane's own values land in 32-byte pieces spread
  // over its block, so storing them directly touched four times the cache
  // lines per store instruction.
  __shared__ __attribute__((aligned(16))) half_t s_out[32 * 256];
  const uint64_t first_blk = (uint64_t)(blockIdx.x - convert_blocks) * 32u;
  const uint64_t id = first_blk * 8u + threadIdx.x;
  const uint64_t total_blocks = (uint64_t)rows * blocks_per_row;
  const uint32_t lb = threadIdx.x / 8u;  // block within the workgroup
  const uint32_t c = threadIdx.x % 8u;
  if (id < total_blocks * 8u) {
    ChunkDecoder<F, true> dec;
    dec.decode(weight + (first_blk + lb) * KqFormat<F>::kBytes, c);
    half_t* o = s_out + lb * 256u;
#pragma unroll
    for (int half_i = 0; half_i < 2; ++half_i) {
      half8_t h0, h1;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        h0[j] = static_cast<half_t>(dec.v0[8 * half_i + j]);
        h1[j] = static_cast<half_t>(dec.v1[8 * half_i + j]);
      }
      *reinterpret_cast<half8_t*>(o + dec.p0 + 8 * half_i) = h0;
      *reinterpret_cast<half8_t*>(o + dec.p1 + 8 * half_i) = h1;
    }
  }
  __syncthreads();
  const uint64_t valid = total_blocks - first_blk < 32u ? total_blocks - first_blk : 32u;
  half8_t* dst = reinterpret_cast<half8_t*>(out + first_blk * 256u);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t piece = (uint32_t)j * 256u + threadIdx.x;  // 16-byte piece, 32 per block
    if (piece / 32u < valid) {
      // Nontemporal: the GEMM launch reads the fp16 weights once, from memory.
      __builtin_nontemporal_store(reinterpret_cast<const u32x4_t*>(s_out)[piece],
                                  reinterpret_cast<u32x4_t*>(dst) + piece);
    }
  }
}

// ------------------------------------------------------------------ GEMM ----
// C[t][r] = sum_k X[t][k] W[r][k] with X [M = tokens][K], W [N = rows][K] fp16
// (both K-contiguous), C fp32 [M][N].  TM x TN tile per workgroup of four
// waves (128 x 128, or 64 x 64 when the large tiles would leave most CUs
// idle); wave w owns tokens TM/2 (w / 2) .. + TM/2 - 1 and rows TN/2 (w % 2)
// .. + TN/2 - 1 as (TM/64) x (TN/64) tiles of v_mfma_f32_32x32x16_f16.  K
// steps of 64 through two LDS stages; a 16-byte chunk j of tile row i (128
// bytes) lives at chunk j ^ gemm_swizzle(i).  A ds_read_b128 is served 16
// lanes at a time from 64 four-byte banks (256 bytes), so the 16 rows one
// fragment read visits (consecutive i, one chunk each) must cover all 16
// 16-byte bank groups: row i starts at group 8 (i & 1), and (i >> 1) & 7 gives
// the even and the odd rows eight distinct chunks each.  (j ^ (i & 7) put rows
// i and i + 8 on the same banks.)
constexpr int kGK = 64;
__device__ __forceinline__ int gemm_swizzle(int row) { return (row >> 1) & 7; }
typedef float float16v_t __attribute__((ext_vector_type(16)));

template <int TM, int TN>
__global__ __launch_bounds__(256) void gemm_f16_nt_kernel(const half_t* x, const half_t* w,
                                                          float* c, uint32_t m, uint32_t n,
                                                          uint32_t k, uint32_t split_steps,
                                                          const float* residual) {
  static_assert(TM % 64 == 0 && TN % 64 == 0, "whole 32 x 32 MFMA tiles per wave");
  constexpr int IA = TM / 64;   // MFMA tiles per wave along tokens
  constexpr int JB = TN / 64;   // along rows
  constexpr int LA = TM / 32;   // 16-byte chunks per thread per A tile step
  constexpr int LB = TN / 32;
  __shared__ __attribute__((aligned(16))) half_t s_a[2][TM * kGK];
  __shared__ __attribute__((aligned(16))) half_t s_b[2][TN * kGK];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const uint32_t m0 = blockIdx.y * TM;
  const uint32_t n0 = blockIdx.x * TN;
  // Range-checked operands: rows past the matrix read as zeros.
  const __amdgpu_buffer_rsrc_t xr =
    make_buffer_rsrc(x + (uint64_t)m0 * k, (uint32_t)min((uint64_t)TM, (uint64_t)(m - m0)) * k * 2u);
  const __amdgpu_buffer_rsrc_t wr =
    make_buffer_rsrc(w + (uint64_t)n0 * k, (uint32_t)min((uint64_t)TN, (uint64_t)(n - n0)) * k * 2u);
  // Global -> register staging: thread t moves chunks t + 256 i of each
  // T x 64 tile (row = idx / 8, chunk = idx % 8).
  u32x4_t ra[LA], rb[LB];
  auto load_step = [&](uint32_t kk) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < LA; ++i) {
      const int idx = tid + 256 * i;
      const uint32_t row = (uint32_t)(idx >> 3);
      const uint32_t off = (row * k + kk + 8u * (uint32_t)(idx & 7)) * 2u;
      ra[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(xr, (int)off, 0, 0));
    }
#pragma unroll
    for (int i = 0; i < LB; ++i) {
      const int idx = tid + 256 * i;
      const uint32_t row = (uint32_t)(idx >> 3);
      const uint32_t off = (row * k + kk + 8u * (uint32_t)(idx & 7)) * 2u;
      rb[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(wr, (int)off, 0, 0));
    }
  };
  auto store_step = [&](int st) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < LA; ++i) {
      const int idx = tid + 256 * i;
      const int row = idx >> 3;
      const int chunk = (idx & 7) ^ gemm_swizzle(row);
      *reinterpret_cast<u32x4_t*>(&s_a[st][row * kGK + 8 * chunk]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < LB; ++i) {
      const int idx = tid + 256 * i;
      const int row = idx >> 3;
      const int chunk = (idx & 7) ^ gemm_swizzle(row);
      *reinterpret_cast<u32x4_t*>(&s_b[st][row * kGK + 8 * chunk]) = rb[i];
    }
  };
  float16v_t acc[IA][JB];
#pragma unroll
  for (int i = 0; i < IA; ++i) {
#pragma unroll
    for (int j = 0; j < JB; ++j) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        acc[i][j][e] = 0.0f;
      }
    }
  }
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int frow = lane & 31;
  const int fk = lane >> 5;
  // K split z (blockIdx.z) takes K steps [z * split_steps, ...) and writes its
  // partial sums to plane z of c (split_steps = all steps: one plane, C itself).
  const uint32_t s_begin = blockIdx.z * split_steps;
  const uint32_t total_steps = k / kGK;
  const uint32_t steps = s_begin < total_steps ? min(total_steps - s_begin, split_steps) : 0u;
  c += (uint64_t)blockIdx.z * m * n;
  load_step(s_begin * kGK);
  store_step(0);
  __syncthreads();
  for (uint32_t s = 0; s < steps; ++s) {
    const int st = (int)(s & 1u);
    if (s + 1 < steps) {
      load_step((s_begin + s + 1) * kGK);
    }
#pragma unroll
    for (int ks = 0; ks < kGK / 16; ++ks) {
      half8_t fa[IA], fb[JB];
#pragma unroll
      for (int i = 0; i < IA; ++i) {
        const int row = (TM / 2) * wm + 32 * i + frow;
        const int chunk = (2 * ks + fk) ^ gemm_swizzle(row);
        fa[i] = *reinterpret_cast<const half8_t*>(&s_a[st][row * kGK + 8 * chunk]);
      }
#pragma unroll
      for (int j = 0; j < JB; ++j) {
        const int row = (TN / 2) * wn + 32 * j + frow;
        const int chunk = (2 * ks + fk) ^ gemm_swizzle(row);
        fb[j] = *reinterpret_cast<const half8_t*>(&s_b[st][row * kGK + 8 * chunk]);
      }
#pragma unroll
      for (int i = 0; i < IA; ++i) {
#pragma unroll
        for (int j = 0; j < JB; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
      }
    }
    if (s + 1 < steps) {
      store_step(st ^ 1);
    }
    __syncthreads();
  }
  // D layout: lane l holds column (row of W) l % 32 and tokens
  // 8 (e / 4) + 4 (l / 32) + e % 4 of its 32 x 32 tile.
#pragma unroll
  for (int i = 0; i < IA; ++i) {
#pragma unroll
    for (int j = 0; j < JB; ++j) {
      const uint32_t col = n0 + (TN / 2) * wn + 32u * j + (uint32_t)frow;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint32_t row = m0 + (TM / 2) * wm + 32u * i + 8u * (e / 4) + 4u * fk + (e % 4);
        if (row < m && col < n) {
          const uint64_t at = (uint64_t)row * n + col;
          store_through(&c[at], residual != nullptr ? residual[at] + acc[i][j][e] : acc[i][j][e]);
        }
      }
    }
  }
}

// The same GEMM, pipelined: the operand tiles go global -> LDS with
// direct-to-LDS copies (no staging registers) through NS stages, so the copies
// of K step s + NS - 1 are issued while step s computes.  With one step of
// prefetch the kernel above waits for each step's loads (a step of 16 MFMAs
// per wave is shorter than a load's latency).  Tile 128 tokens x TN rows
// (TN = 128: 4 stages of 32 KB; TN = 256: 3 stages of 48 KB, one workgroup per
// CU either way); wave w owns tokens 64 (w / 2) .. + 63 and rows TN/2 (w % 2)
// .. + TN/2 - 1.  The LDS layout (16-byte chunk j of tile row i at
// j ^ gemm_swizzle(i)) and the MFMA order over K are those of gemm_f16_nt_kernel, so each output
// gets the same bits; copy lane l of a wave fills LDS slot 64 c + l of its
// share and so loads the logical chunk that slot holds.
template <int TN>
struct GemmPipe {
  static constexpr int kTM = 128;
  static constexpr int kStages = TN == 128 ? 4 : 3;
  static constexpr int kStageHalfs = (kTM + TN) * kGK;
  static constexpr int kCopiesA = kTM / 32;  // per wave per stage
  static constexpr int kCopiesB = TN / 32;
  static constexpr int kCopies = kCopiesA + kCopiesB;
};

template <int TN>
__global__ __launch_bounds__(256) void gemm_f16_pipe_kernel(const half_t* x, const half_t* w,
                                                            float* c, uint32_t m, uint32_t n,
                                                            uint32_t k, uint32_t split_steps,
                                                            const float* residual) {
  using G = GemmPipe<TN>;
  constexpr int TM = G::kTM;
  constexpr int NS = G::kStages;
  constexpr int IA = TM / 64;
  constexpr int JB = TN / 64;
  static_assert(NS * G::kStageHalfs * 2 <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(16))) half_t s_ab[NS * G::kStageHalfs];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t m0 = blockIdx.y * TM;
  const uint32_t n0 = blockIdx.x * TN;
  // Range-checked operands: rows past the matrix read as zeros.
  const i32x4_t xr = rsrc_words(x + (uint64_t)m0 * k,
                                (uint32_t)min((uint64_t)TM, (uint64_t)(m - m0)) * k * 2u);
  const i32x4_t wr = rsrc_words(w + (uint64_t)n0 * k,
                                (uint32_t)min((uint64_t)TN, (uint64_t)(n - n0)) * k * 2u);
  // Byte offset (at K step 0) of the chunk copy i of this lane moves: LDS slot
  // P = 64 (kCopies_op * wave + i) + lane of the operand tile.
  uint32_t voff_a[G::kCopiesA], voff_b[G::kCopiesB];
#pragma unroll
  for (int i = 0; i < G::kCopiesA; ++i) {
    const uint32_t slot = 64u * (uint32_t)(G::kCopiesA * wave + i) + (uint32_t)lane;
    const uint32_t row = slot >> 3;
    voff_a[i] = (row * k + 8u * ((slot & 7u) ^ (uint32_t)gemm_swizzle((int)row))) * 2u;
  }
#pragma unroll
  for (int i = 0; i < G::kCopiesB; ++i) {
    const uint32_t slot = 64u * (uint32_t)(G::kCopiesB * wave + i) + (uint32_t)lane;
    const uint32_t row = slot >> 3;
    voff_b[i] = (row * k + 8u * ((slot & 7u) ^ (uint32_t)gemm_swizzle((int)row))) * 2u;
  }
  const uint32_t s_begin = blockIdx.z * split_steps;
  const uint32_t total_steps = k / kGK;
  const uint32_t steps = s_begin < total_steps ? min(total_steps - s_begin, split_steps) : 0u;
  c += (uint64_t)blockIdx.z * m * n;
  // LDS byte addresses of this wave's first A and B copy in stage 0.
  const uint32_t lds_base = (uint32_t)(uintptr_t)(lds_void_t*)s_ab;
  const uint32_t lds_a = lds_base + (uint32_t)(G::kCopiesA * wave) * 1024u;
  const uint32_t lds_b = lds_base + (uint32_t)(TM * kGK * 2) + (uint32_t)(G::kCopiesB * wave) * 1024u;
  auto issue = [&](uint32_t step, int st) __attribute__((always_inline)) {
    const uint32_t kb = (s_begin + step) * (uint32_t)kGK * 2u;
    const uint32_t so = (uint32_t)st * (uint32_t)(G::kStageHalfs * 2);
#pragma unroll
    for (int i = 0; i < G::kCopiesA; ++i) {
      copy16_to_lds_addr(xr, voff_a[i] + kb, lds_a + so + (uint32_t)i * 1024u);
    }
#pragma unroll
    for (int i = 0; i < G::kCopiesB; ++i) {
      copy16_to_lds_addr(wr, voff_b[i] + kb, lds_b + so + (uint32_t)i * 1024u);
    }
  };
  float16v_t acc[IA][JB];
#pragma unroll
  for (int i = 0; i < IA; ++i) {
#pragma unroll
    for (int j = 0; j < JB; ++j) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        acc[i][j][e] = 0.0f;
      }
    }
  }
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int frow = lane & 31;
  const int fk = lane >> 5;
#pragma unroll
  for (int st = 0; st < NS - 1; ++st) {
    if ((uint32_t)st < steps) {
      issue((uint32_t)st, st);
    }
  }
  for (uint32_t s = 0; s < steps; ++s) {
    // Step s's copies are the oldest in flight; those of the NS - 2 steps after
    // it may stay outstanding (loads complete in issue order).
    if (s + (NS - 2) < steps) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NS - 2) * G::kCopies) : "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();  // step s is in LDS; every wave is done with step s - 1's stage
    if (s + (NS - 1) < steps) {
      issue(s + (NS - 1), (int)((s + (NS - 1)) % NS));
    }
    const half_t* sa = s_ab + (int)(s % NS) * G::kStageHalfs;
    const half_t* sb = sa + TM * kGK;
    // Fragments of substep ks + 1 are read while substep ks's MFMAs run.
    half8_t fa[2][IA], fb[2][JB];
    auto read_frags = [&](int ks, int slot) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < IA; ++i) {
        const int row = (TM / 2) * wm + 32 * i + frow;
        const int chunk = (2 * ks + fk) ^ gemm_swizzle(row);
        fa[slot][i] = *reinterpret_cast<const half8_t*>(&sa[row * kGK + 8 * chunk]);
      }
#pragma unroll
      for (int j = 0; j < JB; ++j) {
        const int row = (TN / 2) * wn + 32 * j + frow;
        const int chunk = (2 * ks + fk) ^ gemm_swizzle(row);
        fb[slot][j] = *reinterpret_cast<const half8_t*>(&sb[row * kGK + 8 * chunk]);
      }
    };
    read_frags(0, 0);
#pragma unroll
    for (int ks = 0; ks < kGK / 16; ++ks) {
      if (ks + 1 < kGK / 16) {
        read_frags(ks + 1, (ks + 1) & 1);
      }
      // Keeps the reads ahead of the MFMAs (the scheduler would otherwise
      // interleave them back to one set of fragment registers).
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < IA; ++i) {
#pragma unroll
        for (int j = 0; j < JB; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[ks & 1][i], fb[ks & 1][j],
                                                            acc[i][j], 0, 0, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // D layout: lane l holds column (row of W) l % 32 and tokens
  // 8 (e / 4) + 4 (l / 32) + e % 4 of its 32 x 32 tile.
#pragma unroll
  for (int i = 0; i < IA; ++i) {
#pragma unroll
    for (int j = 0; j < JB; ++j) {
      const uint32_t col = n0 + (TN / 2) * wn + 32u * j + (uint32_t)frow;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint32_t row = m0 + (TM / 2) * wm + 32u * i + 8u * (e / 4) + 4u * fk + (e % 4);
        if (row < m && col < n) {
          const uint64_t at = (uint64_t)row * n + col;
          store_through(&c[at], residual != nullptr ? residual[at] + acc[i][j][e] : acc[i][j][e]);
        }
      }
    }
  }
}

// The same GEMM with the weights dequantized inside it: the B tile is decoded
// from the K-quant blocks on its way into LDS, so the fp16 weight matrix is
// never written and read back (the unfused path's dequantization pass wrote
// 2 bytes per weight and the GEMM read them again, against 0.56-0.82 bytes per
// weight of quant data here).  128 x 128 output tile, four waves as above, K
// steps of 128 (half a 256-value super-block: every format's chunks 4 s' ..
// 4 s' + 3 cover block positions 128 s' .. + 127), two LDS stages of 32 KB per
// operand.  Thread t decodes chunks 2 (t & 1) and + 1 of its K step for tile
// row t / 2 with the dequantization's exact arithmetic (ChunkDecoder<F, true>,
// then RNE to fp16), so the B tile holds the values the unfused pass wrote,
// and the MFMAs run over K in the same order: the result equals the unfused
// path's.  Rows past the matrix decode its last row (never stored).  16-byte
// chunk j of an LDS row lives at j ^ (row & 15).
constexpr int kQK = 128;

// Several matrices of one format that multiply the same input, in one grid:
// their 128-row tiles are numbered one after the other along blockIdx.x
// (matrix i owns tiles tile_end[i - 1] .. tile_end[i] - 1).
struct KqGroup {
  const uint8_t* w[kKquantGroupMax];
  float* c[kKquantGroupMax];
  uint32_t rows[kKquantGroupMax];
  uint32_t tile_end[kKquantGroupMax];
  uint32_t count;
};

template <int F, bool kGroup = false>
__global__ __launch_bounds__(256) void gemm_kq_kernel(const float* x, const uint8_t* wq,
                                                      float* c, uint32_t m, uint32_t n,
                                                      uint32_t k, uint32_t split_steps,
                                                      const float* residual,
                                                      KqGroup group = KqGroup{}) {
  constexpr int TM = 128;
  constexpr int TN = 128;
  constexpr int IA = TM / 64;
  constexpr int JB = TN / 64;
  constexpr int LA = TM * kQK / 8 / 256;  // 16-byte chunks of the A tile per thread
  __shared__ __attribute__((aligned(16))) half_t s_a[2][TM * kQK];
  __shared__ __attribute__((aligned(16))) half_t s_b[2][TN * kQK];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const uint32_t m0 = blockIdx.y * TM;
  uint32_t tile = blockIdx.x;
  if constexpr (kGroup) {
    uint32_t i = 0;
    while (i + 1 < group.count && tile >= group.tile_end[i]) {
      ++i;
    }
    tile -= i == 0 ? 0u : group.tile_end[i - 1];
    wq = group.w[i];
    c = group.c[i];
    n = group.rows[i];
  }
  const uint32_t n0 = tile * TN;
  const uint32_t bpr = k / 256u;
  // The f32 inputs, rounded to fp16 (RNE) on their way into LDS.
  const __amdgpu_buffer_rsrc_t xr =
    make_buffer_rsrc(x + (uint64_t)m0 * k, (uint32_t)min((uint64_t)TM, (uint64_t)(m - m0)) * k * 4u);
  // This thread's B row (clamped to the matrix) and chunk pair.
  const uint32_t brow = (uint32_t)tid >> 1;
  const uint8_t* wrow =
    wq + (uint64_t)min(n0 + brow, n - 1u) * bpr * KqFormat<F>::kBytes;
  const uint32_t cpair = 2u * ((uint32_t)tid & 1u);
  float4 ra[LA][2];
  RawChunk rb[2];
  auto load_step = [&](uint32_t st) __attribute__((always_inline)) {
    const uint32_t kk = st * kQK;
#pragma unroll
    for (int i = 0; i < LA; ++i) {
      const int idx = tid + 256 * i;
      const uint32_t row = (uint32_t)(idx >> 4);
      const uint32_t off = (row * k + kk + 8u * (uint32_t)(idx & 15)) * 4u;
      ra[i][0] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xr, (int)off, 0, 0));
      ra[i][1] = __builtin_bit_cast(float4,
                                    __builtin_amdgcn_raw_buffer_load_b128(xr, (int)off + 16, 0, 0));
    }
    const uint8_t* block = wrow + (uint64_t)(st >> 1) * KqFormat<F>::kBytes;
    const uint32_t c0 = 4u * (st & 1u) + cpair;
    rb[0] = load_raw<F, false>(block, c0);
    rb[1] = load_raw<F, false>(block, c0 + 1u);
  };
  auto store_step = [&](uint32_t st, int stage) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < LA; ++i) {
      const int idx = tid + 256 * i;
      const int row = idx >> 4;
      const int chunk = (idx & 15) ^ (row & 15);
      const float4 a = ra[i][0];
      const float4 b = ra[i][1];
      const half8_t h = {static_cast<half_t>(a.x), static_cast<half_t>(a.y),
                         static_cast<half_t>(a.z), static_cast<half_t>(a.w),
                         static_cast<half_t>(b.x), static_cast<half_t>(b.y),
                         static_cast<half_t>(b.z), static_cast<half_t>(b.w)};
      *reinterpret_cast<half8_t*>(&s_a[stage][row * kQK + 8 * chunk]) = h;
    }
    const uint32_t c0 = 4u * (st & 1u) + cpair;
    const uint32_t base = 128u * (st & 1u);
    half_t* brow_lds = &s_b[stage][brow * kQK];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      ChunkDecoder<F, true> dec;
      dec.compute(rb[q], c0 + (uint32_t)q);
#pragma unroll
      for (int half_i = 0; half_i < 2; ++half_i) {
        half8_t h0, h1;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          h0[j] = static_cast<half_t>(dec.v0[8 * half_i + j]);
          h1[j] = static_cast<half_t>(dec.v1[8 * half_i + j]);
        }
        const uint32_t j0 = (dec.p0 - base) / 8u + (uint32_t)half_i;
        const uint32_t j1 = (dec.p1 - base) / 8u + (uint32_t)half_i;
        *reinterpret_cast<half8_t*>(brow_lds + 8u * (j0 ^ (brow & 15u))) = h0;
        *reinterpret_cast<half8_t*>(brow_lds + 8u * (j1 ^ (brow & 15u))) = h1;
      }
    }
  };
  float16v_t acc[IA][JB];
#pragma unroll
  for (int i = 0; i < IA; ++i) {
#pragma unroll
    for (int j = 0; j < JB; ++j) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        acc[i][j][e] = 0.0f;
      }
    }
  }
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int frow = lane & 31;
  const int fk = lane >> 5;
  const uint32_t s_begin = blockIdx.z * split_steps;
  const uint32_t total_steps = k / kQK;
  const uint32_t steps = s_begin < total_steps ? min(total_steps - s_begin, split_steps) : 0u;
  c += (uint64_t)blockIdx.z * m * n;
  if (steps > 0) {
    load_step(s_begin);
    store_step(s_begin, 0);
  }
  __syncthreads();
  for (uint32_t s = 0; s < steps; ++s) {
    const int stage = (int)(s & 1u);
    if (s + 1 < steps) {
      load_step(s_begin + s + 1);
    }
#pragma unroll
    for (int ks = 0; ks < kQK / 16; ++ks) {
      half8_t fa[IA], fb[JB];
#pragma unroll
      for (int i = 0; i < IA; ++i) {
        const int row = (TM / 2) * wm + 32 * i + frow;
        const int chunk = (2 * ks + fk) ^ (row & 15);
        fa[i] = *reinterpret_cast<const half8_t*>(&s_a[stage][row * kQK + 8 * chunk]);
      }
#pragma unroll
      for (int j = 0; j < JB; ++j) {
        const int row = (TN / 2) * wn + 32 * j + frow;
        const int chunk = (2 * ks + fk) ^ (row & 15);
        fb[j] = *reinterpret_cast<const half8_t*>(&s_b[stage][row * kQK + 8 * chunk]);
      }
#pragma unroll
      for (int i = 0; i < IA; ++i) {
#pragma unroll
        for (int j = 0; j < JB; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
      }
    }
    if (s + 1 < steps) {
      store_step(s_begin + s + 1, stage ^ 1);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < IA; ++i) {
#pragma unroll
    for (int j = 0; j < JB; ++j) {
      const uint32_t col = n0 + (TN / 2) * wn + 32u * j + (uint32_t)frow;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint32_t row = m0 + (TM / 2) * wm + 32u * i + 8u * (e / 4) + 4u * fk + (e % 4);
        if (row < m && col < n) {
          const uint64_t at = (uint64_t)row * n + col;
          store_through(&c[at], residual != nullptr ? residual[at] + acc[i][j][e] : acc[i][j][e]);
        }
      }
    }
  }
}

// K splits: a 128 x 128 grid that would fill less than half of a 256-CU chip
// (the 1024-row projections at 1024 tokens: 64 tiles) splits K into up to four
// ranges of whole 64-deep steps, each writing an fp32 partial plane that one
// more pass sums in a fixed order.  Smaller tiles instead (64 x 64: four times
// the workgroups) were measured slower at K = 2048: each CU then loads twice
// the operand bytes per MFMA, and a CU's load path is what bounds the kernel.
constexpr uint64_t kGemmSmallGrid = 128;
constexpr uint32_t kGemmMaxSplits = 4;

uint32_t gemm_k_splits(size_t rows, size_t cols, size_t tokens) {
  const uint64_t tiles = (uint64_t)((rows + 127) / 128) * ((tokens + 127) / 128);
  const uint32_t steps = (uint32_t)(cols / kGK);
  uint32_t splits = 1;
  while (splits < kGemmMaxSplits && tiles * splits * 2 <= 2 * kGemmSmallGrid && steps >= 8 * splits * 2) {
    splits *= 2;
  }
  // The plane sum moves float4s: the output must be a whole number of them.
  return tiles >= kGemmSmallGrid || (tokens * rows) % 4u != 0 ? 1u : splits;
}

__global__ __launch_bounds__(256) void sum_planes_kernel(const float* planes, float* out,
                                                         uint64_t n4, uint32_t count,
                                                         const float* residual) {
  const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  if (i >= n4) {
    return;
  }
  const float4* p = reinterpret_cast<const float4*>(planes);
  float4 acc = p[i];
  for (uint32_t z = 1; z < count; ++z) {
    const float4 v = p[z * n4 + i];
    acc.x += v.x;
    acc.y += v.y;
    acc.z += v.z;
    acc.w += v.w;
  }
  if (residual != nullptr) {  // add_f32_in_place(residual, W x) on the sum
    const float4 r = reinterpret_cast<const float4*>(residual)[i];
    acc = make_float4(r.x + acc.x, r.y + acc.y, r.z + acc.z, r.w + acc.w);
  }
  reinterpret_cast<float4*>(out)[i] = acc;
}

// ---------------------------------------------------------------- argmax ----
struct ArgCand {
  float value;
  uint32_t index;
  float sum;  // sum of exp(v - value) over the candidate's range
};

__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi) {
  return v > bv || (v == bv && i < bi);
}

// Candidate of [begin, end) of `values`, reduced over a 256-thread workgroup.
// `with_sum` adds the range's sum of exp(v - max).
__device__ ArgCand block_candidate(const float* values, uint64_t begin, uint64_t end,
                                   uint32_t size_marker, bool with_sum) {
  __shared__ float s_v[256];
  __shared__ uint32_t s_i[256];
  __shared__ float s_s[256];
  const int tid = threadIdx.x;
  float bv = -INFINITY;
  uint32_t bi = size_marker;
  for (uint64_t i = begin + tid; i < end; i += 256) {
    const float v = values[i];
    if (better(v, (uint32_t)i, bv, bi)) {
      bv = v;
      bi = (uint32_t)i;
    }
  }
  s_v[tid] = bv;
  s_i[tid] = bi;
  __syncthreads();
  for (int stride = 128; stride > 0; stride >>= 1) {
    if (tid < stride && better(s_v[tid + stride], s_i[tid + stride], s_v[tid], s_i[tid])) {
      s_v[tid] = s_v[tid + stride];
      s_i[tid] = s_i[tid + stride];
    }
    __syncthreads();
  }
  ArgCand r{s_v[0], s_i[0], 0.0f};
  if (with_sum) {
    // A range whose values are all -inf or NaN has r.value == -inf; its -inf
    // entries count 0 (they add exp(-inf) to any finite overall maximum) and
    // its NaNs stay NaN, so the merged sum is what one pass would give.
    float sum = 0.0f;
    for (uint64_t i = begin + tid; i < end; i += 256) {
      const float v = values[i];
      sum += (v == -INFINITY && r.value == -INFINITY) ? 0.0f : expf(v - r.value);
    }
    s_s[tid] = sum;
    __syncthreads();
    for (int stride = 128; stride > 0; stride >>= 1) {
      if (tid < stride) {
        s_s[tid] += s_s[tid + stride];
      }
      __syncthreads();
    }
    r.sum = s_s[0];
  }
  __syncthreads();
  return r;
}

// Phase 1: workgroup g takes [g * span, (g + 1) * span).
__global__ __launch_bounds__(256) void argmax_partial_kernel(const float* values, uint64_t size,
                                                             uint64_t span, bool with_sum,
                                                             ArgCand* cands) {
  const uint64_t begin = (uint64_t)blockIdx.x * span;
  const uint64_t end = min(size, begin + span);
  const ArgCand r = block_candidate(values, begin, end, (uint32_t)size, with_sum);
  if (threadIdx.x == 0) {
    cands[blockIdx.x] = r;
  }
}

// Phase 2 (or the whole job when cands == nullptr): merges candidates.
// `max_above_neg_inf`: the K-quant top-1/argmax rule (mps_backend.mm:692-750,
// 1652-1690: the reduction starts from index 0 at -inf), where the token is 0
// unless some value exceeds -inf; otherwise the generic argmax_f32_i32 rule (the
// first index of the maximum, `size` when every value is NaN).
__global__ __launch_bounds__(256) void argmax_final_kernel(const float* values, uint64_t size,
                                                           const ArgCand* cands, uint32_t count,
                                                           bool with_sum, bool max_above_neg_inf,
                                                           int32_t* token_out,
                                                           float* probability_out) {
  __shared__ float s_v[256];
  __shared__ uint32_t s_i[256];
  __shared__ float s_s[256];
  const int tid = threadIdx.x;
  if (cands == nullptr) {
    const ArgCand r = block_candidate(values, 0, size, (uint32_t)size, with_sum);
    if (tid == 0) {
      token_out[0] = max_above_neg_inf && !(r.value > -INFINITY) ? 0 : (int32_t)r.index;
      if (probability_out != nullptr) {
        probability_out[0] = r.sum > 0.0f ? 1.0f / r.sum : 0.0f;
      }
    }
    return;
  }
  float bv = -INFINITY;
  uint32_t bi = (uint32_t)size;
  for (uint32_t g = tid; g < count; g += 256) {
    if (better(cands[g].value, cands[g].index, bv, bi)) {
      bv = cands[g].value;
      bi = cands[g].index;
    }
  }
  s_v[tid] = bv;
  s_i[tid] = bi;
  __syncthreads();
  for (int stride = 128; stride > 0; stride >>= 1) {
    if (tid < stride && better(s_v[tid + stride], s_i[tid + stride], s_v[tid], s_i[tid])) {
      s_v[tid] = s_v[tid + stride];
      s_i[tid] = s_i[tid + stride];
    }
    __syncthreads();
  }
  const float gmax = s_v[0];
  const uint32_t gidx = s_i[0];
  if (with_sum) {
    float sum = 0.0f;
    for (uint32_t g = tid; g < count; g += 256) {
      sum += cands[g].sum * expf(cands[g].value - gmax);
    }
    s_s[tid] = sum;
    __syncthreads();
    for (int stride = 128; stride > 0; stride >>= 1) {
      if (tid < stride) {
        s_s[tid] += s_s[tid + stride];
      }
      __syncthreads();
    }
  }
  if (tid == 0) {
    token_out[0] = max_above_neg_inf && !(gmax > -INFINITY) ? 0 : (int32_t)gidx;
    if (probability_out != nullptr) {
      probability_out[0] = s_s[0] > 0.0f ? 1.0f / s_s[0] : 0.0f;
    }
  }
}

constexpr uint64_t kArgmaxSingleMax = 16384;  // one workgroup up to this size
constexpr uint64_t kArgmaxSpan = 4096;        // values per phase-1 workgroup

template <int F>
hipError_t launch_gemv_f(const GemvArgs& base, hipStream_t stream) {
  const uint32_t bpr = base.blocks_per_row;
  const int bc = bpr >= 5 ? 8 : (bpr >= 3 ? 4 : (bpr == 2 ? 2 : 1));
  const uint32_t rows_per_wg = 64u / (8u * (uint32_t)bc);
  const dim3 grid((base.rows + rows_per_wg - 1) / rows_per_wg);
  for (uint32_t t0 = 0; t0 < base.tokens;) {
    GemvArgs a = base;
    a.token_base = t0;
    const uint32_t left = base.tokens - t0;
    const int tg = left >= 8 ? 8 : (left >= 4 ? 4 : (left >= 2 ? 2 : 1));
#define KQ_GEMV_CASE(BC, TG) \
  if (bc == BC && tg == TG) kq_gemv_kernel<F, BC, TG><<<grid, 64, 0, stream>>>(a);
#define KQ_GEMV_BC(BC) KQ_GEMV_CASE(BC, 1) KQ_GEMV_CASE(BC, 2) KQ_GEMV_CASE(BC, 4) KQ_GEMV_CASE(BC, 8)
    KQ_GEMV_BC(1) KQ_GEMV_BC(2) KQ_GEMV_BC(4) KQ_GEMV_BC(8)
#undef KQ_GEMV_BC
#undef KQ_GEMV_CASE
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
      return e;
    }
    t0 += (uint32_t)tg;
  }
  return hipSuccess;
}

template <int F, int XF>
hipError_t launch_gemv_fused_fx(const FusedGemvArgs& a, hipStream_t stream) {
  const uint32_t bpr = a.blocks_per_row;
  const int bc = bpr >= 5 ? 8 : (bpr >= 3 ? 4 : (bpr == 2 ? 2 : 1));
  const uint32_t rows_per_wg = 64u / (8u * (uint32_t)bc);
  const dim3 grid((a.rows + rows_per_wg - 1) / rows_per_wg);
  switch (bc) {
    case 8:
      kq_gemv_fused_kernel<F, 8, XF><<<grid, 64, 0, stream>>>(a);
      break;
    case 4:
      kq_gemv_fused_kernel<F, 4, XF><<<grid, 64, 0, stream>>>(a);
      break;
    case 2:
      kq_gemv_fused_kernel<F, 2, XF><<<grid, 64, 0, stream>>>(a);
      break;
    default:
      kq_gemv_fused_kernel<F, 1, XF><<<grid, 64, 0, stream>>>(a);
      break;
  }
  return hipGetLastError();
}

constexpr uint32_t kXsMaxWorkgroups = 1024;  // four per CU, over all matrices
// Up to this many workgroups the launch covers every row in one trip (the
// workgroups beyond those resident start as others finish).
constexpr uint32_t kXsOneTripWorkgroups = 2 * kXsMaxWorkgroups;
constexpr uint32_t kXsMaxBlocksPerRow = 16;   // two chunks per lane

template <int LR, int PPL, int XF>
hipError_t launch_xs(MultiGemvArgs a, hipStream_t stream) {
  // Workgroups per matrix: enough to cover its rows in one trip, or, past
  // kXsOneTripWorkgroups, the resident count shared in proportion (then every
  // workgroup takes two rows per lane per trip, the next two prefetched, and
  // computes the transformed input once for all its trips).
  constexpr uint32_t rows_per_wg = kXsWaves * (64 / LR);
  // Two chunks per lane take about twice the registers: two workgroups per CU.
  constexpr uint32_t max_wgs = PPL == 1 ? kXsMaxWorkgroups : kXsMaxWorkgroups / 2;
  uint32_t need[kXsMaxMatrices] = {0, 0, 0, 0};
  uint32_t total = 0;
  for (uint32_t m = 0; m < a.count; ++m) {
    need[m] = (a.rows[m] + rows_per_wg - 1) / rows_per_wg;
    total += need[m];
  }
  const bool one_trip = total <= kXsOneTripWorkgroups;
  a.wg_begin[0] = 0;
  for (uint32_t m = 0; m < kXsMaxMatrices; ++m) {
    uint32_t n = 0;
    if (m < a.count) {
      n = one_trip ? need[m]
                   : (uint32_t)(((uint64_t)need[m] * max_wgs + total - 1) / total);
      n = n == 0 ? 1 : n;
    }
    a.wg_begin[m + 1] = a.wg_begin[m] + n;
  }
  const dim3 grid(a.wg_begin[a.count]);
  if (a.conv_pool != nullptr) {
    // The conv epilogue comes with the RMSNorm input (the joint projection).
    if constexpr (XF == 1) {
      if (one_trip) {
        kq_gemv_xs_kernel<LR, PPL, XF, 1, true><<<grid, 64 * kXsWaves, 0, stream>>>(a);
      } else {
        kq_gemv_xs_kernel<LR, PPL, XF, 2, true><<<grid, 64 * kXsWaves, 0, stream>>>(a);
      }
      return hipGetLastError();
    } else {
      return hipErrorInvalidValue;
    }
  }
  if (one_trip) {
    kq_gemv_xs_kernel<LR, PPL, XF, 1><<<grid, 64 * kXsWaves, 0, stream>>>(a);
  } else {
    kq_gemv_xs_kernel<LR, PPL, XF, 2><<<grid, 64 * kXsWaves, 0, stream>>>(a);
  }
  return hipGetLastError();
}

template <int XF>
hipError_t launch_xs_x(const MultiGemvArgs& a, hipStream_t stream) {
  const uint32_t chunks = 8u * a.blocks_per_row;
  if (chunks <= 8u) return launch_xs<8, 1, XF>(a, stream);
  if (chunks <= 16u) return launch_xs<16, 1, XF>(a, stream);
  if (chunks <= 32u) return launch_xs<32, 1, XF>(a, stream);
  if (chunks <= 64u) return launch_xs<64, 1, XF>(a, stream);
  return launch_xs<64, 2, XF>(a, stream);
}

hipError_t launch_multi(MultiGemvArgs a, hipStream_t stream) {
  // Q6_K matrices read as whole-wave spans (format 3) when every 16-byte piece
  // of a span lies wholly inside or wholly outside the matrix: a 16-byte
  // aligned base and rows * blocks_per_row * 210 a multiple of 16.
  for (uint32_t m = 0; m < a.count; ++m) {
    if (a.format[m] == 2 && ((uintptr_t)a.weight[m] & 15u) == 0 &&
        ((uint64_t)a.rows[m] * a.blocks_per_row) % 8u == 0) {
      a.format[m] = 3;
    }
  }
  if (a.gate_factor != nullptr) {
    return launch_xs_x<3>(a, stream);
  }
  if (a.norm_weight != nullptr) {
    return launch_xs_x<1>(a, stream);
  }
  if (a.up != nullptr) {
    return launch_xs_x<2>(a, stream);
  }
  return launch_xs_x<0>(a, stream);
}

template <int F>
hipError_t launch_gemv_fused_f(const FusedGemvArgs& a, hipStream_t stream) {
  if (a.blocks_per_row <= kXsMaxBlocksPerRow) {
    MultiGemvArgs m{};
    m.weight[0] = a.weight;
    m.output[0] = a.output;
    m.residual[0] = a.residual;
    m.rows[0] = a.rows;
    m.format[0] = F;
    m.count = 1;
    m.input = a.input;
    m.norm_weight = a.norm_weight;
    m.up = a.up;
    m.cols = a.cols;
    m.blocks_per_row = a.blocks_per_row;
    m.eps = a.eps;
    return launch_multi(m, stream);
  }
  if (a.norm_weight != nullptr) {
    return launch_gemv_fused_fx<F, 1>(a, stream);
  }
  if (a.up != nullptr) {
    return launch_gemv_fused_fx<F, 2>(a, stream);
  }
  return launch_gemv_fused_fx<F, 0>(a, stream);
}

hipError_t launch_gemv_fused(int format, const FusedGemvArgs& a, hipStream_t stream) {
  switch (format) {
    case 0:
      return launch_gemv_fused_f<0>(a, stream);
    case 1:
      return launch_gemv_fused_f<1>(a, stream);
    case 2:
      return launch_gemv_fused_f<2>(a, stream);
    default:
      return hipErrorInvalidValue;
  }
}

hipError_t launch_gemv(int format, const GemvArgs& a, hipStream_t stream) {
  switch (format) {
    case 0:
      return launch_gemv_f<0>(a, stream);
    case 1:
      return launch_gemv_f<1>(a, stream);
    case 2:
      return launch_gemv_f<2>(a, stream);
    default:
      return hipErrorInvalidValue;
  }
}

size_t align256(size_t v) { return (v + 255u) & ~static_cast<size_t>(255u); }

}  // namespace

uint32_t kquant_block_bytes(int format) {
  return format == 0 ? 144u : (format == 1 ? 176u : (format == 2 ? 210u : 0u));
}

// The GEMM form per format: the fused one (weights decoded in the B tile) for
// Q4_K, the two-pass one (the weights dequantized to an fp16 matrix in the
// workspace, then the fp16 GEMM) for Q5_K and Q6_K, whose decode costs more
// VALU work per weight than the fused tile hides under its MFMAs (measured on
// the Qwen3.5-0.8B shapes at 1024 tokens: Q4_K 3584 x 1024 31.3 -> 28.0 us,
// Q5_K 6144 x 1024 38.2 -> 48.3 us, Q6_K 1024 x 3584 32.5 -> 40.1 us).
// KRAKEN_KQUANT_GEMM=fused or =unfused forces one form for every format.
bool kquant_gemm_unfused(int format) {
  const char* v = std::getenv("KRAKEN_KQUANT_GEMM");
  if (v != nullptr && std::strcmp(v, "unfused") == 0) {
    return true;
  }
  if (v != nullptr && std::strcmp(v, "fused") == 0) {
    return false;
  }
  return format != 0;
}

// The fp16 GEMM of the two-pass form.  All of them give the same bits (same
// LDS layout, same MFMA order over K, same K split); KRAKEN_GEMM_F16=plain
// selects the one-step-prefetch kernel.  Without a K split: 128 x 192 tiles
// when the rows divide into them and give at least 224 workgroups, else
// 128 x 256 when those give at least 160 (one per CU); otherwise 128 x 128.
enum class GemmKernel { plain, pipe128, pipe192, pipe256 };
GemmKernel gemm_f16_kernel_choice(size_t rows, size_t tokens, uint32_t splits) {
  const char* env = std::getenv("KRAKEN_GEMM_F16");
  if (env != nullptr && std::strcmp(env, "plain") == 0) {
    return GemmKernel::plain;
  }
  // 128 x 192 tiles where they give close to one workgroup per CU (the
  // 6144-row tensor at 1024 tokens: 256 of them against 192 of 128 x 256,
  // 34.4 -> 30.8 us per call).
  const uint64_t tiles192 = (uint64_t)((rows + 191) / 192) * ((tokens + 127) / 128);
  if (splits == 1 && rows % 192 == 0 && tiles192 >= 224) {
    return GemmKernel::pipe192;
  }
  const uint64_t tiles256 = (uint64_t)((rows + 255) / 256) * ((tokens + 127) / 128);
  return splits == 1 && tiles256 >= 160 ? GemmKernel::pipe256 : GemmKernel::pipe128;
}

hipError_t launch_kquant_matmul_group(int format, size_t count, const void* const* weights,
                                      const size_t* rows, size_t cols, size_t tokens,
                                      const float* input, float* const* outputs,
                                      hipStream_t stream) {
  if (count == 0 || count > kKquantGroupMax || tokens <= kKquantGemvMaxTokens ||
      kquant_gemm_unfused(format)) {
    return hipErrorNotSupported;
  }
  KqGroup g{};
  uint32_t tiles = 0;
  for (size_t i = 0; i < count; ++i) {
    g.w[i] = static_cast<const uint8_t*>(weights[i]);
    g.c[i] = outputs[i];
    g.rows[i] = (uint32_t)rows[i];
    tiles += (uint32_t)((rows[i] + 127) / 128);
    g.tile_end[i] = tiles;
  }
  g.count = (uint32_t)count;
  const dim3 grid(tiles, (uint32_t)((tokens + 127) / 128), 1);
  const uint32_t steps = (uint32_t)(cols / kQK);
  switch (format) {
    case 0:
      gemm_kq_kernel<0, true><<<grid, 256, 0, stream>>>(input, nullptr, nullptr, (uint32_t)tokens,
                                                        0u, (uint32_t)cols, steps, nullptr, g);
      break;
    case 1:
      gemm_kq_kernel<1, true><<<grid, 256, 0, stream>>>(input, nullptr, nullptr, (uint32_t)tokens,
                                                        0u, (uint32_t)cols, steps, nullptr, g);
      break;
    case 2:
      gemm_kq_kernel<2, true><<<grid, 256, 0, stream>>>(input, nullptr, nullptr, (uint32_t)tokens,
                                                        0u, (uint32_t)cols, steps, nullptr, g);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Input groups of eight from which the first pass converts four per thread.
constexpr uint64_t kWideConvertGroups = 262144;

size_t kquant_matmul_workspace_bytes(int format, size_t rows, size_t cols, size_t tokens,
                                     bool swiglu) {
  if (tokens <= kKquantGemvMaxTokens) {
    return 0;
  }
  const uint32_t splits = gemm_k_splits(rows, cols, tokens);
  return (swiglu || kquant_gemm_unfused(format)
            ? align256(rows * cols * 2u) + align256(tokens * cols * 2u)
            : 0u) +
         (splits > 1 ? align256(splits * tokens * rows * 4u) : 0u);
}

hipError_t launch_kquant_matmul(int format, const void* weight, size_t rows, size_t cols,
                                size_t tokens, const float* input, float* output,
                                void* workspace, size_t workspace_bytes, hipStream_t stream,
                                const float* up, const float* residual) {
  const uint32_t bpr = (uint32_t)(cols / 256u);
  if (tokens == 1 && bpr <= kXsMaxBlocksPerRow) {
    FusedGemvArgs f{static_cast<const uint8_t*>(weight), input, nullptr, nullptr, nullptr, output,
                    (uint32_t)rows, (uint32_t)cols, bpr, 0.0f};
    return launch_gemv_fused(format, f, stream);
  }
  if ((up != nullptr || residual != nullptr) && tokens <= kKquantGemvMaxTokens) {
    return hipErrorInvalidValue;  // the GEMM path only
  }
  if (tokens <= kKquantGemvMaxTokens) {
    // The reference's batched matvec (4 to 8 tokens) multiplies fp16-rounded
    // weights with fp32 inputs; 1 to 3 tokens stay fp32 throughout.
    GemvArgs a{static_cast<const uint8_t*>(weight), input, output, (uint32_t)rows,
               (uint32_t)cols, bpr, (uint32_t)tokens, 0u, tokens >= 4u ? 1u : 0u};
    return launch_gemv(format, a, stream);
  }
  const size_t need = kquant_matmul_workspace_bytes(format, rows, cols, tokens, up != nullptr);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    return hipErrorInvalidValue;
  }
  // Workspace: [fp16 weights] [fp16 inputs] (two-pass form only) [K-split planes].
  // A SwiGLU input takes the two-pass form, whose first pass forms it.
  const bool unfused = up != nullptr || kquant_gemm_unfused(format);
  half_t* w16 = static_cast<half_t*>(workspace);
  half_t* x16 = reinterpret_cast<half_t*>(static_cast<char*>(workspace) +
                                          (unfused ? align256(rows * cols * 2u) : 0u));
  const uint8_t* wq = static_cast<const uint8_t*>(weight);
  hipError_t e = hipSuccess;
  if (unfused) {
    const uint64_t blocks = (uint64_t)rows * bpr;
    const uint64_t n8 = (uint64_t)tokens * cols / 8u;
    // A large plain input (the 3584-wide FFN activations) converts four groups
    // of eight per thread: Q6_K 1024 x 3584 at 1024 tokens 31.0 -> 28.7 us; a
    // 1024-wide one keeps one group (Q5_K 30.2 against 31.5 us with four), and
    // so does the SwiGLU input, whose exponentials make four groups a long
    // chain (first pass 9.9 -> 11.1 us in the whole-model prefill).
    const bool wide = n8 >= kWideConvertGroups && up == nullptr;
    const uint32_t per_wg = wide ? 1024u : 256u;
    const uint32_t convert_blocks = (uint32_t)((n8 + per_wg - 1) / per_wg);
    const dim3 dq(convert_blocks + (uint32_t)((blocks + 31) / 32));
    auto first_pass = [&](auto kernel) {
      kernel<<<dq, 256, 0, stream>>>(wq, (uint32_t)rows, bpr, w16, input, x16, n8,
                                     convert_blocks, up);
    };
    if (format == 0) {
      wide ? first_pass(kq_dequant_f16_kernel<0, 4>) : first_pass(kq_dequant_f16_kernel<0, 1>);
    } else if (format == 1) {
      wide ? first_pass(kq_dequant_f16_kernel<1, 4>) : first_pass(kq_dequant_f16_kernel<1, 1>);
    } else {
      wide ? first_pass(kq_dequant_f16_kernel<2, 4>) : first_pass(kq_dequant_f16_kernel<2, 1>);
    }
    if ((e = hipGetLastError()) != hipSuccess) {
      return e;
    }
  }
  const uint32_t splits = gemm_k_splits(rows, cols, tokens);
  float* planes = splits > 1 ? reinterpret_cast<float*>(
                                 static_cast<char*>(workspace) +
                                 (unfused ? align256(rows * cols * 2u) + align256(tokens * cols * 2u)
                                          : 0u))
                             : output;
  const dim3 grid((uint32_t)((rows + 127) / 128), (uint32_t)((tokens + 127) / 128), splits);
  // Without K splits the GEMM adds the residual itself; with them the plane sum does.
  const float* res = splits == 1 ? residual : nullptr;
  if (unfused) {
    const uint32_t steps = (uint32_t)(cols / kGK);
    const uint32_t split_steps = (steps + splits - 1) / splits;
    const GemmKernel kernel = gemm_f16_kernel_choice(rows, tokens, splits);
    if (kernel == GemmKernel::pipe192) {
      const dim3 g192((uint32_t)((rows + 191) / 192), (uint32_t)((tokens + 127) / 128), splits);
      gemm_f16_pipe_kernel<192><<<g192, 256, 0, stream>>>(x16, w16, planes, (uint32_t)tokens,
                                                          (uint32_t)rows, (uint32_t)cols,
                                                          split_steps, res);
    } else if (kernel == GemmKernel::pipe256) {
      const dim3 g256((uint32_t)((rows + 255) / 256), (uint32_t)((tokens + 127) / 128), splits);
      gemm_f16_pipe_kernel<256><<<g256, 256, 0, stream>>>(x16, w16, planes, (uint32_t)tokens,
                                                          (uint32_t)rows, (uint32_t)cols,
                                                          split_steps, res);
    } else if (kernel == GemmKernel::pipe128) {
      gemm_f16_pipe_kernel<128><<<grid, 256, 0, stream>>>(x16, w16, planes, (uint32_t)tokens,
                                                          (uint32_t)rows, (uint32_t)cols,
                                                          split_steps, res);
    } else {
      gemm_f16_nt_kernel<128, 128><<<grid, 256, 0, stream>>>(x16, w16, planes, (uint32_t)tokens,
                                                             (uint32_t)rows, (uint32_t)cols,
                                                             split_steps, res);
    }
  } else {
    const uint32_t steps = (uint32_t)(cols / kQK);
    const uint32_t split_steps = (steps + splits - 1) / splits;
    if (format == 0) {
      gemm_kq_kernel<0><<<grid, 256, 0, stream>>>(input, wq, planes, (uint32_t)tokens,
                                                  (uint32_t)rows, (uint32_t)cols, split_steps,
                                                  res);
    } else if (format == 1) {
      gemm_kq_kernel<1><<<grid, 256, 0, stream>>>(input, wq, planes, (uint32_t)tokens,
                                                  (uint32_t)rows, (uint32_t)cols, split_steps,
                                                  res);
    } else {
      gemm_kq_kernel<2><<<grid, 256, 0, stream>>>(input, wq, planes, (uint32_t)tokens,
                                                  (uint32_t)rows, (uint32_t)cols, split_steps,
                                                  res);
    }
  }
  if ((e = hipGetLastError()) != hipSuccess || splits == 1) {
    return e;
  }
  const uint64_t n4 = (uint64_t)tokens * rows / 4u;
  sum_planes_kernel<<<dim3((uint32_t)((n4 + 255) / 256)), 256, 0, stream>>>(planes, output, n4,
                                                                         splits, residual);
  return hipGetLastError();
}

hipError_t launch_kquant_dequantize_rows(int format, const void* weight, size_t rows,
                                         const int32_t* row_ids, size_t fixed_row,
                                         size_t tokens, size_t cols, float* output,
                                         hipStream_t stream) {
  const uint32_t bpr = (uint32_t)(cols / 256u);
  const uint64_t threads = (uint64_t)tokens * bpr * 8u;
  const dim3 grid((uint32_t)((threads + 255) / 256));
  const uint8_t* w = static_cast<const uint8_t*>(weight);
  if (format == 0) {
    kq_dequant_rows_kernel<0><<<grid, 256, 0, stream>>>(w, row_ids, (uint32_t)fixed_row,
                                                        (uint32_t)rows, (uint32_t)tokens, bpr,
                                                        output);
  } else if (format == 1) {
    kq_dequant_rows_kernel<1><<<grid, 256, 0, stream>>>(w, row_ids, (uint32_t)fixed_row,
                                                        (uint32_t)rows, (uint32_t)tokens, bpr,
                                                        output);
  } else {
    kq_dequant_rows_kernel<2><<<grid, 256, 0, stream>>>(w, row_ids, (uint32_t)fixed_row,
                                                        (uint32_t)rows, (uint32_t)tokens, bpr,
                                                        output);
  }
  return hipGetLastError();
}

size_t argmax_workspace_bytes(size_t size) {
  if (size <= kArgmaxSingleMax) {
    return 0;
  }
  const size_t groups = (size + kArgmaxSpan - 1) / kArgmaxSpan;
  return groups * sizeof(ArgCand);
}

hipError_t launch_argmax(const float* values, size_t size, int32_t* token_out,
                         float* probability_out, void* workspace, size_t workspace_bytes,
                         hipStream_t stream, bool kquant_rule) {
  const bool with_sum = probability_out != nullptr;
  if (size <= kArgmaxSingleMax) {
    argmax_final_kernel<<<1, 256, 0, stream>>>(values, size, nullptr, 0, with_sum, kquant_rule,
                                               token_out, probability_out);
    return hipGetLastError();
  }
  const size_t groups = (size + kArgmaxSpan - 1) / kArgmaxSpan;
  if (workspace == nullptr || workspace_bytes < groups * sizeof(ArgCand)) {
    return hipErrorInvalidValue;
  }
  ArgCand* cands = static_cast<ArgCand*>(workspace);
  argmax_partial_kernel<<<dim3((uint32_t)groups), 256, 0, stream>>>(values, size, kArgmaxSpan,
                                                                    with_sum, cands);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return e;
  }
  argmax_final_kernel<<<1, 256, 0, stream>>>(values, size, cands, (uint32_t)groups, with_sum,
                                             kquant_rule, token_out, probability_out);
  return hipGetLastError();
}

size_t kquant_argmax_workspace_bytes(size_t rows) {
  return align256(rows * sizeof(float)) + argmax_workspace_bytes(rows);
}

hipError_t launch_kquant_matvec_fused(int format, const void* weight, size_t rows, size_t cols,
                                      const float* input, const float* norm_weight, float eps,
                                      const float* up, const float* residual, float* output,
                                      hipStream_t stream) {
  FusedGemvArgs a{static_cast<const uint8_t*>(weight), input, norm_weight, up, residual, output,
                  (uint32_t)rows, (uint32_t)cols, (uint32_t)(cols / 256u), eps};
  return launch_gemv_fused(format, a, stream);
}

hipError_t launch_kquant_matvec_multi(uint32_t count, const int* formats,
                                      const void* const* weights, const size_t* rows,
                                      size_t cols, const float* input, const float* norm_weight,
                                      float eps, const float* up,
                                      const float* const* residuals, float* const* outputs,
                                      hipStream_t stream, const GemvConvEpilogue* conv) {
  if (count == 0 || count > (uint32_t)kXsMaxMatrices || cols / 256u > kXsMaxBlocksPerRow) {
    return hipErrorInvalidValue;
  }
  MultiGemvArgs m{};
  for (uint32_t i = 0; i < count; ++i) {
    m.weight[i] = static_cast<const uint8_t*>(weights[i]);
    m.output[i] = outputs[i];
    m.residual[i] = residuals[i];
    m.rows[i] = (uint32_t)rows[i];
    m.format[i] = formats[i];
  }
  m.count = count;
  m.input = input;
  m.norm_weight = norm_weight;
  m.up = up;
  m.cols = (uint32_t)cols;
  m.blocks_per_row = (uint32_t)(cols / 256u);
  m.eps = eps;
  m.conv_pool = conv != nullptr ? conv->pool : nullptr;
  m.conv_offset = conv != nullptr ? conv->offset : nullptr;
  m.conv_pool_elems = conv != nullptr ? conv->pool_elems : 0u;
  m.conv_weights = conv != nullptr ? conv->weights : nullptr;
  return launch_multi(m, stream);
}

hipError_t launch_kquant_matvec_head_norm(int format, const void* weight, size_t rows,
                                          size_t cols, const float* input,
                                          const float* gate_factor, float eps,
                                          const float* residual, float* output,
                                          hipStream_t stream) {
  if (cols / 256u > kXsMaxBlocksPerRow || cols % 128u != 0) {
    return hipErrorInvalidValue;
  }
  MultiGemvArgs m{};
  m.weight[0] = static_cast<const uint8_t*>(weight);
  m.output[0] = output;
  m.residual[0] = residual;
  m.rows[0] = (uint32_t)rows;
  m.format[0] = format;
  m.count = 1;
  m.input = input;
  m.gate_factor = gate_factor;
  m.cols = (uint32_t)cols;
  m.blocks_per_row = (uint32_t)(cols / 256u);
  m.eps = eps;
  return launch_multi(m, stream);
}

hipError_t launch_kquant_argmax(int format, const void* weight, size_t rows, size_t cols,
                                const float* input, int32_t* token_out, float* probability_out,
                                void* workspace, size_t workspace_bytes, hipStream_t stream,
                                const float* norm_weight, float eps) {
  if (workspace == nullptr || workspace_bytes < kquant_argmax_workspace_bytes(rows)) {
    return hipErrorInvalidValue;
  }
  float* logits = static_cast<float*>(workspace);
  hipError_t e;
  if (norm_weight != nullptr || cols / 256u <= kXsMaxBlocksPerRow) {
    e = launch_kquant_matvec_fused(format, weight, rows, cols, input, norm_weight, eps, nullptr,
                                   nullptr, logits, stream);
  } else {
    GemvArgs a{static_cast<const uint8_t*>(weight), input, logits, (uint32_t)rows,
               (uint32_t)cols, (uint32_t)(cols / 256u), 1u, 0u, 0u};
    e = launch_gemv(format, a, stream);
  }
  if (e != hipSuccess) {
    return e;
  }
  void* rest = static_cast<char*>(workspace) + align256(rows * sizeof(float));
  return launch_argmax(logits, rows, token_out, probability_out, rest,
                       workspace_bytes - align256(rows * sizeof(float)), stream,
                       /*kquant_rule=*/true);
}

}  // namespace kraken
