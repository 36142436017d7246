/*
 * kquant_oracle.c -- CPU restatement of the reference's K-quant (GGUF Q4_K,
 * Q5_K, Q6_K) projection operators and device argmax.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP backend, never a product
 * path (same rules as kraken_oracle.c).
 *
 * The block formats are GGUF's (ggml's k-quants, 256 values per super-block),
 * as the reference's Metal kernels read them (mps_backend.mm:751-770 for the
 * structs; the arithmetic below follows the get-row kernels :1448-1540 and the
 * matvec kernels :284-460, which compute the same dequantized values):
 *   Q4_K, 144 bytes: f16 d, f16 dmin, 12 bytes of packed 6-bit (scale, min)
 *         pairs for 8 sub-blocks of 32, 128 bytes of 4-bit quants.  Value
 *         64 s + i (s = 0..3, i < 32) is d*sc(2s) * lo4(qs[32 s + i]) - dmin*m(2s);
 *         value 64 s + 32 + i uses hi4(qs[32 s + i]) and sub-block 2 s + 1.
 *   Q5_K, 176 bytes: as Q4_K plus qh[32]; bit 2 s (low nibble) or 2 s + 1
 *         (high nibble) of qh[i] adds 16 to the quant.
 *   Q6_K, 210 bytes: ql[128], qh[64], int8 scales[16], f16 d.  In half h
 *         (128 values), value 128 h + 32 g + i (g = 0..3, i < 32) is
 *         d * scales[8 h + 2 g + i / 16] * (q - 32), q = lo4/hi4 of
 *         ql[64 h + i + 32 (g & 1)] (g < 2: low nibble) with bits 2 g .. 2 g + 1
 *         of qh[32 h + i] above them.
 * The 6-bit (scale, min) unpacking is mps_backend.mm:284-293 (q4_k_scale_min).
 *
 * Pinning (tests/test_oracle_kquant.py): the reference smoke test's known
 * answers for one block of each format, matvec, two-token matmul, get-rows
 * with swapped row ids and the 65-row batched matmuls (smoke_test.cpp:875-1149);
 * an encode -> decode round trip through an independent numpy packer written
 * from the format description above, on random fields (every scale, min, quant
 * and high bit position exercised); single-quant blocks that must land at the
 * documented position; argmax known answers (smoke_test.cpp:1614-1638), ties,
 * NaN and -inf handling against a brute-force scan.
 */
#include "kraken_oracle.h"

#include <math.h>
#include <string.h>

size_t oracle_kquant_block_bytes(int format) {
  switch (format) {
    case ORACLE_Q4_K:
      return 144;
    case ORACLE_Q5_K:
      return 176;
    case ORACLE_Q6_K:
      return 210;
    default:
      return 0;
  }
}

static float f16_at(const uint8_t* p) {
  return oracle_f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
}

/* q4_k_scale_min, mps_backend.mm:284-293: 6-bit scale and min of sub-block j. */
static void scale_min(int j, const uint8_t* s, unsigned* sc, unsigned* m) {
  if (j < 4) {
    *sc = s[j] & 63u;
    *m = s[j + 4] & 63u;
  } else {
    *sc = (s[j + 4] & 0xFu) | ((unsigned)(s[j - 4] >> 6) << 4);
    *m = (unsigned)(s[j + 4] >> 4) | ((unsigned)(s[j] >> 6) << 4);
  }
}

/* q4_k_get_row / q5_k_get_row, mps_backend.mm:1448-1505. */
static void dequantize_q45(const uint8_t* b, int q5, float* y) {
  const float d = f16_at(b);
  const float dmin = f16_at(b + 2);
  const uint8_t* scales = b + 4;
  const uint8_t* qh = q5 ? b + 16 : NULL;
  const uint8_t* qs = b + (q5 ? 48 : 16);
  for (int s = 0; s < 4; ++s) {
    for (int half = 0; half < 2; ++half) {
      unsigned sc, m;
      scale_min(2 * s + half, scales, &sc, &m);
      const float ds = d * (float)sc;
      const float ms = dmin * (float)m;
      for (int i = 0; i < 32; ++i) {
        const unsigned packed = qs[32 * s + i];
        unsigned q = half == 0 ? (packed & 0xFu) : (packed >> 4);
        if (q5) {
          const unsigned mask = half == 0 ? (1u << (2 * s)) : (2u << (2 * s));
          q += (qh[i] & mask) != 0 ? 16u : 0u;
        }
        y[64 * s + 32 * half + i] = ds * (float)q - ms;
      }
    }
  }
}

/* q6_k_get_row, mps_backend.mm:1507-1540. */
static void dequantize_q6(const uint8_t* b, float* y) {
  const float d = f16_at(b + 208);
  for (int h = 0; h < 2; ++h) {
    const uint8_t* ql = b + 64 * h;
    const uint8_t* qh = b + 128 + 32 * h;
    const int8_t* scales = (const int8_t*)(b + 192 + 8 * h);
    for (int i = 0; i < 32; ++i) {
      const unsigned q1 = (ql[i] & 0xFu) | (((qh[i] >> 0) & 3u) << 4);
      const unsigned q2 = (ql[i + 32] & 0xFu) | (((qh[i] >> 2) & 3u) << 4);
      const unsigned q3 = (unsigned)(ql[i] >> 4) | (((qh[i] >> 4) & 3u) << 4);
      const unsigned q4 = (unsigned)(ql[i + 32] >> 4) | (((qh[i] >> 6) & 3u) << 4);
      const int is = i / 16;
      y[128 * h + i] = d * (float)scales[is + 0] * (float)((int)q1 - 32);
      y[128 * h + 32 + i] = d * (float)scales[is + 2] * (float)((int)q2 - 32);
      y[128 * h + 64 + i] = d * (float)scales[is + 4] * (float)((int)q3 - 32);
      y[128 * h + 96 + i] = d * (float)scales[is + 6] * (float)((int)q4 - 32);
    }
  }
}

void oracle_kquant_dequantize(int format, const uint8_t* data, size_t blocks, float* out) {
  const size_t bytes = oracle_kquant_block_bytes(format);
  for (size_t b = 0; b < blocks; ++b) {
    const uint8_t* block = data + b * bytes;
    float* y = out + 256 * b;
    if (format == ORACLE_Q6_K) {
      dequantize_q6(block, y);
    } else {
      dequantize_q45(block, format == ORACLE_Q5_K, y);
    }
  }
}

void oracle_kquant_matmul(int format, const uint8_t* weight, size_t rows, size_t cols,
                          const float* input, size_t tokens, int weight_f16, int input_f16,
                          float* out) {
  const size_t blocks = cols / 256;
  const size_t row_bytes = blocks * oracle_kquant_block_bytes(format);
  float w[256];
  for (size_t r = 0; r < rows; ++r) {
    for (size_t t = 0; t < tokens; ++t) {
      double acc = 0.0;
      for (size_t b = 0; b < blocks; ++b) {
        oracle_kquant_dequantize(format, weight + r * row_bytes + b * oracle_kquant_block_bytes(format),
                                 1, w);
        const float* x = input + t * cols + 256 * b;
        for (int i = 0; i < 256; ++i) {
          const float wi = weight_f16 ? oracle_f16_to_f32(oracle_f32_to_f16(w[i])) : w[i];
          const float xi = input_f16 ? oracle_f16_to_f32(oracle_f32_to_f16(x[i])) : x[i];
          acc += (double)wi * (double)xi;
        }
      }
      out[t * rows + r] = (float)acc;
    }
  }
}

/* argmax_f32_i32 / argmax_prob_f32_i32, mps_backend.mm:2681-2779: the first
 * index of the maximum (NaN never compares greater, so NaNs are skipped; with
 * no candidate the index is `size`); probability = 1 / sum exp(v - max) when
 * that sum is positive, else 0. */
int32_t oracle_argmax(const float* values, size_t size, float* probability) {
  size_t best = size;
  float best_value = -INFINITY;
  for (size_t i = 0; i < size; ++i) {
    const float v = values[i];
    if (v > best_value || (v == best_value && i < best)) {
      best_value = v;
      best = i;
    }
  }
  if (probability != NULL) {
    double sum = 0.0;
    for (size_t i = 0; i < size; ++i) {
      sum += exp((double)values[i] - (double)best_value);
    }
    *probability = sum > 0.0 ? (float)(1.0 / sum) : 0.0f;
  }
  return (int32_t)best;
}
