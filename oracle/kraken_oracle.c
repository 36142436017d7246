/*
 * kraken_oracle.c -- CPU restatement of the Qwen3.5 attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP backend, never a product
 * path.  Loaded by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg only.
 *
 * How each function is pinned (tests/test_oracle_golden.py and
 * tests/test_oracle_properties.py hold the checks):
 *   f16 conversions       -- exhaustive round trip of all 65536 bit patterns against
 *                            numpy.float16; RNE ties and overflow boundary cases.
 *   qk_norm, norm_gated   -- smoke_test.cpp:1211-1246 known answers.
 *   l2_norm, split_qkv    -- smoke_test.cpp:1281-1328 known answers.
 *   ssm_conv, conv state, -- smoke_test.cpp:1330-1400 known answers.
 *   ssm_conv1_stateful
 *   gated_delta_net       -- smoke_test.cpp:1402-1445 known answers (1 and 2 tokens),
 *                            :1447-1517 head_dim-128 vectors, plus closed forms
 *                            (beta=0 => pure decay; S=0,g=0,beta=1,k=e_i => y=v*q_i/sqrt(d)).
 *   mrope                 -- smoke_test.cpp:1255-1273 known answers; rotation preserves
 *                            pair norms; position 0 is the identity.
 *   sigmoid/softplus/silu,-- smoke_test.cpp:1547-1589 known answers.
 *   prepare_gate_beta
 *   copy rows (+to f16)   -- smoke_test.cpp:1598-1612 known answers.
 *   attention             -- smoke_test.cpp:1640-1725 known answers (single key, 2x3
 *                            causal batch, q=0 uniform average); brute force against an
 *                            independent numpy softmax; permutation/GQA invariants.
 *   qwen3_* legacy path   -- qk_norm/rope closed forms; attention equals the generic
 *                            attention on an fp32 cache (two implementations).
 */
#include "kraken_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- f16 ---- */

uint16_t oracle_f32_to_f16(float value) {
  uint32_t x;
  memcpy(&x, &value, sizeof(x));
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t absx = x & 0x7fffffffu;
  if (absx >= 0x7f800000u) { /* inf / nan */
    return (uint16_t)(sign | 0x7c00u | (absx > 0x7f800000u ? 0x0200u : 0u));
  }
  if (absx >= 0x477ff000u) { /* >= 65520 rounds to +-inf under RNE */
    return (uint16_t)(sign | 0x7c00u);
  }
  if (absx < 0x38800000u) { /* below 2^-14: binary16 subnormal, m * 2^-24 */
    float magnitude;
    memcpy(&magnitude, &absx, sizeof(magnitude));
    const float scaled = magnitude * 16777216.0f; /* exact power-of-two scaling */
    const uint32_t m = (uint32_t)nearbyintf(scaled); /* default rounding: RNE */
    return (uint16_t)(sign | m);
  }
  const uint32_t exponent = (absx >> 23) - 127u + 15u;
  const uint32_t mantissa = absx & 0x7fffffu;
  uint32_t h = (exponent << 10) | (mantissa >> 13);
  const uint32_t rest = mantissa & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) {
    h += 1u; /* a carry into the exponent field is the correct rounding */
  }
  return (uint16_t)(sign | h);
}

float oracle_f16_to_f32(uint16_t bits) {
  const uint32_t sign = ((uint32_t)bits & 0x8000u) << 16;
  const uint32_t exponent = ((uint32_t)bits >> 10) & 31u;
  const uint32_t mantissa = (uint32_t)bits & 1023u;
  uint32_t out;
  if (exponent == 0u) {
    const float magnitude = (float)mantissa * 5.9604644775390625e-8f; /* 2^-24 */
    float result = sign ? -magnitude : magnitude;
    return result;
  }
  if (exponent == 31u) {
    out = sign | 0x7f800000u | (mantissa << 13);
  } else {
    out = sign | ((exponent - 15u + 127u) << 23) | (mantissa << 13);
  }
  float result;
  memcpy(&result, &out, sizeof(result));
  return result;
}

void oracle_f32_to_f16_array(const float* src, uint16_t* dst, size_t count) {
  for (size_t i = 0; i < count; ++i) {
    dst[i] = oracle_f32_to_f16(src[i]);
  }
}

void oracle_f16_to_f32_array(const uint16_t* src, float* dst, size_t count) {
  for (size_t i = 0; i < count; ++i) {
    dst[i] = oracle_f16_to_f32(src[i]);
  }
}

static double sigmoid_d(double x) { return 1.0 / (1.0 + exp(-x)); }

/* ---------------------------------------------------------- norms ------ */

void oracle_qk_norm_f32_batched(float* values, const float* weight, size_t tokens,
                                size_t heads, size_t head_dim, float eps) {
  for (size_t t = 0; t < tokens; ++t) {
    for (size_t h = 0; h < heads; ++h) {
      float* x = values + (t * heads + h) * head_dim;
      double sum = 0.0;
      for (size_t d = 0; d < head_dim; ++d) {
        sum += (double)x[d] * (double)x[d];
      }
      const double scale = 1.0 / sqrt(sum / (double)head_dim + (double)eps);
      for (size_t d = 0; d < head_dim; ++d) {
        x[d] = (float)((double)x[d] * scale * (double)weight[d]);
      }
    }
  }
}

void oracle_norm_gated_f32(float* values, const float* weight, const float* gate,
                           size_t tokens, size_t heads, size_t head_dim, float eps) {
  for (size_t t = 0; t < tokens; ++t) {
    for (size_t h = 0; h < heads; ++h) {
      const size_t base = (t * heads + h) * head_dim;
      double sum = 0.0;
      for (size_t d = 0; d < head_dim; ++d) {
        sum += (double)values[base + d] * (double)values[base + d];
      }
      const double scale = 1.0 / sqrt(sum / (double)head_dim + (double)eps);
      for (size_t d = 0; d < head_dim; ++d) {
        const double z = gate[base + d];
        const double silu = z * sigmoid_d(z);
        values[base + d] = (float)((double)values[base + d] * scale * (double)weight[d] * silu);
      }
    }
  }
}

void oracle_l2_norm_f32(float* values, size_t rows, size_t row_size, float eps) {
  for (size_t r = 0; r < rows; ++r) {
    float* x = values + r * row_size;
    double sum = 0.0;
    for (size_t d = 0; d < row_size; ++d) {
      sum += (double)x[d] * (double)x[d];
    }
    double norm = sqrt(sum);
    if (norm < (double)eps) {
      norm = (double)eps;
    }
    for (size_t d = 0; d < row_size; ++d) {
      x[d] = (float)((double)x[d] / norm);
    }
  }
}

void oracle_split_qkv_l2_norm(const float* source, float* query, float* key, float* value,
                              size_t tokens, size_t key_heads, size_t value_heads,
                              size_t head_dim, float eps) {
  const size_t key_dim = key_heads * head_dim;
  const size_t channels = 2u * key_dim + value_heads * head_dim;
  for (size_t t = 0; t < tokens; ++t) {
    const float* row = source + t * channels;
    for (size_t part = 0; part < 2; ++part) {
      float* dst = part == 0 ? query : key;
      for (size_t h = 0; h < key_heads; ++h) {
        const float* x = row + part * key_dim + h * head_dim;
        double sum = 0.0;
        for (size_t d = 0; d < head_dim; ++d) {
          sum += (double)x[d] * (double)x[d];
        }
        double norm = sqrt(sum);
        if (norm < (double)eps) {
          norm = (double)eps;
        }
        float* y = dst + (t * key_heads + h) * head_dim;
        for (size_t d = 0; d < head_dim; ++d) {
          y[d] = (float)((double)x[d] / norm);
        }
      }
    }
    for (size_t h = 0; h < value_heads; ++h) {
      memcpy(value + (t * value_heads + h) * head_dim, row + 2u * key_dim + h * head_dim,
             head_dim * sizeof(float));
    }
  }
}

/* ------------------------------------------------------- gated delta --- */

void oracle_gated_delta_net(const float* query, const float* key, const float* value,
                            const float* gate, const float* beta, float* state,
                            size_t tokens, size_t key_heads, size_t value_heads,
                            size_t head_dim, float* output) {
  const double scale = 1.0 / sqrt((double)head_dim);
  for (size_t h = 0; h < value_heads; ++h) {
    const size_t kh = h % key_heads;
    float* s_head = state + h * head_dim * head_dim;
    for (size_t t = 0; t < tokens; ++t) {
      const float* q = query + (t * key_heads + kh) * head_dim;
      const float* k = key + (t * key_heads + kh) * head_dim;
      const float* v = value + (t * value_heads + h) * head_dim;
      const double decay = exp((double)gate[t * value_heads + h]);
      const double b = beta[t * value_heads + h];
      float* y = output + (t * value_heads + h) * head_dim;
      for (size_t r = 0; r < head_dim; ++r) {
        float* s = s_head + r * head_dim;
        double sk = 0.0;
        for (size_t c = 0; c < head_dim; ++c) {
          s[c] = (float)((double)s[c] * decay);
          sk += (double)s[c] * (double)k[c];
        }
        const double delta = ((double)v[r] - sk) * b;
        double acc = 0.0;
        for (size_t c = 0; c < head_dim; ++c) {
          s[c] = (float)((double)s[c] + (double)k[c] * delta);
          acc += (double)s[c] * (double)q[c];
        }
        y[r] = (float)(acc * scale);
      }
    }
  }
}

/* ----------------------------------------------------------- conv ------ */

void oracle_ssm_conv(const float* input, const float* kernel, size_t conv_kernel,
                     size_t channels, size_t tokens, size_t sequences, float* output) {
  const size_t span = conv_kernel - 1u + tokens;
  for (size_t s = 0; s < sequences; ++s) {
    for (size_t t = 0; t < tokens; ++t) {
      for (size_t c = 0; c < channels; ++c) {
        const float* x = input + (s * channels + c) * span + t;
        const float* w = kernel + c * conv_kernel;
        double sum = 0.0;
        for (size_t j = 0; j < conv_kernel; ++j) {
          sum += (double)x[j] * (double)w[j];
        }
        output[(s * tokens + t) * channels + c] = (float)sum;
      }
    }
  }
}

void oracle_ssm_conv1_stateful(float* state, const float* input, const float* kernel,
                               size_t conv_kernel, size_t channels, float* output) {
  const size_t width = conv_kernel - 1u;
  for (size_t c = 0; c < channels; ++c) {
    float* st = state + c * width;
    const float* w = kernel + c * conv_kernel;
    double sum = 0.0;
    for (size_t j = 0; j < width; ++j) {
      sum += (double)st[j] * (double)w[j];
    }
    sum += (double)input[c] * (double)w[width];
    for (size_t j = 0; j + 1u < width; ++j) {
      st[j] = st[j + 1u];
    }
    st[width - 1u] = input[c];
    output[c] = (float)sum;
  }
}

void oracle_build_ssm_conv_state(float* state, const float* input, size_t conv_kernel,
                                 size_t channels, size_t tokens, float* conv_input) {
  const size_t width = conv_kernel - 1u;
  const size_t span = width + tokens;
  for (size_t c = 0; c < channels; ++c) {
    float* st = state + c * width;
    float* ci = conv_input + c * span;
    for (size_t j = 0; j < width; ++j) {
      ci[j] = st[j];
    }
    for (size_t t = 0; t < tokens; ++t) {
      ci[width + t] = input[t * channels + c];
    }
    /* The new state is the last K-1 entries of [old state | chunk]. */
    for (size_t j = 0; j < width; ++j) {
      st[j] = ci[tokens + j];
    }
  }
}

/* ----------------------------------------------------------- rope ------ */

void oracle_mrope_f32(float* values, const int32_t* positions, size_t tokens, size_t heads,
                      size_t head_dim, size_t n_dims, size_t section_0, size_t section_1,
                      size_t section_2, size_t section_3, float theta) {
  const size_t half_dims = n_dims / 2u;
  const size_t sections = section_0 + section_1 + section_2 + section_3;
  if (sections == 0) {
    return;
  }
  for (size_t t = 0; t < tokens; ++t) {
    for (size_t h = 0; h < heads; ++h) {
      float* x = values + (t * heads + h) * head_dim;
      for (size_t i = 0; i < half_dims; ++i) {
        const size_t sector = i % sections;
        size_t row = 3;
        if (sector < section_0) {
          row = 0;
        } else if (sector < section_0 + section_1) {
          row = 1;
        } else if (sector < section_0 + section_1 + section_2) {
          row = 2;
        }
        const double position = (double)positions[t + tokens * row];
        const double freq = 1.0 / pow((double)theta, (double)(2u * i) / (double)n_dims);
        const double angle = position * freq;
        const double c = cos(angle);
        const double s = sin(angle);
        const double x0 = x[i];
        const double x1 = x[half_dims + i];
        x[i] = (float)(x0 * c - x1 * s);
        x[half_dims + i] = (float)(x1 * c + x0 * s);
      }
    }
  }
}

void oracle_make_mrope_positions(int32_t* positions, size_t start_position, size_t tokens) {
  for (size_t row = 0; row < 4u; ++row) {
    for (size_t t = 0; t < tokens; ++t) {
      positions[t + tokens * row] = (int32_t)(start_position + t);
    }
  }
}

/* ---------------------------------------------------- elementwise ------ */

void oracle_sigmoid_f32(float* values, size_t size) {
  for (size_t i = 0; i < size; ++i) {
    values[i] = (float)sigmoid_d(values[i]);
  }
}

static double softplus_d(double x) { return x > 20.0 ? x : log1p(exp(x)); }

void oracle_softplus_f32(float* values, size_t size) {
  for (size_t i = 0; i < size; ++i) {
    values[i] = (float)softplus_d(values[i]);
  }
}

void oracle_silu_f32(float* values, size_t size) {
  for (size_t i = 0; i < size; ++i) {
    const double x = values[i];
    values[i] = (float)(x * sigmoid_d(x));
  }
}

void oracle_mul_f32(float* target, const float* rhs, size_t size) {
  for (size_t i = 0; i < size; ++i) {
    target[i] = target[i] * rhs[i];
  }
}

void oracle_add_f32(float* target, const float* delta, size_t size) {
  for (size_t i = 0; i < size; ++i) {
    target[i] = target[i] + delta[i];
  }
}

void oracle_silu_mul_f32(float* gate, const float* up, size_t size) {
  for (size_t i = 0; i < size; ++i) {
    const double g = gate[i];
    gate[i] = (float)(g * sigmoid_d(g) * (double)up[i]);
  }
}

void oracle_prepare_gdn_gate_beta(float* gate, float* beta, const float* gate_bias,
                                  const float* gate_scale, size_t rows, size_t row_size) {
  for (size_t r = 0; r < rows; ++r) {
    for (size_t c = 0; c < row_size; ++c) {
      const size_t i = r * row_size + c;
      const double g = (double)gate[i] + (double)gate_bias[c];
      gate[i] = (float)(softplus_d(g) * (double)gate_scale[c]);
      beta[i] = (float)sigmoid_d(beta[i]);
    }
  }
}

void oracle_copy_f32_rows(const float* source, float* destination, size_t rows,
                          size_t row_size, size_t source_stride, size_t source_offset,
                          size_t destination_stride, size_t destination_offset) {
  for (size_t r = 0; r < rows; ++r) {
    memcpy(destination + destination_offset + r * destination_stride,
           source + source_offset + r * source_stride, row_size * sizeof(float));
  }
}

void oracle_copy_f32_rows_to_f16(const float* source, uint16_t* destination, size_t rows,
                                 size_t row_size, size_t source_stride, size_t source_offset,
                                 size_t destination_stride, size_t destination_offset) {
  for (size_t r = 0; r < rows; ++r) {
    for (size_t c = 0; c < row_size; ++c) {
      destination[destination_offset + r * destination_stride + c] =
        oracle_f32_to_f16(source[source_offset + r * source_stride + c]);
    }
  }
}

/* ------------------------------------------------------- attention ----- */

static double cache_value(const void* cache, int kv_f16, size_t index) {
  if (kv_f16) {
    return (double)oracle_f16_to_f32(((const uint16_t*)cache)[index]);
  }
  return (double)((const float*)cache)[index];
}

void oracle_attention_batched(const float* query, const void* key_cache,
                              const void* value_cache, int kv_f16, size_t layer,
                              size_t start_position, size_t tokens, size_t capacity_tokens,
                              size_t heads, size_t kv_heads, size_t head_dim,
                              int round_query_f16, float* output) {
  const size_t group = heads / kv_heads;
  const size_t kv_dim = kv_heads * head_dim;
  const double scale = (double)(1.0f / sqrtf((float)head_dim));
  double* scores = (double*)malloc((start_position + tokens) * sizeof(double));
  double* acc = (double*)malloc(head_dim * sizeof(double));
  double* q = (double*)malloc(head_dim * sizeof(double));
  for (size_t t = 0; t < tokens; ++t) {
    const size_t position = start_position + t;
    for (size_t h = 0; h < heads; ++h) {
      const size_t kvh = h / group;
      const float* qrow = query + (t * heads + h) * head_dim;
      for (size_t d = 0; d < head_dim; ++d) {
        q[d] = round_query_f16 ? (double)oracle_f16_to_f32(oracle_f32_to_f16(qrow[d]))
                               : (double)qrow[d];
      }
      double max_score = -INFINITY;
      for (size_t j = 0; j <= position; ++j) {
        const size_t base = (layer * capacity_tokens + j) * kv_dim + kvh * head_dim;
        double s = 0.0;
        for (size_t d = 0; d < head_dim; ++d) {
          s += q[d] * cache_value(key_cache, kv_f16, base + d);
        }
        s *= scale;
        scores[j] = s;
        if (s > max_score) {
          max_score = s;
        }
      }
      double denom = 0.0;
      for (size_t d = 0; d < head_dim; ++d) {
        acc[d] = 0.0;
      }
      for (size_t j = 0; j <= position; ++j) {
        const double w = exp(scores[j] - max_score);
        denom += w;
        const size_t base = (layer * capacity_tokens + j) * kv_dim + kvh * head_dim;
        for (size_t d = 0; d < head_dim; ++d) {
          acc[d] += w * cache_value(value_cache, kv_f16, base + d);
        }
      }
      float* out = output + (t * heads + h) * head_dim;
      for (size_t d = 0; d < head_dim; ++d) {
        out[d] = denom == 0.0 ? 0.0f : (float)(acc[d] / denom);
      }
    }
  }
  free(q);
  free(acc);
  free(scores);
}

void oracle_sigmoid_gate_mul(float* output, const float* gate, size_t size) {
  for (size_t i = 0; i < size; ++i) {
    output[i] = (float)((double)output[i] * sigmoid_d(gate[i]));
  }
}

/* -------------------------------------------- legacy Qwen3 CPU path ---- */

void oracle_qwen3_qk_norm(float* values, size_t heads, size_t head_dim, const float* weight,
                          double eps) {
  for (size_t head = 0; head < heads; ++head) {
    double mean_square = 0.0;
    const size_t base = head * head_dim;
    for (size_t i = 0; i < head_dim; ++i) {
      mean_square += (double)values[base + i] * values[base + i];
    }
    mean_square /= (double)head_dim;
    const float scale = (float)(1.0 / sqrt(mean_square + eps));
    for (size_t i = 0; i < head_dim; ++i) {
      values[base + i] *= scale * weight[i];
    }
  }
}

void oracle_qwen3_rope(float* values, size_t heads, size_t head_dim, size_t position,
                       double theta) {
  const size_t half_dim = head_dim / 2u;
  for (size_t head = 0; head < heads; ++head) {
    const size_t base = head * head_dim;
    for (size_t i = 0; i < half_dim; ++i) {
      const double freq = 1.0 / pow(theta, (double)(2u * i) / (double)head_dim);
      const double angle = (double)position * freq;
      const float cos_v = (float)cos(angle);
      const float sin_v = (float)sin(angle);
      const float x0 = values[base + i];
      const float x1 = values[base + half_dim + i];
      values[base + i] = x0 * cos_v - x1 * sin_v;
      values[base + half_dim + i] = x1 * cos_v + x0 * sin_v;
    }
  }
}

void oracle_qwen3_attention(const float* key_cache, const float* value_cache,
                            size_t capacity_tokens, size_t layer, size_t position,
                            const float* query, size_t heads, size_t kv_heads,
                            size_t head_dim, float* output) {
  const size_t group = heads / kv_heads;
  const size_t kv_dim = kv_heads * head_dim;
  const float scale = 1.0f / sqrtf((float)head_dim);
  float* scores = (float*)malloc((position + 1u) * sizeof(float));
  for (size_t head = 0; head < heads; ++head) {
    const size_t kv_head = head / group;
    const size_t q_base = head * head_dim;
    float max_score = -INFINITY;
    for (size_t t = 0; t <= position; ++t) {
      const float* key = key_cache + (layer * capacity_tokens + t) * kv_dim + kv_head * head_dim;
      float score = 0.0f;
      for (size_t d = 0; d < head_dim; ++d) {
        score += query[q_base + d] * key[d];
      }
      score *= scale;
      scores[t] = score;
      max_score = score > max_score ? score : max_score;
    }
    float denom = 0.0f;
    for (size_t t = 0; t <= position; ++t) {
      scores[t] = expf(scores[t] - max_score);
      denom += scores[t];
    }
    for (size_t d = 0; d < head_dim; ++d) {
      float value = 0.0f;
      for (size_t t = 0; t <= position; ++t) {
        const float* cached =
          value_cache + (layer * capacity_tokens + t) * kv_dim + kv_head * head_dim;
        value += (scores[t] / denom) * cached[d];
      }
      output[q_base + d] = value;
    }
  }
  free(scores);
}

int oracle_qwen3_attention_sequence(const float* q_raw, const float* k_raw,
                                    const float* v_raw, size_t positions, size_t heads,
                                    size_t kv_heads, size_t head_dim, const float* q_norm_w,
                                    const float* k_norm_w, double eps, double theta,
                                    float* key_cache, float* value_cache, float* q_out,
                                    float* output) {
  const size_t attn_dim = heads * head_dim;
  const size_t kv_dim = kv_heads * head_dim;
  float* k = (float*)malloc(kv_dim * sizeof(float));
  for (size_t p = 0; p < positions; ++p) {
    float* q = q_out + p * attn_dim;
    memcpy(q, q_raw + p * attn_dim, attn_dim * sizeof(float));
    memcpy(k, k_raw + p * kv_dim, kv_dim * sizeof(float));
    oracle_qwen3_qk_norm(q, heads, head_dim, q_norm_w, eps);
    oracle_qwen3_qk_norm(k, kv_heads, head_dim, k_norm_w, eps);
    oracle_qwen3_rope(q, heads, head_dim, p, theta);
    oracle_qwen3_rope(k, kv_heads, head_dim, p, theta);
    memcpy(key_cache + p * kv_dim, k, kv_dim * sizeof(float));
    memcpy(value_cache + p * kv_dim, v_raw + p * kv_dim, kv_dim * sizeof(float));
    oracle_qwen3_attention(key_cache, value_cache, positions, 0, p, q, heads, kv_heads,
                           head_dim, output + p * attn_dim);
  }
  free(k);
  return 0;
}
