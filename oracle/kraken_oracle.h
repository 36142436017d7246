/*
 * kraken_oracle.h -- CPU restatement of the Qwen3.5 attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP
 * backend: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.  No product code path links it or falls back to it.
 *
 * Every function restates one reference operation; the citation next to each
 * declaration names the file:line of /root/reference it follows.  Layouts are
 * the reference's (row-major, element offsets, fp16 as raw IEEE binary16 bits).
 *
 * Precision policy: reductions (dot products, sums of squares, softmax
 * denominators) are accumulated in double so the oracle is at least as accurate
 * as the fp32 Metal kernels it restates; state tensors stay fp32 where the
 * reference keeps them fp32 (GDN state, conv state).  The legacy Qwen3 CPU path
 * (qwen3_*) is restated operation for operation in float/double exactly as the
 * reference writes it, because it doubles as the timed CPU baseline.
 *
 * Pinning (what checks each function beyond its own formula) is listed in the
 * header comment of oracle/kraken_oracle.c.
 */
#ifndef KRAKEN_ORACLE_H
#define KRAKEN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE binary16 conversions, round-to-nearest-even (Metal half(x), mps_backend.mm:2665). */
uint16_t oracle_f32_to_f16(float value);
float oracle_f16_to_f32(uint16_t bits);
void oracle_f32_to_f16_array(const float* src, uint16_t* dst, size_t count);
void oracle_f16_to_f32_array(const uint16_t* src, float* dst, size_t count);

/* qk_norm_f32_f32_batched, mps_backend.mm:1991-2024 (also rms_norm of GDN output,
 * qwen35_runtime.cpp:2999-3001).  values [tokens][heads][head_dim] in place. */
void oracle_qk_norm_f32_batched(float* values, const float* weight, size_t tokens,
                                size_t heads, size_t head_dim, float eps);

/* qwen35_norm_gated_f32_in_place, mps_backend.mm:2026-2063: RMSNorm * w * silu(gate). */
void oracle_norm_gated_f32(float* values, const float* weight, const float* gate,
                           size_t tokens, size_t heads, size_t head_dim, float eps);

/* l2_norm_f32_in_place, mps_backend.mm:2065-2095: x / max(||x||, eps). */
void oracle_l2_norm_f32(float* values, size_t rows, size_t row_size, float eps);

/* split_qkv_l2_norm_f32_qwen35, mps_backend.mm:2097-2153. source [tokens][2*Hk*D + Hv*D]. */
void oracle_split_qkv_l2_norm(const float* source, float* query, float* key, float* value,
                              size_t tokens, size_t key_heads, size_t value_heads,
                              size_t head_dim, float eps);

/* gated_delta_net_f32_batched_qwen35 / _batched_in_place, mps_backend.mm:2225-2374.
 * state [value_heads][head_dim rows (v)][head_dim cols (k)], key_head = head % key_heads. */
void oracle_gated_delta_net(const float* query, const float* key, const float* value,
                            const float* gate, const float* beta, float* state,
                            size_t tokens, size_t key_heads, size_t value_heads,
                            size_t head_dim, float* output);

/* ssm_conv_f32, mps_backend.mm:2376-2400.  input [sequences][channels][K-1+tokens],
 * kernel [channels][K], output [sequences][tokens][channels]. */
void oracle_ssm_conv(const float* input, const float* kernel, size_t conv_kernel,
                     size_t channels, size_t tokens, size_t sequences, float* output);

/* ssm_conv1_f32_stateful, mps_backend.mm:2402-2426 (single-token conv with state shift). */
void oracle_ssm_conv1_stateful(float* state, const float* input, const float* kernel,
                               size_t conv_kernel, size_t channels, float* output);

/* build_ssm_conv_state_f32, mps_backend.mm:2428-2457.  state [channels][K-1],
 * input [tokens][channels], conv_input [channels][K-1+tokens]. */
void oracle_build_ssm_conv_state(float* state, const float* input, size_t conv_kernel,
                                 size_t channels, size_t tokens, float* conv_input);

/* mrope_f32_in_place, mps_backend.mm:2482-2527.  positions int32 [4][tokens]. */
void oracle_mrope_f32(float* values, const int32_t* positions, size_t tokens, size_t heads,
                      size_t head_dim, size_t n_dims, size_t section_0, size_t section_1,
                      size_t section_2, size_t section_3, float theta);

/* Qwen3.5 text MRoPE positions, qwen35_runtime.cpp:1848-1877: all 4 rows = start + token. */
void oracle_make_mrope_positions(int32_t* positions, size_t start_position, size_t tokens);

/* Elementwise ops, mps_backend.mm:2539-2618. */
void oracle_sigmoid_f32(float* values, size_t size);
void oracle_softplus_f32(float* values, size_t size);
void oracle_silu_f32(float* values, size_t size);
void oracle_mul_f32(float* target, const float* rhs, size_t size);
/* add_f32_in_place (mps_backend.mm:2529-2537): target += delta. */
void oracle_add_f32(float* target, const float* delta, size_t size);
/* silu_mul_f32_in_place (mps_backend.mm:2620-2629): gate = silu(gate) * up. */
void oracle_silu_mul_f32(float* gate, const float* up, size_t size);
void oracle_prepare_gdn_gate_beta(float* gate, float* beta, const float* gate_bias,
                                  const float* gate_scale, size_t rows, size_t row_size);

/* copy_f32_rows / copy_f32_rows_to_f16, mps_backend.mm:2639-2666. */
void oracle_copy_f32_rows(const float* source, float* destination, size_t rows,
                          size_t row_size, size_t source_stride, size_t source_offset,
                          size_t destination_stride, size_t destination_offset);
void oracle_copy_f32_rows_to_f16(const float* source, uint16_t* destination, size_t rows,
                                 size_t row_size, size_t source_stride, size_t source_offset,
                                 size_t destination_stride, size_t destination_offset);

/* Causal GQA attention over a KV cache [layers][capacity][kv_heads][head_dim],
 * mps_backend.mm:2943-3008 (online, f32 Q) and 3398-3643 (flash256, Q rounded to
 * f16 first when round_query_f16 != 0).  Query token t sits at position
 * start_position + t and attends keys 0..position; kv_head = head / (heads / kv_heads);
 * scale = 1/sqrt(head_dim).  kv_f16 selects the cache element type (uint16_t or float). */
void oracle_attention_batched(const float* query, const void* key_cache,
                              const void* value_cache, int kv_f16, size_t layer,
                              size_t start_position, size_t tokens, size_t capacity_tokens,
                              size_t heads, size_t kv_heads, size_t head_dim,
                              int round_query_f16, float* output);

/* Output gate of the full-attention layer, qwen35_runtime.cpp:3347-3355:
 * out *= sigmoid(gate). */
void oracle_sigmoid_gate_mul(float* output, const float* gate, size_t size);

/* Legacy Qwen3 CPU path, restated op for op from src/runtime/cpu/qwen_cpu_model.cpp. */
/* qk_norm, qwen_cpu_model.cpp:1019-1033 (mean square in double). values [heads][head_dim]. */
void oracle_qwen3_qk_norm(float* values, size_t heads, size_t head_dim, const float* weight,
                          double eps);
/* apply_rope, qwen_cpu_model.cpp:1035-1053 (angles in double, half-split pairs). */
void oracle_qwen3_rope(float* values, size_t heads, size_t head_dim, size_t position,
                       double theta);
/* attention, qwen_cpu_model.cpp:1074-1130 over KvCache layout kv_cache.cpp:85-87. */
void oracle_qwen3_attention(const float* key_cache, const float* value_cache,
                            size_t capacity_tokens, size_t layer, size_t position,
                            const float* query, size_t heads, size_t kv_heads,
                            size_t head_dim, float* output);
/* One layer's attention over a token sequence, as apply_layer drives it
 * (qwen_cpu_model.cpp:914-940): per position, qk_norm(q,k) -> rope(q,k) ->
 * store_kv -> attention.  q_raw [positions][heads][D], k_raw/v_raw
 * [positions][kv_heads][D]; key/value caches [positions][kv_heads][D] are written;
 * q_out receives the normed+roped query, out the attention output.  Returns 0. */
int oracle_qwen3_attention_sequence(const float* q_raw, const float* k_raw,
                                    const float* v_raw, size_t positions, size_t heads,
                                    size_t kv_heads, size_t head_dim, const float* q_norm_w,
                                    const float* k_norm_w, double eps, double theta,
                                    float* key_cache, float* value_cache, float* q_out,
                                    float* output);

/* K-quant projections and argmax (oracle/kquant_oracle.c).  Formats: */
enum { ORACLE_Q4_K = 0, ORACLE_Q5_K = 1, ORACLE_Q6_K = 2 };
/* Bytes per 256-value block: 144, 176, 210 (0 for an unknown format). */
size_t oracle_kquant_block_bytes(int format);
/* q4_k/q5_k/q6_k_get_row, mps_backend.mm:1448-1540: `blocks` consecutive blocks
 * into 256 * blocks floats, in the reference's float arithmetic. */
void oracle_kquant_dequantize(int format, const uint8_t* data, size_t blocks, float* out);
/* matvec / matmul (mps_backend.mm:295-460, 1268-1440): out[t][r] =
 * sum_c w[r][c] x[t][c], accumulated in double; weight rows of cols/256 blocks.
 * weight_f16 / input_f16 round each dequantized weight / input to binary16
 * first (the reference's many-token mul_mm path, mps_backend.mm:1082-1230). */
void oracle_kquant_matmul(int format, const uint8_t* weight, size_t rows, size_t cols,
                          const float* input, size_t tokens, int weight_f16, int input_f16,
                          float* out);
/* argmax_f32_i32 / argmax_prob_f32_i32, mps_backend.mm:2681-2779 (probability
 * may be NULL). */
int32_t oracle_argmax(const float* values, size_t size, float* probability);

#ifdef __cplusplus
}
#endif

#endif /* KRAKEN_ORACLE_H */
