/*
 * kraken_hip.h -- C ABI of the MI355X (gfx950) backend for the Qwen3.5
 * attention hot path of kraken-infer.
 *
 * This is the thin C layer under the backend interface.  Each entry point
 * replaces one operation of toyllm::mps::MpsContext
 * (reference: include/toyllm/backends/mps/mps_backend.hpp:76-428); the comment
 * on each declaration cites the method it replaces and its Metal
 * implementation.  Semantics carried over from the reference:
 *
 *  - Status codes keep the order of toyllm::StatusCode
 *    (include/toyllm/core/status.hpp:8-13).  Every call returns one; a non-OK
 *    call leaves a message readable with kraken_hip_last_error() on the calling
 *    thread (the C counterpart of Status::message()).  Nothing throws across
 *    this boundary.
 *  - Argument checks run in the reference's order (mps_backend.mm:10625-10713):
 *    context valid -> dimensions positive / divisible / bounded -> capacity ->
 *    size_t overflow -> each buffer initialized and large enough -> every
 *    parameter fits uint32.  A failed check returns KRAKEN_INVALID_ARGUMENT.
 *  - Buffers are caller-owned device allocations described by a non-owning
 *    {data, byte_size} view (the reference's MpsBuffer, mps_backend.hpp:26-47).
 *    data == NULL means "not initialized".  Ops never allocate caller-visible
 *    memory; "_at" variants take element offsets into caller buffers.
 *  - Synchronisation (mps_backend.mm:4416-4467): outside begin_graph/commit_graph
 *    every op is enqueued on the context's stream and waited for; inside, ops are
 *    only enqueued and commit_graph waits once.  Host copies wait for pending work.
 *  - A context is used by one thread at a time; contexts are independent.
 *
 * Everything here is plain C: pointers, sizes, floats.  No torch or HIP types
 * cross the boundary (streams travel as void*).
 */
#ifndef KRAKEN_HIP_H
#define KRAKEN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define KRAKEN_API __attribute__((visibility("default")))
#else
#define KRAKEN_API
#endif

/* toyllm::StatusCode, include/toyllm/core/status.hpp:8-13 (same order). */
typedef enum kraken_status {
  KRAKEN_OK = 0,
  KRAKEN_INVALID_ARGUMENT = 1,
  KRAKEN_UNAVAILABLE = 2,
  KRAKEN_INTERNAL_ERROR = 3
} kraken_status;

/* Non-owning view of device memory; stands in for toyllm::mps::MpsBuffer
 * (mps_backend.hpp:26-47): valid() == (data != NULL), byte_size() == byte_size. */
typedef struct kraken_buffer {
  void* data;
  size_t byte_size;
} kraken_buffer;

typedef struct kraken_hip_context kraken_hip_context;

/* ------------------------------------------------------------ context ---- */

/* MpsContext::create (mps_backend.hpp:87; mps_backend.mm:5043-5085).  Binds the
 * current HIP device and creates the context's stream.  KRAKEN_UNAVAILABLE when no
 * HIP device is present (the stub backend's answer, mps_backend_stub.cpp:52-54). */
KRAKEN_API int kraken_hip_context_create(kraken_hip_context** out_context);

/* A context with no device, for host-side tests of argument checking: every op runs
 * its full validation and, when the arguments are accepted, returns
 * KRAKEN_UNAVAILABLE with the message "validation-only context: arguments accepted"
 * instead of launching.  It never computes anything.  No reference counterpart
 * (the reference checks arguments only on a live Metal device). */
KRAKEN_API int kraken_hip_context_create_validation_only(kraken_hip_context** out_context);

/* ~MpsContext (mps_backend.mm:4461-4467).  Aborts an open graph. */
KRAKEN_API void kraken_hip_context_destroy(kraken_hip_context* context);

/* Enqueue on a caller-owned hipStream_t (passed as void*) instead of the
 * context's own stream; NULL restores the context's stream.  No reference
 * counterpart (Metal owns its command queue, mps_backend.mm:4330-4332). */
KRAKEN_API int kraken_hip_context_set_stream(kraken_hip_context* context, void* hip_stream);
KRAKEN_API void* kraken_hip_context_stream(const kraken_hip_context* context);

/* Status::message() of the last non-OK call on this thread ("" if none). */
KRAKEN_API const char* kraken_hip_last_error(void);

/* MpsContext::begin_graph / commit_graph / abort_graph (mps_backend.hpp:90-94;
 * mps_backend.mm:4430-4459).  begin while active -> KRAKEN_INVALID_ARGUMENT;
 * commit without begin -> KRAKEN_OK. */
KRAKEN_API int kraken_hip_begin_graph(kraken_hip_context* context);
KRAKEN_API int kraken_hip_commit_graph(kraken_hip_context* context);
KRAKEN_API void kraken_hip_abort_graph(kraken_hip_context* context);

/* MpsContext::make_buffer (mps_backend.hpp:96): device allocation owned by the caller
 * until kraken_hip_free_buffer. */
KRAKEN_API int kraken_hip_make_buffer(kraken_hip_context* context, size_t byte_size,
                                      kraken_buffer* out_buffer);
KRAKEN_API int kraken_hip_free_buffer(kraken_hip_context* context, kraken_buffer* buffer);

/* MpsContext::copy_to_buffer[_at] / copy_from_buffer[_at] / copy_buffer_region /
 * zero_buffer (mps_backend.hpp:97-114; mps_backend.mm:5763-5874).  Host copies
 * first finish pending work, as the reference commits the open graph.
 * copy_buffer_region also commits first, then enqueues the device copy on the
 * context's stream and waits for it; overlapping ranges copy as memmove, staged
 * through the context's workspace (which grows once, then is reused). */
KRAKEN_API int kraken_hip_copy_to_buffer(kraken_hip_context* context, kraken_buffer buffer,
                                         const void* data, size_t byte_size);
KRAKEN_API int kraken_hip_copy_to_buffer_at(kraken_hip_context* context, kraken_buffer buffer,
                                            size_t destination_offset, const void* data,
                                            size_t byte_size);
KRAKEN_API int kraken_hip_copy_from_buffer(kraken_hip_context* context, kraken_buffer buffer,
                                           void* data, size_t byte_size);
KRAKEN_API int kraken_hip_copy_from_buffer_at(kraken_hip_context* context,
                                              kraken_buffer buffer, size_t source_offset,
                                              void* data, size_t byte_size);
KRAKEN_API int kraken_hip_copy_buffer_region(kraken_hip_context* context, kraken_buffer source,
                                             kraken_buffer destination, size_t source_offset,
                                             size_t destination_offset, size_t byte_size);
KRAKEN_API int kraken_hip_zero_buffer(kraken_hip_context* context, kraken_buffer buffer,
                                      size_t byte_size);

/* Many byte ranges from one buffer to another in one launch (no counterpart in
 * the reference, which copies range by range; the prefix cache store uses it to
 * move a block's rows of every layer at once).  `regions` is a host array of
 * `count` triples {source_offset, destination_offset, byte_size}; count is at
 * most KRAKEN_COPY_REGIONS_MAX and every range must lie inside its buffer.
 * Ranges must not overlap each other's destinations or a source they read.
 * Enqueued on the context's stream with no allocation; like the other ops it
 * waits for completion unless a begin_graph / commit_graph batch is open. */
#define KRAKEN_COPY_REGIONS_MAX 64
typedef struct kraken_copy_region {
  size_t source_offset;
  size_t destination_offset;
  size_t byte_size;
} kraken_copy_region;
KRAKEN_API int kraken_hip_copy_regions(kraken_hip_context* context, kraken_buffer source,
                                       kraken_buffer destination,
                                       const kraken_copy_region* regions, size_t count);

/* ------------------------------------------------------- attention ------ */

/* MpsContext::attention_f32_batched_f16_kv (mps_backend.hpp:415-420;
 * mps_backend.mm:10619-10869).  query f32 [tokens][heads][head_dim]; key/value cache
 * f16 [layers][capacity_tokens][kv_heads][head_dim]; output f32 like query.  Query
 * token t sits at position start_position + t and attends cache keys 0..position of
 * `layer` (causal; the chunk's own K/V must already be in the cache).
 * Dispatch: head_dim 256 with tokens >= 64 runs the flash256 MFMA prefill kernel
 * (Q rounded to f16, as mps_backend.mm:3458-3461); otherwise the split-K decode
 * kernel (f32 Q, mps_backend.mm:2943-3008).  KRAKEN_QWEN35_FLASH_ATTENTION=0/1
 * forces the choice like mps_backend.mm:3716-3733. */
KRAKEN_API int kraken_hip_attention_f32_batched_f16_kv(
  kraken_hip_context* context, kraken_buffer query, kraken_buffer key_cache,
  kraken_buffer value_cache, size_t layer, size_t start_position, size_t tokens,
  size_t capacity_tokens, size_t heads, size_t kv_heads, size_t head_dim,
  kraken_buffer output);

/* attention_f32_batched_f16_kv with an f16 query: query holds f16 values
 * [tokens][heads][head_dim].  No single MpsContext method corresponds: the
 * reference's flash path rounds its f32 query to f16 on load
 * (mps_backend.mm:3458-3461), and this entry takes queries that are f16
 * already (the C2 prefill inputs are fp16), so the flash kernel reads half the
 * query bytes.  Same checks (the query sized in f16 values), dispatch and
 * results as the f32 entry given the same values; the decode path converts the
 * query to f32 first. */
KRAKEN_API int kraken_hip_attention_f16q_batched_f16_kv(
  kraken_hip_context* context, kraken_buffer query, kraken_buffer key_cache,
  kraken_buffer value_cache, size_t layer, size_t start_position, size_t tokens,
  size_t capacity_tokens, size_t heads, size_t kv_heads, size_t head_dim,
  kraken_buffer output);

/* MpsContext::attention_f32_batched (mps_backend.hpp:404-414; F32 KV twin,
 * mps_backend.mm:2879-2941): same contract with an f32 cache. */
KRAKEN_API int kraken_hip_attention_f32_batched(
  kraken_hip_context* context, kraken_buffer query, kraken_buffer key_cache,
  kraken_buffer value_cache, size_t layer, size_t start_position, size_t tokens,
  size_t capacity_tokens, size_t heads, size_t kv_heads, size_t head_dim,
  kraken_buffer output);

/* attention_f32_batched_f16_kv followed by the full-attention output gate
 * out *= sigmoid(gate) (qwen35_runtime.cpp:3333-3355: the attention call, then
 * sigmoid_f32_in_place and mul_f32_in_place), fused into the attention epilogue.
 * gate f32 [tokens][heads][head_dim]. */
KRAKEN_API int kraken_hip_attention_f32_batched_f16_kv_gated(
  kraken_hip_context* context, kraken_buffer query, kraken_buffer key_cache,
  kraken_buffer value_cache, kraken_buffer gate, size_t layer, size_t start_position,
  size_t tokens, size_t capacity_tokens, size_t heads, size_t kv_heads, size_t head_dim,
  kraken_buffer output);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): kraken_hip_attention_f32_batched_f16_kv_gated with the
 * same arguments, kernels and results, but its split partials live in a static
 * 8 MiB device array that the library holds on each GPU until the process
 * ends, so the call allocates nothing.  Shapes whose partials need more
 * (e.g. long prefills split over the KV) are rejected with
 * KRAKEN_INVALID_ARGUMENT; single-token decode at any supported KV length
 * fits.  All calls on one GPU share the array: calls that overlap in time on
 * one GPU (other contexts or streams) race and must be serialised by the
 * caller.  Nothing in the array needs to start at zero. */
KRAKEN_API int kraken_hip_attention_f32_batched_f16_kv_gated_no_alloc(
  kraken_hip_context* context, kraken_buffer query, kraken_buffer key_cache,
  kraken_buffer value_cache, kraken_buffer gate, size_t layer, size_t start_position,
  size_t tokens, size_t capacity_tokens, size_t heads, size_t kv_heads, size_t head_dim,
  kraken_buffer output);

/* The full-attention prologue of run_qwen35_full_attention_layer_chunk
 * (qwen35_runtime.cpp:3229-3326) fused into one launch; no single MpsContext
 * method corresponds.  It replaces, with the same arithmetic:
 *   copy_f32_rows x2 (split of q_gate [tokens][heads][2*head_dim], per head the
 *   query then its gate) -> query_out, gate_out [tokens][heads][head_dim];
 *   qk_norm_f32_f32_batched of the query (q_norm) and key (k_norm) rows;
 *   mrope_f32_in_place of both (n_dims, sections, theta);
 *   copy_f32_rows_to_f16 of key and value [tokens][kv_heads*head_dim] into the
 *   F16 caches at element (layer*capacity_tokens + start_position)*kv_dim.
 * positions is int32 [4][tokens]; with positions.data == NULL every row holds
 * mrope_start_position + t (make_qwen35_mrope_positions, qwen35_runtime.cpp:
 * 1848-1877).  key and value are not modified.  head_dim <= 256. */
KRAKEN_API int kraken_hip_qwen35_attention_prologue_f16_kv(
  kraken_hip_context* context, kraken_buffer q_gate, kraken_buffer key, kraken_buffer value,
  kraken_buffer q_norm, kraken_buffer k_norm, kraken_buffer positions,
  size_t mrope_start_position, kraken_buffer key_cache, kraken_buffer value_cache, size_t layer,
  size_t start_position, size_t tokens, size_t capacity_tokens, size_t heads, size_t kv_heads,
  size_t head_dim, size_t n_dims, size_t section_0, size_t section_1, size_t section_2,
  size_t section_3, float theta, float eps, kraken_buffer query_out, kraken_buffer gate_out);

/* kraken_hip_qwen35_attention_prologue_f16_kv followed by
 * kraken_hip_attention_f32_batched_f16_kv_gated(query_out, key_cache,
 * value_cache, gate_out, layer, start_position, tokens, capacity_tokens,
 * heads, kv_heads, head_dim, output): the fused-order full-attention core of
 * run_qwen35_full_attention_layer_chunk (qwen35_runtime.cpp:3229-3355).  No
 * counterpart in the reference as one call; it is for the decode loop, where
 * the two launches cost more than the work.  One token (tokens == 1) with
 * head_dim 256, heads / kv_heads in {1, 2, 4} and start_position < 256 runs as
 * a single launch that writes the same output and cache rows and leaves
 * query_out and gate_out unwritten; every other shape, and
 * KRAKEN_QWEN35_ATTENTION_PROLOGUE=two_launch, runs the two entries above
 * (query_out and gate_out are their scratch).  Arguments as the two entries;
 * output f32 [tokens][heads][head_dim]. */
KRAKEN_API int kraken_hip_qwen35_attention_prologue_gated_f16_kv(
  kraken_hip_context* context, kraken_buffer q_gate, kraken_buffer key, kraken_buffer value,
  kraken_buffer q_norm, kraken_buffer k_norm, kraken_buffer positions,
  size_t mrope_start_position, kraken_buffer key_cache, kraken_buffer value_cache, size_t layer,
  size_t start_position, size_t tokens, size_t capacity_tokens, size_t heads, size_t kv_heads,
  size_t head_dim, size_t n_dims, size_t section_0, size_t section_1, size_t section_2,
  size_t section_3, float theta, float eps, kraken_buffer query_out, kraken_buffer gate_out,
  kraken_buffer output);

/* ------------------------------------------------------ gated delta net -- */

/* MpsContext::gated_delta_net_f32_batched_in_place_at (mps_backend.hpp:296-300;
 * mps_backend.mm:8517-8701, kernels :2225-2374).  q,k f32 [tokens][key_heads][D],
 * v f32 [tokens][value_heads][D], gate/beta f32 [tokens][value_heads], state f32
 * [value_heads][D][D] at element offset state_offset, output [tokens][value_heads][D].
 * key_head = head % key_heads; scale 1/sqrt(D).  The state is updated in place. */
KRAKEN_API int kraken_hip_gated_delta_net_f32_batched_in_place_at(
  kraken_hip_context* context, kraken_buffer query, kraken_buffer key, kraken_buffer value,
  kraken_buffer gate, kraken_buffer beta, kraken_buffer state, size_t state_offset,
  size_t tokens, size_t key_heads, size_t value_heads, size_t head_dim, kraken_buffer output);

/* MpsContext::gated_delta_net_f32_batched_in_place (mps_backend.hpp:291-295):
 * state_offset 0. */
KRAKEN_API int kraken_hip_gated_delta_net_f32_batched_in_place(
  kraken_hip_context* context, kraken_buffer query, kraken_buffer key, kraken_buffer value,
  kraken_buffer gate, kraken_buffer beta, kraken_buffer state, size_t tokens,
  size_t key_heads, size_t value_heads, size_t head_dim, kraken_buffer output);

/* MpsContext::gated_delta_net_f32_in_place[_at] (mps_backend.hpp:270-289; one
 * token, mps_backend.mm:2155-2223). */
KRAKEN_API int kraken_hip_gated_delta_net_f32_in_place_at(
  kraken_hip_context* context, kraken_buffer query, kraken_buffer key, kraken_buffer value,
  kraken_buffer gate, kraken_buffer beta, kraken_buffer state, size_t state_offset,
  size_t key_heads, size_t value_heads, size_t head_dim, kraken_buffer output);

/* MpsContext::ssm_conv_f32 (mps_backend.hpp:301-307; mps_backend.mm:2376-2400,
 * 8703-8796).  input [sequences][channels][K-1+tokens], kernel [channels][K],
 * output [sequences][tokens][channels]. */
KRAKEN_API int kraken_hip_ssm_conv_f32(kraken_hip_context* context, kraken_buffer input,
                                       kraken_buffer kernel, size_t conv_kernel,
                                       size_t channels, size_t tokens, size_t sequences,
                                       kraken_buffer output);

/* MpsContext::build_ssm_conv_state_f32 (mps_backend.hpp:308-314;
 * mps_backend.mm:2428-2457, 8801-8912).  state [channels][K-1] at element offset
 * state_offset, input [tokens][channels], conv_input [channels][K-1+tokens]. */
KRAKEN_API int kraken_hip_build_ssm_conv_state_f32(kraken_hip_context* context,
                                                   kraken_buffer state, size_t state_offset,
                                                   kraken_buffer input, size_t conv_kernel,
                                                   size_t channels, size_t tokens,
                                                   kraken_buffer conv_input);

/* MpsContext::ssm_conv1_f32_stateful_at (mps_backend.hpp:315-327;
 * mps_backend.mm:2402-2426). */
KRAKEN_API int kraken_hip_ssm_conv1_f32_stateful_at(kraken_hip_context* context,
                                                    kraken_buffer state, size_t state_offset,
                                                    kraken_buffer input, kraken_buffer kernel,
                                                    size_t conv_kernel, size_t channels,
                                                    kraken_buffer output);

/* The linear-attention prologue of run_qwen35_linear_layer_chunk
 * (qwen35_runtime.cpp:2746-2796): build_ssm_conv_state_f32 + ssm_conv_f32 +
 * silu_f32_in_place + split_qkv_l2_norm_f32_qwen35 fused in one kernel.  qkv
 * [tokens][2*key_heads*D + value_heads*D] (the conv input projection), conv_state
 * [channels][K-1] at state_offset (updated), conv_kernel_weights [channels][K];
 * writes q,k (L2-normalised) [tokens][key_heads][D] and v [tokens][value_heads][D]. */
KRAKEN_API int kraken_hip_qwen35_conv_split_l2_f32(
  kraken_hip_context* context, kraken_buffer qkv, kraken_buffer conv_state,
  size_t state_offset, kraken_buffer conv_kernel_weights, size_t conv_kernel, size_t tokens,
  size_t key_heads, size_t value_heads, size_t head_dim, float eps, kraken_buffer query,
  kraken_buffer key, kraken_buffer value);

/* The recurrent core of run_qwen35_linear_layer_chunk (qwen35_runtime.cpp:2913-3008):
 * prepare_qwen35_gdn_gate_beta_f32 + gated_delta_net_f32_batched_in_place_at +
 * qwen35_norm_gated_f32_in_place fused.  alpha/beta_raw [tokens][value_heads] are the
 * raw projections (not modified), dt_bias/ssm_a [value_heads], z [tokens][value_heads][D]
 * the output gate, norm_weight [D]; output receives RMSNorm(y)*w*silu(z). */
KRAKEN_API int kraken_hip_qwen35_gdn_gated_f32(
  kraken_hip_context* context, kraken_buffer query, kraken_buffer key, kraken_buffer value,
  kraken_buffer alpha, kraken_buffer beta_raw, kraken_buffer dt_bias, kraken_buffer ssm_a,
  kraken_buffer z, kraken_buffer norm_weight, kraken_buffer state, size_t state_offset,
  size_t tokens, size_t key_heads, size_t value_heads, size_t head_dim, float eps,
  kraken_buffer output);

/* ---------------------------------------------- prologue / epilogue ops -- */

/* MpsContext::split_qkv_l2_norm_f32_qwen35 (mps_backend.hpp:266-269;
 * mps_backend.mm:2097-2153). */
KRAKEN_API int kraken_hip_split_qkv_l2_norm_f32_qwen35(
  kraken_hip_context* context, kraken_buffer source, kraken_buffer query, kraken_buffer key,
  kraken_buffer value, size_t tokens, size_t key_heads, size_t value_heads, size_t head_dim,
  float eps);

/* MpsContext::l2_norm_f32_in_place (mps_backend.hpp:262-265; mps_backend.mm:2065-2095). */
KRAKEN_API int kraken_hip_l2_norm_f32_in_place(kraken_hip_context* context,
                                               kraken_buffer values, size_t rows,
                                               size_t row_size, float eps);

/* MpsContext::qk_norm_f32_f32_batched (mps_backend.hpp:252-257;
 * mps_backend.mm:1991-2024). */
KRAKEN_API int kraken_hip_qk_norm_f32_f32_batched(kraken_hip_context* context,
                                                  kraken_buffer values, kraken_buffer weight,
                                                  size_t tokens, size_t heads,
                                                  size_t head_dim, float eps);

/* MpsContext::qwen35_norm_gated_f32_in_place (mps_backend.hpp:258-261;
 * mps_backend.mm:2026-2063). */
KRAKEN_API int kraken_hip_qwen35_norm_gated_f32_in_place(
  kraken_hip_context* context, kraken_buffer values, kraken_buffer weight, kraken_buffer gate,
  size_t tokens, size_t heads, size_t head_dim, float eps);

/* MpsContext::prepare_qwen35_gdn_gate_beta_f32 (mps_backend.hpp:356-358;
 * mps_backend.mm:2588-2605). */
KRAKEN_API int kraken_hip_prepare_qwen35_gdn_gate_beta_f32(
  kraken_hip_context* context, kraken_buffer gate, kraken_buffer beta,
  kraken_buffer gate_bias, kraken_buffer gate_scale, size_t rows, size_t row_size);

/* MpsContext::mrope_f32_in_place (mps_backend.hpp:331-341; mps_backend.mm:2482-2527).
 * positions int32 [4][tokens]. */
KRAKEN_API int kraken_hip_mrope_f32_in_place(kraken_hip_context* context,
                                             kraken_buffer values, kraken_buffer positions,
                                             size_t tokens, size_t heads, size_t head_dim,
                                             size_t n_dims, size_t section_0,
                                             size_t section_1, size_t section_2,
                                             size_t section_3, float theta);

/* MpsContext::copy_f32_rows_to_f16 / copy_f32_rows / copy_f16_rows
 * (mps_backend.hpp:366-383; mps_backend.mm:2627-2679): strided row copies in
 * element units; the f16 variant rounds to nearest even. */
KRAKEN_API int kraken_hip_copy_f32_rows_to_f16(kraken_hip_context* context,
                                               kraken_buffer source, kraken_buffer destination,
                                               size_t rows, size_t row_size,
                                               size_t source_stride, size_t source_offset,
                                               size_t destination_stride,
                                               size_t destination_offset);
KRAKEN_API int kraken_hip_copy_f32_rows(kraken_hip_context* context, kraken_buffer source,
                                        kraken_buffer destination, size_t rows,
                                        size_t row_size, size_t source_stride,
                                        size_t source_offset, size_t destination_stride,
                                        size_t destination_offset);
KRAKEN_API int kraken_hip_copy_f16_rows(kraken_hip_context* context, kraken_buffer source,
                                        kraken_buffer destination, size_t rows,
                                        size_t row_size, size_t source_stride,
                                        size_t source_offset, size_t destination_stride,
                                        size_t destination_offset);

/* Elementwise ops: MpsContext::sigmoid_f32_in_place / softplus_f32_in_place /
 * silu_f32_in_place / mul_f32_in_place / add_f32_row_in_place / mul_f32_row_in_place
 * (mps_backend.hpp:344-359; mps_backend.mm:2539-2618). */
KRAKEN_API int kraken_hip_sigmoid_f32_in_place(kraken_hip_context* context,
                                               kraken_buffer values, size_t size);
KRAKEN_API int kraken_hip_softplus_f32_in_place(kraken_hip_context* context,
                                                kraken_buffer values, size_t size);
KRAKEN_API int kraken_hip_silu_f32_in_place(kraken_hip_context* context,
                                            kraken_buffer values, size_t size);
KRAKEN_API int kraken_hip_mul_f32_in_place(kraken_hip_context* context, kraken_buffer target,
                                           kraken_buffer rhs, size_t size);
KRAKEN_API int kraken_hip_add_f32_row_in_place(kraken_hip_context* context,
                                               kraken_buffer target, kraken_buffer row,
                                               size_t rows, size_t row_size);
KRAKEN_API int kraken_hip_mul_f32_row_in_place(kraken_hip_context* context,
                                               kraken_buffer target, kraken_buffer row,
                                               size_t rows, size_t row_size);

/* The residual and FFN ops of a decoder layer around the hot path:
 * add_f32_in_place (mps_backend.hpp:342-343; target += delta),
 * silu_mul_f32_in_place (mps_backend.hpp:360-361; gate = silu(gate) * up) and
 * rms_norm_f32_f32_batched (mps_backend.hpp:238-243; output[t] = input[t] *
 * rsqrt(mean(input[t]^2) + eps) * weight for `tokens` rows of `size`; output
 * may be input). */
KRAKEN_API int kraken_hip_add_f32_in_place(kraken_hip_context* context, kraken_buffer target,
                                           kraken_buffer delta, size_t size);
KRAKEN_API int kraken_hip_silu_mul_f32_in_place(kraken_hip_context* context, kraken_buffer gate,
                                                kraken_buffer up, size_t size);
KRAKEN_API int kraken_hip_rms_norm_f32_f32_batched(kraken_hip_context* context,
                                                   kraken_buffer input, kraken_buffer weight,
                                                   size_t tokens, size_t size, float eps,
                                                   kraken_buffer output);

/* ---- Ragged multi-sequence decode ------------------------------------------
 * No counterpart in the reference, which serves one sequence per context
 * (README.md:540); for callers that batch the decode step of many sequences
 * (the layer drivers run_qwen35_full_attention_layer_chunk /
 * run_qwen35_linear_layer_chunk, qwen35_runtime.cpp:2634-3423, applied to one
 * token of each sequence).  Sequence b contributes row b of every [sequences][...]
 * operand.  Per-sequence tables are device buffers: seq_*_offsets are uint64
 * element offsets into caller-owned pools, seq_positions are uint32 positions
 * (the query at position p attends keys 0..p; the new key/value row is row p).
 * Kernels bound every access to its pool: an offset outside it reads zeros
 * (KV) or skips that sequence (states, appends). */

/* Decode attention over per-sequence F16 K/V rows [position][kv_heads][head_dim]
 * at seq_kv_offsets[b] of key_pool / value_pool (same size); optional fused
 * output gate (gate.data == NULL: none); max_position bounds every position.
 * Semantics per sequence: attention_f32_batched_f16_kv with tokens = 1
 * (mps_backend.hpp:415-420; mps_backend.mm:2943-3008) and, with a gate,
 * out *= sigmoid(gate) (qwen35_runtime.cpp:3347-3355).  head_dim 64/128/256,
 * 1/2/4/8 query heads per KV head, 16-byte aligned buffers. */
KRAKEN_API int kraken_hip_attention_f32_ragged_f16_kv(
  kraken_hip_context* context, kraken_buffer query, kraken_buffer key_pool,
  kraken_buffer value_pool, kraken_buffer gate, kraken_buffer seq_kv_offsets,
  kraken_buffer seq_positions, size_t sequences, size_t max_position, size_t heads,
  size_t kv_heads, size_t head_dim, kraken_buffer output);

/* KV append: f32 rows [sequences][row_size] -> f16 row seq_positions[b] of each
 * sequence's K and V (copy_f32_rows_to_f16, mps_backend.hpp:372-376, at the
 * per-sequence destination). */
KRAKEN_API int kraken_hip_append_kv_ragged_f16(kraken_hip_context* context,
                                               kraken_buffer key_rows, kraken_buffer value_rows,
                                               kraken_buffer key_pool, kraken_buffer value_pool,
                                               kraken_buffer seq_kv_offsets,
                                               kraken_buffer seq_positions, size_t sequences,
                                               size_t row_size);

/* One recurrent step per sequence: gated_delta_net_f32_batched_in_place_at with
 * tokens = 1 (mps_backend.hpp:296-300) on the state [value_heads][D][D] at
 * seq_state_offsets[b] of state_pool. */
KRAKEN_API int kraken_hip_gated_delta_net_f32_ragged_decode(
  kraken_hip_context* context, kraken_buffer query, kraken_buffer key, kraken_buffer value,
  kraken_buffer gate, kraken_buffer beta, kraken_buffer state_pool,
  kraken_buffer seq_state_offsets, size_t sequences, size_t key_heads, size_t value_heads,
  size_t head_dim, kraken_buffer output);

/* Fused linear-attention prologue for one token per sequence
 * (kraken_hip_qwen35_conv_split_l2_f32 semantics) with the conv state
 * [channels][conv_kernel - 1] of sequence b at seq_conv_offsets[b] of conv_pool. */
KRAKEN_API int kraken_hip_qwen35_conv_split_l2_ragged_decode_f32(
  kraken_hip_context* context, kraken_buffer qkv, kraken_buffer conv_pool,
  kraken_buffer seq_conv_offsets, kraken_buffer conv_kernel_weights, size_t conv_kernel,
  size_t sequences, size_t key_heads, size_t value_heads, size_t head_dim, float eps,
  kraken_buffer query, kraken_buffer key, kraken_buffer value);

/* One decode step of the Qwen3.5 linear-attention core for `sequences`
 * sequences (one token each): the ragged conv prologue
 * (kraken_hip_qwen35_conv_split_l2_ragged_decode_f32), the ragged gated delta
 * rule (kraken_hip_gated_delta_net_f32_ragged_decode) and the norm-gated
 * epilogue (qwen35_norm_gated_f32_in_place), i.e. qwen35_runtime.cpp:2740-3008
 * between the projections.  No single MpsContext method corresponds.
 * qkv, conv_pool, seq_conv_offsets and conv_kernel_weights as for the ragged conv
 * prologue; gate/beta [sequences][value_heads] are the raw alpha/beta
 * projections when dt_bias and ssm_a [value_heads] are given (both or neither;
 * prepared as in prepare_qwen35_gdn_gate_beta_f32), else the prepared decay
 * and beta; z [sequences][value_heads][head_dim]; norm_weight [head_dim];
 * state_pool and seq_state_offsets as for the ragged gated delta net.  output
 * [sequences][value_heads][head_dim] receives RMSNorm(y) * norm_weight * silu(z).
 * One kernel for head_dim 128, conv_kernel 4 and key_heads == value_heads
 * (bit-identical to the chain); other shapes run the three kernels, using
 * context workspace.  A sequence whose offsets are outside a pool is skipped. */
KRAKEN_API int kraken_hip_qwen35_gdn_layer_ragged_decode_f32(
  kraken_hip_context* context, kraken_buffer qkv, kraken_buffer conv_pool,
  kraken_buffer seq_conv_offsets, kraken_buffer conv_kernel_weights, size_t conv_kernel,
  kraken_buffer gate, kraken_buffer beta, kraken_buffer dt_bias, kraken_buffer ssm_a,
  kraken_buffer z, kraken_buffer norm_weight, kraken_buffer state_pool,
  kraken_buffer seq_state_offsets, size_t sequences, size_t key_heads, size_t value_heads,
  size_t head_dim, float eps, kraken_buffer output);

/* No counterpart in the reference: the gated delta rule of
 * kraken_hip_qwen35_gdn_layer_ragged_decode_f32 alone, for the device decode
 * loop's three-launch linear-attention layer (input projection with the conv
 * folded in, this, output projection with the norm-gated epilogue finished on
 * its input).  qkv [sequences][3 * value_heads * head_dim] holds q, k and v
 * after the conv and SiLU (kraken_hip_kquant_matvec_multi_conv_f32's matrix 0
 * output); q and k are L2-normalised here.  gate, beta, dt_bias, ssm_a, z,
 * norm_weight, state_pool and seq_state_offsets as for the layer entry.
 * output [sequences][value_heads][head_dim] receives y * rsqrt(head_dim) and
 * gate_output (same shape) norm_weight[c % head_dim] * silu(z[c]): the
 * norm-gated epilogue is then y * rsqrt(mean(y^2) + eps) * gate_output per
 * head (kraken_hip_kquant_matvec_head_norm_f32).  State and y equal the layer
 * entry's bit for bit given the same qkv.  head_dim 128 and key_heads ==
 * value_heads only.  A sequence whose state offset is outside the pool is
 * skipped. */
KRAKEN_API int kraken_hip_qwen35_gdn_state_ragged_decode_f32(
  kraken_hip_context* context, kraken_buffer qkv, kraken_buffer gate, kraken_buffer beta,
  kraken_buffer dt_bias, kraken_buffer ssm_a, kraken_buffer z, kraken_buffer norm_weight,
  kraken_buffer state_pool, kraken_buffer seq_state_offsets, size_t sequences,
  size_t key_heads, size_t value_heads, size_t head_dim, float eps, kraken_buffer output,
  kraken_buffer gate_output);

/* ---- K-quant projections (GGUF Q4_K / Q5_K / Q6_K weights) and argmax ----
 *
 * Weights are rows of GGUF super-blocks of 256 values (Q4_K 144 bytes, Q5_K
 * 176, Q6_K 210 per block), row-major [rows][cols / 256]; cols must be a
 * multiple of 256.  Outputs are f32.  Validation follows the reference's
 * order and messages ("HIP" for "MPS").  Beyond the reference, the weight must
 * be 4-byte aligned (Q6_K: 2-byte) and inputs and dequantized outputs 16-byte
 * aligned, as every allocation of this library is.
 *
 * matvec_*_device: output[rows] = W @ input[cols], fp32 arithmetic
 *   (mps_backend.hpp:137-140, 158-161, 179-182).
 * matvec_*_top1: token_output[0] = argmax_r (W @ input)[r] and
 *   probability_output[0] = its softmax probability over all rows; _argmax
 *   only the token (mps_backend.hpp:141-149, 162-170, 183-191).  Limited to
 *   cols <= 4096 (16 blocks per row), as the reference's kernels are.
 * matmul_*_device: output[tokens][rows] = input[tokens][cols] @ W^T
 *   (mps_backend.hpp:150-154, 171-175, 192-196).  Up to 8 tokens the weights
 *   are dequantized to f32 and multiplied in fp32; above 8, as in the
 *   reference's tiled kernel, weights and inputs are rounded to f16 and
 *   multiplied with f32 accumulation (MFMA), using context workspace of
 *   2 * (rows + tokens) * cols bytes.
 * dequantize_row_*: output[cols] = row `row` of W (mps_backend.hpp:197-200,
 *   207-210, 217-220).  dequantize_rows_*: output[tokens][cols], row
 *   row_ids[t] (i32) for token t; an id outside [0, rows) gives a zero row
 *   (mps_backend.hpp:201-206, 211-216, 221-226). */
KRAKEN_API int kraken_hip_matvec_q4_k_f32_device(kraken_hip_context* context,
                                              kraken_buffer weight, size_t rows, size_t cols,
                                              kraken_buffer input, kraken_buffer output);
KRAKEN_API int kraken_hip_matvec_q4_k_f32_top1(kraken_hip_context* context, kraken_buffer weight,
                                            size_t rows, size_t cols, kraken_buffer input,
                                            kraken_buffer token_output,
                                            kraken_buffer probability_output);
KRAKEN_API int kraken_hip_matvec_q4_k_f32_argmax(kraken_hip_context* context,
                                              kraken_buffer weight, size_t rows, size_t cols,
                                              kraken_buffer input, kraken_buffer token_output);
KRAKEN_API int kraken_hip_matmul_q4_k_f32_device(kraken_hip_context* context,
                                              kraken_buffer weight, size_t rows, size_t cols,
                                              size_t tokens, kraken_buffer input,
                                              kraken_buffer output);
KRAKEN_API int kraken_hip_dequantize_row_q4_k_f32(kraken_hip_context* context,
                                               kraken_buffer weight, size_t row, size_t cols,
                                               kraken_buffer output);
KRAKEN_API int kraken_hip_dequantize_rows_q4_k_f32(kraken_hip_context* context,
                                                kraken_buffer weight, size_t rows,
                                                kraken_buffer row_ids, size_t tokens,
                                                size_t cols, kraken_buffer output);

KRAKEN_API int kraken_hip_matvec_q5_k_f32_device(kraken_hip_context* context,
                                              kraken_buffer weight, size_t rows, size_t cols,
                                              kraken_buffer input, kraken_buffer output);
KRAKEN_API int kraken_hip_matvec_q5_k_f32_top1(kraken_hip_context* context, kraken_buffer weight,
                                            size_t rows, size_t cols, kraken_buffer input,
                                            kraken_buffer token_output,
                                            kraken_buffer probability_output);
KRAKEN_API int kraken_hip_matvec_q5_k_f32_argmax(kraken_hip_context* context,
                                              kraken_buffer weight, size_t rows, size_t cols,
                                              kraken_buffer input, kraken_buffer token_output);
KRAKEN_API int kraken_hip_matmul_q5_k_f32_device(kraken_hip_context* context,
                                              kraken_buffer weight, size_t rows, size_t cols,
                                              size_t tokens, kraken_buffer input,
                                              kraken_buffer output);
KRAKEN_API int kraken_hip_dequantize_row_q5_k_f32(kraken_hip_context* context,
                                               kraken_buffer weight, size_t row, size_t cols,
                                               kraken_buffer output);
KRAKEN_API int kraken_hip_dequantize_rows_q5_k_f32(kraken_hip_context* context,
                                                kraken_buffer weight, size_t rows,
                                                kraken_buffer row_ids, size_t tokens,
                                                size_t cols, kraken_buffer output);

KRAKEN_API int kraken_hip_matvec_q6_k_f32_device(kraken_hip_context* context,
                                              kraken_buffer weight, size_t rows, size_t cols,
                                              kraken_buffer input, kraken_buffer output);
KRAKEN_API int kraken_hip_matvec_q6_k_f32_top1(kraken_hip_context* context, kraken_buffer weight,
                                            size_t rows, size_t cols, kraken_buffer input,
                                            kraken_buffer token_output,
                                            kraken_buffer probability_output);
KRAKEN_API int kraken_hip_matvec_q6_k_f32_argmax(kraken_hip_context* context,
                                              kraken_buffer weight, size_t rows, size_t cols,
                                              kraken_buffer input, kraken_buffer token_output);
KRAKEN_API int kraken_hip_matmul_q6_k_f32_device(kraken_hip_context* context,
                                              kraken_buffer weight, size_t rows, size_t cols,
                                              size_t tokens, kraken_buffer input,
                                              kraken_buffer output);
KRAKEN_API int kraken_hip_dequantize_row_q6_k_f32(kraken_hip_context* context,
                                               kraken_buffer weight, size_t row, size_t cols,
                                               kraken_buffer output);
KRAKEN_API int kraken_hip_dequantize_rows_q6_k_f32(kraken_hip_context* context,
                                                kraken_buffer weight, size_t rows,
                                                kraken_buffer row_ids, size_t tokens,
                                                size_t cols, kraken_buffer output);

/* No counterpart in the reference: the one-token K-quant GEMV with a decoder
 * layer's neighbouring ops folded in, for the device decode loop.  ggml_type is
 * the GGUF type id (12 Q4_K, 13 Q5_K, 14 Q6_K); weight, rows and cols as for
 * matvec_*_f32_device.  output[r] = residual[r] + sum_k W[r][k] x_k, where x =
 * input * rsqrt(mean(input^2) + eps) * norm_weight when norm_weight is given
 * (rms_norm_f32_f32_batched), silu(input) * up when up is given
 * (silu_mul_f32_in_place), else input; residual may be empty (then 0) or the
 * output buffer itself (add_f32_in_place).  norm_weight and up are exclusive;
 * they and input must be 16-byte aligned. */
KRAKEN_API int kraken_hip_kquant_matvec_fused_f32(kraken_hip_context* context, uint32_t ggml_type,
                                                  kraken_buffer weight, size_t rows, size_t cols,
                                                  kraken_buffer input, kraken_buffer norm_weight,
                                                  float eps, kraken_buffer up,
                                                  kraken_buffer residual, kraken_buffer output);
/* No counterpart in the reference: up to four kraken_hip_kquant_matvec_fused_f32
 * calls that share input, norm_weight / up and eps, in one launch (the
 * projections of one normed hidden state).  Arrays of `count` (1..4) entries
 * give each matrix's type, weight, rows, residual (data may be NULL) and
 * output; cols <= 4096. */
KRAKEN_API int kraken_hip_kquant_matvec_multi_f32(
  kraken_hip_context* context, size_t count, const uint32_t* ggml_types,
  const kraken_buffer* weights, const size_t* rows, size_t cols, kraken_buffer input,
  kraken_buffer norm_weight, float eps, kraken_buffer up, const kraken_buffer* residuals,
  const kraken_buffer* outputs);
/* No counterpart in the reference: matmul_q*_k_f32_device (mps_backend.mm:
 * 6336-6450) with a decoder layer's neighbouring ops folded in, for the chunked
 * prefill: output = residual + W x, where x = silu(input) * up when up is given
 * (silu_mul_f32_in_place, then the matmul's fp16 rounding of its input) and
 * input otherwise; residual may be empty (then 0) or the output buffer itself
 * (add_f32_in_place), but no other view that overlaps the output.  The same
 * bits as the separate ops.  More than 8 tokens (the GEMM path); up and
 * residual 16-byte aligned; a given up takes the two-pass GEMM form. */
KRAKEN_API int kraken_hip_kquant_matmul_fused_f32(kraken_hip_context* context, uint32_t ggml_type,
                                                  kraken_buffer weight, size_t rows, size_t cols,
                                                  size_t tokens, kraken_buffer input,
                                                  kraken_buffer up, kraken_buffer residual,
                                                  kraken_buffer output);
/* No counterpart in the reference: up to four matmul_q*_k_f32_device calls
 * (mps_backend.mm:6336-6450) that share input, cols and tokens, for the chunked
 * prefill's projections of one normed hidden state (the linear-attention z, beta
 * and alpha; the FFN up and gate).  Arrays of `count` (1..4) entries give each
 * matrix's GGUF type (12 Q4_K, 13 Q5_K, 14 Q6_K), weight, rows and output
 * [tokens][rows]; each is checked as its matmul entry checks it.  When every
 * matrix has the same type, more than 8 tokens and the type takes the GEMM
 * form that decodes the weights in its B tile (Q4_K by default), the matrices
 * run as one launch with no K split; otherwise, or with
 * KRAKEN_KQUANT_GROUP=off, each runs as its matmul entry.  A matrix whose own
 * entry would split K then sums in another order: within fp32 rounding of its
 * separate result, bit-identical to it when it would not split.  Outputs must
 * not overlap each other or the input. */
KRAKEN_API int kraken_hip_kquant_matmul_multi_f32(kraken_hip_context* context, size_t count,
                                                  const uint32_t* ggml_types,
                                                  const kraken_buffer* weights,
                                                  const size_t* rows, size_t cols, size_t tokens,
                                                  kraken_buffer input,
                                                  const kraken_buffer* outputs);
/* No counterpart in the reference: kraken_hip_kquant_matvec_multi_f32 (no up
 * input, no residuals) whose matrix 0 rows are the conv channels of one
 * sequence's linear-attention prologue: each row's value x becomes
 * silu(sum_j state[r][j] * w[r][j] + x * w[r][3]) and the conv state row
 * [r][0..2] shifts in x (ssm_conv1_f32_stateful_at then silu_f32_in_place,
 * qwen35_runtime.cpp:2171-2178, for one token).
 * conv_pool holds f32 conv states; conv_offset is one uint64 in device memory,
 * the element offset of this sequence's [rows[0]][3] state (a state outside the
 * pool leaves matrix 0's output and state untouched); conv_kernel_weights
 * [rows[0]][4]; conv_kernel must be 4, and norm_weight must be given (the
 * joint projection of a normed hidden state). */
KRAKEN_API int kraken_hip_kquant_matvec_multi_conv_f32(
  kraken_hip_context* context, size_t count, const uint32_t* ggml_types,
  const kraken_buffer* weights, const size_t* rows, size_t cols, kraken_buffer input,
  kraken_buffer norm_weight, float eps, const kraken_buffer* outputs, kraken_buffer conv_pool,
  kraken_buffer conv_offset, kraken_buffer conv_kernel_weights, size_t conv_kernel);
/* No counterpart in the reference: the one-token GEMV of the linear-attention
 * output projection with the norm-gated epilogue finished on its input: x[c]
 * = input[c] * rsqrt(mean over c's head of input^2 + eps) * gate_factor[c]
 * (gate_factor = norm_weight * silu(z) from
 * kraken_hip_qwen35_gdn_state_ragged_decode_f32; qwen35_norm_gated_f32_in_place
 * over heads of head_dim values), output = residual + W x as for
 * kraken_hip_kquant_matvec_fused_f32.  head_dim must be 128, cols <= 4096;
 * gate_factor 16-byte aligned. */
KRAKEN_API int kraken_hip_kquant_matvec_head_norm_f32(
  kraken_hip_context* context, uint32_t ggml_type, kraken_buffer weight, size_t rows,
  size_t cols, kraken_buffer input, kraken_buffer gate_factor, size_t head_dim, float eps,
  kraken_buffer residual, kraken_buffer output);
/* No counterpart in the reference: matvec_q*_k_f32_top1 (probability_output
 * given) or matvec_q*_k_f32_argmax (probability_output empty) with the output
 * RMSNorm folded into the logits GEMV when norm_weight is given. */
KRAKEN_API int kraken_hip_kquant_top1_fused_f32(kraken_hip_context* context, uint32_t ggml_type,
                                                kraken_buffer weight, size_t rows, size_t cols,
                                                kraken_buffer input, kraken_buffer norm_weight,
                                                float eps, kraken_buffer token_output,
                                                kraken_buffer probability_output);

/* argmax_f32_i32 (mps_backend.hpp:384-386): output[0] = the first index of
 * the largest of values[size]; NaN never wins, -inf can; all-NaN gives size.
 * argmax_prob_f32_i32 (mps_backend.hpp:387-390): also probability_output[0]
 * = 1 / sum_i exp(values[i] - max), or 0 when that sum is not positive.
 * Inputs above 16384 values use context workspace (12 bytes per 4096). */
KRAKEN_API int kraken_hip_argmax_f32_i32(kraken_hip_context* context, kraken_buffer values,
                                         size_t size, kraken_buffer output);
KRAKEN_API int kraken_hip_argmax_prob_f32_i32(kraken_hip_context* context, kraken_buffer values,
                                              size_t size, kraken_buffer token_output,
                                              kraken_buffer probability_output);

#ifdef __cplusplus
}
#endif

#endif /* KRAKEN_HIP_H */
