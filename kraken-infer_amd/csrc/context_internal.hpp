// Host-side internals shared by the C-ABI translation units: the context
// object, the status/last-error convention, argument validation helpers, and
// the launch functions each kernel translation unit provides.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <limits>
#include <string>
#include <vector>

#include "kraken_hip.h"

struct kraken_hip_context {
  bool validation_only = false;
  int device = -1;
  int cu_count = 0;
  hipStream_t own_stream = nullptr;
  hipStream_t stream = nullptr;  // where work is enqueued (own or caller's)
  bool graph_active = false;
  // Device workspace owned by the context (split-K partials, chunk operands,
  // staging).  Grown on demand outside of any kernel; the reference likewise owns only its flash-tail
  // scratch (mps_backend.mm:4402-4407).  A workspace that is outgrown is kept,
  // not freed, until the context is destroyed: a HIP graph captured earlier may
  // hold its address and replay into it.  Growth at least doubles, so the kept
  // ones add up to less than the current one.
  void* workspace = nullptr;
  size_t workspace_bytes = 0;
  std::vector<void*> retired_workspaces;
  // This device's copy of the static scratch array used by the allocation-free
  // entry point (device address, resolved at context creation).
  void* no_alloc_scratch = nullptr;
};

// Returns from the calling entry point with the status of `expr` unless it is OK.
#define KRAKEN_TRY(expr)            \
  do {                              \
    const int kraken_s_ = (expr);   \
    if (kraken_s_ != KRAKEN_OK) {   \
      return kraken_s_;             \
    }                               \
  } while (0)

namespace kraken {

// --------------------------------------------------------------- status ----
// Records `message` as this thread's last error and returns `code`.
int fail(int code, const std::string& message);
inline int invalid(const std::string& m) { return fail(KRAKEN_INVALID_ARGUMENT, m); }
inline int unavailable(const std::string& m) { return fail(KRAKEN_UNAVAILABLE, m); }
inline int internal(const std::string& m) { return fail(KRAKEN_INTERNAL_ERROR, m); }

// Context validity (first check of every op, mps_backend.mm:10625-10627).
int check_context(const kraken_hip_context* ctx);

// After validation: a validation-only context stops here with KRAKEN_UNAVAILABLE;
// a live context selects its device.  Returns KRAKEN_OK to proceed.
int begin_launch(kraken_hip_context* ctx);

// After enqueueing: checks the launch and, outside a graph, waits for the stream
// (finish_command_buffer, mps_backend.mm:4416-4428).
int finish_launch(kraken_hip_context* ctx, const char* error_prefix);

// Ensures ctx->workspace holds at least `bytes`.  A larger workspace is a new
// allocation; the old one stays valid (and allocated) until the context is
// destroyed, so work already enqueued or captured into a graph keeps a valid
// address and nothing waits.  Returns KRAKEN_OK or an error status.
int ensure_workspace(kraken_hip_context* ctx, size_t bytes);

// Size of the static per-device scratch array of the allocation-free entry
// point, and the lookup of its device address on `device` (which must be the
// current device); the address is resolved once per device and cached.
constexpr size_t kNoAllocScratchBytes = size_t{8} << 20;
int resolve_no_alloc_scratch(int device, void** out);

// ------------------------------------------------------------ validation ----
// Restatements of the reference's helpers, mps_backend.mm:4196-4308.
inline bool checked_mul(size_t a, size_t b, size_t& out) {
  if (a != 0 && b > std::numeric_limits<size_t>::max() / a) {
    return false;
  }
  out = a * b;
  return true;
}

inline bool checked_add(size_t a, size_t b, size_t& out) {
  if (a > std::numeric_limits<size_t>::max() - b) {
    return false;
  }
  out = a + b;
  return true;
}

inline bool fits_u32(size_t v) { return v <= std::numeric_limits<uint32_t>::max(); }

// checked_u32: `name` exceeds uint32 range -> invalid argument.
int check_u32(size_t value, const char* name);

// validate_f32/f16/i32_buffer: byte count overflow, "not initialized", "too small".
int validate_buffer(const kraken_buffer& buffer, size_t values, size_t element_bytes,
                    const char* name);
inline int validate_f32(const kraken_buffer& b, size_t values, const char* name) {
  return validate_buffer(b, values, sizeof(float), name);
}
inline int validate_f16(const kraken_buffer& b, size_t values, const char* name) {
  return validate_buffer(b, values, sizeof(uint16_t), name);
}
inline int validate_i32(const kraken_buffer& b, size_t values, const char* name) {
  return validate_buffer(b, values, sizeof(int32_t), name);
}

// validate_f32_buffer_region: [offset, offset+values) must fit; returns status.
int validate_f32_region(const kraken_buffer& b, size_t offset, size_t values,
                        const char* name);

// strided_f32_region_end (mps_backend.mm:4203-4231): end element of a strided
// row range; invalid argument on zero rows/row_size, stride < row_size, overflow.
int strided_region_end(size_t offset, size_t rows, size_t stride, size_t row_size,
                       const char* name, size_t& end);

// -------------------------------------------------------------- launches ----
// Implemented by the kernel translation units; all enqueue on `stream` and
// return hipSuccess or the launch error.

struct AttentionArgs {
  const float* query;
  // f16 query [tokens][heads][head_dim] for the flash path (query unused then).
  const void* query_f16 = nullptr;
  const void* key_cache;
  const void* value_cache;
  const float* gate;  // nullable: fused sigmoid output gate
  float* output;
  uint32_t layer, start_position, tokens, capacity_tokens, heads, kv_heads, head_dim;
  bool kv_f16;
  // Ragged multi-sequence decode (set together, else null/0): token t is the
  // one query token of sequence t, at position seq_positions[t] (it attends
  // keys 0..position), whose K/V rows [position][kv_heads][head_dim] start at
  // element seq_kv_offsets[t] of key_cache/value_cache (pools of pool_elems
  // elements each).  max_position bounds every position (sizes the grid).
  const uint64_t* seq_kv_offsets = nullptr;
  const uint32_t* seq_positions = nullptr;
  uint64_t pool_elems = 0;
  uint32_t max_position = 0;
};

// Bytes of workspace the split-K decode path needs for these arguments.
size_t attention_decode_workspace_bytes(const AttentionArgs& a, int cu_count);
hipError_t launch_attention_decode(const AttentionArgs& a, int cu_count, void* workspace,
                                   size_t workspace_bytes, hipStream_t stream);
// Merges per-split (m, l, o) partials (log2-domain m) into the final output,
// applying the optional sigmoid gate.  Partials are laid out
// [tokens][kv_heads][splits][group][head_dim] (ml: [...][group][2]).
struct CombineArgs {
  // Partial outputs: f32 sums (o, with its max and denominator in partial_ml),
  // or, with partial_f16, each split's o / l rounded to f16 (at most 16 splits).
  const float* partial_o;
  const float* partial_ml;
  uint32_t partial_f16;
  const float* gate;
  float* output;
  uint32_t tokens, heads, kv_heads, splits, head_dim;
  // Split s covers keys [s*keys_per_split, (s+1)*keys_per_split); token t has
  // positions[t] + 1 keys (ragged) or start_position + t + 1, so only its first
  // ceil(keys / keys_per_split) splits hold partials.  keys_per_split == 0:
  // all `splits` partials are valid for every token.
  const uint32_t* positions;
  uint32_t start_position, keys_per_split;
};
hipError_t launch_attention_combine(const CombineArgs& c, hipStream_t stream);
// out[i] = (float)in[i] for i < count (f16 -> f32, exact).
hipError_t launch_f16_to_f32(const void* in, float* out, size_t count, hipStream_t stream);
// True when the flash MFMA prefill kernel supports these arguments.
bool flash_prefill_supported(const AttentionArgs& a);
size_t attention_flash_workspace_bytes(const AttentionArgs& a, int cu_count);
hipError_t launch_attention_flash(const AttentionArgs& a, int cu_count, void* workspace,
                                  size_t workspace_bytes, hipStream_t stream);

struct GdnArgs {
  const float* query;
  const float* key;
  const float* value;
  const float* gate;   // prepared gate (log decay) unless `prepare` is set
  const float* beta;   // prepared beta unless `prepare` is set
  float* state;
  float* output;
  uint32_t tokens, key_heads, value_heads, head_dim;
  // Fused prologue/epilogue (kraken_hip_qwen35_gdn_gated_f32); null otherwise.
  const float* dt_bias;      // prepare: gate = softplus(alpha + dt_bias) * ssm_a
  const float* ssm_a;        //          beta = sigmoid(beta_raw)
  const float* z;            // epilogue: out = RMSNorm(y) * norm_weight * silu(z)
  const float* norm_weight;
  float eps;
  // Ragged decode: `tokens` sequences with one token each; sequence b's state
  // [value_heads][D][D] at element seq_state_offsets[b] of `state` (a pool of
  // pool_elems elements).  Null for the single-sequence form.
  const uint64_t* seq_state_offsets = nullptr;
  uint64_t pool_elems = 0;
};
// Multi-token calls at head_dim 128 take the chunked (WY) path, which needs
// gdn_workspace_bytes() of context workspace; other calls need none.
size_t gdn_workspace_bytes(const GdnArgs& a);
hipError_t launch_gated_delta_net(const GdnArgs& a, int cu_count, void* workspace,
                                  size_t workspace_bytes, hipStream_t stream);
// Chunked prefill (csrc/gdn_chunked.hip).
bool gdn_chunked_supported(const GdnArgs& a);
size_t gdn_chunked_workspace_bytes(const GdnArgs& a);
hipError_t launch_gdn_chunked(const GdnArgs& a, void* workspace, size_t workspace_bytes,
                              hipStream_t stream);

// Ragged decode of a whole Qwen3.5 linear-attention core in one kernel
// (kraken_hip_qwen35_gdn_layer_ragged_decode_f32): conv prologue, gated delta
// rule and norm-gated epilogue, one workgroup per (sequence, value head).
struct GdnLayerArgs {
  const float* qkv;           // [sequences][3 * heads * 128]
  float* conv_pool;           // per sequence [channels][3] at seq_conv_offsets[b]
  const uint64_t* seq_conv_offsets;
  uint64_t conv_pool_elems;
  const float* conv_weights;  // [channels][4]
  const float* gate;          // [sequences][heads] (raw alpha when dt_bias is set)
  const float* beta;          // [sequences][heads] (raw when dt_bias is set)
  const float* dt_bias;       // null: gate and beta are prepared
  const float* ssm_a;
  const float* z;             // [sequences][heads][128]
  const float* norm_weight;   // [128]
  float* state_pool;          // per sequence [heads][128][128] at seq_state_offsets[b]
  const uint64_t* seq_state_offsets;
  uint64_t state_pool_elems;
  float* output;              // [sequences][heads][128]
  // gdn_state_split_kernel: norm_weight[c % 128] * silu(z[c]) per output value.
  float* gate_factor;
  uint32_t sequences, heads;
  float eps;
};
// True when the one-kernel layer supports the shape (head_dim 128, conv kernel
// 4, key_heads == value_heads).
bool gdn_layer_fused_supported(uint32_t head_dim, uint32_t conv_kernel, uint32_t key_heads,
                               uint32_t value_heads);
hipError_t launch_gdn_layer_ragged(const GdnLayerArgs& a, hipStream_t stream);
// The one-kernel layer's gated delta rule alone (qkv already through the conv
// and SiLU; conv fields unused): output gets y * scale and gate_factor the
// epilogue's norm_weight * silu(z); the per-head RMS scale is left to the
// caller.  Same shape limits.
hipError_t launch_gdn_state_ragged(const GdnLayerArgs& a, hipStream_t stream);

hipError_t launch_ssm_conv(const float* input, const float* kernel, float* output,
                           uint32_t conv_kernel, uint32_t channels, uint32_t tokens,
                           uint32_t sequences, hipStream_t stream);
hipError_t launch_build_ssm_conv_state(float* state, const float* input, float* conv_input,
                                       uint32_t conv_kernel, uint32_t channels,
                                       uint32_t tokens, hipStream_t stream);
hipError_t launch_ssm_conv1_stateful(float* state, const float* input, const float* kernel,
                                     float* output, uint32_t conv_kernel, uint32_t channels,
                                     hipStream_t stream);
hipError_t launch_conv_split_l2(const float* qkv, float* conv_state, const float* weights,
                                uint32_t conv_kernel, uint32_t tokens, uint32_t key_heads,
                                uint32_t value_heads, uint32_t head_dim, float eps,
                                float* query, float* key, float* value, hipStream_t stream);
// Ragged decode form: one token per sequence, per-sequence conv state offsets.
hipError_t launch_conv_split_l2_ragged(const float* qkv, float* conv_pool,
                                       const uint64_t* seq_conv_offsets, uint64_t pool_elems,
                                       const float* weights, uint32_t conv_kernel,
                                       uint32_t sequences, uint32_t key_heads,
                                       uint32_t value_heads, uint32_t head_dim, float eps,
                                       float* query, float* key, float* value,
                                       hipStream_t stream);
// Ragged KV append: rows[b] (f32, row_size) -> f16 at element
// seq_offsets[b] + seq_positions[b] * row_size of the pool, for K and V.
hipError_t launch_append_kv_ragged(const float* key_rows, const float* value_rows,
                                   void* key_pool, void* value_pool,
                                   const uint64_t* seq_offsets, const uint32_t* seq_positions,
                                   uint64_t pool_elems, uint32_t sequences, uint32_t row_size,
                                   hipStream_t stream);

hipError_t launch_split_qkv_l2(const float* source, float* q, float* k, float* v,
                               uint32_t tokens, uint32_t key_heads, uint32_t value_heads,
                               uint32_t head_dim, float eps, hipStream_t stream);
hipError_t launch_l2_norm(float* values, uint32_t rows, uint32_t row_size, float eps,
                          hipStream_t stream);
// Fused full-attention prologue (attention_prologue.hip): Q/gate split, q and k
// RMSNorm, MRoPE of q and k, K/V append to the F16 cache.
struct PrologueArgs {
  const float* q_gate;       // [tokens][heads][2 * head_dim] (query, then gate)
  const float* key;          // [tokens][kv_heads * head_dim]
  const float* value;        // [tokens][kv_heads * head_dim]
  const float* q_norm;       // [head_dim]
  const float* k_norm;       // [head_dim]
  const int32_t* positions;  // [4][tokens], or null: mrope_start + t in every row
  uint32_t mrope_start;
  _Float16* key_cache;       // f16; rows written from element cache_offset
  _Float16* value_cache;
  size_t cache_offset;       // (layer * capacity + start_position) * kv_dim
  float* query_out;          // [tokens][heads][head_dim]
  float* gate_out;           // [tokens][heads][head_dim]
  uint32_t tokens, heads, kv_heads, head_dim, n_dims, s0, s1, s2, s3;
  float theta, eps;
};
hipError_t launch_attention_prologue(const PrologueArgs& a, hipStream_t stream);
// The prologue and the gated decode attention of one token in one launch
// (attention_decode.hip, attention_decode_short.hip): a.query_out and
// a.gate_out are not written; output [heads][head_dim] receives what
// launch_attention_decode with the prologue's query and gate would write.
// Returns hipErrorNotSupported, launching nothing, outside the folded kernel's
// contract: one token, head_dim 256, heads / kv_heads in {1, 2, 4}, at most
// 256 keys (start_position < 256), 16-byte aligned caches and output, and no
// KRAKEN_DECODE_KERNEL (other than "short") or KRAKEN_DECODE_KEYS_PER_SPLIT.
hipError_t launch_attention_prologue_decode(const PrologueArgs& a, uint32_t layer,
                                            uint32_t start_position, uint32_t capacity_tokens,
                                            float* output, hipStream_t stream);

// K-quant projections (kquant.hip).  format: 0 = Q4_K, 1 = Q5_K, 2 = Q6_K;
// weights are row-major blocks (cols / 256 per row).  Up to
// kKquantGemvMaxTokens tokens take the fp32 GEMV; more take the fp16 MFMA
// GEMM, which stages fp16 weights and inputs in the workspace.
constexpr size_t kKquantGemvMaxTokens = 8;
// Matrices per grouped GEMM launch (launch_kquant_matmul_group).
constexpr size_t kKquantGroupMax = 4;
uint32_t kquant_block_bytes(int format);
// With `up` (GEMM path only), the input is silu(input) * up (the two-pass
// form's first pass forms it, as silu_mul_f32_in_place rounds it); with
// `residual` (GEMM path only; it may be `output`), output = residual + W x, the
// sum add_f32_in_place would form.  swiglu: whether `up` will be given.
size_t kquant_matmul_workspace_bytes(int format, size_t rows, size_t cols, size_t tokens,
                                     bool swiglu = false);
hipError_t launch_kquant_matmul(int format, const void* weight, size_t rows, size_t cols,
                                size_t tokens, const float* input, float* output,
                                void* workspace, size_t workspace_bytes, hipStream_t stream,
                                const float* up = nullptr, const float* residual = nullptr);
// Up to kKquantGroupMax matmuls of one format that share input, cols and
// tokens (kquant.hip).  More than kKquantGemvMaxTokens tokens with the fused
// GEMM form (weights decoded in the B tile) run as one launch whose grid holds
// every matrix's tiles, without K splits; anything else runs
// launch_kquant_matmul per matrix.  Returns hipErrorNotSupported, launching
// nothing, when it would not be one launch, so the caller can use the
// per-matrix entry points (and their workspace) instead.
hipError_t launch_kquant_matmul_group(int format, size_t count, const void* const* weights,
                                      const size_t* rows, size_t cols, size_t tokens,
                                      const float* input, float* const* outputs,
                                      hipStream_t stream);
// Rows row_ids[t] (or fixed_row when row_ids is null, tokens = 1) dequantized
// into output [tokens][cols]; ids outside [0, rows) give zero rows.
hipError_t launch_kquant_dequantize_rows(int format, const void* weight, size_t rows,
                                         const int32_t* row_ids, size_t fixed_row,
                                         size_t tokens, size_t cols, float* output,
                                         hipStream_t stream);
// argmax (probability_out null) or argmax with probability over `size` values:
// the first index of the maximum, NaN never wins.  With nothing above -inf the
// token is `size` (every value NaN) or the first -inf index, or 0 under
// `kquant_rule` (the K-quant top-1/argmax kernels' reduction, which starts from
// index 0).
size_t argmax_workspace_bytes(size_t size);
hipError_t launch_argmax(const float* values, size_t size, int32_t* token_out,
                         float* probability_out, void* workspace, size_t workspace_bytes,
                         hipStream_t stream, bool kquant_rule = false);
// GEMV of one token into workspace logits, then argmax (and probability).
size_t kquant_argmax_workspace_bytes(size_t rows);
// input = RMSNorm(input) * norm_weight when norm_weight is given (eps as for
// rms_norm_f32_f32_batched) before the products.
hipError_t launch_kquant_argmax(int format, const void* weight, size_t rows, size_t cols,
                                const float* input, int32_t* token_out, float* probability_out,
                                void* workspace, size_t workspace_bytes, hipStream_t stream,
                                const float* norm_weight = nullptr, float eps = 0.0f);
// Up to four one-token GEMVs over the same transformed input in one launch
// (cols / 256 <= 16), each with its own format, rows, residual and output.
constexpr uint32_t kKquantMultiMaxMatrices = 4;
constexpr size_t kKquantMultiMaxCols = 4096;
// Conv epilogue of a multi GEMV's matrix 0 (its rows are the conv channels of
// one sequence): state [rows][3] at pool + *offset (device value, checked
// against pool_elems), weights [rows][4].
struct GemvConvEpilogue {
  float* pool;
  const uint64_t* offset;
  uint64_t pool_elems;
  const float* weights;
};
hipError_t launch_kquant_matvec_multi(uint32_t count, const int* formats,
                                      const void* const* weights, const size_t* rows,
                                      size_t cols, const float* input, const float* norm_weight,
                                      float eps, const float* up,
                                      const float* const* residuals, float* const* outputs,
                                      hipStream_t stream,
                                      const GemvConvEpilogue* conv = nullptr);
// One-token GEMV of the gated delta net's output: x = per 128-value head,
// input * rsqrt(mean(input^2) + eps) * gate_factor[c]; output = residual + W x
// (residual may be null or the output).
hipError_t launch_kquant_matvec_head_norm(int format, const void* weight, size_t rows,
                                          size_t cols, const float* input,
                                          const float* gate_factor, float eps,
                                          const float* residual, float* output,
                                          hipStream_t stream);
// One-token GEMV output[r] = residual[r] (if given) + sum_k W[r][k] x_k, with x =
// RMSNorm(input) * norm_weight (if norm_weight), silu(input) * up (if up), or input.
hipError_t launch_kquant_matvec_fused(int format, const void* weight, size_t rows, size_t cols,
                                      const float* input, const float* norm_weight, float eps,
                                      const float* up, const float* residual, float* output,
                                      hipStream_t stream);

// RMSNorm of `rows` rows of `size` values, input -> output (may alias).
hipError_t launch_rms_norm_rows(const float* input, const float* weight, float* output,
                                uint32_t rows, uint32_t size, float eps, hipStream_t stream);
hipError_t launch_rms_norm_heads(float* values, const float* weight, const float* gate,
                                 uint32_t tokens, uint32_t heads, uint32_t head_dim,
                                 float eps, hipStream_t stream);
hipError_t launch_prepare_gate_beta(float* gate, float* beta, const float* bias,
                                    const float* scale, uint32_t rows, uint32_t row_size,
                                    hipStream_t stream);
hipError_t launch_mrope(float* values, const int32_t* positions, uint32_t tokens,
                        uint32_t heads, uint32_t head_dim, uint32_t n_dims, uint32_t s0,
                        uint32_t s1, uint32_t s2, uint32_t s3, float theta,
                        hipStream_t stream);
enum class CopyKind { f32, f32_to_f16, f16 };
hipError_t launch_copy_rows(CopyKind kind, const void* source, void* destination,
                            size_t rows, size_t row_size, size_t source_stride,
                            size_t source_offset, size_t destination_stride,
                            size_t destination_offset, hipStream_t stream);
enum class UnaryKind { sigmoid, softplus, silu };
hipError_t launch_unary(UnaryKind kind, float* values, size_t size, hipStream_t stream);
enum class BinaryKind { mul, add_row, mul_row, add, silu_mul };
hipError_t launch_binary(BinaryKind kind, float* target, const float* rhs, size_t size,
                         size_t row_size, hipStream_t stream);

}  // namespace kraken
