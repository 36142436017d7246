// C-ABI entry points of the K-quant projections and the device argmax:
// argument validation in the reference's order and wording ("HIP" in place of
// "MPS"), then dispatch to kquant.hip.  Host dispatchers followed:
// make_q*_k_matvec_layout / make_k_quant_matmul_layout (mps_backend.mm:
// 4036-4189), matvec_q*_k_f32_device (:6134-6197), matvec_q*_k_f32_top1
// (:6199-6271), matvec_q*_k_f32_argmax (:6273-6334), matmul_q*_k_f32_device
// (:6336-6450), dequantize_row(s)_q*_k_f32 (:7217-7756), argmax_f32_i32 /
// argmax_prob_f32_i32 (:10004-10120).  The Q5_K and Q6_K methods repeat the
// Q4_K ones with their names and block sizes.
//
// Beyond the reference, the device kernels read weights as 32-bit words and
// the input as 16-byte vectors, so the weight must be 4-byte aligned (Q6_K:
// 2-byte, its blocks are 210 bytes) and the input 16-byte aligned; any
// allocation of this library or of torch is.
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>
#include <string>

#include "context_internal.hpp"

using namespace kraken;

namespace {

constexpr size_t kTop1MaxBlocksPerRow = 16;  // kKQuantTop1MaxBlocksPerRow, mps_backend.mm:3798

const char* fmt_name(int format) {
  return format == 0 ? "Q4_K" : (format == 1 ? "Q5_K" : "Q6_K");
}

struct Layout {
  size_t blocks_per_row = 0;
  size_t weight_bytes = 0;
};

// make_q*_k_matvec_layout (mps_backend.mm:4036-4141).
int matvec_layout(int format, size_t rows, size_t cols, Layout& out) {
  const std::string p = std::string("HIP ") + fmt_name(format) + " matvec ";
  if (rows == 0 || cols == 0) {
    return invalid(p + "rows and cols must be greater than zero");
  }
  if (cols % 256u != 0) {
    return invalid(p + "cols must be divisible by 256");
  }
  if (!fits_u32(cols)) {
    return invalid(p + "cols exceeds uint32 range");
  }
  out.blocks_per_row = cols / 256u;
  size_t total_blocks = 0;
  if (!checked_mul(rows, out.blocks_per_row, total_blocks)) {
    return invalid(p + "block count overflow");
  }
  if (!checked_mul(total_blocks, kquant_block_bytes(format), out.weight_bytes)) {
    return invalid(p + "weight byte count overflow");
  }
  size_t bytes = 0;
  if (!checked_mul(cols, sizeof(float), bytes) || !checked_mul(rows, sizeof(float), bytes)) {
    return invalid(p + "buffer byte count overflow");
  }
  return KRAKEN_OK;
}

int check_alignment(int format, const kraken_buffer& weight, const kraken_buffer& input,
                    const char* what) {
  const uintptr_t need = format == 2 ? 2u : 4u;
  if (((uintptr_t)weight.data & (need - 1u)) != 0) {
    return invalid(std::string("HIP ") + fmt_name(format) + " " + what +
                   " weight buffer must be " + (format == 2 ? "2" : "4") + "-byte aligned");
  }
  if (((uintptr_t)input.data & 15u) != 0) {
    return invalid(std::string("HIP ") + fmt_name(format) + " " + what +
                   " input buffer must be 16-byte aligned");
  }
  return KRAKEN_OK;
}

// matvec_q*_k_f32_device (mps_backend.mm:6134-6197).
int matvec_entry(kraken_hip_context* ctx, int format, const kraken_buffer& weight, size_t rows,
                 size_t cols, const kraken_buffer& input, const kraken_buffer& output) {
  KRAKEN_TRY(check_context(ctx));
  const std::string f = fmt_name(format);
  if (weight.data == nullptr) {
    return invalid("HIP " + f + " weight buffer is not initialized");
  }
  Layout l;
  KRAKEN_TRY(matvec_layout(format, rows, cols, l));
  if (weight.byte_size < l.weight_bytes) {
    return invalid("HIP " + f + " weight buffer is too small");
  }
  KRAKEN_TRY(validate_f32(input, cols, (f + " matvec input").c_str()));
  KRAKEN_TRY(validate_f32(output, rows, (f + " matvec output").c_str()));
  KRAKEN_TRY(check_alignment(format, weight, input, "matvec"));
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e =
    launch_kquant_matmul(format, weight.data, rows, cols, 1, static_cast<const float*>(input.data),
                         static_cast<float*>(output.data), nullptr, 0, ctx->stream);
  if (e != hipSuccess) {
    return internal("HIP " + f + " matvec launch failed: " + hipGetErrorString(e));
  }
  return finish_launch(ctx, ("HIP " + f + " matvec command failed: ").c_str());
}

// matvec_q*_k_f32_top1 / _argmax (mps_backend.mm:6199-6334): the logits of
// one token, then their argmax (and the top probability for top1).
int top1_entry(kraken_hip_context* ctx, int format, bool with_probability,
               const kraken_buffer& weight, size_t rows, size_t cols, const kraken_buffer& input,
               const kraken_buffer& token_output, const kraken_buffer* probability_output) {
  KRAKEN_TRY(check_context(ctx));
  const std::string f = fmt_name(format);
  const std::string w = with_probability ? " top1" : " argmax";
  if (weight.data == nullptr) {
    return invalid("HIP " + f + w + " weight buffer is not initialized");
  }
  Layout l;
  KRAKEN_TRY(matvec_layout(format, rows, cols, l));
  if (l.blocks_per_row > kTop1MaxBlocksPerRow) {
    return invalid("HIP " + f + w + " block count exceeds kernel limit");
  }
  if (weight.byte_size < l.weight_bytes) {
    return invalid("HIP " + f + w + " weight buffer is too small");
  }
  KRAKEN_TRY(validate_f32(input, cols, (f + w + " input").c_str()));
  KRAKEN_TRY(validate_i32(token_output, 1, (f + w + " token output").c_str()));
  if (with_probability) {
    KRAKEN_TRY(validate_f32(*probability_output, 1, (f + w + " probability output").c_str()));
  }
  KRAKEN_TRY(check_alignment(format, weight, input, w.c_str() + 1));
  KRAKEN_TRY(ensure_workspace(ctx, kquant_argmax_workspace_bytes(rows)));
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e = launch_kquant_argmax(
    format, weight.data, rows, cols, static_cast<const float*>(input.data),
    static_cast<int32_t*>(token_output.data),
    with_probability ? static_cast<float*>(probability_output->data) : nullptr, ctx->workspace,
    ctx->workspace_bytes, ctx->stream);
  if (e != hipSuccess) {
    return internal("HIP " + f + w + " launch failed: " + hipGetErrorString(e));
  }
  return finish_launch(ctx, ("HIP " + f + w + " command failed: ").c_str());
}

// matmul_q*_k_f32_device with make_k_quant_matmul_layout (mps_backend.mm:
// 4143-4189, 6336-6450).
int matmul_check(kraken_hip_context* ctx, int format, const kraken_buffer& weight, size_t rows,
                 size_t cols, size_t tokens, const kraken_buffer& input,
                 const kraken_buffer& output) {
  KRAKEN_TRY(check_context(ctx));
  const std::string f = fmt_name(format);
  const std::string p = "HIP " + f + " matmul ";
  if (weight.data == nullptr) {
    return invalid("HIP " + f + " weight buffer is not initialized");
  }
  if (rows == 0 || cols == 0 || tokens == 0) {
    return invalid(p + "rows, cols and tokens must be greater than zero");
  }
  if (cols % 256u != 0) {
    return invalid(p + "cols must be divisible by 256");
  }
  if (!fits_u32(cols) || !fits_u32(rows) || !fits_u32(tokens)) {
    return invalid(p + "dimensions exceed uint32 range");
  }
  const size_t blocks_per_row = cols / 256u;
  size_t total_blocks = 0;
  size_t weight_bytes = 0;
  if (!checked_mul(rows, blocks_per_row, total_blocks)) {
    return invalid(p + "block count overflow");
  }
  if (!checked_mul(total_blocks, kquant_block_bytes(format), weight_bytes)) {
    return invalid(p + "weight byte count overflow");
  }
  size_t input_values = 0;
  size_t output_values = 0;
  size_t bytes = 0;
  if (!checked_mul(tokens, cols, input_values) || !checked_mul(tokens, rows, output_values) ||
      !checked_mul(input_values, sizeof(float), bytes) ||
      !checked_mul(output_values, sizeof(float), bytes)) {
    return invalid(p + "buffer byte count overflow");
  }
  if (weight.byte_size < weight_bytes) {
    return invalid(p + "weight buffer is too small");
  }
  KRAKEN_TRY(validate_f32(input, input_values, (f + " matmul input").c_str()));
  KRAKEN_TRY(validate_f32(output, output_values, (f + " matmul output").c_str()));
  KRAKEN_TRY(check_alignment(format, weight, input, "matmul"));
  return KRAKEN_OK;
}

int matmul_entry(kraken_hip_context* ctx, int format, const kraken_buffer& weight, size_t rows,
                 size_t cols, size_t tokens, const kraken_buffer& input,
                 const kraken_buffer& output) {
  KRAKEN_TRY(matmul_check(ctx, format, weight, rows, cols, tokens, input, output));
  const std::string p = std::string("HIP ") + fmt_name(format) + " matmul ";
  KRAKEN_TRY(ensure_workspace(ctx, kquant_matmul_workspace_bytes(format, rows, cols, tokens)));
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e = launch_kquant_matmul(
    format, weight.data, rows, cols, tokens, static_cast<const float*>(input.data),
    static_cast<float*>(output.data), ctx->workspace, ctx->workspace_bytes, ctx->stream);
  if (e != hipSuccess) {
    return internal(p + "launch failed: " + hipGetErrorString(e));
  }
  return finish_launch(ctx, (p + "command failed: ").c_str());
}

// dequantize_row_q*_k_f32 (mps_backend.mm:7217-7283).
int get_row_entry(kraken_hip_context* ctx, int format, const kraken_buffer& weight, size_t row,
                  size_t cols, const kraken_buffer& output) {
  KRAKEN_TRY(check_context(ctx));
  const std::string f = fmt_name(format);
  const std::string p = "HIP " + f + " get-row ";
  if (weight.data == nullptr) {
    return invalid(p + "weight buffer is not initialized");
  }
  if (cols == 0 || cols % 256u != 0) {
    return invalid(p + "cols must be positive and divisible by 256");
  }
  const size_t blocks_per_row = cols / 256u;
  size_t row_bytes = 0;
  size_t required = 0;
  if (row == SIZE_MAX || !checked_mul(blocks_per_row, kquant_block_bytes(format), row_bytes) ||
      !checked_mul(row + 1u, row_bytes, required)) {
    return invalid(p + "weight byte count overflow");
  }
  if (weight.byte_size < required) {
    return invalid(p + "weight buffer is too small");
  }
  KRAKEN_TRY(validate_f32(output, cols, (f + " get-row output").c_str()));
  KRAKEN_TRY(check_u32(row, (f + " get-row row").c_str()));
  KRAKEN_TRY(check_u32(cols, (f + " get-row cols").c_str()));
  KRAKEN_TRY(check_u32(blocks_per_row, (f + " get-row blocks").c_str()));
  if (((uintptr_t)weight.data & (format == 2 ? 1u : 3u)) != 0 ||
      ((uintptr_t)output.data & 15u) != 0) {
    return invalid(p + "weight or output buffer is not aligned");
  }
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e = launch_kquant_dequantize_rows(format, weight.data, row + 1u, nullptr, row,
                                                     1, cols, static_cast<float*>(output.data),
                                                     ctx->stream);
  if (e != hipSuccess) {
    return internal(p + "launch failed: " + hipGetErrorString(e));
  }
  return finish_launch(ctx, (p + "command failed: ").c_str());
}

// dequantize_rows_q*_k_f32 (mps_backend.mm:7285-7380): row_ids i32 [tokens].
int get_rows_entry(kraken_hip_context* ctx, int format, const kraken_buffer& weight, size_t rows,
                   const kraken_buffer& row_ids, size_t tokens, size_t cols,
                   const kraken_buffer& output) {
  KRAKEN_TRY(check_context(ctx));
  const std::string f = fmt_name(format);
  const std::string p = "HIP " + f + " get-rows ";
  if (weight.data == nullptr) {
    return invalid(p + "weight buffer is not initialized");
  }
  if (rows == 0 || tokens == 0 || cols == 0 || cols % 256u != 0) {
    return invalid(p + "rows, tokens and cols must be positive and cols divisible by 256");
  }
  const size_t blocks_per_row = cols / 256u;
  size_t row_bytes = 0;
  size_t required = 0;
  if (!checked_mul(blocks_per_row, kquant_block_bytes(format), row_bytes) ||
      !checked_mul(rows, row_bytes, required)) {
    return invalid(p + "weight byte count overflow");
  }
  if (weight.byte_size < required) {
    return invalid(p + "weight buffer is too small");
  }
  KRAKEN_TRY(validate_i32(row_ids, tokens, (f + " get-rows row ids").c_str()));
  size_t total = 0;
  if (!checked_mul(cols, tokens, total)) {
    return invalid(p + "value count overflow");
  }
  KRAKEN_TRY(validate_f32(output, total, (f + " get-rows output").c_str()));
  KRAKEN_TRY(check_u32(rows, (f + " get-rows rows").c_str()));
  KRAKEN_TRY(check_u32(tokens, (f + " get-rows tokens").c_str()));
  KRAKEN_TRY(check_u32(cols, (f + " get-rows cols").c_str()));
  if (((uintptr_t)weight.data & (format == 2 ? 1u : 3u)) != 0 ||
      ((uintptr_t)output.data & 15u) != 0) {
    return invalid(p + "weight or output buffer is not aligned");
  }
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e = launch_kquant_dequantize_rows(
    format, weight.data, rows, static_cast<const int32_t*>(row_ids.data), 0, tokens, cols,
    static_cast<float*>(output.data), ctx->stream);
  if (e != hipSuccess) {
    return internal(p + "launch failed: " + hipGetErrorString(e));
  }
  return finish_launch(ctx, (p + "command failed: ").c_str());
}

// argmax_f32_i32 / argmax_prob_f32_i32 (mps_backend.mm:10004-10120).
int argmax_entry(kraken_hip_context* ctx, bool with_probability, const kraken_buffer& values,
                 size_t size, const kraken_buffer& token_output,
                 const kraken_buffer* probability_output) {
  KRAKEN_TRY(check_context(ctx));
  const std::string w = with_probability ? "argmax probability" : "argmax";
  if (size == 0) {
    return invalid("HIP " + w + " size must be positive");
  }
  KRAKEN_TRY(check_u32(size, (w + " size").c_str()));
  KRAKEN_TRY(validate_f32(values, size, (w + " values").c_str()));
  const std::string out = with_probability ? " token output" : " output";
  if (token_output.data == nullptr) {
    return invalid("HIP " + w + out + " buffer is not initialized");
  }
  if (token_output.byte_size < sizeof(int32_t)) {
    return invalid("HIP " + w + out + " buffer is too small");
  }
  if (with_probability) {
    KRAKEN_TRY(validate_f32(*probability_output, 1, (w + " output").c_str()));
  }
  KRAKEN_TRY(ensure_workspace(ctx, argmax_workspace_bytes(size)));
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e = launch_argmax(
    static_cast<const float*>(values.data), size, static_cast<int32_t*>(token_output.data),
    with_probability ? static_cast<float*>(probability_output->data) : nullptr, ctx->workspace,
    ctx->workspace_bytes, ctx->stream);
  if (e != hipSuccess) {
    return internal("HIP " + w + " launch failed: " + hipGetErrorString(e));
  }
  return finish_launch(ctx, ("HIP " + w + " command failed: ").c_str());
}

// GGUF type id (12, 13, 14) -> this file's format index, or -1.
int format_of_ggml_type(uint32_t ggml_type) {
  return ggml_type >= 12u && ggml_type <= 14u ? (int)(ggml_type - 12u) : -1;
}

// Checks shared by the fused entries: type, weight, dimensions, input; returns
// the format index through `format`.
int fused_common(kraken_hip_context* ctx, const char* what, uint32_t ggml_type,
                 const kraken_buffer& weight, size_t rows, size_t cols,
                 const kraken_buffer& input, const kraken_buffer& norm_weight, int& format) {
  KRAKEN_TRY(check_context(ctx));
  const std::string p = std::string("HIP ") + what + " ";
  format = format_of_ggml_type(ggml_type);
  if (format < 0) {
    return invalid(p + "weight type must be Q4_K (12), Q5_K (13) or Q6_K (14)");
  }
  if (weight.data == nullptr) {
    return invalid(p + "weight buffer is not initialized");
  }
  Layout l;
  KRAKEN_TRY(matvec_layout(format, rows, cols, l));
  if (weight.byte_size < l.weight_bytes) {
    return invalid(p + "weight buffer is too small");
  }
  KRAKEN_TRY(validate_f32(input, cols, (std::string(what) + " input").c_str()));
  if (norm_weight.data != nullptr) {
    KRAKEN_TRY(validate_f32(norm_weight, cols, (std::string(what) + " norm weight").c_str()));
    if (((uintptr_t)norm_weight.data & 15u) != 0) {
      return invalid(p + "norm weight buffer must be 16-byte aligned");
    }
  }
  return check_alignment(format, weight, input, what);
}

}  // namespace

extern "C" {

#define KRAKEN_KQUANT_ENTRIES(FMT, ID)                                                          \
  KRAKEN_API int kraken_hip_matvec_##FMT##_f32_device(kraken_hip_context* ctx,                 \
                                                      kraken_buffer weight, size_t rows,        \
                                                      size_t cols, kraken_buffer input,         \
                                                      kraken_buffer output) {                   \
    return matvec_entry(ctx, ID, weight, rows, cols, input, output);                           \
  }                                                                                            \
  KRAKEN_API int kraken_hip_matvec_##FMT##_f32_top1(                                           \
    kraken_hip_context* ctx, kraken_buffer weight, size_t rows, size_t cols,                   \
    kraken_buffer input, kraken_buffer token_output, kraken_buffer probability_output) {       \
    return top1_entry(ctx, ID, true, weight, rows, cols, input, token_output,                  \
                      &probability_output);                                                    \
  }                                                                                            \
  KRAKEN_API int kraken_hip_matvec_##FMT##_f32_argmax(kraken_hip_context* ctx,                 \
                                                      kraken_buffer weight, size_t rows,        \
                                                      size_t cols, kraken_buffer input,         \
                                                      kraken_buffer token_output) {             \
    return top1_entry(ctx, ID, false, weight, rows, cols, input, token_output, nullptr);       \
  }                                                                                            \
  KRAKEN_API int kraken_hip_matmul_##FMT##_f32_device(                                         \
    kraken_hip_context* ctx, kraken_buffer weight, size_t rows, size_t cols, size_t tokens,    \
    kraken_buffer input, kraken_buffer output) {                                               \
    return matmul_entry(ctx, ID, weight, rows, cols, tokens, input, output);                   \
  }                                                                                            \
  KRAKEN_API int kraken_hip_dequantize_row_##FMT##_f32(kraken_hip_context* ctx,                \
                                                       kraken_buffer weight, size_t row,        \
                                                       size_t cols, kraken_buffer output) {     \
    return get_row_entry(ctx, ID, weight, row, cols, output);                                  \
  }                                                                                            \
  KRAKEN_API int kraken_hip_dequantize_rows_##FMT##_f32(                                       \
    kraken_hip_context* ctx, kraken_buffer weight, size_t rows, kraken_buffer row_ids,         \
    size_t tokens, size_t cols, kraken_buffer output) {                                        \
    return get_rows_entry(ctx, ID, weight, rows, row_ids, tokens, cols, output);               \
  }

KRAKEN_KQUANT_ENTRIES(q4_k, 0)
KRAKEN_KQUANT_ENTRIES(q5_k, 1)
KRAKEN_KQUANT_ENTRIES(q6_k, 2)
#undef KRAKEN_KQUANT_ENTRIES

KRAKEN_API int kraken_hip_argmax_f32_i32(kraken_hip_context* ctx, kraken_buffer values,
                                         size_t size, kraken_buffer output) {
  return argmax_entry(ctx, false, values, size, output, nullptr);
}

KRAKEN_API int kraken_hip_argmax_prob_f32_i32(kraken_hip_context* ctx, kraken_buffer values,
                                              size_t size, kraken_buffer token_output,
                                              kraken_buffer probability_output) {
  return argmax_entry(ctx, true, values, size, token_output, &probability_output);
}

// No counterpart in the reference: the one-token K-quant GEMV with the
// decoder layer's RMSNorm (or SwiGLU) on its input and residual add on its
// output folded in (see include/kraken_hip.h).
KRAKEN_API int kraken_hip_kquant_matvec_fused_f32(kraken_hip_context* ctx, uint32_t ggml_type,
                                                  kraken_buffer weight, size_t rows, size_t cols,
                                                  kraken_buffer input, kraken_buffer norm_weight,
                                                  float eps, kraken_buffer up,
                                                  kraken_buffer residual, kraken_buffer output) {
  const char* what = "K-quant fused matvec";
  int format = -1;
  KRAKEN_TRY(fused_common(ctx, what, ggml_type, weight, rows, cols, input, norm_weight, format));
  if (norm_weight.data != nullptr && up.data != nullptr) {
    return invalid("HIP K-quant fused matvec takes a norm weight or an up input, not both");
  }
  if (up.data != nullptr) {
    KRAKEN_TRY(validate_f32(up, cols, "K-quant fused matvec up"));
    if (((uintptr_t)up.data & 15u) != 0) {
      return invalid("HIP K-quant fused matvec up buffer must be 16-byte aligned");
    }
  }
  if (residual.data != nullptr) {
    KRAKEN_TRY(validate_f32(residual, rows, "K-quant fused matvec residual"));
  }
  KRAKEN_TRY(validate_f32(output, rows, "K-quant fused matvec output"));
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e = launch_kquant_matvec_fused(
    format, weight.data, rows, cols, static_cast<const float*>(input.data),
    static_cast<const float*>(norm_weight.data), eps, static_cast<const float*>(up.data),
    static_cast<const float*>(residual.data), static_cast<float*>(output.data), ctx->stream);
  if (e != hipSuccess) {
    return internal(std::string("HIP K-quant fused matvec launch failed: ") +
                    hipGetErrorString(e));
  }
  return finish_launch(ctx, "HIP K-quant fused matvec command failed: ");
}

// No counterpart in the reference: matvec_q*_k_f32_top1 / _argmax with the
// output norm folded into the logits GEMV (norm_weight may be empty);
// probability_output may be empty for the argmax alone.
KRAKEN_API int kraken_hip_kquant_top1_fused_f32(kraken_hip_context* ctx, uint32_t ggml_type,
                                                kraken_buffer weight, size_t rows, size_t cols,
                                                kraken_buffer input, kraken_buffer norm_weight,
                                                float eps, kraken_buffer token_output,
                                                kraken_buffer probability_output) {
  const char* what = "K-quant fused top1";
  int format = -1;
  KRAKEN_TRY(fused_common(ctx, what, ggml_type, weight, rows, cols, input, norm_weight, format));
  if (cols / 256u > kTop1MaxBlocksPerRow) {
    return invalid("HIP K-quant fused top1 block count exceeds kernel limit");
  }
  KRAKEN_TRY(validate_i32(token_output, 1, "K-quant fused top1 token output"));
  if (probability_output.data != nullptr) {
    KRAKEN_TRY(validate_f32(probability_output, 1, "K-quant fused top1 probability output"));
  }
  KRAKEN_TRY(ensure_workspace(ctx, kquant_argmax_workspace_bytes(rows)));
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e = launch_kquant_argmax(
    format, weight.data, rows, cols, static_cast<const float*>(input.data),
    static_cast<int32_t*>(token_output.data), static_cast<float*>(probability_output.data),
    ctx->workspace, ctx->workspace_bytes, ctx->stream,
    static_cast<const float*>(norm_weight.data), eps);
  if (e != hipSuccess) {
    return internal(std::string("HIP K-quant fused top1 launch failed: ") + hipGetErrorString(e));
  }
  return finish_launch(ctx, "HIP K-quant fused top1 command failed: ");
}

// No counterpart in the reference: up to four fused one-token GEMVs that read
// the same input (the projections of one normed hidden state) in one launch.
KRAKEN_API int kraken_hip_kquant_matvec_multi_f32(
  kraken_hip_context* ctx, size_t count, const uint32_t* ggml_types, const kraken_buffer* weights,
  const size_t* rows, size_t cols, kraken_buffer input, kraken_buffer norm_weight, float eps,
  kraken_buffer up, const kraken_buffer* residuals, const kraken_buffer* outputs) {
  const char* what = "K-quant multi matvec";
  KRAKEN_TRY(check_context(ctx));
  if (count == 0 || count > kKquantMultiMaxMatrices) {
    return invalid("HIP K-quant multi matvec takes 1 to 4 matrices");
  }
  if (ggml_types == nullptr || weights == nullptr || rows == nullptr || residuals == nullptr ||
      outputs == nullptr) {
    return invalid("HIP K-quant multi matvec array argument is null");
  }
  if (cols > kKquantMultiMaxCols) {
    return invalid("HIP K-quant multi matvec cols exceeds 4096");
  }
  if (norm_weight.data != nullptr && up.data != nullptr) {
    return invalid("HIP K-quant multi matvec takes a norm weight or an up input, not both");
  }
  int formats[kKquantMultiMaxMatrices];
  const void* w[kKquantMultiMaxMatrices];
  const float* res[kKquantMultiMaxMatrices];
  float* out[kKquantMultiMaxMatrices];
  for (size_t i = 0; i < count; ++i) {
    KRAKEN_TRY(fused_common(ctx, what, ggml_types[i], weights[i], rows[i], cols, input,
                            norm_weight, formats[i]));
    if (residuals[i].data != nullptr) {
      KRAKEN_TRY(validate_f32(residuals[i], rows[i], "K-quant multi matvec residual"));
    }
    KRAKEN_TRY(validate_f32(outputs[i], rows[i], "K-quant multi matvec output"));
    w[i] = weights[i].data;
    res[i] = static_cast<const float*>(residuals[i].data);
    out[i] = static_cast<float*>(outputs[i].data);
  }
  if (up.data != nullptr) {
    KRAKEN_TRY(validate_f32(up, cols, "K-quant multi matvec up"));
    if (((uintptr_t)up.data & 15u) != 0) {
      return invalid("HIP K-quant multi matvec up buffer must be 16-byte aligned");
    }
  }
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e = launch_kquant_matvec_multi(
    (uint32_t)count, formats, w, rows, cols, static_cast<const float*>(input.data),
    static_cast<const float*>(norm_weight.data), eps, static_cast<const float*>(up.data), res,
    out, ctx->stream);
  if (e != hipSuccess) {
    return internal(std::string("HIP K-quant multi matvec launch failed: ") +
                    hipGetErrorString(e));
  }
  return finish_launch(ctx, "HIP K-quant multi matvec command failed: ");
}

// No counterpart in the reference: the multi GEMV above (no up input, no
// residuals) whose matrix 0 rows are the conv channels of one sequence: each
// row's value goes through the depthwise conv (kernel 4) and SiLU of the
// linear-attention prologue, and its conv state shifts, as the row is written.
KRAKEN_API int kraken_hip_kquant_matmul_fused_f32(kraken_hip_context* ctx, uint32_t ggml_type,
                                                  kraken_buffer weight, size_t rows, size_t cols,
                                                  size_t tokens, kraken_buffer input,
                                                  kraken_buffer up, kraken_buffer residual,
                                                  kraken_buffer output) {
  KRAKEN_TRY(check_context(ctx));
  const int format = format_of_ggml_type(ggml_type);
  if (format < 0) {
    return invalid("HIP K-quant fused matmul type must be Q4_K, Q5_K or Q6_K");
  }
  KRAKEN_TRY(matmul_check(ctx, format, weight, rows, cols, tokens, input, output));
  if (tokens <= kKquantGemvMaxTokens) {
    return invalid("HIP K-quant fused matmul needs more than 8 tokens");
  }
  if (up.data != nullptr) {
    KRAKEN_TRY(validate_f32(up, tokens * cols, "K-quant fused matmul up"));
    if (((uintptr_t)up.data & 15u) != 0) {
      return invalid("HIP K-quant fused matmul up buffer must be 16-byte aligned");
    }
  }
  if (residual.data != nullptr) {
    KRAKEN_TRY(validate_f32(residual, tokens * rows, "K-quant fused matmul residual"));
    if (((uintptr_t)residual.data & 15u) != 0) {
      return invalid("HIP K-quant fused matmul residual buffer must be 16-byte aligned");
    }
    // Each output element is read from the residual and written by one thread:
    // the residual may be the output itself, but not a shifted view of it.
    const uintptr_t r0 = (uintptr_t)residual.data, o0 = (uintptr_t)output.data;
    const size_t bytes = tokens * rows * sizeof(float);
    if (r0 != o0 && r0 < o0 + bytes && o0 < r0 + bytes) {
      return invalid("HIP K-quant fused matmul residual overlaps the output");
    }
  }
  const std::string p = std::string("HIP ") + fmt_name(format) + " fused matmul ";
  KRAKEN_TRY(ensure_workspace(
    ctx, kquant_matmul_workspace_bytes(format, rows, cols, tokens, up.data != nullptr)));
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e = launch_kquant_matmul(
    format, weight.data, rows, cols, tokens, static_cast<const float*>(input.data),
    static_cast<float*>(output.data), ctx->workspace, ctx->workspace_bytes, ctx->stream,
    static_cast<const float*>(up.data), static_cast<const float*>(residual.data));
  if (e != hipSuccess) {
    return internal(p + "launch failed: " + hipGetErrorString(e));
  }
  return finish_launch(ctx, (p + "command failed: ").c_str());
}

KRAKEN_API int kraken_hip_kquant_matmul_multi_f32(kraken_hip_context* ctx, size_t count,
                                                  const uint32_t* ggml_types,
                                                  const kraken_buffer* weights, const size_t* rows,
                                                  size_t cols, size_t tokens, kraken_buffer input,
                                                  const kraken_buffer* outputs) {
  KRAKEN_TRY(check_context(ctx));
  if (count == 0 || count > kKquantGroupMax) {
    return invalid("HIP K-quant multi matmul takes 1 to 4 matrices");
  }
  if (ggml_types == nullptr || weights == nullptr || rows == nullptr || outputs == nullptr) {
    return invalid("HIP K-quant multi matmul array argument is null");
  }
  int formats[kKquantGroupMax];
  const void* w[kKquantGroupMax];
  float* out[kKquantGroupMax];
  bool same_format = true;
  for (size_t i = 0; i < count; ++i) {
    formats[i] = format_of_ggml_type(ggml_types[i]);
    if (formats[i] < 0) {
      return invalid("HIP K-quant multi matmul type must be Q4_K, Q5_K or Q6_K");
    }
    KRAKEN_TRY(matmul_check(ctx, formats[i], weights[i], rows[i], cols, tokens, input,
                            outputs[i]));
    w[i] = weights[i].data;
    out[i] = static_cast<float*>(outputs[i].data);
    same_format = same_format && formats[i] == formats[0];
  }
  const char* group = std::getenv("KRAKEN_KQUANT_GROUP");
  if (same_format && (group == nullptr || std::strcmp(group, "off") != 0)) {
    KRAKEN_TRY(begin_launch(ctx));
    const hipError_t e =
      launch_kquant_matmul_group(formats[0], count, w, rows, cols, tokens,
                                 static_cast<const float*>(input.data), out, ctx->stream);
    if (e == hipSuccess) {
      return finish_launch(ctx, "HIP K-quant multi matmul command failed: ");
    }
    if (e != hipErrorNotSupported) {
      return internal(std::string("HIP K-quant multi matmul launch failed: ") +
                      hipGetErrorString(e));
    }
  }
  for (size_t i = 0; i < count; ++i) {
    KRAKEN_TRY(matmul_entry(ctx, formats[i], weights[i], rows[i], cols, tokens, input,
                            outputs[i]));
  }
  return KRAKEN_OK;
}

KRAKEN_API int kraken_hip_kquant_matvec_multi_conv_f32(
  kraken_hip_context* ctx, size_t count, const uint32_t* ggml_types, const kraken_buffer* weights,
  const size_t* rows, size_t cols, kraken_buffer input, kraken_buffer norm_weight, float eps,
  const kraken_buffer* outputs, kraken_buffer conv_pool, kraken_buffer conv_offset,
  kraken_buffer conv_kernel_weights, size_t conv_kernel) {
  const char* what = "K-quant multi conv matvec";
  KRAKEN_TRY(check_context(ctx));
  if (count == 0 || count > kKquantMultiMaxMatrices) {
    return invalid("HIP K-quant multi conv matvec takes 1 to 4 matrices");
  }
  if (ggml_types == nullptr || weights == nullptr || rows == nullptr || outputs == nullptr) {
    return invalid("HIP K-quant multi conv matvec array argument is null");
  }
  if (cols > kKquantMultiMaxCols) {
    return invalid("HIP K-quant multi conv matvec cols exceeds 4096");
  }
  if (conv_kernel != 4) {
    return invalid("HIP K-quant multi conv matvec conv_kernel must be 4");
  }
  if (norm_weight.data == nullptr) {
    return invalid("HIP K-quant multi conv matvec needs a norm weight");
  }
  int formats[kKquantMultiMaxMatrices];
  const void* w[kKquantMultiMaxMatrices];
  const float* res[kKquantMultiMaxMatrices] = {nullptr, nullptr, nullptr, nullptr};
  float* out[kKquantMultiMaxMatrices];
  for (size_t i = 0; i < count; ++i) {
    KRAKEN_TRY(fused_common(ctx, what, ggml_types[i], weights[i], rows[i], cols, input,
                            norm_weight, formats[i]));
    KRAKEN_TRY(validate_f32(outputs[i], rows[i], "K-quant multi conv matvec output"));
    w[i] = weights[i].data;
    out[i] = static_cast<float*>(outputs[i].data);
  }
  size_t state_values = 0, kernel_values = 0;
  if (!checked_mul(rows[0], conv_kernel - 1u, state_values) ||
      !checked_mul(rows[0], conv_kernel, kernel_values)) {
    return invalid("HIP K-quant multi conv matvec value count overflow");
  }
  KRAKEN_TRY(validate_f32(conv_pool, state_values, "K-quant multi conv matvec conv pool"));
  if (conv_pool.byte_size % sizeof(float) != 0) {
    return invalid("HIP K-quant multi conv matvec conv pool size is not a whole number of "
                   "elements");
  }
  KRAKEN_TRY(validate_buffer(conv_offset, 1, sizeof(uint64_t),
                             "K-quant multi conv matvec conv offset"));
  KRAKEN_TRY(validate_f32(conv_kernel_weights, kernel_values,
                          "K-quant multi conv matvec conv kernel"));
  KRAKEN_TRY(begin_launch(ctx));
  const GemvConvEpilogue conv{static_cast<float*>(conv_pool.data),
                              static_cast<const uint64_t*>(conv_offset.data),
                              (uint64_t)(conv_pool.byte_size / sizeof(float)),
                              static_cast<const float*>(conv_kernel_weights.data)};
  const hipError_t e = launch_kquant_matvec_multi(
    (uint32_t)count, formats, w, rows, cols, static_cast<const float*>(input.data),
    static_cast<const float*>(norm_weight.data), eps, nullptr, res, out, ctx->stream, &conv);
  if (e != hipSuccess) {
    return internal(std::string("HIP K-quant multi conv matvec launch failed: ") +
                    hipGetErrorString(e));
  }
  return finish_launch(ctx, "HIP K-quant multi conv matvec command failed: ");
}

// No counterpart in the reference: the one-token GEMV of the linear-attention
// output projection with the rest of the norm-gated epilogue
// (qwen35_norm_gated_f32_in_place) on its input, given the epilogue's
// per-value factor, and the residual add on its output.
KRAKEN_API int kraken_hip_kquant_matvec_head_norm_f32(
  kraken_hip_context* ctx, uint32_t ggml_type, kraken_buffer weight, size_t rows, size_t cols,
  kraken_buffer input, kraken_buffer gate_factor, size_t head_dim, float eps,
  kraken_buffer residual, kraken_buffer output) {
  const char* what = "K-quant head-norm matvec";
  int format = -1;
  const kraken_buffer none{};
  KRAKEN_TRY(fused_common(ctx, what, ggml_type, weight, rows, cols, input, none, format));
  if (head_dim != 128) {
    return invalid("HIP K-quant head-norm matvec head_dim must be 128");
  }
  if (cols > kKquantMultiMaxCols) {
    return invalid("HIP K-quant head-norm matvec cols exceeds 4096");
  }
  KRAKEN_TRY(validate_f32(gate_factor, cols, "K-quant head-norm matvec gate factor"));
  if (((uintptr_t)gate_factor.data & 15u) != 0) {
    return invalid("HIP K-quant head-norm matvec gate factor must be 16-byte aligned");
  }
  if (residual.data != nullptr) {
    KRAKEN_TRY(validate_f32(residual, rows, "K-quant head-norm matvec residual"));
  }
  KRAKEN_TRY(validate_f32(output, rows, "K-quant head-norm matvec output"));
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e = launch_kquant_matvec_head_norm(
    format, weight.data, rows, cols, static_cast<const float*>(input.data),
    static_cast<const float*>(gate_factor.data), eps, static_cast<const float*>(residual.data),
    static_cast<float*>(output.data), ctx->stream);
  if (e != hipSuccess) {
    return internal(std::string("HIP K-quant head-norm matvec launch failed: ") +
                    hipGetErrorString(e));
  }
  return finish_launch(ctx, "HIP K-quant head-norm matvec command failed: ");
}

}  // extern "C"
