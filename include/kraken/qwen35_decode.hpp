// The Qwen3.5 decode step on the device: token embedding, the main-layer loop
// of run_qwen35_decode_tokens (src/runtime/qwen35_runtime.cpp:3860-3936) with
// each layer's norm, projections, attention core, residuals and SwiGLU FFN
// (run_qwen35_linear_layer_chunk :2634-3144, run_qwen35_full_attention_layer_chunk
// :3146-3423), the output norm (:3461-3503) and the greedy LM head
// (run_qwen35_lm_head_logits :3505-3647, its rows == 1 top-1 path), and the
// generation loop around it (:6212-6263: one graph per token, committed once).
//
// The next token never leaves the device inside the loop: the LM-head argmax
// writes it into a device token array, and the next step's embedding reads
// its row id from there.  Each step is one begin_graph / commit_graph batch,
// so the host waits once per token; the tokens are read back at the end.
#pragma once

#include <array>
#include <cstddef>
#include <cstdint>
#include <functional>
#include <string>
#include <vector>

#include "kraken/qwen35_layers.hpp"

namespace kraken::qwen35 {

// GGUF tensor type ids of the weights the decode step reads (gguf_reader.hpp).
enum class TensorType : std::uint32_t { f32 = 0, q4_k = 12, q5_k = 13, q6_k = 14 };

// A weight in device memory.  For a projection, rows = output values and
// cols = input values (GGUF shape {cols, rows}).
struct Tensor {
  const HipBuffer* buffer{nullptr};
  TensorType type{TensorType::f32};
  std::size_t rows{0};
  std::size_t cols{0};
};

// The weights of one main layer.  Layers of either kind have the norms and the
// FFN; the projections and core weights of the other kind stay empty.
struct DecoderLayerWeights {
  const HipBuffer* attn_norm{nullptr};            // [hidden]
  const HipBuffer* post_attention_norm{nullptr};  // [hidden]
  Tensor ffn_gate, ffn_up, ffn_down;
  // Linear attention: attn_qkv [conv_channels], attn_gate (z) [inner],
  // ssm_beta and ssm_alpha [value_heads], ssm_out [hidden] from [inner].
  Tensor qkv, gate, beta, alpha, ssm_out;
  LinearAttentionWeights linear;
  // Full attention: attn_q [heads * 2 * head_dim] (query and gate per head),
  // attn_k and attn_v [kv_heads * head_dim], attn_output [hidden] from
  // [heads * head_dim].
  Tensor q, k, v, output;
  FullAttentionWeights full;
};

struct ModelWeights {
  Tensor token_embd;                      // [vocab][hidden], a K-quant type
  const HipBuffer* output_norm{nullptr};  // [hidden]
  Tensor output;                          // LM head [vocab][hidden]; token_embd when tied
  std::vector<DecoderLayerWeights> layers;  // plan.main_layers entries
  std::array<std::size_t, 4> mrope_sections{11, 11, 10, 0};
  float rope_theta{1.0e7f};
  float rms_eps{1.0e-6f};
};

// run_qwen35_quant_matmul (qwen35_runtime.cpp:1972-2048): output[tokens][rows]
// = input[tokens][cols] times the K-quant weight.
[[nodiscard]] inline Status project(const HipContext& ctx, const Tensor& w,
                                    const HipBuffer& input, std::size_t tokens,
                                    HipBuffer& output) {
  if (tokens == 0) {
    return Status::invalid_argument("Qwen3.5 matmul requires tokens");
  }
  if (w.buffer == nullptr || w.rows == 0 || w.cols == 0) {
    return Status::invalid_argument("Qwen3.5 matmul weight is missing");
  }
  switch (w.type) {
    case TensorType::q4_k:
      return ctx.matmul_q4_k_f32_device(*w.buffer, w.rows, w.cols, tokens, input, output);
    case TensorType::q5_k:
      return ctx.matmul_q5_k_f32_device(*w.buffer, w.rows, w.cols, tokens, input, output);
    case TensorType::q6_k:
      return ctx.matmul_q6_k_f32_device(*w.buffer, w.rows, w.cols, tokens, input, output);
    default:
      return Status::invalid_argument("Qwen3.5 matmul weight type is not a K-quant type");
  }
}

// Up to four projections of the same input [tokens][cols] (one launch where
// kraken_hip_kquant_matmul_multi_f32 allows; the same checks as project).
[[nodiscard]] inline Status project_group(const HipContext& ctx, std::size_t count,
                                          const Tensor* const* w, const HipBuffer& input,
                                          std::size_t tokens, HipBuffer* const* outputs) {
  if (tokens == 0) {
    return Status::invalid_argument("Qwen3.5 matmul requires tokens");
  }
  if (count == 0 || count > 4) {
    return Status::invalid_argument("Qwen3.5 grouped matmul takes 1 to 4 weights");
  }
  std::uint32_t types[4];
  const HipBuffer* bufs[4];
  std::size_t rows[4];
  for (std::size_t i = 0; i < count; ++i) {
    if (w[i]->buffer == nullptr || w[i]->rows == 0 || w[i]->cols == 0) {
      return Status::invalid_argument("Qwen3.5 matmul weight is missing");
    }
    if (w[i]->type != TensorType::q4_k && w[i]->type != TensorType::q5_k &&
        w[i]->type != TensorType::q6_k) {
      return Status::invalid_argument("Qwen3.5 matmul weight type is not a K-quant type");
    }
    if (w[i]->cols != w[0]->cols) {
      return Status::invalid_argument("Qwen3.5 grouped matmul weights differ in cols");
    }
    types[i] = static_cast<std::uint32_t>(w[i]->type);
    bufs[i] = w[i]->buffer;
    rows[i] = w[i]->rows;
  }
  return ctx.kquant_matmul_multi_f32(count, types, bufs, rows, w[0]->cols, tokens, input,
                                     outputs);
}

// A projection of more than 8 tokens with the input's SwiGLU (up, or null) and
// the residual add (residual, or null; it may be `out`) folded into the GEMM.
[[nodiscard]] inline Status project_gemm_fused(const HipContext& ctx, const Tensor& w,
                                               const HipBuffer& input, std::size_t tokens,
                                               const HipBuffer* up, const HipBuffer* residual,
                                               HipBuffer& out) {
  if (w.buffer == nullptr || w.rows == 0 || w.cols == 0) {
    return Status::invalid_argument("Qwen3.5 matmul weight is missing");
  }
  const HipBuffer none;
  return ctx.kquant_matmul_fused_f32(static_cast<std::uint32_t>(w.type), *w.buffer, w.rows,
                                     w.cols, tokens, input, up != nullptr ? *up : none,
                                     residual != nullptr ? *residual : none, out);
}

// Device buffers one decode step reuses; sized for the plan on first use.
class DecodeScratch {
 public:
  HipBuffer hidden, normed, a, b, c, d, attn, ffn_gate, ffn_up;
  LayerWorkspace layer_ws;

  [[nodiscard]] Status prepare(const HipContext& ctx, const ExecutionPlan& plan,
                               const ModelWeights& w) {
    std::size_t widest = plan.hidden_size;
    for (const auto& l : w.layers) {
      for (const Tensor* t : {&l.ffn_gate, &l.ffn_up, &l.qkv, &l.gate, &l.q, &l.k, &l.v}) {
        widest = t->rows > widest ? t->rows : widest;
      }
    }
    widest = plan.linear_inner_size > widest ? plan.linear_inner_size : widest;
    widest = plan.attention_heads * plan.head_dim > widest ? plan.attention_heads * plan.head_dim
                                                           : widest;
    for (HipBuffer* buf : {&hidden, &normed, &a, &b, &c, &d, &attn, &ffn_gate, &ffn_up}) {
      if (!buf->valid() || buf->byte_size() < widest * sizeof(float)) {
        auto made = ctx.make_buffer(widest * sizeof(float));
        if (!made.is_ok()) {
          return made.status();
        }
        *buf = std::move(made.value());
      }
    }
    return Status::ok();
  }
};

namespace detail {

[[nodiscard]] inline Status embed_token(const HipContext& ctx, const Tensor& e,
                                        const HipBuffer& token_id, std::size_t hidden,
                                        HipBuffer& out) {
  if (e.buffer == nullptr || e.cols != hidden) {
    return Status::invalid_argument("Qwen3.5 token embedding shape mismatch");
  }
  switch (e.type) {
    case TensorType::q4_k:
      return ctx.dequantize_rows_q4_k_f32(*e.buffer, e.rows, token_id, 1, hidden, out);
    case TensorType::q5_k:
      return ctx.dequantize_rows_q5_k_f32(*e.buffer, e.rows, token_id, 1, hidden, out);
    case TensorType::q6_k:
      return ctx.dequantize_rows_q6_k_f32(*e.buffer, e.rows, token_id, 1, hidden, out);
    default:
      return Status::invalid_argument(
        "Qwen3.5 device token embedding needs a K-quant token_embd");
  }
}

[[nodiscard]] inline Status lm_head_argmax(const HipContext& ctx, const Tensor& w,
                                           const HipBuffer& normed, HipBuffer& token_out) {
  switch (w.type) {
    case TensorType::q4_k:
      return ctx.matvec_q4_k_f32_argmax(*w.buffer, w.rows, w.cols, normed, token_out);
    case TensorType::q5_k:
      return ctx.matvec_q5_k_f32_argmax(*w.buffer, w.rows, w.cols, normed, token_out);
    case TensorType::q6_k:
      return ctx.matvec_q6_k_f32_argmax(*w.buffer, w.rows, w.cols, normed, token_out);
    default:
      return Status::invalid_argument("Qwen3.5 greedy LM head needs a K-quant output weight");
  }
}

// One-token projection with the fused GEMV: RMSNorm(input) * norm first when
// `norm` is given, silu(input) * up when `up` is given, and the result added to
// `residual` when given (which may be `out`).
[[nodiscard]] inline Status project_fused(const HipContext& ctx, const Tensor& w,
                                          const HipBuffer& input, const HipBuffer* norm,
                                          float eps, const HipBuffer* up,
                                          const HipBuffer* residual, HipBuffer& out) {
  if (w.buffer == nullptr) {
    return Status::invalid_argument("Qwen3.5 matmul weight is missing");
  }
  const HipBuffer none;
  return ctx.kquant_matvec_fused_f32(static_cast<std::uint32_t>(w.type), *w.buffer, w.rows,
                                     w.cols, input, norm != nullptr ? *norm : none, eps,
                                     up != nullptr ? *up : none,
                                     residual != nullptr ? *residual : none, out);
}

// Up to four one-token projections of the same input, RMSNorm(input) * norm
// first, in one launch (separate fused GEMVs where the input is wider than one
// launch takes).
[[nodiscard]] inline Status project_multi(const HipContext& ctx, std::size_t count,
                                          const Tensor* const* w, HipBuffer* const* out,
                                          const HipBuffer& input, const HipBuffer& norm,
                                          float eps) {
  if (count == 0 || count > 4) {
    return Status::invalid_argument("Qwen3.5 joint projection takes 1 to 4 weights");
  }
  std::uint32_t types[4];
  std::size_t rows[4];
  const HipBuffer* weights[4];
  const HipBuffer* residuals[4] = {nullptr, nullptr, nullptr, nullptr};
  for (std::size_t i = 0; i < count; ++i) {
    if (w[i]->buffer == nullptr) {
      return Status::invalid_argument("Qwen3.5 matmul weight is missing");
    }
    if (w[i]->cols != w[0]->cols) {
      return Status::invalid_argument("Qwen3.5 joint projection weights differ in width");
    }
    types[i] = static_cast<std::uint32_t>(w[i]->type);
    rows[i] = w[i]->rows;
    weights[i] = w[i]->buffer;
  }
  if (w[0]->cols > 4096) {
    for (std::size_t i = 0; i < count; ++i) {
      Status st = project_fused(ctx, *w[i], input, &norm, eps, nullptr, nullptr, *out[i]);
      if (!st.is_ok()) {
        return st;
      }
    }
    return Status::ok();
  }
  const HipBuffer none;
  return ctx.kquant_matvec_multi_f32(count, types, weights, rows, w[0]->cols, input, norm, eps,
                                     none, residuals, out);
}

// KRAKEN_QWEN35_GDN_DECODE=one_kernel keeps the one-kernel linear-attention
// core in the fused decode step instead of the three-launch layer below.
[[nodiscard]] inline bool gdn_decode_split_enabled() {
  const char* value = std::getenv("KRAKEN_QWEN35_GDN_DECODE");
  return value == nullptr || std::string_view{value} != "one_kernel";
}

// A linear-attention layer of one decode token in three launches, for head_dim
// 128, conv kernel 4 and key_heads == value_heads (qwen35_runtime.cpp:
// 2720-3034): the joint input projection (RMSNorm folded in) whose qkv rows go
// through the conv and SiLU as they are written (each row owns its conv
// channel, so the conv-state update has one writer); the gated delta rule over
// up to 256 workgroups, which also forms the epilogue's norm_weight * silu(z);
// ssm_out with the rest of the norm-gated epilogue (the per-head RMS scale) on
// its input and the residual add on its output.  The one-kernel core keeps a head in one
// workgroup because of those two steps.  linear_layer_decode_split_applies
// says whether the shape, weights and cache allow it.
[[nodiscard]] inline bool linear_layer_decode_split_applies(const ExecutionPlan& plan,
                                                            const DeviceCache& cache,
                                                            const DecoderLayerWeights& l,
                                                            std::size_t linear_layer) {
  const LinearAttentionWeights& w = l.linear;
  return gdn_decode_split_enabled() && cache.recurrent_offsets.valid() &&
         plan.linear_key_head_dim == 128 && plan.linear_key_heads == plan.linear_value_heads &&
         plan.linear_conv_kernel == 4 && l.qkv.cols <= 4096 && l.ssm_out.cols <= 4096 &&
         w.conv1d != nullptr && w.dt_bias != nullptr && w.ssm_a != nullptr &&
         w.ssm_norm != nullptr && l.ssm_out.buffer != nullptr && l.attn_norm != nullptr &&
         linear_layer < plan.cache.linear_attention_layers;
}

[[nodiscard]] inline Status linear_layer_decode_split(const HipContext& ctx,
                                                      const ExecutionPlan& plan,
                                                      DeviceCache& cache,
                                                      const DecoderLayerWeights& l,
                                                      std::size_t linear_layer, float eps,
                                                      DecodeScratch& s) {
  const LinearAttentionWeights& w = l.linear;
  const std::size_t hk = plan.linear_key_heads;
  const std::size_t hv = plan.linear_value_heads;
  const std::size_t dk = plan.linear_key_head_dim;
  const Tensor* t[4] = {&l.qkv, &l.gate, &l.beta, &l.alpha};
  std::uint32_t types[4];
  std::size_t rows[4];
  const HipBuffer* weights[4];
  for (std::size_t i = 0; i < 4; ++i) {
    if (t[i]->buffer == nullptr || t[i]->cols != l.qkv.cols) {
      return Status::invalid_argument("Qwen3.5 linear attention projection weights are missing");
    }
    types[i] = static_cast<std::uint32_t>(t[i]->type);
    rows[i] = t[i]->rows;
    weights[i] = t[i]->buffer;
  }
  HipBuffer* out[4] = {&s.a, &s.b, &s.c, &s.d};
  // Recurrent row 0 of this layer: the offset table holds (conv, state)
  // element offsets per slot.
  const std::size_t slot = linear_layer * plan.cache.recurrent_rows;
  auto* table = static_cast<unsigned char*>(cache.recurrent_offsets.data());
  const HipBuffer conv_offset =
    HipBuffer::borrow(table + 2 * slot * sizeof(std::uint64_t), sizeof(std::uint64_t));
  const HipBuffer state_offset =
    HipBuffer::borrow(table + (2 * slot + 1) * sizeof(std::uint64_t), sizeof(std::uint64_t));
  Status st = ctx.kquant_matvec_multi_conv_f32(4, types, weights, rows, l.qkv.cols, s.hidden,
                                               *l.attn_norm, eps, out, cache.recurrent_r_cache,
                                               conv_offset, *w.conv1d, 4);
  // s.normed (free in the fused order) takes the epilogue's gate factor.
  if (st.is_ok()) {
    st = ctx.qwen35_gdn_state_ragged_decode_f32(s.a, s.d, s.c, *w.dt_bias, *w.ssm_a, s.b,
                                                *w.ssm_norm, cache.recurrent_s_cache,
                                                state_offset, 1, hk, hv, dk, eps, s.attn,
                                                s.normed);
  }
  if (st.is_ok()) {
    st = ctx.kquant_matvec_head_norm_f32(static_cast<std::uint32_t>(l.ssm_out.type),
                                         *l.ssm_out.buffer, l.ssm_out.rows, l.ssm_out.cols,
                                         s.attn, s.normed, dk, eps, s.hidden, s.hidden);
  }
  return st;
}

// The FFN half of a layer (qwen35_runtime.cpp:3024-3144): hidden += down(silu(gate(n)) *
// up(n)) with n = RMSNorm(hidden) * post_attention_norm.  OpOrder::reference issues
// the reference's six ops; OpOrder::fused three fused GEMVs.
[[nodiscard]] inline Status ffn_block(const HipContext& ctx, const ExecutionPlan& plan,
                                      const DecoderLayerWeights& l, float eps, OpOrder order,
                                      DecodeScratch& s) {
  const std::size_t h = plan.hidden_size;
  if (order == OpOrder::fused) {
    const Tensor* w[2] = {&l.ffn_up, &l.ffn_gate};
    HipBuffer* out[2] = {&s.ffn_up, &s.ffn_gate};
    Status st = project_multi(ctx, 2, w, out, s.hidden, *l.post_attention_norm, eps);
    if (st.is_ok()) {
      st = project_fused(ctx, l.ffn_down, s.ffn_gate, nullptr, eps, &s.ffn_up, &s.hidden,
                         s.hidden);
    }
    return st;
  }
  Status st = ctx.rms_norm_f32_f32_batched(s.hidden, *l.post_attention_norm, 1, h, eps, s.normed);
  if (st.is_ok()) st = project(ctx, l.ffn_up, s.normed, 1, s.ffn_up);
  if (st.is_ok()) st = project(ctx, l.ffn_gate, s.normed, 1, s.ffn_gate);
  if (st.is_ok()) st = ctx.silu_mul_f32_in_place(s.ffn_gate, s.ffn_up, l.ffn_gate.rows);
  if (st.is_ok()) st = project(ctx, l.ffn_down, s.ffn_gate, 1, s.a);
  if (st.is_ok()) st = ctx.add_f32_in_place(s.hidden, s.a, h);
  return st;
}

}  // namespace detail

// Enqueues one decode step for the token whose id (int32) is at
// token_in[0], at sequence position `position`: embedding, every main layer,
// output norm and the greedy LM head, whose argmax lands in token_out[0].
// Recurrent row 0 and the F16 KV cache of `cache` are read and advanced.
// OpOrder::reference issues the reference's op sequence (separate RMSNorm,
// projections, residual adds and SwiGLU); OpOrder::fused folds each RMSNorm into
// the projections that read it, SwiGLU and the residual add into the down and
// output projections, and the output norm into the LM head.
// `after_layer`, when given, is called with each main layer's index once its
// output is in s.hidden (for inspection; it may wait for the device).
using LayerHook = std::function<Status(std::size_t layer, const HipBuffer& hidden)>;

[[nodiscard]] inline Status enqueue_decode_step(const HipContext& ctx, const ExecutionPlan& plan,
                                                DeviceCache& cache, const ModelWeights& w,
                                                DecodeScratch& s, const HipBuffer& token_in,
                                                HipBuffer& token_out, std::size_t position,
                                                const LayerHook* after_layer = nullptr,
                                                OpOrder order = OpOrder::fused) {
  if (w.layers.size() != plan.main_layers || w.output_norm == nullptr) {
    return Status::invalid_argument("Qwen3.5 decode weights do not match the plan");
  }
  if (position >= plan.cache.attention_capacity_tokens) {
    return Status::invalid_argument("Qwen3.5 decode position exceeds cache capacity");
  }
  const std::size_t h = plan.hidden_size;
  const float eps = w.rms_eps;
  const bool fused = order == OpOrder::fused;
  Status st = detail::embed_token(ctx, w.token_embd, token_in, h, s.hidden);
  if (!st.is_ok()) {
    return st;
  }
  // The projections of the layer's normed input: fused, one launch normalises
  // s.hidden and runs them all; otherwise one RMSNorm into s.normed feeds one
  // projection each.
  auto proj_in = [&](const Tensor& t, HipBuffer& out) { return project(ctx, t, s.normed, 1, out); };
  // The output projection with the residual add.
  auto proj_out = [&](const Tensor& t, const HipBuffer& in) {
    if (fused) {
      return detail::project_fused(ctx, t, in, nullptr, eps, nullptr, &s.hidden, s.hidden);
    }
    Status r = project(ctx, t, in, 1, s.a);
    return r.is_ok() ? ctx.add_f32_in_place(s.hidden, s.a, h) : r;
  };
  st = for_each_main_layer(plan, [&](std::size_t index, LayerKind kind, std::size_t kind_index) {
    const DecoderLayerWeights& l = w.layers[index];
    if (l.attn_norm == nullptr || l.post_attention_norm == nullptr) {
      return Status::invalid_argument("Qwen3.5 decode layer is missing its norms");
    }
    Status r = fused ? Status::ok()
                     : ctx.rms_norm_f32_f32_batched(s.hidden, *l.attn_norm, 1, h, eps, s.normed);
    if (kind == LayerKind::linear_attention && fused &&
        detail::linear_layer_decode_split_applies(plan, cache, l, kind_index)) {
      if (r.is_ok()) r = detail::linear_layer_decode_split(ctx, plan, cache, l, kind_index, eps, s);
      if (r.is_ok()) r = detail::ffn_block(ctx, plan, l, eps, order, s);
      if (r.is_ok() && after_layer != nullptr) r = (*after_layer)(index, s.hidden);
      return r;
    }
    if (kind == LayerKind::linear_attention) {
      // qwen35_runtime.cpp:2720-3034: qkv, z, beta, alpha projections; the
      // attention core; ssm_out; residual.
      if (fused) {
        const Tensor* t[4] = {&l.qkv, &l.gate, &l.beta, &l.alpha};
        HipBuffer* out[4] = {&s.a, &s.b, &s.c, &s.d};
        if (r.is_ok()) r = detail::project_multi(ctx, 4, t, out, s.hidden, *l.attn_norm, eps);
      } else {
        if (r.is_ok()) r = proj_in(l.qkv, s.a);
        if (r.is_ok()) r = proj_in(l.gate, s.b);
        if (r.is_ok()) r = proj_in(l.beta, s.c);
        if (r.is_ok()) r = proj_in(l.alpha, s.d);
      }
      if (r.is_ok()) {
        r = run_linear_attention_chunk(ctx, plan, cache, l.linear, kind_index, 0, s.a, s.b, s.c,
                                       s.d, 1, eps, order, s.layer_ws, s.attn);
      }
      if (r.is_ok()) r = proj_out(l.ssm_out, s.attn);
    } else {
      // qwen35_runtime.cpp:3200-3400: joint Q/gate, K and V projections; the
      // attention core with the F16 KV append at `position`; attn_output;
      // residual.
      if (fused) {
        const Tensor* t[3] = {&l.q, &l.k, &l.v};
        HipBuffer* out[3] = {&s.a, &s.b, &s.c};
        if (r.is_ok()) r = detail::project_multi(ctx, 3, t, out, s.hidden, *l.attn_norm, eps);
      } else {
        if (r.is_ok()) r = proj_in(l.q, s.a);
        if (r.is_ok()) r = proj_in(l.k, s.b);
        if (r.is_ok()) r = proj_in(l.v, s.c);
      }
      if (r.is_ok()) {
        r = run_full_attention_chunk(ctx, plan, cache, l.full, kind_index, s.a, s.b, s.c, 1,
                                     position, position, w.mrope_sections, w.rope_theta, eps,
                                     nullptr, order, s.layer_ws, s.attn);
      }
      if (r.is_ok()) r = proj_out(l.output, s.attn);
    }
    if (r.is_ok()) r = detail::ffn_block(ctx, plan, l, eps, order, s);
    if (r.is_ok() && after_layer != nullptr) r = (*after_layer)(index, s.hidden);
    return r;
  });
  if (!st.is_ok()) {
    return st;
  }
  if (fused) {
    HipBuffer no_probability;
    return ctx.kquant_top1_fused_f32(static_cast<std::uint32_t>(w.output.type), *w.output.buffer,
                                     w.output.rows, w.output.cols, s.hidden, *w.output_norm, eps,
                                     token_out, no_probability);
  }
  st = ctx.rms_norm_f32_f32_batched(s.hidden, *w.output_norm, 1, h, eps, s.normed);
  if (!st.is_ok()) {
    return st;
  }
  return detail::lm_head_argmax(ctx, w.output, s.normed, token_out);
}

// Greedy generation of `steps` tokens after `first_token` at `start_position`
// (the decode loop of qwen35_runtime.cpp:6212-6263 with sampling off): step i
// feeds the token of step i - 1 (first_token for i = 0) at position
// start_position + i.  Each step is one graph batch committed once, so the host
// waits once per token; the device keeps the tokens and they are read back
// after the last step.  Returns the generated token ids.
[[nodiscard]] inline Result<std::vector<std::int32_t>> greedy_decode(
  const HipContext& ctx, const ExecutionPlan& plan, DeviceCache& cache, const ModelWeights& w,
  DecodeScratch& s, std::int32_t first_token, std::size_t start_position, std::size_t steps,
  const LayerHook* after_layer = nullptr, OpOrder order = OpOrder::fused) {
  if (steps == 0) {
    return std::vector<std::int32_t>{};
  }
  if (start_position + steps > plan.cache.attention_capacity_tokens) {
    return Status::invalid_argument("Qwen3.5 decode position exceeds cache capacity");
  }
  Status st = s.prepare(ctx, plan, w);
  if (!st.is_ok()) {
    return st;
  }
  auto tokens = ctx.make_buffer((steps + 1) * sizeof(std::int32_t));
  if (!tokens.is_ok()) {
    return tokens.status();
  }
  st = ctx.copy_to_buffer(tokens.value(), &first_token, sizeof(first_token));
  if (!st.is_ok()) {
    return st;
  }
  auto* base = static_cast<unsigned char*>(tokens.value().data());
  for (std::size_t i = 0; i < steps; ++i) {
    const HipBuffer in = HipBuffer::borrow(base + i * sizeof(std::int32_t), sizeof(std::int32_t));
    HipBuffer out =
      HipBuffer::borrow(base + (i + 1) * sizeof(std::int32_t), sizeof(std::int32_t));
    st = ctx.begin_graph();
    if (st.is_ok()) {
      st = enqueue_decode_step(ctx, plan, cache, w, s, in, out, start_position + i, after_layer,
                               order);
    }
    if (!st.is_ok()) {
      ctx.abort_graph();
      return st;
    }
    st = ctx.commit_graph();
    if (!st.is_ok()) {
      return st;
    }
  }
  std::vector<std::int32_t> all(steps + 1);
  st = ctx.copy_from_buffer(tokens.value(), all.data(), all.size() * sizeof(std::int32_t));
  if (!st.is_ok()) {
    return st;
  }
  return std::vector<std::int32_t>(all.begin() + 1, all.end());
}

}  // namespace kraken::qwen35
