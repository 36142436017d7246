// Whole-model chunked prefill on the device and the generation loop around it:
// the prompt pass of generate_qwen35_metal (src/runtime/qwen35_runtime.cpp:
// 5717-6045) with the reference's chunk walk (:5787-6004): the prompt's token
// embeddings (:5737-5746), then per chunk of plan.prefill.chunk_tokens tokens
// every main layer over the whole chunk (run_qwen35_linear_layer_chunk
// :2634-3144 and run_qwen35_full_attention_layer_chunk :3146-3423, each with
// its RMSNorm, K-quant GEMM projections, attention core, output projection,
// residual and SwiGLU FFN), one graph commit per chunk (the reference's
// chunk commit mode, :5976-5996), and after the last chunk the output norm and
// greedy LM head of its last row (:6005-6045).  Decode then starts at the
// prompt's length (:6047-6052, :6212-6263), from the filled caches.
//
// The chunk's projections are the K-quant GEMMs (more than 8 tokens) or the
// few-token GEMV (up to 8), as run_qwen35_quant_matmul picks them.  The layer
// cores take the whole chunk: flash256 attention over the F16 KV prefix and
// the chunk, and the chunked gated delta rule.
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <vector>

#include "kraken/qwen35_decode.hpp"

namespace kraken::qwen35 {

// Device buffers of one prefill chunk: [chunk_tokens][widest] f32 each, plus
// the prompt's token ids and the greedy token.  Sized on first use.
class PrefillScratch {
 public:
  HipBuffer hidden, normed, a, b, c, d, attn, ffn_gate, ffn_up, token_ids, token_out;
  LayerWorkspace layer_ws;

  [[nodiscard]] Status prepare(const HipContext& ctx, const ExecutionPlan& plan,
                               const ModelWeights& w, std::size_t chunk_tokens,
                               std::size_t prompt_tokens) {
    std::size_t widest = plan.hidden_size;
    for (const auto& l : w.layers) {
      for (const Tensor* t : {&l.ffn_gate, &l.ffn_up, &l.qkv, &l.gate, &l.q, &l.k, &l.v}) {
        widest = t->rows > widest ? t->rows : widest;
      }
    }
    widest = plan.linear_inner_size > widest ? plan.linear_inner_size : widest;
    widest = plan.attention_heads * plan.head_dim > widest ? plan.attention_heads * plan.head_dim
                                                           : widest;
    std::size_t bytes = 0;
    if (!detail::mul3(chunk_tokens, widest, sizeof(float), bytes)) {
      return Status::invalid_argument("Qwen3.5 prefill chunk size overflow");
    }
    for (HipBuffer* buf : {&hidden, &normed, &a, &b, &c, &d, &attn, &ffn_gate, &ffn_up}) {
      if (!buf->valid() || buf->byte_size() < bytes) {
        *buf = HipBuffer();
        auto made = ctx.make_buffer(bytes);
        if (!made.is_ok()) {
          return made.status();
        }
        *buf = std::move(made.value());
      }
    }
    const std::size_t id_bytes = (prompt_tokens > 0 ? prompt_tokens : 1) * sizeof(std::int32_t);
    if (!token_ids.valid() || token_ids.byte_size() < id_bytes) {
      token_ids = HipBuffer();
      auto made = ctx.make_buffer(id_bytes);
      if (!made.is_ok()) {
        return made.status();
      }
      token_ids = std::move(made.value());
    }
    if (!token_out.valid()) {
      auto made = ctx.make_buffer(sizeof(std::int32_t));
      if (!made.is_ok()) {
        return made.status();
      }
      token_out = std::move(made.value());
    }
    return Status::ok();
  }
};

// Called after each main layer of a chunk with the layer index, the chunk's
// hidden state [tokens][hidden] (valid once the device has run the layer: the
// hook may wait for it), the chunk's first position and its token count.
using ChunkLayerHook = std::function<Status(std::size_t layer, const HipBuffer& hidden,
                                            std::size_t chunk_start, std::size_t tokens)>;

namespace detail {

[[nodiscard]] inline Status embed_tokens(const HipContext& ctx, const Tensor& e,
                                         const HipBuffer& ids, std::size_t tokens,
                                         std::size_t hidden, HipBuffer& out) {
  if (e.buffer == nullptr || e.cols != hidden) {
    return Status::invalid_argument("Qwen3.5 token embedding shape mismatch");
  }
  switch (e.type) {
    case TensorType::q4_k:
      return ctx.dequantize_rows_q4_k_f32(*e.buffer, e.rows, ids, tokens, hidden, out);
    case TensorType::q5_k:
      return ctx.dequantize_rows_q5_k_f32(*e.buffer, e.rows, ids, tokens, hidden, out);
    case TensorType::q6_k:
      return ctx.dequantize_rows_q6_k_f32(*e.buffer, e.rows, ids, tokens, hidden, out);
    default:
      return Status::invalid_argument(
        "Qwen3.5 device token embedding needs a K-quant token_embd");
  }
}

}  // namespace detail

// Enqueues every main layer over one chunk whose input hidden state
// [tokens][hidden] is in s.hidden, at positions chunk_start .. chunk_start +
// tokens - 1; on return s.hidden holds the chunk's output of the last layer.
// Recurrent row 0 and the F16 KV cache of `cache` are read and advanced.  The
// layer cores follow `order` (OpOrder::reference: the reference's separate ops;
// OpOrder::fused: the fused conv/recurrence/epilogue and attention entries, and
// the z / beta / alpha and FFN up / gate projections as grouped matmuls); the
// norms, residual adds and SwiGLU are the reference's ops in both.
[[nodiscard]] inline Status enqueue_prefill_chunk(const HipContext& ctx,
                                                  const ExecutionPlan& plan, DeviceCache& cache,
                                                  const ModelWeights& w, PrefillScratch& s,
                                                  std::size_t chunk_start, std::size_t tokens,
                                                  const ChunkLayerHook* after_layer = nullptr,
                                                  OpOrder order = OpOrder::fused) {
  if (w.layers.size() != plan.main_layers) {
    return Status::invalid_argument("Qwen3.5 prefill weights do not match the plan");
  }
  if (tokens == 0) {
    return Status::invalid_argument("Qwen3.5 prefill chunk requires tokens");
  }
  if (chunk_start >= plan.cache.attention_capacity_tokens ||
      tokens > plan.cache.attention_capacity_tokens - chunk_start) {
    return Status::invalid_argument("Qwen3.5 chunk position exceeds cache capacity");
  }
  const std::size_t h = plan.hidden_size;
  const float eps = w.rms_eps;
  const std::size_t th = tokens * h;
  auto proj = [&](const Tensor& t, const HipBuffer& in, HipBuffer& out) {
    return project(ctx, t, in, tokens, out);
  };
  // The fused order folds the residual adds (and the FFN's SwiGLU) into the
  // GEMMs of the output projections, which take more than 8 tokens.
  const bool fold = order == OpOrder::fused && tokens > 8;
  auto proj_residual = [&](const Tensor& t, HipBuffer& in, const HipBuffer* up) {
    if (fold) {
      return project_gemm_fused(ctx, t, in, tokens, up, &s.hidden, s.hidden);
    }
    Status st = up != nullptr ? ctx.silu_mul_f32_in_place(in, *up, tokens * t.cols) : Status::ok();
    if (st.is_ok()) st = proj(t, in, s.a);
    if (st.is_ok()) st = ctx.add_f32_in_place(s.hidden, s.a, th);
    return st;
  };
  return for_each_main_layer(plan, [&](std::size_t index, LayerKind kind, std::size_t kind_index) {
    const DecoderLayerWeights& l = w.layers[index];
    if (l.attn_norm == nullptr || l.post_attention_norm == nullptr) {
      return Status::invalid_argument("Qwen3.5 prefill layer is missing its norms");
    }
    Status r = ctx.rms_norm_f32_f32_batched(s.hidden, *l.attn_norm, tokens, h, eps, s.normed);
    if (kind == LayerKind::linear_attention) {
      // qwen35_runtime.cpp:2720-2745 projections, the core, :3010-3034 ssm_out
      // and the residual.
      if (r.is_ok()) r = proj(l.qkv, s.normed, s.a);
      if (r.is_ok() && order == OpOrder::fused) {
        // z, beta and alpha share the normed input: one launch where their types allow.
        const Tensor* zba[3] = {&l.gate, &l.beta, &l.alpha};
        HipBuffer* outs[3] = {&s.b, &s.c, &s.d};
        r = project_group(ctx, 3, zba, s.normed, tokens, outs);
      } else {
        if (r.is_ok()) r = proj(l.gate, s.normed, s.b);
        if (r.is_ok()) r = proj(l.beta, s.normed, s.c);
        if (r.is_ok()) r = proj(l.alpha, s.normed, s.d);
      }
      if (r.is_ok()) {
        r = run_linear_attention_chunk(ctx, plan, cache, l.linear, kind_index, 0, s.a, s.b, s.c,
                                       s.d, tokens, eps, order, s.layer_ws, s.attn);
      }
      if (r.is_ok()) r = proj_residual(l.ssm_out, s.attn, nullptr);
    } else {
      // qwen35_runtime.cpp:3200-3228 projections, the core over the cached
      // prefix and the chunk, :3357-3400 attn_output and the residual.
      if (r.is_ok()) r = proj(l.q, s.normed, s.a);
      if (r.is_ok()) r = proj(l.k, s.normed, s.b);
      if (r.is_ok()) r = proj(l.v, s.normed, s.c);
      if (r.is_ok()) {
        r = run_full_attention_chunk(ctx, plan, cache, l.full, kind_index, s.a, s.b, s.c, tokens,
                                     chunk_start, chunk_start, w.mrope_sections, w.rope_theta, eps,
                                     nullptr, order, s.layer_ws, s.attn);
      }
      if (r.is_ok()) r = proj_residual(l.output, s.attn, nullptr);
    }
    // qwen35_runtime.cpp:3036-3144: the FFN half.
    if (r.is_ok()) {
      r = ctx.rms_norm_f32_f32_batched(s.hidden, *l.post_attention_norm, tokens, h, eps, s.normed);
    }
    if (r.is_ok() && order == OpOrder::fused) {
      const Tensor* ug[2] = {&l.ffn_up, &l.ffn_gate};
      HipBuffer* outs[2] = {&s.ffn_up, &s.ffn_gate};
      r = project_group(ctx, 2, ug, s.normed, tokens, outs);
    } else {
      if (r.is_ok()) r = proj(l.ffn_up, s.normed, s.ffn_up);
      if (r.is_ok()) r = proj(l.ffn_gate, s.normed, s.ffn_gate);
    }
    if (r.is_ok()) r = proj_residual(l.ffn_down, s.ffn_gate, &s.ffn_up);
    if (r.is_ok() && after_layer != nullptr) {
      r = (*after_layer)(index, s.hidden, chunk_start, tokens);
    }
    return r;
  });
}

// Prefills `prompt` (token ids) from position 0 in chunks of
// plan.prefill.chunk_tokens, one graph batch and one host wait per chunk, and
// returns the greedy token after the prompt: the argmax of the LM head over the
// output-normed last hidden row (fused into the top-1 GEMV with
// OpOrder::fused).  The caches then hold the prompt's K/V rows and the
// recurrent state after its last token, so decode continues at position
// prompt.size().
[[nodiscard]] inline Result<std::int32_t> prefill_prompt(
  const HipContext& ctx, const ExecutionPlan& plan, DeviceCache& cache, const ModelWeights& w,
  PrefillScratch& s, const std::vector<std::int32_t>& prompt,
  const ChunkLayerHook* after_layer = nullptr, OpOrder order = OpOrder::fused) {
  const std::size_t n = prompt.size();
  const std::size_t chunk = plan.prefill.chunk_tokens;
  if (n == 0) {
    return Status::invalid_argument("Qwen3.5 prefill requires prompt tokens");
  }
  if (chunk == 0) {
    return Status::invalid_argument("Qwen3.5 prefill chunk tokens must be positive");
  }
  if (n > plan.cache.attention_capacity_tokens) {
    return Status::invalid_argument("Qwen3.5 prompt exceeds cache capacity");
  }
  if (w.output_norm == nullptr || w.output.buffer == nullptr) {
    return Status::invalid_argument("Qwen3.5 prefill needs the output norm and LM head");
  }
  for (const std::int32_t t : prompt) {
    if (t < 0 || static_cast<std::size_t>(t) >= w.token_embd.rows) {
      return Status::invalid_argument("Qwen3.5 prompt token id is out of range");
    }
  }
  Status st = s.prepare(ctx, plan, w, chunk < n ? chunk : n, n);
  if (!st.is_ok()) {
    return st;
  }
  st = ctx.copy_to_buffer(s.token_ids, prompt.data(), n * sizeof(std::int32_t));
  if (!st.is_ok()) {
    return st;
  }
  const std::size_t h = plan.hidden_size;
  const float eps = w.rms_eps;
  auto* ids = static_cast<unsigned char*>(s.token_ids.data());
  for (std::size_t start = 0; start < n; start += chunk) {
    const std::size_t tokens = chunk < n - start ? chunk : n - start;
    const bool last = start + tokens == n;
    st = ctx.begin_graph();
    if (st.is_ok()) {
      const HipBuffer chunk_ids = HipBuffer::borrow(ids + start * sizeof(std::int32_t),
                                                    tokens * sizeof(std::int32_t));
      st = detail::embed_tokens(ctx, w.token_embd, chunk_ids, tokens, h, s.hidden);
    }
    if (st.is_ok()) {
      st = enqueue_prefill_chunk(ctx, plan, cache, w, s, start, tokens, after_layer, order);
    }
    if (st.is_ok() && last) {
      // The last row's output norm and greedy LM head (qwen35_runtime.cpp:
      // 6005-6045, run_qwen35_output_logits with argmax).
      auto* hidden = static_cast<unsigned char*>(s.hidden.data());
      const HipBuffer row =
        HipBuffer::borrow(hidden + (tokens - 1) * h * sizeof(float), h * sizeof(float));
      if (order == OpOrder::fused) {
        HipBuffer no_probability;
        st = ctx.kquant_top1_fused_f32(static_cast<std::uint32_t>(w.output.type),
                                       *w.output.buffer, w.output.rows, w.output.cols, row,
                                       *w.output_norm, eps, s.token_out, no_probability);
      } else {
        st = ctx.rms_norm_f32_f32_batched(row, *w.output_norm, 1, h, eps, s.normed);
        if (st.is_ok()) st = detail::lm_head_argmax(ctx, w.output, s.normed, s.token_out);
      }
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
  std::int32_t token = 0;
  st = ctx.copy_from_buffer(s.token_out, &token, sizeof(token));
  if (!st.is_ok()) {
    return st;
  }
  return token;
}

// Greedy generation of `steps` tokens for `prompt`: the prompt's chunked
// prefill picks the first token, then the device decode loop the rest at
// positions prompt.size() onwards (qwen35_runtime.cpp:6047-6263 with sampling
// off).  Returns the generated token ids.
[[nodiscard]] inline Result<std::vector<std::int32_t>> generate_greedy(
  const HipContext& ctx, const ExecutionPlan& plan, DeviceCache& cache, const ModelWeights& w,
  PrefillScratch& ps, DecodeScratch& ds, const std::vector<std::int32_t>& prompt,
  std::size_t steps, OpOrder order = OpOrder::fused) {
  if (steps == 0) {
    return std::vector<std::int32_t>{};
  }
  if (prompt.size() + steps > plan.cache.attention_capacity_tokens + 1) {
    return Status::invalid_argument("Qwen3.5 generation exceeds cache capacity");
  }
  auto first = prefill_prompt(ctx, plan, cache, w, ps, prompt, nullptr, order);
  if (!first.is_ok()) {
    return first.status();
  }
  std::vector<std::int32_t> out{first.value()};
  if (steps == 1) {
    return out;
  }
  auto rest = greedy_decode(ctx, plan, cache, w, ds, first.value(), prompt.size(), steps - 1,
                            nullptr, order);
  if (!rest.is_ok()) {
    return rest.status();
  }
  out.insert(out.end(), rest.value().begin(), rest.value().end());
  return out;
}

}  // namespace kraken::qwen35
