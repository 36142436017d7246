// Layer drivers of the Qwen3.5 hot path: the op sequence of
// run_qwen35_linear_layer_chunk (src/runtime/qwen35_runtime.cpp:2634-3144) and
// run_qwen35_full_attention_layer_chunk (qwen35_runtime.cpp:3146-3423) between
// the projections, and the layer loop of run_qwen35_decode_tokens
// (qwen35_runtime.cpp:3860-3936).
//
// The projections (K-quant GEMV/GEMM), the RMSNorm of the hidden state, the
// residual adds and the FFN are not part of this library: a driver takes the
// projection outputs of one chunk (device f32 buffers) and produces the
// attention output that the reference feeds to ssm_out / attn_output.
//
// Every op goes through HipContext (kraken/hip_context.hpp), so the drivers
// enqueue on the context's stream and return the first failing op's Status.
#pragma once

#include <array>
#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <functional>
#include <limits>
#include <string>
#include <string_view>
#include <vector>

#include "kraken/qwen35_plan.hpp"

namespace kraken::qwen35 {

// Per-layer weights the hot path reads (f32 device buffers).
struct LinearAttentionWeights {
  const HipBuffer* conv1d{nullptr};    // [conv_channels][conv_kernel] (GGUF shape {K, C})
  const HipBuffer* dt_bias{nullptr};   // [value_heads]
  const HipBuffer* ssm_a{nullptr};     // [value_heads]
  const HipBuffer* ssm_norm{nullptr};  // [key_head_dim]
};

struct FullAttentionWeights {
  const HipBuffer* q_norm{nullptr};  // [head_dim]
  const HipBuffer* k_norm{nullptr};  // [head_dim]
};

// How a driver issues the ops.
enum class OpOrder {
  // The reference's ops one at a time, in its order and with its
  // intermediate buffers.
  reference,
  // The same arithmetic through the fused entry points: conv state + conv +
  // SiLU + split + L2 in one kernel; gate/beta prepare and the norm-gated
  // epilogue with the recurrence; the sigmoid output gate inside attention.
  fused,
};

// The reference's KRAKEN_QWEN35_FUSED_NORM_GATED switch
// (qwen35_runtime.cpp:1014-1023): the norm-gated epilogue as one op instead
// of RMSNorm, SiLU and multiply.
[[nodiscard]] inline bool fused_norm_gated_enabled() {
  const char* value = std::getenv("KRAKEN_QWEN35_FUSED_NORM_GATED");
  if (value == nullptr) {
    return false;
  }
  const std::string_view s{value};
  return s == "1" || s == "true" || s == "TRUE" || s == "on" || s == "ON" || s == "yes" ||
         s == "YES";
}

// Scratch buffers a driver reuses across calls; each slot grows to the
// largest size asked of it.  One workspace per stream of calls.
class LayerWorkspace {
 public:
  [[nodiscard]] Result<HipBuffer*> get(const HipContext& ctx, std::size_t slot,
                                       std::size_t bytes) {
    if (slot >= buffers_.size()) {
      return Status::internal_error("layer workspace slot out of range");
    }
    HipBuffer& b = buffers_[slot];
    if (!b.valid() || b.byte_size() < bytes) {
      b = HipBuffer();
      auto fresh = ctx.make_buffer(bytes);
      if (!fresh.is_ok()) {
        return fresh.status();
      }
      b = std::move(fresh.value());
    }
    return &b;
  }

 private:
  std::array<HipBuffer, 8> buffers_;
};

namespace detail {

// True when a * b * c fits size_t; the product in `out`.
[[nodiscard]] inline bool mul3(std::size_t a, std::size_t b, std::size_t c, std::size_t& out) {
  const std::size_t m = std::numeric_limits<std::size_t>::max();
  if ((a != 0 && b > m / a) || (a * b != 0 && c > m / (a * b))) {
    return false;
  }
  out = a * b * c;
  return true;
}

}  // namespace detail

// Positions of make_qwen35_mrope_positions (qwen35_runtime.cpp:1848-1877) for
// text: int32 [4][tokens], every row start_position + t.
[[nodiscard]] inline Result<std::vector<std::int32_t>> make_mrope_positions(
  std::size_t start_position, std::size_t tokens) {
  if (tokens == 0) {
    return Status::invalid_argument("Qwen3.5 batched MRoPE positions require tokens");
  }
  const auto max32 = static_cast<std::size_t>(std::numeric_limits<std::int32_t>::max());
  if (start_position > max32 || tokens - 1 > max32 - start_position) {
    return Status::invalid_argument("Qwen3.5 batched MRoPE position exceeds int32 range");
  }
  std::vector<std::int32_t> positions(4 * tokens);
  for (std::size_t section = 0; section < 4; ++section) {
    for (std::size_t t = 0; t < tokens; ++t) {
      positions[section * tokens + t] = static_cast<std::int32_t>(start_position + t);
    }
  }
  return positions;
}

// run_qwen35_linear_layer_chunk (qwen35_runtime.cpp:2634-3144), from the
// outputs of the qkv, z (gate), beta and alpha projections to the attention
// output that feeds ssm_out:
//   qkv_mixed [tokens][conv_channels]; z [tokens][inner]; beta, alpha
//   [tokens][value_heads] (raw projections); output [tokens][inner].
// With OpOrder::reference, beta becomes sigma(beta), alpha the decay gate g and
// (unless the fused norm-gated switch is on) z becomes silu(z), as in the
// reference; OpOrder::fused leaves z, beta and alpha unchanged.
// The conv state R and recurrent state S read and updated are those of linear
// layer `linear_layer` (its index among the linear-attention layers) and
// recurrent row `row`: element offsets (linear_layer * recurrent_rows + row) *
// elements_per_layer, which for one row is the reference's
// recurrent_layer_index * elements_per_layer.
[[nodiscard]] inline Status run_linear_attention_chunk(
  const HipContext& ctx, const ExecutionPlan& plan, DeviceCache& cache,
  const LinearAttentionWeights& w, std::size_t linear_layer, std::size_t row,
  const HipBuffer& qkv_mixed, HipBuffer& z, HipBuffer& beta, HipBuffer& alpha,
  std::size_t tokens, float rms_eps, OpOrder order, LayerWorkspace& ws, HipBuffer& output) {
  if (w.conv1d == nullptr || w.dt_bias == nullptr || w.ssm_a == nullptr ||
      w.ssm_norm == nullptr) {
    return Status::invalid_argument("Qwen3.5 linear attention layer is missing weights");
  }
  const std::size_t kc = plan.linear_conv_kernel;
  const std::size_t channels = plan.linear_conv_channels;
  const std::size_t hk = plan.linear_key_heads;
  const std::size_t dk = plan.linear_key_head_dim;
  const std::size_t hv = plan.linear_value_heads;
  const std::size_t inner = plan.linear_inner_size;
  if (tokens == 0 || hk == 0 || dk == 0 || hv == 0 || inner == 0) {
    return Status::invalid_argument("Qwen3.5 linear attention chunk dimensions must be positive");
  }
  const std::size_t key_dim = hk * dk;
  if (inner != hv * dk || channels != 2 * key_dim + inner) {
    return Status::invalid_argument("Qwen3.5 linear attention chunk dimensions are inconsistent");
  }
  if (linear_layer >= plan.cache.linear_attention_layers || row >= plan.cache.recurrent_rows) {
    return Status::invalid_argument("Qwen3.5 recurrent layer or row out of range");
  }
  const std::size_t slot = linear_layer * plan.cache.recurrent_rows + row;
  std::size_t r_offset = 0;
  std::size_t s_offset = 0;
  if (!detail::mul3(slot, plan.cache.recurrent_r_elements_per_layer, 1, r_offset) ||
      !detail::mul3(slot, plan.cache.recurrent_s_elements_per_layer, 1, s_offset)) {
    return Status::invalid_argument("Qwen3.5 recurrent cache offset overflow");
  }

  std::size_t key_bytes = 0;
  std::size_t value_bytes = 0;
  if (!detail::mul3(tokens, key_dim, sizeof(float), key_bytes) ||
      !detail::mul3(tokens, inner, sizeof(float), value_bytes)) {
    return Status::invalid_argument("Qwen3.5 linear attention chunk size overflow");
  }
  auto q = ws.get(ctx, 0, key_bytes);
  auto k = ws.get(ctx, 1, key_bytes);
  auto v = ws.get(ctx, 2, value_bytes);
  for (const Status& s : {q.status(), k.status(), v.status()}) {
    if (!s.is_ok()) {
      return s;
    }
  }
  HipBuffer& qb = *q.value();
  HipBuffer& kb = *k.value();
  HipBuffer& vb = *v.value();

  Status s;
  if (order == OpOrder::fused && tokens == 1 && cache.recurrent_offsets.valid()) {
    // One decode token: conv prologue, gated delta rule and norm-gated epilogue
    // in one launch, the slot's offsets read from the cache's offset table.
    auto* table = static_cast<unsigned char*>(cache.recurrent_offsets.data());
    const HipBuffer conv_offset =
      HipBuffer::borrow(table + 2 * slot * sizeof(std::uint64_t), sizeof(std::uint64_t));
    const HipBuffer state_offset =
      HipBuffer::borrow(table + (2 * slot + 1) * sizeof(std::uint64_t), sizeof(std::uint64_t));
    return ctx.qwen35_gdn_layer_ragged_decode_f32(
      qkv_mixed, cache.recurrent_r_cache, conv_offset, *w.conv1d, kc, alpha, beta, *w.dt_bias,
      *w.ssm_a, z, *w.ssm_norm, cache.recurrent_s_cache, state_offset, 1, hk, hv, dk, rms_eps,
      output);
  }
  if (order == OpOrder::fused) {
    s = ctx.qwen35_conv_split_l2_f32(qkv_mixed, cache.recurrent_r_cache, r_offset, *w.conv1d, kc,
                                     tokens, hk, hv, dk, rms_eps, qb, kb, vb);
    if (!s.is_ok()) {
      return s;
    }
    return ctx.qwen35_gdn_gated_f32(qb, kb, vb, alpha, beta, *w.dt_bias, *w.ssm_a, z,
                                    *w.ssm_norm, cache.recurrent_s_cache, s_offset, tokens, hk,
                                    hv, dk, rms_eps, output);
  }

  std::size_t conv_in_bytes = 0;
  std::size_t conv_out_bytes = 0;
  if (!detail::mul3(channels, tokens + kc - 1, sizeof(float), conv_in_bytes) ||
      !detail::mul3(tokens, channels, sizeof(float), conv_out_bytes)) {
    return Status::invalid_argument("Qwen3.5 linear attention chunk size overflow");
  }
  auto conv_input = ws.get(ctx, 3, conv_in_bytes);
  if (!conv_input.is_ok()) {
    return conv_input.status();
  }
  auto conv_output = ws.get(ctx, 4, conv_out_bytes);
  if (!conv_output.is_ok()) {
    return conv_output.status();
  }
  HipBuffer& ci = *conv_input.value();
  HipBuffer& co = *conv_output.value();
  // qwen35_runtime.cpp:2746-2796: conv state, depthwise conv, SiLU, split + L2.
  s = ctx.build_ssm_conv_state_f32(cache.recurrent_r_cache, r_offset, qkv_mixed, kc, channels,
                                   tokens, ci);
  if (s.is_ok()) {
    s = ctx.ssm_conv_f32(ci, *w.conv1d, kc, channels, tokens, 1, co);
  }
  if (s.is_ok()) {
    s = ctx.silu_f32_in_place(co, tokens * channels);
  }
  if (s.is_ok()) {
    s = ctx.split_qkv_l2_norm_f32_qwen35(co, qb, kb, vb, tokens, hk, hv, dk, rms_eps);
  }
  // :2913-2919 gate/beta prepare; :2966-2971 the recurrence.
  if (s.is_ok()) {
    s = ctx.prepare_qwen35_gdn_gate_beta_f32(alpha, beta, *w.dt_bias, *w.ssm_a, tokens, hv);
  }
  if (s.is_ok()) {
    s = ctx.gated_delta_net_f32_batched_in_place_at(qb, kb, vb, alpha, beta,
                                                    cache.recurrent_s_cache, s_offset, tokens,
                                                    hk, hv, dk, output);
  }
  if (!s.is_ok()) {
    return s;
  }
  // :2985-3008 norm-gated epilogue.
  if (fused_norm_gated_enabled()) {
    return ctx.qwen35_norm_gated_f32_in_place(output, *w.ssm_norm, z, tokens, hv, dk, rms_eps);
  }
  s = ctx.qk_norm_f32_f32_batched(output, *w.ssm_norm, tokens, hv, dk, rms_eps);
  if (s.is_ok()) {
    s = ctx.silu_f32_in_place(z, tokens * inner);
  }
  if (s.is_ok()) {
    s = ctx.mul_f32_in_place(output, z, tokens * inner);
  }
  return s;
}

// run_qwen35_full_attention_layer_chunk (qwen35_runtime.cpp:3146-3423), from
// the joint Q/gate projection and the K and V projections to the gated
// attention output that feeds attn_output:
//   q_gate [tokens][heads][2 * head_dim] (per head the query, then its gate:
//   the GGUF's interleaved layout); key, value [tokens][kv_heads * head_dim]
//   (with OpOrder::reference key is normalised and rotated in place, as in the
//   reference; OpOrder::fused with an F16 cache leaves it unchanged); output
//   [tokens][heads * head_dim].
// OpOrder::fused with an F16 cache issues two launches: the fused prologue
// (split, q/k RMSNorm, MRoPE, K/V append) and attention with the output gate.
// K and V are appended to full-attention layer `attention_layer` of the cache
// at positions start_position .. start_position + tokens - 1, and attention
// runs causally over positions 0 .. start_position + t.  `positions` (int32
// [4][tokens]) may be null: text positions from mrope_start_position are made.
[[nodiscard]] inline Status run_full_attention_chunk(
  const HipContext& ctx, const ExecutionPlan& plan, DeviceCache& cache,
  const FullAttentionWeights& w, std::size_t attention_layer, const HipBuffer& q_gate,
  HipBuffer& key, const HipBuffer& value, std::size_t tokens, std::size_t start_position,
  std::size_t mrope_start_position, const std::array<std::size_t, 4>& mrope_sections,
  float rope_theta, float rms_eps, const HipBuffer* positions, OpOrder order,
  LayerWorkspace& ws, HipBuffer& output) {
  if (w.q_norm == nullptr || w.k_norm == nullptr) {
    return Status::invalid_argument("Qwen3.5 full attention layer is missing weights");
  }
  const std::size_t heads = plan.attention_heads;
  const std::size_t kv_heads = plan.kv_heads;
  const std::size_t head_dim = plan.head_dim;
  const std::size_t capacity = plan.cache.attention_capacity_tokens;
  if (tokens == 0 || heads == 0 || kv_heads == 0 || head_dim == 0 || capacity == 0) {
    return Status::invalid_argument("Qwen3.5 full attention chunk dimensions must be positive");
  }
  const std::size_t pairs =
    mrope_sections[0] + mrope_sections[1] + mrope_sections[2] + mrope_sections[3];
  const std::size_t mrope_dims = 2 * pairs;
  if (mrope_dims == 0 || mrope_dims > head_dim) {
    return Status::invalid_argument("Qwen3.5 MRoPE sections do not fit head_dim");
  }
  if (attention_layer >= plan.cache.full_attention_layers) {
    return Status::invalid_argument("Qwen3.5 full attention layer out of range");
  }
  if (start_position >= capacity || tokens > capacity - start_position) {
    return Status::invalid_argument("Qwen3.5 chunk position exceeds cache capacity");
  }
  const std::size_t attn_dim = heads * head_dim;
  const std::size_t kv_dim = kv_heads * head_dim;
  std::size_t attn_bytes = 0;
  std::size_t cache_offset = 0;
  if (!detail::mul3(tokens, attn_dim, sizeof(float), attn_bytes) ||
      !detail::mul3(attention_layer * capacity + start_position, kv_dim, 1, cache_offset)) {
    return Status::invalid_argument("Qwen3.5 full attention chunk size overflow");
  }
  auto query = ws.get(ctx, 5, attn_bytes);
  auto gate = ws.get(ctx, 6, attn_bytes);
  for (const Status& s : {query.status(), gate.status()}) {
    if (!s.is_ok()) {
      return s;
    }
  }
  HipBuffer& qb = *query.value();
  HipBuffer& gb = *gate.value();

  if (order == OpOrder::fused && cache.kv_cache_f16) {
    const HipBuffer none;
    return ctx.qwen35_attention_prologue_gated_f16_kv(
      q_gate, key, value, *w.q_norm, *w.k_norm, positions != nullptr ? *positions : none,
      mrope_start_position, cache.key_cache, cache.value_cache, attention_layer, start_position,
      tokens, capacity, heads, kv_heads, head_dim, mrope_dims, mrope_sections[0],
      mrope_sections[1], mrope_sections[2], mrope_sections[3], rope_theta, rms_eps, qb, gb,
      output);
  }

  // :3229-3268 split of the joint projection, q and k RMSNorm.
  Status s = ctx.copy_f32_rows(q_gate, qb, tokens * heads, head_dim, 2 * head_dim, 0, head_dim, 0);
  if (s.is_ok()) {
    s = ctx.copy_f32_rows(q_gate, gb, tokens * heads, head_dim, 2 * head_dim, head_dim, head_dim,
                          0);
  }
  if (s.is_ok()) {
    s = ctx.qk_norm_f32_f32_batched(qb, *w.q_norm, tokens, heads, head_dim, rms_eps);
  }
  if (s.is_ok()) {
    s = ctx.qk_norm_f32_f32_batched(key, *w.k_norm, tokens, kv_heads, head_dim, rms_eps);
  }
  if (!s.is_ok()) {
    return s;
  }

  // :3270-3301 MRoPE on q and k.
  const HipBuffer* pos = positions;
  if (pos == nullptr) {
    auto made = make_mrope_positions(mrope_start_position, tokens);
    if (!made.is_ok()) {
      return made.status();
    }
    const std::size_t bytes = made.value().size() * sizeof(std::int32_t);
    auto pb = ws.get(ctx, 7, bytes);
    if (!pb.is_ok()) {
      return pb.status();
    }
    s = ctx.copy_to_buffer(*pb.value(), made.value().data(), bytes);
    if (!s.is_ok()) {
      return s;
    }
    pos = pb.value();
  } else if (pos->byte_size() < tokens * 4 * sizeof(std::int32_t)) {
    return Status::invalid_argument("Qwen3.5 chunk MRoPE position buffer is too small");
  }
  s = ctx.mrope_f32_in_place(qb, *pos, tokens, heads, head_dim, mrope_dims, mrope_sections[0],
                             mrope_sections[1], mrope_sections[2], mrope_sections[3],
                             rope_theta);
  if (s.is_ok()) {
    s = ctx.mrope_f32_in_place(key, *pos, tokens, kv_heads, head_dim, mrope_dims,
                               mrope_sections[0], mrope_sections[1], mrope_sections[2],
                               mrope_sections[3], rope_theta);
  }
  // :3303-3326 KV append.
  if (s.is_ok()) {
    s = cache.kv_cache_f16 ? ctx.copy_f32_rows_to_f16(key, cache.key_cache, tokens, kv_dim, kv_dim,
                                                      0, kv_dim, cache_offset)
                           : ctx.copy_f32_rows(key, cache.key_cache, tokens, kv_dim, kv_dim, 0,
                                               kv_dim, cache_offset);
  }
  if (s.is_ok()) {
    s = cache.kv_cache_f16 ? ctx.copy_f32_rows_to_f16(value, cache.value_cache, tokens, kv_dim,
                                                      kv_dim, 0, kv_dim, cache_offset)
                           : ctx.copy_f32_rows(value, cache.value_cache, tokens, kv_dim, kv_dim,
                                               0, kv_dim, cache_offset);
  }
  if (!s.is_ok()) {
    return s;
  }
  // :3328-3355 attention, then the sigmoid output gate.
  s = cache.kv_cache_f16
        ? ctx.attention_f32_batched_f16_kv(qb, cache.key_cache, cache.value_cache, attention_layer,
                                           start_position, tokens, capacity, heads, kv_heads,
                                           head_dim, output)
        : ctx.attention_f32_batched(qb, cache.key_cache, cache.value_cache, attention_layer,
                                    start_position, tokens, capacity, heads, kv_heads, head_dim,
                                    output);
  if (s.is_ok()) {
    s = ctx.sigmoid_f32_in_place(gb, tokens * attn_dim);
  }
  if (s.is_ok()) {
    s = ctx.mul_f32_in_place(output, gb, tokens * attn_dim);
  }
  return s;
}

// The layer loop of run_qwen35_decode_tokens (qwen35_runtime.cpp:3885-3933):
// walks the plan's main layers in order and calls `layer` with the layer's
// index, its kind and its index among the layers of that kind (the KV-cache
// layer for full attention, the R/S-cache layer for linear attention).  Stops
// at the first failing layer; an MTP layer in the main pass and a count that
// disagrees with the plan's cache are errors, as in the reference.
[[nodiscard]] inline Status for_each_main_layer(
  const ExecutionPlan& plan,
  const std::function<Status(std::size_t layer_index, LayerKind kind, std::size_t kind_index)>&
    layer) {
  std::size_t linear = 0;
  std::size_t full = 0;
  std::size_t main = 0;
  for (std::size_t i = 0; i < plan.main_layers; ++i) {
    const LayerKind kind = plan.layer_kinds[i];
    Status s;
    switch (kind) {
      case LayerKind::linear_attention:
        s = layer(i, kind, linear);
        ++linear;
        break;
      case LayerKind::full_attention:
        s = layer(i, kind, full);
        ++full;
        break;
      case LayerKind::mtp:
        return Status::invalid_argument("Qwen3.5 decode layer loop reached MTP layer");
    }
    if (!s.is_ok()) {
      return s;
    }
    ++main;
  }
  if (main != plan.main_layers || linear != plan.cache.linear_attention_layers ||
      full != plan.cache.full_attention_layers) {
    return Status::internal_error("Qwen3.5 decode layer execution count mismatch");
  }
  return Status::ok();
}

}  // namespace kraken::qwen35
