// Cache and execution plan of the Qwen3.5 hot path, and the device caches it
// sizes.
//
// Mirrors Qwen35RuntimeOptions / Qwen35CachePlan / Qwen35PrefillPlan /
// Qwen35ExecutionPlan (include/toyllm/runtime/qwen35_runtime.hpp:16-67),
// build_qwen35_execution_plan and format_qwen35_execution_plan
// (src/runtime/qwen35_runtime.cpp:4379-4558) and Qwen35MetalCache with
// allocate_qwen35_metal_cache (qwen35_runtime.cpp:35-45, 1252-1330).  The plan
// reads the model's dimensions from ModelShape, which stands in for the
// ModelConfig fields (GGUF metadata) and the weight map's layer kinds; GGUF
// parsing and the weight map itself are not part of this library.
//
// Cache layout (the layer drivers in kraken/qwen35_layers.hpp index it so):
//   key_cache / value_cache  [full_attention_layers][capacity][kv_heads * head_dim]
//                            f16 (or f32 when kv_cache_f16 is false)
//   recurrent_r_cache        [linear_attention_layers][recurrent_rows][(K - 1) * C] f32
//   recurrent_s_cache        [linear_attention_layers][recurrent_rows][dk * inner] f32
// with C = inner + 2 * linear_key_heads * dk the conv channels and K the conv kernel.
#pragma once

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <limits>
#include <sstream>
#include <string>
#include <vector>

#include "kraken/hip_context.hpp"

namespace kraken::qwen35 {

using hip::HipBuffer;
using hip::HipContext;
using hip::Result;
using hip::Status;

// qwen35_weight_map.hpp:13-17
enum class LayerKind { full_attention, linear_attention, mtp };

// Model dimensions the plan reads (ModelConfig field names in comments).
struct ModelShape {
  std::int64_t hidden_size{0};             // hidden_size
  std::int64_t main_layer_count{0};        // main_layer_count = block_count - nextn layers
  std::int64_t total_layer_count{0};       // total_layer_count = block_count
  std::int64_t head_dim{0};                // head_dim (attention.key_length)
  std::int64_t num_attention_heads{0};     // num_attention_heads
  std::int64_t num_key_value_heads{0};     // num_key_value_heads
  std::int64_t linear_num_key_heads{0};    // linear_num_key_heads (ssm.group_count)
  std::int64_t linear_num_value_heads{0};  // linear_num_value_heads
  std::int64_t linear_key_head_dim{0};     // linear_key_head_dim (ssm.state_size)
  std::int64_t linear_inner_size{0};       // linear_inner_size (ssm.inner_size)
  std::int64_t linear_conv_kernel_dim{0};  // linear_conv_kernel_dim (ssm.conv_kernel)
  // One entry per layer, main layers first (the weight map's kinds).
  std::vector<LayerKind> layer_kinds;
};

// The reference's default schedule (model loader, full_attention_interval
// default 4): main layer i is full attention when (i + 1) % interval == 0,
// linear attention otherwise; layers past the main ones are MTP layers.
[[nodiscard]] inline std::vector<LayerKind> default_layer_kinds(std::size_t main_layers,
                                                                std::size_t total_layers,
                                                                std::size_t interval = 4) {
  std::vector<LayerKind> kinds;
  kinds.reserve(total_layers);
  for (std::size_t i = 0; i < total_layers; ++i) {
    if (i >= main_layers) {
      kinds.push_back(LayerKind::mtp);
    } else if (interval != 0 && (i + 1) % interval == 0) {
      kinds.push_back(LayerKind::full_attention);
    } else {
      kinds.push_back(LayerKind::linear_attention);
    }
  }
  return kinds;
}

// Qwen3.5-0.8B (the GGUF the reference benchmarks): 24 main layers, 18 linear
// attention + 6 full attention (layers 3, 7, ..., 23), no MTP layer.
[[nodiscard]] inline ModelShape qwen35_0_8b_shape() {
  ModelShape s;
  s.hidden_size = 1024;
  s.main_layer_count = 24;
  s.total_layer_count = 24;
  s.head_dim = 256;
  s.num_attention_heads = 8;
  s.num_key_value_heads = 2;
  s.linear_num_key_heads = 16;
  s.linear_num_value_heads = 16;
  s.linear_key_head_dim = 128;
  s.linear_inner_size = 2048;
  s.linear_conv_kernel_dim = 4;
  s.layer_kinds = default_layer_kinds(24, 24);
  return s;
}

// qwen35_runtime.hpp:16-24
struct RuntimeOptions {
  std::size_t context_tokens{0};
  std::size_t decode_tokens{1};
  std::size_t prefill_chunk_tokens{1024};
  std::size_t sequence_slots{1};
  std::size_t recurrent_snapshot_count{0};
  bool kv_cache_f16{true};
  bool output_all_prompt_logits{false};
};

// qwen35_runtime.hpp:26-41
struct CachePlan {
  std::size_t attention_capacity_tokens{0};
  std::size_t recurrent_slots{0};
  std::size_t recurrent_rows{0};
  std::size_t full_attention_layers{0};
  std::size_t linear_attention_layers{0};
  std::size_t kv_dim{0};
  std::size_t kv_cache_element_bytes{sizeof(std::uint16_t)};
  bool kv_cache_f16{true};
  std::size_t recurrent_r_elements_per_layer{0};
  std::size_t recurrent_s_elements_per_layer{0};
  std::uint64_t kv_cache_bytes{0};
  std::uint64_t recurrent_r_cache_bytes{0};
  std::uint64_t recurrent_s_cache_bytes{0};
  std::uint64_t total_cache_bytes{0};
};

// qwen35_runtime.hpp:43-49
struct PrefillPlan {
  std::size_t prompt_tokens{0};
  std::size_t chunk_tokens{0};
  std::size_t chunk_count{0};
  std::size_t final_chunk_tokens{0};
  bool output_only_last_token{true};
};

// qwen35_runtime.hpp:51-67
struct ExecutionPlan {
  std::size_t hidden_size{0};
  std::size_t main_layers{0};
  std::size_t total_layers{0};
  std::size_t head_dim{0};
  std::size_t attention_heads{0};
  std::size_t kv_heads{0};
  std::size_t linear_key_heads{0};
  std::size_t linear_value_heads{0};
  std::size_t linear_key_head_dim{0};
  std::size_t linear_value_head_dim{0};
  std::size_t linear_inner_size{0};
  std::size_t linear_conv_kernel{0};
  std::size_t linear_conv_channels{0};
  std::vector<LayerKind> layer_kinds;
  CachePlan cache;
  PrefillPlan prefill;
};

namespace detail {

// qwen35_runtime.cpp:442-451
[[nodiscard]] inline Result<std::size_t> positive_size(std::int64_t value, const char* name) {
  if (value <= 0) {
    return Status::invalid_argument(std::string{name} + " must be positive");
  }
  const auto u = static_cast<std::uint64_t>(value);
  if (u > static_cast<std::uint64_t>(std::numeric_limits<std::size_t>::max())) {
    return Status::invalid_argument(std::string{name} + " exceeds size_t range");
  }
  return static_cast<std::size_t>(u);
}

// a * b * c * d with the overflow message of qwen35_runtime.cpp:468-495.
[[nodiscard]] inline Result<std::uint64_t> cache_bytes(std::size_t a, std::size_t b,
                                                       std::size_t c, std::size_t d,
                                                       const char* name) {
  std::uint64_t bytes = a;
  for (const std::uint64_t f : {static_cast<std::uint64_t>(b), static_cast<std::uint64_t>(c),
                                static_cast<std::uint64_t>(d)}) {
    if (bytes != 0 && f > std::numeric_limits<std::uint64_t>::max() / bytes) {
      return Status::invalid_argument(std::string{name} + " byte count overflow");
    }
    bytes *= f;
  }
  return bytes;
}

[[nodiscard]] inline Result<std::uint64_t> add_bytes(std::uint64_t lhs, std::uint64_t rhs,
                                                     const char* name) {
  if (rhs > std::numeric_limits<std::uint64_t>::max() - lhs) {
    return Status::invalid_argument(std::string{name} + " byte count overflow");
  }
  return lhs + rhs;
}

[[nodiscard]] inline std::size_t ceil_div(std::size_t value, std::size_t divisor) {
  return value == 0 ? 0 : 1 + (value - 1) / divisor;
}

}  // namespace detail

// build_qwen35_execution_plan (qwen35_runtime.cpp:4379-4531): same checks in
// the same order, same messages, same cache arithmetic.
[[nodiscard]] inline Result<ExecutionPlan> build_execution_plan(const ModelShape& shape,
                                                                std::size_t prompt_tokens,
                                                                const RuntimeOptions& options) {
  if (prompt_tokens == 0) {
    return Status::invalid_argument("Qwen3.5 execution plan requires at least one prompt token");
  }
  if (options.prefill_chunk_tokens == 0) {
    return Status::invalid_argument("Qwen3.5 prefill chunk size must be positive");
  }
  if (options.sequence_slots == 0) {
    return Status::invalid_argument("Qwen3.5 sequence slot count must be positive");
  }
  struct Field {
    std::int64_t value;
    const char* name;
    std::size_t* out;
  };
  ExecutionPlan plan;
  std::size_t linear_inner = 0;
  const Field fields[] = {
    {shape.hidden_size, "hidden_size", &plan.hidden_size},
    {shape.main_layer_count, "main_layer_count", &plan.main_layers},
    {shape.total_layer_count, "total_layer_count", &plan.total_layers},
    {shape.head_dim, "head_dim", &plan.head_dim},
    {shape.num_attention_heads, "attention_heads", &plan.attention_heads},
    {shape.num_key_value_heads, "kv_heads", &plan.kv_heads},
    {shape.linear_num_key_heads, "linear_key_heads", &plan.linear_key_heads},
    {shape.linear_num_value_heads, "linear_value_heads", &plan.linear_value_heads},
    {shape.linear_key_head_dim, "linear_key_head_dim", &plan.linear_key_head_dim},
    {shape.linear_inner_size, "linear_inner_size", &linear_inner},
    {shape.linear_conv_kernel_dim, "linear_conv_kernel_dim", &plan.linear_conv_kernel},
  };
  for (const Field& f : fields) {
    auto v = detail::positive_size(f.value, f.name);
    if (!v.is_ok()) {
      return v.status();
    }
    *f.out = v.value();
  }
  if (linear_inner % plan.linear_value_heads != 0) {
    return Status::invalid_argument("linear_inner_size must be divisible by linear_value_heads");
  }
  if (shape.layer_kinds.size() < plan.main_layers) {
    return Status::invalid_argument("Qwen3.5 weight map has fewer layers than main layers");
  }

  plan.linear_inner_size = linear_inner;
  plan.linear_value_head_dim = linear_inner / plan.linear_value_heads;
  plan.linear_conv_channels = linear_inner + 2 * plan.linear_key_heads * plan.linear_key_head_dim;
  plan.layer_kinds.assign(shape.layer_kinds.begin(),
                          shape.layer_kinds.begin() + static_cast<std::ptrdiff_t>(plan.main_layers));

  plan.prefill.prompt_tokens = prompt_tokens;
  plan.prefill.chunk_tokens = options.prefill_chunk_tokens;
  plan.prefill.chunk_count = detail::ceil_div(prompt_tokens, options.prefill_chunk_tokens);
  plan.prefill.final_chunk_tokens =
    prompt_tokens - (plan.prefill.chunk_count - 1) * options.prefill_chunk_tokens;
  plan.prefill.output_only_last_token = !options.output_all_prompt_logits;

  CachePlan& c = plan.cache;
  c.attention_capacity_tokens = std::max(
    options.context_tokens, std::max<std::size_t>(1, prompt_tokens + options.decode_tokens));
  c.recurrent_slots = options.sequence_slots;
  c.recurrent_rows = options.sequence_slots * (1 + options.recurrent_snapshot_count);
  // The weight map counts the layers of each kind over all its layers.
  for (const LayerKind k : shape.layer_kinds) {
    c.full_attention_layers += k == LayerKind::full_attention ? 1 : 0;
    c.linear_attention_layers += k == LayerKind::linear_attention ? 1 : 0;
  }
  c.kv_dim = plan.kv_heads * plan.head_dim;
  c.kv_cache_f16 = options.kv_cache_f16;
  c.kv_cache_element_bytes = options.kv_cache_f16 ? sizeof(std::uint16_t) : sizeof(float);
  c.recurrent_r_elements_per_layer = (plan.linear_conv_kernel - 1) * plan.linear_conv_channels;
  c.recurrent_s_elements_per_layer = plan.linear_key_head_dim * plan.linear_inner_size;

  auto kv = detail::cache_bytes(c.full_attention_layers, c.attention_capacity_tokens,
                                c.kv_dim * 2, c.kv_cache_element_bytes, "Qwen3.5 KV cache");
  if (!kv.is_ok()) {
    return kv.status();
  }
  auto r = detail::cache_bytes(c.linear_attention_layers, c.recurrent_rows,
                               c.recurrent_r_elements_per_layer, sizeof(float),
                               "Qwen3.5 recurrent R cache");
  if (!r.is_ok()) {
    return r.status();
  }
  auto s = detail::cache_bytes(c.linear_attention_layers, c.recurrent_rows,
                               c.recurrent_s_elements_per_layer, sizeof(float),
                               "Qwen3.5 recurrent S cache");
  if (!s.is_ok()) {
    return s.status();
  }
  auto total = detail::add_bytes(kv.value(), r.value(), "Qwen3.5 total cache");
  if (!total.is_ok()) {
    return total.status();
  }
  total = detail::add_bytes(total.value(), s.value(), "Qwen3.5 total cache");
  if (!total.is_ok()) {
    return total.status();
  }
  c.kv_cache_bytes = kv.value();
  c.recurrent_r_cache_bytes = r.value();
  c.recurrent_s_cache_bytes = s.value();
  c.total_cache_bytes = total.value();
  return plan;
}

// format_qwen35_execution_plan (qwen35_runtime.cpp:4533-4558), same text.
[[nodiscard]] inline std::string format_execution_plan(const ExecutionPlan& plan) {
  std::ostringstream o;
  o << "Qwen3.5 execution plan: ok\n";
  o << "Layers: " << plan.main_layers << " main / " << plan.total_layers << " total\n";
  o << "- full_attention: " << plan.cache.full_attention_layers << '\n';
  o << "- linear_attention: " << plan.cache.linear_attention_layers << '\n';
  o << "Hidden: " << plan.hidden_size << '\n';
  o << "Full attention: heads=" << plan.attention_heads << ", kv_heads=" << plan.kv_heads
    << ", head_dim=" << plan.head_dim << ", kv_dim=" << plan.cache.kv_dim << '\n';
  o << "Linear attention: key_heads=" << plan.linear_key_heads
    << ", value_heads=" << plan.linear_value_heads
    << ", key_head_dim=" << plan.linear_key_head_dim
    << ", value_head_dim=" << plan.linear_value_head_dim
    << ", inner=" << plan.linear_inner_size
    << ", conv_channels=" << plan.linear_conv_channels << '\n';
  o << "Prefill: prompt_tokens=" << plan.prefill.prompt_tokens
    << ", chunk_tokens=" << plan.prefill.chunk_tokens << ", chunks=" << plan.prefill.chunk_count
    << ", final_chunk=" << plan.prefill.final_chunk_tokens
    << ", output_only_last=" << (plan.prefill.output_only_last_token ? "yes" : "no") << '\n';
  o << "Cache bytes: kv=" << plan.cache.kv_cache_bytes << " ("
    << (plan.cache.kv_cache_f16 ? "f16" : "f32") << ")"
    << ", recurrent_r=" << plan.cache.recurrent_r_cache_bytes
    << ", recurrent_s=" << plan.cache.recurrent_s_cache_bytes
    << ", total=" << plan.cache.total_cache_bytes << '\n';
  return o.str();
}

// Qwen35MetalCache (qwen35_runtime.cpp:35-45): the caller-owned caches the
// layer drivers read and write, one device allocation each.
struct DeviceCache {
  // One device allocation holding the four caches below, each 256-byte aligned;
  // key_cache .. recurrent_s_cache are views into it (a cache of zero bytes is
  // an empty view).  One allocation lets a single region-copy launch move rows
  // of several caches at once.
  HipBuffer storage;
  HipBuffer key_cache;
  HipBuffer value_cache;
  HipBuffer recurrent_r_cache;
  HipBuffer recurrent_s_cache;
  // Per recurrent slot (linear_layer * recurrent_rows + row) the pair of element
  // offsets {R offset, S offset}, uint64, so one-sequence decode can address its
  // slot through the ragged layer kernel without a per-token upload.
  HipBuffer recurrent_offsets;
  bool kv_cache_f16{true};
  std::uint64_t key_cache_bytes{0};
  std::uint64_t value_cache_bytes{0};
  std::uint64_t recurrent_r_cache_bytes{0};
  std::uint64_t recurrent_s_cache_bytes{0};
};

// allocate_qwen35_metal_cache (qwen35_runtime.cpp:1252-1330): K and V halves
// of kv_cache_bytes, R and S caches, all zeroed, as views into one allocation.
// A cache of zero bytes (no layer of that kind) is an empty view.
[[nodiscard]] inline Result<DeviceCache> allocate_device_cache(const HipContext& context,
                                                               const ExecutionPlan& plan) {
  if (plan.cache.kv_cache_bytes % 2 != 0) {
    return Status::invalid_argument("Qwen3.5 KV cache byte count must split evenly");
  }
  DeviceCache cache;
  cache.kv_cache_f16 = plan.cache.kv_cache_f16;
  cache.key_cache_bytes = plan.cache.kv_cache_bytes / 2;
  cache.value_cache_bytes = plan.cache.kv_cache_bytes / 2;
  cache.recurrent_r_cache_bytes = plan.cache.recurrent_r_cache_bytes;
  cache.recurrent_s_cache_bytes = plan.cache.recurrent_s_cache_bytes;
  struct Part {
    HipBuffer* buffer;
    std::uint64_t bytes;
    const char* name;
  };
  const Part parts[] = {
    {&cache.key_cache, cache.key_cache_bytes, "Qwen3.5 key cache"},
    {&cache.value_cache, cache.value_cache_bytes, "Qwen3.5 value cache"},
    {&cache.recurrent_r_cache, cache.recurrent_r_cache_bytes, "Qwen3.5 recurrent R cache"},
    {&cache.recurrent_s_cache, cache.recurrent_s_cache_bytes, "Qwen3.5 recurrent S cache"},
  };
  constexpr std::uint64_t kMax = std::numeric_limits<std::size_t>::max();
  std::uint64_t part_offsets[4] = {0, 0, 0, 0};
  std::uint64_t total = 0;
  for (int i = 0; i < 4; ++i) {
    if (parts[i].bytes > kMax) {
      return Status::invalid_argument(std::string{parts[i].name} + " exceeds size_t range");
    }
    part_offsets[i] = total;
    if (parts[i].bytes > kMax - 255 - total) {
      return Status::invalid_argument("Qwen3.5 total cache exceeds size_t range");
    }
    total = (total + parts[i].bytes + 255) / 256 * 256;
  }
  if (total > 0) {
    auto b = context.make_buffer(static_cast<std::size_t>(total));
    if (!b.is_ok()) {
      return b.status();
    }
    cache.storage = std::move(b.value());
    const Status z = context.zero_buffer(cache.storage, static_cast<std::size_t>(total));
    if (!z.is_ok()) {
      return z;
    }
    auto* base = static_cast<unsigned char*>(cache.storage.data());
    for (int i = 0; i < 4; ++i) {
      if (parts[i].bytes != 0) {
        *parts[i].buffer = HipBuffer::borrow(base + part_offsets[i],
                                             static_cast<std::size_t>(parts[i].bytes));
      }
    }
  }
  const std::size_t slots = plan.cache.linear_attention_layers * plan.cache.recurrent_rows;
  if (slots > 0) {
    std::vector<std::uint64_t> offsets(2 * slots);
    for (std::size_t i = 0; i < slots; ++i) {
      offsets[2 * i] = static_cast<std::uint64_t>(i) * plan.cache.recurrent_r_elements_per_layer;
      offsets[2 * i + 1] =
        static_cast<std::uint64_t>(i) * plan.cache.recurrent_s_elements_per_layer;
    }
    const std::size_t bytes = offsets.size() * sizeof(std::uint64_t);
    auto b = context.make_buffer(bytes);
    if (!b.is_ok()) {
      return b.status();
    }
    cache.recurrent_offsets = std::move(b.value());
    const Status c = context.copy_to_buffer(cache.recurrent_offsets, offsets.data(), bytes);
    if (!c.is_ok()) {
      return c;
    }
  }
  return cache;
}

}  // namespace kraken::qwen35
