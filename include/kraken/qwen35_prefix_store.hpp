// Prompt prefix cache payload store: for each block the index holds, the cache
// state after that block's prefill chunk, so a later prompt with the same
// prefix restores it instead of recomputing it.
//
// Mirrors Qwen35HostPrefixCache (qwen35_runtime.cpp:516-929): the layout key
// (:516-555), configure / lookup / commit_block / restore / last_hidden /
// stats (:614-719), and the payload contents (:761-881):
//   K and V: per full-attention layer the block's rows of the cache,
//            [layer][block_tokens][kv_dim] elements of kv_element_bytes;
//   R and S: the whole recurrent caches as they stand after the block;
//   last hidden: the block chunk's last hidden row, hidden_size floats.
// Restoring writes each block's K/V rows back to the same cache rows and the R
// and S caches of the last block (:885-921).
//
// Where the reference keeps payloads in host memory (unified memory on its
// platform), this store keeps them in HBM: one device allocation per block,
// filled and drained with device-to-device copies, so neither commit nor
// restore crosses PCIe.  The rows of all layers move in one launch
// (kraken_hip_copy_regions) rather than one copy per layer and cache.  A block evicted by
// the index hands its allocation to the next commit.  Its size is fixed by the
// layout, e.g. about 19 MiB a block for Qwen3.5-0.8B with 1024-token blocks.
#pragma once

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <limits>
#include <optional>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "kraken/hip_context.hpp"
#include "kraken/qwen35_plan.hpp"
#include "kraken/qwen35_prefix_cache.hpp"

namespace kraken::qwen35 {

// qwen35_runtime.cpp:516-555: the cache is dropped whenever any field changes.
struct PrefixCacheLayout {
  std::string model_dir;
  std::string model_file;
  std::uint64_t gguf_version{0};
  std::uint64_t gguf_tensor_count{0};
  std::uint64_t gguf_metadata_count{0};
  std::uint64_t gguf_file_size{0};
  std::uint64_t tokenizer_fingerprint{0};
  std::size_t block_tokens{0};
  std::size_t full_attention_layers{0};
  std::size_t linear_attention_layers{0};
  std::size_t kv_dim{0};
  std::size_t kv_element_bytes{0};
  std::size_t hidden_size{0};
  std::uint64_t recurrent_r_cache_bytes{0};
  std::uint64_t recurrent_s_cache_bytes{0};
  bool kv_cache_f16{true};

  [[nodiscard]] bool operator==(const PrefixCacheLayout& o) const {
    return model_dir == o.model_dir && model_file == o.model_file &&
           gguf_version == o.gguf_version && gguf_tensor_count == o.gguf_tensor_count &&
           gguf_metadata_count == o.gguf_metadata_count && gguf_file_size == o.gguf_file_size &&
           tokenizer_fingerprint == o.tokenizer_fingerprint && block_tokens == o.block_tokens &&
           full_attention_layers == o.full_attention_layers &&
           linear_attention_layers == o.linear_attention_layers && kv_dim == o.kv_dim &&
           kv_element_bytes == o.kv_element_bytes && hidden_size == o.hidden_size &&
           recurrent_r_cache_bytes == o.recurrent_r_cache_bytes &&
           recurrent_s_cache_bytes == o.recurrent_s_cache_bytes &&
           kv_cache_f16 == o.kv_cache_f16;
  }
};

// The layout fields a plan fixes (qwen35_runtime.cpp:5555-5564); the model and
// tokenizer identity fields are the caller's.
[[nodiscard]] inline PrefixCacheLayout prefix_layout_from_plan(const ExecutionPlan& plan,
                                                               std::size_t block_tokens) {
  PrefixCacheLayout l;
  l.block_tokens = block_tokens;
  l.full_attention_layers = plan.cache.full_attention_layers;
  l.linear_attention_layers = plan.cache.linear_attention_layers;
  l.kv_dim = plan.cache.kv_dim;
  l.kv_element_bytes = plan.cache.kv_cache_element_bytes;
  l.hidden_size = plan.hidden_size;
  l.recurrent_r_cache_bytes = plan.cache.recurrent_r_cache_bytes;
  l.recurrent_s_cache_bytes = plan.cache.recurrent_s_cache_bytes;
  l.kv_cache_f16 = plan.cache.kv_cache_f16;
  return l;
}

// qwen35_runtime.cpp:607-610
struct PrefixCommitResult {
  bool committed{false};
  bool evicted{false};
};

class PrefixCacheStore {
 public:
  // qwen35_runtime.cpp:614-625: a new layout or configuration empties the store.
  void configure(const PrefixCacheLayout& layout, PrefixCacheConfig config) {
    const PrefixCacheConfig& c = index_.config();
    if (!layout_.has_value() || !(*layout_ == layout) || config.block_tokens != c.block_tokens ||
        config.capacity_blocks != c.capacity_blocks ||
        config.min_reuse_tokens != c.min_reuse_tokens || config.enabled != c.enabled) {
      layout_ = layout;
      index_ = PrefixCacheIndex(config);
      payloads_.clear();
      spare_ = Payload{};
    }
  }

  [[nodiscard]] PrefixCacheLookup lookup(const std::vector<std::int64_t>& tokens) {
    return index_.lookup(tokens);
  }

  // qwen35_runtime.cpp:639-675: after the prefill chunk [token_start,
  // token_start + chunk_tokens) of `tokens`, store its payload if it is one
  // whole block not yet stored.  `chunk_hidden` holds the chunk's hidden rows,
  // [chunk_tokens][hidden_size] floats.
  [[nodiscard]] Result<PrefixCommitResult> commit_block(
    const HipContext& ctx, const DeviceCache& cache, const ExecutionPlan& plan,
    const HipBuffer& chunk_hidden, const std::vector<std::int64_t>& tokens,
    std::size_t token_start, std::size_t chunk_tokens) {
    if (!layout_.has_value() || chunk_tokens != layout_->block_tokens ||
        token_start > tokens.size() || layout_->block_tokens > tokens.size() - token_start) {
      return PrefixCommitResult{};
    }
    const std::optional<std::uint64_t> hash = index_.hash_for_block(tokens, token_start);
    if (!hash.has_value() || payloads_.count(*hash) != 0) {
      return PrefixCommitResult{};
    }
    Result<Payload> payload = Status::ok();
    const Status read = deferred(ctx, [&]() {
      payload = read_payload(ctx, cache, plan, chunk_hidden, token_start, chunk_tokens);
      return payload.status();
    });
    if (!read.is_ok()) {
      return read;
    }
    if (!payload.is_ok()) {
      return payload.status();
    }
    const PrefixCacheCommit commit = index_.commit_block(tokens, token_start);
    PrefixCommitResult result;
    if (!commit.inserted) {
      spare_ = std::move(payload.value());
      return result;
    }
    if (commit.evicted) {
      const auto it = payloads_.find(commit.evicted_hash);
      if (it != payloads_.end()) {
        spare_ = std::move(it->second);
        payloads_.erase(it);
      }
      result.evicted = true;
    }
    payloads_[commit.hash] = std::move(payload.value());
    result.committed = true;
    return result;
  }

  // qwen35_runtime.cpp:677-706: the K/V rows of every hit block, then the
  // recurrent caches of the last one.
  [[nodiscard]] Status restore(const HipContext& ctx, DeviceCache& cache,
                               const ExecutionPlan& plan,
                               const std::vector<std::uint64_t>& block_hashes) const {
    if (!layout_.has_value()) {
      return Status::ok();
    }
    return deferred(ctx, [&]() { return restore_blocks(ctx, cache, plan, block_hashes); });
  }

  // qwen35_runtime.cpp:708-715: the stored last hidden row of a block, as a
  // device view of hidden_size floats (copy it out with copy_buffer_region),
  // or nullptr when the block is not stored.
  [[nodiscard]] const HipBuffer* last_hidden(std::uint64_t hash) const {
    const auto it = payloads_.find(hash);
    return it == payloads_.end() ? nullptr : &it->second.last_hidden;
  }

  [[nodiscard]] PrefixCacheStats stats() const { return index_.stats(); }

 private:
  // Runs `body` with the context's per-launch host wait off, so the copies are
  // waited for once at the end; inside a caller's open graph the caller's
  // commit waits for them instead.
  template <class Body>
  [[nodiscard]] static Status deferred(const HipContext& ctx, Body&& body) {
    if (!ctx.begin_graph().is_ok()) {
      return body();
    }
    const Status s = body();
    if (!s.is_ok()) {
      ctx.abort_graph();
      return s;
    }
    return ctx.commit_graph();
  }

  [[nodiscard]] Status restore_blocks(const HipContext& ctx, DeviceCache& cache,
                                      const ExecutionPlan& plan,
                                      const std::vector<std::uint64_t>& block_hashes) const {
    for (std::size_t i = 0; i < block_hashes.size(); ++i) {
      const auto it = payloads_.find(block_hashes[i]);
      if (it == payloads_.end()) {
        return Status::invalid_argument("Qwen3.5 prefix cache payload is missing");
      }
      const Status s = restore_kv_block(ctx, cache, plan, it->second, i * layout_->block_tokens);
      if (!s.is_ok()) {
        return s;
      }
    }
    if (!block_hashes.empty()) {
      const auto it = payloads_.find(block_hashes.back());
      if (it == payloads_.end()) {
        return Status::invalid_argument("Qwen3.5 prefix cache payload is missing");
      }
      return restore_recurrent(ctx, cache, it->second);
    }
    return Status::ok();
  }

  struct Payload {
    HipBuffer storage;      // K | V | R | S | last hidden, one allocation
    HipBuffer last_hidden;  // view into storage
  };
  struct Offsets {
    std::size_t kv_block_layer;  // bytes of one layer's block rows
    std::size_t key, value, r, s, hidden, total;
    std::size_t r_bytes, s_bytes, hidden_bytes;
  };

  PrefixCacheIndex index_{PrefixCacheConfig{}};
  std::optional<PrefixCacheLayout> layout_;
  std::unordered_map<std::uint64_t, Payload> payloads_;
  Payload spare_;

  [[nodiscard]] static bool mul(std::size_t a, std::size_t b, std::size_t& out) {
    if (a != 0 && b > std::numeric_limits<std::size_t>::max() / a) {
      return false;
    }
    out = a * b;
    return true;
  }
  [[nodiscard]] static bool add(std::size_t a, std::size_t b, std::size_t& out) {
    if (b > std::numeric_limits<std::size_t>::max() - a) {
      return false;
    }
    out = a + b;
    return true;
  }

  // Issues `regions` in launches of at most KRAKEN_COPY_REGIONS_MAX ranges.
  [[nodiscard]] static Status copy_all(const HipContext& ctx, const HipBuffer& source,
                                       HipBuffer& destination,
                                       const std::vector<kraken_copy_region>& regions) {
    for (std::size_t i = 0; i < regions.size(); i += KRAKEN_COPY_REGIONS_MAX) {
      const std::size_t n = std::min<std::size_t>(KRAKEN_COPY_REGIONS_MAX, regions.size() - i);
      const Status s = ctx.copy_regions(source, destination, regions.data() + i, n);
      if (!s.is_ok()) {
        return s;
      }
    }
    return Status::ok();
  }

  // The block's rows of every full-attention layer: {cache offset, payload offset}.
  [[nodiscard]] Result<std::vector<kraken_copy_region>> kv_regions(const ExecutionPlan& plan,
                                                                   const Offsets& o,
                                                                   std::size_t token_start,
                                                                   bool to_payload) const {
    std::vector<kraken_copy_region> regions;
    regions.reserve(layout_->full_attention_layers);
    for (std::size_t layer = 0; layer < layout_->full_attention_layers; ++layer) {
      auto row = cache_row_offset(plan, layer, token_start);
      if (!row.is_ok()) {
        return row.status();
      }
      const std::size_t at = layer * o.kv_block_layer;
      regions.push_back(to_payload ? kraken_copy_region{row.value(), at, o.kv_block_layer}
                                   : kraken_copy_region{at, row.value(), o.kv_block_layer});
    }
    return regions;
  }

  // Payload sizes and sections (qwen35_runtime.cpp:725-750, 766-777, 811-857),
  // each section 256-byte aligned.
  [[nodiscard]] Result<Offsets> offsets() const {
    if (!layout_.has_value()) {
      return Status::invalid_argument("Qwen3.5 prefix cache layout is not configured");
    }
    const PrefixCacheLayout& l = *layout_;
    Offsets o{};
    std::size_t elements = 0;
    if (!mul(l.block_tokens, l.kv_dim, elements)) {
      return Status::invalid_argument("Qwen3.5 prefix cache KV block size overflow");
    }
    if (!mul(elements, l.kv_element_bytes, o.kv_block_layer)) {
      return Status::invalid_argument("Qwen3.5 prefix cache KV block bytes overflow");
    }
    std::size_t kv_bytes = 0;
    if (!mul(l.full_attention_layers, o.kv_block_layer, kv_bytes)) {
      return Status::invalid_argument("Qwen3.5 prefix cache KV payload overflow");
    }
    constexpr std::uint64_t kMax = std::numeric_limits<std::size_t>::max();
    if (l.recurrent_r_cache_bytes > kMax) {
      return Status::invalid_argument("Qwen3.5 recurrent R cache exceeds size_t range");
    }
    if (l.recurrent_s_cache_bytes > kMax) {
      return Status::invalid_argument("Qwen3.5 recurrent S cache exceeds size_t range");
    }
    o.r_bytes = static_cast<std::size_t>(l.recurrent_r_cache_bytes);
    o.s_bytes = static_cast<std::size_t>(l.recurrent_s_cache_bytes);
    if (!mul(l.hidden_size, sizeof(float), o.hidden_bytes)) {
      return Status::invalid_argument("Qwen3.5 prefix last hidden bytes overflow");
    }
    const std::size_t sizes[5] = {kv_bytes, kv_bytes, o.r_bytes, o.s_bytes, o.hidden_bytes};
    std::size_t* starts[5] = {&o.key, &o.value, &o.r, &o.s, &o.hidden};
    std::size_t at = 0;
    for (int i = 0; i < 5; ++i) {
      *starts[i] = at;
      if (!add(at, sizes[i], at) || !add(at, 255, at)) {
        return Status::invalid_argument("Qwen3.5 prefix cache payload overflow");
      }
      at &= ~static_cast<std::size_t>(255);
    }
    o.total = at;
    return o;
  }

  // qwen35_runtime.cpp:752-774: byte offset of cache row `token_start` of
  // full-attention layer `layer`.
  [[nodiscard]] static Result<std::size_t> cache_row_offset(const ExecutionPlan& plan,
                                                            std::size_t layer,
                                                            std::size_t token_start) {
    std::size_t row = 0;
    if (!mul(layer, plan.cache.attention_capacity_tokens, row)) {
      return Status::invalid_argument("Qwen3.5 active KV layer offset overflow");
    }
    if (!add(row, token_start, row)) {
      return Status::invalid_argument("Qwen3.5 active KV token offset overflow");
    }
    std::size_t elements = 0;
    if (!mul(row, plan.cache.kv_dim, elements)) {
      return Status::invalid_argument("Qwen3.5 active KV element offset overflow");
    }
    std::size_t bytes = 0;
    if (!mul(elements, plan.cache.kv_cache_element_bytes, bytes)) {
      return Status::invalid_argument("Qwen3.5 active KV byte offset overflow");
    }
    return bytes;
  }

  // qwen35_runtime.cpp:776-859
  [[nodiscard]] Result<Payload> read_payload(const HipContext& ctx, const DeviceCache& cache,
                                             const ExecutionPlan& plan,
                                             const HipBuffer& chunk_hidden,
                                             std::size_t token_start,
                                             std::size_t chunk_tokens) {
    auto off = offsets();
    if (!off.is_ok()) {
      return off.status();
    }
    const Offsets& o = off.value();
    std::size_t hidden_row = 0;
    std::size_t hidden_offset = 0;
    if (chunk_tokens == 0 || !mul(chunk_tokens - 1, layout_->hidden_size, hidden_row) ||
        !mul(hidden_row, sizeof(float), hidden_offset)) {
      return Status::invalid_argument("Qwen3.5 prefix last hidden offset overflow");
    }
    Payload p = std::move(spare_);
    spare_ = Payload{};
    if (!p.storage.valid() || p.storage.byte_size() != o.total) {
      auto b = ctx.make_buffer(o.total);
      if (!b.is_ok()) {
        return b.status();
      }
      p.storage = std::move(b.value());
    }
    // K and V rows: the K section is the payload's start and the V section
    // follows it, so the same ranges shifted by o.value serve V.
    auto kv = kv_regions(plan, o, token_start, true);
    if (!kv.is_ok()) {
      return kv.status();
    }
    std::vector<kraken_copy_region> v_regions = kv.value();
    for (kraken_copy_region& g : v_regions) {
      g.destination_offset += o.value;
    }
    Status s = copy_all(ctx, cache.key_cache, p.storage, kv.value());
    if (s.is_ok()) {
      s = copy_all(ctx, cache.value_cache, p.storage, v_regions);
    }
    if (s.is_ok() && o.r_bytes != 0) {
      s = copy_all(ctx, cache.recurrent_r_cache, p.storage, {{0, o.r, o.r_bytes}});
    }
    if (s.is_ok() && o.s_bytes != 0) {
      s = copy_all(ctx, cache.recurrent_s_cache, p.storage, {{0, o.s, o.s_bytes}});
    }
    if (s.is_ok()) {
      s = copy_all(ctx, chunk_hidden, p.storage, {{hidden_offset, o.hidden, o.hidden_bytes}});
    }
    if (!s.is_ok()) {
      return s;
    }
    p.last_hidden = HipBuffer::borrow(static_cast<unsigned char*>(p.storage.data()) + o.hidden,
                                      o.hidden_bytes);
    return p;
  }

  // qwen35_runtime.cpp:861-893
  [[nodiscard]] Status restore_kv_block(const HipContext& ctx, DeviceCache& cache,
                                        const ExecutionPlan& plan, const Payload& p,
                                        std::size_t token_start) const {
    auto off = offsets();
    if (!off.is_ok()) {
      return off.status();
    }
    const Offsets& o = off.value();
    auto kv = kv_regions(plan, o, token_start, false);
    if (!kv.is_ok()) {
      return kv.status();
    }
    std::vector<kraken_copy_region> v_regions = kv.value();
    for (kraken_copy_region& g : v_regions) {
      g.source_offset += o.value;
    }
    const Status s = copy_all(ctx, p.storage, cache.key_cache, kv.value());
    return s.is_ok() ? copy_all(ctx, p.storage, cache.value_cache, v_regions) : s;
  }

  // qwen35_runtime.cpp:895-921
  [[nodiscard]] Status restore_recurrent(const HipContext& ctx, DeviceCache& cache,
                                         const Payload& p) const {
    auto off = offsets();
    if (!off.is_ok()) {
      return off.status();
    }
    const Offsets& o = off.value();
    if (o.r_bytes != 0) {
      const Status s = copy_all(ctx, p.storage, cache.recurrent_r_cache, {{o.r, 0, o.r_bytes}});
      if (!s.is_ok()) {
        return s;
      }
    }
    if (o.s_bytes != 0) {
      return copy_all(ctx, p.storage, cache.recurrent_s_cache, {{o.s, 0, o.s_bytes}});
    }
    return Status::ok();
  }
};

}  // namespace kraken::qwen35
