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
// platform), this store keeps them in HBM: one arena of capacity_blocks + 1
// payload slots, allocated at the first commit, filled and drained with
// device-to-device region copies (kraken_hip_copy_regions), so neither commit
// nor restore crosses PCIe.  With the device cache in one allocation
// (allocate_device_cache), a commit is two launches (cache parts, hidden row)
// and a restore of n blocks ceil((12 n + 2) / 64) launches for Qwen3.5-0.8B,
// with one host wait each.  The spare slot takes a commit's payload before the
// index decides, so a failed copy never touches a stored block.  A payload is
// 32.8 MB for Qwen3.5-0.8B with 1024-token blocks.
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
      slot_of_.clear();
      free_slots_.clear();
      arena_ = HipBuffer{};
    }
  }

  [[nodiscard]] PrefixCacheLookup lookup(const std::vector<std::int64_t>& tokens) {
    return index_.lookup(tokens);
  }

  // qwen35_runtime.cpp:639-675: after the prefill chunk [token_start,
  // token_start + chunk_tokens) of `tokens`, store its payload if it is one
  // whole block not yet stored.  `chunk_hidden` holds the chunk's hidden rows,
  // [chunk_tokens][hidden_size] floats.  `cache` comes from allocate_device_cache.
  [[nodiscard]] Result<PrefixCommitResult> commit_block(
    const HipContext& ctx, const DeviceCache& cache, const ExecutionPlan& plan,
    const HipBuffer& chunk_hidden, const std::vector<std::int64_t>& tokens,
    std::size_t token_start, std::size_t chunk_tokens) {
    if (!layout_.has_value() || chunk_tokens != layout_->block_tokens ||
        token_start > tokens.size() || layout_->block_tokens > tokens.size() - token_start) {
      return PrefixCommitResult{};
    }
    const std::optional<std::uint64_t> hash = index_.hash_for_block(tokens, token_start);
    if (!hash.has_value() || slot_of_.count(*hash) != 0) {
      return PrefixCommitResult{};
    }
    auto off = offsets();
    if (!off.is_ok()) {
      return off.status();
    }
    const Status ready = ensure_arena(off.value());
    if (!ready.is_ok()) {
      return ready;
    }
    const std::size_t slot = free_slots_.back();
    const Status read = deferred(ctx, [&]() {
      return read_payload(ctx, cache, plan, chunk_hidden, off.value(), slot, token_start,
                          chunk_tokens);
    });
    if (!read.is_ok()) {
      return read;
    }
    const PrefixCacheCommit commit = index_.commit_block(tokens, token_start);
    PrefixCommitResult result;
    if (!commit.inserted) {
      return result;
    }
    free_slots_.pop_back();
    if (commit.evicted) {
      const auto it = slot_of_.find(commit.evicted_hash);
      if (it != slot_of_.end()) {
        free_slots_.push_back(it->second);
        slot_of_.erase(it);
      }
      result.evicted = true;
    }
    slot_of_[commit.hash] = slot;
    result.committed = true;
    return result;
  }

  // qwen35_runtime.cpp:677-706: the K/V rows of every hit block, then the
  // recurrent caches of the last one.
  [[nodiscard]] Status restore(const HipContext& ctx, DeviceCache& cache,
                               const ExecutionPlan& plan,
                               const std::vector<std::uint64_t>& block_hashes) const {
    if (!layout_.has_value() || block_hashes.empty()) {
      return Status::ok();
    }
    std::vector<std::size_t> slots;
    slots.reserve(block_hashes.size());
    for (const std::uint64_t h : block_hashes) {
      const auto it = slot_of_.find(h);
      if (it == slot_of_.end()) {
        return Status::invalid_argument("Qwen3.5 prefix cache payload is missing");
      }
      slots.push_back(it->second);
    }
    auto off = offsets();
    if (!off.is_ok()) {
      return off.status();
    }
    const Offsets& o = off.value();
    std::vector<kraken_copy_region> regions;
    for (std::size_t i = 0; i < slots.size(); ++i) {
      const Status s = add_kv_regions(cache, plan, o, slots[i], i * layout_->block_tokens,
                                      false, regions);
      if (!s.is_ok()) {
        return s;
      }
    }
    const std::size_t last = slots.back() * o.total;
    add_region(regions, last + o.r, part_offset(cache, cache.recurrent_r_cache), o.r_bytes);
    add_region(regions, last + o.s, part_offset(cache, cache.recurrent_s_cache), o.s_bytes);
    return deferred(ctx, [&]() { return copy_all(ctx, arena_, cache.storage, regions); });
  }

  // qwen35_runtime.cpp:708-715: the stored last hidden row of a block, as a
  // device view of hidden_size floats (copy it out with copy_buffer_region),
  // or an empty view (valid() false) when the block is not stored.
  [[nodiscard]] HipBuffer last_hidden(std::uint64_t hash) const {
    const auto it = slot_of_.find(hash);
    auto off = offsets();
    if (it == slot_of_.end() || !off.is_ok() || !arena_.valid()) {
      return HipBuffer{};
    }
    return HipBuffer::borrow(static_cast<unsigned char*>(arena_.data()) +
                               it->second * off.value().total + off.value().hidden,
                             off.value().hidden_bytes);
  }

  [[nodiscard]] PrefixCacheStats stats() const { return index_.stats(); }

 private:
  struct Offsets {
    std::size_t kv_block_layer;  // bytes of one layer's block rows
    std::size_t key, value, r, s, hidden, total;
    std::size_t r_bytes, s_bytes, hidden_bytes;
  };

  PrefixCacheIndex index_{PrefixCacheConfig{}};
  std::optional<PrefixCacheLayout> layout_;
  // The arena belongs to the store, not to the request context that first
  // commits: requests create and destroy their contexts (qwen35_runtime.cpp:
  // 5583-5589) while the store lives on, so the arena is allocated through a
  // context of the store's own, created at the first commit on the device that
  // is current then.  Declared before arena_, so it outlives the allocation.
  std::optional<HipContext> own_context_;
  HipBuffer arena_;                                      // (capacity + 1) payload slots
  std::unordered_map<std::uint64_t, std::size_t> slot_of_;  // stored block -> arena slot
  std::vector<std::size_t> free_slots_;

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

  static void add_region(std::vector<kraken_copy_region>& regions, std::size_t source,
                         std::size_t destination, std::size_t bytes) {
    if (bytes != 0) {
      regions.push_back(kraken_copy_region{source, destination, bytes});
    }
  }

  // Byte offset of one of the cache's parts within its one allocation.
  [[nodiscard]] static std::size_t part_offset(const DeviceCache& cache, const HipBuffer& part) {
    if (!part.valid()) {
      return 0;
    }
    return static_cast<std::size_t>(static_cast<const unsigned char*>(part.data()) -
                                    static_cast<const unsigned char*>(cache.storage.data()));
  }

  // Allocates the arena at the first commit: capacity + 1 slots, all free.
  [[nodiscard]] Status ensure_arena(const Offsets& o) {
    if (arena_.valid()) {
      return Status::ok();
    }
    std::size_t bytes = 0;
    const std::size_t slots = index_.config().capacity_blocks + 1;
    if (slots == 0 || !mul(slots, o.total, bytes)) {
      return Status::invalid_argument("Qwen3.5 prefix cache arena size overflow");
    }
    if (!own_context_.has_value()) {
      auto c = HipContext::create();
      if (!c.is_ok()) {
        return c.status();
      }
      own_context_.emplace(std::move(c.value()));
    }
    auto b = own_context_->make_buffer(bytes);
    if (!b.is_ok()) {
      return b.status();
    }
    arena_ = std::move(b.value());
    free_slots_.clear();
    for (std::size_t i = slots; i-- > 0;) {
      free_slots_.push_back(i);
    }
    return Status::ok();
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
  // full-attention layer `layer`, within the K (or V) cache.
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

  // The block's K and V rows of every full-attention layer, between arena slot
  // `slot` and the cache's allocation (to_arena: cache -> arena).
  [[nodiscard]] Status add_kv_regions(const DeviceCache& cache, const ExecutionPlan& plan,
                                      const Offsets& o, std::size_t slot,
                                      std::size_t token_start, bool to_arena,
                                      std::vector<kraken_copy_region>& regions) const {
    const std::size_t base = slot * o.total;
    const std::size_t k_part = part_offset(cache, cache.key_cache);
    const std::size_t v_part = part_offset(cache, cache.value_cache);
    // Each layer's rows must lie inside the K and V caches themselves, as the
    // reference's per-buffer copies check (mps_backend.mm:5768-5830): a block
    // past the capacity would otherwise run into the next part of the one
    // allocation.
    const std::size_t part_bytes =
      std::min(cache.key_cache.byte_size(), cache.value_cache.byte_size());
    for (std::size_t layer = 0; layer < layout_->full_attention_layers; ++layer) {
      auto row = cache_row_offset(plan, layer, token_start);
      if (!row.is_ok()) {
        return row.status();
      }
      if (row.value() > part_bytes || o.kv_block_layer > part_bytes - row.value()) {
        return Status::invalid_argument(to_arena ? "HIP copy size exceeds source buffer size"
                                                 : "HIP copy size exceeds destination buffer size");
      }
      const std::size_t at = layer * o.kv_block_layer;
      const std::size_t pk = base + o.key + at, ck = k_part + row.value();
      const std::size_t pv = base + o.value + at, cv = v_part + row.value();
      if (to_arena) {
        add_region(regions, ck, pk, o.kv_block_layer);
        add_region(regions, cv, pv, o.kv_block_layer);
      } else {
        add_region(regions, pk, ck, o.kv_block_layer);
        add_region(regions, pv, cv, o.kv_block_layer);
      }
    }
    return Status::ok();
  }

  // qwen35_runtime.cpp:776-859: K/V rows, R and S from the cache's allocation in
  // one launch, then the chunk's last hidden row.
  [[nodiscard]] Status read_payload(const HipContext& ctx, const DeviceCache& cache,
                                    const ExecutionPlan& plan, const HipBuffer& chunk_hidden,
                                    const Offsets& o, std::size_t slot, std::size_t token_start,
                                    std::size_t chunk_tokens) {
    std::size_t hidden_row = 0;
    std::size_t hidden_offset = 0;
    if (chunk_tokens == 0 || !mul(chunk_tokens - 1, layout_->hidden_size, hidden_row) ||
        !mul(hidden_row, sizeof(float), hidden_offset)) {
      return Status::invalid_argument("Qwen3.5 prefix last hidden offset overflow");
    }
    if (!cache.storage.valid() && (o.r_bytes != 0 || o.s_bytes != 0 ||
                                   layout_->full_attention_layers != 0)) {
      return Status::invalid_argument(
        "Qwen3.5 prefix cache needs a device cache from allocate_device_cache");
    }
    std::vector<kraken_copy_region> regions;
    const Status k = add_kv_regions(cache, plan, o, slot, token_start, true, regions);
    if (!k.is_ok()) {
      return k;
    }
    const std::size_t base = slot * o.total;
    add_region(regions, part_offset(cache, cache.recurrent_r_cache), base + o.r, o.r_bytes);
    add_region(regions, part_offset(cache, cache.recurrent_s_cache), base + o.s, o.s_bytes);
    HipBuffer& arena = arena_;
    Status s = copy_all(ctx, cache.storage, arena, regions);
    if (s.is_ok()) {
      s = copy_all(ctx, chunk_hidden, arena, {{hidden_offset, base + o.hidden, o.hidden_bytes}});
    }
    return s;
  }
};

}  // namespace kraken::qwen35
