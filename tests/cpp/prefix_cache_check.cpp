// Drives the prompt prefix cache (include/kraken/qwen35_prefix_cache.hpp and
// qwen35_prefix_store.hpp) for the test suite.
//
//   prefix_cache_check index        reads an operation script on stdin and
//                                   prints one result line per operation (the
//                                   CPU oracle prints the same lines);
//   prefix_cache_check store        commit / restore / evict round trip over a
//                                   real device cache (needs a GPU).
#include <chrono>
#include <cinttypes>
#include <cstdio>
#include <cstring>
#include <iostream>
#include <sstream>
#include <string>
#include <vector>

#include "kraken/hip_context.hpp"
#include "kraken/qwen35_plan.hpp"
#include "kraken/qwen35_prefix_cache.hpp"
#include "kraken/qwen35_prefix_store.hpp"

using kraken::hip::HipBuffer;
using kraken::hip::HipContext;
using kraken::hip::Status;
namespace q35 = kraken::qwen35;

namespace {

std::vector<std::int64_t> read_tokens(std::istringstream& in) {
  std::size_t n = 0;
  in >> n;
  std::vector<std::int64_t> t(n);
  for (auto& v : t) {
    in >> v;
  }
  return t;
}

int run_index() {
  q35::PrefixCacheIndex index{q35::PrefixCacheConfig{}};
  std::string line;
  while (std::getline(std::cin, line)) {
    std::istringstream in(line);
    std::string op;
    in >> op;
    if (op == "new") {
      int enabled = 0;
      q35::PrefixCacheConfig c;
      in >> enabled >> c.block_tokens >> c.capacity_blocks >> c.min_reuse_tokens;
      c.enabled = enabled != 0;
      index = q35::PrefixCacheIndex(c);
      std::printf("new\n");
    } else if (op == "lookup") {
      const auto r = index.lookup(read_tokens(in));
      std::printf("lookup %zu", r.hit_tokens);
      for (const auto h : r.block_hashes) {
        std::printf(" %" PRIu64, h);
      }
      std::printf("\n");
    } else if (op == "commit") {
      std::size_t start = 0;
      in >> start;
      const auto r = index.commit_block(read_tokens(in), start);
      std::printf("commit %d %d %" PRIu64 " %" PRIu64 " %zu\n", r.inserted ? 1 : 0,
                  r.evicted ? 1 : 0, r.hash, r.evicted_hash, r.slot);
    } else if (op == "hash") {
      std::size_t start = 0;
      in >> start;
      const auto h = index.hash_for_block(read_tokens(in), start);
      if (h.has_value()) {
        std::printf("hash %" PRIu64 "\n", *h);
      } else {
        std::printf("hash none\n");
      }
    } else if (op == "block") {
      std::uint64_t h = 0;
      in >> h;
      const auto* b = index.block(h);
      if (b == nullptr) {
        std::printf("block none\n");
      } else {
        std::printf("block %" PRIu64 " %" PRIu64 " %zu %zu %zu %" PRIu64, b->hash, b->parent_hash,
                    b->slot, b->token_start, b->token_count, b->last_used_tick);
        for (const auto t : b->tokens) {
          std::printf(" %" PRId64, t);
        }
        std::printf("\n");
      }
    } else if (op == "clear") {
      index.clear();
      std::printf("clear\n");
    } else if (op == "stats") {
      const auto s = index.stats();
      std::printf("stats %d %zu %zu %zu %zu %zu %zu %zu\n", s.enabled ? 1 : 0, s.block_tokens,
                  s.capacity_blocks, s.stored_blocks, s.hit_tokens, s.miss_tokens,
                  s.committed_tokens, s.evicted_blocks);
    } else if (!op.empty()) {
      std::printf("unknown op %s\n", op.c_str());
      return 2;
    }
  }
  return 0;
}

bool check(const Status& s, const char* what) {
  if (!s.is_ok()) {
    std::printf("FAIL %s: %s\n", what, s.message().c_str());
    return false;
  }
  return true;
}

// Deterministic bytes for fill pattern `seed`.
std::vector<std::uint8_t> pattern(std::size_t bytes, unsigned seed) {
  std::vector<std::uint8_t> v(bytes);
  for (std::size_t i = 0; i < bytes; ++i) {
    v[i] = static_cast<std::uint8_t>((i * 131u + seed * 29u + (i >> 9) * 7u) & 0xffu);
  }
  return v;
}

struct HostCache {
  std::vector<std::uint8_t> k, v, r, s;
};

bool fill(const HipContext& ctx, q35::DeviceCache& dc, unsigned seed, HostCache& host) {
  host.k = pattern(dc.key_cache.byte_size(), seed);
  host.v = pattern(dc.value_cache.byte_size(), seed + 1);
  host.r = pattern(dc.recurrent_r_cache.byte_size(), seed + 2);
  host.s = pattern(dc.recurrent_s_cache.byte_size(), seed + 3);
  return check(ctx.copy_to_buffer(dc.key_cache, host.k.data(), host.k.size()), "fill k") &&
         check(ctx.copy_to_buffer(dc.value_cache, host.v.data(), host.v.size()), "fill v") &&
         check(ctx.copy_to_buffer(dc.recurrent_r_cache, host.r.data(), host.r.size()), "fill r") &&
         check(ctx.copy_to_buffer(dc.recurrent_s_cache, host.s.data(), host.s.size()), "fill s");
}

bool read(const HipContext& ctx, const HipBuffer& b, std::vector<std::uint8_t>& out) {
  out.resize(b.byte_size());
  return check(ctx.copy_from_buffer(b, out.data(), out.size()), "read back");
}

// Rows [first, first + count) of every layer of a [layers][capacity][row_bytes] cache.
bool rows_equal(const std::vector<std::uint8_t>& got, const std::vector<std::uint8_t>& want,
                std::size_t layers, std::size_t capacity, std::size_t row_bytes,
                std::size_t first, std::size_t count, const char* what) {
  for (std::size_t l = 0; l < layers; ++l) {
    const std::size_t at = (l * capacity + first) * row_bytes;
    if (std::memcmp(got.data() + at, want.data() + at, count * row_bytes) != 0) {
      std::printf("FAIL %s rows %zu..%zu of layer %zu differ\n", what, first, first + count, l);
      return false;
    }
  }
  return true;
}

bool all_zero(const std::vector<std::uint8_t>& got, std::size_t layers, std::size_t capacity,
              std::size_t row_bytes, std::size_t first, const char* what) {
  for (std::size_t l = 0; l < layers; ++l) {
    for (std::size_t i = (l * capacity + first) * row_bytes; i < (l + 1) * capacity * row_bytes;
         ++i) {
      if (got[i] != 0) {
        std::printf("FAIL %s: byte %zu of layer %zu written past the restored rows\n", what, i, l);
        return false;
      }
    }
  }
  return true;
}

int run_store() {
  auto ctx_r = HipContext::create();
  if (!check(ctx_r.status(), "create")) {
    return 1;
  }
  const HipContext& ctx = ctx_r.value();
  constexpr std::size_t kBlock = 4;
  q35::RuntimeOptions options;
  options.context_tokens = 32;
  auto plan_r = q35::build_execution_plan(q35::qwen35_0_8b_shape(), 12, options);
  if (!check(plan_r.status(), "plan")) {
    return 1;
  }
  const q35::ExecutionPlan& plan = plan_r.value();
  auto cache_r = q35::allocate_device_cache(ctx, plan);
  if (!check(cache_r.status(), "cache")) {
    return 1;
  }
  q35::DeviceCache& dc = cache_r.value();
  const std::size_t layers = plan.cache.full_attention_layers;
  const std::size_t cap = plan.cache.attention_capacity_tokens;
  const std::size_t row = plan.cache.kv_dim * plan.cache.kv_cache_element_bytes;
  const std::size_t hidden = plan.hidden_size;

  std::vector<std::int64_t> tokens(12);
  for (std::size_t i = 0; i < tokens.size(); ++i) {
    tokens[i] = 1000 + static_cast<std::int64_t>(i * 37 % 11);
  }
  auto hidden_b = ctx.make_buffer(kBlock * hidden * sizeof(float));
  if (!check(hidden_b.status(), "hidden")) {
    return 1;
  }
  q35::PrefixCacheStore store;
  const q35::PrefixCacheConfig config{true, kBlock, 2, 0};
  store.configure(q35::prefix_layout_from_plan(plan, kBlock), config);

  // Block 0 after pattern A, block 1 after pattern B.
  HostCache a, b;
  std::vector<std::uint8_t> hidden_a = pattern(kBlock * hidden * sizeof(float), 40);
  std::vector<std::uint8_t> hidden_bytes_b = pattern(kBlock * hidden * sizeof(float), 50);
  if (!fill(ctx, dc, 1, a) ||
      !check(ctx.copy_to_buffer(hidden_b.value(), hidden_a.data(), hidden_a.size()), "h")) {
    return 1;
  }
  auto c0 = store.commit_block(ctx, dc, plan, hidden_b.value(), tokens, 0, kBlock);
  if (!check(c0.status(), "commit 0")) {
    return 1;
  }
  if (!fill(ctx, dc, 9, b) ||
      !check(ctx.copy_to_buffer(hidden_b.value(), hidden_bytes_b.data(), hidden_bytes_b.size()),
             "h")) {
    return 1;
  }
  auto c1 = store.commit_block(ctx, dc, plan, hidden_b.value(), tokens, kBlock, kBlock);
  auto again = store.commit_block(ctx, dc, plan, hidden_b.value(), tokens, 0, kBlock);
  auto partial = store.commit_block(ctx, dc, plan, hidden_b.value(), tokens, 8, 3);
  if (!check(c1.status(), "commit 1") || !check(again.status(), "commit again") ||
      !check(partial.status(), "commit partial")) {
    return 1;
  }
  std::printf("commits %d%d %d%d %d%d %d%d\n", c0.value().committed, c0.value().evicted,
              c1.value().committed, c1.value().evicted, again.value().committed,
              again.value().evicted, partial.value().committed, partial.value().evicted);

  // Wipe the device cache, then restore the two blocks.
  for (HipBuffer* buf : {&dc.key_cache, &dc.value_cache, &dc.recurrent_r_cache,
                         &dc.recurrent_s_cache}) {
    if (!check(ctx.zero_buffer(*buf, buf->byte_size()), "zero")) {
      return 1;
    }
  }
  const auto hit = store.lookup(tokens);
  std::printf("lookup %zu %zu\n", hit.hit_tokens, hit.block_hashes.size());
  if (!check(store.restore(ctx, dc, plan, hit.block_hashes), "restore")) {
    return 1;
  }
  std::vector<std::uint8_t> k, v, r, s, h(hidden * sizeof(float));
  if (!read(ctx, dc.key_cache, k) || !read(ctx, dc.value_cache, v) ||
      !read(ctx, dc.recurrent_r_cache, r) || !read(ctx, dc.recurrent_s_cache, s)) {
    return 1;
  }
  bool ok = rows_equal(k, a.k, layers, cap, row, 0, kBlock, "K block 0") &&
            rows_equal(v, a.v, layers, cap, row, 0, kBlock, "V block 0") &&
            rows_equal(k, b.k, layers, cap, row, kBlock, kBlock, "K block 1") &&
            rows_equal(v, b.v, layers, cap, row, kBlock, kBlock, "V block 1") &&
            all_zero(k, layers, cap, row, 2 * kBlock, "K") &&
            all_zero(v, layers, cap, row, 2 * kBlock, "V");
  if (ok && (r != b.r || s != b.s)) {
    std::printf("FAIL recurrent caches are not the last block's\n");
    ok = false;
  }
  const HipBuffer last = store.last_hidden(hit.block_hashes.back());
  if (ok && (!last.valid() ||
             !check(ctx.copy_from_buffer(last, h.data(), h.size()), "last hidden") ||
             std::memcmp(h.data(), hidden_bytes_b.data() + (kBlock - 1) * h.size(), h.size()) !=
               0)) {
    std::printf("FAIL last hidden row\n");
    ok = false;
  }
  if (!ok) {
    return 1;
  }

  // A third block evicts the least recently used one (block 0, looked up
  // before block 1), which breaks the chain at its start.
  auto c2 = store.commit_block(ctx, dc, plan, hidden_b.value(), tokens, 2 * kBlock, kBlock);
  if (!check(c2.status(), "commit 2")) {
    return 1;
  }
  const auto after = store.lookup(tokens);
  const Status missing = store.restore(ctx, dc, plan, {hit.block_hashes.front()});
  std::printf("evict %d%d lookup %zu missing '%s' evicted-hidden %d\n", c2.value().committed,
              c2.value().evicted, after.hit_tokens, missing.message().c_str(),
              store.last_hidden(hit.block_hashes.front()).valid() ? 1 : 0);
  auto st = store.stats();
  std::printf("stats %zu %zu %zu %zu %zu\n", st.stored_blocks, st.hit_tokens, st.miss_tokens,
              st.committed_tokens, st.evicted_blocks);
  store.configure(q35::prefix_layout_from_plan(plan, kBlock), config);
  std::printf("same-config stored %zu\n", store.stats().stored_blocks);
  auto other = q35::prefix_layout_from_plan(plan, kBlock);
  other.tokenizer_fingerprint = 7;
  store.configure(other, config);
  std::printf("new-layout stored %zu\n", store.stats().stored_blocks);
  std::printf("ok\n");
  return 0;
}

// The store outlives the request contexts that use it: a block committed
// through one context, which is then destroyed with its cache, is restored
// through a second context; reconfiguring then frees the arena (through the
// store's own context) and a commit allocates it again.  A block whose rows
// would run past the attention capacity is rejected, not copied.
int run_lifetime() {
  constexpr std::size_t kBlock = 4;
  q35::RuntimeOptions options;
  options.context_tokens = 32;
  auto plan_r = q35::build_execution_plan(q35::qwen35_0_8b_shape(), 12, options);
  if (!check(plan_r.status(), "plan")) {
    return 1;
  }
  const q35::ExecutionPlan& plan = plan_r.value();
  const std::size_t layers = plan.cache.full_attention_layers;
  const std::size_t cap = plan.cache.attention_capacity_tokens;
  const std::size_t row = plan.cache.kv_dim * plan.cache.kv_cache_element_bytes;
  const std::size_t hidden = plan.hidden_size;
  std::vector<std::int64_t> tokens(cap + 2 * kBlock);
  for (std::size_t i = 0; i < tokens.size(); ++i) {
    tokens[i] = 500 + static_cast<std::int64_t>(i * 13 % 17);
  }
  q35::PrefixCacheStore store;
  const q35::PrefixCacheConfig config{true, kBlock, 4, 0};
  store.configure(q35::prefix_layout_from_plan(plan, kBlock), config);
  HostCache a;
  const std::vector<std::uint8_t> hidden_a = pattern(kBlock * hidden * sizeof(float), 70);
  {
    auto first_r = HipContext::create();
    if (!check(first_r.status(), "create first")) {
      return 1;
    }
    const HipContext& first = first_r.value();
    auto cache_r = q35::allocate_device_cache(first, plan);
    auto hidden_r = first.make_buffer(kBlock * hidden * sizeof(float));
    if (!check(cache_r.status(), "cache first") || !check(hidden_r.status(), "hidden first") ||
        !fill(first, cache_r.value(), 21, a) ||
        !check(first.copy_to_buffer(hidden_r.value(), hidden_a.data(), hidden_a.size()), "h")) {
      return 1;
    }
    auto c0 = store.commit_block(first, cache_r.value(), plan, hidden_r.value(), tokens, 0,
                                 kBlock);
    if (!check(c0.status(), "commit first") || !c0.value().committed) {
      std::printf("FAIL first commit not stored\n");
      return 1;
    }
  }  // the first context, its cache and its hidden buffer are gone
  auto second_r = HipContext::create();
  if (!check(second_r.status(), "create second")) {
    return 1;
  }
  const HipContext& second = second_r.value();
  auto cache_r = q35::allocate_device_cache(second, plan);
  if (!check(cache_r.status(), "cache second")) {
    return 1;
  }
  q35::DeviceCache& dc = cache_r.value();
  for (HipBuffer* buf : {&dc.key_cache, &dc.value_cache, &dc.recurrent_r_cache,
                         &dc.recurrent_s_cache}) {
    if (!check(second.zero_buffer(*buf, buf->byte_size()), "zero")) {
      return 1;
    }
  }
  const auto hit = store.lookup(tokens);
  if (hit.block_hashes.size() != 1 ||
      !check(store.restore(second, dc, plan, hit.block_hashes), "restore second")) {
    std::printf("FAIL lookup after the first context: %zu blocks\n", hit.block_hashes.size());
    return 1;
  }
  std::vector<std::uint8_t> k, v, r, st, h(hidden * sizeof(float));
  if (!read(second, dc.key_cache, k) || !read(second, dc.value_cache, v) ||
      !read(second, dc.recurrent_r_cache, r) || !read(second, dc.recurrent_s_cache, st)) {
    return 1;
  }
  if (!rows_equal(k, a.k, layers, cap, row, 0, kBlock, "K") ||
      !rows_equal(v, a.v, layers, cap, row, 0, kBlock, "V") || r != a.r || st != a.s) {
    return 1;
  }
  const HipBuffer last = store.last_hidden(hit.block_hashes.back());
  if (!last.valid() || !check(second.copy_from_buffer(last, h.data(), h.size()), "hidden") ||
      std::memcmp(h.data(), hidden_a.data() + (kBlock - 1) * h.size(), h.size()) != 0) {
    std::printf("FAIL last hidden row after the first context\n");
    return 1;
  }
  std::printf("restored-after-destroy ok\n");

  // A new layout drops the arena; a commit through the second context
  // allocates a new one.
  auto other = q35::prefix_layout_from_plan(plan, kBlock);
  other.tokenizer_fingerprint = 3;
  store.configure(other, config);
  auto hidden_r = second.make_buffer(kBlock * hidden * sizeof(float));
  if (!check(hidden_r.status(), "hidden second")) {
    return 1;
  }
  auto c1 = store.commit_block(second, dc, plan, hidden_r.value(), tokens, 0, kBlock);
  if (!check(c1.status(), "commit after reconfigure") || !c1.value().committed) {
    return 1;
  }
  std::printf("reconfigured stored %zu\n", store.stats().stored_blocks);

  // The block at rows [cap, cap + kBlock) is past the K/V caches' capacity.
  if (cap % kBlock != 0) {
    std::printf("FAIL capacity %zu is not whole blocks\n", cap);
    return 1;
  }
  auto past = store.commit_block(second, dc, plan, hidden_r.value(), tokens, cap, kBlock);
  std::printf("past-capacity '%s' stored %zu\n",
              past.is_ok() ? "accepted" : past.status().message().c_str(),
              store.stats().stored_blocks);
  std::printf("ok\n");
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  const std::string mode = argc > 1 ? argv[1] : "index";
  if (mode == "index") {
    return run_index();
  }
  if (mode == "store") {
    return run_store();
  }
  if (mode == "lifetime") {
    return run_lifetime();
  }
  std::printf("usage: prefix_cache_check index | store | lifetime\n");
  return 2;
}
