// Prompt prefix cache index: which whole blocks of a prompt's tokens already
// have their cache state stored, chained by a rolling 64-bit hash.
//
// Mirrors toyllm::Qwen35PrefixCacheIndex (include/toyllm/runtime/
// qwen35_prefix_cache.hpp:10-80, src/runtime/qwen35_prefix_cache.cpp:1-213):
// the same configuration, statistics, lookup / commit / eviction results and
// hashes.  The hash of block b (tokens [b*B, (b+1)*B)) starts from its parent
// block's hash (for block 0 the root constant 1469598103934665603: the
// reference's literal, which is FNV-1a 64's published offset basis
// 14695981039346656037 without its last digit) and folds in B, b and each token
// as a 64-bit word with FNV-1a's step h = (h ^ word) * prime; a hash of 0
// becomes 1.  Blocks live in slots 0 .. capacity-1; when every slot is
// taken the least recently used block (the one with the oldest use tick) gives
// up its slot.
//
// Storage: a slot-indexed table plus a hash -> slot map, so a lookup costs one
// map probe per block instead of the reference's scan over all blocks.  Every
// lookup hit and commit takes a fresh tick, so use ticks are unique and the
// eviction victim is the same block the reference's scan picks.
#pragma once

#include <cstddef>
#include <cstdint>
#include <optional>
#include <unordered_map>
#include <vector>

namespace kraken::qwen35 {

// qwen35_prefix_cache.hpp:10-15
struct PrefixCacheConfig {
  bool enabled{false};
  std::size_t block_tokens{1024};
  std::size_t capacity_blocks{16};
  std::size_t min_reuse_tokens{0};
};

// qwen35_prefix_cache.hpp:17-26
struct PrefixCacheStats {
  bool enabled{false};
  std::size_t block_tokens{0};
  std::size_t capacity_blocks{0};
  std::size_t stored_blocks{0};
  std::size_t hit_tokens{0};
  std::size_t miss_tokens{0};
  std::size_t committed_tokens{0};
  std::size_t evicted_blocks{0};
};

// qwen35_prefix_cache.hpp:28-36
struct PrefixBlockMetadata {
  std::uint64_t hash{0};
  std::uint64_t parent_hash{0};
  std::size_t slot{0};
  std::size_t token_start{0};
  std::size_t token_count{0};
  std::vector<std::int64_t> tokens;
  std::uint64_t last_used_tick{0};
};

// qwen35_prefix_cache.hpp:38-41
struct PrefixCacheLookup {
  std::size_t hit_tokens{0};
  std::vector<std::uint64_t> block_hashes;
};

// qwen35_prefix_cache.hpp:43-49
struct PrefixCacheCommit {
  bool inserted{false};
  bool evicted{false};
  std::uint64_t hash{0};
  std::uint64_t evicted_hash{0};
  std::size_t slot{0};
};

// The chain's root hash and FNV-1a 64's prime, and the one-word step
// (qwen35_prefix_cache.cpp:11-19).
inline constexpr std::uint64_t kPrefixRootHash = 1469598103934665603ULL;
inline constexpr std::uint64_t kPrefixHashPrime = 1099511628211ULL;

[[nodiscard]] constexpr std::uint64_t prefix_mix_u64(std::uint64_t hash, std::uint64_t word) {
  return (hash ^ word) * kPrefixHashPrime;
}

class PrefixCacheIndex {
 public:
  // qwen35_prefix_cache.cpp:26-34: a zero block size disables the cache.
  explicit PrefixCacheIndex(PrefixCacheConfig config) : config_(config) {
    if (config_.block_tokens == 0) {
      config_.enabled = false;
    }
    reset_stats();
  }

  [[nodiscard]] const PrefixCacheConfig& config() const { return config_; }

  // qwen35_prefix_cache.cpp:40-47
  [[nodiscard]] PrefixCacheStats stats() const {
    PrefixCacheStats s = stats_;
    s.enabled = config_.enabled;
    s.block_tokens = config_.block_tokens;
    s.capacity_blocks = config_.capacity_blocks;
    s.stored_blocks = slot_of_.size();
    return s;
  }

  // qwen35_prefix_cache.cpp:49-93: the longest chain of stored blocks that
  // starts the prompt, each refreshed as used; below min_reuse_tokens it counts
  // as a miss (the refreshed use ticks stay).
  [[nodiscard]] PrefixCacheLookup lookup(const std::vector<std::int64_t>& tokens) {
    PrefixCacheLookup result;
    if (!active()) {
      stats_.miss_tokens += tokens.size();
      return result;
    }
    const std::size_t b = config_.block_tokens;
    std::uint64_t parent = kPrefixRootHash;
    for (std::size_t start = 0; start + b <= tokens.size(); start += b) {
      const std::uint64_t h = block_hash(tokens, start, parent);
      PrefixBlockMetadata* m = find(h);
      if (m == nullptr || m->parent_hash != parent || m->token_count != b ||
          !same_tokens(*m, tokens, start)) {
        break;
      }
      m->last_used_tick = ++tick_;
      result.hit_tokens += b;
      result.block_hashes.push_back(h);
      parent = h;
    }
    if (result.hit_tokens < config_.min_reuse_tokens) {
      result.hit_tokens = 0;
      result.block_hashes.clear();
    }
    stats_.hit_tokens += result.hit_tokens;
    stats_.miss_tokens += tokens.size() - result.hit_tokens;
    return result;
  }

  // qwen35_prefix_cache.cpp:95-142: record block [token_start, token_start+B)
  // of `tokens`.  A block already stored is only refreshed (inserted false).
  [[nodiscard]] PrefixCacheCommit commit_block(const std::vector<std::int64_t>& tokens,
                                               std::size_t token_start) {
    PrefixCacheCommit result;
    const std::size_t b = config_.block_tokens;
    if (!active() || token_start > tokens.size() || b > tokens.size() - token_start) {
      return result;
    }
    const std::uint64_t parent = parent_hash_for(tokens, token_start);
    const std::uint64_t h = block_hash(tokens, token_start, parent);
    result.hash = h;
    if (PrefixBlockMetadata* m = find(h); m != nullptr) {
      m->last_used_tick = ++tick_;
      result.slot = m->slot;
      return result;
    }
    std::size_t slot = slot_of_.size();
    if (slot >= config_.capacity_blocks) {
      slot = lru_slot();
      result.evicted_hash = slots_[slot].hash;
      result.evicted = result.evicted_hash != 0;
      slot_of_.erase(result.evicted_hash);
      if (result.evicted) {
        ++stats_.evicted_blocks;
      }
    } else if (slots_.size() <= slot) {
      slots_.resize(slot + 1);
    }
    result.slot = slot;
    result.inserted = true;

    PrefixBlockMetadata& m = slots_[slot];
    m.hash = h;
    m.parent_hash = parent;
    m.slot = slot;
    m.token_start = token_start;
    m.token_count = b;
    m.tokens.assign(tokens.begin() + static_cast<std::ptrdiff_t>(token_start),
                    tokens.begin() + static_cast<std::ptrdiff_t>(token_start + b));
    m.last_used_tick = ++tick_;
    slot_of_[h] = slot;
    stats_.committed_tokens += b;
    return result;
  }

  // qwen35_prefix_cache.cpp:144-155
  [[nodiscard]] const PrefixBlockMetadata* block(std::uint64_t hash) const {
    const auto it = slot_of_.find(hash);
    return it == slot_of_.end() ? nullptr : &slots_[it->second];
  }

  // qwen35_prefix_cache.cpp:157-165: the hash of a whole, block-aligned block.
  [[nodiscard]] std::optional<std::uint64_t> hash_for_block(
    const std::vector<std::int64_t>& tokens, std::size_t token_start) const {
    const std::size_t b = config_.block_tokens;
    if (b == 0 || token_start > tokens.size() || b > tokens.size() - token_start ||
        token_start % b != 0) {
      return std::nullopt;
    }
    return block_hash(tokens, token_start, parent_hash_for(tokens, token_start));
  }

  // qwen35_prefix_cache.cpp:167-174
  void clear() {
    slots_.clear();
    slot_of_.clear();
    tick_ = 0;
    reset_stats();
  }

 private:
  [[nodiscard]] bool active() const {
    return config_.enabled && config_.block_tokens != 0 && config_.capacity_blocks != 0;
  }

  void reset_stats() {
    stats_ = PrefixCacheStats{};
    stats_.enabled = config_.enabled;
    stats_.block_tokens = config_.block_tokens;
    stats_.capacity_blocks = config_.capacity_blocks;
  }

  // qwen35_prefix_cache.cpp:176-187
  [[nodiscard]] std::uint64_t block_hash(const std::vector<std::int64_t>& tokens,
                                         std::size_t token_start, std::uint64_t parent) const {
    const std::size_t b = config_.block_tokens;
    std::uint64_t h = prefix_mix_u64(parent, static_cast<std::uint64_t>(b));
    h = prefix_mix_u64(h, static_cast<std::uint64_t>(token_start / b));
    for (std::size_t i = 0; i < b; ++i) {
      h = prefix_mix_u64(h, static_cast<std::uint64_t>(tokens[token_start + i]));
    }
    return h == 0 ? 1 : h;
  }

  // qwen35_prefix_cache.cpp:189-196: the chain of whole blocks before token_start.
  [[nodiscard]] std::uint64_t parent_hash_for(const std::vector<std::int64_t>& tokens,
                                              std::size_t token_start) const {
    std::uint64_t parent = kPrefixRootHash;
    for (std::size_t start = 0; start < token_start; start += config_.block_tokens) {
      parent = block_hash(tokens, start, parent);
    }
    return parent;
  }

  [[nodiscard]] PrefixBlockMetadata* find(std::uint64_t hash) {
    const auto it = slot_of_.find(hash);
    return it == slot_of_.end() ? nullptr : &slots_[it->second];
  }

  [[nodiscard]] bool same_tokens(const PrefixBlockMetadata& m,
                                 const std::vector<std::int64_t>& tokens,
                                 std::size_t start) const {
    for (std::size_t i = 0; i < config_.block_tokens; ++i) {
      if (m.tokens[i] != tokens[start + i]) {
        return false;
      }
    }
    return true;
  }

  // qwen35_prefix_cache.cpp:198-211: the stored block with the oldest use tick.
  [[nodiscard]] std::size_t lru_slot() const {
    std::size_t victim = 0;
    for (std::size_t s = 1; s < slots_.size(); ++s) {
      if (slots_[s].last_used_tick < slots_[victim].last_used_tick) {
        victim = s;
      }
    }
    return victim;
  }

  PrefixCacheConfig config_;
  PrefixCacheStats stats_;
  std::vector<PrefixBlockMetadata> slots_;
  std::unordered_map<std::uint64_t, std::size_t> slot_of_;
  std::uint64_t tick_{0};
};

}  // namespace kraken::qwen35
