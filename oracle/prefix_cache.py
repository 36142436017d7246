"""CPU oracle of the prompt prefix cache index (pure Python).

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of
include/kraken/qwen35_prefix_cache.hpp.  Product code never imports it.

Restates toyllm::Qwen35PrefixCacheIndex (src/runtime/qwen35_prefix_cache.cpp)
in its own structure: a list of block records in insertion order, found by a
linear scan, the eviction victim the first record with the smallest use tick,
removed from the list.

Pinning:
* the hash step (FNV-1a 64: xor, then multiply by 1099511628211, mod 2**64) is
  checked against FNV-1a's published test vectors by hashing bytes from FNV's
  published offset basis;
* lookup / commit / eviction / statistics are checked against the reference's
  own known-answer tests (tests/smoke_test.cpp:263-335);
* the root hash 1469598103934665603 is the reference's literal
  (qwen35_prefix_cache.cpp:11; FNV's published basis without its last digit):
  no test vector of the reference fixes it, so that constant is
  "parity unpinned" beyond the citation.
"""
from __future__ import annotations

MASK = (1 << 64) - 1
ROOT_HASH = 1469598103934665603  # qwen35_prefix_cache.cpp:11
PRIME = 1099511628211            # qwen35_prefix_cache.cpp:12
FNV_OFFSET_BASIS = 14695981039346656037  # FNV-1a 64, for the published vectors


def mix_u64(h: int, word: int) -> int:
    """qwen35_prefix_cache.cpp:14-18"""
    return ((h ^ (word & MASK)) * PRIME) & MASK


class PrefixCacheIndex:
    """qwen35_prefix_cache.cpp:26-211"""

    def __init__(self, enabled=False, block_tokens=1024, capacity_blocks=16,
                 min_reuse_tokens=0):
        self.enabled = bool(enabled) and block_tokens != 0  # :26-30
        self.block_tokens = block_tokens
        self.capacity_blocks = capacity_blocks
        self.min_reuse_tokens = min_reuse_tokens
        self.blocks = []  # dicts in insertion order
        self.tick = 0
        self._reset_stats()

    def _reset_stats(self):
        self.hit_tokens = 0
        self.miss_tokens = 0
        self.committed_tokens = 0
        self.evicted_blocks = 0

    def _active(self):
        return self.enabled and self.block_tokens != 0 and self.capacity_blocks != 0

    def _hash(self, tokens, start, parent):  # :176-187
        h = mix_u64(parent, self.block_tokens)
        h = mix_u64(h, start // self.block_tokens)
        for i in range(self.block_tokens):
            h = mix_u64(h, tokens[start + i])
        return 1 if h == 0 else h

    def _parent(self, tokens, start):  # :189-196
        p = ROOT_HASH
        s = 0
        while s < start:
            p = self._hash(tokens, s, p)
            s += self.block_tokens
        return p

    def block(self, h):  # :144-155
        for b in self.blocks:
            if b["hash"] == h:
                return b
        return None

    def stats(self):  # :40-47
        return (int(self.enabled), self.block_tokens, self.capacity_blocks, len(self.blocks),
                self.hit_tokens, self.miss_tokens, self.committed_tokens, self.evicted_blocks)

    def lookup(self, tokens):  # :49-93
        hit, hashes = 0, []
        if not self._active():
            self.miss_tokens += len(tokens)
            return hit, hashes
        parent = ROOT_HASH
        start = 0
        while start + self.block_tokens <= len(tokens):
            h = self._hash(tokens, start, parent)
            m = self.block(h)
            if (m is None or m["parent"] != parent or m["count"] != self.block_tokens
                    or m["tokens"] != list(tokens[start:start + self.block_tokens])):
                break
            self.tick += 1
            m["tick"] = self.tick
            hit += self.block_tokens
            hashes.append(h)
            parent = h
            start += self.block_tokens
        if hit < self.min_reuse_tokens:
            hit, hashes = 0, []
        self.hit_tokens += hit
        self.miss_tokens += len(tokens) - hit
        return hit, hashes

    def commit_block(self, tokens, start):  # :95-142
        """(inserted, evicted, hash, evicted_hash, slot)"""
        if not self._active() or start + self.block_tokens > len(tokens):
            return (0, 0, 0, 0, 0)
        parent = self._parent(tokens, start)
        h = self._hash(tokens, start, parent)
        m = self.block(h)
        if m is not None:
            self.tick += 1
            m["tick"] = self.tick
            return (0, 0, h, 0, m["slot"])
        evicted_hash = 0
        if len(self.blocks) < self.capacity_blocks:  # :198-211
            slot = len(self.blocks)
        else:
            victim = self.blocks[0]
            for b in self.blocks:
                if b["tick"] < victim["tick"]:
                    victim = b
            slot = victim["slot"]
            evicted_hash = victim["hash"]
            self.blocks.remove(victim)
        evicted = int(evicted_hash != 0)
        self.evicted_blocks += evicted
        self.tick += 1
        self.blocks.append({"hash": h, "parent": parent, "slot": slot, "start": start,
                            "count": self.block_tokens,
                            "tokens": list(tokens[start:start + self.block_tokens]),
                            "tick": self.tick})
        self.committed_tokens += self.block_tokens
        return (1, evicted, h, evicted_hash, slot)

    def hash_for_block(self, tokens, start):  # :157-165
        b = self.block_tokens
        if b == 0 or start + b > len(tokens) or start % b != 0:
            return None
        return self._hash(tokens, start, self._parent(tokens, start))

    def clear(self):  # :167-174
        self.blocks = []
        self.tick = 0
        self._reset_stats()


def run_script(lines):
    """Runs the operation script of tests/cpp/prefix_cache_check.cpp `index`
    and returns its output lines."""
    out = []
    idx = PrefixCacheIndex()

    def toks(words):
        n = int(words[0])
        return [int(w) for w in words[1:1 + n]]

    for line in lines:
        w = line.split()
        if not w:
            continue
        op = w[0]
        if op == "new":
            idx = PrefixCacheIndex(int(w[1]) != 0, int(w[2]), int(w[3]), int(w[4]))
            out.append("new")
        elif op == "lookup":
            hit, hashes = idx.lookup(toks(w[1:]))
            out.append(" ".join(["lookup", str(hit)] + [str(h) for h in hashes]))
        elif op == "commit":
            r = idx.commit_block(toks(w[2:]), int(w[1]))
            out.append("commit " + " ".join(str(x) for x in r))
        elif op == "hash":
            h = idx.hash_for_block(toks(w[2:]), int(w[1]))
            out.append(f"hash {'none' if h is None else h}")
        elif op == "block":
            b = idx.block(int(w[1]))
            if b is None:
                out.append("block none")
            else:
                out.append(" ".join(str(x) for x in [
                    "block", b["hash"], b["parent"], b["slot"], b["start"], b["count"],
                    b["tick"]] + b["tokens"]))
        elif op == "clear":
            idx.clear()
            out.append("clear")
        elif op == "stats":
            out.append("stats " + " ".join(str(x) for x in idx.stats()))
        else:
            raise ValueError(op)
    return out
