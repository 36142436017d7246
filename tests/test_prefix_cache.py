"""Prompt prefix cache: the block index (include/kraken/qwen35_prefix_cache.hpp)
and the device payload store (include/kraken/qwen35_prefix_store.hpp), driven by
tests/cpp/prefix_cache_check.cpp.

* CPU: the oracle's hash step against FNV-1a's published vectors; the oracle
  against the reference's known-answer tests (tests/smoke_test.cpp:263-335); the
  C++ index against the oracle, line for line (bit-exact hashes), on those
  scenarios, on edge cases and on seeded random operation scripts.
* GPU: commit / restore / evict round trip of real cache payloads, byte-exact.
"""
import os
import random
import subprocess

import numpy as np
import pytest

import prefix_cache as oracle_pc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "kraken-infer_amd", "build", "prefix_cache_check")


def _run(mode, stdin=""):
    if not os.path.exists(BIN):
        subprocess.run(["make", "-C", os.path.join(ROOT, "kraken-infer_amd")], check=True,
                       capture_output=True)
    proc = subprocess.run([BIN, mode], input=stdin, capture_output=True, text=True, timeout=300)
    print(proc.stdout[-3000:])
    return proc.returncode, proc.stdout


def _fnv1a(data: bytes) -> int:
    h = oracle_pc.FNV_OFFSET_BASIS
    for byte in data:
        h = oracle_pc.mix_u64(h, byte)
    return h


@pytest.mark.parametrize("data,want", [
    (b"", 0xCBF29CE484222325),
    (b"a", 0xAF63DC4C8601EC8C),
    (b"foobar", 0x85944171F73967E8),
])
def test_oracle_hash_step_matches_published_fnv1a(data, want):
    assert _fnv1a(data) == want


def test_oracle_reference_known_answers():
    # tests/smoke_test.cpp:263-304
    c = oracle_pc.PrefixCacheIndex(True, 2, 2, 0)
    first = [1, 2, 3, 4, 5]
    assert c.lookup(first) == (0, [])
    assert c.commit_block(first, 0)[0::4] == (1, 0) and c.commit_block(first, 2)[4] == 1
    hit, hashes = c.lookup(first)
    assert hit == 4 and len(hashes) == 2
    hit, hashes = c.lookup([1, 2, 9, 9])
    assert hit == 2 and len(hashes) == 1
    inserted, evicted, *_ = c.commit_block([7, 8, 9, 10], 0)
    assert inserted and evicted
    assert c.lookup(first)[0] == 2
    s = c.stats()
    assert s[3] == 2 and s[7] == 1
    # tests/smoke_test.cpp:306-335
    c = oracle_pc.PrefixCacheIndex(True, 2, 4, 4)
    tokens = [1, 2, 3, 4, 5]
    assert c.commit_block(tokens, 0)[0]
    assert c.lookup(tokens) == (0, [])
    assert c.commit_block(tokens, 2)[0]
    hit, hashes = c.lookup(tokens)
    assert hit == 4 and len(hashes) == 2
    c.clear()
    assert c.lookup(tokens) == (0, [])
    assert c.stats()[:4] == (1, 2, 4, 0)


def _tok(ts):
    return f"{len(ts)} " + " ".join(str(t) for t in ts)


REFERENCE_SCRIPTS = [
    [  # smoke_test.cpp:263-304
        "new 1 2 2 0", f"lookup {_tok([1, 2, 3, 4, 5])}", f"commit 0 {_tok([1, 2, 3, 4, 5])}",
        f"commit 2 {_tok([1, 2, 3, 4, 5])}", f"lookup {_tok([1, 2, 3, 4, 5])}",
        f"lookup {_tok([1, 2, 9, 9])}", f"commit 0 {_tok([7, 8, 9, 10])}",
        f"lookup {_tok([1, 2, 3, 4, 5])}", "stats",
    ],
    [  # smoke_test.cpp:306-335
        "new 1 2 4 4", f"commit 0 {_tok([1, 2, 3, 4, 5])}", f"lookup {_tok([1, 2, 3, 4, 5])}",
        f"commit 2 {_tok([1, 2, 3, 4, 5])}", f"lookup {_tok([1, 2, 3, 4, 5])}", "clear",
        f"lookup {_tok([1, 2, 3, 4, 5])}", "stats",
    ],
    [  # edges: disabled, zero block size, zero capacity, ragged and unaligned starts,
       # negative and 64-bit tokens, empty prompts, re-commit of a stored block
        "new 0 2 2 0", f"commit 0 {_tok([1, 2])}", f"lookup {_tok([1, 2])}", "stats",
        "new 1 0 2 0", f"commit 0 {_tok([1, 2])}", f"hash 0 {_tok([1, 2])}", "stats",
        "new 1 2 0 0", f"commit 0 {_tok([1, 2])}", f"lookup {_tok([1, 2])}", "stats",
        "new 1 3 3 0", f"lookup {_tok([])}", f"commit 1 {_tok([5, 6, 7, 8])}",
        f"commit 2 {_tok([5, 6, 7, 8])}", f"hash 1 {_tok([5, 6, 7, 8])}",
        f"hash 0 {_tok([5, 6, 7, 8])}", f"hash 3 {_tok([5, 6, 7, 8, 9, 10])}",
        f"commit 0 {_tok([-1, -9223372036854775808, 9223372036854775807])}",
        f"commit 0 {_tok([-1, -9223372036854775808, 9223372036854775807])}",
        f"lookup {_tok([-1, -9223372036854775808, 9223372036854775807, 4])}", "stats",
    ],
]


def _random_script(seed):
    rng = random.Random(seed)
    b = rng.choice([1, 2, 3, 4])
    lines = [f"new 1 {b} {rng.choice([1, 2, 3, 5])} {rng.choice([0, 0, b, 2 * b])}"]
    prompts = []
    for _ in range(60):
        if not prompts or rng.random() < 0.3:
            base = rng.choice(prompts) if prompts and rng.random() < 0.6 else []
            keep = rng.randint(0, len(base))
            p = base[:keep] + [rng.randint(0, 5) for _ in range(rng.randint(0, 4 * b))]
            prompts.append(p)
        p = rng.choice(prompts)
        r = rng.random()
        if r < 0.35:
            lines.append(f"lookup {_tok(p)}")
        elif r < 0.75:
            start = rng.randint(0, max(0, len(p) - 1))
            if rng.random() < 0.7:
                start -= start % b
            lines.append(f"commit {start} {_tok(p)}")
        elif r < 0.85:
            lines.append(f"hash {rng.randint(0, len(p))} {_tok(p)}")
        elif r < 0.95:
            lines.append("stats")
        else:
            lines.append("clear")
    return lines


def _compare(script):
    code, out = _run("index", "\n".join(script) + "\n")
    assert code == 0, out
    want = oracle_pc.run_script(script)
    got = out.splitlines()
    # Every stored block's record, too.
    hashes = {int(w) for line in want if line.startswith(("commit", "lookup"))
              for w in line.split()[1:] if len(w) > 6}
    extra = [f"block {h}" for h in sorted(hashes)]
    if extra:
        code, out2 = _run("index", "\n".join(script + extra) + "\n")
        assert code == 0
        got = out2.splitlines()
        want = oracle_pc.run_script(script + extra)
    assert got == want


@pytest.mark.parametrize("case", range(len(REFERENCE_SCRIPTS)))
def test_index_matches_oracle_reference_scripts(case):
    _compare(REFERENCE_SCRIPTS[case])


@pytest.mark.parametrize("seed", range(12))
def test_index_matches_oracle_random_scripts(seed):
    _compare(_random_script(seed))


@pytest.mark.gpu
def test_store_round_trip_on_device():
    print("prefix store round trip", flush=True)
    code, out = _run("store")
    assert code == 0, out
    lines = dict(line.split(" ", 1) for line in out.splitlines() if " " in line)
    # Block 0 and block 1 committed, the repeat and the partial chunk not.
    assert lines["commits"] == "10 10 00 00"
    assert lines["lookup"] == "8 2"
    # Block 2 evicts block 0 (least recently used), so the chain misses at once
    # and block 0's payload is gone.
    assert lines["evict"] == ("11 lookup 0 missing 'Qwen3.5 prefix cache payload is missing' "
                              "evicted-hidden 0")
    # stored, hit, miss, committed tokens, evicted: lookups of 12 tokens hit 8 then 0.
    assert lines["stats"] == "2 8 16 12 1"
    assert lines["same-config"] == "stored 2"
    assert lines["new-layout"] == "stored 0"
    assert out.strip().endswith("ok")


@pytest.mark.gpu
def test_store_outlives_request_contexts():
    """The store keeps its payload arena through its own context: a block
    committed through a context that is then destroyed restores through a
    second context byte for byte; reconfiguring frees and a commit reallocates
    the arena; a block running past the attention capacity is rejected with the
    reference's region error (mps_backend.mm:5768-5830)."""
    print("prefix store lifetime", flush=True)
    code, out = _run("lifetime")
    assert code == 0, out
    lines = dict(line.split(" ", 1) for line in out.splitlines() if " " in line)
    assert lines["restored-after-destroy"] == "ok"
    assert lines["reconfigured"] == "stored 1"
    assert lines["past-capacity"] == "'HIP copy size exceeds source buffer size' stored 1"
    assert out.strip().endswith("ok")


@pytest.mark.gpu
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_copy_regions_matches_numpy(hip_ctx, seed):
    """kraken_hip_copy_regions: aligned tiles, partial tiles, unaligned starts and byte
    tails, against the same copies done in numpy."""
    import ctypes

    class Region(ctypes.Structure):
        _fields_ = [("s", ctypes.c_size_t), ("d", ctypes.c_size_t), ("n", ctypes.c_size_t)]

    print(f"copy regions seed {seed}", flush=True)
    rng = np.random.default_rng(seed)
    n_src, n_dst = 1 << 20, 1 << 20  # floats
    src = rng.integers(0, 2**32, size=n_src, dtype=np.uint32).view(np.float32)
    dst0 = rng.integers(0, 2**32, size=n_dst, dtype=np.uint32).view(np.float32)
    s_buf, d_buf = hip_ctx.buffer(src), hip_ctx.buffer(dst0)
    # Disjoint destination slots, each range inside both buffers.
    regions, at = [], 0
    sizes = [16384, 16384 * 3, 100000, 7, 16, 1 << 16, 33, 5000]
    for n in sizes:
        s_off = int(rng.integers(0, n_src * 4 - n))
        if rng.random() < 0.5:
            s_off -= s_off % 16
        d_off = at + int(rng.integers(0, 64))
        regions.append((s_off, d_off, n))
        at = d_off + n + 64
    arr = (Region * len(regions))(*regions)
    hip_ctx.copy_regions(s_buf, d_buf, ctypes.addressof(arr), len(regions))
    want = dst0.view(np.uint8).copy()
    sb = src.view(np.uint8)
    for s_off, d_off, n in regions:
        want[d_off:d_off + n] = sb[s_off:s_off + n]
    got = d_buf.download(n_dst).view(np.uint8)
    assert np.array_equal(got, want)
