"""The reference's hot-path micro-benchmarks over the HIP backend
(include/kraken/qwen35_bench.hpp, mirroring benchmark_qwen35_metal_{gdn,attention},
qwen35_runtime.cpp:4808-5236), driven by tests/cpp/qwen35_driver_check.cpp.

* CPU: the argument checks, in the reference's order with its messages.
* GPU: the sample checksum (weighted sum of the first 16 output values, weights 1..16)
  against the CPU oracle run on the same deterministic modular inputs.  The GDN bench
  updates its state in place on every iteration, so the oracle replays warmup + timed
  iterations with the state carried.  Bounds: the weighted sum of the per-value
  tolerances, 1e-4 absolute per GDN value (fp32 state) and 1e-3 + 2e-3 |ref| per
  attention value (fp16 KV).
"""
import os
import subprocess

import numpy as np
import pytest

import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "kraken-infer_amd", "build", "qwen35_driver_check")
WEIGHTS = np.arange(1, 17, dtype=np.float64)


def _bench(*args):
    if not os.path.exists(BIN):
        subprocess.run(["make", "-C", os.path.join(ROOT, "kraken-infer_amd")], check=True,
                       capture_output=True)
    proc = subprocess.run([BIN, *map(str, args)], capture_output=True, text=True, timeout=300)
    print(proc.stdout[-3000:])
    return proc.returncode, proc.stdout


def _checksum(stdout):
    for line in stdout.splitlines():
        if line.startswith("checksum_exact "):
            return float(line.split()[1])
    raise AssertionError("no checksum in output:\n" + stdout)


GDN_CHECKS = [
    # tokens, key_heads, value_heads, head_dim, warmup, timed -> message
    ((0, 16, 16, 128, 1, 1), "Qwen3.5 GDN bench dimensions must be positive"),
    ((4, 0, 16, 128, 1, 1), "Qwen3.5 GDN bench dimensions must be positive"),
    ((4, 16, 16, 0, 1, 1), "Qwen3.5 GDN bench dimensions must be positive"),
    ((4, 16, 16, 128, 1, 0), "Qwen3.5 GDN bench timed iterations must be positive"),
    ((1 << 62, 16, 16, 128, 1, 1), "Qwen3.5 GDN bench value count overflow"),
]
ATTENTION_CHECKS = [
    # tokens, start, capacity, heads, kv_heads, head_dim, warmup, timed, f16 -> message
    ((0, 0, 0, 8, 2, 256, 1, 1, 1), "Qwen3.5 attention bench dimensions must be positive"),
    ((4, 0, 0, 8, 3, 256, 1, 1, 1), "Qwen3.5 attention bench heads must be divisible by kv_heads"),
    ((4, 0, 0, 8, 2, 512, 1, 1, 1), "Qwen3.5 attention bench head_dim must be at most 256"),
    ((4, 0, 0, 8, 2, 256, 1, 0, 1), "Qwen3.5 attention bench timed iterations must be positive"),
    ((4, (1 << 64) - 2, 0, 8, 2, 256, 1, 1, 1), "Qwen3.5 attention bench key count overflow"),
    ((64, 0, 10, 8, 2, 256, 1, 1, 1), "Qwen3.5 attention bench chunk exceeds capacity_tokens"),
    ((1 << 60, 0, 0, 8, 2, 256, 1, 1, 1), "Qwen3.5 attention bench value count overflow"),
]


@pytest.mark.parametrize("args,message", GDN_CHECKS)
def test_gdn_bench_argument_checks(args, message):
    code, out = _bench("bench-gdn", *args)
    assert code == 1 and out.strip() == f"error 1: {message}"


@pytest.mark.parametrize("args,message", ATTENTION_CHECKS)
def test_attention_bench_argument_checks(args, message):
    code, out = _bench("bench-attention", *args)
    assert code == 1 and out.strip() == f"error 1: {message}"


def _gdn_inputs(tokens, hk, hv, d):
    """qwen35_runtime.cpp:4846-4862, in float32 arithmetic."""
    qk = np.arange(tokens * hk * d)
    vv = np.arange(tokens * hv * d)
    gg = np.arange(tokens * hv)
    ss = np.arange(hv * d * d)
    f = np.float32
    q = f(0.001) * (1 + qk % 17).astype(f)
    k = f(0.0007) * (1 + qk % 19).astype(f)
    v = f(0.002) * (1 + vv % 23).astype(f)
    g = f(-0.002) * (1 + gg % 7).astype(f)
    b = f(0.25) + f(0.01) * (gg % 11).astype(f)
    s = f(0.0001) * (1 + ss % 13).astype(f)
    return q, k, v, g, b, s


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(64, 2, 2, 128), (8, 2, 2, 128), (5, 2, 4, 64)])
def test_gdn_bench_checksum_matches_oracle(shape):
    tokens, hk, hv, d = shape
    warmup, timed = 1, 2
    print(f"bench gdn {shape}", flush=True)
    code, out = _bench("bench-gdn", tokens, hk, hv, d, warmup, timed)
    assert code == 0, out
    q, k, v, g, b, s = _gdn_inputs(tokens, hk, hv, d)
    for _ in range(warmup + timed):
        y, s = oracle.gated_delta_net(q, k, v, g, b, s, tokens, hk, hv, d)
    want = float(np.dot(y[:16].astype(np.float64), WEIGHTS[:min(16, y.size)]))
    assert abs(_checksum(out) - want) <= 1e-4 * WEIGHTS.sum(), (_checksum(out), want)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [
    # tokens, start, capacity, heads, kv_heads, head_dim, f16
    (64, 0, 0, 8, 2, 256, 1),     # flash256
    (1, 100, 101, 8, 2, 256, 1),  # split-KV decode, F16 cache
    (3, 40, 50, 4, 2, 128, 0),    # split-KV decode, F32 cache
])
def test_attention_bench_checksum_matches_oracle(shape):
    tokens, start, cap, heads, kv_heads, d, f16 = shape
    print(f"bench attention {shape}", flush=True)
    code, out = _bench("bench-attention", tokens, start, cap, heads, kv_heads, d, 1, 2, f16)
    assert code == 0, out
    cap = cap or start + tokens
    f = np.float32
    qi = np.arange(tokens * heads * d)
    ci = np.arange(cap * kv_heads * d)
    q = ((qi * 13) % 31 - 15).astype(f) * f(0.015)
    kc = ((ci * 7) % 29 - 14).astype(f) * f(0.012)
    vc = ((ci * 11) % 37 - 18).astype(f) * f(0.025)
    if f16:
        kc, vc = oracle.f32_to_f16_bits(kc), oracle.f32_to_f16_bits(vc)
    ref = oracle.attention_batched(q, kc, vc, 0, start, tokens, cap, heads, kv_heads, d,
                                   round_query_f16=bool(f16) and d == 256 and tokens >= 64)
    ref = ref[:16].astype(np.float64)
    want = float(np.dot(ref, WEIGHTS[:ref.size]))
    bound = float(np.dot(1e-3 + 2e-3 * np.abs(ref), WEIGHTS[:ref.size]))
    assert abs(_checksum(out) - want) <= bound, (_checksum(out), want, bound)
