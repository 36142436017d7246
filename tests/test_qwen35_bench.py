"""The reference's hot-path micro-benchmarks over the HIP backend
(include/kraken/qwen35_bench.hpp, mirroring benchmark_qwen35_metal_{matmul,gdn,attention},
qwen35_runtime.cpp:4558-5236), driven by tests/cpp/qwen35_driver_check.cpp.

* CPU: the argument checks, in the reference's order with its messages.
* GPU: the sample checksum (weighted sum of the first 16 output values, weights 1..16)
  against the CPU oracle run on the same deterministic modular inputs.  The GDN bench
  updates its state in place on every iteration, so the oracle replays warmup + timed
  iterations with the state carried.  Bounds: the weighted sum of the per-value
  tolerances, 1e-4 absolute per GDN value (fp32 state) and 1e-3 + 2e-3 |ref| per
  attention value (fp16 KV).  The matmul bench's checksum against the oracle's
  kquant_matmul at the precision of the token count (f16 weights and inputs above 8
  tokens, f16 weights for 4 to 8, fp32 below), 1e-5 of sum |w x| per value.
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


def _small_gguf(path):
    """A GGUF with one Q4_K, one Q6_K and one F32 tensor (tests/gguf_writer.py)."""
    import gguf_writer as gw
    import qwen35_decode_cases as qc

    rng = np.random.default_rng(9)
    tensors = [("w4", (512, 40), gw.GGML_Q4_K, qc.quant(rng, gw.GGML_Q4_K, 40, 512)),
               ("w6", (256, 24), gw.GGML_Q6_K, qc.quant(rng, gw.GGML_Q6_K, 24, 256)),
               ("v", (8,), gw.GGML_F32, np.ones(8, np.float32)),
               ("w3", (256, 2, 2), gw.GGML_Q4_K, qc.quant(rng, gw.GGML_Q4_K, 4, 256))]
    gw.write(path, [("general.architecture", gw.STRING, "qwen35")], tensors)
    return {name: (shape, typ, data) for name, shape, typ, data in tensors}


def test_matmul_bench_argument_checks(tmp_path):
    """benchmark_qwen35_metal_matmul's checks, in its order, with its messages
    (qwen35_runtime.cpp:4560-4626); all of them fail before a context is made."""
    path = tmp_path / "m.gguf"
    _small_gguf(path)
    (tmp_path / "notes.txt").write_text("x")
    empty = tmp_path / "empty"
    empty.mkdir()
    cases = [
        (("", "w4", 8, 1, 1), "error 1: Qwen3.5 matmul bench requires --model"),
        ((path, "", 8, 1, 1), "error 1: Qwen3.5 matmul bench requires --tensor"),
        ((path, "w4", 0, 1, 1), "error 1: Qwen3.5 matmul bench tokens must be positive"),
        ((path, "w4", 8, 1, 0), "error 1: Qwen3.5 matmul bench timed iterations must be positive"),
        ((tmp_path / "absent.gguf", "w4", 8, 1, 1),
         f"error 2: model path does not exist: {tmp_path / 'absent.gguf'}"),
        ((tmp_path / "notes.txt", "w4", 8, 1, 1),
         f"error 1: model file is not a GGUF file: {tmp_path / 'notes.txt'}"),
        ((empty, "w4", 8, 1, 1), f"error 2: no GGUF file found in {empty}"),
        ((path, "nope", 8, 1, 1), "error 1: Qwen3.5 matmul bench tensor not found: nope"),
        ((path, "v", 8, 1, 1), "error 1: Qwen3.5 matmul bench tensor must be 2D: v"),
        ((path, "w3", 8, 1, 1), "error 1: Qwen3.5 matmul bench tensor must be 2D: w3"),
        ((path, "w4", 1 << 62, 1, 1), "error 1: Qwen3.5 matmul bench value count overflow"),
    ]
    for args, message in cases:
        code, out = _bench("bench-matmul", *args)
        assert code == 1 and out.strip() == message, (args, out)


@pytest.mark.gpu
@pytest.mark.parametrize("tensor,tokens", [("w4", 1024), ("w6", 13), ("w4", 5), ("w6", 2)])
def test_matmul_bench_checksum_matches_oracle(tmp_path, tensor, tokens):
    """The sample checksum of the matmul bench (tensor of a GGUF directory, the
    reference's (i mod 23 - 11) / 32 input) against the oracle's product at the
    precision the reference uses for that token count."""
    import qwen35_decode_cases as qc

    model = _small_gguf(tmp_path / "m.gguf")
    print(f"bench matmul {tensor} tokens={tokens}", flush=True)
    code, out = _bench("bench-matmul", tmp_path, tensor, tokens, 1, 2)
    assert code == 0, out
    assert f"Dispatch: {'kquant_gemm_f16_mfma' if tokens > 8 else ''}" in out
    (cols, rows), typ, data = model[tensor]
    x = ((np.arange(tokens * cols) % 23) - 11).astype(np.float32) * np.float32(0.03125)
    fmt = qc.FMT[typ]
    want = oracle.kquant_matmul(fmt, data, rows, cols, x, tokens, weight_f16=tokens >= 4,
                                input_f16=tokens > 8)[:16].astype(np.float64)
    w = oracle.kquant_dequantize(fmt, data, rows * cols // 256).reshape(rows, cols)
    scale = (np.abs(w) @ np.abs(x[:cols]))[:16]
    bound = float(np.dot(1e-5 * scale + 1e-6, WEIGHTS[:want.size]))
    assert abs(_checksum(out) - float(np.dot(want, WEIGHTS[:want.size]))) <= bound
