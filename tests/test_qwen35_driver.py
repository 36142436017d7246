"""The Qwen3.5 execution plan and layer drivers (include/kraken/qwen35_plan.hpp,
include/kraken/qwen35_layers.hpp), driven by tests/cpp/qwen35_driver_check.cpp.

* Plan (CPU): the reference smoke test's known answers for Qwen3.5-0.8B
  (smoke_test.cpp:2146-2167, transcribed in tests/golden/qwen35_plan_known_answers.json),
  the argument checks of build_qwen35_execution_plan (qwen35_runtime.cpp:4379-4413)
  in order with their messages, cache sizes when slots, snapshots and f32 KV
  change every term, and the layer walk of run_qwen35_decode_tokens
  (qwen35_runtime.cpp:3885-3933).
* Layer drivers (GPU): one chunk of run_qwen35_linear_layer_chunk and of
  run_qwen35_full_attention_layer_chunk on the 0.8B plan, in the reference's op
  order and fused, against the same op chain run on the CPU oracle: outputs,
  the cache region the layer owns, and every other layer's region untouched.
  Tolerances: 1e-4 absolute for the GDN path (fp32 state), 2e-3 relative /
  1e-3 absolute for fp16-KV attention outputs; f16 cache rows may differ by one
  unit in the last place where the normed and rotated key rounds differently.
"""
import json
import os
import subprocess
import tempfile

import numpy as np
import pytest

import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "kraken-infer_amd", "build", "qwen35_driver_check")
GOLDEN = os.path.join(ROOT, "tests", "golden", "qwen35_plan_known_answers.json")

# Qwen3.5-0.8B shapes (qwen35_0_8b_shape()).
CONV_K, CHANNELS, HK, HV, DK, INNER = 4, 6144, 16, 16, 128, 2048
LINEAR_LAYERS, FULL_LAYERS = 18, 6
R_ELEMS, S_ELEMS = (CONV_K - 1) * CHANNELS, DK * INNER
HEADS, KV_HEADS, HEAD_DIM = 8, 2, 256
KV_DIM = KV_HEADS * HEAD_DIM
SECTIONS, THETA, EPS = (11, 11, 10, 0), 1e7, 1e-6


def _binary():
    if not os.path.exists(BIN):
        subprocess.run(["make", "-C", os.path.join(ROOT, "kraken-infer_amd")], check=True,
                       capture_output=True)
    return BIN


def _run(*args):
    proc = subprocess.run([_binary(), *args], capture_output=True, text=True, timeout=300)
    print(proc.stdout[-4000:])
    assert proc.returncode == 0, proc.stdout[-2000:] + proc.stderr[-2000:]
    return proc.stdout


def _plan_output():
    out = _run("plan")
    values, statuses, walk, kinds = {}, {}, [], {}
    for line in out.splitlines():
        if line.startswith("status "):
            label, rest = line[len("status "):].split(": ", 1)
            statuses[label] = rest.strip()
        elif line.startswith("walk "):
            _, i, kind, idx = line.split()
            walk.append((int(i), kind, int(idx)))
        elif line.startswith("layer_kind "):
            _, i, kind = line.split()
            kinds[int(i)] = kind
        elif "=" in line and " " not in line:
            k, v = line.split("=", 1)
            values[k] = int(v)
    summaries = out.split("--- summary")
    return out, values, statuses, walk, kinds, summaries


def test_plan_matches_reference_known_answers():
    with open(GOLDEN) as f:
        golden = json.load(f)
    out, values, _, _, kinds, summaries = _plan_output()
    exp = golden["expected"]
    for key, want in exp.items():
        if key == "summary_contains":
            continue
        got = values[key]
        assert got == int(want), (key, got, want)
    for i, kind in golden["model"]["layer_kinds_checked"].items():
        assert kinds[int(i)] == kind
    assert sum(k == "linear_attention" for k in kinds.values()) == golden["model"][
        "linear_attention_layers"]
    for text in exp["summary_contains"]:
        assert text in summaries[1]


def test_plan_argument_checks_in_reference_order():
    _, _, statuses, _, _, _ = _plan_output()
    assert statuses["prompt_zero"] == (
        "invalid_argument Qwen3.5 execution plan requires at least one prompt token")
    assert statuses["chunk_zero"] == "invalid_argument Qwen3.5 prefill chunk size must be positive"
    assert statuses["slots_zero"] == "invalid_argument Qwen3.5 sequence slot count must be positive"
    # hidden_size is checked before head_dim (both invalid in that case).
    assert statuses["hidden_zero"] == "invalid_argument hidden_size must be positive"
    assert statuses["head_dim_negative"] == "invalid_argument head_dim must be positive"
    assert statuses["inner_indivisible"] == (
        "invalid_argument linear_inner_size must be divisible by linear_value_heads")
    assert statuses["kinds_short"] == (
        "invalid_argument Qwen3.5 weight map has fewer layers than main layers")
    assert statuses["kv_overflow"] == "invalid_argument Qwen3.5 KV cache byte count overflow"


def test_plan_cache_terms_with_slots_snapshots_and_f32_kv():
    out, _, _, _, _, summaries = _plan_output()
    s2 = summaries[2]
    # capacity = max(context 262144, 3000 + 64); rows = 2 slots * (1 + 3 snapshots).
    kv = FULL_LAYERS * 262144 * (KV_DIM * 2) * 4
    rows = 2 * (1 + 3)
    r = LINEAR_LAYERS * rows * R_ELEMS * 4
    s = LINEAR_LAYERS * rows * S_ELEMS * 4
    assert f"Cache bytes: kv={kv} (f32), recurrent_r={r}, recurrent_s={s}, total={kv + r + s}" in s2
    assert "chunks=3, final_chunk=1000, output_only_last=no" in s2
    # An MTP layer past the main ones is in neither cache.
    assert "mtp_model: ok main=24 total=25 full=6 linear=18" in out


def test_decode_layer_walk():
    _, _, statuses, walk, _, _ = _plan_output()
    assert len(walk) == 24
    full = [i for i, kind, _ in walk if kind == "full_attention"]
    assert full == [3, 7, 11, 15, 19, 23]
    assert [idx for _, kind, idx in walk if kind == "full_attention"] == list(range(6))
    assert [idx for _, kind, idx in walk if kind == "linear_attention"] == list(range(18))
    assert statuses["walk"] == "ok"
    assert statuses["walk_mtp"] == "invalid_argument Qwen3.5 decode layer loop reached MTP layer"
    assert statuses["walk_count"] == (
        "internal_error Qwen3.5 decode layer execution count mismatch")


def _write(d, name, arr):
    np.ascontiguousarray(arr).tofile(os.path.join(d, name))


def _read(d, name, dtype):
    return np.fromfile(os.path.join(d, name), dtype=dtype)


@pytest.mark.gpu
@pytest.mark.parametrize("tokens,layer", [(1, 5), (80, 1), (7, 17)])
@pytest.mark.parametrize("order", ["reference", "fused"])
def test_linear_attention_driver_matches_oracle_chain(order, tokens, layer):
    rng = np.random.default_rng(100 + tokens)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    qkv = f(tokens, CHANNELS)
    z = f(tokens, INNER)
    beta = f(tokens, HV)
    alpha = f(tokens, HV)
    conv1d = 0.5 * f(CHANNELS, CONV_K)
    dt_bias = f(HV)
    ssm_a = -rng.random(HV).astype(np.float32)
    norm = (1 + 0.1 * f(DK)).astype(np.float32)
    r0 = 0.5 * f(LINEAR_LAYERS * R_ELEMS)
    s0 = 0.1 * f(LINEAR_LAYERS * S_ELEMS)
    with tempfile.TemporaryDirectory() as d:
        with open(os.path.join(d, "meta.txt"), "w") as fh:
            fh.write(f"{tokens} {layer}\n")
        for name, arr in [("qkv", qkv), ("z", z), ("beta", beta), ("alpha", alpha),
                          ("conv1d", conv1d), ("dt_bias", dt_bias), ("ssm_a", ssm_a),
                          ("ssm_norm", norm), ("r0", r0), ("s0", s0)]:
            _write(d, name + ".f32", arr)
        print(f"linear driver order={order} tokens={tokens} layer={layer}", flush=True)
        _run("linear", d, order)
        y = _read(d, "out.f32", np.float32)
        r1 = _read(d, "r1.f32", np.float32)
        s1 = _read(d, "s1.f32", np.float32)

    ro, so = layer * R_ELEMS, layer * S_ELEMS
    # The reference chain (qwen35_runtime.cpp:2746-3008) on the oracle.
    ci, r_new = oracle.build_ssm_conv_state(r0[ro:ro + R_ELEMS], qkv.ravel(), CONV_K, CHANNELS,
                                            tokens)
    conv = oracle.silu(oracle.ssm_conv(ci, conv1d.ravel(), CONV_K, CHANNELS, tokens, 1))
    q, k, v = oracle.split_qkv_l2_norm(conv, tokens, HK, HV, DK, EPS)
    g, b = oracle.prepare_gdn_gate_beta(alpha.ravel(), beta.ravel(), dt_bias, ssm_a, tokens, HV)
    y_ref, s_new = oracle.gated_delta_net(q, k, v, g, b, s0[so:so + S_ELEMS], tokens, HK, HV, DK)
    y_ref = oracle.norm_gated(y_ref, norm, z.ravel(), tokens, HV, DK, EPS)

    np.testing.assert_allclose(y, y_ref, rtol=0, atol=1e-4)
    np.testing.assert_array_equal(r1[ro:ro + R_ELEMS], r_new)
    np.testing.assert_allclose(s1[so:so + S_ELEMS], s_new, rtol=0, atol=1e-4)
    # Other layers' R and S regions are untouched.
    np.testing.assert_array_equal(np.delete(r1, np.s_[ro:ro + R_ELEMS]),
                                  np.delete(r0, np.s_[ro:ro + R_ELEMS]))
    np.testing.assert_array_equal(np.delete(s1, np.s_[so:so + S_ELEMS]),
                                  np.delete(s0, np.s_[so:so + S_ELEMS]))


def _f16_ulp_close(got_bits, want_bits):
    g = got_bits.astype(np.int32)
    w = want_bits.astype(np.int32)
    return np.abs(g - w).max() <= 1


@pytest.mark.gpu
@pytest.mark.parametrize("tokens,start,layer", [(1, 37, 2), (70, 0, 0), (66, 100, 5),
                                                (5, 200, 3)])
@pytest.mark.parametrize("order", ["reference", "fused"])
def test_full_attention_driver_matches_oracle_chain(order, tokens, start, layer):
    cap = start + tokens + 3
    rng = np.random.default_rng(200 + tokens + start)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)
    qg = f(tokens, HEADS, 2, HEAD_DIM)
    key = f(tokens, KV_DIM)
    value = f(tokens, KV_DIM)
    q_norm = (1 + 0.1 * f(HEAD_DIM)).astype(np.float32)
    k_norm = (1 + 0.1 * f(HEAD_DIM)).astype(np.float32)
    kc0 = oracle.f32_to_f16_bits(f(FULL_LAYERS * cap * KV_DIM))
    vc0 = oracle.f32_to_f16_bits(f(FULL_LAYERS * cap * KV_DIM))
    with tempfile.TemporaryDirectory() as d:
        with open(os.path.join(d, "meta.txt"), "w") as fh:
            fh.write(f"{tokens} {start} {layer} {cap}\n")
        for name, arr in [("qg.f32", qg), ("key.f32", key), ("value.f32", value),
                          ("q_norm.f32", q_norm), ("k_norm.f32", k_norm), ("kc0.u16", kc0),
                          ("vc0.u16", vc0)]:
            _write(d, name, arr)
        print(f"full driver order={order} tokens={tokens} start={start} layer={layer}",
              flush=True)
        _run("full", d, order)
        y = _read(d, "out.f32", np.float32)
        kc1 = _read(d, "kc1.u16", np.uint16)
        vc1 = _read(d, "vc1.u16", np.uint16)

    # The reference chain (qwen35_runtime.cpp:3229-3355) on the oracle.
    q = np.ascontiguousarray(qg[:, :, 0, :]).ravel()
    gate = np.ascontiguousarray(qg[:, :, 1, :]).ravel()
    q = oracle.qk_norm_f32_batched(q, q_norm, tokens, HEADS, HEAD_DIM, EPS)
    k = oracle.qk_norm_f32_batched(key.ravel(), k_norm, tokens, KV_HEADS, HEAD_DIM, EPS)
    pos = oracle.make_mrope_positions(start, tokens)
    q = oracle.mrope(q, pos, tokens, HEADS, HEAD_DIM, 2 * sum(SECTIONS), SECTIONS, THETA)
    k = oracle.mrope(k, pos, tokens, KV_HEADS, HEAD_DIM, 2 * sum(SECTIONS), SECTIONS, THETA)
    off = (layer * cap + start) * KV_DIM
    kc = oracle.copy_f32_rows_to_f16(k, kc0, tokens, KV_DIM, KV_DIM, 0, KV_DIM, off)
    vc = oracle.copy_f32_rows_to_f16(value.ravel(), vc0, tokens, KV_DIM, KV_DIM, 0, KV_DIM, off)
    attn = oracle.attention_batched(q, kc, vc, layer, start, tokens, cap, HEADS, KV_HEADS,
                                    HEAD_DIM, round_query_f16=tokens >= 64)
    y_ref = oracle.sigmoid_gate_mul(attn, gate)

    np.testing.assert_allclose(y, y_ref, rtol=2e-3, atol=1e-3)
    rows = slice(off, off + tokens * KV_DIM)
    assert _f16_ulp_close(kc1[rows], kc[rows])
    np.testing.assert_array_equal(vc1, vc)
    np.testing.assert_array_equal(np.delete(kc1, rows), np.delete(kc0, rows))
