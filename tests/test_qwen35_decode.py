"""GGUF loading and the greedy decode loop on the 0.8B plan.

CPU: the GGUF reader (include/kraken/gguf.hpp, through `qwen35_driver_check
gguf-info`) on files written byte by byte by tests/gguf_writer.py: header,
metadata of every value kind, tensor table, alignment padding, tensor bytes
through the mapping, and the reference reader's rejections (bad magic,
version, rank, unknown type, truncation, ranges past the end).

GPU: `qwen35_driver_check decode` loads a synthetic Qwen3.5-0.8B GGUF
(tests/qwen35_decode_cases.py), runs the device decode loop (one graph batch
and one host wait per token, the next token kept on the device) and must
produce the oracle chain's tokens step by step.  A step may pick a different
token only where the oracle's two logits are within 5e-3 of each other (then
the oracle continues from the device's token).  The run with the reference's
separate ops must give the same tokens and a last-step LM-head input within
5e-3 of the oracle's; runs of both op orders that read the hidden state back
after every layer must match the oracle layer by layer, step by step (1e-3 of
the state's magnitude).
"""
import os
import struct
import subprocess

import numpy as np
import pytest

import gguf_writer as gw

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "kraken-infer_amd", "build", "qwen35_driver_check")


def run(*args, timeout=120):
    return subprocess.run([BIN, *map(str, args)], capture_output=True, text=True,
                          timeout=timeout)


def info(path):
    r = run("gguf-info", path)
    return r.returncode, r.stdout


def small_file(path, **kw):
    rng = np.random.default_rng(5)
    a = rng.integers(0, 256, 144 * 3, dtype=np.uint8)
    b = rng.standard_normal(7).astype(np.float32)
    meta = [("general.architecture", gw.STRING, "qwen35"),
            ("qwen35.block_count", gw.U32, 24),
            ("k.i8", gw.I8, -5), ("k.u16", gw.U16, 65535), ("k.i64", gw.I64, -(2 ** 40)),
            ("k.f64", gw.F64, 2.5), ("k.bool", gw.BOOL, True),
            ("k.arr", gw.ARRAY, [3, -4, 5], gw.I32),
            ("k.strs", gw.ARRAY, ["ab", "c"], gw.STRING)]
    meta += kw.get("extra_meta", [])
    tensors = [("blk.0.a", (256, 3), gw.GGML_Q4_K, a), ("b", (7,), gw.GGML_F32, b),
               ("c", (2, 3), gw.GGML_F32, b[:6].reshape(3, 2))]
    offsets = gw.write(path, meta, tensors, alignment=kw.get("alignment", 32))
    return a, b, offsets


def test_gguf_reader_parses_writer_output(tmp_path):
    p = tmp_path / "m.gguf"
    a, b, offsets = small_file(p, alignment=64,
                               extra_meta=[("general.alignment", gw.U32, 64)])
    code, out = info(p)
    assert code == 0, out
    lines = out.splitlines()
    assert lines[0].startswith("version=3 tensors=3 metadata=10 alignment=64")
    data_offset = int(lines[0].split("data_offset=")[1])
    assert data_offset % 64 == 0 and data_offset == offsets[0]
    assert (f"tensor blk.0.a type=12 shape=256,3 offset=0 abs={offsets[0]} bytes=432 "
            f"sum={int(a.sum())}") in lines
    assert (f"tensor b type=0 shape=7 offset=448 abs={offsets[1]} bytes=28 "
            f"sum={int(b.view(np.uint8).sum())}") in lines
    # A tensor after an f32 one starts at the next aligned byte past its 28 bytes.
    assert (f"tensor c type=0 shape=2,3 offset=512 abs={offsets[2]} bytes=24 "
            f"sum={int(b[:6].view(np.uint8).sum())}") in lines
    assert "meta general.architecture kind=8 qwen35" in lines
    assert "meta qwen35.block_count kind=4 24" in lines
    assert "meta k.i8 kind=1 -5" in lines
    assert "meta k.u16 kind=2 65535" in lines
    assert f"meta k.i64 kind=11 {-(2 ** 40)}" in lines
    assert "meta k.f64 kind=12 2.500000" in lines
    assert "meta k.bool kind=7 true" in lines
    assert "meta k.arr kind=9 array[3] first=3" in lines
    assert "meta k.strs kind=9 array[2] first=ab" in lines


def test_gguf_reader_rejections(tmp_path):
    p = tmp_path / "m.gguf"
    small_file(p)
    good = open(p, "rb").read()

    def case(mutate, message):
        q = tmp_path / "bad.gguf"
        open(q, "wb").write(mutate(bytearray(good)))
        code, out = info(q)
        assert code == 1 and out.startswith("error ") and message in out, out

    case(lambda d: b"GGUX" + d[4:], "not a GGUF file")
    case(lambda d: d[:4] + struct.pack("<I", 4) + d[8:], "unsupported GGUF version: 4")
    case(lambda d: d[:200], "unexpected end of GGUF file at byte")
    # The first metadata value type (after the key) set to 13.
    key_len = struct.unpack_from("<Q", good, 24)[0]
    case(lambda d: d[:32 + key_len] + struct.pack("<I", 13) + d[36 + key_len:],
         "unsupported GGUF metadata value type: 13")
    # Tensor table: find the first tensor's name and corrupt its rank / type.
    at = good.index(b"blk.0.a") + len(b"blk.0.a")
    case(lambda d: d[:at] + struct.pack("<I", 0) + d[at + 4:], "invalid GGUF tensor rank for blk.0.a")
    case(lambda d: d[:at + 20] + struct.pack("<I", 4) + d[at + 24:],
         "unsupported GGML tensor type: 4")
    case(lambda d: d[:at + 24] + struct.pack("<Q", 1 << 40) + d[at + 32:],
         "GGUF tensor offset exceeds file size: blk.0.a")
    case(lambda d: d[:len(good) - 8], "GGUF tensor byte range exceeds file size: c")
    # 255 values of Q4_K are not a whole block.
    case(lambda d: d[:at + 4] + struct.pack("<Q", 255) + d[at + 12:],
         "GGUF tensor element count is not divisible by block size: blk.0.a")


@pytest.mark.gpu
def test_greedy_decode_matches_oracle_chain(tmp_path):
    import qwen35_decode_cases as qc

    steps, first = 6, 11
    model = qc.build_model()
    path = tmp_path / "qwen35-0.8b-synthetic.gguf"
    qc.write_gguf(path, model)
    print(f"decode: GGUF written ({os.path.getsize(path) >> 20} MiB)", flush=True)
    # The fused op order (the default), plain: one batch and one wait per token.
    r = run("decode", path, tmp_path, first, steps, timeout=300)
    print(r.stdout[-2000:], flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    got = np.fromfile(tmp_path / "tokens.i32", np.int32)
    assert got.size == steps
    dec = qc.OracleDecoder(model, steps + 1)
    token, switched, ref_normed = first, 0, None
    for i in range(steps):
        want, logits, ref_normed = dec.step(token, i)
        if got[i] != want:
            gap = abs(float(logits[got[i]]) - float(logits[want]))
            assert gap <= 5e-3 * max(1.0, abs(float(logits[want]))), (i, got[i], want, gap)
            switched += 1
        print(f"step {i}: device {got[i]} oracle {want}", flush=True)
        token = int(got[i])
    assert switched <= 1
    # The reference's separate ops: the same tokens, and the last step's LM-head
    # input against the oracle's.
    r = run("decode", path, tmp_path, first, steps, "reference", timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert np.array_equal(np.fromfile(tmp_path / "tokens.i32", np.int32), got)
    normed = np.fromfile(tmp_path / "normed.f32", np.float32)
    np.testing.assert_allclose(normed, ref_normed, rtol=5e-3, atol=5e-3)
    # Both orders with the hidden state read back after every layer: each of the
    # 6 x 24 layer outputs against the oracle's (fed the device's tokens), within
    # 1e-3 of the state's largest magnitude.
    for order in ("fused", "reference"):
        args = ["trace"] + (["reference"] if order == "reference" else [])
        r = run("decode", path, tmp_path, first, steps, *args, timeout=300)
        assert r.returncode == 0, r.stdout + r.stderr
        assert np.array_equal(np.fromfile(tmp_path / "tokens.i32", np.int32), got)
        trace = np.fromfile(tmp_path / "hidden_trace.f32", np.float32).reshape(steps, qc.LAYERS,
                                                                                 -1)
        dec = qc.OracleDecoder(model, steps + 1)
        token, worst = first, 0.0
        for i in range(steps):
            ref = []
            dec.step(token, i, ref)
            for layer, want in enumerate(ref):
                err = float(np.abs(trace[i, layer] - want).max()) / max(
                    1.0, float(np.abs(want).max()))
                worst = max(worst, err)
                assert err <= 1e-3, (order, i, layer, err)
            token = int(got[i])
        print(f"{order}: worst per-layer relative error {worst:.2e}", flush=True)


@pytest.mark.gpu
@pytest.mark.timeout(900)
def test_chunked_prefill_then_decode_matches_oracle_chain(tmp_path):
    """`qwen35_driver_check prefill`: a 1500-token prompt through the whole model in
    chunks of 1024 (the second one ragged, 476 tokens) with the layer cores on
    flash256 and the chunked gated delta rule and the projections on the K-quant
    GEMM, one graph commit per chunk (qwen35_runtime.cpp:5787-6004); then 5 greedy
    decode steps from position 1500 over the filled caches.  Against the oracle's
    chunked prompt pass (tests/qwen35_decode_cases.py prefill_chunk): every
    layer's hidden rows 0, T/2 and T-1 of both chunks, and every layer of every
    decode step, within 1e-3 of the state's largest magnitude; the tokens under
    the decode test's rule (a different token only where the oracle's two logits
    are within 5e-3, and then the oracle continues from the device's token)."""
    import qwen35_decode_cases as qc

    prompt, chunk, steps = 1500, 1024, 6
    model = qc.build_model()
    path = tmp_path / "qwen35-0.8b-synthetic.gguf"
    qc.write_gguf(path, model)
    print("prefill: GGUF written", flush=True)
    r = run("prefill", path, tmp_path, prompt, chunk, steps, "trace", timeout=600)
    print(r.stdout[-1000:], flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    ids = np.fromfile(tmp_path / "prompt.i32", np.int32)
    got = np.fromfile(tmp_path / "tokens.i32", np.int32)
    assert ids.size == prompt and got.size == steps
    assert np.array_equal(ids, (7919 * np.arange(prompt, dtype=np.int64) + 11) % qc.VOCAB)
    chunks = [(0, chunk), (chunk, prompt - chunk)]
    trace = np.fromfile(tmp_path / "prefill_trace.f32", np.float32).reshape(
        len(chunks), qc.LAYERS, 3, qc.HIDDEN)
    dec = qc.OracleDecoder(model, prompt + steps)
    worst = 0.0
    for c, (start, t) in enumerate(chunks):
        ref = []
        h = dec.prefill_chunk(ids[start:start + t].tolist(), start, ref)
        for layer, want in enumerate(ref):
            err = float(np.abs(trace[c, layer] - want).max()) / max(1.0, float(np.abs(want).max()))
            worst = max(worst, err)
            assert err <= 1e-3, ("prefill", c, layer, err)
        print(f"prefill chunk {c} ({t} tokens) matches, worst so far {worst:.2e}", flush=True)

    def agree(i, device, want, logits):
        if device != want:
            gap = abs(float(logits[device]) - float(logits[want]))
            assert gap <= 5e-3 * max(1.0, abs(float(logits[want]))), (i, device, want, gap)
            return 1
        return 0

    want, logits = dec.lm_head(h[-1])
    switched = agree(0, int(got[0]), want, logits)
    steps_trace = np.fromfile(tmp_path / "hidden_trace.f32", np.float32).reshape(
        steps - 1, qc.LAYERS, qc.HIDDEN)
    for i in range(steps - 1):
        ref = []
        want, logits, _ = dec.step(int(got[i]), prompt + i, ref)
        for layer, row in enumerate(ref):
            err = float(np.abs(steps_trace[i, layer] - row).max()) / max(1.0,
                                                                         float(np.abs(row).max()))
            worst = max(worst, err)
            assert err <= 1e-3, ("decode", i, layer, err)
        switched += agree(i + 1, int(got[i + 1]), want, logits)
        print(f"decode step {i}: device {got[i + 1]} oracle {want}", flush=True)
    assert switched <= 1
    print(f"prefill + decode: worst per-layer relative error {worst:.2e}", flush=True)
