"""CPU tests of the C ABI: library loads, exports every declared entry point,
and enforces the reference's argument checks (order and codes) without a GPU.

Checks follow the reference host dispatchers: context validity first
(`unavailable`), then dimensions, divisibility, bounds, capacity, overflow,
buffer initialisation and size, uint32 range (`invalid_argument`), e.g.
mps_backend.mm:10625-10713 for attention.  The validation-only context runs
every check and answers `unavailable` instead of launching.
"""
import ctypes
import glob
import os
import re

import pytest

import kraken_hip as kh

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))
BOUNDARY_HEADERS = [h for h in HEADERS if not h.endswith("kraken_hip_diag.h")]
DIAG_HEADERS = [h for h in HEADERS if h.endswith("kraken_hip_diag.h")]
ACCEPTED = "validation-only context: arguments accepted"


def declared_symbols(headers=None):
    """Entry points declared in the boundary's C headers under include/ (or in
    `headers`)."""
    text = "".join(open(h).read() for h in (BOUNDARY_HEADERS if headers is None else headers))
    return sorted(set(re.findall(r"KRAKEN_API[^;]*?\b(kraken_hip_\w+)\s*\(", text, re.S)))


def exported(path):
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True,
                         check=True).stdout
    return set(re.findall(r"\b(kraken_hip_\w+)\b", out))


def test_library_exports_every_declared_symbol():
    names = declared_symbols()
    assert len(names) >= 40
    lib = kh.lib()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_no_undeclared_exports():
    """The boundary library exports exactly what its headers declare: the
    measurement probes live in their own library."""
    assert exported(kh.LIB_PATH) == set(declared_symbols())


def test_diag_library_exports_its_header():
    assert exported(kh.DIAG_LIB_PATH) == set(declared_symbols(DIAG_HEADERS))
    assert set(kh.DIAG_SIGNATURES) | {"kraken_hip_diag_last_error"} == set(
        declared_symbols(DIAG_HEADERS))


def test_python_signatures_cover_header():
    names = set(declared_symbols())
    special = {"kraken_hip_context_create", "kraken_hip_context_create_validation_only",
               "kraken_hip_context_destroy", "kraken_hip_context_stream",
               "kraken_hip_last_error", "kraken_hip_abort_graph"}
    assert names - special == set(kh.SIGNATURES)


@pytest.fixture()
def vctx():
    ctx = kh.Context(validation_only=True)
    yield ctx
    ctx.close()


def fake(nbytes):
    """A buffer view that is never dereferenced (validation-only context)."""
    return kh.KrakenBuffer(0x1000, nbytes)


def status(ctx, name, *args):
    code = ctx.status(name, *args)
    if "kraken_hip_" + name in kh.DIAG_SIGNATURES:
        return code, kh.diag_lib().kraken_hip_diag_last_error().decode()
    return code, kh.last_error()


def test_null_context_is_unavailable():
    code = kh.lib().kraken_hip_attention_f32_batched_f16_kv(
        None, fake(4), fake(4), fake(4), 0, 0, 1, 1, 1, 1, 1, fake(4))
    assert code == kh.UNAVAILABLE
    assert "not initialized" in kh.last_error()


def test_live_context_without_gpu_is_unavailable():
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU driver is present")
    with pytest.raises(kh.KrakenError) as e:
        kh.Context()
    assert e.value.code == kh.UNAVAILABLE


# ------------------------------------------------------------- attention ----

def attn_args(tokens=1, start=4096, cap=4097, heads=8, kv_heads=2, d=256, layer=0,
              q_bytes=None, kv_bytes=None, out_bytes=None, elem=2):
    qv = tokens * heads * d
    kvv = (layer + 1) * cap * kv_heads * d
    return (fake(q_bytes if q_bytes is not None else 4 * qv),
            fake(kv_bytes if kv_bytes is not None else elem * kvv),
            fake(kv_bytes if kv_bytes is not None else elem * kvv),
            layer, start, tokens, cap, heads, kv_heads, d,
            fake(out_bytes if out_bytes is not None else 4 * qv))


def test_attention_accepts_valid_decode_and_prefill(vctx):
    for kw in ({}, dict(tokens=1024, start=7168, cap=8192), dict(tokens=65, start=0, cap=65,
                                                                 heads=2, kv_heads=1)):
        code, msg = status(vctx, "attention_f32_batched_f16_kv", *attn_args(**kw))
        assert (code, msg) == (kh.UNAVAILABLE, ACCEPTED)


@pytest.mark.parametrize("kw,fragment", [
    (dict(tokens=0), "dimensions must be positive"),
    (dict(heads=0), "dimensions must be positive"),
    (dict(kv_heads=0), "dimensions must be positive"),
    (dict(d=0), "dimensions must be positive"),
    (dict(cap=0, start=0), "dimensions must be positive"),
    (dict(heads=6, kv_heads=4), "divisible by kv_heads"),
    (dict(d=512), "head_dim exceeds 256"),
    (dict(start=4097), "exceeds KV cache capacity"),
    (dict(q_bytes=4 * 8 * 256 - 4), "query buffer is too small"),
    (dict(kv_bytes=2 * 4097 * 512 - 2), "key cache buffer is too small"),
    (dict(out_bytes=16), "output buffer is too small"),
    (dict(layer=1, kv_bytes=2 * 4097 * 512), "key cache buffer is too small"),
])
def test_attention_rejects(vctx, kw, fragment):
    code, msg = status(vctx, "attention_f32_batched_f16_kv", *attn_args(**kw))
    assert code == kh.INVALID_ARGUMENT
    assert fragment in msg, msg


def test_attention_check_order_dimensions_before_buffers(vctx):
    # Zero tokens and a null query: the dimension check fires first.
    args = list(attn_args(tokens=0))
    args[0] = kh.KrakenBuffer(None, 0)
    code, msg = status(vctx, "attention_f32_batched_f16_kv", *args)
    assert code == kh.INVALID_ARGUMENT and "dimensions must be positive" in msg
    args = list(attn_args())
    args[0] = kh.KrakenBuffer(None, 1 << 20)
    code, msg = status(vctx, "attention_f32_batched_f16_kv", *args)
    assert code == kh.INVALID_ARGUMENT and "query buffer is not initialized" in msg


def test_attention_overflow_and_u32_range(vctx):
    big = 1 << 62
    code, msg = status(vctx, "attention_f32_batched_f16_kv",
                       *attn_args(tokens=1, start=0, cap=big, heads=8, kv_heads=2, d=256))
    assert code == kh.INVALID_ARGUMENT and "overflow" in msg
    # capacity beyond uint32 with buffers large enough on paper
    cap = (1 << 32) + 1
    code, msg = status(vctx, "attention_f32_batched_f16_kv",
                       *attn_args(tokens=1, start=0, cap=cap, heads=1, kv_heads=1, d=1))
    assert code == kh.INVALID_ARGUMENT and "exceeds uint32 range" in msg


def test_f32_kv_twin_validates_f32_cache_sizes(vctx):
    args = attn_args(tokens=2, start=1, cap=3, heads=1, kv_heads=1, d=2, elem=4)
    code, msg = status(vctx, "attention_f32_batched", *args)
    assert (code, msg) == (kh.UNAVAILABLE, ACCEPTED)
    args = attn_args(tokens=2, start=1, cap=3, heads=1, kv_heads=1, d=2, elem=2)
    code, msg = status(vctx, "attention_f32_batched", *args)
    assert code == kh.INVALID_ARGUMENT and "key cache buffer is too small" in msg


def test_f16_query_entry_validates_the_query_in_f16_values(vctx):
    # The query is sized in 2-byte values; every other check is the F16 KV entry's.
    args = attn_args(tokens=1024, start=7168, cap=8192, q_bytes=2 * 1024 * 8 * 256)
    code, msg = status(vctx, "attention_f16q_batched_f16_kv", *args)
    assert (code, msg) == (kh.UNAVAILABLE, ACCEPTED)
    args = attn_args(tokens=1024, start=7168, cap=8192, q_bytes=2 * 1024 * 8 * 256 - 2)
    code, msg = status(vctx, "attention_f16q_batched_f16_kv", *args)
    assert code == kh.INVALID_ARGUMENT and "F16 query F16 KV batched attention query buffer is too small" in msg
    code, msg = status(vctx, "attention_f16q_batched_f16_kv", *attn_args(start=4097, q_bytes=4096))
    assert code == kh.INVALID_ARGUMENT and "exceeds KV cache capacity" in msg


def test_gated_attention_validates_gate(vctx):
    q, k, v, *rest = attn_args()
    code, msg = status(vctx, "attention_f32_batched_f16_kv_gated", q, k, v, fake(8), *rest)
    assert code == kh.INVALID_ARGUMENT and "gate buffer is too small" in msg
    code, msg = status(vctx, "attention_f32_batched_f16_kv_gated", q, k, v, fake(4 * 2048),
                       *rest)
    assert (code, msg) == (kh.UNAVAILABLE, ACCEPTED)


# ------------------------------------------------------------------ GDN -----

def gdn_args(tokens=4, hk=16, hv=16, d=128, state_offset=0, state_values=None, **over):
    kv = tokens * hk * d
    vv = tokens * hv * d
    gv = tokens * hv
    sv = state_values if state_values is not None else state_offset + hv * d * d
    a = dict(q=fake(4 * kv), k=fake(4 * kv), v=fake(4 * vv), g=fake(4 * gv), b=fake(4 * gv),
             s=fake(4 * sv), out=fake(4 * vv))
    a.update(over)
    return (a["q"], a["k"], a["v"], a["g"], a["b"], a["s"], state_offset, tokens, hk, hv, d,
            a["out"])


def test_gdn_accepts_and_rejects(vctx):
    name = "gated_delta_net_f32_batched_in_place_at"
    assert status(vctx, name, *gdn_args()) == (kh.UNAVAILABLE, ACCEPTED)
    assert status(vctx, name, *gdn_args(state_offset=3 * 16 * 128 * 128)) == (
        kh.UNAVAILABLE, ACCEPTED)
    cases = [
        (gdn_args(tokens=0), "dimensions must be positive"),
        (gdn_args(hk=3, hv=16), "value heads must repeat key heads"),
        (gdn_args(d=384), "head_dim exceeds 256"),
        (gdn_args(q=fake(16)), "query buffer is too small"),
        (gdn_args(b=kh.KrakenBuffer(None, 0)), "beta buffer is not initialized"),
        (gdn_args(state_offset=10, state_values=16 * 128 * 128), "state buffer region is too small"),
        (gdn_args(out=fake(4)), "output buffer is too small"),
    ]
    for args, fragment in cases:
        code, msg = status(vctx, name, *args)
        assert code == kh.INVALID_ARGUMENT and fragment in msg, (fragment, msg)


def test_conv_ops_validation(vctx):
    # ssm_conv: input [S][C][K-1+T]
    assert status(vctx, "ssm_conv_f32", fake(4 * 2 * 6), fake(4 * 8), 4, 2, 3, 1,
                  fake(4 * 6)) == (kh.UNAVAILABLE, ACCEPTED)
    code, msg = status(vctx, "ssm_conv_f32", fake(4 * 2 * 5), fake(4 * 8), 4, 2, 3, 1, fake(24))
    assert code == kh.INVALID_ARGUMENT and "SSM conv input buffer is too small" in msg
    code, msg = status(vctx, "build_ssm_conv_state_f32", fake(24), 0, fake(16), 1, 2, 2, fake(40))
    assert code == kh.INVALID_ARGUMENT and "conv-state dimensions are invalid" in msg
    assert status(vctx, "build_ssm_conv_state_f32", fake(24), 0, fake(16), 4, 2, 2,
                  fake(40)) == (kh.UNAVAILABLE, ACCEPTED)
    code, msg = status(vctx, "build_ssm_conv_state_f32", fake(24), 1, fake(16), 4, 2, 2, fake(40))
    assert code == kh.INVALID_ARGUMENT and "region is too small" in msg
    code, msg = status(vctx, "qwen35_conv_split_l2_f32", fake(4 * 6144), fake(4 * 3 * 6144), 0,
                       fake(4 * 4 * 6144), 9, 1, 16, 16, 128, 1e-6, fake(8192), fake(8192),
                       fake(8192))
    assert code == kh.INVALID_ARGUMENT and "conv_kernel must be in [2, 8]" in msg
    assert status(vctx, "qwen35_conv_split_l2_f32", fake(4 * 6144), fake(4 * 3 * 6144), 0,
                  fake(4 * 4 * 6144), 4, 1, 16, 16, 128, 1e-6, fake(8192), fake(8192),
                  fake(8192)) == (kh.UNAVAILABLE, ACCEPTED)


def test_small_ops_validation(vctx):
    code, msg = status(vctx, "mrope_f32_in_place", fake(64), fake(16), 1, 1, 8, 10, 1, 1, 1, 1,
                       1e4)
    assert code == kh.INVALID_ARGUMENT and "MRoPE dimensions are invalid" in msg
    code, msg = status(vctx, "mrope_f32_in_place", fake(64), fake(16), 1, 1, 8, 8, 0, 0, 0, 0,
                       1e4)
    assert code == kh.INVALID_ARGUMENT and "sections must not all be zero" in msg
    code, msg = status(vctx, "mrope_f32_in_place", fake(64), fake(8), 1, 1, 8, 8, 1, 1, 1, 1, 1e4)
    assert code == kh.INVALID_ARGUMENT and "position buffer is too small" in msg
    code, msg = status(vctx, "copy_f32_rows", fake(48), fake(36), 3, 2, 1, 1, 3, 0)
    assert code == kh.INVALID_ARGUMENT and "stride must be at least row size" in msg
    code, msg = status(vctx, "copy_f32_rows", fake(40), fake(36), 3, 2, 4, 1, 3, 0)
    assert code == kh.INVALID_ARGUMENT and "copy rows source buffer is too small" in msg
    assert status(vctx, "copy_f32_rows", fake(48), fake(36), 3, 2, 4, 1, 3, 0) == (
        kh.UNAVAILABLE, ACCEPTED)
    code, msg = status(vctx, "copy_f32_rows_to_f16", fake(48), fake(15), 3, 2, 4, 1, 3, 0)
    assert code == kh.INVALID_ARGUMENT and "destination buffer is too small" in msg
    code, msg = status(vctx, "qk_norm_f32_f32_batched", fake(16), fake(4), 2, 1, 2, 0.0)
    assert code == kh.INVALID_ARGUMENT and "weight buffer is too small" in msg
    code, msg = status(vctx, "prepare_qwen35_gdn_gate_beta_f32", fake(16), fake(16), fake(8),
                       fake(8), 0, 2)
    assert code == kh.INVALID_ARGUMENT and "dimensions must be positive" in msg
    code, msg = status(vctx, "split_qkv_l2_norm_f32_qwen35", fake(96), fake(32), fake(32),
                       fake(31), 2, 2, 2, 2, 0.0)
    assert code == kh.INVALID_ARGUMENT and "split qkv value buffer is too small" in msg
    code, msg = status(vctx, "sigmoid_f32_in_place", fake(4), 2)
    assert code == kh.INVALID_ARGUMENT and "sigmoid values buffer is too small" in msg


def test_graph_batching_rules(vctx):
    lib = kh.lib()
    assert lib.kraken_hip_commit_graph(vctx.handle) == kh.OK  # commit without begin
    assert lib.kraken_hip_begin_graph(vctx.handle) == kh.OK
    assert lib.kraken_hip_begin_graph(vctx.handle) == kh.INVALID_ARGUMENT
    assert "already active" in kh.last_error()
    vctx.abort_graph()
    assert lib.kraken_hip_begin_graph(vctx.handle) == kh.OK
    assert lib.kraken_hip_commit_graph(vctx.handle) == kh.OK


def test_copy_rules(vctx):
    data = (ctypes.c_float * 4)()
    code, msg = status(vctx, "copy_to_buffer_at", fake(16), 8, ctypes.addressof(data), 12)
    assert code == kh.INVALID_ARGUMENT and "exceeds destination buffer size" in msg
    code, msg = status(vctx, "copy_from_buffer", fake(16), None, 4)
    assert code == kh.INVALID_ARGUMENT and "destination must not be null" in msg
    code, msg = status(vctx, "zero_buffer", fake(16), 32)
    assert code == kh.INVALID_ARGUMENT and "zero size exceeds buffer size" in msg


# ------------------------------------------------ fused attention prologue --

def prologue_args(tokens=4, start=10, cap=16, heads=8, kv_heads=2, d=256, layer=1, n_dims=64,
                  sections=(11, 11, 10, 0), positions=True, **sizes):
    qv = tokens * heads * d
    kvv = tokens * kv_heads * d
    cache = (layer + 1) * cap * kv_heads * d

    def b(name, n):
        return fake(sizes.get(name, n))

    pos = b("pos", 4 * 4 * tokens) if positions else kh.KrakenBuffer(None, 0)
    return (b("qg", 4 * 2 * qv), b("k", 4 * kvv), b("v", 4 * kvv), b("qn", 4 * d),
            b("kn", 4 * d), pos, start, b("kc", 2 * cache), b("vc", 2 * cache), layer, start,
            tokens, cap, heads, kv_heads, d, n_dims, *sections, 1e7, 1e-6, b("qo", 4 * qv),
            b("go", 4 * qv))


def test_prologue_accepts_valid(vctx):
    for kw in ({}, dict(positions=False), dict(tokens=1, start=15), dict(d=128, n_dims=128,
                                                                         heads=4, kv_heads=4)):
        code, msg = status(vctx, "qwen35_attention_prologue_f16_kv", *prologue_args(**kw))
        assert (code, msg) == (kh.UNAVAILABLE, ACCEPTED), kw


@pytest.mark.parametrize("kw,fragment", [
    (dict(tokens=0), "dimensions must be positive"),
    (dict(heads=6, kv_heads=4), "divisible by kv_heads"),
    (dict(d=512, n_dims=64), "head_dim exceeds 256"),
    (dict(n_dims=63), "MRoPE dimensions are invalid"),
    (dict(n_dims=258), "MRoPE dimensions are invalid"),
    (dict(sections=(0, 0, 0, 0)), "sections must not all be zero"),
    (dict(start=13), "exceeds KV cache capacity"),
    (dict(qg=4 * 2 * 4 * 8 * 256 - 4), "q_gate buffer is too small"),
    (dict(kc=2 * 2 * 16 * 512 - 2), "key cache buffer is too small"),
    (dict(pos=4 * 4 * 4 - 4), "positions buffer is too small"),
    (dict(go=16), "gate output buffer is too small"),
])
def test_prologue_rejects(vctx, kw, fragment):
    code, msg = status(vctx, "qwen35_attention_prologue_f16_kv", *prologue_args(**kw))
    assert code == kh.INVALID_ARGUMENT
    assert fragment in msg, msg


def test_prologue_generated_positions_must_fit_int32(vctx):
    args = list(prologue_args(positions=False))
    args[6] = (1 << 31) - 2  # mrope_start_position: the last of 4 tokens exceeds int32
    code, msg = status(vctx, "qwen35_attention_prologue_f16_kv", *args)
    assert code == kh.INVALID_ARGUMENT and "exceeds int32 range" in msg


def test_prologue_gated_accepts_valid(vctx):
    """The one-launch prologue + gated attention entry takes the prologue's
    arguments and an output [tokens][heads][head_dim]."""
    for kw in ({}, dict(tokens=1, start=15), dict(tokens=1, start=255, cap=300),
               dict(d=128, n_dims=128, heads=4, kv_heads=4)):
        tokens, heads, d = kw.get("tokens", 4), kw.get("heads", 8), kw.get("d", 256)
        args = prologue_args(**kw) + (fake(4 * tokens * heads * d),)
        code, msg = status(vctx, "qwen35_attention_prologue_gated_f16_kv", *args)
        assert (code, msg) == (kh.UNAVAILABLE, ACCEPTED), kw


def test_prologue_gated_rejects(vctx):
    args = prologue_args(tokens=1, start=3) + (fake(4 * 8 * 256 - 4),)
    code, msg = status(vctx, "qwen35_attention_prologue_gated_f16_kv", *args)
    assert code == kh.INVALID_ARGUMENT and "attention prologue output buffer is too small" in msg
    args = prologue_args(tokens=1, start=3, n_dims=63) + (fake(4 * 8 * 256),)
    code, msg = status(vctx, "qwen35_attention_prologue_gated_f16_kv", *args)
    assert code == kh.INVALID_ARGUMENT and "MRoPE dimensions are invalid" in msg


# ------------------------------------------------ fused ragged GDN layer --

def gdn_layer_args(b=4, hk=16, hv=16, d=128, k=4, prepare=True, **sizes):
    ch = (2 * hk + hv) * d

    def buf(name, n):
        return fake(sizes.get(name, n))

    dtb = buf("dtb", 4 * hv) if prepare else kh.KrakenBuffer(None, 0)
    ssa = buf("ssa", 4 * hv) if prepare else kh.KrakenBuffer(None, 0)
    return (buf("qkv", 4 * b * ch), buf("cp", 4 * ch * (k - 1)), buf("co", 8 * b),
            buf("w", 4 * ch * k), k, buf("g", 4 * b * hv), buf("beta", 4 * b * hv), dtb, ssa,
            buf("z", 4 * b * hv * d), buf("nw", 4 * d), buf("sp", 4 * hv * d * d),
            buf("so", 8 * b), b, hk, hv, d, 1e-6, buf("out", 4 * b * hv * d))


def test_gdn_layer_accepts_valid(vctx):
    for kw in ({}, dict(prepare=False), dict(hk=2, hv=4, d=64, k=3)):
        code, msg = status(vctx, "qwen35_gdn_layer_ragged_decode_f32", *gdn_layer_args(**kw))
        assert (code, msg) == (kh.UNAVAILABLE, ACCEPTED), kw


@pytest.mark.parametrize("kw,fragment", [
    (dict(b=0), "dimensions must be positive"),
    (dict(hk=3, hv=4), "value heads must repeat key heads"),
    (dict(k=1), "conv_kernel must be in [2, 8]"),
    (dict(d=512), "head_dim exceeds 256"),
    (dict(qkv=16), "qkv buffer is too small"),
    (dict(cp=16), "conv pool buffer is too small"),
    (dict(sp=16), "state pool buffer is too small"),
    (dict(z=16), "z buffer is too small"),
    (dict(out=16), "output buffer is too small"),
])
def test_gdn_layer_rejects(vctx, kw, fragment):
    code, msg = status(vctx, "qwen35_gdn_layer_ragged_decode_f32", *gdn_layer_args(**kw))
    assert code == kh.INVALID_ARGUMENT
    assert fragment in msg, msg


def test_gdn_layer_dt_bias_and_ssm_a_together(vctx):
    args = list(gdn_layer_args())
    args[8] = kh.KrakenBuffer(None, 0)  # ssm_a missing, dt_bias given
    code, msg = status(vctx, "qwen35_gdn_layer_ragged_decode_f32", *args)
    assert code == kh.INVALID_ARGUMENT and "given together" in msg


def test_diag_probe_argument_checks(vctx):
    """The measurement aids (include/kraken_hip_diag.h, their own library) check
    sizes and alignment, and answer a validation-only context like the boundary."""
    sink = fake(256 * 256 * 4)
    assert status(vctx, "diag_stream_read", fake(1 << 20), 1 << 20, sink) == (kh.UNAVAILABLE,
                                                                             ACCEPTED)
    code, _ = status(vctx, "diag_stream_read", fake(1 << 20), 1000, sink)  # not a multiple of 16
    assert code == kh.INVALID_ARGUMENT
    code, _ = status(vctx, "diag_stream_read", fake(1 << 10), 1 << 20, sink)  # source too small
    assert code == kh.INVALID_ARGUMENT
    code, _ = status(vctx, "diag_stream_read", fake(1 << 20), 1 << 20, fake(16))  # sink too small
    assert code == kh.INVALID_ARGUMENT
    assert status(vctx, "diag_mfma_f16", 256, 10, sink) == (kh.UNAVAILABLE, ACCEPTED)
    code, _ = status(vctx, "diag_mfma_f16", 257, 10, sink)  # sink holds 256 workgroups
    assert code == kh.INVALID_ARGUMENT
    code, _ = status(vctx, "diag_mfma_f16", 256, 0, sink)
    assert code == kh.INVALID_ARGUMENT
    assert status(vctx, "diag_mfma_f16_denormals", fake(48)) == (kh.UNAVAILABLE, ACCEPTED)
    code, _ = status(vctx, "diag_mfma_f16_denormals", fake(44))  # holds 11 of the 12 results
    assert code == kh.INVALID_ARGUMENT


class _Region(ctypes.Structure):
    _fields_ = [("source_offset", ctypes.c_size_t), ("destination_offset", ctypes.c_size_t),
                ("byte_size", ctypes.c_size_t)]


def test_copy_regions_argument_checks(vctx):
    """kraken_hip_copy_regions bounds every range by its buffers and caps the count."""
    src, dst = fake(4096), fake(2048)
    ok = (_Region * 2)((0, 0, 1024), (1024, 1024, 1024))
    assert status(vctx, "copy_regions", src, dst, ctypes.addressof(ok), 2) == (kh.UNAVAILABLE,
                                                                              ACCEPTED)
    for bad in [(4000, 0, 200), (0, 1900, 200), (0, 0, 1 << 62)]:
        r = (_Region * 1)(bad)
        code, _ = status(vctx, "copy_regions", src, dst, ctypes.addressof(r), 1)
        assert code == kh.INVALID_ARGUMENT, bad
    many = (_Region * 65)()
    code, _ = status(vctx, "copy_regions", src, dst, ctypes.addressof(many), 65)
    assert code == kh.INVALID_ARGUMENT


def test_no_alloc_attention_limits_its_scratch(vctx):
    """The allocation-free attention accepts what fits its static 8 MiB array
    (decode at long KV) and rejects, before launching, a prefill whose split
    partials would not fit."""
    h, kvh, d = 8, 2, 256
    for tokens, start, ok in ((1, 262143, True), (64, 0, True), (1024, 7168, False)):
        cap = start + tokens
        q, kv = fake(4 * tokens * h * d), fake(2 * cap * kvh * d)
        code, msg = status(vctx, "attention_f32_batched_f16_kv_gated_no_alloc", q, kv, kv, q,
                           0, start, tokens, cap, h, kvh, d, q)
        if ok:
            assert (code, msg) == (kh.UNAVAILABLE, ACCEPTED)
        else:
            assert code == kh.INVALID_ARGUMENT
            assert msg == ("HIP gated F16 KV batched attention needs 17039360 bytes of split "
                           "partials; the allocation-free entry point has 8388608")


# ------------------------------------------- three-launch GDN decode layer ----

def _multi_conv_args(rows0=6144, conv_kernel=4, pool_bytes=None, kernel_bytes=None,
                     offset_bytes=8, norm=True):
    types = (ctypes.c_uint32 * 1)(13)
    rows = (ctypes.c_size_t * 1)(rows0)
    ws = (kh.KrakenBuffer * 1)(fake(rows0 * 4 * 176))
    outs = (kh.KrakenBuffer * 1)(fake(4 * rows0))
    return (1, types, ws, rows, 1024, fake(4096),
            fake(4096) if norm else kh.KrakenBuffer(None, 0), 1e-6, outs,
            fake(pool_bytes if pool_bytes is not None else 4 * 3 * rows0), fake(offset_bytes),
            fake(kernel_bytes if kernel_bytes is not None else 16 * rows0), conv_kernel)


@pytest.mark.parametrize("kw,fragment", [
    (dict(), None),
    (dict(conv_kernel=3), "conv_kernel must be 4"),
    (dict(pool_bytes=4 * 3 * 6144 - 4), "conv pool buffer is too small"),
    (dict(kernel_bytes=16 * 6144 - 4), "conv kernel buffer is too small"),
    (dict(offset_bytes=4), "conv offset buffer is too small"),
    (dict(norm=False), "needs a norm weight"),
])
def test_multi_conv_matvec_checks(vctx, kw, fragment):
    code, msg = status(vctx, "kquant_matvec_multi_conv_f32", *_multi_conv_args(**kw))
    if fragment is None:
        assert (code, msg) == (kh.UNAVAILABLE, ACCEPTED)
    else:
        assert code == kh.INVALID_ARGUMENT and fragment in msg, msg


@pytest.mark.parametrize("kw,fragment", [
    (dict(), None),
    (dict(head_dim=64), "head_dim must be 128"),
    (dict(gf=fake(4 * 2048 - 4)), "gate factor buffer is too small"),
])
def test_head_norm_matvec_checks(vctx, kw, fragment):
    a = dict(gf=fake(4 * 2048), head_dim=128)
    a.update(kw)
    code, msg = status(vctx, "kquant_matvec_head_norm_f32", 12, fake(1024 * 8 * 144), 1024, 2048,
                       fake(4 * 2048), a["gf"], a["head_dim"], 1e-6, kh.KrakenBuffer(None, 0),
                       fake(4 * 1024))
    if fragment is None:
        assert (code, msg) == (kh.UNAVAILABLE, ACCEPTED)
    else:
        assert code == kh.INVALID_ARGUMENT and fragment in msg, msg


@pytest.mark.parametrize("kw,fragment", [
    (dict(), None),
    (dict(head_dim=64), "needs head_dim 128"),
    (dict(key_heads=8), "needs head_dim 128 and key_heads == value_heads"),
    (dict(ssa=kh.KrakenBuffer(None, 0)), "dt_bias and ssm_a must be given together"),
    (dict(state=fake(4 * 16 * 128 * 128 - 4)), "state pool buffer is too small"),
    (dict(qkv=fake(4 * 6144 - 4)), "qkv buffer is too small"),
    (dict(z=fake(4 * 2048 - 4)), "z buffer is too small"),
    (dict(gout=fake(4 * 2048 - 4)), "gate output buffer is too small"),
])
def test_gdn_state_decode_checks(vctx, kw, fragment):
    a = dict(qkv=fake(4 * 6144), ssa=fake(64), state=fake(4 * 16 * 128 * 128), head_dim=128,
             key_heads=16, z=fake(4 * 2048), gout=fake(4 * 2048))
    a.update(kw)
    code, msg = status(vctx, "qwen35_gdn_state_ragged_decode_f32", a["qkv"], fake(64), fake(64),
                       fake(64), a["ssa"], a["z"], fake(512), a["state"], fake(8), 1,
                       a["key_heads"], 16, a["head_dim"], 1e-6, fake(4 * 2048), a["gout"])
    if fragment is None:
        assert (code, msg) == (kh.UNAVAILABLE, ACCEPTED)
    else:
        assert code == kh.INVALID_ARGUMENT and fragment in msg, msg
