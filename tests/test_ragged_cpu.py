"""CPU checks of the ragged multi-sequence decode entry points (validation-only
context): argument checks, codes and messages.  The per-sequence semantics are
the single-sequence ops' (attention_f32_batched_f16_kv with tokens = 1,
mps_backend.mm:2943-3008; gated_delta_net_f32_batched_in_place_at with
tokens = 1, mps_backend.mm:2307-2374; the fused conv prologue), checked on the
GPU in test_gpu_ragged.py."""
import pytest

import kraken_hip as kh

ACCEPTED = "validation-only context: arguments accepted"


@pytest.fixture()
def vctx():
    ctx = kh.Context(validation_only=True)
    yield ctx
    ctx.close()


def fake(nbytes, addr=0x10000):
    return kh.KrakenBuffer(addr, nbytes)


def none():
    return kh.KrakenBuffer(None, 0)


B, HQ, HKV, D = 4, 8, 2, 256


def attn_args(**over):
    a = dict(query=fake(4 * B * HQ * D), key_pool=fake(2 * 4096 * HKV * D),
             value_pool=fake(2 * 4096 * HKV * D), gate=none(), offsets=fake(8 * B),
             positions=fake(4 * B), sequences=B, max_position=2000, heads=HQ, kv_heads=HKV,
             head_dim=D, output=fake(4 * B * HQ * D))
    a.update(over)
    return [a[k] for k in ("query", "key_pool", "value_pool", "gate", "offsets", "positions",
                           "sequences", "max_position", "heads", "kv_heads", "head_dim",
                           "output")]


def run(ctx, name, args):
    return ctx.status(name, *args), kh.last_error()


def test_ragged_attention_accepts_valid_arguments(vctx):
    assert run(vctx, "attention_f32_ragged_f16_kv", attn_args()) == (kh.UNAVAILABLE, ACCEPTED)
    gated = attn_args(gate=fake(4 * B * HQ * D))
    assert run(vctx, "attention_f32_ragged_f16_kv", gated) == (kh.UNAVAILABLE, ACCEPTED)


@pytest.mark.parametrize("over,message", [
    (dict(sequences=0), "dimensions must be positive"),
    (dict(kv_heads=3), "heads must be divisible by kv_heads"),
    (dict(head_dim=96, query=fake(4 * B * HQ * 96), output=fake(4 * B * HQ * 96)),
     "supports head_dim 64/128/256"),
    (dict(heads=32, query=fake(4 * B * 32 * D), output=fake(4 * B * 32 * D)),
     "1/2/4/8 query heads per kv head"),
    (dict(query=fake(4 * B * HQ * D, addr=0x10004)), "16-byte aligned"),
    (dict(max_position=0xffffffff), "value count overflow"),
    (dict(query=fake(4 * B * HQ * D - 4)), "query buffer is too small"),
    (dict(key_pool=fake(2 * HKV * D - 2)), "key pool buffer is too small"),
    (dict(key_pool=fake(2 * 4096 * HKV * D + 1)), "not a whole number of elements"),
    (dict(value_pool=fake(2 * 4000 * HKV * D)), "key and value pools differ in size"),
    (dict(gate=fake(16)), "gate buffer is too small"),
    (dict(offsets=fake(8 * B - 8)), "kv offsets buffer is too small"),
    (dict(positions=fake(4 * B - 4)), "positions buffer is too small"),
    (dict(output=fake(16)), "output buffer is too small"),
])
def test_ragged_attention_rejects(vctx, over, message):
    code, err = run(vctx, "attention_f32_ragged_f16_kv", attn_args(**over))
    assert code == kh.INVALID_ARGUMENT
    assert message in err
    assert err.startswith("HIP")


def test_ragged_append_checks(vctx):
    good = [fake(4 * B * 512), fake(4 * B * 512), fake(2 * 1024 * 512), fake(2 * 1024 * 512),
            fake(8 * B), fake(4 * B), B, 512]
    assert run(vctx, "append_kv_ragged_f16", good) == (kh.UNAVAILABLE, ACCEPTED)
    bad = list(good)
    bad[0] = fake(4 * B * 512 - 4)
    code, err = run(vctx, "append_kv_ragged_f16", bad)
    assert code == kh.INVALID_ARGUMENT and "key rows buffer is too small" in err
    bad = list(good)
    bad[7] = 0
    code, err = run(vctx, "append_kv_ragged_f16", bad)
    assert code == kh.INVALID_ARGUMENT and "dimensions must be positive" in err


def test_ragged_gdn_checks(vctx):
    hk = hv = 16
    dd = 128
    good = [fake(4 * B * hk * dd), fake(4 * B * hk * dd), fake(4 * B * hv * dd),
            fake(4 * B * hv), fake(4 * B * hv), fake(4 * 3 * hv * dd * dd), fake(8 * B),
            B, hk, hv, dd, fake(4 * B * hv * dd)]
    assert run(vctx, "gated_delta_net_f32_ragged_decode", good) == (kh.UNAVAILABLE, ACCEPTED)
    bad = list(good)
    bad[5] = fake(4 * hv * dd * dd - 4)
    code, err = run(vctx, "gated_delta_net_f32_ragged_decode", bad)
    assert code == kh.INVALID_ARGUMENT and "state pool buffer is too small" in err
    bad = list(good)
    bad[9] = 24
    code, err = run(vctx, "gated_delta_net_f32_ragged_decode", bad)
    assert code == kh.INVALID_ARGUMENT and "value heads must repeat key heads" in err


def test_ragged_conv_checks(vctx):
    hk = hv = 16
    dd = 128
    k = 4
    ch = (2 * hk + hv) * dd
    good = [fake(4 * B * ch), fake(4 * 3 * ch * (k - 1)), fake(8 * B), fake(4 * ch * k), k, B,
            hk, hv, dd, 1e-6, fake(4 * B * hk * dd), fake(4 * B * hk * dd),
            fake(4 * B * hv * dd)]
    assert run(vctx, "qwen35_conv_split_l2_ragged_decode_f32", good) == (kh.UNAVAILABLE,
                                                                         ACCEPTED)
    bad = list(good)
    bad[4] = 9
    code, err = run(vctx, "qwen35_conv_split_l2_ragged_decode_f32", bad)
    assert code == kh.INVALID_ARGUMENT and "conv_kernel must be in [2, 8]" in err
    bad = list(good)
    bad[1] = fake(4 * ch * (k - 1) - 4)
    code, err = run(vctx, "qwen35_conv_split_l2_ragged_decode_f32", bad)
    assert code == kh.INVALID_ARGUMENT and "conv pool buffer is too small" in err
