"""GPU checks of the measurement aids (include/kraken_hip_diag.h) that bench.py uses for
the box's achievable rates: the streaming read visits every 16-byte chunk exactly once
(the per-lane sums add up to the buffer's sum, including a tail that is not a multiple of
the 8-deep unrolled stride), and the MFMA loop writes finite per-lane sums."""
import numpy as np
import pytest

import kraken_hip as kh  # noqa: F401  (fixtures come from conftest)


@pytest.mark.gpu
@pytest.mark.parametrize("floats", [4, 4 * 65536 * 8 + 4 * 3, 1 << 22])
def test_stream_read_probe_reads_every_chunk(hip_ctx, floats):
    print(f"diag stream read {floats}", flush=True)
    rng = np.random.default_rng(floats)
    x = rng.integers(-4, 5, size=floats).astype(np.float32)  # small integers: exact sums
    src = hip_ctx.buffer(x)
    sink = hip_ctx.buffer(byte_size=256 * 256 * 4)
    hip_ctx.diag_stream_read(src, floats * 4, sink)
    got = sink.download(256 * 256).astype(np.float64).sum()
    assert got == float(x.astype(np.float64).sum())


@pytest.mark.gpu
def test_mfma_probe_runs(hip_ctx):
    print("diag mfma", flush=True)
    sink = hip_ctx.buffer(byte_size=8 * 256 * 4)
    hip_ctx.diag_mfma_f16(8, 10, sink)
    assert np.isfinite(sink.download(8 * 256)).all()


@pytest.mark.gpu
def test_mfma_f16_denormal_operands_recorded(hip_ctx, record_property):
    """Records whether v_mfma_f32_16x16x32_f16 and v_mfma_f32_16x16x16_f16 keep an
    f16 denormal operand (2^-15, 2^-24) in A and in B; the smallest normal (2^-14)
    must pass through exactly.  The decode and GDN kernels keep their split lo
    halves normal (2^11 scale) so that their results do not depend on the answer."""
    sink = hip_ctx.buffer(byte_size=12 * 4)
    hip_ctx.diag_mfma_f16_denormals(sink)
    got = sink.download(12).reshape(3, 2, 2)
    values = (2.0 ** -15, 2.0 ** -24, 2.0 ** -14)
    for v, x in enumerate(values):
        for i, ins in enumerate(("16x16x32_f16", "16x16x16f16")):
            for o, operand in enumerate("AB"):
                r = float(got[v, i, o])
                what = "kept" if r == x else "flushed" if r == 0.0 else f"{r!r}"
                print(f"v_mfma_f32_{ins} operand {operand} x=2^{int(np.log2(x))}: {what}",
                      flush=True)
                record_property(f"{ins}_{operand}_2^{int(np.log2(x))}", what)
                assert r == x or r == 0.0
    assert np.all(got[2] == values[2])
