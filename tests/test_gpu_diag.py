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
