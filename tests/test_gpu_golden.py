"""HIP kernels against the reference smoke test's known answers (GPU).

The same transcribed cases that pin the CPU oracle (test_oracle_golden.py) run
here through the C ABI.  Tolerance: the reference test's own (1e-5 absolute,
5e-5 for the head_dim-128 GDN case).
"""
import pytest

import kraken_hip as kh
from golden_cases import check_case, load_cases

CASES = load_cases()


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_hip_matches_smoke_known_answer(hip_ctx, case):
    print(f"golden case {case['name']}", flush=True)
    check_case(kh.NumpyOps(hip_ctx), case)
