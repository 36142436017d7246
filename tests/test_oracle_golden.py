"""The CPU oracle against the reference smoke test's known answers.

Each case is transcribed from the reference's tests/smoke_test.cpp (the
citation travels with the case); passing here is what pins the oracle before
it is used to judge the HIP kernels.
"""
import numpy as np
import pytest

import oracle
from golden_cases import check_case, load_cases

CASES = load_cases()


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_oracle_matches_smoke_known_answer(case):
    check_case(oracle, case)


def test_planted_mistake_in_oracle_is_caught():
    """A dropped term (beta ignored) in a GDN restatement must fail the fixture."""
    case = next(c for c in CASES if c["name"] == "gdn_batched_two_tokens")

    class Broken:
        @staticmethod
        def gated_delta_net(q, k, v, g, b, s, *args):
            return oracle.gated_delta_net(q, k, v, g, np.ones_like(np.asarray(b)), s, *args)

    with pytest.raises(AssertionError):
        check_case(Broken, case)
