"""The committed golden fixtures (tests/golden/*.npz) against the oracle that wrote them, and
against the reference's recorded known answers where one applies."""
import os

import numpy as np
import pytest

from tests.golden import make_golden

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz")) as z:   # allow_pickle stays False
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name", sorted(make_golden.CASES))
def test_fixture_regenerates_bit_for_bit(name):
    stored = load(name)
    fresh = make_golden.CASES[name]()
    assert sorted(stored) == sorted(fresh)
    for k, v in fresh.items():
        np.testing.assert_array_equal(stored[k], np.asarray(v), err_msg=k)


def test_ref_case_matches_reference_recorded_errors(oracle):
    """GEMV rows 0..7: the reference's recorded M=8 max-rel-err of its fp32 GEMV is 1.1e-07
    (results/ncu/w4_gemv_m8.txt:8); the bf16-staged result lies within a bf16 ulp scale of exact."""
    c = load("ref_case")
    y = oracle.gemv_ref_order(c["X"], c["Wq"], c["S"], int(c["G"]))
    assert f"{oracle.max_rel_err(y, c['y_exact']):.1e}" == "1.1e-07"
    assert oracle.max_rel_err(c["y_staged"], c["y_exact"]) < 5e-3
