"""The attention parity check must reject badly wrong outputs.

Built from committed golden fixtures (oracle outputs), on the CPU: an
all-zero output and a half-size output fail `assert_close`, also when the
outputs are as small as they are at long contexts (N(0,1) inputs shrink the
output roughly as sqrt(e/ctx): ~0.01 at 40k tokens), where the per-element
bound alone would accept both.  A correct output rounded to bf16 passes.
"""
import os

import numpy as np
import pytest

import oracle as O
from helpers import TOL_BF16, TOL_FP8, assert_close

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = ["decode_bf16_gqa4_d128", "decode_fp8e4m3_gqa4_d128", "prefill_bf16_gqa4_d128"]


def _expected(name):
    return np.load(os.path.join(GOLD, name + ".npz"))["expected"].astype(np.float64)


def _bf16_round(x):
    return O.decode(O.encode(np.asarray(x, np.float32), O.BF16), O.BF16).astype(np.float64)


@pytest.mark.parametrize("name", FIXTURES)
@pytest.mark.parametrize("shrink", [1.0, 1.0 / 30.0])
def test_rejects_zero_and_half_outputs(name, shrink):
    ref = _expected(name) * shrink
    tol = TOL_FP8 if "fp8" in name else TOL_BF16
    # a correctly computed output rounded to bf16 passes
    assert_close(_bf16_round(ref), ref, tol, "bf16-rounded")
    for bad, what in ((np.zeros_like(ref), "zeros"), (0.5 * ref, "half"), (-ref, "negated")):
        with pytest.raises(AssertionError):
            assert_close(bad, ref, tol, what)


def test_per_element_bound_alone_is_weak_at_long_context():
    """Documents why the whole-output bounds exist: at long-context magnitudes
    the per-element FP8 bound accepts zeros and the bf16 bound a half-size
    output."""
    ref = _expected("decode_fp8e4m3_gqa4_d128") / 30.0
    assert_close(np.zeros_like(ref), ref, TOL_FP8, "zeros", rel_l2_max=None, scale_tol=None)
    assert_close(0.5 * ref, ref, TOL_BF16, "half", rel_l2_max=None, scale_tol=None)


def test_rejects_one_wrong_row():
    """One (sequence, head) row replaced by another row's output fails."""
    ref = _expected("decode_bf16_gqa4_d128")
    got = ref.copy()
    got[1, 3] = ref[0, 5]
    with pytest.raises(AssertionError):
        assert_close(got, ref, TOL_BF16, "row swap")


def test_rejects_non_finite():
    ref = _expected("decode_bf16_gqa4_d128")
    got = ref.copy()
    got[0, 0, 0] = np.nan
    with pytest.raises(AssertionError):
        assert_close(got, ref, TOL_BF16, "nan")
