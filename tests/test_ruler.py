"""The float64 ruler (oracle.ruler.diff_stats) against values fixed by hand.

The known answers of the first table are the reference ruler's own test data
(``tests/core/test_stats.py:20-45`` of the reference: a known perturbation, zero
reference entries, non-finite results); the others follow from the definition.  A
plausible mistake -- the upper instead of the lower median, relative error over zero
references, non-finite values counted into the errors -- fails one of these cases.
"""

import math

import numpy as np
import pytest
import torch

from oracle.ruler import STAT_KEYS, diff_stats, format_stats

NAN, INF = float("nan"), float("inf")

# (result, reference, {statistic: expected value})
KNOWN = [
    # a perturbation of [1, 2, 4, -8] by [0.1, -0.2, 0, 0.4]: |err| = .1 .2 0 .4 and
    # rel = .1 .1 0 .05; the lower median of four values is the second smallest
    (
        [1.1, 1.8, 4.0, -7.6],
        [1.0, 2.0, 4.0, -8.0],
        {"abs_max": 0.4, "abs_mean": 0.175, "abs_median": 0.1,
         "rel_max": 0.1, "rel_mean": 0.0625, "rel_median": 0.05, "nonfinite": 0},
    ),
    # a zero reference has abs error only
    ([1.0, 2.2], [0.0, 2.0], {"abs_max": 1.0, "rel_max": 0.1, "rel_mean": 0.1, "rel_median": 0.1}),
    # NaN and inf results are counted and left out of every error
    ([1.0, NAN, INF, 4.5], [1.0, 2.0, 3.0, 4.0], {"nonfinite": 2, "abs_max": 0.5, "rel_max": 0.125,
                                                  "abs_median": 0.0}),
    # odd count: the middle value
    ([1.0, 2.0, 3.5], [1.0, 1.0, 1.0], {"abs_median": 1.0, "rel_median": 1.0, "abs_mean": 3.5 / 3}),
    # a non-finite reference drops its position from the errors, not from nonfinite
    ([1.0, 5.0], [2.0, INF], {"nonfinite": 0, "abs_max": 1.0, "rel_max": 0.5}),
    # nothing comparable: zeros, cosine 1
    ([NAN], [1.0], {"nonfinite": 1, "abs_max": 0.0, "rel_median": 0.0, "cosine": 1.0}),
]


@pytest.mark.parametrize("result, reference, want", KNOWN)
def test_known_answers(result, reference, want):
    got = diff_stats(np.array(result), np.array(reference))
    assert set(got) == set(STAT_KEYS)
    for key, value in want.items():
        assert math.isclose(got[key], value, rel_tol=1e-12, abs_tol=1e-15), (key, got[key], value)


def test_cosine_is_the_angle_of_the_finite_parts():
    r = np.array([1.1, 1.8, 4.0, -7.6])
    ref = np.array([1.0, 2.0, 4.0, -8.0])
    want = r @ ref / (np.linalg.norm(r) * np.linalg.norm(ref))
    assert math.isclose(diff_stats(r, ref)["cosine"], want, rel_tol=1e-14)
    assert math.isclose(diff_stats(-ref, ref)["cosine"], -1.0, rel_tol=1e-14)


@pytest.mark.parametrize("n", [1, 2, 7, 64, 1001])
def test_medians_agree_with_torch_lower_median(n):
    # torch.median returns the lower middle value: an independent library check.
    g = torch.Generator().manual_seed(n)
    ref = torch.randn(n, generator=g, dtype=torch.float64)
    res = ref + 1e-3 * torch.randn(n, generator=g, dtype=torch.float64)
    st = diff_stats(res, ref)
    err = (res - ref).abs()
    assert st["abs_median"] == err.median().item()
    assert st["rel_median"] == (err / ref.abs()).median().item()
    assert st["abs_max"] == err.max().item()


def test_torch_tensors_of_any_dtype_compare_in_float64():
    g = torch.Generator().manual_seed(3)
    ref = torch.randn(32, 32, generator=g, dtype=torch.float64)
    st = diff_stats(ref.bfloat16(), ref)
    # bf16 rounding: relative error at most half an ulp of an 8-bit significand
    assert 0.0 < st["rel_max"] <= 2.0**-8
    assert st["cosine"] > 0.9999
    assert diff_stats(ref.clone(), ref)["rel_max"] == 0.0


def test_identical_inputs():
    ref = np.linspace(-3.0, 3.0, 50)
    st = diff_stats(ref, ref.copy())
    assert all(st[k] == 0.0 for k in STAT_KEYS if k not in ("cosine", "nonfinite"))
    assert math.isclose(st["cosine"], 1.0, rel_tol=1e-15) and st["nonfinite"] == 0


def test_size_mismatch_is_an_error():
    with pytest.raises(ValueError):
        diff_stats(np.zeros(3), np.zeros(4))


def test_format_names_every_statistic():
    line = format_stats(diff_stats(np.ones(4), np.ones(4)))
    for word in ("abs err", "rel err", "max", "median", "mean", "cosine", "nonfinite"):
        assert word in line
