"""The float64 ruler of the parity tests (test infrastructure only).

The reference judges every device result by its error against the same op computed in
float64 on the CPU (``src/kohakutt/core/stats.py:9-50`` defines the statistics; the
BASELINE tolerance is a bound on their median).  This module computes the same
statistics with numpy, from the definition:

* absolute error ``|r - ref|`` over positions where both values are finite: its largest,
  lower-median and mean value;
* relative error ``|r - ref| / |ref|`` over the finite positions whose reference is
  nonzero (a zero reference has no relative error; it shows in the absolute error only);
* cosine of the angle between the finite parts of both, flattened (1 when either is all
  zero);
* ``nonfinite``: how many results are NaN or infinite (whatever the reference holds).

"Median" is the lower middle value of an even count (the k-th smallest with
k = (n - 1) // 2), the reference's convention; the mean is the plain arithmetic mean.  An
empty selection reports zeros.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU baseline import it.
"""

from __future__ import annotations

import numpy as np

STAT_KEYS = (
    "abs_max",
    "abs_median",
    "abs_mean",
    "rel_max",
    "rel_median",
    "rel_mean",
    "cosine",
    "nonfinite",
)


def _float64(x) -> np.ndarray:
    """Any array-like (a torch tensor of any dtype and device included) as a flat
    float64 numpy vector."""
    if hasattr(x, "detach"):  # a torch tensor: bf16 / fp16 have no numpy dtype
        x = x.detach().to("cpu").double().numpy()
    return np.asarray(x, dtype=np.float64).reshape(-1)


def _lower_median(v: np.ndarray) -> float:
    k = (v.size - 1) // 2
    return float(np.partition(v, k)[k])


def _summary(v: np.ndarray):
    """(max, lower median, mean) of a vector; zeros for an empty one."""
    if v.size == 0:
        return 0.0, 0.0, 0.0
    return float(v.max()), _lower_median(v), float(v.mean())


def diff_stats(result, reference) -> dict:
    """Error statistics of ``result`` against ``reference`` (equal element counts once
    flattened; compared in float64).  Returns a dict with ``STAT_KEYS``."""
    got = _float64(result)
    want = _float64(reference)
    if got.size != want.size:
        raise ValueError(f"diff_stats: {got.size} results against {want.size} reference values")
    ok = np.isfinite(got) & np.isfinite(want)
    delta = np.abs(got[ok] - want[ok])
    scale = np.abs(want[ok])
    has_rel = scale != 0
    rel = delta[has_rel] / scale[has_rel]
    out = {}
    out["abs_max"], out["abs_median"], out["abs_mean"] = _summary(delta)
    out["rel_max"], out["rel_median"], out["rel_mean"] = _summary(rel)
    norms = float(np.linalg.norm(got[ok])) * float(np.linalg.norm(want[ok]))
    out["cosine"] = float(np.dot(got[ok], want[ok]) / norms) if norms > 0 else 1.0
    out["nonfinite"] = int(got.size - np.count_nonzero(np.isfinite(got)))
    return out


def format_stats(stats: dict) -> str:
    """The statistics on one line, for test and log output."""
    return (
        "abs err: max {abs_max:.3e} / median {abs_median:.3e} / mean {abs_mean:.3e}; "
        "rel err: max {rel_max:.3e} / median {rel_median:.3e} / mean {rel_mean:.3e}; "
        "cosine {cosine:.6f}; nonfinite {nonfinite}"
    ).format(**stats)
