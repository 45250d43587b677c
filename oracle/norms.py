"""float64 CPU restatement of the reference's LayerNorm / RMSNorm (test oracle).

Test infrastructure only: imported by ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``; never by the product.

Restates (reference paths under ``src/kohakutt_native/csrc/aten/nn``):

* ``layer_norm`` -- ``aten_norm.cpp:65-127``: y = (x - mean) * rstd * weight + bias over
  the normalized trailing dims, returning mean and rstd with the normalized dims kept as
  size 1; ``ktt_norm/fwd_compute.cpp:275-358``: two-pass statistics (mean, then the
  centred sum of squares), var = relu(M2 / W), rstd = rsqrt(var + eps).
* ``rms_norm`` -- ``aten_norm.cpp:604-652``: y = x * rsqrt(mean(x^2) + eps) * weight,
  eps defaulting to float32 epsilon (``aten_norm.cpp:610``); ``aten_fused.cpp:13-28``
  (``ktt::rms_norm``): the same plus an optional bias.

Pinning (tests/test_oracle_norms.py): torch CPU float64 ``native_layer_norm`` and
``F.rms_norm``; closed forms (a constant row normalises to ``bias``; a row of +-a gives
rstd 1/sqrt(a^2 + eps)); invariance of y under x -> c*x + s for LayerNorm.
"""

from __future__ import annotations

import numpy as np

FLOAT32_EPS = float(np.finfo(np.float32).eps)


def _rows(x, normalized):
    x = np.asarray(x, dtype=np.float64)
    if normalized < 1 or normalized > x.ndim:
        raise ValueError("normalized dims out of range")
    lead = x.shape[: x.ndim - normalized]
    width = int(np.prod(x.shape[x.ndim - normalized :]))
    return x.reshape(-1, width), lead


def layer_norm(x, weight=None, bias=None, eps=1e-5, normalized=1):
    """(y, mean, rstd) in float64; mean/rstd have the normalized dims kept as 1."""
    shape = np.shape(x)
    rows, lead = _rows(x, normalized)
    mean = rows.mean(axis=1, keepdims=True)
    centred = rows - mean
    var = np.maximum((centred * centred).mean(axis=1, keepdims=True), 0.0)
    rstd = 1.0 / np.sqrt(var + eps)
    y = centred * rstd
    if weight is not None:
        y = y * np.asarray(weight, dtype=np.float64).reshape(1, -1)
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64).reshape(1, -1)
    stat_shape = tuple(lead) + (1,) * normalized
    return y.reshape(shape), mean.reshape(stat_shape), rstd.reshape(stat_shape)


def rms_norm(x, weight=None, bias=None, eps=None, normalized=1):
    """(y, rstd) in float64; rstd has the normalized dims kept as 1."""
    if eps is None:
        eps = FLOAT32_EPS
    shape = np.shape(x)
    rows, lead = _rows(x, normalized)
    rstd = 1.0 / np.sqrt((rows * rows).mean(axis=1, keepdims=True) + eps)
    y = rows * rstd
    if weight is not None:
        y = y * np.asarray(weight, dtype=np.float64).reshape(1, -1)
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64).reshape(1, -1)
    return y.reshape(shape), rstd.reshape(tuple(lead) + (1,) * normalized)
