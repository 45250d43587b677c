"""Pins the norm oracle (oracle/norms.py) to torch CPU float64 and closed forms."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import norms as N


def _t64(*shape, seed):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)


@pytest.mark.parametrize("shape", [(1, 33), (5, 70), (2, 3, 50, 128)])
@pytest.mark.parametrize("affine", [True, False])
def test_layer_norm_matches_torch_float64(shape, affine):
    x = _t64(*shape, seed=1) * 3 + 1
    w = _t64(shape[-1], seed=2) if affine else None
    b = _t64(shape[-1], seed=3) if affine else None
    y, mean, rstd = N.layer_norm(x.numpy(), None if w is None else w.numpy(), None if b is None else b.numpy(), 1e-5)
    ty, tm, tr = torch.native_layer_norm(x, [shape[-1]], w, b, 1e-5)
    assert np.abs(y - ty.numpy()).max() < 1e-12
    assert np.abs(mean - tm.numpy()).max() < 1e-12
    assert np.abs(rstd - tr.numpy()).max() < 1e-10
    assert mean.shape == tuple(tm.shape)


def test_layer_norm_over_two_trailing_dims():
    x = _t64(3, 4, 5, seed=4)
    y, mean, _ = N.layer_norm(x.numpy(), eps=1e-5, normalized=2)
    ty, tm, _ = torch.native_layer_norm(x, [4, 5], None, None, 1e-5)
    assert np.abs(y - ty.numpy()).max() < 1e-12 and mean.shape == (3, 1, 1)


@pytest.mark.parametrize("eps", [None, 1e-6])
def test_rms_norm_matches_torch_float64(eps):
    x = _t64(7, 96, seed=5)
    w = _t64(96, seed=6)
    y, rstd = N.rms_norm(x.numpy(), w.numpy(), eps=eps)
    e = torch.finfo(torch.float32).eps if eps is None else eps
    ty = F.rms_norm(x, [96], w, e)
    assert np.abs(y - ty.numpy()).max() < 1e-12
    assert np.allclose(rstd[:, 0], 1 / np.sqrt((x.numpy() ** 2).mean(axis=1) + e))


def test_closed_forms():
    # a constant row normalises to the bias
    x = np.full((2, 16), 3.5)
    b = np.arange(16.0)
    y, mean, rstd = N.layer_norm(x, None, b, 1e-5)
    assert np.allclose(y, b[None, :]) and np.allclose(mean, 3.5) and np.allclose(rstd, 1 / np.sqrt(1e-5))
    # a row of +-a has RMS a
    a = 2.5
    x = np.array([[a, -a] * 8])
    y, rstd = N.rms_norm(x, eps=1e-6)
    assert np.allclose(rstd, 1 / np.sqrt(a * a + 1e-6)) and np.allclose(np.abs(y), a / np.sqrt(a * a + 1e-6))
    # layer norm is invariant to x -> c x + s (c > 0), up to eps
    x = np.random.default_rng(0).standard_normal((3, 64))
    y1, _, _ = N.layer_norm(x, eps=0.0)
    y2, _, _ = N.layer_norm(7.0 * x - 3.0, eps=0.0)
    assert np.abs(y1 - y2).max() < 1e-12


def test_rms_with_bias_is_rms_plus_bias():
    x, w, b = _t64(4, 32, seed=7).numpy(), _t64(32, seed=8).numpy(), _t64(32, seed=9).numpy()
    y0, _ = N.rms_norm(x, w, eps=1e-6)
    y1, _ = N.rms_norm(x, w, b, eps=1e-6)
    assert np.allclose(y1, y0 + b[None, :])
