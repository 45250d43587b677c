"""Host-side logic on the CPU: the package imports without a GPU, leaves CPU tensors to
torch, validates varlen offsets with the reference's errors, and reports refusals."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import kohakutt_amd
from kohakutt_amd import attention as katt
from oracle import norms as N


def test_cpu_tensors_keep_torch_paths():
    kohakutt_amd.reset_counters()
    q = torch.randn(1, 2, 8, 64)
    out = F.scaled_dot_product_attention(q, q, q)
    y = F.layer_norm(q, [64])
    z = F.rms_norm(q, [64])
    assert out.shape == q.shape and y.shape == q.shape and z.shape == q.shape
    c = kohakutt_amd.counters()
    assert c["attention"] == 0 and c["norms"] == 0


def test_refusal_reasons():
    q = torch.randn(1, 2, 8, 64, dtype=torch.bfloat16)
    assert "GPU" in kohakutt_amd.sdpa_refusal(q, q, q)


def test_ktt_rms_norm_composite_on_cpu():
    # The composite computes in fp32 whatever the input dtype, as the reference's does
    # (aten_fused.cpp:13-28): float64 inputs agree with the float64 oracle to fp32 rounding.
    g = torch.Generator().manual_seed(7)
    x = torch.randn(3, 40, dtype=torch.float64, generator=g)
    w = torch.randn(40, dtype=torch.float64, generator=g)
    b = torch.randn(40, dtype=torch.float64, generator=g)
    y = kohakutt_amd.rms_norm(x, w, b, 1e-6)
    yr, _ = N.rms_norm(x.numpy(), w.numpy(), b.numpy(), 1e-6)
    err = np.abs(y.numpy() - yr) / (np.abs(yr) + 1.0)
    assert err.max() < 2e-6


@pytest.mark.parametrize(
    "cu_q,cu_k,causal,msg",
    [
        ([0], [0], False, "cumulative offsets"),
        ([0, 3], [0, 3, 4], False, "cumulative offsets"),
        ([0, 3, 2], [0, 3, 5], False, "must not decrease"),
        ([0, 3], [0, 0], False, "needs keys"),
        ([0, 5], [0, 4], True, "leaves queries without keys"),
    ],
)
def test_varlen_offsets_validated_like_reference(cu_q, cu_k, causal, msg):
    with pytest.raises(ValueError, match=msg):
        katt.check_offsets(cu_q, cu_k, causal)


def test_varlen_offsets_must_end_at_totals():
    with pytest.raises(ValueError, match="must end"):
        katt.check_offsets([0, 3, 5], [0, 3, 5], False, total_q=6, total_k=5)
    assert katt.check_offsets([0, 3, 5], [0, 4, 9], True, 5, 9) == [(3, 4), (2, 5)]


def test_set_enabled_round_trip():
    kohakutt_amd.set_enabled(attention=False, norms=False)
    c = kohakutt_amd.counters()
    assert not c["attention_enabled"] and not c["norms_enabled"]
    kohakutt_amd.set_enabled()
    c = kohakutt_amd.counters()
    assert c["attention_enabled"] and c["norms_enabled"]


def test_varlen_kernels_and_autograd_registered():
    has = torch._C._dispatch_has_kernel_for_dispatch_key
    assert has("torch_attn::_varlen_attn", "CUDA")
    assert has("torch_attn::_varlen_attn_backward", "CUDA")
    for op in ("ktt::_sdpa_lengths", "ktt::_sdpa_varlen", "ktt::_sdpa_varlen_offsets"):
        assert "Autograd[alias]" in torch._C._dispatch_dump(op), op


def test_key_lengths_validation_follows_the_reference():
    """Host key lengths must lie in [1, Sk] with one per batch (``lengths.py:10-29``); a
    GPU tensor is not checked on the host (the kernels clamp it)."""
    from kohakutt_amd.attention import _as_counts

    assert _as_counts([1, 5], 2, 5, "cpu").tolist() == [1, 5]
    assert _as_counts(torch.tensor([3, 4]), 2, 5, "cpu").dtype == torch.int32
    with pytest.raises(ValueError, match="must lie in"):
        _as_counts([0, 5], 2, 5, "cpu")
    with pytest.raises(ValueError, match="must lie in"):
        _as_counts([1, 6], 2, 5, "cpu")
    with pytest.raises(ValueError, match="one length per batch"):
        _as_counts([1, 2, 3], 2, 5, "cpu")


@pytest.mark.parametrize("max_q,max_k", [(2, None), (None, 3), (4, 4)])
def test_varlen_undersized_longest_lengths_are_refused(max_q, max_k):
    """max_q / max_k size the kernels' grid and LDS; values below the longest sequence of
    host offsets are refused before any tensor is read (here on CPU tensors)."""
    q = torch.zeros(8, 2, 64, dtype=torch.bfloat16)
    k = torch.zeros(9, 2, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="below the longest sequence"):
        kohakutt_amd.sdpa_varlen(q, k, k, [0, 3, 8], [0, 4, 9], max_q=max_q, max_k=max_k)
