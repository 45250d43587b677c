"""Pins the attention oracle (oracle/attention.py) to things independent of it: torch CPU
float64 SDPA (torch's is_causal is top-left, like the reference's dense route), closed
forms, brute force, and the reference's offset validation rules."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as A


def _t64(*shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float64)


def _torch_sdpa(q, k, v, mask=None, causal=False, scale=None):
    g = q.size(1) // k.size(1)
    return F.scaled_dot_product_attention(
        q, k.repeat_interleave(g, 1), v.repeat_interleave(g, 1), attn_mask=mask, is_causal=causal, scale=scale
    )


@pytest.mark.parametrize(
    "b,hq,hk,sq,sk,d,causal,scale",
    [
        (2, 4, 4, 17, 17, 8, False, None),
        (1, 6, 2, 23, 23, 16, True, None),
        (2, 3, 1, 5, 40, 8, True, 0.7),  # causal Sq < Sk (top-left)
        (1, 4, 2, 40, 5, 8, True, None),  # causal Sq > Sk
        (3, 2, 2, 1, 33, 16, False, None),  # decode row
    ],
)
def test_dense_matches_torch_float64(b, hq, hk, sq, sk, d, causal, scale):
    q, k, v = _t64(b, hq, sq, d, seed=1), _t64(b, hk, sk, d, seed=2), _t64(b, hk, sk, d, seed=3)
    out, lse = A.sdpa(q.numpy(), k.numpy(), v.numpy(), is_causal=causal, scale=scale)
    ref = _torch_sdpa(q, k, v, causal=causal, scale=scale)
    assert np.abs(out - ref.numpy()).max() < 1e-12
    # lse is the natural log-sum-exp of the logits
    s = scale if scale is not None else 1 / math.sqrt(d)
    logits = s * torch.einsum("bhqd,bhkd->bhqk", q, k.repeat_interleave(hq // hk, 1))
    if causal:
        logits = logits.masked_fill(torch.ones(sq, sk, dtype=torch.bool).tril().logical_not(), float("-inf"))
    assert np.abs(lse - torch.logsumexp(logits, -1).numpy()).max() < 1e-12


@pytest.mark.parametrize("kind", ["bool", "float", "float_bcast"])
def test_masks_match_torch_float64_when_rows_keep_keys(kind):
    b, h, s, d = 2, 4, 19, 8
    q, k, v = _t64(b, h, s, d, seed=4), _t64(b, 2, s, d, seed=5), _t64(b, 2, s, d, seed=6)
    g = torch.Generator().manual_seed(7)
    if kind == "bool":
        mask = torch.rand(b, h, s, s, generator=g) > 0.4
        mask[..., 0] = True
    elif kind == "float":
        mask = torch.randn(b, h, s, s, generator=g, dtype=torch.float64)
    else:
        mask = torch.randn(1, 1, s, s, generator=g, dtype=torch.float64)
        mask = mask.masked_fill(torch.rand(1, 1, s, s, generator=g) < 0.3, float("-inf"))
        mask[..., 2] = 0.0
    out, _ = A.sdpa(q.numpy(), k.numpy(), v.numpy(), mask.numpy())
    ref = _torch_sdpa(q, k, v, mask)
    assert np.abs(out - ref.numpy()).max() < 1e-12


def test_zero_queries_average_visible_values():
    q = np.zeros((1, 2, 6, 4))
    k, v = _t64(1, 2, 6, 4, seed=8).numpy(), _t64(1, 2, 6, 4, seed=9).numpy()
    out, _ = A.sdpa(q, k, v)
    assert np.allclose(out, v.mean(axis=2, keepdims=True).repeat(6, axis=2), atol=1e-14)
    out, _ = A.sdpa(q, k, v, is_causal=True)
    causal_means = np.cumsum(v, axis=2) / np.arange(1, 7).reshape(1, 1, 6, 1)
    assert np.allclose(out, causal_means, atol=1e-14)


def test_one_visible_key_returns_its_value():
    q, k, v = _t64(1, 1, 4, 8, seed=10).numpy(), _t64(1, 1, 9, 8, seed=11).numpy(), _t64(1, 1, 9, 8, seed=12).numpy()
    mask = np.zeros((1, 1, 4, 9), dtype=bool)
    for i in range(4):
        mask[0, 0, i, 2 * i] = True
    out, _ = A.sdpa(q, k, v, mask)
    for i in range(4):
        assert np.allclose(out[0, 0, i], v[0, 0, 2 * i], atol=1e-12)


def test_fully_masked_row_is_unmasked_softmax():
    """Decision D1: the reference clamps masks at -5e5, so a row with no kept key is the
    softmax over its raw scores -- the unmasked row; torch CPU returns zeros instead."""
    q, k, v = _t64(1, 2, 5, 8, seed=13).numpy(), _t64(1, 2, 7, 8, seed=14).numpy(), _t64(1, 2, 7, 8, seed=15).numpy()
    mask = np.zeros((1, 1, 5, 7))
    mask[0, 0, 2] = -np.inf
    bmask = mask == 0
    unmasked, _ = A.sdpa(q, k, v)
    for m in (mask, bmask):
        out, _ = A.sdpa(q, k, v, m)
        assert np.allclose(out[0, :, 2], unmasked[0, :, 2], atol=1e-12)
    t = F.scaled_dot_product_attention(*(torch.from_numpy(a) for a in (q, k, v)), attn_mask=torch.from_numpy(bmask))
    assert torch.all(t[0, :, 2] == 0)  # what torch does instead (documented difference)


def test_masked_keys_get_exactly_zero_weight_at_large_logits():
    d = 8
    q = np.ones((1, 1, 1, d)) * 100.0
    k = np.zeros((1, 1, 4, d))
    k[0, 0, 2:] = 100.0  # logits 1e4 * scale on masked keys
    v = np.arange(4 * d, dtype=np.float64).reshape(1, 1, 4, d)
    keep = np.array([True, True, False, False]).reshape(1, 1, 1, 4)
    out, _ = A.sdpa(q, k, v, keep)
    assert np.array_equal(out[0, 0, 0], v[0, 0, :2].mean(axis=0))


def test_planted_mistake_is_caught():
    """A transposed-causal oracle (keys >= i instead of <= i) differs from torch."""
    q, k, v = _t64(1, 1, 8, 4, seed=16), _t64(1, 1, 8, 4, seed=17), _t64(1, 1, 8, 4, seed=18)
    wrong_mask = np.triu(np.ones((8, 8), dtype=bool))
    wrong, _ = A.sdpa(q.numpy(), k.numpy(), v.numpy(), wrong_mask)
    ref = _torch_sdpa(q, k, v, causal=True).numpy()
    assert np.abs(wrong - ref).max() > 1e-2


# ---------------------------------------------------------------- varlen


def _torch_varlen(q, k, v, cu_q, cu_k, causal, key_mask=None):
    """Per-sequence torch float64 SDPA with an explicitly built bottom-right mask."""
    out = torch.zeros(q.shape[0], q.shape[1], v.shape[2], dtype=torch.float64)
    g = q.size(1) // k.size(1)
    for b in range(len(cu_q) - 1):
        q0, q1, k0, k1 = cu_q[b], cu_q[b + 1], cu_k[b], cu_k[b + 1]
        lq, lk = q1 - q0, k1 - k0
        if lq == 0:
            continue
        allowed = torch.ones(lq, lk, dtype=torch.bool)
        if causal:
            r = torch.arange(lq)[:, None]
            c = torch.arange(lk)[None, :]
            allowed = c < torch.clamp(r + 1 + lk - lq, max=lk)
        add = torch.zeros(lq, lk, dtype=torch.float64).masked_fill(~allowed, float("-inf"))
        if key_mask is not None:
            km = key_mask[k0:k1]
            add = add + (torch.zeros(lk, dtype=torch.float64).masked_fill(~km, float("-inf")))[None, :]
        qs = q[q0:q1].transpose(0, 1)[None]
        ks = k[k0:k1].transpose(0, 1)[None].repeat_interleave(g, 1)
        vs = v[k0:k1].transpose(0, 1)[None].repeat_interleave(g, 1)
        out[q0:q1] = F.scaled_dot_product_attention(qs, ks, vs, attn_mask=add)[0].transpose(0, 1)
    return out.numpy()


@pytest.mark.parametrize("causal", [False, True])
def test_varlen_matches_per_sequence_torch(causal):
    cu_q = [0, 7, 7, 30, 45]
    cu_k = [0, 9, 12, 40, 60] if causal else [0, 3, 12, 40, 41]
    q, k, v = _t64(45, 6, 8, seed=20), _t64(60 if causal else 41, 2, 8, seed=21), _t64(60 if causal else 41, 2, 8, seed=22)
    out, lse = A.sdpa_varlen(q.numpy(), k.numpy(), v.numpy(), cu_q, cu_k, is_causal=causal)
    ref = _torch_varlen(q, k, v, cu_q, cu_k, causal)
    assert np.abs(out - ref).max() < 1e-12
    brute, blse = A.sdpa_varlen_bruteforce(q.numpy(), k.numpy(), v.numpy(), cu_q, cu_k, is_causal=causal)
    assert np.abs(out - brute).max() < 1e-12 and np.abs(lse - blse).max() < 1e-12


@pytest.mark.parametrize("dv", [4, 16])
def test_varlen_value_dim_differs(dv):
    """v [Tk, Hk, Dv] with Dv != D (the reference's packed op takes it,
    aten_varlen.cpp:160-208): the oracle against torch float64 SDPA per sequence (which
    takes a value dim of its own) and the brute-force form; lse does not depend on v."""
    cu_q, cu_k = [0, 5, 21, 30], [0, 9, 27, 40]
    q, k = _t64(30, 4, 8, seed=27), _t64(40, 2, 8, seed=28)
    v = _t64(40, 2, dv, seed=29)
    out, lse = A.sdpa_varlen(q.numpy(), k.numpy(), v.numpy(), cu_q, cu_k, is_causal=True)
    assert out.shape == (30, 4, dv)
    assert np.abs(out - _torch_varlen(q, k, v, cu_q, cu_k, True)).max() < 1e-12
    brute, blse = A.sdpa_varlen_bruteforce(q.numpy(), k.numpy(), v.numpy(), cu_q, cu_k, is_causal=True)
    assert np.abs(out - brute).max() < 1e-12 and np.abs(lse - blse).max() < 1e-12
    _, lse8 = A.sdpa_varlen(q.numpy(), k.numpy(), _t64(40, 2, 8, seed=30).numpy(), cu_q, cu_k, is_causal=True)
    assert np.abs(lse - lse8).max() < 1e-12


def test_varlen_key_mask_and_packed_mask():
    cu = [0, 10, 25]
    q, k, v = _t64(25, 4, 8, seed=23), _t64(25, 4, 8, seed=24), _t64(25, 4, 8, seed=25)
    g = torch.Generator().manual_seed(26)
    km = torch.rand(25, generator=g) > 0.3
    km[0] = km[10] = True
    out, _ = A.sdpa_varlen(q.numpy(), k.numpy(), v.numpy(), cu, key_mask=km.numpy())
    assert np.abs(out - _torch_varlen(q, k, v, cu, cu, False, km)).max() < 1e-12
    # a packed per-sequence mask equal to the key mask (broadcast over rows) gives the same
    blocks = [np.broadcast_to(km.numpy()[a:b], (b - a, b - a)).reshape(-1) for a, b in zip(cu[:-1], cu[1:])]
    out2, _ = A.sdpa_varlen(q.numpy(), k.numpy(), v.numpy(), cu, attn_mask=np.concatenate(blocks))
    assert np.abs(out - out2).max() < 1e-12
    # packed mask + causal equals the dense oracle per sequence with causal folded in
    pm = [np.where(np.random.default_rng(27).random((b - a, b - a)) < 0.2, -np.inf, 0.0) for a, b in zip(cu[:-1], cu[1:])]
    out3, _ = A.sdpa_varlen(q.numpy(), k.numpy(), v.numpy(), cu, is_causal=True,
                            attn_mask=np.concatenate([m.reshape(-1) for m in pm]))
    for (a, b), m in zip(zip(cu[:-1], cu[1:]), pm):
        n = b - a
        fold = np.where(np.tril(np.ones((n, n), dtype=bool)), m, -np.inf)
        dense, _ = A.sdpa(q.numpy()[a:b].transpose(1, 0, 2)[None], k.numpy()[a:b].transpose(1, 0, 2)[None],
                          v.numpy()[a:b].transpose(1, 0, 2)[None], fold[None, None])
        # rows whose every causal key is dropped differ (the oracle keeps causal keys
        # excluded); compare the rest
        keep_rows = np.isfinite(fold).any(axis=1)
        assert np.abs(out3[a:b][keep_rows] - dense[0].transpose(1, 0, 2)[keep_rows]).max() < 1e-12


@pytest.mark.parametrize(
    "cu_q,cu_k,causal,msg",
    [
        ([0], [0], False, "cumulative offsets"),
        ([0, 3], [0, 3, 4], False, "cumulative offsets"),
        ([1, 3], [0, 3], False, "cumulative offsets"),
        ([0, 3, 2], [0, 3, 5], False, "must not decrease"),
        ([0, 3], [0, 0], False, "needs keys"),
        ([0, 5], [0, 4], True, "leaves queries without keys"),
    ],
)
def test_varlen_offset_errors(cu_q, cu_k, causal, msg):
    with pytest.raises(ValueError, match=msg):
        A.intervals(cu_q, cu_k, causal)


@pytest.mark.parametrize("causal", [False, True])
def test_sdpa_lengths_is_attention_over_each_batch_prefix(causal):
    """Key lengths pinned by slicing: batch b's output equals torch CPU float64 SDPA over
    its first L_b keys only (causal top-left over the prefix, query rows past L_b seeing
    the prefix), and lengths outside [1, Sk] clamp."""
    b, hq, hk, sq, sk, d = 4, 6, 2, 9, 37, 16
    q, k, v = _t64(b, hq, sq, d, seed=71), _t64(b, hk, sk, d, seed=72), _t64(b, hk, sk, d, seed=73)
    lengths = [5, 37, 1, 20]
    out, _ = A.sdpa_lengths(q.numpy(), k.numpy(), v.numpy(), lengths, is_causal=causal)
    for i, n in enumerate(lengths):
        qi, ki, vi = q[i : i + 1], k[i : i + 1, :, :n], v[i : i + 1, :, :n]
        if causal:
            keep = torch.arange(n)[None, :] <= torch.arange(sq)[:, None]
            ref = _torch_sdpa(qi, ki, vi, mask=keep)
        else:
            ref = _torch_sdpa(qi, ki, vi)
        assert np.abs(out[i : i + 1] - ref.numpy()).max() < 1e-12, (i, n)
    clamped, _ = A.sdpa_lengths(q.numpy(), k.numpy(), v.numpy(), [0, 99, -3, 20], is_causal=causal)
    expect, _ = A.sdpa_lengths(q.numpy(), k.numpy(), v.numpy(), [1, 37, 1, 20], is_causal=causal)
    assert np.array_equal(clamped, expect)


def test_sdpa_lengths_catches_a_planted_off_by_one():
    """A planted mistake (keys <= L_b kept instead of < L_b) moves the result."""
    b, hq, sq, sk, d = 2, 2, 3, 10, 8
    q, k, v = _t64(b, hq, sq, d, seed=81), _t64(b, hq, sk, d, seed=82), _t64(b, hq, sk, d, seed=83)
    good, _ = A.sdpa_lengths(q.numpy(), k.numpy(), v.numpy(), [4, 7])
    wrong, _ = A.sdpa_lengths(q.numpy(), k.numpy(), v.numpy(), [5, 8])
    assert np.abs(good - wrong).max() > 1e-3
