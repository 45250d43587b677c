"""float64 CPU restatement of the reference's attention semantics (test oracle).

Test infrastructure only: imported by ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``; never by the product.

What each function restates (reference paths under ``src/kohakutt_native/csrc/aten``):

* mask normalisation -- ``attention/aten_attention.cpp:223-238`` (``additive_mask``:
  bool keep-mask -> {0, -inf}), ``attention/ktt_flash/program.cpp:912-919``
  (``mask_operand``: ``clamp(mask, -5e5) / scale`` added to the raw score, so the logit is
  ``scale * q.k + max(mask, -5e5)``) and ``attention/ktt_flash/varlen_plan.hpp:17``
  (``kMaskedLogit = -5e5``).  Consequence: a masked key gets exactly zero probability
  whenever its row keeps any key, and a row whose every key is masked becomes the softmax
  over its raw scores (``docs/reference/kernels/flash-varlen.md:55-59``).
* default scale ``1/sqrt(D)`` -- ``aten_attention.cpp:317-322`` (``scale_of``).
* causal on the dense route is top-left: query ``i`` sees keys ``<= i``
  (``aten_attention.cpp:106-107,431-474``); causal takes no mask (``108-110``).
* head groups: K/V head ``h // (Hq / Hk)`` serves query head ``h``; ``Hk`` must divide
  ``Hq`` (``aten_attention.cpp:90-95``).
* varlen -- ``attention/ktt_flash/varlen_plan.hpp:43-82`` (``intervals``: offsets
  validation and its errors; bottom-right causal: query ``r`` of a sequence sees its first
  ``min(Lk, r + 1 + Lk - Lq)`` keys) and ``src/kohakutt/torch_backend/varlen.py:165-183``
  (``key_mask``: a ``[Tk]`` bool keep-mask or float additive mask clamped at -5e5).

Pinning (tests/test_oracle_attention.py): torch CPU float64
``F.scaled_dot_product_attention`` (an independent library routine; torch's ``is_causal``
is top-left) on dense/GQA/MQA/causal/masked cases and Sq != Sk; per-sequence torch SDPA
with an explicitly built bottom-right mask for varlen; closed forms (zero queries ->
mean of the visible values; one visible key -> that value row; fully-masked row ->
unmasked row); large-logit safety; the committed golden fixtures in ``tests/golden``.
"""

from __future__ import annotations

import math

import numpy as np

MASKED_LOGIT = -5e5


def _f64(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float64)


def additive_logits(mask) -> np.ndarray:
    """A bool keep-mask or a float additive mask in logit units, clamped at the
    reference's masked logit (aten_attention.cpp:223-238, program.cpp:912-919)."""
    m = np.asarray(mask)
    if m.dtype == np.bool_:
        add = np.where(m, 0.0, -np.inf)
    else:
        add = m.astype(np.float64)
    return np.maximum(add, MASKED_LOGIT)


def _softmax_rows(logits: np.ndarray):
    """Row softmax over the last axis and the natural-log log-sum-exp; -inf entries get
    exactly zero weight."""
    mx = logits.max(axis=-1, keepdims=True)
    e = np.exp(logits - mx)
    s = e.sum(axis=-1, keepdims=True)
    lse = (mx + np.log(s))[..., 0]
    return e / s, lse


def sdpa(q, k, v, attn_mask=None, is_causal=False, scale=None):
    """Dense attention of q [B, Hq, Sq, D], k [B, Hk, Sk, D], v [B, Hk, Sk, Dv].

    Returns (out [B, Hq, Sq, Dv], lse [B, Hq, Sq]) in float64.  ``attn_mask`` broadcasts
    to [B, Hq, Sq, Sk]; bool keeps True keys, float is added to the logits; both clamp at
    -5e5 (so a fully-masked row is the softmax over its raw scores).  ``is_causal`` is
    top-left (query i sees keys <= i)."""
    q, k, v = _f64(q), _f64(k), _f64(v)
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k and v must be 4-D")
    b, hq, sq, d = q.shape
    bk, hk, sk, dk = k.shape
    if bk != b or v.shape[0] != b or v.shape[1] != hk or v.shape[2] != sk or dk != d:
        raise ValueError("q, k and v shapes do not match")
    if hq % hk != 0:
        raise ValueError("K / V heads must divide Q heads")
    if is_causal and attn_mask is not None:
        raise ValueError("causal takes no mask")
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    group = hq // hk
    kx = np.repeat(k, group, axis=1)
    vx = np.repeat(v, group, axis=1)
    logits = scale * np.einsum("bhqd,bhkd->bhqk", q, kx)
    if attn_mask is not None:
        logits = logits + np.broadcast_to(additive_logits(attn_mask), logits.shape)
    if is_causal:
        qi = np.arange(sq)[:, None]
        kj = np.arange(sk)[None, :]
        logits = np.where(kj <= qi, logits, -np.inf)
    p, lse = _softmax_rows(logits)
    out = np.einsum("bhqk,bhkd->bhqd", p, vx)
    return out, lse


def sdpa_lengths(q, k, v, key_lengths, is_causal=False, scale=None):
    """Attention with per-batch key lengths (the reference's ``kohakutt.sdpa(key_lengths=)``,
    ``src/kohakutt/attention.py:10-23``): batch b's queries see keys [0, L_b), L_b =
    key_lengths[b] clamped to [1, Sk] (device lengths are clamped,
    ``docs/reference/kernels/flash.md`` "Key lengths"); with causal, also keys <= the
    query's position (top-left).  Restated as the reference's explicit-mask route
    (``torch_backend/lengths.py:79-89``).  Returns (out, lse) in float64."""
    q = _f64(q)
    b, sq, sk = q.shape[0], q.shape[2], np.asarray(k).shape[2]
    lengths = np.clip(np.asarray(key_lengths, dtype=np.int64).reshape(b), 1, sk)
    keys = np.arange(sk)
    keep = (keys[None, :] < lengths[:, None])[:, None, None, :]
    if is_causal:
        keep = keep & (keys[None, :] <= np.arange(sq)[:, None])[None, None]
    return sdpa(q, k, v, keep, False, scale)


def offsets(cu) -> list[int]:
    """Cumulative offsets as a list of ints."""
    return [int(x) for x in np.asarray(cu).reshape(-1).tolist()]


def intervals(cu_q, cu_k, causal):
    """The packed key interval [lo, hi) each packed query sees, with the reference's
    validation and messages (varlen_plan.hpp:43-82)."""
    cu_q, cu_k = offsets(cu_q), offsets(cu_k)
    if len(cu_q) < 2 or len(cu_q) != len(cu_k) or cu_q[0] != 0 or cu_k[0] != 0:
        raise ValueError(
            "sdpa_varlen needs cumulative offsets [0, ..., total] of equal count for "
            "queries and keys"
        )
    lo, hi = [], []
    for b in range(len(cu_q) - 1):
        lq = cu_q[b + 1] - cu_q[b]
        lk = cu_k[b + 1] - cu_k[b]
        if lq < 0 or lk < 0 or (lq > 0 and lk == 0):
            raise ValueError(
                "sdpa_varlen offsets must not decrease, and a sequence with queries "
                "needs keys"
            )
        for r in range(lq):
            seen = min(lk, r + 1 + lk - lq) if causal else lk
            if seen <= 0:
                raise ValueError(
                    "causal sdpa_varlen with more queries than keys in a sequence "
                    "leaves queries without keys"
                )
            lo.append(cu_k[b])
            hi.append(cu_k[b] + seen)
    return np.asarray(lo, dtype=np.int64), np.asarray(hi, dtype=np.int64)


def _varlen_common(q, k, v, cu_q, cu_k, is_causal, scale, key_mask, attn_mask):
    q, k, v = _f64(q), _f64(k), _f64(v)
    cu_q = offsets(cu_q)
    cu_k = cu_q if cu_k is None else offsets(cu_k)
    lo, hi = intervals(cu_q, cu_k, is_causal)
    tq, h, d = q.shape
    tk, hk, _ = k.shape
    if h % hk != 0:
        raise ValueError("K / V heads must divide Q heads")
    if cu_q[-1] != tq or cu_k[-1] != tk:
        raise ValueError("offsets must end at the packed token counts")
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    km = None if key_mask is None else additive_logits(key_mask)
    am = None if attn_mask is None else additive_logits(np.asarray(attn_mask).reshape(-1))
    return q, k, v, cu_q, cu_k, lo, hi, scale, km, am


def sdpa_varlen(
    q,
    k,
    v,
    cu_q,
    cu_k=None,
    is_causal=False,
    scale=None,
    key_mask=None,
    attn_mask=None,
):
    """Packed attention: q [Tq, H, D], k [Tk, Hk, D], v [Tk, Hk, Dv]; each query sees
    the keys of its own sequence, bottom-right causal with ``is_causal``.

    ``key_mask``: [Tk], bool keep-mask or float additive (varlen.py:165-183).
    ``attn_mask``: the block-packed per-sequence mask of this build -- the
    concatenation of every sequence's row-major [Lq_i, Lk_i] block (length
    sum(Lq_i * Lk_i)), shared by all heads; bool keeps True.  Both clamp at -5e5, so a
    query whose visible keys are all masked gets the softmax over their raw scores.
    Keys outside a query's interval (other sequences, causal) are excluded outright.

    Returns (out [Tq, H, Dv], lse [H, Tq]) in float64.  One dense step per sequence."""
    q, k, v, cu_q, cu_k, lo, hi, scale, km, am = _varlen_common(
        q, k, v, cu_q, cu_k, is_causal, scale, key_mask, attn_mask
    )
    tq, h, _ = q.shape
    group = h // k.shape[1]
    out = np.zeros((tq, h, v.shape[2]))
    lse = np.zeros((h, tq))
    block0 = 0
    for b in range(len(cu_q) - 1):
        q0, q1, k0, k1 = cu_q[b], cu_q[b + 1], cu_k[b], cu_k[b + 1]
        lq, lk = q1 - q0, k1 - k0
        if lq == 0:
            continue
        qs = q[q0:q1].transpose(1, 0, 2)  # [H, Lq, D]
        ks = np.repeat(k[k0:k1].transpose(1, 0, 2), group, axis=0)
        vs = np.repeat(v[k0:k1].transpose(1, 0, 2), group, axis=0)
        logits = scale * np.einsum("hqd,hkd->hqk", qs, ks)
        if km is not None:
            logits = logits + km[k0:k1][None, None, :]
        if am is not None:
            logits = logits + am[block0 : block0 + lq * lk].reshape(1, lq, lk)
        cols = np.arange(lk)[None, :] + k0
        visible = (cols >= lo[q0:q1, None]) & (cols < hi[q0:q1, None])
        logits = np.where(visible[None], logits, -np.inf)
        p, l_ = _softmax_rows(logits)
        out[q0:q1] = np.einsum("hqk,hkd->hqd", p, vs).transpose(1, 0, 2)
        lse[:, q0:q1] = l_
        block0 += lq * lk
    return out, lse


def sdpa_varlen_bruteforce(
    q,
    k,
    v,
    cu_q,
    cu_k=None,
    is_causal=False,
    scale=None,
    key_mask=None,
    attn_mask=None,
):
    """``sdpa_varlen`` one (token, head) at a time over its key interval: the
    small-case cross-check of the vectorised form."""
    q, k, v, cu_q, cu_k, lo, hi, scale, km, am = _varlen_common(
        q, k, v, cu_q, cu_k, is_causal, scale, key_mask, attn_mask
    )
    tq, h, _ = q.shape
    group = h // k.shape[1]
    out = np.zeros((tq, h, v.shape[2]))
    lse = np.zeros((h, tq))
    block0 = 0
    for b in range(len(cu_q) - 1):
        q0, q1 = cu_q[b], cu_q[b + 1]
        lk = cu_k[b + 1] - cu_k[b]
        for r in range(q1 - q0):
            t = q0 + r
            kl, kh = int(lo[t]), int(hi[t])
            for head in range(h):
                kvh = head // group
                logits = np.array(
                    [scale * float(np.dot(q[t, head], k[j, kvh])) for j in range(kl, kh)]
                )
                if km is not None:
                    logits = logits + km[kl:kh]
                if am is not None:
                    logits = logits + am[block0 + r * lk : block0 + r * lk + (kh - kl)]
                mx = logits.max()
                e = np.exp(logits - mx)
                out[t, head] = (e / e.sum()) @ v[kl:kh, kvh]
                lse[head, t] = mx + np.log(e.sum())
        block0 += (q1 - q0) * lk
    return out, lse
