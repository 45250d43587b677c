"""GPU parity of the flash backward (``kmi_attn_bwd`` behind the overrideable SDPA
backward, the packed ops and key lengths): dq, dk, dv (causal top-left or not, GQA,
Sq != Sk, ragged lengths, bool and additive masks with fully-masked rows, packed
sequences with key masks and per-row masks, bf16 / fp16) against float64 autograd of the
same attention on the CPU, with the BASELINE bar: median relative error at most 1.5x
torch's CPU autograd at the same dtype."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import attn_cases as C
import numpy as np
from oracle import attention as oatt

pytestmark = pytest.mark.gpu

CASES = [
    # b, hq, hk, sq, sk, d, causal
    (2, 4, 4, 128, 128, 64, False),
    (1, 14, 2, 300, 300, 64, True),
    (2, 8, 2, 100, 260, 128, False),
    (1, 4, 1, 200, 120, 64, True),
    (2, 6, 3, 77, 77, 128, True),
    (1, 2, 2, 1, 45, 64, False),
    # Enough workgroups that dK/dV and dQ run unsplit (direct writes, no partials):
    (16, 8, 8, 256, 256, 64, False),
    (8, 16, 4, 256, 256, 128, True),
]


def _grads(q, k, v, go, causal, dtype, dev=None):
    """(out, dq, dk, dv) of SDPA at ``dtype`` on ``dev`` (CPU when None)."""
    hq, hk = q.size(1), k.size(1)
    ts = [t.to(dtype) for t in (q, k, v)]
    if dev is not None:
        ts = [t.to(dev) for t in ts]
    ts = [t.detach().requires_grad_() for t in ts]
    qq, kk, vv = ts
    if dev is None:
        kk_, vv_ = kk.repeat_interleave(hq // hk, 1), vv.repeat_interleave(hq // hk, 1)
        out = F.scaled_dot_product_attention(qq, kk_, vv_, is_causal=causal)
    else:
        out = F.scaled_dot_product_attention(qq, kk, vv, is_causal=causal, enable_gqa=hq != hk)
    g = go.to(dtype)
    out.backward(g.to(dev) if dev is not None else g)
    return [t.detach().cpu() for t in (out, qq.grad, kk.grad, vv.grad)]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_flash_backward_meets_the_float64_ruler(native, dev, case, dtype):
    b, hq, hk, sq, sk, d, causal = case
    print(f"backward case {case} {dtype}", flush=True)
    g = C.gen(900 + sum(case))
    q, k, v = C.randn(g, b, hq, sq, d, dtype=torch.float32), C.randn(g, b, hk, sk, d, dtype=torch.float32), C.randn(
        g, b, hk, sk, d, dtype=torch.float32)
    go = C.randn(g, b, hq, sq, d, dtype=torch.float32)
    # Inputs rounded to the test dtype first: every path sees the same values.
    q, k, v, go = (t.to(dtype).to(torch.float32) for t in (q, k, v, go))
    native.reset_counters()
    gpu = _grads(q, k, v, go, causal, dtype, dev)
    torch.cuda.synchronize()
    c = native.counters()
    assert c["attention"] == 1 and c["attention_backward"] == 1, c
    ref = _grads(q, k, v, go, causal, torch.float64)
    # Baseline at the same dtype: torch's CPU autograd in that dtype.
    cpu = _grads(q, k, v, go, causal, dtype)
    for name, gg, cc, rr in zip(("out", "dq", "dk", "dv"), gpu, cpu, ref):
        ok, sg, sc = C.ruler_ok(gg, cc, rr, factor=1.5)
        print(f"  {name}: gpu rel_median {sg['rel_median']:.2e}  cpu {sc['rel_median']:.2e}", flush=True)
        assert ok, (name, sg, sc)
        scale = rr.abs().max().item()
        assert (gg.double() - rr).abs().max().item() <= 3e-2 * max(scale, 1.0), (name, scale)


def test_gqa_key_gradients_sum_their_query_heads(native, dev):
    """dk / dv of a K/V head equal the sum over its query heads of the per-head gradients
    (the same call with K/V repeated per query head, reduced afterwards)."""
    g = C.gen(950)
    b, hq, hk, s, d = 1, 6, 2, 96, 64
    q, k, v, go = (C.randn(g, *shape) for shape in ((b, hq, s, d), (b, hk, s, d), (b, hk, s, d), (b, hq, s, d)))
    qd, kd, vd = (t.to(dev).requires_grad_() for t in (q, k, v))
    F.scaled_dot_product_attention(qd, kd, vd, is_causal=True, enable_gqa=True).backward(go.to(dev))
    kr = k.repeat_interleave(3, 1).to(dev).requires_grad_()
    vr = v.repeat_interleave(3, 1).to(dev).requires_grad_()
    q2 = q.to(dev).requires_grad_()
    F.scaled_dot_product_attention(q2, kr, vr, is_causal=True).backward(go.to(dev))
    torch.cuda.synchronize()
    dk_sum = kr.grad.float().view(b, hk, 3, s, d).sum(2)
    dv_sum = vr.grad.float().view(b, hk, 3, s, d).sum(2)
    assert (kd.grad.float() - dk_sum).abs().max().item() < 3e-2
    assert (vd.grad.float() - dv_sum).abs().max().item() < 3e-2
    assert torch.equal(qd.grad, q2.grad)


def _masked_grads(q, k, v, go, mask, dtype, dev=None):
    """(out, dq, dk, dv) of masked SDPA at ``dtype``; on the CPU a fully-masked row follows
    the reference (softmax over its raw scores): its mask entries are lifted to 0."""
    hq, hk = q.size(1), k.size(1)
    ts = [t.to(dtype) for t in (q, k, v)]
    m = mask
    if dev is not None:
        ts = [t.to(dev) for t in ts]
        m = mask.to(dev)
    else:
        keep = mask if mask.dtype == torch.bool else mask > -5e5
        dead = ~keep.any(-1, keepdim=True)
        if mask.dtype == torch.bool:
            m = mask | dead
        else:
            m = mask.masked_fill(dead.expand_as(mask), 0.0)
    if m.is_floating_point():
        m = m.to(dtype)
    ts = [t.detach().requires_grad_() for t in ts]
    qq, kk, vv = ts
    if dev is None:
        out = F.scaled_dot_product_attention(qq, kk.repeat_interleave(hq // hk, 1), vv.repeat_interleave(hq // hk, 1),
                                             attn_mask=m)
    else:
        out = F.scaled_dot_product_attention(qq, kk, vv, attn_mask=m, enable_gqa=hq != hk)
    out.backward(go.to(dtype).to(dev) if dev is not None else go.to(dtype))
    return [t.detach().cpu() for t in (out, qq.grad, kk.grad, vv.grad)]


@pytest.mark.parametrize("kind", ["bool", "additive", "bool_key_padding"])
def test_masked_backward_on_the_kernels(native, dev, kind):
    """Masked calls take the backward kernels with the forward's mask rules, fully-masked
    rows included (the reference's softmax over raw scores)."""
    g = C.gen(951 + len(kind))
    b, hq, hk, sq, sk, d = 2, 4, 2, 70, 90, 64
    q, k, v, go = (C.randn(g, *sh, dtype=torch.float32) for sh in ((b, hq, sq, d), (b, hk, sk, d), (b, hk, sk, d),
                                                                    (b, hq, sq, d)))
    q, k, v, go = (t.bfloat16().float() for t in (q, k, v, go))
    if kind == "bool":
        mask = torch.rand(b, hq, sq, sk, generator=g) > 0.3
        mask[0, 1, 7] = False  # a fully-masked row
    elif kind == "additive":
        mask = torch.randn(b, 1, sq, sk, generator=g).masked_fill(torch.rand(b, 1, sq, sk, generator=g) < 0.2,
                                                                   float("-inf"))
        mask[1, 0, 3] = float("-inf")
    else:
        lens = torch.tensor([90, 17])
        mask = (torch.arange(sk)[None, :] < lens[:, None]).reshape(b, 1, 1, sk)
    native.reset_counters()
    gpu = _masked_grads(q, k, v, go, mask, torch.bfloat16, dev)
    torch.cuda.synchronize()
    c = native.counters()
    assert c["attention"] == 1 and c["attention_backward"] == 1, c
    ref = _masked_grads(q, k, v, go, mask.double() if mask.is_floating_point() else mask, torch.float64)
    cpu = _masked_grads(q, k, v, go, mask, torch.bfloat16)
    for name, gg, cc, rr in zip(("out", "dq", "dk", "dv"), gpu, cpu, ref):
        ok, sg, sc = C.ruler_ok(gg, cc, rr, factor=1.5)
        print(f"  {kind} {name}: gpu rel_median {sg['rel_median']:.2e}  cpu {sc['rel_median']:.2e}", flush=True)
        assert ok, (kind, name, sg, sc)


def test_mask_with_its_own_gradient_takes_the_recompute(native, dev):
    """A float mask that requires grad gets its gradient from the fp32 recompute."""
    g = C.gen(955)
    q, k, v = (C.randn(g, 1, 2, 32, 64) for _ in range(3))
    mask = torch.randn(1, 1, 32, 32, generator=g).to(dev).requires_grad_()
    native.reset_counters()
    out = F.scaled_dot_product_attention(q.to(dev), k.to(dev), v.to(dev), attn_mask=mask.bfloat16())
    out.float().sum().backward()
    torch.cuda.synchronize()
    assert mask.grad is not None and mask.grad.abs().sum().item() > 0
    assert native.counters()["attention_backward"] == 0


def _varlen_ref_grads(q, k, v, go, cu_q, cu_k, causal, key_mask=None):
    """Per-sequence float64 autograd of torch CPU SDPA (bottom-right causal as an explicit
    mask; a bool key mask keeps True keys); packed [T, H, D] gradients."""
    grads = [torch.zeros(t.shape, dtype=torch.float64) for t in (q, k, v)]
    hq, hk = q.size(1), k.size(1)
    for i in range(len(cu_q) - 1):
        a, b, c, d = cu_q[i], cu_q[i + 1], cu_k[i], cu_k[i + 1]
        lq, lk = b - a, d - c
        qs, ks, vs = (t.double().transpose(0, 1)[None].requires_grad_() for t in (q[a:b], k[c:d], v[c:d]))
        keep = torch.ones(lq, lk, dtype=torch.bool)
        if causal:
            keep &= torch.arange(lk)[None, :] <= torch.arange(lq)[:, None] + (lk - lq)
        if key_mask is not None:
            keep &= key_mask[c:d][None, :]
        out = F.scaled_dot_product_attention(qs, ks.repeat_interleave(hq // hk, 1), vs.repeat_interleave(hq // hk, 1),
                                             attn_mask=keep)
        out.backward(go[a:b].double().transpose(0, 1)[None])
        for gsum, t, (lo, hi) in zip(grads, (qs, ks, vs), ((a, b), (c, d), (c, d))):
            gsum[lo:hi] = t.grad[0].transpose(0, 1)
    return grads


@pytest.mark.parametrize("kind", ["causal_self", "cross_noncausal", "causal_fewer_queries", "key_mask"])
def test_varlen_backward_matches_float64_autograd(native, dev, kind):
    """Gradients through ``kohakutt_amd.sdpa_varlen``: every sequence in one set of
    backward kernel launches (bottom-right causal, key masks)."""
    g = C.gen(960 + len(kind))
    hq, hk, d = 8, 2, 64
    if kind == "causal_self":
        lq = [70, 1, 130, 33]
        lk = lq
    elif kind == "cross_noncausal":
        lq, lk = [40, 77, 5], [90, 12, 64]
    else:
        lq, lk = [20, 50, 3], [64, 50, 40]
    cu_q = [0] + list(torch.tensor(lq).cumsum(0).tolist())
    cu_k = [0] + list(torch.tensor(lk).cumsum(0).tolist())
    causal = kind in ("causal_self", "causal_fewer_queries")
    q, go = C.randn(g, cu_q[-1], hq, d), C.randn(g, cu_q[-1], hq, d)
    k, v = C.randn(g, cu_k[-1], hk, d), C.randn(g, cu_k[-1], hk, d)
    key_mask = None
    if kind == "key_mask":
        key_mask = torch.rand(cu_k[-1], generator=g) > 0.3
        for c in cu_k[:-1]:
            key_mask[c] = True  # every row keeps a key
    qd, kd, vd = (t.to(dev).requires_grad_() for t in (q, k, v))
    native.reset_counters()
    out = native.sdpa_varlen(qd, kd, vd, cu_q, cu_k, is_causal=causal,
                             attn_mask=None if key_mask is None else key_mask.to(dev))
    out.backward(go.to(dev))
    torch.cuda.synchronize()
    assert native.counters()["attention_backward"] == 1, native.counters()
    ref = _varlen_ref_grads(q, k, v, go, cu_q, cu_k, causal, key_mask)
    for name, got, want in zip(("dq", "dk", "dv"), (qd.grad, kd.grad, vd.grad), ref):
        err = (got.cpu().double() - want).abs().max().item()
        assert err <= 3e-2 * max(want.abs().max().item(), 1.0), (kind, name, err)


def test_varlen_fp32_inputs_give_fp32_gradients(native, dev):
    """fp32 q / k / v that require gradients: the forward casts to bf16 and returns fp32,
    the backward runs the bf16 kernels on bf16 copies and returns fp32 gradients, within
    bf16 accuracy of float64 autograd."""
    g = C.gen(977)
    hq, hk, d = 4, 2, 64
    lq = [50, 17, 90]
    cu = [0] + list(torch.tensor(lq).cumsum(0).tolist())
    q, go = torch.randn(cu[-1], hq, d, generator=g), torch.randn(cu[-1], hq, d, generator=g)
    k, v = torch.randn(cu[-1], hk, d, generator=g), torch.randn(cu[-1], hk, d, generator=g)
    qd, kd, vd = (t.to(dev).requires_grad_() for t in (q, k, v))
    native.reset_counters()
    out = native.sdpa_varlen(qd, kd, vd, cu, cu, is_causal=True)
    assert out.dtype == torch.float32
    out.backward(go.to(dev))
    torch.cuda.synchronize()
    assert native.counters()["attention_backward"] == 1, native.counters()
    # The kernels see bf16 operands: compare with float64 autograd of those.
    ref = _varlen_ref_grads(*(t.bfloat16() for t in (q, k, v, go)), cu, cu, True)
    for name, got, want in zip(("dq", "dk", "dv"), (qd.grad, kd.grad, vd.grad), ref):
        assert got.dtype == torch.float32, name
        err = (got.cpu().double() - want).abs().max().item()
        assert err <= 3e-2 * max(want.abs().max().item(), 1.0), (name, err)


def test_reference_varlen_ops_forward_and_backward(native, dev):
    """The reference's packed ops as its glue calls them (``torch_backend/varlen.py``):
    ``_varlen_plan`` on the host, ``_sdpa_varlen(..., stats=True, key_mask)`` and
    ``_sdpa_varlen_backward`` from the output, in the reference's key-mask form (bf16,
    divided by the scale).  Gradients also flow through autograd on ``_sdpa_varlen``."""
    g = C.gen(970)
    cu_q, cu_k = [0, 30, 31, 120], [0, 40, 41, 150]
    hq, hk, d = 4, 2, 64
    scale = d ** -0.5
    q, go = C.randn(g, cu_q[-1], hq, d), C.randn(g, cu_q[-1], hq, d)
    k, v = C.randn(g, cu_k[-1], hk, d), C.randn(g, cu_k[-1], hk, d)
    keep = torch.rand(cu_k[-1], generator=g) > 0.25
    for c in cu_k[:-1]:
        keep[c] = True
    # varlen.key_mask: bool -> (mask - 1) * (5e5 / scale) in bf16
    km = ((keep.to(torch.bfloat16) - 1.0) * (5e5 / scale)).to(torch.bfloat16)
    records, masks = torch.ops.ktt._varlen_plan(cu_q, cu_k, True, scale, False)
    records, masks = records.to(dev), masks.to(dev)
    qd, kd, vd = (t.to(dev).requires_grad_() for t in (q, k, v))
    native.reset_counters()
    out, lse = torch.ops.ktt._sdpa_varlen(qd, kd, vd, records, masks, cu_q, cu_k, True, scale, True, km.to(dev),
                                          False)
    assert lse.shape == (hq, cu_q[-1])
    out.backward(go.to(dev))
    torch.cuda.synchronize()
    c = native.counters()
    assert c["attention"] == 1 and c["attention_backward"] == 1, c
    ref_out, _ = oatt.sdpa_varlen(C.f64(q), C.f64(k), C.f64(v), cu_q, cu_k, is_causal=True,
                                  key_mask=keep.numpy())
    assert np.abs(out.detach().cpu().double().numpy() - ref_out).max() < 2e-2
    ref = _varlen_ref_grads(q, k, v, go, cu_q, cu_k, True, keep)
    for name, got, want in zip(("dq", "dk", "dv"), (qd.grad, kd.grad, vd.grad), ref):
        err = (got.cpu().double() - want).abs().max().item()
        assert err <= 3e-2 * max(want.abs().max().item(), 1.0), (name, err)
    # The backward op called directly gives the same gradients.
    dq, dk, dv = torch.ops.ktt._sdpa_varlen_backward(go.to(dev), out.detach(), qd.detach(), kd.detach(), vd.detach(),
                                                     records, masks, records, masks, cu_q, cu_k, True, scale,
                                                     km.to(dev))
    assert torch.equal(dq, qd.grad) and torch.equal(dk, kd.grad) and torch.equal(dv, vd.grad)


def test_varlen_packed_mask_backward(native, dev):
    """Per-row block-packed masks (config 4's masked run form) through autograd, one
    fully-masked row included."""
    g = C.gen(971)
    lens = [40, 75]
    cu = [0, 40, 115]
    hq, hk, d = 4, 2, 128
    q, go = C.randn(g, cu[-1], hq, d), C.randn(g, cu[-1], hq, d)
    k, v = C.randn(g, cu[-1], hk, d), C.randn(g, cu[-1], hk, d)
    blocks = []
    for i, n in enumerate(lens):
        keep = torch.ones(n, n, dtype=torch.bool).tril() & (torch.rand(n, n, generator=g) > 0.1)
        if i == 0:
            keep[5] = False
        blocks.append(torch.zeros(n, n).masked_fill(~keep, float("-inf")).reshape(-1))
    pm = torch.cat(blocks)
    qd, kd, vd = (t.to(dev).requires_grad_() for t in (q, k, v))
    native.reset_counters()
    out = native.sdpa_varlen(qd, kd, vd, cu, is_causal=True, packed_mask=pm.to(dev))
    out.backward(go.to(dev))
    torch.cuda.synchronize()
    assert native.counters()["attention_backward"] == 1
    # float64 reference per sequence with the reference's fully-masked-row rule.
    grads = [torch.zeros(t.shape, dtype=torch.float64) for t in (q, k, v)]
    off = 0
    for a, b in zip(cu[:-1], cu[1:]):
        n = b - a
        m = pm[off:off + n * n].reshape(n, n).double().clamp_min(-5e5)
        off += n * n
        # causal visibility stays; a row whose visible keys are all masked attends over
        # their raw scores (the forward's rule)
        vis = torch.ones(n, n, dtype=torch.bool).tril()
        dead = ((m <= -5e5) | ~vis).all(-1, keepdim=True)
        m = m.masked_fill(dead & vis, 0.0).masked_fill(~vis, float("-inf"))
        qs, ks, vs = (t.double().transpose(0, 1)[None].requires_grad_() for t in (q[a:b], k[a:b], v[a:b]))
        o = F.scaled_dot_product_attention(qs, ks.repeat_interleave(2, 1), vs.repeat_interleave(2, 1), attn_mask=m)
        o.backward(go[a:b].double().transpose(0, 1)[None])
        for gsum, t in zip(grads, (qs, ks, vs)):
            gsum[a:b] = t.grad[0].transpose(0, 1)
    for name, got, want in zip(("dq", "dk", "dv"), (qd.grad, kd.grad, vd.grad), grads):
        err = (got.cpu().double() - want).abs().max().item()
        assert err <= 5e-2 * max(want.abs().max().item(), 1.0), (name, err)


def test_torch_varlen_attn_forward_and_backward(native, dev):
    """torch.nn.attention.varlen.varlen_attn on GPU tensors: both of torch's ops run the
    kernels (``torch_attn::_varlen_attn`` and ``_varlen_attn_backward``)."""
    from torch.nn.attention.varlen import varlen_attn

    g = C.gen(972)
    cu = [0, 50, 51, 130]
    q, go = C.randn(g, cu[-1], 4, 64), C.randn(g, cu[-1], 4, 64)
    k, v = C.randn(g, cu[-1], 4, 64), C.randn(g, cu[-1], 4, 64)
    qd, kd, vd = (t.to(dev).requires_grad_() for t in (q, k, v))
    cu_t = torch.tensor(cu, dtype=torch.int32, device=dev)
    native.reset_counters()
    out = varlen_attn(qd, kd, vd, cu_t, cu_t, 79, 79, is_causal=True)
    out.backward(go.to(dev))
    torch.cuda.synchronize()
    c = native.counters()
    assert c["attention"] == 1 and c["attention_backward"] == 1, c
    ref = _varlen_ref_grads(q, k, v, go, cu, cu, True)
    for name, got, want in zip(("dq", "dk", "dv"), (qd.grad, kd.grad, vd.grad), ref):
        err = (got.cpu().double() - want).abs().max().item()
        assert err <= 3e-2 * max(want.abs().max().item(), 1.0), (name, err)
