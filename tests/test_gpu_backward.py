"""GPU parity of the flash backward (``kmi_attn_bwd`` behind the overrideable SDPA
backward): dq, dk, dv of unmasked calls (causal top-left or not, GQA, Sq != Sk, ragged
lengths, head dim 64 / 128, bf16 / fp16) against float64 autograd of the same attention
on the CPU, with the error of torch's CPU autograd at the same dtype as the ruler (the
float64-ruler rule of the forward).  Masked calls keep the fp32 recompute."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import attn_cases as C

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
    # Baseline at the same dtype: torch's CPU autograd in bf16; for fp16 (no CPU fp16
    # SDPA backward here) the float64 result rounded to fp16, the best an fp16 output holds.
    if dtype == torch.bfloat16:
        cpu = _grads(q, k, v, go, causal, dtype)
    else:
        cpu = [r.to(dtype) for r in ref]
    for name, gg, cc, rr in zip(("out", "dq", "dk", "dv"), gpu, cpu, ref):
        ok, sg, sc = C.ruler_ok(gg, cc, rr, factor=2.0, floor=1e-4)
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


def test_masked_calls_keep_the_recompute_backward(native, dev):
    """A masked call's backward is the fp32 recompute (the flash kernels take no mask)."""
    g = C.gen(951)
    q, k, v = (C.randn(g, 1, 2, 64, 64) for _ in range(3))
    mask = torch.randn(1, 1, 64, 64, generator=g).to(torch.bfloat16)
    qd = q.to(dev).requires_grad_()
    native.reset_counters()
    out = F.scaled_dot_product_attention(qd, k.to(dev), v.to(dev), attn_mask=mask.to(dev))
    out.float().sum().backward()
    torch.cuda.synchronize()
    c = native.counters()
    assert c["attention"] == 1 and c["attention_backward"] == 0, c
    q64 = q.double().requires_grad_()
    F.scaled_dot_product_attention(q64, k.double(), v.double(), attn_mask=mask.double()).sum().backward()
    assert (qd.grad.cpu().double() - q64.grad).abs().max().item() < 5e-2


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
    """Gradients through ``kohakutt_amd.sdpa_varlen``: sequences with the dense causal rule
    and no mask take the flash backward kernels, the others the float64 recompute."""
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
    flash = native.counters()["attention_backward"]
    expect = 0 if key_mask is not None else sum(1 for a, b in zip(lq, lk) if not causal or a == b)
    assert flash == expect, (flash, expect)
    ref = _varlen_ref_grads(q, k, v, go, cu_q, cu_k, causal, key_mask)
    for name, got, want in zip(("dq", "dk", "dv"), (qd.grad, kd.grad, vd.grad), ref):
        err = (got.cpu().double() - want).abs().max().item()
        assert err <= 3e-2 * max(want.abs().max().item(), 1.0), (kind, name, err)
