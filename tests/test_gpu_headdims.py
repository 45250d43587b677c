"""GPU parity of head dims up to 256 (multiples of 8 padded to a multiple of 32 inside the
kernels; others zero-padded to a multiple of 8 by the op layer, the output and gradients
narrowed back): dense, causal, masked, decode (split-KV), varlen and the backward, against
the float64 CPU oracle with the BASELINE bar (median relative error at most 1.5x torch
CPU at the same dtype).  The reference's flash takes any head dim that
fits its L1 (``aten_attention.cpp:57-60``, ``ktt_flash/program.cpp:885-893``)."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import attn_cases as C
from oracle import attention as oatt

pytestmark = pytest.mark.gpu

DIMS = [8, 32, 40, 80, 96, 128, 160, 192, 256, 4, 20, 60, 100, 250]


def _check(gpu, cpu, ref, what):
    ok, sg, sc = C.ruler_ok(gpu, cpu, torch.from_numpy(np.ascontiguousarray(ref)), 1.5)
    print(f"{what}: gpu rel_median {sg['rel_median']:.3e} cpu {sc['rel_median']:.3e}", flush=True)
    assert ok, (what, sg, sc)


@pytest.mark.parametrize("d", DIMS)
@pytest.mark.parametrize("kind", ["dense", "causal_gqa", "masked", "decode"])
def test_forward_head_dims(native, dev, d, kind):
    print(f"head dim {d} {kind}", flush=True)
    g = C.gen(3000 + d + len(kind))
    mask = None
    causal = False
    if kind == "dense":
        b, hq, hk, sq, sk = 2, 4, 4, 70, 70
    elif kind == "causal_gqa":
        b, hq, hk, sq, sk, causal = 1, 6, 2, 130, 130, True
    elif kind == "masked":
        b, hq, hk, sq, sk = 2, 4, 2, 50, 90
    else:
        b, hq, hk, sq, sk = 3, 8, 2, 1, 700
    q = C.randn(g, b, hq, sq, d)
    k = C.randn(g, b, hk, sk, d)
    v = C.randn(g, b, hk, sk, d)
    if kind == "masked":
        mask = torch.randn(b, 1, sq, sk, generator=g).masked_fill(torch.rand(b, 1, sq, sk, generator=g) < 0.2,
                                                                   float("-inf"))
        mask[..., 0] = 0.0
    if kind == "decode":
        lens = torch.tensor([700, 33, 401])
        mask = (torch.arange(sk)[None, :] < lens[:, None]).reshape(b, 1, 1, sk)
    native.reset_counters()
    out = F.scaled_dot_product_attention(q.to(dev), k.to(dev), v.to(dev),
                                         attn_mask=None if mask is None else mask.to(dev), is_causal=causal,
                                         enable_gqa=hq != hk)
    torch.cuda.synchronize()
    assert native.counters()["attention"] == 1, native.counters()
    m64 = None if mask is None else (mask.numpy() if mask.dtype == torch.bool else C.f64(mask))
    ref, _ = oatt.sdpa(C.f64(q), C.f64(k), C.f64(v), m64, causal)
    _check(out.cpu(), C.torch_cpu_sdpa(q, k, v, mask, causal), ref, f"D={d} {kind}")


@pytest.mark.parametrize("d", [40, 96, 256, 60])
def test_varlen_head_dims(native, dev, d):
    g = C.gen(3100 + d)
    cu = [0, 37, 38, 200]
    q = C.randn(g, cu[-1], 4, d)
    k = C.randn(g, cu[-1], 2, d)
    v = C.randn(g, cu[-1], 2, d)
    native.reset_counters()
    out = native.sdpa_varlen(q.to(dev), k.to(dev), v.to(dev), cu, is_causal=True).cpu()
    assert native.counters()["attention"] == 1
    ref, _ = oatt.sdpa_varlen(C.f64(q), C.f64(k), C.f64(v), cu, is_causal=True)
    cpu = []
    for a, b in zip(cu[:-1], cu[1:]):
        n = b - a
        cpu.append(F.scaled_dot_product_attention(
            q[a:b].transpose(0, 1)[None], k[a:b].transpose(0, 1)[None].repeat_interleave(2, 1),
            v[a:b].transpose(0, 1)[None].repeat_interleave(2, 1),
            attn_mask=torch.ones(n, n, dtype=torch.bool).tril())[0].transpose(0, 1))
    _check(out, torch.cat(cpu), ref, f"varlen D={d}")


def _grads(q, k, v, go, causal, dtype, dev=None, mask=None):
    hq, hk = q.size(1), k.size(1)
    ts = [t.to(dtype) for t in (q, k, v)]
    if dev is not None:
        ts = [t.to(dev) for t in ts]
    ts = [t.detach().requires_grad_() for t in ts]
    qq, kk, vv = ts
    m = None if mask is None else (mask.to(dev) if dev is not None else mask)
    if m is not None and m.is_floating_point():
        m = m.to(dtype)
    if dev is None:
        out = F.scaled_dot_product_attention(qq, kk.repeat_interleave(hq // hk, 1), vv.repeat_interleave(hq // hk, 1),
                                             attn_mask=m, is_causal=causal)
    else:
        out = F.scaled_dot_product_attention(qq, kk, vv, attn_mask=m, is_causal=causal, enable_gqa=hq != hk)
    out.backward(go.to(dtype).to(dev) if dev is not None else go.to(dtype))
    return [t.detach().cpu() for t in (out, qq.grad, kk.grad, vv.grad)]


@pytest.mark.parametrize("d", [32, 80, 96, 192, 256, 20, 100, 250])
def test_backward_head_dims(native, dev, d):
    print(f"backward head dim {d}", flush=True)
    g = C.gen(3200 + d)
    b, hq, hk, s = 1, 4, 2, 100
    q, k, v, go = (C.randn(g, *sh, dtype=torch.float32) for sh in ((b, hq, s, d), (b, hk, s, d), (b, hk, s, d),
                                                                    (b, hq, s, d)))
    q, k, v, go = (t.bfloat16().float() for t in (q, k, v, go))
    native.reset_counters()
    gpu = _grads(q, k, v, go, True, torch.bfloat16, dev)
    torch.cuda.synchronize()
    c = native.counters()
    assert c["attention_backward"] == 1, c
    ref = _grads(q, k, v, go, True, torch.float64)
    cpu = _grads(q, k, v, go, True, torch.bfloat16)
    for name, gg, cc, rr in zip(("out", "dq", "dk", "dv"), gpu, cpu, ref):
        ok, sg, sc = C.ruler_ok(gg, cc, rr, factor=1.5)
        print(f"  {name}: gpu {sg['rel_median']:.2e} cpu {sc['rel_median']:.2e}", flush=True)
        assert ok, (d, name, sg, sc)


def test_varlen_odd_dims_forward_and_backward(native, dev):
    """Varlen with q / k and v head dims that are not multiples of 8 (60 and 100): the op
    layer pads both, the outputs and gradients come back at the caller's dims."""
    g = C.gen(3300)
    cu = [0, 37, 38, 120]
    q, k = C.randn(g, cu[-1], 4, 60), C.randn(g, cu[-1], 2, 60)
    v, go = C.randn(g, cu[-1], 2, 100), C.randn(g, cu[-1], 4, 100)
    qd, kd, vd = (t.to(dev).requires_grad_() for t in (q, k, v))
    native.reset_counters()
    out = native.sdpa_varlen(qd, kd, vd, cu, is_causal=True)
    assert out.shape == (cu[-1], 4, 100)
    out.backward(go.to(dev))
    torch.cuda.synchronize()
    c = native.counters()
    assert c["attention"] == 1 and c["attention_backward"] == 1, c
    assert qd.grad.shape == q.shape and kd.grad.shape == k.shape and vd.grad.shape == v.shape
    ref, _ = oatt.sdpa_varlen(C.f64(q), C.f64(k), C.f64(v), cu, is_causal=True)
    assert np.abs(out.detach().cpu().double().numpy() - ref).max() < 2e-2
    # float64 autograd per sequence
    grads = [torch.zeros(t.shape, dtype=torch.float64) for t in (q, k, v)]
    for a, b in zip(cu[:-1], cu[1:]):
        qs, ks, vs = (t.double().transpose(0, 1)[None].requires_grad_() for t in (q[a:b], k[a:b], v[a:b]))
        o = F.scaled_dot_product_attention(qs, ks.repeat_interleave(2, 1), vs.repeat_interleave(2, 1),
                                           attn_mask=torch.ones(b - a, b - a, dtype=torch.bool).tril())
        o.backward(go[a:b].double().transpose(0, 1)[None])
        for gs, t in zip(grads, (qs, ks, vs)):
            gs[a:b] = t.grad[0].transpose(0, 1)
    for name, got, want in zip(("dq", "dk", "dv"), (qd.grad, kd.grad, vd.grad), grads):
        err = (got.cpu().double() - want).abs().max().item()
        assert err <= 3e-2 * max(want.abs().max().item(), 1.0), (name, err)
