"""GPU parity of value head dims that differ from the query / key head dim (Dv != D):
the reference's packed op takes v [Tk, Hk, Dv] and returns out [Tq, H, Dv]
(``aten_varlen.cpp:160-208``), and its backward returns dv shaped like v
(``aten_varlen.cpp:237-319``).  The kernels run at the larger dim, padded; these tests
check the forward (the prefill kernel, the decode kernel and its split merge, packed
masks, dense calls through the C ABI) and the backward against float64 under the 1.5x
ruler.

The same-dtype baseline is torch's CPU SDPA in bf16 on the same attention with the
narrower operand zero-padded to the wider dim (q and k, or v; the scale passed as
1 / sqrt(D); padded output and gradient columns dropped), which is the same mathematics.
Unpadded, torch routes Dv != D to its math path, which upcasts bf16 to fp32 and leaves
only the final rounding: that is not a bf16 computation (measured: the kernels' errors
are the same for Dv != D as for Dv == D, while that path's error drops by a third)."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import attn_cases as C
from oracle import attention as oatt

pytestmark = pytest.mark.gpu

# (D, Dv): each direction, a padded dim that differs only in its padding, the widest.
DIMS = [(128, 64), (64, 128), (192, 128), (96, 32), (32, 96), (64, 256), (120, 72)]


def _pad(t, width):
    """t with zero columns appended to ``width`` in its last dim."""
    return F.pad(t, (0, width - t.size(-1))) if t.size(-1) < width else t


def _per_sequence(q, k, v, go, cu_q, cu_k, causal, dtype):
    """out and (dq, dk, dv) of per-sequence CPU SDPA autograd at ``dtype`` (bottom-right
    causal), packed as the inputs.  Below float64 the narrower operand is zero-padded to
    the wider dim (the bf16 kernel; see the module docstring)."""
    hq, hk, d, dv = q.size(1), k.size(1), q.size(2), v.size(2)
    if dtype != torch.float64 and d != dv:
        w = max(d, dv)
        res = _per_sequence_at(_pad(q, w), _pad(k, w), _pad(v, w), _pad(go, w), cu_q, cu_k, causal, dtype, d ** -0.5)
        return [res[0][..., :dv], res[1][..., :d], res[2][..., :d], res[3][..., :dv]]
    return _per_sequence_at(q, k, v, go, cu_q, cu_k, causal, dtype, d ** -0.5)


def _per_sequence_at(q, k, v, go, cu_q, cu_k, causal, dtype, scale):
    hq, hk = q.size(1), k.size(1)
    out = torch.zeros(q.size(0), hq, v.size(2), dtype=torch.float64)
    grads = [torch.zeros(t.shape, dtype=torch.float64) for t in (q, k, v)]
    for s in range(len(cu_q) - 1):
        a, b, c, d = cu_q[s], cu_q[s + 1], cu_k[s], cu_k[s + 1]
        lq, lk = b - a, d - c
        if lq == 0:
            continue
        qs, ks, vs = (t.to(dtype).transpose(0, 1)[None].detach().requires_grad_() for t in (q[a:b], k[c:d], v[c:d]))
        keep = torch.ones(lq, lk, dtype=torch.bool)
        if causal:
            keep &= torch.arange(lk)[None, :] <= torch.arange(lq)[:, None] + (lk - lq)
        o = F.scaled_dot_product_attention(qs, ks.repeat_interleave(hq // hk, 1), vs.repeat_interleave(hq // hk, 1),
                                           attn_mask=keep, scale=scale)
        o.backward(go[a:b].to(dtype).transpose(0, 1)[None])
        out[a:b] = o.detach()[0].transpose(0, 1).double()
        for gsum, t, (lo, hi) in zip(grads, (qs, ks, vs), ((a, b), (c, d), (c, d))):
            gsum[lo:hi] = t.grad[0].transpose(0, 1).double()
    return [out] + grads


def _offsets(lens):
    return [0] + torch.tensor(lens).cumsum(0).tolist()


@pytest.mark.parametrize("dims", DIMS, ids=lambda t: f"d{t[0]}_dv{t[1]}")
def test_varlen_forward_and_backward(native, dev, dims):
    d, dv = dims
    print(f"value dim case D={d} Dv={dv}", flush=True)
    g = C.gen(1500 + d + 3 * dv)
    lq, lk = [37, 1, 130, 64], [50, 9, 130, 200]
    cu_q, cu_k = _offsets(lq), _offsets(lk)
    hq, hk = 8, 2
    # Inputs rounded to bf16 first: every path sees the same values.
    q = C.randn(g, cu_q[-1], hq, d).float()
    k = C.randn(g, cu_k[-1], hk, d).float()
    v = C.randn(g, cu_k[-1], hk, dv).float()
    go = C.randn(g, cu_q[-1], hq, dv).float()
    qd, kd, vd = (t.to(dev).bfloat16().requires_grad_() for t in (q, k, v))
    native.reset_counters()
    out = native.sdpa_varlen(qd, kd, vd, cu_q, cu_k, is_causal=True)
    assert out.shape == (cu_q[-1], hq, dv)
    out.backward(go.to(dev).bfloat16())
    torch.cuda.synchronize()
    c = native.counters()
    assert c["attention"] == 1 and c["attention_backward"] == 1, c
    ref_out, _ = oatt.sdpa_varlen(C.f64(q), C.f64(k), C.f64(v), cu_q, cu_k, is_causal=True)
    ref = _per_sequence(q, k, v, go, cu_q, cu_k, True, torch.float64)
    assert np.abs(ref[0].numpy() - ref_out).max() < 1e-10
    cpu = _per_sequence(q, k, v, go, cu_q, cu_k, True, torch.bfloat16)
    got = [out.detach(), qd.grad, kd.grad, vd.grad]
    for name, gg, cc, rr in zip(("out", "dq", "dk", "dv"), got, cpu, ref):
        assert gg.shape == rr.shape, (name, gg.shape, rr.shape)
        ok, sg, sc = C.ruler_ok(gg.cpu(), cc, rr, factor=1.5)
        print(f"  {name}: gpu rel_median {sg['rel_median']:.2e}  cpu {sc['rel_median']:.2e}", flush=True)
        assert ok, (dims, name, sg, sc)


@pytest.mark.parametrize("dims", [(128, 64), (64, 128)], ids=lambda t: f"d{t[0]}_dv{t[1]}")
def test_reference_op_and_packed_mask(native, dev, dims):
    """The reference-schema op (``_varlen_plan`` + ``_sdpa_varlen`` with statistics, then
    ``_sdpa_varlen_backward``) and this build's packed per-row mask, with Dv != D."""
    d, dv = dims
    g = C.gen(1600 + d + dv)
    cu_q, cu_k = [0, 30, 31, 120], [0, 40, 41, 150]
    hq, hk = 4, 2
    scale = d ** -0.5
    q, k = C.randn(g, cu_q[-1], hq, d), C.randn(g, cu_k[-1], hk, d)
    v, go = C.randn(g, cu_k[-1], hk, dv), C.randn(g, cu_q[-1], hq, dv)
    records, masks = torch.ops.ktt._varlen_plan(cu_q, cu_k, True, scale, False)
    records, masks = records.to(dev), masks.to(dev)
    qd, kd, vd = (t.to(dev).requires_grad_() for t in (q, k, v))
    out, lse = torch.ops.ktt._sdpa_varlen(qd, kd, vd, records, masks, cu_q, cu_k, True, scale, True, None, False)
    assert out.shape == (cu_q[-1], hq, dv) and lse.shape == (hq, cu_q[-1])
    ref_out, ref_lse = oatt.sdpa_varlen(C.f64(q), C.f64(k), C.f64(v), cu_q, cu_k, is_causal=True)
    assert np.abs(out.detach().cpu().double().numpy() - ref_out).max() < 2e-2
    assert np.abs(lse.detach().cpu().double().numpy() - ref_lse).max() < 2e-2
    dq, dk, dvg = torch.ops.ktt._sdpa_varlen_backward(go.to(dev), out.detach(), qd.detach(), kd.detach(),
                                                      vd.detach(), records, masks, records, masks, cu_q, cu_k, True,
                                                      scale, None)
    assert dq.shape == q.shape and dk.shape == k.shape and dvg.shape == v.shape
    ref = _per_sequence(q.float(), k.float(), v.float(), go.float(), cu_q, cu_k, True, torch.float64)
    for name, got, want in zip(("dq", "dk", "dv"), (dq, dk, dvg), ref[1:]):
        err = (got.cpu().double() - want).abs().max().item()
        assert err <= 3e-2 * max(want.abs().max().item(), 1.0), (name, err)
    # A packed per-row mask (every sequence's [Lq_i, Lk_i] block): 20% of keys dropped,
    # the first key of every row kept.
    lq = [b - a for a, b in zip(cu_q, cu_q[1:])]
    lk = [b - a for a, b in zip(cu_k, cu_k[1:])]
    blocks = []
    for a, b in zip(lq, lk):
        m = torch.rand(a, b, generator=g) > 0.2
        m[:, 0] = True
        blocks.append(m.reshape(-1))
    pm = torch.cat(blocks)
    outm = native.sdpa_varlen(qd.detach(), kd.detach(), vd.detach(), cu_q, cu_k, is_causal=True, packed_mask=pm.to(dev))
    refm, _ = oatt.sdpa_varlen(C.f64(q), C.f64(k), C.f64(v), cu_q, cu_k, is_causal=True, attn_mask=pm.numpy())
    assert outm.shape == (cu_q[-1], hq, dv)
    assert np.abs(outm.cpu().double().numpy() - refm).max() < 2e-2


@pytest.mark.parametrize("dims", [(128, 64), (64, 128), (96, 256)], ids=lambda t: f"d{t[0]}_dv{t[1]}")
def test_decode_split_merge(native, dev, dims):
    """One query per sequence (the decode kernel): long sequences split their keys over
    workgroups and merge in the same launch, short ones take one workgroup."""
    d, dv = dims
    g = C.gen(1700 + d + dv)
    lk = [3000, 17, 1, 900, 2048, 64]
    cu_q, cu_k = list(range(len(lk) + 1)), _offsets(lk)
    hq, hk = 8, 1
    q, k, v = C.randn(g, len(lk), hq, d), C.randn(g, cu_k[-1], hk, d), C.randn(g, cu_k[-1], hk, dv)
    native.reset_counters()
    out, lse = torch.ops.ktt._sdpa_varlen_offsets(
        q.to(dev), k.to(dev), v.to(dev), torch.tensor(cu_q, dtype=torch.int32, device=dev),
        torch.tensor(cu_k, dtype=torch.int32, device=dev), 1, max(lk), True, None, None, None,
    )
    torch.cuda.synchronize()
    assert native.counters()["attention"] == 1
    assert out.shape == (len(lk), hq, dv)
    ref, ref_lse = oatt.sdpa_varlen(C.f64(q), C.f64(k), C.f64(v), cu_q, cu_k, is_causal=True)
    w = max(d, dv)
    cpu = torch.cat([C.torch_cpu_sdpa(_pad(q[i:i + 1], w).transpose(0, 1)[None],
                                      _pad(k[cu_k[i]:cu_k[i + 1]], w).transpose(0, 1)[None],
                                      _pad(v[cu_k[i]:cu_k[i + 1]], w).transpose(0, 1)[None], scale=d ** -0.5)[0]
                     .transpose(0, 1)[..., :dv] for i in range(len(lk))])
    ok, sg, sc = C.ruler_ok(out.cpu(), cpu, torch.from_numpy(ref), factor=1.5)
    assert ok, (dims, sg, sc)
    assert np.abs(lse.cpu().double().numpy() - ref_lse).max() < 2e-2


@pytest.mark.parametrize("dims", [(64, 128), (128, 32)], ids=lambda t: f"d{t[0]}_dv{t[1]}")
def test_dense_calls_through_the_c_abi(native, dev, dims):
    """kmi_attn_fwd takes head_dim_v on dense calls too: causal prefill and a bool-masked
    decode against the float64 oracle."""
    from kohakutt_amd import capi

    d, dv = dims
    g = C.gen(1800 + d + dv)
    for sq, sk, causal in ((300, 300, True), (1, 2500, False)):
        b, hq, hk = 2, 8, 2
        q, k, v = C.randn(g, b, hq, sq, d), C.randn(g, b, hk, sk, d), C.randn(g, b, hk, sk, dv)
        mask = None if causal else torch.rand(b, 1, 1, sk, generator=g) > 0.3
        qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
        out = torch.empty(b, hq, sq, dv, dtype=q.dtype, device=dev)
        a = capi.AttnArgs(q=qd.data_ptr(), k=kd.data_ptr(), v=vd.data_ptr(), out=out.data_ptr(), dtype=capi.KMI_BF16,
                          causal=int(causal), batch=b, heads_q=hq, heads_kv=hk, seq_q=sq, seq_k=sk, head_dim=d,
                          head_dim_v=dv, scale=d ** -0.5)
        a.q_stride[:] = qd.stride()[:3]
        a.k_stride[:] = kd.stride()[:3]
        a.v_stride[:] = vd.stride()[:3]
        a.o_stride[:] = out.stride()[:3]
        md = None
        if mask is not None:
            md = mask.to(dev)
            a.mask, a.mask_dtype, a.mask_mode = md.data_ptr(), capi.KMI_BOOL, capi.KMI_MASK_STRIDED
            a.mask_stride[:] = [md.stride(0), 0, 0, md.stride(3)]
        n = capi.workspace_bytes(a)
        ws = torch.empty(max(n, 1), dtype=torch.uint8, device=dev)
        capi.attn_fwd(a, ws.data_ptr(), n, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        ref, _ = oatt.sdpa(C.f64(q), C.f64(k), C.f64(v), attn_mask=None if mask is None else mask.numpy(),
                           is_causal=causal)
        w = max(d, dv)
        cpu = C.torch_cpu_sdpa(_pad(q, w), _pad(k, w), _pad(v, w), mask=mask, causal=causal, scale=d ** -0.5)[..., :dv]
        ok, sg, sc = C.ruler_ok(out.cpu(), cpu, torch.from_numpy(ref), factor=1.5)
        assert ok, (dims, sq, sk, sg, sc)
