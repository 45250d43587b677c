"""kmi_attn_fwd_noalloc (the forward that allocates nothing: split-KV partials in the
library's per-device scratch array) against kmi_attn_fwd with a workspace from the caller:
bit-identical outputs and LSE, on two calls in a row, the second smaller, so the second
reads nothing the first left in the scratch; a call whose partials exceed the scratch is
refused before anything is launched."""

from __future__ import annotations

import ctypes

import pytest
import torch

import attn_cases as C

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 16 << 20


def _args(q, k, v, mask, num_splits):
    from kohakutt_amd import capi

    b, hq, sq, d = q.shape
    out = torch.empty_like(q)
    lse = torch.empty(b, hq, sq, dtype=torch.float32, device=q.device)
    a = capi.AttnArgs(
        q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(), out=out.data_ptr(), lse=lse.data_ptr(),
        dtype=capi.KMI_BF16, causal=0, batch=b, heads_q=hq, heads_kv=k.size(1), seq_q=sq,
        seq_k=k.size(2), head_dim=d, scale=d**-0.5, num_splits=num_splits,
    )
    a.q_stride[:] = q.stride()[:3]
    a.k_stride[:] = k.stride()[:3]
    a.v_stride[:] = v.stride()[:3]
    a.o_stride[:] = out.stride()[:3]
    a.lse_stride[:] = lse.stride()
    if mask is not None:
        a.mask = mask.data_ptr()
        a.mask_dtype = capi.KMI_BOOL
        a.mask_mode = capi.KMI_MASK_STRIDED
        a.mask_stride[:] = [mask.stride(0), 0, 0, mask.stride(3)]
    return a, out, lse


def _both(q, k, v, mask, num_splits):
    """The same call through kmi_attn_fwd (fresh workspace) and kmi_attn_fwd_noalloc."""
    from kohakutt_amd import capi

    stream = torch.cuda.current_stream().cuda_stream
    a, out, lse = _args(q, k, v, mask, num_splits)
    n = capi.workspace_bytes(a)
    assert 0 < n <= SCRATCH_BYTES, n
    ws = torch.full((n,), 0xFF, dtype=torch.uint8, device=q.device)
    capi.attn_fwd(a, ws.data_ptr(), n, stream)
    b, out2, lse2 = _args(q, k, v, mask, num_splits)
    capi.attn_fwd_noalloc(b, stream)
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu(), out2.cpu(), lse2.cpu()


def _decode(g, b, hk, sk, d, lengths):
    q = C.randn(g, b, 4 * hk, 1, d).cuda()
    k = C.randn(g, b, hk, sk, d).cuda()
    v = C.randn(g, b, hk, sk, d).cuda()
    mask = (torch.arange(sk)[None, :] < torch.tensor(lengths)[:, None]).reshape(b, 1, 1, sk).cuda()
    return q, k, v, mask


def test_noalloc_matches_workspace_entry_on_two_calls(native):
    g = C.gen(900)
    print("call 1: B=6 Hq=8 Hkv=2 Sk=2000 D=128, plan's splits", flush=True)
    q, k, v, m = _decode(g, 6, 2, 2000, 128, [1, 5, 1999, 700, 64, 2000])
    o, l, o2, l2 = _both(q, k, v, m, 0)
    assert torch.isfinite(o.float()).all()
    assert torch.equal(o, o2) and torch.equal(l, l2)
    print("call 2: B=2 Hq=8 Hkv=2 Sk=700 D=96, 7 splits", flush=True)
    q, k, v, m = _decode(g, 2, 2, 700, 96, [700, 300])
    o, l, o2, l2 = _both(q, k, v, m, 7)
    assert torch.isfinite(o.float()).all()
    assert torch.equal(o, o2) and torch.equal(l, l2)
    print("call 3: B=1 Hq=4 Hkv=4 Sq=1 Sk=64 D=64, no split (no scratch)", flush=True)
    from kohakutt_amd import capi

    q = C.randn(g, 1, 4, 1, 64).cuda()
    k = C.randn(g, 1, 4, 64, 64).cuda()
    a, out, _ = _args(q, k, k, None, 1)
    assert capi.workspace_bytes(a) == 0
    capi.attn_fwd_noalloc(a, torch.cuda.current_stream().cuda_stream)
    a1, out1, _ = _args(q, k, k, None, 1)
    capi.attn_fwd(a1, None, 0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), out1.cpu())


def test_noalloc_refuses_partials_beyond_its_scratch(native):
    from kohakutt_amd import capi

    q = torch.zeros(16, 32, 1, 256, dtype=torch.bfloat16, device="cuda")
    k = torch.zeros(16, 8, 8192, 256, dtype=torch.bfloat16, device="cuda")
    a, out, _ = _args(q, k, k, None, 32)
    assert capi.workspace_bytes(a) > SCRATCH_BYTES
    out.fill_(0)
    torch.cuda.synchronize()
    status = capi.lib().kmi_attn_fwd_noalloc(ctypes.byref(a), None)
    assert status == capi.KMI_EUNSUPPORTED
    assert "split-KV scratch" in capi.lib().kmi_last_error().decode()
    torch.cuda.synchronize()
    assert (out == 0).all()
