"""GPU parity of the key-lengths route (``ktt::_sdpa_lengths``, the reference's
``aten_lengths.cpp:69-101`` behind ``kohakutt.sdpa(key_lengths=)``): the kernels take a
per-batch key count instead of a mask.  Checked against the float64 oracle
(``oracle.attention.sdpa_lengths``) on the decode kernel (split and unsplit), the prefill
kernel (causal GQA, non-causal Sq != Sk) and the row-split paths (short key ranges),
with lengths of 1, Sk and ragged values; out-of-range device lengths clamp to [1, Sk];
the backward (fp32 recompute) against float64 autograd."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import attn_cases as C
from oracle import attention as oatt

pytestmark = pytest.mark.gpu

CASES = {
    # name: (B, Hq, Hk, Sq, Sk, D, causal, lengths)
    "c3_decode": None,  # BASELINE config 3 shape with its own lengths
    "decode_ragged_d64": (5, 8, 1, 1, 900, 64, False, [1, 900, 33, 32, 640]),
    "decode_two_rows": (3, 16, 2, 1, 5000, 128, False, [4999, 77, 2500]),
    "prefill_causal_gqa": (3, 14, 2, 300, 300, 64, True, [300, 1, 131]),
    "prefill_causal_d128": (2, 16, 8, 257, 257, 128, True, [200, 257]),
    "prefill_cross_sq_ne_sk": (2, 4, 4, 70, 500, 64, False, [500, 64]),
    "row_split_vit": (4, 12, 12, 197, 197, 64, False, [197, 1, 100, 64]),
    "row_split_staged": (3, 10, 10, 300, 77, 64, False, [77, 5, 40]),
}


def _case(name, dtype=torch.bfloat16):
    if name == "c3_decode":
        c = C.config3(dtype)
        return c["q"], c["k"], c["v"], c["lengths"].tolist(), False
    b, hq, hk, sq, sk, d, causal, lengths = CASES[name]
    g = C.gen(700 + sum(map(ord, name)))
    q = C.randn(g, b, hq, sq, d, dtype=dtype)
    k = C.randn(g, b, hk, sk, d, dtype=dtype)
    v = C.randn(g, b, hk, sk, d, dtype=dtype)
    return q, k, v, lengths, causal


@pytest.mark.parametrize("name", list(CASES))
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_lengths_match_oracle(native, dev, name, dtype):
    q, k, v, lengths, causal = _case(name, dtype)
    print(f"lengths case {name} {dtype} q{tuple(q.shape)} k{tuple(k.shape)}", flush=True)
    ln = torch.tensor(lengths, dtype=torch.int32, device=dev)
    native.reset_counters()
    out = torch.ops.ktt._sdpa_lengths(q.to(dev), k.to(dev), v.to(dev), ln, causal, None, False)
    torch.cuda.synchronize()
    assert native.counters()["attention"] == 1
    ref, _ = oatt.sdpa_lengths(C.f64(q), C.f64(k), C.f64(v), lengths, is_causal=causal)
    err = np.abs(out.cpu().double().numpy() - ref)
    assert err.max() < 2e-2, (name, err.max())
    assert err.mean() < 2e-3, (name, err.mean())
    # The package entry point (host list of lengths) takes the same kernel route.
    native.reset_counters()
    again = native.sdpa(q.to(dev), k.to(dev), v.to(dev), key_lengths=lengths, is_causal=causal)
    torch.cuda.synchronize()
    assert native.counters()["attention"] == 1
    assert torch.equal(again, out)


def test_c3_lengths_meet_the_float64_ruler(native, dev):
    """Config 3 through key lengths: median relative error against float64 at most 1.5x
    torch CPU bf16 SDPA with the equivalent padding mask (the BASELINE tolerance)."""
    c = C.config3()
    q, k, v, lengths = c["q"], c["k"], c["v"], c["lengths"]
    out = native.sdpa(q.to(dev), k.to(dev), v.to(dev), key_lengths=lengths.to(dev))
    torch.cuda.synchronize()
    ref, _ = oatt.sdpa_lengths(C.f64(q), C.f64(k), C.f64(v), lengths.tolist())
    cpu = C.torch_cpu_sdpa(q, k, v, mask=c["mask"])
    ok, sg, sc = C.ruler_ok(out.cpu(), cpu, torch.from_numpy(ref))
    assert ok, (sg, sc)


def test_device_lengths_clamp_to_the_key_range(native, dev):
    """Device lengths are not checked on the host: the kernels clamp them to [1, Sk]
    (``flash.md`` "Key lengths"), bit-identical to the clamped values."""
    q, k, v, _, _ = _case("decode_ragged_d64")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    wild = torch.tensor([0, -7, 10**6, 900, 2], dtype=torch.int32, device=dev)
    tame = torch.tensor([1, 1, 900, 900, 2], dtype=torch.int32, device=dev)
    a = torch.ops.ktt._sdpa_lengths(qd, kd, vd, wild, False, None, False)
    b = torch.ops.ktt._sdpa_lengths(qd, kd, vd, tame, False, None, False)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_lengths_match_the_mask_route(native, dev):
    """The kernel route and the explicit-mask route (a bool padding mask through the same
    kernels) agree to bf16 rounding on a causal GQA prefill."""
    q, k, v, lengths, causal = _case("prefill_causal_gqa")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    ln = torch.tensor(lengths, dtype=torch.int32, device=dev)
    a = torch.ops.ktt._sdpa_lengths(qd, kd, vd, ln, causal, None, False)
    from kohakutt_amd.attention import _padding_mask

    keep = _padding_mask(ln, qd.size(2), kd.size(2), causal)
    b = F.scaled_dot_product_attention(qd, kd, vd, attn_mask=keep, enable_gqa=qd.size(1) != kd.size(1))
    torch.cuda.synchronize()
    assert (a.float() - b.float()).abs().max().item() < 2e-2


@pytest.mark.parametrize("causal", [False, True])
def test_lengths_backward_matches_float64_autograd(native, dev, causal):
    """Gradients through ``kohakutt_amd.sdpa(key_lengths=)``: dq, dk, dv against float64
    autograd of the oracle's semantics; keys past a length get exactly zero dk, dv."""
    g = C.gen(777 + causal)
    b, hq, hk, s, d = 3, 4, 2, 96, 64
    q = C.randn(g, b, hq, s, d)
    k = C.randn(g, b, hk, s, d)
    v = C.randn(g, b, hk, s, d)
    go = C.randn(g, b, hq, s, d)
    lengths = [96, 1, 50]
    qd, kd, vd = (t.to(dev).requires_grad_() for t in (q, k, v))
    out = native.sdpa(qd, kd, vd, key_lengths=lengths, is_causal=causal)
    out.backward(go.to(dev))
    torch.cuda.synchronize()

    q64, k64, v64 = (t.double().requires_grad_() for t in (q, k, v))
    keys = torch.arange(s)
    keep = (keys[None, :] < torch.tensor(lengths)[:, None])[:, None, None, :]
    if causal:
        keep = keep & (keys[None, :] <= torch.arange(s)[:, None])[None, None]
    ref = torch.nn.functional.scaled_dot_product_attention(
        q64, k64.repeat_interleave(hq // hk, 1), v64.repeat_interleave(hq // hk, 1), attn_mask=keep
    )
    ref.backward(go.double())
    assert (out.detach().cpu().double() - ref.detach()).abs().max().item() < 2e-2
    for got, want, name in ((qd.grad, q64.grad, "dq"), (kd.grad, k64.grad, "dk"), (vd.grad, v64.grad, "dv")):
        err = (got.cpu().double() - want).abs()
        scale = want.abs().max().item()
        assert err.max().item() < 2e-2 * max(scale, 1.0), (name, err.max().item(), scale)
    assert kd.grad[1, :, 1:].abs().max().item() == 0.0
    assert vd.grad[2, :, 50:].abs().max().item() == 0.0
