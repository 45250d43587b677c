"""GPU parity of the decode path (at most 16 query rows per K/V head): the kernel that
deals key tiles round-robin to wavefronts, skips tiles of a shared padding mask whose keys
are all masked, merges its wavefronts in LDS and either writes the output (one workgroup
per unit) or fp32 partials for the split merge.  Checked against the float64 oracle,
including the reference's fully-masked-row rule (softmax over raw scores,
``aten_attention.cpp:139-140`` clamp at -5e5), which no CPU torch call reproduces."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import attn_cases as C
from oracle import attention as oatt

pytestmark = pytest.mark.gpu


def _padding(lengths, sk):
    lengths = torch.tensor(lengths)
    return (torch.arange(sk)[None, :] < lengths[:, None]).reshape(len(lengths), 1, 1, sk)


def _case(name):
    g = C.gen(300 + sum(map(ord, name)))
    if name == "padding_with_empty_rows":
        q, k = C.randn(g, 6, 8, 1, 128), C.randn(g, 6, 2, 2000, 128)
        mask = _padding([0, 5, 1999, 700, 64, 65], 2000)
    elif name == "kept_keys_only_late":
        q, k = C.randn(g, 2, 8, 1, 128), C.randn(g, 2, 2, 2000, 128)
        mask = torch.zeros(2, 1, 1, 2000, dtype=torch.bool)
        mask[..., 1500:] = True
    elif name == "per_head_mask":
        q, k = C.randn(g, 3, 8, 1, 64), C.randn(g, 3, 2, 900, 64)
        mask = torch.rand(3, 8, 1, 900, generator=g) > 0.5
        mask[1, 3] = False  # one fully masked row
    elif name == "additive_f32_padding":
        q, k = C.randn(g, 4, 16, 1, 128), C.randn(g, 4, 2, 1500, 128)
        mask = torch.randn(4, 1, 1, 1500, generator=g)
        mask = mask.masked_fill(~_padding([100, 1500, 1, 777], 1500), float("-inf"))
    elif name == "gqa_two_queries":
        q, k = C.randn(g, 2, 8, 2, 128), C.randn(g, 2, 2, 1200, 128)
        mask = _padding([300, 1200], 1200)
    elif name == "one_workgroup_per_unit":
        q, k = C.randn(g, 64, 32, 1, 64), C.randn(g, 64, 8, 300, 64)
        mask = None
    elif name == "one_workgroup_per_unit_masked":
        q, k = C.randn(g, 64, 16, 1, 64), C.randn(g, 64, 8, 700, 64)
        mask = _padding(torch.randint(1, 701, (64,), generator=g).tolist(), 700)
    elif name == "long_cache":
        q, k = C.randn(g, 1, 8, 1, 64), C.randn(g, 1, 1, 70000, 64)
        mask = _padding([51234], 70000)
    else:
        raise KeyError(name)
    v = C.randn(g, *k.shape)
    return q, k, v, mask


@pytest.mark.parametrize(
    "name",
    [
        "padding_with_empty_rows",
        "kept_keys_only_late",
        "per_head_mask",
        "additive_f32_padding",
        "gqa_two_queries",
        "one_workgroup_per_unit",
        "one_workgroup_per_unit_masked",
        "long_cache",
    ],
)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_matches_oracle(native, dev, name, dtype):
    q, k, v, mask = _case(name)
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    print(f"decode case {name} {dtype} q{tuple(q.shape)} k{tuple(k.shape)}", flush=True)
    native.reset_counters()
    out = F.scaled_dot_product_attention(
        q.to(dev), k.to(dev), v.to(dev), attn_mask=None if mask is None else mask.to(dev),
        enable_gqa=q.size(1) != k.size(1),
    )
    torch.cuda.synchronize()
    assert native.counters()["attention"] == 1
    m64 = None if mask is None else (mask.numpy() if mask.dtype == torch.bool else C.f64(mask))
    ref, _ = oatt.sdpa(C.f64(q), C.f64(k), C.f64(v), m64)
    out = out.cpu()
    # Rows that keep a key: the ruler against torch CPU at the same dtype (1.5x its median
    # relative error against float64).  Rows whose every key is masked follow the
    # reference (softmax over the raw scores) where torch CPU returns zeros, so they are
    # compared with the oracle alone.
    if m64 is None:
        kept = np.ones(out.shape[:-1], dtype=bool)
    else:
        keeps = m64 if m64.dtype == np.bool_ else m64 > -5e5
        kept = np.broadcast_to(keeps.any(-1), out.shape[:-1])
    cpu = C.torch_cpu_sdpa(q, k, v, mask)
    sel = torch.from_numpy(np.ascontiguousarray(kept))
    ok, sg, sc = C.ruler_ok(out[sel], cpu[sel], torch.from_numpy(np.ascontiguousarray(ref[kept])))
    print(f"  kept rows: gpu rel_median {sg['rel_median']:.3e} cpu {sc['rel_median']:.3e}", flush=True)
    assert ok, (name, sg, sc)
    if (~kept).any():
        err = np.abs(out.double().numpy()[~kept] - ref[~kept])
        assert err.max() < 2e-2, (name, err.max())


@pytest.mark.parametrize("nseq,hk", [(8, 2), (600, 1)])
def test_varlen_decode_output_and_lse(native, dev, nseq, hk):
    """One query per sequence (bottom-right causal: it sees all its keys): 8 sequences
    split their keys over workgroups (partials + merge), 600 take one workgroup each
    (direct output).  Both the output and the natural-log LSE match the oracle."""
    g = C.gen(400 + nseq)
    lk = torch.randint(1, 900, (nseq,), generator=g).tolist()
    cu_q = list(range(nseq + 1))
    cu_k = [0]
    for n in lk:
        cu_k.append(cu_k[-1] + n)
    q = C.randn(g, nseq, 4 * hk, 128)
    k = C.randn(g, cu_k[-1], hk, 128)
    v = C.randn(g, cu_k[-1], hk, 128)
    native.reset_counters()
    out, lse = torch.ops.ktt._sdpa_varlen_offsets(
        q.to(dev), k.to(dev), v.to(dev),
        torch.tensor(cu_q, dtype=torch.int32, device=dev), torch.tensor(cu_k, dtype=torch.int32, device=dev),
        1, max(lk), True, None, None, None,
    )
    torch.cuda.synchronize()
    assert native.counters()["attention"] == 1
    ref, ref_lse = oatt.sdpa_varlen(C.f64(q), C.f64(k), C.f64(v), cu_q, cu_k, is_causal=True)
    assert np.abs(out.cpu().double().numpy() - ref).max() < 2e-2
    assert np.abs(lse.cpu().double().numpy() - ref_lse).max() < 2e-2


def _capi_call(q, k, v, mask, num_splits):
    """One kmi_attn_fwd call on dense tensors with a bool [B, 1, 1, Sk] mask."""
    from kohakutt_amd import capi

    b, hq, sq, d = q.shape
    out = torch.empty_like(q)
    lse = torch.empty(b, hq, sq, dtype=torch.float32, device=q.device)
    a = capi.AttnArgs(
        q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(), out=out.data_ptr(), lse=lse.data_ptr(),
        dtype=capi.KMI_BF16, causal=0, batch=b, heads_q=hq, heads_kv=k.size(1), seq_q=sq,
        seq_k=k.size(2), head_dim=d, scale=d**-0.5, mask=mask.data_ptr(), mask_dtype=capi.KMI_BOOL,
        mask_mode=capi.KMI_MASK_STRIDED, num_splits=num_splits,
    )
    a.q_stride[:] = q.stride()[:3]
    a.k_stride[:] = k.stride()[:3]
    a.v_stride[:] = v.stride()[:3]
    a.o_stride[:] = out.stride()[:3]
    a.lse_stride[:] = lse.stride()
    a.mask_stride[:] = [mask.stride(0), 0, 0, mask.stride(3)]
    n = capi.workspace_bytes(a)
    ws = torch.empty(max(n, 1), dtype=torch.uint8, device=q.device)
    capi.attn_fwd(a, ws.data_ptr(), n, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu(), n


def test_decode_split_counts_agree(native, dev):
    """Every split count (1: the prefill kernel; 2, 3, 7, 32 and the plan's own: the decode
    kernel with that many workgroups per unit) matches the oracle, output and LSE;
    repeated calls are bit-identical (the merge order is fixed).  Row 0 has no kept key:
    the raw-score softmax over all its keys."""
    q, k, v, mask = _case("padding_with_empty_rows")
    qd, kd, vd, md = q.to(dev), k.to(dev), v.to(dev), mask.to(dev)
    ref, ref_lse = oatt.sdpa(C.f64(q), C.f64(k), C.f64(v), mask.numpy())
    raw, _ = oatt.sdpa(C.f64(q[:1]), C.f64(k[:1]), C.f64(v[:1]))
    assert np.abs(ref[:1] - raw).max() < 1e-8
    for ns in (0, 1, 2, 3, 7, 32):
        print(f"num_splits {ns}", flush=True)
        out, lse, n = _capi_call(qd, kd, vd, md, ns)
        assert (n > 0) == (ns != 1), (ns, n)
        assert np.abs(out.double().numpy() - ref).max() < 2e-2, ns
        # Row 0's LSE carries the -5e5 clamp, whose fp32 spacing is 1/32.
        assert np.allclose(lse.double().numpy(), ref_lse, rtol=1e-7, atol=2e-2), ns
        again, lse2, _ = _capi_call(qd, kd, vd, md, ns)
        assert torch.equal(again, out) and torch.equal(lse2, lse), ns


def test_decode_merge_is_the_same_on_every_stream(native, dev):
    """The split merge runs inside the decode kernel (the last workgroup of a unit merges,
    found by a per-stream counter that the merge clears) on up to 16 streams and as a
    launch of its own beyond them, with the same arithmetic: twenty streams in turn, each
    called twice, give bit-identical output and LSE, and match the oracle."""
    q, k, v, mask = _case("padding_with_empty_rows")
    qd, kd, vd, md = q.to(dev), k.to(dev), v.to(dev), mask.to(dev)
    ref, _ = oatt.sdpa(C.f64(q), C.f64(k), C.f64(v), mask.numpy())
    first, first_lse, _ = _capi_call(qd, kd, vd, md, 0)
    assert np.abs(first.double().numpy() - ref).max() < 2e-2
    streams = [torch.cuda.Stream() for _ in range(20)]
    for i, s in enumerate(streams):
        with torch.cuda.stream(s):
            for rep in range(2):
                out, lse, _ = _capi_call(qd, kd, vd, md, 0)
                assert torch.equal(out, first) and torch.equal(lse, first_lse), (i, rep)
    # More than 32 splits (past the counter word's split bits): the separate merge.
    q, k, v, mask = _case("long_cache")
    ref, _ = oatt.sdpa(C.f64(q), C.f64(k), C.f64(v), mask.numpy())
    for ns in (33, 40):
        print(f"num_splits {ns}", flush=True)
        out, _, _ = _capi_call(q.to(dev), k.to(dev), v.to(dev), mask.to(dev), ns)
        assert np.abs(out.double().numpy() - ref).max() < 2e-2, ns
