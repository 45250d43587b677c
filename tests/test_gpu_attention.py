"""GPU parity of the attention kernels against the float64 CPU oracle, with the
reference's ruler: median relative error no worse than 1.5x torch CPU at the same dtype
(``tests/hardware/ops/test_flash.py:15,56-145`` bound the same ratio by rel RMS).

Every call goes through the torch op surface (F.scaled_dot_product_attention,
torch.nn.attention.varlen.varlen_attn, kohakutt_amd.sdpa_varlen), which calls the C ABI;
``counters()`` proves the kernels ran rather than a torch fallback."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import attn_cases as C
from oracle import attention as oatt

pytestmark = pytest.mark.gpu


def _ran(native, n=1):
    c = native.counters()
    assert c["attention"] == n, c


def _check(gpu, cpu, ref, what, factor=1.5):
    ok, sg, sc = C.ruler_ok(gpu, cpu, torch.from_numpy(np.ascontiguousarray(ref)), factor)
    print(f"{what}: gpu rel_median {sg['rel_median']:.3e} cpu {sc['rel_median']:.3e}", flush=True)
    assert ok, (what, sg, sc)


def _dense_case(native, dev, q, k, v, mask=None, causal=False, scale=None, rows=None):
    native.reset_counters()
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    md = mask.to(dev) if mask is not None else None
    out = F.scaled_dot_product_attention(
        qd, kd, vd, attn_mask=md, is_causal=causal, scale=scale, enable_gqa=q.size(1) != k.size(1)
    )
    torch.cuda.synchronize()
    _ran(native)
    out = out.cpu()
    if rows is not None:
        q = q[:, :, rows]
        out = out[:, :, rows]
        if mask is not None and mask.size(-2) > 1:
            mask = mask[..., rows, :]
    m64 = None if mask is None else (mask.numpy() if mask.dtype == torch.bool else C.f64(mask))
    ref, _ = oatt.sdpa(C.f64(q), C.f64(k), C.f64(v), m64, causal, scale)
    cpu = C.torch_cpu_sdpa(q, k, v, mask, causal, scale)
    return out, cpu, ref


@pytest.mark.parametrize(
    "b,hq,hk,sq,sk,d,causal",
    [
        (1, 4, 4, 64, 64, 64, False),
        (2, 3, 3, 37, 37, 64, False),
        (1, 4, 2, 70, 70, 64, True),
        (1, 6, 1, 130, 130, 128, True),  # MQA
        (2, 8, 2, 33, 300, 128, False),
        (1, 4, 4, 40, 100, 64, True),  # causal Sq < Sk: top-left
        (1, 4, 2, 100, 40, 64, True),  # causal Sq > Sk: rows past Sk see every key
        (1, 2, 2, 1, 513, 64, False),
        (3, 16, 2, 1, 1000, 128, False),  # decode-shaped, split-KV
    ],
)
def test_dense_shapes(native, dev, b, hq, hk, sq, sk, d, causal):
    g = C.gen(b * 1000 + sq * 7 + sk)
    q = C.randn(g, b, hq, sq, d)
    k = C.randn(g, b, hk, sk, d)
    v = C.randn(g, b, hk, sk, d)
    out, cpu, ref = _dense_case(native, dev, q, k, v, causal=causal)
    _check(out, cpu, ref, f"dense {b}x{hq}/{hk}x{sq}x{sk}x{d} causal={causal}")


def test_fp16_and_scale(native, dev):
    g = C.gen(5)
    q = C.randn(g, 2, 4, 90, 64, dtype=torch.float16)
    k = C.randn(g, 2, 2, 90, 64, dtype=torch.float16)
    v = C.randn(g, 2, 2, 90, 64, dtype=torch.float16)
    out, cpu, ref = _dense_case(native, dev, q, k, v, causal=True, scale=0.3)
    _check(out, cpu, ref, "fp16 scale 0.3")


def test_fp32_inputs_cast_like_reference(native, dev):
    g = C.gen(6)
    q = torch.randn(1, 4, 50, 64, generator=g)
    k = torch.randn(1, 4, 50, 64, generator=g)
    v = torch.randn(1, 4, 50, 64, generator=g)
    native.reset_counters()
    out = F.scaled_dot_product_attention(q.to(dev), k.to(dev), v.to(dev)).cpu()
    _ran(native)
    assert out.dtype == torch.float32
    ref, _ = oatt.sdpa(C.f64(q), C.f64(k), C.f64(v))
    cpu = C.torch_cpu_sdpa(q.bfloat16(), k.bfloat16(), v.bfloat16()).float()
    _check(out, cpu, ref, "fp32 cast to bf16")


@pytest.mark.parametrize("s", [96, 100, 99])
@pytest.mark.parametrize("mask_kind", ["bool_key", "bool_full", "add_bf16", "add_f32_bcast_heads"])
def test_masks(native, dev, mask_kind, s):
    """Mask kinds and dtypes.  S = 96 and 100 read whole tiles' mask values four keys per
    load (100 ends in a partial tile, read key by key); S = 99 gives strides that are not
    multiples of four, read key by key throughout."""
    g = C.gen(11)
    b, h, d = 2, 4, 64
    q = C.randn(g, b, h, s, d)
    k = C.randn(g, b, 2, s, d)
    v = C.randn(g, b, 2, s, d)
    if mask_kind == "bool_key":
        lengths = torch.tensor([17, 96])
        mask = (torch.arange(s)[None, :] < lengths[:, None]).reshape(b, 1, 1, s)
    elif mask_kind == "bool_full":
        mask = torch.rand(b, h, s, s, generator=g) > 0.3
        mask[..., 0] = True
    elif mask_kind == "add_bf16":
        mask = (torch.randn(b, h, s, s, generator=g)).bfloat16()
    else:
        mask = torch.randn(b, 1, s, s, generator=g).masked_fill(torch.rand(b, 1, s, s, generator=g) < 0.2, float("-inf"))
        mask[..., 0] = 0.0
    out, cpu, ref = _dense_case(native, dev, q, k, v, mask=mask)
    _check(out, cpu, ref, f"mask {mask_kind} s={s}")


def test_fully_masked_row_is_softmax_of_raw_scores(native, dev):
    """Decision D1: as the reference, a row whose every key is masked attends over its
    raw scores (the clamp to -5e5 leaves their differences); torch CPU gives zeros."""
    g = C.gen(12)
    q = C.randn(g, 1, 2, 64, 64)
    k = C.randn(g, 1, 2, 80, 64)
    v = C.randn(g, 1, 2, 80, 64)
    mask = torch.zeros(1, 1, 64, 80)
    mask[..., 3, :] = float("-inf")
    mask[..., 9, ::2] = float("-inf")
    native.reset_counters()
    out = F.scaled_dot_product_attention(q.to(dev), k.to(dev), v.to(dev), attn_mask=mask.to(dev)).cpu()
    _ran(native)
    unmasked, _ = oatt.sdpa(C.f64(q), C.f64(k), C.f64(v))
    got = out[0, :, 3].double().numpy()
    assert np.isfinite(got).all()
    assert np.abs(got - unmasked[0, :, 3]).max() < 2e-2
    ref, _ = oatt.sdpa(C.f64(q), C.f64(k), C.f64(v), mask.numpy())
    assert np.abs(out.double().numpy() - ref).max() < 2e-2


def test_large_logits_masked_keys_contribute_nothing(native, dev):
    """Masked keys whose logits dwarf the kept ones still get exactly zero weight
    (test_flash.py:120-145 pins this up to logits of 1e5)."""
    g = C.gen(13)
    d = 64
    q = C.randn(g, 1, 1, 32, d)
    k = C.randn(g, 1, 1, 128, d)
    v = C.randn(g, 1, 1, 128, d)
    k[..., 64:, :] = (q[0, 0].float().mean(0) * 2000).bfloat16()  # huge scores on masked keys
    keep = torch.zeros(1, 1, 1, 128, dtype=torch.bool)
    keep[..., :64] = True
    native.reset_counters()
    out = F.scaled_dot_product_attention(q.to(dev), k.to(dev), v.to(dev), attn_mask=keep.to(dev)).cpu()
    _ran(native)
    ref, _ = oatt.sdpa(C.f64(q[..., :, :]), C.f64(k[..., :64, :]), C.f64(v[..., :64, :]))
    assert np.abs(out.double().numpy() - ref).max() < 2e-2


def test_nan_mask_entries_act_as_masked_keys(native, dev):
    """Decision D6: a NaN in an additive mask is a masked key here (the -5e5 clamp keeps
    max(NaN, -5e5) = -5e5), so the row stays finite; the reference's raw-mask path keeps
    the NaN (flash_dm.hpp:93-94) and that row comes out NaN.  Pinned so that a change is
    deliberate: the output equals the oracle's with the NaN entries set to -inf."""
    g = C.gen(14)
    q = C.randn(g, 1, 2, 32, 64)
    k = C.randn(g, 1, 2, 64, 64)
    v = C.randn(g, 1, 2, 64, 64)
    mask = torch.zeros(1, 1, 32, 64)
    mask[..., 5, 10] = float("nan")
    mask[..., 7, ::3] = float("nan")
    mask[..., 9, :] = float("nan")  # every key: the fully-masked rule (D1)
    native.reset_counters()
    out = F.scaled_dot_product_attention(q.to(dev), k.to(dev), v.to(dev), attn_mask=mask.to(dev)).cpu()
    _ran(native)
    assert torch.isfinite(out).all()
    as_masked = mask.masked_fill(mask.isnan(), float("-inf"))
    ref, _ = oatt.sdpa(C.f64(q), C.f64(k), C.f64(v), as_masked.numpy())
    assert np.abs(out.double().numpy() - ref).max() < 2e-2


def test_split_kv_matches_single_pass(native, dev):
    """Decode shapes split the keys across workgroups; the merged result matches the
    oracle and the per-(batch, head) rows stay isolated."""
    g = C.gen(14)
    q = C.randn(g, 4, 8, 1, 128)
    k = C.randn(g, 4, 1, 3000, 128)
    v = C.randn(g, 4, 1, 3000, 128)
    out, cpu, ref = _dense_case(native, dev, q, k, v)
    _check(out, cpu, ref, "split-KV MQA decode")
    # isolation: changing batch 1 leaves batch 0 bit-identical
    k2 = k.clone()
    k2[1] = -k2[1]
    out2 = F.scaled_dot_product_attention(q.to(dev), k2.to(dev), v.to(dev), enable_gqa=True).cpu()
    assert torch.equal(out2[0], out[0]) and torch.equal(out2[2:], out[2:])


def test_repeat_calls_bit_identical(native, dev):
    cfg = C.config1()
    q, k, v = cfg["q"].to(dev), cfg["k"].to(dev), cfg["v"].to(dev)
    a = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
    b = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
    assert torch.equal(a, b)


def test_config1_causal_gqa_prefill(native, dev):
    cfg = C.config1()
    out, cpu, ref = _dense_case(native, dev, cfg["q"], cfg["k"], cfg["v"], causal=True)
    _check(out, cpu, ref, "C1 causal GQA 1x14/2x2048x64")


@pytest.mark.parametrize("batch", [1, 32])
def test_config2_vit(native, dev, batch):
    cfg = C.config2(batch)
    q, k, v = cfg["q"], cfg["k"], cfg["v"]
    if batch > 4:
        # Every batch: the ruler over the whole output (and no non-finite value), plus each
        # batch on its own against float64 within the same factor of the CPU's error.
        native.reset_counters()
        full = F.scaled_dot_product_attention(q.to(dev), k.to(dev), v.to(dev)).cpu()
        _ran(native)
        ref, _ = oatt.sdpa(C.f64(q), C.f64(k), C.f64(v))
        cpu = C.torch_cpu_sdpa(q, k, v)
        _check(full, cpu, ref, f"C2 ViT B={batch} (all batches)")
        for b in range(batch):
            ok, sg, sc = C.ruler_ok(full[b], cpu[b], torch.from_numpy(np.ascontiguousarray(ref[b])))
            assert ok, (b, sg, sc)
    else:
        out, cpu, ref = _dense_case(native, dev, q, k, v)
        _check(out, cpu, ref, "C2 ViT B=1")


def test_config3_decode_padding_mask(native, dev):
    cfg = C.config3()
    out, cpu, ref = _dense_case(native, dev, cfg["q"], cfg["k"], cfg["v"], mask=cfg["mask"])
    _check(out, cpu, ref, "C3 decode 8x16/2x4096x128 bool mask")


def test_config5_self_and_cross(native, dev):
    cfg = C.config5()
    rows = torch.arange(0, 4096, 16)
    out, cpu, ref = _dense_case(native, dev, cfg["q"], cfg["k"], cfg["v"], rows=rows)
    _check(out, cpu, ref, "C5 self 2x10x4096x64 (every 16th row)")
    out, cpu, ref = _dense_case(native, dev, cfg["q"], cfg["ck"], cfg["cv"])
    _check(out, cpu, ref, "C5 cross 4096q x 77kv")


# ---------------------------------------------------------------- varlen


def _varlen_cpu_bf16(q, k, v, cu, causal):
    """torch CPU SDPA per sequence at the inputs' dtype (the reference's CPU plan for
    config 4), bottom-right causal as an explicit mask."""
    outs = []
    g = q.size(1) // k.size(1)
    for a, b in zip(cu[:-1], cu[1:]):
        qs = q[a:b].transpose(0, 1)[None]
        ks = k[a:b].transpose(0, 1)[None].repeat_interleave(g, 1)
        vs = v[a:b].transpose(0, 1)[None].repeat_interleave(g, 1)
        mask = None
        if causal:
            n = b - a
            mask = torch.ones(n, n, dtype=torch.bool).tril()
        outs.append(F.scaled_dot_product_attention(qs, ks, vs, attn_mask=mask)[0].transpose(0, 1))
    return torch.cat(outs)


def test_config4_varlen_causal(native, dev):
    from torch.nn.attention.varlen import varlen_attn

    cfg = C.config4()
    cu = cfg["cu"]
    q, k, v = cfg["q"], cfg["k"], cfg["v"]
    cu_t = torch.tensor(cu, dtype=torch.int32, device=dev)
    native.reset_counters()
    mx = max(cfg["lengths"])
    out = varlen_attn(q.to(dev), k.to(dev), v.to(dev), cu_t, cu_t, mx, mx, is_causal=True).cpu()
    _ran(native)
    ref, _ = oatt.sdpa_varlen(C.f64(q), C.f64(k), C.f64(v), cu, is_causal=True)
    _check(out, _varlen_cpu_bf16(q, k, v, cu, True), ref, "C4 varlen causal (varlen_attn)")
    native.reset_counters()
    out2 = native.sdpa_varlen(q.to(dev), k.to(dev), v.to(dev), cu, is_causal=True).cpu()
    _ran(native)
    assert torch.equal(out, out2)


def test_config4_varlen_packed_mask(native, dev):
    cfg = C.config4()
    cu = cfg["cu"]
    q, k, v, pm = cfg["q"], cfg["k"], cfg["v"], cfg["packed_mask"]
    native.reset_counters()
    out = native.sdpa_varlen(q.to(dev), k.to(dev), v.to(dev), cu, is_causal=True, packed_mask=pm.to(dev)).cpu()
    _ran(native)
    ref, _ = oatt.sdpa_varlen(C.f64(q), C.f64(k), C.f64(v), cu, is_causal=True, attn_mask=pm.numpy())
    # CPU bf16 per sequence with the same additive mask (fully-masked row excluded: torch
    # CPU zeroes it, the reference attends over raw scores).
    outs, off = [], 0
    for a, b in zip(cu[:-1], cu[1:]):
        n = b - a
        m = pm[off : off + n * n].reshape(1, 1, n, n).bfloat16()
        off += n * n
        qs = q[a:b].transpose(0, 1)[None]
        ks = k[a:b].transpose(0, 1)[None].repeat_interleave(2, 1)
        vs = v[a:b].transpose(0, 1)[None].repeat_interleave(2, 1)
        outs.append(F.scaled_dot_product_attention(qs, ks, vs, attn_mask=m)[0].transpose(0, 1))
    cpu = torch.cat(outs)
    keep = torch.ones(q.size(0), dtype=torch.bool)
    keep[5] = False
    _check(out[keep], cpu[keep], ref[keep.numpy()], "C4 varlen masked run")
    # The fully-masked row (token 5 of sequence 0, causal: keys 0..5): the reference
    # attends over its raw scores, which is unmasked attention of that row -- so torch CPU
    # bf16 without the mask is its same-dtype baseline, under the same ruler.
    assert cu[0] == 0 and cu[1] > 5
    qs = q[5:6].transpose(0, 1)[None]
    ks = k[0:6].transpose(0, 1)[None].repeat_interleave(2, 1)
    vs = v[0:6].transpose(0, 1)[None].repeat_interleave(2, 1)
    cpu5 = F.scaled_dot_product_attention(qs, ks, vs)[0].transpose(0, 1)[0]
    _check(out[5], cpu5, ref[5], "C4 fully-masked row (raw-score softmax)")


def test_varlen_key_mask_and_neighbour_independence(native, dev):
    g = C.gen(21)
    cu = [0, 40, 41, 170, 300]
    t = cu[-1]
    q = C.randn(g, t, 4, 64)
    k = C.randn(g, t, 2, 64)
    v = C.randn(g, t, 2, 64)
    km = torch.rand(t, generator=g) > 0.2
    for a in cu[:-1]:
        km[a] = True
    out = native.sdpa_varlen(q.to(dev), k.to(dev), v.to(dev), cu, attn_mask=km.to(dev)).cpu()
    ref, _ = oatt.sdpa_varlen(C.f64(q), C.f64(k), C.f64(v), cu, key_mask=km.numpy())
    assert np.abs(out.double().numpy() - ref).max() < 2e-2
    # a sequence's output does not depend on its neighbours' tokens
    q2, k2, v2 = q.clone(), k.clone(), v.clone()
    q2[:40] = 0
    k2[170:] = 1
    v2[41:170] = -v2[41:170]
    out2 = native.sdpa_varlen(q2.to(dev), k2.to(dev), v2.to(dev), cu, attn_mask=km.to(dev)).cpu()
    assert torch.equal(out[40:41], out2[40:41])


def test_varlen_op_refuses_undersized_longest_lengths(native, dev):
    """The packed op checks max_q / max_k against host offsets itself (callers may reach
    it without the Python front)."""
    q = torch.randn(8, 2, 64, device=dev, dtype=torch.bfloat16)
    k = torch.randn(9, 2, 64, device=dev, dtype=torch.bfloat16)
    cu_q, cu_k = torch.tensor([0, 3, 8]), torch.tensor([0, 4, 9])
    with pytest.raises(ValueError, match="below the longest sequence"):
        torch.ops.ktt._sdpa_varlen_offsets(q, k, k, cu_q, cu_k, 4, 5, False, None, None, None)
    out, _ = torch.ops.ktt._sdpa_varlen_offsets(q, k, k, cu_q, cu_k, 5, 5, False, None, None, None)
    assert torch.isfinite(out).all()


def test_varlen_cross_lengths_bottom_right(native, dev):
    g = C.gen(22)
    cu_q = [0, 10, 30, 31]
    cu_k = [0, 50, 70, 200]
    q = C.randn(g, 31, 8, 128)
    k = C.randn(g, 200, 2, 128)
    v = C.randn(g, 200, 2, 128)
    out = native.sdpa_varlen(q.to(dev), k.to(dev), v.to(dev), cu_q, cu_k, is_causal=True).cpu()
    ref, _ = oatt.sdpa_varlen(C.f64(q), C.f64(k), C.f64(v), cu_q, cu_k, is_causal=True)
    assert np.abs(out.double().numpy() - ref).max() < 2e-2


@pytest.mark.parametrize(
    "b,hq,hk,sq,sk,d",
    [
        (16, 16, 4, 300, 200, 128),  # GQA, 7 key tiles: one row block per wavefront
        (8, 8, 8, 512, 100, 64),
        (32, 8, 2, 128, 256, 64),  # exactly 8 key tiles
        (4, 16, 16, 1024, 77, 128),  # three tiles staged once in LDS, partial last tile
    ],
)
def test_short_key_ranges_output_and_lse(native, dev, b, hq, hk, sq, sk, d):
    """Short unmasked key ranges run one row block per wavefront (no key split, no merge;
    up to four key tiles are staged once per workgroup in LDS); output and natural-log LSE
    match the oracle through the C ABI."""
    from kohakutt_amd import capi

    g = C.gen(500 + sq)
    q, k, v = C.randn(g, b, hq, sq, d), C.randn(g, b, hk, sk, d), C.randn(g, b, hk, sk, d)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    out = torch.empty_like(qd)
    lse = torch.empty(b, hq, sq, dtype=torch.float32, device=dev)
    a = capi.AttnArgs(
        q=qd.data_ptr(), k=kd.data_ptr(), v=vd.data_ptr(), out=out.data_ptr(), lse=lse.data_ptr(),
        dtype=capi.KMI_BF16, causal=0, batch=b, heads_q=hq, heads_kv=hk, seq_q=sq, seq_k=sk,
        head_dim=d, scale=d**-0.5,
    )
    a.q_stride[:] = qd.stride()[:3]
    a.k_stride[:] = kd.stride()[:3]
    a.v_stride[:] = vd.stride()[:3]
    a.o_stride[:] = out.stride()[:3]
    a.lse_stride[:] = lse.stride()
    assert capi.workspace_bytes(a) == 0
    capi.attn_fwd(a, 0, 0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    ref, ref_lse = oatt.sdpa(C.f64(q), C.f64(k), C.f64(v))
    _check(out.cpu(), C.torch_cpu_sdpa(q, k, v), ref, f"short keys {b}x{hq}/{hk}x{sq}x{sk}x{d}")
    assert np.abs(lse.cpu().double().numpy() - ref_lse).max() < 2e-2


@pytest.mark.parametrize("b,hq,hk,s", [(24, 16, 16, 128), (6, 28, 4, 300)])
def test_causal_paired_query_tiles(native, dev, b, hq, hk, s):
    """Causal grids just above one round of resident workgroups run their shortest query
    tiles two to a workgroup; every row still matches the oracle and repeat calls are
    bit-identical."""
    g = C.gen(600 + s)
    q, k, v = C.randn(g, b, hq, s, 64), C.randn(g, b, hk, s, 64), C.randn(g, b, hk, s, 64)
    out, cpu, ref = _dense_case(native, dev, q, k, v, causal=True)
    _check(out, cpu, ref, f"causal paired {b}x{hq}/{hk}x{s}")
    again = F.scaled_dot_product_attention(q.to(dev), k.to(dev), v.to(dev), is_causal=True,
                                           enable_gqa=hq != hk).cpu()
    assert torch.equal(again, out)


@pytest.mark.parametrize("sk,d,causal", [(77, 64, False), (301, 128, False), (130, 64, True)])
def test_broadcast_key_rows_and_partial_tiles(native, dev, sk, d, causal):
    """K and V given with a zero sequence stride (one row repeated over every key: an
    expanded view) and key counts that end inside a tile: the tile loads read the repeated
    row and stop at the last key.  The result equals the oracle on the materialised K/V
    (for non-causal rows: exactly V's row, since every key scores the same)."""
    from kohakutt_amd import capi

    b, hq, hk, sq = 2, 8, 2, 96
    g = C.gen(700 + sk)
    q = C.randn(g, b, hq, sq, d)
    k1, v1 = C.randn(g, b, hk, 1, d), C.randn(g, b, hk, 1, d)
    k, v = k1.expand(b, hk, sk, d), v1.expand(b, hk, sk, d)
    qd, kd, vd = q.to(dev), k1.to(dev).expand(b, hk, sk, d), v1.to(dev).expand(b, hk, sk, d)
    assert kd.stride(2) == 0 and vd.stride(2) == 0
    out = torch.empty_like(qd)
    a = capi.AttnArgs(
        q=qd.data_ptr(), k=kd.data_ptr(), v=vd.data_ptr(), out=out.data_ptr(), lse=0,
        dtype=capi.KMI_BF16, causal=int(causal), batch=b, heads_q=hq, heads_kv=hk, seq_q=sq, seq_k=sk,
        head_dim=d, scale=d**-0.5,
    )
    a.q_stride[:] = qd.stride()[:3]
    a.k_stride[:] = kd.stride()[:3]
    a.v_stride[:] = vd.stride()[:3]
    a.o_stride[:] = out.stride()[:3]
    n = capi.workspace_bytes(a)
    ws = torch.empty(max(n, 1), dtype=torch.uint8, device=dev)
    capi.attn_fwd(a, ws.data_ptr(), n, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    ref, _ = oatt.sdpa(C.f64(q), C.f64(k.contiguous()), C.f64(v.contiguous()), is_causal=causal)
    err = np.abs(out.cpu().double().numpy() - ref)
    # Every visible key holds the same V row: the output is that row, rounded to bf16.
    assert err.max() < 1e-2, err.max()


@pytest.mark.parametrize("sk,causal", [(100, True), (77, False)])
def test_overlapping_key_rows(native, dev, sk, causal):
    """K and V rows that overlap in memory (a row stride of 32 elements at head dim 64, as
    an as_strided view makes): every key row is read in full, including the last, whose
    end lies 32 elements past the start of the row after it; the result equals the
    oracle on the materialised K/V."""
    from kohakutt_amd import capi

    b, hq, hk, sq, d, rs = 1, 4, 2, 96, 64, 32
    g = C.gen(800 + sk)
    q = C.randn(g, b, hq, sq, d)
    kb, vb = C.randn(g, b * hk * (sk * rs + d)), C.randn(g, b * hk * (sk * rs + d))
    shape, stride = (b, hk, sk, d), (hk * (sk * rs + d), sk * rs + d, rs, 1)
    k, v = kb.as_strided(shape, stride), vb.as_strided(shape, stride)
    qd = q.to(dev)
    kbd, vbd = kb.to(dev), vb.to(dev)
    kd, vd = kbd.as_strided(shape, stride), vbd.as_strided(shape, stride)
    out = torch.empty_like(qd)
    a = capi.AttnArgs(
        q=qd.data_ptr(), k=kd.data_ptr(), v=vd.data_ptr(), out=out.data_ptr(), lse=0,
        dtype=capi.KMI_BF16, causal=int(causal), batch=b, heads_q=hq, heads_kv=hk, seq_q=sq, seq_k=sk,
        head_dim=d, scale=d**-0.5,
    )
    a.q_stride[:] = qd.stride()[:3]
    a.k_stride[:] = kd.stride()[:3]
    a.v_stride[:] = vd.stride()[:3]
    a.o_stride[:] = out.stride()[:3]
    n = capi.workspace_bytes(a)
    ws = torch.empty(max(n, 1), dtype=torch.uint8, device=dev)
    capi.attn_fwd(a, ws.data_ptr(), n, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    kc, vc = k.contiguous(), v.contiguous()
    ref, _ = oatt.sdpa(C.f64(q), C.f64(kc), C.f64(vc), is_causal=causal)
    _check(out.cpu(), C.torch_cpu_sdpa(q, kc, vc, None, causal, d**-0.5), ref, f"overlapping rows sk={sk}")


@pytest.mark.parametrize("b,s,h,hk,d,causal", [(2, 197, 12, 12, 64, False), (1, 300, 8, 2, 128, True)])
def test_head_view_inputs_give_a_projection_layout_output(native, dev, b, s, h, hk, d, causal):
    """q, k, v as head views of [B, S, C] projections (a fused qkv for MHA, separate q and
    kv projections for GQA) are read in place, and the output comes back as a [B, H, S, D]
    view of a dense [B, S, H D] tensor (the reference's pitched route,
    aten_attention.cpp:605-628): transposing it back to the projection layout is free.
    With gradients required the output stays dense [B, H, S, D]."""
    g = C.gen(800 + s)
    if h == hk:
        qkv = C.randn(g, b, s, 3 * h * d)
        q, k, v = (qkv[..., i * h * d:(i + 1) * h * d].view(b, s, h, d).transpose(1, 2) for i in range(3))
        dev_views = lambda: (lambda x: [x[..., i * h * d:(i + 1) * h * d].view(b, s, h, d).transpose(1, 2)
                                        for i in range(3)])(qkv.to(dev))
    else:
        qp, kvp = C.randn(g, b, s, h * d), C.randn(g, b, s, 2 * hk * d)
        q = qp.view(b, s, h, d).transpose(1, 2)
        k, v = (kvp[..., i * hk * d:(i + 1) * hk * d].view(b, s, hk, d).transpose(1, 2) for i in range(2))
        def dev_views():
            qx, kvx = qp.to(dev), kvp.to(dev)
            return [qx.view(b, s, h, d).transpose(1, 2)] + [
                kvx[..., i * hk * d:(i + 1) * hk * d].view(b, s, hk, d).transpose(1, 2) for i in range(2)]
    qd, kd, vd = dev_views()
    assert qd.stride(1) == d and kd.stride(1) == d  # head views, not contiguous copies
    native.reset_counters()
    out = F.scaled_dot_product_attention(qd, kd, vd, is_causal=causal, enable_gqa=h != hk)
    torch.cuda.synchronize()
    _ran(native)
    assert out.shape == (b, h, s, d)
    assert out.stride() == (s * h * d, d, h * d, 1), out.stride()
    assert out.transpose(1, 2).is_contiguous()
    ref, _ = oatt.sdpa(C.f64(q), C.f64(k), C.f64(v), None, causal)
    _check(out.cpu(), C.torch_cpu_sdpa(q.contiguous(), k.contiguous(), v.contiguous(), None, causal), ref,
           f"head views {b}x{s}x{h}/{hk}x{d}")
    qg = qd.detach().clone().requires_grad_(True)
    out_g = F.scaled_dot_product_attention(qg, kd, vd, is_causal=causal, enable_gqa=h != hk)
    assert out_g.is_contiguous()
    assert torch.equal(out_g.detach().cpu(), out.cpu())


def test_mask_with_unaligned_base_reads_key_by_key(native, dev):
    """A mask view starting one element into its storage (base not aligned to four
    elements) takes the key-by-key loads; results match the oracle."""
    g = C.gen(13)
    b, h, s, d = 2, 4, 128, 64
    q, k, v = C.randn(g, b, h, s, d), C.randn(g, b, h, s, d), C.randn(g, b, h, s, d)
    big = torch.randn(b * h * s * s + 1, generator=g)
    mask = big[1:].view(b, h, s, s).masked_fill(torch.rand(b, h, s, s, generator=g) < 0.2, float("-inf"))
    mask[..., 0] = 0.0
    native.reset_counters()
    md = torch.randn(b * h * s * s + 1, device=dev)[1:].view(b, h, s, s)
    md.copy_(mask.to(dev))
    assert md.storage_offset() == 1
    out = F.scaled_dot_product_attention(q.to(dev), k.to(dev), v.to(dev), attn_mask=md).cpu()
    _ran(native)
    ref, _ = oatt.sdpa(C.f64(q), C.f64(k), C.f64(v), C.f64(mask))
    _check(out, C.torch_cpu_sdpa(q, k, v, mask), ref, "unaligned mask base")


@pytest.mark.parametrize(
    "b,hq,hk,sq,sk,d,causal,masked",
    [
        (2, 4, 2, 90, 90, 64, True, False),  # prefill, 16/32-row tiles
        (2, 8, 8, 70, 300, 128, False, True),  # prefill, masked
        (4, 16, 2, 1, 700, 128, False, False),  # decode, split-KV
        (4, 16, 2, 1, 700, 128, False, True),  # decode with a padding mask
        (32, 12, 12, 197, 197, 64, False, False),  # row-split mode
    ],
)
def test_negative_scale(native, dev, b, hq, hk, sq, sk, d, causal, masked):
    """A negative softmax scale (legal in SDPA) flips which key has the largest logit:
    every kernel takes it exactly (Q's sign is flipped) and matches the oracle."""
    g = C.gen(900 + sk)
    q, k, v = C.randn(g, b, hq, sq, d), C.randn(g, b, hk, sk, d), C.randn(g, b, hk, sk, d)
    mask = None
    if masked:
        lengths = torch.randint(1, sk + 1, (b,), generator=g)
        mask = (torch.arange(sk)[None, :] < lengths[:, None]).reshape(b, 1, 1, sk)
    out, cpu, ref = _dense_case(native, dev, q, k, v, mask=mask, causal=causal, scale=-0.2)
    _check(out, cpu, ref, f"negative scale {b}x{hq}/{hk}x{sq}x{sk}x{d}")


@pytest.mark.parametrize("b,hq,hk,sq,sk,d", [(1, 4, 4, 100, 1, 64), (2, 8, 2, 1, 1, 128), (3, 6, 3, 33, 2, 64)])
def test_one_or_two_keys(native, dev, b, hq, hk, sq, sk, d):
    """Key ranges of one or two keys (a single partial tile, every other row of it past
    the end): each output row is the softmax-weighted V rows, matching the oracle."""
    g = C.gen(950 + sq)
    q, k, v = C.randn(g, b, hq, sq, d), C.randn(g, b, hk, sk, d), C.randn(g, b, hk, sk, d)
    out, cpu, ref = _dense_case(native, dev, q, k, v)
    _check(out, cpu, ref, f"few keys {b}x{hq}/{hk}x{sq}x{sk}x{d}")


def test_bool_mask_reaches_the_kernels_unconverted(native, dev):
    """F.scaled_dot_product_attention with a bool mask (no gradients) runs the kernels on
    the bool mask itself; the output is bit-identical to the same mask given additively
    (0 / -inf in bf16, what torch's composite would have made of it), including a
    fully-masked row (softmax over its raw scores)."""
    g = C.gen(21)
    b, h, hk, s, sk, d = 2, 8, 2, 5, 700, 128
    q, k, v = C.randn(g, b, h, s, d), C.randn(g, b, hk, sk, d), C.randn(g, b, hk, sk, d)
    keep = torch.rand(b, 1, s, sk, generator=g) > 0.3
    keep[1, 0, 2] = False
    qd, kd, vd, md = q.to(dev), k.to(dev), v.to(dev), keep.to(dev)
    add = torch.zeros(keep.shape, dtype=torch.bfloat16).masked_fill(~keep, float("-inf")).to(dev)
    native.reset_counters()
    out_b = F.scaled_dot_product_attention(qd, kd, vd, attn_mask=md, enable_gqa=True)
    out_a = F.scaled_dot_product_attention(qd, kd, vd, attn_mask=add, enable_gqa=True)
    torch.cuda.synchronize()
    assert native.counters()["attention"] == 2
    assert torch.equal(out_b, out_a)
    ref, _ = oatt.sdpa(C.f64(q), C.f64(k), C.f64(v), keep.numpy())
    assert np.abs(out_b.cpu().double().numpy() - ref).max() < 2e-2


def test_bool_mask_with_gradients_and_scopes_keep_torch_routes(native, dev):
    """With gradients a bool-mask call goes through torch's composite (overrideable op +
    the fp32 recompute backward); under sdpa_kernel(MATH) the kernels are not used."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    g = C.gen(22)
    b, h, s, d = 2, 4, 64, 64
    q, k, v = C.randn(g, b, h, s, d), C.randn(g, b, h, s, d), C.randn(g, b, h, s, d)
    keep = torch.rand(b, 1, s, s, generator=g) > 0.3
    keep[..., 0] = True
    qd = q.to(dev).requires_grad_()
    kd, vd, md = k.to(dev), v.to(dev), keep.to(dev)
    native.reset_counters()
    out = F.scaled_dot_product_attention(qd, kd, vd, attn_mask=md)
    out.float().sum().backward()
    torch.cuda.synchronize()
    assert native.counters()["attention"] == 1
    q64 = q.double().requires_grad_()
    ref = F.scaled_dot_product_attention(q64, k.double(), v.double(), attn_mask=keep)
    ref.sum().backward()
    assert (qd.grad.cpu().double() - q64.grad).abs().max().item() < 5e-2
    native.reset_counters()
    with sdpa_kernel([SDPBackend.MATH]):
        out_m = F.scaled_dot_product_attention(qd.detach(), kd, vd, attn_mask=md)
    torch.cuda.synchronize()
    assert native.counters()["attention"] == 0
    assert (out_m.float() - out.detach().float()).abs().max().item() < 3e-2
