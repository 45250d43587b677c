"""Seeded inputs of the BASELINE configs and the float64-ruler checks shared by the GPU
parity tests and bench.py's CPU baseline.

Inputs follow the generation rule of the benchmark plan: a CPU ``torch.Generator`` seeded
``1000 + config``, fp32 ``randn`` drawn in the listed order and cast to bf16 on the CPU,
so the CPU oracle and the GPU see identical bits.
"""

from __future__ import annotations

import math

import numpy as np
import torch


def gen(seed):
    return torch.Generator().manual_seed(seed)


def randn(g, *shape, dtype=torch.bfloat16):
    return torch.randn(*shape, generator=g).to(dtype)


def config1(dtype=torch.bfloat16):
    """Qwen2.5-0.5B prefill block: rms_norm x [1,2048,896], then causal GQA 14/2, D 64."""
    g = gen(1001)
    x = randn(g, 1, 2048, 896, dtype=dtype)
    w = (1 + 0.02 * torch.randn(896, generator=g)).to(dtype)
    q = randn(g, 1, 14, 2048, 64, dtype=dtype)
    k = randn(g, 1, 2, 2048, 64, dtype=dtype)
    v = randn(g, 1, 2, 2048, 64, dtype=dtype)
    return dict(x=x, w=w, eps=1e-6, q=q, k=k, v=v, causal=True)


def config2(batch=1, dtype=torch.bfloat16):
    """ViT-B/16 block: layer_norm [1,197,768] eps 1e-6, then MHA B x 12 x 197 x 64."""
    g = gen(1002)
    x = randn(g, 1, 197, 768, dtype=dtype)
    w = (1 + 0.02 * torch.randn(768, generator=g)).to(dtype)
    b = (0.02 * torch.randn(768, generator=g)).to(dtype)
    q = randn(g, batch, 12, 197, 64, dtype=dtype)
    k = randn(g, batch, 12, 197, 64, dtype=dtype)
    v = randn(g, batch, 12, 197, 64, dtype=dtype)
    return dict(x=x, w=w, b=b, eps=1e-6, q=q, k=k, v=v, causal=False)


def config3(dtype=torch.bfloat16):
    """Qwen2.5-3B decode: q [8,16,1,128], K/V cache [8,2,4096,128], valid lengths
    U[77, 4096] as a bool padding mask [8,1,1,4096]; rms_norm [8,1,2048]."""
    g = gen(1003)
    q = randn(g, 8, 16, 1, 128, dtype=dtype)
    k = randn(g, 8, 2, 4096, 128, dtype=dtype)
    v = randn(g, 8, 2, 4096, 128, dtype=dtype)
    lengths = torch.randint(77, 4097, (8,), generator=g)
    mask = (torch.arange(4096)[None, :] < lengths[:, None]).reshape(8, 1, 1, 4096)
    x = randn(g, 8, 1, 2048, dtype=dtype)
    w = (1 + 0.02 * torch.randn(2048, generator=g)).to(dtype)
    return dict(q=q, k=k, v=v, mask=mask, lengths=lengths, x=x, w=w, eps=1e-6)


def config4(dtype=torch.bfloat16):
    """Packed varlen causal GQA: 8 sequences, lengths U[64, 1024], Hq 16, Hkv 8, D 128;
    plus the masked run's block-packed additive mask (0 where allowed, -inf on a random
    10% of allowed keys per row, causal folded in, row 5 of sequence 0 fully masked)."""
    g = gen(1004)
    lengths = torch.randint(64, 1025, (8,), generator=g)
    cu = [0]
    for n in lengths.tolist():
        cu.append(cu[-1] + n)
    t = cu[-1]
    q = randn(g, t, 16, 128, dtype=dtype)
    k = randn(g, t, 8, 128, dtype=dtype)
    v = randn(g, t, 8, 128, dtype=dtype)
    blocks = []
    for i, n in enumerate(lengths.tolist()):
        allowed = torch.ones(n, n, dtype=torch.bool).tril()
        drop = torch.rand(n, n, generator=g) < 0.1
        keep = allowed & ~drop
        if i == 0:
            keep[5, :] = False
        m = torch.zeros(n, n).masked_fill(~keep, float("-inf"))
        blocks.append(m.reshape(-1))
    packed = torch.cat(blocks)
    return dict(q=q, k=k, v=v, cu=cu, lengths=lengths.tolist(), packed_mask=packed)


def config5(dtype=torch.bfloat16):
    """SDXL-UNet 1024px CFG step: layer_norm [2,4096,640] eps 1e-5; self-attention
    2 x 10 x 4096 x 64; cross-attention 4096 queries over 77 keys projected from a
    N(0,1) context [2,77,2048] by N(0, 0.02) weights."""
    g = gen(1005)
    x = randn(g, 2, 4096, 640, dtype=dtype)
    w = (1 + 0.02 * torch.randn(640, generator=g)).to(dtype)
    b = (0.02 * torch.randn(640, generator=g)).to(dtype)
    q = randn(g, 2, 10, 4096, 64, dtype=dtype)
    k = randn(g, 2, 10, 4096, 64, dtype=dtype)
    v = randn(g, 2, 10, 4096, 64, dtype=dtype)
    ctx = torch.randn(2, 77, 2048, generator=g)
    wk = 0.02 * torch.randn(2048, 640, generator=g)
    wv = 0.02 * torch.randn(2048, 640, generator=g)
    ck = (ctx @ wk).view(2, 77, 10, 64).transpose(1, 2).to(dtype).contiguous()
    cv = (ctx @ wv).view(2, 77, 10, 64).transpose(1, 2).to(dtype).contiguous()
    return dict(x=x, w=w, b=b, eps=1e-5, q=q, k=k, v=v, ck=ck, cv=cv)


# ---------------------------------------------------------------- FLOP / byte counts

def attn_flops(d, hq, pairs):
    """Algorithmic attention FLOPs: 4 * D * Hq * (query, key) pairs."""
    return 4.0 * d * hq * pairs


def causal_pairs(b, s):
    return b * s * (s + 1) // 2


# ---------------------------------------------------------------- CPU references

def torch_cpu_sdpa(q, k, v, mask=None, causal=False, scale=None):
    """The reference's CPU path: torch CPU SDPA at the inputs' dtype (K/V heads expanded
    per group)."""
    g = q.size(1) // k.size(1)
    if g > 1:
        k = k.repeat_interleave(g, 1)
        v = v.repeat_interleave(g, 1)
    return torch.nn.functional.scaled_dot_product_attention(
        q, k, v, attn_mask=mask, is_causal=causal, scale=scale
    )


def ruler_ok(gpu, cpu_same_dtype, ref64, factor=1.5, floor=0.0):
    """(ok, gpu stats, cpu stats): the GPU's median relative error against float64 is at
    most ``factor`` times the CPU same-dtype error (plus ``floor``), with no non-finite
    values.  The tolerance of the benchmark plan is factor 1.5."""
    from oracle.ruler import diff_stats

    sg = diff_stats(gpu, ref64)
    sc = diff_stats(cpu_same_dtype, ref64)
    ok = sg["nonfinite"] == 0 and sg["rel_median"] <= factor * sc["rel_median"] + floor
    return ok, sg, sc


def f64(t):
    return t.double().numpy() if isinstance(t, torch.Tensor) else np.asarray(t, np.float64)


def default_scale(d):
    return 1.0 / math.sqrt(d)
