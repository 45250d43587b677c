"""Writes tests/golden/golden.npz: small seeded attention / norm cases with inputs as bf16
bit patterns (uint16) and expected outputs computed by torch CPU float64 -- independent of
oracle/.  The reference commits no numeric goldens (its .pt files are generated on demand,
tests/hardware/golden/test_goldens.py:15-19), so these fixtures are this build's own.

Run from the repo root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

OUT = Path(__file__).resolve().parent / "golden.npz"


def bf16(g, *shape):
    return torch.randn(*shape, generator=g).bfloat16()


def bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def sdpa64(q, k, v, mask=None, causal=False):
    g = q.size(1) // k.size(1)
    k, v = k.double().repeat_interleave(g, 1), v.double().repeat_interleave(g, 1)
    return F.scaled_dot_product_attention(q.double(), k, v, attn_mask=mask, is_causal=causal)


def main():
    g = torch.Generator().manual_seed(20261201)
    data = {}

    def dense(name, b, hq, hk, sq, sk, d, causal):
        q, k, v = bf16(g, b, hq, sq, d), bf16(g, b, hk, sk, d), bf16(g, b, hk, sk, d)
        data[f"{name}/q"], data[f"{name}/k"], data[f"{name}/v"] = bits(q), bits(k), bits(v)
        data[f"{name}/causal"] = np.array(causal)
        data[f"{name}/out"] = sdpa64(q, k, v, causal=causal).numpy()

    dense("mha", 2, 3, 3, 37, 37, 64, False)
    dense("gqa_causal", 1, 4, 2, 70, 70, 64, True)
    dense("mqa_causal_sq_lt_sk", 1, 4, 1, 5, 40, 128, True)

    # decode with a key-padding bool mask
    q, k, v = bf16(g, 2, 8, 1, 128), bf16(g, 2, 2, 100, 128), bf16(g, 2, 2, 100, 128)
    keep = (torch.arange(100)[None, :] < torch.tensor([33, 100])[:, None]).reshape(2, 1, 1, 100)
    data.update({"decode_mask/q": bits(q), "decode_mask/k": bits(k), "decode_mask/v": bits(v),
                 "decode_mask/mask": keep.numpy(), "decode_mask/out": sdpa64(q, k, v, keep).numpy()})

    # additive mask with -inf entries and one fully-masked row: its expected output is the
    # unmasked softmax of that row (the reference's clamp at -5e5; torch would give zeros)
    q, k, v = bf16(g, 1, 2, 48, 64), bf16(g, 1, 2, 48, 64), bf16(g, 1, 2, 48, 64)
    add = torch.randn(1, 1, 48, 48, generator=g, dtype=torch.float64)
    add = add.masked_fill(torch.rand(1, 1, 48, 48, generator=g) < 0.2, float("-inf"))
    add[..., :, 0] = 0.0
    add[..., 7, :] = float("-inf")
    add = add.float().double()  # stored as fp32: the expected output uses the stored values
    out = sdpa64(q, k, v, add)
    out[:, :, 7] = sdpa64(q, k, v)[:, :, 7]
    data.update({"additive_mask/q": bits(q), "additive_mask/k": bits(k), "additive_mask/v": bits(v),
                 "additive_mask/mask": add.float().numpy(), "additive_mask/out": out.numpy()})

    # packed varlen, bottom-right causal
    cu = [0, 20, 21, 60]
    q, k, v = bf16(g, 60, 4, 64), bf16(g, 60, 2, 64), bf16(g, 60, 2, 64)
    out = torch.zeros(60, 4, 64, dtype=torch.float64)
    for a, b in zip(cu[:-1], cu[1:]):
        n = b - a
        keep = torch.ones(n, n, dtype=torch.bool).tril()  # Lq == Lk: bottom-right == top-left
        out[a:b] = sdpa64(q[a:b].transpose(0, 1)[None], k[a:b].transpose(0, 1)[None],
                          v[a:b].transpose(0, 1)[None], keep)[0].transpose(0, 1)
    data.update({"varlen_causal/q": bits(q), "varlen_causal/k": bits(k), "varlen_causal/v": bits(v),
                 "varlen_causal/cu": np.array(cu, dtype=np.int32), "varlen_causal/out": out.numpy()})

    # norms
    x = bf16(g, 5, 70)
    w = (1 + 0.1 * torch.randn(70, generator=g)).bfloat16()
    b = (0.1 * torch.randn(70, generator=g)).bfloat16()
    y, mean, rstd = torch.native_layer_norm(x.double(), [70], w.double(), b.double(), 1e-5)
    data.update({"layer_norm/x": bits(x), "layer_norm/w": bits(w), "layer_norm/b": bits(b),
                 "layer_norm/y": y.numpy(), "layer_norm/mean": mean.numpy(), "layer_norm/rstd": rstd.numpy()})
    y = F.rms_norm(x.double(), [70], w.double(), 1e-6)
    data.update({"rms_norm/x": bits(x), "rms_norm/w": bits(w), "rms_norm/y": y.numpy()})
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(data)} arrays)")


if __name__ == "__main__":
    main()
