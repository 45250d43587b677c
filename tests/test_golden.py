"""The committed golden fixtures (tests/golden/golden.npz, torch CPU float64 expected
outputs): they pin the oracle on the CPU and the kernels on the GPU."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as A
from oracle import norms as N

G = np.load(Path(__file__).resolve().parent / "golden" / "golden.npz")


def tb(name):
    """bf16 tensor from stored bit patterns."""
    return torch.from_numpy(G[name].view(np.int16).copy()).view(torch.bfloat16)


def f64(name):
    return tb(name).double().numpy()


DENSE = ["mha", "gqa_causal", "mqa_causal_sq_lt_sk"]


@pytest.mark.parametrize("case", DENSE)
def test_oracle_dense_matches_golden(case):
    out, _ = A.sdpa(f64(f"{case}/q"), f64(f"{case}/k"), f64(f"{case}/v"), is_causal=bool(G[f"{case}/causal"]))
    assert np.abs(out - G[f"{case}/out"]).max() < 1e-12


@pytest.mark.parametrize("case", ["decode_mask", "additive_mask"])
def test_oracle_masked_matches_golden(case):
    out, _ = A.sdpa(f64(f"{case}/q"), f64(f"{case}/k"), f64(f"{case}/v"), G[f"{case}/mask"])
    assert np.abs(out - G[f"{case}/out"]).max() < 1e-9


def test_oracle_varlen_matches_golden():
    out, _ = A.sdpa_varlen(f64("varlen_causal/q"), f64("varlen_causal/k"), f64("varlen_causal/v"),
                           G["varlen_causal/cu"], is_causal=True)
    assert np.abs(out - G["varlen_causal/out"]).max() < 1e-12


def test_oracle_norms_match_golden():
    y, mean, rstd = N.layer_norm(f64("layer_norm/x"), f64("layer_norm/w"), f64("layer_norm/b"), 1e-5)
    assert np.abs(y - G["layer_norm/y"]).max() < 1e-12
    assert np.abs(mean - G["layer_norm/mean"]).max() < 1e-12
    y, _ = N.rms_norm(f64("rms_norm/x"), f64("rms_norm/w"), eps=1e-6)
    assert np.abs(y - G["rms_norm/y"]).max() < 1e-12


def _ruler(gpu, cpu, ref):
    from oracle.ruler import diff_stats

    sg = diff_stats(gpu, ref)
    sc = diff_stats(cpu, ref)
    assert sg["nonfinite"] == 0 and sg["rel_median"] <= 1.5 * sc["rel_median"], (sg, sc)


@pytest.mark.gpu
@pytest.mark.parametrize("case", DENSE + ["decode_mask", "additive_mask"])
def test_gpu_dense_matches_golden(native, dev, case):
    q, k, v = tb(f"{case}/q"), tb(f"{case}/k"), tb(f"{case}/v")
    causal = bool(G[f"{case}/causal"]) if f"{case}/causal" in G else False
    mask = torch.from_numpy(G[f"{case}/mask"]) if f"{case}/mask" in G else None
    native.reset_counters()
    out = F.scaled_dot_product_attention(q.to(dev), k.to(dev), v.to(dev), is_causal=causal,
                                         attn_mask=None if mask is None else mask.to(dev),
                                         enable_gqa=q.size(1) != k.size(1)).cpu()
    assert native.counters()["attention"] == 1
    g = q.size(1) // k.size(1)
    cpu = F.scaled_dot_product_attention(q, k.repeat_interleave(g, 1), v.repeat_interleave(g, 1),
                                         is_causal=causal, attn_mask=mask)
    ref = G[f"{case}/out"]
    if case == "additive_mask":  # torch CPU zeroes the fully-masked row 7: compare the rest
        keep = np.ones(ref.shape[2], dtype=bool)
        keep[7] = False
        assert np.abs(out[:, :, 7].double().numpy() - ref[:, :, 7]).max() < 2e-2
        out, cpu, ref = out[:, :, keep], cpu[:, :, keep], ref[:, :, keep]
    _ruler(out, cpu, ref)


@pytest.mark.gpu
def test_gpu_varlen_matches_golden(native, dev):
    q, k, v = tb("varlen_causal/q"), tb("varlen_causal/k"), tb("varlen_causal/v")
    cu = G["varlen_causal/cu"].tolist()
    out = native.sdpa_varlen(q.to(dev), k.to(dev), v.to(dev), cu, is_causal=True).cpu()
    assert np.abs(out.double().numpy() - G["varlen_causal/out"]).max() < 2e-2


@pytest.mark.gpu
def test_gpu_norms_match_golden(native, dev):
    x, w, b = tb("layer_norm/x"), tb("layer_norm/w"), tb("layer_norm/b")
    y, mean, rstd = torch.ops.aten.native_layer_norm(x.to(dev), [70], w.to(dev), b.to(dev), 1e-5)
    assert np.abs(y.cpu().double().numpy() - G["layer_norm/y"]).max() < 2e-2
    assert np.allclose(mean.cpu().double().numpy(), G["layer_norm/mean"], rtol=1e-6, atol=1e-7)
    assert np.allclose(rstd.cpu().double().numpy(), G["layer_norm/rstd"], rtol=1e-6)
    y = F.rms_norm(tb("rms_norm/x").to(dev), [70], tb("rms_norm/w").to(dev), 1e-6)
    assert np.abs(y.cpu().double().numpy() - G["rms_norm/y"]).max() < 2e-2
