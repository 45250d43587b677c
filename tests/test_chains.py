"""The torch.compile RMSNorm chain rewrite (``kohakutt_amd.chains``; the reference's norm
rewrite, ``src/kohakutt/torch_backend/chains.py:278-338``): which spellings become one
``ktt::rms_norm`` call, which are left alone, and that the rewritten graph computes the
chain's result (CPU: ``ktt::rms_norm``'s composite kernel, fp32 inside)."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import kohakutt_amd  # noqa: F401  (registers ktt::rms_norm)
from kohakutt_amd import chains


def _compile(fn, *args):
    """Runs fn through torch.compile with the rewrite; returns (result, rewrites, code)."""
    seen = []

    def backend(gm, example_inputs):
        n = chains.rewrite_rms_norms(gm)
        seen.append((n, gm.code))
        return gm.forward

    torch._dynamo.reset()
    out = torch.compile(fn, backend=backend, fullgraph=True)(*args)
    assert len(seen) == 1
    return out, seen[0][0], seen[0][1]


def _hf(x, w, eps=1e-6):
    h = x.to(torch.float32)
    v = h.pow(2).mean(-1, keepdim=True)
    h = h * torch.rsqrt(v + eps)
    return w * h.to(x.dtype)


def _rel(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


def test_hugging_face_spelling_becomes_one_call():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(3, 7, 896, generator=g).bfloat16()
    w = (1 + 0.02 * torch.randn(896, generator=g)).bfloat16()
    y, n, code = _compile(_hf, x, w)
    assert n == 1 and code.count("ktt.rms_norm") == 1
    assert "rsqrt" not in code and "mean" not in code and "pow" not in code
    assert y.dtype == torch.bfloat16 and y.shape == x.shape
    ref = F.rms_norm(x.double(), [896], w.double(), 1e-6)
    # One rounding instead of the chain's two (bf16 before the weight product).
    assert _rel(y, ref) <= 1.5 * _rel(_hf(x, w), ref) + 1e-3


def test_square_as_product_weight_second_fp32():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(5, 64, generator=g)
    w = torch.randn(64, generator=g)

    def f(x, w):
        return (x * torch.rsqrt(torch.mean(x * x, dim=-1, keepdim=True) + 1e-5)) * w

    y, n, code = _compile(f, x, w)
    assert n == 1 and "ktt.rms_norm" in code
    torch.testing.assert_close(y, F.rms_norm(x, [64], w, 1e-5), rtol=1e-5, atol=1e-6)


def test_no_weight_and_two_norms_in_one_graph():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(4, 32, generator=g)

    def f(x):
        a = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)
        b = a + 1
        return b * torch.rsqrt(b.pow(2).mean(dim=[-1], keepdim=True) + 1e-6)

    y, n, code = _compile(f, x)
    assert n == 2 and code.count("ktt.rms_norm") == 2
    torch.testing.assert_close(y, f(x), rtol=1e-5, atol=1e-6)


def test_wider_result_reads_the_fp32_cast():
    """A bf16 input normalised in fp32 and multiplied by an fp32 weight ends in fp32: the
    fused op reads the fp32 cast (ktt::rms_norm returns its input's dtype)."""
    g = torch.Generator().manual_seed(4)
    x = torch.randn(6, 128, generator=g).bfloat16()
    w = torch.randn(128, generator=g)

    def f(x, w):
        h = x.float()
        return h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6) * w

    y, n, code = _compile(f, x, w)
    assert n == 1 and y.dtype == torch.float32
    torch.testing.assert_close(y, f(x, w), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("case", ["grad", "shared_variance", "first_dim", "no_keepdim", "cube"])
def test_left_alone(case):
    g = torch.Generator().manual_seed(5)
    x = torch.randn(4, 16, generator=g)
    w = torch.randn(16, generator=g)
    if case == "grad":
        x.requires_grad_()

        def f(x, w):
            return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * w
    elif case == "shared_variance":

        def f(x, w):
            v = x.pow(2).mean(-1, keepdim=True)
            return x * torch.rsqrt(v + 1e-6) * w, v
    elif case == "first_dim":

        def f(x, w):
            return x * torch.rsqrt(x.pow(2).mean(0, keepdim=True) + 1e-6)
    elif case == "no_keepdim":

        def f(x, w):
            return (x.t() * torch.rsqrt(x.pow(2).mean(-1) + 1e-6)).t()
    else:

        def f(x, w):
            return x * torch.rsqrt(x.pow(3).mean(-1, keepdim=True) + 1e-6)

    y, n, code = _compile(f, x, w)
    assert n == 0 and "ktt.rms_norm" not in code


def test_env_selects_the_rewrites(monkeypatch):
    g = torch.Generator().manual_seed(6)
    x = torch.randn(2, 64, generator=g).bfloat16()
    w = torch.ones(64, dtype=torch.bfloat16)
    monkeypatch.setenv("KTT_FUSE_CHAINS", "0")
    assert _compile(_hf, x, w)[1] == 0
    monkeypatch.setenv("KTT_FUSE_CHAINS", "Mask, GQA")
    assert chains.selected() == {"mask", "gqa"}
    assert _compile(_hf, x, w)[1] == 0
    monkeypatch.setenv("KTT_FUSE_CHAINS", "norm")
    assert _compile(_hf, x, w)[1] == 1
    monkeypatch.setenv("KTT_FUSE_CHAINS", "all")
    assert chains.selected() == set(chains.REWRITES)
    monkeypatch.setenv("KTT_FUSE_CHAINS", "norm,fuse")
    with pytest.raises(ValueError, match="unknown rewrite.*fuse"):
        chains.selected()


@pytest.mark.parametrize("order", ["xw_r", "w_xr", "r_wx", "cast_r"])
def test_factor_order_and_nesting_do_not_matter(order):
    """The product is matched as a factor set: any nesting of x, the statistic and the
    weight is one call, and a cast on the statistic factor is peeled."""
    g = torch.Generator().manual_seed(9)
    x = torch.randn(6, 48, generator=g)
    w = torch.randn(48, generator=g)

    def f(x, w):
        r = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-5)
        if order == "xw_r":
            return (x * w) * r
        if order == "w_xr":
            return w * (x * r)
        if order == "r_wx":
            return r * (w * x)
        return x * r.to(torch.float32) * w

    y, n, code = _compile(f, x, w)
    assert n == 1 and code.count("ktt.rms_norm") == 1
    torch.testing.assert_close(y, F.rms_norm(x, [48], w, 1e-5), rtol=1e-5, atol=1e-6)


def test_in_place_write_inside_the_region_is_refused():
    g = torch.Generator().manual_seed(10)
    x = torch.randn(4, 32, generator=g)

    def f(x):
        r = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)
        x.mul_(2)
        return x * r

    y, n, code = _compile(f, x.clone())
    assert n == 0 and "ktt.rms_norm" not in code


@pytest.mark.parametrize("extra", ["weight_twice", "scalar"])
def test_extra_factors_stay_outside_the_fused_call(extra):
    """A product with more factors than a norm keeps the extra ones: the largest
    sub-product that is a norm becomes the call and the rest multiplies its result."""
    g = torch.Generator().manual_seed(11)
    x = torch.randn(4, 32, generator=g)
    w = torch.randn(32, generator=g)

    def f(x, w):
        r = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)
        return x * r * w * w if extra == "weight_twice" else x * r * 2.0

    y, n, code = _compile(f, x, w)
    assert n == 1 and code.count("ktt.rms_norm") == 1
    ref = F.rms_norm(x, [32], w, 1e-6) * w if extra == "weight_twice" else F.rms_norm(x, [32], None, 1e-6) * 2.0
    torch.testing.assert_close(y, ref, rtol=1e-5, atol=1e-5)


def test_shared_statistic_is_left_alone():
    g = torch.Generator().manual_seed(12)
    x = torch.randn(4, 32, generator=g)
    w = torch.randn(32, generator=g)

    def f(x, w):
        r = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)
        return x * r * w, r

    y, n, code = _compile(f, x, w)
    assert n == 0 and "ktt.rms_norm" not in code


def test_transformers_qwen2_norm_module():
    transformers = pytest.importorskip("transformers")
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RMSNorm

    g = torch.Generator().manual_seed(7)
    norm = Qwen2RMSNorm(896, eps=1e-6).to(torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.02 * torch.randn(896, generator=g))
    x = torch.randn(2, 9, 896, generator=g).bfloat16()
    with torch.no_grad():
        y, n, code = _compile(norm, x)
        ref = F.rms_norm(x.double(), [896], norm.weight.double(), 1e-6)
        assert n == 1 and "ktt.rms_norm" in code
        assert _rel(y, ref) <= 1.5 * _rel(norm(x), ref) + 1e-3
    assert transformers is not None


def test_backend_entry_point():
    g = torch.Generator().manual_seed(8)
    x = torch.randn(3, 40, generator=g)
    torch._dynamo.reset()
    y = torch.compile(lambda x: x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6),
                      backend=chains.backend)(x)
    torch.testing.assert_close(y, F.rms_norm(x, [40], None, 1e-6), rtol=1e-5, atol=1e-6)
