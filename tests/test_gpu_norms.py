"""GPU parity of LayerNorm / RMSNorm against float64, with the reference's bar
(``tests/hardware/ops/test_norm.py:25-38,95-113``): relative RMS error of y no worse than
1.02x torch CPU at the same dtype (plus a 2e-6 floor for fp32), fp32 statistics within
1e-6 relative of float64, repeat calls bit-identical (``test_norm.py:186-192``)."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import attn_cases as C
from oracle import norms as onorm

pytestmark = pytest.mark.gpu

SHAPES = [(1, 33), (5, 70), (32, 64), (77, 1000), (2, 40, 4096), (3, 16384), (4096, 768), (65536, 64),
          (300, 4097), (2, 3, 50, 1280), (5, 2056), (7, 12288), (9, 8192)]
SLACK = 1.02


def _rel(a, ref):
    a = torch.as_tensor(a).double().flatten()
    ref = torch.as_tensor(ref).double().flatten()
    return ((a - ref).norm() / ref.norm().clamp_min(1e-300)).item()


def _check(name, gpu, cpu, ref, dtype):
    assert torch.isfinite(gpu).all(), name
    t, c = _rel(gpu, ref), _rel(cpu, ref)
    floor = 2e-6 if dtype == torch.float32 else 0.0
    print(f"{name}: gpu {t:.3e} cpu {c:.3e}", flush=True)
    assert t <= SLACK * c + floor, (name, t, c)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("affine", [True, False])
def test_layer_norm(native, dev, shape, dtype, affine):
    g = C.gen(hash((shape, affine)) % 10000)
    x = (torch.randn(*shape, generator=g) * 3 + 0.5).to(dtype)
    w = (1 + 0.1 * torch.randn(shape[-1], generator=g)).to(dtype) if affine else None
    b = (0.1 * torch.randn(shape[-1], generator=g)).to(dtype) if affine else None
    native.reset_counters()
    y, mean, rstd = torch.ops.aten.native_layer_norm(
        x.to(dev), [shape[-1]], None if w is None else w.to(dev), None if b is None else b.to(dev), 1e-5)
    torch.cuda.synchronize()
    assert native.counters()["norms"] == 1
    assert mean.dtype == torch.float32 and rstd.dtype == torch.float32
    yr, mr, rr = onorm.layer_norm(C.f64(x), None if w is None else C.f64(w), None if b is None else C.f64(b), 1e-5)
    cpu = F.layer_norm(x, [shape[-1]], w, b, 1e-5)
    _check(f"LN {shape} {dtype} affine={affine}", y.cpu(), cpu, torch.from_numpy(yr), dtype)
    assert np.allclose(mean.cpu().double().numpy(), mr, rtol=1e-6, atol=1e-6 * np.abs(mr).max())
    assert np.allclose(rstd.cpu().double().numpy(), rr, rtol=1e-6, atol=0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", SHAPES)
def test_rms_norm(native, dev, shape, dtype):
    g = C.gen(hash(shape) % 10000 + 7)
    x = (torch.randn(*shape, generator=g) * 2).to(dtype)
    w = (1 + 0.1 * torch.randn(shape[-1], generator=g)).to(dtype)
    native.reset_counters()
    y = F.rms_norm(x.to(dev), [shape[-1]], w.to(dev), 1e-6)
    torch.cuda.synchronize()
    assert native.counters()["norms"] == 1
    yr, _ = onorm.rms_norm(C.f64(x), C.f64(w), eps=1e-6)
    # the reference's CPU path at the same dtype (tests/hardware/ops/test_norm.py:25-38)
    cpu = F.rms_norm(x, [shape[-1]], w, 1e-6)
    _check(f"RMS {shape} {dtype}", y.cpu(), cpu, torch.from_numpy(yr), dtype)


def test_ktt_rms_norm_bias_and_stats(native, dev):
    g = C.gen(31)
    x = C.randn(g, 7, 896)
    w = C.randn(g, 896)
    b = C.randn(g, 896)
    y = torch.ops.ktt.rms_norm(x.to(dev), w.to(dev), b.to(dev), 1e-6).cpu()
    yr, _ = onorm.rms_norm(C.f64(x), C.f64(w), C.f64(b), eps=1e-6)
    # ktt::rms_norm's CPU path: the fp32 composite (aten_fused.cpp:13-28) rounded once
    cpu = torch.ops.ktt.rms_norm(x, w, b, 1e-6)
    _check("ktt.rms_norm bias", y, cpu, torch.from_numpy(yr), torch.bfloat16)


def test_rms_norm_backward_matches_float64(native, dev):
    g = C.gen(32)
    x = torch.randn(16, 256, generator=g, dtype=torch.float64)
    w = 1 + 0.1 * torch.randn(256, generator=g, dtype=torch.float64)
    gy = torch.randn(16, 256, generator=g, dtype=torch.float64)
    xd = x.float().to(dev).requires_grad_()
    wd = w.float().to(dev).requires_grad_()
    F.rms_norm(xd, [256], wd, 1e-6).backward(gy.float().to(dev))
    xr = x.clone().requires_grad_()
    wr = w.clone().requires_grad_()
    F.rms_norm(xr, [256], wr, 1e-6).backward(gy)
    assert torch.allclose(xd.grad.cpu().double(), xr.grad, rtol=1e-4, atol=1e-5)
    assert torch.allclose(wd.grad.cpu().double(), wr.grad, rtol=1e-4, atol=1e-4)


def test_layer_norm_backward_uses_fp32_stats(native, dev):
    g = C.gen(33)
    x = torch.randn(8, 512, generator=g, dtype=torch.float64)
    w = 1 + 0.1 * torch.randn(512, generator=g, dtype=torch.float64)
    b = 0.1 * torch.randn(512, generator=g, dtype=torch.float64)
    gy = torch.randn(8, 512, generator=g, dtype=torch.float64)
    xd = x.float().to(dev).requires_grad_()
    F.layer_norm(xd, [512], w.float().to(dev), b.float().to(dev), 1e-5).backward(gy.float().to(dev))
    xr = x.clone().requires_grad_()
    F.layer_norm(xr, [512], w, b, 1e-5).backward(gy)
    assert torch.allclose(xd.grad.cpu().double(), xr.grad, rtol=1e-4, atol=1e-5)


def test_norm_configs_and_repeat_bit_identical(native, dev):
    c1, c2, c3, c5 = C.config1(), C.config2(), C.config3(), C.config5()
    for name, x, w, b, eps, kind in [
        ("C1 rms [1,2048,896]", c1["x"], c1["w"], None, 1e-6, "rms"),
        ("C2 LN [1,197,768]", c2["x"], c2["w"], c2["b"], 1e-6, "ln"),
        ("C3 rms [8,1,2048]", c3["x"], c3["w"], None, 1e-6, "rms"),
        ("C5 LN [2,4096,640]", c5["x"], c5["w"], c5["b"], 1e-5, "ln"),
    ]:
        xd, wd = x.to(dev), w.to(dev)
        W = x.size(-1)
        if kind == "rms":
            y = F.rms_norm(xd, [W], wd, eps)
            y2 = F.rms_norm(xd, [W], wd, eps)
            yr, _ = onorm.rms_norm(C.f64(x), C.f64(w), eps=eps)
            cpu = F.rms_norm(x, [W], w, eps)
        else:
            y = F.layer_norm(xd, [W], wd, b.to(dev), eps)
            y2 = F.layer_norm(xd, [W], wd, b.to(dev), eps)
            yr, _, _ = onorm.layer_norm(C.f64(x), C.f64(w), C.f64(b), eps)
            cpu = F.layer_norm(x, [W], w, b, eps)
        assert torch.equal(y, y2), name
        _check(name, y.cpu(), cpu, torch.from_numpy(yr), torch.bfloat16)


@pytest.mark.parametrize(
    "shape,x_dtype,w_dtype",
    [
        ((2048, 896), torch.bfloat16, torch.bfloat16),
        ((8, 1, 2048), torch.float16, torch.float32),
        ((3, 5, 77), torch.float32, None),
        ((4100, 640), torch.bfloat16, torch.bfloat16),
    ],
)
def test_rms_norm_backward_kernels_match_float64(native, dev, shape, x_dtype, w_dtype):
    """F.rms_norm gradients from the backward kernels (dx per row, dw as a fixed-order
    column sum over row chunks) against float64 autograd on the CPU; repeat calls are
    bit-identical."""
    g = torch.Generator().manual_seed(31 + len(shape))
    width = shape[-1]
    x = torch.randn(*shape, generator=g).to(x_dtype)
    gy = torch.randn(*shape, generator=g).to(x_dtype)
    w = None if w_dtype is None else (1 + 0.02 * torch.randn(width, generator=g)).to(w_dtype)
    xd = x.to(dev).requires_grad_()
    wd = None if w is None else w.to(dev).requires_grad_()
    native.reset_counters()
    F.rms_norm(xd, (width,), wd, 1e-6).backward(gy.to(dev))
    torch.cuda.synchronize()
    assert native.counters()["norms_backward"] == 1
    x64 = x.double().requires_grad_()
    w64 = None if w is None else w.double().requires_grad_()
    F.rms_norm(x64, (width,), w64, 1e-6).backward(gy.double())
    pairs = [(xd.grad, x64.grad)] + ([] if w is None else [(wd.grad, w64.grad)])
    for got, want in pairs:
        err = (got.cpu().double() - want).abs()
        scale = want.abs().max().item()
        tol = 2e-2 if got.dtype in (torch.bfloat16, torch.float16) else 1e-4
        assert err.max().item() <= tol * max(scale, 1.0), (got.dtype, err.max().item(), scale)
    first = [t.clone() for t, _ in pairs]
    xd.grad = None
    if wd is not None:
        wd.grad = None
    F.rms_norm(xd, (width,), wd, 1e-6).backward(gy.to(dev))
    torch.cuda.synchronize()
    again = [xd.grad] + ([] if wd is None else [wd.grad])
    assert all(torch.equal(a, b) for a, b in zip(first, again))


LN_BWD = [
    # shape, x dtype, weight dtype (None: no affine), bias
    ((1, 197, 768), torch.bfloat16, torch.bfloat16, True),
    ((2, 4096, 640), torch.bfloat16, torch.bfloat16, True),
    ((33, 64), torch.float16, torch.float32, True),
    ((5, 7, 1000), torch.float32, torch.float32, False),
    ((3, 2048), torch.bfloat16, None, False),
    ((1025, 128), torch.bfloat16, torch.bfloat16, False),
]


@pytest.mark.parametrize("shape,x_dtype,w_dtype,has_bias", LN_BWD)
def test_layer_norm_backward_kernel(native, dev, shape, x_dtype, w_dtype, has_bias):
    """aten::native_layer_norm_backward on the one-pass kernel: dx, dweight, dbias against
    float64 autograd; median relative error at most 1.5x torch CPU autograd at the same
    dtype; repeat calls bit-identical."""
    from oracle.ruler import diff_stats

    print(f"LN backward {shape} {x_dtype} {w_dtype} bias={has_bias}", flush=True)
    g = torch.Generator().manual_seed(41 + shape[-1])
    width = shape[-1]
    x = (torch.randn(*shape, generator=g) * 2 + 0.3).to(x_dtype)
    gy = torch.randn(*shape, generator=g).to(x_dtype)
    w = None if w_dtype is None else (1 + 0.1 * torch.randn(width, generator=g)).to(w_dtype)
    b = None if not has_bias else (0.1 * torch.randn(width, generator=g)).to(w_dtype)

    def run(device, dtype=None):
        # Fresh leaves every run (x.to("cpu") would be x itself).
        cast = (lambda t: t.to(dtype)) if dtype is not None else (lambda t: t)
        xx = cast(x).to(device).detach().clone().requires_grad_()
        ww = None if w is None else cast(w).to(device).detach().clone().requires_grad_()
        bb = None if b is None else cast(b).to(device).detach().clone().requires_grad_()
        F.layer_norm(xx, (width,), ww, bb, 1e-5).backward(cast(gy).to(device))
        return [t.grad for t in (xx, ww, bb) if t is not None]

    native.reset_counters()
    got = run(dev)
    torch.cuda.synchronize()
    assert native.counters()["norms_backward"] == 1, native.counters()
    ref = run("cpu", torch.float64)
    cpu = run("cpu")
    for name, a, c, r in zip(("dx", "dw", "db"), got, cpu, ref):
        sg, sc = diff_stats(a.cpu(), r), diff_stats(c, r)
        print(f"  {name}: gpu rel_median {sg['rel_median']:.2e} cpu {sc['rel_median']:.2e}", flush=True)
        assert sg["nonfinite"] == 0 and sg["rel_median"] <= 1.5 * sc["rel_median"] + 1e-7, (name, sg, sc)
    again = run(dev)
    torch.cuda.synchronize()
    assert all(torch.equal(a, b2) for a, b2 in zip(got, again))


def test_norm_backward_column_sums_are_the_same_on_every_stream(native, dev):
    """dweight / dbias add their blocks' partials in two levels: in one launch (the last
    part of a column chunk to finish adds the parts, found by a per-stream counter that it
    clears) on up to 16 streams, and in a second launch with the same additions beyond
    them: twenty streams in turn, each called twice, give bit-identical gradients."""
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(4096, 640, generator=g) * 2 + 0.3).bfloat16().to(dev)
    gy = torch.randn(4096, 640, generator=g).bfloat16().to(dev)
    w = (1 + 0.1 * torch.randn(640, generator=g)).bfloat16().to(dev)
    b = (0.1 * torch.randn(640, generator=g)).bfloat16().to(dev)

    def run():
        xx, ww, bb = (t.detach().clone().requires_grad_() for t in (x, w, b))
        F.layer_norm(xx, (640,), ww, bb, 1e-5).backward(gy)
        rr, rw = xx.detach().clone().requires_grad_(), w.detach().clone().requires_grad_()
        F.rms_norm(rr, (640,), rw, 1e-6).backward(gy)
        return [xx.grad, ww.grad, bb.grad, rr.grad, rw.grad]

    first = run()
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in range(20)]
    for i, s in enumerate(streams):
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for rep in range(2):
                got = run()
                s.synchronize()
                assert all(torch.equal(a, f) for a, f in zip(got, first)), (i, rep)


@pytest.mark.parametrize("case", ["x_offset_1", "weight_slice_bf16", "weight_slice_f32"])
def test_layer_norm_backward_misaligned_operands(native, dev, case):
    """A contiguous x at storage offset 1 and a weight sliced at offset 4 from a flat
    parameter buffer are valid LayerNorm inputs: the forward takes them and the backward
    (whose one-pass kernel needs 16-byte vectors) copies the misaligned operand once and
    runs the kernel; the gradients match float64 autograd under the ruler."""
    from oracle.ruler import diff_stats

    print(f"LN backward misaligned {case}", flush=True)
    g = torch.Generator().manual_seed(43)
    rows, width = 37, 256
    wdt = torch.float32 if case == "weight_slice_f32" else torch.bfloat16
    xs = torch.randn(rows * width + 1, generator=g).bfloat16()
    ws = (1 + 0.1 * torch.randn(width + 4, generator=g)).to(wdt)
    b = (0.1 * torch.randn(width, generator=g)).to(wdt)
    gy = torch.randn(rows, width, generator=g).bfloat16()
    x_off = 1 if case == "x_offset_1" else 0
    w_off = 4 if case != "x_offset_1" else 0

    def run(device, dtype=None):
        cast = (lambda t: t.to(dtype)) if dtype is not None else (lambda t: t)
        xbuf = cast(xs).to(device).detach().clone().requires_grad_()
        wbuf = cast(ws).to(device).detach().clone().requires_grad_()
        bb = cast(b).to(device).detach().clone().requires_grad_()
        x = xbuf[x_off:x_off + rows * width].view(rows, width)
        w = wbuf[w_off:w_off + width]
        F.layer_norm(x, (width,), w, bb, 1e-5).backward(cast(gy).to(device))
        return (xbuf.grad[x_off:x_off + rows * width].view(rows, width), wbuf.grad[w_off:w_off + width], bb.grad)

    native.reset_counters()
    got = run(dev)
    torch.cuda.synchronize()
    c = native.counters()
    assert c["norms"] == 1 and c["norms_backward"] == 1, c
    ref, cpu = run("cpu", torch.float64), run("cpu")
    for name, a, c, r in zip(("dx", "dw", "db"), got, cpu, ref):
        sg, sc = diff_stats(a.cpu(), r), diff_stats(c, r)
        assert sg["nonfinite"] == 0 and sg["rel_median"] <= 1.5 * sc["rel_median"] + 1e-7, (name, sg, sc)


def test_layer_norm_backward_wide_rows_keep_torch_kernel(native, dev):
    """Rows past 256 vectors take torch's own CUDA backward (fed this build's statistics)."""
    x = torch.randn(4, 4096, device=dev, dtype=torch.bfloat16, requires_grad=True)
    native.reset_counters()
    F.layer_norm(x, (4096,)).sum().backward()
    torch.cuda.synchronize()
    c = native.counters()
    assert c["norms"] == 1 and c["norms_backward"] == 0, c
    assert torch.isfinite(x.grad).all()


def _rows_close(got, want, tol):
    err = (got.double() - want).abs().max().item()
    assert err <= tol * max(want.abs().max().item(), 1.0), (err, tol)


def test_row_counts_past_one_grid_dimension(native, dev):
    """Row counts whose one-block-per-row (2^24 rows) or one-wavefront-per-row (2^26 rows)
    grids pass HIP's 2^32 work-items per grid dimension: forward element path, forward
    wavefront path and the RMSNorm backward element path, checked on the first and last
    rows against float64 (rows are independent) and dweight against its float64 sum."""
    g = torch.Generator(device=dev).manual_seed(61)
    sample = lambda t: torch.cat([t[:2048], t[-2048:]]).cpu()  # noqa: E731

    rows = (1 << 24) + 3  # width 3: the element path, one block per row
    x = torch.randn(rows, 3, device=dev, generator=g).bfloat16()
    w = (1 + 0.05 * torch.randn(3, device=dev, generator=g)).bfloat16()
    native.reset_counters()
    y = F.rms_norm(x, (3,), w, 1e-6)
    torch.cuda.synchronize()
    assert native.counters()["norms"] == 1
    want, _ = onorm.rms_norm(sample(x).double().numpy(), w.cpu().double().numpy(), eps=1e-6)
    _rows_close(sample(y), torch.from_numpy(want), 2e-2)

    xg = x.clone().requires_grad_()
    wg = w.clone().requires_grad_()
    dy = torch.randn(rows, 3, device=dev, generator=g).bfloat16()
    F.rms_norm(xg, (3,), wg, 1e-6).backward(dy)
    torch.cuda.synchronize()
    assert native.counters()["norms_backward"] == 1
    xs = sample(x).double().requires_grad_()
    F.rms_norm(xs, (3,), w.cpu().double(), 1e-6).backward(sample(dy).double())
    _rows_close(sample(xg.grad), xs.grad, 2e-2)
    x64, dy64 = x.double(), dy.double()
    r64 = torch.rsqrt(x64.pow(2).mean(-1, keepdim=True) + 1e-6)
    terms = dy64 * x64 * r64
    dw = terms.sum(0).cpu()
    spread = terms.pow(2).sum(0).sqrt().cpu()
    assert ((wg.grad.cpu().double() - dw).abs() <= 1e-2 * spread + 1e-3 * dw.abs()).all(), (wg.grad, dw)
    del xg, wg, dy, x64, dy64, r64, terms

    rows = (1 << 26) + 5  # width 8: one 16-byte vector, one wavefront per row
    x = torch.randn(rows, 8, device=dev, generator=g).bfloat16()
    wl = (1 + 0.05 * torch.randn(8, device=dev, generator=g)).bfloat16()
    bl = (0.1 * torch.randn(8, device=dev, generator=g)).bfloat16()
    y, mean, rstd = torch.native_layer_norm(x, (8,), wl, bl, 1e-5)
    torch.cuda.synchronize()
    want, m64, r64 = onorm.layer_norm(sample(x).double().numpy(), wl.cpu().double().numpy(),
                                      bl.cpu().double().numpy(), eps=1e-5)
    _rows_close(sample(y), torch.from_numpy(want), 2e-2)
    _rows_close(sample(rstd), torch.from_numpy(r64), 1e-5)
    _rows_close(sample(mean), torch.from_numpy(m64), 1e-5)


def test_rms_norm_forward_and_backward_capture_in_a_graph(native, dev):
    """RMSNorm forward and backward captured in one HIP graph after a side-stream warm-up
    (the autograd engine runs each backward node on its forward's stream, so the forward
    is captured on the capture stream too); every replay matches the eager result."""
    g = torch.Generator().manual_seed(77)
    x = torch.randn(2048, 896, generator=g).bfloat16().to(dev).requires_grad_()
    w = (1 + 0.02 * torch.randn(896, generator=g)).bfloat16().to(dev).requires_grad_()
    gy = torch.randn(2048, 896, generator=g).bfloat16().to(dev)

    def step():
        x.grad = None
        w.grad = None
        y = F.rms_norm(x, (896,), w, 1e-6)
        y.backward(gy)
        return y

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    y_eager = step().detach().clone()
    dx_eager, dw_eager = x.grad.clone(), w.grad.clone()
    graph = torch.cuda.CUDAGraph()
    x.grad = None
    w.grad = None
    with torch.cuda.graph(graph):
        y_static = F.rms_norm(x, (896,), w, 1e-6)
        y_static.backward(gy)
    dx_static, dw_static = x.grad, w.grad
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_static, y_eager)
        assert torch.equal(dx_static, dx_eager) and torch.equal(dw_static, dw_eager)
        step()  # eager work between replays
        torch.cuda.synchronize()


def test_compiled_rms_norm_chain_runs_the_kernel(native, dev):
    """torch.compile with kohakutt_amd.chains.backend turns a Hugging Face RMSNorm chain
    into ktt::rms_norm, which runs the norm kernel on the GPU (one call, counted)."""
    from kohakutt_amd import chains

    g = torch.Generator().manual_seed(91)
    x = torch.randn(2, 37, 896, generator=g).bfloat16()
    w = (1 + 0.02 * torch.randn(896, generator=g)).bfloat16()

    def hf(x, w):
        h = x.to(torch.float32)
        h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6)
        return w * h.to(x.dtype)

    torch._dynamo.reset()
    f = torch.compile(hf, backend=chains.backend, fullgraph=True)
    native.reset_counters()
    y = f(x.to(dev), w.to(dev))
    torch.cuda.synchronize()
    assert native.counters()["norms"] == 1, native.counters()
    ref = F.rms_norm(x.double(), [896], w.double(), 1e-6)
    _check("compiled rms chain", y.cpu(), hf(x, w), ref, torch.bfloat16)
