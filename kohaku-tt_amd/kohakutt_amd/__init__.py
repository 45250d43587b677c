"""kohakutt_amd: Kohaku-TT's attention + norm hot path on MI355X (gfx950).

Importing the package loads ``_torch_ops.so``, whose static registrations put the
reference's op surface on the CUDA/HIP dispatch keys (the reference does the same for
PrivateUse1 when ``kohakutt`` is imported, ``src/kohakutt/torch_backend/registration.py:
13-27``):

* ``F.scaled_dot_product_attention`` on bf16 / fp16 GPU tensors routes to the
  ``overrideable`` backend (``aten::_fused_sdp_choice`` and its dispatch stub) and runs
  ``aten::_scaled_dot_product_fused_attention_overrideable`` on the gfx950 kernels;
* ``F.layer_norm`` (``aten::native_layer_norm``) and ``F.rms_norm`` (``aten::rms_norm`` at
  AutogradCUDA) run the gfx950 norm kernels with fp32 statistics;
* ``torch.ops.ktt.rms_norm``, ``torch.ops.ktt.sdpa_refusal`` and the reference's packed ops
  ``torch.ops.ktt._varlen_plan`` / ``_sdpa_varlen`` / ``_sdpa_varlen_backward``, plus this
  build's ``_sdpa_varlen_offsets`` (tensor offsets, per-row packed masks), all
  differentiable where the reference's are;
* ``torch.nn.attention.varlen.varlen_attn`` (``torch_attn::_varlen_attn`` and its
  backward) on GPU tensors.

Calls the kernels do not take keep torch's own CUDA/HIP paths.  The package raises
ImportError when its native libraries are missing: there is no CPU or eager fallback.
"""

from __future__ import annotations

from pathlib import Path

import torch

_PKG = Path(__file__).resolve().parent
CAPI_LIB = _PKG / "libkohakutt_amd.so"
OPS_LIB = _PKG / "_torch_ops.so"


def _load():
    missing = [p.name for p in (CAPI_LIB, OPS_LIB) if not p.exists()]
    if missing:
        raise ImportError(
            "kohakutt_amd: native libraries not built ("
            + ", ".join(missing)
            + "); run `python -c 'import __graft_entry__ as g; g.build()'` at the repo root"
        )
    torch.ops.load_library(str(OPS_LIB))


_load()

from . import attention  # noqa: E402
from . import chains  # noqa: E402,F401
from .attention import sdpa, sdpa_varlen  # noqa: E402,F401

attention.install()

AVAILABLE = True


def rms_norm(x, weight=None, bias=None, eps=1e-6):
    """RMSNorm over the last dim with an optional bias: ``ktt::rms_norm`` (the
    reference's ``torch.ops.ktt.rms_norm``, ``aten_fused.cpp:60-85``)."""
    return torch.ops.ktt.rms_norm(x, weight, bias, float(eps))


def set_enabled(attention: bool = True, norms: bool = True) -> None:
    """Switches the kernels on or off for attention and norms (off: torch's own paths)."""
    torch.ops.ktt._set_enabled(bool(attention), bool(norms))


def counters() -> dict:
    """Calls taken by the kernels since load (or ``reset_counters``)."""
    c = torch.ops.ktt.counters()
    return {
        "attention": c[0],
        "attention_declined": c[1],
        "norms": c[2],
        "attention_enabled": bool(c[3]),
        "norms_enabled": bool(c[4]),
        "attention_backward": c[5],
        "norms_backward": c[6],
    }


def reset_counters() -> None:
    torch.ops.ktt.reset_counters()


def sdpa_refusal(q, k, v, mask=None, dropout_p=0.0, is_causal=False, scale=None) -> str:
    """Why the kernels do not take this attention call ('' when they do); sizes, dtypes
    and devices only, so meta tensors answer too (``ktt::sdpa_refusal``)."""
    return torch.ops.ktt.sdpa_refusal(
        q, k, v, mask, float(dropout_p), bool(is_causal), None if scale is None else float(scale)
    )
