"""ctypes binding of the C ABI (``include/kohakutt_amd.h``).

The torch op layer (``_torch_ops.so``) is the library's own caller; this binding is
what a non-torch host (or a test) uses to call ``libkohakutt_amd.so`` directly with raw
device pointers.  The reference's counterpart is its own ctypes binding of
``ktt_capi.h`` (``src/kohakutt/tinygrad_backend``).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libkohakutt_amd.so"

KMI_BF16, KMI_F16, KMI_F32, KMI_BOOL = 1, 2, 3, 4
KMI_OK, KMI_EINVAL, KMI_EUNSUPPORTED, KMI_EHIP, KMI_EWORKSPACE = 0, -1, -2, -3, -4
KMI_MASK_NONE, KMI_MASK_STRIDED, KMI_MASK_PACKED = 0, 1, 2

EXPORTS = (
    "kmi_attn_workspace_bytes",
    "kmi_attn_fwd",
    "kmi_attn_fwd_noalloc",
    "kmi_attn_bwd_workspace_bytes",
    "kmi_attn_bwd",
    "kmi_layer_norm_fwd",
    "kmi_rms_norm_fwd",
    "kmi_rms_norm_bwd_workspace_bytes",
    "kmi_rms_norm_bwd",
    "kmi_layer_norm_bwd_workspace_bytes",
    "kmi_layer_norm_bwd",
    "kmi_last_error",
    "kmi_abi_version",
)

_I64x3 = ctypes.c_int64 * 3
_I64x4 = ctypes.c_int64 * 4


class AttnArgs(ctypes.Structure):
    """``kmi_attn_args``, field for field."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("causal", ctypes.c_int32),
        ("batch", ctypes.c_int64),
        ("heads_q", ctypes.c_int64),
        ("heads_kv", ctypes.c_int64),
        ("seq_q", ctypes.c_int64),
        ("seq_k", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("q_stride", _I64x3),
        ("k_stride", _I64x3),
        ("v_stride", _I64x3),
        ("o_stride", _I64x3),
        ("lse_stride", _I64x3),
        ("scale", ctypes.c_double),
        ("mask", ctypes.c_void_p),
        ("mask_dtype", ctypes.c_int32),
        ("mask_mode", ctypes.c_int32),
        ("mask_stride", _I64x4),
        ("mask_numel", ctypes.c_int64),
        ("cu_seqlens_q", ctypes.c_void_p),
        ("cu_seqlens_k", ctypes.c_void_p),
        ("total_q", ctypes.c_int64),
        ("total_k", ctypes.c_int64),
        ("num_splits", ctypes.c_int32),
        ("head_dim_v", ctypes.c_int32),
        ("key_lengths", ctypes.c_void_p),
        ("mask_offsets", ctypes.c_void_p),
    ]


class AttnBwdArgs(ctypes.Structure):
    """``kmi_attn_bwd_args``, field for field."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("grad_out", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("grad_q", ctypes.c_void_p),
        ("grad_k", ctypes.c_void_p),
        ("grad_v", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("causal", ctypes.c_int32),
        ("batch", ctypes.c_int64),
        ("heads_q", ctypes.c_int64),
        ("heads_kv", ctypes.c_int64),
        ("seq_q", ctypes.c_int64),
        ("seq_k", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("q_stride", _I64x3),
        ("k_stride", _I64x3),
        ("v_stride", _I64x3),
        ("o_stride", _I64x3),
        ("do_stride", _I64x3),
        ("dq_stride", _I64x3),
        ("dk_stride", _I64x3),
        ("dv_stride", _I64x3),
        ("lse_stride", _I64x3),
        ("scale", ctypes.c_double),
        ("mask", ctypes.c_void_p),
        ("mask_dtype", ctypes.c_int32),
        ("mask_mode", ctypes.c_int32),
        ("mask_stride", _I64x4),
        ("mask_numel", ctypes.c_int64),
        ("mask_offsets", ctypes.c_void_p),
        ("cu_seqlens_q", ctypes.c_void_p),
        ("cu_seqlens_k", ctypes.c_void_p),
        ("total_q", ctypes.c_int64),
        ("total_k", ctypes.c_int64),
        ("key_lengths", ctypes.c_void_p),
        ("head_dim_v", ctypes.c_int64),
    ]


class KmiError(RuntimeError):
    def __init__(self, status, message):
        super().__init__(f"kmi status {status}: {message}")
        self.status = status


_LIB = None


def lib():
    """The loaded ``libkohakutt_amd.so`` with argument types set (ImportError if absent)."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise ImportError(f"kohakutt_amd: {LIB_PATH.name} is not built")
        h = ctypes.CDLL(str(LIB_PATH))
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
        h.kmi_attn_workspace_bytes.argtypes = [ctypes.POINTER(AttnArgs), ctypes.POINTER(ctypes.c_size_t)]
        h.kmi_attn_fwd.argtypes = [ctypes.POINTER(AttnArgs), vp, ctypes.c_size_t, vp]
        h.kmi_attn_fwd_noalloc.argtypes = [ctypes.POINTER(AttnArgs), vp]
        h.kmi_attn_bwd_workspace_bytes.argtypes = [ctypes.POINTER(AttnBwdArgs), ctypes.POINTER(ctypes.c_size_t)]
        h.kmi_attn_bwd.argtypes = [ctypes.POINTER(AttnBwdArgs), vp, ctypes.c_size_t, vp]
        h.kmi_layer_norm_fwd.argtypes = [vp, vp, vp, vp, vp, vp, i64, i64, i32, i32, i32, ctypes.c_double, vp]
        h.kmi_rms_norm_fwd.argtypes = [vp, vp, vp, vp, vp, i64, i64, i32, i32, i32, ctypes.c_double, vp]
        h.kmi_rms_norm_bwd_workspace_bytes.argtypes = [i64, i64, ctypes.POINTER(ctypes.c_size_t)]
        h.kmi_rms_norm_bwd.argtypes = [vp, vp, vp, vp, vp, vp, i64, i64, i32, i32, vp, ctypes.c_size_t, vp]
        h.kmi_layer_norm_bwd_workspace_bytes.argtypes = [i64, i64, ctypes.POINTER(ctypes.c_size_t)]
        h.kmi_layer_norm_bwd.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, i32, i32, i32, vp,
                                         ctypes.c_size_t, vp]
        h.kmi_last_error.restype = ctypes.c_char_p
        h.kmi_last_error.argtypes = []
        h.kmi_abi_version.argtypes = []
        for name in EXPORTS:
            if name not in ("kmi_last_error",):
                getattr(h, name).restype = ctypes.c_int
        _LIB = h
    return _LIB


def check(status: int) -> None:
    if status != KMI_OK:
        raise KmiError(status, lib().kmi_last_error().decode())


def workspace_bytes(args: AttnArgs) -> int:
    n = ctypes.c_size_t(0)
    check(lib().kmi_attn_workspace_bytes(ctypes.byref(args), ctypes.byref(n)))
    return n.value


def attn_fwd(args: AttnArgs, workspace: int, workspace_bytes_: int, stream: int) -> None:
    check(lib().kmi_attn_fwd(ctypes.byref(args), workspace, workspace_bytes_, stream))


def attn_fwd_noalloc(args: AttnArgs, stream: int) -> None:
    check(lib().kmi_attn_fwd_noalloc(ctypes.byref(args), stream))


def layer_norm_fwd(x, w, b, y, mean, rstd, rows, width, x_dtype, w_dtype, b_dtype, eps, stream) -> None:
    check(lib().kmi_layer_norm_fwd(x, w, b, y, mean, rstd, rows, width, x_dtype, w_dtype, b_dtype, eps, stream))


def rms_norm_fwd(x, w, b, y, rstd, rows, width, x_dtype, w_dtype, b_dtype, eps, stream) -> None:
    check(lib().kmi_rms_norm_fwd(x, w, b, y, rstd, rows, width, x_dtype, w_dtype, b_dtype, eps, stream))
