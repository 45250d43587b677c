"""The C ABI library (include/kohakutt_amd.h) on the CPU: it loads, exports every
function the header declares, and rejects malformed calls on the host -- before any
launch -- with a status and a kmi_last_error message (the reference's C ABI error model,
ktt_capi.h / capi.cpp:19,58-79).  No call here reaches a GPU."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from kohakutt_amd import capi

HEADER = Path(__file__).resolve().parent.parent / "include" / "kohakutt_amd.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kmi_[a-z_0-9]+)\s*\(", text)))


def test_header_declares_the_exports():
    assert _declared() == sorted(capi.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = capi.lib()
    for name in _declared():
        assert hasattr(lib, name), name


def test_abi_version_matches_header():
    m = re.search(r"#define KMI_ABI_VERSION (\d+)", HEADER.read_text())
    assert capi.lib().kmi_abi_version() == int(m.group(1))


@pytest.mark.parametrize("struct,cls", [("kmi_attn_args", "AttnArgs"), ("kmi_attn_bwd_args", "AttnBwdArgs")])
def test_struct_layout_matches_header_field_order(struct, cls):
    text = HEADER.read_text()
    start = text.index("{", text.index("typedef struct " + struct)) + 1
    body = text[start : text.index("} " + struct + ";")]
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    names = []
    for decl in body.split(";"):
        for part in decl.split(","):
            idents = re.findall(r"[A-Za-z_]\w*", re.sub(r"\[.*?\]", "", part))
            if idents:
                names.append(idents[-1])
    assert names == [f[0] for f in getattr(capi, cls)._fields_]


def _args(**kw):
    a = capi.AttnArgs()
    a.q = a.k = a.v = a.out = 0x1000
    a.dtype = capi.KMI_BF16
    a.batch, a.heads_q, a.heads_kv, a.seq_q, a.seq_k, a.head_dim = 1, 4, 2, 8, 8, 64
    for f in ("q_stride", "k_stride", "v_stride", "o_stride"):
        getattr(a, f)[:] = [4 * 8 * 64, 8 * 64, 64]
    a.scale = 0.125
    for k_, v_ in kw.items():
        setattr(a, k_, v_)
    return a


@pytest.mark.parametrize(
    "kw,msg",
    [
        (dict(head_dim=84), "head_dim must be a multiple of 8 up to 256"),
        (dict(head_dim=264), "head_dim must be a multiple of 8 up to 256"),
        (dict(dtype=capi.KMI_F32), "dtype must be BF16 or F16"),
        (dict(heads_kv=3), "heads_kv must divide heads_q"),
        (dict(q=0), "null q"),
        (dict(q=0x1008), "16-byte aligned"),
        (dict(seq_k=0), "sizes must be positive"),
        (dict(mask_mode=capi.KMI_MASK_STRIDED), "mask_mode set without a mask"),
        (dict(mask_mode=capi.KMI_MASK_PACKED, mask=0x2000, mask_dtype=capi.KMI_BOOL), "varlen only"),
        (dict(cu_seqlens_q=0x3000), "go together"),
        (dict(k_stride=(ctypes.c_int64 * 3)(4 * 8 * 64, 8 * 64, (1 << 24) + 8)), "row strides"),
        (dict(v_stride=(ctypes.c_int64 * 3)(4 * 8 * 64, 8 * 64, -64)), "row strides"),
        (dict(head_dim_v=72 + 4), "head_dim_v must be 0 or a multiple of 8 up to 256"),
        (dict(head_dim_v=264), "head_dim_v must be 0 or a multiple of 8 up to 256"),
    ],
)
def test_attention_rejects_malformed_calls(kw, msg):
    a = _args(**kw)
    status = capi.lib().kmi_attn_fwd(ctypes.byref(a), None, 0, None)
    assert status == capi.KMI_EINVAL
    assert msg in capi.lib().kmi_last_error().decode()
    with pytest.raises(capi.KmiError, match=msg):
        capi.workspace_bytes(a)


def test_workspace_sizes_follow_the_split_plan():
    # decode-shaped: split-KV partials (fp32 O and lse per split)
    a = _args(batch=8, heads_q=16, heads_kv=2, seq_q=1, seq_k=4096, head_dim=128)
    n = capi.workspace_bytes(a)
    assert n > 0 and n % (16 * 8 * 130 * 4) == 0
    # prefill-shaped: no split
    b = _args(batch=1, heads_q=14, heads_kv=2, seq_q=2048, seq_k=2048)
    assert capi.workspace_bytes(b) == 0


def test_value_head_dim_sizes_the_split_partials():
    # The split partials are as wide as the larger head dim, padded (to 32, 64, 96, 128,
    # 192 or 256; head_dim_v 0 means head_dim): D 128 with Dv 200 keeps partials of 256
    # columns (+ 2 statistics).
    a = _args(batch=8, heads_q=16, heads_kv=2, seq_q=1, seq_k=4096, head_dim=128)
    same = capi.workspace_bytes(a)
    a.head_dim_v = 128
    assert capi.workspace_bytes(a) == same
    a.head_dim_v = 200
    wide = capi.workspace_bytes(a)
    assert wide * 130 == same * 258
    a.head_dim_v = 64
    assert capi.workspace_bytes(a) == same


def test_missing_workspace_is_refused_before_launch():
    a = _args(batch=8, heads_q=16, heads_kv=2, seq_q=1, seq_k=4096, head_dim=128)
    status = capi.lib().kmi_attn_fwd(ctypes.byref(a), None, 0, None)
    assert status == capi.KMI_EWORKSPACE
    assert "workspace" in capi.lib().kmi_last_error().decode()


def test_empty_query_is_a_no_op():
    a = _args(seq_q=0)
    assert capi.lib().kmi_attn_fwd(ctypes.byref(a), None, 0, None) == capi.KMI_OK


def test_norms_reject_malformed_calls():
    lib = capi.lib()
    assert lib.kmi_rms_norm_fwd(0x1000, None, None, 0x2000, None, 4, 64, 9, 0, 0, 1e-6, None) == capi.KMI_EINVAL
    assert "x dtype" in lib.kmi_last_error().decode()
    assert lib.kmi_layer_norm_fwd(None, None, None, None, None, None, 4, 64, capi.KMI_BF16, 0, 0, 1e-5,
                                  None) == capi.KMI_EINVAL
    assert "null x or y" in lib.kmi_last_error().decode()
    assert lib.kmi_layer_norm_fwd(0x1000, 0x3000, None, 0x2000, None, None, 4, 64, capi.KMI_BF16, 7, 0, 1e-5,
                                  None) == capi.KMI_EINVAL
    # zero rows: nothing to do, nothing launched
    assert lib.kmi_rms_norm_fwd(None, None, None, None, None, 0, 64, capi.KMI_BF16, 0, 0, 1e-6, None) == capi.KMI_OK


def test_backward_rejects_malformed_calls_before_launch():
    a = capi.AttnBwdArgs()
    assert capi.lib().kmi_attn_bwd(ctypes.byref(a), None, 0, None) == capi.KMI_EINVAL
    a.q = a.k = a.v = a.out = a.grad_out = a.lse = a.grad_q = a.grad_k = a.grad_v = 0x1000
    a.dtype = capi.KMI_BF16
    a.batch, a.heads_q, a.heads_kv, a.seq_q, a.seq_k, a.head_dim = 1, 4, 3, 8, 8, 64
    assert capi.lib().kmi_attn_bwd(ctypes.byref(a), None, 0, None) == capi.KMI_EINVAL
    assert "heads_kv must divide" in capi.lib().kmi_last_error().decode()
    a.heads_kv = 2
    n = ctypes.c_size_t()
    assert capi.lib().kmi_attn_bwd_workspace_bytes(ctypes.byref(a), ctypes.byref(n)) == capi.KMI_OK
    # fp32 row dot products only: each key tile sees two (query head, row block) items,
    # below the eight a split needs, so dK / dV are written directly (no partials).
    assert n.value == 4 * 8 * 4
    # Longer rows split: 2048 query rows give 7 x 64 items per key tile of C1's GQA,
    # twelve splits of at most 40 (fp32 dK and dV partials per K/V head and split), and
    # 64 key tiles per dQ workgroup two key splits (fp32 dQ partials per head and split).
    a.heads_q, a.heads_kv, a.seq_q, a.seq_k = 14, 2, 2048, 2048
    assert capi.lib().kmi_attn_bwd_workspace_bytes(ctypes.byref(a), ctypes.byref(n)) == capi.KMI_OK
    assert n.value == (14 * 2048 + 2 * (2 * 12 * 2048 * 64) + 14 * 2 * 2048 * 64) * 4
    # Head dim 128: at most 22 items a workgroup: 64 items, three splits,
    # with 8 x 8 x 16 key-tile workgroups (no fill splits) and no dQ key splits.
    a.batch, a.heads_q, a.heads_kv, a.seq_q, a.seq_k, a.head_dim = 8, 16, 8, 1024, 1024, 128
    assert capi.lib().kmi_attn_bwd_workspace_bytes(ctypes.byref(a), ctypes.byref(n)) == capi.KMI_OK
    assert n.value == (16 * 8 * 1024 + 2 * (8 * 3 * 8 * 1024 * 128)) * 4
    a.batch, a.head_dim = 1, 64
    a.heads_q, a.heads_kv, a.seq_q, a.seq_k = 4, 2, 8, 8
    assert capi.lib().kmi_attn_bwd(ctypes.byref(a), None, 0, None) == capi.KMI_EWORKSPACE
    # The staging loads address a 32-row tile with 32-bit byte offsets: row strides stop
    # below 2^25 elements.
    a.k_stride[2] = 1 << 25
    assert capi.lib().kmi_attn_bwd_workspace_bytes(ctypes.byref(a), ctypes.byref(n)) == capi.KMI_EINVAL
    assert "row strides must be below 2^25" in capi.lib().kmi_last_error().decode()
    a.k_stride[2] = (1 << 25) - 8
    assert capi.lib().kmi_attn_bwd_workspace_bytes(ctypes.byref(a), ctypes.byref(n)) == capi.KMI_OK


def test_rms_norm_backward_rejects_malformed_calls_before_launch():
    lib = capi.lib()
    n = ctypes.c_size_t()
    assert lib.kmi_rms_norm_bwd_workspace_bytes(2048, 896, ctypes.byref(n)) == capi.KMI_OK
    # the larger of the one-pass kernel's partial rows (2 x 512 blocks of four rows, then
    # 2 x 8 rows of per-part column sums) and the element path's 16-row chunks (128) of
    # fp32 column sums
    assert n.value == max(2 * 512 + 2 * 8, 128) * 896 * 4
    assert lib.kmi_rms_norm_bwd_workspace_bytes(-1, 896, ctypes.byref(n)) == capi.KMI_EINVAL
    p = 0x1000
    # Unknown dtype, null operands, dweight without weight, missing workspace.
    assert lib.kmi_rms_norm_bwd(p, p, p, p, p, p, 4, 64, 9, capi.KMI_BF16, None, 0, None) == capi.KMI_EINVAL
    assert lib.kmi_rms_norm_bwd(None, p, p, p, p, p, 4, 64, capi.KMI_BF16, capi.KMI_BF16, None, 0, None) == capi.KMI_EINVAL
    assert lib.kmi_rms_norm_bwd(p, p, None, p, p, p, 4, 64, capi.KMI_BF16, 0, None, 0, None) == capi.KMI_EINVAL
    assert "dweight needs weight" in lib.kmi_last_error().decode()
    assert lib.kmi_rms_norm_bwd(p, p, p, p, p, p, 4, 64, capi.KMI_BF16, capi.KMI_BF16, None, 0, None) == capi.KMI_EWORKSPACE
    # No rows: nothing to do.
    assert lib.kmi_rms_norm_bwd(p, p, p, p, p, p, 0, 64, capi.KMI_BF16, capi.KMI_BF16, None, 0, None) == capi.KMI_OK


def test_layer_norm_backward_rejects_malformed_calls_before_launch():
    lib = capi.lib()
    n = ctypes.c_size_t()
    assert lib.kmi_layer_norm_bwd_workspace_bytes(8192, 640, ctypes.byref(n)) == capi.KMI_OK
    # dweight and dbias partial rows of 512 blocks, then of the column sums' 8 parts
    assert n.value == (2 * 512 + 2 * 8) * 640 * 4
    assert lib.kmi_layer_norm_bwd_workspace_bytes(3, 640, ctypes.byref(n)) == capi.KMI_OK
    assert n.value == (2 * 1 + 2 * 8) * 640 * 4
    p = 0x1000
    bf = capi.KMI_BF16
    call = lib.kmi_layer_norm_bwd
    assert call(p, p, p, p, p, p, p, p, 4, 64, 9, bf, bf, None, 0, None) == capi.KMI_EINVAL
    assert call(p, p, None, p, p, p, p, p, 4, 64, bf, bf, bf, None, 0, None) == capi.KMI_EINVAL
    assert call(p, p, p, p, None, p, p, None, 4, 64, bf, bf, bf, None, 0, None) == capi.KMI_EINVAL
    assert "dweight needs weight" in lib.kmi_last_error().decode()
    assert call(p, p, p, p, p, p, p, p, 4, 64, bf, bf, bf, None, 0, None) == capi.KMI_EWORKSPACE
    # rows that are not whole 16-byte vectors, or too wide for the one-pass kernel
    assert call(p, p, p, p, p, p, None, None, 4, 60, bf, bf, bf, None, 0, None) == capi.KMI_EUNSUPPORTED
    assert call(p, p, p, p, p, p, None, None, 4, 4096, bf, bf, bf, None, 0, None) == capi.KMI_EUNSUPPORTED
    assert call(p, p, p, p, p, p, p, p, 0, 64, bf, bf, bf, None, 0, None) == capi.KMI_OK
