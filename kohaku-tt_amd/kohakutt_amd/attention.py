"""Attention entry points beyond torch's own (the reference's ``kohakutt.sdpa`` and
``kohakutt.sdpa_varlen``, ``src/kohakutt/attention.py:10-76``), and the GPU kernel of
``torch_attn::_varlen_attn`` (``torch.nn.attention.varlen.varlen_attn``), which the
reference registers for its device in ``src/kohakutt/torch_backend/varlen.py:62-104,
247-252``."""

from __future__ import annotations

import torch
import torch.nn.functional as F

_MASKED_LOGIT = -5e5


def sdpa(q, k, v, key_lengths=None, is_causal=False, scale=None):
    """``F.scaled_dot_product_attention`` of q [B, H, Sq, D], k / v [B, Hk, Sk, D] with
    the key mask ``key < key_lengths[b]`` (B ints in [1, Sk]: a list, CPU or GPU tensor),
    as the reference's ``kohakutt.sdpa`` (``attention.py:10-23``).  On the kernels
    (``ktt::_sdpa_lengths``) the lengths go to the kernel as a per-batch key count: no
    mask is built, key tiles past a length are not read.  Calls the kernels do not take
    run SDPA with a bool mask built on the device (``lengths.py:79-89``)."""
    gqa = q.size(1) != k.size(1)
    if key_lengths is None:
        return F.scaled_dot_product_attention(
            q, k, v, is_causal=is_causal, scale=scale, enable_gqa=gqa
        )
    lengths = device_lengths(key_lengths, q.size(0), k.size(-2), q.device)
    if kernel_takes(q, k, v, is_causal):
        return _lengths_kernel(q, k, v, lengths, is_causal, scale)
    return _lengths_masked(q, k, v, lengths, is_causal, scale)


def device_lengths(key_lengths, batch, keys, device):
    """``key_lengths`` as an int32 [batch] tensor on ``device`` (``lengths.py:10-29``): a
    list or a CPU tensor is checked to lie in [1, keys]; a GPU tensor is taken as it is
    (the kernels clamp it to [1, keys], so it is never downloaded)."""
    if isinstance(key_lengths, torch.Tensor) and key_lengths.device.type != "cpu":
        lengths = key_lengths.to(device=device, dtype=torch.int32)
    else:
        lengths = torch.as_tensor(key_lengths, dtype=torch.int32)
        if lengths.numel() and (int(lengths.min()) < 1 or int(lengths.max()) > keys):
            raise ValueError(
                f"kohakutt_amd.sdpa: key_lengths must lie in [1, {keys}], got {lengths.tolist()}"
            )
        lengths = lengths.to(device)
    if lengths.dim() != 1 or lengths.size(0) != batch:
        raise ValueError(
            f"kohakutt_amd.sdpa: key_lengths must hold one length per batch ({batch}), "
            f"got shape {tuple(lengths.shape)}"
        )
    return lengths.contiguous()


def kernel_takes(q, k, v, is_causal):
    """True when ``ktt::_sdpa_lengths`` takes q, k, v (``lengths.py:36-50``): GPU tensors
    the attention kernels cover; with gradients, causal needs Sq == Sk."""
    tensors = (q, k, v)
    grads = torch.is_grad_enabled() and any(t.requires_grad for t in tensors)
    return all(t.is_cuda and t.dim() == 4 for t in tensors) and bool(
        torch.ops.ktt._sdpa_lengths_supported(q, k, v, bool(is_causal), grads)
    )


class _Lengths(torch.autograd.Function):
    """The kernel route with autograd (``lengths.py:53-69``): dq, dk, dv from
    ``ktt::_sdpa_lengths_backward``; the lengths get no gradient."""

    @staticmethod
    def forward(ctx, q, k, v, lengths, causal, scale):
        out = torch.ops.ktt._sdpa_lengths(q, k, v, lengths, causal, scale, True)
        ctx.save_for_backward(q, k, v, lengths, out)
        ctx.args = (causal, scale)
        return out

    @staticmethod
    def backward(ctx, grad):
        q, k, v, lengths, out = ctx.saved_tensors
        causal, scale = ctx.args
        dq, dk, dv = torch.ops.ktt._sdpa_lengths_backward(
            grad.contiguous(), out, q, k, v, lengths, causal, scale
        )
        return dq, dk, dv, None, None, None


def _lengths_kernel(q, k, v, lengths, is_causal, scale):
    if torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v)):
        return _Lengths.apply(q, k, v, lengths, bool(is_causal), scale)
    return torch.ops.ktt._sdpa_lengths(q, k, v, lengths, bool(is_causal), scale, False)


def _lengths_masked(q, k, v, lengths, is_causal, scale):
    """The explicit-mask route: a bool [B, 1, Sq, Sk] mask built on the device."""
    b, sq, sk = q.size(0), q.size(2), k.size(2)
    keys = torch.arange(sk, device=q.device, dtype=torch.int32)
    keep = (keys[None, :] < lengths.reshape(b, 1))[:, None, None, :]
    if is_causal:
        rows = torch.arange(sq, device=q.device, dtype=torch.int32)
        keep = keep & (keys[None, :] <= rows[:, None])[None, None]
    return F.scaled_dot_product_attention(
        q, k, v, attn_mask=keep, scale=scale, enable_gqa=q.size(1) != k.size(1)
    )


def offsets(cu_seq):
    """Cumulative offsets as a tuple of host ints (a list, or a CPU or GPU int tensor; a
    GPU tensor is downloaded)."""
    if isinstance(cu_seq, torch.Tensor):
        return tuple(int(x) for x in cu_seq.detach().cpu().tolist())
    return tuple(int(x) for x in cu_seq)


def check_offsets(cu_q, cu_k, causal, total_q=None, total_k=None):
    """Validates host offsets with the reference's rules and messages
    (``ktt_flash/varlen_plan.hpp:43-82``); returns the per-sequence (Lq, Lk)."""
    if len(cu_q) < 2 or len(cu_q) != len(cu_k) or cu_q[0] != 0 or cu_k[0] != 0:
        raise ValueError(
            "kohakutt_amd: sdpa_varlen needs cumulative offsets [0, ..., total] of equal "
            "count for queries and keys"
        )
    lengths = []
    for b in range(len(cu_q) - 1):
        lq, lk = cu_q[b + 1] - cu_q[b], cu_k[b + 1] - cu_k[b]
        if lq < 0 or lk < 0 or (lq > 0 and lk == 0):
            raise ValueError(
                "kohakutt_amd: sdpa_varlen offsets must not decrease, and a sequence with "
                "queries needs keys"
            )
        if causal and lq > lk:
            raise ValueError(
                "kohakutt_amd: causal sdpa_varlen with more queries than keys in a "
                "sequence leaves queries without keys"
            )
        lengths.append((lq, lk))
    if total_q is not None and cu_q[-1] != total_q:
        raise ValueError(f"kohakutt_amd: cu_seq_q must end at the {total_q} packed queries")
    if total_k is not None and cu_k[-1] != total_k:
        raise ValueError(f"kohakutt_amd: cu_seq_k must end at the {total_k} packed keys")
    return lengths


def _host(cu):
    return not isinstance(cu, torch.Tensor) or not cu.is_cuda


def sdpa_varlen(
    q,
    k,
    v,
    cu_seq_q,
    cu_seq_k=None,
    max_q=None,
    max_k=None,
    is_causal=False,
    scale=None,
    attn_mask=None,
    packed_mask=None,
):
    """Scaled dot-product attention over packed variable-length sequences (the
    reference's ``kohakutt.sdpa_varlen``, ``attention.py:26-76``).

    q [Tq, H, D], k [Tk, Hkv, D], v [Tk, Hkv, D] (bf16 / fp16; fp32 is cast to bf16)
    hold every sequence's tokens back to back.  ``cu_seq_q`` / ``cu_seq_k`` are the
    cumulative offsets [0, ..., total] (a list or an int tensor; ``cu_seq_k`` defaults to
    ``cu_seq_q``).  Each query attends to the keys of its own sequence; with
    ``is_causal``, query r of a sequence sees its first min(Lk, r + 1 + Lk - Lq) keys.
    Returns [Tq, H, D].

    ``attn_mask``: a key mask [Tk] (bool: True keeps the key; float: added to its
    logits, clamped at -5e5), as the reference takes it.
    ``packed_mask``: this build's per-row mask -- every sequence's row-major
    [Lq_i, Lk_i] block concatenated (bool or additive, shared by the heads), usable
    together with ``is_causal``.

    Host offsets (lists, CPU tensors) are validated with the reference's errors; GPU
    offsets are trusted (the kernels clamp them into the packed token ranges)."""
    cu_k_in = cu_seq_q if cu_seq_k is None else cu_seq_k
    if _host(cu_seq_q) and _host(cu_k_in):
        cu_q, cu_k = offsets(cu_seq_q), offsets(cu_k_in)
        lengths = check_offsets(cu_q, cu_k, is_causal, q.size(0), k.size(0))
        if max_q is None:
            max_q = max((a for a, _ in lengths), default=0)
        if max_k is None:
            max_k = max((b for _, b in lengths), default=0)
        if packed_mask is not None and packed_mask.numel() != sum(a * b for a, b in lengths):
            raise ValueError(
                "kohakutt_amd.sdpa_varlen: packed_mask must hold sum(Lq_i * Lk_i) = "
                f"{sum(a * b for a, b in lengths)} values, got {packed_mask.numel()}"
            )
        cu_q_t = torch.tensor(cu_q, dtype=torch.int32, device=q.device)
        cu_k_t = torch.tensor(cu_k, dtype=torch.int32, device=q.device)
    else:
        cu_q_t = torch.as_tensor(cu_seq_q, device=q.device).to(torch.int32)
        cu_k_t = torch.as_tensor(cu_k_in, device=q.device).to(torch.int32)
        if max_q is None:
            max_q = int((cu_q_t[1:] - cu_q_t[:-1]).max().item())
        if max_k is None:
            max_k = int((cu_k_t[1:] - cu_k_t[:-1]).max().item())
    if attn_mask is not None and packed_mask is not None:
        raise ValueError("kohakutt_amd: sdpa_varlen takes attn_mask or packed_mask, not both")
    if attn_mask is not None and (attn_mask.dim() != 1 or attn_mask.size(0) != k.size(0)):
        raise ValueError(
            f"kohakutt_amd.sdpa_varlen: attn_mask must be [{k.size(0)}] (one value per "
            f"packed key), got {tuple(attn_mask.shape)}"
        )
    args = (cu_q_t, cu_k_t, int(max_q), int(max_k), bool(is_causal), None if scale is None else float(scale),
            attn_mask, packed_mask)
    if torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v)):
        return _Varlen.apply(q, k, v, *args)
    out, _ = torch.ops.ktt._sdpa_varlen(q, k, v, *args)
    return out


class _Varlen(torch.autograd.Function):
    """Packed attention with autograd (the reference's ``_sdpa_varlen_backward``,
    ``aten_varlen.cpp:240-300``, behind ``varlen.py:62-104``).  The backward goes sequence
    by sequence: an unmasked sequence whose causal rule is the dense one (non-causal, or
    Lq == Lk, where bottom-right and top-left agree) runs the flash backward kernels
    (``ktt::_sdpa_flash_backward``) on [1, H, L, D] head views of the packed tensors and
    the forward's lse; any other sequence recomputes in float64 with the forward's mask
    rules (masked keys at -5e5, so a fully-masked row is the softmax over its raw scores)."""

    @staticmethod
    def forward(ctx, q, k, v, cu_q_t, cu_k_t, max_q, max_k, causal, scale, attn_mask, packed_mask):
        out, lse = torch.ops.ktt._sdpa_varlen(q, k, v, cu_q_t, cu_k_t, max_q, max_k, causal, scale, attn_mask,
                                              packed_mask)
        ctx.save_for_backward(q, k, v, out, lse, cu_q_t, cu_k_t, attn_mask, packed_mask)
        ctx.args = (causal, scale)
        return out

    @staticmethod
    def backward(ctx, grad):
        q, k, v, out, lse, cu_q_t, cu_k_t, attn_mask, packed_mask = ctx.saved_tensors
        causal, scale = ctx.args
        cu_q, cu_k = offsets(cu_q_t), offsets(cu_k_t)
        grad = grad.contiguous()
        dq, dk, dv = torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v)
        heads = lambda t, a, b: t[a:b].transpose(0, 1).unsqueeze(0)  # [1, H, L, D] view
        kernels = q.dtype in (torch.bfloat16, torch.float16) and q.size(-1) in (64, 128)
        off = 0  # packed-mask offset of this sequence's block
        for i in range(len(cu_q) - 1):
            a, b, c, d = cu_q[i], cu_q[i + 1], cu_k[i], cu_k[i + 1]
            lq, lk = b - a, d - c
            block = None
            if packed_mask is not None:
                block = packed_mask.reshape(-1)[off:off + lq * lk].view(lq, lk)
            off += lq * lk
            if lq == 0 or lk == 0:
                continue
            if kernels and attn_mask is None and block is None and (not causal or lq == lk):
                gq, gk, gv = torch.ops.ktt._sdpa_flash_backward(
                    heads(grad, a, b), heads(q, a, b), heads(k, c, d), heads(v, c, d), heads(out, a, b),
                    lse[:, a:b].unsqueeze(0), bool(causal), scale)
            else:
                key = None if attn_mask is None else attn_mask[c:d]
                gq, gk, gv = _varlen_recompute_grads(heads(q, a, b), heads(k, c, d), heads(v, c, d),
                                                     heads(grad, a, b), causal, scale, key, block)
            dq[a:b] = gq[0].transpose(0, 1).to(dq.dtype)
            dk[c:d] = gk[0].transpose(0, 1).to(dk.dtype)
            dv[c:d] = gv[0].transpose(0, 1).to(dv.dtype)
        return dq, dk, dv, None, None, None, None, None, None, None, None


def _varlen_recompute_grads(q, k, v, grad, causal, scale, key_mask, block):
    """Gradients of one sequence in float64 with the forward's rules: bottom-right causal
    (invisible keys excluded), masked keys at the -5e5 logit (bool False, or additive
    values clamped there)."""
    with torch.enable_grad():  # a Function's backward runs with grad mode off
        return _recompute(q, k, v, grad, causal, scale, key_mask, block)


def _recompute(q, k, v, grad, causal, scale, key_mask, block):
    q64, k64, v64 = (t.detach().double().requires_grad_() for t in (q, k, v))
    hq, hk, lq, lk = q.size(1), k.size(1), q.size(2), k.size(2)
    kk, vv = k64.repeat_interleave(hq // hk, 1), v64.repeat_interleave(hq // hk, 1)
    s = (scale if scale is not None else q.size(-1) ** -0.5) * (q64 @ kk.transpose(-2, -1))
    add = torch.zeros(lq, lk, dtype=torch.float64, device=q.device)
    for m in (None if key_mask is None else key_mask.reshape(1, lk), block):
        if m is None:
            continue
        m = m.to(q.device)
        if m.dtype == torch.bool:
            add = add + torch.where(m, 0.0, _MASKED_LOGIT).to(torch.float64)
        else:
            add = add + m.to(torch.float64)
    s = s + add.clamp_min(_MASKED_LOGIT)
    if causal:
        rows = torch.arange(lq, device=q.device)[:, None]
        keys = torch.arange(lk, device=q.device)[None, :]
        s = s.masked_fill(keys > rows + (lk - lq), float("-inf"))
    out = torch.softmax(s, -1) @ vv
    return torch.autograd.grad(out, (q64, k64, v64), grad.double())


def _varlen_attn_gpu(query, key, value, cu_seq_q, cu_seq_k, max_q, max_k, is_causal=False):
    """torch_attn::_varlen_attn on GPU tensors: (output [Tq, H, D], log-sum-exp [H, Tq],
    rng state), as the reference's ``varlen._forward`` (``varlen.py:62-104``)."""
    out, lse = torch.ops.ktt._sdpa_varlen(
        query,
        key,
        value,
        cu_seq_q,
        cu_seq_k,
        int(max_q),
        int(max_k),
        bool(is_causal),
        None,
        None,
        None,
    )
    return out, lse, torch.zeros((2,), dtype=torch.uint64, device=query.device)


def install_varlen_kernel() -> bool:
    """Registers the GPU kernel of ``torch_attn::_varlen_attn`` when this torch has the
    op (``torch.nn.attention.varlen``); returns whether it did."""
    try:
        from torch.nn.attention import varlen as _tv  # noqa: F401
    except ImportError:
        return False
    op = getattr(torch.ops.torch_attn, "_varlen_attn", None)
    if op is None:
        return False
    torch.library.register_kernel("torch_attn::_varlen_attn", "cuda", _varlen_attn_gpu)
    return True
