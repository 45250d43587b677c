"""Python side of the attention op surface.

* ``sdpa(q, k, v, key_lengths=...)`` -- the reference's ``kohakutt.sdpa``
  (``src/kohakutt/attention.py:10-23``): SDPA whose batch entry b sees keys
  ``[0, key_lengths[b])``.  The counts reach the kernels as an int32 tensor
  (``ktt::_sdpa_lengths``); nothing of size [B, Sk] is built for calls the kernels take.
* ``sdpa_varlen(q, k, v, cu_seq_q, ...)`` -- the reference's ``kohakutt.sdpa_varlen``
  (``src/kohakutt/attention.py:26-76``) over ``ktt::_sdpa_varlen_offsets``.
* Gradients: the backward formulas are registered on the ops themselves
  (``torch.library.register_autograd``), so ``torch.ops.ktt._sdpa_lengths``,
  ``ktt::_sdpa_varlen`` and ``ktt::_sdpa_varlen_offsets`` are differentiable wherever they
  are called from; each backward is one set of kernel launches
  (``ktt::_sdpa_lengths_backward``, ``ktt::_sdpa_varlen_backward``,
  ``ktt::_sdpa_varlen_offsets_backward``).
* The GPU kernels of torch's ``torch_attn::_varlen_attn`` and its backward
  (``torch.nn.attention.varlen.varlen_attn``), which the reference registers for its device
  (``src/kohakutt/torch_backend/varlen.py:247-252``).

Host offsets are validated with the reference's rules and messages (``check_offsets``,
``ktt_flash/varlen_plan.hpp:43-82``); offsets already on the GPU are trusted (the kernels
clamp them into the packed token ranges) and never downloaded.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

# ---------------------------------------------------------------- key lengths


def _as_counts(key_lengths, batch: int, keys: int, device) -> torch.Tensor:
    """``key_lengths`` as the int32 [batch] tensor the kernels read, on ``device``.

    Host values (a list, tuple or CPU tensor) must lie in [1, keys], as the reference
    requires (``torch_backend/lengths.py:10-29``).  A GPU tensor is used as it is: reading
    it back would synchronise, and the kernels clamp every count to [1, keys] anyway."""
    on_gpu = isinstance(key_lengths, torch.Tensor) and key_lengths.device.type != "cpu"
    counts = torch.as_tensor(key_lengths).to(dtype=torch.int32)
    if counts.dim() != 1 or counts.numel() != batch:
        raise ValueError(
            f"kohakutt_amd.sdpa: key_lengths must hold one length per batch ({batch}), "
            f"got shape {tuple(counts.shape)}"
        )
    if not on_gpu and counts.numel():
        lo, hi = int(counts.min()), int(counts.max())
        if lo < 1 or hi > keys:
            raise ValueError(
                f"kohakutt_amd.sdpa: key_lengths must lie in [1, {keys}], got {counts.tolist()}"
            )
    return counts.to(device).contiguous()


def _grads_wanted(*tensors) -> bool:
    return torch.is_grad_enabled() and any(t.requires_grad for t in tensors)


def _kernels_take_lengths(q, k, v, is_causal) -> bool:
    """Whether ``ktt::_sdpa_lengths`` takes the call (the reference's
    ``lengths.kernel_takes``, ``torch_backend/lengths.py:36-50``)."""
    if not all(t.is_cuda and t.dim() == 4 for t in (q, k, v)):
        return False
    return bool(
        torch.ops.ktt._sdpa_lengths_supported(q, k, v, bool(is_causal), _grads_wanted(q, k, v))
    )


def _padding_mask(counts: torch.Tensor, sq: int, sk: int, causal: bool) -> torch.Tensor:
    """The bool keep-mask [B, 1, Sq, Sk] equivalent to key counts (with the dense
    top-left causal rule folded in), for calls the kernels do not take."""
    key_idx = torch.arange(sk, device=counts.device, dtype=torch.int32)
    keep = key_idx.view(1, 1, 1, sk) < counts.view(-1, 1, 1, 1)
    if causal:
        keep = keep & torch.ones(sq, sk, dtype=torch.bool, device=counts.device).tril()
    return keep


def sdpa(q, k, v, key_lengths=None, is_causal=False, scale=None):
    """``F.scaled_dot_product_attention`` of q [B, H, Sq, D], k / v [B, Hk, Sk, D] where
    batch entry b sees keys [0, key_lengths[b]) (B ints in [1, Sk]: a list, or a CPU or GPU
    tensor).  Rows past a length still see the first ``key_lengths[b]`` keys.  GQA is
    taken when Hk divides H.  Differentiable in q, k and v."""
    enable_gqa = q.size(1) != k.size(1)
    if key_lengths is None:
        return F.scaled_dot_product_attention(
            q, k, v, is_causal=is_causal, scale=scale, enable_gqa=enable_gqa
        )
    counts = _as_counts(key_lengths, q.size(0), k.size(-2), q.device)
    if _kernels_take_lengths(q, k, v, is_causal):
        stats = _grads_wanted(q, k, v)
        return torch.ops.ktt._sdpa_lengths(q, k, v, counts, bool(is_causal), scale, stats)
    keep = _padding_mask(counts, q.size(-2), k.size(-2), bool(is_causal))
    return F.scaled_dot_product_attention(
        q, k, v, attn_mask=keep, scale=scale, enable_gqa=enable_gqa
    )


def _lengths_setup(ctx, inputs, output):
    q, k, v, counts, is_causal, scale, _stats = inputs
    ctx.save_for_backward(q, k, v, counts, output)
    ctx.causal, ctx.scale = is_causal, scale


def _lengths_backward(ctx, grad):
    q, k, v, counts, out = ctx.saved_tensors
    dq, dk, dv = torch.ops.ktt._sdpa_lengths_backward(
        grad.contiguous(), out, q, k, v, counts, ctx.causal, ctx.scale
    )
    return dq, dk, dv, None, None, None, None


# ---------------------------------------------------------------- varlen


def host_offsets(cu_seq):
    """Cumulative offsets as a tuple of host ints (a list, or a CPU or GPU int tensor; a
    GPU tensor is read back)."""
    if isinstance(cu_seq, torch.Tensor):
        return tuple(int(x) for x in cu_seq.detach().to("cpu").tolist())
    return tuple(int(x) for x in cu_seq)


def check_offsets(cu_q, cu_k, causal, total_q=None, total_k=None):
    """Validates host offsets with the reference's rules and messages
    (``ktt_flash/varlen_plan.hpp:43-82``); returns the per-sequence (Lq, Lk)."""
    if len(cu_q) < 2 or len(cu_q) != len(cu_k) or cu_q[0] != 0 or cu_k[0] != 0:
        raise ValueError(
            "kohakutt_amd: sdpa_varlen needs cumulative offsets [0, ..., total] of equal "
            "count for queries and keys"
        )
    pairs = [(b - a, d - c) for a, b, c, d in zip(cu_q, cu_q[1:], cu_k, cu_k[1:])]
    for lq, lk in pairs:
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
    if total_q is not None and cu_q[-1] != total_q:
        raise ValueError(f"kohakutt_amd: cu_seq_q must end at the {total_q} packed queries")
    if total_k is not None and cu_k[-1] != total_k:
        raise ValueError(f"kohakutt_amd: cu_seq_k must end at the {total_k} packed keys")
    return pairs


def _on_host(cu) -> bool:
    return not (isinstance(cu, torch.Tensor) and cu.is_cuda)


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

    q [Tq, H, D], k [Tk, Hkv, D], v [Tk, Hkv, Dv] (bf16 / fp16; fp32 is cast to bf16;
    Dv may differ from D, as in the reference's packed op) hold every sequence's tokens
    back to back.  ``cu_seq_q`` / ``cu_seq_k`` are the
    cumulative offsets [0, ..., total] (a list or an int tensor, host or GPU;
    ``cu_seq_k`` defaults to ``cu_seq_q``).  Each query attends to the keys of its own
    sequence; with ``is_causal``, query r of a sequence sees its first
    min(Lk, r + 1 + Lk - Lq) keys.  Returns [Tq, H, Dv]; differentiable in q, k and v.

    ``attn_mask``: a key mask [Tk] (bool: True keeps the key; float: added to its logits,
    clamped at -5e5), as the reference takes it.  ``packed_mask``: this build's per-row
    mask -- every sequence's row-major [Lq_i, Lk_i] block concatenated (bool or additive,
    shared by the heads), usable together with ``is_causal``.

    ``max_q`` / ``max_k`` (the longest sequence): derived from host offsets when not given
    (and checked when given); with GPU offsets they are read back unless given."""
    cu_k_in = cu_seq_q if cu_seq_k is None else cu_seq_k
    if attn_mask is not None and packed_mask is not None:
        raise ValueError("kohakutt_amd: sdpa_varlen takes attn_mask or packed_mask, not both")
    if attn_mask is not None and (attn_mask.dim() != 1 or attn_mask.size(0) != k.size(0)):
        raise ValueError(
            f"kohakutt_amd.sdpa_varlen: attn_mask must be [{k.size(0)}] (one value per "
            f"packed key), got {tuple(attn_mask.shape)}"
        )
    if _on_host(cu_seq_q) and _on_host(cu_k_in):
        cu_q, cu_k = host_offsets(cu_seq_q), host_offsets(cu_k_in)
        pairs = check_offsets(cu_q, cu_k, is_causal, q.size(0), k.size(0))
        longest_q = max((a for a, _ in pairs), default=0)
        longest_k = max((b for _, b in pairs), default=0)
        if (max_q is not None and max_q < longest_q) or (max_k is not None and max_k < longest_k):
            raise ValueError(
                f"kohakutt_amd.sdpa_varlen: max_q / max_k ({max_q}, {max_k}) are below the "
                f"longest sequence ({longest_q}, {longest_k})"
            )
        max_q = longest_q if max_q is None else max_q
        max_k = longest_k if max_k is None else max_k
        cu_q_t = torch.tensor(cu_q, dtype=torch.int32)
        cu_k_t = torch.tensor(cu_k, dtype=torch.int32)
    else:
        cu_q_t = torch.as_tensor(cu_seq_q, device=q.device).to(torch.int32)
        cu_k_t = torch.as_tensor(cu_k_in, device=q.device).to(torch.int32)
        if max_q is None:
            max_q = int((cu_q_t[1:] - cu_q_t[:-1]).max())
        if max_k is None:
            max_k = int((cu_k_t[1:] - cu_k_t[:-1]).max())
    out, _ = torch.ops.ktt._sdpa_varlen_offsets(
        q, k, v, cu_q_t, cu_k_t, int(max_q), int(max_k), bool(is_causal),
        None if scale is None else float(scale), attn_mask, packed_mask,
    )
    return out


def _offsets_setup(ctx, inputs, output):
    q, k, v, cu_q, cu_k, max_q, max_k, causal, scale, key_mask, packed_mask = inputs
    out, lse = output
    ctx.save_for_backward(q, k, v, out, lse, cu_q, cu_k, key_mask, packed_mask)
    ctx.args = (max_q, max_k, causal, scale)


def _narrowed_backward(grad, q, k, v, out, *rest):
    """The varlen backward kernels on (grad, q, k, v, out).  fp32 operands -- the forward
    casts them to bf16 and returns fp32 -- run on bf16 copies, and the gradients come
    back in fp32."""
    wide = q.dtype == torch.float32
    if wide:
        grad, q, k, v, out = (t.to(torch.bfloat16) for t in (grad, q, k, v, out))
    grads = torch.ops.ktt._sdpa_varlen_offsets_backward(grad.contiguous(), q, k, v, out, *rest)
    return tuple(g.float() for g in grads) if wide else tuple(grads)


def _offsets_backward(ctx, grad, _grad_lse):
    q, k, v, out, lse, cu_q, cu_k, key_mask, packed_mask = ctx.saved_tensors
    max_q, max_k, causal, scale = ctx.args
    dq, dk, dv = _narrowed_backward(
        grad, q, k, v, out, lse, cu_q, cu_k, max_q, max_k, causal, scale, key_mask, packed_mask,
    )
    return dq, dk, dv, None, None, None, None, None, None, None, None


def _reference_setup(ctx, inputs, output):
    q, k, v, plan, masks, cu_q, cu_k, causal, scale, _stats, key_mask, _center = inputs
    out, _ = output
    ctx.save_for_backward(q, k, v, out, plan, masks, key_mask)
    ctx.args = (list(cu_q), list(cu_k), causal, scale)


def _reference_backward(ctx, grad, _grad_lse):
    q, k, v, out, plan, masks, key_mask = ctx.saved_tensors
    cu_q, cu_k, causal, scale = ctx.args
    dq, dk, dv = torch.ops.ktt._sdpa_varlen_backward(
        grad.contiguous(), out, q, k, v, plan, masks, plan, masks, cu_q, cu_k, causal, scale,
        key_mask,
    )
    return (dq, dk, dv) + (None,) * 9


# ---------------------------------------------------------------- torch_attn kernels


def _varlen_attn_gpu(query, key, value, cu_seq_q, cu_seq_k, max_q, max_k, is_causal=False):
    """torch_attn::_varlen_attn on GPU tensors: (output [Tq, H, D], log-sum-exp [H, Tq],
    rng state), as the reference's ``varlen._forward`` returns them
    (``torch_backend/varlen.py:62-104``)."""
    out, lse = torch.ops.ktt._sdpa_varlen_offsets(
        query, key, value, cu_seq_q, cu_seq_k, int(max_q), int(max_k), bool(is_causal),
        None, None, None,
    )
    return out, lse, torch.zeros((2,), dtype=torch.uint64, device=query.device)


def _varlen_attn_backward_gpu(grad_out, query, key, value, out, lse, cu_seq_q, cu_seq_k,
                              max_q, max_k, is_causal, rng_state):
    """torch_attn::_varlen_attn_backward on GPU tensors: (dq, dk, dv) from the forward's
    output and lse (``torch_backend/varlen.py:117-160``)."""
    return _narrowed_backward(
        grad_out, query, key, value, out, lse, cu_seq_q, cu_seq_k,
        int(max_q), int(max_k), bool(is_causal), None, None, None,
    )


def install() -> None:
    """Registers the autograd formulas of the ktt attention ops and, when this torch has
    ``torch.nn.attention.varlen``, the GPU kernels of ``torch_attn::_varlen_attn`` and its
    backward."""
    torch.library.register_autograd(
        "ktt::_sdpa_lengths", _lengths_backward, setup_context=_lengths_setup
    )
    torch.library.register_autograd(
        "ktt::_sdpa_varlen_offsets", _offsets_backward, setup_context=_offsets_setup
    )
    torch.library.register_autograd(
        "ktt::_sdpa_varlen", _reference_backward, setup_context=_reference_setup
    )
    try:
        from torch.nn.attention import varlen as _tv  # noqa: F401
    except ImportError:
        return
    if getattr(torch.ops.torch_attn, "_varlen_attn", None) is None:
        return
    torch.library.register_kernel("torch_attn::_varlen_attn", "cuda", _varlen_attn_gpu)
    if getattr(torch.ops.torch_attn, "_varlen_attn_backward", None) is not None:
        torch.library.register_kernel(
            "torch_attn::_varlen_attn_backward", "cuda", _varlen_attn_backward_gpu
        )
