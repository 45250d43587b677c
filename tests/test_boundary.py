"""The op surface as the reference's own callers bind it (CPU: schemas, meta tensors,
host planning and tracing; no kernel runs).

* ``ktt::sdpa_refusal`` is called on meta tensors by the reference's compile pass
  (``torch_backend/chains.py:595-606``) with the argument list
  ``(q, k, v, mask, float(dropout), bool(causal), scale)``.
* ``ktt::_varlen_plan`` / ``ktt::_sdpa_varlen`` / ``ktt::_sdpa_varlen_backward`` are called
  by the reference's varlen glue (``torch_backend/varlen.py:31-45,62-104,117-160``) with
  the schemas of ``aten_varlen.cpp:323-341``.
* Traced (fake) CUDA tensors must take torch's composite routes: no kernel may run on them.
"""

import pytest
import torch
import torch.nn.functional as F

import kohakutt_amd  # noqa: F401  (registers torch.ops.ktt)

REFERENCE_SCHEMAS = {
    "sdpa_refusal": "ktt::sdpa_refusal(Tensor q, Tensor k, Tensor v, Tensor? mask, float dropout_p, bool is_causal, "
    "float? scale) -> str",
    "_varlen_plan": "ktt::_varlen_plan(int[] cu_q, int[] cu_k, bool is_causal, float scale, bool key_side) -> "
    "(Tensor, Tensor)",
    "_sdpa_varlen": "ktt::_sdpa_varlen(Tensor q, Tensor k, Tensor v, Tensor plan, Tensor masks, int[] cu_q, "
    "int[] cu_k, bool is_causal, float? scale, bool stats, Tensor? key_mask=None, bool center=False) -> "
    "(Tensor, Tensor)",
    "_sdpa_varlen_backward": "ktt::_sdpa_varlen_backward(Tensor grad, Tensor out, Tensor q, Tensor k, Tensor v, "
    "Tensor plan, Tensor masks, Tensor key_plan, Tensor key_masks, int[] cu_q, int[] cu_k, bool is_causal, "
    "float? scale, Tensor? key_mask=None) -> (Tensor, Tensor, Tensor)",
    "rms_norm": "ktt::rms_norm(Tensor x, Tensor? weight, Tensor? bias, float eps) -> Tensor",
}


@pytest.mark.parametrize("name", sorted(REFERENCE_SCHEMAS))
def test_schemas_are_the_reference_ones(name):
    assert str(getattr(torch.ops.ktt, name).default._schema) == REFERENCE_SCHEMAS[name]


def _meta(*shape, dtype=torch.bfloat16):
    return torch.empty(*shape, dtype=dtype, device="meta")


def test_refusal_answers_on_meta_tensors_with_the_callers_arguments():
    q, k = _meta(1, 14, 32, 64), _meta(1, 2, 32, 64)
    mask = _meta(1, 1, 32, 32, dtype=torch.bool)
    # chains.py's call: meta(q), meta(k), meta(v), meta(mask), float(dropout), bool(causal), scale
    assert torch.ops.ktt.sdpa_refusal(q, k, k, None, float(0.0), bool(True), None) == ""
    assert torch.ops.ktt.sdpa_refusal(q, k, k, mask, 0.0, False, 0.125) == ""
    assert torch.ops.ktt.sdpa_refusal(q, k, k, mask, 0.0, True, None) == "causal takes no mask"
    assert torch.ops.ktt.sdpa_refusal(q, k, k, None, 0.1, False, None) == "dropout"
    assert "head dim" in torch.ops.ktt.sdpa_refusal(_meta(1, 2, 8, 264), _meta(1, 2, 8, 264),
                                                    _meta(1, 2, 8, 264), None, 0.0, False, None)
    assert "divide" in torch.ops.ktt.sdpa_refusal(_meta(1, 3, 8, 64), _meta(1, 2, 8, 64), _meta(1, 2, 8, 64),
                                                  None, 0.0, False, None)
    # head dims up to 256 (the op layer zero-pads those that are not multiples of 8)
    for d in (1, 4, 8, 20, 32, 40, 60, 80, 96, 100, 128, 160, 250, 256):
        t = _meta(1, 2, 8, d)
        assert torch.ops.ktt.sdpa_refusal(t, t, t, None, 0.0, False, None) == "", d
    # CPU tensors are refused (the kernels are GPU only)
    c = torch.zeros(1, 2, 8, 64, dtype=torch.bfloat16)
    assert "GPU" in torch.ops.ktt.sdpa_refusal(c, c, c, None, 0.0, False, None)


def test_varlen_plan_with_the_callers_arguments():
    cu_q, cu_k = (0, 3, 5), (0, 4, 9)
    # varlen.py: _varlen_plan(list(cu_q), list(cu_k), bool(is_causal), float(scale), bool(key_side))
    records, masks = torch.ops.ktt._varlen_plan(list(cu_q), list(cu_k), True, float(0.125), False)
    assert records.dtype == torch.int32 and records.tolist() == [list(cu_q), list(cu_k)]
    assert masks.dtype == torch.int64 and masks.tolist() == [0, 3 * 4, 3 * 4 + 2 * 5]
    key_side = torch.ops.ktt._varlen_plan(list(cu_q), list(cu_k), True, 0.125, True)
    assert torch.equal(key_side[0], records)


@pytest.mark.parametrize(
    "cu_q,cu_k,causal,msg",
    [
        ([0, 3], [0, 3, 5], False, "of equal count"),
        ([1, 3], [0, 3], False, "of equal count"),
        ([0, 3, 2], [0, 3, 5], False, "must not decrease"),
        ([0, 3], [0, 0], False, "queries needs keys"),
        ([0, 4], [0, 3], True, "leaves queries without keys"),
    ],
)
def test_varlen_plan_rejects_bad_offsets_with_the_reference_messages(cu_q, cu_k, causal, msg):
    with pytest.raises(ValueError, match=msg):
        torch.ops.ktt._varlen_plan(cu_q, cu_k, causal, 0.125, False)


def test_varlen_plan_needs_a_positive_scale():
    with pytest.raises(NotImplementedError, match="scale must be positive"):
        torch.ops.ktt._varlen_plan([0, 2], [0, 2], False, 0.0, False)


def test_sdpa_varlen_binds_the_callers_positional_arguments():
    """varlen.py:86-101 calls _sdpa_varlen(query, key, value, records, masks, list(cu_q),
    list(cu_k), causal, scale, True, None, center): the arguments bind (the call then
    reaches the dispatcher, which has no CPU kernel)."""
    q = torch.zeros(5, 4, 64, dtype=torch.bfloat16)
    k = torch.zeros(9, 2, 64, dtype=torch.bfloat16)
    records, masks = torch.ops.ktt._varlen_plan([0, 3, 5], [0, 4, 9], True, 0.125, False)
    with pytest.raises(NotImplementedError, match="CPU"):
        torch.ops.ktt._sdpa_varlen(q, k, k, records, masks, [0, 3, 5], [0, 4, 9], True, 0.125, True, None, False)
    with pytest.raises(NotImplementedError, match="CPU"):
        torch.ops.ktt._sdpa_varlen_backward(q, q, q, k, k, records, masks, records, masks, [0, 3, 5], [0, 4, 9],
                                            True, 0.125)


def test_traced_cuda_tensors_take_the_composite_routes():
    """Under FakeTensorMode with fake CUDA tensors, SDPA with a bool mask and rms_norm
    (the ops taken on AutogradCUDA) trace through torch's composites: no kernel is
    launched on data that does not exist."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    kohakutt_amd.reset_counters()
    with FakeTensorMode(allow_non_fake_inputs=False) as mode:
        q = mode.from_tensor(torch.empty(1, 4, 16, 64, dtype=torch.bfloat16), static_shapes=True)
        q = torch.empty(1, 4, 16, 64, dtype=torch.bfloat16, device="cuda")
        m = torch.ones(1, 1, 1, 16, dtype=torch.bool, device="cuda")
        out = F.scaled_dot_product_attention(q, q, q, attn_mask=m)
        x = torch.empty(8, 64, dtype=torch.bfloat16, device="cuda")
        w = torch.empty(64, dtype=torch.bfloat16, device="cuda")
        y = F.rms_norm(x, [64], w, 1e-6)
    assert out.shape == (1, 4, 16, 64) and y.shape == (8, 64)
    c = kohakutt_amd.counters()
    assert c["attention"] == 0 and c["norms"] == 0
