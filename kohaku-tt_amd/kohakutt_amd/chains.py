"""torch.compile graph pass: RMSNorm written out in torch ops becomes one ``ktt::rms_norm``.

The reference's compile backends rewrite such chains before lowering
(``src/kohakutt/torch_backend/chains.py:1-4,278-338``); this module does the same for
graphs compiled for the MI355X kernels, so a model that spells RMSNorm as

    h = x.to(torch.float32)
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    y = weight * h.to(x.dtype)

(Hugging Face's Llama / Qwen2 norms) runs the fused norm kernel instead of five
elementwise and reduction kernels.  What is matched: ``t * rsqrt(mean(t*t or t**2, last
dim, keepdim) + eps)``, ``t`` optionally a cast of the source, followed by casts and at
most one multiplication by a ``[width]`` floating weight.  What is refused (the graph is
left as it was): intermediate values with other users, chains whose result needs a
gradient (``ktt::rms_norm`` has no derivative), a result shaped unlike the input, a
result dtype that neither the source nor its cast has, and graphs that write the source
or the weight in place between the chain's first node and its end.

``KTT_FUSE_CHAINS`` (read at each compile) selects rewrites as in the reference: unset,
``1``, ``on`` or ``true`` the default set, ``0``, ``off`` or ``false`` none, ``all``, or a
comma list of ``norm``, ``rotary``, ``mask``, ``gqa``; another name raises ValueError.
Only ``norm`` is a rewrite here: RoPE fusion and the reference's mask / GQA conversions
serve its own device and are outside this build's hot path.
"""

from __future__ import annotations

import operator
import os

import torch
import torch.fx

__all__ = ["REWRITES", "selected", "rewrite_rms_norms", "backend"]

REWRITES = ("norm", "rotary", "mask", "gqa")

_A = torch.ops.aten
_P = torch.ops.prims
# What a node computes, keyed by call_function target or call_method name.
_BY_TARGET = {
    operator.mul: "mul", torch.mul: "mul", _A.mul.Tensor: "mul",
    operator.add: "add", torch.add: "add", _A.add.Tensor: "add", _A.add.Scalar: "add",
    torch.rsqrt: "rsqrt", _A.rsqrt.default: "rsqrt",
    operator.pow: "pow", torch.pow: "pow", _A.pow.Tensor_Scalar: "pow",
    torch.mean: "mean", _A.mean.dim: "mean",
    _A._to_copy.default: "cast", _P.convert_element_type.default: "cast",
}
_BY_METHOD = {
    "mul": "mul", "add": "add", "rsqrt": "rsqrt", "pow": "pow", "mean": "mean",
    "to": "cast", "float": "cast", "bfloat16": "cast", "half": "cast", "type_as": "cast",
}


def selected() -> set:
    """The rewrites ``KTT_FUSE_CHAINS`` asks for (see the module docstring)."""
    raw = os.environ.get("KTT_FUSE_CHAINS")
    names = [t.strip().lower() for t in (raw or "").split(",") if t.strip()]
    if not names or names in (["1"], ["on"], ["true"]):
        return set(REWRITES)
    if names in (["0"], ["off"], ["false"]):
        return set()
    bad = sorted(n for n in names if n not in REWRITES and n != "all")
    if bad:
        raise ValueError(
            f"KTT_FUSE_CHAINS={raw!r}: unknown {', '.join(bad)}; use 0, 1, all or a comma list of "
            f"{', '.join(REWRITES)}"
        )
    return set(REWRITES) if "all" in names else set(names)


def _what(n) -> str | None:
    if not isinstance(n, torch.fx.Node):
        return None
    if n.op == "call_function":
        return _BY_TARGET.get(n.target)
    if n.op == "call_method":
        return _BY_METHOD.get(n.target)
    return None


def _operand(n: torch.fx.Node, i: int, name: str | None = None, default=None):
    if len(n.args) > i:
        return n.args[i]
    if name is not None and name in n.kwargs:
        return n.kwargs[name]
    if i == 0:
        return n.kwargs.get("input", n.kwargs.get("self", default))
    return default


class _Graph:
    """A graph module and what its nodes compute (fake or real tensors)."""

    def __init__(self, gm: torch.fx.GraphModule):
        self.gm = gm
        self.order = {n: i for i, n in enumerate(gm.graph.nodes)}

    def value(self, n):
        """The tensor a node computes, from its metadata (Dynamo ``example_value``, AOT
        ``val``) or, for a module attribute, the attribute itself; else None."""
        if not isinstance(n, torch.fx.Node):
            return None
        v = n.meta.get("val", n.meta.get("example_value"))
        if v is None and n.op == "get_attr":
            obj = self.gm
            try:
                for part in str(n.target).split("."):
                    obj = getattr(obj, part)
            except AttributeError:
                return None
            v = obj
        return v if isinstance(v, torch.Tensor) else None


def _pair(n, kind):
    """The two operands of a binary node of `kind`, else None."""
    if _what(n) != kind:
        return None
    a, b = _operand(n, 0), _operand(n, 1, "other")
    return (a, b) if b is not None else None


def _square_of(g: _Graph, n):
    """t when n computes t * t or t ** 2."""
    p = _pair(n, "mul")
    if p is not None and p[0] is p[1] and isinstance(p[0], torch.fx.Node):
        return p[0]
    if _what(n) == "pow" and _operand(n, 1, "exponent") == 2:
        t = _operand(n, 0)
        return t if isinstance(t, torch.fx.Node) else None
    return None


def _over_last_dim(dims, rank: int) -> bool:
    if isinstance(dims, (list, tuple)):
        if len(dims) != 1:
            return False
        dims = dims[0]
    return isinstance(dims, int) and dims in (-1, rank - 1)


def _match_core(g: _Graph, r: torch.fx.Node):
    """(core, t, eps, nodes) for r = rsqrt(mean(t^2, -1, keepdim) + eps) with a user
    core = t * r, else None."""
    den = _operand(r, 0)
    p = _pair(den, "add")
    if p is None:
        return None
    mean, eps = (p[0], p[1]) if isinstance(p[1], (int, float)) else (p[1], p[0])
    if not isinstance(eps, (int, float)) or isinstance(eps, bool) or _what(mean) != "mean":
        return None
    sq = _operand(mean, 0)
    sv = g.value(sq)
    if sv is None or sv.dim() == 0 or not _over_last_dim(_operand(mean, 1, "dim"), sv.dim()):
        return None
    if not _operand(mean, 2, "keepdim", False) or _operand(mean, 3, "dtype") is not None:
        return None
    t = _square_of(g, sq)
    if t is None:
        return None
    for user in r.users:
        q = _pair(user, "mul")
        if q is not None and (q[0] is t or q[1] is t) and (q[0] is r or q[1] is r):
            return user, t, float(eps), [den, mean, sq, r]
    return None


def _writes(n: torch.fx.Node, targets) -> bool:
    """Whether n may write one of `targets` in place (an in-place method or a mutating
    aten overload taking it)."""
    if not any(a in targets for a in n.all_input_nodes):
        return False
    if n.op == "call_method":
        return str(n.target).endswith("_")
    schema = getattr(n.target, "_schema", None)
    return bool(schema is not None and schema.is_mutable)


def _rewrite_one(g: _Graph, r: torch.fx.Node) -> bool:
    found = _match_core(g, r)
    if found is None:
        return False
    core, t, eps, inner = found
    if any(len(n.users) != 1 for n in inner):
        return False
    source = _operand(t, 0) if _what(t) == "cast" else t
    xv = g.value(source)
    if xv is None or xv.dim() == 0 or not xv.dtype.is_floating_point:
        return False
    width = xv.shape[-1]
    # Forward from t * r: single-user casts and at most one weight row.
    chain, end, weight = inner + [core], core, None
    while len(end.users) == 1:
        nxt = next(iter(end.users))
        if _what(nxt) == "cast":
            end = nxt
        elif weight is None and _pair(nxt, "mul") is not None:
            a, b = _pair(nxt, "mul")
            w = b if a is end else a
            wv = g.value(w)
            if wv is None or tuple(wv.shape) != (width,) or not wv.dtype.is_floating_point:
                break
            end, weight = nxt, w
        else:
            break
        chain.append(end)
    ev = g.value(end)
    if ev is None or tuple(ev.shape) != tuple(xv.shape) or ev.requires_grad:
        return False
    # ktt::rms_norm returns its input's dtype: read the source, or the cast the chain
    # starts from when that one has the result's dtype.
    if ev.dtype != xv.dtype:
        tv = g.value(t)
        if t is source or tv is None or tv.dtype != ev.dtype:
            return False
        source = t
    elif t is not source:
        chain.append(t)  # the cast goes with the chain when nothing else reads it
    first = min(g.order[n] for n in chain)
    last = g.order[end]
    guarded = {source} | ({weight} if isinstance(weight, torch.fx.Node) else set())
    if any(_writes(n, guarded) for n in g.gm.graph.nodes if first <= g.order[n] <= last):
        return False
    graph = g.gm.graph
    with graph.inserting_before(end):
        fused = graph.call_function(torch.ops.ktt.rms_norm.default, (source, weight, None, eps))
    fused.meta = dict(end.meta)
    end.replace_all_uses_with(fused)
    for n in sorted(set(chain), key=lambda n: -g.order[n]):
        if not n.users:
            graph.erase_node(n)
    return True


def rewrite_rms_norms(gm: torch.fx.GraphModule) -> int:
    """Rewrites every RMSNorm chain of `gm` into ``ktt::rms_norm`` (when ``KTT_FUSE_CHAINS``
    selects ``norm``); returns how many, recompiling `gm` when any."""
    if "norm" not in selected():
        return 0
    done = 0
    for r in [n for n in gm.graph.nodes if _what(n) == "rsqrt"]:
        if r.graph is gm.graph and _rewrite_one(_Graph(gm), r):
            done += 1
    if done:
        gm.graph.lint()
        gm.recompile()
    return done


def backend(gm: torch.fx.GraphModule, example_inputs):
    """A ``torch.compile`` backend: the selected rewrites, then the graph as is (its ops
    dispatch to this build's kernels on GPU tensors)."""
    rewrite_rms_norms(gm)
    return gm.forward
