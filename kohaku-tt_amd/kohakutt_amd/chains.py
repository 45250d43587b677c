"""torch.compile graph pass: an RMSNorm written out in torch ops becomes one ``ktt::rms_norm``.

The reference's compile backends fuse such chains before lowering
(``src/kohakutt/torch_backend/chains.py:1-4``); this module does it for graphs compiled
for the MI355X kernels, so a model that spells RMSNorm as

    h = x.to(torch.float32)
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    y = weight * h.to(x.dtype)

(Hugging Face's Llama / Qwen2 norms) runs the fused norm kernel instead of five
elementwise and reduction kernels.

How it matches.  RMSNorm is a product: ``x · rsqrt(rowmean(x²) + eps) · w``.  The pass
therefore looks at products, not at chains of calls:

1. Each FX node is read as a term of a small vocabulary (``_term``): ``mul``, ``add``,
   ``sq`` (both ``t * t`` and ``t ** 2``), ``rowmean`` (a mean over the last dim with
   keepdim and no dtype), ``rsqrt`` and ``cast`` (any dtype conversion), whatever the
   spelling (torch function, operator, tensor method, aten or prims overload).
2. Every maximal product in the graph (nested ``mul`` nodes, casts between them included)
   is flattened into its factor list, last product first.
3. The factors must be: one ``rsqrt(rowmean(sq(u)) + eps)`` (either operand order of the
   add, eps a Python number), one tensor ``t`` that is ``u`` up to casts, and at most one
   floating vector whose size is the row width.  Factor order and nesting do not matter,
   so ``(x * r) * w``, ``w * (x * r)`` and ``(x * w) * r`` all match.
4. The fused op reads the cast of ``x`` (or ``x`` itself) whose dtype is the product's,
   because ``ktt::rms_norm`` returns its input's dtype; a product in a dtype that no such
   value has is left alone.
5. The nodes between that input, the weight and the product's result form the region
   the fused call replaces.  It must be closed (no node outside it reads an interior
   node), hold only nodes of the vocabulary, and see no in-place write to its input or
   weight between its first node and its result.  Results that need a gradient are left
   alone (``ktt::rms_norm`` has no derivative here), as are results shaped unlike the
   input.

``KTT_FUSE_CHAINS`` (read at each compile) selects rewrites by the reference's names:
unset, ``1``, ``on``, ``true`` or ``all`` every one; ``0``, ``off`` or ``false`` none; else
a comma list of ``norm``, ``rotary``, ``mask``, ``gqa`` (an unknown name raises
ValueError).  Only ``norm`` exists here: RoPE fusion and the reference's mask / GQA
conversions serve its own device and are outside this build's hot path.
"""

from __future__ import annotations

import functools
import operator
import os

import torch
import torch.fx

__all__ = ["REWRITES", "selected", "rewrite_rms_norms", "backend"]

REWRITES = ("norm", "rotary", "mask", "gqa")

_ALL_WORDS = ("", "1", "on", "true", "all")
_NONE_WORDS = ("0", "off", "false")


def selected() -> set:
    """The rewrite names ``KTT_FUSE_CHAINS`` selects (case and spaces ignored)."""
    raw = os.environ.get("KTT_FUSE_CHAINS", "")
    words = {w.strip().lower() for w in raw.split(",")} - {""}
    if len(words) <= 1:
        word = next(iter(words), "")
        if word in _ALL_WORDS:
            return set(REWRITES)
        if word in _NONE_WORDS:
            return set()
    unknown = sorted(words - set(REWRITES) - {"all"})
    if unknown:
        raise ValueError(
            f"KTT_FUSE_CHAINS={raw!r} names unknown rewrite(s) {', '.join(unknown)}; "
            f"give 0, 1, all, or names from {', '.join(REWRITES)}"
        )
    return set(REWRITES) if "all" in words else words


# --- step 1: nodes as terms -------------------------------------------------------------

# Names of dtype conversions, as aten / prims packets and as tensor methods.
_CASTS = frozenset({"_to_copy", "convert_element_type", "to", "float", "half", "bfloat16",
                    "double", "type_as"})
# Positional parameter names of each operation; keyword spellings map onto them.
_PARAMS = {
    "mul": ("a", "b"), "add": ("a", "b"), "pow": ("a", "exp"), "rsqrt": ("a",),
    "mean": ("a", "dim", "keepdim", "dtype"), "cast": ("a",),
}
_KEYWORDS = {"input": "a", "self": "a", "other": "b", "exponent": "exp"}


def _op_name(n) -> str | None:
    """The operation an FX node calls, by name, for calls into torch, ``operator``, tensor
    methods and the aten / prims namespaces; None for anything else."""
    if not isinstance(n, torch.fx.Node):
        return None
    if n.op == "call_method":
        name = n.target
    elif n.op == "call_function":
        fn = n.target
        if isinstance(fn, torch._ops.OpOverload):
            if fn.namespace not in ("aten", "prims"):
                return None
            name = fn.overloadpacket.__name__
        else:
            name = getattr(fn, "__name__", None)
            if name is None or not (getattr(torch, name, None) is fn
                                    or getattr(operator, name, None) is fn):
                return None
    else:
        return None
    return "cast" if name in _CASTS else name


def _bind(n: torch.fx.Node, op: str) -> dict:
    """The node's operands under the parameter names of `op`."""
    bound = dict(zip(_PARAMS[op], n.args))
    for key, value in n.kwargs.items():
        bound.setdefault(_KEYWORDS.get(key, key), value)
    return bound


def _term(n):
    """(kind, operands) of a node in the pass's vocabulary, or None.

    kinds: ``mul`` (a, b), ``add`` (a, b), ``sq`` (t,), ``rowmean`` (t,), ``rsqrt`` (t,),
    ``cast`` (t,).  ``rowmean`` needs the node's value to know the rank, so it is decided in
    ``_Region``; here a mean is returned as ``mean`` with its bound operands."""
    op = _op_name(n)
    if op not in _PARAMS:
        return None
    b = _bind(n, op)
    if op == "mul":
        if b.get("b") is None:
            return None
        if b["a"] is b["b"] and isinstance(b["a"], torch.fx.Node):
            return "sq", (b["a"],)
        return "mul", (b["a"], b["b"])
    if op == "pow":
        e = b.get("exp")
        if isinstance(e, (int, float)) and not isinstance(e, bool) and e == 2:
            return "sq", (b["a"],)
        return None
    if op == "add":
        if b.get("b") is None or b.get("alpha", 1) != 1:
            return None
        return "add", (b["a"], b["b"])
    if op == "mean":
        return "mean", (b.get("a"), b.get("dim"), b.get("keepdim", False), b.get("dtype"))
    return op, (b.get("a"),)


def _is_number(v) -> bool:
    return isinstance(v, (int, float)) and not isinstance(v, bool)


def _mutates(n: torch.fx.Node) -> bool:
    """Whether a node may write one of its operands in place."""
    if n.op == "call_method":
        name = str(n.target)
        return name.endswith("_") and not name.endswith("__")
    if n.op == "call_function":
        return n.is_impure()
    return n.op == "call_module"


class _Region:
    """One attempt at one product root of a graph."""

    def __init__(self, gm: torch.fx.GraphModule):
        self.gm = gm
        self.pos = {n: i for i, n in enumerate(gm.graph.nodes)}

    def value(self, n):
        """The (fake or real) tensor a node computes, or None."""
        if not isinstance(n, torch.fx.Node):
            return None
        v = n.meta.get("val", n.meta.get("example_value"))
        if v is None and n.op == "get_attr":
            try:
                v = functools.reduce(getattr, str(n.target).split("."), self.gm)
            except AttributeError:
                v = None
        return v if isinstance(v, torch.Tensor) else None

    def kind(self, n):
        t = _term(n)
        if t is None or t[0] != "mean":
            return t
        src, dim, keepdim, dtype = t[1]
        sv = self.value(src)
        if sv is None or sv.dim() == 0 or keepdim is not True or dtype is not None:
            return None
        if isinstance(dim, (list, tuple)):
            dim = dim[0] if len(dim) == 1 else None
        if not _is_number(dim) or int(dim) % sv.dim() != sv.dim() - 1:
            return None
        return "rowmean", (src,)

    # --- step 2: flatten a product ------------------------------------------------------

    def factors(self, root: torch.fx.Node):
        """The factor list of the maximal product ending at `root` (casts peeled at the top
        and between products), or None when root is not a product."""
        top = root
        while (k := self.kind(top)) is not None and k[0] == "cast":
            top = k[1][0]
        k = self.kind(top)
        if k is None or k[0] != "mul":
            return None
        out, todo = [], list(k[1])
        while todo:
            f = todo.pop()
            if not isinstance(f, torch.fx.Node):
                out.append(f)
                continue
            # A product read only by this one joins it, through casts read only here.
            inner = f
            while len(inner.users) == 1 and (fk := self.kind(inner)) is not None and fk[0] == "cast":
                inner = fk[1][0]
            fk = self.kind(inner)
            if fk is not None and fk[0] == "mul" and len(inner.users) == 1:
                todo.extend(fk[1])
            else:
                out.append(f)
        return out

    # --- step 3: classify the factors ---------------------------------------------------

    def statistic(self, f):
        """(u, eps) when f = rsqrt(rowmean(sq(u)) + eps), possibly cast, else None."""
        k = self.kind(self.cast_chain(f)[-1])
        if k is None or k[0] != "rsqrt":
            return None
        k = self.kind(k[1][0])
        if k is None or k[0] != "add":
            return None
        a, b = k[1]
        mean, eps = (a, b) if _is_number(b) else (b, a)
        if not _is_number(eps):
            return None
        k = self.kind(mean)
        if k is None or k[0] != "rowmean":
            return None
        k = self.kind(k[1][0])
        if k is None or k[0] != "sq":
            return None
        return k[1][0], float(eps)

    def cast_chain(self, n):
        """n, then each value it is a cast of, down to the first node that is not a cast."""
        chain = [n]
        while isinstance(n, torch.fx.Node) and (k := self.kind(n)) is not None and k[0] == "cast":
            n = k[1][0]
            chain.append(n)
        return chain

    def match(self, root: torch.fx.Node):
        """(input, weight, eps, region) for an RMSNorm product ending at root, else None."""
        fs = self.factors(root)
        if fs is None or not 2 <= len(fs) <= 3:
            return None
        stats = [(i, s) for i, f in enumerate(fs) if (s := self.statistic(f)) is not None]
        if len(stats) != 1:
            return None
        i, (u, eps) = stats[0]
        rest = fs[:i] + fs[i + 1:]
        u_chain = self.cast_chain(u)
        rv = self.value(root)
        if rv is None or rv.requires_grad or rv.dim() == 0:
            return None
        width = rv.shape[-1]
        picks = []
        for ti, t in enumerate(rest):
            t_chain = self.cast_chain(t)
            if t_chain[-1] is not u_chain[-1]:
                continue
            others = rest[:ti] + rest[ti + 1:]
            w = others[0] if others else None
            if w is not None:
                wv = self.value(w)
                if wv is None or tuple(wv.shape) != (width,) or not wv.dtype.is_floating_point:
                    continue
            # step 4: the input whose dtype is the result's, the source first
            for cand in reversed(t_chain + u_chain):
                cv = self.value(cand)
                if (cv is not None and cv.dtype == rv.dtype and cv.dtype.is_floating_point
                        and tuple(cv.shape) == tuple(rv.shape)):
                    picks.append((cand, w))
                    break
        for x, w in picks:
            region = self.region(root, {x, w})
            if region is not None:
                return x, w, eps, region
        return None

    # --- step 5: the region -------------------------------------------------------------

    def region(self, root: torch.fx.Node, stops: set):
        """Nodes that root depends on short of `stops`, when they form a closed region of
        vocabulary nodes with no in-place write to a stop inside its span; else None."""
        inside, todo = set(), [root]
        while todo:
            n = todo.pop()
            if n in inside or n in stops:
                continue
            k = self.kind(n)
            if k is None:
                return None
            inside.add(n)
            todo.extend(a for a in n.all_input_nodes)
        if any(u not in inside for n in inside if n is not root for u in n.users):
            return None
        first = min(self.pos[n] for n in inside)
        last = self.pos[root]
        guarded = {s for s in stops if isinstance(s, torch.fx.Node)}
        for n in self.gm.graph.nodes:
            if first <= self.pos[n] <= last and _mutates(n) and guarded & set(n.all_input_nodes):
                return None
        return inside


def rewrite_rms_norms(gm: torch.fx.GraphModule) -> int:
    """Replaces every RMSNorm product of `gm` by one ``ktt::rms_norm`` call (when
    ``KTT_FUSE_CHAINS`` selects ``norm``); returns how many, recompiling `gm` when any."""
    if "norm" not in selected():
        return 0
    graph, done, gone = gm.graph, 0, set()
    for root in reversed(list(graph.nodes)):
        if root in gone or _term(root) is None or _term(root)[0] not in ("mul", "cast"):
            continue
        found = _Region(gm).match(root)
        if found is None:
            continue
        x, w, eps, region = found
        with graph.inserting_before(root):
            fused = graph.call_function(torch.ops.ktt.rms_norm.default, (x, w, None, eps))
        fused.meta = dict(root.meta)
        root.replace_all_uses_with(fused)
        order = {n: i for i, n in enumerate(graph.nodes)}
        for n in sorted(region, key=order.__getitem__, reverse=True):
            graph.erase_node(n)
            gone.add(n)
        done += 1
    if done:
        graph.lint()
        gm.recompile()
    return done


def backend(gm: torch.fx.GraphModule, example_inputs):
    """A ``torch.compile`` backend: the selected rewrites, then the graph as is (its ops
    dispatch to this build's kernels on GPU tensors)."""
    rewrite_rms_norms(gm)
    return gm.forward
