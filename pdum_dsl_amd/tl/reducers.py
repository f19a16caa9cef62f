"""Composite reducers: structured-state folds declared by lift / combine / project.

Restates the reference's CompositeReducer (packages/tensorlib/src/pdum/tl/
mdsl.py:103-118, declared by ``defreducer`` at mdsl.py:221-261) and its
evaluation (compute.py:216-260): each element (m aligned scalars) is LIFTED
to a state of k scalars, states COMBINE left to right, and the answer is the
PROJECTION of the last state. The sweep starts from the first element's
lift; ``init`` (the declared identity) is the state of an empty reduction.

Here the three parts are Python functions over ``Term``s, traced into tile
vocabulary (tl.pointwise over aligned fields) wherever they are needed:
  - the interpreters trace them into small regions and sweep the reduced
    dim (``parts``);
  - ``grad`` lowers a composite tl.reduce / tl.scan to a tl.fold whose step
    is combine(state, lift(element)) (``lower``), so its adjoint is the
    fold's reverse sweep: the reference's composite back-propagation through
    the sweep (autodiff.py:335-400) by the route every fold takes.

    flashsm = defreducer("zoo.flashsm", state=3, element=2,
        lift=lambda s, v: (s, 1.0, v),
        combine=lambda l, r: ...,       # the rescaling merge
        init=(-1e30, 0.0, 0.0),
        project=lambda m, den, o: o / den)
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

from .ir import F64, Builder, Dim, Node, Region, TensorType, minus_dim


@dataclass(frozen=True, eq=False)
class CompositeReducer:
    name: str
    state: int  # k scalars per state
    element: int  # m element operands
    lift: Callable  # (*m terms) -> k terms
    combine: Callable  # (left k-tuple, right k-tuple) -> k terms
    init: tuple  # the identity state: an empty reduction's
    project: Callable | None  # (*k terms) -> term; None = the first component
    associative: bool = True  # declared, not verified (property-test it)

    def __repr__(self) -> str:
        return self.name


_REGISTRY: dict[str, CompositeReducer] = {}


def defreducer(name: str, *, state: int, element: int, lift, combine, init, project=None,
               associative: bool = True) -> CompositeReducer:
    """Declares (and registers under ``name``) a composite reducer; the
    functions are traced once here to check their arities."""
    if not isinstance(state, int) or state < 1 or not isinstance(element, int) or element < 1:
        raise ValueError("state and element are positive counts")
    init = tuple(float(v) for v in init)
    if len(init) != state:
        raise ValueError(f"init must have {state} components, got {len(init)}")
    r = CompositeReducer(name, state, element, lift, combine, init, project, associative)
    parts(r, TensorType((Dim("_x", 0, 1),)))  # arity check by tracing
    _REGISTRY[name] = r  # a redeclaration replaces the definition (and its traced parts)
    return r


def lookup(name: str) -> CompositeReducer:
    try:
        return _REGISTRY[name]
    except KeyError:
        raise TypeError(f"unknown reducer {name!r} (neither a primitive nor a declared composite)") from None


def is_composite(name: str) -> bool:
    return name in _REGISTRY


class Term:
    """A traced value: a node of one aligned field type, or a constant.
    Arithmetic emits tl.pointwise; constants broadcast."""

    __slots__ = ("b", "node", "tt")

    def __init__(self, b: Builder, node: Node, tt: TensorType):
        self.b, self.node, self.tt = b, node, tt

    def _pw(self, f, *xs):
        args = [x.node if isinstance(x, Term) else _const(self.b, float(x)) for x in xs]
        return Term(self.b, self.b.emit("tl.pointwise", *args, f=f), self.tt)

    def __add__(self, o):
        return self._pw("add", self, o)

    def __radd__(self, o):
        return self._pw("add", o, self)

    def __sub__(self, o):
        return self._pw("sub", self, o)

    def __rsub__(self, o):
        return self._pw("sub", o, self)

    def __mul__(self, o):
        return self._pw("mul", self, o)

    def __rmul__(self, o):
        return self._pw("mul", o, self)

    def __truediv__(self, o):
        return self._pw("div", self, o)

    def __rtruediv__(self, o):
        return self._pw("div", o, self)

    def __neg__(self):
        return self._pw("neg", self)


def _const(b: Builder, v: float) -> Node:
    return b.emit("core.const", type=F64, value=float(v))


def _any_term(xs):
    for x in xs:
        if isinstance(x, Term):
            return x
    raise TypeError("a reducer marker needs at least one traced operand")


def _marker(f):
    def apply(*xs):
        return _any_term(xs)._pw(f, *xs)

    apply.__name__ = f
    return apply


exp, log, tanh, sqrt, maximum, minimum, where = (
    _marker(f) for f in ("exp", "log", "tanh", "sqrt", "maximum", "minimum", "where"))


def _field(b: Builder, x, tt: TensorType) -> Node:
    """A traced result as a field of ``tt`` (a constant becomes a tl.const)."""
    if isinstance(x, Term):
        return x.node
    return b.emit("tl.const", value=float(x), dims=tuple((d.name, (d.start, d.stop)) for d in tt.dims))


def apply_lift(b: Builder, f: CompositeReducer, elems, tt: TensorType) -> tuple:
    out = f.lift(*(Term(b, e, tt) for e in elems))
    out = tuple(out) if isinstance(out, (tuple, list)) else (out,)
    if len(out) != f.state:
        raise ValueError(f"{f.name}: lift must produce {f.state} components, got {len(out)}")
    return tuple(_field(b, x, tt) for x in out)


def apply_combine(b: Builder, f: CompositeReducer, left, right, tt: TensorType) -> tuple:
    out = f.combine(tuple(Term(b, x, tt) for x in left), tuple(Term(b, x, tt) for x in right))
    out = tuple(out) if isinstance(out, (tuple, list)) else (out,)
    if len(out) != f.state:
        raise ValueError(f"{f.name}: combine must produce {f.state} components, got {len(out)}")
    return tuple(_field(b, x, tt) for x in out)


def apply_project(b: Builder, f: CompositeReducer, state, tt: TensorType) -> Node:
    if f.project is None:
        return state[0]
    return _field(b, f.project(*(Term(b, x, tt) for x in state)), tt)


@dataclass(frozen=True)
class Parts:
    """lift / combine / project as regions over one aligned field type."""

    lift: Region
    combine: Region
    project: Region


_PARTS: dict[str, dict] = {}


def parts(f: CompositeReducer, tt: TensorType) -> Parts:
    """The reducer's three functions traced as regions whose params all have
    type ``tt`` (cached per reducer and frame set)."""
    from .dialect import OPS

    memo = _PARTS.setdefault(f.name, {})
    key = tuple((d.name, d.start, d.stop) for d in tt.dims)
    if key in memo and memo[key][0] is f:
        return memo[key][1]
    b = Builder(OPS)

    def region(params, ys):
        y = ys[0] if len(ys) == 1 else b.emit("core.tuple", *ys)
        return Region(params=tuple(params), body=(b.emit("core.yield", y),))

    ep = tuple(b.param(("lift", j), tt) for j in range(f.element))
    lp = tuple(b.param(("left", i), tt) for i in range(f.state))
    rp = tuple(b.param(("right", i), tt) for i in range(f.state))
    sp = tuple(b.param(("state", i), tt) for i in range(f.state))
    out = Parts(region(ep, apply_lift(b, f, ep, tt)), region(lp + rp, apply_combine(b, f, lp, rp, tt)),
                region(sp, (apply_project(b, f, sp, tt),)))
    memo[key] = (f, out)
    return out


# ------------------------------------------------------------- lowering for AD


def _zeros(b: Builder, tt: TensorType, value: float = 0.0) -> Node:
    return b.emit("tl.const", value=float(value), dims=tuple((d.name, (d.start, d.stop)) for d in tt.dims))


def _step(f: CompositeReducer, tt: TensorType, emit: bool) -> Region:
    """The fold step: (state | element) -> combine(state, lift(element)),
    and, for a scan, the projection of the new state as the emission."""
    from .dialect import OPS

    b = Builder(OPS)
    sp = tuple(b.param(("s", i), tt) for i in range(f.state))
    ep = tuple(b.param(("e", j), tt) for j in range(f.element))
    new = apply_combine(b, f, sp, apply_lift(b, f, ep, tt), tt)
    ys = new + ((apply_project(b, f, new, tt),) if emit else ())
    y = ys[0] if len(ys) == 1 else b.emit("core.tuple", *ys)
    return Region(params=sp + ep, body=(b.emit("core.yield", y),))


def lower(b: Builder, n: Node, args: tuple) -> Node:
    """A composite tl.reduce / tl.scan ``n`` as tile vocabulary over the
    (re-emitted) element operands ``args``: the first element's lift, a fold
    of combine(state, lift(element)) over the rest, the projection (a scan:
    the fold emits each step's projection; the first position holds the
    first lift's)."""
    f = lookup(n.attr("f"))
    scan = n.op == "tl.scan"
    dim = n.attr("dim") if scan else (lambda d: d if isinstance(d, str) else d[0])(n.attr("dims"))
    tt = args[0].type
    d = tt.dim(dim)
    st = minus_dim(tt, dim)
    if d.size == 0:  # an empty dim: the declared identity state (a scan has nothing to emit)
        if scan:
            return _zeros(b, tt)
        return apply_project(b, f, tuple(_zeros(b, st, v) for v in f.init), st)
    first = tuple(b.emit("tl.select", a, coords=((dim, d.start),)) for a in args)
    s0 = apply_lift(b, f, first, st)
    rest = tuple(b.emit("tl.slice", a, ranges=((dim, (d.start + 1, d.stop)),)) for a in args)
    fat = {"dim": dim, "state": tuple(f"{f.name}.s{i}" for i in range(f.state)),
           "element": tuple(f"{f.name}.e{j}" for j in range(f.element))}
    if not scan:
        finals = tuple(b.emit("tl.fold", *s0, *rest, regions=(_step(f, st, False),), out=("final", i), **fat)
                       for i in range(f.state))
        return apply_project(b, f, finals, st)
    head = b.emit("tl.repeat", apply_project(b, f, s0, st), name=dim, extent=(d.start, d.start + 1))
    head = b.emit("tl.pad", head, extents=((dim, (d.start, d.stop)),), fill=0.0)
    if d.size == 1:
        return head
    em = b.emit("tl.fold", *s0, *rest, regions=(_step(f, st, True),), out=("emit",), **fat)
    em = b.emit("tl.pad", em, extents=((dim, (d.start, d.stop)),), fill=0.0)
    return b.emit("tl.pointwise", head, em, f="add")


def lower_region(region: Region, names: dict) -> tuple[Region, dict]:
    """``region`` with every composite reduce / scan lowered (fold steps
    included), and ``names`` carried to the replacement nodes."""
    from .dialect import OPS

    if not any(_has_composite(nd) for nd in _walk_all(region)):
        return region, names
    b = Builder(OPS)
    memo: dict[int, Node] = {id(p): p for p in region.params}
    new_names = dict(names)

    def go(nd: Node) -> Node:
        if id(nd) in memo:
            return memo[id(nd)]
        args = tuple(go(a) for a in nd.args)
        regions = tuple(lower_region(r, {})[0] for r in nd.regions)
        if nd.op in ("tl.reduce", "tl.scan") and is_composite(nd.attr("f")):
            out = lower(b, nd, args)
        elif all(x is y for x, y in zip(args, nd.args)) and all(x is y for x, y in zip(regions, nd.regions)):
            out = nd
        else:
            explicit = {} if OPS[nd.op].type_rule is not None else {"type": nd.type}
            out = b.emit(nd.op, *args, regions=regions, loc=nd.loc, **explicit, **dict(nd.attrs))
        memo[id(nd)] = out
        if id(nd) in names and out is not nd:
            new_names[id(out)] = names[id(nd)]
        return out

    y = go(region.body[-1])
    return Region(params=region.params, body=(y,)), new_names


def _walk_all(region: Region):
    from .ir import walk

    for nd in walk(region):
        yield nd
        for r in nd.regions:
            yield from _walk_all(r)


def _has_composite(nd: Node) -> bool:
    return nd.op in ("tl.reduce", "tl.scan") and is_composite(nd.attr("f"))


__all__ = ["CompositeReducer", "defreducer", "lookup", "is_composite", "Term", "parts", "lower", "lower_region",
           "exp", "log", "tanh", "sqrt", "maximum", "minimum", "where"]
