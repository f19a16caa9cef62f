"""Reverse-mode AD over a tile-vocabulary region: the joint (target, *grads).

Restates the contract of the reference's ``autodiff.grad``
(packages/tensorlib/src/pdum/tl/autodiff.py:102-148): a region, the name of
its target, a SEED (the target's cotangent, a runtime input appended as the
joint's LAST param) and the names of the inputs to differentiate; the result
is a ``RegionGrad`` whose joint region yields ``(target, *grads)``.

This is the part of the reference's AD the fusion templates' backward is
built from (the naive attention twin of zoo/tiles.py:238-252 and the row
templates), over the vocabulary this backend reads:

  tl.pointwise   the derivative of each numpy marker (dsl/derivative.py's
                 table restated per marker below)
  tl.reduce      sum -> broadcast; mean -> broadcast / N;
                 max / min -> the cotangent to the FIRST position attaining
                 the extremum along each reduced dim, found by a tl.scan
                 prefix count of the hits (autodiff.py:635-665)
  tl.scan        sum -> the scan of the cotangent the other way (a prefix
                 sum's adjoint is a suffix sum, autodiff.py:667-677); other
                 primitive reducers refuse, as in the reference
  tl.repeat_like / tl.repeat   -> sum over the added dims
  tl.take        -> tl.scatter_add of the cotangent at the same indices
                 (duplicates sum), and tl.scatter_add -> tl.take
                 (autodiff.py:846-856); indices carry no gradient
  layout views (autodiff.py:765-806): tl.shift -> the opposite shift,
                 tl.slice -> tl.pad with zeros back to the operand's frames,
                 tl.pad -> tl.slice (the fill carries no gradient),
                 tl.flip -> tl.flip, tl.select -> repeat at the point + pad,
                 tl.split -> tl.merge, tl.merge -> tl.split
  softmax        the max of a max-subtracted softmax that feeds nothing else
                 gets no cotangent (shift invariance: its terms sum to zero);
                 grad(..., shift_invariant_softmax=False) keeps the
                 reference's route through the max's adjoint
  taps and strides (autodiff.py:680-763): tl.window / tl.stencil -> each
                 tap's slice of the cotangent shifted back (a stencil's fill
                 carries nothing); tl.decimate -> the cotangent spread onto
                 every factor-th cell, zero between; tl.diagonal -> the
                 cotangent where all parts agree, zero elsewhere
  tl.round_to    straight-through, or no flow with grad="zero"
                 (autodiff.py:843-845)
  tl.stage       identity
  core.const / tl.const / tl.iota / comparisons / stop_gradient: no flow

  tl.fold        a reverse fold over the flipped sequences whose step is the
                 forward step's VJP (grad of the step against the carried
                 cotangent), states before each step from the forward
                 trajectory (autodiff.py:411-605), under the reference's
                 schedules (one segment, K uniform segments, binomial
                 revolve). Read at its final state the carry starts at the
                 cotangent; an emitting fold's reverse step also takes each
                 emission's cotangent as an element.
  composite tl.reduce / tl.scan   lowered to the fold they denote (the first
                 element's lift, combine(state, lift(element)), the
                 projection; pdum_dsl_amd.tl.reducers.lower) and
                 differentiated as that fold: the composite sweep's
                 back-propagation (autodiff.py:335-400)

Anything else (argtopk) refuses by name: a primitive joins the AD with its
linearization, or not at all.
"""

from __future__ import annotations

from dataclasses import dataclass
from functools import lru_cache

from .dialect import OPS
from .ir import F64, Builder, Node, Region, TensorType
from .reducers import lower_region

# markers through which no gradient flows (piecewise-constant or boolean)
_FLAT = frozenset({"eq", "ne", "le", "lt", "ge", "gt", "floor", "stop_gradient"})


@dataclass(frozen=True)
class RegionGrad:
    """The joint region and its naming (autodiff.py:136-148): ``region``
    yields (target, *grads); ``outputs`` names the yield slots in order;
    ``grads`` maps each requested input name to its gradient's name (None:
    no gradient flows); ``names`` maps node ids to names; ``nodes`` maps the
    yielded names to nodes. The seed is the joint's LAST param."""

    region: Region
    grads: dict
    names: dict
    outputs: tuple
    nodes: dict


def region_names(region: Region, param_names, outputs=("out",)) -> dict:
    """The naming assignment grad joins on: params by position, then the
    yielded value(s) (dialect.region_names in the reference)."""
    if len(param_names) != len(region.params):
        raise ValueError(f"{len(region.params)} params need {len(region.params)} names, got {len(param_names)}")
    names = {id(p): nm for p, nm in zip(region.params, param_names)}
    y = region.body[-1].args[0]
    ys = y.args if y.op == "core.tuple" else (y,)
    if len(outputs) != len(ys):
        raise ValueError(f"{len(ys)} yielded value(s) need {len(ys)} output name(s)")
    for n, nm in zip(ys, outputs):
        names[id(n)] = nm
    return names


def _is_tensor(n) -> bool:
    return isinstance(n.type, TensorType)


def grad(
    region: Region,
    target: str,
    inputs: dict | None = None,
    seed: str | None = None,
    wrt: tuple | None = None,
    target_unit=None,
    fold_segments: int | None = None,
    fold_slots: int | None = None,
    *,
    names=None,
    shift_invariant_softmax: bool = True,
) -> RegionGrad:
    """Reverse-mode AD of ``region``'s node named ``target``, with the
    reference's signature and positional order (autodiff.py:102-113).

    ``seed`` names the target's cotangent (required for a non-scalar target:
    reverse mode computes vector-Jacobian products); it becomes the joint's
    last param. ``wrt`` names the params to differentiate (all params by
    default).

    ``inputs`` (input signatures) and ``target_unit`` feed the reference's
    unit inference, which this backend does not model: a dict of inputs is
    accepted and ignored, a target unit other than None refuses.
    ``fold_segments`` / ``fold_slots`` pick the reference's checkpointed fold
    schedules (autodiff.py:563-605): K uniform segments (K must divide the
    fold's extent), or binomial revolve over ``fold_slots`` checkpoint slots.
    Both trade recomputation for memory and leave the gradient's values
    unchanged; None for both is the one-segment adjoint.

    ``shift_invariant_softmax`` (keyword only, on by default): the max of a
    max-subtracted softmax that feeds nothing else takes no cotangent. With
    False the max's cotangent flows through the first-occurrence adjoint as
    in the reference, and the joint carries its tl.scan."""
    if names is None:
        raise ValueError("grad joins on names — pass names=region_names(region, param_names)")
    if inputs is not None and not isinstance(inputs, dict):
        raise TypeError(f"inputs must be a dict of input signatures (got {type(inputs).__name__})")
    if fold_segments is not None and fold_slots is not None:
        raise ValueError(
            "pass fold_segments (uniform K-way checkpointing) OR fold_slots (binomial revolve), not both — "
            "they name different schedules"
        )
    if fold_slots is not None and int(fold_slots) < 1:
        raise ValueError("fold_slots must be >= 1 (the number of checkpoint slots)")
    if fold_segments is not None and int(fold_segments) < 1:
        raise ValueError("fold_segments must be >= 1")
    if target_unit is not None:
        raise NotImplementedError("grad: target_unit — units are not modelled by this backend; pass None")
    schedule = (None if fold_segments is None else int(fold_segments), None if fold_slots is None else int(fold_slots))
    # composite reductions differentiate as the folds they are (first lift, combine, project)
    region, names = lower_region(region, names)
    by_name: dict = {}
    for p in region.params:
        by_name.setdefault(names[id(p)], p)
    for n in _ancestors(region.body[-1]):
        nm = names.get(id(n))
        if nm is not None:
            by_name.setdefault(nm, n)
    if target not in by_name:
        raise KeyError(f"target {target!r} is not defined by the program")
    if seed is not None and seed in by_name:
        raise ValueError(f"seed name {seed!r} collides with a program variable; pick a fresh name")
    tnode = by_name[target]
    if wrt is None:
        wrt = tuple(names[id(p)] for p in region.params)
    for nm in wrt:
        if nm not in by_name or by_name[nm].op != "core.param":
            raise KeyError(f"{nm!r} names no param of the program")

    b = Builder(OPS)
    const = lambda v: b.emit("core.const", type=F64, value=float(v))  # noqa: E731
    pw = lambda f, *xs: b.emit("tl.pointwise", *xs, f=f)  # noqa: E731

    def rl(x, like):  # x broadcast over like's dims (a scalar cotangent onto a zero field of like's shape)
        if _is_tensor(x):
            return b.emit("tl.repeat_like", x, like)
        zero = b.emit("tl.const", value=0.0, dims=tuple((d.name, (d.start, d.stop)) for d in like.type.dims))
        return b.emit("tl.pointwise", zero, x, f="add")

    if seed is None:
        if _is_tensor(tnode) and tnode.type.dims:
            raise ValueError(
                f"target {target!r} is not a scalar; pass seed= (the name of a runtime input aligned with the "
                "target) — reverse mode computes vector-Jacobian products"
            )
        seed_node = const(1.0)
        seed_param = None
    else:
        seed_param = b.param(("grad.seed",), tnode.type)
        seed_node = seed_param

    cot: dict[int, list] = {id(tnode): [seed_node]}
    inert = _softmax_shifts(tnode) if shift_invariant_softmax else set()

    def contribute(n, g):
        if n.op in ("core.const", "tl.const", "tl.iota") or id(n) in inert:
            return
        cot.setdefault(id(n), []).append(g)

    def total(n):
        parts = cot.get(id(n))
        if not parts:
            return None
        acc = parts[0]
        for p in parts[1:]:
            acc = pw("add", acc, p)
        return acc

    order = [n for n in _ancestors_of(tnode)]
    # only nodes with a wrt param among their ancestors carry a cotangent anyone reads
    wanted = {id(by_name[nm]) for nm in wrt}
    live: set = set()
    for n in order:  # operands before users
        if id(n) in wanted or any(id(a) in live for a in n.args):
            live.add(id(n))
    final: dict[int, Node] = {}
    for n in reversed(order):
        c = total(n)
        final[id(n)] = c
        if c is None or n.op == "core.param" or id(n) not in live:
            continue
        op = n.op
        if op in ("core.const", "tl.const", "tl.iota"):
            continue
        if op == "tl.stage":
            contribute(n.args[0], c)
        elif op == "tl.pointwise":
            _pointwise_rule(n, c, contribute, pw, const)
        elif op == "tl.reduce":
            x = n.args[0]
            f = n.attr("f")
            dims = n.attr("dims")
            dims = (dims,) if isinstance(dims, str) else tuple(dims)
            if f == "sum":
                contribute(x, rl(c, x))
            elif f == "mean":
                cnt = 1
                for d in dims:
                    cnt *= x.type.dim(d).size
                contribute(x, rl(pw("div", c, const(cnt)), x))
            elif f in ("max", "min"):
                # The cotangent goes to the FIRST position attaining the
                # extremum along each reduced dim (autodiff.py:635-665): hits
                # are eq(x, extremum); an inclusive prefix count of hits
                # (tl.scan sum) equals 1 from the first hit up to the second,
                # so hit * (count == 1) keeps the first alone. A multi-dim
                # reduce is taken one dim at a time, innermost link last.
                links, src = [], x
                for i, name in enumerate(dims):
                    dst = n if i == len(dims) - 1 else b.emit("tl.reduce", src, dims=(name,), f=f)
                    links.append((src, dst, name))
                    src = dst
                back = c
                for src, dst, name in reversed(links):
                    hit = pw("eq", src, rl(dst, src))
                    count = b.emit("tl.scan", pw("where", hit, const(1.0), const(0.0)), dim=name, f="sum")
                    first = pw("mul", hit, pw("eq", count, const(1.0)))
                    back = pw("mul", first, rl(back, src))
                contribute(x, back)
            else:
                raise NotImplementedError(f"tl.reduce {f!r} has no adjoint rule here")
        elif op == "tl.scan":
            if n.attr("f") != "sum":
                raise NotImplementedError(f"tl.scan {n.attr('f')!r} has no adjoint rule (only scan sum)")
            rev = not n.attr("reverse", False)
            extra = {"reverse": True} if rev else {}
            contribute(n.args[0], b.emit("tl.scan", c, dim=n.attr("dim"), f="sum", **extra))
        elif op == "tl.repeat_like":
            x, like = n.args
            added = tuple(d.name for d in like.type.dims if not x.type.has(d.name))
            contribute(x, b.emit("tl.reduce", c, dims=added, f="sum") if added else c)
        elif op == "tl.repeat":
            contribute(n.args[0], b.emit("tl.reduce", c, dims=(n.attr("name"),), f="sum"))
        elif op == "tl.take":
            # the gather's adjoint is the scatter-add at the same indices: rows
            # gathered twice receive the sum (autodiff.py:846-853); the
            # indices carry no gradient
            table, idx = n.args
            d = table.type.dim(n.attr("dim"))
            survivors = {x.name for x in table.type.dims if x.name != d.name}
            spliced = tuple(nm for nm in idx.type.names if nm not in survivors)
            contribute(table, b.emit("tl.scatter_add", c, idx, dim=d.name, extent=(d.start, d.stop), over=spliced))
        elif op == "tl.scatter_add":  # and the scatter-add's is the gather (autodiff.py:854-856)
            contribute(n.args[0], b.emit("tl.take", c, n.args[1], dim=n.attr("dim")))
        elif op == "tl.shift":  # a relabelling of frames: shift back
            back = tuple((nm, -int(dv)) for nm, dv in n.attr("deltas"))
            contribute(n.args[0], b.emit("tl.shift", c, deltas=back))
        elif op == "tl.slice":  # the window's cotangent, zero outside it
            x = n.args[0]
            ext = tuple((nm, (x.type.dim(nm).start, x.type.dim(nm).stop)) for nm, _ in n.attr("ranges"))
            contribute(x, b.emit("tl.pad", c, extents=ext, fill=0.0))
        elif op == "tl.pad":  # the operand's cells; the fill is a constant
            x = n.args[0]
            rng = tuple((nm, (x.type.dim(nm).start, x.type.dim(nm).stop)) for nm, _ in n.attr("extents"))
            contribute(x, b.emit("tl.slice", c, ranges=rng))
        elif op == "tl.flip":
            contribute(n.args[0], b.emit("tl.flip", c, name=n.attr("name")))
        elif op == "tl.select":  # the point's cotangent, zero elsewhere along each fixed dim
            x = n.args[0]
            cur = c
            for nm, i in n.attr("coords"):
                cur = b.emit("tl.repeat", cur, name=nm, extent=(int(i), int(i) + 1))
            ext = tuple((nm, (x.type.dim(nm).start, x.type.dim(nm).stop)) for nm, _ in n.attr("coords"))
            contribute(x, b.emit("tl.pad", cur, extents=ext, fill=0.0))
        elif op == "tl.split":  # the blocks merged back, outer first
            parts = tuple(nm for nm, _ in n.attr("parts"))
            contribute(n.args[0], b.emit("tl.merge", c, parts=parts, name=n.attr("name")))
        elif op == "tl.merge":
            x = n.args[0]
            parts = n.attr("parts")
            parts = (parts,) if isinstance(parts, str) else tuple(parts)
            contribute(x, b.emit("tl.split", c, name=n.attr("name"),
                                 parts=tuple((nm, x.type.dim(nm).size) for nm in parts)))
        elif op == "tl.rename":  # a relabelling: the cotangent takes the operand's names back
            back = tuple(sorted((new, old) for old, new in n.attr("mapping")))
            contribute(n.args[0], b.emit("tl.rename", c, mapping=back))
        elif op == "tl.fold":
            _fold_rule(b, n, c, contribute, const, *schedule)
        elif op in ("tl.window", "tl.stencil"):
            _tap_rule(b, n, c, contribute)
        elif op == "tl.decimate":
            _decimate_rule(b, n, c, contribute, pw, const)
        elif op == "tl.diagonal":
            _diagonal_rule(b, n, c, contribute, pw, const)
        elif op == "tl.round_to":  # straight-through unless declared zero (autodiff.py:843-845)
            if n.attr("grad", "straight_through") != "zero":
                contribute(n.args[0], c)
        else:
            raise NotImplementedError(
                f"{op} has no adjoint rule in this build (a primitive joins the AD with its linearization)"
            )

    grads, nodes = {}, {target: tnode}
    ys = [tnode]
    outputs = [target]
    jnames = dict(names)
    for nm in wrt:
        g = final.get(id(by_name[nm]))
        if g is None:
            grads[nm] = None
            continue
        gname = f"d{nm}"
        grads[nm] = gname
        ys.append(g)
        outputs.append(gname)
        nodes[gname] = g
        jnames[id(g)] = gname
    params = tuple(region.params) + ((seed_param,) if seed_param is not None else ())
    if seed_param is not None:
        jnames[id(seed_param)] = seed
    y = b.emit("core.tuple", *ys) if len(ys) > 1 else ys[0]
    joint = Region(params=params, body=(b.emit("core.yield", y),))
    return RegionGrad(joint, grads, jnames, tuple(outputs), nodes)


@lru_cache(maxsize=None)
def revolve_cost(slots: int, steps: int) -> float:
    """The fewest forward steps re-advanced to reverse ``steps`` fold steps
    with ``slots`` checkpoint slots (Griewank & Walther's binomial revolve):
    a range that fits the slots (or is one step) is reversed as stored; a
    longer one advances a head of m steps, checkpoints, reverses the tail with
    one slot fewer, then the head with the same slots."""
    if steps <= 1 or slots >= steps:
        return 0.0
    if slots < 1:
        return float("inf")
    return min(m + revolve_cost(slots - 1, steps - m) + revolve_cost(slots, m) for m in range(1, steps))


@lru_cache(maxsize=None)
def revolve_split(slots: int, steps: int) -> int:
    """The head length of an optimal revolve split (1 <= slots < steps, steps
    >= 2), the longest among the optimal ones: the schedule the reference's
    split rule picks (autodiff.py:88-99), so the joints agree in shape."""
    best = revolve_cost(slots, steps)
    return max(m for m in range(1, steps)
               if m + revolve_cost(slots - 1, steps - m) + revolve_cost(slots, m) == best)


def _fold_rule(b, n, c, contribute, const, fold_segments=None, fold_slots=None):
    """The adjoint of a fold read at its final state o (autodiff.py:411-605):
    reverse folds over the flipped sequences whose carry is the cotangent of
    the states after each step.

    - The states before step t: each state's trajectory (an emitting fold of
      the same step) shifted one step later, the initial state at the first.
    - The reverse step is the VJP of the forward step: ``grad`` of the scalar
      sum_i <ct_i, step(s, e)_i> with respect to the step's own params, the
      ct_i bound as extra params. Its state gradients are the next carry, its
      element gradients the emissions.
    - The reverse carry starts at (c for state o, zero for the others): the
      cotangent of the final states. The reference injects c at the last step
      through a padded sequence instead; the sum is the same.
    - The schedule: one segment (the whole range reversed from the stored
      trajectory); ``fold_segments`` = K uniform segments, each reversed from
      its start state, which a forward fold over the segments before it
      re-advances; or ``fold_slots`` = S, binomial revolve: a range longer
      than its slots is split (revolve_split), its tail reversed from a
      checkpoint with one slot fewer, then its head.
    The carry's final value is the initial states' cotangent; the emissions,
    flipped back and padded to the whole range, the element sources'. Nested
    folds in the step differentiate through the same rule (grad recurses,
    one segment)."""
    state = tuple(n.attr("state"))
    k = len(state)
    dim = n.attr("dim")
    out = tuple(n.attr("out"))
    emits = out[0] == "emit"  # c is then the cotangent of every step's emission, stacked along dim
    o = None if emits else out[1]
    inits, elems = n.args[:k], n.args[k:]
    d = elems[0].type.dim(dim)
    start, stop = d.start, d.stop
    step = n.regions[0]
    y = step.body[-1].args[0]
    ynodes = tuple(y.args) if y.op == "core.tuple" else (y,)
    sp, ep = step.params[:k], step.params[k:]
    fat = {"dim": dim, "state": state, "element": tuple(n.attr("element"))}

    def zeros(tt):
        return b.emit("tl.const", value=0.0, dims=tuple((x.name, (x.start, x.stop)) for x in tt.dims))

    if stop == start:  # no step runs: the fold is its initial state (and emits nothing)
        if not emits:
            contribute(inits[o], c)
        return

    def with_yield(vals):
        wb = Builder(OPS)
        yy = vals[0] if len(vals) == 1 else wb.emit("core.tuple", *vals)
        return Region(params=step.params, body=(wb.emit("core.yield", yy),))

    if emits:  # the states alone, for the folds that re-advance them
        step = with_yield(ynodes[:k])
    # the step's VJP: grad of sum_i <ct_i, y_i> over the step's params (an
    # emitting fold's emission y_k pairs with the emission's cotangent ct_k)
    nct = k + (1 if emits else 0)
    wb = Builder(OPS)
    cts = tuple(wb.param(("fold.ct", i), ynodes[i].type) for i in range(nct))
    tgt = None
    for i in range(nct):
        t_ = wb.emit("tl.pointwise", ynodes[i], cts[i], f="mul")
        if t_.type.dims:
            t_ = wb.emit("tl.reduce", t_, dims=tuple(x.name for x in t_.type.dims), f="sum")
        tgt = t_ if tgt is None else wb.emit("tl.pointwise", tgt, t_, f="add")
    wrapper = Region(params=tuple(step.params) + cts, body=(wb.emit("core.yield", tgt),))
    pnames = tuple(f"s{i}" for i in range(k)) + tuple(f"e{j}" for j in range(len(ep))) + tuple(
        f"ct{i}" for i in range(nct))
    vjp = grad(wrapper, "fold.vjp", wrt=pnames[:k + len(ep)], names=region_names(wrapper, pnames, ("fold.vjp",)))
    flows = tuple(vjp.grads.get(f"s{i}") is not None for i in range(k))

    def g_of(nm, tt):
        gname = vjp.grads.get(nm)
        return zeros(tt) if gname is None else vjp.nodes[gname]

    dstate = tuple(g_of(f"s{i}", sp[i].type) for i in range(k))
    # reverse step: carries ct, elements (states before the step, the step's
    # elements, and for an emitting fold the emission's cotangent)
    rparams = cts[:k] + tuple(step.params) + cts[k:]
    rat = {"dim": dim, "state": tuple(f"fold.ct{i}" for i in range(k)),
           "element": tuple(f"fold.prev{i}" for i in range(k)) + fat["element"] + (("fold.ce",) if emits else ())}

    def rstep(extra=()):
        rb = Builder(OPS)
        vals = dstate + tuple(extra)
        yy = vals[0] if len(vals) == 1 else rb.emit("core.tuple", *vals)
        return Region(params=rparams, body=(rb.emit("core.yield", yy),))

    flip = lambda v: b.emit("tl.flip", v, name=dim)  # noqa: E731

    def seg(lo, hi):  # the element sequences over steps [lo, hi)
        if (lo, hi) == (start, stop):
            return tuple(elems)
        return tuple(b.emit("tl.slice", e, ranges=((dim, (lo, hi)),)) for e in elems)

    def advance(s0, lo, hi):  # the states after steps [lo, hi), from s0
        se = seg(lo, hi)
        return tuple(b.emit("tl.fold", *s0, *se, regions=(step,), out=("final", i), **fat) for i in range(k))

    def leaf(lo, hi, s0, cur):
        """Steps [lo, hi) reversed from their start state s0 and the carry cur
        after hi: the element cotangents contributed, the carry at lo returned."""
        se = seg(lo, hi)
        prev = []
        for i in range(k):
            traj = b.emit("tl.fold", *s0, *se, regions=(with_yield(ynodes[:k] + (ynodes[i],)),), out=("emit",),
                          **fat)
            if hi - lo > 1:
                later = b.emit("tl.slice", b.emit("tl.shift", traj, deltas=((dim, 1),)), ranges=((dim, (lo + 1, hi)),))
                later = b.emit("tl.pad", later, extents=((dim, (lo, hi)),), fill=0.0)
            else:
                later = zeros(traj.type)
            first = b.emit("tl.pointwise", b.emit("tl.iota", later, name=dim), const(lo), f="eq")
            init_t = b.emit("tl.repeat", s0[i], name=dim, extent=(lo, hi))
            prev.append(b.emit("tl.pointwise", first, init_t, later, f="where"))
        rsrc = tuple(flip(v) for v in prev) + tuple(flip(v) for v in se)
        if emits:
            ce = c if (lo, hi) == (start, stop) else b.emit("tl.slice", c, ranges=((dim, (lo, hi)),))
            rsrc += (flip(ce),)
        for j, ev_ in enumerate(elems):
            if vjp.grads.get(f"e{j}") is None:
                continue
            em = flip(b.emit("tl.fold", *cur, *rsrc, regions=(rstep((vjp.nodes[vjp.grads[f"e{j}"]],)),),
                             out=("emit",), **rat))
            if (lo, hi) != (start, stop):
                em = b.emit("tl.pad", em, extents=((dim, (start, stop)),), fill=0.0)
            contribute(ev_, em)
        return tuple(b.emit("tl.fold", *cur, *rsrc, regions=(rstep(),), out=("final", i), **rat) if flows[i]
                     else zeros(inits[i].type) for i in range(k))

    cur = tuple(c if i == o else zeros(inits[i].type) for i in range(k))  # o is None for an emitting fold
    T = stop - start
    if fold_slots is not None:
        def revolve(lo, hi, slots, boundary):
            nonlocal cur
            if hi - lo <= 1 or slots >= hi - lo:
                cur = leaf(lo, hi, boundary, cur)
                return
            mid = lo + revolve_split(slots, hi - lo)
            revolve(mid, hi, slots - 1, advance(boundary, lo, mid))
            revolve(lo, mid, slots, boundary)

        revolve(start, stop, int(fold_slots), tuple(inits))
    else:
        K = 1 if fold_segments is None else min(int(fold_segments), T)
        if K < 1:
            raise ValueError("fold_segments must be >= 1")
        if T % K:
            raise ValueError(f"fold_segments={K} must divide the fold extent {T} (pad the dim or pick a divisor)")
        L_ = T // K
        starts = [tuple(inits)]
        for j in range(K - 1):
            starts.append(advance(starts[-1], start + j * L_, start + (j + 1) * L_))
        for j in reversed(range(K)):
            cur = leaf(start + j * L_, start + (j + 1) * L_, starts[j], cur)
    for i in range(k):
        if flows[i]:
            contribute(inits[i], cur[i])


def _tap_rule(b, n, c, contribute):
    """tl.window / tl.stencil (autodiff.py:680-697): tap j read x at
    x' + dilation j, so its slice of the cotangent shifts back by dilation j;
    the cells a stencil tap read outside the domain (the fill) carry nothing."""
    x = n.args[0]
    name = n.attr("name")
    d = x.type.dim(name)
    kn = n.attr("k_name") or f"{name}_k"
    kd, dil = n.type.dim(kn), n.attr("dilation", 1)
    for j in range(kd.start, kd.stop):
        t = b.emit("tl.shift", b.emit("tl.select", c, coords=((kn, j),)), deltas=((name, j * dil),))
        sd = t.type.dim(name)
        lo, hi = max(d.start, sd.start), min(d.stop, sd.stop)
        if hi <= lo:
            continue
        if (lo, hi) != (sd.start, sd.stop):
            t = b.emit("tl.slice", t, ranges=((name, (lo, hi)),))
        if (lo, hi) != (d.start, d.stop):
            t = b.emit("tl.pad", t, extents=((name, (d.start, d.stop)),), fill=0.0)
        contribute(x, t)


def _fresh(names, base):
    i = 0
    while f"_{base}{i}" in names:
        i += 1
    return f"_{base}{i}"


def _decimate_rule(b, n, c, contribute, pw, const):
    """tl.decimate (autodiff.py:699-736): output j read x at factor j + p.
    The cotangent, renumbered from 0, gains a phase dim of size factor that
    is zero except at phase 0; merged (outer j, inner phase) and shifted to
    factor j0 + p it lands on the read cells, then is cut and padded to x's
    domain. Any domain works (no divisibility needed)."""
    x = n.args[0]
    name, f = n.attr("name"), n.attr("factor")
    p = int(n.attr("phase", 0)) % f
    d, od = x.type.dim(name), n.type.dim(name)
    if od.size == 0:
        return
    taken = set(n.type.names) | set(x.type.names)
    cn = _fresh(taken, "c")
    ph = _fresh(taken | {cn}, "ph")
    r = b.emit("tl.shift", b.emit("tl.rename", c, mapping=((name, cn),)), deltas=((cn, -od.start),))
    r = b.emit("tl.repeat", r, name=ph, extent=(0, f))
    r = pw("where", pw("eq", b.emit("tl.iota", r, name=ph), const(0.0)), r, const(0.0))
    r = b.emit("tl.merge", r, parts=(cn, ph), name=name)
    lo = f * od.start + p
    r = b.emit("tl.shift", r, deltas=((name, lo),))
    hi = min(d.stop, lo + f * od.size)
    if hi != lo + f * od.size:
        r = b.emit("tl.slice", r, ranges=((name, (lo, hi)),))
    if (lo, hi) != (d.start, d.stop):
        r = b.emit("tl.pad", r, extents=((name, (d.start, d.stop)),), fill=0.0)
    contribute(x, r)


def _diagonal_rule(b, n, c, contribute, pw, const):
    """tl.diagonal (autodiff.py:738-763, for any number of parts): the
    cotangent at z goes to the cell where every part equals z. It takes the
    first part's name, is repeated over the other parts' domains, kept where
    their coordinates equal the first's, and padded to the first's domain."""
    x = n.args[0]
    parts = n.attr("parts")
    parts = (parts,) if isinstance(parts, str) else tuple(parts)
    z = n.attr("name")
    zd = n.type.dim(z)
    if zd.size == 0:
        return
    x0 = parts[0]
    r = c if z == x0 else b.emit("tl.rename", c, mapping=((z, x0),))
    for q in parts[1:]:
        qd = x.type.dim(q)
        r = b.emit("tl.repeat", r, name=q, extent=(qd.start, qd.stop))
    keep = None
    for q in parts[1:]:
        m = pw("eq", b.emit("tl.iota", r, name=x0), b.emit("tl.iota", r, name=q))
        keep = m if keep is None else pw("mul", keep, m)
    r = pw("where", keep, r, const(0.0))
    d0 = x.type.dim(x0)
    if (zd.start, zd.stop) != (d0.start, d0.stop):
        r = b.emit("tl.pad", r, extents=((x0, (d0.start, d0.stop)),), fill=0.0)
    contribute(x, r)


def _pointwise_rule(n, c, contribute, pw, const):
    f = n.attr("f")
    A = n.args
    if f in _FLAT:
        return
    if f == "add":
        for a in A:
            contribute(a, c)
    elif f == "sub":
        contribute(A[0], c)
        contribute(A[1], pw("neg", c))
    elif f == "neg":
        contribute(A[0], pw("neg", c))
    elif f == "mul":
        contribute(A[0], pw("mul", c, A[1]))
        contribute(A[1], pw("mul", c, A[0]))
    elif f == "div":
        contribute(A[0], pw("div", c, A[1]))
        contribute(A[1], pw("neg", pw("div", pw("mul", c, n), A[1])))  # -c a / b^2 = -(c (a/b)) / b
    elif f == "exp":
        contribute(A[0], pw("mul", c, n))
    elif f == "log":
        contribute(A[0], pw("div", c, A[0]))
    elif f == "sqrt":
        contribute(A[0], pw("div", c, pw("mul", n, const(2.0))))
    elif f == "tanh":
        contribute(A[0], pw("mul", c, pw("sub", const(1.0), pw("mul", n, n))))
    elif f == "zoo.gelu":  # a composite marker: its derived partial marker f.d0 (autodiff.py:303-309)
        contribute(A[0], pw("mul", c, pw("zoo.gelu.d0", A[0])))
    elif f == "sin":
        contribute(A[0], pw("mul", c, pw("cos", A[0])))
    elif f == "cos":
        contribute(A[0], pw("neg", pw("mul", c, pw("sin", A[0]))))
    elif f == "abs":
        contribute(A[0], pw("where", pw("ge", A[0], const(0.0)), c, pw("neg", c)))
    elif f in ("maximum", "minimum"):
        first = pw("ge" if f == "maximum" else "le", A[0], A[1])
        contribute(A[0], pw("where", first, c, const(0.0)))
        contribute(A[1], pw("where", first, const(0.0), c))
    elif f == "where":
        m, x, y = A
        contribute(x, pw("where", m, c, const(0.0)))
        contribute(y, pw("where", m, const(0.0), c))
    else:
        raise NotImplementedError(f"marker {f!r} has no entry in the derivative table")


def _softmax_shifts(root: Node) -> set:
    """ids of the max (and its broadcast) of every softmax
    div(exp(x - rl(max x)), rl(sum exp(x - rl(max x)))) under ``root`` that
    feeds nothing but that softmax. Softmax is invariant to the shift, so
    the max's total derivative is zero in exact arithmetic: the reference's
    rules route the cotangent through the max's first-occurrence adjoint
    (autodiff.py:635-665), where the terms cancel (sum_s P_s (dP_s - delta) =
    0); here they are not emitted at all."""
    from .fusion import match_softmax

    order = _ancestors_of(root)
    users: dict[int, list] = {}
    for n in order:
        for a in n.args:
            users.setdefault(id(a), []).append(n)
    users.setdefault(id(root), []).append(None)  # the target is read by the joint

    def only(n, *allowed):
        us = users.get(id(n), [])
        return bool(us) and all(u is not None and any(u is x for x in allowed) for u in us)

    inert: set = set()
    for n in order:
        m = match_softmax(n)
        if m is None:
            continue
        mx, den = m["max"], m["den"]
        e, rld = n.args
        sub = e.args[0]
        rlm = sub.args[1]
        # rld = repeat_like(den, e) reads e for its shape only
        if (only(mx, rlm) and only(rlm, sub) and only(sub, e) and only(e, n, den, rld) and only(den, rld)
                and only(rld, n)):
            inert.update((id(mx), id(rlm)))
    return inert


def _ancestors_of(root: Node):
    """Nodes the root depends on, operands before users (each once)."""
    seen: set[int] = set()
    out: list = []
    stack = [(root, False)]
    while stack:
        x, done = stack.pop()
        if done:
            out.append(x)
            continue
        if id(x) in seen:
            continue
        seen.add(id(x))
        stack.append((x, True))
        for a in reversed(x.args):
            if id(a) not in seen:
                stack.append((a, False))
    return out


def _ancestors(yield_node: Node):
    return _ancestors_of(yield_node)
