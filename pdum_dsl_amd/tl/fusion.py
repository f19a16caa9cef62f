"""The fusion registry rows this backend serves, and the plan they produce.

Restates the reference's packages/tensorlib/src/pdum/tl/fusion.py for the
template rows on the HIP hot path:

  flash               contraction -> closed mask -> row softmax -> contraction
                      over the same dim (fusion.py:480-615); the generator
                      emits the online-softmax fold; certified licensed-
                      differential under flash.online-softmax with the
                      template's own adversarial families (fusion.py:618-656),
                      on a twin shrunk to extent <= 128 (fusion.py:693-759);
                      with a machine, the mask-derived prune (fusion.py:659-690)
  row-normalization   the softmax chain over a param: rows staged once,
                      proved-exact by stage erasure (fusion.py:371-400, 818-825)
  contraction-epilogue  one sum over a two-operand product (or of one
                      operand), prologue / epilogue pointwise chains around
                      it (fusion.py:159-324); the generator emits the k-tiled
                      accumulation fold, certified proved-licensed under
                      gemm.k-reassoc (the fold inlines back to one sum)
  row-statistics      the two-pass layernorm core + scale/shift epilogue
                      (fusion.py:403-443, 826-843)
  map-chain           a pointwise chain over params, consts and iotas
                      (fusion.py:844-854); proved-exact

Everything else is a RED "uncompiled" group with the reason — never an
exception (fusion.py:855-868). Plans are data.
"""

from __future__ import annotations

from dataclasses import dataclass, field, replace

import numpy as np

from .analysis import defanalysis
from .certify import Certificate, certify
from .dialect import OPS, check_tier
from .interp import Field
from .ir import F64, Builder, Dim, Region, TensorType, minus_dim, walk
from .licenses import FLASH_ONLINE_SOFTMAX, GEMM_K_REASSOC
from .launch import fit_affine, propose, tri_eval

_MAP_OPS = frozenset(
    {"core.param", "core.const", "core.yield", "tl.pointwise", "tl.iota", "tl.const", "tl.select", "tl.split",
     "tl.repeat", "tl.repeat_like", "tl.rename", "tl.shift", "tl.slice", "tl.window", "tl.decimate", "tl.diagonal"}
)  # the affine views read in place (tl.stencil's fill needs a guarded read: it stays red)
_EXACT_OPS = frozenset({"tl.pointwise", "tl.repeat_like", "tl.rename", "tl.repeat", "tl.iota", "core.const",
                        "tl.const"})


@dataclass(frozen=True)
class Group:
    """One fusion group (fusion.py:127-141): the claiming template, the
    generated tile kernel, its certificate, the confidence color, plan
    parameters, the refusal reason, launch, prune and surfaced artifacts."""

    template: str
    kernel: Region | None = field(repr=False)
    certificate: Certificate | None
    confidence: str
    params: tuple = ()
    reason: str = ""
    launch: tuple = ()
    prune: tuple = ()
    artifacts: tuple = ()


@dataclass(frozen=True)
class Plan:
    groups: tuple


def _dims_of(n) -> tuple:
    d = n.attr("dims")
    return (d,) if isinstance(d, str) else tuple(d)


def pick_ki(extent: int) -> int:
    """The v1 tile width: the largest divisor <= min(32, extent/2), else extent (fusion.py:259-265)."""
    for ki in range(min(32, extent // 2), 0, -1):
        if extent % ki == 0:
            return ki
    return extent


# ------------------------------------------------------------ matchers


def match_softmax(pr):
    """div(exp(sm - rl(max_s sm)), rl(sum_s exp(...))) over one dim -> {sm, s, max, den}."""
    if pr.op != "tl.pointwise" or pr.attr("f") != "div" or len(pr.args) != 2:
        return None
    e, rld = pr.args
    if e.op != "tl.pointwise" or e.attr("f") != "exp" or rld.op != "tl.repeat_like":
        return None
    sume = rld.args[0]
    if sume.op != "tl.reduce" or sume.attr("f") != "sum" or sume.args[0] is not e:
        return None
    sub = e.args[0]
    if sub.op != "tl.pointwise" or sub.attr("f") != "sub" or len(sub.args) != 2:
        return None
    sm, rlm = sub.args
    if rlm.op != "tl.repeat_like":
        return None
    mx = rlm.args[0]
    if mx.op != "tl.reduce" or mx.attr("f") != "max" or mx.args[0] is not sm:
        return None
    if rlm.args[1] is not sm or rld.args[1] not in (sm, e):
        return None
    sd, md = _dims_of(sume), _dims_of(mx)
    if sd != md or len(sd) != 1:
        return None
    return {"sm": sm, "s": sd[0], "max": mx, "den": sume}


def match_rowstat(pr):
    """div(xc, rl(sqrt(mean(xc*xc) + eps))) with xc = x - rl(mean x), one feat dim -> {x, feat, eps, node}."""
    if pr.op != "tl.pointwise" or pr.attr("f") != "div" or len(pr.args) != 2:
        return None
    xc, rld = pr.args
    if rld.op != "tl.repeat_like":
        return None
    sd = rld.args[0]
    if sd.op != "tl.pointwise" or sd.attr("f") != "sqrt":
        return None
    add = sd.args[0]
    if add.op != "tl.pointwise" or add.attr("f") != "add" or len(add.args) != 2:
        return None
    var, eps = add.args
    if eps.op not in ("core.const", "tl.const") or var.op != "tl.reduce" or var.attr("f") != "mean":
        return None
    sq = var.args[0]
    if sq.op != "tl.pointwise" or sq.attr("f") != "mul" or sq.args[0] is not sq.args[1] or sq.args[0] is not xc:
        return None
    if xc.op != "tl.pointwise" or xc.attr("f") != "sub" or len(xc.args) != 2:
        return None
    x, rlm = xc.args
    if rlm.op != "tl.repeat_like":
        return None
    mu = rlm.args[0]
    if mu.op != "tl.reduce" or mu.attr("f") != "mean" or mu.args[0] is not x:
        return None
    vd, md = _dims_of(var), _dims_of(mu)
    if vd != md or len(vd) != 1:
        return None
    return {"x": x, "feat": vd[0], "eps": float(eps.attr("value")), "node": pr}


def contract_core(red, kname=None):
    """reduce(sum, mul(rl(x, y), rl(y, x)), (dim,)) -> (x, y, dim)."""
    if red.op != "tl.reduce" or red.attr("f") != "sum":
        return None
    dims = _dims_of(red)
    if len(dims) != 1 or (kname is not None and dims[0] != kname):
        return None
    prod = red.args[0]
    if prod.op != "tl.pointwise" or prod.attr("f") != "mul" or len(prod.args) != 2:
        return None
    ra, rb = prod.args
    if ra.op != "tl.repeat_like" or rb.op != "tl.repeat_like":
        return None
    x, y = ra.args[0], rb.args[0]
    if rb.args[1] is not x or ra.args[1] is not y:
        return None
    return x, y, dims[0]


def forest_is_closed(n) -> bool:
    """A mask forest is CLOSED when it reads no data: pointwise/consts over iota leaves."""
    if n.op in ("tl.iota", "core.const", "tl.const"):
        return True
    if n.op in _MAP_OPS and n.op != "core.param":
        return all(forest_is_closed(x) for x in n.args)
    return False


def _flashsm_core(y):
    """reduce(zoo.flashsm, (repeat_like(sm, v), repeat_like(v, sm)), s): the
    masked scores fed to the online-softmax reducer (zoo/attention.py:180-186)
    -> (sm, v, s); the same denotation as the softmax composition."""
    from .reducers import is_composite, lookup
    from .zoo import flashsm

    if y.op != "tl.reduce" or not is_composite(y.attr("f")) or lookup(y.attr("f")) is not flashsm:
        return None
    dims = y.attr("dims")
    dims = (dims,) if isinstance(dims, str) else tuple(dims)
    se, ve = y.args
    if len(dims) != 1 or se.op != "tl.repeat_like" or ve.op != "tl.repeat_like":
        return None
    sm, v = se.args[0], ve.args[0]
    if se.args[1] is not v or ve.args[1] is not sm:
        return None
    return sm, v, dims[0]


def match_flash(region: Region):
    """The flash composition over bare params q:(t,e), k:(s,e), v:(s,o), with
    an optional artifact yield (out, max, den) (fusion.py:480-539). The
    masked scores may also reach v through the flashsm composite reducer:
    the same program by its denotation, so the same row serves it."""
    y = region.body[-1].args[0]
    artifacts = False
    if y.op == "core.tuple":
        if len(y.args) != 3:
            return None
        y, m_out, den_out = y.args
        artifacts = True
    fsm = None if artifacts else _flashsm_core(y)
    if fsm is not None:
        smn, v, s = fsm
        if v.op != "core.param":
            return None
    else:
        out = contract_core(y)
        if out is None:
            return None
        pr, v, s = out
        sm_m = match_softmax(pr)
        if sm_m is None or sm_m["s"] != s:
            return None
        if artifacts and (m_out is not sm_m["max"] or den_out is not sm_m["den"]):
            return None
        if v.op != "core.param":
            return None
        smn = sm_m["sm"]
    if smn.op != "tl.pointwise" or smn.attr("f") != "where" or len(smn.args) != 3:
        return None
    mask, sc, fill = smn.args
    if fill.op not in ("core.const", "tl.const") or not forest_is_closed(mask):
        return None
    core = contract_core(sc)
    if core is None:
        return None
    q, k, e = core
    if q.op != "core.param" or k.op != "core.param":
        return None
    if {id(q), id(k), id(v)} != {id(p) for p in region.params}:
        return None
    qd, kd, vd = (p.type.names for p in (q, k, v))
    if len(qd) != 2 or kd != (s, e) or len(vd) != 2 or vd[0] != s:
        return None
    sdim = k.type.dim(s)
    if sdim.start != 0:
        return None
    return {
        "q": q, "k": k, "v": v, "mask": mask, "fill": float(fill.attr("value")),
        "t": next(nm for nm in qd if nm != e), "s": s, "e": e, "o": vd[1], "extent": sdim.stop,
        "artifacts": artifacts,
    }


# -------------------------------------------------- contraction-epilogue


def _uncore(x):
    """A contraction operand's core: broadcasts peeled (fusion.py:98-122)."""
    while x.op in ("tl.repeat_like", "tl.repeat"):
        x = x.args[0]
    return x


def _cone(n) -> set:
    out, stack = set(), list(n.args)
    while stack:
        x = stack.pop()
        if id(x) in out:
            continue
        out.add(id(x))
        stack.extend(x.args)
    return out


def match_contraction_epilogue(region: Region):
    """The contraction row (fusion.py:158-254): exactly one OUTER reduce —
    sum or mean over one or two dims of a two-operand product whose operands
    both carry the contracted dims (or of a single operand, the plain shape)
    — and every other node drawn from the recompute-exact vocabulary.
    Operands may be computed chains; a broadcast pair is the GEMM shape,
    same-space operands the ROWSUM shape. Anything else declines."""
    y = region.body[-1].args[0]
    if y.op == "core.tuple":
        return None
    reduces = [n for n in walk(region) if n.op == "tl.reduce"]
    red = None
    if len(reduces) == 1:
        red = reduces[0]
    else:  # tile-local reduces may live in operand prologues: the outer one's cone holds the rest
        for r in reduces:
            cone = _cone(r)
            if all(o is r or id(o) in cone for o in reduces):
                red = r
                break
    if red is None:
        return None
    f = red.attr("f")
    dims = _dims_of(red)
    if f not in ("sum", "mean") or len(dims) not in (1, 2):
        return None
    for r in reduces:  # a prologue reduce must be tile-local: disjoint from the swept dims
        if r is not red and set(_dims_of(r)) & set(dims):
            return None
    prod = red.args[0]
    if prod.op == "tl.pointwise" and prod.attr("f") == "mul" and len(prod.args) == 2:
        cores = [_uncore(x) for x in prod.args]
    else:  # PLAIN: a sum with no product (bias gradients)
        cores = [prod]
    if any(not c.type.has(k) for c in cores for k in dims if isinstance(c.type, TensorType)):
        return None
    if any(not isinstance(c.type, TensorType) for c in cores):
        return None
    keeps = [tuple(nm for nm in c.type.names if nm not in dims) for c in cores]
    out = red.type.names
    if set(out) != set().union(*map(set, keeps)):
        return None
    ca = cores[0]
    cb = cores[1] if len(cores) == 2 else None
    if cb is None:
        shape = "plain"
    else:
        shape = "rowsum" if ca.type.names == cb.type.names else "gemm"
    core = {id(red), id(prod)} | {id(r) for r in reduces}
    for n in walk(region):  # the whole region is exact vocabulary, or decline
        if id(n) in core or n.op in ("core.yield", "core.param"):
            continue
        if n.op not in _EXACT_OPS:
            return None
    total = 1
    for k in dims:
        kd = ca.type.dim(k)
        kb = kd if cb is None else cb.type.dim(k)
        if (kd.start, kd.stop) != (kb.start, kb.stop) or kd.start != 0:
            return None
        total *= kd.stop
    if any(d.start != 0 for d in red.type.dims):
        return None
    # the fold runs over the WIDEST contracted dim; the rest reduce inside the step whole
    k = max(dims, key=lambda nm: ca.type.dim(nm).stop)
    return {
        "reduce": red, "k": k, "extent": ca.type.dim(k).stop, "rest": tuple(nm for nm in dims if nm != k),
        "total": total, "a": ca, "b": cb, "shape": shape, "f": f,
    }


def generate_contraction(region: Region, m: dict, ki: int) -> Region:
    """The fused tile kernel (fusion.py:268-324): split k into (ko, ki), fold
    over ko with staged operand slices, the epilogue rebuilt over the
    accumulator; prologue chains rebuild ahead of the split."""
    k, extent, red = m["k"], m["extent"], m["reduce"]
    ko = extent // ki
    b = Builder(OPS)
    newp = {id(p): b.param(i, p.type) for i, p in enumerate(region.params)}
    memo: dict = dict(newp)
    shape = m["shape"]
    at = b.emit("tl.split", rebuild_into(b, memo, m["a"]), name=k, parts=(("ko", ko), ("ki", ki)))
    bt = None
    if shape != "plain":
        bt = b.emit("tl.split", rebuild_into(b, memo, m["b"]), name=k, parts=(("ko", ko), ("ki", ki)))
    acc0 = b.emit("tl.const", value=0.0, dims=tuple((d.name, d.stop) for d in red.type.dims))

    sb = Builder(OPS)
    p_acc = sb.param(0, acc0.type)
    p_a = sb.param(1, minus_dim(at.type, "ko"))
    a_s = sb.emit("tl.stage", p_a, level="shared")
    if shape == "plain":
        prod, params = a_s, (p_acc, p_a)
    else:
        p_b = sb.param(2, minus_dim(bt.type, "ko"))
        b_s = sb.emit("tl.stage", p_b, level="shared")
        params = (p_acc, p_a, p_b)
        if shape == "rowsum":
            prod = sb.emit("tl.pointwise", a_s, b_s, f="mul")
        else:
            prod = sb.emit("tl.pointwise", sb.emit("tl.repeat_like", a_s, b_s), sb.emit("tl.repeat_like", b_s, a_s),
                           f="mul")
    part = sb.emit("tl.reduce", prod, dims=("ki", *m["rest"]), f="sum")
    nxt = sb.emit("tl.pointwise", p_acc, part, f="add")
    step = Region(params=params, body=(sb.emit("core.yield", nxt),))
    srcs = (at,) if shape == "plain" else (at, bt)
    names = ("a",) if shape == "plain" else ("a", "b")
    fold = b.emit("tl.fold", acc0, *srcs, regions=(step,), dim="ko", state=("acc",), element=names, out=("final", 0))
    memo[id(red)] = fold
    if m["f"] == "mean":  # the divide-by-N finalize: N static, one scalar op
        memo[id(red)] = b.emit("tl.pointwise", fold, b.emit("core.const", type=F64, value=1.0 / m["total"]), f="mul")
    y = rebuild_into(b, memo, region.body[-1].args[0])
    fused = Region(params=tuple(newp[id(p)] for p in region.params), body=(b.emit("core.yield", y),))
    return check_tier(fused)


# pointwise markers defined on part of the line only: a param that reaches
# one of their arguments is drawn inside the domain
_HALF_LINE = frozenset(("sqrt", "log"))


def domain_restricted_params(region: Region) -> frozenset:
    """Positions of the params whose values flow (through any path) into the
    argument of a sqrt or log of ``region``."""
    pos = {id(p): i for i, p in enumerate(region.params)}
    reach: dict[int, frozenset] = {}
    hit: set[int] = set()
    for n in walk(region):
        acc = {pos[id(n)]} if id(n) in pos else set()
        for a in n.args:
            acc |= reach.get(id(a), frozenset())
        reach[id(n)] = frozenset(acc)
        if n.op == "tl.pointwise" and n.attr("f") in _HALF_LINE:
            for a in n.args:
                hit |= reach.get(id(a), frozenset())
    return frozenset(hit)


def contraction_families(region: Region, seed: int = 5):
    """Adversarial draws for a contraction's differential tier (used when
    normalization cannot walk back, e.g. a mean's finalize): unit-normal and
    wide-magnitude operands, drawn inside the operators' domains (the
    "finite operands" domain gemm.k-reassoc declares):

    * every param is drawn signed first, so sign cancellations (the cases
      that stress k-reassociation) are drawn wherever the domain allows;
    * the wide family starts at x64 and is narrowed by factors of 8 until the
      naive twin evaluates without overflow or an invalid operation (an exp
      of a wide product saturates long before x64), never below x1;
    * only when the signed draw still leaves the domain at x1 (the naive
      twin raises or returns a non-finite value) are the params that reach a
      sqrt or log drawn positive, (|z| + 1/2) scaled, and narrowed the same way.

    A draw that still leaves the domain is refused by ``certify``."""
    from .interp import field, run_region

    restricted = domain_restricted_params(region)

    def values(scale, s, positive):
        rng = np.random.default_rng(s)
        vals = []
        for i, p in enumerate(region.params):
            z = rng.standard_normal(p.type.shape)
            vals.append(field(((np.abs(z) + 0.5) if i in positive else z) * scale, p.type.names))
        return vals

    def inside(vals):
        try:
            with np.errstate(over="raise", invalid="raise", divide="raise"):
                out = run_region(region, vals)
        except FloatingPointError:
            return False
        outs = out if isinstance(out, (tuple, list)) else (out,)
        return all(np.isfinite(np.asarray(getattr(o, "arr", o), dtype=np.float64)).all() for o in outs)

    def draw(scale, s):
        def factory():
            vals = None
            for positive in (frozenset(), restricted) if restricted else (frozenset(),):
                sc = scale
                while True:
                    vals = values(sc, s, positive)
                    if inside(vals):
                        return vals
                    if sc <= 1.0:
                        break
                    sc = max(1.0, sc / 8.0)
            return vals

        return factory

    return (("unit", draw(1.0, seed)), ("wide", draw(64.0, seed + 1)))


# ----------------------------------------------------------- generators


def rebuild_into(b: Builder, memo: dict, n):
    """Re-emit ``n`` with a seeded memo (params, holes)."""
    if id(n) in memo:
        return memo[id(n)]
    args = tuple(rebuild_into(b, memo, x) for x in n.args)
    explicit = {} if OPS[n.op].type_rule is not None else {"type": n.type}
    out = b.emit(n.op, *args, regions=n.regions, loc=n.loc, **explicit, **dict(n.attrs))
    memo[id(n)] = out
    return out


def stage_params(region: Region, staged_ids) -> Region:
    """The same chain with the named params staged once to "shared" (fusion.py:339-350)."""
    b = Builder(OPS)
    newp = {id(p): b.param(i, p.type) for i, p in enumerate(region.params)}
    memo: dict = dict(newp)
    for pid in staged_ids:
        memo[pid] = b.emit("tl.stage", newp[pid], level="shared")
    y = rebuild_into(b, memo, region.body[-1].args[0])
    return check_tier(Region(params=tuple(newp[id(p)] for p in region.params), body=(b.emit("core.yield", y),)))


def flash_step(types: tuple, e: str, fill: float) -> Region:
    """The online-softmax step over (m, den, o | q, k-tile, v-tile, mask-tile):
        sc = sum_e q k; sm = where(mask, sc, fill); m' = max(m, max_si sm)
        a = exp(m - m'); p = exp(sm - m'); den' = den a + sum_si p
        o' = o a + sum_si p v
    (fusion.py:570-604). Shared by the generator and the HIP recognizer, so
    a tile kernel is recognized exactly when its step has this content key."""
    sb = Builder(OPS)
    p_m, p_den, p_o, p_q, p_k, p_v, p_mk = (sb.param(i, t) for i, t in enumerate(types))
    ks = sb.emit("tl.stage", p_k, level="shared")
    vs = sb.emit("tl.stage", p_v, level="shared")
    prod = sb.emit("tl.pointwise", sb.emit("tl.repeat_like", p_q, ks), sb.emit("tl.repeat_like", ks, p_q), f="mul")
    sc = sb.emit("tl.reduce", prod, dims=(e,), f="sum")
    sm = sb.emit("tl.pointwise", p_mk, sc, sb.emit("core.const", type=F64, value=float(fill)), f="where")
    m_new = sb.emit("tl.pointwise", p_m, sb.emit("tl.reduce", sm, dims=("si",), f="max"), f="maximum")
    alpha = sb.emit("tl.pointwise", sb.emit("tl.pointwise", p_m, m_new, f="sub"), f="exp")
    p_w = sb.emit("tl.pointwise", sb.emit("tl.pointwise", sm, sb.emit("tl.repeat_like", m_new, sm), f="sub"), f="exp")
    den_new = sb.emit(
        "tl.pointwise", sb.emit("tl.pointwise", p_den, alpha, f="mul"), sb.emit("tl.reduce", p_w, dims=("si",), f="sum"),
        f="add",
    )
    pv = sb.emit("tl.pointwise", sb.emit("tl.repeat_like", p_w, vs), sb.emit("tl.repeat_like", vs, p_w), f="mul")
    o_new = sb.emit(
        "tl.pointwise",
        sb.emit("tl.pointwise", p_o, sb.emit("tl.repeat_like", alpha, p_o), f="mul"),
        sb.emit("tl.reduce", pv, dims=("si",), f="sum"),
        f="add",
    )
    return Region(
        params=(p_m, p_den, p_o, p_q, p_k, p_v, p_mk),
        body=(sb.emit("core.yield", sb.emit("core.tuple", m_new, den_new, o_new)),),
    )


FOLD_KW = dict(dim="so", state=("m", "den", "o"), element=("q", "k", "v", "mask"))


def generate_flash(region: Region, m: dict, si: int) -> Region:
    """The online-softmax tile region (fusion.py:542-615): the mask forest
    re-rooted on a const (t, s) lattice and split along s as an element
    source, K/V split (so, si), q as a stride-0 repeat over so, two (three
    with artifacts) fold nodes sharing one step for the finals."""
    s, t, fill = m["s"], m["t"], m["fill"]
    so = m["extent"] // si
    tdim = m["q"].type.dim(t)
    odim = m["v"].type.dim(m["o"])
    b = Builder(OPS)
    newp = {id(p): b.param(i, p.type) for i, p in enumerate(region.params)}
    nq, nk, nv = newp[id(m["q"])], newp[id(m["k"])], newp[id(m["v"])]
    lattice = b.emit("tl.const", value=0.0, dims=((t, tdim.stop), (s, m["extent"])))
    memo: dict = dict(newp)
    for n in walk(region):  # iota backings re-root on the lattice: values were never read
        if n.op == "tl.iota":
            memo[id(n)] = b.emit("tl.iota", lattice, name=n.attr("name"))
    mask = rebuild_into(b, memo, m["mask"])
    parts = (("so", so), ("si", si))
    kt = b.emit("tl.split", nk, name=s, parts=parts)
    vt = b.emit("tl.split", nv, name=s, parts=parts)
    mt = b.emit("tl.split", mask, name=s, parts=parts)
    qr = b.emit("tl.repeat", nq, name="so", extent=so)
    m0 = b.emit("tl.const", value=-1e30, dims=((t, tdim.stop),))
    den0 = b.emit("tl.const", value=0.0, dims=((t, tdim.stop),))
    o0 = b.emit("tl.const", value=0.0, dims=((t, tdim.stop), (m["o"], odim.stop)))
    types = (m0.type, den0.type, o0.type, minus_dim(qr.type, "so"), minus_dim(kt.type, "so"),
             minus_dim(vt.type, "so"), minus_dim(mt.type, "so"))
    step = flash_step(types, m["e"], fill)
    args = (m0, den0, o0, qr, kt, vt, mt)
    f_o = b.emit("tl.fold", *args, regions=(step,), out=("final", 2), **FOLD_KW)
    f_den = b.emit("tl.fold", *args, regions=(step,), out=("final", 1), **FOLD_KW)
    out = b.emit("tl.pointwise", f_o, b.emit("tl.repeat_like", f_den, f_o), f="div")
    if m.get("artifacts"):
        f_m = b.emit("tl.fold", *args, regions=(step,), out=("final", 0), **FOLD_KW)
        out = b.emit("core.tuple", out, f_m, f_den)
    fused = Region(params=tuple(newp[id(p)] for p in region.params), body=(b.emit("core.yield", out),))
    return check_tier(fused)


# ------------------------------------------------------- certification


def score_families(region: Region, seed: int = 11):
    """Adversarial families (fusion.py:618-656): unit gaussians, wide scores
    (x8), and a dominant key (row 0 of param 1 x40). Params consumed as
    where-conditions draw as boolean masks."""
    masks = set()
    for n in walk(region):
        if n.op == "tl.pointwise" and n.attr("f", "").startswith("where"):
            r = n.args[0]
            while r.op in ("tl.repeat_like", "tl.repeat", "tl.select"):
                r = r.args[0]
            if r.op == "core.param":
                masks.add(id(r))

    def draw(scale, subseed, spike=False):
        def factory():
            rng = np.random.default_rng(subseed)
            out = []
            for i, p in enumerate(region.params):
                shape = p.type.shape
                if id(p) in masks:
                    out.append(Field(rng.random(shape) < 0.5, p.type.dims))
                    continue
                arr = scale * rng.standard_normal(shape)
                if spike and i == 1:
                    arr[0] *= 40.0
                out.append(Field(arr, p.type.dims))
            return out

        return factory

    return (
        ("gaussian", draw(1.0, seed)),
        ("wide-scores", draw(8.0, seed + 1)),
        ("dominant-key", draw(1.0, seed + 2, spike=True)),
    )


CERT_CAP = 128


@defanalysis("fusion.certify", 1)
def _certify_analysis(tile: Region, naive: Region, *, kind: str) -> Certificate:
    if kind == "flash":
        return certify(tile, naive, licenses=FLASH_ONLINE_SOFTMAX, families=score_families(naive))
    if kind == "contraction":
        return certify(tile, naive, licenses=GEMM_K_REASSOC, families=contraction_families(naive))
    return certify(tile, naive)


def _cert_fact(tile: Region, naive: Region, kind: str) -> Certificate:
    """Certification as a cached fact keyed by both regions' content
    (the reference caches it the same way, fusion.py:696-715): a warm
    re-plan certifies nothing."""
    return _certify_analysis(tile, naive, kind=kind).value


def shrink(region: Region, cap: int) -> Region | None:
    """The same program over extents clamped to ``cap`` (fusion.py:718-755)."""
    if any(d.start != 0 for p in region.params for d in p.type.dims):
        return None
    b = Builder(OPS)
    memo: dict = {}
    for i, p in enumerate(region.params):
        memo[id(p)] = b.param(i, TensorType(tuple(Dim(d.name, 0, min(d.stop, cap)) for d in p.type.dims)))

    def clamp(e):
        return (e[0], min(int(e[1]), cap)) if isinstance(e, tuple) else min(int(e), cap)

    def rebuild(n):
        if id(n) in memo:
            return memo[id(n)]
        args = tuple(rebuild(x) for x in n.args)
        at = dict(n.attrs)
        if n.op == "tl.const" and "dims" in at:
            at["dims"] = tuple((nm, clamp(e)) for nm, e in at["dims"])
        if n.op == "tl.repeat" and "extent" in at:
            at["extent"] = clamp(at["extent"])
        explicit = {} if OPS[n.op].type_rule is not None else {"type": n.type}
        out = b.emit(n.op, *args, regions=n.regions, loc=n.loc, **explicit, **at)
        memo[id(n)] = out
        return out

    y = rebuild(region.body[-1].args[0])
    return Region(params=tuple(memo[id(p)] for p in region.params), body=(b.emit("core.yield", y),))


def oversized(region: Region, cap: int) -> bool:
    return any(d.size > cap for p in region.params for d in p.type.dims)


def prune_flash(region: Region, *, tile: int, si: int):
    """Mask-derived fold bounds (fusion.py:659-690): per t-program [lo, hi)
    over s-tiles, as exact floor-affine fits, or None when any program or
    row is fully masked (uniform-softmax semantics)."""
    fm = match_flash(region)
    if fm is None:
        return None
    t, s, mask, S = fm["t"], fm["s"], fm["mask"], fm["extent"]
    so = S // si
    td = fm["q"].type.dim(t)
    sbox = [(q * si, (q + 1) * si - 1) for q in range(so)]
    los, his = [], []
    for g in range(-((td.start - td.stop) // tile)):
        tb = (td.start + g * tile, min(td.start + (g + 1) * tile, td.stop) - 1)
        act = [q for q in range(so) if tri_eval(mask, {t: tb, s: sbox[q]})[1] != "F"]
        if not act:
            return None
        los.append(act[0])
        his.append(act[-1] + 1)
    for r in range(td.start, td.stop):
        if all(tri_eval(mask, {t: (r, r), s: sb})[1] == "F" for sb in sbox):
            return None
    flo, fhi = fit_affine(los, 0, so), fit_affine(his, 0, so)
    return (flo, fhi) if flo is not None and fhi is not None else None


# ----------------------------------------------------------------- plan


def plan_region(region: Region, machine=None, floor: int = 1024) -> Plan:
    """Recognize the whole region against the registry, certify, and (with a
    machine) attach the analytic default launch and the flash prune
    (fusion.py:762-785)."""
    plan = _recognize(region)
    if machine is None:
        return plan
    groups = []
    for g in plan.groups:
        cands = propose(g.kernel, machine, floor) if g.kernel is not None else ()
        if cands:
            g = replace(g, launch=cands[0])
        if g.template == "flash" and len(g.launch) == 1:
            pr = prune_flash(region, tile=g.launch[0][1], si=dict(g.params)["si"])
            if pr is not None:
                g = replace(g, prune=(("so", *pr),))
        groups.append(g)
    return Plan(tuple(groups))


def _layout_root(n):
    """The value under a chain of layout views (fusion.py:353-356)."""
    while n.op in ("tl.shift", "tl.slice", "tl.stage", "tl.rename"):
        n = n.args[0]
    return n


def neighborhood_params(region: Region) -> frozenset:
    """The stencil signal (fusion.py:359-368): params read at two or more
    DISTINCT shifts have overlapping neighborhoods, so staging their halo
    once pays."""
    shifts: dict = {}
    for n in walk(region):
        if n.op == "tl.shift":
            root = _layout_root(n.args[0])
            if root.op == "core.param":
                shifts.setdefault(id(root), set()).add(n.attrs)
    return frozenset(pid for pid, deltas in shifts.items() if len(deltas) >= 2)


def _is_map_chain(region: Region):
    for n in walk(region):
        if n.op not in _MAP_OPS:
            return n.op
    return None


def _recognize(region: Region) -> Plan:
    fm = match_flash(region)
    if fm is not None:
        si = pick_ki(fm["extent"])
        kernel = generate_flash(region, fm, si)
        csrc, ckern = region, kernel
        if oversized(region, CERT_CAP):  # certify the shrunk twin: the program, not the size
            shr = shrink(region, CERT_CAP)
            fm2 = match_flash(shr) if shr is not None else None
            if fm2 is not None:
                csrc, ckern = shr, generate_flash(shr, fm2, pick_ki(fm2["extent"]))
        cert = _cert_fact(ckern, csrc, "flash")
        arts = ("m", "den") if fm["artifacts"] else ()
        return Plan((Group("flash", kernel, cert, "yellow", params=(("si", si),), artifacts=arts),))
    cm = match_contraction_epilogue(region)
    if cm is not None:
        ki = pick_ki(cm["extent"])
        kernel = generate_contraction(region, cm, ki)
        csrc, ckern = region, kernel
        if oversized(region, CERT_CAP):  # certify the shrunk twin: the program, not the size
            shr = shrink(region, CERT_CAP)
            cm2 = match_contraction_epilogue(shr) if shr is not None else None
            if cm2 is not None:
                csrc, ckern = shr, generate_contraction(shr, cm2, pick_ki(cm2["extent"]))
        cert = _cert_fact(ckern, csrc, "contraction")
        return Plan((Group("contraction-epilogue", kernel, cert, "yellow", params=(("ki", ki), ("shape", cm["shape"]))),))
    sm = match_softmax(region.body[-1].args[0])
    if sm is not None:
        rows = frozenset(id(p) for p in region.params if p.type.has(sm["s"]))
        kernel = stage_params(region, rows)
        return Plan((Group("row-normalization", kernel, _cert_fact(kernel, region, "exact"), "yellow"),))
    rs = next((m for n in walk(region) if (m := match_rowstat(n)) is not None), None)
    if rs is not None:
        reduces = [n for n in walk(region) if n.op == "tl.reduce"]
        feat_ok = all(r.attr("f") == "mean" and _dims_of(r) == (rs["feat"],) for r in reduces)
        vocab_ok = all(n.op in _EXACT_OPS or n.op in ("core.yield", "core.param", "tl.reduce") for n in walk(region))
        if len(reduces) == 2 and feat_ok and vocab_ok:
            rows = frozenset(id(p) for p in region.params if p.type.has(rs["feat"]))
            kernel = stage_params(region, rows)
            return Plan((Group("row-statistics", kernel, _cert_fact(kernel, region, "exact"), "yellow"),))
    offender = _is_map_chain(region)
    if offender is None:
        halos = neighborhood_params(region)
        if halos:  # the stencil row (fusion.py:846-851): halos staged once, exact by erasure
            kernel = stage_params(region, halos)
            idxs = tuple(i for i, p in enumerate(region.params) if id(p) in halos)
            return Plan((Group("stencil", kernel, _cert_fact(kernel, region, "exact"), "yellow",
                               params=(("staged", idxs),)),))
        kernel = check_tier(region)
        return Plan((Group("map-chain", kernel, _cert_fact(kernel, region, "exact"), "yellow"),))
    return Plan(
        (
            Group(
                "uncompiled", None, None, "red",
                reason=f"no recognized schedule: {offender} has no template row — the reference serves this group",
            ),
        )
    )
