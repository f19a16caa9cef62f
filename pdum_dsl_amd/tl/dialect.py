"""The tl op family this backend reads, with the alignment law as type rules.

Restates the subset of the reference's tl dialect that the fusion templates
emit and consume (packages/tensorlib/src/pdum/tl/dialect.py:115-487):

  core.param / core.const / core.tuple / core.yield
  tl.pointwise  f=<marker>      operands aligned BY NAME; scalars broadcast
  tl.reduce     f, dims         sum | max | min | prod | mean (mean = sum / N)
  tl.scan       f, dim[, reverse]  inclusive prefix reduce along one dim (the
                                dim keeps its domain); reverse folds suffixes
  tl.repeat_like x, like        adds like's missing dims (stride-0 broadcast)
  tl.repeat     name, extent    adds one stride-0 dim
  tl.split      name, parts     x -> (outer .. inner) blocking, x = sum w_j i_j
  tl.stage      level[, order]  a copy to a residence level (identity in value)
  tl.select     coords          fixes dims to points
  tl.iota       name            the coordinate field along a dim of the lattice
  tl.const      value, dims     a constant field
  tl.fold       dim, state, element, out, step region; out ('final', i) is
                the last value of state i, ('emit',) stacks each step's extra
                (last) yield along the scan dim
  tl.rename     mapping         renames dims in place (a view: no data moves)
  tl.shift      deltas          moves dims' frames by integer deltas (a view)
  tl.slice      ranges          restricts dims to absolute [lo, hi) (a view)
  tl.pad        extents[, fill] widens dims' frames to [lo, hi), new cells = fill
                                (slice's adjoint)
  tl.flip       name            reverses one dim: out[c] = x[start + stop - 1 - c]
  tl.merge      parts, name     (outer .. inner) dims -> one dim at [0, N):
                                split's inverse (and adjoint)
  tl.take       dim             out = table[idx, rest]: a gather, no template row
  tl.scatter_add dim, extent[, over]  take's adjoint: out[v, rest] = sum of
                                values at the positions p with idx[p] == v
  tl.window     name, k_name, k[, dilation]  a tap dim after name:
                                out[x, j] = x[x + dilation j], name shrunk so
                                every tap stays inside its old domain
  tl.stencil    name, k[, k_name, fill, dilation]  the same taps over name's
                                whole domain (k an INCLUSIVE range), fill where
                                a tap leaves it
  tl.decimate   name, factor[, phase]  every factor-th cell (i = phase mod
                                factor), renumbered j = (i - phase) / factor
  tl.diagonal   parts, name     the cells where all parts agree, as one dim
                                over the intersection of their domains
  tl.round_to   encoding[, grad]  encode-then-decode to bf16 / f16 / f32,
                                round to nearest even (the one precision op)
  tl.reduce / tl.scan with a composite reducer (pdum_dsl_amd.tl.reducers):
                                m aligned element operands folded through
                                its lift / combine / project
  tl.argtopk    (typed only: a non-template op the planner must refuse)
"""

from __future__ import annotations

from .ir import F64, BOOL, Builder, Dim, OpDef, Region, Scalar, TensorType, TupleType, minus_dim, walk

MARKERS = (
    "add sub mul div neg exp log maximum minimum tanh sqrt sin cos abs floor "
    "where eq ne le lt ge gt stop_gradient zoo.gelu zoo.gelu.d0"
).split()
REDUCERS = ("sum", "max", "min", "prod", "mean")


def _dims_arg(v) -> tuple:
    return (v,) if isinstance(v, str) else tuple(v)


def _aligned(ts: list[TensorType]) -> None:
    ref = {d.name: d for d in ts[0].dims}
    for t in ts[1:]:
        other = {d.name: d for d in t.dims}
        if set(other) != set(ref):
            raise TypeError(f"tl.pointwise wants ALIGNED operands: dims {sorted(ref)} vs {sorted(other)}")
        for n, d in other.items():
            if (d.start, d.stop) != (ref[n].start, ref[n].stop):
                raise TypeError(
                    f"tl.pointwise wants ALIGNED operands: dim {n!r} domain "
                    f"[{ref[n].start}, {ref[n].stop}) vs [{d.start}, {d.stop})"
                )


def _r_pointwise(args, at, regions):
    if at["f"] not in MARKERS:
        raise TypeError(f"unknown pointwise marker {at['f']!r}")
    ts = [a for a in args if isinstance(a, TensorType)]
    if not ts:
        raise TypeError("tl.pointwise wants at least one tensor operand")
    _aligned(ts)
    return TensorType(ts[0].dims)


def _composite(args, at, dims) -> TensorType:
    """The element operands of a composite reduce / scan: as many as the
    reducer's element count, aligned, folded along exactly one dim
    (compute.py:216-240 in the reference)."""
    from .reducers import lookup

    f = lookup(at["f"])
    if len(args) != f.element:
        raise TypeError(f"{f.name} consumes {f.element} element operand(s), got {len(args)}")
    _aligned(list(args))
    if len(dims) != 1:
        raise TypeError(f"{f.name}: composite reducers fold one dim at a time")
    args[0].dim(dims[0])
    return args[0]


def _r_reduce(args, at, regions):
    dims = _dims_arg(at["dims"])
    if at["f"] not in REDUCERS:
        x = _composite(args, at, dims)
        return TensorType(tuple(d for d in x.dims if d.name not in dims))
    (x,) = args
    for d in dims:
        x.dim(d)
    return TensorType(tuple(d for d in x.dims if d.name not in dims))


def _r_scan(args, at, regions):
    """Inclusive prefix reduce along ONE dim (compute.py:318-350 in the
    reference): out[.., t, ..] folds x[.., start..t, ..]; a mean divides by the
    running count. ``reverse=True`` folds the suffix x[.., t..stop, ..] instead
    (the reference spells it flip . scan . flip)."""
    if not isinstance(at["dim"], str):
        raise TypeError("tl.scan folds exactly one dim (pass its name)")
    if at["f"] not in REDUCERS:
        if at.get("reverse"):
            raise TypeError("tl.scan: a composite reducer scans forward (flip the operands for a suffix scan)")
        return TensorType(_composite(args, at, (at["dim"],)).dims)
    (x,) = args
    x.dim(at["dim"])
    return TensorType(x.dims)


def _r_repeat_like(args, at, regions):
    x, like = args
    have = set(x.names)
    return TensorType(x.dims + tuple(d for d in like.dims if d.name not in have))


def _range(extent):
    return (int(extent[0]), int(extent[1])) if isinstance(extent, tuple) else (0, int(extent))


def _r_repeat(args, at, regions):
    (x,) = args
    if x.has(at["name"]):
        raise TypeError(f"dim {at['name']!r} already exists")
    lo, hi = _range(at["extent"])
    return TensorType(x.dims + (Dim(at["name"], lo, hi),))


def _r_split(args, at, regions):
    (x,) = args
    d = x.dim(at["name"])
    parts = tuple(at["parts"])
    n = 1
    for _, size in parts:
        n *= int(size)
    if n != d.size:
        raise TypeError(f"tl.split: parts {parts} do not tile dim {d.name!r} of size {d.size}")
    if d.start != 0:
        raise TypeError("tl.split: only dims starting at 0 split here")
    out = []
    for e in x.dims:
        if e.name == d.name:
            out.extend(Dim(pn, 0, int(ps)) for pn, ps in parts)
        else:
            if any(e.name == pn for pn, _ in parts):
                raise TypeError(f"part name {e.name!r} collides with an existing dim")
            out.append(e)
    return TensorType(tuple(out))


def _r_stage(args, at, regions):
    (x,) = args
    order = at.get("order")
    if order:
        return TensorType(tuple(x.dim(n) for n in order))
    return TensorType(x.dims)


def _r_select(args, at, regions):
    (x,) = args
    coords = dict(at["coords"])
    for n, i in coords.items():
        d = x.dim(n)
        if not d.start <= i < d.stop:
            raise TypeError(f"select {n}={i} outside [{d.start}, {d.stop})")
    return TensorType(tuple(d for d in x.dims if d.name not in coords))


def _r_iota(args, at, regions):
    (x,) = args
    if not isinstance(x, TensorType) or not x.has(at["name"]):
        raise TypeError(f"tl.iota: the lattice has no dim {at['name']!r}")
    return TensorType(x.dims)


def _r_const(args, at, regions):
    return TensorType(tuple(Dim(n, *_range(e)) for n, e in at["dims"]))


def _frames(t: TensorType):
    return sorted(((d.name, d.start, d.stop) for d in t.dims))


def _r_fold(args, at, regions):
    state, element = tuple(at["state"]), tuple(at["element"])
    k, m = len(state), len(element)
    if k < 1 or len(args) != k + m:
        raise TypeError(f"tl.fold takes {k} state init(s) + {m} element source(s), got {len(args)} operands")
    (step,) = regions
    dim = at["dim"]
    inits, srcs = args[:k], args[k:]
    for s in srcs:
        if not s.has(dim):
            raise TypeError(f"tl.fold: element source has no scan dim {dim!r}")
    want = tuple(inits) + tuple(minus_dim(s, dim) for s in srcs)
    binders = tuple(p.type for p in step.params)
    if len(binders) != len(want) or any(_frames(a) != _frames(b) for a, b in zip(binders, want)):
        raise TypeError("tl.fold: step binders do not match (state inits + element slices)")
    y = step.body[-1].args[0]
    ytypes = tuple(a.type for a in y.args) if y.op == "core.tuple" else (y.type,)
    out = tuple(at["out"])
    if out[0] not in ("final", "emit"):
        raise TypeError("tl.fold: out is ('final', i) or ('emit',)")
    emit = out[0] == "emit"
    if len(ytypes) != k + (1 if emit else 0):
        raise TypeError(f"tl.fold: the step must yield the {k} next state(s)" + (" and the emission" if emit else ""))
    for i in range(k):
        if _frames(ytypes[i]) != _frames(inits[i]):
            raise TypeError(f"tl.fold: carry {state[i]!r} changes the state type")
    if emit:  # every step's last yield, stacked along the scan dim (its frame from the element sources)
        d = srcs[0].dim(dim) if srcs else None
        if d is None:
            raise TypeError("tl.fold: an emitting fold needs an element source")
        if ytypes[k].has(dim):
            raise TypeError(f"tl.fold: the emission already has the scan dim {dim!r}")
        return TensorType(ytypes[k].dims + (Dim(dim, d.start, d.stop),))
    return inits[out[1]]


def _r_rename(args, at, regions):
    (x,) = args
    mapping = dict(at["mapping"])
    for old in mapping:
        x.dim(old)
    return TensorType(tuple(Dim(mapping.get(d.name, d.name), d.start, d.stop) for d in x.dims))


def _r_shift(args, at, regions):
    """Moves dims' frames: [start, stop) -> [start + d, stop + d); the value at
    new coordinate c is the input's at c - d (layout.py shift)."""
    (x,) = args
    deltas = dict(at["deltas"])
    for nm in deltas:
        x.dim(nm)
    return TensorType(tuple(Dim(d.name, d.start + int(deltas.get(d.name, 0)), d.stop + int(deltas.get(d.name, 0)))
                            for d in x.dims))


def _r_slice(args, at, regions):
    """Restricts dims to [lo, hi) in absolute coordinates, inside their domains."""
    (x,) = args
    ranges = dict(at["ranges"])
    out = []
    for d in x.dims:
        if d.name in ranges:
            lo, hi = (int(v) for v in ranges[d.name])
            if not d.start <= lo <= hi <= d.stop:
                raise TypeError(f"tl.slice {d.name}=[{lo}, {hi}) outside [{d.start}, {d.stop})")
            out.append(Dim(d.name, lo, hi))
        else:
            out.append(d)
    for nm in ranges:
        x.dim(nm)
    return TensorType(tuple(out))


def _r_pad(args, at, regions):
    """Widens dims' frames to absolute [lo, hi) containing their domains
    (layout.py pad): the new cells hold ``fill``."""
    (x,) = args
    ext = dict(at["extents"])
    for nm, (lo, hi) in ext.items():
        d = x.dim(nm)
        if not int(lo) <= d.start <= d.stop <= int(hi):
            raise TypeError(f"tl.pad {nm}=[{lo}, {hi}) does not contain [{d.start}, {d.stop})")
    return TensorType(tuple(Dim(d.name, *(int(v) for v in ext[d.name])) if d.name in ext else d for d in x.dims))


def _r_flip(args, at, regions):
    (x,) = args
    x.dim(at["name"])
    return TensorType(x.dims)


def _r_merge(args, at, regions):
    """Merges the dims ``parts`` (outer first, each starting at 0) into one
    dim ``name`` at [0, prod) placed where the first part is (layout.py merge)."""
    (x,) = args
    parts = _dims_arg(at["parts"])
    if len(parts) < 1 or len(set(parts)) != len(parts):
        raise TypeError(f"tl.merge parts {parts} must be distinct dims")
    size = 1
    for nm in parts:
        d = x.dim(nm)
        if d.start != 0:
            raise TypeError(f"tl.merge: part {nm!r} must start at 0")
        size *= d.size
    name = at["name"]
    if x.has(name) and name not in parts:
        raise TypeError(f"tl.merge: dim {name!r} already exists")
    out = []
    for d in x.dims:
        if d.name == parts[0]:
            out.append(Dim(name, 0, size))
        elif d.name not in parts:
            out.append(d)
    return TensorType(tuple(out))


def _r_take(args, at, regions):
    """out = table[idx, rest]: the taken dim is replaced IN PLACE by idx's dims
    (indexing.py:120-138); idx dims the table already carries must align."""
    table, idx = args
    d = table.dim(at["dim"])
    survivors = {x.name: x for x in table.dims if x.name != d.name}
    for n in idx.dims:
        if n.name in survivors and (survivors[n.name].start, survivors[n.name].stop) != (n.start, n.stop):
            raise TypeError(f"tl.take: idx dim {n.name!r} does not align with the table's")
    spliced = tuple(n for n in idx.dims if n.name not in survivors)
    out = []
    for x in table.dims:
        out.extend(spliced if x.name == d.name else (x,))
    return TensorType(tuple(out))


def _extent(v) -> tuple:
    """An extent attr: an int width (start 0) or a (start, stop) pair."""
    if isinstance(v, int):
        return 0, v
    lo, hi = (int(x) for x in v)
    return lo, hi


def _r_scatter_add(args, at, regions):
    """take's adjoint (indexing.py:153-190, 223-259): the idx dims named by
    ``over`` (default: all of them) are consumed, each a values dim with the
    same domain; the declared dim (domain ``extent``) takes the place of the
    first consumed dim; idx dims not consumed align and ride; the other
    values dims stay verbatim."""
    values, idx = args
    over = at.get("over")
    consumed = tuple(idx.names) if over is None else _dims_arg(over)
    for n in idx.dims:
        if not values.has(n.name):
            raise TypeError(f"tl.scatter_add: idx dim {n.name!r} is not a values dim")
        v = values.dim(n.name)
        if (v.start, v.stop) != (n.start, n.stop):
            raise TypeError(f"tl.scatter_add: idx dim {n.name!r} does not align with the values'")
    for nm in consumed:
        if nm not in idx.names:
            raise TypeError(f"tl.scatter_add: over={nm!r} is not an idx dim {idx.names}")
    if not consumed:
        raise TypeError("tl.scatter_add consumes at least one idx dim")
    lo, hi = _extent(at["extent"])
    if values.has(at["dim"]) and at["dim"] not in consumed:
        raise TypeError(f"tl.scatter_add: the declared dim {at['dim']!r} is already a values dim")
    out = []
    for x in values.dims:
        if x.name == consumed[0]:
            out.append(Dim(at["dim"], lo, hi))
        elif x.name not in consumed:
            out.append(x)
    return TensorType(tuple(out))


def _taps(k) -> tuple:
    """A window's half-open tap-index range: an int n is [0, n)."""
    if isinstance(k, int):
        return 0, int(k)
    lo, hi = (int(v) for v in k)
    return lo, hi


def _dilation(at) -> int:
    dil = at.get("dilation", 1)
    if not isinstance(dil, int) or dil < 1:
        raise TypeError(f"dilation must be a positive int, got {dil!r}")
    return dil


def _r_window(args, at, regions):
    """layout.py:700-740: the tap dim k_name (half-open tap range k) goes
    right after name, whose domain shrinks to the cells whose every tap
    x + dilation j lands inside the old one."""
    (x,) = args
    d = x.dim(at["name"])
    kn = at["k_name"]
    if x.has(kn):
        raise TypeError(f"tl.window: dim {kn!r} already exists")
    dil = _dilation(at)
    lo, hi = _taps(at["k"])
    if hi <= lo:
        raise TypeError(f"tl.window needs a non-empty tap range, got [{lo}, {hi})")
    ns, ne = d.start - dil * lo, d.stop - dil * (hi - 1)
    if ne < ns:
        raise TypeError(f"tl.window: taps [{lo}, {hi}) x {dil} are wider than {d.name}'s domain")
    out = []
    for e in x.dims:
        out.extend((Dim(e.name, ns, ne), Dim(kn, lo, hi)) if e.name == d.name else (e,))
    return TensorType(tuple(out))


def _r_stencil(args, at, regions):
    """guarded.py:463-520: name keeps its domain; the tap dim (INCLUSIVE
    tap range k = (kmin, kmax), named k_name or name + '_k') follows it.
    Taps that leave the domain read the fill."""
    (x,) = args
    d = x.dim(at["name"])
    kn = at.get("k_name") or f"{d.name}_k"
    if x.has(kn):
        raise TypeError(f"tl.stencil: dim {kn!r} already exists")
    _dilation(at)
    kmin, kmax = (int(v) for v in at["k"])
    if kmax < kmin:
        raise TypeError(f"tl.stencil: empty tap range ({kmin}, {kmax})")
    out = []
    for e in x.dims:
        out.extend((e, Dim(kn, kmin, kmax + 1)) if e.name == d.name else (e,))
    return TensorType(tuple(out))


def _r_decimate(args, at, regions):
    """layout.py:742-771: cells i = phase (mod factor) of name, renumbered
    j = (i - phase) / factor over [ceil((start - p) / f), floor((stop - 1 - p) / f] + 1)."""
    (x,) = args
    d = x.dim(at["name"])
    f = at["factor"]
    if not isinstance(f, int) or f < 1:
        raise TypeError(f"tl.decimate: factor must be a positive int, got {f!r}")
    p = int(at.get("phase", 0)) % f
    j0 = -((p - d.start) // f)
    j1 = (d.stop - 1 - p) // f
    return TensorType(tuple(Dim(e.name, j0, max(j0, j1 + 1)) if e.name == d.name else e for e in x.dims))


def _r_diagonal(args, at, regions):
    """layout.py:669-698: the parts (two or more) walked at once, as one dim
    ``name`` over the intersection of their domains, placed where the first
    of them sits in the operand."""
    (x,) = args
    parts = _dims_arg(at["parts"])
    if len(parts) < 2 or len(set(parts)) != len(parts):
        raise TypeError(f"tl.diagonal needs two or more distinct dims, got {parts}")
    ds = [x.dim(nm) for nm in parts]
    name = at["name"]
    if x.has(name) and name not in parts:
        raise TypeError(f"tl.diagonal: dim {name!r} already exists")
    start = max(d.start for d in ds)
    stop = max(start, min(d.stop for d in ds))
    out, placed = [], False
    for e in x.dims:
        if e.name in parts:
            if not placed:
                out.append(Dim(name, start, stop))
                placed = True
        else:
            out.append(e)
    return TensorType(tuple(out))


ENCODINGS = ("f32", "f16", "bf16")


def _r_round_to(args, at, regions):
    (x,) = args
    if at["encoding"] not in ENCODINGS:
        raise TypeError(f"tl.round_to: unknown encoding {at['encoding']!r} (one of {ENCODINGS})")
    if at.get("grad", "straight_through") not in ("straight_through", "zero"):
        raise TypeError("tl.round_to: grad is 'straight_through' or 'zero'")
    return TensorType(x.dims)


def _r_tuple(args, at, regions):
    return TupleType(tuple(args))


def _r_yield(args, at, regions):
    return args[0] if len(args) == 1 else TupleType(tuple(args))


def _r_argtopk(args, at, regions):
    (x,) = args
    return TensorType(tuple(Dim(at["k_name"], 0, at["k"]) if d.name == at["dim"] else d for d in x.dims))


OPS: dict[str, OpDef] = {
    "core.param": OpDef("core.param"),
    "core.const": OpDef("core.const"),
    "core.tuple": OpDef("core.tuple", _r_tuple),
    "core.yield": OpDef("core.yield", _r_yield),
    "tl.pointwise": OpDef("tl.pointwise", _r_pointwise),
    "tl.reduce": OpDef("tl.reduce", _r_reduce),
    "tl.scan": OpDef("tl.scan", _r_scan),
    "tl.repeat_like": OpDef("tl.repeat_like", _r_repeat_like),
    "tl.repeat": OpDef("tl.repeat", _r_repeat),
    "tl.split": OpDef("tl.split", _r_split),
    "tl.stage": OpDef("tl.stage", _r_stage),
    "tl.select": OpDef("tl.select", _r_select),
    "tl.iota": OpDef("tl.iota", _r_iota),
    "tl.const": OpDef("tl.const", _r_const),
    "tl.fold": OpDef("tl.fold", _r_fold, nregions=1),
    "tl.argtopk": OpDef("tl.argtopk", _r_argtopk),
    "tl.rename": OpDef("tl.rename", _r_rename),
    "tl.shift": OpDef("tl.shift", _r_shift),
    "tl.slice": OpDef("tl.slice", _r_slice),
    "tl.pad": OpDef("tl.pad", _r_pad),
    "tl.flip": OpDef("tl.flip", _r_flip),
    "tl.merge": OpDef("tl.merge", _r_merge),
    "tl.take": OpDef("tl.take", _r_take),
    "tl.scatter_add": OpDef("tl.scatter_add", _r_scatter_add),
    "tl.window": OpDef("tl.window", _r_window),
    "tl.stencil": OpDef("tl.stencil", _r_stencil),
    "tl.decimate": OpDef("tl.decimate", _r_decimate),
    "tl.diagonal": OpDef("tl.diagonal", _r_diagonal),
    "tl.round_to": OpDef("tl.round_to", _r_round_to),
}

# ops no template row reads: a region holding one plans it red
TILE_OPS = frozenset(OPS) - {"tl.argtopk", "tl.take", "tl.scatter_add", "tl.pad", "tl.flip", "tl.merge", "tl.stencil",
                             "tl.round_to"}


def builder() -> Builder:
    return Builder(OPS)


def const(b: Builder, value: float):
    return b.emit("core.const", type=F64, value=float(value))


def check_tier(region: Region, tier: str = "tile") -> Region:
    """The tile-tier gate (dialect.py:1150-1180): every op the region (and
    its fold steps) carries must be tile vocabulary; the first violation
    refuses, naming the op."""
    if tier != "tile":
        raise ValueError(f"only the tile tier is checked here (got {tier!r})")
    for n in walk(region):
        if n.op not in TILE_OPS:
            raise ValueError(f"{n.op} is a host citizen here — it has no tile-tier meaning (290)")
        for r in n.regions:
            check_tier(r, "tile")
    return region


__all__ = ["OPS", "MARKERS", "REDUCERS", "ENCODINGS", "builder", "const", "check_tier", "F64", "BOOL", "Scalar", "TensorType"]
