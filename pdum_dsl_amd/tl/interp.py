"""Plan-time reference interpreter for certification.

The reference's planner certifies every template kernel against its naive
twin by EVALUATING both (certify.py:567-609 calls dialect.run_region,
dialect.py:1349-1473). This module is that evaluator for the tile
vocabulary of pdum_dsl_amd.tl.dialect, in float64 numpy, used ONLY by
``certify`` to decide a Group's certificate at plan time. It is never on the
execution path: compile_tile_hip's runners launch HIP kernels and nothing
else.

Semantics follow the reference: pointwise aligns operands by dim NAME
(compute.py:95-123), reduce is the numpy ufunc reduce with the reducer's
identity (max has none; mean = sum / static N, compute.py:184-214), fold
iterates its scan dim and hands the step each element source SELECTED at the
absolute coordinate (dialect.py:1448-1470).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .ir import Dim, Node, Region, TensorType, minus_dim
from .reducers import is_composite, lookup, parts

_PW = {
    "add": np.add, "sub": np.subtract, "mul": np.multiply, "div": np.divide, "neg": np.negative,
    "exp": np.exp, "log": np.log, "maximum": np.maximum, "minimum": np.minimum, "tanh": np.tanh,
    "sqrt": np.sqrt, "sin": np.sin, "cos": np.cos, "abs": np.abs, "floor": np.floor, "where": np.where,
    "eq": np.equal, "ne": np.not_equal, "le": np.less_equal, "lt": np.less, "ge": np.greater_equal,
    "gt": np.greater, "stop_gradient": np.positive,
    # the composite marker zoo_common.py:20 registers: 0.5 x (1 + tanh(c (x + 0.044715 x^3)))
    "zoo.gelu": lambda x: 0.5 * x * (1 + np.tanh(0.7978845608028654 * (x + 0.044715 * x * x * x))),
    # its partial, the derived marker f.d0 (autodiff.py:303-309 derives it from the body)
    "zoo.gelu.d0": lambda x: _gelu_d0(np, x),
}


def _gelu_d0(lib, x):
    """d/dx of 0.5 x (1 + tanh(u)), u = c (x + 0.044715 x^3):
    0.5 (1 + tanh u) + 0.5 x (1 - tanh^2 u) c (1 + 3 * 0.044715 x^2)."""
    c = 0.7978845608028654
    t = lib.tanh(c * (x + 0.044715 * x * x * x))
    return 0.5 * (1 + t) + 0.5 * x * (1 - t * t) * c * (1 + 0.134145 * x * x)


_RED = {"sum": (np.add, 0.0), "prod": (np.multiply, 1.0), "max": (np.maximum, None), "min": (np.minimum, None)}

# significant bits, exponent of the smallest quantum (subnormal), largest finite value
_FORMATS = {"f32": (24, -149, 3.4028234663852886e38), "f16": (11, -24, 65504.0),
            "bf16": (8, -133, 3.3895313892515355e38)}


def round_to(arr, encoding: str) -> np.ndarray:
    """encode-then-decode (encoding.py:40-42, compute.py:368-375): round to
    the nearest value of the format, ties to even, subnormals kept; a value
    that rounds past the largest finite one refuses, as non-finite patterns
    refuse at decode (encoding.py:45-51)."""
    bits, qmin, top = _FORMATS[encoding]
    a = np.asarray(arr, dtype=np.float64)
    _, e = np.frexp(a)  # a = m 2^e, 1/2 <= |m| < 1
    q = np.maximum(e - bits, qmin)  # the quantum's exponent at a's binade
    out = np.ldexp(np.rint(np.ldexp(a, -q)), q)
    if not np.isfinite(out).all() or (np.abs(out) > top).any():
        raise ValueError(f"tl.round_to({encoding}): a value is not finite in the format (inf/nan refuse at decode)")
    return out


@dataclass
class Field:
    """A named-dim array: ``arr`` axes follow ``dims``."""

    arr: np.ndarray
    dims: tuple[Dim, ...]

    @property
    def names(self):
        return tuple(d.name for d in self.dims)

    def to_numpy(self, order=None) -> np.ndarray:
        if order is None:
            return self.arr
        return np.transpose(self.arr, [self.names.index(n) for n in order])

    def aligned_to(self, names) -> np.ndarray:
        return self.to_numpy(tuple(names))

    def select(self, name: str, i: int) -> "Field":
        ax = self.names.index(name)
        d = self.dims[ax]
        return Field(np.take(self.arr, i - d.start, axis=ax), tuple(x for x in self.dims if x.name != name))


def _canon(x: Field, tt: TensorType) -> Field:
    """``x`` with its axes in its type's dim order (values align by name, so
    an op that works by axis position first puts the axes where the type has
    them)."""
    if not isinstance(x, Field) or x.names == tt.names:
        return x
    return Field(x.to_numpy(tt.names), tuple(x.dims[x.names.index(nm)] for nm in tt.names))


def field(arr, names) -> Field:
    arr = np.asarray(arr)
    return Field(arr, tuple(Dim(n, 0, s) for n, s in zip(names, arr.shape)))


def _as_field(x, ref: Field) -> np.ndarray:
    if isinstance(x, Field):
        return x.aligned_to(ref.names)
    return np.full(ref.arr.shape, float(x))


def run_region(region: Region, values: list):
    """Evaluate ``region`` over Field values (positional per param)."""
    memo: dict[int, object] = {}
    bind = {id(p): v for p, v in zip(region.params, values)}

    def ev(n: Node):
        k = id(n)
        if k not in memo:
            memo[k] = _ev(n)
        return memo[k]

    def _ev(n: Node):
        if id(n) in bind:
            v = bind[id(n)]
            tt = n.type
            if isinstance(v, Field) and isinstance(tt, TensorType):
                # a value bound by names alone (field() frames start at 0) takes
                # the param's declared frames: a seed aligned with an offset target
                frames = {d.name: d for d in tt.dims}
                if set(v.names) == set(frames) and all(d.size == frames[d.name].size for d in v.dims):
                    v = Field(v.arr, tuple(frames[d.name] for d in v.dims))
            return v
        op = n.op
        if op == "core.const":
            return float(n.attr("value"))
        if op == "core.yield":
            return ev(n.args[0])
        if op == "core.tuple":
            return tuple(ev(a) for a in n.args)
        if op == "tl.pointwise":
            vals = [ev(a) for a in n.args]
            ref = next(v for v in vals if isinstance(v, Field))
            arrs = [_as_field(v, ref) for v in vals]
            return Field(np.asarray(_PW[n.attr("f")](*arrs)), ref.dims)
        if op in ("tl.reduce", "tl.scan") and is_composite(n.attr("f")):
            return _composite(n, [ev(a) for a in n.args])
        if op == "tl.reduce":
            x = ev(n.args[0])
            dims = n.attr("dims")
            dims = (dims,) if isinstance(dims, str) else tuple(dims)
            axes = tuple(x.names.index(d) for d in dims)
            f = n.attr("f")
            arr = x.arr.astype(np.float64) if x.arr.dtype == bool else x.arr
            if f == "mean":
                cnt = 1
                for ax in axes:
                    cnt *= arr.shape[ax]
                out = np.add.reduce(arr, axis=axes) / cnt
            else:
                fn, ident = _RED[f]
                out = fn.reduce(arr, axis=axes) if ident is None else fn.reduce(arr, axis=axes, initial=ident)
            return Field(np.asarray(out), tuple(d for d in x.dims if d.name not in dims))
        if op == "tl.scan":  # ufunc accumulate along the dim, as compute.py:340-350
            x = ev(n.args[0])
            ax = x.names.index(n.attr("dim"))
            f = n.attr("f")
            arr = x.arr.astype(np.float64) if x.arr.dtype == bool else x.arr
            if n.attr("reverse", False):
                arr = np.flip(arr, axis=ax)
            fn = np.add if f == "mean" else _RED[f][0]
            out = fn.accumulate(arr, axis=ax)
            if f == "mean":
                shape = [1] * arr.ndim
                shape[ax] = arr.shape[ax]
                out = out / np.arange(1, arr.shape[ax] + 1).reshape(shape)
            if n.attr("reverse", False):
                out = np.flip(out, axis=ax)
            return Field(np.ascontiguousarray(out), x.dims)
        if op == "tl.repeat_like":
            x, like = ev(n.args[0]), ev(n.args[1])
            extra = tuple(d for d in like.dims if d.name not in x.names)
            arr = x.arr.reshape(x.arr.shape + (1,) * len(extra))
            return Field(np.broadcast_to(arr, x.arr.shape + tuple(d.size for d in extra)), x.dims + extra)
        if op == "tl.repeat":
            x = ev(n.args[0])
            (d,) = [e for e in n.type.dims if e.name == n.attr("name")]
            return Field(np.broadcast_to(x.arr[..., None], x.arr.shape + (d.size,)), x.dims + (d,))
        if op == "tl.split":
            x = _canon(ev(n.args[0]), n.args[0].type)
            name = n.attr("name")
            ax = x.names.index(name)
            sizes = tuple(int(s) for _, s in n.attr("parts"))
            arr = x.arr.reshape(x.arr.shape[:ax] + sizes + x.arr.shape[ax + 1:])
            return Field(arr, n.type.dims)
        if op == "tl.stage":
            x = ev(n.args[0])
            order = n.attr("order")
            return Field(x.to_numpy(tuple(order)), n.type.dims) if order else x
        if op == "tl.select":
            x = ev(n.args[0])
            for name, i in n.attr("coords"):
                x = x.select(name, i)
            return x
        if op == "tl.iota":  # a closed form: the lattice's values are never read
            tt: TensorType = n.type
            name = n.attr("name")
            ax = tt.names.index(name)
            d = tt.dims[ax]
            shape = [1] * len(tt.dims)
            shape[ax] = d.size
            coords = np.arange(d.start, d.stop, dtype=np.int64).reshape(shape)
            return Field(np.broadcast_to(coords, tt.shape), tt.dims)
        if op in ("tl.rename", "tl.shift"):  # relabelings: names or frames move, values stay
            x = _canon(ev(n.args[0]), n.args[0].type)
            return Field(x.arr, n.type.dims)
        if op == "tl.slice":  # dims matched by name: a value's axis order may differ from its type's
            x = ev(n.args[0])
            out = tuple(n.type.dim(d.name) for d in x.dims)
            idx = tuple(slice(o.start - d.start, o.stop - d.start) for d, o in zip(x.dims, out))
            return Field(x.arr[idx], out)
        if op == "tl.pad":
            x = ev(n.args[0])
            out = tuple(n.type.dim(d.name) for d in x.dims)
            widths = [(d.start - o.start, o.stop - d.stop) for d, o in zip(x.dims, out)]
            return Field(np.pad(x.arr, widths, constant_values=float(n.attr("fill", 0.0))), out)
        if op == "tl.flip":
            x = ev(n.args[0])
            return Field(np.flip(x.arr, axis=x.names.index(n.attr("name"))), x.dims)
        if op == "tl.merge":
            x = _canon(ev(n.args[0]), n.args[0].type)
            parts = n.attr("parts")
            parts = (parts,) if isinstance(parts, str) else tuple(parts)
            rest = [nm for nm in x.names if nm not in parts]
            at = x.names.index(parts[0]) - sum(1 for nm in x.names[:x.names.index(parts[0])] if nm in parts)
            order = rest[:at] + list(parts) + rest[at:]
            arr = x.to_numpy(tuple(order))
            shp = arr.shape[:at] + (int(np.prod(arr.shape[at:at + len(parts)])),) + arr.shape[at + len(parts):]
            return Field(arr.reshape(shp), n.type.dims)
        if op == "tl.take":
            table, idx = _canon(ev(n.args[0]), n.args[0].type), _canon(ev(n.args[1]), n.args[1].type)
            dim = n.attr("dim")
            d = table.dims[table.names.index(dim)]
            ia = np.asarray(idx.arr)
            if ia.size and (ia.min() < d.start or ia.max() >= d.stop):
                raise IndexError(f"tl.take: index outside [{d.start}, {d.stop}) along {dim!r}")
            surv = [x.name for x in table.dims if x.name != dim]
            aligned = [nm for nm in idx.names if nm in surv]
            spliced = [nm for nm in idx.names if nm not in surv]
            if aligned:
                raise NotImplementedError("run_region: batched tl.take (aligned idx dims) is not evaluated here")
            ax = table.names.index(dim)
            got = np.take(table.arr, ia.astype(np.int64) - d.start, axis=ax)
            return Field(got.reshape(table.arr.shape[:ax] + ia.shape + table.arr.shape[ax + 1:]), n.type.dims)
        if op == "tl.scatter_add":
            vals, idx = ev(n.args[0]), ev(n.args[1])
            over = n.attr("over")
            consumed = list(idx.names) if over is None else ([over] if isinstance(over, str) else list(over))
            if any(nm not in consumed for nm in idx.names):
                raise NotImplementedError("run_region: batched tl.scatter_add (aligned idx dims) is not evaluated here")
            d = n.type.dim(n.attr("dim"))
            ia = np.asarray(idx.arr).astype(np.int64)
            if ia.size and (ia.min() < d.start or ia.max() >= d.stop):
                raise IndexError(f"tl.scatter_add: index outside [{d.start}, {d.stop}) along {d.name!r}")
            rest = [nm for nm in vals.names if nm not in consumed]
            va = vals.to_numpy(tuple(idx.names) + tuple(rest)).reshape((ia.size,) + tuple(
                vals.dims[vals.names.index(nm)].size for nm in rest))
            acc = np.zeros((d.size,) + va.shape[1:])
            np.add.at(acc, ia.reshape(-1) - d.start, va)  # duplicates sum, in order
            src = (d.name,) + tuple(rest)
            return Field(np.transpose(acc, [src.index(x.name) for x in n.type.dims]), n.type.dims)
        if op in ("tl.window", "tl.stencil", "tl.decimate"):
            return _taps(n, _canon(ev(n.args[0]), n.args[0].type))
        if op == "tl.diagonal":
            x = _canon(ev(n.args[0]), n.args[0].type)
            parts = n.attr("parts")
            parts = (parts,) if isinstance(parts, str) else tuple(parts)
            axes = [x.names.index(nm) for nm in parts]
            z = n.type.dim(n.attr("name"))
            arr = np.moveaxis(x.arr, axes, range(len(axes)))
            cz = np.arange(z.start, z.stop)
            got = arr[tuple(cz - x.dims[ax].start for ax in axes)]  # (z, the other dims in order)
            at = n.type.names.index(z.name)
            return Field(np.moveaxis(got, 0, at), n.type.dims)
        if op == "tl.round_to":
            x = ev(n.args[0])
            return Field(round_to(x.arr, n.attr("encoding")), x.dims)
        if op == "tl.const":
            tt = n.type
            return Field(np.full(tt.shape, float(n.attr("value"))), tt.dims)
        if op == "tl.fold":
            state = tuple(n.attr("state"))
            k = len(state)
            dim = n.attr("dim")
            vals = [ev(a) for a in n.args]
            carried, srcs = list(vals[:k]), vals[k:]
            d = n.args[k].type.dim(dim)
            step = n.regions[0]
            out = tuple(n.attr("out"))
            emitted = []
            for q in range(d.start, d.stop):
                res = run_region(step, carried + [s.select(dim, q) for s in srcs])
                res = list(res) if isinstance(res, tuple) else [res]
                carried = res[:k]
                if out[0] == "emit":  # the emission in the node's dim order, less the scan dim
                    e = res[k]
                    emitted.append(e.to_numpy(tuple(x.name for x in n.type.dims if x.name != dim)))
            if out[0] == "emit":
                return Field(np.stack(emitted, axis=-1), n.type.dims)
            return carried[out[1]]
        raise NotImplementedError(f"run_region: {op} has no evaluation rule here")

    return ev(region.body[-1])


def _taps(n: Node, x: Field) -> Field:
    """tl.window / tl.stencil / tl.decimate: gathers along one dim by an
    index grid over the output's coordinates (layout.py:700-771,
    guarded.py:463-520)."""
    name = n.attr("name")
    ax = x.names.index(name)
    d = x.dims[ax]
    if n.op == "tl.decimate":
        f = n.attr("factor")
        j = np.arange(n.type.dim(name).start, n.type.dim(name).stop)
        idx = f * j + int(n.attr("phase", 0)) % f
        return Field(np.take(x.arr, idx - d.start, axis=ax), n.type.dims)
    dil = n.attr("dilation", 1)
    kn = n.attr("k_name") or f"{name}_k"
    xo, ko = n.type.dim(name), n.type.dim(kn)
    idx = np.arange(xo.start, xo.stop)[:, None] + dil * np.arange(ko.start, ko.stop)[None, :]
    if n.op == "tl.window":  # every tap lands inside by construction
        return Field(np.take(x.arr, idx - d.start, axis=ax), n.type.dims)
    live = (idx >= d.start) & (idx < d.stop)
    got = np.take(x.arr, np.clip(idx - d.start, 0, max(d.size - 1, 0)), axis=ax) if d.size else \
        np.zeros(x.arr.shape[:ax] + idx.shape + x.arr.shape[ax + 1:])
    shape = (1,) * ax + live.shape + (1,) * (x.arr.ndim - ax - 1)
    return Field(np.where(live.reshape(shape), got, float(n.attr("fill", 0.0))), n.type.dims)


def _composite(n: Node, vals: list) -> Field:
    """A composite reducer's sweep along its dim (compute.py:230-260): the
    first element's lift, then combine(state, lift(element)) in order; a
    reduce projects the last state (the declared init for an empty dim), a
    scan each one."""
    f = lookup(n.attr("f"))
    dim = n.attr("dim") if n.op == "tl.scan" else ((lambda d: d if isinstance(d, str) else d[0])(n.attr("dims")))
    tt = n.args[0].type
    st = minus_dim(tt, dim)
    P = parts(f, st)
    d = tt.dim(dim)

    def run(region, xs):
        r = run_region(region, list(xs))
        return tuple(r) if isinstance(r, tuple) else (r,)

    order = st.names
    state, outs = None, []
    for q in range(d.start, d.stop):
        lifted = run(P.lift, [v.select(dim, q) for v in vals])
        state = lifted if state is None else run(P.combine, state + lifted)
        if n.op == "tl.scan":
            outs.append(run(P.project, state)[0].to_numpy(order))
    if n.op == "tl.scan":
        arr = np.stack(outs, axis=len(order)) if outs else np.zeros(st.shape + (0,))
        names = order + (dim,)
        return Field(np.transpose(arr, [names.index(x.name) for x in n.type.dims]), n.type.dims)
    if state is None:  # an empty dim: the declared identity state
        state = tuple(Field(np.full(st.shape, v), st.dims) for v in f.init)
    out = run(P.project, state)[0]
    return Field(out.to_numpy(n.type.names), n.type.dims)
