"""ORACLE — test infrastructure only (the checker, never the product).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package.

A float64 region evaluator on torch's CPU backend: the restatement of the
reference's second oracle, the substrate-generic interpreter with its torch
substrate (conformance/region_evaluator.py:167-471 + conformance/
torch_evaluator.py:27-139, float64 by default). It interprets the same
regions pdum_dsl_amd.tl builds — the naive twins (the denotation) and the
generated tile programs — by its own dispatch, independent of the
planner's numpy interpreter, so each can check the other:

  tl.pointwise   operands aligned by dim NAME, scalars broadcast
                 (region_evaluator.py:289-318; compute.py:95-123)
  tl.reduce      sum/prod/max/min via torch reductions; mean = sum / N
                 (compute.py:184-214; region_evaluator.py:320-352)
  tl.scan        inclusive prefix along one dim: cumsum / cumprod / cummax /
                 cummin; mean divides by the running count (compute.py:318-350)
  tl.repeat_like / tl.repeat / tl.split / tl.stage / tl.select / tl.iota /
  tl.const       layout views (region_evaluator.py:372-430)
  tl.rename / tl.shift / tl.slice   relabelings and a window (layout.py)
  tl.pad / tl.flip / tl.merge       a widened frame, a reversal, split's inverse
                 (layout.py)
  tl.take        the gather (indexing.py:120-230)
  tl.scatter_add its adjoint, duplicates summed (indexing.py:153-190, 223-259)
  tl.window / tl.stencil / tl.decimate   gathers along one dim by index
                 arithmetic (layout.py:700-771, guarded.py:463-520)
  tl.diagonal    the cells whose parts agree (layout.py:669-698)
  tl.round_to    nearest value of bf16 / f16 / f32, ties to even
                 (encoding.py:40-51, compute.py:368-375)
  composite tl.reduce / tl.scan   the sequential sweep of compute.py:230-260
                 over the reducer's traced lift / combine / project
  tl.fold        a Python loop over the scan dim (out ('final', i): the last
                 state i; ('emit',): each step's last yield stacked along the
                 scan dim), each element source
                 selected at the ABSOLUTE coordinate (dialect.py:1448-1470;
                 region_evaluator.py:431-465)

Values are (tensor, names) pairs; every float is float64.
"""

from __future__ import annotations

import numpy as np
import torch

_PW = {
    "add": torch.add, "sub": torch.sub, "mul": torch.mul, "div": torch.div, "neg": torch.neg,
    "exp": torch.exp, "log": torch.log, "maximum": torch.maximum, "minimum": torch.minimum,
    "tanh": torch.tanh, "sqrt": torch.sqrt, "sin": torch.sin, "cos": torch.cos, "abs": torch.abs,
    "floor": torch.floor, "eq": torch.eq, "ne": torch.ne, "le": torch.le, "lt": torch.lt, "ge": torch.ge,
    "gt": torch.gt, "stop_gradient": lambda x: x,
    "zoo.gelu": lambda x: 0.5 * x * (1 + torch.tanh(0.7978845608028654 * (x + 0.044715 * x * x * x))),
    # the derived partial marker zoo.gelu.d0 (autodiff.py:303-309): d/dx of the body above
    "zoo.gelu.d0": lambda x: _gelu_d0(x),
}


def _gelu_d0(x):
    c = 0.7978845608028654
    t = torch.tanh(c * (x + 0.044715 * x * x * x))
    return 0.5 * (1 + t) + 0.5 * x * (1 - t * t) * c * (1 + 0.134145 * x * x)


class V:
    """A named-dim float64 (or bool) tensor; dims = tuple of (name, start, stop)."""

    __slots__ = ("t", "dims")

    def __init__(self, t: torch.Tensor, dims):
        self.t, self.dims = t, tuple(dims)

    @property
    def names(self):
        return tuple(d[0] for d in self.dims)

    def order(self, names) -> torch.Tensor:
        return self.t.permute([self.names.index(n) for n in names])

    def numpy(self, names=None) -> np.ndarray:
        t = self.t if names is None else self.order(names)
        return t.detach().cpu().numpy()


def value(arr, ir_type) -> V:
    """Wrap a numpy array as a value of a TensorType (axes in type-dim order)."""
    dims = tuple((d.name, d.start, d.stop) for d in ir_type.dims)
    t = torch.as_tensor(np.asarray(arr))
    if t.dtype != torch.bool:
        t = t.to(torch.float64)
    return V(t, dims)


def _canon(x, tt):
    """``x`` with its axes in its type's dim order (for ops that work by axis position)."""
    names = tuple(d.name for d in tt.dims)
    if not isinstance(x, V) or x.names == names:
        return x
    return V(x.order(names), tuple(x.dims[x.names.index(nm)] for nm in names))


def _dims_arg(d):
    return (d,) if isinstance(d, str) else tuple(d)


def evaluate(region, values: list):
    """Evaluate ``region`` on V values positional per param; returns V or a tuple of V."""
    memo: dict[int, object] = {}
    params = {id(p): v for p, v in zip(region.params, values)}

    def ev(n):
        k = id(n)
        if k in memo:
            return memo[k]
        r = params[k] if k in params else _dispatch(n, ev)
        memo[k] = r
        return r

    return ev(region.body[-1])


def _attr(n, name, default=None):
    for k, v in n.attrs:
        if k == name:
            return v
    return default


_BITS = {"f32": (24, -149, 3.4028234663852886e38), "f16": (11, -24, 65504.0),
         "bf16": (8, -133, 3.3895313892515355e38)}


def _round(t: torch.Tensor, enc: str) -> torch.Tensor:
    bits, qmin, top = _BITS[enc]
    m, e = torch.frexp(t)
    q = torch.clamp(e - bits, min=qmin)
    out = torch.round(torch.ldexp(m, (e - q).to(torch.float64))) * torch.pow(torch.tensor(2.0, dtype=torch.float64),
                                                                            q.to(torch.float64))
    if not torch.isfinite(out).all() or bool((out.abs() > top).any()):
        raise ValueError(f"round_to({enc}): not finite in the format")
    return out


def _gather(x: V, n):
    """window / stencil / decimate: out[.., c, ..] = x[.., src(c), ..]."""
    name = _attr(n, "name")
    ax = x.names.index(name)
    _, lo, hi = x.dims[ax]
    out_dims = tuple((d.name, d.start, d.stop) for d in n.type.dims)
    od = next(d for d in n.type.dims if d.name == name)
    if n.op == "tl.decimate":
        f = _attr(n, "factor")
        src = torch.arange(od.start, od.stop) * f + int(_attr(n, "phase", 0) or 0) % f
        return V(torch.index_select(x.t, ax, src - lo), out_dims)
    kn = _attr(n, "k_name") or f"{name}_k"
    kd = next(d for d in n.type.dims if d.name == kn)
    dil = _attr(n, "dilation", 1) or 1
    src = torch.arange(od.start, od.stop).unsqueeze(1) + dil * torch.arange(kd.start, kd.stop).unsqueeze(0)
    live = (src >= lo) & (src < hi)
    safe = torch.where(live, src - lo, torch.zeros_like(src))
    if hi == lo:
        got = torch.zeros(tuple(x.t.shape[:ax]) + tuple(src.shape) + tuple(x.t.shape[ax + 1:]), dtype=torch.float64)
    else:
        got = torch.index_select(x.t, ax, safe.reshape(-1)).reshape(
            tuple(x.t.shape[:ax]) + tuple(src.shape) + tuple(x.t.shape[ax + 1:]))
    if n.op == "tl.stencil":
        shape = (1,) * ax + tuple(live.shape) + (1,) * (x.t.dim() - ax - 1)
        got = torch.where(live.reshape(shape), got, torch.tensor(float(_attr(n, "fill", 0.0) or 0.0),
                                                                 dtype=torch.float64))
    return V(got, out_dims)


def _sweep(n, ev):
    """A composite reducer: lift the first element, combine the rest in
    order (compute.py:230-260); project the last state, or each (a scan)."""
    from pdum_dsl_amd.tl.ir import minus_dim
    from pdum_dsl_amd.tl.reducers import lookup, parts

    f = lookup(_attr(n, "f"))
    dim = _attr(n, "dim") if n.op == "tl.scan" else _dims_arg(_attr(n, "dims"))[0]
    st = minus_dim(n.args[0].type, dim)
    P = parts(f, st)
    xs = [ev(a) for a in n.args]
    ax = xs[0].names.index(dim)
    _, lo, hi = xs[0].dims[ax]

    def run(region, vals):
        r = evaluate(region, list(vals))
        return tuple(r) if isinstance(r, tuple) else (r,)

    rest = tuple(d for d in xs[0].dims if d[0] != dim)
    state, outs = None, []
    for c in range(lo, hi):
        el = []
        for x in xs:
            a = x.names.index(dim)
            el.append(V(x.t.select(a, c - x.dims[a][1]), x.dims[:a] + x.dims[a + 1:]))
        lifted = run(P.lift, el)
        state = lifted if state is None else run(P.combine, state + lifted)
        if n.op == "tl.scan":
            outs.append(run(P.project, state)[0].order([d[0] for d in rest]))
    names = [d[0] for d in rest]
    if n.op == "tl.scan":
        t = torch.stack(outs, dim=len(names)) if outs else torch.zeros([d[2] - d[1] for d in rest] + [0],
                                                                        dtype=torch.float64)
        src = names + [dim]
        return V(t.permute([src.index(d.name) for d in n.type.dims]), tuple((d.name, d.start, d.stop)
                                                                              for d in n.type.dims))
    if state is None:
        state = tuple(V(torch.full([d[2] - d[1] for d in rest], v, dtype=torch.float64), rest) for v in f.init)
    out = run(P.project, state)[0]
    return V(out.order([d.name for d in n.type.dims]), tuple((d.name, d.start, d.stop) for d in n.type.dims))


def _dispatch(n, ev):
    op = n.op
    if op in ("tl.reduce", "tl.scan"):
        from pdum_dsl_amd.tl.reducers import is_composite

        if is_composite(_attr(n, "f")):
            return _sweep(n, ev)
    if op in ("tl.window", "tl.stencil", "tl.decimate"):
        return _gather(_canon(ev(n.args[0]), n.args[0].type), n)
    if op == "tl.diagonal":
        x = _canon(ev(n.args[0]), n.args[0].type)
        parts = _dims_arg(_attr(n, "parts"))
        axes = [x.names.index(nm) for nm in parts]
        z = next(d for d in n.type.dims if d.name == _attr(n, "name"))
        t = x.t.movedim(axes, list(range(len(axes))))
        cz = torch.arange(z.start, z.stop)
        got = t[tuple(cz - x.dims[a][1] for a in axes)]
        at = [d.name for d in n.type.dims].index(z.name)
        return V(got.movedim(0, at), tuple((d.name, d.start, d.stop) for d in n.type.dims))
    if op == "tl.round_to":
        x = ev(n.args[0])
        return V(_round(x.t, _attr(n, "encoding")), x.dims)
    if op == "core.const":
        return float(_attr(n, "value"))
    if op == "core.yield":
        return ev(n.args[0])
    if op == "core.tuple":
        return tuple(ev(a) for a in n.args)
    if op == "tl.pointwise":
        vals = [ev(a) for a in n.args]
        ref = next(v for v in vals if isinstance(v, V))
        ts = [v.order(ref.names) if isinstance(v, V) else v for v in vals]
        f = _attr(n, "f")
        if f == "where":
            c, a, b = ts
            a = a if torch.is_tensor(a) else torch.tensor(a, dtype=torch.float64)
            b = b if torch.is_tensor(b) else torch.tensor(b, dtype=torch.float64)
            out = torch.where(c.bool(), a, b)
        else:
            ts = [t if torch.is_tensor(t) else torch.tensor(t, dtype=torch.float64) for t in ts]
            out = _PW[f](*ts)
        return V(out, ref.dims)
    if op == "tl.reduce":
        x = ev(n.args[0])
        dims = _dims_arg(_attr(n, "dims"))
        axes = [x.names.index(d) for d in dims]
        f = _attr(n, "f")
        t = x.t.to(torch.float64) if x.t.dtype == torch.bool else x.t
        if f in ("sum", "mean"):
            out = t.sum(dim=axes) if axes else t
            if f == "mean":
                cnt = 1
                for a in axes:
                    cnt *= t.shape[a]
                out = out / cnt
        elif f == "prod":
            out = t
            for a in sorted(axes, reverse=True):
                out = out.prod(dim=a)
        else:
            out = t
            for a in sorted(axes, reverse=True):
                out = out.amax(dim=a) if f == "max" else out.amin(dim=a)
        return V(out, tuple(d for d in x.dims if d[0] not in dims))
    if op == "tl.scan":  # inclusive prefix reduce along one dim (compute.py:318-350)
        x = ev(n.args[0])
        ax = x.names.index(_attr(n, "dim"))
        f = _attr(n, "f")
        t = x.t.to(torch.float64) if x.t.dtype == torch.bool else x.t
        rev = bool(_attr(n, "reverse") or False)
        if rev:
            t = torch.flip(t, dims=(ax,))
        if f in ("sum", "mean"):
            out = torch.cumsum(t, dim=ax)
            if f == "mean":
                shape = [1] * t.dim()
                shape[ax] = t.shape[ax]
                out = out / torch.arange(1, t.shape[ax] + 1, dtype=torch.float64).reshape(shape)
        elif f == "prod":
            out = torch.cumprod(t, dim=ax)
        else:
            out = (torch.cummax if f == "max" else torch.cummin)(t, dim=ax).values
        if rev:
            out = torch.flip(out, dims=(ax,))
        return V(out, x.dims)
    if op == "tl.repeat_like":
        x, like = ev(n.args[0]), ev(n.args[1])
        extra = tuple(d for d in like.dims if d[0] not in x.names)
        t = x.t.reshape(tuple(x.t.shape) + (1,) * len(extra))
        return V(t.expand(tuple(x.t.shape) + tuple(d[2] - d[1] for d in extra)), x.dims + extra)
    if op == "tl.repeat":
        x = ev(n.args[0])
        ext = _attr(n, "extent")
        lo, hi = (ext if isinstance(ext, tuple) else (0, ext))
        return V(x.t.unsqueeze(-1).expand(tuple(x.t.shape) + (hi - lo,)), x.dims + ((_attr(n, "name"), lo, hi),))
    if op == "tl.split":
        x = ev(n.args[0])
        name = _attr(n, "name")
        ax = x.names.index(name)
        parts = tuple(_attr(n, "parts"))
        sizes = tuple(int(s) for _, s in parts)
        t = x.t.reshape(tuple(x.t.shape[:ax]) + sizes + tuple(x.t.shape[ax + 1:]))
        dims = x.dims[:ax] + tuple((p, 0, int(s)) for p, s in parts) + x.dims[ax + 1:]
        return V(t, dims)
    if op == "tl.stage":
        x = ev(n.args[0])
        order = _attr(n, "order")
        if order:
            return V(x.order(order), tuple(x.dims[x.names.index(o)] for o in order))
        return x
    if op == "tl.select":
        x = ev(n.args[0])
        for name, i in _attr(n, "coords"):
            ax = x.names.index(name)
            x = V(x.t.select(ax, i - x.dims[ax][1]), x.dims[:ax] + x.dims[ax + 1:])
        return x
    if op == "tl.iota":
        dims = tuple((d.name, d.start, d.stop) for d in n.type.dims)
        name = _attr(n, "name")
        ax = [d[0] for d in dims].index(name)
        lo, hi = dims[ax][1], dims[ax][2]
        shape = [1] * len(dims)
        shape[ax] = hi - lo
        coords = torch.arange(lo, hi, dtype=torch.float64).reshape(shape)
        return V(coords.expand([d[2] - d[1] for d in dims]), dims)
    if op in ("tl.rename", "tl.shift"):  # layout.py rename / shift: relabelings, no data moves
        x = _canon(ev(n.args[0]), n.args[0].type)
        return V(x.t, tuple((d.name, d.start, d.stop) for d in n.type.dims))
    if op == "tl.slice":  # layout.py slice: absolute [lo, hi) per dim, matched by name
        x = ev(n.args[0])
        t = x.t
        out = tuple(n.type.dim(d[0]) for d in x.dims)
        for ax, (d, o) in enumerate(zip(x.dims, out)):
            t = t.narrow(ax, o.start - d[1], o.stop - o.start)
        return V(t, tuple((d.name, d.start, d.stop) for d in out))
    if op == "tl.pad":  # layout.py pad: frames widened, new cells = fill
        x = ev(n.args[0])
        out_dims = tuple((o.name, o.start, o.stop) for o in (n.type.dim(d[0]) for d in x.dims))
        t = torch.full([d[2] - d[1] for d in out_dims], float(_attr(n, "fill", 0.0)), dtype=torch.float64)
        window = tuple(slice(xd[1] - od[1], xd[2] - od[1]) for xd, od in zip(x.dims, out_dims))
        t[window] = x.t
        return V(t, out_dims)
    if op == "tl.flip":  # layout.py flip: coordinate c reads start + stop - 1 - c
        x = ev(n.args[0])
        return V(torch.flip(x.t, dims=(x.names.index(_attr(n, "name")),)), x.dims)
    if op == "tl.merge":  # layout.py merge: split's inverse, parts outer first
        x = _canon(ev(n.args[0]), n.args[0].type)
        parts = _attr(n, "parts")
        parts = (parts,) if isinstance(parts, str) else tuple(parts)
        rest = [nm for nm in x.names if nm not in parts]
        first = x.names.index(parts[0])
        at = first - sum(1 for nm in x.names[:first] if nm in parts)
        order = rest[:at] + list(parts) + rest[at:]
        t = x.order(tuple(order))
        t = t.reshape(tuple(t.shape[:at]) + (-1,) + tuple(t.shape[at + len(parts):]))
        return V(t, tuple((d.name, d.start, d.stop) for d in n.type.dims))
    if op == "tl.take":  # indexing.py:192-230: the taken dim replaced in place by idx's dims
        table, idx = _canon(ev(n.args[0]), n.args[0].type), _canon(ev(n.args[1]), n.args[1].type)
        name = _attr(n, "dim")
        ax = table.names.index(name)
        lo, hi = table.dims[ax][1], table.dims[ax][2]
        it = idx.t.to(torch.int64)
        if it.numel() and (int(it.min()) < lo or int(it.max()) >= hi):
            raise IndexError(f"tl.take: index outside [{lo}, {hi}) along {name!r}")
        got = torch.index_select(table.t, ax, (it - lo).reshape(-1))
        shape = tuple(table.t.shape[:ax]) + tuple(it.shape) + tuple(table.t.shape[ax + 1:])
        return V(got.reshape(shape), tuple((d.name, d.start, d.stop) for d in n.type.dims))
    if op == "tl.scatter_add":  # indexing.py:223-259: take's adjoint, duplicates summed
        vals, idx = ev(n.args[0]), ev(n.args[1])
        over = _attr(n, "over")
        consumed = list(idx.names) if over is None else ([over] if isinstance(over, str) else list(over))
        if any(nm not in consumed for nm in idx.names):
            raise NotImplementedError("tl.scatter_add with aligned (riding) idx dims")
        name = _attr(n, "dim")
        od = next(d for d in n.type.dims if d.name == name)
        it = idx.t.to(torch.int64).reshape(-1)
        if it.numel() and (int(it.min()) < od.start or int(it.max()) >= od.stop):
            raise IndexError(f"tl.scatter_add: index outside [{od.start}, {od.stop}) along {name!r}")
        rest = [nm for nm in vals.names if nm not in consumed]
        vt = vals.t.permute([vals.names.index(nm) for nm in list(idx.names) + rest])
        vt = vt.reshape((it.numel(),) + tuple(vt.shape[len(idx.names):]))
        acc = torch.zeros((od.stop - od.start,) + tuple(vt.shape[1:]), dtype=torch.float64)
        acc.index_add_(0, it - od.start, vt)
        src = [name] + rest
        return V(acc.permute([src.index(d.name) for d in n.type.dims]),
                 tuple((d.name, d.start, d.stop) for d in n.type.dims))
    if op == "tl.const":
        dims = tuple((d.name, d.start, d.stop) for d in n.type.dims)
        return V(torch.full([d[2] - d[1] for d in dims], float(_attr(n, "value")), dtype=torch.float64), dims)
    if op == "tl.fold":
        state = tuple(_attr(n, "state"))
        k = len(state)
        dim = _attr(n, "dim")
        vals = [ev(a) for a in n.args]
        carried, srcs = list(vals[:k]), vals[k:]
        d = next(x for x in srcs[0].dims if x[0] == dim)
        step = n.regions[0]
        out = tuple(_attr(n, "out"))
        emitted = []
        for q in range(d[1], d[2]):
            sel = []
            for s in srcs:
                ax = s.names.index(dim)
                sel.append(V(s.t.select(ax, q - s.dims[ax][1]), s.dims[:ax] + s.dims[ax + 1:]))
            res = evaluate(step, carried + sel)
            res = list(res) if isinstance(res, tuple) else [res]
            carried = res[:k]
            if out[0] == "emit":  # the step's last yield, stacked along the scan dim (last)
                e = res[k]
                want = [x.name for x in n.type.dims if x.name != dim]
                emitted.append(e.t.permute([e.names.index(nm) for nm in want]))
        if out[0] == "emit":
            return V(torch.stack(emitted, dim=-1), tuple((x.name, x.start, x.stop) for x in n.type.dims))
        return carried[out[1]]
    raise NotImplementedError(f"oracle evaluator: no rule for {op}")
