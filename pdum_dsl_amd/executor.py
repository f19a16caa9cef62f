"""The carved-plan executor on the device: a whole model run carve by carve
on MI355X, every boundary tensor resident in HBM.

The reference carves a model (partition.plan_model) and runs the carves in
dependency order on its CPU oracle only (packages/tensorlib/tests/
test_partition.py:15-37, 124-193: a worklist, free views resolved at the
edges, red groups through the evaluator). Here the same plan runs on HIP
kernels, one step per carve:

  flash                 pdh_flash_fwd, the closed mask bound as a band, the
                        (m, den) artifacts when the carve yields them
  flash-joint           pdh_flash_fwd with artifacts + pdh_flash_bwd seeded by
                        the joint's last param: (out, *grads)
  contraction-epilogue  operand packs (pdh_map_chain: prologue chains,
                        transposes, zero padding of k) + pdh_contract with the
                        epilogue program; several m, n or k dims flatten into
                        one, a single rider dim is the batch
  row-normalization     the softmax input materialized first when it is
                        computed (a dissolved score contraction, or a map
                        chain), then pdh_row_softmax_dt over the reduced dim
  row-statistics        pdh_layernorm_dt with the affine epilogue
  map-chain, stencil    pdh_map_chain (shifted reads as offset views)
  ROWSUM / PLAIN        pdh_reduce_rows
  red bare max / min    pdh_reduce_rows_ex (a softmax's row max a backward
                        joint materializes)
  softmax + PV carves   when they compute banded attention per head (the
                        scores dissolved into the softmax carve, its
                        probabilities read by one contraction carve alone):
                        one pdh_flash_fwd launch for the pair
  red, tl.take          pdh_take_rows for the gather, the rest of the carve
                        as a map chain
  red, tl.scatter_add   pdh_scatter_add_rows (the gather's adjoint: an
                        embedding table's gradient) over stored operands
  red, tl.scan          pdh_scan between two map chains; where the scan meets
                        a reduction, a gather or another scan, the carve is
                        split at its first scan and the operand and the rest
                        run as nested plans. Any other red carve refuses

Layout policy: every value (parameter, boundary, output) is a dense tensor in
its IR type's dim order, so every program's strides are fixed when the
executor is built; a run allocates, launches and frees (a value is released
after its last consumer). A rename is a view (the same memory under new
names). Parameters are converted to the executor's element type once, at
``bind``; the token ids stay int64.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

from . import _lib as L
from . import ewprog
from .hip_tile import Untranslatable, recognize_layernorm
from .tl.dialect import OPS
from .tl.fusion import contract_core, forest_is_closed, match_contraction_epilogue, match_softmax, plan_region
from .tl.ir import Builder, Dim, Region, walk

_TORCH_DT = {"f32": "float32", "bf16": "bfloat16", "f16": "float16"}
_CUS = 256  # MI355X compute units


def _torch():
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("the carved-plan executor launches HIP kernels: no GPU is visible")
    return torch


def _dense_strides(shape) -> list:
    out, acc = [0] * len(shape), 1
    for i in range(len(shape) - 1, -1, -1):
        out[i] = acc
        acc *= shape[i]
    return out


def _strides_by_name(names, shape) -> dict:
    return dict(zip(names, _dense_strides(shape)))


def _strided_view(tt, riders, rows, kd):
    """(batch, row) element strides under which a dense value of type ``tt``
    reads as [batch][rows][k] with k contiguous, or None: its dims must be
    exactly riders + rows + kd, the kd dims innermost in order, and the row
    dims composing into one stride."""
    names = tt.names
    if set(names) != set(riders) | set(rows) | set(kd) or len(names) != len(riders) + len(rows) + len(kd):
        return None
    if tuple(names[len(names) - len(kd):]) != tuple(kd):
        return None
    st = _strides_by_name(names, tt.shape)
    for a, b in zip(rows[:-1], rows[1:]):
        if st[a] != st[b] * tt.dim(b).size:
            return None
    row = st[rows[-1]] if rows else 0
    batch = st[riders[0]] if riders else 0
    return (batch, row)


def _big_tiles(Bs, M, N, kc=64 * 64):
    """The launcher's tile choice (contract_launch in contract.hip): 128 x 128
    workgroup tiles when they give every compute unit one, neither output side
    is 64 or under and a workgroup's k (kc columns) is over 128; 64 x 64
    otherwise."""
    return Bs * -(-M // 128) * -(-N // 128) >= _CUS and M > 64 and N > 64 and kc > 128


# Microseconds per 64-column k tile of one workgroup of the fp32 split kernel
# on MI355X, by workgroups resident on a compute unit: 64 x 64 tiles (up to
# five resident), 128 x 128 tiles (two; one alone runs a little faster).
_SMALL_STEP = {1: 1.7, 2: 2.0, 3: 2.7, 4: 3.4, 5: 4.2}
_BIG_STEP2, _BIG_STEP1 = 5.0, 4.0


def _ksplit_est(B, M, N, kt, S):
    """Estimated microseconds of an fp32 contraction of B (M x N) outputs over
    kt 64-column k tiles run as S k slices: the busiest compute unit's tiles at
    the measured per-tile rates, plus a fixed 4 us, plus the pass that adds
    the S partial planes (S + 1 planes of HBM traffic at 5 TB/s)."""
    kc = -(-kt // S)
    if _big_tiles(B * S, M, N, 64 * kc):
        per = -(-(B * S * -(-M // 128) * -(-N // 128)) // _CUS)
        t = (per // 2) * kc * _BIG_STEP2 + (per % 2) * kc * _BIG_STEP1
    else:
        per = -(-(B * S * -(-M // 64) * -(-N // 64)) // _CUS)
        t = (per // 5) * kc * _SMALL_STEP[5] + (kc * _SMALL_STEP[per % 5] if per % 5 else 0.0)
    fin = (S + 1) * B * M * N * 4 / 5e6 if S > 1 else 0.0
    return 4.0 + t + fin


def _ksplit_order(B, M, N, kt):
    """k slice counts (1..16, none empty, each of at least two k tiles) for
    an fp32 contraction, cheapest first under :func:`_ksplit_est`, a model
    fitted to measured times of the gpt2 gradient's contractions on MI355X."""
    cands = [S for S in range(1, 17) if (S - 1) * -(-kt // S) < kt and (S == 1 or -(-kt // S) >= 2)]
    return sorted(cands, key=lambda S: (_ksplit_est(B, M, N, kt, S), S))


def _view3(tt, riders, rows, kd):
    """(batch, row, k) element strides under which a dense value of type
    ``tt`` reads as [batch][rows][k] in place, or None: its dims must be
    exactly riders + rows + kd, in any order, with the row dims composing into
    one stride and the k dims into another, and one of those two strides 1
    (k contiguous, or the rows: a transposed tensor). The fp32 contraction
    reads such operands directly (pdh_contract_views)."""
    names = tt.names
    if set(names) != set(riders) | set(rows) | set(kd) or len(names) != len(riders) + len(rows) + len(kd):
        return None
    st = _strides_by_name(names, tt.shape)

    def one(group):
        for a, b in zip(group[:-1], group[1:]):
            if st[a] != st[b] * tt.dim(b).size:
                return None
        return st[group[-1]]

    row = one(rows) if rows else 1  # a single row: any stride reads it
    kst = one(kd)
    if row is None or kst is None or (row != 1 and kst != 1):
        return None
    return (st[riders[0]] if riders else 0, row, kst)


def _holds_reduce(node) -> bool:
    """Whether a tl.reduce (a dissolved carve) feeds ``node``'s values. The
    second operand of tl.repeat_like only gives the broadcast its shape and
    is never read, so a contraction there does not count."""
    stack, seen = [node], set()
    while stack:
        n = stack.pop()
        if id(n) in seen or not hasattr(n, "op"):
            continue
        seen.add(id(n))
        if n.op == "tl.reduce":
            return True
        if n.op != "core.param":
            stack.extend(n.args[:1] if n.op == "tl.repeat_like" else n.args)
    return False


def _stencils_as_windows(k: Region) -> Region:
    """The carve with every tl.stencil written as a window over a pad of its
    operand: stencil(x)[c, j] = x[c + dil j] inside x's domain, else the fill,
    is window(pad(x, fill))[c, j] over a pad wide enough for every tap, cut
    back to x's domain. Same values; the pads then materialize like any
    other and the window is read in place."""
    b = Builder(OPS)
    memo: dict = {id(p): p for p in k.params}

    def go(n):
        if id(n) in memo:
            return memo[id(n)]
        args = tuple(go(a) for a in n.args)
        if n.op == "tl.stencil":
            (x,) = args
            name, dil = n.attr("name"), int(n.attr("dilation", 1))
            kmin, kmax = (int(v) for v in n.attr("k"))
            d = x.type.dim(name)
            lo, hi = min(d.start, d.start + dil * kmin), max(d.stop, d.stop + dil * kmax)
            pad = b.emit("tl.pad", x, extents=((name, (lo, hi)),), fill=float(n.attr("fill", 0.0)))
            out = b.emit("tl.window", pad, name=name, k_name=n.attr("k_name") or f"{name}_k", k=(kmin, kmax + 1),
                         dilation=dil)
            od = out.type.dim(name)
            if (od.start, od.stop) != (d.start, d.stop):
                out = b.emit("tl.slice", out, ranges=((name, (d.start, d.stop)),))
        elif all(x is y for x, y in zip(args, n.args)):
            out = n
        else:
            explicit = {} if OPS[n.op].type_rule is not None else {"type": n.type}
            out = b.emit(n.op, *args, regions=n.regions, loc=n.loc, **explicit, **dict(n.attrs))
        memo[id(n)] = out
        return out

    return Region(params=k.params, body=(go(k.body[-1]),))


def _yielding(k: Region, node) -> Region:
    """The region over k's params that yields ``node``."""
    return Region(params=k.params, body=(Builder(OPS).emit("core.yield", node),))


def _base(n):
    while n.op == "tl.rename":
        n = n.args[0]
    return n


def _over(view_names, view_shape, lattice) -> list:
    """Element strides of a dense value (dims ``view_names``) over ``lattice``
    (0 where the value lacks a dim: a broadcast)."""
    st = _strides_by_name(view_names, view_shape)
    return [st.get(d.name, 0) for d in lattice]


def _under_renames(n):
    while n.op == "tl.rename":
        n = n.args[0]
    return n


def _band_has_empty_row(T: int, S: int, lo, hi) -> bool:
    import numpy as np

    r = np.arange(T)
    first = np.zeros(T, np.int64) if lo is None else np.maximum(0, r + lo)
    last = np.full(T, S - 1, np.int64) if hi is None else np.minimum(S - 1, r + hi)
    return bool((first > last).any())


@dataclass(frozen=True)
class _AttentionChain:
    """A softmax carve and the contraction carve reading its probabilities,
    launched as one flash forward (``_attention_chains``)."""

    soft: object  # the row-normalization Carve
    pv: object  # the contraction-epilogue Carve
    drop: tuple  # the carves the launch replaces besides pv: soft, and the score carve when there is one
    nodes: tuple  # the model nodes q, k, v
    sources: tuple  # per q, k, v: None (a boundary value, read as is) or (region, bounds) computing it
    bounds: tuple  # every boundary node the launch reads, per q, k, v in turn
    root: object  # the attention output: pv's root
    t: str
    s: str
    e: str
    o: str
    heads: tuple  # the shared head dim (or none)
    band: tuple  # mask_to_band of the closed mask
    fill: float
    merged: tuple | None = None  # (activation, (wq, wk, wv), contracted dim, q scale): one GEMM makes q, k, v


def _merged_projection(q, k, v, t, s, e, o, heads):
    """q, k and v as projections of one activation by three weight params,
    q optionally times a positive constant (the attention scale folded into
    q): (activation, (wq, wk, wv), contracted dim, scale), or None. The
    three then come out of one GEMM over the concatenated weights (a third
    of the launches, three times the workgroups), and the scale moves into
    the flash launch (it multiplies q.k in fp32 there instead of q before
    rounding)."""
    scale = 1.0
    if q.op == "tl.pointwise" and q.attr("f") == "mul" and len(q.args) == 2:
        x, c = q.args
        if c.op not in ("core.const", "tl.const"):
            x, c = c, x
        if c.op in ("core.const", "tl.const") and float(c.attr("value")) > 0:
            q, scale = x, float(c.attr("value"))
    acts, ws, dn = [], [], None
    for node, rows, feat in ((q, t, e), (k, s, e), (v, s, o)):
        core = contract_core(node)
        if core is None:
            return None
        x, y, d = core
        w, a = (x, y) if feat in x.type.names else (y, x)
        if w.op != "core.param" or dn not in (None, d) or set(w.type.names) != {d, feat, *heads}:
            return None
        if tuple(a.type.names) != (rows, d) or a.type.dim(d).start != 0:
            return None
        dn = d
        acts.append(_under_renames(a))
        ws.append(w)
    if not (acts[0] is acts[1] is acts[2]) or tuple(acts[0].type.names) != (t, dn):
        return None
    return acts[0], tuple(ws), dn, scale


def _attention_chains(carves, region, dtype: str, merge: bool = True) -> list:
    """Banded attention that the reference plan carves in two or three: a
    row-normalization carve softmax_s(where(mask, sum_e q*k, fill)) whose
    score contraction is dissolved into it (over boundary values q and k) or
    carved on its own (a contraction carve with no epilogue, read by the
    softmax alone), and a contraction carve sum_s p*v over its probabilities
    p and a boundary value v (partition.py:458-607 on the attention of
    zoo/gpt2.py, the traffic gate choosing between the two forms: the head
    dim keeps fusion.py:480-539's flash matcher from claiming it whole). Per head
    the pair is flash attention, so the executor launches pdh_flash_fwd once
    for it instead of a score GEMM, a row softmax and a PV GEMM, and the
    (t, s) scores never reach HBM.

    A pair is bound only where that is exact: a closed mask forest that is a
    band with a live key in every row; a fill at or below -1e6 (a masked
    score then adds exp(fill - max) == 0 in fp32, so dead key tiles may be
    skipped); the probabilities read by the PV carve alone and yielded by
    nothing; no artifacts; t and s starting at 0; at most one shared head
    dim; and the flash kernel's widths (16-bit: e == od in {64, 128}; fp32:
    od <= 512). q, k and v are boundary values, or values the carves compute
    from theirs (a projection the traffic gate dissolved into its consumer):
    those are extracted as regions and materialized first."""
    from .hip_tile import mask_to_band
    from .tl.partition import extract

    def source(x, carve):
        cb = {id(n) for n in carve.bounds}
        if id(x) in cb:
            return None, (x,)
        members, todo = set(), [x]
        while todo:
            n = todo.pop()
            if id(n) in members or id(n) in cb:
                continue
            members.add(id(n))
            todo.extend(n.args)
        sub, sb = extract(x, members)
        return (sub, sb), sb

    reads: dict = {}
    for c in carves:
        for b in c.bounds:
            i = id(_under_renames(b))
            reads[i] = reads.get(i, 0) + 1
    y = region.body[-1].args[0]
    yielded = {id(_under_renames(x)) for x in (y.args if y.op == "core.tuple" else (y,))}
    soft = {id(c.root): c for c in carves if c.root is not None and c.group.template == "row-normalization"}
    contr = {id(c.root): c for c in carves if c.root is not None and c.group.template == "contraction-epilogue"}
    out = []
    for c in carves:
        if c.root is None or c.group.template != "contraction-epilogue" or c.artifacts:
            continue
        core = contract_core(c.root)
        if core is None:
            continue
        x, w, s = core
        pairs = [(p, v) for p, v in ((x, w), (w, x)) if id(p) in soft]
        if len(pairs) != 1:
            continue
        pr, v = pairs[0]
        sc = soft[id(pr)]
        if sc.artifacts or reads.get(id(pr)) != 1 or id(pr) in yielded:
            continue
        sm = match_softmax(pr)
        if sm is None or sm["s"] != s:
            continue
        wh = sm["sm"]
        if wh.op != "tl.pointwise" or wh.attr("f") != "where" or len(wh.args) != 3:
            continue
        mask, scores, fill = wh.args
        if fill.op not in ("core.const", "tl.const") or float(fill.attr("value")) > -1e6:
            continue
        if not forest_is_closed(mask):
            continue
        core2 = contract_core(scores)
        if core2 is None:
            continue
        a, b, e = core2
        q, k = (b, a) if s in a.type.names else (a, b)
        drop, qk_carve = (sc,), sc
        if id(scores) in {id(n) for n in sc.bounds}:  # the scores carved on their own
            scc = contr.get(id(scores))
            if scc is None or scc.artifacts or reads.get(id(scores)) != 1 or id(scores) in yielded:
                continue
            drop, qk_carve = (sc, scc), scc
        if id(v) == id(pr):
            continue
        qn, kn, vn, on = (tuple(n.type.names) for n in (q, k, v, c.root))
        heads = tuple(d for d in qn if d != e and d in kn)
        ts = [d for d in qn if d not in heads and d != e]
        os_ = [d for d in vn if d not in heads and d != s]
        if len(heads) > 1 or len(ts) != 1 or len(os_) != 1 or s in qn:
            continue
        t, o = ts[0], os_[0]
        if set(kn) != {s, e, *heads} or set(vn) != {s, o, *heads} or set(on) != {t, o, *heads}:
            continue
        if any(n.type.dim(h) != q.type.dim(h) for n in (k, v) for h in heads) or v.type.dim(s) != k.type.dim(s):
            continue
        if q.type.dim(t).start != 0 or k.type.dim(s).start != 0:
            continue
        T, S, E, OD = q.type.dim(t).size, k.type.dim(s).size, q.type.dim(e).size, v.type.dim(o).size
        if (dtype != "f32" and not (E == OD and E in (64, 128))) or OD > 512:
            continue
        try:
            band = mask_to_band(mask, t, s, T, S)
        except Untranslatable:
            continue
        if band[0] == "band" and _band_has_empty_row(T, S, band[1], band[2]):
            continue
        srcs = [source(q, qk_carve), source(k, qk_carve), source(v, c)]
        bounds = tuple(b for _, bs in srcs for b in bs)
        merged = None
        if merge and all(x is not None for x, _ in srcs):  # all computed: one GEMM where they share an activation
            merged = _merged_projection(q, k, v, t, s, e, o, heads)
            if merged is not None:
                bounds = (merged[0],) + merged[1]
        out.append(_AttentionChain(sc, c, drop, (q, k, v), tuple(x for x, _ in srcs), bounds,
                                   c.root, t, s, e, o, heads, band, float(fill.attr("value")), merged))
    return out


@dataclass
class _Pack:
    """One contraction operand laid out [batch][rows][kp] (k contiguous, zero
    past k): the input itself (``direct``), or a map-chain program over the
    kernel's params; a dissolved contraction in the operand's chain is first
    materialized by ``pre`` (its value is program slot None, or used as is
    when ``pre_direct``)."""

    direct: int | None  # kernel param index used as is
    prog: object = None
    slots: tuple = ()  # kernel param index per program operand (None: the pre value)
    shape: tuple = ()
    zero: bool = False
    pre: object = None
    pre_direct: bool = False
    strides: tuple = ()  # (batch, row) element strides of the operand as the product reads it
    pro: object = None  # (program over (batch, rows, k), slots): computed in the k loop, never stored


@dataclass
class Step:
    """One launched carve: ``ins`` are value ids (positional per kernel param),
    ``outs`` the value ids it defines (its root, then artifacts or the other
    outputs of a joint), in the order ``run`` returns them."""

    kind: str
    ins: tuple
    outs: tuple
    run: object = field(repr=False)
    source: str = ""


class PlanExecutor:
    """Runs a ModelPlan of ``region`` on the device. ``dtype`` is the element
    type of every floating value (f32, bf16 or f16). ``fuse_attention``
    launches a softmax carve and its PV carve as one flash forward where they
    compute banded attention (``_attention_chains``); ``merge_projections``
    then makes q, k and v with one GEMM where they project one activation.
    ``f32_contract`` (dtype f32) is how the contractions run: "bf16x6" (fp32
    grade, the default), "bf16x3", "bf16" (operands rounded to bf16, fp32
    accumulation and storage: the numerics of a bf16 autocast) or "fma"."""

    def __init__(self, plan, region: Region, dtype: str = "bf16", fuse_attention: bool = True,
                 merge_projections: bool = True, _shared=None, f32_contract: str = "bf16x6"):
        if dtype not in _TORCH_DT:
            raise ValueError(f"dtype {dtype!r}: f32, bf16 or f16")
        from .kernels import F32_CONTRACT

        if f32_contract not in F32_CONTRACT:
            raise ValueError(f"f32_contract {f32_contract!r}: one of {sorted(F32_CONTRACT)}")
        self.f32_contract = f32_contract
        self.region, self.dtype = region, dtype
        self.params = region.params
        self.nested: list = []
        self._bad: list = []
        # weight packs and the ids of the bound floating tensors, shared with nested executors
        self._packs, self._static = _shared if _shared is not None else ({}, set())
        have = {id(p) for p in region.params}
        self.alias: dict = {}  # rename view id -> the value id it reads
        pending = [c for c in plan.carves if c.root is not None]
        rootless = [c for c in plan.carves if c.root is None]
        if rootless:
            raise Untranslatable(f"a multi-output residue cannot run on the device: {rootless[0].group.reason}")
        if fuse_attention:  # a softmax carve and its PV carve as one flash launch
            chains = _attention_chains(pending, region, dtype, merge_projections)
            dropped = {id(d) for ch in chains for d in ch.drop}
            by_pv = {id(ch.pv): ch for ch in chains}
            pending = [by_pv.get(id(c), c) for c in pending if id(c) not in dropped]
        self.steps: list = []
        while pending:
            for c in pending:
                ins = [self._resolve(b, have) for b in c.bounds]
                if all(i is not None for i in ins):
                    st = self._step(c, tuple(ins))
                    self.steps.append(st)
                    have.update(st.outs)
                    pending.remove(c)
                    break
            else:
                raise Untranslatable("plan stalled: a carve's boundary is never produced")
        y = region.body[-1].args[0]
        ys = y.args if y.op == "core.tuple" else (y,)
        self.outputs = tuple(self._resolve(x, have) for x in ys)
        if any(o is None for o in self.outputs):
            raise Untranslatable("an output of the model is not produced by any carve")
        self.single = y.op != "core.tuple"
        last: dict = {}
        for k, st in enumerate(self.steps):
            for i in st.ins:
                last[i] = k
        keep = set(self.outputs)
        self.release = [[i for i, k in last.items() if k == s and i not in keep] for s in range(len(self.steps))]
        self.bound: dict | None = None

    # ------------------------------------------------------------ building

    def _resolve(self, node, have):
        """The value id a boundary node reads: itself, or (a rename) the value
        under it."""
        if id(node) in have:
            return id(node)
        if node.op == "tl.rename":
            src = self._resolve(node.args[0], have)
            if src is not None:
                self.alias[id(node)] = src
                return src
        return None

    def _step(self, carve, ins):
        if isinstance(carve, _AttentionChain):
            run, src = self._attention(carve)
            return Step("flash-chain", ins, (id(carve.root),), run, src)
        tmpl = carve.group.template
        k = carve.kernel
        outs = (id(carve.root),)
        if tmpl == "flash":
            run, src = self._flash(k)
            outs = outs + tuple(id(a) for a in carve.artifacts)
        elif tmpl == "flash-joint":
            run, src = self._flash_joint(k)
            outs = tuple(id(x) for x in k.body[-1].args[0].args)
        elif tmpl == "contraction-epilogue":
            run, src = self._contraction(k)
        elif tmpl == "row-normalization":
            run, src = self._softmax(k)
        elif tmpl == "row-statistics":
            run, src = self._layernorm(k)
        elif tmpl in ("map-chain", "stencil"):
            run, src = self._map_chain(k)
        elif carve.group.confidence == "red" and any(n.op == "tl.scatter_add" for n in walk(k)):
            run, src = self._scatter(k)
        elif carve.group.confidence == "red" and any(n.op == "tl.take" for n in walk(k)):
            run, src = self._take(k)
        elif carve.group.confidence == "red" and any(n.op in ("tl.pad", "tl.stencil") for n in walk(k)):
            # padded views (a stencil's adjoint; a tl.stencil, as a window over a pad of its
            # fill): the pads materialized, then one map chain
            run, src = self._padded(_stencils_as_windows(k))
        elif carve.group.confidence == "red" and any(n.op == "tl.round_to" for n in walk(k)):
            # the precision op (compute vocabulary, so red): one map chain with its round trip
            run, src = self._map_chain(k)
        elif carve.group.confidence == "red" and any(n.op == "tl.scan" for n in walk(k)):
            # the first-occurrence max / min adjoint's prefix count: pdh_scan
            run, src = self._scan(k)
        elif (carve.group.confidence == "red" and k.body[-1].args[0].op == "tl.reduce"
              and k.body[-1].args[0].attr("f") in ("max", "min")):
            # a bare row max / min (a softmax's max a backward joint keeps): pdh_reduce_rows_ex
            run, src = self._bare_reduce(k)
        else:
            raise Untranslatable(f"carve {tmpl} ({carve.group.reason or carve.root_op}) has no device step")
        return Step(tmpl, ins, outs, run, src)

    def _flash(self, k):
        """A flash carve (fusion.py:480-539 over the carve's params): the
        forward kernel with the closed mask bound as a band, the (m, den)
        artifacts when the carve yields them."""
        from . import kernels as K
        from .hip_tile import mask_to_band
        from .tl.fusion import match_flash

        fm = match_flash(k)
        if fm is None:
            raise Untranslatable("flash carve that the flash matcher does not bind")
        t, s_, e, o = fm["t"], fm["s"], fm["e"], fm["o"]
        q_, k_, v_ = fm["q"], fm["k"], fm["v"]
        T, S, E, OD = q_.type.dim(t).size, fm["extent"], q_.type.dim(e).size, v_.type.dim(o).size
        if self.dtype != "f32" and not (E == OD and E in (64, 128)):
            raise Untranslatable(f"{self.dtype} flash needs e == od in {{64, 128}} (got {E}, {OD})")
        band = mask_to_band(fm["mask"], t, s_, T, S)
        kband = None if band[0] == "none" else K.Band(band[1], band[2])
        iq, ik, iv = (self._index(k, x) for x in (q_, k_, v_))
        y = k.body[-1].args[0]
        out_names = (y.args[0] if y.op == "core.tuple" else y).type.names
        arts, fill = fm["artifacts"], fm["fill"]

        def mat(x, names, want, rows, cols):  # a dense (rows, cols) view in the kernel's order
            return (x if names == want else x.t()).contiguous().view(1, 1, rows, cols)

        def run(vals):
            res = K.flash_fwd(mat(vals[iq], q_.type.names, (t, e), T, E), mat(vals[ik], k_.type.names, (s_, e), S, E),
                              mat(vals[iv], v_.type.names, (s_, o), S, OD), scale=1.0, band=kband, fill=fill,
                              want_lse=False, want_artifacts=arts)
            out = res.o.view(T, OD)
            out = out if out_names == (t, o) else out.t().contiguous()
            return (out, res.m.view(T), res.den.view(T)) if arts else (out,)

        return run, f"flash_fwd t={T} s={S} e={E} od={OD} band={band} artifacts={arts}"

    def _attention(self, ch):
        """The pair of ``_attention_chains`` as one pdh_flash_fwd launch: q, k,
        v (materialized first by nested plans where a carve computed them)
        and the output read as [1, heads, rows, features] views of dense
        tensors (copied only where the feature dim is not the innermost or a
        stride breaks the kernel's 16-byte rows)."""
        from . import kernels as K
        from .tl.partition import plan_model

        q_, k_, v_ = ch.nodes
        if ch.merged is not None:
            return self._attention_merged(ch)
        getters, at = [], 0
        for src in ch.sources:
            if src is None:
                getters.append((None, None, at, 1))
                at += 1
            else:
                sub, sb = src
                nested = PlanExecutor(plan_model(sub, dissolve=False), sub, self.dtype,
                                      _shared=(self._packs, self._static), f32_contract=self.f32_contract)
                self.nested.append(nested)
                getters.append((nested, sub, at, len(sb)))
                at += len(sb)

        def operand(vals, g):
            nested, sub, i, n = g
            if nested is None:
                return vals[i]
            return nested._run({id(p): v for p, v in zip(sub.params, vals[i:i + n])}, self._bad)
        t, s_, e, o, heads = ch.t, ch.s, ch.e, ch.o, ch.heads
        T, S, E, OD = q_.type.dim(t).size, k_.type.dim(s_).size, q_.type.dim(e).size, v_.type.dim(o).size
        H = q_.type.dim(heads[0]).size if heads else 1
        kband = None if ch.band[0] == "none" else K.Band(ch.band[1], ch.band[2])
        out_names, out_shape = ch.root.type.names, ch.root.type.shape

        def perm(names, rows, feat):
            return [names.index(h) for h in heads] + [names.index(rows), names.index(feat)]

        plans = [perm(n.type.names, r, f) for n, r, f in ((q_, t, e), (k_, s_, e), (v_, s_, o))]
        oplan = perm(out_names, t, o)

        def usable(x):
            return x.stride(-1) == 1 and all(st % 8 == 0 for st in x.stride()[:-1]) and x.data_ptr() % 16 == 0

        def heads4(x):
            return x.unsqueeze(0) if heads else x.unsqueeze(0).unsqueeze(0)

        def run(vals):
            torch = _torch()
            ops = []
            for g, pm in zip(getters, plans):
                xv = operand(vals, g).permute(*pm)
                ops.append(heads4(xv if usable(xv) else xv.contiguous()))
            out = torch.empty(out_shape, dtype=ops[0].dtype, device=ops[0].device)
            ov = out.permute(*oplan)
            direct = usable(ov)
            o4 = heads4(ov) if direct else None
            res = K.flash_fwd(*ops, scale=1.0, band=kband, fill=ch.fill, want_lse=False, out=o4)
            if not direct:
                ov.copy_(res.o.view(ov.shape))
            return (out,)

        made = "".join("b" if x is None else "m" for x in ch.sources)
        return run, (f"flash_fwd (softmax + PV carves) heads={H} t={T} s={S} e={E} od={OD} band={ch.band} "
                     f"qkv={made}")

    def _attention_merged(self, ch):
        """An attention chain whose q, k, v are projections of one activation:
        one GEMM against the weights concatenated along n (packed once per
        bind), q, k and v read as strided views of its output, then the flash
        launch with q's scale."""
        from . import kernels as K
        from .tl.ir import TensorType

        act, ws, dn, scale = ch.merged
        t, e, o, heads = ch.t, ch.e, ch.o, ch.heads
        T, D = act.type.dim(t).size, act.type.dim(dn).size
        H = ws[0].type.dim(heads[0]).size if heads else 1
        E, OD = ws[0].type.dim(e).size, ws[2].type.dim(o).size
        widths = (H * E, H * E, H * OD)
        NT = sum(widths)
        b = Builder(OPS)
        A = b.param(0, act.type)
        Bt = b.param(1, TensorType((Dim("_qkv", 0, NT), Dim(dn, 0, D))))
        prod = b.emit("tl.pointwise", b.emit("tl.repeat_like", A, Bt), b.emit("tl.repeat_like", Bt, A), f="mul")
        red = b.emit("tl.reduce", prod, dims=(dn,), f="sum")
        gemm, gsrc = self._contraction(Region(params=(A, Bt), body=(b.emit("core.yield", red),)))
        transposed = red.type.names[0] != t
        perms = [[w.type.names.index(h) for h in heads] + [w.type.names.index(f), w.type.names.index(dn)]
                 for w, f in zip(ws, (e, e, o))]
        kband = None if ch.band[0] == "none" else K.Band(ch.band[1], ch.band[2])
        out_names, out_shape = ch.root.type.names, ch.root.type.shape
        oplan = [out_names.index(h) for h in heads] + [out_names.index(t), out_names.index(o)]

        def usable(x):
            return x.stride(-1) == 1 and all(st % 8 == 0 for st in x.stride()[:-1]) and x.data_ptr() % 16 == 0

        def run(vals):
            torch = _torch()
            a, wq, wk, wv = vals
            key = ("qkv", id(wq), id(wk), id(wv))
            bt = self._packs.get(key)
            if bt is None:
                bt = torch.cat([w.permute(*pm).reshape(wd, D) for w, pm, wd in zip((wq, wk, wv), perms, widths)])
                if all(id(w) in self._static for w in (wq, wk, wv)):
                    self._packs[key] = bt
            y = gemm([a, bt])
            y = y.t() if transposed else y  # (T, NT)
            ops, at = [], 0
            for wd, f in zip(widths, (E, E, OD)):
                x = y[:, at:at + wd].reshape(T, H, f).permute(1, 0, 2).unsqueeze(0)  # [1, H, T, f]
                ops.append(x if usable(x) else x.contiguous())
                at += wd
            out = torch.empty(out_shape, dtype=a.dtype, device=a.device)
            ov = out.permute(*oplan)
            ov = ov if heads else ov.unsqueeze(0)
            direct = usable(ov)
            res = K.flash_fwd(*ops, scale=scale, band=kband, fill=ch.fill, want_lse=False,
                              out=ov.unsqueeze(0) if direct else None)
            if not direct:
                ov.copy_(res.o.view(ov.shape))
            return (out,)

        return run, (f"flash_fwd (softmax + PV carves) heads={H} t={T} s={T} e={E} od={OD} band={ch.band} "
                     f"qkv=merged scale={scale:g} [{gsrc}]")

    def _flash_joint(self, k):
        """The flash joint claimed whole: the forward with its artifacts and
        the fused backward seeded by the joint's last param; returns (out,
        *grads) in the joint's yield order."""
        from . import kernels as K
        from .hip_tile import mask_to_band
        from .tl.partition import match_flash_joint

        fj = match_flash_joint(k)
        if fj is None:
            raise Untranslatable("flash-joint carve that the joint matcher does not bind")
        q_, k_, v_ = fj["q"], fj["k"], fj["v"]
        t, s_, e, o = fj["t"], fj["s"], fj["e"], fj["o"]
        T, S, E, OD = q_.type.dim(t).size, k_.type.dim(s_).size, q_.type.dim(e).size, v_.type.dim(o).size
        if self.dtype != "f32" and not (E == OD and E in (64, 128)):
            raise Untranslatable(f"{self.dtype} flash joint needs e == od in {{64, 128}} (got {E}, {OD})")
        band = mask_to_band(fj["mask"], t, s_, T, S)
        kband = None if band[0] == "none" else K.Band(band[1], band[2])
        iq, ik, iv, iseed = (self._index(k, x) for x in (q_, k_, v_, k.params[-1]))
        ys = k.body[-1].args[0].args
        seed_names = k.params[-1].type.names

        def mat(x, names, want, rows, cols):
            return (x if names == want else x.t()).contiguous().view(1, 1, rows, cols)

        def back(x, order, names, rows, cols):  # the kernel's (rows, cols) result in the output's dim order
            x = x.view(rows, cols)
            return x if tuple(names) == order else x.t().contiguous()

        def run(vals):
            q = mat(vals[iq], q_.type.names, (t, e), T, E)
            kk = mat(vals[ik], k_.type.names, (s_, e), S, E)
            v = mat(vals[iv], v_.type.names, (s_, o), S, OD)
            do = mat(vals[iseed], seed_names, (t, o), T, OD)
            res = K.flash_fwd(q, kk, v, scale=1.0, band=kband, fill=fj["fill"], want_artifacts=True)
            dq, dk, dv = K.flash_bwd(q, kk, v, res.o, do, res.lse, m=res.m, den=res.den, scale=1.0, band=kband,
                                     fill=fj["fill"])
            grads = {"q": (dq, (t, e), T, E), "k": (dk, (s_, e), S, E), "v": (dv, (s_, o), S, OD)}
            outs = [back(res.o, (t, o), ys[0].type.names, T, OD)]
            for nm, g in zip(fj["wrt"], ys[1:]):
                x, order, r, c = grads[nm]
                outs.append(back(x, order, g.type.names, r, c))
            return tuple(outs)

        return run, f"flash_fwd + flash_bwd t={T} s={S} e={E} od={OD} band={band} wrt={','.join(fj['wrt'])}"

    def _index(self, region, node):
        return next(i for i, p in enumerate(region.params) if p is node)

    def _map_prog(self, region, root, lattice, out_strides, extra_leaves=()):
        leaves = {id(p): p for p in region.params}
        for n in extra_leaves:
            leaves[id(n)] = n
        try:
            low = ewprog.lower(root, lattice, leaves)
        except ewprog.Unlowerable as exc:
            raise Untranslatable(f"map chain: {exc}") from None
        strides = [_over(op.type.names, op.type.shape, lattice) for op in low.operands]
        return low, low.program(out_strides, strides)

    def _materialize(self, k, node):
        """A callable computing ``node`` (a value inside carve kernel ``k``)
        from k's param values. Carves dissolved into ``node`` (re-derived per
        tile in the reference's plan) are split back out: the sub-region
        yielding it is carved with every claim root materialized
        (plan_model(dissolve=False)) and run by a nested executor."""
        from .tl.partition import plan_model

        sub = _yielding(k, node)
        nested = PlanExecutor(plan_model(sub, dissolve=False), sub, self.dtype, _shared=(self._packs, self._static),
                              f32_contract=self.f32_contract)
        self.nested.append(nested)

        def run(vals):
            return nested._run({id(p): v for p, v in zip(sub.params, vals)}, self._bad)

        return run

    def _padded(self, k):
        """A pointwise carve over tl.pad views (the reference leaves it red:
        tl.pad has no template row). Each pad, inner ones first, is
        materialized once: a buffer of its frame filled with its fill, its
        operand's chain written into the interior by a map chain whose output
        view starts at the operand's frame. The carve's value is then one map
        chain reading the pad buffers through their shifted / sliced views
        (in-bounds offset reads, as a stencil reads its halo). A value that
        a view reads and that is computed inside the carve (a tap's slice of
        a cotangent) is materialized the same way first, densely."""
        y = k.body[-1].args[0]
        if y.op == "core.tuple" or not y.type.names:
            raise Untranslatable("a padded carve with one tensor output")
        views = ("tl.shift", "tl.slice", "tl.select", "tl.window", "tl.decimate", "tl.diagonal", "tl.rename", "tl.stage")

        def under_views(n):
            while n.op in views:
                n = n.args[0]
            return n

        pads, seen, stack, mats = [], set(), [(y, False)], set()
        while stack:  # post-order: a pad (or a viewed value) after those inside its operand
            n, done = stack.pop()
            if done:
                if n.op == "tl.pad":
                    pads.append(n)
                elif n.op in views[:6]:
                    base = under_views(n)
                    if base.op not in ("core.param", "tl.pad") and id(base) not in mats:
                        mats.add(id(base))
                        pads.append(base)
                continue
            if id(n) in seen or not hasattr(n, "op") or n.op == "core.param":
                continue
            seen.add(id(n))
            stack.append((n, True))
            stack.extend((a, False) for a in (n.args[:1] if n.op == "tl.repeat_like" else n.args))
        leaves = {id(p): p for p in k.params}
        idx = {id(p): i for i, p in enumerate(k.params)}
        plans = []
        tdt = _TORCH_DT[self.dtype]

        def chain(x, dims, out_st, out_off):
            try:
                low = ewprog.lower(x, dims, leaves, allow_views=True)
            except ewprog.Unlowerable as exc:
                raise Untranslatable(f"padded carve: {exc}") from None
            slots, views = [], []
            for j, base in enumerate(low.bases):
                st, off = low.operand_view(j, _strides_by_name(base.type.names, base.type.shape))
                if off < 0:
                    raise Untranslatable("a shifted read starts before its tensor")
                slots.append(("p", idx[id(base)]) if id(base) in idx else ("pad", id(base)))
                views.append((st, off))
            return low.program(out_st, [st for st, _o in views]), slots, [o for _s, o in views], out_off, len(low.insns)

        for pad in pads:
            pst = _strides_by_name(pad.type.names, pad.type.shape)
            if pad.op != "tl.pad":  # a viewed value, written densely
                plans.append((pad, chain(pad, pad.type.dims, [pst[d.name] for d in pad.type.dims], 0)))
                leaves[id(pad)] = pad
                continue
            x = pad.args[0]
            off = sum((x.type.dim(nm).start - pad.type.dim(nm).start) * pst[nm] for nm in x.type.names)
            plans.append((pad, chain(x, x.type.dims, [pst[d.name] for d in x.type.dims], off)))
            leaves[id(pad)] = pad
        final = chain(y, y.type.dims, _dense_strides(y.type.shape), 0)
        shape = y.type.shape

        def run(vals):
            torch = _torch()
            from . import kernels as K

            dt = getattr(torch, tdt)
            bufs = {}

            def operand(slot, o):
                t = vals[slot[1]] if slot[0] == "p" else bufs[slot[1]]
                return t.reshape(-1)[o:]

            for pad, (prog, slots, offs, out_off, _n) in plans:
                if pad.op == "tl.pad":
                    buf = torch.full(pad.type.shape, float(pad.attr("fill")), device="cuda", dtype=dt)
                else:
                    buf = torch.empty(pad.type.shape, device="cuda", dtype=dt)
                K.map_chain(prog, [operand(sl, o) for sl, o in zip(slots, offs)], buf.reshape(-1)[out_off:])
                bufs[id(pad)] = buf
            prog, slots, offs, _o, _n = final
            out = torch.empty(shape, device="cuda", dtype=dt)
            K.map_chain(prog, [operand(sl, o) for sl, o in zip(slots, offs)], out)
            return out

        return run, f"padded pads={len(pads)} + map_chain insns={final[4]}"

    def _map_chain(self, k):
        """A map chain or stencil carve: shifted / sliced reads of a value
        are offset views of its one stored tensor."""
        y = k.body[-1].args[0]
        leaves = {id(p): p for p in k.params}
        try:
            low = ewprog.lower(y, y.type.dims, leaves, allow_views=True)
        except ewprog.Unlowerable as exc:
            raise Untranslatable(f"map chain: {exc}") from None
        slots, views = [], []
        for j, base in enumerate(low.bases):
            st, off = low.operand_view(j, _strides_by_name(base.type.names, base.type.shape))
            if off < 0:
                raise Untranslatable("a shifted read starts before its tensor")
            slots.append(self._index(k, base))
            views.append((st, off))
        prog = low.program(_dense_strides(y.type.shape), [st for st, _off in views])
        offs = [off for _st, off in views]
        shape = y.type.shape

        def run(vals):
            torch = _torch()
            from . import kernels as K

            out = torch.empty(shape, device="cuda", dtype=getattr(torch, _TORCH_DT[self.dtype]))
            K.map_chain(prog, [vals[i].reshape(-1)[o:] for i, o in zip(slots, offs)], out)
            return out

        return run, f"map_chain insns={len(low.insns)} shifted={sum(1 for o in offs if o)}"

    def _contraction(self, k, yroot=None, rowred=None):
        """GEMM-shaped contraction with its epilogue (and prologue chains).
        With ``rowred`` = (reducer, outer reduce, outer yield) the epilogue's
        values are not stored but reduced over the contraction's n dims (the
        outer reduce) by row partials (pdh_contract_views_rowred), which a row
        reduction finishes through the outer yield's program."""
        m = match_contraction_epilogue(k)
        if m is None:
            raise Untranslatable("contraction carve does not match the contraction row")
        if m["shape"] != "gemm":
            return self._reduce(k, m, yroot)
        red = m["reduce"]
        kd = (red.attr("dims"),) if isinstance(red.attr("dims"), str) else tuple(red.attr("dims"))
        ca, cb = m["a"], m["b"]
        keep_a = [nm for nm in ca.type.names if nm not in kd]
        keep_b = [nm for nm in cb.type.names if nm not in kd]
        out_names = red.type.names
        riders = [nm for nm in out_names if nm in keep_a and nm in keep_b]
        mdims = [nm for nm in out_names if nm in keep_a and nm not in riders]
        ndims = [nm for nm in out_names if nm in keep_b and nm not in riders]
        if len(riders) > 1:
            raise Untranslatable("contraction-epilogue: at most one batch (rider) dim on the device")
        size = {d.name: d for d in red.type.dims}
        kdim = {nm: ca.type.dim(nm) for nm in kd}
        # absent groups stand in as unit dims, so the lattice is always (batch, m.., n..)
        bdim = size[riders[0]] if riders else Dim("_unit_b", 0, 1)
        if not mdims:
            size["_unit_m"] = Dim("_unit_m", 0, 1)
            mdims = ["_unit_m"]
        if not ndims:
            size["_unit_n"] = Dim("_unit_n", 0, 1)
            ndims = ["_unit_n"]
        B = bdim.size
        M = math.prod(size[nm].size for nm in mdims)
        N = math.prod(size[nm].size for nm in ndims)
        Kx = math.prod(kdim[nm].size for nm in kd)
        KP = -(-Kx // 64) * 64
        if any(kdim[nm].start != 0 for nm in kd):
            raise Untranslatable("contracted dims must start at 0")

        def pack(core, rows_names, nrows):
            """[B][rows][KP] from the operand chain ``core``."""
            lat = (bdim,) + tuple(size[nm] for nm in rows_names) + tuple(kdim[nm] for nm in kd)
            if len(lat) > L.EW_MAX_DIMS:
                raise Untranslatable(f"an operand pack over {len(lat)} dims (max {L.EW_MAX_DIMS})")
            base = _base(core)
            real_rows = [nm for nm in rows_names if not nm.startswith("_unit")]
            if views:  # fp32: any dense view with k or its rows contiguous, read in place
                st = _view3(core.type, riders, real_rows, kd)
            else:
                st = _strided_view(core.type, riders, real_rows, kd) if Kx == KP else None
            if base.op == "core.param" and st is not None:
                return _Pack(direct=self._index(k, base), strides=st)
            pre = None
            if _holds_reduce(core):
                # carves dissolved into this operand (the traffic gate's
                # re-derivation per tile): materialized once, by their own plan
                pre = self._materialize(k, core)
                if st is not None:
                    return _Pack(direct=None, pre=pre, pre_direct=True, strides=st)
            rs = KP * math.prod(size[nm].size for nm in rows_names)
            out_st = [rs if riders else 0]
            acc = KP
            row_st = []
            for nm in reversed(rows_names):
                row_st.insert(0, acc)
                acc *= size[nm].size
            out_st += row_st
            kst, acc = [], 1
            for nm in reversed(kd):
                kst.insert(0, acc)
                acc *= kdim[nm].size
            out_st += kst
            low, prog = self._map_prog(k, core, lat, out_st, extra_leaves=(core,) if pre is not None else ())
            slots = tuple(None if (pre is not None and b is core) else self._index(k, b) for b in low.bases)
            if fuse and pre is None and any(ins[0] != "LOAD" for ins in low.insns):
                # a chain that computes: evaluated in the k loop (pdh_contract_views_pro)
                # over (batch, rows, k); a pure relayout stays a (cacheable) pack
                dense, acc = [], 1
                for d in reversed(lat):
                    dense.insert(0, acc)
                    acc *= d.size
                nr = len(rows_names)
                try:
                    p3 = ewprog.merge_dims(low.program(dense, [_over(op.type.names, op.type.shape, lat)
                                                               for op in low.operands]),
                                           [[0], list(range(1, 1 + nr)), list(range(1 + nr, len(lat)))])
                    return _Pack(None, strides=(0, 0, 1), pro=(p3, slots))
                except ewprog.Unlowerable:
                    pass  # strides that do not flatten: materialized below
            return _Pack(None, prog, slots, (B, nrows, KP), KP != Kx, pre,
                         strides=(nrows * KP, KP, 1) if views else (nrows * KP, KP))

        views = self.dtype == "f32"  # pdh_contract_views: operands in place, any k
        # computed operands in the k loop (pdh_contract_views_pro): fp32, and bf16
        # (where the other operand is read through a one-LOAD program)
        fuse = rowred is None and self.dtype in ("f32", "bf16")
        pa, pb = pack(ca, mdims, M), pack(cb, ndims, N)
        y = k.body[-1].args[0] if yroot is None else yroot
        if y.type.names and set(y.type.names) != set(out_names):
            raise Untranslatable("the epilogue changes the contraction's lattice")
        lat = (bdim,) + tuple(size[nm] for nm in mdims) + tuple(size[nm] for nm in ndims)
        if len(lat) > L.EW_MAX_DIMS:
            raise Untranslatable(f"an epilogue over {len(lat)} dims (max {L.EW_MAX_DIMS})")
        leaves = {id(p): p for p in k.params}
        try:
            epi = ewprog.lower(y, lat, leaves, acc=red, acc_scale=(1.0 / Kx) if m["f"] == "mean" else None)
        except ewprog.Unlowerable as exc:
            raise Untranslatable(f"contraction epilogue: {exc}") from None
        out_st = _over(y.type.names, y.type.shape, lat)
        prog = epi.program(out_st, [_over(op.type.names, op.type.shape, lat) for op in epi.operands])
        groups = [[0], list(range(1, 1 + len(mdims))), list(range(1 + len(mdims), len(lat)))]
        try:
            prog = ewprog.merge_dims(prog, groups)
        except ewprog.Unlowerable as exc:
            raise Untranslatable(f"contraction epilogue: {exc}") from None
        eslots = tuple(self._index(k, b) for b in epi.bases)
        shape = y.type.shape
        tdt = _TORCH_DT[self.dtype]
        # Split k: an fp32 contraction whose output tiles would leave compute
        # units idle or lightly loaded runs S slices of each batch entry's k
        # (whole 64-column tiles, the last ragged) as S workgroups per tile
        # (pdh_contract_views: partial sums into an fp32 workspace
        # [B][S][M][N]), and a map chain adds the slices in order and applies
        # the epilogue; S is the cheapest under the cost model whose sum fits
        # one map-chain program.
        S, fin, ident = 1, None, None
        if views and KP // 64 >= 4 and rowred is None:
            for pick in _ksplit_order(B, M, N, KP // 64):
                fin = ewprog.splitk_sum(prog, pick, (pick * M * N, N, 1)) if pick > 1 else None
                if pick == 1 or fin is not None:
                    break
            if fin is not None:
                S = pick
                ident = L.EwProgram()
                ident.n_insns, ident.n_operands, ident.ndim, ident.out_reg = 1, 0, 3, 0
                for d, (ext, st) in enumerate(zip((B * S, M, N), (M * N, N, 1))):
                    ident.shape[d], ident.out_stride[d] = ext, st
                ident.insns[0].op = L.EW["ACC"]

        def build(p, vals, dt):
            torch = _torch()
            from . import kernels as K

            if p.direct is not None:
                return vals[p.direct]
            if p.pro is not None:
                return None
            pv = p.pre(vals) if p.pre is not None else None
            if p.pre_direct:
                return pv
            ins = [pv if i is None else vals[i] for i in p.slots]
            # a pack of bound parameters only (a weight's transpose) is
            # made once per bind and reused by every run
            key = (id(p), tuple(id(t) for t in ins))
            static = pv is None and all(id(t) in self._static for t in ins)
            if static and key in self._packs:
                return self._packs[key]
            buf = (torch.zeros if p.zero else torch.empty)(p.shape, device="cuda", dtype=dt)
            K.map_chain(p.prog, ins, buf)
            if static:
                self._packs[key] = buf
            return buf

        def how(p):
            if p.pro is not None:
                return "prologue"
            t = "^t" if len(p.strides) == 3 and p.strides[2] != 1 else ""  # read rows-contiguous (transposed)
            return ("direct" + t) if p.direct is not None else (("plan" + t) if p.pre_direct else
                                                                ("plan+pack" if p.pre else "pack"))

        def pro_of(p, vals):
            return None if p.pro is None else (p.pro[0], [vals[i] for i in p.pro[1]])

        src = f"contract batch={B} m={M} n={N} k={Kx} a={how(pa)} b={how(pb)} epilogue={len(epi.insns)}"
        if rowred is not None:
            if not views:
                raise Untranslatable("row partials of a contraction: fp32 only")
            return self._rowred_run(k, rowred, build, pa, pb, prog, eslots, (B, M, N, Kx), bdim, mdims, ndims, size,
                                    riders, src + f" f32={self.f32_contract}")

        def run(vals):
            torch = _torch()
            from . import kernels as K

            dt = getattr(torch, tdt)

            a, bt = build(pa, vals, dt), build(pb, vals, dt)
            pra, prb = pro_of(pa, vals), pro_of(pb, vals)
            out = torch.empty(shape, device="cuda", dtype=dt)

            def views_call(e, ops, o, **kw):
                if pra is None and prb is None:
                    K.contract_views(a, pa.strides, bt, pb.strides, (B, M, N, Kx), e, ops, o, **kw)
                else:
                    K.contract_views_pro(a, pa.strides, bt, pb.strides, (B, M, N, Kx), e, ops, o, pro_a=pra,
                                         pro_b=prb, **kw)

            if S > 1:  # k in S slices: partial sums, then their total through the epilogue
                ws = torch.empty((B * S, M, N), device="cuda", dtype=torch.float32)
                views_call(ident, [], ws, f32_mode=self.f32_contract, ksplit=S)
                flat = ws.reshape(-1)
                K.map_chain(fin, [flat[s_ * M * N:] for s_ in range(S)] + [vals[i] for i in eslots], out)
                return out
            if views:
                views_call(prog, [vals[i] for i in eslots], out, f32_mode=self.f32_contract)
            elif pra is not None or prb is not None:  # bf16: both operands through programs

                def as_prog(p, t, pr, rows):
                    if pr is not None:
                        return pr
                    st = tuple(p.strides) if len(p.strides) == 3 else (p.strides[0], p.strides[1], 1)
                    return K.view_program((B, rows, Kx), st), [t]

                K.contract_views_pro(None, None, None, None, (B, M, N, Kx), prog, [vals[i] for i in eslots], out,
                                     pro_a=as_prog(pa, a, pra, M), pro_b=as_prog(pb, bt, prb, N))
            elif KP == Kx:  # every operand as stored (or as packed), through its strides
                K.contract_strided(a, pa.strides, bt, pb.strides, (B, M, N, Kx), prog,
                                   [vals[i] for i in eslots], out, f32_mode=self.f32_contract)
            else:  # zero-padded packs
                K.contract(a, bt, Kx, prog, [vals[i] for i in eslots], out, f32_mode=self.f32_contract)
            return out

        if S > 1:
            src += f" ksplit={S}"
        if self.dtype == "f32":
            src += f" f32={self.f32_contract}"
        return run, src

    def _rowred_run(self, k, rowred, build, pa, pb, prog, eslots, shape4, bdim, mdims, ndims, size, riders, src):
        """The run of a row reduction over a contraction's epilogue values:
        partials [B][M][ceil(N / 32)] by pdh_contract_views_rowred, then
        pdh_reduce_rows_ex over them with the outer yield's program."""
        reducer, ored, y = rowred
        B, M, N, Kx = shape4
        od = (ored.attr("dims"),) if isinstance(ored.attr("dims"), str) else tuple(ored.attr("dims"))
        if set(od) != set(ndims) or any(nm.startswith("_unit") for nm in ndims):
            raise Untranslatable("the row reduction is not over the contraction's n dims")
        nblk = -(-N // 32)
        row_lat = (bdim,) + tuple(size[nm] for nm in mdims)
        if len(row_lat) + 1 > L.EW_MAX_DIMS:
            raise Untranslatable(f"a row reduction over {len(row_lat) + 1} lattice dims (max {L.EW_MAX_DIMS})")
        # the finishing summand: partial (b, m.., j) at ((b M) + m) nblk + j
        pst, acc = [], nblk
        for nm in reversed(mdims):
            pst.insert(0, acc)
            acc *= size[nm].size
        pst = [M * nblk if riders else 0] + pst + [1]
        ps = L.EwProgram()
        ps.n_insns, ps.n_operands, ps.ndim, ps.out_reg = 1, 1, len(row_lat) + 1, 0
        for d, dim in enumerate(row_lat + (Dim("_blk", 0, nblk),)):
            ps.shape[d], ps.start[d], ps.in_stride[0][d] = dim.size, dim.start, pst[d]
        ps.insns[0].op, ps.insns[0].dst, ps.insns[0].a = L.EW["LOAD"], 0, 0
        leaves = {id(p): p for p in k.params}
        try:
            le = ewprog.lower(y, row_lat, leaves, acc=ored, acc_scale=(1.0 / N) if ored.attr("f") == "mean" else None,
                              allow_views=True)
        except ewprog.Unlowerable as exc:
            raise Untranslatable(f"row reduction: {exc}") from None
        slots, views = [], []
        for j, base in enumerate(le.bases):
            st, off = le.operand_view(j, _strides_by_name(base.type.names, base.type.shape))
            if off < 0:
                raise Untranslatable("a shifted read starts before its tensor")
            slots.append(self._index(k, base))
            views.append((st, off))
        if 1 + len(slots) > L.EW_MAX_OPERANDS:
            raise Untranslatable(f"the row epilogue reads {len(slots)} operands")
        pe = le.program(_over(y.type.names, y.type.shape, row_lat), [st for st, _o in views])
        ps, pe = ewprog.with_slots(ps, 0, 1 + len(slots)), ewprog.with_slots(pe, 1, 1 + len(slots))
        offs = [o for _st, o in views]
        tdt = _TORCH_DT[self.dtype]
        yshape = y.type.shape

        def run(vals):
            torch = _torch()
            from . import kernels as K

            dt = getattr(torch, tdt)
            a, bt = build(pa, vals, dt), build(pb, vals, dt)
            part = torch.empty((B, M, nblk), device="cuda", dtype=torch.float32)
            K.contract_views_rowred(a, pa.strides, bt, pb.strides, (B, M, N, Kx), prog, [vals[i] for i in eslots],
                                    reducer, part, f32_mode=self.f32_contract)
            out = torch.empty(yshape, device="cuda", dtype=dt)
            K.reduce_rows(ps, 1, pe, [part.reshape(-1)] + [vals[i].reshape(-1)[o:] for i, o in zip(slots, offs)],
                          out, reducer)
            return out

        return run, f"{src} rowred={reducer} + reduce_rows blocks={nblk} epilogue={len(le.insns)}"

    def _reduce_rowred(self, k, m, y, reducer):
        """A row reduction whose summand is one contraction under a
        pointwise chain (a softmax's max or denominator over the scores), as
        a contraction whose epilogue is that chain, reduced to row partials;
        Untranslatable when the shape does not fit."""
        red = m["reduce"]
        x = red.args[0]
        inner, stack, seen = [], [x], set()
        while stack:  # the carves under the summand's values
            n = stack.pop()
            if id(n) in seen or not hasattr(n, "op"):
                continue
            seen.add(id(n))
            if n.op == "tl.reduce":
                inner.append(n)
            elif n.op != "core.param":
                stack.extend(n.args[:1] if n.op == "tl.repeat_like" else n.args)
        if len(inner) != 1 or inner[0].attr("f") != "sum":
            raise Untranslatable("the summand is not one contraction under a pointwise chain")
        sub = Region(params=k.params, body=(Builder(OPS).emit("core.yield", x),))
        mm = match_contraction_epilogue(sub)
        if mm is None or mm["shape"] != "gemm" or mm["reduce"] is not inner[0]:
            raise Untranslatable("the summand's contraction is not GEMM-shaped")
        return self._contraction(sub, yroot=x, rowred=(reducer, red, y))

    def _bare_reduce(self, k):
        """A red carve that is one max / min reduction: pdh_reduce_rows_ex over
        its operand chain, or, when the operand holds a dissolved contraction
        (the scores under a softmax's max), over that operand materialized
        first by its own plan."""
        red = k.body[-1].args[0]
        f, x = red.attr("f"), red.args[0]
        if not _holds_reduce(x):
            return self._reduce(k, {"reduce": red, "a": x, "f": f, "shape": f"bare-{f}"}, reducer=f)
        if self.dtype == "f32":
            try:  # the scores never materialized: row partials of the contraction
                return self._reduce_rowred(k, {"reduce": red, "a": x, "f": f, "shape": f"bare-{f}"}, red, f)
            except Untranslatable:
                pass
        pre = self._materialize(k, x)
        b = Builder(OPS)
        xp = b.param(0, x.type)
        r2 = b.emit("tl.reduce", xp, dims=red.attr("dims"), f=f)
        sub = Region(params=(xp,), body=(b.emit("core.yield", r2),))
        run2, src = self._reduce(sub, {"reduce": r2, "a": xp, "f": f, "shape": f"bare-{f}"}, reducer=f)

        def run(vals):
            return run2([pre(vals)])

        return run, f"{src} input=plan"

    def _reduce_materialized(self, k, m, y, reducer):
        """A row reduction whose summand holds a dissolved contraction (the
        probabilities under a softmax backward's rowsum): the summand is
        materialized by its own plan, then reduced, with the epilogue, as a
        region over k's params plus that tensor."""
        from .tl.fusion import rebuild_into

        red, x = m["reduce"], m["reduce"].args[0]
        pre = self._materialize(k, x)
        b = Builder(OPS)
        memo = {id(p): b.param(i, p.type) for i, p in enumerate(k.params)}
        xp = b.param(len(k.params), x.type)
        memo[id(x)] = xp
        y2 = rebuild_into(b, memo, y)
        sub = Region(params=tuple(memo[id(p)] for p in k.params) + (xp,), body=(b.emit("core.yield", y2),))
        red2 = next(n for n in walk(sub) if n.op == "tl.reduce" and n.args[0] is xp)
        run2, src = self._reduce(sub, dict(m, reduce=red2, a=xp), reducer=reducer)

        def run(vals):
            return run2(list(vals) + [pre(vals)])

        return run, f"{src} summand=plan"

    def _reduce(self, k, m, yroot=None, reducer="sum"):
        """The ROWSUM / PLAIN contraction shapes: the summand (the product of
        same-space operands, or the one operand chain) summed over the
        contracted dims by pdh_reduce_rows, the epilogue on the sum."""
        red = m["reduce"]
        kd = (red.attr("dims"),) if isinstance(red.attr("dims"), str) else tuple(red.attr("dims"))
        row_dims = tuple(red.type.dims) or (Dim("_unit_r", 0, 1),)
        kdims = tuple(m["a"].type.dim(nm) for nm in kd)
        lat_s = row_dims + kdims
        if len(lat_s) > L.EW_MAX_DIMS:
            raise Untranslatable(f"a reduction over {len(lat_s)} lattice dims (max {L.EW_MAX_DIMS})")
        leaves = {id(p): p for p in k.params}
        y = k.body[-1].args[0] if yroot is None else yroot
        total = math.prod(d.size for d in kdims)
        if _holds_reduce(red.args[0]):
            if self.dtype == "f32":
                try:  # the summand never materialized: row partials of its contraction
                    return self._reduce_rowred(k, m, y, reducer)
                except Untranslatable:
                    pass
            return self._reduce_materialized(k, m, y, reducer)
        try:
            ls = ewprog.lower(red.args[0], lat_s, leaves, allow_views=True)
            le = ewprog.lower(y, row_dims, leaves, acc=red, acc_scale=(1.0 / total) if m["f"] == "mean" else None,
                              allow_views=True)
        except ewprog.Unlowerable as exc:
            raise Untranslatable(f"row reduction: {exc}") from None
        slots, views = [], []
        for low in (ls, le):
            for j, base in enumerate(low.bases):
                st, off = low.operand_view(j, _strides_by_name(base.type.names, base.type.shape))
                if off < 0:
                    raise Untranslatable("a shifted read starts before its tensor")
                slots.append(self._index(k, base))
                views.append((st, off))
        n_s = len(ls.operands)
        if len(slots) > L.EW_MAX_OPERANDS:
            raise Untranslatable(f"summand and epilogue read {len(slots)} operands (max {L.EW_MAX_OPERANDS})")
        ps = ls.program([0] * len(lat_s), [st for st, _o in views[:n_s]])
        pe = le.program(_over(y.type.names, y.type.shape, row_dims), [st for st, _o in views[n_s:]])
        ps, pe = ewprog.with_slots(ps, 0, len(slots)), ewprog.with_slots(pe, n_s, len(slots))
        offs = [o for _st, o in views]
        shape = y.type.shape
        nk = len(kdims)

        def run(vals):
            torch = _torch()
            from . import kernels as K

            out = torch.empty(shape, device="cuda", dtype=getattr(torch, _TORCH_DT[self.dtype]))
            K.reduce_rows(ps, nk, pe, [vals[i].reshape(-1)[o:] for i, o in zip(slots, offs)], out, reducer)
            return out

        return run, f"reduce_rows {m['shape']} rows={math.prod(d.size for d in row_dims)} k={total} " \
                    f"summand={len(ls.insns)} epilogue={len(le.insns)}"

    def _softmax(self, k):
        y = k.body[-1].args[0]
        sm = match_softmax(y)
        if sm is None:
            raise Untranslatable("row-normalization carve without the softmax chain")
        s = sm["s"]
        x = sm["sm"]
        if x.type.names[-1] != s or y.type.names != x.type.names:
            raise Untranslatable("row-normalization: the reduced dim must be the input's last")
        rows = math.prod(d.size for d in x.type.dims[:-1])
        cols = x.type.dim(s).size
        if _base(x).op == "core.param":
            xi = self._index(k, _base(x))
            pre, pre_src = None, "input"
        else:  # a computed input (the dissolved score contraction): materialized first
            sub = _yielding(k, x)
            tmpl = plan_region(sub).groups[0].template
            if tmpl == "contraction-epilogue":
                pre, pre_src = self._contraction(sub)
            else:
                pre, pre_src = self._materialize(k, x), "plan"
            xi = None
        shape = y.type.shape

        def run(vals):
            from . import kernels as K

            xin = vals[xi] if pre is None else pre(vals)
            return K.row_softmax(xin.reshape(rows, cols)).reshape(shape)

        return run, f"row_softmax rows={rows} cols={cols} input={pre_src}"

    def _layernorm(self, k):
        lb = recognize_layernorm(k)
        if lb is None:
            raise Untranslatable("row-statistics carve is not an (affine) layernorm over params")
        x, feat = lb["x"], lb["feat"]
        if x.type.names[-1] != feat:
            raise Untranslatable("row-statistics: the feature dim must be the input's last")
        ix = self._index(k, x)
        ig = None if lb["gamma"] is None else self._index(k, lb["gamma"])
        ib = None if lb["beta"] is None else self._index(k, lb["beta"])
        eps = lb["eps"]
        cols = x.type.dim(feat).size
        y = k.body[-1].args[0]
        if y.type.names != x.type.names:
            raise Untranslatable("row-statistics: the output's dims must follow the input's")

        def run(vals):
            from . import kernels as K

            xin = vals[ix]
            g = None if ig is None else vals[ig]
            b = None if ib is None else vals[ib]
            return K.layernorm(xin.reshape(-1, cols), g, b, eps=eps).reshape(xin.shape)

        return run, f"layernorm cols={cols} eps={eps:g} affine={ig is not None or ib is not None}"

    def _take(self, k):
        takes = [n for n in walk(k) if n.op == "tl.take"]
        specs = []
        for t in takes:
            table, idx = t.args
            if _base(table).op != "core.param" or _base(idx).op != "core.param":
                raise Untranslatable("tl.take over computed operands")
            dim = t.attr("dim")
            if table.type.names[0] != dim:
                raise Untranslatable("tl.take runs along the table's leading dim only")
            specs.append((self._index(k, _base(table)), self._index(k, _base(idx)), t.type.shape))
        y = k.body[-1].args[0]
        shape = y.type.shape
        if y.op == "tl.take":
            low = prog = None
        else:
            low, prog = self._map_prog(k, y, y.type.dims, _dense_strides(shape), extra_leaves=takes)
        tdt = _TORCH_DT[self.dtype]

        def run(vals):
            torch = _torch()
            from . import kernels as K

            bad = torch.zeros(1, dtype=torch.int32, device="cuda")
            got = {}
            for t, (ti, ii, tshape) in zip(takes, specs):
                got[id(t)] = K.take_rows(vals[ti], vals[ii], bad=bad).reshape(tshape)
            self._bad.append(bad)
            if prog is None:
                return got[id(takes[0])]
            ops = [got[id(b)] if id(b) in got else vals[self._index(k, b)] for b in low.bases]
            out = torch.empty(shape, device="cuda", dtype=getattr(torch, tdt))
            K.map_chain(prog, ops, out)
            return out

        return run, f"take_rows x{len(takes)}" + ("" if prog is None else f" + map_chain insns={len(low.insns)}")

    def _scatter(self, k):
        """A red carve that is one tl.scatter_add over stored operands (the
        reference evaluates it on its CPU oracle, indexing.py:223-259):
        pdh_scatter_add_rows, with the consumed index dims leading the values
        and the declared dim leading the result."""
        y = k.body[-1].args[0]
        if y.op != "tl.scatter_add" or sum(n.op == "tl.scatter_add" for n in walk(k)) != 1:
            raise Untranslatable("a tl.scatter_add carve holding other computation")
        vals_n, idx_n = y.args
        if _base(vals_n).op != "core.param" or _base(idx_n).op != "core.param":
            raise Untranslatable("tl.scatter_add over computed operands")
        inames = idx_n.type.names
        over = y.attr("over")
        consumed = tuple(inames) if over is None else ((over,) if isinstance(over, str) else tuple(over))
        if consumed != tuple(inames) or tuple(vals_n.type.names[:len(inames)]) != tuple(inames):
            raise Untranslatable("tl.scatter_add needs every idx dim consumed, leading the values")
        d = y.type.dim(y.attr("dim"))
        if y.type.names[0] != d.name:
            raise Untranslatable("tl.scatter_add's declared dim must lead its result")
        iv, ii = self._index(k, _base(vals_n)), self._index(k, _base(idx_n))
        shape, lo = y.type.shape, d.start
        from .kernels import SCATTER_MAX_IDX

        if math.prod(idx_n.type.shape) > SCATTER_MAX_IDX:
            raise Untranslatable(f"tl.scatter_add over more than {SCATTER_MAX_IDX} positions")

        def run(vals):
            torch = _torch()
            from . import kernels as K

            bad = torch.zeros(1, dtype=torch.int32, device="cuda")
            idx = vals[ii] if lo == 0 else vals[ii] - lo
            out = K.scatter_add_rows(vals[iv], idx, shape[0], bad=bad)
            self._bad.append(bad)
            return out.reshape(shape)

        return run, f"scatter_add_rows rows={shape[0]}"

    def _scan(self, k):
        """A red carve around one tl.scan (the reference serves it on its
        evaluator): the scan's operand chain by pdh_map_chain (or the stored
        param as is), the scan by pdh_scan along its dim, and the rest of the
        carve as a map chain with the scan's result as one more leaf."""
        scans = [n for n in walk(k) if n.op == "tl.scan"]
        if len(scans) != 1 or any(n.op in ("tl.reduce", "tl.take", "tl.fold") for n in walk(k)):
            return self._scan_split(k, scans[0])
        sc = scans[0]
        xs = sc.args[0]
        shape = xs.type.shape
        ax = xs.type.names.index(sc.attr("dim"))
        outer, inner = math.prod(shape[:ax]), math.prod(shape[ax + 1:])
        f, rev = sc.attr("f"), bool(sc.attr("reverse", False))
        if f not in ("sum", "max", "min", "prod", "mean"):
            raise Untranslatable(f"tl.scan {f!r}")
        pre = None if xs.op == "core.param" else self._map_prog(k, xs, xs.type.dims, _dense_strides(shape))
        y = k.body[-1].args[0]
        post = None if y is sc else self._map_prog(k, y, y.type.dims, _dense_strides(y.type.shape), extra_leaves=[sc])
        tdt = _TORCH_DT[self.dtype]

        def run(vals):
            torch = _torch()
            from . import kernels as K

            dt = getattr(torch, tdt)
            if pre is None:
                x = vals[self._index(k, xs)]
            else:
                low, prog = pre
                x = torch.empty(shape, device="cuda", dtype=dt)
                K.map_chain(prog, [vals[self._index(k, b)] for b in low.bases], x)
            s_out = K.scan(x.contiguous(), ax, f, reverse=rev)
            if post is None:
                return s_out
            low2, prog2 = post
            out = torch.empty(y.type.shape, device="cuda", dtype=dt)
            K.map_chain(prog2, [s_out if b is sc else vals[self._index(k, b)] for b in low2.bases], out)
            return out

        src = "scan " + f + (" reverse" if rev else "") + f" along {sc.attr('dim')} [{outer} x {shape[ax]} x {inner}]"
        if pre is not None:
            src = f"map_chain insns={len(pre[0].insns)} + " + src
        if post is not None:
            src += f" + map_chain insns={len(post[0].insns)}"
        return run, src

    def _scan_split(self, k, sc):
        """A red carve in which a scan meets work a map chain cannot hold (a
        reduction, a gather, further scans), split at ``sc``, its first scan
        in program order: the scan's operand (no scan above it) is
        materialized by a nested plan, the scan runs by pdh_scan, and the
        rest of the carve, with the scan's result as one more param, is
        planned again and run by a nested executor. Each level holds one
        scan fewer, so the splitting ends."""
        from .tl.fusion import rebuild_into
        from .tl.partition import plan_model

        xs = sc.args[0]
        shape = xs.type.shape
        ax = xs.type.names.index(sc.attr("dim"))
        f, rev = sc.attr("f"), bool(sc.attr("reverse", False))
        if f not in ("sum", "max", "min", "prod", "mean"):
            raise Untranslatable(f"tl.scan {f!r}")
        operand = None if xs.op == "core.param" else self._materialize(k, xs)
        y = k.body[-1].args[0]
        rest = None
        if y is not sc:
            b = Builder(OPS)
            memo = {id(p): b.param(i, p.type) for i, p in enumerate(k.params)}
            hole = memo[id(sc)] = b.param(len(k.params), sc.type)
            params = tuple(memo[id(p)] for p in k.params) + (hole,)
            region = Region(params=params, body=(b.emit("core.yield", rebuild_into(b, memo, y)),))
            nested = PlanExecutor(plan_model(region, dissolve=False), region, self.dtype,
                                  _shared=(self._packs, self._static), f32_contract=self.f32_contract)
            self.nested.append(nested)
            rest = (region, nested)

        def run(vals):
            from . import kernels as K

            x = vals[self._index(k, xs)] if operand is None else operand(vals)
            s_out = K.scan(x.contiguous(), ax, f, reverse=rev)
            if rest is None:
                return s_out
            region, nested = rest
            return nested._run({id(p): v for p, v in zip(region.params, [*vals, s_out])}, self._bad)

        src = f"split at scan {f}" + (" reverse" if rev else "") + f" along {sc.attr('dim')}"
        nested_parts = [w for w, there in (("operand", operand is not None), ("rest", rest is not None)) if there]
        if nested_parts:
            src += " (" + " and ".join(nested_parts) + " by nested plans)"
        return run, src

    # ------------------------------------------------------------- running

    def bind(self, inputs: list) -> None:
        """Upload / convert the region's params (positional) once: floating
        values to the executor's type, dense in their type order; integer
        arrays (token ids) to int64."""
        torch = _torch()
        dt = getattr(torch, _TORCH_DT[self.dtype])
        bound = {}
        for p, v in zip(self.params, inputs):
            t = torch.as_tensor(v)
            if t.shape != tuple(p.type.shape):
                raise ValueError(f"param {p.attr('index')}: shape {tuple(t.shape)} != {p.type.shape}")
            if t.dtype in (torch.int32, torch.int64):
                t = t.to(device="cuda", dtype=torch.int64)
            else:
                t = t.to(device="cuda", dtype=dt)
            bound[id(p)] = t.contiguous()
        self.bound = bound
        self._graph = None
        self._packs.clear()
        self._static.clear()
        self._static.update(id(t) for t in bound.values() if t.is_floating_point())

    def run(self):
        """One pass over the plan; returns the output (device tensor, dims in
        the region's yield order). Raises if a gather or a scatter-add saw an
        index out of range."""
        if self.bound is None:
            raise RuntimeError("bind() the params first")
        bads: list = []
        out = self._run(self.bound, bads)
        for bad in bads:
            if int(bad.item()) != 0:
                raise IndexError(f"tl.take / tl.scatter_add: {int(bad.item())} index(es) outside the table")
        return out

    def capture(self):
        """Record one pass as a HIP graph (torch.cuda.CUDAGraph over the
        stream every kernel here launches on), so a replay issues the whole
        model with no host work per kernel. A warm-up pass first compiles the
        specialized kernels and fills the weight-pack cache outside the
        capture. Returns the graph's output tensor (rewritten by every
        replay). Re-capture after ``bind``."""
        torch = _torch()
        if self.bound is None:
            raise RuntimeError("bind() the params first")
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self._run(self.bound, [])
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        bads: list = []
        with torch.cuda.graph(graph):
            out = self._run(self.bound, bads)
        self._graph, self._graph_out, self._graph_bads = graph, out, bads
        return out

    def release_graph(self) -> None:
        """Drop the captured graph and the tensors it holds (its output and
        the memory pool torch keeps for it go with the last reference)."""
        self._graph = self._graph_out = self._graph_bads = None

    def replay(self, check: bool = True):
        """Replay the captured pass; with ``check``, synchronize and raise if a
        gather saw an index out of range."""
        if getattr(self, "_graph", None) is None:
            raise RuntimeError("capture() first")
        self._graph.replay()
        if check:
            for bad in self._graph_bads:
                if int(bad.item()) != 0:
                    raise IndexError(f"tl.take / tl.scatter_add: {int(bad.item())} index(es) outside the table")
        return self._graph_out

    def _run(self, bound: dict, bads: list):
        self._bad = bads
        for n in self.nested:
            n._bad = bads
        vals = dict(bound)
        for st, rel in zip(self.steps, self.release):
            got = st.run([vals[i] for i in st.ins])
            for oid, t in zip(st.outs, got if isinstance(got, tuple) else (got,)):
                vals[oid] = t
            for i in rel:
                if i not in bound:
                    vals.pop(i, None)
        outs = tuple(vals[o] for o in self.outputs)
        return outs[0] if self.single else outs

    def sources(self) -> list:
        return [f"{st.kind}: {st.source}" for st in self.steps]


__all__ = ["PlanExecutor", "Step"]
