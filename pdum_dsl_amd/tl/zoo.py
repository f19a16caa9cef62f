"""Subject regions for the template rows, spelled op by op with the Builder.

The reference spells these in packages/tensorlib/src/pdum/tl/zoo/tiles.py
(flash_tile: the hand-written online-softmax tile and its naive twin,
:143-264) and zoo/zoo_common.py (softmax, causal_softmax, layernorm,
:56-86). Masks are CLOSED forms over iota (the template refuses data masks);
the reference fills masked scores with -1e9.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

import numpy as np

from .dialect import OPS, check_tier
from .interp import Field
from .ir import F64, Builder, Region, minus_dim, tensor_type
from .reducers import defreducer, exp, maximum

FILL = -1e9


@dataclass(frozen=True)
class Subject:
    region: Region  # the naive twin (the denotation the planner reads)
    inputs: list  # Field values, positional per param
    oracle: Callable | None = None  # list[np.ndarray] -> np.ndarray (float64 closed form)
    tile: Region | None = None  # a hand-written tile program, where one exists

    def numpy_inputs(self) -> list:
        return [f.arr for f in self.inputs]


def _c(b: Builder, v: float):
    return b.emit("core.const", type=F64, value=float(v))


def scores(b: Builder, q, k, e: str = "e"):
    """sc[t, s] = sum_e q[t, e] k[s, e] — the contract idiom."""
    prod = b.emit("tl.pointwise", b.emit("tl.repeat_like", q, k), b.emit("tl.repeat_like", k, q), f="mul")
    return b.emit("tl.reduce", prod, dims=(e,), f="sum")


def softmax_chain(b: Builder, sm, s: str):
    """div(exp(sm - rl(max_s sm)), rl(sum_s exp(...))) — zoo_common.softmax."""
    mx = b.emit("tl.reduce", sm, dims=(s,), f="max")
    ex = b.emit("tl.pointwise", b.emit("tl.pointwise", sm, b.emit("tl.repeat_like", mx, sm), f="sub"), f="exp")
    den = b.emit("tl.reduce", ex, dims=(s,), f="sum")
    return b.emit("tl.pointwise", ex, b.emit("tl.repeat_like", den, ex), f="div"), mx, den


def mask_forest(b: Builder, lattice, kind, T: int, S: int):
    """A closed mask over the (t, s) lattice:
    "causal"  le(iota_s, iota_t)      "strict" lt(iota_s, iota_t)
    "all"     lt(iota_s, const S)      ("window", W): causal AND t - s < W."""
    it_s = b.emit("tl.iota", lattice, name="s")
    it_t = b.emit("tl.iota", lattice, name="t")
    if kind == "causal":
        return b.emit("tl.pointwise", it_s, it_t, f="le")
    if kind == "strict":
        return b.emit("tl.pointwise", it_s, it_t, f="lt")
    if kind == "all":
        return b.emit("tl.pointwise", it_s, _c(b, S), f="lt")
    if isinstance(kind, tuple) and kind[0] == "window":
        causal = b.emit("tl.pointwise", it_s, it_t, f="le")
        inwin = b.emit("tl.pointwise", b.emit("tl.pointwise", it_t, it_s, f="sub"), _c(b, kind[1]), f="lt")
        return b.emit("tl.pointwise", causal, inwin, f="mul")  # bool AND
    raise ValueError(f"unknown mask kind {kind!r}")


def attention(T=6, S=None, E=3, OD=2, *, mask="causal", artifacts=False, seed=7, scale=1.0) -> Subject:
    """The naive attention region softmax(where(mask, q k^T, -1e9)) v over
    q:(t,e), k:(s,e), v:(s,o) params; ``artifacts`` yields (out, max, den).
    ``scale`` multiplies the drawn q (the template has no score scale)."""
    S = T if S is None else S
    rng = np.random.default_rng(seed)
    Q = scale * rng.standard_normal((T, E))
    Kv = rng.standard_normal((S, E))
    V = rng.standard_normal((S, OD))
    b = Builder(OPS)
    pq = b.param(0, tensor_type(("t", "e"), Q.shape))
    pk = b.param(1, tensor_type(("s", "e"), Kv.shape))
    pv = b.param(2, tensor_type(("s", "o"), V.shape))
    sc = scores(b, pq, pk)
    m = mask_forest(b, sc, mask, T, S)
    sm = b.emit("tl.pointwise", m, sc, _c(b, FILL), f="where")
    pr, mx, den = softmax_chain(b, sm, "s")
    prod = b.emit("tl.pointwise", b.emit("tl.repeat_like", pr, pv), b.emit("tl.repeat_like", pv, pr), f="mul")
    out = b.emit("tl.reduce", prod, dims=("s",), f="sum")
    y = b.emit("core.tuple", out, mx, den) if artifacts else out
    region = Region(params=(pq, pk, pv), body=(b.emit("core.yield", y),))
    inputs = [Field(Q, pq.type.dims), Field(Kv, pk.type.dims), Field(V, pv.type.dims)]

    def oracle(arrs):
        q, k, v = (np.asarray(a, dtype=np.float64) for a in arrs)
        sc = q @ k.T
        t_i, s_i = np.arange(T)[:, None], np.arange(S)[None, :]
        live = {
            "causal": s_i <= t_i,
            "strict": s_i < t_i,
            "all": np.ones((T, S), dtype=bool),
        }.get(mask) if not isinstance(mask, tuple) else (s_i <= t_i) & (t_i - s_i < mask[1])
        sm = np.where(live, sc, FILL)
        p = np.exp(sm - sm.max(axis=1, keepdims=True))
        return (p / p.sum(axis=1, keepdims=True)) @ v

    return Subject(region, inputs, oracle)


def _flash_combine(left, right):
    """The online-softmax merge (zoo/attention.py:40-46): both sides rescaled
    to the joint max; associative."""
    (ml, dl, ol), (mr, dr, or_) = left, right
    m = maximum(ml, mr)
    al, ar = exp(ml - m), exp(mr - m)
    return m, dl * al + dr * ar, ol * al + or_ * ar


# (running max, denominator, weighted sum) over (score, value) elements;
# init is the identity (exp(-1e30 - m) underflows to 0) (zoo/attention.py:54-62)
flashsm = defreducer("zoo.flashsm", state=3, element=2, lift=lambda s, v: (s, 1.0, v), combine=_flash_combine,
                     init=(-1e30, 0.0, 0.0), project=lambda m, den, o: o / den)


def flash_attention(T=5, E=3, OD=2, seed=6) -> Subject:
    """Masked scores fed to the flashsm composite reducer
    (zoo/attention.py:167-196): sm = where(s <= t, q k^T, -1e9), each score
    and value repeated onto the (t, s, o) lattice, reduced over s. Same
    denotation as ``attention(mask="causal")``; the gradient of the reduce
    is the fold adjoint of its lowering."""
    nv = attention(T, T, E, OD, mask="causal", seed=seed)
    b = Builder(OPS)
    pq, pk, pv = (b.param(i, p.type) for i, p in enumerate(nv.region.params))
    sc = scores(b, pq, pk)
    sm = b.emit("tl.pointwise", mask_forest(b, sc, "causal", T, T), sc, _c(b, FILL), f="where")
    se = b.emit("tl.repeat_like", sm, pv)
    ve = b.emit("tl.repeat_like", pv, sm)
    out = b.emit("tl.reduce", se, ve, dims=("s",), f=flashsm.name)
    region = Region(params=(pq, pk, pv), body=(b.emit("core.yield", out),))
    return Subject(region, nv.inputs, nv.oracle)


def flash_tile(T=6, E=3, OD=2, SI=2, seed=7) -> Subject:
    """The hand-written flash tile (zoo/tiles.py:143-264): the causal mask as
    a closed form on a (t, s) lattice built from q, split along s and riding
    as an element source; q as a stride-0 repeat over so; (m, den, o)
    carried through a fold whose step is shared by the o and den finals."""
    from .fusion import FOLD_KW, flash_step

    nv = attention(T, T, E, OD, mask="causal", seed=seed)
    SO = T // SI
    b = Builder(OPS)
    pq = b.param(0, nv.region.params[0].type)
    pk = b.param(1, nv.region.params[1].type)
    pv = b.param(2, nv.region.params[2].type)
    ts = b.emit("tl.repeat", b.emit("tl.select", pq, coords=(("e", 0),)), name="s", extent=T)
    mask = b.emit("tl.pointwise", b.emit("tl.iota", ts, name="s"), b.emit("tl.iota", ts, name="t"), f="le")
    parts = (("so", SO), ("si", SI))
    kt = b.emit("tl.split", pk, name="s", parts=parts)
    vt = b.emit("tl.split", pv, name="s", parts=parts)
    mt = b.emit("tl.split", mask, name="s", parts=parts)
    qr = b.emit("tl.repeat", pq, name="so", extent=SO)
    m0 = b.emit("tl.const", value=-1e30, dims=(("t", T),))
    den0 = b.emit("tl.const", value=0.0, dims=(("t", T),))
    o0 = b.emit("tl.const", value=0.0, dims=(("t", T), ("o", OD)))
    types = (m0.type, den0.type, o0.type, minus_dim(qr.type, "so"), minus_dim(kt.type, "so"),
             minus_dim(vt.type, "so"), minus_dim(mt.type, "so"))
    step = flash_step(types, "e", FILL)
    args = (m0, den0, o0, qr, kt, vt, mt)
    f_o = b.emit("tl.fold", *args, regions=(step,), out=("final", 2), **FOLD_KW)
    f_den = b.emit("tl.fold", *args, regions=(step,), out=("final", 1), **FOLD_KW)
    out = b.emit("tl.pointwise", f_o, b.emit("tl.repeat_like", f_den, f_o), f="div")
    tile = check_tier(Region(params=(pq, pk, pv), body=(b.emit("core.yield", out),)))
    return Subject(nv.region, nv.inputs, nv.oracle, tile)


def row_softmax(rows=4, cols=6, seed=9, names=("t", "s")) -> Subject:
    """softmax over the last name of a 2-D param (test_fusion.py:102-120's subject)."""
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((rows, cols))
    b = Builder(OPS)
    p = b.param(0, tensor_type(names, X.shape))
    pr, _, _ = softmax_chain(b, p, names[-1])
    region = Region(params=(p,), body=(b.emit("core.yield", pr),))

    def oracle(arrs):
        x = np.asarray(arrs[0], dtype=np.float64)
        e = np.exp(x - x.max(axis=1, keepdims=True))
        return e / e.sum(axis=1, keepdims=True)

    return Subject(region, [Field(X, p.type.dims)], oracle)


def layernorm(rows=4, feat=6, *, affine=True, eps=1e-5, seed=2) -> Subject:
    """Two-pass layernorm over feat with the gamma/beta epilogue (zoo_common.py:56-60)."""
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((rows, feat))
    G = 1 + 0.1 * rng.standard_normal(feat)
    Bt = 0.1 * rng.standard_normal(feat)
    b = Builder(OPS)
    px = b.param(0, tensor_type(("t", "d"), X.shape))
    params = [px]
    mu = b.emit("tl.reduce", px, dims=("d",), f="mean")
    xc = b.emit("tl.pointwise", px, b.emit("tl.repeat_like", mu, px), f="sub")
    var = b.emit("tl.reduce", b.emit("tl.pointwise", xc, xc, f="mul"), dims=("d",), f="mean")
    sd = b.emit("tl.pointwise", b.emit("tl.pointwise", var, _c(b, eps), f="add"), f="sqrt")
    y = b.emit("tl.pointwise", xc, b.emit("tl.repeat_like", sd, px), f="div")
    inputs = [Field(X, px.type.dims)]
    if affine:
        pg = b.param(1, tensor_type(("d",), (feat,)))
        pb = b.param(2, tensor_type(("d",), (feat,)))
        y = b.emit("tl.pointwise", y, b.emit("tl.repeat_like", pg, px), f="mul")
        y = b.emit("tl.pointwise", y, b.emit("tl.repeat_like", pb, px), f="add")
        params += [pg, pb]
        inputs += [Field(G, pg.type.dims), Field(Bt, pb.type.dims)]
    region = Region(params=tuple(params), body=(b.emit("core.yield", y),))

    def oracle(arrs):
        x = np.asarray(arrs[0], dtype=np.float64)
        m = x.mean(axis=1, keepdims=True)
        v = ((x - m) ** 2).mean(axis=1, keepdims=True)
        out = (x - m) / np.sqrt(v + eps)
        if affine:
            out = out * np.asarray(arrs[1]) + np.asarray(arrs[2])
        return out

    return Subject(region, inputs, oracle)


def linear_gelu(T=8, D=16, F=12, seed=5) -> Subject:
    """gelu_tanh(x @ w + b): a transformer MLP's up-projection with its bias
    and activation (the contraction-epilogue row's motivating shape, the
    reference's relu(a @ b + bias) subject of test_fusion.py:21-42 with the
    tanh-approximated gelu of gpt2's MLP)."""
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((T, D))
    W = rng.standard_normal((D, F)) * D**-0.5
    Bv = 0.1 * rng.standard_normal(F)
    b = Builder(OPS)
    px = b.param(0, tensor_type(("t", "d"), X.shape))
    pw = b.param(1, tensor_type(("d", "f"), W.shape))
    pb = b.param(2, tensor_type(("f",), Bv.shape))
    prod = b.emit("tl.pointwise", b.emit("tl.repeat_like", px, pw), b.emit("tl.repeat_like", pw, px), f="mul")
    acc = b.emit("tl.reduce", prod, dims=("d",), f="sum")
    z = b.emit("tl.pointwise", acc, b.emit("tl.repeat_like", pb, acc), f="add")
    z3 = b.emit("tl.pointwise", b.emit("tl.pointwise", z, z, f="mul"), z, f="mul")
    inner = b.emit("tl.pointwise", b.emit("tl.pointwise", z, b.emit("tl.pointwise", z3, _c(b, 0.044715), f="mul"),
                                          f="add"), _c(b, 0.7978845608028654), f="mul")
    y = b.emit("tl.pointwise", b.emit("tl.pointwise", z, _c(b, 0.5), f="mul"),
               b.emit("tl.pointwise", b.emit("tl.pointwise", inner, f="tanh"), _c(b, 1.0), f="add"), f="mul")
    region = Region(params=(px, pw, pb), body=(b.emit("core.yield", y),))

    def oracle(arrs):
        zz = np.asarray(arrs[0]) @ np.asarray(arrs[1]) + np.asarray(arrs[2])
        return 0.5 * zz * (1.0 + np.tanh(0.7978845608028654 * (zz + 0.044715 * zz**3)))

    return Subject(region, [Field(X, px.type.dims), Field(W, pw.type.dims), Field(Bv, pb.type.dims)], oracle)


def masked_activation(I=5, J=7, seed=1) -> Subject:
    """where(iota_j > iota_i, tanh(x * s_j) + exp(-|x|), 0): a map chain over
    a broadcast operand, coordinates and a closed mask."""
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((I, J))
    Sv = rng.standard_normal(J)
    b = Builder(OPS)
    x = b.param(0, tensor_type(("i", "j"), (I, J)))
    s = b.param(1, tensor_type(("j",), (J,)))
    t = b.emit("tl.pointwise", b.emit("tl.pointwise", x, b.emit("tl.repeat_like", s, x), f="mul"), f="tanh")
    e = b.emit("tl.pointwise", b.emit("tl.pointwise", b.emit("tl.pointwise", x, f="abs"), f="neg"), f="exp")
    lat = b.emit("tl.const", value=0.0, dims=(("i", I), ("j", J)))
    m = b.emit("tl.pointwise", b.emit("tl.iota", lat, name="j"), b.emit("tl.iota", lat, name="i"), f="gt")
    y = b.emit("tl.pointwise", m, b.emit("tl.pointwise", t, e, f="add"), _c(b, 0.0), f="where")
    region = Region(params=(x, s), body=(b.emit("core.yield", y),))

    def oracle(arrs):
        xx, ss = np.asarray(arrs[0]), np.asarray(arrs[1])
        ii, jj = np.meshgrid(np.arange(xx.shape[0]), np.arange(xx.shape[1]), indexing="ij")
        return np.where(jj > ii, np.tanh(xx * ss) + np.exp(-np.abs(xx)), 0.0)

    return Subject(region, [Field(X, x.type.dims), Field(Sv, s.type.dims)], oracle)


# ------------------------------------------------------------------ gpt2

GELU_C = 0.7978845608028654  # sqrt(2/pi), the tanh-approximated gelu's constant


def np_gelu(x):
    return 0.5 * x * (1 + np.tanh(GELU_C * (x + 0.044715 * x**3)))


def np_layernorm(x, g, beta, eps, axis=-1):
    mu = x.mean(axis=axis, keepdims=True)
    v = ((x - mu) ** 2).mean(axis=axis, keepdims=True)
    return (x - mu) / np.sqrt(v + eps) * g + beta


def np_softmax(s, axis):
    e = np.exp(s - s.max(axis=axis, keepdims=True))
    return e / e.sum(axis=axis, keepdims=True)


@dataclass(frozen=True)
class GPT2Config:
    """The reference's default toy (zoo/gpt2.py:34-42) unless sized up."""

    t: int = 4  # sequence
    d: int = 6  # model width
    nh: int = 2  # heads
    hk: int = 3  # head width
    m: int = 8  # mlp width
    layers: int = 2
    v: int = 5  # vocab (the embedding table is tied to the head)
    eps: float = 1e-5


@dataclass(frozen=True)
class Model:
    """A whole-model subject (zoo_common.py ZooModel): the region, inputs by
    name, the numpy denotation, the output's dim order and the names of the
    region's params."""

    region: Region
    inputs: dict  # name -> np.ndarray in the param's type-dim order
    ref: Callable  # dict[name, ndarray] -> ndarray
    order: tuple
    names: dict  # id(param) -> name

    def values(self) -> list:
        """Inputs positional per region param."""
        return [self.inputs[self.names[id(p)]] for p in self.region.params]


class _B:
    """Tensor-level spellings over the Builder, mirroring compute.py's
    (contract, reduce, repeat_like, pointwise)."""

    def __init__(self):
        self.b = Builder(OPS)

    def pw(self, f, *xs):
        return self.b.emit("tl.pointwise", *xs, f=f)

    def rl(self, x, like):
        return self.b.emit("tl.repeat_like", x, like)

    def red(self, f, x, dims):
        return self.b.emit("tl.reduce", x, dims=(dims,) if isinstance(dims, str) else tuple(dims), f=f)

    def c(self, v):
        return _c(self.b, v)

    def contract(self, x, y, axis):
        """reduce(sum, mul(rl(x, y), rl(y, x)), axis): compute.py:148-154."""
        return self.red("sum", self.pw("mul", self.rl(x, y), self.rl(y, x)), axis)

    def rename(self, x, **mapping):
        return self.b.emit("tl.rename", x, mapping=tuple(sorted(mapping.items())))

    def layernorm(self, x, g, beta, feat, eps):
        """zoo_common.py:56-60, two-pass, eps inside the sqrt."""
        mu = self.red("mean", x, feat)
        xc = self.pw("sub", x, self.rl(mu, x))
        sd = self.pw("sqrt", self.pw("add", self.red("mean", self.pw("mul", xc, xc), feat), self.c(eps)))
        y = self.pw("div", xc, self.rl(sd, x))
        return self.pw("add", self.pw("mul", y, self.rl(g, x)), self.rl(beta, x))

    def causal_softmax(self, sc, q="t", k="s"):
        """zoo_common.py:83-86: le(iota_k, iota_q) mask, fill -1e9, softmax over k."""
        mask = self.pw("le", self.b.emit("tl.iota", sc, name=k), self.b.emit("tl.iota", sc, name=q))
        sm = self.pw("where", mask, sc, self.c(FILL))
        e = self.pw("exp", self.pw("sub", sm, self.rl(self.red("max", sm, k), sm)))
        return self.pw("div", e, self.rl(self.red("sum", e, k), sm))


def gpt2(cfg: GPT2Config = GPT2Config(), seed: int = 7, init: str = "toy") -> Model:
    """GPT-2 from token ids to tied-head logits (zoo/gpt2.py:46-166): embedding
    gather + learned positions, ``layers`` pre-norm blocks (causal attention
    with heads as a dim, gelu MLP), final layernorm, head contracted against
    the embedding table. Inputs draw from ``default_rng(seed)``: ids first,
    then every weight in declaration order. ``init="toy"`` (the reference
    toy's draw): std 0.1 for wpe and 0.4 else. ``init="gpt2"`` (GPT-2's own
    initialization scale): std 0.02 for the projections and wte, 0.01 for
    wpe, layernorm gains 1 + 0.02 z and biases 0.02 z."""
    if init not in ("toy", "gpt2"):
        raise ValueError(f"init {init!r}: 'toy' or 'gpt2'")
    D, H, K, M = cfg.d, cfg.nh, cfg.hk, cfg.m
    rng = np.random.default_rng(seed)
    inputs = {"ids": rng.integers(0, cfg.v, cfg.t)}
    shapes: dict = {}

    def declare(name, **dims):
        shapes[name] = dims
        z = rng.standard_normal(tuple(dims.values()))
        if init == "toy":
            inputs[name] = (0.1 if name == "wpe" else 0.4) * z
        elif name.endswith("g") and "ln" in name:  # a layernorm gain
            inputs[name] = 1.0 + 0.02 * z
        else:
            inputs[name] = (0.01 if name == "wpe" else 0.02) * z

    declare("wte", v=cfg.v, d=D)
    declare("wpe", t=cfg.t, d=D)
    declare("lnfg", d=D)
    declare("lnfb", d=D)
    for i in range(cfg.layers):
        p = f"h.{i}."
        declare(p + "attn.ln1g", d=D)
        declare(p + "attn.ln1b", d=D)
        declare(p + "attn.wq", d=D, nh=H, hk=K)
        declare(p + "attn.wk", d=D, nh=H, hk=K)
        declare(p + "attn.wv", d=D, nh=H, hk=K)
        declare(p + "attn.wo", nh=H, hk=K, d=D)
        declare(p + "mlp.ln2g", d=D)
        declare(p + "mlp.ln2b", d=D)
        declare(p + "mlp.w1", d=D, m=M)
        declare(p + "mlp.b1", m=M)
        declare(p + "mlp.w2", m=M, d=D)
        declare(p + "mlp.b2", d=D)

    t = _B()
    params, names = [], {}
    ids = t.b.param(0, tensor_type(("t",), (cfg.t,)))
    params.append(ids)
    names[id(ids)] = "ids"
    P = {}
    for name, dims in shapes.items():
        p = t.b.param(len(params), tensor_type(tuple(dims), tuple(dims.values())))
        params.append(p)
        names[id(p)] = name
        P[name] = p

    h = t.pw("add", t.b.emit("tl.take", P["wte"], ids, dim="v"), P["wpe"])
    scale = 1.0 / np.sqrt(K)
    for i in range(cfg.layers):
        p = f"h.{i}."
        a = t.layernorm(h, P[p + "attn.ln1g"], P[p + "attn.ln1b"], "d", cfg.eps)
        q = t.contract(a, P[p + "attn.wq"], "d")
        k = t.contract(t.rename(a, t="s"), P[p + "attn.wk"], "d")
        v = t.contract(t.rename(a, t="s"), P[p + "attn.wv"], "d")
        sc = t.contract(t.pw("mul", q, t.c(scale)), k, "hk")
        pr = t.causal_softmax(sc)
        cx = t.contract(pr, v, "s")
        h = t.pw("add", h, t.contract(cx, P[p + "attn.wo"], ("nh", "hk")))
        a2 = t.layernorm(h, P[p + "mlp.ln2g"], P[p + "mlp.ln2b"], "d", cfg.eps)
        u = t.contract(a2, P[p + "mlp.w1"], "d")
        mm = t.pw("zoo.gelu", t.pw("add", u, t.rl(P[p + "mlp.b1"], u)))
        h = t.pw("add", t.pw("add", h, t.contract(mm, P[p + "mlp.w2"], "m")), t.rl(P[p + "mlp.b2"], h))
    hf = t.layernorm(h, P["lnfg"], P["lnfb"], "d", cfg.eps)
    logits = t.contract(hf, P["wte"], "d")
    region = Region(params=tuple(params), body=(t.b.emit("core.yield", logits),))

    T_, eps = cfg.t, cfg.eps

    def ref(inp):
        hh = inp["wte"][inp["ids"]] + inp["wpe"]
        mask = np.tril(np.ones((T_, T_), dtype=bool))
        for i in range(cfg.layers):
            p = f"h.{i}."
            a = np_layernorm(hh, inp[p + "attn.ln1g"], inp[p + "attn.ln1b"], eps)
            q = np.einsum("td,dhk->thk", a, inp[p + "attn.wq"]) / np.sqrt(K)
            kk = np.einsum("sd,dhk->shk", a, inp[p + "attn.wk"])
            vv = np.einsum("sd,dhk->shk", a, inp[p + "attn.wv"])
            sc = np.einsum("thk,shk->tsh", q, kk)
            sc = np.where(mask[:, :, None], sc, FILL)
            pr = np_softmax(sc, axis=1)
            ctx = np.einsum("tsh,shk->thk", pr, vv)
            hh = hh + np.einsum("thk,hkd->td", ctx, inp[p + "attn.wo"])
            a2 = np_layernorm(hh, inp[p + "mlp.ln2g"], inp[p + "mlp.ln2b"], eps)
            mm = np_gelu(a2 @ inp[p + "mlp.w1"] + inp[p + "mlp.b1"])
            hh = hh + mm @ inp[p + "mlp.w2"] + inp[p + "mlp.b2"]
        hf_ = np_layernorm(hh, inp["lnfg"], inp["lnfb"], eps)
        return hf_ @ inp["wte"].T

    return Model(region, inputs, ref, ("t", "v"), names)


# -------------------------------------------------------- tile flagships


@dataclass(frozen=True)
class Flagship:
    """A hand-written tile program beside its naive twin (zoo/tiles.py:32-40)."""

    region: Region  # the tile-tier program
    naive: Region  # the erased idiom: the denotation
    inputs: list  # Field values, positional per param (both regions)
    oracle: Callable  # list[np.ndarray] -> np.ndarray


def stencil_tile(MI: int = 6, NI: int = 8, alpha: float = 0.1, seed: int = 17) -> Flagship:
    """The fused 5-point stencil step (zoo/tiles.py:94-140): the halo u over
    [0, MI+2) x [0, NI+2); neighbor(dx, dy) = u shifted by (-dx, -dy) and
    sliced to the interior [1, MI+1) x [1, NI+1); out = u + alpha * (sum of
    the four neighbors - 4 u). The tile program reads every neighbor from
    the halo staged once to "shared"; the twin reads the param."""
    rng = np.random.default_rng(seed)
    U = rng.standard_normal((MI + 2, NI + 2))

    def body(b, halo):
        def neighbor(dx, dy):
            sh = b.emit("tl.shift", halo, deltas=(("x", -dx), ("y", -dy)))
            return b.emit("tl.slice", sh, ranges=(("x", (1, MI + 1)), ("y", (1, NI + 1))))

        center = neighbor(0, 0)
        ew = b.emit("tl.pointwise", neighbor(0, 1), neighbor(0, -1), f="add")
        ns = b.emit("tl.pointwise", neighbor(1, 0), neighbor(-1, 0), f="add")
        nsum = b.emit("tl.pointwise", ew, ns, f="add")
        lap = b.emit("tl.pointwise", nsum, b.emit("tl.pointwise", _c(b, 4.0), center, f="mul"), f="sub")
        return b.emit("tl.pointwise", center, b.emit("tl.pointwise", _c(b, alpha), lap, f="mul"), f="add")

    b = Builder(OPS)
    ph = b.param(0, tensor_type(("x", "y"), U.shape))
    region = Region(params=(ph,), body=(b.emit("core.yield", body(b, b.emit("tl.stage", ph, level="shared"))),))
    nb = Builder(OPS)
    nh = nb.param(0, tensor_type(("x", "y"), U.shape))
    naive = Region(params=(nh,), body=(nb.emit("core.yield", body(nb, nh)),))

    def oracle(arrs):
        u = np.asarray(arrs[0], dtype=np.float64)
        lap = u[:-2, 1:-1] + u[2:, 1:-1] + u[1:-1, :-2] + u[1:-1, 2:] - 4 * u[1:-1, 1:-1]
        return u[1:-1, 1:-1] + alpha * lap

    return Flagship(check_tier(region), naive, [Field(U, ph.type.dims)], oracle)


def gemm_tile(MI: int = 8, NI: int = 6, K: int = 8, KI: int = 2, seed: int = 13) -> Flagship:
    """The GEMM flagship (zoo/tiles.py:43-91): acc carried through a fold over
    k tiles, both operand slices staged, the contraction as
    repeat_like / mul / reduce; the twin contracts unsplit."""
    KO = K // KI
    rng = np.random.default_rng(seed)
    A = rng.standard_normal((MI, K))
    Bm = rng.standard_normal((K, NI))
    b = Builder(OPS)
    pa = b.param(0, tensor_type(("mi", "k"), A.shape))
    pb = b.param(1, tensor_type(("k", "ni"), Bm.shape))
    at = b.emit("tl.split", pa, name="k", parts=(("ko", KO), ("ki", KI)))
    bt = b.emit("tl.split", pb, name="k", parts=(("ko", KO), ("ki", KI)))
    acc0 = b.emit("tl.const", value=0.0, dims=(("mi", MI), ("ni", NI)))
    sb = Builder(OPS)
    p_acc = sb.param(0, acc0.type)
    p_a = sb.param(1, minus_dim(at.type, "ko"))
    p_b = sb.param(2, minus_dim(bt.type, "ko"))
    a_s = sb.emit("tl.stage", p_a, level="shared")
    b_s = sb.emit("tl.stage", p_b, level="shared")
    prod = sb.emit("tl.pointwise", sb.emit("tl.repeat_like", a_s, b_s), sb.emit("tl.repeat_like", b_s, a_s), f="mul")
    part = sb.emit("tl.reduce", prod, dims=("ki",), f="sum")
    step = Region(params=(p_acc, p_a, p_b), body=(sb.emit("core.yield", sb.emit("tl.pointwise", p_acc, part, f="add")),))
    fold = b.emit("tl.fold", acc0, at, bt, regions=(step,), dim="ko", state=("acc",), element=("a", "b"),
                  out=("final", 0))
    region = Region(params=(pa, pb), body=(b.emit("core.yield", fold),))
    nb = Builder(OPS)
    na = nb.param(0, tensor_type(("mi", "k"), A.shape))
    nbb = nb.param(1, tensor_type(("k", "ni"), Bm.shape))
    nprod = nb.emit("tl.pointwise", nb.emit("tl.repeat_like", na, nbb), nb.emit("tl.repeat_like", nbb, na), f="mul")
    naive = Region(params=(na, nbb), body=(nb.emit("core.yield", nb.emit("tl.reduce", nprod, dims=("k",), f="sum")),))
    return Flagship(check_tier(region), naive, [Field(A, pa.type.dims), Field(Bm, pb.type.dims)],
                    lambda arrs: np.asarray(arrs[0]) @ np.asarray(arrs[1]))
