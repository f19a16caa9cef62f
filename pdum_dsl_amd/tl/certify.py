# Portions of this file restate, statement for statement, code from
# habemus-papadum/pdum_dsl (packages/tensorlib/src/pdum/tl/certify.py: _rewrite, normalize), which is distributed under the MIT License:
#
# MIT License
#
# Copyright (c) 2026 Nehal Patel
#
# Permission is hereby granted, free of charge, to any person obtaining a copy
# of this software and associated documentation files (the "Software"), to deal
# in the Software without restriction, including without limitation the rights
# to use, copy, modify, merge, publish, distribute, sublicense, and/or sell
# copies of the Software, and to permit persons to whom the Software is
# furnished to do so, subject to the following conditions:
#
# The above copyright notice and this permission notice shall be included in all
# copies or substantial portions of the Software.
#
# THE SOFTWARE IS PROVIDED "AS IS", WITHOUT WARRANTY OF ANY KIND, EXPRESS OR
# IMPLIED, INCLUDING BUT NOT LIMITED TO THE WARRANTIES OF MERCHANTABILITY,
# FITNESS FOR A PARTICULAR PURPOSE AND NONINFRINGEMENT. IN NO EVENT SHALL THE
# AUTHORS OR COPYRIGHT HOLDERS BE LIABLE FOR ANY CLAIM, DAMAGES OR OTHER
# LIABILITY, WHETHER IN AN ACTION OF CONTRACT, TORT OR OTHERWISE, ARISING FROM,
# OUT OF OR IN CONNECTION WITH THE SOFTWARE OR THE USE OR OTHER DEALINGS IN THE
# SOFTWARE.
"""The equivalence harness: certify a tile kernel against its naive twin.

Restates packages/tensorlib/src/pdum/tl/certify.py:567-609 and the stage
erasure of transforms.py:48-78, with the three verdicts:

  proved-exact           normalization (here: stage erasure + exact rewrites)
                         reaches the twin's content key — no numerics;
  proved-licensed        the key is reached through licensed rewrites (the
                         declared licenses' kinds enable them: a k-tiled
                         accumulation fold inlines back to one sum);
  licensed-differential  normalization stops short (flash's online-softmax
                         lemma is algebra, not syntax), so the declared
                         licenses gate an adversarial differential over the
                         caller's families, tolerances quoted FROM the licenses.

An undeclared deviation refuses loudly.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .dialect import OPS
from .ir import Builder, Region, walk
from .interp import Field, run_region


@dataclass(frozen=True)
class Certificate:
    verdict: str  # "proved-exact" | "proved-licensed" | "licensed-differential"
    licenses: tuple
    families: tuple
    key_reached: bool


def _emit_like(b: Builder, n, args, regs):
    explicit = {} if OPS[n.op].type_rule is not None else {"type": n.type}
    return b.emit(n.op, *args, regions=regs, loc=n.loc, **explicit, **dict(n.attrs))


def erase_stages(region: Region) -> Region:
    """A stage moves residence, never values: rebuild without tl.stage nodes
    (recursing into fold steps); params keep their identity."""
    b = Builder(OPS)
    memo: dict[int, object] = {}

    def rebuild(n):
        if id(n) in memo:
            return memo[id(n)]
        if n.op == "tl.stage":
            out = rebuild(n.args[0])
        elif n.op == "core.param":
            out = n
        else:
            out = _emit_like(b, n, tuple(rebuild(a) for a in n.args), tuple(erase_stages(r) for r in n.regions))
        memo[id(n)] = out
        return out

    return Region(params=region.params, body=tuple(rebuild(x) for x in region.body))


def _dims_of(v) -> tuple:
    return (v,) if isinstance(v, str) else tuple(v)


_ASSOC_COMM = ("sum", "prod", "max", "min")


def _r_fuse_reduce(b, n, args, regs):
    """reduce_f(reduce_f(x, inner), outer) == reduce_f(x, outer + inner) — exact for one monoid."""
    if n.op != "tl.reduce" or args[0].op != "tl.reduce":
        return None
    fo, fi = n.attr("f"), args[0].attr("f")
    if fo != fi or fo not in _ASSOC_COMM:
        return None
    return b.emit("tl.reduce", args[0].args[0], f=fo, dims=_dims_of(n.attr("dims")) + _dims_of(args[0].attr("dims")))


def _r_commute_split(b, n, args, regs):
    """F(split(x), split(y), ...) == split(F(x, y, ...)) for pointwise and
    repeat_like over operands split identically (certify.py:113-128): exact,
    layout ops move coordinates, never values."""
    if n.op not in ("tl.pointwise", "tl.repeat_like"):
        return None
    tens = [x for x in args if x.op != "core.const"]
    if not tens or any(x.op != "tl.split" for x in tens):
        return None
    specs = {(x.attr("name"), tuple(x.attr("parts"))) for x in tens}
    if len(specs) != 1:
        return None
    ((name, parts),) = specs
    inner = tuple(x.args[0] if x.op == "tl.split" else x for x in args)
    return b.emit("tl.split", b.emit(n.op, *inner, **dict(n.attrs)), name=name, parts=parts)


def _r_inline_fold(b, n, args, regs):
    """LICENSED (reassociation; certify.py:131-175): a one-state fold from a
    zero init whose step yields acc + R(elements) is the sum over the scan
    dim of R over the sources. R per slice equals the slice of R over the
    whole sources (pointwise and reduces over other dims commute with the
    fold's absolute select); the sum's re-bracketing is the licensed part."""
    if n.op != "tl.fold" or len(tuple(n.attr("state"))) != 1 or tuple(n.attr("out")) != ("final", 0):
        return None
    init, srcs = args[0], args[1:]
    if init.op != "tl.const" or float(init.attr("value")) != 0.0 or not srcs:
        return None
    step = regs[0]
    if any(x.regions for x in walk(step)):
        return None  # nested control flow: decline, never guess
    p_acc = step.params[0]
    y = step.body[-1].args[0]
    if y.op != "tl.pointwise" or y.attr("f") != "add" or len(y.args) != 2:
        return None
    if y.args[0] is p_acc:
        r = y.args[1]
    elif y.args[1] is p_acc:
        r = y.args[0]
    else:
        return None
    if sum(1 for x in walk(step) for arg in x.args if arg is p_acc) != 1:
        return None  # the carry must be pure accumulation
    sub = {id(p): src for p, src in zip(step.params[1:], srcs)}
    memo: dict[int, object] = {}

    def subst(x):
        if id(x) in sub:
            return sub[id(x)]
        if id(x) not in memo:
            memo[id(x)] = _emit_like(b, x, tuple(subst(g) for g in x.args), ())
        return memo[id(x)]

    return b.emit("tl.reduce", subst(r), f="sum", dims=(n.attr("dim"),))


def _r_cancel_reduce_split(b, n, args, regs):
    """LICENSED (reassociation; certify.py:178-195): a reduce over BOTH parts
    of a split is the reduce over the source dim — the tiling re-bracketed."""
    if n.op != "tl.reduce" or args[0].op != "tl.split" or n.attr("f") not in _ASSOC_COMM:
        return None
    sp = args[0]
    pnames = tuple(p for p, _ in sp.attr("parts"))
    dims = _dims_of(n.attr("dims"))
    if not set(pnames) <= set(dims):
        return None
    newdims = tuple(sp.attr("name") if d == pnames[0] else d for d in dims if d == pnames[0] or d not in pnames)
    return b.emit("tl.reduce", sp.args[0], f=n.attr("f"), dims=newdims)


# (kind, rule): "exact" rules always run; licensed kinds only when declared
_RULES = (
    ("exact", _r_fuse_reduce),
    ("exact", _r_commute_split),
    ("reassociation", _r_inline_fold),
    ("reassociation", _r_cancel_reduce_split),
)


def _rewrite(region: Region, rule) -> Region:
    b = Builder(OPS)
    memo: dict[int, object] = {}

    def go(n):
        if id(n) in memo:
            return memo[id(n)]
        if n.op == "core.param":
            out = n
        else:
            args = tuple(go(a) for a in n.args)
            regs = tuple(_rewrite(r, rule) for r in n.regions)
            out = rule(b, n, args, regs)
            if out is None:
                out = _emit_like(b, n, args, regs)
        memo[id(n)] = out
        return out

    return Region(params=region.params, body=tuple(go(x) for x in region.body))


def normalize(region: Region, kinds: frozenset = frozenset()) -> tuple[Region, frozenset]:
    """The rule set to a content-key fixpoint (certify.py:203-222). ``kinds``
    names the license kinds the caller declared; licensed rules outside it
    never run. Returns (normal form, the licensed kinds actually used)."""
    used: set[str] = set()
    cur = region
    for _ in range(16):
        before = cur.key
        for kind, rule in _RULES:
            if kind != "exact" and kind not in kinds:
                continue
            nxt = _rewrite(cur, rule)
            if nxt.key != cur.key:
                cur = nxt
                if kind != "exact":
                    used.add(kind)
        if cur.key == before:
            break
    return cur, frozenset(used)


def certify(tile: Region, naive: Region, *, licenses=(), families=()) -> Certificate:
    kinds = frozenset(lic.kind for lic in licenses)
    norm_t, used = normalize(erase_stages(tile), kinds)
    norm_n, _ = normalize(naive, kinds)
    if norm_t.key == norm_n.key:
        if used:
            return Certificate("proved-licensed", tuple(sorted(lic.name for lic in licenses if lic.kind in used)), (),
                               True)
        return Certificate("proved-exact", (), (), True)
    if not licenses:
        raise ValueError(
            "unlicensed deviation: normalization did not reach the twin's content key and no license is "
            "declared — a tile program either normalizes to its twin or names its deviation"
        )
    rtol = max(lic.rtol for lic in licenses)
    atol = max(lic.atol for lic in licenses)
    names = tuple(sorted(lic.name for lic in licenses))
    ran = []
    for fname, factory in families:
        vals = list(factory())
        # overflow / invalid / divide-by-zero inside either evaluation means
        # the draw left the operators' domain, where a comparison checks
        # nothing: refuse rather than compare inf or NaN
        try:
            with np.errstate(over="raise", invalid="raise", divide="raise"):
                got_n = run_region(naive, vals)
                got_t = run_region(tile, vals)
        except FloatingPointError as exc:
            raise ValueError(
                f"family {fname!r} left the operators' domain ({exc}): the draw certifies nothing "
                f"({', '.join(names)})"
            ) from None
        outs_n = got_n if isinstance(got_n, tuple) else (got_n,)
        outs_t = got_t if isinstance(got_t, tuple) else (got_t,)
        for gt, gn in zip(outs_t, outs_n):
            assert isinstance(gt, Field) and isinstance(gn, Field)
            want, got = gn.arr, gt.to_numpy(gn.names)
            # a draw outside an operator's domain checks nothing: NaN against
            # NaN would "agree" — such a family refuses instead of passing
            for side, arr in (("naive twin", want), ("tile program", got)):
                if not np.isfinite(arr).all():
                    raise ValueError(
                        f"family {fname!r} left the operators' domain: the {side}'s output is not finite, "
                        f"so the draw certifies nothing ({', '.join(names)})"
                    )
            np.testing.assert_allclose(
                got, want, rtol=rtol, atol=atol, equal_nan=False,
                err_msg=f"family {fname!r} exceeded the declared license bound ({', '.join(names)})",
            )
        ran.append(fname)
    if not ran:
        raise ValueError("licensed-differential certification needs adversarial families")
    return Certificate("licensed-differential", names, tuple(ran), False)
