"""The equivalence harness: certify a tile kernel against its naive twin.

Restates packages/tensorlib/src/pdum/tl/certify.py:567-609 and the stage
erasure of transforms.py:48-78, with the three verdicts:

  proved-exact           normalization (here: stage erasure + exact rewrites)
                         reaches the twin's content key — no numerics;
  proved-licensed        the key is reached through licensed rewrites;
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
from .ir import Builder, Region
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


def _r_fuse_reduce(b, n, args):
    """reduce_f(reduce_f(x, inner), outer) == reduce_f(x, outer + inner) — exact for one monoid."""
    if n.op != "tl.reduce" or args[0].op != "tl.reduce":
        return None
    fo, fi = n.attr("f"), args[0].attr("f")
    if fo != fi or fo not in ("sum", "prod", "max", "min"):
        return None
    d = lambda x: (x,) if isinstance(x, str) else tuple(x)  # noqa: E731
    return b.emit("tl.reduce", args[0].args[0], f=fo, dims=d(n.attr("dims")) + d(args[0].attr("dims")))


_EXACT_RULES = (_r_fuse_reduce,)


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
            out = rule(b, n, args) if not regs else None
            if out is None:
                out = _emit_like(b, n, args, regs)
        memo[id(n)] = out
        return out

    return Region(params=region.params, body=tuple(go(x) for x in region.body))


def normalize(region: Region) -> Region:
    cur = region
    for _ in range(8):
        before = cur.key
        for rule in _EXACT_RULES:
            cur = _rewrite(cur, rule)
        if cur.key == before:
            break
    return cur


def certify(tile: Region, naive: Region, *, licenses=(), families=()) -> Certificate:
    norm_t = normalize(erase_stages(tile))
    norm_n = normalize(naive)
    if norm_t.key == norm_n.key:
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
        got_n = run_region(naive, vals)
        got_t = run_region(tile, vals)
        outs_n = got_n if isinstance(got_n, tuple) else (got_n,)
        outs_t = got_t if isinstance(got_t, tuple) else (got_t,)
        for gt, gn in zip(outs_t, outs_n):
            assert isinstance(gt, Field) and isinstance(gn, Field)
            np.testing.assert_allclose(
                gt.to_numpy(gn.names), gn.arr, rtol=rtol, atol=atol,
                err_msg=f"family {fname!r} exceeded the declared license bound ({', '.join(names)})",
            )
        ran.append(fname)
    if not ran:
        raise ValueError("licensed-differential certification needs adversarial families")
    return Certificate("licensed-differential", names, tuple(ran), False)
