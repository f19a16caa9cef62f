# Portions of this file restate, statement for statement, code from
# habemus-papadum/pdum_dsl (packages/tensorlib/src/pdum/tl/launch.py: _tri_apply, fit_affine), which is distributed under the MIT License:
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
"""Launch plans and the closed-form emptiness engine.

Restates packages/tensorlib/src/pdum/tl/launch.py:
  * the launch plan is DATA: ordered (output dim, tile) pairs on the Group;
    the program count is a product of cdivs, never chosen (launch.py:1-22);
  * feasibility is analytic: per-program resident bytes = every tl.stage
    x 2 (double buffer) + every fold carry, at pow2-padded, launch-clipped
    extents, 4-byte items, against the tightest machine level (launch.py:75-92);
  * the proposal ladder walks each output dim, smallest tile above the
    granularity floor first (launch.py:95-124);
  * tri_eval: three-valued interval evaluation of a closed mask forest over
    coordinate boxes (launch.py:138-197); fit_affine: the exact floor-affine
    bound fitter clamp((a + d g) // c) (launch.py:200-227).

The MI355X row: 160 KiB of LDS per CU, 128-byte lines (MI355X_SHARED).
"""

from __future__ import annotations

from dataclasses import dataclass

from .ir import walk_deep

ITEM = 4  # the translated column's item size (f32)


def _pow2(n: int) -> int:
    return 1 << (n - 1).bit_length() if n > 1 else 1


@dataclass(frozen=True)
class TileLevel:
    name: str
    granule: int
    capacity: int
    bandwidth: float | None = None


@dataclass(frozen=True)
class TileMachine:
    levels: tuple

    def tightest(self) -> int:
        return min(lv.capacity for lv in self.levels)


MI355X_SHARED = TileMachine((TileLevel("shared", 128, 160 * 1024, 8.0e12),))


def _clipped(dims, launch: dict) -> int:
    b = ITEM
    for d in dims:
        b *= _pow2(min(launch.get(d.name, d.size), d.size))
    return b


def footprint(region, launch: tuple = ()) -> int:
    lm = dict(launch)
    total = 0
    for n in walk_deep(region):
        if n.op == "tl.stage":
            total += 2 * _clipped(n.type.dims, lm)
        elif n.op == "tl.fold":
            k = len(tuple(n.attr("state")))
            for init in n.args[:k]:
                total += _clipped(init.type.dims, lm)
    return total


def feasible(region, launch, machine: TileMachine) -> tuple[bool, int]:
    fp = footprint(region, launch)
    return fp <= machine.tightest(), fp


def propose(region, machine: TileMachine, floor: int = 1024) -> tuple:
    """Feasible launches, smallest tile first, each output dim in turn."""
    y = region.body[-1].args[0]
    if y.op == "core.tuple":
        y = y.args[0]  # artifacts ride the output's launch
    dims = y.type.dims
    out = []
    for i, lead in enumerate(dims):
        rest = 1
        for j, d in enumerate(dims):
            if j != i:
                rest *= d.size
        found = []
        t = _pow2(lead.size)
        while True:
            if feasible(region, ((lead.name, t),), machine)[0]:
                found.append(((lead.name, t),))
            if t == 1 or rest * t <= floor:
                break
            t //= 2
        out.extend(reversed(found))
    return tuple(out)


# ----------------------------------------------------- emptiness engine

_INF = float("inf")


def tri_eval(n, boxes: dict) -> tuple:
    """("bool", "F"|"T"|"M") or ("num", lo, hi) of a closed forest over
    inclusive integer boxes keyed by dim name. Unspelled ops give "M"."""
    if n.op == "tl.iota":
        lo, hi = boxes[n.attr("name")]
        return ("num", float(lo), float(hi))
    if n.op in ("core.const", "tl.const"):
        v = float(n.attr("value"))
        return ("num", v, v)
    if n.op in ("tl.repeat_like", "tl.repeat"):
        return tri_eval(n.args[0], boxes)
    if n.op == "tl.pointwise":
        return _tri_apply(n.attr("f"), [tri_eval(x, boxes) for x in n.args])
    return ("bool", "M")


def _tri_apply(f, args) -> tuple:
    nums = all(a[0] == "num" for a in args)
    if f in ("le", "lt", "ge", "gt") and nums and len(args) == 2:
        (_, a1, b1), (_, a2, b2) = args
        if f in ("ge", "gt"):
            (a1, b1), (a2, b2) = (a2, b2), (a1, b1)
            f = "le" if f == "ge" else "lt"
        if f == "le":
            return ("bool", "T" if b1 <= a2 else "F" if a1 > b2 else "M")
        return ("bool", "T" if b1 < a2 else "F" if a1 >= b2 else "M")
    if nums:
        iv = [(a[1], a[2]) for a in args]
        if f == "add":
            return ("num", iv[0][0] + iv[1][0], iv[0][1] + iv[1][1])
        if f == "sub":
            return ("num", iv[0][0] - iv[1][1], iv[0][1] - iv[1][0])
        if f == "neg":
            return ("num", -iv[0][1], -iv[0][0])
        if f == "mul":
            c = [x * y for x in iv[0] for y in iv[1]]
            return ("num", min(c), max(c))
        if f == "maximum":
            return ("num", max(iv[0][0], iv[1][0]), max(iv[0][1], iv[1][1]))
        if f == "minimum":
            return ("num", min(iv[0][0], iv[1][0]), min(iv[0][1], iv[1][1]))
        return ("num", -_INF, _INF)
    if all(a[0] == "bool" for a in args):
        ts = [a[1] for a in args]
        if f == "mul":  # AND
            return ("bool", "F" if "F" in ts else "T" if all(t == "T" for t in ts) else "M")
        if f == "maximum":  # OR
            return ("bool", "T" if "T" in ts else "F" if all(t == "F" for t in ts) else "M")
    if f == "where" and len(args) == 3 and args[0][0] == "bool":
        c, a, b = args
        if c[1] == "T":
            return a
        if c[1] == "F":
            return b
        if a[0] == b[0] == "bool":
            return ("bool", a[1] if a[1] == b[1] else "M")
        if a[0] == b[0] == "num":
            return ("num", min(a[1], b[1]), max(a[2], b[2]))
    return ("bool", "M")


def fit_affine(seq, lo_nat: int, hi_nat: int):
    """(a, d, c) with clamp((a + d g) // c, lo_nat, hi_nat) == seq[g] for all g, or None."""
    n = len(seq)
    if n == 1:
        return (seq[0], 0, 1)

    def ok(a, d, c):
        return all(min(hi_nat, max(lo_nat, (a + d * g) // c)) == s for g, s in enumerate(seq))

    for d in sorted({seq[g + 1] - seq[g] for g in range(n - 1)}):  # pure affine first
        for g0 in range(n):
            a = seq[g0] - d * g0
            if ok(a, d, 1):
                return (a, d, 1)
    span = seq[-1] - seq[0]
    for c in range(2, 65):
        d0 = round(span * c / (n - 1))
        for d in (d0 - 1, d0, d0 + 1):
            for g0 in (0, n // 2, n - 1):
                base = seq[g0] * c - d * g0
                for r in range(c):
                    if ok(base + r, d, c):
                        return (base + r, d, c)
    return None
