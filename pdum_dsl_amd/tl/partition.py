"""Whole-model plans: one model region carved into template-shaped groups.

Behaviour follows the reference's packages/tensorlib/src/pdum/tl/partition.py
(``carve_model`` :458-582, ``plan_model`` :586-607); the gpt2 carve counts of
its tests/test_partition.py:38-49 pin it. The implementation is this
module's own: a dependence index built once (``_Deps``), a carver object
that owns the ownership / travel state and climbs a ladder of claim rungs,
a residue split by reverse-topological labelling, and a canonical extraction
that numbers params in the order its own rebuild reaches them.

What a carve is. A claim is (root, members, artifacts): the members are the
interior model nodes one kernel computes, the root the value it
materializes, artifacts extra statistics it surfaces. Zero-cost views
(constants, renames, broadcasts) are shared: they join every claim that
reads them and are re-emitted per kernel, so they never block a claim and a
claim's inputs are always real values.

The ladder (most specific first, so a taller chain keeps its anchor):

  flash          a three-reduce attention composition over any q, k, v
                 values. If an inner value is read outside, the claim
                 survives only by surfacing its row statistics (m, den) and
                 by marking the other leaked values' producer cones as TRAVEL
                 (copies a consumer re-derives); a cone that reduces over a
                 swept dim, or holds anything but map work, cannot travel;
  row-norm       a bare softmax over any input;
  row-stat       a layernorm-shaped statistics chain, its scale-shift tail
                 absorbed downstream;
  contraction    a sum / mean over one or two dims of a product (or of a
                 plain operand): elementwise prologues are absorbed upstream
                 while every reader of the absorbed value is already inside,
                 elementwise epilogues downstream while the output has a
                 single reader.

A claim is admitted only when none of its members is owned already (travel
copies excepted) and no member other than its root is read outside it: one
kernel has one output. The unowned rest is split per weakly connected
component into single-output parts, and a claim whose root only feeds other
claims may then dissolve into them (its members become travel copies) when
re-deriving it per consumer moves fewer elements than writing and reading it
back. ``dissolve=False`` keeps every root materialized.

The MI355X joint claim. The reference carves the autodiff joint of flash
attention into a flash-with-artifacts group plus contraction carves for dV,
dQ, dK and the row statistic D (partition.py:476-557). On MI355X the whole
joint runs as ONE forward-with-artifacts kernel and ONE fused backward
launch, so ``plan_model`` first tries to claim a joint whole, as the carve
``flash-joint``: its first yield must be a ``flash`` composition
(fusion.match_flash over q, k, v params) and the rest of the yield exactly
the vector-Jacobian product of that forward, checked by REGENERATING it with
``autodiff.grad`` and comparing content keys node for node. Plans are data:
what no rung covers becomes a red carve with its reason, never an exception.
"""

from __future__ import annotations

import itertools
from collections import Counter, defaultdict
from dataclasses import dataclass, field
from typing import NamedTuple

from .autodiff import grad, region_names
from .certify import Certificate
from .dialect import OPS
from .fusion import Group, contract_core, forest_is_closed, match_flash, match_rowstat, match_softmax, pick_ki
from .fusion import plan_region, rebuild_into
from .ir import Builder, Region, walk

_CONSTS = frozenset(("core.const", "tl.const"))
# zero-cost views: shared between claims and re-emitted by every kernel that reads them
_VIEWS = _CONSTS | {"tl.rename", "tl.repeat_like", "tl.repeat"}
_TAIL = frozenset(("tl.pointwise", "tl.repeat_like"))  # what extends a claim downstream
_RECOMPUTE = frozenset(("tl.pointwise", "tl.iota"))  # what extends a claim upstream, and may travel


@dataclass(frozen=True)
class Carve:
    """One carved group: the canonical kernel, the plan the recognizer made
    for it, and the claim's footprint in the model."""

    kernel: Region = field(repr=False)
    group: Group
    nodes: int  # interior model nodes counted to this carve (a travel copy counts once, where first held)
    root_op: str
    root: object = field(default=None, repr=False)
    bounds: tuple = field(default=(), repr=False)  # the model values bound to the kernel's params, in order
    artifacts: tuple = field(default=(), repr=False)  # surfaced statistics, in tuple-yield order


@dataclass(frozen=True)
class ModelPlan:
    """A whole-model plan: carves, the interior node count, coverage derived."""

    carves: tuple
    interior: int

    def coverage(self) -> float:
        if self.interior == 0:
            return 1.0
        return sum(c.nodes for c in self.carves if c.group.confidence != "red") / self.interior

    def distinct_kernels(self) -> int:
        return len({c.kernel.key for c in self.carves})


class Claim(NamedTuple):
    """(root, members keyed by node id, surfaced artifacts)."""

    root: object
    members: dict
    artifacts: tuple = ()


def _is_view(n) -> bool:
    return n.op in _VIEWS


def _dims_of(reduce_node) -> frozenset:
    d = reduce_node.attr("dims")
    return frozenset((d,) if isinstance(d, str) else d)


def _extent(t) -> int:
    total = 1
    for d in getattr(t, "dims", ()):
        total *= d.size
    return total


def _strip_broadcast(x):
    """A contraction operand with its broadcasts peeled off."""
    while x.op in ("tl.repeat_like", "tl.repeat"):
        x = x.args[0]
    return x


# --------------------------------------------------------- the dependence index


class _Deps:
    """One region's interior (program order) and every value's readers."""

    def __init__(self, region: Region):
        out = region.body[-1]
        self.exits = {id(out)}
        if out.args[0].op == "core.tuple":
            self.exits.add(id(out.args[0]))
        params = {id(p) for p in region.params}
        self.readers: dict = defaultdict(list)
        self.interior: list = []
        for n in walk(region):
            if id(n) in params:
                continue
            for a in n.args:
                self.readers[id(a)].append(n)
            if n is out or n.op == "core.tuple" or _is_view(n):
                continue
            self.interior.append(n)

    def read_outside(self, v, inside, export=None) -> bool:
        """Does ``v``'s value reach a reader outside ``inside``? Views inside
        only forward the value, so their readers are examined in turn;
        ``export`` (the claim's output) is the sanctioned way out."""
        pending, looked = [v], set()
        while pending:
            x = pending.pop()
            for r in self.readers.get(id(x), ()):
                if r is export:
                    continue
                if id(r) not in inside:
                    return True
                if _is_view(r) and id(r) not in looked:
                    looked.add(id(r))
                    pending.append(r)
        return False

    def value_readers(self, v) -> list:
        """Every reader of ``v``'s value, views included and looked through."""
        found, pending, looked = [], [v], set()
        while pending:
            x = pending.pop()
            for r in self.readers.get(id(x), ()):
                if id(r) in looked:
                    continue
                looked.add(id(r))
                found.append(r)
                if _is_view(r):
                    pending.append(r)
        return found


def _producers(root, stop, within=None) -> dict:
    """``root`` and what it is computed from, up to (excluding) ``stop`` and
    params; with ``within``, only nodes in it (the root always)."""
    got, pending = {}, [root]
    while pending:
        n = pending.pop()
        if id(n) in got or id(n) in stop or n.op == "core.param":
            continue
        if within is not None and n is not root and id(n) not in within:
            continue
        got[id(n)] = n
        pending.extend(n.args)
    return got


def _close(members: dict, travel=()) -> dict:
    """Add the non-constant views members read and the travel copies they
    read, transitively: a claim's inputs are real, materialized values."""
    pending = list(members.values())
    while pending:
        n = pending.pop()
        for a in n.args:
            if id(a) in members:
                continue
            if id(a) in travel or (_is_view(a) and a.op not in _CONSTS):
                members[id(a)] = a
                pending.append(a)
    return members


def _flash_shape(r):
    """The attention composition ending at reduce ``r``:
    sum_s softmax_s(where(mask, sum_e q*k, fill)) * v with a closed mask
    forest and a constant fill. q, k, v are any values (the carve makes
    them params). Returns the bindings or None."""
    outer = contract_core(r)
    if outer is None:
        return None
    probs, v, s = outer
    sm = match_softmax(probs)
    if sm is None or sm["s"] != s:
        return None
    masked = sm["sm"]
    if masked.op != "tl.pointwise" or masked.attr("f") != "where" or len(masked.args) != 3:
        return None
    mask, scores, fill = masked.args
    if fill.op not in _CONSTS or not forest_is_closed(mask):
        return None
    inner = contract_core(scores)
    if inner is None:
        return None
    q, k, e = inner
    qn, kn, vn = q.type.names, k.type.names, v.type.names
    if len(qn) != 2 or kn != (s, e) or len(vn) != 2 or vn[0] != s:
        return None
    (t,) = [d for d in qn if d != e]
    return {"q": q, "k": k, "v": v, "m": sm["max"], "den": sm["den"], "t": t, "s": s}


# ------------------------------------------------------------------ the carver


class _Carver:
    """Ownership state of one carving: the claims made so far, the interior
    node ids they own, and the travel copies (nodes any claim may re-derive)."""

    def __init__(self, region: Region):
        self.region = region
        self.deps = _Deps(region)
        self.claims: list = []
        self.owned: set = set()
        self.travel: dict = {}

    # -- admission

    def _free(self, members) -> bool:
        return all(i not in self.owned or i in self.travel for i in members)

    def _record(self, claim: Claim) -> None:
        self.claims.append(claim)
        self.owned.update(i for i, m in claim.members.items() if not _is_view(m))

    def _admit(self, root, members: dict) -> bool:
        """Record a single-output claim unless a member other than its root
        (or a view or travel copy) is read outside it."""
        _close(members)
        for m in members.values():
            if m is root or _is_view(m) or id(m) in self.travel:
                continue
            if self.deps.read_outside(m, members, root):
                return False
        self._record(Claim(root, members))
        return True

    def _admit_with_statistics(self, root, shape, members: dict) -> bool:
        """A flash claim whose inner values are read outside: it surfaces its
        row statistics, and every other value read outside must be
        re-derivable by its readers (map work, or reductions over neither of
        the claim's swept dims); those producer cones become travel copies."""
        _close(members)
        stats = {id(shape["m"]), id(shape["den"])}
        swept = {shape["t"], shape["s"]}
        copies: dict = {}
        for m in list(members.values()):
            if m is root or id(m) in stats or not self.deps.read_outside(m, members, root):
                continue
            value = m
            while _is_view(value) and value.args:  # a leaked view: the value it forwards
                value = value.args[0]
            if value is root or id(value) in stats or id(value) not in members:
                continue
            cone = _copyable(value, members, stats, swept)
            if cone is None:
                return False
            copies.update(cone)
        self._record(Claim(root, members, (shape["m"], shape["den"])))
        self.travel.update(copies)
        return True

    # -- growth

    def _grow_up(self, members: dict) -> dict:
        """Prologue absorption: unowned elementwise producers join while
        every reader of their value is already inside; travel copies and
        views join unconditionally. Membership only grows and the condition
        only gets easier, so rounds to a fixpoint give the least closure."""
        while True:
            _close(members, self.travel)
            joining = {}
            for m in list(members.values()):
                for a in m.args:
                    if id(a) in members or id(a) in joining or id(a) in self.owned or a.op not in _RECOMPUTE:
                        continue
                    if not self.deps.read_outside(a, members):
                        joining[id(a)] = a
            if not joining:
                return members
            members.update(joining)

    def _grow_down(self, root, members: dict):
        """Epilogue absorption: while the output's single reader is unowned
        elementwise work, it joins and becomes the output. A broadcast of the
        output onto another lattice ends the walk (that is another claim's
        operand); a side operand broadcast onto a member's lattice rides along
        (its value stays an input). Returns the final output."""
        while True:
            readers = self.deps.readers.get(id(root), ())
            if len(readers) != 1:
                return root
            (nxt,) = readers
            if nxt.op not in _TAIL or id(nxt) in self.owned or id(nxt) in self.deps.exits:
                return root
            if nxt.op == "tl.repeat_like" and nxt.args[0] is root:
                return root
            for side in nxt.args:
                if side.op == "tl.repeat_like" and id(side) not in members and id(side.args[1]) in members:
                    members[id(side)] = side
            members[id(nxt)] = nxt
            root = nxt

    # -- the rungs (each called on unowned interior nodes in program order)

    def rung_flash(self, n) -> None:
        if n.op != "tl.reduce":
            return
        shape = _flash_shape(n)
        if shape is None:
            return
        cone = _producers(n, {id(shape["q"]), id(shape["k"]), id(shape["v"])})
        if self._free(cone) and not self._admit(n, dict(cone)):
            self._admit_with_statistics(n, shape, cone)

    def rung_row_norm(self, n) -> None:
        sm = match_softmax(n)
        if sm is None:
            return
        members = _close(_producers(n, {id(sm["sm"])}), self.travel)
        if self._free(members):
            self._admit(n, members)

    def rung_row_stat(self, n) -> None:
        rs = match_rowstat(n)
        if rs is None:
            return
        members = _close(_producers(n, {id(rs["x"])}), self.travel)
        if self._free(members):
            self._admit(self._grow_down(n, members), members)

    def rung_contraction(self, n) -> None:
        if n.op != "tl.reduce" or n.attr("f") not in ("sum", "mean") or n.attr("zero") is not None:
            return
        dims = _dims_of(n)
        if len(dims) not in (1, 2):
            return
        body = n.args[0]
        product = body.op == "tl.pointwise" and body.attr("f") == "mul" and len(body.args) == 2
        operands = [_strip_broadcast(x) for x in body.args] if product else [body]
        for x in operands:  # every operand carries every contracted dim
            if not hasattr(x.type, "dims") or not all(x.type.has(d) for d in dims):
                return
        kept = set()
        for x in operands:
            kept.update(nm for nm in x.type.names if nm not in dims)
        if set(n.type.names) != kept:
            return
        seed = {id(n): n}
        if product:  # a plain sum leaves its operand to absorption: it may be another claim's output
            seed[id(body)] = body
        if any(i in self.owned for i in seed):
            return
        members = self._grow_up(seed)
        self._admit(self._grow_down(n, members), members)

    # -- what the rungs leave

    def split_residue(self) -> None:
        rest = [n for n in self.deps.interior if id(n) not in self.owned]
        for comp in _components(rest):
            self._split(comp)

    def _split(self, comp: list) -> None:
        """Single-output parts of one residue component (``comp`` in program
        order). Walking readers before producers, a node is an output when
        something outside the component reads it, or when its readers inside
        belong to different parts; otherwise it joins its readers' part.
        Each part then takes the views and travel copies it reads."""
        inside = {id(n) for n in comp}
        part: dict = {}
        for n in reversed(comp):
            readers = self.deps.readers.get(id(n), ())
            if any(id(r) not in inside for r in readers):
                part[id(n)] = id(n)
                continue
            labels = {part[id(r)] for r in readers if id(r) in part}
            if len(labels) == 1:
                part[id(n)] = labels.pop()
            elif labels:
                part[id(n)] = id(n)
        groups: dict = {}
        for n in comp:
            if id(n) in part:
                groups.setdefault(part[id(n)], {})[id(n)] = n
        for n in comp:
            if part.get(id(n)) == id(n):
                self._record(Claim(n, _close(groups[id(n)], self.travel)))

    def let_roots_travel(self) -> None:
        """A claim whose output only feeds other claims dissolves into them
        (its members become travel copies each reader re-derives) when all
        of: it surfaces no artifacts; its members are map work and
        reductions; none of its reductions runs over a dim a reading claim
        sweeps; nothing the region yields reads it; and re-deriving moves
        fewer elements than materializing (2 x output elements, a write and a
        read back, against readers x the elements of its inputs). Candidates
        are tried fewest reductions first; repeated to a fixpoint."""
        while True:
            pick = self._traveller()
            if pick is None:
                return
            gone = self.claims.pop(pick)
            self.travel.update(gone.members)
            self.travel[id(gone.root)] = gone.root
            for c in self.claims:
                _close(c.members, self.travel)

    def _traveller(self):
        holders: dict = defaultdict(set)
        for ci, c in enumerate(self.claims):
            for i in c.members:
                holders[i].add(ci)
        swept = [frozenset().union(*(_dims_of(m) for m in c.members.values()
                                     if m.op == "tl.reduce" and id(m) not in self.travel))
                 for c in self.claims]
        reduces = [sum(m.op == "tl.reduce" for m in c.members.values()) for c in self.claims]
        for ci in sorted(range(len(self.claims)), key=reduces.__getitem__):
            if self._may_travel(ci, holders, swept):
                return ci
        return None

    def _may_travel(self, ci, holders, swept) -> bool:
        root, members, arts = self.claims[ci]
        if root is None or arts:
            return False
        for m in members.values():
            if id(m) not in self.travel and not (_is_view(m) or m.op in _RECOMPUTE or m.op == "tl.reduce"):
                return False
        readers = self.deps.value_readers(root)
        if not readers:
            return False
        eaters: set = set()
        for r in readers:
            if id(r) in self.deps.exits:
                return False
            if _is_view(r):
                continue
            who = holders.get(id(r), set()) - {ci}
            if not who:
                return False
            eaters |= who
        mine = frozenset().union(*(_dims_of(m) for m in members.values() if m.op == "tl.reduce"))
        if any(mine & swept[cj] for cj in eaters):
            return False
        inputs = {id(a): a for m in members.values() for a in m.args if id(a) not in members and a.op not in _CONSTS}
        return 2 * _extent(root.type) > len(eaters) * sum(_extent(a.type) for a in inputs.values())


def _copyable(x, members, stats, swept):
    """``x``'s producers inside the claim, stopped at the statistics and at
    the claim's inputs, if a reader can re-derive them per tile: views, map
    work and reductions over none of the swept dims. Returns them or None."""
    cone, pending = {}, [x]
    while pending:
        n = pending.pop()
        if id(n) in cone or id(n) in stats or id(n) not in members:
            continue
        if n.op == "tl.reduce":
            if _dims_of(n) & swept:
                return None
        elif not (_is_view(n) or n.op in _RECOMPUTE):
            return None
        cone[id(n)] = n
        pending.extend(n.args)
    return cone


def _components(nodes: list) -> list:
    """Weakly connected components of ``nodes`` under argument edges, each
    listed in program order, ordered by their earliest node."""
    index = {id(n): i for i, n in enumerate(nodes)}
    parent = list(range(len(nodes)))

    def find(i):
        while parent[i] != i:
            parent[i] = parent[parent[i]]
            i = parent[i]
        return i

    for i, n in enumerate(nodes):
        for a in n.args:
            j = index.get(id(a))
            if j is not None:
                ri, rj = find(i), find(j)
                if ri != rj:
                    parent[max(ri, rj)] = min(ri, rj)
    comps: dict = {}
    for i, n in enumerate(nodes):
        comps.setdefault(find(i), []).append(n)
    return [comps[k] for k in sorted(comps)]


# ---------------------------------------------------------------- extraction


def extract(outputs, members):
    """A claim as a standalone canonical region. The rebuild walks each
    output's arguments left to right, depth first; a value outside
    ``members`` (any container of node ids) becomes the next param the first
    time the walk reaches it, constants are re-emitted. Identical claims
    from different layers therefore rebuild to one content key. One output
    is yielded bare, several as a tuple. Returns (region, bounds): bounds
    are the model values bound to the params, in order."""
    outputs = (outputs,) if not isinstance(outputs, (tuple, list)) else tuple(outputs)
    bounds, seen = [], set()
    for out in outputs:  # the rebuild's own visiting order, with an explicit stack of argument iterators
        if id(out) in seen:
            continue
        seen.add(id(out))
        frames = [iter(out.args)]
        while frames:
            a = next(frames[-1], None)
            if a is None:
                frames.pop()
            elif id(a) not in seen:
                seen.add(id(a))
                if id(a) in members:
                    frames.append(iter(a.args))
                elif a.op not in _CONSTS:
                    bounds.append(a)
    b = Builder(OPS)
    memo = {id(x): b.param(i, x.type) for i, x in enumerate(bounds)}
    params = tuple(memo[id(x)] for x in bounds)
    built = tuple(rebuild_into(b, memo, o) for o in outputs)
    y = built[0] if len(built) == 1 else b.emit("core.tuple", *built)
    return Region(params=params, body=(b.emit("core.yield", y),)), tuple(bounds)


# ------------------------------------------------------------------- the API


def carve_model(region: Region, dissolve: bool = True):
    """The partition alone: (claims, interior_count, travel). Claims are
    ``Claim(root, members, artifacts)`` with members keyed by node id;
    travel holds the nodes any claim may re-derive. ``dissolve=False`` keeps
    every claim's root a materialized value (the device executor's choice
    for values it cannot re-derive per tile)."""
    cv = _Carver(region)
    for rung in (cv.rung_flash, cv.rung_row_norm, cv.rung_row_stat, cv.rung_contraction):
        for n in cv.deps.interior:
            if id(n) not in cv.owned:
                rung(n)
    cv.split_residue()
    if dissolve:
        cv.let_roots_travel()
    return cv.claims, len(cv.deps.interior), cv.travel


def plan_model(region: Region, machine=None, floor: int = 1024, dissolve: bool = True) -> ModelPlan:
    """Carve ``region`` and plan each distinct kernel once. A flash joint is
    claimed whole first (the fused backward's carve)."""
    fj = match_flash_joint(region)
    if fj is not None:
        return _plan_joint(region, fj, machine, floor)
    claims, interior, _travel = carve_model(region, dissolve=dissolve)
    first_holder: dict = {}
    for ci, c in enumerate(claims):
        for i, m in c.members.items():
            if not _is_view(m):
                first_holder.setdefault(i, ci)
    counts = Counter(first_holder.values())
    planned: dict = {}
    carves = []
    for ci, (root, members, arts) in enumerate(claims):
        if root is None:
            ops = sorted({m.op for m in members.values() if not _is_view(m)})
            g = Group("uncompiled", None, None, "red", reason=f"multi-output residue over {ops}")
            carves.append(Carve(region, g, counts[ci], "residue"))
            continue
        kernel, bounds = extract((root, *arts), members)
        if kernel.key not in planned:
            planned[kernel.key] = plan_region(kernel, machine=machine, floor=floor).groups[0]
        carves.append(Carve(kernel, planned[kernel.key], counts[ci], root.op, root, bounds, arts))
    return ModelPlan(tuple(carves), interior)


# ----------------------------------------------------------- the joint claim


def match_flash_joint(region: Region):
    """The joint ``grad(flash_forward, out, seed, wrt)`` yields: returns a
    binding (the forward's match plus the wrt order and seed) or None."""
    y = region.body[-1].args[0]
    if y.op != "core.tuple" or len(y.args) < 2 or len(region.params) < 4:
        return None
    out, grads = y.args[0], y.args[1:]
    seed = region.params[-1]
    fwd_params = region.params[:-1]
    if len(fwd_params) != 3 or seed.op != "core.param" or seed.type != out.type:
        return None
    fwd = Region(params=fwd_params, body=(Builder(OPS).emit("core.yield", out),))
    fm = match_flash(fwd)
    if fm is None or fm["artifacts"]:
        return None
    pnames = {id(fm["q"]): "q", id(fm["k"]): "k", id(fm["v"]): "v"}
    order = tuple(pnames[id(p)] for p in fwd_params)
    names = region_names(fwd, order, ("out",))
    # which params do the grads belong to? every ordered subset of (q, k, v)
    # of the right length is regenerated and compared (at most 6)
    for wrt in itertools.permutations(("q", "k", "v"), len(grads)):
        rg = grad(fwd, "out", seed="dO", wrt=wrt, names=names)
        ys = rg.region.body[-1].args[0]
        rys = ys.args[1:] if ys.op == "core.tuple" else ()
        if len(rys) != len(grads):
            continue
        # the regenerated joint's seed is a fresh param: it must match the given one's type
        if rg.region.params[-1].type != seed.type or rg.region.params[-1].attrs != seed.attrs:
            continue
        if all(a.key == b.key for a, b in zip(rys, grads)):
            return {**fm, "wrt": wrt, "seed": seed, "param_order": order}
    return None


def _plan_joint(region: Region, fj, machine, floor) -> ModelPlan:
    interior = [n for n in walk(region)
                if not _is_view(n) and n.op not in ("core.param", "core.yield", "core.tuple")]
    out = region.body[-1].args[0].args[0]
    fwd = Region(params=region.params[:-1], body=(Builder(OPS).emit("core.yield", out),))
    fplan = plan_region(fwd, machine=machine, floor=floor).groups[0]
    cert = Certificate("proved-exact", fplan.certificate.licenses if fplan.certificate else (), (), True)
    g = Group(
        "flash-joint",
        region,
        cert,
        "yellow",
        params=(("si", pick_ki(fj["extent"])), ("wrt", fj["wrt"]), ("forward", fplan.template)),
        launch=fplan.launch,
        prune=fplan.prune,
        artifacts=("m", "den"),
    )
    carve = Carve(region, g, len(interior), out.op, out, tuple(region.params), ("m", "den"))
    return ModelPlan((carve,), len(interior))


__all__ = ["Carve", "Claim", "ModelPlan", "carve_model", "extract", "plan_model", "match_flash_joint"]
