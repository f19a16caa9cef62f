"""Whole-model plans: carve a region into template groups (the reference's
packages/tensorlib/src/pdum/tl/partition.py, ``carve_model`` and
``plan_model``).

**The anchor-and-absorb partition** (partition.py:1-24, 458-582), restated:
every reduce must live in some claim, and claims run most-specific first —
flash compositions (three reduces), then bare row normalizations (two), then
row statistics, then single-reduce contractions. Contraction claims absorb
both ways: epilogues walk downstream while the root has exactly one
consumer; operand prologues walk upstream through the recompute-exact
vocabulary while every consumer lies inside the claim. A fork ends a walk
and leaves a materialized boundary. A claim whose interior would be
consumed outside it is refused (v1 groups have one output), except that a
flash claim may surface its row statistics as ARTIFACTS and mark the other
leaked values' cones as TRAVEL (copies consumers re-derive). The unclaimed
residue splits into per-root components (map chains where pure map work,
red groups where not). Finally claims whose root only feeds other claims
DISSOLVE into them when re-deriving per tile moves fewer elements than
materializing (the traffic gate), to fixpoint. Every claim is rebuilt as a
canonical region (boundaries become params in first-use order) so repeated
layers share one content key, and ``plan_model`` plans each distinct kernel
once.

**The MI355X joint claim.** The reference carves the autodiff joint of flash attention into a
flash-with-artifacts group plus contraction carves for dV, dQ, dK and the
row statistic D (partition.py:476-557), each compiled separately. On MI355X
the whole joint runs as ONE forward-with-artifacts kernel and ONE fused
backward launch, so this partitioner claims the joint whole, as the carve
``flash-joint``:

  * the joint's first yield must be a ``flash`` composition (fusion.match_flash
    over q, k, v params);
  * the rest of the yield must be exactly the vector-Jacobian product of that
    forward — checked by REGENERATING it with ``autodiff.grad`` from the
    extracted forward and comparing content keys, node for node (the same
    recognize-by-regeneration law the HIP seat applies to flash tiles);
  * its certificate is proved-exact (the key is reached), and the forward's
    own flash certificate rides along in ``Group.params``.

``plan_model`` tries that claim first; any other region goes through
``carve_model``. What no row covers is a red carve with the reason — plans
are data, never exceptions.
"""

from __future__ import annotations

from dataclasses import dataclass, field

from .autodiff import grad, region_names
from .certify import Certificate
from .dialect import OPS
from .fusion import Group, contract_core, forest_is_closed, match_flash, match_rowstat, match_softmax, pick_ki
from .fusion import plan_region, rebuild_into
from .ir import Builder, Region, walk

_CONSTS = ("core.const", "tl.const")
# zero-cost views: shared by claims, duplicated at rebuild (partition.py:47-53)
_FREE = _CONSTS + ("tl.rename", "tl.repeat_like", "tl.repeat")
_EPILOGUE = ("tl.pointwise", "tl.repeat_like")  # what an epilogue walk may absorb
_COMPUTE = ("tl.pointwise", "tl.iota")  # what a prologue walk may absorb
_SINKS = ("core.param", "core.yield", "core.tuple")


@dataclass(frozen=True)
class Carve:
    """One carved group (partition.py:58-70): the canonical kernel, the plan
    the recognizer produced for it, and the claim's footprint in the model."""

    kernel: Region = field(repr=False)
    group: Group
    nodes: int  # interior (non-free) model nodes this carve claims
    root_op: str
    root: object = field(default=None, repr=False)
    bounds: tuple = field(default=(), repr=False)  # the model nodes its params bind to, in param order
    artifacts: tuple = field(default=(), repr=False)  # surfaced statistics, tuple-yield order


@dataclass(frozen=True)
class ModelPlan:
    """A whole-model plan is data (partition.py:73-85): carves in dependency
    order, the interior node count, coverage derived."""

    carves: tuple
    interior: int

    def coverage(self) -> float:
        if self.interior == 0:
            return 1.0
        return sum(c.nodes for c in self.carves if c.group.confidence != "red") / self.interior

    def distinct_kernels(self) -> int:
        return len({c.kernel.key for c in self.carves})


def _interior(region: Region) -> list:
    return [n for n in walk(region) if n.op not in _FREE and n.op not in _SINKS]


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
    fwd = Region(params=fwd_params, body=(_yield(out),))
    fm = match_flash(fwd)
    if fm is None or fm["artifacts"]:
        return None
    pnames = {id(fm["q"]): "q", id(fm["k"]): "k", id(fm["v"]): "v"}
    order = tuple(pnames[id(p)] for p in fwd_params)
    names = region_names(fwd, order, ("out",))
    # which params do the grads belong to? try every ordered subset the
    # regenerated VJP could have been asked for (at most 3! + ... = 15)
    for wrt in _wrt_candidates(len(grads)):
        rg = grad(fwd, "out", seed="dO", wrt=wrt, names=names)
        ys = rg.region.body[-1].args[0]
        rys = ys.args[1:] if ys.op == "core.tuple" else ()
        if len(rys) != len(grads):
            continue
        # the regenerated joint's seed is a fresh param: compare against the
        # given joint with its seed bound to the same index
        if rg.region.params[-1].type != seed.type or rg.region.params[-1].attrs != seed.attrs:
            continue
        if all(a.key == b.key for a, b in zip(rys, grads)):
            return {**fm, "wrt": wrt, "seed": seed, "param_order": order}
    return None


def _yield(n):
    from .dialect import OPS
    from .ir import Builder

    return Builder(OPS).emit("core.yield", n)


def _wrt_candidates(n: int):
    import itertools

    for combo in itertools.permutations(("q", "k", "v"), n):
        yield combo




# ------------------------------------------------------- the graph and claims


def _graph(region: Region):
    """Interior nodes in dependency order (params, sinks and free views
    excluded) and the consumer lists of every value (partition.py:88-103)."""
    params = {id(p) for p in region.params}
    yld = region.body[-1]
    order, consumers = [], {}
    for n in walk(region):
        if id(n) in params:
            continue
        for a in n.args:
            consumers.setdefault(id(a), []).append(n)
        if n is yld or n.op == "core.tuple":
            continue
        order.append(n)
    return [n for n in order if n.op not in _FREE], consumers


def _cone(root, stops: set, allow: set | None = None) -> dict:
    """The producer cone of ``root`` (id -> node), exclusive of ``stops`` and
    params, optionally restricted to ``allow`` (partition.py:106-118)."""
    members, todo = {}, [root]
    while todo:
        n = todo.pop()
        if id(n) in members or id(n) in stops or n.op == "core.param":
            continue
        if allow is not None and id(n) not in allow and n is not root:
            continue
        members[id(n)] = n
        todo.extend(n.args)
    return members


def _attach_free_fringe(members: dict) -> dict:
    """Free views (not consts) that members read join the claim, to fixpoint:
    a boundary is always a real value, never a view (partition.py:121-133)."""
    while True:
        grown = [a for m in list(members.values()) for a in m.args
                 if id(a) not in members and a.op in _FREE and a.op not in _CONSTS]
        if not grown:
            return members
        for a in grown:
            members[id(a)] = a


def _outside(a, members, consumers, root=None) -> bool:
    """Is ``a``'s value consumed outside ``members``? Free views forward their
    value, so the check looks through them to their consumers; reaching the
    claim's root is the export itself (partition.py:136-148)."""
    for c in consumers.get(id(a), ()):
        if c is root:
            continue
        if id(c) not in members:
            return True
        if c.op in _FREE and _outside(c, members, consumers, root):
            return True
    return False


def _leaks(root, members, consumers, travel=()) -> bool:
    """A non-root interior member consumed outside would need a second output
    (partition.py:151-159); travel copies are exempt."""
    return any(m is not root and m.op not in _FREE and id(m) not in travel and _outside(m, members, consumers, root)
               for m in members.values())


def _absorb_up(members, consumers, claimed, travel=()) -> dict:
    """The prologue walk (partition.py:162-188): compute nodes join while every
    consumer already lies inside the claim; travel copies join unconditionally."""
    while True:
        _attach_free_fringe(members)
        added = False
        for m in list(members.values()):
            for a in m.args:
                if id(a) in members:
                    continue
                if id(a) in travel:
                    members[id(a)] = a
                    added = True
                elif id(a) not in claimed and a.op in _COMPUTE and not _outside(a, members, consumers):
                    members[id(a)] = a
                    added = True
        if not added:
            return members


def _absorb_travel(members, travel) -> dict:
    """Free views and travel copies only, to fixpoint (partition.py:191-205)."""
    while True:
        _attach_free_fringe(members)
        grown = [a for m in list(members.values()) for a in m.args if id(a) not in members and id(a) in travel]
        if not grown:
            return members
        for a in grown:
            members[id(a)] = a


def _absorb(root, members, consumers, claimed):
    """The epilogue walk (partition.py:208-227): while the root has exactly one
    consumer in the epilogue vocabulary, it joins and becomes the root; a
    broadcast side operand of an absorbed node rides along."""
    while True:
        cs = consumers.get(id(root), ())
        if len(cs) != 1:
            return root
        c = cs[0]
        if c.op not in _EPILOGUE or id(c) in claimed or c.op == "core.yield":
            return root
        if c.op == "tl.repeat_like" and c.args[0] is root:
            return root  # broadcasting INTO another claim's lattice is that claim's product
        for side in c.args:
            if side is root or id(side) in members or side.op in _CONSTS:
                continue
            if side.op == "tl.repeat_like" and id(side.args[1]) in members:
                members[id(side)] = side
        members[id(c)] = c
        root = c


def _claim_flash(r):
    """The flash shape on bare nodes (partition.py:230-255): q, k, v are any
    values (the carve makes them params); riders decline."""
    out = contract_core(r)
    if out is None:
        return None
    pr, v, s = out
    sm = match_softmax(pr)
    if sm is None or sm["s"] != s:
        return None
    smn = sm["sm"]
    if smn.op != "tl.pointwise" or smn.attr("f") != "where" or len(smn.args) != 3:
        return None
    mask, sc, fill = smn.args
    if fill.op not in _CONSTS or not forest_is_closed(mask):
        return None
    core = contract_core(sc)
    if core is None:
        return None
    q, k, e = core
    qd, kd, vd = (x.type.names for x in (q, k, v))
    if len(qd) != 2 or kd != (s, e) or len(vd) != 2 or vd[0] != s:
        return None
    t = next(n for n in qd if n != e)
    return {"q": q, "k": k, "v": v, "m": sm["max"], "den": sm["den"], "t": t, "s": s}


def _reduce_dims(n) -> set:
    d = n.attr("dims")
    return {d} if isinstance(d, str) else set(d)


def _duplicable_cone(x, members, stats, sweep):
    """``x``'s cone inside the claim, stopped at artifacts and boundaries: map
    work and tile-local reductions travel, a reduction over a swept dim does
    not (partition.py:258-276). Returns the cone or None."""
    cone, todo = {}, [x]
    while todo:
        n = todo.pop()
        if id(n) in cone or id(n) in stats or id(n) not in members:
            continue
        if n.op == "tl.reduce":
            if _reduce_dims(n) & sweep:
                return None
        elif n.op not in _FREE and n.op not in _COMPUTE:
            return None
        cone[id(n)] = n
        todo.extend(n.args)
    return cone


def _extract(root, members, artifacts=()):
    """Rebuild a claim as a canonical standalone region (partition.py:296-324):
    boundaries become params in first-use order (a depth-first walk that
    mirrors the rebuild's argument order), so structurally identical claims
    from different layers share one content key. With artifacts the region
    yields (output, *artifacts). Returns (region, bounds)."""
    bounds, seen = [], set()
    for r in (root, *artifacts):
        todo = [r]
        while todo:
            n = todo.pop()
            if id(n) in seen:
                continue
            seen.add(id(n))
            for a in reversed(n.args):
                if id(a) in members:
                    todo.append(a)
                elif id(a) not in seen and a.op not in _CONSTS:
                    seen.add(id(a))
                    bounds.append(a)
    b = Builder(OPS)
    memo = {id(x): b.param(i, x.type) for i, x in enumerate(bounds)}
    params = tuple(memo[id(x)] for x in bounds)
    built = tuple(rebuild_into(b, memo, r) for r in (root, *artifacts))
    y = built[0] if len(built) == 1 else b.emit("core.tuple", *built)
    return Region(params=params, body=(b.emit("core.yield", y),)), tuple(bounds)


def _components(nodes, consumers):
    """Weakly connected components of the unclaimed residue, each with the
    members consumed outside it (its roots) (partition.py:327-355)."""
    pool = {id(n): n for n in nodes}
    nbr: dict = {}
    for n in nodes:
        for a in n.args:
            if id(a) in pool:
                nbr.setdefault(id(n), set()).add(id(a))
                nbr.setdefault(id(a), set()).add(id(n))
    seen, comps = set(), []
    for n in nodes:
        if id(n) in seen:
            continue
        comp, todo = [], [id(n)]
        while todo:
            i = todo.pop()
            if i in seen:
                continue
            seen.add(i)
            comp.append(pool[i])
            todo.extend(nbr.get(i, ()))
        ids = {id(x) for x in comp}
        roots = [m for m in comp if any(id(c) not in ids for c in consumers.get(id(m), ()))]
        comps.append((comp, roots))
    return comps


def _elems(t) -> int:
    n = 1
    for d in getattr(t, "dims", ()):
        n *= d.size
    return n


def _dissolve(claims, consumers, travel, region):
    """Root travel (partition.py:358-455): a claim whose root feeds only other
    claims, with nothing but map work and reductions the consumers do not
    sweep, dissolves into them when re-deriving it moves fewer elements than
    materializing it (2 x root elements vs consumers x boundary inputs). Pure
    map claims are tried first; repeats to fixpoint."""
    yld = region.body[-1]
    sinks = {id(yld)} | ({id(yld.args[0])} if yld.args[0].op == "core.tuple" else set())

    def value_consumers(x, out, seen):
        for c in consumers.get(id(x), ()):
            if id(c) in seen:
                continue
            seen.add(id(c))
            out.append(c)
            if c.op in _FREE:
                value_consumers(c, out, seen)
        return out

    while True:
        owner: dict = {}
        for ci, (_root, members, _arts) in enumerate(claims):
            for i in members:
                owner.setdefault(i, set()).add(ci)
        sweeps = []
        for _root, members, _arts in claims:
            sw: set = set()
            for m in members.values():
                if m.op == "tl.reduce" and id(m) not in travel:
                    sw |= _reduce_dims(m)
            sweeps.append(sw)
        order = sorted(range(len(claims)), key=lambda ci: sum(m.op == "tl.reduce" for m in claims[ci][1].values()))
        gone = None
        for ci in order:
            root, members, arts = claims[ci]
            if root is None or arts:
                continue
            if any(m.op not in _FREE and m.op not in _COMPUTE and m.op != "tl.reduce" and id(m) not in travel
                   for m in members.values()):
                continue
            mine: set = set()
            for m in members.values():
                if m.op == "tl.reduce":
                    mine |= _reduce_dims(m)
            cons = value_consumers(root, [], set())
            ok, eaters = bool(cons), set()
            for c in cons:
                if id(c) in sinks:
                    ok = False
                    break
                if c.op in _FREE:
                    continue
                who = owner.get(id(c), set()) - {ci}
                if not who:
                    ok = False
                    break
                eaters |= who
            if not ok or any(mine & sweeps[cj] for cj in eaters):
                continue
            binputs, seenb = 0, set()
            for m in members.values():
                for a in m.args:
                    if id(a) not in members and id(a) not in seenb and a.op not in _CONSTS:
                        seenb.add(id(a))
                        binputs += _elems(a.type)
            if 2 * _elems(root.type) <= len(eaters) * binputs:
                continue  # materializing is cheaper: the carve stays
            gone = ci
            break
        if gone is None:
            return claims
        root, members, _arts = claims.pop(gone)
        travel.update(members)
        travel[id(root)] = root
        for _r, mem, _a in claims:
            _absorb_travel(mem, travel)


def carve_model(region: Region, dissolve: bool = True):
    """The partition alone (partition.py:458-582): returns (claims,
    interior_count, travel), claims as (root, members, artifacts) with members
    keyed by id; a rootless claim is a multi-output residue. ``dissolve=False``
    skips root travel, so every claim's root stays a materialized boundary
    (the device executor's policy for values it cannot re-derive per tile)."""
    interior, consumers = _graph(region)
    claimed: set = set()
    travel: dict = {}
    claims: list = []

    def take(root, members, arts=()):
        _attach_free_fringe(members)
        if _leaks(root, members, consumers, travel):
            return False
        claims.append((root, members, arts))
        claimed.update(i for i, m in members.items() if m.op not in _FREE)
        return True

    def take_flash_artifacts(r, f, members):
        _attach_free_fringe(members)
        stats = {id(f["m"]), id(f["den"])}
        sweep = {f["t"], f["s"]}
        new_travel: dict = {}
        for m in members.values():
            if m is r or id(m) in stats or not _outside(m, members, consumers, r):
                continue
            while m.op in _FREE and m.args:  # a leaked view: classify the value it reads
                m = m.args[0]
            if m is r or id(m) in stats or id(m) not in members:
                continue
            cone = _duplicable_cone(m, members, stats, sweep)
            if cone is None:
                return False
            new_travel.update(cone)
        claims.append((r, members, (f["m"], f["den"])))
        travel.update(new_travel)
        claimed.update(i for i, m in members.items() if m.op not in _FREE)
        return True

    def free_of_claims(members):
        return not any(i in claimed and i not in travel for i in members)

    for r in interior:  # flash compositions: three reduces, most specific
        if r.op != "tl.reduce" or id(r) in claimed:
            continue
        f = _claim_flash(r)
        if f is not None:
            members = _cone(r, {id(f["q"]), id(f["k"]), id(f["v"])})
            if free_of_claims(members) and not take(r, dict(members)):
                take_flash_artifacts(r, f, members)
    for n in interior:  # bare row normalizations (two reduces)
        if id(n) in claimed:
            continue
        sm = match_softmax(n)
        if sm is None:
            continue
        members = _absorb_travel(_cone(n, {id(sm["sm"])}), travel)
        if free_of_claims(members):
            take(n, members)
    for n in interior:  # row statistics, the scale-shift absorbed as epilogue
        if id(n) in claimed:
            continue
        rs = match_rowstat(n)
        if rs is None:
            continue
        members = _absorb_travel(_cone(n, {id(rs["x"])}), travel)
        if free_of_claims(members):
            take(_absorb(n, members, consumers, claimed), members)
    for r in interior:  # single-reduce contractions: prologues up, epilogues down
        if r.op != "tl.reduce" or id(r) in claimed:
            continue
        dims = tuple(_reduce_dims(r))
        if r.attr("f") not in ("sum", "mean") or len(dims) not in (1, 2) or r.attr("zero") is not None:
            continue
        mul = r.args[0]
        if mul.op == "tl.pointwise" and mul.attr("f") == "mul" and len(mul.args) == 2:
            cores = [_core(x) for x in mul.args]
        else:  # the plain shape: a sum with no product
            cores = [mul]
        if any(not hasattr(c.type, "dims") or not c.type.has(k) for c in cores for k in dims):
            continue
        keeps = [{nm for nm in c.type.names if nm not in dims} for c in cores]
        if set(r.type.names) != set().union(*keeps):
            continue
        members = {id(r): r}
        if len(cores) == 2:
            members[id(mul)] = mul
        if any(i in claimed for i in members):
            continue
        _absorb_up(members, consumers, claimed, travel)
        take(_absorb(r, members, consumers, claimed), members)
    residue = [n for n in interior if id(n) not in claimed]
    for comp, roots in _components(residue, consumers):
        comp_ids = {id(m) for m in comp}
        allow = comp_ids | set(travel)
        pool = {id(m): m for m in comp}
        rootset = [id(x) for x in roots]
        while True:  # one part per root; promote internal fan-ins until the parts tile
            parts, used = [], set()
            for ri in rootset:
                stops = (set(rootset) - {ri}) | used
                mem = _absorb_travel(_cone(pool[ri], stops, allow=allow), travel)
                parts.append((pool[ri], mem))
                used |= {i for i in mem if i in comp_ids}
            promote = []
            for _rt, mem in parts:
                for m in mem.values():
                    for a in m.args:
                        if id(a) in comp_ids and id(a) not in mem and id(a) not in rootset and id(a) not in promote:
                            promote.append(id(a))
            if not promote:
                claims.extend((rt, mem, ()) for rt, mem in parts)
                break
            rootset.extend(promote)
    if dissolve:
        _dissolve(claims, consumers, travel, region)
    return claims, len(interior), travel


def _core(x):
    """A contraction operand under its broadcasts (fusion.py:98-122)."""
    while x.op in ("tl.repeat_like", "tl.repeat"):
        x = x.args[0]
    return x


def plan_model(region: Region, machine=None, floor: int = 1024, dissolve: bool = True) -> ModelPlan:
    """Carve ``region`` and plan each distinct carve once (partition.py:586-607).
    A flash joint is claimed whole first (the fused backward's carve)."""
    fj = match_flash_joint(region)
    if fj is not None:
        return _plan_joint(region, fj, machine, floor)
    claims, interior, _travel = carve_model(region, dissolve=dissolve)
    seen: dict = {}
    carves = []
    counted: set = set()  # travel copies count once, in their first claim
    for root, members, arts in claims:
        n_interior = sum(1 for i, m in members.items() if m.op not in _FREE and i not in counted)
        counted.update(i for i, m in members.items() if m.op not in _FREE)
        if root is None:
            ops = sorted({m.op for m in members.values() if m.op not in _FREE})
            g = Group("uncompiled", None, None, "red", reason=f"multi-output residue over {ops}")
            carves.append(Carve(region, g, n_interior, "residue"))
            continue
        kernel, bounds = _extract(root, members, arts)
        g = seen.get(kernel.key)
        if g is None:
            g = plan_region(kernel, machine=machine, floor=floor).groups[0]
            seen[kernel.key] = g
        carves.append(Carve(kernel, g, n_interior, root.op, root, bounds, arts))
    return ModelPlan(tuple(carves), interior)


def _plan_joint(region: Region, fj, machine, floor) -> ModelPlan:
    interior = _interior(region)
    out = region.body[-1].args[0].args[0]
    fwd = Region(params=region.params[:-1], body=(_yield(out),))
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


__all__ = ["Carve", "ModelPlan", "carve_model", "plan_model", "match_flash_joint"]
