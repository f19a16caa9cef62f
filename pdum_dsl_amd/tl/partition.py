"""Whole-model plans: carve a region into template groups (the reference's
packages/tensorlib/src/pdum/tl/partition.py:458-607, ``carve_model`` and
``plan_model``) — as far as the HIP hot path needs it.

The reference carves the autodiff joint of flash attention into a
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

A region that is not a flash joint is planned as one group by
``fusion.plan_region`` (its single-template rows). What neither covers is a
red carve with the reason — plans are data, never exceptions.
"""

from __future__ import annotations

from dataclasses import dataclass, field

from .autodiff import grad, region_names
from .certify import Certificate
from .fusion import Group, match_flash, pick_ki, plan_region
from .ir import Region, walk

_FREE = ("core.const", "tl.const", "tl.repeat_like", "tl.repeat", "core.param", "core.yield", "core.tuple")


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
    return [n for n in walk(region) if n.op not in _FREE]


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


def plan_model(region: Region, machine=None, floor: int = 1024) -> ModelPlan:
    """Carve ``region`` and plan each carve (partition.py:586-607)."""
    interior = _interior(region)
    fj = match_flash_joint(region)
    if fj is not None:
        out = region.body[-1].args[0].args[0]
        fwd = Region(params=region.params[:-1], body=(_yield(out),))
        fplan = plan_region(fwd, machine=machine, floor=floor).groups[0]
        cert = Certificate("proved-exact", fplan.certificate.licenses if fplan.certificate else (), (), True)
        si = pick_ki(fj["extent"])
        g = Group(
            "flash-joint",
            region,
            cert,
            "yellow",
            params=(("si", si), ("wrt", fj["wrt"]), ("forward", fplan.template)),
            launch=fplan.launch,
            prune=fplan.prune,
            artifacts=("m", "den"),
        )
        carve = Carve(region, g, len(interior), out.op, out, tuple(region.params), ("m", "den"))
        return ModelPlan((carve,), len(interior))
    (g,) = plan_region(region, machine=machine, floor=floor).groups
    y = region.body[-1].args[0]
    root = y.args[0] if y.op == "core.tuple" else y
    kern = g.kernel if g.kernel is not None else region
    return ModelPlan((Carve(kern, g, len(interior), root.op, root, tuple(region.params), g.artifacts),), len(interior))


__all__ = ["Carve", "ModelPlan", "plan_model", "match_flash_joint"]
