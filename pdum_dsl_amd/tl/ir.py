"""The IR the backend consumes: one frozen node type, regions, a builder that
runs type rules at emission, and content keys.

Restates the reference's IR core (packages/dsl/src/pdum/dsl/ir.py:89-156,
ops.py:39-45) at the size this backend needs: a ``Node`` IS its SSA value
(op, type, args, regions, attrs); identity is structural and a sha256
content key is memoized per node; ``loc`` is outside identity. Attributes
are canonically sorted at emission so two spellings of one op share a key.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass, field
from typing import Callable, Hashable


class VerifyError(Exception):
    """Malformed IR, refused at construction."""


# ------------------------------------------------------------------ types


@dataclass(frozen=True)
class Type:
    pass


@dataclass(frozen=True)
class Scalar(Type):
    """A scalar carrier (the reference's f64 / i64 / bool lattice, types.py)."""

    name: str

    def __repr__(self) -> str:
        return self.name


F64 = Scalar("f64")
BOOL = Scalar("bool")


@dataclass(frozen=True)
class Dim:
    """A named lattice dimension with domain [start, stop) — the observable
    frame of a layout dim (layout.py:89-118 in the reference)."""

    name: str
    start: int
    stop: int

    def __post_init__(self):
        if self.stop < self.start:
            raise ValueError(f"dim {self.name}: stop {self.stop} < start {self.start}")

    @property
    def size(self) -> int:
        return self.stop - self.start


@dataclass(frozen=True)
class TensorType(Type):
    """A tensor-typed SSA value: an ordered tuple of named dims. Alignment is
    by name (order is presentation, never semantics)."""

    dims: tuple[Dim, ...]

    def __post_init__(self):
        names = [d.name for d in self.dims]
        if len(set(names)) != len(names):
            raise TypeError(f"duplicate dim names in {names}")

    @property
    def names(self) -> tuple[str, ...]:
        return tuple(d.name for d in self.dims)

    @property
    def shape(self) -> tuple[int, ...]:
        return tuple(d.size for d in self.dims)

    def dim(self, name: str) -> Dim:
        for d in self.dims:
            if d.name == name:
                return d
        raise KeyError(f"no dim {name!r} in {self.names}")

    def has(self, name: str) -> bool:
        return any(d.name == name for d in self.dims)

    def __repr__(self) -> str:
        inner = ", ".join(f"{d.name}[{d.start}:{d.stop}]" for d in self.dims)
        return f"T({inner})"


@dataclass(frozen=True)
class TupleType(Type):
    elems: tuple[Type, ...]


def tensor_type(names, shape) -> TensorType:
    """TensorType over dims ``names`` with extents ``shape`` (all starting at 0)."""
    return TensorType(tuple(Dim(n, 0, int(s)) for n, s in zip(names, shape)))


def minus_dim(tt: TensorType, name: str) -> TensorType:
    """The fold-element type: the source minus its scan dim (dialect.py:122)."""
    return TensorType(tuple(d for d in tt.dims if d.name != name))


# -------------------------------------------------------------- IR nodes


def _h(*parts: bytes) -> bytes:
    m = hashlib.sha256()
    for p in parts:
        m.update(len(p).to_bytes(4, "little"))
        m.update(p)
    return m.digest()


@dataclass(frozen=True, eq=False)
class Node:
    """One SSA value. Equality is object identity; ``key`` is the content
    key (op, type, attrs, arg keys, region keys)."""

    op: str
    type: Type
    args: tuple = ()
    regions: tuple = ()
    attrs: tuple = ()
    loc: object = field(default=None, compare=False)
    _key: bytes | None = field(default=None, init=False, repr=False, compare=False)

    @property
    def key(self) -> bytes:
        if self._key is None:
            parts = [self.op.encode(), repr(self.type).encode(), repr(self.attrs).encode()]
            parts += [a.key for a in self.args] + [r.key for r in self.regions]
            object.__setattr__(self, "_key", _h(*parts))
        return self._key

    def attr(self, name: str, default=None):
        for k, v in self.attrs:
            if k == name:
                return v
        return default

    def __repr__(self) -> str:  # never recurse the DAG
        return f"Node({self.op}, {self.type!r})"


@dataclass(frozen=True, eq=False)
class Region:
    params: tuple = ()
    body: tuple = ()
    _key: bytes | None = field(default=None, init=False, repr=False, compare=False)

    @property
    def key(self) -> bytes:
        if self._key is None:
            parts = [b"region"] + [p.key for p in self.params] + [n.key for n in self.body]
            object.__setattr__(self, "_key", _h(*parts))
        return self._key

    @property
    def result(self) -> Node:
        return self.body[-1].args[0]


@dataclass(frozen=True)
class OpDef:
    name: str
    type_rule: Callable | None = None  # (arg_types, attrs: dict, regions) -> Type
    nregions: int = 0


class Builder:
    """The construction path: canonical attrs, the op's type rule run at
    emission (or an explicit ``type=`` where no rule exists)."""

    def __init__(self, ops: dict):
        self.ops = ops

    def emit(self, op: str, *args: Node, regions: tuple = (), loc=None, type: Type | None = None, **attrs) -> Node:
        od = self.ops.get(op)
        if od is None:
            raise VerifyError(f"unknown op {op!r}")
        if len(regions) != od.nregions:
            raise VerifyError(f"{op} takes {od.nregions} region(s), got {len(regions)}")
        for v in attrs.values():
            try:
                hash(v)
            except TypeError as exc:
                raise VerifyError(f"{op}: attribute values must be hashable ({exc})") from None
        canon = tuple(sorted(attrs.items()))
        if type is None:
            if od.type_rule is None:
                raise VerifyError(f"{op} has no type rule; pass type=")
            type = od.type_rule(tuple(a.type for a in args), dict(canon), tuple(regions))
        return Node(op, type, tuple(args), tuple(regions), canon, loc)

    def param(self, index: Hashable, type: Type) -> Node:
        return Node("core.param", type, attrs=(("index", index),))


def walk(region: Region):
    """Nodes reachable from the region body, operands before users (each once)."""
    seen: set[int] = set()
    out: list[Node] = []

    def go(n: Node):
        stack = [(n, False)]
        while stack:
            x, done = stack.pop()
            if done:
                out.append(x)
                continue
            if id(x) in seen:
                continue
            seen.add(id(x))
            stack.append((x, True))
            for a in reversed(x.args):
                if id(a) not in seen:
                    stack.append((a, False))

    for b in region.body:
        go(b)
    return out


def walk_deep(region: Region):
    """Every node of the region and of its sub-regions (fold steps), each
    ONCE: a step region shared by several fold nodes is visited once."""
    seen: set[int] = set()
    todo = [region]
    seen_regions: set[int] = set()
    while todo:
        r = todo.pop()
        if id(r) in seen_regions:
            continue
        seen_regions.add(id(r))
        for n in walk(r):
            if id(n) in seen:
                continue
            seen.add(id(n))
            yield n
            todo.extend(n.regions)
