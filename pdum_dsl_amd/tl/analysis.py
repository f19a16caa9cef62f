"""Analyses as cached facts, and measurements as a persistent ledger.

Behaviour follows the reference's analysis cache
(packages/tensorlib/src/pdum/tl/analysis.py:1-155): an analysis is declared
as name@version over a function; calling it yields a ``Fact`` keyed by the
analysis, its inputs' content and its keyword parameters; a Fact passed as
an input contributes its key and hands the function its value; a
``ledger=True`` analysis is a MEASUREMENT whose plain-JSON value persists
across sessions; inside ``no_reanalysis()`` every miss raises. There is no
invalidation: regions are immutable and content-addressed, so a changed
program is a different key.

The design here is this module's own:

  * keys are the sha256 of a typed token stream (``_Digest``): each input is
    walked once and written as tag, length and payload, so no intermediate
    structure is built and no two differently typed inputs share a key;
  * one ``_FactStore`` holds the facts, the measurement subset, the miss
    count and the warm-loop depth;
  * the ledger file is JSON Lines: a header line naming the format, then
    one measurement per line, sorted by key, written to a temporary file
    and renamed over the target, so an interrupted save never leaves half a
    ledger. Loading never replaces a fact already held in this session.
"""

from __future__ import annotations

import contextlib
import hashlib
import json
import math
import os
import struct
from dataclasses import dataclass
from pathlib import Path
from typing import Callable

import numpy as np

_LEDGER_HEADER = {"ledger": "pdum_dsl_amd.measurements", "format": 1}


class Reanalysis(RuntimeError):
    """A cache miss inside ``no_reanalysis()``."""


@dataclass(frozen=True)
class Fact:
    """One cached analysis result: ``key`` is its identity, ``analysis`` its
    provenance (name@vN), ``value`` the payload."""

    key: str
    analysis: str
    value: object


class _Digest:
    """sha256 over (tag, length, payload) records; ``add`` walks one value."""

    def __init__(self) -> None:
        self._h = hashlib.sha256()

    def record(self, tag: bytes, payload: bytes = b"") -> None:
        self._h.update(tag + struct.pack("<Q", len(payload)) + payload)

    def add(self, x) -> None:
        if isinstance(x, Fact):
            self.record(b"fact", x.key.encode())
        elif isinstance(getattr(x, "key", None), bytes):  # IR regions and nodes carry content keys
            self.record(b"ir", x.key)
        elif x is None:
            self.record(b"none")
        elif isinstance(x, (bool, np.bool_)):
            self.record(b"bool", b"1" if x else b"0")
        elif isinstance(x, (int, np.integer)):
            self.record(b"int", str(int(x)).encode())
        elif isinstance(x, (float, np.floating)):
            v = float(x)
            self.record(b"float", b"nan" if math.isnan(v) else v.hex().encode())
        elif isinstance(x, str):
            self.record(b"str", x.encode("utf-8", "surrogatepass"))
        elif isinstance(x, (bytes, bytearray)):
            self.record(b"bytes", bytes(x))
        elif isinstance(x, (tuple, list)):
            self.record(b"seq", str(len(x)).encode())
            for e in x:
                self.add(e)
        elif isinstance(x, (set, frozenset)):
            parts = sorted(_digest_of(e) for e in x)  # order-free: members by their own digests
            self.record(b"set", b"".join(parts))
        elif isinstance(x, dict):
            self.record(b"map", str(len(x)).encode())
            for k in sorted(x, key=lambda k: (type(k).__name__, str(k))):
                self.add(k)
                self.add(x[k])
        elif isinstance(x, np.ndarray):
            a = np.ascontiguousarray(x)
            self.record(b"array", f"{a.dtype.str}{a.shape}".encode())
            self._h.update(a.tobytes())
        else:
            raise TypeError(
                f"an analysis input must be content-keyable (a Fact, an IR region or node, plain data or an "
                f"ndarray), not {type(x).__name__}: without a content key the cache cannot tell two calls apart"
            )

    def hexdigest(self) -> str:
        return self._h.hexdigest()


def _digest_of(x) -> bytes:
    d = _Digest()
    d.add(x)
    return d._h.digest()


class _FactStore:
    """Every fact this process holds; ``measured`` is the ledger subset."""

    def __init__(self) -> None:
        self.facts: dict = {}
        self.measured: dict = {}
        self.misses = 0
        self.warm_depth = 0

    def adopt(self, fact: Fact, measured: bool) -> Fact:
        held = self.facts.setdefault(fact.key, fact)
        if measured:
            self.measured.setdefault(fact.key, held)
        return held


_STORE = _FactStore()
LEDGER = _STORE.measured  # the measurement facts save_ledger writes (read-only view by convention)


def misses() -> int:
    """Computations performed so far in this process (cache misses)."""
    return _STORE.misses


@dataclass(frozen=True)
class Analysis:
    """A declared analysis. Bump ``version`` when the computation's meaning
    changes: every key derived from it changes with it."""

    name: str
    version: int
    fn: Callable
    ledger: bool = False

    @property
    def tag(self) -> str:
        return f"{self.name}@v{self.version}"

    def key_of(self, *inputs, **params) -> str:
        d = _Digest()
        d.record(b"analysis", self.tag.encode())
        d.add(list(inputs))
        d.add(params)
        return d.hexdigest()

    def __call__(self, *inputs, **params) -> Fact:
        key = self.key_of(*inputs, **params)
        held = _STORE.facts.get(key)
        if held is not None:
            return held
        if _STORE.warm_depth:
            raise Reanalysis(f"{self.tag} missed inside no_reanalysis() (key {key[:12]})")
        _STORE.misses += 1
        value = self.fn(*(x.value if isinstance(x, Fact) else x for x in inputs), **params)
        if self.ledger:
            value = _as_record(self.tag, value)
        return _STORE.adopt(Fact(key, self.tag, value), self.ledger)


def _as_record(tag: str, value):
    """A measurement's value as it will read back from the ledger file (tuples
    become lists): the in-session fact and a reloaded one are identical."""
    try:
        return json.loads(json.dumps(value, allow_nan=False))
    except (TypeError, ValueError) as exc:
        raise TypeError(
            f"measurement {tag} returned {type(value).__name__}, which is not plain data "
            f"(JSON: dicts, lists, strings, finite numbers, booleans, null): {exc}"
        ) from exc


def defanalysis(name: str, version: int = 1, *, ledger: bool = False):
    """Declare an analysis over a function of the unwrapped inputs;
    ``ledger=True`` marks a measurement."""

    def deco(fn: Callable) -> Analysis:
        return Analysis(name, version, fn, ledger)

    return deco


@contextlib.contextmanager
def no_reanalysis():
    """Everything inside must be a cache hit; a miss raises ``Reanalysis``."""
    _STORE.warm_depth += 1
    try:
        yield
    finally:
        _STORE.warm_depth -= 1


def save_ledger(path) -> int:
    """Write every measurement to ``path`` (JSON Lines, see the module
    docstring); returns how many. Other facts never persist: they are
    recomputed from their inputs."""
    path = Path(path)
    lines = [json.dumps(_LEDGER_HEADER, sort_keys=True)]
    for key in sorted(_STORE.measured):
        f = _STORE.measured[key]
        lines.append(json.dumps({"key": key, "analysis": f.analysis, "value": f.value}, sort_keys=True))
    tmp = path.with_name(path.name + ".partial")
    tmp.write_text("\n".join(lines) + "\n")
    os.replace(tmp, path)
    return len(lines) - 1


def read_ledger(path) -> list:
    """The measurement records of a ledger file, as Facts (nothing cached)."""
    rows = [ln for ln in Path(path).read_text().splitlines() if ln.strip()]
    if not rows or json.loads(rows[0]) != _LEDGER_HEADER:
        raise ValueError(f"{path} is not a measurement ledger (its first line must be {json.dumps(_LEDGER_HEADER)})")
    out = []
    for n, ln in enumerate(rows[1:], start=2):
        rec = json.loads(ln)
        if not isinstance(rec, dict) or set(rec) != {"key", "analysis", "value"}:
            raise ValueError(f"{path}:{n}: a ledger record holds exactly key, analysis and value")
        out.append(Fact(rec["key"], rec["analysis"], rec["value"]))
    return out


def load_ledger(path) -> int:
    """Seed the cache from a saved ledger, so a reloaded measurement is a hit
    and is never taken again; returns how many records the file holds.
    A measurement already taken in this session is kept."""
    facts = read_ledger(path)
    for f in facts:
        _STORE.adopt(f, measured=True)
    return len(facts)


def clear(ledger_too: bool = False) -> None:
    """Drop cached facts; measurements stay hits unless ``ledger_too``."""
    _STORE.facts.clear()
    if ledger_too:
        _STORE.measured.clear()
    else:
        _STORE.facts.update(_STORE.measured)


__all__ = ["Analysis", "Fact", "LEDGER", "Reanalysis", "clear", "defanalysis", "load_ledger", "misses",
           "no_reanalysis", "read_ledger", "save_ledger"]
