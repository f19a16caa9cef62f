"""Analyses as cached facts, and measurements as a persistent ledger.

Restates the reference's analysis cache
(packages/tensorlib/src/pdum/tl/analysis.py:1-155):

  * an ``Analysis`` is declared as name@version over a function; calling it
    on inputs yields a ``Fact`` whose key is the sha256 of the fingerprint,
    the canonical inputs and the keyword parameters (analysis.py:95-123);
  * inputs canonicalize by content: a Fact contributes its KEY (so a fact
    derived from another never recomputes its prefix), IR regions and nodes
    their content key, plain data structurally, ndarrays by dtype, shape and
    a digest of their bytes; anything else refuses (analysis.py:52-82);
  * ``ledger=True`` marks a MEASUREMENT: its value must be plain JSON data
    and it is recorded in ``LEDGER``, which ``save_ledger`` / ``load_ledger``
    round-trip through a JSON file, so an identically keyed measurement is
    never taken twice, across sessions too (analysis.py:126-155);
  * ``no_reanalysis()`` is the warmth law: inside it, any cache miss raises
    (the reference forbids the ``analysis.miss`` event, analysis.py:121-124).

There is no invalidation: regions are immutable and content-addressed, so a
changed program is a different key.
"""

from __future__ import annotations

import contextlib
import hashlib
import json
from dataclasses import dataclass
from pathlib import Path
from typing import Callable

import numpy as np


class Reanalysis(RuntimeError):
    """A cache miss inside ``no_reanalysis()``."""


@dataclass(frozen=True)
class Fact:
    """One cached analysis result: ``key`` is its identity, ``analysis`` its
    provenance (name@vN), ``value`` the payload."""

    key: str
    analysis: str
    value: object


_CACHE: dict[str, Fact] = {}
LEDGER: dict[str, Fact] = {}  # the measurement subset: what save/load persist
_FORBID = [0]  # nesting depth of no_reanalysis()
MISSES = [0]  # total misses this process (computations performed)


def _canon(x):
    """A stable content-addressed shape for one analysis input."""
    if isinstance(x, Fact):
        return ("fact", x.key)
    k = getattr(x, "key", None)
    if isinstance(k, bytes):
        return ("ir", k.hex())
    if x is None or isinstance(x, bool):
        return ("lit", x)
    if isinstance(x, (str, int, float)):
        return ("lit", x)
    if isinstance(x, bytes):
        return ("bytes", x.hex())
    if isinstance(x, (tuple, list)):
        return ("seq", tuple(_canon(e) for e in x))
    if isinstance(x, (set, frozenset)):
        return ("set", tuple(sorted(repr(_canon(e)) for e in x)))
    if isinstance(x, dict):
        return ("map", tuple(sorted((str(kk), _canon(v)) for kk, v in x.items())))
    if isinstance(x, np.ndarray):
        a = np.ascontiguousarray(x)
        return ("arr", str(a.dtype), a.shape, hashlib.sha256(a.tobytes()).hexdigest())
    raise TypeError(
        f"analysis inputs must be content-keyable (Fact, Region/Node, plain data, ndarray); got "
        f"{type(x).__name__}: an unkeyable input has no honest cache identity"
    )


@dataclass(frozen=True)
class Analysis:
    """A declared analysis. Bump ``version`` when the computation's meaning
    changes: every key derived from it changes with it."""

    name: str
    version: int
    fn: Callable
    ledger: bool = False

    def key_of(self, *inputs, **params) -> str:
        payload = ("analysis", self.name, self.version, _canon(inputs), _canon(params))
        return hashlib.sha256(repr(payload).encode()).hexdigest()

    def __call__(self, *inputs, **params) -> Fact:
        key = self.key_of(*inputs, **params)
        hit = _CACHE.get(key)
        if hit is not None:
            return hit
        if _FORBID[0]:
            raise Reanalysis(f"analysis miss inside no_reanalysis(): {self.name}@v{self.version}")
        MISSES[0] += 1
        args = tuple(x.value if isinstance(x, Fact) else x for x in inputs)
        value = self.fn(*args, **params)
        if self.ledger:
            # measurements are records: normalized through JSON now, so the
            # in-session value and a reloaded one are identical
            try:
                value = json.loads(json.dumps(value))
            except TypeError as exc:
                raise TypeError(
                    f"ledger analysis {self.name!r} produced a non-JSON value ({type(value).__name__}): "
                    "measurements are plain data"
                ) from exc
        fact = Fact(key, f"{self.name}@v{self.version}", value)
        _CACHE[key] = fact
        if self.ledger:
            LEDGER[key] = fact
        return fact


def defanalysis(name: str, version: int = 1, *, ledger: bool = False):
    """Declare an analysis over a function of the unwrapped inputs;
    ``ledger=True`` marks a measurement."""

    def deco(fn: Callable) -> Analysis:
        return Analysis(name, version, fn, ledger)

    return deco


@contextlib.contextmanager
def no_reanalysis():
    """Everything inside must be a cache hit; a miss raises ``Reanalysis``."""
    _FORBID[0] += 1
    try:
        yield
    finally:
        _FORBID[0] -= 1


def save_ledger(path) -> int:
    """Write the measurement facts to ``path`` as sorted JSON; returns the count.
    Non-ledger facts never persist (they are rebuilt from their keys)."""
    data = {k: {"analysis": f.analysis, "value": f.value} for k, f in sorted(LEDGER.items())}
    Path(path).write_text(json.dumps(data, indent=1, sort_keys=True))
    return len(data)


def load_ledger(path) -> int:
    """Seed the cache from a saved ledger: a reloaded measurement is a hit and
    is never taken again. Loading is a cold act (do it outside warm loops)."""
    data = json.loads(Path(path).read_text())
    for key, rec in data.items():
        fact = Fact(key, rec["analysis"], rec["value"])
        LEDGER[key] = fact
        _CACHE[key] = fact
    return len(data)


def clear(ledger_too: bool = False) -> None:
    """Drop cached facts (tests use this to start cold)."""
    _CACHE.clear()
    if ledger_too:
        LEDGER.clear()
    else:
        _CACHE.update(LEDGER)  # measurements stay hits


__all__ = ["Analysis", "Fact", "LEDGER", "Reanalysis", "clear", "defanalysis", "load_ledger", "no_reanalysis",
           "save_ledger"]
