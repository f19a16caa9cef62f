"""Measurements on MI355X as ledger facts, and the measured picks built on them.

The reference's measured-pick loop (packages/tensorlib/src/pdum/tl/analysis.py:85-155,
conformance/test_fusion_triton.py:87-117) declares a measurement as an
analysis whose evaluator is the machine: its value is plain JSON, it is keyed
by (kernel content, machine, parameters), it is never taken twice for the
same key (across sessions once the ledger is saved and reloaded), and a
group's confidence turns green only on the strength of such a fact.

Here the machine is named by its ISA (``gfx950``), read from the device, so
a ledger written on one MI355X is valid on another. Two measurements:

  * ``hip_ms``: the HIP seat (``compile_tile_hip``) run end to end on seeded
    inputs, host copies included, exactly what the reference times for its
    Triton runner (median of wall-clock laps after one warm-up call);
  * ``decode_split_ms``: the device-resident split-K decode at one split
    count, timed with HIP events on the launch stream.

``tune_decode_splits`` is the autotune-lite pick over the decode's split
ladder; its per-candidate facts are what makes the pick a fact.

``no_compiles`` is the warmth law of the reference's timed loops
(``events.forbid(*WARMTH)``, benchmarks/bench_zoo.py:128-152): inside it no
elementwise program may be compiled by hipRTC, so a first-use compile can
never be timed as kernel work. The HIP
attention, row and contraction kernels have fixed tile shapes on this part,
so the launch ladder of the plan changes no launched work there and is not
measured.
"""

from __future__ import annotations

import contextlib
import ctypes as C
import time
from dataclasses import replace

import numpy as np

from .tl.analysis import defanalysis
from .tl.fusion import Group

DECODE_SPLITS = (1, 2, 4, 8, 16)


def machine_name() -> str:
    """The ISA of device 0, e.g. ``gfx950``; raises without a GPU."""
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("measurements need a GPU: no HIP device is visible")
    arch = torch.cuda.get_device_properties(0).gcnArchName
    return arch.split(":")[0]


def jit_stats() -> dict:
    """The library's runtime-specialization counters: programs compiled by
    hipRTC, launches through specialized kernels, compile failures."""
    from . import _lib

    st = (C.c_int64 * 3)()
    _lib.lib().pdh_ew_jit_stats(st)
    return {"compiled": int(st[0]), "launches": int(st[1]), "failures": int(st[2])}


class WarmthError(RuntimeError):
    """A hipRTC compile happened inside a region declared warm."""


@contextlib.contextmanager
def no_compiles(what: str = "timed region"):
    """Raise ``WarmthError`` if any elementwise program is compiled (or a
    compile fails) while the block runs: timed loops must run warm."""
    before = jit_stats()
    yield
    after = jit_stats()
    if after["compiled"] != before["compiled"] or after["failures"] != before["failures"]:
        raise WarmthError(
            f"{what}: {after['compiled'] - before['compiled']} hipRTC compile(s) and "
            f"{after['failures'] - before['failures']} failure(s) inside a warm region — warm it up first"
        )


def _draw_inputs(kernel, seed: int) -> list:
    rng = np.random.default_rng(seed)
    return [rng.standard_normal(tuple(d.size for d in p.type.dims)) for p in kernel.params]


@defanalysis("fusion.hip-ms", 1, ledger=True)
def hip_ms(kernel, *, machine: str, launch=(), prune=(), dtype: str = "f32", reps: int = 20, seed: int = 0):
    """Median wall-clock ms of the HIP seat's ``run`` on ``kernel`` (inputs
    seeded from the params' types; the compile and the first call stay out of
    the laps)."""
    from .hip_tile import compile_tile_hip

    if machine != machine_name():
        raise RuntimeError(f"asked to measure on {machine!r} but the device is {machine_name()!r}")
    run = compile_tile_hip(kernel, tuple(launch), tuple(prune), dtype=dtype)
    arrays = _draw_inputs(kernel, seed)
    run(arrays)
    laps = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run(arrays)
        laps.append(time.perf_counter() - t0)
    return {"ms": sorted(laps)[len(laps) // 2] * 1e3, "reps": reps, "source": run.source}


def measured_green(group: Group, *, dtype: str = "f32", machine: str | None = None):
    """Measure ``group``'s kernel on this machine and return the group with
    confidence ``green`` together with the fact that licenses the upgrade."""
    if group.kernel is None or group.confidence == "red":
        raise ValueError(f"a {group.confidence} group has no kernel to measure ({group.reason})")
    machine = machine or machine_name()
    fact = hip_ms(group.kernel, machine=machine, launch=group.launch, prune=group.prune, dtype=dtype)
    if not fact.value["ms"] > 0:
        raise RuntimeError(f"measurement {fact.key} reports no time")
    return replace(group, confidence="green"), fact


@defanalysis("decode.split-ms", 1, ledger=True)
def decode_split_ms(*, machine: str, B: int, Hq: int, Hkv: int, S: int, D: int, dtype: str, nsplit: int,
                    reps: int = 20, seed: int = 0):
    """Device time (ms, HIP events on the launch stream, mean of ``reps``
    back-to-back calls) of the split-K decode at ``nsplit``."""
    import torch

    from . import kernels as K

    if machine != machine_name():
        raise RuntimeError(f"asked to measure on {machine!r} but the device is {machine_name()!r}")
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dtype]
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn((B, Hq, 1, D), generator=g, device="cuda").to(tdt)
    k = torch.randn((B, Hkv, S, D), generator=g, device="cuda").to(tdt)
    v = torch.randn((B, Hkv, S, D), generator=g, device="cuda").to(tdt)
    ws = None
    for _ in range(3):
        _, _ = K.attn_decode(q, k, v, nsplit=nsplit, workspace=ws)
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        K.attn_decode(q, k, v, nsplit=nsplit)
    e1.record(stream)
    e1.synchronize()
    return {"ms": e0.elapsed_time(e1) / reps, "reps": reps}


def tune_decode_splits(B: int, Hq: int, Hkv: int, S: int, D: int, *, dtype: str = "bf16",
                       candidates=DECODE_SPLITS, machine: str | None = None):
    """The measured pick over the decode's split ladder: returns
    ``(best_nsplit, facts)``, one fact per legal candidate (ties go to the
    fewer splits). Every candidate is a ledger fact, so a warm re-tune (or a
    reloaded ledger) measures nothing."""
    machine = machine or machine_name()
    cands = [n for n in candidates if 1 <= n <= max(1, S // 32)]
    if not cands:
        raise ValueError(f"no legal split count among {tuple(candidates)} for S={S}")
    facts = {n: decode_split_ms(machine=machine, B=B, Hq=Hq, Hkv=Hkv, S=S, D=D, dtype=dtype, nsplit=n)
             for n in cands}
    best = min(cands, key=lambda n: (facts[n].value["ms"], n))
    return best, facts


__all__ = ["DECODE_SPLITS", "WarmthError", "decode_split_ms", "hip_ms", "jit_stats", "machine_name", "measured_green",
           "no_compiles", "tune_decode_splits"]
