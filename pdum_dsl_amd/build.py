"""Build libpdhip.so — every HIP source under csrc/ compiled for gfx950 and
linked into one shared library that sits next to this file (in-tree, so it
travels with the repository snapshot to the GPU host).

    python -m pdum_dsl_amd.build            # compile (always rebuilds)
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libpdhip.so"
ARCH = "gfx950"

# -packed-fp32-ops off: v_pk_{add,mul,fma}_f32 stay out of every code object.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found: the HIP backend needs ROCm's hipcc to build")
    return exe


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr}")


def build(verbose: bool = False) -> Path:
    """Compile every csrc/*.hip and link libpdhip.so (atomically replaced)."""
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    with tempfile.TemporaryDirectory(prefix="pdhip_build_") as tmp:
        objs = [Path(tmp) / (s.stem + ".o") for s in srcs]
        workers = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", "8"))))
        with cf.ThreadPoolExecutor(workers) as ex:
            list(ex.map(_compile, srcs, objs))
        out_tmp = LIB.with_suffix(".so.tmp")
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(out_tmp), *map(str, objs)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link of libpdhip.so failed:\n{res.stderr}")
        os.replace(out_tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
