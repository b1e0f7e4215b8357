"""Compile the HIP sources under `csrc/` into `libomnia_hip.so` for gfx950.

Run as a script (`python mlx-omnia_amd/build.py`) or through `build_library()`. Every
translation unit is compiled separately (in parallel) and linked into one shared
library next to this file, which is where the runtime loader looks for it.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
REPO = PACKAGE.parent
CSRC = PACKAGE / "csrc"
INCLUDE = REPO / "include"
OBJDIR = PACKAGE / "_build"
LIBRARY = PACKAGE / "libomnia_hip.so"

ARCH = "gfx950"

FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    # Results are compared with a CPU restatement operation by operation; no
    # contraction of a*b+c into fma unless a kernel asks for one explicitly.
    "-ffp-contract=off",
    # No packed-fp32 instructions in any kernel.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise FileNotFoundError("hipcc not found (expected /opt/rocm/bin/hipcc)")
    return found


# Diagnostic library: the router and the ABI bookkeeping compiled with the phase-clock
# marks on (`bench.py --phase-clocks` loads it). Not loaded by the package.
CLOCKS_LIBRARY = PACKAGE / "libomnia_router_clocks.so"
CLOCKS_SOURCES = ("router.hip", "abi.cpp")


def _compile(source: Path, defines: tuple[str, ...] = (), tag: str = "") -> Path:
    obj = OBJDIR / (source.name + tag + ".o")
    cmd = [_hipcc(), *FLAGS, *defines, "-c", str(source), "-o", str(obj)]
    if source.suffix == ".hip":
        cmd[1:1] = ["-x", "hip"]
    done = subprocess.run(cmd, capture_output=True, text=True)
    if done.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source.name}:\n{done.stdout}\n{done.stderr}")
    return obj


def _link(objects: list[Path], target: Path) -> None:
    staged = target.with_suffix(".so.tmp")
    cmd = [_hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objects),
           "-o", str(staged)]
    done = subprocess.run(cmd, capture_output=True, text=True)
    if done.returncode != 0:
        raise RuntimeError(f"link failed:\n{done.stdout}\n{done.stderr}")
    os.replace(staged, target)


def build_library(verbose: bool = True) -> Path:
    """Compile every source under `csrc/` and link `libomnia_hip.so` (and the router's
    phase-clock diagnostic library); returns the product library's path."""
    OBJDIR.mkdir(exist_ok=True)
    sources = sorted([*CSRC.glob("*.hip"), *CSRC.glob("*.cpp")])
    if not sources:
        raise FileNotFoundError(f"no sources under {CSRC}")
    clock_sources = [CSRC / name for name in CLOCKS_SOURCES]
    workers = min(len(sources) + len(clock_sources), max(1, (os.cpu_count() or 2) // 2), 8)
    with ThreadPoolExecutor(max_workers=workers) as pool:
        product = [pool.submit(_compile, source) for source in sources]
        clocks = [pool.submit(_compile, source, ("-DOMNIA_PHASE_CLOCKS",), ".clocks")
                  for source in clock_sources]
        objects = [job.result() for job in product]
        clock_objects = [job.result() for job in clocks]
    _link(objects, LIBRARY)
    _link(clock_objects, CLOCKS_LIBRARY)
    if verbose:
        print(f"built {LIBRARY.relative_to(REPO)} from {len(sources)} sources "
              f"(and {CLOCKS_LIBRARY.name})", flush=True)
    return LIBRARY


if __name__ == "__main__":
    build_library(verbose=True)
    sys.exit(0)
