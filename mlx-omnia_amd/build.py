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
    # gfx950 can hand a kernel's leading scalar and pointer arguments to it in user
    # SGPRs at wave launch (kernarg preloading, LLVM AMDGPUUsage "Preloaded Kernel
    # Arguments"): no scalar load round trip before the first vector load. Arguments
    # passed as a struct by value are not preloaded; those kernels are unchanged. Each
    # kernel keeps a compatibility entry that loads the arguments itself, which firmware
    # without preloading runs instead.
    "-mllvm",
    "-amdgpu-kernarg-preload-count=16",
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


def build_library(verbose: bool = True, clocks: bool | None = None) -> Path:
    """Compile every source under `csrc/` and link `libomnia_hip.so`; returns its path.

    `clocks` (default: the environment variable OMNIA_BUILD_CLOCKS=1) also builds the
    router's phase-clock diagnostic library, which only `bench.py --phase-clocks` loads
    (see `build_clocks_library`)."""
    if clocks is None:
        clocks = os.environ.get("OMNIA_BUILD_CLOCKS", "") == "1"
    OBJDIR.mkdir(exist_ok=True)
    sources = sorted([*CSRC.glob("*.hip"), *CSRC.glob("*.cpp")])
    if not sources:
        raise FileNotFoundError(f"no sources under {CSRC}")
    workers = min(len(sources), max(1, (os.cpu_count() or 2) // 2), 8)
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(_compile, sources))
    _link(objects, LIBRARY)
    if verbose:
        print(f"built {LIBRARY.relative_to(REPO)} from {len(sources)} sources", flush=True)
    if clocks:
        build_clocks_library(verbose)
    return LIBRARY


def build_clocks_library(verbose: bool = True) -> Path:
    """The router and the ABI bookkeeping compiled with the phase-clock marks on, linked
    into `libomnia_router_clocks.so` beside the product library (never loaded by the
    package)."""
    OBJDIR.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(CLOCKS_SOURCES)) as pool:
        objects = list(pool.map(
            lambda name: _compile(CSRC / name, ("-DOMNIA_PHASE_CLOCKS",), ".clocks"),
            CLOCKS_SOURCES))
    _link(objects, CLOCKS_LIBRARY)
    if verbose:
        print(f"built {CLOCKS_LIBRARY.relative_to(REPO)} (diagnostic)", flush=True)
    return CLOCKS_LIBRARY


if __name__ == "__main__":
    build_library(verbose=True, clocks="--clocks" in sys.argv[1:] or None)
    sys.exit(0)
