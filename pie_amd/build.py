"""Build libpie_hip.so (the gfx950 kernels + C ABI) in-tree with hipcc.

    python -m pie_amd.build          # or: python pie_amd/build.py

Each ``csrc/*.hip`` file is compiled in parallel to ``pie_amd/_build/*.o`` and linked into
``pie_amd/libpie_hip.so``. hipcc cross-compiles for gfx950 without a GPU present.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libpie_hip.so"
# measurement probes (plain kernels with a hot-path kernel's access pattern; bench.py --op ceiling)
PROBE_SRC = PKG / "probe" / "probe.hip"
PROBE_LIB = PKG / "libpie_probe.so"
ARCH = "gfx950"

# Packed fp32 VALU ops are disabled: hipcc would otherwise form v_pk_{add,mul,fma}_f32 from
# ordinary float code, and some of their forms are unreliable on the target machines.
HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (needs ROCm)")


def _compile(hipcc: str, src: Path, build_dir: Path, defines: tuple[str, ...]) -> Path:
    obj = build_dir / (src.stem + ".o")
    cmd = [hipcc, *HIP_FLAGS, *[f"-D{d}" for d in defines], "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = False, out: Path | None = None, defines: tuple[str, ...] = ()) -> Path:
    """Compile every kernel source and link libpie_hip.so (or ``out``); returns its path.
    ``defines`` (e.g. ``("PIE_NT_LOAD=0",)``) produce measurement variants of the library."""
    hipcc = _hipcc()
    lib = Path(out) if out else LIB
    build_dir = BUILD if not defines else BUILD / ("v_" + "_".join(defines).replace("=", ""))
    build_dir.mkdir(parents=True, exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError(f"no kernel sources under {CSRC}")
    jobs = min(len(srcs), int(os.environ.get("MAX_JOBS", "8")), 16)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(hipcc, s, build_dir, tuple(defines)), srcs))
    tmp = lib.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib}")
    if not defines and out is None:
        build_probe(verbose)
    return lib


def build_probe(verbose: bool = False) -> Path:
    """The measurement-probe library (not part of the C ABI)."""
    tmp = PROBE_LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), *HIP_FLAGS, "-shared", "-o", str(tmp), str(PROBE_SRC)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {PROBE_SRC.name}:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, PROBE_LIB)
    if verbose:
        print(f"built {PROBE_LIB}")
    return PROBE_LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
