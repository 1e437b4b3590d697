"""Build libdispec_hip.so from dispec_amd/csrc/*.hip for gfx950 with hipcc.

Every source is compiled to an object in dispec_amd/_build/ (in parallel), then linked
into dispec_amd/libdispec_hip.so in-tree, where the loader looks for it, and the fast
binding csrc/fastcall.c into the dispec_amd._fastcall module.  Run as
`python -m dispec_amd.build`.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ_DIR = PKG / "_build"
LIB = PKG / "libdispec_hip.so"
ARCH = os.environ.get("DISPEC_HIP_ARCH", "gfx950")

# Packed-fp32 VALU ops are switched off for all device code: hipcc would otherwise form
# v_pk_{add,mul,fma}_f32 from plain float code.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Wno-unused-command-line-argument",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", str(PKG.parent / "include"),
]


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the HIP toolchain is needed to build libdispec_hip.so")
    return path


def _compile(src: Path, verbose: bool, obj_dir: Path = OBJ_DIR) -> Path:
    obj = obj_dir / (src.stem + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def _link(objs: list[Path], lib: Path, verbose: bool) -> Path:
    tmp = lib.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of {lib.name} failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, lib)
    return lib


def _build_fastcall(verbose: bool) -> Path:
    """csrc/fastcall.c -> the CPython module dispec_amd._fastcall (gcc; host code only)."""
    import sysconfig
    out = PKG / ("_fastcall" + sysconfig.get_config_var("EXT_SUFFIX"))
    tmp = out.with_name(out.name + ".tmp")
    cmd = ["gcc", "-O2", "-shared", "-fPIC", "-Wall", "-I", sysconfig.get_paths()["include"],
           str(CSRC / "fastcall.c"), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"gcc failed on fastcall.c:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    return out


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every csrc/*.hip into libdispec_hip.so (the product library) and
    csrc/fastcall.c into the dispec_amd._fastcall module.  Returns the library path."""
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    OBJ_DIR.mkdir(exist_ok=True)
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 2)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda s: _compile(s, verbose), sources))
    _build_fastcall(verbose)
    return _link(objs, LIB, verbose)


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
