"""Build libdispec_probe.so, the bandwidth probes bench.py calibrates its rooflines with.

The probes (read_probe.hip, declared in dsp_probe.h) are measurement instruments, not part
of the product library: nothing in the KV path calls them and libdispec_hip.so does not
contain them.  They use the product's device helpers (dispec_amd/csrc/dsp_common.h) and
the same hipcc flags.  Run as `python -m bench_probes.build`; __graft_entry__.build()
calls it after the product build.
"""

from __future__ import annotations

import sys
from pathlib import Path

from dispec_amd.build import _compile, _link

HERE = Path(__file__).resolve().parent
LIB = HERE / "libdispec_probe.so"
OBJ_DIR = HERE / "_build"


def build(verbose: bool = False) -> Path:
    OBJ_DIR.mkdir(exist_ok=True)
    objs = [_compile(src, verbose, OBJ_DIR) for src in sorted(HERE.glob("*.hip"))]
    return _link(objs, LIB, verbose)


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
