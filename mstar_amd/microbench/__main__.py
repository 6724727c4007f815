"""Build and run the micro-benchmarks on the current GPU.

``python -m mstar_amd.microbench``      machine ceilings (peak.hip)
``python -m mstar_amd.microbench lds``  ds_read_b128 lane passes (lds_banks.hip)

Binaries are written to ``mstar_amd/_build/``."""
from __future__ import annotations

import os
import subprocess
import sys

from mstar_amd.build import ARCH, _hipcc

HERE = os.path.dirname(os.path.abspath(__file__))
BUILD = os.path.join(os.path.dirname(HERE), "_build")
PROGRAMS = {"peak": "peak.hip", "lds": "lds_banks.hip"}


def build(name: str = "peak") -> str:
    out = os.path.join(BUILD, name)
    os.makedirs(BUILD, exist_ok=True)
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           os.path.join(HERE, PROGRAMS[name]), "-o", out]
    subprocess.run(cmd, check=True, capture_output=True)
    return out


if __name__ == "__main__":
    args = [a for a in sys.argv[1:] if not a.startswith("--")]
    name = args[0] if args else "peak"
    out = os.path.join(BUILD, name)
    exe = out if "--no-build" in sys.argv and os.path.exists(out) else build(name)
    sys.exit(subprocess.run([exe]).returncode)
