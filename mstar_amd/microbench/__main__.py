"""Build and run the machine-ceiling micro-benchmarks (peak.hip) on the
current GPU: ``python -m mstar_amd.microbench``.  The binary is written to
``mstar_amd/_build/peak``."""
from __future__ import annotations

import os
import subprocess
import sys

from mstar_amd.build import ARCH, _hipcc

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(os.path.dirname(HERE), "_build", "peak")


def build() -> str:
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           os.path.join(HERE, "peak.hip"), "-o", OUT]
    subprocess.run(cmd, check=True, capture_output=True)
    return OUT


if __name__ == "__main__":
    exe = OUT if "--no-build" in sys.argv and os.path.exists(OUT) else build()
    sys.exit(subprocess.run([exe]).returncode)
