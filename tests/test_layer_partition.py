"""Host-side check of the one-launch decode layer's work partition
(mstar_amd/csrc/layer_sync.h, the code the kernel runs): for every down
range, the gate_up ranges it claims before waiting cover every gate_up item
of its experts -- the condition under which no down-phase wait can depend on
a gate_up range nobody has claimed.  Brute force over the shapes the kernel
serves and small odd ones; the header is compiled with g++."""
from __future__ import annotations

import os
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HDR = os.path.join(ROOT, "mstar_amd", "csrc", "layer_sync.h")

PROG = r'''
#include <cstdio>
#include "layer_sync.h"
using namespace mstar;
int main() {
  long checked = 0;
  const int ipes[][2] = {{96, 128}, {48, 64}, {96, 64}, {3, 5}, {7, 2}, {1, 1}};
  const int nwgs[] = {1, 7, 64, 80, 256, 304, 1024};
  for (auto& pp : ipes)
    for (int nwg : nwgs)
      for (int n_act = 0; n_act <= 260; n_act += (n_act < 20 ? 1 : 37)) {
        const int ipe1 = pp[0], ipe2 = pp[1];
        const int total1 = n_act * ipe1;
        const int t1 = (total1 + nwg - 1) / nwg;
        for (int r = 0; r < nwg; ++r) {
          int d0, d1, lo, hi;
          layer_range(n_act, ipe2, nwg, r, &d0, &d1);
          layer_dependencies(n_act, ipe1, ipe2, nwg, r, &lo, &hi);
          if (d0 >= d1) { if (hi >= lo) { printf("FAIL empty r=%d\n", r); return 1; } continue; }
          for (int a = d0 / ipe2; a <= (d1 - 1) / ipe2; ++a)
            for (int it = a * ipe1; it < (a + 1) * ipe1; ++it) {
              const int q = it / t1;  // the gate_up range that holds item it
              int q0, q1;
              layer_range(n_act, ipe1, nwg, q, &q0, &q1);
              if (!(q0 <= it && it < q1)) { printf("FAIL range n=%d q=%d\n", n_act, q); return 1; }
              if (q < lo || q > hi) {
                printf("FAIL dep nwg=%d n_act=%d ipe=%d/%d r=%d item=%d q=%d [%d,%d]\n",
                       nwg, n_act, ipe1, ipe2, r, it, q, lo, hi);
                return 1;
              }
              ++checked;
            }
          // No claim outside the gate_up ranges that exist.
          if (lo < 0 || hi > nwg - 1) { printf("FAIL bounds\n"); return 1; }
        }
      }
  printf("ok %ld\n", checked);
  return 0;
}
'''


def test_down_ranges_claim_every_gate_range_they_wait_on():
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "t.cpp"), os.path.join(d, "t")
        open(src, "w").write(PROG)
        r = subprocess.run(["g++", "-O2", "-std=c++17", "-I", os.path.dirname(HDR), src, "-o", exe],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr
        out = subprocess.run([exe], capture_output=True, text=True, timeout=120)
        assert out.returncode == 0 and out.stdout.startswith("ok"), out.stdout
