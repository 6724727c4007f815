"""Host-side model of the one-launch decode layer's forward-progress protocol
(stream_fp8.hip, LayerSync), run under adversarial schedules.

The kernel's rule: a workgroup claims its own gate_up range when it starts
(0 -> 1); if another workgroup took it first, it stops its gate_up work and
reports nothing for it.  After its own gate_up work it claims (0 -> 2) every
gate_up range its down range depends on (layer_dependencies in
mstar_amd/csrc/layer_sync.h, the header the kernel uses) and runs the ones it
won, reporting each.  Then its down phase waits, expert by expert, until the
expert's gate_up work is fully reported.

This test replays that state machine in an event simulation compiled from
the same header: only R of the launch's workgroups are resident at a time
(R down to 1), workgroups start in a random order and at random delays, and
work takes random time.  It checks that every launch completes (no wait
depends on a workgroup that is not running), that every gate_up range is
reported exactly once, and that every expert's count reaches its target.
A protocol without the take-over step (claims only) deadlocks under the same
schedules, which the test also checks, so the model is not vacuous."""
from __future__ import annotations

import os
import subprocess
import tempfile

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HDR_DIR = os.path.join(ROOT, "mstar_amd", "csrc")

PROG = r'''
#include <cstdio>
#include <cstdlib>
#include <vector>
#include <queue>
#include <random>
#include <algorithm>
#include "layer_sync.h"
using namespace mstar;

// One launch: nwg workgroups, R resident at a time. Returns 0 ok, 1 deadlock, 2 double report.
static int simulate(int n_act, int ipe1, int ipe2, int nwg, int R, bool take_over, unsigned seed,
                    long* reports_out) {
  std::mt19937 rng(seed);
  std::uniform_real_distribution<double> U(0.0, 1.0);
  std::vector<int> rows(n_act);
  for (auto& r : rows) r = 1 + (int)(U(rng) * 4);
  std::vector<long> target(n_act), done(n_act, 0);
  for (int a = 0; a < n_act; ++a) target[a] = (long)ipe1 * rows[a];
  std::vector<int> claim(nwg, 0), reported(nwg, 0);
  enum St { NOT_STARTED, OWN, STEALS, DOWN, FINISHED };
  struct WG { St st = NOT_STARTED; bool own_ok = false; std::vector<int> steals; size_t next = 0;
              double t = 0; int a_wait = 0; int a_end = -1; };
  std::vector<WG> wg(nwg);
  // dispatch order: random permutation (hardware order is by index; late CUs model delays)
  std::vector<int> order(nwg);
  for (int i = 0; i < nwg; ++i) order[i] = i;
  std::shuffle(order.begin(), order.end(), rng);
  size_t disp = 0;
  int running = 0;
  auto report = [&](int q) -> bool {
    if (reported[q]++) return false;  // a second report of a range
    int i0, i1;
    layer_range(n_act, ipe1, nwg, q, &i0, &i1);
    for (int it = i0; it < i1; ++it) done[it / ipe1] += rows[it / ipe1];
    return true;
  };
  auto range_items = [&](int q) { int i0, i1; layer_range(n_act, ipe1, nwg, q, &i0, &i1); return i1 - i0; };
  // Event loop: repeatedly pick a random runnable workgroup and advance it one step.
  for (long iter = 0; iter < 50000000; ++iter) {
    while (running < R && disp < order.size()) {  // fill free slots
      WG& w = wg[order[disp++]];
      w.st = OWN;
      ++running;
      const int b = order[disp - 1];
      w.own_ok = claim[b] == 0;
      if (w.own_ok) claim[b] = 1;
    }
    std::vector<int> runnable;
    bool all_done = true;
    for (int b = 0; b < nwg; ++b) {
      WG& w = wg[b];
      if (w.st != FINISHED) all_done = false;
      if (w.st == OWN || w.st == STEALS) runnable.push_back(b);
      if (w.st == DOWN) {
        if (w.a_wait > w.a_end || done[w.a_wait] >= target[w.a_wait]) runnable.push_back(b);
      }
    }
    if (all_done) {
      for (int a = 0; a < n_act; ++a) if (done[a] != target[a]) return 3;
      long n = 0; for (int q = 0; q < nwg; ++q) n += reported[q];
      *reports_out = n;
      return 0;
    }
    if (runnable.empty()) return 1;  // every resident workgroup waits: deadlock
    const int b = runnable[(size_t)(U(rng) * runnable.size()) % runnable.size()];
    WG& w = wg[b];
    if (w.st == OWN) {
      // own range done (or stopped because it was taken); report only if ours
      if (w.own_ok && range_items(b) > 0 && !report(b)) return 2;
      // claim the ranges the down range depends on
      int lo, hi;
      layer_dependencies(n_act, ipe1, ipe2, nwg, b, &lo, &hi);
      if (take_over)
        for (int q = lo; q <= hi; ++q)
          if (claim[q] == 0) { claim[q] = 2; w.steals.push_back(q); }
      w.st = STEALS;
    } else if (w.st == STEALS) {
      if (w.next < w.steals.size()) {
        const int q = w.steals[w.next++];
        if (range_items(q) > 0 && !report(q)) return 2;
      } else {
        int d0, d1;
        layer_range(n_act, ipe2, nwg, b, &d0, &d1);
        w.a_wait = d0 < d1 ? d0 / ipe2 : 1;
        w.a_end = d0 < d1 ? (d1 - 1) / ipe2 : 0;
        w.st = DOWN;
      }
    } else if (w.st == DOWN) {
      if (w.a_wait > w.a_end) { w.st = FINISHED; --running; }
      else ++w.a_wait;  // this expert's rows are all reported: stage and compute it
    }
  }
  return 4;
}

int main(int argc, char** argv) {
  const bool take_over = atoi(argv[1]) != 0;
  const int shapes[][3] = {{115, 96, 128}, {8, 96, 128}, {40, 48, 64}, {128, 96, 128}, {3, 96, 128}};
  const int Rs[] = {256, 200, 64, 16, 1};
  int fails = 0, runs = 0;
  for (auto& s : shapes)
    for (int R : Rs)
      for (unsigned seed = 1; seed <= 6; ++seed) {
        long reports = 0;
        const int r = simulate(s[0], s[1], s[2], 256, R, take_over, seed * 7919u + R, &reports);
        ++runs;
        if (r != 0) {
          ++fails;
          if (take_over) printf("FAIL code=%d n_act=%d R=%d seed=%u\n", r, s[0], R, seed);
        }
      }
  printf("runs %d fails %d\n", runs, fails);
  return 0;
}
'''


def _run(take_over: int) -> str:
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "m.cpp"), os.path.join(d, "m")
        open(src, "w").write(PROG)
        r = subprocess.run(["g++", "-O2", "-std=c++17", "-I", HDR_DIR, src, "-o", exe],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr
        out = subprocess.run([exe, str(take_over)], capture_output=True, text=True, timeout=300)
        assert out.returncode == 0, out.stderr
        return out.stdout


def test_every_launch_completes_with_each_range_reported_once():
    out = _run(1)
    last = out.strip().splitlines()[-1]
    assert last.endswith("fails 0"), out


def test_without_take_over_some_schedules_deadlock():
    out = _run(0)
    fails = int(out.strip().splitlines()[-1].split()[-1])
    assert fails > 0, out
