"""Two host threads make their first library calls at the same time, as the
reference's per-GPU executor threads do (mstar/worker/worker.py:1164-1175;
test/modular/test_worker_thread_device.py:45-80).  The run happens in a
fresh process so that the per-device launch state (CU count, LDS opt-ins,
occupancy) is built by those concurrent first calls; each thread runs on
its own stream, and both results must match the oracle."""
from __future__ import annotations

import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu
REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = r'''
import threading, torch
from oracle import moe_oracle as O
from tests._util import assert_moe_close
from tests.test_gpu_moe import _fp8_ref, _hidden, _routing

DEV = "cuda"
H, E, I, k = 2048, 128, 768, 8
g = torch.Generator().manual_seed(0)
w1 = torch.randn(E, 2 * I, H, generator=g) * 0.02
w2 = torch.randn(E, H, I, generator=g) * 0.02
# Quantised on the CPU so that no library call happens before the threads start.
from mstar_amd import quant as Q
q1, s1 = Q.quantize_fp8_block(w1)
q2, s2 = Q.quantize_fp8_block(w2)
q1, s1, q2, s2 = (t.to(DEV) for t in (q1, s1, q2, s2))
cases = {}
for M in (32, 700):
    x = _hidden(M, H, seed=M)
    tw, ti = _routing(M, E, k, seed=M, bias=M > 32)
    cases[M] = (x, tw, ti)
dev_in = {M: (x.to(DEV), tw.to(DEV), ti.to(DEV)) for M, (x, tw, ti) in cases.items()}
torch.cuda.synchronize()
from mstar_amd.fused_moe import fused_experts
results, errors = {}, []
barrier = threading.Barrier(2)

def worker(order):
    try:
        torch.cuda.set_device(0)
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            barrier.wait()
            for M in order:
                x, tw, ti = dev_in[M]
                out = fused_experts(x, q1, q2, tw, ti, quant="fp8_w8a8", w1_scale=s1, w2_scale=s2)
                s.synchronize()
                results[(order[0], M)] = out.cpu()
    except Exception as e:  # reported by the main thread
        errors.append(repr(e))

ts = [threading.Thread(target=worker, args=(o,)) for o in ((32, 700), (700, 32))]
for t in ts: t.start()
for t in ts: t.join()
assert not errors, errors
assert len(results) == 4
for (first, M), out in results.items():
    x, tw, ti = cases[M]
    ref = _fp8_ref(x, q1, s1, q2, s2, tw, ti)
    assert_moe_close(out, ref, what=f"thread starting with M={first}, M={M}")
for M in (32, 700):
    assert torch.equal(results[(32, M)], results[(700, M)])
print("threads ok")
'''


def test_concurrent_first_calls_from_two_threads():
    env = dict(os.environ)
    env["PYTHONPATH"] = REPO + os.pathsep + env.get("PYTHONPATH", "")
    print("child: two threads, first fused_experts calls (fp8 M=32 / M=700)", flush=True)
    r = subprocess.run([sys.executable, "-c", CHILD], cwd=REPO, env=env, capture_output=True,
                       text=True, timeout=100)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "threads ok" in r.stdout
