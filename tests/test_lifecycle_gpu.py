"""GPU checks of the library's lifetime, each in a fresh process so its
tlg_init / tlg_shutdown calls leave the test session's library alone.

* Split mm_atb reductions queued by a grouped launch (their partials live in
  the library's workspace) run when tlg_shutdown is called, before the
  workspace is freed: the result is complete and, after a new tlg_init,
  nothing is left queued.
* tlg_dev_sgemm_tn_acc_noalloc works in a process that never called
  tlg_init (its header promises it does not initialise the library), against
  the fp64 product, to the parity bar (max|err| / mean|ref| <= 1e-4,
  tinylm.c:4782-4784).
"""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu
REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

PRELUDE = f"""
import sys
sys.path[:0] = [{os.path.join(REPO, 'tinylm-c_amd')!r}, {os.path.join(REPO, 'oracle')!r}]
import numpy as np, torch, tlgemm
from oracle import normwise_rel
lib = tlgemm.load()
s = torch.cuda.current_stream().cuda_stream
r = np.random.default_rng(4242)
M, K, N = 4096, 256, 768                 # the m3 W1 / W3 weight gradient: a split reduction
X = r.standard_normal((M, K), dtype=np.float32)
dY = (0.01 * r.standard_normal((M, N))).astype(np.float32)
dW0 = r.standard_normal((K, N), dtype=np.float32)
x, g, o = (torch.from_numpy(a).cuda() for a in (X, dY, dW0))
want = dW0.astype(np.float64) + X.astype(np.float64).T @ dY.astype(np.float64)
"""

DRAIN = PRELUDE + """
lib.check(lib.tlg_init(0), "tlg_init")
lib.group([dict(op="mm_atb", beta=1, C=o.data_ptr(), M=M, K=K, N=N, A=[x.data_ptr()], B=[g.data_ptr()])],
          s, flush=False)
assert lib.dll.tlg_dev_gemm_pending() > 0, "the grouped mm_atb left no split reduction queued"
lib.dll.tlg_shutdown()                   # runs the queued reduction, then frees the workspace
got = o.cpu().numpy()
err = normwise_rel(got, want)
assert err <= 1e-4, err
lib.check(lib.tlg_init(0), "tlg_init again")
assert lib.dll.tlg_dev_gemm_pending() == 0
lib.dll.tlg_shutdown()
print("OK", err, flush=True)
"""

NOINIT = PRELUDE + """
rc = lib.dll.tlg_dev_sgemm_tn_acc_noalloc(o.data_ptr(), x.data_ptr(), g.data_ptr(), M, K, N, s)
assert rc == 0, lib.dll.tlg_last_error()
torch.cuda.synchronize()
err = normwise_rel(o.cpu().numpy(), want)
assert err <= 1e-4, err
print("OK", err, flush=True)
"""


def _run(code):
    p = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=180)
    print(p.stdout[-2000:], p.stderr[-2000:], flush=True)
    assert p.returncode == 0 and "OK" in p.stdout


def test_shutdown_runs_queued_reductions():
    _run(DRAIN)


def test_noalloc_without_init():
    _run(NOINIT)
