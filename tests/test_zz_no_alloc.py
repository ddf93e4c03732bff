"""GPU check of tlg_dev_sgemm_tn_acc_noalloc, the mm_atb entry point that
allocates nothing (its split partials live in a fixed device array of the
library).  It must give what tlg_dev_sgemm_tn_acc gives on the same inputs --
bit for bit, since both launch the same kernels with the same split plan --
and stay within the parity bar of the CPU oracle (max|err| / mean|ref| <=
1e-4, tinylm.c:4782-4784).  Two calls in a row, the second smaller, so stale
partials of the first call in the shared array would show."""
import ctypes

import numpy as np
import pytest

from oracle import normwise_rel

pytestmark = pytest.mark.gpu
TOL = 1e-4


def _run(lib, entry, dW0, X, dY):
    import torch
    M, K = X.shape
    N = dY.shape[1]
    o = torch.from_numpy(dW0.copy()).cuda()
    x = torch.from_numpy(X).cuda()
    g = torch.from_numpy(dY).cuda()
    s = torch.cuda.current_stream().cuda_stream
    lib.check(getattr(lib.dll, entry)(o.data_ptr(), x.data_ptr(), g.data_ptr(), M, K, N, s), entry)
    torch.cuda.synchronize()
    return o.cpu().numpy()


# (M, K, N): the m3 W1/W3 weight gradient (split reduction over 4096 rows),
# then a smaller ragged one (scalar staging, fewer splits)
CASES = [(4096, 256, 768), (777, 67, 45)]


def test_noalloc_matches_workspace_entry(lib, orc):
    r = np.random.default_rng(20261202)
    for M, K, N in CASES:
        print("noalloc case", (M, K, N), flush=True)
        X = r.standard_normal((M, K), dtype=np.float32)
        dY = (0.01 * r.standard_normal((M, N))).astype(np.float32)
        dW0 = r.standard_normal((K, N), dtype=np.float32)
        got = _run(lib, "tlg_dev_sgemm_tn_acc_noalloc", dW0, X, dY)
        ref = _run(lib, "tlg_dev_sgemm_tn_acc", dW0, X, dY)
        assert np.array_equal(got, ref), normwise_rel(got, ref)
        want = orc.mm_atb(dW0.copy(), X, dY)
        assert normwise_rel(got, want) <= TOL
        # the increment alone, against fp64 (the prefill dominates the sum)
        inc64 = X.astype(np.float64).T @ dY.astype(np.float64)
        assert normwise_rel(got.astype(np.float64) - dW0, inc64) <= TOL


def test_noalloc_rejects_oversized_dw(lib):
    # 2048 x 2048 floats is above the 2^21-float limit: refused before any launch
    rc = lib.dll.tlg_dev_sgemm_tn_acc_noalloc(None, None, None, 16, 2048, 2048, None)
    assert rc == -1
    assert b"no-allocation limit" in lib.dll.tlg_last_error()
    assert lib.dll.tlg_dev_sgemm_tn_acc_noalloc(None, None, None, -1, 4, 4, None) == -1
