"""GPU parity of the three primitives through the C ABI.

Each case runs libtlgemm.so's HIP kernels and compares with (a) the golden
outputs written by tinylm.c's own kernels and (b) the CPU oracle and its fp64
textbook form on the same seeded inputs.  Bar (north_star): max|gpu - ref| /
mean|ref| <= 1e-4, the reference selftest's normwise metric
(tinylm.c:4782-4784).
"""
import os

import numpy as np
import pytest

from conftest import golden, load_npz
from oracle import normwise_rel

pytestmark = pytest.mark.gpu
TOL = 1e-4
PRIMS = golden("prim_*.npz")


def _torch():
    import torch
    return torch


def dev(a):
    return _torch().from_numpy(np.ascontiguousarray(a)).cuda()


def stream():
    return _torch().cuda.current_stream().cuda_stream


def run_mm(lib, X, W, garbage=np.nan):
    M, K = X.shape
    N = W.shape[1]
    t = _torch()
    Y = t.full((M, N), float(garbage), dtype=t.float32, device="cuda")
    x, w = dev(X), dev(W)            # keep the inputs alive until the result is read
    lib.mm(Y.data_ptr(), x.data_ptr(), w.data_ptr(), M, K, N, stream())
    return Y.cpu().numpy()


def run_mm_bt(lib, dX0, dY, W):
    M, N = dY.shape
    K = W.shape[0]
    o, g, w = dev(dX0), dev(dY), dev(W)
    lib.mm_bt(o.data_ptr(), g.data_ptr(), w.data_ptr(), M, K, N, stream())
    return o.cpu().numpy()


def run_mm_atb(lib, dW0, X, dY):
    M, K = X.shape
    N = dY.shape[1]
    o, x, g = dev(dW0), dev(X), dev(dY)
    lib.mm_atb(o.data_ptr(), x.data_ptr(), g.data_ptr(), M, K, N, stream())
    return o.cpu().numpy()


@pytest.mark.parametrize("path", PRIMS, ids=[os.path.basename(p)[5:-4] for p in PRIMS])
def test_golden_device_entries(lib, orc, path):
    d = load_npz(path)
    print("case", os.path.basename(path), flush=True)
    Y = run_mm(lib, d["X"], d["W"])
    assert normwise_rel(Y, d["Y"]) <= TOL
    assert normwise_rel(Y, orc.mm_f64(d["X"], d["W"])) <= TOL
    dX = run_mm_bt(lib, d["dX0"], d["dY"], d["W"])
    assert normwise_rel(dX, d["dX"]) <= TOL
    assert normwise_rel(dX, orc.mm_bt_f64(d["dX0"].copy(), d["dY"], d["W"])) <= TOL
    dW = run_mm_atb(lib, d["dW0"], d["X"], d["dY"])
    assert normwise_rel(dW, d["dW"]) <= TOL
    assert normwise_rel(dW, orc.mm_atb_f64(d["dW0"].copy(), d["X"], d["dY"])) <= TOL


@pytest.mark.parametrize("path", PRIMS[:6], ids=[os.path.basename(p)[5:-4] for p in PRIMS[:6]])
def test_golden_host_entries(lib, path):
    """The drop-ins with the reference's signatures, on host pointers."""
    d = load_npz(path)
    M, K, N = int(d["M"]), int(d["K"]), int(d["N"])
    Y = np.full((M, N), np.nan, np.float32)
    lib.tlg_sgemm_nn(Y.ctypes.data, d["X"].ctypes.data, d["W"].ctypes.data, M, K, N)
    assert normwise_rel(Y, d["Y"]) <= TOL
    dX = d["dX0"].copy()
    lib.tlg_sgemm_nt_acc(dX.ctypes.data, d["dY"].ctypes.data, d["W"].ctypes.data, M, K, N)
    assert normwise_rel(dX, d["dX"]) <= TOL
    dW = d["dW0"].copy()
    lib.tlg_sgemm_tn_acc(dW.ctypes.data, d["X"].ctypes.data, d["dY"].ctypes.data, M, K, N)
    assert normwise_rel(dW, d["dW"]) <= TOL


# Every distinct (M, K, N) of BASELINE configs 0-2 per primitive (reference
# labels; tinylm.c:981-1141, :1015-1016, :1044-1067, :1085-1086), plus the
# cfg4 router/expert shapes at a reduced expert row count.
CFG_SHAPES = sorted({
    # cfg0: R=2048 D=128 KD=32 F=384 V=2048
    (2048, 128, 128), (2048, 128, 32), (2048, 128, 384), (2048, 384, 128), (2048, 2048, 128),
    # cfg1: R=4096 D=256 KD=64 F=768
    (4096, 256, 256), (4096, 256, 64), (4096, 256, 768), (4096, 768, 256), (4096, 2048, 256),
    # cfg2: R=8192 D=384 KD=96 F=1024 (MTP heads reuse (R,D,D) and (R,V,D))
    (8192, 384, 384), (8192, 384, 96), (8192, 384, 1024), (8192, 1024, 384), (8192, 2048, 384),
    # cfg4 router and a skewed expert's rows
    (4096, 256, 4), (614, 256, 768), (410, 768, 256),
})


def seeded(shape, scale, key):
    """Independent N(0, scale^2) draws; `key` names the operand, so no two
    operands of a case share a stream (a shared stream would make dY a
    multiple of X and X^T dY ill-conditioned)."""
    import zlib
    r = np.random.default_rng(zlib.crc32(repr((key, shape)).encode()))
    return (r.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float32)


@pytest.mark.parametrize("M,K,N", CFG_SHAPES)
def test_config_shapes_against_oracle(lib, orc, M, K, N):
    print("shape", M, K, N, flush=True)
    X = seeded((M, K), 1.0, "X")
    W = seeded((K, N), 0.02, "W")
    dY = seeded((M, N), 0.01, "dY")
    P1 = seeded((M, K), 1.0, "P1")
    P2 = seeded((K, N), 0.02, "P2")
    Y = run_mm(lib, X, W)
    assert normwise_rel(Y, orc.mm(X, W)) <= TOL
    dX = run_mm_bt(lib, P1, dY, W)
    assert normwise_rel(dX, orc.mm_bt(P1.copy(), dY, W)) <= TOL
    dW = run_mm_atb(lib, P2, X, dY)
    ref = orc.mm_atb(P2.copy(), X, dY)
    assert normwise_rel(dW, ref) <= TOL
    # the update itself (dW - prefill) must also meet the bar: the prefill
    # alone could hide a wrong product
    assert normwise_rel(dW - P2, ref - P2) <= TOL * 10
    assert normwise_rel(dW - P2, orc.mm_atb_f64(np.zeros_like(P2), X, dY)) <= TOL


@pytest.mark.parametrize("M,K,N", [(1, 384, 384), (2, 384, 96), (4, 384, 1024), (8, 1024, 384),
                                   (1, 2048, 384), (8, 2048, 384), (5, 7, 3), (3, 130, 66)])
def test_decode_rows(lib, orc, M, K, N):
    """cfg3 decode shapes, M = 1..8 rows (tinylm.c:3748-3829)."""
    X = seeded((M, K), 1.0, "X")
    W = seeded((K, N), 0.02, "W")
    dY = seeded((M, N), 1.0, "dY")
    assert normwise_rel(run_mm(lib, X, W), orc.mm_f64(X, W)) <= TOL
    P = seeded((M, K), 1.0, "P")
    assert normwise_rel(run_mm_bt(lib, P, dY, W), orc.mm_bt_f64(P.copy(), dY, W)) <= TOL
    Q = seeded((K, N), 1.0, "Q")
    assert normwise_rel(run_mm_atb(lib, Q, X, dY), orc.mm_atb_f64(Q.copy(), X, dY)) <= TOL


GEMV_SHAPES = [(1, 1, 1), (1, 5003, 65), (2, 384, 96), (3, 131, 259), (5, 64, 1), (6, 1024, 384),
               (7, 9, 700), (8, 2048, 384), (8, 384, 1024)]


@pytest.mark.parametrize("M,K,N", GEMV_SHAPES, ids=[f"{m}x{k}x{n}" for m, k, n in GEMV_SHAPES])
def test_gemv_kernels(lib, M, K, N):
    """M <= 8 mm / mm_bt take the weight-streaming GEMV kernels; ragged K/N,
    every row bucket, set semantics on a NaN-filled Y, accumulate onto a
    prefill, against the fp64 oracle."""
    from oracle import Oracle
    orc = Oracle()
    print("gemv", M, K, N, flush=True)
    assert lib.kernel_name("mm", M, K, N)[0].startswith("k_gemv")
    assert lib.kernel_name("mm_bt", M, K, N)[0].startswith("k_gemv")
    X = seeded((M, K), 1.0, "X")
    W = seeded((K, N), 0.02, "W")
    dY = seeded((M, N), 1.0, "dY")
    P = seeded((M, K), 1.0, "P")
    assert normwise_rel(run_mm(lib, X, W), orc.mm_f64(X, W)) <= TOL
    got = run_mm_bt(lib, P, dY, W)
    ref = orc.mm_bt_f64(P.copy(), dY, W)
    assert normwise_rel(got, ref) <= TOL
    assert normwise_rel(got - P, ref - P) <= TOL * 10


def test_gemv_group(lib):
    """A grouped launch of M <= 8 calls (the decode runs: several mm on one
    input, an mm_bt chain into one output) against fp64; then the same with
    one call at M > 8, which sends the whole group to the MFMA tiles."""
    from oracle import Oracle
    orc = Oracle()
    t = _torch()
    for M in (3, 8, 9):
        X = seeded((M, 384), 1.0, "gX")
        Ws = [seeded((384, n), 0.02, f"gW{n}") for n in (96, 1024)]
        dYs = [seeded((M, n), 1.0, f"gdY{n}") for n in (384, 96, 1024)]
        Wb = [seeded((384, n), 0.02, f"gWb{n}") for n in (384, 96, 1024)]
        P = seeded((M, 384), 1.0, "gP")
        keep = [dev(a) for a in [X] + Ws + dYs + Wb]
        x, w96, w1024, d384, d96, d1024, b384, b96, b1024 = keep
        y96 = t.full((M, 96), float("nan"), device="cuda")
        y1024 = t.full((M, 1024), float("nan"), device="cuda")
        dx = dev(P)
        lib.group([
            dict(op="mm", C=y96.data_ptr(), M=M, K=384, N=96, A=[x.data_ptr()], B=[w96.data_ptr()]),
            dict(op="mm", C=y1024.data_ptr(), M=M, K=384, N=1024, A=[x.data_ptr()], B=[w1024.data_ptr()]),
            dict(op="mm_bt", beta=1, C=dx.data_ptr(), M=M, K=384, N=384, Nseg=[384, 96, 1024],
                 A=[d384.data_ptr(), d96.data_ptr(), d1024.data_ptr()],
                 B=[b384.data_ptr(), b96.data_ptr(), b1024.data_ptr()]),
        ], stream())
        assert normwise_rel(y96.cpu().numpy(), orc.mm_f64(X, Ws[0])) <= TOL
        assert normwise_rel(y1024.cpu().numpy(), orc.mm_f64(X, Ws[1])) <= TOL
        ref = P.astype(np.float64)
        for a, b in zip(dYs, Wb):
            ref = ref + a.astype(np.float64) @ b.astype(np.float64).T
        assert normwise_rel(dx.cpu().numpy(), ref) <= TOL
        if M <= 8:
            assert lib.tlg_group_kernel().decode().startswith("k_gemv")


# Sched<> tile variants (configurations 24-50: a stage's fragment reads issued
# before its MFMAs, out-of-range chunks loaded from a zero buffer) beside the
# shapes they reorder
SCHED_CFGS = [3, 24, 25, 14, 26, 20, 27, 22, 28, 13, 29, 15, 30, 0, 31, 1, 32, 8, 33, 11, 34, 21, 35, 23, 36, 18, 37,
              38, 39, 40, 41, 42, 43, 44, 45, 46, 47, 48, 49, 50]


@pytest.mark.parametrize("gcfg", SCHED_CFGS)
def test_group_ragged_tiles(lib, gcfg):
    """One grouped launch of the three primitives on ragged shapes (777 rows,
    a 260-step reduction, 132 columns: partial row tiles, column tiles and
    stages) on each tile configuration, against fp64 -- set and accumulate,
    a split mm_atb reduction included (its partials summed by the flush)."""
    t = _torch()
    M, K, N = 777, 260, 132
    X = seeded((M, K), 1.0, "rgX")
    W = seeded((K, N), 0.02, "rgW")
    dY = seeded((M, N), 0.01, "rgdY")
    P = seeded((M, K), 1.0, "rgP")
    G = seeded((K, N), 1.0, "rgG")
    x, w, dy = dev(X), dev(W), dev(dY)
    y = t.full((M, N), float("nan"), device="cuda")
    dx, dw = dev(P), dev(G)
    lib.check(lib.tlg_tune_group(gcfg), "tune")
    try:
        lib.group([
            dict(op="mm", C=y.data_ptr(), M=M, K=K, N=N, A=[x.data_ptr()], B=[w.data_ptr()]),
            dict(op="mm_bt", beta=1, C=dx.data_ptr(), M=M, K=K, N=N, A=[dy.data_ptr()], B=[w.data_ptr()]),
            dict(op="mm_atb", beta=1, C=dw.data_ptr(), M=M, K=K, N=N, A=[x.data_ptr()], B=[dy.data_ptr()]),
        ], stream())
        name = lib.tlg_group_kernel().decode()
    finally:
        lib.check(lib.tlg_tune_group(-1), "tune")
    X64, W64, dY64 = (a.astype(np.float64) for a in (X, W, dY))
    assert normwise_rel(y.cpu().numpy(), X64 @ W64) <= TOL, (gcfg, name, "mm")
    assert normwise_rel(dx.cpu().numpy() - P, dY64 @ W64.T) <= TOL, (gcfg, name, "mm_bt")
    assert normwise_rel(dw.cpu().numpy() - G, X64.T @ dY64) <= TOL, (gcfg, name, "mm_atb")


@pytest.mark.parametrize("gcfg", [-1, 3, 24, 38, 39, 14, 40, 20, 22, 41, 15, 44, 13, 0, 45, 1])
def test_group_block_dot(lib, gcfg):
    """An mm_bt with the block-dot epilogue (TlgGemmCall.dotB / dotOut): dX as
    without it, and dotOut[i][b] = the dot of dX's and dotB's 32-column block b
    of row i, against fp64; on every kind of tile (one and several wave groups
    per stage, the 128 x 128 shapes falling back to 64 x 64), a ragged row count,
    beside an mm_atb of the same launch.  The attention backward's D =
    dO . O per row and head (tinylm.c:750-768)."""
    t = _torch()
    for M, K, N in ((4096, 256, 256), (777, 96, 132)):
        dY = seeded((M, N), 0.1, f"bdY{M}")
        W = seeded((K, N), 0.02, f"bdW{M}")
        O = seeded((M, K), 1.0, f"bdO{M}")
        X = seeded((M, K), 1.0, f"bdX{M}")
        G = seeded((K, N), 1.0, f"bdG{M}")
        dy, w, o, x = dev(dY), dev(W), dev(O), dev(X)
        dx = t.full((M, K), float("nan"), device="cuda")
        d = t.full((M, K // 32), float("nan"), device="cuda")
        dw = dev(G)
        if gcfg >= 0:
            lib.check(lib.tlg_tune_group(gcfg), "tune")
        try:
            lib.group([dict(op="mm_bt", beta=0, C=dx.data_ptr(), M=M, K=K, N=N, A=[dy.data_ptr()], B=[w.data_ptr()],
                            dotB=o.data_ptr(), dotOut=d.data_ptr()),
                       dict(op="mm_atb", beta=1, C=dw.data_ptr(), M=M, K=K, N=N, A=[x.data_ptr()],
                            B=[dy.data_ptr()])], stream())
        finally:
            lib.check(lib.tlg_tune_group(-1), "tune")
        want = dY.astype(np.float64) @ W.astype(np.float64).T
        got = dx.cpu().numpy()
        assert normwise_rel(got, want) <= TOL, (gcfg, M)
        # D from the stored dX (the chains the epilogue runs, in its order)
        ref = np.empty((M, K // 32), np.float32)
        g32, o32 = got.reshape(M, K // 32, 32), O.reshape(M, K // 32, 32)
        h0 = np.zeros((M, K // 32), np.float32)
        h1 = np.zeros((M, K // 32), np.float32)
        for c in range(16):
            h0 = (h0.astype(np.float64) + g32[:, :, c].astype(np.float64) * o32[:, :, c]).astype(np.float32)
            h1 = (h1.astype(np.float64) + g32[:, :, 16 + c].astype(np.float64) * o32[:, :, 16 + c]).astype(np.float32)
        ref = h0 + h1
        dd = d.cpu().numpy()
        assert normwise_rel(dd, ref) <= 1e-6, (gcfg, M)
        d64 = (want.reshape(M, K // 32, 32) * O.reshape(M, K // 32, 32)).sum(-1)
        assert normwise_rel(dd, d64) <= TOL, (gcfg, M)
        assert normwise_rel(dw.cpu().numpy() - G, X.astype(np.float64).T @ dY.astype(np.float64)) <= TOL
    bad = [dict(op="mm_bt", beta=1, C=dx.data_ptr(), M=M, K=K, N=N, A=[dy.data_ptr()], B=[w.data_ptr()],
                dotB=o.data_ptr(), dotOut=d.data_ptr())]
    with pytest.raises(Exception):
        lib.group(bad, stream())


def _one_alloc(parts):
    """Matrices laid out back to back in one device allocation, as
    map_weights lays out wq | wk | wv and w1 | w3 (tinylm.c:361-393)."""
    flat = np.concatenate([p.ravel() for p in parts]).astype(np.float32)
    d = dev(flat)
    ptrs, off = [], 0
    for p in parts:
        ptrs.append(d.data_ptr() + 4 * off)
        off += p.size
    return d, ptrs


ONE_MM = [(1, 384, (384, 96, 96)), (2, 96, (36, 100)), (3, 132, (1024, 1024)), (5, 1024, (384,)),
          (8, 384, (384, 96, 96)), (8, 1024, (44,))]


@pytest.mark.parametrize("tpb", ["128", "256"])
@pytest.mark.parametrize("cl", ["8", "4", "2"])
@pytest.mark.parametrize("M,K,segs", ONE_MM, ids=[f"{m}x{k}x{'-'.join(map(str, s))}" for m, k, s in ONE_MM])
def test_gemv_one_matrix_mm(lib, M, K, segs, cl, tpb):
    """Grouped M <= 8 mm calls over one input whose weight matrices follow
    each other in memory run as one matrix (k_gemv_cols): 32-, 16- and 8-column
    blocks, workgroups of 128 and 256 threads, ragged K and N, 1-3 segments,
    every row bucket, against fp64 (shapes no instance covers take the
    general kernel)."""
    from oracle import Oracle
    orc = Oracle()
    t = _torch()
    os.environ["TLG_GEMV_CL"] = cl
    os.environ["TLG_GEMV_TPB"] = tpb
    try:
        X = seeded((M, K), 1.0, "omX")
        Ws = [seeded((K, n), 0.02, f"omW{i}") for i, n in enumerate(segs)]
        x = dev(X)
        keep, ptrs = _one_alloc(Ws)
        Ys = [t.full((M, n), float("nan"), device="cuda") for n in segs]
        lib.group([dict(op="mm", C=y.data_ptr(), M=M, K=K, N=n, A=[x.data_ptr()], B=[b])
                   for y, n, b in zip(Ys, segs, ptrs)], stream())
        name = lib.tlg_group_kernel().decode()
        rg = int(tpb) // int(cl)
        need = -(-K // (4 * rg))
        if need <= 4 or (need <= 8 and rg == 32):
            assert name.startswith("k_gemv_cols") and f", {cl}, " in name and name.endswith(f", {tpb}>"), name
        else:
            assert name.startswith("k_gemv<"), name
        for y, w in zip(Ys, Ws):
            assert normwise_rel(y.cpu().numpy(), orc.mm_f64(X, w)) <= TOL, (M, K, segs)
    finally:
        del os.environ["TLG_GEMV_CL"]
        del os.environ["TLG_GEMV_TPB"]


ONE_BT = [(1, 384, (384, 96, 96)), (1, 1028, (13, 20, 7)), (2, 96, (2048,)), (3, 132, (1024, 1024)),
          (4, 1024, (384,)), (7, 384, (100, 12)), (8, 1024, (384,)), (8, 260, (16, 8, 40))]


@pytest.mark.parametrize("M,R,segs", ONE_BT, ids=[f"{m}x{r}x{'-'.join(map(str, s))}" for m, r, s in ONE_BT])
def test_gemv_one_matrix_mm_bt(lib, M, R, segs):
    """Grouped M <= 8 mm_bt calls over one input whose weights (decode
    layout W^T [out][in]) follow each other in memory run as one matrix
    (k_gemv_rows): 1-3 output segments of any row count, reductions shorter
    and longer than one batch of loads, set and accumulate, against fp64."""
    from oracle import Oracle
    orc = Oracle()
    t = _torch()
    A = seeded((M, R), 1.0, "obA")
    Wt = [seeded((n, R), 0.02, f"obW{i}") for i, n in enumerate(segs)]
    a = dev(A)
    keep, ptrs = _one_alloc(Wt)
    for beta in (0, 1):
        P = [seeded((M, n), 1.0, f"obP{i}") for i, n in enumerate(segs)]
        Cs = [dev(p) if beta else t.full((M, n), float("nan"), device="cuda") for p, n in zip(P, segs)]
        lib.group([dict(op="mm_bt", beta=beta, C=c.data_ptr(), M=M, K=n, N=R, A=[a.data_ptr()], B=[b])
                   for c, n, b in zip(Cs, segs, ptrs)], stream())
        assert lib.tlg_group_kernel().decode().startswith("k_gemv_rows")
        for c, w, p in zip(Cs, Wt, P):
            want = A.astype(np.float64) @ w.astype(np.float64).T
            got = c.cpu().numpy()
            if beta:
                got = got - p
            assert normwise_rel(got, want) <= TOL, (M, R, segs, beta)


def test_gemv_one_matrix_decode_forms(lib):
    """tlg_dev_dec_gemv on one matrix: q | k | v with the RMSNorm prologue at
    M = 1, 3, 8, and a MoE expert row (weight slice chosen on the device,
    gate-scaled, added into C) with the SwiGLU prologue, against fp64."""
    import tlgemm
    from oracle import StepFns
    t = _torch()
    st = StepFns("oracle")
    r = np.random.default_rng(23)
    D, KD, F, E = 384, 96, 1024, 4
    C = tlgemm.TlgDecGemv
    for M in (1, 3, 8):
        x = r.standard_normal((M, D)).astype(np.float32)
        gain = (1.0 + 0.1 * r.standard_normal(D)).astype(np.float32)
        Wt = [(0.02 * r.standard_normal((n, D))).astype(np.float32) for n in (D, KD, KD)]
        keep, ptrs = _one_alloc(Wt)
        dx, dg = dev(x), dev(gain)
        outs = [t.full((M, n), float("nan"), device="cuda") for n in (D, KD, KD)]
        calls = (C * 3)(*[C(1, 0, o.data_ptr(), M, n, D, dx.data_ptr(), b, 1, dg.data_ptr(), None)
                          for o, n, b in zip(outs, (D, KD, KD), ptrs)])
        lib.check(lib.tlg_dev_dec_gemv(calls, 3, stream()), "dec_gemv qkv")
        xn, _ = st.rmsnorm_fwd(x, gain)
        for o, w in zip(outs, Wt):
            assert normwise_rel(o.cpu().numpy(), xn.astype(np.float64) @ w.astype(np.float64).T) <= TOL, M
    # MoE row: res += gate * (silu(g) * u) @ W2_e^T, expert e picked on the device
    g = r.standard_normal((1, F)).astype(np.float32)
    u = r.standard_normal((1, F)).astype(np.float32)
    W2t = (0.02 * r.standard_normal((E, D, F))).astype(np.float32)
    res = r.standard_normal((1, D)).astype(np.float32)
    for e, gate in ((2, 0.625), (0, 1.5)):
        dgg, du, dw, dres = dev(g), dev(u), dev(W2t), dev(res)
        sel = t.tensor([e], dtype=t.int32, device="cuda")
        gt = t.tensor([gate], dtype=t.float32, device="cuda")
        one = (C * 1)(C(1, 1, dres.data_ptr(), 1, D, F, dgg.data_ptr(), dw.data_ptr(), 2, None, du.data_ptr(),
                        sel.data_ptr(), D * F, gt.data_ptr()))
        lib.check(lib.tlg_dev_dec_gemv(one, 1, stream()), "dec_gemv moe row")
        act = g.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64))) * u.astype(np.float64)
        want = gate * (act @ W2t[e].astype(np.float64).T)
        assert normwise_rel(dres.cpu().numpy() - res, want) <= TOL, e


def test_gemv_split_repeats(lib):
    """The M <= 8 mm splits W's rows over several workgroups whose partial
    sums meet in a tagged workspace that is reused launch after launch: 120
    back-to-back launches of interleaved shapes (different splits and
    column blocks land on the same words), every result against fp64, the
    same inputs bit-identical every time, and no wait ever timed out."""
    from oracle import Oracle
    orc = Oracle()
    t = _torch()
    shapes = [(1, 384, 1024), (8, 1024, 384), (2, 384, 96), (4, 5003, 64), (1, 1024, 384), (3, 384, 384)]
    cases = []
    for i, (M, K, N) in enumerate(shapes):
        X = seeded((M, K), 1.0, f"rX{i}")
        W = seeded((K, N), 0.02, f"rW{i}")
        cases.append((M, K, N, dev(X), dev(W), orc.mm_f64(X, W)))
    first = {}
    for rep in range(20):
        outs = []
        for i, (M, K, N, x, w, _) in enumerate(cases):
            Y = t.full((M, N), float("nan"), device="cuda")
            lib.mm(Y.data_ptr(), x.data_ptr(), w.data_ptr(), M, K, N, stream())
            outs.append(Y)
        for i, Y in enumerate(outs):
            got = Y.cpu().numpy()
            assert normwise_rel(got, cases[i][5]) <= TOL, (rep, cases[i][:3])
            if rep == 0:
                first[i] = got
            else:
                assert np.array_equal(got, first[i]), (rep, cases[i][:3])
    assert lib.tlg_gemv_status() == 0


@pytest.mark.parametrize("M,K,N", [(4096, 256, 256), (67, 36, 44), (5, 8, 12)])
def test_residual_mm(lib, M, K, N):
    """TlgGemmCall.R: C = R + X W in the store, bit for bit the mm result plus
    R (the reference adds after mm, tinylm.c:994-995); M <= 8 leaves the
    GEMV kernels for the MFMA tiles."""
    t = _torch()
    X = seeded((M, K), 1.0, "rX")
    W = seeded((K, N), 0.05, "rW")
    Rr = seeded((M, N), 1.0, "rR")
    x, w, r = dev(X), dev(W), dev(Rr)
    y = t.full((M, N), float("nan"), device="cuda")
    fused = t.full((M, N), float("nan"), device="cuda")
    lib.group([dict(op="mm", C=y.data_ptr(), M=M, K=K, N=N, A=[x.data_ptr()], B=[w.data_ptr()])], stream())
    lib.group([dict(op="mm", C=fused.data_ptr(), M=M, K=K, N=N, A=[x.data_ptr()], B=[w.data_ptr()],
                    R=r.data_ptr())], stream())
    if M > 8:
        assert np.array_equal(fused.cpu().numpy(), y.cpu().numpy() + Rr)
    ref = Rr.astype(np.float64) + X.astype(np.float64) @ W.astype(np.float64)
    assert normwise_rel(fused.cpu().numpy(), ref) <= TOL


def test_residual_reads_pending_reduction(lib, orc):
    """A residual operand that a deferred split reduction still has to write
    is flushed first: mm_atb (split at this shape) into dW, then mm with
    R = dW."""
    t = _torch()
    X = seeded((4096, 256), 1.0, "pX")
    dY = seeded((4096, 64), 0.01, "pdY")
    A2 = seeded((32, 64), 1.0, "pA")
    W2 = seeded((64, 64), 0.1, "pW")
    dw = t.zeros((256, 64), device="cuda")
    x, dy, a2, w2 = dev(X), dev(dY), dev(A2), dev(W2)
    y = t.full((32, 64), float("nan"), device="cuda")
    lib.group([dict(op="mm_atb", beta=1, C=dw.data_ptr(), M=4096, K=256, N=64, A=[x.data_ptr()],
                    B=[dy.data_ptr()])], stream(), flush=False)
    lib.group([dict(op="mm", C=y.data_ptr(), M=32, K=64, N=64, A=[a2.data_ptr()], B=[w2.data_ptr()],
                    R=dw.data_ptr())], stream())
    dW = orc.mm_atb_f64(np.zeros((256, 64), np.float32), X, dY)
    assert normwise_rel(dw.cpu().numpy(), dW) <= TOL
    ref = dW[:32] + A2.astype(np.float64) @ W2.astype(np.float64)
    assert normwise_rel(y.cpu().numpy(), ref) <= TOL


def _silu64(z):
    return z / (1.0 + np.exp(-z))


FFN = [(4096, 256, 768), (4096, 768, 256), (67, 32, 48), (1, 16, 8), (300, 64, 96)]


@pytest.mark.parametrize("M,K,N", FFN)
def test_swiglu_mm(lib, M, K, N):
    """tlg_dev_swiglu_mm: g = X W1, u = X W3, act = silu(g) u (tinylm.c:1002-1006)
    from one launch, against float64; without g / u it still writes act."""
    t = _torch()
    X = seeded((M, K), 1.0, "sX")
    W1 = seeded((K, N), 0.1, "sW1")
    W3 = seeded((K, N), 0.1, "sW3")
    x, w1, w3 = dev(X), dev(W1), dev(W3)
    act, g, u = (t.full((M, N), float("nan"), device="cuda") for _ in range(3))
    lib.check(lib.tlg_dev_swiglu_mm(x.data_ptr(), w1.data_ptr(), w3.data_ptr(), act.data_ptr(), g.data_ptr(),
                                    u.data_ptr(), M, K, N, stream()), "swiglu_mm")
    g64 = X.astype(np.float64) @ W1.astype(np.float64)
    u64 = X.astype(np.float64) @ W3.astype(np.float64)
    assert normwise_rel(g.cpu().numpy(), g64) <= TOL
    assert normwise_rel(u.cpu().numpy(), u64) <= TOL
    assert normwise_rel(act.cpu().numpy(), _silu64(g64) * u64) <= TOL
    act2 = t.full((M, N), float("nan"), device="cuda")
    lib.check(lib.tlg_dev_swiglu_mm(x.data_ptr(), w1.data_ptr(), w3.data_ptr(), act2.data_ptr(), None, None, M, K,
                                    N, stream()), "swiglu_mm")
    assert np.array_equal(act2.cpu().numpy(), act.cpu().numpy())


@pytest.mark.parametrize("M,K,N", FFN)
def test_mm_bt_swiglu_bwd(lib, M, K, N):
    """tlg_dev_mm_bt_swiglu_bwd: dact = dY W2^T, then dg = dact u silu'(g) and
    du = dact silu(g) in place of g, u (tinylm.c:1102-1109), against float64."""
    t = _torch()
    dY = seeded((M, N), 1.0, "bdY")
    W2 = seeded((K, N), 0.1, "bW2")
    G0 = seeded((M, K), 1.0, "bG")
    U0 = seeded((M, K), 1.0, "bU")
    dy, w2, g, u = dev(dY), dev(W2), dev(G0), dev(U0)
    lib.check(lib.tlg_dev_mm_bt_swiglu_bwd(dy.data_ptr(), w2.data_ptr(), g.data_ptr(), u.data_ptr(), M, K, N,
                                           stream()), "mm_bt_swiglu_bwd")
    dact = dY.astype(np.float64) @ W2.astype(np.float64).T
    z = G0.astype(np.float64)
    sg = 1.0 / (1.0 + np.exp(-z))
    assert normwise_rel(g.cpu().numpy(), dact * U0 * (sg + z * sg * (1 - sg))) <= TOL
    assert normwise_rel(u.cpu().numpy(), dact * z * sg) <= TOL


def test_fused_ffn_carries_pending_reduction(lib, orc):
    """A dense fused launch after a grouped launch with a split mm_atb: the
    deferred reduction rides along (or is flushed) and both results hold."""
    t = _torch()
    X = seeded((4096, 256), 1.0, "cX")
    dYa = seeded((4096, 64), 0.01, "cdY")
    dw = t.zeros((256, 64), device="cuda")
    x, dya = dev(X), dev(dYa)
    lib.group([dict(op="mm_atb", beta=1, C=dw.data_ptr(), M=4096, K=256, N=64, A=[x.data_ptr()],
                    B=[dya.data_ptr()])], stream(), flush=False)
    assert lib.tlg_dev_gemm_pending() > 0
    dY = seeded((512, 64), 1.0, "cdY2")
    W2 = seeded((96, 64), 0.1, "cW2")
    G0 = seeded((512, 96), 1.0, "cG")
    U0 = seeded((512, 96), 1.0, "cU")
    dy, w2, g, u = dev(dY), dev(W2), dev(G0), dev(U0)
    lib.check(lib.tlg_dev_mm_bt_swiglu_bwd(dy.data_ptr(), w2.data_ptr(), g.data_ptr(), u.data_ptr(), 512, 96, 64,
                                           stream()), "mm_bt_swiglu_bwd")
    assert lib.tlg_dev_gemm_pending() == 0
    assert normwise_rel(dw.cpu().numpy(), orc.mm_atb_f64(np.zeros((256, 64), np.float32), X, dYa)) <= TOL
    dact = dY.astype(np.float64) @ W2.astype(np.float64).T
    z = G0.astype(np.float64)
    sg = 1.0 / (1.0 + np.exp(-z))
    assert normwise_rel(u.cpu().numpy(), dact * z * sg) <= TOL


def test_empty_dimensions(lib):
    t = _torch()
    # K = 0: mm clears Y (tinylm.c:461), the accumulating forms leave theirs
    Y = t.full((5, 7), 3.0, device="cuda")
    lib.mm(Y.data_ptr(), 0, 0, 5, 0, 7, stream())
    assert (Y.cpu() == 0).all()
    dW = t.full((4, 6), 2.0, device="cuda")
    lib.mm_atb(dW.data_ptr(), 0, 0, 0, 4, 6, stream())          # M = 0
    assert (dW.cpu() == 2.0).all()
    dX = t.full((3, 4), 1.5, device="cuda")
    lib.mm_bt(dX.data_ptr(), 0, 0, 3, 4, 0, stream())           # N = 0
    assert (dX.cpu() == 1.5).all()
    lib.mm(0, 0, 0, 0, 5, 5, stream())                           # M = 0: no-op


def test_negative_dimension_is_an_error(lib):
    rc = lib.tlg_dev_sgemm_nn(0, 0, 0, -1, 4, 4, None)
    assert rc != 0 and b"negative" in lib.tlg_last_error()


def test_chain_fixture(lib):
    d = load_npz(golden("chain_dnorm.npz")[0])
    t = _torch()
    R, D = d["out"].shape
    out = t.empty((R, D), device="cuda")
    lib.zero(out.data_ptr(), out.numel(), stream())
    for g, w in (("dq", "Wq"), ("dk", "Wk"), ("dv", "Wv")):
        gg, ww = dev(d[g]), dev(d[w])
        lib.mm_bt(out.data_ptr(), gg.data_ptr(), ww.data_ptr(), R, D, d[g].shape[1], stream())
        _torch().cuda.synchronize()
    assert normwise_rel(out.cpu().numpy(), d["out"]) <= TOL


def test_split_reduction_deterministic_and_reset(lib, orc):
    """mm_atb at cfg1's dWq shape takes the split-reduction path; two calls in
    a row must give bit-identical sums (fixed split order) and the second must
    still be right (tile counters reset)."""
    M, K, N = 4096, 256, 256
    X = seeded((M, K), 1.0, "X")
    dY = seeded((M, N), 0.01, "dY")
    P = np.zeros((K, N), np.float32)
    a = run_mm_atb(lib, P, X, dY)
    b = run_mm_atb(lib, P, X, dY)
    assert np.array_equal(a, b)
    assert normwise_rel(a, orc.mm_atb_f64(P.copy(), X, dY)) <= TOL


def test_host_registry_device_residency(lib, orc):
    """Operands inside a registered range are used in place on the device; the
    output stays there until tlg_pull (hipMemcpy only at step boundaries)."""
    M, K, N = 256, 128, 96
    buf = np.zeros(M * K + K * N + M * N, np.float32)
    X = buf[:M * K].reshape(M, K)
    W = buf[M * K:M * K + K * N].reshape(K, N)
    Y = buf[M * K + K * N:].reshape(M, N)
    X[:] = seeded((M, K), 1.0, "X")
    W[:] = seeded((K, N), 0.02, "W")
    lib.check(lib.tlg_register(buf.ctypes.data, buf.nbytes), "register")
    try:
        lib.tlg_sgemm_nn(Y.ctypes.data, X.ctypes.data, W.ctypes.data, M, K, N)
        assert (Y == 0).all()                    # result lives in the mirror
        lib.check(lib.tlg_pull(buf.ctypes.data), "pull")
        assert normwise_rel(Y, orc.mm_f64(X.copy(), W.copy())) <= TOL
        W *= 2                                   # host update, then push
        lib.check(lib.tlg_push(buf.ctypes.data), "push")
        lib.tlg_sgemm_nn(Y.ctypes.data, X.ctypes.data, W.ctypes.data, M, K, N)
        lib.check(lib.tlg_pull(buf.ctypes.data), "pull")
        assert normwise_rel(Y, orc.mm_f64(X.copy(), W.copy())) <= TOL
        assert lib.tlg_mirror(W.ctypes.data) is not None
    finally:
        lib.check(lib.tlg_unregister(buf.ctypes.data), "unregister")
    assert lib.tlg_mirror(buf.ctypes.data) is None


@pytest.mark.parametrize("cfg", [0, 1, 2, 3, 4, 5, 6, 7, 8, 13, 14, 15])
def test_every_tile_config(lib, orc, cfg):
    """Each instantiated tile shape, with and without a split reduction, on a
    ragged shape (scalar staging) and an aligned one (float4 staging)."""
    try:
        for splits in (1, 3):
            lib.check(lib.tlg_tune_force(cfg, splits), "force")
            for M, K, N in ((201, 131, 259), (256, 160, 192)):
                X = seeded((M, K), 1.0, "X")
                W = seeded((K, N), 0.02, "W")
                dY = seeded((M, N), 0.01, "dY")
                P1 = seeded((M, K), 1.0, "P1")
                P2 = seeded((K, N), 0.02, "P2")
                assert normwise_rel(run_mm(lib, X, W), orc.mm_f64(X, W)) <= TOL
                assert normwise_rel(run_mm_bt(lib, P1, dY, W), orc.mm_bt_f64(P1.copy(), dY, W)) <= TOL
                assert normwise_rel(run_mm_atb(lib, P2, X, dY), orc.mm_atb_f64(P2.copy(), X, dY)) <= TOL
    finally:
        lib.check(lib.tlg_tune_force(-1, 0), "auto")


@pytest.mark.parametrize("args", [[], ["1", "384", "384"], ["8", "2048", "384"], ["512", "256", "768", "7"]],
                         ids=["selftest", "decode", "unembed", "ffn"])
def test_c_selftest_through_seam(args):
    """host/tl_selftest.c: mm / mm_bt / mm_atb called with the reference's
    signatures (the -DUSE_HIP seam), checked against double precision loops
    like tinylm.c's own selftest (tinylm.c:4750-4788), at the 1e-4 bar."""
    import subprocess
    exe = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "tinylm-c_amd", "tl_selftest")
    r = subprocess.run([exe] + args, capture_output=True, text=True, timeout=100)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0 and "PASS" in r.stdout
