"""GPU parity of the device-resident training step (include/tltrain.h and
host/tl_train.h) through the C ABI.

Kernel by kernel, each HIP entry point is compared with the CPU oracle
(oracle/tl_oracle_step.c, pinned in tests/test_step_oracle.py) on the same
seeded inputs, and with the golden fixtures the reference's own code wrote.
Whole steps (forward + backward, then gradnorm + AdamW) are compared with the
fixtures and with the oracle's step at the nano and m3 model shapes.

Bars: embedding gather / scatter bit-exact; everything else within 1e-4
normwise (max|err| / mean|ref|, tinylm.c:4782-4784) per tensor, and the loss
within 1e-5 relative.  Graph replays equal eager steps bit for bit.
"""
import os

import numpy as np
import pytest

from conftest import golden, load_npz
from oracle import StepFns, model, normwise_rel, param_regions

pytestmark = pytest.mark.gpu
TOL = 1e-4


def _t():
    import torch
    return torch


def dev(a):
    return _t().from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.cpu().numpy()


def nan_like(shape):
    t = _t()
    return t.full(shape, float("nan"), dtype=t.float32, device="cuda")


def stream():
    return _t().cuda.current_stream().cuda_stream


@pytest.fixture(scope="module")
def st():
    s = StepFns("oracle")
    return s


# ------------------------------------------------------------------ rmsnorm --
@pytest.mark.parametrize("rows,D", [(9, 768), (3, 2052), (2, 4100)])
def test_rmsnorm_fwd_wide(lib, st, rows, D):
    """The forward's other row widths: 4 float4 columns per lane, and rows wider
    than 2048 (read twice instead of kept in registers)."""
    print("rmsnorm_fwd", rows, D, flush=True)
    r = np.random.default_rng(rows * D)
    x = r.standard_normal((rows, D)).astype(np.float32)
    g = (1 + 0.1 * r.standard_normal(D)).astype(np.float32)
    X, Gn = dev(x), dev(g)
    out, rinv = nan_like((rows, D)), nan_like((rows,))
    lib.check(lib.tlg_dev_rmsnorm_fwd(X.data_ptr(), Gn.data_ptr(), out.data_ptr(), rinv.data_ptr(), rows, D,
                                      stream()), "rmsnorm_fwd")
    ro, rr = st.rmsnorm_fwd(x, g)
    assert normwise_rel(host(out), ro) <= TOL and normwise_rel(host(rinv), rr) <= TOL


@pytest.mark.parametrize("rows,D", [(4096, 256), (1027, 384), (37, 48), (5, 2048)])
def test_rmsnorm(lib, st, rows, D):
    print("rmsnorm", rows, D, flush=True)
    r = np.random.default_rng(rows + D)
    x = r.standard_normal((rows, D)).astype(np.float32)
    g = (1 + 0.1 * r.standard_normal(D)).astype(np.float32)
    X, Gn = dev(x), dev(g)
    out, rinv = nan_like((rows, D)), nan_like((rows,))
    lib.check(lib.tlg_dev_rmsnorm_fwd(X.data_ptr(), Gn.data_ptr(), out.data_ptr(), rinv.data_ptr(), rows, D,
                                      stream()), "rmsnorm_fwd")
    ro, rr = st.rmsnorm_fwd(x, g)
    assert normwise_rel(host(out), ro) <= TOL and normwise_rel(host(rinv), rr) <= TOL
    dy = (0.01 * r.standard_normal((rows, D))).astype(np.float32)
    base = r.standard_normal((rows, D)).astype(np.float32)
    dg0 = (0.01 * r.standard_normal(D)).astype(np.float32)
    # dx = base + ..., dx += ... (in place), dx = 0 + ...
    for mode in ("sep", "inplace", "zero"):
        DX = dev(base) if mode == "inplace" else nan_like((rows, D))
        DXI = dev(base) if mode == "sep" else (DX if mode == "inplace" else None)
        DG, RI, DY = dev(dg0), dev(rr), dev(dy)
        lib.check(lib.tlg_dev_rmsnorm_bwd(X.data_ptr(), Gn.data_ptr(), RI.data_ptr(), DY.data_ptr(),
                                          None if DXI is None else DXI.data_ptr(), DX.data_ptr(), DG.data_ptr(),
                                          rows, D, stream()), "rmsnorm_bwd")
        want = (np.zeros_like(base) if mode == "zero" else base.copy())
        wdg = dg0.copy()
        st.rmsnorm_bwd(x, g, rr, dy, want, wdg)
        b0 = 0 if mode == "zero" else base
        assert normwise_rel(host(DX) - b0, want - b0) <= TOL, mode
        assert normwise_rel(host(DG) - dg0, wdg - dg0) <= TOL, mode


@pytest.mark.parametrize("rows,D", [(4096, 256), (1027, 384), (37, 48), (5, 2048)])
def test_rmsnorm_bwd_defer(lib, rows, D):
    """The deferred gain sum equals tlg_dev_rmsnorm_bwd's bit for bit, when it
    rides along in the next grouped GEMM launch, when a second call on the
    same partials flushes it first, and through tlg_dev_gemm_flush."""
    print("rmsnorm_bwd_defer", rows, D, flush=True)
    t = _t()
    r = np.random.default_rng(7 * rows + D)
    x = r.standard_normal((rows, D)).astype(np.float32)
    g = (1 + 0.1 * r.standard_normal(D)).astype(np.float32)
    rr = (1 + 0.1 * r.random(rows)).astype(np.float32)
    dys = [(0.01 * r.standard_normal((rows, D))).astype(np.float32) for _ in range(2)]
    base = r.standard_normal((rows, D)).astype(np.float32)
    dg0 = (0.01 * r.standard_normal(D)).astype(np.float32)
    X, Gn, RI, B = dev(x), dev(g), dev(rr), dev(base)
    want = []
    for dy in dys:
        DX, DG = nan_like((rows, D)), dev(dg0)
        lib.check(lib.tlg_dev_rmsnorm_bwd(X.data_ptr(), Gn.data_ptr(), RI.data_ptr(), dev(dy).data_ptr(),
                                          B.data_ptr(), DX.data_ptr(), DG.data_ptr(), rows, D, stream()), "bwd")
        want.append((host(DX), host(DG)))
    nblk = (rows + 15) // 16
    part = t.empty(nblk * D, dtype=t.float32, device="cuda")
    # a GEMM to ride on (its own buffers)
    M, K, N = 256, 64, 128
    Xg, Wg = dev(r.standard_normal((M, K)).astype(np.float32)), dev(r.standard_normal((K, N)).astype(np.float32))
    Yg = nan_like((M, N))
    gemm = dict(op="mm", C=Yg.data_ptr(), M=M, K=K, N=N, A=[Xg.data_ptr()], B=[Wg.data_ptr()])
    for how in ("ride", "twice", "flush"):
        DYs = [dev(dy) for dy in dys]
        DXs, DGs = [nan_like((rows, D)) for _ in dys], [dev(dg0) for _ in dys]
        n = 2 if how == "twice" else 1
        for i in range(n):
            lib.check(lib.tlg_dev_rmsnorm_bwd_defer(X.data_ptr(), Gn.data_ptr(), RI.data_ptr(), DYs[i].data_ptr(),
                                                    B.data_ptr(), DXs[i].data_ptr(), DGs[i].data_ptr(), rows, D,
                                                    part.data_ptr(), nblk * D, stream()), "defer")
        if how == "flush":
            lib.check(lib.tlg_dev_gemm_flush(stream()), "flush")
        else:
            lib.group([gemm], stream(), flush=False)
            lib.check(lib.tlg_dev_gemm_flush(stream()), "flush")
        for i in range(n):
            assert np.array_equal(host(DXs[i]), want[i][0]), (how, i)
            assert np.array_equal(host(DGs[i]), want[i][1]), (how, i)
        assert normwise_rel(host(Yg), host(Xg).astype(np.float64) @ host(Wg).astype(np.float64)) <= TOL
    import tlgemm
    with pytest.raises(tlgemm.TlgError):
        lib.check(lib.tlg_dev_rmsnorm_bwd_defer(X.data_ptr(), Gn.data_ptr(), RI.data_ptr(), DYs[0].data_ptr(),
                                                None, DXs[0].data_ptr(), DGs[0].data_ptr(), rows, D,
                                                part.data_ptr(), nblk * D - 1, stream()), "short partials")


def test_rmsnorm_fixture(lib):
    d = load_npz(golden("step_rmsnorm.npz")[0])
    rows, D = d["x"].shape
    out, rinv = nan_like((rows, D)), nan_like((rows,))
    X, Gn = dev(d["x"]), dev(d["g"])
    lib.check(lib.tlg_dev_rmsnorm_fwd(X.data_ptr(), Gn.data_ptr(), out.data_ptr(), rinv.data_ptr(), rows, D,
                                      stream()), "fwd")
    assert normwise_rel(host(out), d["out"]) <= TOL
    DX, DG, RI, DY = dev(d["dx0"]), dev(d["dg0"]), dev(d["rinv"]), dev(d["dy"])
    lib.check(lib.tlg_dev_rmsnorm_bwd(X.data_ptr(), Gn.data_ptr(), RI.data_ptr(), DY.data_ptr(),
                                      DX.data_ptr(), DX.data_ptr(), DG.data_ptr(), rows, D, stream()), "bwd")
    assert normwise_rel(host(DX) - d["dx0"], d["dx"] - d["dx0"]) <= TOL
    assert normwise_rel(host(DG) - d["dg0"], d["dg"] - d["dg0"]) <= TOL


# --------------------------------------------------------------------- rope --
@pytest.mark.parametrize("rows,T,nh,hd", [(4096, 256, 8, 32), (40, 16, 3, 32), (70, 70, 1, 32), (50, 10, 2, 6)])
def test_rope(lib, st, rows, T, nh, hd):
    """hd 32: the float4 kernel; hd 6: the scalar one."""
    r = np.random.default_rng(rows)
    buf = r.standard_normal((rows, nh * hd)).astype(np.float32)
    cs, sn = st.rope_table(T, hd)
    C, S = dev(cs), dev(sn)
    for back in (0, 1):
        B = dev(buf)
        lib.check(lib.tlg_dev_rope(B.data_ptr(), None, T, rows, nh, hd, C.data_ptr(), S.data_ptr(), T, back,
                                   stream()), "rope")
        want = buf.copy()
        st.rope(want, T, nh, hd, back)
        assert normwise_rel(host(B), want) <= TOL, back


# ---------------------------------------------------------------- attention --
ATTN = [  # B, T, H, KV, win
    (2, 256, 8, 2, 0),      # m3 heads
    (2, 256, 4, 1, 0),      # nano heads
    (2, 256, 12, 3, 0),     # m8 heads
    (3, 70, 2, 1, 0),       # ragged T
    (2, 100, 4, 2, 40),     # sliding window
    (2, 100, 8, 2, 40),     # sliding window, GQA groups of 4 (the group kernels)
    (1, 33, 2, 2, 0),       # MHA
    (4, 1, 4, 1, 0),        # one token
]


def gpu_attn(lib, q, k, v, datt, B, T, H, KV, win):
    t = _t()
    Q, K, Vv = dev(q), dev(k), dev(v)
    out, lse = nan_like(q.shape), nan_like((B * T, H))
    lib.check(lib.tlg_dev_attn_fwd(Q.data_ptr(), K.data_ptr(), Vv.data_ptr(), out.data_ptr(), lse.data_ptr(), B, T,
                                   H, KV, 32, win, stream()), "attn_fwd")
    dq, dk, dv, DA = nan_like(q.shape), nan_like(k.shape), nan_like(v.shape), dev(datt)
    lib.check(lib.tlg_dev_attn_bwd(Q.data_ptr(), K.data_ptr(), Vv.data_ptr(), out.data_ptr(), lse.data_ptr(),
                                   DA.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), B, T, H, KV,
                                   32, win, stream()), "attn_bwd")
    t.cuda.synchronize()
    return host(out), host(dq), host(dk), host(dv)


@pytest.mark.parametrize("B,T,H,KV,win", ATTN)
def test_attention(lib, st, B, T, H, KV, win):
    print("attention", B, T, H, KV, win, flush=True)
    r = np.random.default_rng(T * 7 + H)
    q = r.standard_normal((B * T, H * 32)).astype(np.float32)
    k = r.standard_normal((B * T, KV * 32)).astype(np.float32)
    v = r.standard_normal((B * T, KV * 32)).astype(np.float32)
    datt = (0.01 * r.standard_normal((B * T, H * 32))).astype(np.float32)
    out, dq, dk, dv = gpu_attn(lib, q, k, v, datt, B, T, H, KV, win)
    assert normwise_rel(out, st.attn_fwd(q, k, v, B, T, H, KV, 32, win)) <= TOL
    wq, wk, wv = st.attn_bwd(q, k, v, datt, B, T, H, KV, 32, win)
    for got, want, name in ((dq, wq, "dq"), (dk, wk, "dk"), (dv, wv, "dv")):
        assert normwise_rel(got, want) <= TOL, name


def test_attention_unaligned_lse(lib, st):
    """GQA groups of 4 with an lse array that is not 16-byte aligned: the
    backward takes the dQ group kernel and the per-head dK / dV kernel instead
    of the one-launch group path (which reads lse rows as float4)."""
    B, T, H, KV, win = 2, 100, 8, 2, 0
    t = _t()
    r = np.random.default_rng(5)
    q = r.standard_normal((B * T, H * 32)).astype(np.float32)
    k = r.standard_normal((B * T, KV * 32)).astype(np.float32)
    v = r.standard_normal((B * T, KV * 32)).astype(np.float32)
    datt = (0.01 * r.standard_normal((B * T, H * 32))).astype(np.float32)
    Q, K, Vv, DA = dev(q), dev(k), dev(v), dev(datt)
    out, lse1 = nan_like(q.shape), nan_like((B * T * H + 4,))
    lp = lse1.data_ptr() + 4                                   # one float in: 4-byte aligned only
    lib.check(lib.tlg_dev_attn_fwd(Q.data_ptr(), K.data_ptr(), Vv.data_ptr(), out.data_ptr(), lp, B, T, H, KV, 32,
                                   win, stream()), "attn_fwd")
    dq, dk, dv = nan_like(q.shape), nan_like(k.shape), nan_like(v.shape)
    lib.check(lib.tlg_dev_attn_bwd(Q.data_ptr(), K.data_ptr(), Vv.data_ptr(), out.data_ptr(), lp, DA.data_ptr(),
                                   dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), B, T, H, KV, 32, win, stream()),
              "attn_bwd")
    t.cuda.synchronize()
    wq, wk, wv = st.attn_bwd(q, k, v, datt, B, T, H, KV, 32, win)
    assert normwise_rel(host(out), st.attn_fwd(q, k, v, B, T, H, KV, 32, win)) <= TOL
    for got, want, name in ((host(dq), wq, "dq"), (host(dk), wk, "dk"), (host(dv), wv, "dv")):
        assert normwise_rel(got, want) <= TOL, name


@pytest.mark.parametrize("path", golden("step_attn_*.npz"), ids=os.path.basename)
def test_attention_fixture(lib, path):
    d = load_npz(path)
    B, T, H, KV, win = (int(d[k]) for k in ("B", "T", "H", "KV", "win"))
    out, dq, dk, dv = gpu_attn(lib, d["q"], d["k"], d["v"], d["datt"], B, T, H, KV, win)
    for got, key in ((out, "out"), (dq, "dq"), (dk, "dk"), (dv, "dv")):
        assert normwise_rel(got, d[key]) <= TOL, key


ATTN_ROPE = [  # B, T, H, KV, win: GQA groups of 4 or 8 heads
    (2, 256, 8, 2, 0),      # m3 heads
    (2, 256, 12, 3, 0),     # m8 heads
    (3, 70, 4, 1, 0),       # ragged T
    (2, 100, 8, 1, 40),     # sliding window, 8 heads per KV head
    (1, 256, 16, 2, 0),     # 8 heads per KV head, full causal (two dQ items per dK / dV item)
    (4, 1, 4, 1, 0),        # one token
]


@pytest.mark.parametrize("B,T,H,KV,win", ATTN_ROPE)
def test_attention_rope_fused(lib, st, B, T, H, KV, win):
    """tlg_dev_attn_{fwd,bwd}_rope on pre-rope q, k against the reference's
    sequence: rope_apply(q), rope_apply(k), attn_fwd; attn_bwd, then the
    transposed rope_apply on dq and dk (tinylm.c:988-990, :1130-1133)."""
    print("attention rope", B, T, H, KV, win, flush=True)
    t = _t()
    r = np.random.default_rng(T * 11 + H + win)
    q = r.standard_normal((B * T, H * 32)).astype(np.float32)
    k = r.standard_normal((B * T, KV * 32)).astype(np.float32)
    v = r.standard_normal((B * T, KV * 32)).astype(np.float32)
    datt = (0.01 * r.standard_normal((B * T, H * 32))).astype(np.float32)
    cs, sn = st.rope_table(T, 32)
    qr, kr = q.copy(), k.copy()
    st.rope(qr, T, H, 32, 0)
    st.rope(kr, T, KV, 32, 0)
    want_out = st.attn_fwd(qr, kr, v, B, T, H, KV, 32, win)
    wq, wk, wv = st.attn_bwd(qr, kr, v, datt, B, T, H, KV, 32, win)
    st.rope(wq, T, H, 32, 1)
    st.rope(wk, T, KV, 32, 1)
    Q, K, Vv, C, S = dev(q), dev(k), dev(v), dev(cs), dev(sn)
    out, lse = nan_like(q.shape), nan_like((B * T, H))
    lib.check(lib.tlg_dev_attn_fwd_rope(Q.data_ptr(), K.data_ptr(), Vv.data_ptr(), out.data_ptr(), lse.data_ptr(), B,
                                        T, H, KV, 32, win, C.data_ptr(), S.data_ptr(), stream()), "attn_fwd_rope")
    dq, dk, dv, DA = nan_like(q.shape), nan_like(k.shape), nan_like(v.shape), dev(datt)
    lib.check(lib.tlg_dev_attn_bwd_rope(Q.data_ptr(), K.data_ptr(), Vv.data_ptr(), out.data_ptr(), lse.data_ptr(),
                                        DA.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), B, T, H, KV, 32,
                                        win, C.data_ptr(), S.data_ptr(), stream()), "attn_bwd_rope")
    t.cuda.synchronize()
    # q and k are inputs: the fused kernels must leave them pre-rope
    assert np.array_equal(host(Q), q) and np.array_equal(host(K), k)
    assert normwise_rel(host(out), want_out) <= TOL
    for got, want, name in ((host(dq), wq, "dq"), (host(dk), wk, "dk"), (host(dv), wv, "dv")):
        assert normwise_rel(got, want) <= TOL, name


def test_attention_rope_needs_groups_of_4(lib):
    Z = dev(np.zeros(64 * 64, np.float32))
    p = Z.data_ptr()
    assert lib.tlg_dev_attn_fwd_rope(p, p, p, p, p, 1, 2, 2, 1, 32, 0, p, p, stream()) != 0
    assert lib.tlg_dev_attn_fwd_rope(p, p, p, p, p, 1, 2, 4, 1, 32, 0, None, None, stream()) != 0
    lib.tlg_last_error()


def test_attention_rejects_bad_shapes(lib):
    Z = dev(np.zeros(64 * 64, np.float32))
    p = Z.data_ptr()
    assert lib.tlg_dev_attn_fwd(p, p, p, p, p, 1, 2, 2, 1, 16, 0, stream()) != 0      # head_dim 16
    assert lib.tlg_dev_attn_fwd(p, p, p, p, p, 1, 2, 3, 2, 32, 0, stream()) != 0      # H % KV
    lib.tlg_last_error()


# ------------------------------------------------- softmax-CE, elementwise --
@pytest.mark.parametrize("N,V,scale,spread", [(300, 2048, None, 1.0), (97, 2048, 0.2, 1.0), (4, 50, None, 1.0),
                                               (300, 2048, None, 3.0)])
def test_xent(lib, st, N, V, scale, spread):
    """dlogits has one entry per row near -scale and the rest near scale/V,
    so max|err| / mean|ref| is ~V/2 ulps for ANY fp32 evaluation (the
    oracle itself is at 6e-5 against float64 at V = 2048): the normwise bar
    is ill-conditioned here.  Each entry above 1e-3 of its row's largest is
    held to 1e-5 relative of float64 instead, every entry to 1e-6 of its
    row's largest, and the loss to 1e-5 relative of the oracle's."""
    import ctypes
    r = np.random.default_rng(N)
    lg = (spread * r.standard_normal((N, V))).astype(np.float32)
    tgt = r.integers(0, V, N).astype(np.int32)
    sc = 1.0 / N if scale is None else scale / N
    DL, loss, LG, TG = nan_like((N, V)), nan_like((1,)), dev(lg), dev(tgt)
    lib.check(lib.tlg_dev_xent(LG.data_ptr(), TG.data_ptr(), DL.data_ptr(), loss.data_ptr(), sc, N, V,
                               stream()), "xent")
    got = host(DL)
    want = np.empty_like(lg)
    fp, ip = ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_int)
    wl = st._fn("xent")(lg.ctypes.data_as(fp), tgt.ctypes.data_as(ip), want.ctypes.data_as(fp), sc, N, V)
    assert abs(float(host(loss)[0]) - wl) <= 1e-5 * wl
    l64 = lg.astype(np.float64)
    p64 = np.exp(l64 - l64.max(1, keepdims=True))
    p64 /= p64.sum(1, keepdims=True)
    d64 = p64 * sc
    d64[np.arange(N), tgt] -= sc
    rowmax = np.abs(d64).max(1, keepdims=True)
    big = np.abs(d64) > 1e-3 * rowmax
    assert (np.abs(got - d64)[big] / np.abs(d64)[big]).max() <= 1e-5
    assert (np.abs(got - d64) / rowmax).max() <= 1e-6


@pytest.mark.parametrize("n,off", [(1_000_003, 0), (1_000_003, 1), (5, 0), (3, 2)])
def test_gradnorm_any_alignment(lib, n, off):
    """The norm's float4 pass (16-byte aligned G) and its element-wise pass
    (G offset by one or two floats, and the n % 4 tail) against float64."""
    r = np.random.default_rng(n + off)
    G = (0.01 * r.standard_normal(n + off)).astype(np.float32)
    Gd = dev(G)
    norm = nan_like((1,))
    lib.check(lib.tlg_dev_gradnorm(Gd.data_ptr() + 4 * off, n, norm.data_ptr(), stream()), "gradnorm")
    want = np.sqrt((G[off:].astype(np.float64) ** 2).sum())
    assert abs(float(host(norm)[0]) - want) <= 1e-6 * want


@pytest.mark.parametrize("N,V", [(300, 2048), (4, 50), (4096, 2048)])
def test_loss_in_gradnorm_is_bit_identical(lib, N, V):
    """The training step's split of tlg_dev_xent: tlg_dev_xent_rows (per-row
    losses, no sum) then tlg_dev_gradnorm_loss (the norm and the loss mean in
    one last kernel) give tlg_dev_xent's loss and dlogits and
    tlg_dev_gradnorm's norm bit for bit."""
    t = _t()
    r = np.random.default_rng(N + V)
    lg = r.standard_normal((N, V)).astype(np.float32)
    tgt = r.integers(0, V, N).astype(np.int32)
    G = (0.01 * r.standard_normal(200_003)).astype(np.float32)
    LG, TG, Gd = dev(lg), dev(tgt), dev(G)
    dl0, dl1 = nan_like((N, V)), nan_like((N, V))
    loss0, loss1, n0, n1 = nan_like((1,)), nan_like((1,)), nan_like((1,)), nan_like((1,))
    rows = t.full((N,), float("nan"), dtype=t.float64, device="cuda")
    lib.check(lib.tlg_dev_xent(LG.data_ptr(), TG.data_ptr(), dl0.data_ptr(), loss0.data_ptr(), 1.0 / N, N, V,
                               stream()), "xent")
    lib.check(lib.tlg_dev_gradnorm(Gd.data_ptr(), G.size, n0.data_ptr(), stream()), "gradnorm")
    lib.check(lib.tlg_dev_xent_rows(LG.data_ptr(), TG.data_ptr(), dl1.data_ptr(), rows.data_ptr(), 1.0 / N, N, V,
                                    stream()), "xent_rows")
    lib.check(lib.tlg_dev_gradnorm_loss(Gd.data_ptr(), G.size, n1.data_ptr(), rows.data_ptr(), N,
                                        loss1.data_ptr(), stream()), "gradnorm_loss")
    assert np.array_equal(host(dl0), host(dl1))
    assert host(loss0)[0] == host(loss1)[0] and host(n0)[0] == host(n1)[0]
    p = Gd.data_ptr()
    assert lib.tlg_dev_gradnorm_loss(p, 10, p, 0, N, p, stream()) != 0            # no rows
    assert lib.tlg_dev_xent_rows(p, p, p, 0, 1.0, N, V, stream()) != 0            # no rows
    lib.tlg_last_error()


def test_embedding_bit_exact(lib, st):
    import ctypes
    r = np.random.default_rng(1)
    V, D, N = 2048, 256, 4096
    emb = r.standard_normal((V, D)).astype(np.float32)
    tok = r.integers(0, V, N).astype(np.int32)
    tok[100:400] = 7                                   # one long bucket
    out, T, EM = nan_like((N, D)), dev(tok), dev(emb)
    lib.check(lib.tlg_dev_embed_fwd(out.data_ptr(), EM.data_ptr(), T.data_ptr(), N, D, V, stream()), "fwd")
    assert np.array_equal(host(out), emb[tok])
    dout = r.standard_normal((N, D)).astype(np.float32)
    de0 = r.standard_normal((V, D)).astype(np.float32)
    DE, DO = dev(de0), dev(dout)
    lib.check(lib.tlg_dev_embed_bwd(DE.data_ptr(), DO.data_ptr(), T.data_ptr(), N, D, V, stream()), "bwd")
    want = de0.copy()
    fp, ip = ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_int)
    st._fn("embed_bwd")(want.ctypes.data_as(fp), dout.ctypes.data_as(fp), tok.ctypes.data_as(ip), N, D)
    assert np.array_equal(host(DE), want)


@pytest.mark.parametrize("V,D,N", [(2048, 256, 4096), (50, 36, 77), (300, 1028, 130), (40, 2048, 9),
                                   (30, 2052, 5)])
def test_embed_rmsnorm_fwd_is_bit_identical(lib, V, D, N):
    """tlg_dev_embed_rmsnorm_fwd against tlg_dev_embed_fwd then
    tlg_dev_rmsnorm_fwd: x, out and rinv bit for bit, NaN rows for tokens
    outside [0, V) included; D of one to eight float4 columns per lane, and
    D > 2048 (the two-pass fallback)."""
    print("embed_rmsnorm", V, D, N, flush=True)
    r = np.random.default_rng(V * D + N)
    emb = r.standard_normal((V, D)).astype(np.float32)
    g = (1.0 + 0.1 * r.standard_normal(D)).astype(np.float32)
    tok = r.integers(0, V, N).astype(np.int32)
    tok[::5] = V                                        # outside [0, V): NaN rows
    tok[1::7] = -3
    EM, G, T = dev(emb), dev(g), dev(tok)
    x0, o0, x1, o1 = nan_like((N, D)), nan_like((N, D)), nan_like((N, D)), nan_like((N, D))
    r0, r1 = nan_like((N,)), nan_like((N,))
    lib.check(lib.tlg_dev_embed_fwd(x0.data_ptr(), EM.data_ptr(), T.data_ptr(), N, D, V, stream()), "embed")
    lib.check(lib.tlg_dev_rmsnorm_fwd(x0.data_ptr(), G.data_ptr(), o0.data_ptr(), r0.data_ptr(), N, D, stream()),
              "rms")
    lib.check(lib.tlg_dev_embed_rmsnorm_fwd(EM.data_ptr(), T.data_ptr(), V, x1.data_ptr(), G.data_ptr(),
                                            o1.data_ptr(), r1.data_ptr(), N, D, stream()), "embed_rms")
    for a0, a1 in ((x0, x1), (o0, o1), (r0, r1)):
        assert np.array_equal(host(a0), host(a1), equal_nan=True)
    assert np.isnan(host(x1)[::5]).all() and not np.isnan(host(x1)[2]).any()


@pytest.mark.parametrize("V,D,N", [(2048, 384, 8192), (50, 128, 5000), (37, 36, 77), (2048, 1028, 300),
                                   (64, 64, 4100)])
def test_embedding_bwd_shapes(lib, V, D, N):
    """The one-launch scatter (D <= 1024: several 4096-token passes, heavy
    buckets, ragged D / 4) and the counting-sort path (D > 1024) against
    token-order float32 adds; ids outside [0, V) are skipped."""
    print("embed_bwd", V, D, N, flush=True)
    r = np.random.default_rng(V + D + N)
    tok = r.integers(0, V, N).astype(np.int32)
    tok[N // 3: N // 3 + min(N // 3, 2000)] = V // 2          # a heavy bucket
    tok[::97] = -1
    tok[5::101] = V
    dout = r.standard_normal((N, D)).astype(np.float32)
    de0 = r.standard_normal((V, D)).astype(np.float32)
    DE, DO, T = dev(de0), dev(dout), dev(tok)
    lib.check(lib.tlg_dev_embed_bwd(DE.data_ptr(), DO.data_ptr(), T.data_ptr(), N, D, V, stream()), "bwd")
    want = de0.copy()
    for n in range(N):
        t = int(tok[n])
        if 0 <= t < V:
            want[t] += dout[n]
    assert np.array_equal(host(DE), want)


def test_elementwise(lib):
    r = np.random.default_rng(2)
    n = 100003
    a, b, x = (r.standard_normal(n).astype(np.float32) for _ in range(3))
    A, Bt, X = dev(a), dev(b), dev(x)
    a64, b64, x64 = a.astype(np.float64), b.astype(np.float64), x.astype(np.float64)
    sg = 1 / (1 + np.exp(-a64))
    y = nan_like((n,))
    lib.check(lib.tlg_dev_swiglu_fwd(y.data_ptr(), A.data_ptr(), Bt.data_ptr(), n, stream()), "swiglu")
    assert normwise_rel(host(y), a64 * sg * b64) <= TOL
    y2 = nan_like((n,))
    lib.check(lib.tlg_dev_swiglu_bwd(X.data_ptr(), A.data_ptr(), Bt.data_ptr(), y.data_ptr(), y2.data_ptr(), n,
                                     stream()), "swiglu_bwd")
    ds = sg + a64 * sg * (1 - sg)
    assert normwise_rel(host(y), x64 * b64 * ds) <= TOL and normwise_rel(host(y2), x64 * a64 * sg) <= TOL
    lib.check(lib.tlg_dev_silu_res(y.data_ptr(), X.data_ptr(), A.data_ptr(), n, stream()), "silu_res")
    assert normwise_rel(host(y), x64 + a64 * sg) <= TOL
    lib.check(lib.tlg_dev_silu_bwd(y.data_ptr(), X.data_ptr(), A.data_ptr(), n, stream()), "silu_bwd")
    assert normwise_rel(host(y), x64 * ds) <= TOL
    Y = dev(b)
    lib.check(lib.tlg_dev_add(Y.data_ptr(), X.data_ptr(), n, stream()), "add")
    assert np.array_equal(host(Y), b + x)


def test_gradnorm_and_adamw(lib, st):
    r = np.random.default_rng(3)
    n = 1_000_003
    P = (0.02 * r.standard_normal(n)).astype(np.float32)
    G = (0.01 * r.standard_normal(n)).astype(np.float32)
    M = (0.001 * r.standard_normal(n)).astype(np.float32)
    V = np.abs(1e-5 * r.standard_normal(n)).astype(np.float32)
    Pd, Gd, Md, Vd = dev(P), dev(G), dev(M), dev(V)
    norm = nan_like((1,))
    lib.check(lib.tlg_dev_gradnorm(Gd.data_ptr(), n, norm.data_ptr(), stream()), "gradnorm")
    gn = float(host(norm)[0])
    assert abs(gn - np.sqrt((G.astype(np.float64) ** 2).sum())) <= 1e-6 * gn
    assert gn > 1.0                                                      # the clip is active
    t = 7
    hyper = np.array([3e-4, 0.9, 0.95, 0.1, 1 - np.float32(0.9) ** t, 1 - np.float32(0.95) ** t, 0, 0], np.float32)
    hyper[4] = np.float32(1.0) - np.power(np.float32(0.9), np.float32(t))
    hyper[5] = np.float32(1.0) - np.power(np.float32(0.95), np.float32(t))
    HY = dev(hyper)
    lib.check(lib.tlg_dev_adamw(Pd.data_ptr(), Gd.data_ptr(), Md.data_ptr(), Vd.data_ptr(), n,
                                HY.data_ptr(), norm.data_ptr(), stream()), "adamw")
    st.adamw(P, G, M, V, 3e-4, 0.9, 0.95, 0.1, t, np.float32(1.0) / np.float32(gn))
    for got, want, name in ((Pd, P, "P"), (Md, M, "M"), (Vd, V, "V")):
        assert normwise_rel(host(got), want) <= 1e-6, name


# ------------------------------------------------------------ whole steps --
def fixture_model(d):
    V, D, L, H, KV, F, T, n_mtp, n_exp, win, fe = (int(x) for x in d["model"])
    return dict(V=V, D=D, L=L, H=H, KV=KV, F=F, T=T, n_mtp=n_mtp, n_exp=n_exp, win=win, full_every=fe)


def regions(st, kw):
    return param_regions(st, model(**kw))


def run_step(tr, P, tok, tgt, tgt_mtp):
    s = stream()
    tr.upload(P, s)
    tr.set_batch(tok, tgt, tgt_mtp if tr.model.n_mtp else None, s)
    tr.forward(s)
    tr.backward(s)
    _t().cuda.synchronize()
    loss = tr.loss(s)
    G = np.empty(tr.np, np.float32)
    import tlgemm
    L = tlgemm.load()
    L.check(L.tlg_memcpy_d2h(G.ctypes.data, tr.buf(1), G.nbytes, s), "d2h")
    L.check(L.tlg_stream_sync(s), "sync")
    return loss, G


@pytest.mark.parametrize("path", golden("step_train_*.npz"), ids=os.path.basename)
def test_train_step_matches_reference_fixture(lib, st, path):
    import tlgemm
    d = load_npz(path)
    kw = fixture_model(d)
    print("train fixture", os.path.basename(path), kw, flush=True)
    tr = tlgemm.host().train(kw, int(d["B"]))
    loss, G = run_step(tr, d["P"], d["tok"], d["tgt"], d["tgt_mtp"])
    assert abs(loss - float(d["loss"])) <= 1e-5 * float(d["loss"])
    for name, a, b in regions(st, kw):
        assert normwise_rel(G[a:b], d["G"][a:b]) <= TOL, name


SHAPES = {
    "nano": (dict(V=2048, D=128, L=1, H=4, KV=1, F=384, T=256), 8),
    "m3": (dict(V=2048, D=256, L=6, H=8, KV=2, F=768, T=256), 16),
    "m8_mtp2": (dict(V=2048, D=384, L=2, H=12, KV=3, F=1024, T=256, n_mtp=2), 8),
    "m3_moe": (dict(V=2048, D=256, L=2, H=8, KV=2, F=768, T=256, n_exp=4), 16),
}


@pytest.mark.parametrize("name", list(SHAPES))
def test_train_step_matches_oracle(lib, st, name):
    import tlgemm
    kw, B = SHAPES[name]
    print("train step", name, kw, B, flush=True)
    m = model(**kw)
    P = st.init_params(m, 1234567891011)
    P[m.V * m.D:] += (0.01 * np.random.default_rng(0).standard_normal(P.size - m.V * m.D)).astype(np.float32)
    r = np.random.default_rng(5)
    N = B * m.T
    tok, tgt = (r.integers(0, m.V, N).astype(np.int32) for _ in range(2))
    tm = r.integers(0, m.V, (max(m.n_mtp, 1), N)).astype(np.int32)
    tr = tlgemm.host().train(kw, B)
    loss, G = run_step(tr, P, tok, tgt, tm)
    st.dll.orc_set_threads(16)
    wl, WG = st.train_step(m, B, P, tok, tgt, tm)
    assert abs(loss - wl) <= 1e-5 * wl
    worst = sorted(((normwise_rel(G[a:b], WG[a:b]), n) for n, a, b in regions(st, kw)), reverse=True)
    print("worst tensors", [(f"{e:.2e}", n) for e, n in worst[:4]], flush=True)
    assert worst[0][0] <= TOL, worst[0]


def test_optimizer_step_matches_oracle(lib, st):
    """gradnorm + clip + AdamW on the device step's own G (tinylm.c:2630-2633)."""
    import tlgemm
    kw, B = SHAPES["nano"]
    m = model(**kw)
    P = st.init_params(m, 7)
    r = np.random.default_rng(6)
    N = B * m.T
    tok, tgt = (r.integers(0, m.V, N).astype(np.int32) for _ in range(2))
    tr = tlgemm.host().train(kw, B)
    s = stream()
    _, G = run_step(tr, P, tok, tgt, None)
    tr.set_hyper(1e-3, 0.9, 0.95, 0.1, 1, s)
    tr.optimize(s)
    gn = tr.gnorm(s)
    want_gn = st.gradnorm(G)
    assert abs(gn - want_gn) <= 1e-6 * want_gn
    P1 = np.empty_like(P)
    lib.check(lib.tlg_memcpy_d2h(P1.ctypes.data, tr.buf(0), P1.nbytes, s), "d2h")
    lib.check(lib.tlg_stream_sync(s), "sync")
    Mo, Vo = np.zeros_like(P), np.zeros_like(P)
    gs = np.float32(1.0) / np.float32(gn) if gn > 1.0 else np.float32(1.0)
    st.adamw(P, G, Mo, Vo, 1e-3, 0.9, 0.95, 0.1, 1, gs)
    assert normwise_rel(P1, P) <= 1e-6


def test_graph_replays_match_eager(lib, st):
    """Three captured steps (forward + backward + AdamW) replayed from the
    same start equal three eager steps bit for bit, loss and parameters."""
    import tlgemm
    kw, B = dict(V=256, D=64, L=2, H=2, KV=1, F=96, T=64, n_mtp=1), 4
    m = model(**kw)
    P0 = st.init_params(m, 3)
    r = np.random.default_rng(7)
    N = B * m.T
    tok, tgt = (r.integers(0, m.V, N).astype(np.int32) for _ in range(2))
    tm = r.integers(0, m.V, (1, N)).astype(np.int32)
    tr = tlgemm.host().train(kw, B)
    s = lib.tlg_stream_create()          # a capturable stream (not the legacy default one)

    def run(graph):
        tr.upload(P0, s)
        tr.set_batch(tok, tgt, tm, s)
        losses = []
        for it in range(3):
            tr.set_hyper(1e-3, 0.9, 0.95, 0.1, it + 1, s)
            if graph:
                tr.graph_step(s)
            else:
                tr.step(s)
            losses.append(tr.loss(s))
        P = np.empty_like(P0)
        lib.check(lib.tlg_memcpy_d2h(P.ctypes.data, tr.buf(0), P.nbytes, s), "d2h")
        lib.check(lib.tlg_stream_sync(s), "sync")
        return losses, P

    eager_l, eager_P = run(False)
    tr.graph_build(s)
    for rep in range(2):
        l, P = run(True)
        assert l == eager_l, rep
        assert np.array_equal(P, eager_P), rep
    assert eager_l[2] < eager_l[0]                # AdamW steps lower the loss on a fixed batch


def test_autotuned_step_matches_and_replays(lib, st):
    """tl_train_autotune pins a tile configuration per grouped launch: the
    parameters are left as they were, a step with the table gives the
    untuned step's loss and gradients within the bar (only the tile shapes
    change), and the graph captured after it replays the eager tuned step
    bit for bit."""
    import tlgemm
    kw, B = dict(V=256, D=128, L=2, H=4, KV=1, F=192, T=64, n_mtp=1), 4
    m = model(**kw)
    P0 = st.init_params(m, 5)
    r = np.random.default_rng(11)
    N = B * m.T
    tok, tgt = (r.integers(0, m.V, N).astype(np.int32) for _ in range(2))
    tm = r.integers(0, m.V, (1, N)).astype(np.int32)
    s = lib.tlg_stream_create()

    def fetch(tr, which):
        X = np.empty_like(P0)
        lib.check(lib.tlg_memcpy_d2h(X.ctypes.data, tr.buf(which), X.nbytes, s), "d2h")
        lib.check(lib.tlg_stream_sync(s), "sync")
        return X

    def one_step(tr, graph=False):
        tr.upload(P0, s)
        tr.set_batch(tok, tgt, tm, s)
        tr.set_hyper(1e-3, 0.9, 0.95, 0.1, 1, s)
        if graph:
            tr.graph_step(s)
        else:
            tr.step(s)
        return tr.loss(s), fetch(tr, 1)            # loss and the step's gradients

    l0, G_auto = one_step(tlgemm.host().train(kw, B))
    tuned = tlgemm.host().train(kw, B)
    one_step(tuned)                                  # sizes the scratch
    tuned.upload(P0, s)
    tiles = tuned.autotune([3, 14, 15, 20], 1, s)
    assert tiles and all(c in (3, 14, 15, 20) for c in tiles), tiles
    assert np.array_equal(fetch(tuned, 0), P0)      # autotuning does not step the model
    l1, G_tuned = one_step(tuned)
    assert abs(l1 - l0) <= 1e-5 * abs(l0)
    assert normwise_rel(G_tuned, G_auto) <= TOL
    tuned.graph_build(s)
    l2, G_graph = one_step(tuned, graph=True)
    assert l2 == l1 and np.array_equal(G_graph, G_tuned)
