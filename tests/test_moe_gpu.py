"""GPU parity of the top-1 MoE layer (tinylm.c:857-947) through the C ABI.

Each case runs tlg_dev_moe_grouped_fwd / _bwd (or the host-pointer drop-ins)
and compares with the golden vectors written by tinylm.c's own moe_forward /
moe_backward, with the CPU oracle on the same seeded inputs, and with a
float64 brute force (torch autograd on the CPU, routing held fixed).

Bars: routing (assign) identical; rprobs and gate within 1e-6 absolute;
every output within 1e-4 normwise (max|err| / mean|ref|, tinylm.c:4782-4784)
of the fp32 reference, and each gradient increment and d_fnorm within 1e-4
of float64.  The expert part of `out` is checked on its own (out - fin, up to
out's final rounding), so its error is not hidden behind fin.
"""
import os
import zlib

import numpy as np
import pytest

from conftest import golden, load_npz
from oracle import normwise_rel

pytestmark = pytest.mark.gpu
TOL = 1e-4
MOES = golden("moe_*.npz")


def _torch():
    import torch
    return torch


def dev(a):
    return _torch().from_numpy(np.ascontiguousarray(a)).cuda()


def stream():
    return _torch().cuda.current_stream().cuda_stream


def gpu_forward(lib, fnorm, fin, wr, w1, w3, w2):
    t = _torch()
    N, D = fnorm.shape
    E, F = wr.shape[1], w1.shape[2]
    ins = [dev(a) for a in (fnorm, fin, wr, w1, w3, w2)]
    out = t.full((N, D), float("nan"), dtype=t.float32, device="cuda")
    assign = t.full((N,), -7, dtype=t.int32, device="cuda")
    gate = t.full((N,), float("nan"), dtype=t.float32, device="cuda")
    rprobs = t.full((N, E), float("nan"), dtype=t.float32, device="cuda")
    f, fi, r, a1, a3, a2 = (x.data_ptr() for x in ins)
    lib.moe_fwd(f, fi, out.data_ptr(), N, D, F, E, r, a1, a3, a2, assign.data_ptr(), gate.data_ptr(),
                rprobs.data_ptr(), stream())
    return out.cpu().numpy(), assign.cpu().numpy(), gate.cpu().numpy(), rprobs.cpu().numpy()


def gpu_backward(lib, fnorm, dout, assign, gate, rprobs, wr, w1, w3, w2, gwr0, gw10, gw30, gw20):
    t = _torch()
    N, D = fnorm.shape
    E, F = wr.shape[1], w1.shape[2]
    ins = [dev(a) for a in (fnorm, dout, assign, gate, rprobs, wr, w1, w3, w2)]
    grads = [dev(a) for a in (gwr0, gw10, gw30, gw20)]
    dfn = t.full((N, D), float("nan"), dtype=t.float32, device="cuda")
    p = [x.data_ptr() for x in ins]
    g = [x.data_ptr() for x in grads]
    lib.moe_bwd(p[0], p[1], dfn.data_ptr(), p[2], p[3], p[4], N, D, F, E, p[5], p[6], p[7], p[8],
                g[0], g[1], g[2], g[3], stream())
    return dfn.cpu().numpy(), [x.cpu().numpy() for x in grads]


def f64_moe(fnorm, fin, wr, w1, w3, w2, dout, assign):
    """Float64 brute force, expert by expert, with the routing fixed to
    `assign`: out, d_fnorm and the gradients of wr, w1, w3, w2 of
    L = <out, dout> + 0.01 E sum_e (cnt_e / N) mean_n p[n, e]."""
    torch = _torch()
    N, D = fnorm.shape
    E = wr.shape[1]
    t = lambda a: torch.tensor(a, dtype=torch.float64, requires_grad=True)  # noqa: E731
    x, r, a1, a3, a2 = t(fnorm), t(wr), t(w1), t(w3), t(w2)
    fi = torch.tensor(fin, dtype=torch.float64)
    do = torch.tensor(dout, dtype=torch.float64)
    a = torch.tensor(assign.astype(np.int64))
    p = torch.softmax(x @ r, dim=1)
    out = fi.clone()
    for e in range(E):
        rows = (a == e).nonzero().flatten()
        if len(rows) == 0:
            continue
        xe = x[rows]
        h = torch.nn.functional.silu(xe @ a1[e]) * (xe @ a3[e])
        out = out.index_add(0, rows, p[rows, e:e + 1] * (h @ a2[e]))
    cnt = torch.bincount(a, minlength=E).to(torch.float64)
    loss = (out * do).sum() + 0.01 * E * ((cnt / N) * p.mean(dim=0)).sum()
    loss.backward()
    return (out.detach().numpy(), x.grad.numpy(), r.grad.numpy(), a1.grad.numpy(), a3.grad.numpy(),
            a2.grad.numpy())


def case(N, D, F, E, seed, skew=0.0, dead=()):
    """Seeded inputs; `skew` tilts the router towards low expert indices and
    experts in `dead` are never chosen (their router column is -inf-like)."""
    rng = np.random.default_rng(seed)
    fnorm = rng.standard_normal((N, D), dtype=np.float32)
    fin = rng.standard_normal((N, D), dtype=np.float32)
    wr = (0.1 * rng.standard_normal((D, E))).astype(np.float32)
    if skew:
        # a shared direction of the tokens scores experts in decreasing order
        fnorm[:, 0] = np.abs(fnorm[:, 0]) + 1.0
        wr[0, :] += (skew * np.linspace(1.0, 0.0, E)).astype(np.float32)
    for e in dead:
        fnorm[:, 1] = np.abs(fnorm[:, 1]) + 1.0
        wr[1, e] = -50.0
    w1 = (0.05 * rng.standard_normal((E, D, F))).astype(np.float32)
    w3 = (0.05 * rng.standard_normal((E, D, F))).astype(np.float32)
    w2 = (0.05 * rng.standard_normal((E, F, D))).astype(np.float32)
    dout = (0.01 * rng.standard_normal((N, D))).astype(np.float32)
    g0 = [rng.standard_normal(s, dtype=np.float32) for s in ((D, E), (E, D, F), (E, D, F), (E, F, D))]
    return dict(fnorm=fnorm, fin=fin, wr=wr, w1=w1, w3=w3, w2=w2, dout=dout,
                gwr0=g0[0], gw10=g0[1], gw30=g0[2], gw20=g0[3])


def check_forward(got, ref_out, ref_assign, ref_gate, ref_rprobs, fin):
    out, assign, gate, rprobs = got
    assert np.array_equal(assign, ref_assign), np.nonzero(assign != ref_assign)[0][:8]
    assert np.abs(rprobs - ref_rprobs).max() <= 1e-6
    assert np.abs(gate - ref_gate).max() <= 1e-6
    assert normwise_rel(out, ref_out) <= TOL
    assert_delta(out - fin, ref_out - fin, ref_out)


def assert_delta(got, ref, out):
    """An increment (out = base + increment, e.g. fin + gate*y, or a gradient
    added onto its prefill) within the bar, up to the final fp32 rounding of
    out (half an ulp on each side when `ref` is fp32 too)."""
    bound = TOL * np.abs(ref).mean() + np.spacing(np.abs(out).astype(np.float32))
    assert (np.abs(got - ref) <= bound).all(), float((np.abs(got - ref) / bound).max())


def check_backward(dfn, grads, ref_dfn, ref_grads, g0, f64):
    """Outputs (d_fnorm set, gradients accumulated onto g0) against the
    fp32 reference; d_fnorm and the gradient increments against float64.
    (Increments are compared with float64 only: with the router's softmax
    cancellation an fp32 increment carries its own ~1e-4 error, so two fp32
    computations may differ by twice the bar while both meet it.)"""
    dfn64, g64 = f64
    assert normwise_rel(dfn, ref_dfn) <= TOL
    assert normwise_rel(dfn, dfn64) <= TOL
    for name, got, ref, base, exact in zip(("gwr", "gw1", "gw3", "gw2"), grads, ref_grads, g0, g64):
        assert normwise_rel(got, ref) <= TOL, name
        assert_delta(got - base, exact, got)


@pytest.mark.parametrize("path", MOES, ids=[os.path.basename(p)[4:-4] for p in MOES])
def test_golden(lib, path):
    """Against the golden vectors of the reference's own moe_forward/_backward."""
    d = load_npz(path)
    print("case", os.path.basename(path), flush=True)
    got = gpu_forward(lib, d["fnorm"], d["fin"], d["wr"], d["w1"], d["w3"], d["w2"])
    check_forward(got, d["out"], d["assign"], d["gate"], d["rprobs"], d["fin"])
    g0 = [d[k] for k in ("gwr0", "gw10", "gw30", "gw20")]
    dfn, grads = gpu_backward(lib, d["fnorm"], d["dout"], d["assign"], d["gate"], d["rprobs"], d["wr"],
                              d["w1"], d["w3"], d["w2"], *g0)
    check_backward(dfn, grads, d["dfn"], [d[k] for k in ("gwr", "gw1", "gw3", "gw2")], g0, fixture_f64(d))


def fixture_f64(d):
    _, dfn64, *g64 = f64_moe(d["fnorm"], d["fin"], d["wr"], d["w1"], d["w3"], d["w2"], d["dout"], d["assign"])
    return dfn64, g64


def test_golden_host_entries(lib):
    """tlg_moe_grouped_fwd / _bwd on host pointers (the drop-in form)."""
    import ctypes
    d = load_npz(golden("moe_n96_*.npz")[0])
    N, D = d["fnorm"].shape
    E, F = d["wr"].shape[1], d["w1"].shape[2]
    P = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    c = {k: np.ascontiguousarray(v) for k, v in d.items()}
    out = np.full((N, D), np.nan, np.float32)
    assign = np.full(N, -1, np.int32)
    gate = np.full(N, np.nan, np.float32)
    rprobs = np.full((N, E), np.nan, np.float32)
    lib.tlg_moe_grouped_fwd(P(c["fnorm"]), P(c["fin"]), P(out), N, D, F, E, P(c["wr"]), P(c["w1"]),
                            P(c["w3"]), P(c["w2"]), P(assign), P(gate), P(rprobs))
    check_forward((out, assign, gate, rprobs), d["out"], d["assign"], d["gate"], d["rprobs"], d["fin"])
    g = [c[k].copy() for k in ("gwr0", "gw10", "gw30", "gw20")]
    dfn = np.full((N, D), np.nan, np.float32)
    lib.tlg_moe_grouped_bwd(P(c["fnorm"]), P(c["dout"]), P(dfn), P(assign), P(gate), P(rprobs), N, D, F, E,
                            P(c["wr"]), P(c["w1"]), P(c["w3"]), P(c["w2"]), *[P(x) for x in g])
    check_backward(dfn, g, d["dfn"], [d[k] for k in ("gwr", "gw1", "gw3", "gw2")],
                   [d[k] for k in ("gwr0", "gw10", "gw30", "gw20")], fixture_f64(d))


SHAPES = [
    # N, D, F, E, skew, dead experts
    (4096, 256, 768, 4, 2.0, ()),      # the MoE training config, skewed routing
    (4096, 256, 768, 4, 0.0, ()),
    (67, 32, 48, 3, 0.0, ()),          # ragged N, odd E
    (2500, 64, 96, 5, 1.0, (3,)),      # several 1024-token index chunks, an empty expert
    (9000, 16, 32, 4, 1.0, ()),        # crosses the index kernel's 8192-token rounds
    (300, 16, 32, 64, 0.0, ()),        # the maximum E: most experts hold 0-10 rows
    (1, 8, 8, 4, 0.0, ()),             # one token
    (513, 32, 64, 1, 0.0, ()),         # one expert takes every token
]


@pytest.mark.parametrize("N,D,F,E,skew,dead", SHAPES, ids=[f"{s[0]}x{s[1]}x{s[2]}_e{s[3]}" for s in SHAPES])
def test_against_oracle_and_f64(lib, orc, N, D, F, E, skew, dead):
    seed = zlib.crc32(f"moe {N} {D} {F} {E} {skew}".encode())
    print("case", N, D, F, E, skew, dead, "seed", seed, flush=True)
    c = case(N, D, F, E, seed, skew, dead)
    r_out, r_assign, r_gate, r_rprobs = orc.moe_forward(c["fnorm"], c["fin"], c["wr"], c["w1"], c["w3"],
                                                         c["w2"])
    got = gpu_forward(lib, c["fnorm"], c["fin"], c["wr"], c["w1"], c["w3"], c["w2"])
    check_forward(got, r_out, r_assign, r_gate, r_rprobs, c["fin"])
    for e in dead:
        assert not (got[1] == e).any()
    g0 = [c[k] for k in ("gwr0", "gw10", "gw30", "gw20")]
    ref_g = [x.copy() for x in g0]
    r_dfn = orc.moe_backward(c["fnorm"], c["dout"], c["wr"], c["w1"], c["w3"], c["w2"], *ref_g,
                             r_assign, r_gate, r_rprobs)
    dfn, grads = gpu_backward(lib, c["fnorm"], c["dout"], r_assign, r_gate, r_rprobs, c["wr"], c["w1"],
                              c["w3"], c["w2"], *g0)
    o64, dfn64, *g64 = f64_moe(c["fnorm"], c["fin"], c["wr"], c["w1"], c["w3"], c["w2"], c["dout"], r_assign)
    assert_delta(got[0] - c["fin"], o64 - c["fin"], o64)
    check_backward(dfn, grads, r_dfn, ref_g, g0, (dfn64, g64))


@pytest.mark.parametrize("cfg", [3, 14, 15, 18, 22])
@pytest.mark.parametrize("sched", [0, 1, 2])
def test_expert_tile_forms(lib, orc, cfg, sched):
    """Every tile shape and stage order an expert launch can take (pinned with
    tlg_tune_expert), on the MoE training config with skewed routing and on a
    ragged one, against the oracle and fp64."""
    lib.check(lib.tlg_tune_expert(cfg, sched), "tune expert")
    try:
        for N, D, F, E, skew in ((4096, 256, 768, 4, 2.0), (67, 32, 48, 3, 0.0)):
            seed = zlib.crc32(f"moe tiles {N} {D} {F} {E} {skew}".encode())
            print("case", cfg, sched, N, D, F, E, skew, "seed", seed, flush=True)
            c = case(N, D, F, E, seed, skew, ())
            r_out, r_assign, r_gate, r_rprobs = orc.moe_forward(c["fnorm"], c["fin"], c["wr"], c["w1"],
                                                                 c["w3"], c["w2"])
            got = gpu_forward(lib, c["fnorm"], c["fin"], c["wr"], c["w1"], c["w3"], c["w2"])
            check_forward(got, r_out, r_assign, r_gate, r_rprobs, c["fin"])
            g0 = [c[k] for k in ("gwr0", "gw10", "gw30", "gw20")]
            ref_g = [x.copy() for x in g0]
            r_dfn = orc.moe_backward(c["fnorm"], c["dout"], c["wr"], c["w1"], c["w3"], c["w2"], *ref_g,
                                     r_assign, r_gate, r_rprobs)
            dfn, grads = gpu_backward(lib, c["fnorm"], c["dout"], r_assign, r_gate, r_rprobs, c["wr"],
                                      c["w1"], c["w3"], c["w2"], *g0)
            o64, dfn64, *g64 = f64_moe(c["fnorm"], c["fin"], c["wr"], c["w1"], c["w3"], c["w2"], c["dout"],
                                      r_assign)
            assert_delta(got[0] - c["fin"], o64 - c["fin"], o64)
            check_backward(dfn, grads, r_dfn, ref_g, g0, (dfn64, g64))
    finally:
        lib.check(lib.tlg_tune_expert(-1, -1), "tune expert")
    assert lib.tlg_tune_expert(8, 1) != 0 and lib.tlg_tune_expert(3, 3) != 0


def test_skewed_split(lib):
    """The skewed config really is unbalanced (so the test above exercises
    experts of very different row counts)."""
    c = case(4096, 256, 768, 4, zlib.crc32(b"moe 4096 256 768 4 2.0"), 2.0)
    _, assign, _, _ = gpu_forward(lib, c["fnorm"], c["fin"], c["wr"], c["w1"], c["w3"], c["w2"])
    cnt = np.bincount(assign, minlength=4)
    assert cnt.max() > 2 * cnt.min() and cnt.min() > 0, cnt


def test_deterministic(lib):
    c = case(1000, 64, 128, 4, 7, 1.0)
    a = gpu_forward(lib, c["fnorm"], c["fin"], c["wr"], c["w1"], c["w3"], c["w2"])
    b = gpu_forward(lib, c["fnorm"], c["fin"], c["wr"], c["w1"], c["w3"], c["w2"])
    for x, y in zip(a, b):
        assert np.array_equal(x, y)
    g0 = [c[k] for k in ("gwr0", "gw10", "gw30", "gw20")]
    r1 = gpu_backward(lib, c["fnorm"], c["dout"], a[1], a[2], a[3], c["wr"], c["w1"], c["w3"], c["w2"], *g0)
    r2 = gpu_backward(lib, c["fnorm"], c["dout"], a[1], a[2], a[3], c["wr"], c["w1"], c["w3"], c["w2"], *g0)
    assert np.array_equal(r1[0], r2[0])
    for x, y in zip(r1[1], r2[1]):
        assert np.array_equal(x, y)


def gpu_pair_kept(lib, c, interleave=None, finish="flush"):
    """Forward with kept state, then (after `interleave()`, other MoE calls
    that reuse the library's scratch) the backward from that state.  The
    backward leaves reductions queued (dWr's column sum, the dW1 / dW3 slice
    sums); `finish` completes them with tlg_dev_gemm_flush, or ("free") with
    tlg_dev_free of an unrelated buffer, which must launch them first."""
    t = _torch()
    N, D = c["fnorm"].shape
    E, F = c["wr"].shape[1], c["w1"].shape[2]
    ins = {k: dev(c[k]) for k in ("fnorm", "fin", "wr", "w1", "w3", "w2", "dout")}
    grads = [dev(c[k]) for k in ("gwr0", "gw10", "gw30", "gw20")]
    out = t.full((N, D), float("nan"), dtype=t.float32, device="cuda")
    assign = t.full((N,), -7, dtype=t.int32, device="cuda")
    gate = t.full((N,), float("nan"), dtype=t.float32, device="cuda")
    rprobs = t.full((N, E), float("nan"), dtype=t.float32, device="cuda")
    nb = lib.tlg_moe_keep_bytes(N, D, F, E)
    assert nb > 0
    keep = t.full((nb // 4,), float("nan"), dtype=t.float32, device="cuda")
    p = {k: v.data_ptr() for k, v in ins.items()}
    lib.moe_fwd_keep(p["fnorm"], p["fin"], out.data_ptr(), N, D, F, E, p["wr"], p["w1"], p["w3"], p["w2"],
                     assign.data_ptr(), gate.data_ptr(), rprobs.data_ptr(), keep.data_ptr(), nb, stream())
    if interleave:
        interleave()
    dfn = t.full((N, D), float("nan"), dtype=t.float32, device="cuda")
    g = [x.data_ptr() for x in grads]
    lib.moe_bwd_kept(p["fnorm"], p["dout"], dfn.data_ptr(), assign.data_ptr(), gate.data_ptr(), rprobs.data_ptr(),
                     N, D, F, E, p["wr"], p["w1"], p["w3"], p["w2"], g[0], g[1], g[2], g[3], keep.data_ptr(), nb,
                     stream())
    if finish == "free":
        assert lib.tlg_dev_gemm_pending() > 0, "the kept backward left nothing queued"
        other = lib.tlg_dev_malloc(256)
        lib.check(lib.tlg_dev_free(other), "tlg_dev_free")
        assert lib.tlg_dev_gemm_pending() == 0, "tlg_dev_free left reductions queued"
    lib.check(lib.tlg_dev_gemm_flush(stream()), "flush")      # dWr's deferred column sum
    fwd = (out.cpu().numpy(), assign.cpu().numpy(), gate.cpu().numpy(), rprobs.cpu().numpy())
    return fwd, dfn.cpu().numpy(), [x.cpu().numpy() for x in grads]


@pytest.mark.parametrize("N,D,F,E,skew,dead", [(4096, 256, 768, 4, 2.0, ()), (67, 32, 48, 3, 0.0, ()),
                                              (2500, 64, 96, 5, 1.0, (3,)), (513, 32, 64, 1, 0.0, ())])
def test_kept_state_pair_is_bit_identical(lib, N, D, F, E, skew, dead):
    """tlg_dev_moe_grouped_fwd_keep + _bwd_kept give the recomputing pair's
    results bit for bit, also when other MoE calls run between them, and when
    tlg_dev_free (not a flush) is what runs the reductions they leave queued."""
    print("kept pair", N, D, F, E, flush=True)
    c = case(N, D, F, E, zlib.crc32(f"kept {N} {D} {F} {E}".encode()), skew, dead)
    ref_f = gpu_forward(lib, c["fnorm"], c["fin"], c["wr"], c["w1"], c["w3"], c["w2"])
    g0 = [c[k] for k in ("gwr0", "gw10", "gw30", "gw20")]
    ref_b = gpu_backward(lib, c["fnorm"], c["dout"], ref_f[1], ref_f[2], ref_f[3], c["wr"], c["w1"], c["w3"],
                         c["w2"], *g0)
    other = case(300, 16, 32, 7, 5)

    def interleave():
        f = gpu_forward(lib, other["fnorm"], other["fin"], other["wr"], other["w1"], other["w3"], other["w2"])
        gpu_backward(lib, other["fnorm"], other["dout"], f[1], f[2], f[3], other["wr"], other["w1"], other["w3"],
                     other["w2"], *[other[k] for k in ("gwr0", "gw10", "gw30", "gw20")])

    for inter, finish in ((None, "flush"), (interleave, "flush"), (None, "free")):
        fwd, dfn, grads = gpu_pair_kept(lib, c, inter, finish)
        for x, y in zip(fwd, ref_f):
            assert np.array_equal(x, y)
        assert np.array_equal(dfn, ref_b[0])
        for x, y in zip(grads, ref_b[1]):
            assert np.array_equal(x, y)


@pytest.mark.parametrize("N,E,skew,dead", [(4096, 4, 2.0, ()), (1, 3, 0.0, ()), (67, 3, 0.0, ()),
                                          (2500, 5, 1.0, (3,)), (5000, 64, 0.0, ()), (513, 1, 0.0, ())])
def test_forward_index_is_a_stable_sort(lib, N, E, skew, dead):
    """The forward's expert index (the router's per-block counts and ranks,
    then the many-workgroup placement), read from the kept state: idx lists
    the tokens of expert 0, then 1, .. each in ascending order (moe_forward's
    per-expert gather, tinylm.c:876-879), pos inverts idx, eoff is the
    prefix of the per-expert counts; against numpy's stable argsort of the
    assignments the forward returned."""
    print("index", N, E, flush=True)
    t = _torch()
    D, F = 32, 16
    c = case(N, D, F, E, zlib.crc32(f"index {N} {E}".encode()), skew, dead)
    ins = {k: dev(c[k]) for k in ("fnorm", "fin", "wr", "w1", "w3", "w2")}
    out = t.full((N, D), float("nan"), dtype=t.float32, device="cuda")
    assign = t.full((N,), -7, dtype=t.int32, device="cuda")
    gate = t.full((N,), float("nan"), dtype=t.float32, device="cuda")
    rprobs = t.full((N, E), float("nan"), dtype=t.float32, device="cuda")
    nb = lib.tlg_moe_keep_bytes(N, D, F, E)
    keep = t.full((nb // 4,), -9, dtype=t.int32, device="cuda")
    p = {k: v.data_ptr() for k, v in ins.items()}
    lib.moe_fwd_keep(p["fnorm"], p["fin"], out.data_ptr(), N, D, F, E, p["wr"], p["w1"], p["w3"], p["w2"],
                     assign.data_ptr(), gate.data_ptr(), rprobs.data_ptr(), keep.data_ptr(), nb, stream())
    k = keep.cpu().numpy()
    al = lambda x: (x + 255) // 256 * 256 // 4          # the kept layout's 256-byte slots, in ints
    idx, pos, eoff = k[:N], k[al(4 * N):al(4 * N) + N], k[2 * al(4 * N):2 * al(4 * N) + E + 1]
    a = assign.cpu().numpy()
    assert a.min() >= 0 and a.max() < E
    want = np.argsort(a, kind="stable")
    assert np.array_equal(idx, want)
    assert np.array_equal(pos[want], np.arange(N))
    assert np.array_equal(eoff, np.concatenate([[0], np.cumsum(np.bincount(a, minlength=E))]))
    for e in dead:
        assert eoff[e + 1] == eoff[e]


def test_kept_state_size_checked(lib):
    import tlgemm
    t = _torch()
    N, D, F, E = 64, 16, 32, 4
    nb = lib.tlg_moe_keep_bytes(N, D, F, E)
    assert nb >= 4 * N * (3 * F + D) and lib.tlg_moe_keep_bytes(N, D, F, 65) == 0
    buf = t.zeros(1 << 16, dtype=t.float32, device="cuda")
    p = buf.data_ptr()
    ip = t.zeros(N, dtype=t.int32, device="cuda").data_ptr()
    with pytest.raises(tlgemm.TlgError):
        lib.moe_fwd_keep(p, p, p, N, D, F, E, p, p, p, p, ip, p, p, p, nb - 16, stream())
    with pytest.raises(tlgemm.TlgError):
        lib.moe_bwd_kept(p, p, p, ip, p, p, N, D, F, E, p, p, p, p, p, p, p, p, p, nb - 16, stream())


def test_bad_shapes_rejected(lib):
    import tlgemm
    t = _torch()
    buf = t.zeros(1 << 16, dtype=t.float32, device="cuda")
    p = buf.data_ptr()
    ip = t.zeros(64, dtype=t.int32, device="cuda").data_ptr()
    with pytest.raises(tlgemm.TlgError):          # D not a multiple of 4
        lib.moe_fwd(p, p, p, 8, 6, 8, 4, p, p, p, p, ip, p, p, stream())
    with pytest.raises(tlgemm.TlgError):          # more experts than the router supports
        lib.moe_fwd(p, p, p, 8, 8, 8, 65, p, p, p, p, ip, p, p, stream())
    # N = 0 is a no-op
    lib.moe_fwd(p, p, p, 0, 8, 8, 4, p, p, p, p, ip, p, p, stream())
