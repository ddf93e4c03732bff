"""CPU pinning of the oracle's training-step restatement (oracle/tl_oracle_step.c).

Each function is held against (a) the golden fixtures the reference's own
compiled code wrote (tests/golden/step_*.npz, tests/golden/make_golden.py),
(b) an independent float64 model written here with torch autograd (so the
backward formulas are checked by differentiation, not by retyping them), and
(c) closed forms: RoPE is a rotation (norms kept, back undoes fwd), softmax
rows of dlogits sum to zero, a one-key attention returns v, and uniform
logits give a loss of log V.  Where oracle/_ref is built, the oracle's whole
step is also compared with the reference's on fresh inputs.
"""
import os

import numpy as np
import pytest

from conftest import golden, load_npz
from oracle import SEQ_LIB, StepFns, model, normwise_rel, param_regions

TOL = 1e-4          # the north_star bar (normwise, tinylm.c:4782-4784)
FIX = 2e-6          # oracle vs the reference's own fp32 arithmetic


@pytest.fixture(scope="module")
def st():
    return StepFns("oracle")


def torch64():
    import torch
    return torch


# ---------------------------------------------------------------- fixtures --
def test_rmsnorm_matches_reference_fixture(st):
    d = load_npz(golden("step_rmsnorm.npz")[0])
    out, rinv = st.rmsnorm_fwd(d["x"], d["g"])
    assert normwise_rel(out, d["out"]) <= FIX and normwise_rel(rinv, d["rinv"]) <= FIX
    dx, dg = d["dx0"].copy(), d["dg0"].copy()
    st.rmsnorm_bwd(d["x"], d["g"], d["rinv"], d["dy"], dx, dg)
    assert normwise_rel(dx, d["dx"]) <= FIX
    assert normwise_rel(dg - d["dg0"], d["dg"] - d["dg0"]) <= 1e-5


def test_rope_matches_reference_fixture(st):
    d = load_npz(golden("step_rope.npz")[0])
    cs, sn = st.rope_table(64, 32)
    assert np.array_equal(cs, d["cs"]) and np.array_equal(sn, d["sn"])
    for back, key in ((0, "fwd"), (1, "back")):
        b = d["buf"].copy()
        st.rope(b, int(d["T"]), int(d["nh"]), int(d["hd"]), back)
        assert normwise_rel(b, d[key]) <= FIX, key


@pytest.mark.parametrize("path", golden("step_attn_*.npz"), ids=os.path.basename)
def test_attention_matches_reference_fixture(st, path):
    d = load_npz(path)
    a = [int(d[k]) for k in ("B", "T", "H", "KV", "hd", "win")]
    out = st.attn_fwd(d["q"], d["k"], d["v"], *a)
    assert normwise_rel(out, d["out"]) <= FIX
    dq, dk, dv = st.attn_bwd(d["q"], d["k"], d["v"], d["datt"], *a)
    for got, key in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        assert normwise_rel(got, d[key]) <= 1e-5, key


def test_adamw_and_gradnorm_match_reference_fixture(st):
    d = load_npz(golden("step_adamw.npz")[0])
    assert abs(st.gradnorm(d["G"]) - float(d["gnorm"])) <= 1e-6 * float(d["gnorm"])
    P, M, V = d["P"].copy(), d["M"].copy(), d["V"].copy()
    st.adamw(P, d["G"], M, V, float(d["lr"]), float(d["b1"]), float(d["b2"]), float(d["wd"]), int(d["t"]),
             float(d["gscale"]))
    for got, key in ((P, "P1"), (M, "M1"), (V, "V1")):
        assert normwise_rel(got, d[key]) <= FIX, key


def fixture_model(d):
    V, D, L, H, KV, F, T, n_mtp, n_exp, win, fe = (int(x) for x in d["model"])
    return model(V=V, D=D, L=L, H=H, KV=KV, F=F, T=T, n_mtp=n_mtp, n_exp=n_exp, win=win, full_every=fe)


@pytest.mark.parametrize("path", golden("step_train_*.npz"), ids=os.path.basename)
def test_train_step_matches_reference_fixture(st, path):
    d = load_npz(path)
    m = fixture_model(d)
    P = st.init_params(m, 1234567891011 + {"dense_mtp1": 11, "window": 12, "moe_e4": 13}[
        os.path.basename(path)[len("step_train_"):-4]])
    assert np.array_equal(P, d["P"]), "init_params differs from the reference's"
    loss, G = st.train_step(m, int(d["B"]), d["P"], d["tok"], d["tgt"], d["tgt_mtp"])
    assert abs(loss - float(d["loss"])) <= 1e-6 * abs(float(d["loss"]))
    for name, a, b in param_regions(st, m):
        assert normwise_rel(G[a:b], d["G"][a:b]) <= 1e-5, name


# -------------------------------------------------- float64 autograd model --
def torch_step(m, B, P, tok, tgt, tgt_mtp, st):
    """forward loss (with the MTP heads' weighted losses, whose gradients
    mtp_grad adds) of a dense model, in float64 with torch autograd."""
    torch = torch64()
    D, H, KV, F, T, V = m.D, m.H, m.KV, m.F, m.T, m.V
    hd = D // H
    KD = KV * hd
    N = B * T
    Pt = torch.tensor(P.astype(np.float64), requires_grad=True)

    def W(off, r, c):
        return Pt[off:off + r * c].view(r, c)

    def rms(x, g):
        return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + 1e-5) * g

    pos = torch.arange(N) % T
    inv = torch.tensor([10000.0 ** (-(2.0 * i) / hd) for i in range(hd // 2)], dtype=torch.float64)
    ang = pos[:, None].double() * inv[None, :]
    cos, sin = torch.cos(ang), torch.sin(ang)

    def rope(x, nh):
        x = x.view(N, nh, hd)
        a, b = x[..., :hd // 2], x[..., hd // 2:]
        c, s = cos[:, None, :], sin[:, None, :]
        return torch.cat([a * c - b * s, b * c + a * s], -1).view(N, nh * hd)

    def attn(q, k, v, win):
        q = q.view(B, T, H, hd).transpose(1, 2)
        k = k.view(B, T, KV, hd).transpose(1, 2).repeat_interleave(H // KV, 1)
        v = v.view(B, T, KV, hd).transpose(1, 2).repeat_interleave(H // KV, 1)
        s = q @ k.transpose(-1, -2) / np.sqrt(hd)
        t = torch.arange(T)
        mask = t[None, :] <= t[:, None]
        if win > 0:
            mask = mask & (t[None, :] > t[:, None] - win)
        s = s.masked_fill(~mask, float("-inf"))
        return (torch.softmax(s, -1) @ v).transpose(1, 2).reshape(N, D)

    x = W(0, V, D)[torch.tensor(tok.astype(np.int64))]
    for l in range(m.L):
        w = st.layer_map(m, l)
        win = 0 if m.win <= 0 or (m.full_every > 0 and (l + 1) % m.full_every == 0) else m.win
        a = rms(x, Pt[w["an1"]:w["an1"] + D])
        q, k, v = a @ W(w["wq"], D, D), a @ W(w["wk"], D, KD), a @ W(w["wv"], D, KD)
        f = x + attn(rope(q, H), rope(k, KV), v, win) @ W(w["wo"], D, D)
        fn = rms(f, Pt[w["an2"]:w["an2"] + D])
        g, u = fn @ W(w["w1"], D, F), fn @ W(w["w3"], D, F)
        x = f + (torch.nn.functional.silu(g) * u) @ W(w["w2"], F, D)
    w = st.layer_map(m, 0)
    fn = rms(x, Pt[w["nf"]:w["nf"] + D])
    E = W(0, V, D)
    ce = torch.nn.functional.cross_entropy
    loss = ce(fn @ E.T, torch.tensor(tgt.astype(np.int64)))
    total = loss
    for h in range(m.n_mtp):
        hk = fn + torch.nn.functional.silu(fn @ W(w["mtp0"] + h * D * D, D, D))
        wk = 0.2 * 0.8 ** h
        total = total + wk * ce(hk @ E.T, torch.tensor(tgt_mtp[h].astype(np.int64)))
    total.backward()
    return float(loss.detach()), Pt.grad.numpy()


@pytest.mark.parametrize("name", ["dense_mtp1", "window"])
def test_train_step_matches_float64_autograd(st, name):
    """The oracle's hand-written backward equals the derivative of its
    forward: every parameter tensor's gradient within the bar of float64
    autograd on a model written independently here."""
    pytest.importorskip("torch")
    d = load_npz(golden(f"step_train_{name}.npz")[0])
    m = fixture_model(d)
    B = int(d["B"])
    loss, G = st.train_step(m, B, d["P"], d["tok"], d["tgt"], d["tgt_mtp"])
    loss64, G64 = torch_step(m, B, d["P"], d["tok"], d["tgt"], d["tgt_mtp"], st)
    assert abs(loss - loss64) <= 1e-5 * loss64
    for tname, a, b in param_regions(st, m):
        assert normwise_rel(G[a:b], G64[a:b]) <= TOL, tname


# ------------------------------------------------------------ closed forms --
def test_rope_is_a_rotation(st):
    r = np.random.default_rng(3)
    x = r.standard_normal((50, 2 * 32)).astype(np.float32)
    y = x.copy()
    st.rope(y, 17, 2, 32, 0)
    pair = lambda a: np.hypot(a.reshape(50, 2, 2, 16)[:, :, 0], a.reshape(50, 2, 2, 16)[:, :, 1])  # noqa: E731
    assert np.allclose(pair(y), pair(x), rtol=1e-5, atol=1e-6)
    assert np.array_equal(y[0], x[0])                     # position 0: angle 0
    st.rope(y, 17, 2, 32, 1)
    assert np.allclose(y, x, rtol=1e-5, atol=1e-5)


def test_attention_closed_forms(st):
    r = np.random.default_rng(4)
    # one key per sequence: out = v
    q, k, v = (r.standard_normal((3, 64)).astype(np.float32) for _ in range(3))
    out = st.attn_fwd(q, k[:, :32].copy(), v[:, :32].copy(), 3, 1, 2, 1, 32)
    assert np.allclose(out.reshape(3, 2, 32), v[:, None, :32], rtol=1e-6, atol=1e-6)
    # zero queries: uniform weights -> running mean of v
    T = 9
    v = r.standard_normal((T, 32)).astype(np.float32)
    out = st.attn_fwd(np.zeros((T, 32), np.float32), r.standard_normal((T, 32)).astype(np.float32), v, 1, T, 1, 1,
                      32)
    assert np.allclose(out, np.cumsum(v, 0) / np.arange(1, T + 1)[:, None], rtol=1e-5, atol=1e-6)


def test_xent_closed_forms(st):
    import ctypes
    fp, ip = ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_int)
    N, V = 6, 50
    tgt = np.arange(N, dtype=np.int32) * 7 % V
    dl = np.empty((N, V), np.float32)
    lg = np.zeros((N, V), np.float32)
    loss = st._fn("xent")(lg.ctypes.data_as(fp), tgt.ctypes.data_as(ip), dl.ctypes.data_as(fp), 1.0 / N, N, V)
    assert abs(loss - np.log(V)) <= 1e-6
    assert np.allclose(dl.sum(1), 0.0, atol=1e-7)
    assert np.allclose(dl[np.arange(N), tgt], (1.0 / V - 1.0) / N, rtol=1e-5)


def test_embedding_gather_scatter(st):
    import ctypes
    r = np.random.default_rng(5)
    emb = r.standard_normal((10, 8)).astype(np.float32)
    tok = np.array([3, 1, 3, 9, 0, 3], np.int32)
    out = np.empty((6, 8), np.float32)
    fp, ip = ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_int)
    st._fn("embed_fwd")(out.ctypes.data_as(fp), emb.ctypes.data_as(fp), tok.ctypes.data_as(ip), 6, 8)
    assert np.array_equal(out, emb[tok])
    de = np.zeros_like(emb)
    st._fn("embed_bwd")(de.ctypes.data_as(fp), out.ctypes.data_as(fp), tok.ctypes.data_as(ip), 6, 8)
    want = np.zeros_like(emb)
    np.add.at(want, tok, out)
    assert np.allclose(de, want, rtol=1e-6)


# -------------------------------------------- against the reference itself --
@pytest.mark.skipif(not os.path.exists(SEQ_LIB), reason="oracle/_ref not built (needs /root/reference)")
def test_train_step_matches_reference_on_fresh_inputs(st):
    ref = StepFns("reference")
    m = model(V=128, D=96, L=2, H=3, KV=1, F=64, T=40, n_mtp=2)
    P = st.init_params(m, 99)
    assert np.array_equal(P, ref.init_params(m, 99))
    r = np.random.default_rng(9)
    B = 3
    N = B * m.T
    tok, tgt = (r.integers(0, m.V, N).astype(np.int32) for _ in range(2))
    tm = r.integers(0, m.V, (2, N)).astype(np.int32)
    l1, G1 = st.train_step(m, B, P, tok, tgt, tm)
    l2, G2 = ref.train_step(m, B, P, tok, tgt, tm)
    assert abs(l1 - l2) <= 1e-6 * l2
    for name, a, b in param_regions(st, m):
        assert normwise_rel(G1[a:b], G2[a:b]) <= 1e-5, name


# ------------------------------------------------------------------ decode --
def test_half_and_fast_expf_match_reference_fixture():
    from oracle import half_fns
    d = load_npz(golden("step_half_exp.npz")[0])
    f2h, h2f, fe = half_fns("oracle")
    assert np.array_equal(f2h(d["x"]), d["h"])
    assert np.array_equal(h2f(d["h"]), d["hx"])
    assert np.array_equal(fe(d["e_in"]), d["e_out"])
    # closed forms: f16 keeps 11 significant bits (relative step <= 2^-11
    # in the normal range); fast_expf is within 1e-4 of exp and exact at 0
    normal = (np.abs(d["x"]) > 6.2e-5) & (np.abs(d["x"]) < 65504)
    rel = np.abs(d["hx"][normal].astype(np.float64) - d["x"][normal]) / np.abs(d["x"][normal])
    assert rel.max() <= 2.0 ** -11
    ok = (d["e_in"] > -80) & (d["e_in"] <= 88)          # inside the clamp
    assert np.allclose(d["e_out"][ok], np.exp(d["e_in"][ok].astype(np.float64)), rtol=1e-4, atol=0)
    assert d["e_out"][d["e_in"] == 0.0][0] == 1.0


def test_decode_matches_reference_forward_fixture():
    """Decoding token by token through the ring cache (f32 cache, expf) gives
    the reference's own forward() logits; the f16 cache and fast_expf (the
    reference's decode defaults) move them by their rounding only."""
    from oracle import Decoder
    d = load_npz(golden("step_decode_forward.npz")[0])
    V, D, L, H, KV, F, T = (int(x) for x in d["model"])
    m = model(V=V, D=D, L=L, H=H, KV=KV, F=F, T=T)
    for kvdt, exact, bar in ((0, 1, 5e-6), (0, 0, 5e-4), (1, 1, 5e-3), (1, 0, 5e-3)):
        dec = Decoder(m, d["P"], T, kvdt=kvdt, exact=exact, maxpos=64)
        lg = np.concatenate([dec.chunk(d["tok"][i:i + 1], i) for i in range(T)])
        assert normwise_rel(lg, d["logits"]) <= bar, (kvdt, exact)
        dec2 = Decoder(m, d["P"], T, kvdt=kvdt, exact=exact, maxpos=64)
        chunks = np.concatenate([dec2.chunk(d["tok"][0:7], 0), dec2.chunk(d["tok"][7:15], 7),
                                 dec2.chunk(d["tok"][15:], 15)])
        assert np.array_equal(chunks, lg), "chunked prefill differs from token-by-token decode"


def test_decode_ring_closed_forms():
    """A ring of W slots equals an unbounded cache while positions < W, and
    with a window of w attends to exactly the last w positions: decoding with
    win = W' through a ring of W' slots equals a larger ring with win = W'."""
    from oracle import Decoder
    kw = dict(V=64, D=64, L=1, H=2, KV=1, F=32, T=16)
    m = model(**kw)
    P = StepFns("oracle").init_params(m, 9)
    tok = np.random.default_rng(1).integers(0, 64, 40).astype(np.int32)
    big = Decoder(m, P, 64, kvdt=0, exact=1, maxpos=64)
    ring = Decoder(m, P, 16, kvdt=0, exact=1, maxpos=64)
    a = np.concatenate([big.chunk(tok[i:i + 1], i) for i in range(16)])
    b = np.concatenate([ring.chunk(tok[i:i + 1], i) for i in range(16)])
    assert np.array_equal(a, b)
    mw = model(**dict(kw, win=16))
    big_w = Decoder(mw, P, 64, kvdt=0, exact=1, maxpos=64)
    ring2 = Decoder(m, P, 16, kvdt=0, exact=1, maxpos=64)
    a = np.concatenate([big_w.chunk(tok[i:i + 1], i) for i in range(40)])
    b = np.concatenate([ring2.chunk(tok[i:i + 1], i) for i in range(40)])
    assert np.array_equal(a, b)
