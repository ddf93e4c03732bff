#!/usr/bin/env python3
"""Write the golden fixtures of the GEMM hot path from the reference's own code.

Run in the build container only (needs /root/reference):

    make -C oracle ref && python tests/golden/make_golden.py

It loads oracle/_ref/libtlref.so -- mm / mm_bt / mm_atb, the RNG and the MoE
layer of /root/reference/tinylm.c compiled from their own lines by
oracle/Makefile -- and _ref/libtlref_seq.so (the training step's norms, RoPE,
attention, AdamW and whole forward + backward passes), draws every input with the reference's rnd_normal
(tinylm.c:127-134) and records inputs and outputs as .npz files next to this
script.  The fixtures are data (inputs and expected outputs); no reference
source is stored.  Tests check both the CPU oracle and the GPU path against
them.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "oracle"))
from oracle import Reference  # noqa: E402

# (name, M, K, N, scale of W): the selftest shape (tinylm.c:4755), decode rows
# M=1..8 at m8 widths, the N=E=4 router, ragged tiny shapes, KD=96, a long
# reduction for mm_atb and a 4-multiple square.
PRIM_CASES = [
    ("selftest_201x131x259", 201, 131, 259, 1.0),
    ("decode_m1_384x128", 1, 384, 128, 0.02),
    ("decode_m2_384x96", 2, 384, 96, 0.02),
    ("decode_m3_96x256", 3, 96, 256, 0.02),
    ("decode_m4_256x96", 4, 256, 96, 0.02),
    ("decode_m8_128x384", 8, 128, 384, 0.02),
    ("unembed_m2_2048x32", 2, 2048, 32, 0.02),
    ("router_67x96x4", 67, 96, 4, 0.02),
    ("tiny_1x1x1", 1, 1, 1, 1.0),
    ("tiny_3x5x7", 3, 5, 7, 1.0),
    ("tiny_7x13x5", 7, 13, 5, 1.0),
    ("tiny_9x3x17", 9, 3, 17, 1.0),
    ("kv96_33x384x96", 33, 384, 96, 0.02),
    ("longred_1024x32x48", 1024, 32, 48, 0.02),
    ("square_128x128x128", 128, 128, 128, 0.02),
]


def prim_case(ref, name, M, K, N, wscale, seed):
    ref.seed(seed)
    X = ref.normal((M, K))
    W = ref.normal((K, N), wscale)
    dY = ref.normal((M, N), 0.01 if wscale != 1.0 else 1.0)
    dX0 = ref.normal((M, K))          # non-zero prefills: accumulate semantics
    dW0 = ref.normal((K, N), wscale)
    Y = np.full((M, N), 12345.0, np.float32)   # garbage that `mm` must overwrite
    ref.mm(X, W, Y)
    dX = dX0.copy()
    ref.mm_bt(dX, dY, W)
    dW = dW0.copy()
    ref.mm_atb(dW, X, dY)
    np.savez(os.path.join(HERE, f"prim_{name}.npz"), M=M, K=K, N=N, seed=seed,
             X=X, W=W, dY=dY, Y=Y, dX0=dX0, dX=dX, dW0=dW0, dW=dW)


def chain_case(ref, seed):
    """dnorm <- dq Wq^T + dk Wk^T + dv Wv^T after a memset (tinylm.c:1134-1138)."""
    ref.seed(seed)
    R, D, KD = 64, 128, 32
    dq, dk, dv = ref.normal((R, D), 0.01), ref.normal((R, KD), 0.01), ref.normal((R, KD), 0.01)
    Wq, Wk, Wv = ref.normal((D, D), 0.02), ref.normal((D, KD), 0.02), ref.normal((D, KD), 0.02)
    out = np.zeros((R, D), np.float32)
    ref.mm_bt(out, dq, Wq)
    ref.mm_bt(out, dk, Wk)
    ref.mm_bt(out, dv, Wv)
    np.savez(os.path.join(HERE, "chain_dnorm.npz"), seed=seed, dq=dq, dk=dk, dv=dv,
             Wq=Wq, Wk=Wk, Wv=Wv, out=out)


def moe_case(ref, name, N, D, F, E, seed, tie=False):
    """One top-1 MoE layer forward + backward through the reference's
    moe_forward / moe_backward (tinylm.c:857-947)."""
    ref.seed(seed)
    fnorm = ref.normal((N, D))
    fin = ref.normal((N, D))
    wr = ref.normal((D, E), 0.5)
    if tie:
        wr[:, 2] = wr[:, 1]              # experts 1 and 2 always tie: lowest index wins
    w1 = ref.normal((E, D, F), 0.02)
    w3 = ref.normal((E, D, F), 0.02)
    w2 = ref.normal((E, F, D), 0.02)
    dout = ref.normal((N, D), 0.01)
    out, assign, gate, rprobs = ref.moe_forward(fnorm, fin, wr, w1, w3, w2)
    gwr0 = ref.normal((D, E), 0.01)
    gw10 = ref.normal((E, D, F), 0.01)
    gw30 = ref.normal((E, D, F), 0.01)
    gw20 = ref.normal((E, F, D), 0.01)
    gwr, gw1, gw3, gw2 = gwr0.copy(), gw10.copy(), gw30.copy(), gw20.copy()
    dfn = ref.moe_backward(fnorm, dout, wr, w1, w3, w2, gwr, gw1, gw3, gw2, assign, gate, rprobs)
    np.savez(os.path.join(HERE, f"moe_{name}.npz"), N=N, D=D, F=F, E=E, seed=seed,
             fnorm=fnorm, fin=fin, wr=wr, w1=w1, w3=w3, w2=w2, dout=dout,
             out=out, assign=assign, gate=gate, rprobs=rprobs,
             gwr0=gwr0, gw10=gw10, gw30=gw30, gw20=gw20,
             gwr=gwr, gw1=gw1, gw3=gw3, gw2=gw2, dfn=dfn)


def rng_case(ref, seed):
    """The first draws of rnd_normal from a seed, plus the raw xorshift state."""
    ref.seed(seed)
    z = ref.normal((4096,))
    np.savez(os.path.join(HERE, "rng_normal.npz"), seed=seed, z=z)


def seq_case(name, B, T, D, H, KV, F, V, L, n_mtp):
    """GEMM call list of the reference's own forward + backward (compiled from
    tinylm.c:539-1154 with logged call sites, oracle/Makefile)."""
    import json
    from oracle import reference_train_log
    log = reference_train_log(B, T, D, H, KV, F, V, L, n_mtp)
    json.dump({"B": B, "T": T, "D": D, "H": H, "KV": KV, "F": F, "V": V, "L": L, "n_mtp": n_mtp,
               "calls": [[op, list(o), list(a), list(b), M, K, N] for op, o, a, b, M, K, N in log]},
              open(os.path.join(HERE, f"seq_{name}.json"), "w"))


def step_cases(ref):
    """The training step's non-GEMM functions and whole steps, through the
    reference's own code (oracle/_ref/libtlref_seq.so: tinylm.c:539-1176
    compiled from its lines): rmsnorm, RoPE, attention, AdamW / gradnorm,
    and forward + backward of three small models."""
    from oracle import StepFns, model
    st = StepFns("reference")
    rng = np.random.default_rng(77)
    f32 = lambda *s, sc=1.0: (sc * rng.standard_normal(s)).astype(np.float32)  # noqa: E731

    # rmsnorm forward / backward with non-zero dx and dg prefills
    x, g = f32(37, 48), (1.0 + f32(48, sc=0.1)).astype(np.float32)
    out, rinv = st.rmsnorm_fwd(x, g)
    dy, dx0, dg0 = f32(37, 48, sc=0.01), f32(37, 48, sc=0.01), f32(48, sc=0.01)
    dx, dg = dx0.copy(), dg0.copy()
    st.rmsnorm_bwd(x, g, rinv, dy, dx, dg)
    np.savez(os.path.join(HERE, "step_rmsnorm.npz"), x=x, g=g, out=out, rinv=rinv, dy=dy, dx0=dx0, dx=dx,
             dg0=dg0, dg=dg)

    # RoPE: rope_init's table and rope_apply both ways at positions r % T
    cs, sn = st.rope_table(64, 32)
    buf = f32(40, 3 * 32)
    fwd, back = buf.copy(), buf.copy()
    st.rope(fwd, 16, 3, 32, 0)
    st.rope(back, 16, 3, 32, 1)
    np.savez(os.path.join(HERE, "step_rope.npz"), T=16, nh=3, hd=32, cs=cs, sn=sn, buf=buf, fwd=fwd, back=back)

    # attention forward / backward (GQA; one ragged sequence with a window)
    for name, B, T, H, KV, win in (("gqa_b2_t40_h4_kv2", 2, 40, 4, 2, 0), ("win_b1_t70_h2_kv1", 1, 70, 2, 1, 24)):
        hd = 32
        q, k, v = f32(B * T, H * hd), f32(B * T, KV * hd), f32(B * T, KV * hd)
        out = st.attn_fwd(q, k, v, B, T, H, KV, hd, win)
        datt = f32(B * T, H * hd, sc=0.01)
        dq, dk, dv = st.attn_bwd(q, k, v, datt, B, T, H, KV, hd, win)
        np.savez(os.path.join(HERE, f"step_attn_{name}.npz"), B=B, T=T, H=H, KV=KV, hd=hd, win=win, q=q, k=k,
                 v=v, out=out, datt=datt, dq=dq, dk=dk, dv=dv)

    # AdamW step t = 3 with a clip scale, and the gradient norm
    n = 1000
    P, G, M, V = f32(n, sc=0.02), f32(n, sc=0.01), f32(n, sc=0.001), np.abs(f32(n, sc=1e-5))
    gn = st.gradnorm(G)
    P1, M1, V1 = P.copy(), M.copy(), V.copy()
    st.adamw(P1, G, M1, V1, 3e-4, 0.9, 0.95, 0.1, 3, 0.5)
    np.savez(os.path.join(HERE, "step_adamw.npz"), P=P, G=G, M=M, V=V, gnorm=np.float32(gn), lr=3e-4, b1=0.9,
             b2=0.95, wd=0.1, t=3, gscale=0.5, P1=P1, M1=M1, V1=V1)

    # whole steps: forward + memset(G) + backward (train_loop, :2627-2629)
    for name, kw, B, seed in (
            ("dense_mtp1", dict(V=64, D=64, L=2, H=2, KV=1, F=48, T=32, n_mtp=1), 2, 11),
            ("window", dict(V=96, D=64, L=2, H=2, KV=2, F=32, T=48, win=20, full_every=2), 1, 12),
            ("moe_e4", dict(V=64, D=64, L=1, H=2, KV=1, F=48, T=32, n_exp=4), 2, 13)):
        m = model(**kw)
        P = st.init_params(m, 1234567891011 + seed)
        N = B * m.T
        tok = rng.integers(0, m.V, N).astype(np.int32)
        tgt = rng.integers(0, m.V, N).astype(np.int32)
        tm = rng.integers(0, m.V, (max(m.n_mtp, 1), N)).astype(np.int32)
        loss, G = st.train_step(m, B, P, tok, tgt, tm)
        np.savez(os.path.join(HERE, f"step_train_{name}.npz"), B=B, model=np.array(
            [m.V, m.D, m.L, m.H, m.KV, m.F, m.T, m.n_mtp, m.n_exp, m.win, m.full_every], np.int32),
            P=P, tok=tok, tgt=tgt, tgt_mtp=tm, loss=np.float32(loss), G=G)


def decode_cases():
    """The decode path's pins: the reference's forward() logits of a small
    model (a token-by-token decode with an f32 cache and expf must give
    them), and its f2h / h2f / fast_expf on a spread of inputs."""
    from oracle import StepFns, half_fns, model, ref_forward_logits
    st = StepFns("reference")
    m = model(V=96, D=64, L=2, H=2, KV=1, F=48, T=40)
    P = st.init_params(m, 5)
    P[m.V * m.D:] += (0.05 * np.random.default_rng(1).standard_normal(P.size - m.V * m.D)).astype(np.float32)
    tok = np.random.default_rng(2).integers(0, m.V, m.T).astype(np.int32)
    logits = ref_forward_logits(m, 1, P, tok)
    np.savez(os.path.join(HERE, "step_decode_forward.npz"), model=np.array(
        [m.V, m.D, m.L, m.H, m.KV, m.F, m.T], np.int32), P=P, tok=tok, logits=logits)
    f2h, h2f, fe = half_fns("reference")
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(3000) * 10, rng.standard_normal(1000) * 1e-5,
                        [0.0, -0.0, 65504.0, 65520.0, 1e6, -1e6, 6e-8, 3e-8, 2.98e-8]]).astype(np.float32)
    h = f2h(x)
    e_in = np.concatenate([-np.abs(rng.standard_normal(3000) * 8), [-100.0, -87.0, 0.0, 1.0, 88.0, 100.0]])
    e_in = e_in.astype(np.float32)
    np.savez(os.path.join(HERE, "step_half_exp.npz"), x=x, h=h, hx=h2f(h), e_in=e_in, e_out=fe(e_in))


def main():
    if not os.path.isdir("/root/reference"):
        sys.exit("make_golden.py needs /root/reference (build container only)")
    ref = Reference()
    ref.set_threads(4)
    for i, (name, M, K, N, ws) in enumerate(PRIM_CASES):
        prim_case(ref, name, M, K, N, ws, 1000 + i)
    chain_case(ref, 2024)
    moe_case(ref, "n96_d32_f48_e4", 96, 32, 48, 4, 31337)
    moe_case(ref, "tie_n64_d16_f24_e4", 64, 16, 24, 4, 4242, tie=True)
    rng_case(ref, 1234567891011)
    seq_case("train_l2_mtp2", 2, 16, 32, 4, 1, 48, 64, 2, 2)
    seq_case("train_l3", 1, 24, 48, 6, 2, 40, 96, 3, 0)
    step_cases(ref)
    decode_cases()
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
