#!/usr/bin/env python3
"""Write the golden fixtures of the GEMM hot path from the reference's own code.

Run in the build container only (needs /root/reference):

    make -C oracle ref && python tests/golden/make_golden.py

It loads oracle/_ref/libtlref.so -- mm / mm_bt / mm_atb, the RNG and the MoE
layer of /root/reference/tinylm.c compiled from their own lines by
oracle/Makefile -- draws every input with the reference's rnd_normal
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
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
