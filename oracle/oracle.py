"""numpy front end of the CPU oracle (liboracle.so) and of the compiled
reference (_ref/libtlref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, always as the checker or the CPU baseline,
never as a product path.
"""
import ctypes
import os
import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libtlref.so")

_fp = ctypes.POINTER(ctypes.c_float)
_ip = ctypes.POINTER(ctypes.c_int)
_i = ctypes.c_int


def _f(a):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_fp)


def _n(a):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(_ip)


class _Prims:
    """mm / mm_bt / mm_atb on numpy arrays with the reference's semantics."""

    prefix = ""

    def mm(self, X, W, Y=None):
        M, K = X.shape
        N = W.shape[1]
        if Y is None:
            Y = np.empty((M, N), np.float32)
        getattr(self.dll, self.prefix + "mm")(_f(Y), _f(X), _f(W), M, K, N)
        return Y

    def mm_bt(self, dX, dY, W):
        """dX += dY @ W.T in place (W is [K][N])."""
        M, N = dY.shape
        K = W.shape[0]
        getattr(self.dll, self.prefix + "mm_bt")(_f(dX), _f(dY), _f(W), M, K, N)
        return dX

    def mm_atb(self, dW, X, dY):
        """dW += X.T @ dY in place."""
        M, K = X.shape
        N = dY.shape[1]
        getattr(self.dll, self.prefix + "mm_atb")(_f(dW), _f(X), _f(dY), M, K, N)
        return dW


class Oracle(_Prims):
    prefix = "orc_"

    def __init__(self, path=LIB):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run make -C oracle")
        d = ctypes.CDLL(path)
        for n in ("orc_mm", "orc_mm_bt", "orc_mm_atb", "orc_mm_f64", "orc_mm_bt_f64", "orc_mm_atb_f64"):
            getattr(d, n).argtypes = [_fp, _fp, _fp, _i, _i, _i]
            getattr(d, n).restype = None
        d.orc_rnd_normal.restype = ctypes.c_float
        d.orc_xorshift.restype = ctypes.c_uint64
        d.orc_rng_seed.argtypes = [ctypes.c_uint64]
        d.orc_rng_state.restype = ctypes.c_uint64
        d.orc_fill_normal.argtypes = [_fp, ctypes.c_size_t, ctypes.c_float]
        d.orc_set_pool.argtypes = [_i]
        d.orc_set_gemv_split.argtypes = [_i]
        d.orc_set_threads.argtypes = [_i]
        d.orc_threads.restype = _i
        d.orc_moe_forward.argtypes = [_i, _i, _i, _i, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _ip, _fp, _fp]
        d.orc_moe_backward.argtypes = [_i, _i, _i, _i, _fp, _fp, _fp, _fp, _fp, _fp, _fp,
                                       _fp, _fp, _fp, _fp, _ip, _fp, _fp]
        d.orc_run_calls.argtypes = [ctypes.c_void_p, _i, _i]
        d.orc_run_calls.restype = None
        self.dll = d

    def run_calls(self, arr, reps=1):
        """Run plan_calls_native(...) `reps` times in C."""
        self.dll.orc_run_calls(ctypes.cast(arr, ctypes.c_void_p), len(arr), reps)

    # fp64 textbook references (accumulating forms add into the prefill)
    def mm_f64(self, X, W):
        M, K = X.shape
        N = W.shape[1]
        Y = np.empty((M, N), np.float32)
        self.dll.orc_mm_f64(_f(Y), _f(X), _f(W), M, K, N)
        return Y

    def mm_bt_f64(self, dX, dY, W):
        M, N = dY.shape
        self.dll.orc_mm_bt_f64(_f(dX), _f(dY), _f(W), M, W.shape[0], N)
        return dX

    def mm_atb_f64(self, dW, X, dY):
        M, K = X.shape
        self.dll.orc_mm_atb_f64(_f(dW), _f(X), _f(dY), M, K, dY.shape[1])
        return dW

    def seed(self, s):
        self.dll.orc_rng_seed(s)

    def normal(self, shape, scale=1.0):
        a = np.empty(shape, np.float32)
        self.dll.orc_fill_normal(_f(a), a.size, scale)
        return a

    def set_threads(self, n):
        self.dll.orc_set_threads(n)

    def threads(self):
        return self.dll.orc_threads()

    def set_pool(self, n):
        self.dll.orc_set_pool(n)

    def moe_forward(self, fnorm, fin, wr, w1, w3, w2):
        N, D = fnorm.shape
        E = wr.shape[1]
        F = w1.shape[2]
        out = np.empty((N, D), np.float32)
        assign = np.empty(N, np.int32)
        gate = np.empty(N, np.float32)
        rprobs = np.empty((N, E), np.float32)
        self.dll.orc_moe_forward(N, D, F, E, _f(fnorm), _f(fin), _f(out), _f(wr), _f(w1), _f(w3),
                                 _f(w2), _n(assign), _f(gate), _f(rprobs))
        return out, assign, gate, rprobs

    def moe_backward(self, fnorm, dout, wr, w1, w3, w2, gwr, gw1, gw3, gw2, assign, gate, rprobs):
        N, D = fnorm.shape
        E = wr.shape[1]
        F = w1.shape[2]
        dfn = np.empty((N, D), np.float32)
        self.dll.orc_moe_backward(N, D, F, E, _f(fnorm), _f(dout), _f(dfn), _f(wr), _f(w1), _f(w3),
                                  _f(w2), _f(gwr), _f(gw1), _f(gw3), _f(gw2), _n(assign), _f(gate),
                                  _f(rprobs))
        return dfn


class Reference(_Prims):
    """The reference's own kernels (built by `make -C oracle ref` from
    /root/reference/tinylm.c; present only where that tree was)."""

    prefix = "tlref_"

    def __init__(self, path=REF_LIB):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        d = ctypes.CDLL(path)
        for n in ("tlref_mm", "tlref_mm_bt", "tlref_mm_atb"):
            getattr(d, n).argtypes = [_fp, _fp, _fp, _i, _i, _i]
            getattr(d, n).restype = None
        d.tlref_seed.argtypes = [ctypes.c_uint64]
        d.tlref_normal.restype = ctypes.c_float
        d.tlref_threads.argtypes = [_i]
        d.tlref_moe_forward.argtypes = [_i, _i, _i, _i, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _ip, _fp, _fp]
        d.tlref_moe_backward.argtypes = [_i, _i, _i, _i, _fp, _fp, _fp, _fp, _fp, _fp, _fp,
                                         _fp, _fp, _fp, _fp, _ip, _fp, _fp]
        self.dll = d

    def seed(self, s):
        self.dll.tlref_seed(s)

    def normal(self, shape, scale=1.0):
        a = np.empty(shape, np.float32)
        flat = a.reshape(-1)
        for i in range(flat.size):
            flat[i] = scale * self.dll.tlref_normal()
        return a

    def set_threads(self, n):
        self.dll.tlref_threads(n)

    def run_calls(self, arr, reps=1):
        """Run plan_calls_native(...) `reps` times in C through the
        reference's own mm / mm_bt / mm_atb."""
        f = self.dll.tlref_run_calls
        f.argtypes = [ctypes.c_void_p, _i, _i]
        f.restype = None
        f(ctypes.cast(arr, ctypes.c_void_p), len(arr), reps)

    def moe_forward(self, fnorm, fin, wr, w1, w3, w2):
        N, D = fnorm.shape
        E = wr.shape[1]
        F = w1.shape[2]
        out = np.empty((N, D), np.float32)
        assign = np.empty(N, np.int32)
        gate = np.empty(N, np.float32)
        rprobs = np.empty((N, E), np.float32)
        self.dll.tlref_moe_forward(N, D, F, E, _f(fnorm), _f(fin), _f(out), _f(wr), _f(w1), _f(w3),
                                   _f(w2), _n(assign), _f(gate), _f(rprobs))
        return out, assign, gate, rprobs

    def moe_backward(self, fnorm, dout, wr, w1, w3, w2, gwr, gw1, gw3, gw2, assign, gate, rprobs):
        N, D = fnorm.shape
        E = wr.shape[1]
        F = w1.shape[2]
        dfn = np.empty((N, D), np.float32)
        self.dll.tlref_moe_backward(N, D, F, E, _f(fnorm), _f(dout), _f(dfn), _f(wr), _f(w1),
                                    _f(w3), _f(w2), _f(gwr), _f(gw1), _f(gw3), _f(gw2), _n(assign),
                                    _f(gate), _f(rprobs))
        return dfn


def normwise_rel(got, ref):
    """max|got - ref| / mean|ref|: the reference selftest's metric
    (tinylm.c:4782-4784)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    if ref.size == 0:
        return 0.0
    den = np.abs(ref).mean()
    num = np.abs(got - ref).max()
    if den == 0.0:
        return float(num)
    return float(num / den)


def reference_train_log(B, T, D, H, KV, F, V, L, n_mtp, path=os.path.join(HERE, "_ref", "libtlref_seq.so")):
    """GEMM call list of the reference's own forward + backward (tinylm.c:968-1154),
    from _ref/libtlref_seq.so: list of (op, (out, off), (a, off), (b, off), M, K, N)
    with buffers named after tinylm.c's P / G / Acts fields."""
    d = ctypes.CDLL(path)
    d.tlref_train_log.argtypes = [_i] * 9 + [ctypes.POINTER(ctypes.c_longlong), _i]
    d.tlref_train_log.restype = _i
    d.tlref_seq_name.argtypes = [_i]
    d.tlref_seq_name.restype = ctypes.c_char_p
    cap = 4096
    buf = (ctypes.c_longlong * (10 * cap))()
    n = d.tlref_train_log(B, T, D, H, KV, F, V, L, n_mtp, buf, cap)
    ops = {0: "mm", 1: "mm_bt", 2: "mm_atb"}
    name = lambda i: d.tlref_seq_name(int(i)).decode()  # noqa: E731
    out = []
    for i in range(n):
        o = buf[10 * i:10 * i + 10]
        out.append((ops[o[0]], (name(o[1]), o[2]), (name(o[3]), o[4]), (name(o[5]), o[6]), o[7], o[8], o[9]))
    return out


def run_plan_cpu(plan, arrays, prims):
    """Execute a plan's calls (tlgemm.Plan.calls) on the CPU.

    `arrays` maps buffer name -> flat float32 numpy array; `prims` is an
    Oracle (the restatement) or a Reference (the reference's own kernels).
    Each call gets row-major views at the plan's offsets, exactly the
    operands the device executor hands the HIP kernels."""
    names = [b[0] for b in plan.bufs]

    def view(name, off, rows, cols):
        return arrays[name][off:off + rows * cols].reshape(rows, cols)

    for c in plan.calls:
        out = names[c["out"]]
        if c["op"] == "zero":
            arrays[out][c["out_off"]:c["out_off"] + c["n"]] = 0.0
            continue
        M, K, N = c["M"], c["K"], c["N"]
        a, b = names[c["a"]], names[c["b"]]
        if c["op"] == "mm":
            prims.mm(view(a, c["a_off"], M, K), view(b, c["b_off"], K, N), view(out, c["out_off"], M, N))
        elif c["op"] == "mm_bt":
            prims.mm_bt(view(out, c["out_off"], M, K), view(a, c["a_off"], M, N), view(b, c["b_off"], K, N))
        else:
            prims.mm_atb(view(out, c["out_off"], K, N), view(a, c["a_off"], M, K), view(b, c["b_off"], M, N))


class _Call(ctypes.Structure):
    """OrcCall / TlrefCall: one call of a plan for the C loop runners."""
    _fields_ = [("op", ctypes.c_int), ("out", ctypes.c_void_p), ("a", ctypes.c_void_p), ("b", ctypes.c_void_p),
                ("M", ctypes.c_int), ("K", ctypes.c_int), ("N", ctypes.c_int), ("n", ctypes.c_size_t)]


def plan_calls_native(plan, arrays):
    """The plan's calls as a C array of (op, pointers into `arrays`, dims),
    for prims.run_calls: the same operands run_plan_cpu passes."""
    names = [b[0] for b in plan.bufs]
    ops = {"mm": 0, "mm_bt": 1, "mm_atb": 2, "zero": 3}
    arr = (_Call * len(plan.calls))()

    def ptr(name, off):
        a = arrays[name]
        return a.ctypes.data + 4 * off

    for i, c in enumerate(plan.calls):
        d = arr[i]
        d.op = ops[c["op"]]
        d.out = ptr(names[c["out"]], c["out_off"])
        if c["op"] != "zero":
            d.a = ptr(names[c["a"]], c["a_off"])
            d.b = ptr(names[c["b"]], c["b_off"])
        d.M, d.K, d.N, d.n = c["M"], c["K"], c["N"], c["n"]
    return arr


class F64Prims:
    """mm / mm_bt / mm_atb with the fp64 textbook sums (orc_*_f64), usable by
    run_plan_cpu to execute a whole plan in double precision."""

    def __init__(self, orc):
        self.o = orc

    def mm(self, X, W, Y):
        M, K = X.shape
        self.o.dll.orc_mm_f64(_f(Y), _f(X), _f(W), M, K, W.shape[1])
        return Y

    def mm_bt(self, dX, dY, W):
        return self.o.mm_bt_f64(dX, dY, W)

    def mm_atb(self, dW, X, dY):
        return self.o.mm_atb_f64(dW, X, dY)


# ---- training-step glue (tl_oracle_step.c / the reference's own functions) ----
SEQ_LIB = os.path.join(HERE, "_ref", "libtlref_seq.so")
_sz = ctypes.c_size_t
_fl = ctypes.c_float


class OrcModel(ctypes.Structure):
    """tl_oracle.h OrcModel: the model shape (tinylm.c Cfg without shared
    experts)."""
    _fields_ = [(n, ctypes.c_int) for n in ("V", "D", "L", "H", "KV", "F", "T", "n_mtp", "n_exp", "win",
                                            "full_every")] + [("rope_base", ctypes.c_float),
                                                              ("qknorm", ctypes.c_int)]


def model(V, D, L, H, KV, F, T, n_mtp=0, n_exp=0, win=0, full_every=0, rope_base=10000.0, qknorm=0):
    return OrcModel(V, D, L, H, KV, F, T, n_mtp, n_exp, win, full_every, rope_base, qknorm)


class OrcLayerMap(ctypes.Structure):
    _fields_ = [(n, ctypes.c_size_t) for n in ("emb", "an1", "wq", "wk", "wv", "wo", "qn", "kn", "an2", "wr",
                                               "w1", "w3", "w2", "nf", "mtp0", "total")]


class StepFns:
    """The step's non-GEMM functions and a whole forward + backward step,
    either from the oracle's restatement (which="oracle", liboracle.so) or
    from the reference's own compiled code (which="reference",
    _ref/libtlref_seq.so).  Same methods and semantics for both, so a test
    can hold one against the other."""

    def __init__(self, which="oracle"):
        self.ref = which == "reference"
        path = SEQ_LIB if self.ref else LIB
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        d = ctypes.CDLL(path)
        p = "tlref_" if self.ref else "orc_"
        self.p, self.dll = p, d
        sig = {
            "rmsnorm_fwd": (None, [_fp, _fp, _fp, _fp, _i, _i]),
            "rmsnorm_bwd": (None, [_fp, _fp, _fp, _fp, _fp, _fp, _i, _i]),
            "attn_fwd": (None, [_fp, _fp, _fp, _fp, _i, _i, _i, _i, _i, _i]),
            "attn_bwd": (None, [_fp, _fp, _fp, _fp, _fp, _fp, _fp, _i, _i, _i, _i, _i, _i]),
            "adamw": (None, [_fp, _fp, _fp, _fp, _sz, _fl, _fl, _fl, _fl, _i, _fl]),
            "gradnorm": (_fl, [_fp, _sz]),
        }
        if self.ref:
            sig.update({
                "rope_table": (None, [_fp, _fp, _i, _i]),
                "rope": (None, [_fp, _ip, _i, _i, _i, _i, _i]),
                "param_count": (_sz, [_i] * 9),
                "init_params": (None, [_fp, ctypes.c_ulonglong] + [_i] * 9),
                "train_step": (_fl, [_fp, _fp, _ip, _ip, _ip] + [_i] * 12),
            })
        else:
            sig.update({
                "rope_table": (None, [_fp, _fp, _i, _i, _fl]),
                "rope": (None, [_fp, _ip, _i, _i, _i, _i, _fp, _fp, _i]),
                "param_map": (None, [ctypes.POINTER(OrcModel), _i, ctypes.POINTER(OrcLayerMap)]),
                "init_params": (None, [ctypes.POINTER(OrcModel), _fp, ctypes.c_uint64]),
                "train_step": (_fl, [ctypes.POINTER(OrcModel), _i, _fp, _fp, _ip, _ip, _ip]),
                "xent": (ctypes.c_double, [_fp, _ip, _fp, _fl, _i, _i]),
                "embed_fwd": (None, [_fp, _fp, _ip, _i, _i]),
                "embed_bwd": (None, [_fp, _fp, _ip, _i, _i]),
            })
        for name, (res, args) in sig.items():
            f = getattr(d, p + name)
            f.restype, f.argtypes = res, args

    def _fn(self, name):
        return getattr(self.dll, self.p + name)

    def rmsnorm_fwd(self, x, g):
        rows, D = x.shape
        out = np.empty_like(x)
        rinv = np.empty(rows, np.float32)
        self._fn("rmsnorm_fwd")(_f(x), _f(g), _f(out), _f(rinv), rows, D)
        return out, rinv

    def rmsnorm_bwd(self, x, g, rinv, dy, dx, dg):
        """dx += ..., dg += ... in place."""
        rows, D = x.shape
        self._fn("rmsnorm_bwd")(_f(x), _f(g), _f(rinv), _f(dy), _f(dx), _f(dg), rows, D)

    def rope_table(self, maxpos, hd):
        cs = np.empty((maxpos, hd // 2), np.float32)
        sn = np.empty_like(cs)
        if self.ref:
            self._fn("rope_table")(_f(cs), _f(sn), maxpos, hd)
        else:
            self._fn("rope_table")(_f(cs), _f(sn), maxpos, hd, 10000.0)
        return cs, sn

    def rope(self, buf, T, nh, hd, back, pos=None):
        """In place on buf [rows][nh*hd]; row r at pos[r], else r % T."""
        rows = buf.shape[0]
        if pos is None:
            pos = (np.arange(rows) % T).astype(np.int32)
        maxpos = int(pos.max()) + 1 if rows else 1
        if self.ref:
            self._fn("rope")(_f(buf), _n(pos), rows, nh, hd, maxpos, back)
        else:
            cs, sn = self.rope_table(maxpos, hd)
            self._fn("rope")(_f(buf), _n(pos), T, rows, nh, hd, _f(cs), _f(sn), back)

    def attn_fwd(self, q, k, v, B, T, H, KV, hd, win=0):
        out = np.zeros_like(q)
        self._fn("attn_fwd")(_f(q), _f(k), _f(v), _f(out), B, T, H, KV, hd, win)
        return out

    def attn_bwd(self, q, k, v, datt, B, T, H, KV, hd, win=0):
        dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
        self._fn("attn_bwd")(_f(q), _f(k), _f(v), _f(datt), _f(dq), _f(dk), _f(dv), B, T, H, KV, hd, win)
        return dq, dk, dv

    def adamw(self, P, G, M, V, lr, b1, b2, wd, t, gscale):
        self._fn("adamw")(_f(P), _f(G), _f(M), _f(V), P.size, lr, b1, b2, wd, t, gscale)

    def gradnorm(self, G):
        return float(self._fn("gradnorm")(_f(G), G.size))

    # whole model
    def param_count(self, m):
        if self.ref:
            return int(self._fn("param_count")(m.V, m.D, m.L, m.H, m.KV, m.F, m.T, m.n_mtp, m.n_exp))
        mp = OrcLayerMap()
        self._fn("param_map")(ctypes.byref(m), 0, ctypes.byref(mp))
        return int(mp.total)

    def layer_map(self, m, l):
        """map_weights offsets of layer l (oracle side)."""
        mp = OrcLayerMap()
        getattr(self.dll, "orc_param_map")(ctypes.byref(m), l, ctypes.byref(mp))
        return {n: int(getattr(mp, n)) for n, _ in OrcLayerMap._fields_}

    def init_params(self, m, seed):
        P = np.empty(self.param_count(m), np.float32)
        if self.ref:
            self._fn("init_params")(_f(P), seed, m.V, m.D, m.L, m.H, m.KV, m.F, m.T, m.n_mtp, m.n_exp)
        else:
            self._fn("init_params")(ctypes.byref(m), _f(P), seed)
        return P

    def train_step(self, m, B, P, tok, tgt, tgt_mtp=None):
        """forward + memset(G) + backward; returns (loss, G)."""
        G = np.zeros_like(P)
        N = B * m.T
        tm = tgt_mtp if tgt_mtp is not None and m.n_mtp else np.zeros((max(m.n_mtp, 1), N), np.int32)
        tm = np.ascontiguousarray(tm, np.int32)
        if self.ref:
            loss = self._fn("train_step")(_f(P), _f(G), _n(tok), _n(tgt), _n(tm), B, m.V, m.D, m.L, m.H, m.KV,
                                          m.F, m.T, m.n_mtp, m.n_exp, m.win, m.full_every)
        else:
            loss = self._fn("train_step")(ctypes.byref(m), B, _f(P), _f(G), _n(tok), _n(tgt), _n(tm))
        return float(loss), G


def param_regions(st, m):
    """(name, start, end) of every parameter tensor of model m in
    map_weights order (tinylm.c:361-393), from the oracle's layout."""
    D, KD, F, E = m.D, m.KV * (m.D // m.H), m.F, max(m.n_exp, 1)
    hq = (m.D // m.H) if m.qknorm else 0
    out = [("emb", 0, m.V * D)]
    for l in range(m.L):
        w = st.layer_map(m, l)
        sizes = dict(an1=D, wq=D * D, wk=D * KD, wv=D * KD, wo=D * D, qn=hq, kn=hq, an2=D, wr=D * m.n_exp,
                     w1=E * D * F, w3=E * D * F, w2=E * F * D)
        out += [(f"{k}[{l}]", w[k], w[k] + n) for k, n in sizes.items() if n]
    w = st.layer_map(m, 0)
    out.append(("nf", w["nf"], w["nf"] + D))
    out += [(f"mtp[{k}]", w["mtp0"] + k * D * D, w["mtp0"] + (k + 1) * D * D) for k in range(m.n_mtp)]
    return out


class Decoder:
    """The oracle's decode restatement (orc_dec_*, forward_chunk of
    tinylm.c:3721-3830): a ring KV cache of W positions, f32 (kvdt 0) or
    f16 (kvdt 1) storage, fast_expf (exact 0) or expf (exact 1)."""

    def __init__(self, m, P, W, kvdt=1, exact=0, maxpos=4096, path=LIB):
        d = ctypes.CDLL(path)
        d.orc_dec_new.argtypes = [ctypes.POINTER(OrcModel), _i, _i, _i, _i]
        d.orc_dec_new.restype = ctypes.c_void_p
        d.orc_dec_free.argtypes = [ctypes.c_void_p]
        d.orc_dec_chunk.argtypes = [ctypes.c_void_p, _fp, _ip, _i, _i, _fp]
        d.orc_dec_chunk_fn.argtypes = [ctypes.c_void_p, _fp, _ip, _i, _i, _fp, _fp]
        d.orc_mtp_argmax.argtypes = [ctypes.POINTER(OrcModel), _fp, _fp, _i, _fp]
        d.orc_mtp_argmax.restype = _i
        d.orc_dec_set_ring.argtypes = [ctypes.c_void_p, _i, ctypes.c_void_p, ctypes.c_void_p]
        d.orc_dec_set_store.argtypes = [ctypes.c_void_p, _i]
        d.orc_dec_ring.argtypes = [ctypes.c_void_p, _i, _i]
        d.orc_dec_ring.restype = ctypes.c_void_p
        self.dll, self.m, self.P = d, m, np.ascontiguousarray(P, np.float32)
        self.W, self.kvdt = W, kvdt
        self.h = d.orc_dec_new(ctypes.byref(m), W, kvdt, exact, maxpos)

    def set_ring(self, l, K, V):
        """Overwrite layer l's ring with K, V ([W][KD] of uint16 f16 bits for
        an f16 ring, float32 for an f32 ring)."""
        dt = np.uint16 if self.kvdt else np.float32
        n = self.W * self.m.KV * (self.m.D // self.m.H)
        K, V = (np.ascontiguousarray(a, dt).reshape(-1) for a in (K, V))
        assert K.size == n and V.size == n
        self.dll.orc_dec_set_ring(self.h, l, K.ctypes.data, V.ctypes.data)

    def ring(self, l):
        """Copies of layer l's K and V rings ([W][KD], as set_ring takes them)."""
        dt = np.uint16 if self.kvdt else np.float32
        KD = self.m.KV * (self.m.D // self.m.H)
        out = []
        for v in (0, 1):
            buf = (ctypes.c_char * (self.W * KD * np.dtype(dt).itemsize)).from_address(
                self.dll.orc_dec_ring(self.h, l, v))
            out.append(np.frombuffer(buf, dt).reshape(self.W, KD).copy())
        return out

    def set_store(self, store):
        """store False: chunks attend over the ring as set, storing nothing."""
        self.dll.orc_dec_set_store(self.h, 1 if store else 0)

    def chunk(self, tok, start):
        tok = np.ascontiguousarray(tok, np.int32)
        out = np.empty((tok.size, self.m.V), np.float32)
        self.dll.orc_dec_chunk(self.h, _f(self.P), _n(tok), tok.size, start, _f(out))
        return out

    def chunk_fn(self, tok, start):
        """(logits [m][V], final-normed rows fn [m][D])."""
        tok = np.ascontiguousarray(tok, np.int32)
        out = np.empty((tok.size, self.m.V), np.float32)
        fn = np.empty((tok.size, self.m.D), np.float32)
        self.dll.orc_dec_chunk_fn(self.h, _f(self.P), _n(tok), tok.size, start, _f(out), _f(fn))
        return out, fn

    def mtp_argmax(self, fn1, k):
        """MTP head k's draft token from a final-normed row (and its logits)."""
        fn1 = np.ascontiguousarray(fn1, np.float32)
        lg = np.empty(self.m.V, np.float32)
        t = self.dll.orc_mtp_argmax(ctypes.byref(self.m), _f(self.P), _f(fn1), k, _f(lg))
        return int(t), lg

    def generate_spec(self, prompt, n, prefill):
        """run_generation's greedy self-speculative loop (tinylm.c:3977-3995,
        no stop token): prefill in chunks of `prefill` rows; then each round
        takes x1 = argmax of the current logits row, the K heads' drafts from
        its final-normed row, and one chunk of the K+1 tokens at pos; draft
        r+1 is kept while it equals row r's argmax.  Returns (tokens, chunks,
        rows) with rows[i] the logits row token i was chosen from."""
        K = self.m.n_mtp
        prompt = np.ascontiguousarray(prompt, np.int32)
        i = 0
        while i < prompt.size:
            mm = min(prefill, prompt.size - i)
            lg, fn = self.chunk_fn(prompt[i:i + mm], i)
            i += mm
        pos, lg_cur, fn_cur = prompt.size, lg[-1], fn[-1]
        out, rows, chunks = [], [], 0
        while len(out) < n:
            draft = [int(np.argmax(lg_cur))] + [self.mtp_argmax(fn_cur, k)[0] for k in range(K)]
            lg, fn = self.chunk_fn(np.array(draft, np.int32), pos)
            chunks += 1
            out.append(draft[0])
            rows.append(lg_cur)
            acc = 0
            while acc < K and len(out) < n and draft[acc + 1] == int(np.argmax(lg[acc])):
                out.append(draft[acc + 1])
                rows.append(lg[acc])
                acc += 1
            pos += acc + 1
            lg_cur, fn_cur = lg[acc], fn[acc]
        return out, chunks, rows

    def __del__(self):
        try:
            self.dll.orc_dec_free(self.h)
        except Exception:
            pass


DEC_LIB = os.path.join(HERE, "_ref", "libtlref_dec.so")


class DecAttn:
    """One layer's decode attention step -- the new rows' ring stores, then
    attention of the query rows over their windows -- from the oracle
    (orc_dec_attn) or from the reference's own kv_store and attn_body
    (_ref/libtlref_dec.so, forward_chunk's unsplit path, tinylm.c:3759-3795).
    Ring of W = T positions, f32 (kvdt 0) or f16 (kvdt 1), fast_expf."""

    def __init__(self, which, D, H, KV, T, L=1, win=0, full_every=0, kvdt=1):
        self.D, self.KD = D, KV * (D // H)
        if which == "oracle":
            d = ctypes.CDLL(LIB)
            d.orc_dec_new.argtypes = [ctypes.POINTER(OrcModel), _i, _i, _i, _i]
            d.orc_dec_new.restype = ctypes.c_void_p
            d.orc_dec_attn.argtypes = [ctypes.c_void_p, _i, _fp, _fp, _fp, _i, _i, _fp]
            self.m = model(1, D, L, H, KV, 4, T, win=win, full_every=full_every)
            self.h = d.orc_dec_new(ctypes.byref(self.m), T, kvdt, 0, T)
            self.fn = d.orc_dec_attn
        else:
            d = ctypes.CDLL(DEC_LIB)
            d.tlref_dec_new.argtypes = [_i] * 8
            d.tlref_dec_new.restype = ctypes.c_void_p
            d.tlref_dec_attn.argtypes = [ctypes.c_void_p, _i, _fp, _fp, _fp, _i, _i, _fp]
            d.tlref_dec_attn.restype = _i
            self.h = d.tlref_dec_new(D, H, KV, T, L, win, full_every, kvdt)
            self.fn = d.tlref_dec_attn
        self.dll = d

    def attn(self, l, q, k, v, start):
        q, k, v = (np.ascontiguousarray(a, np.float32) for a in (q, k, v))
        m = q.shape[0]
        ctx = np.empty((m, self.D), np.float32)
        self.fn(self.h, l, _f(q), _f(k), _f(v), m, start, _f(ctx))
        return ctx


def qknorm(buf, gain, nheads, which="oracle"):
    """qknorm_apply (tinylm.c:597-605) on buf [rows][nheads*hd], a copy."""
    buf = np.array(buf, np.float32, copy=True, order="C")
    gain = np.ascontiguousarray(gain, np.float32)
    rows = buf.shape[0]
    hd = buf.shape[1] // nheads
    if which == "oracle":
        d = ctypes.CDLL(LIB)
        d.orc_qknorm.argtypes = [_fp, _fp, _i, _i, _i]
        d.orc_qknorm(_f(buf), _f(gain), rows, nheads, hd)
    else:
        d = ctypes.CDLL(DEC_LIB)
        d.tlref_qknorm.argtypes = [_fp, _fp, _i, _i, _i]
        d.tlref_qknorm(_f(buf), _f(gain), rows, nheads, hd)
    return buf


def dec_moe(fnorm, fin, wr, w1, w3, w2, E):
    """The oracle's decode MoE layer (orc_dec_moe): (out, assign, gate, rprobs)."""
    d = ctypes.CDLL(LIB)
    d.orc_dec_moe.argtypes = [_i, _i, _i, _i, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _ip, _fp, _fp]
    fnorm, fin = (np.ascontiguousarray(a, np.float32) for a in (fnorm, fin))
    N, D = fnorm.shape
    F = w1.size // (E * D)
    out = np.empty_like(fin)
    assign = np.empty(N, np.int32)
    gate = np.empty(N, np.float32)
    rprobs = np.empty((N, E), np.float32)
    d.orc_dec_moe(N, D, F, E, _f(fnorm), _f(fin), _f(out), _f(np.ascontiguousarray(wr, np.float32)),
                  _f(np.ascontiguousarray(w1, np.float32)), _f(np.ascontiguousarray(w3, np.float32)),
                  _f(np.ascontiguousarray(w2, np.float32)), _n(assign), _f(gate), _f(rprobs))
    return out, assign, gate, rprobs


class RefDecode:
    """The reference's own decode pieces (_ref/libtlref_dec.so): a whole
    model's Gen (gen_new, no int8 copies) and, on the flat parameters P,
    moe_forward_q8's fp32 branch for layer l (tinylm.c:3433-3458) and
    mtp_argmax (:3930-3936).  Test infrastructure: built and run only where
    /root/reference exists."""

    def __init__(self, m, kvdt=1):
        d = ctypes.CDLL(DEC_LIB)
        d.tlref_gen_new.argtypes = [_i] * 11
        d.tlref_gen_new.restype = ctypes.c_void_p
        d.tlref_dec_moe.argtypes = [ctypes.c_void_p, _fp, _i, _fp, _fp, _fp, _i, _ip, _fp, _fp]
        d.tlref_dec_moe.restype = _i
        d.tlref_mtp_argmax.argtypes = [ctypes.c_void_p, _fp, _fp, _i, _fp]
        d.tlref_mtp_argmax.restype = _i
        self.dll, self.m = d, m
        self.h = d.tlref_gen_new(m.V, m.D, m.H, m.KV, m.F, m.T, m.L, m.n_exp, m.n_mtp, m.qknorm, kvdt)

    def moe(self, P, l, fnorm, fin):
        P = np.ascontiguousarray(P, np.float32)
        fnorm, fin = (np.ascontiguousarray(a, np.float32) for a in (fnorm, fin))
        N = fnorm.shape[0]
        out = np.empty_like(fin)
        assign = np.empty(N, np.int32)
        gate = np.empty(N, np.float32)
        rprobs = np.empty((N, self.m.n_exp), np.float32)
        rc = self.dll.tlref_dec_moe(self.h, _f(P), l, _f(fnorm), _f(fin), _f(out), N, _n(assign), _f(gate),
                                    _f(rprobs))
        assert rc == 0
        return out, assign, gate, rprobs

    def mtp_argmax(self, P, fn1, k):
        P, fn1 = (np.ascontiguousarray(a, np.float32) for a in (P, fn1))
        lg = np.empty(self.m.V, np.float32)
        t = self.dll.tlref_mtp_argmax(self.h, _f(P), _f(fn1), k, _f(lg))
        return int(t), lg


def ref_forward_logits(m, B, P, tok, path=SEQ_LIB):
    """forward()'s logits [B*T][V] from the reference's own code."""
    d = ctypes.CDLL(path)
    d.tlref_forward_logits.argtypes = [_fp, _ip, _fp] + [_i] * 11
    out = np.empty((B * m.T, m.V), np.float32)
    d.tlref_forward_logits(_f(np.ascontiguousarray(P, np.float32)), _n(np.ascontiguousarray(tok, np.int32)),
                           _f(out), B, m.V, m.D, m.L, m.H, m.KV, m.F, m.T, m.n_exp, m.win, m.full_every)
    return out


def half_fns(which="oracle"):
    """(f2h, h2f, fast_expf) on numpy arrays from the oracle or the reference."""
    if which == "oracle":
        d = ctypes.CDLL(LIB)
        d.orc_f2h.restype, d.orc_f2h.argtypes = ctypes.c_ushort, [ctypes.c_float]
        d.orc_h2f.restype, d.orc_h2f.argtypes = ctypes.c_float, [ctypes.c_ushort]
        d.orc_fast_expf.restype, d.orc_fast_expf.argtypes = ctypes.c_float, [ctypes.c_float]
        f2h = lambda x: np.array([d.orc_f2h(float(v)) for v in x], np.uint16)  # noqa: E731
        h2f = lambda h: np.array([d.orc_h2f(int(v)) for v in h], np.float32)  # noqa: E731
        fe = lambda x: np.array([d.orc_fast_expf(float(v)) for v in x], np.float32)  # noqa: E731
        return f2h, h2f, fe
    d = ctypes.CDLL(SEQ_LIB)
    up = ctypes.POINTER(ctypes.c_ushort)
    d.tlref_f2h.argtypes = [_fp, up, _i]
    d.tlref_h2f.argtypes = [up, _fp, _i]
    d.tlref_fast_expf.argtypes = [_fp, _fp, _i]

    def f2h(x):
        x = np.ascontiguousarray(x, np.float32)
        h = np.empty(x.size, np.uint16)
        d.tlref_f2h(_f(x), h.ctypes.data_as(up), x.size)
        return h

    def h2f(h):
        h = np.ascontiguousarray(h, np.uint16)
        x = np.empty(h.size, np.float32)
        d.tlref_h2f(h.ctypes.data_as(up), _f(x), h.size)
        return x

    def fe(x):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        d.tlref_fast_expf(_f(x), _f(y), x.size)
        return y
    return f2h, h2f, fe
