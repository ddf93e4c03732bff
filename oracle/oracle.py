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
