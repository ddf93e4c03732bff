"""ctypes binding of libtlgemm.so (include/tlgemm.h) for Python callers.

This is the stub a Python user of the library would write; the tests and
bench.py go through it, so every GPU result they check comes from the HIP
kernels behind the C ABI.  There is no fallback: if the shared library is
missing, loading raises.
"""
import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "libtlgemm.so")
HEADER = os.path.join(REPO, "include", "tlgemm.h")
TRAIN_HEADER = os.path.join(REPO, "include", "tltrain.h")
DECODE_HEADER = os.path.join(REPO, "include", "tldecode.h")

_fp = ctypes.POINTER(ctypes.c_float)
_ip = ctypes.POINTER(ctypes.c_int)
_vp = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t

# name -> (restype, argtypes)
SIGNATURES = {
    "tlg_init": (_i, [_i]),
    "tlg_shutdown": (None, []),
    "tlg_last_error": (ctypes.c_char_p, []),
    "tlg_sgemm_nn": (None, [_vp, _vp, _vp, _i, _i, _i]),
    "tlg_sgemm_nt_acc": (None, [_vp, _vp, _vp, _i, _i, _i]),
    "tlg_sgemm_tn_acc": (None, [_vp, _vp, _vp, _i, _i, _i]),
    "tlg_register": (_i, [_vp, _sz]),
    "tlg_unregister": (_i, [_vp]),
    "tlg_push": (_i, [_vp]),
    "tlg_pull": (_i, [_vp]),
    "tlg_mirror": (_vp, [_vp]),
    "tlg_dev_sgemm_nn": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "tlg_dev_sgemm_nt_acc": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "tlg_dev_sgemm_tn_acc": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "tlg_dev_sgemm_tn_acc_noalloc": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "tlg_dev_zero": (_i, [_vp, _sz, _vp]),
    "tlg_dev_malloc": (_vp, [_sz]),
    "tlg_dev_free": (_i, [_vp]),
    "tlg_memcpy_h2d": (_i, [_vp, _vp, _sz, _vp]),
    "tlg_memcpy_d2h": (_i, [_vp, _vp, _sz, _vp]),
    "tlg_memcpy_d2d": (_i, [_vp, _vp, _sz, _vp]),
    "tlg_stream_create": (_vp, []),
    "tlg_stream_destroy": (_i, [_vp]),
    "tlg_stream_sync": (_i, [_vp]),
    "tlg_event_create": (_vp, []),
    "tlg_event_destroy": (_i, [_vp]),
    "tlg_event_record": (_i, [_vp, _vp]),
    "tlg_event_elapsed_ms": (ctypes.c_float, [_vp, _vp]),
    "tlg_dev_fill_normal": (_i, [_vp, _sz, ctypes.c_ulonglong, ctypes.c_float, _vp]),
    "tlg_kernel_name": (_i, [_i, _i, _i, _i, ctypes.c_char_p, _i, _ip]),
    "tlg_tune_force": (_i, [_i, _i]),
    "tlg_dev_copy": (_i, [_vp, _vp, _sz, _vp]),
    "tlg_dev_read": (_i, [_vp, _sz, _vp, _vp]),
    "tlg_dev_mfma_peak": (_i, [_vp, _i, _i, _vp]),
    "tlg_dev_gemm_group": (_i, [_vp, _i, _vp]),
    "tlg_dev_gemm_flush": (_i, [_vp]),
    "tlg_dev_gemm_pending": (_i, []),
    "tlg_group_kernel": (ctypes.c_char_p, []),
    "tlg_gemv_status": (_i, []),
    "tlg_tune_group": (_i, [_i]),
    "tlg_tune_group_policy": (_i, [_ip, _i, ctypes.c_double, _i]),
    "tlg_tune_group_split": (_i, [_i]),
    "tlg_tune_expert": (_i, [_i, _i]),
    "tlg_graph_begin": (_i, [_vp]),
    "tlg_graph_end": (_vp, [_vp]),
    "tlg_graph_launch": (_i, [_vp, _vp]),
    "tlg_graph_destroy": (_i, [_vp]),
    "tlg_dev_moe_grouped_fwd": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "tlg_dev_moe_grouped_bwd": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp,
                                     _vp, _vp, _vp, _vp, _vp]),
    "tlg_moe_keep_bytes": (_sz, [_i, _i, _i, _i]),
    "tlg_dev_moe_grouped_fwd_keep": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                          _vp, _sz, _vp]),
    "tlg_dev_moe_grouped_bwd_kept": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp,
                                          _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "tlg_moe_grouped_fwd": (None, [_vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "tlg_moe_grouped_bwd": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp,
                                   _vp, _vp, _vp, _vp]),
    # include/tltrain.h
    "tlg_dev_embed_fwd": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "tlg_dev_embed_bwd": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "tlg_dev_rmsnorm_fwd": (_i, [_vp, _vp, _vp, _vp, _i, _i, _vp]),
    "tlg_dev_rmsnorm_bwd": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp]),
    "tlg_dev_rmsnorm_bwd_defer": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp, _sz, _vp]),
    "tlg_dev_rope": (_i, [_vp, _vp, _i, _i, _i, _i, _vp, _vp, _i, _i, _vp]),
    "tlg_dev_attn_fwd": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "tlg_dev_attn_bwd": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "tlg_dev_swiglu_mm": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "tlg_dev_mm_bt_swiglu_bwd": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "tlg_dev_attn_fwd_rope": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp]),
    "tlg_dev_attn_bwd_rope": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp, _vp,
                                   _vp]),
    "tlg_dev_attn_bwd_rope_d": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp,
                                     _vp, _vp]),
    "tlg_dev_add": (_i, [_vp, _vp, _sz, _vp]),
    "tlg_dev_swiglu_fwd": (_i, [_vp, _vp, _vp, _sz, _vp]),
    "tlg_dev_swiglu_bwd": (_i, [_vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "tlg_dev_silu_res": (_i, [_vp, _vp, _vp, _sz, _vp]),
    "tlg_dev_silu_bwd": (_i, [_vp, _vp, _vp, _sz, _vp]),
    "tlg_dev_xent": (_i, [_vp, _vp, _vp, _vp, ctypes.c_float, _i, _i, _vp]),
    "tlg_dev_gradnorm": (_i, [_vp, _sz, _vp, _vp]),
    "tlg_dev_embed_rmsnorm_fwd": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _vp, _i, _i, _vp]),
    "tlg_dev_xent_rows": (_i, [_vp, _vp, _vp, _vp, ctypes.c_float, _i, _i, _vp]),
    "tlg_dev_gradnorm_loss": (_i, [_vp, _sz, _vp, _vp, _i, _vp, _vp]),
    "tlg_dev_adamw": (_i, [_vp, _vp, _vp, _vp, _sz, _vp, _vp, _vp]),
    # include/tldecode.h
    "tlg_dev_dec_embed": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "tlg_dev_kv_store": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp]),
    "tlg_dev_dec_attn": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _vp]),
    "tlg_dev_dec_argmax": (_i, [_vp, _i, _i, _vp, _vp, _vp]),
    "tlg_dev_dec_gemv": (_i, [_vp, _i, _vp]),
    "tlg_dev_transpose": (_i, [_vp, _vp, _i, _i, _vp]),
    "tlg_dev_dec_qknorm": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "tlg_dev_dec_moe_route": (_i, [_vp, _i, _i, _vp, _vp, _vp]),
    "tlg_dev_dec_mtp_mix": (_i, [_vp, _vp, _vp, _vp, _i, _vp]),
    "tlg_dev_argmax_rows": (_i, [_vp, _i, _i, _vp, _vp]),
    "tlg_dev_dec_rope_attn": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i,
                                   _vp]),
    "tlg_dec_persist_xbytes": (_sz, [_i, _i, _i, _i]),
    "tlg_dev_dec_persist": (_i, [_vp, _i, _vp]),
    "tlg_dev_dec_chunks": (_i, [_vp, _i, _vp, _i, _vp]),
    "tlg_dec_persist_status": (_i, [_vp, _vp]),
}


def header_symbols(path=None):
    """Function names declared in a C header (tlg_*/tl_* prototypes); by
    default the library's two public headers."""
    names = set()
    for p in ([path] if path else [HEADER, TRAIN_HEADER, DECODE_HEADER]):
        text = open(p).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(tlg?_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


class TlgError(RuntimeError):
    pass


class TlgGemmCall(ctypes.Structure):
    """include/tlgemm.h TlgGemmCall: one call of a grouped launch."""
    _fields_ = [("op", ctypes.c_int), ("beta", ctypes.c_int), ("C", _vp),
                ("M", ctypes.c_int), ("K", ctypes.c_int), ("N", ctypes.c_int), ("nseg", ctypes.c_int),
                ("A", _vp * 3), ("B", _vp * 3), ("Nseg", ctypes.c_int * 3), ("R", _vp),
                ("dotB", _vp), ("dotOut", _vp)]


class TlgDecGemv(ctypes.Structure):
    """include/tldecode.h TlgDecGemv: one GEMV of a fused decode launch."""
    _fields_ = [("op", ctypes.c_int), ("beta", ctypes.c_int), ("C", _vp),
                ("M", ctypes.c_int), ("K", ctypes.c_int), ("N", ctypes.c_int), ("A", _vp), ("B", _vp),
                ("pro", ctypes.c_int), ("gain", _vp), ("A2", _vp), ("bsel", _vp), ("bstride", ctypes.c_longlong),
                ("cgate", _vp)]


class Lib:
    """Loaded libtlgemm.so with typed entry points."""

    def __init__(self, path=LIB_PATH):
        if not os.path.exists(path):
            raise FileNotFoundError(
                f"{path} is not built; run __graft_entry__.build() (make -C tinylm-c_amd)")
        self.path = path
        self.dll = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(self.dll, name)
            f.restype = res
            f.argtypes = args

    def __getattr__(self, name):
        return getattr(self.dll, name)

    def check(self, rc, what=""):
        if rc != 0:
            msg = self.dll.tlg_last_error().decode(errors="replace")
            raise TlgError(f"{what} failed ({rc}): {msg}")
        return rc

    # device-pointer helpers: integer addresses (e.g. torch tensor.data_ptr())
    def mm(self, Y, X, W, M, K, N, stream=0):
        return self.check(self.dll.tlg_dev_sgemm_nn(Y, X, W, M, K, N, stream), "tlg_dev_sgemm_nn")

    def mm_bt(self, dX, dY, W, M, K, N, stream=0):
        return self.check(self.dll.tlg_dev_sgemm_nt_acc(dX, dY, W, M, K, N, stream), "tlg_dev_sgemm_nt_acc")

    def mm_atb(self, dW, X, dY, M, K, N, stream=0):
        return self.check(self.dll.tlg_dev_sgemm_tn_acc(dW, X, dY, M, K, N, stream), "tlg_dev_sgemm_tn_acc")

    def zero(self, p, n, stream=0):
        return self.check(self.dll.tlg_dev_zero(p, n, stream), "tlg_dev_zero")

    def moe_fwd(self, fnorm, fin, out, N, D, F, E, wr, w1, w3, w2, assign, gate, rprobs, stream=0):
        """Device-pointer top-1 MoE forward (tinylm.c:857-891)."""
        return self.check(self.dll.tlg_dev_moe_grouped_fwd(fnorm, fin, out, N, D, F, E, wr, w1, w3, w2,
                                                           assign, gate, rprobs, stream),
                          "tlg_dev_moe_grouped_fwd")

    def moe_fwd_keep(self, fnorm, fin, out, N, D, F, E, wr, w1, w3, w2, assign, gate, rprobs, keep, keep_bytes,
                     stream=0):
        """MoE forward that also keeps the index and expert rows for moe_bwd_kept."""
        return self.check(self.dll.tlg_dev_moe_grouped_fwd_keep(fnorm, fin, out, N, D, F, E, wr, w1, w3, w2, assign,
                                                                gate, rprobs, keep, keep_bytes, stream),
                          "tlg_dev_moe_grouped_fwd_keep")

    def moe_bwd_kept(self, fnorm, dout, d_fnorm, assign, gate, rprobs, N, D, F, E, wr, w1, w3, w2,
                     gwr, gw1, gw3, gw2, kept, kept_bytes, stream=0):
        """MoE backward from a kept forward state (no recompute)."""
        return self.check(self.dll.tlg_dev_moe_grouped_bwd_kept(fnorm, dout, d_fnorm, assign, gate, rprobs,
                                                                N, D, F, E, wr, w1, w3, w2, gwr, gw1, gw3,
                                                                gw2, kept, kept_bytes, stream),
                          "tlg_dev_moe_grouped_bwd_kept")

    def moe_bwd(self, fnorm, dout, d_fnorm, assign, gate, rprobs, N, D, F, E, wr, w1, w3, w2,
                gwr, gw1, gw3, gw2, stream=0):
        """Device-pointer top-1 MoE backward (tinylm.c:895-947)."""
        return self.check(self.dll.tlg_dev_moe_grouped_bwd(fnorm, dout, d_fnorm, assign, gate, rprobs,
                                                           N, D, F, E, wr, w1, w3, w2, gwr, gw1, gw3,
                                                           gw2, stream),
                          "tlg_dev_moe_grouped_bwd")

    def group(self, calls, stream=0, flush=True):
        """tlg_dev_gemm_group over dicts {op, beta, C, M, K, N, A: [..], B: [..], Nseg: [..], R}."""
        arr = (TlgGemmCall * len(calls))()
        for i, c in enumerate(calls):
            a = arr[i]
            a.op, a.beta, a.C = {"mm": 0, "mm_bt": 1, "mm_atb": 2}[c["op"]], c.get("beta", 0), c["C"]
            a.R = c.get("R", None)
            a.dotB, a.dotOut = c.get("dotB", None), c.get("dotOut", None)
            a.M, a.K, a.N = c["M"], c["K"], c["N"]
            a.nseg = len(c["A"])
            for s_ in range(a.nseg):
                a.A[s_], a.B[s_] = c["A"][s_], c["B"][s_]
                a.Nseg[s_] = c.get("Nseg", [c["N"]] * 3)[s_]
        self.check(self.dll.tlg_dev_gemm_group(arr, len(calls), stream), "tlg_dev_gemm_group")
        if flush:
            self.check(self.dll.tlg_dev_gemm_flush(stream), "tlg_dev_gemm_flush")

    def kernel_name(self, op, M, K, N):
        """(rocprof kernel name, splits) a device call of op 'mm'/'mm_bt'/'mm_atb' uses."""
        buf = ctypes.create_string_buffer(128)
        sp = ctypes.c_int(0)
        code = {"mm": 0, "mm_bt": 1, "mm_atb": 2}[op]
        self.check(self.dll.tlg_kernel_name(code, M, K, N, buf, 128, ctypes.byref(sp)), "tlg_kernel_name")
        return buf.value.decode(), sp.value


_LIB = None


def load():
    global _LIB
    if _LIB is None:
        _LIB = Lib()
    return _LIB


# ----------------------------------------------------------- host library --
HOST_PATH = os.path.join(HERE, "libtlhost.so")
HOST_HEADER = os.path.join(HERE, "host", "tl_plan.h")
OPS = {0: "mm", 1: "mm_bt", 2: "mm_atb", 3: "zero"}


class TlBuf(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 16), ("floats", ctypes.c_size_t), ("init", ctypes.c_int)]


class TlCall(ctypes.Structure):
    _fields_ = [("op", ctypes.c_int), ("out", ctypes.c_int), ("a", ctypes.c_int), ("b", ctypes.c_int),
                ("out_off", ctypes.c_size_t), ("a_off", ctypes.c_size_t), ("b_off", ctypes.c_size_t),
                ("M", ctypes.c_int), ("K", ctypes.c_int), ("N", ctypes.c_int),
                ("n", ctypes.c_size_t), ("line", ctypes.c_int), ("what", ctypes.c_char * 16),
                ("run", ctypes.c_int), ("hoist", ctypes.c_int)]


class TlPlan(ctypes.Structure):
    _fields_ = [("nbuf", ctypes.c_int), ("ncall", ctypes.c_int), ("cap", ctypes.c_int),
                ("buf", TlBuf * 48), ("call", ctypes.POINTER(TlCall)),
                ("R", ctypes.c_int), ("D", ctypes.c_int), ("KD", ctypes.c_int), ("F", ctypes.c_int),
                ("V", ctypes.c_int), ("L", ctypes.c_int), ("n_mtp", ctypes.c_int),
                ("run", ctypes.c_int)]


class TlCkpt(ctypes.Structure):
    """host/tl_ckpt.h: the header of a tinylm.c model file."""
    _fields_ = [(n, _i) for n in ("version", "V", "D", "L", "H", "KV", "F", "T", "eot", "tmpl", "n_mtp",
                                  "n_exp", "win", "full_every", "n_shared", "qknorm", "topk")] + [
        ("n_params", _sz), ("params_offset", _sz), ("tok_len", ctypes.c_longlong)]


class CheckpointError(ValueError):
    """A model file tl_ckpt_open / tl_ckpt_read refused; `code` is the
    TL_CKPT_E* value."""

    def __init__(self, code, text, path):
        super().__init__(f"{path}: {text} (code {code})")
        self.code = code


class TlWeightMap(ctypes.Structure):
    _fields_ = [(n, ctypes.c_size_t) for n in
                ("emb", "an1", "wq", "wk", "wv", "wo", "an2", "w1", "w3", "w2", "nf", "mtp0", "total")]


class TlModel(ctypes.Structure):
    """host/tl_train.h TlModel (tinylm.c Cfg fields of the training step and
    the decoder)."""
    _fields_ = [(n, ctypes.c_int) for n in ("V", "D", "L", "H", "KV", "F", "T", "n_mtp", "n_exp", "win",
                                            "full_every")] + [("rope_base", ctypes.c_float),
                                                              ("qknorm", ctypes.c_int)]


class Train:
    """One TlTrain: device P / G / AdamW state and activations of a model."""

    def __init__(self, host, model, B):
        if isinstance(model, dict):
            model = TlModel(**{"rope_base": 10000.0, **model})
        self.host, self.model, self.B = host, model, B
        self.N = B * model.T
        self.h = host.dll.tl_train_new(ctypes.byref(model), B)
        if not self.h:
            raise TlgError("tl_train_new failed: bad model shape or out of device memory")
        self.np = host.dll.tl_train_nparams(self.h)

    def buf(self, which):
        """Device address of 0 P, 1 G, 2 M, 3 V."""
        return self.host.dll.tl_train_buf(self.h, which)

    def act(self, name, layer=0):
        return self.host.dll.tl_train_act(self.h, name.encode(), layer)

    def _ck(self, rc, what):
        if rc != 0:
            lib = load()
            raise TlgError(f"{what} failed ({rc}): {lib.dll.tlg_last_error().decode(errors='replace')}")
        return 0

    def upload(self, P, stream):
        import numpy as np
        P = np.ascontiguousarray(P, np.float32)
        assert P.size == self.np
        return self._ck(self.host.dll.tl_train_upload(self.h, P.ctypes.data, stream), "tl_train_upload")

    def set_batch(self, tok, tgt, tgt_mtp, stream):
        import numpy as np
        tok = np.ascontiguousarray(tok, np.int32)
        tgt = np.ascontiguousarray(tgt, np.int32)
        tm = None if tgt_mtp is None else np.ascontiguousarray(tgt_mtp, np.int32)
        return self._ck(self.host.dll.tl_train_set_batch(self.h, tok.ctypes.data, tgt.ctypes.data,
                                                  None if tm is None else tm.ctypes.data, stream),
                 "tl_train_set_batch")

    def set_hyper(self, lr, b1, b2, wd, step, stream):
        return self._ck(self.host.dll.tl_train_set_hyper(self.h, lr, b1, b2, wd, step, stream), "tl_train_set_hyper")

    def forward(self, stream):
        return self._ck(self.host.dll.tl_train_forward(self.h, stream), "tl_train_forward")

    def backward(self, stream):
        return self._ck(self.host.dll.tl_train_backward(self.h, stream), "tl_train_backward")

    def optimize(self, stream):
        return self._ck(self.host.dll.tl_train_optimize(self.h, stream), "tl_train_optimize")

    def step(self, stream):
        return self._ck(self.host.dll.tl_train_step(self.h, stream), "tl_train_step")

    def graph_build(self, stream):
        return self._ck(self.host.dll.tl_train_graph_build(self.h, stream), "tl_train_graph_build")

    def graph_step(self, stream):
        return self._ck(self.host.dll.tl_train_graph_step(self.h, stream), "tl_train_graph_step")

    def loss(self, stream):
        return float(self.host.dll.tl_train_loss(self.h, stream))

    def gnorm(self, stream):
        return float(self.host.dll.tl_train_gnorm(self.h, stream))

    def time_phases(self, stream):
        ms = (ctypes.c_float * 3)()
        self._ck(self.host.dll.tl_train_time_phases(self.h, ms, stream), "tl_train_time_phases")
        return list(ms)

    def autotune(self, cands, reps, stream, rts=(0,)):
        """Per grouped launch of the step, the fastest tile configuration of
        `cands`, with each split target of `rts` (tl_train_autotune_split; 0 =
        the library's automatic target); returns the chosen tile table."""
        arr = (ctypes.c_int * len(cands))(*cands)
        rarr = (ctypes.c_int * len(rts))(*rts)
        self._ck(self.host.dll.tl_train_autotune_split(self.h, arr, len(cands), rarr, len(rts), reps, stream),
                 "tl_train_autotune_split")
        return self.tiles()

    def tiles(self):
        buf = (ctypes.c_int * 512)()
        n = self.host.dll.tl_train_tiles(self.h, buf, 512)
        return list(buf[:n])

    def splits(self):
        buf = (ctypes.c_int * 512)()
        n = self.host.dll.tl_train_splits(self.h, buf, 512)
        return list(buf[:n])

    def close(self):
        """Free the device state now rather than at garbage collection."""
        if self.h:
            self.host.dll.tl_train_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Decode:
    """One TlDecode: device weights, KV ring cache and greedy state."""

    def __init__(self, host, model, W, kv_f16, exact_exp, maxpos, mmax, pool):
        if isinstance(model, dict):
            model = TlModel(**{"rope_base": 10000.0, **model})
        self.host, self.model, self.W, self.kv_f16 = host, model, W, kv_f16
        self.h = host.dll.tl_decode_new(ctypes.byref(model), W, kv_f16, exact_exp, maxpos, mmax, pool)
        if not self.h:
            raise TlgError("tl_decode_new failed: bad model shape or out of device memory")
        self.np = host.dll.tl_decode_nparams(self.h)

    def _ck(self, rc, what):
        if rc != 0:
            raise TlgError(f"{what} failed ({rc}): {load().dll.tlg_last_error().decode(errors='replace')}")
        return 0

    def upload(self, P, stream):
        import numpy as np
        P = np.ascontiguousarray(P, np.float32)
        assert P.size == self.np
        return self._ck(self.host.dll.tl_decode_upload(self.h, P.ctypes.data, stream), "tl_decode_upload")

    def reset(self, stream):
        return self._ck(self.host.dll.tl_decode_reset(self.h, stream), "tl_decode_reset")

    def params(self, copy=0):
        """Device address of weight copy `copy`."""
        return self.host.dll.tl_decode_params(self.h, copy)

    def pack(self, stream):
        """Rebuild the decode layout after writing weights through params()."""
        return self._ck(self.host.dll.tl_decode_pack(self.h, stream), "tl_decode_pack")

    def chunk(self, tok, start, stream):
        """forward_chunk of host tokens; returns the logits [m][V] (host)."""
        import numpy as np
        tok = np.ascontiguousarray(tok, np.int32)
        self._ck(self.host.dll.tl_decode_chunk(self.h, tok.ctypes.data, tok.size, start, stream), "tl_decode_chunk")
        return self.logits(tok.size, stream)

    def logits(self, m, stream):
        import numpy as np
        out = np.empty((m, self.model.V), np.float32)
        L = load()
        L.check(L.tlg_memcpy_d2h(out.ctypes.data, self.host.dll.tl_decode_logits(self.h), out.nbytes, stream), "d2h")
        L.check(L.tlg_stream_sync(stream), "sync")
        return out

    def ring(self, l, stream):
        """Layer l's K and V rings as host arrays [W][KD] (uint16 f16 bits or
        float32, as the decoder stores them)."""
        import numpy as np
        L = load()
        dt = np.uint16 if self.kv_f16 else np.float32
        KD = self.model.KV * (self.model.D // self.model.H)
        out = []
        for v in (0, 1):
            a = np.empty((self.W, KD), dt)
            L.check(L.tlg_memcpy_d2h(a.ctypes.data, self.host.dll.tl_decode_ring(self.h, l, v), a.nbytes, stream),
                    "d2h")
            out.append(a)
        L.check(L.tlg_stream_sync(stream), "sync")
        return out

    def prime(self, prompt, stream):
        import numpy as np
        p = np.ascontiguousarray(prompt, np.int32)
        return self._ck(self.host.dll.tl_decode_prime(self.h, p.ctypes.data, p.size, stream), "tl_decode_prime")

    def greedy_step(self, stream, copy=0):
        return self._ck(self.host.dll.tl_decode_greedy_step(self.h, copy, stream), "tl_decode_greedy_step")

    def mtp_draft(self, row, k, dtok, stream):
        """MTP head k's draft from row `row` of the last chunk into the device
        int dtok (tl_decode_mtp_draft)."""
        return self._ck(self.host.dll.tl_decode_mtp_draft(self.h, row, k, dtok, stream), "tl_decode_mtp_draft")

    def generate_spec(self, prompt, n, stream):
        """Greedy self-speculative generation (tl_decode_generate_spec):
        (tokens, verification chunks)."""
        import numpy as np
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(n, np.int32)
        ch = ctypes.c_int(0)
        self._ck(self.host.dll.tl_decode_generate_spec(self.h, p.ctypes.data, p.size, n, out.ctypes.data,
                                                       ctypes.byref(ch), stream), "tl_decode_generate_spec")
        return out, ch.value

    def graph_build(self, stream):
        return self._ck(self.host.dll.tl_decode_graph_build(self.h, stream), "tl_decode_graph_build")

    def graph_step(self, stream):
        return self._ck(self.host.dll.tl_decode_graph_step(self.h, stream), "tl_decode_graph_step")

    def persist(self, n, stream, toks=None):
        """n greedy steps in one persistent launch (asynchronous); toks: a
        device int32 buffer of n entries for the chosen tokens, or None."""
        return self._ck(self.host.dll.tl_decode_persist(self.h, n, toks, stream), "tl_decode_persist")

    def persist_chunks(self, m, toks, n, stream, out=None):
        """n chunks of m rows of the device int32 tokens `toks` (n * m of
        them) in one persistent launch (asynchronous); out: a device int32
        buffer of n * m entries for every row's argmax, or None."""
        return self._ck(self.host.dll.tl_decode_chunks(self.h, m, toks, n, out, stream), "tl_decode_chunks")

    def persist_status(self, stream):
        """Synchronize; raises if a persistent launch aborted."""
        return self._ck(self.host.dll.tl_decode_persist_status(self.h, stream), "tl_decode_persist_status")

    def set_fused(self, fused):
        """1: glue folded into the GEMV / attention launches (default);
        0: every glue op as its own launch."""
        return self._ck(self.host.dll.tl_decode_set_fused(self.h, 1 if fused else 0), "tl_decode_set_fused")

    def state(self, stream):
        s = (ctypes.c_int * 3)()
        self._ck(self.host.dll.tl_decode_state(self.h, s, stream), "tl_decode_state")
        return list(s)

    def close(self):
        """Free the device state now rather than at garbage collection."""
        if self.h:
            self.host.dll.tl_decode_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Plan:
    """A built TlPlan: buffers (name, floats, init) and calls as dicts."""

    def __init__(self, host, raw):
        self.host = host
        self.raw = raw
        self.bufs = [(b.name.decode(), b.floats, b.init) for b in raw.buf[:raw.nbuf]]
        self.calls = []
        for i in range(raw.ncall):
            c = raw.call[i]
            self.calls.append(dict(op=OPS[c.op], out=c.out, a=c.a, b=c.b, out_off=c.out_off,
                                   a_off=c.a_off, b_off=c.b_off, M=c.M, K=c.K, N=c.N, n=c.n,
                                   line=c.line, what=c.what.decode(), run=c.run))

    def buf_id(self, name):
        return [b[0] for b in self.bufs].index(name)

    def flops(self):
        return sum(2.0 * c["M"] * c["K"] * c["N"] for c in self.calls if c["op"] != "zero")

    def regions(self, name):
        """(label, start, end) float ranges of buffer `name` that separate GEMM
        outputs: one per weight matrix for P/G (map_weights layout), one per
        layer slice for the per-layer activation buffers, else the whole."""
        r = self.raw
        n = self.bufs[self.buf_id(name)][1]
        if name in ("P", "G"):
            out = []
            for l in range(r.L):
                m = TlWeightMap()
                self.host.dll.tl_weight_map(r.V, r.D, r.KD, r.F, r.L, r.n_mtp, l, ctypes.byref(m))
                if l == 0:
                    out.append(("emb", m.emb, m.emb + r.V * r.D))
                for w, sz in (("wq", r.D * r.D), ("wk", r.D * r.KD), ("wv", r.D * r.KD),
                              ("wo", r.D * r.D), ("w1", r.D * r.F), ("w3", r.D * r.F), ("w2", r.F * r.D)):
                    off = getattr(m, w)
                    out.append((f"{w}[{l}]", off, off + sz))
            for k in range(r.n_mtp):
                off = m.mtp0 + k * r.D * r.D
                out.append((f"mtp[{k}]", off, off + r.D * r.D))
            return out
        if self.raw.L > 1 and n % self.raw.L == 0 and name in (
                "a_in", "a_norm", "q", "k", "v", "att_ctx", "f_in", "f_norm", "g", "u"):
            s = n // self.raw.L
            return [(f"{name}[{l}]", l * s, (l + 1) * s) for l in range(self.raw.L)]
        return [(name, 0, n)]

    def __del__(self):
        try:
            self.host.dll.tl_plan_free(ctypes.byref(self.raw))
        except Exception:
            pass


class Host:
    """libtlhost.so: the -DUSE_HIP seam (mm/mm_bt/mm_atb) and the plan executor."""

    def __init__(self, path=HOST_PATH):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built; run __graft_entry__.build()")
        d = ctypes.CDLL(path)
        P = ctypes.POINTER(TlPlan)
        d.tl_plan_train.argtypes = [P] + [_i] * 7
        d.tl_plan_train.restype = _i
        for n in ("tl_plan_decode", "tl_plan_decode_packed"):
            getattr(d, n).argtypes = [P] + [_i] * 6
            getattr(d, n).restype = _i
        d.tl_weight_map.argtypes = [_i] * 7 + [ctypes.POINTER(TlWeightMap)]
        d.tl_weight_map.restype = None
        d.tl_plan_free.argtypes = [P]
        d.tl_plan_free.restype = None
        C = ctypes.POINTER(TlCkpt)
        d.tl_ckpt_open.argtypes = [ctypes.c_char_p, C]
        d.tl_ckpt_open.restype = _i
        d.tl_ckpt_read.argtypes = [ctypes.c_char_p, C, _vp, _sz]
        d.tl_ckpt_read.restype = _i
        d.tl_ckpt_param_count.argtypes = [C]
        d.tl_ckpt_param_count.restype = _sz
        d.tl_ckpt_error.argtypes = [_i]
        d.tl_ckpt_error.restype = ctypes.c_char_p
        d.tl_ckpt_model.argtypes = [C, ctypes.POINTER(TlModel)]
        d.tl_ckpt_model.restype = _i
        d.tl_run_new.argtypes = [P, _i]
        d.tl_run_new.restype = _vp
        d.tl_run_free.argtypes = [_vp]
        d.tl_run_free.restype = None
        d.tl_run_fill.argtypes = [_vp, ctypes.c_ulonglong, _vp]
        d.tl_run_buf.argtypes = [_vp, _i]
        d.tl_run_buf.restype = _vp
        for n in ("tl_run_step", "tl_run_step_grouped", "tl_run_graph_step"):
            getattr(d, n).argtypes = [_vp, _vp]
            getattr(d, n).restype = _i
        d.tl_run_graph_build.argtypes = [_vp, _vp, _i]
        d.tl_run_graph_build.restype = _i
        d.tl_run_grouped_launches.argtypes = [_vp]
        d.tl_run_grouped_launches.restype = _i
        d.tl_run_time_launches.argtypes = [_vp, ctypes.POINTER(_vp), _i, _vp]
        d.tl_run_time_launches.restype = _i
        d.tl_run_launch_info.argtypes = [_vp, _i, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]
        d.tl_run_launch_info.restype = _i
        d.tl_run_autotune.argtypes = [_vp, _ip, _i, _i, _vp]
        d.tl_run_autotune.restype = _i
        d.tl_run_launch_config.argtypes = [_vp, _i]
        d.tl_run_launch_config.restype = _i
        d.tl_run_set_launch_config.argtypes = [_vp, _i, _i]
        d.tl_run_set_launch_config.restype = _i
        d.tl_run_autotune_split.argtypes = [_vp, _ip, _i, _ip, _i, _i, _vp]
        d.tl_run_autotune_split.restype = _i
        d.tl_run_launch_split.argtypes = [_vp, _i]
        d.tl_run_launch_split.restype = _i
        d.tl_run_set_launch_split.argtypes = [_vp, _i, _i]
        d.tl_run_set_launch_split.restype = _i
        d.tl_run_launch_kernel.argtypes = [_vp, _i]
        d.tl_run_launch_kernel.restype = ctypes.c_char_p
        d.tl_run_call.argtypes = [_vp, _i, _vp]
        d.tl_run_call.restype = _i
        for n in ("mm", "mm_bt", "mm_atb"):
            getattr(d, n).argtypes = [_vp, _vp, _vp, _i, _i, _i]
            getattr(d, n).restype = None
        # host/tl_train.h
        d.tl_train_new.argtypes = [ctypes.POINTER(TlModel), _i]
        d.tl_train_new.restype = _vp
        d.tl_train_free.argtypes = [_vp]
        d.tl_train_free.restype = None
        d.tl_train_nparams.argtypes = [_vp]
        d.tl_train_nparams.restype = _sz
        d.tl_train_buf.argtypes = [_vp, _i]
        d.tl_train_buf.restype = _vp
        d.tl_train_act.argtypes = [_vp, ctypes.c_char_p, _i]
        d.tl_train_act.restype = _vp
        d.tl_train_upload.argtypes = [_vp, _vp, _vp]
        d.tl_train_set_batch.argtypes = [_vp, _vp, _vp, _vp, _vp]
        d.tl_train_set_hyper.argtypes = [_vp, ctypes.c_float, ctypes.c_float, ctypes.c_float, ctypes.c_float, _i, _vp]
        for n in ("tl_train_forward", "tl_train_backward", "tl_train_optimize", "tl_train_step",
                  "tl_train_graph_build", "tl_train_graph_step"):
            getattr(d, n).argtypes = [_vp, _vp]
            getattr(d, n).restype = _i
        for n in ("tl_train_loss", "tl_train_gnorm"):
            getattr(d, n).argtypes = [_vp, _vp]
            getattr(d, n).restype = ctypes.c_float
        d.tl_train_time_phases.argtypes = [_vp, ctypes.POINTER(ctypes.c_float), _vp]
        d.tl_train_autotune.argtypes = [_vp, ctypes.POINTER(ctypes.c_int), _i, _i, _vp]
        d.tl_train_tiles.argtypes = [_vp, ctypes.POINTER(ctypes.c_int), _i]
        d.tl_train_autotune_split.argtypes = [_vp, ctypes.POINTER(ctypes.c_int), _i, ctypes.POINTER(ctypes.c_int),
                                              _i, _i, _vp]
        d.tl_train_splits.argtypes = [_vp, ctypes.POINTER(ctypes.c_int), _i]
        # host/tl_decode.h
        d.tl_decode_new.argtypes = [ctypes.POINTER(TlModel), _i, _i, _i, _i, _i, _i]
        d.tl_decode_new.restype = _vp
        d.tl_decode_free.argtypes = [_vp]
        d.tl_decode_free.restype = None
        d.tl_decode_nparams.argtypes = [_vp]
        d.tl_decode_nparams.restype = _sz
        for n in ("tl_decode_params",):
            getattr(d, n).argtypes = [_vp, _i]
            getattr(d, n).restype = _vp
        d.tl_decode_logits.argtypes = [_vp]
        d.tl_decode_logits.restype = _vp
        d.tl_decode_ring.argtypes = [_vp, _i, _i]
        d.tl_decode_ring.restype = _vp
        for n in ("tl_decode_upload", "tl_decode_state"):
            getattr(d, n).argtypes = [_vp, _vp, _vp]
            getattr(d, n).restype = _i
        for n in ("tl_decode_reset", "tl_decode_pack", "tl_decode_graph_build", "tl_decode_graph_step"):
            getattr(d, n).argtypes = [_vp, _vp]
            getattr(d, n).restype = _i
        d.tl_decode_chunk.argtypes = [_vp, _vp, _i, _i, _vp]
        d.tl_decode_prime.argtypes = [_vp, _vp, _i, _vp]
        d.tl_decode_greedy_step.argtypes = [_vp, _i, _vp]
        d.tl_decode_persist.argtypes = [_vp, _i, _vp, _vp]
        d.tl_decode_persist.restype = _i
        d.tl_decode_chunks.argtypes = [_vp, _i, _vp, _i, _vp, _vp]
        d.tl_decode_chunks.restype = _i
        d.tl_decode_persist_status.argtypes = [_vp, _vp]
        d.tl_decode_persist_status.restype = _i
        d.tl_decode_set_fused.argtypes = [_vp, _i]
        d.tl_decode_set_fused.restype = _i
        d.tl_decode_mtp_draft.argtypes = [_vp, _i, _i, _vp, _vp]
        d.tl_decode_mtp_draft.restype = _i
        d.tl_decode_generate_spec.argtypes = [_vp, _vp, _i, _i, _vp, _vp, _vp]
        d.tl_decode_generate_spec.restype = _i
        self.dll = d

    def load_checkpoint(self, path):
        """A tinylm.c model file (host/tl_ckpt.h): (header fields as a dict,
        the fp32 parameters in map_weights' order as a numpy array).  Raises
        CheckpointError for files the reader refuses (quantized TLQ files,
        a bad magic, a truncated body)."""
        import numpy as np
        info = TlCkpt()
        bpath = os.fsencode(path)
        rc = self.dll.tl_ckpt_open(bpath, ctypes.byref(info))
        if rc != 0:
            raise CheckpointError(rc, self.dll.tl_ckpt_error(rc).decode(), path)
        P = np.empty(info.n_params, np.float32)
        rc = self.dll.tl_ckpt_read(bpath, ctypes.byref(info), P.ctypes.data, P.size)
        if rc != 0:
            raise CheckpointError(rc, self.dll.tl_ckpt_error(rc).decode(), path)
        return {n: getattr(info, n) for n, _ in TlCkpt._fields_}, P

    def decode(self, model, W, kv_f16=1, exact_exp=0, maxpos=4096, mmax=8, pool=1):
        """Device-resident decoding (host/tl_decode.h)."""
        return Decode(self, model, W, kv_f16, exact_exp, maxpos, mmax, pool)

    def train(self, model, B):
        """A device-resident training step (host/tl_train.h) for `model`
        (a TlModel or a dict of its fields) and batches of B sequences."""
        return Train(self, model, B)

    def plan_train(self, R, D, KD, F, V, L, n_mtp=0):
        raw = TlPlan()
        if self.dll.tl_plan_train(ctypes.byref(raw), R, D, KD, F, V, L, n_mtp) != 0:
            raise ValueError("tl_plan_train failed")
        return Plan(self, raw)

    def plan_decode(self, M, D, KD, F, V, L, packed=False):
        raw = TlPlan()
        fn = self.dll.tl_plan_decode_packed if packed else self.dll.tl_plan_decode
        if fn(ctypes.byref(raw), M, D, KD, F, V, L) != 0:
            raise ValueError("tl_plan_decode failed")
        return Plan(self, raw)


_HOST = None


def host():
    global _HOST
    if _HOST is None:
        _HOST = Host()
    return _HOST
