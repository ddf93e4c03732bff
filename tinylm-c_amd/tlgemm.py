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
    "tlg_dev_zero": (_i, [_vp, _sz, _vp]),
}


def header_symbols(path=HEADER):
    """Function names declared in a C header (tlg_*/tl_* prototypes)."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tlg?_[a-z0-9_]+)\s*\(", text)))


class TlgError(RuntimeError):
    pass


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


_LIB = None


def load():
    global _LIB
    if _LIB is None:
        _LIB = Lib()
    return _LIB
