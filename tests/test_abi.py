"""CPU checks of the drop-in boundary: the shared library exists, loads
without a GPU, and exports every function include/tlgemm.h declares (no
compute call is made here)."""
import ctypes
import os
import subprocess

import tlgemm


def test_library_built():
    assert os.path.exists(tlgemm.LIB_PATH), "run __graft_entry__.build()"


def test_exports_every_header_symbol():
    declared = tlgemm.header_symbols()
    assert "tlg_sgemm_nn" in declared and "tlg_dev_sgemm_tn_acc" in declared
    dll = ctypes.CDLL(tlgemm.LIB_PATH)
    missing = [s for s in declared if not hasattr(dll, s)]
    assert not missing, missing


def test_binding_covers_header():
    assert set(tlgemm.header_symbols()) <= set(tlgemm.SIGNATURES)


def test_no_cpu_fallback_symbols():
    """The product library contains no CPU GEMM: it must not link the oracle."""
    out = subprocess.run(["nm", "-D", "--defined-only", tlgemm.LIB_PATH],
                         capture_output=True, text=True, check=True).stdout
    assert "orc_" not in out and "tlref_" not in out
