"""The model-file reader (host/tl_ckpt.h, libtlhost.so) on the CPU.

The files are written here byte for byte as the reference lays them out:
model_save_bundle (tinylm.c:1895-1913) writes the 4-byte magic, the int32
header, the fp32 parameters and an int32 tokenizer length plus blob; hdr_ints
(:1691-1700) fixes the header length of TLM1-TLM7 and cfg_from_hdr
(:1705-1718) the order of its fields.  The parameter count the reader derives
is pinned against the reference's own param_count (oracle/_ref, compiled from
tinylm.c:345-358) for the fields that function takes, and against its two
optional terms (QK-norm gains, shared experts) as differences between counts.
"""
import ctypes
import os
import struct

import numpy as np
import pytest

import tlgemm
from oracle import SEQ_LIB, StepFns, model

# header fields in cfg_from_hdr's order and the count of each version
FIELDS = ("V", "D", "L", "H", "KV", "F", "T", "eot", "tmpl", "n_mtp", "n_exp", "win", "full_every",
          "n_shared", "qknorm", "topk")
HDR_INTS = {1: 8, 2: 9, 3: 10, 4: 11, 5: 13, 6: 15, 7: 16}

E_IO, E_MAGIC, E_QUANT, E_SHAPE, E_TRUNC = -1, -2, -3, -4, -5


@pytest.fixture(scope="module")
def host():
    return tlgemm.host()


def write_model(path, version, cfg, P, tok=b"", magic=None):
    """A model file as model_save_bundle writes it, for any header version."""
    hdr = [int(cfg.get(n, 0)) for n in FIELDS[:HDR_INTS[version]]]
    with open(path, "wb") as f:
        f.write(magic if magic is not None else f"TLM{version}".encode())
        f.write(struct.pack(f"<{len(hdr)}i", *hdr))
        f.write(np.asarray(P, np.float32).tobytes())
        if version >= 2:
            f.write(struct.pack("<i", len(tok)))
            f.write(tok)


def ref_count(cfg):
    """The reference's param_count for the fields it takes (oracle/_ref when
    built, else the restatement the step tests pin against it)."""
    fns = StepFns("reference" if os.path.exists(SEQ_LIB) else "oracle")
    m = model(cfg["V"], cfg["D"], cfg["L"], cfg["H"], cfg["KV"], cfg["F"], cfg["T"], n_mtp=cfg.get("n_mtp", 0),
              n_exp=cfg.get("n_exp", 0))
    return fns.param_count(m)


BASE = dict(V=96, D=64, L=2, H=4, KV=2, F=80, T=24, eot=2)
CASES = [
    dict(BASE),                                                   # dense
    dict(BASE, n_mtp=2),                                          # Medusa heads
    dict(BASE, n_exp=4),                                          # top-1 MoE
    dict(BASE, n_exp=3, n_mtp=1, H=8, KV=1),                      # GQA 8:1 + MoE + MTP
]


@pytest.mark.parametrize("cfg", CASES)
def test_param_count_is_the_reference_count(host, tmp_path, cfg):
    P = np.zeros(ref_count(cfg), np.float32)
    path = tmp_path / "m.bin"
    write_model(path, 4, cfg, P)
    info, got = host.load_checkpoint(path)
    assert info["n_params"] == P.size == got.size


def test_optional_terms_of_the_count(host, tmp_path):
    """QK-norm adds two gains of head_dim per layer; shared experts add whole
    expert FFNs per layer (param_count :345-358): checked as differences, the
    base count being the reference's."""
    D, F, L, hd = BASE["D"], BASE["F"], BASE["L"], BASE["D"] // BASE["H"]
    moe = dict(BASE, n_exp=4)
    base = ref_count(moe)
    for extra, want in ((dict(qknorm=1), base + L * 2 * hd),
                        (dict(n_shared=2), base + L * 2 * 3 * D * F),
                        (dict(qknorm=1, n_shared=1), base + L * 2 * hd + L * 3 * D * F)):
        cfg = dict(moe, **extra)
        path = tmp_path / "m6.bin"
        write_model(path, 6, cfg, np.zeros(want, np.float32))
        info, P = host.load_checkpoint(path)
        assert info["n_params"] == want == P.size
    # a dense model ignores n_shared, as n_slots does (:71)
    cfg = dict(BASE, n_shared=3)
    write_model(tmp_path / "d.bin", 6, cfg, np.zeros(ref_count(BASE), np.float32))
    assert host.load_checkpoint(tmp_path / "d.bin")[0]["n_params"] == ref_count(BASE)


@pytest.mark.parametrize("version", [1, 2, 3, 4, 5, 6, 7])
def test_every_version_round_trips(host, tmp_path, version):
    """Each version's header fields come back, the ones it lacks read 0, and
    the parameters come back bit for bit (NaN and signed-zero patterns too)."""
    cfg = dict(BASE, tmpl=1, n_mtp=1, n_exp=0, win=8, full_every=2, topk=1)
    keep = FIELDS[:HDR_INTS[version]]
    eff = {n: (cfg.get(n, 0) if n in keep else 0) for n in FIELDS}
    n = ref_count(eff)
    P = np.random.default_rng(version).standard_normal(n).astype(np.float32)
    P[:3] = [np.nan, -0.0, np.inf]
    tok = bytes(range(37)) if version >= 2 else b""
    path = tmp_path / f"v{version}.bin"
    write_model(path, version, cfg, P, tok)
    info, got = host.load_checkpoint(path)
    assert info["version"] == version
    for k in FIELDS:
        assert info[k] == eff[k], k
    assert info["params_offset"] == 4 + 4 * HDR_INTS[version]
    assert info["tok_len"] == (len(tok) if version >= 2 else -1)
    assert got.view(np.uint32).tobytes() == P.view(np.uint32).tobytes()


def test_model_fields_for_the_decoder(host, tmp_path):
    cfg = dict(BASE, n_mtp=1, win=8, full_every=2)
    write_model(tmp_path / "m.bin", 5, cfg, np.zeros(ref_count(cfg), np.float32))
    info, m = tlgemm.TlCkpt(), tlgemm.TlModel()
    assert host.dll.tl_ckpt_open(os.fsencode(tmp_path / "m.bin"), ctypes.byref(info)) == 0
    host.dll.tl_ckpt_model(ctypes.byref(info), ctypes.byref(m))
    for k in ("V", "D", "L", "H", "KV", "F", "T", "n_mtp", "n_exp", "win", "full_every"):
        assert getattr(m, k) == cfg.get(k, 0), k
    assert m.rope_base == 10000.0


def test_refused_files(host, tmp_path):
    n = ref_count(BASE)
    P = np.zeros(n, np.float32)

    def code(path):
        with pytest.raises(tlgemm.CheckpointError) as e:
            host.load_checkpoint(path)
        return e.value.code

    assert code(tmp_path / "missing.bin") == E_IO
    write_model(tmp_path / "magic.bin", 4, BASE, P, magic=b"GGUF")
    assert code(tmp_path / "magic.bin") == E_MAGIC
    write_model(tmp_path / "q.bin", 4, BASE, P, magic=b"TLQ1")
    assert code(tmp_path / "q.bin") == E_QUANT
    # a body one float short, a header cut off, a tokenizer blob cut off
    write_model(tmp_path / "short.bin", 4, BASE, P[:-1], tok=b"")
    with open(tmp_path / "short.bin", "r+b") as f:          # drop the tokenizer length too
        f.truncate(4 + 44 + 4 * (n - 1))
    assert code(tmp_path / "short.bin") == E_TRUNC
    with open(tmp_path / "hdr.bin", "wb") as f:
        f.write(b"TLM7" + struct.pack("<5i", 1, 2, 3, 4, 5))
    assert code(tmp_path / "hdr.bin") == E_TRUNC
    write_model(tmp_path / "tok.bin", 4, BASE, P, tok=b"abcdef")
    with open(tmp_path / "tok.bin", "r+b") as f:
        f.truncate(os.path.getsize(tmp_path / "tok.bin") - 2)
    assert code(tmp_path / "tok.bin") == E_TRUNC
    # dimensions that describe no model
    for bad in (dict(BASE, D=0), dict(BASE, H=-1), dict(BASE, n_exp=-2)):
        write_model(tmp_path / "shape.bin", 4, bad, P)
        assert code(tmp_path / "shape.bin") == E_SHAPE
    # a TLM1 file (no tokenizer field) of exactly header + body is whole
    write_model(tmp_path / "v1.bin", 1, BASE, P)
    assert host.load_checkpoint(tmp_path / "v1.bin")[0]["tok_len"] == -1


E_UNSUP = -6


def test_models_the_step_cannot_run_are_refused(host, tmp_path):
    """Shared experts are refused by the reference itself (check_supported,
    :1946-1953) and top-k > 1 routing is not the top-1 layer built here: the
    header reads, but tl_ckpt_model refuses to describe such a model.  A
    QK-norm model (TLM6/7) is described, with qknorm set: the decoder runs it
    (the training step refuses it, as the reference does, :2707-2713)."""
    def model_rc(version, cfg):
        info = tlgemm.TlCkpt(version=version, **{k: int(cfg.get(k, 0)) for k in FIELDS[:HDR_INTS[version]]})
        m = tlgemm.TlModel()
        return host.dll.tl_ckpt_model(ctypes.byref(info), ctypes.byref(m)), m

    rc, m = model_rc(6, dict(BASE, qknorm=1))
    assert rc == 0 and m.qknorm == 1 and m.V == BASE["V"]
    assert host.dll.tl_train_new(ctypes.byref(m), 1) is None
    assert model_rc(6, dict(BASE, n_exp=4, n_shared=1))[0] == E_UNSUP
    assert model_rc(7, dict(BASE, n_exp=4, topk=2))[0] == E_UNSUP
    assert model_rc(7, dict(BASE, n_exp=4, topk=1))[0] == 0
    assert model_rc(7, dict(BASE, topk=2))[0] == 0                # dense: topk unused
    assert host.dll.tl_ckpt_error(E_UNSUP).decode().startswith("model uses shared experts")


def test_header_whose_count_overflows_is_refused(host, tmp_path):
    """A crafted header whose parameter count does not fit in 64-bit byte
    offsets is refused as describing no model (not wrapped to a small count
    that would pass the length check)."""
    cfg = dict(BASE, D=1 << 24, F=1 << 24, H=1 << 19, KV=1, n_exp=65536, n_shared=65536, L=65536)
    write_model(tmp_path / "big.bin", 6, cfg, np.zeros(4, np.float32))
    with pytest.raises(tlgemm.CheckpointError) as e:
        host.load_checkpoint(tmp_path / "big.bin")
    assert e.value.code == E_SHAPE
    # the largest fields a header can hold, still refused without wrapping
    cfg = dict(BASE, V=2**31 - 1, D=2**31 - 1, F=2**31 - 1, H=1, KV=1, L=2**31 - 1, n_exp=2**31 - 1,
               n_shared=2**31 - 1, n_mtp=2**31 - 1)
    write_model(tmp_path / "max.bin", 6, cfg, np.zeros(4, np.float32))
    with pytest.raises(tlgemm.CheckpointError) as e:
        host.load_checkpoint(tmp_path / "max.bin")
    assert e.value.code == E_SHAPE
