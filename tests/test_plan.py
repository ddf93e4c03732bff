"""CPU tests of the GEMM call sequences (tinylm-c_amd/host/tl_plan.c).

The training plan is compared call by call with the GEMM call list of the
reference's own forward + backward, recorded by compiling tinylm.c:539-1154
with its mm / mm_bt / mm_atb call sites logged (oracle/Makefile, fixtures in
tests/golden/seq_*.json): operation, every operand's buffer and offset, and
(M, K, N) must all match.
"""
import json
import os

import pytest

import tlgemm
from conftest import golden

SEQS = golden("seq_*.json")


def plan_gemms(p):
    out = []
    for c in p.calls:
        if c["op"] == "zero":
            continue
        nm = lambda i, o: [p.bufs[i][0], o]  # noqa: E731
        out.append([c["op"], nm(c["out"], c["out_off"]), nm(c["a"], c["a_off"]),
                    nm(c["b"], c["b_off"]), c["M"], c["K"], c["N"]])
    return out


@pytest.mark.parametrize("path", SEQS, ids=[os.path.basename(p)[4:-5] for p in SEQS])
def test_train_plan_matches_reference_call_list(path):
    d = json.load(open(path))
    p = tlgemm.host().plan_train(d["B"] * d["T"], d["D"], d["KV"] * (d["D"] // d["H"]), d["F"],
                                 d["V"], d["L"], d["n_mtp"])
    mine = plan_gemms(p)
    assert len(mine) == len(d["calls"])
    for i, (a, b) in enumerate(zip(mine, d["calls"])):
        assert a == b, f"call {i}: plan {a} != reference {b}"


def test_live_reference_log_when_available():
    """Where the reference tree exists, re-derive one log live."""
    lib = os.path.join(tlgemm.REPO, "oracle", "_ref", "libtlref_seq.so")
    if not os.path.exists(lib):
        pytest.skip("oracle/_ref not built here")
    from oracle import reference_train_log
    ref = reference_train_log(2, 8, 64, 8, 2, 96, 128, 2, 1)
    p = tlgemm.host().plan_train(16, 64, 16, 96, 128, 2, 1)
    mine = [[c[0], tuple(c[1]), tuple(c[2]), tuple(c[3]), c[4], c[5], c[6]] for c in plan_gemms(p)]
    assert [list(r) for r in ref] == [list(m) for m in mine]


@pytest.mark.parametrize("name", ["nano", "m3", "m8"])
def test_plan_counts_and_flops(name):
    import bench
    cfg = bench.TRAIN[name]
    p = tlgemm.host().plan_train(**cfg)
    g = [c for c in p.calls if c["op"] != "zero"]
    L, n_mtp = cfg["L"], cfg["n_mtp"]
    # 7 forward + 14 backward per layer, 3 head GEMMs, 6 per MTP head
    assert len(g) == 21 * L + 3 + 6 * n_mtp
    if name == "m3":
        assert abs(p.flops() / 1e9 - 124.02) < 0.01       # cfg1's GEMM flop per step
    # every accumulating GEMM into an activation buffer has a clear before it
    # since that buffer's last setting write
    cleared = set()
    for c in p.calls:
        key = (c["out"], c["out_off"])
        if c["op"] == "zero":
            cleared.add(c["out"])
        elif c["op"] in ("mm_bt",) and p.bufs[c["out"]][0] not in ("dfn",):
            assert c["out"] in cleared, c


def test_decode_plan_shapes():
    p = tlgemm.host().plan_decode(1, 384, 96, 1024, 2048, 8)
    g = [c for c in p.calls if c["op"] != "zero"]
    assert len(g) == 8 * 7 + 1
    wbytes = sum(4 * c["K"] * c["N"] for c in g)
    assert abs(wbytes / 1e6 - 52.69) < 0.01                # cfg3's weight bytes per decode step
    assert g[-1]["op"] == "mm_bt" and (g[-1]["K"], g[-1]["N"]) == (2048, 384)


def test_bad_plan_arguments():
    with pytest.raises(ValueError):
        tlgemm.host().plan_train(0, 8, 8, 8, 8, 1)
