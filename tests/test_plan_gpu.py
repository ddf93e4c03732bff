"""GPU parity of whole GEMM steps: the plan executor (C, libtlhost.so) runs a
step's calls on device-resident buffers through libtlgemm; the CPU oracle runs
the same calls on copies of the same initial buffers; every buffer must agree
to the north_star bar (max|err| / mean|ref| <= 1e-4).  Also: HIP-graph replays
equal eager launches bit for bit, replay after replay."""
import ctypes

import numpy as np
import pytest

import bench
import tlgemm
from oracle import F64Prims, normwise_rel, run_plan_cpu

pytestmark = pytest.mark.gpu
TOL = 1e-4


def snapshot(lib, host, plan, run, stream):
    out = {}
    for i, (name, n, _) in enumerate(plan.bufs):
        a = np.empty(n, np.float32)
        ptr = host.dll.tl_run_buf(run, i)
        lib.check(lib.tlg_memcpy_d2h(a.ctypes.data, ptr, a.nbytes, stream), "d2h")
        out[name] = a
    lib.check(lib.tlg_stream_sync(stream), "sync")
    return out


def new_run(lib, host, plan, pool=1, seed=99):
    """A device run of `plan` with every buffer seeded; buffers the plan
    starts from zero (outputs, G) are filled with noise instead, so a clear
    or a setting GEMM that did not happen cannot pass for one that did."""
    stream = lib.tlg_stream_create()
    run = host.dll.tl_run_new(ctypes.byref(plan.raw), pool)
    assert run, lib.tlg_last_error()
    fill(lib, host, plan, run, stream, seed)
    return run, stream


def fill(lib, host, plan, run, stream, seed):
    lib.check(host.dll.tl_run_fill(run, seed, stream), "fill")
    for i, (name, n, init) in enumerate(plan.bufs):
        if init == 3:
            lib.check(lib.tlg_dev_fill_normal(host.dll.tl_run_buf(run, i), n, seed * 31 + i, 1.0, stream), name)


@pytest.mark.parametrize("grouped", [0, 1], ids=["calls", "grouped"])
@pytest.mark.parametrize("name", ["nano", "m3", "m8"])
def test_train_step_matches_oracle(lib, orc, name, grouped):
    host = tlgemm.host()
    plan = host.plan_train(**bench.TRAIN[name])
    print("train step", name, len(plan.calls), "calls", "grouped" if grouped else "", flush=True)
    run, stream = new_run(lib, host, plan)
    try:
        init = snapshot(lib, host, plan, run, stream)
        step = host.dll.tl_run_step_grouped if grouped else host.dll.tl_run_step
        lib.check(step(run, stream), "step")
        got = snapshot(lib, host, plan, run, stream)
    finally:
        host.dll.tl_run_free(run)
    f64 = {k: v.copy() for k, v in init.items()}
    orc.set_threads(16)
    run_plan_cpu(plan, init, orc)            # the reference arithmetic
    run_plan_cpu(plan, f64, F64Prims(orc))   # textbook sums in double
    worst = []
    for bname, _, _ in plan.bufs:
        for label, a, b in plan.regions(bname):
            e_ref = normwise_rel(got[bname][a:b], init[bname][a:b])
            e_64 = normwise_rel(got[bname][a:b], f64[bname][a:b])
            ref_64 = normwise_rel(init[bname][a:b], f64[bname][a:b])
            worst.append((e_ref, e_64, ref_64, label))
    worst.sort(reverse=True)
    print("worst regions (gpu-vs-ref, gpu-vs-fp64, ref-vs-fp64):",
          [(f"{a:.2e}", f"{b:.2e}", f"{c:.2e}", lab) for a, b, c, lab in worst[:4]], flush=True)
    for e_ref, e_64, _, label in worst:
        assert e_ref <= TOL, f"{name}: {label} vs reference arithmetic {e_ref:.3e}"
        assert e_64 <= TOL, f"{name}: {label} vs fp64 {e_64:.3e}"


@pytest.mark.parametrize("grouped", [0, 1], ids=["calls", "grouped"])
def test_graph_replays_match_eager(lib, grouped):
    """Replay a captured step several times with eager work (re-fills) in
    between; each replay must equal the eager step bit for bit."""
    host = tlgemm.host()
    plan = host.plan_train(**bench.TRAIN["m8"] if grouped else bench.TRAIN["nano"])
    run, stream = new_run(lib, host, plan, seed=5)
    try:
        step = host.dll.tl_run_step_grouped if grouped else host.dll.tl_run_step
        lib.check(step(run, stream), "eager")
        eager = snapshot(lib, host, plan, run, stream)
        lib.check(host.dll.tl_run_graph_build(run, stream, grouped), "graph")
        for rep in range(3):
            fill(lib, host, plan, run, stream, 5)
            lib.check(host.dll.tl_run_graph_step(run, stream), "replay")
            got = snapshot(lib, host, plan, run, stream)
            for bname, _, _ in plan.bufs:
                assert np.array_equal(got[bname], eager[bname]), f"replay {rep}: {bname}"
    finally:
        host.dll.tl_run_free(run)


@pytest.mark.parametrize("packed", [False, True], ids=["reference_layout", "decode_layout"])
@pytest.mark.parametrize("grouped", [0, 1], ids=["calls", "grouped"])
@pytest.mark.parametrize("M", [1, 2, 4, 8])
def test_decode_step_matches_oracle(lib, orc, M, grouped, packed):
    """The decode GEMV set (forward_chunk's projections, tinylm.c:3748-3829)
    against the oracle under the reference's decode dispatch, on the
    reference's weight layout (mm) and on the decode layout (memset + mm_bt
    over transposed weights)."""
    host = tlgemm.host()
    plan = host.plan_decode(M, packed=packed, **bench.DECODE)
    run, stream = new_run(lib, host, plan, pool=2, seed=3)
    try:
        init = snapshot(lib, host, plan, run, stream)
        lib.check(host.dll.tl_run_graph_build(run, stream, grouped), "graph")
        for _ in range(2):                                # both pool copies
            lib.check(host.dll.tl_run_graph_step(run, stream), "step")
        got = snapshot(lib, host, plan, run, stream)
    finally:
        host.dll.tl_run_free(run)
    orc.set_pool(7)                                       # decode dispatch rule
    try:
        run_plan_cpu(plan, init, orc)
    finally:
        orc.set_pool(1)
    for bname, _, _ in plan.bufs:
        assert normwise_rel(got[bname], init[bname]) <= TOL, bname


def test_use_hip_seam(lib, orc):
    """mm / mm_bt / mm_atb with tinylm.c's exact signatures (libtlhost.so,
    built -DUSE_HIP) on host buffers."""
    host = tlgemm.host()
    r = np.random.default_rng(8)
    M, K, N = 257, 96, 130
    X = r.standard_normal((M, K), dtype=np.float32)
    W = (0.02 * r.standard_normal((K, N))).astype(np.float32)
    dY = (0.01 * r.standard_normal((M, N))).astype(np.float32)
    Y = np.full((M, N), np.nan, np.float32)
    host.dll.mm(Y.ctypes.data, X.ctypes.data, W.ctypes.data, M, K, N)
    assert normwise_rel(Y, orc.mm(X, W)) <= TOL
    dX = r.standard_normal((M, K), dtype=np.float32)
    ref = orc.mm_bt(dX.copy(), dY, W)
    host.dll.mm_bt(dX.ctypes.data, dY.ctypes.data, W.ctypes.data, M, K, N)
    assert normwise_rel(dX, ref) <= TOL
    dW = r.standard_normal((K, N), dtype=np.float32)
    ref = orc.mm_atb(dW.copy(), X, dY)
    host.dll.mm_atb(dW.ctypes.data, X.ctypes.data, dY.ctypes.data, M, K, N)
    assert normwise_rel(dW, ref) <= TOL


@pytest.mark.parametrize("gcfg", [0, 1, 3, 4, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20, 21, 22, 23,
                                  24, 25, 26, 27, 28, 29, 30, 31, 32, 33, 34, 35, 36, 37, 38, 39, 40, 41,
                                  42, 43, 44, 45, 46, 47, 48, 49, 50])
def test_group_tile_configs(lib, orc, gcfg):
    """Every tile shape grouped launches can use, on the nano step."""
    host = tlgemm.host()
    plan = host.plan_train(**bench.TRAIN["nano"])
    lib.check(lib.tlg_tune_group(gcfg), "tune")
    run, stream = new_run(lib, host, plan, seed=gcfg)
    try:
        init = snapshot(lib, host, plan, run, stream)
        lib.check(host.dll.tl_run_step_grouped(run, stream), "step")
        got = snapshot(lib, host, plan, run, stream)
    finally:
        host.dll.tl_run_free(run)
        lib.check(lib.tlg_tune_group(-1), "tune")
    run_plan_cpu(plan, init, orc)
    for bname, _, _ in plan.bufs:
        for label, a, b in plan.regions(bname):
            assert normwise_rel(got[bname][a:b], init[bname][a:b]) <= TOL, (gcfg, label)


@pytest.mark.parametrize("cfg,rt", [(3, 64), (15, 256), (22, 512), (20, 2048), (14, 8192)])
def test_split_targets_keep_results(lib, orc, cfg, rt):
    """A pinned split target (tl_run_set_launch_split) changes only how the
    mm_atb reductions are cut into work items (from 32 pieces of 64 rows to
    none, over the nano step's 2048-row dW reductions): the step still meets
    the bar against the oracle, and an eager step and a graph replay agree bit
    for bit."""
    host = tlgemm.host()
    plan = host.plan_train(**bench.TRAIN["nano"])
    run, stream = new_run(lib, host, plan, seed=cfg)
    try:
        L = host.dll.tl_run_grouped_launches(run)
        for k in range(L):
            assert host.dll.tl_run_set_launch_config(run, k, cfg) == 0
            assert host.dll.tl_run_set_launch_split(run, k, rt) == 0
        assert host.dll.tl_run_set_launch_split(run, 0, 63) != 0        # below the minimum
        assert host.dll.tl_run_launch_split(run, 0) == rt
        init = snapshot(lib, host, plan, run, stream)
        lib.check(host.dll.tl_run_step_grouped(run, stream), "step")
        got = snapshot(lib, host, plan, run, stream)
        fill(lib, host, plan, run, stream, cfg)
        lib.check(host.dll.tl_run_graph_build(run, stream, 1), "graph")
        fill(lib, host, plan, run, stream, cfg)
        lib.check(host.dll.tl_run_graph_step(run, stream), "replay")
        replay = snapshot(lib, host, plan, run, stream)
    finally:
        host.dll.tl_run_free(run)
    run_plan_cpu(plan, init, orc)
    for bname, _, _ in plan.bufs:
        assert np.array_equal(got[bname], replay[bname]), bname
        for label, a, b in plan.regions(bname):
            assert normwise_rel(got[bname][a:b], init[bname][a:b]) <= TOL, (cfg, rt, label)


@pytest.mark.parametrize("name", ["nano", "m3", "m8"])
def test_bench_tables_match_oracle(lib, orc, name):
    """The configuration bench.py measures: every grouped launch on the tile
    configuration and split target of bench.TUNED / bench.SPLITS; the step
    (eager and replayed from a graph) meets the bar against the oracle."""
    host = tlgemm.host()
    plan = host.plan_train(**bench.TRAIN[name])
    run, stream = new_run(lib, host, plan, seed=17)
    try:
        L = host.dll.tl_run_grouped_launches(run)
        assert len(bench.TUNED[name]) == L and len(bench.SPLITS[name]) == L
        for k in range(L):
            assert host.dll.tl_run_set_launch_config(run, k, bench.TUNED[name][k]) == 0
            assert host.dll.tl_run_set_launch_split(run, k, bench.SPLITS[name][k]) == 0
        init = snapshot(lib, host, plan, run, stream)
        lib.check(host.dll.tl_run_step_grouped(run, stream), "step")
        got = snapshot(lib, host, plan, run, stream)
        fill(lib, host, plan, run, stream, 17)
        lib.check(host.dll.tl_run_graph_build(run, stream, 1), "graph")
        fill(lib, host, plan, run, stream, 17)
        lib.check(host.dll.tl_run_graph_step(run, stream), "replay")
        replay = snapshot(lib, host, plan, run, stream)
    finally:
        host.dll.tl_run_free(run)
    run_plan_cpu(plan, init, orc)
    for bname, _, _ in plan.bufs:
        assert np.array_equal(got[bname], replay[bname]), bname
        for label, a, b in plan.regions(bname):
            assert normwise_rel(got[bname][a:b], init[bname][a:b]) <= TOL, (name, label)


def test_split_target_hook_rejects_small_targets(lib):
    assert lib.tlg_tune_group_split(63) != 0
    assert lib.tlg_tune_group_split(0) == 0


def test_autotuned_step_matches_oracle(lib, orc):
    """tl_run_autotune gives each grouped launch its own tile shape; the
    mixed step (eager and replayed from a graph) still meets the bar."""
    host = tlgemm.host()
    plan = host.plan_train(**bench.TRAIN["nano"])
    run, stream = new_run(lib, host, plan, seed=11)
    try:
        cands = (ctypes.c_int * 4)(3, 14, 15, 0)
        lib.check(host.dll.tl_run_autotune(run, cands, 4, 2, stream), "autotune")
        picks = [host.dll.tl_run_launch_config(run, k) for k in range(host.dll.tl_run_grouped_launches(run))]
        print("per-launch configs", picks, flush=True)
        assert all(p in (-1, 3, 14, 15, 0) for p in picks)
        fill(lib, host, plan, run, stream, 11)
        init = snapshot(lib, host, plan, run, stream)
        lib.check(host.dll.tl_run_step_grouped(run, stream), "step")
        got = snapshot(lib, host, plan, run, stream)
        fill(lib, host, plan, run, stream, 11)
        lib.check(host.dll.tl_run_graph_build(run, stream, 1), "graph")
        fill(lib, host, plan, run, stream, 11)
        lib.check(host.dll.tl_run_graph_step(run, stream), "replay")
        replay = snapshot(lib, host, plan, run, stream)
    finally:
        host.dll.tl_run_free(run)
    run_plan_cpu(plan, init, orc)
    for bname, _, _ in plan.bufs:
        assert np.array_equal(got[bname], replay[bname]), bname
        for label, a, b in plan.regions(bname):
            assert normwise_rel(got[bname][a:b], init[bname][a:b]) <= TOL, label
