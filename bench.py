#!/usr/bin/env python3
"""Benchmark of the fp32 GEMM hot path (tinylm.c's mm / mm_bt / mm_atb) on MI355X.

A "step" is one pass of the reference's GEMM call sequence over one batch:
for the default workload ("m3"), every forward and
backward projection GEMM of a 6-layer training step on 4096 rows plus the
tied-unembedding head (129 GEMMs, 124.0 GFLOP), in the order and with the
operands tinylm.c's forward/backward use (tinylm-c_amd/host/tl_plan.c),
issued through libtlgemm's C ABI on device-resident buffers (replayed as one
HIP graph).  Inputs are synthetic seeded Gaussians (X ~ N(0,1),
W ~ N(0,0.02^2), dY ~ N(0,0.01^2)) already in HBM when timing starts.

Prints one JSON line: train tokens/s (value), the dominant kernel's roofline,
the decode GEMV figures at M = 1, 2, 4, 8, the top-1
MoE layer, the whole device-resident training step (forward +
backward + AdamW at the same model shape, "train_step"), the achievable
copy / MFMA peaks of this box, and the CPU baseline -- the reference's own
kernels and whole step (oracle/_ref) timed on this host on a bounded sample.
"""
import argparse
import ctypes
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(REPO, "tinylm-c_amd"), os.path.join(REPO, "oracle")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_FP32_MFMA_TFLOPS = 157.3      # MI355X dense fp32 matrix peak
PEAK_HBM_GBS = 8000.0              # MI355X HBM3E
RIDGE = PEAK_FP32_MFMA_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)   # flop per byte

# BASELINE.json configs (reference argument labels, tinylm.c:361-393 layout)
TRAIN = {
    "nano": dict(R=2048, D=128, KD=32, F=384, V=2048, L=1, n_mtp=0),
    "m3": dict(R=4096, D=256, KD=64, F=768, V=2048, L=6, n_mtp=0),
    "m8": dict(R=8192, D=384, KD=96, F=1024, V=2048, L=8, n_mtp=2),
}
DECODE = dict(D=384, KD=96, F=1024, V=2048, L=8)
# top-1 MoE at m3 scale; the router rows are tilted so the
# experts receive about 50 / 22 / 17 / 11 % of the tokens
MOE = dict(N=4096, D=256, F=768, E=4)
ROUTER_TILT = (1.0, 0.5, 0.2, 0.0)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def check(rc, what):
    if rc != 0:
        import tlgemm
        raise RuntimeError(f"{what} failed ({rc}): {tlgemm.load().tlg_last_error().decode()}")


def roofline_class(flops, nbytes):
    return "mfma" if flops / max(nbytes, 1.0) >= RIDGE else "hbm"


def warm_for(lib, fn, stream, seconds=0.1, label="warmup"):
    """Untimed steps for about `seconds` of GPU work (at least 8), so the
    clocks have ramped before a phase's timed region."""
    t0, n = time.perf_counter(), 0
    while n < 8 or time.perf_counter() - t0 < seconds:
        for _ in range(8):
            check(fn(), label)
        n += 8
        check(lib.tlg_stream_sync(stream), "sync")
    return n


def time_steps(lib, fn, stream, n):
    e0, e1 = lib.tlg_event_create(), lib.tlg_event_create()
    check(lib.tlg_stream_sync(stream), "sync")
    t0 = time.perf_counter()
    check(lib.tlg_event_record(e0, stream), "event")
    for _ in range(n):
        check(fn(), "step")
    check(lib.tlg_event_record(e1, stream), "event")
    check(lib.tlg_stream_sync(stream), "sync")
    wall = time.perf_counter() - t0
    ms = lib.tlg_event_elapsed_ms(e0, e1)
    lib.tlg_event_destroy(e0)
    lib.tlg_event_destroy(e1)
    return ms, wall


def kernel_census(lib, host, plan, run, stream, reps):
    """Average launch duration per kernel instance, from HIP events on the
    stream the kernels run on: each GEMM call of the step is launched `reps`
    times back to back between two events."""
    import tlgemm  # noqa: F401
    ev = [lib.tlg_event_create() for _ in range(2 * len(plan.calls))]
    for i, c in enumerate(plan.calls):
        if c["op"] == "zero":
            continue
        check(lib.tlg_event_record(ev[2 * i], stream), "event")
        for _ in range(reps):
            check(host.dll.tl_run_call(run, i, stream), "call")
        check(lib.tlg_event_record(ev[2 * i + 1], stream), "event")
    check(lib.tlg_stream_sync(stream), "sync")
    groups = {}
    for i, c in enumerate(plan.calls):
        if c["op"] == "zero":
            continue
        ms = lib.tlg_event_elapsed_ms(ev[2 * i], ev[2 * i + 1]) / reps
        name, splits = lib.kernel_name(c["op"], c["M"], c["K"], c["N"])
        g = groups.setdefault(name, dict(launches=0, ms=0.0, flops=0.0, bytes=0.0, shapes=set()))
        M, K, N = c["M"], c["K"], c["N"]
        g["launches"] += 1
        g["ms"] += ms
        g["flops"] += 2.0 * M * K * N
        acc = c["op"] != "mm"
        out = M * N if c["op"] == "mm" else (M * K if c["op"] == "mm_bt" else K * N)
        ins = {"mm": M * K + K * N, "mm_bt": M * N + K * N, "mm_atb": M * K + M * N}[c["op"]]
        g["bytes"] += 4.0 * (ins + out * (2 if acc else 1))
        g["shapes"].add(f"{c['op']}({M},{K},{N})x{splits}")
    for e in ev:
        lib.tlg_event_destroy(e)
    return groups


def launch_census(lib, host, run, stream, reps):
    """Average duration of each launch of a grouped step, from HIP events the
    executor records on the kernels' stream before every launch (reps steps),
    summed per kernel instance."""
    L = host.dll.tl_run_grouped_launches(run)
    ev = [lib.tlg_event_create() for _ in range(L + 2)]
    arr = (ctypes.c_void_p * (L + 2))(*ev)
    dt = [0.0] * (L + 1)
    for _ in range(reps):
        check(host.dll.tl_run_time_launches(run, arr, L + 2, stream), "timed step")
        check(lib.tlg_stream_sync(stream), "sync")
        for k in range(L + 1):
            dt[k] += lib.tlg_event_elapsed_ms(ev[k], ev[k + 1]) / reps
    groups = {}
    fl, by = ctypes.c_double(), ctypes.c_double()
    table = []
    for k in range(L + 1):
        kind = host.dll.tl_run_launch_info(run, k, ctypes.byref(fl), ctypes.byref(by))
        kname = host.dll.tl_run_launch_kernel(run, k)
        table.append((k, kind, fl.value, by.value, dt[k]))
        if kname is None:
            continue                      # a flush with no split partials: nothing launched
        name = kname.decode()
        g = groups.setdefault(name, dict(launches=0, ms=0.0, flops=0.0, bytes=0.0, shapes=set()))
        g["launches"] += 1
        g["ms"] += dt[k]
        g["flops"] += fl.value
        g["bytes"] += by.value
        g["shapes"].add({0: "grouped GEMMs", 1: "clear", 2: "split flush"}[kind])
    for e in ev:
        lib.tlg_event_destroy(e)
    if os.environ.get("TLG_BENCH_LAUNCHES"):
        for k, kind, f, b, ms in table:
            log(f"[launch {k:3d}] kind {kind} {f / 1e9:7.3f} GF {b / 1e6:8.2f} MB {ms * 1e3:8.2f} us "
                f"{f / (ms * 1e-3) / 1e12 if ms > 0 else 0:6.1f} TF")
    return groups


def read_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed PMC summary
    (profiles/traffic_m3.txt: FETCH_SIZE + WRITE_SIZE per dispatch, scaled by
    the copy-kernel calibration), or None if not measured."""
    path = os.path.join(REPO, "profiles", "traffic_m3.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        parts = line.strip().split("\t")
        if len(parts) >= 2 and parts[0] == kernel:
            try:
                return float(parts[1])
            except ValueError:
                return None
    return None


def read_profile_row(fname, kernel):
    """The tab-separated fields after `kernel` in a committed profiles/ summary
    (its machine-readable tail), or None."""
    path = os.path.join(REPO, "profiles", fname)
    if not os.path.exists(path):
        return None
    for line in open(path):
        parts = line.rstrip("\n").split("\t")
        if len(parts) >= 2 and parts[0] == kernel:
            return parts[1:]
    return None


def read_rocprof_avg_us(kernel):
    """rocprofv3's average duration of `kernel` in the committed m3 kernel
    trace (profiles/m3_step_kernel_trace.md, the stats table), or None."""
    path = os.path.join(REPO, "profiles", "m3_step_kernel_trace.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        cells = [c.strip() for c in line.split("|")]
        if len(cells) > 4 and cells[1].strip("`") == "void " + kernel:
            try:
                return float(cells[3])
            except ValueError:
                return None
    return None


AUTOTUNE_CANDS = (3, 14, 13, 15, 0, 1, 20, 21, 22, 23, 24, 26, 27, 28, 29, 30, 31, 32, 33, 34, 35, 36, 37,
                  38, 39, 40, 41, 42, 43, 44, 45, 46, 47, 48, 49, 50)
# split targets tried with each tile candidate (tlg_tune_group_split: reduction
# steps per split work item of the mm_atb problems; 0 = the library's rule)
AUTOTUNE_RTS = (0, 256, 512, 1024, 2048, 4096)

# Tile configuration and split target of every grouped launch of each training
# step: per launch the configuration tl_run_autotune_split chose most often
# over 3 timing runs on an MI355X (10 timed steps per (configuration, split
# target) pair, split targets 0, 256, 512, 1024, 2048 and 4096; ties to the
# fastest run), and the split target those runs chose most often with it.  A
# split target only changes launches with mm_atb problems (the backward ones);
# elsewhere it is whatever the timing noise picked.  A fixed table keeps the
# step's kernels -- and so the roofline kernel and its rocprofv3 profiles --
# the same from box to box; --autotune re-times the candidates instead.
TUNED = {
    "nano": [30, 15, 44, 15, 39, 44, 15, 44, 30, 30],
    "m3": [40, 41, 39, 22, 40, 41, 39, 22, 40, 41, 39, 41, 40, 41, 39, 41, 40, 41, 39, 41, 40, 41, 39, 41, 38, 38, 38, 38, 44, 39, 24, 38, 13, 38, 24, 38, 13, 38, 24, 38, 44, 39, 24, 38, 44, 39, 38, 24, 13, 38],
    "m8": [40, 39, 45, 42, 40, 38, 45, 38, 40, 38, 45, 42, 40, 38, 45, 38, 40, 38, 45, 38, 40, 38, 45, 38, 40, 38, 45, 38, 40, 38, 45, 38, 0, 38, 38, 39, 37, 38, 39, 38, 38, 38, 45, 39, 39, 38, 45, 39, 38, 38, 45, 39, 39, 24, 38, 39, 24, 38, 45, 39, 39, 38, 38, 39, 39, 38, 45, 39, 38, 38, 45, 39],
}
# (0 = the library's automatic rule)
SPLITS = {
    "nano": [1024, 256, 1024, 1024, 2048, 1024, 0, 256, 256, 256],
    "m3": [1024, 256, 512, 1024, 1024, 0, 1024, 256, 512, 512, 1024, 512, 512, 512, 512, 512, 1024, 256, 1024, 0, 2048, 512, 1024, 512, 512, 1024, 0, 512, 1024, 512, 512, 512, 0, 512, 512, 512, 0, 512, 512, 512, 1024, 512, 512, 512, 1024, 256, 512, 512, 0, 512],
    "m8": [2048, 256, 1024, 512, 256, 512, 1024, 2048, 2048, 512, 1024, 512, 4096, 2048, 1024, 1024, 2048, 512, 1024, 2048, 4096, 1024, 1024, 1024, 256, 512, 0, 2048, 2048, 1024, 0, 1024, 512, 2048, 512, 1024, 1024, 2048, 1024, 256, 1024, 1024, 256, 1024, 1024, 2048, 256, 1024, 2048, 1024, 256, 1024, 1024, 2048, 256, 1024, 1024, 2048, 256, 1024, 1024, 2048, 256, 1024, 1024, 1024, 256, 1024, 1024, 2048, 256, 1024],
}


def apply_tiles(lib, host, run, stream, name, retime=False, reps=3):
    """Set each grouped launch's tile configuration and split target (the
    TUNED and SPLITS tables, or a fresh timing when retime or a table does
    not fit); returns {config: launches}."""
    L = host.dll.tl_run_grouped_launches(run)
    table, splits = TUNED.get(name), SPLITS.get(name)
    if retime or table is None or len(table) != L or splits is None or len(splits) != L:
        arr = (ctypes.c_int * len(AUTOTUNE_CANDS))(*AUTOTUNE_CANDS)
        rts = (ctypes.c_int * len(AUTOTUNE_RTS))(*AUTOTUNE_RTS)
        check(host.dll.tl_run_autotune_split(run, arr, len(AUTOTUNE_CANDS), rts, len(AUTOTUNE_RTS), reps, stream),
              "autotune")
    else:
        for k, (c, rt) in enumerate(zip(table, splits)):
            check(host.dll.tl_run_set_launch_config(run, k, c), "set tile config")
            check(host.dll.tl_run_set_launch_split(run, k, rt), "set split target")
    picks = {}
    for k in range(L):
        c = host.dll.tl_run_launch_config(run, k)
        picks[c] = picks.get(c, 0) + 1
    return picks


def roof_time_ms(plan):
    """Summed per-GEMM roofline time of a step: max(flops / MFMA peak,
    compulsory bytes / HBM peak) per call, clears at HBM speed."""
    roof_ms = 0.0
    for c in plan.calls:
        if c["op"] == "zero":
            roof_ms += 4.0 * c["n"] / (PEAK_HBM_GBS * 1e9) * 1e3
            continue
        M, K, N = c["M"], c["K"], c["N"]
        fl = 2.0 * M * K * N
        out = M * N if c["op"] == "mm" else (M * K if c["op"] == "mm_bt" else K * N)
        ins = {"mm": M * K + K * N, "mm_bt": M * N + K * N, "mm_atb": M * K + M * N}[c["op"]]
        by = 4.0 * (ins + out * (1 if c["op"] == "mm" else 2))
        roof_ms += max(fl / (PEAK_FP32_MFMA_TFLOPS * 1e12), by / (PEAK_HBM_GBS * 1e9)) * 1e3
    return roof_ms


def bench_train_config(lib, host, stream, name, steps, tune=True, retime=False):
    """Another BASELINE training config (nano = configs[0], m8 = configs[2]):
    the same grouped, graph-replayed GEMM step."""
    cfg = TRAIN[name]
    plan = host.plan_train(**cfg)
    run = host.dll.tl_run_new(ctypes.byref(plan.raw), 1)
    if not run:
        raise RuntimeError("tl_run_new failed: " + lib.tlg_last_error().decode())
    check(host.dll.tl_run_fill(run, 1234567891011, stream), "fill")
    tuned = apply_tiles(lib, host, run, stream, name, retime) if tune else None
    check(host.dll.tl_run_graph_build(run, stream, 1), "graph build")
    step = lambda: host.dll.tl_run_graph_step(run, stream)  # noqa: E731
    warm_for(lib, step, stream)
    ms, _ = time_steps(lib, step, stream, steps)
    per = ms / steps
    roof = roof_time_ms(plan)
    launches = host.dll.tl_run_grouped_launches(run)
    host.dll.tl_run_free(run)
    return {
        "calls": len(plan.calls), "grouped_launches": launches, "gflop": round(plan.flops() / 1e9, 2),
        "steps": steps, "ms_per_step": round(per, 4), "tok_s": round(cfg["R"] / (per * 1e-3), 1),
        "tflops": round(plan.flops() / (per * 1e-3) / 1e12, 2),
        "sum_of_gemm_roof_ms": round(roof, 4), "roof_frac": round(roof / per, 4),
        "tile_configs": tuned,
    }


def bench_decode(lib, host, stream, steps, M=1, pool=6, packed=False, eager=False):
    """cfg3: per token 8 layers x 7 GEMVs + unembed at M rows, one grouped
    launch per GEMV run (q/k/v, o, w1/w3, w2, head: the reference runs glue
    between them); the weights (52.7 MB) rotate through `pool` copies
    (> 256 MB Infinity Cache).  packed: the decode layout (every linear
    weight stored transposed, each mm as memset + mm_bt), as the device
    decoder keeps its weights.  Steps are replayed from a HIP graph."""
    plan = host.plan_decode(M, packed=packed, **DECODE)
    run = host.dll.tl_run_new(ctypes.byref(plan.raw), pool)
    if not run:
        raise RuntimeError("tl_run_new(decode) failed")
    check(host.dll.tl_run_fill(run, 7, stream), "fill")
    if eager:                       # launch by launch (profilers trace these)
        step = lambda: host.dll.tl_run_step_grouped(run, stream)  # noqa: E731
    else:
        check(host.dll.tl_run_graph_build(run, stream, 1), "decode graph")
        step = lambda: host.dll.tl_run_graph_step(run, stream)  # noqa: E731
    warm_for(lib, step, stream, label="decode warmup")    # every weight copy, many times over
    ms, _ = time_steps(lib, step, stream, steps)
    launches = host.dll.tl_run_grouped_launches(run)
    wbytes = sum(4.0 * c["K"] * c["N"] for c in plan.calls if c["op"] != "zero")
    # weights, the activation rows in, the output rows out (a clear folded
    # into the GEMV makes every output a set)
    allbytes = sum(4.0 * (c["K"] * c["N"] + c["M"] * (c["K"] + c["N"])) for c in plan.calls if c["op"] != "zero")
    per_tok_ms = ms / steps
    host.dll.tl_run_free(run)
    return {
        "rows": M, "steps": steps, "us_per_step": round(per_tok_ms * 1e3, 3),
        "tok_s": round(M * 1e3 / per_tok_ms, 1),
        "weight_bytes_per_step": int(wbytes),
        "hbm_gbs": round(allbytes / (per_tok_ms * 1e-3) / 1e9, 1),
        "hbm_frac": round(allbytes / (per_tok_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
        "gemv_calls_per_step": sum(1 for c in plan.calls if c["op"] != "zero"),
        "launches_per_step": launches,
        "weight_pool_copies": pool,
        "layout": "decode (W^T, mm_bt form)" if packed else "reference (W [in][out], mm)",
        "launch": "launch by launch" if eager else "one HIP graph per step",
    }


def bench_moe(lib, stream, steps):
    """tlg_dev_moe_grouped_fwd + _bwd (tinylm.c:857-947) on 4096
    tokens, 4 experts 256 -> 768 -> 256, skewed routing; seeded inputs
    uploaded once, timed fwd+bwd pairs on device-resident buffers."""
    import numpy as np
    N, D, F, E = MOE["N"], MOE["D"], MOE["F"], MOE["E"]
    rng = np.random.default_rng(4)
    fnorm = rng.standard_normal((N, D), dtype=np.float32)
    fnorm[:, 0] = np.abs(fnorm[:, 0]) + 1.0
    wr = (0.1 * rng.standard_normal((D, E))).astype(np.float32)
    wr[0, :] += np.array(ROUTER_TILT, np.float32)
    host = {
        "fnorm": fnorm, "fin": rng.standard_normal((N, D), dtype=np.float32), "wr": wr,
        "w1": (0.02 * rng.standard_normal((E, D, F))).astype(np.float32),
        "w3": (0.02 * rng.standard_normal((E, D, F))).astype(np.float32),
        "w2": (0.02 * rng.standard_normal((E, F, D))).astype(np.float32),
        "dout": (0.01 * rng.standard_normal((N, D))).astype(np.float32),
    }
    dev = {}
    for k, a in host.items():
        dev[k] = lib.tlg_dev_malloc(a.nbytes)
        check(lib.tlg_memcpy_h2d(dev[k], a.ctypes.data, a.nbytes, stream), "upload")
    for k, n in (("out", N * D), ("assign", N), ("gate", N), ("rprobs", N * E), ("dfn", N * D),
                 ("gwr", D * E), ("gw1", E * D * F), ("gw3", E * D * F), ("gw2", E * F * D)):
        dev[k] = lib.tlg_dev_malloc(4 * n)
        check(lib.tlg_dev_zero(dev[k], n, stream), "zero")
    d = dev

    def step():
        rc = lib.tlg_dev_moe_grouped_fwd(d["fnorm"], d["fin"], d["out"], N, D, F, E, d["wr"], d["w1"], d["w3"],
                                         d["w2"], d["assign"], d["gate"], d["rprobs"], stream)
        return rc or lib.tlg_dev_moe_grouped_bwd(d["fnorm"], d["dout"], d["dfn"], d["assign"], d["gate"],
                                                 d["rprobs"], N, D, F, E, d["wr"], d["w1"], d["w3"], d["w2"],
                                                 d["gwr"], d["gw1"], d["gw3"], d["gw2"], stream)
    warm_for(lib, step, stream, label="moe warmup")
    ms, _ = time_steps(lib, step, stream, steps)
    # the same pair from a kept forward state (tlg_dev_moe_grouped_fwd_keep /
    # _bwd_kept: no index rebuild, no W1 | W3 and W2 recompute in the backward)
    kb = lib.tlg_moe_keep_bytes(N, D, F, E)
    dev["keep"] = lib.tlg_dev_malloc(kb)

    def step_kept():
        rc = lib.tlg_dev_moe_grouped_fwd_keep(d["fnorm"], d["fin"], d["out"], N, D, F, E, d["wr"], d["w1"],
                                              d["w3"], d["w2"], d["assign"], d["gate"], d["rprobs"], d["keep"], kb,
                                              stream)
        return rc or lib.tlg_dev_moe_grouped_bwd_kept(d["fnorm"], d["dout"], d["dfn"], d["assign"], d["gate"],
                                                      d["rprobs"], N, D, F, E, d["wr"], d["w1"], d["w3"], d["w2"],
                                                      d["gwr"], d["gw1"], d["gw3"], d["gw2"], d["keep"], kb, stream)
    warm_for(lib, step_kept, stream, label="moe kept warmup")
    ms_k, _ = time_steps(lib, step_kept, stream, steps)
    # the kept backward leaves dWr's column sum and the dW1 / dW3 slice sums
    # queued (they read the kept index and write gwr, gw1, gw3): run them
    # before those buffers are freed
    check(lib.tlg_dev_gemm_flush(stream), "flush")
    assign = np.empty(N, np.int32)
    check(lib.tlg_memcpy_d2h(assign.ctypes.data, d["assign"], assign.nbytes, stream), "download")
    check(lib.tlg_stream_sync(stream), "sync")
    for v in dev.values():
        lib.tlg_dev_free(v)
    unit = 2.0 * N * D * F                      # one expert GEMM over all N rows
    router = 3 * 2.0 * N * D * E
    algo = 9 * unit + router                    # fwd 3 + bwd 6 expert GEMMs
    executed = 12 * unit + router               # + the recomputed forward (tinylm.c:911-914)
    per = ms / steps
    return {
        "workload": f"configs[4]: {N} tokens, D={D}, E={E} experts F={F}, top-1, fwd+bwd",
        "steps": steps, "ms_per_step": round(per, 4), "tok_s": round(N / (per * 1e-3), 1),
        "expert_rows": np.bincount(assign, minlength=E).tolist(),
        "gflop_algorithmic": round(algo / 1e9, 3), "gflop_executed": round(executed / 1e9, 3),
        "tflops_algorithmic": round(algo / (per * 1e-3) / 1e12, 2),
        "tflops_executed": round(executed / (per * 1e-3) / 1e12, 2),
        "kept_state": {
            "entries": "tlg_dev_moe_grouped_fwd_keep + tlg_dev_moe_grouped_bwd_kept (same results bit for bit)",
            "ms_per_step": round(ms_k / steps, 4), "tok_s": round(N / (ms_k / steps * 1e-3), 1),
            "keep_bytes": kb, "tflops_algorithmic": round(algo / (ms_k / steps * 1e-3) / 1e12, 2),
        },
    }


def probes(lib, stream):
    """Achievable peaks on this box: a streaming copy (k_copy, 1 GiB each
    way), a streaming read (k_read, 1 GiB) and register-only fp32 MFMA
    (k_mfma_peak)."""
    n = 1 << 28
    src, dst = lib.tlg_dev_malloc(4 * n), lib.tlg_dev_malloc(4 * n)
    check(lib.tlg_dev_fill_normal(src, n, 3, 1.0, stream), "fill")
    for _ in range(2):
        check(lib.tlg_dev_copy(dst, src, n, stream), "copy")
    ms, _ = time_steps(lib, lambda: lib.tlg_dev_copy(dst, src, n, stream), stream, 5)
    hbm = 2 * 4.0 * n / (ms / 5 * 1e-3) / 1e9
    for _ in range(2):
        check(lib.tlg_dev_read(src, n, dst, stream), "read")
    ms_r, _ = time_steps(lib, lambda: lib.tlg_dev_read(src, n, dst, stream), stream, 5)
    hbm_read = 4.0 * n / (ms_r / 5 * 1e-3) / 1e9
    blocks, iters = 2048, 2000
    check(lib.tlg_dev_mfma_peak(dst, blocks, iters, stream), "mfma")
    ms2, _ = time_steps(lib, lambda: lib.tlg_dev_mfma_peak(dst, blocks, iters, stream), stream, 5)
    mfma = blocks * 4 * 4 * iters * 4096.0 / (ms2 / 5 * 1e-3) / 1e12
    lib.tlg_dev_free(src)
    lib.tlg_dev_free(dst)
    return {"hbm_copy_gbs": round(hbm, 1), "hbm_read_gbs": round(hbm_read, 1), "copy_bytes_each_way": 4 * n,
            "mfma_fp32_tflops": round(mfma, 1)}


def host_cpu_share():
    """Threads for the CPU baseline: the physical cores this process may run
    on (distinct (package, core) pairs of its affinity set, so no two threads
    share a core's SMT siblings), capped by the box's CPU share for one GPU
    when OMP_NUM_THREADS states it (16 on the GPU boxes).  Returns (threads,
    facts about the host) -- read at run time, printed in the report."""
    cpus = sorted(os.sched_getaffinity(0))
    cores = set()
    for c in cpus:
        base = f"/sys/devices/system/cpu/cpu{c}/topology/"
        try:
            with open(base + "physical_package_id") as f:
                pkg = f.read().strip()
            with open(base + "core_id") as f:
                core = f.read().strip()
            cores.add((pkg, core))
        except OSError:
            cores.add(("?", str(c)))
    phys = len(cores)
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    threads = min(phys, share) if share > 0 else phys
    return max(threads, 1), {"affinity_cpus": len(cpus), "physical_cores": phys,
                             "omp_num_threads_env": share or None}


CPU_FLAGS = ("gcc -O3 -march=x86-64-v3 -ffast-math -funroll-loops -fopenmp -flto (the reference's portable "
             "flags; x86-64-v3: 256-bit AVX2 vectors, as -mprefer-vector-width=256)")


def median_time(fn, reps, warmup=2):
    """2 untimed warmups (as cmd_bench, tinylm.c:4732), then the median of
    `reps` timed runs, in seconds."""
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2], ts


def cpu_baseline(host, cfgname, reps, threads, facts):
    """The build's CPU restatement of mm / mm_bt / mm_atb (oracle/liboracle:
    the reference's blocking and FMA chains, bit-identical to tinylm.c's own
    kernels on the committed fixtures) running the whole plan on host cores,
    OpenMP static over the reference's 4-row blocks (tinylm.c:447-448, :515)."""
    import numpy as np
    import oracle
    prims = oracle.Oracle()
    prims.set_pool(1)
    prims.set_threads(threads)
    cfg = TRAIN[cfgname]
    plan = host.plan_train(**cfg)
    rng = np.random.default_rng(5)
    scale = {0: 1.0, 1: 0.02, 2: 0.01, 3: 0.0}
    arrays = {}
    for name, n, init in plan.bufs:
        a = rng.standard_normal(n, dtype=np.float32) if init != 3 else np.zeros(n, np.float32)
        if init != 3:
            a *= np.float32(scale[init])
        arrays[name] = a
    calls = oracle.plan_calls_native(plan, arrays)
    dt, ts = median_time(lambda: prims.run_calls(calls, 1), reps)
    return {
        "value": round(cfg["R"] / dt, 1), "unit": "train tokens/s (GEMM set only)",
        "cores": threads, "kind": "port", "host": facts,
        "sample": f"median of {reps} full {cfgname} GEMM-set steps "
                  f"({sum(1 for c in plan.calls if c['op'] != 'zero')} calls each, the plan looped in C) after 2 "
                  f"warmups, OpenMP static on {threads} threads pinned one per physical core; {CPU_FLAGS}; "
                  f"{sum(ts):.1f} s timed",
        "s_per_step": round(dt, 4),
    }


def cpu_decode_baseline(host, M, steps, threads):
    """configs[3] decode GEMVs on the host with the restatement, one weight
    copy (cache-resident, as the reference's own decode runs), the call list
    looped in C, two dispatches: "as_dispatched" is the reference's decode
    rule with its worker pool live (tl_for runs a range of fewer items than
    workers on the caller, tinylm.c:237-239, so mm at M <= 8 (:444-446) and
    mm_bt at M = 1 (:486) run serially); "threaded" splits each GEMV's
    outputs over the OpenMP threads (not what the reference does; the same
    per-element chains)."""
    import numpy as np
    import oracle
    prims = oracle.Oracle()
    prims.set_threads(threads)
    plan = host.plan_decode(M, **DECODE)
    rng = np.random.default_rng(6)
    arrays = {}
    for name, n, init in plan.bufs:
        a = rng.standard_normal(n, dtype=np.float32) if init != 3 else np.zeros(n, np.float32)
        if init == 1:
            a *= np.float32(0.02)
        arrays[name] = a
    calls = oracle.plan_calls_native(plan, arrays)
    out = {"rows": M, "kind": "port", "gemvs_per_step": sum(1 for c in plan.calls if c["op"] != "zero")}
    for label, pool, split, nthr in (("as_dispatched", threads, 0, threads), ("threaded", 1, 1, threads)):
        prims.set_pool(pool)
        prims.dll.orc_set_gemv_split(split)
        try:
            dt, ts = median_time(lambda: prims.run_calls(calls, steps), 5)
        finally:
            prims.set_pool(1)
            prims.dll.orc_set_gemv_split(0)
        out[label] = {"us_per_step": round(dt / steps * 1e6, 1), "tok_s": round(M * steps / dt, 1),
                      "cores": 1 if label == "as_dispatched" else nthr,
                      "sample": f"median of 5 runs of {steps} decode steps after 2 warmups ({sum(ts):.2f} s)"}
    return out


def model_of(name):
    """The TRAIN config as a whole model (head_dim 32, T = 256)."""
    cfg = TRAIN[name]
    return dict(V=cfg["V"], D=cfg["D"], L=cfg["L"], H=cfg["D"] // 32, KV=cfg["KD"] // 32, F=cfg["F"], T=256,
                n_mtp=cfg["n_mtp"]), cfg["R"] // 256


def bench_full_step(lib, host, stream, name, steps, warmup=3, eager=False, tune=True):
    """The whole training step on the device (host/tl_train.h): forward,
    backward with the MTP heads, gradnorm and AdamW -- tinylm.c's
    train_loop body (:2627-2633), every activation resident in HBM --
    replayed as one HIP graph.  Weights ~ N(0, 0.02^2) drawn on the device,
    random tokens."""
    import numpy as np
    kw, B = model_of(name)
    tr = host.train(kw, B)
    check(lib.tlg_dev_fill_normal(tr.buf(0), tr.np, 99, 0.02, stream), "fill P")
    rng = np.random.default_rng(3)
    N = B * kw["T"]
    tok, tgt = (rng.integers(0, kw["V"], N).astype(np.int32) for _ in range(2))
    tm = rng.integers(0, kw["V"], (max(kw["n_mtp"], 1), N)).astype(np.int32) if kw["n_mtp"] else None
    tr.set_batch(tok, tgt, tm, stream)
    tr.set_hyper(3e-4, 0.9, 0.95, 0.1, 1, stream)
    tr.step(stream)                                   # sizes every scratch buffer
    loss0 = tr.loss(stream)
    # per grouped launch, the fastest tile configuration (forward + backward
    # passes only: the parameters stay as the first step left them)
    tiles = tr.autotune(list(AUTOTUNE_CANDS), 3, stream, AUTOTUNE_RTS) if tune else None
    splits = tr.splits() if tune else None
    phases = tr.time_phases(stream)
    if eager:                                       # kernel by kernel (profilers trace these)
        run = lambda: tr.step(stream)  # noqa: E731
    else:
        tr.graph_build(stream)
        run = lambda: tr.graph_step(stream)  # noqa: E731
    for _ in range(warmup):
        run()
    check(lib.tlg_stream_sync(stream), "sync")
    ms, _ = time_steps(lib, run, stream, steps)
    loss1 = tr.loss(stream)
    ms_step = ms / steps
    tr.close()
    return {"model": kw, "batch": B, "rows": N, "params": tr.np, "steps": steps,
            "ms_per_step": round(ms_step, 4), "tok_s": round(N / (ms_step / 1e3), 1),
            "phases_ms_eager": {"forward": round(phases[0], 4), "backward": round(phases[1], 4),
                                "gradnorm_adamw": round(phases[2], 4)},
            "loss_first": round(loss0, 4), "loss_after": round(loss1, 4),
            "launch": "enqueued step by step" if eager else "one HIP graph per step",
            "tiles": ("per grouped launch, tl_train_autotune_split over " + str(list(AUTOTUNE_CANDS)) + " x split "
                      "targets " + str(list(AUTOTUNE_RTS)) + ": " + str(tiles) + ", targets " + str(splits))
                     if tune else "the library's automatic policy"}


DECODE_MODEL = dict(V=2048, D=384, L=8, H=12, KV=3, F=1024, T=256)


def bench_decode_step(lib, host, stream, steps, pool=6, prompt_len=16, warmup=8, fused=1, eager=False):
    """The whole decode step on the device (host/tl_decode.h): greedy
    single-token steps of the m8 model through a 256-position f16 KV ring
    with the reference's fast_expf (its decode defaults), token and position
    kept in device memory, one captured graph per weight copy; `pool` copies
    rotate so the 52.7 MB of weights stream from HBM.  Weights ~ N(0, 0.02^2)
    drawn on the device."""
    import numpy as np
    maxpos = prompt_len + warmup + steps + 8
    dec = host.decode(DECODE_MODEL, 256, kv_f16=1, exact_exp=0, maxpos=maxpos, mmax=8, pool=pool)
    dec.set_fused(fused)
    for c in range(pool):
        check(lib.tlg_dev_fill_normal(dec.params(c), dec.np, 77, 0.02, stream), "fill P")
    dec.pack(stream)
    dec.reset(stream)
    prompt = np.random.default_rng(5).integers(0, DECODE_MODEL["V"], prompt_len).astype(np.int32)
    t0 = time.perf_counter()
    dec.prime(prompt, stream)
    prefill_ms = (time.perf_counter() - t0) * 1e3
    if eager:                       # launch by launch (profilers trace these), copies rotating
        cnt = [0]

        def step():
            cnt[0] += 1
            return dec.greedy_step(stream, (cnt[0] - 1) % pool)
    else:
        dec.graph_build(stream)
        step = lambda: dec.graph_step(stream)  # noqa: E731
    for _ in range(warmup):
        step()
    check(lib.tlg_stream_sync(stream), "sync")
    ms, _ = time_steps(lib, step, stream, steps)
    state = dec.state(stream)
    per = ms / steps
    dec.close()
    return {"model": DECODE_MODEL, "kv_cache": "f16 ring, 256 positions", "exp": "fast_expf",
            "weights_pool": pool, "steps": steps, "ms_per_token": round(per, 4),
            "tok_s": round(1e3 / per, 1), "prefill_ms_host_timed": round(prefill_ms, 3),
            "final_position": state[0], "fused": bool(fused),
            "launch": "enqueued step by step" if eager else "one HIP graph per step",
            "launches_per_token": 1 + 8 * 5 + 2 if fused else 1 + 8 * 13 + 3}


def bench_decode_persist(lib, host, stream, steps, pool=6, prompt_len=16, warmup=16):
    """The same greedy decode as bench_decode_step, run by the persistent
    kernel (tl_decode_persist: every token of the timed run in ONE cooperative
    launch, workgroups exchanging each phase's outputs through memory); the
    weight copies rotate per token, so the weights stream from HBM."""
    import numpy as np
    maxpos = prompt_len + warmup + steps + 8
    dec = host.decode(DECODE_MODEL, 256, kv_f16=1, exact_exp=0, maxpos=maxpos, mmax=8, pool=pool)
    for c in range(pool):
        check(lib.tlg_dev_fill_normal(dec.params(c), dec.np, 77, 0.02, stream), "fill P")
    dec.pack(stream)
    dec.reset(stream)
    prompt = np.random.default_rng(5).integers(0, DECODE_MODEL["V"], prompt_len).astype(np.int32)
    dec.prime(prompt, stream)
    dec.persist(warmup, stream)
    dec.persist_status(stream)
    ms, _ = time_steps(lib, lambda: dec.persist(steps, stream), stream, 1)
    dec.persist_status(stream)
    state = dec.state(stream)
    per = ms / steps
    wbytes = 4 * (DECODE_MODEL["V"] * 384 + 8 * (384 * 384 * 2 + 2 * 384 * 96 + 3 * 384 * 1024))
    dec.close()
    return {"model": DECODE_MODEL, "kv_cache": "f16 ring, 256 positions", "exp": "fast_expf",
            "weights_pool": pool, "steps": steps, "launches": 1, "ms_per_token": round(per, 4),
            "tok_s": round(1e3 / per, 1), "weight_bytes_per_token": wbytes,
            "weight_gbs": round(wbytes / (per * 1e-3) / 1e9, 1),
            "hbm_frac": round(wbytes / (per * 1e-3) / 8e12, 4), "final_position": state[0]}


def bench_decode_chunks(lib, host, stream, M, positions=512, pool=6, prompt_len=16):
    """configs[3] at M rows: forward_chunk over `positions` given tokens in
    chunks of M rows (prefill / speculative verification), every chunk of the
    timed run in ONE persistent launch (tl_decode_chunks); the weight copies
    rotate per chunk, so each chunk streams the 52.7 MB of weights from HBM
    once for its M tokens."""
    import numpy as np
    n = positions // M
    warm = max(1, 64 // M)
    maxpos = prompt_len + (warm + n) * M + 8
    dec = host.decode(DECODE_MODEL, 256, kv_f16=1, exact_exp=0, maxpos=maxpos, mmax=8, pool=pool)
    for c in range(pool):
        check(lib.tlg_dev_fill_normal(dec.params(c), dec.np, 77, 0.02, stream), "fill P")
    dec.pack(stream)
    dec.reset(stream)
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, DECODE_MODEL["V"], prompt_len).astype(np.int32)
    toks = rng.integers(0, DECODE_MODEL["V"], (warm + n) * M).astype(np.int32)
    dtoks = lib.tlg_dev_malloc(toks.nbytes)
    check(lib.tlg_memcpy_h2d(dtoks, toks.ctypes.data, toks.nbytes, stream), "tokens")
    dec.prime(prompt, stream)
    dec.persist_chunks(M, dtoks, warm, stream)
    dec.persist_status(stream)
    ms, _ = time_steps(lib, lambda: dec.persist_chunks(M, dtoks + 4 * warm * M, n, stream), stream, 1)
    dec.persist_status(stream)
    state = dec.state(stream)
    lib.tlg_dev_free(dtoks)
    per = ms / n
    wbytes = 4 * (DECODE_MODEL["V"] * 384 + 8 * (384 * 384 * 2 + 2 * 384 * 96 + 3 * 384 * 1024))
    dec.close()
    return {"rows": M, "chunks": n, "launches": 1, "kv_cache": "f16 ring, 256 positions", "exp": "fast_expf",
            "weights_pool": pool, "us_per_chunk": round(per * 1e3, 3), "tok_s": round(M * 1e3 / per, 1),
            "weight_bytes_per_chunk": wbytes, "weight_gbs": round(wbytes / (per * 1e-3) / 1e9, 1),
            "hbm_frac": round(wbytes / (per * 1e-3) / 8e12, 4), "final_position": state[0]}


def cpu_decode_step(threads, steps=40):
    """The oracle's forward_chunk restatement (kind "port": the reference's
    decode state is not compiled from its lines) at M = 1 on host cores."""
    import numpy as np
    import oracle
    st = oracle.StepFns("oracle")
    st.dll.orc_set_threads(threads)
    m = oracle.model(**DECODE_MODEL)
    P = st.init_params(m, 1)
    dec = oracle.Decoder(m, P, 256, kvdt=1, exact=0, maxpos=8 * steps + 32)
    prompt = np.random.default_rng(5).integers(0, m.V, 16).astype(np.int32)
    lg = dec.chunk(prompt, 0)
    state = [int(np.argmax(lg[-1])), 16]

    def run():
        for _ in range(steps):
            lg = dec.chunk(np.array([state[0]], np.int32), state[1])
            state[0], state[1] = int(np.argmax(lg[-1])), state[1] + 1

    dt, ts = median_time(run, 5)
    return {"value": round(steps / dt, 1), "unit": "decode tokens/s (whole step, M = 1)", "cores": threads,
            "kind": "port", "ms_per_token": round(dt / steps * 1e3, 3),
            "sample": f"median of 5 runs of {steps} greedy single-token steps of the m8 decode model (after a "
                      f"16-token prefill and 2 warmup runs), f16 ring cache, fast_expf; {sum(ts):.2f} s timed"}


def cpu_full_step(name, threads, reps=5):
    """The restatement's whole training step (oracle/tl_oracle_step.c:
    forward + memset(G) + backward + gradnorm + AdamW, tinylm.c:2627-2633,
    pinned to the reference's own code by the step fixtures) on host cores
    at the same model shape."""
    import numpy as np
    import oracle
    st = oracle.StepFns("oracle")
    st.dll.orc_set_threads(threads)
    kw, B = model_of(name)
    m = oracle.model(**kw)
    P = st.init_params(m, 1234567891011)
    rng = np.random.default_rng(3)
    N = B * m.T
    tok, tgt = (rng.integers(0, m.V, N).astype(np.int32) for _ in range(2))
    tm = rng.integers(0, m.V, (max(m.n_mtp, 1), N)).astype(np.int32)
    M, V = np.zeros_like(P), np.zeros_like(P)
    t = [0]

    def one():
        t[0] += 1
        _, G = st.train_step(m, B, P, tok, tgt, tm)
        gn = st.gradnorm(G)
        st.adamw(P, G, M, V, 3e-4, 0.9, 0.95, 0.1, t[0], 1.0 / gn if gn > 1.0 else 1.0)

    dt, ts = median_time(one, reps)
    return {"value": round(N / dt, 1), "unit": "train tokens/s (whole step)", "cores": threads,
            "kind": "port", "s_per_step": round(dt, 4),
            "sample": f"median of {reps} whole {name} training steps (forward + backward + gradnorm + AdamW) "
                      f"after 2 warmups, {threads} OpenMP threads; {sum(ts):.1f} s timed"}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # untimed: about 0.13 s of m3 steps, so the clocks have ramped before the
    # timed region (5 warmup steps read 1.5 % slower on the same box)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--config", default="m3", choices=sorted(TRAIN))
    ap.add_argument("--eager", action="store_true", help="enqueue each step directly instead of replaying a HIP graph")
    ap.add_argument("--calls", action="store_true",
                    help="one launch per reference call instead of one grouped launch per GEMM run")
    ap.add_argument("--census-reps", type=int, default=5)
    ap.add_argument("--group-cfg", type=int, default=None, help="tile config of grouped launches (tuning)")
    ap.add_argument("--decode-steps", type=int, default=512)
    ap.add_argument("--cpu-steps", type=int, default=5, help="timed CPU-baseline steps (median of them)")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--moe-steps", type=int, default=20)
    ap.add_argument("--other-steps", type=int, default=20, help="timed steps of the other training configs")
    ap.add_argument("--no-probes", action="store_true", help="skip the copy / MFMA peak probes")
    ap.add_argument("--no-autotune", action="store_true",
                    help="keep the library's automatic tile policy instead of the tuned per-launch table")
    ap.add_argument("--autotune", action="store_true",
                    help="time the tile candidates per launch on this box instead of using the tuned table")
    ap.add_argument("--decode-full-steps", type=int, default=512,
                    help="timed greedy decode steps of the whole device decode step; 0 skips")
    ap.add_argument("--decode-mode", default="fused", choices=("both", "fused", "unfused"),
                    help="decode step: fused launches (default), glue as separate launches, or both")
    ap.add_argument("--decode-persist-steps", type=int, default=512,
                    help="greedy decode steps in one persistent launch (tl_decode_persist); 0 skips")
    ap.add_argument("--full-steps", type=int, default=30,
                    help="timed whole training steps (forward + backward + AdamW on the device); 0 skips")
    ap.add_argument("--full-eager", action="store_true",
                    help="enqueue the whole training step launch by launch instead of replaying its graph")
    ap.add_argument("--decode-eager", action="store_true",
                    help="enqueue the decode step launch by launch instead of replaying its graphs")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build measures one MI355X "
              "(the path would shard M across GPUs with one all-reduce of dW)",
              file=sys.stderr)
        sys.exit(2)

    # one OpenMP thread per physical core for the CPU baseline (read by
    # libgomp when the oracle library first loads, after this point)
    os.environ.setdefault("OMP_PLACES", "cores")
    os.environ.setdefault("OMP_PROC_BIND", "close")
    import tlgemm
    lib = tlgemm.load()
    check(lib.tlg_init(0), "tlg_init")
    host = tlgemm.host()
    if args.group_cfg is not None:
        check(lib.tlg_tune_group(args.group_cfg), "tlg_tune_group")
    cfg = TRAIN[args.config]
    plan = host.plan_train(**cfg)
    run = host.dll.tl_run_new(ctypes.byref(plan.raw), 1)
    if not run:
        raise RuntimeError("tl_run_new failed: " + lib.tlg_last_error().decode())
    stream = lib.tlg_stream_create()
    check(host.dll.tl_run_fill(run, 1234567891011, stream), "fill")
    grouped = 0 if args.calls else 1
    launches = host.dll.tl_run_grouped_launches(run) if grouped else None
    tuned = (apply_tiles(lib, host, run, stream, args.config, args.autotune)
             if grouped and args.group_cfg is None and not args.no_autotune else None)
    if args.eager:
        fn = host.dll.tl_run_step_grouped if grouped else host.dll.tl_run_step
        step = lambda: fn(run, stream)  # noqa: E731
    else:
        check(host.dll.tl_run_graph_build(run, stream, grouped), "graph build")
        step = lambda: host.dll.tl_run_graph_step(run, stream)  # noqa: E731
    log(f"[bench] {args.config}: {len(plan.calls)} calls/step, {plan.flops() / 1e9:.2f} GFLOP/step, "
        f"{launches if grouped else 'one launch per call'} grouped launches; warmup {args.warmup}")
    for _ in range(args.warmup):
        check(step(), "warmup")
    check(lib.tlg_stream_sync(stream), "sync")
    ms, wall = time_steps(lib, step, stream, args.steps)
    ms_step = ms / args.steps
    tok_s = cfg["R"] * args.steps / (ms / 1e3)
    tflops = plan.flops() / (ms_step / 1e3) / 1e12
    log(f"[bench] timed {args.steps} steps: {ms_step:.4f} ms/step (wall {wall / args.steps * 1e3:.4f}), "
        f"{tok_s:,.0f} tok/s, {tflops:.1f} TFLOP/s")

    roof_ms = roof_time_ms(plan)

    if grouped:
        groups = launch_census(lib, host, run, stream, args.census_reps)
    else:
        groups = kernel_census(lib, host, plan, run, stream, args.census_reps)
    dom_name, dom = max(groups.items(), key=lambda kv: kv[1]["ms"])
    bound = roofline_class(dom["flops"], dom["bytes"])
    # Average launch duration of the dominant kernel over the timed region:
    # the timed step time apportioned to the kernels by their event-timed
    # shares, over the kernel's launches per step.  (Events around single
    # launches also count the gap before each launch; inside the graph replay
    # the launches run back to back, which is what rocprofv3's kernel trace
    # measures.)
    event_total = sum(g["ms"] for g in groups.values())
    avg_ms = ms_step * (dom["ms"] / event_total) / dom["launches"]
    event_avg_ms = dom["ms"] / dom["launches"]
    if bound == "mfma":
        achieved = dom["flops"] / dom["launches"] / (avg_ms / 1e3) / 1e12
        peak, unit = PEAK_FP32_MFMA_TFLOPS, "TFLOP/s"
    else:
        achieved = dom["bytes"] / dom["launches"] / (avg_ms / 1e3) / 1e9
        peak, unit = PEAK_HBM_GBS, "GB/s"
    census = {k: {"launches": v["launches"], "avg_us": round(v["ms"] / v["launches"] * 1e3, 3),
                  "timed_avg_us": round(ms_step * (v["ms"] / event_total) / v["launches"] * 1e3, 3),
                  "share": round(v["ms"] / sum(g["ms"] for g in groups.values()), 4),
                  "tflops": round(v["flops"] / (v["ms"] / 1e3) / 1e12, 2),
                  "shapes": sorted(v["shapes"])} for k, v in groups.items()}
    for k, v in sorted(census.items(), key=lambda kv: -kv[1]["share"]):
        log(f"[census] {k}: {v['launches']} launches avg {v['avg_us']} us, share {v['share']}, "
            f"{v['tflops']} TFLOP/s")

    others = {}
    if args.other_steps > 0:
        for name in TRAIN:
            if name != args.config:
                others[name] = bench_train_config(lib, host, stream, name, args.other_steps,
                                                  tune=not args.no_autotune, retime=args.autotune)
                log(f"[train] {name}: {others[name]}")
    decode, decode_packed = {}, {}
    if args.decode_steps > 0:
        for M in (1, 2, 4, 8):
            decode[M] = bench_decode(lib, host, stream, args.decode_steps, M=M, eager=args.decode_eager)
            log(f"[decode] M={M}: {decode[M]}")
        for M in (1, 2, 4, 8):
            decode_packed[M] = bench_decode(lib, host, stream, args.decode_steps, M=M, packed=True,
                                            eager=args.decode_eager)
            log(f"[decode, decode layout] M={M}: {decode_packed[M]}")
    moe = None
    if args.moe_steps > 0:
        moe = bench_moe(lib, stream, args.moe_steps)
        log(f"[moe] {moe}")
    full = None
    if args.full_steps > 0:
        full = bench_full_step(lib, host, stream, args.config, args.full_steps, eager=args.full_eager,
                               tune=not args.no_autotune)
        full["gemm_set_share"] = round(ms_step / full["ms_per_step"], 4)
        log(f"[full step] {full}")
    dec_full = None
    if args.decode_full_steps > 0:
        if args.decode_mode == "unfused":
            dec_full = bench_decode_step(lib, host, stream, args.decode_full_steps, fused=0, eager=args.decode_eager)
        else:
            dec_full = bench_decode_step(lib, host, stream, args.decode_full_steps, eager=args.decode_eager)
        log(f"[decode step] {dec_full}")
        if args.decode_mode == "both":
            dec_full["unfused"] = bench_decode_step(lib, host, stream, min(args.decode_full_steps, 128), fused=0,
                                                    eager=args.decode_eager)
            log(f"[decode step, unfused] {dec_full['unfused']}")
    dec_persist = None
    if args.decode_persist_steps > 0:
        dec_persist = bench_decode_persist(lib, host, stream, args.decode_persist_steps)
        log(f"[decode step, persistent] {dec_persist}")
        dec_persist["chunks"] = {}
        for M in (1, 2, 4, 8):
            dec_persist["chunks"][str(M)] = bench_decode_chunks(lib, host, stream, M)
            log(f"[decode chunks, persistent] M={M}: {dec_persist['chunks'][str(M)]}")
    peaks = None if args.no_probes else probes(lib, stream)
    if peaks:
        log(f"[probes] {peaks}")

    cpu = None
    if not args.no_cpu:
        threads, facts = host_cpu_share()
        if args.cpu_threads:
            threads = args.cpu_threads
        log(f"[cpu] host {facts}: timing the CPU restatement on {threads} threads ...")
        cpu = cpu_baseline(host, args.config, args.cpu_steps, threads, facts)
        log(f"[cpu] {cpu}")
        if args.full_steps > 0:
            cpu["train_step"] = cpu_full_step(args.config, threads)
            log(f"[cpu] whole step {cpu['train_step']}")
        if args.decode_full_steps > 0:
            cpu["decode_step"] = cpu_decode_step(threads)
            log(f"[cpu] decode step {cpu['decode_step']}")
        if args.decode_steps > 0:
            cpu["decode"] = {str(M): cpu_decode_baseline(host, M, 100 if M == 1 else 30, threads) for M in (1, 8)}
            log(f"[cpu] decode {cpu['decode']}")

    host.dll.tl_run_free(run)
    rocprof_avg = read_rocprof_avg_us(dom_name)            # profiles/m3_step_kernel_trace.md
    mfma_row = read_profile_row("mfma_counters_m3_moe.txt", dom_name)
    result = {
        "metric": "train tokens/s (m3-scale); GEMM TFLOP/s & % roofline; M=1 decode tok/s",
        "value": round(tok_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic: seeded Gaussian activations/weights/gradients resident in HBM",
        "config": {
            "workload": f"BASELINE {args.config} training-step GEMM set: {len(plan.calls)} calls "
                        f"(tinylm.c forward/backward order), {plan.flops() / 1e9:.2f} GFLOP/step, "
                        f"{'grouped: %d launches per step' % launches if grouped else 'one launch per call'}, "
                        f"{'enqueued directly' if args.eager else 'replayed as one HIP graph'}",
            "rows": cfg["R"], "d_model": cfg["D"], "kv_dim": cfg["KD"], "ffn": cfg["F"],
            "vocab": cfg["V"], "layers": cfg["L"], "mtp_heads": cfg["n_mtp"],
            "global_batch": cfg["R"] // 256, "seq_len": 256, "parallelism": "single GPU",
        },
        "tflops": round(tflops, 2),
        "tile_configs": tuned,
        "step_roofline": {"sum_of_gemm_roof_ms": round(roof_ms, 4),
                          "frac": round(roof_ms / ms_step, 4)},
        "roofline": {
            "kernel": dom_name, "bound": bound, "achieved": round(achieved, 2), "peak": peak,
            "unit": unit, "frac": round(achieved / peak, 4),
            "traffic": read_traffic(dom_name),
            "frac_of_achievable": round(achieved / peaks[("mfma_fp32_tflops" if bound == "mfma" else "hbm_copy_gbs")], 4)
            if peaks else None,
            "launches_per_step": dom["launches"], "avg_launch_us": round(avg_ms * 1e3, 3),
            "avg_launch_us_source": "this run: the timed graph-replayed step apportioned by the launches' "
                                    "event-census shares",
            "event_census_avg_us": round(event_avg_ms * 1e3, 3),
            "rocprof_avg_us": rocprof_avg,
            "frac_rocprof": (round(dom["flops"] / dom["launches"] / (rocprof_avg * 1e-6) / 1e12 / peak, 4)
                             if rocprof_avg and bound == "mfma" else None),
            "mfma_busy": float(mfma_row[0]) if mfma_row else None,
            "mfma_executed_gflop_per_launch": float(mfma_row[1]) if mfma_row else None,
            "algorithmic_bytes_per_launch": round(dom["bytes"] / dom["launches"]),
            "algorithmic_flops_per_launch": round(dom["flops"] / dom["launches"]),
        },
        "kernels": census,
        "other_configs": others,
        "decode_m1": decode.get(1),
        "decode": {str(k): v for k, v in decode.items()},
        "decode_packed": {str(k): v for k, v in decode_packed.items()},
        "moe": moe,
        "train_step": full,
        "decode_step": dec_full,
        "decode_step_persistent": dec_persist,
        "achievable": peaks,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)
    # tear down explicitly, before the interpreter exits: a profiler that has
    # already finalised must not see the library's device memory and streams
    # released by exit handlers
    import gc
    gc.collect()
    lib.tlg_stream_destroy(stream)
    lib.tlg_shutdown()


if __name__ == "__main__":
    main()
