"""Benchmark of the Needle-3 hot path on one MI355X.

Headline ("codebook GEMV GB/s (% HBM peak)"): the codebook dequant-GEMV,
W [3072 x 768] uint8 codes, one 256-entry fp32 codebook per 64 rows, x [768],
batch 1 -- over R = 448 distinct weight copies per step (1.09 GB, beyond the
256 MB MALL), as one strided launch.  A step is one such launch; value =
algorithmic bytes / time.

Also reported ("secondary"):
  - int8-KV decode attention at ctx 2048, 12 heads x 64, over 320
    independent session caches per step (append one token + attend), and
    the batch-1 latencies of both kernels; attention alone at ctx 512 and
    8192 over 1 GiB of caches;
  - the Cactus-Quants (Format A) decode GEMV, tolerance and reference order,
    streaming and at the shipped shapes;
  - the Format B prefill GEMM on bf16 MFMA;
  - the Needle-3 forward (shipped geometry, random init, int8 KV cache):
    one session with a 128-token prompt and 256 greedy tokens, and 64
    sessions each prefilled with 2048 tokens then 128 greedy tokens in
    lockstep ("decode tok/s @ ctx2048 int8 KV"), whose tokens are then
    checked (untimed) against batch-1 device runs and the oracle.

cpu_baseline: the oracle (the reference's CPU arithmetic restated in C) on
the host cores, 1 thread and all threads, on bounded samples of configs
1-5; the headline value is config 1's GEMV at all threads.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "needle-rs_amd"))

# The forward's four-stream run needs a hardware queue per stream besides
# the default stream's.  HIP gives a process four by default, with which two
# of the four streams share one and run one after the other (3.27 against
# 1.82 ms a step); set before anything initialises HIP.
if int(os.environ.get("GPU_MAX_HW_QUEUES", "4")) < 8:
    os.environ["GPU_MAX_HW_QUEUES"] = "8"

HBM_PEAK_GBS = 8000.0
FP32_MFMA_TFLOPS = 157.3
GEMV_OUT, GEMV_IN = 3072, 768
GEMV_BYTES = GEMV_OUT * GEMV_IN + (GEMV_OUT // 64) * 256 * 4 + GEMV_IN * 4 + GEMV_OUT * 4
GEMV_COPIES = 448
ATT_H, ATT_D, ATT_CTX, ATT_SESSIONS = 12, 64, 2048, 320
# int8 K and V plus their f32 scales over the span, plus q (fp32) in and out.
ATT_BYTES = ATT_CTX * (2 * ATT_H * ATT_D + 2 * ATT_H * 4) + 2 * ATT_H * ATT_D * 4


def pmc_traffic(kernel):
    """HBM bytes per launch of `kernel` as measured by the FETCH_SIZE /
    WRITE_SIZE counter runs summarised in profiles/hbm_traffic_pmc.md."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic_pmc.md")
    try:
        for line in open(path):
            parts = line.split()
            if len(parts) == 3 and parts[0] == "traffic_bytes_per_launch" and parts[1] == kernel:
                return int(parts[2])
    except OSError:
        pass
    return None


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-secondary", action="store_true")
    p.add_argument("--no-forward", action="store_true", help="skip the Needle-3 forward runs")
    p.add_argument("--forward-sessions", type=int, default=64)
    p.add_argument("--forward-ctx", type=int, default=2048)
    p.add_argument("--no-check", action="store_true",
                   help="skip the untimed token check of the multi-session forward")
    p.add_argument("--only", choices=["gemv", "attn", "forward", "gemm", "cqa"], default=None,
                   help="run one workload only, without the batch-1 latency probes "
                        "(for per-kernel profiles)")
    p.add_argument("--min-warm", type=float, default=0.5,
                   help="seconds of untimed warm-up before each timed loop (0 for counter runs)")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="also run a plain 1 GiB device copy (PMC byte-counter scale)")
    p.add_argument("--summarize-trace", metavar="CSV", default=None,
                   help="no GPU: print per-kernel statistics of the last --tail-steps forward "
                        "steps of a rocprofv3 kernel-trace CSV (steps end at k_final); with "
                        "--tail-steps 0, of every launch, per kernel and grid size")
    p.add_argument("--tail-steps", type=int, default=128)
    p.add_argument("--skip-steps", type=int, default=0,
                   help="with --summarize-trace: leave out the trace's last N forward steps "
                        "(e.g. 256: the two-stream run of 2 x 128 steps that ends --only forward)")
    p.add_argument("--summarize-pmc", metavar="CSV", default=None,
                   help="no GPU: print the mean of each counter per dispatch of a rocprofv3 "
                        "--pmc counter-collection CSV, per kernel and grid size")
    p.add_argument("--pmc-period", type=int, default=0,
                   help="with --summarize-pmc: also split each (kernel, grid) group by the "
                        "dispatch's index modulo this period (e.g. 20: the layer of a step)")
    p.add_argument("--pmc-runs", type=int, default=0,
                   help="with --summarize-pmc: also split each group into this many runs of "
                        "consecutive dispatches (e.g. 2: the two shapes --only gemm times "
                        "with one grid)")
    return p.parse_args()


def summarize_trace(path, nsteps, skip=0):
    """Per-kernel durations over the last `nsteps` forward steps of a
    rocprofv3 --kernel-trace CSV (plain or gzipped), leaving out the last
    `skip` steps.  Each step launches k_final once, so the window runs from
    the end of the (nsteps + skip + 1)-th last k_final to the end of the
    (skip + 1)-th last; kernels of the side stream in that window are
    included.  With nsteps 0, every launch of the trace, grouped by kernel and
    grid size."""
    import collections
    import csv
    import gzip
    rows = []
    with (gzip.open(path, "rt") if path.endswith(".gz") else open(path)) as f:
        for r in csv.DictReader(f):
            grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"], grid))
    rows.sort()
    if nsteps == 0:
        agg = collections.defaultdict(list)
        for a, b, n, grid in rows:
            agg[(n, grid)].append(b - a)
        print("| kernel | grid | launches | avg us | min us | max us |")
        print("|---|---|---|---|---|---|")
        for (n, grid), v in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
            name = n.replace("(anonymous namespace)::", "").split("(")[0]
            if name.startswith("void "):
                name = name[5:]
            print(f"| `{name}` | {grid} | {len(v)} | {sum(v) / len(v) / 1e3:.2f} | "
                  f"{min(v) / 1e3:.2f} | {max(v) / 1e3:.2f} |")
        return
    finals = [i for i, r in enumerate(rows) if "::k_final(" in r[2]]
    t0 = rows[finals[-(nsteps + skip + 1)]][1]
    t1 = rows[finals[-(skip + 1)]][1]
    sel = [r for r in rows if t0 < r[0] and r[1] <= t1]
    agg = collections.defaultdict(list)
    for a, b, n, _ in sel:
        agg[n].append(b - a)
    span = (t1 - t0) / 1e3
    print(f"last {nsteps} steps: {span / nsteps:.1f} us per step (profiler on), {len(sel)} kernels")
    print("| kernel | per step | avg us | min us | max us | us per step |")
    print("|---|---|---|---|---|---|")
    for n, v in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
        name = n.replace("(anonymous namespace)::", "").split("(")[0]
        if name.startswith("void "):
            name = name[5:]
        print(f"| `{name}` | {len(v) / nsteps:.2f} | {sum(v) / len(v) / 1e3:.2f} | "
              f"{min(v) / 1e3:.2f} | {max(v) / 1e3:.2f} | {sum(v) / nsteps / 1e3:.1f} |")


def summarize_pmc(path, period, runs):
    """Mean counter values per dispatch of a rocprofv3 --pmc CSV, grouped by
    kernel and grid size (a workload's launches of one shape), with the mean
    dispatch duration under the profiler.  With `period`, each group is also
    split by the dispatch's index within the group modulo `period`; with
    `runs`, into that many runs of consecutive dispatches."""
    import collections
    import csv
    disp = collections.OrderedDict()
    with open(path) as f:
        for r in csv.DictReader(f):
            k = int(r["Dispatch_Id"])
            e = disp.get(k)
            if e is None:
                name = r["Kernel_Name"].replace("(anonymous namespace)::", "").split("(")[0]
                name = name[5:] if name.startswith("void ") else name
                e = disp[k] = {"name": name, "grid": int(r["Grid_Size"]), "c": {},
                               "us": (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3}
            e["c"][r["Counter_Name"]] = float(r["Counter_Value"])
    groups = collections.OrderedDict()
    for k in sorted(disp):
        e = disp[k]
        groups.setdefault((e["name"], e["grid"]), []).append(e)
    names = sorted({c for e in disp.values() for c in e["c"]})
    print("| kernel | grid | part | dispatches | us (profiled) | " + " | ".join(names) + " |")
    print("|---|---|---|---|---|" + "---|" * len(names))

    def row(key, part, es):
        us = sum(e["us"] for e in es) / len(es)
        vals = [sum(e["c"].get(c, 0.0) for e in es) / len(es) for c in names]
        print(f"| `{key[0]}` | {key[1]} | {part} | {len(es)} | {us:.2f} | " +
              " | ".join(f"{v:,.0f}" for v in vals) + " |")

    for key, es in groups.items():
        row(key, "all", es)
        if period > 0 and len(es) >= period:
            for j in range(period):
                sub = es[j::period]
                if sub:
                    row(key, f"{j} mod {period}", sub)
        if runs > 1 and len(es) >= runs:
            n = len(es) // runs
            for j in range(runs):
                row(key, f"run {j + 1} of {runs}", es[j * n:(j + 1) * n])


MIN_WARM_S = 0.5


def timed_loop(torch, fn, steps, warmup, min_warm_s=None):
    """W untimed warm-up steps (continued until `min_warm_s` has passed, so the
    clocks have left their idle state), then exactly `steps` timed steps
    between two events on the stream the kernels run on."""
    if min_warm_s is None:
        min_warm_s = MIN_WARM_S
    t0 = time.perf_counter()
    n = 0
    while n < warmup or time.perf_counter() - t0 < min_warm_s:
        fn()
        n += 1
        if n % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms


def _threads_all():
    """Host threads this process may use: its CPU affinity, capped by
    OMP_NUM_THREADS when that is set (the OpenMP default the oracle uses)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def _time_for(fn, seconds, min_calls=1):
    calls, t0 = 0, time.perf_counter()
    while True:
        fn()
        calls += 1
        el = time.perf_counter() - t0
        if el >= seconds and calls >= min_calls:
            return calls, el


def cpu_baseline(sec=2.5):
    """The reference's CPU path, as the oracle restates it, on the host cores
    of this run: 1 thread and all threads, each on a bounded sample of the
    same workloads the GPU lines run.  Threads split the work as the
    reference's rayon pool would (row bands past cq.rs's size rules; one
    session per thread for independent sessions, as a server runs one
    V3Cache per session).  The Cactus-Quants kernels are the reference's
    const-generic LUT loops (P = 2 and 4 instantiated separately, eight
    lanes as vector multiplies then adds); Format B, which has no reference
    function, runs the same eight-lane dot with one level per byte, and its
    GEMM decodes each weight row once for all activation rows, as
    matmul_rows_prepared does."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    import v3_synth as S
    T = _threads_all()
    rng = np.random.default_rng(1)
    out = {}

    # config 1: the codebook GEMV, 64 distinct copies (151 MB)
    copies = 64
    W = rng.integers(0, 256, size=(copies, GEMV_OUT, GEMV_IN), dtype=np.uint8)
    CB = rng.normal(0, 0.02, size=(copies, GEMV_OUT // 64, 256)).astype(np.float32)
    X = rng.normal(size=(copies, GEMV_IN)).astype(np.float32)
    y = np.zeros(GEMV_OUT, np.float32)
    it = [0]

    def gemv(par):
        i = it[0] % copies
        it[0] += 1
        O.cb8_gemv_lanes(W[i], CB[i], X[i], T if par else 1, y)
    gemv(True)
    n1, e1 = _time_for(lambda: gemv(False), sec, copies // 8)
    nT, eT = _time_for(lambda: gemv(True), 2 * sec, copies)
    g1, gT = n1 * GEMV_BYTES / e1 / 1e9, nT * GEMV_BYTES / eT / 1e9
    del W, CB, X
    out["config1_gemv_GBps"] = {"1_thread": round(g1, 3), "all_threads": round(gT, 3),
                                "sample": f"{n1} and {nT} GEMVs of 3072x768 over 64 copies"}

    # config 2: the Format B GEMM, M 512 x K 768, N 3072 and 768
    gemm = {}
    for N in (3072, 768):
        x = rng.normal(size=(512, 768)).astype(np.float32)
        w = rng.integers(0, 256, size=(N, 768), dtype=np.uint8)
        cb = rng.normal(0, 0.02, size=(N // 64, 256)).astype(np.float32)
        yy = np.zeros((512, N), np.float32)
        flops = 2.0 * 512 * 768 * N
        a, ea = _time_for(lambda: O.cb8_gemm_lanes(x, w, cb, 1, yy), sec / 2)
        b, eb = _time_for(lambda: O.cb8_gemm_lanes(x, w, cb, T, yy), sec / 2)
        gemm[f"m512_n{N}_k768_GFLOPs"] = {"1_thread": round(a * flops / ea / 1e9, 2),
                                          "all_threads": round(b * flops / eb / 1e9, 2)}
    out["config2_gemm"] = gemm

    # config 3: int8-KV decode attention at ctx 2048, 12 heads x 64 (MHA),
    # over 64 sessions' own caches (214 MB)
    H, D, ctxn, ns = ATT_H, ATT_D, ATT_CTX, 64
    kq = rng.integers(-127, 128, size=(ns, ctxn * H * D), dtype=np.int8)
    vq = rng.integers(-127, 128, size=(ns, ctxn * H * D), dtype=np.int8)
    ks = (rng.random((ns, ctxn * H)) * 0.03 + 1e-3).astype(np.float32)
    vs = (rng.random((ns, ctxn * H)) * 0.03 + 1e-3).astype(np.float32)
    q = rng.normal(size=(ns, H * D)).astype(np.float32)
    o = np.zeros((ns, H * D), np.float32)

    def att(threads, n):
        O.attend_step_i8_sessions(q[:n], kq[:n], ks[:n], vq[:n], vs[:n], ctxn, 0, ctxn - 1,
                                  H, H, D, D, threads, o[:n])
    a, ea = _time_for(lambda: att(1, 8), sec / 2)
    b, eb = _time_for(lambda: att(T, ns), sec / 2)
    out["config3_attention_ctx2048_GBps"] = {
        "1_thread": round(a * 8 * ATT_BYTES / ea / 1e9, 3),
        "all_threads": round(b * ns * ATT_BYTES / eb / 1e9, 3),
        "sample": f"{a} x 8 and {b} x {ns} session decodes (one session per thread)"}
    del kq, vq, ks, vs

    # config 4: one session's decode step on the shipped geometry after a
    # 128-token prompt (the reference's split rules: only the LM head splits)
    g, recs = S.build_records(None, seed=0)
    om = O.V3Model(g, recs, S.CODEBOOK)
    prompt = S.prompt_tokens(128, 4)
    cache = om.new_cache(128 + 64, True)
    O.set_threads(T, O.SPLIT_ALL)  # prefill the prompt quickly (same bits)
    lg = None
    for t in prompt:
        lg = cache.decode_step(int(t))
    res4, done = {}, 0
    for name, th in (("1_thread", 1), ("all_threads", T)):
        O.set_threads(th, O.SPLIT_REFERENCE)

        def dec():
            nonlocal lg
            lg = cache.decode_step(int(np.argmax(lg)))
        n, e = _time_for(dec, sec / 2, 4)
        done += n
        res4[name] = round(e / n * 1e3, 2)
    O.set_threads(1, O.SPLIT_REFERENCE)
    out["config4_decode_ms_per_token"] = dict(res4, sample=f"{done} greedy steps at positions "
                                              f"128..{128 + done} after a 128-token prompt")

    # config 5: 64 sessions at ctx 2048, one session per thread; the caches
    # are put at position 2048 with seeded contents (the per-step work of a
    # prefilled session, without prefilling 131k positions on the CPU)
    ns = 64
    caches = [om.new_cache(2048 + 128, True) for _ in range(ns)]
    for i, c in enumerate(caches):
        c.fill_synthetic(2048, 1000 + i)
    toks = np.array(S.prompt_tokens(ns, 9), np.uint32)
    a, ea = _time_for(lambda: O.v3_decode_sessions(om, caches[:4], toks[:4], 1), sec / 2)
    b, eb = _time_for(lambda: O.v3_decode_sessions(om, caches, toks, T), sec / 2)
    out["config5_sessions64_ctx2048_tok_per_s"] = {
        "1_thread": round(a * 4 / ea, 2), "all_threads": round(b * ns / eb, 2),
        "sample": f"{a} x 4 and {b} x {ns} session steps at positions 2048+ (synthetic cache "
                  "contents at the real spans)"}
    del caches
    return {"value": round(gT, 3), "unit": "GB/s", "cores": T, "kind": "port",
            "sample": f"config 1: {nT} GEMVs of 3072x768 u8 over 64 distinct weight copies in "
                      f"{eT:.1f} s (oracle or_cb8_gemv_lanes: the reference's eight-lane LUT "
                      f"dot with one level per byte, row bands on {T} OpenMP threads)",
            "value_1_thread": round(g1, 3), "nproc": os.cpu_count(), "cpu_model": _cpu_model(),
            "configs": out}


BF16_MFMA_PEAK_TFLOPS = 2500.0


def gemm_runs(torch, nd, ctx, gen, steps):
    """Format B prefill GEMM, Y [512 x N] = X [512 x 768] . decode(W [N x 768]),
    bf16 MFMA with fp32 accumulate, for the two projection widths; R
    distinct problems per launch (one launch per step) so the step is long
    enough to time on the device.  Both widths launch 768 tiles of 256 x 256
    (three per CU): at N 768 with 64 problems (384 tiles, a wave and a half)
    the second half-wave left half the CUs idle."""
    out = {}
    M, K = 512, 768
    for N, R in ((3072, 32), (768, 128)):
        X = torch.randn(R, M, K, device="cuda", generator=gen)
        W = torch.randint(0, 256, (R, N, K), dtype=torch.uint8, device="cuda", generator=gen)
        CB = torch.randn(R, N // 64, 256, device="cuda", generator=gen) * 0.02
        Y = torch.empty(R, M, N, device="cuda")
        ms = timed_loop(torch, lambda: nd.cb8_gemm_batched(ctx, X, W, CB, Y), steps, 10)
        flops = 2.0 * M * N * K * R
        tf = flops / (ms * 1e-3) / 1e12
        out[f"m{M}_n{N}_k{K}"] = {"problems_per_launch": R, "us_per_launch": round(ms * 1e3, 2),
                                  "us_per_gemm": round(ms * 1e3 / R, 3), "TFLOPs": round(tf, 2),
                                  "frac_bf16_mfma_dense_peak": round(tf / BF16_MFMA_PEAK_TFLOPS, 4),
                                  "flops_per_gemm": 2 * M * N * K}
        del X, W, CB, Y
    # M = 64 (64 sessions' rows at once): each code feeds 64 rows, so the
    # launch is bound by streaming the codes; 448 weights of 3072 x 768
    # (1.06 GB) are read from HBM per launch
    M, N, R = 64, 3072, 448
    X = torch.randn(R, M, K, device="cuda", generator=gen)
    W = torch.randint(0, 256, (R, N, K), dtype=torch.uint8, device="cuda", generator=gen)
    CB = torch.randn(R, N // 64, 256, device="cuda", generator=gen) * 0.02
    Y = torch.empty(R, M, N, device="cuda")
    ms = timed_loop(torch, lambda: nd.cb8_gemm_batched(ctx, X, W, CB, Y), steps, 10)
    nbytes = R * (N * K + N // 64 * 256 * 4 + M * K * 4 + M * N * 4)
    gbs = nbytes / (ms * 1e-3) / 1e9
    tf = 2.0 * M * N * K * R / (ms * 1e-3) / 1e12
    out[f"m{M}_n{N}_k{K}"] = {"problems_per_launch": R, "us_per_launch": round(ms * 1e3, 2),
                              "bytes_per_launch": nbytes, "GBps": round(gbs, 1),
                              "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "TFLOPs": round(tf, 2)}
    del X, W, CB, Y
    return out


def _cq_blob(rng, rows, inn, bits, group=128):
    """A Cactus-Quants blob (cq.rs:181-238): uniform random packed codes, then
    FP16 norms ~ N(0, 0.02) * sqrt(group)."""
    import numpy as np
    per = {2: 4, 4: 2}[bits]
    row_bytes = inn // per
    ng = inn // group
    packed = rng.integers(0, 256, size=rows * row_bytes, dtype=np.uint8)
    norms = (rng.standard_normal(rows * ng, dtype=np.float32) * np.float32(0.02 * math.sqrt(group)))
    return np.concatenate([packed, norms.astype(np.float16).view(np.uint8)]), row_bytes, ng


def format_a_runs(torch, nd, steps):
    """Cactus-Quants (Format A) decode GEMV, batch 1, in 768, group 128.

    Streaming: one tall weight of the q projection's shape stacked 4096 times
    (2-bit, 2,359,296 rows) and one of the LM head's shape stacked 160 times
    (4-bit, 1,310,720 rows) -- each over 450 MB, beyond the MALL -- timed as
    one call over all rows; bytes = packed + f32 norms + xh + y.  Both the
    tolerance kernel and the reference-order (bit-exact) kernel.
    Latency: one call on each projection shape of the shipped Needle-3 model."""
    import numpy as np
    import v3_synth as S
    rng = np.random.default_rng(11)
    ctx = nd.Ctx(0)
    inn = 768
    out = {}
    for name, shape_rows, copies, bits in (("q576x768_2bit", 576, 4096, 2),
                                           ("lm_head8192x768_4bit", 8192, 160, 4)):
        rows = shape_rows * copies
        blob, row_bytes, ng = _cq_blob(rng, rows, inn, bits)
        w = nd.CqWeight(ctx, blob, rows, inn, 128, bits, S.CODEBOOK)
        del blob
        xh = torch.randn(inn, device="cuda")
        y = torch.empty(rows, device="cuda")
        nbytes = rows * (row_bytes + 4 * ng + 4) + 4 * inn
        rec = {"rows": rows, "bytes_per_call": nbytes}
        for tag, exact in (("tolerance", False), ("exact", True)):
            ms = timed_loop(torch, lambda: w.matvec_rows_prepared(xh, 0, rows, y, exact=exact),
                            max(10, steps // 2), 3)
            gbs = nbytes / (ms * 1e-3) / 1e9
            rec[tag] = {"us": round(ms * 1e3, 1), "GBps": round(gbs, 1),
                        "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
        out[name + "_stream"] = rec
        w.close()
        del y
    lat = {}
    for name, rows, bits in (("q", 576, 2), ("k", 96, 2), ("v", 128, 2), ("gate_out", 768, 2),
                             ("lm_head", 8192, 4)):
        blob, row_bytes, ng = _cq_blob(rng, rows, inn, bits)
        w = nd.CqWeight(ctx, blob, rows, inn, 128, bits, S.CODEBOOK)
        xh = torch.randn(inn, device="cuda")
        y = torch.empty(rows, device="cuda")
        lat[name] = {tag: round(timed_loop(torch, lambda: w.matvec_rows_prepared(
            xh, 0, rows, y, exact=exact), 200, 20, 0.1) * 1e3, 2)
            for tag, exact in (("tolerance_us", False), ("exact_us", True))}
        w.close()
    out["single_call_latency"] = lat
    # prefill GEMM (matmul_rows_prepared, fp32 MFMA): 512 prepared rows
    # against the q projection's shape (2-bit) and the LM head's (4-bit)
    gemm = {}
    for name, rows, bits in (("q576x768_2bit", 576, 2), ("lm_head8192x768_4bit", 8192, 4)):
        blob, row_bytes, ng = _cq_blob(rng, rows, inn, bits)
        w = nd.CqWeight(ctx, blob, rows, inn, 128, bits, S.CODEBOOK)
        M = 512
        xh = torch.randn(M, inn, device="cuda")
        y = torch.empty(M * rows, device="cuda")
        ms = timed_loop(torch, lambda: w.matmul_rows_prepared(xh, M, 0, rows, y), max(20, steps), 5)
        tf = 2.0 * M * rows * inn / (ms * 1e-3) / 1e12
        gemm[name + "_m512"] = {"us": round(ms * 1e3, 2), "TFLOPs": round(tf, 2),
                                "frac_fp32_mfma_peak": round(tf / FP32_MFMA_TFLOPS, 4)}
        w.close()
    out["prefill_gemm_fp32_mfma"] = gemm
    ctx.close()
    return out


def attention_ctx_runs(torch, nd, ctx, gen, steps):
    """Decode attention over the int8 cache at ctx 512 and 8192 (12 heads x
    64, MHA, scale 1/8): as many independent session caches as stream over
    1 GiB per step, attention only; plus one session's latency."""
    out = {}
    for ctx_len in (512, 8192):
        per = ctx_len * (2 * ATT_H * ATT_D + 2 * ATT_H * 4) + 2 * ATT_H * ATT_D * 4
        S = -(-(1 << 30) // per)
        g = nd.kv_geom(ATT_H, ATT_H, ATT_D, ATT_D, ctx_len)
        nb = nd.kv_block_bytes(g)
        off = nd.kv_offsets(g)
        blk = torch.empty(S * nb, dtype=torch.uint8, device="cuda")
        view = blk.view(S, nb)
        view[:, :off["ks"]].copy_(torch.randint(-127, 128, (S, off["ks"]), dtype=torch.int8,
                                                device="cuda", generator=gen).view(torch.uint8))
        scales = torch.rand(S, 2 * ATT_H * ctx_len, device="cuda", generator=gen) * 0.03 + 1e-3
        view[:, off["ks"]:off["ks"] + 8 * ATT_H * ctx_len].copy_(scales.view(torch.uint8).view(S, -1))
        del scales
        q = torch.randn(S, ATT_H * ATT_D, device="cuda", generator=gen)
        hi = torch.full((S,), ctx_len - 1, dtype=torch.int32, device="cuda")
        lo = torch.zeros(S, dtype=torch.int32, device="cuda")
        o = torch.empty(S, ATT_H * ATT_D, device="cuda")
        ms = timed_loop(torch, lambda: nd.attend_step_i8(ctx, g, blk, nb, lo, hi, q,
                                                         quant_query=True, out=o),
                        max(10, steps // 2), 5)
        ms1 = timed_loop(torch, lambda: nd.attend_step_i8(ctx, g, blk, nb, lo[:1], hi[:1], q[:1],
                                                          quant_query=True, out=o[:1]), 200, 20)
        gbs = S * per / (ms * 1e-3) / 1e9
        out[f"decode_attention_int8_ctx{ctx_len}"] = {
            "workload": f"{S} sessions x 12 heads x 64, ctx {ctx_len}, int8 K/V + f32 scales",
            "attention_GBps": round(gbs, 2), "attention_frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "bytes_per_session_decode": per, "sessions": S,
            "single_session_attention_us": round(ms1 * 1e3, 2)}
        del blk, view, q, o
    return out


def exact_attention_runs(torch, nd, ctx, gen):
    """One session's reference-order decode attention (nd_attend_step_i8_exact,
    the forward's attention) over spans of 384..4096 positions, at the
    forward's head geometry (12 q / 2 kv heads, qk 48, vd 64): microseconds
    per call.  Spans of 1024 and more sum the softmax with the parallel fold."""
    H, KVH, QK, VD = 12, 2, 48, 64
    out = {}
    for span in (384, 1024, 2048, 4096):
        g = nd.kv_geom(H, KVH, QK, VD, span)
        nb = nd.kv_block_bytes(g)
        off = nd.kv_offsets(g)
        blk = torch.empty(nb, dtype=torch.uint8, device="cuda")
        blk[:off["ks"]].copy_(torch.randint(-127, 128, (off["ks"],), dtype=torch.int8, device="cuda",
                                            generator=gen).view(torch.uint8))
        scales = torch.rand(2 * KVH * span, device="cuda", generator=gen) * 0.03 + 1e-3
        blk[off["ks"]:off["ks"] + 8 * KVH * span].copy_(scales.view(torch.uint8))
        q = torch.randn(1, H * QK, device="cuda", generator=gen)
        lo = torch.zeros(1, dtype=torch.int32, device="cuda")
        hi = torch.full((1,), span - 1, dtype=torch.int32, device="cuda")
        o = torch.empty(1, H * VD, device="cuda")
        ms = timed_loop(torch, lambda: nd.attend_step_i8(ctx, g, blk, nb, lo, hi, q, quant_query=True,
                                                         out=o, exact=True), 200, 20)
        out[f"span{span}_us"] = round(ms * 1e3, 2)
        del blk, scales, q, o
    return out


def forward_runs(torch, nd, ctx, sessions, ctx_len, check=True):
    """The Needle-3 forward on the device: batch 1 (128-token prompt, 256
    greedy steps) and `sessions` sessions prefilled with `ctx_len` tokens
    then 128 greedy steps.  Wall-clock over host-driven steps, each greedy
    step ending with its tokens back on the host.  Then, untimed, the
    multi-session tokens are checked: sessions 0 and sessions-1 against
    batch-1 device runs and against the oracle's decode_step over every
    position."""
    import numpy as np
    import v3_synth as S
    g, recs = S.build_records(None, seed=0)
    model = nd.V3Model(ctx, g, recs, S.CODEBOOK)
    out = {}

    def run(B, prompt_len, steps, chunk, prompts=None, device_loop=True):
        """Prefill, then `steps` greedy steps; returns the prefill and decode
        wall times and the tokens each step fed ([B][steps]).  device_loop:
        the steps run as nd_v3_generate (each choice fed back on the
        device); else as nd_v3_step calls that return each step's tokens to
        the host, which feeds them back."""
        batch = nd.V3Batch(model, B, max_len=prompt_len + steps, max_chunk=chunk)
        if prompts is None:
            prompts = np.stack([S.prompt_tokens(prompt_len, 100 + i) for i in range(B)])
        prompts = np.ascontiguousarray(prompts, np.int32)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        nxt = None
        for t in range(0, prompt_len, chunk):
            t1 = min(prompt_len, t + chunk)
            nxt = batch.prefill(prompts[:, t:t1], want_next=(t1 == prompt_len))
        torch.cuda.synchronize()
        t_pre = time.perf_counter() - t0
        t0 = time.perf_counter()
        if device_loop:
            out = batch.greedy(nxt, steps)
            toks = np.concatenate([nxt[:, None], out[:, :-1]], axis=1)
        else:
            toks = []
            for _ in range(steps):
                toks.append(nxt)
                nxt = batch.step(nxt)
            toks = np.stack(toks, axis=1)
        t_dec = time.perf_counter() - t0
        batch.close()
        return t_pre, t_dec, toks

    # warm, untimed: code objects, and about half a second of steps so the
    # clocks have left their idle state before the timed decode
    run(1, 16, 240, 16)
    run(1, 16, 240, 16, device_loop=False)
    t_pre, t_dec, toks1 = run(1, 128, 256, 128)
    _, t_dec_h, toks1_h = run(1, 128, 256, 128, device_loop=False)
    out["batch1_prompt128_greedy256"] = {
        "workload": "shipped Needle-3 geometry (20 layers, d 768, 12 q / 2 kv heads, vocab "
                    "8192), random init, Cactus-Quants weights, int8 KV; one session, "
                    "128-token uniform prompt prefilled in one pass, then 256 greedy tokens "
                    "(the greedy loop on the device, nd_v3_generate; host_stepped: one "
                    "nd_v3_step call per token, its token back on the host)",
        "prefill_ms": round(t_pre * 1e3, 3),
        "prefill_ms_per_token": round(t_pre / 128 * 1e3, 4),
        "decode_ms_per_token": round(t_dec / 256 * 1e3, 3),
        "decode_tok_per_s": round(256 / t_dec, 1),
        "decode_ms_per_token_host_stepped": round(t_dec_h / 256 * 1e3, 3),
        "tokens_equal_host_stepped": bool(np.array_equal(toks1, toks1_h)),
    }
    steps = 128
    t_pre, t_dec, toks = run(sessions, ctx_len, steps, 32)
    _, t_dec_h, toks_h = run(sessions, ctx_len, steps, 32, device_loop=False)
    key = f"sessions{sessions}_ctx{ctx_len}_greedy{steps}"
    out[key] = {
        "workload": f"{sessions} sessions of the same model in lockstep, each prefilled with "
                    f"{ctx_len} uniform prompt tokens (32 positions per pass), then {steps} greedy "
                    "steps; projections batched over sessions, attention per session; the "
                    "greedy loop on the device (nd_v3_generate), and host_stepped: one "
                    "nd_v3_step call per step, the tokens back on the host",
        "decode_tok_per_s": round(sessions * steps / t_dec, 1),
        "decode_ms_per_step": round(t_dec / steps * 1e3, 3),
        "decode_tok_per_s_host_stepped": round(sessions * steps / t_dec_h, 1),
        "decode_ms_per_step_host_stepped": round(t_dec_h / steps * 1e3, 3),
        "tokens_equal_host_stepped": bool(np.array_equal(toks, toks_h)),
        "prefill_tok_per_s": round(sessions * ctx_len / t_pre, 1),
    }
    # the same sessions as n batches of sessions / n on n streams, their
    # greedy loops enqueued in turn from this thread (nd_v3_generate_many):
    # one batch's one-workgroup-per-session kernels run beside another's
    # projections and attention; projections batched over sessions / n
    for n, name in ((2, "two_streams"), (4, "four_streams")):
        if sessions % n:
            continue
        part = sessions // n
        streams = [torch.cuda.Stream() for _ in range(n)]
        ctxs = [nd.Ctx(0, stream=st) for st in streams]
        batches, firsts = [], []
        for k in range(n):
            b = nd.V3Batch(model, part, max_len=ctx_len + steps, max_chunk=32, ctx=ctxs[k])
            pr = np.ascontiguousarray(np.stack([S.prompt_tokens(ctx_len, 100 + k * part + i)
                                                for i in range(part)]), np.int32)
            nxt = None
            for t in range(0, ctx_len, 32):
                t1 = min(ctx_len, t + 32)
                nxt = b.prefill(pr[:, t:t1], want_next=(t1 == ctx_len))
            batches.append(b)
            firsts.append(nxt)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        outs = nd.V3Batch.greedy_many(batches, firsts, steps)
        t_dec2 = time.perf_counter() - t0
        toks2 = np.concatenate([np.concatenate([f[:, None], o[:, :-1]], axis=1)
                                for f, o in zip(firsts, outs)], axis=0)
        out[key][name] = {
            "workload": f"the same {sessions} sessions as {n} batches of {part} on {n} streams, "
                        "their greedy loops enqueued in turn from one host thread "
                        "(nd_v3_generate_many); projections batched over each batch's "
                        f"{part} sessions; {os.environ.get('GPU_MAX_HW_QUEUES', '4')} "
                        "hardware queues a process",
            "decode_tok_per_s": round(sessions * steps / t_dec2, 1),
            "decode_ms_per_step": round(t_dec2 / steps * 1e3, 3),
            "tokens_equal_one_batch": bool(np.array_equal(toks2, toks)),
        }
        for b in batches:
            b.close()
        for c in ctxs:
            c.close()
    if check:
        out[key]["check"] = forward_check(model, g, recs, toks, ctx_len, steps, run)
    model.close()
    return out


def forward_check(model, g, recs, toks, ctx_len, steps, run):
    """The timed multi-session run's greedy tokens for sessions 0 and B-1:
    equal to a batch-1 device run of the session, and to the oracle's
    decode_step over all ctx_len + steps positions (two host threads, the
    oracle splitting rows and heads across the rest, which keeps its bits)."""
    import threading
    import numpy as np
    import v3_synth as S
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    B = toks.shape[0]
    picks = sorted({0, B - 1})
    t0 = time.perf_counter()
    om = O.V3Model(g, recs, S.CODEBOOK)
    O.set_threads(max(1, _threads_all() // len(picks)), O.SPLIT_ALL)
    want = {}

    def oracle(i):
        want[i] = O.v3_generate(om, S.prompt_tokens(ctx_len, 100 + i), steps,
                                hint=ctx_len + steps)[0].astype(np.int32)
    th = [threading.Thread(target=oracle, args=(i,)) for i in picks]
    for t in th:
        t.start()
    batch1 = {i: run(1, ctx_len, steps, 32, S.prompt_tokens(ctx_len, 100 + i)[None])[2][0]
              for i in picks}
    for t in th:
        t.join()
    O.set_threads(1, O.SPLIT_REFERENCE)
    return {"sessions": picks, "tokens_per_session": steps,
            "equal_to_batch1_device_run": all(np.array_equal(batch1[i], toks[i]) for i in picks),
            "equal_to_oracle": all(np.array_equal(want[i], toks[i]) for i in picks),
            "seconds": round(time.perf_counter() - t0, 1)}


def main():
    global MIN_WARM_S
    args = parse()
    MIN_WARM_S = args.min_warm
    if args.summarize_trace:
        summarize_trace(args.summarize_trace, args.tail_steps, args.skip_steps)
        return
    if args.summarize_pmc:
        summarize_pmc(args.summarize_pmc, args.pmc_period, args.pmc_runs)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    import needle_amd as nd

    assert torch.cuda.is_available(), "bench needs a GPU"
    torch.cuda.set_device(0)
    ctx = nd.Ctx(0)
    gen = torch.Generator(device="cuda").manual_seed(1234)

    # ---- headline: batched codebook GEMV ------------------------------------
    R = GEMV_COPIES if args.only in (None, "gemv") else 1
    if args.only == "gemm":
        print(json.dumps({"secondary": {"prefill_gemm_bf16": gemm_runs(torch, nd, ctx, gen, args.steps)}}))
        ctx.close()
        return
    if args.only == "cqa":
        print(json.dumps({"secondary": {"format_a_gemv": format_a_runs(torch, nd, args.steps)}}))
        ctx.close()
        return
    if args.only == "forward":
        out = {"secondary": {"needle3_forward": forward_runs(
            torch, nd, ctx, args.forward_sessions, args.forward_ctx, not args.no_check)}}
        ctx.close()
        print(json.dumps(out))
        return
    W = torch.randint(0, 256, (R, GEMV_OUT, GEMV_IN), dtype=torch.uint8, device="cuda", generator=gen)
    CB = torch.randn(R, GEMV_OUT // 64, 256, device="cuda", generator=gen) * 0.02
    X = torch.randn(R, GEMV_IN, device="cuda", generator=gen)
    Y = torch.empty(R, GEMV_OUT, device="cuda")

    def gemv_step():
        nd.cb8_gemv_batched(ctx, W, CB, X, Y)

    ms = ms1 = float("nan")
    if args.only in (None, "gemv"):
        ms = timed_loop(torch, gemv_step, args.steps, args.warmup)
    step_bytes = R * GEMV_BYTES
    gbs = step_bytes / (ms * 1e-3) / 1e9

    if args.only is None:
        # batch-1 latency of one GEMV (a single 2.4 MB weight; L2/MALL-warm)
        w1, cb1, x1, y1 = W[0], CB[0], X[0], Y[0]
        ms1 = timed_loop(torch, lambda: nd.cb8_gemv(ctx, w1, cb1, x1, y1), 200, 20)

    result = {
        "metric": "codebook GEMV GB/s (% HBM peak); decode tok/s @ ctx2048 int8 KV",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "codebook dequant-GEMV, batch 1: W [3072 x 768] uint8 codes uniform "
                        "0..255, one 256-entry fp32 codebook per 64 rows ~N(0,0.02), x fp32 "
                        "[768] ~N(0,1); 448 distinct (W, codebook, x) problems per step in one "
                        "launch (1.086 GB per step)",
            "bytes_per_gemv": GEMV_BYTES,
            "gemvs_per_step": R,
            "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
            "single_gemv_us": round(ms1 * 1e3, 2),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": pmc_traffic("cb8_gemv_kernel<3>"),
            "kernel": "cb8_gemv_kernel<3>",
        },
    }

    # ---- secondary: int8 KV append + decode attention at ctx 2048 -----------
    if not args.no_secondary and args.only in (None, "attn"):
        S = ATT_SESSIONS
        g = nd.kv_geom(ATT_H, ATT_H, ATT_D, ATT_D, ATT_CTX)
        nb = nd.kv_block_bytes(g)
        off = nd.kv_offsets(g)
        blk = torch.empty(S * nb, dtype=torch.uint8, device="cuda")
        view = blk.view(S, nb)
        codes = torch.randint(-127, 128, (S, off["ks"]), dtype=torch.int8, device="cuda",
                              generator=gen)
        view[:, :off["ks"]].copy_(codes.view(torch.uint8))
        del codes
        scales = torch.rand(S, 2 * ATT_H * ATT_CTX, device="cuda", generator=gen) * 0.03 + 1e-3
        view[:, off["ks"]:off["ks"] + 8 * ATT_H * ATT_CTX].copy_(scales.view(torch.uint8).view(S, -1))
        del scales
        q = torch.randn(S, ATT_H * ATT_D, device="cuda", generator=gen)
        knew = torch.randn(S, ATT_H * ATT_D, device="cuda", generator=gen)
        vnew = torch.randn(S, ATT_H * ATT_D, device="cuda", generator=gen)
        pos = torch.full((S,), ATT_CTX - 1, dtype=torch.int32, device="cuda")
        lo = torch.zeros(S, dtype=torch.int32, device="cuda")
        out = torch.empty(S, ATT_H * ATT_D, device="cuda")

        def attn_only():
            nd.attend_step_i8(ctx, g, blk, nb, lo, pos, q, quant_query=True, out=out)

        def decode_step():
            nd.kv_write(ctx, g, blk, nb, pos, knew, vnew)
            attn_only()

        ms_dec = ms_att1 = float("nan")
        if args.only is None:
            ms_dec = timed_loop(torch, decode_step, max(10, args.steps // 2), 5)
        ms_att = timed_loop(torch, attn_only, max(10, args.steps // 2), 5)
        att_gbs = S * ATT_BYTES / (ms_att * 1e-3) / 1e9
        if args.only is None:
            one = lambda: nd.attend_step_i8(ctx, g, blk, nb, lo[:1], pos[:1], q[:1],
                                            quant_query=True, out=out[:1])
            ms_att1 = timed_loop(torch, one, 200, 20)
        result["secondary"] = {
            "decode_attention_int8_ctx2048": {
                "workload": f"{S} sessions x 12 heads x 64, ctx 2048, int8 K/V + f32 scales; "
                            "step = append one token per session + decode attention",
                "session_tokens_per_s": round(S / (ms_dec * 1e-3), 1),
                "ms_per_step": round(ms_dec, 4),
                "attention_GBps": round(att_gbs, 2),
                "attention_frac_hbm": round(att_gbs / HBM_PEAK_GBS, 4),
                "attention_traffic_bytes": pmc_traffic("attn_i8_kernel<1,64,64,16>"),
                "attention_algorithmic_bytes": S * ATT_BYTES,
                "bytes_per_session_decode": ATT_BYTES,
                "single_session_attention_us": round(ms_att1 * 1e3, 2),
            }
        }

    if not args.no_secondary and args.only in (None, "attn"):
        result.setdefault("secondary", {}).update(attention_ctx_runs(torch, nd, ctx, gen, args.steps))
        result["secondary"]["exact_attention_one_session"] = exact_attention_runs(torch, nd, ctx, gen)

    if not args.no_secondary and args.only is None:
        result.setdefault("secondary", {})["prefill_gemm_bf16"] = gemm_runs(torch, nd, ctx, gen, 50)

    if not args.no_secondary and args.only is None:
        result.setdefault("secondary", {})["format_a_gemv"] = format_a_runs(torch, nd, 50)

    if not args.no_secondary and not args.no_forward and args.only is None:
        result.setdefault("secondary", {})["needle3_forward"] = forward_runs(
            torch, nd, ctx, args.forward_sessions, args.forward_ctx, not args.no_check)

    if args.calibrate_copy:
        # A plain device copy of exactly 1 GiB: the byte counters' reference.
        a = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        del a, b

    ctx.close()
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result))


if __name__ == "__main__":
    main()
