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
  - the Needle-3 forward (shipped geometry, random init, int8 KV cache),
    bit-identical to the CPU oracle: one session with a 128-token prompt and
    256 greedy tokens, and 64 sessions each prefilled with 2048 tokens then
    128 greedy tokens in lockstep ("decode tok/s @ ctx2048 int8 KV").

cpu_baseline: the oracle's Format-B GEMV (the closed form, fp32, row-parallel
with OpenMP like the reference's rayon row bands) on the host cores, on a
bounded sample of the same workload.

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
    p.add_argument("--only", choices=["gemv", "attn", "forward", "gemm", "cqa"], default=None,
                   help="run one workload only, without the batch-1 latency probes "
                        "(for per-kernel profiles)")
    p.add_argument("--min-warm", type=float, default=0.5,
                   help="seconds of untimed warm-up before each timed loop (0 for counter runs)")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="also run a plain 1 GiB device copy (PMC byte-counter scale)")
    p.add_argument("--summarize-trace", metavar="CSV", default=None,
                   help="no GPU: print per-kernel statistics of the last --tail-steps forward "
                        "steps of a rocprofv3 kernel-trace CSV (steps end at k_final)")
    p.add_argument("--tail-steps", type=int, default=128)
    return p.parse_args()


def summarize_trace(path, nsteps):
    """Per-kernel durations over the last `nsteps` forward steps of a
    rocprofv3 --kernel-trace CSV.  Each step launches k_final once, so the
    window starts after the (nsteps + 1)-th last k_final ends; kernels of the
    side stream in that window are included."""
    import collections
    import csv
    rows = []
    with open(path) as f:
        for r in csv.DictReader(f):
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    rows.sort()
    finals = [i for i, r in enumerate(rows) if "::k_final(" in r[2]]
    t0 = rows[finals[-(nsteps + 1)]][1]
    sel = [r for r in rows if r[0] > t0]
    agg = collections.defaultdict(list)
    for a, b, n in sel:
        agg[n].append(b - a)
    span = (max(r[1] for r in sel) - t0) / 1e3
    print(f"last {nsteps} steps: {span / nsteps:.1f} us per step (profiler on), {len(sel)} kernels")
    print("| kernel | per step | avg us | min us | max us | us per step |")
    print("|---|---|---|---|---|---|")
    for n, v in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
        name = n.replace("(anonymous namespace)::", "").split("(")[0]
        if name.startswith("void "):
            name = name[5:]
        print(f"| `{name}` | {len(v) / nsteps:.2f} | {sum(v) / len(v) / 1e3:.2f} | "
              f"{min(v) / 1e3:.2f} | {max(v) / 1e3:.2f} | {sum(v) / nsteps / 1e3:.1f} |")


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


def cpu_baseline(seconds=12.0):
    """Oracle Format-B GEMV on the host: 64 distinct copies (151 MB), looped
    until `seconds` have elapsed, OpenMP over the rows."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    rng = np.random.default_rng(1)
    copies = 64
    W = rng.integers(0, 256, size=(copies, GEMV_OUT, GEMV_IN), dtype=np.uint8)
    CB = rng.normal(0, 0.02, size=(copies, GEMV_OUT // 64, 256)).astype(np.float32)
    X = rng.normal(size=(copies, GEMV_IN)).astype(np.float32)
    y = np.zeros(GEMV_OUT, np.float32)
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    O.cb8_gemv_omp(W[0], CB[0], X[0], y)  # warm
    calls, t0 = 0, time.perf_counter()
    while True:
        i = calls % copies
        O.cb8_gemv_omp(W[i], CB[i], X[i], y)
        calls += 1
        el = time.perf_counter() - t0
        if el >= seconds and calls >= copies:
            break
    return {"value": round(calls * GEMV_BYTES / el / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"{calls} GEMVs of 3072x768 u8 over 64 distinct weight copies in "
                      f"{el:.1f} s (oracle or_cb8_gemv_omp, {threads} OpenMP threads)"}


BF16_MFMA_PEAK_TFLOPS = 2500.0


def gemm_runs(torch, nd, ctx, gen, steps):
    """Format B prefill GEMM, Y [512 x N] = X [512 x 768] . decode(W [N x 768]),
    bf16 MFMA with fp32 accumulate, for the two projection widths; R
    distinct problems per launch (one launch per step) so the step is long
    enough to time on the device."""
    out = {}
    M, K = 512, 768
    for N, R in ((3072, 32), (768, 64)):
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
    per call.  Spans of 2048 and more sum the softmax with the parallel fold."""
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


def forward_runs(torch, nd, ctx, sessions, ctx_len, cpu_tokens=8):
    """The Needle-3 forward on the device: batch 1 (128-token prompt, 256
    greedy steps) and `sessions` sessions prefilled with `ctx_len` tokens
    then 128 greedy steps.  Wall-clock over host-driven steps, each greedy
    step ending with its tokens back on the host."""
    import numpy as np
    import v3_synth as S
    g, recs = S.build_records(None, seed=0)
    model = nd.V3Model(ctx, g, recs, S.CODEBOOK)
    out = {}

    def run(B, prompt_len, steps, chunk):
        batch = nd.V3Batch(model, B, max_len=prompt_len + steps, max_chunk=chunk)
        prompts = np.stack([S.prompt_tokens(prompt_len, 100 + i) for i in range(B)]).astype(np.int32)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        nxt = None
        for t in range(0, prompt_len, chunk):
            t1 = min(prompt_len, t + chunk)
            nxt = batch.prefill(prompts[:, t:t1], want_next=(t1 == prompt_len))
        torch.cuda.synchronize()
        t_pre = time.perf_counter() - t0
        t0 = time.perf_counter()
        for _ in range(steps):
            nxt = batch.step(nxt)
        t_dec = time.perf_counter() - t0
        batch.close()
        return t_pre, t_dec

    # warm, untimed: code objects, and about half a second of steps so the
    # clocks have left their idle state before the timed decode
    run(1, 16, 240, 16)
    t_pre, t_dec = run(1, 128, 256, 128)
    out["batch1_prompt128_greedy256"] = {
        "workload": "shipped Needle-3 geometry (20 layers, d 768, 12 q / 2 kv heads, vocab "
                    "8192), random init, Cactus-Quants weights, int8 KV; one session, "
                    "128-token uniform prompt prefilled in one pass, then 256 greedy tokens",
        "prefill_ms": round(t_pre * 1e3, 3),
        "prefill_ms_per_token": round(t_pre / 128 * 1e3, 4),
        "decode_ms_per_token": round(t_dec / 256 * 1e3, 3),
        "decode_tok_per_s": round(256 / t_dec, 1),
    }
    t_pre, t_dec = run(sessions, ctx_len, 128, 32)
    out[f"sessions{sessions}_ctx{ctx_len}_greedy128"] = {
        "workload": f"{sessions} sessions of the same model in lockstep, each prefilled with "
                    f"{ctx_len} uniform prompt tokens (32 positions per pass), then 128 greedy "
                    "steps; projections batched over sessions, attention per session",
        "decode_tok_per_s": round(sessions * 128 / t_dec, 1),
        "decode_ms_per_step": round(t_dec / 128 * 1e3, 3),
        "prefill_tok_per_s": round(sessions * ctx_len / t_pre, 1),
    }
    # the oracle's decode step on one host core, for scale
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    om = O.V3Model(g, recs, S.CODEBOOK)
    cache = om.new_cache(64, True)
    toks = S.prompt_tokens(cpu_tokens, 7)
    cache.decode_step(toks[0])
    t0 = time.perf_counter()
    for t in toks[1:]:
        cache.decode_step(t)
    out["cpu_oracle_decode_ms_per_token"] = round((time.perf_counter() - t0) / (cpu_tokens - 1) * 1e3, 2)
    out["cpu_oracle_note"] = ("the oracle's scalar decode step (1 host core, reference float "
                              "order) on the same model; the reference publishes 8.72 ms/token "
                              "for its own multi-threaded NEON build on an M5 Max")
    out["bit_identical_to_oracle"] = "yes (tests/test_gpu_v3.py)"
    model.close()
    return out


def main():
    global MIN_WARM_S
    args = parse()
    MIN_WARM_S = args.min_warm
    if args.summarize_trace:
        summarize_trace(args.summarize_trace, args.tail_steps)
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
            torch, nd, ctx, args.forward_sessions, args.forward_ctx)}}
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
            torch, nd, ctx, args.forward_sessions, args.forward_ctx)

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
