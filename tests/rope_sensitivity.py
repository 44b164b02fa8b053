"""How much the greedy tokens of the full-forward workloads depend on the last
bits of the RoPE table's transcendentals (libm 0.2.16's powf/cosf/sinf,
model.rs:376-394, math.rs:13-36), on the oracle.

Three tables: the reference's (libm restated), the same with theta^e
correctly rounded (or_powf is one ulp off at 3 of the 24 frequencies of the
shipped geometry), and the C library's powf/cosf/sinf.  Workloads: the
shipped geometry at random init (seed 0, int8 KV); one session with a
128-token prompt and 256 greedy tokens, and sessions 0 and 63 of the
64-session run (2048-token prompts, 128 greedy tokens), with the prompts
the benchmark uses.  Prints one JSON line per run and a summary.

Usage: python tests/rope_sensitivity.py [--jobs N] [--short]
(--short: 32-token prompts and 32 greedy tokens, a smoke run)."""
import argparse
import json
import os
import sys
import time
from concurrent.futures import ProcessPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
for p in (os.path.join(ROOT, "oracle"), os.path.join(ROOT, "needle-rs_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

VARIANTS = {"libm": 0, "powf_correctly_rounded": 1, "glibc": 2}


def run(job):
    import numpy as np
    import oracle as O
    import v3_synth as S
    name, prompt_len, seed, steps, variant = job
    O.set_rope_variant(VARIANTS[variant])
    g, recs = S.build_records(None, seed=0)
    om = O.V3Model(g, recs, S.CODEBOOK)
    t0 = time.perf_counter()
    toks, margins = O.v3_generate(om, S.prompt_tokens(prompt_len, seed), steps,
                                  hint=prompt_len + steps)
    return {"workload": name, "variant": variant, "tokens": toks.tolist(),
            "min_margin": float(np.min(margins)), "seconds": round(time.perf_counter() - t0, 1)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=os.cpu_count() or 1)
    ap.add_argument("--short", action="store_true")
    a = ap.parse_args()
    if a.short:
        work = [("1 session, 32 + 32", 32, 100, 32)]
    else:
        work = [("1 session, prompt 128 + 256 greedy", 128, 100, 256),
                ("session 0 of 64, prompt 2048 + 128 greedy", 2048, 100, 128),
                ("session 63 of 64, prompt 2048 + 128 greedy", 2048, 163, 128)]
    jobs = [(n, pl, sd, st, v) for (n, pl, sd, st) in work for v in VARIANTS]
    with ProcessPoolExecutor(max_workers=a.jobs) as ex:
        res = list(ex.map(run, jobs))
    summary = []
    for n, *_ in work:
        rows = {r["variant"]: r for r in res if r["workload"] == n}
        base = rows["libm"]["tokens"]
        for v, r in rows.items():
            diff = [i for i, (x, y) in enumerate(zip(base, r["tokens"])) if x != y]
            line = {"workload": n, "variant": v, "tokens": len(base),
                    "tokens_differing_from_libm": len(diff),
                    "first_differing_step": diff[0] if diff else None,
                    "min_top1_top2_margin": round(r["min_margin"], 6), "seconds": r["seconds"]}
            print(json.dumps(line), flush=True)
            summary.append(line)
    print(json.dumps({"all_tokens_identical": all(s["tokens_differing_from_libm"] == 0
                                                  for s in summary)}))


if __name__ == "__main__":
    main()
