#!/usr/bin/env python3
"""Benchmark of BASELINE.json's metric: us per decoded token (batch 1, ctx 1024) and the fraction of
the HBM roofline, on one MI355X.

Workload: the full 27-layer DeepSeek-V2-Lite with random-init bf16 weights
~N(0, 0.02) from a seed (norm weights 1.0), a 1,024-token prompt drawn uniformly from the 102,400-id
vocabulary with a seed, an untimed prefill that writes the latent caches of positions 0..1022
(--prefill batched, the default: one forward pass over all prompt positions, fleet/prefill.py;
--prefill decode: teacher-forced iterations of the persistent kernel, head skipped), then greedy
decode at batch 1. A "step" is one decoded token; `--steps` tokens are timed, starting at position 1023
(so every timed token attends over 1,024..1,024+steps-1 positions), after `--warmup` untimed
tokens at the same positions. Inputs are resident in HBM when the timed region starts.

value        us per decoded token: the K timed tokens are one persistent launch of K iterations
             (--launch one, the default: fx_launch with iters = K, as the reference's run_fleet.py
             decodes its 32 tokens in one mpk() call, harness/run_fleet.py:590-593); HIP events on
             the launch's stream around it / K. --launch per-token queues K one-iteration launches
             back to back instead (no host wait in between; each launch adds its own start-up).
             The warmup tokens are one launch of their own before the events. Decode runs under the
             kernel symbol fx_persistent (a --prefill decode prefill under fx_prefill, the batched
             one in rocBLAS and fx_pf_* kernels), so a kernel trace of this command lists the
             decode launches alone under fx_persistent
roofline     algorithmic HBM bytes per token (every weight the token touches once -- 8 of the 66
             experts per MoE layer -- plus the latent-cache rows read and the embedding row; mean
             over the timed tokens) / us per token, against the published 8 TB/s (the same as the
             launch's bytes / its duration); traffic = the measured HBM bytes per token from the
             committed rocprofv3 --pmc summary x the tokens of one timed launch
cpu_baseline the CPU oracle (oracle/, a C port of harness/numpy_ref.py semantics, OpenMP) decoding
             the first `--cpu-tokens` tokens of the same run on this host's cores, checked for
             equal ids; weights it touches are copied to host memory before its timed region

    python bench.py [--gpus 1] [--steps 32] [--warmup 2]
"""
import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "fleet-amd-task_amd"))

import numpy as np  # noqa: E402

from fleet import build_graph as B  # noqa: E402
from fleet import graph_plan as G  # noqa: E402
from fleet import pack_weights as P  # noqa: E402
from fleet import prefill as PF  # noqa: E402
from fleet import runtime as R  # noqa: E402

HBM_PEAK_GBPS = 8000.0
METRIC = "µs/decoded token (batch 1, ctx 1024) and % of HBM roofline on 1 MI355X"


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def traffic_per_token(ctx):
    """Measured HBM bytes per decoded token of fx_persistent from the committed rocprofv3 --pmc summary
    (FETCH_SIZE and WRITE_SIZE per dispatch, each scaled by the same counter's reading on a copy kernel
    of known size, over the dispatch's decode iterations), or None. Counters cannot be read inside
    this process, so the figure comes from the profile runs."""
    f = ROOT / "profiles" / "fx_persistent_decode_ctx1024_traffic.json"
    if ctx != 1024 or not f.exists():
        return None
    t = json.loads(f.read_text())
    return t["bytes_per_dispatch"] / t.get("iters_per_dispatch", 1)


def config_name(ctx):
    """The BASELINE.json config a context length is quoted on: configs[3] at 1,024, configs[4] at 16,384."""
    return {1024: "BASELINE configs[3]", 16384: "BASELINE configs[4]"}.get(ctx, f"BASELINE configs[3] at ctx {ctx}")


def cpu_baseline(rt, runner, bufs, plan, prompt, ctx, n_tok, gpu_ids):
    """Time the oracle on the host decoding n_tok tokens from position ctx - 1 with the GPU prefill's
    cache rows 0..ctx-2 (test infrastructure: the checker, run here only as the reported baseline)."""
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as O
    from oracle import model as M

    d = plan.dims
    cfg = M.cfg_for_plan(plan)
    cache = M.Cache(cfg, plan.s_max)
    for l in range(d.L):
        cache.c_kv[l][:ctx - 1] = runner.host[f"c_kv_{l}"].download()[:ctx - 1]
        cache.k_pe[l][:ctx - 1] = runner.host[f"k_pe_{l}"].download()[:ctx - 1]
    cos, sin = M.rope_tables(plan.s_max)
    # host copies of every weight the sampled tokens touch (routes from the GPU run's route log)
    W = {}
    for key in ("W_embed", "w_final_norm"):
        W[key] = bufs[key].download()
    head_q = None
    if plan.fp8_head:
        buf = bufs["W_lmq"]
        head_q = (buf.download_range(0, d.V * d.H).reshape(d.V, d.H),
                  buf.download_range(d.V * d.H, 4 * d.V).view(np.float32))
    else:
        W["W_lm"] = bufs["W_lm"].download()
    for l in range(d.L):
        for key in (f"w_norm1_{l}", f"w_norm2_{l}", f"W_qkva_{l}", f"w_kv_norm_{l}", f"W_uk_{l}", f"W_uv_{l}", f"W_o_{l}"):
            W[key] = bufs[key].download()
    W["W_gu_0"], W["W_down_0"] = bufs["W_gu_0"].download(), bufs["W_down_0"].download()
    rl = runner.host["route_log"].download()
    experts = {}
    fp8 = plan.fp8_experts
    for l in range(1, d.L):
        W[f"W_gate_{l}"] = bufs[f"W_gate_{l}"].download()
        for i in range(n_tok):
            for e in rl[i, l - 1].tolist():
                if fp8:
                    for key, rows, K in ((f"W13q_{l}", 2 * d.I_MOE, d.H), (f"W2q_{l}", d.H, d.I_MOE)):
                        if (key, e) not in experts:
                            buf = bufs[key]
                            q = buf.download_range(e * rows * K, rows * K).reshape(rows, K)
                            sc = buf.download_range(d.E_TOTAL * rows * K + 4 * e * rows, 4 * rows).view(np.float32)
                            experts[(key, e)] = (q, sc)
                    continue
                for key, per in ((f"W13_{l}", 2 * d.I_MOE * d.H), (f"W2_{l}", d.H * d.I_MOE)):
                    if (key, e) not in experts:
                        shape = bufs[key].shape[1:]
                        experts[(key, e)] = bufs[key].download_range(e * per, per).reshape(shape)

    class HostW(dict):
        fp8_experts = fp8
        fp8_head = plan.fp8_head

        def fp8_rows(self, key, rows, K):
            return head_q

        def expert(self, key, e):
            return experts[(key, e)]

        def fp8_expert(self, key, e, rows, K):
            return experts[(key, e)]

    Wh = HostW(W)
    threads = O.num_threads()
    tok = int(prompt[ctx - 1])
    times, ids = [], []
    for i in range(n_tok):
        t0 = time.perf_counter()
        tok, _, _ = M.decode_step(cfg, Wh, cache, cos, sin, tok, ctx - 1 + i, d.L, True)
        times.append(time.perf_counter() - t0)
        ids.append(tok)
    return {"value": round(1e6 * statistics.median(times), 1), "unit": "µs/token", "cores": threads,
            "kind": "port", "sample": f"{n_tok} greedy decode tokens (positions {ctx - 1}..{ctx - 2 + n_tok}) of the "
                                      f"same 27-layer model and prompt; oracle/fleet_oracle.c with {threads} OpenMP "
                                      f"threads, weights resident in host memory; median per token",
            "ids_equal_gpu": ids == gpu_ids[:n_tok]}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=32, help="timed decode tokens")
    ap.add_argument("--warmup", type=int, default=2, help="untimed decode tokens before the timed ones")
    ap.add_argument("--ctx", type=int, default=1024, help="prompt length (positions attended by the first token)")
    ap.add_argument("--seed", type=int, default=20261201)
    ap.add_argument("--cpu-tokens", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--n-splits", type=int, default=None, help="attention split count (default: the plan's own)")
    ap.add_argument("--split", type=int, default=None, help="attention split length in positions (a multiple of 32)")
    ap.add_argument("--no-pair", action="store_true",
                    help="run o_proj and the expert gate|up stage as two operators (no early expert loads)")
    ap.add_argument("--attn", choices=("mfma", "xcd", "valu"), default=None,
                    help="attention kernel: matrix cores over all workers (mfma), matrix cores with the merge on one "
                         "XCD (xcd), or vector-ALU chains per XCD (valu); default: the plan's own choice for the "
                         "cache length")
    ap.add_argument("--fp8-experts", action="store_true",
                    help="the experts' weights as FP8 (weight-only e4m3, per-row scales) instead of bf16")
    ap.add_argument("--fp8-head", action="store_true", help="the LM head's weights as FP8 too (implies --fp8-experts)")
    ap.add_argument("--launch", choices=("one", "per-token"), default="one",
                    help="the timed tokens as one launch of --steps iterations, or one launch per token")
    ap.add_argument("--prefill", choices=("batched", "decode"), default="batched",
                    help="how the untimed prefill writes the caches (batched forward pass or the decode kernel)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (this build has no multi-GPU path; --gpus {args.gpus} is not "
              f"supported): run it with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py is single-process, single-GPU", file=sys.stderr)
        sys.exit(2)

    d = P.REAL_DIMS
    ctx, K, Wm = args.ctx, args.steps, args.warmup
    s_max = ctx + max(K, Wm, 1)
    rt = R.Runtime(0)
    log("device", rt.info())
    t0 = time.time()
    bufs = P.fill_seeded(rt, d, args.seed, d.L, True)
    gen_s = time.time() - t0
    log(f"seeded weights: {P.packed_bytes(d) / 2**30:.2f} GiB in {gen_s:.1f} s")
    prompt = P.prompt_ids(args.seed, ctx, d.V)
    if args.fp8_head:
        args.fp8_experts = True
    if args.fp8_experts:
        t0 = time.time()
        P.quantize_experts(rt, bufs, d, d.L)
        if args.fp8_head:
            P.quantize_head(rt, bufs, d)
        log(f"FP8 experts{' and LM head' if args.fp8_head else ''}: quantized in {time.time() - t0:.1f} s")
    plan_kw = dict(split=args.split, n_splits=args.n_splits, fp8_experts=args.fp8_experts, fp8_head=args.fp8_head,
                   attn=args.attn, pair=not args.no_pair)
    plan = G.build_plan(d, s_max, d.L, True, **plan_kw)
    meta = B.make_meta(rt, s_max, prompt)
    cap = B.make_capture(rt, plan)
    runner = B.build(rt, bufs, cap, meta, d, s_max, d.L, True, **plan_kw)
    log(f"plan: {len(runner.stages)} stages/iteration, {plan.n_splits} splits of {plan.split}, s_max {s_max}")
    t0 = time.time()
    prefill_warm_s = None
    if args.prefill == "batched":
        pf = PF.Prefill(rt, bufs, runner.host, d, ctx, d.L, plan.eps, plan.scale, G.ROUTED_SCALING)
        pf.run(runner.host["tokens"])
        prefill_s = time.time() - t0
        # again, past rocBLAS's one-time kernel loading (the same inputs write the same rows)
        t1 = time.time()
        pf.run(runner.host["tokens"])
        prefill_warm_s = time.time() - t1
        pf.free()
    else:
        runner.run(ctx - 1, 0, ctx)
        prefill_s = time.time() - t0
    log(f"{args.prefill} prefill of {ctx - 1} positions: {prefill_s:.2f} s"
        + (f", {prefill_warm_s:.3f} s once the GEMM kernels are loaded" if prefill_warm_s else ""))
    assert K + 1 <= R.FX_MAX_MARKS, "at most 255 timed tokens"
    if Wm > 0:
        runner.launch(Wm, ctx - 1, ctx)
        runner.finish()
        log(f"warmup: {Wm} tokens")
    t0 = time.perf_counter()
    rt.mark(0)
    if args.launch == "one":
        runner.launch(K, ctx - 1, ctx)
        rt.mark(1)
    else:
        for i in range(K):
            runner.launch(1, ctx - 1 + i, ctx)
            rt.mark(i + 1)
    runner.finish()
    wall_ms = 1e3 * (time.perf_counter() - t0)
    n_marks = 1 if args.launch == "one" else K
    us_tok = 1e3 * rt.marks_ms(0, n_marks) / K
    # per-token times: the kernel's own iteration stamps (one launch) or the events around each launch
    per_tok = ([float(x) for x in runner.timing_us()] if args.launch == "one"
               else [1e3 * rt.marks_ms(i, i + 1) for i in range(K)])
    ids = runner.host["tokens"].download()[ctx:ctx + K].tolist()
    mean_bytes = sum(P.bytes_per_token(d, ctx + i, fp8_experts=args.fp8_experts, fp8_head=args.fp8_head)
                     for i in range(K)) / K
    achieved = mean_bytes / (us_tok * 1e-6) / 1e9
    tokens_per_launch = K if args.launch == "one" else 1
    tpt = traffic_per_token(ctx)
    what = "in-kernel per-iteration" if args.launch == "one" else "per-launch event"
    log(f"decode: {us_tok:.1f} us/token (events, {args.launch} launch), wall {wall_ms / K * 1e3:.1f} us/token, "
        f"{what} median {statistics.median(per_tok):.1f} min {min(per_tok):.1f} max {max(per_tok):.1f} us; "
        f"{achieved:.0f} GB/s = {100 * achieved / HBM_PEAK_GBPS:.1f}% of 8 TB/s")
    log(f"ids {ids}")
    out = {
        "metric": METRIC, "value": round(us_tok, 2), "unit": "µs/token", "n_gpus": 1, "steps": K, "warmup": Wm,
        "ms_per_step": round(us_tok / 1e3, 5), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": ("fp8-e4m3 expert and LM head weights x bf16" if args.fp8_head else
                  "fp8-e4m3 expert weights x bf16" if args.fp8_experts else "bf16"),
        "data": "synthetic: seeded N(0,0.02) bf16 weights" + (
            " (experts and LM head quantized to FP8, per-row scales)" if args.fp8_head else
            " (experts quantized to FP8, per-row scales)" if args.fp8_experts else "")
                + f", seeded uniform {ctx}-token prompt",
        "config": {"workload": f"{config_name(ctx)}: DeepSeek-V2-Lite 27 layers, {ctx}-token prompt (prefill untimed), "
                               "greedy decode at batch 1", "layers": d.L, "batch": 1, "ctx": ctx, "decode_tokens": K,
                   "splits": plan.n_splits, "split": plan.split, "attn": plan.attn, "pair": plan.pair, "seed": args.seed, "fp8_experts": args.fp8_experts,
                   "fp8_head": args.fp8_head},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": None if args.fp8_experts or tpt is None else int(tpt * tokens_per_launch),
                     "bytes_per_launch": int(mean_bytes * tokens_per_launch), "tokens_per_launch": tokens_per_launch,
                     "bytes_per_token": int(mean_bytes), "kernel": "fx_persistent"},
        "launch": args.launch, "token_us_median": round(statistics.median(per_tok), 2),
        "token_us_source": "fx_persistent iteration stamps (s_memrealtime)" if args.launch == "one"
                           else "HIP events around each launch",
        "prefill": args.prefill,
        "prefill_s": round(prefill_s, 3), "prefill_warm_s": None if prefill_warm_s is None else round(prefill_warm_s, 3),
        "ids": ids,
    }
    if not args.no_cpu_baseline:
        log(f"cpu baseline: oracle on {args.cpu_tokens} tokens")
        try:
            out["cpu_baseline"] = cpu_baseline(rt, runner, bufs, plan, prompt, ctx, args.cpu_tokens, ids)
            log(f"cpu baseline {out['cpu_baseline']['value']} us/token on {out['cpu_baseline']['cores']} threads, "
                f"ids equal: {out['cpu_baseline']['ids_equal_gpu']}")
        except Exception as e:  # the baseline is reported, never the measured value
            out["cpu_baseline"] = {"value": None, "error": repr(e)}
    print(json.dumps(out), flush=True)
    # explicit teardown (every device buffer freed, then the context destroyed) before the
    # interpreter exits, so no HIP call runs during its finalisation
    del runner, bufs, cap, meta
    rt.close()


if __name__ == "__main__":
    main()
