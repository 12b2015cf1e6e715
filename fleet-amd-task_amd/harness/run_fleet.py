#!/usr/bin/env python3
"""Decode driver of the gfx950 path: the counterpart of the reference's harness/run_fleet.py
(main :449-616), writing the same run directory files that harness/compare.py reads.

    python fleet-amd-task_amd/harness/run_fleet.py --layers 27 --head --iters 32 [--ctx 1024 | --prompt ids.json]
                                                   [--seed S] [--stop-after L1.o_proj] [--out DIR] [--event-timing]

What differs from the reference, and why:
  * without --model-dir the weights are the seeded bf16 model (fleet/pack_weights.fill_seeded,
    plain RoPE, scale 192^-0.5); with it, the checkpoint's safetensors shards are loaded into the
    same packed keys (fleet/checkpoint.py) and the config's YaRN tables, softmax scale and norm eps
    are used;
  * the prompt's cache rows 0 .. n_prompt - 2 are produced on the GPU instead of being captured from
    the HF prefill (--ref's ref_cache.safetensors): by default by the decode kernel itself
    (teacher-forced iterations, head skipped; the whole run is one fx_run over positions
    0 .. n_prompt - 2 + iters), with --prefill batched by one forward pass over all prompt positions
    (fleet/prefill.py: rocBLAS GEMMs + this library's row kernels), then fx_run from n_prompt - 1;
  * there is no compile step (fx_load_plan validates and uploads the task table).

Files written to --out (the reference's names and formats):
  plan.json              the plan (build_graph.plan_json)
  fleet_run_meta.json    the run's arguments, sizes, device buffer addresses, outputs, "completed"
  fleet_output_ids.json  the greedy ids at positions n_prompt .. n_prompt + iters - 1
  fleet_route_log.json   [step][moe layer] {"idx": [8 expert ids], "w": []}
  fleet_boundaries.safetensors  the boundary tensors under the reference's keys (harness/boundaries.py):
                         decode step 0's when --iters 1, else the last iteration's (cache rows and
                         the first token are always step 0's)
  event_timing.json      with --event-timing: per-stage timing of the last iteration (fx_set_profile)
  wall.json              wall-clock seconds of the fill, build and run
Exit status 0 on success; a failed launch raises FxError with the library's message (nonzero exit).
"""
import argparse
import json
import sys
import time
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(PKG))
from fleet import build_graph as B  # noqa: E402
from fleet import graph_plan as G  # noqa: E402
from fleet import pack_weights as P  # noqa: E402
from fleet import checkpoint as CK  # noqa: E402
from fleet import prefill as PF  # noqa: E402
from fleet import runtime as R  # noqa: E402

sys.path.insert(0, str(Path(__file__).resolve().parent))
import boundaries as BD  # noqa: E402

N_PROMPT = 1024
SEED = 20261201


def build_parser():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--layers", type=int, default=None, help="decoder layers (default: all 27)")
    ap.add_argument("--head", action="store_true", help="final norm + LM head + greedy argmax")
    ap.add_argument("--iters", type=int, default=1, help="decode iterations from position n_prompt - 1")
    ap.add_argument("--stop-after", default=None, help="operator label, e.g. L1.o_proj (truncated graph)")
    ap.add_argument("--prompt", default=None, help="JSON list of prompt token ids (default: --ctx seeded ids)")
    ap.add_argument("--ctx", type=int, default=N_PROMPT, help="seeded prompt length when --prompt is not given")
    ap.add_argument("--seed", type=int, default=SEED, help="weight and prompt seed")
    ap.add_argument("--split", type=int, default=None, help="attention split length (a multiple of 32)")
    ap.add_argument("--n-splits", type=int, default=None, help="attention split count (default: the plan's own)")
    ap.add_argument("--attn", choices=("mfma", "xcd", "valu"), default=None,
                    help="attention kernel: matrix cores over all workers (mfma), matrix cores with the merge on one "
                         "XCD (xcd), or vector-ALU chains per XCD (valu); default: the plan's own choice")
    ap.add_argument("--out", default=None, help="run directory (default: harness/fleet_out/<name>)")
    ap.add_argument("--event-timing", action="store_true", help="per-stage stamps of the last iteration")
    ap.add_argument("--prefill", choices=("decode", "batched"), default="decode",
                    help="decode: the prompt positions run through the decode kernel (teacher-forced, bit-exact "
                         "with the oracle); batched: one forward pass over all prompt positions (fleet/prefill.py)")
    ap.add_argument("--final", action="store_true", help="accepted for the reference's command line; this build "
                                                         "has one configuration")
    ap.add_argument("--model-dir", default=None, help="HF snapshot directory (config.json + safetensors shards); "
                                                      "default: the seeded model")
    return ap


def run_name(args):
    parts = [f"L{args.layers}", "head" if args.head else "nohead", f"it{args.iters}"]
    if args.stop_after:
        parts.append(f"stop-{args.stop_after}")
    return "_".join(parts)


def route_log_json(rl, iters, n_moe):
    return [[{"idx": rl[s, j].tolist(), "w": []} for j in range(n_moe)] for s in range(iters)]


def run(args, rt=None):
    """Run the decode described by `args` (build_parser's namespace) and write the run directory.
    Returns the fleet_run_meta dict. `rt`: an existing Runtime (else one is created)."""
    d = P.REAL_DIMS
    mcfg = None
    if args.model_dir:
        if not (Path(args.model_dir) / "config.json").exists():
            raise SystemExit(f"run_fleet: {args.model_dir} has no config.json (an HF snapshot directory is expected)")
        mcfg = CK.read_config(args.model_dir)
        if mcfg.dims != d:
            raise SystemExit(f"run_fleet: the kernels are built for DeepSeek-V2-Lite's shapes {d}; {args.model_dir} "
                             f"has {mcfg.dims}")
    layers = args.layers if args.layers is not None else d.L
    if not 1 <= layers <= d.L:
        raise SystemExit(f"run_fleet: --layers must be in [1, {d.L}]")
    if args.iters < 1:
        raise SystemExit("run_fleet: --iters must be >= 1")
    if args.prompt:
        prompt = np.asarray(json.loads(Path(args.prompt).read_text()), np.int64)
    else:
        prompt = P.prompt_ids(args.seed, args.ctx, d.V)
    n_prompt = len(prompt)
    if n_prompt < 1 or prompt.min() < 0 or prompt.max() >= d.V:
        raise SystemExit(f"run_fleet: the prompt needs at least one id, every id in [0, {d.V})")
    s_max = n_prompt + args.iters
    out = Path(args.out) if args.out else PKG / "harness" / "fleet_out" / run_name(args)
    out.mkdir(parents=True, exist_ok=True)
    own_rt = rt is None
    if own_rt:
        rt = R.Runtime(0)
    try:
        t0 = time.time()
        if mcfg is not None:
            packed = CK.load_packed(rt, args.model_dir, d, layers=layers, head=args.head)
        else:
            packed = P.fill_seeded(rt, d, args.seed, layers=layers, head=args.head)
        t_pack = time.time() - t0
        t1 = time.time()
        plan_kw = {"attn": args.attn}
        if mcfg is not None:
            plan_kw.update(softmax_scale=mcfg.scale, eps=mcfg.eps)
        if args.split:
            plan_kw["split"] = args.split
        if args.n_splits:
            plan_kw["n_splits"] = args.n_splits
        meta = B.make_meta(rt, s_max, prompt)
        cap = B.make_capture(rt, G.build_plan(d, s_max, layers, args.head, **plan_kw),
                             tables=mcfg.tables(s_max) if mcfg is not None else None)
        runner = B.build(rt, packed, cap, meta, d, s_max, layers, args.head, stop_after=args.stop_after, **plan_kw)
        pj = B.plan_json(runner.plan)
        (out / "plan.json").write_text(json.dumps(pj) + "\n")
        t_build = time.time() - t1
        meta_out = {
            "layers": layers, "head": args.head, "iters": args.iters, "stop_after": args.stop_after,
            "s_max": s_max, "n_prompt": n_prompt, "seed": None if mcfg else args.seed,
            "model_dir": args.model_dir, "softmax_scale": runner.plan.scale, "eps": runner.plan.eps,
            "split": runner.plan.split,
            "n_splits": runner.plan.n_splits, "ops": len(pj["calls"]), "stages": len(runner.stages),
            "device": rt.info(), "addresses": {k: int(v.ptr) for k, v in runner.host.items()}, "completed": False,
        }
        (out / "fleet_run_meta.json").write_text(json.dumps(meta_out, indent=2) + "\n")
        total = n_prompt - 1 + args.iters
        t2 = time.time()
        t_prefill = None
        step0, n_iter = 0, total
        if args.prefill == "batched":
            pf = PF.Prefill(rt, packed, runner.host, d, n_prompt, layers, runner.plan.eps, runner.plan.scale,
                            G.ROUTED_SCALING)
            pf.run(runner.host["tokens"])
            pf.free()
            t_prefill = time.time() - t2
            step0, n_iter = n_prompt - 1, args.iters
        if args.event_timing:
            rows = runner.profile(n_iter, step0, n_prompt, iteration=n_iter - 1)
            (out / "event_timing.json").write_text(json.dumps(rows) + "\n")
        else:
            runner.run(n_iter, step0, n_prompt)
        t_run = time.time() - t2
        ids = runner.host["tokens"].download()[n_prompt:n_prompt + args.iters].tolist()
        if not args.head or args.stop_after:
            ids = [0] * args.iters   # a truncated graph writes no ids (compare.py skips them)
        (out / "fleet_output_ids.json").write_text(json.dumps(ids) + "\n")
        n_moe = max(0, layers - 1)
        if n_moe and "route_log" in runner.host:
            rl = runner.host["route_log"].download()
            (out / "fleet_route_log.json").write_text(json.dumps(route_log_json(rl, args.iters, n_moe)) + "\n")
        bnd, notes = BD.dump(pj["calls"], runner.host, n_prompt, d.TOPK, d.Q_OUT, args.iters)
        BD.write(out / "fleet_boundaries.safetensors", bnd, {"iters": args.iters, "n_prompt": n_prompt})
        meta_out.update({"boundaries": sorted(bnd), "boundary_notes": notes})
        wall = {"run_wall_s": t_run, "iters": args.iters, "positions": total, "pack_s": t_pack, "build_s": t_build,
                "prefill": args.prefill, "prefill_s": t_prefill}
        (out / "wall.json").write_text(json.dumps(wall) + "\n")
        meta_out.update({"output_ids": ids, "timings_s": wall, "completed": True})
        (out / "fleet_run_meta.json").write_text(json.dumps(meta_out, indent=2) + "\n")
        print(f"ids {ids}; {total} positions in {t_run * 1e3:.1f} ms -> {out}", flush=True)
        return meta_out
    finally:
        if own_rt:
            rt.close()


def main(argv=None):
    run(build_parser().parse_args(argv))


if __name__ == "__main__":
    main()
