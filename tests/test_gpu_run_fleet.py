"""run_fleet.py end to end on the GPU against a reference directory written from the oracle, then
judged by compare.py: the reference's run_fleet -> compare flow (harness/run_fleet.py:449-616,
harness/compare.py:318-378) on a 2-layer model, ids, route log and boundary tensors (decode step 0
and the last iteration, as the reference's F2 rule reads them)."""
import json
import sys
from pathlib import Path

import numpy as np
import pytest

from oracle import model as M
from fleet import graph_plan as G
from fleet import pack_weights as P
from fxtest import SEED, GpuWeights, ref_boundaries

sys.path.insert(0, str(Path(__file__).resolve().parent.parent / "fleet-amd-task_amd" / "harness"))
import boundaries as BD  # noqa: E402
import compare as C  # noqa: E402
import run_fleet as RF  # noqa: E402

pytestmark = pytest.mark.gpu


def test_run_fleet_then_compare(rt, tmp_path):
    layers, ctx, iters = 2, 40, 3
    fleet = tmp_path / "fleet"
    print(f"[run_fleet] layers={layers} ctx={ctx} iters={iters}", flush=True)
    meta = RF.run(RF.build_parser().parse_args(["--layers", str(layers), "--head", "--iters", str(iters),
                                                "--ctx", str(ctx), "--out", str(fleet)]), rt=rt)
    assert meta["completed"] and len(meta["output_ids"]) == iters
    for f in ("plan.json", "fleet_run_meta.json", "fleet_output_ids.json", "fleet_route_log.json", "wall.json"):
        assert (fleet / f).exists(), f
    # the reference directory from the oracle on the same seeded model and prompt
    d = P.REAL_DIMS
    s_max = ctx + iters
    plan = G.build_plan(d, s_max, layers, True)
    cfg = M.cfg_for_plan(plan)
    cos, sin = M.rope_tables(s_max)
    W = GpuWeights(P.fill_seeded(rt, d, SEED, layers=layers, head=True))
    prompt = P.prompt_ids(SEED, ctx, d.V)
    cache = M.Cache(cfg, s_max, layers)
    for pos in range(ctx - 1):
        M.decode_step(cfg, W, cache, cos, sin, prompt[pos], pos, layers, head=False)
    ids, routes, recs = [], [], []
    tok = int(prompt[-1])
    for i in range(iters):
        rec = {}
        tok, r, _ = M.decode_step(cfg, W, cache, cos, sin, tok, ctx - 1 + i, layers, head=True, rec=rec)
        ids.append(tok)
        routes.append(r)
        recs.append(rec)
    ref = tmp_path / "ref"
    ref.mkdir()
    (ref / "ref_output_ids.json").write_text(json.dumps(ids))
    (ref / "ref_route_log.json").write_text(json.dumps([[{"idx": r[:d.TOPK]} for r in step] for step in routes]))
    BD.write(ref / "ref_boundaries_step0.safetensors", ref_boundaries(recs[0], d.TOPK))
    BD.write(ref / f"ref_boundaries_step{iters - 1}.safetensors", ref_boundaries(recs[-1], d.TOPK))
    res = C.run(ref, fleet, fleet / "correctness_report.md")
    print(f"[run_fleet] fleet ids {meta['output_ids']} oracle ids {ids}: {res['overall']}", flush=True)
    assert res["output_ids"]["result"] == "PASS", res["output_ids"]
    assert res["route_log"]["result"] == "PASS", res["route_log"]["mismatches"][:3]
    rows = res["boundaries"]
    keys = {r["key"] for r in rows}
    for k in ("L1.B2.q", "L0.B3.c_kv", "L1.B3.k_pe", "L1.B4.q_pe", "L1.B6.attn", "L1.B7.x_res_attn",
              "L1.B8.router_logits", "L1.B9.topk_idx", "L1.B10.topk_w", "L1.B12.shared", "L1.B13.layer_out",
              "head.B15.logits", "head.B16.token"):
        assert k in keys, k
    assert sum(k.startswith("L1.B11.expert_") for k in keys) == d.TOPK
    bad = [(r["key"], r["result"], r.get("rel_err"), r.get("detail")) for r in rows if r["result"] != "PASS"]
    assert not bad, bad
    # this build is bit-exact with the oracle at every boundary
    assert all(r.get("rel_err", 0.0) == 0.0 for r in rows), [(r["key"], r["rel_err"]) for r in rows if r.get("rel_err")]
    assert res["overall"] == "PASS" and res["n_not_comparable"] == 0


def test_bitdiff_of_two_runs_is_zero(rt, tmp_path):
    """bitdiff.py over two run_fleet dumps of the same seeded run: every boundary key on both sides,
    no element differs (the decode is deterministic to the bit)."""
    import bitdiff as BDIFF
    dirs = []
    for name in ("a", "b"):
        out = tmp_path / name
        print(f"[bitdiff] run_fleet into {out}", flush=True)
        meta = RF.run(RF.build_parser().parse_args(["--layers", "2", "--head", "--iters", "2", "--ctx", "24",
                                                    "--out", str(out)]), rt=rt)
        assert meta["completed"]
        dirs.append(out)
    text = BDIFF.run(*dirs, out=tmp_path / "bitdiff.md")
    rows = [l for l in text.splitlines() if l.startswith("| `")]
    assert len(rows) >= 20, text
    assert "only in" not in text, text
    for l in rows:
        c = [x.strip() for x in l.split("|")[1:-1]]
        assert c[3] == "0" and c[4] == "0", l
