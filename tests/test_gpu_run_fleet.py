"""run_fleet.py end to end on the GPU against a reference directory written from the oracle, then
judged by compare.py: the reference's run_fleet -> compare flow (harness/run_fleet.py:449-616,
harness/compare.py:318-378) on a 2-layer model."""
import json
import sys
from pathlib import Path

import pytest

from oracle import model as M
from fleet import graph_plan as G
from fleet import pack_weights as P
from fxtest import SEED, GpuWeights

sys.path.insert(0, str(Path(__file__).resolve().parent.parent / "fleet-amd-task_amd" / "harness"))
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
    cfg = M.Cfg(H=d.H, NH=d.NH, D_N=d.D_N, D_R=d.D_R, D_V=d.D_V, D_C=d.D_C, V=d.V, L=d.L, I_DENSE=d.I_DENSE,
                I_MOE=d.I_MOE, E=d.E, TOPK=d.TOPK, N_SHARED=d.N_SHARED, eps=plan.eps, scale=plan.scale,
                split=plan.split, n_splits=plan.n_splits)
    cos, sin = M.rope_tables(s_max)
    W = GpuWeights(P.fill_seeded(rt, d, SEED, layers=layers, head=True))
    ids, routes = M.generate(cfg, W, M.Cache(cfg, s_max, layers), cos, sin,
                             P.prompt_ids(SEED, ctx, d.V), iters, layers=layers)
    ref = tmp_path / "ref"
    ref.mkdir()
    (ref / "ref_output_ids.json").write_text(json.dumps(ids))
    (ref / "ref_route_log.json").write_text(json.dumps([[{"idx": r[:d.TOPK]} for r in step] for step in routes]))
    res = C.run(ref, fleet, fleet / "correctness_report.md")
    print(f"[run_fleet] fleet ids {meta['output_ids']} oracle ids {ids}: {res['overall']}", flush=True)
    assert res["output_ids"]["result"] == "PASS", res["output_ids"]
    assert res["route_log"]["result"] == "PASS", res["route_log"]["mismatches"][:3]
    assert res["overall"] == "PASS"
