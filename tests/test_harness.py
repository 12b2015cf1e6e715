"""The run-directory harness (fleet-amd-task_amd/harness/run_fleet.py, compare.py) on the CPU: the
verdict rules of the reference's harness/compare.py (compare_ids :161-178, compare_route_log
:181-236) on constructed run directories, and run_fleet's argument checks (no GPU is touched)."""
import json
import sys
from pathlib import Path

import numpy as np
import pytest

sys.path.insert(0, str(Path(__file__).resolve().parent.parent / "fleet-amd-task_amd" / "harness"))
import compare as C  # noqa: E402
import run_fleet as RF  # noqa: E402


def test_compare_ids_prefix_rules():
    assert C.compare_ids([1, 2, 3], [1, 2, 3])["result"] == "PASS"
    r = C.compare_ids([1, 2, 3], [1, 2])
    assert r["result"] == "PARTIAL" and r["matched_prefix"] == 2
    r = C.compare_ids([1, 2, 3], [1, 5, 3])
    assert r["result"] == "FAIL" and r["first_divergence"] == 1 and r["matched_prefix"] == 1


def _log(steps):
    return [[{"idx": list(ids), "w": []} for ids in step] for step in steps]


def test_route_log_exact_rule():
    ref = _log([[[1, 2, 3, 4, 5, 6]], [[6, 5, 4, 3, 2, 1]]])
    # Fleet logs the forced shared experts after the top-6; order inside the top-k is free
    fleet = _log([[[6, 5, 4, 3, 2, 1, 64, 65]], [[1, 2, 3, 4, 5, 6, 64, 65]]])
    assert C.compare_route_log(ref, fleet)["result"] == "PASS"
    fleet[1][0]["idx"][0] = 7
    r = C.compare_route_log(ref, fleet)
    assert r["result"] == "FAIL" and r["rule"] == "exact" and len(r["mismatches"]) == 1


def test_route_log_tie_cascade_disagreement():
    w = [0.0] * 64
    w[1], w[7] = 0.100, 0.1005          # within 1.5 % of the larger: a tie
    w[2], w[9] = 0.200, 0.100            # far apart: not a tie
    ref = [[{"idx": [1, 3, 4, 5, 6, 8], "w_all": w}], [{"idx": [2, 3, 4, 5, 6, 8], "w_all": w}]]
    tie_then_cascade = _log([[[7, 3, 4, 5, 6, 8]], [[9, 3, 4, 5, 6, 8]]])
    r = C.compare_route_log(ref, tie_then_cascade)
    assert r["rule"] == "tie" and len(r["ties"]) == 1 and len(r["cascades"]) == 1 and r["result"] == "PASS"
    disagreement_first = _log([[[1, 3, 4, 5, 6, 8]], [[9, 3, 4, 5, 6, 8]]])
    r = C.compare_route_log(ref, disagreement_first)
    assert len(r["disagreements"]) == 1 and r["result"] == "FAIL"


def test_run_writes_report(tmp_path):
    ref, fleet = tmp_path / "ref", tmp_path / "fleet"
    ref.mkdir()
    fleet.mkdir()
    (ref / "ref_output_ids.json").write_text(json.dumps([5, 6, 7]))
    (ref / "ref_route_log.json").write_text(json.dumps(_log([[[1, 2, 3, 4, 5, 6]]])))
    (fleet / "fleet_output_ids.json").write_text(json.dumps([5, 6, 7]))
    (fleet / "fleet_route_log.json").write_text(json.dumps(_log([[[1, 2, 3, 4, 5, 6, 64, 65]]])))
    (fleet / "fleet_run_meta.json").write_text(json.dumps({"head": True, "stop_after": None}))
    assert C.main(["--ref", str(ref), "--fleet", str(fleet)]) == 0
    rep = json.loads((fleet / "correctness_report.json").read_text())
    assert rep["overall"] == "PASS" and rep["output_ids"]["result"] == "PASS"
    (fleet / "fleet_output_ids.json").write_text(json.dumps([5, 9, 7]))
    assert C.main(["--ref", str(ref), "--fleet", str(fleet)]) == 1
    # a truncated run's placeholder ids are skipped, not failed
    (fleet / "fleet_run_meta.json").write_text(json.dumps({"head": False, "stop_after": "L1.o_proj"}))
    assert C.main(["--ref", str(ref), "--fleet", str(fleet)]) == 0


def test_run_fleet_refuses_bad_model_dirs_and_args(tmp_path):
    ap = RF.build_parser()
    with pytest.raises(SystemExit, match="no config.json"):
        RF.run(ap.parse_args(["--model-dir", str(tmp_path / "nonexistent"), "--out", str(tmp_path)]))
    other = tmp_path / "other"
    other.mkdir()
    (other / "config.json").write_text(json.dumps({
        "hidden_size": 4096, "num_attention_heads": 16, "qk_nope_head_dim": 128, "qk_rope_head_dim": 64,
        "v_head_dim": 128, "kv_lora_rank": 512, "vocab_size": 102400, "num_hidden_layers": 27,
        "intermediate_size": 10944, "moe_intermediate_size": 1408, "n_routed_experts": 64,
        "num_experts_per_tok": 6, "n_shared_experts": 2}))
    with pytest.raises(SystemExit, match="built for DeepSeek-V2-Lite"):
        RF.run(ap.parse_args(["--model-dir", str(other), "--out", str(tmp_path)]))
    with pytest.raises(SystemExit, match="--layers"):
        RF.run(ap.parse_args(["--layers", "28", "--out", str(tmp_path)]))
    with pytest.raises(SystemExit, match="--iters"):
        RF.run(ap.parse_args(["--iters", "0", "--out", str(tmp_path)]))


def test_route_log_json_format():
    rl = np.arange(2 * 3 * 8, dtype=np.int32).reshape(2, 3, 8)
    j = RF.route_log_json(rl, 2, 3)
    assert len(j) == 2 and len(j[0]) == 3 and j[1][2] == {"idx": list(range(40, 48)), "w": []}
