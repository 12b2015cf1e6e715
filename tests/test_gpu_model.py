"""End-to-end parity of the persistent decode kernel (fx_run) against the oracle composition
(oracle/model.py) on the same seeded weights and prompt: greedy ids, per-layer route ids, every
latent-cache row the run wrote, the final hidden state and the last step's intermediate buffers,
all bit for bit.

The full 27-layer model at BASELINE configs 3 and 4 is in test_gpu_full_model.py; here the real
dims with fewer layers keep the oracle in seconds. Both attention kernels (matrix-core "mfma", the
default, and vector-ALU "valu") run every case."""
import numpy as np
import pytest

from oracle import oracle as O
from oracle import model as M
from fleet import build_graph as B
from fleet import graph_plan as G
from fleet import pack_weights as P
from fxtest import SEED, GpuWeights, mismatch

pytestmark = pytest.mark.gpu


def oracle_cfg(plan, layers):
    return M.cfg_for_plan(plan)


def _run_model(rt, layers, n_prompt, n_new, s_max, attn, seed=SEED):
    """attn: the plan's attention, with "-nopair" for o_proj and the gate|up stage as two operators."""
    pair = not attn.endswith("-nopair")
    attn = attn.split("-")[0]
    d = P.REAL_DIMS
    bufs = P.fill_seeded(rt, d, seed, layers=layers, head=True)
    prompt = P.prompt_ids(seed, n_prompt, d.V)
    plan = G.build_plan(d, s_max, layers, True, attn=attn, pair=pair)
    meta = B.make_meta(rt, s_max, prompt)
    cap = B.make_capture(rt, plan)
    runner = B.build(rt, bufs, cap, meta, d, s_max, layers, True, attn=attn, pair=pair)
    print(f"[model] attn={attn} pair={pair} layers={layers} n_prompt={n_prompt} n_new={n_new} "
          f"stages={len(runner.stages)}", flush=True)
    runner.run(n_prompt - 1 + n_new, 0, n_prompt)
    return d, bufs, prompt, plan, runner, cap


@pytest.mark.parametrize("attn", ["mfma", "mfma-nopair", "xcd", "valu"])
@pytest.mark.parametrize("layers,n_prompt,n_new", [(2, 40, 4), (3, 70, 3)])
def test_decode_matches_oracle(rt, layers, n_prompt, n_new, attn):
    s_max = 96
    d, bufs, prompt, plan, runner, cap = _run_model(rt, layers, n_prompt, n_new, s_max, attn)
    W = GpuWeights(bufs)
    cfg = oracle_cfg(plan, layers)
    cos, sin = M.rope_tables(s_max)
    cache = M.Cache(cfg, s_max, layers)
    ids, routes = M.generate(cfg, W, cache, cos, sin, prompt, n_new, layers=layers)
    got_tokens = runner.host["tokens"].download()
    print(f"[model] oracle ids {ids} gpu ids {got_tokens[n_prompt:n_prompt + n_new].tolist()}", flush=True)
    # caches first: they localise a divergence to a position and a layer
    last = n_prompt - 1 + n_new - 1
    for l in range(layers):
        gck = cap[f"c_kv_{l}"].download()[:last + 1]
        gkp = cap[f"k_pe_{l}"].download()[:last + 1]
        bad = [t for t in range(last + 1) if mismatch(gck[t], cache.c_kv[l][t]) or mismatch(gkp[t], cache.k_pe[l][t])]
        assert not bad, f"layer {l}: cache rows differ from position {bad[0]} ({len(bad)} rows)"
    assert got_tokens[n_prompt:n_prompt + n_new].tolist() == ids
    assert got_tokens[:n_prompt].tolist() == prompt.tolist()
    if layers >= 2:
        rl = runner.host["route_log"].download()
        for i in range(n_new):
            for j, r in enumerate(routes[i]):
                assert rl[i, j].tolist() == r, (i, j, rl[i, j].tolist(), r)


@pytest.mark.parametrize("attn", ["mfma", "xcd", "valu"])
def test_last_step_buffers_match_oracle(rt, attn):
    """One decode iteration of a 2-layer model from a seeded random cache (BASELINE config 0's
    setting: 1,024 cached positions ~N(0,1)); every workspace the last layer leaves behind is
    compared (qkva, ql_nope, q_pe, partials, merged o, attn, router logits, top-k, act8, out8,
    logits, x_res)."""
    d = P.REAL_DIMS
    layers, s_max, step = 2, 1056, 1024
    bufs = P.fill_seeded(rt, d, SEED, layers=layers, head=True)
    plan = G.build_plan(d, s_max, layers, True, attn=attn)
    cache = {"c_kv": [], "k_pe": []}
    for l in range(layers):
        cache["c_kv"].append(O.gen_normal_bf16(SEED, P.fnv1a32(f"cache.c_kv.{l}"), step * d.D_C, 1.0).reshape(step, d.D_C))
        cache["k_pe"].append(O.gen_normal_bf16(SEED, P.fnv1a32(f"cache.k_pe.{l}"), step * d.D_R, 1.0).reshape(step, d.D_R))
    token = 4242
    tokens = np.zeros(s_max, np.int64)
    tokens[step] = token
    meta = B.make_meta(rt, s_max, tokens)
    cap = B.make_capture(rt, plan, cache)
    runner = B.build(rt, bufs, cap, meta, d, s_max, layers, True, attn=attn)
    runner.run(1, step, step + 1)
    W = GpuWeights(bufs)
    cfg = oracle_cfg(plan, layers)
    cos, sin = M.rope_tables(s_max)
    oc = M.Cache(cfg, s_max, layers)
    for l in range(layers):
        oc.c_kv[l][:step] = cache["c_kv"][l]
        oc.k_pe[l][:step] = cache["k_pe"][l]
    rec = {}
    tok, routes, x = M.decode_step(cfg, W, oc, cos, sin, token, step, layers, True, rec)
    h = runner.host
    l = layers - 1
    live = -(-(step + 1) // plan.split)
    checks = {
        "qkva": (h["qkva"].download(), np.concatenate([rec[f"L{l}.B2.q"], rec[f"L{l}.kva"]])),
        "ql_nope": (h["ql_nope"].download(), rec[f"L{l}.ql_nope"]),
        "q_pe": (h["q_pe"].download(), rec[f"L{l}.B4.q_pe"]),
        "partials": (h["partials"].download()[:live, :, :d.D_C + 1], rec[f"L{l}.partials"][:live, :, :d.D_C + 1]),
        "o_merged": (h["o_merged"].download(), rec[f"L{l}.o_merged"]),
        "attn": (h["attn"].download(), rec[f"L{l}.B6.attn"]),
        "logits_router": (h["logits_router"].download(), rec[f"L{l}.B8.router_logits"]),
        "topk_w": (h["topk_w"].download(), rec[f"L{l}.B10.topk_w"]),
        "mask": (h["mask"].download(), rec[f"L{l}.mask"]),
        "act8": (h["act8"].download(), rec[f"L{l}.act8"]),
        "out8": (h["out8"].download(), rec[f"L{l}.out8"]),
        "logits": (h["logits"].download(), rec["head.B15.logits"]),
        "x_res": (runner.x_res(), x),
        "c_kv row": (cap[f"c_kv_{l}"].download()[step], rec[f"L{l}.B3.c_kv"]),
    }
    bad = {k: mismatch(a, b) for k, (a, b) in checks.items()}
    print(f"[buffers] mismatches {bad}", flush=True)
    assert all(v == 0 for v in bad.values()), bad
    assert int(h["tokens"].download()[step + 1]) == tok
