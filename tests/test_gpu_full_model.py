"""The whole 27-layer model through the persistent kernel against the oracle, bit for bit, at the
BASELINE's full-model configs (the reference judges its own 27-layer run with compare.py,
harness/compare.py:318-378, after run_fleet.py --layers 27 --head --iters 32, README.md:308):

- ctx 1,024. Every layer's latent cache holds N(0,1) rows at positions 0..1022 (the
  oracle generator's streams, written on the device by the bit-identical generator), the token at
  position 1023 is the prompt's last; 4 greedy tokens from step 1023.
- ctx 16,384 with 128 attention splits of 128 positions: 16,383 cached rows, 2 tokens,
  so the first token attends over exactly 128 splits and the second over 129.

Compared: the greedy ids, every layer's route ids, every cache row the run wrote (all 27 layers),
and the residual stream after the last layer (x_res), each bit for bit.

The prompt's other tokens are not decoded (the cache stands in for their prefill); the GPU prefill
at the benched size is covered by test_gpu_prefill.py."""
import numpy as np
import pytest

from oracle import oracle as O
from oracle import model as M
from fleet import build_graph as B
from fleet import graph_plan as G
from fleet import pack_weights as P
from fxtest import SEED, GpuWeights, mismatch

pytestmark = pytest.mark.gpu


def _seed_caches(rt, cap, layers, rows, d):
    for l in range(layers):
        rt.gen_normal_bf16(cap[f"c_kv_{l}"], rows * d.D_C, SEED, P.fnv1a32(f"cache.c_kv.{l}"), 1.0)
        rt.gen_normal_bf16(cap[f"k_pe_{l}"], rows * d.D_R, SEED, P.fnv1a32(f"cache.k_pe.{l}"), 1.0)
    rt.synchronize()


@pytest.mark.parametrize("ctx,n_new,split", [(1024, 4, None), (16384, 2, 128)], ids=["configs3_ctx1024", "configs4_ctx16384"])
def test_full_model_decode_matches_oracle(rt, ctx, n_new, split):
    d = P.REAL_DIMS
    L = d.L
    s_max = ctx + n_new
    print(f"[full] layers={L} ctx={ctx} n_new={n_new} split={split}", flush=True)
    bufs = P.fill_seeded(rt, d, SEED, L, True)
    prompt = P.prompt_ids(SEED, ctx, d.V)
    plan = G.build_plan(d, s_max, L, True, split=split)
    if split:
        assert plan.split == split and -(-ctx // split) == 128
    cap = B.make_capture(rt, plan)
    _seed_caches(rt, cap, L, ctx - 1, d)
    runner = B.build(rt, bufs, cap, B.make_meta(rt, s_max, prompt), d, s_max, L, True, split=split)
    print(f"[full] plan: {len(runner.stages)} stages, {plan.n_splits} splits of {plan.split}, attn {plan.attn}",
          flush=True)
    runner.run(n_new, ctx - 1, ctx)
    got_ids = runner.host["tokens"].download()[ctx:ctx + n_new].tolist()
    route_log = runner.host["route_log"].download()
    x_gpu = runner.x_res()
    print(f"[full] gpu ids {got_ids}", flush=True)

    # the oracle from the same cache rows (the device generator's bits are checked on a slice)
    cfg = M.cfg_for_plan(plan)
    cache = M.Cache(cfg, s_max, L)
    for l in range(L):
        cache.c_kv[l][:ctx - 1] = cap[f"c_kv_{l}"].download()[:ctx - 1]
        cache.k_pe[l][:ctx - 1] = cap[f"k_pe_{l}"].download()[:ctx - 1]
    ref0 = O.gen_normal_bf16(SEED, P.fnv1a32("cache.c_kv.0"), 4096, 1.0)
    assert mismatch(cache.c_kv[0].reshape(-1)[:4096], ref0) == 0
    cos, sin = M.rope_tables(s_max)
    W = GpuWeights(bufs)
    tok = int(prompt[ctx - 1])
    ids, routes, x = [], [], None
    for i in range(n_new):
        tok, r, x = M.decode_step(cfg, W, cache, cos, sin, tok, ctx - 1 + i, L, True)
        ids.append(tok)
        routes.append(r)
    print(f"[full] oracle ids {ids}", flush=True)

    # cache rows first: they localise a divergence to a layer and a position
    for l in range(L):
        g_ck = cap[f"c_kv_{l}"].download_range((ctx - 1) * d.D_C, n_new * d.D_C).reshape(n_new, d.D_C)
        g_kp = cap[f"k_pe_{l}"].download_range((ctx - 1) * d.D_R, n_new * d.D_R).reshape(n_new, d.D_R)
        assert mismatch(g_ck, cache.c_kv[l][ctx - 1:ctx - 1 + n_new]) == 0, f"layer {l}: c_kv rows differ"
        assert mismatch(g_kp, cache.k_pe[l][ctx - 1:ctx - 1 + n_new]) == 0, f"layer {l}: k_pe rows differ"
    for i in range(n_new):
        for j, r in enumerate(routes[i]):
            assert route_log[i, j].tolist() == r, (i, j, route_log[i, j].tolist(), r)
    assert got_ids == ids
    assert mismatch(x_gpu, x) == 0
