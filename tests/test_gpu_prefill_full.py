"""The batched GPU prefill (fleet/prefill.py) at the benched size: 27 layers, ctx 1,024 (BASELINE
configs[3]; the reference times its prefill and checks its decode the same way,
harness/run_reference.py:367-376, 414-425).

  * decode after the batched prefill: 4 greedy tokens from position 1023 with the persistent
    kernel, against the oracle decoding from the same cache rows: the ids and every MoE layer's
    route ids equal (the decode path is bit-exact given its cache);
  * the batched prefill's cache rows against the teacher-forced prefill of the decode kernel (the
    path whose every step is bit-exact with the oracle: test_gpu_model.py, test_gpu_full_model.py),
    per layer: relative error of c_kv and k_pe, reported. The batched prefill runs its GEMMs
    through rocBLAS in another summation order, so its rows differ by bf16 roundings, and each layer
    adds its own to the residual stream it inherits: measured on MI355X, layer 0 is bit-equal,
    layer 1 at 7.6e-3 and the error grows as a random walk to 3.5e-2 at layer 26 (about 7e-3
    sqrt(l)). The bound held is the reference's class threshold for these boundaries (1e-2,
    harness/common.py:27-37) per layer, accumulated in quadrature: 1e-2 sqrt(l) at layer l >= 1.
"""
import time

import numpy as np
import pytest

from oracle import model as M
from fleet import build_graph as B
from fleet import graph_plan as G
from fleet import pack_weights as P
from fleet import prefill as PF
from fxtest import SEED, GpuWeights

pytestmark = pytest.mark.gpu


def test_batched_prefill_27_layers_ctx1024(rt):
    d = P.REAL_DIMS
    L, ctx, n_new = d.L, 1024, 4
    s_max = ctx + n_new
    print(f"[prefill27] layers={L} ctx={ctx} n_new={n_new}", flush=True)
    packed = P.fill_seeded(rt, d, SEED, L, True)
    prompt = P.prompt_ids(SEED, ctx, d.V)
    plan = G.build_plan(d, s_max, L, True)
    cap = B.make_capture(rt, plan)
    runner = B.build(rt, packed, cap, B.make_meta(rt, s_max, prompt), d, s_max, L, True)
    cfg = M.cfg_for_plan(plan)

    t0 = time.time()
    pf = PF.Prefill(rt, packed, runner.host, d, ctx, L, plan.eps, plan.scale)
    pf.run(runner.host["tokens"])
    rt.synchronize()
    print(f"[prefill27] batched prefill of {ctx - 1} positions in {time.time() - t0:.2f} s", flush=True)
    batched = {}
    for l in range(L):
        batched[l] = (cap[f"c_kv_{l}"].download()[:ctx - 1], cap[f"k_pe_{l}"].download()[:ctx - 1])

    # decode from the batched prefill's cache; the oracle from the same rows
    runner.run(n_new, ctx - 1, ctx)
    got_ids = runner.host["tokens"].download()[ctx:ctx + n_new].tolist()
    route_log = runner.host["route_log"].download()
    cos, sin = M.rope_tables(s_max)
    W = GpuWeights(packed)
    cache = M.Cache(cfg, s_max, L)
    for l in range(L):
        cache.c_kv[l][:ctx - 1], cache.k_pe[l][:ctx - 1] = batched[l]
    want, routes = M.generate(cfg, W, cache, cos, sin, prompt, n_new, layers=L, prefill_from=ctx - 1)
    print(f"[prefill27] decode ids {got_ids} oracle {want}", flush=True)
    assert got_ids == want
    for i in range(n_new):
        for j, r in enumerate(routes[i]):
            assert route_log[i, j].tolist() == r, (i, j, route_log[i, j].tolist(), r)

    # the decode kernel's teacher-forced prefill of the same prompt, then the per-layer comparison
    t0 = time.time()
    runner.run(ctx - 1, 0, ctx)
    print(f"[prefill27] decode-kernel prefill of {ctx - 1} positions in {time.time() - t0:.2f} s", flush=True)
    worst = 0.0
    for l in range(L):
        for k, name in enumerate(("c_kv", "k_pe")):
            ref = cap[f"{name}_{l}"].download()[:ctx - 1]
            got = batched[l][k]
            a, b = P.bf16_to_f32(got).astype(np.float64), P.bf16_to_f32(ref).astype(np.float64)
            rel = float(np.linalg.norm(a - b) / np.linalg.norm(b))
            mx = float(np.max(np.abs(a - b)))
            same = float(np.mean(got == ref))
            print(f"[prefill27] layer {l:2d} {name}: rel err {rel:.2e}, max abs {mx:.3g}, bit-equal {100 * same:.1f} %",
                  flush=True)
            worst = max(worst, rel)
            if l == 0:
                assert same > 0.99, (l, name, same)
            else:
                assert rel < 1e-2 * np.sqrt(l), (l, name, rel)
    print(f"[prefill27] worst per-layer rel err {worst:.2e}", flush=True)
    pf.free()
