"""Whole-model composition of the oracle: one batch-1 decode step of DeepSeek-V2-Lite.

TEST INFRASTRUCTURE ONLY (see oracle/oracle.py). It chains the per-kernel oracle functions in the
order of the reference's task graph (fleet/graph_plan.py:380-603, the --final stack of
harness/run_fleet.py:291-298): embed, then per layer norm1+qkva, mla_prep (with the cache
append), mla_attend, merge+W_uv, o_proj with the residual, then the dense MLP (layer 0) or the
router, w13+silu, w2 and the combine (layers >= 1), then the final norm, the LM head and the
argmax. numpy_ref.py has no whole-model driver (numpy_ref.py:1-26); this composition follows HF
modeling_deepseek.py:1193-1234 (decoder layer: residual around attention and around the MLP).

Weights are a mapping of the plan's packed keys (pack_weights names, suffix _l per layer) to
uint16 arrays; a mapping may also provide .expert(key, e) to hand over one expert slab lazily.
A mapping with fp8_experts = True provides .fp8_expert(key, e, rows, K) -> (codes uint8 [rows, K],
scales float32 [rows]) of the FP8 expert weights (W13q_l, W2q_l) instead.
"""
from dataclasses import dataclass

import numpy as np

from . import oracle as O


@dataclass(frozen=True)
class Cfg:
    H: int = 2048
    NH: int = 16
    D_N: int = 128
    D_R: int = 64
    D_V: int = 128
    D_C: int = 512
    V: int = 102400
    L: int = 27
    I_DENSE: int = 10944
    I_MOE: int = 1408
    E: int = 64
    TOPK: int = 6
    N_SHARED: int = 2
    eps: float = 1e-6
    scale: float = float(np.float32(1.0 / np.sqrt(192.0)))
    split: int = 32
    n_splits: int = 33
    attn: str = "valu"      # attention arithmetic: "valu" (chains) or "mfma" (matrix-core order)

    @property
    def Q_OUT(self):
        return self.NH * (self.D_N + self.D_R)


def cfg_for_plan(plan):
    """The oracle configuration of a decode plan (fleet.graph_plan.Plan): its dims, eps, softmax
    scale, attention splits and attention arithmetic."""
    d = plan.dims
    return Cfg(H=d.H, NH=d.NH, D_N=d.D_N, D_R=d.D_R, D_V=d.D_V, D_C=d.D_C, V=d.V, L=d.L, I_DENSE=d.I_DENSE,
               I_MOE=d.I_MOE, E=d.E, TOPK=d.TOPK, N_SHARED=d.N_SHARED, eps=plan.eps, scale=plan.scale,
               split=plan.split, n_splits=plan.n_splits, attn=getattr(plan, "attn", "valu"))


def _expert(W, key, e):
    if hasattr(W, "expert"):
        return W.expert(key, e)
    return W[key][e]


class Cache:
    """Latent cache of every layer: c_kv [L][S_max, D_C], k_pe [L][S_max, D_R] (bf16 bits)."""

    def __init__(self, cfg, s_max, layers=None):
        n = cfg.L if layers is None else layers
        self.c_kv = [np.zeros((s_max, cfg.D_C), np.uint16) for _ in range(n)]
        self.k_pe = [np.zeros((s_max, cfg.D_R), np.uint16) for _ in range(n)]
        self.s_max = s_max


def layer_step(cfg, W, cache, cos, sin, x_res, step, l, rec=None):
    """One decoder layer at position `step`; returns the new x_res. rec (a dict) collects the
    boundaries under the harness's keys (harness/common.py:44-59)."""
    c = cfg
    qkva, h1 = O.linear(W[f"W_qkva_{l}"], x_res, norm_w=W[f"w_norm1_{l}"], eps=c.eps)
    c_row, k_pe_row, ql, qp = O.mla_prep(qkva, W[f"w_kv_norm_{l}"], W[f"W_uk_{l}"], cos[step], sin[step],
                                        c.NH, c.D_N, c.D_R, c.D_C, c.eps)
    cache.c_kv[l][step] = c_row
    cache.k_pe[l][step] = k_pe_row
    attend = O.mla_attend_mfma if c.attn in ("mfma", "xcd") else O.mla_attend
    partials = attend(ql, qp, cache.c_kv[l], cache.k_pe[l], step, c.scale, c.split, c.n_splits)
    attn, obf = O.mla_merge_uv(partials, W[f"W_uv_{l}"], step, c.split)
    x_attn, _ = O.linear(W[f"W_o_{l}"], attn, res=x_res)
    if rec is not None:
        rec.update({f"L{l}.B1.norm1": h1, f"L{l}.B2.q": qkva[:c.Q_OUT], f"L{l}.kva": qkva[c.Q_OUT:],
                    f"L{l}.B3.c_kv": c_row, f"L{l}.B3.k_pe": k_pe_row, f"L{l}.B4.q_pe": qp,
                    f"L{l}.ql_nope": ql, f"L{l}.partials": partials, f"L{l}.o_merged": obf,
                    f"L{l}.B6.attn": attn, f"L{l}.B7.x_res_attn": x_attn})
    if l == 0:
        h, act, x_out = O.dense_mlp(x_attn, W[f"w_norm2_{l}"], W[f"W_gu_{l}"], W[f"W_down_{l}"], c.eps)
        if rec is not None:
            rec.update({f"L{l}.norm2": h, f"L{l}.act": act, f"L{l}.B13.layer_out": x_out})
        return x_out, None
    h, logits, topk_w, routing, mask = O.moe_router(x_attn, W[f"W_gate_{l}"], norm_w=W[f"w_norm2_{l}"], eps=c.eps,
                                                    topk=c.TOPK, n_forced=c.N_SHARED)
    n_slots = c.TOPK + c.N_SHARED
    ids = [int(e) for e in mask[:n_slots]]
    local = np.arange(n_slots + 1, dtype=np.int32)
    local[n_slots] = n_slots
    if getattr(W, "fp8_experts", False):
        # FP8 expert weights: codes and per-row scales of each slot's expert
        q13, s13 = zip(*[W.fp8_expert(f"W13q_{l}", e, 2 * c.I_MOE, c.H) for e in ids])
        q2, s2 = zip(*[W.fp8_expert(f"W2q_{l}", e, c.H, c.I_MOE) for e in ids])
        act = O.moe_w13_silu_fp8(h, np.stack(q13), np.stack(s13), local, n_slots)
        out8 = O.moe_w2_fp8(act, np.stack(q2), np.stack(s2), local, n_slots)
    else:
        W13 = np.stack([_expert(W, f"W13_{l}", e) for e in ids])
        W2 = np.stack([_expert(W, f"W2_{l}", e) for e in ids])
        act = O.moe_w13_silu(h, W13, local, n_slots)
        out8 = O.moe_w2(act, W2, local, n_slots)
    x_out = O.moe_combine(out8, topk_w, x_attn)
    if rec is not None:
        rec.update({f"L{l}.norm2": h, f"L{l}.B8.router_logits": logits, f"L{l}.B9.topk_idx": mask[:c.TOPK].copy(),
                    f"L{l}.B10.topk_w": topk_w, f"L{l}.routing": routing, f"L{l}.mask": mask,
                    f"L{l}.act8": act, f"L{l}.out8": out8, f"L{l}.B13.layer_out": x_out})
    return x_out, ids


def decode_step(cfg, W, cache, cos, sin, token, step, layers=None, head=True, rec=None):
    """Embed `token` at position `step`, run the layers and (head) the LM head + argmax.
    Returns (next_token or None, route ids per MoE layer [list of 8 ids], final x_res)."""
    n = cfg.L if layers is None else layers
    x = np.ascontiguousarray(W["W_embed"][int(token)])
    routes = []
    for l in range(n):
        x, ids = layer_step(cfg, W, cache, cos, sin, x, step, l, rec)
        if ids is not None:
            routes.append(ids)
    if not head:
        return None, routes, x
    if getattr(W, "fp8_head", False):
        q, sc = W.fp8_rows("W_lmq", cfg.V, cfg.H)
        logits, hf = O.linear_fp8(q, sc, x, norm_w=W["w_final_norm"], eps=cfg.eps)
    else:
        logits, hf = O.linear(W["W_lm"], x, norm_w=W["w_final_norm"], eps=cfg.eps)
    tok = O.argmax_bf16(logits)
    if rec is not None:
        rec.update({"head.B14.norm": hf, "head.B15.logits": logits, "head.B16.token": np.array([tok], np.int64)})
    return tok, routes, x


def generate(cfg, W, cache, cos, sin, prompt, n_new, layers=None, prefill_from=0, on_token=None):
    """Prefill positions [prefill_from, len(prompt)-1) without the head (the cache rows before
    prefill_from must already be in `cache`), then n_new greedy steps from position len(prompt)-1.
    Returns (ids [n_new], routes [n_new][moe layers][8])."""
    n_prompt = len(prompt)
    for pos in range(prefill_from, n_prompt - 1):
        decode_step(cfg, W, cache, cos, sin, prompt[pos], pos, layers, head=False)
    ids, routes = [], []
    tok = int(prompt[-1])
    for i in range(n_new):
        step = n_prompt - 1 + i
        tok, r, _ = decode_step(cfg, W, cache, cos, sin, tok, step, layers, head=True)
        ids.append(tok)
        routes.append(r)
        if on_token is not None:
            on_token(i, tok, r)
    return ids, routes


def rope_tables(s_max, d_r=64, theta=10000.0):
    """cos / sin [s_max, d_r] as bf16 bits: HF layout cat(freqs, freqs), plain RoPE, computed in
    float64 and rounded to float32 then bf16 (fleet/tasks/kernel_tests.py:325-330)."""
    inv_freq = 1.0 / (theta ** (np.arange(0, d_r, 2, dtype=np.float64) / d_r))
    freqs = np.arange(s_max, dtype=np.float64)[:, None] * inv_freq[None, :]
    emb = np.concatenate([freqs, freqs], axis=-1)
    return O.f32_to_bf16(np.cos(emb).astype(np.float32)), O.f32_to_bf16(np.sin(emb).astype(np.float32))
