"""The decode task graph as data (the reference's fleet/graph_plan.py:54-603, re-derived for gfx950).

A plan is a list of operator calls (method name, tensor names, parameters, label) plus the tensors to
allocate or attach. The method names and labels are the reference's (L{l}.qkva, L{l}.mla_prep,
L{l}.mla_attend, L{l}.mla_merge_uv, L{l}.o_proj, L{l}.router, L{l}.w13, L{l}.w2, L{l}.combine,
head.lm_head, head.argmax_reduce, prologue.embed) so --stop-after, the boundary dump and the compare
keep their keys. What changes is how calls hand data to each other: instead of the mirage event
chain, every activation that crosses workgroups is a packet tensor (dtype pk16: bf16 values, two
per 8-byte packet with the producer's tag; pk32: one f32 per packet), and each consumer waits on
exactly the packets it reads. The attention runs split by positions over all workers, every head
per split (attn="mfma"), or per XCD with heads 2x, 2x+1 on XCD x (attn="valu"); everything else
runs over all 256 workers. The residual stream alternates
between two packet vectors, x_res (layer input) and x_mid (after attention).
"""
import struct
from dataclasses import dataclass, field

from fleet.pack_weights import Dims, REAL_DIMS, XCDS, fp8_nbytes

SPLIT = 32                 # positions per attention split (the reference's D11); tiles of 32
N_FORCED = 2
TOPK_TOTAL_SLOTS = 8
SOFTMAX_SCALE = float(struct.unpack("<f", struct.pack("<f", 1.0 / 192 ** 0.5))[0])   # BASELINE: 1/sqrt(192)
ROUTED_SCALING = 1.0
RMS_EPS = 1e-6
WORKERS = 256
XWORKERS = WORKERS // XCDS


def float_bits(x: float) -> int:
    return struct.unpack("<i", struct.pack("<f", x))[0]


@dataclass
class Tensor:
    name: str
    shape: tuple
    dtype: str = "bf16"           # bf16 | f32 | i32 | i64 | pk16 | pk32 (packets)
    kind: str = "new"             # new | input (weights, captured cache, meta)
    source: str = ""


@dataclass
class Call:
    method: str
    args: dict
    tasks: int
    label: str = ""
    note: str = ""


OUTPUT_ARGS = {
    "embed_layer": ["output"],
    "linear_gemv_layer": ["output", "amax"],
    "mla_prep_layer": ["c_kv", "k_pe", "ql_nope", "q_pe", "crow"],
    "mla_attend_layer": ["partials", "done"],
    "mla_merge_uv_layer": ["output", "o_merged", "slices"],
    "moe_router_layer": ["logits_x"],
    "gang_moe_w13_gemv_layer": ["output", "topk_w", "routing", "mask", "logits", "route_log", "h", "sel"],
    "gang_moe_w2_linear_layer": ["output"],
    "moe_mul_sum_add_layer": ["output"],
    "gang_linear_silu_layer": ["output", "h"],
    "argmax_reduce_layer": ["output"],
}


def _tensor_args(call, names):
    out = set()
    for k in names:
        v = call.args.get(k)
        if v is None or not isinstance(v, str):
            continue
        out.add(v)
    return out


@dataclass
class Plan:
    dims: Dims
    s_max: int
    layers: int
    head: bool
    split: int
    n_splits: int
    tensors: dict = field(default_factory=dict)
    calls: list = field(default_factory=list)
    fp8_experts: bool = False   # W13 / W2 are FP8 (codes + per-row scales, pack_weights.quantize_experts)
    fp8_head: bool = False      # W_lm is FP8 too (pack_weights.quantize_head; needs fp8_experts)
    attn: str = "mfma"          # attention kernel: "mfma" (matrix cores, splits over all workers) or "valu"
    pair: bool = True           # o_proj and the expert gate|up stage after it run as one operator (FX_F_PAIR)

    def t(self, name, shape, dtype="bf16", kind="new", source=""):
        assert name not in self.tensors, name
        self.tensors[name] = Tensor(name, tuple(shape), dtype, kind, source)
        return name

    def op(self, method, tasks, label="", note="", **args):
        self.calls.append(Call(method, args, tasks, label, note))

    def index_of(self, label):
        for i, c in enumerate(self.calls):
            if c.label == label:
                return i
        raise KeyError(label)

    def truncate(self, stop_label):
        """Keep the calls up to and including the labelled one (the reference's --stop-after). A w2
        keeps its combine, which runs inside the same stage."""
        i = self.index_of(stop_label)
        if i + 1 < len(self.calls) and self.calls[i].method == "gang_moe_w2_linear_layer":
            i += 1
        self.calls = self.calls[: i + 1]
        return self

    def chain_violations(self):
        """Consecutive calls that share no tensor from the producer's outputs to the consumer's inputs."""
        bad = []
        for prev, cur in zip(self.calls, self.calls[1:]):
            outs = _tensor_args(prev, OUTPUT_ARGS[prev.method])
            ins = _tensor_args(cur, [k for k in cur.args if k not in OUTPUT_ARGS[cur.method]])
            if not (outs & ins):
                bad.append((prev.label, cur.label))
        return bad

    @property
    def n_ops(self):
        return len(self.calls)

    @property
    def n_tasks(self):
        return sum(c.tasks for c in self.calls)


def partials_row(d_c):
    """o (d_c floats) then lse, padded to a multiple of 4 floats (the reference's graph_plan.py:214-218)."""
    return ((d_c + 1 + 3) // 4) * 4


def splits_for(s_max, split=SPLIT, n_splits=None):
    """(split, n_splits): either a split length (n_splits = ceil(s_max / split)) or a split count
    (split = ceil(s_max / n_splits) rounded up to a multiple of the 32-position tile)."""
    if n_splits:
        split = -(-s_max // n_splits)
        split = -(-split // 32) * 32
        n_splits = -(-s_max // split)
    else:
        n_splits = -(-s_max // split)
    return split, n_splits


def default_attn(s_max):
    """The attention of a plan whose caller names none: the matrix-core attention spread over all
    workers. (The single-XCD form keeps the attention's exchanges in one XCD's L2 but gives each of
    its 32 workers a whole head's merge and 64 W_uv rows; measured at ctx 1024 on MI355X it is
    ~80 us/token slower, so it is not a default.)"""
    return "mfma"


def default_splits(s_max, attn="mfma"):
    """(split, n_splits) of the decode plan.
    valu, xcd: the fewest 32-position tiles per split that keep every split on its own worker of an
    XCD (at most 32 splits), so the attention runs in one round and the merge reads at most 32
    partials per head.
    mfma: one split per worker and every head per split, so the splits are short: 32 positions per
    4,096 of the cache (rounded to the nearest multiple; at least 32), i.e. about 128 splits once the
    cache passes 4,096 positions. Measured at ctx 16,384 on MI355X (us/token): split 64 (257 splits)
    2,704, 96 2,490, 128 2,381, 160 2,396, 192 2,433, 288 (57 splits) 2,611; at ctx 1,024 the 33
    splits of 32."""
    if attn in ("valu", "xcd"):
        return splits_for(s_max, n_splits=XWORKERS)
    return splits_for(s_max, SPLIT * max(1, round(s_max / 4096)))


def build_plan(dims: Dims = REAL_DIMS, s_max: int = 1056, layers: int = 27, head: bool = True, split: int = None,
               n_splits: int = None, iters_cap: int = 32, softmax_scale: float = SOFTMAX_SCALE,
               eps: float = RMS_EPS, fp8_experts: bool = False, fp8_head: bool = False, attn: str = None,
               pair: bool = True) -> Plan:
    """split / n_splits: the attention split (positions) or split count; neither: default_splits.
    attn: "mfma" (the matrix-core attention: splits over all workers, every head per split), "xcd"
    (the same attention and its merge on the 32 workers of one XCD, partials in its L2), "valu"
    (heads over XCDs, score chains on the vector ALUs), or None: default_attn(s_max).
    pair: each MoE layer's o_proj issues the expert gate|up stage's first weight loads while it waits
    for the attention (the two run as one operator of the persistent kernel; same results)."""
    d = dims
    assert 1 <= layers <= d.L
    attn = default_attn(s_max) if attn is None else attn
    assert attn in ("mfma", "valu", "xcd"), attn
    split, n_splits = splits_for(s_max, split, n_splits) if (split or n_splits) else default_splits(s_max, attn)
    p = Plan(d, s_max, layers, head, split, n_splits)
    p.attn = attn
    p.pair = pair
    p.scale = softmax_scale
    p.eps = eps
    p.fp8_experts = fp8_experts
    assert fp8_experts or not fp8_head, "an FP8 LM head runs in the FP8 kernel variant: fp8_experts too"
    p.fp8_head = fp8_head
    p.iters_cap = iters_cap
    # ---- meta and shared tensors
    p.t("tokens", (s_max + 1,), "i64", "input", "meta:tokens")
    p.t("W_embed", (d.V, d.H), kind="input", source="W_embed")
    p.t("x_res", (d.H,), "pk16")
    p.t("x_mid", (d.H,), "pk16")
    p.t("qkva", (d.Q_OUT + d.KVA_OUT,), "pk16")
    p.t("ql_nope", (d.NH, d.D_C), "pk16")
    p.t("q_pe", (d.NH, d.D_R), "pk16")
    p.t("crow", (XCDS, d.D_C + d.D_R), "pk16")
    p.t("partials", (n_splits, d.NH, partials_row(d.D_C)), "f32")
    p.t("att_done", (XCDS, XWORKERS), "pk32")
    p.t("o_merged", (d.NH, d.D_C))
    p.t("o_slices", (d.NH, d.D_C), "pk16")   # merged o of each head, exchanged between its merge workers
    p.t("attn", (d.NH * d.D_V,), "pk16")
    p.t("cos", (s_max, d.D_R), kind="input", source="capture:cos")
    p.t("sin", (s_max, d.D_R), kind="input", source="capture:sin")
    p.t("amax", (2 * WORKERS,), "pk32")
    if layers >= 1:
        p.t("act", (d.I_DENSE,), "pk16")
        p.t("h", (d.H,))
    if layers >= 2:
        p.t("logits_x", (d.E,), "pk32")
        p.t("topk_w", (TOPK_TOTAL_SLOTS,), "f32")
        p.t("routing", (d.E_TOTAL,), "i32")
        p.t("mask", (d.E_TOTAL + 1,), "i32")
        p.t("logits_router", (d.E,), "f32")
        p.t("sel", (XCDS,), "i32")
        p.t("act8", (TOPK_TOTAL_SLOTS, d.I_MOE), "pk16")
        p.t("out8", (TOPK_TOTAL_SLOTS, d.H))
        p.t("route_log", (iters_cap, d.L - 1, TOPK_TOTAL_SLOTS), "i32")

    p.op("embed_layer", 1, "prologue.embed", "folded into L0.qkva's input prologue",
         input="tokens", weight="W_embed", output="x_res", amax="amax" if head else None)
    for l in range(layers):
        p.t(f"w_norm1_{l}", (d.H,), kind="input", source=f"w_norm1_{l}")
        p.t(f"w_norm2_{l}", (d.H,), kind="input", source=f"w_norm2_{l}")
        p.t(f"W_qkva_{l}", (d.Q_OUT + d.KVA_OUT, d.H), kind="input", source=f"W_qkva_{l}")
        p.t(f"w_kv_norm_{l}", (d.D_C,), kind="input", source=f"w_kv_norm_{l}")
        p.t(f"W_uk_{l}", (d.NH, d.D_N, d.D_C), kind="input", source=f"W_uk_{l}")
        p.t(f"W_uv_{l}", (d.NH, d.D_V, d.D_C), kind="input", source=f"W_uv_{l}")
        p.t(f"W_o_{l}", (d.H, d.NH * d.D_V), kind="input", source=f"W_o_{l}")
        p.t(f"c_kv_{l}", (s_max, d.D_C), kind="input", source=f"capture:c_kv_{l}")
        p.t(f"k_pe_{l}", (s_max, d.D_R), kind="input", source=f"capture:k_pe_{l}")
        p.op("linear_gemv_layer", WORKERS, f"L{l}.qkva", input="x_res", w_norm=f"w_norm1_{l}",
             weight=f"W_qkva_{l}", residual=None, output="qkva", norm=True)
        p.op("mla_prep_layer", XCDS * (2 * d.D_C // 32 + 1), f"L{l}.mla_prep", qkva="qkva",
             w_kv_norm=f"w_kv_norm_{l}", w_uk=f"W_uk_{l}", cos="cos", sin="sin", c_kv=f"c_kv_{l}",
             k_pe=f"k_pe_{l}", ql_nope="ql_nope", q_pe="q_pe", crow="crow")
        p.op("mla_attend_layer", XCDS * n_splits, f"L{l}.mla_attend", ql_nope="ql_nope", q_pe="q_pe", crow="crow",
             c_kv=f"c_kv_{l}", k_pe=f"k_pe_{l}", partials="partials", done="att_done",
             softmax_scale=softmax_scale, split=split, n_splits=n_splits)
        p.op("mla_merge_uv_layer", WORKERS, f"L{l}.mla_merge_uv", input="partials", done="att_done",
             w_uv=f"W_uv_{l}", output="attn", o_merged="o_merged", slices="o_slices", split=split,
             n_splits=n_splits)
        p.op("linear_gemv_layer", WORKERS, f"L{l}.o_proj", input="attn", w_norm=None, weight=f"W_o_{l}",
             residual="x_res", output="x_mid", norm=False)
        if l == 0:
            p.t("W_gu_0", (2 * d.I_DENSE, d.H), kind="input", source="W_gu_0")
            p.t("W_down_0", (d.H, d.I_DENSE), kind="input", source="W_down_0")
            p.op("gang_linear_silu_layer", WORKERS, f"L{l}.gate_up", input="x_mid", w_norm=f"w_norm2_{l}",
                 weight="W_gu_0", output="act", h="h")
            p.op("linear_gemv_layer", WORKERS, f"L{l}.down", input="act", w_norm=None, weight="W_down_0",
                 residual="x_mid", output="x_res", norm=False)
        else:
            p.t(f"W_gate_{l}", (d.E, d.H), kind="input", source=f"W_gate_{l}")
            if fp8_experts:
                p.t(f"W13_{l}", (fp8_nbytes(d, "W13"),), "u8", kind="input", source=f"W13q_{l}")
                p.t(f"W2_{l}", (fp8_nbytes(d, "W2"),), "u8", kind="input", source=f"W2q_{l}")
            else:
                p.t(f"W13_{l}", (d.E_TOTAL, 2 * d.I_MOE, d.H), kind="input", source=f"W13_{l}")
                p.t(f"W2_{l}", (d.E_TOTAL, d.H, d.I_MOE), kind="input", source=f"W2_{l}")
            p.op("moe_router_layer", d.E, f"L{l}.router", input="x_mid", w_norm=f"w_norm2_{l}",
                 w_gate=f"W_gate_{l}", logits_x="logits_x")
            p.op("gang_moe_w13_gemv_layer", WORKERS, f"L{l}.w13", input="x_mid", w_norm=f"w_norm2_{l}",
                 logits_x="logits_x", weight=f"W13_{l}", output="act8", topk_w="topk_w", routing="routing",
                 mask="mask", logits="logits_router", route_log="route_log", h="h", sel="sel", layer_index=l - 1)
            p.op("gang_moe_w2_linear_layer", WORKERS, f"L{l}.w2", input="act8", logits_x="logits_x",
                 weight=f"W2_{l}", output="out8")
            p.op("moe_mul_sum_add_layer", WORKERS, f"L{l}.combine", "folded into the w2 stage (8 rows per worker, all slots)",
                 input="out8", weight="topk_w", residual="x_mid", output="x_res")
    if head:
        p.t("w_final_norm", (d.H,), kind="input", source="w_final_norm")
        if fp8_head:
            p.t("W_lm", (fp8_nbytes(d, "W_lm"),), "u8", kind="input", source="W_lmq")
        else:
            p.t("W_lm", (d.V, d.H), kind="input", source="W_lm")
        p.t("logits", (d.V,))
        p.op("linear_gemv_layer", WORKERS, "head.lm_head", input="x_res", w_norm="w_final_norm",
             weight="W_lm", residual=None, output="logits", amax="amax", norm=True)
        p.op("argmax_reduce_layer", 1, "head.argmax_reduce",
             "folded into the next iteration's embed; the last iteration's runs as the epilogue",
             input="amax", output="tokens")
    return p


def summary(p: Plan) -> dict:
    return {"ops": p.n_ops, "tasks": p.n_tasks, "n_splits": p.n_splits, "split": p.split,
            "packet_tensors": sum(t.dtype in ("pk16", "pk32") for t in p.tensors.values())}
