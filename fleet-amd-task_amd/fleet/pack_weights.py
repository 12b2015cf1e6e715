"""Packed weight layout of the decode path, filled from a seed.

Mirrors the reference's fleet/pack_weights.py (Dims :30-87, REAL_DIMS :89-90, pack_qkva :144-147,
split_uk_uv :150-161, pack_moe :187-210, pack_attention :213-233, packed_bytes :240-251): the same
packed keys (suffix _l per layer) and the same layouts --
  W_qkva [Q_OUT + KVA_OUT, H]   q_proj rows (head-major, nope then rope), then kv_a_proj_with_mqa rows
  W_uk / W_uv [NH, D_N|D_V, D_C] the per-head halves of kv_b_proj
  W13 [E + N_SHARED, 2 I_MOE, H] gate rows then up rows; experts E, E+1 are the two halves of the
                                 shared MLP (D6 of the reference's decisions)
  W2 [E + N_SHARED, H, I_MOE]   the matching down projections
-- except layer 0's dense MLP, kept unpadded and unshuffled as W_gu_0 [2 I_DENSE, H] (gate rows,
then up rows) and W_down_0 [H, I_DENSE]. The reference pads to 11,264 and shuffles for its CK
tiles (pack_dense_mlp :164-184); the lane-order GEMV here takes any K that is a multiple of 8.

There is no checkpoint (BASELINE: random-init weights ~N(0, 0.02) from a seed, norm weights 1.0).
Every HF tensor (its name as in the checkpoint, layer_names :258-272) is one stream of a
counter-based generator -- Philox4x32-10 keyed by the seed, counter (element // 4, stream, 0x5EED),
Box-Muller (fleet_mi355x.h, fx_gen_normal_bf16) -- with stream = FNV-1a-32 of the name. A packed key
is a list of segments of those streams, so the GPU fills it in place and the CPU oracle can
regenerate any slice (one expert, one head) bit for bit.
"""
import math
from dataclasses import dataclass, field

import numpy as np

XCDS = 8
WEIGHT_SCALE = 0.02
ONE_BF16 = 0x3F80


@dataclass(frozen=True)
class Dims:
    H: int
    NH: int
    D_N: int
    D_R: int
    D_V: int
    D_C: int
    V: int
    L: int
    I_DENSE: int
    I_MOE: int
    E: int
    TOPK: int
    N_SHARED: int

    @classmethod
    def from_config(cls, cfg):
        get = (lambda k: getattr(cfg, k)) if not isinstance(cfg, dict) else (lambda k: cfg[k])
        return cls(H=get("hidden_size"), NH=get("num_attention_heads"), D_N=get("qk_nope_head_dim"),
                   D_R=get("qk_rope_head_dim"), D_V=get("v_head_dim"), D_C=get("kv_lora_rank"), V=get("vocab_size"),
                   L=get("num_hidden_layers"), I_DENSE=get("intermediate_size"), I_MOE=get("moe_intermediate_size"),
                   E=get("n_routed_experts"), TOPK=get("num_experts_per_tok"), N_SHARED=get("n_shared_experts"))

    @property
    def Q_OUT(self):
        return self.NH * (self.D_N + self.D_R)

    @property
    def KVA_OUT(self):
        return self.D_C + self.D_R

    @property
    def KVB_OUT(self):
        return self.NH * (self.D_N + self.D_V)

    @property
    def E_TOTAL(self):
        return self.E + self.N_SHARED

    @property
    def I_SHARED(self):
        return self.I_MOE * self.N_SHARED

    @property
    def N_SLOTS(self):
        return self.TOPK + self.N_SHARED


REAL_DIMS = Dims(H=2048, NH=16, D_N=128, D_R=64, D_V=128, D_C=512, V=102400, L=27, I_DENSE=10944, I_MOE=1408, E=64,
                 TOPK=6, N_SHARED=2)


def check_dims(d: Dims):
    """What the gfx950 kernels assume (checked again by fx_load_plan before any launch)."""
    assert d.NH == 2 * XCDS and d.D_C == 512 and d.D_R == 64 and d.D_N == 128, "MLA kernels: 16 heads, 512/64/128"
    assert d.H == 2048, "router / expert / prologue kernels: H = 2048"
    assert d.N_SLOTS == XCDS, "one MoE slot per XCD: topk + shared = 8"
    assert d.E <= 64, "router softmax on one wave"
    assert d.I_MOE % 8 == 0 and (d.I_MOE // 8 + 63) // 64 <= 3, "w2 K"
    assert d.I_DENSE % 8 == 0 and d.I_DENSE <= 11264, "dense down K"


# ---- streams --------------------------------------------------------------------------------------

def fnv1a32(name: str) -> int:
    h = 0x811C9DC5
    for b in name.encode():
        h = ((h ^ b) * 0x01000193) & 0xFFFFFFFF
    return h


def layer_names(d: Dims, l):
    """HF tensor names of layer l (the reference's pack_weights.layer_names :258-272)."""
    p = f"model.layers.{l}."
    names = [p + s for s in ("input_layernorm.weight", "post_attention_layernorm.weight", "self_attn.q_proj.weight",
                             "self_attn.kv_a_proj_with_mqa.weight", "self_attn.kv_a_layernorm.weight",
                             "self_attn.kv_b_proj.weight", "self_attn.o_proj.weight")]
    if l == 0:
        names += [p + f"mlp.{s}.weight" for s in ("gate_proj", "up_proj", "down_proj")]
    else:
        names.append(p + "mlp.gate.weight")
        names += [p + f"mlp.shared_experts.{s}.weight" for s in ("gate_proj", "up_proj", "down_proj")]
        for e in range(d.E):
            names += [p + f"mlp.experts.{e}.{s}.weight" for s in ("gate_proj", "up_proj", "down_proj")]
    return names


@dataclass(frozen=True)
class Segment:
    """dst[dst_offset + r * dst_stride + j] = bf16(scale * z_stream(src_offset + r * src_stride + j))."""
    dst_offset: int
    rows: int
    row_len: int
    stream_name: str
    src_offset: int = 0
    dst_stride: int = 0
    src_stride: int = 0
    scale: float = WEIGHT_SCALE

    @property
    def stream(self):
        return fnv1a32(self.stream_name)

    @property
    def n(self):
        return self.rows * self.row_len


def _contig(dst_offset, n, name, src_offset=0):
    return Segment(dst_offset, 1, n, name, src_offset, n, n)


@dataclass
class PackedTensor:
    key: str
    shape: tuple
    init: object            # "ones" (a norm weight: 1.0 in the seeded model) or a list of Segment
    source: str = ""        # the HF tensor a "ones" key is loaded from (checkpoint.py)

    @property
    def numel(self):
        return int(np.prod(self.shape, dtype=np.int64))

    @property
    def nbytes(self):
        return 2 * self.numel


def seeded_layout(d: Dims = REAL_DIMS, layers: int = None, head: bool = True):
    """key -> PackedTensor for the whole model (or its first `layers` layers, with/without head)."""
    L = d.L if layers is None else layers
    H, I, E = d.H, d.I_MOE, d.E
    out = {"W_embed": PackedTensor("W_embed", (d.V, H), [_contig(0, d.V * H, "model.embed_tokens.weight")])}
    if head:
        out["W_lm"] = PackedTensor("W_lm", (d.V, H), [_contig(0, d.V * H, "lm_head.weight")])
        out["w_final_norm"] = PackedTensor("w_final_norm", (H,), "ones", "model.norm.weight")
    for l in range(L):
        p = f"model.layers.{l}."
        out[f"w_norm1_{l}"] = PackedTensor(f"w_norm1_{l}", (H,), "ones", p + "input_layernorm.weight")
        out[f"w_norm2_{l}"] = PackedTensor(f"w_norm2_{l}", (H,), "ones", p + "post_attention_layernorm.weight")
        out[f"w_kv_norm_{l}"] = PackedTensor(f"w_kv_norm_{l}", (d.D_C,), "ones", p + "self_attn.kv_a_layernorm.weight")
        out[f"W_qkva_{l}"] = PackedTensor(f"W_qkva_{l}", (d.Q_OUT + d.KVA_OUT, H), [
            _contig(0, d.Q_OUT * H, p + "self_attn.q_proj.weight"),
            _contig(d.Q_OUT * H, d.KVA_OUT * H, p + "self_attn.kv_a_proj_with_mqa.weight")])
        kvb = p + "self_attn.kv_b_proj.weight"
        blk = (d.D_N + d.D_V) * d.D_C
        out[f"W_uk_{l}"] = PackedTensor(f"W_uk_{l}", (d.NH, d.D_N, d.D_C), [
            _contig(h * d.D_N * d.D_C, d.D_N * d.D_C, kvb, h * blk) for h in range(d.NH)])
        out[f"W_uv_{l}"] = PackedTensor(f"W_uv_{l}", (d.NH, d.D_V, d.D_C), [
            _contig(h * d.D_V * d.D_C, d.D_V * d.D_C, kvb, h * blk + d.D_N * d.D_C) for h in range(d.NH)])
        out[f"W_o_{l}"] = PackedTensor(f"W_o_{l}", (H, d.NH * d.D_V), [_contig(0, H * d.NH * d.D_V, p + "self_attn.o_proj.weight")])
        if l == 0:
            Id = d.I_DENSE
            out["W_gu_0"] = PackedTensor("W_gu_0", (2 * Id, H), [
                _contig(0, Id * H, p + "mlp.gate_proj.weight"), _contig(Id * H, Id * H, p + "mlp.up_proj.weight")])
            out["W_down_0"] = PackedTensor("W_down_0", (H, Id), [_contig(0, H * Id, p + "mlp.down_proj.weight")])
        else:
            out[f"W_gate_{l}"] = PackedTensor(f"W_gate_{l}", (E, H), [_contig(0, E * H, p + "mlp.gate.weight")])
            segs13, segs2 = [], []
            for e in range(E):
                q = p + f"mlp.experts.{e}."
                segs13 += [_contig(e * 2 * I * H, I * H, q + "gate_proj.weight"),
                           _contig(e * 2 * I * H + I * H, I * H, q + "up_proj.weight")]
                segs2.append(_contig(e * H * I, H * I, q + "down_proj.weight"))
            for s in range(d.N_SHARED):
                q = p + "mlp.shared_experts."
                e = E + s
                segs13 += [_contig(e * 2 * I * H, I * H, q + "gate_proj.weight", s * I * H),
                           _contig(e * 2 * I * H + I * H, I * H, q + "up_proj.weight", s * I * H)]
                # columns [s*I, (s+1)*I) of the shared down_proj [H, N_SHARED*I]
                segs2.append(Segment(e * H * I, H, I, q + "down_proj.weight", s * I, I, d.I_SHARED))
            out[f"W13_{l}"] = PackedTensor(f"W13_{l}", (d.E_TOTAL, 2 * I, H), segs13)
            out[f"W2_{l}"] = PackedTensor(f"W2_{l}", (d.E_TOTAL, H, I), segs2)
    return out


def expert_segments(pt: PackedTensor, e: int, per_expert: int):
    """The segments of one expert slab [e] of W13/W2, re-based to the slab."""
    lo, hi = e * per_expert, (e + 1) * per_expert
    return [Segment(s.dst_offset - lo, s.rows, s.row_len, s.stream_name, s.src_offset, s.dst_stride, s.src_stride, s.scale)
            for s in pt.init if lo <= s.dst_offset < hi]


def packed_bytes(d: Dims = REAL_DIMS):
    """Bytes of the whole packed model (the reference's packed_bytes :240-251 without the dense pad)."""
    per_layer = 2 * d.H + (d.Q_OUT + d.KVA_OUT) * d.H + d.D_C + d.KVB_OUT * d.D_C + d.H * d.NH * d.D_V
    dense = 3 * d.I_DENSE * d.H
    moe = d.E * d.H + d.E_TOTAL * 2 * d.I_MOE * d.H + d.E_TOTAL * d.H * d.I_MOE
    return 2 * (2 * d.V * d.H + d.H + d.L * per_layer + dense + (d.L - 1) * moe)


def bytes_per_token(d: Dims = REAL_DIMS, ctx: int = 1024, layers: int = None, head: bool = True,
                    fp8_experts: bool = False, fp8_head: bool = False):
    """Algorithmic HBM bytes of one decode step attending over `ctx` positions (positions 0..ctx-1):
    every weight the step touches once (8 of the 66 experts per MoE layer) plus the latent-cache rows
    read, plus the embedding row. Activations (KBs) are not counted. fp8_experts: the experts' weights
    at one byte each plus one f32 scale per row; fp8_head: the LM head likewise."""
    L = d.L if layers is None else layers
    attn = (d.Q_OUT + d.KVA_OUT) * d.H + d.KVB_OUT * d.D_C + d.H * d.NH * d.D_V + 2 * d.H + d.D_C
    moe = d.E * d.H + d.N_SLOTS * 3 * d.I_MOE * d.H
    if fp8_experts:   # in bf16 units (the sum is doubled below)
        moe = d.E * d.H + (d.N_SLOTS * 3 * d.I_MOE * d.H + 4 * d.N_SLOTS * (2 * d.I_MOE + d.H)) // 2
    dense = 3 * d.I_DENSE * d.H
    w = L * attn + (dense if L >= 1 else 0) + max(0, L - 1) * moe + d.H
    if head:
        w += (d.V * d.H + 4 * d.V) // 2 + d.H if fp8_head else d.V * d.H + d.H
    kv = L * ctx * (d.D_C + d.D_R)
    return 2 * (w + kv)


def fill_seeded(rt, d: Dims = REAL_DIMS, seed: int = 0, layers: int = None, head: bool = True, keys=None):
    """Allocate every packed key on the device and fill it from the seed. Returns key -> DeviceBuffer."""
    check_dims(d)
    bufs = {}
    for key, pt in seeded_layout(d, layers, head).items():
        if keys is not None and key not in keys:
            continue
        buf = rt.alloc(pt.shape, "bf16")
        if pt.init == "ones":
            rt.fill_u16(buf, ONE_BF16)
        else:
            for s in pt.init:
                rt.gen_normal_bf16(buf, s.n, seed, s.stream, s.scale, dst_offset=s.dst_offset, src_offset=s.src_offset,
                                   rows=s.rows, row_len=s.row_len, dst_stride=s.dst_stride, src_stride=s.src_stride)
        bufs[key] = buf
    rt.synchronize()
    return bufs


# ---- FP8 expert weights ---------------------------------------------------------------------------

def fp8_rows(d: Dims, key: str):
    """(rows, K) of the FP8 form of a W13 / W2 packed key (rows over all E + N_SHARED experts) or of
    the LM head W_lm."""
    if key.startswith("W_lm"):
        return d.V, d.H
    if key.startswith("W13"):
        return d.E_TOTAL * 2 * d.I_MOE, d.H
    return d.E_TOTAL * d.H, d.I_MOE


def fp8_nbytes(d: Dims, key: str):
    """Bytes of an FP8 expert key: the codes [rows][K], then one f32 scale per row."""
    rows, K = fp8_rows(d, key)
    return rows * K + 4 * rows


def quantize_experts(rt, bufs, d: Dims, layers: int = None, free_bf16: bool = True):
    """Add W13q_l / W2q_l (FP8 codes + per-row scales, fx_quantize_fp8) for every MoE layer from the
    bf16 W13_l / W2_l in `bufs` (weight-only, per output row: scale = max|w| / 448); the bf16 expert
    keys are freed unless free_bf16 is False. Returns bufs."""
    L = d.L if layers is None else layers
    for l in range(1, L):
        for key in (f"W13_{l}", f"W2_{l}"):
            rows, K = fp8_rows(d, key)
            q = rt.alloc((fp8_nbytes(d, key),), "u8")
            rt.check(rt.L.fx_quantize_fp8(rt.h, bufs[key].ptr, q.ptr, rows, K, None), "fx_quantize_fp8")
            bufs[key.replace("_", "q_", 1)] = q
            if free_bf16:
                rt.synchronize()
                bufs.pop(key).free()
    rt.synchronize()
    return bufs


def quantize_head(rt, bufs, d: Dims, free_bf16: bool = True):
    """Add W_lmq (the LM head as FP8 codes + per-row scales, fx_quantize_fp8, as quantize_experts)
    from the bf16 W_lm in `bufs`; W_lm is freed unless free_bf16 is False. Returns bufs."""
    rows, K = fp8_rows(d, "W_lm")
    q = rt.alloc((fp8_nbytes(d, "W_lm"),), "u8")
    rt.check(rt.L.fx_quantize_fp8(rt.h, bufs["W_lm"].ptr, q.ptr, rows, K, None), "fx_quantize_fp8")
    bufs["W_lmq"] = q
    rt.synchronize()
    if free_bf16:
        bufs.pop("W_lm").free()
    return bufs


def materialize(pt: PackedTensor, seed: int, gen, segments=None, shape=None):
    """Host copy of a packed tensor (or of the given segments into `shape`) with a CPU generator
    gen(seed, stream, n, scale, offset) -> uint16[n] that follows the same stream definition."""
    shape = pt.shape if shape is None else shape
    out = np.empty(int(np.prod(shape)), np.uint16)
    if pt.init == "ones":
        out[:] = ONE_BF16
        return out.reshape(shape)
    for s in (pt.init if segments is None else segments):
        if s.rows == 1:
            out[s.dst_offset:s.dst_offset + s.row_len] = gen(seed, s.stream, s.row_len, s.scale, s.src_offset)
        else:
            for r in range(s.rows):
                o = s.dst_offset + r * s.dst_stride
                out[o:o + s.row_len] = gen(seed, s.stream, s.row_len, s.scale, s.src_offset + r * s.src_stride)
    return out.reshape(shape)


# ---- host-side seeded inputs (Philox4x32-10 in numpy, identical to the device/oracle streams) ------

def philox4x32(seed: int, block, stream: int):
    """Philox4x32-10 of counters (block, stream, 0x5EED) under key `seed`; block is an int array."""
    block = np.asarray(block, np.uint64)
    c0 = (block & np.uint64(0xFFFFFFFF)).astype(np.uint64)
    c1 = (block >> np.uint64(32)).astype(np.uint64)
    c2 = np.full_like(c0, stream & 0xFFFFFFFF)
    c3 = np.full_like(c0, 0x5EED)
    k0, k1 = seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF
    M32 = np.uint64(0xFFFFFFFF)
    for r in range(10):
        p0 = np.uint64(0xD2511F53) * c0
        p1 = np.uint64(0xCD9E8D57) * c2
        n0 = (p1 >> np.uint64(32)) ^ c1 ^ np.uint64(k0)
        n1 = p1 & M32
        n2 = (p0 >> np.uint64(32)) ^ c3 ^ np.uint64(k1)
        n3 = p0 & M32
        c0, c1, c2, c3 = n0, n1, n2, n3
        if r < 9:
            k0 = (k0 + 0x9E3779B9) & 0xFFFFFFFF
            k1 = (k1 + 0xBB67AE85) & 0xFFFFFFFF
    return np.stack([c0, c1, c2, c3], axis=-1).astype(np.uint32)


def prompt_ids(seed: int, n: int, vocab: int, name: str = "prompt"):
    """n token ids uniform in [0, vocab): (u32 * vocab) >> 32 of word i % 4 of Philox block i // 4."""
    i = np.arange(n, dtype=np.uint64)
    words = philox4x32(seed, i >> np.uint64(2), fnv1a32(name))
    w = words[np.arange(n), (i & np.uint64(3)).astype(np.int64)].astype(np.uint64)
    return ((w * np.uint64(vocab)) >> np.uint64(32)).astype(np.int64)


def rope_tables(s_max, d_r=64, theta=10000.0):
    """cos / sin [s_max, d_r] as bf16 bits, HF layout cat(freqs, freqs), plain RoPE (the reference
    kernel suite's tables, fleet/tasks/kernel_tests.py:325-330): float64, then float32, then bf16 RNE."""
    inv_freq = 1.0 / (theta ** (np.arange(0, d_r, 2, dtype=np.float64) / d_r))
    freqs = np.arange(s_max, dtype=np.float64)[:, None] * inv_freq[None, :]
    emb = np.concatenate([freqs, freqs], axis=-1)
    return f32_to_bf16(np.cos(emb).astype(np.float32)), f32_to_bf16(np.sin(emb).astype(np.float32))


def f32_to_bf16(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    return u.astype(np.uint16)


def bf16_to_f32(u):
    return (np.asarray(u, np.uint16).astype(np.uint32) << 16).view(np.float32)
