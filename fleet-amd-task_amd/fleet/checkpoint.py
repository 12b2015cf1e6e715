"""The real checkpoint into the packed keys: the counterpart of the reference's
fleet/pack_weights.py loader (layer_names :258-272, Shards :275-293, pack_layer :304-318,
pack_all :321-345) plus what the model's config adds on top of the seeded model: YaRN RoPE
tables and the YaRN softmax scale (DeepSeek-V2-Lite: rope_scaling {type yarn, factor 40,
original_max_position_embeddings 4096, beta_fast 32, beta_slow 1, mscale 0.707,
mscale_all_dim 0.707}; the reference's harness/common.py:21 SOFTMAX_SCALE = 0.1147213867929261).

    cfg = read_config(model_dir)                      # Dims, eps, scale, tables
    bufs = load_packed(rt, model_dir, cfg.dims, layers, head)

The packed keys and layouts are pack_weights.seeded_layout's: every key is a list of segments of
named HF tensors (q_proj | kv_a_proj_with_mqa -> W_qkva, kv_b_proj's per-head halves -> W_uk /
W_uv, gate | up -> W13 per expert, the shared MLP's halves -> experts E and E + 1, down_proj ->
W2 with the shared down_proj's column halves), and the norm keys name their HF tensor; the
loader copies each segment from the memory-mapped shard into the device buffer, so the model is
never held in host memory. Every tensor must be BF16 (as the reference asserts).
"""
import json
import math
import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from fleet.pack_weights import Dims, REAL_DIMS, check_dims, f32_to_bf16, rope_tables, seeded_layout


# ---- safetensors shards, memory-mapped ------------------------------------------------------------

class Shards:
    """The checkpoint's tensors by HF name: model.safetensors.index.json's weight_map (or a single
    model.safetensors), each shard memory-mapped once; get(name) is a read-only uint16 view of a
    BF16 tensor (no copy)."""

    def __init__(self, model_dir):
        self.dir = Path(model_dir)
        idx = self.dir / "model.safetensors.index.json"
        if idx.exists():
            self.map = json.loads(idx.read_text())["weight_map"]
        else:
            single = self.dir / "model.safetensors"
            if not single.exists():
                raise FileNotFoundError(f"{self.dir}: neither model.safetensors.index.json nor model.safetensors")
            self.map = {n: "model.safetensors" for n in self._header(single)[0] if n != "__metadata__"}
        self.files = {}

    @staticmethod
    def _header(path):
        with open(path, "rb") as f:
            n = struct.unpack("<Q", f.read(8))[0]
            return json.loads(f.read(n)), 8 + n

    def _shard(self, fname):
        if fname not in self.files:
            path = self.dir / fname
            header, base = self._header(path)
            self.files[fname] = (header, base, np.memmap(path, dtype=np.uint8, mode="r"))
        return self.files[fname]

    def __contains__(self, name):
        return name in self.map

    def info(self, name):
        if name not in self.map:
            raise KeyError(f"{name}: not in the checkpoint's weight map")
        header, _, _ = self._shard(self.map[name])
        return header[name]

    def get(self, name):
        header, base, mm = self._shard(self.map[name])
        t = header[name]
        if t["dtype"] != "BF16":
            raise TypeError(f"{name}: {t['dtype']}, the packed model is BF16")
        a, e = t["data_offsets"]
        return mm[base + a:base + e].view("<u2").reshape(t["shape"])


# ---- config: dims, eps, YaRN tables and scale -----------------------------------------------------

def yarn_get_mscale(scale=1.0, mscale=1.0):
    """modeling_deepseek.py:247-250."""
    if scale <= 1:
        return 1.0
    return 0.1 * mscale * math.log(scale) + 1.0


def yarn_correction_range(low_rot, high_rot, dim, base, max_pos):
    """The first and last rotary dims of the YaRN ramp (modeling_deepseek.py:226-244): a dim whose
    wavelength fits num_rotations times into max_pos is the bound, floor / ceil, clamped."""
    def corr(rot):
        return (dim * math.log(max_pos / (rot * 2 * math.pi))) / (2 * math.log(base))
    return max(math.floor(corr(low_rot)), 0), min(math.ceil(corr(high_rot)), dim - 1)


def yarn_inv_freq(d_r, theta, factor, orig_max, beta_fast, beta_slow):
    """float32 inverse frequencies of YaRN RoPE (modeling_deepseek.py:285-306): extrapolated
    (unchanged) below the ramp's low end of the frequency index, interpolated (divided by `factor`)
    above its high end, linear in between. The model computes theta^(i/d) with float32 pow, whose
    last bit differs between implementations; here the two frequency sets are the float64 values
    rounded once to float32, and the blend follows the model's float32 steps."""
    idx = np.arange(0, d_r, 2, dtype=np.float64)
    base_pow = float(theta) ** (idx / d_r)
    extra = (1.0 / base_pow).astype(np.float32)
    inter = (1.0 / (float(factor) * base_pow)).astype(np.float32)
    low, high = yarn_correction_range(beta_fast, beta_slow, d_r, theta, orig_max)
    hi = high + 0.001 if low == high else high
    ramp = np.clip((np.arange(d_r // 2, dtype=np.float32) - np.float32(low)) / np.float32(hi - low), 0, 1)
    mask = (np.float32(1.0) - ramp).astype(np.float32)
    return (inter * (np.float32(1.0) - mask) + extra * mask).astype(np.float32)


def yarn_rope_tables(s_max, d_r, theta, factor, orig_max, beta_fast, beta_slow, mscale, mscale_all_dim):
    """cos / sin [s_max, d_r] as bf16 bits in the HF layout cat(freqs, freqs), computed as the
    model's rotary embedding computes them (float32 throughout, times the amplitude
    mscale(factor, mscale) / mscale(factor, mscale_all_dim), then bf16)."""
    inv = yarn_inv_freq(d_r, theta, factor, orig_max, beta_fast, beta_slow)
    t = np.arange(s_max, dtype=np.float32)
    freqs = np.outer(t, inv).astype(np.float32)
    emb = np.concatenate([freqs, freqs], axis=-1)
    amp = np.float32(yarn_get_mscale(factor, mscale) / yarn_get_mscale(factor, mscale_all_dim))
    return (f32_to_bf16((np.cos(emb) * amp).astype(np.float32)), f32_to_bf16((np.sin(emb) * amp).astype(np.float32)))


@dataclass
class ModelConfig:
    dims: Dims
    eps: float
    scale: float               # attention softmax scale
    theta: float
    rope_scaling: dict         # None: plain RoPE

    def tables(self, s_max):
        """cos / sin [s_max, D_R] (bf16 bits) for this model."""
        d = self.dims
        rs = self.rope_scaling
        if not rs or rs.get("type", rs.get("rope_type")) != "yarn" or float(rs.get("factor", 1.0)) <= 1.0:
            return rope_tables(s_max, d.D_R, self.theta)
        return yarn_rope_tables(s_max, d.D_R, self.theta, float(rs["factor"]),
                                int(rs.get("original_max_position_embeddings", 4096)),
                                float(rs.get("beta_fast", 32)), float(rs.get("beta_slow", 1)),
                                float(rs.get("mscale", 1)), float(rs.get("mscale_all_dim", 0)))


def config_from_dict(cfg):
    """ModelConfig of an HF config.json dict (modeling_deepseek.py:94-108, 568-589: the softmax
    scale is q_head_dim^-0.5, times mscale(factor, mscale_all_dim)^2 under YaRN)."""
    d = Dims.from_config(cfg)
    scale = (d.D_N + d.D_R) ** -0.5
    rs = cfg.get("rope_scaling")
    if rs:
        m_all = rs.get("mscale_all_dim", 0)
        if m_all:
            m = yarn_get_mscale(float(rs["factor"]), float(m_all))
            scale = scale * m * m
    return ModelConfig(d, float(cfg.get("rms_norm_eps", 1e-6)), float(np.float32(scale)),
                       float(cfg.get("rope_theta", 10000.0)), rs)


def read_config(model_dir):
    return config_from_dict(json.loads((Path(model_dir) / "config.json").read_text()))


# ---- the loader --------------------------------------------------------------------------------------

def hf_shapes(d: Dims, layers=None, head=True):
    """name -> shape of every HF tensor the packed model of `layers` layers (and the head) reads
    (nn.Linear weights [out, in]; the reference's layer_names :258-272 plus embed, norm, lm_head)."""
    L = d.L if layers is None else layers
    s = {"model.embed_tokens.weight": (d.V, d.H)}
    if head:
        s.update({"lm_head.weight": (d.V, d.H), "model.norm.weight": (d.H,)})
    for l in range(L):
        p = f"model.layers.{l}."
        s.update({p + "input_layernorm.weight": (d.H,), p + "post_attention_layernorm.weight": (d.H,),
                  p + "self_attn.q_proj.weight": (d.Q_OUT, d.H),
                  p + "self_attn.kv_a_proj_with_mqa.weight": (d.KVA_OUT, d.H),
                  p + "self_attn.kv_a_layernorm.weight": (d.D_C,), p + "self_attn.kv_b_proj.weight": (d.KVB_OUT, d.D_C),
                  p + "self_attn.o_proj.weight": (d.H, d.NH * d.D_V)})
        if l == 0:
            s.update({p + "mlp.gate_proj.weight": (d.I_DENSE, d.H), p + "mlp.up_proj.weight": (d.I_DENSE, d.H),
                      p + "mlp.down_proj.weight": (d.H, d.I_DENSE)})
            continue
        s[p + "mlp.gate.weight"] = (d.E, d.H)
        q = p + "mlp.shared_experts."
        s.update({q + "gate_proj.weight": (d.I_SHARED, d.H), q + "up_proj.weight": (d.I_SHARED, d.H),
                  q + "down_proj.weight": (d.H, d.I_SHARED)})
        for e in range(d.E):
            q = p + f"mlp.experts.{e}."
            s.update({q + "gate_proj.weight": (d.I_MOE, d.H), q + "up_proj.weight": (d.I_MOE, d.H),
                      q + "down_proj.weight": (d.H, d.I_MOE)})
    return s


def _segment_source(src, s):
    """The elements a Segment takes from the flattened HF tensor `src`, rows stacked."""
    flat = src.reshape(-1)
    if s.rows == 1:
        return flat[s.src_offset:s.src_offset + s.row_len]
    end = s.src_offset + (s.rows - 1) * s.src_stride + s.row_len
    if end > flat.size:
        raise ValueError(f"{s.stream_name}: segment reads past the tensor ({end} > {flat.size})")
    return np.lib.stride_tricks.as_strided(flat[s.src_offset:], shape=(s.rows, s.row_len),
                                           strides=(s.src_stride * 2, 2), writeable=False)


def pack_into(sink, shards, d: Dims, layers=None, head=True):
    """Walk the packed layout: sink(key, shape) -> handle, then handle.put(dst_offset, uint16 array)
    for every contiguous run of the key; the norm keys are read from their HF tensors. Every HF
    tensor's dtype and shape are checked before any copy."""
    layout = seeded_layout(d, layers, head)
    need = hf_shapes(d, layers, head)
    missing = [n for n in need if n not in shards]
    if missing:
        raise KeyError(f"the checkpoint lacks {len(missing)} tensors the packed model needs, e.g. {missing[:3]}")
    for n, shape in need.items():
        info = shards.info(n)
        if info["dtype"] != "BF16" or tuple(info["shape"]) != tuple(shape):
            raise ValueError(f"{n}: {info['dtype']} {info['shape']}, the packed model needs BF16 {list(shape)}")
    out = {}
    for key, pt in layout.items():
        h = sink(key, pt.shape)
        if pt.init == "ones":
            src = shards.get(pt.source).reshape(-1)
            if src.size != pt.numel:
                raise ValueError(f"{pt.source}: {src.size} elements, {key} has {pt.numel}")
            h.put(0, src)
        else:
            for s in pt.init:
                vals = _segment_source(shards.get(s.stream_name), s)
                if s.rows == 1 or s.dst_stride == s.row_len:
                    h.put(s.dst_offset, np.ascontiguousarray(vals).reshape(-1))
                else:
                    for r in range(s.rows):
                        h.put(s.dst_offset + r * s.dst_stride, np.ascontiguousarray(vals[r]))
        out[key] = h
    return out


class _HostSink:
    def __init__(self, key, shape):
        self.a = np.zeros(int(np.prod(shape)), np.uint16)
        self.shape = shape

    def put(self, off, vals):
        self.a[off:off + vals.size] = vals


def load_host(model_dir, d: Dims = None, layers=None, head=True):
    """key -> numpy uint16 array (bf16 bits) of the packed model: the loader's layout on the host
    (tests and small models)."""
    d = d or read_config(model_dir).dims
    out = pack_into(lambda k, shape: _HostSink(k, shape), Shards(model_dir), d, layers, head)
    return {k: h.a.reshape(h.shape) for k, h in out.items()}


def load_packed(rt, model_dir, d: Dims = None, layers=None, head=True):
    """Allocate every packed key on the device and fill it from the checkpoint. Returns key ->
    DeviceBuffer (the keys fill_seeded returns)."""
    d = d or read_config(model_dir).dims
    check_dims(d)

    class DevSink:
        def __init__(self, key, shape):
            self.buf = rt.alloc(shape, "bf16")

        def put(self, off, vals):
            self.buf.upload_at(vals, off)

    out = pack_into(lambda k, shape: DevSink(k, shape), Shards(model_dir), d, layers, head)
    rt.synchronize()
    return {k: h.buf for k, h in out.items()}


def real_model(d: Dims):
    """True when the dims are DeepSeek-V2-Lite's (the shapes the kernels are built for)."""
    return d == REAL_DIMS
