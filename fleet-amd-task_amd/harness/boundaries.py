"""Boundary tensors of a decode run: the join between a reference run directory and a Fleet run
directory (the reference's harness/common.py:22-110 keys and classes, and its
run_fleet.boundary_dump :69-147 for this build's workspaces).

A boundary key is "L{l}.B{n}.{name}" for a layer, "head.B{n}.{name}" for the head; the class of a
key sets the rel_err threshold compare.py applies to it (THRESHOLD_MULTIPLIER x a calibrated floor
replaces the starting value when the reference directory holds calibration.json). Keys that are
not boundaries ("L1.norm2", "L1.kva", "L1.ql_nope", "L1.o_merged") are written as auxiliary
tensors and never judged.

Workspaces hold the values of the last stage that wrote them in the last iteration: dump() maps
each workspace to the key of its last writer in the plan (a truncated graph, --stop-after, moves
the writers), as the reference does. The cache rows at position n_prompt - 1 and the first token
are written at decode step 0 and never again; every other boundary of a run of `iters` decode
iterations comes from iteration iters - 1 (boundary_iteration).

Files are safetensors (https://github.com/huggingface/safetensors: u64 header length, JSON header,
raw little-endian data). numpy has no bfloat16, so bf16 tensors are handled as their uint16 bit
patterns: write() stores a uint16 array as BF16, read() returns BF16 tensors as float32 (exact).
"""
import json
import re
import struct
import sys
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(PKG))
from fleet import graph_plan as G  # noqa: E402

# rel_err thresholds per class (starting values) and the calibration multiplier
CLASS_THRESHOLD = {"norm": 1e-2, "rope": 1e-2, "gemv": 2e-2, "scores": 3e-2, "attention": 3e-2, "router": 2e-2,
                   "expert": 3e-2, "layer": 5e-2, "logits": 5e-2, "exact": 0.0}
THRESHOLD_MULTIPLIER = 4.0

# (key suffix, boundary id, class); "B11.expert_*" carries the expert id
LAYER_BOUNDARIES = [
    ("B1.norm1", "B1", "norm"), ("B2.q", "B2", "gemv"), ("B3.c_kv", "B3", "norm"), ("B3.k_pe", "B3", "rope"),
    ("B4.q_pe", "B4", "rope"), ("B5.scores", "B5", "scores"), ("B6.attn", "B6", "attention"),
    ("B7.x_res_attn", "B7", "gemv"), ("B8.router_logits", "B8", "router"), ("B9.topk_idx", "B9", "exact"),
    ("B10.topk_w", "B10", "router"), ("B11.expert_*", "B11", "expert"), ("B12.shared", "B12", "expert"),
    ("B13.layer_out", "B13", "layer"),
]
HEAD_BOUNDARIES = [("head.B14.norm", "B14", "norm"), ("head.B15.logits", "B15", "logits"),
                   ("head.B16.token", "B16", "exact")]
STEP_INVARIANT = ("B3.c_kv", "B3.k_pe", "B16.token")


def boundary_class(key):
    """The class of a boundary key, None for an auxiliary tensor."""
    if key.startswith("head."):
        return next((c for k, _, c in HEAD_BOUNDARIES if k == key), None)
    m = re.match(r"^L\d+\.(.+)$", key)
    if not m:
        return None
    suffix = m.group(1)
    for k, _, c in LAYER_BOUNDARIES:
        if (k.endswith("*") and suffix.startswith(k[:-1])) or suffix == k:
            return c
    return None


def boundary_id(key):
    return key.split(".")[1]


def boundary_iteration(key, iters):
    """The decode iteration whose values a dumped key holds in a run of `iters` iterations."""
    if iters <= 1 or any(key.endswith(s) for s in STEP_INVARIANT):
        return 0
    return iters - 1


def layer_of(label):
    m = re.match(r"^L(\d+)\.", label or "")
    return int(m.group(1)) if m else None


def last_writers(calls):
    """workspace name -> label of the last plan call that writes it (plan_json()["calls"] order)."""
    w = {}
    for c in calls:
        for arg in G.OUTPUT_ARGS.get(c["method"], []):
            v = c["args"].get(arg)
            if isinstance(v, str):
                w[v] = c["label"]
    return w


def _f32(bits):
    """float32 values of bf16 bit patterns."""
    return (np.asarray(bits, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def dump(calls, host, n_prompt, topk, q_out, iters=1):
    """The boundary tensors of a finished run. calls: plan_json()["calls"] of the run's (possibly
    truncated) plan; host: workspace name -> object with .download() (bf16 as uint16 bits, packets
    unpacked) and .dtype; n_prompt: prompt length (decode step 0 runs at position n_prompt - 1).
    Returns (dict key -> numpy array, notes)."""
    w = last_writers(calls)
    b, notes = {}, []
    if iters != 1:
        notes.append(f"boundaries other than {', '.join(STEP_INVARIANT)} are from iteration {iters - 1}, "
                     f"not decode step 0")
    get = {}

    def val(name):
        if name not in get:
            get[name] = host[name].download()
        return get[name]

    lab = w.get("h")
    if lab:
        l = layer_of(lab)
        if lab.endswith((".w13", ".gate_up", ".router")):
            b[f"L{l}.norm2"] = val("h")           # the MLP / router input norm, fused into that stage
    lab = w.get("qkva")
    if lab:
        l = layer_of(lab)
        q = val("qkva").reshape(-1)
        b[f"L{l}.B2.q"] = q[:q_out].copy()
        b[f"L{l}.kva"] = q[q_out:].copy()
    lab = w.get("q_pe")
    if lab:
        l = layer_of(lab)
        b[f"L{l}.B4.q_pe"] = val("q_pe")
        b[f"L{l}.ql_nope"] = val("ql_nope")

    def row(name, r):
        buf = host[name]
        width = int(np.prod(buf.shape[1:]))
        if hasattr(buf, "download_range"):
            return buf.download_range(r * width, width).reshape(buf.shape[1:])
        return buf.download()[r].copy()

    for name in w:
        m = re.match(r"^c_kv_(\d+)$", name)
        if m:
            l = int(m.group(1))
            b[f"L{l}.B3.c_kv"] = row(name, n_prompt - 1)
            b[f"L{l}.B3.k_pe"] = row(f"k_pe_{l}", n_prompt - 1)
    lab = w.get("attn")
    if lab:
        b[f"L{layer_of(lab)}.B6.attn"] = val("attn")
    lab = w.get("o_merged")
    if lab:
        b[f"L{layer_of(lab)}.o_merged"] = val("o_merged")
    lab = w.get("x_mid")
    if lab and lab.endswith(".o_proj"):
        b[f"L{layer_of(lab)}.B7.x_res_attn"] = val("x_mid")
    lab = w.get("x_res")
    if lab and lab.endswith((".combine", ".down")):
        b[f"L{layer_of(lab)}.B13.layer_out"] = val("x_res")
    lab = w.get("mask")
    if lab:
        l = layer_of(lab)
        mask = val("mask").astype(np.int32)
        b[f"L{l}.B8.router_logits"] = val("logits_router").astype(np.float32)
        b[f"L{l}.B9.topk_idx"] = mask[:topk].copy()
        b[f"L{l}.B10.topk_w"] = val("topk_w")[:topk].astype(np.float32)
        if layer_of(w.get("out8")) == l:
            out8 = val("out8")
            for s in range(topk):
                b[f"L{l}.B11.expert_{int(mask[s])}"] = out8[s].copy()
            b[f"L{l}.B12.shared"] = _f32(out8[topk]) + _f32(out8[topk + 1])
    if w.get("logits"):
        b["head.B15.logits"] = val("logits")
    if w.get("tokens") and w["tokens"] == "head.argmax_reduce":
        b["head.B16.token"] = val("tokens")[n_prompt:n_prompt + 1].astype(np.int64)
    return b, notes


# ------------------------------------------------------------------------------------------------
# safetensors

_DT_WRITE = {np.dtype(np.uint16): "BF16", np.dtype(np.float32): "F32", np.dtype(np.float64): "F64",
             np.dtype(np.int32): "I32", np.dtype(np.int64): "I64", np.dtype(np.float16): "F16",
             np.dtype(np.uint8): "U8", np.dtype(np.int8): "I8", np.dtype(np.bool_): "BOOL"}
_DT_READ = {"F32": np.float32, "F64": np.float64, "I32": np.int32, "I64": np.int64, "F16": np.float16,
            "U8": np.uint8, "I8": np.int8, "BOOL": np.bool_, "I16": np.int16, "U16": np.uint16,
            "U32": np.uint32, "U64": np.uint64}


def write(path, tensors, metadata=None):
    """Write {name: numpy array} as safetensors; uint16 arrays are bf16 bit patterns (BF16)."""
    header, blobs, off = {}, [], 0
    for name in sorted(tensors):
        a = np.ascontiguousarray(tensors[name])
        if a.dtype not in _DT_WRITE:
            raise TypeError(f"{name}: dtype {a.dtype} has no safetensors type here")
        raw = a.astype(a.dtype.newbyteorder("<"), copy=False).tobytes()
        header[name] = {"dtype": _DT_WRITE[a.dtype], "shape": list(a.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    if metadata:
        header["__metadata__"] = {str(k): str(v) for k, v in metadata.items()}
    h = json.dumps(header, separators=(",", ":")).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for raw in blobs:
            f.write(raw)


def read_raw(path):
    """{name: (safetensors dtype, numpy array)} of a safetensors file with the stored bits kept:
    BF16 tensors come back as their uint16 bit patterns (the bit-diff report reads these)."""
    data = Path(path).read_bytes()
    n = struct.unpack("<Q", data[:8])[0]
    header = json.loads(data[8:8 + n])
    base = 8 + n
    out = {}
    for name, t in header.items():
        if name == "__metadata__":
            continue
        a, e = t["data_offsets"]
        dt = np.uint16 if t["dtype"] == "BF16" else _DT_READ.get(t["dtype"])
        if dt is None:
            raise TypeError(f"{name}: safetensors dtype {t['dtype']} not supported")
        arr = np.frombuffer(data[base + a:base + e], np.dtype(dt).newbyteorder("<")).astype(dt)
        out[name] = (t["dtype"], arr.reshape(t["shape"]))
    return out


def read(path):
    """{name: numpy array} of a safetensors file; BF16 tensors come back as float32 (exact)."""
    data = Path(path).read_bytes()
    n = struct.unpack("<Q", data[:8])[0]
    header = json.loads(data[8:8 + n])
    base = 8 + n
    out = {}
    for name, t in header.items():
        if name == "__metadata__":
            continue
        a, e = t["data_offsets"]
        raw = data[base + a:base + e]
        if t["dtype"] == "BF16":
            arr = _f32(np.frombuffer(raw, "<u2"))
        elif t["dtype"] in _DT_READ:
            arr = np.frombuffer(raw, np.dtype(_DT_READ[t["dtype"]]).newbyteorder("<")).astype(_DT_READ[t["dtype"]])
        else:
            raise TypeError(f"{name}: safetensors dtype {t['dtype']} not supported")
        out[name] = arr.reshape(t["shape"])
    return out
