"""ctypes wrapper of the CPU oracle (oracle/_build/liboracle.so).

TEST INFRASTRUCTURE ONLY: the checker the GPU path is compared against. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module; the product
path (fleet-amd-task_amd/) never does.

Every function takes and returns numpy arrays: bf16 tensors as uint16 bit patterns, FP32 as
float32, ids as int32/int64. Each one cites the numpy_ref.py function whose semantics it
restates; the FP32 summation orders are the spec written in fleet_oracle.c's header.
"""
import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"

_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_vp = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_u32 = ctypes.c_uint32
_f = ctypes.c_float


def build():
    """Compile the oracle library with its Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def _load():
    if not LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    sig = {
        "or_exp": (_f, [_f]), "or_log": (_f, [_f]), "or_silu": (_f, [_f]),
        "or_exp_array": (None, [_f32p, _f32p, _i64]), "or_log_array": (None, [_f32p, _f32p, _i64]),
        "or_silu_array": (None, [_f32p, _f32p, _i64]),
        "or_f32_to_bf16": (ctypes.c_uint16, [_f]),
        "or_round_bf16_array": (None, [_f32p, _u16p, _i64]),
        "or_dot_lanes": (_f, [_u16p, _u16p, _i]),
        "or_mfma_dot32": (_f, [_u16p, _u16p, _i, _f]),
        "or_dot2": (_f, [ctypes.c_uint16, ctypes.c_uint16, ctypes.c_uint16, ctypes.c_uint16, _f]),
        "or_mfma_cases": (None, [_u16p, _u16p, _f32p, _f32p, _i64]),
        "or_rmsnorm": (None, [_u16p, _u16p, _i, _f, _u16p]),
        "or_rope": (None, [_u16p, _u16p, _u16p, _i, _u16p]),
        "or_linear": (None, [_u16p, _u16p, _vp, _f, _vp, _i64, _i, _u16p, _vp]),
        "or_linear_f32": (None, [_u16p, _u16p, _i64, _i, _f32p]),
        "or_mla_prep": (None, [_u16p, _u16p, _u16p, _u16p, _u16p, _i, _i, _i, _i, _f, _u16p, _u16p, _u16p, _u16p]),
        "or_mla_attend": (None, [_u16p, _u16p, _u16p, _u16p, _i, _f, _i, _i, _i, _i, _i, _i, _f32p, _vp, _i]),
        "or_mla_attend_mfma": (None, [_u16p, _u16p, _u16p, _u16p, _i, _f, _i, _i, _i, _i, _i, _i, _f32p]),
        "or_mla_merge_uv": (None, [_f32p, _u16p, _i, _i, _i, _i, _i, _i, _u16p, _vp]),
        "or_moe_router": (None, [_u16p, _vp, _f, _u16p, _i, _i, _i, _i, _f, _vp, _f32p, _f32p, _i32p, _i32p]),
        "or_moe_w13_silu": (None, [_u16p, _u16p, _i32p, _i, _i, _i, _u16p]),
        "or_moe_w2": (None, [_u16p, _u16p, _i32p, _i, _i, _i, _u16p]),
        "or_e4m3_decode": (None, [_f32p]),
        "or_quantize_fp8": (None, [_u16p, ctypes.c_int64, _i, _u8p, _f32p]),
        "or_linear_fp8": (None, [_u8p, _f32p, _u16p, _vp, _f, _i64, _i, _u16p, _vp]),
        "or_moe_w13_silu_fp8": (None, [_u16p, _u8p, _f32p, _i32p, _i, _i, _i, _u16p]),
        "or_moe_w2_fp8": (None, [_u16p, _u8p, _f32p, _i32p, _i, _i, _i, _u16p]),
        "or_moe_combine": (None, [_u16p, _f32p, _u16p, _i, _i, _u16p]),
        "or_dense_mlp": (None, [_u16p, _u16p, _f, _u16p, _u16p, _i, _i, _vp, _vp, _u16p]),
        "or_argmax_bf16": (_i64, [_u16p, _i64]),
        "or_philox4x32_raw": (None, [_u32p, _u32p, _u32p]),
        "or_normal": (_f, [_u64, _u32, _u64]),
        "or_gen_normal_bf16": (None, [_u64, _u32, _u64, _i64, _f, _u16p]),
        "or_gen_tokens": (None, [_u64, _u32, _i64, _i64, _i64p]),
        "or_num_threads": (_i, []), "or_set_num_threads": (None, [_i]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        _LIB = _load()
    return _LIB


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def _ptr(a):
    return None if a is None else a.ctypes.data


# ---- bf16 -------------------------------------------------------------------------------------

def f32_to_bf16(x):
    """numpy_ref.bf16 (numpy_ref.py:36-42) as bits: round to nearest even."""
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().or_round_bf16_array(x.reshape(-1), out.reshape(-1), x.size)
    return out


def bf16_to_f32(u):
    return (np.asarray(u, np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---- spec functions ---------------------------------------------------------------------------

def exp_s(x):
    x = _c(x, np.float32)
    y = np.empty_like(x)
    lib().or_exp_array(x.reshape(-1), y.reshape(-1), x.size)
    return y


def log_s(x):
    x = _c(x, np.float32)
    y = np.empty_like(x)
    lib().or_log_array(x.reshape(-1), y.reshape(-1), x.size)
    return y


def silu_s(x):
    """numpy_ref.silu (numpy_ref.py:248-253) with the spec's exp."""
    x = _c(x, np.float32)
    y = np.empty_like(x)
    lib().or_silu_array(x.reshape(-1), y.reshape(-1), x.size)
    return y


def mfma_cases(A, B, C):
    """gfx950 v_mfma_f32_16x16x32_bf16 per case: D = A B + C with the instruction's own
    accumulation (fleet_oracle.c, or_mfma_dot32). A [n, 16, 32], B [n, 32, 16] bf16 bits, C f32."""
    A, B = _c(A, np.uint16), _c(B, np.uint16)
    C = _c(C, np.float32)
    n = A.shape[0]
    assert A.shape == (n, 16, 32) and B.shape == (n, 32, 16) and C.shape == (n, 16, 16)
    D = np.empty((n, 16, 16), np.float32)
    lib().or_mfma_cases(A.reshape(-1), B.reshape(-1), C.reshape(-1), D.reshape(-1), n)
    return D


def mfma_dot32(a, b, c=0.0):
    """One output of the instruction: c + sum_k a[k] b[k] over 32 bf16 pairs."""
    a, b = _c(a, np.uint16), _c(b, np.uint16)
    assert a.size == 32 and b.size == 32
    return np.float32(lib().or_mfma_dot32(a, b, 1, float(c)))


def dot_lanes(a, b):
    a, b = _c(a, np.uint16), _c(b, np.uint16)
    return np.float32(lib().or_dot_lanes(a, b, a.size))


def dot2(a0, a1, b0, b1, acc=0.0):
    """gfx950 v_dot2c_f32_bf16: acc + a0 b0 + a1 b1 (bf16 bits) with the instruction's own
    accumulation (fleet_oracle.c, dot2_hw)."""
    return np.float32(lib().or_dot2(int(a0), int(a1), int(b0), int(b1), float(acc)))


def rmsnorm(x, w, eps=1e-6):
    """numpy_ref.rmsnorm (numpy_ref.py:54-60)."""
    x, w = _c(x, np.uint16), _c(w, np.uint16)
    y = np.empty(x.size, np.uint16)
    lib().or_rmsnorm(x, w, x.size, eps, y)
    return y


def rope(x, cos_row, sin_row):
    """numpy_ref.rope (numpy_ref.py:63-71) on the last dim; x [..., d]."""
    x = _c(x, np.uint16)
    d = x.shape[-1]
    c, s = _c(cos_row, np.uint16), _c(sin_row, np.uint16)
    flat = x.reshape(-1, d)
    out = np.empty_like(flat)
    for r in range(flat.shape[0]):
        row = np.ascontiguousarray(flat[r])
        o = np.empty(d, np.uint16)
        lib().or_rope(row, c, s, d, o)
        out[r] = o
    return out.reshape(x.shape)


def linear(W, x, norm_w=None, eps=1e-6, res=None):
    """numpy_ref.linear / linear_norm / linear_residual (numpy_ref.py:295-313).
    Returns (out, h): h is the normalised row when norm_w is given, else None."""
    W, x = _c(W, np.uint16), _c(x, np.uint16)
    N, K = W.shape
    out = np.empty(N, np.uint16)
    nw = _c(norm_w, np.uint16) if norm_w is not None else None
    r = _c(res, np.uint16) if res is not None else None
    h = np.empty(K, np.uint16) if norm_w is not None else None
    lib().or_linear(W, x, _ptr(nw), eps, _ptr(r), N, K, out, _ptr(h))
    return out, h


def linear_f32(W, x):
    W, x = _c(W, np.uint16), _c(x, np.uint16)
    out = np.empty(W.shape[0], np.float32)
    lib().or_linear_f32(W, x, W.shape[0], W.shape[1], out)
    return out


def mla_prep(qkva, w_kv_norm, W_uk, cos_row, sin_row, nh=16, d_n=128, d_r=64, d_c=512, eps=1e-6):
    """numpy_ref.mla_prep (numpy_ref.py:85-103): (c_row, k_pe_row, ql_nope, q_pe)."""
    c_row = np.empty(d_c, np.uint16)
    k_pe_row = np.empty(d_r, np.uint16)
    ql = np.empty((nh, d_c), np.uint16)
    qp = np.empty((nh, d_r), np.uint16)
    lib().or_mla_prep(_c(qkva, np.uint16), _c(w_kv_norm, np.uint16), _c(W_uk, np.uint16), _c(cos_row, np.uint16),
                      _c(sin_row, np.uint16), nh, d_n, d_r, d_c, eps, c_row, k_pe_row, ql, qp)
    return c_row, k_pe_row, ql, qp


def partials_row(d_c):
    """Row width of the partials buffer: o then lse, padded to 4 floats (graph_plan.py:214-218)."""
    return ((d_c + 1 + 3) // 4) * 4


def mla_attend(ql_nope, q_pe, c_kv, k_pe, step, softmax_scale, split=32, n_splits=None, with_scores=False):
    """numpy_ref.mla_attend (numpy_ref.py:110-149): partials [n_splits, nh, prow] f32
    (o at [:d_c], lse at d_c). with_scores: also the scaled scores [nh, s_max]."""
    ql, qp = _c(ql_nope, np.uint16), _c(q_pe, np.uint16)
    ck, kp = _c(c_kv, np.uint16), _c(k_pe, np.uint16)
    nh, d_c = ql.shape
    d_r = qp.shape[1]
    s_max = ck.shape[0]
    n_splits = n_splits or -(-s_max // split)
    prow = partials_row(d_c)
    part = np.zeros((n_splits, nh, prow), np.float32)
    scores = np.zeros((nh, s_max), np.float32) if with_scores else None
    lib().or_mla_attend(ql, qp, ck, kp, step, softmax_scale, split, n_splits, nh, d_c, d_r, prow, part,
                        _ptr(scores), s_max)
    return (part, scores) if with_scores else part


def mla_attend_mfma(ql_nope, q_pe, c_kv, k_pe, step, softmax_scale, split=32, n_splits=None):
    """numpy_ref.mla_attend (numpy_ref.py:110-149) in the matrix-core order of the gfx950 kernel
    (fleet_oracle.c, or_mla_attend_mfma): partials [n_splits, nh, prow] f32."""
    ql, qp = _c(ql_nope, np.uint16), _c(q_pe, np.uint16)
    ck, kp = _c(c_kv, np.uint16), _c(k_pe, np.uint16)
    nh, d_c = ql.shape
    d_r = qp.shape[1]
    assert (d_c + d_r) % 32 == 0 and split % 32 == 0
    s_max = ck.shape[0]
    n_splits = n_splits or -(-s_max // split)
    prow = partials_row(d_c)
    part = np.zeros((n_splits, nh, prow), np.float32)
    lib().or_mla_attend_mfma(ql, qp, ck, kp, step, softmax_scale, split, n_splits, nh, d_c, d_r, prow, part)
    return part


def mla_merge_uv(partials, W_uv, step, split=32):
    """numpy_ref.mla_merge_uv (numpy_ref.py:152-174): (attn [nh*d_v], o_bf [nh, d_c])."""
    p = _c(partials, np.float32)
    W = _c(W_uv, np.uint16)
    nh, d_v, d_c = W.shape
    attn = np.empty(nh * d_v, np.uint16)
    obf = np.empty((nh, d_c), np.uint16)
    lib().or_mla_merge_uv(p, W, step, split, nh, d_c, d_v, p.shape[2], attn, obf.ctypes.data)
    return attn, obf


def moe_router(x, W_gate, norm_w=None, eps=1e-6, topk=6, n_forced=2, scaling=1.0):
    """numpy_ref.moe_router_norm / moe_router (numpy_ref.py:205-245):
    (h, logits f32 [E], topk_w f32 [topk+forced], routing i32 [E+forced], mask i32 [E+forced+1])."""
    W = _c(W_gate, np.uint16)
    E, H = W.shape
    x = _c(x, np.uint16)
    nw = _c(norm_w, np.uint16) if norm_w is not None else None
    h = np.empty(H, np.uint16)
    logits = np.empty(E, np.float32)
    topk_w = np.empty(topk + n_forced, np.float32)
    routing = np.empty(E + n_forced, np.int32)
    mask = np.empty(E + n_forced + 1, np.int32)
    lib().or_moe_router(x, _ptr(nw), eps, W, E, H, topk, n_forced, scaling, h.ctypes.data, logits, topk_w,
                        routing, mask)
    return h, logits, topk_w, routing, mask


def moe_w13_silu(h, W13, mask, n_slots=8):
    """numpy_ref.moe_w13 then the silu-mul of moe_w2 (numpy_ref.py:256-292): act [n_slots, I]."""
    W = _c(W13, np.uint16)
    I2, H = W.shape[1], W.shape[2]
    act = np.zeros((n_slots, I2 // 2), np.uint16)
    lib().or_moe_w13_silu(_c(h, np.uint16), W, _c(mask, np.int32), n_slots, I2 // 2, H, act)
    return act


def e4m3_decode():
    """The 256 OCP e4m3fn code values (float32; NaN at 0x7F, 0xFF)."""
    out = np.empty(256, np.float32)
    lib().or_e4m3_decode(out)
    return out


def quantize_fp8(w):
    """Weight-only FP8 of bf16 rows w [rows, K]: (codes uint8 [rows, K], scales float32 [rows]);
    scale = max|w| / 448 (1 for a zero row), code = e4m3(w / scale), nearest even, saturated."""
    w = _c(w, np.uint16)
    rows, K = w.shape
    q = np.empty((rows, K), np.uint8)
    s = np.empty(rows, np.float32)
    lib().or_quantize_fp8(w, rows, K, q, s)
    return q, s


def linear_fp8(Wq, S, x, norm_w=None, eps=1e-6):
    """linear() with FP8 weights (codes Wq [N, K], per-row scales S [N]): out[n] =
    bf16(dot_lanes16(codes, x') * S[n]), x' the normalised row when norm_w is given. Returns (out, h)."""
    Wq, x = _c(Wq, np.uint8), _c(x, np.uint16)
    N, K = Wq.shape
    out = np.empty(N, np.uint16)
    nw = _c(norm_w, np.uint16) if norm_w is not None else None
    h = np.empty(K, np.uint16) if norm_w is not None else None
    lib().or_linear_fp8(Wq, _c(S, np.float32), x, _ptr(nw), eps, N, K, out, _ptr(h))
    return out, h


def moe_w13_silu_fp8(h, W13q, W13s, mask, n_slots=8):
    """moe_w13_silu with FP8 experts: codes [slots, 2I, H], scales [slots, 2I]."""
    Wq = _c(W13q, np.uint8)
    I2, H = Wq.shape[1], Wq.shape[2]
    act = np.zeros((n_slots, I2 // 2), np.uint16)
    lib().or_moe_w13_silu_fp8(_c(h, np.uint16), Wq, _c(W13s, np.float32), _c(mask, np.int32), n_slots, I2 // 2, H, act)
    return act


def moe_w2_fp8(act, W2q, W2s, mask, n_slots=8):
    """moe_w2 with FP8 experts: codes [slots, H, I], scales [slots, H]."""
    Wq = _c(W2q, np.uint8)
    H, I = Wq.shape[1], Wq.shape[2]
    out = np.zeros((n_slots, H), np.uint16)
    lib().or_moe_w2_fp8(_c(act, np.uint16), Wq, _c(W2s, np.float32), _c(mask, np.int32), n_slots, I, H, out)
    return out


def moe_w2(act, W2, mask, n_slots=8):
    """numpy_ref.moe_w2's product (numpy_ref.py:275-292): out8 [n_slots, H]."""
    W = _c(W2, np.uint16)
    H, I = W.shape[1], W.shape[2]
    out = np.zeros((n_slots, H), np.uint16)
    lib().or_moe_w2(_c(act, np.uint16), W, _c(mask, np.int32), n_slots, I, H, out)
    return out


def moe_combine(out8, topk_w, x_res):
    """numpy_ref.moe_combine (numpy_ref.py:316-321)."""
    o = _c(out8, np.uint16)
    out = np.empty(o.shape[1], np.uint16)
    lib().or_moe_combine(o, _c(topk_w, np.float32), _c(x_res, np.uint16), o.shape[0], o.shape[1], out)
    return out


def dense_mlp(x_res, w_norm2, W_gu, W_d, eps=1e-6):
    """Layer-0 MLP (HF DeepseekV2MLP, modeling_deepseek.py:381-398, with numpy_ref's rounding
    points): (h, act, x_res')."""
    W_gu, W_d = _c(W_gu, np.uint16), _c(W_d, np.uint16)
    I, H = W_gu.shape[0] // 2, W_gu.shape[1]
    h = np.empty(H, np.uint16)
    act = np.empty(I, np.uint16)
    out = np.empty(H, np.uint16)
    lib().or_dense_mlp(_c(x_res, np.uint16), _c(w_norm2, np.uint16), eps, W_gu, W_d, I, H, h.ctypes.data,
                       act.ctypes.data, out)
    return h, act, out


def argmax_bf16(logits):
    l = _c(logits, np.uint16)
    return int(lib().or_argmax_bf16(l, l.size))


# ---- generator --------------------------------------------------------------------------------

def philox4x32_raw(ctr, key):
    out = np.empty(4, np.uint32)
    lib().or_philox4x32_raw(_c(ctr, np.uint32), _c(key, np.uint32), out)
    return out


def gen_normal_bf16(seed, stream, n, scale, offset=0):
    out = np.empty(n, np.uint16)
    lib().or_gen_normal_bf16(seed, stream, offset, n, scale, out)
    return out


def normal_f32(seed, stream, idx):
    return np.array([lib().or_normal(seed, stream, int(i)) for i in np.asarray(idx).reshape(-1)], np.float32)


def gen_tokens(seed, stream, n, vocab):
    out = np.empty(n, np.int64)
    lib().or_gen_tokens(seed, stream, n, vocab, out)
    return out


def num_threads():
    return lib().or_num_threads()


def set_num_threads(n):
    lib().or_set_num_threads(int(n))
