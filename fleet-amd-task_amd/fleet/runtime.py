"""ctypes binding of libfleet_mi355x.so (include/fleet_mi355x.h).

The host side of the drop-in boundary: device buffers, the task-table entry (fx_stage) and the
calls that replace the mirage runtime's PersistentKernel / compile / run (fleet/build_graph.py:561-593,
harness/run_fleet.py:551-593 in the reference). No torch: device memory comes from the library's
own hipMalloc wrapper, so the same process can run under rocprofv3.

The library must be built (fleet-amd-task_amd/csrc/Makefile, or __graft_entry__.build()); a missing
library or a non-gfx950 device raises FxError, there is no fallback.
"""
import atexit
import ctypes
import os
import weakref
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent.parent
LIB_PATH = Path(os.environ.get("FX_LIB", PKG / "lib" / "libfleet_mi355x.so"))

FX_OP_GEMV, FX_OP_MLA_PREP, FX_OP_MLA_ATTEND, FX_OP_MLA_MERGE_UV = 1, 2, 3, 4
FX_OP_MOE_ROUTER, FX_OP_MOE_W13, FX_OP_MOE_W2 = 5, 6, 7
FX_OP_DENSE_GU, FX_OP_ARGMAX = 9, 10
FX_IN_VEC, FX_IN_EMBED = 0, 1
FX_F_NORM, FX_F_RESIDUAL, FX_F_ARGMAX, FX_F_HEAD, FX_F_OUT_LL, FX_F_RES_EMBED, FX_F_ROUTER = 1, 2, 8, 16, 32, 64, 128
FX_F_FP8 = 256
FX_F_MFMA = 512
FX_F_XLOCAL = 1024
FX_F_XCD = 2048
FX_F_SKIP_XCD = 4096
FX_F_PAIR = 8192
FX_F_LOW16 = 16384
FX_MAX_ITERS, FX_MAX_MARKS, FX_PROF_SLOTS = 65536, 256, 8
FX_ABI_VERSION = 4
WORKERS = 256          # one worker workgroup per CU
XCDS = 8


class FxError(RuntimeError):
    pass


class FxStage(ctypes.Structure):
    """Mirror of struct fx_stage (include/fleet_mi355x.h)."""
    _fields_ = [(n, ctypes.c_int32) for n in (
        "op", "flags", "in_kind", "layer", "n_rows", "k", "n_slots", "topk", "n_forced", "split", "n_splits",
        "d_c", "d_r", "d_n", "prow", "s_max", "aux_i0", "aux_i1")] + [("src", ctypes.c_int32 * 4)] + \
        [(n, ctypes.c_float) for n in ("eps", "scale", "scaling", "aux_f")] + \
        [(n, ctypes.c_uint64) for n in ("w", "x", "w_norm", "res", "out")] + [("aux", ctypes.c_uint64 * 8)]

    def set(self, **kw):
        for k, v in kw.items():
            if k == "aux":
                for i, p in v.items():
                    self.aux[i] = int(p or 0)
            elif k == "src":
                for i, p in enumerate(v):
                    self.src[i] = int(p)
            else:
                setattr(self, k, v if not isinstance(v, DeviceBuffer) else v.ptr)
        return self

    def to_dict(self):
        d = {n: getattr(self, n) for n, _ in self._fields_ if n not in ("aux", "src")}
        d["aux"] = list(self.aux)
        d["src"] = list(self.src)
        return d


assert ctypes.sizeof(FxStage) == 208, ctypes.sizeof(FxStage)   # static_assert in fx_runtime.hip

_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise FxError(f"{LIB_PATH} is missing: build it with `make -C fleet-amd-task_amd/csrc` "
                      f"or __graft_entry__.build()")
    L = ctypes.CDLL(str(LIB_PATH))
    vp, i32, i64, u64, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64, ctypes.c_size_t
    sig = {
        "fx_abi_version": (ctypes.c_int, []),
        "fx_create": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(vp)]),
        "fx_destroy": (ctypes.c_int, [vp]),
        "fx_last_error": (ctypes.c_char_p, [vp]),
        "fx_device_info": (ctypes.c_int, [vp, ctypes.POINTER(i32), ctypes.POINTER(i32), ctypes.POINTER(i32),
                                          ctypes.POINTER(i32)]),
        "fx_malloc": (ctypes.c_int, [vp, sz, ctypes.POINTER(vp)]),
        "fx_free": (ctypes.c_int, [vp, vp]),
        "fx_memcpy_htod": (ctypes.c_int, [vp, vp, vp, sz]),
        "fx_memcpy_dtoh": (ctypes.c_int, [vp, vp, vp, sz]),
        "fx_memcpy_dtod": (ctypes.c_int, [vp, vp, vp, sz]),
        "fx_memset": (ctypes.c_int, [vp, vp, ctypes.c_int, sz]),
        "fx_synchronize": (ctypes.c_int, [vp]),
        "fx_load_plan": (ctypes.c_int, [vp, ctypes.POINTER(FxStage), i32, ctypes.POINTER(FxStage), i32]),
        "fx_run": (ctypes.c_int, [vp, i32, i32, i32, vp, vp]),
        "fx_launch": (ctypes.c_int, [vp, i32, i32, i32, vp, vp]),
        "fx_finish": (ctypes.c_int, [vp, vp]),
        "fx_mark": (ctypes.c_int, [vp, i32, vp]),
        "fx_marks_ms": (ctypes.c_int, [vp, i32, i32, ctypes.POINTER(ctypes.c_float)]),
        "fx_read_timing": (ctypes.c_int, [vp, ctypes.POINTER(ctypes.c_uint64), i32]),
        "fx_last_run_ms": (ctypes.c_int, [vp, ctypes.POINTER(ctypes.c_float)]),
        "fx_set_profile": (ctypes.c_int, [vp, i32]),
        "fx_read_profile": (ctypes.c_int, [vp, ctypes.POINTER(ctypes.c_uint64), i32]),
        "fx_run_stage": (ctypes.c_int, [vp, ctypes.POINTER(FxStage), i32, ctypes.c_uint32, i32, vp]),
        "fx_mla_attend_merge_noalloc": (ctypes.c_int, [vp, ctypes.POINTER(FxStage), ctypes.POINTER(FxStage), i32,
                                                       ctypes.c_uint32, i32, vp]),
        "fx_time_stages": (ctypes.c_int, [vp, ctypes.POINTER(FxStage), i32, i32, i32, ctypes.c_uint32, i32, vp,
                                          ctypes.POINTER(ctypes.c_float)]),
        "fx_gen_normal_bf16": (ctypes.c_int, [vp, vp, u64, u64, u64, u64, u64, u64, ctypes.c_uint32, ctypes.c_float]),
        "fx_fill_u16": (ctypes.c_int, [vp, vp, u64, ctypes.c_uint16]),
        "fx_quantize_fp8": (ctypes.c_int, [vp, vp, vp, i64, i32, vp]),
        "fx_dequantize_fp8": (ctypes.c_int, [vp, vp, vp, i64, i32, vp]),
        "fx_gemm": (ctypes.c_int, [vp, i32, i32, i32, i32, i32, ctypes.c_float, vp, i64, i64, vp, i64, i64,
                                   ctypes.c_float, vp, i64, i64, vp, i64, i64, i32, i32, vp]),
        "fx_pf_embed": (ctypes.c_int, [vp, vp, vp, vp, i32, i32, vp]),
        "fx_pf_rmsnorm": (ctypes.c_int, [vp, vp, i64, vp, vp, i64, i32, i32, ctypes.c_float, vp]),
        "fx_pf_prep": (ctypes.c_int, [vp, vp, i64, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32,
                                      ctypes.c_float, vp]),
        "fx_pf_softmax": (ctypes.c_int, [vp, vp, i64, i64, vp, i64, i64, vp, i64, i32, i32, i32, i32, ctypes.c_float,
                                         vp]),
        "fx_pf_attn_out": (ctypes.c_int, [vp, vp, vp, vp, i32, i32, i32, vp]),
        "fx_pf_silu": (ctypes.c_int, [vp, vp, vp, i32, i32, vp]),
        "fx_pf_route": (ctypes.c_int, [vp, vp, vp, vp, i32, i32, i32, i32, ctypes.c_float, vp]),
        "fx_pf_gather": (ctypes.c_int, [vp, vp, vp, vp, i32, i32, vp]),
        "fx_pf_combine": (ctypes.c_int, [vp, vp, vp, vp, vp, vp, i32, i32, i32, vp]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


EXPORTS = ("fx_abi_version", "fx_create", "fx_destroy", "fx_last_error", "fx_device_info", "fx_malloc", "fx_free",
           "fx_memcpy_htod", "fx_memcpy_dtoh", "fx_memcpy_dtod", "fx_memset", "fx_synchronize", "fx_load_plan",
           "fx_run", "fx_launch", "fx_finish", "fx_mark", "fx_marks_ms", "fx_last_run_ms", "fx_set_profile",
           "fx_read_profile", "fx_read_timing", "fx_run_stage", "fx_mla_attend_merge_noalloc", "fx_time_stages", "fx_gen_normal_bf16", "fx_fill_u16",
           "fx_quantize_fp8", "fx_dequantize_fp8", "fx_gemm", "fx_pf_embed", "fx_pf_rmsnorm", "fx_pf_prep", "fx_pf_softmax", "fx_pf_attn_out", "fx_pf_silu",
           "fx_pf_route", "fx_pf_gather", "fx_pf_combine")


def _close_at_exit(ref):
    rt = ref()
    if rt is not None:
        rt.close()


class Runtime:
    """One device context (fx_create). Owns nothing of the model; buffers are DeviceBuffer objects."""

    def __init__(self, device=0):
        self.L = lib()
        v = self.L.fx_abi_version()
        if v != FX_ABI_VERSION:
            raise FxError(f"libfleet_mi355x ABI {v}, this module expects {FX_ABI_VERSION}: rebuild the library")
        h = ctypes.c_void_p()
        rc = self.L.fx_create(device, ctypes.byref(h))
        self.h = h
        if rc:
            msg = self.L.fx_last_error(h).decode() if h.value else f"fx_create failed ({rc})"
            raise FxError(msg)
        self._live = weakref.WeakSet()     # every DeviceBuffer of this context not yet freed
        # tear down before the interpreter's own finalisation (and the HIP runtime's exit handlers)
        # starts: buffers freed, then the context destroyed, while every library is still loaded
        atexit.register(_close_at_exit, weakref.ref(self))

    def check(self, rc, what=""):
        if rc:
            raise FxError(f"{what}: {self.L.fx_last_error(self.h).decode()} (code {rc})")

    def info(self):
        v = [ctypes.c_int32() for _ in range(4)]
        self.check(self.L.fx_device_info(self.h, *[ctypes.byref(x) for x in v]), "fx_device_info")
        return dict(zip(("cus", "xcds", "workers", "lds_bytes"), [x.value for x in v]))

    def alloc(self, shape, dtype):
        return DeviceBuffer(self, shape, dtype)

    def synchronize(self):
        self.check(self.L.fx_synchronize(self.h), "fx_synchronize")

    def gen_normal_bf16(self, buf, n, seed, stream, scale, dst_offset=0, src_offset=0, rows=1, row_len=None,
                        dst_stride=None, src_stride=None):
        """buf[dst_offset + r*dst_stride + j] = bf16(scale * N(seed, stream, src_offset + r*src_stride + j))."""
        row_len = n if row_len is None else row_len
        dst_stride = row_len if dst_stride is None else dst_stride
        src_stride = row_len if src_stride is None else src_stride
        ptr = buf.ptr + 2 * dst_offset
        self.check(self.L.fx_gen_normal_bf16(self.h, ptr, rows, row_len, dst_stride, src_offset, src_stride, seed,
                                             stream, scale), "fx_gen_normal_bf16")

    def fill_u16(self, buf, value, n=None, offset=0):
        n = buf.nbytes // 2 - offset if n is None else n
        self.check(self.L.fx_fill_u16(self.h, buf.ptr + 2 * offset, n, value), "fx_fill_u16")

    def load_plan(self, stages, epilogue=()):
        arr = (FxStage * len(stages))(*stages)
        epi = (FxStage * max(1, len(epilogue)))(*epilogue) if epilogue else None
        self.check(self.L.fx_load_plan(self.h, arr, len(stages), epi, len(epilogue)), "fx_load_plan")

    def run(self, iters, step0, n_prompt, tokens):
        self.check(self.L.fx_run(self.h, iters, step0, n_prompt, tokens.ptr, None), "fx_run")

    def launch(self, iters, step0, n_prompt, tokens):
        """Enqueue one persistent launch (no host wait); finish() waits and checks."""
        self.check(self.L.fx_launch(self.h, iters, step0, n_prompt, tokens.ptr, None), "fx_launch")

    def finish(self):
        self.check(self.L.fx_finish(self.h, None), "fx_finish")

    def mark(self, idx):
        self.check(self.L.fx_mark(self.h, idx, None), "fx_mark")

    def marks_ms(self, i, j):
        ms = ctypes.c_float()
        self.check(self.L.fx_marks_ms(self.h, i, j, ctypes.byref(ms)), "fx_marks_ms")
        return ms.value

    def last_run_ms(self):
        """HIP-event milliseconds of the last fx_run launch (events on the launch stream)."""
        ms = ctypes.c_float()
        self.check(self.L.fx_last_run_ms(self.h, ctypes.byref(ms)), "fx_last_run_ms")
        return ms.value

    def set_profile(self, iteration):
        """Record per-stage, per-worker stamps of `iteration` in the next run (-1: off)."""
        self.check(self.L.fx_set_profile(self.h, iteration), "fx_set_profile")

    def read_profile(self, n_stages):
        """[n_stages, 256, FX_PROF_SLOTS] s_memrealtime stamps (100 MHz) of the profiled iteration."""
        n = n_stages * 256 * FX_PROF_SLOTS
        buf = (ctypes.c_uint64 * n)()
        m = self.L.fx_read_profile(self.h, buf, n)
        if m != n:
            raise FxError(f"fx_read_profile returned {m} of {n}")
        return np.array(buf, np.uint64).reshape(n_stages, 256, FX_PROF_SLOTS)

    def timing(self, n):
        buf = (ctypes.c_uint64 * (n + 1))()
        m = self.L.fx_read_timing(self.h, buf, n + 1)
        return np.array(buf[:max(m, 0)], np.uint64)

    def run_stage(self, stage, step=0, tbase=1000, sidx=5):
        """One stage as a standalone launch: packet inputs must carry tbase + src[k] + 1, outputs get
        tbase + sidx + 1."""
        self.check(self.L.fx_run_stage(self.h, ctypes.byref(stage), step, tbase, sidx, None), "fx_run_stage")

    def attend_merge_noalloc(self, attend, merge, step=0, tbase=1000, sidx=5):
        """The attend + merge stage pair with the library's own scratch for the split partials and
        done packets (fx_mla_attend_merge_noalloc): no device allocation."""
        self.check(self.L.fx_mla_attend_merge_noalloc(self.h, ctypes.byref(attend), ctypes.byref(merge), step, tbase,
                                                      sidx, None), "fx_mla_attend_merge_noalloc")

    def time_stages(self, stages, reps=10, step=0, tbase=1000, sidx=5):
        """Mean µs per standalone launch of `stages` launched in turn, `reps` rounds (fx_time_stages)."""
        arr = (FxStage * len(stages))(*stages)
        us = ctypes.c_float()
        self.check(self.L.fx_time_stages(self.h, arr, len(stages), reps, step, tbase, sidx, None, ctypes.byref(us)),
                   "fx_time_stages")
        return us.value

    def close(self):
        """Free every live buffer of this context, then destroy the context (idempotent)."""
        if not self.h:
            return
        for b in list(self._live):
            b.free()
        self.L.fx_destroy(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


_DT = {"bf16": np.uint16, "f32": np.float32, "i32": np.int32, "i64": np.int64, "u16": np.uint16, "u8": np.uint8,
       "u64": np.uint64, "pk16": np.uint64, "pk32": np.uint64}


class DeviceBuffer:
    """A device allocation with a shape and a dtype name (bf16 kept as uint16 bit patterns)."""

    def __init__(self, rt, shape, dtype):
        self.rt = rt
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = dtype
        self.np_dtype = _DT[dtype]
        n = int(np.prod(self.shape, dtype=np.int64))
        if dtype == "pk16":         # bf16 values as packets: 2 values + tag per 8 bytes
            assert n % 4 == 0, (shape, "packet vectors hold a multiple of 4 bf16 values")
            n //= 2
        self.n_words = n
        self.nbytes = n * np.dtype(self.np_dtype).itemsize
        p = ctypes.c_void_p()
        rt.check(rt.L.fx_malloc(rt.h, max(self.nbytes, 16), ctypes.byref(p)), "fx_malloc")
        self.ptr = p.value
        rt._live.add(self)

    def upload(self, arr):
        assert self.dtype not in ("pk16", "pk32"), "packet buffers: upload_packets"
        a = np.ascontiguousarray(arr, dtype=self.np_dtype)
        assert a.nbytes == self.nbytes, (a.shape, self.shape)
        self.rt.check(self.rt.L.fx_memcpy_htod(self.rt.h, self.ptr, a.ctypes.data, a.nbytes), "htod")
        return self

    def upload_at(self, arr, elem_offset):
        a = np.ascontiguousarray(arr, dtype=self.np_dtype)
        it = np.dtype(self.np_dtype).itemsize
        assert elem_offset * it + a.nbytes <= self.nbytes
        self.rt.check(self.rt.L.fx_memcpy_htod(self.rt.h, self.ptr + elem_offset * it, a.ctypes.data, a.nbytes), "htod")

    def download_raw(self):
        out = np.empty(self.n_words, self.np_dtype)
        self.rt.check(self.rt.L.fx_memcpy_dtoh(self.rt.h, out.ctypes.data, self.ptr, self.nbytes), "dtoh")
        return out

    def download(self, tag=None):
        """The values (packets unpacked: bf16 bits as uint16, f32 as float32); with `tag`, every packet
        must carry it."""
        raw = self.download_raw()
        if self.dtype in ("pk16", "pk32"):
            vals, tags = unpack_packets(raw, self.dtype)
            if tag is not None and not (tags == np.uint32(tag)).all():
                bad = np.flatnonzero(tags != np.uint32(tag))
                raise FxError(f"packet tags differ from {tag} at {bad[:8].tolist()} ({len(bad)} packets): {tags[bad[:8]].tolist()}")
            return vals.reshape(self.shape)
        return raw.reshape(self.shape)

    def upload_packets(self, values, tag):
        """Write `values` (bf16 bits for pk16, float32 for pk32) as packets carrying `tag`."""
        self.upload_raw(pack_packets(values, self.dtype, tag))
        return self

    def upload_raw(self, arr):
        a = np.ascontiguousarray(arr, dtype=self.np_dtype).reshape(-1)
        assert a.nbytes == self.nbytes, (a.shape, self.shape)
        self.rt.check(self.rt.L.fx_memcpy_htod(self.rt.h, self.ptr, a.ctypes.data, a.nbytes), "htod")
        return self

    def download_range(self, elem_offset, n):
        it = np.dtype(self.np_dtype).itemsize
        out = np.empty(n, self.np_dtype)
        self.rt.check(self.rt.L.fx_memcpy_dtoh(self.rt.h, out.ctypes.data, self.ptr + elem_offset * it, n * it), "dtoh")
        return out

    def zero(self):
        self.rt.check(self.rt.L.fx_memset(self.rt.h, self.ptr, 0, self.nbytes), "memset")
        return self

    def free(self):
        if self.ptr and self.rt.h:
            self.rt.L.fx_free(self.rt.h, self.ptr)
            self.rt._live.discard(self)
        self.ptr = None

    def __del__(self):
        try:
            if self.ptr and self.rt.h:
                self.free()
        except Exception:
            pass


def pack_packets(values, dtype, tag):
    """Packet words (uint64) of a value vector: pk16 = two bf16 (uint16 bits, element 2i low) per
    packet, pk32 = one float32 per packet; the tag in the high 32 bits."""
    v = np.ascontiguousarray(values).reshape(-1)
    if dtype == "pk16":
        u = v.astype(np.uint16).astype(np.uint64)
        payload = u[0::2] | (u[1::2] << np.uint64(16))
    else:
        payload = np.ascontiguousarray(v, np.float32).view(np.uint32).astype(np.uint64)
    return payload | (np.uint64(tag & 0xFFFFFFFF) << np.uint64(32))


def unpack_packets(words, dtype):
    """(values, tags) of packet words: values as uint16 bf16 bits (pk16) or float32 (pk32)."""
    w = np.ascontiguousarray(words, np.uint64)
    payload = (w & np.uint64(0xFFFFFFFF)).astype(np.uint32)
    tags = (w >> np.uint64(32)).astype(np.uint32)
    if dtype == "pk16":
        vals = np.empty(2 * len(w), np.uint16)
        vals[0::2] = (payload & np.uint32(0xFFFF)).astype(np.uint16)
        vals[1::2] = (payload >> np.uint32(16)).astype(np.uint16)
        return vals, tags
    return payload.view(np.float32), tags
