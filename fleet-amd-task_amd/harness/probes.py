#!/usr/bin/env python3
"""gfx950 memory-system probes (csrc/fx_probe.hip, lib/libfleet_probe.so): the stream rate of the
GEMV load pattern against bytes per workgroup and loads in flight, dependent-load latency per cache
policy (idle and under a full-chip stream), and the flag round trip between two workgroups.
The reference's env/hw/probes (stream_read.cu, chase.cu, fence_probe.cu) measured the same on
MI300X; the decode kernel's prefetch depth and synchronisation design follow these numbers.

    python fleet-amd-task_amd/harness/probes.py [--out probes.md]
"""
import argparse
import ctypes
import sys
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(PKG))
from fleet import runtime as R  # noqa: E402

TICK_NS = 10.0   # s_memrealtime: 100 MHz


def probe_lib():
    p = PKG / "lib" / "libfleet_probe.so"
    if not p.exists():
        raise R.FxError(f"{p} is missing: make -C fleet-amd-task_amd/csrc probe")
    L = ctypes.CDLL(str(p))
    vp, u64, u32 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32
    L.fxp_stream.argtypes = [vp, u64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(u64),
                             ctypes.POINTER(ctypes.c_float)]
    L.fxp_chase.argtypes = [vp, u32, ctypes.c_int, vp, u64, ctypes.c_int, ctypes.POINTER(u64)]
    L.fxp_pingpong.argtypes = [ctypes.c_int, ctypes.c_int, u32, ctypes.c_int, vp, u64, ctypes.c_int,
                               ctypes.POINTER(u64)]
    L.fxp_loaded.argtypes = [ctypes.c_int, ctypes.c_int, u32, ctypes.c_int, ctypes.c_int, vp, u64, ctypes.c_int,
                             ctypes.c_int, ctypes.POINTER(u64)]
    L.fxp_gemv.argtypes = [vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(u64),
                           ctypes.POINTER(ctypes.c_float)]
    L.fxp_lanes.argtypes = [ctypes.POINTER(ctypes.c_float)]
    L.fxp_valu.argtypes = [ctypes.POINTER(u64)]
    L.fxp_icache.argtypes = [vp, u64, ctypes.POINTER(u64)]
    L.fxp_clock.argtypes = [ctypes.c_int, vp, u64, ctypes.POINTER(u64)]
    L.fxp_lds_dma.argtypes = [ctypes.POINTER(u32)]
    L.fxp_fp8.argtypes = [ctypes.POINTER(ctypes.c_float)]
    return L


def check_lanes(L):
    """The DPP / row-swap lane exchange of the butterflies returns lane ^ 2^k for k < 6."""
    buf = (ctypes.c_float * (64 * 6))()
    assert L.fxp_lanes(buf) == 0
    got = np.array(buf, np.float32).reshape(64, 6).astype(np.int64)
    exp = np.array([[l ^ (1 << k) for k in range(6)] for l in range(64)])
    bad = np.argwhere(got != exp)
    return bad, got


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", default=None)
    ap.add_argument("--lanes-only", action="store_true")
    ap.add_argument("--stream-only", action="store_true")
    ap.add_argument("--clock", action="store_true")
    ap.add_argument("--pingpong-only", action="store_true", help="only the flag round trips")
    ap.add_argument("--valu", action="store_true", help="only the VALU issue rate of FMA chains")
    ap.add_argument("--gemv", action="store_true",
                    help="only the decode GEMV walk (Tile<4, 4>, K = 2048) against the same loads without the dot")
    ap.add_argument("--gemv-rows", default="400,100,36", help="rows per block of the --gemv walks (multiples of 4)")
    ap.add_argument("--gemv-modes", default="0,3,4,1",
                    help="the walks --gemv times: 0 tile_dot, 1 xor only, 2 contiguous xor, 3/4 sliced, 5 rolling, "
                         "6 FP8 tile_dot, 7 FP8 rolling, 8/9 tile_dot with per-row / per-tile stores of the results, "
                         "10 with the results stored after the walk, 11/12 tiles of 2 rows (two-tile / rolling), 13/14 tiles of 1 row (rolling / two-tile)")
    ap.add_argument("--loaded", action="store_true",
                    help="only the sc1 flag round trip against the depth of a concurrent full-chip stream")
    ap.add_argument("--reuse", action="store_true",
                    help="cold (first touch) against warm (re-read) streams, register and direct-to-LDS loads")
    args = ap.parse_args()
    rt = R.Runtime(0)
    L = probe_lib()
    bad, got = check_lanes(L)
    print(f"lane exchange: {'ok' if len(bad) == 0 else f'{len(bad)} wrong, first (lane, k) {bad[:4].tolist()}'}",
          flush=True)
    if len(bad):
        print(got[:20], flush=True)
        sys.exit(1)
    # the packed FP8 -> f32 conversion of the FP8 expert tiles: OCP e4m3fn (bias 7, 448 max, NaN at
    # 0x7F / 0xFF) or the FNUZ variant (bias 8, NaN at 0x80)?
    f8 = (ctypes.c_float * 256)()
    assert L.fxp_fp8(f8) == 0
    g8 = np.array(f8, np.float32)
    c = np.arange(256)
    e, m, neg = (c >> 3) & 15, c & 7, (c & 0x80) != 0
    ocp = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1 + m / 8.0) * 2.0 ** (e - 7.0)) * np.where(neg, -1, 1)
    ocp[(e == 15) & (m == 7)] = np.nan
    same = (g8 == ocp.astype(np.float32)) | (np.isnan(g8) & np.isnan(ocp))
    print(f"FP8 conversion: {'OCP e4m3fn on all 256 codes' if same.all() else f'{(~same).sum()} codes differ from OCP e4m3fn'}"
          f" (0x38 -> {g8[0x38]}, 0x7E -> {g8[0x7E]}, 0x01 -> {g8[0x01]})", flush=True)
    if args.lanes_only:
        return
    lines = []
    if args.valu:
        out = (ctypes.c_uint64 * 4)()
        for rep in range(2):
            assert L.fxp_valu(out) == 0
        for v, chains in enumerate((1, 2, 4, 8)):
            print(f"VALU: 1024 v_fmac_f32 per lane as {chains} interleaved dependent chain(s), one wave per SIMD: "
                  f"{out[v]} core cycles, {out[v] / 1024:.2f} cycles per instruction", flush=True)
        big = rt.alloc((2 << 30,), "u8")
        oc = (ctypes.c_uint64 * 2)()
        for rep, load in enumerate((False, False, True, True)):
            assert L.fxp_icache(ctypes.c_void_p(big.ptr) if load else None, big.nbytes, oc) == 0
            print(f"instruction fetch ({'under stream' if load else 'idle'}, launch {rep}): 4096 x 8-byte v_fmac_f32 "
                  f"straight-line, cold pass {oc[0]} cycles ({oc[0] / 4096:.2f}/instr), warm pass {oc[1]} cycles "
                  f"({oc[1] / 4096:.2f}/instr)", flush=True)
        rt.close()
        return
    if args.gemv:
        rows = 102400
        W = rt.alloc((rows * 2048 * 2,), "u8")
        # contents do not matter for the timing (uninitialised bf16 words)
        cold = rt.alloc((1 << 30,), "u8")
        ticks = (ctypes.c_uint64 * 256)()
        ms = ctypes.c_float()
        print("| walk | rows per block | MiB per block | GB/s (events) | median us/block | max us/block |", flush=True)
        print("|---|---|---|---|---|---|", flush=True)
        names = {0: "tile_dot (decode GEMV)", 1: "same loads, xor only", 2: "contiguous KiB order, xor only",
                 3: "sliced, 2 slices in flight", 4: "sliced, 4 slices in flight",
                 5: "rolling tile_dot", 6: "FP8 tile_dot (TileQ<4, 2>)", 7: "FP8 rolling tile_dot",
                 8: "tile_dot + a 2-byte store per row (the LM head's logits)",
                 9: "tile_dot + one 8-byte store per tile",
                 10: "tile_dot, results into LDS, 8-byte stores after the walk",
                 11: "tile_dot, tiles of 2 rows", 12: "rolling tile_dot, tiles of 2 rows",
                 13: "rolling tile_dot, tiles of 1 row", 14: "tile_dot, tiles of 1 row"}
        modes = [int(m) for m in args.gemv_modes.split(",")]
        for rpb in [int(r) for r in args.gemv_rows.split(",")]:
            for mode in modes:
                for rep in range(2):
                    # evict W from the last-level cache between timed walks
                    assert L.fxp_stream(ctypes.c_void_p(cold.ptr), cold.nbytes // 256, 256, 256, 8, 0, ticks, ctypes.byref(ms)) == 0
                    assert L.fxp_gemv(ctypes.c_void_p(W.ptr), 2048, rpb, 256, mode, ticks, ctypes.byref(ms)) == 0
                t = np.array(ticks[:256], np.float64) * TICK_NS / 1e3
                nb = rpb * 2048 * (1 if mode in (6, 7) else 2)
                print(f"| {names[mode]} | {rpb} | {nb / 2**20:.2f} | {256 * nb / (ms.value * 1e6):.0f} | "
                      f"{np.median(t):.2f} | {t.max():.2f} |", flush=True)
        rt.close()
        return
    if args.loaded:
        big = rt.alloc((2 << 30,), "u8")
        out = (ctypes.c_uint64 * 4)()
        print("| a (XCD) | b (XCD) | stream KiB in flight per wave | fma per KiB (< 0: the flag blocks' own waves "
              "stream too, -x KiB tiles) | ns/round trip | stream GB/s |", flush=True)
        print("|---|---|---|---|---|---|", flush=True)
        # fma per KiB < 0: the ping-pong blocks' other waves stream too, -fma KiB per tile
        for a, b in ((8, 9), (8, 16)):
            for work in (0, -4, -16, 16):
                for depth in (0, 2, 4, 8, 16, 24):
                    if depth == 0 and work > 0:
                        continue
                    rc = L.fxp_loaded(a, b, 2000, depth, work, ctypes.c_void_p(big.ptr), big.nbytes, 256, 256, out)
                    assert rc == 0, rc
                    rt_ns = f"{out[0] * TICK_NS / 2000:.0f}" if out[1] == 1 else "no round trip within 1 s"
                    gbs = out[2] / (out[3] * TICK_NS) if out[3] else 0.0
                    fl = "idle" if depth == 0 else f"{depth}..{2 * depth}"
                    print(f"| {a} ({a % 8}) | {b} ({b % 8}) | {fl} | {work} | {rt_ns} | {gbs:.0f} |", flush=True)
        rt.close()
        return
    if args.clock:
        big = rt.alloc((2 << 30,), "u8")
        out = (ctypes.c_uint64 * 3)()
        for load in (False, True, False):
            assert L.fxp_clock(2_000_000, ctypes.c_void_p(big.ptr) if load else None, big.nbytes, out) == 0
            # s_memtime counts the shader clock (core ticks); s_memrealtime 100 MHz
            mhz = out[0] / (out[1] * 1e-8) / 1e6
            ns = out[1] * 10.0 / 2_000_000
            print(f"shader clock {'under stream' if load else 'idle'}: {mhz:.0f} MHz, loop of one dependent fma "
                  f"+ scalar counter + taken branch: {ns:.2f} ns/iteration ({ns * mhz / 1e3:.1f} core cycles)", flush=True)
        return

    def say(s):
        print(s, flush=True)
        lines.append(s)

    big = rt.alloc((2 << 30,), "u8")
    rt.fill_u16(big, 0x3F80, n=big.nbytes // 2)
    rt.synchronize()
    if args.pingpong_only:
        pingpong(L, big, say)
        if args.out:
            Path(args.out).write_text("\n".join(lines) + "\n")
        rt.close()
        return
    if args.reuse:
        # global_load_lds with 16 bytes per lane: lane l's bytes land at the LDS base + 16 l
        got = (ctypes.c_uint32 * 512)()
        assert L.fxp_lds_dma(got) == 0
        g = np.array(got, np.uint32)
        exp = np.concatenate([np.arange(256), (256 + np.arange(256).reshape(64, 4)[::-1]).reshape(-1)])
        say(f"direct-to-LDS layout (16 B per lane at base + 16 * lane): {'ok' if (g == exp).all() else 'DIFFERENT'}; "
            f"first words {g[:8].tolist()}, words 256.. {g[256:264].tolist()}\n")
        say("## cold and warm streams: 256 workgroups x 256 threads; cold = a region no launch has read since "
            "1 GiB of other reads, warm = the same region again right after\n")
        say("| loads | depth | KiB/workgroup | cold median µs/wg | cold max | warm median µs/wg | warm max | "
            "cold GB/s (max) |")
        say("|---|---|---|---|---|---|---|---|")
        ticks = (ctypes.c_uint64 * 256)()
        ms = ctypes.c_float()
        half = big.nbytes // 2
        off = 0
        for pat, depth in ((0, 8), (3, 8), (4, 16), (4, 32)):
            for kib in (64, 96, 288, 1024):
                by = kib * 1024
                if off + 256 * by > half:
                    off = 0
                # flush: stream the second half of the buffer (1 GiB, beyond the last-level cache)
                assert L.fxp_stream(ctypes.c_void_p(big.ptr + half), half // 256, 256, 256, 8, 0, ticks,
                                    ctypes.byref(ms)) == 0
                res = []
                for rep in range(2):
                    assert L.fxp_stream(ctypes.c_void_p(big.ptr + off), by, 256, 256, depth, pat, ticks,
                                        ctypes.byref(ms)) == 0
                    res.append(np.array(ticks, np.float64) * TICK_NS / 1e3)
                off += 256 * by
                c, w = res
                name = {0: "registers", 3: "registers, double-buffered", 4: "direct to LDS"}[pat]
                say(f"| {name} | {depth} | {kib} | {np.median(c):.2f} | {c.max():.2f} | {np.median(w):.2f} | "
                    f"{w.max():.2f} | {256 * by / (c.max() * 1e-6) / 1e9:.0f} |")
        if args.out:
            Path(args.out).write_text("\n".join(lines) + "\n")
        return
    # ---- stream
    say("## stream: 256 workgroups, 1 KiB wave loads (each wave: `depth` loads in flight)\n")
    say("pattern: contiguous = the wave's loads walk one block in order; gemv = the GEMV tile order (4 rows of "
        "4 KiB, chunk-major); pairs = the same with two of the rows in the block's second half (gate | up); double-buffered = "
        "the GEMV pipeline, the next `depth` loads issued before the current ones are consumed\n")
    say("| threads | depth | pattern | KiB/workgroup | GB/s (events) | median µs/wg | max µs/wg |")
    say("|---|---|---|---|---|---|---|")
    ticks = (ctypes.c_uint64 * 256)()
    ms = ctypes.c_float()
    cases = [(256, d, 0, k) for d in (4, 8, 16, 32) for k in (16, 64, 256, 1024, 4096)]
    cases += [(512, d, 0, k) for d in (4, 8, 16) for k in (64, 256, 1024, 4096)]
    cases += [(256, d, pat, k) for pat in (1, 2) for d in (16, 32) for k in (64, 256, 1024, 4096)]
    cases += [(256, d, 3, k) for d in (4, 8, 16) for k in (64, 256, 1024, 4096)]
    for threads, depth, pat, kib in cases:
        by = kib * 1024
        for rep in range(2):
            rc = L.fxp_stream(ctypes.c_void_p(big.ptr), by, 256, threads, depth, pat, ticks, ctypes.byref(ms))
            assert rc == 0, rc
        t = np.array(ticks, np.float64) * TICK_NS / 1e3
        name = ("contiguous", "gemv", "pairs", "double-buffered")[pat]
        say(f"| {threads} | {depth} | {name} | {kib} | {256 * by / (ms.value * 1e-3) / 1e9:.0f} | {np.median(t):.2f} | "
            f"{t.max():.2f} |")
    if args.stream_only:
        if args.out:
            Path(args.out).write_text("\n".join(lines) + "\n")
        return
    chase(rt, L, big, say)
    pingpong(L, big, say)
    if args.out:
        Path(args.out).write_text("\n".join(lines) + "\n")
    rt.close()


def chase(rt, L, big, say):
    say("\n## dependent-load latency (one lane, pointer chase, stride 256 B)\n")
    say("| footprint | policy | load | ns/load |")
    say("|---|---|---|---|")
    rng = np.random.default_rng(1)
    for slots, name in ((4096, "1 MiB"), (2 << 20, "512 MiB")):
        stride = 64
        perm = rng.permutation(slots).astype(np.uint32)
        nxt = np.zeros(slots * stride, np.uint32)
        # a single cycle through the permutation
        order = perm
        nxt[order[:-1] * stride] = order[1:] * stride
        nxt[order[-1] * stride] = order[0] * stride
        buf = rt.alloc((slots * stride,), "i32")
        buf.upload(nxt.view(np.int32))
        out = (ctypes.c_uint64 * 3)()
        hops = 2000
        for mode, pol in ((0, "plain"), (1, "sc1"), (2, "nt")):
            for load in (False, True):
                lp = ctypes.c_void_p(big.ptr) if load else None
                rc = L.fxp_chase(ctypes.c_void_p(buf.ptr), hops, mode, lp, big.nbytes, 256, out)
                assert rc == 0, rc
                say(f"| {name} | {pol} | {'stream' if load else 'idle'} | {out[0] * TICK_NS / hops:.0f} |")
        buf.free()


def pingpong(L, big, say):
    say("\n## flag round trip between two workgroups\n")
    say("policy: agent = agent-scope relaxed atomic store / load; sc1 = buffer store / load with sc1 (the decode "
        "kernel's packets); sc0 = buffer store / load with sc0 (same XCD only; the rest likewise)\n")
    say("| a (XCD) | b (XCD) | policy | load | ns/round trip |")
    say("|---|---|---|---|---|")
    out = (ctypes.c_uint64 * 5)()
    for a, b in ((8, 16), (8, 9), (8, 13)):
        for mode, pol in ((0, "agent"), (2, "sc1"), (4, "sc0"), (1, "sc0 load, plain store"),
                          (3, "plain store, L1 invalidate + plain load"), (5, "sc1 store, sc0 load"),
                          (6, "sc0 store, sc1 load")):
            if mode in (1, 3, 4, 5) and a % 8 != b % 8:
                continue
            for load in (False, True):
                lp = ctypes.c_void_p(big.ptr) if load else None
                rc = L.fxp_pingpong(a, b, 2000, mode, lp, big.nbytes, 256, out)
                assert rc == 0, rc
                rt_ns = f"{out[0] * TICK_NS / 2000:.0f}" if out[1] == 1 else "no round trip within 1 s"
                say(f"| {a} ({out[3]}) | {b} ({out[4]}) | {pol} | {'stream' if load else 'idle'} | {rt_ns} |")


if __name__ == "__main__":
    main()
