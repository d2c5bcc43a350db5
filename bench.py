#!/usr/bin/env python3
"""Benchmark of the fused 4-bit dequant-GEMV on one MI355X.

A "step" is one fused dequant-GEMV call over one layer for one batch of activations,
with the packed weight and x already resident in HBM.  The default workload is the
north-star layer: GF4 (Jenks-16 codebooks, group 128), K=8192 -> N=28672, batch 1
Prints ONE JSON line (metric, value, unit, roofline, cpu_baseline, ...);
``--sweep`` additionally writes one line per config shape to ``--sweep-out``.

Throughput = algorithmic bytes per call / time per call, with
GF4 bytes = N*K/2 + N*(K/128)*32 + B*K*2 + B*N*2 and
E2M1 bytes = N*K/2 + N*(K/32) + B*K*2 + B*N*2 (each byte counted once).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from if_i_could_turn_back_time_amd import PackedWeight, fwht_block_for  # noqa: E402
from if_i_could_turn_back_time_amd import _capi as C  # noqa: E402
from if_i_could_turn_back_time_amd import workloads  # noqa: E402

PEAK_GBS = 8000.0
METRIC = "achieved HBM GB/s (% of roofline) & µs/call, 4-bit dequant-GEMV at batch 1"

# name -> (fmt, K, N, B, generator, rotated); generators per the benchmark configs
WORKLOADS = workloads.WORKLOADS
DEFAULT = workloads.DEFAULT


MALL_BYTES = 256 * 2**20  # MI355X Infinity Cache (memory-side, in front of HBM)
MIN_WARM_S = 0.25  # least wall time of back-to-back warm-up calls before a timed region
LAST_WARMUP_CALLS = 0  # warm-up calls the last time_gpu ran (>= the requested warm-up)
PRE_CALLS = 3  # untimed calls enqueued before each start event (busy GPU at the stamp)
MEDIAN_WINDOWS = 9  # further timed regions of --steps calls; value is the median of all 10
SWEEP_WINDOWS = 6  # further regions per --sweep line (its median over 7 regions is reported)


def n_copies(nbytes: int, cold: bool) -> int:
    """Weight copies cycled through so that every call streams from HBM: their total
    is >= 3x the Infinity Cache, so a copy is evicted before it is read again."""
    if not cold:
        return 1
    return int(min(256, max(2, -(-3 * MALL_BYTES // nbytes))))


def time_gpu(pw: PackedWeight, x: torch.Tensor, y: torch.Tensor, steps: int, warmup: int,
             cold: bool = True, windows: int = 0, mx: str = ""):
    """Back-to-back launches on the current stream, timed with HIP events on that stream
    (the stream fb_gemv launches on).  cold: cycle through weight copies that together
    exceed the Infinity Cache.

    The timed region is exactly ``steps`` calls, bracketed by device synchronisations.
    Inside it, ``PRE_CALLS`` untimed calls are enqueued before the start event, so the
    event is stamped on a busy GPU: the host's first launch latency (argument checks,
    plan, ctypes) would otherwise land inside the region.  ``windows`` more regions of
    the same length follow for the median.  Returns (mean ms per call of the first
    region, number of weight copies, [ms per call of each extra region]).  mx: "split" times
    fb_gemv_mx (the native FP4 path, its x split included) instead of fb_gemv; "presplit"
    times fb_gemv_mx_presplit on one split made beforehand (what each further layer with the
    same input costs); "splitfloor" the same after an empty kernel with the split's launch
    shape (fb_phase_mx_floor of the diagnostic library): the floor of a separate split."""
    L = C.lib()
    shape = pw.shape(x.shape[0], x.dtype, y.dtype)
    sref = ctypes.byref(shape)
    ncp = n_copies(pw.wdev.numel(), cold)
    copies = [pw.wdev] + [pw.wdev.clone() for _ in range(ncp - 1)]
    wps = [c.data_ptr() for c in copies]
    xp, yp = x.data_ptr(), y.data_ptr()
    if mx == "split":
        ws = torch.zeros(C.mx_workspace_bytes(shape), dtype=torch.uint8, device=x.device)
        gemv = L.fb_gemv_mx
    elif mx in ("presplit", "splitfloor"):
        xsplit = C.mx_split_raw(x, shape)
        xp = xsplit.data_ptr()
        nws = L.fb_mx_presplit_workspace_bytes(sref)
        ws = torch.zeros(nws, dtype=torch.uint8, device=x.device) if nws else None
        gemv = L.fb_gemv_mx_presplit
        if mx == "splitfloor":
            tl = ctypes.CDLL(str(ROOT / "if_i_could_turn_back_time_amd" / "libfourbit_trace.so"))
            vp = ctypes.c_void_p
            gemv = tl.fb_phase_mx_floor
            gemv.restype = ctypes.c_int
            gemv.argtypes = [vp, vp, vp, ctypes.POINTER(C.FbShape), vp, ctypes.c_size_t, vp]
    else:
        ws = C.new_workspace(shape, x.device)
        gemv = L.fb_gemv
    wsp, nws = (ws.data_ptr(), ws.numel()) if ws is not None else (None, 0)
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    # Warm-up: at least `warmup` calls and at least MIN_WARM_S of back-to-back calls.  After
    # idle, MI355X runs the first ~20 ms of calls at lower clocks (~37 against ~30.5 us/call
    # on the north-star layer), so a short warm-up would time the clock ramp, not the kernel.
    done, t_end = 0, time.perf_counter() + MIN_WARM_S
    while done < warmup or time.perf_counter() < t_end:
        for _ in range(50):
            C.check(gemv(wps[done % ncp], xp, yp, sref, wsp, nws, sp))
            done += 1
        torch.cuda.synchronize()
    global LAST_WARMUP_CALLS
    LAST_WARMUP_CALLS = done

    def region():
        torch.cuda.synchronize()
        for i in range(PRE_CALLS):
            gemv(wps[i % ncp], xp, yp, sref, wsp, nws, sp)
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for i in range(steps):
            gemv(wps[(PRE_CALLS + i) % ncp], xp, yp, sref, wsp, nws, sp)
        t1.record(stream)
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / steps

    first = region()
    extra = [region() for _ in range(windows)]
    del copies
    return first, ncp, extra


def time_gpu_graph(pw, x, y, steps: int, reps: int = 5):
    """Same calls (one weight copy) captured in one HIP graph: launch overhead removed."""
    L = C.lib()
    shape = pw.shape(x.shape[0], x.dtype, y.dtype)
    sref = ctypes.byref(shape)
    ws = C.new_workspace(shape, x.device)
    wsp, nws = (ws.data_ptr(), ws.numel()) if ws is not None else (None, 0)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        C.check(L.fb_gemv(pw.wdev.data_ptr(), x.data_ptr(), y.data_ptr(), sref, wsp, nws,
                          s.cuda_stream))
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            for _ in range(steps):
                L.fb_gemv(pw.wdev.data_ptr(), x.data_ptr(), y.data_ptr(), sref, wsp, nws,
                          torch.cuda.current_stream().cuda_stream)
    graph.replay()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(reps):
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record()
        graph.replay()
        t1.record()
        torch.cuda.synchronize()
        best = min(best, t0.elapsed_time(t1) / steps)
    return best


def cpu_baseline(pw: PackedWeight, x: torch.Tensor, budget_s: float = 12.0):
    """The reference's forward structure on the host CPU (layers.py:36-38): every call
    dequantizes the packed weight to fp32 [N,K], then F.linear.  Run on a bounded row
    sample; throughput is the sample's algorithmic bytes per second."""
    from oracle import fourbit_oracle as O

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    codes_all = pw.codes
    meta_all = pw.meta
    N = pw.N
    rows = N

    def one_call(r):
        codes = O.unpack_nibbles(codes_all[:r].numpy())
        if pw.fmt_name == "gf4":
            W = O.dequant_f32("gf4", codes, meta_all[:r].numpy().view(np.uint16))
        else:
            W = O.dequant_f32("e2m1", codes, meta_all[:r].numpy())
        return torch.nn.functional.linear(x.float(), W)

    # size the sample so one call takes about a second
    probe = min(N, 512)
    t = time.perf_counter()
    one_call(probe)
    per_row = (time.perf_counter() - t) / probe
    rows = int(max(64, min(N, 1.0 / max(per_row, 1e-9))))
    one_call(rows)  # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 10 or (time.perf_counter() - t_start) < budget_s * 0.5:
        t = time.perf_counter()
        one_call(rows)
        times.append(time.perf_counter() - t)
        if time.perf_counter() - t_start > budget_s:
            break
    med = float(np.median(times))
    B = x.shape[0]
    frac = rows / N
    sample_bytes = pw.algorithmic_bytes(B) * frac
    # secondary: F.linear on an already-dequantized fp32 weight (the hard_quant forward,
    # layers.py:34-35), same rows
    codes = O.unpack_nibbles(codes_all[:rows].numpy())
    if pw.fmt_name == "gf4":
        Wc = O.dequant_f32("gf4", codes, meta_all[:rows].numpy().view(np.uint16))
    else:
        Wc = O.dequant_f32("e2m1", codes, meta_all[:rows].numpy())
    torch.nn.functional.linear(x.float(), Wc)
    hq = []
    t_start = time.perf_counter()
    while len(hq) < 10 or (time.perf_counter() - t_start) < 2.0:
        t = time.perf_counter()
        torch.nn.functional.linear(x.float(), Wc)
        hq.append(time.perf_counter() - t)
        if time.perf_counter() - t_start > 4.0:
            break
    hq_med = float(np.median(hq))
    return {
        "value": sample_bytes / med / 1e9,
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{rows} of {N} rows per call (dequantize packed->fp32 then F.linear, "
                   f"median of {len(times)} calls); CPU: {cpu_model()}, "
                   f"os.cpu_count()={threads}"),
        "us_per_call_full_layer_est": med / frac * 1e6,
        "hard_quant_cached_fp32": {
            "GBps_of_packed_bytes": sample_bytes / hq_med / 1e9,
            "us_per_call_full_layer_est": hq_med / frac * 1e6,
            "note": "F.linear on a cached fp32 weight (reads N*K*4 bytes, not the packed ones)",
        },
    }


def load_traffic(name: str):
    p = ROOT / "profiles" / f"traffic_{name}.json"
    if p.exists():
        try:
            return json.loads(p.read_text()).get("traffic_bytes")
        except Exception:
            return None
    return None


def time_gpu_pack(w: torch.Tensor, pw: PackedWeight, reps: int = 3):
    """The GPU Jenks packer (fb_quantize_gf4_gpu) on the same weights the host packer
    packed: best-of-reps seconds with the weights already in HBM, and whether its bytes
    equal the host packer's."""
    wd = w.to("cuda:0")
    best = float("inf")
    for _ in range(reps):
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record()
        codes, book = C.quantize_gf4_gpu(wd)
        t1.record()
        torch.cuda.synchronize()
        best = min(best, t0.elapsed_time(t1) / 1e3)
    same = bool(torch.equal(codes.cpu(), pw.codes) and torch.equal(book.cpu(), pw.meta))
    del wd, codes, book
    return {"gpu_s": best, "identical_to_host": same}


def run_workload(name: str, steps: int, warmup: int, want_cpu: bool, check: bool = True,
                 warm: bool = False, cache: dict | None = None, pack_check: bool = False,
                 packer: str = "host", windows: int = 0, cpu_budget_s: float = 12.0,
                 mx: str = ""):
    """cache: packed weights by (fmt, K, N, kind, rotation), reused across batch sizes (the
    weights are drawn before the activations, so they do not depend on the batch).  mx:
    "split" / "presplit", the native FP4 path (unrotated E2M1 workloads; see time_gpu)."""
    fmt, K, N, B, kind, fwht = WORKLOADS[name]
    if mx and (fmt != "e2m1" or fwht):
        raise ValueError(f"{name}: the native FP4 path takes unrotated E2M1 layers")
    xdt = torch.float16 if fmt in ("gf4", "int4ref") else torch.bfloat16
    w, x = workloads.synth(kind, N, K, B, xdt)
    fb = fwht_block_for(K) if fwht else 0
    key = (fmt, K, N, kind, fb)
    t = time.perf_counter()
    if cache is not None and key in cache:
        pw = cache[key]
    else:
        if fmt == "int4ref":
            # layers.py:23-26 and :39-45 with the rounding gate closed: level = floor(w / s),
            # s = amax / 7 + 1e-12, packed as integer levels times s
            sc = w.abs().amax(dim=1, keepdim=True) / 7 + 1e-12
            pw = PackedWeight.from_levels(torch.floor(w / sc), sc.reshape(-1), device="cuda:0")
        else:
            pw = PackedWeight.quantize(w, fmt, fwht_block=fb, device="cuda:0", packer=packer)
        if cache is not None:
            cache.clear()  # one layer's packed weights resident at a time
            cache[key] = pw
    pack_s = time.perf_counter() - t
    gpu_pack = None
    if pack_check and fmt == "gf4" and pw.fmt_name == "gf4":
        gpu_pack = time_gpu_pack(w if not fb else C.fwht_rows(w, fb), pw)
    del w
    xd = x.to("cuda:0")
    y = torch.empty(B, N, dtype=xdt, device="cuda:0")
    ms, ncp, extra = time_gpu(pw, xd, y, steps, warmup, cold=True, windows=windows, mx=mx)
    warm_calls = LAST_WARMUP_CALLS
    ms_warm = time_gpu(pw, xd, y, steps, warmup, cold=False)[0] if warm else None
    ms_graph = time_gpu_graph(pw, xd, y, min(steps, 200)) if warm else None
    nbytes = pw.algorithmic_bytes(B)
    # the reported time per call: the median over the timed regions (each the mean of its
    # back-to-back calls); the first region's mean is kept beside it
    ms_first = ms
    ms = float(np.median([ms_first] + extra))
    gbs = nbytes / (ms * 1e-3) / 1e9
    rec = {
        "workload": name, "fmt": fmt, "K": K, "N": N, "B": B, "fwht_block": fb,
        "path": {"split": "fp4_mfma", "presplit": "fp4_mfma_presplit",
                 "splitfloor": "fp4_mfma_presplit_after_empty_split"}.get(mx, "exact_decode"),
        "bytes_per_call": nbytes, "weight_stream_bytes": N * K // 2,
        "us_per_call": ms * 1e3, "GBps": gbs, "frac_of_8TBps": gbs / PEAK_GBS,
        "weight_copies_cycled": ncp, "warmup_calls_run": warm_calls,
        "us_per_call_warm": None if ms_warm is None else ms_warm * 1e3,
        "GBps_warm": None if ms_warm is None else nbytes / (ms_warm * 1e-3) / 1e9,
        "us_per_call_graph": None if ms_graph is None else ms_graph * 1e3,
        "GBps_graph": None if ms_graph is None else nbytes / (ms_graph * 1e-3) / 1e9,
        "tokens_per_s_equiv": B / (ms * 1e-3), "pack_s": pack_s, "gpu_pack": gpu_pack,
        "us_per_call_windows": [v * 1e3 for v in [ms_first] + extra],
        "us_per_call_median": ms * 1e3,
        "us_per_call_first_region": ms_first * 1e3,
    }
    if check:  # spot parity: sampled rows vs exact host decode + F.linear (fp32)
        yk = torch.empty(B, N, dtype=torch.float32, device="cuda:0")
        if mx == "split":
            pw.gemv_mx(xd, out=yk)
        elif mx in ("presplit", "splitfloor"):
            sh = pw.shape(B, xd.dtype, torch.float32)
            C.gemv_mx_presplit(pw.wdev, C.mx_split_raw(xd, sh), yk, sh)
        else:
            pw.gemv(xd, out=yk)
        rows = torch.randint(0, N, (64,), generator=torch.Generator().manual_seed(1))
        Wr = torch.from_numpy(np.stack([pw.dequant_host_row(int(r)) for r in rows]))
        xin = x.float()
        if fb:
            from oracle import fourbit_oracle as O
            xin = O.rotate_x(xin, fb)
        yref = torch.nn.functional.linear(xin, Wr)
        err = (yk.cpu()[:, rows] - yref).abs()
        rec["parity_ok"] = bool((err <= 1e-2 + 1e-3 * yref.abs()).all())
        rec["parity_max_abs_err"] = float(err.max())
    if want_cpu:
        rec["cpu_baseline"] = cpu_baseline(pw, x, cpu_budget_s)
    return rec, pw


def cpu_model() -> str:
    """The host CPU's model string (``/proc/cpuinfo``), for the CPU baseline record."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


PHASES = {  # lane index in the diagnostic build's per-wave record -> phase
    1: "x loads issued", 2: "x arrived", 3: "first unit issued", 4: "first 256 points done",
    5: "phase barrier", 6: "rotation done", 7: "x staged (barrier)", 12: "slice 1 staged",
    13: "slice 2 staged", 8: "first unit done", 14: "slice 0 loop end",
    15: "slice 1 loop end", 18: "first 4096-point group loaded", 19: "unit decoded ahead",
    9: "last loop end", 10: "final barrier", 11: "end",
}


def phase_trace(name: str, calls: int, packer: str, parts: int = 0) -> dict:
    """Per-wave phase timestamps of the GEMV on workload ``name``, from the diagnostic copy
    of the library (``libfourbit_trace.so``, built with FB_PHASE_TRACE: each wave records a
    100 MHz chip-wide clock at fixed points of the kernel).  ``calls`` traced calls run back
    to back after the usual warm-up, on cold weight copies; times are relative to the
    call's first wave start.  Also: each workgroup's end (its last wave's), grouped by the
    XCD it ran on, and the gap between one call's last end and the next call's first
    start.  ``parts`` (2, 4, 8; -1 = none) forces the split-K part count of batch >= 2
    calls in the diagnostic library (0: its own choice); a split-K call's second kernel
    (the part sum) is not traced."""
    tl = ctypes.CDLL(str(ROOT / "if_i_could_turn_back_time_amd" / "libfourbit_trace.so"))
    vp = ctypes.c_void_p
    tl.fb_gemv.restype = ctypes.c_int
    tl.fb_gemv.argtypes = [vp, vp, vp, ctypes.POINTER(C.FbShape), vp, ctypes.c_size_t, vp]
    tl.fb_phase_trace_set.argtypes = [vp, ctypes.c_size_t]
    ip = ctypes.POINTER(ctypes.c_int)
    tl.fb_phase_plan.argtypes = [ctypes.POINTER(C.FbShape), ip, ip, ip, ip, ip, ip]
    tl.fb_workspace_bytes.restype = ctypes.c_size_t
    tl.fb_workspace_bytes.argtypes = [ctypes.POINTER(C.FbShape)]
    C.check(tl.fb_phase_force_parts(parts))
    fmt, K, N, B, kind, fwht = WORKLOADS[name]
    xdt = torch.float16 if fmt in ("gf4", "int4ref") else torch.bfloat16
    w, x = workloads.synth(kind, N, K, B, xdt)
    fb = fwht_block_for(K) if fwht else 0
    if fmt == "int4ref":
        sc = w.abs().amax(dim=1, keepdim=True) / 7 + 1e-12
        pw = PackedWeight.from_levels(torch.floor(w / sc), sc.reshape(-1), device="cuda:0")
    else:
        pw = PackedWeight.quantize(w, fmt, fwht_block=fb, device="cuda:0", packer=packer)
    xd = x.to("cuda:0")
    y = torch.empty(B, N, dtype=xdt, device="cuda:0")
    shape = pw.shape(B, xd.dtype, y.dtype)
    need = tl.fb_workspace_bytes(ctypes.byref(shape))  # the diagnostic library's plan
    ws = torch.zeros(need, dtype=torch.uint8, device=xd.device) if need else None
    wsp, nws = (ws.data_ptr(), ws.numel()) if ws is not None else (None, 0)
    # with a workspace a rotated GEMV runs unrotated on the rotated x: that is the plan traced
    rot_once = ws is not None and fb and B * K >= 16384
    launched = C.make_shape(N, K, B, pw.fmt, 0 if rot_once else fb,
                            C.DTYPE_CODE[xd.dtype], C.DTYPE_CODE[y.dtype])
    plan = [ctypes.c_int() for _ in range(6)]
    C.check(tl.fb_phase_plan(ctypes.byref(launched), *[ctypes.byref(v) for v in plan]))
    grid, nw, S, tq, tr, P = (v.value for v in plan)
    wgs = grid * max(1, P)  # workgroups per call
    ncp = n_copies(pw.wdev.numel(), True)
    copies = [pw.wdev] + [pw.wdev.clone() for _ in range(ncp - 1)]
    sref = ctypes.byref(shape)
    sp = torch.cuda.current_stream().cuda_stream
    per_call = wgs * nw * 64
    bufs = torch.zeros(calls, per_call, dtype=torch.int64, device="cuda:0")

    def run(f, n, traced=False):
        for i in range(n):
            if traced:
                tl.fb_phase_trace_set(bufs[i].data_ptr(), per_call)
            C.check(f(copies[i % ncp].data_ptr(), xd.data_ptr(), y.data_ptr(), sref, wsp, nws, sp))
        if traced:
            tl.fb_phase_trace_set(None, 0)

    def timed(f, n=200):
        run(f, PRE_CALLS)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        run(f, n)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n * 1e3

    t_end = time.perf_counter() + MIN_WARM_S
    while time.perf_counter() < t_end:
        run(tl.fb_gemv, 50)
        torch.cuda.synchronize()
    run(tl.fb_gemv, PRE_CALLS)
    run(tl.fb_gemv, calls, traced=True)
    torch.cuda.synchronize()
    us_traced_lib = timed(tl.fb_gemv)
    us_product = timed(C.lib().fb_gemv)
    C.check(tl.fb_phase_force_parts(0))
    t = bufs.cpu().numpy().astype(np.int64).reshape(calls, wgs, nw, 64)
    del bufs, copies
    start = t[..., 0]
    g0 = start.reshape(calls, -1).min(axis=1)[:, None, None]
    us = lambda v: v / 100.0  # 100 MHz ticks -> us

    def stats(v):
        return {"median": round(float(np.median(v)), 3), "p90": round(float(np.percentile(v, 90)), 3),
                "max": round(float(v.max()), 3)}

    phases = {"wave start": stats(us(start - g0))}
    for i, label in PHASES.items():
        v = t[..., i]
        ok = v != 0
        if not ok.any():
            continue
        phases[label] = dict(stats(us((v - g0)[ok])),
                             from_own_start_median=round(float(np.median(us((v - start)[ok]))), 3))
    wg_end = us(t[..., 11].max(axis=2) - g0[:, :, 0])            # [calls, grid]
    xcc = t[:, :, 0, 16] & 0xF                                    # [calls, grid]
    xcd_med = np.array([[np.median(wg_end[c][xcc[c] == k]) if (xcc[c] == k).any() else np.nan
                         for k in range(8)] for c in range(calls)])
    span = wg_end.max(axis=1)
    gaps = [us(start[c + 1].min() - t[c, ..., 11].max()) for c in range(calls - 1)]
    period = [us(start[c + 1].min() - start[c].min()) for c in range(calls - 1)]
    return {
        "phase_trace": name, "calls": calls, "plan": {"grid": grid, "waves": nw, "slices": S,
                                                      "tiles_per_wg": tq, "wgs_with_one_more": tr,
                                                      "splitk_parts": P},
        "rotate_once": bool(rot_once),
        "us_per_call_untraced": round(us_product, 3), "us_per_call_trace_build": round(us_traced_lib, 3),
        "phases_us_from_call_start": phases,
        "workgroup_end_us": dict(stats(wg_end), p10=round(float(np.percentile(wg_end, 10)), 3),
                                 min=round(float(wg_end.min()), 3)),
        "first_start_to_last_end_us_median": round(float(np.median(span)), 3),
        "xcd_median_end_us_per_call": [[round(float(v), 2) for v in row] for row in xcd_med],
        "slowest_xcd_per_call": [int(np.nanargmax(row)) for row in xcd_med],
        "xcd_spread_us_median": round(float(np.median(np.nanmax(xcd_med, 1) - np.nanmin(xcd_med, 1))), 3),
        "gap_last_end_to_next_start_us": stats(np.array(gaps)) if gaps else None,
        "start_to_next_start_us": stats(np.array(period)) if period else None,
        # whether the slow workgroups are the same ones from call to call
        "slowest_workgroups_per_call": [[int(g) for g in np.argsort(wg_end[c])[-4:][::-1]]
                                        for c in range(calls)],
        "workgroup_end_rank_corr_between_calls": round(float(np.mean(
            [np.corrcoef(np.argsort(np.argsort(wg_end[c])), np.argsort(np.argsort(wg_end[c + 1])))[0, 1]
             for c in range(calls - 1)])), 3) if calls > 1 else None,
        "workgroup_start_us": stats(us(start.min(axis=2) - g0[:, :, 0])),
        # each phase after the workgroup's first wave start, median by wave index (the SIMDs
        # issue a workgroup's older waves first)
        "phase_by_wave_us": {label: [round(float(np.median(us(t[:, :, i, k] - start.min(axis=2))[
            t[:, :, i, k] != 0])), 3) if (t[:, :, i, k] != 0).any() else None for i in range(nw)]
            for k, label in PHASES.items() if (t[..., k] != 0).any()},
        "corr_start_end": round(float(np.corrcoef(us(start.min(axis=2) - g0[:, :, 0]).ravel(),
                                                  wg_end.ravel())[0, 1]), 3),
    }


def jenks2_bench(n: int, steps: int) -> dict:
    """Two-class natural breaks (fb_jenks2_gpu) over n resident fp32 values: sort, blocked
    fp64 prefix sums, SSD per split, first argmin, mask.  Timed with HIP events over
    back-to-back calls on one preallocated workspace; the host twin (fb_jenks2_host, one
    thread) runs once on the same values and must give the same split, GVF and mask."""
    L = C.lib()
    g = torch.Generator().manual_seed(7)
    w = (torch.randn(n, generator=g) * 0.05)
    wd = w.to("cuda:0")
    need = ctypes.c_size_t(0)
    C.check(L.fb_jenks2_workspace(n, ctypes.byref(need)))
    ws = torch.empty(need.value + 256, dtype=torch.uint8, device="cuda:0")
    wsp = ws.data_ptr() + (-ws.data_ptr()) % 256
    keep = torch.empty(n, dtype=torch.uint8, device="cuda:0")
    out = torch.empty(2, dtype=torch.float64, device="cuda:0")
    sp = torch.cuda.current_stream().cuda_stream

    def call():
        C.check(L.fb_jenks2_gpu(wd.data_ptr(), n, keep.data_ptr(), out.data_ptr(),
                                out.data_ptr() + 8, wsp, need.value, sp))

    t_end = time.perf_counter() + MIN_WARM_S
    while time.perf_counter() < t_end:
        for _ in range(5):
            call()
        torch.cuda.synchronize()
    regions = []
    for _ in range(5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        call()
        e0.record()
        for _ in range(steps):
            call()
        e1.record()
        torch.cuda.synchronize()
        regions.append(e0.elapsed_time(e1) / steps * 1e3)
    host = out.cpu()
    split = int(host[:1].view(torch.int64).item())
    t = time.perf_counter()
    hk, hsplit, hgvf = C.jenks2_host(w)
    host_s = time.perf_counter() - t
    same = (hsplit == split and hgvf == float(host[1].item())
            and torch.equal(hk, keep.cpu().bool()))
    us = float(np.median(regions))
    return {"jenks2_values": n, "us_per_call_median": us, "us_per_call_regions": regions,
            "values_per_s": n / (us * 1e-6), "workspace_bytes": need.value,
            "split": split, "gvf": float(host[1].item()), "host_twin_s": host_s,
            "host_twin_threads": 1, "identical_to_host": bool(same)}


def jenks2_filters_bench(shape, steps: int) -> dict:
    """The per-filter two-class split (fb_jenks2_filters_gpu, the reference's Conv_Mask) over
    a resident [out, in, kh, kw] fp32 weight: one 64-lane workgroup per filter.  Timed with
    HIP events over back-to-back calls; the host twin (fb_jenks2_filters_host, 16 threads)
    runs once on the same weight and must give the same splits, GVFs and mask."""
    L = C.lib()
    out_c, in_c, kh, kw = shape
    nf, n = out_c * in_c, kh * kw
    g = torch.Generator().manual_seed(8)
    w = torch.randn(nf, n, generator=g) * 0.05
    wd = w.to("cuda:0")
    keep = torch.empty(nf, n, dtype=torch.uint8, device="cuda:0")
    split = torch.empty(nf, dtype=torch.int32, device="cuda:0")
    gvf = torch.empty(nf, dtype=torch.float64, device="cuda:0")
    sp = torch.cuda.current_stream().cuda_stream

    def call():
        C.check(L.fb_jenks2_filters_gpu(wd.data_ptr(), nf, n, keep.data_ptr(), split.data_ptr(),
                                        gvf.data_ptr(), sp))

    t_end = time.perf_counter() + MIN_WARM_S
    while time.perf_counter() < t_end:
        for _ in range(5):
            call()
        torch.cuda.synchronize()
    regions = []
    for _ in range(5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        call()
        e0.record()
        for _ in range(steps):
            call()
        e1.record()
        torch.cuda.synchronize()
        regions.append(e0.elapsed_time(e1) / steps * 1e3)
    t = time.perf_counter()
    hk, hs, hg = C.jenks2_filters_host(w, nthreads=16)
    host_s = time.perf_counter() - t
    same = (torch.equal(hk, keep.cpu().bool()) and torch.equal(hs, split.cpu())
            and torch.equal(hg.view(torch.int64), gvf.cpu().view(torch.int64)))
    us = float(np.median(regions))
    return {"jenks2_filters": list(shape), "filters": nf, "values_per_filter": n,
            "us_per_call_median": us, "us_per_call_regions": regions,
            "filters_per_s": nf / (us * 1e-6), "host_twin_s": host_s, "host_twin_threads": 16,
            "identical_to_host": bool(same)}


def xfill_bench(steps: int = 200) -> list:
    """The fill rate of x staging alone (fb_phase_xfill of the diagnostic library): one
    workgroup per CU reads the same x bytes into LDS in 16-byte chunks, the way the GEMV's x
    preload does, with no weight stream beside it.  Per size (16 KiB ... 256 KiB: batch 1 to 16
    at K = 8192), threads (1024 = the 16-wave plan, 512 = the 8-wave one) and passes (a second
    pass reads what the first left in the caches): the median over waves of the time from the
    wave's own start until its loads are issued, until they have arrived and until the
    barrier, in µs of the 100 MHz chip clock, and µs per launch back to back (HIP events)."""
    tl = ctypes.CDLL(str(ROOT / "if_i_could_turn_back_time_amd" / "libfourbit_trace.so"))
    vp, ci = ctypes.c_void_p, ctypes.c_int
    tl.fb_phase_xfill.argtypes = [vp, ci, ci, ci, ci, vp, vp]
    tl.fb_phase_xfill.restype = ci
    grid = torch.cuda.get_device_properties(0).multi_processor_count
    x = torch.randint(0, 255, (256 * 1024,), dtype=torch.uint8, device="cuda:0")
    ts = torch.zeros(grid * 16 * 4, dtype=torch.int64, device="cuda:0")
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    out = []
    for threads in (1024, 512):
        for kib in (16, 32, 64, 128, 256):
            for passes in (1, 2):
                args = (x.data_ptr(), kib * 1024, threads, passes, grid, ts.data_ptr(), sp)
                for _ in range(200):  # past the clock ramp
                    C.check(tl.fb_phase_xfill(*args))
                torch.cuda.synchronize()
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for _ in range(steps):
                    tl.fb_phase_xfill(*args)
                e1.record(stream)
                C.check(tl.fb_phase_xfill(*args))  # the launch whose timestamps are read
                torch.cuda.synchronize()
                nw = threads // 64
                t = ts[: grid * nw * 4].view(grid * nw, 4).cpu().double() / 100.0
                own = [float((t[:, i] - t[:, 0]).median()) for i in (1, 2, 3)]
                out.append({"xfill_KiB": kib, "threads": threads, "passes": passes, "grid": grid,
                            "us_per_launch": e0.elapsed_time(e1) / steps * 1e3,
                            "issued_us": own[0], "arrived_us": own[1], "barrier_us": own[2],
                            "span_us": float(t[:, 3].max() - t[:, 0].min())})
    return out


FLOOR_WORKLOADS = ("gf4_k4096_n4096_b1", "e2m1_k4096_n4096_b1", "e2m1_k4096_n11008_b1",
                   "e2m1_k11008_n4096_b1", "gf4fwht_k4096_n4096_b1", "gf4fwht_k4096_n11008_b1",
                   "gf4fwht_k11008_n4096_b1", "gf4_k8192_n28672_b1")


def floor_bench(names, steps: int, regions: int = 10) -> list:
    """The launch floor of each batch-1 workload's plan: an empty kernel with the GEMV's
    grid, waves, LDS, register count and argument block (fb_phase_floor of the diagnostic
    library), launched back to back, against the product GEMV launched the same way (cold:
    weight copies cycled).  Each is timed twice: launched from Python one call at a time
    (host launch work included, as in the default bench), and replayed from a HIP graph of
    ``steps`` launches (the device's own cost per launch).  Median µs per call over
    ``regions`` regions, HIP events on the launch stream."""
    tl = ctypes.CDLL(str(ROOT / "if_i_could_turn_back_time_amd" / "libfourbit_trace.so"))
    vp = ctypes.c_void_p
    tl.fb_phase_floor.argtypes = [ctypes.POINTER(C.FbShape), vp]
    tl.fb_phase_floor.restype = ctypes.c_int
    out = []
    for name in names:
        fmt, K, N, B, kind, fwht = WORKLOADS[name]
        xdt = torch.float16 if fmt == "gf4" else torch.bfloat16
        w, x = workloads.synth(kind, N, K, B, xdt)
        fb = fwht_block_for(K) if fwht else 0
        pw = PackedWeight.quantize(w, fmt, fwht_block=fb, device="cuda:0", packer="gpu")
        xd = x.to("cuda:0")
        y = torch.empty(B, N, dtype=xdt, device="cuda:0")
        shape = pw.shape(B, xd.dtype, y.dtype)
        sref = ctypes.byref(shape)
        stream = torch.cuda.current_stream()
        sp = stream.cuda_stream
        for _ in range(2000):  # warm-up past the clock ramp
            C.check(tl.fb_phase_floor(sref, sp))
        torch.cuda.synchronize()
        floor = []
        for _ in range(regions):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            for _ in range(PRE_CALLS):
                tl.fb_phase_floor(sref, sp)
            e0.record(stream)
            for _ in range(steps):
                tl.fb_phase_floor(sref, sp)
            e1.record(stream)
            torch.cuda.synchronize()
            floor.append(e0.elapsed_time(e1) / steps * 1e3)
        first, _, extra = time_gpu(pw, xd, y, steps, 50, cold=True, windows=regions - 1)
        gemv = [v * 1e3 for v in [first] + extra]
        # the same launches replayed from a HIP graph: no host work per launch
        ncp = n_copies(pw.wdev.numel(), True)
        copies = [pw.wdev] + [pw.wdev.clone() for _ in range(ncp - 1)]
        L = C.lib()
        g_floor, g_gemv = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            C.check(L.fb_gemv(copies[0].data_ptr(), xd.data_ptr(), y.data_ptr(), sref, None, 0,
                              side.cuda_stream))
            torch.cuda.synchronize()
            with torch.cuda.graph(g_floor, stream=side):
                for _ in range(steps):
                    C.check(tl.fb_phase_floor(sref, side.cuda_stream))
            with torch.cuda.graph(g_gemv, stream=side):
                for i in range(steps):
                    C.check(L.fb_gemv(copies[i % ncp].data_ptr(), xd.data_ptr(), y.data_ptr(),
                                      sref, None, 0, side.cuda_stream))
        torch.cuda.synchronize()

        def replay(gr):
            vals = []
            for _ in range(3):
                gr.replay()
            torch.cuda.synchronize()
            for _ in range(regions):
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                gr.replay()
                e1.record(stream)
                torch.cuda.synchronize()
                vals.append(e0.elapsed_time(e1) / steps * 1e3)
            return vals

        floor_g, gemv_g = replay(g_floor), replay(g_gemv)
        del g_floor, g_gemv, copies
        nbytes = pw.algorithmic_bytes(B)
        f_med, g_med = float(np.median(floor)), float(np.median(gemv))
        fg_med, gg_med = float(np.median(floor_g)), float(np.median(gemv_g))
        out.append({"workload": name, "bytes_per_call": nbytes,
                    "floor_us_per_call_median": f_med, "floor_us_per_call_regions": floor,
                    "gemv_us_per_call_median": g_med, "gemv_us_per_call_regions": gemv,
                    "graph_floor_us_per_call_median": fg_med,
                    "graph_gemv_us_per_call_median": gg_med,
                    "graph_floor_us_per_call_regions": floor_g,
                    "graph_gemv_us_per_call_regions": gemv_g,
                    "GBps_eager": nbytes / (g_med * 1e-6) / 1e9,
                    "GBps_graph": nbytes / (gg_med * 1e-6) / 1e9})
        del pw, xd, y
        torch.cuda.empty_cache()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--workload", default=DEFAULT, choices=sorted(WORKLOADS))
    ap.add_argument("--sweep", action="store_true", help="also time every config shape")
    ap.add_argument("--sweep-out", default="bench_sweep.jsonl")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-pack-check", action="store_true",
                    help="skip timing the GPU packer against the host packer")
    ap.add_argument("--packer", choices=("host", "gpu"), default="host",
                    help="where the GF4 Jenks search runs when packing the synthetic weights "
                         "(same bytes either way)")
    ap.add_argument("--warm", action="store_true",
                    help="also time one weight copy (Infinity-Cache warm) and a HIP graph")
    ap.add_argument("--calib-copy", type=int, default=0, metavar="BYTES",
                    help="only run device-to-device copies of BYTES bytes (PMC calibration)")
    ap.add_argument("--phase-trace", action="store_true",
                    help="only trace the GEMV's phases on --workload (diagnostic library) and "
                         "print a JSON summary")
    ap.add_argument("--parts", type=int, default=0,
                    help="with --phase-trace: force the split-K part count (2, 4, 8; -1 none)")
    ap.add_argument("--jenks2", type=int, default=0, metavar="N",
                    help="only time the two-class Jenks mask (fb_jenks2_gpu) over N values")
    ap.add_argument("--mx", action="store_true",
                    help="only compare the native FP4 path (fb_gemv_mx) with the exact-decode "
                         "path on every unrotated E2M1 workload (or --workload, if it is one), "
                         "one JSON line per path, with the FP4 GEMV on a pre-made split, alone "
                         "and after an empty kernel of the split's launch shape")
    ap.add_argument("--floor", action="store_true",
                    help="only time the launch floor (an empty kernel with each batch-1 "
                         "workload's plan) against the GEMV, one JSON line per workload "
                         "(--workload narrows it to one)")
    ap.add_argument("--xfill", action="store_true",
                    help="only time x staging alone (every CU reading the same 16-256 KiB into "
                         "LDS, no weights), one JSON line per size, thread count and pass count")
    ap.add_argument("--jenks2-filters", default="", metavar="OUT,IN,KH,KW",
                    help="only time the per-filter Jenks mask (fb_jenks2_filters_gpu) on a "
                         "convolution weight of that shape")
    args = ap.parse_args()
    if args.calib_copy:
        # a plain copy kernel of known size: FETCH_SIZE / WRITE_SIZE per dispatch of it
        # give the scale between those counters and bytes moved
        src = torch.randint(0, 255, (args.calib_copy,), dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calib_copy_bytes": args.calib_copy, "copies": args.steps}))
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (got --gpus {args.gpus}); the "
              "multi-GPU sharding of the GEMV is a design note, not a measured path.",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        sys.exit(1)
    if args.phase_trace:
        print(json.dumps(phase_trace(args.workload, 20, args.packer, args.parts)))
        return
    if args.jenks2:
        print(json.dumps(jenks2_bench(args.jenks2, min(args.steps, 50))))
        return
    if args.xfill:
        for rec in xfill_bench(min(args.steps, 200)):
            print(json.dumps(rec), flush=True)
        return
    if args.floor:
        names = [args.workload] if args.workload in FLOOR_WORKLOADS and "--workload" in sys.argv \
            else list(FLOOR_WORKLOADS)
        for rec in floor_bench(names, min(args.steps, 400)):
            print(json.dumps(rec), flush=True)
        return
    if args.mx:
        names = [n for n in sorted(WORKLOADS) if WORKLOADS[n][0] == "e2m1" and not WORKLOADS[n][5]]
        if args.workload in names:
            names = [args.workload]
        cache = {}
        for name in names:
            for mx in ("", "split", "presplit", "splitfloor"):
                rec, pw = run_workload(name, args.steps, args.warmup, False, cache=cache,
                                       windows=MEDIAN_WINDOWS, mx=mx)
                del pw
                print(json.dumps({k: rec[k] for k in (
                    "workload", "path", "K", "N", "B", "bytes_per_call", "us_per_call_median",
                    "us_per_call_windows", "parity_ok", "parity_max_abs_err")}), flush=True)
        return
    if args.jenks2_filters:
        shape = tuple(int(v) for v in args.jenks2_filters.split(","))
        if len(shape) != 4:
            ap.error("--jenks2-filters takes OUT,IN,KH,KW")
        print(json.dumps(jenks2_filters_bench(shape, min(args.steps, 50))))
        return

    if args.sweep:
        Path(args.sweep_out).parent.mkdir(parents=True, exist_ok=True)
        cache = {}
        order = sorted(WORKLOADS, key=lambda n: WORKLOADS[n][:3] + WORKLOADS[n][4:])
        with open(args.sweep_out, "w") as f:
            for name in order:
                if name == args.workload:
                    continue
                rec, pw = run_workload(name, max(50, args.steps // 2), args.warmup, False,
                                       warm=args.warm, cache=cache, packer=args.packer,
                                       windows=SWEEP_WINDOWS)
                del pw
                torch.cuda.empty_cache()
                f.write(json.dumps(rec) + "\n")
                f.flush()
                print(f"[sweep] {name}: {rec['us_per_call_median']:.2f} us (median), "
                      f"{rec['GBps']:.0f} GB/s, "
                      f"parity {rec.get('parity_ok')}", file=sys.stderr, flush=True)

    rec, pw = run_workload(args.workload, args.steps, args.warmup, not args.no_cpu,
                           warm=args.warm, pack_check=not args.no_pack_check, packer=args.packer,
                           windows=MEDIAN_WINDOWS)
    del pw
    torch.cuda.empty_cache()
    cfg1 = None
    if not args.no_cpu and args.workload != workloads.CPU_CONFIG:
        # the configuration the reference's CPU path is quoted on, GPU and CPU side by side
        r1, pw1 = run_workload(workloads.CPU_CONFIG, args.steps, args.warmup, True,
                               windows=MEDIAN_WINDOWS, cpu_budget_s=8.0)
        del pw1
        cfg1 = {"workload": workloads.CPU_CONFIG, "gpu_us_per_call": r1["us_per_call"],
                "gpu_us_per_call_median": r1["us_per_call_median"], "gpu_GBps": r1["GBps"],
                "parity_ok": r1.get("parity_ok"),
                "cpu": {k: v for k, v in r1["cpu_baseline"].items() if k != "hard_quant_cached_fp32"},
                "cpu_hard_quant_cached_fp32": r1["cpu_baseline"]["hard_quant_cached_fp32"]}
    fmt, K, N, B = rec["fmt"], rec["K"], rec["N"], rec["B"]
    achieved = rec["GBps"]
    out = {
        "metric": METRIC,
        "value": achieved,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": rec["us_per_call"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16" if fmt == "gf4" else "bf16",
        "data": "synthetic (seeded; weights packed by the native Jenks/E2M1 packer)",
        "config": {
            "workload": args.workload, "format": fmt, "K": K, "N": N, "batch": B,
            "fwht_block": rec["fwht_block"], "group": 128 if fmt == "gf4" else 32,
            "accumulate": "fp32", "us_per_call": rec["us_per_call"],
            "frac_of_peak": achieved / PEAK_GBS,
            "tokens_per_s_equiv": rec["tokens_per_s_equiv"],
            "bytes_per_call": rec["bytes_per_call"],
            "weight_stream_bytes": rec["weight_stream_bytes"],
            "timing": (f"cold: {rec['weight_copies_cycled']} weight copies cycled so every "
                       "call streams from HBM, not the 256 MiB Infinity Cache; warm-up of "
                       f"{rec['warmup_calls_run']} calls (at least --warmup and "
                       f"{MIN_WARM_S} s, past the GPU's clock ramp after idle)"),
            "us_per_call_median": rec["us_per_call_median"],
            "us_per_call_first_region": rec["us_per_call_first_region"],
            "median_note": (f"value, ms_per_step and us_per_call are the median over "
                            f"{1 + MEDIAN_WINDOWS} timed regions of --steps back-to-back calls "
                            "(each region's mean per call); the first region's mean is "
                            "us_per_call_first_region"),
            "us_per_call_regions": rec["us_per_call_windows"],
            "us_per_call_warm_single_copy": rec["us_per_call_warm"],
            "GBps_warm_single_copy": rec["GBps_warm"],
            "us_per_call_hipgraph_warm": rec["us_per_call_graph"],
            "parity_ok": rec.get("parity_ok"),
            "pack_host_s": rec["pack_s"],
            "pack_gpu": rec["gpu_pack"],
            "cpu_hard_quant_cached_fp32": (rec["cpu_baseline"] or {}).get("hard_quant_cached_fp32")
            if rec.get("cpu_baseline") else None,
            "cpu_config1": cfg1,
        },
        "roofline": {
            "bound": "hbm", "achieved": achieved, "peak": PEAK_GBS, "unit": "GB/s",
            "frac": achieved / PEAK_GBS, "traffic": load_traffic(args.workload),
            "traffic_source": (f"profiles/traffic_{args.workload}.json: rocprofv3 --pmc "
                               "FETCH_SIZE + WRITE_SIZE per dispatch, each scaled by the same "
                               "counter on a plain copy of known size; not measured in this run")
            if load_traffic(args.workload) is not None else None,
        },
        "cpu_baseline": rec.get("cpu_baseline"),
    }
    if out["cpu_baseline"] is not None:
        out["cpu_baseline"] = {k: v for k, v in out["cpu_baseline"].items()
                               if k in ("value", "unit", "cores", "kind", "sample")}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
