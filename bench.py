"""Benchmark of the MI355X conv hot path on BASELINE.json's metric:
"conv TFLOP/s (% fp32-MFMA peak) + decoder audio-sec/sec at 1 and 8 streams".

One step = BASELINE config 5, the largest single-GPU configuration: 8 independent decoder requests
(T ~ U[56, 400] frames, seeded) on 8 contexts / HIP streams driven by 8 pthreads, plus one
long-form request of T = 1500 frames through 96-frame overlap-save windows with 16-frame context
on a ninth context, all sharing one uploaded weight set.  Inputs are resident in HBM before the
timed region; `value` is the step's audio seconds divided by its wall time.  Alongside: config 4
(one request, T = 226) on one stream, eager, replayed as a HIP graph and eight at a time, and
driven through the reference ABI on host buffers (PCIe-inclusive); the long-form request window by
window (time to first audio) and batched; the queue-fed server; the container load and
pt_v21_matmul; configs 1-3 in TFLOP/s; the dominant kernel against the fp32-MFMA roofline and the
tail kernel against HBM (HIP events on the stream they run on); and the reference's CPU conv path
timed on this host on a bounded sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
       python bench.py --kernel-loop N   (only the dominant kernel and the tail kernel, N launches
                                          each after a clock warm-up: for rocprofv3)
       python bench.py --decode-loop N [--batch B]   (N config-4 decodes, for a kernel trace)
       python bench.py --streams8-loop N   (N steps of the T = 226 request on 8 concurrent
                                          streams after ~60 ms of the same, for a kernel trace)
       python bench.py --queue-table KERNEL_TRACE_CSV [--steps N]   (the last N steps of a
                                          --streams8-loop trace: busy time, kernels in flight,
                                          kernel time per hardware queue, per kernel)
       python bench.py --layer-table KERNEL_TRACE_CSV [--batch B] [--counters COUNTER_CSV]
                                          (per-launch table of that trace, MFMA utilisation from a
                                          --pmc pass over the same loop)
"""
from __future__ import annotations

import argparse
import ctypes as C
import importlib.util
import json
import os
import pathlib
import re
import sys
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
SR = 16000
HOP = 256                      # output samples per frame
MFMA_F32_PEAK = 157.3          # TFLOP/s, MI355X dense fp32 matrix (vendor figure)
HBM_PEAK = 8000.0              # GB/s


def _package():
    init = ROOT / "prime-tts_amd" / "__init__.py"
    spec = importlib.util.spec_from_file_location("prime_tts_amd", init,
                                                  submodule_search_locations=[str(init.parent)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["prime_tts_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


PROFILE_DOMINANT = ROOT / "profiles" / "conv_mfma_mrf256_group_T904.md"


def measured_traffic():
    """HBM bytes per launch of the dominant kernel, as the committed rocprofv3 summary states them
    (FETCH_SIZE and WRITE_SIZE passes over `bench.py --kernel-loop`, scaled by the copy-kernel
    calibration); None when the summary is absent."""
    try:
        text = PROFILE_DOMINANT.read_text()
    except OSError:
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", text, re.M)
    return int(m.group(1)) if m else None


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class EventTimer:
    """HIP events recorded on a context's stream (the stream the kernels run on)."""

    def __init__(self, pkg, ctx):
        self.lib, self.ctx = pkg.load(), ctx
        self.e0, self.e1 = self.lib.ptd_event_create(), self.lib.ptd_event_create()
        self.w = [self.lib.ptd_event_create(), self.lib.ptd_event_create()]

    def warm(self, fn, ms=None):
        """Untimed calls of fn issued for `ms` of host time (WARM_MS), the device kept busy: after
        an idle spell the MI355X's clock climbs for ~30 ms of sustained load, and launches timed
        inside that climb run up to 15 % slower.  The stream is not drained afterwards: the timed
        calls queue behind these (small launches issued into a just-drained stream ran ~20 %
        slower for their first hundred or so)."""
        ms = WARM_MS if ms is None else ms
        t0 = time.perf_counter()
        k = 0
        while (time.perf_counter() - t0) * 1e3 < ms:
            t1 = time.perf_counter()
            for _ in range(16):
                fn()
                if (time.perf_counter() - t1) * 1e3 >= 1.0:
                    break
            # at most two batches (16 calls or 1 ms of issue each) queued: wait for the end of the
            # previous batch (elapsed time of an event to itself waits for it), then mark the end
            # of this one
            if k:
                self.lib.ptd_event_elapsed_ms(self.w[(k - 1) & 1], self.w[(k - 1) & 1])
            self.lib.ptd_event_record(self.ctx.ptr, self.w[k & 1])
            k += 1

    def time(self, fn, reps, warmup=0, warm_ms=None, blocker=None):
        """ms per call of fn over reps calls, after WARM_MS (or warm_ms) of untimed calls and then
        warmup more untimed calls on the same stream.  blocker (for launches of a few us, whose
        issue from Python takes ~4 us each): untimed GPU work of ~1 ms queued right before the
        start event, so all reps calls are queued before the GPU reaches them and the host's
        issue rate cannot set the measured one."""
        self.warm(fn, warm_ms)
        for _ in range(warmup):
            fn()
        if blocker is not None:
            blocker()
        self.lib.ptd_event_record(self.ctx.ptr, self.e0)
        for _ in range(reps):
            fn()
        self.lib.ptd_event_record(self.ctx.ptr, self.e1)
        ms = self.lib.ptd_event_elapsed_ms(self.e0, self.e1)
        if ms < 0:
            raise RuntimeError("event timing failed")
        return ms / reps

    def close(self):
        for e in [self.e0, self.e1] + self.w:
            self.lib.ptd_event_destroy(e)


def mrf_depth_setup(pkg, ctx, stage, T):
    """Inputs of one MRF residual unit as the decoder hands them over: the branch inputs and their
    LeakyReLU(0.1) copies (written by the producing conv's epilogue in the decoder)."""
    C_ = 256 if stage == 0 else 128
    rng = np.random.default_rng(77)
    xr = [rng.standard_normal((C_, T)).astype(np.float32) for _ in range(3)]
    xs = [pkg.DevBuf.of(ctx, x) for x in xr]
    xls = [pkg.DevBuf.of(ctx, np.where(x >= 0, x, np.float32(0.1) * x).astype(np.float32)) for x in xr]
    a_s = [pkg.DevBuf(C_ * T) for _ in range(3)]
    ys = [pkg.DevBuf(C_ * T) for _ in range(3)]
    arr = lambda bufs: (C.c_void_p * 3)(*[b.ptr for b in bufs])  # noqa: E731
    return xs + xls + a_s + ys, arr(xs), arr(xls), arr(a_s), arr(ys)


TAIL_L = 16 * 226 + 1   # conv_post frames of a T = 226 request


def tail_setup(pkg, ctx, L, batch):
    """conv_post-shaped input [batch][72][L] (log-magnitudes and phase logits ~ N(0, 0.5)) and the
    waveform buffer for ptd_tail."""
    p = (0.7 * np.random.default_rng(9).standard_normal((batch, 72, L))).astype(np.float32)
    return pkg.DevBuf.of(ctx, p), pkg.DevBuf(batch * 16 * (L - 1))


def tail_bytes(L, batch):
    """Algorithmic HBM bytes of one tail launch: read conv_post's 72 rows, write the waveform."""
    return 4.0 * batch * (72 * L + 16 * (L - 1))


# Untimed load before each timed leg: the chip's clock reaches its sustained value ~30 ms into a
# run of launches after an idle spell (the dominant launch: 28-30 us per launch for the first
# ~7 ms, 24.3 us from ~30 ms on).
WARM_MS = 60.0


def decode_loop_warm(batch):
    """Warm-up decodes of `--decode-loop` (dropped from its layer table): about WARM_MS of load at
    ~0.3 ms per request."""
    return max(3, int(WARM_MS / (0.3 * batch)))

# The 19 launches of one decode at T = 226 frames, in issue order (pt_decoder.c decode_impl), with
# the algorithmic work of one request: flop for the conv launches (the MRF entries are grouped
# launches of the three branch convs, K 3 + 7 + 11), HBM bytes for the elementwise and tail ones.
_T1, _T2, _L = 4 * 226, 16 * 226, 16 * 226 + 1
DECODE_LAUNCHES = (
    [("conv_pre 192->512 K7", "flop", 2.0 * 512 * 192 * 7 * 226),
     ("ups.0 convT 512->256 K16 s4", "flop", 2.0 * 256 * 512 * 4 * _T1)]
    + [(f"MRF-256 d{d} {w} (K 3/7/11)", "flop", 2.0 * 256 * 256 * _T1 * 21)
       for d in (1, 3, 5) for w in ("c1", "c2")]
    + [("branch avg + leaky (256)", "bytes", 4.0 * 4 * 256 * _T1),
       ("ups.1 convT 256->128 K16 s4", "flop", 2.0 * 128 * 256 * 4 * _T2)]
    + [(f"MRF-128 d{d} {w} (K 3/7/11)", "flop", 2.0 * 128 * 128 * _T2 * 21)
       for d in (1, 3, 5) for w in ("c1", "c2")]
    + [("branch avg + leaky (128)", "bytes", 4.0 * 4 * 128 * _T2),
       ("conv_post 128->72 K7", "flop", 2.0 * 72 * 128 * 7 * _L),
       ("tail: iSTFT + PQMF", "bytes", 4.0 * (72 * _L + 16 * (_L - 1)))])


# flop per GEMM column of the 40 conv launches of a decode, in ptd_window_cols order: conv_pre,
# ups.0 (phase form: a column is 4 outputs of 4 taps each), MRF-256 (depth, branch K 3/7/11,
# c1 / c2), ups.1, MRF-128, conv_post
_COL_FLOP = ([2.0 * 512 * 192 * 7, 2.0 * 4 * 256 * 512 * 4]
             + [2.0 * 256 * 256 * K for _d in range(3) for K in (3, 7, 11) for _c in range(2)]
             + [2.0 * 4 * 128 * 256 * 4]
             + [2.0 * 128 * 128 * K for _d in range(3) for K in (3, 7, 11) for _c in range(2)]
             + [2.0 * 72 * 128 * 7])


def window_conv_gflop(lib, T, win, ctx_):
    """Conv work of ptd_decode_windows(T, win, ctx_) in GFLOP: (the columns it computes, every
    column of every window).  The schedule restates pt_decoder.c's win_schedule / win_plan_make:
    full-width windows run as one batched decode, other widths alone; each launch covers the
    columns ptd_window_cols names."""
    ws, a, emitted = [], 0, 0
    while emitted < T:
        w = min(win, T - a)
        last = a + w >= T
        lo, hi = (0 if a == 0 else ctx_), (w if last else w - ctx_)
        e0, e1 = max(a + lo, emitted), min(a + hi, T)
        ws.append((a, w, e0, e1))
        emitted = max(emitted, e1)
        if last:
            break
        a = max(e1 - ctx_, 1)
    full = [x for x in ws if x[1] == win]
    runs = [(x[1], 1, (x[2] - x[0], x[2] - x[0], x[3] - x[0], x[3] - x[0])) for x in ws if x[1] != win]
    if full:
        f0, fl = full[0], full[-1]
        runs.append((win, len(full), (f0[2] - f0[0], ctx_, win - ctx_, fl[3] - fl[0])))
    done = every = 0.0
    out = (C.c_int64 * (5 * 40))()
    for width, batch, (lo_first, lo, hi, hi_last) in runs:
        if lib.ptd_window_cols(width, batch, lo_first * HOP, lo * HOP, hi * HOP, hi_last * HOP, out) < 0:
            raise RuntimeError("ptd_window_cols failed")
        for i in range(40):
            q0, nq, el, er, shape = out[5 * i:5 * i + 5]
            cols = batch * nq + el + er
            done += _COL_FLOP[i] * cols
            every += _COL_FLOP[i] * batch * shape
    return done / 1e9, every / 1e9


def decode_conv_gflop(T):
    """Conv work of one full decode of T frames in GFLOP (every GEMM column)."""
    cols = [T, T + 1] + [4 * T] * 18 + [4 * T + 1] + [16 * T] * 18 + [16 * T + 1]
    return sum(f * c for f, c in zip(_COL_FLOP, cols)) / 1e9


_DECODER_KERNELS = ("conv_mfma_kernel", "avg3_leaky_kernel", "avg3_leaky4_kernel", "tail_kernel")
GRBM_XCDS, SIMDS = 8, 1024     # GRBM_GUI_ACTIVE sums the 8 XCDs; 256 CUs x 4 SIMDs


def _decodes(rows, batch):
    """Decoder dispatches (weight relayouts and copies excluded) in issue order, cut into decodes
    of 19, the warm-up decodes dropped."""
    rows = sorted(rows, key=lambda r: int(r["Dispatch_Id"]))
    ks = [r for r in rows if r["Kernel_Name"].removeprefix("void ").startswith(_DECODER_KERNELS)]
    n = len(DECODE_LAUNCHES)
    if len(ks) % n:
        raise SystemExit(f"{len(ks)} decoder dispatches is not a multiple of {n}")
    return [ks[i:i + n] for i in range(0, len(ks), n)][decode_loop_warm(batch):]


def _mfma_util(counter_csv, batch):
    """Per launch position: mean MFMA utilisation, SQ_VALU_MFMA_BUSY_CYCLES /
    (GRBM_GUI_ACTIVE / 8 XCDs x 1024 SIMDs) (rocprofv3's MfmaUtil), from a --pmc pass over the
    same decode loop."""
    import csv
    by = {}
    for r in csv.DictReader(open(counter_csv)):
        e = by.setdefault(r["Dispatch_Id"], {"Dispatch_Id": r["Dispatch_Id"], "Kernel_Name": r["Kernel_Name"]})
        e[r["Counter_Name"]] = float(r["Counter_Value"])
    dec = _decodes(list(by.values()), batch)
    out = []
    for i in range(len(DECODE_LAUNCHES)):
        u = [d[i]["SQ_VALU_MFMA_BUSY_CYCLES"] / (d[i]["GRBM_GUI_ACTIVE"] / GRBM_XCDS * SIMDS) for d in dec]
        out.append(100.0 * sum(u) / len(u))
    return out


def _kname(r):
    return r["Kernel_Name"].removeprefix("void ")


def queue_table(csv_path, steps, per_step=8 * 19):
    """Summary of the last `steps` steps of `bench.py --streams8-loop` from a rocprofv3 kernel
    trace (the last steps x per_step decoder dispatches by start time): busy share of the span,
    kernels in flight, kernel time per hardware queue (Queue_Id), and per kernel."""
    import collections
    import csv
    import statistics as st
    rows = [r for r in csv.DictReader(open(csv_path)) if _kname(r).startswith(_DECODER_KERNELS)]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    if len(rows) < steps * per_step:
        raise SystemExit(f"{len(rows)} decoder dispatches, fewer than {steps} steps of {per_step}")
    iv = [(int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r) for r in rows[-steps * per_step:]]
    t0, t1 = min(a for a, _, _ in iv), max(b for _, b, _ in iv)
    ev = sorted([(a, 1) for a, _, _ in iv] + [(b, -1) for _, b, _ in iv])
    inflight, k, prev = collections.Counter(), 0, ev[0][0]
    for t, d in ev:
        inflight[k] += t - prev
        k += d
        prev = t
    queue, qn, kinds = collections.Counter(), collections.Counter(), collections.defaultdict(list)
    for a, b, r in iv:
        queue[r["Queue_Id"]] += (b - a) / 1e3
        qn[r["Queue_Id"]] += 1
        kinds[_kname(r).split("(")[0]].append((b - a) / 1e3)
    span = (t1 - t0) / 1e3
    tot = sum(b - a for a, b, _ in iv) / 1e3
    out = [f"{steps} steps: {span / steps:.1f} us per step; kernels running {100 * (1 - inflight[0] / (t1 - t0)):.1f} % "
           f"of the span; {tot / span:.2f} kernels in flight on average",
           "in flight: " + ", ".join(f"{n}: {100 * v / (t1 - t0):.1f} %" for n, v in sorted(inflight.items())),
           "per hardware queue (kernel us per step, launches per step): "
           + ", ".join(f"{q}: {v / steps:.1f} us, {qn[q] / steps:.1f}" for q, v in sorted(queue.items()))]
    for name, v in sorted(kinds.items(), key=lambda x: -sum(x[1])):
        out.append(f"  {name}: {len(v) / steps:.1f} per step, mean {st.mean(v):.2f} us")
    return "\n".join(out)


def layer_table(csv_path, batch, counter_csv=None):
    """Per-launch table of `bench.py --decode-loop N --batch B` from a rocprofv3 kernel trace, each
    launch position averaged over the decodes after the warm-up; with a --pmc pass of
    SQ_VALU_MFMA_BUSY_CYCLES and GRBM_GUI_ACTIVE over the same loop, the MFMA utilisation too."""
    import csv
    rows = [r for r in csv.DictReader(open(csv_path)) if r.get("Kind", "KERNEL_DISPATCH") == "KERNEL_DISPATCH"]
    dec = _decodes(rows, batch)
    util = _mfma_util(counter_csv, batch) if counter_csv else None
    head = "| # | launch | kernel | us | rate | % of peak |" + (" MFMA util % |" if util else "")
    out = [f"{len(dec)} decodes of T = 226 x batch {batch} (after {decode_loop_warm(batch)} warm-up decodes)", "",
           head, "|---" * (7 if util else 6) + "|"]
    tot_us = tot_flop = 0.0
    for i, (name, kind, work) in enumerate(DECODE_LAUNCHES):
        names = {d[i]["Kernel_Name"] for d in dec}
        if len(names) != 1:
            raise SystemExit(f"launch {i} is not one kernel across decodes: {names}")
        us = sum(int(d[i]["End_Timestamp"]) - int(d[i]["Start_Timestamp"]) for d in dec) / len(dec) / 1e3
        kname = names.pop().replace("void ", "").split("(")[0]
        w = work * batch
        tot_us += us
        if kind == "flop":
            tot_flop += w
            rate = w / (us * 1e-6) / 1e12
            out.append(f"| {i} | {name} | `{kname}` | {us:.2f} | {rate:.1f} TFLOP/s | "
                       f"{100 * rate / MFMA_F32_PEAK:.1f} % fp32 MFMA |"
                       + (f" {util[i]:.1f} |" if util else ""))
        else:
            rate = w / (us * 1e-6) / 1e9
            out.append(f"| {i} | {name} | `{kname}` | {us:.2f} | {rate:.0f} GB/s | "
                       f"{100 * rate / HBM_PEAK:.1f} % HBM |" + (" - |" if util else ""))
    out += ["", f"sum of kernel times: {tot_us:.1f} us per decode; conv launches "
                f"{tot_flop / 1e9:.2f} GFLOP = {tot_flop / (tot_us * 1e-6) / 1e12:.1f} TFLOP/s over "
                f"the kernel time (gaps between launches excluded)"]
    return "\n".join(out)


def abi_leg(pkg, lib, ctx, model, ws, bs, T=226, reps=5):
    """Config 4's request through the reference ABI with host buffers (tests/abi_decoder.py: the
    decoder's 38 convs and 2 upsampling convTs as pt_v21_conv / pt_v21_convT calls on host arrays,
    driven the way the reference's interpreter drives the library), in three of the interpreter's
    modes: per call (every call copies its input up and its output back and waits), chained (the
    interpreter's default conv -> conv chains: c1 results stay on the device for c2) and resident
    (PT_V21_DEVADD: residual adds, LeakyReLUs and branch sums on device buffers as well).  Each
    request's wall time splits into the time inside library calls and the Python glue's between
    them.  The PCIe-inclusive per-call path, reported beside the value, never as it.  conv_post's
    output is compared with the device-resident decoder's (ptd_decode_stages) on the same
    latents."""
    sys.path.insert(0, str(ROOT / "tests"))
    import abi_decoder
    z = pkg.synth.latent(T, 77)
    pd = abi_decoder.device_conv_post(pkg, ctx, model, z)
    rms = np.sqrt(np.mean(pd.astype(np.float64) ** 2))
    out = {"frames": T, "path": "decoder convs / convTs through pt_v21_conv / pt_v21_convT on host "
                                "buffers (weights pool-resident, c1 + conv_pre LeakyReLU as "
                                "epilogue code 1, host glue in numpy); tail not included"}
    for mode in abi_decoder.MODES:
        run = abi_decoder.AbiDecoder(pkg, ctx, ws, bs, mode=mode)
        p = run.request(z)
        times, libs = [], []
        for _ in range(reps):
            l0 = run.lib_s
            t0 = time.perf_counter()
            run.request(z)
            times.append(time.perf_counter() - t0)
            libs.append(run.lib_s - l0)
        run.close()
        i = int(np.argsort(times)[len(times) // 2])   # the median request, split
        ms, lib_ms = times[i] * 1e3, libs[i] * 1e3
        rel = float(np.max(np.abs(p.astype(np.float64) - pd)) / rms)
        out[mode] = {"conv_calls": run.calls[0] // (reps + 1), "convT_calls": run.calls[1] // (reps + 1),
                     "ms_per_request": round(ms, 3), "library_ms": round(lib_ms, 3),
                     "glue_ms": round(ms - lib_ms, 3),
                     "audio_s_per_s": round(T * HOP / SR / (ms * 1e-3), 2),
                     "library_audio_s_per_s": round(T * HOP / SR / (lib_ms * 1e-3), 2),
                     "conv_post_vs_device_decoder_max_abs_over_rms": float(f"{rel:.3g}")}
    return out


# The drop-in path's narrow late stages, as the reference interpreter hands them to the library
# for a T = 226 request (ref/v21_graph_trace.txt:4265-4315): the PQMF synthesis FIR (/dec/Conv,
# 4 -> 1, K 63, over the 31|31-padded upsampled bands: 57918 input columns, 57856 outputs) through
# pt_v21_conv, and the iSTFT overlap-add (/dec/ConvTranspose, batch 4, 16 -> 1, K 16, s 4: 3617
# frames -> 14480 samples) through pt_v21_convT.  Both have cout4 = 4 output rows of which one is
# the channel and three are the layout's padding.
NARROW_FIR = dict(cin=4, T=57856 + 62, K=63, cout=1)
NARROW_OLA = dict(batch=4, cin=16, tin=3617, K=16, s=4, cout=1)


def narrow_abi_loop(pkg, lib, ctx, n):
    """n pt_v21_conv calls at the PQMF FIR's shape and n pt_v21_convT calls at the iSTFT
    overlap-add's, on host buffers (each call copies, launches the narrow kernel and waits), for a
    rocprofv3 kernel trace of the two narrow kernels."""
    f, o = NARROW_FIR, NARROW_OLA
    rng = np.random.default_rng(5)
    fp = pkg.fptr
    x = rng.standard_normal((f["cin"], f["T"])).astype(np.float32)
    tout = f["T"] - f["K"] + 1
    y = np.empty((4, tout), np.float32)
    w = pkg.synth.pack_conv((0.1 * rng.standard_normal((f["cout"], f["cin"], f["K"]))).astype(np.float32))
    b = np.zeros(f["cout"], np.float32)
    pad0 = ctx.get_i64("conv_pad_in")
    ctx.set_i64("conv_pad_in", 0)
    try:
        for _ in range(n):
            if lib.pt_v21_conv(ctx.ptr, fp(x), f["T"], f["cin"], fp(y), tout, tout, f["cout"], f["K"],
                               1, 0, 1, fp(w), fp(b), 1, -1, -1, 0, 0, 0.0, 0.0) != 0:
                raise RuntimeError("narrow conv failed")
    finally:
        ctx.set_i64("conv_pad_in", pad0)
    xo = rng.standard_normal((o["batch"], o["cin"], o["tin"])).astype(np.float32)
    lout = (o["tin"] - 1) * o["s"] + o["K"]
    yo = np.empty((o["batch"], 4, lout), np.float32)
    wo = pkg.synth.pack_convtranspose(
        (0.1 * rng.standard_normal((o["cin"], o["cout"], o["K"]))).astype(np.float32), o["s"])
    bo = np.zeros(o["cout"], np.float32)
    for _ in range(n):
        if lib.pt_v21_convT(ctx.ptr, fp(xo), o["tin"], o["cin"], o["tin"], fp(yo), lout, o["cout"],
                            o["s"], 0, o["K"], fp(wo), fp(bo), o["batch"], -1, -1) != 0:
            raise RuntimeError("narrow convT failed")
    log(f"kernel loop: {n} narrow ABI conv (PQMF FIR) and {n} convT (iSTFT OLA, batch 4) calls done")


def sndr_db(est, ref):
    """Signal to noise-and-distortion ratio of est against ref, in dB."""
    est = np.asarray(est, np.float64)
    ref = np.asarray(ref, np.float64)
    err = float(np.sum((est - ref) ** 2))
    return float("inf") if err == 0.0 else float(10.0 * np.log10(float(np.sum(ref ** 2)) / err))


def cpu_baseline(pkg, gpu_wavs=None, gpu_long=None, gpu_226=None):
    """The reference's own CPU conv path (oracle/_ref, built from the reference sources) inside the
    oracle's decoder driver, or the C restatement when _ref is absent.  Timed two ways: config 5's
    eight requests as eight host threads pinned to eight distinct cores (the reference's
    one-thread-per-stream model, main_v21_par.c:134-140), and one config-4 request on one thread.
    gpu_wavs: the same eight requests' waveforms from the timed GPU step, compared (SNDR) with the
    CPU ones.  gpu_long: the timed step's stitched long-form windows (T = 1500, 96/16), compared
    with one full decode of the same latents on the same CPU path, its conv nodes split over the
    host's threads (bit-identical to one thread; untimed).  gpu_226: a GPU waveform of
    the config-4 latents, compared with the single-thread decode."""
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib as ol
    ws, bs = pkg.synth.decoder_weights(1234)
    kind = "reference" if ol.have_ref() else "port"
    use_ref = kind == "reference"
    cores = sorted(os.sched_getaffinity(0))
    # eight requests of config 5 (the long-form request is left out of the CPU sample)
    Ts = pkg.synth.request_lengths(5, 8)
    zs = [pkg.synth.latent(T, 900 + i) for i, T in enumerate(Ts)]
    nthr = min(8, len(cores))
    cpu_wavs, dt8 = ol.decoder_threads(ws, bs, zs, cores[:nthr], use_ref=use_ref)
    audio8 = sum(Ts) * HOP / SR
    # one config-4 request on one thread
    T = 226
    z = pkg.synth.latent(T, 226)
    t0 = time.perf_counter()
    wav226 = ol.decoder(ws, bs, z, use_ref=use_ref)
    dt1 = time.perf_counter() - t0
    audio1 = T * HOP / SR
    layers = _cpu_layers(pkg, ol, ws, bs, use_ref, cores[0])
    mm = _cpu_matmul(ol) if use_ref else None
    long_db = None
    if gpu_long is not None:
        T_long = gpu_long.size // HOP
        ref_long = ol.decoder(ws, bs, pkg.synth.latent(T_long, 900 + 8), use_ref=use_ref,
                              threads=ol.host_threads())
        long_db = round(sndr_db(gpu_long, ref_long), 2)
    return {"value": round(audio8 / dt8, 4), "unit": "audio-s/s", "cores": nthr, "kind": kind,
            "sample": f"config 5's 8 requests (T={Ts}, {audio8:.2f} s audio; the T=1500 long-form "
                      f"request not included) as {nthr} threads pinned to cores {cores[:nthr]}: "
                      f"{dt8:.2f} s wall",
            "single_thread": {"value": round(audio1 / dt1, 4), "unit": "audio-s/s", "cores": 1,
                              "sample": f"one config-4 decode (T=226, {audio1:.3f} s audio) on 1 "
                                        f"thread: {dt1:.2f} s"},
            "configs_1_3_single_thread": layers,
            "matmul_us_per_call": mm,
            "host_cpus": len(cores), "nproc": os.cpu_count(), "model": _cpu_model(),
            # the same requests' waveforms from the timed GPU step against these CPU ones
            "sndr_vs_gpu_db": [round(sndr_db(g, c), 2) for g, c in zip(gpu_wavs, cpu_wavs)]
            if gpu_wavs is not None else None,
            "longform_sndr_vs_gpu_db": long_db,
            "config4_sndr_vs_gpu_db": round(sndr_db(gpu_226, wav226), 2) if gpu_226 is not None else None}


MATMUL_SHAPES = [(37, 53, 29), (120, 192, 120), (120, 96, 192)]   # m, k, n: encoder attention


def _cpu_matmul(ol):
    """The reference's CPU matmul (pt_v21_matmul_cpu) at the shapes the device matmul is timed on,
    on the calling thread: us per call."""
    out = {}
    for m_, k_, n_ in MATMUL_SHAPES:
        rngm = np.random.default_rng(m_ + k_ + n_)
        A = rngm.standard_normal((m_, k_)).astype(np.float32)
        B = rngm.standard_normal((k_, n_)).astype(np.float32)
        Cm = np.zeros((m_, n_), np.float32)
        ol.ref_matmul(A, m_, k_, k_, B, n_, n_, Cm, n_)
        t0 = time.perf_counter()
        for _ in range(50):
            ol.ref_matmul(A, m_, k_, k_, B, n_, n_, Cm, n_)
        out[f"{m_}x{k_}x{n_}"] = round((time.perf_counter() - t0) / 50 * 1e6, 1)
    return out


def _cpu_layers(pkg, ol, ws, bs, use_ref, core):
    """Configs 1-3 through the same CPU conv path on one thread pinned to one core, with the
    weights and inputs the GPU legs of configs 1-3 use.  The LeakyReLU in front of config 2's
    convT and the MRF glue run inside the timed region as the host ops they are in the
    reference's interpreter."""
    lib = ol.ref() if use_ref else None
    z = pkg.synth.latent(226, 226)
    prev = os.sched_getaffinity(0)
    os.sched_setaffinity(0, {core})
    try:
        out = {}
        t0 = time.perf_counter()
        h = ol.conv(z, ws[0], bs[0], 512, 7, 1, 3, 1, epi0=1, a0=0.1, lib=lib)
        dt = time.perf_counter() - t0
        out["config1_conv_gflops"] = round(2 * 512 * 192 * 7 * 226 / dt / 1e9, 3)
        t0 = time.perf_counter()
        hl = np.where(h >= 0, h, np.float32(0.1) * h).astype(np.float32)
        ol.convT(hl, ws[1], bs[1], 256, 16, 4, 6, lib=lib)
        dt = time.perf_counter() - t0
        out["config2_convT_gflops"] = round(2 * 256 * 512 * 4 * 904 / dt / 1e9, 3)
        for first, (C_, T) in ((2, (256, 904)), (21, (128, 3616))):
            x = np.random.default_rng(5).standard_normal((C_, T)).astype(np.float32)
            t0 = time.perf_counter()
            ol.mrf(ws[first:first + 18], bs[first:first + 18], x, 0.1, use_ref=use_ref)
            dt = time.perf_counter() - t0
            out[f"config3_mrf{C_}_gflops"] = round(2 * C_ * C_ * T * 126 / dt / 1e9, 3)
    finally:
        os.sched_setaffinity(0, prev)
    out["cores"] = 1
    out["core"] = core
    return out


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def streams8_leg(pkg, lib, ctx, model, args, steps=None):
    """Config 4's request shape on 8 concurrent streams: 8 contexts of a ptd_server, each driven by
    its own pthread, one T = 226 decode each (the latents of the batch-8 leg), after 60 ms of the
    same.  Returns the figures, whether every stream's waveform equals the batched decode's item
    bit for bit, and stream 0's waveform (the config-4 latents)."""
    T, n = 226, 8
    zs = [pkg.synth.latent(T, 226 + i) for i in range(n)]
    dz = [pkg.DevBuf.of(ctx, z) for z in zs]
    dw = [pkg.DevBuf(HOP * T) for _ in range(n)]
    reqs = (pkg.Request * n)(*[pkg.Request(dz[i].ptr, dw[i].ptr, T, 0, 0) for i in range(n)])
    srv = lib.ptd_server_create(n, int(lib.ptd_decode_arena_bytes(T, 1)) + (16 << 20))
    if not srv:
        raise RuntimeError("ptd_server_create failed")
    wall = C.c_double()

    def step():
        if lib.ptd_serve_run(srv, model.ptr, reqs, n, C.byref(wall)) != 0:
            raise RuntimeError("serve run failed")
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < WARM_MS:
        step()
    lib.ptd_device_sync()
    steps = steps or max(args.steps, 20)
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    lib.ptd_device_sync()
    ms = (time.perf_counter() - t0) / steps * 1e3
    lib.ptd_server_destroy(srv)
    wavs = [b.download(ctx) for b in dw]
    db = pkg.DevBuf.of(ctx, np.concatenate(zs))
    wb = pkg.DevBuf(n * HOP * T)
    if lib.ptd_decode(ctx.ptr, model.ptr, db.ptr, T, n, wb.ptr) != 0:
        raise RuntimeError("batched decode failed")
    batched = wb.download(ctx).reshape(n, -1)
    same = all(np.array_equal(wavs[i], batched[i]) for i in range(n))
    for b in dz + dw + [db, wb]:
        b.free()
    return ({"config4_8streams_ms_per_step": round(ms, 4),
             "config4_8streams_audio_s_per_s": round(n * T * HOP / SR / (ms * 1e-3), 2),
             "config4_8streams_decoder_tflops": round(n * 32.571e9 / (ms * 1e-3) / 1e12, 3),
             "equal_batched_decode": same}, wavs[0])


def queue_leg(pkg, lib, model, zs, wv, Ts, T_long, arena, args):
    """Config 5's requests through ptd_queue (all submitted at the start of a step, long-form
    last, deadline = submission time): step wall time, the long-form job's time to first audio
    (its 48-frame first window complete) and every request's latency, medians over the steps."""
    WF, WIN, CTX = 48, 96, 16
    arena = max(arena, int(lib.ptd_windows2_arena_bytes(T_long, WF, WIN, CTX)))
    q = lib.ptd_queue_create(model.ptr, len(Ts) + 1, arena, 64)
    if not q:
        raise RuntimeError("ptd_queue_create failed")
    jobs = [pkg.Job(zs[i].ptr, wv[i].ptr, T, 0, 0, 0, 0.0) for i, T in enumerate(Ts)]
    jobs.append(pkg.Job(zs[-1].ptr, wv[-1].ptr, T_long, WF, WIN, CTX, 0.0))
    walls, ttfa, lat = [], [], []

    def step():
        ids = []
        for j in jobs:
            j.deadline_ms = lib.ptd_now_ms()
            ids.append(lib.ptd_queue_submit(q, C.byref(j)))
            if ids[-1] < 0:
                raise RuntimeError("ptd_queue_submit refused a job")
        sts = []
        for i in ids:
            st = pkg.JobStatus()
            if lib.ptd_queue_wait(q, i, C.byref(st)) != 0 or st.rc != 0:
                raise RuntimeError("queue job failed")
            sts.append(st)
        t0 = min(st.t_submit for st in sts)
        return (max(st.t_end for st in sts) - t0, sts[-1].t_first - sts[-1].t_submit,
                [st.t_end - st.t_submit for st in sts[:-1]])

    try:
        for _ in range(args.warmup):
            step()
        for _ in range(args.steps):
            w, f, l8 = step()
            walls.append(w)
            ttfa.append(f)
            lat.extend(l8)
        # the long-form job alone on an idle queue: its first window without the load
        alone = []
        for _ in range(5):
            jl = jobs[-1]
            jl.deadline_ms = lib.ptd_now_ms()
            i = lib.ptd_queue_submit(q, C.byref(jl))
            st = pkg.JobStatus()
            if i < 0 or lib.ptd_queue_wait(q, i, C.byref(st)) != 0 or st.rc != 0:
                raise RuntimeError("queue job failed")
            alone.append(st.t_first - st.t_submit)
    finally:
        lib.ptd_queue_destroy(q)
    audio = (sum(Ts) + T_long) * HOP / SR
    med = lambda xs: float(np.median(xs))
    return {"workers": len(Ts) + 1, "longform_windows": f"{WF} then {WIN}, ctx {CTX}",
            "ms_per_step": round(med(walls), 4), "audio_s_per_s": round(audio / (med(walls) / 1e3), 2),
            "longform_first_audio_ms": round(med(ttfa), 4), "longform_first_audio_max_ms": round(max(ttfa), 4),
            "longform_first_audio_idle_ms": round(med(alone), 4),
            "request_latency_ms": {"median": round(med(lat), 4), "max": round(max(lat), 4)}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-loop", type=int, default=0)
    ap.add_argument("--decode-loop", type=int, default=0)
    ap.add_argument("--streams8-loop", type=int, default=0)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--layer-table", metavar="KERNEL_TRACE_CSV")
    ap.add_argument("--queue-table", metavar="KERNEL_TRACE_CSV")
    ap.add_argument("--counters", metavar="COUNTER_COLLECTION_CSV")
    args = ap.parse_args()
    if args.layer_table:
        print(layer_table(args.layer_table, args.batch, args.counters))
        return
    if args.queue_table:
        print(queue_table(args.queue_table, args.steps))
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the decoder path would shard by request, with no exchange between GPUs)", file=sys.stderr)
        sys.exit(2)

    pkg = _package()
    lib = pkg.load()
    ctx = pkg.Ctx(arena_mb=1024)
    ws, bs = pkg.synth.decoder_weights(1234)
    model = pkg.Model(ctx, ws, bs)
    timer = EventTimer(pkg, ctx)

    if args.decode_loop:
        # config 4 decodes (T = 226, `--batch` requests per decode), eager, for a kernel trace
        B = args.batch
        dz = pkg.DevBuf.of(ctx, np.stack([pkg.synth.latent(226, 226 + i) for i in range(B)]))
        dw = pkg.DevBuf(B * HOP * 226)
        for _ in range(decode_loop_warm(B) + args.decode_loop):
            if lib.ptd_decode(ctx.ptr, model.ptr, dz.ptr, 226, B, dw.ptr) != 0:
                raise RuntimeError("decode failed")
        ctx.sync()
        log(f"decode loop: {decode_loop_warm(B)} + {args.decode_loop} decodes of T 226 x {B} done")
        return

    if args.streams8_loop:
        fig, _ = streams8_leg(pkg, lib, ctx, model, args, steps=args.streams8_loop)
        log(f"8-stream loop: {args.streams8_loop} steps after the warm-up: {fig}")
        return

    # ---------------------------------------------------------------- dominant kernel
    # one MRF-256 depth at config 3 (C=256, T=904): two grouped conv launches of 3 branches each
    flop_launch = 2.0 * 256 * 256 * 904 * (3 + 7 + 11)
    bufs, xin, xinl, a_s, ys = mrf_depth_setup(pkg, ctx, 0, 904)
    run_depth = lambda: lib.ptd_mrf_depth(ctx.ptr, model.ptr, 0, 2, xin, xinl, a_s, ys, None, 904)  # noqa: E731
    if args.kernel_loop:
        N = args.kernel_loop
        # the narrow late stages too: the fused tail kernel at config 4's shape, N launches of one
        # request and N of 64 requests at once (256- and 1024-sample tiles); buffers made first, so
        # the loops below run back to back
        tails = [(tb,) + tuple(tail_setup(pkg, ctx, TAIL_L, tb)) for tb in (1, 64)]
        tail_call = lambda tb, tp, tw: lib.ptd_tail(ctx.ptr, model.ptr, tp.ptr, TAIL_L, tb, tw.ptr)  # noqa: E731
        # the clock first: WARM_MS of the batch-64 tail, a kernel of its own, so that every conv
        # dispatch of a trace of this loop is a measured one (an elementwise add of the same
        # length did not bring the clock up for the MFMA launches: 27.5 us per conv launch after
        # it, 24.8 after the tail, 24.3 after the conv itself)
        timer.warm(lambda: tail_call(*tails[1]))
        for _ in range(N):
            if run_depth() != 0:
                raise RuntimeError("mrf depth failed")
        for tb, tp, tw in tails:
            for _ in range(N):
                if tail_call(tb, tp, tw) != 0:
                    raise RuntimeError("tail failed")
        ctx.sync()
        for _, tp, tw in tails:
            tp.free(); tw.free()
        log(f"kernel loop: {WARM_MS:.0f} ms of the batch-64 tail, then {2 * N} conv launches, "
            f"{N} tail launches of batch 1 and {N} of batch 64 done")
        narrow_abi_loop(pkg, lib, ctx, args.kernel_loop)
        # calibration for the HBM byte counters: the elementwise add over 64 Mi floats (aligned
        # buffers: add4_kernel, four per thread) reads exactly 512 MiB and writes 256 MiB per launch
        n = 64 << 20
        a, b2, y = pkg.DevBuf(n), pkg.DevBuf(n), pkg.DevBuf(n)
        for _ in range(5):
            if lib.pt_v21_devadd_run(ctx.ptr, a.ptr, b2.ptr, y.ptr, n, 0, 0.0) != 0:
                raise RuntimeError("calibration add failed")
        ctx.sync()
        log("calibration: 5 add4_kernel launches of 64 Mi floats (read 524288 KiB, write 262144 KiB)")
        return
    ms_depth = timer.time(run_depth, 50)
    ms_launch = ms_depth / 2.0
    achieved = flop_launch / (ms_launch * 1e-3) / 1e12
    # algorithmic bytes of one launch (c1 group): 3 inputs + weights + biases + 3 outputs
    bytes_launch = 4.0 * (3 * 256 * 904 + 256 * 256 * (3 + 7 + 11) + 3 * 256 + 3 * 256 * 904)
    log(f"dominant kernel: MRF-256 grouped conv {ms_launch * 1e3:.1f} us/launch = {achieved:.2f} TFLOP/s")
    # ~1 ms of GPU work (20 residual units, ~0.16 ms to issue) queued ahead of the timed calls of
    # the short launches below
    block = lambda: [run_depth() for _ in range(20)]  # noqa: E731

    # ---------------------------------------------------------------- narrow late stages (GB/s)
    tail = {}
    for batch in (1, 8, 64):
        tp, tw = tail_setup(pkg, ctx, TAIL_L, batch)
        ft = lambda: lib.ptd_tail(ctx.ptr, model.ptr, tp.ptr, TAIL_L, batch, tw.ptr)  # noqa: E731
        ft()
        ms = timer.time(ft, 50, blocker=block)
        tail[f"batch{batch}"] = {"us": round(ms * 1e3, 2),
                                 "gbps": round(tail_bytes(TAIL_L, batch) / (ms * 1e-3) / 1e9, 1)}
        tp.free(); tw.free()
    log(f"tail kernel (iSTFT + PQMF, L {TAIL_L}): {tail}")

    # ---------------------------------------------------------------- configs 1-3 (TFLOP/s)
    cfg = {}
    z226 = pkg.synth.latent(226, 226)
    dz = pkg.DevBuf.of(ctx, z226)
    dh = pkg.DevBuf(512 * 226)
    # single launches: 20 untimed calls first, so the timed 100 run at the clock a sustained
    # stream of them gets (the first tens of launches of a layer run a few % slower)
    f1 = lambda: lib.ptd_layer(ctx.ptr, model.ptr, 0, dz.ptr, 226, 1, dh.ptr, 0.0, 0.1)  # noqa: E731
    ms = timer.time(f1, 100, warmup=20, blocker=block)
    cfg["config1_conv_tflops"] = round(2 * 512 * 192 * 7 * 226 / (ms * 1e-3) / 1e12, 3)
    cfg["config1_frac"] = round(cfg["config1_conv_tflops"] / MFMA_F32_PEAK, 4)
    dx0 = pkg.DevBuf(256 * 904)
    f2 = lambda: lib.ptd_layer(ctx.ptr, model.ptr, 1, dh.ptr, 226, 1, dx0.ptr, 0.1, 0.0)  # noqa: E731
    ms = timer.time(f2, 100, warmup=20, blocker=block)
    cfg["config2_convT_tflops"] = round(2 * 256 * 512 * 4 * 904 / (ms * 1e-3) / 1e12, 3)
    cfg["config2_frac"] = round(cfg["config2_convT_tflops"] / MFMA_F32_PEAK, 4)
    ctx.sync()
    for b in bufs:      # the dominant launch's buffers, last used by the blocker
        b.free()
    for stage, (C_, T) in enumerate([(256, 904), (128, 3616)]):
        x = pkg.DevBuf.of(ctx, np.random.default_rng(5).standard_normal((C_, T)).astype(np.float32))
        y = pkg.DevBuf(C_ * T)
        f3 = lambda: lib.ptd_mrf(ctx.ptr, model.ptr, stage, x.ptr, T, 0.1, y.ptr)  # noqa: E731
        ms = timer.time(f3, 20, warmup=3)
        # 3 dilations x (c1 + c2) x branches K 3 + 7 + 11 = 126 tap-weighted convs of C x C
        cfg[f"config3_mrf{C_}_tflops"] = round(2 * C_ * C_ * T * 126 / (ms * 1e-3) / 1e12, 3)
        cfg[f"config3_mrf{C_}_frac"] = round(cfg[f"config3_mrf{C_}_tflops"] / MFMA_F32_PEAK, 4)
        x.free()
        y.free()
    # config 4: one request, one stream
    dw = pkg.DevBuf(HOP * 226)
    f4 = lambda: lib.ptd_decode(ctx.ptr, model.ptr, dz.ptr, 226, 1, dw.ptr)  # noqa: E731
    for _ in range(3):
        f4()
    ms4 = timer.time(f4, 20)
    cfg["config4_ms_per_request"] = round(ms4, 4)
    cfg["config4_audio_s_per_s_1stream"] = round(226 * HOP / SR / (ms4 * 1e-3), 2)
    cfg["config4_decoder_tflops"] = round(32.571e9 / (ms4 * 1e-3) / 1e12, 3)
    # the same request captured once as a HIP graph and replayed (a serving loop that reuses its
    # buffers): its 19 launches go to the device as one submission
    graph = lib.ptd_decode_graph(ctx.ptr, model.ptr, dz.ptr, 226, 1, dw.ptr)
    if not graph:
        raise RuntimeError("ptd_decode_graph failed")
    f4g = lambda: lib.ptd_graph_launch(ctx.ptr, graph)  # noqa: E731
    for _ in range(3):
        f4g()
    ms4g = timer.time(f4g, 20)
    lib.ptd_graph_destroy(graph)
    cfg["config4_graph_ms_per_request"] = round(ms4g, 4)
    cfg["config4_graph_audio_s_per_s_1stream"] = round(226 * HOP / SR / (ms4g * 1e-3), 2)
    # the same request shape eight at a time in one batched decode (one stream): the kernels at
    # fuller occupancy than one request gives them
    z8 = pkg.DevBuf.of(ctx, np.concatenate([pkg.synth.latent(226, 226 + i) for i in range(8)]))
    w8 = pkg.DevBuf(8 * HOP * 226)
    f48 = lambda: lib.ptd_decode(ctx.ptr, model.ptr, z8.ptr, 226, 8, w8.ptr)  # noqa: E731
    for _ in range(2):
        f48()
    ms48 = timer.time(f48, 10)
    cfg["config4_batch8_ms"] = round(ms48, 4)
    cfg["config4_batch8_decoder_tflops"] = round(8 * 32.571e9 / (ms48 * 1e-3) / 1e12, 3)
    z8.free()
    w8.free()
    for b in (dz, dh, dx0, dw):
        b.free()
    log(f"configs: {cfg}")
    # config 4's request through the reference ABI on host buffers (the drop-in path)
    abi = abi_leg(pkg, lib, ctx, model, ws, bs)
    log(f"abi path: {abi}")

    # ---------------------------------------------------------------- the container path and the
    # matmul entry point (the last two scope rows): the decoder's records written as the
    # reference's exporter writes them (fp16 layers), then opened, parsed, uploaded as fp16,
    # expanded and relaid on the device; and pt_v21_matmul at the encoder's attention shapes with
    # host buffers, as the reference's interpreter calls it
    sys.path.insert(0, str(ROOT / "tests"))
    import tempfile
    import ptk_writer as pw
    with tempfile.TemporaryDirectory() as td:
        path = pathlib.Path(td) / "decoder.ptk"
        pw.write(path, pw.decoder_tensors(ws, bs, half=True))
        size = path.stat().st_size
        t0 = time.perf_counter()
        ptk = pkg.Ptk(path)
        t1 = time.perf_counter()
        model2 = pkg.Model.from_ptk(ctx, ptk)
        ctx.sync()
        t2 = time.perf_counter()
        nrec = int(lib.ptd_ptk_count(ptk.ptr))
        ptk.close()
        model2.close()
    container = {"file_mb": round(size / 1e6, 3), "records": nrec,
                 "open_parse_ms": round((t1 - t0) * 1e3, 2),
                 "model_create_ms": round((t2 - t1) * 1e3, 2),
                 "total_ms": round((t2 - t0) * 1e3, 2)}
    log(f"container load: {container}")
    mm = {}
    for m_, k_, n_ in MATMUL_SHAPES:
        rngm = np.random.default_rng(m_ + k_ + n_)
        A = rngm.standard_normal((m_, k_)).astype(np.float32)
        B = rngm.standard_normal((k_, n_)).astype(np.float32)
        Cm = np.zeros((m_, n_), np.float32)
        fmm = lambda: lib.pt_v21_matmul(ctx.ptr, pkg.fptr(A), m_, k_, k_, pkg.fptr(B), n_, n_,  # noqa: E731
                                        pkg.fptr(Cm), n_)
        for _ in range(3):
            if fmm() != 0:
                raise RuntimeError("pt_v21_matmul failed")
        t0 = time.perf_counter()
        for _ in range(50):
            fmm()
        mm[f"{m_}x{k_}x{n_}"] = round((time.perf_counter() - t0) / 50 * 1e6, 1)
    log(f"pt_v21_matmul us per call (host buffers): {mm}")

    # ---------------------------------------------------------------- streaming (config 5's
    # long-form request on one stream): the first 96-frame window alone (time to first audio),
    # every window one at a time as the reference's --stream driver issues them, and the batched
    # windowed decode
    T_long, WIN, CTX = 1500, 96, 16
    zl = pkg.DevBuf.of(ctx, pkg.synth.latent(T_long, 900 + 8))
    pcm, wl = pkg.DevBuf(HOP * WIN), pkg.DevBuf(HOP * T_long)
    nout = C.c_int64()
    starts = list(range(0, T_long, WIN - 2 * CTX))
    starts = starts[:next(i for i, a in enumerate(starts) if a + WIN >= T_long) + 1]

    def chunk(a):
        if lib.ptd_decode_chunk(ctx.ptr, model.ptr, zl.ptr, T_long, a, WIN, pcm.ptr, C.byref(nout)) != 0:
            raise RuntimeError("chunk decode failed")

    def all_chunks():
        for a in starts:
            chunk(a)

    def batched():
        if lib.ptd_decode_windows(ctx.ptr, model.ptr, zl.ptr, T_long, WIN, CTX, wl.ptr) != 0:
            raise RuntimeError("windowed decode failed")

    for f in (all_chunks, batched):
        f()
    stream = {"frames": T_long, "win": WIN, "ctx": CTX, "windows": len(starts),
              "first_chunk_ms": round(timer.time(lambda: chunk(0), 20), 4),
              "chunked_total_ms": round(timer.time(all_chunks, 5), 4),
              "batched_windows_ms": round(timer.time(batched, 10), 4)}
    stream["audio_s"] = round(T_long * HOP / SR, 4)
    # each window computes only the columns its kept samples depend on (ptd_window_cols)
    g_done, g_all = window_conv_gflop(lib, T_long, WIN, CTX)
    stream["batched_windows_conv_gflop"] = {"computed": round(g_done, 2), "all_columns": round(g_all, 2)}
    stream["batched_windows_tflops"] = round(g_done / stream["batched_windows_ms"], 2)
    for b in (zl, pcm, wl):
        b.free()
    log(f"streaming: {stream}")

    # ---------------------------------------------------------------- config 5: the timed step
    Ts = pkg.synth.request_lengths(5, 8)
    T_long = 1500
    zs = [pkg.DevBuf.of(ctx, pkg.synth.latent(T, 900 + i)) for i, T in enumerate(Ts + [T_long])]
    wv = [pkg.DevBuf(HOP * T) for T in Ts + [T_long]]
    reqs = [pkg.Request(zs[i].ptr, wv[i].ptr, T, 0, 0) for i, T in enumerate(Ts)]
    reqs.append(pkg.Request(zs[-1].ptr, wv[-1].ptr, T_long, 96, 16))
    req_arr = (pkg.Request * len(reqs))(*reqs)
    arena = max(int(lib.ptd_decode_arena_bytes(max(Ts), 1)),
                int(lib.ptd_windows_arena_bytes(T_long, 96, 16))) + (64 << 20)
    srv = lib.ptd_server_create(len(reqs), arena)
    if not srv:
        raise RuntimeError("ptd_server_create failed")
    wall = C.c_double()
    for _ in range(args.warmup):
        if lib.ptd_serve_run(srv, model.ptr, req_arr, len(reqs), C.byref(wall)) != 0:
            raise RuntimeError("serve run failed")
    lib.ptd_device_sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        if lib.ptd_serve_run(srv, model.ptr, req_arr, len(reqs), C.byref(wall)) != 0:
            raise RuntimeError("serve run failed")
    lib.ptd_device_sync()
    dt = time.perf_counter() - t0
    audio_step = sum(Ts + [T_long]) * HOP / SR
    value = audio_step * args.steps / dt
    audio8 = sum(Ts) * HOP / SR
    log(f"config 5: {value:.1f} audio-s/s ({dt / args.steps * 1e3:.2f} ms/step)")
    # conv work of one step as computed: 8 full decodes + the windowed long-form request
    step_gflop = sum(decode_conv_gflop(T) for T in Ts) + window_conv_gflop(lib, T_long, 96, 16)[0]
    # the timed step's own outputs (after the timed region): the eight requests are compared with
    # the reference's CPU path in the cpu_baseline leg, the long-form windows with one full
    # (unwindowed) decode of the same latents
    c5_wavs = [b.download(ctx) for b in wv]
    dfull = pkg.DevBuf(HOP * T_long)
    if lib.ptd_decode(ctx.ptr, model.ptr, zs[-1].ptr, T_long, 1, dfull.ptr) != 0:
        raise RuntimeError("full long-form decode failed")
    parity = {"gate_db": 60.0,
              "config5_longform_windows_vs_full_decode_sndr_db": round(sndr_db(c5_wavs[-1], dfull.download(ctx)), 2)}
    dfull.free()
    lib.ptd_server_destroy(srv)

    # ---------------------------------------------------------------- config 5 through the queue
    # The same nine requests submitted to the queue-fed server (ptd_queue: 9 persistent workers,
    # earliest-deadline-first, deadline = arrival time), the long-form request as a streaming job
    # with the reference's short first window (48 frames, then 96-frame windows, 16 of context).
    # Reported beside the value, not in it: time to first audio under this load, per-request
    # latency, and the throughput of the queue path.
    queue = queue_leg(pkg, lib, model, zs, wv, Ts, T_long, arena, args)
    log(f"queue: {queue}")
    for b in zs + wv:
        b.free()
    # the north star's own case: the T = 226 request on 8 concurrent streams (made after config
    # 5's, so that leg's streams land on the hardware queues they always did)
    streams8, c4_wav0 = streams8_leg(pkg, lib, ctx, model, args)
    parity["config4_8streams_equal_batched_decode"] = streams8.pop("equal_batched_decode")
    log(f"config 4 on 8 streams: {streams8}")
    cfg.update(streams8)

    out = {
        "metric": "decoder audio-sec/sec at 8 streams (+ conv TFLOP/s, % fp32-MFMA peak)",
        "value": round(value, 2),
        "unit": "audio-s/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded random-init decoder weights, N(0,1) latents)",
        "config": {
            "workload": "config 5: 8 concurrent MB-iSTFT decoder requests (T ~ U[56,400], seed 5) "
                        "on 8 HIP streams + one T=1500 request in 96/16 overlap-save windows, "
                        "one shared weight set",
            "request_frames": Ts, "longform_frames": T_long, "audio_s_per_step": round(audio_step, 4),
            "audio_s_8_requests": round(audio8, 4), "parallelism": "1 GPU, 9 streams",
            "step_conv_gflop": round(step_gflop, 2),
            "step_conv_tflops": round(step_gflop / (dt / args.steps * 1e3), 2),
            "io": "latents and waveforms device-resident in the timed step (uploaded before it, "
                  "read back after it)",
        },
        "roofline": {
            "kernel": "conv_mfma_kernel (MRF-256 grouped launch: 3 branch convs K 3/7/11, C 256, T 904)",
            "bound": "mfma", "achieved": round(achieved, 3), "peak": MFMA_F32_PEAK,
            "unit": "TFLOP/s", "frac": round(achieved / MFMA_F32_PEAK, 4),
            "traffic": measured_traffic(),
            "traffic_source": str(PROFILE_DOMINANT.relative_to(ROOT)),
            "flop_per_launch": flop_launch, "alg_bytes_per_launch": bytes_launch,
            "us_per_launch": round(ms_launch * 1e3, 3),
        },
        "abi_path": abi,
        "narrow_stages": {
            "kernel": f"tail_kernel (iSTFT + PQMF synthesis fused; conv_post output [72][{TAIL_L}] "
                      f"-> {16 * (TAIL_L - 1)} samples per request)",
            "bound": "hbm", "peak_gbps": HBM_PEAK,
            "alg_bytes_per_request": tail_bytes(TAIL_L, 1), **tail,
        },
        "streaming": stream,
        "serving_queue": queue,
        "container_load": container,
        "matmul_us_per_call": mm,
        **cfg,
    }
    out["parity"] = parity
    if not args.no_cpu_baseline:
        log("cpu baseline (reference conv path: 8 pinned threads, then 1 thread for config 4 and configs 1-3) ...")
        out["cpu_baseline"] = cpu_baseline(pkg, c5_wavs[:8], c5_wavs[-1], c4_wav0)
        parity["config4_8streams_vs_reference_cpu_sndr_db"] = out["cpu_baseline"].pop("config4_sndr_vs_gpu_db")
        snd = out["cpu_baseline"].pop("sndr_vs_gpu_db")
        parity["config5_requests_vs_reference_cpu_sndr_db"] = {"min": min(snd), "per_request": snd}
        parity["config5_longform_windows_vs_reference_cpu_full_decode_sndr_db"] = \
            out["cpu_baseline"].pop("longform_sndr_vs_gpu_db")
    log(f"parity: {parity}")
    timer.close()
    model.close()
    ctx.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
