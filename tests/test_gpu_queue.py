"""GPU tests of the queue-fed server (ptd_queue_*) and of the reference's streaming window schedule
(ptd_decode_windows2), through the C ABI.

- The batched two-width schedule equals the reference's streaming loop (main_v21_serve.c:219-257:
  first window 48 frames, then 256, 16 frames of context) run one window at a time through
  ptd_decode_chunk and stitched the way that loop keeps samples, bit for bit, and stays >= 60 dB
  from one full decode.
- Jobs held back and released together are taken earliest-deadline-first, equal deadlines in
  submission order (main_v21_serve.c:129-160), and each output equals its single decode.
- Jobs submitted while others run, on several workers, plain and streaming, each equal their
  single decode bit for bit; a streaming job's first audio is complete before its end.
- A full queue and a job larger than the workers' arenas are refused; destroying the queue runs
  what is still queued."""
from __future__ import annotations

import ctypes as C
import sys
import time

import numpy as np
import pytest

import np_ref
from conftest import load_package

pkg = load_package()
synth = pkg.synth
pytestmark = pytest.mark.gpu
HOP = 256


def say(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def env():
    ctx = pkg.Ctx(arena_mb=1024)
    ws, bs = synth.decoder_weights(1234)
    model = pkg.Model(ctx, ws, bs)
    yield ctx, model
    model.close()
    ctx.close()


def _decode(ctx, model, z):
    T = z.shape[-1]
    dz, dw = pkg.DevBuf.of(ctx, z), pkg.DevBuf(HOP * T)
    assert ctx.lib.ptd_decode(ctx.ptr, model.ptr, dz.ptr, T, 1, dw.ptr) == 0
    out = dw.download(ctx)
    dz.free(); dw.free()
    return out


def _stream_loop(ctx, model, z, win_first, win, cx):
    """The reference's synth_stream loop (main_v21_serve.c:219-257), one window at a time, with
    its widths raised to at least 2*ctx + 8 (:223-224)."""
    lib = ctx.lib
    T = z.shape[-1]
    win_first, win = max(win_first, 2 * cx + 8), max(win, 2 * cx + 8)
    dz = pkg.DevBuf.of(ctx, z)
    pcm = pkg.DevBuf(HOP * max(win_first, win))
    n = C.c_int64()
    out = np.full(HOP * T, np.nan, np.float32)
    a = emitted = 0
    while emitted < T:
        w = win_first if a == 0 else win
        weff = min(w, T - a)
        last = a + weff >= T
        assert lib.ptd_decode_chunk(ctx.ptr, model.ptr, dz.ptr, T, a, weff, pcm.ptr, C.byref(n)) == 0
        p = pcm.download(ctx, n.value)
        lo = 0 if a == 0 else cx
        hi = weff if last else weff - cx
        e0, e1 = max(a + lo, emitted), min(a + hi, T)
        if e1 > e0:
            out[e0 * HOP:e1 * HOP] = p[(e0 - a) * HOP:(e1 - a) * HOP]
            emitted = e1
        if last:
            break
        a = max(e1 - cx, 1)
    dz.free(); pcm.free()
    return out


@pytest.mark.parametrize("T,wf,w,cx", [(1500, 48, 256, 16), (300, 48, 256, 16), (200, 48, 96, 16),
                                       (40, 48, 256, 16), (600, 96, 96, 16), (260, 48, 256, 16),
                                       (300, 36, 96, 16), (200, 36, 36, 16)])
def test_windows2_matches_the_reference_stream_loop(env, T, wf, w, cx):
    ctx, model = env
    lib = ctx.lib
    say(f"windows2 T={T} first {wf} then {w} ctx {cx}")
    z = synth.latent(T, 7000 + T)
    ref = _stream_loop(ctx, model, z, wf, w, cx)
    assert np.all(np.isfinite(ref))
    assert lib.ptd_windows2_arena_bytes(T, wf, w, cx) <= 1024 << 20
    dz, dw = pkg.DevBuf.of(ctx, z), pkg.DevBuf(HOP * T)
    dw.upload(ctx, np.full(HOP * T, np.nan, np.float32))
    assert lib.ptd_debug_fill_arena(ctx.ptr, 0xFF) == 0   # columns never written read as NaN
    assert lib.ptd_decode_windows2(ctx.ptr, model.ptr, dz.ptr, T, wf, w, cx, dw.ptr) == 0
    got = dw.download(ctx)
    dz.free(); dw.free()
    assert np.array_equal(got, ref)
    if T >= 200:
        assert np_ref.sndr(got, _decode(ctx, model, z)) >= 60.0


def _jobs(ctx, specs):
    """specs: (T, seed, win_first, win, ctx, deadline) -> (device buffers, Job structs)"""
    bufs, jobs = [], []
    for T, seed, wf, w, cx, dl in specs:
        dz, dw = pkg.DevBuf.of(ctx, synth.latent(T, seed)), pkg.DevBuf(HOP * T)
        dw.upload(ctx, np.full(HOP * T, np.nan, np.float32))
        bufs.append((dz, dw))
        jobs.append(pkg.Job(dz.ptr, dw.ptr, T, wf, w, cx, dl))
    return bufs, jobs


def _expected(ctx, model, spec):
    T, seed, wf, w, cx, _ = spec
    z = synth.latent(T, seed)
    if w == 0:
        return _decode(ctx, model, z)
    dz, dw = pkg.DevBuf.of(ctx, z), pkg.DevBuf(HOP * T)
    assert ctx.lib.ptd_decode_windows2(ctx.ptr, model.ptr, dz.ptr, T, wf, w, cx, dw.ptr) == 0
    out = dw.download(ctx)
    dz.free(); dw.free()
    return out


def test_queue_pops_earliest_deadline_first(env):
    ctx, model = env
    lib = ctx.lib
    say("queue EDF order (1 worker, held)")
    q = lib.ptd_queue_create(model.ptr, 1, 256 << 20, 16)
    assert q
    deadlines = [5.0, 1.0, 3.0, 1.0, 2.0, 0.5, 3.0]
    specs = [(40 + 7 * i, 300 + i, 0, 0, 0, d) for i, d in enumerate(deadlines)]
    specs[2] = (120, 302, 48, 96, 16, 3.0)   # one streaming job among them
    bufs, jobs = _jobs(ctx, specs)
    try:
        lib.ptd_queue_hold(q, 1)
        ids = [lib.ptd_queue_submit(q, C.byref(j)) for j in jobs]
        assert all(i >= 0 for i in ids) and len(set(ids)) == len(ids)
        time.sleep(0.05)
        st = pkg.JobStatus()
        assert lib.ptd_queue_poll(q, ids[0], C.byref(st)) == 0   # held: nothing taken yet
        lib.ptd_queue_hold(q, 0)
        stats = []
        for i in ids:
            s = pkg.JobStatus()
            assert lib.ptd_queue_wait(q, i, C.byref(s)) == 0
            stats.append(s)
        assert all(s.rc == 0 and s.worker == 0 for s in stats)
        want = sorted(range(len(deadlines)), key=lambda k: (deadlines[k], k))
        got = sorted(range(len(deadlines)), key=lambda k: stats[k].order)
        assert got == want, (got, want)
        for k, spec in enumerate(specs):
            assert np.array_equal(bufs[k][1].download(ctx), _expected(ctx, model, spec)), k
        assert lib.ptd_queue_poll(q, ids[0], C.byref(st)) == -1   # consumed by the wait
    finally:
        lib.ptd_queue_destroy(q)
        for dz, dw in bufs:
            dz.free(); dw.free()


def test_queue_staggered_submissions(env):
    ctx, model = env
    lib = ctx.lib
    say("queue: staggered submissions on 4 workers")
    q = lib.ptd_queue_create(model.ptr, 4, 512 << 20, 64)
    assert q
    Ts = synth.request_lengths(11, 10)
    specs = []
    for i, T in enumerate(Ts):
        if i % 3 == 2:
            specs.append((T + 300, 500 + i, 48, 256, 16, float(i)))   # streaming
        else:
            specs.append((T, 500 + i, 0, 0, 0, float(i)))
    bufs, jobs = _jobs(ctx, specs)
    try:
        ids = []
        for k, j in enumerate(jobs):
            ids.append(lib.ptd_queue_submit(q, C.byref(j)))
            assert ids[-1] >= 0
            if k in (3, 6):
                time.sleep(0.002)   # later jobs arrive while the first ones run
        done = {}
        t_end = time.time() + 60
        while len(done) < len(ids) and time.time() < t_end:
            for k, i in enumerate(ids):
                if k in done:
                    continue
                s = pkg.JobStatus()
                r = lib.ptd_queue_poll(q, i, C.byref(s))
                assert r in (0, 1)
                if r == 1:
                    done[k] = s
            time.sleep(0.001)
        assert len(done) == len(ids)
        assert {s.worker for s in done.values()} <= {0, 1, 2, 3}
        for k, spec in enumerate(specs):
            s = done[k]
            assert s.rc == 0
            assert s.t_submit <= s.t_start <= s.t_first <= s.t_end
            if spec[3] > 0:
                assert s.t_first < s.t_end
            assert np.array_equal(bufs[k][1].download(ctx), _expected(ctx, model, spec)), k
    finally:
        lib.ptd_queue_destroy(q)
        for dz, dw in bufs:
            dz.free(); dw.free()


@pytest.mark.parametrize("parts_env", [("PTD_WINDOW_PARTS", "4"), ("PTD_WINDOW_STREAMS", "1"),
                                       ("PTD_WINDOW_STREAMS", "2")])
def test_queue_window_split_beyond_prepared_streams(env, parts_env, knob_env):
    """The queue makes each worker's extra stream for the default two-part split when it is
    created.  A split in four parts asked for afterwards makes the two more streams it needs on
    first use. Keeping every run on one stream, or splitting every run in two, works on the same
    prepared workers.  Each output equals the one-stream windowed decode bit for bit."""
    ctx, model = env
    lib = ctx.lib
    T, seed, wf, w, cx = 2600, 77, 48, 96, 16   # 39 full windows: four parts of at least 8
    say(f"queue: window split with {parts_env[0]}={parts_env[1]} after the queue is made")
    knob_env.delenv("PTD_WINDOW_PARTS", raising=False)
    knob_env.delenv("PTD_WINDOW_STREAMS", raising=False)
    arena = int(lib.ptd_windows2_arena_bytes(T, wf, w, cx)) + (16 << 20)
    knob_env.setenv("PTD_WINDOW_STREAMS", "1")
    ref = _expected(ctx, model, (T, seed, wf, w, cx, 0.0))
    knob_env.delenv("PTD_WINDOW_STREAMS")
    q = lib.ptd_queue_create(model.ptr, 2, arena, 8)
    assert q
    knob_env.setenv(*parts_env)
    bufs, jobs = _jobs(ctx, [(T, seed, wf, w, cx, 0.0), (T, seed, wf, w, cx, 1.0)])
    try:
        ids = [lib.ptd_queue_submit(q, C.byref(j)) for j in jobs]
        assert min(ids) >= 0
        for k, i in enumerate(ids):
            s = pkg.JobStatus()
            assert lib.ptd_queue_wait(q, i, C.byref(s)) == 0 and s.rc == 0
            assert np.array_equal(bufs[k][1].download(ctx), ref), k
    finally:
        lib.ptd_queue_destroy(q)
        for dz, dw in bufs:
            dz.free(); dw.free()


def test_queue_refusals_and_drain_on_destroy(env):
    ctx, model = env
    lib = ctx.lib
    say("queue: capacity, arena refusal, drain on destroy")
    q = lib.ptd_queue_create(model.ptr, 1, 64 << 20, 2)
    assert q
    specs = [(50, 800, 0, 0, 0, 1.0), (60, 801, 0, 0, 0, 2.0), (70, 802, 0, 0, 0, 3.0)]
    bufs, jobs = _jobs(ctx, specs)
    big = pkg.DevBuf(192 * 2000)
    bigw = pkg.DevBuf(HOP * 2000)
    try:
        lib.ptd_queue_hold(q, 1)
        a = lib.ptd_queue_submit(q, C.byref(jobs[0]))
        b = lib.ptd_queue_submit(q, C.byref(jobs[1]))
        assert a >= 0 and b >= 0
        assert lib.ptd_queue_submit(q, C.byref(jobs[2])) == -1      # capacity 2
        too_big = pkg.Job(big.ptr, bigw.ptr, 2000, 0, 0, 0, 0.0)      # needs > 64 MiB of arena
        assert lib.ptd_queue_submit(q, C.byref(too_big)) == -1
        bad = pkg.Job(big.ptr, bigw.ptr, 100, 48, 20, 16, 0.0)        # window < 2*ctx + 1
        assert lib.ptd_queue_submit(q, C.byref(bad)) == -1
        lib.ptd_queue_hold(q, 0)
        assert lib.ptd_queue_wait(q, a, None) == 0
        c = lib.ptd_queue_submit(q, C.byref(jobs[2]))                 # a slot is free again
        assert c >= 0
        lib.ptd_queue_hold(q, 1)
    finally:
        lib.ptd_queue_destroy(q)   # runs what is still queued, then joins
    for k, spec in enumerate(specs):
        assert np.array_equal(bufs[k][1].download(ctx), _expected(ctx, model, spec)), k
    for dz, dw in bufs:
        dz.free(); dw.free()
    big.free(); bigw.free()
