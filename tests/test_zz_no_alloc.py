"""ptd_decode_noalloc (the decode whose activations live in the library's static device scratch,
for callers that cannot allocate) against ptd_decode, through the C ABI.

Two calls in a row on one context, the second with a smaller input (so the scratch still holds
the first call's larger contents), each bit-identical to ptd_decode of the same input; a batched
call likewise; and decodes that need more than the scratch's 64 MiB are refused before anything
is queued.  The output buffers are filled with NaN first, so every compared sample was written.

That it allocates nothing: with every device allocation of the library made to fail
(ptd_debug_fail_allocs) and on a context whose 1 MiB arena cannot hold the decode, it still
decodes bit-identically.  That calls on different contexts are ordered on the GPU: two contexts
call it one right after the other, with no host synchronisation, and each output is right.  That
it can be captured: one call recorded into a HIP graph on the context's stream (the library's
capture helpers) and replayed three times, with eager calls on other inputs in between, gives
ptd_decode's bits every time."""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np
import pytest

from conftest import load_package

pkg = load_package()
synth = pkg.synth
pytestmark = pytest.mark.gpu
SCRATCH_BYTES = 64 << 20


def say(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def env():
    ctx = pkg.Ctx(arena_mb=256)
    ws, bs = synth.decoder_weights(1234)
    model = pkg.Model(ctx, ws, bs)
    yield ctx, model
    model.close()
    ctx.close()


def _run(ctx, model, fn, z, batch=1):
    T = z.shape[-1]
    dz = pkg.DevBuf.of(ctx, z)
    dw = pkg.DevBuf(256 * T * batch)
    dw.upload(ctx, np.full(256 * T * batch, np.nan, np.float32))
    rc = fn(ctx.ptr, model.ptr, dz.ptr, T, batch, dw.ptr)
    out = dw.download(ctx) if rc == 0 else None
    dz.free(); dw.free()
    return rc, out


def test_noalloc_decode_matches_decode(env):
    ctx, model = env
    lib = ctx.lib
    for T, seed in ((226, 41), (57, 42)):   # the second call smaller than the first
        say(f"ptd_decode_noalloc T={T}")
        z = synth.latent(T, seed)
        rc0, ref = _run(ctx, model, lib.ptd_decode, z)
        rc1, out = _run(ctx, model, lib.ptd_decode_noalloc, z)
        assert rc0 == 0 and rc1 == 0
        assert np.all(np.isfinite(out))
        assert np.array_equal(out, ref), f"T={T}"


def test_noalloc_batched_matches_decode(env):
    ctx, model = env
    lib = ctx.lib
    T, batch = 100, 3
    say(f"ptd_decode_noalloc T={T} batch {batch}")
    z = np.stack([synth.latent(T, 50 + i) for i in range(batch)])
    rc0, ref = _run(ctx, model, lib.ptd_decode, z, batch)
    rc1, out = _run(ctx, model, lib.ptd_decode_noalloc, z, batch)
    assert rc0 == 0 and rc1 == 0
    assert np.array_equal(out, ref)


def test_noalloc_refuses_decodes_above_the_scratch(env):
    ctx, model = env
    lib = ctx.lib
    say("ptd_decode_noalloc size limit")
    t_max = max(T for T in range(1, 2000) if lib.ptd_decode_arena_bytes(T, 1) <= SCRATCH_BYTES)
    assert t_max >= 400    # config 5's longest request fits
    # refused on the host before anything is queued: these never reach the device
    for T, batch in ((t_max + 1, 1), (1500, 1), (226, 2)):
        assert lib.ptd_decode_arena_bytes(T, batch) > SCRATCH_BYTES
        dz = pkg.DevBuf(192 * T * batch)
        dw = pkg.DevBuf(256 * T * batch)
        assert lib.ptd_decode_noalloc(ctx.ptr, model.ptr, dz.ptr, T, batch, dw.ptr) == -1
        dz.free(); dw.free()
    # the largest accepted size decodes like ptd_decode
    z = synth.latent(t_max, 43)
    rc0, ref = _run(ctx, model, lib.ptd_decode, z)
    rc1, out = _run(ctx, model, lib.ptd_decode_noalloc, z)
    assert rc0 == 0 and rc1 == 0 and np.array_equal(out, ref)


def test_noalloc_allocates_nothing(env):
    ctx, model = env
    lib = ctx.lib
    T = 226
    say("ptd_decode_noalloc with every device allocation failing, on a 1 MiB arena")
    z = synth.latent(T, 61)
    rc0, ref = _run(ctx, model, lib.ptd_decode, z)
    assert rc0 == 0
    small = pkg.Ctx(arena_mb=1)
    dz, dw = pkg.DevBuf.of(small, z), pkg.DevBuf(256 * T)
    try:
        assert lib.ptd_decode_arena_bytes(T, 1) > (1 << 20)
        lib.ptd_debug_fail_allocs(0, 1 << 30)
        try:
            assert lib.ptd_decode(small.ptr, model.ptr, dz.ptr, T, 1, dw.ptr) == -1   # arena too small
            for _ in range(2):
                dw.upload(small, np.full(256 * T, np.nan, np.float32))
                assert lib.ptd_decode_noalloc(small.ptr, model.ptr, dz.ptr, T, 1, dw.ptr) == 0
                assert np.array_equal(dw.download(small), ref)
        finally:
            lib.ptd_debug_fail_allocs(0, 0)
    finally:
        dz.free(); dw.free()
        small.close()


def test_noalloc_calls_on_two_contexts_are_ordered(env):
    ctx, model = env
    lib = ctx.lib
    say("ptd_decode_noalloc on two contexts, back to back without synchronising")
    other = pkg.Ctx(arena_mb=64)
    cases = [(400, 71), (150, 72), (300, 73), (57, 74)]
    refs = [_run(ctx, model, lib.ptd_decode, synth.latent(T, seed))[1] for T, seed in cases]
    bufs = []
    try:
        for T, seed in cases:
            dz, dw = pkg.DevBuf.of(ctx, synth.latent(T, seed)), pkg.DevBuf(256 * T)
            dw.upload(ctx, np.full(256 * T, np.nan, np.float32))
            bufs.append((dz, dw))
        for rep in range(2):
            for i, (T, _) in enumerate(cases):   # alternate contexts; nothing waits on the host
                c = ctx if i % 2 == 0 else other
                dz, dw = bufs[i]
                assert lib.ptd_decode_noalloc(c.ptr, model.ptr, dz.ptr, T, 1, dw.ptr) == 0
            ctx.sync()
            other.sync()
            for i, (T, _) in enumerate(cases):
                assert np.array_equal(bufs[i][1].download(ctx), refs[i]), f"rep {rep} case {i}"
    finally:
        for dz, dw in bufs:
            dz.free(); dw.free()
        other.close()


def test_noalloc_decode_captured_and_replayed(env):
    ctx, model = env
    lib = ctx.lib
    lib.ptk_capture_begin.argtypes = [C.c_void_p]
    lib.ptk_capture_end.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
    lib.ptk_graph_launch.argtypes = [C.c_void_p, C.c_void_p]
    lib.ptk_graph_destroy.argtypes = [C.c_void_p]
    T = 180
    say(f"ptd_decode_noalloc captured on the context's stream, T={T}")
    z = synth.latent(T, 81)
    rc0, ref = _run(ctx, model, lib.ptd_decode, z)
    assert rc0 == 0
    zo = synth.latent(90, 82)
    rco, ref_o = _run(ctx, model, lib.ptd_decode, zo)
    assert rco == 0
    stream = ctx.get_ptr("g_stream")
    dz, dw = pkg.DevBuf.of(ctx, z), pkg.DevBuf(256 * T)
    exe = C.c_void_p()
    try:
        assert lib.ptk_capture_begin(stream) == 0
        rc = lib.ptd_decode_noalloc(ctx.ptr, model.ptr, dz.ptr, T, 1, dw.ptr)
        assert lib.ptk_capture_end(stream, C.byref(exe) if rc == 0 else None) == 0
        assert rc == 0 and exe.value
        for rep in range(3):
            dw.upload(ctx, np.full(256 * T, np.nan, np.float32))
            assert lib.ptk_graph_launch(exe, stream) == 0
            ctx.sync()
            assert np.array_equal(dw.download(ctx), ref), f"replay {rep}"
            rc1, out = _run(ctx, model, lib.ptd_decode_noalloc, zo)   # eager, other input
            assert rc1 == 0 and np.array_equal(out, ref_o)
    finally:
        if exe.value:
            ctx.sync()
            lib.ptk_graph_destroy(exe)
        dz.free(); dw.free()
