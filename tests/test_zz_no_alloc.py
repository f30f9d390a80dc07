"""ptd_decode_noalloc (the decode whose activations live in the library's static device scratch,
for callers that cannot allocate) against ptd_decode, through the C ABI.

Two calls in a row on one context, the second with a smaller input (so the scratch still holds
the first call's larger contents), each bit-identical to ptd_decode of the same input; a batched
call likewise; and decodes that need more than the scratch's 64 MiB are refused before anything
is queued.  The output buffers are filled with NaN first, so every compared sample was written."""
from __future__ import annotations

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
