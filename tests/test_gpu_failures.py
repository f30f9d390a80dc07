"""Error paths, forced from the host: a device allocation that fails (the library's own injector,
ptd_debug_fail_allocs), an arena too small for the call, a graph whose scratch cannot be had.
Every failure here happens on the host before anything is launched; each test checks that the
call reports it (-1 / NULL), leaves nothing half-built, and that the same context then works and
gives the right answer.  The reference's contract (pt_v21_cuda.cu:1782-1801): a full arena falls
back to an owned allocation; a failed allocation is an error return, never a crash."""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np
import pytest

import np_ref
import oracle_lib as ol
from conftest import load_package

pytestmark = pytest.mark.gpu
pkg = load_package()
synth = pkg.synth
TOL = 1e-4


def say(msg):
    print(f"[gpu failures] {msg}", file=sys.stderr, flush=True)


@pytest.fixture(autouse=True)
def _injector_off():
    yield
    pkg.load().ptd_debug_fail_allocs(0, 0)


def relerr(a, b):
    return float(np.max(np.abs(a - b)) / (np.sqrt(np.mean(b.astype(np.float64) ** 2)) + 1e-30))


def conv_rc(ctx, x, wp, bias, cout, K, pad, dil):
    """pt_v21_conv with unpadded rows (conv_pad_in = pad); returns (rc, y)."""
    B, cin, T = x.shape
    Tout = T + 2 * pad - (K - 1) * dil
    c4 = (cout + 3) // 4 * 4
    ctx.set_i64("conv_pad_in", pad)
    y = np.full((B, c4, Tout), np.nan, np.float32)
    rc = ctx.lib.pt_v21_conv(ctx.ptr, pkg.fptr(x), T, cin, pkg.fptr(y), Tout, Tout, cout, K, 1, pad,
                             dil, pkg.fptr(wp), pkg.fptr(bias), B, -1, -1, 0, 0, 0.0, 0.0)
    return rc, y


def _mrf_case(seed=5):
    rng = np.random.default_rng(seed)
    C_, T, K, d = 256, 904, 3, 5
    x = rng.standard_normal((1, C_, T)).astype(np.float32)
    W = (rng.standard_normal((C_, C_, K)) / np.sqrt(C_ * K)).astype(np.float32)
    b = (0.1 * rng.standard_normal(C_)).astype(np.float32)
    wp = np.ascontiguousarray(synth.pack_conv(W))
    ref = ol.conv(x, wp, b, C_, K, 1, d * (K - 1) // 2, d, 0, 0, 0.0, 0.0)
    return x, wp, b, C_, K, d, ref


def test_context_init_allocation_failure():
    """pt_v21_cuda_init reports a failed arena allocation and leaves no stream behind; the next
    init works."""
    say("context init with a failing arena allocation")
    lib = pkg.load()
    lib.ptd_debug_fail_allocs(0, 1)
    with pytest.raises(RuntimeError):
        pkg.Ctx(arena_mb=64)
    lib.ptd_debug_fail_allocs(0, 0)
    ctx = pkg.Ctx(arena_mb=64)
    assert ctx.get_int("use_cuda") == 1
    ctx.close()


def test_conv_full_arena_falls_back_to_owned_memory():
    """An arena too small for the operands: pt_v21_conv takes owned allocations instead and the
    result is unchanged (the reference's fallback, pt_v21_cuda.cu:1782-1793)."""
    say("conv through a 1 MiB arena")
    x, wp, b, C_, K, d, ref = _mrf_case()
    ctx = pkg.Ctx(arena_mb=1)
    try:
        rc, y = conv_rc(ctx, x, wp, b, C_, K, d * (K - 1) // 2, d)
        assert rc == 0
        assert relerr(y[:, :C_], ref) < TOL
    finally:
        ctx.close()


@pytest.mark.parametrize("skip", [0, 1, 2])
def test_conv_owned_allocation_failure_is_an_error(skip):
    """With the arena full, the first, second or third owned allocation of a conv fails: the call
    returns -1, frees what it took, and the same context then computes the conv correctly."""
    say(f"conv owned allocation failure after {skip}")
    x, wp, b, C_, K, d, ref = _mrf_case()
    ctx = pkg.Ctx(arena_mb=1)
    try:
        ctx.lib.ptd_debug_fail_allocs(skip, 1)
        rc, _ = conv_rc(ctx, x, wp, b, C_, K, d * (K - 1) // 2, d)
        assert rc == -1
        ctx.lib.ptd_debug_fail_allocs(0, 0)
        rc, y = conv_rc(ctx, x, wp, b, C_, K, d * (K - 1) // 2, d)
        assert rc == 0
        assert relerr(y[:, :C_], ref) < TOL
    finally:
        ctx.close()


@pytest.fixture(scope="module")
def env():
    ctx = pkg.Ctx(arena_mb=256)
    ws, bs = synth.decoder_weights(1234)
    model = pkg.Model(ctx, ws, bs)
    yield ctx, model, ws, bs
    model.close()
    ctx.close()


def _decode(ctx, model, z, T, batch=1):
    dz, dw = pkg.DevBuf.of(ctx, z), pkg.DevBuf(batch * 256 * T)
    try:
        rc = ctx.lib.ptd_decode(ctx.ptr, model.ptr, dz.ptr, T, batch, dw.ptr)
        return rc, (dw.download(ctx) if rc == 0 else None)
    finally:
        dz.free()
        dw.free()


@pytest.mark.parametrize("skip", [0, 1])
def test_model_create_allocation_failure(env, skip):
    """ptd_model_create with its weight slab or its staging buffer allocation failing (an fp32
    model takes those two) returns NULL; the next model builds."""
    ctx, model, ws, bs = env
    say(f"model create failing after {skip}")
    ctx.lib.ptd_debug_fail_allocs(skip, 1)
    with pytest.raises(RuntimeError):
        pkg.Model(ctx, ws, bs)
    ctx.lib.ptd_debug_fail_allocs(0, 0)
    m2 = pkg.Model(ctx, ws, bs)
    m2.close()


def test_decode_arena_too_small_then_recovers(env):
    """A decode larger than the context's arena is refused with -1 before anything is queued
    (ptd_decode_arena_bytes is checked up front); a decode that fits then runs on the same
    context, bit-identical to the same decode before."""
    ctx, model, ws, bs = env
    say("decode larger than the arena")
    T_big = 2500
    assert ctx.lib.ptd_decode_arena_bytes(T_big, 1) > 256 << 20
    z_small = synth.latent(100, 100)
    rc, before = _decode(ctx, model, z_small, 100)
    assert rc == 0
    rc, _ = _decode(ctx, model, synth.latent(T_big, 7), T_big)
    assert rc == -1
    rc, after = _decode(ctx, model, z_small, 100)
    assert rc == 0
    assert np.array_equal(before, after)
    assert np_ref.sndr(after, ol.decoder(ws, bs, z_small)) >= 60.0


def test_graph_scratch_allocation_failure(env):
    """ptd_decode_graph whose scratch allocation fails returns NULL without leaving the stream in
    capture; eager decodes and a later graph on the same context work."""
    ctx, model, ws, bs = env
    say("graph scratch allocation failure")
    T = 64
    z = synth.latent(T, 64)
    dz, dw = pkg.DevBuf.of(ctx, z), pkg.DevBuf(256 * T)
    try:
        ctx.lib.ptd_debug_fail_allocs(0, 1)
        assert not ctx.lib.ptd_decode_graph(ctx.ptr, model.ptr, dz.ptr, T, 1, dw.ptr)
        ctx.lib.ptd_debug_fail_allocs(0, 0)
        rc, eager = _decode(ctx, model, z, T)
        assert rc == 0
        g = ctx.lib.ptd_decode_graph(ctx.ptr, model.ptr, dz.ptr, T, 1, dw.ptr)
        assert g
        try:
            assert ctx.lib.ptd_graph_launch(ctx.ptr, g) == 0
            assert np.array_equal(dw.download(ctx), eager)
        finally:
            ctx.lib.ptd_graph_destroy(g)
    finally:
        dz.free()
        dw.free()


def test_server_partial_creation_failure(env):
    """ptd_server_create whose third context cannot get its arena returns NULL and tears down the
    two it built; a server created next serves requests correctly."""
    ctx, model, ws, bs = env
    say("server creation failing at the third context")
    lib = ctx.lib
    arena = int(lib.ptd_decode_arena_bytes(120, 1)) + (16 << 20)
    lib.ptd_debug_fail_allocs(2, 1)
    assert not lib.ptd_server_create(4, arena)
    lib.ptd_debug_fail_allocs(0, 0)
    srv = lib.ptd_server_create(2, arena)
    assert srv
    try:
        Ts = [120, 77]
        zs = [synth.latent(T, 300 + T) for T in Ts]
        dz = [pkg.DevBuf.of(ctx, z) for z in zs]
        dw = [pkg.DevBuf(256 * T) for T in Ts]
        reqs = (pkg.Request * 2)(*[pkg.Request(dz[i].ptr, dw[i].ptr, T, 0, 0) for i, T in enumerate(Ts)])
        wall = C.c_double()
        assert lib.ptd_serve_run(srv, model.ptr, reqs, 2, C.byref(wall)) == 0
        for i, T in enumerate(Ts):
            rc, single = _decode(ctx, model, zs[i], T)
            assert rc == 0
            assert np.array_equal(dw[i].download(ctx), single)
        for b in dz + dw:
            b.free()
    finally:
        lib.ptd_server_destroy(srv)
