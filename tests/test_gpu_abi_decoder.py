"""The decoder driven through the reference's device ABI on host buffers (tests/abi_decoder.py: the
38 convs and 2 upsampling convTs as pt_v21_conv / pt_v21_convT calls, weights pool-resident, the
LeakyReLU after conv_pre and each c1 as epilogue code 1, host glue in numpy), the way the
reference's graph interpreter drives the library.  Its conv_post output must meet the per-layer
bar against the oracle's decoder (which runs the reference's own CPU conv loops over the same
graph) and against the device-resident decoder, and the waveform the tail makes of it the
end-to-end bar.  The interpreter's chained mode (c1 -> c2 kept on the device through conv_keep /
conv_in_dev) and its PT_V21_DEVADD residency (residual adds, LeakyReLUs and branch sums through
pt_v21_devadd_run / pt_v21_devleaky_run on device buffers) give the same bits as the per-call
mode: the same kernels sum in the same order, and the device Add and LeakyReLU are the same fp32
operations as the host's."""
from __future__ import annotations

import sys

import numpy as np
import pytest

import abi_decoder
import np_ref
import oracle_lib as ol
from conftest import load_package

pkg = load_package()
synth = pkg.synth
TOL = 1e-4
pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu abi] {msg}", flush=True)
    sys.stdout.flush()


def relerr(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.sqrt(np.mean(b ** 2)), 1e-30))


@pytest.fixture(scope="module")
def env():
    ctx = pkg.Ctx(arena_mb=256)
    ws, bs = synth.decoder_weights(2024)
    model = pkg.Model(ctx, ws, bs)
    run = abi_decoder.AbiDecoder(pkg, ctx, ws, bs)
    yield ctx, model, ws, bs, run
    run.close()
    model.close()
    ctx.close()


@pytest.mark.parametrize("T", [9, 40])
def test_abi_decoder_vs_oracle(env, T):
    """conv_post through the ABI within 1e-4 x RMS of the oracle's; the tail of it (ptd_tail) at
    >= 60 dB from the oracle's waveform; the call counts are the graph's."""
    ctx, model, ws, bs, run = env
    say(f"ABI-driven decoder vs oracle, T={T}")
    z = synth.latent(T, 600 + T)
    c0 = list(run.calls)
    p = run.request(z)
    assert [run.calls[0] - c0[0], run.calls[1] - c0[1]] == [38, 2]
    wav_ref, st = ol.decoder(ws, bs, z, stages=True)
    L = 16 * T + 1
    assert relerr(p, st[5].reshape(72, L)) < TOL
    dp, dw = pkg.DevBuf.of(ctx, p), pkg.DevBuf(16 * (L - 1))
    assert ctx.lib.ptd_tail(ctx.ptr, model.ptr, dp.ptr, L, 1, dw.ptr) == 0
    wav = dw.download(ctx)
    dp.free(); dw.free()
    assert np_ref.sndr(wav, wav_ref) >= 60.0


def test_abi_decoder_vs_device_decoder_T226(env):
    """At config 4's size: the ABI-driven conv_post against the device-resident decoder's
    (ptd_decode_stages) on the same latents, within 1e-4 x RMS; the ABI path is repeatable bit
    for bit."""
    ctx, model, ws, bs, run = env
    say("ABI-driven decoder vs device-resident decoder, T=226")
    z = synth.latent(226, 3)
    p = run.request(z)
    pd = abi_decoder.device_conv_post(pkg, ctx, model, z)
    assert relerr(p, pd) < TOL
    assert np.array_equal(run.request(z), p)


@pytest.mark.parametrize("mode", ["chained", "resident"])
def test_abi_decoder_modes_match_per_call(env, mode):
    ctx, model, ws, bs, run = env
    say(f"ABI-driven decoder, {mode} mode, vs per-call mode")
    other = abi_decoder.AbiDecoder(pkg, ctx, ws, bs, mode=mode)
    try:
        for T in (40, 226):
            z = synth.latent(T, 700 + T)
            ref = run.request(z)
            c0 = list(other.calls)
            got = other.request(z)
            assert [other.calls[0] - c0[0], other.calls[1] - c0[1]] == [38, 2]
            assert np.array_equal(got, ref), f"T={T}"
            assert np.array_equal(other.request(z), ref), f"T={T} repeated"
    finally:
        other.close()
