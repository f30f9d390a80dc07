"""The device-resident decoder against the reference's own graph interpreter and streaming driver.

The synthetic full model of tests/full_model.py is written as a .ptk container, read by the
library's container reader (ptd_ptk_open) and turned into a device model (ptd_model_create_ptk,
fp16 records expanded on the device).  ptd_decode_stages then decodes the latents the reference's
CPU driver fed its decoder, and each stage and the waveform are compared with what that driver
computed (tests/golden/ref_decoder_ckpt.npz at T = 35 and ref_decoder_ckpt_T198.npz at T = 198,
written by tests/golden/gen_decoder_ckpt.py through the driver's checkpoint option,
main_v21.c:218-219, :307-321).

The overlap-save windows are compared with the waveforms the same driver stitched in its
`--stream WIN CTX` mode (main_v21.c:331-370 over pt_v21_stream_chunk, pt_v21_host.c:2866-2902):
ptd_decode_windows (one batched decode), ptd_decode_windows2 with equal widths, and
ptd_decode_chunk window by window stitched by the driver's loop.

Bars: per stage max |err| <= 1e-4 x RMS; waveform >= 60 dB SNDR.
Since the 96/16 stream sits only 77 dB from the full decode, the windows must also be at least
20 dB closer to the stream than to the full decode."""
from __future__ import annotations

import ctypes as C
import pathlib
import sys

import numpy as np
import pytest

import full_model as fm
import np_ref
import oracle_lib as ol
from conftest import load_package

pkg = load_package()
GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
FIXTURES = {"T35": GOLDEN / "ref_decoder_ckpt.npz", "T198": GOLDEN / "ref_decoder_ckpt_T198.npz"}
STAGES = ["stage0", "stage1", "stage2", "stage3", "stage4", "stage5"]
pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


def relerr(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.max(np.abs(a - b)) / max(np.sqrt(np.mean(b ** 2)), 1e-30))


def stage_relerr(g, k, got) -> float:
    """max |err| / RMS against the reference's stage k: the whole array where the fixture stores
    it, else its stored samples against the whole stage's RMS."""
    got = np.asarray(got, np.float64).ravel()
    if k in g.files:
        return relerr(got, g[k])
    d = np.max(np.abs(got[g[k + "_idx"]] - g[k + "_val"].astype(np.float64)))
    return float(d / max(float(g[k + "_rms"]), 1e-30))


def _decode_stages(ctx, model, z):
    T = z.shape[-1]
    dz = pkg.DevBuf.of(ctx, z)
    dw = pkg.DevBuf(256 * T)
    lens = [512 * T, 1024 * T, 1024 * T, 2048 * T, 2048 * T, 72 * (16 * T + 1)]
    sb = [pkg.DevBuf(n) for n in lens]
    arr = (C.c_void_p * 6)(*[b.ptr for b in sb])
    try:
        assert ctx.lib.ptd_decode_stages(ctx.ptr, model.ptr, dz.ptr, T, dw.ptr, arr) == 0
        return dw.download(ctx), [b.download(ctx) for b in sb]
    finally:
        dz.free(); dw.free()
        for b in sb:
            b.free()


@pytest.fixture(scope="module", params=list(FIXTURES))
def ptk_model(request, tmp_path_factory):
    """The container model of the fixture's seed on the device, the fixture, and the same layers
    as arrays."""
    g = np.load(FIXTURES[request.param])
    path = tmp_path_factory.mktemp("ptk") / "model.ptk"
    fm.write_container(path, seed=int(g["container_seed"]))
    f = pkg.Ptk(path)
    ctx = pkg.Ctx(arena_mb=512)
    m = None
    try:
        assert f.check_decoder()
        m = pkg.Model.from_ptk(ctx, f)
        f.close()
        yield ctx, m, g
    finally:
        if m is not None:
            m.close()
        f.close()
        ctx.close()


def test_container_decoder_matches_reference_interpreter(ptk_model):
    ctx, m_ptk, g = ptk_model
    T = g["z"].shape[-1]
    say(f"container model vs the reference interpreter's checkpoints, T = {T}")
    wav, st = _decode_stages(ctx, m_ptk, g["z"])
    for i, k in enumerate(STAGES):
        e = stage_relerr(g, k, st[i])
        say(f"  {k}: max|err|/rms = {e:.3g}")
        assert e <= 1e-4, k
    s = np_ref.sndr(wav, g["wav"])
    say(f"  waveform SNDR {s:.1f} dB")
    assert s >= 60.0
    # the same layers handed over as arrays give the same bits
    ws, bs = fm.decoder_layers(int(g["container_seed"]))
    m_arr = pkg.Model(ctx, ws, bs)
    try:
        wav2, st2 = _decode_stages(ctx, m_arr, g["z"])
    finally:
        m_arr.close()
    assert np.array_equal(wav, wav2)
    assert all(np.array_equal(a, b) for a, b in zip(st, st2))


def test_windows_match_reference_stream(ptk_model):
    """ptd_decode_windows / ptd_decode_windows2 (equal widths) / ptd_decode_chunk stitched by the
    driver's loop, against the reference driver's --stream waveforms."""
    ctx, m, g = ptk_model
    lib = ctx.lib
    z = g["z"]
    T = z.shape[-1]
    dz = pkg.DevBuf.of(ctx, z)
    dw = pkg.DevBuf(256 * T)
    n = C.c_int64(0)
    try:
        for win, cx in (tuple(int(v) for v in s) for s in g["streams"]):
            ref = g[f"stream_{win}_{cx}"]
            say(f"  T = {T}: windows {win}/{cx} vs the reference's stream")
            dw.upload(ctx, np.full(256 * T, np.nan, np.float32))
            assert lib.ptd_debug_fill_arena(ctx.ptr, 0xFF) == 0   # columns never written read as NaN
            assert lib.ptd_decode_windows(ctx.ptr, m.ptr, dz.ptr, T, win, cx, dw.ptr) == 0
            wins = dw.download(ctx)
            s_stream, s_full = np_ref.sndr(wins, ref), np_ref.sndr(wins, g["wav"])
            say(f"    ptd_decode_windows: {s_stream:.1f} dB vs the stream, {s_full:.1f} dB vs the full decode")
            assert s_stream >= 60.0
            assert s_stream >= s_full + 20.0
            dw.upload(ctx, np.full(256 * T, np.nan, np.float32))
            assert lib.ptd_decode_windows2(ctx.ptr, m.ptr, dz.ptr, T, win, win, cx, dw.ptr) == 0
            assert np.array_equal(dw.download(ctx), wins)
            dp = pkg.DevBuf(256 * win)

            def chunk(a, w):
                assert lib.ptd_decode_chunk(ctx.ptr, m.ptr, dz.ptr, T, a, w, dp.ptr, C.byref(n)) == 0
                assert n.value == 256 * w
                return dp.download(ctx)[:n.value]

            try:
                stitched = ol.stream_stitch(chunk, T, win, cx)
            finally:
                dp.free()
            assert np.array_equal(stitched, wins)
    finally:
        dz.free(); dw.free()
