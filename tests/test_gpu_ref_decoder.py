"""The device-resident decoder against the reference's own graph interpreter.

The synthetic full model of tests/full_model.py is written as a .ptk container, read by the
library's container reader (ptd_ptk_open) and turned into a device model (ptd_model_create_ptk,
fp16 records expanded on the device).  ptd_decode_stages then decodes the latents the reference's
CPU driver fed its decoder, and each stage and the waveform are compared with what that driver
computed (tests/golden/ref_decoder_ckpt.npz, written by tests/golden/gen_decoder_ckpt.py through
the driver's checkpoint option, main_v21.c:218-219, :307-321).

Bars: per stage max |err| <= 1e-4 x RMS; waveform >= 60 dB SNDR."""
from __future__ import annotations

import ctypes as C
import pathlib
import sys

import numpy as np
import pytest

import full_model as fm
import np_ref
from conftest import load_package

pkg = load_package()
GOLD = pathlib.Path(__file__).resolve().parent / "golden" / "ref_decoder_ckpt.npz"
STAGES = ["stage0", "stage1", "stage2", "stage3", "stage4", "stage5"]
pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


def relerr(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.max(np.abs(a - b)) / max(np.sqrt(np.mean(b ** 2)), 1e-30))


def _decode_stages(ctx, model, z):
    T = z.shape[-1]
    dz = pkg.DevBuf.of(ctx, z)
    dw = pkg.DevBuf(256 * T)
    g = np.load(GOLD)
    sb = [pkg.DevBuf(g[k].size) for k in STAGES]
    arr = (C.c_void_p * 6)(*[b.ptr for b in sb])
    try:
        assert ctx.lib.ptd_decode_stages(ctx.ptr, model.ptr, dz.ptr, T, dw.ptr, arr) == 0
        return dw.download(ctx), [b.download(ctx) for b in sb]
    finally:
        dz.free(); dw.free()
        for b in sb:
            b.free()


def test_container_decoder_matches_reference_interpreter(tmp_path):
    g = np.load(GOLD)
    say("container model vs the reference interpreter's checkpoints")
    path = tmp_path / "model.ptk"
    fm.write_container(path, seed=int(g["container_seed"]))
    f = pkg.Ptk(path)
    ctx = pkg.Ctx(arena_mb=256)
    try:
        assert f.check_decoder()
        m_ptk = pkg.Model.from_ptk(ctx, f)
        f.close()
        wav, st = _decode_stages(ctx, m_ptk, g["z"])
        for i, k in enumerate(STAGES):
            e = relerr(st[i], g[k])
            say(f"  {k}: max|err|/rms = {e:.3g}")
            assert e <= 1e-4, k
        s = np_ref.sndr(wav, g["wav"])
        say(f"  waveform SNDR {s:.1f} dB")
        assert s >= 60.0
        # the same layers handed over as arrays give the same bits
        ws, bs = fm.decoder_layers(int(g["container_seed"]))
        m_arr = pkg.Model(ctx, ws, bs)
        wav2, st2 = _decode_stages(ctx, m_arr, g["z"])
        assert np.array_equal(wav, wav2)
        assert all(np.array_equal(a, b) for a, b in zip(st, st2))
        m_arr.close()
        m_ptk.close()
    finally:
        f.close()
        ctx.close()
