"""Container loaders on the device: the weight pool from a .ptk (ptd_pool_load_ptk, fp16 records
expanded by the device kernel) and the decoder model from a .ptk (ptd_model_create_ptk).

Bars: pool records are bit-identical to the host reader's fp32 values (which the CPU tests pin to
the reference's own reader); a decoder built from a container decodes bit-identically to one built
from the same (fp16-rounded) weights as arrays, and meets the 60 dB SNDR bar against the oracle."""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np
import pytest

import np_ref
import oracle_lib as ol
import ptk_writer as pw
from conftest import load_package

pkg = load_package()
synth = pkg.synth
pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu ptk] {msg}", file=sys.stderr, flush=True)


def test_pool_from_container(tmp_path):
    say("pool from container")
    rng = np.random.default_rng(12)
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    tensors = [
        ("w.fp32", rng.standard_normal((64, 7, 96)).astype(np.float32), 4),
        ("w.codes#h", np.concatenate([codes, rng.standard_normal(1000).astype(np.float16)]), 2),
        ("w.small#h", (rng.standard_normal(37) * 1e-5).astype(np.float32), 2),
        ("unused", np.ones(8, np.float32), 4),
    ]
    path = tmp_path / "pool.ptk"
    pw.write(path, tensors)
    f = pkg.Ptk(path)
    ctx = pkg.Ctx(arena_mb=64)
    try:
        ctab = ["w.codes#h", None, "absent", "w.fp32", "w.small#h"]
        arr = (C.c_char_p * len(ctab))(*[None if n is None else n.encode() for n in ctab])
        assert ctx.lib.ptd_pool_load_ptk(ctx.ptr, f.ptr, len(ctab), arr) == 0
        for k, name in enumerate(ctab):
            rec = ctx.lib.ptd_pool_record(k)
            i = -1 if name is None else f.find(name)
            if i < 0:
                assert not rec
                continue
            want = f.read(i).reshape(-1)
            out = np.empty_like(want)
            assert ctx.lib.ptd_d2h(ctx.ptr, out.ctypes.data_as(C.c_void_p), rec, out.nbytes) == 0
            assert np.array_equal(out.view(np.uint32), want.view(np.uint32)), name
    finally:
        ctx.close()
        f.close()


def _decode(ctx, model, z):
    T = z.shape[-1]
    dz = pkg.DevBuf.of(ctx, z)
    dw = pkg.DevBuf(256 * T)
    assert ctx.lib.ptd_decode(ctx.ptr, model.ptr, dz.ptr, T, 1, dw.ptr) == 0
    wav = dw.download(ctx)
    dz.free(); dw.free()
    return wav


@pytest.mark.parametrize("half", [True, False])
def test_decoder_from_container(tmp_path, half):
    say(f"decoder from container (fp16 layers: {half})")
    ws, bs = synth.decoder_weights(77)
    path = tmp_path / "dec.ptk"
    pw.write(path, pw.decoder_tensors(ws, bs, half=half))
    wsr = pw.half_rounded(ws) if half else ws
    f = pkg.Ptk(path)
    ctx = pkg.Ctx(arena_mb=256)
    try:
        assert f.check_decoder()
        m_ptk = pkg.Model.from_ptk(ctx, f)
        f.close()   # the model owns its device copy
        m_arr = pkg.Model(ctx, wsr, bs)
        z = synth.latent(40, 8)
        a = _decode(ctx, m_ptk, z)
        b = _decode(ctx, m_arr, z)
        assert np.array_equal(a, b)
        assert np_ref.sndr(a, ol.decoder(wsr, bs, z)) >= 60.0
        m_ptk.close(); m_arr.close()
    finally:
        f.close()
        ctx.close()


def test_decoder_container_refused_when_tail_differs(tmp_path):
    say("container with a foreign tail is refused")
    ws, bs = synth.decoder_weights(3)
    t = [(n, a * np.float32(0.5) if n == "dec.ConvTranspose_1.wp" else a, s)
         for n, a, s in pw.decoder_tensors(ws, bs)]
    path = tmp_path / "bad.ptk"
    pw.write(path, t)
    f = pkg.Ptk(path)
    ctx = pkg.Ctx(arena_mb=64)
    try:
        assert not ctx.lib.ptd_model_create_ptk(ctx.ptr, f.ptr)
    finally:
        ctx.close()
        f.close()
