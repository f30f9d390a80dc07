"""GPU parity of the device-resident decoder path (ptd_*) against the CPU oracle, at the BASELINE
configs: per layer (configs 1, 2), the MRF stacks (config 3), the full decoder (config 4), and the
concurrent / long-form serving (config 5).

Bars: per layer max |err| <= 1e-4 x RMS; end-to-end SNDR >= 60 dB.
Size-independent properties at full size: 8 concurrent streams give bit-identical output to one
stream (the kernels are deterministic); a delayed input gives the exactly delayed output, per layer
at the decoder's full shapes and through the whole decoder at T = 1500; batched items equal single
decodes bit for bit; and the overlap-save windowed decode of T = 1500 stays >= 60 dB from the full
decode."""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np
import pytest

import np_ref
import oracle_lib as ol
from conftest import load_package

pkg = load_package()
synth = pkg.synth
TOL = 1e-4
pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


def relerr(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.sqrt(np.mean(b ** 2)), 1e-30))


@pytest.fixture(scope="module")
def env():
    ctx = pkg.Ctx(arena_mb=2048)
    ws, bs = synth.decoder_weights(1234)
    model = pkg.Model(ctx, ws, bs)
    yield ctx, model, ws, bs
    model.close()
    ctx.close()


def dev_of(ctx, a):
    return pkg.DevBuf.of(ctx, a)


def test_config1_conv_pre(env):
    ctx, model, ws, bs = env
    say("config 1 conv_pre T=226")
    z = synth.latent(226, 11)
    ref = ol.conv(z, ws[0], bs[0], 512, 7, 1, 3, 1, 1, 0, 0.1)[0]
    dz, dy = dev_of(ctx, z), pkg.DevBuf(512 * 226)
    assert ctx.lib.ptd_layer(ctx.ptr, model.ptr, 0, dz.ptr, 226, 1, dy.ptr, 0.0, 0.1) == 0
    y = dy.download(ctx).reshape(512, 226)
    assert relerr(y, ref) < TOL
    dz.free(); dy.free()


def test_config2_ups0_with_input_leaky(env):
    ctx, model, ws, bs = env
    say("config 2 ups.0 T=226")
    x = np.random.default_rng(12).standard_normal((512, 226)).astype(np.float32)
    ref = ol.convT(np.where(x >= 0, x, np.float32(0.1) * x), ws[1], bs[1], 256, 16, 4, 6)[0]
    dx, dy = dev_of(ctx, x), pkg.DevBuf(256 * 904)
    assert ctx.lib.ptd_layer(ctx.ptr, model.ptr, 1, dx.ptr, 226, 1, dy.ptr, 0.1, 0.0) == 0
    y = dy.download(ctx).reshape(256, 904)
    assert relerr(y, ref) < TOL
    dx.free(); dy.free()


@pytest.mark.parametrize("layer", [2, 3, 10, 11, 18, 19, 21, 28, 37, 39])
def test_decoder_layers(env, layer):
    """Single decoder layers at their decoder shapes (T = 226 frames)."""
    ctx, model, ws, bs = env
    g = synth.dec_layer(layer)
    T = {True: 904, False: 3616}[layer < 20] if layer not in (0, 39) else 3617
    say(f"layer {layer} {g} T={T}")
    x = np.random.default_rng(layer).standard_normal((g["cin"], T)).astype(np.float32)
    ref = ol.conv(x, ws[layer], bs[layer], g["cout"], g["K"], 1, g["pad"], g["d"])[0]
    c4 = (g["cout"] + 3) // 4 * 4
    dx, dy = dev_of(ctx, x), pkg.DevBuf(c4 * T)
    assert ctx.lib.ptd_layer(ctx.ptr, model.ptr, layer, dx.ptr, T, 1, dy.ptr, 0.0, 0.0) == 0
    y = dy.download(ctx).reshape(c4, T)
    assert relerr(y, ref) < TOL
    dx.free(); dy.free()


@pytest.mark.parametrize("stage,C_,T", [(0, 256, 904), (1, 128, 3616)])
def test_config3_mrf(env, stage, C_, T):
    ctx, model, ws, bs = env
    say(f"config 3 MRF stage {stage} C={C_} T={T}")
    x = np.random.default_rng(30 + stage).standard_normal((C_, T)).astype(np.float32)
    base = 2 if stage == 0 else 21
    ref = ol.mrf(ws[base:base + 18], bs[base:base + 18], x, 0.1)
    dx, dy = dev_of(ctx, x), pkg.DevBuf(C_ * T)
    assert ctx.lib.ptd_mrf(ctx.ptr, model.ptr, stage, dx.ptr, T, 0.1, dy.ptr) == 0
    y = dy.download(ctx).reshape(C_, T)
    assert relerr(y, ref) < TOL
    dx.free(); dy.free()


def _decode(ctx, model, z, stages=False):
    T = z.shape[-1]
    dz = dev_of(ctx, z)
    dw = pkg.DevBuf(256 * T)
    if stages:
        lens = [ol.oracle().orc_dec_stage_len(i, T) for i in range(6)]
        sb = [pkg.DevBuf(n) for n in lens]
        arr = (C.c_void_p * 6)(*[b.ptr for b in sb])
        assert ctx.lib.ptd_decode_stages(ctx.ptr, model.ptr, dz.ptr, T, dw.ptr, arr) == 0
    else:
        assert ctx.lib.ptd_decode(ctx.ptr, model.ptr, dz.ptr, T, 1, dw.ptr) == 0
    wav = dw.download(ctx)
    out = (wav, [b.download(ctx) for b in sb]) if stages else wav
    dz.free(); dw.free()
    if stages:
        for b in sb:
            b.free()
    return out


@pytest.mark.parametrize("T", [1, 2, 5, 37])
def test_decoder_small_vs_oracle(env, T):
    """Every stage and the waveform against the oracle, down to one latent frame (conv_post's
    reflect pad and the tail's trim then touch both ends of the sequence in one tile)."""
    ctx, model, ws, bs = env
    say(f"decoder T={T}")
    z = synth.latent(T, 100 + T)
    ref, rst = ol.decoder(ws, bs, z, stages=True)
    wav, st = _decode(ctx, model, z, stages=True)
    for i in range(6):
        assert relerr(st[i], rst[i]) < TOL, f"stage {i}"
    assert np_ref.sndr(wav, ref) >= 60.0


def test_config4_decoder_T226_vs_oracle(env):
    """Config 4 at its BASELINE length: each of the six stages within 1e-4 x RMS of the oracle and
    the waveform >= 60 dB."""
    ctx, model, ws, bs = env
    say("config 4 decoder T=226")
    z = synth.latent(226, 226)
    ref, rst = ol.decoder(ws, bs, z, stages=True)
    wav, st = _decode(ctx, model, z, stages=True)
    assert wav.shape == (57856,)
    for i in range(6):
        assert relerr(st[i], rst[i]) < TOL, f"stage {i}"
    assert np_ref.sndr(wav, ref) >= 60.0


@pytest.mark.parametrize("L,batch", [(2, 1), (37, 2), (3617, 1)])
def test_tail_alone_vs_oracle(env, L, batch):
    """ptd_tail (the fused iSTFT + PQMF kernel) on random conv_post outputs against the oracle's
    tail, per batch item: max |err| <= 1e-4 x RMS (exp / sin / cos on the device against libm)."""
    ctx, model, ws, bs = env
    say(f"tail alone L={L} batch={batch}")
    rng = np.random.default_rng(L + batch)
    p = (0.7 * rng.standard_normal((batch, 72, L))).astype(np.float32)
    dp = dev_of(ctx, p)
    dw = pkg.DevBuf(batch * 16 * (L - 1))
    assert ctx.lib.ptd_tail(ctx.ptr, model.ptr, dp.ptr, L, batch, dw.ptr) == 0
    got = dw.download(ctx).reshape(batch, 16 * (L - 1))
    for i in range(batch):
        ref = ol.tail(p[i], ws[40], bs[40])
        assert relerr(got[i], ref) < 1e-4
    dp.free(); dw.free()


PLANTED_PHASES = [100.0, -100.0, 1000.0, -1000.0, 1600.0, -1600.0, 1e4, -1e4, 1e5, -3e5]


@pytest.mark.parametrize("scale", [5.0, 20.0, "planted"])
def test_tail_large_phase_logits_vs_oracle(env, scale):
    """The phase channels (9..17 of each band's 18) are raw conv outputs, unbounded: at sigma 5 and
    20, and with planted values up to |p| = 3e5 among sigma-20 logits (the hardware sine's input
    domain is 256 revolutions, |p| ~ 1608), the tail stays within 1e-4 x RMS of the oracle's
    double-precision sin.  The magnitude channels keep sigma 0.7 (exp overflows past 88)."""
    ctx, model, ws, bs = env
    say(f"tail with phase logits at scale {scale}")
    L, batch = 1001, 2
    rng = np.random.default_rng(99)
    p = 0.7 * rng.standard_normal((batch, 72, L))
    phase = np.zeros(72, bool)
    for band in range(4):
        phase[band * 18 + 9: band * 18 + 18] = True
    sig = 20.0 if scale == "planted" else scale
    p[:, phase, :] = sig * rng.standard_normal((batch, int(phase.sum()), L))
    if scale == "planted":
        rows = np.flatnonzero(phase)
        for b in range(batch):
            for i, v in enumerate(PLANTED_PHASES * 8):
                p[b, rows[(7 * i + b) % rows.size], (97 * i + 13 * b) % L] = v
    p = p.astype(np.float32)
    dp = dev_of(ctx, p)
    dw = pkg.DevBuf(batch * 16 * (L - 1))
    assert ctx.lib.ptd_tail(ctx.ptr, model.ptr, dp.ptr, L, batch, dw.ptr) == 0
    got = dw.download(ctx).reshape(batch, 16 * (L - 1))
    for i in range(batch):
        e = relerr(got[i], ol.tail(p[i], ws[40], bs[40]))
        say(f"  item {i}: max|err|/rms = {e:.3g}")
        assert e < 1e-4
    dp.free(); dw.free()


@pytest.mark.parametrize("L,batch", [(2, 1), (65, 3), (3617, 2)])
def test_tail_block_size_gives_the_same_samples(env, L, batch, knob_env):
    """The tail kernel's tile size (256, 512 or 1024 samples, chosen from the work; forced here
    through PTK_TAIL_OUT) and its grid (a workgroup per tile, or fewer workgroups looping over the
    tiles, split into one run per XCD when the grid is a multiple of 8: PTK_TAIL_GRID) only change
    which workgroup makes a sample: the waveform is bit-identical, and within the oracle bar."""
    ctx, model, ws, bs = env
    say(f"tail tile sizes and grids L={L} batch={batch}")
    rng = np.random.default_rng(7 * L + batch)
    p = (0.7 * rng.standard_normal((batch, 72, L))).astype(np.float32)
    dp = dev_of(ctx, p)
    dw = pkg.DevBuf(batch * 16 * (L - 1))
    outs = []
    for size, grid in (("256", "-1"), ("512", "-1"), ("1024", "-1"), ("256", "3"), ("1024", "2"),
                       ("512", "0"), ("256", "8"), ("512", "16")):
        knob_env.setenv("PTK_TAIL_OUT", size)
        knob_env.setenv("PTK_TAIL_GRID", grid)
        dw.upload(ctx, np.full(batch * 16 * (L - 1), np.nan, np.float32))
        assert ctx.lib.ptd_tail(ctx.ptr, model.ptr, dp.ptr, L, batch, dw.ptr) == 0
        outs.append(dw.download(ctx).reshape(batch, 16 * (L - 1)))
    knob_env.delenv("PTK_TAIL_OUT")
    knob_env.delenv("PTK_TAIL_GRID")
    for o in outs[1:]:
        assert np.array_equal(outs[0], o)
    for i in range(batch):
        assert relerr(outs[1][i], ol.tail(p[i], ws[40], bs[40])) < 1e-4
    dp.free(); dw.free()


def test_decoder_final_conv_is_an_input():
    """The final PQMF synthesis conv (layer 40) comes from the caller's weights: a random filter
    with a bias gives the oracle's waveform, not the model constant's."""
    say("decoder with a random final conv and bias, T=20")
    ctx = pkg.Ctx(arena_mb=256)
    ws, bs = synth.decoder_weights(99)
    rng = np.random.default_rng(40)
    W = (rng.standard_normal((1, 4, 63)) * 0.05).astype(np.float32)
    ws[40] = synth.pack_conv(W)
    bs[40] = np.array([0.25], np.float32)
    model = pkg.Model(ctx, ws, bs)
    z = synth.latent(20, 40)
    ref = ol.decoder(ws, bs, z)
    wav = _decode(ctx, model, z)
    model.close(); ctx.close()
    assert np_ref.sndr(wav, ref) >= 60.0


@pytest.mark.parametrize("T,batch", [(24, 3), (226, 8)])
def test_batched_decode_matches_single(env, T, batch):
    """batch > 1 (used by the windowed path) equals per-item decodes bit for bit: the conv tiling,
    the channel split included, is chosen from one item's shape, never from the batch size."""
    ctx, model, ws, bs = env
    say(f"batched decode T={T} batch={batch}")
    zs = [synth.latent(T, 500 + i) for i in range(batch)]
    singles = [_decode(ctx, model, z) for z in zs]
    dz = dev_of(ctx, np.stack(zs))
    dw = pkg.DevBuf(batch * 256 * T)
    assert ctx.lib.ptd_decode(ctx.ptr, model.ptr, dz.ptr, T, batch, dw.ptr) == 0
    wb = dw.download(ctx).reshape(batch, 256 * T)
    for i in range(batch):
        assert np.array_equal(wb[i], singles[i])
    dz.free(); dw.free()


# (layer, T, cols relative to the full launch: q0 offset, nq, ext_l, ext_r)
LAYER_COLS = [(0, 150, 20, 70, 13, 31), (1, 60, 9, 33, 5, 17), (20, 90, 30, 41, 29, 2),
              (18, 300, 37, 151, 36, 100), (37, 200, 100, 1, 99, 99), (38, 130, 1, 64, 0, 0),
              (39, 257, 64, 128, 40, 65)]


@pytest.mark.parametrize("rb,split", [(0, 0), (16, 1), (32, 2), (32, 4), (16, 4), (16, 8), (32, 8)])
def test_layer_cols_per_item(env, rb, split, knob_env):
    """A launch over part of the columns (the windowed decode's form: middle items [q0, q0 + nq),
    item 0 from ext_l earlier, the last item to ext_r later, tile shape of the full width) writes
    exactly those columns of each item, bit-identical to the full launch, and nothing else: conv
    and both convT layers, an MRF K = 11 conv at dilation 5, conv_post; batches 1, 2 and 3; every
    tile shape (rb, split 0: the launcher's choice)."""
    ctx, model, ws, bs = env
    say(f"layer columns rb={rb} split={split}")
    if rb:
        knob_env.setenv("PTK_CONV_RB", str(rb))
        knob_env.setenv("PTK_CONV_SPLIT", str(split))
    lib = ctx.lib
    rng = np.random.default_rng(rb * 10 + split)
    for layer, T, off, nq, el, er in LAYER_COLS:
        g = synth.dec_layer(layer)
        cin, cout4 = g["cin"], (g["cout"] + 3) // 4 * 4
        convT = g["convT"]
        Tout = 4 * T if convT else T
        q_full0, nq_full = (1, T + 1) if convT else (0, T)
        for batch in (1, 2, 3):
            x = rng.standard_normal((batch, cin, T)).astype(np.float32)
            dx = dev_of(ctx, x)
            sentinel = np.float32(-12345.5)
            dfull = pkg.DevBuf(batch * cout4 * Tout)
            assert lib.ptd_layer(ctx.ptr, model.ptr, layer, dx.ptr, T, batch, dfull.ptr, 0.1, 0.1) == 0
            full = dfull.download(ctx).reshape(batch, cout4, Tout)
            dy = pkg.DevBuf.of(ctx, np.full(batch * cout4 * Tout, sentinel, np.float32))
            q0 = q_full0 + off
            cols = (C.c_int64 * 5)(q0, nq, el, er, nq_full)
            assert lib.ptd_layer_cols(ctx.ptr, model.ptr, layer, dx.ptr, T, batch, dy.ptr, 0.1, 0.1,
                                      cols) == 0
            y = dy.download(ctx).reshape(batch, cout4, Tout)
            for b in range(batch):
                a = q0 - el if b == 0 else q0
                e = q0 + nq + er if b == batch - 1 else q0 + nq
                lo, hi = (max(4 * a - 6, 0), min(4 * e - 6, Tout)) if convT else (a, e)
                assert np.array_equal(y[b, :, lo:hi], full[b, :, lo:hi]), (layer, batch, b)
                assert np.all(y[b, :, :lo] == sentinel) and np.all(y[b, :, hi:] == sentinel), \
                    (layer, batch, b)
            dx.free(); dfull.free(); dy.free()


@pytest.mark.parametrize("rb,split", [(16, 1), (16, 2), (16, 4), (16, 8), (32, 1), (32, 2), (32, 4),
                                      (32, 8)])
def test_tile_shapes_vs_oracle(env, rb, split, knob_env):
    """Every tile shape the launcher can pick (16- or 32-row tiles, channel split 1 / 2 / 4, and 8
    on the single-problem launches; forced through PTK_CONV_RB / PTK_CONV_SPLIT) against the
    oracle: a conv with a LeakyReLU epilogue,
    both convT phase forms (input LeakyReLU, C4 = 256 and 128), the 72-row conv_post whose last
    row block is partial, an MRF stack (grouped K 3 / 7 / 11, residual adds, branch sums) and a
    whole decode."""
    ctx, model, ws, bs = env
    say(f"tile shape rb={rb} split={split}")
    knob_env.setenv("PTK_CONV_RB", str(rb))
    knob_env.setenv("PTK_CONV_SPLIT", str(split))
    rng = np.random.default_rng(40 + rb + split)
    cases = [(0, 226, 0.0, 0.1), (1, 61, 0.1, 0.0), (20, 97, 0.1, 0.0), (39, 203, 0.0, 0.0)]
    for layer, T, in_a, epi_a in cases:
        g = synth.dec_layer(layer)
        x = rng.standard_normal((g["cin"], T)).astype(np.float32)
        xin = np.where(x >= 0, x, np.float32(in_a) * x) if in_a > 0 else x
        if g.get("convT"):
            ref = ol.convT(xin, ws[layer], bs[layer], g["cout"], g["K"], g["s"], g["pad"])[0]
        else:
            e0 = 1 if epi_a > 0 else 0
            ref = ol.conv(xin, ws[layer], bs[layer], g["cout"], g["K"], 1, g["pad"], g["d"], e0, 0, epi_a)[0]
        c4 = (g["cout"] + 3) // 4 * 4
        dx, dy = dev_of(ctx, x), pkg.DevBuf(c4 * ref.shape[-1])
        assert ctx.lib.ptd_layer(ctx.ptr, model.ptr, layer, dx.ptr, T, 1, dy.ptr, in_a, epi_a) == 0
        y = dy.download(ctx).reshape(c4, -1)
        e = relerr(y, ref)
        say(f"  layer {layer} T={T}: {e:.3g}")
        assert e < TOL, layer
        dx.free(); dy.free()
    x = rng.standard_normal((128, 300)).astype(np.float32)
    ref = ol.mrf(ws[21:39], bs[21:39], x, 0.1)
    dx, dy = dev_of(ctx, x), pkg.DevBuf(128 * 300)
    assert ctx.lib.ptd_mrf(ctx.ptr, model.ptr, 1, dx.ptr, 300, 0.1, dy.ptr) == 0
    assert relerr(dy.download(ctx).reshape(128, 300), ref) < TOL
    dx.free(); dy.free()
    z = synth.latent(29, 929)
    ref, rst = ol.decoder(ws, bs, z, stages=True)
    wav, st = _decode(ctx, model, z, stages=True)
    for i in range(6):
        assert relerr(st[i], rst[i]) < TOL, f"stage {i}"
    assert np_ref.sndr(wav, ref) >= 60.0


@pytest.mark.parametrize("rb,split", [(0, 0), (16, 4), (16, 8), (32, 8)])
def test_general_epilogue_matches_fast(env, rb, split, knob_env):
    """The per-element epilogue (every block forced onto it with PTK_CONV_FAST=0) writes the fast
    epilogue's bits: a conv with a LeakyReLU epilogue, both convTs (the decoder's rows
    interleaved by phase, whose fast path stores sample pairs), conv_post with its partial row
    block, an MRF stack (residual adds) and whole decodes at batch 2 (the convTs' LeakyReLU
    copies, the branch averages); on the launcher's tiles and forced 16-row / 8-way ones."""
    ctx, model, ws, bs = env
    say(f"general vs fast epilogue rb={rb} split={split}")
    if rb:
        knob_env.setenv("PTK_CONV_RB", str(rb))
        knob_env.setenv("PTK_CONV_SPLIT", str(split))
    lib = ctx.lib

    def run_all():
        outs = []
        for layer, T, in_a, epi_a in [(0, 226, 0.0, 0.1), (1, 61, 0.1, 0.0), (20, 97, 0.1, 0.0),
                                      (39, 203, 0.0, 0.0)]:
            g = synth.dec_layer(layer)
            x = np.random.default_rng(layer).standard_normal((g["cin"], T)).astype(np.float32)
            c4 = (g["cout"] + 3) // 4 * 4
            tout = 4 * T if g.get("convT") else T
            dx, dy = dev_of(ctx, x), pkg.DevBuf(c4 * tout)
            assert lib.ptd_layer(ctx.ptr, model.ptr, layer, dx.ptr, T, 1, dy.ptr, in_a, epi_a) == 0
            outs.append(dy.download(ctx))
            dx.free(); dy.free()
        x = np.random.default_rng(3).standard_normal((128, 300)).astype(np.float32)
        dx, dy = dev_of(ctx, x), pkg.DevBuf(128 * 300)
        assert lib.ptd_mrf(ctx.ptr, model.ptr, 1, dx.ptr, 300, 0.1, dy.ptr) == 0
        outs.append(dy.download(ctx))
        dx.free(); dy.free()
        for T in (3, 45):
            z = np.stack([synth.latent(T, 600 + T), synth.latent(T, 700 + T)])
            dz, dw = dev_of(ctx, z), pkg.DevBuf(2 * 256 * T)
            assert lib.ptd_decode(ctx.ptr, model.ptr, dz.ptr, T, 2, dw.ptr) == 0
            outs.append(dw.download(ctx))
            dz.free(); dw.free()
        return outs

    fast = run_all()
    knob_env.setenv("PTK_CONV_FAST", "0")
    general = run_all()
    knob_env.delenv("PTK_CONV_FAST")
    for i, (a, b) in enumerate(zip(fast, general)):
        assert np.array_equal(a, b), i


def _oracle_windows(ws, bs, z, win, ctx_):
    """The reference's overlap-save schedule (main_v21_serve.c:229-257) composed on the oracle."""
    T = z.shape[-1]
    out = np.zeros(256 * T, np.float32)
    a = emitted = 0
    while emitted < T:
        w = min(win, T - a)
        last = a + w >= T
        lo = 0 if a == 0 else ctx_
        hi = w if last else w - ctx_
        e0, e1 = max(a + lo, emitted), min(a + hi, T)
        pcm = ol.decoder(ws, bs, np.ascontiguousarray(z[:, a:a + w]))
        if e1 > e0:
            out[e0 * 256:e1 * 256] = pcm[(e0 - a) * 256:(e1 - a) * 256]
            emitted = e1
        if last:
            break
        a = max(e1 - ctx_, 1)
    return out


def test_windows_small_vs_oracle(env):
    ctx, model, ws, bs = env
    say("windows T=70 win=32 ctx=8")
    T, win, cx = 70, 32, 8
    z = synth.latent(T, 70)
    ref = _oracle_windows(ws, bs, z, win, cx)
    dz, dw = dev_of(ctx, z), pkg.DevBuf(256 * T)
    assert ctx.lib.ptd_decode_windows(ctx.ptr, model.ptr, dz.ptr, T, win, cx, dw.ptr) == 0
    wav = dw.download(ctx)
    assert np_ref.sndr(wav, ref) >= 60.0
    dz.free(); dw.free()


@pytest.mark.parametrize("T,win,cx", [(20, 32, 8), (32, 32, 8), (48, 32, 8), (57, 32, 8), (70, 32, 8),
                                      (100, 40, 4), (50, 16, 0)])
def test_windows_schedule_edges_bitexact(env, T, win, cx):
    """The windowed decode (one batched decode reading the latents in place, each window's kept
    frames written straight to the output) equals per-window single decodes stitched by the
    reference's schedule (main_v21_serve.c:229-257) bit for bit: T shorter than a window, exactly
    one window, a full last window, a short last window."""
    ctx, model, ws, bs = env
    say(f"windows edges T={T} win={win} ctx={cx}")
    z = synth.latent(T, 300 + T)
    ref = np.zeros(256 * T, np.float32)
    a = emitted = 0
    while emitted < T:
        w = min(win, T - a)
        last = a + w >= T
        lo = 0 if a == 0 else cx
        hi = w if last else w - cx
        e0, e1 = max(a + lo, emitted), min(a + hi, T)
        pcm = _decode(ctx, model, np.ascontiguousarray(z[:, a:a + w]))
        if e1 > e0:
            ref[e0 * 256:e1 * 256] = pcm[(e0 - a) * 256:(e1 - a) * 256]
            emitted = e1
        if last:
            break
        a = max(e1 - cx, 1)
    dz, dw = dev_of(ctx, z), pkg.DevBuf.of(ctx, np.full(256 * T, np.nan, np.float32))
    assert ctx.lib.ptd_debug_fill_arena(ctx.ptr, 0xFF) == 0   # columns never written read as NaN
    assert ctx.lib.ptd_decode_windows(ctx.ptr, model.ptr, dz.ptr, T, win, cx, dw.ptr) == 0
    wav = dw.download(ctx)
    assert np.array_equal(wav, ref), f"max diff {np.nanmax(np.abs(wav - ref))}"
    dz.free(); dw.free()


def test_config5_longform_windows_vs_full(env):
    """T = 1500 through 96-frame windows with 16-frame context >= 60 dB from one full decode."""
    ctx, model, ws, bs = env
    say("config 5 long-form T=1500")
    T = 1500
    z = synth.latent(T, 1500)
    full = _decode(ctx, model, z)
    dz, dw = dev_of(ctx, z), pkg.DevBuf(256 * T)
    assert ctx.lib.ptd_decode_windows(ctx.ptr, model.ptr, dz.ptr, T, 96, 16, dw.ptr) == 0
    wav = dw.download(ctx)
    assert np_ref.sndr(wav, full) >= 60.0
    dz.free(); dw.free()


@pytest.mark.parametrize("T,win,cx", [(1500, 96, 16), (777, 96, 16), (400, 48, 16)])
def test_window_columns_change_no_sample(env, T, win, cx, knob_env):
    """The windowed decode computes only the columns its kept samples depend on: with the arena
    poisoned (every column it leaves out reads NaN) its output is bit-identical to the same decode
    computing every column (PTD_WINDOW_CONE=0), at config 5's long-form shape and two others."""
    ctx, model, ws, bs = env
    say(f"window columns T={T} win={win} ctx={cx}")
    lib = ctx.lib
    z = synth.latent(T, 900 + T)
    dz, dw = dev_of(ctx, z), pkg.DevBuf(256 * T)
    knob_env.setenv("PTD_WINDOW_CONE", "0")
    assert lib.ptd_decode_windows(ctx.ptr, model.ptr, dz.ptr, T, win, cx, dw.ptr) == 0
    whole = dw.download(ctx)
    knob_env.delenv("PTD_WINDOW_CONE")
    dw.upload(ctx, np.full(256 * T, np.nan, np.float32))
    assert lib.ptd_debug_fill_arena(ctx.ptr, 0xFF) == 0
    assert lib.ptd_decode_windows(ctx.ptr, model.ptr, dz.ptr, T, win, cx, dw.ptr) == 0
    wav = dw.download(ctx)
    assert np.all(np.isfinite(wav))
    assert np.array_equal(wav, whole)
    dz.free(); dw.free()


@pytest.mark.parametrize("tout,grid", [("256", "7"), ("1024", "3"), ("512", "-1"), ("256", "8"),
                                       ("1024", "24")])
def test_window_tail_tiles_and_grid_change_no_sample(env, tout, grid, knob_env):
    """A windowed decode's tail skips the tiles with no kept samples: with a few workgroups looping
    over the tiles (PTK_TAIL_GRID), or one per tile, at every tile size, the long-form request
    (T = 1500 in 96/16 windows) is bit-identical to the default launch, and every sample is
    written."""
    ctx, model, ws, bs = env
    say(f"windowed tail tiles {tout} grid {grid}")
    lib = ctx.lib
    T = 1500
    z = synth.latent(T, 4242)
    dz, dw = dev_of(ctx, z), pkg.DevBuf(256 * T)
    assert lib.ptd_decode_windows(ctx.ptr, model.ptr, dz.ptr, T, 96, 16, dw.ptr) == 0
    ref = dw.download(ctx)
    knob_env.setenv("PTK_TAIL_OUT", tout)
    knob_env.setenv("PTK_TAIL_GRID", grid)
    dw.upload(ctx, np.full(256 * T, np.nan, np.float32))
    assert lib.ptd_decode_windows(ctx.ptr, model.ptr, dz.ptr, T, 96, 16, dw.ptr) == 0
    wav = dw.download(ctx)
    knob_env.delenv("PTK_TAIL_OUT")
    knob_env.delenv("PTK_TAIL_GRID")
    assert np.all(np.isfinite(wav))
    assert np.array_equal(wav, ref)
    dz.free(); dw.free()


@pytest.mark.parametrize("T,mode", [(1500, "default"), (300, "2"), (1500, "2"), (600, "default")])
def test_window_streams_change_no_sample(env, T, mode, knob_env):
    """A batched run of windows split over the context's stream and a second stream (the default
    for runs of 16 windows or more; PTD_WINDOW_STREAMS=2 splits any run of two, =1 none) gives the
    same samples as the unsplit run, bit for bit, with the context's arena poisoned first; and a
    decode queued on the context right after it, which reuses the arena the second half used,
    still matches its own reference (it waits for the second stream).  Every T here ends in a
    clipped window, decoded on the context's stream inside the first half's arena region while
    the second half already runs (the split forks ahead of it)."""
    ctx, model, ws, bs = env
    say(f"window streams T={T} mode={mode}")
    lib = ctx.lib
    z = synth.latent(T, 7100 + T)
    z2 = synth.latent(150, 7200)
    dz, dw = dev_of(ctx, z), pkg.DevBuf(256 * T)
    dz2, dw2 = dev_of(ctx, z2), pkg.DevBuf(256 * 150)
    knob_env.setenv("PTD_WINDOW_STREAMS", "1")
    assert lib.ptd_decode_windows(ctx.ptr, model.ptr, dz.ptr, T, 96, 16, dw.ptr) == 0
    ref = dw.download(ctx)
    assert lib.ptd_decode(ctx.ptr, model.ptr, dz2.ptr, 150, 1, dw2.ptr) == 0
    ref2 = dw2.download(ctx)
    if mode == "default":
        knob_env.delenv("PTD_WINDOW_STREAMS")
    else:
        knob_env.setenv("PTD_WINDOW_STREAMS", mode)
    for rep in range(2):
        dw.upload(ctx, np.full(256 * T, np.nan, np.float32))
        dw2.upload(ctx, np.full(256 * 150, np.nan, np.float32))
        assert lib.ptd_debug_fill_arena(ctx.ptr, 0xFF) == 0
        assert lib.ptd_decode_windows(ctx.ptr, model.ptr, dz.ptr, T, 96, 16, dw.ptr) == 0
        assert lib.ptd_decode(ctx.ptr, model.ptr, dz2.ptr, 150, 1, dw2.ptr) == 0
        assert np.array_equal(dw.download(ctx), ref), f"rep {rep}"
        assert np.array_equal(dw2.download(ctx), ref2), f"rep {rep}"
    for b in (dz, dw, dz2, dw2):
        b.free()


def test_window_split_falls_back_to_one_stream_in_a_small_arena(env, knob_env):
    """A context whose arena holds the unsplit batched run (22 windows of the T = 1500 request) but
    not both halves of the split at once keeps the run on its own stream: the decode succeeds and
    matches the split decode of a roomy context bit for bit."""
    ctx, model, ws, bs = env
    say("window split fallback in a small arena")
    lib = ctx.lib
    T = 1500
    z = synth.latent(T, 7300)
    dz, dref, dw = dev_of(ctx, z), pkg.DevBuf(256 * T), pkg.DevBuf(256 * T)
    assert lib.ptd_decode_windows(ctx.ptr, model.ptr, dz.ptr, T, 96, 16, dref.ptr) == 0
    ref = dref.download(ctx)
    unsplit = int(lib.ptd_decode_arena_bytes(96, 22))
    assert int(lib.ptd_windows_arena_bytes(T, 96, 16)) > unsplit + 2048
    srv = lib.ptd_server_create(1, unsplit + 2048)
    assert srv
    try:
        c = lib.ptd_server_ctx(srv, 0)
        assert lib.ptd_decode_windows(c, model.ptr, dz.ptr, T, 96, 16, dw.ptr) == 0
        assert lib.ptd_device_sync() == 0
    finally:
        lib.ptd_server_destroy(srv)
    assert np.array_equal(dw.download(ctx), ref)
    for b in (dz, dref, dw):
        b.free()


@pytest.mark.parametrize("T,win,cx", [(20, 32, 8), (57, 32, 8), (70, 32, 8), (300, 96, 16), (50, 16, 0)])
def test_stream_chunks_stitched_equal_windows(env, T, win, cx):
    """ptd_decode_chunk window by window, stitched the way the reference's --stream driver does
    (main_v21.c:341-362: step win - 2*ctx, keep [ctx, win_eff - ctx) frames of each window, the
    first from 0 and the last to its end), equals the batched ptd_decode_windows bit for bit."""
    ctx, model, ws, bs = env
    say(f"stream chunks T={T} win={win} ctx={cx}")
    lib = ctx.lib
    z = synth.latent(T, 500 + T)
    dz = dev_of(ctx, z)
    dp = pkg.DevBuf(256 * win)
    n = C.c_int64(0)
    out = []
    step = max(win - 2 * cx, 1)
    a = 0
    while True:
        w = min(win, T - a)
        first, last = a == 0, a + w >= T
        assert lib.ptd_decode_chunk(ctx.ptr, model.ptr, dz.ptr, T, a, w, dp.ptr, C.byref(n)) == 0
        assert n.value == 256 * w
        pcm = dp.download(ctx)[:n.value]
        lo = 0 if first else cx * 256
        hi = n.value if last else min((w - cx) * 256, n.value)
        if hi > lo:
            out.append(pcm[lo:hi])
        if last:
            break
        a += step
    stitched = np.concatenate(out)
    dw = pkg.DevBuf(256 * T)
    assert lib.ptd_debug_fill_arena(ctx.ptr, 0xFF) == 0   # columns never written read as NaN
    assert lib.ptd_decode_windows(ctx.ptr, model.ptr, dz.ptr, T, win, cx, dw.ptr) == 0
    wav = dw.download(ctx)
    assert stitched.shape == wav.shape
    assert np.array_equal(stitched, wav), f"max diff {np.max(np.abs(stitched - wav))}"
    dz.free(); dp.free(); dw.free()


def test_stream_chunk_clipping_and_oracle(env):
    """pt_v21_stream_chunk's argument rules (pt_v21_host.c:2874-2878): a < 0 reads as 0, win < 1
    as 1, a window past the end is clipped, nothing left is an error; a clipped window's waveform
    matches the oracle's decode of the same frames."""
    ctx, model, ws, bs = env
    say("stream chunk clipping")
    lib = ctx.lib
    T = 40
    z = synth.latent(T, 41)
    dz, dp = dev_of(ctx, z), pkg.DevBuf(256 * 64)
    n = C.c_int64(-5)
    assert lib.ptd_decode_chunk(ctx.ptr, model.ptr, dz.ptr, T, T, 8, dp.ptr, C.byref(n)) == -1
    assert n.value == 0
    assert lib.ptd_decode_chunk(ctx.ptr, model.ptr, dz.ptr, T, -3, 0, dp.ptr, C.byref(n)) == 0
    assert n.value == 256
    one = dp.download(ctx)[:256]
    assert np.array_equal(one, _decode(ctx, model, np.ascontiguousarray(z[:, :1])))
    assert np_ref.sndr(one, ol.decoder(ws, bs, np.ascontiguousarray(z[:, :1]))) >= 60.0
    assert lib.ptd_decode_chunk(ctx.ptr, model.ptr, dz.ptr, T, 25, 64, dp.ptr, C.byref(n)) == 0
    assert n.value == 256 * 15
    got = dp.download(ctx)[:n.value]
    ref = ol.decoder(ws, bs, np.ascontiguousarray(z[:, 25:]))
    assert np_ref.sndr(got, ref) >= 60.0
    dz.free(); dp.free()


# (layer, T, cin, rows of y, output columns per input column, half receptive field in input columns)
# layers 18 / 19: MRF-256 K 11 c1 at dilation 5 and c2; 37: MRF-128 K 11 c1 at dilation 5
_SHIFT_LAYERS = [(0, 226, 192, 512, 1, 3), (1, 226, 512, 256, 4, 4), (18, 904, 256, 256, 1, 25),
                 (19, 904, 256, 256, 1, 5), (20, 904, 256, 128, 4, 4), (37, 3616, 128, 128, 1, 25),
                 (39, 3616, 128, 72, 1, 3)]


@pytest.mark.parametrize("layer,T,cin,rows,up,half", _SHIFT_LAYERS,
                         ids=[f"layer{c[0]}-T{c[1]}" for c in _SHIFT_LAYERS])
def test_layer_shift_equivariance_full_size(env, layer, T, cin, rows, up, half):
    """At the decoder's full shapes (conv_pre and ups.0 at T = 226, MRF-256 at 904, ups.1 at 904,
    MRF-128 and conv_post at 3616): an input delayed by s columns gives the output delayed by
    up*s columns, bit for bit, wherever neither receptive field reaches an edge.  Each output
    column is summed in the same order whichever tile holds it, so this checks every tile position
    of the full-size grid without the oracle."""
    ctx, model, ws, bs = env
    s = 37
    say(f"shift equivariance layer {layer} T={T}")
    rng = np.random.default_rng(layer)
    x = rng.standard_normal((cin, T)).astype(np.float32)
    x2 = np.empty_like(x)
    x2[:, s:] = x[:, :-s]
    x2[:, :s] = rng.standard_normal((cin, s)).astype(np.float32)
    lib = ctx.lib
    outs = []
    for xx in (x, x2):
        dx, dy = dev_of(ctx, xx), pkg.DevBuf(rows * up * T + 64)
        assert lib.ptd_layer(ctx.ptr, model.ptr, layer, dx.ptr, T, 1, dy.ptr, 0.1, 0.0) == 0
        outs.append(dy.download(ctx)[:rows * up * T].reshape(rows, up * T))
        dx.free(); dy.free()
    y, y2 = outs
    lo, hi = up * (s + half + 1), up * (T - half - 1)
    assert hi - lo > up * T // 2
    assert np.array_equal(y2[:, lo:hi], y[:, lo - up * s:hi - up * s])


def test_decoder_shift_equivariance_T1500(env):
    """The whole decoder at config 5's long-form length (T = 1500, too long for the oracle in a
    test): latents delayed by s frames give the waveform delayed by 256*s samples, bit for bit,
    away from both ends.  Every stage computes each column (sample) in an order that does not
    depend on its position, so this holds exactly through all 19 launches."""
    ctx, model, ws, bs = env
    T, s, margin = 1500, 37, 48
    say("decoder shift equivariance T=1500")
    z = synth.latent(T, 1501)
    z2 = np.empty_like(z)
    z2[:, s:] = z[:, :-s]
    z2[:, :s] = synth.latent(s, 1502)
    w, w2 = _decode(ctx, model, z), _decode(ctx, model, z2)
    lo, hi = 256 * (s + margin), 256 * (T - margin)
    assert np.array_equal(w2[lo:hi], w[lo - 256 * s:hi - 256 * s])
    # and the delay really is visible: the waveforms differ near the start
    assert not np.array_equal(w2[:256 * s], w[:256 * s])


def test_decode_graph_replays_match_eager(env):
    """A decode captured as a HIP graph, replayed three times with eager decodes of another input
    on the same context (its arena) and a synchronising read between the replays, gives the eager
    decode's waveform bit for bit every time; refilling the input buffer makes the next replay
    decode the new input; another context cannot launch it."""
    ctx, model, ws, bs = env
    say("decode graph replays")
    lib = ctx.lib
    T, To = 120, 200
    z1, z2, zo = synth.latent(T, 61), synth.latent(T, 62), synth.latent(To, 63)
    ref1, ref2 = _decode(ctx, model, z1), _decode(ctx, model, z2)
    dz, dw = dev_of(ctx, z1), pkg.DevBuf(256 * T)
    dzo, dwo = dev_of(ctx, zo), pkg.DevBuf(256 * To)
    g = lib.ptd_decode_graph(ctx.ptr, model.ptr, dz.ptr, T, 1, dw.ptr)
    assert g
    try:
        for _ in range(3):
            dw.upload(ctx, np.full(256 * T, np.nan, np.float32))
            assert lib.ptd_graph_launch(ctx.ptr, g) == 0
            assert lib.ptd_decode(ctx.ptr, model.ptr, dzo.ptr, To, 1, dwo.ptr) == 0
            assert np.array_equal(dw.download(ctx), ref1)
        dz.upload(ctx, z2)
        assert lib.ptd_graph_launch(ctx.ptr, g) == 0
        assert np.array_equal(dw.download(ctx), ref2)
        other = pkg.Ctx(arena_mb=64)
        try:
            assert lib.ptd_graph_launch(other.ptr, g) == -1
        finally:
            other.close()
    finally:
        lib.ptd_graph_destroy(g)
    for b in (dz, dw, dzo, dwo):
        b.free()


def test_config5_as_benchmarked(env):
    """Config 5 exactly as bench.py times it: 8 requests, T ~ U[56, 400] (seed 5), plus the T = 1500
    request in 96-frame overlap-save windows with 16 frames of context, on 9 contexts / streams
    sharing one weight set, with bench.py's arena size.  Run twice: every output equals its
    single-stream decode bit for bit, each of the 8 requests reaches >= 60 dB against the oracle
    (decoded on host threads, as the reference's parallel driver gates its streams,
    main_v21_par.c:99-109, :142-157), and the long-form request reaches >= 60 dB against one full
    decode of the same latents.  The long-form request is also gated against the oracle at
    T = 1500 (its conv nodes split over host threads, bit-identical to one thread): the stitched
    windows >= 60 dB against the oracle's full decode and against the oracle's own windows stitched
    by the reference driver's loop, and each of the six stages of ptd_decode_stages at T = 1500
    within 1e-4 x RMS of the oracle's."""
    ctx, model, ws, bs = env
    lib = ctx.lib
    Ts = synth.request_lengths(5, 8)
    T_long, WIN, CTX = 1500, 96, 16
    say(f"config 5 as benchmarked: T={Ts} + {T_long} in {WIN}/{CTX} windows")
    zs = [synth.latent(T, 900 + i) for i, T in enumerate(Ts + [T_long])]
    dz = [dev_of(ctx, z) for z in zs]
    singles = [_decode(ctx, model, z) for z in zs[:8]]
    dlw = pkg.DevBuf(256 * T_long)
    assert lib.ptd_decode_windows(ctx.ptr, model.ptr, dz[-1].ptr, T_long, WIN, CTX, dlw.ptr) == 0
    single_long = dlw.download(ctx)
    assert lib.ptd_decode(ctx.ptr, model.ptr, dz[-1].ptr, T_long, 1, dlw.ptr) == 0
    full_long = dlw.download(ctx)
    dlw.free()
    arena = max(int(lib.ptd_decode_arena_bytes(max(Ts), 1)),
                int(lib.ptd_windows_arena_bytes(T_long, WIN, CTX))) + (64 << 20)
    srv = lib.ptd_server_create(9, arena)
    assert srv
    dw = [pkg.DevBuf(256 * T) for T in Ts + [T_long]]
    reqs = [pkg.Request(dz[i].ptr, dw[i].ptr, T, 0, 0) for i, T in enumerate(Ts)]
    reqs.append(pkg.Request(dz[-1].ptr, dw[-1].ptr, T_long, WIN, CTX))
    arr = (pkg.Request * 9)(*reqs)
    wall = C.c_double()
    try:
        for rep in range(2):
            for b in dw:
                b.upload(ctx, np.full(b.n, np.nan, np.float32))
            assert lib.ptd_serve_run(srv, model.ptr, arr, 9, C.byref(wall)) == 0
            outs = [b.download(ctx) for b in dw]
            for i in range(8):
                assert np.array_equal(outs[i], singles[i]), f"run {rep} stream {i}"
            assert np.array_equal(outs[8], single_long), f"run {rep} long-form"
    finally:
        lib.ptd_server_destroy(srv)
    s_long = np_ref.sndr(outs[8], full_long)
    say(f"  long-form windows vs full decode: {s_long:.1f} dB")
    assert s_long >= 60.0
    say(f"  oracle at T = {T_long} on {ol.host_threads()} host threads")
    ref_long, ref_st = ol.decoder(ws, bs, zs[-1], stages=True, threads=ol.host_threads())
    s_or = np_ref.sndr(outs[8], ref_long)
    say(f"  long-form windows vs the oracle's full decode: {s_or:.1f} dB")
    assert s_or >= 60.0
    ref_win = ol.decoder_stream(ws, bs, zs[-1], WIN, CTX, threads=ol.host_threads())
    s_ow = np_ref.sndr(outs[8], ref_win)
    say(f"  long-form windows vs the oracle's windows: {s_ow:.1f} dB")
    assert s_ow >= 60.0
    _, st_long = _decode(ctx, model, zs[-1], stages=True)
    for i in range(6):
        e = relerr(st_long[i], ref_st[i])
        say(f"  T = {T_long} stage {i}: max|err|/rms = {e:.3g}")
        assert e < TOL, f"stage {i}"
    refs, _ = ol.decoder_threads(ws, bs, zs[:8], cores=list(range(8)))
    for i in range(8):
        s = np_ref.sndr(outs[i], refs[i])
        say(f"  request {i} (T={Ts[i]}): {s:.1f} dB vs the oracle")
        assert s >= 60.0, f"request {i}"
    for b in dz + dw:
        b.free()


def test_server_stream_placement_changes_no_sample(env, knob_env):
    """ptd_server_create times where its contexts' streams sit on HIP's hardware queues (idle
    ballast streams made first, a bounded single-workgroup kernel per stream) and keeps the most
    even arrangement: the T = 226 request on 8 concurrent streams gives the same samples with the
    placement on and off (PTD_SERVER_PLACE=0), both equal to the batched decode, over repeated
    servers (the ballast streams are released with each)."""
    ctx, model, ws, bs = env
    say("server stream placement: 8 streams of T = 226, placement on / off")
    lib = ctx.lib
    T, n = 226, 8
    zs = [synth.latent(T, 226 + i) for i in range(n)]
    dz = [dev_of(ctx, z) for z in zs]
    db = dev_of(ctx, np.concatenate(zs))
    wb = pkg.DevBuf(n * 256 * T)
    assert lib.ptd_decode(ctx.ptr, model.ptr, db.ptr, T, n, wb.ptr) == 0
    batched = wb.download(ctx).reshape(n, -1)
    arena = int(lib.ptd_decode_arena_bytes(T, 1)) + (16 << 20)
    try:
        for place in ("1", "0", "1"):
            knob_env.setenv("PTD_SERVER_PLACE", place)
            srv = lib.ptd_server_create(n, arena)
            assert srv
            dw = [pkg.DevBuf.of(ctx, np.full(256 * T, np.nan, np.float32)) for _ in range(n)]
            reqs = (pkg.Request * n)(*[pkg.Request(dz[i].ptr, dw[i].ptr, T, 0, 0) for i in range(n)])
            wall = C.c_double()
            try:
                assert lib.ptd_serve_run(srv, model.ptr, reqs, n, C.byref(wall)) == 0
            finally:
                lib.ptd_server_destroy(srv)
            for i in range(n):
                assert np.array_equal(dw[i].download(ctx), batched[i]), (place, i)
            for b in dw:
                b.free()
    finally:
        for b in dz + [db, wb]:
            b.free()
