"""CPU tests that pin the C oracle: the reference's own outputs (golden fixtures written by
oracle/_ref, and the live reference library where it was built), float64 brute force of the ONNX
definitions, torch's CPU conv1d / conv_transpose1d, closed forms, invariants, and the six layout
mutation trials of the reference's docs (docs/v21_layers.md:103-106), each of which must fail."""
from __future__ import annotations

import pathlib

import numpy as np
import pytest
import torch

import np_ref
import oracle_lib as ol
from conftest import ROOT, load_package

synth = load_package().synth
GOLD = np.load(ROOT / "tests" / "golden" / "ref_conv_cases.npz")


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.sqrt(np.mean(b ** 2)), 1e-30))


def _conv_cases():
    return sorted({k.split("_")[0] for k in GOLD.files if k.startswith("conv") and not k.startswith("convT")})


def _convT_cases():
    return sorted({k.split("_")[0] for k in GOLD.files if k.startswith("convT")})


@pytest.mark.parametrize("case", _conv_cases())
def test_conv_golden_bitexact(case):
    B, cin, cout, T, K, s, pad, d, e0, e1, hb = GOLD[case + "_cfg"].tolist()
    a0, a1 = GOLD[case + "_alpha"].tolist()
    b = GOLD[case + "_b"] if hb else None
    y = ol.conv(GOLD[case + "_x"], GOLD[case + "_wp"], b, cout, K, s, pad, d, e0, e1, a0, a1)
    assert np.array_equal(y, GOLD[case + "_y"])
    # the fixture itself against the ONNX definition in float64 (pre-epilogue cases)
    if e0 == 0 and e1 == 0:
        for bi in range(B):
            ref = np_ref.conv1d(GOLD[case + "_x"][bi], GOLD[case + "_w"], b, s, pad, d)
            assert rel(GOLD[case + "_y"][bi, :cout], ref) < 2e-6


@pytest.mark.parametrize("case", _convT_cases())
def test_convT_golden_bitexact(case):
    B, cin, cout, tin, K, s, pad, hb = GOLD[case + "_cfg"].tolist()
    b = GOLD[case + "_b"] if hb else None
    y = ol.convT(GOLD[case + "_x"], GOLD[case + "_wp"], b, cout, K, s, pad)
    assert np.array_equal(y, GOLD[case + "_y"])
    for bi in range(B):
        ref = np_ref.conv_transpose1d(GOLD[case + "_x"][bi], GOLD[case + "_w"], b, s, pad)
        assert rel(GOLD[case + "_y"][bi, :cout], ref) < 2e-6


def _rand_conv(rng):
    B = int(rng.integers(1, 3))
    cin, cout = int(rng.integers(1, 12)), int(rng.integers(1, 12))
    K, s, d = int(rng.integers(1, 8)), int(rng.integers(1, 3)), int(rng.integers(1, 4))
    pad = int(rng.integers(0, d * (K - 1) // 2 + 2))
    T = int(rng.integers((K - 1) * d + 1, 40))
    return B, cin, cout, K, s, d, pad, T


@pytest.mark.parametrize("seed", range(8))
def test_conv_vs_torch_and_ref(seed):
    rng = np.random.default_rng(seed)
    B, cin, cout, K, s, d, pad, T = _rand_conv(rng)
    x = rng.standard_normal((B, cin, T)).astype(np.float32)
    W = rng.standard_normal((cout, cin, K)).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32)
    y = ol.conv(x, synth.pack_conv(W), b, cout, K, s, pad, d)
    t = torch.nn.functional.conv1d(torch.from_numpy(x).double(), torch.from_numpy(W).double(),
                                   torch.from_numpy(b).double(), stride=s, padding=pad, dilation=d)
    assert rel(y[:, :cout], t.numpy()) < 2e-6
    assert np.all(y[:, cout:] == 0.0)   # padding rows: zero bias, zero weights
    if ol.have_ref():
        yr = ol.conv(x, synth.pack_conv(W), b, cout, K, s, pad, d, lib=ol.ref())
        assert np.array_equal(y, yr)


@pytest.mark.parametrize("seed", range(8))
def test_convT_vs_torch_and_ref(seed):
    rng = np.random.default_rng(100 + seed)
    B = int(rng.integers(1, 3))
    cin, cout = int(rng.integers(1, 10)), int(rng.integers(1, 10))
    s = int(rng.integers(1, 5))
    K = int(rng.integers(1, 17))
    pad = int(rng.integers(0, (K - 1) // 2 + 1))
    tin = int(rng.integers(2, 30))
    if (tin - 1) * s - 2 * pad + K <= 0:
        pad = 0
    x = rng.standard_normal((B, cin, tin)).astype(np.float32)
    W = rng.standard_normal((cin, cout, K)).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32)
    y = ol.convT(x, synth.pack_convtranspose(W, s), b, cout, K, s, pad)
    t = torch.nn.functional.conv_transpose1d(torch.from_numpy(x).double(), torch.from_numpy(W).double(),
                                             torch.from_numpy(b).double(), stride=s, padding=pad)
    assert rel(y[:, :cout], t.numpy()) < 2e-6
    if ol.have_ref():
        yr = ol.convT(x, synth.pack_convtranspose(W, s), b, cout, K, s, pad, lib=ol.ref())
        assert np.array_equal(y, yr)


def test_epilogue_codes():
    lib = ol.oracle()
    for v in (-2.5, -0.0, 0.0, 3.0):
        assert lib.orc_epi(v, 1, 0.1) == pytest.approx(v if v >= 0 else np.float32(0.1) * np.float32(v))
        assert lib.orc_epi(v, 2, 0.0) == (v if v > 0 else 0.0)
        assert lib.orc_epi(v, 3, 2.0) == v * 2.0
        assert lib.orc_epi(v, 4, 1.0) == v + 1.0
        assert lib.orc_epi(v, 0, 9.0) == v


def test_convT_delta_and_phase_cover():
    """A delta input reproduces the kernel; every output index gets exactly one (q, r)."""
    K, s, pad = 16, 4, 6
    rng = np.random.default_rng(3)
    W = rng.standard_normal((1, 1, K)).astype(np.float32)
    x = np.zeros((1, 1, 9), np.float32)
    x[0, 0, 4] = 1.0
    y = ol.convT(x, synth.pack_convtranspose(W, s), None, 1, K, s, pad)[0, 0]
    ref = np.zeros_like(y)
    for k in range(K):
        t = 4 * s + k - pad
        if 0 <= t < y.size:
            ref[t] = W[0, 0, k]
    assert np.array_equal(y, ref)
    tin = 9
    Lout = (tin - 1) * s - 2 * pad + K
    nt = synth.ntap(K, s)
    hits = np.zeros(Lout, int)
    for q in range(tin + nt - 1):
        for r in range(s):
            oi = q * s + r - pad
            if 0 <= oi < Lout:
                hits[oi] += 1
    assert np.all(hits == 1)


# ---------------------------------------------------------------- mutation trials
def _convT_mut(x, W, b, s, pad, mode):
    """Packed-phase convT evaluation (tools/export_v21.py:193-227 form) with one planted mistake."""
    cin, cout, K = W.shape
    nt = synth.ntap(K, s)
    Wph = np.zeros((s, cout, cin, nt))
    for r in range(s):
        for j in range(nt):
            k = (r * nt + j) if mode == "phase_map" else (r + j * s)
            if k < K:
                Wph[r, :, :, j] = W[:, :, k].T
    tin = x.shape[-1]
    Q = tin if mode == "no_flush" else tin + nt - 1
    Lout = (tin - 1) * s - 2 * pad + K
    out = np.zeros((cout, Lout))
    for q in range(Q):
        for r in range(s):
            oi = q * s + r - pad
            if not 0 <= oi < Lout:
                continue
            acc = np.zeros(cout) if mode == "no_bias" else b.astype(np.float64).copy()
            for j in range(nt):
                col = q + j if mode == "tap_sign" else q - j
                if 0 <= col < tin:
                    acc += Wph[r, :, :, j] @ x[:, col]
            out[:, oi] = acc
    return out


@pytest.mark.parametrize("mode", ["none", "phase_map", "no_flush", "tap_sign", "no_bias"])
def test_convT_mutations_fail(mode):
    rng = np.random.default_rng(11)
    x = rng.standard_normal((6, 12))
    W = rng.standard_normal((6, 5, 16))
    b = rng.standard_normal(5)
    ref = np_ref.conv_transpose1d(x, W, b, 4, 6)
    got = _convT_mut(x, W, b, 4, 6, mode)
    if mode == "none":
        assert rel(got, ref) < 1e-12
    else:
        assert rel(got, ref) > 1e-2


def test_layout_mutations_fail():
    """convT-layout W in the conv loop, and a flipped pack transpose, must both be caught."""
    rng = np.random.default_rng(12)
    x = rng.standard_normal((8, 30)).astype(np.float32)
    W = rng.standard_normal((8, 8, 4)).astype(np.float32)
    b = np.zeros(8, np.float32)
    ref = np_ref.conv1d(x, W, b, 1, 1, 1)
    good = ol.conv(x, synth.pack_conv(W), b, 8, 4, 1, 1, 1)[0]
    assert rel(good, ref) < 2e-6
    flipped = np.ascontiguousarray(synth.pack_conv(W).transpose(0, 1, 3, 2)).reshape(2, 4, 8, 4)
    bad = ol.conv(x, np.ascontiguousarray(flipped), b, 8, 4, 1, 1, 1)[0]
    assert rel(bad, ref) > 1e-2
    # the ONNX convT operand order [Cin][Cout][K] handed to the conv packer (a transposed operand)
    bad2 = ol.conv(x, synth.pack_conv(np.ascontiguousarray(W.transpose(1, 0, 2))), b, 8, 4, 1, 1, 1)[0]
    assert rel(bad2, ref) > 1e-2


# ---------------------------------------------------------------- decoder and constants
def test_constants_closed_forms():
    hann, bc, bs = ol.constants()
    assert np.allclose(hann, np_ref.hann16(), atol=1e-7)
    # the trace's own preview values of /dec/Constant_109 (ref/v21_graph_trace.txt:4009)
    assert np.allclose(hann[:8], [0.0, 0.03806025, 0.14644662, 0.3086583, 0.5, 0.69134176,
                                  0.8535534, 0.9619398], atol=1e-7)
    rng = np.random.default_rng(5)
    spec = rng.standard_normal((9, 7)) + 1j * rng.standard_normal((9, 7))
    frames = bc.T.astype(np.float64) @ spec.real + bs.T.astype(np.float64) @ spec.imag
    assert np.allclose(frames, np.fft.irfft(spec, n=16, axis=0), atol=1e-6)


def test_pqmf_filter_is_the_models():
    """The decoder's last conv weight is the model constant /dec/Constant_134 (1, 4, 63).  The
    packaged copy must equal the trace's own preview of it (ref/v21_graph_trace.txt:4064) and, where
    the reference tree exists, the full raw bytes in spec/v21_layers.json."""
    h = synth.pqmf_synthesis()
    assert h.shape == (1, 4, 63)
    assert np.array_equal(h.ravel()[:8], np.array(
        [1.6410408e-05, 5.2573592e-05, 8.4096690e-05, 6.8166526e-05, 1.0740955e-05,
         3.3666347e-05, 3.3252931e-04, 9.7845600e-04], np.float32))
    spec_file = pathlib.Path("/root/reference/spec/v21_layers.json")
    if spec_file.exists():
        import importlib.util
        ex = ROOT / "tests" / "golden" / "extract_constants.py"
        sp = importlib.util.spec_from_file_location("extract_constants", ex)
        mod = importlib.util.module_from_spec(sp)
        sp.loader.exec_module(mod)
        import json
        ref = mod.constant(json.loads(spec_file.read_text()), "/dec/Constant_134")
        assert np.array_equal(ref, h)
    # a cosine-modulated synthesis bank: band 0 carries the DC gain, the others sum to ~0
    sums = h[0].astype(np.float64).sum(axis=1)
    assert abs(sums[0] - 1.314) < 1e-3 and np.all(np.abs(sums[1:]) < 1e-4)


@pytest.mark.parametrize("T", [4, 9])
def test_decoder_vs_float64(T):
    ws, bs, raw = synth.decoder_weights(7, raw=True)
    z = synth.latent(T, 3)
    wav, st = ol.decoder(ws, bs, z, stages=True)
    ref, mid = np_ref.decoder(raw, bs, z)
    assert wav.shape == (256 * T,)
    assert np_ref.sndr(wav, ref) > 90.0
    for i, k in enumerate(["h", "x0", "m0", "x1", "m1", "p"]):
        assert rel(st[i].reshape(mid[k].shape), mid[k]) < 1e-4, k


def test_decoder_ref_conv_bitexact():
    if not ol.have_ref():
        pytest.skip("oracle/_ref not built (the reference tree is absent on this machine)")
    ws, bs = synth.decoder_weights(8)
    z = synth.latent(5, 4)
    assert np.array_equal(ol.decoder(ws, bs, z), ol.decoder(ws, bs, z, use_ref=True))


@pytest.mark.parametrize("m,k,n,pad", [(37, 53, 29, 0), (120, 96, 192, 3), (5, 0, 7, 2)])
def test_ref_matmul_shim(m, k, n, pad):
    """The reference's CPU matmul through the shim (the device matmul's second check and its CPU
    baseline): C = A B over the first k / n columns, padding columns of C left as they were, and
    k = 0 gives zeros."""
    if not ol.have_ref():
        pytest.skip("oracle/_ref not built (the reference tree is absent on this machine)")
    rng = np.random.default_rng(m + n)
    lda, ldb, ldc = k + pad, n + pad, n + pad
    A = rng.standard_normal((m, max(lda, 1))).astype(np.float32)
    B = rng.standard_normal((max(k, 1), ldb)).astype(np.float32)
    Cm = np.full((m, ldc), 7.0, np.float32)
    ol.ref_matmul(A, m, k, lda, B, ldb, n, Cm, ldc)
    want = A[:, :k].astype(np.float64) @ B[:k, :n]
    assert np.abs(Cm[:, :n] - want).max() <= 1e-5 * max(1.0, np.abs(want).max())
    assert np.all(Cm[:, n:] == 7.0)


def test_decoder_mutation_caught():
    """Dropping the /3 of the branch average (a plausible glue mistake) fails the float64 gate."""
    ws, bs, raw = synth.decoder_weights(7, raw=True)
    z = synth.latent(4, 3)
    ref, mid = np_ref.decoder(raw, bs, z)
    m0_bad = np_ref.leaky(3.0 * np_ref.mrf(raw[2:20], bs[2:20], mid["x0"], 0.1), 0.1)
    assert rel(m0_bad, mid["m0"]) > 1e-2


def test_decoder_threads_match_single():
    """The threaded driver bench.py's CPU baseline uses gives each request exactly its
    single-threaded decode."""
    import os
    ws, bs = synth.decoder_weights(31)
    zs = [synth.latent(T, 40 + T) for T in (9, 14, 11)]
    cores = sorted(os.sched_getaffinity(0))[:2]
    for use_ref in ([False, True] if ol.have_ref() else [False]):
        wavs, _ = ol.decoder_threads(ws, bs, zs, cores, use_ref=use_ref)
        for z, w in zip(zs, wavs):
            assert np.array_equal(w, ol.decoder(ws, bs, z, use_ref=use_ref))
