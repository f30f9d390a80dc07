"""The oracle's decoder wiring against the reference's own graph interpreter.

tests/golden/ref_decoder_ckpt.npz holds the decoder input, the six stage tensors and the waveform
that the reference's CPU driver (runtime/v21/src/main_v21.c with pt_v21_host.c, compiled from its
sources) computed on the synthetic full model of tests/full_model.py, dumped through its own
checkpoint option (script: tests/golden/gen_decoder_ckpt.py).  The oracle's decoder
(oracle/pt_oracle.c orc_decoder) is fed the same latents and the container's dec.* records:

  - each stage (conv_pre + LeakyReLU, ups.0, MRF-256 out, ups.1, MRF-128 out, conv_post) must be
    bit-identical (the gate is 1e-4 x RMS; both sides run the same fp32 operations in the same
    order, so equality is what holds);
  - the waveform must reach >= 90 dB SNDR (the tail's exp / sin / cos and irfft products are
    summed in another order than the interpreter's einsum and Mul nodes).

Planted wiring mistakes in the oracle's inputs (two convs of an MRF unit swapped, a branch's
order of dilations reversed) must fail the same gates, so the fixture can tell them apart."""
from __future__ import annotations

import pathlib

import numpy as np
import pytest

import full_model as fm
import np_ref
import oracle_lib as ol

GOLD = pathlib.Path(__file__).resolve().parent / "golden" / "ref_decoder_ckpt.npz"
STAGES = ["stage0", "stage1", "stage2", "stage3", "stage4", "stage5"]


def relerr(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.max(np.abs(a - b)) / max(np.sqrt(np.mean(b ** 2)), 1e-30))


@pytest.fixture(scope="module")
def gold():
    g = np.load(GOLD)
    ws, bs = fm.decoder_layers(int(g["container_seed"]))
    return g, ws, bs


def test_fixture_shapes(gold):
    g, _, _ = gold
    T = g["z"].shape[-1]
    assert g["z"].shape == (192, T) and T == 35
    assert g["stage5"].shape == (72, 16 * T + 1) and g["wav"].shape == (256 * T,)


@pytest.mark.parametrize("use_ref", [False, True], ids=["oracle_conv", "reference_conv"])
def test_oracle_decoder_matches_reference_interpreter(gold, use_ref):
    g, ws, bs = gold
    wav, st = ol.decoder(ws, bs, g["z"], stages=True, use_ref=use_ref and ol.have_ref())
    for i, k in enumerate(STAGES):
        assert relerr(st[i], g[k]) <= 1e-4, k
        assert np.array_equal(st[i], g[k].ravel()), k
    assert np_ref.sndr(wav, g["wav"]) >= 90.0


def _swap(xs, i, j):
    xs = list(xs)
    xs[i], xs[j] = xs[j], xs[i]
    return xs


# MRF-256 layer index = 2 + 6*branch + 2*depth + conv (synth.dec_layer order)
MUTATIONS = {
    # c1 and c2 of branch K=7, dilation 3 exchanged: same shapes, wrong wiring
    "c1_c2_swapped": lambda ws, bs: (_swap(ws, 2 + 6 + 2, 2 + 6 + 3), _swap(bs, 2 + 6 + 2, 2 + 6 + 3)),
    # branch K=3 runs its dilations 5 before 1 (its c1 weights exchanged between depths 0 and 2)
    "dilations_reversed": lambda ws, bs: (_swap(ws, 2, 2 + 4), _swap(bs, 2, 2 + 4)),
    # the MRF-128 stack's first c2 bias dropped
    "bias_dropped": lambda ws, bs: (ws, [np.zeros_like(b) if i == 22 else b for i, b in enumerate(bs)]),
}


@pytest.mark.parametrize("name", list(MUTATIONS))
def test_planted_wiring_mistakes_fail(gold, name):
    g, ws, bs = gold
    mw, mb = MUTATIONS[name](ws, bs)
    wav, st = ol.decoder(mw, mb, g["z"], stages=True)
    worst = max(relerr(st[i], g[k]) for i, k in enumerate(STAGES))
    assert worst > 1e-4
    assert np_ref.sndr(wav, g["wav"]) < 60.0
