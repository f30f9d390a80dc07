"""The oracle's decoder wiring, and its overlap-save streaming, against the reference's own graph
interpreter and streaming driver.

tests/golden/ref_decoder_ckpt.npz (T = 35) and ref_decoder_ckpt_T198.npz (T = 198) hold the
decoder input, the six stage tensors and the waveform that the reference's CPU driver
(runtime/v21/src/main_v21.c with pt_v21_host.c, compiled from its sources) computed on the
synthetic full model of tests/full_model.py, dumped through its own checkpoint option, and the
waveforms its `--stream WIN CTX` mode stitched from decoder windows (main_v21.c:331-370 over
pt_v21_stream_chunk, pt_v21_host.c:2866-2902).  Script: tests/golden/gen_decoder_ckpt.py.  The
oracle's decoder (oracle/pt_oracle.c orc_decoder) is fed the same latents and the container's
dec.* records:

  - each stage (conv_pre + LeakyReLU, ups.0, MRF-256 out, ups.1, MRF-128 out, conv_post) must be
    bit-identical: whole arrays where stored, else the sha256 of the stage's float32 bytes (both
    sides run the same fp32 operations in the same order, so equality is what holds; the gate is
    1e-4 x RMS);
  - the waveform must reach >= 90 dB SNDR (the tail's exp / sin / cos and irfft products are
    summed in another order than the interpreter's einsum and Mul nodes);
  - the oracle decoded window by window and stitched by the reference driver's loop
    (oracle_lib.stream_windows) must reach >= 90 dB against each streamed waveform.  The streams
    sit 14-77 dB from the full decode, so this pins the window edges, the per-window reflect pad
    and the kept ranges.

Planted mistakes must fail the same gates: wiring errors in the oracle's inputs (two convs of an
MRF unit swapped, a branch's order of dilations reversed, a dropped bias), and stitching errors
(the full decode instead of windows, windows read one frame late, the last window not clipped to
the sequence)."""
from __future__ import annotations

import hashlib
import pathlib

import numpy as np
import pytest

import full_model as fm
import np_ref
import oracle_lib as ol

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
FIXTURES = {"T35": GOLDEN / "ref_decoder_ckpt.npz", "T198": GOLDEN / "ref_decoder_ckpt_T198.npz"}
STAGES = ["stage0", "stage1", "stage2", "stage3", "stage4", "stage5"]


def relerr(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.max(np.abs(a - b)) / max(np.sqrt(np.mean(b ** 2)), 1e-30))


def stage_matches(g, k, got) -> bool:
    """got equals the reference's stage k bit for bit (whole array, or its sha256 and samples)."""
    got = np.ascontiguousarray(got, np.float32).ravel()
    if k in g.files:
        return np.array_equal(got, g[k].ravel())
    return (hashlib.sha256(got.tobytes()).hexdigest() == str(g[k + "_sha256"])
            and np.array_equal(got[g[k + "_idx"]], g[k + "_val"]))


def stage_relerr(g, k, got) -> float:
    """max |err| / RMS against the reference's stage k (over the stored samples where the stage is
    not stored whole; the RMS is then the whole stage's)."""
    got = np.asarray(got, np.float64).ravel()
    if k in g.files:
        return relerr(got, g[k])
    d = np.max(np.abs(got[g[k + "_idx"]] - g[k + "_val"].astype(np.float64)))
    return float(d / max(float(g[k + "_rms"]), 1e-30))


@pytest.fixture(scope="module", params=list(FIXTURES))
def gold(request):
    g = np.load(FIXTURES[request.param])
    ws, bs = fm.decoder_layers(int(g["container_seed"]))
    return g, ws, bs


@pytest.fixture(scope="module")
def gold198():
    g = np.load(FIXTURES["T198"])
    ws, bs = fm.decoder_layers(int(g["container_seed"]))
    return g, ws, bs


def test_fixture_shapes(gold):
    g, _, _ = gold
    T = g["z"].shape[-1]
    assert g["z"].shape == (192, T) and T in (35, 198)
    assert g["stage5"].shape == (72, 16 * T + 1) and g["wav"].shape == (256 * T,)
    for k, n in zip(STAGES[:5], [512 * T, 1024 * T, 1024 * T, 2048 * T, 2048 * T]):
        size = g[k].size if k in g.files else int(np.prod(g[k + "_shape"]))
        assert size == n, k
    assert len(g["streams"]) == 2
    for win, cx in g["streams"]:
        assert g[f"stream_{win}_{cx}"].shape == (256 * T,)


@pytest.mark.parametrize("use_ref", [False, True], ids=["oracle_conv", "reference_conv"])
def test_oracle_decoder_matches_reference_interpreter(gold, use_ref):
    g, ws, bs = gold
    wav, st = ol.decoder(ws, bs, g["z"], stages=True, use_ref=use_ref and ol.have_ref(),
                         threads=ol.host_threads())
    for i, k in enumerate(STAGES):
        assert stage_relerr(g, k, st[i]) <= 1e-4, k
        assert stage_matches(g, k, st[i]), k
    assert np_ref.sndr(wav, g["wav"]) >= 90.0


def test_oracle_stream_matches_reference_stream(gold):
    """The oracle's windows stitched by the reference driver's loop against the driver's own
    streamed waveforms (>= 90 dB), which differ from the full decode."""
    g, ws, bs = gold
    for win, cx in g["streams"]:
        ref = g[f"stream_{win}_{cx}"]
        got = ol.decoder_stream(ws, bs, g["z"], int(win), int(cx), threads=ol.host_threads())
        assert got.shape == ref.shape
        assert np_ref.sndr(got, ref) >= 90.0, (win, cx)
        assert np_ref.sndr(g["wav"], ref) < 80.0, (win, cx)   # the stream is not the full decode


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
    wav, st = ol.decoder(mw, mb, g["z"], stages=True, threads=ol.host_threads())
    worst = max(stage_relerr(g, k, st[i]) for i, k in enumerate(STAGES))
    assert worst > 1e-4
    assert not stage_matches(g, "stage5", st[5])   # downstream of every planted mistake
    assert np_ref.sndr(wav, g["wav"]) < 60.0


def _late(z, a, w):
    """window frames read one frame late (clipped at the end of the sequence)"""
    T = z.shape[-1]
    a1 = a + 1 if a > 0 else 0
    x = np.zeros((z.shape[0], w), np.float32)
    part = z[:, a1:min(a1 + w, T)]
    x[:, :part.shape[1]] = part
    return x


def _unclipped(z, a, w, win):
    """the last window decoded over `win` frames, the frames past the sequence zero"""
    x = np.zeros((z.shape[0], win), np.float32)
    x[:, :w] = z[:, a:a + w]
    return x


STITCH_MUTATIONS = {
    "full_decode": None,
    "windows_one_frame_late": lambda ws, bs, z, a, w, win: ol.decoder(ws, bs, _late(z, a, w)),
    "last_window_unclipped": lambda ws, bs, z, a, w, win: ol.decoder(
        ws, bs, _unclipped(z, a, w, win))[:256 * w],
}


@pytest.mark.parametrize("name", list(STITCH_MUTATIONS))
def test_planted_stitching_mistakes_fail(gold198, name):
    """At T = 198 with the 96/16 windows (config 5's; the stream closest to the full decode)."""
    g, ws, bs = gold198
    z, win, cx = g["z"], 96, 16
    ref = g["stream_96_16"]
    with ol.node_threads(ol.host_threads()):
        if name == "full_decode":
            got = ol.decoder(ws, bs, z)
        else:
            fn = STITCH_MUTATIONS[name]
            got = ol.stream_stitch(lambda a, w: fn(ws, bs, z, a, w, win), z.shape[-1], win, cx)
    assert np_ref.sndr(got, ref) < 90.0
