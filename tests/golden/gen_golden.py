"""Writes tests/golden/ref_conv_cases.npz: inputs and outputs of the reference's OWN CPU conv path
(pt_v21_conv_cpu / pt_v21_convT_cpu, runtime/v21/src/pt_v21_host.c:2299-2361 and 2547-2593),
compiled from the unmodified reference sources into oracle/_ref/libptref.so by oracle/Makefile.
Run here, where the reference tree exists; the GPU box has only the committed .npz.

Each case covers an edge the reference's node handlers exercise: batch > 1 (the iSTFT convs run
batch 4), cout not a multiple of 4 (cout4 padding rows), stride > 1, dilation, fused epilogues,
a convT with K not a multiple of s (partial last tap), K == s (ntap 1), zeros in the input (the
reference skips exact-zero inputs), and a NULL bias."""
from __future__ import annotations

import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
sys.path.insert(0, str(HERE.parent.parent / "prime-tts_amd"))
import oracle_lib as ol  # noqa: E402
from synth import pack_conv, pack_convtranspose  # noqa: E402

CONV_CASES = [  # batch, cin, cout, T, K, stride, pad, dil, epi0, epi1, a0, a1, bias
    (1, 8, 16, 40, 7, 1, 3, 1, 1, 0, 0.1, 0.0, True),
    (4, 16, 1, 37, 5, 1, 0, 1, 0, 0, 0.0, 0.0, False),
    (2, 5, 6, 33, 3, 2, 1, 1, 2, 3, 0.0, 0.5, True),
    (1, 12, 8, 29, 11, 1, 25, 5, 1, 4, 0.1, -0.25, True),
    (1, 4, 4, 64, 63, 1, 31, 1, 0, 0, 0.0, 0.0, False),
    (3, 7, 9, 21, 3, 3, 2, 2, 4, 1, 1.5, 0.01, True),
]
CONVT_CASES = [  # batch, cin, cout, tin, K, s, pad, bias
    (1, 8, 8, 20, 16, 4, 6, True),
    (4, 16, 1, 13, 16, 4, 0, False),
    (1, 4, 4, 17, 4, 4, 0, False),
    (2, 6, 5, 11, 7, 3, 1, True),
    (1, 3, 12, 9, 5, 2, 0, True),
]


def main():
    if not ol.have_ref():
        raise SystemExit("oracle/_ref/libptref.so missing: run make -C oracle first")
    rng = np.random.default_rng(20261201)
    out = {}
    for i, (B, cin, cout, T, K, s, pad, d, e0, e1, a0, a1, hb) in enumerate(CONV_CASES):
        x = rng.standard_normal((B, cin, T)).astype(np.float32)
        x[rng.random(x.shape) < 0.1] = 0.0
        W = (rng.standard_normal((cout, cin, K)) / np.sqrt(cin * K)).astype(np.float32)
        wp = pack_conv(W)
        b = (0.1 * rng.standard_normal(cout)).astype(np.float32) if hb else None
        y = ol.conv(x, wp, b, cout, K, s, pad, d, e0, e1, a0, a1, lib=ol.ref())
        out[f"conv{i}_x"] = x
        out[f"conv{i}_w"] = W
        out[f"conv{i}_wp"] = wp
        if b is not None:
            out[f"conv{i}_b"] = b
        out[f"conv{i}_y"] = y
        out[f"conv{i}_cfg"] = np.array([B, cin, cout, T, K, s, pad, d, e0, e1, hb], np.int64)
        out[f"conv{i}_alpha"] = np.array([a0, a1], np.float32)
    for i, (B, cin, cout, tin, K, s, pad, hb) in enumerate(CONVT_CASES):
        x = rng.standard_normal((B, cin, tin)).astype(np.float32)
        x[rng.random(x.shape) < 0.1] = 0.0
        W = (rng.standard_normal((cin, cout, K)) / np.sqrt(cin * K / s)).astype(np.float32)
        wp = pack_convtranspose(W, s)
        b = (0.1 * rng.standard_normal(cout)).astype(np.float32) if hb else None
        y = ol.convT(x, wp, b, cout, K, s, pad, lib=ol.ref())
        out[f"convT{i}_x"] = x
        out[f"convT{i}_w"] = W
        out[f"convT{i}_wp"] = wp
        if b is not None:
            out[f"convT{i}_b"] = b
        out[f"convT{i}_y"] = y
        out[f"convT{i}_cfg"] = np.array([B, cin, cout, tin, K, s, pad, hb], np.int64)
    np.savez_compressed(HERE / "ref_conv_cases.npz", **out)
    print("wrote", HERE / "ref_conv_cases.npz", len(out), "arrays")


if __name__ == "__main__":
    main()
