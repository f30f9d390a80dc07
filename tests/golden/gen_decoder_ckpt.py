"""Writes the reference-interpreter decoder fixtures: the decoder's input, stage tensors and
waveform as the reference's OWN graph interpreter computes them on the synthetic full model of
tests/full_model.py, plus the waveform its overlap-save streaming driver stitches from windows.

The reference's single-stream driver (runtime/v21/src/main_v21.c) is compiled from its unmodified
sources into oracle/_ref/pt_v21_cpu by oracle/Makefile (its plain CPU build).  It runs the whole
text-to-waveform graph on the synthetic container and, through its own checkpoint option
(`--checkpoints NAMES --ckdir DIR`, main_v21.c:218-219, :307-321; saved per node by ck_save,
pt_v21_host.c:2715-2747), writes these graph tensors (names from ref/v21_graph_trace.txt):

  z       /Mul_7_output_0                      conv_pre's input [192][T]            (trace :4058)
  stage0  /dec/LeakyRelu_output_0              LeakyReLU(0.1)(conv_pre) [512][T]    (:4059)
  stage1  /dec/ups.0/ConvTranspose_output_0    ups.0 [256][4T]                      (:4060)
  stage2  /dec/LeakyRelu_1_output_0            LeakyReLU(0.1)(MRF-256 sum / 3)      (:4108)
  stage3  /dec/ups.1/ConvTranspose_output_0    ups.1 [128][16T]                     (:4109)
  stage4  /dec/LeakyRelu_2_output_0            LeakyReLU(0.01)(MRF-128 sum / 3)     (:4157)
  stage5  /dec/subband_conv_post/Conv_output_0 conv_post after the reflect pad [72][16T+1]
  wav     wav                                  the waveform [256 T]                 (:4315)

PT_V21_FUSE=0 turns the interpreter's node fusion off, so every one of these tensors is
materialised (pt_v21_host.c:1277); the waveform of the default (fused) run is checked to be
identical before anything is written.

Streaming: `--stream WIN CTX` (main_v21.c:211, :225, :331-370) runs the encoder once
(pt_v21_stream_open, pt_v21_host.c:2789-2864), then the decoder on windows [a, a + WIN) clipped
to the sequence, a stepping by WIN - 2 CTX (pt_v21_stream_chunk, :2866-2902), and keeps samples
[CTX, win - CTX) frames of each window (from 0 for the first, to its end for the last).  The
stitched waveform is stored as stream_WIN_CTX; the fused and unfused runs must agree.

Two cases (container seed 0 for both):
  ref_decoder_ckpt.npz       16 tokens, case seed 1: T = 35 frames, every stage stored whole;
                             streams 16/4 and 24/8.
  ref_decoder_ckpt_T198.npz  97 tokens, case seed 97 (the drop-in test's second case):
                             T = 198 frames.  z, stage5 and wav whole; stages 0-4 as a sha256
                             digest of their float32 bytes, their RMS and 4096 values at seeded
                             flat indices (the file stays small); streams 96/16 (config 5's
                             windows) and 48/16 (the reference server's first-window width).

Run here, where the reference tree exists and oracle/Makefile has built oracle/_ref; the GPU box
has only the committed .npz files."""
from __future__ import annotations

import hashlib
import os
import pathlib
import subprocess
import sys
import tempfile

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
import full_model as fm  # noqa: E402

ROOT = HERE.parent.parent
CPU_BIN = ROOT / "oracle" / "_ref" / "pt_v21_cpu"
CONTAINER_SEED = 0
NAMES = {
    "z": "/Mul_7_output_0",
    "stage0": "/dec/LeakyRelu_output_0",
    "stage1": "/dec/ups.0/ConvTranspose_output_0",
    "stage2": "/dec/LeakyRelu_1_output_0",
    "stage3": "/dec/ups.1/ConvTranspose_output_0",
    "stage4": "/dec/LeakyRelu_2_output_0",
    "stage5": "/dec/subband_conv_post/Conv_output_0",
    "wav": "wav",
}
# name, tokens, case seed, streams (WIN, CTX), stages kept whole
CASES = [
    ("ref_decoder_ckpt.npz", 16, 1, [(16, 4), (24, 8)], list(NAMES)),
    ("ref_decoder_ckpt_T198.npz", 97, 97, [(96, 16), (48, 16)], ["z", "stage5", "wav"]),
]
N_SAMPLES = 4096


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a, np.float32).tobytes()).hexdigest()


def sample_index(n: int, key: str) -> np.ndarray:
    """The flat indices a stage's sampled values sit at: seeded by the stage name."""
    rng = np.random.default_rng(int(hashlib.sha256(key.encode()).hexdigest()[:8], 16))
    return np.sort(rng.choice(n, size=min(N_SAMPLES, n), replace=False)).astype(np.int64)


def _run(tmp: pathlib.Path, fuse: int, ckdir: pathlib.Path | None = None,
         stream: tuple[int, int] | None = None) -> np.ndarray:
    out = tmp / f"wav_fuse{fuse}_{stream}.npy"
    cmd = [str(CPU_BIN), "--cpu", "--container", str(tmp / "model.ptk"), "--case", str(tmp / "case"),
           "--out", str(out)]
    if ckdir is not None:
        ckdir.mkdir()
        (tmp / "names.txt").write_text("\n".join(NAMES.values()) + "\n")
        cmd += ["--checkpoints", str(tmp / "names.txt"), "--ckdir", str(ckdir)]
    if stream is not None:
        cmd += ["--stream", str(stream[0]), str(stream[1])]
    env = dict(os.environ, PT_V21_FUSE=str(fuse))
    r = subprocess.run(cmd, capture_output=True, text=True, env=env, timeout=600)
    if not out.exists():
        raise RuntimeError(f"reference driver failed:\n{r.stdout}\n{r.stderr}")
    return np.load(out).ravel()


def make_case(fname, n_tokens, case_seed, streams, whole):
    out = HERE / fname
    with tempfile.TemporaryDirectory() as d:
        tmp = pathlib.Path(d)
        fm.write_container(tmp / "model.ptk", seed=CONTAINER_SEED)
        fm.write_case(tmp / "case", n_tokens=n_tokens, seed=case_seed)
        ck = tmp / "ck"
        wav_unfused = _run(tmp, 0, ck)
        wav_fused = _run(tmp, 1)
        if not np.array_equal(wav_unfused, wav_fused):
            raise RuntimeError("fused and unfused reference runs differ")
        arrays = {}
        for key, name in NAMES.items():
            a = np.load(ck / (name.replace("/", "_") + ".npy"))
            assert a.dtype == np.float32, (name, a.dtype)
            arrays[key] = np.ascontiguousarray(a.reshape(a.shape[1:]) if a.shape[0] == 1 else a)
        assert np.array_equal(arrays["wav"].ravel(), wav_unfused)
        T = arrays["z"].shape[-1]
        arrays["wav"] = arrays["wav"].ravel()
        shapes = {"z": (192, T), "stage0": (512, T), "stage1": (256, 4 * T),
                  "stage2": (256, 4 * T), "stage3": (128, 16 * T),
                  "stage4": (128, 16 * T), "stage5": (72, 16 * T + 1), "wav": (256 * T,)}
        for k, s in shapes.items():
            assert arrays[k].shape == s, (k, arrays[k].shape, s)
        for win, cx in streams:
            s1 = _run(tmp, 1, stream=(win, cx))
            s0 = _run(tmp, 0, stream=(win, cx))
            if not np.array_equal(s0, s1):
                raise RuntimeError(f"fused and unfused streamed runs differ ({win}/{cx})")
            assert s1.shape == (256 * T,), s1.shape
            arrays[f"stream_{win}_{cx}"] = s1.astype(np.float32)
    keep = {}
    for k, a in arrays.items():
        if k.startswith("stage") and k not in whole:
            flat = a.ravel()
            idx = sample_index(flat.size, k)
            keep[k + "_sha256"] = np.array(digest(a))
            keep[k + "_rms"] = np.array(np.sqrt(np.mean(flat.astype(np.float64) ** 2)))
            keep[k + "_idx"] = idx
            keep[k + "_val"] = flat[idx]
            keep[k + "_shape"] = np.array(a.shape, np.int64)
        else:
            keep[k] = a
    streams_arr = np.array(streams, np.int64).reshape(-1, 2)
    np.savez_compressed(out, container_seed=CONTAINER_SEED, case_seed=case_seed,
                        n_tokens=n_tokens, streams=streams_arr, **keep)
    print(f"wrote {out} (T = {T} frames, {out.stat().st_size} bytes)")


def main():
    if not CPU_BIN.exists():
        raise SystemExit(f"{CPU_BIN} missing: run `make -C oracle` where /root/reference exists")
    for case in CASES:
        make_case(*case)


if __name__ == "__main__":
    main()
