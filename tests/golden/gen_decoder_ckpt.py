"""Writes tests/golden/ref_decoder_ckpt.npz: the decoder's input, stage tensors and waveform as the
reference's OWN graph interpreter computes them, on the synthetic full model of tests/full_model.py.

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

Run here, where the reference tree exists and oracle/Makefile has built oracle/_ref; the GPU box
has only the committed .npz.  Inputs are deterministic: container seed 0, case seed 1, 16 tokens."""
from __future__ import annotations

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
OUT = HERE / "ref_decoder_ckpt.npz"
CONTAINER_SEED, CASE_SEED, N_TOKENS = 0, 1, 16
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


def _run(tmp: pathlib.Path, fuse: int, ckdir: pathlib.Path | None) -> np.ndarray:
    out = tmp / f"wav_fuse{fuse}.npy"
    cmd = [str(CPU_BIN), "--cpu", "--container", str(tmp / "model.ptk"), "--case", str(tmp / "case"),
           "--out", str(out)]
    if ckdir is not None:
        ckdir.mkdir()
        (tmp / "names.txt").write_text("\n".join(NAMES.values()) + "\n")
        cmd += ["--checkpoints", str(tmp / "names.txt"), "--ckdir", str(ckdir)]
    env = dict(os.environ, PT_V21_FUSE=str(fuse))
    r = subprocess.run(cmd, capture_output=True, text=True, env=env, timeout=600)
    if not out.exists():
        raise RuntimeError(f"reference driver failed:\n{r.stdout}\n{r.stderr}")
    return np.load(out).ravel()


def main():
    if not CPU_BIN.exists():
        raise SystemExit(f"{CPU_BIN} missing: run `make -C oracle` where /root/reference exists")
    with tempfile.TemporaryDirectory() as d:
        tmp = pathlib.Path(d)
        fm.write_container(tmp / "model.ptk", seed=CONTAINER_SEED)
        fm.write_case(tmp / "case", n_tokens=N_TOKENS, seed=CASE_SEED)
        ck = tmp / "ck"
        wav_unfused = _run(tmp, 0, ck)
        wav_fused = _run(tmp, 1, None)
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
    np.savez_compressed(OUT, container_seed=CONTAINER_SEED, case_seed=CASE_SEED,
                        n_tokens=N_TOKENS, **arrays)
    print(f"wrote {OUT} (T = {T} frames, {OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
