"""Test infrastructure: a synthetic full PrimeTTS v2.1 model as a .ptk container, and an input case,
for running the reference's own driver (main_v21.c) end to end, once as its CPU build and once
linked against libptconv_hip.so.

Every record of tests/golden/v21_records.json is written under its name, shape and width:
  - model constants keep the model's values;
  - the decoder's fixed tail convTs (overlap-add delta, window-sum Hann^2, PQMF zero-insert) and
    its PQMF synthesis filter keep their real forms;
  - everything else is seeded random init at the usual scales: conv / convT weights
    N(0, 1/fan_in), biases N(0, 0.05^2), LayerNorm 1 + N(0, 0.05^2) / N(0, 0.05^2), embeddings
    N(0, 1/192), relative-position tables N(0, 1/96).
The case is the graph's seven feeds (x, tone, lang, x_lengths, sid, noise_scale = 0,
length_scale = 1), as the reference's goldens use them (tests/golden_v21/MANIFEST.json)."""
from __future__ import annotations

import json
import pathlib

import numpy as np

import ptk_writer as pw

synth = pw.synth
MANIFEST = pathlib.Path(__file__).resolve().parent / "golden" / "v21_records.json"
TAIL_FORMS = {"dec.ConvTranspose.wp": "dec.ConvTranspose", "dec.ConvTranspose_1.wp": "dec.ConvTranspose_1",
              "dec.ConvTranspose_2.wp": "dec.ConvTranspose_2"}


def records():
    return json.loads(MANIFEST.read_text())["records"]


def _weight(rec, rng):
    name, cin, cout, K, s = rec["name"], rec["cin"], rec["cout"], rec["K"], rec["stride"]
    if name in TAIL_FORMS:
        W = synth.tail_convT_weights()[TAIL_FORMS[name]]
        return synth.pack_convtranspose(W, s)
    if name == "dec.Conv.wp":
        return synth.pack_conv(synth.pqmf_synthesis())
    if rec["convT"]:
        W = rng.standard_normal((cin, cout, K)) * np.sqrt(s / (cin * K))
        return synth.pack_convtranspose(W.astype(np.float32), s)
    W = rng.standard_normal((cout, cin, K)) * np.sqrt(1.0 / (cin * K))
    return synth.pack_conv(W.astype(np.float32))


def tensors(seed: int = 0):
    """[(name, array, itemsize)] for every record, in the graph's constant-table order."""
    rng = np.random.default_rng(seed)
    out = []
    for rec in records():
        role, shape = rec["role"], tuple(rec["shape"])
        if role == "const":
            a = np.asarray(rec["values"], np.float32).reshape(shape)
        elif role == "w":
            a = _weight(rec, rng)
            assert a.shape == shape, (rec["name"], a.shape, shape)
        elif role == "b":
            fixed = rec["name"].startswith(("dec.ConvTranspose", "dec.Conv."))
            a = np.zeros(shape, np.float32) if fixed else (0.05 * rng.standard_normal(shape)).astype(np.float32)
        elif role == "ln_g":
            a = (1.0 + 0.05 * rng.standard_normal(shape)).astype(np.float32)
        elif role == "ln_b":
            a = (0.05 * rng.standard_normal(shape)).astype(np.float32)
        elif role == "emb":
            a = (rng.standard_normal(shape) / np.sqrt(192.0)).astype(np.float32)
        elif role == "relpos":
            a = (rng.standard_normal(shape) / np.sqrt(96.0)).astype(np.float32)
        else:
            raise ValueError(rec)
        out.append((rec["name"], a, rec["isz"]))
    return out


def write_container(path, seed: int = 0) -> None:
    pw.write(path, tensors(seed))


def decoder_layers(seed: int = 0):
    """The 41 decoder layers (synth.dec_layer order) of the container write_container(seed)
    writes, as any reader of it sees them: packed weights with fp16 records expanded to fp32,
    biases cut to cout.  Returns (ws, bs)."""
    recs = {name: (a, isz) for name, a, isz in tensors(seed)}
    ws, bs = [], []
    for i in range(synth.N_LAYER):
        mod = synth.layer_module(i)
        a, isz = recs[mod + ".wp#h"] if mod + ".wp#h" in recs else recs[mod + ".wp"]
        if isz == 2:
            a = a.astype(np.float16).astype(np.float32)
        ws.append(np.ascontiguousarray(a, np.float32))
        b, _ = recs[mod + ".b"]
        bs.append(np.ascontiguousarray(b[:synth.dec_layer(i)["cout"]], np.float32))
    return ws, bs


def write_case(case_dir, n_tokens: int = 40, seed: int = 0, sid: int = 0) -> None:
    """The seven graph feeds of one request (ids interleaved with blanks, as add_blank does) and a
    one-sample placeholder wav.npy for the driver's parity print."""
    d = pathlib.Path(case_dir)
    d.mkdir(parents=True, exist_ok=True)
    rng = np.random.default_rng(seed)
    ids = rng.integers(1, 88, n_tokens)
    ids[::2] = 0
    feeds = {
        "x": ids.reshape(1, -1).astype(np.int64),
        "tone": rng.integers(0, 6, (1, n_tokens)).astype(np.int64),
        "lang": np.zeros((1, n_tokens), np.int64),
        "x_lengths": np.array([n_tokens], np.int64),
        "sid": np.array([sid], np.int64),
        "noise_scale": np.array([0.0], np.float32),
        "length_scale": np.array([1.0], np.float32),
        "wav": np.zeros((1, 1, 1), np.float32),
    }
    for k, v in feeds.items():
        np.save(d / f"{k}.npy", v)
