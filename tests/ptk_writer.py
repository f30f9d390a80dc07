"""Test infrastructure: writes .ptk weight containers, restating the layout the reference's
exporter writes (tools/export_v21.py:5-23 describes it, :232-255 write_ptk writes it):

  header   24 bytes, little-endian: u32 magic 0x50544B31 'PTK1', u32 version, u32 n_tensor,
           i32 reserved, i64 data_bytes
  records  n_tensor x 136 bytes: name (64 bytes, NUL-padded), i32 ndim, 4 pad bytes, i64 dim[6],
           i64 nelem, i64 offset of the payload from the data start
  padding  zeros up to the next 64-byte boundary, where the data starts
  data     each payload (fp32, or fp16 for '#h' records) padded with zeros to 64 bytes

and, as the exporter does (export_v21.py:908-911), an fp32 "dtype.table" record last: the bytes
per item of every record, in record order, itself included."""
from __future__ import annotations

import struct

import numpy as np

from conftest import load_package

synth = load_package().synth

MAGIC = 0x50544B31
HEADER = struct.Struct("<IIIiq")
RECORD = struct.Struct("<64si4x6qqq")


def pad64(n: int) -> int:
    return -(-n // 64) * 64


def payload(a: np.ndarray, itemsize: int) -> bytes:
    return (np.asarray(a).astype(np.float16) if itemsize == 2 else np.asarray(a, np.float32)).tobytes()


def write(path, tensors, version: int = 2, table: bool = True) -> None:
    """tensors: [(name, array, itemsize)], itemsize 4 (fp32) or 2 (fp16, values rounded)."""
    tensors = list(tensors)
    if table:
        tensors.append(("dtype.table",
                        np.array([float(t[2]) for t in tensors] + [4.0], np.float32), 4))
    blobs, recs, off = [], [], 0
    for name, a, isz in tensors:
        a = np.asarray(a)
        dims = list(a.shape) + [0] * (6 - a.ndim)
        recs.append(RECORD.pack(name.encode(), a.ndim, *dims, a.size, off))
        b = payload(a, isz)
        blobs.append(b + bytes(pad64(len(b)) - len(b)))
        off += len(blobs[-1])
    head = HEADER.pack(MAGIC, version, len(tensors), 0, off) + b"".join(recs)
    with open(path, "wb") as f:
        f.write(head + bytes(pad64(len(head)) - len(head)))
        for b in blobs:
            f.write(b)


def decoder_tensors(ws, bs, half: bool = True):
    """The decoder's records as the exporter names them: conv / convT weights of layers 0-38 as
    fp16 '#h' records (half=True), conv_post and the final conv in fp32, fp32 biases zero-padded to
    cout4, and the three fixed tail convTs packed like any convT."""
    out = []
    for i in range(synth.N_LAYER):
        mod = synth.layer_module(i)
        h = half and i < 39
        out.append((mod + (".wp#h" if h else ".wp"), ws[i], 2 if h else 4))
        b = np.zeros(synth.r4(synth.dec_layer(i)["cout"]), np.float32)
        b[:bs[i].size] = bs[i]
        out.append((mod + ".b", b, 4))
    for mod, W in synth.tail_convT_weights().items():
        cout = W.shape[1]
        out.append((mod + ".wp", synth.pack_convtranspose(W, 4), 4))
        out.append((mod + ".b", np.zeros(synth.r4(cout), np.float32), 4))
    return out


def half_rounded(ws):
    """The fp32 weights a container with fp16 layers 0-38 carries (what a reader must return)."""
    return [w.astype(np.float16).astype(np.float32) if i < 39 else w for i, w in enumerate(ws)]
