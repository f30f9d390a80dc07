"""Packed weight layouts and seeded synthetic decoder inputs.

The packed layouts are the contract the C entry points accept (docs/v21_layers.md:27-41 in the
reference):

* conv weight ``[Cout][Cin][K]`` -> ``[Cout4/4][K][Cin][4]``, Cout zero-padded to a multiple of 4
  (tools/export_v21.py:88-94, ``pack_conv``);
* convT weight ONNX ``[Cin][Cout][K]``, stride ``s`` -> ``s`` phases x ``ntap = ceil(K/s)`` taps,
  row ``r*C4 + c`` = phase ``r``, channel ``c``, tap ``j`` = ONNX tap ``k = r + j*s``, then packed
  like a conv: ``[s*C4/4][ntap][Cin][4]`` (tools/export_v21.py:107-121, ``pack_convtranspose``).

The synthetic decoder follows BASELINE configs 1-5: weights ~ N(0, 1/(Cin*K)) (convT:
N(0, 1/(Cin*K/4))), bias ~ N(0, 0.01), inputs ~ N(0, 1); layer geometry from the reference graph
trace (ref/v21_graph_trace.txt:3819-3935).
"""
from __future__ import annotations

import numpy as np

import pathlib

MRF_K = (3, 7, 11)
MRF_D = (1, 3, 5)
N_LAYER = 41          # 40 conv layers + the final PQMF synthesis conv (/dec/Conv)
Z_CH = 192
PQMF_FILE = pathlib.Path(__file__).resolve().parent / "data" / "v21_pqmf_synthesis.npy"


def r4(n: int) -> int:
    return (n + 3) // 4 * 4


def ntap(K: int, s: int) -> int:
    return (K + s - 1) // s


def pack_conv(W: np.ndarray) -> np.ndarray:
    """[Cout][Cin][K] -> [Cout4/4][K][Cin][4] (zero rows for the Cout..Cout4 padding)."""
    cout, cin, K = W.shape
    c4 = r4(cout)
    Wp = np.zeros((c4, cin, K), np.float32)
    Wp[:cout] = W
    return np.ascontiguousarray(Wp.reshape(c4 // 4, 4, cin, K).transpose(0, 3, 2, 1))


def unpack_conv(Wp: np.ndarray) -> np.ndarray:
    nb, K, cin, _ = Wp.shape
    return np.ascontiguousarray(Wp.transpose(0, 3, 2, 1)).reshape(nb * 4, cin, K)


def pack_convtranspose(W: np.ndarray, s: int) -> np.ndarray:
    """ONNX [Cin][Cout][K] -> [s*C4/4][ntap][Cin][4]; phase r, tap j holds ONNX tap r + j*s."""
    cin, cout, K = W.shape
    c4, nt = r4(cout), ntap(K, s)
    Wph = np.zeros((s * c4, cin, nt), np.float32)
    for r in range(s):
        for j in range(nt):
            k = r + j * s
            if k < K:
                Wph[r * c4:r * c4 + cout, :, j] = W[:, :, k].T
    return pack_conv(Wph)


def conv_out_len(T: int, K: int, stride: int, pad: int, dil: int) -> int:
    """Output length of a conv node (runtime/v21/src/pt_v21_host.c:3250)."""
    return (T + 2 * pad - (K - 1) * dil - 1) // stride + 1


def convT_out_len(tin: int, K: int, s: int, pad: int) -> int:
    """Output length of a convT node (pt_v21_host.c:3413)."""
    return (tin - 1) * s - 2 * pad + K


def dec_layer(i: int) -> dict:
    """Geometry of decoder layer i (0 conv_pre, 1 ups.0, 2..19 MRF-256, 20 ups.1, 21..38 MRF-128,
    39 conv_post).  MRF index order: branch (K 3, 7, 11), dilation (1, 3, 5), conv (c1, c2)."""
    if i == 0:
        return dict(cin=192, cout=512, K=7, s=1, d=1, pad=3, convT=False)
    if i in (1, 20):
        return dict(cin=512 if i == 1 else 256, cout=256 if i == 1 else 128, K=16, s=4, d=1,
                    pad=6, convT=True)
    if i == 39:
        return dict(cin=128, cout=72, K=7, s=1, d=1, pad=3, convT=False)
    if i == 40:   # /dec/Conv after /dec/Pad 31|31: 4 subbands -> 1, K 63, fixed weights
        return dict(cin=4, cout=1, K=63, s=1, d=1, pad=0, convT=False)
    base, C = (2, 256) if i < 20 else (21, 128)
    o = i - base
    b, j, c = o // 6, (o % 6) // 2, o % 2
    K = MRF_K[b]
    d = MRF_D[j] if c == 0 else 1
    return dict(cin=C, cout=C, K=K, s=1, d=d, pad=d * (K - 1) // 2, convT=False)


def layer_module(i: int) -> str:
    """Container module name of decoder layer i (its records are <module>.wp[#h] and <module>.b;
    spec/v21_layers.json, the dec.* packed records)."""
    fixed = {0: "dec.conv_pre", 1: "dec.ups.0", 20: "dec.ups.1", 39: "dec.subband_conv_post",
             40: "dec.Conv"}
    if i in fixed:
        return fixed[i]
    base = 2 if i < 20 else 21
    o = i - base
    return f"dec.resblocks.{o // 6 + (0 if i < 20 else 3)}.convs{o % 2 + 1}.{(o % 6) // 2}"


def tail_convT_weights():
    """ONNX weights [Cin][Cout][K] of the decoder's three fixed tail convTs (stride 4): iSTFT
    overlap-add 16 -> 1 with the delta kernel, window-sum 1 -> 1 with the squared periodic
    Hann(16), PQMF zero-insert 4 -> 4 with 4 at tap 0 (ref/v21_graph_trace.txt:3616-3617,
    :4044-4046)."""
    ola = np.zeros((16, 1, 16), np.float32)
    ola[np.arange(16), 0, np.arange(16)] = 1.0
    n = np.arange(16)
    hann = 0.5 - 0.5 * np.cos(2 * np.pi * n / 16)
    wsum = (hann * hann).astype(np.float32).reshape(1, 1, 16)
    up = np.zeros((4, 4, 4), np.float32)
    up[np.arange(4), np.arange(4), 0] = 4.0
    return {"dec.ConvTranspose": ola, "dec.ConvTranspose_1": wsum, "dec.ConvTranspose_2": up}


def conv_weights(rng: np.random.Generator, cin: int, cout: int, K: int):
    W = rng.standard_normal((cout, cin, K), dtype=np.float64) * np.sqrt(1.0 / (cin * K))
    b = rng.standard_normal(cout, dtype=np.float64) * 0.1
    return W.astype(np.float32), b.astype(np.float32)


def convT_weights(rng: np.random.Generator, cin: int, cout: int, K: int, s: int):
    W = rng.standard_normal((cin, cout, K), dtype=np.float64) * np.sqrt(1.0 / (cin * K / s))
    b = rng.standard_normal(cout, dtype=np.float64) * 0.1
    return W.astype(np.float32), b.astype(np.float32)


def pqmf_synthesis() -> np.ndarray:
    """The model's PQMF synthesis filter, /dec/Constant_134 (1, 4, 63): the weight of the
    decoder's last conv (data/v21_pqmf_synthesis.npy, decoded from the reference's
    spec/v21_layers.json by tests/golden/extract_constants.py)."""
    h = np.load(PQMF_FILE, allow_pickle=False)
    assert h.shape == (1, 4, 63) and h.dtype == np.float32
    return h


def decoder_weights(seed: int = 1234, raw: bool = False):
    """Packed weights + biases of the 41 decoder layers: the 40 convs synthetic and random-init,
    layer 40 the model's own PQMF synthesis conv (no bias).  With raw=True the ONNX-layout
    weights are returned too (conv [Cout][Cin][K], convT [Cin][Cout][K])."""
    rng = np.random.default_rng(seed)
    ws, bs, raws = [], [], []
    for i in range(N_LAYER):
        g = dec_layer(i)
        if i == 40:
            W = pqmf_synthesis()
            ws.append(pack_conv(W))
            bs.append(np.zeros(1, np.float32))
            raws.append(W)
            continue
        if g["convT"]:
            W, b = convT_weights(rng, g["cin"], g["cout"], g["K"], g["s"])
            ws.append(pack_convtranspose(W, g["s"]))
        else:
            W, b = conv_weights(rng, g["cin"], g["cout"], g["K"])
            ws.append(pack_conv(W))
        bs.append(b)
        raws.append(W)
    return (ws, bs, raws) if raw else (ws, bs)


def request_lengths(seed: int = 5, n: int = 8, lo: int = 56, hi: int = 400):
    """Config 5: per-request frame counts T ~ U[lo, hi] (integers, both ends included)."""
    rng = np.random.default_rng(seed)
    return [int(t) for t in rng.integers(lo, hi + 1, size=n)]


def latent(T: int, seed: int) -> np.ndarray:
    """Decoder input z [192][T] ~ N(0, 1)."""
    rng = np.random.default_rng(seed)
    return rng.standard_normal((Z_CH, T), dtype=np.float64).astype(np.float32)
