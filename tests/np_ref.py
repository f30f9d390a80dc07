"""Float64 NumPy restatement of the synthetic decoder from the ONNX operator definitions, written
independently of the packed layouts: conv / convTranspose by explicit index scatter (the form of
tools/export_v21.py:967-1000 conv1d_brute / conv_transpose1d_brute), the iSTFT through
numpy.fft.irfft, the window through its closed form and the PQMF synthesis as a plain conv.
It pins the C oracle from the mathematics side: a dropped term, a wrong sign or index, or a
transposed operand in the oracle shows up as a large error against this."""
from __future__ import annotations

import numpy as np


def conv1d(x, W, b, stride=1, pad=0, dil=1):
    """ONNX Conv: x [Cin][T], W [Cout][Cin][K] -> [Cout][Tout] (float64)."""
    x = np.asarray(x, np.float64)
    W = np.asarray(W, np.float64)
    cout, cin, K = W.shape
    T = x.shape[-1]
    xp = np.zeros((cin, T + 2 * pad))
    xp[:, pad:pad + T] = x
    Tout = (T + 2 * pad - dil * (K - 1) - 1) // stride + 1
    out = np.zeros((cout, Tout))
    for k in range(K):
        cols = np.arange(Tout) * stride + k * dil
        out += W[:, :, k] @ xp[:, cols]
    if b is not None:
        out += np.asarray(b, np.float64)[:, None]
    return out


def conv_transpose1d(x, W, b, stride, pad):
    """ONNX ConvTranspose: x [Cin][Tin], W [Cin][Cout][K]; output index t = q*stride + k - pad."""
    x = np.asarray(x, np.float64)
    W = np.asarray(W, np.float64)
    cin, cout, K = W.shape
    tin = x.shape[-1]
    Tout = (tin - 1) * stride - 2 * pad + K
    out = np.zeros((cout, Tout))
    for k in range(K):
        t = np.arange(tin) * stride + k - pad
        ok = (t >= 0) & (t < Tout)
        out[:, t[ok]] += W[:, :, k].T @ x[:, ok]
    if b is not None:
        out += np.asarray(b, np.float64)[:, None]
    return out


def leaky(x, a):
    return np.where(x >= 0, x, a * x)


def hann16():
    n = np.arange(16)
    return 0.5 - 0.5 * np.cos(2 * np.pi * n / 16)


def mrf(raw, bias, x, alpha):
    l0 = leaky(x, 0.1)
    outs = []
    for br, K in enumerate((3, 7, 11)):
        y = x
        for j, d in enumerate((1, 3, 5)):
            i1 = br * 6 + j * 2
            inp = l0 if j == 0 else leaky(y, 0.1)
            a = leaky(conv1d(inp, raw[i1], bias[i1], 1, d * (K - 1) // 2, d), 0.1)
            y = conv1d(a, raw[i1 + 1], bias[i1 + 1], 1, (K - 1) // 2, 1) + y
        outs.append(y)
    return leaky((outs[0] + outs[1] + outs[2]) / 3.0, alpha)


def tail(p, syn, syn_bias=None):
    """conv_post output p [72][L] -> waveform [16(L-1)] via irfft, Hann OLA and PQMF synthesis;
    syn [4][63]: the weight of the final conv (/dec/Conv), syn_bias its bias (or None)."""
    p = np.asarray(p, np.float64)
    L = p.shape[-1]
    win = hann16()
    Ly = 4 * (L - 1)
    ys = np.zeros((4, Ly))
    for band in range(4):
        mag = np.exp(p[band * 18:band * 18 + 9])
        ph = np.pi * np.sin(p[band * 18 + 9:band * 18 + 18])
        spec = mag * np.exp(1j * ph)                       # [9][L]
        frames = np.fft.irfft(spec, n=16, axis=0) * win[:, None]   # [16][L]
        ola = np.zeros(4 * (L - 1) + 16)
        wsum = np.zeros_like(ola)
        for t in range(L):
            ola[4 * t:4 * t + 16] += frames[:, t]
            wsum[4 * t:4 * t + 16] += win ** 2
        ys[band] = (ola / np.maximum(wsum, 1e-9))[8:-8]
    syn = np.asarray(syn, np.float64).reshape(4, 63)
    u = np.zeros((4, 4 * Ly))
    u[:, ::4] = 4.0 * ys
    up = np.pad(u, ((0, 0), (31, 31)))
    wav = np.zeros(4 * Ly)
    for band in range(4):
        wav += np.convolve(up[band], syn[band][::-1], mode="valid")
    if syn_bias is not None:
        wav += float(np.asarray(syn_bias).ravel()[0])
    return wav


def decoder(raw, bias, z):
    h = leaky(conv1d(z, raw[0], bias[0], 1, 3, 1), 0.1)
    x0 = conv_transpose1d(h, raw[1], bias[1], 4, 6)
    m0 = mrf(raw[2:20], bias[2:20], x0, 0.1)
    x1 = conv_transpose1d(m0, raw[20], bias[20], 4, 6)
    m1 = mrf(raw[21:39], bias[21:39], x1, 0.01)
    rp = np.concatenate([m1[:, 1:2], m1], axis=1)
    p = conv1d(rp, raw[39], bias[39], 1, 3, 1)
    return tail(p, raw[40], bias[40]), dict(h=h, x0=x0, m0=m0, x1=x1, m1=m1, p=p)


def sndr(est, ref):
    est = np.asarray(est, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    d = est - ref
    return 10 * np.log10(np.sum(ref ** 2) / max(np.sum(d ** 2), 1e-300))
