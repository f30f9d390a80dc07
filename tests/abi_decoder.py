"""The synthetic decoder driven through the reference's device ABI with host buffers, the way the
reference's graph interpreter drives the library (its conv / convT node handlers,
runtime/v21/src/pt_v21_host.c:2287-2361, :2547-2593, and the graph's decoder section,
ref/v21_graph_trace.txt:3819-4065): the 38 convs and 2 upsampling convTs up to conv_post as
pt_v21_conv / pt_v21_convT calls on host arrays, weights and biases resident in the process pool
(wtab / btab), unpadded rows (conv_pad_in = pad), the LeakyReLU after conv_pre and after each c1
conv fused as the reference's epilogue code 1, and the host ops between the calls (the LeakyReLU
ahead of a conv, residual adds, branch averages, the reflect pad) in numpy.  Used by the GPU tests
(tests/test_gpu_abi_decoder.py) and by bench.py's PCIe-inclusive ABI leg."""
from __future__ import annotations

import ctypes as C

import numpy as np

NREC = 40          # decoder layers 0..39 (convs and convTs); layer 40 is the tail's
EPI_LEAKY = 1      # the reference's epilogue code for LeakyReLU (pt_v21_host.c:2287-2297)


class AbiDecoder:
    def __init__(self, pkg, ctx, ws, bs):
        self.pkg, self.ctx, self.lib = pkg, ctx, ctx.lib
        self.host = [np.ascontiguousarray(w, np.float32) for w in ws[:NREC]] + \
                    [np.ascontiguousarray(b, np.float32) for b in bs[:NREC]]
        ptrs = (C.c_void_p * len(self.host))(*[h.ctypes.data for h in self.host])
        sizes = (C.c_size_t * len(self.host))(*[h.nbytes for h in self.host])
        if self.lib.ptd_pool_load(ctx.ptr, len(self.host), ptrs, sizes) != 0:
            raise RuntimeError("ptd_pool_load failed")
        self.pad_in0 = ctx.get_i64("conv_pad_in")
        self.calls = [0, 0]

    def close(self):
        self.ctx.set_i64("conv_pad_in", self.pad_in0)

    @staticmethod
    def leaky(x, a):
        return np.where(x >= 0, x, np.float32(a) * x).astype(np.float32)

    def conv(self, x, i, cout, K, pad, dil, epi=0, a=0.0):
        x = np.ascontiguousarray(x, np.float32)
        cin, n_in = x.shape
        n = n_in + 2 * pad - dil * (K - 1)
        y = np.empty(((cout + 3) // 4 * 4, n), np.float32)
        self.ctx.set_i64("conv_pad_in", pad)
        f = self.pkg.fptr
        if self.lib.pt_v21_conv(self.ctx.ptr, f(x), n_in, cin, f(y), n, n, cout, K, 1, pad, dil,
                                f(self.host[i]), f(self.host[NREC + i]), 1, i, NREC + i, epi, 0,
                                a, 0.0) != 0:
            raise RuntimeError(f"pt_v21_conv layer {i} failed")
        self.calls[0] += 1
        return y[:cout]

    def convT(self, x, i, cout):
        x = np.ascontiguousarray(x, np.float32)
        cin, tin = x.shape
        lout = (tin - 1) * 4 - 12 + 16      # stride 4, pad 6, K 16
        y = np.empty(((cout + 3) // 4 * 4, lout), np.float32)
        f = self.pkg.fptr
        if self.lib.pt_v21_convT(self.ctx.ptr, f(x), tin, cin, tin, f(y), lout, cout, 4, 6, 16,
                                 f(self.host[i]), f(self.host[NREC + i]), 1, i, NREC + i) != 0:
            raise RuntimeError(f"pt_v21_convT layer {i} failed")
        self.calls[1] += 1
        return y[:cout]

    def mrf(self, x, base, C_, alpha):
        l0 = self.leaky(x, 0.1)
        outs = []
        for br, K in enumerate((3, 7, 11)):
            y = x
            for j, d in enumerate((1, 3, 5)):
                i1 = base + br * 6 + j * 2
                a = self.conv(l0 if j == 0 else self.leaky(y, 0.1), i1, C_, K, d * (K - 1) // 2, d,
                              EPI_LEAKY, 0.1)
                y = self.conv(a, i1 + 1, C_, K, (K - 1) // 2, 1) + y
            outs.append(y)
        return self.leaky((outs[0] + outs[1] + outs[2]) / np.float32(3.0), alpha)

    def request(self, z):
        """z [192][T] -> conv_post's output [72][16 T + 1]."""
        h = self.conv(z, 0, 512, 7, 3, 1, EPI_LEAKY, 0.1)
        m0 = self.mrf(self.convT(h, 1, 256), 2, 256, 0.1)
        m1 = self.mrf(self.convT(m0, 20, 128), 21, 128, 0.01)
        return self.conv(np.concatenate([m1[:, 1:2], m1], axis=1), 39, 72, 7, 3, 1)


def device_conv_post(pkg, ctx, model, z):
    """conv_post's output of the device-resident decoder (ptd_decode_stages) for latents z."""
    T = z.shape[-1]
    L = 16 * T + 1
    dz, dw, dp = pkg.DevBuf.of(ctx, z), pkg.DevBuf(256 * T), pkg.DevBuf(72 * L)
    arr = (C.c_void_p * 6)(None, None, None, None, None, dp.ptr)
    if ctx.lib.ptd_decode_stages(ctx.ptr, model.ptr, dz.ptr, T, dw.ptr, arr) != 0:
        raise RuntimeError("ptd_decode_stages failed")
    out = dp.download(ctx).reshape(72, L)
    for b in (dz, dw, dp):
        b.free()
    return out
