"""The synthetic decoder driven through the reference's device ABI with host buffers, the way the
reference's graph interpreter drives the library (its conv / convT node handlers,
runtime/v21/src/pt_v21_host.c:2287-2361, :2547-2593, and the graph's decoder section,
ref/v21_graph_trace.txt:3819-4065): the 38 convs and 2 upsampling convTs up to conv_post as
pt_v21_conv / pt_v21_convT calls on host arrays, weights and biases resident in the process pool
(wtab / btab), unpadded rows (conv_pad_in = pad), the LeakyReLU after conv_pre and after each c1
conv fused as the reference's epilogue code 1, and the host ops between the calls (the LeakyReLU
ahead of a conv, residual adds, branch averages, the reflect pad) in numpy.

Three of the interpreter's modes (mode=):
  per_call  every call copies its input up and its output back (PT_V21_CHAIN=0);
  chained   the interpreter's default chain rule (pt_v21_host.c:3337-3363): a conv whose result's
            only consumer is another conv keeps it on the device (conv_keep) and that conv reads it
            there (conv_in_dev): every c1 -> c2 pair of the MRF stacks;
  resident  PT_V21_DEVADD (pt_v21_host.c:2364-2543, :3070-3097) on top of the chains: the c2
            results stay on the device for their residual Add (pt_v21_devadd_run), the residual
            stream stays there for the next depth's LeakyReLU (pt_v21_devleaky_run, after which the
            interpreter brings its input to the host, :3089) and Add (whose host operand is
            uploaded, pt_v21_dev_upload), and the branch sums run on the device, the last one
            published to the host for the Div (a host op).
lib_s accumulates the wall time spent inside library calls, so a request's time splits into the
library's share (kernels, copies, waits) and the Python glue's.

Used by the GPU tests (tests/test_gpu_abi_decoder.py) and by bench.py's PCIe-inclusive ABI leg."""
from __future__ import annotations

import ctypes as C
import time

import numpy as np

NREC = 40          # decoder layers 0..39 (convs and convTs); layer 40 is the tail's
EPI_LEAKY = 1      # the reference's epilogue code for LeakyReLU (pt_v21_host.c:2287-2297)
MODES = ("per_call", "chained", "resident")


class AbiDecoder:
    def __init__(self, pkg, ctx, ws, bs, mode="per_call"):
        assert mode in MODES, mode
        self.pkg, self.ctx, self.lib, self.mode = pkg, ctx, ctx.lib, mode
        self.host = [np.ascontiguousarray(w, np.float32) for w in ws[:NREC]] + \
                    [np.ascontiguousarray(b, np.float32) for b in bs[:NREC]]
        ptrs = (C.c_void_p * len(self.host))(*[h.ctypes.data for h in self.host])
        sizes = (C.c_size_t * len(self.host))(*[h.nbytes for h in self.host])
        if self.lib.ptd_pool_load(ctx.ptr, len(self.host), ptrs, sizes) != 0:
            raise RuntimeError("ptd_pool_load failed")
        self.pad_in0 = ctx.get_i64("conv_pad_in")
        self.calls = [0, 0]
        self.lib_s = 0.0

    def close(self):
        self.ctx.set_i64("conv_pad_in", self.pad_in0)

    def _call(self, fn, *args):
        t0 = time.perf_counter()
        r = fn(*args)
        self.lib_s += time.perf_counter() - t0
        return r

    @staticmethod
    def leaky(x, a):
        return np.where(x >= 0, x, np.float32(a) * x).astype(np.float32)

    def conv(self, x, i, cout, K, pad, dil, epi=0, a=0.0, x_dev=None, n_in=None, keep=False):
        """One conv node.  x: host [cin][T], or None with x_dev a device pointer to [cin][n_in]
        (conv_in_dev).  keep: the result stays on the device and its pointer is returned
        (conv_keep); else the host result [cout][Tout]."""
        if x_dev is None:
            x = np.ascontiguousarray(x, np.float32)
            cin, n_in = x.shape
        else:
            cin = self.host[i].size // (((cout + 3) // 4) * 4 * K)
        n = n_in + 2 * pad - dil * (K - 1)
        y = np.empty(((cout + 3) // 4 * 4, n), np.float32)
        ctx, f = self.ctx, self.pkg.fptr
        ctx.set_i64("conv_pad_in", pad)
        ctx.set_ptr("conv_in_dev", x_dev)
        ctx.set_int("conv_keep", 1 if keep else 0)
        try:
            rc = self._call(self.lib.pt_v21_conv, ctx.ptr, None if x_dev else f(x), n_in, cin, f(y),
                            n, n, cout, K, 1, pad, dil, f(self.host[i]), f(self.host[NREC + i]), 1,
                            i, NREC + i, epi, 0, a, 0.0)
            out_dev = ctx.get_ptr("conv_out_dev")
        finally:
            ctx.set_ptr("conv_in_dev", None)
            ctx.set_int("conv_keep", 0)
        if rc != 0:
            raise RuntimeError(f"pt_v21_conv layer {i} failed")
        self.calls[0] += 1
        if keep:
            if not out_dev:
                raise RuntimeError(f"pt_v21_conv layer {i} kept no device output")
            return out_dev
        return y[:cout]

    def convT(self, x, i, cout):
        x = np.ascontiguousarray(x, np.float32)
        cin, tin = x.shape
        lout = (tin - 1) * 4 - 12 + 16      # stride 4, pad 6, K 16
        y = np.empty(((cout + 3) // 4 * 4, lout), np.float32)
        f = self.pkg.fptr
        if self._call(self.lib.pt_v21_convT, self.ctx.ptr, f(x), tin, cin, tin, f(y), lout, cout, 4,
                      6, 16, f(self.host[i]), f(self.host[NREC + i]), 1, i, NREC + i) != 0:
            raise RuntimeError(f"pt_v21_convT layer {i} failed")
        self.calls[1] += 1
        return y[:cout]

    # ---- the residency calls (PT_V21_DEVADD)
    def _dev_alloc(self, n):
        p = self._call(self.lib.pt_v21_dev_alloc, self.ctx.ptr, n * 4)
        if not p:
            raise RuntimeError("pt_v21_dev_alloc failed")
        return p

    def _dev_free(self, p):
        self._call(self.lib.pt_v21_dev_free, self.ctx.ptr, p)

    def _dev_upload(self, x):
        x = np.ascontiguousarray(x, np.float32)
        p = self._call(self.lib.pt_v21_dev_upload, self.ctx.ptr, x.ctypes.data_as(C.c_void_p), x.size)
        if not p:
            raise RuntimeError("pt_v21_dev_upload failed")
        return p

    def _dev_to_host(self, p, shape):
        out = np.empty(shape, np.float32)
        self._call(self.lib.pt_v21_dev_sync_host, self.ctx.ptr, out.ctypes.data_as(C.c_void_p), p,
                   out.size)
        return out

    def _dev_add(self, a, b, n):
        y = self._dev_alloc(n)
        if self._call(self.lib.pt_v21_devadd_run, self.ctx.ptr, a, b, y, n, 0, 0.0) != 0:
            raise RuntimeError("pt_v21_devadd_run failed")
        return y

    def _dev_leaky(self, a, n, alpha):
        y = self._dev_alloc(n)
        if self._call(self.lib.pt_v21_devleaky_run, self.ctx.ptr, a, y, n, alpha) != 0:
            raise RuntimeError("pt_v21_devleaky_run failed")
        return y

    def mrf(self, x, base, C_, alpha):
        if self.mode == "resident":
            return self._mrf_resident(x, base, C_, alpha)
        chain = self.mode == "chained"
        l0 = self.leaky(x, 0.1)
        T = x.shape[-1]
        outs = []
        for br, K in enumerate((3, 7, 11)):
            y = x
            for j, d in enumerate((1, 3, 5)):
                i1 = base + br * 6 + j * 2
                a = self.conv(l0 if j == 0 else self.leaky(y, 0.1), i1, C_, K, d * (K - 1) // 2, d,
                              EPI_LEAKY, 0.1, keep=chain)
                if chain:
                    c = self.conv(None, i1 + 1, C_, K, (K - 1) // 2, 1, x_dev=a, n_in=T)
                else:
                    c = self.conv(a, i1 + 1, C_, K, (K - 1) // 2, 1)
                y = c + y
            outs.append(y)
        return self.leaky((outs[0] + outs[1] + outs[2]) / np.float32(3.0), alpha)

    def _mrf_resident(self, x, base, C_, alpha):
        T = x.shape[-1]
        n = C_ * T
        l0 = self.leaky(x, 0.1)             # x (a convT output) is not resident: a host op
        outs = []
        for br, K in enumerate((3, 7, 11)):
            y_dev, y_host = None, x
            for j, d in enumerate((1, 3, 5)):
                i1 = base + br * 6 + j * 2
                if j == 0:
                    a = self.conv(l0, i1, C_, K, d * (K - 1) // 2, d, EPI_LEAKY, 0.1, keep=True)
                else:
                    l_dev = self._dev_leaky(y_dev, n, 0.1)
                    # the interpreter then brings the leaky's input to the host (:3089), so the next
                    # Add uploads it again
                    y_host = self._dev_to_host(y_dev, (C_, T))
                    self._dev_free(y_dev)
                    a = self.conv(None, i1, C_, K, d * (K - 1) // 2, d, EPI_LEAKY, 0.1, x_dev=l_dev,
                                  n_in=T, keep=True)
                    self._dev_free(l_dev)
                c = self.conv(None, i1 + 1, C_, K, (K - 1) // 2, 1, x_dev=a, n_in=T, keep=True)
                y_dev = self._dev_add(c, self._dev_upload(y_host), n)
            outs.append(y_dev)
        s01 = self._dev_add(outs[0], outs[1], n)
        s012 = self._dev_add(s01, outs[2], n)
        for p in (outs[0], outs[1], outs[2], s01):
            self._dev_free(p)
        host = self._dev_to_host(s012, (C_, T))   # its reader, the Div, is a host op
        self._dev_free(s012)
        return self.leaky(host / np.float32(3.0), alpha)

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
