"""ctypes access to the CPU oracle (oracle/liboracle.so) and, where it was built, the reference's own
CPU conv path (oracle/_ref/libptref.so).  Test infrastructure: the checker, never the product."""
from __future__ import annotations

import ctypes as C
import pathlib

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent.parent
ORACLE_SO = ROOT / "oracle" / "liboracle.so"
REF_SO = ROOT / "oracle" / "_ref" / "libptref.so"

F = C.POINTER(C.c_float)
I64 = C.c_int64

CONV_ARGS = [F, I64, I64, F, I64, I64, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, F, F, I64,
             C.c_int, C.c_int, C.c_float, C.c_float]
CONVT_ARGS = [F, I64, I64, I64, F, I64, C.c_int, C.c_int, C.c_int, C.c_int, F, F, I64]


def fptr(a: np.ndarray | None):
    if a is None:
        return F()
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(F)


_oracle = None
_ref = None


def oracle():
    global _oracle
    if _oracle is None:
        lib = C.CDLL(str(ORACLE_SO))
        lib.orc_conv.argtypes = CONV_ARGS
        lib.orc_convT.argtypes = CONVT_ARGS
        lib.orc_epi.argtypes = [C.c_float, C.c_int, C.c_float]
        lib.orc_epi.restype = C.c_float
        lib.orc_decoder.argtypes = [C.c_void_p, F, I64, F, C.POINTER(F)]
        lib.orc_mrf.argtypes = [C.POINTER(F), C.POINTER(F), C.c_int, I64, F, C.c_float, F]
        lib.orc_tail.argtypes = [F, I64, F, F, F]
        lib.orc_dec_constants.argtypes = [F, F, F]
        lib.orc_dec_stage_len.argtypes = [C.c_int, I64]
        lib.orc_dec_stage_len.restype = I64
        lib.orc_set_conv_impl.argtypes = [C.c_void_p, C.c_void_p]
        lib.orc_set_threads.argtypes = [C.c_int]
        lib.orc_get_threads.restype = C.c_int
        _oracle = lib
    return _oracle


def have_ref() -> bool:
    return REF_SO.exists()


def ref():
    global _ref
    if _ref is None:
        lib = C.CDLL(str(REF_SO))
        lib.ref_conv_cpu.argtypes = CONV_ARGS
        lib.ref_convT_cpu.argtypes = CONVT_ARGS
        lib.ref_ctx_layout.argtypes = [C.POINTER(C.c_long), C.c_int]
        lib.ref_matmul_cpu.argtypes = [F, I64, I64, I64, F, I64, I64, F, I64]
        _ref = lib
    return _ref


def ref_matmul(A, m, k, lda, B, ldb, n, Cm, ldc):
    """The reference's CPU matmul (pt_v21_matmul_cpu, pt_v21_host.c:2635-2650) in place on Cm."""
    assert ref().ref_matmul_cpu(fptr(A), m, k, lda, fptr(B), ldb, n, fptr(Cm), ldc) == 0
    return Cm


def pad_rows(x: np.ndarray, pad: int) -> np.ndarray:
    """The interpreter's zero-padded conv scratch (pt_v21_host.c:3274-3281)."""
    *lead, T = x.shape
    out = np.zeros((*lead, T + 2 * pad), np.float32)
    out[..., pad:pad + T] = x
    return np.ascontiguousarray(out)


def conv(x, wp, bias, cout, K, stride=1, pad=0, dil=1, epi0=0, epi1=0, a0=0.0, a1=0.0, lib=None):
    """CPU conv over unpadded x [batch][cin][T] -> [batch][cout4][Tout], via the oracle (or lib)."""
    lib = lib or oracle()
    fn = lib.orc_conv if hasattr(lib, "orc_conv") else lib.ref_conv_cpu
    x = np.ascontiguousarray(x, np.float32)
    if x.ndim == 2:
        x = x[None]
    batch, cin, T = x.shape
    xp = pad_rows(x, pad)
    Tout = (T + 2 * pad - (K - 1) * dil - 1) // stride + 1
    c4 = (cout + 3) // 4 * 4
    y = np.zeros((batch, c4, Tout), np.float32)
    fn(fptr(xp), xp.shape[-1], cin, fptr(y), Tout, Tout, cout, K, stride, pad, dil,
       fptr(np.ascontiguousarray(wp, np.float32)),
       fptr(None if bias is None else np.ascontiguousarray(bias, np.float32)), batch, epi0, epi1,
       a0, a1)
    return y


def convT(x, wp, bias, cout, K, s, pad, lib=None):
    lib = lib or oracle()
    fn = lib.orc_convT if hasattr(lib, "orc_convT") else lib.ref_convT_cpu
    x = np.ascontiguousarray(x, np.float32)
    if x.ndim == 2:
        x = x[None]
    batch, cin, tin = x.shape
    Lout = (tin - 1) * s - 2 * pad + K
    c4 = (cout + 3) // 4 * 4
    y = np.zeros((batch, c4, Lout), np.float32)
    fn(fptr(x), tin, cin, tin, fptr(y), Lout, cout, s, pad, K,
       fptr(np.ascontiguousarray(wp, np.float32)),
       fptr(None if bias is None else np.ascontiguousarray(bias, np.float32)), batch)
    return y


N_DEC = 41   # 40 conv layers + the final PQMF synthesis conv (oracle/pt_oracle.h ORC_DEC_NLAYER)


class DecWeights(C.Structure):
    _fields_ = [("w", F * N_DEC), ("b", F * N_DEC)]


def dec_weights_struct(ws, bs):
    assert len(ws) == N_DEC and len(bs) == N_DEC
    st = DecWeights()
    for i in range(N_DEC):
        st.w[i] = fptr(ws[i])
        st.b[i] = fptr(bs[i])
    return st


class node_threads:
    """Context manager: run the oracle's batch-1 conv / convT nodes on n host threads (their
    output-channel quads split into slices; bit-identical to one thread) inside the block."""

    def __init__(self, n: int):
        self.n = int(n)

    def __enter__(self):
        self.prev = oracle().orc_get_threads()
        oracle().orc_set_threads(self.n)
        return self

    def __exit__(self, *exc):
        oracle().orc_set_threads(self.prev)
        return False


def host_threads() -> int:
    """Threads a test may use for the oracle: the cores this process may run on, at most 16 (the
    GPU box's CPU share)."""
    import os
    return max(1, min(16, len(os.sched_getaffinity(0))))


def decoder(ws, bs, z, stages=False, use_ref=False, threads=None):
    """The oracle's decoder on z [192][T]: waveform (and the six stage tensors).  threads: host
    threads per conv node (bit-identical to one; default one)."""
    if threads is not None and threads > 1:
        with node_threads(threads):
            return decoder(ws, bs, z, stages=stages, use_ref=use_ref)
    lib = oracle()
    if use_ref:
        r = ref()
        lib.orc_set_conv_impl(C.cast(r.ref_conv_cpu, C.c_void_p), C.cast(r.ref_convT_cpu, C.c_void_p))
    try:
        T = z.shape[-1]
        wav = np.zeros(256 * T, np.float32)
        st = dec_weights_struct(ws, bs)
        bufs = None
        sp = C.POINTER(F)()
        if stages:
            bufs = [np.zeros(lib.orc_dec_stage_len(i, T), np.float32) for i in range(6)]
            arr = (F * 6)(*[fptr(b) for b in bufs])
            sp = C.cast(arr, C.POINTER(F))
        rc = lib.orc_decoder(C.byref(st), fptr(np.ascontiguousarray(z, np.float32)), T, fptr(wav), sp)
        assert rc == 0
    finally:
        if use_ref:
            lib.orc_set_conv_impl(None, None)
    return (wav, bufs) if stages else wav


def decoder_threads(ws, bs, zs, cores, use_ref=False):
    """Decode the requests zs concurrently, one host thread per request, thread i pinned to
    cores[i % len(cores)] (the reference's one-thread-per-stream model, main_v21_par.c:134-140).
    The conv implementation is chosen once for all threads.  Returns (waveforms, wall seconds)."""
    import os
    import threading
    import time
    lib = oracle()
    if use_ref:
        r = ref()
        lib.orc_set_conv_impl(C.cast(r.ref_conv_cpu, C.c_void_p), C.cast(r.ref_convT_cpu, C.c_void_p))
    st = dec_weights_struct(ws, bs)
    zs = [np.ascontiguousarray(z, np.float32) for z in zs]
    wavs = [np.zeros(256 * z.shape[-1], np.float32) for z in zs]
    rcs = [None] * len(zs)
    start = threading.Barrier(len(zs) + 1)

    def work(i):
        os.sched_setaffinity(0, {cores[i % len(cores)]})   # 0 = the calling thread on Linux
        start.wait()
        rcs[i] = lib.orc_decoder(C.byref(st), fptr(zs[i]), zs[i].shape[-1], fptr(wavs[i]),
                                 C.POINTER(F)())

    ts = [threading.Thread(target=work, args=(i,)) for i in range(len(zs))]
    try:
        for t in ts:
            t.start()
        start.wait()
        t0 = time.perf_counter()
        for t in ts:
            t.join()
        dt = time.perf_counter() - t0
    finally:
        if use_ref:
            lib.orc_set_conv_impl(None, None)
    assert all(rc == 0 for rc in rcs), rcs
    return wavs, dt


def mrf(wts, bts, x, alpha, use_ref=False):
    lib = oracle()
    if use_ref:
        r = ref()
        lib.orc_set_conv_impl(C.cast(r.ref_conv_cpu, C.c_void_p), C.cast(r.ref_convT_cpu, C.c_void_p))
    try:
        C_, T = x.shape
        out = np.zeros_like(x)
        wa = (F * 18)(*[fptr(w) for w in wts])
        ba = (F * 18)(*[fptr(b) for b in bts])
        rc = lib.orc_mrf(wa, ba, C_, T, fptr(np.ascontiguousarray(x)), alpha, fptr(out))
        assert rc == 0
    finally:
        if use_ref:
            lib.orc_set_conv_impl(None, None)
    return out


def tail(p, wfir, bfir=None):
    """wfir / bfir: packed weight and bias of the final PQMF conv (decoder layer 40)."""
    lib = oracle()
    L = p.shape[-1]
    wav = np.zeros(16 * (L - 1), np.float32)
    assert lib.orc_tail(fptr(np.ascontiguousarray(p, np.float32)), L,
                        fptr(np.ascontiguousarray(wfir, np.float32)),
                        fptr(None if bfir is None else np.ascontiguousarray(bfir, np.float32)),
                        fptr(wav)) == 0
    return wav


def constants():
    hann = np.zeros(16, np.float32)
    bc = np.zeros(144, np.float32)
    bs = np.zeros(144, np.float32)
    oracle().orc_dec_constants(fptr(hann), fptr(bc), fptr(bs))
    return hann, bc.reshape(9, 16), bs.reshape(9, 16)


def stream_windows(T: int, win: int, ctx: int):
    """The windows of the reference's overlap-save driver (`--stream WIN CTX`, main_v21.c:341-362):
    window k starts at a = k * max(win - 2 ctx, 1) and spans w = min(win, T - a) frames; of its
    256 w samples it keeps [lo, hi): lo = 0 for the first window, else 256 ctx; hi = 256 w for the
    last window (a + w >= T), else min(256 (w - ctx), 256 w).  Yields (a, w, lo, hi)."""
    step = max(win - 2 * ctx, 1)
    a = 0
    while True:
        w = min(win, T - a)
        first, last = a == 0, a + w >= T
        n = 256 * w
        lo = 0 if first else 256 * ctx
        hi = n if last else min(256 * (w - ctx), n)
        yield a, w, lo, hi
        if last:
            return
        a += step


def stream_stitch(decode_window, T: int, win: int, ctx: int) -> np.ndarray:
    """Stitches decode_window(a, w) -> 256 w samples over stream_windows(T, win, ctx), keeping
    [lo, hi) of each window in order, as the reference driver's loop copies them."""
    out = []
    for a, w, lo, hi in stream_windows(T, win, ctx):
        pcm = decode_window(a, w)
        assert pcm.shape == (256 * w,)
        if hi > lo:
            out.append(pcm[lo:hi])
    return np.concatenate(out) if out else np.zeros(0, np.float32)


def decoder_stream(ws, bs, z, win: int, ctx: int, threads=None) -> np.ndarray:
    """The oracle's decoder on each window of the reference's --stream driver, stitched."""
    T = z.shape[-1]
    return stream_stitch(lambda a, w: decoder(ws, bs, np.ascontiguousarray(z[:, a:a + w]),
                                              threads=threads), T, win, ctx)
