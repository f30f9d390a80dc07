"""GPU parity of the reference C-ABI entry points (pt_v21_conv / pt_v21_convT / matmul / device
residency) against the CPU oracle and the golden vectors written by the reference's own code.

Bar: max |err| <= 1e-4 x output RMS per layer.  The MFMA kernels sum
in a different order than the reference's sequential fp32 loop, so results are compared within
that tolerance, not bit for bit; the same call twice must be bit-identical (deterministic)."""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np
import pytest

import oracle_lib as ol
from conftest import ROOT, load_package

pkg = load_package()
synth = pkg.synth
GOLD = np.load(ROOT / "tests" / "golden" / "ref_conv_cases.npz")
TOL = 1e-4

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


def relerr(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    rms = np.sqrt(np.mean(b ** 2))
    return float(np.max(np.abs(a - b)) / max(rms, 1e-30))


@pytest.fixture(scope="module")
def ctx():
    c = pkg.Ctx(arena_mb=512)
    yield c
    c.close()


def gpu_conv(ctx, x, wp, bias, cout, K, stride=1, pad=0, dil=1, epi0=0, epi1=0, a0=0.0, a1=0.0,
             padded=False, wtab=-1, btab=-1, ldy_extra=0):
    """pt_v21_conv exactly as the reference interpreter calls it: unpadded rows with
    conv_pad_in = pad (the GEMM path), or zero-padded rows with conv_pad_in = -1."""
    x = np.ascontiguousarray(x, np.float32)
    if x.ndim == 2:
        x = x[None]
    B, cin, T = x.shape
    Tout = (T + 2 * pad - (K - 1) * dil - 1) // stride + 1
    c4 = (cout + 3) // 4 * 4
    if padded:
        xin = ol.pad_rows(x, pad)
        ctx.set_i64("conv_pad_in", -1)
    else:
        xin = x
        ctx.set_i64("conv_pad_in", pad)
    ldy = Tout + ldy_extra
    y = np.full((B, c4, ldy), np.nan, np.float32)
    rc = ctx.lib.pt_v21_conv(ctx.ptr, pkg.fptr(xin), xin.shape[-1], cin, pkg.fptr(y), ldy, Tout,
                             cout, K, stride, pad, dil, pkg.fptr(np.ascontiguousarray(wp)),
                             pkg.fptr(None if bias is None else np.ascontiguousarray(bias)), B,
                             wtab, btab, epi0, epi1, a0, a1)
    assert rc == 0
    return y[..., :Tout]


def gpu_convT(ctx, x, wp, bias, cout, K, s, pad, wtab=-1, btab=-1):
    x = np.ascontiguousarray(x, np.float32)
    if x.ndim == 2:
        x = x[None]
    B, cin, tin = x.shape
    Lout = (tin - 1) * s - 2 * pad + K
    c4 = (cout + 3) // 4 * 4
    y = np.full((B, c4, Lout), np.nan, np.float32)
    rc = ctx.lib.pt_v21_convT(ctx.ptr, pkg.fptr(x), tin, cin, tin, pkg.fptr(y), Lout, cout, s, pad,
                              K, pkg.fptr(np.ascontiguousarray(wp)),
                              pkg.fptr(None if bias is None else np.ascontiguousarray(bias)), B,
                              wtab, btab)
    assert rc == 0
    return y


def test_mfma_lane_layout(ctx):
    """In-bounds check of the fp32 32x32x2 MFMA builtin's operand / result lane layout."""
    say("mfma probe")
    rng = np.random.default_rng(0)
    a = rng.standard_normal((32, 2)).astype(np.float32)
    b = rng.standard_normal((2, 32)).astype(np.float32)
    d = np.zeros((32, 32), np.float32)
    assert ctx.lib.ptd_mfma_probe(ctx.ptr, pkg.fptr(a), pkg.fptr(b), pkg.fptr(d)) == 0
    assert np.allclose(d, a.astype(np.float64) @ b, atol=1e-5), d[:4, :4]


def test_mfma16_lane_layout(ctx):
    """The same for the fp32 16x16x4 builtin: lane l holds A[l % 16][l / 16], B[l / 16][l % 16] and
    result rows 4*(l / 16) + r of column l % 16 (the layout of the 16-row conv tiles)."""
    say("mfma16 probe")
    rng = np.random.default_rng(1)
    a = rng.standard_normal((16, 4)).astype(np.float32)
    b = rng.standard_normal((4, 16)).astype(np.float32)
    d = np.zeros((16, 16), np.float32)
    assert ctx.lib.ptd_mfma16_probe(ctx.ptr, pkg.fptr(a), pkg.fptr(b), pkg.fptr(d)) == 0
    assert np.allclose(d, a.astype(np.float64) @ b, atol=1e-5), d[:4, :4]


def _gold_conv_cases():
    return sorted({k.split("_")[0] for k in GOLD.files if k.startswith("conv") and not k.startswith("convT")})


@pytest.mark.parametrize("case", _gold_conv_cases())
@pytest.mark.parametrize("padded", [False, True])
def test_conv_golden(ctx, case, padded):
    B, cin, cout, T, K, s, pad, d, e0, e1, hb = GOLD[case + "_cfg"].tolist()
    a0, a1 = GOLD[case + "_alpha"].tolist()
    say(f"conv golden {case} padded={padded} cfg={GOLD[case + '_cfg'].tolist()}")
    b = GOLD[case + "_b"] if hb else None
    y = gpu_conv(ctx, GOLD[case + "_x"], GOLD[case + "_wp"], b, cout, K, s, pad, d, e0, e1, a0, a1,
                 padded=padded)
    ref = GOLD[case + "_y"]
    assert y.shape == ref.shape
    assert relerr(y, ref) < TOL


@pytest.mark.parametrize("case", sorted({k.split("_")[0] for k in GOLD.files if k.startswith("convT")}))
def test_convT_golden(ctx, case):
    B, cin, cout, tin, K, s, pad, hb = GOLD[case + "_cfg"].tolist()
    say(f"convT golden {case} cfg={GOLD[case + '_cfg'].tolist()}")
    b = GOLD[case + "_b"] if hb else None
    y = gpu_convT(ctx, GOLD[case + "_x"], GOLD[case + "_wp"], b, cout, K, s, pad)
    assert relerr(y, GOLD[case + "_y"]) < TOL


WIDE_CONV = [  # batch, cin, cout, T, K, stride, pad, dil, epi0, epi1  (MFMA path shapes)
    (1, 192, 512, 226, 7, 1, 3, 1, 1, 0),      # config 1: conv_pre + leaky
    (1, 256, 256, 904, 11, 1, 25, 5, 1, 0),    # MRF-256 K11 d5 c1
    (1, 256, 256, 904, 3, 1, 1, 1, 0, 0),      # MRF-256 K3 c2
    (1, 128, 128, 300, 7, 1, 9, 3, 1, 0),
    (1, 128, 72, 3617, 7, 1, 3, 1, 0, 0),      # conv_post shape (72 = 2.25 row blocks)
    (2, 64, 40, 97, 5, 2, 2, 1, 2, 3),         # stride 2, batch 2, cout not a multiple of 32
    (3, 33, 20, 45, 3, 1, 1, 2, 4, 1),         # odd cin, batch 3
    (1, 16, 16, 40, 1, 1, 0, 1, 0, 0),         # K = 1
    # the other graphs' convs (spec/v21_layers.json: enc, dp, flow), all through the same ABI
    (1, 192, 768, 120, 3, 1, 0, 1, 2, 0),      # enc FFN conv 1 + ReLU
    (1, 768, 192, 120, 3, 1, 0, 1, 3, 0),      # enc FFN conv 2 + mask multiply
    (1, 192, 384, 150, 5, 1, 2, 1, 0, 0),      # flow WN in-layer, K 5
    (1, 256, 1536, 64, 1, 1, 0, 1, 0, 0),      # flow 256 -> 1536 projection
    (1, 192, 96, 150, 1, 1, 0, 1, 3, 0),       # flow post, K 1 + multiply
    (1, 256, 1, 90, 1, 1, 0, 1, 3, 0),         # dp projection to one channel (SIMT path)
]


@pytest.mark.parametrize("cfg", WIDE_CONV, ids=[str(c) for c in WIDE_CONV])
def test_conv_wide_vs_oracle(ctx, cfg):
    B, cin, cout, T, K, s, pad, d, e0, e1 = cfg
    say(f"conv wide {cfg}")
    rng = np.random.default_rng(sum(cfg))
    x = rng.standard_normal((B, cin, T)).astype(np.float32)
    W = (rng.standard_normal((cout, cin, K)) / np.sqrt(cin * K)).astype(np.float32)
    b = (0.1 * rng.standard_normal(cout)).astype(np.float32)
    wp = synth.pack_conv(W)
    ref = ol.conv(x, wp, b, cout, K, s, pad, d, e0, e1, 0.1, 0.5)
    y = gpu_conv(ctx, x, wp, b, cout, K, s, pad, d, e0, e1, 0.1, 0.5)
    assert relerr(y, ref) < TOL
    y2 = gpu_conv(ctx, x, wp, b, cout, K, s, pad, d, e0, e1, 0.1, 0.5, padded=True, ldy_extra=3)
    assert relerr(y2, ref) < TOL
    y3 = gpu_conv(ctx, x, wp, b, cout, K, s, pad, d, e0, e1, 0.1, 0.5)
    assert np.array_equal(y, y3)   # deterministic


WIDE_CONVT = [  # batch, cin, cout, tin, K, s, pad
    (1, 512, 256, 226, 16, 4, 6),   # config 2: ups.0
    (1, 256, 128, 904, 16, 4, 6),   # ups.1
    (2, 64, 36, 50, 7, 3, 1),
    (1, 40, 16, 33, 4, 4, 0),       # ntap 1
]


@pytest.mark.parametrize("cfg", WIDE_CONVT, ids=[str(c) for c in WIDE_CONVT])
def test_convT_wide_vs_oracle(ctx, cfg):
    B, cin, cout, tin, K, s, pad = cfg
    say(f"convT wide {cfg}")
    rng = np.random.default_rng(sum(cfg))
    x = rng.standard_normal((B, cin, tin)).astype(np.float32)
    W = (rng.standard_normal((cin, cout, K)) / np.sqrt(cin * K / s)).astype(np.float32)
    b = (0.1 * rng.standard_normal(cout)).astype(np.float32)
    wp = synth.pack_convtranspose(W, s)
    ref = ol.convT(x, wp, b, cout, K, s, pad)
    y = gpu_convT(ctx, x, wp, b, cout, K, s, pad)
    assert relerr(y, ref) < TOL


def test_conv_empty_and_degenerate(ctx):
    say("conv empty")
    x = np.ones((1, 8, 4), np.float32)
    wp = np.ones((1, 1, 8, 4), np.float32)
    y = np.zeros((1, 4, 1), np.float32)
    ctx.set_i64("conv_pad_in", 0)
    # n = 0 and batch = 0 are no-ops that succeed
    assert ctx.lib.pt_v21_conv(ctx.ptr, pkg.fptr(x), 4, 8, pkg.fptr(y), 1, 0, 4, 1, 1, 0, 1,
                               pkg.fptr(wp), pkg.fptr(None), 1, -1, -1, 0, 0, 0.0, 0.0) == 0
    assert ctx.lib.pt_v21_conv(ctx.ptr, pkg.fptr(x), 4, 8, pkg.fptr(y), 1, 1, 4, 1, 1, 0, 1,
                               pkg.fptr(wp), pkg.fptr(None), 0, -1, -1, 0, 0, 0.0, 0.0) == 0
    # invalid geometry is an error, not a launch
    assert ctx.lib.pt_v21_conv(ctx.ptr, pkg.fptr(x), 4, 8, pkg.fptr(y), 1, 1, 4, 0, 1, 0, 1,
                               pkg.fptr(wp), pkg.fptr(None), 1, -1, -1, 0, 0, 0.0, 0.0) == -1


def test_conv_chain_keep(ctx):
    """conv_keep leaves the output on the device; the next conv reads it via conv_in_dev
    (the reference's chain, pt_v21_host.c:3337-3363); the chain's end copies back."""
    say("conv chain")
    rng = np.random.default_rng(7)
    x = rng.standard_normal((1, 64, 120)).astype(np.float32)
    W1 = (rng.standard_normal((64, 64, 3)) / 14).astype(np.float32)
    W2 = (rng.standard_normal((32, 64, 5)) / 18).astype(np.float32)
    b1 = rng.standard_normal(64).astype(np.float32)
    wp1, wp2 = synth.pack_conv(W1), synth.pack_conv(W2)
    ref1 = ol.conv(x, wp1, b1, 64, 3, 1, 1, 1, 1, 0, 0.1)
    ref2 = ol.conv(ref1, wp2, None, 32, 5, 1, 2, 1)
    used0 = ctx.get_i64("g_arena_used")
    ctx.set_int("conv_keep", 1)
    y1 = np.zeros((1, 64, 120), np.float32)
    ctx.set_i64("conv_pad_in", 1)
    assert ctx.lib.pt_v21_conv(ctx.ptr, pkg.fptr(x), 120, 64, pkg.fptr(y1), 120, 120, 64, 3, 1, 1, 1,
                               pkg.fptr(wp1), pkg.fptr(b1), 1, -1, -1, 1, 0, 0.1, 0.0) == 0
    dev = ctx.get_ptr("conv_out_dev")
    assert dev and np.all(y1 == 0)   # host copy untouched: the output stayed on the device
    ctx.set_int("conv_keep", 0)
    ctx.set_ptr("conv_in_dev", dev)
    ctx.set_i64("conv_pad_in", 2)
    y2 = np.zeros((1, 32, 120), np.float32)
    assert ctx.lib.pt_v21_conv(ctx.ptr, F_NULL(), 120, 64, pkg.fptr(y2), 120, 120, 32, 5, 1, 2, 1,
                               pkg.fptr(wp2), pkg.fptr(None), 1, -1, -1, 0, 0, 0.0, 0.0) == 0
    ctx.set_ptr("conv_in_dev", None)
    assert relerr(y2, ref2) < TOL
    assert ctx.get_ptr("chain_mark") is None
    assert ctx.get_i64("g_arena_used") == used0   # the chain end released every link


def F_NULL():
    return C.POINTER(C.c_float)()


def test_pool_resident_weights(ctx):
    """Records loaded into the weight pool (wtab/btab) give the same result as per-call weights;
    the relayout is cached per record."""
    say("pool")
    rng = np.random.default_rng(9)
    x = rng.standard_normal((1, 96, 200)).astype(np.float32)
    W = (rng.standard_normal((64, 96, 7)) / 26).astype(np.float32)
    b = rng.standard_normal(64).astype(np.float32)
    wp = synth.pack_conv(W)
    recs = [wp, b]
    ptrs = (C.c_void_p * 2)(*[r.ctypes.data for r in recs])
    sizes = (C.c_size_t * 2)(*[r.nbytes for r in recs])
    assert ctx.lib.ptd_pool_load(ctx.ptr, 2, ptrs, sizes) == 0
    assert ctx.lib.pt_v21_cuda_weights_mib(ctx.ptr) > 0
    ref = ol.conv(x, wp, b, 64, 7, 1, 3, 1)
    y_call = gpu_conv(ctx, x, wp, b, 64, 7, 1, 3, 1)
    y_res = gpu_conv(ctx, x, wp, b, 64, 7, 1, 3, 1, wtab=0, btab=1)
    y_res2 = gpu_conv(ctx, x, wp, b, 64, 7, 1, 3, 1, wtab=0, btab=1)
    assert relerr(y_res, ref) < TOL
    assert np.array_equal(y_call, y_res) and np.array_equal(y_res, y_res2)
    # a wtab whose record is too small for the call is not trusted: per-call upload instead
    y_small = gpu_conv(ctx, x, wp, b, 64, 7, 1, 3, 1, wtab=1, btab=1)
    assert np.array_equal(y_small, y_call)


@pytest.mark.parametrize("m,k,n,pad", [(37, 53, 29, 0), (120, 192, 120, 0), (120, 96, 192, 0),
                                       (70, 13, 65, 3), (5, 0, 7, 1), (1, 1, 1, 0), (65, 129, 33, 2),
                                       (3, 1000, 7, 0), (64, 8, 64, 0), (129, 7, 1, 5)])
def test_matmul(ctx, m, k, n, pad):
    """pt_v21_matmul (fp32 MFMA) against float64, with tight and padded leading dimensions
    (lda = k + pad, ldb = ldc = n + pad) and the k = 0 case (C = 0)."""
    say(f"matmul {m}x{k}x{n} pad {pad}")
    rng = np.random.default_rng(3 + m)
    lda, ldb, ldc = k + pad, n + pad, n + pad
    Af = rng.standard_normal((m, max(lda, 1))).astype(np.float32)
    Bf = rng.standard_normal((max(k, 1), ldb)).astype(np.float32)
    Cf = np.full((m, ldc), 7.0, np.float32)
    assert ctx.lib.pt_v21_matmul(ctx.ptr, pkg.fptr(Af), m, k, lda, pkg.fptr(Bf), ldb, n,
                                 pkg.fptr(Cf), ldc) == 0
    ref = Af[:, :k].astype(np.float64) @ Bf[:k, :n]
    if k == 0:
        assert np.all(Cf[:, :n] == 0.0)
    else:
        assert relerr(Cf[:, :n], ref) < 1e-5
    assert np.all(Cf[:, n:] == 7.0)   # columns past n untouched
    if ol.have_ref():
        # the reference's own CPU matmul on the same operands: same values within fp32 summation
        # order, and the same untouched padding
        Cr = ol.ref_matmul(Af, m, k, lda, Bf, ldb, n, np.full((m, ldc), 7.0, np.float32), ldc)
        if k == 0:
            assert np.array_equal(Cr, Cf)
        else:
            assert relerr(Cf[:, :n], Cr[:, :n].astype(np.float64)) < 1e-5
        assert np.all(Cr[:, n:] == 7.0)


def test_device_residency(ctx):
    """dev_upload / devadd (+fused leaky) / devleaky / dev_sync_host / dev_free / reclaim."""
    say("residency")
    rng = np.random.default_rng(4)
    a = rng.standard_normal(5000).astype(np.float32)
    b = rng.standard_normal(5000).astype(np.float32)
    lib = ctx.lib
    da = lib.pt_v21_dev_upload(ctx.ptr, a.ctypes.data, a.size)
    db = lib.pt_v21_dev_upload(ctx.ptr, b.ctypes.data, b.size)
    dy = lib.pt_v21_dev_alloc(ctx.ptr, a.nbytes)
    assert da and db and dy
    assert lib.pt_v21_devadd_run(ctx.ptr, da, db, dy, a.size, 1, 0.1) == 0
    out = np.zeros_like(a)
    lib.pt_v21_dev_sync_host(ctx.ptr, out.ctypes.data, dy, a.size)
    s = a + b
    assert np.array_equal(out, np.where(s >= 0, s, np.float32(0.1) * s))
    assert lib.pt_v21_devleaky_run(ctx.ptr, da, dy, a.size, 0.2) == 0
    lib.pt_v21_dev_sync_host(ctx.ptr, out.ctypes.data, dy, a.size)
    assert np.array_equal(out, np.where(a >= 0, a, np.float32(0.2) * a))
    lib.pt_v21_dev_free(ctx.ptr, dy)
    lib.pt_v21_dev_reclaim(ctx.ptr)
    # after the reclaim the whole slab is free again: a big block fits at the base
    p = lib.pt_v21_dev_alloc(ctx.ptr, 32 << 20)
    assert p == da
    lib.pt_v21_dev_free(ctx.ptr, p)


def test_contexts_brought_up_concurrently():
    """Eight contexts initialised at once from eight threads (the reference brings one up per
    stream thread, concurrently: pt_v21_host.c:1149-1175, main_v21_par.c:63-73); each runs a conv
    on its own stream that matches a single-threaded one bit for bit."""
    import threading
    say("8 contexts from 8 threads")
    rng = np.random.default_rng(17)
    x = rng.standard_normal((1, 64, 120)).astype(np.float32)
    W = (rng.standard_normal((48, 64, 5)) / 18).astype(np.float32)
    wp = synth.pack_conv(W)
    b = rng.standard_normal(48).astype(np.float32)
    base = pkg.Ctx(arena_mb=64)
    want = gpu_conv(base, x, wp, b, 48, 5, 1, 2, 1)
    ctxs, outs, errs = [None] * 8, [None] * 8, []
    start = threading.Barrier(8)

    def work(i):
        try:
            start.wait()
            ctxs[i] = pkg.Ctx(arena_mb=64)
            outs[i] = gpu_conv(ctxs[i], x, wp, b, 48, 5, 1, 2, 1)
        except Exception as e:   # noqa: BLE001 - reported below
            errs.append(repr(e))

    ts = [threading.Thread(target=work, args=(i,)) for i in range(8)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    for c in ctxs:
        if c is not None:
            c.close()
    base.close()
    assert not errs, errs
    for o in outs:
        assert np.array_equal(o, want)


def _random_conv_cases(n=48, seed=2024):
    """Seeded random pt_v21_conv calls: odd channel counts around the 4/8/32 tile edges, lengths
    that leave partial column tiles, strides, dilations, both row layouts, padded output rows,
    batch, and every pair of the reference's epilogue codes."""
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        B = int(rng.integers(1, 4))
        cin = int(rng.choice([2, 3, 7, 8, 9, 16, 31, 33, 64, 96, 130, 192, 257]))
        cout = int(rng.choice([1, 2, 4, 5, 15, 16, 17, 31, 32, 33, 64, 72, 100, 129, 256]))
        K = int(rng.integers(1, 12))
        dil = int(rng.integers(1, 6)) if K > 1 else 1
        stride = int(rng.choice([1, 1, 1, 2, 3]))
        pad = int(rng.integers(0, (K - 1) * dil // 2 + 2))
        T = int(rng.integers(1, 300))
        Tout = (T + 2 * pad - (K - 1) * dil - 1) // stride + 1
        if Tout < 1 or B * cin * cout * K * Tout > 3e7:
            continue
        e0, e1 = (int(v) for v in rng.integers(0, 5, 2))
        cases.append((B, cin, cout, T, K, stride, pad, dil, e0, e1, bool(rng.integers(0, 2)),
                      int(rng.choice([0, 0, 5]))))
    return cases


@pytest.mark.parametrize("cfg", _random_conv_cases(), ids=lambda c: "-".join(str(int(v)) for v in c))
def test_conv_random_vs_oracle(ctx, cfg):
    B, cin, cout, T, K, s, pad, d, e0, e1, padded, ldy_extra = cfg
    say(f"conv random {cfg}")
    rng = np.random.default_rng(abs(hash(cfg)) % (1 << 32))
    x = rng.standard_normal((B, cin, T)).astype(np.float32)
    W = (rng.standard_normal((cout, cin, K)) / np.sqrt(cin * K)).astype(np.float32)
    b = (0.1 * rng.standard_normal(cout)).astype(np.float32) if rng.integers(0, 4) else None
    wp = synth.pack_conv(W)
    ref = ol.conv(x, wp, b, cout, K, s, pad, d, e0, e1, 0.1, 0.5)
    y = gpu_conv(ctx, x, wp, b, cout, K, s, pad, d, e0, e1, 0.1, 0.5, padded=padded,
                 ldy_extra=ldy_extra)
    assert y.shape == ref.shape
    assert relerr(y, ref) < TOL


def _random_convT_cases(n=24, seed=7):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        B = int(rng.integers(1, 4))
        cin = int(rng.choice([1, 2, 5, 16, 33, 64, 130, 256]))
        cout = int(rng.choice([1, 3, 4, 16, 17, 36, 64, 128]))
        K = int(rng.integers(1, 18))
        s = int(rng.integers(1, 6))
        pad = int(rng.integers(0, K))
        tin = int(rng.integers(1, 200))
        Lout = (tin - 1) * s - 2 * pad + K
        if Lout < 1 or B * cin * cout * K * tin > 3e7:
            continue
        cases.append((B, cin, cout, tin, K, s, pad))
    return cases


@pytest.mark.parametrize("cfg", _random_convT_cases(), ids=lambda c: "-".join(str(v) for v in c))
def test_convT_random_vs_oracle(ctx, cfg):
    B, cin, cout, tin, K, s, pad = cfg
    say(f"convT random {cfg}")
    rng = np.random.default_rng(sum(cfg) * 7919)
    x = rng.standard_normal((B, cin, tin)).astype(np.float32)
    W = (rng.standard_normal((cin, cout, K)) / np.sqrt(max(cin * K / s, 1.0))).astype(np.float32)
    b = (0.1 * rng.standard_normal(cout)).astype(np.float32)
    wp = synth.pack_convtranspose(W, s)
    ref = ol.convT(x, wp, b, cout, K, s, pad)
    y = gpu_convT(ctx, x, wp, b, cout, K, s, pad)
    assert y.shape == ref.shape
    assert relerr(y, ref) < TOL


# Narrow shapes the reference interpreter hands to the ABI (cout4 < 16), and variants:
# (batch, cin, T, cout, K, stride, pad, dil, epi0, epi1, a0, a1, padded rows, bias)
NARROW_CONV = [
    (1, 4, 57856 + 62, 1, 63, 1, 0, 1, 0, 0, 0.0, 0.0, True, True),   # the PQMF synthesis FIR
    (2, 3, 500, 6, 5, 2, 2, 3, 1, 4, 0.1, 0.25, False, True),          # stride, dilation, epilogues
    (3, 8, 300, 12, 7, 1, 3, 1, 0, 0, 0.0, 0.0, False, False),         # batch, no bias
    (1, 1, 1000, 4, 11, 1, 5, 2, 2, 3, 0.0, 1.5, False, True),         # cin 1, relu then scale
    (1, 40, 700, 2, 9, 3, 4, 4, 0, 0, 0.0, 0.0, False, True),          # window past LDS: generic
]
# (batch, cin, tin, cout, K, stride, pad, bias)
NARROW_CONVT = [
    (4, 16, 3617, 1, 16, 4, 0, False),   # the iSTFT overlap-add
    (4, 1, 3617, 1, 16, 4, 0, False),    # the window sum
    (1, 4, 14464, 4, 4, 4, 0, False),    # the PQMF x4 zero-insert
    (2, 5, 300, 3, 7, 3, 2, True),       # a partial last tap (K % s != 0), padding
    (1, 70, 100, 8, 16, 4, 6, True),     # window past LDS: generic
]


@pytest.mark.parametrize("case", NARROW_CONV, ids=[f"conv{i}" for i in range(len(NARROW_CONV))])
def test_narrow_conv_matches_generic_and_oracle(ctx, case, knob_env):
    """The narrow conv kernel (input window staged in LDS, real rows only) gives the generic SIMT
    kernel's bits (PTK_NARROW=0) on the narrow ABI shapes, and both meet the oracle bar."""
    B, cin, T, cout, K, st, pad, dil, e0, e1, a0, a1, padded, with_bias = case
    say(f"narrow conv {case}")
    rng = np.random.default_rng(cin * 1000 + K)
    x = rng.standard_normal((B, cin, T)).astype(np.float32)
    W = (rng.standard_normal((cout, cin, K)) / np.sqrt(cin * K)).astype(np.float32)
    wp = synth.pack_conv(W)
    bias = (0.1 * rng.standard_normal(cout)).astype(np.float32) if with_bias else None
    args = dict(stride=st, pad=pad, dil=dil, epi0=e0, epi1=e1, a0=a0, a1=a1, padded=padded)
    knob_env.setenv("PTK_NARROW", "0")
    generic = gpu_conv(ctx, x, wp, bias, cout, K, **args)
    knob_env.delenv("PTK_NARROW")
    narrow = gpu_conv(ctx, x, wp, bias, cout, K, **args)
    assert np.all(np.isfinite(narrow))
    assert np.array_equal(narrow, generic)
    ref = ol.conv(x, wp, bias, cout, K, st, pad, dil, e0, e1, a0, a1)
    assert relerr(narrow, ref) < TOL


@pytest.mark.parametrize("case", NARROW_CONVT, ids=[f"convT{i}" for i in range(len(NARROW_CONVT))])
def test_narrow_convT_matches_generic_and_oracle(ctx, case, knob_env):
    """The narrow convT kernel (a delay-line step per thread, its s phases) gives the generic SIMT
    kernel's bits on the narrow ABI shapes, and both meet the oracle bar."""
    B, cin, tin, cout, K, st, pad, with_bias = case
    say(f"narrow convT {case}")
    rng = np.random.default_rng(cin * 100 + K + st)
    x = rng.standard_normal((B, cin, tin)).astype(np.float32)
    W = (rng.standard_normal((cin, cout, K)) * np.sqrt(st / (cin * K))).astype(np.float32)
    wp = synth.pack_convtranspose(W, st)
    bias = (0.1 * rng.standard_normal(cout)).astype(np.float32) if with_bias else None
    knob_env.setenv("PTK_NARROW", "0")
    generic = gpu_convT(ctx, x, wp, bias, cout, K, st, pad)
    knob_env.delenv("PTK_NARROW")
    narrow = gpu_convT(ctx, x, wp, bias, cout, K, st, pad)
    assert np.all(np.isfinite(narrow))
    assert np.array_equal(narrow, generic)
    ref = ol.convT(x, wp, bias, cout, K, st, pad)
    assert relerr(narrow, ref) < TOL


@pytest.mark.parametrize("n", [4, 7, 1027, 462848 + 3])
def test_elementwise_vector_and_scalar_kernels_agree(ctx, n):
    """The elementwise glue (branch average + LeakyReLU, add (+ LeakyReLU), LeakyReLU) runs four
    elements per thread on 16-byte aligned operands and one per thread otherwise: both give the
    bits of numpy's float32 arithmetic in the same order (((a + b) + c) / 3, then the slope), the
    n % 4 tail included."""
    say(f"elementwise n={n}")
    lib = ctx.lib
    VP, I64 = C.c_void_p, C.c_int64
    for name, args in (("ptk_avg3_leaky", [VP, VP, VP, VP, I64, C.c_float, VP]),
                       ("ptk_add", [VP, VP, VP, I64, C.c_int, C.c_float, VP]),
                       ("ptk_leaky", [VP, VP, I64, C.c_float, VP])):
        getattr(lib, name).argtypes = args
        getattr(lib, name).restype = C.c_int
    rng = np.random.default_rng(n)
    a, b, c = (rng.standard_normal(n).astype(np.float32) for _ in range(3))
    s = ctx.get_ptr("g_stream")
    f32 = np.float32
    alpha = f32(0.1)

    def leaky(v):
        return np.where(v >= 0, v, alpha * v).astype(np.float32)

    want = {"avg3": leaky(((a + b) + c) / f32(3.0)), "add": leaky(a + b), "add0": (a + b),
            "leaky": leaky(a)}
    for off in (0, 1):   # 0: 16-byte aligned (four per thread), 1: one float in (one per thread)
        bufs = [pkg.DevBuf(n + 1) for _ in range(4)]
        for buf, h in zip(bufs[:3], (a, b, c)):
            buf.upload(ctx, np.concatenate([np.zeros(off, np.float32), h]))
        pa, pb, pc, py = (buf.ptr + 4 * off for buf in bufs)
        got = {}
        assert lib.ptk_avg3_leaky(pa, pb, pc, py, n, alpha, s) == 0
        got["avg3"] = bufs[3].download(ctx)[off:off + n]
        assert lib.ptk_add(pa, pb, py, n, 1, alpha, s) == 0
        got["add"] = bufs[3].download(ctx)[off:off + n]
        assert lib.ptk_add(pa, pb, py, n, 0, alpha, s) == 0
        got["add0"] = bufs[3].download(ctx)[off:off + n]
        assert lib.ptk_leaky(pa, py, n, alpha, s) == 0
        got["leaky"] = bufs[3].download(ctx)[off:off + n]
        for k, v in want.items():
            assert np.array_equal(got[k].view(np.uint32), v.view(np.uint32)), (k, off)
        for buf in bufs:
            buf.free()
