"""The columns a windowed decode computes (ptd_window_cols, the plan behind ptd_decode_windows):
a float64 decode of one window in which every column the plan leaves out of a launch is set to
NaN must give the kept samples finite and exactly equal to the full decode's.  A column the plan
wrongly drops poisons every kept sample that depends on it.  Host-only: the plan is computed on
the CPU, the decode is tests/np_ref.py's, masked launch by launch."""
import ctypes as C

import numpy as np
import pytest

import np_ref

HOP = 256


@pytest.fixture(scope="module")
def lib(pkg):
    return pkg.load()


@pytest.fixture(scope="module")
def model(pkg):
    ws, bs, raw = pkg.synth.decoder_weights(31, raw=True)
    return raw, bs


def plan_of(lib, T, batch, lo_first, lo, hi, hi_last):
    out = (C.c_int64 * (5 * 40))()
    rc = lib.ptd_window_cols(T, batch, lo_first, lo, hi, hi_last, out)
    return rc, np.array(out[:], np.int64).reshape(40, 5)


def item_cols(plan, i, item):
    q0, nq, el, er, _ = (int(v) for v in plan[i])
    a = q0 - el if item in ("first", "one") else q0
    b = q0 + nq + er if item in ("last", "one") else q0 + nq
    return a, b


def masked_decoder(raw, bias, z, plan, item):
    """np_ref.decoder with the columns launch i leaves out of this item set to NaN after it."""
    leaky, conv1d, convT = np_ref.leaky, np_ref.conv1d, np_ref.conv_transpose1d

    def keep(y, i):
        a, b = item_cols(plan, i, item)
        out = np.full_like(y, np.nan)
        a, b = max(a, 0), min(b, y.shape[1])
        out[:, a:b] = y[:, a:b]
        return out

    def keep_t(y, i):   # convT s4 p6 phase form: column q writes outputs 4q - 6 .. 4q - 3
        a, b = item_cols(plan, i, item)
        out = np.full_like(y, np.nan)
        lo, hi = max(4 * a - 6, 0), min(4 * b - 6, y.shape[1])
        out[:, lo:hi] = y[:, lo:hi]
        return out

    def mrf(rw, bs, x, alpha, base):
        l0 = leaky(x, 0.1)
        outs = []
        for br, K in enumerate((3, 7, 11)):
            y = x
            for j, d in enumerate((1, 3, 5)):
                i1 = br * 6 + j * 2
                inp = l0 if j == 0 else leaky(y, 0.1)
                a = keep(leaky(conv1d(inp, rw[i1], bs[i1], 1, d * (K - 1) // 2, d), 0.1),
                         base + (j * 3 + br) * 2)
                y = keep(conv1d(a, rw[i1 + 1], bs[i1 + 1], 1, (K - 1) // 2, 1) + y,
                         base + (j * 3 + br) * 2 + 1)
            outs.append(y)
        return leaky((outs[0] + outs[1] + outs[2]) / 3.0, alpha)

    h = keep(leaky(conv1d(z, raw[0], bias[0], 1, 3, 1), 0.1), 0)
    x0 = keep_t(convT(h, raw[1], bias[1], 4, 6), 1)
    m0 = mrf(raw[2:20], bias[2:20], x0, 0.1, 2)
    x1 = keep_t(convT(m0, raw[20], bias[20], 4, 6), 20)
    m1 = mrf(raw[21:39], bias[21:39], x1, 0.01, 21)
    rp = np.concatenate([m1[:, 1:2], m1], axis=1)
    p = keep(conv1d(rp, raw[39], bias[39], 1, 3, 1), 39)
    return np_ref.tail(p, raw[40], bias[40])


def check(raw, bs, z, plan, item, s0, s1, full):
    wav = masked_decoder(raw, bs, z, plan, item)
    kept = wav[s0:s1]
    assert np.all(np.isfinite(kept)), f"{item}: a kept sample reads a column the plan left out"
    assert np.array_equal(kept, full[s0:s1]), item
    return wav


# (T, lo_first, lo, hi, hi_last): the reference's 96-frame windows with 16 frames of context, its
# 48-frame first window, and bounds off the frame grid
CASES = [
    (96, 0, 16 * HOP, 80 * HOP, 96 * HOP),
    (48, 0, 16 * HOP, 32 * HOP, 32 * HOP),
    (64, 3 * HOP + 37, 9 * HOP + 5, 50 * HOP - 101, 57 * HOP + 3),
]


@pytest.mark.parametrize("case", CASES, ids=["win96", "first48", "ragged"])
def test_masked_columns_keep_the_samples(lib, model, pkg, case):
    T, lo_first, lo, hi, hi_last = case
    raw, bs = model
    z = pkg.synth.latent(T, 11).astype(np.float64)
    full, _ = np_ref.decoder(raw, bs, z)
    rc, plan = plan_of(lib, T, 3, lo_first, lo, hi, hi_last)
    assert rc == 1
    for item, s0, s1 in (("first", lo_first, hi), ("mid", lo, hi), ("last", lo, hi_last)):
        check(raw, bs, z, plan, item, s0, s1, full)
    # one window alone keeping [lo_first, hi) (the first window of a schedule)
    rc1, plan1 = plan_of(lib, T, 1, lo_first, lo, hi, hi)
    assert rc1 == 1
    check(raw, bs, z, plan1, "one", lo_first, hi, full)


def test_plan_leaves_out_columns(lib):
    """The 96/16 window's MRF-128 launches skip about a third of their columns, the plan names
    the full window's widths as the tile shape, and a middle item's columns lie inside both
    ends' columns."""
    T = 96
    rc, plan = plan_of(lib, T, 22, 0, 16 * HOP, 80 * HOP, 96 * HOP)
    assert rc == 1
    widths = [16 * T] * 18
    assert list(plan[21:39, 4]) == widths and plan[0, 4] == T and plan[1, 4] == T + 1
    assert plan[20, 4] == 4 * T + 1 and plan[39, 4] == 16 * T + 1
    frac = plan[21:39, 1].sum() / (18 * 16 * T)
    assert 0.6 < frac < 0.8, frac
    assert np.all(plan[:, 1] > 0) and np.all(plan[:, 2] >= 0) and np.all(plan[:, 3] >= 0)
    # conv_pre and ups.0 are needed whole at these window widths: K=11 at dilation 5 reaches past
    # the 16-frame context by the MRF-256 stage
    assert plan[0, 1] + plan[0, 2] + plan[0, 3] <= T


def test_plan_whole_window(lib):
    """A window that keeps every sample needs every column: no plan (rc 0, the full launches)."""
    T = 40
    rc, plan = plan_of(lib, T, 1, 0, 0, 256 * T, 256 * T)
    assert rc == 0
    assert plan[0].tolist() == [0, T, 0, 0, T]
    assert plan[1].tolist() == [1, T + 1, 0, 0, T + 1]
    assert plan[39].tolist() == [0, 16 * T + 1, 0, 0, 16 * T + 1]
    assert lib.ptd_window_cols(0, 1, 0, 0, 1, 1, (C.c_int64 * 200)()) == -1


@pytest.mark.parametrize("launch,side", [(38, "left"), (39, "right"), (21, "right")],
                         ids=["mrf128-last-c2", "conv_post", "mrf128-first-c1"])
def test_one_column_less_poisons(lib, model, pkg, launch, side):
    """The check above can fail: the same plan with one launch narrowed by one column at the edge
    its kept samples need (the last MRF-128 launch, conv_post, the first MRF-128 launch of the
    K=3 branch) leaves NaN in the kept samples."""
    T, lo, hi = 96, 16 * HOP, 80 * HOP
    raw, bs = model
    z = pkg.synth.latent(T, 11).astype(np.float64)
    rc, plan = plan_of(lib, T, 3, 0, lo, hi, 96 * HOP)
    assert rc == 1
    plan = plan.copy()
    if side == "left":
        plan[launch, 0] += 1
    plan[launch, 1] -= 1
    wav = masked_decoder(raw, bs, z, plan, "mid")
    assert not np.all(np.isfinite(wav[lo:hi]))


def test_server_widths_raised_to_two_ctx_plus_eight(lib):
    """ptd_decode_windows2 (the reference server's schedule) raises a first or later width below
    2*ctx + 8 to it (main_v21_serve.c:223-224), so its arena need equals that of the raised widths;
    ptd_decode_windows (the --stream driver's form, which takes win as given) does not."""
    T, cx = 300, 16
    low, raised = 2 * cx + 4, 2 * cx + 8
    a_low = lib.ptd_windows2_arena_bytes(T, low, 96, cx)
    assert a_low > 0 and a_low == lib.ptd_windows2_arena_bytes(T, raised, 96, cx)
    assert lib.ptd_windows2_arena_bytes(T, low, low, cx) == lib.ptd_windows2_arena_bytes(T, raised, raised, cx)
    assert lib.ptd_windows_arena_bytes(T, low, cx) != lib.ptd_windows_arena_bytes(T, raised, cx)
    assert lib.ptd_windows_arena_bytes(T, 2 * cx, cx) == 0   # below 2*ctx + 1: refused
