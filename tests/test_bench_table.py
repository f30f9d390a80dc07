"""bench.py's per-launch decode table (`--layer-table`), on a synthetic rocprofv3 kernel trace:
dispatch order, the warm-up cut, per-position averages and the rates against the peaks."""
from __future__ import annotations

import csv
import importlib.util
import pathlib

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


def _bench():
    spec = importlib.util.spec_from_file_location("bench_mod", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _kernel_of(name):
    if name.startswith("branch avg"):
        # the decoder's operands are aligned: the four-wide form of the branch average
        return "avg3_leaky4_kernel(float const*, float const*, float const*, float*, long long, float)"
    if name.startswith("tail"):
        return "tail_kernel(float const*, long long, long long, long long, float*, long long)"
    return "void conv_mfma_kernel<11, 1, 0>(ConvGroup)"


def _write_trace(path, bench, ndec, us_of, extra_first=True):
    cols = ["Kind", "Agent_Id", "Queue_Id", "Stream_Id", "Thread_Id", "Dispatch_Id", "Kernel_Id",
            "Kernel_Name", "Correlation_Id", "Start_Timestamp", "End_Timestamp"]
    rows, did, t = [], 1, 1_000_000
    if extra_first:   # a weight relayout and an upload copy before the decodes: not decoder launches
        for name in ("relayout_kernel(float*, float const*, int, int, int, int, long long)",
                     "__amd_rocclr_copyBuffer"):
            rows.append([name, t, t + 5000])
            t += 10000
    for dec in range(ndec):
        for i, (name, _, _) in enumerate(bench.DECODE_LAUNCHES):
            ns = int(us_of(dec, i) * 1000)
            rows.append([_kernel_of(name), t, t + ns])
            t += ns + 1500
    # rows out of dispatch order in the file: the table must sort them
    order = list(range(len(rows)))
    order = order[1::2] + order[0::2]
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(cols)
        for k in order:
            name, t0, t1 = rows[k]
            w.writerow(["KERNEL_DISPATCH", "Agent 1", 1, 1, 7, k + 1, 3, name, k + 1, t0, t1])


@pytest.mark.parametrize("batch", [1, 8])
def test_layer_table_averages_after_warmup(tmp_path, batch):
    """The warm-up decodes (about 60 ms of load: more of them at batch 1) are cut before the
    per-position averages."""
    bench = _bench()
    n = len(bench.DECODE_LAUNCHES)
    assert n == 19
    warm = bench.decode_loop_warm(batch)
    assert warm >= 3 and (batch == 1 or warm < bench.decode_loop_warm(1))

    # warm-up decodes are 10x slower; measured decodes alternate 10 us / 30 us at position i
    def us_of(dec, i):
        base = 10.0 + i if dec % 2 == 0 else 30.0 + i
        return 10 * base if dec < warm else base

    p = tmp_path / "trace.csv"
    _write_trace(p, bench, warm + 4, us_of)
    text = bench.layer_table(str(p), batch)
    lines = [ln for ln in text.splitlines() if ln.startswith("| ") and ln[2].isdigit()]
    assert len(lines) == n
    for i, ln in enumerate(lines):
        cells = [c.strip() for c in ln.strip("|").split("|")]
        assert int(cells[0]) == i
        # decodes warm..warm+3 are even/odd alternately: mean of (10+i, 30+i) = 20+i
        assert float(cells[3]) == pytest.approx(20.0 + i, abs=0.01)
    # conv_pre: 311 MFLOP per request in 20 us
    first = [c.strip() for c in lines[0].strip("|").split("|")]
    assert first[4] == f"{batch * 2 * 512 * 192 * 7 * 226 / 20e-6 / 1e12:.1f} TFLOP/s"
    assert "sum of kernel times" in text


def test_layer_table_rejects_a_partial_decode(tmp_path):
    bench = _bench()
    p = tmp_path / "trace.csv"
    _write_trace(p, bench, 5, lambda dec, i: 10.0)
    with open(p) as f:
        body = f.read().splitlines()
    # drop one decoder dispatch: 5 * 19 - 1 is not a multiple of 19
    victim = next(k for k, ln in enumerate(body) if "tail_kernel" in ln)
    del body[victim]
    p.write_text("\n".join(body) + "\n")
    with pytest.raises(SystemExit):
        bench.layer_table(str(p), 1)


def test_layer_table_mfma_util_from_counters(tmp_path):
    """--counters: per launch position, SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 x 1024)
    averaged over the measured decodes; '-' for the launches without MFMA work."""
    bench = _bench()
    warm = bench.decode_loop_warm(1)
    trace = tmp_path / "trace.csv"
    _write_trace(trace, bench, warm + 2, lambda dec, i: 10.0)
    cols = ["Correlation_Id", "Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]
    rows, did = [], 1
    rows.append([did, did, "relayout_kernel(float*)", "GRBM_GUI_ACTIVE", 1.0])
    rows.append([did, did, "relayout_kernel(float*)", "SQ_VALU_MFMA_BUSY_CYCLES", 0.0])
    for dec in range(warm + 2):
        for i, (name, _, _) in enumerate(bench.DECODE_LAUNCHES):
            did += 1
            gui = 8000.0                       # per SIMD: 8000 / 8 = 1000 cycles
            frac = 0.9 if dec < warm else (0.2 + 0.01 * i if dec % 2 else 0.4 + 0.01 * i)
            rows.append([did, did, _kernel_of(name), "GRBM_GUI_ACTIVE", gui])
            rows.append([did, did, _kernel_of(name), "SQ_VALU_MFMA_BUSY_CYCLES", frac * 1000 * 1024])
    pmc = tmp_path / "pmc.csv"
    with open(pmc, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(cols)
        w.writerows(rows)
    text = bench.layer_table(str(trace), 1, str(pmc))
    lines = [ln for ln in text.splitlines() if ln.startswith("| ") and ln[2].isdigit()]
    assert len(lines) == len(bench.DECODE_LAUNCHES)
    for i, ln in enumerate(lines):
        cells = [c.strip() for c in ln.strip("|").split("|")]
        kind = bench.DECODE_LAUNCHES[i][1]
        if kind == "flop":
            assert float(cells[6]) == pytest.approx(100 * (0.3 + 0.01 * i), abs=0.05)
        else:
            assert cells[6] == "-"


def test_bench_refuses_more_than_one_gpu():
    """This build measures one GPU: --gpus N > 1 exits with a message before touching a device."""
    import subprocess
    import sys
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


class _FakeLib:
    """The four event calls EventTimer makes, logged in order; a call of the timed function is
    logged by the test's own fn."""

    def __init__(self):
        self.log, self.n = [], 0

    def ptd_event_create(self):
        self.n += 1
        return f"e{self.n}"

    def ptd_event_record(self, stream, e):
        self.log.append(("record", e))
        return 0

    def ptd_event_elapsed_ms(self, e0, e1):
        self.log.append(("wait", e1))
        return 1.0

    def ptd_event_destroy(self, e):
        pass


class _FakeCtx:
    ptr = "ctx"

    def __init__(self, log):
        self.log = log

    def sync(self):
        self.log.append(("sync", None))


def test_warm_keeps_the_stream_fed(monkeypatch):
    """EventTimer.warm issues the function for about WARM_MS of host time in batches of at most 16
    calls, waits only for the previous batch's end event (never drains the stream), and a timed
    call after it follows without a synchronisation."""
    bench = _bench()
    lib = _FakeLib()
    pkg = type("P", (), {"load": staticmethod(lambda: lib)})
    t = bench.EventTimer(pkg, _FakeCtx(lib.log))
    clock = [0.0]
    monkeypatch.setattr(bench.time, "perf_counter", lambda: clock[0])

    def fn():
        lib.log.append(("call", None))
        clock[0] += 0.0002      # 0.2 ms of host time per call: a batch ends at 16 calls

    t.warm(fn, ms=20.0)
    calls = [k for k, _ in lib.log if k == "call"]
    assert len(calls) >= 100                      # ~20 ms at 0.2 ms per call
    assert ("sync", None) not in lib.log
    # between two event records there are at most 16 calls, and every wait names the event
    # recorded one batch earlier
    recorded, since = [], 0
    for kind, e in lib.log:
        if kind == "call":
            since += 1
            assert since <= 16
        elif kind == "record":
            recorded.append(e)
            since = 0
        elif kind == "wait":
            assert recorded and e == recorded[-1]
    assert set(recorded) == set(t.w)
    lib.log.clear()
    ms = t.time(fn, 5, warm_ms=0.0)
    assert ms == pytest.approx(1.0 / 5)
    assert ("sync", None) not in lib.log
    # a blocker goes in after the warm-up calls and before the start event
    lib.log.clear()
    t.time(fn, 3, warmup=2, warm_ms=0.0, blocker=lambda: lib.log.append(("blocker", None)))
    kinds = [k if k != "record" else e for k, e in lib.log]
    assert kinds[:5] == ["call", "call", "blocker", t.e0, "call"]
    assert kinds[-2:] == [t.e1, "wait"]


def test_queue_table_of_a_multi_stream_trace(tmp_path):
    """--queue-table: over the last N steps, the share of the span with a kernel running, the
    kernels in flight and the kernel time per hardware queue, on a synthetic two-queue trace
    (queue 1: one 10 us kernel after another; queue 2: 30 us kernels, overlapping queue 1)."""
    bench = _bench()
    cols = ["Kind", "Queue_Id", "Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"]
    rows, did = [], 1
    for step in range(3):
        base = step * 100_000
        for i in range(2):
            rows.append(["KERNEL_DISPATCH", 1, did, "void conv_mfma_kernel<11>(ConvGroup)",
                         base + i * 10_000, base + (i + 1) * 10_000])
            did += 1
        rows.append(["KERNEL_DISPATCH", 2, did, "tail_kernel<256>(float const*)", base, base + 30_000])
        did += 1
    p = tmp_path / "trace.csv"
    with open(p, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(cols)
        w.writerows(rows)
    text = bench.queue_table(str(p), 2, per_step=3)
    assert "1: 20.0 us, 2.0" in text and "2: 30.0 us, 3" not in text
    assert "2: 30.0 us, 1.0" in text
    # steps 1 and 2 span 130 us, kernels run 60 us of it: 2 in flight for 20 us of each step
    assert "kernels running 46.2 %" in text
