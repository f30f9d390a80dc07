"""The drop-in, end to end: the reference's own single-stream driver (runtime/v21/src/main_v21.c
with its graph interpreter pt_v21_host.c, compiled from the reference sources by oracle/Makefile)
runs a synthetic full PrimeTTS v2.1 model twice: as the reference's CPU build, and compiled with
-DPT_V21_CUDA and linked against libptconv_hip.so, so that every conv, convT and matmul of the
graph goes through this library's C ABI on the MI355X.  The device build must reproduce the CPU
build's waveform: the driver's own parity gate (SNDR >= 60 dB, main_v21.c) and the same check
here.  The reference's multi-stream driver (main_v21_par.c) then runs eight concurrent streams,
each bringing up its own context on its own thread against one shared weight pool, under the
same gate.  Skipped where oracle/_ref was not built (the reference tree is absent)."""
from __future__ import annotations

import re
import shutil
import subprocess
import sys

import numpy as np
import pytest

import full_model as fm
import np_ref
from conftest import ROOT

REF = ROOT / "oracle" / "_ref"
CPU_BIN, DEV_BIN, PAR_BIN = REF / "pt_v21_cpu", REF / "pt_v21_mi355x", REF / "pt_v21_par_mi355x"
pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not (CPU_BIN.exists() and DEV_BIN.exists()),
                                 reason="oracle/_ref driver builds absent (reference tree not present)")]


def say(msg):
    print(f"[gpu dropin] {msg}", file=sys.stderr, flush=True)


def _run(cmd, timeout, env=None):
    import os
    full_env = dict(os.environ, **(env or {}))
    r = subprocess.run([str(x) for x in cmd], capture_output=True, text=True, timeout=timeout,
                       env=full_env)
    for line in (r.stdout + r.stderr).splitlines()[-8:]:
        say(line)
    return r


@pytest.fixture(scope="module", params=[40, 97], ids=lambda n: f"{n}tok")
def model(tmp_path_factory, request):
    """A synthetic full model, a 40- or 97-token case (different frame counts through the whole
    graph), and the reference CPU build's waveform for it (stored as the case's wav.npy, which
    the drivers compare against)."""
    n_tokens = request.param
    d = tmp_path_factory.mktemp(f"dropin{n_tokens}")
    say(f"synthetic full model + {n_tokens}-token case")
    fm.write_container(d / "model.ptk", seed=0)
    case = d / "case"
    fm.write_case(case, n_tokens=n_tokens, seed=n_tokens)
    cpu_wav = d / "cpu.npy"
    say("reference CPU build")
    _run([CPU_BIN, "--cpu", "--container", d / "model.ptk", "--case", case, "--out", cpu_wav], 600)
    assert cpu_wav.exists()
    shutil.copy(cpu_wav, case / "wav.npy")
    return d, case, cpu_wav


# the host's own switches (pt_v21_host.c): defaults (epilogue fusion and conv chains on), device
# residency for the residual adds and activations on (PT_V21_DEVADD, :2364-2543), and fusion and
# chaining off (every conv a plain call, every Add / LeakyRelu a host op)
HOST_MODES = {"default": {}, "devadd": {"PT_V21_DEVADD": "1"},
              "unfused": {"PT_V21_FUSE": "0", "PT_V21_CHAIN": "0"}}


@pytest.mark.parametrize("mode", list(HOST_MODES))
def test_reference_driver_through_the_library(model, tmp_path, mode):
    d, case, cpu_wav = model
    dev_wav = tmp_path / "dev.npy"
    say(f"reference driver linked against libptconv_hip.so, host mode {mode}")
    r = _run([DEV_BIN, "--container", d / "model.ptk", "--case", case, "--out", dev_wav], 300,
             HOST_MODES[mode])
    assert r.returncode == 0, "the driver's own gate (SNDR >= 60 dB against the CPU build) failed"
    a, b = np.load(dev_wav).ravel(), np.load(cpu_wav).ravel()
    assert a.shape == b.shape and a.size > 10000
    assert np_ref.sndr(a, b) >= 60.0
    # every conv / convT / matmul of the graph went through the library
    m = re.search(r"conv=(\d+) convT=(\d+) matmul=(\d+)", r.stdout)
    assert m and tuple(int(v) for v in m.groups()) == (124, 5, 50), r.stdout
    assert "pt_v21 hip: context ready" in r.stderr


# PT_V21_GPU, the reference's per-op bisection switch (pt_v21_cuda.cu:70-76; substring test, so
# "conv" keeps conv and drops convT): the ops it leaves out run on the host's CPU path
ROUTES = {"matmul_only": ("matmul", {"conv", "convT"}), "conv_only": ("conv", {"convT"})}


@pytest.mark.parametrize("route", list(ROUTES))
def test_reference_driver_per_op_routing(model, tmp_path, route):
    """With convs routed to the CPU path the library answers pt_v21_conv_pads_in_kernel = 0, so the
    host pads rows and chains nothing, and the host's CPU conv gets the rows it expects; the
    waveform still passes the driver's gate.  The routed ops take host-CPU time (the device path
    needs a few ms for the whole graph), which shows they really ran there."""
    d, case, cpu_wav = model
    value, on_cpu = ROUTES[route]
    say(f"reference driver with PT_V21_GPU={value}")
    r = _run([DEV_BIN, "--container", d / "model.ptk", "--case", case, "--out", tmp_path / "w.npy"],
             600, {"PT_V21_GPU": value})
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    a, b = np.load(tmp_path / "w.npy").ravel(), np.load(cpu_wav).ravel()
    assert a.shape == b.shape and np_ref.sndr(a, b) >= 60.0
    m = re.search(r"conv=(\d+) convT=(\d+) matmul=(\d+)\s+conv ([0-9.]+) ms\s+convT ([0-9.]+) ms", r.stdout)
    assert m, r.stdout[-2000:]
    assert tuple(int(v) for v in m.groups()[:3]) == (124, 5, 50)
    conv_ms, convT_ms = float(m.group(4)), float(m.group(5))
    say(f"conv {conv_ms} ms, convT {convT_ms} ms")
    assert (conv_ms > 100.0) == ("conv" in on_cpu)
    assert (convT_ms > 20.0) == ("convT" in on_cpu)


def test_reference_driver_gpu_split(model, tmp_path):
    """PT_V21_CUDAPROF=1, the reference's phase profiler: the linked driver prints its own
    "gpu split" line from the context fields this library fills (alloc / copy / kernel+sync /
    free per call, the device synchronised between phases), the phases are all non-negative, the
    uploads and the kernels take time, and their sum stays within the driver's own total for the
    conv / convT / matmul calls.  The waveform still passes the driver's gate."""
    d, case, _ = model
    say("reference driver with PT_V21_CUDAPROF=1")
    r = _run([DEV_BIN, "--container", d / "model.ptk", "--case", case, "--out", tmp_path / "w.npy"],
             300, {"PT_V21_CUDAPROF": "1"})
    assert r.returncode == 0
    m = re.search(r"gpu split: alloc ([0-9.]+) ms\s+copy ([0-9.]+) ms\s+kernel\+sync ([0-9.]+) ms"
                  r"\s+free ([0-9.]+) ms", r.stderr)
    assert m, r.stderr[-2000:]
    alloc, copy, kern, free = (float(v) for v in m.groups())
    say(f"gpu split: alloc {alloc} copy {copy} kernel+sync {kern} free {free} ms")
    assert min(alloc, copy, kern, free) >= 0.0 and copy > 0.0 and kern > 0.0
    t = re.search(r"conv ([0-9.]+) ms\s+convT ([0-9.]+) ms\s+matmul ([0-9.]+) ms", r.stdout)
    assert t, r.stdout[-2000:]
    total = sum(float(v) for v in t.groups())
    assert alloc + copy + kern + free <= total * 1.05 + 1.0


CONV_NODES = ROOT / "tests" / "golden" / "v21_conv_nodes.json"


def test_reference_driver_every_conv_node(model, tmp_path):
    """The reference's C-runtime parity method (a checkpoint of every node, tests/v21_parity_c.py)
    on the conv path: both builds of the reference driver run the case with the interpreter's node
    fusion and device chaining off (PT_V21_FUSE=0, PT_V21_CHAIN=0: every conv and convT output
    is materialised on the host) and dump, through the driver's checkpoint option
    (main_v21.c:307-321), the output of each of the graph's 124 conv and 5 convT nodes
    (tests/golden/v21_conv_nodes.json, from the reference's generated node table).  Each node of
    the build linked against the library must be within 1e-4 x RMS of the CPU build's, with the
    differences of every node before it carried along (encoder, flow and decoder, the device
    matmuls included)."""
    import json
    d, case, _ = model
    names = [n["name"] for n in json.loads(CONV_NODES.read_text())["nodes"]]
    (tmp_path / "names.txt").write_text("\n".join(names) + "\n")
    env = {"PT_V21_FUSE": "0", "PT_V21_CHAIN": "0"}
    runs = {}
    for label, binary, extra in (("cpu", CPU_BIN, ["--cpu"]), ("dev", DEV_BIN, [])):
        ck = tmp_path / f"ck_{label}"
        ck.mkdir()
        say(f"reference driver ({label} build) with checkpoints of {len(names)} conv nodes")
        r = _run([binary, *extra, "--container", d / "model.ptk", "--case", case, "--out",
                  tmp_path / f"{label}.npy", "--checkpoints", tmp_path / "names.txt", "--ckdir", ck],
                 600, env)
        assert (tmp_path / f"{label}.npy").exists(), r.stdout[-2000:] + r.stderr[-2000:]
        runs[label] = ck
    worst, rows = 0.0, []
    for nm in names:
        f = nm.replace("/", "_") + ".npy"
        a = np.load(runs["dev"] / f).astype(np.float64).ravel()
        b = np.load(runs["cpu"] / f).astype(np.float64).ravel()
        assert a.shape == b.shape, nm
        e = float(np.max(np.abs(a - b)) / max(np.sqrt(np.mean(b ** 2)), 1e-30))
        rows.append((e, nm))
        worst = max(worst, e)
    rows.sort(reverse=True)
    for e, nm in rows[:5]:
        say(f"  {nm}: max|err|/rms = {e:.3g}")
    say(f"{len(names)} conv / convT nodes, worst max|err|/rms {worst:.3g}, median {rows[len(rows) // 2][0]:.3g}")
    assert worst <= 1e-4, rows[:5]


STREAM_FIXTURE = ROOT / "tests" / "golden" / "ref_decoder_ckpt_T198.npz"


@pytest.mark.parametrize("win,cx", [(96, 16), (48, 16)])
def test_reference_stream_driver_through_the_library(model, tmp_path, win, cx):
    """The reference's overlap-save streaming path (`--stream WIN CTX`: pt_v21_stream_open runs
    the encoder once, then pt_v21_stream_chunk the decoder's convs and convTs on each window,
    main_v21.c:331-370, pt_v21_host.c:2789-2902) with the library as its device: the stitched
    waveform against what the reference's CPU build stitched on the same case (for the 97-token
    case the committed tests/golden/ref_decoder_ckpt_T198.npz, written by
    tests/golden/gen_decoder_ckpt.py on the same container and case; for the 40-token case the CPU
    build run here in stream mode), >= 60 dB and closer to it than to the full decode."""
    d, case, cpu_wav = model
    g = np.load(STREAM_FIXTURE)
    full = np.load(cpu_wav).ravel()
    if int(np.load(case / "x_lengths.npy")[0]) == int(g["n_tokens"]):
        assert np.array_equal(full, g["wav"])   # the same container and case as the fixture
        ref = g[f"stream_{win}_{cx}"]
    else:
        say(f"reference CPU build --stream {win} {cx}")
        rc = _run([CPU_BIN, "--cpu", "--container", d / "model.ptk", "--case", case, "--out",
                   tmp_path / "cpu_s.npy", "--stream", win, cx], 600)
        assert (tmp_path / "cpu_s.npy").exists(), rc.stdout[-2000:] + rc.stderr[-2000:]
        ref = np.load(tmp_path / "cpu_s.npy").ravel()
    say(f"reference driver --stream {win} {cx} through the library")
    r = _run([DEV_BIN, "--container", d / "model.ptk", "--case", case, "--out", tmp_path / "s.npy",
              "--stream", win, cx], 300)
    # (its exit code is its gate against the full decode, which a stream need not pass)
    assert (tmp_path / "s.npy").exists() and f"win={win} ctx={cx}" in r.stderr, \
        r.stdout[-2000:] + r.stderr[-2000:]
    got = np.load(tmp_path / "s.npy").ravel()
    assert got.shape == ref.shape == full.shape
    s_stream, s_full = np_ref.sndr(got, ref), np_ref.sndr(got, full)
    say(f"stream {win}/{cx}: {s_stream:.1f} dB vs the CPU build's stream, {s_full:.1f} dB vs its full decode")
    assert s_stream >= 60.0 and s_stream >= s_full + 20.0
    m = re.search(r"conv=(\d+) convT=(\d+) matmul=(\d+)", r.stdout)
    assert m and int(m.group(1)) > 0 and int(m.group(2)) > 0, r.stdout


@pytest.mark.skipif(not PAR_BIN.exists(), reason="oracle/_ref/pt_v21_par_mi355x not built")
@pytest.mark.parametrize("wait", [{}, {"PT_V21_WAIT_US": "200"},
                                  {"PT_V21_WAIT_US": "200", "PT_V21_WAIT_ADAPT": "0"},
                                  {"PT_V21_SYNC": "0"}, {"PT_V21_SYNC": "1"},
                                  {"PT_V21_UP_PAR": "0"}],
                         ids=["runtime-wait", "sleep-poll-200us", "sleep-poll-always",
                              "sync-spin", "sync-blocking", "upload-serialised"])
def test_reference_multistream_driver(model, wait):
    """8 concurrent streams under the driver's own gate, with the runtime's stream wait and with
    the reference's sleep-poll wait policy (its default 200 us, adaptive or always sleeping), with
    its host-wait scheduling modes (PT_V21_SYNC 0 spin, 1 blocking), and with the weight upload
    serialised under the pool lock (PT_V21_UP_PAR=0: the first context copies every record, the
    other seven find them resident)."""
    d, case, _ = model
    say("reference multi-stream driver, 8 streams")
    rp = _run([PAR_BIN, "--container", d / "model.ptk", "--case", case, "--parallel", 8], 300, wait)
    # the driver's own gate: every stream >= 60 dB against the CPU build's waveform
    assert rp.returncode == 0, rp.stdout + rp.stderr
    sndrs = [float(v) for v in re.findall(r"stream \d+: L=\d+ .*?SNDR=([0-9.]+) dB", rp.stdout)]
    assert len(sndrs) == 8 and min(sndrs) >= 60.0, rp.stdout
