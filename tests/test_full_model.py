"""The synthetic full-model container (tests/full_model.py) is a model the reference's own driver
accepts: its CPU build (oracle/_ref/pt_v21_cpu) reads every record through pt_v21_open and runs
the whole graph to a finite waveform of the expected length.  Skipped where oracle/_ref was not
built."""
from __future__ import annotations

import re
import subprocess

import numpy as np
import pytest

import full_model as fm
from conftest import ROOT

CPU_BIN = ROOT / "oracle" / "_ref" / "pt_v21_cpu"


def test_manifest_covers_the_graph():
    recs = fm.records()
    assert len(recs) == 336 and len({r["name"] for r in recs}) == 336
    t = fm.tensors(seed=0)
    payload = sum(-(-np.asarray(a).size * isz // 64) * 64 for _, a, isz in t)
    # The reference's own container holds 89077824 payload bytes in 339 records
    # (spec/v21_layers.json `counts`).  Three are metadata the graph never reads
    # (tools/export_v21.py:895-911): model.meta (<= 16 floats: 64 B), dec.geom (24 floats: 128 B)
    # and dtype.table (339 floats: 1408 B), 1600 B in all; the graph's 336 records are the rest.
    assert payload == 89077824 - (64 + 128 + 1408)


@pytest.mark.skipif(not CPU_BIN.exists(), reason="oracle/_ref/pt_v21_cpu not built")
def test_reference_cpu_driver_runs_the_synthetic_model(tmp_path):
    fm.write_container(tmp_path / "model.ptk", seed=0)
    fm.write_case(tmp_path / "case", n_tokens=20, seed=1)
    out = tmp_path / "wav.npy"
    r = subprocess.run([str(CPU_BIN), "--cpu", "--container", str(tmp_path / "model.ptk"), "--case",
                        str(tmp_path / "case"), "--out", str(out)], capture_output=True, text=True,
                       timeout=600)
    assert out.exists(), r.stdout + r.stderr
    w = np.load(out).ravel()
    L = int(re.search(r"L=(\d+)", r.stdout).group(1))
    assert w.size == L and L % 256 == 0 and L >= 20 * 256
    assert np.all(np.isfinite(w)) and float(np.abs(w).max()) > 0
