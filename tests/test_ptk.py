"""The .ptk container reader (ptd_ptk_*, host code of libptconv_hip.so; no device call here).

Pinned by: containers written by tests/ptk_writer.py (the exporter's layout, restated); exact
float16 values (numpy) for every non-NaN fp16 code; the reference's own C reader
(pt_v21_host.c:1086-1220, oracle/_ref) for every fp16 code, NaN payloads included, and for the
decoder's records; and refusal of each kind of corrupt file."""
from __future__ import annotations

import struct
import subprocess
import sys

import numpy as np
import pytest

import ptk_writer as pw
from conftest import ROOT, load_package

pkg = load_package()
synth = pkg.synth
REF_LIB = ROOT / "oracle" / "_ref" / "libptref.so"


def all_codes() -> np.ndarray:
    return np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)


def sample_tensors():
    rng = np.random.default_rng(3)
    return [
        ("a.w", rng.standard_normal((3, 5, 7)).astype(np.float32), 4),
        ("b.h#h", rng.standard_normal((4, 9)).astype(np.float32), 2),
        ("codes#h", all_codes(), 2),
        ("scalar", np.float32(2.5).reshape(()), 4),
        ("empty", np.zeros((0,), np.float32), 4),
        ("n" * 63, np.arange(6, dtype=np.float32).reshape(2, 3), 4),
    ]


@pytest.fixture(scope="module")
def sample(tmp_path_factory):
    path = tmp_path_factory.mktemp("ptk") / "sample.ptk"
    pw.write(path, sample_tensors())
    f = pkg.Ptk(path)
    yield f
    f.close()


def test_records_roundtrip(sample):
    ts = sample_tensors()
    assert len(sample) == len(ts) + 1   # + dtype.table
    for i, (name, a, isz) in enumerate(ts):
        assert sample.find(name) == i
        nm, shape, got_isz = sample.info(i)
        assert (nm, shape, got_isz) == (name, a.shape, isz)
        v = sample.read(i)
        want = np.asarray(a).astype(np.float16).astype(np.float32) if isz == 2 else a
        assert v.shape == a.shape
        ok = np.isnan(want) | (v.view(np.uint32) == want.view(np.uint32)) if isz == 2 else v == want
        assert np.all(ok)
    t = sample.find("dtype.table")
    assert t == len(ts)
    assert list(sample.read(t)) == [float(x[2]) for x in ts] + [4.0]
    assert sample.find("missing") == -1


def test_fp16_expansion_exact(sample):
    """Every non-NaN fp16 code expands to exactly its value (zero signs, subnormals, infinities
    included); NaN codes stay NaN with their sign and payload."""
    codes = all_codes()
    v = sample.read(sample.find("codes#h"))
    finite = ~np.isnan(codes)
    want = codes.astype(np.float32)
    assert np.array_equal(v[finite], want[finite])
    assert np.array_equal(np.signbit(v[finite]), np.signbit(want[finite]))
    sub = finite & (codes != 0) & (np.abs(codes.astype(np.float32)) < 2.0 ** -14)
    assert sub.sum() == 2 * 1023 and np.all(v[sub] != 0)
    raw = codes.view(np.uint16).astype(np.uint32)
    nan = ~finite
    bits = v.view(np.uint32)
    assert np.all(np.isnan(v[nan]))
    assert np.array_equal(bits[nan] >> 31, raw[nan] >> 15)
    assert np.array_equal(bits[nan] & 0x7FFFFF, (raw[nan] & 0x3FF) << 13)


def _ref_dump(container, tmp_path):
    out = tmp_path / "ref.npz"
    r = subprocess.run([sys.executable, str(ROOT / "tests" / "ref_ptk_dump.py"), str(container),
                        str(out)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    return np.load(out, allow_pickle=False)


@pytest.mark.skipif(not REF_LIB.exists(), reason="oracle/_ref not built (reference tree absent)")
def test_matches_reference_reader(tmp_path):
    """Bit-for-bit against the reference's reader on a decoder container whose fp16 conv_pre
    record holds every fp16 code (NaNs included) and whose other records are synthetic weights."""
    ws, bs = synth.decoder_weights(21)
    tensors = pw.decoder_tensors(ws, bs)
    w0 = ws[0].reshape(-1).astype(np.float16)
    w0[:65536] = all_codes()
    tensors[0] = (tensors[0][0], w0.reshape(ws[0].shape), 2)
    path = tmp_path / "dec.ptk"
    pw.write(path, tensors)
    ref = _ref_dump(path, tmp_path)
    f = pkg.Ptk(path)
    try:
        names = [t[0] for t in tensors]
        assert sorted(k for k in ref.files if not k.startswith("__isz__")) == sorted(names)
        for name in names:
            i = f.find(name)
            assert f.info(i)[2] == int(ref["__isz__" + name])
            mine = f.read(i).reshape(-1)
            assert np.array_equal(mine.view(np.uint32), ref[name].view(np.uint32)), name
    finally:
        f.close()


# ------------------------------------------------------------------ corrupt containers
def _good_bytes(tmp_path):
    p = tmp_path / "g.ptk"
    pw.write(p, [("x", np.arange(10, dtype=np.float32), 4), ("y#h", np.ones(5, np.float32), 2)])
    return bytearray(p.read_bytes())


def _refused(tmp_path, data: bytes) -> bool:
    p = tmp_path / "bad.ptk"
    p.write_bytes(bytes(data))
    try:
        pkg.Ptk(p).close()
    except ValueError:
        return True
    return False


REC0 = pw.HEADER.size   # first record


def _set(buf, off, fmt, v):
    struct.pack_into(fmt, buf, off, v)
    return buf


CORRUPTIONS = {
    "empty file": lambda b: b[:0],
    "short header": lambda b: b[:10],
    "bad magic": lambda b: _set(b, 0, "<I", 0x50544B32),
    "records past the end": lambda b: _set(b, 8, "<I", 100000),
    "data past the end": lambda b: _set(b, 16, "<q", len(b)),
    "negative data size": lambda b: _set(b, 16, "<q", -64),
    "truncated payload": lambda b: b[:-64],
    "ndim 7": lambda b: _set(b, REC0 + 64, "<i", 7),
    "negative ndim": lambda b: _set(b, REC0 + 64, "<i", -1),
    "nelem not the product of dims": lambda b: _set(b, REC0 + 120, "<q", 11),
    "negative offset": lambda b: _set(b, REC0 + 128, "<q", -64),
    "payload offset past the data": lambda b: _set(b, REC0 + 128, "<q", 1 << 40),
    "huge dims": lambda b: _set(_set(b, REC0 + 72, "<q", 1 << 62), REC0 + 120, "<q", 1 << 62),
    "no dtype.table": lambda b: _set(b, REC0 + 2 * pw.RECORD.size, "<11s", b"dtype.tablX"),
    "table entry 3": None,
    "table says fp16 for itself": None,
}


@pytest.mark.parametrize("what", list(CORRUPTIONS))
def test_corrupt_containers_refused(tmp_path, what):
    b = _good_bytes(tmp_path)
    assert not _refused(tmp_path, b)
    if what.startswith("table"):
        tab_rec = REC0 + 2 * pw.RECORD.size
        data = pw.pad64(REC0 + 3 * pw.RECORD.size)
        toff = struct.unpack_from("<q", b, tab_rec + 128)[0]
        entry = 0 if what == "table entry 3" else 2
        struct.pack_into("<f", b, data + toff + 4 * entry, 3.0 if entry == 0 else 2.0)
    else:
        b = CORRUPTIONS[what](b)
    assert _refused(tmp_path, b), what


def test_missing_file_refused(tmp_path):
    with pytest.raises(ValueError):
        pkg.Ptk(tmp_path / "nope.ptk")


def test_width_comes_from_the_table(tmp_path):
    """As in the reference's C reader, dtype.table (not the name suffix) sets the item size."""
    p = tmp_path / "w.ptk"
    pw.write(p, [("plain", np.array([1.0, -2.0, 3.0], np.float32), 2)])
    f = pkg.Ptk(p)
    try:
        assert f.info(0)[2] == 2 and np.array_equal(f.read(0), [1.0, -2.0, 3.0])
    finally:
        f.close()


# ------------------------------------------------------------------ decoder containers
def _decoder_container(tmp_path, mutate=None):
    ws, bs = synth.decoder_weights(5)
    t = pw.decoder_tensors(ws, bs)
    if mutate:
        t = mutate(t)
    p = tmp_path / "d.ptk"
    pw.write(p, t)
    return pkg.Ptk(p)


def _replace(name, fn):
    def m(ts):
        return [(n, fn(a) if n == name else a, s) for n, a, s in ts]
    return m


@pytest.mark.parametrize("mutate,ok", [
    (None, True),
    (lambda ts: [x for x in ts if x[0] != "dec.resblocks.4.convs2.1.wp#h"], False),
    (lambda ts: [x for x in ts if x[0] != "dec.ups.1.b"], False),
    (lambda ts: [x for x in ts if x[0] != "dec.Conv.b"], True),        # the final conv's bias is optional
    (_replace("dec.conv_pre.wp#h", lambda a: a.reshape(-1)[:-4]), False),
    (_replace("dec.ConvTranspose_1.wp", lambda a: a * np.float32(1.001)), False),
    (_replace("dec.ConvTranspose.wp", lambda a: np.roll(a, 4)), False),
    (_replace("dec.ConvTranspose_2.wp", lambda a: a / 4), False),
    (_replace("dec.ConvTranspose_2.b", lambda a: a + 1), False),
    (lambda ts: [(n.replace("#h", ""), a, 4) for n, a, s in ts], True),   # all-fp32 container
])
def test_check_decoder(tmp_path, mutate, ok):
    f = _decoder_container(tmp_path, mutate)
    try:
        assert f.check_decoder() == ok
    finally:
        f.close()


def test_synthetic_container_has_fp16_subnormals():
    """The fp16 decoder weights the GPU container tests use include subnormals (so a flushing
    expansion would change the decoded waveform)."""
    ws, _ = synth.decoder_weights(1234)
    h = np.concatenate([w.reshape(-1) for w in ws[:39]]).astype(np.float16)
    a = np.abs(h.astype(np.float32))
    assert np.count_nonzero((a > 0) & (a < 2.0 ** -14)) > 1000
