"""CPU checks of the C-ABI boundary: the library loads without a GPU, exports every symbol the
headers in include/ declare, lays struct pt_ctx out exactly like the reference header, and its
tail constants equal the oracle's closed forms.  No compute call reaches the device here."""
from __future__ import annotations

import json
import re

import numpy as np

import oracle_lib as ol
from conftest import ROOT, load_package

pkg = load_package()


def _declared_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b(pt_v21_\w+|ptd_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_every_declared_symbol_is_exported():
    lib = pkg.load()
    names = _declared_symbols()
    assert "pt_v21_conv" in names and "pt_v21_convT" in names and "ptd_decode" in names
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing


def test_reference_abi_names_present():
    """The device entry points the reference host calls (runtime/v21/src/pt_v21.h:208-259)."""
    lib = pkg.load()
    for n in ["pt_v21_cuda_init", "pt_v21_cuda_prewarm", "pt_v21_cuda_shutdown", "pt_v21_conv",
              "pt_v21_convT", "pt_v21_matmul", "pt_v21_conv_pads_in_kernel",
              "pt_v21_cuda_weights_mib", "pt_v21_cuda_active", "pt_v21_cuda_keepwarm",
              "pt_v21_gpu_cur_freq", "pt_v21_gpu_max_freq", "pt_v21_dev_alloc", "pt_v21_dev_free",
              "pt_v21_dev_reclaim", "pt_v21_dev_upload", "pt_v21_dev_sync_host",
              "pt_v21_devadd_run", "pt_v21_devleaky_run"]:
        assert hasattr(lib, n), n


def test_ctx_layout_matches_reference():
    lay = pkg.ctx_layout()
    mine = [lay["sizeof"]] + [lay[f] for f in pkg.CTX_FIELDS]
    gold = json.loads((ROOT / "tests" / "golden" / "ref_ctx_layout.json").read_text())["layout"]
    assert mine == gold
    if ol.have_ref():
        import ctypes as C
        buf = (C.c_long * 64)()
        n = ol.ref().ref_ctx_layout(buf, 64)
        assert mine == list(buf[:n])


def test_tail_constants_match_oracle():
    lib = pkg.load()
    import ctypes as C
    out = np.zeros(pkg.TAIL_NCONST, np.float32)
    lib.ptd_tail_constants(out.ctypes.data_as(C.POINTER(C.c_float)))
    hann, bc, bs = ol.constants()
    assert out.size == 304
    assert np.array_equal(out[:16], hann)
    assert np.array_equal(out[16:160], bc.ravel())
    assert np.array_equal(out[160:304], bs.ravel())


def test_host_only_calls_fail_loudly_without_device():
    """A context that was never brought up has no CPU path in this library: the call must fail
    (return -1), never compute on the host."""
    import ctypes as C
    lib = pkg.load()
    buf = C.create_string_buffer(pkg.ctx_layout()["sizeof"])
    x = np.ones((1, 4, 8), np.float32)
    y = np.zeros((1, 4, 8), np.float32)
    w = np.ones((1, 1, 4, 4), np.float32)
    rc = lib.pt_v21_conv(C.cast(buf, C.c_void_p), pkg.fptr(x), 8, 4, pkg.fptr(y), 8, 8, 4, 1, 1, 0,
                         1, pkg.fptr(w), pkg.fptr(None), 1, -1, -1, 0, 0, 0.0, 0.0)
    assert rc == -1
    assert np.all(y == 0)


def test_pads_in_kernel_follows_the_op_switch():
    """PT_V21_GPU without "conv" routes convs to the host's CPU path, which reads padded rows, so the
    library tells the host to pad (pt_v21_conv_pads_in_kernel = 0); by default it pads in-kernel.
    No device call: run in child processes with the environment set."""
    import subprocess
    import sys
    code = ("import ctypes, sys; lib = ctypes.CDLL(sys.argv[1]); "
            "print(lib.pt_v21_conv_pads_in_kernel(None))")
    lib = str(ROOT / "prime-tts_amd" / "libptconv_hip.so")
    out = {}
    for v in (None, "conv,convT,matmul", "convT", "matmul", ""):
        env = {k: x for k, x in __import__("os").environ.items() if k != "PT_V21_GPU"}
        if v is not None:
            env["PT_V21_GPU"] = v
        r = subprocess.run([sys.executable, "-c", code, lib], env=env, capture_output=True,
                           text=True, timeout=60)
        out[v] = int(r.stdout.strip())
    assert out == {None: 1, "conv,convT,matmul": 1, "convT": 1, "matmul": 0, "": 1}


def test_simt_launcher_refuses_a_tensor_add_without_its_tensor():
    """ptk_conv_simt takes epilogue codes without a residual tensor, so code 5 (tensor add) would
    read through a null pointer on the device: refused on the host, before any HIP call."""
    import ctypes as C
    lib = pkg.load()
    f = lib.ptk_conv_simt
    f.restype = C.c_int
    f.argtypes = [C.c_void_p, C.c_int64, C.c_int64, C.c_int64, C.c_int, C.c_void_p, C.c_void_p,
                  C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_int64, C.c_int64,
                  C.c_int64, C.c_int, C.c_int, C.c_float, C.c_int, C.c_float, C.c_void_p]
    dummy = C.c_void_p(16)   # never dereferenced: the refusal comes first
    for e0, e1 in ((5, 0), (1, 5)):
        rc = f(dummy, 8, 32, 8, 4, dummy, None, 1, 3, 1, 1, 1, dummy, 8, 32, 8, 1, e0, 0.1, e1,
               0.0, None)
        assert rc == -1
        lib.ptk_last_error.restype = C.c_char_p
        assert b"tensor add" in lib.ptk_last_error()


def test_phase_interleaved_relayout_refuses_a_wrong_phase_count():
    """ptk_relayout_il interleaves the rows of a stride-4 convT (row m: phase m & 3 of channel
    m >> 2), which needs M = 4 x the rows per phase: any other count is refused on the host,
    before any HIP call, for both the 32-row and the 16-row layouts."""
    import ctypes as C
    lib = pkg.load()
    lib.ptk_last_error.restype = C.c_char_p
    dummy = C.c_void_p(16)   # never dereferenced: the refusal comes first
    for name in ("ptk_relayout_il", "ptk_relayout16_il"):
        f = getattr(lib, name)
        f.restype = C.c_int
        f.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p]
        for M, il in ((512, 100), (512, 256), (510, 128), (512, -1)):
            assert f(dummy, dummy, M, 4, 256, il, None) == -1, (name, M, il)
            assert b"phase interleave" in lib.ptk_last_error()
