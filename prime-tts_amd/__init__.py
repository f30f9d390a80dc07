"""prime-tts_amd: MI355X-native (gfx950) conv hot path of the PrimeTTS v2.1 MB-iSTFT decoder.

The product is the C-ABI shared library ``libptconv_hip.so`` built from ``csrc/`` (HIP kernels + a
C gnu11 host layer exporting the reference's ``pt_v21_*`` device entry points, plus the ``ptd_*``
device-resident decoder API).  This module loads it with ctypes for tests and bench.py; it never
computes anything itself.  ``synth`` holds the packed layouts and seeded synthetic inputs.
"""
from __future__ import annotations

import ctypes as C
import os
import pathlib

import numpy as np

from . import synth  # noqa: F401

HERE = pathlib.Path(__file__).resolve().parent
# PTD_LIB: another build of the same library (e.g. the host AddressSanitizer build, `make asan`)
LIB_PATH = pathlib.Path(os.environ["PTD_LIB"]) if os.environ.get("PTD_LIB") else HERE / "libptconv_hip.so"

F = C.POINTER(C.c_float)
I64 = C.c_int64
VP = C.c_void_p

# name: (restype, argtypes) -- signatures of include/pt_v21_dev.h and include/ptd.h
_SIGS = {
    "pt_v21_cuda_init": (C.c_int, [VP, C.c_int]),
    "pt_v21_cuda_prewarm": (C.c_int, []),
    "pt_v21_cuda_shutdown": (None, [VP]),
    "pt_v21_cuda_weights_mib": (C.c_double, [VP]),
    "pt_v21_cuda_active": (None, [C.c_int]),
    "pt_v21_cuda_keepwarm": (C.c_int, [C.c_int]),
    "pt_v21_gpu_cur_freq": (C.c_long, []),
    "pt_v21_gpu_max_freq": (C.c_long, []),
    "pt_v21_conv_pads_in_kernel": (C.c_int, [VP]),
    "pt_v21_conv": (C.c_int, [VP, F, I64, I64, F, I64, I64, C.c_int, C.c_int, C.c_int, C.c_int,
                              C.c_int, F, F, I64, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float,
                              C.c_float]),
    "pt_v21_convT": (C.c_int, [VP, F, I64, I64, I64, F, I64, C.c_int, C.c_int, C.c_int, C.c_int,
                               F, F, I64, C.c_int, C.c_int]),
    "pt_v21_matmul": (C.c_int, [VP, F, I64, I64, I64, F, I64, I64, F, I64]),
    "pt_v21_devadd_run": (C.c_int, [VP, VP, VP, VP, I64, C.c_int, C.c_float]),
    "pt_v21_devleaky_run": (C.c_int, [VP, VP, VP, I64, C.c_float]),
    "pt_v21_dev_upload": (VP, [VP, VP, I64]),
    "pt_v21_dev_sync_host": (None, [VP, VP, VP, I64]),
    "pt_v21_dev_alloc": (VP, [VP, C.c_size_t]),
    "pt_v21_dev_free": (None, [VP, VP]),
    "pt_v21_dev_reclaim": (None, [VP]),
    "ptd_pool_load": (C.c_int, [VP, C.c_int, C.POINTER(VP), C.POINTER(C.c_size_t)]),
    "ptd_pool_record": (VP, [C.c_int]),
    "ptd_ptk_open": (VP, [C.c_char_p]),
    "ptd_ptk_close": (None, [VP]),
    "ptd_ptk_count": (C.c_int, [VP]),
    "ptd_ptk_find": (C.c_int, [VP, C.c_char_p]),
    "ptd_ptk_info": (C.c_int, [VP, C.c_int, C.c_char_p, C.POINTER(C.c_int), C.POINTER(I64),
                               C.POINTER(I64), C.POINTER(C.c_int)]),
    "ptd_ptk_payload": (VP, [VP, C.c_int]),
    "ptd_ptk_read_f32": (C.c_int, [VP, C.c_int, F, I64]),
    "ptd_ptk_check_decoder": (C.c_int, [VP]),
    "ptd_pool_load_ptk": (C.c_int, [VP, VP, C.c_int, C.POINTER(C.c_char_p)]),
    "ptd_model_create_ptk": (VP, [VP, VP]),
    "ptd_model_create": (VP, [VP, C.POINTER(F), C.POINTER(F)]),
    "ptd_model_destroy": (None, [VP]),
    "ptd_decode": (C.c_int, [VP, VP, VP, I64, C.c_int, VP]),
    "ptd_decode_noalloc": (C.c_int, [VP, VP, VP, I64, C.c_int, VP]),
    "ptd_decode_arena_bytes": (C.c_size_t, [I64, C.c_int]),
    "ptd_decode_stages": (C.c_int, [VP, VP, VP, I64, VP, C.POINTER(VP)]),
    "ptd_layer": (C.c_int, [VP, VP, C.c_int, VP, I64, C.c_int, VP, C.c_float, C.c_float]),
    "ptd_layer_cols": (C.c_int, [VP, VP, C.c_int, VP, I64, C.c_int, VP, C.c_float, C.c_float, VP]),
    "ptd_window_cols": (C.c_int, [I64, C.c_int, I64, I64, I64, I64, VP]),
    "ptd_tail": (C.c_int, [VP, VP, VP, I64, C.c_int, VP]),
    "ptd_mrf": (C.c_int, [VP, VP, C.c_int, VP, I64, C.c_float, VP]),
    "ptd_mrf_depth": (C.c_int, [VP, VP, C.c_int, C.c_int, C.POINTER(VP), C.POINTER(VP),
                                C.POINTER(VP), C.POINTER(VP), C.POINTER(VP), I64]),
    "ptd_device_sync": (C.c_int, []),
    "ptd_decode_windows": (C.c_int, [VP, VP, VP, I64, C.c_int, C.c_int, VP]),
    "ptd_windows_arena_bytes": (C.c_size_t, [I64, C.c_int, C.c_int]),
    "ptd_decode_windows2": (C.c_int, [VP, VP, VP, I64, C.c_int, C.c_int, C.c_int, VP]),
    "ptd_windows2_arena_bytes": (C.c_size_t, [I64, C.c_int, C.c_int, C.c_int]),
    "ptd_queue_create": (VP, [VP, C.c_int, C.c_size_t, C.c_int]),
    "ptd_queue_destroy": (None, [VP]),
    "ptd_queue_hold": (None, [VP, C.c_int]),
    "ptd_queue_submit": (I64, [VP, VP]),
    "ptd_queue_poll": (C.c_int, [VP, I64, VP]),
    "ptd_queue_wait": (C.c_int, [VP, I64, VP]),
    "ptd_now_ms": (C.c_double, []),
    "ptd_decode_chunk": (C.c_int, [VP, VP, VP, I64, I64, I64, VP, C.POINTER(I64)]),
    "ptd_decode_graph": (VP, [VP, VP, VP, I64, C.c_int, VP]),
    "ptd_graph_launch": (C.c_int, [VP, VP]),
    "ptd_graph_destroy": (None, [VP]),
    "ptd_server_create": (VP, [C.c_int, C.c_size_t]),
    "ptd_server_destroy": (None, [VP]),
    "ptd_server_ctx": (VP, [VP, C.c_int]),
    "ptd_serve_run": (C.c_int, [VP, VP, VP, C.c_int, C.POINTER(C.c_double)]),
    "ptd_malloc": (VP, [C.c_size_t]),
    "ptd_free": (None, [VP]),
    "ptd_debug_fail_allocs": (None, [C.c_int, C.c_int]),
    "ptd_debug_reload_env": (None, []),
    "ptd_debug_fill_arena": (C.c_int, [VP, C.c_int]),
    "ptd_h2d": (C.c_int, [VP, VP, VP, C.c_size_t]),
    "ptd_d2h": (C.c_int, [VP, VP, VP, C.c_size_t]),
    "ptd_sync": (C.c_int, [VP]),
    "ptd_event_create": (VP, []),
    "ptd_event_destroy": (None, [VP]),
    "ptd_event_record": (C.c_int, [VP, VP]),
    "ptd_event_elapsed_ms": (C.c_float, [VP, VP]),
    "ptd_mfma_probe": (C.c_int, [VP, F, F, F]),
    "ptd_mfma16_probe": (C.c_int, [VP, F, F, F]),
    "ptd_tail_constants": (None, [F]),
    "ptd_ctx_layout": (C.c_int, [C.POINTER(C.c_long), C.c_int]),
}

# pt_ctx field order reported by ptd_ctx_layout (after sizeof at index 0)
CTX_FIELDS = ["use_cuda", "n_conv", "n_convT", "n_matmul", "g_alloc_ms", "g_calls",
              "dev_bytes_weights", "dev_bytes_res", "devres_oom", "arena_alloc_bytes", "g_weights",
              "g_arena", "g_stream", "g_arena_bytes", "g_arena_used", "conv_pad_in", "conv_in_dev",
              "conv_keep", "conv_keep_res", "dev_live", "conv_out_dev", "chain_mark", "devres"]
TAIL_NCONST = 16 + 144 + 144   # closed-form part of the tail table (Hann, irfft basis)


class Request(C.Structure):
    _fields_ = [("z", VP), ("wav", VP), ("T", I64), ("win", C.c_int), ("ctx", C.c_int)]


class Job(C.Structure):
    """ptd_job: one decode request for ptd_queue_submit (win > 0: streaming windows)."""
    _fields_ = [("z", VP), ("wav", VP), ("T", I64), ("win_first", C.c_int), ("win", C.c_int),
                ("ctx", C.c_int), ("deadline_ms", C.c_double)]


class JobStatus(C.Structure):
    """ptd_job_status: result and host times (ptd_now_ms) of a finished queue job."""
    _fields_ = [("rc", C.c_int), ("worker", C.c_int), ("order", I64), ("t_submit", C.c_double),
                ("t_start", C.c_double), ("t_first", C.c_double), ("t_end", C.c_double)]


_lib = None


def load() -> C.CDLL:
    """Load the built library (fails loudly when it is missing: there is no fallback)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build() (make -C prime-tts_amd)")
        lib = C.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_GLOBAL)
        for name, (res, args) in _SIGS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def ctx_layout() -> dict:
    lib = load()
    buf = (C.c_long * 64)()
    n = lib.ptd_ctx_layout(buf, 64)
    vals = list(buf[:n])
    return {"sizeof": vals[0], **dict(zip(CTX_FIELDS, vals[1:]))}


def fptr(a):
    if a is None:
        return F()
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(F)


class Ctx:
    """A pt_ctx the way the reference host owns one: zeroed memory of the reference's size, brought
    up with pt_v21_cuda_init (stream + arena + shared weights) and torn down with shutdown."""

    def __init__(self, arena_mb: int | None = None):
        self.lib = load()
        self.lay = ctx_layout()
        self.buf = C.create_string_buffer(self.lay["sizeof"])
        self.ptr = C.cast(self.buf, VP)
        old = os.environ.get("PT_V21_ARENA_MB")
        if arena_mb is not None:
            os.environ["PT_V21_ARENA_MB"] = str(arena_mb)
        try:
            rc = self.lib.pt_v21_cuda_init(self.ptr, 0)
        finally:
            if arena_mb is not None:
                if old is None:
                    del os.environ["PT_V21_ARENA_MB"]
                else:
                    os.environ["PT_V21_ARENA_MB"] = old
        if rc != 0:
            raise RuntimeError("pt_v21_cuda_init failed")

    def _addr(self, field):
        return C.addressof(self.buf) + self.lay[field]

    def get_i64(self, field):
        return C.c_int64.from_address(self._addr(field)).value

    def set_i64(self, field, v):
        C.c_int64.from_address(self._addr(field)).value = v

    def get_int(self, field):
        return C.c_int.from_address(self._addr(field)).value

    def set_int(self, field, v):
        C.c_int.from_address(self._addr(field)).value = v

    def get_ptr(self, field):
        return C.c_void_p.from_address(self._addr(field)).value

    def set_ptr(self, field, v):
        C.c_void_p.from_address(self._addr(field)).value = v

    def get_long(self, field):
        return C.c_long.from_address(self._addr(field)).value

    def sync(self):
        if self.lib.ptd_sync(self.ptr) != 0:
            raise RuntimeError("stream sync failed")

    def close(self):
        if self.ptr is not None:
            self.lib.pt_v21_cuda_shutdown(self.ptr)
            self.ptr = None


class DevBuf:
    """Device buffer of float32 owned by the library's allocator."""

    def __init__(self, n: int):
        self.lib = load()
        self.n = int(n)
        self.ptr = self.lib.ptd_malloc(max(self.n, 1) * 4)
        if not self.ptr:
            raise MemoryError(f"ptd_malloc({self.n * 4}) failed")

    @classmethod
    def of(cls, ctx: Ctx, a: np.ndarray) -> "DevBuf":
        a = np.ascontiguousarray(a, np.float32)
        b = cls(a.size)
        b.upload(ctx, a)
        return b

    def upload(self, ctx: Ctx, a: np.ndarray):
        a = np.ascontiguousarray(a, np.float32)
        assert a.size <= self.n
        if self.lib.ptd_h2d(ctx.ptr, self.ptr, a.ctypes.data_as(VP), a.size * 4) != 0:
            raise RuntimeError("ptd_h2d failed")

    def download(self, ctx: Ctx, n: int | None = None) -> np.ndarray:
        n = self.n if n is None else n
        out = np.empty(n, np.float32)
        if self.lib.ptd_d2h(ctx.ptr, out.ctypes.data_as(VP), self.ptr, n * 4) != 0:
            raise RuntimeError("ptd_d2h failed")
        return out

    def free(self):
        if self.ptr:
            self.lib.ptd_free(self.ptr)
            self.ptr = None


class Ptk:
    """A .ptk weight container opened by the library's reader (ptd_ptk_open)."""

    def __init__(self, path):
        self.lib = load()
        self.ptr = self.lib.ptd_ptk_open(str(path).encode())
        if not self.ptr:
            raise ValueError(f"ptd_ptk_open refused {path}")

    def __len__(self):
        return self.lib.ptd_ptk_count(self.ptr)

    def find(self, name: str) -> int:
        return self.lib.ptd_ptk_find(self.ptr, name.encode())

    def info(self, i: int):
        """(name, shape, itemsize) of record i."""
        name = C.create_string_buffer(65)
        nd, isz = C.c_int(), C.c_int()
        dims, nel = (I64 * 6)(), I64()
        if self.lib.ptd_ptk_info(self.ptr, i, name, C.byref(nd), dims, C.byref(nel), C.byref(isz)):
            raise IndexError(i)
        return name.value.decode(), tuple(dims[:nd.value]), isz.value

    def read(self, i: int) -> np.ndarray:
        """Record i as float32 (fp16 payloads expanded by the library)."""
        _, shape, _ = self.info(i)
        out = np.empty(shape, np.float32)
        if self.lib.ptd_ptk_read_f32(self.ptr, i, out.ctypes.data_as(F), out.size):
            raise RuntimeError(f"ptd_ptk_read_f32({i}) failed")
        return out

    def check_decoder(self) -> bool:
        return self.lib.ptd_ptk_check_decoder(self.ptr) == 0

    def close(self):
        if self.ptr:
            self.lib.ptd_ptk_close(self.ptr)
            self.ptr = None


class Model:
    """The decoder's weights on the device (ptd_model): from packed arrays, or from a container
    (Model.from_ptk)."""

    @classmethod
    def from_ptk(cls, ctx: Ctx, ptk: Ptk) -> "Model":
        m = cls.__new__(cls)
        m.lib = load()
        m.ptr = m.lib.ptd_model_create_ptk(ctx.ptr, ptk.ptr)
        if not m.ptr:
            raise RuntimeError("ptd_model_create_ptk failed")
        return m

    def __init__(self, ctx: Ctx, ws, bs):
        self.lib = load()
        self._ws = [np.ascontiguousarray(w, np.float32) for w in ws]
        self._bs = [np.ascontiguousarray(b, np.float32) for b in bs]
        assert len(self._ws) == synth.N_LAYER and len(self._bs) == synth.N_LAYER
        wa = (F * synth.N_LAYER)(*[fptr(w) for w in self._ws])
        ba = (F * synth.N_LAYER)(*[fptr(b) for b in self._bs])
        self.ptr = self.lib.ptd_model_create(ctx.ptr, wa, ba)
        if not self.ptr:
            raise RuntimeError("ptd_model_create failed")

    def close(self):
        if self.ptr:
            self.lib.ptd_model_destroy(self.ptr)
            self.ptr = None
