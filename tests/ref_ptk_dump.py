"""Test infrastructure: reads a .ptk container with the reference's own C reader
(runtime/v21/src/pt_v21_host.c pt_v21_open, compiled unmodified into oracle/_ref/libptref.so)
and saves every record it loads, as pt_v21_cont returns it (fp32, fp16 records expanded by the
reference), into an .npz keyed by record name, with the item sizes under "__isz__<name>".

Run as a child process (the reference reader keeps process-global state that supports one
container per process):  python tests/ref_ptk_dump.py CONTAINER OUT.npz"""
import ctypes as C
import pathlib
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[1]
N_CONT = 336   # PT_N_CONT of the reference's generated graph (gen/pt_graph_tab.h)


def main(container: str, out: str) -> int:
    lib = C.CDLL(str(ROOT / "oracle" / "_ref" / "libptref.so"))
    lib.pt_v21_open.restype = C.c_void_p
    lib.pt_v21_open.argtypes = [C.c_char_p]
    lib.pt_v21_cont.restype = C.POINTER(C.c_float)
    lib.pt_v21_cont.argtypes = [C.c_void_p, C.c_int]
    lib.pt_v21_cont_bytes.restype = C.c_size_t
    lib.pt_v21_cont_bytes.argtypes = [C.c_void_p, C.c_int]
    lib.pt_v21_cont_itemsize.restype = C.c_int
    lib.pt_v21_cont_itemsize.argtypes = [C.c_void_p, C.c_int]
    lib.pt_v21_n_cont.restype = C.c_int
    lib.pt_v21_n_cont.argtypes = [C.c_void_p]
    lib.pt_v21_close.argtypes = [C.c_void_p]
    ctab = (C.c_char_p * N_CONT).in_dll(lib, "pt_graph_ctab")
    ctx = lib.pt_v21_open(container.encode())
    if not ctx:
        print("pt_v21_open refused the container", file=sys.stderr)
        return 3
    assert lib.pt_v21_n_cont(ctx) == N_CONT
    res = {}
    for k in range(N_CONT):
        p = lib.pt_v21_cont(ctx, k)
        if not p:
            continue
        n = lib.pt_v21_cont_bytes(ctx, k) // 4
        name = ctab[k].decode()
        res[name] = np.ctypeslib.as_array(p, (n,)).copy()
        res["__isz__" + name] = np.int32(lib.pt_v21_cont_itemsize(ctx, k))
    lib.pt_v21_close(ctx)
    np.savez(out, **res)
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1], sys.argv[2]))
