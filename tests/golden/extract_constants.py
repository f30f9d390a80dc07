"""Writes prime-tts_amd/data/v21_pqmf_synthesis.npy: the MB-iSTFT decoder's PQMF synthesis filter, the model constant
/dec/Constant_134 of shape (1, 4, 63) (the weight of the final /dec/Conv, 4 subbands -> 1 sample
stream, 63 taps).  The reference keeps its raw fp32 bytes in spec/v21_layers.json (the node's
"value" attribute, protobuf text format); this script decodes them.  Run where the reference tree
exists: python tests/golden/extract_constants.py [/root/reference]"""
from __future__ import annotations

import json
import pathlib
import re
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
DATA = HERE.parents[1] / "prime-tts_amd" / "data"
ESC = {"n": 10, "t": 9, "r": 13, '"': 34, "'": 39, "\\": 92, "a": 7, "b": 8, "f": 12, "v": 11}


def unescape(text: str) -> bytes:
    """Protobuf text-format string escapes: \\NNN octal, \\xHH, and the C escapes."""
    out, i = bytearray(), 0
    while i < len(text):
        c = text[i]
        if c != "\\":
            out.append(ord(c))
            i += 1
            continue
        n = text[i + 1]
        if n in "01234567":
            j, v = i + 1, 0
            while j < len(text) and j < i + 4 and text[j] in "01234567":
                v = v * 8 + int(text[j])
                j += 1
            out.append(v)
            i = j
        elif n == "x":
            out.append(int(text[i + 2:i + 4], 16))
            i += 4
        else:
            out.append(ESC[n])
            i += 2
    return bytes(out)


def constant(spec: dict, name: str) -> np.ndarray:
    node = next(l for l in spec["layers"] if l.get("name") == name)
    value = node["attrs"]["value"]
    dims = [int(d) for d in re.findall(r"dims: (\d+)", value)]
    raw = unescape(re.search(r'raw_data: "((?:[^"\\]|\\.)*)"', value, re.S).group(1))
    assert "data_type: 1" in value, "expected an fp32 constant"
    return np.frombuffer(raw, dtype="<f4").reshape(dims).copy()


def main():
    ref = pathlib.Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    spec = json.loads((ref / "spec" / "v21_layers.json").read_text())
    h = constant(spec, "/dec/Constant_134")
    assert h.shape == (1, 4, 63), h.shape
    np.save(DATA / "v21_pqmf_synthesis.npy", h.astype(np.float32))
    print(f"wrote {DATA / 'v21_pqmf_synthesis.npy'}: {h.shape}, band sums {h[0].sum(axis=1)}")


if __name__ == "__main__":
    main()
