"""Writes tests/golden/v21_records.json: every record the reference graph reads from its container,
in the graph's constant-table order (runtime/v21/gen/pt_graph.c, pt_graph_ctab), with what a
synthetic full-model container needs to hold for it:

  role "const"   the model constant itself (float32 values and shape, spec/v21_layers.json
                 `constants`: the graph's own numbers, e.g. sqrt(192) scales, mask fills);
  role "w"/"b"   a conv / convT weight (packed shape, cin, cout, K, stride) or its bias;
  role "ln_g"/"ln_b", "emb", "relpos"   LayerNorm scale / shift, an embedding table, a relative
                 position table, with their shapes.

Run where the reference tree exists:  python tests/golden/make_records_manifest.py [/root/reference]"""
from __future__ import annotations

import importlib.util
import json
import pathlib
import re
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
_spec = importlib.util.spec_from_file_location(
    "extract_constants", HERE / "extract_constants.py")
extract = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(extract)


def main(ref: pathlib.Path) -> None:
    spec = json.loads((ref / "spec" / "v21_layers.json").read_text())
    src = (ref / "runtime" / "v21" / "gen" / "pt_graph.c").read_text()
    blk = src[src.index("pt_graph_ctab[PT_N_CONT] = {"):]
    ctab = re.findall(r'"([^"]+)"', blk[:blk.index("};")])
    consts = {c["container"]: c for c in spec["constants"] if c.get("container")}
    owner = {}
    for layer in spec["layers"]:
        for i, name in enumerate(layer.get("packed", [])):
            owner.setdefault(name, (i, layer))
    out = []
    for name in ctab:
        rec = {"name": name, "isz": 2 if name.endswith("#h") else 4}
        if name in consts:
            c = consts[name]
            assert c["dtype"] == "float32", name
            values = c["values"] or []
            if len(values) != int(np.prod(c["shape"], dtype=np.int64)):
                # the spec lists a preview only: decode the node's raw bytes
                node = spec["layers"][c["idx"]]["name"]
                values = extract.constant(spec, node).reshape(-1).tolist()
            assert len(values) == int(np.prod(c["shape"], dtype=np.int64)), name
            rec.update(role="const", shape=c["shape"], values=values)
        else:
            i, layer = owner[name]
            op, p = layer["onnx_op"], layer.get("params") or {}
            if op in ("Conv", "ConvTranspose"):
                common = dict(cin=p["cin"], cout=p["cout"], K=p["kernel"],
                              stride=p["stride"], convT=op == "ConvTranspose")
                if i == 0:
                    rec.update(role="w", shape=layer["packed_shape"], **common)
                else:
                    rec.update(role="b", shape=layer["B_shape"], **common)
            elif op == "LayerNormalization":
                rec.update(role="ln_g" if i == 0 else "ln_b", shape=[p["C"]])
            elif op == "Gather":
                rec.update(role="emb", shape=[p["rows"], p["cols"]])
            elif op == "Pad":
                rec.update(role="relpos", shape=p["table"])
            else:
                raise ValueError(f"{name}: unexpected owner op {op}")
        out.append(rec)
    path = HERE / "v21_records.json"
    path.write_text(json.dumps({"source": "spec/v21_layers.json + runtime/v21/gen/pt_graph.c",
                                "records": out}, indent=0))
    print(f"wrote {path}: {len(out)} records")


if __name__ == "__main__":
    main(pathlib.Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference"))
