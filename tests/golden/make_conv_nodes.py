"""Writes tests/golden/v21_conv_nodes.json: the output tensor name of every Conv and ConvTranspose
node of the reference graph, in graph order, with the node's op, kernel size, cout and cin (the
generated node table runtime/v21/gen/pt_graph.c pt_ndefs: op, i0 = K, f0 = cout, f1 = cin, the
output list; pt_graph_tnames gives the names).  tests/test_gpu_dropin.py hands these names to the
reference driver's checkpoint option (main_v21.c:307-321) to dump every conv node's output in the
CPU build and in the build linked against the library.

Run where the reference tree exists:  python tests/golden/make_conv_nodes.py [/root/reference]"""
from __future__ import annotations

import json
import pathlib
import re
import sys

HERE = pathlib.Path(__file__).resolve().parent
OUT = HERE / "v21_conv_nodes.json"


def main(ref: pathlib.Path) -> None:
    src = (ref / "runtime" / "v21" / "gen" / "pt_graph.c").read_text()
    tn = src[src.index("pt_graph_tnames[PT_N_TENSOR] = {"):]
    names = re.findall(r'"((?:[^"\\]|\\.)*)"', tn[:tn.index("};")])
    nd = src[src.index("pt_ndefs[PT_N_NODE] = {"):]
    nd = nd[:nd.index("};")]
    nodes = []
    for m in re.finditer(r"\{\s*(PT_CONVT|PT_CONV)\s*,([^{]*)\{([^}]*)\}\s*,\s*\{([^}]*)\}", nd):
        op, scalars, _ins, outs = m.groups()
        sc = [v.strip() for v in scalars.split(",") if v.strip()]
        K, cout, cin = int(sc[0]), float(sc[4].rstrip("f")), float(sc[5].rstrip("f"))
        out = [int(v) for v in outs.split(",") if int(v) >= 0]
        nodes.append({"op": "convT" if op == "PT_CONVT" else "conv", "name": names[out[0]],
                      "K": K, "cout": int(cout), "cin": int(cin)})
    OUT.write_text(json.dumps({"nodes": nodes}, indent=1) + "\n")
    print(f"wrote {OUT}: {sum(n['op'] == 'conv' for n in nodes)} conv, "
          f"{sum(n['op'] == 'convT' for n in nodes)} convT nodes")


if __name__ == "__main__":
    main(pathlib.Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference"))
