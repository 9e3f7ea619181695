"""Writes tests/golden/winograd_tables.json: the exact (AT, G, BT) tables of the three Winograd variants the conv
family uses (F(4, 3), F(4, 4), F(2, 3)), as fraction strings. These are the values every Winograd GPU parity case
and every U / tr operand was built with (the tables the kernels were validated against); tests/test_winograd.py
checks lokinfer_amd.winograd against them. The file was written once, before that module was rewritten from the
Lagrange-interpolation construction; regenerating it from the module would make the check circular."""
import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from lokinfer_amd import winograd as W  # noqa: E402

VARIANTS = {"F(4,3)": (4, 3, None), "F(4,4)": (4, 4, None), "F(2,3)": (2, 3, W.POINTS_TILE2)}


def main():
    out = {}
    for name, (m, r, pts) in VARIANTS.items():
        at, g, bt = W.transforms_exact(m, r, pts)
        out[name] = {k: [[str(v) for v in row] for row in mat] for k, mat in (("AT", at), ("G", g), ("BT", bt))}
    lines = ["{"]
    for i, (name, mats) in enumerate(out.items()):
        lines.append(f' "{name}": {{')
        for j, (k, mat) in enumerate(mats.items()):
            rows = ",\n".join("   " + json.dumps(row) for row in mat)
            lines.append(f'  "{k}": [\n{rows}\n  ]' + ("," if j < 2 else ""))
        lines.append(" }" + ("," if i < len(out) - 1 else ""))
    lines.append("}")
    (Path(__file__).parent / "winograd_tables.json").write_text("\n".join(lines) + "\n")


if __name__ == "__main__":
    main()
