"""Writes golden fixtures from the model inputs of the reference's IR lit tests (lariaus/lokinfer tests/lit/*/*.lkir).

Run in the build container (it needs /root/reference and oracle/_ref/lkm-ref-tool, see make_ir_golden.py). For each
lit input it keeps only the model text (the `//` RUN / CHECK lines are the reference's test script and are not
copied), as tests/golden/ir/lit/DIR_NAME.lkir, and writes with the reference's own IR library:
  DIR_NAME.stage.txt   the model after the passes the lit test runs (its RUN line's --pass list, --pipeline, or none),
                       or the single line "rejected" when the reference rejects the model at that stage
  DIR_NAME.stage       the pass list used
  DIR_NAME.pipeline.txt / .lkm / .lkm.txt   as make_ir_golden.py, when the model survives the pipeline and has no
                       external constants"""
import re
import subprocess
import sys
from pathlib import Path

REF = Path("/root/reference/tests/lit")
HERE = Path(__file__).resolve().parent / "ir" / "lit"
TOOL = Path(__file__).resolve().parents[2] / "oracle" / "_ref" / "lkm-ref-tool"


def run(*args):
    r = subprocess.run([str(TOOL), *map(str, args)], capture_output=True, text=True)
    return r.returncode, r.stdout


def main():
    if not TOOL.exists():
        sys.exit(f"{TOOL} is not built: make -f oracle/ref_ir.mk")
    HERE.mkdir(exist_ok=True)
    for src in sorted(REF.glob("*/*.lkir")):
        name = f"{src.parent.name}_{src.stem}"
        text = src.read_text()
        run_line = next((l for l in text.splitlines() if l.startswith("// RUN:")), "")
        m = re.search(r"--pass=([\w,-]+)", run_line)
        passes = m.group(1) if m else ("pipeline" if "--pipeline" in run_line else "-")
        model = "\n".join(l for l in text.splitlines() if not l.lstrip().startswith("//")).strip() + "\n"
        inp = HERE / f"{name}.lkir"
        inp.write_text(model)
        (HERE / f"{name}.stage").write_text(passes + "\n")
        rc, out = run("passes", passes, inp) if passes != "-" else run("print", inp)
        (HERE / f"{name}.stage.txt").write_text(out if rc == 0 else "rejected\n")
        rc, out = run("passes", "pipeline", inp)
        if rc == 0:
            (HERE / f"{name}.pipeline.txt").write_text(out)
            if "const.external" not in model:
                lkm = HERE / f"{name}.lkm"
                if run("to-lkm", "pipeline", inp, lkm)[0] == 0:
                    (HERE / f"{name}.lkm.txt").write_text(run("from-lkm", lkm)[1])
        print("wrote", name)


if __name__ == "__main__":
    main()
