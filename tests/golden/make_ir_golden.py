"""Writes the golden text-IR and .lkm fixtures of tests/golden/ir/ with the reference's own IR library.

Run in the build container (it needs /root/reference): `make -f oracle/ref_ir.mk` builds oracle/_ref/lkm-ref-tool
from the reference's src/ir + src/compiler sources, then `python tests/golden/make_ir_golden.py` runs it over every
tests/golden/ir/*.lkir and writes, next to each input:
  NAME.print.txt      the parsed model printed back
  NAME.P.txt          after the passes P (bufferize = dce,bufferize; plan = dce,bufferize,plan-memory; pipeline)
  NAME.lkm            the pipeline's result saved as .lkm v2, internal constants filled with fixture bytes
                      (byte k of constant c = (k * 29 + sum of c's name bytes) mod 251)
  NAME.lkm.txt        that file read back and printed
Models with external constants get no .lkm (the format cannot hold them)."""
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent / "ir"
TOOL = Path(__file__).resolve().parents[2] / "oracle" / "_ref" / "lkm-ref-tool"
PASSES = {"bufferize": "dce,bufferize", "plan": "dce,bufferize,plan-memory", "pipeline": "pipeline"}


def run(*args):
    return subprocess.run([str(TOOL), *map(str, args)], check=True, capture_output=True, text=True).stdout


def main():
    if not TOOL.exists():
        sys.exit(f"{TOOL} is not built: make -f oracle/ref_ir.mk")
    for src in sorted(HERE.glob("*.lkir")):
        name = src.stem
        (HERE / f"{name}.print.txt").write_text(run("print", src))
        for tag, passes in PASSES.items():
            (HERE / f"{name}.{tag}.txt").write_text(run("passes", passes, src))
        if "const.external" not in src.read_text():
            lkm = HERE / f"{name}.lkm"
            run("to-lkm", "pipeline", src, lkm)
            (HERE / f"{name}.lkm.txt").write_text(run("from-lkm", lkm))
        print("wrote", name)


if __name__ == "__main__":
    main()
