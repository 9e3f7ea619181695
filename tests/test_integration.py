"""The reference-side binding (integration/hip_backend.cpp) compiles against the reference's own headers
(lariaus/lokinfer include/lokinfer/runtime/kernel.h, ir/ir.h) and this backend's C-ABI (include/lokinfer_hip.h), so
the registration, the prepare / run / destroy lifecycle and the float-attribute count a maintainer adds are real
code, not a sketch. Runs in the build container, where /root/reference is present; skipped elsewhere."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
REF = Path("/root/reference/include")


@pytest.mark.skipif(not REF.exists() or not shutil.which("g++"), reason="reference headers or g++ not available")
def test_binding_compiles_against_reference_headers():
    r = subprocess.run(["g++", "-std=c++20", "-fsyntax-only", f"-I{REF}", f"-I{ROOT / 'include'}",
                        str(ROOT / "integration" / "hip_backend.cpp")], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_binding_uses_only_declared_entry_points():
    src = (ROOT / "integration" / "hip_backend.cpp").read_text()
    hdr = (ROOT / "include" / "lokinfer_hip.h").read_text()
    import re

    used = set(re.findall(r"\b(lk_\w+)\s*\(", src))
    assert used and all(re.search(rf"\b{u}\s*\(", hdr) for u in used), used
