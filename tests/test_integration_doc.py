"""The integration guide's reference-side C++ binding compiles against
include/sfg_hip.h (CPU only): every ```cpp block of the guide, in order, as one
translation unit, checked with g++ -std=c++20 -fsyntax-only -- so a stub call
with the wrong number or type of arguments fails here."""
from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
ROCM = Path("/opt/rocm")


@pytest.mark.skipif(shutil.which("g++") is None or not (ROCM / "include" / "hip").exists(),
                    reason="needs g++ and the HIP headers")
def test_integration_stub_compiles(tmp_path):
    text = (ROOT / "INTEGRATION.md").read_text()
    blocks = re.findall(r"```cpp\n(.*?)```", text, re.S)
    assert len(blocks) >= 4
    src = tmp_path / "integration_stub.cpp"
    src.write_text("\n".join(blocks))
    r = subprocess.run(["g++", "-std=c++20", "-fsyntax-only", "-Wall", "-D__HIP_PLATFORM_AMD__",
                        f"-I{ROOT / 'include'}", f"-I{ROCM / 'include'}", str(src)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
