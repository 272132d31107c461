"""Build libsfg_hip.so (gfx950) and the C++20 host runtime in-tree.

Every translation unit under csrc/ is compiled to an object in parallel, then
linked into schedforge_amd/lib/libsfg_hip.so.  Flags:
  --offload-arch=gfx950          MI355X only
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                 no packed-fp32 VALU ops in device code
  -O3 -std=c++20 -fPIC
The host runtime under runtime/ is plain C++20 (g++, the reference's own
toolchain) against the HIP runtime API: schedforge_amd/lib/libsfg_decoder.so
and the drivers schedforge_amd/bin/sfg-decoder and sfg-decoder-bench.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIBDIR = PKG / "lib"
LIB = LIBDIR / "libsfg_hip.so"
RUNTIME = PKG / "runtime"
BINDIR = PKG / "bin"
RUNTIME_LIB = LIBDIR / "libsfg_decoder.so"
DECODER_CLI = BINDIR / "sfg-decoder"
BENCH_CLI = BINDIR / "sfg-decoder-bench"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
CXX = os.environ.get("CXX", "g++")
HOST_FLAGS = ["-std=c++20", "-O2", "-Wall", "-Wextra", "-fPIC", "-D__HIP_PLATFORM_AMD__",
              f"-I{PKG.parent / 'include'}", f"-I{ROCM / 'include'}"]
HIP_LINK = [f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}", "-ldl", "-pthread"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; drop
    # those lines, keep everything else.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def _run(cmd: list, what: str) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"{what} failed:\n{proc.stderr}")
    if proc.stderr.strip():
        sys.stderr.write(proc.stderr)


def build_runtime() -> Path:
    """libsfg_decoder.so + sfg-decoder + sfg-decoder-bench from runtime/*.cpp."""
    BUILD.mkdir(exist_ok=True)
    BINDIR.mkdir(exist_ok=True)
    lib_srcs = ["sfg_decoder", "sfg_package", "sfg_optimizer"]
    clis = {"sfg_decoder_cli": DECODER_CLI, "sfg_decoder_bench_cli": BENCH_CLI}
    units = [(RUNTIME / f"{n}.cpp", BUILD / f"{n}.o") for n in [*lib_srcs, *clis]]
    with cf.ThreadPoolExecutor(max_workers=len(units)) as pool:
        jobs = [pool.submit(_run, [CXX, *HOST_FLAGS, "-c", str(src), "-o", str(obj)], f"g++ {src.name}")
                for src, obj in units]
        for j in jobs:
            j.result()
    tmp = RUNTIME_LIB.with_suffix(".so.tmp")
    _run([CXX, "-shared", "-o", str(tmp), *(str(BUILD / f"{n}.o") for n in lib_srcs), *HIP_LINK],
         "link libsfg_decoder.so")
    os.replace(tmp, RUNTIME_LIB)
    for name, exe in clis.items():
        tmp_cli = exe.with_suffix(".tmp")
        _run([CXX, "-o", str(tmp_cli), str(BUILD / f"{name}.o"), f"-L{LIBDIR}", "-lsfg_decoder",
              "-Wl,-rpath,$ORIGIN/../lib", *HIP_LINK], f"link {exe.name}")
        os.replace(tmp_cli, exe)
    return DECODER_CLI


def build(verbose: bool = False) -> Path:
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    BUILD.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    jobs = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    build_runtime()
    if verbose:
        print(f"built {LIB}, {RUNTIME_LIB} and {DECODER_CLI}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
