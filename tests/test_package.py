""".sfe GPU packages of a compiled decoder plan (schedforge_amd/runtime/
sfg_package.cpp), after the reference's AOT package format 1
(src/aot_runtime.cpp:217-316; docs/AOT_DEPLOYMENT.md:6-35).

CPU: a package written here by an independent Python writer (its own FNV-1a,
pinned by the algorithm's published test vectors, and its own ELF / offload
bundle reader) passes `sfg-decoder --inspect`; every tampered variant the
reference's loader rejects (format version, ABI, target, checksums, embedded
metadata, duplicate or missing fields, paths outside the package) is rejected
with a std::runtime_error, and a code object that differs from the one the
library embeds is rejected too.
GPU: a plan compiled, packaged and loaded back gives the compiled plan's output
bit for bit (same kernels, same device constants), for fp32, bf16 decode over a
paged cache and int8-weight MoE plans; a tampered buffer is refused at load.
"""
from __future__ import annotations

import functools
import shutil
import struct
from pathlib import Path

import numpy as np
import pytest

import oracle
from schedforge_amd import CONFIG_SEEDS
from schedforge_amd.build import DECODER_CLI, LIB

from _helpers import SMALL, TOL
from test_runtime import cfg_args, load, run_cli

pytestmark = pytest.mark.skipif(not DECODER_CLI.exists() or not LIB.exists(),
                                reason="sfg-decoder / libsfg_hip.so not built")


# ------------------------------------------------------------------ Python writer


@functools.lru_cache(maxsize=64)
def fnv1a64(data: bytes) -> str:
    h = 0xCBF29CE484222325
    for b in data:
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return f"{h:016x}"


def test_fnv1a64_published_vectors():
    """FNV-1a 64-bit test vectors (Fowler/Noll/Vo reference values)."""
    assert fnv1a64(b"") == "cbf29ce484222325"
    assert fnv1a64(b"a") == "af63dc4c8601ec8c"
    assert fnv1a64(b"foobar") == "85944171f73967e8"


def code_objects(lib: bytes):
    """(target id, bytes) of each amdgcn entry of the clang offload bundles in
    the .hip_fatbin section."""
    shoff, = struct.unpack_from("<Q", lib, 0x28)
    shentsize, shnum, shstrndx = struct.unpack_from("<HHH", lib, 0x3A)
    secs = [struct.unpack_from("<IIQQQQ", lib, shoff + i * shentsize) for i in range(shnum)]
    names = secs[shstrndx][4]
    fat = next(s for s in secs if lib[names + s[0]:].split(b"\0", 1)[0] == b".hip_fatbin")
    sec = lib[fat[4]:fat[4] + fat[5]]
    out, pos = [], 0
    while pos + 32 <= len(sec):
        if sec[pos:pos + 24] != b"__CLANG_OFFLOAD_BUNDLE__":
            pos += 8
            continue
        n, = struct.unpack_from("<Q", sec, pos + 24)
        p = end = pos + 32
        for _ in range(n):
            off, size, idl = struct.unpack_from("<QQQ", sec, p)
            tid = sec[p + 24:p + 24 + idl].decode()
            p += 24 + idl
            if size and "amdgcn" in tid:
                out.append((tid, sec[pos + off:pos + off + size]))
            end = max(end, pos + off + size)
        pos = (max(end, p) + 7) // 8 * 8
    return out


def test_library_embeds_gfx950_code_objects():
    objs = code_objects(LIB.read_bytes())
    assert objs
    for tid, blob in objs:
        assert tid.endswith("--gfx950")
        assert blob[:4] == b"\x7fELF"
        e_machine, = struct.unpack_from("<H", blob, 18)
        assert e_machine == 224  # EM_AMDGPU


def _manifest_lines(root: Path, lib_meta: str, buffers, extra=None):
    cfg = SMALL["c1"]
    lib = (root / "libsfg_hip.so").read_bytes()
    plan = (root / "plan.sfe").read_bytes()
    const = (root / "constants.bin").read_bytes()
    f = {
        "format_version": "1", "schedforge_version": "0.9.0", "abi": "sfg_hip_decoder_layer_v1",
        "symbol": "sfg_hip_decoder_layer_v1", "target": "gfx950", "library_abi": "1",
        "library_metadata": lib_meta, "batch": cfg.batch, "sequence": cfg.sequence,
        "hidden": cfg.hidden, "intermediate": cfg.intermediate, "query_heads": cfg.query_heads,
        "kv_heads": cfg.kv_heads, "head_dim": cfg.head_dim, "rms_epsilon": "9.99999997e-07",
        "rope_theta": "10000", "causal": 1, "ffn": "dense_swiglu", "experts": 4, "top_k": 2,
        "context_sequence": 0, "precision": "f32", "page_tokens": 16, "weight_layout": 0,
        "kv_splits": 0, "gemm_tile": 0, "attn_waves": 0, "pages_per_seq": 0, "num_pages": 0,
        "routing_trace": 0,
        "workspace_bytes": 4096, "naive_bytes": 1,
        "plan": f"plan.sfe,{len(plan)},{fnv1a64(plan)}",
        "library": f"libsfg_hip.so,{len(lib)},{fnv1a64(lib)}",
        "constants": f"constants.bin,{len(const)},{fnv1a64(const)}",
    }
    objs = sorted((root / "kernels").iterdir())
    f["code_objects"] = len(objs)
    for i, (tid, _) in enumerate(code_objects(lib)):
        blob = objs[i].read_bytes()
        f[f"code_object.{i}"] = f"kernels/{objs[i].name},{len(blob)},{fnv1a64(blob)},{tid}"
    f["buffers"] = len(buffers)
    for i, (name, off, data) in enumerate(buffers):
        f[f"buffer.{i}"] = f"{name},{off},{len(data)},{fnv1a64(data)}"
    f["constant_table"] = 1
    f["constant.0"] = "rms1_weight;256;256;f32;1024"
    f.update(extra or {})
    return [f"{k}={v}" for k, v in f.items() if v is not None]


def write_package(root: Path, extra=None, corrupt=None):
    """A package of synthetic content around the real libsfg_hip.so."""
    import ctypes
    root.mkdir(parents=True)
    (root / "kernels").mkdir()
    shutil.copyfile(LIB, root / "libsfg_hip.so")
    for i, (_, blob) in enumerate(code_objects(LIB.read_bytes())):
        (root / "kernels" / f"{i:02d}.gfx950.hsaco").write_bytes(blob)
    (root / "plan.sfe").write_text("sfe.decoder_executable version=0.9.0 target=gfx950 {\n}\n")
    rng = np.random.default_rng(5)
    a = rng.standard_normal(256).astype(np.float32).tobytes()
    b = rng.standard_normal(300).astype(np.float32).tobytes()
    off_b = (len(a) + 255) // 256 * 256
    const = a + bytes(off_b - len(a)) + b
    (root / "constants.bin").write_bytes(const)
    if corrupt:
        corrupt(root)
    meta = ctypes.CDLL(str(LIB)).sfg_hip_metadata_v1
    meta.restype = ctypes.c_char_p
    lines = _manifest_lines(root, meta().decode(), [("rms1_weight", 0, a), ("rms2_weight", off_b, b)],
                            extra)
    (root / "manifest.sfe").write_text("# SchedForge GPU Executable\n" + "\n".join(lines) + "\n")
    return root


def inspect(path):
    return run_cli([f"--inspect={path}"], timeout=120)


def test_inspect_accepts_python_written_package(tmp_path):
    """The C++ FNV-1a, manifest parser and code-object reader agree with this
    file's independent ones."""
    r = inspect(write_package(tmp_path / "ok.sfe"))
    assert r.returncode == 0, r.stderr
    assert "package valid" in r.stdout and "format_version=1" in r.stdout
    assert "sfe.decoder_executable" in r.stdout


def _flip(rel, at=100):
    def corrupt(root):
        p = root / rel
        data = bytearray(p.read_bytes())
        data[at] ^= 0x40
        p.write_bytes(bytes(data))
    return corrupt


@pytest.mark.parametrize("extra, corrupt, message", [
    ({"format_version": "2"}, None, "unsupported .sfe format version"),
    ({"abi": "schedforge_matmul_v1"}, None, "unsupported .sfe ABI"),
    ({"symbol": "sfg_hip_gemm_v1"}, None, "unsupported .sfe ABI"),
    ({"target": "gfx942"}, None, "unsupported .sfe target"),
    ({"library_metadata": "abi=1;arch=gfx950"}, None, "embedded metadata mismatch: library_metadata"),
    ({"library_abi": "2"}, None, "embedded metadata mismatch: library_abi"),
    ({"hidden": None}, None, "missing .sfe manifest field: hidden"),
    ({"hidden": "100"}, None, ".sfe configuration"),
    ({"plan": "../plan.sfe,10,0123456789abcdef"}, None, "invalid .sfe package path"),
    ({"buffer.1": "rms2_weight,100,1200,0123456789abcdef"}, None, "outside constants.bin"),
])
def test_inspect_rejects_manifest_mismatch(tmp_path, extra, corrupt, message):
    r = inspect(write_package(tmp_path / "bad.sfe", extra, corrupt))
    assert r.returncode == 1 and message in r.stderr, r.stderr


def test_inspect_rejects_duplicate_field(tmp_path):
    root = write_package(tmp_path / "dup.sfe")
    with open(root / "manifest.sfe", "a") as f:
        f.write("target=gfx950\n")
    r = inspect(root)
    assert r.returncode == 1 and "duplicate .sfe manifest field: target" in r.stderr


def test_inspect_rejects_changed_files(tmp_path):
    """A byte changed after the manifest was written: the file checksum; a
    buffer changed with the whole-file checksum rewritten: the buffer's own; a
    code object replaced with its checksum rewritten: the comparison with the
    one embedded in the library."""
    root = write_package(tmp_path / "a.sfe")
    _flip("constants.bin")(root)
    r = inspect(root)
    assert r.returncode == 1 and "checksum mismatch: constants.bin" in r.stderr

    r = inspect(write_package(tmp_path / "b.sfe", corrupt=_flip("constants.bin", 1100)))
    assert r.returncode == 1 and "checksum mismatch: buffer rms2_weight" in r.stderr

    root = write_package(tmp_path / "c.sfe")
    _flip("libsfg_hip.so", 5000)(root)
    r = inspect(root)
    assert r.returncode == 1 and "checksum mismatch: libsfg_hip.so" in r.stderr

    r = inspect(write_package(tmp_path / "d.sfe", corrupt=_flip("kernels/00.gfx950.hsaco", 300)))
    assert r.returncode == 1 and "differs from the one embedded" in r.stderr

    r = inspect(tmp_path / "missing.sfe")
    assert r.returncode == 1 and "not a directory" in r.stderr


# ------------------------------------------------------------------ GPU


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["c1", "c2", "c5"])
def test_package_round_trip_is_bit_exact(tmp_path, name):
    cfg = SMALL[name]
    seed = CONFIG_SEEDS[name] + 31
    pkg = tmp_path / f"{name}.sfe"
    a, b = tmp_path / "compiled.bin", tmp_path / "loaded.bin"
    args = cfg_args(cfg, seed) + ["--repetitions=1", "-o", str(tmp_path / "plan.sfe")]
    print("sfg-decoder compile+package", name, flush=True)
    r = run_cli(args + [f"--package={pkg}", f"--dump-output={a}"], timeout=240)
    assert r.returncode == 0, r.stderr
    assert "[Package]" in r.stdout
    manifest = (pkg / "manifest.sfe").read_text()
    assert f"precision={cfg.dtype}" in manifest and "target=gfx950" in manifest
    assert (pkg / "plan.sfe").read_text() == (tmp_path / "plan.sfe").read_text()
    # the oracle's output for the same seeded inputs: the loaded plan is checked
    # against it (benchmark_aot_package validates against the reference,
    # aot_runtime.cpp:346-350), not only against the plan it was saved from
    ref = oracle.decoder_layer(cfg, oracle.make_layer_data(cfg, seed))
    expect = tmp_path / "expect.bin"
    ref.astype(np.float32).tofile(expect)
    print("sfg-decoder load-package", name, flush=True)
    r = run_cli([f"--load-package={pkg}", f"--seed={seed}", "--repetitions=1",
                 f"--router-bias-std={cfg.router_bias_std!r}", f"--dump-output={b}",
                 f"--expect={expect}", f"--max-error={TOL[cfg.dtype]}",
                 "-o", str(tmp_path / "plan2.sfe")], timeout=240)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr
    assert "max relative error" in r.stdout
    loaded = load(b).reshape(ref.shape)
    assert oracle.rel_error(loaded, ref) < TOL[cfg.dtype]
    np.testing.assert_array_equal(load(a).view(np.uint32), load(b).view(np.uint32))
    compiled = (tmp_path / "plan.sfe").read_text().splitlines()
    reloaded = (tmp_path / "plan2.sfe").read_text().splitlines()
    strip = lambda lines: [l for l in lines if not l.startswith("compile_ms=")]
    assert strip(compiled) == strip(reloaded)


@pytest.mark.gpu
def test_load_refuses_tampered_buffer(tmp_path):
    cfg = SMALL["c1"]
    pkg = tmp_path / "c1.sfe"
    r = run_cli(cfg_args(cfg, 7) + ["--repetitions=1", f"--package={pkg}", "-o",
                                    str(tmp_path / "plan.sfe")], timeout=240)
    assert r.returncode == 0, r.stderr
    _flip("constants.bin", 2000)(pkg)
    r = run_cli([f"--load-package={pkg}", "--repetitions=1"], timeout=240)
    assert r.returncode == 1 and "checksum mismatch" in r.stderr
