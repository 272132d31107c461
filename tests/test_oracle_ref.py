"""The oracle's fp32 GEMM (sfgo_matmul) against the reference's own CPU GEMM
runtime -- CPU only.

oracle/_ref/libsfg_ref_gemm.so is the reference's runtime, IR and compiler
sources compiled where they lie (oracle/Makefile, target `ref`) behind a
small C entry point (oracle/ref_gemm.cpp).  It plans each GEMM with
apply_schedule() under the schedule the reference decoder gives its
projections (decoder_schedule(), src/decoder_compiler.cpp:196-208) and runs it
with execute() (src/runtime.cpp:581-623), as the decoder's run step does
(src/decoder_compiler.cpp:230, 252, 272-276).  The oracle must agree bit for
bit: on the fp32 layer's four projection GEMMs at the reference's
CPU-runnable size, and on ragged shapes that reach each of the reference's
code paths (16-wide and 8-wide register kernels, 1..4-row remainders, the
scalar column tail), under both schedule families and several thread counts.

Skipped where neither the built library nor the reference sources are
present (the GPU box runs only `-m gpu`).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle

ref = oracle.ref_gemm_lib()
pytestmark = pytest.mark.skipif(ref is None, reason="reference GEMM library not buildable here")


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _operands(m, n, k, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((m, k)).astype(np.float32),
            rng.standard_normal((k, n)).astype(np.float32))


# configs[0] (rows 128, hidden 256, intermediate 688, 4 query / 2 kv heads of 64)
_C1 = {"qkv": (128, 256 + 2 * 128, 256), "output": (128, 256, 256),
       "gate_up": (128, 2 * 688, 256), "down": (128, 256, 688)}


@pytest.mark.parametrize("name", sorted(_C1))
@pytest.mark.parametrize("threads", [1, 4])
def test_layer_projection_gemms_match_reference_execute(name, threads):
    m, n, k = _C1[name]
    a, b = _operands(m, n, k, 11)
    want = oracle.reference_gemm(a, b, family=0, threads=threads)
    np.testing.assert_array_equal(_bits(oracle.matmul(a, b)), _bits(want))


# (m, n, k): m % 4 remainders of 1..3 rows; n with 16-wide, 8-wide and scalar
# column tails; k = 1 and odd k
_RAGGED = [(1, 1, 1), (3, 5, 7), (5, 23, 33), (7, 9, 1), (33, 100, 77), (2, 40, 129),
           (257, 130, 600), (64, 1376, 256)]


@pytest.mark.parametrize("m,n,k", _RAGGED)
@pytest.mark.parametrize("family", [0, 1])
def test_ragged_gemms_match_reference_execute(m, n, k, family):
    a, b = _operands(m, n, k, m * 1000 + n + k)
    want = oracle.reference_gemm(a, b, family=family, threads=3)
    np.testing.assert_array_equal(_bits(oracle.matmul(a, b)), _bits(want))


def test_comparison_sees_a_change_of_rounding():
    """A chain that rounds each product before adding it (no FMA) differs
    from the reference in the low bits on random operands, so the bit-for-bit
    comparisons above would catch an oracle that lost its fused steps."""
    a, b = _operands(3, 5, 40, 5)
    want = oracle.reference_gemm(a, b)
    unfused = np.zeros((3, 5), np.float32)
    for kk in range(40):
        unfused = (unfused + (a[:, kk:kk + 1] * b[kk:kk + 1, :]).astype(np.float32)).astype(np.float32)
    assert not np.array_equal(_bits(unfused), _bits(want))
    np.testing.assert_allclose(unfused, want, rtol=1e-5, atol=1e-5)


def test_reference_rejects_bad_extents():
    c = np.empty(1, np.float32)
    assert ref.sfgr_decoder_gemm(oracle._f(c), oracle._f(c), oracle._f(c), 0, 1, 1, 0, 1) == 1
