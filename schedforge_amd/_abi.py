"""ctypes binding of include/sfg_hip.h (libsfg_hip.so).

Loading fails loudly: there is no CPU fallback anywhere in this package.
Status codes map to the reference's error convention: codes below 16 raise
ValueError (std::invalid_argument in decoder_compiler.cpp:26-39 and friends),
codes from 16 up raise RuntimeError (std::runtime_error).
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libsfg_hip.so"

ABI_VERSION = 1

F32, BF16, I8, I32 = 0, 1, 2, 3
EPI_NONE, EPI_RESIDUAL, EPI_SWIGLU, EPI_GLU_SILU_UP = 0, 1, 2, 3
LAYOUT_NK, LAYOUT_TILED = 0, 1
# sfg_gemm_tile
TILE_AUTO, TILE_256x256_PP, TILE_256x256_W8, TILE_256x256_W4, TILE_256x128, TILE_128x256, \
    TILE_128x128, TILE_256x256_V, TILE_COUNT = range(9)

TAP_ATTN, TAP_RESIDUAL1, TAP_NORM2, TAP_ROUTE_INPUT, TAP_ROUTE_IDS, TAP_ROUTE_WEIGHTS, NUM_TAPS = range(7)

(MARK_START, MARK_NORM1, MARK_QKV, MARK_ROPE, MARK_ATTN_MAIN, MARK_ATTN, MARK_OPROJ,
 MARK_NORM2, MARK_ROUTE, MARK_FFN_UP, MARK_FFN_DOWN, MARK_END, NUM_MARKS) = range(13)

ERR_INVALID_CONFIG, ERR_SHAPE, ERR_GUARD, ERR_UNSUPPORTED, ERR_ABI = 1, 2, 3, 4, 5
ERR_DEVICE, ERR_WORKSPACE = 16, 17

c_i32, c_i64, c_f32, c_vp, c_sz = (ctypes.c_int32, ctypes.c_int64, ctypes.c_float,
                                    ctypes.c_void_p, ctypes.c_size_t)


class SfgError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[sfg {code}] {message}")
        self.code = code


class SfgInvalidArgument(ValueError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[sfg {code}] {message}")
        self.code = code


class TargetInfo(ctypes.Structure):
    _fields_ = [
        ("architecture", ctypes.c_char * 64), ("wavefront", c_i32), ("compute_units", c_i32),
        ("xcds", c_i32), ("simds_per_cu", c_i32), ("lds_bytes_per_cu", c_i64),
        ("l2_bytes_per_xcd", c_i64), ("hbm_bytes", c_i64), ("engine_clock_ghz", ctypes.c_double),
        ("hbm_gbps", ctypes.c_double), ("mfma_bf16_tflops", ctypes.c_double),
        ("valu_fp32_tflops", ctypes.c_double),
    ]


class GemmArgs(ctypes.Structure):
    _fields_ = [
        ("a", c_vp), ("a_dtype", c_i32), ("lda", c_i64),
        ("b", c_vp), ("b_dtype", c_i32), ("ldb", c_i64), ("b_scales", c_vp),
        ("c", c_vp), ("c_dtype", c_i32), ("ldc", c_i64),
        ("residual", c_vp), ("ldr", c_i64),
        ("m", c_i64), ("n", c_i64), ("k", c_i64),
        ("epilogue", c_i32), ("b_layout", c_i32), ("tile", c_i32),
    ]


class LayerDesc(ctypes.Structure):
    _fields_ = [
        ("abi", c_i32),
        ("batch", c_i32), ("sequence", c_i32), ("hidden", c_i32), ("intermediate", c_i32),
        ("query_heads", c_i32), ("kv_heads", c_i32), ("head_dim", c_i32),
        ("rms_epsilon", c_f32), ("rope_theta", c_f32),
        ("causal", c_i32), ("ffn", c_i32), ("experts", c_i32), ("top_k", c_i32),
        ("context", c_i32), ("page_tokens", c_i32), ("pages_per_seq", c_i32),
        ("num_pages", c_i32), ("act_dtype", c_i32), ("weight_dtype", c_i32),
        ("kv_splits", c_i32), ("use_routing_trace", c_i32), ("weight_layout", c_i32),
        ("kv_append", c_i32), ("gemm_tile", c_i32), ("attn_waves", c_i32),
    ]


class LayerWeights(ctypes.Structure):
    _fields_ = [
        ("rms1", c_vp), ("rms2", c_vp),
        ("w_qkv", c_vp), ("s_qkv", c_vp),
        ("w_o", c_vp), ("s_o", c_vp),
        ("w_gate_up", c_vp), ("s_gate_up", c_vp),
        ("w_down", c_vp), ("s_down", c_vp),
        ("router", c_vp), ("router_bias", c_vp),
        ("w13", c_vp), ("s13", c_vp),
        ("w2", c_vp), ("s2", c_vp),
        ("k_pool", c_vp), ("v_pool", c_vp),
        ("page_table", c_vp),
        ("rope_table", c_vp),
    ]


class LayerIO(ctypes.Structure):
    _fields_ = [
        ("x", c_vp), ("out", c_vp),
        ("trace_ids", c_vp), ("trace_weights", c_vp),
        ("stage_events", ctypes.POINTER(c_vp)),
        ("seq_lens", c_vp),
    ]


_SIGNATURES = {
    "sfg_hip_abi_version": (c_i32, []),
    "sfg_hip_metadata_v1": (ctypes.c_char_p, []),
    "sfg_hip_last_error": (ctypes.c_char_p, []),
    "sfg_hip_device_info_v1": (c_i32, [ctypes.c_int, ctypes.POINTER(ctypes.c_int),
                                       ctypes.POINTER(ctypes.c_int), ctypes.POINTER(c_i64)]),
    "sfg_hip_target_info_v1": (c_i32, [ctypes.c_int, ctypes.POINTER(TargetInfo)]),
    "sfg_hip_pack_weight_v1": (c_i32, [c_vp, c_i64, c_i64, c_i64, c_vp, ctypes.c_int, ctypes.c_int,
                                       c_vp]),
    "sfg_hip_quantize_weight_v1": (c_i32, [c_vp, c_i64, c_i64, c_vp, c_vp, ctypes.c_int, c_vp]),
    "sfg_hip_preferred_weight_layout_v1": (c_i32, [c_i64, c_i64, ctypes.c_int]),
    "sfg_hip_to_bf16_v1": (c_i32, [c_vp, c_vp, c_i64, c_vp]),
    "sfg_hip_rope_table_host_v1": (c_i32, [c_vp, c_i64, c_i64, c_f32]),
    "sfg_hip_rmsnorm_v1": (c_i32, [c_vp, c_vp, c_vp, ctypes.c_int, c_i64, c_i64, c_f32, c_vp]),
    "sfg_hip_gemm_workspace_v1": (c_sz, [c_i64, c_i64, c_i64]),
    "sfg_hip_gemm_v1": (c_i32, [ctypes.POINTER(GemmArgs), c_vp, c_sz, c_vp]),
    "sfg_hip_qkv_split_rope_v1": (c_i32, [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64,
                                          c_vp, c_vp, c_vp, ctypes.c_int, c_vp]),
    "sfg_hip_attn_prefill_v1": (c_i32, [c_vp, c_vp, c_vp, c_vp, ctypes.c_int, ctypes.c_int,
                                        c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, ctypes.c_int,
                                        c_f32, c_vp]),
    "sfg_hip_attn_vt_ld_v1": (c_i64, [c_i64]),
    "sfg_hip_qkv_split_rope_vt_v1": (c_i32, [c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64,
                                             c_vp, c_vp, c_vp, c_i64, c_vp]),
    "sfg_hip_attn_prefill_vt_v1": (c_i32, [c_vp, c_vp, c_vp, c_i64, c_vp, ctypes.c_int, c_i64,
                                           c_i64, c_i64, c_i64, c_i64, c_i64, ctypes.c_int, c_f32,
                                           c_vp]),
    "sfg_hip_attn_decode_workspace_v1": (c_sz, [c_i64, c_i64, c_i64, c_i64, c_i64, c_i32]),
    "sfg_hip_attn_decode_paged_v1": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, ctypes.c_int,
                                             c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,
                                             c_i64, c_i32, c_f32, ctypes.c_int, c_vp, c_sz,
                                             c_vp]),
    "sfg_hip_attn_decode_paged_noalloc_v1": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, ctypes.c_int,
                                                     c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,
                                                     c_i64, c_i32, c_f32, c_vp]),
    "sfg_hip_gemm_grouped_v1": (c_i32, [ctypes.POINTER(GemmArgs), c_vp, c_i64, c_vp, ctypes.c_int, c_i64, c_i64, c_vp, c_sz,
                                        c_vp]),
    "sfg_hip_attn_paged_workspace_v1": (c_sz, [c_i64, c_i64, c_i64, c_i64, c_i64, ctypes.c_int, c_i64,
                                               c_i64, c_i32]),
    "sfg_hip_attn_paged_v1": (c_i32, [c_vp, c_vp, c_vp, ctypes.c_int, c_vp, c_vp, c_vp, ctypes.c_int,
                                      c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,
                                      ctypes.c_int, c_i32, c_f32, ctypes.c_int, c_vp, c_sz, c_vp]),
    "sfg_hip_kv_append_pool_v1": (c_i32, [c_vp, c_vp, ctypes.c_int, c_vp, c_vp, ctypes.c_int, c_vp, c_vp,
                                          c_i64, ctypes.c_int, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,
                                          c_i64, c_vp]),
    "sfg_hip_kv_gather_pool_v1": (c_i32, [c_vp, c_vp, ctypes.c_int, c_vp, c_i64, c_i64, c_i64, c_i64,
                                          c_i64, c_i64, c_i64, c_vp, c_vp, c_vp]),
    "sfg_hip_kv_append_paged_v1": (c_i32, [c_vp, c_vp, ctypes.c_int, c_vp, c_vp, c_vp, c_vp, c_i64,
                                           ctypes.c_int, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,
                                           c_i64, c_vp]),
    "sfg_hip_kv_gather_paged_v1": (c_i32, [c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,
                                           c_i64, c_vp, c_vp, c_vp]),
    "sfg_hip_moe_route_workspace_v1": (c_sz, [c_i64, c_i64, c_i64]),
    "sfg_hip_moe_route_v1": (c_i32, [c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp,
                                     c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_sz, c_vp]),
    "sfg_hip_moe_dispatch_trace_v1": (c_i32, [c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp,
                                              c_vp, c_vp, c_vp, c_vp]),
    "sfg_hip_moe_expert_workspace_v1": (c_sz, [c_i64, c_i64, c_i64, c_i64, c_i64]),
    "sfg_hip_moe_experts_v1": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, ctypes.c_int,
                                       ctypes.c_int, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp,
                                       c_sz, c_vp]),
    "sfg_hip_moe_combine_v1": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp]),
    "sfg_hip_decoder_layer_workspace_v1": (c_sz, [ctypes.POINTER(LayerDesc)]),
    "sfg_hip_decoder_layer_tap_v1": (c_i32, [ctypes.POINTER(LayerDesc), ctypes.c_int,
                                             ctypes.POINTER(c_sz), ctypes.POINTER(c_sz),
                                             ctypes.POINTER(ctypes.c_int)]),
    "sfg_hip_decoder_layer_v1": (c_i32, [ctypes.POINTER(LayerDesc), ctypes.POINTER(LayerWeights),
                                         ctypes.POINTER(LayerIO), c_vp, c_sz, c_vp]),
    "sfg_hip_events_create_v1": (c_i32, [ctypes.c_int, ctypes.POINTER(c_vp)]),
    "sfg_hip_events_destroy_v1": (c_i32, [ctypes.c_int, ctypes.POINTER(c_vp)]),
    "sfg_hip_event_elapsed_v1": (c_i32, [c_vp, c_vp, ctypes.POINTER(c_f32)]),
    "sfg_hip_stream_synchronize_v1": (c_i32, [c_vp]),
}

EXPORTED = tuple(_SIGNATURES)

_lib = None


def load(path: os.PathLike | str | None = None) -> ctypes.CDLL:
    """Load libsfg_hip.so; raise if it is missing (build with __graft_entry__.build())."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise RuntimeError(f"libsfg_hip.so not built: {p} is missing "
                           "(run python -c 'import __graft_entry__ as g; g.build()')")
    lib = ctypes.CDLL(str(p))
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if lib.sfg_hip_abi_version() != ABI_VERSION:
        raise RuntimeError("libsfg_hip.so ABI version mismatch")
    if path is None:
        _lib = lib
    return lib


def check(rc: int) -> None:
    if rc == 0:
        return
    msg = load().sfg_hip_last_error().decode(errors="replace")
    if rc < 16:
        raise SfgInvalidArgument(rc, msg)
    raise SfgError(rc, msg)
