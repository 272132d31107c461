"""CPU oracle for the decoder-layer path -- TEST INFRASTRUCTURE ONLY.

Python front of oracle/_build/libsfg_oracle.so (a C restatement of the
reference, sfg_oracle.c).  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this package, and only as the checker; the product
(schedforge_amd) never does.

Also holds the seeded input generator used by the parity tests: counter-based
N(mean, std) per (config seed, tensor id, index), tensor ids as listed below,
bf16 configs rounded to bf16 (RNE) before either side sees them, and a seeded
Fisher-Yates permutation for the physical page assignment.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libsfg_oracle.so"

# tensor ids of the synthetic-input spec
TID = {"x": 0, "rms1": 1, "wq": 2, "wk": 3, "wv": 4, "wo": 5, "rms2": 6, "wg": 7, "wu": 8,
       "wd": 9, "router": 10, "router_bias": 11, "w1": 12, "w3": 13, "w2": 14, "k_cache": 15,
       "v_cache": 16, "pages": 17}

_lib = None

fp = ctypes.POINTER(ctypes.c_float)
ip = ctypes.POINTER(ctypes.c_int32)
i8p = ctypes.POINTER(ctypes.c_int8)
i64 = ctypes.c_int64


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


# The reference's own CPU GEMM runtime (oracle/ref_gemm.cpp over the reference
# sources, `make ref`): built in this container only, where the sources are;
# the built library travels with the tree.
REF_ROOT = Path("/root/reference")
REF_LIB_PATH = HERE / "_ref" / "libsfg_ref_gemm.so"
_ref_lib = None


def build_ref() -> Path | None:
    """Compile the reference GEMM library when the reference sources are
    present; None (nothing built) where they are not."""
    if not (REF_ROOT / "src" / "runtime.cpp").is_file():
        return None
    subprocess.run(["make", "-s", "-j8", "-C", str(HERE), "ref", f"REF={REF_ROOT}"], check=True)
    return REF_LIB_PATH


def ref_gemm_lib() -> ctypes.CDLL | None:
    """The reference GEMM library, built if it can be; None if neither a built
    library nor the sources are here."""
    global _ref_lib
    if _ref_lib is None:
        if not REF_LIB_PATH.exists() and build_ref() is None:
            return None
        _ref_lib = ctypes.CDLL(str(REF_LIB_PATH))
        _ref_lib.sfgr_decoder_gemm.restype = ctypes.c_int
        _ref_lib.sfgr_decoder_gemm.argtypes = [fp, fp, fp] + [ctypes.c_int] * 5
    return _ref_lib


def reference_gemm(a, b, family: int = 0, threads: int = 1) -> np.ndarray:
    """a @ b by the reference's execute() under the schedule its decoder gives
    the projections (family 0 Latency, 1 Throughput)."""
    ref = ref_gemm_lib()
    if ref is None:
        raise RuntimeError("reference GEMM library not built and reference sources absent")
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    c = np.empty((m, n), np.float32)
    if ref.sfgr_decoder_gemm(_f(a), _f(b), _f(c), m, n, k, family, threads) != 0:
        raise RuntimeError("reference execute() failed")
    return c


class AttnCfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("batch", "query_heads", "kv_heads", "seq_q",
                                               "seq_kv", "head_dim", "head_dim_value", "causal")] + \
               [("scale", ctypes.c_float)]


class LayerCfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("batch", "sequence", "hidden", "intermediate",
                                               "query_heads", "kv_heads", "head_dim")] + \
               [("rms_epsilon", ctypes.c_float), ("rope_theta", ctypes.c_float)] + \
               [(n, ctypes.c_int32) for n in ("causal", "moe", "experts", "top_k", "context",
                                               "int8_weights", "threads", "kv_append",
                                               "kv_pool_f32")]


class LayerData(ctypes.Structure):
    _fields_ = [(n, fp) for n in ("input", "rms1", "wq", "wk", "wv", "wo", "rms2", "wg", "wu",
                                  "wd", "router", "router_bias", "w1", "w3", "w2", "cached_k",
                                  "cached_v")] + \
               [("trace_ids", ip), ("trace_weights", fp),
                ("q8", i8p * 7), ("s8", fp * 7),
                ("e1q", i8p), ("e1s", fp), ("e3q", i8p), ("e3s", fp), ("e2q", i8p), ("e2s", fp)]


class LayerTaps(ctypes.Structure):
    _fields_ = [("normalized1", fp), ("qkv", fp), ("attn_merged", fp), ("residual1", fp),
                ("normalized2", fp), ("ids", ip), ("weights", fp), ("counts", ip),
                ("new_k", fp), ("new_v", fp)]


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        _lib.sfgo_splitmix64.restype = ctypes.c_uint64
        _lib.sfgo_splitmix64.argtypes = [ctypes.c_uint64]
        _lib.sfgo_max_abs_error.restype = ctypes.c_double
        _lib.sfgo_num_threads.restype = ctypes.c_int
    return _lib


def _f(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(fp)


def _i(a: np.ndarray):
    assert a.dtype == np.int32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ip)


def _b(a: np.ndarray):
    assert a.dtype == np.int8 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(i8p)


def _opt_f(a):
    return None if a is None else _f(a)


# ---------------------------------------------------------------- generators
def normal(seed: int, tensor: str | int, shape, std: float = 1.0, mean: float = 0.0) -> np.ndarray:
    tid = TID[tensor] if isinstance(tensor, str) else int(tensor)
    out = np.empty(shape, dtype=np.float32)
    lib().sfgo_fill_normal(ctypes.c_uint64(seed), ctypes.c_uint32(tid), ctypes.c_float(mean),
                           ctypes.c_float(std), _f(out), i64(out.size))
    return out


def page_permutation(seed: int, count: int) -> np.ndarray:
    out = np.empty(count, dtype=np.int32)
    lib().sfgo_page_permutation(ctypes.c_uint64(seed), _i(out), i64(count))
    return out


def to_bf16_bits(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().sfgo_to_bf16(_f(a), out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), i64(a.size))
    return out


def round_bf16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32).copy()
    lib().sfgo_round_bf16(_f(a), i64(a.size))
    return a


# ---------------------------------------------------------------- operators
def rms_norm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    rows, width = x.shape
    lib().sfgo_rms_norm(_f(x), _f(np.ascontiguousarray(w, np.float32)), _f(y), i64(rows),
                        i64(width), ctypes.c_float(eps))
    return y


def matmul(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    c = np.empty((m, n), np.float32)
    lib().sfgo_matmul(_f(a), _f(b), _f(c), i64(m), i64(n), i64(k))
    return c


def split_qkv_rope(qkv, batch, seq, hidden, q_heads, kv_heads, head_dim, theta):
    qkv = np.ascontiguousarray(qkv, np.float32)
    q = np.empty((batch, q_heads, seq, head_dim), np.float32)
    k = np.empty((batch, kv_heads, seq, head_dim), np.float32)
    v = np.empty_like(k)
    lib().sfgo_split_qkv_rope(_f(qkv), i64(batch), i64(seq), i64(hidden), i64(q_heads),
                              i64(kv_heads), i64(head_dim), ctypes.c_float(theta), _f(q), _f(k),
                              _f(v))
    return q, k, v


def attention(q, k, v, causal=True, scale=0.0):
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    b, hq, sq, d = q.shape
    _, hkv, skv, _ = k.shape
    cfg = AttnCfg(b, hq, hkv, sq, skv, d, v.shape[3], int(causal), scale)
    out = np.empty((b, hq, sq, v.shape[3]), np.float32)
    lib().sfgo_attention(ctypes.byref(cfg), _f(q), _f(k), _f(v), _f(out))
    return out


def paged_gather(pool, page_table, batch, kv_heads, ctx, page_tokens, head_dim):
    pool = np.ascontiguousarray(pool, np.float32)
    pt = np.ascontiguousarray(page_table, np.int32)
    flat = np.empty((batch, kv_heads, ctx, head_dim), np.float32)
    lib().sfgo_paged_gather(_f(pool), _i(pt), i64(batch), i64(kv_heads), i64(ctx),
                            i64(page_tokens), i64(head_dim), i64(pt.shape[1]), _f(flat))
    return flat


def paged_scatter(flat, page_table, num_pages, page_tokens):
    flat = np.ascontiguousarray(flat, np.float32)
    pt = np.ascontiguousarray(page_table, np.int32)
    batch, kv_heads, ctx, head_dim = flat.shape
    pool = np.zeros((num_pages, kv_heads, page_tokens, head_dim), np.float32)
    lib().sfgo_paged_scatter(_f(flat), _i(pt), i64(batch), i64(kv_heads), i64(ctx),
                             i64(page_tokens), i64(head_dim), i64(pt.shape[1]), _f(pool))
    return pool


def route_topk(x, router, bias, top_k):
    x = np.ascontiguousarray(x, np.float32)
    router = np.ascontiguousarray(router, np.float32)
    t, h = x.shape
    e = router.shape[1]
    ids = np.empty((t, top_k), np.int32)
    w = np.empty((t, top_k), np.float32)
    counts = np.empty(e, np.int32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().sfgo_route_topk(_f(x), _f(router), _opt_f(b), i64(t), i64(h), i64(e), i64(top_k),
                          _i(ids), _f(w), _i(counts))
    return ids, w, counts


def dispatch(ids, weights, experts):
    ids = np.ascontiguousarray(ids, np.int32)
    weights = np.ascontiguousarray(weights, np.float32)
    t, k = ids.shape
    counts = np.bincount(ids.reshape(-1), minlength=experts).astype(np.int32)
    offsets = np.empty(experts + 1, np.int32)
    token_ids = np.empty(t * k, np.int32)
    slots = np.empty(t * k, np.int32)
    rw = np.empty(t * k, np.float32)
    lib().sfgo_dispatch(_i(ids), _f(weights), _i(counts), i64(t), i64(experts), i64(k),
                        _i(offsets), _i(token_ids), _i(slots), _f(rw))
    return counts, offsets, token_ids, slots, rw


def moe_reference(x, w1, w3, w2, ids, weights):
    x = np.ascontiguousarray(x, np.float32)
    t, h = x.shape
    inter = w1.shape[2]
    out = np.empty((t, h), np.float32)
    lib().sfgo_moe_reference(_f(x), _f(np.ascontiguousarray(w1, np.float32)),
                             _f(np.ascontiguousarray(w3, np.float32)),
                             _f(np.ascontiguousarray(w2, np.float32)), i64(t), i64(h), i64(inter),
                             i64(ids.shape[1]), _i(np.ascontiguousarray(ids, np.int32)),
                             _f(np.ascontiguousarray(weights, np.float32)), _f(out))
    return out


def quantize_kn(w_kn):
    """transpose_decoder_weight + quantize_matmul_weights: [K][N] -> int8 [N][K], scales [N]."""
    w = np.ascontiguousarray(w_kn, np.float32)
    k, n = w.shape
    wt = np.empty((n, k), np.float32)
    lib().sfgo_transpose(_f(w), i64(k), i64(n), _f(wt))
    q = np.empty((n, k), np.int8)
    s = np.empty(n, np.float32)
    lib().sfgo_quantize_nk(_f(wt), i64(n), i64(k), _b(q), _f(s))
    return q, s


def quantized_matmul(x, q_nk, scales):
    x = np.ascontiguousarray(x, np.float32)
    m, k = x.shape
    n = q_nk.shape[0]
    out = np.empty((m, n), np.float32)
    lib().sfgo_quantized_matmul(_f(x), _b(np.ascontiguousarray(q_nk)), _f(scales), i64(m), i64(n),
                                i64(k), _f(out))
    return out


def quantized_moe(x, e1, e3, e2, ids, weights):
    """execute_quantized_moe_once restated (sfgo_quantized_moe): e1 / e3 / e2 are
    per-expert (q [N][K] int8, scales [N]) pairs from quantize_kn of W1[e],
    W3[e] ([H][I]) and W2[e] ([I][H])."""
    x = np.ascontiguousarray(x, np.float32)
    t, h = x.shape
    ids = np.ascontiguousarray(ids, np.int32)
    weights = np.ascontiguousarray(weights, np.float32)
    top_k = ids.shape[1]
    inter = e1[0][0].shape[0]
    stk = [np.ascontiguousarray(np.stack([p[j] for p in e])) for e in (e1, e3, e2) for j in (0, 1)]
    out = np.empty((t, h), np.float32)
    lib().sfgo_quantized_moe(_f(x), _b(stk[0]), _f(stk[1]), _b(stk[2]), _f(stk[3]), _b(stk[4]),
                             _f(stk[5]), i64(t), i64(h), i64(inter), i64(top_k), _i(ids),
                             _f(weights), _f(out))
    return out


def max_abs_error(a, b):
    a = np.ascontiguousarray(a, np.float32).reshape(-1)
    b = np.ascontiguousarray(b, np.float32).reshape(-1)
    assert a.size == b.size
    return float(lib().sfgo_max_abs_error(_f(a), _f(b), i64(a.size)))


def rel_error(got, ref):
    """max|got - ref| / max(max|ref|, 1e-6) -- the build's relative criterion."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref)) / max(float(np.max(np.abs(ref))), 1e-6))


from .data import make_layer_data, quantize_layer, decoder_layer, decoder_layer_rows, prepared_layer  # noqa: E402,F401
