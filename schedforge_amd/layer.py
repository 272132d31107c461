"""Decoder-layer plan and execution over the C ABI (libsfg_hip.so).

Python mirror of the reference's operator boundary (decoder_compiler.h:205-223):
  compile_decoder(config, data)          ~ DecoderCompiler::compile
  execute_decoder_layer(plan, ...)       ~ execute_decoder_layer (warmup, reps, median)
Device memory and streams come from PyTorch (plumbing only); every kernel is
one of libsfg_hip.so's.  Weights are packed once at compile time into the
device layouts (constant specialisation, decoder_compiler.cpp:535-552):
  w_qkv [H + 2 kvD][H], w_o [H][H], w_gate_up [2I][H], w_down [H][I],
  w13 [E][2I][H] (W1^T rows then W3^T rows), w2 [E][H][I];
  bf16 (round to nearest even) or int8 + per-channel scales.
Decode steps read K/V from paged pools in the activation dtype (bf16, fp32 on
the fp32 path) -- K [page][Hkv][page_tokens][D], V [page][Hkv][D][page_tokens]
-- addressed by a per-sequence page table.
"""
from __future__ import annotations

import ctypes
import statistics
import time
from dataclasses import dataclass, field
from typing import Any, Callable, Optional

import numpy as np
import torch

from . import _abi
from ._abi import BF16, F32, I8, check
from .configs import DecoderConfig


@dataclass
class DecoderData:
    """Mirror of schedforge::DecoderData (decoder_compiler.h:34-49): fp32 tensors
    in the reference's layouts ([K][N] weights).  Fields may be numpy arrays,
    torch tensors (host or device) or, for expert weights, callables e -> [K][N]."""
    input: Any = None
    rms1_weight: Any = None
    query_weight: Any = None
    key_weight: Any = None
    value_weight: Any = None
    output_weight: Any = None
    rms2_weight: Any = None
    gate_weight: Any = None
    up_weight: Any = None
    down_weight: Any = None
    router_weight: Any = None
    router_bias: Any = None           # build extension
    w1: Any = None
    w3: Any = None
    w2: Any = None
    cached_key: Any = None            # [B, Hkv, ctx, D]
    cached_value: Any = None
    routing_trace: Optional[tuple] = None   # (ids [T,k] int32, weights [T,k] f32)
    page_table: Any = None            # build extension: [B, pages_per_seq] int32


@dataclass
class DecoderBenchmarkResult:
    """Mirror of schedforge::DecoderBenchmarkResult (decoder_compiler.h:119-130)."""
    milliseconds: float = 0.0
    attention_milliseconds: float = 0.0
    projection_milliseconds: float = 0.0
    norm_rope_milliseconds: float = 0.0
    ffn_milliseconds: float = 0.0
    residual_milliseconds: float = 0.0
    dispatch_overhead_milliseconds: float = 0.0
    tokens_per_second: float = 0.0
    max_error: float = float("nan")   # NaN unless expected outputs were given
    output: Any = None
    stages: dict = field(default_factory=dict)


def _dev(x, device, dtype=torch.float32) -> torch.Tensor:
    if isinstance(x, torch.Tensor):
        return x.to(device=device, dtype=dtype).contiguous()
    return torch.from_numpy(np.ascontiguousarray(np.asarray(x))).to(device=device, dtype=dtype)


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream_handle(stream: Optional[torch.cuda.Stream] = None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _expert(w, e):
    if callable(w):
        return w(e)
    return w[e]


class DecoderExecutablePlan:
    """Device-resident plan: packed weights, page tables, RoPE table, workspace."""

    def __init__(self, config: DecoderConfig, device):
        self.config = config
        self.device = torch.device(device)
        self.t: dict[str, torch.Tensor] = {}
        self.desc = _abi.LayerDesc()
        self.weights = _abi.LayerWeights()
        self.workspace: Optional[torch.Tensor] = None
        self.trace: Optional[tuple] = None
        self.lengths: Optional[np.ndarray] = None  # append plans: host copy of the cached lengths
        self.lib = _abi.load()

    # ---- helpers -------------------------------------------------------
    def _pack(self, name_rows: list, k: int, wdt: int, stream: int, key: str,
              layout: int = _abi.LAYOUT_NK) -> None:
        """Pack a list of (fp32 [k][n] weight) blocks into one [sum n][k] matrix."""
        n_total = sum(int(w.shape[1]) for w in name_rows)
        if wdt == I8:
            dst = torch.empty((n_total, k), dtype=torch.int8, device=self.device)
            scales = torch.empty((n_total,), dtype=torch.float32, device=self.device)
        else:
            dst = torch.empty((n_total, k), dtype=torch.float32 if wdt == F32 else torch.int16,
                              device=self.device)
            scales = None
        row = 0
        esz = dst.element_size()
        for w in name_rows:
            wd = _dev(w, self.device)
            n = int(wd.shape[1])
            if wdt == I8:
                check(self.lib.sfg_hip_quantize_weight_v1(wd.data_ptr(), k, n,
                                                          dst.data_ptr() + row * k * esz,
                                                          scales.data_ptr() + row * 4, layout,
                                                          stream))
            else:
                check(self.lib.sfg_hip_pack_weight_v1(wd.data_ptr(), k, n, n,
                                                      dst.data_ptr() + row * k * esz, wdt, layout,
                                                      stream))
            torch.cuda.current_stream(self.device).synchronize()
            del wd
            row += n
        self.t[key] = dst
        if scales is not None:
            self.t["s_" + key] = scales

    def _pack_experts(self, ws: list, k_dim: int, rows_per_expert: int, wdt: int, stream: int,
                      key: str, experts: int, layout: int = _abi.LAYOUT_NK) -> None:
        if wdt == I8:
            dst = torch.empty((experts, rows_per_expert, k_dim), dtype=torch.int8, device=self.device)
            scales = torch.empty((experts, rows_per_expert), dtype=torch.float32, device=self.device)
        else:
            dst = torch.empty((experts, rows_per_expert, k_dim),
                              dtype=torch.float32 if wdt == F32 else torch.int16, device=self.device)
            scales = None
        esz = dst.element_size()
        for e in range(experts):
            row = 0
            for w in ws:
                wd = _dev(_expert(w, e), self.device)
                n = int(wd.shape[1])
                base = (e * rows_per_expert + row)
                if wdt == I8:
                    check(self.lib.sfg_hip_quantize_weight_v1(
                        wd.data_ptr(), k_dim, n, dst.data_ptr() + base * k_dim * esz,
                        scales.data_ptr() + base * 4, layout, stream))
                else:
                    check(self.lib.sfg_hip_pack_weight_v1(
                        wd.data_ptr(), k_dim, n, n, dst.data_ptr() + base * k_dim * esz, wdt,
                        layout, stream))
                torch.cuda.current_stream(self.device).synchronize()
                del wd
                row += n
        self.t[key] = dst
        if scales is not None:
            self.t["s_" + key] = scales


def compile_decoder(config: DecoderConfig, data: DecoderData, device="cuda",
                    kv_splits: int = 0, page_permutation: Optional[np.ndarray] = None,
                    gemm_tile: int = 0, attn_waves: int = 0) -> DecoderExecutablePlan:
    """DecoderCompiler::compile for the gfx950 target (decoder_compiler.cpp:518-620):
    validate, pack constants on the device, build the paged KV pool, size the
    workspace.  kv_splits, gemm_tile (sfg_gemm_tile) and attn_waves (4 or 8)
    are the plan policy (DecoderPlanPolicy, decoder_compiler.h:55-65); 0 picks
    per shape, and every choice computes the same layer."""
    cfg = config
    cfg.validate()
    plan = DecoderExecutablePlan(cfg, device)
    lib = plan.lib
    stream = _stream_handle()
    H, I, D = cfg.hidden, cfg.intermediate, cfg.head_dim
    act = F32 if cfg.dtype == "f32" else BF16
    wdt = {"f32": F32, "bf16": BF16, "w8": I8}[cfg.dtype]
    t = plan.t
    t["rms1"] = _dev(data.rms1_weight, plan.device)
    t["rms2"] = _dev(data.rms2_weight, plan.device)
    # One weight layout for the whole plan: fragment-tiled when every product
    # runs on the decode (skinny) kernel -- every depth takes it and every
    # width is a multiple of 64, which its 16-, 32- and 64-column tiles
    # divide -- [N][K] otherwise.
    layout = _abi.LAYOUT_NK
    if wdt != F32:
        ks = [H, I]
        tiled = all(lib.sfg_hip_preferred_weight_layout_v1(cfg.rows, k, 0) == _abi.LAYOUT_TILED
                    for k in ks) and all(n % 64 == 0 for n in (cfg.qkv_width, H, I))
        if cfg.moe:
            tiled = tiled and all(lib.sfg_hip_preferred_weight_layout_v1(
                cfg.rows * cfg.top_k, k, 1) == _abi.LAYOUT_TILED for k in ks)
        layout = _abi.LAYOUT_TILED if tiled else _abi.LAYOUT_NK
    plan.layout = layout
    plan._pack([data.query_weight, data.key_weight, data.value_weight], H, wdt, stream, "w_qkv",
               layout)
    plan._pack([data.output_weight], H, wdt, stream, "w_o", layout)
    if cfg.moe:
        t["router"] = _dev(data.router_weight, plan.device)
        if data.router_bias is not None:
            t["router_bias"] = _dev(data.router_bias, plan.device)
        plan._pack_experts([data.w1, data.w3], H, 2 * I, wdt, stream, "w13", cfg.experts, layout)
        plan._pack_experts([data.w2], I, H, wdt, stream, "w2", cfg.experts, layout)
    else:
        plan._pack([data.gate_weight, data.up_weight], H, wdt, stream, "w_gate_up", layout)
        plan._pack([data.down_weight], I, wdt, stream, "w_down", layout)

    # RoPE table [positions][D/2][2], host-computed with the reference's
    # expressions: the step's positions, or for append plans every position the
    # cache can reach (tokens rotate at their true positions there).
    positions = max(cfg.sequence, cfg.capacity) if cfg.kv_append else cfg.sequence
    table = np.empty((positions, D // 2, 2), dtype=np.float32)
    check(lib.sfg_hip_rope_table_host_v1(table.ctypes.data, positions, D,
                                         ctypes.c_float(cfg.rope_theta)))
    t["rope"] = torch.from_numpy(table).to(plan.device)

    pages_per_seq = num_pages = 0
    if cfg.decode:
        pt = cfg.page_tokens
        pages_per_seq = (cfg.capacity + pt - 1) // pt
        num_pages = cfg.batch * pages_per_seq
        if data.page_table is not None:
            table_pages = np.asarray(data.page_table, dtype=np.int32).reshape(cfg.batch, pages_per_seq)
        else:
            perm = (np.arange(num_pages, dtype=np.int32) if page_permutation is None
                    else np.asarray(page_permutation, dtype=np.int32).reshape(-1))
            if perm.size != num_pages:
                raise ValueError(f"page_permutation holds {perm.size} page ids; the plan's tables "
                                 f"need batch x pages_per_seq = {num_pages}")
            table_pages = perm.reshape(cfg.batch, pages_per_seq)
        if table_pages.min() < 0 or table_pages.max() >= num_pages:
            raise ValueError("invalid physical KV page")
        # one physical page per logical page: a page named twice would hold two
        # sequences' keys at once
        if np.unique(table_pages).size != table_pages.size:
            raise ValueError("a physical KV page is assigned twice")
        t["page_table"] = torch.from_numpy(np.ascontiguousarray(table_pages)).to(plan.device)
        for name, src in (("k_pool", data.cached_key), ("v_pool", data.cached_value)):
            flat = _dev(src, plan.device).reshape(cfg.batch, cfg.kv_heads, cfg.context_sequence, D)
            padded = torch.zeros((cfg.batch, cfg.kv_heads, pages_per_seq * pt, D),
                                 dtype=torch.float32, device=plan.device)
            padded[:, :, :cfg.context_sequence] = flat
            del flat
            blocks = padded.reshape(cfg.batch, cfg.kv_heads, pages_per_seq, pt, D) \
                           .permute(0, 2, 1, 3, 4)
            if name == "v_pool":  # V is token-minor inside a page: [page][Hkv][D][16]
                blocks = blocks.transpose(-1, -2)
            # contiguous [page][Hkv][...] memory, whatever strides the view
            # has (a batch of one reshapes the permuted view without a copy)
            blocks = blocks.reshape(num_pages, cfg.kv_heads, *blocks.shape[-2:]).contiguous()
            del padded
            pool32 = torch.empty(blocks.shape, dtype=torch.float32, device=plan.device)
            idx = t["page_table"].reshape(-1).long()
            pool32[idx] = blocks
            del blocks
            if cfg.dtype == "f32":  # the fp32 path keeps fp32 pools
                t[name] = pool32
                continue
            pool = torch.empty(pool32.shape, dtype=torch.int16, device=plan.device)
            check(lib.sfg_hip_to_bf16_v1(pool32.data_ptr(), pool.data_ptr(), pool32.numel(), stream))
            torch.cuda.current_stream(plan.device).synchronize()
            del pool32
            t[name] = pool

    if data.routing_trace is not None:
        ids, wts = data.routing_trace
        t["trace_ids"] = _dev(ids, plan.device, torch.int32)
        t["trace_weights"] = _dev(wts, plan.device)

    d = plan.desc
    d.abi = _abi.ABI_VERSION
    d.batch, d.sequence, d.hidden, d.intermediate = cfg.batch, cfg.sequence, H, I
    d.query_heads, d.kv_heads, d.head_dim = cfg.query_heads, cfg.kv_heads, D
    d.rms_epsilon, d.rope_theta = cfg.rms_epsilon, cfg.rope_theta
    d.causal = int(cfg.causal)
    d.ffn = 1 if cfg.moe else 0
    d.experts, d.top_k = cfg.experts, cfg.top_k
    d.context = cfg.context_sequence
    d.page_tokens, d.pages_per_seq, d.num_pages = cfg.page_tokens, pages_per_seq, num_pages
    d.act_dtype, d.weight_dtype = act, wdt
    d.kv_splits = kv_splits
    d.gemm_tile = gemm_tile
    d.attn_waves = attn_waves
    d.use_routing_trace = int(data.routing_trace is not None)
    d.weight_layout = layout
    d.kv_append = int(cfg.kv_append)
    if cfg.kv_append:
        # per-sequence cached lengths on the device, advanced by every step
        t["seq_lens"] = torch.full((cfg.batch,), cfg.context_sequence, dtype=torch.int32,
                                   device=plan.device)
        plan.lengths = np.full(cfg.batch, cfg.context_sequence, dtype=np.int64)

    w = plan.weights
    w.rms1, w.rms2 = _ptr(t["rms1"]), _ptr(t["rms2"])
    w.w_qkv, w.s_qkv = _ptr(t["w_qkv"]), _ptr(t.get("s_w_qkv"))
    w.w_o, w.s_o = _ptr(t["w_o"]), _ptr(t.get("s_w_o"))
    if cfg.moe:
        w.router, w.router_bias = _ptr(t["router"]), _ptr(t.get("router_bias"))
        w.w13, w.s13 = _ptr(t["w13"]), _ptr(t.get("s_w13"))
        w.w2, w.s2 = _ptr(t["w2"]), _ptr(t.get("s_w2"))
    else:
        w.w_gate_up, w.s_gate_up = _ptr(t["w_gate_up"]), _ptr(t.get("s_w_gate_up"))
        w.w_down, w.s_down = _ptr(t["w_down"]), _ptr(t.get("s_w_down"))
    if cfg.decode:
        w.k_pool, w.v_pool, w.page_table = _ptr(t["k_pool"]), _ptr(t["v_pool"]), _ptr(t["page_table"])
    w.rope_table = _ptr(t["rope"])

    ws = lib.sfg_hip_decoder_layer_workspace_v1(ctypes.byref(d))
    if ws == 0:
        check(_abi.ERR_INVALID_CONFIG)
    # zero-filled once so that a stage tap read before the first call is
    # defined; every call writes each buffer before reading it
    plan.workspace = torch.zeros(ws, dtype=torch.uint8, device=plan.device)
    torch.cuda.synchronize(plan.device)
    return plan


class StageEvents:
    """SFG_NUM_MARKS HIP events created through the ABI, for per-stage timing."""

    def __init__(self, lib, marks=None):
        """marks: iterable of mark ids to record (None: all).  Unrecorded marks
        stay NULL and the layer skips them."""
        self.lib = lib
        self.arr = (ctypes.c_void_p * _abi.NUM_MARKS)()
        check(lib.sfg_hip_events_create_v1(_abi.NUM_MARKS, self.arr))
        if marks is not None:
            keep = set(marks)
            for i in range(_abi.NUM_MARKS):
                if i not in keep:
                    lib.sfg_hip_events_destroy_v1(1, ctypes.byref(ctypes.c_void_p(self.arr[i])))
                    self.arr[i] = None

    def elapsed(self, a: int, b: int) -> float:
        ms = ctypes.c_float()
        check(self.lib.sfg_hip_event_elapsed_v1(self.arr[a], self.arr[b], ctypes.byref(ms)))
        return float(ms.value)

    def close(self):
        if self.arr is not None:
            self.lib.sfg_hip_events_destroy_v1(_abi.NUM_MARKS, self.arr)
            self.arr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def run_layer(plan: DecoderExecutablePlan, x: torch.Tensor, out: torch.Tensor,
              events: Optional[StageEvents] = None, stream: Optional[torch.cuda.Stream] = None) -> None:
    """One enqueue of the whole layer (execute_once, decoder_compiler.cpp:218-304)."""
    io = _abi.LayerIO()
    io.x, io.out = x.data_ptr(), out.data_ptr()
    if "trace_ids" in plan.t:
        io.trace_ids, io.trace_weights = plan.t["trace_ids"].data_ptr(), plan.t["trace_weights"].data_ptr()
    io.stage_events = events.arr if events is not None else None
    if plan.config.kv_append:
        # append_paged_kv's guard (next_milestones.cpp:488-489), kept on the host
        if int(plan.lengths.max()) + plan.config.sequence > plan.config.capacity:
            raise ValueError("paged KV capacity exceeded")
        io.seq_lens = plan.t["seq_lens"].data_ptr()
        plan.lengths += plan.config.sequence
    check(plan.lib.sfg_hip_decoder_layer_v1(ctypes.byref(plan.desc), ctypes.byref(plan.weights),
                                            ctypes.byref(io), plan.workspace.data_ptr(),
                                            plan.workspace.numel(), _stream_handle(stream)))


def stage_times(ev: StageEvents) -> dict:
    m = _abi
    return {
        "norm_rope": ev.elapsed(m.MARK_START, m.MARK_NORM1) + ev.elapsed(m.MARK_QKV, m.MARK_ROPE)
        + ev.elapsed(m.MARK_OPROJ, m.MARK_NORM2),
        "projection": ev.elapsed(m.MARK_NORM1, m.MARK_QKV) + ev.elapsed(m.MARK_ATTN, m.MARK_OPROJ),
        "attention": ev.elapsed(m.MARK_ROPE, m.MARK_ATTN),
        "attention_main": ev.elapsed(m.MARK_ROPE, m.MARK_ATTN_MAIN),
        "route": ev.elapsed(m.MARK_NORM2, m.MARK_ROUTE),
        "ffn_up": ev.elapsed(m.MARK_ROUTE, m.MARK_FFN_UP),
        "ffn_down": ev.elapsed(m.MARK_FFN_UP, m.MARK_FFN_DOWN),
        "total": ev.elapsed(m.MARK_START, m.MARK_END),
    }


def layer_taps(plan: DecoderExecutablePlan) -> dict:
    """The stage intermediates the last layer call left in the plan's workspace
    (sfg_hip_decoder_layer_tap_v1), as host arrays: "attn" merged attention
    [rows][H], "residual1" r1 [rows][H], "normalized2" [rows][H] (fp32 views of
    bf16 values when the activations are bf16); for a MoE layer "route_input"
    (the router's fp32 rows) and, routed on the device, "ids" / "weights"
    [rows][k]."""
    cfg = plan.config
    torch.cuda.synchronize(plan.device)
    shapes = {_abi.TAP_ATTN: ("attn", cfg.hidden), _abi.TAP_RESIDUAL1: ("residual1", cfg.hidden),
              _abi.TAP_NORM2: ("normalized2", cfg.hidden)}
    if cfg.moe:
        shapes[_abi.TAP_ROUTE_INPUT] = ("route_input", cfg.hidden)
    if cfg.moe and not plan.desc.use_routing_trace:
        shapes[_abi.TAP_ROUTE_IDS] = ("ids", cfg.top_k)
        shapes[_abi.TAP_ROUTE_WEIGHTS] = ("weights", cfg.top_k)
    out = {}
    for tap, (name, width) in shapes.items():
        off, nbytes, dt = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_int()
        check(plan.lib.sfg_hip_decoder_layer_tap_v1(ctypes.byref(plan.desc), tap, ctypes.byref(off),
                                                    ctypes.byref(nbytes), ctypes.byref(dt)))
        raw = plan.workspace[off.value:off.value + nbytes.value].cpu().numpy()
        if dt.value == BF16:
            a = (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
        elif dt.value == _abi.I32:
            a = raw.view(np.int32)
        else:
            a = raw.view(np.float32)
        out[name] = a.reshape(cfg.rows, width)
    return out


def max_abs_error(output: np.ndarray, expected: np.ndarray) -> float:
    """max_abs_error (runtime.cpp:628-635): the largest |float(a - b)| taken in
    double; infinity on a size mismatch.  As there, std::max keeps the running
    value when a difference is NaN, so NaNs are not reported here."""
    a = np.asarray(output, np.float32).reshape(-1)
    b = np.asarray(expected, np.float32).reshape(-1)
    if a.size != b.size:
        return float("inf")
    d = np.abs((a - b).astype(np.float64))
    d = d[~np.isnan(d)]
    return float(d.max(initial=0.0))


def execute_decoder_layer(plan: DecoderExecutablePlan, x, warmup: int = 1,
                          repetitions: int = 5, expected=None) -> DecoderBenchmarkResult:
    """execute_decoder_layer (decoder_compiler.cpp:675-692): warmup, timed
    repetitions, median by time, tokens/s = rows * 1000 / ms.  The reference
    sets max_error against its scalar reference_decoder_layer (690); here the
    caller passes the expected [rows][H] output (from any checker) and
    max_error is max |output - expected|, or NaN when none is given."""
    cfg = plan.config
    xd = _dev(x, plan.device)
    out = torch.empty((cfg.rows, cfg.hidden), dtype=torch.float32, device=plan.device)
    for _ in range(max(0, warmup)):
        run_layer(plan, xd, out)
    torch.cuda.synchronize(plan.device)
    ev = StageEvents(plan.lib)
    results = []
    for _ in range(max(1, repetitions)):
        run_layer(plan, xd, out, events=ev)
        torch.cuda.synchronize(plan.device)
        st = stage_times(ev)
        results.append(st)
    ev.close()
    results.sort(key=lambda r: r["total"])
    med = results[len(results) // 2]
    r = DecoderBenchmarkResult()
    r.milliseconds = med["total"]
    r.attention_milliseconds = med["attention"]
    r.projection_milliseconds = med["projection"]
    r.norm_rope_milliseconds = med["norm_rope"]
    r.ffn_milliseconds = med["route"] + med["ffn_up"] + med["ffn_down"]
    accounted = (r.attention_milliseconds + r.projection_milliseconds + r.norm_rope_milliseconds
                 + r.ffn_milliseconds)
    r.dispatch_overhead_milliseconds = max(0.0, r.milliseconds - accounted)
    r.tokens_per_second = cfg.rows * 1000.0 / r.milliseconds if r.milliseconds > 0 else 0.0
    r.output = out.cpu().numpy()
    r.stages = med
    if expected is not None:
        r.max_error = max_abs_error(r.output, expected)
    return r
