"""Decoder-layer benchmark on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c4] [--decode-config c5]

A step is one execution of the whole decoder layer (execute_once,
decoder_compiler.cpp:218-304) on one batch of synthetic input, inputs resident in
HBM.  The metric is the reference's: equivalent tokens/s = rows * 1000 / ms
(decoder_compiler.cpp:301-302, 688-689), rows = batch * sequence.

BASELINE.json's metric names no configuration, so the headline is the largest
single-GPU configuration: config 4 (Llama-3-8B-shaped prefill, S 8192, bf16),
MFMA-bound.  The same line nests, under "decode", config 5 (Mixtral-shaped int8
decode over a paged 8192-token cache), HBM-bound, with its own value and
roofline; --decode-config none leaves it out, --config picks another headline.

Each measured block carries:
  roofline      the dominant kernel's achieved fraction of its MI355X peak:
                algorithmic FLOPs (prefill: the FFN up-projection GEMM) or bytes
                (decode: the paged Split-KV attention kernel) per launch over
                the launch's average duration, from HIP events recorded around
                it on the layer's stream in every --mark-every'th timed step (an
                event record drains the queue, so only some steps are marked);
                "traffic" is the kernel's HBM bytes per launch from the
                rocprofv3 FETCH_SIZE / WRITE_SIZE passes in
                profiles/pmc_traffic.txt, scaled by the same counters' reading
                for a 1 GiB copy (--copy-calibration);
  cpu_baseline  the CPU restatement (oracle/sfg_oracle.c, a C restatement of the
                reference path) on this host's cores: whole layer steps of the
                same workload, the median of as many as --cpu-seconds allows
                (at least one; a C4 step is a few tens of seconds);
  cold          decode configurations whose layer fits twice in the 256 MB
                Infinity Cache (C2): the same steps rotating over independent
                copies of the weights and KV pool, together over twice its
                size, so no step is served from the previous step's cache.
Synthetic data: activations N(0,1), weights N(0,0.02), cached K/V N(0,1), drawn
on the device; norm gains 1; random page table.
"""
from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

TRAFFIC_FILE = ROOT / "profiles" / "pmc_traffic.txt"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--config", default="c4", choices=["c1", "c2", "c3", "c4", "c5"])
    p.add_argument("--decode-config", default="c5", choices=["c2", "c5", "none"],
                   help="decode configuration nested under 'decode' when the headline is a prefill")
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="CPU-baseline budget: whole layer steps are repeated until it is spent (at least one)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--mark-every", type=int, default=5,
                   help="bracket the roofline kernel with HIP events in every N-th timed step")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                   help="before warmup, stream MIB MiB through one elementwise kernel "
                        "(reads MIB, writes MIB): the known-size reference for the "
                        "FETCH_SIZE / WRITE_SIZE counter runs")
    return p.parse_args()


# ---------------------------------------------------------------- data
def make_device_data(cfg, seed, device):
    """Synthetic DecoderData drawn on the device (reference layouts, fp32)."""
    import torch
    from schedforge_amd.layer import DecoderData
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    H, I, D = cfg.hidden, cfg.intermediate, cfg.head_dim
    kvd = cfg.kv_heads * D

    def n(*shape, std=1.0):
        return torch.randn(*shape, generator=g, device=device, dtype=torch.float32) * std

    d = DecoderData()
    d.input = n(cfg.rows, H)
    d.rms1_weight = torch.ones(H, device=device)
    d.rms2_weight = torch.ones(H, device=device)
    d.query_weight = n(H, H, std=0.02)
    d.key_weight = n(H, kvd, std=0.02)
    d.value_weight = n(H, kvd, std=0.02)
    d.output_weight = n(H, H, std=0.02)
    if cfg.moe:
        d.router_weight = n(H, cfg.experts, std=0.02)
        if cfg.router_bias_std > 0:
            d.router_bias = n(cfg.experts, std=cfg.router_bias_std)
        # experts drawn one matrix at a time while packing (keeps HBM use low)
        d.w1 = lambda e: n(H, I, std=0.02)
        d.w3 = lambda e: n(H, I, std=0.02)
        d.w2 = lambda e: n(I, H, std=0.02)
    else:
        d.gate_weight = n(H, I, std=0.02)
        d.up_weight = n(H, I, std=0.02)
        d.down_weight = n(I, H, std=0.02)
    perm = None
    if cfg.decode:
        d.cached_key = n(cfg.batch, cfg.kv_heads, cfg.context_sequence, D)
        d.cached_value = n(cfg.batch, cfg.kv_heads, cfg.context_sequence, D)
        pps = (cfg.context_sequence + cfg.page_tokens - 1) // cfg.page_tokens
        perm = torch.randperm(cfg.batch * pps, generator=torch.Generator().manual_seed(seed)).numpy()
    return d, perm


def timing_data(cfg, seed):
    """Host data in the oracle's layouts for timing only, and for int8 configs
    the quantized weights: each tensor is a random 1 Mi-element block repeated
    to its shape (the oracle's cost does not depend on the values, and drawing
    and quantizing 10^9 values would dominate the sample)."""
    import numpy as np
    from types import SimpleNamespace
    rng = np.random.default_rng(seed)
    block = rng.standard_normal(1 << 20, dtype=np.float32)
    qblock = rng.integers(-127, 128, size=1 << 20, dtype=np.int8)

    def fill(shape, src):
        out = np.empty(int(np.prod(shape)), src.dtype)
        whole = out.size // src.size * src.size
        out[:whole].reshape(-1, src.size)[:] = src
        out[whole:] = src[:out.size - whole]
        return out.reshape(shape)

    def t(shape, std=1.0):
        return fill(shape, block * np.float32(std))

    def q8(n, k):  # int8 [N][K] and per-channel scales, as quantize_kn returns
        return fill((n, k), qblock), np.full(n, 0.02 / 127 * 4, np.float32)

    H, I, D, E = cfg.hidden, cfg.intermediate, cfg.head_dim, cfg.experts
    kvd = cfg.kv_heads * D
    w8 = cfg.dtype == "w8"
    d = SimpleNamespace(routing_trace=None, router_bias=None, gate_weight=None, up_weight=None,
                        down_weight=None, router_weight=None, w1=None, w3=None, w2=None,
                        cached_key=None, cached_value=None, query_weight=None, key_weight=None,
                        value_weight=None, output_weight=None)
    d.input = t((cfg.rows, H))
    d.rms1_weight = d.rms2_weight = np.ones(H, np.float32)
    quant = None
    if w8:
        quant = SimpleNamespace(dense=[q8(H, H), q8(kvd, H), q8(kvd, H), q8(H, H)])
        if cfg.moe:
            quant.e1 = [q8(I, H) for _ in range(E)]
            quant.e3 = [q8(I, H) for _ in range(E)]
            quant.e2 = [q8(H, I) for _ in range(E)]
        else:
            quant.dense += [q8(I, H), q8(I, H), q8(H, I)]
    else:
        d.query_weight, d.output_weight = t((H, H), 0.02), t((H, H), 0.02)
        d.key_weight, d.value_weight = t((H, kvd), 0.02), t((H, kvd), 0.02)
    if cfg.moe:
        d.router_weight = t((H, E), 0.02)
        if not w8:
            d.w1, d.w3, d.w2 = t((E, H, I), 0.02), t((E, H, I), 0.02), t((E, I, H), 0.02)
    elif not w8:
        d.gate_weight, d.up_weight, d.down_weight = t((H, I), 0.02), t((H, I), 0.02), t((I, H), 0.02)
    if cfg.decode:
        d.cached_key = t((cfg.batch, cfg.kv_heads, cfg.context_sequence, D))
        d.cached_value = t((cfg.batch, cfg.kv_heads, cfg.context_sequence, D))
    return d, quant


# ---------------------------------------------------------------- roofline inputs
def decode_attention_bytes(cfg):
    """Algorithmic HBM bytes of one paged decode-attention launch: K + V pages
    (bf16), Q (fp32), the merged output (bf16) and the page table."""
    pps = (cfg.context_sequence + cfg.page_tokens - 1) // cfg.page_tokens
    kv = 2 * cfg.batch * cfg.kv_heads * cfg.context_sequence * cfg.head_dim * 2
    q = cfg.batch * cfg.query_heads * cfg.head_dim * 4
    o = cfg.batch * cfg.query_heads * cfg.head_dim * 2
    pt = cfg.batch * pps * 4
    return kv + q + o + pt


def measured_traffic(config: str):
    """HBM bytes per launch of the config's roofline kernel from
    profiles/pmc_traffic.txt: FETCH_SIZE and WRITE_SIZE (KiB per dispatch),
    each scaled by copy_mib * 1024 / (the counter's KiB for the calibration
    copy, which reads copy_mib MiB and writes copy_mib MiB).  None when the file
    holds no entry for the config."""
    if not TRAFFIC_FILE.exists():
        return None
    cal, rows = None, {}
    for line in TRAFFIC_FILE.read_text().splitlines():
        parts = line.split()
        if not parts or line.startswith("#"):
            continue
        kv = dict(p.split("=", 1) for p in parts[1:] if "=" in p)
        if parts[0] == "calibration":
            cal = kv
        else:
            rows[parts[0]] = kv
    if cal is None or config not in rows:
        return None
    moved_kib = float(cal["copy_mib"]) * 1024.0
    fs, ws = moved_kib / float(cal["fetch_kib"]), moved_kib / float(cal["write_kib"])
    r = rows[config]
    return {"bytes": round((float(r["fetch_kib"]) * fs + float(r["write_kib"]) * ws) * 1024),
            "kernel": r.get("kernel", "")}


def stage_tflops(cfg, work, avg):
    """Algorithmic TFLOP/s of the MFMA stages (projection = QKV + O; FFN up and
    down, which for MoE are both inside ffn_up; attention)."""
    out = {"projection": work["proj_flops"] / (avg("projection") * 1e-3) / 1e12,
           "attention": work["attn_flops"] / (avg("attention_main") * 1e-3) / 1e12}
    if cfg.moe:
        out["experts"] = 6 * cfg.rows * cfg.top_k * cfg.hidden * cfg.intermediate / (avg("ffn_up") * 1e-3) / 1e12
    else:
        out["ffn_up"] = 4 * cfg.rows * cfg.hidden * cfg.intermediate / (avg("ffn_up") * 1e-3) / 1e12
        out["ffn_down"] = 2 * cfg.rows * cfg.hidden * cfg.intermediate / (avg("ffn_down") * 1e-3) / 1e12
    return {k: round(v, 2) for k, v in out.items()}


# ---------------------------------------------------------------- CPU baseline
def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def reference_gemm_check(cfg, threads):
    """One 64-row slice of the workload's up-projection GEMM (hidden ->
    2 x intermediate, fp32) through the reference's own CPU GEMM runtime
    (apply_schedule + execute under decoder_schedule's Latency family, built
    from the reference sources into oracle/_ref) and through the oracle's
    sfgo_matmul, same operands, same thread count: both rates, and whether
    the two results agree bit for bit."""
    import numpy as np
    import oracle
    if oracle.ref_gemm_lib() is None:
        return "oracle/_ref/libsfg_ref_gemm.so not built"
    m, n, k = 64, 2 * cfg.intermediate, cfg.hidden
    a = oracle.normal(7, 0, (m, k))
    b = oracle.normal(7, 1, (k, n), std=0.02)
    flops = 2.0 * m * n * k
    t = time.perf_counter()
    want = oracle.reference_gemm(a, b, family=0, threads=threads)
    ref_s = time.perf_counter() - t
    t = time.perf_counter()
    got = oracle.matmul(a, b)
    port_s = time.perf_counter() - t
    return {"shape_mnk": [m, n, k], "threads": threads,
            "reference_execute_gflops": round(flops / ref_s / 1e9, 2),
            "oracle_gflops": round(flops / port_s / 1e9, 2),
            "bit_identical": bool(np.array_equal(got.view(np.uint32), want.view(np.uint32)))}


def cpu_baseline(cfg, budget_s: float):
    """Time the CPU restatement on whole layer steps of the workload.

    Every configuration, C4's 8192-row prefill included, runs complete layer
    steps (sfgo_decoder_layer: every row through every stage, nothing
    extrapolated), repeated until budget_s is spent, at least once; the value
    is rows over the median step time (the reference's execute_decoder_layer
    reports the median, decoder_compiler.cpp:684-687), with the fastest and
    slowest steps beside it.  The oracle's products are register-blocked
    (4 x 32 outputs per AVX2 kernel, as the reference's register_kernel_16/8,
    runtime.cpp:278-370), so a C4 layer is a few tens of seconds on a
    16-thread host."""
    import statistics
    import oracle
    threads = oracle.lib().sfgo_num_threads()
    d, q = timing_data(cfg, 99)
    step = oracle.prepared_layer(cfg, d, quant=q)  # inputs marshalled once, outside the timing
    steps, spent = [], 0.0
    while True:
        t = time.time()
        step()
        steps.append(time.time() - t)
        spent += steps[-1]
        if spent > budget_s or len(steps) >= 1000:
            break
    med = statistics.median(steps)
    return {"value": round(cfg.rows / med, 3), "unit": "tokens/s", "cores": threads,
            "kind": "port",
            "what": "restatement: oracle/sfg_oracle.c, a C restatement of reference_decoder_layer "
                    "(OpenMP over the host's threads)",
            "method": f"measured: median of {len(steps)} whole layer step(s), nothing extrapolated",
            "reference_cpu_path": "decoder, attention and MoE compilers not built: they call "
                                  "the LLVM JIT (LLVMJITBackend), and LLVM 18 is not in this "
                                  "image; the reference's GEMM runtime is built and timed in "
                                  "reference_gemm",
            "reference_gemm": reference_gemm_check(cfg, threads),
            "cpu_model": cpu_model(), "threads": threads,
            "step_s": {"median": round(med, 4), "min": round(min(steps), 4),
                       "max": round(max(steps), 4)},
            "sample": f"{len(steps)} full layer step(s) of {cfg.rows} rows in {spent:.1f} s "
                      f"({med * 1e3:.1f} ms per step, median)"}


# ---------------------------------------------------------------- one configuration
def workload_name(name, cfg):
    return (f"BASELINE config {name[1]}: " + ("decode" if cfg.decode else "prefill")
            + f" B{cfg.batch} S{cfg.sequence} H{cfg.hidden} Hq{cfg.query_heads}/Hkv{cfg.kv_heads}"
            + f" D{cfg.head_dim} "
            + (f"MoE E{cfg.experts} top{cfg.top_k} I{cfg.intermediate}" if cfg.moe
               else f"SwiGLU I{cfg.intermediate}")
            + (f" ctx{cfg.context_sequence} paged{cfg.page_tokens}" if cfg.decode else "")
            + {"f32": " fp32", "bf16": " bf16", "w8": " int8 weights / bf16 activations"}[cfg.dtype])


def measure(name, args, device="cuda:0"):
    import torch
    from schedforge_amd import CONFIGS, CONFIG_SEEDS, algorithmic_work
    from schedforge_amd import configs as C
    from schedforge_amd import _abi
    from schedforge_amd.layer import StageEvents, compile_decoder, run_layer, stage_times

    cfg = CONFIGS[name]
    data, perm = make_device_data(cfg, CONFIG_SEEDS[name], device)
    plan = compile_decoder(cfg, data, device, page_permutation=perm)
    x = data.input.contiguous()
    del data
    torch.cuda.empty_cache()
    out = torch.empty((cfg.rows, cfg.hidden), dtype=torch.float32, device=device)

    for _ in range(args.warmup):
        run_layer(plan, x, out)
    torch.cuda.synchronize()

    # Timed region: K layer steps; in every mark_every-th step two HIP events
    # on the layer's stream bracket the roofline kernel: the paged attention
    # kernel (decode) or the FFN up-projection GEMM (prefill; for MoE the
    # grouped expert GEMMs).
    marks = (_abi.MARK_ROPE, _abi.MARK_ATTN_MAIN) if cfg.decode else (_abi.MARK_ROUTE, _abi.MARK_FFN_UP)
    every = max(1, args.mark_every)
    events = {i: StageEvents(plan.lib, marks) for i in range(0, args.steps, every)}
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        run_layer(plan, x, out, events=events.get(i))
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    kern_times = [e.elapsed(*marks) for e in events.values()]
    for e in events.values():
        e.close()
    ms_per_step = wall_ms / args.steps
    tokens_s = cfg.rows * 1000.0 / ms_per_step

    # Stage breakdown (untimed, informative): a few steps with every mark.
    full = [StageEvents(plan.lib) for _ in range(5)]
    for e in full:
        run_layer(plan, x, out, events=e)
    torch.cuda.synchronize()
    stages = [stage_times(e) for e in full]
    for e in full:
        e.close()
    del plan, x, out
    torch.cuda.empty_cache()
    work = algorithmic_work(cfg)
    cold = cold_decode(name, cfg, work, args, device) if cfg.decode else None

    def avg(key):
        return sum(s[key] for s in stages) / len(stages)

    traffic = measured_traffic(name)
    kern_ms = sum(kern_times) / len(kern_times)
    if cfg.decode:
        bytes_ = decode_attention_bytes(cfg)
        achieved = bytes_ / (kern_ms * 1e-3) / 1e9
        roofline = {"bound": "hbm", "kernel": "attn_decode_split_kernel", "achieved":
                    round(achieved, 1), "peak": C.PEAK_HBM_GBPS, "unit": "GB/s",
                    "frac": round(achieved / C.PEAK_HBM_GBPS, 4),
                    "traffic": traffic["bytes"] if traffic else None,
                    "algorithmic_bytes": bytes_, "avg_ms": round(kern_ms, 5),
                    "timed_launches": len(kern_times)}
    else:
        # prefill: the FFN up-projection's algorithmic FLOPs (2 rows H 2I for
        # the packed gate|up GEMM; 4 T k H I for the grouped W1|W3 expert GEMM
        # plus 2 T k H I for W2) over its bracketed time
        peak = C.PEAK_F32_TFLOPS if cfg.dtype == "f32" else C.PEAK_BF16_TFLOPS
        T, H, I, K, E = cfg.rows, cfg.hidden, cfg.intermediate, cfg.top_k, cfg.experts
        esz = 4 if cfg.dtype == "f32" else 2
        if cfg.moe:
            kflops = 6 * T * K * H * I
            kname = "gemm_dma_kernel grouped expert GEMMs (W1|W3 + SwiGLU, W2)"
            # W1|W3: x rows gathered, weights, act out; W2: act in, weights, fp32 y out
            kbytes = esz * (T * H + E * 2 * I * H + T * K * I) + esz * (T * K * I + E * H * I) + 4 * T * K * H
        else:
            kflops = 2 * T * H * 2 * I
            kname = ("gemm_vec_kernel" if cfg.dtype == "f32" else "gemm_dma_kernel") + " (gate|up + SwiGLU)"
            kbytes = esz * (T * H + 2 * I * H + T * I)
        achieved = kflops / (kern_ms * 1e-3) / 1e12
        layer_tf = work["flops"] / (ms_per_step * 1e-3) / 1e12
        roofline = {"bound": "mfma", "kernel": kname,
                    "achieved": round(achieved, 2), "peak": peak, "unit": "TFLOP/s",
                    "frac": round(achieved / peak, 4),
                    "traffic": traffic["bytes"] if traffic else None, "algorithmic_bytes": kbytes,
                    "algorithmic_flops": kflops, "avg_ms": round(kern_ms, 5),
                    "timed_launches": len(kern_times),
                    "layer_tflops": round(layer_tf, 2), "layer_frac": round(layer_tf / peak, 4)}
    block = {
        "value": round(tokens_s, 2),
        "ms_per_step": round(ms_per_step, 5),
        "dtype": {"f32": "f32", "bf16": "bf16", "w8": "int8-weight/bf16"}[cfg.dtype],
        "config": {"workload": workload_name(name, cfg), "rows": cfg.rows,
                   "layer_hbm_gbps": round(work["bytes"] / (ms_per_step * 1e-3) / 1e9, 1),
                   "stage_ms": {k: round(avg(k), 5) for k in stages[0]},
                   "stage_tflops": stage_tflops(cfg, work, avg)},
        "roofline": roofline,
    }
    if cold is not None:
        block["cold"] = cold
    if not args.no_cpu_baseline:
        block["cpu_baseline"] = cpu_baseline(cfg, args.cpu_seconds)
    return block


# Infinity Cache (MALL) of one MI355X: a decode step whose weights and KV fit
# in it is served from it when steps repeat.
MALL_BYTES = 256 << 20


def cold_decode(name, cfg, work, args, device):
    """Decode steps whose working set is not cache-resident: when one layer's
    bytes (weights + KV + activations) fit twice in the MALL, build enough
    independent copies (own weights, KV pool, page table and workspace) that
    together they exceed twice its size, and time args.steps steps that rotate
    over them, so no step finds its data in the MALL or L2 from the step
    before.  Returns None when one layer already exceeds twice the MALL."""
    import math
    import torch
    from schedforge_amd import CONFIG_SEEDS
    from schedforge_amd.layer import compile_decoder, run_layer

    per_layer = work["bytes"]
    if per_layer >= 2 * MALL_BYTES:
        return None
    copies = max(2, math.ceil(2 * MALL_BYTES / per_layer) + 1)
    plans, xs = [], []
    for c in range(copies):
        data, perm = make_device_data(cfg, CONFIG_SEEDS[name] + 1000 + c, device)
        plans.append(compile_decoder(cfg, data, device, page_permutation=perm))
        xs.append(data.input.contiguous())
        del data
    out = torch.empty((cfg.rows, cfg.hidden), dtype=torch.float32, device=device)
    for i in range(max(args.warmup, copies)):
        run_layer(plans[i % copies], xs[i % copies], out)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        run_layer(plans[i % copies], xs[i % copies], out)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    del plans, xs, out
    torch.cuda.empty_cache()
    return {"value": round(cfg.rows * 1000.0 / ms, 2), "ms_per_step": round(ms, 5), "copies": copies,
            "rotated_mb": round(copies * per_layer / 1e6, 1),
            "note": "steps rotate over independent weight sets and KV pools larger than the MALL"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported here "
              "(multi-GPU sharding is design-only for this backend).", file=sys.stderr)
        sys.exit(2)
    import torch
    from schedforge_amd import CONFIGS, load

    load()
    device = "cuda:0"
    if args.copy_calibration > 0:
        n = args.copy_calibration * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.mul(src, 1.0, out=dst)   # one launch: n*4 bytes read, n*4 written
        torch.cuda.synchronize()
        del src, dst
        torch.cuda.empty_cache()

    head = measure(args.config, args, device)
    line = {
        "metric": "decoder-layer equiv. tokens/s (1 GPU)",
        "value": head["value"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head["dtype"],
        "data": "synthetic (device-drawn N(0,1) activations / KV, N(0,0.02) weights)",
        "config": head["config"],
        "roofline": head["roofline"],
    }
    if "cold" in head:
        line["cold"] = head["cold"]
    if "cpu_baseline" in head:
        line["cpu_baseline"] = head["cpu_baseline"]
    if not CONFIGS[args.config].decode and args.decode_config != "none":
        dec = measure(args.decode_config, args, device)
        line["decode"] = {"metric": line["metric"], "unit": "tokens/s", "steps": args.steps,
                          "warmup": args.warmup, **dec}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
