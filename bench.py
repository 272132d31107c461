"""Decoder-layer benchmark on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2]

A step is one execution of the whole decoder layer (execute_once,
decoder_compiler.cpp:218-304) on one batch of synthetic input, inputs resident in
HBM.  The default workload is BASELINE config 2 (medium dense decode, bf16,
paged KV) -- the configuration the headline metric is quoted on.  The metric is
the reference's: equivalent tokens/s = rows * 1000 / ms (decoder_compiler.cpp:
301-302, 688-689), rows = batch * sequence.

The JSON line also carries:
  roofline      the dominant kernel's achieved fraction of its MI355X peak,
                from HIP events recorded around it on the layer's stream in
                every --mark-every'th step of the timed region (decode: the
                paged Split-KV attention kernel, HBM bound; prefill: the FFN
                up-projection GEMM).  An event record drains the queue around
                the kernel it brackets (about 6 us per marked decode step), so
                marking only some steps keeps that cost out of the throughput;
  cpu_baseline  the CPU oracle (a C restatement of the reference path) timed on
                this host on a bounded sample of the same workload.
Synthetic data: activations N(0,1), weights N(0,0.02), cached K/V N(0,1), drawn
on the device; norm gains 1; random page table.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

# HBM traffic per launch of the roofline kernel, from two rocprofv3 --pmc runs
# of this script (FETCH_SIZE, then WRITE_SIZE; KiB per dispatch) with
# --copy-calibration 1024.  The calibration kernel reads 1 GiB and writes 1 GiB;
# the counters read 524311.8 KiB and 1048576.0 KiB for it, so FETCH_SIZE is
# scaled by 1048576 / 524311.8 and WRITE_SIZE by 1.  Summaries:
# profiles/pmc_traffic_c2.md, profiles/pmc_traffic_c5.md (decode attention),
# profiles/pmc_traffic_prefill_gemm.md (C4 gate|up GEMM, C3 grouped experts).
PMC_FETCH_SCALE = 1048576.0 / 524311.8
PMC_WRITE_SCALE = 1.0
PMC_ROOFLINE_KIB = {           # roofline kernel(s) per launch: (FETCH_SIZE, WRITE_SIZE)
    "c2": (66117.8, 1088.0),                    # attn_decode_split_kernel
    "c5": (1049963.6, 2112.0),                  # attn_decode_split_kernel
    "c4": (1376849.7, 229376.0),                # gate|up GEMM + SwiGLU
    "c3": (143115.5 + 71003.0, 11264.0 + 32768.0),  # grouped W1|W3 + W2 expert GEMMs
}
MEASURED_TRAFFIC = {k: round((f * PMC_FETCH_SCALE + w * PMC_WRITE_SCALE) * 1024)
                    for k, (f, w) in PMC_ROOFLINE_KIB.items()}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5"])
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="bound on the CPU-baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--mark-every", type=int, default=5,
                   help="bracket the roofline kernel with HIP events in every N-th timed step")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                   help="before warmup, stream MIB MiB through one elementwise kernel "
                        "(reads MIB, writes MIB): the known-size reference for the "
                        "FETCH_SIZE / WRITE_SIZE counter runs")
    return p.parse_args()


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


def decode_attention_bytes(cfg):
    """Algorithmic HBM bytes of one paged decode-attention launch: K + V pages
    (bf16), Q (fp32), the merged output (bf16) and the page table."""
    pps = (cfg.context_sequence + cfg.page_tokens - 1) // cfg.page_tokens
    kv = 2 * cfg.batch * cfg.kv_heads * cfg.context_sequence * cfg.head_dim * 2
    q = cfg.batch * cfg.query_heads * cfg.head_dim * 4
    o = cfg.batch * cfg.query_heads * cfg.head_dim * 2
    pt = cfg.batch * pps * 4
    return kv + q + o + pt


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


def cpu_baseline(cfg, budget_s: float):
    """Time the CPU oracle (C restatement of reference_decoder_layer) on a
    bounded sample of the workload: full-size layer steps for decode / small
    prefill configs, a row-sliced prefill for the large ones."""
    import numpy as np
    import oracle
    threads = oracle.lib().sfgo_num_threads()
    sample = cfg
    note = "full layer step"
    if not cfg.decode and cfg.rows > 256:
        # the prefill's cost is dominated by the GEMMs and attention over all
        # rows; sample a prefix of the sequence and scale by rows
        seq = 256 if cfg.sequence > 256 else cfg.sequence
        sample = cfg.replace(batch=1, sequence=seq)
        note = f"prefill sample batch 1 seq {seq} (scaled per row)"
    t0 = time.time()
    d = oracle.make_layer_data(sample, 99)
    gen_s = time.time() - t0
    q = oracle.quantize_layer(sample, d) if sample.dtype == "w8" else None
    reps, spent = 0, 0.0
    while True:
        t = time.time()
        oracle.decoder_layer(sample, d, quant=q)
        spent += time.time() - t
        reps += 1
        if spent > budget_s or reps >= 1000:  # the time budget governs
            break
    per_step = spent / reps
    tok_s = sample.rows / per_step
    return {"value": round(tok_s, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{note}: {reps} x {sample.rows} rows in {spent:.1f} s "
                      f"({per_step * 1e3:.1f} ms/step; data generation {gen_s:.1f} s untimed)"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported here "
              "(multi-GPU sharding is design-only for this backend).", file=sys.stderr)
        sys.exit(2)
    import torch
    from schedforge_amd import CONFIGS, CONFIG_SEEDS, algorithmic_work, load
    from schedforge_amd import configs as C
    from schedforge_amd import _abi
    from schedforge_amd.layer import StageEvents, compile_decoder, run_layer, stage_times

    load()
    device = "cuda:0"
    cfg = CONFIGS[args.config]
    data, perm = make_device_data(cfg, CONFIG_SEEDS[args.config], device)
    plan = compile_decoder(cfg, data, device, page_permutation=perm)
    x = data.input.contiguous()
    del data
    torch.cuda.empty_cache()
    out = torch.empty((cfg.rows, cfg.hidden), dtype=torch.float32, device=device)
    stream = torch.cuda.current_stream()

    if args.copy_calibration > 0:
        n = args.copy_calibration * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.mul(src, 1.0, out=dst)   # one launch: n*4 bytes read, n*4 written
        torch.cuda.synchronize()
        del src, dst
        torch.cuda.empty_cache()

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

    def avg(key):
        return sum(s[key] for s in stages) / len(stages)

    work = algorithmic_work(cfg)
    if cfg.decode:
        att_ms = sum(kern_times) / len(kern_times)
        bytes_ = decode_attention_bytes(cfg)
        achieved = bytes_ / (att_ms * 1e-3) / 1e9
        roofline = {"bound": "hbm", "kernel": "attn_decode_split_kernel", "achieved":
                    round(achieved, 1), "peak": C.PEAK_HBM_GBPS, "unit": "GB/s",
                    "frac": round(achieved / C.PEAK_HBM_GBPS, 4),
                    "traffic": MEASURED_TRAFFIC.get(args.config),
                    "algorithmic_bytes": bytes_, "avg_ms": round(att_ms, 5),
                    "timed_launches": len(kern_times)}
    else:
        # prefill: the FFN up-projection's algorithmic FLOPs (2 rows H 2I for
        # the packed gate|up GEMM; 4 T k H I for the grouped W1|W3 expert GEMM
        # plus 2 T k H I for W2) over its bracketed time
        peak = C.PEAK_F32_TFLOPS if cfg.dtype == "f32" else C.PEAK_BF16_TFLOPS
        ffn_ms = sum(kern_times) / len(kern_times)
        T, H, I, K, E = cfg.rows, cfg.hidden, cfg.intermediate, cfg.top_k, cfg.experts
        esz = 4 if cfg.dtype == "f32" else 2
        if cfg.moe:
            kflops = 6 * T * K * H * I
            kname = "gemm_dma_kernel grouped expert GEMMs (W1|W3 + SwiGLU, W2)"
            # W1|W3: x rows gathered, weights, act out; W2: act in, weights, fp32 y out
            kbytes = esz * (T * H + E * 2 * I * H + T * K * I) + esz * (T * K * I + E * H * I) + 4 * T * K * H
        else:
            kflops = 2 * T * H * 2 * I
            kname = ("gemm_f32_kernel" if cfg.dtype == "f32" else "gemm_dma_kernel") + " (gate|up + SwiGLU)"
            kbytes = esz * (T * H + 2 * I * H + T * I)
        achieved = kflops / (ffn_ms * 1e-3) / 1e12
        roofline = {"bound": "mfma", "kernel": kname,
                    "achieved": round(achieved, 2), "peak": peak, "unit": "TFLOP/s",
                    "frac": round(achieved / peak, 4),
                    "traffic": MEASURED_TRAFFIC.get(args.config), "algorithmic_bytes": kbytes,
                    "algorithmic_flops": kflops, "avg_ms": round(ffn_ms, 5),
                    "timed_launches": len(kern_times),
                    "layer_tflops": round(work["flops"] / (ms_per_step * 1e-3) / 1e12, 2),
                    "layer_frac": round(work["flops"] / (ms_per_step * 1e-3) / 1e12 / peak, 4)}
    layer_gbps = work["bytes"] / (ms_per_step * 1e-3) / 1e9
    line = {
        "metric": "decoder-layer equiv. tokens/s (1 GPU)",
        "value": round(tokens_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"f32": "f32", "bf16": "bf16", "w8": "int8-weight/bf16"}[cfg.dtype],
        "data": "synthetic (device-drawn N(0,1) activations / KV, N(0,0.02) weights)",
        "config": {"workload": f"BASELINE config {args.config[1]}: "
                   + ("decode" if cfg.decode else "prefill")
                   + f" B{cfg.batch} S{cfg.sequence} H{cfg.hidden} Hq{cfg.query_heads}/Hkv{cfg.kv_heads}"
                   + f" D{cfg.head_dim} {'MoE E%d top%d I%d' % (cfg.experts, cfg.top_k, cfg.intermediate) if cfg.moe else 'SwiGLU I%d' % cfg.intermediate}"
                   + (f" ctx{cfg.context_sequence} paged{cfg.page_tokens}" if cfg.decode else ""),
                   "rows": cfg.rows, "layer_hbm_gbps": round(layer_gbps, 1),
                   "stage_ms": {k: round(avg(k), 5) for k in stages[0]},
                   "stage_tflops": stage_tflops(cfg, work, avg)},
        "roofline": roofline,
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(cfg, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
