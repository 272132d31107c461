"""Decoder-layer configuration (mirror of schedforge::DecoderConfig,
decoder_compiler.h:17-32) and the five benchmark configurations.

Build extensions beyond the reference's fields:
  dtype        "f32" | "bf16" | "w8"  (w8: int8 per-channel weights, bf16 activations)
  page_tokens  paged-KV page size for decode steps
  router_bias_std  std of the per-expert router logit bias (0: no bias)
"""
from __future__ import annotations

import dataclasses
from dataclasses import dataclass


@dataclass
class DecoderConfig:
    batch: int = 1
    sequence: int = 16
    hidden: int = 64
    intermediate: int = 128
    query_heads: int = 4
    kv_heads: int = 2
    head_dim: int = 16
    rms_epsilon: float = 1.0e-5
    rope_theta: float = 10000.0
    causal: bool = True
    ffn: str = "dense"          # "dense" | "moe"  (DecoderFFNKind)
    experts: int = 4
    top_k: int = 2
    context_sequence: int = 0   # 0: prefill; > 0: decode step over cached K/V
    # build extensions
    dtype: str = "f32"
    page_tokens: int = 16
    router_bias_std: float = 0.0
    # decode only: append the step's K/V into the paged cache at the true
    # position (not the reference's semantics; see sfg_layer_desc.kv_append)
    kv_append: bool = False
    # page-table capacity in tokens for append plans (0: context + 1)
    kv_capacity: int = 0

    @property
    def rows(self) -> int:
        return self.batch * self.sequence

    @property
    def kv_width(self) -> int:
        return self.kv_heads * self.head_dim

    @property
    def qkv_width(self) -> int:
        return self.hidden + 2 * self.kv_width

    @property
    def moe(self) -> bool:
        return self.ffn == "moe"

    @property
    def decode(self) -> bool:
        return self.context_sequence > 0

    def validate(self) -> None:
        """validate() of decoder_compiler.cpp:26-39."""
        if (self.batch <= 0 or self.sequence <= 0 or self.hidden <= 0 or self.intermediate <= 0
                or self.query_heads <= 0 or self.kv_heads <= 0 or self.head_dim <= 0
                or self.hidden != self.query_heads * self.head_dim
                or self.query_heads % self.kv_heads != 0 or not self.rms_epsilon > 0.0):
            raise ValueError("invalid decoder configuration")
        if self.moe and (self.experts <= 0 or self.top_k <= 0 or self.top_k > self.experts):
            raise ValueError("invalid decoder MoE configuration")
        if self.context_sequence < 0:
            raise ValueError("invalid decoder context sequence")
        if self.dtype not in ("f32", "bf16", "w8"):
            raise ValueError(f"unknown dtype {self.dtype}")
        if self.kv_append and not self.decode:
            raise ValueError("kv append needs a decode step (context > 0)")

    @property
    def capacity(self) -> int:
        """Tokens the per-sequence page tables hold: the cached context, or for
        append plans room for the tokens still to come."""
        if not self.kv_append:
            return self.context_sequence
        return max(self.kv_capacity, self.context_sequence + self.sequence)

    def replace(self, **kw) -> "DecoderConfig":
        return dataclasses.replace(self, **kw)


# BASELINE.json configs[0..4]
CONFIGS = {
    "c1": DecoderConfig(batch=1, sequence=128, hidden=256, intermediate=688, query_heads=4,
                        kv_heads=2, head_dim=64, rms_epsilon=1e-6, dtype="f32"),
    "c2": DecoderConfig(batch=16, sequence=1, hidden=2048, intermediate=5632, query_heads=16,
                        kv_heads=4, head_dim=128, context_sequence=4096, dtype="bf16"),
    "c3": DecoderConfig(batch=4, sequence=512, hidden=2048, intermediate=1408, query_heads=16,
                        kv_heads=4, head_dim=128, ffn="moe", experts=8, top_k=2, dtype="bf16",
                        router_bias_std=0.5),
    "c4": DecoderConfig(batch=1, sequence=8192, hidden=4096, intermediate=14336, query_heads=32,
                        kv_heads=8, head_dim=128, dtype="bf16"),
    "c5": DecoderConfig(batch=64, sequence=1, hidden=4096, intermediate=14336, query_heads=32,
                        kv_heads=8, head_dim=128, ffn="moe", experts=8, top_k=2,
                        context_sequence=8192, dtype="w8"),
}

CONFIG_SEEDS = {"c1": 1000, "c2": 2000, "c3": 3000, "c4": 4000, "c5": 5000}


def causal_pairs(sq: int, skv: int) -> int:
    """Number of allowed (query, key) pairs under the reference's causal rule
    j <= Skv - Sq + i (attention_compiler.cpp:68-72)."""
    off = skv - sq
    total = 0
    for i in range(sq):
        total += min(skv, max(0, off + i + 1))
    return total


def algorithmic_work(cfg: DecoderConfig, expert_rows: int | None = None) -> dict:
    """Per-layer-step algorithmic FLOPs and HBM bytes (the roofline units).

    proj = 2 rows H (H + 2 kvD) + 2 rows H^2; dense FFN = 6 rows H I;
    MoE = 6 T k H I + 2 T H E; attention = 2 (D + Dv) x allowed pairs x B x Hq.
    Bytes: every weight byte once, KV once (decode), activations in and out.

    A decode step with the reference's semantics attends over the cache only
    and discards the step's own K / V (decoder_compiler.cpp:238-243), so the
    layer computes only the Q columns of the QKV product: that step counts
    2 rows H H for it and reads only Wq's bytes.  "reference_proj_flops" keeps
    the reference's full 2 rows H (H + 2 kvD).
    """
    rows, H, I = cfg.rows, cfg.hidden, cfg.intermediate
    D, kvd = cfg.head_dim, cfg.kv_width
    wbytes = {"f32": 4, "bf16": 2, "w8": 1}[cfg.dtype]
    abytes = 4 if cfg.dtype == "f32" else 2
    qkv_cols = H if cfg.decode and not cfg.kv_append else H + 2 * kvd
    reference_proj_flops = 2 * rows * H * (H + 2 * kvd) + 2 * rows * H * H
    proj_flops = 2 * rows * H * qkv_cols + 2 * rows * H * H
    proj_w = (H * qkv_cols + H * H) * wbytes
    skv = cfg.context_sequence if cfg.decode else cfg.sequence
    pairs = (causal_pairs(cfg.sequence, skv) if cfg.causal else cfg.sequence * skv)
    attn_flops = 2 * (D + D) * pairs * cfg.batch * cfg.query_heads
    if cfg.moe:
        assign = rows * cfg.top_k
        ffn_flops = 6 * assign * H * I + 2 * rows * H * cfg.experts
        ffn_w = 3 * cfg.experts * H * I * wbytes + H * cfg.experts * 4
    else:
        ffn_flops = 6 * rows * H * I
        ffn_w = 3 * H * I * wbytes
    # the paged pools hold the activation dtype: fp32 on the fp32 path, bf16 otherwise
    kv_bytes = 2 * cfg.batch * cfg.kv_heads * cfg.context_sequence * D * abytes if cfg.decode else 0
    act_bytes = rows * H * 4 * 2  # x in, out
    return {
        "flops": proj_flops + attn_flops + ffn_flops,
        "proj_flops": proj_flops, "attn_flops": attn_flops, "ffn_flops": ffn_flops,
        "reference_proj_flops": reference_proj_flops,
        "weight_bytes": proj_w + ffn_w, "kv_bytes": kv_bytes, "act_bytes": act_bytes,
        "bytes": proj_w + ffn_w + kv_bytes + act_bytes,
        "act_elem_bytes": abytes,
    }


# MI355X published peaks
PEAK_HBM_GBPS = 8000.0
PEAK_BF16_TFLOPS = 2500.0
PEAK_I8_TOPS = 5000.0
PEAK_F32_TFLOPS = 157.3
