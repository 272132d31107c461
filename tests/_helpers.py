"""Shared test helpers: device buffers, oracle-data -> DecoderData, reduced configs."""
from __future__ import annotations

import ctypes

import numpy as np

from schedforge_amd import CONFIGS

# Reduced versions of the five configs: same structure (dtype, GQA ratio,
# head_dim 128, paging, MoE top-2 of 8) at sizes the CPU oracle finishes in
# seconds.
SMALL = {
    "c1": CONFIGS["c1"],
    "c2": CONFIGS["c2"].replace(batch=4, hidden=1024, intermediate=2816, query_heads=8,
                                kv_heads=2, context_sequence=1000),
    "c3": CONFIGS["c3"].replace(batch=2, sequence=256, hidden=1024, intermediate=512,
                                query_heads=8, kv_heads=2),
    "c4": CONFIGS["c4"].replace(sequence=512, hidden=1024, intermediate=2048, query_heads=8,
                                kv_heads=2),
    "c5": CONFIGS["c5"].replace(batch=16, hidden=1024, intermediate=2048, query_heads=8,
                                kv_heads=2, context_sequence=1024),
}

TOL = {"f32": 1e-4, "bf16": 2e-2, "w8": 1e-2}


def decoder_data(d):
    from schedforge_amd.layer import DecoderData
    return DecoderData(**{k: getattr(d, k) for k in DecoderData.__dataclass_fields__
                          if hasattr(d, k)})


# Device tensors handed to the C ABI as raw pointers must outlive the
# asynchronous kernels that read them: a temporary's block goes back to
# torch's caching allocator at once and the next allocation can reuse it.
# Every tensor made here stays referenced until the test ends (see the
# autouse fixture in conftest.py, which synchronises first).
KEEP_ALIVE: list = []


def stream():
    import torch
    return torch.cuda.current_stream().cuda_stream


def dev(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    t = t.cuda()
    KEEP_ALIVE.append(t)
    return t


def bf16_dev(a):
    """fp32 numpy -> device int16 tensor holding bf16 bits (RNE)."""
    import oracle
    import torch
    bits = oracle.to_bf16_bits(a).view(np.int16)
    t = torch.from_numpy(bits).cuda()
    KEEP_ALIVE.append(t)
    return t


def host(t):
    return t.detach().cpu().numpy()


def bf16_host(t):
    """device int16 bf16 bits -> fp32 numpy."""
    bits = host(t).view(np.uint16).astype(np.uint32) << 16
    return bits.view(np.float32)


def tile_nk(w_nk, kind):
    """NumPy restatement of SFG_LAYOUT_TILED for an [N][K] matrix.
    bf16: [N/16][K/128][4 s][64 lanes][8], lane l holds row l % 16,
          k = 32 s + 8 (l // 16) + j;
    int8: [N/16][K/128][2 t][64 lanes][16], k = 32 (l // 16) + 16 t + j."""
    n, k = w_nk.shape
    lanes = np.arange(64)
    r, g = lanes % 16, lanes // 16
    if kind == "bf16":
        s = np.arange(4)[:, None, None]
        j = np.arange(8)[None, None, :]
        kk = 32 * s + 8 * g[None, :, None] + j                      # [4][64][8]
        rows = np.broadcast_to(r[None, :, None], kk.shape)
    else:
        t = np.arange(2)[:, None, None]
        j = np.arange(16)[None, None, :]
        kk = 32 * g[None, :, None] + 16 * t + j                     # [2][64][16]
        rows = np.broadcast_to(r[None, :, None], kk.shape)
    nt = np.arange(n // 16)[:, None, None, None, None] * 16
    kc = np.arange(k // 128)[None, :, None, None, None] * 128
    return np.ascontiguousarray(w_nk[nt + rows[None, None], kc + kk[None, None]])
