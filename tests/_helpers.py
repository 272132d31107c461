"""Shared test helpers: device buffers, oracle-data -> DecoderData, reduced configs."""
from __future__ import annotations

import ctypes
import json
import os

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


# ---------------------------------------------------------------- layer checks
def _rel(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref)) / max(float(np.max(np.abs(ref))), 1e-6))


def branch_errors(x, out, taps, ref_out, ref_taps):
    """Relative errors of the layer output and of each of its branches, each
    against its own largest magnitude (max|got - ref| / max|ref|):
      out          the layer output;
      attn         the merged attention output (the attention kernel alone);
      attn_branch  r1 - x, what the attention block adds to the residual stream;
      ffn_branch   out - r1, what the FFN block adds.
    With N(0, 0.02) weights the residual stream dominates the output, so the
    whole-output error alone barely sees a broken attention; each branch is
    checked on its own scale."""
    x = np.asarray(x, np.float64)
    r1, rr1 = np.asarray(taps["residual1"], np.float64), np.asarray(ref_taps["residual1"], np.float64)
    return {"out": _rel(out, ref_out),
            "attn": _rel(taps["attn"], ref_taps["attn_merged"]),
            "attn_branch": _rel(r1 - x, rr1 - x),
            "ffn_branch": _rel(np.asarray(out, np.float64) - r1, np.asarray(ref_out, np.float64) - rr1)}


def assert_branches(x, out, taps, ref_out, ref_taps, tol, label=""):
    """Every branch error below tol.  With SFG_PARITY_LOG set to a file path,
    each check also appends {label, tol, rows, errors} to it as a JSON line
    (the record of the parity margins)."""
    err = branch_errors(x, out, taps, ref_out, ref_taps)
    print(f"{label} " + " ".join(f"{k} {v:.3e}" for k, v in err.items()))
    log = os.environ.get("SFG_PARITY_LOG")
    if log:
        with open(log, "a") as f:
            f.write(json.dumps({"label": label, "tol": tol, "rows": int(np.asarray(out).shape[0]),
                                **{k: float(v) for k, v in err.items()}}) + "\n")
    bad = {k: v for k, v in err.items() if not v < tol}
    assert not bad, f"{label}: over tolerance {tol}: {bad}"
    return err


# Router logits are O(1) here (N(0, 0.02) router weights over H >= 2048
# features, plus the bias).  The device's router input (its fp32 RMSNorm rows)
# may move the logits by at most this much against the oracle's; measured
# deviations are 1e-4 (decode) to 5e-3 (C3 prefill, whose attention branch
# carries bf16 rounding into the residual stream).
ROUTE_LOGIT_DEV_MAX = 1e-2


def route_logits(route_input, router, bias):
    lg = np.asarray(route_input, np.float64) @ np.asarray(router, np.float64)
    return lg + (0.0 if bias is None else np.asarray(bias, np.float64))


def near_tie_rows(logits, top_k, gap):
    """Rows whose top k + 1 sorted logits have an adjacent gap below `gap`: the
    only rows whose top-k set or slot order can change when every logit moves by
    less than gap / 2."""
    srt = -np.sort(-logits, axis=1)[:, :top_k + 1]
    return np.nonzero(np.min(srt[:, :-1] - srt[:, 1:], axis=1) < gap)[0]


def check_device_routing(dev_taps, ref_taps, router, bias, top_k):
    """Device routing against the oracle's.  With delta the largest logit
    deviation between the two router inputs (asserted below
    ROUTE_LOGIT_DEV_MAX), two experts can swap order only if the oracle's logits
    are closer than 2 delta: every row whose ids differ must be such a near tie,
    and rows that agree carry the same weights to within delta / 2.  Returns
    the rows that differ (the only rows the caller may exempt from the output
    tolerance)."""
    dev_logits = route_logits(dev_taps["route_input"], router, bias)
    ref_logits = route_logits(ref_taps["normalized2"], router, bias)
    delta = float(np.max(np.abs(dev_logits - ref_logits)))
    assert delta < ROUTE_LOGIT_DEV_MAX, f"router input deviates: logit error {delta:.3e}"
    # slack for the device's own fp32 logit chains against this fp64 product
    margin = 2 * delta + 1e-5
    differ = np.nonzero(np.any(dev_taps["ids"] != ref_taps["ids"], axis=1))[0]
    ties = near_tie_rows(ref_logits, top_k, margin)
    assert set(differ.tolist()) <= set(ties.tolist()), (differ, ties)
    # renormalised top-k weights move by at most half the logit deviation
    same = np.setdiff1d(np.arange(len(ref_logits)), differ)
    wdev = float(np.max(np.abs(dev_taps["weights"][same] - ref_taps["weights"][same]), initial=0.0))
    assert wdev <= delta / 2 + 1e-6, (wdev, delta)
    print(f"routing: logit deviation {delta:.2e}, near ties (gap < {margin:.2e}) {len(ties)}, "
          f"rows routed differently {len(differ)}")
    return differ
