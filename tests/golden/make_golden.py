"""Write tests/golden/golden_v1.npz: small input/output vectors for the oracle.

The expected outputs are computed here in float64 NumPy straight from the
reference's definitions (cited per case), NOT by the oracle, so the fixtures pin
the oracle independently of its own code.  Inputs are fixed by a NumPy seed and
stored with the outputs.  Regenerate with:  python tests/golden/make_golden.py
"""
from __future__ import annotations

from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "golden_v1.npz"


def rmsnorm(x, w, eps):
    # decoder_compiler.cpp:41-62
    return x / np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + eps) * w


def attention(q, k, v, causal):
    # attention_compiler.cpp:742-781 (+ causal alignment 68-72, GQA 150/310)
    b, hq, sq, d = q.shape
    hkv, skv = k.shape[1], k.shape[2]
    out = np.zeros((b, hq, sq, v.shape[3]))
    for bi in range(b):
        for h in range(hq):
            kh = h * hkv // hq
            s = q[bi, h].astype(np.float64) @ k[bi, kh].T.astype(np.float64) / np.sqrt(d)
            if causal:
                for i in range(sq):
                    s[i, skv - sq + i + 1:] = -np.inf
            p = np.exp(s - s.max(1, keepdims=True))
            p /= p.sum(1, keepdims=True)
            out[bi, h] = p @ v[bi, kh]
    return out


def route(x, router, bias, k):
    # moe_compiler.cpp:412-455; ties to the lower expert index
    logits = x.astype(np.float64) @ router.astype(np.float64)
    if bias is not None:
        logits = logits + bias
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    ids = np.argsort(-logits, axis=1, kind="stable")[:, :k].astype(np.int32)
    sel = np.take_along_axis(p, ids, 1)
    return ids, sel / sel.sum(1, keepdims=True)


def dispatch(ids, experts):
    # moe_compiler.cpp:496-528: stable by (expert, token, slot)
    flat = ids.reshape(-1)
    order = np.argsort(flat, kind="stable")
    counts = np.bincount(flat, minlength=experts)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    k = ids.shape[1]
    return offsets, (order // k).astype(np.int32), (order % k).astype(np.int32)


def moe(x, w1, w3, w2, ids, wts):
    # moe_compiler.cpp:640-682: (x W1) * silu(x W3), then W2, weighted sum
    out = np.zeros((x.shape[0], w2.shape[2]))
    for t in range(x.shape[0]):
        for s in range(ids.shape[1]):
            e = ids[t, s]
            g = x[t] @ w1[e]
            u = x[t] @ w3[e]
            out[t] += wts[t, s] * ((g * (u / (1 + np.exp(-u)))) @ w2[e])
    return out


def quantize_kn(w_kn):
    # next_milestones.cpp:611-637 on the transposed weight; std::round = half away
    w = w_kn.T.astype(np.float32)
    m = np.abs(w).max(1)
    s = np.where(m > 0, (m / np.float32(127.0)).astype(np.float32), np.float32(1.0)).astype(np.float32)
    r = (w / s[:, None]).astype(np.float32)
    q = np.sign(r) * np.floor(np.abs(r) + 0.5)
    return np.clip(q, -127, 127).astype(np.int8), s


def rope(t, theta):
    # decoder_compiler.cpp:96-114, pos = index within the sequence
    b, h, s, d = t.shape
    out = t.astype(np.float64).copy()
    for pos in range(s):
        for i in range(0, d, 2):
            f = np.float32(theta) ** (-np.float32(i) / np.float32(d))
            a = np.float64(np.float32(pos) * np.float32(f))
            e, o = t[:, :, pos, i].astype(np.float64), t[:, :, pos, i + 1].astype(np.float64)
            out[:, :, pos, i] = e * np.cos(a) - o * np.sin(a)
            out[:, :, pos, i + 1] = e * np.sin(a) + o * np.cos(a)
    return out


def main():
    rng = np.random.default_rng(20261201)
    f = lambda *s, sd=1.0: (rng.standard_normal(s) * sd).astype(np.float32)  # noqa: E731
    g = {}
    x = f(5, 64); w = f(64, sd=0.3) + 1.0
    g["rms_x"], g["rms_w"], g["rms_y"] = x, w, rmsnorm(x, w, 1e-5)
    q, k, v = f(1, 4, 6, 16), f(1, 2, 9, 16), f(1, 2, 9, 16)
    g["att_q"], g["att_k"], g["att_v"] = q, k, v
    g["att_causal"] = attention(q, k, v, True)
    g["att_full"] = attention(q, k, v, False)
    xr, router, bias = f(24, 32), f(32, 6, sd=0.3), f(6, sd=0.5)
    ids, wts = route(xr, router, bias, 2)
    g["route_x"], g["route_w"], g["route_b"], g["route_ids"], g["route_wts"] = xr, router, bias, ids, wts
    off, tok, slot = dispatch(ids, 6)
    g["disp_offsets"], g["disp_tokens"], g["disp_slots"] = off, tok, slot
    w1, w3, w2 = f(6, 32, 20, sd=0.2), f(6, 32, 20, sd=0.2), f(6, 20, 32, sd=0.2)
    g["moe_w1"], g["moe_w3"], g["moe_w2"] = w1, w3, w2
    g["moe_out"] = moe(xr, w1, w3, w2, ids, wts.astype(np.float32))
    wq = f(48, 10, sd=0.05)
    wq[:, 4] = 0.0
    qq, ss = quantize_kn(wq)
    g["q_w"], g["q_q"], g["q_s"] = wq, qq, ss
    t = f(1, 2, 7, 16)
    g["rope_in"], g["rope_out"] = t, rope(t, 10000.0)
    vals = np.array([-1.25, 0.0, 0.75, 3.5, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -2.0 ** -130,
                     3.1415926, 65504.0], np.float32)
    bits = vals.view(np.uint32).astype(np.uint64)
    g["bf16_in"] = vals
    g["bf16_bits"] = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)
    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT} ({len(g)} arrays)")


if __name__ == "__main__":
    main()
