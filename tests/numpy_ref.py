"""Independent numpy restatements used to pin the oracle.

Written from the mathematics of the reference path, not from oracle.cpp:
float64 closed forms for the model arithmetic, and float32 emulation only
where a test checks an exact rounding sequence.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32


def round_half_away(x):
    return np.sign(x) * np.floor(np.abs(x) + 0.5)


def q8_quantize(x):
    """quantize_row_q8_0 in float32 arithmetic: per 32-block d = amax/127,
    inv = 1/d, q = round-half-away(x * inv) clamped to +-127."""
    x = np.asarray(x, F32).reshape(-1, 32)
    amax = np.max(np.abs(x), axis=1).astype(F32)
    d = (amax / F32(127.0)).astype(F32)
    with np.errstate(divide="ignore"):
        inv = np.where(d == 0, F32(0), F32(1.0) / np.where(d == 0, F32(1), d)).astype(F32)
    p = (x * inv[:, None]).astype(F32)
    q = np.clip(round_half_away(p), -127, 127).astype(np.int8)
    q[d == 0] = 0
    return q.reshape(-1), d


def q4_codes(qs, n, k):
    """Reference nibble order: element 2i = low nibble of byte i, 2i+1 = high."""
    qs = np.asarray(qs, np.uint8).reshape(n, k // 2)
    out = np.empty((n, k), np.int64)
    out[:, 0::2] = qs & 0x0F
    out[:, 1::2] = qs >> 4
    return out


def gemv_q4_exact_f32(x, qs, scales, n, k):
    """Bit-exact emulation of the reference Q4 GEMV for small shapes:
    integer block sums (int64 brute force), scale = f32(d_w * d_a),
    total += f32(isum * scale) sequentially from 0."""
    q, d = q8_quantize(x)
    codes = q4_codes(qs, n, k) - 8
    sc = np.asarray(scales, F32).reshape(n, k // 32)
    nb = k // 32
    out = np.empty(n, F32)
    qa = q.astype(np.int64).reshape(nb, 32)
    for j in range(n):
        total = F32(0.0)
        cj = codes[j].reshape(nb, 32)
        for b in range(nb):
            isum = int(np.dot(cj[b], qa[b]))
            scale = F32(sc[j, b] * d[b])
            total = F32(total + F32(F32(isum) * scale))
        out[j] = total
    return out


def gemv_q8w_exact_f32(x, w, scales, n, k):
    q, d = q8_quantize(x)
    w = np.asarray(w, np.int64).reshape(n, k)
    sc = np.asarray(scales, F32).reshape(n, k // 32)
    nb = k // 32
    out = np.empty(n, F32)
    qa = q.astype(np.int64).reshape(nb, 32)
    for j in range(n):
        total = F32(0.0)
        wj = w[j].reshape(nb, 32)
        for b in range(nb):
            isum = int(np.dot(wj[b], qa[b]))
            total = F32(total + F32(F32(isum) * F32(sc[j, b] * d[b])))
        out[j] = total
    return out


def dequant_q4(qs, scales, n, k):
    codes = q4_codes(qs, n, k).astype(np.float64) - 8.0
    return codes * np.repeat(np.asarray(scales, np.float64).reshape(n, k // 32), 32, axis=1)


def dequant_q8(w, scales, n, k):
    return np.asarray(w, np.float64).reshape(n, k) * np.repeat(
        np.asarray(scales, np.float64).reshape(n, k // 32), 32, axis=1)


def linear64(x, wdeq):
    """x [m,k] -> Q8 activations (float32 decisions) -> float64 product."""
    rows = []
    for r in np.atleast_2d(x):
        q, d = q8_quantize(r)
        a = q.astype(np.float64) * np.repeat(d.astype(np.float64), 32)
        rows.append(wdeq @ a)
    return np.array(rows)


def rmsnorm64(x, w, eps):
    x = np.asarray(x, np.float64)
    ms = np.mean(x * x, axis=-1, keepdims=True)
    return x / np.sqrt(ms + eps) * np.asarray(w, np.float64)


def rope64(x, pos0, theta=500000.0):
    """Rotate-half RoPE on rows of x (row i at position pos0 + i)."""
    x = np.array(x, np.float64)
    hd = x.shape[-1]
    mid = hd // 2
    j = np.arange(mid)
    inv = 1.0 / theta ** (2.0 * j / hd)
    for i in range(x.shape[0]):
        a = (pos0 + i) * inv
        re, im = x[i, :mid].copy(), x[i, mid:].copy()
        x[i, :mid] = re * np.cos(a) - im * np.sin(a)
        x[i, mid:] = re * np.sin(a) + im * np.cos(a)
    return x


def model_forward64(spec_dims, weights, tokens, kv_round=None):
    """Full model in float64 over `tokens` from position 0 (causal).

    spec_dims: (n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, eps)
    weights: dict with embed, final_norm, lm_head (deq), layers:[{norm0, norm1,
    q,k,v,o,gate,up,down (deq [n,k])}].  Returns logits of the last row.
    kv_round: optional function applied to stored K/V (f16 caches)."""
    L, H, nq, nkv, hd, F, eps = spec_dims
    T = len(tokens)
    x = np.asarray(weights["embed"], np.float64)[np.asarray(tokens)]
    rep = nq // nkv
    for lw in weights["layers"]:
        hn = rmsnorm64(x, lw["norm0"], eps)
        q = linear64(hn, lw["q"])
        k = linear64(hn, lw["k"])
        v = linear64(hn, lw["v"])
        ctx = np.zeros((T, nq * hd))
        for g in range(nkv):
            kr = rope64(k[:, g * hd:(g + 1) * hd], 0)
            vr = v[:, g * hd:(g + 1) * hd]
            if kv_round is not None:
                kr, vr = kv_round(kr), kv_round(vr)
            for hr in range(rep):
                h = g * rep + hr
                qr = rope64(q[:, h * hd:(h + 1) * hd], 0)
                s = qr @ kr.T / np.sqrt(hd)
                s = np.where(np.tril(np.ones((T, T), bool)), s, -np.inf)
                p = np.exp(s - s.max(axis=1, keepdims=True))
                p /= p.sum(axis=1, keepdims=True)
                ctx[:, h * hd:(h + 1) * hd] = p @ vr
        h1 = x + linear64(ctx, lw["o"])
        h2 = rmsnorm64(h1, lw["norm1"], eps)
        g_ = linear64(h2, lw["gate"])
        u_ = linear64(h2, lw["up"])
        m = g_ / (1.0 + np.exp(-g_)) * u_
        x = h1 + linear64(m, lw["down"])
    fn = rmsnorm64(x[-1:], weights["final_norm"], eps)
    return linear64(fn, weights["lm_head"])[0]
