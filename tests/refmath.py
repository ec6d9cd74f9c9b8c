"""Float64 textbook definitions used to pin the oracle (and, through it, the HIP path).

These are the mathematical definitions of the operations -- softmax attention, RMS
normalisation, rotary embedding as a rotation by angle pos*theta^(-2i/R) -- written
independently of the oracle's float32 step order.  They check the oracle up to rounding.
"""
from __future__ import annotations

import numpy as np


def rms_norm_heads(x, w, n_heads, head_size, eps):
    x = np.asarray(x, np.float64).reshape(n_heads, head_size)
    r = 1.0 / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps)
    return (x * r * np.asarray(w, np.float64)[None, :]).reshape(-1)


def rope_angles(rope_dim, pos, theta, linear_freq_scale=1.0, float32_angle=True):
    """Angle pos * theta^(-2i/R).  RoPE.java:83-101 forms frequency and angle in float32
    (`float angle = pos * freq`); float32_angle=True applies that rounding, which matters at
    large pos (the angle error is ~pos * 2^-24 rad)."""
    i = np.arange(rope_dim // 2, dtype=np.float64)
    freq = theta ** (-2.0 * i / rope_dim)
    if linear_freq_scale > 1.0:
        freq = freq / linear_freq_scale
    if float32_angle:
        return (np.float32(pos) * freq.astype(np.float32)).astype(np.float64)
    return pos * freq


def rope_rotate(x, n_heads, head_size, rope_dim, rope_type, angles):
    """Rotate each (x0, x1) pair by `angles` (NORMAL pairs (2i,2i+1), NEOX pairs (i,i+R/2))."""
    x = np.asarray(x, np.float64).reshape(n_heads, head_size).copy()
    half = rope_dim // 2
    c, s = np.cos(angles), np.sin(angles)
    if rope_type == 0:
        i0, i1 = np.arange(half) * 2, np.arange(half) * 2 + 1
    else:
        i0, i1 = np.arange(half), np.arange(half) + half
    a, b = x[:, i0].copy(), x[:, i1].copy()
    x[:, i0] = a * c - b * s
    x[:, i1] = a * s + b * c
    return x.reshape(-1)


def attention(q, kcache, vcache, n_heads, n_kv_heads, head_size, start, pos, scale,
              softcap=0.0, sinks=None):
    """out_h = softmax_t(s_t) . V_t over t in [start, pos], s_t = scale * q_h.K_t (soft-capped
    as c*tanh(s/c) when softcap > 0); kv head of query head h is h // (Hq/Hkv).  With sinks,
    head h's softmax has one more logit sinks[h] that takes no value (a denominator term)."""
    q = np.asarray(q, np.float64).reshape(n_heads, head_size)
    kv_dim = n_kv_heads * head_size
    K = np.asarray(kcache, np.float64).reshape(-1, kv_dim)[start:pos + 1]
    V = np.asarray(vcache, np.float64).reshape(-1, kv_dim)[start:pos + 1]
    g = n_heads // n_kv_heads
    out = np.zeros((n_heads, head_size))
    for h in range(n_heads):
        kh = h // g
        Kh = K[:, kh * head_size:(kh + 1) * head_size]
        Vh = V[:, kh * head_size:(kh + 1) * head_size]
        s = Kh @ q[h] * scale
        if softcap > 0:
            s = softcap * np.tanh(s / softcap)
        if sinks is None:
            p = np.exp(s - s.max())
            p /= p.sum()
        else:
            mx = max(s.max(), float(sinks[h]))
            p = np.exp(s - mx)
            p /= p.sum() + np.exp(float(sinks[h]) - mx)
        out[h] = p @ Vh
    return out.reshape(-1)


def assert_close(got, want, atol=1e-4, rtol=1e-3, what=""):
    """The parity bar of the path: |got - want| <= atol + rtol*|want| elementwise."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    err = np.abs(got - want)
    bound = atol + rtol * np.abs(want)
    bad = err > bound
    if bad.any():
        i = int(np.argmax(err - bound))
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{err.size} elements out of tolerance "
            f"(atol={atol}, rtol={rtol}); worst idx {i}: got {got.flat[i]!r} want "
            f"{want.flat[i]!r}; max abs err {err.max():.3e}")
