"""CPU check of the arithmetic behind the int8-MFMA scores of the Q8_0 decode kernel.

Per (query head, 32-dim block) the kernel holds the scaled query as three int8 parts,
q = s*(Q1 + (Q2 + Q3/F)/F) with s = max|q|/127 and F = 254.  It takes three exact integer dot
products with the block's K quants and forms sum_b ks_b*s_b*(D1 + (D2 + D3/F)/F) in fp32.  This
test restates that arithmetic in numpy with the kernel's fp32 rounding steps.  It checks it
against float64 dot products of the same values (the dequantised cache of KVCache.dotK in
Q8_0 mode, KVCache.java:187-195):
- the parts stay in int8 range;
- the reconstruction error is below 2^-22 of the block maximum;
- the score error is at the fp32 rounding level of a 128-term dot product.
Zero blocks, single dominant elements and 1e-6..1e4 magnitudes are included."""
import numpy as np

F32 = np.float32
F = F32(254.0)
INV_F = F32(1.0) / F


def _parts(x):
    """The kernel's split of one 32-value block (q8_query_split): fp32 steps, rint ties to even."""
    mx = np.max(np.abs(x)).astype(F32)
    s = F32(mx / F32(127.0))
    inv = F32(1.0) / s if s != 0 else F32(0.0)
    v = (x * inv).astype(F32)
    q1 = np.clip(np.rint(v), -127, 127).astype(F32)
    r1 = ((v - q1) * F).astype(F32)
    q2 = np.clip(np.rint(r1), -127, 127).astype(F32)
    r2 = ((r1 - q2) * F).astype(F32)
    q3 = np.clip(np.rint(r2), -127, 127).astype(F32)
    return s, q1.astype(np.int32), q2.astype(np.int32), q3.astype(np.int32)


def _score(q, kq, ks):
    """Score of one key as the kernel forms it (consume: f per block, fma with ks*s)."""
    acc = F32(0.0)
    for b in range(q.size // 32):
        s, q1, q2, q3 = _parts(q[32 * b:32 * b + 32])
        k = kq[32 * b:32 * b + 32].astype(np.int32)
        d1, d2, d3 = (int(np.dot(p, k)) for p in (q1, q2, q3))
        f = F32(F32(d1) + F32(F32(F32(d2) + F32(F32(d3) * INV_F)) * INV_F))
        acc = F32(f * F32(ks[b] * s) + acc)
    return acc


def _blocks(rng, n, scale):
    x = (rng.standard_normal(n) * scale).astype(F32)
    return x


def test_parts_in_range_and_reconstruction():
    rng = np.random.default_rng(11)
    worst = 0.0
    for t in range(400):
        x = _blocks(rng, 32, 10.0 ** rng.uniform(-6, 4))
        if t % 5 == 0:
            x[rng.integers(32)] *= F32(300.0)          # one dominant element
        if t % 7 == 0:
            x[:] = 0                                   # all-zero block
        s, q1, q2, q3 = _parts(x)
        for p in (q1, q2, q3):
            assert p.min() >= -127 and p.max() <= 127
        rec = float(s) * (q1 + (q2 + q3 / 254.0) / 254.0)
        mx = float(np.max(np.abs(x)))
        if mx == 0.0:
            assert s == 0 and not q1.any() and not q2.any() and not q3.any()
            continue
        worst = max(worst, float(np.max(np.abs(rec - x.astype(np.float64)))) / mx)
    assert worst < 2.0 ** -22, worst


def test_scores_match_float64_dot_products():
    rng = np.random.default_rng(12)
    for t in range(300):
        D = int(rng.choice([64, 128, 256]))
        q = _blocks(rng, D, 10.0 ** rng.uniform(-3, 2))
        if t % 4 == 0:
            q[32:64] = 0
        if t % 6 == 0:
            q[rng.integers(D)] *= F32(50.0)
        kq = rng.integers(-128, 128, D).astype(np.int8)
        ks = (rng.uniform(0.1, 2.0, D // 32) / 127).astype(F32)
        got = float(_score(q, kq, ks))
        kf = (kq.astype(np.float64).reshape(-1, 32) * ks.astype(np.float64)[:, None]).reshape(-1)
        exact = float(np.dot(q.astype(np.float64), kf))
        mag = float(np.dot(np.abs(q.astype(np.float64)), np.abs(kf)))
        assert abs(got - exact) <= 2e-6 * mag + 1e-30, (t, got, exact, mag)
