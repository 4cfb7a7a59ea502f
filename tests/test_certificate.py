"""The fp16 certificate's error bound, checked numerically on the CPU.

The certified global path and the batched global path nominate candidates with fp16
rows and certify them with a bound eps on |fp16-path score - fp32-path score|. This
test rebuilds each score the way the kernels compute it, bit for bit where the order is
fixed:
  * fp32 Q=1 scan (QF32): lane s of a 16-lane group chains fmaf over floats
    64c + 4s + j (c = 0..D/64-1, j = 0..3), then a 4-step xor tree (8, 4, 2, 1);
  * fp16 Q=1 scan (QF16): the same over halves 128c + 8s + j (j = 0..7), fp32 query;
  * MFMA (batched): fp16 rows times the fp16-rounded query, exact products, fp32
    accumulation in an unspecified order (several orders are tried);
then checks the documented bound on adversarial data (fp16 subnormals, rounding
midpoints, large norms, lopsided queries), and that a certificate that passes always
names exactly the fp32 scan's top-K.
"""
from __future__ import annotations

import numpy as np

U = 2.0 ** -24
F32 = np.float32


def fma32(a, b, c):
    """fp32 fmaf via fp64 (the product of two fp32 values is exact in fp64)."""
    return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(F32)


def tree16(acc):
    """(rows, 16) lane sums -> the 16-lane xor tree of row16_sum, in fp32."""
    v = acc.astype(F32)
    for j in (8, 4, 2, 1):
        v = (v + v[:, np.arange(16) ^ j]).astype(F32)
    return v[:, 0]


def dot_qf32(e, q):
    n, d = e.shape
    acc = np.zeros((n, 16), F32)
    for c in range(d // 64):
        for j in range(4):
            idx = 64 * c + 4 * np.arange(16) + j
            acc = fma32(e[:, idx], q[idx][None, :], acc)
    return tree16(acc)


def dot_qf16(e16, q):
    n, d = e16.shape
    e = e16.astype(F32)
    acc = np.zeros((n, 16), F32)
    for c in range(d // 128):
        for j in range(8):
            idx = 128 * c + 8 * np.arange(16) + j
            acc = fma32(e[:, idx], q[idx][None, :], acc)
    return tree16(acc)


def dot_mfma(e16, q16, order):
    """fp16 x fp16 products (exact in fp32), accumulated in fp32 in a given order."""
    p = (e16.astype(np.float64) * q16.astype(np.float64)).astype(F32)       # exact
    n, d = p.shape
    if order == "exact":
        return p.astype(np.float64).sum(1).astype(F32)
    if order == "serial":
        acc = np.zeros(n, F32)
        for i in range(d):
            acc = (acc + p[:, i]).astype(F32)
        return acc
    # k-steps of 32: each step's 32 products summed exactly, then added to the accumulator
    acc = np.zeros(n, F32)
    for k0 in range(0, d, 32):
        acc = (acc + p[:, k0:k0 + 32].astype(np.float64).sum(1).astype(F32)).astype(F32)
    return acc


def ftz16(h):
    f = h.astype(F32)
    return np.where(np.abs(f) < 2.0 ** -14, F32(0), f)


def norms(e, e16):
    e64 = e.astype(np.float64)
    return (np.sqrt((e64 ** 2).sum(1)).max(), np.sqrt((e16.astype(np.float64) ** 2).sum(1)).max(),
            np.sqrt(((ftz16(e16).astype(np.float64) - e64) ** 2).sum(1)).max())


def eps_certified(e32n, e16n, de, qn, d):
    nq = d / 16 + 4
    gs = nq * U / (1 - nq * U)
    return (de * qn + gs * (e16n + e32n) * qn + U * (e16n + e32n) * qn * (1 + gs)) * 1.01 + 1e-30 * d


def eps_batched(e32n, e16n, de, q, q16, d):
    qn = np.sqrt((q.astype(np.float64) ** 2).sum())
    q16n = np.sqrt((q16.astype(np.float64) ** 2).sum())
    dq = np.sqrt(((ftz16(q16).astype(np.float64) - q.astype(np.float64)) ** 2).sum())
    g_m = 2 * d * U / (1 - d * U)
    nq = d / 16 + 4
    g_s = nq * U / (1 - nq * U)
    e = (e16n * dq + g_m * e16n * q16n + g_s * e32n * qn +
         U * (e16n * q16n * (1 + g_m) + e32n * qn * (1 + g_s)))
    return (e + de * qn) * 1.01 + 1e-30 * d


def fused(dot, w):
    return (dot.astype(F32) * w).astype(F32)


def make_cases(rng, n=600, d=256):
    e = rng.standard_normal((n, d)).astype(F32)
    e /= np.linalg.norm(e, axis=1, keepdims=True)
    cases = [("unit rows", e.copy(), None)]
    sub = e.copy()
    sub[:, ::3] *= F32(3e-5)                                     # many fp16 subnormals
    cases.append(("subnormal elements", sub, None))
    mid = e.copy()
    # elements at fp16 rounding midpoints (ties to even)
    h = mid.astype(np.float16).astype(F32)
    up = np.nextafter(mid.astype(np.float16), np.float16(np.inf)).astype(F32)
    mid[:, ::2] = ((h + up) / 2).astype(F32)[:, ::2]
    cases.append(("rounding midpoints", mid, None))
    cases.append(("large norms", (e * F32(900.0)).astype(F32), None))
    q = rng.standard_normal(d).astype(F32)
    q[: d // 2] *= F32(1e-4)
    cases.append(("lopsided query", e.copy(), q / np.linalg.norm(q)))
    return cases


def test_bound_covers_every_row():
    rng = np.random.default_rng(7)
    for name, e, q in make_cases(rng):
        d = e.shape[1]
        if q is None:
            q = e[3] + F32(0.01) * rng.standard_normal(d).astype(F32)
        q = q.astype(F32)
        e16 = e.astype(np.float16)
        q16 = q.astype(np.float16)
        e32n, e16n, de = norms(e, e16)
        qn = float(np.sqrt((q.astype(np.float64) ** 2).sum()))
        w = np.exp(-0.1 * rng.uniform(0, 30, size=e.shape[0])).astype(F32)
        s32 = fused(dot_qf32(e, q), w).astype(np.float64)
        s16 = fused(dot_qf16(e16, q), w).astype(np.float64)
        eps_c = eps_certified(e32n, e16n, de, qn, d)
        assert np.abs(s16 - s32).max() <= eps_c, (name, np.abs(s16 - s32).max(), eps_c)
        eps_b = eps_batched(e32n, e16n, de, q, q16, d)
        for order in ("exact", "serial", "ksteps"):
            sm = fused(dot_mfma(e16, q16, order), w).astype(np.float64)
            assert np.abs(sm - s32).max() <= eps_b, (name, order, np.abs(sm - s32).max(), eps_b)
        # the bound is not vacuous: within a small factor of the largest error seen
        assert eps_c <= 200 * max(np.abs(s16 - s32).max(), 1e-12), (name, eps_c)


def keys(scores):
    """Ascending (score desc, id asc) order."""
    return np.lexsort((np.arange(len(scores)), -scores))


def test_certificate_names_the_fp32_top_k():
    rng = np.random.default_rng(11)
    n, d, k, c = 3000, 256, 10, 16
    certified = uncertified = 0
    for trial in range(40):
        e = rng.standard_normal((n, d)).astype(F32)
        e /= np.linalg.norm(e, axis=1, keepdims=True)
        if trial % 4 == 0:                                   # planted near-ties at the cut
            e[100:130] = e[7] + F32(1e-5) * rng.standard_normal((30, d)).astype(F32)
        q = (e[7] + F32(0.2) * rng.standard_normal(d).astype(F32)).astype(F32)
        e16 = e.astype(np.float16)
        e32n, e16n, de = norms(e, e16)
        qn = float(np.sqrt((q.astype(np.float64) ** 2).sum()))
        w = np.exp(-0.1 * rng.uniform(0, 20, size=n)).astype(F32)
        if trial % 4 == 0:
            w[100:130] = w[7] = F32(1.0)
        s32 = fused(dot_qf32(e, q), w)
        s16 = fused(dot_qf16(e16, q), w)
        cand = keys(s16)[:c]
        exact = cand[keys(s32[cand])]
        eps = eps_certified(e32n, e16n, de, qn, d)
        ok = float(s32[exact[k - 1]]) > float(s16[cand[c - 1]]) + eps
        if ok:
            certified += 1
            np.testing.assert_array_equal(exact[:k], keys(s32)[:k])
        else:
            uncertified += 1
    assert certified >= 25 and uncertified >= 1, (certified, uncertified)
