"""The certificates' error bounds (fp16 and int8 candidate scans), checked numerically
on the CPU.

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


# ---- the int8 candidate scan (k_scan8) ----------------------------------------------------
# Row r is kept as bytes v in [-127, 127] and a scale s = fl(max|e| / 127). The query is split
# into two int8 parts, q = s_hi q_hi + s_lo q_lo + r2, and the MFMA sums v . q_hi and v . q_lo
# exactly in int32; the scan's dot is fmaf(s_lo, lo, s_hi * hi) * s. Its key is the upper bound
# U = fl(w * X), X = fmaf(|q|_up, c_r, dot8) + tau raised by max(|X| 2^-20, 1e-35), with
# tau = (max|e| + max c) (|r2| + 3.1 u (|s_hi q_hi| + |s_lo q_lo|)); the interval BFS uses
# fin = fl(w * dot8) with half-width eps8 = (|q| max c + 4u |q| (max|e| + max c)) * 1.01 + tau
# + 1e-30 d.

def up32(x):
    """fp32 values >= x (float64 array)."""
    f = np.asarray(x, np.float64).astype(F32)
    return np.where(f.astype(np.float64) < x, np.nextafter(f, F32(np.inf)), f).astype(F32)


def quantize_i8(e):
    """The int8 copy of rows e: bytes, scales, per-row bounds c (quantize_row_i8)."""
    d = e.shape[1]
    s = (np.abs(e).max(1).astype(F32) / F32(127)).astype(F32)
    with np.errstate(divide="ignore", invalid="ignore"):
        t = np.where(s[:, None] > 0, np.rint((e / s[:, None]).astype(F32)), F32(0))
    v = np.clip(t, -127, 127).astype(np.int8)
    e64, eh = e.astype(np.float64), s[:, None].astype(np.float64) * v.astype(np.float64)
    nu = (d / 16 + 6) * U
    g = nu / (1 - nu)
    c = (np.sqrt(((eh - e64) ** 2).sum(1)) + g * (np.sqrt((eh ** 2).sum(1)) + np.sqrt((e64 ** 2).sum(1)))) * (1 + 1e-9)
    return v, s, up32(c)


def split_query(q):
    """k_scan8's query split: (s_hi, s_lo, q_hi, q_lo, |r2|, |s_hi q_hi|, |s_lo q_lo|)."""
    s_hi = F32(np.abs(q).max()) / F32(127)
    qh = np.clip(np.rint((q / s_hi).astype(F32)), -127, 127) if s_hi > 0 else np.zeros_like(q)
    r1 = fma32(np.full_like(q, -s_hi), qh.astype(F32), q)
    s_lo = F32(np.abs(r1).max()) / F32(127)
    ql = np.clip(np.rint((r1 / s_lo).astype(F32)), -127, 127) if s_lo > 0 else np.zeros_like(q)
    hq, lq = np.float64(s_hi) * qh.astype(np.float64), np.float64(s_lo) * ql.astype(np.float64)
    r2 = q.astype(np.float64) - hq - lq
    return (s_hi, s_lo, qh.astype(np.int64), ql.astype(np.int64), float(np.sqrt((r2 ** 2).sum())),
            float(np.sqrt((hq ** 2).sum())), float(np.sqrt((lq ** 2).sum())))


def dot_mfma8(v, s, q):
    s_hi, s_lo, qh, ql = split_query(q)[:4]
    hi = (v.astype(np.int64) @ qh).astype(F32)                # exact int32 sums, exact in fp32
    lo = (v.astype(np.int64) @ ql).astype(F32)
    return (fma32(np.full_like(lo, s_lo), lo, (s_hi * hi).astype(F32)) * s).astype(F32)


def tau_i8(c, e, q):
    _, _, _, _, r2, nh, nl = split_query(q)
    en = float(up32(np.sqrt((e.astype(np.float64) ** 2).sum(1)).max())) + float(c.max())
    return float(up32(en * (r2 + 3.1 * U * (nh + nl)) * (1 + 1e-6) + 1e-30))


def upper_i8(dot8, c, q, w, tau):
    qn_up = up32(np.sqrt((q.astype(np.float64) ** 2).sum()) * (1 + 1e-12))
    x = (fma32(np.full_like(dot8, qn_up), c, dot8) + F32(tau)).astype(F32)
    x = (x + np.maximum(np.abs(x) * F32(2.0 ** -20), F32(1e-35))).astype(F32)
    return fused(x, w)


def eps_i8(c, e, q, tau):
    d = e.shape[1]
    qn = float(np.sqrt((q.astype(np.float64) ** 2).sum()))
    en = float(up32(np.sqrt((e.astype(np.float64) ** 2).sum(1)).max()))
    cm = float(c.max())
    return (cm * qn + 4 * U * (en + cm) * qn) * 1.01 + tau + 1e-30 * d


def make_cases_i8(rng, n=600, d=768):
    e = rng.standard_normal((n, d)).astype(F32)
    e /= np.linalg.norm(e, axis=1, keepdims=True)
    cases = [("unit rows", e.copy())]
    spike = e.copy()
    spike[::2, 5] = F32(0.9)                                     # one large element: coarse scale
    cases.append(("spiked rows", (spike / np.linalg.norm(spike, axis=1, keepdims=True)).astype(F32)))
    mid = e.copy()
    s = (np.abs(mid).max(1) / F32(127)).astype(F32)
    k = np.rint(mid / s[:, None])
    half = ((k[:, 1::2] + np.sign(k[:, 1::2]) * 0.5) * s[:, None]).astype(F32)     # int8 midpoints
    mid[:, 1::2] = np.clip(half, -np.abs(mid).max(1, keepdims=True), np.abs(mid).max(1, keepdims=True))
    cases.append(("rounding midpoints", mid))
    cases.append(("large norms", (e * F32(900.0)).astype(F32)))
    tiny = (e * F32(1e-30)).astype(F32)
    cases.append(("tiny rows", tiny))
    z = e.copy()
    z[::7] = 0.0
    cases.append(("zero rows", z))
    return cases


def test_int8_upper_bound_covers_every_row():
    rng = np.random.default_rng(17)
    for name, e in make_cases_i8(rng):
        d = e.shape[1]
        for qi, q in enumerate((e[3] + F32(0.01) * rng.standard_normal(d).astype(F32),
                                rng.standard_normal(d).astype(F32) * np.where(np.arange(d) < d // 2, F32(1e-4), F32(1)))):
            q = q.astype(F32)
            v, s, c = quantize_i8(e)
            w = np.exp(-0.1 * rng.uniform(0, 30, size=e.shape[0])).astype(F32)
            s32 = fused(dot_qf32(e, q), w).astype(np.float64)
            d8 = dot_mfma8(v, s, q)
            tau = tau_i8(c, e, q)
            s8 = fused(d8, w).astype(np.float64)
            up = upper_i8(d8, c, q, w, tau).astype(np.float64)
            assert (up >= s32).all(), (name, qi, float((s32 - up).max()))
            eps = eps_i8(c, e, q, tau)
            assert np.abs(s8 - s32).max() <= eps, (name, qi, np.abs(s8 - s32).max(), eps)
            # the bounds are not vacuous: within a small factor of the errors seen
            gap = np.abs(s8 - s32).max()
            if name != "tiny rows":                          # there the 1e-30 d floor dominates
                assert eps <= 60 * gap, (name, qi, eps, gap)


def test_int8_quantization_error_is_what_c_states():
    """c_r is the row's residual norm plus rounding terms of relative size ~(d/16) u,
    and the byte codes round to nearest (ties to even) within [-127, 127]."""
    rng = np.random.default_rng(19)
    e = rng.standard_normal((200, 512)).astype(F32)
    v, s, c = quantize_i8(e)
    resid = np.sqrt(((s[:, None].astype(np.float64) * v - e.astype(np.float64)) ** 2).sum(1))
    assert (c >= resid).all() and (c <= resid * 1.01 + 1e-4).all()
    assert np.abs(v).max() == 127 and (np.abs(v) == 127).sum(1).min() >= 1      # every row uses its range
    assert (np.abs(e / s[:, None] - v) <= 0.5 + 1e-6).all()
    assert np.array_equal(np.rint(np.array([0.5, 1.5, 2.5, -0.5], F32)), np.array([0, 2, 2, 0], F32))


def workgroup_candidates(up, n_wg=8, block=64, kw=16, cands=64):
    """k_scan8 + k_cert_bfs candidate selection: rows dealt to n_wg workgroups in blocks of
    64 consecutive ids, each keeps its kw best keys; the cands best of their union, and the
    bound key above which every other row lies (the cands-th candidate's, or the smallest
    kw-th key of a full list)."""
    order = keys(up)
    wg = (np.arange(len(up)) // block) % n_wg
    kept, last = [], []
    for b in range(n_wg):
        mine = order[wg[order] == b]
        kept.extend(mine[:kw])
        if len(mine) > kw:
            last.append(mine[kw - 1])
    kept = np.array(kept)
    cand = kept[keys(up[kept])][:cands]
    # key order: a smaller (score desc, id asc) rank is a smaller key
    rank = np.empty(len(up), np.int64)
    rank[order] = np.arange(len(up))
    bound = [cand[-1]] if len(cand) == cands else []
    bound += last
    return cand, (min(bound, key=lambda r: rank[r]) if bound else None)


def test_int8_certificate_names_the_fp32_top_k():
    rng = np.random.default_rng(23)
    n, d, k, cands = 3000, 512, 10, 64
    certified = uncertified = 0
    for trial in range(30):
        e = rng.standard_normal((n, d)).astype(F32)
        e /= np.linalg.norm(e, axis=1, keepdims=True)
        if trial % 4 == 0:                                   # planted near-ties at the cut
            e[100:180] = e[7] + F32(1e-5) * rng.standard_normal((80, d)).astype(F32)
        if trial % 4 == 1:                                   # 40 near-copies in one workgroup
            e[576:616] = e[7] + F32(0.05) * rng.standard_normal((40, d)).astype(F32)
        q = (e[7] + F32(0.2) * rng.standard_normal(d).astype(F32)).astype(F32)
        v, s, c = quantize_i8(e)
        w = np.exp(-0.1 * rng.uniform(0, 20, size=n)).astype(F32)
        if trial % 4 == 0:
            w[100:180] = w[7] = F32(1.0)
        s32 = fused(dot_qf32(e, q), w)
        up = upper_i8(dot_mfma8(v, s, q), c, q, w, tau_i8(c, e, q))
        cand, bnd = workgroup_candidates(up)
        exact = cand[keys(s32[cand])]
        ok = bnd is None or float(s32[exact[k - 1]]) > float(up[bnd])
        if ok:
            certified += 1
            np.testing.assert_array_equal(exact[:k], keys(s32)[:k])
        else:
            uncertified += 1
    assert certified >= 20 and uncertified >= 1, (certified, uncertified)


def rerank_dot(x, y):
    """k_knn_rerank's fp32 dot (batch.hip): lane l sums elements 4 l + 256 j .. + 3 in one fmaf
    chain (j ascending), then lane 0's view of the 64-lane xor butterfly (32, 16, .., 1).
    fmaf is taken as one rounding of the float64 value a * b + c."""
    d = x.size
    lanes = np.zeros(64, F32)
    for lane in range(64):
        acc = F32(0)
        for j in range((d + 255) // 256):
            i = 256 * j + 4 * lane
            if i < d:
                for c in range(4):
                    acc = F32(np.float64(x[i + c]) * np.float64(y[i + c]) + np.float64(acc))
        lanes[lane] = acc
    for m in (32, 16, 8, 4, 2, 1):
        lanes = (lanes + lanes[np.arange(64) ^ m]).astype(F32)
    return lanes[0]


def test_rerank_dot_within_its_error_bound():
    """The k-NN certificate charges the rescoring gamma_n |x||y| with n = 4 ceil(d/256) + 6
    (the longest per-lane fmaf chain plus the six butterfly levels); the emulated kernel
    arithmetic stays within gamma_n sum |x_i y_i| on rows built for cancellation, at every
    supported width (384 leaves the upper 32 lanes with one 4-term piece)."""
    rng = np.random.default_rng(11)
    for d in (256, 384, 512, 768):
        n = 4 * ((d + 255) // 256) + 6
        g = n * U / (1 - n * U)
        worst = 0.0
        for t in range(40):
            x = rng.standard_normal(d).astype(F32)
            y = rng.standard_normal(d).astype(F32)
            if t % 2:
                y = (x * F32(1 + 1e-3) + rng.standard_normal(d).astype(F32) * F32(1e-4)).astype(F32)
                y[::2] *= F32(-1)                    # large terms of both signs: heavy cancellation
            exact = float(np.dot(x.astype(np.float64), y.astype(np.float64)))
            got = float(rerank_dot(x, y))
            scale = float(np.abs(x.astype(np.float64) * y.astype(np.float64)).sum())
            assert abs(got - exact) <= g * scale, (d, t, got, exact)
            worst = max(worst, abs(got - exact) / (g * scale))
        assert worst > 0.0                           # the emulation rounds somewhere
