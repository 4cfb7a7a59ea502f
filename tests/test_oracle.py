"""Pin the CPU oracle before it is trusted as the parity reference.

Each oracle function is checked against something independent of its own
formula: the reference's own code (oracle/_ref, golden fixtures), numpy /
scipy computations, closed forms, and hand-derived small cases chosen so that
a plausible mistake (wrong parent order, unclamped age, dropped decay, tie
rule reversed, ...) fails.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest
import scipy.sparse as sp
from scipy.sparse.csgraph import shortest_path

import oracle

FLT_MAX = float(np.finfo(np.float32).max)


# ---------------------------------------------------------------- episode CSR
def test_episode_csr_matches_golden(golden):
    z = np.load(golden / "episode_csr.npz")
    for name in ("kids30", "shuffled", "single", "one_node"):
        off, mem = oracle.episode_csr(z[f"{name}_ids"])
        assert len(off) - 1 == int(z[f"{name}_num"]), name
        np.testing.assert_array_equal(off, z[f"{name}_offsets"], err_msg=name)
        np.testing.assert_array_equal(mem, z[f"{name}_members"], err_msg=name)


@pytest.mark.skipif(oracle.ref is None, reason="oracle/_ref not built (reference tree absent)")
def test_episode_csr_matches_reference_build(rng):
    for n, n_ep in [(1, 1), (10, 3), (1000, 50), (5000, 4000)]:
        ids = rng.integers(0, n_ep, size=n).astype(np.int32)
        ne = C.c_int32()
        oracle.ref.ref_build_episode_csr(C.c_void_p(ids.ctypes.data), n, C.byref(ne), None, None)
        off_r = np.zeros(ne.value + 1, np.int32)
        mem_r = np.zeros(n, np.int32)
        oracle.ref.ref_build_episode_csr(C.c_void_p(ids.ctypes.data), n, C.byref(ne),
                                         C.c_void_p(off_r.ctypes.data), C.c_void_p(mem_r.ctypes.data))
        off, mem = oracle.episode_csr(ids)
        np.testing.assert_array_equal(off, off_r)
        np.testing.assert_array_equal(mem, mem_r)


def test_episode_csr_closed_form(rng):
    ids = rng.integers(0, 40, size=777).astype(np.int32)
    off, mem = oracle.episode_csr(ids)
    np.testing.assert_array_equal(np.diff(off), np.bincount(ids, minlength=len(off) - 1))
    # members = stable argsort by episode id (ascending node id inside an episode)
    np.testing.assert_array_equal(mem, np.argsort(ids, kind="stable"))


# ---------------------------------------------------------------- fp16 rounding
def test_float_to_half_matches_numpy_rne(rng):
    specials = np.array([0.0, -0.0, 1.0, 65504.0, 65519.99, 65520.0, 1e-8, 2 ** -24, 2 ** -25,
                         2 ** -25 * 1.0000001, 3 * 2 ** -26, 5.96e-8, 6.1e-5, 1 + 2 ** -11, 1 + 3 * 2 ** -11,
                         np.inf, -np.inf], np.float32)
    bits = rng.integers(0, 2 ** 32, size=200000, dtype=np.uint64).astype(np.uint32)
    rand = bits.view(np.float32)
    rand = rand[np.isfinite(rand)]
    x = np.concatenate([specials, rand, rng.standard_normal(100000).astype(np.float32) * 0.05])
    got = oracle.to_f16_bits(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, want)


# ---------------------------------------------------------------- scores
def _tiny_graph(rng, n=300, d=96):
    emb = rng.standard_normal((n, d)).astype(np.float32)
    emb /= np.linalg.norm(emb, axis=1, keepdims=True)
    mods = rng.integers(0, 3, size=n).astype(np.int32)
    ts = rng.uniform(0, 600, size=n).astype(np.float32)
    return emb, mods, ts


def test_scores_vs_numpy_fp64(rng):
    emb, mods, ts = _tiny_graph(rng)
    g = oracle.make_graph(emb, mods, ts)
    q = emb[7]
    t_q, lam = np.float32(600.0), np.float32(0.1)
    fin, scale = oracle.scores(g, q, float(t_q), float(lam))
    age = np.maximum(np.float32(0), t_q - ts).astype(np.float64)     # fp32 age, as the kernel
    want = (emb.astype(np.float64) @ q.astype(np.float64)) * np.exp(-np.float64(lam) * age)
    np.testing.assert_allclose(fin, want, rtol=1e-12, atol=1e-15)
    np.testing.assert_allclose(scale, np.abs(emb.astype(np.float64) * q).sum(1) * np.exp(-np.float64(lam) * age),
                               rtol=1e-12)


def test_scores_decay_closed_forms(rng):
    emb, mods, ts = _tiny_graph(rng, n=5, d=8)
    ts[:] = [600.0, 610.0, 590.0, 0.0, 600.0]     # same time, future (clamped), -10 s, -600 s
    g = oracle.make_graph(emb, mods, ts)
    q = emb[0]
    dots = emb.astype(np.float64) @ q.astype(np.float64)
    fin, _ = oracle.scores(g, q, 600.0, 0.1)
    assert fin[0] == pytest.approx(dots[0], rel=1e-15)              # age 0 -> weight 1
    assert fin[1] == pytest.approx(dots[1], rel=1e-15)              # future memory: age clamped to 0
    lam = np.float64(np.float32(0.1))                               # lambda is an fp32 parameter
    assert fin[2] == pytest.approx(dots[2] * np.exp(-lam * 10.0), rel=1e-12)
    assert fin[3] == pytest.approx(dots[3] * np.exp(-lam * 600.0), rel=1e-12)
    fin0, _ = oracle.scores(g, q, 600.0, 0.0)                        # lambda 0: plain cosine
    np.testing.assert_allclose(fin0, dots, rtol=1e-15)


def test_scores_modality_filter(rng):
    emb, mods, ts = _tiny_graph(rng, n=64, d=16)
    g = oracle.make_graph(emb, mods, ts)
    fin, scale = oracle.scores(g, emb[0], 600.0, 0.1, mod_filter=2)
    assert np.all(fin[mods != 2] == -FLT_MAX)
    assert np.all(scale[mods != 2] == 0.0)
    assert np.all(fin[mods == 2] > -2.0)


def test_scores_fp16_rows(rng):
    emb, mods, ts = _tiny_graph(rng)
    g = oracle.make_graph(emb, mods, ts, fp16=True)
    q = emb[3]
    fin, _ = oracle.scores(g, q, 600.0, 0.1)
    e16 = emb.astype(np.float16).astype(np.float64)
    age = np.maximum(np.float32(0), np.float32(600.0) - ts).astype(np.float64)
    want = (e16 @ q.astype(np.float64)) * np.exp(-np.float64(np.float32(0.1)) * age)
    np.testing.assert_allclose(fin, want, rtol=1e-12, atol=1e-15)


# ---------------------------------------------------------------- top-K
def test_topk_tie_rule_matches_lexsort(rng):
    vals = rng.integers(0, 20, size=5000).astype(np.float64) / 7.0   # many exact ties
    vals[[5, 9, 4000]] = -FLT_MAX
    for k in (1, 10, 64, 5000):
        idx, val = oracle.topk(vals, k)
        want = np.lexsort((np.arange(len(vals)), -vals))[:k]
        np.testing.assert_array_equal(idx, want)
        np.testing.assert_array_equal(val, vals[want])
    idx, _ = oracle.topk(vals[:3], 10)                                 # K > N -> N seeds
    assert len(idx) == 3


def test_topk_signed_zero_equal():
    vals = np.array([0.0, -0.0, 0.0, -0.0], np.float64)
    idx, _ = oracle.topk(vals, 4)
    np.testing.assert_array_equal(idx, [0, 1, 2, 3])


# ---------------------------------------------------------------- BFS
def _csr(n, edges):
    adj = [set() for _ in range(n)]
    for a, b in edges:
        if a != b:
            adj[a].add(b)
            adj[b].add(a)
    row = np.zeros(n + 1, np.int32)
    for i in range(n):
        row[i + 1] = row[i] + len(adj[i])
    col = np.concatenate([np.array(sorted(a), np.int32) for a in adj]) if row[-1] else np.zeros(0, np.int32)
    return row, col


def test_bfs_levels_match_shortest_paths(rng):
    n = 400
    edges = rng.integers(0, n, size=(900, 2))
    row, col = _csr(n, edges)
    fin = rng.standard_normal(n)
    seeds = rng.choice(n, size=7, replace=False).astype(np.int32)
    m = sp.csr_matrix((np.ones(len(col)), col, row), shape=(n, n))
    dist = shortest_path(m, unweighted=True, indices=seeds).min(axis=0)
    for hops in (0, 1, 2, 3):
        r = oracle.bfs(row, col, fin, seeds, fin[seeds], hops, 0.5)
        want = np.where(dist <= hops, dist, -1).astype(np.int32)
        np.testing.assert_array_equal(r["hop_by_node"], want)
        assert sorted(r["ids"]) == sorted(np.nonzero(want >= 0)[0])
        np.testing.assert_array_equal(r["hops"], want[r["ids"]])


def test_bfs_first_discoverer_in_seed_order():
    # seeds [1, 0]; node 2 is a neighbour of both. Sequential BFS visits seed 1
    # first, so 1 is the parent: score = max(s1*d, f2*0.8), not max(s0*d, ...).
    row, col = _csr(5, [(0, 2), (1, 2), (2, 3), (0, 4)])
    fin = np.array([0.9, 0.5, 0.1, 0.05, 0.02])
    r = oracle.bfs(row, col, fin, np.array([1, 0], np.int32), np.array([0.5, 0.9]), 2, 0.5)
    order = list(r["ids"])
    assert order == [1, 0, 2, 4, 3]          # frontier order: seed 1's row first, then seed 0's
    sc = dict(zip(order, r["scores"]))
    assert sc[2] == pytest.approx(max(0.5 * 0.5, 0.1 * 0.8))      # parent 1 (0.25), not 0 (0.45)
    assert sc[4] == pytest.approx(max(0.9 * 0.5, 0.02 * 0.8))
    assert sc[3] == pytest.approx(max(sc[2] * 0.5, 0.05 * 0.8))
    par = dict(zip(order, r["parent"]))
    assert order[par[2]] == 1 and order[par[3]] == 2


def test_bfs_own_score_wins_when_larger():
    row, col = _csr(3, [(0, 1), (1, 2)])
    fin = np.array([0.2, 0.9, 0.95])
    r = oracle.bfs(row, col, fin, np.array([0], np.int32), np.array([0.2]), 2, 0.5)
    sc = dict(zip(r["ids"], r["scores"]))
    assert sc[1] == pytest.approx(0.9 * 0.8) and sc[2] == pytest.approx(0.95 * 0.8)


def test_bfs_scales_hand_chains():
    """bfs_scales on hand graphs: a seed keeps its own scale; a child takes
    max(|decay| * parent's, 0.8 * own). The chain 3 -> 1 -> 0 -> 2 is visited out of id
    order, so a parent looked up by id instead of visit position fails; the branch
    4 -> {5, 6} checks that siblings share one parent scale."""
    row, col = _csr(7, [(3, 1), (1, 0), (0, 2), (4, 5), (4, 6)])
    fin = np.array([0.1, 0.2, 0.05, 0.9, 0.6, 0.3, 0.01])
    r = oracle.bfs(row, col, fin, np.array([3, 4], np.int32), np.array([0.9, 0.6]), 3, 0.5)
    scale = np.array([2.0, 1.0, 0.5, 3.0, 0.25, 4.0, 0.1])
    got = dict(zip(r["ids"].tolist(), oracle.bfs_scales(r, scale, 0.5).tolist()))
    want = {3: 3.0, 4: 0.25}
    want[1] = max(0.5 * want[3], 0.8 * 1.0)          # 1.5
    want[5] = max(0.5 * want[4], 0.8 * 4.0)          # 3.2: own scale wins
    want[6] = max(0.5 * want[4], 0.8 * 0.1)          # 0.125: the parent's wins
    want[0] = max(0.5 * want[1], 0.8 * 2.0)          # 1.6
    want[2] = max(0.5 * want[0], 0.8 * 0.5)          # 0.8
    assert got == pytest.approx(want)
    # a negative decay scales by its magnitude
    neg = dict(zip(r["ids"].tolist(), oracle.bfs_scales(r, scale, -0.5).tolist()))
    assert neg == pytest.approx(want)


def test_result_scales_seeds_are_the_row_scale(rng):
    """result_scales of a whole query: every result has a scale; a seed's is the row scale
    w * sum_d |e_d q_d| (numpy, fp64), and no node's is below 0.8 times its own."""
    g = _query_graph(rng)
    q = g.embeddings[3]
    cfg = oracle.config(8, 2, 1e-3, 0.5, -1, 200)
    ref = oracle.query(g, q, 600.0, cfg)
    scl = oracle.result_scales(g, q, 600.0, cfg, ref)
    ids = [r[0] for r in ref["results"]]
    assert set(ids) <= set(scl)
    # w = exp(-lambda * age), the age taken in fp32 as the reference does
    age = np.maximum(np.float32(0), np.float32(600.0) - g.timestamps.astype(np.float32)).astype(np.float64)
    w = np.exp(-np.float64(np.float32(1e-3)) * age)
    row_scale = w * np.abs(g.embeddings.astype(np.float64) * q.astype(np.float64)).sum(1)
    for s in ref["seeds"]:
        assert scl[int(s)] == pytest.approx(row_scale[int(s)], rel=1e-6)
    for u, v in scl.items():
        assert v >= 0.8 * row_scale[u] * (1 - 1e-9)


def test_bfs_stops_on_empty_frontier():
    row, col = _csr(4, [(0, 1)])
    r = oracle.bfs(row, col, np.zeros(4), np.array([0], np.int32), np.array([1.0]), 5, 0.5)
    assert r["levels"] == 2 and sorted(r["ids"]) == [0, 1]


# ---------------------------------------------------------------- whole query
def _query_graph(rng, n=500, d=64, n_ep=50):
    emb, mods, ts = _tiny_graph(rng, n, d)
    ep = np.sort(rng.integers(0, n_ep, size=n)).astype(np.int32)
    row, col = _csr(n, rng.integers(0, n, size=(3 * n, 2)))
    return oracle.make_graph(emb, mods, ts, row, col, ep)


def test_query_global_composition(rng):
    g = _query_graph(rng)
    q = g.embeddings[11]
    cfg = oracle.config(top_k=10, bfs_max_hops=2, time_decay_lambda=0.1, max_results_returned=25)
    r = oracle.query(g, q, 600.0, cfg)
    fin, _ = oracle.scores(g, q, 600.0, 0.1)
    np.testing.assert_allclose(r["final"], fin)
    idx, val = oracle.topk(fin, 10)
    np.testing.assert_array_equal(r["seeds"], idx)
    b = oracle.bfs(g.row_offsets, g.col_indices, fin, idx, val, 2, 0.5)
    assert r["visited"] == len(b["ids"]) and r["n_results"] == min(25, len(b["ids"]))
    order = np.lexsort((b["ids"], -b["scores"]))[:25]
    assert [x[0] for x in r["results"]] == list(b["ids"][order])
    assert [x[3] for x in r["results"]] == list(b["hops"][order])
    assert [x[2] for x in r["results"]] == list(g.modalities[b["ids"][order]])


def test_query_episode_scope(rng):
    g = _query_graph(rng)
    ep = 7
    b, e = int(g.ep_offsets[ep]), int(g.ep_offsets[ep + 1])
    members = g.ep_members[b:e]
    assert len(members) >= 3
    q = g.embeddings[members[0]]
    cfg = oracle.config(top_k=len(members), time_decay_lambda=0.1, retrieval_scope=1, query_episode_id=ep,
                        query_episode_member_begin=b, query_episode_member_count=e - b)
    r = oracle.query(g, q, 600.0, cfg)
    assert r["scoped"] and r["levels"] == 0
    fin, _ = oracle.scores(g, q, 600.0, 0.1)
    want = members[np.lexsort((members, -fin[members]))]
    assert [x[0] for x in r["results"]] == list(want)
    assert all(x[3] == 0 for x in r["results"])
    # K > M: the reference pads with the lowest-id non-members at -FLT_MAX
    cfg.top_k = len(members) + 3
    r = oracle.query(g, q, 600.0, cfg)
    pad = [i for i in range(len(g.modalities)) if i not in set(members)][:3]
    assert [x[0] for x in r["results"][-3:]] == pad
    assert all(x[1] == -FLT_MAX for x in r["results"][-3:])


def test_query_episode_invalid_range_falls_back_to_global(rng):
    g = _query_graph(rng)
    cfg = oracle.config(top_k=5, retrieval_scope=1, query_episode_id=3, query_episode_member_begin=0,
                        query_episode_member_count=10 ** 6)
    r = oracle.query(g, g.embeddings[0], 600.0, cfg)
    assert not r["scoped"] and r["levels"] >= 1


def test_query_boost_only_same_episode(rng):
    g = _query_graph(rng)
    q = g.embeddings[0]
    base = oracle.query(g, q, 600.0, oracle.config(time_decay_lambda=0.1, query_episode_id=4))["final"]
    boosted = oracle.query(g, q, 600.0, oracle.config(time_decay_lambda=0.1, query_episode_id=4,
                                                      episode_same_boost=0.5))["final"]
    same = g.episode_ids == 4
    np.testing.assert_allclose(boosted[same], base[same] * 1.5)
    np.testing.assert_array_equal(boosted[~same], base[~same])


def test_tiled_equals_global_topk(rng):
    emb, mods, ts = _tiny_graph(rng, n=1000, d=32)
    g = oracle.make_graph(emb, mods, ts)
    fin, _ = oracle.scores(g, emb[1], 600.0, 0.1)
    want, _ = oracle.topk(fin, 10)
    for tile in (1000, 333, 64, 10):
        ids, sc = oracle.tiled_query(g, emb[1], 600.0, 0.1, 10, tile)
        np.testing.assert_array_equal(ids, want)


def test_reference_kids_corpus_episode_hit(golden):
    """Outcome fixture: on the reference's own kids corpus every episode-scoped
    query returns its episode's TEXT and AUDIO members (published hit@15 = 1.0)."""
    z = np.load(golden / "kids_small.npz")
    g = oracle.make_graph(z["emb"], z["mods"], z["ts"], z["row"], z["col"], z["ep"])
    img = np.nonzero(z["mods"] == 2)[0][:20]
    for node in img:
        ep = int(z["ep"][node])
        b, e = int(g.ep_offsets[ep]), int(g.ep_offsets[ep + 1])
        cfg = oracle.config(top_k=15, time_decay_lambda=8e-6, bfs_score_decay=0.55, max_results_returned=15,
                            retrieval_scope=1, query_episode_id=ep, query_episode_member_begin=b,
                            query_episode_member_count=e - b)
        r = oracle.query(g, z["emb"][node], float(z["ts"][node]), cfg)
        mods = {x[2] for x in r["results"] if z["ep"][x[0]] == ep}
        assert {0, 1} <= mods


# ---------------------------------------------------------------- k-NN
def test_knn_matches_numpy_lexsort(rng):
    n, d, k = 300, 32, 8
    emb = rng.standard_normal((n, d)).astype(np.float32)
    emb /= np.linalg.norm(emb, axis=1, keepdims=True)
    emb[50] = emb[10]                     # exact ties: equal similarity, lower id first
    emb[51] = emb[10]
    qids = np.array([0, 10, 50, 51, 299, 7], np.int32)
    ids, sims = oracle.knn(emb, qids, k)
    e64 = emb.astype(np.float64)
    for row, u in enumerate(qids):
        s = e64 @ e64[u]
        s[u] = -np.inf
        order = np.lexsort((np.arange(n), -s))[:k]
        np.testing.assert_array_equal(ids[row], order, err_msg=f"node {u}")
        np.testing.assert_allclose(sims[row], s[order], rtol=0, atol=1e-12)
    # node 50's two nearest are its exact copies 10 and 51 (sim 1), lower id first
    assert list(ids[2][:2]) == [10, 51]


def test_knn_restricted_prefix_and_short_rows(rng):
    emb = rng.standard_normal((40, 16)).astype(np.float32)
    ids, sims = oracle.knn(emb, np.array([3, 4], np.int32), 8, n=5)   # only rows 0..4 exist
    assert set(ids[0][:4]) == {0, 1, 2, 4} and list(ids[0][4:]) == [-1] * 4
    assert np.all(np.isneginf(sims[0][4:]))
    assert 4 not in ids[1] and ids[1][4] == -1


# ---------------------------------------------------------------- streaming insert edges
def _sets_insert(row, col, n_old, n_new, ep, knn):
    adj = [set(col[row[i]:row[i + 1]]) if row is not None else set() for i in range(n_old)]
    adj += [set() for _ in range(n_new)]
    for i in range(n_new):
        u = n_old + i
        peers = [n_old + j for j in range(n_new) if ep is not None and j != i and ep[j] == ep[i]]
        for v in peers + [int(x) for x in knn[i] if x >= 0]:
            if v != u:
                adj[u].add(v)
                adj[v].add(u)
    r = np.zeros(n_old + n_new + 1, np.int32)
    c = []
    for i, a in enumerate(adj):
        c += sorted(a)
        r[i + 1] = len(c)
    return r, np.array(c, np.int32)


def _random_csr(rng, n, deg):
    adj = [set() for _ in range(n)]
    for u in range(n):
        for v in rng.choice(n, size=deg, replace=False):
            if v != u:
                adj[u].add(int(v))
                adj[int(v)].add(u)
    row = np.zeros(n + 1, np.int32)
    col = []
    for i, a in enumerate(adj):
        col += sorted(a)
        row[i + 1] = len(col)
    return row, np.array(col, np.int32)


def test_insert_edges_match_set_brute_force(rng):
    for n_old, n_new, k in [(0, 12, 3), (30, 10, 4), (60, 1, 8), (25, 17, 2)]:
        row, col = _random_csr(rng, n_old, 3) if n_old else (None, None)
        ep = rng.integers(100, 104, size=n_new).astype(np.int32)
        knn = rng.integers(-1, n_old + n_new, size=(n_new, k)).astype(np.int32)
        got_r, got_c = oracle.insert_edges(row, col, n_old, n_new, ep, knn)
        want_r, want_c = _sets_insert(row, col, n_old, n_new, ep, knn)
        np.testing.assert_array_equal(got_r, want_r)
        np.testing.assert_array_equal(got_c, want_c)


def test_insert_edges_two_batches_equal_one(rng):
    """Edge union is associative: inserting A then B (same neighbour lists, B's
    episodes new) equals inserting A+B at once."""
    n_old = 40
    row, col = _random_csr(rng, n_old, 4)
    ep = np.array([7] * 5 + [8] * 6 + [9] * 4, np.int32)
    knn = rng.integers(0, n_old + 15, size=(15, 5)).astype(np.int32)
    knn[:11] = np.minimum(knn[:11], n_old + 10)      # batch A only sees nodes up to its own
    r1, c1 = oracle.insert_edges(row, col, n_old, 11, ep[:11], knn[:11])
    r2, c2 = oracle.insert_edges(r1, c1, n_old + 11, 4, ep[11:], knn[11:])
    ra, ca = oracle.insert_edges(row, col, n_old, 15, ep, knn)
    np.testing.assert_array_equal(r2, ra)
    np.testing.assert_array_equal(c2, ca)


def _sets_link(row, col, n, first, knn):
    adj = [set() if row is None else set(col[row[i]:row[i + 1]].tolist()) for i in range(n)]
    for i, lst in enumerate(knn):
        u = first + i
        for v in lst.tolist():
            if 0 <= v < n and v != u:
                adj[u].add(v)
                adj[v].add(u)
    r = np.zeros(n + 1, np.int32)
    r[1:] = np.cumsum([len(a) for a in adj])
    c = np.array([v for a in adj for v in sorted(a)], np.int32)
    return r, c


def test_link_edges_match_set_brute_force(rng):
    for n, first, count, k in [(20, 0, 20, 3), (50, 30, 20, 4), (40, 39, 1, 8), (64, 10, 0, 2)]:
        row, col = _random_csr(rng, n, 3)
        knn = rng.integers(-2, n + 2, size=(count, k)).astype(np.int32)
        got_r, got_c = oracle.link_edges(row, col, n, first, knn)
        want_r, want_c = _sets_link(row, col, n, first, knn)
        np.testing.assert_array_equal(got_r, want_r)
        np.testing.assert_array_equal(got_c, want_c)


def test_insert_then_link_equals_insert_with_knn(rng):
    """Deferred linking: insert with no k-NN, then link the same lists = one insert."""
    n_old = 45
    row, col = _random_csr(rng, n_old, 4)
    ep = np.array([3] * 6 + [4] * 4 + [5] * 5, np.int32)
    knn = rng.integers(-1, n_old + 15, size=(15, 6)).astype(np.int32)
    r0, c0 = oracle.insert_edges(row, col, n_old, 15, ep, np.empty((15, 0), np.int32))
    r1, c1 = oracle.link_edges(r0, c0, n_old + 15, n_old, knn)
    ra, ca = oracle.insert_edges(row, col, n_old, 15, ep, knn)
    np.testing.assert_array_equal(r1, ra)
    np.testing.assert_array_equal(c1, ca)
    # linking is idempotent, and linking in two parts equals one
    r2, c2 = oracle.link_edges(r1, c1, n_old + 15, n_old, knn)
    np.testing.assert_array_equal(r2, r1)
    np.testing.assert_array_equal(c2, c1)
    ra1, ca1 = oracle.link_edges(r0, c0, n_old + 15, n_old, knn[:7])
    ra2, ca2 = oracle.link_edges(ra1, ca1, n_old + 15, n_old + 7, knn[7:])
    np.testing.assert_array_equal(ra2, r1)
    np.testing.assert_array_equal(ca2, c1)


def _check_flush_invariants(row0, col0, row1, col1, n_old, n_new):
    assert len(row1) == n_old + n_new + 1
    for i in range(n_old):                    # every old edge kept
        assert set(col0[row0[i]:row0[i + 1]]) <= set(col1[row1[i]:row1[i + 1]]), i
    edges = set()
    for i in range(n_old + n_new):
        r = col1[row1[i]:row1[i + 1]]
        assert np.all(np.diff(r) > 0), f"row {i} not strictly ascending"
        assert i not in set(r.tolist())
        edges |= {(i, int(v)) for v in r}
    assert all((v, u) in edges for (u, v) in edges), "not symmetric"
    assert len(col1) > len(col0)              # T15: edges were added
    for i in range(n_old, n_old + n_new):     # every new node linked
        assert row1[i + 1] > row1[i], i


def test_insert_edges_keep_reference_flush_invariants(golden):
    """The reference's own flush (fixture made by StreamingBuffer, streaming.cpp:35-163)
    and the oracle's rule share its contract: old edges kept, symmetric, rows
    ascending, every new node linked."""
    z = np.load(golden / "stream_flush.npz")
    n_old = len(z["before_mods"])
    n_new = len(z["new_mods"])
    _check_flush_invariants(z["before_row"], z["before_col"], z["after_row"], z["after_col"], n_old, n_new)
    emb = np.concatenate([z["before_emb"].reshape(n_old, -1), z["new_emb"]]).astype(np.float32)
    knn, _ = oracle.knn(emb, np.arange(n_old, n_old + n_new, dtype=np.int32), 8)
    ep = np.array([0] * 4 + [1] * 3 + [2] * 3, np.int32)
    r, c = oracle.insert_edges(z["before_row"], z["before_col"], n_old, n_new, ep, knn)
    _check_flush_invariants(z["before_row"], z["before_col"], r, c, n_old, n_new)


# ---------------------------------------------------------------- the kids sweep's probe sample
def _mt19937_raw(seed: int, count: int) -> np.ndarray:
    """Raw 32-bit outputs of std::mt19937(seed), from numpy's own MT19937 with the
    standard's init_genrand seeding: an implementation independent of the C++ library."""
    bg = np.random.MT19937()
    bg._legacy_seeding(seed)
    return bg.random_raw(count)


def _uniform_index(raw, hi: int, count: int):
    """uniform_int_distribution<size_t>(0, hi) over a 32-bit engine: Lemire's
    nearly-divisionless method (ACM TOMACS 29(1), 2019; arXiv 1805.10941), which libstdc++
    uses when the engine's range is exactly 32 bits: product = draw * (hi + 1); a low half
    below (2^32 - (hi + 1)) mod (hi + 1) rejects the draw; the result is the high half."""
    rng_range = hi + 1
    thr = ((1 << 32) - rng_range) % rng_range
    out, i = [], 0
    while len(out) < count:
        prod = int(raw[i]) * rng_range
        i += 1
        if (prod & 0xFFFFFFFF) < thr:
            continue
        out.append(prod >> 32)
    return np.array(out, np.int64)


def test_mt19937_known_answer():
    """The C++ standard's known answer for mt19937 ([rand.predef]: the 10000th output of a
    default-constructed engine, seed 5489, is 4123659995) holds for the stream the sampler
    pin below reads."""
    assert int(_mt19937_raw(5489, 10000)[-1]) == 4123659995


@pytest.mark.parametrize("n,n_image", [(1000, 300), (5000, 1500), (10000, 3000), (50000, 15000), (7, 1), (12345, 4097)])
def test_kids_probes_match_independent_sampler(n, n_image):
    """oracle_kids_probes (bench_kids_sweep.cu:624-632: std::mt19937(N ^ 0xA5A5A5A5) and
    uniform_int_distribution<size_t>(0, n_image - 1), 256 draws) against numpy's MT19937
    and Lemire's method restated above. A wrong seed, range bound or distribution fails."""
    got = oracle.kids_probes(n, n_image, 256)
    seed = (n ^ 0xA5A5A5A5) & 0xFFFFFFFF
    want = _uniform_index(_mt19937_raw(seed, 4096), n_image - 1, 256)
    np.testing.assert_array_equal(got, want)
    assert got.min() >= 0 and got.max() < n_image
