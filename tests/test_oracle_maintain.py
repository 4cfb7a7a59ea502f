"""Pins of the oracle's importance / novelty / edge-hit / maintenance restatements
(memory_cuda.cu:1466-1658) by hand-derived values, closed forms and independent
numpy / scipy computations. The reference's kernels are CUDA and cannot be built
here, so these are the pins."""
from __future__ import annotations

import numpy as np
import pytest
from scipy.sparse import csr_matrix
from scipy.sparse.csgraph import shortest_path

import oracle


def test_importance_hand_values():
    # decay 0.5 then boost 0.25 (exact binary values): a boost-before-decay order would
    # give 0.625 for node 1; node 3 is listed twice and clamps at 1.0; -1 and 9 skipped
    out = oracle.importance_update(np.ones(4, np.float32), [1, 3, 3, -1, 9], boost=0.25, decay_rate=0.5, max_imp=1.0)
    np.testing.assert_array_equal(out, np.float32([0.5, 0.75, 0.5, 1.0]))
    # no decay: the boost alone, rounded in fp32
    out = oracle.importance_update(np.ones(3, np.float32), [0], boost=0.1, decay_rate=0.0, max_imp=5.0)
    assert out[0] == np.float32(1.0) + np.float32(0.1) and out[1] == 1.0
    # only the first n nodes decay
    out = oracle.importance_update(np.ones(3, np.float32), [], boost=0.1, decay_rate=0.5, n=2)
    np.testing.assert_array_equal(out, np.float32([0.5, 0.5, 1.0]))


def test_importance_fixed_points():
    # with the reference defaults a node boosted every step saturates at max_importance
    # exactly (5 * 0.999 + 0.1 > 5), and an unboosted one follows 0.999^k
    imp = np.ones(2, np.float32)
    for _ in range(2000):
        imp = oracle.importance_update(imp, [0])
    assert imp[0] == np.float32(5.0)
    assert abs(float(imp[1]) - 0.999 ** 2000) <= 2000 * 2.0 ** -23 * 0.999 ** 2000 + 1e-7


def test_novelty_against_numpy():
    rng = np.random.default_rng(5)
    emb = rng.standard_normal((500, 64)).astype(np.float32)
    emb /= np.linalg.norm(emb, axis=1, keepdims=True)
    g = oracle.make_graph(emb, np.zeros(500, np.int32), np.zeros(500, np.float32))
    for q in (emb[17], rng.standard_normal(64).astype(np.float32)):
        v, scale = oracle.novelty(g, q)
        want = float(np.max(emb.astype(np.float64) @ q.astype(np.float64)))
        assert v == pytest.approx(max(want, -1.0), abs=1e-12)
        assert scale >= abs(v) - 1e-12
    assert oracle.novelty(g, emb[17])[0] == pytest.approx(float(emb[17].astype(np.float64) @ emb[17]), abs=1e-12)
    # every dot below -1: the reference's floor
    q = (-3.0 * emb.mean(axis=0) / np.linalg.norm(emb.mean(axis=0))).astype(np.float32)
    far = oracle.make_graph(np.tile(-q / 3.0 * 2.0, (4, 1)).astype(np.float32), np.zeros(4, np.int32),
                            np.zeros(4, np.float32))
    assert oracle.novelty(far, q)[0] == -1.0


def csr_from_edges(n, edges):
    adj = [set() for _ in range(n)]
    for a, b in edges:
        adj[a].add(b)
        adj[b].add(a)
    row = np.zeros(n + 1, np.int32)
    col = []
    for i in range(n):
        col.extend(sorted(adj[i]))
        row[i + 1] = len(col)
    return row, np.array(col, np.int32)


def test_edge_hits_hand_graphs():
    # path 0-1-2-3, seed 0: each node's edge back towards the seed is hit once
    row, col = csr_from_edges(4, [(0, 1), (1, 2), (2, 3)])
    hits = oracle.edge_hits(row, col, [0, 1, 2, 3])
    np.testing.assert_array_equal(hits, [0, 1, 0, 1, 0, 1])       # rows [1] [0,2] [1,3] [2]
    # diamond 0-1, 0-2, 1-3, 2-3 from seed 0: node 3 has two parents, both edges hit
    row, col = csr_from_edges(4, [(0, 1), (0, 2), (1, 3), (2, 3)])
    hits = oracle.edge_hits(row, col, [0, 1, 1, 2])
    np.testing.assert_array_equal(hits, [0, 0, 1, 0, 1, 0, 1, 1])  # rows [1,2] [0,3] [0,3] [1,2]
    # unvisited nodes and seeds add nothing; counts accumulate
    hits = oracle.edge_hits(row, col, [0, -1, 1, -1], hits)
    np.testing.assert_array_equal(hits, [0, 0, 1, 0, 2, 0, 1, 1])


def test_edge_hits_bfs_tree_invariant():
    # on a symmetric graph every visited non-seed node has an edge to its BFS parent,
    # so it has at least one hit edge; levels agree with scipy's shortest paths
    rng = np.random.default_rng(11)
    n = 400
    edges = {(int(a), int(b)) for a, b in rng.integers(0, n, (900, 2)) if a != b}
    row, col = csr_from_edges(n, edges)
    fin = rng.random(n)
    seeds = np.argsort(-fin)[:5].astype(np.int32)
    b = oracle.bfs(row, col, fin, seeds, fin[seeds], 3, 0.5)
    hop = b["hop_by_node"]
    m = csr_matrix((np.ones(len(col)), col, row), shape=(n, n))
    dist = shortest_path(m, unweighted=True, indices=seeds).min(axis=0)
    np.testing.assert_array_equal(np.where(hop >= 0, hop, -1), np.where(dist <= 3, dist, -1).astype(np.int32))
    hits = oracle.edge_hits(row, col, hop)
    per_row = np.add.reduceat(hits, row[:-1]) if len(col) else np.zeros(n)
    per_row = np.where(np.diff(row) > 0, per_row, 0)
    assert np.all(per_row[hop > 0] >= 1) and np.all(per_row[hop <= 0] == 0)


def test_maintain_hand_values():
    hits = np.int32([0, 2, 1, 0, 5])
    assert oracle.maintain(hits, 0)[0] == 2
    assert oracle.maintain(hits, 1)[0] == 3
    assert oracle.maintain(hits, -1)[0] == 0
    low, after = oracle.maintain(hits, 4)
    assert low == 4 and not after.any()
