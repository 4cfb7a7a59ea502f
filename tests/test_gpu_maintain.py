"""Importance, novelty, edge hits and the maintenance sweep on the GPU (through the C
ABI) against the oracle (memory_cuda.cu:1466-1658).

Bars:
  * importance: bit for bit against the oracle's fp32 rule after every update (ragged
    node counts, repeated / negative / out-of-range ids, ids in device memory, nodes
    inserted after init);
  * novelty: within the fp32 dot bound RTOL_F32 * max_i sum_d |E_id q_d| of the oracle's
    fp64 maximum, and bit-identical between the graph's own certified context, an fp32
    context and a certified caller context;
  * edge hits: equal to the oracle's counts over the BFS levels of the same queries, on
    both query paths, through inserts that relocate rows and links that rewrite them
    (counters follow their edges; new edges start at 0);
  * maintenance: the oracle's low-utility count, and every counter zero afterwards.
"""
from __future__ import annotations

import numpy as np
import pytest

import mars_amd
import oracle
from conftest import RTOL_F32
from mars_amd import RetrievalConfig, RetrievalScope, corpus

from test_gpu_insert import K_NN, Live

pytestmark = pytest.mark.gpu
T_Q = corpus.QUERY_TIME
N0 = 4099                      # not a multiple of 4 or of the 1024-node slices


@pytest.fixture(scope="module")
def full():
    return corpus.make_corpus(N0 + 300, 768, seed=123)


def insert(live, m, knn_k=K_NN):
    """Insert the next m corpus nodes in new episodes of two (the corpus's own ids would
    continue an episode that N0 cuts)."""
    nxt = getattr(live, "ep_next", int(live.c.episode_ids[:live.n].max()) + 1)
    live.ep_next = nxt + (m + 1) // 2
    return live.insert(m, knn_k=knn_k, ep=(nxt + np.arange(m) // 2).astype(np.int32))


def bits_equal(a, b):
    np.testing.assert_array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def test_importance_matches_oracle(full):
    live = Live(full, N0, N0 + 300)
    try:
        mars_amd.init_importance(live.dg)
        want = np.ones(N0, np.float32)
        bits_equal(mars_amd.read_importance(live.dg), want)
        rng = np.random.default_rng(3)
        params = [(0.1, 0.001, 5.0), (0.25, 0.5, 1.0), (0.3, 0.01, 1.2)]
        for step in range(12):
            ids = rng.integers(-5, N0 + 5, size=int(rng.integers(0, 80))).astype(np.int32)
            if step % 3 == 0:
                ids = np.concatenate([ids, ids[:5], ids[:2]])                  # repeats
            boost, decay, mx = params[step % 3]
            mars_amd.update_importance(live.dg, ids, boost, decay, mx)
            want = oracle.importance_update(want, ids, boost, decay, mx)
            bits_equal(mars_amd.read_importance(live.dg), want)
        ids = np.int32([7, N0 - 1, 7, 0, -3])                                  # device-resident ids
        buf = mars_amd.DeviceBuffer.from_array(ids)
        try:
            mars_amd.update_importance(live.dg, len(ids), device_ptr=buf.ptr)
        finally:
            buf.free()
        want = oracle.importance_update(want, ids)
        bits_equal(mars_amd.read_importance(live.dg), want)
        insert(live, 100)                                                        # new nodes start at 1.0
        want = np.concatenate([want, np.ones(100, np.float32)])
        bits_equal(mars_amd.read_importance(live.dg), want)
        ids = np.int32([N0 + 50, 3, N0 + 99])
        mars_amd.update_importance(live.dg, ids, 0.2, 0.05, 2.0)
        want = oracle.importance_update(want, ids, 0.2, 0.05, 2.0)
        bits_equal(mars_amd.read_importance(live.dg), want)
        bits_equal(mars_amd.read_importance(live.dg, N0 + 40, 20), want[N0 + 40:N0 + 60])
    finally:
        live.close()


def test_novelty_matches_oracle(full):
    live = Live(full, N0, N0 + 300)
    cert = mars_amd.create_query_context(N0 + 300, 768, 64)
    cert.certified = True
    rng = np.random.default_rng(8)
    try:
        qs = [full.embeddings[i] for i in (0, 17, N0 - 1, N0 + 5)]
        qs += [rng.standard_normal(768).astype(np.float32) for _ in range(3)]
        qs.append(-full.embeddings[4])
        for i, q in enumerate(qs):
            want, scale = oracle.novelty(live.og, q)
            own = mars_amd.compute_novelty(live.dg, q)
            f32 = mars_amd.compute_novelty(live.dg, q, ctx=live.ctx)
            crt = mars_amd.compute_novelty(live.dg, q, ctx=cert)
            assert own == f32 == crt, (i, own, f32, crt)
            assert abs(own - want) <= RTOL_F32 * max(scale, abs(want)), (i, own, want)
        buf = mars_amd.DeviceBuffer.from_array(qs[5])
        try:
            assert mars_amd.compute_novelty(live.dg, device_ptr=buf.ptr) == mars_amd.compute_novelty(live.dg, qs[5])
        finally:
            buf.free()
        insert(live, 50)                       # inserted rows are seen by the next call
        q = full.embeddings[N0 + 10]
        want, scale = oracle.novelty(live.og, q)
        got = mars_amd.compute_novelty(live.dg, q)
        assert abs(got - want) <= RTOL_F32 * max(scale, abs(want))
        assert got == mars_amd.compute_novelty(live.dg, q, ctx=live.ctx)
    finally:
        mars_amd.destroy_query_context(cert)
        live.close()


def oracle_levels(live, q, cfg):
    ocfg = oracle.config(top_k=cfg.top_k, bfs_max_hops=cfg.bfs_max_hops, time_decay_lambda=cfg.time_decay_lambda,
                         bfs_score_decay=cfg.bfs_score_decay, modality_filter=cfg.modality_filter)
    r = oracle.query(live.og, q, T_Q, ocfg)
    b = oracle.bfs(live.row, live.col, r["final"], r["seeds"], r["seed_vals"], cfg.bfs_max_hops, cfg.bfs_score_decay)
    return r, b["hop_by_node"]


def carried(old_row, old_col, old_hits, row, col):
    """Counters of the new CSR when each (v, u) edge keeps its count and new edges start at 0."""
    have = {}
    for v in range(len(old_row) - 1):
        for e in range(old_row[v], old_row[v + 1]):
            have[(v, int(old_col[e]))] = int(old_hits[e])
    out = np.zeros(len(col), np.int32)
    for v in range(len(row) - 1):
        for e in range(row[v], row[v + 1]):
            out[e] = have.get((v, int(col[e])), 0)
    return out


def no_duplicate_edges(row, col):
    for v in range(len(row) - 1):
        r = col[row[v]:row[v + 1]]
        assert len(np.unique(r)) == len(r)


def test_edge_hits_and_maintenance(full):
    live = Live(full, N0, N0 + 300)
    cert = mars_amd.create_query_context(N0 + 300, 768, 64)
    cert.certified = True
    try:
        no_duplicate_edges(live.row, live.col)
        mars_amd.init_edge_hits(live.dg)
        hits = np.zeros(len(live.col), np.int32)
        np.testing.assert_array_equal(mars_amd.read_edge_hits(live.dg), hits)
        qs = corpus.pick_queries(full.modalities[:N0], 16, seed=9)

        def run(j, node):
            ctx = cert if j % 2 == 0 else live.ctx
            cfg = RetrievalConfig(top_k=10, bfs_max_hops=1 + j % 3, modality_filter=-1 if j % 3 else 2)
            q = full.embeddings[node]
            res = mars_amd.query_memory_fast(live.dg, ctx, q, T_Q, cfg)
            r, hop = oracle_levels(live, q, cfg)
            assert [x.node_id for x in res] == [x[0] for x in r["results"]][:len(res)]
            assert [x.hops_from_seed for x in res] == [x[3] for x in r["results"]][:len(res)]
            mars_amd.count_edge_hits(live.dg, ctx)
            return oracle.edge_hits(live.row, live.col, hop, hits)

        for j, node in enumerate(qs[:6]):
            hits = run(j, node)
            np.testing.assert_array_equal(mars_amd.read_edge_hits(live.dg), hits)
        assert hits.sum() > 0
        # an episode-scoped query leaves no BFS levels: counting is a no-op
        ep = int(full.episode_ids[qs[0]])
        off, mem = live.dg.download_episode_csr()
        cfg = RetrievalConfig(retrieval_scope=RetrievalScope.EpisodeScoped, query_episode_id=ep,
                              query_episode_member_begin=int(off[ep]),
                              query_episode_member_count=int(off[ep + 1] - off[ep]))
        mars_amd.query_memory_fast(live.dg, live.ctx, full.embeddings[qs[0]], T_Q, cfg)
        mars_amd.count_edge_hits(live.dg, live.ctx)
        np.testing.assert_array_equal(mars_amd.read_edge_hits(live.dg), hits)
        # inserts: rows that grow are appended in place or relocated with their counters
        old = (live.row.copy(), live.col.copy(), hits.copy())
        st, _ = insert(live, 60)
        assert st.rows_relocated > 0
        no_duplicate_edges(live.row, live.col)
        hits = carried(*old, live.row, live.col)
        np.testing.assert_array_equal(mars_amd.read_edge_hits(live.dg), hits)
        for j, node in enumerate(qs[6:10]):
            hits = run(j, node)
            np.testing.assert_array_equal(mars_amd.read_edge_hits(live.dg), hits)
        # deferred links rewrite whole rows: counters follow their edges
        first = live.n
        old = (live.row.copy(), live.col.copy(), hits.copy())
        insert(live, 40, knn_k=0)
        hits = carried(*old, live.row, live.col)
        np.testing.assert_array_equal(mars_amd.read_edge_hits(live.dg), hits)
        old = (live.row.copy(), live.col.copy(), hits.copy())
        st, got = mars_amd.link_knn(live.dg, first, 40, K_NN, return_knn=True)
        assert st.rows_relocated > 0
        live.row, live.col = oracle.link_edges(live.row, live.col, live.n, first, got)
        hits = carried(*old, live.row, live.col)
        np.testing.assert_array_equal(mars_amd.read_edge_hits(live.dg), hits)
        for j, node in enumerate(qs[10:14]):
            hits = run(j, node)
            np.testing.assert_array_equal(mars_amd.read_edge_hits(live.dg), hits)
        # maintenance: low-utility count, then every counter zero
        want, _ = oracle.maintain(hits, 1)
        assert mars_amd.maintain_graph(live.dg, 1) == want
        hits = np.zeros(len(live.col), np.int32)
        np.testing.assert_array_equal(mars_amd.read_edge_hits(live.dg), hits)
        hits = run(1, qs[14])
        want, _ = oracle.maintain(hits, 0)
        assert mars_amd.maintain_graph(live.dg, 0) == want
        hits = run(2, qs[15])
        assert mars_amd.maintain_graph(live.dg, -1) == 0
        np.testing.assert_array_equal(mars_amd.read_edge_hits(live.dg), np.zeros(len(live.col), np.int32))
        assert mars_amd.maintain_graph(live.dg, 0) == len(live.col)
        # a new CSR zeroes the counters
        hits = run(3, qs[1])
        mars_amd.set_csr(live.dg, live.row, live.col)
        np.testing.assert_array_equal(mars_amd.read_edge_hits(live.dg), np.zeros(len(live.col), np.int32))
    finally:
        mars_amd.destroy_query_context(cert)
        live.close()


def test_maintenance_errors(full):
    live = Live(full, 200, 300)
    try:
        with pytest.raises(mars_amd.MarsError):
            mars_amd.update_importance(live.dg, [1])          # not initialised
        with pytest.raises(mars_amd.MarsError):
            mars_amd.count_edge_hits(live.dg, live.ctx)
        assert mars_amd.maintain_graph(live.dg) == 0          # no counters: nothing to sweep
        mars_amd.init_importance(live.dg)
        with pytest.raises(mars_amd.MarsError):
            mars_amd.read_importance(live.dg, 150, 100)       # past the node count
    finally:
        live.close()
