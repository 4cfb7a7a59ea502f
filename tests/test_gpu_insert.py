"""GPU streaming insert (mars_graph_insert through the C ABI) against the oracle.

Bars (as applied here):
  * neighbour lists the GPU found for the new nodes: equal to the oracle's fp64
    k-NN (ties: lower id) except ids whose exact similarity lies within 1e-5 of
    the k-th one;
  * device CSR after every insert: bit-exact equal to the oracle's edge rule
    (oracle.insert_edges) applied to the previous CSR with those lists;
  * device episode CSR: bit-exact equal to build_episode_csr of all episode ids;
  * queries after inserts: the global / episode parity bars of test_gpu_parity
    (scores 1e-5, BFS visit order / hops exact) on the grown graph.
Edge cases: capacity (nodes, edges), invalid episode ids, no fp16 copy, graphs
without episode ids, rows that move to the tail and later grow in place, and
queries running on another thread while inserts land.
"""
from __future__ import annotations

import threading

import numpy as np
import pytest

import mars_amd
import oracle
from mars_amd import RetrievalConfig, RetrievalScope, corpus
from mars_amd._lib import MarsError

from parity import T_Q, check_global, ocfg

pytestmark = pytest.mark.gpu
K_NN = corpus.KNN_K
BASE, EXTRA = 3000, 200


@pytest.fixture(scope="module")
def full():
    """3,200-node corpus: the first 3,000 nodes are resident, the last 20 episodes arrive."""
    return corpus.make_corpus(BASE + EXTRA, 768, seed=77)


class Live:
    """A resident graph that grows, with its expected CSR."""

    def __init__(self, c, n0, cap_n, episodes=True, fp16=True, capacity_edges=0):
        self.c = c
        emb, mods, ts = c.embeddings[:n0], c.modalities[:n0], c.timestamps[:n0]
        ep = c.episode_ids[:n0]
        knn = corpus.knn(emb, K_NN)
        self.row, self.col = corpus.build_nsn_csr(ep if episodes else np.arange(n0, dtype=np.int32), knn)
        g = mars_amd.MemoryGraph(n0, emb.shape[1], self.row, self.col, emb, mods, ts)
        self.dg = mars_amd.upload_to_device(g, capacity_nodes=cap_n, capacity_edges=capacity_edges)
        self.episodes = episodes
        if episodes:
            mars_amd.upload_episode_ids(self.dg, ep)
            mars_amd.upload_episode_csr(self.dg, mars_amd.build_episode_csr(ep, n0))
        if fp16:
            mars_amd.upload_fp16_embeddings(self.dg)
        self.ctx = mars_amd.create_query_context(cap_n, emb.shape[1], 64)
        self.n = n0

    def close(self):
        mars_amd.destroy_query_context(self.ctx)
        mars_amd.free_device(self.dg)

    @property
    def og(self):
        n = self.n
        return oracle.make_graph(self.c.embeddings[:n], self.c.modalities[:n], self.c.timestamps[:n], self.row,
                                 self.col, self.c.episode_ids[:n] if self.episodes else None)

    def query(self, q, cfg, t_q=T_Q):
        st = mars_amd.RetrievalStats()
        return mars_amd.query_memory_fast(self.dg, self.ctx, q, t_q, cfg, st), st

    def insert(self, m, knn_k=K_NN, ep=None):
        n, c = self.n, self.c
        if ep is None and self.episodes:
            ep = c.episode_ids[n:n + m]
        st, got = mars_amd.insert_nodes(self.dg, c.embeddings[n:n + m], c.modalities[n:n + m],
                                        c.timestamps[n:n + m], ep, knn_k=knn_k, return_knn=True)
        assert st.first_node == n and st.nodes_added == m
        self.row, self.col = oracle.insert_edges(self.row, self.col, n, m, ep, got)
        self.n = n + m
        return st, got


def check_knn(c, n_after, first, got, k):
    want, sims = oracle.knn(c.embeddings, np.arange(first, n_after, dtype=np.int32), k, n=n_after)
    e = c.embeddings[:n_after].astype(np.float64)
    for i in range(len(got)):
        assert len(set(got[i].tolist())) == k and first + i not in got[i]
        for j in set(got[i].tolist()) ^ set(want[i].tolist()):
            s = float(e[first + i] @ e[j])
            assert abs(s - sims[i, k - 1]) <= 1e-5, (first + i, j, s, sims[i, k - 1])


def check_device_csr(live):
    row, col = live.dg.download_csr()
    np.testing.assert_array_equal(row, live.row)
    np.testing.assert_array_equal(col, live.col)
    assert live.dg.num_nodes == live.n and live.dg.num_edges == len(live.col)


def test_insert_matches_oracle_and_queries_stay_exact(full):
    live = Live(full, BASE, BASE + EXTRA)
    try:
        for n_eps in (1, 3, 6, 10):                       # 10 + 30 + 60 + 100 nodes
            m = 10 * n_eps
            first, e_before = live.n, len(live.col)
            st, got = live.insert(m)
            check_knn(full, first + m, first, got, K_NN)
            check_device_csr(live)
            assert st.edges_added == len(live.col) - e_before
            assert 0 < st.queryable_us <= st.linked_us
            off, mem = live.dg.download_episode_csr()
            want_off, want_mem = oracle.episode_csr(full.episode_ids[:live.n])
            np.testing.assert_array_equal(off, want_off)
            np.testing.assert_array_equal(mem, want_mem)
            # T17 analogue: every new node has a neighbour of another modality
            mods = full.modalities
            for u in range(first, live.n):
                r = live.col[live.row[u]:live.row[u + 1]]
                assert np.any(mods[r] != mods[u]), u
        assert live.n == BASE + EXTRA
        # queries over the grown graph, seeded on inserted and old nodes
        qs = np.concatenate([corpus.pick_queries(full.modalities[BASE:], 6, seed=5) + BASE,
                             corpus.pick_queries(full.modalities[:BASE], 4, seed=6)])
        off = live.dg.download_episode_csr()[0]
        for node in qs:
            q = full.embeddings[node]
            cfg = RetrievalConfig(top_k=10, bfs_max_hops=2, time_decay_lambda=corpus.DECAY_LAMBDA,
                                  max_results_returned=15)
            check_global(live, q, cfg)
            ep = int(full.episode_ids[node])
            cfg = RetrievalConfig(top_k=10, bfs_max_hops=2, time_decay_lambda=corpus.DECAY_LAMBDA,
                                  retrieval_scope=RetrievalScope.EpisodeScoped, query_episode_id=ep,
                                  query_episode_member_begin=int(off[ep]),
                                  query_episode_member_count=int(off[ep + 1] - off[ep]))
            res, st = live.query(q, cfg)
            ref = oracle.query(live.og, q, T_Q, ocfg(cfg))
            assert st.scope_fallback == 0
            assert [r.node_id for r in res] == [w[0] for w in ref["results"]]
        # fp16 rows of the inserted nodes are the RNE rows enable_fp16 would make
        live.ctx.use_fp16 = True
        og = live.og
        emb16 = oracle.to_f16_bits(full.embeddings[:live.n])
        og16 = oracle.Graph(og.embeddings, og.modalities, og.timestamps, og.row_offsets, og.col_indices,
                            og.episode_ids, og.ep_offsets, og.ep_members, emb16)
        for node in qs[:3]:
            cfg = RetrievalConfig(top_k=10, bfs_max_hops=2, time_decay_lambda=corpus.DECAY_LAMBDA)
            res, st = live.query(full.embeddings[node], cfg)
            assert st.used_fp16 == 1
            fin = live.ctx.last_scores(live.n)
            ref_fin, scale = oracle.scores(og16, full.embeddings[node], T_Q, corpus.DECAY_LAMBDA)
            assert np.all(np.abs(fin - ref_fin) <= 1e-5 * np.maximum(np.abs(ref_fin), scale) + 1e-30)
    finally:
        live.close()


def test_insert_rows_move_then_grow_in_place(full):
    """Near-copies of one old node: its row gains a neighbour per insert, moves to
    the tail once, then grows inside its reserved slots."""
    c = full
    n0 = BASE
    live = Live(c, n0, n0 + 40, episodes=False)
    try:
        target = 123
        rng = np.random.default_rng(3)
        extra = c.embeddings[target] + 1e-3 * rng.standard_normal((40, c.embeddings.shape[1])).astype(np.float32)
        extra /= np.linalg.norm(extra, axis=1, keepdims=True)
        emb = np.concatenate([c.embeddings[:n0], extra]).astype(np.float32)
        grown = corpus.Corpus(emb, np.concatenate([c.modalities[:n0], np.full(40, 2, np.int32)]),
                              np.concatenate([c.timestamps[:n0], np.full(40, 599.0, np.float32)]),
                              np.arange(n0 + 40, dtype=np.int32), c.seed)
        live.c = grown
        moved = appended = 0
        for _ in range(12):
            first = live.n
            st, got = live.insert(1)
            assert target in got[0]
            check_knn(grown, live.n, first, got, K_NN)
            check_device_csr(live)
            moved += st.rows_relocated
            appended += st.rows_appended
        assert moved > 0 and appended > 0
        for m in (7, 20):                                  # multi-node batches, no episodes
            st, got = live.insert(m)
            check_device_csr(live)
        check_global(live, grown.embeddings[target], RetrievalConfig(top_k=10, bfs_max_hops=2,
                                                                    time_decay_lambda=corpus.DECAY_LAMBDA))
    finally:
        live.close()


def test_insert_errors_leave_graph_unchanged(full):
    c = full
    live = Live(c, BASE, BASE + 15)
    try:
        row0, col0 = live.dg.download_csr()
        n = live.n

        def bad(code, **kw):
            args = dict(embeddings=c.embeddings[n:n + 10], modalities=c.modalities[n:n + 10],
                        timestamps=c.timestamps[n:n + 10], episode_ids=c.episode_ids[n:n + 10], knn_k=8)
            args.update(kw)
            with pytest.raises(MarsError) as e:
                mars_amd.insert_nodes(live.dg, **args)
            assert e.value.code == code
            row, col = live.dg.download_csr()
            np.testing.assert_array_equal(row, row0)
            np.testing.assert_array_equal(col, col0)
            assert live.dg.num_nodes == n

        bad(-1, episode_ids=np.full(10, 5, np.int32))            # episode 5 exists already
        bad(-1, episode_ids=None)                                  # graph has episode ids
        bad(-1, knn_k=17)
        bad(-4, embeddings=c.embeddings[n:n + 20], modalities=c.modalities[n:n + 20],
            timestamps=c.timestamps[n:n + 20], episode_ids=c.episode_ids[n:n + 20])   # 20 > 15 spare nodes
        mars_amd.free_fp16_embeddings(live.dg)
        bad(-5)                                                    # k-NN needs the fp16 rows
        # without neighbour search: episode pairs only
        st = live.insert(10, knn_k=0)[0]
        assert st.edges_added == 10 * 9
        check_device_csr(live)
    finally:
        live.close()
    tight = Live(c, BASE, BASE + 10, capacity_edges=1)          # no room beyond the base CSR
    try:
        with pytest.raises(MarsError) as e:
            tight.insert(10)
        assert e.value.code == -4
        assert tight.dg.download_csr()[0].shape[0] == BASE + 1
    finally:
        tight.close()


def test_queries_while_inserting(full):
    """A second thread inserts episodes while this one queries: every query
    succeeds and returns ids of published nodes; afterwards the graph and the
    queries match the oracle."""
    live = Live(full, BASE, BASE + EXTRA)
    errors = []
    done = threading.Event()

    def writer():
        try:
            for _ in range(EXTRA // 10):
                a = live_n[0]
                _, got = mars_amd.insert_nodes(live.dg, full.embeddings[a:a + 10], full.modalities[a:a + 10],
                                               full.timestamps[a:a + 10], full.episode_ids[a:a + 10], knn_k=K_NN,
                                               return_knn=True)
                lists.append(got)
                live_n[0] += 10
        except Exception as exc:                          # reported below
            errors.append(exc)
        finally:
            done.set()

    live_n = [BASE]
    lists = []
    t = threading.Thread(target=writer)
    qs = corpus.pick_queries(full.modalities, 64, seed=17)
    cfg = RetrievalConfig(top_k=10, bfs_max_hops=2, time_decay_lambda=corpus.DECAY_LAMBDA,
                          max_results_returned=15)
    t.start()
    n_q = 0
    try:
        while not done.is_set() or n_q < 20:
            node = int(qs[n_q % len(qs)]) % BASE
            res, st = live.query(full.embeddings[node], cfg)
            assert 0 < len(res) <= 15
            assert all(0 <= r.node_id < BASE + EXTRA and r.hops_from_seed >= 0 for r in res)
            sc = [r.score for r in res]
            assert sc == sorted(sc, reverse=True)
            n_q += 1
        t.join()
        assert not errors, errors
        assert live_n[0] == BASE + EXTRA
        # final state: the edge rule applied batch by batch with the lists the GPU found
        live.dg.refresh()
        assert live.dg.num_nodes == BASE + EXTRA
        row, col = live.dg.download_csr()
        er, ec = live.row, live.col
        for b, got in enumerate(lists):
            a = BASE + 10 * b
            check_knn(full, a + 10, a, got, K_NN)
            er, ec = oracle.insert_edges(er, ec, a, 10, full.episode_ids[a:a + 10], got)
        np.testing.assert_array_equal(row, er)
        np.testing.assert_array_equal(col, ec)
        # old rows only grew; rows of new nodes hold episode peers + neighbours
        for u in range(BASE):
            old = live.col[live.row[u]:live.row[u + 1]]
            new = col[row[u]:row[u + 1]]
            np.testing.assert_array_equal(new[:len(old)], old)
            assert np.all(new[len(old):] >= BASE)
        live.row, live.col, live.n = row, col, BASE + EXTRA
        for node in qs[:6]:
            check_global(live, full.embeddings[int(node)], cfg)
    finally:
        done.wait()
        live.close()


def test_stream_driver_paced_inserts_and_queries(full):
    """mars_bench_stream: paced inserts on one thread, paced mixed queries on the
    caller's; the grown graph keeps every old edge and is symmetric."""
    import ctypes as C
    from mars_amd import _lib
    live = Live(full, BASE, BASE + EXTRA)
    try:
        row0, col0 = live.row, live.col
        nq = 60
        qs = corpus.pick_queries(full.modalities[:BASE], nq, seed=23)
        dq = mars_amd.DeviceBuffer.from_array(full.embeddings[qs])
        off = mars_amd.build_episode_csr(full.episode_ids[:BASE], BASE).ep_csr_offsets
        cfgs = (_lib.RetrievalConfigC * nq)()
        for i, node in enumerate(qs):
            ep = int(full.episode_ids[node])
            cfg = RetrievalConfig(top_k=10, bfs_max_hops=2, time_decay_lambda=corpus.DECAY_LAMBDA)
            if i % 2:
                cfg = RetrievalConfig(top_k=10, time_decay_lambda=corpus.DECAY_LAMBDA,
                                      retrieval_scope=RetrievalScope.EpisodeScoped, query_episode_id=ep,
                                      query_episode_member_begin=int(off[ep]),
                                      query_episode_member_count=int(off[ep + 1] - off[ep]))
            cfgs[i] = cfg.to_c()
        M = EXTRA
        emb = np.ascontiguousarray(full.embeddings[BASE:])
        mods, ts = np.ascontiguousarray(full.modalities[BASE:]), np.ascontiguousarray(full.timestamps[BASE:])
        ep = np.ascontiguousarray(full.episode_ids[BASE:])
        ins = (_lib.InsertStatsC * (M // 10))()
        lat, qst, ist = np.zeros(nq), np.zeros(nq), np.zeros(M // 10)
        v = lambda a: a.ctypes.data
        b = _lib.StreamBenchC(dq.ptr, 768, nq, T_Q, C.cast(cfgs, C.c_void_p).value, 2000.0, v(emb), v(mods), v(ts),
                              v(ep), M, 10, 4000.0, K_NN, v(lat), v(qst), C.cast(ins, C.c_void_p).value, v(ist))
        _lib.check(_lib.lib.mars_bench_stream(live.dg.handle, live.ctx.handle, C.byref(b)), "mars_bench_stream")
        dq.free()
        assert np.all(lat > 0) and np.all(np.diff(qst) > 0)
        assert [s.nodes_added for s in ins] == [10] * (M // 10)
        assert [s.first_node for s in ins] == list(range(BASE, BASE + M, 10))
        assert all(0 < s.queryable_us <= s.linked_us for s in ins)
        row, col = live.dg.download_csr()
        assert len(row) == BASE + M + 1
        edges = set()
        for u in range(BASE + M):
            r = col[row[u]:row[u + 1]]
            assert np.all(np.diff(r) > 0)
            if u < BASE:
                np.testing.assert_array_equal(r[:row0[u + 1] - row0[u]], col0[row0[u]:row0[u + 1]])
            edges |= {(u, int(x)) for x in r}
        assert all((y, x) in edges for (x, y) in edges)
    finally:
        live.close()
