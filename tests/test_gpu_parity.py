"""GPU parity: the HIP path (through the C ABI) against the CPU oracle on the
same seeded inputs.

The bars are those of tests/parity.py: fused scores within 1e-5 * max(|oracle|, w * sum|e q|)
(fp32) or 2e-3 of that scale (fp16 path against the fp32 oracle), BFS scores with the scale
carried along the BFS, seeds and results equal up to near-ties, BFS visit order and hops
bit-exact, episode-scoped ids exact.
"""
from __future__ import annotations

import numpy as np
import pytest

import mars_amd
import oracle
from mars_amd import RetrievalConfig, RetrievalScope, corpus

from conftest import RTOL_F16_VS_F32, RTOL_F32
from parity import (FLT_MAX, LAM, T_Q, Dev, batch_check, check_batch_topk, check_episode, check_episode_results,
                    check_global, check_results_exact, check_scores, episode_cfg, ocfg, random_graph)

pytestmark = pytest.mark.gpu


# ---------------------------------------------------------------- corpus N=10K (CPU plumbing size)
@pytest.fixture(scope="module")
def dev10k(corpus_10k):
    c = corpus_10k
    d = Dev(c.embeddings, c.modalities, c.timestamps, c.row_offsets, c.col_indices, c.episode_ids, fp16=True)
    yield d
    d.close()


def test_episode_csr_on_device_matches(dev10k, corpus_10k):
    off, mem = dev10k.dg.download_episode_csr()
    want_off, want_mem = oracle.episode_csr(corpus_10k.episode_ids)
    np.testing.assert_array_equal(off, want_off)
    np.testing.assert_array_equal(mem, want_mem)


def test_global_parity_10k(dev10k, corpus_10k):
    qs = corpus.pick_queries(corpus_10k.modalities, 60, seed=101)
    cfg = RetrievalConfig(top_k=10, bfs_max_hops=2, time_decay_lambda=LAM, bfs_score_decay=0.5,
                          max_results_returned=15)
    dev10k.ctx.use_fp16 = False
    for node in qs:
        check_global(dev10k, corpus_10k.embeddings[node], cfg)


def test_global_parity_variants_10k(dev10k, corpus_10k):
    dev10k.ctx.use_fp16 = False
    q = corpus_10k.embeddings[corpus.pick_queries(corpus_10k.modalities, 1, seed=7)[0]]
    for cfg in [
        RetrievalConfig(top_k=64, bfs_max_hops=2, time_decay_lambda=LAM, max_results_returned=2000),
        RetrievalConfig(top_k=1, bfs_max_hops=3, time_decay_lambda=LAM),
        RetrievalConfig(top_k=10, bfs_max_hops=0, time_decay_lambda=LAM),
        RetrievalConfig(top_k=10, bfs_max_hops=2, time_decay_lambda=1e-8, modality_filter=0),
        RetrievalConfig(top_k=10, bfs_max_hops=2, time_decay_lambda=LAM, query_episode_id=17,
                        episode_same_boost=0.5),
        RetrievalConfig(top_k=200, bfs_max_hops=1, time_decay_lambda=LAM, bfs_score_decay=0.85),
    ]:
        check_global(dev10k, q, cfg)


def test_episode_parity_10k(dev10k, corpus_10k):
    qs = corpus.pick_queries(corpus_10k.modalities, 100, seed=202)
    off = dev10k.csr.ep_csr_offsets
    for i, node in enumerate(qs):
        ep = int(corpus_10k.episode_ids[node])
        k = 15 if i % 2 else 10          # K > M=10 exercises the reference padding
        cfg = RetrievalConfig(top_k=k, time_decay_lambda=LAM, max_results_returned=15,
                              retrieval_scope=RetrievalScope.EpisodeScoped, query_episode_id=ep,
                              query_episode_member_begin=int(off[ep]),
                              query_episode_member_count=int(off[ep + 1] - off[ep]))
        res, st = dev10k.query(corpus_10k.embeddings[node], cfg)
        assert st.scope_fallback == 0 and st.nodes_scanned == 10 and st.bfs_waves == 0
        check_episode_results(dev10k, corpus_10k.embeddings[node], cfg, res)
        # published outcome: episode-scoped retrieval returns the episode's TEXT and AUDIO
        mods = {r.modality for r in res if corpus_10k.episode_ids[r.node_id] == ep}
        assert {0, 1} <= mods


def test_episode_invalid_range_falls_back(dev10k, corpus_10k):
    cfg = RetrievalConfig(top_k=10, time_decay_lambda=LAM, retrieval_scope=RetrievalScope.EpisodeScoped,
                          query_episode_id=3, query_episode_member_begin=9990, query_episode_member_count=50)
    res, st = dev10k.query(corpus_10k.embeddings[30], cfg)
    assert st.scope_fallback == 1 and st.nodes_scanned == 10000 and len(res) == 10


def test_fp16_parity_10k(dev10k, corpus_10k):
    emb16 = oracle.to_f16_bits(corpus_10k.embeddings)
    dev10k.ctx.use_fp16 = True
    try:
        cfg = RetrievalConfig(top_k=10, bfs_max_hops=2, time_decay_lambda=LAM, max_results_returned=15)
        for node in corpus.pick_queries(corpus_10k.modalities, 20, seed=303):
            q = corpus_10k.embeddings[node]
            check_global(dev10k, q, cfg, emb16=emb16)
            res, st = dev10k.query(q, cfg)
            assert st.used_fp16 == 1
            # fp16 path against the fp32 oracle
            fin32, scale = oracle.scores(dev10k.og, q, T_Q, LAM)
            check_scores(dev10k.ctx.last_scores(dev10k.n), fin32, scale, RTOL_F16_VS_F32)
    finally:
        dev10k.ctx.use_fp16 = False


def test_repeat_query_is_stable(dev10k, corpus_10k):
    cfg = RetrievalConfig(top_k=10, time_decay_lambda=LAM, max_results_returned=50)
    a, _ = dev10k.query(corpus_10k.embeddings[40], cfg)
    b, _ = dev10k.query(corpus_10k.embeddings[1240], cfg)
    c, _ = dev10k.query(corpus_10k.embeddings[40], cfg)
    assert a == c and a != b


def test_device_query_pointer(dev10k, corpus_10k):
    q = corpus_10k.embeddings[1234]
    cfg = RetrievalConfig(top_k=10, time_decay_lambda=LAM, max_results_returned=15)
    host, _ = dev10k.query(q, cfg)
    buf = mars_amd.DeviceBuffer.from_array(q)
    np.testing.assert_array_equal(buf.to_array(np.float32, q.size), q)
    dev_res = mars_amd.query_memory_fast_device(dev10k.dg, dev10k.ctx, buf.ptr, T_Q, cfg)
    buf.free()
    assert host == dev_res


def test_result_counts_up_to_the_compaction_cap(rng):
    """max_results_returned above one LDS sort (8,192): results go out in sorted bands, up to
    the reference's compaction cap min(max_nodes, max_k * 500) (memory_cuda.cu:1059); a
    larger request returns that many, as the reference's compaction truncates there."""
    emb, mods, ts, row, col, ep = random_graph(rng, 40000, 128, deg=5)
    dev = Dev(emb, mods, ts, row, col, ep)
    try:
        cfg = RetrievalConfig(top_k=10, bfs_max_hops=4, time_decay_lambda=LAM, max_results_returned=20000)
        res = check_global(dev, emb[7], cfg)
        assert len(res) == 20000
        _, st = dev.query(emb[7], cfg)
        assert st.visited > 32000 and st.results_capped == 0   # 20,000 asked, below the cap
        big = RetrievalConfig(top_k=8, bfs_max_hops=4, time_decay_lambda=LAM, max_results_returned=39000)
        res, st = dev.query(emb[7], big)
        assert len(res) == 32000                               # 64 * 500
        assert st.results_capped == 1                          # the cap cut the results
        small_ctx = mars_amd.create_query_context(dev.n, dev.d, 8)   # cap 8 * 500; K = 8 on both
        try:
            st8 = mars_amd.RetrievalStats()
            res8 = mars_amd.query_memory_fast(dev.dg, small_ctx, emb[7], T_Q, big, st8)
            assert len(res8) == 4000 and res8 == res[:4000] and st8.results_capped == 1
            # above the cap, but the visit set fits in it: nothing was cut
            few = RetrievalConfig(top_k=8, bfs_max_hops=1, time_decay_lambda=LAM, max_results_returned=39000)
            resf = mars_amd.query_memory_fast(dev.dg, small_ctx, emb[7], T_Q, few, st8)
            assert st8.results_capped == 0 and len(resf) == st8.visited < 4000
        finally:
            mars_amd.destroy_query_context(small_ctx)
    finally:
        dev.close()


# ---------------------------------------------------------------- the reference's own corpus
def test_reference_kids_corpus(golden):
    z = np.load(golden / "kids_small.npz")
    dev = Dev(z["emb"], z["mods"], z["ts"], z["row"], z["col"], z["ep"])
    try:
        img = np.nonzero(z["mods"] == 2)[0]
        off = dev.csr.ep_csr_offsets
        for node in img[:30]:
            q, t = z["emb"][node], float(z["ts"][node])
            ep = int(z["ep"][node])
            cfg = RetrievalConfig(top_k=15, time_decay_lambda=8e-6, bfs_score_decay=0.55,
                                  max_results_returned=15)
            res, st = dev.query(q, cfg, t_q=t)
            ref = oracle.query(dev.og, q, t, ocfg(cfg), seeds_in=dev.ctx.last_seeds()[0])
            ids, hops, _ = dev.ctx.last_visited()
            assert st.visited == ref["visited"] == len(ids)
            cfg_s = RetrievalConfig(top_k=15, time_decay_lambda=8e-6, max_results_returned=15,
                                    retrieval_scope=RetrievalScope.EpisodeScoped, query_episode_id=ep,
                                    query_episode_member_begin=int(off[ep]),
                                    query_episode_member_count=int(off[ep + 1] - off[ep]))
            res, st = dev.query(q, cfg_s, t_q=t)
            ref = oracle.query(dev.og, q, t, ocfg(cfg_s))
            assert [r.node_id for r in res] == [w[0] for w in ref["results"]]
            mods = {r.modality for r in res if z["ep"][r.node_id] == ep}
            assert {0, 1} <= mods                           # published episode hit@15 = 1.0
    finally:
        dev.close()


# ---------------------------------------------------------------- shapes and edge cases
@pytest.mark.parametrize("n,d", [(5, 768), (300, 100), (3000, 384), (2000, 1024), (777, 256), (1500, 64)])
def test_shapes(n, d, rng):
    """Global queries at several dimensions, and episode-scoped ones through each episode
    kernel variant (register-fragment rows for d = 256 / 384 / 768, the loop otherwise)."""
    emb, mods, ts, row, col, ep = random_graph(rng, n, d)
    dev = Dev(emb, mods, ts, row, col, ep, fp16=True)
    try:
        for node in (0, n // 2, n - 1):
            check_global(dev, emb[node], RetrievalConfig(top_k=10, time_decay_lambda=LAM, max_results_returned=20))
            check_episode(dev, emb[node], int(ep[node]), 10)
        dev.ctx.use_fp16 = True
        e16 = oracle.to_f16_bits(emb)
        check_global(dev, emb[1], RetrievalConfig(top_k=10, time_decay_lambda=LAM), emb16=e16)
    finally:
        dev.close()


def test_no_edges_graph(rng):
    n, d = 500, 128
    emb = rng.standard_normal((n, d)).astype(np.float32)
    emb /= np.linalg.norm(emb, axis=1, keepdims=True)
    dev = Dev(emb, np.zeros(n, np.int32), np.zeros(n, np.float32), None, None)
    try:
        res = check_global(dev, emb[3], RetrievalConfig(top_k=10, time_decay_lambda=LAM, max_results_returned=30))
        assert len(res) == 10 and res[0].node_id == 3 and all(r.hops_from_seed == 0 for r in res)
    finally:
        dev.close()


def test_large_frontier_and_visited(rng):
    """Hubs: the level-1 frontier exceeds one LDS chunk (4096) and the visited set
    exceeds the LDS sort (8192), exercising the chunked BFS and radix-select path."""
    n, d = 60000, 64
    emb = rng.standard_normal((n, d)).astype(np.float32)
    emb /= np.linalg.norm(emb, axis=1, keepdims=True)
    q = emb[0]
    hubs = np.argsort(-(emb @ q))[:10]
    edges = [(int(h), int(t)) for h in hubs for t in rng.choice(n, 800, replace=False)]
    edges += [(int(a), int(b)) for a, b in rng.integers(0, n, size=(60000, 2))]
    adj = [set() for _ in range(n)]
    for a, b in edges:
        if a != b:
            adj[a].add(b)
            adj[b].add(a)
    row = np.zeros(n + 1, np.int32)
    row[1:] = np.cumsum([len(s) for s in adj])
    col = np.concatenate([np.array(sorted(s), np.int32) for s in adj])
    # every memory at the query time: no decay, so the seeds are exactly the hubs
    dev = Dev(emb, rng.integers(0, 3, n).astype(np.int32), np.full(n, T_Q, np.float32), row, col)
    try:
        cfg = RetrievalConfig(top_k=10, bfs_max_hops=2, time_decay_lambda=LAM, max_results_returned=5000)
        check_global(dev, q, cfg)
        _, st = dev.query(q, cfg)
        assert st.visited > 8192
    finally:
        dev.close()


# ---------------------------------------------------------------- batched MFMA scoring
def test_batch_parity_q64(dev10k, corpus_10k):
    qn = corpus.pick_queries(corpus_10k.modalities, 64, seed=404)
    batch_check(dev10k, qn, RetrievalConfig(top_k=10, time_decay_lambda=LAM), T_Q, corpus_10k.embeddings)


@pytest.mark.parametrize("q,k,filt", [(1, 10, -1), (200, 16, -1), (130, 5, 1), (64, 16, 2), (520, 16, -1),
                                       (600, 10, 2)])
def test_batch_parity_shapes(dev10k, corpus_10k, q, k, filt, rng):
    qn = corpus.pick_queries(corpus_10k.modalities, q, seed=q)
    tq = rng.uniform(400, 600, size=q).astype(np.float32)             # per-query times
    batch_check(dev10k, qn, RetrievalConfig(top_k=k, time_decay_lambda=LAM, modality_filter=filt), tq,
                 corpus_10k.embeddings)


@pytest.mark.parametrize("d,k,filt,uniform", [(256, 5, -1, False), (384, 16, 1, True), (512, 8, 2, False),
                                               (768, 3, -1, True)])
def test_batch_tiled_widths(d, k, filt, uniform, rng):
    """1,030 queries (k_batch_rq, five groups of 256 queries per row range, the last with six):
    every supported width, both list sizes (K <= 8 and K <= 16), ragged row tiles (2,600
    rows), filters and per-query times, against the oracle's top-K."""
    n = 2600
    emb, mods, ts, row, col, _ = random_graph(rng, n, d)
    dev = Dev(emb, mods, ts, row, col, fp16=True)
    try:
        qn = rng.choice(n, 1030, replace=False)
        tq = np.float32(T_Q) if uniform else rng.uniform(300, 600, 1030).astype(np.float32)
        batch_check(dev, qn, RetrievalConfig(top_k=k, time_decay_lambda=LAM, modality_filter=filt), tq, emb)
    finally:
        dev.close()


@pytest.mark.parametrize("n,k,filt,uniform,lam", [(60_000, 10, -1, True, LAM), (60_000, 16, 1, False, LAM),
                                                   (110_000, 4, -1, False, 0.0), (110_000, 8, 2, True, LAM),
                                                   (110_000, 16, -1, False, LAM)])
def test_batch_tiled_long_ranges(n, k, filt, uniform, lam, rng):
    """Batches of 1,030 fused-score queries over long row ranges (k_batch_rq): 60,000 rows
    without the sampled pass, 110,000 rows with it (its floors drop rows from the first
    tile on); decay per query and per batch, no decay, filters. A quarter of the queries
    and the six of the last, partial query group are checked against the oracle's top-K."""
    d, q = 256, 1030
    emb, mods, ts, row, col, _ = random_graph(rng, n, d)
    dev = Dev(emb, mods, ts, row, col, fp16=True)
    try:
        qs = emb[rng.choice(n, q, replace=False)]
        tq = np.full(q, T_Q, np.float32) if uniform else rng.uniform(300, 600, q).astype(np.float32)
        cfg = RetrievalConfig(top_k=k, time_decay_lambda=lam, modality_filter=filt)
        buf = mars_amd.DeviceBuffer.from_array(qs)
        try:
            ids, sc = mars_amd.query_batch(dev.dg, dev.ctx, buf.ptr, q, tq if not uniform else np.float32(T_Q), cfg)
        finally:
            buf.free()
        check_batch_topk(dev.og, qs, tq, cfg, ids, sc, n, check_rows=list(range(0, 1024, 4)) + list(range(1024, q)))
    finally:
        dev.close()


@pytest.mark.parametrize("d", [256, 384, 512])
def test_knn_tiled_widths(d, rng):
    """The k-NN builder (plain dot products, the node itself excluded) at the other widths
    against the exact CPU k-NN: the first 1,024 nodes through k_batch_mm, the other 476
    through k_batch_rq; differing neighbours must be near-ties with the 8th."""
    n = 1500
    emb, mods, ts, _, _, _ = random_graph(rng, n, d)
    dev = Dev(emb, mods, ts, None, None, fp16=True)
    try:
        got = mars_amd.graph_knn(dev.dg, 8)
        want, sims = corpus.knn_cpu(emb, 8)
        s = emb @ emb.T
        np.fill_diagonal(s, -np.inf)
        mism = 0
        for i in range(n):
            if not np.array_equal(got[i], want[i]):
                mism += 1
                for j in set(got[i].tolist()) ^ set(want[i].tolist()):
                    assert abs(s[i, j] - sims[i, 7]) <= 1e-3, (i, j)
        assert mism <= 0.02 * n
        assert np.all(got != np.arange(n)[:, None])
    finally:
        dev.close()


def test_batch_matches_single_query_seeds(dev10k, corpus_10k):
    """The batched seeds agree with the Q=1 fp16 path's seeds up to fp16 near-ties."""
    qn = corpus.pick_queries(corpus_10k.modalities, 32, seed=505)
    cfg = RetrievalConfig(top_k=10, time_decay_lambda=LAM)
    ids, _ = batch_check(dev10k, qn, cfg, T_Q, corpus_10k.embeddings)
    dev10k.ctx.use_fp16 = True
    try:
        agree = 0
        for i, node in enumerate(qn):
            dev10k.query(corpus_10k.embeddings[node], cfg)
            seeds, _ = dev10k.ctx.last_seeds()
            agree += len(set(seeds.tolist()) & set(ids[i].tolist()))
        assert agree >= 0.98 * 10 * len(qn)
    finally:
        dev10k.ctx.use_fp16 = False


def test_gpu_knn_matches_cpu_exact():
    c = corpus.make_corpus(6000, 768, seed=31)
    dev = Dev(c.embeddings, c.modalities, c.timestamps, None, None, fp16=True)
    try:
        got = mars_amd.graph_knn(dev.dg, 8)
        want, sims = corpus.knn_cpu(c.embeddings, 8)
        s = c.embeddings @ c.embeddings.T
        np.fill_diagonal(s, -np.inf)
        mism = 0
        for i in range(c.num_nodes):
            if not np.array_equal(got[i], want[i]):
                mism += 1
                # every differing neighbour is a near-tie with the 8th exact score
                for j in set(got[i].tolist()) ^ set(want[i].tolist()):
                    assert abs(s[i, j] - sims[i, 7]) <= 1e-5, (i, j)
        assert mism <= 0.01 * c.num_nodes
        assert np.all(got != np.arange(c.num_nodes)[:, None])
        # blocks of 1,700 ids (the last one ragged): one call, and block by block
        whole = mars_amd.graph_knn(dev.dg, 8, 1700)
        seen = []
        parts = mars_amd.graph_knn(dev.dg, 8, 1700, progress=lambda d, t: seen.append((d, t)))
        np.testing.assert_array_equal(parts, whole)
        assert seen == [(1, 4), (2, 4), (3, 4), (4, 4)]
        blk = np.arange(c.num_nodes) // 1700
        assert np.all(blk[whole] == blk[:, None])          # neighbours within the node's block
        # the all-pairs build in query ranges (ragged last range) and in pieces with progress
        n = c.num_nodes
        ranged = np.concatenate([mars_amd.graph_knn_range(dev.dg, 8, a, min(1000, n - a)) for a in range(0, n, 1000)])
        np.testing.assert_array_equal(ranged, got)
        seen = []
        pieced = mars_amd.graph_knn(dev.dg, 8, 0, progress=lambda d, t: seen.append((d, t)), piece=2500)
        np.testing.assert_array_equal(pieced, got)
        assert seen == [(1, 3), (2, 3), (3, 3)]
        assert mars_amd.graph_knn_range(dev.dg, 8, n, 0).shape == (0, 8)
        from mars_amd._lib import MarsError
        with pytest.raises(MarsError) as e:
            mars_amd.graph_knn_range(dev.dg, 8, n - 10, 20)
        assert e.value.code == -1
    finally:
        dev.close()


# ---------------------------------------------------------------- replayed query graphs
def test_graph_replay_matches_eager(dev10k, corpus_10k):
    """Replays of the query graph (arguments rewritten per query) interleaved with
    eager queries: every replay returns exactly the eager result, and each replay is
    checked against the oracle (scores, seeds, BFS and results for global queries; ids
    and scores for episode-scoped ones). A filtered, boosted global query between plain
    ones switches the scan kernel variant, so the graph is rebuilt rather than replayed
    with the wrong kernel. The query time changes between replays, which the reference's
    recapture key misses (memory_cuda.cu:1375-1385)."""
    qs = corpus.pick_queries(corpus_10k.modalities, 24, seed=606)
    emb16 = oracle.to_f16_bits(corpus_10k.embeddings)
    try:
        for fp16 in (False, True):
            dev10k.ctx.use_fp16 = fp16
            for i, node in enumerate(qs):
                ep = int(corpus_10k.episode_ids[node])
                q = corpus_10k.embeddings[node]
                cfgs = [RetrievalConfig(top_k=10, time_decay_lambda=LAM, max_results_returned=15),
                        RetrievalConfig(top_k=10, time_decay_lambda=LAM, max_results_returned=15,
                                        modality_filter=int(corpus_10k.modalities[node]), query_episode_id=ep,
                                        episode_same_boost=0.5),
                        episode_cfg(dev10k.csr, ep, 10, 15)]
                for cfg in cfgs:
                    t = T_Q - 5.0 * (i % 3)                   # the query time changes between replays
                    dev10k.ctx.use_cuda_graph = False
                    eager, _ = dev10k.query(q, cfg, t_q=t)
                    dev10k.ctx.use_cuda_graph = True
                    replay, _ = dev10k.query(q, cfg, t_q=t)
                    replay2, st2 = dev10k.query(q, cfg, t_q=t)
                    assert replay == eager and replay2 == eager, (fp16, i, cfg.retrieval_scope)
                    if i % 4:                                 # the oracle on every fourth query
                        continue
                    if cfg.retrieval_scope == RetrievalScope.EpisodeScoped:   # fp32 rows on both paths
                        check_episode_results(dev10k, q, cfg, replay2, t_q=t)
                    else:
                        check_global(dev10k, q, cfg, emb16=emb16 if fp16 else None, t_q=t, res=replay2, st=st2)
    finally:
        dev10k.ctx.use_cuda_graph = False
        dev10k.ctx.use_fp16 = False


def test_completion_word_matches_stream_sync(dev10k, corpus_10k):
    """Queries that complete through the host-mapped completion word (the default) and
    ones that synchronise the stream (MARS_CTX_TIMING) return the same results, and the
    debug readers see the polled query's state."""
    qs = corpus.pick_queries(corpus_10k.modalities, 12, seed=607)
    off = dev10k.csr.ep_csr_offsets
    try:
        for certified in (False, True):
            dev10k.ctx.certified = certified
            for node in qs:
                ep = int(corpus_10k.episode_ids[node])
                for cfg in (RetrievalConfig(top_k=10, time_decay_lambda=LAM, max_results_returned=100),
                            RetrievalConfig(top_k=10, time_decay_lambda=LAM,
                                            retrieval_scope=RetrievalScope.EpisodeScoped, query_episode_id=ep,
                                            query_episode_member_begin=int(off[ep]),
                                            query_episode_member_count=int(off[ep + 1] - off[ep]))):
                    dev10k.ctx.timing = True
                    synced, _ = dev10k.query(corpus_10k.embeddings[node], cfg)
                    dev10k.ctx.timing = False
                    polled, _ = dev10k.query(corpus_10k.embeddings[node], cfg)
                    assert polled == synced
        dev10k.ctx.certified = False
        res, _ = dev10k.query(corpus_10k.embeddings[qs[0]], RetrievalConfig(top_k=10, time_decay_lambda=LAM))
        ids, hops, scores = dev10k.ctx.last_visited()
        assert len(ids) >= len(res) and set(r.node_id for r in res) <= set(int(i) for i in ids)
    finally:
        dev10k.ctx.timing = False
        dev10k.ctx.certified = False


def test_read_ceiling(rng):
    """The streaming-read ceiling of a graph's rows: positive and below the HBM peak for
    fp32 and fp16 rows, and for the four access patterns; MARS_ERR_INVALID for an unknown
    pattern; MARS_ERR_UNSUPPORTED once the fp16 and int8 copies are gone."""
    from mars_amd._lib import MarsError
    emb, mods, ts, row, col, ep = random_graph(rng, 40000, 768)
    dev = Dev(emb, mods, ts, row, col, ep, fp16=True)
    mars_amd.upload_int8_embeddings(dev.dg)
    try:
        for fp16 in (False, True):
            gbs = mars_amd.read_ceiling(dev.dg, fp16=fp16, reps=3)
            assert 0.0 < gbs < 8000.0 * 1.1, (fp16, gbs)
        for pattern in (mars_amd.READ_STREAM, mars_amd.READ_FRAGMENTS, mars_amd.READ_FRAGMENTS_NT,
                        mars_amd.READ_STREAM_INT8):
            gbs = mars_amd.read_pattern(dev.dg, pattern, reps=3)
            assert 0.0 < gbs < 8000.0 * 1.1, (pattern, gbs)
        with pytest.raises(MarsError) as e:
            mars_amd.read_pattern(dev.dg, 4)
        assert e.value.code == -1
        mars_amd.free_fp16_embeddings(dev.dg)
        mars_amd.free_int8_embeddings(dev.dg)
        for call in (lambda: mars_amd.read_ceiling(dev.dg, fp16=True),
                     lambda: mars_amd.read_pattern(dev.dg, mars_amd.READ_FRAGMENTS),
                     lambda: mars_amd.read_pattern(dev.dg, mars_amd.READ_STREAM_INT8)):
            with pytest.raises(MarsError) as e:
                call()
            assert e.value.code == -5
    finally:
        dev.close()
