"""GPU parity: the HIP path (through the C ABI) against the CPU oracle on the
same seeded inputs.

Bars (written here as the tests apply them):
  * fused scores:  |gpu - oracle| <= 1e-5 * max(|oracle|, w * sum|e q|)  (fp32; fp16 rows
                   against the oracle on the same RNE-rounded rows), and <= 2e-3 of the
                   same scale for the fp16 path against the fp32 oracle;
  * seeds / results: identical id sets except ids whose oracle score lies within
                   that tolerance of the cut;
  * BFS given the GPU's seeds: visit order (ids), hop levels and visited count
                   bit-exact; BFS scores within the score tolerance;
  * episode CSR / episode-scoped results: ids and hops exact.
"""
from __future__ import annotations

import numpy as np
import pytest

import mars_amd
import oracle
from mars_amd import RetrievalConfig, RetrievalScope, corpus

from conftest import RTOL_F16_VS_F32, RTOL_F32

pytestmark = pytest.mark.gpu
FLT_MAX = float(np.finfo(np.float32).max)
T_Q = corpus.QUERY_TIME
LAM = corpus.DECAY_LAMBDA


class Dev:
    def __init__(self, emb, mods, ts, row, col, ep=None, max_k=64, fp16=False):
        self.n, self.d = emb.shape
        g = mars_amd.MemoryGraph(self.n, self.d, row, col, emb, mods, ts)
        self.dg = mars_amd.upload_to_device(g)
        self.csr = None
        if ep is not None:
            mars_amd.upload_episode_ids(self.dg, ep)
            self.csr = mars_amd.build_episode_csr(ep, self.n)
            mars_amd.upload_episode_csr(self.dg, self.csr)
        if fp16:
            mars_amd.upload_fp16_embeddings(self.dg)
        self.ctx = mars_amd.create_query_context(self.n, self.d, max_k)
        self.og = oracle.make_graph(emb, mods, ts, row, col, ep)

    def close(self):
        mars_amd.destroy_query_context(self.ctx)
        mars_amd.free_device(self.dg)

    def query(self, q, cfg, t_q=T_Q):
        st = mars_amd.RetrievalStats()
        res = mars_amd.query_memory_fast(self.dg, self.ctx, q, t_q, cfg, st)
        return res, st


def ocfg(cfg: RetrievalConfig):
    return oracle.config(cfg.top_k, cfg.bfs_max_hops, cfg.time_decay_lambda, cfg.bfs_score_decay,
                         cfg.modality_filter, cfg.max_results_returned, int(cfg.retrieval_scope),
                         cfg.query_episode_id, cfg.query_episode_member_begin, cfg.query_episode_member_count,
                         cfg.episode_same_boost)


def check_scores(gpu, ref, scale, rtol):
    bound = rtol * np.maximum(np.abs(ref), scale) + 1e-30
    filt = ref == -FLT_MAX
    assert np.all(gpu[filt] == np.float32(-FLT_MAX))
    err = np.abs(gpu[~filt].astype(np.float64) - ref[~filt])
    worst = np.max(err / bound[~filt]) if err.size else 0.0
    assert worst <= 1.0, f"score error {worst:.3f}x the bound"


def check_global(dev: Dev, q, cfg: RetrievalConfig, emb16=None, rtol=RTOL_F32):
    """Full global-query parity for one query; returns the GPU results."""
    res, st = dev.query(q, cfg)
    assert st.scope_fallback == 0 or cfg.retrieval_scope == RetrievalScope.EpisodeScoped
    og = dev.og
    if emb16 is not None:
        og = oracle.Graph(og.embeddings, og.modalities, og.timestamps, og.row_offsets, og.col_indices,
                          og.episode_ids, og.ep_offsets, og.ep_members, emb16)
    ref = oracle.query(og, q, T_Q, ocfg(cfg))
    fin_ref = ref["final"]
    _, scale = oracle.scores(og, q, T_Q, cfg.time_decay_lambda, cfg.modality_filter)
    tol = rtol * np.maximum(np.abs(fin_ref), scale)
    # 1) fused scores over all N
    fin_gpu = dev.ctx.last_scores(dev.n)
    if cfg.episode_same_boost > 0:
        scale = scale * (1.0 + cfg.episode_same_boost)
    check_scores(fin_gpu, fin_ref, scale, rtol)
    # 2) seeds: same set up to near-ties at the K-th score
    seeds, seed_vals = dev.ctx.last_seeds()
    k = ref["k"]
    assert len(seeds) == min(k, dev.n)
    kth = fin_ref[ref["seeds"][-1]]
    diff = set(seeds.tolist()) ^ set(ref["seeds"].tolist())
    assert all(abs(fin_ref[i] - kth) <= 2 * tol[i] + 2 * tol[ref["seeds"][-1]] for i in diff), diff
    np.testing.assert_array_equal(seed_vals, fin_gpu[seeds])
    # seeds come out in (score desc, id asc) order of the GPU's own scores
    order = np.lexsort((seeds, -seed_vals.astype(np.float64)))
    np.testing.assert_array_equal(order, np.arange(len(seeds)))
    # 3) BFS from the GPU's seeds: visit order / hops exact, scores in tolerance
    ids, hops, vsc = dev.ctx.last_visited()
    b = oracle.bfs(og.row_offsets, og.col_indices, fin_ref, seeds, fin_ref[seeds],
                   max(0, cfg.bfs_max_hops), cfg.bfs_score_decay)
    np.testing.assert_array_equal(ids, b["ids"])
    np.testing.assert_array_equal(hops, b["hops"])
    vtol = rtol * np.maximum(np.abs(b["scores"]), np.max(scale)) + 1e-30
    assert np.all(np.abs(vsc - b["scores"]) <= vtol)
    assert st.visited == len(ids)
    # 4) final results: oracle given the same seeds
    r2 = oracle.query(og, q, T_Q, ocfg(cfg), seeds_in=seeds)
    want = r2["results"]
    assert len(res) == len(want) == r2["n_results"]
    vis_score = dict(zip(b["ids"].tolist(), b["scores"].tolist()))
    vis_hop = dict(zip(b["ids"].tolist(), b["hops"].tolist()))
    for j, (r, w) in enumerate(zip(res, want)):
        if r.node_id != w[0]:
            assert abs(vis_score[r.node_id] - w[1]) <= 2 * RTOL_F32 * max(abs(w[1]), 1.0), (j, r, w)
        assert r.hops_from_seed == vis_hop[r.node_id]
        assert r.modality == int(dev.og.modalities[r.node_id])
        assert abs(r.score - vis_score[r.node_id]) <= rtol * max(abs(vis_score[r.node_id]), 1.0)
    return res


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
        ref = oracle.query(dev10k.og, corpus_10k.embeddings[node], T_Q, ocfg(cfg))
        assert ref["scoped"]
        assert [r.node_id for r in res] == [w[0] for w in ref["results"]]
        assert all(r.hops_from_seed == 0 for r in res)
        for r, w in zip(res, ref["results"]):
            if w[1] == -FLT_MAX:
                assert r.score == np.float32(-FLT_MAX)
            else:
                assert abs(r.score - w[1]) <= RTOL_F32 * max(abs(w[1]), 1.0)
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


def test_unsupported_result_count(dev10k, corpus_10k):
    cfg = RetrievalConfig(top_k=10, max_results_returned=9000)
    with pytest.raises(mars_amd.MarsError, match="MARS_ERR_UNSUPPORTED"):
        dev10k.query(corpus_10k.embeddings[0], cfg)


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
def _random_graph(rng, n, d, deg=6, n_ep=None):
    emb = rng.standard_normal((n, d)).astype(np.float32)
    emb /= np.linalg.norm(emb, axis=1, keepdims=True)
    mods = rng.integers(0, 3, size=n).astype(np.int32)
    ts = rng.uniform(0, 600, size=n).astype(np.float32)
    ep = (np.arange(n) // 10).astype(np.int32) if n_ep is None else np.sort(rng.integers(0, n_ep, n)).astype(np.int32)
    knn = rng.integers(0, n, size=(n, deg)).astype(np.int32)
    row, col = corpus.build_nsn_csr(ep, knn)
    return emb, mods, ts, row, col, ep


def check_episode(dev, q, ep, k):
    """Episode-scoped query against the oracle (ids exact, scores to the fp32 bar)."""
    off = dev.csr.ep_csr_offsets
    cfg = RetrievalConfig(top_k=k, time_decay_lambda=LAM, max_results_returned=k,
                          retrieval_scope=RetrievalScope.EpisodeScoped, query_episode_id=ep,
                          query_episode_member_begin=int(off[ep]),
                          query_episode_member_count=int(off[ep + 1] - off[ep]))
    res, st = dev.query(q, cfg)
    ref = oracle.query(dev.og, q, T_Q, ocfg(cfg))
    assert ref["scoped"] and st.scope_fallback == 0
    assert [r.node_id for r in res] == [w[0] for w in ref["results"]]
    for r, w in zip(res, ref["results"]):
        if w[1] == -FLT_MAX:
            assert r.score == np.float32(-FLT_MAX)
        else:
            assert abs(r.score - w[1]) <= RTOL_F32 * max(abs(w[1]), 1.0)


@pytest.mark.parametrize("n,d", [(5, 768), (300, 100), (3000, 384), (2000, 1024), (777, 256), (1500, 64)])
def test_shapes(n, d, rng):
    """Global queries at several dimensions, and episode-scoped ones through each episode
    kernel variant (register-fragment rows for d = 256 / 384 / 768, the loop otherwise)."""
    emb, mods, ts, row, col, ep = _random_graph(rng, n, d)
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
def _batch_check(dev: Dev, qnodes, cfg, t_q, emb):
    qs = emb[qnodes]
    buf = mars_amd.DeviceBuffer.from_array(qs)
    try:
        ids, sc = mars_amd.query_batch(dev.dg, dev.ctx, buf.ptr, len(qnodes), t_q, cfg)
    finally:
        buf.free()
    tq = np.broadcast_to(np.asarray(t_q, np.float32), (len(qnodes),))
    k = cfg.top_k
    for i in range(len(qnodes)):
        fin, scale = oracle.scores(dev.og, qs[i], float(tq[i]), cfg.time_decay_lambda, cfg.modality_filter)
        want, _ = oracle.topk(fin, k)
        tol = RTOL_F16_VS_F32 * np.maximum(np.abs(fin), scale)
        got = ids[i][ids[i] >= 0]
        assert len(got) == min(k, dev.n)
        ok = fin[got] != -FLT_MAX
        assert np.all(np.abs(sc[i][: len(got)][ok] - fin[got][ok]) <= tol[got][ok])
        kth = fin[want[-1]]
        for j in set(got.tolist()) ^ set(want.tolist()):
            assert abs(fin[j] - kth) <= 2 * (tol[j] + tol[want[-1]]), (i, j)
        assert np.all(np.diff(sc[i][: len(got)].astype(np.float64)) <= 0)      # sorted desc
    return ids, sc


def test_batch_parity_q64(dev10k, corpus_10k):
    qn = corpus.pick_queries(corpus_10k.modalities, 64, seed=404)
    _batch_check(dev10k, qn, RetrievalConfig(top_k=10, time_decay_lambda=LAM), T_Q, corpus_10k.embeddings)


@pytest.mark.parametrize("q,k,filt", [(1, 10, -1), (200, 16, -1), (130, 5, 1), (64, 16, 2), (520, 16, -1),
                                       (600, 10, 2)])
def test_batch_parity_shapes(dev10k, corpus_10k, q, k, filt, rng):
    qn = corpus.pick_queries(corpus_10k.modalities, q, seed=q)
    tq = rng.uniform(400, 600, size=q).astype(np.float32)             # per-query times
    _batch_check(dev10k, qn, RetrievalConfig(top_k=k, time_decay_lambda=LAM, modality_filter=filt), tq,
                 corpus_10k.embeddings)


def test_batch_matches_single_query_seeds(dev10k, corpus_10k):
    """The batched seeds agree with the Q=1 fp16 path's seeds up to fp16 near-ties."""
    qn = corpus.pick_queries(corpus_10k.modalities, 32, seed=505)
    cfg = RetrievalConfig(top_k=10, time_decay_lambda=LAM)
    ids, _ = _batch_check(dev10k, qn, cfg, T_Q, corpus_10k.embeddings)
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
    finally:
        dev.close()


# ---------------------------------------------------------------- replayed query graphs
def test_graph_replay_matches_eager(dev10k, corpus_10k):
    """Replays of the query graph (arguments rewritten per query) interleaved with
    eager queries: every replay returns exactly the eager result. A filtered,
    boosted global query between plain ones switches the scan kernel variant, so the
    graph is rebuilt rather than replayed with the wrong kernel."""
    qs = corpus.pick_queries(corpus_10k.modalities, 24, seed=606)
    off = dev10k.csr.ep_csr_offsets
    try:
        for fp16 in (False, True):
            dev10k.ctx.use_fp16 = fp16
            for i, node in enumerate(qs):
                ep = int(corpus_10k.episode_ids[node])
                cfgs = [RetrievalConfig(top_k=10, time_decay_lambda=LAM, max_results_returned=15),
                        RetrievalConfig(top_k=10, time_decay_lambda=LAM, max_results_returned=15,
                                        modality_filter=int(corpus_10k.modalities[node]), query_episode_id=ep,
                                        episode_same_boost=0.5),
                        RetrievalConfig(top_k=10, time_decay_lambda=LAM, max_results_returned=15,
                                        retrieval_scope=RetrievalScope.EpisodeScoped, query_episode_id=ep,
                                        query_episode_member_begin=int(off[ep]),
                                        query_episode_member_count=int(off[ep + 1] - off[ep]))]
                for cfg in cfgs:
                    t = T_Q - 5.0 * (i % 3)                   # the query time changes between replays
                    dev10k.ctx.use_cuda_graph = False
                    eager, _ = dev10k.query(corpus_10k.embeddings[node], cfg, t_q=t)
                    dev10k.ctx.use_cuda_graph = True
                    replay, _ = dev10k.query(corpus_10k.embeddings[node], cfg, t_q=t)
                    replay2, _ = dev10k.query(corpus_10k.embeddings[node], cfg, t_q=t)
                    assert replay == eager and replay2 == eager, (fp16, i, cfg.retrieval_scope)
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
    fp32 and fp16 rows; MARS_ERR_UNSUPPORTED once the fp16 copy is gone."""
    from mars_amd._lib import MarsError
    emb, mods, ts, row, col, ep = _random_graph(rng, 40000, 768)
    dev = Dev(emb, mods, ts, row, col, ep, fp16=True)
    try:
        for fp16 in (False, True):
            gbs = mars_amd.read_ceiling(dev.dg, fp16=fp16, reps=3)
            assert 0.0 < gbs < 8000.0 * 1.1, (fp16, gbs)
        mars_amd.free_fp16_embeddings(dev.dg)
        with pytest.raises(MarsError) as e:
            mars_amd.read_ceiling(dev.dg, fp16=True)
        assert e.value.code == -5
    finally:
        dev.close()
