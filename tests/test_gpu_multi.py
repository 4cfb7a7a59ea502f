"""Batched global queries (mars_query_global_batch through the C ABI).

Bar: every query's results (ids, scores, modalities, hops, order, count) are
bit-identical to the Q=1 global path's (mars_query_device on the same device
vector), whichever way the batch answered it: shared fp16 scan + certified
exact seeds + batched BFS, or the Q=1 path for a query whose seeds missed the
certificate or whose visit set outgrew the batched table. The Q=1 path itself
is held to the oracle by test_gpu_parity.py; a few batched answers are also
checked against the oracle directly here.

Cases: K in {1, 5, 10, 16}, max_results 0 / 15 / 200, hops 0-3, modality
filter, lambda 0, per-query times, fp16 context, Q=600 (the LDS-tiled MFMA
kernel), duplicated rows (certificate fails -> Q=1), a 9,000-edge hub (visit
overflow -> Q=1), configurations the batch does not take (episode scope, boost,
K > 16), and rows inserted after the fp16 copy was made.
"""
from __future__ import annotations

import numpy as np
import pytest

import mars_amd
from mars_amd import BatchStats, RetrievalConfig, RetrievalScope, corpus

import parity
from parity import check_global, check_results_exact

pytestmark = pytest.mark.gpu
T_Q = corpus.QUERY_TIME
LAM = corpus.DECAY_LAMBDA


class Dev(parity.Dev):
    """parity.Dev with the fp16 copy every batched call reads."""

    def __init__(self, emb, mods, ts, row, col, ep=None, cap_nodes=0, max_k=64):
        super().__init__(emb, mods, ts, row, col, ep, max_k=max_k, fp16=True, capacity_nodes=cap_nodes)


def run_both(dev: Dev, qs: np.ndarray, t_q, cfg: RetrievalConfig, cap: int = 256):
    """Batched answers and Q=1 answers for the same device query vectors."""
    qs = np.ascontiguousarray(qs, np.float32)
    q = qs.shape[0]
    tq = np.broadcast_to(np.asarray(t_q, np.float32), (q,)).copy()
    buf = mars_amd.DeviceBuffer.from_array(qs)
    try:
        st = BatchStats()
        got = mars_amd.query_global_batch(dev.dg, dev.ctx, buf.ptr, q, tq, cfg, cap=cap, stats=st)
        want = [mars_amd.query_memory_fast_device(dev.dg, dev.ctx, buf.ptr + i * qs.shape[1] * 4, float(tq[i]), cfg)
                for i in range(q)]
    finally:
        buf.free()
    assert st.queries == q and st.batched + st.uncertified + st.overflow == q or st.whole_batch_q1 == 1
    return got, want, st


def assert_same(got, want, cap=256):
    assert len(got) == len(want)
    for i, (g, w) in enumerate(zip(got, want)):
        w = w[:cap]
        assert len(g) == len(w), (i, len(g), len(w))
        for j, (a, b) in enumerate(zip(g, w)):
            assert (a.node_id, a.modality, a.hops_from_seed) == (b.node_id, b.modality, b.hops_from_seed), (i, j, a, b)
            assert np.float32(a.score).tobytes() == np.float32(b.score).tobytes(), (i, j, a.score, b.score)


@pytest.fixture(scope="module")
def dev10k(corpus_10k):
    c = corpus_10k
    d = Dev(c.embeddings, c.modalities, c.timestamps, c.row_offsets, c.col_indices, c.episode_ids)
    yield d
    d.close()


CONFIGS = [
    RetrievalConfig(top_k=10, time_decay_lambda=LAM),
    RetrievalConfig(top_k=10, time_decay_lambda=LAM, max_results_returned=15),
    RetrievalConfig(top_k=1, time_decay_lambda=LAM, bfs_max_hops=1),
    RetrievalConfig(top_k=5, time_decay_lambda=LAM, bfs_max_hops=3, max_results_returned=200),
    RetrievalConfig(top_k=10, time_decay_lambda=LAM, bfs_max_hops=0),
    RetrievalConfig(top_k=10, time_decay_lambda=LAM, modality_filter=1),
    RetrievalConfig(top_k=10, time_decay_lambda=0.0, bfs_score_decay=0.85),
    RetrievalConfig(top_k=16, time_decay_lambda=LAM),
]


@pytest.mark.parametrize("ci", range(len(CONFIGS)))
def test_batched_equals_q1(dev10k, corpus_10k, ci):
    cfg = CONFIGS[ci]
    qn = corpus.pick_queries(corpus_10k.modalities, 48, seed=700 + ci)
    got, want, st = run_both(dev10k, corpus_10k.embeddings[qn], T_Q, cfg)
    assert_same(got, want)
    assert st.n_live == dev10k.n and st.whole_batch_q1 == 0
    if cfg.top_k <= 10:
        # the synthetic corpus leaves wide gaps below the K-th score: almost every
        # query is certified and answered by the batch itself
        assert st.batched >= 0.9 * len(qn), st
        assert st.min_margin > 0


def test_single_query_batch(dev10k, corpus_10k):
    """A batch of one global query takes the certified Q=1 path: same answers."""
    for i, cfg in enumerate(CONFIGS[:4]):
        qn = corpus.pick_queries(corpus_10k.modalities, 1, seed=840 + i)
        got, want, st = run_both(dev10k, corpus_10k.embeddings[qn], T_Q, cfg)
        assert_same(got, want)
        assert st.batched == 1


def test_batched_per_query_times(dev10k, corpus_10k, rng):
    qn = corpus.pick_queries(corpus_10k.modalities, 40, seed=801)
    tq = rng.uniform(300, 600, size=40).astype(np.float32)
    got, want, st = run_both(dev10k, corpus_10k.embeddings[qn], tq, RetrievalConfig(top_k=10, time_decay_lambda=LAM))
    assert_same(got, want)
    assert st.batched >= 36


def test_batched_fp16_context(dev10k, corpus_10k):
    """With the fp16 context flag the Q=1 path scans fp16 rows; the batch follows it."""
    dev10k.ctx.use_fp16 = True
    try:
        qn = corpus.pick_queries(corpus_10k.modalities, 32, seed=802)
        got, want, st = run_both(dev10k, corpus_10k.embeddings[qn], T_Q, RetrievalConfig(top_k=10, time_decay_lambda=LAM))
        assert_same(got, want)
        assert st.batched >= 29
    finally:
        dev10k.ctx.use_fp16 = False


def test_batched_large_q_uses_tiled_kernel(dev10k, corpus_10k):
    qn = corpus.pick_queries(corpus_10k.modalities, 600, seed=803)
    got, want, st = run_both(dev10k, corpus_10k.embeddings[qn], T_Q, RetrievalConfig(top_k=10, time_decay_lambda=LAM),
                             cap=32)
    assert_same(got, want, cap=32)
    assert st.batched >= 540


def test_batched_results_against_oracle(dev10k, corpus_10k):
    """Batched answers against the fp64 oracle run from the same seeds (the seed set
    itself is held to the oracle's top-K up to near-ties)."""
    c = corpus_10k
    cfg = RetrievalConfig(top_k=10, time_decay_lambda=LAM, max_results_returned=15)
    qn = corpus.pick_queries(c.modalities, 4, seed=804)
    got, want, st = run_both(dev10k, c.embeddings[qn], T_Q, cfg)
    assert_same(got, want)
    assert st.batched == 4
    for i, node in enumerate(qn):
        q = c.embeddings[node]
        st1 = mars_amd.RetrievalStats()
        res = mars_amd.query_memory_fast(dev10k.dg, dev10k.ctx, q, T_Q, cfg, st1)
        check_results_exact(got[i], res)
        # the Q=1 answer (equal to the batch's) against the oracle: scores, seeds, BFS, results
        check_global(dev10k, q, cfg, res=res, st=st1)


def test_uncertified_queries_fall_back(corpus_10k):
    """40 copies of one row: exact and fp16 scores tie across more rows than the batch
    keeps, so the certificate fails and the Q=1 path answers."""
    c = corpus_10k
    emb = c.embeddings.copy()
    ts = c.timestamps.copy()
    src = int(corpus.pick_queries(c.modalities, 1, seed=805)[0])
    dups = np.arange(100, 140)
    emb[dups] = emb[src]
    ts[dups] = ts[src]
    dev = Dev(emb, c.modalities, ts, c.row_offsets, c.col_indices)
    try:
        others = corpus.pick_queries(c.modalities, 7, seed=806)
        qs = np.concatenate([emb[src][None], emb[others]])
        got, want, st = run_both(dev, qs, T_Q, RetrievalConfig(top_k=10, time_decay_lambda=0.0))
        assert_same(got, want)
        assert st.uncertified >= 1 and st.batched >= 5
    finally:
        dev.close()


def test_visit_overflow_falls_back():
    """A seed joined to 9,000 nodes: the visit set outgrows the batched table."""
    c = corpus.make_corpus(12000, 768, seed=61)
    n = c.num_nodes
    hub = int(corpus.pick_queries(c.modalities, 1, seed=807)[0])
    leaves = np.array([i for i in range(n) if i != hub][:9000], np.int32)
    adj = [[] for _ in range(n)]
    for v in leaves:
        adj[hub].append(int(v))
        adj[int(v)].append(hub)
    row = np.zeros(n + 1, np.int32)
    row[1:] = np.cumsum([len(a) for a in adj])
    col = np.concatenate([np.sort(np.array(a, np.int32)) for a in adj if a]).astype(np.int32)
    dev = Dev(c.embeddings, c.modalities, c.timestamps, row, col)
    try:
        others = corpus.pick_queries(c.modalities, 5, seed=808)
        qs = np.concatenate([c.embeddings[hub][None], c.embeddings[others]])
        got, want, st = run_both(dev, qs, T_Q, RetrievalConfig(top_k=10, time_decay_lambda=0.01), cap=64)
        assert_same(got, want, cap=64)
        assert st.overflow >= 1
    finally:
        dev.close()


def test_configurations_sent_to_q1(dev10k, corpus_10k):
    c = corpus_10k
    qn = corpus.pick_queries(c.modalities, 6, seed=809)
    node = int(qn[0])
    ep = int(c.episode_ids[node])
    csr = mars_amd.build_episode_csr(c.episode_ids, c.num_nodes)
    b, e = int(csr.ep_csr_offsets[ep]), int(csr.ep_csr_offsets[ep + 1])
    cfgs = [
        RetrievalConfig(top_k=10, time_decay_lambda=LAM, retrieval_scope=RetrievalScope.EpisodeScoped,
                        query_episode_id=ep, query_episode_member_begin=b, query_episode_member_count=e - b),
        RetrievalConfig(top_k=10, time_decay_lambda=LAM, query_episode_id=ep, episode_same_boost=0.5),
        RetrievalConfig(top_k=20, time_decay_lambda=LAM),
    ]
    for cfg in cfgs:
        got, want, st = run_both(dev10k, c.embeddings[qn], T_Q, cfg)
        assert_same(got, want)
        assert st.whole_batch_q1 == 1


def test_inserted_rows_are_covered():
    """Rows appended after the fp16 copy raise the graph's norm bounds: large-norm
    inserted rows must neither break the certificate nor be missed."""
    c = corpus.make_corpus(8000, 768, seed=62)
    c = corpus.nsn_graph(c)
    dev = Dev(c.embeddings, c.modalities, c.timestamps, c.row_offsets, c.col_indices, c.episode_ids,
              cap_nodes=8100)
    try:
        rng = np.random.default_rng(5)
        src = corpus.pick_queries(c.modalities, 20, seed=810)
        new = (c.embeddings[src] * 3.0 + 0.01 * rng.standard_normal((20, 768))).astype(np.float32)
        mods = c.modalities[src].copy()
        ts = np.full(20, T_Q - 1.0, np.float32)
        epi = np.repeat(np.arange(20) // 10 + int(c.episode_ids.max()) + 1, 1).astype(np.int32)
        mars_amd.insert_nodes(dev.dg, new, mods, ts, epi, knn_k=8)
        qs = c.embeddings[src[:12]]
        got, want, st = run_both(dev, qs, T_Q, RetrievalConfig(top_k=10, time_decay_lambda=LAM))
        assert st.n_live == 8020
        assert_same(got, want)
        # the scaled copies score about 3x their sources: they are the top seeds
        for i, g in enumerate(got):
            assert g[0].node_id >= 8000
    finally:
        dev.close()
