"""Certified global queries (MARS_CTX_CERTIFIED through the C ABI).

Bar: with the flag, every global query returns bit-for-bit the results of the fp32
path (ids, scores, modalities, hops, order, count) — whether the fp16 scan's seeds
were certified (stats.seeds_certified = 1) or the fp32 scan answered. The fp32 path
is held to the oracle by test_gpu_parity.py.

Cases: K in {1, 5, 10, 16, 64}, max_results, hops 0-3, modality filter, lambda 0,
host and device query vectors, duplicated rows (certificate fails), a 9,000-edge
hub (visit overflow), the fp16 context flag (certified ignored), graph replay flag,
rows inserted after the fp16 copy was made, and queries interleaved with the
fp32 path on one context.
"""
from __future__ import annotations

import numpy as np
import pytest

import mars_amd
from mars_amd import RetrievalConfig, RetrievalStats, corpus

from test_gpu_multi import CONFIGS, Dev, assert_same

pytestmark = pytest.mark.gpu
T_Q = corpus.QUERY_TIME
LAM = corpus.DECAY_LAMBDA


@pytest.fixture(scope="module")
def dev10k(corpus_10k):
    c = corpus_10k
    d = Dev(c.embeddings, c.modalities, c.timestamps, c.row_offsets, c.col_indices, c.episode_ids)
    yield d
    d.close()


def both(dev, qs, cfg, t_q=T_Q, device=True):
    """(certified answers, their stats, fp32 answers) for the same query vectors."""
    got, stats, want = [], [], []
    buf = mars_amd.DeviceBuffer.from_array(np.ascontiguousarray(qs, np.float32)) if device else None
    try:
        for flag, out in ((True, got), (False, want)):
            dev.ctx.certified = flag
            for i, q in enumerate(qs):
                st = RetrievalStats()
                if device:
                    r = mars_amd.query_memory_fast_device(dev.dg, dev.ctx, buf.ptr + i * qs.shape[1] * 4, t_q, cfg, st)
                else:
                    r = mars_amd.query_memory_fast(dev.dg, dev.ctx, q, t_q, cfg, st)
                out.append(r)
                if flag:
                    stats.append(st)
    finally:
        dev.ctx.certified = False
        if buf:
            buf.free()
    return got, stats, want


@pytest.mark.parametrize("ci", range(len(CONFIGS)))
def test_certified_equals_fp32(dev10k, corpus_10k, ci):
    cfg = CONFIGS[ci]
    qn = corpus.pick_queries(corpus_10k.modalities, 40, seed=900 + ci)
    got, stats, want = both(dev10k, corpus_10k.embeddings[qn], cfg)
    assert_same(got, want)
    cert = sum(s.seeds_certified for s in stats)
    if cfg.top_k <= 16:
        assert cert >= 0.9 * len(qn), cert
    for s in stats:
        if s.seeds_certified:
            assert s.used_fp16 == 1 and s.nodes_scanned == dev10k.n


def test_certified_host_vectors_and_k64(dev10k, corpus_10k):
    qn = corpus.pick_queries(corpus_10k.modalities, 12, seed=950)
    for cfg in (RetrievalConfig(top_k=10, time_decay_lambda=LAM, max_results_returned=15),
                RetrievalConfig(top_k=64, time_decay_lambda=LAM)):
        got, stats, want = both(dev10k, corpus_10k.embeddings[qn], cfg, device=False)
        assert_same(got, want)


def test_certified_interleaved_with_fp32(dev10k, corpus_10k):
    """One context switching modes query by query: the scan's candidate state is reset
    by either path, so neither disturbs the other."""
    qn = corpus.pick_queries(corpus_10k.modalities, 20, seed=951)
    cfg = RetrievalConfig(top_k=10, time_decay_lambda=LAM)
    ref = [mars_amd.query_memory_fast(dev10k.dg, dev10k.ctx, corpus_10k.embeddings[n], T_Q, cfg) for n in qn]
    got = []
    try:
        for i, n in enumerate(qn):
            dev10k.ctx.certified = i % 2 == 0
            got.append(mars_amd.query_memory_fast(dev10k.dg, dev10k.ctx, corpus_10k.embeddings[n], T_Q, cfg))
    finally:
        dev10k.ctx.certified = False
    assert_same(got, ref)


def test_certified_flag_ignored_with_fp16_context(dev10k, corpus_10k):
    qn = corpus.pick_queries(corpus_10k.modalities, 6, seed=952)
    cfg = RetrievalConfig(top_k=10, time_decay_lambda=LAM)
    dev10k.ctx.use_fp16 = True
    try:
        got, stats, want = both(dev10k, corpus_10k.embeddings[qn], cfg)
    finally:
        dev10k.ctx.use_fp16 = False
    assert_same(got, want)
    assert all(s.seeds_certified == 0 and s.used_fp16 == 1 for s in stats)


def test_certified_with_graph_replay_flag(dev10k, corpus_10k):
    qn = corpus.pick_queries(corpus_10k.modalities, 8, seed=953)
    cfg = RetrievalConfig(top_k=10, time_decay_lambda=LAM)
    dev10k.ctx.use_cuda_graph = True
    try:
        got, stats, want = both(dev10k, corpus_10k.embeddings[qn], cfg)
    finally:
        dev10k.ctx.use_cuda_graph = False
    assert_same(got, want)
    assert sum(s.seeds_certified for s in stats) >= 7


def test_certificate_fails_on_ties_and_fp32_answers(corpus_10k):
    c = corpus_10k
    emb, ts = c.embeddings.copy(), c.timestamps.copy()
    src = int(corpus.pick_queries(c.modalities, 1, seed=954)[0])
    dups = np.arange(200, 260)
    emb[dups] = emb[src]
    ts[dups] = ts[src]
    dev = Dev(emb, c.modalities, ts, c.row_offsets, c.col_indices)
    try:
        qs = np.concatenate([emb[src][None], emb[corpus.pick_queries(c.modalities, 5, seed=955)]])
        got, stats, want = both(dev, qs, RetrievalConfig(top_k=10, time_decay_lambda=0.0))
        assert_same(got, want)
        assert stats[0].seeds_certified == 0
        assert sum(s.seeds_certified for s in stats[1:]) >= 4
    finally:
        dev.close()


def test_certified_visit_overflow_falls_back():
    c = corpus.make_corpus(12000, 768, seed=63)
    n = c.num_nodes
    hub = int(corpus.pick_queries(c.modalities, 1, seed=956)[0])
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
        qs = np.concatenate([c.embeddings[hub][None], c.embeddings[corpus.pick_queries(c.modalities, 3, seed=957)]])
        cfg = RetrievalConfig(top_k=10, time_decay_lambda=0.01, max_results_returned=100)
        got, stats, want = both(dev, qs, cfg)
        assert_same(got, want)
        assert stats[0].seeds_certified == 0
    finally:
        dev.close()


def test_certified_after_inserts():
    """Inserted rows of larger norm raise the bound: the answers stay the fp32 path's."""
    c = corpus.nsn_graph(corpus.make_corpus(8000, 768, seed=64))
    dev = Dev(c.embeddings, c.modalities, c.timestamps, c.row_offsets, c.col_indices, c.episode_ids, cap_nodes=8100)
    try:
        rng = np.random.default_rng(9)
        src = corpus.pick_queries(c.modalities, 20, seed=958)
        new = (c.embeddings[src] * 2.5 + 0.01 * rng.standard_normal((20, 768))).astype(np.float32)
        epi = (np.arange(20) // 10 + int(c.episode_ids.max()) + 1).astype(np.int32)
        mars_amd.insert_nodes(dev.dg, new, c.modalities[src], np.full(20, T_Q - 2.0, np.float32), epi, knn_k=8)
        got, stats, want = both(dev, c.embeddings[src[:10]], RetrievalConfig(top_k=10, time_decay_lambda=LAM))
        assert_same(got, want)
        assert all(g[0].node_id >= 8000 for g in got)
    finally:
        dev.close()
