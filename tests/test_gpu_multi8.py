"""Batched global queries and neighbour searches over the int8 copy (k_split8, k_scan8m,
k_cert_multi8 through mars_query_global_batch / mars_query_global_batch_knn).

Bars:
  * with the int8 copy, a batch of up to 16 global queries and neighbour searches is
    answered by one pass over it (stats.candidate_rows == 8), and every global answer
    (ids, scores, modalities, hops, order, count) is bit-identical to the Q=1 path's;
  * the neighbour lists equal the exact CPU k-NN up to near-ties (1e-5), the node itself
    excluded, and the same lists come back with global queries in the batch;
  * above 16 queries the fp16 MFMA scan answers (candidate_rows == 16), with the same
    answers;
  * the widths of k_scan8m (D = 256, 512, 1024) and both operand counts (1-8 and 9-16
    queries), per-query times and a modality filter.
"""
from __future__ import annotations

import numpy as np
import pytest

import mars_amd
import oracle
from mars_amd import BatchStats, RetrievalConfig, corpus

from test_gpu_multi import CONFIGS, Dev, assert_same, run_both

pytestmark = pytest.mark.gpu
T_Q = corpus.QUERY_TIME
LAM = corpus.DECAY_LAMBDA


@pytest.fixture(scope="module")
def dev8(corpus_10k):
    c = corpus_10k
    d = Dev(c.embeddings, c.modalities, c.timestamps, c.row_offsets, c.col_indices, c.episode_ids)
    mars_amd.upload_int8_embeddings(d.dg)
    yield d
    d.close()


def check_knn_exact(emb, first, got, k):
    want, sims = oracle.knn(emb, np.arange(first, first + len(got), dtype=np.int32), k)
    e = emb.astype(np.float64)
    for i in range(len(got)):
        assert len(set(got[i].tolist())) == k and first + i not in got[i], (first + i, got[i])
        for j in set(got[i].tolist()) ^ set(want[i].tolist()):
            s = float(e[first + i] @ e[j])
            assert abs(s - sims[i, k - 1]) <= 1e-5, (first + i, j, s, sims[i, k - 1])


@pytest.mark.parametrize("q", [2, 5, 8, 9, 16])
@pytest.mark.parametrize("ci", [0, 1, 3, 5, 6, 7])
def test_int8_batch_equals_q1(dev8, corpus_10k, q, ci):
    cfg = CONFIGS[ci]
    qn = corpus.pick_queries(corpus_10k.modalities, q, seed=8000 + 10 * q + ci)
    got, want, st = run_both(dev8, corpus_10k.embeddings[qn], T_Q, cfg)
    assert_same(got, want)
    assert st.candidate_rows == 8, st
    if cfg.top_k <= 10:
        assert st.batched >= q - 1, st


def test_int8_batch_per_query_times(dev8, corpus_10k, rng):
    qn = corpus.pick_queries(corpus_10k.modalities, 12, seed=8101)
    tq = rng.uniform(300, 600, 12).astype(np.float32)
    got, want, st = run_both(dev8, corpus_10k.embeddings[qn], tq, RetrievalConfig(top_k=10, time_decay_lambda=LAM))
    assert_same(got, want)
    assert st.candidate_rows == 8


def test_above_16_queries_take_the_fp16_scan(dev8, corpus_10k):
    qn = corpus.pick_queries(corpus_10k.modalities, 17, seed=8102)
    got, want, st = run_both(dev8, corpus_10k.embeddings[qn], T_Q, RetrievalConfig(top_k=10, time_decay_lambda=LAM))
    assert_same(got, want)
    assert st.candidate_rows == 16


@pytest.mark.parametrize("nq,nk", [(0, 1), (0, 16), (3, 5), (8, 8), (1, 15)])
def test_int8_neighbour_search(dev8, corpus_10k, nq, nk):
    c = corpus_10k
    first = 4321
    qn = corpus.pick_queries(c.modalities, max(nq, 1), seed=8103)[:nq]
    cfg = RetrievalConfig(top_k=10, time_decay_lambda=LAM)
    buf = mars_amd.DeviceBuffer.from_array(np.ascontiguousarray(c.embeddings[qn])) if nq else None
    try:
        st = BatchStats()
        got, knn = mars_amd.query_global_batch_knn(dev8.dg, dev8.ctx, buf.ptr if buf else 0, nq, T_Q, cfg, first, nk,
                                                   8, stats=st)
        assert st.candidate_rows == 8, st
        check_knn_exact(c.embeddings, first, knn, 8)
        if nq:
            want = [mars_amd.query_memory_fast_device(dev8.dg, dev8.ctx, buf.ptr + i * 768 * 4, T_Q, cfg)
                    for i in range(nq)]
            assert_same(got, want, cap=64)
            # the same neighbour lists without the global queries
            _, knn0 = mars_amd.query_global_batch_knn(dev8.dg, dev8.ctx, 0, 0, T_Q, cfg, first, nk, 8)
            np.testing.assert_array_equal(knn0, knn)
    finally:
        if buf:
            buf.free()


@pytest.mark.parametrize("d", [256, 512, 1024])
def test_int8_batch_widths(d):
    c = corpus.nsn_graph(corpus.make_corpus(6000, d, seed=500 + d))
    dev = Dev(c.embeddings, c.modalities, c.timestamps, c.row_offsets, c.col_indices, c.episode_ids)
    mars_amd.upload_int8_embeddings(dev.dg)
    try:
        for q, cfg in ((6, RetrievalConfig(top_k=10, time_decay_lambda=LAM, max_results_returned=15)),
                       (13, RetrievalConfig(top_k=5, time_decay_lambda=LAM, modality_filter=1))):
            qn = corpus.pick_queries(c.modalities, q, seed=8200 + q)
            got, want, st = run_both(dev, c.embeddings[qn], T_Q, cfg)
            assert_same(got, want)
            assert st.candidate_rows == 8 and st.batched >= q - 1, st
        if d <= 768:                                  # neighbour searches need the fp16 batched widths
            _, knn = mars_amd.query_global_batch_knn(dev.dg, dev.ctx, 0, 0, T_Q, RetrievalConfig(), 100, 16, 8)
            check_knn_exact(c.embeddings, 100, knn, 8)
    finally:
        dev.close()


def test_insert_knn_over_int8(corpus_10k):
    """An insert of up to 16 nodes finds their neighbours with one int8 pass: the lists
    are the exact k-NN among all rows (near-ties aside) and equal the batched neighbour
    search's over the same rows."""
    c = corpus.make_corpus(8020, 768, seed=91)
    base = 8000
    g = corpus.nsn_graph(corpus.Corpus(c.embeddings[:base], c.modalities[:base], c.timestamps[:base],
                                       c.episode_ids[:base], 91))
    dev = Dev(g.embeddings, g.modalities, g.timestamps, g.row_offsets, g.col_indices, g.episode_ids, cap_nodes=8020)
    mars_amd.upload_int8_embeddings(dev.dg)
    try:
        st, got = mars_amd.insert_nodes(dev.dg, c.embeddings[base:base + 10], c.modalities[base:base + 10],
                                        c.timestamps[base:base + 10], c.episode_ids[base:base + 10], knn_k=8,
                                        return_knn=True)
        assert st.nodes_added == 10
        check_knn_exact(c.embeddings[:base + 10], base, got, 8)
        bst = BatchStats()
        _, knn = mars_amd.query_global_batch_knn(dev.dg, dev.ctx, 0, 0, T_Q, RetrievalConfig(), base, 10, 8,
                                                 stats=bst)
        assert bst.candidate_rows == 8
        np.testing.assert_array_equal(knn, got)
    finally:
        dev.close()


def test_insert_knn_ties_fall_back():
    """Nodes whose neighbours tie: 25 rows of the corpus are one vector, and two of the
    inserted nodes are that vector too, so the 8th and 16th best scores of their lists are
    equal and the fp16 search cannot certify them. The insert then takes the int8 pass (64
    candidates, past the ties) or, where its certificate fails too, the fp16 lists: either
    way the exact k-NN up to the ties (eight of the copies), the other nodes' lists exact,
    a node never its own neighbour."""
    c = corpus.make_corpus(8008, 768, seed=93)
    base = 8000
    emb = c.embeddings.copy()
    dup = emb[17].copy()
    copies = np.arange(100, 100 + 24 * 300, 300)
    emb[copies] = dup
    emb[base:base + 2] = dup
    g = corpus.nsn_graph(corpus.Corpus(emb[:base], c.modalities[:base], c.timestamps[:base],
                                       c.episode_ids[:base], 93))
    dev = Dev(g.embeddings, g.modalities, g.timestamps, g.row_offsets, g.col_indices, g.episode_ids, cap_nodes=8008)
    mars_amd.upload_int8_embeddings(dev.dg)
    try:
        st, got = mars_amd.insert_nodes(dev.dg, emb[base:base + 8], c.modalities[base:base + 8],
                                        c.timestamps[base:base + 8], c.episode_ids[base:base + 8], knn_k=8,
                                        return_knn=True)
        assert st.nodes_added == 8
        check_knn_exact(emb[:base + 8], base, got, 8)
        for i in (0, 1):                      # the copies: eight of the tied rows
            allowed = (set(copies.tolist()) | {17, base, base + 1}) - {base + i}
            assert set(got[i].tolist()) <= allowed, got[i]
    finally:
        dev.close()
