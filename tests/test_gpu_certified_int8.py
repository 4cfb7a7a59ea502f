"""Certified global queries over the int8 copy (mars_graph_enable_int8, k_scan8).

Bar: the int8 copy holds exactly the bytes, scales and bounds that the numpy
restatement in test_certificate.py computes from the same fp32 rows, also for rows
inserted or replaced later; and with MARS_CTX_CERTIFIED every global query returns bit
for bit the fp32 path's results (ids, scores, modalities, hops, order, count), whether
the int8 scan's candidates were certified or the fp32 scan answered. The fp32 path is
held to the oracle by test_gpu_parity.py; the bound the certificate rests on is checked
against simulated kernel arithmetic in test_certificate.py.

Cases: the CONFIGS of test_gpu_multi (K 1-16, max_results, hops 0-3, modality filter,
lambda 0, hop decay 0.85), host vectors and K = 64, duplicated rows (certificate fails),
a 9,000-edge hub (visit overflow), inserted and replaced rows, and the int8 copy without
the fp16 copy. Graph: the 10K corpus of conftest.py with its NSN CSR.
"""
from __future__ import annotations

import numpy as np
import pytest

import mars_amd
from mars_amd import RetrievalConfig, corpus

from test_certificate import quantize_i8
from test_gpu_certified import both
from test_gpu_multi import CONFIGS, Dev, assert_same

pytestmark = pytest.mark.gpu
T_Q = corpus.QUERY_TIME
LAM = corpus.DECAY_LAMBDA


def with_int8(dev):
    mars_amd.upload_int8_embeddings(dev.dg)
    return dev


def check_copy(dev, emb, first=0):
    b, m = mars_amd.read_int8(dev.dg, first, emb.shape[0])
    v, s, c = quantize_i8(np.ascontiguousarray(emb, np.float32))
    np.testing.assert_array_equal(b, v)
    np.testing.assert_array_equal(m[:, 0], s)
    np.testing.assert_array_equal(m[:, 1], c)


@pytest.fixture(scope="module")
def dev8(corpus_10k):
    c = corpus_10k
    d = with_int8(Dev(c.embeddings, c.modalities, c.timestamps, c.row_offsets, c.col_indices, c.episode_ids))
    yield d
    d.close()


def test_int8_copy_matches_numpy(dev8, corpus_10k):
    check_copy(dev8, corpus_10k.embeddings)


@pytest.mark.parametrize("ci", range(len(CONFIGS)))
def test_int8_certified_equals_fp32(dev8, corpus_10k, ci):
    cfg = CONFIGS[ci]
    qn = corpus.pick_queries(corpus_10k.modalities, 40, seed=1900 + ci)
    got, stats, want = both(dev8, corpus_10k.embeddings[qn], cfg)
    assert_same(got, want)
    cert = sum(s.seeds_certified for s in stats)
    print(f"config {ci}: {cert}/{len(qn)} certified")
    if cfg.top_k <= 16:
        assert cert >= 0.9 * len(qn), cert


def test_int8_certified_host_vectors_and_k64(dev8, corpus_10k):
    qn = corpus.pick_queries(corpus_10k.modalities, 12, seed=1950)
    for cfg in (RetrievalConfig(top_k=10, time_decay_lambda=LAM, max_results_returned=15),
                RetrievalConfig(top_k=64, time_decay_lambda=LAM)):
        got, stats, want = both(dev8, corpus_10k.embeddings[qn], cfg, device=False)
        assert_same(got, want)


def test_int8_certificate_fails_on_ties(corpus_10k):
    c = corpus_10k
    emb, ts = c.embeddings.copy(), c.timestamps.copy()
    src = int(corpus.pick_queries(c.modalities, 1, seed=1954)[0])
    dups = np.arange(200, 280)                               # 80 copies: more than the 64 candidates
    emb[dups] = emb[src]
    ts[dups] = ts[src]
    dev = with_int8(Dev(emb, c.modalities, ts, c.row_offsets, c.col_indices))
    try:
        qs = np.concatenate([emb[src][None], emb[corpus.pick_queries(c.modalities, 5, seed=1955)]])
        got, stats, want = both(dev, qs, RetrievalConfig(top_k=10, time_decay_lambda=0.0))
        assert_same(got, want)
        assert stats[0].seeds_certified == 0
        assert sum(s.seeds_certified for s in stats[1:]) >= 4
    finally:
        dev.close()


def test_int8_certified_visit_overflow_falls_back():
    c = corpus.make_corpus(12000, 768, seed=63)
    n = c.num_nodes
    hub = int(corpus.pick_queries(c.modalities, 1, seed=1956)[0])
    leaves = np.array([i for i in range(n) if i != hub][:9000], np.int32)
    adj = [[] for _ in range(n)]
    for v in leaves:
        adj[hub].append(int(v))
        adj[int(v)].append(hub)
    row = np.zeros(n + 1, np.int32)
    row[1:] = np.cumsum([len(a) for a in adj])
    col = np.concatenate([np.sort(np.array(a, np.int32)) for a in adj if a]).astype(np.int32)
    dev = with_int8(Dev(c.embeddings, c.modalities, c.timestamps, row, col))
    try:
        qs = np.concatenate([c.embeddings[hub][None], c.embeddings[corpus.pick_queries(c.modalities, 3, seed=1957)]])
        cfg = RetrievalConfig(top_k=10, time_decay_lambda=0.01, max_results_returned=100)
        got, stats, want = both(dev, qs, cfg)
        assert_same(got, want)
        assert stats[0].seeds_certified == 0
    finally:
        dev.close()


def test_int8_after_inserts_and_set_rows():
    """Inserted rows (larger norms: coarser scales, larger bounds) and rows replaced by
    set_rows are quantized like the rest; the answers stay the fp32 path's."""
    c = corpus.nsn_graph(corpus.make_corpus(8000, 768, seed=64))
    dev = with_int8(Dev(c.embeddings, c.modalities, c.timestamps, c.row_offsets, c.col_indices, c.episode_ids,
                        cap_nodes=8100))
    try:
        rng = np.random.default_rng(9)
        src = corpus.pick_queries(c.modalities, 20, seed=1958)
        new = (c.embeddings[src] * 2.5 + 0.01 * rng.standard_normal((20, 768))).astype(np.float32)
        epi = (np.arange(20) // 10 + int(c.episode_ids.max()) + 1).astype(np.int32)
        mars_amd.insert_nodes(dev.dg, new, c.modalities[src], np.full(20, T_Q - 2.0, np.float32), epi, knn_k=8)
        check_copy(dev, new, first=8000)
        got, stats, want = both(dev, c.embeddings[src[:10]], RetrievalConfig(top_k=10, time_decay_lambda=LAM))
        assert_same(got, want)
        assert all(g[0].node_id >= 8000 for g in got)
        assert sum(s.seeds_certified for s in stats) >= 9
        # replace 50 rows with scaled copies of query rows: the copy and the answers follow
        rows = np.arange(3000, 3050)
        rep = (c.embeddings[src[np.arange(50) % 20]] * 0.5 + 0.02 * rng.standard_normal((50, 768))).astype(np.float32)
        mars_amd.set_rows(dev.dg, 3000, rep, c.modalities[rows], c.timestamps[rows])
        check_copy(dev, rep, first=3000)
        got, stats, want = both(dev, c.embeddings[src[10:]], RetrievalConfig(top_k=10, time_decay_lambda=LAM))
        assert_same(got, want)
    finally:
        dev.close()


def test_int8_without_fp16_copy(corpus_10k):
    c = corpus_10k
    dev = with_int8(parity_dev(c))
    try:
        qn = corpus.pick_queries(c.modalities, 24, seed=1960)
        got, stats, want = both(dev, c.embeddings[qn], RetrievalConfig(top_k=10, time_decay_lambda=LAM))
        assert_same(got, want)
        assert sum(s.seeds_certified for s in stats) >= 22
        # without either copy the flag is ignored: the fp32 scan answers
        mars_amd.free_int8_embeddings(dev.dg)
        got, stats, want = both(dev, c.embeddings[qn[:4]], RetrievalConfig(top_k=10, time_decay_lambda=LAM))
        assert_same(got, want)
        assert all(s.seeds_certified == 0 for s in stats)
    finally:
        dev.close()


def parity_dev(c):
    from parity import Dev as PDev
    return PDev(c.embeddings, c.modalities, c.timestamps, c.row_offsets, c.col_indices, c.episode_ids, fp16=False)
