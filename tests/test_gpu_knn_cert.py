"""Certified k-NN builds (mars_graph_knn / _range / _blocked and mars_graph_knn_report).

Bars:
  * every list of an all-pairs build is exact: the k-NN of 2,000 sampled nodes of the
    100K benchmark corpus (and 1,000 of a 150K one, whose row ranges take the sampled
    floors) equal the fp64 oracle's up to near-ties (1e-5), and the report says that every
    node the certificate missed was scanned again exactly;
  * rows whose neighbours tie (80 copies of one row) miss the certificate, are scanned
    again, and their lists hold copies of the row (score 1, the node itself excluded);
  * a build within blocks counts the nodes the certificate missed and scans none again;
  * the range builder in pieces reports the same lists as the one-call build.
"""
from __future__ import annotations

import numpy as np
import pytest

import mars_amd
import oracle
from mars_amd import corpus

pytestmark = pytest.mark.gpu
D = 768


def device_graph(emb, mods, ts):
    g = mars_amd.MemoryGraph(len(mods), emb.shape[1], None, None, emb, mods, ts)
    dg = mars_amd.upload_to_device(g)
    mars_amd.upload_fp16_embeddings(dg)
    return dg


def check_lists(emb, nodes, got, k=8):
    want, sims = oracle.knn(emb, np.asarray(nodes, np.int32), k)
    e = emb.astype(np.float64)
    for i, node in enumerate(nodes):
        assert len(set(got[i].tolist())) == k and node not in got[i], (node, got[i])
        for j in set(got[i].tolist()) ^ set(want[i].tolist()):
            s = float(e[node] @ e[j])
            assert abs(s - sims[i, k - 1]) <= 1e-5, (node, j, s, sims[i, k - 1])


def test_all_pairs_100k_exact():
    c = corpus.make_corpus(100_000, D, seed=2026, threads=16)
    dg = device_graph(c.embeddings, c.modalities, c.timestamps)
    try:
        got = mars_amd.graph_knn(dg, 8)
        u, r = dg.knn_report
        print(f"100K all-pairs 8-NN: {u} lists uncertified, {r} scanned again")
        assert r == u and u <= 1000
        nodes = np.random.default_rng(5).choice(100_000, 2000, replace=False)
        check_lists(c.embeddings, nodes, got[nodes])
        # in pieces of 30,000 query nodes: the same lists
        got2 = mars_amd.graph_knn(dg, 8, progress=lambda *_: None, piece=30_000)
        np.testing.assert_array_equal(got2, got)
        assert dg.knn_report == (u, r)
    finally:
        mars_amd.free_device(dg)


def test_all_pairs_150k_with_floors_exact():
    """150,000 nodes: row ranges of 2,560 rows, long enough for the sampled pass, so
    k_batch_mm's thresholds start from its floors; 1,000 sampled nodes against the fp64
    oracle, up to near-ties, and every list the certificate missed scanned again."""
    c = corpus.make_corpus(150_000, D, seed=2027, threads=16)
    dg = device_graph(c.embeddings, c.modalities, c.timestamps)
    try:
        got = mars_amd.graph_knn(dg, 8)
        u, r = dg.knn_report
        assert r == u and u <= 1500
        nodes = np.random.default_rng(6).choice(150_000, 1000, replace=False)
        check_lists(c.embeddings, nodes, got[nodes])
    finally:
        mars_amd.free_device(dg)


def test_knn_range_2_2m_multi_tile_floors_exact():
    """2,200,000 nodes: row ranges of 34,560 rows, whose sampled pass covers 528 rows
    (three tiles, the last one partial), so k_batch_mm's floors come from block maxima kept
    over several tiles. The 2,048 query nodes start at range 28's first row, so 528 of them
    have their own row among the sampled rows. 100 of them against the fp64 oracle, up to
    near-ties."""
    n = 2_200_000
    c = corpus.make_corpus(n, D, seed=2028, threads=16)
    dg = device_graph(c.embeddings, c.modalities, c.timestamps)
    try:
        first = 28 * 34_560
        got = mars_amd.graph_knn_range(dg, 8, first, 2048)
        u, r = mars_amd.graph_knn_report(dg)
        assert r == u and u <= 20
        idx = np.sort(np.concatenate([np.arange(0, 528, 11), np.random.default_rng(7).choice(np.arange(528, 2048), 52, replace=False)]))
        check_lists(c.embeddings, first + idx, got[idx])
    finally:
        mars_amd.free_device(dg)


def test_tied_rows_are_scanned_again():
    c = corpus.make_corpus(6000, D, seed=17)
    emb = c.embeddings.copy()
    dups = np.arange(1000, 1080)                        # 80 copies of row 1000
    emb[dups] = emb[1000]
    dg = device_graph(emb, c.modalities, c.timestamps)
    try:
        got = mars_amd.graph_knn(dg, 8)
        u, r = dg.knn_report
        assert u >= 80 and r == u, (u, r)
        for node in dups:
            assert set(got[node].tolist()) <= set(dups.tolist()) - {int(node)}
        check_lists(emb, np.arange(0, 6000, 7), got[::7])
    finally:
        mars_amd.free_device(dg)


def test_blocked_build_counts_only():
    c = corpus.make_corpus(6000, D, seed=18)
    emb = c.embeddings.copy()
    emb[10:30] = emb[10]                                 # ties inside block 0
    dg = device_graph(emb, c.modalities, c.timestamps)
    try:
        got = mars_amd.graph_knn(dg, 8, block_rows=2000)
        u, r = dg.knn_report
        assert u >= 20 and r == 0, (u, r)
        for b in range(3):                              # lists stay inside their block
            assert np.all((got[2000 * b:2000 * (b + 1)] // 2000) == b)
    finally:
        mars_amd.free_device(dg)
