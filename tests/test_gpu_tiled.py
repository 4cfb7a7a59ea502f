"""GPU tiled out-of-core comparator (mars_tiled_query through the C ABI) against
the oracle's restatement of tiled_query (src/tiled_query.cu:174-314).

Bar: the K ids equal the oracle's except ids whose oracle score lies within the
fp32 score tolerance of the K-th one; scores within 1e-5 * max(|oracle|, w*sum|e q|);
rows removed by the modality filter never returned; tile size never changes the
answer. Edge cases: one tile, ragged last tile, tile of 997 rows, K = 1 and 64,
everything filtered out, pinned host buffers, argument errors.
"""
from __future__ import annotations

import numpy as np
import pytest

import mars_amd
import oracle
from mars_amd import TiledQueryConfig, corpus
from mars_amd._lib import MarsError

from conftest import RTOL_F32

pytestmark = pytest.mark.gpu
T_Q = corpus.QUERY_TIME
N = 20000


@pytest.fixture(scope="module")
def data():
    c = corpus.make_corpus(N, 768, seed=41)
    og = oracle.make_graph(c.embeddings, c.modalities, c.timestamps)
    ctx = mars_amd.create_tiled_context(N, 768, 64)
    yield c, og, ctx
    mars_amd.destroy_tiled_context(ctx)


def check(c, og, res, q, lam, k, tile, mod):
    want_ids, want_sc = oracle.tiled_query(og, q, T_Q, lam, k, tile, mod)
    fin, scale = oracle.scores(og, q, T_Q, lam, mod)
    assert len(res) == len(want_ids)
    got = np.array([r.node_id for r in res], np.int64)
    if len(got) == 0:
        return
    tol = RTOL_F32 * np.maximum(np.abs(fin), scale)
    kth = want_sc[-1]
    for g in set(got.tolist()) ^ set(want_ids.tolist()):
        assert abs(fin[g] - kth) <= 2 * tol[g] + 2 * tol[want_ids[-1]], (g, fin[g], kth)
    for r in res:
        assert abs(r.score - fin[r.node_id]) <= tol[r.node_id] + 1e-30
        assert r.modality == int(c.modalities[r.node_id])
        assert mod < 0 or r.modality == mod
    sc = [r.score for r in res]
    assert sc == sorted(sc, reverse=True)


@pytest.mark.parametrize("tile", [N, 3000, 997])
def test_tiled_matches_oracle(data, tile):
    c, og, ctx = data
    qs = corpus.pick_queries(c.modalities, 6, seed=tile)
    for i, node in enumerate(qs):
        k = (10, 1, 64)[i % 3]
        lam = (corpus.DECAY_LAMBDA, 1e-8)[i % 2]
        mod = (-1, 0, -1, 2, -1, 1)[i]
        st = mars_amd.TiledQueryStats()
        res = mars_amd.tiled_query(ctx, c.embeddings, c.modalities, c.timestamps, c.embeddings[node], T_Q,
                                   TiledQueryConfig(tile_size=tile, top_k=k, time_decay_lambda=lam,
                                                    modality_filter=mod), st)
        check(c, og, res, c.embeddings[node], lam, k, tile, mod)
        assert st.num_tiles == (N + tile - 1) // tile and st.total_nodes == N
        assert st.transfer_ms > 0 and st.compute_ms > 0


def test_tile_size_does_not_change_the_answer(data):
    c, og, ctx = data
    q = c.embeddings[int(corpus.pick_queries(c.modalities, 1, seed=9)[0])]
    runs = [mars_amd.tiled_query(ctx, c.embeddings, c.modalities, c.timestamps, q, T_Q,
                                 TiledQueryConfig(tile_size=t, top_k=20, time_decay_lambda=corpus.DECAY_LAMBDA))
            for t in (N, 5000, 1234, 640)]
    for r in runs[1:]:
        assert [x.node_id for x in r] == [x.node_id for x in runs[0]]
        assert [x.score for x in r] == [x.score for x in runs[0]]


def test_tiled_equals_resident_seeds(data):
    """With no BFS, the HBM-resident query's seeds are the tiled answer."""
    c, og, ctx = data
    g = mars_amd.MemoryGraph(N, 768, None, None, c.embeddings, c.modalities, c.timestamps)
    dg = mars_amd.upload_to_device(g)
    qc = mars_amd.create_query_context(N, 768, 64)
    try:
        for node in corpus.pick_queries(c.modalities, 4, seed=3):
            q = c.embeddings[node]
            cfg = mars_amd.RetrievalConfig(top_k=10, bfs_max_hops=0, time_decay_lambda=corpus.DECAY_LAMBDA)
            mars_amd.query_memory_fast(dg, qc, q, T_Q, cfg)
            seeds, vals = qc.last_seeds()
            res = mars_amd.tiled_query(ctx, c.embeddings, c.modalities, c.timestamps, q, T_Q,
                                       TiledQueryConfig(tile_size=4096, top_k=10,
                                                        time_decay_lambda=corpus.DECAY_LAMBDA))
            assert [r.node_id for r in res] == seeds.tolist()
            assert [r.score for r in res] == vals.tolist()
    finally:
        mars_amd.destroy_query_context(qc)
        mars_amd.free_device(dg)


def test_all_rows_filtered_returns_nothing(data):
    c, og, ctx = data
    res = mars_amd.tiled_query(ctx, c.embeddings, c.modalities, c.timestamps, c.embeddings[0], T_Q,
                               TiledQueryConfig(tile_size=7000, top_k=10, modality_filter=7))
    assert res == []


def test_pinned_host_corpus(data):
    c, og, ctx = data
    bufs = [mars_amd.HostBuffer(c.embeddings.shape, np.float32), mars_amd.HostBuffer((N,), np.int32),
            mars_amd.HostBuffer((N,), np.float32)]
    try:
        bufs[0].array[:] = c.embeddings
        bufs[1].array[:] = c.modalities
        bufs[2].array[:] = c.timestamps
        q = c.embeddings[int(corpus.pick_queries(c.modalities, 1, seed=12)[0])]
        cfg = TiledQueryConfig(tile_size=2500, top_k=10, time_decay_lambda=corpus.DECAY_LAMBDA)
        a = mars_amd.tiled_query(ctx, bufs[0].array, bufs[1].array, bufs[2].array, q, T_Q, cfg)
        b = mars_amd.tiled_query(ctx, c.embeddings, c.modalities, c.timestamps, q, T_Q, cfg)
        assert a == b
        check(c, og, a, q, corpus.DECAY_LAMBDA, 10, 2500, -1)
    finally:
        for b in bufs:
            b.free()


def test_tiled_argument_errors(data):
    c, og, ctx = data
    q = c.embeddings[0]
    with pytest.raises(MarsError) as e:
        mars_amd.tiled_query(ctx, c.embeddings, c.modalities, c.timestamps, q, T_Q, TiledQueryConfig(top_k=65))
    assert e.value.code == -5
    small = mars_amd.create_tiled_context(1000, 768, 16)
    try:
        with pytest.raises(MarsError) as e:
            mars_amd.tiled_query(small, c.embeddings, c.modalities, c.timestamps, q, T_Q,
                                 TiledQueryConfig(tile_size=5000))
        assert e.value.code == -4
        with pytest.raises(MarsError) as e:
            mars_amd.tiled_query(small, c.embeddings[:, :512], c.modalities, c.timestamps, q[:512], T_Q,
                                 TiledQueryConfig(tile_size=500))
        assert e.value.code == -1
        res = mars_amd.tiled_query(small, c.embeddings, c.modalities, c.timestamps, q, T_Q,
                                   TiledQueryConfig(tile_size=1000, top_k=16))
        check(c, og, res, q, 1e-8, 16, 1000, -1)
    finally:
        mars_amd.destroy_tiled_context(small)
