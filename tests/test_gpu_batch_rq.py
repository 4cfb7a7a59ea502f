"""GPU parity of the batched scoring kernel for 65 .. 1023 queries (k_batch_rq: 128 or 256
queries per workgroup in registers, 16-row tiles through LDS, a sampled score floor).

- against the fp32 oracle's top-K (the bar of tests/parity.py: scores within 2e-3 of the
  scale, id sets equal up to near-ties) at every supported width, both list sizes, with
  and without a modality filter, one or per-query times, ragged row counts;
- bit for bit against k_batch_scan (batches of at most 64 queries), which computes the
  same MFMA products in the same order: the same queries scored in one batch (256, 128 or
  96 queries) and in batches of 32 give the same ids and scores;
- with a corpus large enough that each row range is sampled for the score floor, against
  the oracle and bit for bit against batches of 32 (which take no floor);
- the neighbour-search form (plain dot products, the node itself excluded) against the
  exact CPU k-NN.
"""
from __future__ import annotations

import numpy as np
import pytest

import mars_amd
from mars_amd import RetrievalConfig, corpus

from parity import LAM, T_Q, Dev, batch_check, random_graph

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("d,q,k,filt,uniform", [(256, 129, 5, -1, True), (384, 200, 16, 1, False),
                                                 (512, 256, 8, 2, True), (768, 300, 10, -1, False),
                                                 (768, 520, 16, 0, True), (256, 1000, 3, -1, True),
                                                 (768, 65, 10, -1, True), (384, 96, 16, 2, False),
                                                 (512, 100, 8, -1, False), (768, 128, 16, 1, True)])
def test_rq_against_oracle(d, q, k, filt, uniform, rng):
    n = 3001                                   # ragged: not a multiple of the 16-row tile
    emb, mods, ts, row, col, _ = random_graph(rng, n, d)
    dev = Dev(emb, mods, ts, row, col, fp16=True)
    try:
        qn = rng.choice(n, q, replace=False)
        tq = np.float32(T_Q) if uniform else rng.uniform(300, 600, q).astype(np.float32)
        batch_check(dev, qn, RetrievalConfig(top_k=k, time_decay_lambda=LAM, modality_filter=filt), tq, emb)
    finally:
        dev.close()


@pytest.mark.parametrize("q,k,filt,uniform", [(256, 10, -1, True), (256, 5, 1, False), (128, 16, 2, True),
                                               (96, 10, -1, False)])
def test_rq_equals_scan_bit_for_bit(q, k, filt, uniform, rng):
    n, d = 20000, 768
    emb, mods, ts, row, col, _ = random_graph(rng, n, d)
    dev = Dev(emb, mods, ts, row, col, fp16=True)
    qs = np.ascontiguousarray(emb[rng.choice(n, q, replace=False)])
    tq = np.full(q, T_Q, np.float32) if uniform else rng.uniform(300, 600, q).astype(np.float32)
    cfg = RetrievalConfig(top_k=k, time_decay_lambda=LAM, modality_filter=filt)
    buf = mars_amd.DeviceBuffer.from_array(qs)
    try:
        ids, sc = mars_amd.query_batch(dev.dg, dev.ctx, buf.ptr, q, tq, cfg)                  # k_batch_rq
        parts = [mars_amd.query_batch(dev.dg, dev.ctx, buf.ptr + j * d * 4, 32, tq[j:j + 32], cfg)
                 for j in range(0, q, 32)]                                                   # k_batch_scan
    finally:
        buf.free()
        dev.close()
    np.testing.assert_array_equal(ids, np.concatenate([p[0] for p in parts]))
    np.testing.assert_array_equal(sc, np.concatenate([p[1] for p in parts]))


def test_rq_sampled_floor(rng):
    """200K rows, 600 queries (three 256-query groups over 80 row ranges of 2,512 rows):
    each range's first sixty-fourth (32 rows) is scored first and sets the queries' floors."""
    n, d = 200_000, 256
    emb = rng.standard_normal((n, d)).astype(np.float32)
    emb /= np.linalg.norm(emb, axis=1, keepdims=True)
    mods = rng.integers(0, 3, size=n).astype(np.int32)
    ts = rng.uniform(0, 600, size=n).astype(np.float32)
    dev = Dev(emb, mods, ts, None, None, fp16=True)
    try:
        qn = rng.choice(n, 600, replace=False)
        ids, _ = batch_check(dev, qn[:600], RetrievalConfig(top_k=10, time_decay_lambda=LAM), T_Q, emb)
        assert np.all(ids[:, 0] >= 0)
        batch_check(dev, qn[:300], RetrievalConfig(top_k=16, time_decay_lambda=LAM, modality_filter=1), T_Q, emb)
    finally:
        dev.close()


@pytest.mark.parametrize("q,k,filt,uniform", [(600, 10, -1, True), (300, 16, 1, False), (600, 5, 2, False)])
def test_rq_sampled_floor_equals_scan_bit_for_bit(q, k, filt, uniform, rng):
    """The sampled floor drops no row that belongs in a list: on 200K rows (each 256-query
    group's ranges sampled for the floor), the batch's ids and score bits equal those of
    the same queries scored in batches of 32 by k_batch_scan (no floor), with a modality
    filter and with per-query times too."""
    n, d = 200_000, 256
    emb = rng.standard_normal((n, d)).astype(np.float32)
    emb /= np.linalg.norm(emb, axis=1, keepdims=True)
    mods = rng.integers(0, 3, size=n).astype(np.int32)
    ts = rng.uniform(0, 600, size=n).astype(np.float32)
    dev = Dev(emb, mods, ts, None, None, fp16=True)
    qs = np.ascontiguousarray(emb[rng.choice(n, q, replace=False)])
    tq = np.full(q, T_Q, np.float32) if uniform else rng.uniform(300, 600, q).astype(np.float32)
    cfg = RetrievalConfig(top_k=k, time_decay_lambda=LAM, modality_filter=filt)
    buf = mars_amd.DeviceBuffer.from_array(qs)
    try:
        ids, sc = mars_amd.query_batch(dev.dg, dev.ctx, buf.ptr, q, tq, cfg)                  # sampled floor
        parts = [mars_amd.query_batch(dev.dg, dev.ctx, buf.ptr + j * d * 4, min(32, q - j), tq[j:j + 32], cfg)
                 for j in range(0, q, 32)]                                                   # k_batch_scan
    finally:
        buf.free()
        dev.close()
    np.testing.assert_array_equal(ids, np.concatenate([p[0] for p in parts]))
    np.testing.assert_array_equal(sc.view(np.uint32), np.concatenate([p[1] for p in parts]).view(np.uint32))


def test_rq_sampled_floor_sparse_filter_and_neighbours(rng):
    """280K rows, 300 queries (two 256-query groups over 128 row ranges of 2,192 rows,
    sampled): a modality filter that keeps 1 row in 2,000 (the sampled rows hold fewer than
    K of them, so the floors are -FLT_MAX scores), and the neighbour-search form (plain dot
    products, self excluded) over the same sampled ranges."""
    n, d = 280_000, 256
    emb = rng.standard_normal((n, d)).astype(np.float32)
    emb /= np.linalg.norm(emb, axis=1, keepdims=True)
    mods = (rng.random(n) < 0.0005).astype(np.int32)
    ts = rng.uniform(0, 600, size=n).astype(np.float32)
    dev = Dev(emb, mods, ts, None, None, fp16=True)
    try:
        qn = rng.choice(n, 300, replace=False)
        batch_check(dev, qn, RetrievalConfig(top_k=10, time_decay_lambda=LAM, modality_filter=1), T_Q, emb)
        got = mars_amd.graph_knn_range(dev.dg, 8, 5000, 300)
    finally:
        dev.close()
    q = emb[5000:5300]
    s = q @ emb.T
    s[np.arange(300), 5000 + np.arange(300)] = -np.inf
    want = np.argsort(-s, axis=1, kind="stable")[:, :8]
    for i in range(300):
        if not np.array_equal(np.sort(got[i]), np.sort(want[i])):
            kth = s[i, want[i, 7]]
            for j in set(got[i].tolist()) ^ set(want[i].tolist()):
                assert abs(s[i, j] - kth) <= 1e-3, (i, j)
    assert np.all(got != 5000 + np.arange(300)[:, None])


def test_rq_neighbour_search(rng):
    """graph_knn_range over 300 nodes runs one batch of 300 plain queries (self excluded)."""
    n, d = 2500, 512
    emb, mods, ts, _, _, _ = random_graph(rng, n, d)
    dev = Dev(emb, mods, ts, None, None, fp16=True)
    try:
        got = mars_amd.graph_knn_range(dev.dg, 8, 100, 300)
    finally:
        dev.close()
    want, sims = corpus.knn_cpu(emb, 8)
    s = emb[100:400] @ emb.T
    for i in range(300):
        s[i, 100 + i] = -np.inf
        if not np.array_equal(got[i], want[100 + i]):
            for j in set(got[i].tolist()) ^ set(want[100 + i].tolist()):
                assert abs(s[i, j] - sims[100 + i, 7]) <= 1e-3, (i, j)
    assert np.all(got != np.arange(100, 400)[:, None])
