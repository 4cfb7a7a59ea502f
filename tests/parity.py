"""Parity checks shared by the GPU tests: the HIP path (through the C ABI) against the
CPU oracle on the same inputs.

Bars (as these helpers apply them):
  * fused scores:  |gpu - oracle| <= rtol * max(|oracle|, w * sum_d |e_d q_d|), rtol = 1e-5
                   for fp32 (fp16 rows: against the oracle on the same RNE-rounded rows),
                   2e-3 for the fp16 path against the fp32 oracle;
  * BFS scores:    the same bound with the error scale carried along the BFS: a seed keeps
                   its own scale, a node reached from parent p takes
                   max(delta * scale_p, 0.8 * scale_u), the two terms its score is the
                   larger of (memory_cuda.cu:686-693, scripts/bench_cpu.py:128-134);
  * seeds / results: identical id sets except ids whose oracle score lies within
                   that tolerance of the cut;
  * BFS given the GPU's seeds: visit order (ids), hop levels and visited count
                   bit-exact;
  * episode CSR / episode-scoped results: ids and hops exact.
"""
from __future__ import annotations

import numpy as np

import mars_amd
import oracle
from mars_amd import RetrievalConfig, RetrievalScope, corpus

from conftest import RTOL_F16_VS_F32, RTOL_F32

FLT_MAX = float(np.finfo(np.float32).max)
T_Q = corpus.QUERY_TIME
LAM = corpus.DECAY_LAMBDA


class Dev:
    """A device graph and one query context over host arrays, with the oracle's view of
    the same arrays."""

    def __init__(self, emb, mods, ts, row, col, ep=None, max_k=64, fp16=False, capacity_nodes=0):
        self.n, self.d = emb.shape
        g = mars_amd.MemoryGraph(self.n, self.d, row, col, emb, mods, ts)
        self.dg = mars_amd.upload_to_device(g, capacity_nodes=capacity_nodes)
        self.csr = None
        if ep is not None:
            mars_amd.upload_episode_ids(self.dg, ep)
            self.csr = mars_amd.build_episode_csr(ep, self.n)
            mars_amd.upload_episode_csr(self.dg, self.csr)
        if fp16:
            mars_amd.upload_fp16_embeddings(self.dg)
        self.ctx = mars_amd.create_query_context(max(self.n, capacity_nodes), self.d, max_k)
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


def score_bound(ref, scl, rtol):
    return rtol * max(abs(ref), scl) + 1e-30


def check_global(dev: Dev, q, cfg: RetrievalConfig, emb16=None, rtol=RTOL_F32, t_q=T_Q, res=None, st=None):
    """Full global-query parity for one query; returns the GPU results. With res/st given,
    checks the context's last query (already run with q, cfg, t_q) instead of running it."""
    if res is None:
        res, st = dev.query(q, cfg, t_q)
    assert st.scope_fallback == 0 or cfg.retrieval_scope == RetrievalScope.EpisodeScoped
    og = dev.og
    if emb16 is not None:
        og = oracle.Graph(og.embeddings, og.modalities, og.timestamps, og.row_offsets, og.col_indices,
                          og.episode_ids, og.ep_offsets, og.ep_members, emb16)
    ref = oracle.query(og, q, t_q, ocfg(cfg))
    fin_ref = ref["final"]
    _, scale = oracle.scores(og, q, t_q, cfg.time_decay_lambda, cfg.modality_filter)
    if cfg.episode_same_boost > 0:
        scale = scale * (1.0 + cfg.episode_same_boost)
    tol = rtol * np.maximum(np.abs(fin_ref), scale)
    # 1) fused scores over all N
    fin_gpu = dev.ctx.last_scores(dev.n)
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
    bscale = oracle.bfs_scales(b, scale, cfg.bfs_score_decay)
    vtol = rtol * np.maximum(np.abs(b["scores"]), bscale) + 1e-30
    assert np.all(np.abs(vsc - b["scores"]) <= vtol)
    assert st.visited == len(ids)
    # 4) final results: oracle given the same seeds
    r2 = oracle.query(og, q, t_q, ocfg(cfg), seeds_in=seeds, cap=max(8192, len(res)))
    want = r2["results"]
    assert len(res) == len(want) == r2["n_results"]
    pos = {int(u): j for j, u in enumerate(b["ids"])}
    for j, (r, w) in enumerate(zip(res, want)):
        pr, pw = pos[r.node_id], pos[w[0]]
        if r.node_id != w[0]:
            assert abs(b["scores"][pr] - w[1]) <= 2 * (vtol[pr] + vtol[pw]), (j, r, w)
        assert r.hops_from_seed == b["hops"][pr]
        assert r.modality == int(dev.og.modalities[r.node_id])
        assert abs(r.score - b["scores"][pr]) <= vtol[pr]
    return res


def check_results_exact(a, b):
    """Two result lists equal in ids, modality, hops and score bits."""
    assert len(a) == len(b)
    for x, y in zip(a, b):
        assert (x.node_id, x.modality, x.hops_from_seed) == (y.node_id, y.modality, y.hops_from_seed), (x, y)
        assert np.float32(x.score).view(np.uint32) == np.float32(y.score).view(np.uint32), (x, y)


def episode_cfg(csr, ep, k=10, max_results=-1, lam=LAM):
    off = csr.ep_csr_offsets
    return RetrievalConfig(top_k=k, time_decay_lambda=lam, max_results_returned=max_results,
                           retrieval_scope=RetrievalScope.EpisodeScoped, query_episode_id=int(ep),
                           query_episode_member_begin=int(off[ep]),
                           query_episode_member_count=int(off[ep + 1] - off[ep]))


def check_episode_results(dev: Dev, q, cfg, res, t_q=T_Q):
    """Episode-scoped results against the oracle: ids and hops exact, scores to the fp32
    bar with each member's own scale (-FLT_MAX padding exact)."""
    ref = oracle.query(dev.og, q, t_q, ocfg(cfg))
    assert ref["scoped"]
    assert [r.node_id for r in res] == [w[0] for w in ref["results"]]
    _, scale = oracle.scores(dev.og, q, t_q, cfg.time_decay_lambda, cfg.modality_filter)
    for r, w in zip(res, ref["results"]):
        assert r.hops_from_seed == 0 == w[3]
        if w[1] == -FLT_MAX:
            assert r.score == np.float32(-FLT_MAX)
        else:
            assert abs(r.score - w[1]) <= score_bound(w[1], scale[w[0]], RTOL_F32), (r, w)
    return ref


def check_episode(dev: Dev, q, ep, k, t_q=T_Q):
    """Episode-scoped query against the oracle."""
    cfg = episode_cfg(dev.csr, ep, k, k)
    res, st = dev.query(q, cfg, t_q)
    assert st.scope_fallback == 0
    check_episode_results(dev, q, cfg, res, t_q)
    return res


def check_batch_topk(og, qs, tq, cfg, ids, sc, n, check_rows=None):
    """Batched scoring (fp16 MFMA) against the fp32 oracle: scores within 2e-3 of the scale,
    top-K id sets equal up to near-ties, each query's list sorted descending."""
    k = cfg.top_k
    rows = range(len(qs)) if check_rows is None else check_rows
    for i in rows:
        fin, scale = oracle.scores(og, qs[i], float(tq[i]), cfg.time_decay_lambda, cfg.modality_filter)
        want, _ = oracle.topk(fin, k)
        tol = RTOL_F16_VS_F32 * np.maximum(np.abs(fin), scale)
        got = ids[i][ids[i] >= 0]
        assert len(got) == min(k, n)
        ok = fin[got] != -FLT_MAX
        assert np.all(np.abs(sc[i][: len(got)][ok] - fin[got][ok]) <= tol[got][ok])
        kth = fin[want[-1]]
        for j in set(got.tolist()) ^ set(want.tolist()):
            assert abs(fin[j] - kth) <= 2 * (tol[j] + tol[want[-1]]), (i, j)
        assert np.all(np.diff(sc[i][: len(got)].astype(np.float64)) <= 0)      # sorted desc


def batch_check(dev: Dev, qnodes, cfg, t_q, emb):
    qs = emb[qnodes]
    buf = mars_amd.DeviceBuffer.from_array(qs)
    try:
        ids, sc = mars_amd.query_batch(dev.dg, dev.ctx, buf.ptr, len(qnodes), t_q, cfg)
    finally:
        buf.free()
    tq = np.broadcast_to(np.asarray(t_q, np.float32), (len(qnodes),))
    check_batch_topk(dev.og, qs, tq, cfg, ids, sc, dev.n)
    return ids, sc


def random_graph(rng, n, d, deg=6, n_ep=None):
    emb = rng.standard_normal((n, d)).astype(np.float32)
    emb /= np.linalg.norm(emb, axis=1, keepdims=True)
    mods = rng.integers(0, 3, size=n).astype(np.int32)
    ts = rng.uniform(0, 600, size=n).astype(np.float32)
    ep = (np.arange(n) // 10).astype(np.int32) if n_ep is None else np.sort(rng.integers(0, n_ep, n)).astype(np.int32)
    knn = rng.integers(0, n, size=(n, deg)).astype(np.int32)
    row, col = corpus.build_nsn_csr(ep, knn)
    return emb, mods, ts, row, col, ep
