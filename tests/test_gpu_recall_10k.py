"""The outcome metric of the N = 10,000 configuration: TEXT+AUDIO recall in the top 15.

Workload: the seeded benchmark corpus at N = 10,000, D = 768 (1,000 episodes of 4 IMAGE /
3 TEXT / 3 AUDIO nodes), NSN graph of intra-episode pairs + exact 8-NN, 1,000 IMAGE query
nodes at query time 600 s, K = 10, 15 results, decay lambda 0.1/s; global scope with
depth-2 BFS (hop decay 0.5) and episode scope.

Metrics per query (demos/embodied_scene/bench_kids_sweep.cu:65-82 for the first):
  * hit@15: the query's episode has a TEXT node and an AUDIO node among the 15 results;
  * recall@15: the fraction of the episode's 6 TEXT and AUDIO members among them.

Bar: the GPU's metric equals the oracle's on every query (the oracle runs from the GPU's
seeds, which must equal its own up to near-ties at the K-th score); a query whose two
result lists differ only by near-ties at the 15th score may differ in its metric and is
counted. Episode scope returns the whole 10-node episode: hit and recall 1.0.
"""
from __future__ import annotations

import numpy as np
import pytest

import mars_amd
import oracle
from mars_amd import RetrievalConfig, corpus

from parity import LAM, T_Q, Dev, episode_cfg, ocfg

pytestmark = pytest.mark.gpu
N_QUERIES = 1000
GCFG = RetrievalConfig(top_k=10, bfs_max_hops=2, time_decay_lambda=LAM, bfs_score_decay=0.5,
                       max_results_returned=15)


@pytest.fixture(scope="module")
def dev10k(corpus_10k):
    c = corpus_10k
    d = Dev(c.embeddings, c.modalities, c.timestamps, c.row_offsets, c.col_indices, c.episode_ids)
    yield d
    d.close()


def test_text_audio_recall_top15(dev10k, corpus_10k):
    c, dev = corpus_10k, dev10k
    off, mem = dev.csr.ep_csr_offsets, dev.csr.ep_csr_members
    nodes = corpus.pick_queries(c.modalities, N_QUERIES, seed=2026)
    qs = np.ascontiguousarray(c.embeddings[nodes])
    buf = mars_amd.DeviceBuffer.from_array(qs)
    g_hit, g_rec, o_hit, o_rec, e_hit, e_rec = [], [], [], [], [], []
    near_ties = 0
    try:
        for i, node in enumerate(nodes):
            ep = int(c.episode_ids[node])
            members = mem[off[ep]:off[ep + 1]]
            ptr = buf.ptr + i * qs.shape[1] * 4
            res = mars_amd.query_memory_fast_device(dev.dg, dev.ctx, ptr, T_Q, GCFG)
            seeds, _ = dev.ctx.last_seeds()
            ids = [r.node_id for r in res]
            assert len(ids) == 15
            # the oracle: its own seeds must equal the GPU's up to near-ties, then it runs from them
            ref = oracle.query(dev.og, qs[i], T_Q, ocfg(GCFG))
            fin = ref["final"]
            _, scale = oracle.scores(dev.og, qs[i], T_Q, LAM)
            tol = 1e-5 * np.maximum(np.abs(fin), scale)
            kth = ref["seeds"][-1]
            for j in set(seeds.tolist()) ^ set(ref["seeds"].tolist()):
                assert abs(fin[j] - fin[kth]) <= 2 * (tol[j] + tol[kth]), (i, j)
            ref = oracle.query(dev.og, qs[i], T_Q, ocfg(GCFG), seeds_in=seeds)
            want = [w[0] for w in ref["results"]]
            gh = corpus.cross_modal_hit(ids, c.modalities, c.episode_ids, ep)
            gr = corpus.cross_modal_recall(ids, c.modalities, c.episode_ids, ep, members)
            oh = corpus.cross_modal_hit(want, c.modalities, c.episode_ids, ep)
            orr = corpus.cross_modal_recall(want, c.modalities, c.episode_ids, ep, members)
            if set(ids) != set(want):
                # only near-ties at the 15th score: the oracle's BFS scores (from the same
                # seeds) of the ids in one list only, within the fp32 bar of the cut
                b = oracle.bfs(dev.og.row_offsets, dev.og.col_indices, fin, seeds, fin[seeds], 2, 0.5)
                bsc = oracle.bfs_scales(b, scale, 0.5)
                pos = {int(u): j for j, u in enumerate(b["ids"])}
                cut = ref["results"][-1][1]
                for x in set(ids) ^ set(want):
                    sx = b["scores"][pos[x]]
                    assert abs(sx - cut) <= 4e-5 * max(abs(cut), bsc[pos[x]]), (i, x, sx, cut)
                near_ties += 1
            else:
                assert (gh, gr) == (oh, orr), i
            g_hit.append(gh); g_rec.append(gr); o_hit.append(oh); o_rec.append(orr)
            # episode scope: the whole episode comes back
            eres = mars_amd.query_memory_fast_device(dev.dg, dev.ctx, ptr, T_Q, episode_cfg(dev.csr, ep, 10, 15))
            eids = [r.node_id for r in eres]
            assert sorted(eids) == sorted(members.tolist())
            e_hit.append(corpus.cross_modal_hit(eids, c.modalities, c.episode_ids, ep))
            e_rec.append(corpus.cross_modal_recall(eids, c.modalities, c.episode_ids, ep, members))
    finally:
        buf.free()
    print(f"N=10K, {N_QUERIES} IMAGE queries: global hit@15 {np.mean(g_hit):.4f} recall@15 {np.mean(g_rec):.4f} "
          f"(oracle {np.mean(o_hit):.4f} / {np.mean(o_rec):.4f}, {near_ties} near-tie lists); episode scope "
          f"{np.mean(e_hit):.4f} / {np.mean(e_rec):.4f}")
    assert near_ties <= N_QUERIES // 100
    assert abs(np.mean(g_hit) - np.mean(o_hit)) <= near_ties / N_QUERIES
    assert np.mean(e_hit) == 1.0 and np.mean(e_rec) == 1.0
