"""GPU parity at the benchmark's own sizes: N = 100K, 1M, 13M (streaming) and 50M rows of
D = 768, the seeded episode corpus (4 IMAGE / 3 TEXT / 3 AUDIO per 10-node episode,
timestamps in [0, 600] s, lambda = 0.1/s, query time 600 s, K = 10, depth-2 BFS).

Graphs (intra-episode pairs + 8 neighbours per node, symmetrised; the oracle reads the
same CSR, so parity does not depend on how the neighbours were found):
  * 100K and 1M: the benchmark's NSN graph with the exact 8-NN from the GPU builder (fp16
    MFMA candidates, exact fp32 rescoring);
  * 13M: the 8-NN within blocks of 1M consecutive ids (mars_graph_knn_blocked, about
    40 s; the exact all-pairs build takes 6 minutes);
  * 50M: 8 seeded uniform random neighbours per node (an exact 8-NN is 3.8e18 FLOP). The
    random edges give depth-2 visit sets of several thousand nodes, so the BFS, the
    certified path's interval marking and its visit-table fallback all run at full size.

Bars: those of tests/parity.py (fp32 scores within 1e-5 of max(|s|, w * sum|e q|), BFS
scales carried along the BFS, seeds equal up to near-ties, BFS visit order and hops
exact); the certified path (fp16 or int8 candidate scan, exact fp32 results)
bit-identical to the fp32 path;
batched fp16 MFMA scoring within 2e-3 of the fp32 oracle's scale. The reference's harness
reports recall against a CPU top-K at scale (latency_bench.cu:399-409); these tests
assert it.

Each size is one test class whose graph lives only while its tests run. The module is
named to run after the other GPU tests.
"""
from __future__ import annotations

import gc
import threading

import numpy as np
import pytest

import mars_amd
import oracle
from mars_amd import RetrievalConfig, corpus

from parity import LAM, T_Q, check_batch_topk, check_episode, check_global, check_results_exact, episode_cfg
from test_certificate import quantize_i8

pytestmark = pytest.mark.gpu
D = 768
THREADS = 16                      # host threads for corpus generation (the box's CPU share)
GCFG = RetrievalConfig(top_k=10, bfs_max_hops=2, time_decay_lambda=LAM, bfs_score_decay=0.5,
                       max_results_returned=15)


class ScaleGraph:
    """A resident graph of the benchmark corpus (first n rows of an n + extra corpus), its
    episode CSR, an fp16 copy, one query context, and the oracle's view of the same arrays."""

    def __init__(self, n, knn_k, extra=0, seed=2026, int8=False, knn_block=0, knn_random=False):
        self.full = corpus.make_corpus(n + extra, D, seed=seed, threads=THREADS)
        f = self.full
        self.n = n
        self.c = corpus.Corpus(f.embeddings[:n], f.modalities[:n], f.timestamps[:n], f.episode_ids[:n], seed)
        g = mars_amd.MemoryGraph(n, D, None, None, self.c.embeddings, self.c.modalities, self.c.timestamps)
        self.dg = mars_amd.upload_to_device(g, capacity_nodes=n + extra,
                                            capacity_edges=(int(n) * 10 + 1_000_000) if extra else 0)
        mars_amd.upload_fp16_embeddings(self.dg)
        if int8:
            mars_amd.upload_int8_embeddings(self.dg)
        if knn_random:
            nb = np.random.default_rng(seed + 1).integers(0, n, size=(n, knn_k), dtype=np.int32)
        elif knn_k:
            nb = mars_amd.graph_knn(self.dg, knn_k, block_rows=knn_block)
        else:
            nb = np.empty((n, 0), np.int32)
        corpus.nsn_graph(self.c, nb, threads=THREADS)
        mars_amd.set_csr(self.dg, self.c.row_offsets, self.c.col_indices)
        mars_amd.upload_episode_ids(self.dg, self.c.episode_ids)
        self.csr = mars_amd.build_episode_csr(self.c.episode_ids, n)
        mars_amd.upload_episode_csr(self.dg, self.csr)
        self.ctx = mars_amd.create_query_context(n + extra, D, 64)
        self.og = oracle.make_graph(self.c.embeddings, self.c.modalities, self.c.timestamps, self.c.row_offsets,
                                    self.c.col_indices, self.c.episode_ids)

    def query(self, q, cfg, t_q=T_Q):
        st = mars_amd.RetrievalStats()
        return mars_amd.query_memory_fast(self.dg, self.ctx, q, t_q, cfg, st), st

    def close(self):
        mars_amd.destroy_query_context(self.ctx)
        mars_amd.free_device(self.dg)
        self.full = self.c = self.og = None
        gc.collect()


def certified_equals_fp32(sg: ScaleGraph, nodes, cfg=GCFG):
    """The certified path's answers equal the fp32 path's bit for bit; returns how many
    queries the certificate covered (the rest are answered by the fp32 scan inside the call)."""
    n_cert = 0
    try:
        for node in nodes:
            q = sg.full.embeddings[node]
            sg.ctx.certified = False
            want, _ = sg.query(q, cfg)
            sg.ctx.certified = True
            got, st = sg.query(q, cfg)
            check_results_exact(got, want)
            n_cert += st.seeds_certified
    finally:
        sg.ctx.certified = False
    return n_cert


# ------------------------------------------------------------------------------ N = 100K
@pytest.mark.timeout(600)
class TestScale100K:
    """N = 100,000 (Q=1 episode-scoped and global)."""

    @pytest.fixture(scope="class")
    def sg(self):
        s = ScaleGraph(100_000, knn_k=8)
        yield s
        s.close()

    def test_global_fp32_and_certified(self, sg):
        nodes = corpus.pick_queries(sg.c.modalities, 50, seed=1001)
        for node in nodes:
            check_global(sg, sg.c.embeddings[node], GCFG)
        assert certified_equals_fp32(sg, nodes) >= 45

    def test_episode_scoped(self, sg):
        for node in corpus.pick_queries(sg.c.modalities, 50, seed=1002):
            res = check_episode(sg, sg.c.embeddings[node], int(sg.c.episode_ids[node]), 10)
            assert len(res) == 10


# ------------------------------------------------------------------------------ N = 1M
@pytest.mark.timeout(600)
class TestScale1M:
    """N = 1,000,000: fp32 and fp16 rows, Q=1 episode-scoped and global, batched Q=64."""

    @pytest.fixture(scope="class")
    def sg(self):
        s = ScaleGraph(1_000_000, knn_k=8)
        yield s
        s.close()

    def test_global_fp32(self, sg):
        for node in corpus.pick_queries(sg.c.modalities, 20, seed=2001):
            check_global(sg, sg.c.embeddings[node], GCFG)

    def test_certified_bit_identical_200(self, sg):
        nodes = corpus.pick_queries(sg.c.modalities, 200, seed=2002)
        assert certified_equals_fp32(sg, nodes) >= 190

    def test_fp16_rows(self, sg):
        """The fp16 path against the oracle on the same RNE-rounded rows."""
        emb16 = oracle.to_f16_bits(sg.c.embeddings)
        sg.ctx.use_fp16 = True
        try:
            for node in corpus.pick_queries(sg.c.modalities, 5, seed=2003):
                res = check_global(sg, sg.c.embeddings[node], GCFG, emb16=emb16)
                assert len(res) == 15
        finally:
            sg.ctx.use_fp16 = False

    def test_episode_scoped(self, sg):
        for node in corpus.pick_queries(sg.c.modalities, 20, seed=2004):
            check_episode(sg, sg.c.embeddings[node], int(sg.c.episode_ids[node]), 10)

    def test_batched_q64(self, sg):
        nodes = corpus.pick_queries(sg.c.modalities, 64, seed=2005)
        qs = np.ascontiguousarray(sg.c.embeddings[nodes])
        buf = mars_amd.DeviceBuffer.from_array(qs)
        try:
            cfg = RetrievalConfig(top_k=10, time_decay_lambda=LAM)
            ids, sc = mars_amd.query_batch(sg.dg, sg.ctx, buf.ptr, 64, T_Q, cfg)
        finally:
            buf.free()
        check_batch_topk(sg.og, qs, np.full(64, T_Q, np.float32), cfg, ids, sc, sg.n)

    def test_int8_certified_bit_identical_200(self, sg):
        """The int8 candidate scan: its copy equals the numpy quantization (a sample of
        rows), and 200 certified answers equal the fp32 path's."""
        mars_amd.upload_int8_embeddings(sg.dg)
        try:
            for first in (0, 517_000, sg.n - 3000):
                b, m = mars_amd.read_int8(sg.dg, first, 3000)
                v, s, c = quantize_i8(sg.c.embeddings[first:first + 3000])
                np.testing.assert_array_equal(b, v)
                np.testing.assert_array_equal(m[:, 0], s)
                np.testing.assert_array_equal(m[:, 1], c)
            nodes = corpus.pick_queries(sg.c.modalities, 200, seed=2006)
            assert certified_equals_fp32(sg, nodes) >= 195
        finally:
            mars_amd.free_int8_embeddings(sg.dg)


# ------------------------------------------------------------------------------ N = 13M streaming
@pytest.mark.timeout(900)
class TestScale13MStreaming:
    """N = 13,000,000 fp32 + fp16 + int8 rows over the blocked 8-NN graph: global queries
    against the oracle, then one 10-node episode inserted with 8-NN edges on the graph's
    side stream while another context keeps querying (certified queries scan the int8
    copy, which the insert extends)."""

    N0, M = 13_000_000, 10

    @pytest.fixture(scope="class")
    def sg(self):
        s = ScaleGraph(self.N0, knn_k=8, knn_block=1_000_000, extra=self.M, int8=True)
        yield s
        s.close()

    def test_global_against_oracle(self, sg):
        """Depth-2 BFS over the k-NN edges: the fp32 path against the oracle, and the
        certified (int8 candidate) path bit-identical to it on 20 queries."""
        nodes = corpus.pick_queries(sg.c.modalities, 20, seed=3003)
        for node in nodes[:4]:
            res = check_global(sg, sg.c.embeddings[node], GCFG)
            assert len(res) == 15
        assert max(r.hops_from_seed for r in res) >= 1
        assert certified_equals_fp32(sg, nodes) >= 18

    def test_insert_under_queries(self, sg):
        n0, m, f = self.N0, self.M, sg.full
        old_row, old_col = sg.c.row_offsets, sg.c.col_indices
        ctx2 = mars_amd.create_query_context(n0 + m, D, 64, flags=mars_amd.MARS_CTX_CERTIFIED)
        qn = corpus.pick_queries(sg.c.modalities, 6, seed=3001)
        qeps = [int(sg.c.episode_ids[x]) for x in qn]

        def ask(i):
            node = int(qn[i // 2])
            if i % 2:
                cfg = episode_cfg(sg.csr, qeps[i // 2], 10, 15)
            else:
                cfg = GCFG
            return mars_amd.query_memory_fast(sg.dg, ctx2, f.embeddings[node], T_Q, cfg)

        before = [ask(i) for i in range(2 * len(qn))]
        seen, stop, errors = [], threading.Event(), []

        def loop():
            try:
                i = 0
                while not stop.is_set() or i < 4 * len(qn):
                    seen.append((i % (2 * len(qn)), ask(i % (2 * len(qn)))))
                    i += 1
            except Exception as e:                       # noqa: BLE001 - reported below
                errors.append(e)

        th = threading.Thread(target=loop)
        th.start()
        try:
            st, got = mars_amd.insert_nodes(sg.dg, f.embeddings[n0:], f.modalities[n0:], f.timestamps[n0:],
                                            f.episode_ids[n0:], knn_k=8, return_knn=True)
        finally:
            stop.set()
            th.join()
        assert not errors, errors
        assert st.first_node == n0 and st.nodes_added == m and 0 < st.queryable_us <= st.linked_us
        after = [ask(i) for i in range(2 * len(qn))]
        # concurrent answers: the graph before or after the insert (old-episode queries;
        # global queries whose seeds hold no new node, so the state between publishing
        # the rows and their edges answers as before)
        for i, res in seen:
            if i % 2 or all(r.node_id < n0 for r in after[i]):
                assert res == before[i] or res == after[i], i
        for i in range(1, 2 * len(qn), 2):
            assert after[i] == before[i]
        # k-NN of the new nodes over all n0 + m rows, against the fp64 oracle
        want, sims = oracle.knn(f.embeddings, np.arange(n0, n0 + m, dtype=np.int32), 8)
        e = f.embeddings
        for i in range(m):
            assert len(set(got[i].tolist())) == 8 and n0 + i not in got[i]
            for j in set(got[i].tolist()) ^ set(want[i].tolist()):
                s = float(e[n0 + i].astype(np.float64) @ e[j].astype(np.float64))
                assert abs(s - sims[i, 7]) <= 1e-5, (n0 + i, j, s, sims[i, 7])
        # the device CSR: the oracle's edge rule applied to the old CSR, bit for bit
        row, col = sg.dg.download_csr()
        wrow, wcol = oracle.insert_edges(old_row, old_col, n0, m, f.episode_ids[n0:], got)
        np.testing.assert_array_equal(row, wrow)
        np.testing.assert_array_equal(col, wcol)
        off, mem = sg.dg.download_episode_csr()
        woff, wmem = oracle.episode_csr(f.episode_ids)
        np.testing.assert_array_equal(off, woff)
        np.testing.assert_array_equal(mem, wmem)
        mars_amd.destroy_query_context(ctx2)
        # the grown graph against the oracle: a query on a new node and one on an old node
        sg.n = n0 + m
        sg.csr = mars_amd.build_episode_csr(f.episode_ids, n0 + m)
        sg.og = oracle.make_graph(f.embeddings, f.modalities, f.timestamps, wrow, wcol, f.episode_ids)
        new_img = n0 + int(np.nonzero(f.modalities[n0:] == 2)[0][0])
        for node in (new_img, int(qn[0])):
            check_global(sg, f.embeddings[node], GCFG)
        check_episode(sg, f.embeddings[new_img], int(f.episode_ids[new_img]), 10)
        # the inserted rows' int8 copy, then certified == fp32 on 20 queries of the grown
        # graph, the new nodes among them
        b, mt = mars_amd.read_int8(sg.dg, n0, m)
        v, sc, c = quantize_i8(f.embeddings[n0:n0 + m])
        np.testing.assert_array_equal(b, v)
        np.testing.assert_array_equal(mt, np.stack([sc, c], 1))
        nodes = np.concatenate([np.arange(n0, n0 + m), corpus.pick_queries(f.modalities, 10, seed=3002)])
        assert certified_equals_fp32(sg, nodes) >= 18


# ------------------------------------------------------------------------------ N = 50M resident
@pytest.mark.timeout(900)
class TestScale50M:
    """N = 50,000,000: 154 GB of fp32 rows, 77 GB of fp16 rows and 39 GB of int8 rows
    resident in HBM, over intra-episode pairs + 8 random neighbours per node."""

    @pytest.fixture(scope="class")
    def sg(self):
        s = ScaleGraph(50_000_000, knn_k=8, knn_random=True, int8=True)
        yield s
        s.close()

    def test_global_fp32_against_oracle(self, sg):
        for node in corpus.pick_queries(sg.c.modalities, 4, seed=4002):
            res = check_global(sg, sg.c.embeddings[node], GCFG)
            assert len(res) == 15
            assert sg.ctx.last_visited()[0].size > 1000         # the random edges' wide BFS

    def test_certified_equals_fp32(self, sg):
        """Over the int8 copy (the benchmark's path), then over the fp16 copy alone."""
        nodes = corpus.pick_queries(sg.c.modalities, 20, seed=4001)
        assert certified_equals_fp32(sg, nodes) >= 16
        mars_amd.free_int8_embeddings(sg.dg)
        assert certified_equals_fp32(sg, nodes[:10]) >= 8

    def test_episode_scoped(self, sg):
        for node in corpus.pick_queries(sg.c.modalities, 4, seed=4003):
            check_episode(sg, sg.c.embeddings[node], int(sg.c.episode_ids[node]), 10)

    def test_batched_q256(self, sg):
        nodes = corpus.pick_queries(sg.c.modalities, 256, seed=4004)
        qs = np.ascontiguousarray(sg.c.embeddings[nodes])
        buf = mars_amd.DeviceBuffer.from_array(qs)
        try:
            cfg = RetrievalConfig(top_k=10, time_decay_lambda=LAM)
            ids, sc = mars_amd.query_batch(sg.dg, sg.ctx, buf.ptr, 256, T_Q, cfg)
        finally:
            buf.free()
        check_batch_topk(sg.og, qs, np.full(256, T_Q, np.float32), cfg, ids, sc, sg.n, check_rows=range(0, 256, 16))
