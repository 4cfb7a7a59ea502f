"""GPU deferred k-NN linking (mars_graph_link / mars_graph_link_knn /
mars_query_global_batch_knn through the C ABI) against the oracle.

Bars (as applied here):
  * inserting with knn_k = 0 and then linking gives, bit for bit, the device CSR a
    single insert with knn_k gives (same neighbour lists, same edge rule);
  * the device CSR after every link equals oracle.link_edges (set union, rows
    ascending) applied to the previous CSR with the lists the GPU found;
  * a shared scan's neighbour lists equal mars_graph_link_knn's, and its global
    answers equal the Q=1 path's;
  * argument errors leave the graph unchanged.
"""
from __future__ import annotations

import threading

import numpy as np
import pytest

import mars_amd
import oracle
from mars_amd import BatchStats, RetrievalConfig, corpus
from mars_amd._lib import MarsError

from test_gpu_insert import BASE, EXTRA, K_NN, Live, check_device_csr, check_knn
from test_gpu_multi import assert_same

pytestmark = pytest.mark.gpu
T_Q = corpus.QUERY_TIME


@pytest.fixture(scope="module")
def full():
    return corpus.make_corpus(BASE + EXTRA, 768, seed=77)


def insert_plain(live, m):
    """Insert the next m nodes with episode pairs only (k-NN deferred)."""
    st, _ = live.insert(m, knn_k=0)
    return st


def link(live, first, count, k=K_NN):
    st, got = mars_amd.link_knn(live.dg, first, count, k, return_knn=True)
    live.row, live.col = oracle.link_edges(live.row, live.col, live.n, first, got)
    return st, got


def test_insert_then_link_equals_insert_with_knn(full):
    a = Live(full, BASE, BASE + 40)
    b = Live(full, BASE, BASE + 40)
    try:
        _, got_a = a.insert(30)
        insert_plain(b, 30)
        check_device_csr(b)
        st, got_b = link(b, BASE, 30)
        np.testing.assert_array_equal(got_b, got_a)
        check_knn(full, BASE + 30, BASE, got_b, K_NN)
        check_device_csr(b)
        ra, ca = a.dg.download_csr()
        rb, cb = b.dg.download_csr()
        np.testing.assert_array_equal(rb, ra)
        np.testing.assert_array_equal(cb, ca)
        assert st.nodes_added == 30 and st.edges_added > 0 and st.knn_us > 0
        # linking the same nodes again adds nothing
        st2, _ = link(b, BASE, 30)
        assert st2.edges_added == 0
        check_device_csr(b)
    finally:
        a.close()
        b.close()


def test_link_in_parts_after_several_inserts(full):
    """Three inserts, then two links over the published nodes: one insert of all 30
    nodes with k-NN gives the same graph (the lists are found over the same nodes)."""
    a = Live(full, BASE, BASE + 40)
    b = Live(full, BASE, BASE + 40)
    try:
        a.insert(30)
        for _ in range(3):
            insert_plain(b, 10)
        link(b, BASE, 20)
        check_device_csr(b)
        link(b, BASE + 20, 10)
        check_device_csr(b)
        ra, ca = a.dg.download_csr()
        rb, cb = b.dg.download_csr()
        np.testing.assert_array_equal(rb, ra)
        np.testing.assert_array_equal(cb, ca)
    finally:
        a.close()
        b.close()


def test_link_given_lists_and_unsorted_duplicates(full):
    """mars_graph_link with caller lists: -1, self and already present ids skipped;
    old rows that gain ids below their last entry are rewritten ascending."""
    live = Live(full, BASE, BASE + 20)
    try:
        insert_plain(live, 10)
        first = BASE
        nb = np.full((10, 4), -1, np.int32)
        nb[:, 0] = np.arange(first, first + 10) ^ 1          # an episode peer: present already
        nb[:, 1] = np.arange(first, first + 10)              # self
        nb[:, 2] = np.arange(10) * 7 + 5                     # old nodes, low ids
        nb[3, 3] = 2                                         # old node 2 gains a high id
        st = mars_amd.link(live.dg, first, nb)
        live.row, live.col = oracle.link_edges(live.row, live.col, live.n, first, nb)
        check_device_csr(live)
        assert st.edges_added == 2 * 11
        assert st.rows_relocated > 0
    finally:
        live.close()


def test_shared_scan_knn_equals_link_knn(full):
    a = Live(full, BASE, BASE + 40)
    b = Live(full, BASE, BASE + 40)
    try:
        insert_plain(a, 20)
        insert_plain(b, 20)
        qn = corpus.pick_queries(full.modalities[:BASE], 12, seed=31)
        qs = np.ascontiguousarray(full.embeddings[qn])
        buf = mars_amd.DeviceBuffer.from_array(qs)
        try:
            cfg = RetrievalConfig(top_k=10, time_decay_lambda=corpus.DECAY_LAMBDA)
            st = BatchStats()
            got, knn = mars_amd.query_global_batch_knn(a.dg, a.ctx, buf.ptr, len(qn), T_Q, cfg, BASE, 20, K_NN,
                                                       stats=st)
            want = [mars_amd.query_memory_fast_device(a.dg, a.ctx, buf.ptr + i * 768 * 4, T_Q, cfg)
                    for i in range(len(qn))]
            assert_same(got, want, cap=64)
            assert st.batched >= 10
            # neighbour search only (no global queries)
            _, knn0 = mars_amd.query_global_batch_knn(a.dg, a.ctx, 0, 0, T_Q, cfg, BASE, 20, K_NN)
            np.testing.assert_array_equal(knn0, knn)
        finally:
            buf.free()
        _, want_knn = link(b, BASE, 20)
        np.testing.assert_array_equal(knn, want_knn)
        mars_amd.link(a.dg, BASE, knn)
        ra, ca = a.dg.download_csr()
        rb, cb = b.dg.download_csr()
        np.testing.assert_array_equal(ra, rb)
        np.testing.assert_array_equal(ca, cb)
    finally:
        a.close()
        b.close()


def test_link_errors_leave_graph_unchanged(full):
    live = Live(full, BASE, BASE + 20)
    try:
        insert_plain(live, 10)
        row0, col0 = live.dg.download_csr()

        def bad(code, fn):
            with pytest.raises(MarsError) as e:
                fn()
            assert e.value.code == code
            row, col = live.dg.download_csr()
            np.testing.assert_array_equal(row, row0)
            np.testing.assert_array_equal(col, col0)

        bad(-1, lambda: mars_amd.link_knn(live.dg, BASE + 5, 10, K_NN))      # past the published nodes
        bad(-1, lambda: mars_amd.link_knn(live.dg, BASE, 10, 17))
        bad(-1, lambda: mars_amd.link(live.dg, BASE + 8, np.zeros((5, 2), np.int32)))
        mars_amd.free_fp16_embeddings(live.dg)
        bad(-5, lambda: mars_amd.link_knn(live.dg, BASE, 10, K_NN))
    finally:
        live.close()


def test_queries_while_linking(full):
    """Links land on the side stream while another thread queries: every query
    succeeds; afterwards the CSR matches the oracle and queries match the oracle."""
    live = Live(full, BASE, BASE + EXTRA)
    try:
        for _ in range(EXTRA // 10):
            insert_plain(live, 10)
        errors = []
        lists = []

        def linker():
            try:
                for j in range(EXTRA // 20):
                    _, got = mars_amd.link_knn(live.dg, BASE + 20 * j, 20, K_NN, return_knn=True)
                    lists.append(got)
            except Exception as exc:                      # reported below
                errors.append(exc)

        t = threading.Thread(target=linker)
        t.start()
        cfg = RetrievalConfig(top_k=10, bfs_max_hops=2, time_decay_lambda=corpus.DECAY_LAMBDA)
        qn = corpus.pick_queries(full.modalities[:BASE + EXTRA], 40, seed=8)
        n_q = 0
        while t.is_alive() or n_q < 40:
            res, _ = live.query(full.embeddings[qn[n_q % 40]], cfg)
            assert len(res) >= 10 and all(0 <= r.node_id < live.dg.num_nodes for r in res)
            n_q += 1
        t.join()
        assert not errors, errors
        for j, got in enumerate(lists):
            live.row, live.col = oracle.link_edges(live.row, live.col, live.n, BASE + 20 * j, got)
        check_device_csr(live)
        from parity import check_global
        for node in qn[:4]:
            check_global(live, full.embeddings[node], cfg)
    finally:
        live.close()
