"""Checkpoint of a device-resident graph (mars_graph_save) as a MARS v1 file.

Bar: after streaming inserts (k-NN edges linked in place, rows relocated), the file
holds exactly the published graph: the packed CSR the device returns, and the rows,
modalities and timestamps of every node, the inserted ones included; it loads through
the file reader (checksum checked) and rebuilds a device graph whose queries equal the
original's.
"""
from __future__ import annotations

import numpy as np
import pytest

import mars_amd
from mars_amd import RetrievalConfig, corpus

from test_gpu_insert import BASE, EXTRA, Live

pytestmark = pytest.mark.gpu


def test_device_checkpoint_after_inserts(tmp_path):
    full = corpus.make_corpus(BASE + EXTRA, 768, seed=78)
    live = Live(full, BASE, BASE + EXTRA)
    try:
        live.insert(20)
        live.insert(20, knn_k=0)
        n = BASE + 40
        path = tmp_path / "live.mars"
        mars_amd.save_device_graph(live.dg, path)
        g = mars_amd.load_graph(path)
        row, col = live.dg.download_csr()
        assert g.num_nodes == n and g.embedding_dim == 768
        np.testing.assert_array_equal(g.row_offsets, row)
        np.testing.assert_array_equal(g.col_indices, col)
        np.testing.assert_array_equal(g.embeddings, full.embeddings[:n])
        np.testing.assert_array_equal(g.modalities, full.modalities[:n])
        np.testing.assert_array_equal(g.timestamps, full.timestamps[:n])
        # the restored graph answers like the live one
        dg2 = mars_amd.upload_to_device(g)
        ctx2 = mars_amd.create_query_context(n, 768, 64)
        try:
            cfg = RetrievalConfig(top_k=10, time_decay_lambda=corpus.DECAY_LAMBDA)
            for node in corpus.pick_queries(full.modalities[:n], 6, seed=5):
                want, _ = live.query(full.embeddings[node], cfg)
                got = mars_amd.query_memory_fast(dg2, ctx2, full.embeddings[node], corpus.QUERY_TIME, cfg)
                assert got == want
        finally:
            mars_amd.destroy_query_context(ctx2)
            mars_amd.free_device(dg2)
    finally:
        live.close()
