"""Certified global queries at other embedding widths (D = 256, 384, 512, 640, 1024, 1536).

The certified path has one kernel instance per width: k_scan8<NK> (NK = D / 64) for the
int8 candidate scan, k_scan<__half, QF16<D / 128>> for the fp16 one, and k_cert_bfs<QF32<D
/ 64>> for the exact rescoring. This file runs each instance on a seeded corpus of the
benchmark generator at that width (episodes of 4 IMAGE / 3 TEXT / 3 AUDIO, NSN graph of
intra-episode pairs + exact 8-NN).

Bars:
  * the int8 copy holds exactly the bytes, scales and bounds of quantize_i8 (the numpy
    restatement in test_certificate.py);
  * with MARS_CTX_CERTIFIED every global query returns bit for bit the fp32 path's
    results (ids, scores, modalities, hops, order, count), over the int8 copy and over
    the fp16 copy alone;
  * the certificate covers at least 90% of the K <= 16 queries where the width has an
    exact-rescoring kernel (D in 256, 384, 512, 768, 1024) and a candidate copy (int8: D
    a multiple of 256); at D = 640 and 1536 the flag leaves the fp32 scan to answer;
  * the fp32 path itself against the oracle (tests/parity.py) on a few queries.
"""
from __future__ import annotations

import numpy as np
import pytest

import mars_amd
from mars_amd import RetrievalConfig, corpus

from parity import LAM, check_global
from test_certificate import quantize_i8
from test_gpu_certified import both
from test_gpu_multi import CONFIGS, Dev, assert_same

pytestmark = pytest.mark.gpu
N = 8000
DIMS = [256, 384, 512, 640, 1024, 1536]
# K = 10 plain, max_results 15, K = 5 with hops 3 and 200 results, modality filter, K = 16
CFG_IDX = [0, 1, 3, 5, 7]


def fp16_width(d):
    return d in (256, 384, 512, 768, 1024)


def int8_width(d):
    return fp16_width(d) and d % 256 == 0


@pytest.fixture(scope="module", params=DIMS, ids=[f"d{d}" for d in DIMS])
def wide(request):
    d = request.param
    c = corpus.nsn_graph(corpus.make_corpus(N, d, seed=300 + d))
    dev = Dev(c.embeddings, c.modalities, c.timestamps, c.row_offsets, c.col_indices, c.episode_ids)
    yield d, c, dev
    dev.close()


def run_configs(dev, c, d, seed0):
    """Certified vs fp32 over CFG_IDX; returns (certified, asked) over the K <= 16 configs."""
    cert = asked = 0
    for ci in CFG_IDX:
        cfg = CONFIGS[ci]
        qn = corpus.pick_queries(c.modalities, 16, seed=seed0 + ci)
        got, stats, want = both(dev, c.embeddings[qn], cfg)
        assert_same(got, want)
        cert += sum(s.seeds_certified for s in stats)
        asked += len(qn)
    return cert, asked


def test_fp32_path_against_oracle(wide):
    d, c, dev = wide
    cfg = RetrievalConfig(top_k=10, bfs_max_hops=2, time_decay_lambda=LAM, max_results_returned=15)
    for node in corpus.pick_queries(c.modalities, 3, seed=40 + d):
        check_global(dev, c.embeddings[node], cfg)


def test_fp16_certified_equals_fp32(wide):
    d, c, dev = wide
    cert, asked = run_configs(dev, c, d, 4100 + d)
    print(f"D={d} fp16 candidates: {cert}/{asked} certified")
    if fp16_width(d):
        assert cert >= 0.9 * asked, (cert, asked)
    else:
        assert cert == 0


def test_int8_certified_equals_fp32(wide):
    d, c, dev = wide
    if d % 256 != 0:                     # no int8 copy at this width
        with pytest.raises(mars_amd.MarsError):
            mars_amd.upload_int8_embeddings(dev.dg)
        return
    mars_amd.upload_int8_embeddings(dev.dg)
    try:
        b, m = mars_amd.read_int8(dev.dg, 0, c.num_nodes)
        v, s, cb = quantize_i8(c.embeddings)
        np.testing.assert_array_equal(b, v)
        np.testing.assert_array_equal(m[:, 0], s)
        np.testing.assert_array_equal(m[:, 1], cb)
        cert, asked = run_configs(dev, c, d, 4200 + d)
        print(f"D={d} int8 candidates: {cert}/{asked} certified")
        if int8_width(d):
            assert cert >= 0.9 * asked, (cert, asked)
        else:
            assert cert == 0
    finally:
        mars_amd.free_int8_embeddings(dev.dg)
