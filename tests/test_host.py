"""Host-side tests of libmars_amd (no GPU): the C ABI loads and exports every
declared symbol, the corpus generator / k-NN / CSR builders hold their
invariants (the reference's T1-T7 / T18-T19 analogues), the product's episode
CSR is bit-exact with the reference's, and argument errors are reported
before any device work.
"""
from __future__ import annotations

import ctypes as C
import re

import numpy as np
import pytest

import mars_amd
from mars_amd import _lib, corpus

from conftest import ROOT


def _declared_functions():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(mars_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    names = _declared_functions()
    assert len(names) >= 25
    lib = C.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) <= set(_lib.SIGNATURES), sorted(set(names) - set(_lib.SIGNATURES))
    assert lib.mars_abi_version() == 1


def test_config_defaults_match_reference():
    c = _lib.RetrievalConfigC()
    _lib.lib.mars_config_default(C.byref(c))
    py = mars_amd.RetrievalConfig()
    for name, _ in _lib.RetrievalConfigC._fields_:
        assert getattr(c, name) == pytest.approx(float(getattr(py, name))), name
    assert (c.top_k, c.bfs_max_hops, c.modality_filter, c.max_results_returned) == (10, 2, -1, -1)
    assert c.bfs_score_decay == pytest.approx(0.5) and c.time_decay_lambda == pytest.approx(1e-8)


def test_struct_layouts():
    assert C.sizeof(_lib.QueryResultC) == 16
    assert C.sizeof(_lib.RetrievalConfigC) == 48
    assert C.sizeof(_lib.TiledResultC) == 12                      # TiledQueryResult
    assert C.sizeof(_lib.TiledConfigC) == 20
    assert C.sizeof(_lib.InsertStatsC) == 48
    assert C.sizeof(_lib.StatsC) == 64 and _lib.StatsC.wall_us.offset == 56
    assert _lib.InsertStatsC.queryable_us.offset == 24
    assert C.sizeof(_lib.StreamBenchC) == 128 and _lib.StreamBenchC.knn_k.offset == 88
    assert C.sizeof(_lib.BatchStatsC) == 64 and _lib.BatchStatsC.wall_us.offset == 48
    assert C.sizeof(_lib.ServeBenchC) == 216 and _lib.ServeBenchC.g_done_us.offset == 128
    assert _lib.ServeBenchC.ins_linked_us.offset == 192


def test_tiled_config_defaults_match_reference():
    """TiledQueryConfig defaults (include/tiled_query.h:33-39)."""
    c = _lib.TiledConfigC()
    _lib.lib.mars_tiled_config_default(C.byref(c))
    assert (c.tile_size, c.top_k, c.modality_filter, c.use_fp16) == (5_000_000, 10, -1, 1)
    assert c.time_decay_lambda == pytest.approx(1e-8)
    py = mars_amd.TiledQueryConfig()
    assert (py.tile_size, py.top_k, py.modality_filter) == (c.tile_size, c.top_k, c.modality_filter)


# ------------------------------------------------------------------ corpus
def test_corpus_deterministic_and_thread_independent():
    a = corpus.make_corpus(1234, 96, seed=5, threads=1)
    b = corpus.make_corpus(1234, 96, seed=5, threads=7)
    for x, y in [(a.embeddings, b.embeddings), (a.modalities, b.modalities), (a.timestamps, b.timestamps),
                 (a.episode_ids, b.episode_ids)]:
        np.testing.assert_array_equal(x, y)
    c = corpus.make_corpus(1234, 96, seed=6)
    assert not np.array_equal(a.embeddings, c.embeddings)


def test_corpus_workload_shape(corpus_small):
    c = corpus_small
    n = c.num_nodes
    np.testing.assert_allclose(np.linalg.norm(c.embeddings, axis=1), 1.0, atol=1e-5)     # T2 analogue
    slot = np.arange(n) % 10
    want_mod = np.where(slot < 4, 2, np.where(slot < 7, 0, 1))
    np.testing.assert_array_equal(c.modalities, want_mod)                                  # 4 IMAGE 3 TEXT 3 AUDIO
    np.testing.assert_array_equal(c.episode_ids, np.arange(n) // 10)
    assert c.timestamps.min() >= 0.0 and c.timestamps.max() <= 600.0
    span = np.array([np.ptp(c.timestamps[c.episode_ids == e]) for e in range(5)])
    assert np.all(span < 1.0)                                                              # packed in 1 s
    e = c.embeddings
    img_img = float(e[0] @ e[1])
    img_txt = float(e[0] @ e[4])
    cross = np.abs(e[:10] @ e[10:20].T).max()
    assert 0.85 < img_img < 0.97 and 0.15 < img_txt < 0.45 and cross < 0.2


def test_knn_cpu_exact(rng):
    emb = rng.standard_normal((600, 48)).astype(np.float32)
    emb /= np.linalg.norm(emb, axis=1, keepdims=True)
    emb[100] = emb[200]                                     # exact tie: lower id first
    nb, sims = corpus.knn_cpu(emb, 8)
    s = emb @ emb.T
    np.fill_diagonal(s, -np.inf)
    want = np.lexsort((np.broadcast_to(np.arange(600), s.shape), -s), axis=1)[:, :8]
    np.testing.assert_array_equal(nb, want)
    np.testing.assert_allclose(sims, np.take_along_axis(s, want, 1), rtol=1e-5, atol=1e-6)


def test_nsn_csr_invariants(corpus_small):
    c = corpus_small
    n, row, col = c.num_nodes, c.row_offsets, c.col_indices
    assert row[0] == 0 and row[-1] == len(col) and np.all(np.diff(row) >= 0)          # T3
    for i in range(0, n, 37):
        r = col[row[i]:row[i + 1]]
        assert np.all(np.diff(r) > 0) and np.all((r >= 0) & (r < n))                  # sorted, unique, in range
        assert i not in set(r)                                                         # T5
    edges = set()
    for i in range(n):
        for j in col[row[i]:row[i + 1]]:
            edges.add((i, int(j)))
    assert all((j, i) in edges for (i, j) in edges)                                    # T4
    for e in range(0, n // 10, 13):                                                    # intra-episode pairs
        mem = range(10 * e, 10 * e + 10)
        assert all((a, b) in edges for a in mem for b in mem if a != b)
    nb, _ = corpus.knn_cpu(c.embeddings[:50], 8)                                       # k-NN of a sub-corpus
    full_nb, _ = corpus.knn_cpu(c.embeddings, 8)
    assert all((i, int(j)) in edges for i in range(n) for j in full_nb[i])
    deg = np.diff(row)
    assert deg.min() >= 9 and deg.mean() < 40                                          # T7 analogue


def test_pick_queries_are_image_nodes(corpus_small):
    q = corpus.pick_queries(corpus_small.modalities, 500, seed=3)
    assert np.all(corpus_small.modalities[q] == 2)
    np.testing.assert_array_equal(q, corpus.pick_queries(corpus_small.modalities, 500, seed=3))
    assert len(np.unique(q)) > 300


# ------------------------------------------------------------------ episode CSR
def test_product_episode_csr_matches_golden(golden):
    z = np.load(golden / "episode_csr.npz")
    for name in ("kids30", "shuffled", "single", "one_node"):
        ids = z[f"{name}_ids"]
        csr = mars_amd.build_episode_csr(ids, len(ids))
        assert csr.num_episodes == int(z[f"{name}_num"])
        np.testing.assert_array_equal(csr.ep_csr_offsets, z[f"{name}_offsets"])
        np.testing.assert_array_equal(csr.ep_csr_members, z[f"{name}_members"])


def test_product_episode_csr_edge_cases():
    assert mars_amd.build_episode_csr([], 0).num_episodes == 0          # memory_graph.cpp:15-16
    assert mars_amd.build_episode_csr([0, 1], 3).num_episodes == 0      # size mismatch -> empty
    with pytest.raises(mars_amd.MarsError):
        mars_amd.build_episode_csr([0, -1, 2], 3)                       # negative id: rejected


# ------------------------------------------------------------------ errors before device work
def _desc(n=4, d=8, row=None, col=None):
    emb = np.ones((n, d), np.float32)
    mods = np.zeros(n, np.int32)
    ts = np.zeros(n, np.float32)
    keep = (emb, mods, ts, row, col)
    desc = _lib.GraphDescC(n, 0 if col is None else len(col), d,
                           None if row is None else row.ctypes.data, None if col is None else col.ctypes.data,
                           emb.ctypes.data, mods.ctypes.data, ts.ctypes.data, 0, 0, 0)
    return desc, keep


@pytest.mark.parametrize("row,col,msg", [
    ([0, 1, 1, 1, 2], [1, 5], "out of range"),
    ([0, 2, 2, 2, 2], [1, 1], "twice"),
    ([1, 1, 1, 1, 1], [2], "expected 0"),
    ([0, 2, 1, 2, 2], [1, 2], "decrease"),
    ([0, 1, 1, 1, 3], [1, 2], "expected num_edges"),
])
def test_graph_create_rejects_bad_csr(row, col, msg):
    desc, keep = _desc(row=np.array(row, np.int32), col=np.array(col, np.int32))
    h = C.c_void_p()
    rc = _lib.lib.mars_graph_create(C.byref(desc), C.byref(h))
    assert rc == -1 and msg in _lib.lib.mars_last_error().decode()
    assert not h.value


def test_ctx_create_rejects_bad_sizes():
    h = C.c_void_p()
    assert _lib.lib.mars_ctx_create(0, 768, 10, 0, C.byref(h)) == -1
    assert _lib.lib.mars_ctx_create(10, 768, 0, 0, C.byref(h)) == -1


def test_no_silent_cpu_path_without_gpu():
    """Without a gfx950 device every device entry point fails loudly."""
    try:
        mars_amd.init(0)
    except mars_amd.MarsError as e:
        assert e.code in (-2, -6)
    else:
        pytest.skip("a gfx950 device is present")
    desc, keep = _desc()
    h = C.c_void_p()
    assert _lib.lib.mars_graph_create(C.byref(desc), C.byref(h)) in (-2, -6)


def test_cross_modal_metrics():
    """hit@15 / recall@15 of the recall pass (bench_kids_sweep.cu:65-82's hit rule) on a
    hand-made episode: members 10-19 (TEXT 10-12, AUDIO 13-15, IMAGE 16-19)."""
    mods = np.array([2] * 10 + [0, 0, 0, 1, 1, 1, 2, 2, 2, 2] + [0, 1] * 5, np.int32)
    ep = np.array([0] * 10 + [1] * 10 + [2] * 10, np.int32)
    members = np.arange(10, 20)
    # TEXT and AUDIO of episode 1, plus other episodes' TEXT / AUDIO (not counted)
    ids = [16, 20, 21, 10, 13, 11]
    assert corpus.cross_modal_hit(ids, mods, ep, 1)
    assert corpus.cross_modal_recall(ids, mods, ep, 1, members) == 3 / 6
    # only TEXT of the episode: no hit
    assert not corpus.cross_modal_hit([10, 11, 21, 16], mods, ep, 1)
    # the AUDIO node beyond the first `top` results does not count
    assert not corpus.cross_modal_hit([10] + [0] * 14 + [13], mods, ep, 1)
    assert corpus.cross_modal_hit([10] + [0] * 13 + [13], mods, ep, 1)
    assert corpus.cross_modal_recall([10] + [0] * 14 + [13], mods, ep, 1, members) == 1 / 6
    # the whole episode: hit and recall 1
    assert corpus.cross_modal_recall(list(members), mods, ep, 1, members) == 1.0
    # out-of-range ids are skipped
    assert not corpus.cross_modal_hit([-1, 99, 10], mods, ep, 1)
