"""The JSON-line engine server (mars_amd/mars_engine) on the GPU.

Default edges (--edges nsn, the reference server's policy, engine_server.cu:187-200): the
engine's QUERY answers against the CPU oracle on the engine's own graph (read back from its
SAVE file), whose edges are the reference's NSN builder's at the reference's rebuild points.

--edges knn: the engine adds no semantics of its own over the C ABI. The engine answers on
the certified path; a replica queried on the fp32 path and built with the same library calls
the engine makes (first ADD creates the graph, each later ADD is a one-node insert with
k-NN edges once 8 nodes exist, embeddings normalised as the engine does, DELETE as an
in-place tombstone) answers every QUERY with the same ids, modalities and hops, and scores
equal to the engine's 6-decimal output; SAVE writes the file the replica's checkpoint
writes, byte for byte, and a second engine LOADs it and answers the same.
"""
from __future__ import annotations

import json
import subprocess

import numpy as np
import pytest

import mars_amd
from mars_amd import RetrievalConfig, corpus

from conftest import ROOT

pytestmark = pytest.mark.gpu
ENGINE = ROOT / "mars_amd" / "mars_engine"
N, D, CAP = 300, 768, 1000


class Engine:
    def __init__(self, *args):
        self.p = subprocess.Popen([str(ENGINE), "--dim", str(D), "--capacity", str(CAP), *args],
                                  stdin=subprocess.PIPE, stdout=subprocess.PIPE, text=True, bufsize=1)

    def __call__(self, **req):
        self.p.stdin.write(json.dumps(req) + "\n")
        self.p.stdin.flush()
        return json.loads(self.p.stdout.readline())

    def close(self):
        if self.p.poll() is None:
            self.p.stdin.write(json.dumps({"cmd": "SHUTDOWN"}) + "\n")
            self.p.stdin.flush()
            self.p.stdout.readline()
        self.p.wait(timeout=60)


def normalised(e):
    """fp32 sum of squares in order, sqrt, + 1e-8 (engine_server.cu:164-170)."""
    sq = np.float32(0.0)
    for x in e.astype(np.float32):
        sq = np.float32(sq + np.float32(x * x))
    norm = np.float32(np.sqrt(sq)) + np.float32(1e-8)
    return (e.astype(np.float32) / norm).astype(np.float32)


def replica(c):
    rows = np.stack([normalised(c.embeddings[i]) for i in range(N)])
    g = mars_amd.MemoryGraph(1, D, np.zeros(2, np.int32), np.zeros(0, np.int32), rows[:1], c.modalities[:1],
                             c.timestamps[:1])
    dg = mars_amd.upload_to_device(g, capacity_nodes=CAP)
    mars_amd.upload_fp16_embeddings(dg)
    for i in range(1, N):
        mars_amd.insert_nodes(dg, rows[i:i + 1], c.modalities[i:i + 1], c.timestamps[i:i + 1], None,
                              knn_k=8 if i >= 8 else 0)
    return dg


def same_answer(eng, dg, ctx, q, t, top_k=10, hops=2, filt=-1):
    got = eng(cmd="QUERY", embedding=q.tolist(), top_k=top_k, bfs_max_hops=hops, modality_filter=filt, timestamp=t)
    cfg = RetrievalConfig(top_k=top_k, bfs_max_hops=hops, time_decay_lambda=1e-8, bfs_score_decay=0.5,
                          modality_filter=filt)
    want = mars_amd.query_memory_fast(dg, ctx, q, t, cfg)
    assert len(got["results"]) == len(want) and got["gpu_ms"] >= 0.0
    for g, w in zip(got["results"], want):
        assert (g["id"], g["modality"], g["hops"]) == (w.node_id, w.modality, w.hops_from_seed)
        assert g["score"] == float(f"{float(w.score):.6f}")
    return got["results"]


def test_engine_matches_library(tmp_path):
    c = corpus.make_corpus(N, D, seed=91)
    eng = Engine("--edges", "knn")
    dg = replica(c)
    ctx = mars_amd.create_query_context(CAP, D, 64)
    eng2 = None
    try:
        for i in range(N):
            assert eng(cmd="ADD", id=i, modality=int(c.modalities[i]), embedding=c.embeddings[i].tolist(),
                       timestamp=float(c.timestamps[i])) == {"ok": True}
        st = eng(cmd="STATS")
        row, col = dg.download_csr()
        assert st["n"] == N and st["edges"] == len(col) // 2 and st["vram_mb"] > 0.0
        qs = corpus.pick_queries(c.modalities, 8, seed=3)
        first = None
        for j, node in enumerate(qs):
            res = same_answer(eng, dg, ctx, c.embeddings[node], corpus.QUERY_TIME, top_k=5 + j, hops=j % 3,
                              filt=-1 if j % 2 else int(c.modalities[node]))
            first = first or res
        # DELETE leaves a tombstone: zero row, timestamp -1, modality kept
        victim = first[0]["id"]
        assert eng(cmd="DELETE", id=victim) == {"ok": True}
        mars_amd.set_rows(dg, victim, np.zeros((1, D), np.float32), c.modalities[victim:victim + 1],
                          np.float32([-1.0]))
        for node in qs[:4]:
            same_answer(eng, dg, ctx, c.embeddings[node], corpus.QUERY_TIME)
        # ADD of an existing id rewrites its row
        new = normalised(c.embeddings[qs[0]])
        assert eng(cmd="ADD", id=7, modality=2, embedding=c.embeddings[qs[0]].tolist(), timestamp=5.0) == {"ok": True}
        mars_amd.set_rows(dg, 7, new[None], np.int32([2]), np.float32([5.0]))
        same_answer(eng, dg, ctx, c.embeddings[qs[0]], corpus.QUERY_TIME)
        # SAVE: the replica's checkpoint byte for byte; LOAD into a second engine
        assert eng(cmd="SAVE", path=str(tmp_path / "eng.mars")) == {"ok": True}
        mars_amd.save_device_graph(dg, tmp_path / "rep.mars")
        assert (tmp_path / "eng.mars").read_bytes() == (tmp_path / "rep.mars").read_bytes()
        eng2 = Engine("--edges", "knn")
        assert eng2(cmd="LOAD", path=str(tmp_path / "eng.mars")) == {"ok": True, "n": N}
        for node in qs:
            q = c.embeddings[node].tolist()
            a = eng(cmd="QUERY", embedding=q, top_k=10, timestamp=corpus.QUERY_TIME)
            b = eng2(cmd="QUERY", embedding=q, top_k=10, timestamp=corpus.QUERY_TIME)
            assert a["results"] == b["results"]
        bad = tmp_path / "bad.mars"
        raw = bytearray((tmp_path / "eng.mars").read_bytes())
        raw[100] ^= 0xFF
        bad.write_bytes(bytes(raw))
        r = eng2(cmd="LOAD", path=str(bad))
        assert r["ok"] is False and "checksum" in r["error"]
    finally:
        eng.close()
        if eng2:
            eng2.close()
        mars_amd.destroy_query_context(ctx)
        mars_amd.free_device(dg)


def check_against_oracle(got, g, q, t, top_k, hops, filt):
    """Engine QUERY results against oracle.query on the engine's graph g (a MemoryGraph read
    from its SAVE file): the reference server's lambda 1e-8 and hop decay 0.5, K = top_k.
    Ids, modalities and hops exact up to near-ties; scores within the fp32 bar plus the
    6-decimal rounding of the response."""
    import oracle
    og = oracle.make_graph(g.embeddings, g.modalities, g.timestamps, g.row_offsets, g.col_indices)
    cfg = oracle.config(top_k, hops, 1e-8, 0.5, filt)
    ref = oracle.query(og, q, t, cfg)
    scl = oracle.result_scales(og, q, t, cfg, ref)
    want = ref["results"]
    assert len(got) == len(want)
    for r, w in zip(got, want):
        tol = 1e-5 * max(abs(w[1]), scl[w[0]]) + 5e-7
        if r["id"] == w[0]:
            assert abs(r["score"] - w[1]) <= tol and (r["modality"], r["hops"]) == (w[2], w[3]), (r, w)
        else:
            assert abs(r["score"] - w[1]) <= 2 * tol, (r, w)


def test_engine_nsn_edges_against_oracle(tmp_path):
    """ADDs in two waves around the reference's rebuild points: the first QUERY builds the
    NSN graph over 1,300 nodes; 600 more nodes (under 1000 new, not doubled) get no edges
    and leave the graph as it was; 800 more (1,400 since the build) trigger a rebuild over
    all 2,700. After each wave the engine's SAVE file holds exactly the reference builder's
    CSR over the nodes built (corpus.nsn_edges, edge-identical to the reference's own), and
    QUERY answers match the oracle on that graph."""
    from mars_amd import load_graph
    c = corpus.make_corpus(2700, D, seed=92)
    eng = Engine("--capacity", "4000")
    try:
        def add(lo, hi):
            for i in range(lo, hi):
                assert eng(cmd="ADD", id=i, modality=int(c.modalities[i]), embedding=c.embeddings[i].tolist(),
                           timestamp=float(c.timestamps[i])) == {"ok": True}

        def check(n_nodes, n_built, seed):
            path = tmp_path / f"e{n_nodes}.mars"
            assert eng(cmd="SAVE", path=str(path)) == {"ok": True}
            g = load_graph(path)
            assert g.num_nodes == n_nodes
            row, col = corpus.nsn_edges(c.modalities[:n_built], 6, 0.15)
            want_row = np.concatenate([row, np.full(n_nodes - n_built, row[-1], np.int32)])
            np.testing.assert_array_equal(g.row_offsets, want_row)
            np.testing.assert_array_equal(g.col_indices, col)
            for j, node in enumerate(corpus.pick_queries(c.modalities[:n_nodes], 6, seed=seed)):
                q = c.embeddings[node]
                top_k, hops, filt = 5 + 3 * j, j % 3, (-1 if j % 2 else int(c.modalities[node]))
                got = eng(cmd="QUERY", embedding=q.tolist(), top_k=top_k, bfs_max_hops=hops, modality_filter=filt,
                          timestamp=corpus.QUERY_TIME)["results"]
                check_against_oracle(got, g, q, corpus.QUERY_TIME, top_k, hops, filt)

        add(0, 1300)
        eng(cmd="QUERY", embedding=c.embeddings[0].tolist(), top_k=10, timestamp=corpus.QUERY_TIME)
        check(1300, 1300, 1)
        add(1300, 1900)
        check(1900, 1300, 2)
        add(1900, 2700)
        eng(cmd="QUERY", embedding=c.embeddings[0].tolist(), top_k=10, timestamp=corpus.QUERY_TIME)
        check(2700, 2700, 3)
        assert eng(cmd="STATS")["edges"] == len(corpus.nsn_edges(c.modalities, 6, 0.15)[1]) // 2
    finally:
        eng.close()
