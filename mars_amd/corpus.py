"""Seeded benchmark corpus (include/mars_corpus.h) as numpy arrays.

``make_corpus(n, dim, seed)`` returns embeddings, modalities, timestamps and
episode ids; ``nsn_graph`` adds the NSN CSR (intra-episode pairs + k-NN,
symmetrised); ``pick_queries`` draws IMAGE query nodes.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional

import numpy as np

from ._lib import CorpusParamsC, check, lib

QUERY_TIME = 600.0          # seconds: every timestamp of the corpus is <= 600
DECAY_LAMBDA = 0.1          # per second
KNN_K = 8


@dataclass
class Corpus:
    embeddings: np.ndarray   # (n, dim) float32, unit rows
    modalities: np.ndarray   # (n,) int32
    timestamps: np.ndarray   # (n,) float32
    episode_ids: np.ndarray  # (n,) int32
    seed: int
    row_offsets: Optional[np.ndarray] = None
    col_indices: Optional[np.ndarray] = None

    @property
    def num_nodes(self) -> int:
        return int(self.embeddings.shape[0])

    @property
    def dim(self) -> int:
        return int(self.embeddings.shape[1])


def _p(a: np.ndarray):
    return C.c_void_p(a.ctypes.data)


def make_corpus(n: int, dim: int = 768, seed: int = 2026, threads: int = 0, embeddings: bool = True,
                out_emb: Optional[np.ndarray] = None) -> Corpus:
    """Seeded corpus of the benchmark generator; out_emb (an (n, dim) float32 C-contiguous
    array, e.g. a pinned HostBuffer view) receives the rows instead of a new array."""
    p = CorpusParamsC()
    lib.mars_corpus_default(C.byref(p), int(n), int(dim), int(seed))
    if out_emb is not None:
        if out_emb.shape != (n, dim) or out_emb.dtype != np.float32 or not out_emb.flags.c_contiguous:
            raise ValueError("out_emb must be a C-contiguous float32 array of shape (n, dim)")
        emb = out_emb
    else:
        emb = np.empty((n, dim) if embeddings else (0, dim), np.float32)
    mods = np.empty(n, np.int32)
    ts = np.empty(n, np.float32)
    ep = np.empty(n, np.int32)
    check(lib.mars_corpus_generate(C.byref(p), _p(emb) if embeddings else None, _p(mods), _p(ts), _p(ep),
                                   int(threads)), "mars_corpus_generate")
    return Corpus(emb, mods, ts, ep, seed)


def knn_cpu(emb: np.ndarray, k: int = KNN_K, threads: int = 0):
    emb = np.ascontiguousarray(emb, np.float32)
    n, d = emb.shape
    nb = np.empty((n, k), np.int32)
    sims = np.empty((n, k), np.float32)
    check(lib.mars_knn_cpu(_p(emb), n, d, k, _p(nb), _p(sims), int(threads)), "mars_knn_cpu")
    return nb, sims


def knn(emb: np.ndarray, k: int = KNN_K, threads: int = 0) -> np.ndarray:
    """k-NN ids of every row: exact CPU k-NN (the GPU builder takes over where available)."""
    return knn_cpu(emb, k, threads)[0]


def build_nsn_csr(episode_ids: np.ndarray, knn: np.ndarray, threads: int = 0):
    ep = np.ascontiguousarray(episode_ids, np.int32)
    knn = np.ascontiguousarray(knn, np.int32)
    n = len(ep)
    k = knn.shape[1] if knn.ndim == 2 else 0
    row = np.empty(n + 1, np.int32)
    ne = C.c_int64()
    check(lib.mars_build_nsn_csr(n, _p(ep), _p(knn), k, _p(row), None, C.byref(ne), int(threads)),
          "mars_build_nsn_csr")
    col = np.empty(max(ne.value, 1), np.int32)
    check(lib.mars_build_nsn_csr(n, _p(ep), _p(knn), k, _p(row), _p(col), C.byref(ne), int(threads)),
          "mars_build_nsn_csr")
    return row, col[: ne.value]


def nsn_graph(c: Corpus, knn: Optional[np.ndarray] = None, threads: int = 0) -> Corpus:
    """Attach the NSN CSR: intra-episode pairs + k-NN (CPU exact k-NN unless given)."""
    if knn is None:
        knn, _ = knn_cpu(c.embeddings, KNN_K, threads)
    c.row_offsets, c.col_indices = build_nsn_csr(c.episode_ids, knn, threads)
    return c


def pick_queries(modalities: np.ndarray, n_queries: int, seed: int, modality: int = 2) -> np.ndarray:
    mods = np.ascontiguousarray(modalities, np.int32)
    out = np.empty(n_queries, np.int32)
    check(lib.mars_corpus_pick_queries(_p(mods), len(mods), modality, n_queries, int(seed), _p(out)),
          "mars_corpus_pick_queries")
    return out


NSN_RING, NSN_SKIPS, NSN_HUBS, NSN_REWIRE, NSN_BRIDGES = 0x1, 0x2, 0x4, 0x8, 0x10
NSN_ALL = 0x1F


def nsn_edges(modalities: np.ndarray, k: int = 6, p: float = 0.15, phases: int = NSN_ALL):
    """MemoryGraph::build_nsn_edges_configurable (src/memory_graph.cpp:102-189): the
    reference's 5-phase NSN graph over len(modalities) nodes. Returns (row_offsets, col)."""
    mods = np.ascontiguousarray(modalities, np.int32)
    n = len(mods)
    bound = C.c_int64()
    check(lib.mars_nsn_edges(n, _p(mods) if n else None, int(k), float(p), int(phases), None, None, 0,
                             C.byref(bound)), "mars_nsn_edges")
    row = np.zeros(n + 1, np.int32)
    col = np.empty(max(bound.value, 1), np.int32)
    ne = C.c_int64()
    check(lib.mars_nsn_edges(n, _p(mods) if n else None, int(k), float(p), int(phases), _p(row), _p(col),
                             len(col), C.byref(ne)), "mars_nsn_edges")
    return row, col[: ne.value].copy()


MOD_TEXT, MOD_AUDIO, MOD_IMAGE = 0, 1, 2


def cross_modal_hit(ids, modalities: np.ndarray, episode_ids: np.ndarray, query_episode: int, top: int = 15) -> bool:
    """episode_cross_modal_hit (demos/embodied_scene/bench_kids_sweep.cu:65-82): among the
    first `top` result ids, the query's episode has a TEXT node and an AUDIO node."""
    has = set()
    for nid in list(ids)[:top]:
        nid = int(nid)
        if 0 <= nid < len(episode_ids) and int(episode_ids[nid]) == query_episode:
            has.add(int(modalities[nid]))
    return MOD_TEXT in has and MOD_AUDIO in has


def cross_modal_recall(ids, modalities: np.ndarray, episode_ids: np.ndarray, query_episode: int,
                       members: np.ndarray, top: int = 15) -> float:
    """Fraction of the query episode's TEXT and AUDIO members (`members`: the episode's node
    ids) found among the first `top` result ids."""
    want = {int(m) for m in members if int(modalities[m]) in (MOD_TEXT, MOD_AUDIO)}
    if not want:
        return 1.0
    got = {int(x) for x in list(ids)[:top]}
    return len(want & got) / len(want)
