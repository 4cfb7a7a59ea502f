"""mars_amd — MI355X (gfx950) retrieval hot path of MARS behind a C ABI.

Python mirror of the reference's query API (include/memory_cuda.cuh and
include/memory_graph.h of MARS), calling libmars_amd.so through ctypes:

    dg  = upload_to_device(graph)                  # memory_cuda.cuh:87
    upload_episode_ids(dg, episode_ids)            # :89-91
    upload_episode_csr(dg, build_episode_csr(ids, n))   # :92-93, memory_graph.h:77-78
    upload_fp16_embeddings(dg)                     # :96
    ctx = create_query_context(n, 768, max_k=64)   # :212-213
    res = query_memory_fast(dg, ctx, q, t, cfg, stats)  # :216-222
    destroy_query_context(ctx); free_device(dg)

Every query runs the HIP kernels of libmars_amd.so; there is no CPU path.
"""
from __future__ import annotations

import ctypes as C
import enum
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

from . import _lib
from ._lib import (MARS_CTX_CERTIFIED, MARS_CTX_TIMING, MARS_CTX_USE_FP16, MARS_CTX_USE_GRAPH, MARS_DESC_DEVICE_POINTERS,
                   MarsError, check, lib)

__all__ = [
    "Modality", "RetrievalScope", "RetrievalConfig", "RetrievalStats", "QueryResult", "MemoryGraph",
    "HostEpisodeCSR", "DeviceMemoryGraph", "QueryContext", "build_episode_csr", "upload_to_device",
    "upload_episode_ids", "upload_episode_csr", "upload_fp16_embeddings", "free_fp16_embeddings",
    "upload_int8_embeddings", "free_int8_embeddings", "read_int8",
    "free_device", "create_query_context", "destroy_query_context", "query_memory_fast",
    "query_memory_fast_device", "init", "MarsError", "corpus", "DeviceBuffer", "query_batch", "query_global_batch",
    "BatchStats", "query_global_batch_knn", "link", "link_knn", "graph_knn", "set_csr",
    "init_importance", "update_importance", "read_importance", "compute_novelty", "init_edge_hits",
    "count_edge_hits", "read_edge_hits", "maintain_graph", "set_rows",
]

MOD_TEXT, MOD_AUDIO, MOD_IMAGE = 0, 1, 2
# most results one query returns: the reference's compaction cap at max_k = 64 (64 * 500)
RESULT_CAP = 32000


class Modality(enum.IntEnum):                      # memory_graph.h:17-22
    TEXT = 0
    AUDIO = 1
    IMAGE = 2


class RetrievalScope(enum.IntEnum):                # memory_graph.h:79-81
    Global = 0
    EpisodeScoped = 1


@dataclass
class RetrievalConfig:                             # memory_cuda.cuh:107-127 (same defaults)
    top_k: int = 10
    bfs_max_hops: int = 2
    time_decay_lambda: float = 1e-8
    bfs_score_decay: float = 0.5
    modality_filter: int = -1
    use_importance: bool = False
    max_results_returned: int = -1
    retrieval_scope: RetrievalScope = RetrievalScope.Global
    query_episode_id: int = -1
    query_episode_member_begin: int = 0
    query_episode_member_count: int = 0
    episode_same_boost: float = 0.0

    def to_c(self) -> _lib.RetrievalConfigC:
        return _lib.RetrievalConfigC(
            int(self.top_k), int(self.bfs_max_hops), float(self.time_decay_lambda),
            float(self.bfs_score_decay), int(self.modality_filter), int(bool(self.use_importance)),
            int(self.max_results_returned), int(self.retrieval_scope), int(self.query_episode_id),
            int(self.query_episode_member_begin), int(self.query_episode_member_count),
            float(self.episode_same_boost))


@dataclass
class RetrievalStats:                              # memory_cuda.cuh:129-137 (+ extensions)
    gpu_ms_similarity: float = 0.0
    gpu_ms_topk: float = 0.0
    gpu_ms_bfs: float = 0.0
    gpu_ms_rerank: float = 0.0
    gpu_ms_total: float = 0.0
    nodes_scanned: int = 0
    bfs_waves: int = 0
    scope_fallback: int = 0
    visited: int = 0
    bfs_levels_run: int = 0
    used_fp16: int = 0
    seeds_certified: int = 0
    results_capped: int = 0
    wall_us: float = 0.0

    def _fill(self, s: _lib.StatsC) -> None:
        for name, _ in _lib.StatsC._fields_:
            setattr(self, name, getattr(s, name))


@dataclass(frozen=True)
class QueryResult:                                 # memory_cuda.cuh:100-105
    node_id: int
    score: float
    modality: int
    hops_from_seed: int


@dataclass
class MemoryGraph:                                 # memory_graph.h:25-60 (host arrays)
    num_nodes: int
    embedding_dim: int
    row_offsets: np.ndarray
    col_indices: np.ndarray
    embeddings: np.ndarray
    modalities: np.ndarray
    timestamps: np.ndarray

    @property
    def num_edges(self) -> int:
        return int(len(self.col_indices))


@dataclass
class HostEpisodeCSR:                              # memory_graph.h:70-75
    num_episodes: int = 0
    ep_csr_offsets: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int32))
    ep_csr_members: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int32))


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else C.c_void_p(a.ctypes.data)


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int32)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def init(device: int = 0) -> None:
    check(lib.mars_init(device), "mars_init")


def build_episode_csr(episode_ids, num_nodes: int) -> HostEpisodeCSR:
    """memory_graph.cpp:12-44 — counting sort of node ids by episode id."""
    ids = _i32(episode_ids)
    if num_nodes <= 0 or len(ids) != num_nodes:
        return HostEpisodeCSR()
    ne = C.c_int32(0)
    check(lib.mars_build_episode_csr(_ptr(ids), num_nodes, C.byref(ne), None, None), "build_episode_csr")
    off = np.zeros(ne.value + 1, np.int32)
    mem = np.zeros(num_nodes, np.int32)
    check(lib.mars_build_episode_csr(_ptr(ids), num_nodes, C.byref(ne), _ptr(off), _ptr(mem)),
          "build_episode_csr")
    return HostEpisodeCSR(ne.value, off, mem)


class DeviceMemoryGraph:
    """Handle of a device-resident graph (memory_cuda.cuh:63-85)."""

    def __init__(self, handle: C.c_void_p, num_nodes: int, num_edges: int, dim: int):
        self.handle = handle
        self.num_nodes = num_nodes
        self.num_edges = num_edges
        self.embedding_dim = dim

    def view(self) -> _lib.GraphViewC:
        v = _lib.GraphViewC()
        check(lib.mars_graph_get_view(self.handle, C.byref(v)), "mars_graph_get_view")
        return v

    @property
    def episode_num_episodes(self) -> int:
        return self.view().episode_num_episodes

    @property
    def episode_csr_member_total(self) -> int:
        return self.view().episode_csr_member_total

    def refresh(self) -> None:
        """Node / edge counts as published (they grow under streaming inserts)."""
        v = self.view()
        self.num_nodes, self.num_edges = int(v.num_nodes), int(v.num_edges)

    def download_csr(self):
        self.refresh()
        row = np.zeros(self.num_nodes + 1, np.int32)
        col = np.zeros(max(self.num_edges, 1), np.int32)
        check(lib.mars_graph_download(self.handle, _ptr(row), _ptr(col), None, None), "mars_graph_download")
        return row, col[: self.num_edges]

    def download_episode_csr(self):
        v = self.view()
        off = np.zeros(v.episode_num_episodes + 1, np.int32)
        mem = np.zeros(max(v.episode_csr_member_total, 1), np.int32)
        check(lib.mars_graph_download(self.handle, None, None, _ptr(off), _ptr(mem)), "mars_graph_download")
        return off, mem[: v.episode_csr_member_total]


def upload_to_device(g: MemoryGraph, capacity_nodes: int = 0, capacity_edges: int = 0) -> DeviceMemoryGraph:
    """upload_to_device (memory_cuda.cu:776-799)."""
    emb = _f32(g.embeddings).reshape(-1)
    mods, ts = _i32(g.modalities), _f32(g.timestamps)
    row = _i32(g.row_offsets) if g.row_offsets is not None else None
    col = _i32(g.col_indices) if g.col_indices is not None else None
    ne = 0 if col is None else int(len(col))
    desc = _lib.GraphDescC(int(g.num_nodes), ne, int(g.embedding_dim), _ptr(row).value if row is not None else None,
                           _ptr(col).value if col is not None and ne else None, emb.ctypes.data, mods.ctypes.data,
                           ts.ctypes.data, int(capacity_nodes), int(capacity_edges), 0)
    h = C.c_void_p()
    check(lib.mars_graph_create(C.byref(desc), C.byref(h)), "upload_to_device")
    return DeviceMemoryGraph(h, int(g.num_nodes), ne, int(g.embedding_dim))


def set_csr(dg: DeviceMemoryGraph, row_offsets, col_indices) -> None:
    """Replace the graph's NSN CSR (validated)."""
    row, col = _i32(row_offsets), _i32(col_indices)
    check(lib.mars_graph_set_csr(dg.handle, len(col), _ptr(row), _ptr(col) if len(col) else None), "mars_graph_set_csr")
    dg.num_edges = len(col)


def upload_episode_ids(dg: DeviceMemoryGraph, episode_ids) -> None:
    ids = _i32(episode_ids)
    check(lib.mars_graph_set_episode_ids(dg.handle, _ptr(ids), len(ids)), "upload_episode_ids")


def upload_episode_csr(dg: DeviceMemoryGraph, csr: HostEpisodeCSR) -> None:
    off, mem = _i32(csr.ep_csr_offsets), _i32(csr.ep_csr_members)
    tail = int(off[csr.num_episodes]) if csr.num_episodes > 0 else 0
    check(lib.mars_graph_set_episode_csr(dg.handle, int(csr.num_episodes), _ptr(off), _ptr(mem), tail),
          "upload_episode_csr")


def upload_fp16_embeddings(dg: DeviceMemoryGraph) -> None:
    check(lib.mars_graph_enable_fp16(dg.handle), "upload_fp16_embeddings")


def free_fp16_embeddings(dg: DeviceMemoryGraph) -> None:
    check(lib.mars_graph_disable_fp16(dg.handle), "free_fp16_embeddings")


def upload_int8_embeddings(dg: DeviceMemoryGraph) -> None:
    """The int8 copy of the rows that the certified global query scans (no reference
    counterpart; mars_graph_enable_int8)."""
    check(lib.mars_graph_enable_int8(dg.handle), "upload_int8_embeddings")


def free_int8_embeddings(dg: DeviceMemoryGraph) -> None:
    check(lib.mars_graph_disable_int8(dg.handle), "free_int8_embeddings")


def read_int8(dg: DeviceMemoryGraph, first: int = 0, count: int | None = None):
    """Rows [first, first + count) of the int8 copy: (bytes (count, d) int8, meta (count, 2)
    float32 = per-row scale and error bound)."""
    if count is None:
        dg.refresh()
        count = dg.num_nodes - first
    b = np.zeros((count, dg.embedding_dim), np.int8)
    m = np.zeros((count, 2), np.float32)
    check(lib.mars_graph_read_int8(dg.handle, first, count, _ptr(b), _ptr(m)), "read_int8")
    return b, m


def free_device(dg: DeviceMemoryGraph) -> None:
    if dg.handle:
        check(lib.mars_graph_destroy(dg.handle), "free_device")
        dg.handle = C.c_void_p()


class QueryContext:
    """Pre-allocated query context (memory_cuda.cuh:141-209): one per thread."""

    def __init__(self, handle: C.c_void_p, max_nodes: int, dim: int, max_k: int):
        self.handle = handle
        self.max_nodes = max_nodes
        self.embedding_dim = dim
        self.max_k = min(max_k, 64)
        self._out = (_lib.QueryResultC * RESULT_CAP)()

    def _flag(self, bit: int) -> bool:
        f = C.c_uint32()
        check(lib.mars_ctx_get_flags(self.handle, C.byref(f)), "mars_ctx_get_flags")
        return bool(f.value & bit)

    def _set(self, bit: int, on: bool) -> None:
        f = C.c_uint32()
        check(lib.mars_ctx_get_flags(self.handle, C.byref(f)), "mars_ctx_get_flags")
        v = (f.value | bit) if on else (f.value & ~bit)
        check(lib.mars_ctx_set_flags(self.handle, v), "mars_ctx_set_flags")

    use_fp16 = property(lambda s: s._flag(MARS_CTX_USE_FP16), lambda s, v: s._set(MARS_CTX_USE_FP16, v))
    use_cuda_graph = property(lambda s: s._flag(MARS_CTX_USE_GRAPH), lambda s, v: s._set(MARS_CTX_USE_GRAPH, v))
    timing = property(lambda s: s._flag(MARS_CTX_TIMING), lambda s, v: s._set(MARS_CTX_TIMING, v))
    # fp16 scan with certified exact seeds: the fp32 path's results at half the scan bytes
    certified = property(lambda s: s._flag(MARS_CTX_CERTIFIED), lambda s, v: s._set(MARS_CTX_CERTIFIED, v))

    def last_scores(self, n: int) -> np.ndarray:
        out = np.zeros(n, np.float32)
        check(lib.mars_ctx_last_scores(self.handle, _ptr(out), n), "mars_ctx_last_scores")
        return out

    def last_seeds(self):
        idx = np.zeros(64, np.int32)
        val = np.zeros(64, np.float32)
        k = C.c_int32()
        check(lib.mars_ctx_last_seeds(self.handle, _ptr(idx), _ptr(val), 64, C.byref(k)), "mars_ctx_last_seeds")
        return idx[: k.value].copy(), val[: k.value].copy()

    def last_phases(self, n: int = 3):
        """Phase durations (us) after the last global query's scan: 3 for the fp32 path,
        6 for the certified path (see mars_ctx_last_phases)."""
        us = np.zeros(n, np.float64)
        check(lib.mars_ctx_last_phases(self.handle, _ptr(us), n), "mars_ctx_last_phases")
        return us

    def last_visited(self):
        n = C.c_int32()
        check(lib.mars_ctx_last_visited(self.handle, None, None, None, 0, C.byref(n)), "mars_ctx_last_visited")
        ids = np.zeros(max(n.value, 1), np.int32)
        hops = np.zeros(max(n.value, 1), np.int32)
        sc = np.zeros(max(n.value, 1), np.float32)
        check(lib.mars_ctx_last_visited(self.handle, _ptr(ids), _ptr(hops), _ptr(sc), n.value, C.byref(n)),
              "mars_ctx_last_visited")
        return ids[: n.value], hops[: n.value], sc[: n.value]


def create_query_context(max_nodes: int, embedding_dim: int, max_k: int = 64, flags: int = MARS_CTX_TIMING) -> QueryContext:
    h = C.c_void_p()
    check(lib.mars_ctx_create(max_nodes, embedding_dim, max_k, flags, C.byref(h)), "create_query_context")
    return QueryContext(h, max_nodes, embedding_dim, max_k)


def destroy_query_context(ctx: QueryContext) -> None:
    if ctx.handle:
        check(lib.mars_ctx_destroy(ctx.handle), "destroy_query_context")
        ctx.handle = C.c_void_p()


def _results(ctx: QueryContext, n: int) -> List[QueryResult]:
    o = ctx._out
    return [QueryResult(o[i].node_id, o[i].score, o[i].modality, o[i].hops_from_seed) for i in range(min(n, RESULT_CAP))]


def query_memory_fast(dg: DeviceMemoryGraph, ctx: QueryContext, h_query, query_timestamp: float,
                      cfg: RetrievalConfig, stats: Optional[RetrievalStats] = None) -> List[QueryResult]:
    """query_memory_fast (memory_cuda.cu:1351-1464): results sorted by (score desc, id asc)."""
    q = _f32(h_query)
    if q.size != dg.embedding_dim:
        raise ValueError(f"query has {q.size} values, graph dim is {dg.embedding_dim}")
    n = C.c_int32()
    st = _lib.StatsC()
    c = cfg.to_c()
    check(lib.mars_query(dg.handle, ctx.handle, _ptr(q), float(query_timestamp), C.byref(c), ctx._out, RESULT_CAP,
                         C.byref(n), C.byref(st)), "query_memory_fast")
    if stats is not None:
        stats._fill(st)
    return _results(ctx, n.value)


def query_memory_fast_device(dg: DeviceMemoryGraph, ctx: QueryContext, d_query_ptr: int, query_timestamp: float,
                             cfg: RetrievalConfig, stats: Optional[RetrievalStats] = None) -> List[QueryResult]:
    """Same as query_memory_fast with the query vector already in device memory."""
    n = C.c_int32()
    st = _lib.StatsC()
    c = cfg.to_c()
    check(lib.mars_query_device(dg.handle, ctx.handle, C.c_void_p(d_query_ptr), float(query_timestamp),
                                C.byref(c), ctx._out, RESULT_CAP, C.byref(n), C.byref(st)), "query_memory_fast_device")
    if stats is not None:
        stats._fill(st)
    return _results(ctx, n.value)


def query_batch(dg: DeviceMemoryGraph, ctx: QueryContext, d_queries_ptr: int, n_queries: int, t_q,
                cfg: RetrievalConfig, stats: Optional[RetrievalStats] = None):
    """Batched global scoring (fp16 MFMA): returns (ids, scores), each (Q, top_k)."""
    tq = np.ascontiguousarray(np.broadcast_to(np.asarray(t_q, np.float32), (n_queries,)))
    ids = np.empty((n_queries, cfg.top_k), np.int32)
    sc = np.empty((n_queries, cfg.top_k), np.float32)
    st = _lib.StatsC()
    c = cfg.to_c()
    check(lib.mars_query_batch(dg.handle, ctx.handle, C.c_void_p(d_queries_ptr), int(n_queries), _ptr(tq), C.byref(c),
                               _ptr(ids), _ptr(sc), C.byref(st)), "mars_query_batch")
    if stats is not None:
        stats._fill(st)
    return ids, sc


def query_batch_static(dg: DeviceMemoryGraph, d_queries_ptr: int, n_queries: int, d_tq_ptr: int,
                       cfg: RetrievalConfig, d_ids_ptr: int, d_scores_ptr: int, uniform_tq: bool = False,
                       stream: Optional[int] = None) -> None:
    """query_batch with every buffer in device memory and no allocation (the library's static
    scratch): queries, times, ids (int32) and scores (fp32) are device pointers. Asynchronous
    on `stream` (None = the null stream)."""
    c = cfg.to_c()
    check(lib.mars_query_batch_static(dg.handle, C.c_void_p(d_queries_ptr), int(n_queries), C.c_void_p(d_tq_ptr),
                                      1 if uniform_tq else 0, C.byref(c), C.c_void_p(d_ids_ptr),
                                      C.c_void_p(d_scores_ptr), C.c_void_p(stream) if stream else None),
          "mars_query_batch_static")


def synchronize() -> None:
    """Wait for all work on the current device (its null stream included)."""
    check(lib.mars_device_synchronize(), "mars_device_synchronize")


@dataclass
class BatchStats:
    queries: int = 0
    batched: int = 0
    uncertified: int = 0
    overflow: int = 0
    whole_batch_q1: int = 0
    n_live: int = 0
    gpu_ms_scan: float = 0.0
    gpu_ms_seeds: float = 0.0
    gpu_ms_bfs: float = 0.0
    gpu_ms_total: float = 0.0
    min_margin: float = 0.0
    candidate_rows: int = 0          # 8: int8 pass, 16: fp16 MFMA scan, 24: int8 then fp16 for the k-NN
    wall_us: float = 0.0
    q1_us: float = 0.0

    def _fill(self, c) -> None:
        for f in ("queries", "batched", "uncertified", "overflow", "whole_batch_q1", "n_live", "gpu_ms_scan",
                  "gpu_ms_seeds", "gpu_ms_bfs", "gpu_ms_total", "min_margin", "candidate_rows", "wall_us", "q1_us"):
            setattr(self, f, getattr(c, f))


def query_global_batch(dg: DeviceMemoryGraph, ctx: QueryContext, d_queries_ptr: int, n_queries: int, t_q,
                       cfg: RetrievalConfig, cap: int = 64,
                       stats: Optional[BatchStats] = None) -> List[List[QueryResult]]:
    """Q global queries in one call (one shared scan: the int8 copy for up to 16 queries when
    the graph holds it, else the fp16 MFMA scan; certified exact seeds, batched BFS): query
    i's results are exactly query_memory_fast's for it (capped at cap)."""
    tq = np.ascontiguousarray(np.broadcast_to(np.asarray(t_q, np.float32), (n_queries,)))
    out = (_lib.QueryResultC * (max(1, n_queries * cap)))()
    n_out = np.zeros(n_queries, np.int32)
    st = _lib.BatchStatsC()
    c = cfg.to_c()
    check(lib.mars_query_global_batch(dg.handle, ctx.handle, C.c_void_p(d_queries_ptr), int(n_queries), _ptr(tq),
                                      C.byref(c), out, int(cap), _ptr(n_out), C.byref(st)), "mars_query_global_batch")
    if stats is not None:
        stats._fill(st)
    res = []
    for i in range(n_queries):
        b = i * cap
        res.append([QueryResult(out[b + j].node_id, out[b + j].score, out[b + j].modality, out[b + j].hops_from_seed)
                    for j in range(min(int(n_out[i]), cap))])
    return res


def graph_knn_range(dg: DeviceMemoryGraph, k: int, first: int, count: int) -> np.ndarray:
    """All-pairs k nearest neighbours of nodes first .. first + count - 1 (rows of graph_knn)."""
    out = np.empty((count, k), np.int32)
    check(lib.mars_graph_knn_range(dg.handle, int(k), int(first), int(count), _ptr(out)), "mars_graph_knn_range")
    return out


def graph_knn_report(dg: DeviceMemoryGraph):
    """(uncertified, rescanned) of the last k-NN builder call: nodes whose lists the
    certificate did not cover, and of those the ones found again by exact scans."""
    u, r = C.c_int64(), C.c_int64()
    check(lib.mars_graph_knn_report(dg.handle, C.byref(u), C.byref(r)), "mars_graph_knn_report")
    return int(u.value), int(r.value)


def graph_knn(dg: DeviceMemoryGraph, k: int = 8, block_rows: int = 0, progress=None,
              piece: int = 1 << 20) -> np.ndarray:
    """k nearest neighbours of every node (fp16 MFMA candidates + exact fp32 rescoring,
    certified; nodes the certificate misses are scanned again exactly in all-pairs builds);
    block_rows > 0: among the nodes of each block of block_rows consecutive ids
    (progress(done, total) is called after each block when given); block_rows = 0 with a
    progress callback: all pairs, in pieces of `piece` query nodes, progress after each.
    dg.knn_report gets the (uncertified, rescanned) node counts of the whole build."""
    out = np.empty((dg.num_nodes, k), np.int32)
    rep = [0, 0]

    def add():
        u, r = graph_knn_report(dg)
        rep[0] += u
        rep[1] += r

    if block_rows <= 0 and progress is not None:
        n = dg.num_nodes
        total = (n + piece - 1) // piece
        for b in range(total):
            lo = b * piece
            out[lo:lo + piece] = graph_knn_range(dg, k, lo, min(piece, n - lo))
            add()
            progress(b + 1, total)
    elif block_rows > 0 and progress is not None:
        nb = (dg.num_nodes + block_rows - 1) // block_rows
        for b in range(nb):                  # one block per call: the caller reports each
            lo = b * block_rows
            check(lib.mars_graph_knn_blocks(dg.handle, int(k), int(block_rows), b, 1, _ptr(out[lo:])),
                  "mars_graph_knn_blocks")
            add()
            progress(b + 1, nb)
    elif block_rows > 0:
        check(lib.mars_graph_knn_blocked(dg.handle, int(k), int(block_rows), _ptr(out)), "mars_graph_knn_blocked")
        add()
    else:
        check(lib.mars_graph_knn(dg.handle, int(k), _ptr(out)), "mars_graph_knn")
        add()
    dg.knn_report = tuple(rep)
    return out


# ---- files: MARS v1 graph checkpoints (persistence.h) and the KIDS corpus ----------------
def fnv1a64(data) -> int:
    """FNV-1a 64 of a bytes-like object (fnv1a_checksum, persistence.h:37)."""
    buf = np.frombuffer(bytes(data), np.uint8)
    out = C.c_uint64()
    check(lib.mars_fnv1a64(_ptr(buf) if buf.size else None, int(buf.size), C.byref(out)), "mars_fnv1a64")
    return int(out.value)


def save_graph(g: MemoryGraph, path) -> None:
    """save_graph (persistence.h:29): a MARS v1 file of a host graph."""
    ro, col = _i32(g.row_offsets), _i32(g.col_indices)
    emb = np.ascontiguousarray(g.embeddings, np.float32)
    mods, ts = _i32(g.modalities), np.ascontiguousarray(g.timestamps, np.float32)
    check(lib.mars_graph_file_save(str(path).encode(), int(g.num_nodes), int(len(col)), int(g.embedding_dim),
                                   _ptr(ro), _ptr(col), _ptr(emb), _ptr(mods), _ptr(ts)), "mars_graph_file_save")


def load_graph(path) -> MemoryGraph:
    """load_graph (persistence.h:33): a host graph from a MARS v1 file (MarsError when
    the magic, version, size or checksum does not check)."""
    p = str(path).encode()
    n, e, d = C.c_int32(), C.c_int32(), C.c_int32()
    check(lib.mars_graph_file_info(p, C.byref(n), C.byref(e), C.byref(d)), "mars_graph_file_info")
    n, e, d = n.value, e.value, d.value
    ro = np.zeros(n + 1, np.int32)
    col = np.zeros(max(e, 1), np.int32)
    emb = np.zeros((n, d), np.float32)
    mods = np.zeros(max(n, 1), np.int32)
    ts = np.zeros(max(n, 1), np.float32)
    check(lib.mars_graph_file_load(p, n, e, d, _ptr(ro), _ptr(col), _ptr(emb), _ptr(mods), _ptr(ts)),
          "mars_graph_file_load")
    return MemoryGraph(n, d, ro, col[:e], emb, mods[:n], ts[:n])


def save_device_graph(dg: DeviceMemoryGraph, path) -> None:
    """Checkpoint of the device-resident graph (inserts included) as a MARS v1 file."""
    check(lib.mars_graph_save(dg.handle, str(path).encode()), "mars_graph_save")


def write_kids_corpus(path, embeddings, timestamps, modalities, episode_ids) -> None:
    """KIDS binary corpus (bench_kids_sweep.cu:29-37, write_corpus_bin :84-102)."""
    emb = np.ascontiguousarray(embeddings, np.float32)
    n, d = emb.shape
    ts, mods, ep = np.ascontiguousarray(timestamps, np.float32), _i32(modalities), _i32(episode_ids)
    check(lib.mars_kids_file_write(str(path).encode(), int(n), int(d), _ptr(emb), _ptr(ts), _ptr(mods), _ptr(ep)),
          "mars_kids_file_write")


def read_kids_corpus(path):
    """(embeddings, timestamps, modalities, episode_ids) of a KIDS corpus file."""
    p = str(path).encode()
    n, d = C.c_int32(), C.c_int32()
    check(lib.mars_kids_file_info(p, C.byref(n), C.byref(d)), "mars_kids_file_info")
    n, d = n.value, d.value
    emb = np.zeros((n, d), np.float32)
    ts = np.zeros(max(n, 1), np.float32)
    mods = np.zeros(max(n, 1), np.int32)
    ep = np.zeros(max(n, 1), np.int32)
    check(lib.mars_kids_file_read(p, n, d, _ptr(emb), _ptr(ts), _ptr(mods), _ptr(ep)), "mars_kids_file_read")
    return emb, ts[:n], mods[:n], ep[:n]


def read_ceiling(dg: DeviceMemoryGraph, fp16: bool = True, reps: int = 20) -> float:
    """GB/s of a plain streaming read of the graph's rows (no arithmetic): the practical
    ceiling of the row scans on this device."""
    out = C.c_double()
    check(lib.mars_graph_read_ceiling(dg.handle, 1 if fp16 else 0, int(reps), C.byref(out)),
          "mars_graph_read_ceiling")
    return float(out.value)


READ_STREAM, READ_FRAGMENTS, READ_FRAGMENTS_NT, READ_STREAM_INT8 = 0, 1, 2, 3


def read_pattern(dg: DeviceMemoryGraph, pattern: int = READ_FRAGMENTS, reps: int = 20) -> float:
    """GB/s of a read of the rows in an access pattern, with no arithmetic: READ_STREAM
    (the plain stream of read_ceiling over the fp16 rows), READ_FRAGMENTS (the batched
    scan's 16 rows x 64 B per load instruction), READ_FRAGMENTS_NT (the same,
    non-temporal) or READ_STREAM_INT8 (the plain stream over the int8 copy)."""
    out = C.c_double()
    check(lib.mars_graph_read_pattern(dg.handle, int(pattern), int(reps), C.byref(out)), "mars_graph_read_pattern")
    return float(out.value)


@dataclass
class InsertStats:
    first_node: int
    nodes_added: int
    edges_added: int
    rows_relocated: int
    rows_appended: int
    queryable_us: float
    linked_us: float
    knn_us: float


# ---- importance, novelty gate, graph maintenance (memory_cuda.cuh:234-270) ----------
def init_importance(dg: DeviceMemoryGraph) -> None:
    check(lib.mars_importance_init(dg.handle), "mars_importance_init")


def update_importance(dg: DeviceMemoryGraph, result_ids, boost: float = 0.1, decay_rate: float = 0.001,
                      max_importance: float = 5.0, device_ptr: Optional[int] = None) -> None:
    """Decay every node, then boost result_ids (host ints), or n ids at device_ptr."""
    if device_ptr is not None:
        n = int(result_ids)
        check(lib.mars_importance_update(dg.handle, C.c_void_p(device_ptr), n, 1, boost, decay_rate, max_importance),
              "mars_importance_update")
        return
    ids = _i32(result_ids)
    check(lib.mars_importance_update(dg.handle, _ptr(ids) if len(ids) else None, len(ids), 0, boost, decay_rate,
                                     max_importance), "mars_importance_update")


def read_importance(dg: DeviceMemoryGraph, first: int = 0, count: Optional[int] = None) -> np.ndarray:
    dg.refresh()
    count = dg.num_nodes - first if count is None else count
    out = np.empty(max(count, 0), np.float32)
    check(lib.mars_importance_read(dg.handle, _ptr(out), int(first), int(count)), "mars_importance_read")
    return out


def compute_novelty(dg: DeviceMemoryGraph, query=None, ctx: Optional["QueryContext"] = None,
                    device_ptr: Optional[int] = None) -> float:
    """max_i <E_i, q> (>= -1; 0 for an empty graph). query: host vector, or device_ptr."""
    out = C.c_float()
    h = None if query is None else _f32(query)
    check(lib.mars_novelty(dg.handle, ctx.handle if ctx else None, _ptr(h) if h is not None else None,
                           C.c_void_p(device_ptr) if device_ptr is not None else None, C.byref(out)),
          "mars_novelty")
    return float(out.value)


def init_edge_hits(dg: DeviceMemoryGraph) -> None:
    check(lib.mars_edge_hits_init(dg.handle), "mars_edge_hits_init")


def count_edge_hits(dg: DeviceMemoryGraph, ctx: "QueryContext") -> None:
    """+1 on each edge from a node at hop h >= 1 to a node at hop h - 1 of ctx's last query."""
    check(lib.mars_edge_hits_count(dg.handle, ctx.handle), "mars_edge_hits_count")


def read_edge_hits(dg: DeviceMemoryGraph) -> np.ndarray:
    n = C.c_int64()
    check(lib.mars_edge_hits_read(dg.handle, None, 0, C.byref(n)), "mars_edge_hits_read")
    out = np.zeros(max(n.value, 1), np.int32)
    check(lib.mars_edge_hits_read(dg.handle, _ptr(out), len(out), C.byref(n)), "mars_edge_hits_read")
    return out[: n.value]


def maintain_graph(dg: DeviceMemoryGraph, min_hits: int = 0, window_queries: int = 1000) -> int:
    low = C.c_int32()
    check(lib.mars_graph_maintain(dg.handle, int(min_hits), int(window_queries), C.byref(low)), "mars_graph_maintain")
    return int(low.value)


def set_rows(dg: DeviceMemoryGraph, first: int, embeddings, modalities, timestamps) -> None:
    """Replace published rows first.. in place (rows, modalities, timestamps; edges kept)."""
    emb = _f32(embeddings).reshape(-1)
    mods, ts = _i32(modalities), _f32(timestamps)
    if len(ts) != len(mods) or emb.size != len(mods) * dg.embedding_dim:
        raise ValueError("set_rows: rows / modalities / timestamps disagree in length")
    check(lib.mars_graph_set_rows(dg.handle, int(first), len(mods), _ptr(emb), _ptr(mods), _ptr(ts)),
          "mars_graph_set_rows")


def insert_nodes(dg: DeviceMemoryGraph, embeddings, modalities, timestamps, episode_ids=None, knn_k: int = 8,
                 return_knn: bool = False):
    """Streaming insert (replaces StreamingBuffer::insert + flush, src/streaming.cpp:13-163):
    appends the rows on the graph's side stream, links each new node to its episode's
    new nodes and its knn_k nearest neighbours (both directions). Returns InsertStats
    (and the (n_new, knn_k) neighbour ids when return_knn)."""
    emb = _f32(embeddings).reshape(-1)
    mods, ts = _i32(modalities), _f32(timestamps)
    n_new = len(mods)
    if len(ts) != n_new or emb.size != n_new * dg.embedding_dim:
        raise ValueError("insert_nodes: rows / modalities / timestamps disagree in length")
    ep = _i32(episode_ids) if episode_ids is not None else None
    if ep is not None and len(ep) != n_new:
        raise ValueError("insert_nodes: one episode id per new node")
    knn = np.full((n_new, max(knn_k, 1)), -1, np.int32)
    st = _lib.InsertStatsC()
    check(lib.mars_graph_insert(dg.handle, n_new, _ptr(emb), _ptr(mods), _ptr(ts), _ptr(ep), int(knn_k),
                                _ptr(knn) if knn_k > 0 else None, C.byref(st)), "mars_graph_insert")
    dg.refresh()
    out = InsertStats(st.first_node, st.nodes_added, st.edges_added, st.rows_relocated, st.rows_appended,
                      st.queryable_us, st.linked_us, st.knn_us)
    return (out, knn[:, :knn_k]) if return_knn else out


def _istats(st) -> InsertStats:
    return InsertStats(st.first_node, st.nodes_added, st.edges_added, st.rows_relocated, st.rows_appended,
                       st.queryable_us, st.linked_us, st.knn_us)


def link_knn(dg: DeviceMemoryGraph, first: int, count: int, knn_k: int = 8, return_knn: bool = False):
    """Deferred k-NN edges of nodes [first, first + count) inserted with knn_k = 0 (the edge half of
    StreamingBuffer::add_incremental_edges_, src/streaming.cpp:97-163). Returns InsertStats
    (and the (count, knn_k) neighbour ids when return_knn)."""
    knn = np.full((max(count, 1), knn_k), -1, np.int32)
    st = _lib.InsertStatsC()
    check(lib.mars_graph_link_knn(dg.handle, int(first), int(count), int(knn_k), _ptr(knn), C.byref(st)),
          "mars_graph_link_knn")
    dg.refresh()
    return (_istats(st), knn[:count]) if return_knn else _istats(st)


def link(dg: DeviceMemoryGraph, first: int, nbrs) -> InsertStats:
    """Edges between node first + i and each id of nbrs[i] (-1 skipped), both directions (set union)."""
    nb = np.ascontiguousarray(nbrs, np.int32)
    if nb.ndim != 2:
        raise ValueError("link: nbrs must be (count, k)")
    st = _lib.InsertStatsC()
    check(lib.mars_graph_link(dg.handle, int(first), int(nb.shape[0]), int(nb.shape[1]), _ptr(nb), C.byref(st)),
          "mars_graph_link")
    dg.refresh()
    return _istats(st)


def query_global_batch_knn(dg: DeviceMemoryGraph, ctx: QueryContext, d_queries_ptr: int, n_queries: int, t_q,
                           cfg: RetrievalConfig, knn_first: int, knn_count: int, knn_k: int = 8, cap: int = 64,
                           stats: Optional[BatchStats] = None):
    """query_global_batch plus the neighbour search of nodes [knn_first, knn_first + knn_count)
    in the same corpus pass: returns (results, (knn_count, knn_k) neighbour ids)."""
    tq = np.ascontiguousarray(np.broadcast_to(np.asarray(t_q, np.float32), (n_queries,)))
    out = (_lib.QueryResultC * (max(1, n_queries * cap)))()
    n_out = np.zeros(max(1, n_queries), np.int32)
    knn = np.full((max(knn_count, 1), knn_k), -1, np.int32)
    st = _lib.BatchStatsC()
    c = cfg.to_c()
    check(lib.mars_query_global_batch_knn(dg.handle, ctx.handle, C.c_void_p(d_queries_ptr or None), int(n_queries),
                                          _ptr(tq), C.byref(c), out, int(cap), _ptr(n_out), C.byref(st),
                                          int(knn_first), int(knn_count), int(knn_k), _ptr(knn)),
          "mars_query_global_batch_knn")
    if stats is not None:
        stats._fill(st)
    res = []
    for i in range(n_queries):
        b = i * cap
        res.append([QueryResult(out[b + j].node_id, out[b + j].score, out[b + j].modality, out[b + j].hops_from_seed)
                    for j in range(min(int(n_out[i]), cap))])
    return res, knn[:knn_count]


@dataclass
class TiledQueryConfig:                             # tiled_query.h:33-39 (same defaults)
    tile_size: int = 5_000_000
    top_k: int = 10
    time_decay_lambda: float = 1e-8
    modality_filter: int = -1
    use_fp16: bool = True                           # accepted, no effect (as the reference)

    def to_c(self) -> _lib.TiledConfigC:
        return _lib.TiledConfigC(int(self.tile_size), int(self.top_k), float(self.time_decay_lambda),
                                 int(self.modality_filter), int(bool(self.use_fp16)))


@dataclass
class TiledQueryResult:                             # tiled_query.h:41-45
    node_id: int
    score: float
    modality: int


@dataclass
class TiledQueryStats:                              # tiled_query.h:47-54 (+ h2d_gbs)
    total_nodes: int = 0
    num_tiles: int = 0
    total_ms: float = 0.0
    transfer_ms: float = 0.0
    compute_ms: float = 0.0
    merge_ms: float = 0.0
    h2d_gbs: float = 0.0


class TiledQueryContext:
    """create_tiled_context (tiled_query.h:56-83): two device tile buffers."""

    def __init__(self, handle: C.c_void_p, max_tile_size: int, dim: int, max_k: int):
        self.handle, self.max_tile_size, self.embedding_dim, self.max_k = handle, max_tile_size, dim, max_k


def create_tiled_context(max_tile_size: int, embedding_dim: int, max_k: int = 64) -> TiledQueryContext:
    h = C.c_void_p()
    check(lib.mars_tiled_ctx_create(int(max_tile_size), int(embedding_dim), int(max_k), C.byref(h)),
          "create_tiled_context")
    return TiledQueryContext(h, int(max_tile_size), int(embedding_dim), int(max_k))


def destroy_tiled_context(ctx: TiledQueryContext) -> None:
    if ctx.handle:
        check(lib.mars_tiled_ctx_destroy(ctx.handle), "destroy_tiled_context")
        ctx.handle = C.c_void_p()


def tiled_query(ctx: TiledQueryContext, embeddings, modalities, timestamps, query, query_timestamp: float,
                cfg: TiledQueryConfig, stats: Optional[TiledQueryStats] = None) -> List[TiledQueryResult]:
    """tiled_query (tiled_query.cu:174-314) over host arrays (numpy, or HostBuffer views)."""
    emb = _f32(embeddings).reshape(-1)
    mods, ts, q = _i32(modalities), _f32(timestamps), _f32(query)
    n = len(mods)
    out = (_lib.TiledResultC * max(cfg.top_k, 1))()
    nout = C.c_int32()
    st = _lib.TiledStatsC()
    c = cfg.to_c()
    check(lib.mars_tiled_query(ctx.handle, _ptr(emb), _ptr(mods), _ptr(ts), n, len(q), _ptr(q),
                               C.c_float(query_timestamp), C.byref(c), out, cfg.top_k, C.byref(nout), C.byref(st)),
          "tiled_query")
    if stats is not None:
        for f in ("total_nodes", "num_tiles", "total_ms", "transfer_ms", "compute_ms", "merge_ms", "h2d_gbs"):
            setattr(stats, f, getattr(st, f))
    return [TiledQueryResult(out[i].node_id, out[i].score, out[i].modality) for i in range(min(nout.value, cfg.top_k))]


class HostBuffer:
    """Pinned host memory (hipHostMalloc) viewed as a numpy array; freed with free()."""

    def __init__(self, shape, dtype):
        self.array = None
        nbytes = int(np.prod(shape)) * np.dtype(dtype).itemsize
        p = C.c_void_p()
        check(lib.mars_host_alloc(nbytes, C.byref(p)), "mars_host_alloc")
        self.ptr = p.value
        buf = (C.c_char * max(nbytes, 1)).from_address(self.ptr)
        self.array = np.frombuffer(buf, dtype=dtype, count=int(np.prod(shape))).reshape(shape)

    def free(self) -> None:
        if self.ptr:
            self.array = None
            check(lib.mars_host_free(C.c_void_p(self.ptr)), "mars_host_free")
            self.ptr = None


class DeviceBuffer:
    """Device memory owned by libmars_amd's HIP runtime (holds e.g. query vectors)."""

    def __init__(self, nbytes: int):
        p = C.c_void_p()
        check(lib.mars_device_alloc(int(nbytes), C.byref(p)), "mars_device_alloc")
        self.ptr = p.value
        self.nbytes = int(nbytes)

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        check(lib.mars_copy_to_device(C.c_void_p(b.ptr), C.c_void_p(a.ctypes.data), a.nbytes), "mars_copy_to_device")
        return b

    def to_array(self, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype)
        check(lib.mars_copy_to_host(C.c_void_p(out.ctypes.data), C.c_void_p(self.ptr), out.nbytes), "mars_copy_to_host")
        return out

    def free(self) -> None:
        if self.ptr:
            check(lib.mars_device_free(C.c_void_p(self.ptr)), "mars_device_free")
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


from . import corpus  # noqa: E402  (needs lib)
