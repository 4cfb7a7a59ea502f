"""CPU oracle of the retrieval hot path (ctypes over oracle/liboracle.so).

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, which compare GPU results against it or time it as the
CPU baseline. The product (mars_amd) never imports it.

``ref`` (oracle/_ref/libref.so, built from the reference's own host sources
when the reference tree is present) is None when that library is absent.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from pathlib import Path
from typing import Optional

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_PATH = HERE / "_ref" / "libref.so"

VP = C.c_void_p
I32, I64 = C.c_int32, C.c_int64


class OracleConfig(C.Structure):
    _fields_ = [
        ("top_k", I32), ("bfs_max_hops", I32), ("time_decay_lambda", C.c_float),
        ("bfs_score_decay", C.c_float), ("modality_filter", I32), ("use_importance", I32),
        ("max_results_returned", I32), ("retrieval_scope", I32), ("query_episode_id", I32),
        ("query_episode_member_begin", I32), ("query_episode_member_count", I32),
        ("episode_same_boost", C.c_float),
    ]


class OracleGraph(C.Structure):
    _fields_ = [
        ("num_nodes", I64), ("dim", I32), ("pad0", I32), ("row_offsets", VP), ("col_indices", VP),
        ("emb", VP), ("emb16", VP), ("modalities", VP), ("timestamps", VP), ("episode_ids", VP),
        ("ep_offsets", VP), ("ep_members", VP), ("num_episodes", I32), ("member_total", I32),
    ]


class OracleResult(C.Structure):
    _fields_ = [("node_id", I32), ("score", C.c_double), ("modality", I32), ("hops", I32)]


def _load():
    if not LIB_PATH.exists():
        raise ImportError(f"{LIB_PATH} missing: run `make -C oracle`")
    lib = C.CDLL(str(LIB_PATH))
    sig = {
        "oracle_num_threads": (C.c_int, []),
        "oracle_set_num_threads": (None, [C.c_int]),
        "oracle_half_to_double": (C.c_double, [C.c_uint16]),
        "oracle_float_to_half_rne": (C.c_uint16, [C.c_float]),
        "oracle_convert_f16": (None, [VP, VP, I64]),
        "oracle_build_episode_csr": (C.c_int, [VP, I32, C.POINTER(I32), VP, VP]),
        "oracle_scores": (None, [C.POINTER(OracleGraph), VP, C.c_float, C.c_float, I32, VP, VP]),
        "oracle_topk": (I32, [VP, I64, I32, VP, VP]),
        "oracle_bfs": (I32, [VP, VP, I64, VP, VP, VP, I32, I32, C.c_double, VP, VP, VP, VP, I32, VP, VP]),
        "oracle_query": (I32, [C.POINTER(OracleGraph), VP, C.c_float, C.POINTER(OracleConfig), I32, VP, I32,
                               VP, VP, VP, VP, I32, VP]),
        "oracle_tiled_query": (I32, [C.POINTER(OracleGraph), VP, C.c_float, C.c_float, I32, I32, I32, VP, VP]),
        "oracle_knn": (None, [VP, I64, I32, VP, I32, I32, VP, VP]),
        "oracle_insert_edges": (I64, [I32, VP, VP, I32, VP, VP, I32, VP, VP]),
        "oracle_link_edges": (I64, [I32, VP, VP, I32, I32, VP, I32, VP, VP]),
        "oracle_importance_update": (None, [VP, I32, VP, I32, C.c_float, C.c_float, C.c_float]),
        "oracle_novelty": (C.c_double, [C.POINTER(OracleGraph), VP, C.POINTER(C.c_double)]),
        "oracle_edge_hits": (None, [VP, VP, I32, VP, VP]),
        "oracle_maintain": (I32, [VP, I64, I32]),
        "oracle_kids_probes": (None, [I32, I64, I32, VP]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    return lib


lib = _load()


def _load_ref():
    if not REF_PATH.exists():
        return None
    r = C.CDLL(str(REF_PATH))
    sig = {
        "ref_build_episode_csr": (C.c_int, [VP, I32, C.POINTER(I32), VP, VP]),
        "ref_kids_make": (VP, [I32, I32, C.c_uint32, I32, C.c_double]),
        "ref_synthetic_make": (VP, [I32, I32, I32, I32, C.c_uint32, I32, C.c_double]),
        "ref_graph_sizes": (None, [VP, C.POINTER(I32), C.POINTER(I32), C.POINTER(I32)]),
        "ref_graph_copy": (None, [VP, VP, VP, VP, VP, VP, VP]),
        "ref_stream_flush": (I32, [VP, I32, I32, I32, VP, VP, VP]),
        "ref_graph_free": (None, [VP]),
        "ref_fnv1a": (C.c_uint64, [VP, C.c_size_t]),
        "ref_nsn_edges": (I64, [I32, VP, I32, C.c_double, C.c_uint32, VP, VP, I64]),
        "ref_save_graph": (C.c_int, [C.c_char_p, I32, I32, I32, VP, VP, VP, VP, VP]),
        "ref_load_graph": (C.c_int, [C.c_char_p, C.POINTER(I32), C.POINTER(I32), C.POINTER(I32), VP, VP, VP, VP,
                                     VP]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(r, name)
        fn.restype, fn.argtypes = res, args
    return r


ref = _load_ref()


def _p(a: Optional[np.ndarray]):
    return None if a is None else C.c_void_p(a.ctypes.data)


@dataclass
class Graph:
    """Host arrays the oracle reads (kept alive here)."""
    embeddings: np.ndarray
    modalities: np.ndarray
    timestamps: np.ndarray
    row_offsets: Optional[np.ndarray] = None
    col_indices: Optional[np.ndarray] = None
    episode_ids: Optional[np.ndarray] = None
    ep_offsets: Optional[np.ndarray] = None
    ep_members: Optional[np.ndarray] = None
    emb16: Optional[np.ndarray] = None      # uint16 bits; if set, scores use the fp16 rows

    def c(self) -> OracleGraph:
        n, d = self.embeddings.shape
        ne = 0 if self.ep_offsets is None else len(self.ep_offsets) - 1
        mt = 0 if self.ep_offsets is None else int(self.ep_offsets[-1])
        return OracleGraph(n, d, 0, _p(self.row_offsets), _p(self.col_indices), _p(self.embeddings),
                           _p(self.emb16), _p(self.modalities), _p(self.timestamps), _p(self.episode_ids),
                           _p(self.ep_offsets), _p(self.ep_members), ne, mt)


def make_graph(emb, mods, ts, row=None, col=None, ep_ids=None, fp16: bool = False) -> Graph:
    g = Graph(np.ascontiguousarray(emb, np.float32), np.ascontiguousarray(mods, np.int32),
              np.ascontiguousarray(ts, np.float32),
              None if row is None else np.ascontiguousarray(row, np.int32),
              None if col is None else np.ascontiguousarray(col, np.int32),
              None if ep_ids is None else np.ascontiguousarray(ep_ids, np.int32))
    if ep_ids is not None:
        g.ep_offsets, g.ep_members = episode_csr(g.episode_ids)
    if fp16:
        g.emb16 = to_f16_bits(g.embeddings)
    return g


def to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib.oracle_convert_f16(_p(x), _p(out), x.size)
    return out


def episode_csr(ids: np.ndarray):
    ids = np.ascontiguousarray(ids, np.int32)
    ne = I32()
    rc = lib.oracle_build_episode_csr(_p(ids), len(ids), C.byref(ne), None, None)
    if rc != 0:
        raise ValueError("negative episode id")
    off = np.zeros(ne.value + 1, np.int32)
    mem = np.zeros(len(ids), np.int32)
    lib.oracle_build_episode_csr(_p(ids), len(ids), C.byref(ne), _p(off), _p(mem))
    return off, mem


def scores(g: Graph, q, t_q: float, lam: float, mod_filter: int = -1):
    q = np.ascontiguousarray(q, np.float32)
    n = g.embeddings.shape[0]
    fin = np.empty(n, np.float64)
    scl = np.empty(n, np.float64)
    gc = g.c()
    lib.oracle_scores(C.byref(gc), _p(q), t_q, lam, mod_filter, _p(fin), _p(scl))
    return fin, scl


def topk(fin: np.ndarray, k: int):
    fin = np.ascontiguousarray(fin, np.float64)
    idx = np.empty(k, np.int32)
    val = np.empty(k, np.float64)
    m = lib.oracle_topk(_p(fin), len(fin), k, _p(idx), _p(val))
    return idx[:m], val[:m]


def bfs(row, col, fin, seeds, seed_vals, hops: int, decay: float):
    row = None if row is None else np.ascontiguousarray(row, np.int32)
    col = None if col is None else np.ascontiguousarray(col, np.int32)
    fin = np.ascontiguousarray(fin, np.float64)
    seeds = np.ascontiguousarray(seeds, np.int32)
    seed_vals = np.ascontiguousarray(seed_vals, np.float64)
    n = len(fin)
    ids = np.empty(n, np.int32)
    hp = np.empty(n, np.int32)
    sc = np.empty(n, np.float64)
    par = np.empty(n, np.int32)
    hop_by = np.empty(n, np.int32)
    lv = I32()
    m = lib.oracle_bfs(_p(row), _p(col), n, _p(fin), _p(seeds), _p(seed_vals), len(seeds), hops, decay,
                       _p(ids), _p(hp), _p(sc), _p(par), n, _p(hop_by), C.byref(lv))
    return dict(ids=ids[:m], hops=hp[:m], scores=sc[:m], parent=par[:m], hop_by_node=hop_by, levels=lv.value)


def bfs_scales(b, scale, decay):
    """Error scale of each visited node's BFS score, in the visit order of bfs() output b:
    a seed keeps scale[seed]; a node reached from the node at visit position p takes
    max(|decay| * scale_p, 0.8 * scale[node]), the scales of the two terms its score is the
    larger of (memory_cuda.cu:686-693). A score that is within rtol of each term's scale is
    within rtol * this scale of the oracle's, because max() is 1-Lipschitz."""
    ids, par = b["ids"], b["parent"]
    out = np.empty(len(ids), np.float64)
    for j in range(len(ids)):
        p = int(par[j])
        u = int(ids[j])
        out[j] = scale[u] if p < 0 else max(abs(decay) * out[p], 0.8 * scale[u])
    return out


def result_scales(g: "Graph", q, t_q: float, cfg: "OracleConfig", ref: dict) -> dict:
    """node id -> error scale of its result score for query() output ref (the BFS from
    ref's seeds; the per-row scale w * sum_d |e_d q_d| from scores(), times (1 + boost))."""
    _, scale = scores(g, q, t_q, cfg.time_decay_lambda, cfg.modality_filter)
    if cfg.episode_same_boost > 0:
        scale = scale * (1.0 + cfg.episode_same_boost)
    hops = 0 if ref["scoped"] else max(0, cfg.bfs_max_hops)
    b = bfs(g.row_offsets, g.col_indices, ref["final"], ref["seeds"], ref["seed_vals"], hops, cfg.bfs_score_decay)
    return dict(zip(b["ids"].tolist(), bfs_scales(b, scale, cfg.bfs_score_decay).tolist()))


def config(top_k=10, bfs_max_hops=2, time_decay_lambda=1e-8, bfs_score_decay=0.5, modality_filter=-1,
           max_results_returned=-1, retrieval_scope=0, query_episode_id=-1, query_episode_member_begin=0,
           query_episode_member_count=0, episode_same_boost=0.0) -> OracleConfig:
    return OracleConfig(top_k, bfs_max_hops, time_decay_lambda, bfs_score_decay, modality_filter, 0,
                        max_results_returned, retrieval_scope, query_episode_id, query_episode_member_begin,
                        query_episode_member_count, episode_same_boost)


def query(g: Graph, q, t_q: float, cfg: OracleConfig, max_k: int = 64, seeds_in=None, cap: int = 8192):
    """Whole query (memory_cuda.cu:1351-1464). Returns dict with results, final scores, seeds, info."""
    q = np.ascontiguousarray(q, np.float32)
    n = g.embeddings.shape[0]
    out = (OracleResult * cap)()
    fin = np.empty(n, np.float64)
    seeds = np.empty(64, np.int32)
    svals = np.empty(64, np.float64)
    info = np.zeros(4, np.int32)
    sin = None if seeds_in is None else np.ascontiguousarray(seeds_in, np.int32)
    gc = g.c()
    m = lib.oracle_query(C.byref(gc), _p(q), t_q, C.byref(cfg), max_k, out, cap, _p(fin), _p(seeds), _p(svals),
                         _p(sin), 0 if sin is None else len(sin), _p(info))
    if m < 0:
        raise ValueError("oracle_query rejected the arguments")
    nw = min(m, cap)
    res = [(out[i].node_id, out[i].score, out[i].modality, out[i].hops) for i in range(nw)]
    ns = len(sin) if sin is not None else int(min(info[0], n))
    return dict(results=res, final=fin, seeds=seeds[:ns].copy(), seed_vals=svals[:ns].copy(), k=int(info[0]),
                scoped=bool(info[1]), visited=int(info[2]), levels=int(info[3]), n_results=m)


def tiled_query(g: Graph, q, t_q: float, lam: float, k: int, tile: int, mod_filter: int = -1):
    q = np.ascontiguousarray(q, np.float32)
    ids = np.empty(k, np.int32)
    sc = np.empty(k, np.float64)
    gc = g.c()
    m = lib.oracle_tiled_query(C.byref(gc), _p(q), t_q, lam, mod_filter, k, tile, _p(ids), _p(sc))
    return ids[:m], sc[:m]


def knn(emb, qids, k: int, n: Optional[int] = None):
    """k nearest neighbours (fp64 cosine, ties: lower id) of nodes qids among rows [0, n)."""
    emb = np.ascontiguousarray(emb, np.float32)
    n = emb.shape[0] if n is None else int(n)
    qids = np.ascontiguousarray(qids, np.int32)
    ids = np.empty((len(qids), k), np.int32)
    sims = np.empty((len(qids), k), np.float64)
    lib.oracle_knn(_p(emb), n, emb.shape[1], _p(qids), len(qids), k, _p(ids), _p(sims))
    return ids, sims


def link_edges(row, col, n: int, first: int, knn_ids):
    """CSR after linking nodes first .. first + len(knn_ids) - 1 to their listed neighbours
    (both directions, union with the existing edges)."""
    row = None if row is None else np.ascontiguousarray(row, np.int32)
    col = None if col is None else np.ascontiguousarray(col, np.int32)
    kn = np.ascontiguousarray(knn_ids, np.int32)
    count, k = (kn.shape[0], kn.shape[1]) if kn.ndim == 2 else (0, 0)
    if count == 0 or k == 0:
        kn = np.full((1, 1), -1, np.int32)
    out_row = np.empty(n + 1, np.int32)
    e = lib.oracle_link_edges(n, _p(row), _p(col), first, count, _p(kn), k, _p(out_row), None)
    out_col = np.empty(max(e, 1), np.int32)
    lib.oracle_link_edges(n, _p(row), _p(col), first, count, _p(kn), k, _p(out_row), _p(out_col))
    return out_row, out_col[:e]


def insert_edges(row, col, n_old: int, n_new: int, ep_new, knn_ids):
    """CSR after a streaming insert of n_new nodes (episode pairs + given k-NN, both directions)."""
    row = None if row is None else np.ascontiguousarray(row, np.int32)
    col = None if col is None else np.ascontiguousarray(col, np.int32)
    ep = None if ep_new is None else np.ascontiguousarray(ep_new, np.int32)
    kn = np.ascontiguousarray(knn_ids, np.int32)
    k = kn.size // n_new if n_new else 0
    kn = kn.reshape(n_new, k) if k else np.full((1, 1), -1, np.int32)
    out_row = np.empty(n_old + n_new + 1, np.int32)
    e = lib.oracle_insert_edges(n_old, _p(row), _p(col), n_new, _p(ep), _p(kn), k, _p(out_row), None)
    out_col = np.empty(max(e, 1), np.int32)
    lib.oracle_insert_edges(n_old, _p(row), _p(col), n_new, _p(ep), _p(kn), k, _p(out_row), _p(out_col))
    return out_row, out_col[:e]


def importance_update(imp, ids, boost: float = 0.1, decay_rate: float = 0.001, max_imp: float = 5.0, n=None):
    """update_importance on a copy of imp (float32); nodes [0, n) decay (default all)."""
    out = np.array(imp, np.float32, copy=True)
    ids = np.ascontiguousarray(ids, np.int32)
    lib.oracle_importance_update(_p(out), len(out) if n is None else int(n), _p(ids) if len(ids) else None,
                                 len(ids), boost, decay_rate, max_imp)
    return out


def novelty(g: "Graph", q):
    """(max_i <E_i, q> floored at -1 (0 if empty), max_i sum_d |E_id q_d|)."""
    q = np.ascontiguousarray(q, np.float32)
    sc = C.c_double()
    gc = g.c()
    v = lib.oracle_novelty(C.byref(gc), _p(q), C.byref(sc))
    return v, sc.value


def edge_hits(row, col, hop_by_node, hits=None):
    """hits (+)= count_edge_hits over a CSR for the BFS levels hop_by_node (-1 unvisited)."""
    row = np.ascontiguousarray(row, np.int32)
    col = np.ascontiguousarray(col, np.int32)
    hop = np.ascontiguousarray(hop_by_node, np.int32)
    out = np.zeros(len(col), np.int32) if hits is None else np.array(hits, np.int32, copy=True)
    lib.oracle_edge_hits(_p(row), _p(col) if len(col) else None, len(row) - 1, _p(hop), _p(out) if len(out) else None)
    return out


def maintain(hits, min_hits: int = 0):
    """(edges with hits <= min_hits, the counters after the reset)."""
    h = np.array(hits, np.int32, copy=True)
    low = lib.oracle_maintain(_p(h) if len(h) else None, len(h), int(min_hits))
    return int(low), h


def kids_probes(n: int, n_image: int, count: int = 256) -> np.ndarray:
    """Indices into the IMAGE-node list of the kids sweep's probes (bench_kids_sweep.cu:624-632)."""
    out = np.empty(count, np.int64)
    lib.oracle_kids_probes(int(n), int(n_image), int(count), _p(out))
    return out
