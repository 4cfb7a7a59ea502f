"""ctypes binding of libmars_amd.so (the C ABI in include/mars_amd.h and
include/mars_corpus.h).

The library is loaded from the package directory. There is no fallback: if
the shared object is missing, importing this module raises, and every query
runs through the HIP kernels or fails.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmars_amd.so"

MARS_OK = 0
ERRORS = {
    -1: "MARS_ERR_INVALID",
    -2: "MARS_ERR_HIP",
    -3: "MARS_ERR_NOMEM",
    -4: "MARS_ERR_CAPACITY",
    -5: "MARS_ERR_UNSUPPORTED",
    -6: "MARS_ERR_NODEVICE",
}

MARS_DESC_DEVICE_POINTERS = 0x1
MARS_CTX_USE_FP16 = 0x1
MARS_CTX_USE_GRAPH = 0x2
MARS_CTX_TIMING = 0x4
MARS_CTX_CERTIFIED = 0x8


class QueryResultC(C.Structure):
    _fields_ = [("node_id", C.c_int32), ("score", C.c_float), ("modality", C.c_int32),
                ("hops_from_seed", C.c_int32)]


class RetrievalConfigC(C.Structure):
    _fields_ = [
        ("top_k", C.c_int32),
        ("bfs_max_hops", C.c_int32),
        ("time_decay_lambda", C.c_float),
        ("bfs_score_decay", C.c_float),
        ("modality_filter", C.c_int32),
        ("use_importance", C.c_int32),
        ("max_results_returned", C.c_int32),
        ("retrieval_scope", C.c_int32),
        ("query_episode_id", C.c_int32),
        ("query_episode_member_begin", C.c_int32),
        ("query_episode_member_count", C.c_int32),
        ("episode_same_boost", C.c_float),
    ]


class StatsC(C.Structure):
    _fields_ = [
        ("gpu_ms_similarity", C.c_float),
        ("gpu_ms_topk", C.c_float),
        ("gpu_ms_bfs", C.c_float),
        ("gpu_ms_rerank", C.c_float),
        ("gpu_ms_total", C.c_float),
        ("nodes_scanned", C.c_int32),
        ("bfs_waves", C.c_int32),
        ("scope_fallback", C.c_int32),
        ("visited", C.c_int32),
        ("bfs_levels_run", C.c_int32),
        ("used_fp16", C.c_int32),
        ("seeds_certified", C.c_int32),
        ("results_capped", C.c_int32),
        ("wall_us", C.c_double),
    ]


class GraphDescC(C.Structure):
    _fields_ = [
        ("num_nodes", C.c_int32),
        ("num_edges", C.c_int32),
        ("embedding_dim", C.c_int32),
        ("row_offsets", C.c_void_p),
        ("col_indices", C.c_void_p),
        ("embeddings", C.c_void_p),
        ("modalities", C.c_void_p),
        ("timestamps", C.c_void_p),
        ("capacity_nodes", C.c_int32),
        ("capacity_edges", C.c_int64),
        ("flags", C.c_uint32),
    ]


class GraphViewC(C.Structure):
    _fields_ = [
        ("num_nodes", C.c_int32),
        ("num_edges", C.c_int32),
        ("embedding_dim", C.c_int32),
        ("episode_num_episodes", C.c_int32),
        ("episode_csr_member_total", C.c_int32),
        ("has_fp16", C.c_int32),
        ("d_row_words", C.c_void_p),
        ("d_col_indices", C.c_void_p),
        ("d_embeddings", C.c_void_p),
        ("d_embeddings_fp16", C.c_void_p),
        ("d_modalities", C.c_void_p),
        ("d_timestamps", C.c_void_p),
        ("d_episode_ids", C.c_void_p),
        ("d_ep_csr_offsets", C.c_void_p),
        ("d_ep_csr_members", C.c_void_p),
    ]


class InsertStatsC(C.Structure):
    _fields_ = [
        ("first_node", C.c_int32),
        ("nodes_added", C.c_int32),
        ("edges_added", C.c_int64),
        ("rows_relocated", C.c_int32),
        ("rows_appended", C.c_int32),
        ("queryable_us", C.c_double),
        ("linked_us", C.c_double),
        ("knn_us", C.c_double),
    ]


class BatchStatsC(C.Structure):
    _fields_ = [
        ("queries", C.c_int32),
        ("batched", C.c_int32),
        ("uncertified", C.c_int32),
        ("overflow", C.c_int32),
        ("whole_batch_q1", C.c_int32),
        ("n_live", C.c_int32),
        ("gpu_ms_scan", C.c_float),
        ("gpu_ms_seeds", C.c_float),
        ("gpu_ms_bfs", C.c_float),
        ("gpu_ms_total", C.c_float),
        ("min_margin", C.c_float),
        ("candidate_rows", C.c_int32),
        ("wall_us", C.c_double),
        ("q1_us", C.c_double),
    ]


class TiledConfigC(C.Structure):
    _fields_ = [("tile_size", C.c_int32), ("top_k", C.c_int32), ("time_decay_lambda", C.c_float),
                ("modality_filter", C.c_int32), ("use_fp16", C.c_int32)]


class TiledResultC(C.Structure):
    _fields_ = [("node_id", C.c_int32), ("score", C.c_float), ("modality", C.c_int32)]


class TiledStatsC(C.Structure):
    _fields_ = [("total_nodes", C.c_int32), ("num_tiles", C.c_int32), ("total_ms", C.c_float),
                ("transfer_ms", C.c_float), ("compute_ms", C.c_float), ("merge_ms", C.c_float),
                ("h2d_gbs", C.c_double)]


class StreamBenchC(C.Structure):
    _fields_ = [("d_queries", C.c_void_p), ("stride", C.c_int64), ("n_queries", C.c_int32), ("t_q", C.c_float),
                ("cfgs", C.c_void_p), ("query_rate", C.c_double), ("ins_emb", C.c_void_p), ("ins_mods", C.c_void_p),
                ("ins_ts", C.c_void_p), ("ins_ep", C.c_void_p), ("n_insert", C.c_int32), ("insert_batch", C.c_int32),
                ("insert_rate", C.c_double), ("knn_k", C.c_int32), ("query_lat_us", C.c_void_p),
                ("query_start_us", C.c_void_p), ("ins_stats", C.c_void_p), ("ins_start_us", C.c_void_p)]


class ServeBenchC(C.Structure):
    _fields_ = [
        ("t_q", C.c_float), ("max_batch", C.c_int32),
        ("g_queries", C.c_void_p), ("n_global", C.c_int32), ("pad0", C.c_int32),
        ("g_arrival_us", C.c_void_p), ("gcfg", C.c_void_p),
        ("e_queries", C.c_void_p), ("n_episode", C.c_int32), ("pad1", C.c_int32),
        ("e_arrival_us", C.c_void_p), ("ecfgs", C.c_void_p),
        ("ins_emb", C.c_void_p), ("ins_mods", C.c_void_p), ("ins_ts", C.c_void_p), ("ins_ep", C.c_void_p),
        ("n_insert", C.c_int32), ("insert_batch", C.c_int32), ("insert_rate", C.c_double),
        ("knn_k", C.c_int32), ("pad2", C.c_int32),
        ("g_done_us", C.c_void_p), ("g_batch", C.c_void_p), ("e_done_us", C.c_void_p),
        ("ins_stats", C.c_void_p), ("ins_start_us", C.c_void_p),
        ("g_uncertified", C.c_int64), ("g_overflow", C.c_int64),
        ("link_deferred", C.c_int32), ("max_link", C.c_int32), ("ins_linked_us", C.c_void_p),
        ("link_wait_us", C.c_double), ("link_calls", C.c_int64),
    ]


class CorpusParamsC(C.Structure):
    _fields_ = [
        ("num_nodes", C.c_int64),
        ("embedding_dim", C.c_int32),
        ("episode_len", C.c_int32),
        ("seed", C.c_uint64),
        ("image_noise", C.c_float),
        ("other_centroid", C.c_float),
        ("start_max", C.c_float),
        ("slot_dt", C.c_float),
    ]


VP = C.c_void_p
I32 = C.c_int32
I64 = C.c_int64
PI32 = C.POINTER(C.c_int32)

# name -> (restype, argtypes); every exported symbol of include/*.h
SIGNATURES = {
    "mars_last_error": (C.c_char_p, []),
    "mars_abi_version": (C.c_int, []),
    "mars_init": (C.c_int, [I32]),
    "mars_config_default": (None, [C.POINTER(RetrievalConfigC)]),
    "mars_graph_create": (C.c_int, [C.POINTER(GraphDescC), C.POINTER(VP)]),
    "mars_graph_destroy": (C.c_int, [VP]),
    "mars_graph_set_episode_ids": (C.c_int, [VP, VP, I32]),
    "mars_graph_set_episode_csr": (C.c_int, [VP, I32, VP, VP, I32]),
    "mars_graph_enable_fp16": (C.c_int, [VP]),
    "mars_graph_enable_int8": (C.c_int, [VP]),
    "mars_graph_disable_int8": (C.c_int, [VP]),
    "mars_graph_read_int8": (C.c_int, [VP, I32, I32, VP, VP]),
    "mars_graph_disable_fp16": (C.c_int, [VP]),
    "mars_graph_get_view": (C.c_int, [VP, C.POINTER(GraphViewC)]),
    "mars_graph_download": (C.c_int, [VP, VP, VP, VP, VP]),
    "mars_graph_packed_csr": (C.c_int, [VP, C.POINTER(VP), C.POINTER(VP)]),
    "mars_ctx_get_stream": (C.c_int, [VP, C.POINTER(VP)]),
    "mars_ctx_create": (C.c_int, [I32, I32, I32, C.c_uint32, C.POINTER(VP)]),
    "mars_ctx_destroy": (C.c_int, [VP]),
    "mars_ctx_set_flags": (C.c_int, [VP, C.c_uint32]),
    "mars_ctx_get_flags": (C.c_int, [VP, C.POINTER(C.c_uint32)]),
    "mars_query": (C.c_int, [VP, VP, VP, C.c_float, C.POINTER(RetrievalConfigC), VP, I32, PI32,
                             C.POINTER(StatsC)]),
    "mars_query_device": (C.c_int, [VP, VP, VP, C.c_float, C.POINTER(RetrievalConfigC), VP, I32, PI32,
                                    C.POINTER(StatsC)]),
    "mars_ctx_last_scores": (C.c_int, [VP, VP, I64]),
    "mars_query_batch": (C.c_int, [VP, VP, VP, I32, VP, C.POINTER(RetrievalConfigC), VP, VP, C.POINTER(StatsC)]),
    "mars_query_batch_static": (C.c_int, [VP, VP, I32, VP, I32, C.POINTER(RetrievalConfigC), VP, VP, VP]),
    "mars_query_global_batch": (C.c_int, [VP, VP, VP, I32, VP, C.POINTER(RetrievalConfigC), VP, I32, VP,
                                          C.POINTER(BatchStatsC)]),
    "mars_bench_serve": (C.c_int, [VP, VP, VP, C.POINTER(ServeBenchC)]),
    "mars_query_global_batch_knn": (C.c_int, [VP, VP, VP, I32, VP, C.POINTER(RetrievalConfigC), VP, I32, VP,
                                              C.POINTER(BatchStatsC), I32, I32, I32, VP]),
    "mars_graph_link": (C.c_int, [VP, I32, I32, I32, VP, C.POINTER(InsertStatsC)]),
    "mars_graph_link_knn": (C.c_int, [VP, I32, I32, I32, VP, C.POINTER(InsertStatsC)]),
    "mars_graph_knn": (C.c_int, [VP, I32, VP]),
    "mars_graph_knn_blocked": (C.c_int, [VP, I32, I32, VP]),
    "mars_graph_knn_blocks": (C.c_int, [VP, I32, I32, I32, I32, VP]),
    "mars_graph_knn_range": (C.c_int, [VP, I32, I32, I32, VP]),
    "mars_graph_knn_report": (C.c_int, [VP, C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
    "mars_graph_read_ceiling": (C.c_int, [VP, I32, I32, C.POINTER(C.c_double)]),
    "mars_graph_read_pattern": (C.c_int, [VP, I32, I32, C.POINTER(C.c_double)]),
    "mars_fnv1a64": (C.c_int, [VP, I64, C.POINTER(C.c_uint64)]),
    "mars_graph_set_rows": (C.c_int, [VP, I32, I32, VP, VP, VP]),
    "mars_nsn_edges": (C.c_int, [I32, VP, I32, C.c_double, C.c_uint32, VP, VP, I64, C.POINTER(C.c_int64)]),
    "mars_importance_init": (C.c_int, [VP]),
    "mars_importance_update": (C.c_int, [VP, VP, I32, I32, C.c_float, C.c_float, C.c_float]),
    "mars_importance_read": (C.c_int, [VP, VP, I32, I32]),
    "mars_novelty": (C.c_int, [VP, VP, VP, VP, C.POINTER(C.c_float)]),
    "mars_edge_hits_init": (C.c_int, [VP]),
    "mars_edge_hits_count": (C.c_int, [VP, VP]),
    "mars_edge_hits_read": (C.c_int, [VP, VP, I64, C.POINTER(C.c_int64)]),
    "mars_graph_maintain": (C.c_int, [VP, I32, I32, C.POINTER(C.c_int32)]),
    "mars_device_memory": (C.c_int, [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]),
    "mars_graph_file_save": (C.c_int, [C.c_char_p, I32, I32, I32, VP, VP, VP, VP, VP]),
    "mars_graph_file_info": (C.c_int, [C.c_char_p, C.POINTER(I32), C.POINTER(I32), C.POINTER(I32)]),
    "mars_graph_file_load": (C.c_int, [C.c_char_p, I32, I32, I32, VP, VP, VP, VP, VP]),
    "mars_graph_save": (C.c_int, [VP, C.c_char_p]),
    "mars_kids_file_write": (C.c_int, [C.c_char_p, I32, I32, VP, VP, VP, VP]),
    "mars_kids_file_info": (C.c_int, [C.c_char_p, C.POINTER(I32), C.POINTER(I32)]),
    "mars_kids_file_read": (C.c_int, [C.c_char_p, I32, I32, VP, VP, VP, VP]),
    "mars_graph_set_csr": (C.c_int, [VP, I32, VP, VP]),
    "mars_graph_insert": (C.c_int, [VP, I32, VP, VP, VP, VP, I32, VP, C.POINTER(InsertStatsC)]),
    "mars_ctx_last_seeds": (C.c_int, [VP, VP, VP, I32, PI32]),
    "mars_ctx_last_visited": (C.c_int, [VP, VP, VP, VP, I32, PI32]),
    "mars_ctx_last_phases": (C.c_int, [VP, VP, I32]),
    "mars_device_alloc": (C.c_int, [C.c_size_t, C.POINTER(VP)]),
    "mars_device_free": (C.c_int, [VP]),
    "mars_copy_to_device": (C.c_int, [VP, VP, C.c_size_t]),
    "mars_copy_to_host": (C.c_int, [VP, VP, C.c_size_t]),
    "mars_copy_device": (C.c_int, [VP, VP, C.c_size_t]),
    "mars_device_synchronize": (C.c_int, []),
    "mars_bench_queries": (C.c_int, [VP, VP, VP, I64, I32, C.c_float, C.POINTER(RetrievalConfigC), I32, VP, VP,
                                     VP, VP]),
    "mars_bench_queries_host": (C.c_int, [VP, VP, VP, I64, I32, C.c_float, C.POINTER(RetrievalConfigC), I32, VP,
                                          VP]),
    "mars_bench_stream": (C.c_int, [VP, VP, C.POINTER(StreamBenchC)]),
    "mars_tiled_config_default": (None, [C.POINTER(TiledConfigC)]),
    "mars_tiled_ctx_create": (C.c_int, [I32, I32, I32, C.POINTER(VP)]),
    "mars_tiled_ctx_destroy": (C.c_int, [VP]),
    "mars_tiled_query": (C.c_int, [VP, VP, VP, VP, I32, I32, VP, C.c_float, C.POINTER(TiledConfigC), VP, I32, PI32,
                                   C.POINTER(TiledStatsC)]),
    "mars_host_alloc": (C.c_int, [C.c_size_t, C.POINTER(VP)]),
    "mars_host_free": (C.c_int, [VP]),
    # mars_corpus.h
    "mars_corpus_default": (None, [C.POINTER(CorpusParamsC), I64, I32, C.c_uint64]),
    "mars_corpus_generate": (C.c_int, [C.POINTER(CorpusParamsC), VP, VP, VP, VP, I32]),
    "mars_corpus_pick_queries": (C.c_int, [VP, I64, I32, I32, C.c_uint64, VP]),
    "mars_knn_cpu": (C.c_int, [VP, I64, I32, I32, VP, VP, I32]),
    "mars_build_nsn_csr": (C.c_int, [I64, VP, VP, I32, VP, VP, C.POINTER(I64), I32]),
    "mars_build_episode_csr": (C.c_int, [VP, I32, PI32, VP, VP]),
}


class MarsError(RuntimeError):
    def __init__(self, code: int, where: str, msg: str):
        super().__init__(f"{where}: {ERRORS.get(code, code)}: {msg}")
        self.code = code


def _load() -> C.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(f"{LIB_PATH} is not built; run `python mars_amd/build.py` (hipcc, gfx950)")
    lib = C.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def check(code: int, where: str) -> None:
    if code != MARS_OK:
        raise MarsError(code, where, (lib.mars_last_error() or b"").decode(errors="replace"))
