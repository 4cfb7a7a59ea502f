// ============================================================================
//  mars/memory_cuda.cuh — the reference's query API (include/memory_cuda.cuh of
//  MARS, lines 63-231) served by libmars_amd on MI355X. Plain C++17: no CUDA or
//  HIP header is included; code that includes "memory_cuda.cuh" and calls
//  upload_to_device / create_query_context / query_memory_fast compiles against
//  this header and links against libmars_amd.so.
//
//  Same names, members and semantics as the reference, with these differences:
//    * device pointers are opaque (void* / typed where HIP-free); `handle` carries
//      the library objects;
//    * QueryContext::use_cublas / use_cub_topk / use_wmma are accepted and have no
//      effect (scoring and selection always run the fused HIP kernels);
//    * results are sorted by (score desc, node_id asc) and the BFS is the
//      deterministic first-discoverer BFS (no frontier cap); a query returns at most
//      min(max_nodes, max_k * 500) results, the reference's compaction cap, keeping
//      the best of them;
//    * RetrievalStats: gpu_ms_similarity is the fused scan (dot, decay, per-wave
//      top-K), gpu_ms_rerank is 0 (the decay is inside the scan), gpu_ms_topk the
//      seed merge, gpu_ms_bfs the BFS and the sorted results;
//    * DeviceMemoryGraph: d_row_offsets / d_col_indices are a packed copy of the
//      edges (set by upload_to_device and the upload_* calls, made again only when
//      the edges changed); a streaming flush clears them instead of repacking all
//      edges, and refresh_packed_csr() makes them again on demand. The queries read
//      d_row_words and d_col_slots, where a row that grew by an insert can sit apart;
//    * library errors print a message and exit, as CUDA_CHECK does (lines 52-60);
//      malformed episode inputs are silent no-ops and an inactive episode scope
//      falls back to Global, as in the reference (memory_cuda.cu:814-855, 1163-1171).
//  The importance / novelty / graph-maintenance entry points (lines 234-272) are
//  served too. They run synchronously; the stream argument is accepted and unused.
//  d_importance / d_edge_hits stay null (the arrays live in the library's graph).
// ============================================================================
#ifndef MEMORY_CUDA_CUH
#define MEMORY_CUDA_CUH

#include <cstdint>
#include <vector>

#include "memory_graph.h"

struct mars_graph;
struct mars_ctx;

struct DeviceMemoryGraph {
    int32_t num_nodes = 0;
    int32_t num_edges = 0;
    int32_t embedding_dim = 0;
    int32_t* d_row_offsets = nullptr;      // packed CSR [num_nodes + 1]: a copy (see d_row_words)
    int32_t* d_col_indices = nullptr;      // packed CSR [num_edges]
    float* d_embeddings = nullptr;
    void* d_embeddings_fp16 = nullptr;     // binary16 rows
    int32_t* d_modalities = nullptr;
    float* d_timestamps = nullptr;
    int32_t* d_episode_ids = nullptr;
    int32_t* d_ep_csr_offsets = nullptr;
    int32_t* d_ep_csr_members = nullptr;
    int32_t episode_num_episodes = 0;
    int32_t episode_csr_member_total = 0;
    float* d_importance = nullptr;         // null: the library's graph holds the array
    int32_t* d_edge_hits = nullptr;        // null: the library's graph holds the array
    int64_t* d_row_words = nullptr;        // per node: (row length << 32) | row start in d_col_slots
    int32_t* d_col_slots = nullptr;        // the column slots the queries read (rows may have slack)
    mars_graph* handle = nullptr;
};

DeviceMemoryGraph upload_to_device(const MemoryGraph& h);
// Extension: reserve room for capacity_nodes nodes (streaming inserts, mars/streaming.h).
DeviceMemoryGraph upload_to_device(const MemoryGraph& h, int32_t capacity_nodes);
void free_device(DeviceMemoryGraph& d);
void upload_episode_ids(DeviceMemoryGraph& dg, const int32_t* host_episode_ids, int32_t num_ids);
void upload_episode_csr(DeviceMemoryGraph& dg, const HostEpisodeCSR& csr);
void upload_fp16_embeddings(DeviceMemoryGraph& dg);
void free_fp16_embeddings(DeviceMemoryGraph& dg);
// Extension: point d_row_offsets / d_col_indices at a packed copy of the current edges
// (after a streaming flush cleared them).
void refresh_packed_csr(DeviceMemoryGraph& dg);

struct QueryResult {
    int32_t node_id;
    float score;
    int32_t modality;
    int32_t hops_from_seed;
};

struct RetrievalConfig {
    int32_t top_k = 10;
    int32_t bfs_max_hops = 2;
    float time_decay_lambda = 1e-8f;
    float bfs_score_decay = 0.5f;
    int32_t modality_filter = -1;
    bool use_importance = false;
    int32_t max_results_returned = -1;
    RetrievalScope retrieval_scope = RetrievalScope::Global;
    int32_t query_episode_id = -1;
    int32_t query_episode_member_begin = 0;
    int32_t query_episode_member_count = 0;
    float episode_same_boost = 0.0f;
};

struct RetrievalStats {
    float gpu_ms_similarity = 0.0f;
    float gpu_ms_topk = 0.0f;
    float gpu_ms_bfs = 0.0f;
    float gpu_ms_rerank = 0.0f;
    float gpu_ms_total = 0.0f;
    int32_t nodes_scanned = 0;
    int32_t bfs_waves = 0;
};

std::vector<QueryResult> query_memory(const DeviceMemoryGraph& dg, const float* h_query, float query_timestamp,
                                      const RetrievalConfig& cfg, RetrievalStats& stats);

struct QueryContext {
    int32_t max_nodes = 0;
    int32_t embedding_dim = 0;
    int32_t max_k = 0;
    bool valid = false;
    bool use_cuda_graph = false;
    bool use_fp16 = false;
    bool use_cublas = true;       // accepted, no effect
    bool use_cub_topk = true;     // accepted, no effect
    bool use_wmma = false;        // accepted, no effect
    void* stream = nullptr;       // the context's hipStream_t (line 178): its queries run on it
    mars_ctx* handle = nullptr;
};

QueryContext create_query_context(int32_t max_nodes, int32_t embedding_dim, int32_t max_k = 64);
void destroy_query_context(QueryContext& ctx);

std::vector<QueryResult> query_memory_fast(const DeviceMemoryGraph& dg, QueryContext& ctx, const float* h_query,
                                           float query_timestamp, const RetrievalConfig& cfg, RetrievalStats& stats);

// ---- importance, novelty gate, adaptive graph maintenance (lines 234-270) ----------
void init_importance(DeviceMemoryGraph& dg);
// d_result_ids: device memory (mars_device_alloc), as the reference.
void update_importance(DeviceMemoryGraph& dg, const int32_t* d_result_ids, int32_t n_results, float boost = 0.1f,
                       float decay_rate = 0.001f, float max_importance = 5.0f, void* stream = nullptr);
// d_query: device memory. Max over the nodes of <E_i, q>, at least -1.
float compute_novelty(const DeviceMemoryGraph& dg, const float* d_query, void* stream = nullptr);
void init_edge_hits(DeviceMemoryGraph& dg);
int32_t maintain_graph(DeviceMemoryGraph& dg, int32_t min_hits = 0, int32_t window_queries = 1000,
                       void* stream = nullptr);
// Extension (the reference has count_edge_hits_kernel, memory_cuda.cu:1612-1632, and no
// host call for it): count the edges the BFS of ctx's last global query walked.
void count_edge_hits(DeviceMemoryGraph& dg, QueryContext& ctx);

#endif  // MEMORY_CUDA_CUH
