// ============================================================================
//  shim.cpp — the reference's C++ query API (include/mars/memory_cuda.cuh,
//  include/mars/memory_graph.h) over the C ABI of libmars_amd.
//
//  Error behaviour mirrors the reference: a failing library call prints the
//  library's message and exits (CUDA_CHECK, memory_cuda.cuh:52-60); malformed
//  episode inputs are silent no-ops (memory_cuda.cu:814-855).
// ============================================================================
#include "mars/memory_cuda.cuh"
#include "mars/memory_graph.h"
#include "mars/streaming.h"
#include "mars/tiled_query.h"
#include "mars_amd.h"
#include "mars_corpus.h"

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>

namespace {

void die_on(int rc, const char* what) {
    if (rc == MARS_OK) return;
    std::fprintf(stderr, "libmars_amd error in %s (%d): %s\n", what, rc, mars_last_error());
    std::exit(EXIT_FAILURE);
}

// packed: also point d_row_offsets / d_col_indices at the reference's packed CSR (a copy
// the library makes again only when the edges changed since the last one); otherwise they
// are cleared, and refresh_packed_csr() makes them on demand. The queries never read
// them: they read the row words and their column slots.
void refresh_view(DeviceMemoryGraph& d, bool packed = true) {
    mars_graph_view v{};
    die_on(mars_graph_get_view(d.handle, &v), "mars_graph_get_view");
    d.num_nodes = v.num_nodes;
    d.num_edges = v.num_edges;
    d.embedding_dim = v.embedding_dim;
    const int32_t* prow = nullptr;
    const int32_t* pcol = nullptr;
    if (packed) die_on(mars_graph_packed_csr(d.handle, &prow, &pcol), "mars_graph_packed_csr");
    d.d_row_offsets = const_cast<int32_t*>(prow);
    d.d_col_indices = const_cast<int32_t*>(pcol);
    d.d_row_words = static_cast<int64_t*>(v.d_row_words);
    d.d_col_slots = static_cast<int32_t*>(v.d_col_indices);
    d.d_embeddings = static_cast<float*>(v.d_embeddings);
    d.d_embeddings_fp16 = v.d_embeddings_fp16;
    d.d_modalities = static_cast<int32_t*>(v.d_modalities);
    d.d_timestamps = static_cast<float*>(v.d_timestamps);
    d.d_episode_ids = static_cast<int32_t*>(v.d_episode_ids);
    d.d_ep_csr_offsets = static_cast<int32_t*>(v.d_ep_csr_offsets);
    d.d_ep_csr_members = static_cast<int32_t*>(v.d_ep_csr_members);
    d.episode_num_episodes = v.episode_num_episodes;
    d.episode_csr_member_total = v.episode_csr_member_total;
}

mars_retrieval_config to_c(const RetrievalConfig& c) {
    mars_retrieval_config r;
    r.top_k = c.top_k;
    r.bfs_max_hops = c.bfs_max_hops;
    r.time_decay_lambda = c.time_decay_lambda;
    r.bfs_score_decay = c.bfs_score_decay;
    r.modality_filter = c.modality_filter;
    r.use_importance = c.use_importance ? 1 : 0;
    r.max_results_returned = c.max_results_returned;
    r.retrieval_scope = static_cast<int32_t>(c.retrieval_scope);
    r.query_episode_id = c.query_episode_id;
    r.query_episode_member_begin = c.query_episode_member_begin;
    r.query_episode_member_count = c.query_episode_member_count;
    r.episode_same_boost = c.episode_same_boost;
    return r;
}

}  // namespace

HostEpisodeCSR build_episode_csr(const std::vector<int32_t>& episode_ids, int32_t num_nodes) {
    HostEpisodeCSR out;
    if (num_nodes <= 0 || int32_t(episode_ids.size()) != num_nodes) return out;      // memory_graph.cpp:15-16
    int32_t ne = 0;
    if (mars_build_episode_csr(episode_ids.data(), num_nodes, &ne, nullptr, nullptr) != MARS_OK) return out;
    out.num_episodes = ne;
    out.ep_csr_offsets.resize(size_t(ne) + 1);
    out.ep_csr_members.resize(size_t(num_nodes));
    mars_build_episode_csr(episode_ids.data(), num_nodes, &ne, out.ep_csr_offsets.data(), out.ep_csr_members.data());
    return out;
}

DeviceMemoryGraph upload_to_device(const MemoryGraph& h) { return upload_to_device(h, 0); }

DeviceMemoryGraph upload_to_device(const MemoryGraph& h, int32_t capacity_nodes) {
    mars_graph_desc desc{};
    desc.capacity_nodes = capacity_nodes;
    desc.num_nodes = h.num_nodes;
    desc.num_edges = int32_t(h.col_indices.size());
    desc.embedding_dim = h.embedding_dim;
    desc.row_offsets = h.row_offsets.empty() ? nullptr : h.row_offsets.data();
    desc.col_indices = h.col_indices.empty() ? nullptr : h.col_indices.data();
    desc.embeddings = h.embeddings.data();
    desc.modalities = h.modalities.data();
    desc.timestamps = h.timestamps.data();
    DeviceMemoryGraph d;
    die_on(mars_graph_create(&desc, &d.handle), "upload_to_device");
    refresh_view(d);
    return d;
}

void MemoryGraph::build_nsn_edges(int32_t k, double p) {
    NSNConfig cfg;
    cfg.k = k;
    cfg.p = p;
    build_nsn_edges_configurable(cfg);
}

void MemoryGraph::build_nsn_edges_configurable(const NSNConfig& cfg) {
    const uint32_t phases = (cfg.enable_ring ? MARS_NSN_RING : 0u) | (cfg.enable_skips ? MARS_NSN_SKIPS : 0u) |
                            (cfg.enable_hubs ? MARS_NSN_HUBS : 0u) | (cfg.enable_rewire ? MARS_NSN_REWIRE : 0u) |
                            (cfg.enable_bridges ? MARS_NSN_BRIDGES : 0u);
    int64_t bound = 0, ne = 0;
    die_on(mars_nsn_edges(num_nodes, modalities.data(), cfg.k, cfg.p, phases, nullptr, nullptr, 0, &bound),
           "build_nsn_edges");
    row_offsets.assign(size_t(num_nodes) + 1, 0);
    col_indices.resize(size_t(std::max<int64_t>(bound, 1)));
    die_on(mars_nsn_edges(num_nodes, modalities.data(), cfg.k, cfg.p, phases, row_offsets.data(),
                          col_indices.data(), int64_t(col_indices.size()), &ne), "build_nsn_edges");
    col_indices.resize(size_t(ne));
    num_edges = int32_t(ne);
}

void init_importance(DeviceMemoryGraph& dg) { die_on(mars_importance_init(dg.handle), "init_importance"); }

void update_importance(DeviceMemoryGraph& dg, const int32_t* d_result_ids, int32_t n_results, float boost,
                       float decay_rate, float max_importance, void* /*stream*/) {
    const int rc = mars_importance_update(dg.handle, d_result_ids, n_results > 0 ? n_results : 0, 1, boost,
                                          decay_rate, max_importance);
    if (rc == MARS_ERR_UNSUPPORTED) return;          // memory_cuda.cu:1510: no importance array, no-op
    die_on(rc, "update_importance");
}

float compute_novelty(const DeviceMemoryGraph& dg, const float* d_query, void* /*stream*/) {
    float v = 0.0f;
    die_on(mars_novelty(dg.handle, nullptr, nullptr, d_query, &v), "compute_novelty");
    return v;
}

void init_edge_hits(DeviceMemoryGraph& dg) { die_on(mars_edge_hits_init(dg.handle), "init_edge_hits"); }

int32_t maintain_graph(DeviceMemoryGraph& dg, int32_t min_hits, int32_t window_queries, void* /*stream*/) {
    int32_t low = 0;
    die_on(mars_graph_maintain(dg.handle, min_hits, window_queries, &low), "maintain_graph");
    return low;
}

void count_edge_hits(DeviceMemoryGraph& dg, QueryContext& ctx) {
    die_on(mars_edge_hits_count(dg.handle, ctx.handle), "count_edge_hits");
}

void refresh_packed_csr(DeviceMemoryGraph& dg) {
    if (dg.handle) refresh_view(dg, true);
}

void free_device(DeviceMemoryGraph& d) {
    if (d.handle) mars_graph_destroy(d.handle);
    d = DeviceMemoryGraph{};
}

void upload_episode_ids(DeviceMemoryGraph& dg, const int32_t* ids, int32_t n) {
    if (!dg.handle) return;
    (void)mars_graph_set_episode_ids(dg.handle, ids, n);          // bad input: cleared, no error
    refresh_view(dg);
}

void upload_episode_csr(DeviceMemoryGraph& dg, const HostEpisodeCSR& csr) {
    if (!dg.handle) return;
    const bool shaped = csr.num_episodes > 0 && int32_t(csr.ep_csr_offsets.size()) == csr.num_episodes + 1 &&
                        int32_t(csr.ep_csr_members.size()) == csr.ep_csr_offsets.back();
    if (shaped)
        (void)mars_graph_set_episode_csr(dg.handle, csr.num_episodes, csr.ep_csr_offsets.data(),
                                         csr.ep_csr_members.data(), int32_t(csr.ep_csr_members.size()));
    else
        (void)mars_graph_set_episode_csr(dg.handle, 0, nullptr, nullptr, 0);   // cleared, as the reference
    refresh_view(dg);
}

void upload_fp16_embeddings(DeviceMemoryGraph& dg) {
    if (!dg.handle) return;
    die_on(mars_graph_enable_fp16(dg.handle), "upload_fp16_embeddings");
    refresh_view(dg);
}

void free_fp16_embeddings(DeviceMemoryGraph& dg) {
    if (!dg.handle) return;
    die_on(mars_graph_disable_fp16(dg.handle), "free_fp16_embeddings");
    refresh_view(dg);
}

QueryContext create_query_context(int32_t max_nodes, int32_t embedding_dim, int32_t max_k) {
    QueryContext ctx;
    die_on(mars_ctx_create(max_nodes, embedding_dim, max_k, MARS_CTX_TIMING, &ctx.handle), "create_query_context");
    ctx.max_nodes = max_nodes;
    ctx.embedding_dim = embedding_dim;
    ctx.max_k = std::min(max_k, 64);
    die_on(mars_ctx_get_stream(ctx.handle, &ctx.stream), "create_query_context");
    ctx.valid = true;
    return ctx;
}

void destroy_query_context(QueryContext& ctx) {
    if (!ctx.valid) return;
    mars_ctx_destroy(ctx.handle);
    ctx = QueryContext{};
}

std::vector<QueryResult> query_memory_fast(const DeviceMemoryGraph& dg, QueryContext& ctx, const float* h_query,
                                           float query_timestamp, const RetrievalConfig& cfg, RetrievalStats& stats) {
    uint32_t flags = MARS_CTX_TIMING;                         // stats are always filled, as the reference
    if (ctx.use_fp16) flags |= MARS_CTX_USE_FP16;
    if (ctx.use_cuda_graph) flags |= MARS_CTX_USE_GRAPH;
    die_on(mars_ctx_set_flags(ctx.handle, flags), "query_memory_fast");
    const mars_retrieval_config c = to_c(cfg);
    std::vector<mars_query_result> buf(size_t(std::max(1, cfg.max_results_returned > 0 ? cfg.max_results_returned
                                                                                      : std::min(cfg.top_k, 64))));
    int32_t n = 0;
    mars_stats st{};
    die_on(mars_query(dg.handle, ctx.handle, h_query, query_timestamp, &c, buf.data(), int32_t(buf.size()), &n, &st),
           "query_memory_fast");
    std::vector<QueryResult> out;
    out.reserve(size_t(n));
    for (int32_t i = 0; i < std::min<int32_t>(n, int32_t(buf.size())); ++i)
        out.push_back({buf[size_t(i)].node_id, buf[size_t(i)].score, buf[size_t(i)].modality,
                       buf[size_t(i)].hops_from_seed});
    stats.gpu_ms_similarity = st.gpu_ms_similarity;
    stats.gpu_ms_topk = st.gpu_ms_topk;
    stats.gpu_ms_bfs = st.gpu_ms_bfs;
    stats.gpu_ms_rerank = st.gpu_ms_rerank;
    stats.gpu_ms_total = st.gpu_ms_total;
    stats.nodes_scanned = st.nodes_scanned;
    stats.bfs_waves = st.bfs_waves;
    return out;
}

std::vector<QueryResult> query_memory(const DeviceMemoryGraph& dg, const float* h_query, float query_timestamp,
                                      const RetrievalConfig& cfg, RetrievalStats& stats) {
    // the reference allocates per call (memory_cuda.cu:881-1026); so does this one
    QueryContext ctx = create_query_context(dg.num_nodes, dg.embedding_dim, 64);
    std::vector<QueryResult> r = query_memory_fast(dg, ctx, h_query, query_timestamp, cfg, stats);
    destroy_query_context(ctx);
    return r;
}

// ---- tiled out-of-core query (include/tiled_query.h:79-102) --------------------------

TiledQueryContext create_tiled_context(int32_t max_tile_size, int32_t embedding_dim, int32_t max_k) {
    TiledQueryContext ctx;
    die_on(mars_tiled_ctx_create(max_tile_size, embedding_dim, max_k, &ctx.handle), "create_tiled_context");
    ctx.max_tile_size = max_tile_size;
    ctx.embedding_dim = embedding_dim;
    ctx.max_k = std::min(max_k, 64);
    ctx.valid = true;
    return ctx;
}

void destroy_tiled_context(TiledQueryContext& ctx) {
    if (!ctx.valid) return;
    mars_tiled_ctx_destroy(ctx.handle);
    ctx = TiledQueryContext{};
}

std::vector<TiledQueryResult> tiled_query(TiledQueryContext& ctx, const float* h_embeddings,
                                          const int32_t* h_modalities, const float* h_timestamps, int32_t N,
                                          int32_t D, const float* h_query, float query_timestamp,
                                          const TiledQueryConfig& cfg, TiledQueryStats& stats) {
    mars_tiled_config c;
    c.tile_size = cfg.tile_size;
    c.top_k = cfg.top_k;
    c.time_decay_lambda = cfg.time_decay_lambda;
    c.modality_filter = cfg.modality_filter;
    c.use_fp16 = cfg.use_fp16 ? 1 : 0;
    std::vector<mars_tiled_result> buf(static_cast<size_t>(std::max(1, cfg.top_k)));
    int32_t n = 0;
    mars_tiled_stats st{};
    die_on(mars_tiled_query(ctx.handle, h_embeddings, h_modalities, h_timestamps, N, D, h_query, query_timestamp, &c,
                            buf.data(), int32_t(buf.size()), &n, &st),
           "tiled_query");
    std::vector<TiledQueryResult> out;
    for (int32_t i = 0; i < std::min<int32_t>(n, int32_t(buf.size())); ++i)
        out.push_back({buf[size_t(i)].node_id, buf[size_t(i)].score, buf[size_t(i)].modality});
    stats.total_nodes = st.total_nodes;
    stats.num_tiles = st.num_tiles;
    stats.total_ms = st.total_ms;
    stats.transfer_ms = st.transfer_ms;
    stats.compute_ms = st.compute_ms;
    stats.merge_ms = st.merge_ms;
    return out;
}

// ---- streaming insert buffer (include/streaming.h:42-81) ------------------------------

StreamingBuffer::StreamingBuffer(const StreamingConfig& cfg) : cfg_(cfg) {
    buffer_.reserve(size_t(std::max(cfg.capacity, 0)));
}

bool StreamingBuffer::insert(int32_t id, int32_t modality, float timestamp, const float* embedding,
                             int32_t episode_id) {
    std::lock_guard<std::mutex> lock(mu_);
    if (int32_t(buffer_.size()) >= cfg_.capacity) return false;      // streaming.cpp:15-21
    StagedNode n;
    n.id = id;
    n.modality = modality;
    n.timestamp = timestamp;
    n.embedding.assign(embedding, embedding + cfg_.embedding_dim);
    n.episode_id = episode_id;
    buffer_.push_back(std::move(n));
    return true;
}

bool StreamingBuffer::insert(const StagedNode& node) {
    return insert(node.id, node.modality, node.timestamp, node.embedding.data(), node.episode_id);
}

FlushStats StreamingBuffer::flush(DeviceMemoryGraph& target) {
    std::lock_guard<std::mutex> lock(mu_);
    FlushStats stats;
    if (buffer_.empty() || !target.handle) return stats;
    const int32_t n = int32_t(buffer_.size());
    const int32_t d = cfg_.embedding_dim;
    if (d != target.embedding_dim) {
        std::fprintf(stderr, "StreamingBuffer::flush: embedding_dim %d, graph has %d\n", d, target.embedding_dim);
        std::exit(EXIT_FAILURE);
    }
    std::vector<float> rows(size_t(n) * size_t(d));
    std::vector<int32_t> mods(static_cast<size_t>(n)), eps(static_cast<size_t>(n));
    std::vector<float> ts(static_cast<size_t>(n));
    bool with_eps = target.d_episode_ids != nullptr;
    for (int32_t i = 0; i < n; ++i) {
        const StagedNode& s = buffer_[size_t(i)];
        if (s.id != target.num_nodes + i) {
            std::fprintf(stderr, "StreamingBuffer::flush: staged id %d, the graph's next id is %d\n", s.id,
                         target.num_nodes + i);
            std::exit(EXIT_FAILURE);
        }
        std::copy(s.embedding.begin(), s.embedding.end(), rows.begin() + int64_t(i) * d);
        mods[size_t(i)] = s.modality;
        ts[size_t(i)] = s.timestamp;
        eps[size_t(i)] = s.episode_id;
    }
    mars_insert_stats st{};
    die_on(mars_graph_insert(target.handle, n, rows.data(), mods.data(), ts.data(), with_eps ? eps.data() : nullptr,
                             cfg_.nsn_k, nullptr, &st),
           "StreamingBuffer::flush");
    // the packed CSR copy is not rebuilt per flush (an O(N + E) pass): refresh_packed_csr()
    refresh_view(target, false);
    stats.nodes_committed = st.nodes_added;
    stats.edges_added = int32_t(std::min<int64_t>(st.edges_added, INT32_MAX));
    stats.flush_ms = float(st.linked_us / 1000.0);
    stats.queryable_ms = float(st.queryable_us / 1000.0);
    total_flushed_ += n;
    buffer_.clear();
    return stats;
}

int32_t StreamingBuffer::staged_count() const {
    std::lock_guard<std::mutex> lock(mu_);
    return int32_t(buffer_.size());
}

int64_t StreamingBuffer::total_flushed() const {
    std::lock_guard<std::mutex> lock(mu_);
    return total_flushed_;
}

void StreamingBuffer::reset() {
    std::lock_guard<std::mutex> lock(mu_);
    buffer_.clear();
}
