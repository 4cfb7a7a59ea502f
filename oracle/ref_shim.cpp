// ============================================================================
//  oracle/ref_shim.cpp — extern "C" wrappers over the reference's own host
//  code, compiled together with the reference sources (src/memory_graph.cpp,
//  src/streaming.cpp, src/persistence.cpp) where they lie, into
//  oracle/_ref/libref.so.
//
//  TEST INFRASTRUCTURE: used to pin the oracle and the product's host code
//  against the reference's behaviour (episode CSR, kids corpus, NSN builder,
//  streaming flush). Never loaded by the product.
// ============================================================================
#include "memory_graph.h"
#include "persistence.h"
#include "streaming.h"

#include <cstring>
#include <vector>

namespace {
struct RefGraph {
    MemoryGraph g;
    std::vector<int32_t> episode_ids;
};
}  // namespace

extern "C" {

// build_episode_csr (memory_graph.cpp:12-44). Two calls: members==nullptr to
// size, then with buffers (offsets: num_episodes+1, members: N).
int ref_build_episode_csr(const int32_t* ids, int32_t n, int32_t* num_episodes,
                          int32_t* offsets, int32_t* members) {
    std::vector<int32_t> v(ids, ids + (n > 0 ? n : 0));
    HostEpisodeCSR csr = build_episode_csr(v, n);
    *num_episodes = csr.num_episodes;
    if (offsets) std::memcpy(offsets, csr.ep_csr_offsets.data(), csr.ep_csr_offsets.size() * 4);
    if (members) std::memcpy(members, csr.ep_csr_members.data(), csr.ep_csr_members.size() * 4);
    return int(csr.ep_csr_members.size());
}

// EmbodiedKidsBallCorpus::make (memory_graph.cpp:241-295), optionally followed by
// MemoryGraph::build_nsn_edges(k, p) (memory_graph.cpp:95-189).
void* ref_kids_make(int32_t n, int32_t dim, uint32_t seed, int32_t nsn_k, double nsn_p) {
    auto* r = new RefGraph();
    EmbodiedKidsBallCorpus c = EmbodiedKidsBallCorpus::make(n, dim, seed);
    r->g = std::move(c.graph);
    r->episode_ids = std::move(c.episode_ids);
    if (nsn_k > 0) r->g.build_nsn_edges(nsn_k, nsn_p);
    return r;
}

// MemoryGraph::synthetic (memory_graph.cpp:46-92) + build_nsn_edges.
void* ref_synthetic_make(int32_t n_text, int32_t n_audio, int32_t n_image, int32_t dim,
                         uint32_t seed, int32_t nsn_k, double nsn_p) {
    auto* r = new RefGraph();
    r->g = MemoryGraph::synthetic(n_text, n_audio, n_image, dim, seed);
    if (nsn_k > 0) r->g.build_nsn_edges(nsn_k, nsn_p);
    return r;
}

// MemoryGraph::build_nsn_edges_configurable (memory_graph.cpp:102-189) over n nodes of
// the given modalities; phases: ring 1, skips 2, hubs 4, rewire 8, bridges 16.
// Returns the edge count; row (n + 1) and col (when large enough) receive the CSR.
int64_t ref_nsn_edges(int32_t n, const int32_t* mods, int32_t k, double p, uint32_t phases, int32_t* row,
                      int32_t* col, int64_t col_cap) {
    MemoryGraph g;
    g.num_nodes = n;
    g.modalities.assign(mods, mods + n);
    MemoryGraph::NSNConfig cfg;
    cfg.k = k;
    cfg.p = p;
    cfg.enable_ring = phases & 1u;
    cfg.enable_skips = phases & 2u;
    cfg.enable_hubs = phases & 4u;
    cfg.enable_rewire = phases & 8u;
    cfg.enable_bridges = phases & 16u;
    g.build_nsn_edges_configurable(cfg);
    const int64_t e = int64_t(g.col_indices.size());
    if (row) std::memcpy(row, g.row_offsets.data(), g.row_offsets.size() * 4);
    if (col && e <= col_cap && e > 0) std::memcpy(col, g.col_indices.data(), size_t(e) * 4);
    return e;
}

void ref_graph_sizes(void* h, int32_t* n, int32_t* dim, int32_t* num_edges) {
    auto* r = static_cast<RefGraph*>(h);
    *n = r->g.num_nodes; *dim = r->g.embedding_dim; *num_edges = int32_t(r->g.col_indices.size());
}

void ref_graph_copy(void* h, float* emb, int32_t* mods, float* ts, int32_t* ep_ids,
                    int32_t* row_offsets, int32_t* col) {
    auto* r = static_cast<RefGraph*>(h);
    if (emb) std::memcpy(emb, r->g.embeddings.data(), r->g.embeddings.size() * 4);
    if (mods) std::memcpy(mods, r->g.modalities.data(), r->g.modalities.size() * 4);
    if (ts) std::memcpy(ts, r->g.timestamps.data(), r->g.timestamps.size() * 4);
    if (ep_ids && !r->episode_ids.empty())
        std::memcpy(ep_ids, r->episode_ids.data(), r->episode_ids.size() * 4);
    if (row_offsets && !r->g.row_offsets.empty())
        std::memcpy(row_offsets, r->g.row_offsets.data(), r->g.row_offsets.size() * 4);
    if (col && !r->g.col_indices.empty())
        std::memcpy(col, r->g.col_indices.data(), r->g.col_indices.size() * 4);
}

// StreamingBuffer::insert + flush (streaming.cpp:13-80, 97-163): append n_new
// nodes to the graph, returns the number of nodes accepted.
int32_t ref_stream_flush(void* h, int32_t capacity, int32_t nsn_k, int32_t n_new,
                         const int32_t* mods, const float* ts, const float* emb) {
    auto* r = static_cast<RefGraph*>(h);
    StreamingConfig cfg;
    cfg.capacity = capacity;
    cfg.embedding_dim = r->g.embedding_dim;
    cfg.nsn_k = nsn_k;
    cfg.auto_flush = false;
    StreamingBuffer buf(cfg);
    int32_t ok = 0;
    for (int32_t i = 0; i < n_new; ++i)
        ok += buf.insert(r->g.num_nodes + i, mods[i], ts[i],
                         emb + size_t(i) * size_t(r->g.embedding_dim)) ? 1 : 0;
    buf.flush(r->g);
    return ok;
}

void ref_graph_free(void* h) { delete static_cast<RefGraph*>(h); }

// fnv1a_checksum (persistence.cpp:23-31).
uint64_t ref_fnv1a(const void* data, size_t len) { return fnv1a_checksum(data, len); }

// save_graph (persistence.cpp:43-108) of a graph given as arrays; 1 on success.
int ref_save_graph(const char* path, int32_t n, int32_t e, int32_t d, const int32_t* row_offsets,
                   const int32_t* col, const float* emb, const int32_t* mods, const float* ts) {
    MemoryGraph g;
    g.num_nodes = n;
    g.num_edges = e;
    g.embedding_dim = d;
    g.row_offsets.assign(row_offsets, row_offsets + n + 1);
    g.col_indices.assign(col, col + e);
    g.embeddings.assign(emb, emb + size_t(n) * size_t(d));
    g.modalities.assign(mods, mods + n);
    g.timestamps.assign(ts, ts + n);
    return save_graph(g, path) ? 1 : 0;
}

// load_graph (persistence.cpp:110-215); 1 on success. Sizes are always returned;
// arrays are copied where the pointer is not null.
int ref_load_graph(const char* path, int32_t* n, int32_t* e, int32_t* d, int32_t* row_offsets, int32_t* col,
                   float* emb, int32_t* mods, float* ts) {
    MemoryGraph g;
    if (!load_graph(g, path)) return 0;
    *n = g.num_nodes; *e = g.num_edges; *d = g.embedding_dim;
    if (row_offsets) std::memcpy(row_offsets, g.row_offsets.data(), g.row_offsets.size() * 4);
    if (col && !g.col_indices.empty()) std::memcpy(col, g.col_indices.data(), g.col_indices.size() * 4);
    if (emb && !g.embeddings.empty()) std::memcpy(emb, g.embeddings.data(), g.embeddings.size() * 4);
    if (mods && !g.modalities.empty()) std::memcpy(mods, g.modalities.data(), g.modalities.size() * 4);
    if (ts && !g.timestamps.empty()) std::memcpy(ts, g.timestamps.data(), g.timestamps.size() * 4);
    return 1;
}

}  // extern "C"
