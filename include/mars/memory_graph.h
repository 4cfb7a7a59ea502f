// ============================================================================
//  mars/memory_graph.h — host graph types of the MARS query API, declared with
//  the same names and member layout as the reference's include/memory_graph.h
//  (lines 17-93) so that code written against it compiles unchanged.
//
//  Provided by libmars_amd: build_episode_csr (counting sort, identical bytes to
//  src/memory_graph.cpp:12-44) and the NSN builder build_nsn_edges /
//  build_nsn_edges_configurable (the same graph as src/memory_graph.cpp:95-189, edge
//  for edge). The corpus generators (MemoryGraph::synthetic,
//  EmbodiedKidsBallCorpus::make), print_summary and device_bytes are declared for
//  source compatibility only: they belong to the reference's host code
//  (src/memory_graph.cpp), which compiles against this header unchanged.
// ============================================================================
#ifndef MEMORY_GRAPH_H
#define MEMORY_GRAPH_H

#include <cstdint>
#include <string>
#include <vector>

enum Modality : int32_t { MOD_TEXT = 0, MOD_AUDIO = 1, MOD_IMAGE = 2, MOD_COUNT = 3 };

struct MemoryGraph {
    int32_t num_nodes = 0;
    int32_t num_edges = 0;          // CSR entries (both directions)
    int32_t embedding_dim = 0;
    std::vector<int32_t> row_offsets;   // num_nodes + 1
    std::vector<int32_t> col_indices;   // num_edges
    std::vector<float> embeddings;      // num_nodes * embedding_dim, row-major, unit rows
    std::vector<int32_t> modalities;    // num_nodes
    std::vector<float> timestamps;      // num_nodes (seconds)

    static MemoryGraph synthetic(int32_t n_text, int32_t n_audio, int32_t n_image, int32_t dim,
                                 uint32_t seed = 42);
    void build_nsn_edges(int32_t k = 6, double p = 0.15);
    struct NSNConfig {
        int32_t k = 6;
        double p = 0.15;
        bool enable_ring = true;
        bool enable_skips = true;
        bool enable_hubs = true;
        bool enable_rewire = true;
        bool enable_bridges = true;
    };
    void build_nsn_edges_configurable(const NSNConfig& cfg);
    void print_summary() const;
    size_t device_bytes() const;
};

struct HostEpisodeCSR {
    int32_t num_episodes = 0;
    std::vector<int32_t> ep_csr_offsets;   // num_episodes + 1
    std::vector<int32_t> ep_csr_members;   // node ids, ascending inside an episode
};

// Counting sort of node ids by episode id; empty CSR if sizes disagree.
HostEpisodeCSR build_episode_csr(const std::vector<int32_t>& episode_ids, int32_t num_nodes);

enum class RetrievalScope : int32_t { Global = 0, EpisodeScoped = 1 };

struct EmbodiedKidsBallCorpus {
    MemoryGraph graph;
    std::vector<int32_t> episode_ids;
    static EmbodiedKidsBallCorpus make(int32_t n_nodes, int32_t dim, uint32_t seed = 42);
};

#endif  // MEMORY_GRAPH_H
