// ============================================================================
//  mars/streaming.h — the reference's streaming insert buffer
//  (include/streaming.h:21-81 of MARS) over libmars_amd's device-side insert.
//  Plain C++17, no CUDA or HIP header.
//
//  Same staging interface: insert() stages nodes (mutex-guarded, bounded by
//  capacity), staged_count() / total_flushed() / capacity() / reset(). The
//  commit differs on purpose: the reference's flush(MemoryGraph&) appends to the
//  host graph and rebuilds its CSR (streaming.cpp:35-163) before the caller
//  re-uploads; flush(DeviceMemoryGraph&, ...) here appends the staged nodes to the
//  device-resident graph on its side stream (mars_graph_insert): rows become
//  visible to scans first, then their NSN edges (intra-episode pairs + knn_k
//  nearest neighbours, both directions) — queries on other threads keep running.
//  Staged node ids must continue the graph's ids (dg.num_nodes, +1, ...), as in
//  the reference's tests; auto_flush cannot flush without a graph, as there.
// ============================================================================
#ifndef STREAMING_H
#define STREAMING_H

#include <cstdint>
#include <mutex>
#include <vector>

#include "memory_cuda.cuh"
#include "memory_graph.h"

struct StagedNode {
    int32_t id;
    int32_t modality;
    float timestamp;
    std::vector<float> embedding;
    int32_t episode_id = -1;        // required when the device graph has episode ids
};

struct StreamingConfig {
    int32_t capacity = 1024;
    int32_t embedding_dim = 768;
    bool auto_flush = true;
    int32_t nsn_k = 8;              // nearest neighbours linked per new node (k-NN rule)
    double nsn_p = 0.15;            // accepted, unused (no rewiring in the k-NN rule)
};

struct FlushStats {
    int32_t nodes_committed = 0;
    int32_t edges_added = 0;
    float flush_ms = 0.0f;          // wall time of the commit (edges linked)
    float queryable_ms = 0.0f;      // until the rows were visible to scans
};

class StreamingBuffer {
public:
    explicit StreamingBuffer(const StreamingConfig& cfg);
    bool insert(int32_t id, int32_t modality, float timestamp, const float* embedding, int32_t episode_id = -1);
    bool insert(const StagedNode& node);
    FlushStats flush(DeviceMemoryGraph& target);
    int32_t staged_count() const;
    int64_t total_flushed() const;
    int32_t capacity() const { return cfg_.capacity; }
    void reset();

private:
    StreamingConfig cfg_;
    std::vector<StagedNode> buffer_;
    int64_t total_flushed_ = 0;
    mutable std::mutex mu_;
};

#endif  // STREAMING_H
