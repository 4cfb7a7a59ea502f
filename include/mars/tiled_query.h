// ============================================================================
//  mars/tiled_query.h — the reference's out-of-core tiled query API
//  (include/tiled_query.h:33-102 of MARS) served by libmars_amd on MI355X. Plain
//  C++17, no CUDA or HIP header.
//
//  Same names and semantics: per tile the exact decayed scores and the tile's
//  top-K, filtered rows dropped, the K best of all tiles by score (ties: lower
//  node id). Differences:
//    * TiledQueryContext keeps the sizes and an opaque handle; its device
//      buffers (two tile buffers: the copy of tile i+1 overlaps the scan of
//      tile i) are not exposed;
//    * TiledQueryConfig::use_fp16 is accepted and has no effect, as in the
//      reference, whose tiles are always fp32;
//    * TiledQueryStats::transfer_ms / compute_ms are summed over tiles and
//      overlap each other;
//    * errors print the library's message and exit, as CUDA_CHECK does.
// ============================================================================
#ifndef TILED_QUERY_H
#define TILED_QUERY_H

#include <cstdint>
#include <vector>

#include "memory_graph.h"

struct mars_tiled_ctx;

struct TiledQueryConfig {
    int32_t tile_size = 5000000;
    int32_t top_k = 10;
    float time_decay_lambda = 1e-8f;
    int32_t modality_filter = -1;
    bool use_fp16 = true;           // accepted, no effect
};

struct TiledQueryResult {
    int32_t node_id;
    float score;
    int32_t modality;
};

struct TiledQueryStats {
    int32_t total_nodes = 0;
    int32_t num_tiles = 0;
    float total_ms = 0.0f;
    float transfer_ms = 0.0f;
    float compute_ms = 0.0f;
    float merge_ms = 0.0f;
};

struct TiledQueryContext {
    int32_t max_tile_size = 0;
    int32_t embedding_dim = 0;
    int32_t max_k = 0;
    bool valid = false;
    mars_tiled_ctx* handle = nullptr;
};

TiledQueryContext create_tiled_context(int32_t max_tile_size, int32_t embedding_dim, int32_t max_k = 64);
void destroy_tiled_context(TiledQueryContext& ctx);

std::vector<TiledQueryResult> tiled_query(TiledQueryContext& ctx, const float* h_embeddings,
                                          const int32_t* h_modalities, const float* h_timestamps, int32_t N,
                                          int32_t D, const float* h_query, float query_timestamp,
                                          const TiledQueryConfig& cfg, TiledQueryStats& stats);

#endif  // TILED_QUERY_H
