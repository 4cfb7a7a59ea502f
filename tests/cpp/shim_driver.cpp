// ============================================================================
//  tests/cpp/shim_driver.cpp — a driver written against the reference's query
//  API (the calls of demos/embodied_scene/bench_kids_sweep.cu:589-680), built
//  against include/mars/ and linked with libmars_amd.so.
//
//  usage: shim_driver host            host-only checks (no GPU): T19 episode CSR,
//                                     T16 streaming capacity
//         shim_driver query N SEED Q  N-node benchmark corpus; prints one line per
//                                     query: "<scope> <node> id:score:mod:hops ..."
//         shim_driver stream N SEED   StreamingBuffer flush of the next 10-node episode
//                                     onto N nodes (T15), then one global query from an
//                                     inserted node at its own timestamp: "flush ..."
//                                     and "global ..." lines
//         shim_driver tiled N SEED Q  tiled_query over the host corpus (tiles of N/7):
//                                     "tiled <node> id:score:mod ..."
//         shim_driver many N SEED HOPS R  N-node corpus with the reference's NSN graph
//                                     (build_nsn_edges(6, 0.15)): checks the packed CSR
//                                     (d_row_offsets / d_col_indices) against the host
//                                     graph ("packed_csr ok"), then one global query from
//                                     node 0 with HOPS hops and max_results_returned = R:
//                                     "stats ..." and "global 0 id:score:mod:hops ..."
//         shim_driver maintain N SEED Q  the query corpus with importance and edge hits:
//                                     per query "novelty <node> <max dot>" and "ids <node>
//                                     <result ids>"; then "importance <fp32 bits in hex>"
//                                     and "low_utility <maintain_graph(dg, 0)>"
// ============================================================================
#include "mars/memory_cuda.cuh"
#include "mars/memory_graph.h"
#include "mars/streaming.h"
#include "mars/tiled_query.h"
#include "mars_amd.h"
#include "mars_corpus.h"

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

static int host_checks() {
    // T19 (tests/test_memory_graph.cpp:455-478) on 30 nodes in 3 episodes
    std::vector<int32_t> ids(30);
    for (int i = 0; i < 30; ++i) ids[i] = i / 10;
    HostEpisodeCSR csr = build_episode_csr(ids, 30);
    if (csr.num_episodes != 3 || csr.ep_csr_offsets.size() != 4 || csr.ep_csr_offsets[0] != 0 ||
        csr.ep_csr_offsets[3] != 30 || csr.ep_csr_members.size() != 30) {
        std::printf("FAIL episode csr shape\n");
        return 1;
    }
    std::vector<int> seen(30, 0);
    for (int32_t m : csr.ep_csr_members) seen[m]++;
    for (int i = 0; i < 30; ++i)
        if (seen[i] != 1) { std::printf("FAIL member %d\n", i); return 1; }
    HostEpisodeCSR bad = build_episode_csr(ids, 31);
    if (bad.num_episodes != 0) { std::printf("FAIL size mismatch\n"); return 1; }
    // T16 (tests/test_memory_graph.cpp:364-377): the sixth insert into a 5-node buffer fails
    StreamingConfig sc;
    sc.capacity = 5;
    sc.embedding_dim = 32;
    sc.auto_flush = false;
    StreamingBuffer buf(sc);
    std::vector<float> emb(32, 0.5f);
    for (int i = 0; i < 5; ++i)
        if (!buf.insert(i, MOD_AUDIO, 1.0f, emb.data())) { std::printf("FAIL insert %d\n", i); return 1; }
    if (buf.insert(5, MOD_AUDIO, 1.0f, emb.data()) || buf.staged_count() != 5) {
        std::printf("FAIL capacity\n");
        return 1;
    }
    buf.reset();
    if (buf.staged_count() != 0) { std::printf("FAIL reset\n"); return 1; }
    std::printf("host ok\n");
    return 0;
}

static void make_corpus(int32_t N, int32_t D, uint64_t seed, MemoryGraph& g, std::vector<int32_t>& ep) {
    g.num_nodes = N;
    g.embedding_dim = D;
    g.embeddings.resize(size_t(N) * D);
    g.modalities.resize(size_t(N));
    g.timestamps.resize(size_t(N));
    ep.resize(size_t(N));
    mars_corpus_params p;
    mars_corpus_default(&p, N, D, seed);
    mars_corpus_generate(&p, g.embeddings.data(), g.modalities.data(), g.timestamps.data(), ep.data(), 0);
}

static void print_results(const char* tag, int32_t node, const std::vector<QueryResult>& res, const char* tail) {
    std::printf("%s %d", tag, node);
    for (const QueryResult& r : res) std::printf(" %d:%.9g:%d:%d", r.node_id, r.score, r.modality, r.hops_from_seed);
    std::printf(" | %s\n", tail);
}

// T15 (tests/test_memory_graph.cpp:339-362) against the device graph: N nodes of the
// benchmark corpus (episode pairs only), then the next episode streamed in.
static int stream_check(int32_t N, uint64_t seed) {
    const int32_t D = 768;
    MemoryGraph full;
    std::vector<int32_t> ep;
    make_corpus(N + 10, D, seed, full, ep);
    MemoryGraph g;
    g.num_nodes = N;
    g.embedding_dim = D;
    g.embeddings.assign(full.embeddings.begin(), full.embeddings.begin() + int64_t(N) * D);
    g.modalities.assign(full.modalities.begin(), full.modalities.begin() + N);
    g.timestamps.assign(full.timestamps.begin(), full.timestamps.begin() + N);
    std::vector<int32_t> ep0(ep.begin(), ep.begin() + N);
    HostEpisodeCSR csr = build_episode_csr(ep0, N);
    // NSN CSR: intra-episode pairs
    g.row_offsets.assign(size_t(N) + 1, 0);
    for (int32_t i = 0; i < N; ++i) {
        const int32_t e = ep0[size_t(i)];
        for (int32_t m = csr.ep_csr_offsets[size_t(e)]; m < csr.ep_csr_offsets[size_t(e) + 1]; ++m)
            if (csr.ep_csr_members[size_t(m)] != i) g.col_indices.push_back(csr.ep_csr_members[size_t(m)]);
        g.row_offsets[size_t(i) + 1] = int32_t(g.col_indices.size());
    }
    g.num_edges = int32_t(g.col_indices.size());
    DeviceMemoryGraph dg = upload_to_device(g, N + 10);
    upload_episode_ids(dg, ep0.data(), N);
    upload_episode_csr(dg, csr);
    upload_fp16_embeddings(dg);
    StreamingConfig sc;
    sc.capacity = 64;
    sc.embedding_dim = D;
    StreamingBuffer buf(sc);
    for (int32_t i = 0; i < 10; ++i)
        if (!buf.insert(N + i, full.modalities[size_t(N + i)], full.timestamps[size_t(N + i)],
                        &full.embeddings[size_t(N + i) * D], ep[size_t(N + i)])) {
            std::printf("FAIL insert\n");
            return 1;
        }
    const int32_t edges0 = dg.num_edges;
    FlushStats fs = buf.flush(dg);
    std::printf("flush committed=%d edges_added=%d nodes=%d edges=%d staged=%d total=%lld\n", fs.nodes_committed,
                fs.edges_added, dg.num_nodes, dg.num_edges - edges0, buf.staged_count(),
                (long long)buf.total_flushed());
    // the flush cleared the packed CSR copy; refresh_packed_csr makes it again, equal to
    // the graph's edges as the library downloads them
    const bool cleared = dg.d_row_offsets == nullptr && dg.d_col_indices == nullptr;
    refresh_packed_csr(dg);
    std::vector<int32_t> prow(size_t(dg.num_nodes) + 1), pcol(size_t(dg.num_edges));
    std::vector<int32_t> wrow(prow.size()), wcol(pcol.size());
    const bool same = dg.d_row_offsets && dg.d_col_indices &&
                      mars_copy_to_host(prow.data(), dg.d_row_offsets, prow.size() * sizeof(int32_t)) == MARS_OK &&
                      mars_copy_to_host(pcol.data(), dg.d_col_indices, pcol.size() * sizeof(int32_t)) == MARS_OK &&
                      mars_graph_download(dg.handle, wrow.data(), wcol.data(), nullptr, nullptr) == MARS_OK &&
                      prow == wrow && pcol == wcol;
    std::printf("packed cleared=%d same=%d\n", cleared ? 1 : 0, same ? 1 : 0);
    QueryContext ctx = create_query_context(N + 10, D, 64);
    RetrievalConfig cfg;
    cfg.top_k = 10;
    cfg.time_decay_lambda = 0.1f;
    RetrievalStats st;
    const int32_t node = N + 2;
    // query time = the node's own timestamp: it, and every newer node, is undecayed
    auto res = query_memory_fast(dg, ctx, &full.embeddings[size_t(node) * D], full.timestamps[size_t(node)], cfg, st);
    print_results("global", node, res, "");
    destroy_query_context(ctx);
    free_device(dg);
    return 0;
}

static int tiled_check(int32_t N, uint64_t seed, int32_t Q) {
    const int32_t D = 768;
    MemoryGraph g;
    std::vector<int32_t> ep;
    make_corpus(N, D, seed, g, ep);
    const int32_t tile = (N + 6) / 7;
    TiledQueryContext ctx = create_tiled_context(tile, D, 64);
    TiledQueryConfig cfg;
    cfg.tile_size = tile;
    cfg.top_k = 10;
    cfg.time_decay_lambda = 0.1f;
    for (int32_t qi = 0; qi < Q; ++qi) {
        const int32_t node = (qi * 7919) % N;
        TiledQueryStats st;
        auto res = tiled_query(ctx, g.embeddings.data(), g.modalities.data(), g.timestamps.data(), N, D,
                               &g.embeddings[size_t(node) * D], 600.0f, cfg, st);
        std::printf("tiled %d", node);
        for (const TiledQueryResult& r : res) std::printf(" %d:%.9g:%d", r.node_id, r.score, r.modality);
        std::printf(" | tiles=%d\n", st.num_tiles);
    }
    destroy_tiled_context(ctx);
    return 0;
}

// Many results (memory_cuda.cu:1059, 1421-1447) and the device-side members of the
// reference structs (DeviceMemoryGraph::d_row_offsets / d_col_indices, QueryContext::stream,
// RetrievalStats).
static int many_check(int32_t N, uint64_t seed, int32_t hops, int32_t max_results) {
    const int32_t D = 768;
    MemoryGraph g;
    std::vector<int32_t> ep;
    make_corpus(N, D, seed, g, ep);
    g.build_nsn_edges(6, 0.15);
    DeviceMemoryGraph dg = upload_to_device(g);
    std::vector<int32_t> row(size_t(N) + 1), col(size_t(g.num_edges));
    if (!dg.d_row_offsets || !dg.d_col_indices ||
        mars_copy_to_host(row.data(), dg.d_row_offsets, row.size() * sizeof(int32_t)) != MARS_OK ||
        mars_copy_to_host(col.data(), dg.d_col_indices, col.size() * sizeof(int32_t)) != MARS_OK ||
        row != g.row_offsets || col != g.col_indices) {
        std::printf("FAIL packed csr\n");
        return 1;
    }
    std::printf("packed_csr ok %d %d\n", N, g.num_edges);
    QueryContext ctx = create_query_context(N, D, 64);
    if (!ctx.stream) { std::printf("FAIL stream\n"); return 1; }
    RetrievalConfig cfg;
    cfg.top_k = 10;
    cfg.bfs_max_hops = hops;
    cfg.time_decay_lambda = 0.1f;
    cfg.max_results_returned = max_results;
    RetrievalStats st;
    auto res = query_memory_fast(dg, ctx, &g.embeddings[0], 600.0f, cfg, st);
    std::printf("stats similarity=%.6f rerank=%.6f topk=%.6f bfs=%.6f total=%.6f scanned=%d waves=%d\n",
                st.gpu_ms_similarity, st.gpu_ms_rerank, st.gpu_ms_topk, st.gpu_ms_bfs, st.gpu_ms_total,
                st.nodes_scanned, st.bfs_waves);
    print_results("global", 0, res, "");
    destroy_query_context(ctx);
    free_device(dg);
    return 0;
}

int main(int argc, char** argv) {
    if (argc >= 2 && std::strcmp(argv[1], "host") == 0) return host_checks();
    if (argc >= 4 && std::strcmp(argv[1], "stream") == 0)
        return stream_check(std::atoi(argv[2]), std::strtoull(argv[3], nullptr, 10));
    if (argc >= 6 && std::strcmp(argv[1], "many") == 0)
        return many_check(std::atoi(argv[2]), std::strtoull(argv[3], nullptr, 10), std::atoi(argv[4]),
                          std::atoi(argv[5]));
    if (argc >= 5 && std::strcmp(argv[1], "tiled") == 0)
        return tiled_check(std::atoi(argv[2]), std::strtoull(argv[3], nullptr, 10), std::atoi(argv[4]));
    const bool maintain = argc >= 5 && std::strcmp(argv[1], "maintain") == 0;
    if (argc < 5 || (std::strcmp(argv[1], "query") != 0 && !maintain)) {
        std::fprintf(stderr, "usage: shim_driver host | query N SEED Q | maintain N SEED Q\n");
        return 2;
    }
    const int32_t N = std::atoi(argv[2]);
    const uint64_t seed = std::strtoull(argv[3], nullptr, 10);
    const int32_t Q = std::atoi(argv[4]);
    const int32_t D = 768;

    MemoryGraph g;
    g.num_nodes = N;
    g.embedding_dim = D;
    g.embeddings.resize(size_t(N) * D);
    g.modalities.resize(size_t(N));
    g.timestamps.resize(size_t(N));
    std::vector<int32_t> ep(static_cast<size_t>(N));
    mars_corpus_params p;
    mars_corpus_default(&p, N, D, seed);
    mars_corpus_generate(&p, g.embeddings.data(), g.modalities.data(), g.timestamps.data(), ep.data(), 0);
    std::vector<int32_t> knn(size_t(N) * 8);
    mars_knn_cpu(g.embeddings.data(), N, D, 8, knn.data(), nullptr, 0);
    int64_t ne = 0;
    g.row_offsets.resize(size_t(N) + 1);
    mars_build_nsn_csr(N, ep.data(), knn.data(), 8, g.row_offsets.data(), nullptr, &ne, 0);
    g.col_indices.resize(size_t(ne));
    mars_build_nsn_csr(N, ep.data(), knn.data(), 8, g.row_offsets.data(), g.col_indices.data(), &ne, 0);
    g.num_edges = int32_t(ne);

    // the reference driver sequence (bench_kids_sweep.cu:614-680)
    HostEpisodeCSR ep_csr = build_episode_csr(ep, g.num_nodes);
    DeviceMemoryGraph dg = upload_to_device(g);
    upload_episode_ids(dg, ep.data(), g.num_nodes);
    upload_episode_csr(dg, ep_csr);
    QueryContext ctx = create_query_context(g.num_nodes, D, 64);

    std::vector<int32_t> qn(static_cast<size_t>(Q));
    mars_corpus_pick_queries(g.modalities.data(), N, MOD_IMAGE, Q, seed + 1, qn.data());
    if (maintain) {
        // memory_cuda.cuh:234-270 in the order a serving loop would call them
        init_importance(dg);
        init_edge_hits(dg);
        void* d_q = nullptr;
        void* d_ids = nullptr;
        if (mars_device_alloc(size_t(D) * sizeof(float), &d_q) != MARS_OK ||
            mars_device_alloc(64 * sizeof(int32_t), &d_ids) != MARS_OK) {
            std::printf("FAIL alloc\n");
            return 1;
        }
        for (int32_t i = 0; i < Q; ++i) {
            const int32_t node = qn[size_t(i)];
            const float* q = &g.embeddings[size_t(node) * D];
            mars_copy_to_device(d_q, q, size_t(D) * sizeof(float));
            std::printf("novelty %d %.9g\n", node, double(compute_novelty(dg, static_cast<const float*>(d_q))));
            RetrievalConfig cfg;
            cfg.top_k = 10;
            cfg.max_results_returned = 15;
            cfg.time_decay_lambda = 0.1f;
            RetrievalStats stats;
            auto res = query_memory_fast(dg, ctx, q, 600.0f, cfg, stats);
            count_edge_hits(dg, ctx);
            std::vector<int32_t> ids;
            for (const auto& r : res) ids.push_back(r.node_id);
            std::printf("ids %d", node);
            for (int32_t id : ids) std::printf(" %d", id);
            std::printf("\n");
            mars_copy_to_device(d_ids, ids.data(), ids.size() * sizeof(int32_t));
            update_importance(dg, static_cast<const int32_t*>(d_ids), int32_t(ids.size()));
        }
        std::vector<float> imp(static_cast<size_t>(N));
        if (mars_importance_read(dg.handle, imp.data(), 0, N) != MARS_OK) {
            std::printf("FAIL importance read\n");
            return 1;
        }
        std::printf("importance");
        for (const float v : imp) {
            uint32_t u;
            std::memcpy(&u, &v, 4);
            std::printf(" %08x", u);
        }
        std::printf("\n");
        std::printf("low_utility %d\n", maintain_graph(dg, 0));
        mars_device_free(d_q);
        mars_device_free(d_ids);
        destroy_query_context(ctx);
        free_device(dg);
        return 0;
    }
    for (int32_t i = 0; i < Q; ++i) {
        const int32_t node = qn[size_t(i)];
        for (int scope = 0; scope < 2; ++scope) {
            RetrievalConfig cfg;
            cfg.top_k = 10;
            cfg.max_results_returned = 15;
            cfg.bfs_max_hops = 2;
            cfg.time_decay_lambda = 0.1f;
            cfg.bfs_score_decay = 0.5f;
            cfg.retrieval_scope = scope ? RetrievalScope::EpisodeScoped : RetrievalScope::Global;
            const int32_t e = ep[size_t(node)];
            cfg.query_episode_id = e;
            if (scope) {
                cfg.query_episode_member_begin = ep_csr.ep_csr_offsets[size_t(e)];
                cfg.query_episode_member_count = ep_csr.ep_csr_offsets[size_t(e) + 1] - ep_csr.ep_csr_offsets[size_t(e)];
            }
            RetrievalStats stats;
            auto res = query_memory_fast(dg, ctx, &g.embeddings[size_t(node) * D], 600.0f, cfg, stats);
            std::printf("%s %d", scope ? "episode" : "global", node);
            for (const auto& r : res) std::printf(" %d:%.9g:%d:%d", r.node_id, r.score, r.modality, r.hops_from_seed);
            std::printf(" | scanned=%d waves=%d total_ms=%.4f\n", stats.nodes_scanned, stats.bfs_waves,
                        stats.gpu_ms_total);
        }
    }
    destroy_query_context(ctx);
    free_device(dg);
    return 0;
}
