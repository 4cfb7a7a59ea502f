// ============================================================================
//  tests/cpp/shim_driver.cpp — a driver written against the reference's query
//  API (the calls of demos/embodied_scene/bench_kids_sweep.cu:589-680), built
//  against include/mars/ and linked with libmars_amd.so.
//
//  usage: shim_driver host            host-only checks (no GPU): T19 episode CSR
//         shim_driver query N SEED Q  N-node benchmark corpus; prints one line per
//                                     query: "<scope> <node> id:score:mod:hops ..."
// ============================================================================
#include "mars/memory_cuda.cuh"
#include "mars/memory_graph.h"
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
    std::printf("host ok\n");
    return 0;
}

int main(int argc, char** argv) {
    if (argc >= 2 && std::strcmp(argv[1], "host") == 0) return host_checks();
    if (argc < 5 || std::strcmp(argv[1], "query") != 0) {
        std::fprintf(stderr, "usage: shim_driver host | query N SEED Q\n");
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
