/*
 * mars_corpus.h — seeded synthetic corpus of the episode/modality benchmark
 * workload, its NSN graph and episode CSR (host C ABI, no GPU needed unless
 * noted).
 *
 * Workload definition (the benchmark corpus; D = embedding_dim):
 *   * episodes of `episode_len` (default 10) consecutive node ids; slots 0-3 IMAGE,
 *     4-6 TEXT, 7-9 AUDIO (slot s >= 10 cycles that template);
 *   * per episode a centroid c ~ N(0, I_D); per node noise g ~ N(0, I_D);
 *     IMAGE = normalize(c + 0.3 g), TEXT/AUDIO = normalize(0.35 c + g);
 *   * episode start ~ U[0, 599) s, node timestamp = start + 0.1 s * slot
 *     (all nodes of an episode inside 1 s, every timestamp <= 600 s);
 *   * NSN edges: every intra-episode pair plus each node's 8 nearest neighbours
 *     by cosine (ties: lower id), symmetrised, de-duplicated, rows ascending;
 *   * queries: IMAGE nodes drawn with replacement; the query vector is the
 *     node's embedding, query time t = 600 s.
 *
 * Randomness is counter based (SplitMix64 finaliser over (seed, stream, index),
 * Box-Muller in double precision), so any node can be generated independently
 * and the output does not depend on the thread count.
 *
 * Reference analogue (not the same distribution): EmbodiedKidsBallCorpus::make
 * (src/memory_graph.cpp:241-295) and MemoryGraph::build_nsn_edges
 * (src/memory_graph.cpp:95-189).
 */
#ifndef MARS_CORPUS_H
#define MARS_CORPUS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mars_corpus_params {
    int64_t  num_nodes;
    int32_t  embedding_dim;
    int32_t  episode_len;      /* 10 */
    uint64_t seed;
    float    image_noise;      /* 0.3  */
    float    other_centroid;   /* 0.35 */
    float    start_max;        /* 599  */
    float    slot_dt;          /* 0.1  */
} mars_corpus_params;

void mars_corpus_default(mars_corpus_params* p, int64_t num_nodes, int32_t dim, uint64_t seed);

/* Fill embeddings (N*D), modalities, timestamps and episode ids (all N). Any
 * output pointer may be NULL. threads <= 0: hardware concurrency. */
int mars_corpus_generate(const mars_corpus_params* p, float* emb, int32_t* modalities,
                         float* timestamps, int32_t* episode_ids, int32_t threads);

/* n_queries node ids drawn with replacement among nodes whose modality == mod. */
int mars_corpus_pick_queries(const int32_t* modalities, int64_t n, int32_t mod,
                             int32_t n_queries, uint64_t seed, int32_t* out_nodes);

/* Exact k nearest neighbours by fp32 dot product (sequential sum over d, so the
 * result is independent of threading), excluding the node itself; ties by lower
 * id. nbrs: N*k ids (row i sorted by score desc), sims: N*k (may be NULL). */
int mars_knn_cpu(const float* emb, int64_t n, int32_t dim, int32_t k,
                 int32_t* nbrs, float* sims, int32_t threads);

/* NSN CSR = intra-episode pairs U kNN, symmetrised, de-duplicated, rows ascending.
 * Call with col == NULL to get *num_edges, then with a buffer of that size.
 * row_offsets has n+1 entries. episode_ids: n entries (>= 0). knn: n*k (ids < 0 skipped). */
int mars_build_nsn_csr(int64_t n, const int32_t* episode_ids, const int32_t* knn, int32_t k,
                       int32_t* row_offsets, int32_t* col, int64_t* num_edges, int32_t threads);

/* build_episode_csr (src/memory_graph.cpp:12-44): counting sort of node ids by
 * episode id, members ascending inside an episode, num_episodes = max id + 1.
 * Call with offsets == NULL to get *num_episodes. Returns MARS_ERR_INVALID (-1)
 * for a negative id. */
int mars_build_episode_csr(const int32_t* episode_ids, int32_t n, int32_t* num_episodes,
                           int32_t* offsets, int32_t* members);

#ifdef __cplusplus
}
#endif
#endif /* MARS_CORPUS_H */
