/*
 * mars_amd.h — C ABI of the MI355X (gfx950) retrieval hot path.
 *
 * Plain C, plain pointers and sizes. Every entry point returns an int status
 * (MARS_OK == 0, negative on error) and never exits the process; the text of
 * the last error on the calling thread is available from mars_last_error().
 *
 * Object model (mirrors the reference's DeviceMemoryGraph / QueryContext split):
 *   mars_graph  — device-resident corpus: embeddings (fp32, optional fp16 copy),
 *                 timestamps, modalities, NSN CSR, optional episode ids / CSR.
 *   mars_ctx    — per-thread query context: stream, scratch, pinned staging.
 *                 One context serves one thread at a time (same contract as
 *                 the reference's QueryContext).
 *
 * Reference interfaces replaced (paths relative to the MARS source tree):
 *   include/memory_cuda.cuh:63-97    DeviceMemoryGraph, upload_to_device, free_device,
 *                                    upload_episode_ids, upload_episode_csr,
 *                                    upload_fp16_embeddings, free_fp16_embeddings
 *   include/memory_cuda.cuh:100-137  QueryResult, RetrievalConfig, RetrievalStats
 *   include/memory_cuda.cuh:141-231  query_memory, QueryContext, create_query_context,
 *                                    destroy_query_context, query_memory_fast
 *   include/memory_graph.h:70-81     HostEpisodeCSR, build_episode_csr, RetrievalScope
 *   include/streaming.h:42-81        StreamingBuffer::insert / flush (device-side append)
 *   include/tiled_query.h:33-102     TiledQueryConfig/Result/Stats, tiled_query
 */
#ifndef MARS_AMD_H
#define MARS_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MARS_ABI_VERSION 1

/* ---- status codes -------------------------------------------------------- */
#define MARS_OK              0
#define MARS_ERR_INVALID    -1   /* bad argument / inconsistent input          */
#define MARS_ERR_HIP        -2   /* a HIP runtime call failed                  */
#define MARS_ERR_NOMEM      -3   /* device or host allocation failed           */
#define MARS_ERR_CAPACITY   -4   /* input larger than the object was sized for */
#define MARS_ERR_UNSUPPORTED -5  /* valid request this build does not serve    */
#define MARS_ERR_NODEVICE   -6   /* no usable gfx950 device                    */

/* ---- modality tags (memory_graph.h:17-22) --------------------------------- */
#define MARS_MOD_TEXT  0
#define MARS_MOD_AUDIO 1
#define MARS_MOD_IMAGE 2

/* ---- retrieval scope (memory_graph.h:79-81, enum class RetrievalScope) ---- */
#define MARS_SCOPE_GLOBAL          0
#define MARS_SCOPE_EPISODE_SCOPED  1

/* Result record, 16 bytes: same field order as QueryResult (memory_cuda.cuh:100-105). */
typedef struct mars_query_result {
    int32_t node_id;
    float   score;
    int32_t modality;
    int32_t hops_from_seed;   /* 0 = seed, 1+ = reached by BFS */
} mars_query_result;

/* RetrievalConfig (memory_cuda.cuh:107-127) with bool / enum class as int32_t.
 * Field order and defaults are the reference's; see mars_config_default(). */
typedef struct mars_retrieval_config {
    int32_t top_k;                     /* default 10                                 */
    int32_t bfs_max_hops;              /* default 2                                  */
    float   time_decay_lambda;         /* default 1e-8 (per second)                  */
    float   bfs_score_decay;           /* default 0.5 (per-hop multiplier)           */
    int32_t modality_filter;           /* default -1 (any)                           */
    int32_t use_importance;            /* accepted, never read (as in the reference) */
    int32_t max_results_returned;      /* default -1 (= K)                           */
    int32_t retrieval_scope;           /* MARS_SCOPE_*                               */
    int32_t query_episode_id;          /* default -1                                 */
    int32_t query_episode_member_begin;
    int32_t query_episode_member_count;
    float   episode_same_boost;        /* default 0 (off)                            */
} mars_retrieval_config;

/* RetrievalStats (memory_cuda.cuh:129-137) plus fields the reference lacks. */
typedef struct mars_stats {
    float   gpu_ms_similarity;
    float   gpu_ms_topk;
    float   gpu_ms_bfs;
    float   gpu_ms_rerank;
    float   gpu_ms_total;
    int32_t nodes_scanned;
    int32_t bfs_waves;          /* reference semantics: cfg.bfs_max_hops (global), 0 (scoped) */
    /* extensions */
    int32_t scope_fallback;     /* 1 if EpisodeScoped was requested but inactive -> Global */
    int32_t visited;            /* number of nodes reached (seeds + BFS)                  */
    int32_t bfs_levels_run;     /* BFS levels actually expanded                           */
    int32_t used_fp16;          /* 1 if the fp16 corpus was scanned                       */
    int32_t seeds_certified;    /* MARS_CTX_CERTIFIED: 1 if the fp16 scan's seeds were certified
                                   (0: the fp32 scan answered the query)                     */
    int32_t results_capped;     /* 1 if max_results_returned exceeded the context's result cap
                                   min(max_nodes, max_k * 500) and more nodes were reached than
                                   that cap: the call returned the cap's best results (the
                                   reference keeps the first ones in visit order)          */
    double  wall_us;            /* host wall time of the call                             */
} mars_stats;

/* Graph descriptor for mars_graph_create. Pointers are host memory unless
 * flags has MARS_DESC_DEVICE_POINTERS, in which case the graph adopts copies
 * made device-to-device (the caller keeps ownership of its buffers). */
#define MARS_DESC_DEVICE_POINTERS 0x1u
typedef struct mars_graph_desc {
    int32_t        num_nodes;
    int32_t        num_edges;        /* length of col_indices (both directions) */
    int32_t        embedding_dim;
    const int32_t* row_offsets;      /* num_nodes + 1 (may be NULL if num_edges == 0) */
    const int32_t* col_indices;      /* num_edges; no duplicate id inside a row       */
    const float*   embeddings;       /* num_nodes * embedding_dim, row-major, unit L2 */
    const int32_t* modalities;       /* num_nodes                                     */
    const float*   timestamps;       /* num_nodes (seconds)                           */
    int32_t        capacity_nodes;   /* >= num_nodes; room for streaming append (0 = num_nodes) */
    int64_t        capacity_edges;   /* col slots for streaming append; 0 = num_edges + 256 per spare node */
    uint32_t       flags;
} mars_graph_desc;

typedef struct mars_graph mars_graph;
typedef struct mars_ctx   mars_ctx;

/* Read-only view of a graph's device arrays (DeviceMemoryGraph fields). */
typedef struct mars_graph_view {
    int32_t  num_nodes;
    int32_t  num_edges;
    int32_t  embedding_dim;
    int32_t  episode_num_episodes;
    int32_t  episode_csr_member_total;
    int32_t  has_fp16;
    void*    d_row_words;      /* int64 per node: (row length << 32) | row start in col */
    void*    d_col_indices;
    void*    d_embeddings;
    void*    d_embeddings_fp16;
    void*    d_modalities;
    void*    d_timestamps;
    void*    d_episode_ids;
    void*    d_ep_csr_offsets;
    void*    d_ep_csr_members;
} mars_graph_view;

/* ---- library ------------------------------------------------------------- */
const char* mars_last_error(void);
int         mars_abi_version(void);
/* Initialise HIP on `device`; fails with MARS_ERR_NODEVICE if it is not gfx950. */
int         mars_init(int32_t device);
void        mars_config_default(mars_retrieval_config* cfg);

/* ---- graph (memory_cuda.cuh:87-97) ------------------------------------------ */
/* upload_to_device */
int mars_graph_create(const mars_graph_desc* desc, mars_graph** out);
/* free_device */
int mars_graph_destroy(mars_graph* g);
/* The calls below that replace device arrays (mars_graph_set_episode_ids,
 * mars_graph_set_episode_csr, mars_graph_disable_fp16, mars_graph_disable_int8,
 * mars_graph_set_csr) free the
 * arrays they replace: no query, on any context or thread, may run on the graph during
 * them. (Inserts and links do not free what queries read: queries keep running during
 * those.) */
/* upload_episode_ids: n must equal num_nodes; NULL/n<=0 clears (reference: silent no-op). */
int mars_graph_set_episode_ids(mars_graph* g, const int32_t* episode_ids, int32_t n);
/* upload_episode_csr: offsets has num_episodes+1 entries, members has offsets[num_episodes]. */
int mars_graph_set_episode_csr(mars_graph* g, int32_t num_episodes,
                               const int32_t* offsets, const int32_t* members,
                               int32_t member_total);
/* upload_fp16_embeddings / free_fp16_embeddings (RNE fp32->fp16, 64-bit indexing). */
int mars_graph_enable_fp16(mars_graph* g);
int mars_graph_disable_fp16(mars_graph* g);
/* No counterpart in the reference: an int8 copy of the rows for the certified global
 * query (MARS_CTX_CERTIFIED). Row r is kept as bytes v in [-127, 127] with one scale
 * s_r = max|e_r| / 127 and a bound c_r on |int8 dot - fp32 dot| / |q| (its quantisation
 * residual norm plus both scans' rounding), maintained through inserts and
 * mars_graph_set_rows: d + 8 bytes per row (cap_n rows). embedding_dim must be 256, 512,
 * 768, 1024 or 1536 (the certified query uses it up to 1024). */
int mars_graph_enable_int8(mars_graph* g);
int mars_graph_disable_int8(mars_graph* g);
/* Copies rows [first, first + count) of the int8 copy to host memory: count * d bytes
 * and/or count (scale, bound) float pairs (either pointer may be NULL). */
int mars_graph_read_int8(const mars_graph* g, int32_t first, int32_t count, int8_t* bytes, float* meta);
int mars_graph_get_view(const mars_graph* g, mars_graph_view* out);
/* Replace the NSN CSR of a graph (host arrays, validated like mars_graph_create). */
int mars_graph_set_csr(mars_graph* g, int32_t num_edges, const int32_t* row_offsets,
                       const int32_t* col_indices);
/* k nearest neighbours of every node by cosine (the node itself excluded, ties: lower
 * id): an fp16 MFMA scan keeps 16 candidates per node, exact fp32 rescoring keeps
 * k <= 16. Needs the fp16 copy. nbrs: host, num_nodes * k ids. Builds the k-NN part
 * of the NSN graph at corpus sizes a CPU cannot (analogue of the tiled kNN build of
 * src/cmng_build.cu:135-245). Each node's list is certified exact when its k-th exact
 * score beats the 16th candidate's fp16 score by more than the fp16 scan's error bound
 * (from the fp16 copy's row-norm maxima); the lists the certificate does not cover are
 * found again by exact fp32 scans (mars_graph_knn_report counts both). */
int mars_graph_knn(mars_graph* g, int32_t k, int32_t* nbrs);
/* Counts of the last k-NN builder call on g (mars_graph_knn, _blocked, _blocks, _range):
 * the nodes whose lists the certificate did not cover, and of those the nodes found again
 * by exact scans (all-pairs builds; a build within blocks only counts them). No reference
 * counterpart: the reference's builders report nothing of the kind. */
int mars_graph_knn_report(const mars_graph* g, int64_t* uncertified, int64_t* rescanned);
/* The same within blocks: each node's k nearest among the nodes of its block of
 * block_rows consecutive ids (block_rows >= num_nodes: mars_graph_knn). For corpora
 * where the exact all-pairs search is too long to build (13M rows: ~2.6e17 FLOP). */
int mars_graph_knn_blocked(mars_graph* g, int32_t k, int32_t block_rows, int32_t* nbrs);
/* The same for blocks [first_block, first_block + n_blocks) only: nbrs receives the rows
 * of nodes first_block * block_rows .. (at most n_blocks * block_rows rows, clipped to
 * the node count), so a caller can build a large graph block by block. */
int mars_graph_knn_blocks(mars_graph* g, int32_t k, int32_t block_rows, int32_t first_block, int32_t n_blocks,
                          int32_t* nbrs);
/* The all-pairs k-NN of nodes first .. first + count - 1 (each node's k nearest among all
 * nodes, itself excluded; the same answer as rows first .. of mars_graph_knn), so that an
 * all-pairs build can run in pieces (nbrs: count * k). No reference counterpart: the
 * reference builds its graph on the host (memory_graph.cpp:102-189). */
int mars_graph_knn_range(mars_graph* g, int32_t k, int32_t first, int32_t count, int32_t* nbrs);
/* Measurement aid, no counterpart in the reference: the bandwidth (GB/s, best of 256,
 * 512 and 1024 workgroups, reps timed launches each) of a plain streaming read of the
 * graph's fp32 (fp16 = 0) or fp16 rows with no arithmetic, the practical ceiling of the
 * row scans on this device. MARS_ERR_UNSUPPORTED when those rows are absent. */
int mars_graph_read_ceiling(const mars_graph* g, int32_t fp16, int32_t reps, double* gbps);
/* Measurement aid, no counterpart in the reference: the same measurement for an access
 * pattern. pattern 0: the plain stream of mars_graph_read_ceiling over the fp16 rows;
 * 1: the batched scan's fragment loads over the fp16 rows, 16 rows x 64 bytes per load
 * instruction (a row's 64-byte k-chunks back to back, 16-row tiles grid-strided; whole
 * 16-row tiles counted); 2: pattern 1 with non-temporal loads; 3: the plain stream over
 * the int8 copy. MARS_ERR_INVALID for another pattern, MARS_ERR_UNSUPPORTED without the
 * rows the pattern reads or (1, 2) when embedding_dim is not a multiple of 32. */
int mars_graph_read_pattern(const mars_graph* g, int32_t pattern, int32_t reps, double* gbps);
/* Copy device arrays back to host (any pointer may be NULL to skip): the NSN graph as
 * a packed CSR (row_offsets: num_nodes + 1, col_indices: num_edges) and the episode CSR. */
int mars_graph_download(const mars_graph* g, int32_t* row_offsets, int32_t* col_indices,
                        int32_t* ep_offsets, int32_t* ep_members);
/* DeviceMemoryGraph::d_row_offsets / d_col_indices (memory_cuda.cuh:63-85): the graph's
 * edges as a packed CSR in device memory, int32 [num_nodes + 1] and [num_edges]. The
 * queries read the graph's own row words, in which a row that grew by a streaming insert
 * can sit apart from its neighbours; this is a copy made for callers that expect the
 * reference's layout. Built on the first call and again after the edges changed; owned
 * by the graph (valid until the next change of the edges or mars_graph_destroy). */
int mars_graph_packed_csr(mars_graph* g, const int32_t** d_row_offsets, const int32_t** d_col_indices);

/* ---- files: MARS v1 graph checkpoints and the KIDS corpus -------------------
 * MARS v1 (persistence.h:8-18): "MARS", uint32 version 1, int32 num_nodes,
 * num_edges, embedding_dim, row_offsets[num_nodes + 1], col_indices[num_edges],
 * embeddings[num_nodes * dim] (float), modalities[num_nodes], timestamps[num_nodes]
 * (float), then the FNV-1a 64-bit hash of every preceding byte; native byte order.
 * A file loads only if magic, version (MARS_ERR_UNSUPPORTED otherwise), exact size
 * and hash all check (persistence.cpp load_graph returns false on each). */
/* fnv1a_checksum (persistence.h:37): FNV-1a 64 of len bytes. */
int mars_fnv1a64(const void* data, int64_t len, uint64_t* out);
/* save_graph (persistence.h:29) from host arrays. */
int mars_graph_file_save(const char* path, int32_t num_nodes, int32_t num_edges, int32_t dim,
                         const int32_t* row_offsets, const int32_t* col_indices,
                         const float* embeddings, const int32_t* modalities,
                         const float* timestamps);
/* load_graph (persistence.h:33) in two calls: the sizes (header and file size
 * checked), then the arrays into caller buffers of those sizes (hash checked; on an
 * error the buffers' contents are unspecified, as the reference's graph is). */
int mars_graph_file_info(const char* path, int32_t* num_nodes, int32_t* num_edges, int32_t* dim);
int mars_graph_file_load(const char* path, int32_t num_nodes, int32_t num_edges, int32_t dim,
                         int32_t* row_offsets, int32_t* col_indices, float* embeddings,
                         int32_t* modalities, float* timestamps);
/* save_graph of the device-resident graph (streamed inserts included): a checkpoint
 * with no host copy of the whole corpus (rows are streamed in 64 MB pieces). */
int mars_graph_save(const mars_graph* g, const char* path);
/* KIDS binary corpus (bench_kids_sweep.cu:29-37, write_corpus_bin :84-102; reader
 * scripts/bench_kids_ball_cuvs_cagra.py:49-60): uint32 0x5344494b ("KIDS"), uint32
 * version 1, int32 N, D, embeddings[N * D], timestamps[N], modalities[N],
 * episode_ids[N]. Reading checks the magic and the exact size (the version is not
 * read, as in the reference reader). */
int mars_kids_file_write(const char* path, int32_t n, int32_t d, const float* embeddings,
                         const float* timestamps, const int32_t* modalities,
                         const int32_t* episode_ids);
int mars_kids_file_info(const char* path, int32_t* n, int32_t* d);
int mars_kids_file_read(const char* path, int32_t n, int32_t d, float* embeddings, float* timestamps,
                        int32_t* modalities, int32_t* episode_ids);

/* ---- streaming insert (streaming.cpp:35-163, engine_server.cu:154-213) ------- */
typedef struct mars_insert_stats {
    int32_t first_node;       /* id of the first inserted node (ids are consecutive)   */
    int32_t nodes_added;
    int64_t edges_added;      /* CSR entries added (each edge in both directions)      */
    int32_t rows_relocated;   /* old rows moved to a tail region of col                */
    int32_t rows_appended;    /* old rows extended in place                            */
    double  queryable_us;     /* call -> nodes visible to scans and episode scope       */
    double  linked_us;        /* call -> NSN edges visible to the BFS (call returns)    */
    double  knn_us;           /* device time of the neighbour search                   */
} mars_insert_stats;

/* Append n_new nodes (host arrays: rows n_new * embedding_dim, modalities, timestamps)
 * on the graph's side stream; queries on other threads / contexts keep running.
 * Replaces StreamingBuffer::insert + flush (streaming.cpp:13-80) and its
 * add_incremental_edges_ (:97-163), which rebuild the whole CSR on the host before a
 * re-upload. Edge rule: intra-episode pairs among the new nodes plus each new node's
 * knn_k nearest neighbours by cosine over all nodes (fp16 MFMA candidates, exact fp32
 * order, ties by lower id), stored in both directions, rows ascending.
 * episode_ids: required iff the graph has episode ids; each must open a new episode
 * (>= every episode id already present); the episode CSR, when present, is appended.
 * knn_k in [0, 16]; knn_k > 0 needs the fp16 copy. out_knn (nullable): n_new * knn_k
 * neighbour ids found (-1: none). Nodes become visible to scans first (queryable_us),
 * then their edges (linked_us); a query that runs meanwhile sees each row either as
 * before or as after the insert. MARS_ERR_CAPACITY when capacity_nodes /
 * capacity_edges (mars_graph_desc) cannot hold the insert: nothing is changed then.
 * Any other error (MARS_ERR_NOMEM, MARS_ERR_HIP) may come after the nodes were
 * published: they are then queryable without their edges (num_nodes of
 * mars_graph_get_view has moved past them, and their episodes count as opened), and the
 * same insert cannot be repeated. mars_graph_link_knn(g, first, n_new, knn_k, ...) with
 * first = the num_nodes read before the call adds the edges the insert would have. */
int mars_graph_insert(mars_graph* g, int32_t n_new, const float* embeddings, const int32_t* modalities,
                      const float* timestamps, const int32_t* episode_ids, int32_t knn_k,
                      int32_t* out_knn, mars_insert_stats* stats);
/* Replace published rows [first, first + count) in place: fp32 rows, modalities and
 * timestamps (the fp16 copy follows); edges are unchanged. No counterpart function in
 * the reference: its engine server rewrites the host MemoryGraph for an ADD of an
 * existing id or a DELETE tombstone (engine_server.cu:154-191). Rows being replaced
 * must not be read by a concurrent query. */
int mars_graph_set_rows(mars_graph* g, int32_t first, int32_t count, const float* embeddings,
                        const int32_t* modalities, const float* timestamps);

/* Deferred k-NN edges (the second half of add_incremental_edges_, streaming.cpp:97-163,
 * taken out of the insert so that many inserts share one corpus pass): nodes inserted
 * with knn_k = 0 are queryable at once; later their neighbour edges are added here.
 * mars_graph_link adds the edges between node first + i and each id nbrs[i * k + j]
 * (-1 skipped, self skipped), in both directions; the edge set becomes the union (no
 * duplicate entries), rows stay ascending. mars_graph_link_knn first finds each node's
 * knn_k nearest neighbours among all published nodes (as mars_graph_insert does, over
 * the nodes published when it runs; out_knn nullable, count * knn_k ids). Inserting
 * with knn_k = 0 and then linking with knn_k gives the graph a single insert with
 * knn_k gives. Nodes first .. first + count - 1 must be published. Runs on the side
 * stream under the graph mutex; queries keep running and see each row before or after.
 * stats: first_node, nodes_added (= count), edges_added, rows_relocated (rewritten
 * into the tail), rows_appended, linked_us, knn_us. */
int mars_graph_link(mars_graph* g, int32_t first, int32_t count, int32_t k, const int32_t* nbrs,
                    mars_insert_stats* stats);
int mars_graph_link_knn(mars_graph* g, int32_t first, int32_t count, int32_t knn_k, int32_t* out_knn,
                        mars_insert_stats* stats);

/* ---- tiled out-of-core comparator (include/tiled_query.h:33-102) ------------- */
/* TiledQueryConfig (tiled_query.h:33-39), same defaults (mars_tiled_config_default).
 * use_fp16 is accepted and ignored, as in the reference (its tiles are always fp32). */
typedef struct mars_tiled_config {
    int32_t tile_size;             /* rows per tile, default 5,000,000            */
    int32_t top_k;                 /* default 10                                   */
    float   time_decay_lambda;     /* default 1e-8                                 */
    int32_t modality_filter;       /* default -1                                   */
    int32_t use_fp16;              /* default 1, no effect                         */
} mars_tiled_config;
/* TiledQueryResult (tiled_query.h:41-45), 12 bytes. */
typedef struct mars_tiled_result {
    int32_t node_id;
    float   score;
    int32_t modality;
} mars_tiled_result;
/* TiledQueryStats (tiled_query.h:47-54) plus the achieved host-to-device rate.
 * Copies of tile i+1 overlap the scan of tile i, so transfer_ms + compute_ms can
 * exceed total_ms. */
typedef struct mars_tiled_stats {
    int32_t total_nodes;
    int32_t num_tiles;
    float   total_ms;
    float   transfer_ms;           /* sum of tile copy times (events on the copy stream) */
    float   compute_ms;            /* sum of tile scan + merge times                      */
    float   merge_ms;              /* host decode of the K keys                           */
    double  h2d_gbs;               /* bytes copied / transfer_ms                          */
} mars_tiled_stats;
typedef struct mars_tiled_ctx mars_tiled_ctx;
void mars_tiled_config_default(mars_tiled_config* cfg);
/* create_tiled_context / destroy_tiled_context (tiled_query.h:79-83): two device tile
 * buffers of max_tile_size rows (copy of tile i+1 overlaps the scan of tile i). */
int mars_tiled_ctx_create(int32_t max_tile_size, int32_t embedding_dim, int32_t max_k, mars_tiled_ctx** out);
int mars_tiled_ctx_destroy(mars_tiled_ctx* ctx);
/* tiled_query (tiled_query.h:85-102, tiled_query.cu:174-314): host-resident corpus
 * (embeddings n * d fp32, modalities, timestamps); per tile the exact decayed top-K,
 * filtered rows (score -FLT_MAX) dropped, the K best of all tiles by (score desc, id
 * asc) in out[0 .. *n_out). Host arrays from mars_host_alloc are copied at PCIe rate;
 * pageable arrays are staged by the runtime. */
int mars_tiled_query(mars_tiled_ctx* ctx, const float* embeddings, const int32_t* modalities,
                     const float* timestamps, int32_t n, int32_t d, const float* query, float query_timestamp,
                     const mars_tiled_config* cfg, mars_tiled_result* out, int32_t cap, int32_t* n_out,
                     mars_tiled_stats* stats);
/* Pinned host memory (hipHostMalloc) for corpora streamed by mars_tiled_query. */
int mars_host_alloc(size_t bytes, void** ptr);
int mars_host_free(void* ptr);

/* ---- query context (memory_cuda.cuh:141-231) --------------------------------- */
#define MARS_CTX_USE_FP16    0x1u   /* scan the fp16 copy when present (ctx.use_fp16)      */
#define MARS_CTX_USE_GRAPH   0x2u   /* replay the query pipeline as a hipGraph             */
#define MARS_CTX_TIMING      0x4u   /* fill per-stage gpu_ms_* with hipEvents              */
/* Global queries scan a reduced-precision copy and return exactly the fp32 path's
 * results. With the int8 copy (mars_graph_enable_int8; a quarter of the fp32 bytes) the
 * scan ranks rows by an upper bound of their fp32 score (int8 score + |q| c_r) and keeps
 * 64 candidates; when the K-th exact score of the candidates exceeds the 64th candidate's
 * bound, no other row can enter the top K. Otherwise, with the fp16 copy (half the
 * bytes), it keeps 32 candidates (64 for K > 16, 16 for K <= 10) and the certificate
 * asks the K-th exact score to exceed the last candidate's fp16 score by the fp16 error
 * bound of any row (from the rows' rounding residual norms, kept with the fp16 copy).
 * Candidates are rescored in the fp32 scan's own arithmetic, and the BFS then scores
 * every visited node exactly. A query the certificate does not cover is answered by
 * the fp32 scan (stats.seeds_certified = 0). Needs the int8 or the fp16 copy; ignored
 * with MARS_CTX_USE_FP16 (which returns fp16 scores), for episode scope, a same-episode
 * boost, lambda < 0 and embedding_dim not a multiple of 128 (above 1024: int8 copy
 * unused, fp16 copy required up to 1024). MARS_CTX_USE_GRAPH does not apply to it.
 * After a certified query, mars_ctx_last_scores is not filled (the debug hooks describe
 * fp32 scans). */
#define MARS_CTX_CERTIFIED   0x8u
/* create_query_context(max_nodes, embedding_dim, max_k): max_k clamps to 64. A query
 * returns at most min(max_nodes, max_k * 500) results, the reference's compaction cap
 * (max_compact, memory_cuda.cu:1059): 32,000 at the default max_k of 64. */
int mars_ctx_create(int32_t max_nodes, int32_t embedding_dim, int32_t max_k,
                    uint32_t flags, mars_ctx** out);
int mars_ctx_destroy(mars_ctx* ctx);
int mars_ctx_set_flags(mars_ctx* ctx, uint32_t flags);
int mars_ctx_get_flags(const mars_ctx* ctx, uint32_t* flags);
/* QueryContext::stream (memory_cuda.cuh:178): the context's own stream, a hipStream_t
 * passed as void*, on which every kernel of its queries runs. Work the caller enqueues
 * there is ordered with those queries. */
int mars_ctx_get_stream(const mars_ctx* ctx, void** stream);

/* query_memory_fast: one query from a host vector (embedding_dim floats).
 * Writes min(cap, n) results sorted by (score desc, node_id asc) and sets
 * *n_out = n, the number of results the query produced: min(max_results_returned
 * (K when <= 0), nodes visited, the context's result cap); n <= cap is the caller's
 * check. stats may be NULL. With MARS_CTX_TIMING the stage timers follow the
 * reference's split (memory_cuda.cu:1450-1454): gpu_ms_similarity = the scan (dot,
 * decay and per-wave top-K are one kernel), gpu_ms_rerank = 0 (the decay is fused into
 * the scan), gpu_ms_topk = the seed merge, gpu_ms_bfs = the BFS and the sorted results,
 * gpu_ms_total = all of them. */
int mars_query(const mars_graph* g, mars_ctx* ctx, const float* h_query, float t_q,
               const mars_retrieval_config* cfg, mars_query_result* out, int32_t cap,
               int32_t* n_out, mars_stats* stats);
/* Same, with the query vector already in device memory (d_query: embedding_dim floats). */
int mars_query_device(const mars_graph* g, mars_ctx* ctx, const float* d_query, float t_q,
                      const mars_retrieval_config* cfg, mars_query_result* out,
                      int32_t cap, int32_t* n_out, mars_stats* stats);

/* Batched global scoring: Q query vectors in device memory (row-major Q x embedding_dim
 * fp32), query i at time t_q[i] (host array), decay / modality filter from cfg, top-K
 * (cfg->top_k <= 16) per query over the fp16 corpus (mars_graph_enable_fp16) on MFMA
 * fp16 tiles with fp32 accumulation. No BFS, no episode scope: each row of the
 * output is the seed list the Q=1 global path would select (scores within the fp16
 * tolerance). out_ids / out_scores: host, Q x top_k, each row sorted (score desc,
 * id asc). Reference analogue: none (wmma_similarity.cu:55-138 scores one query). */
int mars_query_batch(const mars_graph* g, mars_ctx* ctx, const float* d_queries, int32_t Q,
                     const float* t_q, const mars_retrieval_config* cfg, int32_t* out_ids,
                     float* out_scores, mars_stats* stats);
/* mars_query_batch without allocation. No counterpart in the reference: for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops). The
 * same kernels and results as mars_query_batch, with their scratch in a static device
 * array of the library (about 8.4 MiB, held per GPU until the process ends): Q <= 256
 * queries (MARS_ERR_CAPACITY beyond), top_k <= 16, embedding_dim 256 / 384 / 512 / 768.
 * Inputs and outputs are device memory: d_queries Q x embedding_dim fp32, d_tq Q query
 * times (uniform_tq != 0 promises they are all equal: one decay weight per row), d_ids /
 * d_scores Q x top_k, each row sorted (score desc, id asc), -1 / -FLT_MAX past the rows
 * that exist. Runs on `stream` (a hipStream_t; NULL = the null stream) and returns
 * without waiting; the results are there once the stream reaches that point. Calls that
 * overlap on one GPU share the array and race: order them on one stream. */
int mars_query_batch_static(const mars_graph* g, const float* d_queries, int32_t Q, const float* d_tq,
                            int32_t uniform_tq, const mars_retrieval_config* cfg, int32_t* d_ids,
                            float* d_scores, void* stream);

/* Batched global queries: Q global queries (the same cfg, query i at time t_q[i], a host
 * array; query vectors in device memory, row-major Q x embedding_dim fp32). Query i gets
 * exactly the results mars_query_device gives it with this context (same ids, scores,
 * hops and order; cap and n_out[i] as there), written to out + i * cap.
 * One fp16 MFMA scan of the corpus (mars_graph_enable_fp16) serves the whole batch: it
 * keeps 16 candidates per query, which are rescored in the Q=1 path's arithmetic and
 * certified against the fp16 error bound; certified queries then run their BFS together
 * (one workgroup each). A query whose seeds miss the certificate, or whose visit set
 * outgrows the batched BFS table (7168 nodes), is answered by the Q=1 path, as is the
 * whole batch when cfg is episode-scoped (and active), K > 16, time_decay_lambda < 0,
 * a same-episode boost applies, or the fp16 copy is absent. The node count is read once
 * per call. stats may be NULL. Reference analogue: none (query_memory_fast,
 * memory_cuda.cu:1351-1464, answers one query per call). */
typedef struct mars_batch_stats {
    int32_t queries;            /* Q                                                      */
    int32_t batched;            /* answered by the shared scan and the batched BFS        */
    int32_t uncertified;        /* seeds not certified: answered by the Q=1 path          */
    int32_t overflow;           /* visit set beyond the batched table: Q=1 path           */
    int32_t whole_batch_q1;     /* 1 if the configuration sent every query to the Q=1 path */
    int32_t n_live;             /* nodes the batch was answered over                       */
    float   gpu_ms_scan;        /* MARS_CTX_TIMING: shared fp16 scan + candidate merge     */
    float   gpu_ms_seeds;       /* exact rescoring of the candidates + certificate        */
    float   gpu_ms_bfs;         /* BFS, visit scores and results                          */
    float   gpu_ms_total;
    float   min_margin;         /* smallest certificate margin of a certified query        */
    int32_t candidate_rows;     /* rows the shared scan read: 8 = the int8 copy (up to 16 queries
                                   and neighbour searches per pass, certified exact candidates),
                                   16 = the fp16 MFMA scan, 24 = int8, then fp16 again for the
                                   neighbour searches the int8 certificate did not cover     */
    double  wall_us;            /* host wall time of the call (Q=1 answers included)      */
    double  q1_us;              /* of which Q=1 answers                                   */
} mars_batch_stats;
int mars_query_global_batch(const mars_graph* g, mars_ctx* ctx, const float* d_queries, int32_t Q,
                            const float* t_q, const mars_retrieval_config* cfg,
                            mars_query_result* out, int32_t cap, int32_t* n_out,
                            mars_batch_stats* stats);
/* The same, with the neighbour search of knn_count published nodes knn_first ..
 * knn_first + knn_count - 1 done in the same corpus pass: out_knn (host, knn_count x
 * knn_k, -1 padded) receives each node's knn_k nearest neighbours among the nodes
 * published when the call starts, as mars_graph_link_knn finds them; pass them to
 * mars_graph_link. Q may be 0 (neighbour search only). A streaming server links the
 * nodes it inserted with knn_k = 0 this way, one corpus pass serving both. */
int mars_query_global_batch_knn(const mars_graph* g, mars_ctx* ctx, const float* d_queries, int32_t Q,
                                const float* t_q, const mars_retrieval_config* cfg,
                                mars_query_result* out, int32_t cap, int32_t* n_out,
                                mars_batch_stats* stats, int32_t knn_first, int32_t knn_count,
                                int32_t knn_k, int32_t* out_knn);

/* Debug / parity hooks: copy the last query's per-node fp32 scores (N floats) and
 * its seed list (top-K ids and scores, K entries) to host memory. */
int mars_ctx_last_scores(mars_ctx* ctx, float* h_scores, int64_t n);
int mars_ctx_last_seeds(mars_ctx* ctx, int32_t* h_idx, float* h_val, int32_t k, int32_t* k_out);
/* Durations (us) of the last global query's phases after the scan, from the GPU's
 * 100 MHz realtime counter. fp32 path (n <= 3): seed merge, BFS, result selection.
 * Certified path (n <= 6): candidate merge, exact rescoring + certificate, interval
 * BFS, candidate marking, exact rescoring of the marked nodes, results. */
int mars_ctx_last_phases(mars_ctx* ctx, double* us, int32_t n);
/* The last global query's visit list in discovery order (seeds first, then BFS
 * level by level): node ids, hop levels and BFS scores; *n_out = nodes visited. */
int mars_ctx_last_visited(mars_ctx* ctx, int32_t* h_ids, int32_t* h_hops, float* h_scores,
                          int32_t cap, int32_t* n_out);

/* ---- NSN edges (host) -------------------------------------------------------------------
 * MemoryGraph::build_nsn_edges_configurable (memory_graph.cpp:102-189): the same graph,
 * edge for edge, as the reference built with the same C++ standard library (one
 * std::mt19937 seeded 7, the same draws in the same order). phases: the NSNConfig
 * enables as bits (MARS_NSN_ALL = the defaults). modalities (0..2) are needed for the
 * bridges. Call with col == NULL for an upper bound of the edge count in *num_edges;
 * then with col_cap >= that bound: row_offsets (n + 1) and col (rows ascending) are
 * written and *num_edges is the count. */
#define MARS_NSN_RING     0x1u
#define MARS_NSN_SKIPS    0x2u
#define MARS_NSN_HUBS     0x4u
#define MARS_NSN_REWIRE   0x8u
#define MARS_NSN_BRIDGES  0x10u
#define MARS_NSN_ALL      0x1Fu
int mars_nsn_edges(int32_t n, const int32_t* modalities, int32_t k, double p, uint32_t phases,
                   int32_t* row_offsets, int32_t* col, int64_t col_cap, int64_t* num_edges);

/* ---- importance, novelty gate, graph maintenance --------------------------------------
 * The reference's adjacent features (memory_cuda.cuh:234-270, memory_cuda.cu:1466-1658),
 * kept on the device graph. Each call is synchronous and serialised with inserts. */

/* init_importance (memory_cuda.cuh:240): every node's importance becomes 1.0; nodes
 * inserted later start at 1.0 too. Allocates capacity_nodes floats on first use. */
int mars_importance_init(mars_graph* g);
/* update_importance (memory_cuda.cuh:246-249): importance[i] *= 1 - decay_rate for every
 * node, then importance[id] = min(importance[id] + boost, max_importance) for each
 * listed id, in fp32 operation by operation as the reference. Ids < 0 or >= the node
 * count are skipped; an id listed twice is boosted twice (the reference races there).
 * ids: host memory, or device memory when ids_on_device != 0. */
int mars_importance_update(mars_graph* g, const int32_t* ids, int32_t n_ids, int32_t ids_on_device,
                           float boost, float decay_rate, float max_importance);
int mars_importance_read(const mars_graph* g, float* h_out, int32_t first, int32_t count);
/* compute_novelty (memory_cuda.cuh:256-257): max over the nodes of <E_i, q>, at least -1,
 * and 0 for an empty graph. The query is h_q (host) or d_q (device). ctx may be NULL:
 * the graph's own context (certified fp16 scan, created on first use) answers; with a
 * ctx, this is that context's last query. */
int mars_novelty(const mars_graph* g, mars_ctx* ctx, const float* h_q, const float* d_q, float* max_sim);
/* init_edge_hits (memory_cuda.cuh:261): one zeroed counter per edge. Counters follow
 * their edges through inserts; mars_graph_set_csr zeroes them. */
int mars_edge_hits_init(mars_graph* g);
/* count_edge_hits_kernel (memory_cuda.cu:1612-1632; the reference has no host call for
 * it): for the BFS of ctx's last global single query, +1 on every edge (v, u) with
 * hop(v) >= 1 and hop(u) = hop(v) - 1. No-op after an episode-scoped query or a batch. */
int mars_edge_hits_count(mars_graph* g, mars_ctx* ctx);
/* The counters in the order of the graph's CSR (mars_graph_download's col array).
 * *n_out = edge count; nothing is copied when cap is smaller. */
int mars_edge_hits_read(const mars_graph* g, int32_t* h_hits, int64_t cap, int64_t* n_out);
/* maintain_graph (memory_cuda.cuh:268-270): *low_utility = edges with hits <= min_hits,
 * then every counter is reset to 0. window_queries is unused, as in the reference. */
int mars_graph_maintain(mars_graph* g, int32_t min_hits, int32_t window_queries, int32_t* low_utility);

/* ---- device memory helpers ----------------------------------------------------------
 * Device buffers for callers that hold no HIP runtime of their own (e.g. the ctypes
 * benchmark; a second HIP runtime in the same process, such as the one bundled with
 * a Python framework, must not be mixed with this library's). */
int mars_device_alloc(size_t bytes, void** ptr);
int mars_device_free(void* ptr);
int mars_copy_to_device(void* dst, const void* src, size_t bytes);
int mars_copy_to_host(void* dst, const void* src, size_t bytes);
int mars_copy_device(void* dst, const void* src, size_t bytes);   /* device to device */
int mars_device_memory(size_t* free_bytes, size_t* total_bytes);  /* hipMemGetInfo of the device */
int mars_device_synchronize(void);   /* hipDeviceSynchronize: all streams of the device drained */

/* ---- benchmark loop (harness semantics of src/latency_bench.cu:355-393) ------------ */
/* Runs n single queries back to back, query i reading the device vector
 * d_queries + i*stride with configuration cfgs[n_cfg == 1 ? 0 : i]. lat_us[i]
 * receives the host wall latency of the whole call (steady_clock, measured here,
 * not through any binding layer); with MARS_CTX_TIMING set, kern_us[i] (may be NULL)
 * receives the GPU time of the scan / episode kernel and bfs_us[i] (may be NULL)
 * the GPU time after it (seeds, BFS and results). n_res[i] (may be NULL) gets the
 * result count. */
int mars_bench_queries(const mars_graph* g, mars_ctx* ctx, const float* d_queries, int64_t stride,
                       int32_t n, float t_q, const mars_retrieval_config* cfgs, int32_t n_cfg,
                       double* lat_us, float* kern_us, float* bfs_us, int32_t* n_res);
/* The same loop over host query vectors h_queries + i*stride: each call copies its
 * vector to the device as query_memory_fast does (memory_cuda.cu:1365-1368), and
 * lat_us[i] includes that copy. */
int mars_bench_queries_host(const mars_graph* g, mars_ctx* ctx, const float* h_queries, int64_t stride,
                            int32_t n, float t_q, const mars_retrieval_config* cfgs, int32_t n_cfg,
                            double* lat_us, int32_t* n_res);

/* Streaming workload driver (no reference counterpart; the streaming benchmark
 * configuration): on one thread, n_queries single queries paced at query_rate per
 * second (query i starts at i / query_rate s, or when the previous one returns);
 * on a second thread, n_insert host rows inserted with mars_graph_insert in
 * batches of insert_batch nodes paced at insert_rate nodes per second. Both start
 * together. query_lat_us[i] = wall latency of query i (inside the library);
 * query_start_us[i] = its start since the run began; ins_stats[j] / ins_start_us[j]
 * for insert batch j (ceil(n_insert / insert_batch) batches). */
typedef struct mars_stream_bench {
    const float*                 d_queries;      /* device, n_queries * stride floats   */
    int64_t                      stride;
    int32_t                      n_queries;
    float                        t_q;
    const mars_retrieval_config* cfgs;           /* n_queries configurations            */
    double                       query_rate;     /* queries per second                  */
    const float*                 ins_emb;        /* host, n_insert * embedding_dim      */
    const int32_t*               ins_mods;
    const float*                 ins_ts;
    const int32_t*               ins_ep;         /* NULL if the graph has no episode ids */
    int32_t                      n_insert;
    int32_t                      insert_batch;
    double                       insert_rate;    /* nodes per second                    */
    int32_t                      knn_k;
    double*                      query_lat_us;
    double*                      query_start_us;
    mars_insert_stats*           ins_stats;
    double*                      ins_start_us;
} mars_stream_bench;
int mars_bench_stream(mars_graph* g, mars_ctx* ctx, mars_stream_bench* bench);

/* Serving workload driver (no reference counterpart): three threads start together.
 *  - episode-scoped queries: query i (device vector e_queries + i * embedding_dim,
 *    configuration ecfgs[i]) arrives at e_arrival_us[i] after the start and is answered
 *    on ctx_episode as soon as it has arrived and the one before it is done;
 *  - global queries: query i (g_queries + i * embedding_dim, configuration gcfg) arrives
 *    at g_arrival_us[i]; whenever global queries wait, all that have arrived (at most
 *    max_batch) are answered by one mars_query_global_batch call on ctx_global
 *    (max_batch = 1: one mars_query_device per query);
 *  - inserts: n_insert host rows inserted with mars_graph_insert in batches of
 *    insert_batch nodes paced at insert_rate nodes per second. With link_deferred = 0
 *    each insert finds its nodes' knn_k neighbours itself; with link_deferred = 1 the
 *    inserts pass knn_k = 0 (queryable at once) and the global server links every
 *    published, unlinked node (at most max_link per call) in its next batched call
 *    (mars_query_global_batch_knn + mars_graph_link: one corpus pass for both), or
 *    in a call of its own once the oldest unlinked insert has waited link_wait_us.
 * All queries use query time t_q. g_done_us[i] / e_done_us[i] = when query i's results
 * were in host memory (since the start), so done - arrival is its latency including
 * the wait; g_batch[i] = size of the call that answered global query i;
 * ins_stats[j] / ins_start_us[j] as in mars_bench_stream; ins_linked_us[j] = when the
 * k-NN edges of insert j were visible (since the start). */
typedef struct mars_serve_bench {
    float                        t_q;
    int32_t                      max_batch;
    const float*                 g_queries;      /* device, n_global * embedding_dim     */
    int32_t                      n_global;
    int32_t                      pad0;
    const double*                g_arrival_us;
    const mars_retrieval_config* gcfg;
    const float*                 e_queries;      /* device, n_episode * embedding_dim    */
    int32_t                      n_episode;
    int32_t                      pad1;
    const double*                e_arrival_us;
    const mars_retrieval_config* ecfgs;          /* n_episode configurations             */
    const float*                 ins_emb;        /* host, n_insert * embedding_dim       */
    const int32_t*               ins_mods;
    const float*                 ins_ts;
    const int32_t*               ins_ep;         /* NULL if the graph has no episode ids  */
    int32_t                      n_insert;
    int32_t                      insert_batch;
    double                       insert_rate;    /* nodes per second                     */
    int32_t                      knn_k;
    int32_t                      pad2;
    double*                      g_done_us;
    int32_t*                     g_batch;
    double*                      e_done_us;
    mars_insert_stats*           ins_stats;
    double*                      ins_start_us;
    int64_t                      g_uncertified;  /* out: global queries the batch sent to the Q=1 path */
    int64_t                      g_overflow;     /* out: of which for a visit overflow   */
    int32_t                      link_deferred;
    int32_t                      max_link;
    double*                      ins_linked_us;
    double                       link_wait_us;
    int64_t                      link_calls;     /* out: server calls that linked nodes  */
} mars_serve_bench;
int mars_bench_serve(mars_graph* g, mars_ctx* ctx_global, mars_ctx* ctx_episode, mars_serve_bench* bench);

#ifdef __cplusplus
}
#endif
#endif /* MARS_AMD_H */
