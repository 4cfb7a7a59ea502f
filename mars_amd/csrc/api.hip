// ============================================================================
//  api.hip — C ABI of libmars_amd: graph residency, query contexts and the
//  query pipeline (declared in include/mars_amd.h).
//
//  Global query:   [H2D q] -> k_scan (fused score + per-workgroup top-K)
//                          -> k_finalize (seeds, BFS, sorted results -> pinned host)
//  Episode query:  [H2D q] -> k_episode (member range only -> pinned host)
//  One stream synchronisation per query and no device->host copy: the last
//  kernel writes the result records into mapped pinned memory.
// ============================================================================
#include "internal.hpp"
#include "formats.hpp"

#include <algorithm>
#include <atomic>
#include <cfloat>
#include <chrono>
#include <cstddef>
#include <cstdarg>
#include <cstring>
#include <deque>
#include <mutex>
#include <string>
#include <thread>
#include <vector>


namespace mars {

namespace {
thread_local char g_err[1024] = "";
constexpr int32_t kMaxWg = 4096;     // upper bound of scan workgroups (partials buffer)
// Scan workgroups (grid-stride), 2 per CU on 256 CUs. A count that is not a whole
// multiple of the CU count loads the CUs unevenly (1M x 768 fp16 rows: 235 us at
// 512, 246 us at 768, 270 us at 256, 255 us at 576; fp32 rows: 472 us at 512,
// 510 us at 2048).
constexpr int32_t kTargetWg = 512;
constexpr int32_t kTargetWgF16 = 512;
constexpr int32_t kTargetWgI8 = kScan8MaxLists;


int ensure_device(int* dev) {
    int d = 0;
    MARS_HIP(hipGetDevice(&d));
    hipDeviceProp_t prop;
    MARS_HIP(hipGetDeviceProperties(&prop, d));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return set_error(MARS_ERR_NODEVICE, "device %d is %s, this build targets gfx950 only", d,
                         prop.gcnArchName);
    if (dev) *dev = d;
    return MARS_OK;
}

// CSR checks done on host input: offsets start at 0, non-decreasing, end at E;
// neighbour ids in range; no id twice in one row (the BFS claim relies on it).
int validate_csr(int32_t n, int32_t e, const int32_t* row, const int32_t* col) {
    if (e == 0 && row == nullptr) return MARS_OK;
    MARS_CHECK(row != nullptr && (e == 0 || col != nullptr), MARS_ERR_INVALID,
               "row_offsets/col_indices missing");
    MARS_CHECK(row[0] == 0, MARS_ERR_INVALID, "row_offsets[0] = %d, expected 0", row[0]);
    MARS_CHECK(row[n] == e, MARS_ERR_INVALID, "row_offsets[N] = %d, expected num_edges %d", row[n], e);
    std::vector<int32_t> tmp;
    for (int32_t i = 0; i < n; ++i) {
        const int32_t b = row[i], t = row[i + 1];
        MARS_CHECK(b <= t, MARS_ERR_INVALID, "row_offsets decrease at row %d", i);
        bool ascending = true;
        for (int32_t j = b; j < t; ++j) {
            MARS_CHECK(col[j] >= 0 && col[j] < n, MARS_ERR_INVALID, "col_indices[%d] = %d out of range", j,
                       col[j]);
            if (j > b && col[j] <= col[j - 1]) ascending = false;
        }
        if (!ascending) {
            tmp.assign(col + b, col + t);
            std::sort(tmp.begin(), tmp.end());
            MARS_CHECK(std::adjacent_find(tmp.begin(), tmp.end()) == tmp.end(), MARS_ERR_INVALID,
                       "row %d lists a neighbour twice", i);
        }
    }
    return MARS_OK;
}

bool episode_scoped_active(const Graph& g, const mars_retrieval_config& c) {
    // memory_cuda.cu:1163-1171
    // (episode count and member total grow under streaming inserts: read once each)
    return c.retrieval_scope == MARS_SCOPE_EPISODE_SCOPED && g.ep_off != nullptr && g.ep_mem != nullptr &&
           c.query_episode_id >= 0 && c.query_episode_id < __atomic_load_n(&g.num_eps, __ATOMIC_ACQUIRE) &&
           c.query_episode_member_count > 0 && c.query_episode_member_begin >= 0 &&
           int64_t(c.query_episode_member_begin) + c.query_episode_member_count <=
               __atomic_load_n(&g.member_total, __ATOMIC_ACQUIRE);
}

}  // namespace

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

namespace {

int graph_free(Graph& g) {
    (void)use_device(g.device);
    if (g.ins_stream) (void)hipStreamSynchronize(g.ins_stream);
    dfree(g.emb); dfree(g.emb16); dfree(g.nrm); dfree(g.emb8); dfree(g.meta8); dfree(g.nrm8); dfree(g.mods); dfree(g.ts); dfree(g.ro); dfree(g.rcap); dfree(g.col);
    dfree(g.ep_ids); dfree(g.ep_off); dfree(g.ep_mem);
    dfree(g.imp); dfree(g.hits); dfree(g.imp_ids); dfree(g.sweep_cnt); dfree(g.pk_row); dfree(g.pk_col);
    graph_insert_free(g);
    if (g.ins_stream) (void)hipStreamDestroy(g.ins_stream);
    g = Graph{};
    return MARS_OK;
}

// Row words from a host CSR (rows packed back to back, no slack) and their upload.
int load_csr(Graph& g, int32_t n, int32_t e, const int32_t* row, const int32_t* col, hipMemcpyKind kind) {
    g.ro_h.assign(size_t(g.cap_n), 0);
    g.rcap_h.assign(size_t(g.cap_n), 0);
    std::vector<int32_t> hrow;
    const int32_t* r = row;
    if (row && kind == hipMemcpyDeviceToDevice) {
        hrow.resize(size_t(n) + 1);
        MARS_HIP(hipMemcpy(hrow.data(), row, hrow.size() * sizeof(int32_t), hipMemcpyDeviceToHost));
        r = hrow.data();
    }
    g.max_deg = 0;
    for (int32_t i = 0; i < n; ++i) {
        const int32_t b = r ? r[i] : 0, len = r ? r[i + 1] - r[i] : 0;
        g.ro_h[size_t(i)] = (int64_t(len) << 32) | uint32_t(b);
        g.rcap_h[size_t(i)] = len;
        g.max_deg = std::max(g.max_deg, len);
    }
    MARS_HIP(hipMemcpy(g.ro, g.ro_h.data(), size_t(g.cap_n) * sizeof(int64_t), hipMemcpyHostToDevice));
    MARS_HIP(hipMemcpy(g.rcap, g.rcap_h.data(), size_t(g.cap_n) * sizeof(int32_t), hipMemcpyHostToDevice));
    if (e > 0) MARS_HIP(hipMemcpy(g.col, col, size_t(e) * sizeof(int32_t), kind));
    g.e = e;
    g.e_used = e;
    ++g.csr_version;
    return MARS_OK;
}

// Packed CSR export: row i's live slots col[start, start + len) copied to
// out[off[i], off[i + 1]), 16 lanes per row (one DPP row group), grid-stride.
__global__ __launch_bounds__(256) void k_pack_csr(const int64_t* __restrict__ ro, const int32_t* __restrict__ col,
                                                  const int32_t* __restrict__ off, int32_t* __restrict__ out,
                                                  int32_t n) {
    const int sub = int(threadIdx.x & 15u);
    const int64_t groups = int64_t(gridDim.x) * (blockDim.x / 16);
    for (int64_t i = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) / 16; i < n; i += groups) {
        const int64_t w = ro[i];
        const int32_t b = int32_t(uint32_t(w)), len = int32_t(w >> 32);
        const int32_t o = off[i];
        for (int32_t j = sub; j < len; j += 16) out[o + j] = col[b + j];
    }
}

void graph_slot_free(Ctx::GraphSlot& g);

// Default col room for streaming inserts: 256 slots per node of spare capacity (a new
// row, and the old rows it links to when they move to the tail).
int64_t edge_room(const Graph& g) {
    return int64_t(g.cap_n - g.n) * 256 + (g.cap_n > g.n ? 4096 : 0);
}

void multi_free(Ctx& c) {
    dfree(c.mknn);
    c.mknn_cap = 0;
    dfree(c.m8part); dfree(c.m8qa); dfree(c.m8qp);
    dfree(c.mqn); dfree(c.mseed); dfree(c.mstat); dfree(c.minfo); dfree(c.mmargin);
    dfree(c.mvlist); dfree(c.mvhop); dfree(c.mvpar); dfree(c.mvro); dfree(c.mvfin); dfree(c.mvscore);
    c.mcap_q = 0;
    if (c.h_mres) (void)hipHostFree(c.h_mres);
    c.h_mres = nullptr;
    c.d_mres = nullptr;
    c.mres_bytes = 0;
}

int ctx_free(Ctx& c) {
    (void)use_device(c.device);
    if (c.stream) (void)hipStreamSynchronize(c.stream);
    dfree(c.query); dfree(c.fin); dfree(c.part); dfree(c.vis); dfree(c.claim); dfree(c.vlist);
    dfree(c.vhop); dfree(c.vscore); dfree(c.vro); dfree(c.sortbuf); dfree(c.seed_idx); dfree(c.seed_val);
    dfree(c.gthr); dfree(c.gcnt); dfree(c.hopmap);
    dfree(c.bq); dfree(c.btq); dfree(c.bpart); dfree(c.bout);
    multi_free(c);
    if (c.h_query) (void)hipHostFree(c.h_query);
    if (c.h_res) (void)hipHostFree(c.h_res);
    if (c.h_done) (void)hipHostFree(c.h_done);
    if (c.h_stamps) (void)hipHostFree(c.h_stamps);
    for (auto& e : c.ev) if (e) (void)hipEventDestroy(e);
    graph_slot_free(c.g_global);
    graph_slot_free(c.g_episode);
    if (c.stream) (void)hipStreamDestroy(c.stream);
    c = Ctx{};
    return MARS_OK;
}

void graph_slot_free(Ctx::GraphSlot& g) {
    if (g.exec) (void)hipGraphExecDestroy(g.exec);
    if (g.graph) (void)hipGraphDestroy(g.graph);
    g = Ctx::GraphSlot{};
}

// Launch 1 or 2 dependent kernels as a replayed graph: the graph is built once per
// (kernel, grid) shape and each query only rewrites the kernel-node arguments, so no
// per-query value (query time, epoch, ...) is frozen into it.
int graph_launch(Ctx::GraphSlot& g, int n, const KernelLaunch* l, void* const* args, hipStream_t s) {
    hipKernelNodeParams p[2];
    for (int i = 0; i < n; ++i) {
        p[i] = hipKernelNodeParams{};
        p[i].func = const_cast<void*>(l[i].fn);
        p[i].gridDim = l[i].grid;
        p[i].blockDim = l[i].block;
        p[i].sharedMemBytes = 0;
        p[i].kernelParams = const_cast<void**>(&args[i]);
        p[i].extra = nullptr;
    }
    const bool same = g.exec && g.fn[0] == l[0].fn && (n < 2 || g.fn[1] == l[1].fn) && g.grid0 == l[0].grid.x;
    if (!same) {
        graph_slot_free(g);
        MARS_HIP(hipGraphCreate(&g.graph, 0));
        for (int i = 0; i < n; ++i)
            MARS_HIP(hipGraphAddKernelNode(&g.node[i], g.graph, i ? &g.node[i - 1] : nullptr, i ? 1 : 0, &p[i]));
        MARS_HIP(hipGraphInstantiate(&g.exec, g.graph, nullptr, nullptr, 0));
        for (int i = 0; i < n; ++i) g.fn[i] = l[i].fn;
        g.grid0 = l[0].grid.x;
    } else {
        for (int i = 0; i < n; ++i) MARS_HIP(hipGraphExecKernelNodeSetParams(g.exec, g.node[i], &p[i]));
    }
    MARS_HIP(hipGraphLaunch(g.exec, s));
    return MARS_OK;
}

int ensure_multi_scratch(Ctx& c, int32_t q, int32_t rcap);

// Next sequence number of a Q=1 query (never 0, the word's initial value).
uint32_t next_seq(Ctx& c) {
    if (++c.seq == 0u) c.seq = 1u;
    return c.seq;
}

// Waits for the Q=1 query whose last kernel stores seq into the completion word after
// its results. The host spins on the word; every 50 us it also asks the stream, so a
// failed launch or a fault is reported, and a stream that finished without storing the
// word ends the wait as well (the results are then complete).
int wait_done(const Ctx& c, uint32_t seq, hipStream_t s) {
    using clk = std::chrono::steady_clock;
    auto next = clk::now() + std::chrono::microseconds(50);
    while (__atomic_load_n(c.h_done, __ATOMIC_ACQUIRE) != seq) {
        __builtin_ia32_pause();
        const auto now = clk::now();
        if (now < next) continue;
        const hipError_t e = hipStreamQuery(s);
        if (e == hipSuccess) break;
        if (e != hipErrorNotReady) return set_error(MARS_ERR_HIP, "query stream: %s", hipGetErrorString(e));
        next = now + std::chrono::microseconds(50);
    }
    return MARS_OK;
}

// Certified global query (MARS_CTX_CERTIFIED): a candidate scan of the int8 copy (64
// candidates ranked by per-row upper bounds) or of the fp16 copy (c candidates ranked by
// fp16 scores), exact rescoring + certificate, then the unscored BFS, exact visit scores
// and the results (the batched path's kernels with q = 1). *answered = false when the
// certificate or the BFS table did not hold: the caller runs the fp32 scan.
int certified_query(const Graph& g, Ctx& c, const float* q, float t_q, const mars_retrieval_config* cfg, int32_t K,
                    int32_t hops, int32_t rcap, int32_t n_live, mars_query_result* out, int32_t cap, int32_t* n_out,
                    bool* answered, ResultHeader* hdr_out) {
    *answered = false;
    MARS_TRY(ensure_multi_scratch(c, 1, rcap));
    hipStream_t s = c.stream;
    const bool timing = (c.flags & MARS_CTX_TIMING) != 0;
    const bool i8 = cert_uses_int8(g);
    // candidates the certificate checks
    const int32_t cands = i8 ? 64 : (K <= 10 ? 16 : (K <= 16 ? 32 : 64));
    int32_t rpw = 0, nwg = 0;
    scan_grid(n_live, i8 ? kTargetWgI8 : kTargetWgF16, &rpw, &nwg);
    ScanArgs a{};
    a.emb = i8 ? static_cast<const void*>(g.emb8) : static_cast<const void*>(g.emb16); a.fp16 = i8 ? 0 : 1;
    a.meta8 = g.meta8; a.nrm8 = g.nrm8; a.n = n_live; a.d = g.d; a.q = q; a.ts = g.ts; a.mods = g.mods; a.ep_ids = g.ep_ids;
    a.t_q = t_q; a.lambda = cfg->time_decay_lambda; a.mod_filter = cfg->modality_filter; a.query_ep = -1;
    a.boost = 0.0f; a.k = i8 ? kScan8List : cands; a.fin = c.fin; a.part = c.part; a.gthr = c.gthr;
    a.gcnt = c.gcnt; a.rows_per_wg = rpw; a.num_wg = nwg;
    if (timing) MARS_HIP(hipEventRecord(c.ev[0], s));
    MARS_TRY(i8 ? launch_scan8(a, s) : launch_scan(a, s));
    if (timing) MARS_HIP(hipEventRecord(c.ev[1], s));
    CertArgs ca{};
    ca.part = c.part; ca.gcnt = c.gcnt; ca.gthr = c.gthr; ca.c = cands; ca.k = K; ca.q = q; ca.d = g.d;
    ca.n_lists = i8 ? nwg : 0;
    ca.emb = g.emb; ca.ts = g.ts; ca.mods = g.mods; ca.t_q = t_q; ca.lambda = cfg->time_decay_lambda;
    ca.mod_filter = cfg->modality_filter; ca.nrm = g.nrm; ca.upper = i8 ? 1 : 0; ca.nrm8 = g.nrm8;
    ca.seeds = c.mseed; ca.status = c.mstat;
    ca.margin = c.mmargin; ca.fin16 = c.fin; ca.stamps = c.stamps + 4;
    // one workgroup finishes the query when the interval argument applies
    const float dlt = cfg->bfs_score_decay;
    ca.finish = (rcap <= 64 && dlt >= 0.0f && dlt <= 1.0f) ? 1 : 0;
    // the last kernel (k_cert_bfs, else k_multi_select) stores the completion word
    const uint32_t seq = next_seq(c);
    uint32_t* const done = timing ? nullptr : c.d_done;
    ca.done = ca.finish ? done : nullptr;
    ca.seq = seq;
    MultiArgs m{};
    m.ro = g.ro; m.col = g.col; m.mods = g.mods; m.n_live = n_live; m.hops = hops;
    m.hop_decay = cfg->bfs_score_decay; m.k = K; m.rcap = rcap; m.q = 1; m.seeds = c.mseed; m.seed_stride = 64;
    m.status = c.mstat; m.info = c.minfo; m.vlist = c.mvlist; m.vhop = c.mvhop; m.vpar = c.mvpar;
    m.vro = c.mvro; m.vfin = c.mvfin; m.vscore = c.mvscore;
    m.res = static_cast<ResultHeader*>(c.d_mres);
    m.rec = reinterpret_cast<mars_query_result*>(m.res + 1);
    m.done = ca.finish ? nullptr : done;
    m.seq = seq;
    if (launch_cert_bfs(ca, m, s) != MARS_OK) {
        // the scan appended candidates: clear them for the next query
        (void)hipMemsetAsync(c.gcnt, 0, sizeof(uint32_t), s);
        (void)hipMemsetAsync(c.gthr, 0xFF, sizeof(uint64_t), s);
        (void)hipStreamSynchronize(s);
        return set_error(MARS_ERR_HIP, "certificate launch failed");
    }
    if (!ca.finish) {
        VisitScoreArgs va{};
        va.emb = g.emb; va.fp16 = 0; va.d = g.d; va.ts = g.ts; va.mods = g.mods; va.queries = q;
        va.tq = nullptr; va.lambda = cfg->time_decay_lambda; va.mod_filter = cfg->modality_filter; va.q = 1;
        va.status = c.mstat; va.info = c.minfo; va.vlist = c.mvlist; va.vfin = c.mvfin;
        va.t_q_value = t_q;
        MARS_TRY(launch_visit_scores(va, s));
        MARS_TRY(launch_multi_select(m, s));
    }
    if (timing) {
        MARS_HIP(hipEventRecord(c.ev[2], s));
        MARS_HIP(hipStreamSynchronize(s));
    } else {
        MARS_TRY(wait_done(c, seq, s));
    }
    const auto* hdr = static_cast<const ResultHeader*>(c.h_mres);
    const ResultHeader h = hdr[0];
    if (h.count < 0) return MARS_OK;
    const int32_t nw = std::min(h.count, cap);
    if (nw > 0) std::memcpy(out, hdr + 1, size_t(nw) * sizeof(mars_query_result));
    *n_out = h.count;
    *hdr_out = h;
    *answered = true;
    return MARS_OK;
}

int global_batch_impl(const mars_graph* gh, mars_ctx* ch, const float* dq, int32_t Q, const float* h_tq,
                      const mars_retrieval_config* cfg, mars_query_result* out, int32_t cap, int32_t* n_out,
                      mars_batch_stats* stats, int32_t knn_first, int32_t knn_count, int32_t knn_k, int32_t* out_knn,
                      bool allow_int8, bool q1_route = false);

// A lone certified query over an int8 copy of at least this many rows takes the multi-query
// int8 pass (k_split8, k_scan8m, k_cert_multi8) and the batched BFS: its scan streams the
// copy faster than k_scan8 (the query split done once, no per-row estimate stores: 1.455
// against 1.596 ms at 13M rows), which outweighs the longer chain after it (about 8 us more
// at 1M rows, where k_scan8 and the one-kernel interval BFS stay ahead). Same results.
constexpr int32_t kCertRouteRows = 2000000;

// n_pin >= 0: answer over the first n_pin nodes (a batch that already read the node
// count), else over the nodes published when the query starts. allow_route = false keeps a
// certified query off the multi-query int8 pass (that pass's own fallback).
int query_impl(const mars_graph* gh, mars_ctx* ch, const float* h_q, const float* d_q, float t_q,
               const mars_retrieval_config* cfg, mars_query_result* out, int32_t cap, int32_t* n_out,
               mars_stats* stats, int32_t n_pin = -1, bool allow_route = true) {
    const auto t0 = std::chrono::steady_clock::now();
    MARS_CHECK(gh && ch && cfg && n_out && (h_q || d_q), MARS_ERR_INVALID, "null argument");
    MARS_CHECK(cap >= 0 && (cap == 0 || out), MARS_ERR_INVALID, "bad output buffer");
    const Graph& g = gh->g;
    Ctx& c = ch->c;
    MARS_CHECK(g.d == c.d, MARS_ERR_INVALID, "graph dim %d != context dim %d", g.d, c.d);
    c.hit_n = 0;                           // set again once this query has BFS levels
    // nodes published so far: loaded once, every kernel of this query is bounded by it
    const int32_t n_live = n_pin >= 0 ? n_pin : __atomic_load_n(&g.n, __ATOMIC_ACQUIRE);
    MARS_CHECK(n_live <= c.max_nodes, MARS_ERR_CAPACITY, "graph has %d nodes, context sized for %d", n_live,
               c.max_nodes);
    MARS_CHECK(n_live > 0, MARS_ERR_INVALID, "empty graph");
    MARS_CHECK(cfg->top_k > 0, MARS_ERR_INVALID, "top_k = %d", cfg->top_k);
    const int32_t K = std::min(cfg->top_k, c.max_k);                      // memory_cuda.cu:1361
    const bool scoped = episode_scoped_active(g, *cfg);
    const int32_t hops = scoped ? 0 : std::max(0, cfg->bfs_max_hops);     // :1189
    // results: max_results_returned (else K), at most the context's compaction cap
    // min(max_nodes, max_k * 500) (memory_cuda.cu:1059, 1421-1447)
    const int32_t rcap = std::min(cfg->max_results_returned > 0 ? cfg->max_results_returned : K, c.res_cap);
    const bool capped = cfg->max_results_returned > c.res_cap;          // reported in stats
    MARS_TRY(use_device(c.device));
    hipStream_t s = c.stream;
    const bool timing = (c.flags & MARS_CTX_TIMING) != 0;
    const bool fp16 = !scoped && (c.flags & MARS_CTX_USE_FP16) && g.emb16 != nullptr;
    const bool use_graph = (c.flags & MARS_CTX_USE_GRAPH) != 0;

    const float* q = d_q;
    if (!q) {
        std::memcpy(c.h_query, h_q, size_t(g.d) * sizeof(float));
        MARS_HIP(hipMemcpyAsync(c.query, c.h_query, size_t(g.d) * sizeof(float), hipMemcpyHostToDevice, s));
        q = c.query;
    }
    const float lam = cfg->time_decay_lambda;
    const bool boost_on = g.ep_ids && cfg->query_episode_id >= 0 && cfg->episode_same_boost > 0.0f;
    const bool cert = !scoped && !fp16 && (c.flags & MARS_CTX_CERTIFIED) &&
                      cert_dim_supported(g.d) && (cert_uses_int8(g) || (g.emb16 && g.nrm)) &&
                      !boost_on && lam >= 0.0f && lam <= FLT_MAX && hops < 255;
    if (cert && allow_route && !use_graph && cert_uses_int8(g) && n_live >= kCertRouteRows && K <= kMultiCand &&
        n_pin < 0) {
        mars_batch_stats bst{};
        MARS_TRY(global_batch_impl(gh, ch, q, 1, &t_q, cfg, out, cap, n_out, &bst, 0, 0, 0, nullptr, true, true));
        c.last_certified = 0;                 // no phase stamps on this path
        c.last_visited = 0;
        c.last_n = 0;
        int32_t visited = 0, levels = 0;
        if (bst.batched == 1) {
            const ResultHeader h = static_cast<const ResultHeader*>(c.h_mres)[0];
            visited = h.visited;
            levels = h.levels;
            c.hit_vlist = c.mvlist;           // BFS levels for edge-hit counting
            c.hit_vhop = c.mvhop;
            c.hit_n = h.visited;
            c.last_k = h.n_seeds;
        }
        if (stats) {
            mars_stats st{};
            st.gpu_ms_similarity = bst.gpu_ms_scan;
            st.gpu_ms_topk = bst.gpu_ms_seeds;
            st.gpu_ms_bfs = bst.gpu_ms_bfs;
            st.gpu_ms_total = bst.gpu_ms_total;
            st.nodes_scanned = n_live;
            st.bfs_waves = cfg->bfs_max_hops;
            st.scope_fallback = (cfg->retrieval_scope == MARS_SCOPE_EPISODE_SCOPED) ? 1 : 0;
            st.visited = visited;
            st.bfs_levels_run = levels;
            st.used_fp16 = 1;
            st.seeds_certified = bst.batched;
            st.results_capped = capped && visited > *n_out ? 1 : 0;
            st.wall_us = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
            *stats = st;
        }
        return MARS_OK;
    }
    if (cert) {
        bool answered = false;
        ResultHeader h{};
        MARS_TRY(certified_query(g, c, q, t_q, cfg, K, hops, rcap, n_live, out, cap, n_out, &answered, &h));
        c.last_certified = answered ? 1 : 0;
        if (answered) {
            c.hit_vlist = c.mvlist;           // BFS levels for edge-hit counting
            c.hit_vhop = c.mvhop;
            c.hit_n = h.visited;
            c.last_k = h.n_seeds;
            c.last_visited = 0;               // the debug hooks describe fp32 scans only
            c.last_n = 0;
            if (stats) {
                mars_stats st{};
                if (timing) {
                    float ms = 0.0f;
                    MARS_HIP(hipEventElapsedTime(&ms, c.ev[0], c.ev[1]));
                    st.gpu_ms_similarity = ms;
                    MARS_HIP(hipEventElapsedTime(&ms, c.ev[0], c.ev[2]));
                    st.gpu_ms_total = ms;
                    MARS_HIP(hipEventElapsedTime(&ms, c.ev[1], c.ev[2]));
                    // certificate stamps (from t[4]): candidate merge and exact rescoring +
                    // certificate select the seeds; BFS, marking, exact scores and the results
                    // follow (the single-kernel form; the two-kernel form stamps the first part)
                    const uint64_t* t = c.h_stamps + 4;
                    st.gpu_ms_topk = std::min(ms, float(double(t[2] - t[0]) * 1e-5));
                    st.gpu_ms_bfs = std::max(0.0f, ms - st.gpu_ms_topk);
                }
                st.nodes_scanned = n_live;
                st.bfs_waves = cfg->bfs_max_hops;
                st.scope_fallback = (cfg->retrieval_scope == MARS_SCOPE_EPISODE_SCOPED) ? 1 : 0;
                st.visited = h.visited;
                st.bfs_levels_run = h.levels;
                st.used_fp16 = 1;
                st.seeds_certified = 1;
                st.results_capped = capped && h.visited > h.count ? 1 : 0;
                st.wall_us = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
                *stats = st;
            }
            return MARS_OK;
        }
    }
    if (timing) MARS_HIP(hipEventRecord(c.ev[0], s));
    // the last kernel stores the completion word (timing keeps the stream sync: its
    // events must have completed)
    const uint32_t seq = next_seq(c);
    uint32_t* const done = timing ? nullptr : c.d_done;
    if (scoped) {
        EpisodeArgs a{};
        a.emb = g.emb; a.d = g.d; a.n = n_live; a.q = q; a.ts = g.ts; a.mods = g.mods;
        a.members = g.ep_mem + cfg->query_episode_member_begin;
        a.m = cfg->query_episode_member_count;
        a.t_q = t_q; a.lambda = cfg->time_decay_lambda; a.mod_filter = cfg->modality_filter;
        a.k = K; a.rcap = rcap; a.keybuf = c.sortbuf;
        a.seed_idx = c.seed_idx; a.seed_val = c.seed_val; a.res = c.d_res; a.rec = c.d_rec;
        a.done = done; a.seq = seq;
        if (use_graph) {
            const KernelLaunch l = episode_launch(g.d);
            void* args[1] = {&a};
            MARS_TRY(graph_launch(c.g_episode, 1, &l, args, s));
        } else {
            MARS_TRY(launch_episode(a, s));
        }
        if (timing) MARS_HIP(hipEventRecord(c.ev[1], s));
    } else {
        int32_t rpw = 0, nwg = 0;
        scan_grid(n_live, fp16 ? kTargetWgF16 : kTargetWg, &rpw, &nwg);
        ScanArgs a{};
        a.emb = fp16 ? static_cast<const void*>(g.emb16) : static_cast<const void*>(g.emb);
        a.fp16 = fp16 ? 1 : 0; a.n = n_live; a.d = g.d; a.q = q; a.ts = g.ts; a.mods = g.mods;
        a.ep_ids = g.ep_ids; a.t_q = t_q; a.lambda = cfg->time_decay_lambda;
        a.mod_filter = cfg->modality_filter; a.query_ep = cfg->query_episode_id;
        a.boost = (g.ep_ids && cfg->query_episode_id >= 0) ? cfg->episode_same_boost : 0.0f;
        a.k = K; a.fin = c.fin; a.part = c.part; a.gthr = c.gthr; a.gcnt = c.gcnt; a.rows_per_wg = rpw;
        a.num_wg = nwg;
        // visit stamps / claim generations: no O(N) reset per query
        if (c.epoch == 0xFFFFFFFFu) {
            MARS_HIP(hipMemsetAsync(c.vis, 0, size_t(c.max_nodes) * sizeof(uint32_t), s));
            c.epoch = 0;
        }
        const uint32_t epoch = ++c.epoch;
        const uint32_t span = uint32_t(std::max(hops, 1));
        if (uint64_t(c.gen) + span >= 0xFFFFFFF0ull) {
            MARS_HIP(hipMemsetAsync(c.claim, 0xFF, size_t(c.max_nodes) * sizeof(uint64_t), s));
            c.gen = 0;
        }
        const uint32_t gen_base = c.gen;
        c.gen += span;
        FinalizeArgs f{};
        f.part = c.part; f.gcnt = c.gcnt; f.gthr = c.gthr; f.k = K; f.ro = g.ro; f.col = g.col; f.n_live = n_live; f.fin = c.fin;
        f.mods = g.mods; f.hops = hops; f.hop_decay = cfg->bfs_score_decay; f.epoch = epoch;
        f.gen_base = gen_base; f.vis = c.vis; f.claim = c.claim; f.vlist = c.vlist; f.vhop = c.vhop;
        f.vscore = c.vscore; f.vro = c.vro; f.sortbuf = c.sortbuf; f.cap_visit = c.max_nodes; f.rcap = rcap;
        f.seed_idx = c.seed_idx; f.seed_val = c.seed_val; f.res = c.d_res; f.rec = c.d_rec;
        f.stamps = c.stamps;
        f.done = done; f.seq = seq;
        if (use_graph) {
            // one replayed graph for both kernels (the per-stage split is not timed)
            const KernelLaunch l[2] = {scan_launch(a), finalize_launch()};
            void* args[2] = {&a, &f};
            MARS_TRY(graph_launch(c.g_global, 2, l, args, s));
            if (timing) MARS_HIP(hipEventRecord(c.ev[1], s));
        } else {
            MARS_TRY(launch_scan(a, s));
            if (timing) MARS_HIP(hipEventRecord(c.ev[1], s));
        }
        if (!use_graph && launch_finalize(f, s) != MARS_OK) {
            // the scan already appended candidates: clear them for the next query
            (void)hipMemsetAsync(c.gcnt, 0, sizeof(uint32_t), s);
            (void)hipMemsetAsync(c.gthr, 0xFF, sizeof(uint64_t), s);
            (void)hipStreamSynchronize(s);
            return set_error(MARS_ERR_HIP, "finalize launch failed");
        }
        c.last_n = n_live;
        c.last_certified = 0;
    }
    if (timing) {
        MARS_HIP(hipEventRecord(c.ev[2], s));
        MARS_HIP(hipStreamSynchronize(s));
    } else {
        MARS_TRY(wait_done(c, seq, s));
    }
    const ResultHeader h = *c.h_res;
    const int32_t nw = std::min(h.count, cap);
    if (nw > 0) std::memcpy(out, c.h_rec, size_t(nw) * sizeof(mars_query_result));
    *n_out = h.count;
    c.last_k = h.n_seeds;
    c.last_visited = scoped ? 0 : h.visited;
    if (!scoped) {
        c.hit_vlist = c.vlist;
        c.hit_vhop = c.vhop;
        c.hit_n = h.visited;
    }
    if (stats) {
        mars_stats st{};
        if (timing) {
            float ms = 0.0f;
            MARS_HIP(hipEventElapsedTime(&ms, c.ev[0], c.ev[1]));
            st.gpu_ms_similarity = ms;
            MARS_HIP(hipEventElapsedTime(&ms, c.ev[0], c.ev[2]));
            st.gpu_ms_total = ms;
            MARS_HIP(hipEventElapsedTime(&ms, c.ev[1], c.ev[2]));
            if (scoped) {
                st.gpu_ms_topk = ms;                       // the episode kernel selects as it scores
            } else {
                // finalize stamps: start, seeds merged, BFS done, results written
                const uint64_t* t = c.h_stamps;
                st.gpu_ms_topk = float(double(t[1] - t[0]) * 1e-5);   // 100 MHz counter
                st.gpu_ms_bfs = std::max(0.0f, ms - st.gpu_ms_topk);
            }
        }
        // the decay (the reference's rerank stage) is fused into the scan: gpu_ms_rerank = 0
        st.nodes_scanned = scoped ? cfg->query_episode_member_count : n_live;
        st.bfs_waves = scoped ? 0 : cfg->bfs_max_hops;                     // :1680-1686 semantics
        st.scope_fallback = (cfg->retrieval_scope == MARS_SCOPE_EPISODE_SCOPED && !scoped) ? 1 : 0;
        st.visited = h.visited;
        st.bfs_levels_run = h.levels;
        st.used_fp16 = fp16 ? 1 : 0;
        st.results_capped = capped && h.visited > h.count ? 1 : 0;
        st.wall_us = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
        *stats = st;
    }
    return MARS_OK;
}

}  // namespace

// Row ranges x query blocks for the batched scan: one 512-thread workgroup per CU
// (256 CUs), all query blocks of a row range on one XCD.
void batch_grid(int64_t n, int32_t q, bool plain, int32_t* n_rranges, int32_t* n_qblocks, int64_t* rows_per_range,
                int32_t max_ranges) {
    // n_qblocks counts 64-query blocks (the layout of the partial keys) for every kernel
    const int32_t qblocks = (q + 63) / 64;
    const bool gemm = batch_uses_gemm(q, plain), rq = batch_uses_rq(q, plain);
    const int32_t wgq = gemm ? 256 : (rq ? 64 * batch_rq_tiles(q) : 64);   // queries per workgroup
    const int32_t tiles = (q + wgq - 1) / wgq;                             // workgroups per row range
    const int64_t align = gemm ? 256 : 16;                            // rows per tile
    int32_t rr = std::max(8, (256 / std::max(tiles, 1)) / 8 * 8);
    const int64_t max_rr = std::max<int64_t>(1, (n + align - 1) / align);   // at least one tile per range
    if (rr > max_ranges) rr = std::max(1, max_ranges);
    if (rr > max_rr) rr = int32_t(max_rr);
    *n_qblocks = qblocks;
    *rows_per_range = ((n + rr - 1) / rr + align - 1) / align * align;
    *n_rranges = int32_t((n + *rows_per_range - 1) / *rows_per_range);
}

namespace {

// Scratch of the batched global path: q queries' visit slots, and host-mapped room for
// q result headers + q x rcap results.
int ensure_multi_scratch(Ctx& c, int32_t q, int32_t rcap) {
    if (q > c.mcap_q) {
        dfree(c.mqn); dfree(c.mseed); dfree(c.mstat); dfree(c.minfo); dfree(c.mmargin);
        dfree(c.mvlist); dfree(c.mvhop); dfree(c.mvpar); dfree(c.mvro); dfree(c.mvfin); dfree(c.mvscore);
        c.mcap_q = 0;
        const size_t nv = size_t(q) * kMultiVisit;
        MARS_TRY(dmalloc(&c.mqn, size_t(q) * 4));
        MARS_TRY(dmalloc(&c.mseed, size_t(q) * 64));          // 64 per query (int8 certificate)
        MARS_TRY(dmalloc(&c.mstat, size_t(q)));
        MARS_TRY(dmalloc(&c.minfo, size_t(q) * 4));
        MARS_TRY(dmalloc(&c.mmargin, size_t(q)));
        MARS_TRY(dmalloc(&c.mvlist, nv));
        MARS_TRY(dmalloc(&c.mvhop, nv));
        MARS_TRY(dmalloc(&c.mvpar, nv));
        MARS_TRY(dmalloc(&c.mvro, nv));
        MARS_TRY(dmalloc(&c.mvfin, nv));
        MARS_TRY(dmalloc(&c.mvscore, nv));
        c.mcap_q = q;
    }
    const size_t need = size_t(q) * sizeof(ResultHeader) + size_t(q) * size_t(rcap) * sizeof(mars_query_result);
    if (need > c.mres_bytes) {
        if (c.h_mres) (void)hipHostFree(c.h_mres);
        c.h_mres = nullptr;
        c.d_mres = nullptr;
        c.mres_bytes = 0;
        MARS_HIP(hipHostMalloc(&c.h_mres, need, hipHostMallocMapped));
        MARS_HIP(hipHostGetDevicePointer(&c.d_mres, c.h_mres, 0));
        c.mres_bytes = need;
    }
    return MARS_OK;
}

int ensure_batch_scratch(Ctx& c, int32_t q, int64_t part_keys) {
    if (q > c.bcap_q) {
        dfree(c.bq); dfree(c.btq); dfree(c.bout);
        c.bcap_q = 0;
        MARS_TRY(dmalloc(&c.bq, size_t(q) * size_t(c.d)));
        MARS_TRY(dmalloc(&c.btq, size_t(q)));
        MARS_TRY(dmalloc(&c.bout, size_t(q) * 16));
        c.bcap_q = q;
    }
    if (part_keys > c.bcap_part) {
        dfree(c.bpart);
        c.bcap_part = 0;
        MARS_TRY(dmalloc(&c.bpart, size_t(part_keys)));
        c.bcap_part = part_keys;
    }
    return MARS_OK;
}

}  // namespace
}  // namespace mars

using namespace mars;

// The ctypes mirrors (mars_amd/_lib.py) depend on these layouts.
static_assert(sizeof(mars_query_result) == 16, "mars_query_result layout");
static_assert(sizeof(mars_stats) == 64 && offsetof(mars_stats, seeds_certified) == 44 &&
                  offsetof(mars_stats, results_capped) == 48 && offsetof(mars_stats, wall_us) == 56,
              "mars_stats layout");
static_assert(sizeof(mars_insert_stats) == 48 && offsetof(mars_insert_stats, queryable_us) == 24,
              "mars_insert_stats layout");
static_assert(sizeof(mars_stream_bench) == 128 && offsetof(mars_stream_bench, knn_k) == 88,
              "mars_stream_bench layout");
static_assert(sizeof(mars_batch_stats) == 64 && offsetof(mars_batch_stats, wall_us) == 48,
              "mars_batch_stats layout");
static_assert(sizeof(mars_serve_bench) == 216 && offsetof(mars_serve_bench, g_done_us) == 128 &&
                  offsetof(mars_serve_bench, ins_linked_us) == 192,
              "mars_serve_bench layout");

namespace {

// Best bandwidth (GB/s) of `launch(grid, out, stream)` over 256, 512 and 1024 workgroups:
// two untimed launches, then reps timed ones, on a stream of its own.
template <typename Launch>
int time_read(int64_t bytes, int32_t reps, const char* what, Launch&& launch, double* gbps) {
    constexpr int32_t kGrids[3] = {256, 512, 1024};
    hipStream_t s = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    uint32_t* out = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&out), 1024 * sizeof(uint32_t));
    double best = 0.0;
    int rc = MARS_OK;
    for (int gi = 0; gi < 3 && e == hipSuccess && rc == MARS_OK; ++gi) {
        for (int w = 0; w < 2 && rc == MARS_OK; ++w) rc = launch(kGrids[gi], out, s);
        if (rc != MARS_OK) break;
        e = hipEventRecord(e0, s);
        for (int r = 0; r < reps && rc == MARS_OK && e == hipSuccess; ++r) rc = launch(kGrids[gi], out, s);
        if (rc != MARS_OK || e != hipSuccess) break;
        e = hipEventRecord(e1, s);
        if (e == hipSuccess) e = hipEventSynchronize(e1);
        float ms = 0.0f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
        if (e == hipSuccess && ms > 0.0f) best = std::max(best, double(bytes) * reps / (double(ms) * 1e-3) / 1e9);
    }
    if (s) (void)hipStreamSynchronize(s);
    if (out) (void)hipFree(out);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (s) (void)hipStreamDestroy(s);
    if (rc != MARS_OK) return rc;
    if (e != hipSuccess) return set_error(MARS_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    *gbps = best;
    return MARS_OK;
}

}  // namespace

extern "C" {

const char* mars_last_error(void) { return g_err; }
int mars_abi_version(void) { return MARS_ABI_VERSION; }

int mars_init(int32_t device) {
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= 0) return set_error(MARS_ERR_NODEVICE, "no HIP device");
    MARS_CHECK(device >= 0 && device < count, MARS_ERR_INVALID, "device %d of %d", device, count);
    MARS_HIP(hipSetDevice(device));
    MARS_TRY(ensure_device(nullptr));
    return noalloc_prepare(device);
}

void mars_config_default(mars_retrieval_config* c) {
    // RetrievalConfig defaults, memory_cuda.cuh:107-127
    c->top_k = 10;
    c->bfs_max_hops = 2;
    c->time_decay_lambda = 1e-8f;
    c->bfs_score_decay = 0.5f;
    c->modality_filter = -1;
    c->use_importance = 0;
    c->max_results_returned = -1;
    c->retrieval_scope = MARS_SCOPE_GLOBAL;
    c->query_episode_id = -1;
    c->query_episode_member_begin = 0;
    c->query_episode_member_count = 0;
    c->episode_same_boost = 0.0f;
}

int mars_graph_create(const mars_graph_desc* d, mars_graph** out) {
    MARS_CHECK(d && out, MARS_ERR_INVALID, "null argument");
    *out = nullptr;
    MARS_CHECK(d->num_nodes > 0 && d->embedding_dim > 0 && d->num_edges >= 0, MARS_ERR_INVALID,
               "num_nodes %d, embedding_dim %d, num_edges %d", d->num_nodes, d->embedding_dim, d->num_edges);
    MARS_CHECK(d->embeddings && d->modalities && d->timestamps, MARS_ERR_INVALID,
               "embeddings, modalities and timestamps are required");
    const bool dev = (d->flags & MARS_DESC_DEVICE_POINTERS) != 0;
    if (!dev) MARS_TRY(validate_csr(d->num_nodes, d->num_edges, d->row_offsets, d->col_indices));
    else MARS_CHECK(d->num_edges == 0 || (d->row_offsets && d->col_indices), MARS_ERR_INVALID, "CSR missing");
    int devid = 0;
    MARS_TRY(ensure_device(&devid));
    MARS_TRY(noalloc_prepare(devid));      // mars_query_batch_static's scratch address
    auto* gh = new mars_graph();
    Graph& g = gh->g;
    g.device = devid;
    g.n = d->num_nodes; g.e = d->num_edges; g.d = d->embedding_dim;
    g.cap_n = std::max(d->capacity_nodes, d->num_nodes);
    g.cap_e = d->capacity_edges > 0 ? std::max<int64_t>(d->capacity_edges, d->num_edges)
                                    : int64_t(d->num_edges) + edge_room(g);
    const size_t N = size_t(g.n), D = size_t(g.d), CN = size_t(g.cap_n);
    int rc = MARS_OK;
    auto fail = [&](int r) { graph_free(g); delete gh; return r; };
    if ((rc = dmalloc(&g.emb, CN * D)) || (rc = dmalloc(&g.mods, CN)) || (rc = dmalloc(&g.ts, CN)) ||
        (rc = dmalloc(&g.ro, CN)) || (rc = dmalloc(&g.rcap, CN)) || (rc = dmalloc(&g.col, size_t(g.cap_e))))
        return fail(rc);
    const hipMemcpyKind kind = dev ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
    hipError_t e = hipSuccess;
    if (e == hipSuccess) e = hipMemcpy(g.emb, d->embeddings, N * D * sizeof(float), kind);
    if (e == hipSuccess) e = hipMemcpy(g.mods, d->modalities, N * sizeof(int32_t), kind);
    if (e == hipSuccess) e = hipMemcpy(g.ts, d->timestamps, N * sizeof(float), kind);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&g.ins_stream, hipStreamNonBlocking);
    if (e != hipSuccess) return fail(set_error(MARS_ERR_HIP, "graph upload: %s", hipGetErrorString(e)));
    if ((rc = load_csr(g, g.n, g.e, d->row_offsets, d->col_indices, kind)) != MARS_OK) return fail(rc);
    *out = gh;
    return MARS_OK;
}

int mars_graph_destroy(mars_graph* gh) {
    if (!gh) return MARS_OK;
    if (gh->own_ctx) (void)mars_ctx_destroy(gh->own_ctx);
    graph_free(gh->g);
    delete gh;
    return MARS_OK;
}

int mars_graph_set_csr(mars_graph* gh, int32_t ne, const int32_t* row, const int32_t* col) {
    MARS_CHECK(gh && ne >= 0, MARS_ERR_INVALID, "bad arguments");
    std::lock_guard<std::mutex> lock(gh->mu);
    Graph& g = gh->g;
    MARS_TRY(validate_csr(g.n, ne, row, col));
    MARS_TRY(use_device(g.device));
    MARS_HIP(hipStreamSynchronize(g.ins_stream));
    if (int64_t(ne) + edge_room(g) > g.cap_e) {
        int32_t* ncol = nullptr;
        MARS_TRY(dmalloc(&ncol, size_t(ne + edge_room(g))));
        dfree(g.col);
        g.col = ncol;
        g.cap_e = int64_t(ne) + edge_room(g);
    }
    MARS_TRY(reset_edge_hits(g));
    return load_csr(g, g.n, ne, row, col, hipMemcpyHostToDevice);
}

int mars_graph_set_episode_ids(mars_graph* gh, const int32_t* ids, int32_t n) {
    MARS_CHECK(gh, MARS_ERR_INVALID, "null graph");
    std::lock_guard<std::mutex> lock(gh->mu);
    Graph& g = gh->g;
    MARS_TRY(use_device(g.device));
    dfree(g.ep_ids);                                      // memory_cuda.cu:814-826
    g.ep_next = g.num_eps;
    if (!ids || n <= 0) return MARS_OK;                   // cleared
    MARS_CHECK(n == g.n, MARS_ERR_INVALID, "episode ids: %d entries for %d nodes", n, g.n);
    MARS_TRY(dmalloc(&g.ep_ids, size_t(g.cap_n)));
    MARS_HIP(hipMemcpy(g.ep_ids, ids, size_t(n) * sizeof(int32_t), hipMemcpyHostToDevice));
    for (int32_t i = 0; i < n; ++i)
        if (ids[i] >= g.ep_next) g.ep_next = ids[i] == INT32_MAX ? INT32_MAX : ids[i] + 1;
    return MARS_OK;
}

int mars_graph_set_episode_csr(mars_graph* gh, int32_t num_eps, const int32_t* off, const int32_t* mem,
                               int32_t member_total) {
    MARS_CHECK(gh, MARS_ERR_INVALID, "null graph");
    std::lock_guard<std::mutex> lock(gh->mu);
    Graph& g = gh->g;
    MARS_TRY(use_device(g.device));
    dfree(g.ep_off); dfree(g.ep_mem);                     // memory_cuda.cu:828-855
    g.num_eps = 0;
    g.member_total = 0;
    g.ep_off_cap = g.ep_mem_cap = 0;
    if (num_eps <= 0) return MARS_OK;
    MARS_CHECK(off && (member_total == 0 || mem), MARS_ERR_INVALID, "episode CSR arrays missing");
    MARS_CHECK(off[num_eps] == member_total && member_total >= 0, MARS_ERR_INVALID,
               "episode CSR tail %d != member_total %d", off[num_eps], member_total);
    MARS_CHECK(off[0] == 0, MARS_ERR_INVALID, "episode CSR offsets[0] = %d", off[0]);
    for (int32_t e = 0; e < num_eps; ++e)
        MARS_CHECK(off[e] <= off[e + 1], MARS_ERR_INVALID, "episode CSR offsets decrease at %d", e);
    for (int32_t j = 0; j < member_total; ++j)
        MARS_CHECK(mem[j] >= 0 && mem[j] < g.n, MARS_ERR_INVALID, "episode member %d = %d out of range", j,
                   mem[j]);
    // capacity for episodes appended by streaming inserts (at most one per node)
    g.ep_off_cap = int64_t(std::max(num_eps, g.cap_n)) + 1;
    g.ep_mem_cap = int64_t(std::max(member_total, g.cap_n));
    MARS_TRY(dmalloc(&g.ep_off, size_t(g.ep_off_cap)));
    MARS_TRY(dmalloc(&g.ep_mem, size_t(g.ep_mem_cap)));
    MARS_HIP(hipMemcpy(g.ep_off, off, (size_t(num_eps) + 1) * sizeof(int32_t), hipMemcpyHostToDevice));
    if (member_total > 0)
        MARS_HIP(hipMemcpy(g.ep_mem, mem, size_t(member_total) * sizeof(int32_t), hipMemcpyHostToDevice));
    g.num_eps = num_eps;
    g.member_total = member_total;
    g.ep_next = std::max(g.ep_next, num_eps);
    return MARS_OK;
}

int mars_graph_enable_fp16(mars_graph* gh) {
    MARS_CHECK(gh, MARS_ERR_INVALID, "null graph");
    std::lock_guard<std::mutex> lock(gh->mu);
    Graph& g = gh->g;
    MARS_TRY(use_device(g.device));
    if (!g.emb16) MARS_TRY(dmalloc(&g.emb16, size_t(g.cap_n) * size_t(g.d)));
    if (!g.nrm) MARS_TRY(dmalloc(&g.nrm, 4));
    MARS_HIP(hipMemset(g.nrm, 0, 4 * sizeof(uint32_t)));
    MARS_TRY(launch_convert_f16(g.emb, g.emb16, int64_t(g.n) * g.d, nullptr));
    MARS_TRY(launch_row_norms(g.emb, g.emb16, 0, g.n, g.d, g.nrm, nullptr));
    MARS_HIP(hipStreamSynchronize(nullptr));
    return MARS_OK;
}

int mars_graph_disable_fp16(mars_graph* gh) {
    MARS_CHECK(gh, MARS_ERR_INVALID, "null graph");
    std::lock_guard<std::mutex> lock(gh->mu);
    MARS_TRY(use_device(gh->g.device));
    dfree(gh->g.emb16);
    dfree(gh->g.nrm);
    return MARS_OK;
}

int mars_graph_enable_int8(mars_graph* gh) {
    MARS_CHECK(gh, MARS_ERR_INVALID, "null graph");
    std::lock_guard<std::mutex> lock(gh->mu);
    Graph& g = gh->g;
    MARS_CHECK(scan8_dim_supported(g.d), MARS_ERR_UNSUPPORTED,
               "int8 copy: embedding_dim %d is not 256, 512, 768, 1024 or 1536", g.d);
    MARS_TRY(use_device(g.device));
    const size_t bytes8 = size_t(i8_rows_alloc(g.cap_n)) * size_t(g.d);      // whole 16-row tiles
    if (!g.emb8) {
        MARS_TRY(dmalloc(&g.emb8, bytes8));
        MARS_HIP(hipMemset(g.emb8, 0, bytes8));                             // rows past n score 0
    }
    if (!g.meta8) MARS_TRY(dmalloc(&g.meta8, size_t(g.cap_n) * 2));
    if (!g.nrm8) MARS_TRY(dmalloc(&g.nrm8, 2));
    MARS_HIP(hipMemset(g.nrm8, 0, 2 * sizeof(uint32_t)));
    MARS_TRY(launch_convert_i8(g.emb, 0, g.n, g.d, g.emb8, g.meta8, g.nrm8, nullptr));
    MARS_HIP(hipStreamSynchronize(nullptr));
    return MARS_OK;
}

int mars_graph_disable_int8(mars_graph* gh) {
    MARS_CHECK(gh, MARS_ERR_INVALID, "null graph");
    std::lock_guard<std::mutex> lock(gh->mu);
    MARS_TRY(use_device(gh->g.device));
    dfree(gh->g.emb8);
    dfree(gh->g.meta8);
    dfree(gh->g.nrm8);
    return MARS_OK;
}

int mars_graph_read_int8(const mars_graph* gh, int32_t first, int32_t count, int8_t* bytes, float* meta) {
    MARS_CHECK(gh && (bytes || meta), MARS_ERR_INVALID, "null argument");
    std::lock_guard<std::mutex> lock(gh->mu);
    const Graph& g = gh->g;
    MARS_CHECK(g.emb8 != nullptr, MARS_ERR_UNSUPPORTED, "no int8 copy");
    MARS_CHECK(first >= 0 && count >= 0 && int64_t(first) + count <= g.n, MARS_ERR_INVALID,
               "rows [%d, %lld) outside the %d published nodes", first, (long long)first + count, g.n);
    MARS_TRY(use_device(g.device));
    if (count == 0) return MARS_OK;
    if (bytes) {
        // the 16-row tiles that hold the rows, then back to row-major order
        const int64_t t0 = first / 16, t1 = (int64_t(first) + count + 15) / 16;
        std::vector<int8_t> tiles(size_t(t1 - t0) * 16 * size_t(g.d));
        MARS_HIP(hipMemcpy(tiles.data(), g.emb8 + t0 * 16 * g.d, tiles.size(), hipMemcpyDeviceToHost));
        for (int32_t r = 0; r < count; ++r)
            for (int32_t k = 0; k < g.d; ++k)
                bytes[size_t(r) * g.d + k] = tiles[size_t(i8_offset(int64_t(first) + r, k, g.d) - t0 * 16 * g.d)];
    }
    if (meta) MARS_HIP(hipMemcpy(meta, g.meta8 + size_t(first) * 2, size_t(count) * 2 * sizeof(float),
                                 hipMemcpyDeviceToHost));
    return MARS_OK;
}

int mars_graph_get_view(const mars_graph* gh, mars_graph_view* v) {
    MARS_CHECK(gh && v, MARS_ERR_INVALID, "null argument");
    std::lock_guard<std::mutex> lock(gh->mu);
    const Graph& g = gh->g;
    v->num_nodes = g.n; v->num_edges = g.e; v->embedding_dim = g.d;
    v->episode_num_episodes = g.num_eps; v->episode_csr_member_total = g.member_total;
    v->has_fp16 = g.emb16 ? 1 : 0;
    v->d_row_words = g.ro; v->d_col_indices = g.col; v->d_embeddings = g.emb;
    v->d_embeddings_fp16 = g.emb16; v->d_modalities = g.mods; v->d_timestamps = g.ts;
    v->d_episode_ids = g.ep_ids; v->d_ep_csr_offsets = g.ep_off; v->d_ep_csr_members = g.ep_mem;
    return MARS_OK;
}

int mars_graph_download(const mars_graph* gh, int32_t* row, int32_t* col, int32_t* ep_off, int32_t* ep_mem) {
    MARS_CHECK(gh, MARS_ERR_INVALID, "null graph");
    std::lock_guard<std::mutex> lock(gh->mu);
    const Graph& g = gh->g;
    MARS_TRY(use_device(g.device));
    if (row || col) {
        // rows are (start, length) segments of col: rebuild the packed CSR
        std::vector<int32_t> dcol(size_t(std::max<int64_t>(g.e_used, 1)));
        if (g.e_used > 0)
            MARS_HIP(hipMemcpy(dcol.data(), g.col, size_t(g.e_used) * sizeof(int32_t), hipMemcpyDeviceToHost));
        int64_t pos = 0;
        if (row) row[0] = 0;
        for (int32_t i = 0; i < g.n; ++i) {
            const int64_t w = g.ro_h[size_t(i)];
            const int32_t b = int32_t(uint32_t(w)), len = int32_t(w >> 32);
            if (col) std::memcpy(col + pos, dcol.data() + b, size_t(len) * sizeof(int32_t));
            pos += len;
            if (row) row[i + 1] = int32_t(pos);
        }
    }
    if (ep_off && g.ep_off)
        MARS_HIP(hipMemcpy(ep_off, g.ep_off, (size_t(g.num_eps) + 1) * sizeof(int32_t), hipMemcpyDeviceToHost));
    if (ep_mem && g.ep_mem && g.member_total > 0)
        MARS_HIP(hipMemcpy(ep_mem, g.ep_mem, size_t(g.member_total) * sizeof(int32_t), hipMemcpyDeviceToHost));
    return MARS_OK;
}

int mars_graph_packed_csr(mars_graph* gh, const int32_t** d_row_offsets, const int32_t** d_col_indices) {
    MARS_CHECK(gh && d_row_offsets && d_col_indices, MARS_ERR_INVALID, "null argument");
    std::lock_guard<std::mutex> lock(gh->mu);
    Graph& g = gh->g;
    MARS_TRY(use_device(g.device));
    if (g.pk_row && g.pk_version == g.csr_version && g.pk_cap_n >= int64_t(g.n) + 1) {
        *d_row_offsets = g.pk_row;
        *d_col_indices = g.pk_col;
        return MARS_OK;
    }
    if (g.ins_stream) MARS_HIP(hipStreamSynchronize(g.ins_stream));
    const int32_t n = g.n;
    std::vector<int32_t> off(size_t(n) + 1, 0);
    for (int32_t i = 0; i < n; ++i) off[size_t(i) + 1] = off[size_t(i)] + int32_t(g.ro_h[size_t(i)] >> 32);
    const int64_t ne = off[size_t(n)];
    if (g.pk_cap_n < int64_t(n) + 1) {
        dfree(g.pk_row);
        g.pk_cap_n = 0;
        MARS_TRY(dmalloc(&g.pk_row, size_t(g.cap_n) + 1));
        g.pk_cap_n = int64_t(g.cap_n) + 1;
    }
    if (g.pk_cap_e < std::max<int64_t>(ne, 1)) {
        dfree(g.pk_col);
        g.pk_cap_e = 0;
        MARS_TRY(dmalloc(&g.pk_col, size_t(std::max<int64_t>(ne, 1))));
        g.pk_cap_e = std::max<int64_t>(ne, 1);
    }
    MARS_HIP(hipMemcpy(g.pk_row, off.data(), off.size() * sizeof(int32_t), hipMemcpyHostToDevice));
    if (ne > 0) {
        const int64_t blocks = std::min<int64_t>((int64_t(n) * 16 + 255) / 256, 65536);
        MARS_LAUNCH(k_pack_csr, dim3(unsigned(std::max<int64_t>(blocks, 1))), dim3(256), 0, g.ins_stream, g.ro,
                    g.col, g.pk_row, g.pk_col, n);
        MARS_HIP(hipStreamSynchronize(g.ins_stream));
    }
    g.pk_version = g.csr_version;
    *d_row_offsets = g.pk_row;
    *d_col_indices = g.pk_col;
    return MARS_OK;
}

// MARS v1 checkpoint of the device graph: the published nodes (inserts included) as
// the packed CSR, fp32 rows, modalities and timestamps, streamed to the file in 64 MB
// pieces. Holds the graph's lock, so an insert lands wholly before or after it.
int mars_graph_save(const mars_graph* gh, const char* path) {
    MARS_CHECK(gh && path, MARS_ERR_INVALID, "null argument");
    std::lock_guard<std::mutex> lock(gh->mu);
    const Graph& g = gh->g;
    MARS_TRY(use_device(g.device));
    if (g.ins_stream) MARS_HIP(hipStreamSynchronize(g.ins_stream));
    const int32_t n = g.n, d = g.d;
    std::vector<int32_t> dcol(size_t(std::max<int64_t>(g.e_used, 1)));
    if (g.e_used > 0)
        MARS_HIP(hipMemcpy(dcol.data(), g.col, size_t(g.e_used) * sizeof(int32_t), hipMemcpyDeviceToHost));
    std::vector<int32_t> row(size_t(n) + 1, 0), col;
    col.reserve(size_t(g.e));
    for (int32_t i = 0; i < n; ++i) {
        const int64_t w = g.ro_h[size_t(i)];
        const int32_t b = int32_t(uint32_t(w)), len = int32_t(w >> 32);
        col.insert(col.end(), dcol.begin() + b, dcol.begin() + b + len);
        row[size_t(i) + 1] = int32_t(col.size());
    }
    GraphFileWriter w;
    MARS_TRY(w.open(path, n, int32_t(col.size()), d));
    MARS_TRY(w.put(row.data(), row.size() * sizeof(int32_t)));
    MARS_TRY(w.put(col.data(), col.size() * sizeof(int32_t)));
    const int64_t rows_per = std::max<int64_t>(1, (int64_t(64) << 20) / (int64_t(std::max(d, 1)) * 4));
    std::vector<float> buf(size_t(std::min<int64_t>(rows_per, std::max(n, 1))) * size_t(std::max(d, 1)));
    for (int64_t r0 = 0; r0 < n && d > 0; r0 += rows_per) {
        const int64_t nr = std::min<int64_t>(rows_per, n - r0);
        const size_t bytes = size_t(nr) * size_t(d) * sizeof(float);
        MARS_HIP(hipMemcpy(buf.data(), g.emb + r0 * d, bytes, hipMemcpyDeviceToHost));
        MARS_TRY(w.put(buf.data(), bytes));
    }
    std::vector<int32_t> mods(size_t(std::max(n, 1)));
    std::vector<float> ts(size_t(std::max(n, 1)));
    if (n > 0) {
        MARS_HIP(hipMemcpy(mods.data(), g.mods, size_t(n) * sizeof(int32_t), hipMemcpyDeviceToHost));
        MARS_HIP(hipMemcpy(ts.data(), g.ts, size_t(n) * sizeof(float), hipMemcpyDeviceToHost));
    }
    MARS_TRY(w.put(mods.data(), size_t(n) * sizeof(int32_t)));
    MARS_TRY(w.put(ts.data(), size_t(n) * sizeof(float)));
    return w.finish();
}

int mars_ctx_create(int32_t max_nodes, int32_t dim, int32_t max_k, uint32_t flags, mars_ctx** out) {
    MARS_CHECK(out, MARS_ERR_INVALID, "null argument");
    *out = nullptr;
    MARS_CHECK(max_nodes > 0 && dim > 0 && max_k > 0, MARS_ERR_INVALID, "max_nodes %d, dim %d, max_k %d",
               max_nodes, dim, max_k);
    int devid = 0;
    MARS_TRY(ensure_device(&devid));
    auto* ch = new mars_ctx();
    Ctx& c = ch->c;
    c.device = devid;
    c.max_nodes = max_nodes;
    c.d = dim;
    c.max_k = std::min(max_k, kMaxK);                       // memory_cuda.cu:1036
    c.flags = flags;
    c.max_wg = kMaxWg;
    c.res_cap = std::max(1, std::min(max_nodes, c.max_k * kCompactPerK));   // memory_cuda.cu:1059
    const size_t N = size_t(max_nodes);
    int rc = MARS_OK;
    auto fail = [&](int r) { ctx_free(c); delete ch; return r; };
    hipError_t e = hipStreamCreateWithFlags(&c.stream, hipStreamNonBlocking);
    if (e != hipSuccess) return fail(set_error(MARS_ERR_HIP, "stream: %s", hipGetErrorString(e)));
    if ((rc = dmalloc(&c.query, size_t(dim))) || (rc = dmalloc(&c.fin, N)) ||
        (rc = dmalloc(&c.part, size_t(kMaxWg) * kMaxK)) || (rc = dmalloc(&c.vis, N)) ||
        (rc = dmalloc(&c.claim, N)) || (rc = dmalloc(&c.vlist, N)) || (rc = dmalloc(&c.vhop, N)) ||
        (rc = dmalloc(&c.vscore, N)) || (rc = dmalloc(&c.vro, 2 * N)) || (rc = dmalloc(&c.sortbuf, 2 * size_t(kSortCap))) ||
        (rc = dmalloc(&c.seed_idx, size_t(kMaxK))) || (rc = dmalloc(&c.seed_val, size_t(kMaxK))) ||
        (rc = dmalloc(&c.gthr, 1)) || (rc = dmalloc(&c.gcnt, 1)))
        return fail(rc);
    e = hipMemset(c.vis, 0, N * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemset(c.gthr, 0xFF, sizeof(uint64_t));
    if (e == hipSuccess) e = hipMemset(c.gcnt, 0, sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemset(c.claim, 0xFF, N * sizeof(uint64_t));
    if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void**>(&c.h_query), size_t(dim) * sizeof(float));
    const size_t res_bytes = sizeof(ResultHeader) + size_t(c.res_cap) * sizeof(mars_query_result);
    if (e == hipSuccess)
        e = hipHostMalloc(reinterpret_cast<void**>(&c.h_res), res_bytes, hipHostMallocMapped);
    void* dres = nullptr;
    if (e == hipSuccess) e = hipHostGetDevicePointer(&dres, c.h_res, 0);
    if (e != hipSuccess) return fail(set_error(MARS_ERR_NOMEM, "context setup: %s", hipGetErrorString(e)));
    std::memset(c.h_res, 0, res_bytes);
    c.h_rec = reinterpret_cast<mars_query_result*>(c.h_res + 1);
    c.d_res = static_cast<ResultHeader*>(dres);
    c.d_rec = reinterpret_cast<mars_query_result*>(c.d_res + 1);
    void* ddone = nullptr;
    e = hipHostMalloc(reinterpret_cast<void**>(&c.h_done), 64, hipHostMallocMapped);
    if (e == hipSuccess) e = hipHostGetDevicePointer(&ddone, c.h_done, 0);
    if (e != hipSuccess) return fail(set_error(MARS_ERR_NOMEM, "context setup: %s", hipGetErrorString(e)));
    *c.h_done = 0u;
    c.d_done = static_cast<uint32_t*>(ddone);
    // phase stamps: written by the last kernels of a query, read on the host after it
    void* dst = nullptr;
    e = hipHostMalloc(reinterpret_cast<void**>(&c.h_stamps), 12 * sizeof(uint64_t), hipHostMallocMapped);
    if (e == hipSuccess) e = hipHostGetDevicePointer(&dst, c.h_stamps, 0);
    if (e != hipSuccess) return fail(set_error(MARS_ERR_NOMEM, "context setup: %s", hipGetErrorString(e)));
    std::memset(c.h_stamps, 0, 12 * sizeof(uint64_t));
    c.stamps = static_cast<uint64_t*>(dst);
    for (auto& ev : c.ev) {
        e = hipEventCreate(&ev);
        if (e != hipSuccess) return fail(set_error(MARS_ERR_HIP, "event: %s", hipGetErrorString(e)));
    }
    *out = ch;
    return MARS_OK;
}

int mars_ctx_destroy(mars_ctx* ch) {
    if (!ch) return MARS_OK;
    ctx_free(ch->c);
    delete ch;
    return MARS_OK;
}

int mars_ctx_set_flags(mars_ctx* ch, uint32_t flags) {
    MARS_CHECK(ch, MARS_ERR_INVALID, "null context");
    ch->c.flags = flags;
    return MARS_OK;
}

int mars_ctx_get_stream(const mars_ctx* ch, void** stream) {
    MARS_CHECK(ch && stream, MARS_ERR_INVALID, "null argument");
    *stream = static_cast<void*>(ch->c.stream);
    return MARS_OK;
}

int mars_ctx_get_flags(const mars_ctx* ch, uint32_t* flags) {
    MARS_CHECK(ch && flags, MARS_ERR_INVALID, "null argument");
    *flags = ch->c.flags;
    return MARS_OK;
}

int mars_query(const mars_graph* g, mars_ctx* c, const float* h_query, float t_q,
               const mars_retrieval_config* cfg, mars_query_result* out, int32_t cap, int32_t* n_out,
               mars_stats* stats) {
    MARS_CHECK(h_query, MARS_ERR_INVALID, "null query");
    return query_impl(g, c, h_query, nullptr, t_q, cfg, out, cap, n_out, stats);
}

int mars_query_device(const mars_graph* g, mars_ctx* c, const float* d_query, float t_q,
                      const mars_retrieval_config* cfg, mars_query_result* out, int32_t cap, int32_t* n_out,
                      mars_stats* stats) {
    MARS_CHECK(d_query, MARS_ERR_INVALID, "null query");
    return query_impl(g, c, nullptr, d_query, t_q, cfg, out, cap, n_out, stats);
}

int mars_device_alloc(size_t bytes, void** ptr) {
    MARS_CHECK(ptr, MARS_ERR_INVALID, "null argument");
    *ptr = nullptr;
    MARS_TRY(ensure_device(nullptr));
    hipError_t e = hipMalloc(ptr, bytes ? bytes : 1);
    if (e != hipSuccess) return set_error(MARS_ERR_NOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    return MARS_OK;
}

int mars_device_free(void* ptr) {
    if (ptr) MARS_HIP(hipFree(ptr));
    return MARS_OK;
}

int mars_copy_to_device(void* dst, const void* src, size_t bytes) {
    MARS_CHECK(dst && src, MARS_ERR_INVALID, "null argument");
    MARS_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return MARS_OK;
}

int mars_copy_to_host(void* dst, const void* src, size_t bytes) {
    MARS_CHECK(dst && src, MARS_ERR_INVALID, "null argument");
    MARS_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return MARS_OK;
}

int mars_copy_device(void* dst, const void* src, size_t bytes) {
    MARS_CHECK(dst && src, MARS_ERR_INVALID, "null argument");
    MARS_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice));
    return MARS_OK;
}

int mars_device_memory(size_t* free_bytes, size_t* total_bytes) {
    MARS_CHECK(free_bytes && total_bytes, MARS_ERR_INVALID, "null argument");
    int devid = 0;
    MARS_TRY(ensure_device(&devid));
    MARS_HIP(hipMemGetInfo(free_bytes, total_bytes));
    return MARS_OK;
}

int mars_device_synchronize(void) {
    MARS_TRY(ensure_device(nullptr));
    MARS_HIP(hipDeviceSynchronize());
    return MARS_OK;
}

int mars_bench_queries(const mars_graph* g, mars_ctx* c, const float* dq, int64_t stride, int32_t n, float t_q,
                       const mars_retrieval_config* cfgs, int32_t n_cfg, double* lat_us, float* kern_us,
                       float* bfs_us, int32_t* n_res) {
    MARS_CHECK(g && c && dq && cfgs && lat_us && n >= 0 && (n_cfg == 1 || n_cfg == n) && stride >= g->g.d,
               MARS_ERR_INVALID, "bad benchmark arguments");
    mars_query_result out[64];
    for (int32_t i = 0; i < n; ++i) {
        mars_stats st{};
        int32_t nr = 0;
        const auto t0 = std::chrono::steady_clock::now();
        const int rc = query_impl(g, c, nullptr, dq + int64_t(i) * stride, t_q, &cfgs[n_cfg == 1 ? 0 : i], out, 64,
                                  &nr, &st);
        const auto t1 = std::chrono::steady_clock::now();
        if (rc != MARS_OK) return rc;
        lat_us[i] = std::chrono::duration<double, std::micro>(t1 - t0).count();
        if (kern_us) kern_us[i] = st.gpu_ms_similarity * 1000.0f;
        if (bfs_us) bfs_us[i] = (st.gpu_ms_total - st.gpu_ms_similarity) * 1000.0f;   // after the scan
        if (n_res) n_res[i] = nr;
    }
    return MARS_OK;
}

int mars_bench_queries_host(const mars_graph* g, mars_ctx* c, const float* hq, int64_t stride, int32_t n,
                            float t_q, const mars_retrieval_config* cfgs, int32_t n_cfg, double* lat_us,
                            int32_t* n_res) {
    MARS_CHECK(g && c && hq && cfgs && lat_us && n >= 0 && (n_cfg == 1 || n_cfg == n) && stride >= g->g.d,
               MARS_ERR_INVALID, "bad benchmark arguments");
    mars_query_result out[64];
    for (int32_t i = 0; i < n; ++i) {
        mars_stats st{};
        int32_t nr = 0;
        const auto t0 = std::chrono::steady_clock::now();
        const int rc = query_impl(g, c, hq + int64_t(i) * stride, nullptr, t_q, &cfgs[n_cfg == 1 ? 0 : i], out, 64,
                                  &nr, &st);
        const auto t1 = std::chrono::steady_clock::now();
        if (rc != MARS_OK) return rc;
        lat_us[i] = std::chrono::duration<double, std::micro>(t1 - t0).count();
        if (n_res) n_res[i] = nr;
    }
    return MARS_OK;
}

int mars_bench_serve(mars_graph* g, mars_ctx* cg, mars_ctx* ce, mars_serve_bench* b) {
    MARS_CHECK(g && cg && ce && b && cg != ce && b->n_global >= 0 && b->n_episode >= 0 && b->max_batch >= 1 &&
                   (b->n_global == 0 || (b->g_queries && b->g_arrival_us && b->gcfg && b->g_done_us && b->g_batch)) &&
                   (b->n_episode == 0 || (b->e_queries && b->e_arrival_us && b->ecfgs && b->e_done_us)) &&
                   b->n_insert >= 0 && (b->n_insert == 0 || (b->ins_emb && b->ins_mods && b->ins_ts &&
                   b->ins_stats && b->ins_start_us && b->insert_batch > 0 && b->insert_rate > 0.0)) &&
                   (!b->link_deferred || (b->knn_k >= 1 && b->knn_k <= 16 && b->max_link >= 1)),
               MARS_ERR_INVALID, "bad serving benchmark arguments");
    using clk = std::chrono::steady_clock;
    const auto start = clk::now();
    auto since = [&]() { return std::chrono::duration<double, std::micro>(clk::now() - start).count(); };
    // Arrival times are honoured to about a microsecond: sleep until shortly before (a
    // sleeping thread may wake tens of microseconds late), then spin. Latency is measured
    // from the arrival time, so a late wake-up would count against the query.
    auto wait_until = [&](double us) {
        const auto due = start + std::chrono::duration_cast<clk::duration>(std::chrono::duration<double, std::micro>(us));
        const auto early = due - std::chrono::microseconds(200);
        if (clk::now() < early) std::this_thread::sleep_until(early);
        while (clk::now() < due) std::this_thread::yield();
    };
    const int64_t D = g->g.d;
    const bool deferred = b->link_deferred != 0 && b->n_insert > 0;
    const int32_t n_base = __atomic_load_n(&g->g.n, __ATOMIC_ACQUIRE);
    const int32_t ib = b->n_insert > 0 ? b->insert_batch : 1;
    const int32_t nb_ins = (b->n_insert + ib - 1) / ib;
    std::atomic<int> ins_rc{MARS_OK};
    std::atomic<bool> writer_done{false};
    int ep_rc = MARS_OK;
    std::string ins_err, ep_err;
    // Deferred mode: the global server finds neighbour lists in its corpus passes and
    // hands them over; the writer applies every graph change (inserts and links), so
    // no thread waits on the graph mutex for another.
    struct LinkJob {
        int32_t first, count;
        std::vector<int32_t> knn;
    };
    std::mutex jobs_mu;
    std::deque<LinkJob> jobs;
    std::atomic<bool> server_done{false};
    int32_t linked_done = 0;                    // writer: nodes whose edges are linked
    auto apply_links = [&](bool drain_all) {
        for (;;) {
            LinkJob job;
            {
                std::lock_guard<std::mutex> lk(jobs_mu);
                if (jobs.empty()) return drain_all ? false : true;
                job = std::move(jobs.front());
                jobs.pop_front();
            }
            const int rc = mars_graph_link(g, job.first, job.count, b->knn_k, job.knn.data(), nullptr);
            if (rc != MARS_OK) {
                ins_err = mars_last_error();
                ins_rc.store(rc);
                return false;
            }
            const double t = since();
            linked_done += job.count;
            for (int32_t x = 0; x < nb_ins; ++x) {
                const int64_t last = std::min<int64_t>(int64_t(x + 1) * ib, b->n_insert);
                if (last <= linked_done && last > linked_done - job.count && b->ins_linked_us) b->ins_linked_us[x] = t;
            }
            if (!drain_all) return true;
        }
    };
    std::thread writer([&]() {
        for (int32_t j = 0; j < nb_ins && ins_rc.load() == MARS_OK; ++j) {
            const int64_t first = int64_t(j) * ib;
            const int32_t m = int32_t(std::min<int64_t>(ib, b->n_insert - first));
            const double due = double(first) / b->insert_rate * 1e6;
            if (deferred) {
                // link what the server found while waiting for this insert's time
                while (since() < due && ins_rc.load() == MARS_OK) {
                    bool any;
                    {
                        std::lock_guard<std::mutex> lk(jobs_mu);
                        any = !jobs.empty();
                    }
                    if (any) apply_links(false);
                    else wait_until(std::min(due, since() + 100.0));
                }
            }
            wait_until(due);
            b->ins_start_us[j] = since();
            const int rc = mars_graph_insert(g, m, b->ins_emb + first * D, b->ins_mods + first, b->ins_ts + first,
                                             b->ins_ep ? b->ins_ep + first : nullptr, deferred ? 0 : b->knn_k,
                                             nullptr, &b->ins_stats[j]);
            if (rc != MARS_OK) {
                ins_err = mars_last_error();
                ins_rc.store(rc);
            } else if (!deferred && b->ins_linked_us) {
                b->ins_linked_us[j] = b->ins_start_us[j] + b->ins_stats[j].linked_us;
            }
        }
        writer_done.store(true);
        // the rest of the links, until the server has handed over its last list
        while (deferred && ins_rc.load() == MARS_OK) {
            const bool done = server_done.load();
            bool any;
            {
                std::lock_guard<std::mutex> lk(jobs_mu);
                any = !jobs.empty();
            }
            if (any) apply_links(true);
            else if (done) break;
            else wait_until(since() + 100.0);
        }
    });
    std::thread episode([&]() {
        mars_query_result out[64];
        for (int32_t i = 0; i < b->n_episode && ep_rc == MARS_OK; ++i) {
            wait_until(b->e_arrival_us[i]);
            int32_t nr = 0;
            ep_rc = query_impl(g, ce, nullptr, b->e_queries + int64_t(i) * D, b->t_q, &b->ecfgs[i], out, 64, &nr,
                               nullptr);
            b->e_done_us[i] = since();
            if (ep_rc != MARS_OK) ep_err = mars_last_error();
        }
    });
    int rc = MARS_OK;
    const int32_t mb = b->max_batch;
    std::vector<mars_query_result> out(size_t(mb) * 64);
    std::vector<int32_t> nout(static_cast<size_t>(mb));
    std::vector<float> tq(static_cast<size_t>(mb), b->t_q);
    std::vector<int32_t> knn(size_t(std::max(b->max_link, 1)) * size_t(std::max(b->knn_k, 1)));
    b->g_uncertified = 0;
    b->g_overflow = 0;
    b->link_calls = 0;
    int32_t linked = n_base;                    // nodes below this id are linked
    const int32_t n_end = n_base + b->n_insert;
    int32_t i = 0;
    while (rc == MARS_OK) {
        const double now = since();
        const bool g_wait = i < b->n_global && b->g_arrival_us[i] <= now;
        int32_t n_pub = deferred ? __atomic_load_n(&g->g.n, __ATOMIC_ACQUIRE) : linked;
        // the insert that published node `linked` started before its nodes were published
        const bool l_wait = n_pub > linked &&
                            (g_wait || now - b->ins_start_us[(linked - n_base) / ib] >= b->link_wait_us);
        if (!g_wait && !l_wait) {
            const bool links_left = deferred && linked < n_end && ins_rc.load() == MARS_OK;
            if (i >= b->n_global && !links_left) break;
            if (i >= b->n_global && writer_done.load() && n_pub == linked &&
                __atomic_load_n(&g->g.n, __ATOMIC_ACQUIRE) == linked)
                break;                           // the writer stopped early (its error is reported)
            double next = now + 100.0;           // poll for published nodes
            if (i < b->n_global) next = std::min(next, b->g_arrival_us[i]);
            wait_until(next);
            continue;
        }
        int32_t j = i;
        if (g_wait) {
            j = i + 1;
            while (j < b->n_global && j - i < mb && b->g_arrival_us[j] <= now) ++j;
        }
        int32_t cnt = l_wait ? std::min(n_pub - linked, b->max_link) : 0;
        // with the int8 copy, up to 16 queries and neighbour searches share one int8 pass:
        // link at most what fits beside the global queries (the rest waits for the next call)
        if (cnt > 0 && cert_uses_int8(g->g) && j - i < 8 * kScan8MMaxA) cnt = std::min(cnt, 8 * kScan8MMaxA - (j - i));
        if (mb == 1 && !deferred) {
            rc = query_impl(g, cg, nullptr, b->g_queries + int64_t(i) * D, b->t_q, b->gcfg, out.data(), 64,
                            nout.data(), nullptr);
        } else {
            mars_batch_stats st{};
            rc = mars_query_global_batch_knn(g, cg, b->g_queries + int64_t(i) * D, j - i, tq.data(), b->gcfg,
                                             out.data(), 64, nout.data(), &st, linked, cnt, b->knn_k, knn.data());
            b->g_uncertified += st.uncertified + st.overflow;
            b->g_overflow += st.overflow;
        }
        const double done = since();
        for (int32_t x = i; x < j; ++x) {
            b->g_done_us[x] = done;
            b->g_batch[x] = j - i;
        }
        i = j;
        if (rc == MARS_OK && cnt > 0) {
            LinkJob job{linked, cnt, std::vector<int32_t>(knn.begin(), knn.begin() + size_t(cnt) * b->knn_k)};
            {
                std::lock_guard<std::mutex> lk(jobs_mu);
                jobs.push_back(std::move(job));
            }
            ++b->link_calls;
            linked += cnt;
        }
    }
    server_done.store(true);
    std::string err = rc != MARS_OK ? std::string(mars_last_error()) : std::string();
    episode.join();
    writer.join();
    if (rc != MARS_OK) return set_error(rc, "%s", err.c_str());
    if (ep_rc != MARS_OK) return set_error(ep_rc, "%s", ep_err.c_str());
    if (ins_rc.load() != MARS_OK) return set_error(ins_rc.load(), "%s", ins_err.c_str());
    return MARS_OK;
}

int mars_bench_stream(mars_graph* g, mars_ctx* c, mars_stream_bench* b) {
    MARS_CHECK(g && c && b && b->d_queries && b->cfgs && b->query_lat_us && b->n_queries >= 0 && b->query_rate > 0.0 &&
                   b->stride >= g->g.d && b->n_insert >= 0 && (b->n_insert == 0 || (b->ins_emb && b->ins_mods &&
                   b->ins_ts && b->ins_stats && b->insert_batch > 0 && b->insert_rate > 0.0)),
               MARS_ERR_INVALID, "bad streaming benchmark arguments");
    using clk = std::chrono::steady_clock;
    const auto start = clk::now();
    auto since = [&](clk::time_point t) { return std::chrono::duration<double, std::micro>(t - start).count(); };
    int ins_rc = MARS_OK;
    std::string ins_err;
    std::thread writer([&]() {
        const int32_t nb = (b->n_insert + b->insert_batch - 1) / b->insert_batch;
        const int64_t d = g->g.d;
        for (int32_t j = 0; j < nb && ins_rc == MARS_OK; ++j) {
            const int64_t first = int64_t(j) * b->insert_batch;
            const int32_t m = int32_t(std::min<int64_t>(b->insert_batch, b->n_insert - first));
            std::this_thread::sleep_until(start + std::chrono::duration_cast<clk::duration>(
                                                      std::chrono::duration<double>(double(first) / b->insert_rate)));
            if (b->ins_start_us) b->ins_start_us[j] = since(clk::now());
            ins_rc = mars_graph_insert(g, m, b->ins_emb + first * d, b->ins_mods + first, b->ins_ts + first,
                                       b->ins_ep ? b->ins_ep + first : nullptr, b->knn_k, nullptr, &b->ins_stats[j]);
            if (ins_rc != MARS_OK) ins_err = mars_last_error();
        }
    });
    int rc = MARS_OK;
    mars_query_result out[64];
    for (int32_t i = 0; i < b->n_queries && rc == MARS_OK; ++i) {
        std::this_thread::sleep_until(start + std::chrono::duration_cast<clk::duration>(
                                                  std::chrono::duration<double>(double(i) / b->query_rate)));
        mars_stats st{};
        int32_t nr = 0;
        const auto t0 = clk::now();
        rc = query_impl(g, c, nullptr, b->d_queries + int64_t(i) * b->stride, b->t_q, &b->cfgs[i], out, 64, &nr, &st);
        const auto t1 = clk::now();
        b->query_lat_us[i] = std::chrono::duration<double, std::micro>(t1 - t0).count();
        if (b->query_start_us) b->query_start_us[i] = since(t0);
    }
    writer.join();
    if (rc != MARS_OK) return rc;
    if (ins_rc != MARS_OK) return set_error(ins_rc, "%s", ins_err.c_str());
    return MARS_OK;
}

int mars_query_batch(const mars_graph* gh, mars_ctx* ch, const float* dq, int32_t Q, const float* h_tq,
                     const mars_retrieval_config* cfg, int32_t* out_ids, float* out_scores, mars_stats* stats) {
    const auto t0 = std::chrono::steady_clock::now();
    MARS_CHECK(gh && ch && dq && h_tq && cfg && out_ids && out_scores && Q > 0, MARS_ERR_INVALID, "bad arguments");
    const Graph& g = gh->g;
    Ctx& c = ch->c;
    MARS_CHECK(g.d == c.d, MARS_ERR_INVALID, "graph dim %d != context dim %d", g.d, c.d);
    MARS_CHECK(g.emb16 != nullptr, MARS_ERR_UNSUPPORTED, "batched scoring reads the fp16 corpus: enable it first");
    MARS_CHECK(batch_dim_supported(g.d), MARS_ERR_UNSUPPORTED, "batched scoring: embedding_dim %d unsupported", g.d);
    MARS_CHECK(cfg->top_k >= 1 && cfg->top_k <= 16, MARS_ERR_UNSUPPORTED, "batched top_k %d not in [1, 16]",
               cfg->top_k);
    MARS_TRY(use_device(c.device));
    const int32_t K = cfg->top_k;
    const int32_t n_live = __atomic_load_n(&g.n, __ATOMIC_ACQUIRE);
    int32_t nrr = 0, nqb = 0;
    int64_t rpr = 0;
    batch_grid(n_live, Q, false, &nrr, &nqb, &rpr);
    const int32_t kp = batch_kpart(K);
    MARS_TRY(ensure_batch_scratch(c, Q, int64_t(nqb) * nrr * 64 * kp));
    hipStream_t s = c.stream;
    MARS_HIP(hipMemcpyAsync(c.btq, h_tq, size_t(Q) * sizeof(float), hipMemcpyHostToDevice, s));
    MARS_TRY(launch_f32_to_f16_rows(dq, c.bq, int64_t(Q) * g.d, s));
    const bool timing = (c.flags & MARS_CTX_TIMING) != 0;
    if (timing) MARS_HIP(hipEventRecord(c.ev[0], s));
    BatchArgs a{};
    a.emb16 = g.emb16; a.n = n_live; a.d = g.d; a.qh = c.bq; a.q = Q; a.tq = c.btq; a.ts = g.ts; a.mods = g.mods;
    a.lambda = cfg->time_decay_lambda; a.mod_filter = cfg->modality_filter; a.k = K; a.q_plain = Q; a.self_base = -1;
    a.part = c.bpart; a.rows_per_range = rpr; a.n_rranges = nrr; a.n_qblocks = nqb;
    a.uniform_tq = std::all_of(h_tq, h_tq + Q, [&](float x) { return x == h_tq[0]; }) ? 1 : 0;
    MARS_TRY(launch_batch_topk(a, K, c.bout, s, timing ? c.ev[1] : nullptr));
    if (timing) MARS_HIP(hipEventRecord(c.ev[2], s));
    std::vector<uint64_t> keys(size_t(Q) * K);
    MARS_HIP(hipMemcpyAsync(keys.data(), c.bout, keys.size() * sizeof(uint64_t), hipMemcpyDeviceToHost, s));
    MARS_HIP(hipStreamSynchronize(s));
    for (size_t i = 0; i < keys.size(); ++i) {
        out_ids[i] = keys[i] == kEmptyKey ? -1 : key_id(keys[i]);
        out_scores[i] = keys[i] == kEmptyKey ? -FLT_MAX : key_score(keys[i]);
    }
    if (stats) {
        mars_stats st{};
        if (timing) {
            float ms = 0.0f;
            MARS_HIP(hipEventElapsedTime(&ms, c.ev[0], c.ev[1]));
            st.gpu_ms_similarity = ms;
            MARS_HIP(hipEventElapsedTime(&ms, c.ev[1], c.ev[2]));
            st.gpu_ms_topk = ms;
            MARS_HIP(hipEventElapsedTime(&ms, c.ev[0], c.ev[2]));
            st.gpu_ms_total = ms;
        }
        st.nodes_scanned = n_live;
        st.used_fp16 = 1;
        st.wall_us = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
        *stats = st;
    }
    return MARS_OK;
}

namespace mars {
namespace {

// Scratch of the multi-query int8 pass (k_split8, k_scan8m, k_cert_multi8), sized once for
// the most queries one pass takes.
int ensure_scan8m_scratch(Ctx& c) {
    if (c.m8part) return MARS_OK;
    const int32_t qmax = 8 * kScan8MMaxA;
    MARS_TRY(dmalloc(&c.m8part, size_t(qmax) * size_t(kScan8MPart)));
    MARS_TRY(dmalloc(&c.m8qa, size_t(kScan8MMaxA) * size_t(c.d / 64) * 1024));
    MARS_TRY(dmalloc(&c.m8qp, size_t(qmax) * 4));
    return MARS_OK;
}

// allow_int8 = false keeps the fp16 MFMA scan (the fallback of neighbour searches the int8
// certificate did not cover).
int global_batch_impl(const mars_graph* gh, mars_ctx* ch, const float* dq, int32_t Q, const float* h_tq,
                      const mars_retrieval_config* cfg, mars_query_result* out, int32_t cap, int32_t* n_out,
                      mars_batch_stats* stats, int32_t knn_first, int32_t knn_count, int32_t knn_k, int32_t* out_knn,
                      bool allow_int8, bool q1_route) {
    using clk = std::chrono::steady_clock;
    const auto t0 = clk::now();
    MARS_CHECK(gh && ch && Q >= 0 && knn_count >= 0 && Q + knn_count > 0, MARS_ERR_INVALID, "bad arguments");
    // a batch leaves no single query's BFS levels for edge-hit counting (a routed Q=1 query
    // sets them itself)
    struct HitReset {
        Ctx& c;
        bool on;
        ~HitReset() { if (on) c.hit_n = 0; }
    } hit_reset{ch->c, !q1_route};
    MARS_CHECK(Q == 0 || (dq && h_tq && cfg && n_out && cap >= 0 && (cap == 0 || out)), MARS_ERR_INVALID,
               "bad query arguments");
    const Graph& g = gh->g;
    Ctx& c = ch->c;
    MARS_CHECK(g.d == c.d, MARS_ERR_INVALID, "graph dim %d != context dim %d", g.d, c.d);
    const int32_t n_live = __atomic_load_n(&g.n, __ATOMIC_ACQUIRE);
    MARS_CHECK(n_live <= c.max_nodes, MARS_ERR_CAPACITY, "graph has %d nodes, context sized for %d", n_live,
               c.max_nodes);
    MARS_CHECK(n_live > 0, MARS_ERR_INVALID, "empty graph");
    if (knn_count > 0) {
        MARS_CHECK(knn_k >= 1 && knn_k <= 16 && out_knn, MARS_ERR_INVALID, "k-NN queries: knn_k %d, out_knn %p",
                   knn_k, static_cast<void*>(out_knn));
        MARS_CHECK(knn_first >= 0 && int64_t(knn_first) + knn_count <= n_live, MARS_ERR_INVALID,
                   "k-NN queries: nodes [%d, %lld) are not all published (%d nodes)", knn_first,
                   (long long)knn_first + knn_count, n_live);
        MARS_CHECK(g.emb16 != nullptr && batch_dim_supported(g.d), MARS_ERR_UNSUPPORTED,
                   "k-NN queries need the fp16 rows and embedding_dim in {256, 384, 512, 768}");
    }
    int32_t K = 0, hops = 0, rcap = 0;
    bool fp16 = false, glob_ok = false;
    float lambda = 0.0f;
    if (Q > 0) {
        MARS_CHECK(cfg->top_k > 0, MARS_ERR_INVALID, "top_k = %d", cfg->top_k);
        K = std::min(cfg->top_k, c.max_k);
        const bool scoped = episode_scoped_active(g, *cfg);
        hops = scoped ? 0 : std::max(0, cfg->bfs_max_hops);
        rcap = std::min(cfg->max_results_returned > 0 ? cfg->max_results_returned : K, c.res_cap);
        fp16 = (c.flags & MARS_CTX_USE_FP16) && g.emb16 != nullptr;
        const bool boost = g.ep_ids && cfg->query_episode_id >= 0 && cfg->episode_same_boost > 0.0f;
        lambda = cfg->time_decay_lambda;
        glob_ok = !scoped && K <= kMultiCand && !boost && lambda >= 0.0f && lambda <= FLT_MAX && hops < 255;
    }
    // Up to 16 queries and neighbour searches share one pass over the int8 copy (half the
    // fp16 rows' bytes) with certified exact candidates; larger batches take the fp16 MFMA
    // scan, whose one pass serves any number of queries.
    const int32_t na8 = ((glob_ok ? Q : 0) + knn_count + 7) / 8;
    const bool use8 = allow_int8 && na8 >= 1 && na8 <= kScan8MMaxA && !fp16 && cert_uses_int8(g);
    const bool batched = glob_ok && (use8 || (g.emb16 && g.nrm && batch_dim_supported(g.d)));
    MARS_TRY(use_device(c.device));
    mars_batch_stats st{};
    st.queries = Q;
    st.n_live = n_live;
    st.min_margin = FLT_MAX;
    std::vector<int32_t> q1;                    // queries the Q=1 path answers
    // A lone global query (no neighbour search) is cheaper on the Q=1 certified path (one
    // candidate scan and one kernel for the rest), and the results are the same.
    const bool lone = batched && Q == 1 && knn_count == 0 && !fp16 && cert_dim_supported(g.d) && !q1_route;
    const int32_t Qg = (batched && !lone) ? Q : 0;   // global queries in the shared scan
    const int32_t Qt = Qg + knn_count;               // + k-NN queries (plain dot products)
    bool knn_fallback = false;
    if (!batched) {
        st.whole_batch_q1 = Q > 0 ? 1 : 0;
        for (int32_t j = 0; j < Q; ++j) q1.push_back(j);
    }
    if (lone) {
        const uint32_t saved = c.flags;
        c.flags |= MARS_CTX_CERTIFIED;
        mars_stats s1{};
        const int rc = query_impl(gh, ch, nullptr, dq, h_tq[0], cfg, out, cap, &n_out[0], &s1, n_live);
        c.flags = saved;
        MARS_TRY(rc);
        if (s1.seeds_certified) ++st.batched; else ++st.uncertified;
        st.candidate_rows = cert_uses_int8(g) ? 8 : 16;
        st.q1_us = 0.0;
        st.wall_us = std::chrono::duration<double, std::micro>(clk::now() - t0).count();
        if (stats) *stats = st;
        return MARS_OK;
    }
    if (Qt > 0) {
        st.candidate_rows = use8 ? 8 : 16;
        if (Qg > 0 || use8) MARS_TRY(ensure_multi_scratch(c, use8 ? Qt : Qg, std::max(rcap, 1)));
        if (knn_count > c.mknn_cap) {
            dfree(c.mknn);
            c.mknn_cap = 0;
            MARS_TRY(dmalloc(&c.mknn, size_t(knn_count) * 16));
            c.mknn_cap = knn_count;
        }
        hipStream_t s = c.stream;
        const bool timing = (c.flags & MARS_CTX_TIMING) != 0;
        int32_t seed_stride = kMultiCand;
        std::vector<int32_t> knn_status(static_cast<size_t>(use8 ? knn_count : 0));
        // one query time for every global query: passed by value (no copy)
        const bool uniform = Qg == 0 || std::all_of(h_tq, h_tq + Qg, [&](float x) { return x == h_tq[0]; });
        const float tq0 = Qg > 0 ? h_tq[0] : 0.0f;
        if (use8) {
            MARS_TRY(ensure_scan8m_scratch(c));
            MARS_TRY(ensure_batch_scratch(c, std::max(Qg, 1), 0));              // query times
            if (!uniform) MARS_HIP(hipMemcpyAsync(c.btq, h_tq, size_t(Qg) * sizeof(float), hipMemcpyHostToDevice, s));
            const float* tqd = uniform ? nullptr : c.btq;
            const float* qplain = g.emb + int64_t(knn_first) * g.d;
            Split8Args sp{};
            sp.q_glob = dq; sp.q_plain = qplain; sp.nq = Qt; sp.n_glob = Qg; sp.d = g.d; sp.na = na8;
            sp.nrm8 = g.nrm8; sp.qa = c.m8qa; sp.qp = c.m8qp;
            MARS_TRY(launch_split8(sp, s));
            if (timing) MARS_HIP(hipEventRecord(c.ev[0], s));
            int32_t rpw = 0, nwg = 0;
            scan_grid(n_live, kTargetWgI8, &rpw, &nwg);
            Scan8MArgs sa{};
            sa.emb8 = g.emb8; sa.meta8 = g.meta8; sa.n = n_live; sa.d = g.d; sa.ts = g.ts; sa.mods = g.mods;
            sa.qa = c.m8qa; sa.qp = c.m8qp; sa.tq = tqd; sa.tq_value = tq0; sa.lambda = lambda;
            sa.mod_filter = Qg > 0 ? cfg->modality_filter : -1; sa.nq = Qt; sa.n_glob = Qg;
            sa.self_base = knn_first; sa.part = c.m8part; sa.num_wg = nwg;
            MARS_TRY(launch_scan8m(sa, na8, s));
            if (timing) MARS_HIP(hipEventRecord(c.ev[1], s));
            CertMArgs ca{};
            ca.part = c.m8part; ca.n_lists = nwg; ca.q = Qt; ca.n_glob = Qg; ca.q_glob = dq; ca.q_plain = qplain;
            ca.d = g.d; ca.emb = g.emb; ca.ts = g.ts; ca.mods = g.mods; ca.tq = tqd; ca.tq_value = tq0; ca.lambda = lambda;
            ca.mod_filter = sa.mod_filter; ca.qp = c.m8qp; ca.nrm8 = g.nrm8; ca.k = std::max(K, 1);
            ca.knn_k = std::max(knn_k, 1); ca.seeds = c.mseed; ca.status = c.mstat; ca.margin = c.mmargin;
            ca.knn_out = c.mknn;
            MARS_TRY(launch_cert_multi8(ca, s));
            if (timing) MARS_HIP(hipEventRecord(c.ev[2], s));
            seed_stride = 64;
        } else {
            int32_t nrr = 0, nqb = 0;
            int64_t rpr = 0;
            batch_grid(n_live, Qt, Qg == 0, &nrr, &nqb, &rpr);   // the k-NN queries alone: plain
            const int32_t kp = batch_kpart(kMultiCand);
            MARS_TRY(ensure_batch_scratch(c, Qt, int64_t(nqb) * nrr * 64 * kp));
            if (Qg > 0) {
                MARS_HIP(hipMemcpyAsync(c.btq, h_tq, size_t(Qg) * sizeof(float), hipMemcpyHostToDevice, s));
                MARS_TRY(launch_f32_to_f16_rows(dq, c.bq, int64_t(Qg) * g.d, s));
                MARS_TRY(launch_query_norms(dq, c.bq, Qg, g.d, c.mqn, s));
            }
            if (knn_count > 0)     // the k-NN queries are the nodes' own fp16 rows
                MARS_HIP(hipMemcpyAsync(c.bq + int64_t(Qg) * g.d, g.emb16 + int64_t(knn_first) * g.d,
                                        size_t(knn_count) * size_t(g.d) * sizeof(__half), hipMemcpyDeviceToDevice, s));
            if (timing) MARS_HIP(hipEventRecord(c.ev[0], s));
            BatchArgs b{};
            b.emb16 = g.emb16; b.n = n_live; b.d = g.d; b.qh = c.bq; b.q = Qt; b.tq = c.btq; b.ts = g.ts;
            b.mods = g.mods; b.lambda = Qg > 0 ? lambda : 0.0f; b.mod_filter = Qg > 0 ? cfg->modality_filter : -1;
            b.k = kMultiCand; b.q_plain = Qg; b.self_base = knn_count > 0 ? knn_first : -1; b.part = c.bpart;
            b.rows_per_range = rpr; b.n_rranges = nrr; b.n_qblocks = nqb;
            b.uniform_tq = (Qg == 0 || std::all_of(h_tq, h_tq + Qg, [&](float x) { return x == h_tq[0]; })) ? 1 : 0;
            MARS_TRY(launch_batch_topk(b, kMultiCand, c.bout, s));
            if (timing) MARS_HIP(hipEventRecord(c.ev[1], s));
            if (knn_count > 0)
                MARS_TRY(launch_knn_rerank(g.emb, knn_first, knn_count, g.d, c.bout + int64_t(Qg) * kMultiCand,
                                           kMultiCand, knn_k, c.mknn, s));
            if (Qg > 0) {
                SeedArgs sa{};
                sa.emb = fp16 ? static_cast<const void*>(g.emb16) : static_cast<const void*>(g.emb);
                sa.fp16 = fp16 ? 1 : 0; sa.d = g.d; sa.ts = g.ts; sa.mods = g.mods; sa.queries = dq; sa.tq = c.btq;
                sa.lambda = lambda; sa.mod_filter = cfg->modality_filter; sa.q = Qg; sa.k = K; sa.cand = c.bout;
                sa.qn = c.mqn; sa.nrm = g.nrm; sa.seeds = c.mseed; sa.status = c.mstat; sa.margin = c.mmargin;
                MARS_TRY(launch_multi_seed(sa, s));
            }
            if (timing) MARS_HIP(hipEventRecord(c.ev[2], s));
        }
        std::vector<float> margin(static_cast<size_t>(Qg));
        if (Qg > 0) {
            MultiArgs m{};
            m.ro = g.ro; m.col = g.col; m.mods = g.mods; m.n_live = n_live; m.hops = hops;
            m.hop_decay = cfg->bfs_score_decay; m.k = K; m.rcap = rcap; m.q = Qg; m.seeds = c.mseed;
            m.seed_stride = seed_stride;
            m.status = c.mstat; m.info = c.minfo; m.vlist = c.mvlist; m.vhop = c.mvhop; m.vpar = c.mvpar;
            m.vro = c.mvro; m.vfin = c.mvfin; m.vscore = c.mvscore;
            m.res = static_cast<ResultHeader*>(c.d_mres);
            m.rec = reinterpret_cast<mars_query_result*>(m.res + Qg);
            MARS_TRY(launch_multi_bfs(m, s));
            VisitScoreArgs va{};
            va.emb = fp16 ? static_cast<const void*>(g.emb16) : static_cast<const void*>(g.emb);
            va.fp16 = fp16 ? 1 : 0; va.d = g.d; va.ts = g.ts; va.mods = g.mods; va.queries = dq;
            va.tq = (use8 && uniform) ? nullptr : c.btq; va.t_q_value = tq0; va.lambda = lambda;
            va.mod_filter = cfg->modality_filter; va.q = Qg;
            va.status = c.mstat; va.info = c.minfo; va.vlist = c.mvlist; va.vfin = c.mvfin;
            MARS_TRY(launch_visit_scores(va, s));
            if (q1_route && !timing) {                  // the last kernel stores the completion word
                m.done = c.d_done;
                m.seq = next_seq(c);
            }
            MARS_TRY(launch_multi_select(m, s));
            if (timing) MARS_HIP(hipEventRecord(c.ev[3], s));
            if (!q1_route)
                MARS_HIP(hipMemcpyAsync(margin.data(), c.mmargin, size_t(Qg) * sizeof(float), hipMemcpyDeviceToHost, s));
        } else if (timing) {
            MARS_HIP(hipEventRecord(c.ev[3], s));
        }
        if (knn_count > 0) {
            MARS_HIP(hipMemcpyAsync(out_knn, c.mknn, size_t(knn_count) * size_t(knn_k) * sizeof(int32_t),
                                    hipMemcpyDeviceToHost, s));
            if (use8)
                MARS_HIP(hipMemcpyAsync(knn_status.data(), c.mstat + Qg, size_t(knn_count) * sizeof(int32_t),
                                        hipMemcpyDeviceToHost, s));
        }
        if (q1_route && !timing && Qg == 1) MARS_TRY(wait_done(c, c.seq, s));
        else MARS_HIP(hipStreamSynchronize(s));
        for (const int32_t x : knn_status) knn_fallback = knn_fallback || x != kMultiOk;
        if (Qg > 0) {
            const auto* hdr = static_cast<const ResultHeader*>(c.h_mres);
            const auto* rec = reinterpret_cast<const mars_query_result*>(hdr + Qg);
            for (int32_t j = 0; j < Qg; ++j) {
                const ResultHeader h = hdr[j];
                if (h.count < 0) {
                    if (h.visited == kMultiOverflow) ++st.overflow;
                    else ++st.uncertified;
                    q1.push_back(j);
                    continue;
                }
                const int32_t nw = std::min(h.count, cap);
                if (nw > 0)
                    std::memcpy(out + int64_t(j) * cap, rec + int64_t(j) * rcap, size_t(nw) * sizeof(mars_query_result));
                n_out[j] = h.count;
                ++st.batched;
                st.min_margin = std::min(st.min_margin, margin[size_t(j)]);
            }
        }
        if (timing) {
            float ms = 0.0f;
            MARS_HIP(hipEventElapsedTime(&ms, c.ev[0], c.ev[1]));
            st.gpu_ms_scan = ms;
            MARS_HIP(hipEventElapsedTime(&ms, c.ev[1], c.ev[2]));
            st.gpu_ms_seeds = ms;
            MARS_HIP(hipEventElapsedTime(&ms, c.ev[2], c.ev[3]));
            st.gpu_ms_bfs = ms;
            MARS_HIP(hipEventElapsedTime(&ms, c.ev[0], c.ev[3]));
            st.gpu_ms_total = ms;
        }
    }
    if (knn_fallback) {
        // a neighbour search the int8 certificate did not cover: all of them again on the
        // fp16 scan with exact rescoring
        mars_batch_stats s2{};
        MARS_TRY(global_batch_impl(gh, ch, nullptr, 0, nullptr, nullptr, nullptr, 0, nullptr, &s2, knn_first,
                                   knn_count, knn_k, out_knn, false, false));
        st.candidate_rows = 24;
    }
    const auto t1 = clk::now();
    for (const int32_t j : q1)
        MARS_TRY(query_impl(gh, ch, nullptr, dq + int64_t(j) * g.d, h_tq[j], cfg, cap ? out + int64_t(j) * cap : nullptr,
                            cap, &n_out[j], nullptr, n_live, false));
    const auto t2 = clk::now();
    st.q1_us = std::chrono::duration<double, std::micro>(t2 - t1).count();
    st.wall_us = std::chrono::duration<double, std::micro>(t2 - t0).count();
    if (stats) *stats = st;
    return MARS_OK;
}

}  // namespace
}  // namespace mars

int mars_query_global_batch(const mars_graph* gh, mars_ctx* ch, const float* dq, int32_t Q, const float* h_tq,
                            const mars_retrieval_config* cfg, mars_query_result* out, int32_t cap,
                            int32_t* n_out, mars_batch_stats* stats) {
    MARS_CHECK(Q > 0, MARS_ERR_INVALID, "bad arguments");
    return global_batch_impl(gh, ch, dq, Q, h_tq, cfg, out, cap, n_out, stats, 0, 0, 0, nullptr, true);
}

int mars_query_global_batch_knn(const mars_graph* gh, mars_ctx* ch, const float* dq, int32_t Q, const float* h_tq,
                                const mars_retrieval_config* cfg, mars_query_result* out, int32_t cap,
                                int32_t* n_out, mars_batch_stats* stats, int32_t knn_first, int32_t knn_count,
                                int32_t knn_k, int32_t* out_knn) {
    return global_batch_impl(gh, ch, dq, Q, h_tq, cfg, out, cap, n_out, stats, knn_first, knn_count, knn_k, out_knn,
                             true);
}


int mars_graph_read_ceiling(const mars_graph* gh, int32_t fp16, int32_t reps, double* gbps) {
    MARS_CHECK(gh && gbps && reps > 0, MARS_ERR_INVALID, "bad arguments");
    const Graph& g = gh->g;
    const void* rows = fp16 ? static_cast<const void*>(g.emb16) : static_cast<const void*>(g.emb);
    MARS_CHECK(rows != nullptr, MARS_ERR_UNSUPPORTED, "no %s rows", fp16 ? "fp16" : "fp32");
    const int32_t n = __atomic_load_n(&g.n, __ATOMIC_ACQUIRE);
    const int64_t bytes = int64_t(n) * g.d * (fp16 ? 2 : 4) / 16 * 16;
    MARS_CHECK(bytes > 0, MARS_ERR_INVALID, "empty graph");
    MARS_TRY(use_device(g.device));
    return time_read(bytes, reps, "read ceiling", [&](int32_t wg, uint32_t* out, hipStream_t s) {
        return launch_read_rows(rows, bytes, wg, 0x9E3779B9u, out, s);
    }, gbps);
}

int mars_graph_read_pattern(const mars_graph* gh, int32_t pattern, int32_t reps, double* gbps) {
    MARS_CHECK(gh && gbps && reps > 0, MARS_ERR_INVALID, "bad arguments");
    MARS_CHECK(pattern >= 0 && pattern <= 3, MARS_ERR_INVALID, "read pattern %d not in [0, 3]", pattern);
    if (pattern == 0) return mars_graph_read_ceiling(gh, 1, reps, gbps);
    const Graph& g = gh->g;
    if (pattern == 3) {
        MARS_CHECK(g.emb8 != nullptr, MARS_ERR_UNSUPPORTED, "no int8 rows");
        const int64_t bytes = int64_t(__atomic_load_n(&g.n, __ATOMIC_ACQUIRE)) * g.d / 16 * 16;
        MARS_CHECK(bytes > 0, MARS_ERR_INVALID, "empty graph");
        MARS_TRY(use_device(g.device));
        return time_read(bytes, reps, "read pattern", [&](int32_t wg, uint32_t* out, hipStream_t s) {
            return launch_read_rows(g.emb8, bytes, wg, 0x9E3779B9u, out, s);
        }, gbps);
    }
    MARS_CHECK(g.emb16 != nullptr, MARS_ERR_UNSUPPORTED, "no fp16 rows");
    MARS_CHECK(g.d % 32 == 0, MARS_ERR_UNSUPPORTED, "fragment pattern: embedding_dim %d not a multiple of 32", g.d);
    const int32_t n = __atomic_load_n(&g.n, __ATOMIC_ACQUIRE);
    const int64_t rows16 = int64_t(n) / 16 * 16;
    MARS_CHECK(rows16 > 0, MARS_ERR_INVALID, "fewer than 16 rows");
    MARS_TRY(use_device(g.device));
    const int64_t bytes = rows16 * g.d * 2;
    return time_read(bytes, reps, "read pattern", [&](int32_t wg, uint32_t* out, hipStream_t s) {
        return launch_read_frags(g.emb16, rows16, g.d * 2, wg, pattern == 2, 0x9E3779B9u, out, s);
    }, gbps);
}

namespace {

// The k-NN lists of the nodes the builder's certificate did not cover (cert[i] == 0 for
// node first + i), found again by exact fp32 scans over all rows (the global query path with
// no decay, no BFS and k + 1 seeds, the node itself dropped). Records the counts.
int knn_rescan_uncertified(mars_graph* gh, int32_t k, int64_t first, const std::vector<int32_t>& cert,
                           int32_t* nbrs, bool rescan) {
    Graph& g = gh->g;
    std::vector<int64_t> todo;
    for (size_t i = 0; i < cert.size(); ++i)
        if (!cert[i]) todo.push_back(first + int64_t(i));
    g.knn_uncertified = int64_t(todo.size());
    g.knn_rescanned = 0;
    if (todo.empty() || !rescan) return MARS_OK;
    mars_ctx* ctx = nullptr;
    MARS_TRY(mars_ctx_create(g.cap_n, g.d, 32, 0, &ctx));
    mars_retrieval_config cfg;
    mars_config_default(&cfg);
    cfg.top_k = k + 1;
    cfg.bfs_max_hops = 0;
    cfg.time_decay_lambda = 0.0f;
    cfg.max_results_returned = k + 1;
    std::vector<mars_query_result> res(static_cast<size_t>(k) + 1);
    int rc = MARS_OK;
    for (const int64_t node : todo) {
        int32_t nr = 0;
        rc = query_impl(gh, ctx, nullptr, g.emb + node * g.d, 0.0f, &cfg, res.data(), k + 1, &nr, nullptr);
        if (rc != MARS_OK) break;
        int32_t* row = nbrs + (node - first) * k;
        int32_t w = 0;
        for (int32_t j = 0; j < std::min(nr, k + 1) && w < k; ++j)
            if (res[size_t(j)].node_id != node) row[w++] = res[size_t(j)].node_id;
        for (; w < k; ++w) row[w] = -1;
        ++g.knn_rescanned;
    }
    (void)mars_ctx_destroy(ctx);
    return rc;
}

}  // namespace

int mars_graph_knn_report(const mars_graph* gh, int64_t* uncertified, int64_t* rescanned) {
    MARS_CHECK(gh && uncertified && rescanned, MARS_ERR_INVALID, "null argument");
    *uncertified = gh->g.knn_uncertified;
    *rescanned = gh->g.knn_rescanned;
    return MARS_OK;
}

int mars_graph_knn_blocked(mars_graph* gh, int32_t k, int32_t block_rows, int32_t* nbrs) {
    MARS_CHECK(gh && block_rows > 0, MARS_ERR_INVALID, "k-NN: bad arguments (block_rows=%d)", block_rows);
    const int64_t n = gh->g.n;
    return mars_graph_knn_blocks(gh, k, block_rows, 0, int32_t((n + block_rows - 1) / block_rows), nbrs);
}

int mars_graph_knn_blocks(mars_graph* gh, int32_t k, int32_t block_rows, int32_t first_block, int32_t n_blocks,
                          int32_t* nbrs) {
    MARS_CHECK(gh && nbrs && k >= 1 && k <= 16 && block_rows > 0 && first_block >= 0 && n_blocks >= 0,
               MARS_ERR_INVALID, "k-NN: bad arguments (k=%d, block_rows=%d, blocks %d + %d)", k, block_rows,
               first_block, n_blocks);
    std::lock_guard<std::mutex> lock(gh->mu);
    Graph& g = gh->g;
    MARS_CHECK(g.emb16 != nullptr, MARS_ERR_UNSUPPORTED, "k-NN reads the fp16 corpus: enable it first");
    MARS_CHECK(batch_dim_supported(g.d), MARS_ERR_UNSUPPORTED, "k-NN: embedding_dim %d unsupported", g.d);
    MARS_TRY(use_device(g.device));
    constexpr int32_t kChunk = 1024;                 // queries per launch (16 query blocks)
    constexpr int32_t kCand = 16;
    const int64_t B = std::min<int64_t>(block_rows, g.n);
    // nodes [lo, hi): the requested blocks
    const int64_t lo = std::min<int64_t>(int64_t(first_block) * block_rows, g.n);
    const int64_t hi = std::min<int64_t>(lo + int64_t(n_blocks) * block_rows, g.n);
    if (hi <= lo) return MARS_OK;
    int32_t nrr = 0, nqb = 0;
    int64_t rpr = 0;
    batch_grid(B, kChunk, true, &nrr, &nqb, &rpr);   // the largest block sizes the scratch
    float* tq = nullptr; uint64_t* part = nullptr; uint64_t* cand = nullptr; int32_t* dn = nullptr;
    int32_t* cert = nullptr;
    hipStream_t s = nullptr;
    int rc = MARS_OK;
    auto cleanup = [&]() {
        dfree(tq); dfree(part); dfree(cand); dfree(dn); dfree(cert);
        if (s) (void)hipStreamDestroy(s);
    };
    if ((rc = dmalloc(&tq, kChunk)) || (rc = dmalloc(&part, size_t(nqb) * nrr * 64 * kCand)) ||
        (rc = dmalloc(&cand, size_t(kChunk) * kCand)) || (rc = dmalloc(&dn, size_t(hi - lo) * k)) ||
        (rc = dmalloc(&cert, size_t(hi - lo)))) {
        cleanup();
        return rc;
    }
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipMemsetAsync(tq, 0, kChunk * sizeof(float), s);
    if (e == hipSuccess) e = hipMemsetAsync(cert, 0, size_t(hi - lo) * sizeof(int32_t), s);
    if (e != hipSuccess) { cleanup(); return set_error(MARS_ERR_HIP, "k-NN setup: %s", hipGetErrorString(e)); }
    // block [r0, r1): rows, queries and candidate ids relative to r0
    for (int64_t r0 = lo; r0 < hi && rc == MARS_OK; r0 += B) {
        const int64_t nb = std::min<int64_t>(B, g.n - r0);
        batch_grid(nb, kChunk, true, &nrr, &nqb, &rpr);
        for (int64_t q0 = 0; q0 < nb && rc == MARS_OK; q0 += kChunk) {
            const int32_t q = int32_t(std::min<int64_t>(kChunk, nb - q0));
            BatchArgs a{};
            a.emb16 = g.emb16 + r0 * g.d; a.n = nb; a.d = g.d; a.qh = g.emb16 + (r0 + q0) * g.d; a.q = q; a.tq = tq;
            a.ts = g.ts + r0; a.mods = g.mods + r0; a.lambda = 0.0f; a.mod_filter = -1; a.k = kCand; a.q_plain = 0; a.self_base = q0;
            a.part = part; a.uniform_tq = 1;
            a.rows_per_range = rpr; a.n_rranges = nrr; a.n_qblocks = (q + 63) / 64;
            rc = launch_batch_topk(a, kCand, cand, s);
            if (rc == MARS_OK)
                rc = launch_knn_rerank(g.emb + r0 * g.d, q0, q, g.d, cand, kCand, k, dn + (r0 - lo + q0) * k, s,
                                       g.nrm, g.nrm ? cert + (r0 - lo + q0) : nullptr);
        }
    }
    std::vector<int32_t> hcert(size_t(hi - lo), 0);
    if (rc == MARS_OK) {
        e = hipStreamSynchronize(s);
        if (e == hipSuccess) e = hipMemcpy(nbrs, dn, size_t(hi - lo) * k * sizeof(int32_t), hipMemcpyDeviceToHost);
        if (e == hipSuccess) e = hipMemcpy(hcert.data(), cert, hcert.size() * sizeof(int32_t), hipMemcpyDeviceToHost);
        if (e != hipSuccess) rc = set_error(MARS_ERR_HIP, "k-NN: %s", hipGetErrorString(e));
    }
    cleanup();
    if (rc == MARS_OK && B < g.n) {                      // block-relative ids -> node ids
        for (int64_t i = lo; i < hi; ++i) {
            const int32_t off = int32_t(i / B * B);
            for (int32_t j = 0; j < k; ++j)
                if (nbrs[(i - lo) * k + j] >= 0) nbrs[(i - lo) * k + j] += off;
        }
    }
    // all pairs: the nodes the certificate missed are scanned again exactly; within blocks
    // they are only counted (an exact scan would search beyond the block)
    if (rc == MARS_OK) rc = knn_rescan_uncertified(gh, k, lo, hcert, nbrs, B >= g.n);
    return rc;
}

int mars_graph_knn_range(mars_graph* gh, int32_t k, int32_t first, int32_t count, int32_t* nbrs) {
    MARS_CHECK(gh && nbrs && k >= 1 && k <= 16 && first >= 0 && count >= 0, MARS_ERR_INVALID,
               "k-NN range: bad arguments (k=%d, first=%d, count=%d)", k, first, count);
    std::lock_guard<std::mutex> lock(gh->mu);
    Graph& g = gh->g;
    MARS_CHECK(g.emb16 != nullptr, MARS_ERR_UNSUPPORTED, "k-NN reads the fp16 corpus: enable it first");
    MARS_CHECK(batch_dim_supported(g.d), MARS_ERR_UNSUPPORTED, "k-NN: embedding_dim %d unsupported", g.d);
    MARS_CHECK(int64_t(first) + count <= g.n, MARS_ERR_INVALID, "k-NN range: [%d, %lld) beyond the %d nodes", first,
               (long long)first + count, g.n);
    if (count == 0) return MARS_OK;
    MARS_TRY(use_device(g.device));
    constexpr int32_t kChunk = 1024;                 // queries per launch
    constexpr int32_t kCand = 16;
    const int64_t n = g.n;
    int32_t nrr = 0, nqb = 0;
    int64_t rpr = 0;
    batch_grid(n, kChunk, true, &nrr, &nqb, &rpr);
    float* tq = nullptr; uint64_t* part = nullptr; uint64_t* cand = nullptr; int32_t* dn = nullptr;
    int32_t* cert = nullptr;
    hipStream_t s = nullptr;
    int rc = MARS_OK;
    auto cleanup = [&]() {
        dfree(tq); dfree(part); dfree(cand); dfree(dn); dfree(cert);
        if (s) (void)hipStreamDestroy(s);
    };
    if ((rc = dmalloc(&tq, kChunk)) || (rc = dmalloc(&part, size_t(nqb) * nrr * 64 * kCand)) ||
        (rc = dmalloc(&cand, size_t(kChunk) * kCand)) || (rc = dmalloc(&dn, size_t(count) * k)) ||
        (rc = dmalloc(&cert, size_t(count)))) {
        cleanup();
        return rc;
    }
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipMemsetAsync(tq, 0, kChunk * sizeof(float), s);
    if (e == hipSuccess) e = hipMemsetAsync(cert, 0, size_t(count) * sizeof(int32_t), s);
    if (e != hipSuccess) { cleanup(); return set_error(MARS_ERR_HIP, "k-NN range setup: %s", hipGetErrorString(e)); }
    // queries [q0, q0 + q) against every node; the query's own id is excluded
    for (int64_t q0 = first; q0 < int64_t(first) + count && rc == MARS_OK; q0 += kChunk) {
        const int32_t q = int32_t(std::min<int64_t>(kChunk, int64_t(first) + count - q0));
        BatchArgs a{};
        a.emb16 = g.emb16; a.n = n; a.d = g.d; a.qh = g.emb16 + q0 * g.d; a.q = q; a.tq = tq;
        a.ts = g.ts; a.mods = g.mods; a.lambda = 0.0f; a.mod_filter = -1; a.k = kCand; a.q_plain = 0; a.self_base = q0;
        a.part = part; a.uniform_tq = 1;
        a.rows_per_range = rpr; a.n_rranges = nrr; a.n_qblocks = (q + 63) / 64;
        rc = launch_batch_topk(a, kCand, cand, s);
        if (rc == MARS_OK)
            rc = launch_knn_rerank(g.emb, q0, q, g.d, cand, kCand, k, dn + (q0 - first) * k, s, g.nrm,
                                   g.nrm ? cert + (q0 - first) : nullptr);
    }
    std::vector<int32_t> hcert(static_cast<size_t>(count), 0);
    if (rc == MARS_OK) {
        e = hipStreamSynchronize(s);
        if (e == hipSuccess) e = hipMemcpy(nbrs, dn, size_t(count) * k * sizeof(int32_t), hipMemcpyDeviceToHost);
        if (e == hipSuccess) e = hipMemcpy(hcert.data(), cert, hcert.size() * sizeof(int32_t), hipMemcpyDeviceToHost);
        if (e != hipSuccess) rc = set_error(MARS_ERR_HIP, "k-NN range: %s", hipGetErrorString(e));
    }
    cleanup();
    if (rc == MARS_OK) rc = knn_rescan_uncertified(gh, k, first, hcert, nbrs, true);
    return rc;
}

int mars_graph_knn(mars_graph* gh, int32_t k, int32_t* nbrs) {
    MARS_CHECK(gh, MARS_ERR_INVALID, "null graph");
    return mars_graph_knn_blocked(gh, k, std::max<int32_t>(1, gh->g.n), nbrs);
}

int mars_ctx_last_scores(mars_ctx* ch, float* h, int64_t n) {
    MARS_CHECK(ch && h, MARS_ERR_INVALID, "null argument");
    Ctx& c = ch->c;
    MARS_CHECK(n <= c.last_n && n >= 0, MARS_ERR_INVALID, "asked %lld scores, last global query had %d",
               (long long)n, c.last_n);
    MARS_TRY(use_device(c.device));
    MARS_HIP(hipStreamSynchronize(c.stream));
    MARS_HIP(hipMemcpy(h, c.fin, size_t(n) * sizeof(float), hipMemcpyDeviceToHost));
    return MARS_OK;
}

int mars_ctx_last_seeds(mars_ctx* ch, int32_t* idx, float* val, int32_t k, int32_t* k_out) {
    MARS_CHECK(ch && idx && val && k_out, MARS_ERR_INVALID, "null argument");
    Ctx& c = ch->c;
    MARS_TRY(use_device(c.device));
    MARS_HIP(hipStreamSynchronize(c.stream));
    const int32_t n = std::min(k, c.last_k);
    if (n > 0) {
        MARS_HIP(hipMemcpy(idx, c.seed_idx, size_t(n) * sizeof(int32_t), hipMemcpyDeviceToHost));
        MARS_HIP(hipMemcpy(val, c.seed_val, size_t(n) * sizeof(float), hipMemcpyDeviceToHost));
    }
    *k_out = c.last_k;
    return MARS_OK;
}

int mars_ctx_last_phases(mars_ctx* ch, double* us, int32_t n) {
    MARS_CHECK(ch && us && n >= 0 && n <= 6, MARS_ERR_INVALID, "bad arguments");
    MARS_TRY(use_device(ch->c.device));
    MARS_HIP(hipStreamSynchronize(ch->c.stream));
    const uint64_t* t = ch->c.h_stamps;
    const uint64_t* p = ch->c.last_certified ? t + 4 : t;     // certified: 7 stamps from t[4]
    const int32_t np = ch->c.last_certified ? 6 : 3;
    for (int32_t i = 0; i < n; ++i) us[i] = i < np ? double(p[i + 1] - p[i]) * 0.01 : 0.0;   // 100 MHz counter
    return MARS_OK;
}

int mars_ctx_last_visited(mars_ctx* ch, int32_t* ids, int32_t* hops, float* scores, int32_t cap, int32_t* n_out) {
    MARS_CHECK(ch && n_out && cap >= 0, MARS_ERR_INVALID, "null argument");
    Ctx& c = ch->c;
    MARS_TRY(use_device(c.device));
    MARS_HIP(hipStreamSynchronize(c.stream));
    const int32_t n = std::min(cap, c.last_visited);
    if (n > 0) {
        if (ids) MARS_HIP(hipMemcpy(ids, c.vlist, size_t(n) * sizeof(int32_t), hipMemcpyDeviceToHost));
        if (hops) MARS_HIP(hipMemcpy(hops, c.vhop, size_t(n) * sizeof(int32_t), hipMemcpyDeviceToHost));
        if (scores) MARS_HIP(hipMemcpy(scores, c.vscore, size_t(n) * sizeof(float), hipMemcpyDeviceToHost));
    }
    *n_out = c.last_visited;
    return MARS_OK;
}

}  // extern "C"
