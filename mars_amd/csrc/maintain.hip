// ============================================================================
//  maintain.hip — importance, novelty and edge-hit maintenance on the device
//  graph (reference: src/memory_cuda.cu:1466-1658, include/memory_cuda.cuh:234-270).
//
//  Importance. One fp32 per node, 1.0 at init (nodes inserted later also start at
//  1.0). An update decays every node and then boosts the listed ids, in one launch:
//  each workgroup owns a contiguous slice of nodes, decays it, and after a barrier
//  applies the boosts that fall in its slice, so no node is touched by two
//  workgroups. Arithmetic is the reference's, operation by operation: v * retain
//  rounded, then fminf(v + boost, max) rounded (no contraction into an FMA).
//  HBM: 8 bytes per node (read + write), plus the id list.
//
//  Novelty. The largest <E_i, q> over the live nodes: the global query path with
//  no decay (lambda 0 makes the weight exactly 1), no filter, top-1 and no BFS, so it
//  runs the certified fp16 scan when the context has it (the same answer as the fp32
//  scan, bit for bit). Floored at -1 and 0 for an empty graph, as the reference.
//
//  Edge hits. One int32 per col slot. Counting reads the BFS levels of a context's
//  last global query (its visit list): every visited node v at hop h >= 1 adds one
//  to each of its edges (v, u) whose u was visited at hop h - 1. Two launches: the
//  levels are stamped into a per-context node map (no clear between calls), then
//  16 lanes per visited row test its neighbours. Slots that hold no live edge always
//  hold 0 (inserts move counters with their edges and zero the old slots), so the
//  maintenance sweep is one coalesced pass over the used slots: it counts the slots
//  above min_hits, writes zeros where a counter was set, and the low-utility count is
//  the live edge count minus that.
// ============================================================================
#include "internal.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>

namespace mars {
namespace {

constexpr int kSlice = 1024;            // nodes per workgroup of the importance update (256 x float4)
constexpr int kSweepThreads = 256;

__global__ __launch_bounds__(256) void k_fill_f32(float* __restrict__ p, int64_t n, float v) {
    const int64_t stride = int64_t(gridDim.x) * blockDim.x;
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = v;
}

constexpr int kInlineIds = 64;          // boost ids passed in the kernel arguments (no copy)

struct ImportanceArgs {
    float* imp;
    int32_t n;            // live nodes
    float retain;         // 1 - decay_rate (fp32, as the reference computes it)
    const int32_t* ids;   // boosts, in list order (null: the first n_ids of inline_ids)
    int32_t n_ids;
    float boost;
    float max_imp;
    int32_t inline_ids[kInlineIds];
};

__global__ __launch_bounds__(256) void k_importance_update(ImportanceArgs a) {
    const int64_t lo = int64_t(blockIdx.x) * kSlice;
    const int64_t hi = std::min<int64_t>(lo + kSlice, a.n);
    const int64_t i = lo + int64_t(threadIdx.x) * 4;
    if (i + 4 <= hi) {
        float4 v = *reinterpret_cast<const float4*>(a.imp + i);
        v.x = __fmul_rn(v.x, a.retain);
        v.y = __fmul_rn(v.y, a.retain);
        v.z = __fmul_rn(v.z, a.retain);
        v.w = __fmul_rn(v.w, a.retain);
        *reinterpret_cast<float4*>(a.imp + i) = v;
    } else {
        for (int64_t j = i; j < hi; ++j) a.imp[j] = __fmul_rn(a.imp[j], a.retain);
    }
    if (a.n_ids == 0) return;                          // uniform
    __syncthreads();                                   // the slice's decayed values are visible
    const int32_t* ids = a.ids ? a.ids : a.inline_ids;
    for (int32_t t = threadIdx.x; t < a.n_ids; t += blockDim.x) {
        const int32_t id = ids[t];
        if (id < lo || id >= hi) continue;             // other slices, and ids < 0
        // the first occurrence applies every occurrence of its id, in order
        int32_t reps = 0;
        bool first = true;
        for (int32_t u = 0; u < a.n_ids; ++u) {
            if (ids[u] != id) continue;
            if (u < t) { first = false; break; }
            ++reps;
        }
        if (!first) continue;
        float v = a.imp[id];
        for (int32_t r = 0; r < reps; ++r) v = fminf(__fadd_rn(v, a.boost), a.max_imp);
        a.imp[id] = v;
    }
}

struct HitArgs {
    const int32_t* vlist;
    const int32_t* vhop;
    int32_t nv;
    uint64_t* hopmap;
    int32_t hop_cap;
    uint32_t stamp;
    const int64_t* ro;
    const int32_t* col;
    int32_t* hits;
    int32_t n_rows;       // rows that exist (node ids below it)
};

__global__ __launch_bounds__(256) void k_hop_stamp(HitArgs a) {
    const int32_t i = int32_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= a.nv) return;
    const int32_t v = a.vlist[i];
    if (v >= 0 && v < a.hop_cap) a.hopmap[v] = (uint64_t(a.stamp) << 32) | uint32_t(a.vhop[i]);
}

// 16 lanes per visited node, its row's neighbours strided over them.
__global__ __launch_bounds__(256) void k_edge_hits(HitArgs a) {
    const int64_t g = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) >> 4;
    const int sub = int(threadIdx.x & 15u);
    if (g >= a.nv) return;
    const int32_t v = a.vlist[g];
    const int32_t h = a.vhop[g];
    if (h <= 0 || v < 0 || v >= a.n_rows) return;     // seeds are not reached over an edge
    const int64_t w = a.ro[v];
    const int64_t start = int64_t(uint32_t(w)), len = w >> 32;
    const uint64_t want = (uint64_t(a.stamp) << 32) | uint32_t(h - 1);
    for (int64_t j = sub; j < len; j += 16) {
        const int32_t u = a.col[start + j];
        if (u >= 0 && u < a.hop_cap && a.hopmap[u] == want)
            __hip_atomic_fetch_add(a.hits + start + j, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Counts slots with hits > min_hits over [0, n_slots) and zeroes the set ones.
__global__ __launch_bounds__(kSweepThreads) void k_edge_sweep(int32_t* __restrict__ hits, int64_t n_slots,
                                                              int32_t min_hits, unsigned long long* count) {
    const int64_t stride = int64_t(gridDim.x) * blockDim.x * 8;
    uint32_t above = 0;
    for (int64_t i = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) * 8; i < n_slots; i += stride) {
        if (i + 8 <= n_slots) {
            // both loads in flight before any store (the stores may alias them)
            const int4 h0 = *reinterpret_cast<const int4*>(hits + i);
            const int4 h1 = *(reinterpret_cast<const int4*>(hits + i) + 1);
            above += (h0.x > min_hits) + (h0.y > min_hits) + (h0.z > min_hits) + (h0.w > min_hits);
            above += (h1.x > min_hits) + (h1.y > min_hits) + (h1.z > min_hits) + (h1.w > min_hits);
            if (h0.x | h0.y | h0.z | h0.w) *reinterpret_cast<int4*>(hits + i) = make_int4(0, 0, 0, 0);
            if (h1.x | h1.y | h1.z | h1.w) *(reinterpret_cast<int4*>(hits + i) + 1) = make_int4(0, 0, 0, 0);
        } else {
            for (int64_t j = i; j < n_slots; ++j) {
                above += hits[j] > min_hits;
                if (hits[j]) hits[j] = 0;
            }
        }
    }
    for (int off = 32; off > 0; off >>= 1) above += __shfl_xor(above, off);
    __shared__ uint32_t s_sum[kSweepThreads / 64];
    if ((threadIdx.x & 63u) == 0) s_sum[threadIdx.x >> 6] = above;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long t = 0;
        for (int w = 0; w < kSweepThreads / 64; ++w) t += s_sum[w];
        if (t) __hip_atomic_fetch_add(count, t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

unsigned grid_for(int64_t work, int64_t per_block, int64_t cap) {
    return unsigned(std::max<int64_t>(1, std::min<int64_t>((work + per_block - 1) / per_block, cap)));
}

}  // namespace

// Edge-hit counters of a graph whose col array was replaced (set_csr): all zero.
int reset_edge_hits(Graph& g) {
    if (!g.hits) return MARS_OK;
    dfree(g.hits);
    MARS_TRY(dmalloc(&g.hits, size_t(g.cap_e)));
    MARS_HIP(hipMemset(g.hits, 0, size_t(g.cap_e) * sizeof(int32_t)));
    return MARS_OK;
}

int launch_importance_update(float* imp, int32_t n, float retain, const int32_t* ids, int32_t n_ids, float boost,
                             float max_imp, hipStream_t s, const int32_t* host_ids = nullptr) {
    if (n <= 0) return MARS_OK;
    ImportanceArgs a{};
    a.imp = imp; a.n = n; a.retain = retain; a.ids = ids; a.n_ids = n_ids; a.boost = boost; a.max_imp = max_imp;
    if (host_ids) std::memcpy(a.inline_ids, host_ids, size_t(n_ids) * sizeof(int32_t));   // n_ids <= kInlineIds
    MARS_LAUNCH(k_importance_update, dim3(unsigned((int64_t(n) + kSlice - 1) / kSlice)), dim3(256), 0, s, a);
    return MARS_OK;
}

int launch_edge_sweep(int32_t* hits, int64_t n_slots, int32_t min_hits, unsigned long long* count, hipStream_t s) {
    MARS_LAUNCH(k_edge_sweep, dim3(grid_for(n_slots, int64_t(kSweepThreads) * 8, 65536)), dim3(kSweepThreads),
                0, s, hits, n_slots, min_hits, count);
    return MARS_OK;
}

}  // namespace mars

using namespace mars;

int mars_importance_init(mars_graph* gh) {
    MARS_CHECK(gh, MARS_ERR_INVALID, "null graph");
    std::lock_guard<std::mutex> lock(gh->mu);
    Graph& g = gh->g;
    MARS_TRY(use_device(g.device));
    if (!g.imp) MARS_TRY(dmalloc(&g.imp, size_t(g.cap_n)));
    hipStream_t s = g.ins_stream;
    MARS_LAUNCH(k_fill_f32, dim3(grid_for(g.cap_n, 256, 4096)), dim3(256), 0, s, g.imp, int64_t(g.cap_n), 1.0f);
    MARS_HIP(hipStreamSynchronize(s));
    return MARS_OK;
}

int mars_importance_update(mars_graph* gh, const int32_t* ids, int32_t n_ids, int32_t ids_on_device, float boost,
                           float decay_rate, float max_importance) {
    MARS_CHECK(gh, MARS_ERR_INVALID, "null graph");
    MARS_CHECK(n_ids >= 0 && (n_ids == 0 || ids), MARS_ERR_INVALID, "bad id list");
    std::lock_guard<std::mutex> lock(gh->mu);
    Graph& g = gh->g;
    MARS_CHECK(g.imp, MARS_ERR_UNSUPPORTED, "importance not initialised (mars_importance_init)");
    MARS_TRY(use_device(g.device));
    hipStream_t s = g.ins_stream;
    const int32_t* d_ids = ids;
    const int32_t* h_ids = nullptr;
    if (n_ids > 0 && !ids_on_device && n_ids <= kInlineIds) {
        h_ids = ids;                                              // travel in the kernel arguments
        d_ids = nullptr;
    } else if (n_ids > 0 && !ids_on_device) {
        if (n_ids > g.imp_ids_cap) {
            dfree(g.imp_ids);
            g.imp_ids_cap = 0;
            MARS_TRY(dmalloc(&g.imp_ids, size_t(n_ids)));
            g.imp_ids_cap = n_ids;
        }
        MARS_HIP(hipMemcpyAsync(g.imp_ids, ids, size_t(n_ids) * sizeof(int32_t), hipMemcpyHostToDevice, s));
        d_ids = g.imp_ids;
    }
    const int32_t n = __atomic_load_n(&g.n, __ATOMIC_ACQUIRE);
    const float retain = 1.0f - decay_rate;                       // memory_cuda.cu:1513
    MARS_TRY(launch_importance_update(g.imp, n, retain, d_ids, n_ids, boost, max_importance, s, h_ids));
    MARS_HIP(hipStreamSynchronize(s));
    return MARS_OK;
}

int mars_importance_read(const mars_graph* gh, float* h_out, int32_t first, int32_t count) {
    MARS_CHECK(gh && (count == 0 || h_out), MARS_ERR_INVALID, "null argument");
    std::lock_guard<std::mutex> lock(gh->mu);
    const Graph& g = gh->g;
    MARS_CHECK(g.imp, MARS_ERR_UNSUPPORTED, "importance not initialised (mars_importance_init)");
    MARS_CHECK(first >= 0 && count >= 0 && int64_t(first) + count <= g.n, MARS_ERR_INVALID,
               "nodes [%d, %d + %d) outside the %d nodes", first, first, count, g.n);
    MARS_TRY(use_device(g.device));
    MARS_HIP(hipStreamSynchronize(g.ins_stream));
    if (count) MARS_HIP(hipMemcpy(h_out, g.imp + first, size_t(count) * sizeof(float), hipMemcpyDeviceToHost));
    return MARS_OK;
}

int mars_novelty(const mars_graph* gh, mars_ctx* ctx, const float* h_q, const float* d_q, float* max_sim) {
    MARS_CHECK(gh && max_sim && (h_q || d_q), MARS_ERR_INVALID, "null argument");
    *max_sim = 0.0f;
    std::unique_lock<std::mutex> own;
    if (!ctx) {
        own = std::unique_lock<std::mutex>(gh->own_mu);
        if (!gh->own_ctx) {
            // sized for the graph's capacity (fixed when the graph is created)
            MARS_TRY(mars_ctx_create(gh->g.cap_n, gh->g.d, 1, MARS_CTX_CERTIFIED, &gh->own_ctx));
        }
        ctx = gh->own_ctx;
    }
    if (__atomic_load_n(&gh->g.n, __ATOMIC_ACQUIRE) <= 0) return MARS_OK;
    mars_retrieval_config cfg;
    mars_config_default(&cfg);
    cfg.top_k = 1;
    cfg.bfs_max_hops = 0;
    cfg.time_decay_lambda = 0.0f;
    mars_query_result r{};
    int32_t count = 0;
    const int rc = h_q ? mars_query(gh, ctx, h_q, 0.0f, &cfg, &r, 1, &count, nullptr)
                       : mars_query_device(gh, ctx, d_q, 0.0f, &cfg, &r, 1, &count, nullptr);
    MARS_TRY(rc);
    *max_sim = count > 0 ? std::max(-1.0f, r.score) : 0.0f;     // memory_cuda.cu:1589-1591
    return MARS_OK;
}

int mars_edge_hits_init(mars_graph* gh) {
    MARS_CHECK(gh, MARS_ERR_INVALID, "null graph");
    std::lock_guard<std::mutex> lock(gh->mu);
    Graph& g = gh->g;
    MARS_TRY(use_device(g.device));
    MARS_HIP(hipStreamSynchronize(g.ins_stream));
    if (!g.hits) MARS_TRY(dmalloc(&g.hits, size_t(g.cap_e)));
    MARS_HIP(hipMemset(g.hits, 0, size_t(g.cap_e) * sizeof(int32_t)));
    return MARS_OK;
}

int mars_edge_hits_count(mars_graph* gh, mars_ctx* ch) {
    MARS_CHECK(gh && ch, MARS_ERR_INVALID, "null argument");
    std::lock_guard<std::mutex> lock(gh->mu);
    Graph& g = gh->g;
    Ctx& c = ch->c;
    MARS_CHECK(g.hits, MARS_ERR_UNSUPPORTED, "edge hits not initialised (mars_edge_hits_init)");
    MARS_CHECK(g.d == c.d, MARS_ERR_INVALID, "graph dim %d != context dim %d", g.d, c.d);
    if (c.hit_n <= 0 || !c.hit_vlist) return MARS_OK;            // no BFS levels recorded
    MARS_TRY(use_device(c.device));
    hipStream_t s = c.stream;
    if (!c.hopmap) {
        MARS_TRY(dmalloc(&c.hopmap, size_t(c.max_nodes)));
        MARS_HIP(hipMemsetAsync(c.hopmap, 0, size_t(c.max_nodes) * sizeof(uint64_t), s));
        c.hop_stamp = 0;
    }
    if (++c.hop_stamp == 0) {                                     // stamps wrapped: start clean
        MARS_HIP(hipMemsetAsync(c.hopmap, 0, size_t(c.max_nodes) * sizeof(uint64_t), s));
        c.hop_stamp = 1;
    }
    HitArgs a{};
    a.vlist = c.hit_vlist; a.vhop = c.hit_vhop; a.nv = c.hit_n; a.hopmap = c.hopmap; a.hop_cap = c.max_nodes;
    a.stamp = c.hop_stamp; a.ro = g.ro; a.col = g.col; a.hits = g.hits; a.n_rows = g.n;
    // two launches: one workgroup doing both steps (a barrier between them) measured 3.5x
    // slower on a 1.5K-node visit list (one CU walks every row's dependent loads)
    MARS_LAUNCH(k_hop_stamp, dim3(unsigned((a.nv + 255) / 256)), dim3(256), 0, s, a);
    MARS_LAUNCH(k_edge_hits, dim3(unsigned((int64_t(a.nv) * 16 + 255) / 256)), dim3(256), 0, s, a);
    MARS_HIP(hipStreamSynchronize(s));
    return MARS_OK;
}

int mars_edge_hits_read(const mars_graph* gh, int32_t* h_hits, int64_t cap, int64_t* n_out) {
    MARS_CHECK(gh && n_out && (cap == 0 || h_hits), MARS_ERR_INVALID, "null argument");
    std::lock_guard<std::mutex> lock(gh->mu);
    const Graph& g = gh->g;
    MARS_CHECK(g.hits, MARS_ERR_UNSUPPORTED, "edge hits not initialised (mars_edge_hits_init)");
    MARS_TRY(use_device(g.device));
    MARS_HIP(hipStreamSynchronize(g.ins_stream));
    *n_out = g.e;
    if (cap < g.e) return MARS_OK;                               // sizing call
    std::vector<int32_t> slots(size_t(std::max<int64_t>(g.e_used, 1)));
    if (g.e_used) MARS_HIP(hipMemcpy(slots.data(), g.hits, size_t(g.e_used) * sizeof(int32_t), hipMemcpyDeviceToHost));
    int64_t at = 0;
    for (int32_t i = 0; i < g.n; ++i) {
        const int64_t w = g.ro_h[size_t(i)];
        const int64_t start = int64_t(uint32_t(w)), len = w >> 32;
        std::memcpy(h_hits + at, slots.data() + start, size_t(len) * sizeof(int32_t));
        at += len;
    }
    return MARS_OK;
}

int mars_graph_maintain(mars_graph* gh, int32_t min_hits, int32_t window_queries, int32_t* low_utility) {
    (void)window_queries;                                         // unused, as in the reference
    MARS_CHECK(gh && low_utility, MARS_ERR_INVALID, "null argument");
    std::lock_guard<std::mutex> lock(gh->mu);
    Graph& g = gh->g;
    *low_utility = 0;
    if (!g.hits || g.e <= 0) return MARS_OK;                     // memory_cuda.cu:1639
    MARS_TRY(use_device(g.device));
    hipStream_t s = g.ins_stream;
    if (!g.sweep_cnt) MARS_TRY(dmalloc(&g.sweep_cnt, 1));
    MARS_HIP(hipMemsetAsync(g.sweep_cnt, 0, sizeof(unsigned long long), s));
    MARS_TRY(launch_edge_sweep(g.hits, g.e_used, std::max(min_hits, -1), g.sweep_cnt, s));
    unsigned long long above = 0;
    MARS_HIP(hipMemcpyAsync(&above, g.sweep_cnt, sizeof(above), hipMemcpyDeviceToHost, s));
    MARS_HIP(hipStreamSynchronize(s));
    // counters are >= 0: below 0 nothing is low; otherwise every live edge not above
    *low_utility = min_hits < 0 ? 0 : int32_t(int64_t(g.e) - int64_t(above));
    return MARS_OK;
}
