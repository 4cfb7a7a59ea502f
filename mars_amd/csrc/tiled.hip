// ============================================================================
//  tiled.hip — out-of-core comparator: a query over a corpus held in host RAM,
//  streamed to the GPU in tiles (the contract of the reference's tiled_query,
//  src/tiled_query.cu:174-314 / include/tiled_query.h:33-102).
//
//  Contract kept: per tile, exact decayed scores (modality filter -> -FLT_MAX),
//  the tile's top-K; candidates with score > -FLT_MAX/2 are merged; the K best
//  are returned (score desc; ties here by lower id). No BFS, no episode scope.
//
//  MI355X design: two device tile buffers; tile i+1 is copied on a copy stream
//  while tile i is scanned on the compute stream (the reference copies, then
//  computes, then copies the next tile). Each tile is scanned by the same fused
//  k_scan as the resident path (ids offset by the tile start); the scan's
//  running bound on the K-th key carries across tiles, and k_tile_merge folds a
//  tile's surviving keys into the running K best on the device, so only K keys
//  cross PCIe back. For PCIe-rate copies the host arrays should be pinned
//  (mars_host_alloc); pageable arrays are staged by the HIP runtime.
// ============================================================================
#include "internal.hpp"

#include <algorithm>
#include <cfloat>
#include <chrono>
#include <cstring>
#include <vector>

using namespace mars;

struct mars_tiled_ctx {
    int device = 0;
    int32_t max_tile = 0, d = 0, max_k = 0;
    hipStream_t cs = nullptr;         // compute
    hipStream_t xs = nullptr;         // host -> device copies
    float* emb[2] = {nullptr, nullptr};
    float* ts[2] = {nullptr, nullptr};
    int32_t* mods[2] = {nullptr, nullptr};
    float* query = nullptr;
    float* fin = nullptr;             // scan scores of the current tile (max_tile)
    uint64_t* part = nullptr;         // candidate keys of one tile
    uint64_t* gthr = nullptr;
    uint32_t* gcnt = nullptr;
    uint64_t* carry = nullptr;        // running K best (ascending keys)
    float* h_query = nullptr;         // pinned
    uint64_t* h_keys = nullptr;       // pinned
    std::vector<hipEvent_t> ev;       // 4 per tile: copy start / end, scan start / end
};

namespace {

constexpr int32_t kTiledWg = 2048;

void tiled_free(mars_tiled_ctx* t) {
    (void)use_device(t->device);
    if (t->cs) (void)hipStreamSynchronize(t->cs);
    if (t->xs) (void)hipStreamSynchronize(t->xs);
    for (int b = 0; b < 2; ++b) { dfree(t->emb[b]); dfree(t->ts[b]); dfree(t->mods[b]); }
    dfree(t->query); dfree(t->fin); dfree(t->part); dfree(t->gthr); dfree(t->gcnt); dfree(t->carry);
    if (t->h_query) (void)hipHostFree(t->h_query);
    if (t->h_keys) (void)hipHostFree(t->h_keys);
    for (auto e : t->ev) (void)hipEventDestroy(e);
    if (t->cs) (void)hipStreamDestroy(t->cs);
    if (t->xs) (void)hipStreamDestroy(t->xs);
    delete t;
}

int ensure_events(mars_tiled_ctx* t, size_t n) {
    while (t->ev.size() < n) {
        hipEvent_t e = nullptr;
        MARS_HIP(hipEventCreate(&e));
        t->ev.push_back(e);
    }
    return MARS_OK;
}

}  // namespace

extern "C" {

void mars_tiled_config_default(mars_tiled_config* c) {
    if (!c) return;
    c->tile_size = 5000000;            // tiled_query.h:34-40
    c->top_k = 10;
    c->time_decay_lambda = 1e-8f;
    c->modality_filter = -1;
    c->use_fp16 = 1;
}

int mars_host_alloc(size_t bytes, void** ptr) {
    MARS_CHECK(ptr, MARS_ERR_INVALID, "null argument");
    *ptr = nullptr;
    MARS_HIP(hipHostMalloc(ptr, bytes ? bytes : 1, hipHostMallocDefault));
    return MARS_OK;
}

int mars_host_free(void* ptr) {
    if (ptr) MARS_HIP(hipHostFree(ptr));
    return MARS_OK;
}

int mars_tiled_ctx_create(int32_t max_tile_size, int32_t dim, int32_t max_k, mars_tiled_ctx** out) {
    MARS_CHECK(out, MARS_ERR_INVALID, "null argument");
    *out = nullptr;
    MARS_CHECK(max_tile_size > 0 && dim > 0 && max_k > 0, MARS_ERR_INVALID, "tile %d, dim %d, max_k %d",
               max_tile_size, dim, max_k);
    int dev = 0;
    MARS_HIP(hipGetDevice(&dev));
    hipDeviceProp_t prop;
    MARS_HIP(hipGetDeviceProperties(&prop, dev));
    MARS_CHECK(std::strncmp(prop.gcnArchName, "gfx950", 6) == 0, MARS_ERR_NODEVICE,
               "device %d is %s, this build targets gfx950 only", dev, prop.gcnArchName);
    auto* t = new mars_tiled_ctx();
    t->device = dev;
    t->max_tile = max_tile_size;
    t->d = dim;
    t->max_k = std::min(max_k, kMaxK);
    const size_t T = size_t(max_tile_size);
    int rc = MARS_OK;
    for (int b = 0; b < 2 && rc == MARS_OK; ++b)
        if ((rc = dmalloc(&t->emb[b], T * size_t(dim))) == MARS_OK && (rc = dmalloc(&t->ts[b], T)) == MARS_OK)
            rc = dmalloc(&t->mods[b], T);
    if (rc == MARS_OK) rc = dmalloc(&t->query, size_t(dim));
    if (rc == MARS_OK) rc = dmalloc(&t->fin, T);
    if (rc == MARS_OK) rc = dmalloc(&t->part, size_t(kTiledWg) * kMaxK);
    if (rc == MARS_OK) rc = dmalloc(&t->gthr, 1);
    if (rc == MARS_OK) rc = dmalloc(&t->gcnt, 1);
    if (rc == MARS_OK) rc = dmalloc(&t->carry, size_t(kMaxK));
    hipError_t e = hipSuccess;
    if (rc == MARS_OK) e = hipHostMalloc(reinterpret_cast<void**>(&t->h_query), size_t(dim) * sizeof(float));
    if (rc == MARS_OK && e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void**>(&t->h_keys), kMaxK * 8);
    if (rc == MARS_OK && e == hipSuccess) e = hipStreamCreateWithFlags(&t->cs, hipStreamNonBlocking);
    if (rc == MARS_OK && e == hipSuccess) e = hipStreamCreateWithFlags(&t->xs, hipStreamNonBlocking);
    if (rc == MARS_OK && e != hipSuccess) rc = set_error(MARS_ERR_HIP, "tiled context: %s", hipGetErrorString(e));
    if (rc != MARS_OK) {
        tiled_free(t);
        return rc;
    }
    *out = t;
    return MARS_OK;
}

int mars_tiled_ctx_destroy(mars_tiled_ctx* t) {
    if (t) tiled_free(t);
    return MARS_OK;
}

int mars_tiled_query(mars_tiled_ctx* t, const float* h_emb, const int32_t* h_mods, const float* h_ts, int32_t n,
                     int32_t d, const float* h_query, float t_q, const mars_tiled_config* cfg,
                     mars_tiled_result* out, int32_t cap, int32_t* n_out, mars_tiled_stats* stats) {
    const auto t0 = std::chrono::steady_clock::now();
    MARS_CHECK(t && h_emb && h_mods && h_ts && h_query && cfg && n_out, MARS_ERR_INVALID, "null argument");
    MARS_CHECK(cap >= 0 && (cap == 0 || out), MARS_ERR_INVALID, "bad output buffer");
    MARS_CHECK(n > 0 && d == t->d, MARS_ERR_INVALID, "n %d, dim %d (context dim %d)", n, d, t->d);
    MARS_CHECK(cfg->top_k >= 1 && cfg->top_k <= t->max_k, MARS_ERR_UNSUPPORTED, "top_k %d outside [1, %d]",
               cfg->top_k, t->max_k);
    MARS_CHECK(cfg->tile_size > 0, MARS_ERR_INVALID, "tile_size %d", cfg->tile_size);
    const int32_t K = cfg->top_k;
    const int32_t tile = std::min(cfg->tile_size, n);                     // tiled_query.cu:191
    MARS_CHECK(tile <= t->max_tile, MARS_ERR_CAPACITY, "tile of %d rows, context sized for %d", tile,
               t->max_tile);
    const int32_t num_tiles = (n + tile - 1) / tile;
    MARS_TRY(use_device(t->device));
    MARS_TRY(ensure_events(t, size_t(num_tiles) * 4));
    hipStream_t cs = t->cs, xs = t->xs;
    std::memcpy(t->h_query, h_query, size_t(d) * sizeof(float));
    MARS_HIP(hipMemcpyAsync(t->query, t->h_query, size_t(d) * sizeof(float), hipMemcpyHostToDevice, cs));
    MARS_HIP(hipMemsetAsync(t->carry, 0xFF, size_t(kMaxK) * sizeof(uint64_t), cs));
    MARS_HIP(hipMemsetAsync(t->gthr, 0xFF, sizeof(uint64_t), cs));
    MARS_HIP(hipMemsetAsync(t->gcnt, 0, sizeof(uint32_t), cs));
    double bytes = 0.0;
    for (int32_t i = 0; i < num_tiles; ++i) {
        const int b = i & 1;
        const int64_t off = int64_t(i) * tile;
        const int32_t nt = int32_t(std::min<int64_t>(tile, n - off));
        hipEvent_t* e = &t->ev[size_t(i) * 4];
        // buffer b was last read by the scan of tile i - 2
        if (i >= 2) MARS_HIP(hipStreamWaitEvent(xs, t->ev[size_t(i - 2) * 4 + 3], 0));
        MARS_HIP(hipEventRecord(e[0], xs));
        MARS_HIP(hipMemcpyAsync(t->emb[b], h_emb + off * d, size_t(nt) * size_t(d) * sizeof(float),
                                hipMemcpyHostToDevice, xs));
        MARS_HIP(hipMemcpyAsync(t->mods[b], h_mods + off, size_t(nt) * sizeof(int32_t), hipMemcpyHostToDevice, xs));
        MARS_HIP(hipMemcpyAsync(t->ts[b], h_ts + off, size_t(nt) * sizeof(float), hipMemcpyHostToDevice, xs));
        MARS_HIP(hipEventRecord(e[1], xs));
        bytes += double(nt) * (double(d) * 4.0 + 8.0);
        MARS_HIP(hipStreamWaitEvent(cs, e[1], 0));
        MARS_HIP(hipEventRecord(e[2], cs));
        int32_t rpw = 0, nwg = 0;
        scan_grid(nt, kTiledWg, &rpw, &nwg);
        ScanArgs a{};
        a.emb = t->emb[b]; a.fp16 = 0; a.n = nt; a.d = d; a.q = t->query; a.ts = t->ts[b]; a.mods = t->mods[b];
        a.ep_ids = nullptr; a.t_q = t_q; a.lambda = cfg->time_decay_lambda; a.mod_filter = cfg->modality_filter;
        a.query_ep = -1; a.boost = 0.0f; a.k = K; a.fin = t->fin; a.part = t->part; a.gthr = t->gthr;
        a.gcnt = t->gcnt; a.rows_per_wg = rpw; a.num_wg = nwg; a.id_base = off;
        MARS_TRY(launch_scan(a, cs));
        MARS_TRY(launch_tile_merge(t->part, t->gcnt, t->carry, K, cs));
        MARS_HIP(hipEventRecord(e[3], cs));
    }
    MARS_HIP(hipMemcpyAsync(t->h_keys, t->carry, size_t(K) * sizeof(uint64_t), hipMemcpyDeviceToHost, cs));
    MARS_HIP(hipStreamSynchronize(cs));
    const auto tm = std::chrono::steady_clock::now();
    // merge step of tiled_query.cu:280-302: drop filtered rows, K best by score desc
    int32_t m = 0;
    for (int32_t j = 0; j < K; ++j) {
        const uint64_t key = t->h_keys[j];
        if (key == kEmptyKey) break;
        const float s = key_score(key);
        if (!(s > -FLT_MAX * 0.5f)) continue;
        if (m < cap) out[m] = mars_tiled_result{key_id(key), s, h_mods[key_id(key)]};
        ++m;
    }
    *n_out = m;
    if (stats) {
        mars_tiled_stats st{};
        st.total_nodes = n;
        st.num_tiles = num_tiles;
        float ms = 0.0f, x = 0.0f, c = 0.0f;
        for (int32_t i = 0; i < num_tiles; ++i) {
            MARS_HIP(hipEventElapsedTime(&ms, t->ev[size_t(i) * 4], t->ev[size_t(i) * 4 + 1]));
            x += ms;
            MARS_HIP(hipEventElapsedTime(&ms, t->ev[size_t(i) * 4 + 2], t->ev[size_t(i) * 4 + 3]));
            c += ms;
        }
        const auto t1 = std::chrono::steady_clock::now();
        st.transfer_ms = x;
        st.compute_ms = c;
        st.merge_ms = std::chrono::duration<float, std::milli>(t1 - tm).count();
        st.total_ms = std::chrono::duration<float, std::milli>(t1 - t0).count();
        st.h2d_gbs = x > 0.0f ? bytes / (double(x) * 1e6) : 0.0;
        *stats = st;
    }
    return MARS_OK;
}

}  // extern "C"
