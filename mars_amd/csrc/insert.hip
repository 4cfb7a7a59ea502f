// ============================================================================
//  insert.hip — streaming insert: new nodes appended to a resident graph on the
//  graph's side stream while queries keep running on their own streams.
//
//  Replaces the reference's StreamingBuffer::flush + add_incremental_edges_
//  (src/streaming.cpp:35-163) and the engine's re-upload after ADD
//  (src/engine_server.cu:154-213): the reference rebuilds the whole CSR on the
//  host and uploads the graph again; here only the new rows and the rows that
//  gain a neighbour are written, on the device.
//
//  Edge rule (incremental NSN): each new node u links to
//    * every other new node of its episode (new nodes open new episodes), and
//    * its k nearest neighbours by cosine among all nodes 0 .. n_old + n_new - 1
//      (self excluded; ties by lower id), found by the batched MFMA scan over
//      the fp16 rows and rescored exactly in fp32;
//  every edge is stored in both directions. Rows stay sorted ascending: new ids
//  exceed every old id, so an old row only grows at its end.
//
//  Publication, in two steps:
//    1. rows, modalities, timestamps, episode ids, fp16 rows and the episode CSR
//       tail are copied; then the node count (and episode count) is published:
//       the nodes are visible to global scans and episode scope (queryable);
//    2. k-NN, host planning of the row updates, then two kernels: k_patch_data
//       writes column data, k_patch_rows (a later kernel on the same stream)
//       publishes each changed row word (len << 32 | start). A query running
//       meanwhile reads every row either entirely old or entirely new:
//         - a row that outgrows its reserved slots moves to a tail region that
//           starts on a fresh 256-byte boundary of col, so no query has read
//           (or cached) those lines before its new word appears;
//         - a row with room appends in place into slots that hold -1 since the
//           row was placed; a stale cached line shows -1, which the BFS skips
//           like a neighbour id at or above its node count.
//       Old column data is never overwritten.
// ============================================================================
#include "internal.hpp"

#include <algorithm>
#include <chrono>
#include <cstring>
#include <vector>

namespace mars {
namespace {

constexpr int32_t kCopySlot = INT32_MIN;    // tail value: filled by a relocation copy
constexpr int64_t kRegionAlign = 64;        // 256 bytes of col
constexpr int32_t kInsertChunk = 1024;      // k-NN queries per batched-scan launch
constexpr int32_t kKnnCand = 16;            // fp16 candidates rescored per new node

__global__ void k_patch_data(PatchArgs a) {
    const int64_t tid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t stride = int64_t(gridDim.x) * blockDim.x;
    // relocations: one 64-lane wave per row (rows are short)
    const int64_t wave = tid >> 6, nwaves = stride >> 6;
    const int lane = int(threadIdx.x & 63u);
    for (int64_t r = wave; r < a.n_reloc; r += nwaves) {
        const int64_t src = a.reloc[3 * r], len = a.reloc[3 * r + 1], dst = a.reloc[3 * r + 2];
        for (int64_t i = lane; i < len; i += 64) a.col[dst + i] = a.col[src + i];
    }
    for (int64_t i = tid; i < a.n_tail; i += stride) {
        const int32_t v = a.tail[i];
        if (v != kCopySlot) a.col[a.tail_base + i] = v;
    }
    for (int64_t i = tid; i < a.n_app; i += stride) a.col[a.app[2 * i]] = int32_t(a.app[2 * i + 1]);
}

__global__ void k_patch_rows(PatchArgs a) {
    const int64_t tid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t stride = int64_t(gridDim.x) * blockDim.x;
    for (int64_t i = tid; i < a.n_rows; i += stride) {
        const int64_t node = a.rows[3 * i];
        a.rcap[node] = int32_t(a.rows[3 * i + 2]);
        __hip_atomic_store(reinterpret_cast<unsigned long long*>(a.ro + node),
                           (unsigned long long)a.rows[3 * i + 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

unsigned patch_grid(int64_t work) {
    const int64_t g = (work + 255) / 256;
    return unsigned(std::max<int64_t>(1, std::min<int64_t>(g, 1024)));
}

int64_t align_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

// Slots reserved for a row of `len` entries placed in a tail region.
int64_t row_capacity(int64_t len) { return len + std::max<int64_t>(8, len >> 1); }

template <typename T>
int grow_pinned(void** p, size_t* have, size_t need) {
    if (need <= *have) return MARS_OK;
    if (*p) (void)hipHostFree(*p);
    *p = nullptr;
    *have = 0;
    MARS_HIP(hipHostMalloc(p, need, hipHostMallocDefault));
    *have = need;
    return MARS_OK;
}

int grow_device(void** p, size_t* have, size_t need) {
    if (need <= *have) return MARS_OK;
    if (*p) (void)hipFree(*p);
    *p = nullptr;
    *have = 0;
    hipError_t e = hipMalloc(p, need);
    if (e != hipSuccess) return set_error(MARS_ERR_NOMEM, "hipMalloc(%zu bytes): %s", need, hipGetErrorString(e));
    *have = need;
    return MARS_OK;
}

double us_since(std::chrono::steady_clock::time_point t0) {
    return std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
}

// k nearest neighbours of nodes [first, first + nq) among [0, n): batched fp16 scan
// (no decay, no filter, self excluded) + exact fp32 rescoring of 16 candidates.
int insert_knn(Graph& g, int64_t first, int32_t nq, int64_t n, int32_t k, hipStream_t s) {
    int32_t nrr = 0, nqb = 0;
    int64_t rpr = 0, part_keys = 0;
    for (int32_t q : {std::min(nq, kInsertChunk), nq % kInsertChunk}) {   // full and last chunk
        if (q == 0) continue;
        batch_grid(n, q, &nrr, &nqb, &rpr);
        part_keys = std::max<int64_t>(part_keys, int64_t(nrr) * nqb * 64 * kKnnCand);
    }
    if (part_keys > g.ins_part_cap) {
        dfree(g.ins_part);
        g.ins_part_cap = 0;
        MARS_TRY(dmalloc(&g.ins_part, size_t(part_keys)));
        g.ins_part_cap = part_keys;
    }
    if (!g.ins_cand) {
        MARS_TRY(dmalloc(&g.ins_cand, size_t(kInsertChunk) * kKnnCand));
        MARS_TRY(dmalloc(&g.ins_tq, size_t(kInsertChunk)));
        MARS_HIP(hipMemsetAsync(g.ins_tq, 0, size_t(kInsertChunk) * sizeof(float), s));
    }
    if (nq > g.ins_cap_q) {
        dfree(g.ins_nbrs);
        g.ins_cap_q = 0;
        MARS_TRY(dmalloc(&g.ins_nbrs, size_t(nq) * 16));
        g.ins_cap_q = nq;
    }
    for (int32_t c0 = 0; c0 < nq; c0 += kInsertChunk) {
        const int32_t q = std::min(kInsertChunk, nq - c0);
        batch_grid(n, q, &nrr, &nqb, &rpr);
        BatchArgs a{};
        a.emb16 = g.emb16; a.n = n; a.d = g.d; a.qh = g.emb16 + (first + c0) * g.d; a.q = q; a.tq = g.ins_tq;
        a.ts = g.ts; a.mods = g.mods; a.lambda = 0.0f; a.mod_filter = -1; a.k = kKnnCand;
        a.self_base = first + c0; a.part = g.ins_part; a.rows_per_range = rpr; a.n_rranges = nrr;
        a.n_qblocks = nqb; a.uniform_tq = 1;
        MARS_TRY(launch_batch_scan(a, s));
        MARS_TRY(launch_batch_merge(g.ins_part, nrr, kKnnCand, q, kKnnCand, g.ins_cand, s));
        MARS_TRY(launch_knn_rerank(g.emb, first + c0, q, g.d, g.ins_cand, kKnnCand, k, g.ins_nbrs + int64_t(c0) * k, s));
    }
    return MARS_OK;
}

}  // namespace

int graph_insert_free(Graph& g) {
    if (g.ins_pin) (void)hipHostFree(g.ins_pin);
    g.ins_pin = nullptr;
    g.ins_pin_bytes = 0;
    if (g.ins_dev) (void)hipFree(g.ins_dev);
    g.ins_dev = nullptr;
    g.ins_dev_bytes = 0;
    dfree(g.ins_part); dfree(g.ins_cand); dfree(g.ins_nbrs); dfree(g.ins_tq);
    g.ins_part_cap = 0;
    g.ins_cap_q = 0;
    for (auto& e : g.ins_ev) {
        if (e) (void)hipEventDestroy(e);
        e = nullptr;
    }
    return MARS_OK;
}

}  // namespace mars

using namespace mars;

extern "C" int mars_graph_insert(mars_graph* gh, int32_t n_new, const float* emb, const int32_t* mods,
                                 const float* ts, const int32_t* ep_ids, int32_t knn_k, int32_t* out_knn,
                                 mars_insert_stats* st) {
    const auto t0 = std::chrono::steady_clock::now();
    MARS_CHECK(gh, MARS_ERR_INVALID, "null graph");
    MARS_CHECK(n_new > 0 && emb && mods && ts, MARS_ERR_INVALID, "insert: %d nodes, rows/modalities/times required",
               n_new);
    MARS_CHECK(knn_k >= 0 && knn_k <= 16, MARS_ERR_INVALID, "insert: knn_k %d outside [0, 16]", knn_k);
    std::lock_guard<std::mutex> lock(gh->mu);
    Graph& g = gh->g;
    const int32_t n_old = g.n;
    const int64_t n_after = int64_t(n_old) + n_new;
    const int64_t D = g.d;
    MARS_CHECK(n_after <= g.cap_n, MARS_ERR_CAPACITY, "insert: %lld nodes exceed the graph's capacity of %d",
               (long long)n_after, g.cap_n);
    MARS_CHECK((ep_ids != nullptr) == (g.ep_ids != nullptr), MARS_ERR_INVALID,
               ep_ids ? "insert: the graph has no episode ids (set them first)"
                      : "insert: the graph has episode ids; give the new nodes theirs");
    int32_t ep_hi = g.ep_next;            // episode count after the insert
    if (ep_ids) {
        for (int32_t i = 0; i < n_new; ++i) {
            MARS_CHECK(ep_ids[i] >= g.ep_next && ep_ids[i] < INT32_MAX, MARS_ERR_INVALID,
                       "insert: episode id %d of new node %d does not open a new episode (next free id %d)",
                       ep_ids[i], i, g.ep_next);
            ep_hi = std::max(ep_hi, ep_ids[i] + 1);
        }
    }
    const bool ep_csr = ep_ids && g.ep_off;
    if (ep_csr) {
        MARS_CHECK(int64_t(ep_hi) + 1 <= g.ep_off_cap && int64_t(g.member_total) + n_new <= g.ep_mem_cap,
                   MARS_ERR_CAPACITY, "insert: episode CSR capacity exceeded (%d episodes)", ep_hi);
    }
    for (int32_t i = 0; i < n_new; ++i)
        MARS_CHECK(mods[i] >= 0, MARS_ERR_INVALID, "insert: modality %d of new node %d", mods[i], i);
    if (knn_k > 0) {
        MARS_CHECK(g.emb16 != nullptr, MARS_ERR_UNSUPPORTED, "insert: the neighbour search reads the fp16 rows; "
                   "enable them first (or pass knn_k = 0)");
        MARS_CHECK(batch_dim_supported(g.d), MARS_ERR_UNSUPPORTED, "insert: embedding_dim %d unsupported", g.d);
    }
    // Worst case of col slots this insert can take: new rows hold at most (episode peers
    // + k + reverse links) entries, at most n_new * k old rows change, each gaining at
    // most n_new entries. When it fits, the nodes are published before the neighbour
    // search; otherwise only after the exact plan fits (a failing insert changes nothing).
    bool early = false;
    {
        int64_t peers_max = 0;
        if (ep_ids) {
            std::vector<int32_t> e(ep_ids, ep_ids + n_new);
            std::sort(e.begin(), e.end());
            for (size_t i = 0, j = 0; i < e.size(); i = j) {
                while (j < e.size() && e[j] == e[i]) ++j;
                peers_max = std::max<int64_t>(peers_max, int64_t(j - i) - 1);
            }
        }
        const int64_t new_len = std::min<int64_t>(n_after - 1, peers_max + knn_k + n_new);
        const int64_t old_rows = std::min<int64_t>(n_old, int64_t(n_new) * knn_k);
        const int64_t need = kRegionAlign + int64_t(n_new) * row_capacity(new_len) +
                             old_rows * row_capacity(int64_t(g.max_deg) + n_new);
        early = align_up(g.e_used, kRegionAlign) + need <= g.cap_e;
    }
    MARS_TRY(use_device(g.device));
    hipStream_t s = g.ins_stream;
    for (auto& e : g.ins_ev)
        if (!e) MARS_HIP(hipEventCreate(&e));

    // ---- step 1: rows, attributes, fp16 rows, episode CSR tail ----------------------
    // pinned staging: rows | modalities | times | episode ids | members | offsets
    const size_t row_bytes = size_t(n_new) * size_t(D) * sizeof(float);
    const size_t att_bytes = size_t(n_new) * sizeof(int32_t);
    const int32_t ne_new = ep_csr ? ep_hi - g.num_eps : 0;
    const size_t stage1 = row_bytes + 4 * att_bytes + size_t(ne_new) * sizeof(int32_t);
    MARS_TRY(grow_pinned<char>(&g.ins_pin, &g.ins_pin_bytes, stage1));
    char* pin = static_cast<char*>(g.ins_pin);
    char* p_mods = pin + row_bytes;
    char* p_ts = p_mods + att_bytes;
    char* p_ep = p_ts + att_bytes;
    int32_t* p_mem = reinterpret_cast<int32_t*>(p_ep + att_bytes);
    int32_t* p_off = p_mem + n_new;
    std::memcpy(pin, emb, row_bytes);
    std::memcpy(p_mods, mods, att_bytes);
    std::memcpy(p_ts, ts, att_bytes);
    MARS_HIP(hipMemcpyAsync(g.emb + int64_t(n_old) * D, pin, row_bytes, hipMemcpyHostToDevice, s));
    MARS_HIP(hipMemcpyAsync(g.mods + n_old, p_mods, att_bytes, hipMemcpyHostToDevice, s));
    MARS_HIP(hipMemcpyAsync(g.ts + n_old, p_ts, att_bytes, hipMemcpyHostToDevice, s));
    if (ep_ids) {
        std::memcpy(p_ep, ep_ids, att_bytes);
        MARS_HIP(hipMemcpyAsync(g.ep_ids + n_old, p_ep, att_bytes, hipMemcpyHostToDevice, s));
    }
    if (ep_csr) {
        // build_episode_csr over all ids (src/memory_graph.cpp:12-44) restricted to the
        // appended episodes: counting sort of the new ids, members ascending
        std::vector<int32_t> cnt(static_cast<size_t>(ne_new), 0), cur(static_cast<size_t>(ne_new));
        for (int32_t i = 0; i < n_new; ++i) ++cnt[size_t(ep_ids[i] - g.num_eps)];
        int32_t run = g.member_total;
        for (int32_t e = 0; e < ne_new; ++e) {
            cur[size_t(e)] = run - g.member_total;
            run += cnt[size_t(e)];
            p_off[e] = run;                         // ep_off[num_eps + 1 + e]
        }
        for (int32_t i = 0; i < n_new; ++i) p_mem[cur[size_t(ep_ids[i] - g.num_eps)]++] = n_old + i;
        MARS_HIP(hipMemcpyAsync(g.ep_off + g.num_eps + 1, p_off, size_t(ne_new) * sizeof(int32_t),
                                hipMemcpyHostToDevice, s));
        MARS_HIP(hipMemcpyAsync(g.ep_mem + g.member_total, p_mem, att_bytes, hipMemcpyHostToDevice, s));
    }
    if (g.emb16) {
        MARS_TRY(launch_convert_f16(g.emb + int64_t(n_old) * D, g.emb16 + int64_t(n_old) * D, int64_t(n_new) * D, s));
        // the batched global path's bound covers every published row
        if (g.nrm) MARS_TRY(launch_row_norms(g.emb, g.emb16, n_old, n_after, D, g.nrm, s));
    }
    MARS_HIP(hipStreamSynchronize(s));
    // publish: scans, episode scope and the boost see the new nodes from here on
    double t_queryable = 0.0;
    auto publish = [&]() {
        if (ep_csr) {
            __atomic_store_n(&g.member_total, g.member_total + n_new, __ATOMIC_RELEASE);
            __atomic_store_n(&g.num_eps, ep_hi, __ATOMIC_RELEASE);
        }
        if (ep_ids) g.ep_next = ep_hi;
        __atomic_store_n(&g.n, int32_t(n_after), __ATOMIC_RELEASE);
        t_queryable = us_since(t0);
    };
    if (early) publish();

    // ---- step 2: neighbour search ------------------------------------------------------
    std::vector<int32_t> knn(size_t(n_new) * size_t(knn_k), -1);
    float knn_ms = 0.0f;
    if (knn_k > 0) {
        MARS_HIP(hipEventRecord(g.ins_ev[0], s));
        MARS_TRY(insert_knn(g, n_old, n_new, n_after, knn_k, s));
        MARS_HIP(hipEventRecord(g.ins_ev[1], s));
        MARS_HIP(hipMemcpyAsync(knn.data(), g.ins_nbrs, knn.size() * sizeof(int32_t), hipMemcpyDeviceToHost, s));
        MARS_HIP(hipStreamSynchronize(s));
        MARS_HIP(hipEventElapsedTime(&knn_ms, g.ins_ev[0], g.ins_ev[1]));
    }

    // ---- step 3: plan the row updates on the host -------------------------------------------
    // new rows: episode peers U kNN U reverse kNN among the new nodes
    std::vector<std::vector<int32_t>> nrow(static_cast<size_t>(n_new));
    if (ep_ids) {
        std::vector<int32_t> order(static_cast<size_t>(n_new));
        for (int32_t i = 0; i < n_new; ++i) order[size_t(i)] = i;
        std::stable_sort(order.begin(), order.end(), [&](int32_t a, int32_t b) { return ep_ids[a] < ep_ids[b]; });
        for (size_t i = 0, j = 0; i < order.size(); i = j) {
            while (j < order.size() && ep_ids[order[j]] == ep_ids[order[i]]) ++j;
            for (size_t x = i; x < j; ++x)
                for (size_t y = i; y < j; ++y)
                    if (x != y) nrow[size_t(order[x])].push_back(n_old + order[y]);
        }
    }
    std::vector<std::pair<int32_t, int32_t>> old_add;       // (old node, new node)
    for (int32_t i = 0; i < n_new; ++i) {
        const int32_t u = n_old + i;
        for (int32_t j = 0; j < knn_k; ++j) {
            const int32_t v = knn[size_t(i) * knn_k + j];
            if (v < 0 || v >= n_after || v == u) continue;
            nrow[size_t(i)].push_back(v);
            if (v >= n_old) nrow[size_t(v - n_old)].push_back(u);
            else old_add.emplace_back(v, u);
        }
    }
    std::sort(old_add.begin(), old_add.end());
    old_add.erase(std::unique(old_add.begin(), old_add.end()), old_add.end());
    for (auto& r : nrow) {
        std::sort(r.begin(), r.end());
        r.erase(std::unique(r.begin(), r.end()), r.end());
    }
    std::vector<int64_t> reloc, app, rows;
    std::vector<int32_t> tail;
    const int64_t base = align_up(g.e_used, kRegionAlign);
    int64_t cursor = base;
    int64_t added = 0;
    int32_t n_reloc = 0, n_inplace = 0, max_deg = g.max_deg;
    auto place = [&](int64_t cap) {
        const int64_t at = cursor;
        tail.resize(size_t(at + cap - base), -1);
        cursor += cap;
        return at;
    };
    for (size_t i = 0, j = 0; i < old_add.size(); i = j) {
        const int32_t v = old_add[i].first;
        while (j < old_add.size() && old_add[j].first == v) ++j;
        const int64_t a = int64_t(j - i);
        const int64_t w = g.ro_h[size_t(v)];
        const int64_t start = int64_t(uint32_t(w)), len = w >> 32, cap = g.rcap_h[size_t(v)];
        const int64_t nlen = len + a;
        int64_t nstart = start, ncap = cap;
        if (nlen <= cap) {
            for (int64_t x = 0; x < a; ++x) {
                app.push_back(start + len + x);
                app.push_back(old_add[i + size_t(x)].second);
            }
            ++n_inplace;
        } else {
            ncap = row_capacity(nlen);
            nstart = place(ncap);
            reloc.push_back(start); reloc.push_back(len); reloc.push_back(nstart);
            for (int64_t x = 0; x < len; ++x) tail[size_t(nstart - base + x)] = kCopySlot;
            for (int64_t x = 0; x < a; ++x) tail[size_t(nstart - base + len + x)] = old_add[i + size_t(x)].second;
            ++n_reloc;
        }
        const int64_t nw = (nlen << 32) | int64_t(uint32_t(nstart));
        rows.push_back(v); rows.push_back(nw); rows.push_back(ncap);
        max_deg = std::max<int32_t>(max_deg, int32_t(nlen));
        added += a;
    }
    for (int32_t i = 0; i < n_new; ++i) {
        const auto& r = nrow[size_t(i)];
        const int64_t len = int64_t(r.size()), cap = row_capacity(len);
        const int64_t at = place(cap);
        std::memcpy(tail.data() + (at - base), r.data(), r.size() * sizeof(int32_t));
        const int64_t nw = (len << 32) | int64_t(uint32_t(at));
        rows.push_back(n_old + i); rows.push_back(nw); rows.push_back(cap);
        max_deg = std::max<int32_t>(max_deg, int32_t(len));
        added += len;
    }
    if (cursor > g.cap_e || cursor > int64_t(UINT32_MAX)) {
        if (early)      // cannot happen: the worst case fitted
            return set_error(MARS_ERR_CAPACITY, "insert: planned %lld col slots beyond the worst case "
                             "(nodes published without edges)", (long long)cursor);
        return set_error(MARS_ERR_CAPACITY, "insert: edge capacity %lld too small (used %lld, this insert "
                         "needs %lld)", (long long)g.cap_e, (long long)g.e_used, (long long)(cursor - g.e_used));
    }
    if (!early) publish();

    // ---- step 4: write column data, then publish the row words ------------------------------
    const size_t b_reloc = reloc.size() * sizeof(int64_t), b_app = app.size() * sizeof(int64_t);
    const size_t b_rows = rows.size() * sizeof(int64_t), b_tail = tail.size() * sizeof(int32_t);
    const size_t total = b_reloc + b_app + b_rows + b_tail + 64;
    MARS_TRY(grow_pinned<char>(&g.ins_pin, &g.ins_pin_bytes, total));
    MARS_TRY(grow_device(&g.ins_dev, &g.ins_dev_bytes, total));
    pin = static_cast<char*>(g.ins_pin);          // the staging of step 1 is consumed (synchronised)
    char* dev = static_cast<char*>(g.ins_dev);
    size_t off = 0;
    auto put = [&](const void* src, size_t bytes) {
        const size_t at = off;
        if (bytes) std::memcpy(pin + at, src, bytes);
        off += (bytes + 15) / 16 * 16;
        return at;
    };
    const size_t o_reloc = put(reloc.data(), b_reloc), o_app = put(app.data(), b_app);
    const size_t o_rows = put(rows.data(), b_rows), o_tail = put(tail.data(), b_tail);
    MARS_HIP(hipMemcpyAsync(dev, pin, off, hipMemcpyHostToDevice, s));
    PatchArgs pa{};
    pa.col = g.col; pa.ro = g.ro; pa.rcap = g.rcap;
    pa.reloc = reinterpret_cast<const int64_t*>(dev + o_reloc); pa.n_reloc = int32_t(reloc.size() / 3);
    pa.tail = reinterpret_cast<const int32_t*>(dev + o_tail); pa.tail_base = base; pa.n_tail = int64_t(tail.size());
    pa.app = reinterpret_cast<const int64_t*>(dev + o_app); pa.n_app = int32_t(app.size() / 2);
    pa.rows = reinterpret_cast<const int64_t*>(dev + o_rows); pa.n_rows = int32_t(rows.size() / 3);
    const int64_t data_work = std::max<int64_t>({int64_t(pa.n_reloc) * 64, pa.n_tail, int64_t(pa.n_app)});
    MARS_LAUNCH(k_patch_data, dim3(patch_grid(data_work)), dim3(256), 0, s, pa);
    MARS_LAUNCH(k_patch_rows, dim3(patch_grid(pa.n_rows)), dim3(256), 0, s, pa);
    MARS_HIP(hipStreamSynchronize(s));
    for (size_t i = 0; i < rows.size(); i += 3) {
        g.ro_h[size_t(rows[i])] = rows[i + 1];
        g.rcap_h[size_t(rows[i])] = int32_t(rows[i + 2]);
    }
    g.e_used = cursor;
    g.max_deg = max_deg;
    g.e = int32_t(std::min<int64_t>(int64_t(g.e) + added, INT32_MAX));
    if (out_knn && knn_k > 0) std::memcpy(out_knn, knn.data(), knn.size() * sizeof(int32_t));
    if (st) {
        mars_insert_stats r{};
        r.first_node = n_old;
        r.nodes_added = n_new;
        r.edges_added = added;
        r.rows_relocated = n_reloc;
        r.rows_appended = n_inplace;
        r.queryable_us = t_queryable;
        r.linked_us = us_since(t0);
        r.knn_us = double(knn_ms) * 1000.0;
        *st = r;
    }
    return MARS_OK;
}
