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
#include "device.hpp"

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
// Row ranges (workgroups) of an insert's neighbour search. The search reads the whole
// corpus for a few new nodes and shares HBM with queries in flight; on a quarter of
// the CUs it leaves them most of the bandwidth. At 1M nodes, 2,000 inserts/s and 500
// global queries/s: global p99 573 us with 256 ranges, 299 us with 64 (idle: 278),
// 336 us with 32; new nodes linked after 1.09 ms instead of 0.67 ms. The neighbours do
// not change: every range keeps its own 16 best candidates. Narrowing doubles the
// search's duration, so it applies up to kInsertKnnNarrowRows rows: beyond them one
// search per insert call already fills a large share of the GPU (at 13M rows a
// full-width search takes about 4 ms), and a longer one would only delay the writer.
constexpr int32_t kInsertKnnRanges = 64;
constexpr int64_t kInsertKnnNarrowRows = 2000000;
// Up to that size the narrow fp16 search runs first, its lists certified as the k-NN
// builders' are, and the int8 pass only for the nodes of a failed certificate: the int8
// pass at full width links in 0.29 ms at 1M rows but lifts the global p99 of concurrent
// queries from 199 to 304 us, and at 32 workgroups still to 235-257 us. Above it the int8
// pass runs first, at full width.

// Step 1 of an insert: the staged block (rows | modalities | times | episode ids |
// episode members | episode offsets) is scattered into the graph; each new row is also
// converted to fp16 (round to nearest even, as k_convert_f16) and its norms raise the fp16
// error bounds, and, when the graph holds the int8 copy, quantized into it by the same wave
// (quantize_row_i8, from the staged row). One wave per row, the attributes grid-stride.
struct StageArgs {
    const uint32_t* rows;      // n_new x d fp32 bit patterns
    const int32_t* mods;
    const float* ts;
    const int32_t* ep;         // null: no episode ids
    const int32_t* mem;        // null: no episode CSR
    const int32_t* off;
    float* emb;
    __half* emb16;             // null: no fp16 copy
    uint32_t* nrm;
    int8_t* emb8;              // null: no int8 copy
    float* meta8;
    uint32_t* nrm8;
    int32_t* g_mods;
    float* g_ts;
    int32_t* g_ep;
    int32_t* g_mem;
    int32_t* g_off;
    int64_t n_old;
    int32_t n_new;
    int32_t d;
    int32_t ne_new;
    int32_t mem_at;            // member_total
    int32_t off_at;            // num_eps + 1
};

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(8))) void k_stage_insert(StageArgs a) {
    __builtin_amdgcn_s_setprio(3);     // publication is latency-bound: first issue on a shared CU
    const int64_t tid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t stride = int64_t(gridDim.x) * blockDim.x;
    const int lane = int(threadIdx.x & 63u);
    for (int64_t r = tid >> 6; r < a.n_new; r += stride >> 6) {
        const uint32_t* src = a.rows + r * a.d;
        uint32_t* dst = reinterpret_cast<uint32_t*>(a.emb) + (a.n_old + r) * a.d;
        double s32 = 0.0, s16 = 0.0, sd = 0.0;
        // the row's words in registers, every load of a 768-word chunk issued at once, then
        // the copies: one memory latency per chunk, not one per 64 words (and few enough
        // registers that the kernel still fits beside a batched scan's workgroup)
        constexpr int kRowWords = 12;
        uint32_t w[kRowWords];
        for (int base = 0; base < a.d; base += 64 * kRowWords) {
#pragma unroll
        for (int j = 0; j < kRowWords; ++j) {
            const int i = base + lane + 64 * j;
            w[j] = i < a.d ? src[i] : 0u;
        }
#pragma unroll
        for (int j = 0; j < kRowWords; ++j) {
            const int i = base + lane + 64 * j;
            if (i >= a.d) continue;
            const uint32_t bits = w[j];
            dst[i] = bits;
            if (a.emb16) {
                const float x = __uint_as_float(bits);
                const __half h = __float2half_rn(x);
                a.emb16[(a.n_old + r) * a.d + i] = h;
                const float hv = __half2float(h);
                const float hf = fabsf(hv) < kHalfMinNormal ? 0.0f : hv;
                s32 += double(x) * double(x);
                s16 += double(hv) * double(hv);
                const double df = double(hf) - double(x);
                sd += df * df;
            }
        }
        }
        if (a.emb16 && a.nrm) raise_row_norms(s32, s16, sd, a.nrm);
        if (a.emb8) {
            const int64_t row = a.n_old + r;
            quantize_row_i8<4>(reinterpret_cast<const float*>(src), a.d, a.emb8, row, a.meta8 + 2 * row, a.nrm8);
        }
    }
    for (int64_t i = tid; i < a.n_new; i += stride) {
        a.g_mods[a.n_old + i] = a.mods[i];
        a.g_ts[a.n_old + i] = a.ts[i];
        if (a.g_ep) a.g_ep[a.n_old + i] = a.ep[i];
        if (a.g_mem) a.g_mem[a.mem_at + i] = a.mem[i];
    }
    for (int64_t e = tid; e < a.ne_new; e += stride) a.g_off[a.off_at + e] = a.off[e];
}

__global__ void k_patch_data(PatchArgs a) {
    __builtin_amdgcn_s_setprio(3);     // publication is latency-bound: first issue on a shared CU
    const int64_t tid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t stride = int64_t(gridDim.x) * blockDim.x;
    // relocations: one 64-lane wave per row (rows are short)
    const int64_t wave = tid >> 6, nwaves = stride >> 6;
    const int lane = int(threadIdx.x & 63u);
    // Edge-hit counters move with their edges and leave zeros behind (every source slot
    // is read by one thread only, and sources lie below the tail, destinations in it).
    for (int64_t r = wave; r < a.n_reloc; r += nwaves) {
        const int64_t src = a.reloc[3 * r], len = a.reloc[3 * r + 1], dst = a.reloc[3 * r + 2];
        for (int64_t i = lane; i < len; i += 64) {
            a.col[dst + i] = a.col[src + i];
            if (a.hits) {
                a.hits[dst + i] = a.hits[src + i];
                a.hits[src + i] = 0;
            }
        }
    }
    for (int64_t i = tid; i < a.n_tail; i += stride) {
        const int32_t v = a.tail[i];
        if (v == kCopySlot) continue;
        a.col[a.tail_base + i] = v;
        if (a.hits) {
            const int64_t src = a.tail_src ? a.tail_src[i] : -1;
            int32_t h = 0;
            if (src >= 0) {
                h = a.hits[src];
                a.hits[src] = 0;
            }
            a.hits[a.tail_base + i] = h;
        }
    }
    for (int64_t i = tid; i < a.n_app; i += stride) {
        a.col[a.app[2 * i]] = int32_t(a.app[2 * i + 1]);
        if (a.hits) a.hits[a.app[2 * i]] = 0;
    }
}

__global__ void k_patch_rows(PatchArgs a) {
    __builtin_amdgcn_s_setprio(3);     // publication is latency-bound: first issue on a shared CU
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

// Up to 16 nodes over the int8 copy: one k_scan8m pass (plain dots, self excluded), then
// k_cert_multi8's certified exact neighbours into g.ins_nbrs. *done = false when a node's
// certificate did not hold (the caller then runs the fp16 search for all of them).
int insert_knn_int8(Graph& g, int64_t first, int32_t nq, int64_t n, int32_t k, hipStream_t s, bool* done) {
    *done = false;
    const int32_t qmax = 8 * kScan8MMaxA;
    if (!g.ins8_part) {
        MARS_TRY(dmalloc(&g.ins8_part, size_t(qmax) * size_t(kScan8MPart)));
        MARS_TRY(dmalloc(&g.ins8_qa, size_t(kScan8MMaxA) * size_t(g.d / 64) * 1024));
        MARS_TRY(dmalloc(&g.ins8_qp, size_t(qmax) * 4));
        MARS_TRY(dmalloc(&g.ins8_stat, size_t(qmax)));
        MARS_TRY(dmalloc(&g.ins8_margin, size_t(qmax)));
    }
    if (nq > g.ins_cap_q) {
        dfree(g.ins_nbrs);
        g.ins_cap_q = 0;
        MARS_TRY(dmalloc(&g.ins_nbrs, size_t(nq) * 16));
        g.ins_cap_q = nq;
    }
    const float* rows = g.emb + first * g.d;
    const int32_t na = (nq + 7) / 8;
    Split8Args sp{};
    sp.q_glob = nullptr; sp.q_plain = rows; sp.nq = nq; sp.n_glob = 0; sp.d = g.d; sp.na = na; sp.nrm8 = g.nrm8;
    sp.qa = g.ins8_qa; sp.qp = g.ins8_qp;
    MARS_TRY(launch_split8(sp, s));
    int32_t rpw = 0, nwg = 0;
    scan_grid(n, kScan8MaxLists, &rpw, &nwg);
    Scan8MArgs sa{};
    sa.emb8 = g.emb8; sa.meta8 = g.meta8; sa.n = n; sa.d = g.d; sa.ts = g.ts; sa.mods = g.mods; sa.qa = g.ins8_qa;
    sa.qp = g.ins8_qp; sa.tq = nullptr; sa.lambda = 0.0f; sa.mod_filter = -1; sa.nq = nq; sa.n_glob = 0;
    sa.self_base = first; sa.part = g.ins8_part; sa.num_wg = nwg;
    MARS_TRY(launch_scan8m(sa, na, s));
    CertMArgs ca{};
    ca.part = g.ins8_part; ca.n_lists = nwg; ca.q = nq; ca.n_glob = 0; ca.q_glob = nullptr; ca.q_plain = rows;
    ca.d = g.d; ca.emb = g.emb; ca.ts = g.ts; ca.mods = g.mods; ca.tq = nullptr; ca.lambda = 0.0f;
    ca.mod_filter = -1; ca.qp = g.ins8_qp; ca.nrm8 = g.nrm8; ca.k = 1; ca.knn_k = k; ca.seeds = nullptr;
    ca.status = g.ins8_stat; ca.margin = g.ins8_margin; ca.knn_out = g.ins_nbrs;
    MARS_TRY(launch_cert_multi8(ca, s));
    int32_t stat[8 * kScan8MMaxA];
    MARS_HIP(hipMemcpyAsync(stat, g.ins8_stat, size_t(nq) * sizeof(int32_t), hipMemcpyDeviceToHost, s));
    MARS_HIP(hipStreamSynchronize(s));
    *done = std::all_of(stat, stat + nq, [](int32_t x) { return x == kMultiOk; });
    return MARS_OK;
}

// The fp16 search: a batched fp16 scan (no decay, no filter, self excluded) + exact fp32
// rescoring of 16 candidates per node into g.ins_nbrs. cert given: cert[i] = 1 when node
// first + i's list is certified exact (its k-th exact score beats the 16th candidate's
// fp16 score by the fp16 error bound).
int insert_knn_fp16(Graph& g, int64_t first, int32_t nq, int64_t n, int32_t k, hipStream_t s, int32_t* cert) {
    int32_t nrr = 0, nqb = 0;
    int64_t rpr = 0, part_keys = 0;
    const int32_t ranges = n <= kInsertKnnNarrowRows ? kInsertKnnRanges : 256;
    for (int32_t q : {std::min(nq, kInsertChunk), nq % kInsertChunk}) {   // full and last chunk
        if (q == 0) continue;
        batch_grid(n, q, true, &nrr, &nqb, &rpr, ranges);
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
        batch_grid(n, q, true, &nrr, &nqb, &rpr, ranges);
        BatchArgs a{};
        a.emb16 = g.emb16; a.n = n; a.d = g.d; a.qh = g.emb16 + (first + c0) * g.d; a.q = q; a.tq = g.ins_tq;
        a.ts = g.ts; a.mods = g.mods; a.lambda = 0.0f; a.mod_filter = -1; a.k = kKnnCand;
        a.q_plain = 0; a.self_base = first + c0; a.part = g.ins_part; a.rows_per_range = rpr; a.n_rranges = nrr;
        a.n_qblocks = nqb; a.uniform_tq = 1;
        MARS_TRY(launch_batch_topk(a, kKnnCand, g.ins_cand, s));
        MARS_TRY(launch_knn_rerank(g.emb, first + c0, q, g.d, g.ins_cand, kKnnCand, k, g.ins_nbrs + int64_t(c0) * k, s,
                                   cert ? g.nrm : nullptr, cert ? cert + c0 : nullptr));
    }
    return MARS_OK;
}

// k nearest neighbours of nodes [first, first + nq) among [0, n) into g.ins_nbrs. For at
// most 16 nodes over the int8 copy the result is certified exact: up to
// kInsertKnnNarrowRows rows the narrow fp16 search first and the int8 pass only when a
// list failed its certificate, above it the int8 pass first; when the int8 certificate
// fails too (or for more nodes, or without the int8 copy) the fp16 search's lists stand.
int insert_knn(Graph& g, int64_t first, int32_t nq, int64_t n, int32_t k, hipStream_t s) {
    const bool int8_ok = nq >= 1 && nq <= 8 * kScan8MMaxA && k <= 16 && cert_uses_int8(g);
    bool done = false;
    if (int8_ok && n > kInsertKnnNarrowRows) {
        MARS_TRY(insert_knn_int8(g, first, nq, n, k, s, &done));
        if (done) return MARS_OK;
        return insert_knn_fp16(g, first, nq, n, k, s, nullptr);
    }
    if (!int8_ok || !g.nrm) return insert_knn_fp16(g, first, nq, n, k, s, nullptr);
    if (!g.ins_cert) MARS_TRY(dmalloc(&g.ins_cert, size_t(8 * kScan8MMaxA)));
    MARS_TRY(insert_knn_fp16(g, first, nq, n, k, s, g.ins_cert));
    int32_t cert[8 * kScan8MMaxA];
    MARS_HIP(hipMemcpyAsync(cert, g.ins_cert, size_t(nq) * sizeof(int32_t), hipMemcpyDeviceToHost, s));
    MARS_HIP(hipStreamSynchronize(s));
    if (std::all_of(cert, cert + nq, [](int32_t x) { return x != 0; })) return MARS_OK;
    MARS_TRY(insert_knn_int8(g, first, nq, n, k, s, &done));
    if (done) return MARS_OK;
    return insert_knn_fp16(g, first, nq, n, k, s, nullptr);
}

// Copies rows out of col: spec holds n x {start, len, out offset}; one wave per row.
__global__ void k_gather_rows(const int32_t* __restrict__ col, const int64_t* __restrict__ spec, int32_t n,
                              int32_t* __restrict__ out) {
    const int64_t wave = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
    const int64_t nwaves = (int64_t(gridDim.x) * blockDim.x) >> 6;
    const int lane = int(threadIdx.x & 63u);
    for (int64_t r = wave; r < n; r += nwaves) {
        const int64_t start = spec[3 * r], len = spec[3 * r + 1], off = spec[3 * r + 2];
        for (int64_t i = lane; i < len; i += 64) out[off + i] = col[start + i];
    }
}

// A planned edit of col: relocations (device copies of old rows into the tail), appends
// into row slack, the tail region [base, cursor) and the new row words.
struct Patch {
    std::vector<int64_t> reloc, app, rows;
    std::vector<int32_t> tail;
    std::vector<int64_t> tail_src;   // with edge-hit counters: source slot of each tail entry (-1 new)
    int64_t base = 0, cursor = 0, added = 0;
    int32_t max_deg = 0, n_reloc = 0, n_inplace = 0;
    bool track_src = false;
    int64_t place(int64_t cap) {
        const int64_t at = cursor;
        tail.resize(size_t(at + cap - base), -1);
        if (!tail_src.empty() || track_src) tail_src.resize(tail.size(), -1);
        cursor += cap;
        return at;
    }
};

// Writes the column data, then publishes the row words (a later kernel on the same
// stream), and updates the host mirrors.
int commit_patch(Graph& g, Patch& p, hipStream_t s) {
    const size_t b_reloc = p.reloc.size() * sizeof(int64_t), b_app = p.app.size() * sizeof(int64_t);
    const size_t b_rows = p.rows.size() * sizeof(int64_t), b_tail = p.tail.size() * sizeof(int32_t);
    const size_t b_src = p.tail_src.size() * sizeof(int64_t);
    const size_t total = b_reloc + b_app + b_rows + b_tail + b_src + 96;   // + 16-byte padding of 5 pieces
    MARS_TRY(grow_pinned<char>(&g.ins_pin, &g.ins_pin_bytes, total));
    MARS_TRY(grow_device(&g.ins_dev, &g.ins_dev_bytes, total));
    char* pin = static_cast<char*>(g.ins_pin);
    char* dev = static_cast<char*>(g.ins_dev);
    size_t off = 0;
    auto put = [&](const void* src, size_t bytes) {
        const size_t at = off;
        if (bytes) std::memcpy(pin + at, src, bytes);
        off += (bytes + 15) / 16 * 16;
        return at;
    };
    const size_t o_reloc = put(p.reloc.data(), b_reloc), o_app = put(p.app.data(), b_app);
    const size_t o_rows = put(p.rows.data(), b_rows), o_tail = put(p.tail.data(), b_tail);
    const size_t o_src = p.tail_src.empty() ? 0 : put(p.tail_src.data(), b_src);
    MARS_HIP(hipMemcpyAsync(dev, pin, off, hipMemcpyHostToDevice, s));
    PatchArgs pa{};
    pa.col = g.col; pa.ro = g.ro; pa.rcap = g.rcap;
    pa.reloc = reinterpret_cast<const int64_t*>(dev + o_reloc); pa.n_reloc = int32_t(p.reloc.size() / 3);
    pa.tail = reinterpret_cast<const int32_t*>(dev + o_tail); pa.tail_base = p.base;
    pa.n_tail = int64_t(p.tail.size());
    pa.app = reinterpret_cast<const int64_t*>(dev + o_app); pa.n_app = int32_t(p.app.size() / 2);
    pa.rows = reinterpret_cast<const int64_t*>(dev + o_rows); pa.n_rows = int32_t(p.rows.size() / 3);
    pa.hits = g.hits;
    pa.tail_src = p.tail_src.empty() ? nullptr : reinterpret_cast<const int64_t*>(dev + o_src);
    const int64_t data_work = std::max<int64_t>({int64_t(pa.n_reloc) * 64, pa.n_tail, int64_t(pa.n_app)});
    MARS_LAUNCH(k_patch_data, dim3(patch_grid(data_work)), dim3(256), 0, s, pa);
    MARS_LAUNCH(k_patch_rows, dim3(patch_grid(pa.n_rows)), dim3(256), 0, s, pa);
    MARS_HIP(hipStreamSynchronize(s));
    for (size_t i = 0; i < p.rows.size(); i += 3) {
        g.ro_h[size_t(p.rows[i])] = p.rows[i + 1];
        g.rcap_h[size_t(p.rows[i])] = int32_t(p.rows[i + 2]);
    }
    if (p.cursor > p.base) g.e_used = p.cursor;
    g.max_deg = p.max_deg;
    g.e = int32_t(std::min<int64_t>(int64_t(g.e) + p.added, INT32_MAX));
    ++g.csr_version;
    return MARS_OK;
}

}  // namespace

// k-NN edges of nodes [first, first + count) (already published), knn: count x k ids
// among [0, g.n): the edge set becomes E u {(u, v), (v, u)} for every listed neighbour
// v != u; rows stay ascending and free of duplicates. Rows that only gain ids above
// their last entry and have slack append in place; the others are rewritten whole
// into a fresh tail region (the host gathers their current content first).
// Caller holds the graph mutex.
int link_knn_apply(Graph& g, int32_t first, int32_t count, int32_t k, const int32_t* knn, hipStream_t s,
                   mars_insert_stats* st) {
    const int32_t n = g.n;
    // rows touched: the linked nodes and their neighbours
    std::vector<int32_t> touched;
    touched.reserve(size_t(count) * size_t(k + 1));
    for (int32_t i = 0; i < count; ++i) {
        touched.push_back(first + i);
        for (int32_t j = 0; j < k; ++j) {
            const int32_t v = knn[size_t(i) * k + j];
            if (v >= 0 && v < n && v != first + i) touched.push_back(v);
        }
    }
    std::sort(touched.begin(), touched.end());
    touched.erase(std::unique(touched.begin(), touched.end()), touched.end());
    // gather their current content
    std::vector<int64_t> spec(touched.size() * 3);
    int64_t total = 0;
    for (size_t i = 0; i < touched.size(); ++i) {
        const int64_t w = g.ro_h[size_t(touched[i])];
        spec[3 * i] = int64_t(uint32_t(w));
        spec[3 * i + 1] = w >> 32;
        spec[3 * i + 2] = total;
        total += w >> 32;
    }
    const size_t b_spec = spec.size() * sizeof(int64_t), b_out = size_t(total) * sizeof(int32_t);
    MARS_TRY(grow_pinned<char>(&g.ins_pin, &g.ins_pin_bytes, b_spec + b_out + 64));
    MARS_TRY(grow_device(&g.ins_dev, &g.ins_dev_bytes, b_spec + b_out + 64));
    char* pin = static_cast<char*>(g.ins_pin);
    char* dev = static_cast<char*>(g.ins_dev);
    const size_t o_out = (b_spec + 15) / 16 * 16;
    std::memcpy(pin, spec.data(), b_spec);
    MARS_HIP(hipMemcpyAsync(dev, pin, b_spec, hipMemcpyHostToDevice, s));
    if (!touched.empty())
        MARS_LAUNCH(k_gather_rows, dim3(patch_grid(int64_t(touched.size()) * 64)), dim3(256), 0, s, g.col,
                    reinterpret_cast<const int64_t*>(dev), int32_t(touched.size()),
                    reinterpret_cast<int32_t*>(dev + o_out));
    if (b_out) MARS_HIP(hipMemcpyAsync(pin + o_out, dev + o_out, b_out, hipMemcpyDeviceToHost, s));
    MARS_HIP(hipStreamSynchronize(s));
    const int32_t* content = reinterpret_cast<const int32_t*>(pin + o_out);
    auto row_of = [&](int32_t v) {
        const size_t i = size_t(std::lower_bound(touched.begin(), touched.end(), v) - touched.begin());
        const int32_t* at = content + spec[3 * i + 2];            // offset in the gathered copy
        return std::make_pair(at, at + spec[3 * i + 1]);
    };
    // directed additions not already present
    std::vector<std::pair<int32_t, int32_t>> add;
    for (int32_t i = 0; i < count; ++i) {
        const int32_t u = first + i;
        for (int32_t j = 0; j < k; ++j) {
            const int32_t v = knn[size_t(i) * k + j];
            if (v < 0 || v >= n || v == u) continue;
            add.emplace_back(u, v);
            add.emplace_back(v, u);
        }
    }
    std::sort(add.begin(), add.end());
    add.erase(std::unique(add.begin(), add.end()), add.end());
    add.erase(std::remove_if(add.begin(), add.end(), [&](const std::pair<int32_t, int32_t>& e) {
                  const auto r = row_of(e.first);
                  return std::find(r.first, r.second, e.second) != r.second;   // rows may be unsorted
              }), add.end());
    Patch p;
    p.base = align_up(g.e_used, kRegionAlign);
    p.cursor = p.base;
    p.max_deg = g.max_deg;
    p.track_src = g.hits != nullptr;
    std::vector<std::pair<int32_t, int64_t>> merged;   // (neighbour, col slot it came from or -1)
    for (size_t i = 0, j = 0; i < add.size(); i = j) {
        const int32_t r = add[i].first;
        while (j < add.size() && add[j].first == r) ++j;
        const auto row = row_of(r);
        const int64_t len = row.second - row.first, a = int64_t(j - i);
        const int64_t w = g.ro_h[size_t(r)];
        const int64_t start = int64_t(uint32_t(w)), cap = g.rcap_h[size_t(r)];
        const bool ascending = std::is_sorted(row.first, row.second);
        const int64_t nlen = len + a;
        int64_t nstart = start, ncap = cap;
        if (ascending && (len == 0 || add[i].second > row.second[-1]) && nlen <= cap) {
            for (size_t x = i; x < j; ++x) {
                p.app.push_back(start + len + int64_t(x - i));
                p.app.push_back(add[x].second);
            }
            ++p.n_inplace;
        } else {
            merged.clear();
            for (int64_t x = 0; x < len; ++x) merged.emplace_back(row.first[x], start + x);
            for (size_t x = i; x < j; ++x) merged.emplace_back(add[x].second, -1);
            std::sort(merged.begin(), merged.end());
            ncap = row_capacity(nlen);
            nstart = p.place(ncap);
            for (size_t x = 0; x < merged.size(); ++x) {
                p.tail[size_t(nstart - p.base) + x] = merged[x].first;
                if (p.track_src) p.tail_src[size_t(nstart - p.base) + x] = merged[x].second;
            }
            ++p.n_reloc;
        }
        p.rows.push_back(r); p.rows.push_back((nlen << 32) | int64_t(uint32_t(nstart))); p.rows.push_back(ncap);
        p.max_deg = std::max<int32_t>(p.max_deg, int32_t(nlen));
        p.added += a;
    }
    MARS_CHECK(p.cursor <= g.cap_e && p.cursor <= int64_t(UINT32_MAX), MARS_ERR_CAPACITY,
               "link: edge capacity %lld too small (used %lld, this link needs %lld)", (long long)g.cap_e,
               (long long)g.e_used, (long long)(p.cursor - g.e_used));
    if (!p.rows.empty()) MARS_TRY(commit_patch(g, p, s));
    if (st) {
        st->first_node = first;
        st->nodes_added = count;
        st->edges_added = p.added;
        st->rows_relocated = p.n_reloc;
        st->rows_appended = p.n_inplace;
    }
    return MARS_OK;
}

int graph_insert_free(Graph& g) {
    if (g.ins_pin) (void)hipHostFree(g.ins_pin);
    g.ins_pin = nullptr;
    g.ins_pin_bytes = 0;
    if (g.ins_dev) (void)hipFree(g.ins_dev);
    g.ins_dev = nullptr;
    g.ins_dev_bytes = 0;
    dfree(g.ins_part); dfree(g.ins_cand); dfree(g.ins_nbrs); dfree(g.ins_tq);
    dfree(g.ins8_part); dfree(g.ins8_qa); dfree(g.ins8_qp); dfree(g.ins8_stat); dfree(g.ins8_margin); dfree(g.ins_cert);
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
    if (ep_ids) std::memcpy(p_ep, ep_ids, att_bytes);
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
    }
    // one copy of the staged block, one kernel to place it (each GPU operation waits for
    // a dispatch slot when scans fill the GPU, so an insert issues as few as it can)
    MARS_TRY(grow_device(&g.ins_dev, &g.ins_dev_bytes, stage1));
    char* dev = static_cast<char*>(g.ins_dev);
    MARS_HIP(hipMemcpyAsync(dev, pin, stage1, hipMemcpyHostToDevice, s));
    StageArgs sa{};
    sa.rows = reinterpret_cast<const uint32_t*>(dev);
    sa.mods = reinterpret_cast<const int32_t*>(dev + (p_mods - pin));
    sa.ts = reinterpret_cast<const float*>(dev + (p_ts - pin));
    sa.ep = ep_ids ? reinterpret_cast<const int32_t*>(dev + (p_ep - pin)) : nullptr;
    sa.mem = ep_csr ? reinterpret_cast<const int32_t*>(dev + (reinterpret_cast<char*>(p_mem) - pin)) : nullptr;
    sa.off = ep_csr ? reinterpret_cast<const int32_t*>(dev + (reinterpret_cast<char*>(p_off) - pin)) : nullptr;
    sa.emb = g.emb; sa.emb16 = g.emb16; sa.nrm = g.nrm;
    sa.emb8 = g.emb8; sa.meta8 = g.meta8; sa.nrm8 = g.nrm8;
    sa.g_mods = g.mods; sa.g_ts = g.ts; sa.g_ep = ep_ids ? g.ep_ids : nullptr;
    sa.g_mem = ep_csr ? g.ep_mem : nullptr; sa.g_off = ep_csr ? g.ep_off : nullptr;
    sa.n_old = n_old; sa.n_new = n_new; sa.d = int32_t(D); sa.ne_new = ne_new;
    sa.mem_at = g.member_total; sa.off_at = g.num_eps + 1;
    MARS_LAUNCH(k_stage_insert, dim3(patch_grid(int64_t(n_new) * 64)), dim3(256), 0, s, sa);
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
    Patch p;
    p.base = align_up(g.e_used, kRegionAlign);
    p.cursor = p.base;
    p.max_deg = g.max_deg;
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
                p.app.push_back(start + len + x);
                p.app.push_back(old_add[i + size_t(x)].second);
            }
            ++p.n_inplace;
        } else {
            ncap = row_capacity(nlen);
            nstart = p.place(ncap);
            p.reloc.push_back(start); p.reloc.push_back(len); p.reloc.push_back(nstart);
            for (int64_t x = 0; x < len; ++x) p.tail[size_t(nstart - p.base + x)] = kCopySlot;
            for (int64_t x = 0; x < a; ++x) p.tail[size_t(nstart - p.base + len + x)] = old_add[i + size_t(x)].second;
            ++p.n_reloc;
        }
        const int64_t nw = (nlen << 32) | int64_t(uint32_t(nstart));
        p.rows.push_back(v); p.rows.push_back(nw); p.rows.push_back(ncap);
        p.max_deg = std::max<int32_t>(p.max_deg, int32_t(nlen));
        p.added += a;
    }
    for (int32_t i = 0; i < n_new; ++i) {
        const auto& r = nrow[size_t(i)];
        const int64_t len = int64_t(r.size()), cap = row_capacity(len);
        const int64_t at = p.place(cap);
        std::memcpy(p.tail.data() + (at - p.base), r.data(), r.size() * sizeof(int32_t));
        const int64_t nw = (len << 32) | int64_t(uint32_t(at));
        p.rows.push_back(n_old + i); p.rows.push_back(nw); p.rows.push_back(cap);
        p.max_deg = std::max<int32_t>(p.max_deg, int32_t(len));
        p.added += len;
    }
    if (p.cursor > g.cap_e || p.cursor > int64_t(UINT32_MAX)) {
        if (early)      // cannot happen: the worst case fitted
            return set_error(MARS_ERR_CAPACITY, "insert: planned %lld col slots beyond the worst case "
                             "(nodes published without edges)", (long long)p.cursor);
        return set_error(MARS_ERR_CAPACITY, "insert: edge capacity %lld too small (used %lld, this insert "
                         "needs %lld)", (long long)g.cap_e, (long long)g.e_used, (long long)(p.cursor - g.e_used));
    }
    if (!early) publish();

    // ---- step 4: write column data, then publish the row words ------------------------------
    MARS_TRY(commit_patch(g, p, s));
    if (out_knn && knn_k > 0) std::memcpy(out_knn, knn.data(), knn.size() * sizeof(int32_t));
    if (st) {
        mars_insert_stats r{};
        r.first_node = n_old;
        r.nodes_added = n_new;
        r.edges_added = p.added;
        r.rows_relocated = p.n_reloc;
        r.rows_appended = p.n_inplace;
        r.queryable_us = t_queryable;
        r.linked_us = us_since(t0);
        r.knn_us = double(knn_ms) * 1000.0;
        *st = r;
    }
    return MARS_OK;
}

extern "C" int mars_graph_link(mars_graph* gh, int32_t first, int32_t count, int32_t k, const int32_t* nbrs,
                               mars_insert_stats* st) {
    const auto t0 = std::chrono::steady_clock::now();
    MARS_CHECK(gh && count >= 0 && k >= 0 && (count == 0 || k == 0 || nbrs), MARS_ERR_INVALID,
               "link: bad arguments");
    std::lock_guard<std::mutex> lock(gh->mu);
    Graph& g = gh->g;
    MARS_CHECK(first >= 0 && int64_t(first) + count <= g.n, MARS_ERR_INVALID,
               "link: nodes [%d, %lld) are not all published (%d nodes)", first, (long long)first + count, g.n);
    MARS_TRY(use_device(g.device));
    mars_insert_stats r{};
    if (count > 0 && k > 0) MARS_TRY(link_knn_apply(g, first, count, k, nbrs, g.ins_stream, &r));
    r.first_node = first;
    r.nodes_added = count;
    r.linked_us = us_since(t0);
    if (st) *st = r;
    return MARS_OK;
}

extern "C" int mars_graph_link_knn(mars_graph* gh, int32_t first, int32_t count, int32_t knn_k, int32_t* out_knn,
                                   mars_insert_stats* st) {
    const auto t0 = std::chrono::steady_clock::now();
    MARS_CHECK(gh && count >= 0 && knn_k >= 1 && knn_k <= 16, MARS_ERR_INVALID,
               "link: bad arguments (count %d, knn_k %d)", count, knn_k);
    std::lock_guard<std::mutex> lock(gh->mu);
    Graph& g = gh->g;
    MARS_CHECK(first >= 0 && int64_t(first) + count <= g.n, MARS_ERR_INVALID,
               "link: nodes [%d, %lld) are not all published (%d nodes)", first, (long long)first + count, g.n);
    MARS_CHECK(g.emb16 != nullptr, MARS_ERR_UNSUPPORTED, "link: the neighbour search reads the fp16 rows; "
               "enable them first");
    MARS_CHECK(batch_dim_supported(g.d), MARS_ERR_UNSUPPORTED, "link: embedding_dim %d unsupported", g.d);
    MARS_TRY(use_device(g.device));
    hipStream_t s = g.ins_stream;
    for (auto& e : g.ins_ev)
        if (!e) MARS_HIP(hipEventCreate(&e));
    mars_insert_stats r{};
    std::vector<int32_t> knn(size_t(count) * size_t(knn_k), -1);
    float knn_ms = 0.0f;
    if (count > 0) {
        MARS_HIP(hipEventRecord(g.ins_ev[0], s));
        MARS_TRY(insert_knn(g, first, count, g.n, knn_k, s));
        MARS_HIP(hipEventRecord(g.ins_ev[1], s));
        MARS_HIP(hipMemcpyAsync(knn.data(), g.ins_nbrs, knn.size() * sizeof(int32_t), hipMemcpyDeviceToHost, s));
        MARS_HIP(hipStreamSynchronize(s));
        MARS_HIP(hipEventElapsedTime(&knn_ms, g.ins_ev[0], g.ins_ev[1]));
        MARS_TRY(link_knn_apply(g, first, count, knn_k, knn.data(), s, &r));
    }
    r.first_node = first;
    r.nodes_added = count;
    r.linked_us = us_since(t0);
    r.knn_us = double(knn_ms) * 1000.0;
    if (out_knn && count > 0) std::memcpy(out_knn, knn.data(), knn.size() * sizeof(int32_t));
    if (st) *st = r;
    return MARS_OK;
}

// In-place update of published rows (the engine server's ADD of an existing id and its
// DELETE tombstone): new fp32 rows, modalities and timestamps; the fp16 copy and its
// norm bounds follow (the bounds only rise, so the certificate stays valid). Edges are
// unchanged. Rows being replaced must not be read by a concurrent query.
extern "C" int mars_graph_set_rows(mars_graph* gh, int32_t first, int32_t count, const float* emb,
                                   const int32_t* mods, const float* ts) {
    MARS_CHECK(gh && emb && mods && ts, MARS_ERR_INVALID, "null argument");
    std::lock_guard<std::mutex> lock(gh->mu);
    Graph& g = gh->g;
    MARS_CHECK(first >= 0 && count > 0 && int64_t(first) + count <= g.n, MARS_ERR_INVALID,
               "rows [%d, %lld) outside the %d published nodes", first, (long long)first + count, g.n);
    MARS_TRY(use_device(g.device));
    hipStream_t s = g.ins_stream;
    const size_t D = size_t(g.d);
    MARS_HIP(hipMemcpyAsync(g.emb + size_t(first) * D, emb, size_t(count) * D * sizeof(float),
                            hipMemcpyHostToDevice, s));
    MARS_HIP(hipMemcpyAsync(g.mods + first, mods, size_t(count) * sizeof(int32_t), hipMemcpyHostToDevice, s));
    MARS_HIP(hipMemcpyAsync(g.ts + first, ts, size_t(count) * sizeof(float), hipMemcpyHostToDevice, s));
    if (g.emb16) {
        MARS_TRY(launch_convert_f16(g.emb + size_t(first) * D, g.emb16 + size_t(first) * D, int64_t(count) * g.d, s));
        MARS_TRY(launch_row_norms(g.emb, g.emb16, first, int64_t(first) + count, g.d, g.nrm, s));
    }
    if (g.emb8) MARS_TRY(launch_convert_i8(g.emb, first, int64_t(first) + count, g.d, g.emb8, g.meta8, g.nrm8, s));
    MARS_HIP(hipStreamSynchronize(s));
    return MARS_OK;
}
