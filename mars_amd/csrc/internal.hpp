// ============================================================================
//  internal.hpp — shared internals of libmars_amd (gfx950 only).
//
//  Score keys. Every selection in the library (per-wave top-K, seed merge,
//  final result order) compares 64-bit keys
//        key = (desc32(score) << 32) | node_id
//  where desc32 is an order-reversing bijection of fp32 (larger score ->
//  smaller key, -0.0 folded onto +0.0). Ascending keys are therefore
//  (score desc, node id asc): the order of a stable ascending radix sort of
//  negated scores (reference: src/memory_cuda.cu:1254-1283) and a total order,
//  so top-K and final results are deterministic.
// ============================================================================
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdint>
#include <cstdio>
#include <mutex>
#include <string>
#include <vector>

#include "mars_amd.h"

namespace mars {

// ---- error reporting ---------------------------------------------------------
int set_error(int code, const char* fmt, ...);

// Takes the device address of mars_query_batch_static's scratch array on `dev` (the
// current device) once; mars_init and mars_graph_create call it.
int noalloc_prepare(int dev);
#define MARS_HIP(call)                                                               \
    do {                                                                             \
        hipError_t e__ = (call);                                                     \
        if (e__ != hipSuccess)                                                       \
            return ::mars::set_error(MARS_ERR_HIP, "%s:%d %s -> %s", __FILE__, __LINE__, \
                                     #call, hipGetErrorString(e__));                 \
    } while (0)
#define MARS_CHECK(cond, code, ...)                                                  \
    do {                                                                             \
        if (!(cond)) return ::mars::set_error((code), __VA_ARGS__);                  \
    } while (0)

// Launch a kernel and report this launch's own error only. The thread's last-error
// state can still hold an error that an earlier HIP call recovered from by itself (a
// large pageable copy whose source the runtime failed to pin, then staged), which a
// bare hipGetLastError after the launch would report as the launch's.
#define MARS_LAUNCH(...)                  \
    do {                                  \
        (void)hipGetLastError();          \
        hipLaunchKernelGGL(__VA_ARGS__);  \
        MARS_HIP(hipGetLastError());      \
    } while (0)

#define MARS_TRY(expr)                    \
    do {                                  \
        int rc__ = (expr);                \
        if (rc__ != MARS_OK) return rc__; \
    } while (0)

inline int use_device(int dev) {
    int cur = -1;
    MARS_HIP(hipGetDevice(&cur));
    if (cur != dev) MARS_HIP(hipSetDevice(dev));
    return MARS_OK;
}

template <typename T>
int dmalloc(T** p, size_t count) {
    *p = nullptr;
    if (count == 0) count = 1;
    hipError_t e = hipMalloc(reinterpret_cast<void**>(p), count * sizeof(T));
    if (e != hipSuccess)
        return set_error(MARS_ERR_NOMEM, "hipMalloc(%zu bytes): %s", count * sizeof(T), hipGetErrorString(e));
    return MARS_OK;
}

template <typename T>
void dfree(T*& p) {
    if (p) (void)hipFree(p);
    p = nullptr;
}

// Row ranges x query blocks of the batched scan (defined in api.hip). plain: every query
// is a neighbour search (BatchArgs::q_plain == 0), which picks the kernel as in
// batch_uses_gemm. max_ranges caps the row ranges (workgroups per 64-query block).
void batch_grid(int64_t n, int32_t q, bool plain, int32_t* n_rranges, int32_t* n_qblocks, int64_t* rows_per_range,
                int32_t max_ranges = 256);

constexpr int kMaxK = 64;              // seeds per query (wave-held list), as MAX_TOP_K
constexpr int kSortCap = 8192;         // results sorted in LDS by the finalize kernel (one band)
constexpr int kCompactPerK = 500;      // result cap per seed slot: the reference's max_compact = max_k * 500
constexpr int kFrontierChunk = 4096;   // frontier nodes per BFS chunk (LDS)
constexpr uint64_t kEmptyKey = ~0ull;
// batched global queries: fp16 candidates per query (the batched scan's list), and
// visit slots per query (the LDS-hash BFS never visits more than 6144 + 1024 nodes)
constexpr int kMultiCand = 16;
constexpr int kMultiVisit = 8192;
constexpr int32_t kMultiUncertified = 0;   // seeds not certified: answered by the Q=1 path
constexpr int32_t kMultiOk = 1;
constexpr int32_t kMultiOverflow = 2;      // visit set outgrew the LDS hash: Q=1 path

// ---- score keys ----------------------------------------------------------------
__host__ __device__ inline uint32_t desc32(float s) {
    s = s + 0.0f;                                   // -0.0 -> +0.0
    uint32_t u;
    __builtin_memcpy(&u, &s, 4);
    const uint32_t asc = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ~asc;
}
__host__ __device__ inline float desc32_inv(uint32_t k) {
    const uint32_t asc = ~k;
    const uint32_t u = (asc & 0x80000000u) ? (asc & 0x7fffffffu) : ~asc;
    float s;
    __builtin_memcpy(&s, &u, 4);
    return s;
}
__host__ __device__ inline uint64_t make_key(float s, uint32_t id) {
    return (uint64_t(desc32(s)) << 32) | id;
}
__host__ __device__ inline float key_score(uint64_t k) { return desc32_inv(uint32_t(k >> 32)); }
__host__ __device__ inline int32_t key_id(uint64_t k) { return int32_t(uint32_t(k)); }

// ---- device objects ---------------------------------------------------------------
struct Graph {
    int device = 0;
    int32_t n = 0;            // live nodes (published with __atomic_store_n; queries load it once)
    int32_t e = 0;            // live edges (col entries)
    int32_t d = 0;
    int32_t cap_n = 0;
    int64_t cap_e = 0;
    float* emb = nullptr;
    __half* emb16 = nullptr;
    // with the fp16 copy: upper bounds over the rows of max |e|, |e16| and |e16 - e|
    // (Euclidean norms; e16 with subnormals flushed in the difference), fp32 bit
    // patterns rounded up, raised by atomicMax as rows are converted
    uint32_t* nrm = nullptr;
    // the int8 copy (certified global queries): row r as bytes v in [-127, 127] with one
    // scale, meta8[2r] = s_r (e^ = s_r v), meta8[2r+1] = c_r, the row's bound on
    // |int8 scan dot - fp32 scan dot| / |q|; nrm8[0] = max c_r, nrm8[1] = max |e| (fp32
    // bit patterns rounded up, raised by atomicMax as rows are quantized)
    int8_t* emb8 = nullptr;
    float* meta8 = nullptr;
    uint32_t* nrm8 = nullptr;
    int32_t* mods = nullptr;
    float* ts = nullptr;
    int64_t* ro = nullptr;    // cap_n: (row length << 32) | row start in col
    int32_t* rcap = nullptr;  // cap_n: slots reserved for the row in col (>= length)
    int32_t* col = nullptr;   // cap_e
    int32_t* ep_ids = nullptr;
    int32_t* ep_off = nullptr;
    int32_t* ep_mem = nullptr;
    int32_t num_eps = 0;
    int32_t member_total = 0;
    // host mirrors of the row words / capacities and the used part of col
    std::vector<int64_t> ro_h;
    std::vector<int32_t> rcap_h;
    int64_t e_used = 0;
    int32_t max_deg = 0;                 // longest row
    // streaming inserts (under the graph mutex)
    hipStream_t ins_stream = nullptr;    // side stream
    int32_t ep_next = 0;                 // smallest episode id an insert may open
    int64_t ep_off_cap = 0;              // entries allocated in ep_off / ep_mem
    int64_t ep_mem_cap = 0;
    void* ins_pin = nullptr;             // pinned staging of rows and row patches
    size_t ins_pin_bytes = 0;
    void* ins_dev = nullptr;             // device copy of the row patches
    size_t ins_dev_bytes = 0;
    uint64_t* ins_part = nullptr;        // batched-scan keys of the neighbour search
    int64_t ins_part_cap = 0;
    uint64_t* ins_cand = nullptr;        // merged candidates (1024 x 16)
    int32_t* ins_nbrs = nullptr;         // rescored neighbours
    float* ins_tq = nullptr;             // zero query times (no decay)
    int32_t ins_cap_q = 0;
    hipEvent_t ins_ev[2] = {nullptr, nullptr};
    // the last k-NN builder call: nodes whose lists the certificate did not cover, and of
    // those, how many were found again by exact scans
    int64_t knn_uncertified = 0;
    int64_t knn_rescanned = 0;
    // the neighbour search of up to 16 new nodes over the int8 copy (one k_scan8m pass)
    uint64_t* ins8_part = nullptr;       // [16][kScan8MPart]
    unsigned char* ins8_qa = nullptr;    // A operands
    float* ins8_qp = nullptr;            // [16][4]
    int32_t* ins8_stat = nullptr;        // [16] certificate status
    float* ins8_margin = nullptr;        // [16]
    int32_t* ins_cert = nullptr;         // [16] fp16 k-NN certificate flags
    // importance and edge-hit counters (allocated on request, under the graph mutex)
    float* imp = nullptr;                // cap_n: importance of each node
    int32_t* hits = nullptr;             // cap_e: BFS hits per col slot; slots no row uses hold 0
    int32_t* imp_ids = nullptr;          // device copy of host-supplied boost ids
    int64_t imp_ids_cap = 0;
    unsigned long long* sweep_cnt = nullptr;   // edges counted by the maintenance sweep
    // the packed CSR export (mars_graph_packed_csr), rebuilt when csr_version moved on
    uint64_t csr_version = 0;            // bumped by every change of the edge set
    uint64_t pk_version = ~0ull;
    int32_t* pk_row = nullptr;           // [pk_cap_n + 1]
    int32_t* pk_col = nullptr;           // [pk_cap_e]
    int64_t pk_cap_n = 0;
    int64_t pk_cap_e = 0;
};

// Result staging written by the finalize / episode kernels straight into
// pinned host memory (one PCIe write burst, no D2H copy).
struct ResultHeader {
    int32_t count;        // results written (<= requested cap)
    int32_t visited;      // nodes reached (seeds + BFS)
    int32_t levels;       // BFS levels expanded
    int32_t n_seeds;      // seeds selected
};

struct Ctx {
    int device = 0;
    int32_t max_nodes = 0;
    int32_t d = 0;
    int32_t max_k = 0;
    uint32_t flags = 0;
    hipStream_t stream = nullptr;
    // device scratch
    float* query = nullptr;        // d
    float* fin = nullptr;          // max_nodes: fused score of the last global query
    uint64_t* part = nullptr;      // max_wg * kMaxK candidate keys
    uint64_t* gthr = nullptr;      // scan's running K-th key bound (reset by finalize)
    uint32_t* gcnt = nullptr;      // candidate count (reset by finalize)
    int32_t max_wg = 0;
    uint32_t* vis = nullptr;       // max_nodes visit stamps (epoch)
    uint64_t* claim = nullptr;     // max_nodes BFS claim keys
    int32_t* vlist = nullptr;      // max_nodes visit order (node ids)
    int32_t* vhop = nullptr;       // max_nodes
    float* vscore = nullptr;       // max_nodes
    int64_t* vro = nullptr;        // max_nodes: row (len << 32 | start) of each visited node
    uint64_t* sortbuf = nullptr;   // max_nodes keys (large-result fallback)
    int32_t* seed_idx = nullptr;   // kMaxK
    uint64_t* stamps = nullptr;    // phase stamps (100 MHz realtime counter): device alias of h_stamps
    uint64_t* h_stamps = nullptr;  // 12 stamps in pinned, mapped host memory
    float* seed_val = nullptr;     // kMaxK
    // pinned host staging
    float* h_query = nullptr;      // d
    ResultHeader* h_res = nullptr; // header + results
    mars_query_result* h_rec = nullptr;
    ResultHeader* d_res = nullptr; // device alias of h_res
    mars_query_result* d_rec = nullptr;
    // Completion word (pinned, mapped): the last kernel of a Q=1 query writes the
    // query's sequence number into it after a system-scope fence on its result
    // writes; the host spins on it instead of a stream synchronize (about 5 us less
    // per query, and a tighter tail).
    uint32_t* h_done = nullptr;
    uint32_t* d_done = nullptr;
    uint32_t seq = 0;
    int32_t res_cap = 0;
    uint32_t epoch = 0;            // last visit stamp used
    uint32_t gen = 0;              // next BFS claim generation
    hipEvent_t ev[4] = {nullptr, nullptr, nullptr, nullptr};
    int32_t last_n = 0;            // node count of the last global query
    int32_t last_k = 0;
    int32_t last_visited = 0;      // visit-list length of the last global query
    int32_t last_certified = 0;    // the last global query took the certified path
    // BFS levels of the last global query (edge-hit counting): its visit list
    const int32_t* hit_vlist = nullptr;
    const int32_t* hit_vhop = nullptr;
    int32_t hit_n = 0;
    uint64_t* hopmap = nullptr;    // max_nodes: (stamp << 32) | hop of each visited node
    uint32_t hop_stamp = 0;
    // batched scoring scratch (grown on demand)
    __half* bq = nullptr;          // queries in fp16
    float* btq = nullptr;          // query times
    uint64_t* bpart = nullptr;     // per-(query, row range) keys
    uint64_t* bout = nullptr;      // merged keys per query
    int32_t bcap_q = 0;
    int64_t bcap_part = 0;
    // batched global queries (grown on demand; kMultiVisit visit slots per query)
    double* mqn = nullptr;         // [q][4] |q|, |q16|, |q16 - q|
    uint64_t* mseed = nullptr;     // [q][kMultiCand] certified exact seed keys
    int32_t* mstat = nullptr;      // [q] kMultiOk / kMultiUncertified / kMultiOverflow
    int32_t* minfo = nullptr;      // [q][4] visited, levels, seeds
    float* mmargin = nullptr;      // [q] certificate margin
    int32_t* mvlist = nullptr;
    int32_t* mvhop = nullptr;
    int32_t* mvpar = nullptr;
    int64_t* mvro = nullptr;
    float* mvfin = nullptr;        // exact fused score of each visited node
    float* mvscore = nullptr;
    int32_t mcap_q = 0;
    int32_t* mknn = nullptr;       // neighbour lists of a shared scan's k-NN queries
    int32_t mknn_cap = 0;          // nodes
    // multi-query int8 pass (allocated on first use, for 8 kScan8MMaxA queries)
    uint64_t* m8part = nullptr;    // [q][kScan8MPart] workgroup lists
    unsigned char* m8qa = nullptr; // A operands: kScan8MMaxA x d / 64 x 1 KB
    float* m8qp = nullptr;         // [q][4] query split terms
    void* h_mres = nullptr;        // pinned, mapped: [q] ResultHeader then [q][rcap] results
    void* d_mres = nullptr;
    size_t mres_bytes = 0;
    // replayed query graphs (kernel nodes updated per query)
    struct GraphSlot {
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
        hipGraphNode_t node[2] = {nullptr, nullptr};
        const void* fn[2] = {nullptr, nullptr};
        unsigned grid0 = 0;
    };
    GraphSlot g_global, g_episode;
};

// ---- streaming insert kernels (defined in stream.hip) --------------------------------
struct PatchArgs {
    int32_t* col;
    int64_t* ro;
    int32_t* rcap;
    const int64_t* reloc;      // n_reloc x {src_start, len, dst_start}
    int32_t n_reloc;
    const int32_t* tail;       // values for col[tail_base ..); INT32_MIN: filled by a relocation
    int64_t tail_base;
    int64_t n_tail;
    const int64_t* app;        // n_app x {offset, value}: appends inside existing row slack
    int32_t n_app;
    const int64_t* rows;       // n_rows x {node, row word, capacity}
    int32_t n_rows;
    int32_t* hits;             // null: no edge-hit counters; else they follow the edges
    const int64_t* tail_src;   // null, or per tail slot: the col slot its edge came from (-1: new)
};
int graph_insert_free(Graph& g);     // insert scratch of a graph
int reset_edge_hits(Graph& g);       // zero counters sized to cap_e (maintain.hip), if enabled
// Edges between node first + i and each listed neighbour knn[i * k + j] (-1 skipped),
// both directions, merged into the rows (insert.hip). Caller holds the graph mutex.
int link_knn_apply(Graph& g, int32_t first, int32_t count, int32_t k, const int32_t* knn, hipStream_t s,
                   mars_insert_stats* st);

// ---- launch helpers (defined in kernels.hip) --------------------------------------
struct ScanArgs {
    const void* emb;     // fp32 or fp16 rows
    int32_t fp16;
    int64_t n;
    int32_t d;
    const float* q;
    const float* ts;
    const int32_t* mods;
    const int32_t* ep_ids;
    float t_q;
    float lambda;
    int32_t mod_filter;
    int32_t query_ep;
    float boost;         // > 0 and ep_ids != null: same-episode boost
    int32_t k;
    float* fin;
    uint64_t* part;          // candidate keys appended by the workgroups
    uint64_t* gthr;          // running bound on the K-th best key (atomicMin)
    uint32_t* gcnt;          // number of candidate keys appended (atomicAdd)
    int32_t rows_per_wg;     // unused (grid-stride scan)
    int32_t num_wg;
    int64_t id_base;         // node id of row 0 (tiles of a host-resident corpus)
    const float* meta8;      // int8 rows (launch_scan8): per-row scale and error bound; workgroup b
                             // writes its k (= kScan8List) best keys, ascending and
                             // kEmptyKey-padded, to part[k b .. k b + k - 1] (gthr, gcnt untouched),
                             // and the query's rounding term tau to part[kScan8MaxLists *
                             // kScan8List] (fp32 bits)
    const uint32_t* nrm8;    // launch_scan8: Graph::nrm8
};
// Kernel entry point + launch shape of one launch (for graph kernel nodes).
struct KernelLaunch {
    const void* fn = nullptr;
    dim3 grid;
    dim3 block;
};
int launch_scan(const ScanArgs& a, hipStream_t s);
KernelLaunch scan_launch(const ScanArgs& a);
KernelLaunch finalize_launch();
KernelLaunch episode_launch(int32_t d);
void scan_grid(int64_t n, int32_t max_wg, int32_t* rows_per_wg, int32_t* num_wg);
// int8 candidate scan of the certified global query (scan8.hip): keys rank rows by an
// upper bound of their fp32 scan score, fin gets the int8 estimate of every row.
// The int8 copy is tiled for the MFMA scan: rows are grouped in tiles of 16, and each 64-byte
// k-chunk i of a tile is a 1 KB block whose 16-byte piece 16 g + m holds bytes 64 i + 16 g ..
// 64 i + 16 g + 15 of the tile's row m (the B operand of v_mfma_i32_16x16x64_i8, one load
// instruction per block). d is a multiple of 64.
__host__ __device__ inline int64_t i8_offset(int64_t row, int32_t k, int32_t d) {
    return ((row >> 4) * (d >> 6) + (k >> 6)) * 1024 + ((((k & 63) >> 4) << 4) + (row & 15)) * 16 + (k & 15);
}
__host__ __device__ inline int64_t i8_rows_alloc(int64_t rows) { return (rows + 15) / 16 * 16; }
constexpr int32_t kScan8MaxLists = 512;    // int8 scan workgroups = lists k_cert_bfs merges
constexpr int32_t kScan8List = 16;         // keys per workgroup list
bool scan8_dim_supported(int32_t d);
int launch_scan8(const ScanArgs& a, hipStream_t s);
// The int8 scan for up to 8 kScan8MMaxA queries in one pass (scan8m.hip): query slot j
// holds rows 2 (j % 8), 2 (j % 8) + 1 of A operand j / 8.
constexpr int32_t kScan8MMaxA = 2;
constexpr int64_t kScan8MPart = int64_t(kScan8MaxLists) * kScan8List;   // keys per query
struct Split8Args {
    const float* q_glob;     // [n_glob][d] global queries
    const float* q_plain;    // [nq - n_glob][d] plain queries (a node's own fp32 row)
    int32_t nq;
    int32_t n_glob;
    int32_t d;
    int32_t na;              // A operands (slots 8 na)
    const uint32_t* nrm8;
    void* qa;                // out: [na][d / 64][64] x 16 bytes
    float* qp;               // out: [8 na][4] s_hi, s_lo, tau, |q|
};
struct Scan8MArgs {
    const void* emb8;
    const float* meta8;
    int64_t n;
    int32_t d;
    const float* ts;
    const int32_t* mods;
    const void* qa;
    const float* qp;
    const float* tq;         // [n_glob] query times, or null: every global query at tq_value
    float tq_value;
    float lambda;
    int32_t mod_filter;      // global queries
    int32_t nq;
    int32_t n_glob;          // queries [0, n_glob) global; the rest plain dots
    int64_t self_base;       // plain query j skips row self_base + j - n_glob
    uint64_t* part;          // [nq][kScan8MPart]: workgroup b's 16 best keys at [16 b ..]
    int32_t num_wg;
};
int launch_split8(const Split8Args& a, hipStream_t s);
int launch_scan8m(const Scan8MArgs& a, int na, hipStream_t s);
// Widths with an exact-rescoring kernel (k_cert_bfs / k_cert_multi8 over QF32<d / 64>): the
// certified paths run only at these; any other width is answered by the fp32 scan.
inline bool cert_dim_supported(int32_t d) { return d == 256 || d == 384 || d == 512 || d == 768 || d == 1024; }
// The certified paths scan the int8 copy when there is one (d <= 1024: the exact
// rescoring's QF32 layouts), else the fp16 copy.
inline bool cert_uses_int8(const Graph& g) {
    return g.emb8 && g.meta8 && g.nrm8 && scan8_dim_supported(g.d) && cert_dim_supported(g.d);
}
// Quantizes rows [r0, r1) of emb into emb8 / meta8 and raises nrm8.
int launch_convert_i8(const float* emb, int64_t r0, int64_t r1, int32_t d, int8_t* emb8, float* meta8,
                      uint32_t* nrm8, hipStream_t s);

struct FinalizeArgs {
    const uint64_t* part;    // candidate keys from the scan
    uint32_t* gcnt;          // their count; reset to 0 here for the next query
    uint64_t* gthr;          // scan's running bound; reset to kEmptyKey here
    int32_t k;
    const int64_t* ro;       // per node: (row length << 32) | row start in col
    const int32_t* col;
    int32_t n_live;          // nodes this query sees; neighbours >= n_live are skipped
    const float* fin;
    const int32_t* mods;
    int32_t hops;
    float hop_decay;
    uint32_t epoch;          // visit stamp of this query (vis[i] == epoch: visited)
    uint32_t gen_base;       // claim generation of BFS level 0 (level h uses gen_base + h)
    uint32_t* vis;
    uint64_t* claim;
    int32_t* vlist;
    int32_t* vhop;
    float* vscore;
    int64_t* vro;            // per visit position: the node's (len << 32) | start
    int32_t* vpar;           // per visit position: the parent's position (unscored / interval BFS)
    float* vdv;              // interval BFS: per visit position, a bound on the score's error
    double eps;              // interval BFS: bound on |a.fin - exact fused score| of any row
    int32_t mod_filter;      // interval BFS: filtered rows' scores are exact
    uint64_t* sortbuf;
    int32_t cap_visit;
    int32_t rcap;            // results requested (max_results or K)
    int32_t* seed_idx;
    float* seed_val;
    ResultHeader* res;
    mars_query_result* rec;
    uint64_t* stamps;        // 4 realtime stamps (start, seeds, BFS done, end) or null
    uint32_t* done;          // host-mapped completion word: seq after the results, or null
    uint32_t seq;
};
int launch_finalize(const FinalizeArgs& a, hipStream_t s);
// Tiled query: fold the candidate keys the scan of one tile appended (part[0..*gcnt))
// into the running K best (carry, ascending) and clear *gcnt; the scan's bound stays.
int launch_tile_merge(uint64_t* part, uint32_t* gcnt, uint64_t* carry, int32_t k, hipStream_t s);

struct EpisodeArgs {
    const float* emb;
    int32_t d;
    int64_t n;
    const float* q;
    const float* ts;
    const int32_t* mods;
    const int32_t* members;  // ep_csr_members + begin
    int32_t m;
    float t_q;
    float lambda;
    int32_t mod_filter;
    int32_t k;
    int32_t rcap;
    uint64_t* keybuf;        // >= m keys scratch
    int32_t* seed_idx;
    float* seed_val;
    ResultHeader* res;
    mars_query_result* rec;
    uint32_t* done;          // host-mapped completion word: seq after the results, or null
    uint32_t seq;
};
int launch_episode(const EpisodeArgs& a, hipStream_t s);

int launch_convert_f16(const float* in, __half* out, int64_t count, hipStream_t s);
// Streaming read of bytes (a multiple of 16) with wg workgroups; out holds wg words.
int launch_read_rows(const void* p, int64_t bytes, int32_t wg, uint32_t sentinel, uint32_t* out, hipStream_t s);
// 16 rows x 64 B per load instruction over the first n_rows / 16 * 16 rows (nt: non-temporal)
int launch_read_frags(const void* rows, int64_t n_rows, int32_t row_bytes, int32_t wg, bool nt, uint32_t sentinel,
                      uint32_t* out, hipStream_t s);

// ---- batched MFMA scoring (defined in batch.hip) ---------------------------------------
struct BatchArgs {
    const __half* emb16;     // corpus rows, fp16
    int64_t n;
    int32_t d;
    const __half* qh;        // queries, fp16, row-major q x d
    int32_t q;
    const float* tq;         // q query times
    const float* ts;
    const int32_t* mods;
    float lambda;
    int32_t mod_filter;
    int32_t k;               // <= 16 kept per query
    int32_t q_plain;         // queries q_plain .. q-1 are neighbour searches: plain dot product,
                             // no decay, no filter (the rest use lambda / mod_filter / tq)
    int64_t self_base;       // >= 0: neighbour search j (query q_plain + j) is node self_base + j
                             // and never its own neighbour
    uint64_t* part;          // [n_qblocks][n_rranges][64][K] keys
    int64_t rows_per_range;
    int64_t range_stride;    // row range r starts at row r * range_stride (0: rows_per_range)
    const uint64_t* floor_keys;  // optional: query j keeps no row below the score of key
    int32_t floor_k;             // floor_keys[j * floor_k + floor_k - 1] (a lower bound of its
                                 // final floor_k-th best score; an empty key is no floor)
    int32_t n_rranges;
    int32_t n_qblocks;
    int32_t uniform_tq;      // all query times equal: one decay weight per row
    int32_t sample_pass;     // the sampled pass of launch_batch_topk: its keys serve only as
                             // floors (k_batch_mm then keeps group maxima, not the best K)
};
bool batch_dim_supported(int32_t d);
// Three kernels score a batch, by its size and kind (1M rows, d = 768, one MI355X):
//   Q <= kRqMaxScanQ              k_batch_scan: 64-query blocks, rows streamed into
//                                 registers (Q = 64: 313 us);
//   Q > kRqMaxScanQ               k_batch_rq (batch_rq.hip): the queries held in registers
//                                 (128 or 256 per workgroup, batch_rq_tiles x 16 per wave),
//                                 16-row tiles streamed through LDS, a sampled score floor
//                                 (Q = 256: 549 us; Q = 1024: 1.80 ms);
//   neighbour searches, Q >= kGemmMinQ
//                                 k_batch_mm: 256-query x 256-row LDS tiles, thresholds from
//                                 the sampled floor (the k-NN builders' 1024-query chunks:
//                                 1.90 ms, against 2.86 ms through k_batch_rq). With decayed
//                                 scores its raw-dot thresholds pass far more rows than reach
//                                 the lists, and k_batch_rq is faster (Q = 1024: 1.80 against
//                                 2.50 ms).
// (With 64 queries per workgroup k_batch_rq measured slower than the scan: 445 against
// 408 us on a random 1M corpus.)
constexpr int32_t kGemmMinQ = 1024;
constexpr int32_t kRqMaxScanQ = 64;
bool batch_uses_gemm(int32_t q, bool plain);
bool batch_uses_rq(int32_t q, bool plain);
int batch_rq_tiles(int32_t q);   // 16-query MFMA tiles per k_batch_rq wave: 2 or 4
int launch_batch_rq(const BatchArgs& a, hipStream_t s);
int batch_kpart(int32_t k);  // keys per (query, row range) the scan writes
int launch_batch_scan(const BatchArgs& a, hipStream_t s);
// Batches of at least kGemmMinQ queries: k_batch_mm (batch_mm.hip).
int launch_batch_mm(const BatchArgs& a, hipStream_t s);
int launch_batch_merge(const uint64_t* part, int32_t n_rranges, int32_t kpart, int32_t q, int32_t k_out,
                       uint64_t* out, hipStream_t s);
// Scoring plus the merge: out[j * k_out ..] = query j's k_out best keys over all rows. On
// large corpora (ranges of at least kSampleDiv kSampleRowsMin rows) a first pass over the
// first 1 / kSampleDiv of every range (kSampleRowsMin .. kSampleRowsMax rows), merged into out, gives
// each query a floor (its k_out-th best sampled score, a lower bound of the final one), so
// the full pass keeps only rows at or above it.
// At 1M rows, Q = 256: 1/64 of each range (48 rows) gives a sampled pass of 45 us and a
// full pass of 482 us, 1/32 (112 rows) 77 and 458 us, 1/16 5% slower than 1/32; below
// kSampleRowsMin the floor is too weak to pay for its pass.
constexpr int64_t kSampleDiv = 64;
constexpr int64_t kSampleRowsMin = 32;
constexpr int64_t kSampleRowsMax = 1024;
// `scanned` (optional) is recorded after the full pass, before the final merge.
int launch_batch_topk(BatchArgs a, int32_t k_out, uint64_t* out, hipStream_t s, hipEvent_t scanned = nullptr);
// nrm and cert given: cert[node] = 1 when the node's lists are certified exact (k_knn_rerank)
int launch_knn_rerank(const float* emb, int64_t q0, int64_t nq, int32_t d, const uint64_t* cand, int32_t kc,
                      int32_t k_out, int32_t* nbrs, hipStream_t s, const uint32_t* nrm = nullptr,
                      int32_t* cert = nullptr);
int launch_f32_to_f16_rows(const float* in, __half* out, int64_t count, hipStream_t s);

// ---- batched global queries (multi.hip; BFS / select kernels in kernels.hip) -----------
// Query terms of the fused score, as ScanArgs carries them for one query.
struct QueryTerms {
    float t_q;
    float lambda;
    int32_t mod_filter;
    int32_t query_ep;
    float boost;
};
struct SeedArgs {
    const void* emb;         // rows the Q=1 path scores: fp32, or fp16 when fp16 != 0
    int32_t fp16;
    int32_t d;
    const float* ts;
    const int32_t* mods;
    const float* queries;    // q x d fp32
    const float* tq;         // q query times
    float lambda;
    int32_t mod_filter;
    int32_t q;
    int32_t k;               // seeds per query (<= kMultiCand)
    const uint64_t* cand;    // [q][kMultiCand] fp16 candidate keys, ascending
    const double* qn;        // [q][4] query norms
    const uint32_t* nrm;     // graph row-norm bounds (Graph::nrm)
    uint64_t* seeds;         // [q][kMultiCand] out: exact keys, ascending
    int32_t* status;         // [q] out
    float* margin;           // [q] out: K-th exact score - (C-th fp16 score + bound)
};
struct MultiArgs {
    const int64_t* ro;
    const int32_t* col;
    const int32_t* mods;
    int32_t n_live;
    int32_t hops;
    float hop_decay;
    int32_t k;
    int32_t rcap;
    int32_t q;
    const uint64_t* seeds;   // [q][seed_stride]
    int32_t seed_stride;     // kMultiCand (batched), 64 (certified Q=1)
    int32_t* status;         // [q]
    int32_t* info;           // [q][4] visited, levels, seeds
    int32_t* vlist;          // [q][kMultiVisit] each
    int32_t* vhop;
    int32_t* vpar;
    int64_t* vro;
    float* vfin;
    float* vscore;
    ResultHeader* res;       // [q] (host-mapped)
    mars_query_result* rec;  // [q][rcap] (host-mapped)
    uint32_t* done;          // q = 1: host-mapped completion word (k_multi_select), or null
    uint32_t seq;
};
struct VisitScoreArgs {
    const void* emb;
    int32_t fp16;
    int32_t d;
    const float* ts;
    const int32_t* mods;
    const float* queries;
    const float* tq;         // q query times (device), or null: every query at t_q_value
    float t_q_value;
    float lambda;
    int32_t mod_filter;
    int32_t q;
    const int32_t* status;
    const int32_t* info;
    const int32_t* vlist;
    float* vfin;
};
int launch_row_norms(const float* emb, const __half* emb16, int64_t r0, int64_t r1, int32_t d, uint32_t* nrm,
                     hipStream_t s);
int launch_query_norms(const float* q32, const __half* q16, int32_t q, int32_t d, double* out, hipStream_t s);
int launch_multi_seed(const SeedArgs& a, hipStream_t s);
// Certified Q=1 global query: the fp16 scan (ScanArgs with k = c) appended its
// candidate keys to part; one workgroup merges the c best, rescores them with the
// fp32 scan's arithmetic, certifies the k best (status kMultiOk), resets the scan's
// count and bound, and runs the certified seeds' BFS (k_multi_bfs's work for query 0).
// k_visit_scores / k_multi_select (q = 1) finish the query.
struct CertArgs {
    const uint64_t* part;
    uint32_t* gcnt;
    uint64_t* gthr;
    int32_t c;               // candidates the scan kept (<= 64)
    int32_t n_lists;         // > 0 (<= kScan8MaxLists): part holds n_lists ascending lists of
                             // kScan8List keys (launch_scan8), else the keys the workgroups
                             // appended (gcnt of them)
    int32_t k;               // seeds
    const float* q;          // d floats
    int32_t d;
    const float* emb;        // fp32 rows
    const float* ts;
    const int32_t* mods;
    float t_q;
    float lambda;
    int32_t mod_filter;
    const uint32_t* nrm;     // Graph::nrm
    int32_t upper;           // 1: int8 scan, candidate keys are upper bounds (nrm8 holds the bounds)
    const uint32_t* nrm8;    // Graph::nrm8
    const float* fin16;      // the candidate scan's fused score of every row
    int32_t finish;          // 1: also compute the results (hop decay in [0, 1], rcap <= 64)
    uint64_t* seeds;         // 64 entries: ascending exact keys, the first k are the seeds
    int32_t* status;
    float* margin;
    uint64_t* stamps;        // 7 realtime stamps of the phases, or null
    uint32_t* done;          // finish = 1: host-mapped completion word, or null
    uint32_t seq;
};
int launch_cert_bfs(const CertArgs& a, const struct MultiArgs& m, hipStream_t s);   // + BFS of query 0 of m
// Certified seeds / neighbours of the queries of one k_scan8m pass (one workgroup each).
struct CertMArgs {
    const uint64_t* part;    // [q][kScan8MPart] (launch_scan8m)
    int32_t n_lists;         // scan workgroups
    int32_t q;
    int32_t n_glob;          // queries [0, n_glob) global, the rest plain
    const float* q_glob;
    const float* q_plain;
    int32_t d;
    const float* emb;        // fp32 rows
    const float* ts;
    const int32_t* mods;
    const float* tq;         // or null: every global query at tq_value
    float tq_value;
    float lambda;
    int32_t mod_filter;
    const float* qp;         // launch_split8's per-query terms (tau, |q|)
    const uint32_t* nrm8;
    int32_t k;               // seeds per global query (<= 64)
    int32_t knn_k;           // neighbours per plain query (<= 64)
    uint64_t* seeds;         // [n_glob][64]
    int32_t* status;         // [q]
    float* margin;           // [q]
    int32_t* knn_out;        // [q - n_glob][knn_k] (device)
};
int launch_cert_multi8(const CertMArgs& a, hipStream_t s);
int launch_multi_bfs(const MultiArgs& a, hipStream_t s);
int launch_visit_scores(const VisitScoreArgs& a, hipStream_t s);
int launch_multi_select(const MultiArgs& a, hipStream_t s);

}  // namespace mars

struct mars_graph {
    mars::Graph g;
    mutable std::mutex mu;   // serialises inserts, CSR / episode / fp16 replacement and downloads
    // the graph's own query context (novelty without a caller context): a cache created
    // on first use, so calls on a const graph may create it
    mutable mars_ctx* own_ctx = nullptr;
    mutable std::mutex own_mu;
};
struct mars_ctx { mars::Ctx c; };
