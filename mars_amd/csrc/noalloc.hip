// ============================================================================
//  noalloc.hip — mars_query_batch_static: batched global scoring that allocates
//  nothing, for callers that cannot call hipMalloc (code under HIP graph capture,
//  tight serving loops).
//
//  The same kernels as mars_query_batch (fp32 -> fp16 query rows, k_batch_scan,
//  k_batch_merge), with their scratch in one file-scope device array instead of
//  context buffers: the queries' fp16 rows, the per-row-range partial keys and
//  the merged keys. The device address of that array is taken once per device
//  with hipGetSymbolAddress, at set-up (mars_init, and mars_graph_create on the
//  graph's device), and kept; kernels receive that address, never the array's
//  host-side name. A call makes no HIP API call but its kernel launches on the
//  caller's stream, and nothing waits for them, so the call can be captured into
//  a HIP graph. Every call on one GPU shares the array: calls that overlap on one
//  GPU race. No slot needs clearing: the scan writes every partial key the merge
//  reads, and the merge every key it emits.
// ============================================================================
#include "internal.hpp"

#include <algorithm>
#include <atomic>
#include <cfloat>
#include <mutex>

namespace mars {
namespace {

constexpr int32_t kStaticMaxQ = 256;                      // queries per call
constexpr int32_t kStaticMaxD = 768;                      // widest batched row (batch_dim_supported)
constexpr size_t kStaticQBytes = size_t(kStaticMaxQ) * kStaticMaxD * sizeof(__half);     // 384 KiB
constexpr size_t kStaticPartKeys = size_t(1) << 20;      // 8 MiB of partial keys
constexpr size_t kStaticOutKeys = size_t(kStaticMaxQ) * 16;
constexpr size_t kStaticPartOff = (kStaticQBytes + 255) / 256 * 256;
constexpr size_t kStaticOutOff = kStaticPartOff + kStaticPartKeys * sizeof(uint64_t);
constexpr size_t kStaticBytes = kStaticOutOff + kStaticOutKeys * sizeof(uint64_t);    // ~8.4 MiB
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kStaticBytes];

std::mutex g_scratch_mu;
std::atomic<void*> g_scratch_ptr[kMaxDevices] = {};

// The array's device address on `dev`, set by noalloc_prepare.
int static_scratch(int dev, unsigned char** out) {
    MARS_CHECK(dev >= 0 && dev < kMaxDevices, MARS_ERR_UNSUPPORTED, "device %d beyond %d", dev, kMaxDevices);
    void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    MARS_CHECK(p != nullptr, MARS_ERR_INVALID, "static scratch of device %d not set up (mars_init)", dev);
    *out = static_cast<unsigned char*>(p);
    return MARS_OK;
}

}  // namespace

// The array's device address on `dev` (the current device), taken once.
int noalloc_prepare(int dev) {
    MARS_CHECK(dev >= 0 && dev < kMaxDevices, MARS_ERR_UNSUPPORTED, "device %d beyond %d", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev].load(std::memory_order_relaxed)) return MARS_OK;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
        return set_error(MARS_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev].store(p, std::memory_order_release);
    return MARS_OK;
}

namespace {

// keys -> (id, score) pairs, as mars_query_batch converts them on the host
__global__ __launch_bounds__(256) void k_keys_to_results(const uint64_t* __restrict__ keys, int32_t n,
                                                         int32_t* __restrict__ ids, float* __restrict__ scores) {
    const int32_t i = int32_t(blockIdx.x * blockDim.x + threadIdx.x);
    if (i >= n) return;
    const uint64_t k = keys[i];
    ids[i] = k == kEmptyKey ? -1 : key_id(k);
    scores[i] = k == kEmptyKey ? -FLT_MAX : key_score(k);
}

}  // namespace
}  // namespace mars

using namespace mars;

extern "C" int mars_query_batch_static(const mars_graph* gh, const float* d_queries, int32_t Q, const float* d_tq,
                                       int32_t uniform_tq, const mars_retrieval_config* cfg, int32_t* d_ids,
                                       float* d_scores, void* stream) {
    MARS_CHECK(gh && d_queries && d_tq && cfg && d_ids && d_scores, MARS_ERR_INVALID, "null argument");
    MARS_CHECK(Q >= 1 && Q <= kStaticMaxQ, MARS_ERR_CAPACITY,
               "mars_query_batch_static: %d queries (1 to %d fit its static scratch)", Q, kStaticMaxQ);
    const Graph& g = gh->g;
    MARS_CHECK(g.emb16 != nullptr, MARS_ERR_UNSUPPORTED, "batched scoring reads the fp16 corpus: enable it first");
    MARS_CHECK(batch_dim_supported(g.d) && g.d <= kStaticMaxD, MARS_ERR_UNSUPPORTED,
               "batched scoring: embedding_dim %d unsupported", g.d);
    MARS_CHECK(cfg->top_k >= 1 && cfg->top_k <= 16, MARS_ERR_UNSUPPORTED, "batched top_k %d not in [1, 16]",
               cfg->top_k);
    MARS_TRY(use_device(g.device));
    unsigned char* base = nullptr;
    MARS_TRY(static_scratch(g.device, &base));
    const int32_t K = cfg->top_k;
    const int32_t n_live = __atomic_load_n(&g.n, __ATOMIC_ACQUIRE);
    MARS_CHECK(n_live > 0, MARS_ERR_INVALID, "empty graph");
    int32_t nrr = 0, nqb = 0;
    int64_t rpr = 0;
    batch_grid(n_live, Q, false, &nrr, &nqb, &rpr);
    const int32_t kp = batch_kpart(K);
    const int64_t part_keys = int64_t(nqb) * nrr * 64 * kp;
    MARS_CHECK(part_keys <= int64_t(kStaticPartKeys), MARS_ERR_CAPACITY,
               "mars_query_batch_static: %lld partial keys exceed the static %zu", (long long)part_keys,
               kStaticPartKeys);
    __half* bq = reinterpret_cast<__half*>(base);
    uint64_t* part = reinterpret_cast<uint64_t*>(base + kStaticPartOff);
    uint64_t* out = reinterpret_cast<uint64_t*>(base + kStaticOutOff);
    hipStream_t s = static_cast<hipStream_t>(stream);
    MARS_TRY(launch_f32_to_f16_rows(d_queries, bq, int64_t(Q) * g.d, s));
    BatchArgs a{};
    a.emb16 = g.emb16; a.n = n_live; a.d = g.d; a.qh = bq; a.q = Q; a.tq = d_tq; a.ts = g.ts; a.mods = g.mods;
    a.lambda = cfg->time_decay_lambda; a.mod_filter = cfg->modality_filter; a.k = K; a.q_plain = Q; a.self_base = -1;
    a.part = part; a.rows_per_range = rpr; a.n_rranges = nrr; a.n_qblocks = nqb;
    a.uniform_tq = uniform_tq ? 1 : 0;
    MARS_TRY(launch_batch_topk(a, K, out, s));
    const int32_t n = Q * K;
    MARS_LAUNCH(k_keys_to_results, dim3(unsigned((n + 255) / 256)), dim3(256), 0, s, out, n, d_ids, d_scores);
    return MARS_OK;
}
