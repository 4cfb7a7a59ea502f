// ============================================================================
//  oracle/oracle.cpp — CPU restatement of the MARS retrieval hot path.
//
//  TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and the
//  cpu_baseline leg of bench.py may load this library: to compare GPU results
//  against it, or to time it as the CPU baseline. The product (mars_amd) never
//  calls it.
//
//  Every function cites the reference file:line it restates (paths relative
//  to the MARS source tree). Arithmetic is fp64 throughout (inputs are the
//  same fp32 / fp16 bytes the GPU consumes); the GPU computes in fp32 and is
//  compared against these values with a tolerance.
//
//  Deterministic definitions where the reference is racy or unstable
//  (documented parity decisions):
//    * top-K seeds:   (score desc, node id asc)  == CUB stable ascending sort
//                     of negated keys (memory_cuda.cu:1254-1283)
//    * BFS:           sequential BFS of scripts/bench_cpu.py:115-139 — seeds in
//                     tie-rule order, frontier in discovery order, neighbours in
//                     CSR order, first discoverer is the parent; no frontier cap
//                     (the reference GPU caps at min(N, 20K) and races on the
//                     parent, memory_cuda.cu:661-697, :1322-1323)
//    * final order:   (score desc, node id asc) (reference std::sort is unstable,
//                     memory_cuda.cu:1439); no compaction cap (the reference
//                     drops visited nodes beyond min(N, K*500) in arbitrary order)
//
//  Parity pinning (checked in tests/test_oracle.py): episode CSR against the
//  reference's own build_episode_csr (oracle/_ref) and golden fixtures; scores
//  against an independent numpy fp64 product and the closed forms of the decay;
//  top-K against numpy lexsort; BFS levels against scipy's unweighted shortest
//  paths; BFS parents / scores against hand-derived small graphs.
// ============================================================================
#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <numeric>
#include <set>
#include <random>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

extern "C" {

// Same field layout as mars_retrieval_config / RetrievalConfig (memory_cuda.cuh:107-127).
struct oracle_config {
    int32_t top_k;
    int32_t bfs_max_hops;
    float   time_decay_lambda;
    float   bfs_score_decay;
    int32_t modality_filter;
    int32_t use_importance;
    int32_t max_results_returned;
    int32_t retrieval_scope;
    int32_t query_episode_id;
    int32_t query_episode_member_begin;
    int32_t query_episode_member_count;
    float   episode_same_boost;
};

struct oracle_graph {
    int64_t         num_nodes;
    int32_t         dim;
    int32_t         pad0;
    const int32_t*  row_offsets;   // N+1 (may be null when no edges)
    const int32_t*  col_indices;
    const float*    emb;           // N*D fp32 (used when emb16 is null)
    const uint16_t* emb16;         // N*D IEEE binary16 bits, or null
    const int32_t*  modalities;
    const float*    timestamps;
    const int32_t*  episode_ids;   // N or null
    const int32_t*  ep_offsets;    // num_episodes+1 or null
    const int32_t*  ep_members;
    int32_t         num_episodes;
    int32_t         member_total;
};

struct oracle_result {
    int32_t node_id;
    double  score;
    int32_t modality;
    int32_t hops;
};

int oracle_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void oracle_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

// IEEE binary16 -> double, exact (every half is representable).
static inline double half_bits_to_double(uint16_t h) {
    const int s = (h >> 15) & 1, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    double v;
    if (e == 0)       v = std::ldexp(double(m), -24);                 // subnormal / zero
    else if (e == 31) v = m ? NAN : INFINITY;
    else              v = std::ldexp(double(m | 0x400), e - 25);
    return s ? -v : v;
}

double oracle_half_to_double(uint16_t h) { return half_bits_to_double(h); }

// fp32 -> binary16, round to nearest even (the rounding of __float2half /
// v_cvt_f16_f32 used by convert_f32_to_f16_kernel, memory_cuda.cu:207-211).
uint16_t oracle_float_to_half_rne(float f) {
    uint32_t x; std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t absx = x & 0x7fffffffu;
    if (absx >= 0x7f800000u)                      // inf / nan
        return uint16_t(sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u : 0u));
    if (absx >= 0x477ff000u)                      // >= 65520 rounds to inf
        return uint16_t(sign | 0x7c00u);
    if (absx < 0x33000001u)                       // <= 2^-25 rounds to zero
        return uint16_t(sign);
    int e = int(absx >> 23) - 127;
    uint32_t mant = (absx & 0x7fffffu) | 0x800000u;   // 24-bit significand
    int shift;                                       // bits to drop
    uint32_t base;
    if (e < -14) { shift = 13 + (-14 - e); base = 0; }          // subnormal half
    else         { shift = 13; base = uint32_t(e + 15) << 10; }
    uint32_t q = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    uint32_t r;
    if (e < -14) r = q;                                  // may carry into the exponent: fine
    else         r = base + (q & 0x3ffu) + ((q >> 10) - 1u) * 0x400u;
    return uint16_t(sign | r);
}

void oracle_convert_f16(const float* in, uint16_t* out, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_float_to_half_rne(in[i]);
}

// ---------------------------------------------------------------------------
// build_episode_csr — memory_graph.cpp:12-44 (counting sort; members ascending
// node id inside each episode; num_episodes = max id + 1).
// Call with offsets == nullptr to get num_episodes only. Returns 0, or -1 for a
// negative episode id (undefined behaviour in the reference).
// ---------------------------------------------------------------------------
int oracle_build_episode_csr(const int32_t* ids, int32_t n, int32_t* num_episodes,
                             int32_t* offsets, int32_t* members) {
    *num_episodes = 0;
    if (n <= 0 || ids == nullptr) return 0;                   // :15-16 empty CSR
    int32_t max_ep = 0;
    for (int32_t i = 0; i < n; ++i) {
        if (ids[i] < 0) return -1;
        max_ep = std::max(max_ep, ids[i]);
    }
    *num_episodes = max_ep + 1;                                // :21
    if (offsets == nullptr) return 0;
    std::vector<int32_t> cnt(size_t(max_ep) + 1, 0);
    for (int32_t i = 0; i < n; ++i) ++cnt[size_t(ids[i])];
    offsets[0] = 0;
    for (int32_t e = 0; e <= max_ep; ++e) offsets[e + 1] = offsets[e] + cnt[size_t(e)];
    std::vector<int32_t> cursor(offsets, offsets + max_ep + 1);
    for (int32_t i = 0; i < n; ++i) members[cursor[size_t(ids[i])]++] = i;
    return 0;
}

// ---------------------------------------------------------------------------
// Stage 1+2 — fused score: memory_cuda.cu:105-152 (fp32), :155-201 (fp16),
// :400-418 (temporal_rerank after cuBLAS SGEMV):
//   final[i] = <E_i, q> * exp(-lambda * max(0, t_q - ts_i))   (age in fp32, as
//   the reference computes fmaxf(0.0f, query_ts - timestamps[i]) in fp32)
//   modality_filter >= 0 and modality != filter  ->  -FLT_MAX
// scale[i] = w_i * sum_d |e_d q_d| bounds the fp32 rounding error of the dot.
// ---------------------------------------------------------------------------
static inline double decay_weight(float t_q, float ts, float lambda) {
    const float age = std::fmax(0.0f, t_q - ts);
    return std::exp(-double(lambda) * double(age));
}

static inline void score_row(const oracle_graph* g, int64_t i, const float* q, float t_q,
                             float lambda, int32_t mod_filter, double* fin, double* scl) {
    if (mod_filter >= 0 && g->modalities[i] != mod_filter) {
        *fin = -double(FLT_MAX);
        if (scl) *scl = 0.0;
        return;
    }
    const int32_t D = g->dim;
    double dot = 0.0, absdot = 0.0;
    if (g->emb16) {
        const uint16_t* r = g->emb16 + i * D;
        for (int32_t d = 0; d < D; ++d) {
            const double p = half_bits_to_double(r[d]) * double(q[d]);
            dot += p; absdot += std::fabs(p);
        }
    } else {
        const float* r = g->emb + i * D;
        for (int32_t d = 0; d < D; ++d) {
            const double p = double(r[d]) * double(q[d]);
            dot += p; absdot += std::fabs(p);
        }
    }
    const double w = decay_weight(t_q, g->timestamps[i], lambda);
    *fin = dot * w;
    if (scl) *scl = absdot * w;
}

void oracle_scores(const oracle_graph* g, const float* q, float t_q, float lambda,
                   int32_t mod_filter, double* final_out, double* scale_out) {
    const int64_t N = g->num_nodes;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < N; ++i)
        score_row(g, i, q, t_q, lambda, mod_filter, &final_out[i],
                  scale_out ? &scale_out[i] : nullptr);
}

// ---------------------------------------------------------------------------
// Stage 3 — exact top-K by (score desc, id asc): the order of a stable ascending
// radix sort of negated scores (memory_cuda.cu:737-771, 1254-1283). Signed
// zeros compare equal. Returns min(K, N).
// ---------------------------------------------------------------------------
static inline bool key_less(double va, int64_t ia, double vb, int64_t ib) {
    if (va != vb) return va > vb;
    return ia < ib;
}

int32_t oracle_topk(const double* fin, int64_t N, int32_t K, int32_t* idx, double* val) {
    if (K <= 0 || N <= 0) return 0;
    const int32_t k = int32_t(std::min<int64_t>(K, N));
    // per-thread partial top-k, then merge (deterministic: the comparator is total)
    int nt = oracle_num_threads();
    std::vector<std::vector<int64_t>> part(static_cast<size_t>(nt));
#pragma omp parallel num_threads(nt)
    {
        int t = 0;
#ifdef _OPENMP
        t = omp_get_thread_num();
#endif
        auto cmp = [&](int64_t a, int64_t b) { return key_less(fin[a], a, fin[b], b); };
        std::vector<int64_t>& h = part[size_t(t)];       // max-heap on "worst" under cmp
        const int64_t lo = N * t / nt, hi = N * (t + 1) / nt;
        for (int64_t i = lo; i < hi; ++i) {
            if (int32_t(h.size()) < k) { h.push_back(i); std::push_heap(h.begin(), h.end(), cmp); }
            else if (cmp(i, h.front())) {
                std::pop_heap(h.begin(), h.end(), cmp); h.back() = i;
                std::push_heap(h.begin(), h.end(), cmp);
            }
        }
    }
    std::vector<int64_t> all;
    for (auto& p : part) all.insert(all.end(), p.begin(), p.end());
    std::sort(all.begin(), all.end(),
              [&](int64_t a, int64_t b) { return key_less(fin[a], a, fin[b], b); });
    for (int32_t j = 0; j < k; ++j) { idx[j] = int32_t(all[size_t(j)]); val[j] = fin[all[size_t(j)]]; }
    return k;
}

// ---------------------------------------------------------------------------
// Stage 4 — BFS expansion: scripts/bench_cpu.py:115-139 (sequential order) with
// the kernel's score rule bfs[nb] = max(bfs[parent] * decay, final[nb] * 0.8)
// (memory_cuda.cu:633-697: seeds hop 0 with their top-K value; idx < 0 skipped).
// Outputs, indexed by visit position: ids, hops, scores, parent positions.
// hop_by_node (N entries, -1 = unvisited) is optional. Returns visited count,
// or -1 if cap is too small.
// ---------------------------------------------------------------------------
int32_t oracle_bfs(const int32_t* row_offsets, const int32_t* col, int64_t N,
                   const double* fin, const int32_t* seeds, const double* seed_vals,
                   int32_t n_seeds, int32_t hops, double decay,
                   int32_t* vis_ids, int32_t* vis_hops, double* vis_scores,
                   int32_t* vis_parent, int32_t cap, int32_t* hop_by_node,
                   int32_t* levels_run) {
    std::vector<int32_t> hop(static_cast<size_t>(N), -1);
    std::vector<double>  sc;
    std::vector<int32_t> ids, hp, par;
    for (int32_t s = 0; s < n_seeds; ++s) {
        const int32_t v = seeds[s];
        if (v < 0 || v >= N) continue;                 // bfs_init_seeds_kernel :645
        if (hop[size_t(v)] >= 0) continue;             // a repeated seed is visited once
        hop[size_t(v)] = 0;
        ids.push_back(v); hp.push_back(0); sc.push_back(seed_vals[s]); par.push_back(-1);
    }
    size_t fs = 0, fe = ids.size();
    int32_t run = 0;
    for (int32_t h = 0; h < hops && fs < fe; ++h) {
        for (size_t p = fs; p < fe; ++p) {
            const int32_t node = ids[p];
            const double ps = sc[p];
            if (!row_offsets) continue;
            for (int32_t e = row_offsets[node]; e < row_offsets[node + 1]; ++e) {
                const int32_t nb = col[e];
                if (hop[size_t(nb)] != -1) continue;
                hop[size_t(nb)] = h + 1;
                ids.push_back(nb); hp.push_back(h + 1);
                sc.push_back(std::max(ps * decay, fin[nb] * 0.8));
                par.push_back(int32_t(p));
            }
        }
        ++run;
        fs = fe; fe = ids.size();
    }
    if (levels_run) *levels_run = run;
    const int32_t n = int32_t(ids.size());
    if (n > cap) return -1;
    for (int32_t j = 0; j < n; ++j) {
        vis_ids[j] = ids[size_t(j)]; vis_hops[j] = hp[size_t(j)]; vis_scores[j] = sc[size_t(j)];
        if (vis_parent) vis_parent[j] = par[size_t(j)];
    }
    if (hop_by_node) std::memcpy(hop_by_node, hop.data(), size_t(N) * sizeof(int32_t));
    return n;
}

// episode_scoped_active — memory_cuda.cu:1163-1171
static bool episode_scoped_active(const oracle_graph* g, const oracle_config* c) {
    return c->retrieval_scope == 1 && g->ep_offsets != nullptr && g->ep_members != nullptr &&
           c->query_episode_id >= 0 && c->query_episode_id < g->num_episodes &&
           c->query_episode_member_count > 0 && c->query_episode_member_begin >= 0 &&
           int64_t(c->query_episode_member_begin) + c->query_episode_member_count <=
               g->member_total;
}

// ---------------------------------------------------------------------------
// Whole query — query_memory_fast (memory_cuda.cu:1351-1464) over
// launch_pipeline_kernels (:1177-1349) and the host tail (:1421-1447):
//   K = min(top_k, min(max_k, 64)); scope decision; stage-1 scores (episode:
//   -FLT_MAX except the member range); optional same-episode boost (global
//   only, :1243-1249, :427-440); top-K seeds; BFS (0 hops when scoped); visited
//   set sorted by (score desc, id asc) and truncated to max_results_returned > 0
//   ? that : K.
// final_out (N doubles, optional) receives the stage-1/2 scores; seeds_out /
// seed_vals_out (K entries, optional) the seeds; info[0..3] = {K, scoped,
// visited, levels_run}.
// If seeds_in is non-null the BFS starts from those n_seeds_in seeds (in that
// order) with the oracle's own scores — used to compare BFS given identical seeds.
// Returns the number of results written (<= cap) or -1.
// ---------------------------------------------------------------------------
int32_t oracle_query(const oracle_graph* g, const float* q, float t_q, const oracle_config* c,
                     int32_t ctx_max_k, oracle_result* out, int32_t cap, double* final_out,
                     int32_t* seeds_out, double* seed_vals_out,
                     const int32_t* seeds_in, int32_t n_seeds_in, int32_t* info) {
    const int64_t N = g->num_nodes;
    const int32_t max_k = std::min(ctx_max_k, 64);
    const int32_t K = std::min(c->top_k, max_k);
    if (K <= 0 || N <= 0) return -1;
    const bool scoped = episode_scoped_active(g, c);
    const int32_t hops = scoped ? 0 : std::max(0, c->bfs_max_hops);

    std::vector<double> fin_local;
    double* fin = final_out;
    if (!fin) { fin_local.resize(size_t(N)); fin = fin_local.data(); }

    if (scoped) {
        std::fill(fin, fin + N, -double(FLT_MAX));                         // :1194-1197
        const int32_t b = c->query_episode_member_begin, M = c->query_episode_member_count;
        for (int32_t j = 0; j < M; ++j) {                                  // :443-493
            const int32_t node = g->ep_members[b + j];
            score_row(g, node, q, t_q, c->time_decay_lambda, c->modality_filter, &fin[node], nullptr);
        }
    } else {
        oracle_scores(g, q, t_q, c->time_decay_lambda, c->modality_filter, fin, nullptr);
        if (g->episode_ids && c->query_episode_id >= 0 && c->episode_same_boost > 0.0f) {
            const double mul = 1.0 + double(c->episode_same_boost);
#pragma omp parallel for schedule(static)
            for (int64_t i = 0; i < N; ++i)
                if (fin[i] > -double(FLT_MAX) * 0.5 && g->episode_ids[i] == c->query_episode_id)
                    fin[i] *= mul;
        }
    }

    std::vector<int32_t> sidx(static_cast<size_t>(K));
    std::vector<double>  sval(static_cast<size_t>(K));
    int32_t ns;
    if (seeds_in) {
        ns = n_seeds_in;
        sidx.assign(seeds_in, seeds_in + ns);
        sval.resize(size_t(ns));
        for (int32_t j = 0; j < ns; ++j) sval[size_t(j)] = (sidx[size_t(j)] >= 0) ? fin[sidx[size_t(j)]] : 0.0;
    } else {
        ns = oracle_topk(fin, N, K, sidx.data(), sval.data());
    }
    if (seeds_out) for (int32_t j = 0; j < ns; ++j) seeds_out[j] = sidx[size_t(j)];
    if (seed_vals_out) for (int32_t j = 0; j < ns; ++j) seed_vals_out[j] = sval[size_t(j)];

    std::vector<int32_t> vid(static_cast<size_t>(N)), vh(static_cast<size_t>(N)), vp(static_cast<size_t>(N));
    std::vector<double> vs(static_cast<size_t>(N));
    int32_t lv = 0;
    const int32_t nv = oracle_bfs(g->row_offsets, g->col_indices, N, fin, sidx.data(), sval.data(),
                                  ns, hops, double(c->bfs_score_decay), vid.data(), vh.data(),
                                  vs.data(), vp.data(), int32_t(N), nullptr, &lv);
    if (nv < 0) return -1;

    std::vector<int32_t> order(static_cast<size_t>(nv));
    std::iota(order.begin(), order.end(), 0);
    std::sort(order.begin(), order.end(), [&](int32_t a, int32_t b) {
        return key_less(vs[size_t(a)], vid[size_t(a)], vs[size_t(b)], vid[size_t(b)]);
    });
    const int32_t rcap = (c->max_results_returned > 0) ? std::min(c->max_results_returned, nv)
                                                       : std::min(K, nv);     // :1441-1447
    const int32_t nw = std::min(rcap, cap);
    for (int32_t j = 0; j < nw; ++j) {
        const int32_t p = order[size_t(j)];
        out[j].node_id = vid[size_t(p)];
        out[j].score = vs[size_t(p)];
        out[j].modality = g->modalities[vid[size_t(p)]];
        out[j].hops = vh[size_t(p)];
    }
    if (info) { info[0] = K; info[1] = scoped ? 1 : 0; info[2] = nv; info[3] = lv; }
    return rcap;
}

// ---------------------------------------------------------------------------
// Tiled out-of-core contract — tiled_query.cu:174-314: per tile of tile_size rows,
// decayed scores (modality filter -> -FLT_MAX, :44-51), per-tile top-K, keep
// candidates with score > -FLT_MAX/2 (:280-285), merge by score desc (ties:
// id asc here), truncate to K. No BFS, no episode scope.
// ---------------------------------------------------------------------------
int32_t oracle_tiled_query(const oracle_graph* g, const float* q, float t_q, float lambda,
                           int32_t mod_filter, int32_t K, int32_t tile_size,
                           int32_t* ids_out, double* scores_out) {
    const int64_t N = g->num_nodes;
    if (K <= 0 || tile_size <= 0 || N <= 0) return 0;
    std::vector<double> fin(static_cast<size_t>(N));
    oracle_scores(g, q, t_q, lambda, mod_filter, fin.data(), nullptr);
    std::vector<int64_t> cand;
    std::vector<int32_t> ti(static_cast<size_t>(K));
    std::vector<double> tv(static_cast<size_t>(K));
    for (int64_t off = 0; off < N; off += tile_size) {
        const int64_t nt = std::min<int64_t>(tile_size, N - off);
        const int32_t k = oracle_topk(fin.data() + off, nt, K, ti.data(), tv.data());
        for (int32_t j = 0; j < k; ++j)
            if (tv[size_t(j)] > -double(FLT_MAX) * 0.5) cand.push_back(off + ti[size_t(j)]);
    }
    std::sort(cand.begin(), cand.end(), [&](int64_t a, int64_t b) { return key_less(fin[a], a, fin[b], b); });
    const int32_t n = int32_t(std::min<size_t>(cand.size(), size_t(K)));
    for (int32_t j = 0; j < n; ++j) { ids_out[j] = int32_t(cand[size_t(j)]); scores_out[j] = fin[cand[size_t(j)]]; }
    return n;
}

// ---------------------------------------------------------------------------
// k nearest neighbours by cosine: fp64 dot of the fp32 rows (unit rows, so the
// dot is the cosine) of each node in qids against rows [0, n), the node itself
// excluded, order (similarity desc, id asc). The k-NN half of the benchmark's
// NSN rule ("intra-episode pairs + 8 nearest neighbours"); the reference's own
// neighbour search is the tiled brute force of cmng_build.cu:135-245.
// Fewer than k candidates: the rest of the row is -1 / -inf.
// ---------------------------------------------------------------------------
void oracle_knn(const float* emb, int64_t n, int32_t d, const int32_t* qids, int32_t nq, int32_t k,
                int32_t* out, double* sims) {
#pragma omp parallel for schedule(dynamic, 4)
    for (int32_t i = 0; i < nq; ++i) {
        const int64_t u = qids[i];
        const float* x = emb + u * d;
        std::vector<std::pair<double, int64_t>> best;      // (-sim, id), kept sorted, <= k
        best.reserve(size_t(k) + 1);
        for (int64_t v = 0; v < n; ++v) {
            if (v == u) continue;
            const float* y = emb + v * d;
            double acc = 0.0;
            for (int32_t j = 0; j < d; ++j) acc += double(x[j]) * double(y[j]);
            const std::pair<double, int64_t> key(-acc, v);
            if (int32_t(best.size()) == k && !(key < best.back())) continue;
            best.insert(std::upper_bound(best.begin(), best.end(), key), key);
            if (int32_t(best.size()) > k) best.pop_back();
        }
        for (int32_t j = 0; j < k; ++j) {
            const bool ok = j < int32_t(best.size());
            out[int64_t(i) * k + j] = ok ? int32_t(best[size_t(j)].second) : -1;
            if (sims) sims[int64_t(i) * k + j] = ok ? -best[size_t(j)].first : -HUGE_VAL;
        }
    }
}

// ---------------------------------------------------------------------------
// Streaming insert edge rule. The reference's flush keeps every old edge, adds
// edges for the new nodes to both endpoints through a std::set adjacency and
// re-packs the CSR with rows ascending (streaming.cpp:35-80, 97-104, 155-162);
// which edges it adds (ring lattice by id + sampled cross-modal bridges,
// :111-153) is replaced by the benchmark's NSN rule: for each new node u
// (ids n_old .. n_old + n_new - 1) every other new node with the same episode
// id (ep_new may be NULL: no episode edges) and its k neighbours knn[u] (ids
// < 0 skipped). out_row: n_old + n_new + 1 entries. Returns the edge count;
// call with out_col == NULL to size it.
// ---------------------------------------------------------------------------
int64_t oracle_insert_edges(int32_t n_old, const int32_t* row, const int32_t* col, int32_t n_new,
                            const int32_t* ep_new, const int32_t* knn, int32_t k, int32_t* out_row,
                            int32_t* out_col) {
    const int32_t n = n_old + n_new;
    std::vector<std::set<int32_t>> adj(static_cast<size_t>(n));
    for (int32_t i = 0; i < n_old; ++i)
        if (row)
            for (int32_t j = row[i]; j < row[i + 1]; ++j) adj[size_t(i)].insert(col[j]);
    auto link = [&](int32_t a, int32_t b) {
        if (a == b || b < 0 || b >= n) return;
        adj[size_t(a)].insert(b);
        adj[size_t(b)].insert(a);
    };
    for (int32_t i = 0; i < n_new; ++i) {
        if (ep_new)
            for (int32_t j = 0; j < n_new; ++j)
                if (j != i && ep_new[j] == ep_new[i]) link(n_old + i, n_old + j);
        for (int32_t j = 0; j < k; ++j) link(n_old + i, knn[int64_t(i) * k + j]);
    }
    int64_t e = 0;
    if (out_row) out_row[0] = 0;
    for (int32_t i = 0; i < n; ++i) {
        for (int32_t v : adj[size_t(i)]) {
            if (out_col) out_col[e] = v;
            ++e;
        }
        if (out_row) out_row[i + 1] = int32_t(e);
    }
    return e;
}

// ---------------------------------------------------------------------------
// Deferred k-NN edges of nodes already in the graph (ids first .. first+count-1):
// the same std::set adjacency union as the insert rule above, over an existing
// CSR of n nodes: every old edge kept, (u, v) and (v, u) added for each listed
// neighbour v of u (ids < 0 or >= n and v == u skipped), rows ascending.
// out_row: n + 1 entries. Returns the edge count; out_col == NULL sizes it.
// ---------------------------------------------------------------------------
int64_t oracle_link_edges(int32_t n, const int32_t* row, const int32_t* col, int32_t first, int32_t count,
                          const int32_t* knn, int32_t k, int32_t* out_row, int32_t* out_col) {
    std::vector<std::set<int32_t>> adj(static_cast<size_t>(n));
    for (int32_t i = 0; i < n; ++i)
        if (row)
            for (int32_t j = row[i]; j < row[i + 1]; ++j) adj[size_t(i)].insert(col[j]);
    for (int32_t i = 0; i < count; ++i) {
        const int32_t u = first + i;
        for (int32_t j = 0; j < k; ++j) {
            const int32_t v = knn[int64_t(i) * k + j];
            if (v < 0 || v >= n || v == u) continue;
            adj[size_t(u)].insert(v);
            adj[size_t(v)].insert(u);
        }
    }
    int64_t e = 0;
    if (out_row) out_row[0] = 0;
    for (int32_t i = 0; i < n; ++i) {
        for (int32_t v : adj[size_t(i)]) {
            if (out_col) out_col[e] = v;
            ++e;
        }
        if (out_row) out_row[i + 1] = int32_t(e);
    }
    return e;
}

// ---------------------------------------------------------------------------
// Probe sample of the kids sweep: demos/embodied_scene/bench_kids_sweep.cu:624-632.
// std::mt19937 seeded uint32(N) ^ 0xA5A5A5A5 and uniform_int_distribution<size_t>
// over [0, n_image - 1] (the same engine and distribution of this C++ library);
// out[p] = the index into the IMAGE-node list of probe p. Pinned by tests/test_oracle.py
// against numpy's MT19937 (the standard's seeding; the standard's 10000th-output known
// answer) and Lemire's nearly-divisionless method restated there, the algorithm libstdc++
// uses for a 32-bit engine. The sweep itself is CUDA code and cannot run here.
// ---------------------------------------------------------------------------
void oracle_kids_probes(int32_t N, int64_t n_image, int32_t count, int64_t* out) {
    std::mt19937 rng(uint32_t(N) ^ 0xA5A5A5A5u);
    std::uniform_int_distribution<size_t> pick(0, size_t(n_image) - 1);
    for (int32_t p = 0; p < count; ++p) out[p] = int64_t(pick(rng));
}

// ---------------------------------------------------------------------------
// Importance update: update_importance, memory_cuda.cu:1484-1527. fp32 as the
// reference: retain = 1.0f - decay_rate; every node i < n: imp[i] = imp[i] * retain
// (importance_decay_kernel :1486-1491); then each listed id, in list order:
// imp[id] = fminf(imp[id] + boost, max_imp) (importance_boost_kernel :1494-1505).
// Ids < 0 are skipped (:1502); ids >= n are skipped here (the reference writes out of
// bounds). A repeated id is boosted once per occurrence, in order (the reference's
// threads race on it).
// ---------------------------------------------------------------------------
void oracle_importance_update(float* imp, int32_t n, const int32_t* ids, int32_t n_ids, float boost,
                              float decay_rate, float max_imp) {
    const float retain = 1.0f - decay_rate;
    for (int32_t i = 0; i < n; ++i) imp[i] = imp[i] * retain;
    for (int32_t t = 0; t < n_ids; ++t) {
        const int32_t id = ids[t];
        if (id < 0 || id >= n) continue;
        const float sum = imp[id] + boost;
        imp[id] = std::fmin(sum, max_imp);
    }
}

// ---------------------------------------------------------------------------
// Novelty: compute_novelty, memory_cuda.cu:1547-1596: max over i < N of <E_i, q>
// (fp64 here), starting from -1 (:1589), and 0 when N <= 0 (:1570). *scale gets
// max_i sum_d |E_id q_d|, which bounds the fp32 rounding error of any one dot.
// ---------------------------------------------------------------------------
double oracle_novelty(const oracle_graph* g, const float* q, double* scale) {
    const int64_t N = g->num_nodes, D = g->dim;
    if (scale) *scale = 0.0;
    if (N <= 0) return 0.0;
    double best = -1.0, sc = 0.0;
#pragma omp parallel for reduction(max : best, sc) schedule(static)
    for (int64_t i = 0; i < N; ++i) {
        const float* e = g->emb + i * D;
        double s = 0.0, a = 0.0;
        for (int64_t d = 0; d < D; ++d) {
            const double p = double(e[d]) * double(q[d]);
            s += p;
            a += std::fabs(p);
        }
        best = std::max(best, s);
        sc = std::max(sc, a);
    }
    if (scale) *scale = sc;
    return best;
}

// ---------------------------------------------------------------------------
// Edge hits: count_edge_hits_kernel, memory_cuda.cu:1612-1632. hop[v] is the BFS
// level of node v (-1 = unvisited; hop_by_node of oracle_bfs). For every node v with
// hop[v] > 0 (:1619) and every edge e of v (:1621-1630): hits[e] += 1 when
// hop[col[e]] == hop[v] - 1.
// ---------------------------------------------------------------------------
void oracle_edge_hits(const int32_t* row, const int32_t* col, int32_t n, const int32_t* hop, int32_t* hits) {
    for (int32_t v = 0; v < n; ++v) {
        const int32_t h = hop[v];
        if (h <= 0) continue;
        for (int32_t e = row[v]; e < row[v + 1]; ++e) {
            const int32_t u = col[e];
            if (u >= 0 && u < n && hop[u] == h - 1) ++hits[e];
        }
    }
}

// ---------------------------------------------------------------------------
// Maintenance sweep: maintain_graph, memory_cuda.cu:1636-1658: the number of edges
// with hits <= min_hits (:1647-1649), then every counter reset to 0 (:1652).
// ---------------------------------------------------------------------------
int32_t oracle_maintain(int32_t* hits, int64_t n_edges, int32_t min_hits) {
    int32_t low = 0;
    for (int64_t e = 0; e < n_edges; ++e) {
        if (hits[e] <= min_hits) ++low;
        hits[e] = 0;
    }
    return low;
}

}  // extern "C"

