// ============================================================================
//  corpus.cpp — seeded benchmark corpus, CPU k-NN, NSN CSR assembly and the
//  host episode CSR (declared in include/mars_corpus.h).
// ============================================================================
#include "mars_corpus.h"
#include "mars_amd.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

namespace {

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;

inline uint64_t fmix64(uint64_t z) {                  // SplitMix64 finaliser
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// One 64-bit draw for (seed, stream, index): independent of evaluation order.
inline uint64_t draw(uint64_t seed, uint64_t stream, uint64_t index) {
    uint64_t s = fmix64(seed + kGolden * (stream + 1));
    return fmix64(s + kGolden * (index + 1));
}

inline double unit_open(uint64_t u) {                  // (0, 1)
    return (double(u >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

// Standard normal number `index` of stream `stream` (Box-Muller pair 2j, 2j+1).
inline double normal(uint64_t seed, uint64_t stream, uint64_t index) {
    const uint64_t pair = index >> 1;
    const double u1 = unit_open(draw(seed, stream, 2 * pair));
    const double u2 = unit_open(draw(seed, stream, 2 * pair + 1));
    const double r = std::sqrt(-2.0 * std::log(u1));
    const double th = 6.283185307179586476925286766559 * u2;
    return (index & 1) ? r * std::sin(th) : r * std::cos(th);
}

// Stream ids: (kind << 40) | object id.
enum : uint64_t { kCentroid = 1, kNoise = 2, kStart = 3, kQuery = 4 };
inline uint64_t stream_id(uint64_t kind, uint64_t obj) { return (kind << 40) ^ obj; }

int slot_modality(int32_t slot) {
    const int32_t s = slot % 10;
    if (s < 4) return MARS_MOD_IMAGE;
    if (s < 7) return MARS_MOD_TEXT;
    return MARS_MOD_AUDIO;
}

int resolve_threads(int32_t t) {
    if (t > 0) return t;
    unsigned h = std::thread::hardware_concurrency();
    return h ? int(h) : 1;
}

template <typename F>
void parallel_for(int64_t n, int threads, F&& f) {       // f(lo, hi)
    threads = int(std::max<int64_t>(1, std::min<int64_t>(threads, n)));
    if (threads == 1) { f(int64_t(0), n); return; }
    std::vector<std::thread> pool;
    for (int t = 0; t < threads; ++t) {
        const int64_t lo = n * t / threads, hi = n * (t + 1) / threads;
        pool.emplace_back([&f, lo, hi] { f(lo, hi); });
    }
    for (auto& th : pool) th.join();
}

}  // namespace

extern "C" {

void mars_corpus_default(mars_corpus_params* p, int64_t num_nodes, int32_t dim, uint64_t seed) {
    p->num_nodes = num_nodes;
    p->embedding_dim = dim;
    p->episode_len = 10;
    p->seed = seed;
    p->image_noise = 0.3f;
    p->other_centroid = 0.35f;
    p->start_max = 599.0f;
    p->slot_dt = 0.1f;
}

int mars_corpus_generate(const mars_corpus_params* p, float* emb, int32_t* mods, float* ts,
                         int32_t* ep_ids, int32_t threads) {
    if (!p || p->num_nodes <= 0 || p->embedding_dim <= 0 || p->episode_len <= 0)
        return MARS_ERR_INVALID;
    const int64_t N = p->num_nodes;
    const int32_t D = p->embedding_dim, L = p->episode_len;
    const int64_t n_ep = (N + L - 1) / L;
    parallel_for(n_ep, resolve_threads(threads), [&](int64_t e0, int64_t e1) {
        std::vector<float> c(size_t(D), 0.0f);
        std::vector<double> v(size_t(D), 0.0);
        for (int64_t e = e0; e < e1; ++e) {
            if (emb)
                for (int32_t d = 0; d < D; ++d)
                    c[size_t(d)] = float(normal(p->seed, stream_id(kCentroid, uint64_t(e)), uint64_t(d)));
            const float start = float(unit_open(draw(p->seed, stream_id(kStart, uint64_t(e)), 0)) *
                                      double(p->start_max));
            for (int32_t s = 0; s < L; ++s) {
                const int64_t i = e * L + s;
                if (i >= N) break;
                const int mod = slot_modality(s);
                if (mods) mods[i] = mod;
                if (ts) ts[i] = start + p->slot_dt * float(s);
                if (ep_ids) ep_ids[i] = int32_t(e);
                if (!emb) continue;
                double nrm = 0.0;
                for (int32_t d = 0; d < D; ++d) {
                    const float g = float(normal(p->seed, stream_id(kNoise, uint64_t(i)), uint64_t(d)));
                    const float x = (mod == MARS_MOD_IMAGE) ? c[size_t(d)] + p->image_noise * g
                                                            : p->other_centroid * c[size_t(d)] + g;
                    v[size_t(d)] = double(x);
                    nrm += double(x) * double(x);
                }
                nrm = std::sqrt(nrm);
                float* row = emb + i * D;
                for (int32_t d = 0; d < D; ++d) row[d] = float(v[size_t(d)] / nrm);
            }
        }
    });
    return MARS_OK;
}

int mars_corpus_pick_queries(const int32_t* mods, int64_t n, int32_t mod, int32_t n_queries,
                             uint64_t seed, int32_t* out) {
    if (!mods || n <= 0 || n_queries < 0 || (n_queries > 0 && !out)) return MARS_ERR_INVALID;
    std::vector<int32_t> pool;
    for (int64_t i = 0; i < n; ++i) if (mods[i] == mod) pool.push_back(int32_t(i));
    if (pool.empty()) return n_queries ? MARS_ERR_INVALID : MARS_OK;
    for (int32_t j = 0; j < n_queries; ++j) {
        const uint64_t u = draw(seed, stream_id(kQuery, 0), uint64_t(j));
        const uint64_t pick = uint64_t((unsigned __int128)u * pool.size() >> 64);
        out[j] = pool[size_t(pick)];
    }
    return MARS_OK;
}

int mars_knn_cpu(const float* emb, int64_t n, int32_t D, int32_t k, int32_t* nbrs,
                 float* sims, int32_t threads) {
    if (!emb || n <= 0 || D <= 0 || k <= 0 || !nbrs) return MARS_ERR_INVALID;
    constexpr int QB = 4;     // queries per block
    constexpr int RB = 32;    // corpus rows per tile (tile stored transposed: D x RB)
    const int th = resolve_threads(threads);
    const int64_t ntiles = (n + RB - 1) / RB;
    std::vector<float> tiles(size_t(ntiles) * size_t(D) * RB);
    parallel_for(ntiles, th, [&](int64_t t0, int64_t t1) {
        for (int64_t t = t0; t < t1; ++t) {
            float* tl = &tiles[size_t(t) * size_t(D) * RB];
            for (int r = 0; r < RB; ++r) {
                const int64_t id = t * RB + r;
                for (int32_t d = 0; d < D; ++d)
                    tl[size_t(d) * RB + r] = (id < n) ? emb[id * D + d] : 0.0f;
            }
        }
    });
    const int64_t nqb = (n + QB - 1) / QB;
    parallel_for(nqb, th, [&](int64_t b0, int64_t b1) {
        std::vector<float> bv(size_t(QB) * k);
        std::vector<int32_t> bi(size_t(QB) * k);
        std::vector<float> qv(size_t(QB) * D);
        for (int64_t qb = b0; qb < b1; ++qb) {
            const int64_t q0 = qb * QB;
            const int nq = int(std::min<int64_t>(QB, n - q0));
            std::fill(bv.begin(), bv.end(), -INFINITY);
            std::fill(bi.begin(), bi.end(), -1);
            for (int a = 0; a < QB; ++a)
                for (int32_t d = 0; d < D; ++d)
                    qv[size_t(d) * QB + a] = (a < nq) ? emb[(q0 + a) * D + d] : 0.0f;
            for (int64_t t = 0; t < ntiles; ++t) {
                const int64_t r0 = t * RB;
                const int nr = int(std::min<int64_t>(RB, n - r0));
                const float* tl = &tiles[size_t(t) * size_t(D) * RB];
                float acc[QB][RB];
                for (int a = 0; a < QB; ++a) for (int r = 0; r < RB; ++r) acc[a][r] = 0.0f;
                for (int32_t d = 0; d < D; ++d) {
                    const float* tr = tl + size_t(d) * RB;
                    for (int a = 0; a < QB; ++a) {
                        const float x = qv[size_t(d) * QB + a];
                        for (int r = 0; r < RB; ++r) acc[a][r] += x * tr[r];
                    }
                }
                for (int a = 0; a < nq; ++a) {
                    float* v = &bv[size_t(a) * k];
                    int32_t* ix = &bi[size_t(a) * k];
                    for (int r = 0; r < nr; ++r) {
                        const int64_t id = r0 + r;
                        if (id == q0 + a) continue;
                        const float s = acc[a][r];
                        // not better than the current k-th under (score desc, id asc)
                        if (s < v[k - 1] || (s == v[k - 1] && ix[k - 1] >= 0 && id > ix[k - 1])) continue;
                        int pos = k - 1;
                        while (pos > 0 && (s > v[pos - 1] || (s == v[pos - 1] && id < ix[pos - 1]))) {
                            v[pos] = v[pos - 1]; ix[pos] = ix[pos - 1]; --pos;
                        }
                        v[pos] = s; ix[pos] = int32_t(id);
                    }
                }
            }
            for (int a = 0; a < nq; ++a) {
                std::memcpy(nbrs + (q0 + a) * k, &bi[size_t(a) * k], sizeof(int32_t) * size_t(k));
                if (sims) std::memcpy(sims + (q0 + a) * k, &bv[size_t(a) * k], sizeof(float) * size_t(k));
            }
        }
    });
    return MARS_OK;
}

int mars_build_episode_csr(const int32_t* ids, int32_t n, int32_t* num_episodes, int32_t* offsets,
                           int32_t* members) {
    if (!num_episodes) return MARS_ERR_INVALID;
    *num_episodes = 0;
    if (n <= 0 || !ids) return MARS_OK;                       // empty CSR, as the reference
    int32_t max_ep = 0;
    for (int32_t i = 0; i < n; ++i) {
        if (ids[i] < 0) return MARS_ERR_INVALID;
        if (ids[i] > max_ep) max_ep = ids[i];
    }
    *num_episodes = max_ep + 1;
    if (!offsets) return MARS_OK;
    if (!members) return MARS_ERR_INVALID;
    std::memset(offsets, 0, sizeof(int32_t) * (size_t(max_ep) + 2));
    for (int32_t i = 0; i < n; ++i) ++offsets[ids[i] + 1];
    for (int32_t e = 0; e <= max_ep; ++e) offsets[e + 1] += offsets[e];
    std::vector<int32_t> cursor(offsets, offsets + max_ep + 1);
    for (int32_t i = 0; i < n; ++i) members[cursor[size_t(ids[i])]++] = i;
    return MARS_OK;
}

int mars_build_nsn_csr(int64_t n, const int32_t* ep_ids, const int32_t* knn, int32_t k,
                       int32_t* row_offsets, int32_t* col, int64_t* num_edges, int32_t threads) {
    if (n <= 0 || n > INT32_MAX - 1 || !ep_ids || !row_offsets || !num_edges || k < 0 ||
        (k > 0 && !knn))
        return MARS_ERR_INVALID;
    const int th = resolve_threads(threads);
    // episode membership (ascending ids per episode)
    int32_t n_ep = 0;
    if (mars_build_episode_csr(ep_ids, int32_t(n), &n_ep, nullptr, nullptr) != MARS_OK)
        return MARS_ERR_INVALID;
    std::vector<int32_t> eoff(static_cast<size_t>(n_ep) + 1), emem(static_cast<size_t>(n));
    mars_build_episode_csr(ep_ids, int32_t(n), &n_ep, eoff.data(), emem.data());
    // reverse kNN lists
    std::vector<int64_t> roff(static_cast<size_t>(n) + 1, 0);
    for (int64_t i = 0; i < n * k; ++i) if (knn[i] >= 0 && knn[i] < n) ++roff[size_t(knn[i]) + 1];
    for (int64_t i = 0; i < n; ++i) roff[size_t(i) + 1] += roff[size_t(i)];
    std::vector<int32_t> rev(static_cast<size_t>(roff[size_t(n)]));
    {
        std::vector<int64_t> cur(roff.begin(), roff.end() - 1);
        for (int64_t i = 0; i < n; ++i)
            for (int32_t j = 0; j < k; ++j) {
                const int32_t t = knn[i * k + j];
                if (t >= 0 && t < n) rev[size_t(cur[size_t(t)]++)] = int32_t(i);
            }
    }
    // per-row degree after de-duplication
    auto gather = [&](int64_t i, std::vector<int32_t>& row) {
        row.clear();
        const int32_t e = ep_ids[i];
        for (int32_t m = eoff[size_t(e)]; m < eoff[size_t(e) + 1]; ++m)
            if (emem[size_t(m)] != i) row.push_back(emem[size_t(m)]);
        for (int32_t j = 0; j < k; ++j) {
            const int32_t t = knn[i * k + j];
            if (t >= 0 && t < n && t != i) row.push_back(t);
        }
        for (int64_t r = roff[size_t(i)]; r < roff[size_t(i) + 1]; ++r)
            if (rev[size_t(r)] != i) row.push_back(rev[size_t(r)]);
        std::sort(row.begin(), row.end());
        row.erase(std::unique(row.begin(), row.end()), row.end());
    };
    std::vector<int32_t> deg(static_cast<size_t>(n));
    parallel_for(n, th, [&](int64_t lo, int64_t hi) {
        std::vector<int32_t> row;
        for (int64_t i = lo; i < hi; ++i) { gather(i, row); deg[size_t(i)] = int32_t(row.size()); }
    });
    int64_t total = 0;
    for (int64_t i = 0; i < n; ++i) total += deg[size_t(i)];
    if (total > INT32_MAX) return MARS_ERR_CAPACITY;
    *num_edges = total;
    if (!col) return MARS_OK;
    row_offsets[0] = 0;
    for (int64_t i = 0; i < n; ++i) row_offsets[i + 1] = row_offsets[i] + deg[size_t(i)];
    parallel_for(n, th, [&](int64_t lo, int64_t hi) {
        std::vector<int32_t> row;
        for (int64_t i = lo; i < hi; ++i) {
            gather(i, row);
            std::memcpy(col + row_offsets[i], row.data(), row.size() * sizeof(int32_t));
        }
    });
    return MARS_OK;
}

}  // extern "C"
