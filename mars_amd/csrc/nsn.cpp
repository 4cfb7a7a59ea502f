// ============================================================================
//  nsn.cpp — the 5-phase NSN edge builder of the reference's host graph
//  (MemoryGraph::build_nsn_edges_configurable, src/memory_graph.cpp:102-189),
//  host code of libmars_amd.
//
//  The builder draws from one std::mt19937 seeded 7 and its draws depend on the
//  adjacency built so far (phase 4 draws a new target only when the ring edge is
//  still present and the row keeps more than two neighbours). So it is sequential
//  by construction, and it runs on the host. It uses the same standard-library
//  engine and distributions as the reference, in the same order, so a graph built
//  with the same compiler's standard library is identical, edge for edge.
//
//  The reference keeps one std::unordered_set per node. Rows here are small
//  unsorted vectors (degrees stay near k + 4: ring, a few skips, hub extras,
//  bridges), searched linearly, and sorted once for the CSR. That is the same set
//  semantics with one allocation per row.
//
//  Phases (bits of `phases`, all set = the reference's defaults):
//    1 ring lattice: i -- (i + j) mod N for j = 1..k/2
//    2 skips: for each level l = 1..max(1, floor(log2 N)), i -- (i + 2^l) mod N for i
//      a multiple of 2^l
//    4 hubs: every floor(sqrt N)-th node gets max(2, floor(log2 N) / 2) random edges
//    8 rewiring (with the ring): each ring edge (i, i + j) is, with probability p,
//      replaced by an edge to a random node when i keeps more than two neighbours
//   16 bridges: each node gets one edge to a random node of each other modality
// ============================================================================
#include "mars_amd.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <random>
#include <vector>

namespace mars {
int set_error(int code, const char* fmt, ...);
}

namespace {

constexpr int32_t kModalities = 3;     // MOD_TEXT, MOD_AUDIO, MOD_IMAGE

struct Rows {
    std::vector<std::vector<int32_t>> r;
    explicit Rows(int32_t n) : r(static_cast<size_t>(n)) {}
    bool has(int32_t a, int32_t b) const {
        const auto& v = r[size_t(a)];
        return std::find(v.begin(), v.end(), b) != v.end();
    }
    void insert1(int32_t a, int32_t b) {
        if (!has(a, b)) r[size_t(a)].push_back(b);
    }
    void erase1(int32_t a, int32_t b) {
        auto& v = r[size_t(a)];
        const auto it = std::find(v.begin(), v.end(), b);
        if (it != v.end()) {
            *it = v.back();
            v.pop_back();
        }
    }
    void add(int32_t a, int32_t b) {       // undirected, no self edges
        if (a == b) return;
        insert1(a, b);
        insert1(b, a);
    }
};

int64_t edge_bound(int32_t n, int32_t k) {
    const int64_t N = n;
    const int64_t hub_int = std::max<int64_t>(1, int64_t(std::sqrt(double(N))));
    const int64_t extras = std::max<int64_t>(2, int64_t(std::log2(double(N))) / 2);
    // ring + skips (sum over levels of ceil(N / 2^l) <= N + 31) + hubs + bridges, both
    // directions; rewiring removes an edge for each one it adds
    return 2 * N * std::max(0, k / 2) + 2 * (N + 31) + 2 * ((N + hub_int - 1) / hub_int) * extras +
           2 * N * (kModalities - 1);
}

}  // namespace

extern "C" int mars_nsn_edges(int32_t n, const int32_t* modalities, int32_t k, double p, uint32_t phases,
                              int32_t* row_offsets, int32_t* col, int64_t col_cap, int64_t* num_edges) {
    using mars::set_error;
    if (n < 0 || k < 0 || !num_edges || ((phases & MARS_NSN_BRIDGES) && n > 0 && !modalities))
        return set_error(MARS_ERR_INVALID, "nsn: bad arguments (n %d, k %d)", n, k);
    if (!col) {                                                   // sizing call
        *num_edges = n > 0 ? edge_bound(n, k) : 0;
        return MARS_OK;
    }
    if (!row_offsets) return set_error(MARS_ERR_INVALID, "nsn: null row_offsets");
    if (n == 0) {
        row_offsets[0] = 0;
        *num_edges = 0;
        return MARS_OK;
    }
    if (phases & MARS_NSN_BRIDGES)
        for (int32_t i = 0; i < n; ++i)
            if (modalities[i] < 0 || modalities[i] >= kModalities)
                return set_error(MARS_ERR_INVALID, "nsn: modality %d of node %d outside [0, 3)", modalities[i], i);
    const int32_t N = n;
    Rows s(N);
    std::mt19937 rng(7);                                          // memory_graph.cpp:114-116
    std::uniform_real_distribution<double> U(0.0, 1.0);
    std::uniform_int_distribution<int32_t> RN(0, N - 1);
    const bool ring = (phases & MARS_NSN_RING) != 0;
    if (ring)
        for (int32_t i = 0; i < N; ++i)
            for (int32_t j = 1; j <= k / 2; ++j) s.add(i, int32_t((int64_t(i) + j) % N));
    if (phases & MARS_NSN_SKIPS) {
        const int32_t levels = std::max(1, int32_t(std::log2(double(N))));
        for (int32_t lvl = 1; lvl <= levels && lvl < 31; ++lvl) {
            const int64_t step = int64_t(1) << lvl;
            for (int64_t i = 0; i < N; i += step) s.add(int32_t(i), int32_t((i + step) % N));
        }
    }
    if (phases & MARS_NSN_HUBS) {
        const int32_t hub_int = std::max(1, int32_t(std::sqrt(double(N))));
        const int32_t extras = std::max(2, int32_t(std::log2(double(N))) / 2);
        for (int64_t h = 0; h < N; h += hub_int)
            for (int32_t e = 0; e < extras; ++e) s.add(int32_t(h), RN(rng));
    }
    if ((phases & MARS_NSN_REWIRE) && ring) {
        for (int32_t i = 0; i < N; ++i)
            for (int32_t j = 1; j <= k / 2; ++j) {
                if (U(rng) < p) {
                    const int32_t old_t = int32_t((int64_t(i) + j) % N);
                    if (s.has(i, old_t) && s.r[size_t(i)].size() > 2) {
                        s.erase1(i, old_t);
                        s.erase1(old_t, i);
                        s.add(i, RN(rng));
                    }
                }
            }
    }
    if (phases & MARS_NSN_BRIDGES) {
        std::vector<std::vector<int32_t>> by_mod(kModalities);
        for (int32_t i = 0; i < N; ++i) by_mod[size_t(modalities[i])].push_back(i);
        for (int32_t i = 0; i < N; ++i) {
            const int32_t mine = modalities[i];
            for (int32_t m = 0; m < kModalities; ++m) {
                if (m == mine || by_mod[size_t(m)].empty()) continue;
                const auto& pool = by_mod[size_t(m)];
                s.add(i, pool[rng() % pool.size()]);
            }
        }
    }
    int64_t e = 0;
    row_offsets[0] = 0;
    for (int32_t i = 0; i < N; ++i) {
        e += int64_t(s.r[size_t(i)].size());
        if (e > INT32_MAX) return set_error(MARS_ERR_CAPACITY, "nsn: more than 2^31 - 1 edges");
        row_offsets[i + 1] = int32_t(e);
    }
    *num_edges = e;
    if (e > col_cap) return set_error(MARS_ERR_CAPACITY, "nsn: %lld edges, col holds %lld", (long long)e,
                                      (long long)col_cap);
    for (int32_t i = 0; i < N; ++i) {
        auto& v = s.r[size_t(i)];
        std::sort(v.begin(), v.end());
        std::memcpy(col + row_offsets[i], v.data(), v.size() * sizeof(int32_t));
    }
    return MARS_OK;
}
