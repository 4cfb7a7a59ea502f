// ============================================================================
//  kernels.hip — retrieval hot-path kernels for gfx950 (wave64).
//
//  k_scan       Q=1 global scan. Rows are read by 16-lane groups (a DPP row):
//               lane s of a group reads 16-byte pieces s, s+16, s+32, ... of the
//               row, so one wave load instruction covers four rows with four
//               fully used 256-byte segments. The dot product is finished with a
//               4-step in-row reduction; temporal decay, modality filter and the
//               same-episode boost are applied in registers; the fused score is
//               written once (4 bytes/row) and offered to a wave-held top-K list
//               (lane i holds the i-th smallest key). Each workgroup writes its
//               K best keys. Replaces cublasSgemv + temporal_rerank_kernel +
//               episode_same_boost_kernel + negate/iota/CUB sort/extract
//               (reference src/memory_cuda.cu:1207-1283, :400-440, :737-771).
//  k_finalize   One workgroup: merges the per-workgroup keys into the K seeds,
//               runs the deterministic level-synchronous BFS (first discoverer in
//               (frontier position, CSR slot) order wins, via a 64-bit atomicMin
//               claim and an in-order compaction), then sorts the visited set by
//               (score desc, id asc) and writes the results straight into pinned
//               host memory. Replaces bfs_init_seeds / bfs_expand_device_driven /
//               compact_results and the host std::sort (src/memory_cuda.cu:633-732,
//               :1300-1345, :1421-1447).
//  k_episode    Episode-scoped query in one launch: dot + decay over the member
//               range only, top-K, reference padding, results. Replaces
//               fill_neg_inf_final + cosine_episode_subset_fused + the O(N) sort /
//               compaction (src/memory_cuda.cu:421-424, :443-493, :1194-1206).
//  k_convert_f16  RNE fp32 -> fp16 copy with 64-bit indexing (convert_f32_to_f16,
//               src/memory_cuda.cu:207-211 and :858-868, which overflows int32).
// ============================================================================
#include "device.hpp"

namespace mars {
namespace {

// Row groups of 4 rows (one per 16-lane group) are dealt out grid-stride: wave w of
// workgroup b takes groups (it * gridDim.x * 4 + b * 4 + w) * kUnroll + u, so at any
// moment the grid sweeps one contiguous window of the corpus; kUnroll groups per
// step keep 2 x 4 rows of loads in flight per wave.
constexpr int kScanUnroll = 2;

// SIDE = false: the query has no modality filter and no episode boost, so the
// per-row modality and episode ids are not read (modality 0, episode -1 give
// fuse_score's no-filter, no-boost result). The compiler also schedules that
// variant better: 235 us against 245 us for the fp16 scan of 1M x 768 rows at 512
// workgroups on MI355X.
template <typename T, typename QF, bool SIDE>
__global__ __launch_bounds__(256) void k_scan(ScanArgs a) {
    __shared__ uint64_t s_lists[4][64];
    const int lane = lane_id(), wave = int(threadIdx.x >> 6);
    const int sub = lane & 15, grp = lane >> 4;
    const int k = a.k;
    QF qf;
    if constexpr (std::is_same_v<QF, QGeneric>) qf.d = a.d;
    qf.load(a.q, sub);
    const T* emb = static_cast<const T*>(a.emb);
    const bool use_boost = SIDE && a.boost > 0.0f && a.ep_ids != nullptr;
    uint64_t list = kEmptyKey, thr = kEmptyKey;
    const int64_t ngroups = (a.n + 3) / 4;
    const int64_t gstride = int64_t(gridDim.x) * 4 * kScanUnroll;
    for (int64_t g0 = (int64_t(blockIdx.x) * 4 + wave) * kScanUnroll; g0 < ngroups; g0 += gstride) {
        float dot[kScanUnroll], ts[kScanUnroll];
        int32_t mod[kScanUnroll], ep[kScanUnroll];
#pragma unroll
        for (int u = 0; u < kScanUnroll; ++u) {
            int64_t rr = (g0 + u) * 4 + grp;
            rr = rr < a.n ? rr : a.n - 1;
            ts[u] = a.ts[rr];
            mod[u] = (SIDE && a.mod_filter >= 0) ? a.mods[rr] : 0;
            ep[u] = use_boost ? a.ep_ids[rr] : -1;
            dot[u] = qf.dot(emb + rr * a.d, sub);
        }
#pragma unroll
        for (int u = 0; u < kScanUnroll; ++u) {
            const int64_t r = (g0 + u) * 4 + grp;
            const bool valid = r < a.n;
            const float s = fuse_score(row16_sum(dot[u]), ts[u], mod[u], ep[u], a);
            if (valid && sub == 0) a.fin[r] = s;
            const uint64_t key = valid ? make_key(s, uint32_t(a.id_base + r)) : kEmptyKey;
            list_offer(list, thr, key, sub == 0, lane, k);
        }
    }
    s_lists[wave][lane] = list;
    __syncthreads();
    if (wave == 0) wg_publish(s_lists, lane, k, a);
}

// ---- block-wide helpers (1024 threads) --------------------------------------------
constexpr int kFinThreads = 1024;
constexpr int kFinWaves = kFinThreads / 64;

// Inclusive prefix sum across the wave on DPP: row_shr 1, 2, 4, 8 within each 16-lane row
// (lanes shifted in from outside the row read 0), then row_bcast:15 carries row 0's and row
// 2's totals into rows 1 and 3, and row_bcast:31 the first two rows' total into rows 2, 3.
__device__ inline int wave_incl_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true);
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);
    return v;
}

// Exclusive prefix sum across the block; *total gets the block sum.
__device__ inline int block_excl_scan(int v, int* s_wave, int* total) {
    const int lane = lane_id(), wave = int(threadIdx.x >> 6);
    const int incl = wave_incl_scan(v);
    if (lane == 63) s_wave[wave] = incl;
    __syncthreads();
    int off = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < kFinWaves; ++w) {
        const int x = s_wave[w];
        off += (w < wave) ? x : 0;
        tot += x;
    }
    __syncthreads();
    *total = tot;
    return off + incl - v;
}

// largest p in [0, cn) with eoff[p] <= t (eoff[0] == 0 <= t)
__device__ inline int owner_of(const int32_t* eoff, int cn, int t) {
    int lo = 0, hi = cn;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (eoff[mid] <= t) lo = mid; else hi = mid;
    }
    return lo;
}

// Bitonic sort of n (power of two, <= kSortCap) keys with 16-bit payloads in LDS.
__device__ inline void block_bitonic(uint64_t* key, uint16_t* pay, int n) {
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = int(threadIdx.x); i < (n >> 1); i += kFinThreads) {
                const int lo = 2 * i - (i & (stride - 1));
                const int hi = lo + stride;
                const bool up = (lo & size) == 0;
                const uint64_t a = key[lo], b = key[hi];
                if ((a > b) == up) {
                    key[lo] = b; key[hi] = a;
                    const uint16_t t = pay[lo]; pay[lo] = pay[hi]; pay[hi] = t;
                }
            }
            __syncthreads();
        }
    }
}

constexpr int kHashCap = 8192;              // LDS hash slots (power of two)
constexpr int kRoCache = 2048;              // visit positions whose row words stay in LDS
constexpr int kHashLimit = 6144;            // more distinct nodes: use the global arrays instead
constexpr uint32_t kClaimHop = 0xFFu;       // hop field of a claimed, not yet visited node

struct FinShared {
    union {
        struct {
            uint64_t key[kSortCap];
            uint16_t pay[kSortCap];
        } sort;
        struct {
            int32_t rstart[kFrontierChunk];
            int32_t eoff[kFrontierChunk + 1];
            uint32_t hkey[kHashCap];        // node id + 1 (0 = empty slot)
            uint32_t hval[kHashCap];        // (hop << 16) | visit position
        } bfs;
        uint32_t hist[256];
    } u;
    uint64_t lists[kFinWaves][64];
    int64_t ro_cache[kRoCache];          // row words of visit positions < kRoCache (also in vro)
    int32_t seed_id[64];                 // the seeds' node ids (visit positions 0 .. ns - 1)
    int s_wave[kFinWaves];
    int s_misc[8];
};

__device__ inline uint32_t hash_slot0(int32_t v) { return (uint32_t(v) * 2654435761u) >> (32 - 13); }

// Find (or insert) node v in the LDS hash; -1 when the table is full.
// At most kHashLimit + blockDim inserts ever land (later ones bail out on the
// overflow flag), so the table never fills and every probe sequence ends.
__device__ inline int hash_find_or_insert(FinShared& sh, int32_t v) {
    if (sh.s_misc[5]) return -1;
    const uint32_t k = uint32_t(v) + 1u;
    uint32_t s = hash_slot0(v);
    for (int probe = 0; probe < kHashCap; ++probe) {
        const uint32_t cur = sh.u.bfs.hkey[s];
        if (cur == k) return int(s);
        if (cur == 0u) {
            const uint32_t old = atomicCAS(&sh.u.bfs.hkey[s], 0u, k);
            if (old == 0u) {
                if (atomicAdd(&sh.s_misc[4], 1) >= kHashLimit) sh.s_misc[5] = 1;   // overflow
                return int(s);
            }
            if (old == k) return int(s);
        }
        s = (s + 1u) & uint32_t(kHashCap - 1);
    }
    sh.s_misc[5] = 1;
    return -1;
}

__device__ inline int hash_find(const FinShared& sh, int32_t v) {
    const uint32_t k = uint32_t(v) + 1u;
    uint32_t s = hash_slot0(v);
    for (int probe = 0; probe < kHashCap; ++probe) {
        const uint32_t cur = sh.u.bfs.hkey[s];
        if (cur == k) return int(s);
        if (cur == 0u) return -1;
        s = (s + 1u) & uint32_t(kHashCap - 1);
    }
    return -1;
}

// Degrees of frontier slots [c0, c0+cn) -> sh.u.bfs.eoff / rstart; returns the edge count.
// CACHED: the row word of each visited node was stored in a.vro when it was visited (one
// dependent HBM load less per level), and for the first kRoCache positions in LDS too (no
// global load at all).
template <bool CACHED>
__device__ inline int frontier_edges(FinShared& sh, const FinalizeArgs& a, int c0, int cn) {
    const int tid = int(threadIdx.x);
    int deg[4], rs[4], local = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = tid * 4 + j;
        deg[j] = 0; rs[j] = 0;
        if (i < cn) {
            int64_t ro;
            if constexpr (CACHED) ro = (c0 + i < kRoCache) ? sh.ro_cache[c0 + i] : ld_coherent(a.vro + c0 + i);
            else ro = a.ro[ld_coherent(a.vlist + c0 + i)];
            rs[j] = int32_t(uint32_t(ro));
            deg[j] = int32_t(ro >> 32);
        }
        local += deg[j];
    }
    int total = 0;
    int off = block_excl_scan(local, sh.s_wave, &total);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = tid * 4 + j;
        if (i < cn) { sh.u.bfs.eoff[i] = off; sh.u.bfs.rstart[i] = rs[j]; }
        off += deg[j];
    }
    __syncthreads();
    return total;
}

// In-order compaction of one 1024-edge round: returns the number of winners and
// gives each winner its rank.
__device__ inline int round_rank(FinShared& sh, bool won, int* rank) {
    const int lane = lane_id(), wave = int(threadIdx.x >> 6);
    const uint64_t m = __ballot(won);
    if (lane == 0) sh.s_wave[wave] = __popcll(m);
    __syncthreads();
    int woff = 0, wtot = 0;
#pragma unroll
    for (int w = 0; w < kFinWaves; ++w) {
        const int x = sh.s_wave[w];
        woff += (w < wave) ? x : 0;
        wtot += x;
    }
    *rank = woff + __popcll(m & ((1ull << lane) - 1ull));
    return wtot;
}

// BFS with the visited / claim state in the LDS hash. Returns the visit count,
// or -1 if the visit set outgrew the table (nothing global but the visit lists
// was touched, so the caller can run the global-array BFS instead).
// With rk > 0 every wave also keeps the rk best (score, id) keys it emits in
// `best` (wave 0 starts from the seeds), so the results need only a tree merge.
// Modes: kBfsScored scores every node from a.fin (the finalize kernel). kBfsUnscored
// records the visit set, hops and parents only (a.vpar gets each node's parent
// position, no score is read or written; rk must be 0): the visit order and the
// parents do not depend on scores, so scores can be propagated later. kBfsInterval
// also records parents, scores every node from a.fin as an approximation of a score
// with error <= a.eps per fused score, and writes a bound on each node's error to
// a.vdv; `best` then tracks lower ends (score - bound, rounded down). A non-finite
// score or bound sets sh.s_misc[7].
constexpr int kBfsUnscored = 0, kBfsScored = 1, kBfsInterval = 2;
template <int MODE>
__device__ int bfs_lds(FinShared& sh, const FinalizeArgs& a, int ns, int* levels_out, uint64_t& best,
                       uint64_t& bthr, int rk) {
    constexpr int R = 4;                       // 1024-edge rounds cached in registers
    const int tid = int(threadIdx.x);
    for (int i = tid; i < kHashCap; i += kFinThreads) { sh.u.bfs.hkey[i] = 0u; sh.u.bfs.hval[i] = 0xFFFFFFFFu; }
    if (tid == 0) { sh.s_misc[4] = 0; sh.s_misc[5] = 0; }
    __syncthreads();
    if (tid < ns) {
        const int slot = hash_find_or_insert(sh, sh.seed_id[tid]);
        if (slot >= 0) sh.u.bfs.hval[slot] = uint32_t(tid);          // hop 0, position tid
    }
    __syncthreads();
    int fs = 0, fe = ns, levels = 0;
    for (int h = 0; h < a.hops && fs < fe; ++h) {
        int out = fe;
        for (int c0 = fs; c0 < fe; c0 += kFrontierChunk) {
            const int cn = min(kFrontierChunk, fe - c0);
            const int T = frontier_edges<true>(sh, a, c0, cn);
            for (int s0 = 0; s0 < T; s0 += R * kFinThreads) {
                // claim: the smallest parent position wins; visited nodes keep their
                // smaller (hop < 0xFF) value under the atomicMin. The edge, its slot
                // and the two scores the emit needs stay in registers.
                int32_t nb[R], pp[R], slot[R];
                int64_t rw[R];
                float fv[R], ps[R], pd[R];
                bool filt[R];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const int t = s0 + r * kFinThreads + tid;
                    slot[r] = -1; nb[r] = -1; pp[r] = 0; fv[r] = 0.0f; ps[r] = 0.0f; rw[r] = 0;
                    pd[r] = 0.0f; filt[r] = false;
                    if (t < T) {
                        const int p = owner_of(sh.u.bfs.eoff, cn, t);
                        pp[r] = c0 + p;
                        nb[r] = a.col[sh.u.bfs.rstart[p] + (t - sh.u.bfs.eoff[p])];
                    }
                }
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    if (s0 + r * kFinThreads + tid < T && uint32_t(nb[r]) < uint32_t(a.n_live)) {
                        if constexpr (MODE != kBfsUnscored) {
                            fv[r] = a.fin[nb[r]];
                            ps[r] = ld_coherent(a.vscore + pp[r]);
                        }
                        if constexpr (MODE == kBfsInterval) {
                            pd[r] = ld_coherent(a.vdv + pp[r]);
                            filt[r] = a.mod_filter >= 0 && a.mods[nb[r]] != a.mod_filter;
                        }
                        rw[r] = a.ro[nb[r]];
                        slot[r] = hash_find_or_insert(sh, nb[r]);
                        if (slot[r] >= 0) atomicMin(&sh.u.bfs.hval[slot[r]], (kClaimHop << 16) | uint32_t(pp[r]));
                    }
                }
                __syncthreads();
                if (sh.s_misc[5]) return -1;
                // emit winners in (frontier position, CSR slot) order
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    if (s0 + r * kFinThreads >= T) break;                  // block-uniform
                    const bool won = slot[r] >= 0 &&
                                     sh.u.bfs.hval[slot[r]] == ((kClaimHop << 16) | uint32_t(pp[r]));
                    int rank = 0;
                    const int wtot = round_rank(sh, won, &rank);
                    const float sc = fmaxf(ps[r] * a.hop_decay, fv[r] * 0.8f);
                    uint64_t lkey = kEmptyKey;
                    if (won) {
                        const int pos = out + rank;
                        a.vlist[pos] = nb[r];
                        a.vhop[pos] = h + 1;
                        if constexpr (MODE != kBfsUnscored) a.vscore[pos] = sc;
                        if constexpr (MODE != kBfsScored) a.vpar[pos] = pp[r];
                        if constexpr (MODE == kBfsInterval) {
                            // parent term |fl(x d) - fl(y d)| <= d |x - y| + u d (|x| + |y|); own
                            // term 0.8 eps + rounding (0 for a filtered row: both scans give -FLT_MAX)
                            const double u = 0x1p-24, dl = double(a.hop_decay), dp = double(pd[r]);
                            const double ea = dp > 0.0 ? dl * dp + 2.0 * u * dl * (fabs(double(ps[r])) + dp) : 0.0;
                            const double eb = filt[r] ? 0.0 : 0.8 * a.eps + 0.8 * u * (2.0 * fabs(double(fv[r])) + a.eps);
                            const double d = (ea > eb ? ea : eb) * (1.0 + 1e-6);
                            a.vdv[pos] = float(d) < d ? nextafterf(float(d), __builtin_inff()) : float(d);
                            if ((!(fabs(double(sc)) < 1e38) && !filt[r]) || !(d < 1e30)) sh.s_misc[7] = 1;
                            const double lo = double(sc) - d;
                            float lf = float(lo);
                            if (double(lf) > lo) lf = nextafterf(lf, -__builtin_inff());
                            lkey = make_key(lf, uint32_t(nb[r]));
                        }
                        a.vro[pos] = rw[r];
                        if (pos < kRoCache) sh.ro_cache[pos] = rw[r];
                        sh.u.bfs.hval[slot[r]] = (uint32_t(h + 1) << 16) | uint32_t(pos);
                    }
                    if (MODE == kBfsScored && rk > 0)
                        wave_offer(best, bthr, won ? make_key(sc, uint32_t(nb[r])) : kEmptyKey, lane_id(), rk);
                    if (MODE == kBfsInterval && rk > 0) wave_offer(best, bthr, lkey, lane_id(), rk);
                    out += wtot;
                    __syncthreads();
                }
                __threadfence_block();
            }
            __syncthreads();
        }
        fs = fe;
        fe = out;
        ++levels;
    }
    *levels_out = levels;
    return fe;
}

// BFS with the visited / claim state in global memory (any visit-set size).
__device__ int bfs_global(FinShared& sh, const FinalizeArgs& a, int ns, int* levels_out) {
    const int tid = int(threadIdx.x);
    if (tid < ns) a.vis[ld_coherent(a.vlist + tid)] = a.epoch;
    __threadfence();
    __syncthreads();
    int fs = 0, fe = ns, levels = 0;
    for (int h = 0; h < a.hops && fs < fe; ++h) {
        const uint32_t gen = a.gen_base + uint32_t(h);
        const uint64_t hi = uint64_t(0xFFFFFFFFu - gen) << 32;
        int out = fe;
        for (int c0 = fs; c0 < fe; c0 += kFrontierChunk) {
            const int cn = min(kFrontierChunk, fe - c0);
            const int T = frontier_edges<false>(sh, a, c0, cn);
            for (int t = tid; t < T; t += kFinThreads) {
                const int p = owner_of(sh.u.bfs.eoff, cn, t);
                const int32_t nb = a.col[sh.u.bfs.rstart[p] + (t - sh.u.bfs.eoff[p])];
                if (uint32_t(nb) < uint32_t(a.n_live) && ld_coherent(a.vis + nb) != a.epoch)
                    atomicMin(reinterpret_cast<unsigned long long*>(a.claim + nb),
                              (unsigned long long)(hi | uint32_t(c0 + p)));
            }
            __threadfence();
            __syncthreads();
            for (int r0 = 0; r0 < T; r0 += kFinThreads) {
                const int t = r0 + tid;
                bool won = false;
                int p = 0;
                int32_t nb = 0;
                if (t < T) {
                    p = owner_of(sh.u.bfs.eoff, cn, t);
                    nb = a.col[sh.u.bfs.rstart[p] + (t - sh.u.bfs.eoff[p])];
                    won = uint32_t(nb) < uint32_t(a.n_live) && ld_coherent(a.claim + nb) == (hi | uint32_t(c0 + p));
                }
                int rank = 0;
                const int wtot = round_rank(sh, won, &rank);
                if (won) {
                    const int pos = out + rank;
                    const float ps = ld_coherent(a.vscore + c0 + p);
                    a.vlist[pos] = nb;
                    a.vhop[pos] = h + 1;
                    a.vscore[pos] = fmaxf(ps * a.hop_decay, a.fin[nb] * 0.8f);
                    a.vis[nb] = a.epoch;
                }
                out += wtot;
                __threadfence();
                __syncthreads();
            }
        }
        fs = fe;
        fe = out;
        ++levels;
    }
    *levels_out = levels;
    return fe;
}

__device__ inline void write_result(const FinalizeArgs& a, int j, uint64_t key, int32_t hop) {
    const int32_t id = key_id(key);
    mars_query_result r;
    r.node_id = id;
    r.score = key_score(key);
    r.modality = a.mods[id];
    r.hops_from_seed = hop;
    a.rec[j] = r;
}

// Key of rank `need` (1-based, ascending) among the V visit keys: eight 8-bit radix
// passes over the visit list, counting in LDS.
__device__ uint64_t radix_select_key(FinShared& sh, const FinalizeArgs& a, int V, int need) {
    const int tid = int(threadIdx.x);
    uint64_t prefix = 0, mask = 0;
    for (int shift = 56; shift >= 0; shift -= 8) {
        for (int i = tid; i < 256; i += kFinThreads) sh.u.hist[i] = 0;
        __syncthreads();
        for (int i = tid; i < V; i += kFinThreads) {
            const uint64_t key = make_key(ld_coherent(a.vscore + i), uint32_t(ld_coherent(a.vlist + i)));
            if ((key & mask) == prefix) atomicAdd(&sh.u.hist[(key >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid == 0) {
            int cum = 0, dg = 255;
            for (int b = 0; b < 256; ++b) {
                if (cum + int(sh.u.hist[b]) >= need) { dg = b; break; }
                cum += int(sh.u.hist[b]);
            }
            sh.s_misc[1] = dg;
            sh.s_misc[2] = need - cum;
        }
        __syncthreads();
        prefix |= uint64_t(sh.s_misc[1]) << shift;
        mask |= uint64_t(0xFF) << shift;
        need = sh.s_misc[2];
        __syncthreads();
    }
    return prefix;
}

// Results by full sort of the visit set (bitonic in LDS, radix select beyond).
__device__ void select_sorted(FinShared& sh, const FinalizeArgs& a, int V, int rc) {
    const int tid = int(threadIdx.x);
    if (V <= kSortCap) {
        int n2 = 1;
        while (n2 < V) n2 <<= 1;
        for (int i = tid; i < n2; i += kFinThreads) {
            if (i < V) {
                sh.u.sort.key[i] = make_key(ld_coherent(a.vscore + i), uint32_t(ld_coherent(a.vlist + i)));
                sh.u.sort.pay[i] = uint16_t(i);
            } else {
                sh.u.sort.key[i] = kEmptyKey;
                sh.u.sort.pay[i] = 0;
            }
        }
        __syncthreads();
        block_bitonic(sh.u.sort.key, sh.u.sort.pay, n2);
        for (int j = tid; j < rc; j += kFinThreads)
            write_result(a, j, sh.u.sort.key[j], ld_coherent(a.vhop + sh.u.sort.pay[j]));
        return;
    }
    // Keys are unique. Results go out in bands of at most kSortCap ranks: radix-select
    // the key of the band's last rank, gather the band's keys (above the previous
    // band's last key, at most this one), sort them in LDS and write them. Up to
    // kResultCap results take ceil(rc / kSortCap) bands.
    uint64_t lo_key = 0;
    for (int done = 0; done < rc;) {
        const int band = min(kSortCap, rc - done);
        const uint64_t hi_key = radix_select_key(sh, a, V, done + band);
        int base = 0;
        for (int r0 = 0; r0 < V; r0 += kFinThreads) {
            const int i = r0 + tid;
            uint64_t key = kEmptyKey;
            bool take = false;
            if (i < V) {
                key = make_key(ld_coherent(a.vscore + i), uint32_t(ld_coherent(a.vlist + i)));
                take = key <= hi_key && (done == 0 || key > lo_key);
            }
            int tot = 0;
            const int o = block_excl_scan(take ? 1 : 0, sh.s_wave, &tot);
            if (take) { a.sortbuf[2 * (base + o)] = key; a.sortbuf[2 * (base + o) + 1] = uint64_t(i); }
            base += tot;
        }
        __threadfence();
        __syncthreads();
        int n2 = 1;
        while (n2 < band) n2 <<= 1;
        for (int i = tid; i < n2; i += kFinThreads) {
            sh.u.sort.key[i] = (i < band) ? ld_coherent(a.sortbuf + 2 * i) : kEmptyKey;
            sh.u.sort.pay[i] = uint16_t(i < band ? i : 0);
        }
        __syncthreads();
        block_bitonic(sh.u.sort.key, sh.u.sort.pay, n2);
        for (int j = tid; j < band; j += kFinThreads) {
            const int pos = int(ld_coherent(a.sortbuf + 2 * sh.u.sort.pay[j] + 1));
            write_result(a, done + j, sh.u.sort.key[j], ld_coherent(a.vhop + pos));
        }
        __syncthreads();                        // LDS and sortbuf are reused by the next band
        done += band;
        lo_key = hi_key;
    }
}

// Merge the lists of waves [0, active) pairwise in LDS (waves >= active hold
// empty lists); wave 0 returns the result. `active` is block-uniform.
__device__ inline uint64_t tree_merge(FinShared& sh, uint64_t list, int k, int active = kFinWaves) {
    const int lane = lane_id(), wave = int(threadIdx.x >> 6);
    int span = 1;
    while (span < active) span <<= 1;
    for (int half = span / 2; half > 0; half >>= 1) {
        if (wave >= half && wave < 2 * half) sh.lists[wave][lane] = list;
        __syncthreads();
        if (wave < half) list = wave_merge64(list, sh.lists[wave + half][lane], lane, k);
        __syncthreads();
    }
    return list;
}

// Phase stamps (GPU realtime counter) are kept in LDS by thread 0 and stored once, at the
// end: a store to the host-mapped stamp words takes a PCIe round trip to complete, and every
// later load of the storing wave waits for it (stores and loads share one counter here).
__device__ inline void flush_stamps(const uint64_t* st, int n, uint64_t* out) {
    if (threadIdx.x == 0 && out)
        for (int i = 0; i < n; ++i) out[i] = st[i];
}

__global__ __launch_bounds__(kFinThreads) void k_finalize(FinalizeArgs a) {
    __shared__ FinShared sh;
    __shared__ uint64_t s_st[4];
    const int tid = int(threadIdx.x), lane = lane_id(), wave = tid >> 6;
    const int k = a.k;
    auto stamp = [&](const FinalizeArgs&, int i) {
        if (tid == 0) s_st[i] = __builtin_amdgcn_s_memrealtime();
    };
    stamp(a, 0);

    // ---- A. merge the scan's candidate keys into the K seeds (8 loads in flight per lane)
    // the count and the first 8192 keys are loaded together; slots past the count
    // (left from earlier queries) are masked afterwards
    uint64_t list = kEmptyKey, thr = kEmptyKey;
    const int n_part = int(*a.gcnt);
    // Every key of the K best is <= the scan's final bound (the smallest workgroup K-th
    // key), so keys above it are dropped as they load and never reach the lists.
    const uint64_t gb = *a.gthr;
    {
        uint64_t x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = a.part[wave * 64 + j * kFinThreads + lane];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            wave_offer(list, thr, (wave * 64 + j * kFinThreads + lane < n_part && x[j] <= gb) ? x[j] : kEmptyKey,
                       lane, k);
    }
    for (int base = kFinThreads * 8 + wave * 64; base < n_part; base += kFinThreads * 8) {
        uint64_t x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = base + j * kFinThreads + lane;
            x[j] = (i < n_part) ? a.part[i] : kEmptyKey;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) wave_offer(list, thr, x[j] <= gb ? x[j] : kEmptyKey, lane, k);
    }
    list = tree_merge(sh, list, k, n_part <= kFinThreads ? (n_part + 63) / 64 : kFinWaves);
    if (wave == 0) {
        const int ns = __popcll(__ballot(lane < k && list != kEmptyKey));
        if (lane < ns) {
            const int32_t id = key_id(list);
            const float sc = key_score(list);
            a.seed_idx[lane] = id;
            a.seed_val[lane] = sc;
            a.vlist[lane] = id;
            a.vhop[lane] = 0;
            a.vscore[lane] = sc;
            a.vro[lane] = sh.ro_cache[lane] = a.ro[id];
            sh.seed_id[lane] = id;
        }
        if (lane == 0) sh.s_misc[0] = ns;
    }
    __threadfence_block();        // one workgroup: readers use L2-coherent loads
    __syncthreads();
    const int ns = sh.s_misc[0];
    stamp(a, 1);

    // ---- B. deterministic BFS: LDS hash first, global arrays if it outgrows it
    const int rk = a.rcap <= 64 ? a.rcap : 0;       // results tracked during the BFS
    uint64_t best = (wave == 0 && lane < rk) ? list : kEmptyKey;
    uint64_t bthr = rk > 0 ? __shfl(best, rk - 1) : kEmptyKey;
    int levels = 0;
    int V = (a.hops < int(kClaimHop)) ? bfs_lds<kBfsScored>(sh, a, ns, &levels, best, bthr, rk) : -1;   // hop below the claim mark
    const bool in_lds = V >= 0;
    if (!in_lds) {
        __syncthreads();
        V = bfs_global(sh, a, ns, &levels);
    }

    stamp(a, 2);
    // ---- C. results: (score desc, id asc), first rcap
    const int rc = min(a.rcap, V);
    if (in_lds && rk > 0) {
        // each wave's best emitted keys, merged; hop looked up in the LDS hash
        best = tree_merge(sh, best, rk);
        if (wave == 0) {
            if (lane < rc) {
                const int slot = hash_find(sh, key_id(best));
                write_result(a, lane, best, int32_t(sh.u.bfs.hval[slot] >> 16));
            }
        }
    } else {
        __syncthreads();
        select_sorted(sh, a, V, rc);
    }
    if (tid == 0) {
        ResultHeader h;
        h.count = rc;
        h.visited = V;
        h.levels = levels;
        h.n_seeds = ns;
        *a.res = h;
        *a.gcnt = 0u;                 // ready for the next query's scan
        *a.gthr = kEmptyKey;
    }
    stamp(a, 3);
    flush_stamps(s_st, 4, a.stamps);
    signal_done(a.done, a.seq);
}

// ---- episode-scoped query ------------------------------------------------------------
// ---- batched global queries: one workgroup per query ------------------------------
// The view of query j's visit slots as the finalize helpers take them.
__device__ inline FinalizeArgs multi_view(const MultiArgs& m, int j) {
    FinalizeArgs a{};
    const int64_t base = int64_t(j) * kMultiVisit;
    a.k = m.k; a.ro = m.ro; a.col = m.col; a.n_live = m.n_live; a.mods = m.mods; a.hops = m.hops;
    a.hop_decay = m.hop_decay; a.rcap = m.rcap; a.cap_visit = kMultiVisit;
    a.vlist = m.vlist + base; a.vhop = m.vhop + base; a.vpar = m.vpar + base; a.vro = m.vro + base;
    a.vscore = m.vscore + base; a.rec = m.rec + int64_t(j) * m.rcap;
    return a;
}

// Visit set, hops and parents of query j from its certified seeds: the unscored LDS
// BFS of k_finalize (same claims, same order). A visit set that outgrows the LDS hash
// marks the query kMultiOverflow (the Q=1 path answers it).
// Returns the visit count (-1: the visit set outgrew the LDS hash), block-uniform.
__device__ int multi_bfs_query(FinShared& sh, const MultiArgs& m, int j, int* levels_out = nullptr,
                               int* ns_out = nullptr) {
    const FinalizeArgs a = multi_view(m, j);
    const int tid = int(threadIdx.x), lane = lane_id(), wave = tid >> 6;
    if (wave == 0) {
        const uint64_t key = lane < m.k ? m.seeds[int64_t(j) * m.seed_stride + lane] : kEmptyKey;
        const int ns = __popcll(__ballot(key != kEmptyKey));
        if (key != kEmptyKey) {
            const int32_t id = key_id(key);
            a.vlist[lane] = id;
            a.vhop[lane] = 0;
            a.vpar[lane] = -1;
            a.vscore[lane] = key_score(key);
            a.vro[lane] = sh.ro_cache[lane] = a.ro[id];
            sh.seed_id[lane] = id;
        }
        if (lane == 0) sh.s_misc[0] = ns;
    }
    __threadfence_block();
    __syncthreads();
    const int ns = sh.s_misc[0];
    int levels = 0;
    uint64_t best = kEmptyKey, bthr = kEmptyKey;
    const int V = (a.hops < int(kClaimHop)) ? bfs_lds<kBfsUnscored>(sh, a, ns, &levels, best, bthr, 0) : -1;
    if (tid == 0) {
        if (V < 0) {
            m.status[j] = kMultiOverflow;
        } else {
            m.info[4 * j] = V;
            m.info[4 * j + 1] = levels;
            m.info[4 * j + 2] = ns;
        }
    }
    if (levels_out) *levels_out = levels;
    if (ns_out) *ns_out = ns;
    return V;
}

__global__ __launch_bounds__(kFinThreads) void k_multi_bfs(MultiArgs m) {
    __shared__ FinShared sh;
    const int j = int(blockIdx.x);
    if (m.status[j] != kMultiOk) return;                  // block-uniform
    multi_bfs_query(sh, m, j);
}

// Scores of query j's visit set, level by level in the finalize kernel's arithmetic
// (score = max(parent score * hop_decay, fin * 0.8), seeds keep their exact score),
// then the first rcap by (score desc, id asc) into the host-mapped results. Every
// query writes its header; count -1 marks one the Q=1 path must answer.
__global__ __launch_bounds__(kFinThreads) void k_multi_select(MultiArgs m) {
    __shared__ FinShared sh;
    const int j = int(blockIdx.x);
    const int st = m.status[j];
    if (st != kMultiOk) {
        if (threadIdx.x == 0) {
            ResultHeader h;
            h.count = -1; h.visited = st; h.levels = 0; h.n_seeds = 0;
            m.res[j] = h;
        }
        signal_done(m.done, m.seq);
        return;
    }
    const FinalizeArgs a = multi_view(m, j);
    const int tid = int(threadIdx.x);
    const int V = m.info[4 * j], levels = m.info[4 * j + 1], ns = m.info[4 * j + 2];
    const float* vfin = m.vfin + int64_t(j) * kMultiVisit;
    for (int h = 1; h <= levels; ++h) {
        for (int p = ns + tid; p < V; p += kFinThreads) {
            if (a.vhop[p] == h)
                a.vscore[p] = fmaxf(ld_coherent(a.vscore + a.vpar[p]) * a.hop_decay, vfin[p] * 0.8f);
        }
        __threadfence_block();
        __syncthreads();
    }
    const int rc = min(a.rcap, V);
    if (a.rcap <= 64) {
        // the rc best (score, id) keys from per-wave lists, then each result's hop from
        // the one visit position that holds its node
        __shared__ uint64_t s_res[64];
        __shared__ int32_t s_hop[64];
        const int lane = lane_id(), wave = tid >> 6;
        uint64_t best = kEmptyKey, bthr = kEmptyKey;
        for (int p0 = wave * 64; p0 < V; p0 += kFinThreads) {
            const int p = p0 + lane;
            wave_offer(best, bthr, p < V ? make_key(ld_coherent(a.vscore + p), uint32_t(a.vlist[p])) : kEmptyKey,
                       lane, rc);
        }
        best = tree_merge(sh, best, rc);
        if (wave == 0) s_res[lane] = best;
        __syncthreads();
        for (int p = tid; p < V; p += kFinThreads) {
            const int32_t id = a.vlist[p];
            for (int r = 0; r < rc; ++r)
                if (key_id(s_res[r]) == id) s_hop[r] = a.vhop[p];
        }
        __syncthreads();
        if (tid < rc) write_result(a, tid, s_res[tid], s_hop[tid]);
    } else {
        select_sorted(sh, a, V, rc);
    }
    if (tid == 0) {
        ResultHeader h;
        h.count = rc; h.visited = V; h.levels = levels; h.n_seeds = ns;
        m.res[j] = h;
    }
    signal_done(m.done, m.seq);
}

// The c (<= 64) best keys of nl (<= kScan8MaxLists) ascending lists of kScan8List (16)
// keys at part, one per int8 scan workgroup; wave 0 returns them (lane i: the i-th
// smallest). The lists are read as 1 KB blocks of 8, one block per wave load instruction
// (lane l: keys 2l, 2l + 1 of the block, i.e. keys 2 (l & 7), +1 of list 8b + l / 8), wave w
// taking blocks w, w + 16, ...
// cut = the c-th smallest of the lists' first keys: c lists hold a key <= cut, so the c
// best keys are <= cut, and only those c lists hold keys <= cut: at most c * 16 keys
// (with cut = kEmptyKey, fewer than c lists hold any), compacted into LDS, one per
// thread for the final selection. s_lmin = the smallest 16th key: a row that a full list
// dropped has a key above it (the certificate's bound takes it into account).
__device__ uint64_t merge_lists8(FinShared& sh, const uint64_t* part, int nl, int c, uint64_t& s_lmin,
                                 uint64_t& s_cut) {
    const int tid = int(threadIdx.x), lane = lane_id(), wave = tid >> 6;
    static_assert(kScan8List == 16 && kScan8MaxLists <= 8 * 4 * kFinWaves, "block layout");
    static_assert(kScan8MaxLists + 64 * kScan8List <= kSortCap && 64 * kScan8List <= kFinThreads, "buffers");
    uint64_t x[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int b = wave + i * kFinWaves;
        const bool on = 8 * b + (lane >> 3) < nl;
        const u64x2 v = on ? reinterpret_cast<const u64x2*>(part + int64_t(b) * 128)[lane]
                           : u64x2{kEmptyKey, kEmptyKey};
        x[2 * i] = v.x;
        x[2 * i + 1] = v.y;
    }
    uint64_t* k1 = sh.u.sort.key;                    // the lists' first keys
    uint64_t* buf = sh.u.sort.key + kScan8MaxLists;  // the keys <= cut
    uint64_t l16 = kEmptyKey;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int li = 8 * (wave + i * kFinWaves) + (lane >> 3);
        if ((lane & 7) == 0) k1[li] = li < nl ? x[2 * i] : kEmptyKey;
        if ((lane & 7) == 7 && x[2 * i + 1] < l16) l16 = x[2 * i + 1];
    }
    {
        uint64_t y = xor_lane64<32>(l16); l16 = y < l16 ? y : l16;
        y = xor_lane64<16>(l16); l16 = y < l16 ? y : l16;
        y = xor_lane64<8>(l16); l16 = y < l16 ? y : l16;
        y = xor_lane64<4>(l16); l16 = y < l16 ? y : l16;
        y = xor_lane64<2>(l16); l16 = y < l16 ? y : l16;
        y = xor_lane64<1>(l16); l16 = y < l16 ? y : l16;
    }
    if (tid == 0) { s_lmin = kEmptyKey; sh.s_misc[4] = 0; }
    __syncthreads();
    if (lane == 0) atomicMin(reinterpret_cast<unsigned long long*>(&s_lmin), (unsigned long long)l16);
    uint64_t l1 = kEmptyKey, t1 = kEmptyKey;
    wave_offer(l1, t1, tid < nl ? k1[tid] : kEmptyKey, lane, c);
    l1 = tree_merge(sh, l1, c, (nl + 63) / 64);
    if (wave == 0 && lane == c - 1) s_cut = l1;
    __syncthreads();
    const uint64_t cut = s_cut;
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) cnt += (x[j] <= cut && x[j] != kEmptyKey) ? 1 : 0;
    int at = cnt ? atomicAdd(&sh.s_misc[4], cnt) : 0;
#pragma unroll
    for (int j = 0; j < 8; ++j)
        if (x[j] <= cut && x[j] != kEmptyKey) buf[at++] = x[j];
    __syncthreads();
    const int m = sh.s_misc[4];                      // <= 64 * 16 = kFinThreads
    uint64_t list = kEmptyKey, thr = kEmptyKey;
    wave_offer(list, thr, tid < m ? buf[tid] : kEmptyKey, lane, c);
    return tree_merge(sh, list, c, (m + 63) / 64);
}

// ---- certified Q=1 global query ---------------------------------------------------------
// The candidate scan kept its c best keys per workgroup in part. Here they are merged to
// the c best overall, rescored in the fp32 scan's arithmetic (QF32 dot, 16-lane
// reduction, fuse_score), and the k best exact keys are certified.
//  * fp16 scan (rows e16, query q in fp32): a row outside the candidates has fp16 score
//    <= the c-th candidate's, and
//      |fp16 score - fp32 score| <= |e16 - e|max |q| + g (|e16|max + |e|max) |q| + rounding
//    (g = (d/16 + 4) u, both scans' per-lane chains and reductions; weights <= 1), so a
//    k-th exact score above (c-th fp16 score + that bound) makes the seeds the fp32 scan's.
//  * int8 scan (upper = 1): the keys are per-row upper bounds of the fp32 scan's score,
//    so a k-th exact score above the c-th candidate's key score is the certificate.
template <typename QF>
__global__ __launch_bounds__(kFinThreads) void k_cert_bfs(CertArgs a, MultiArgs m) {
    __shared__ FinShared sh;
    __shared__ uint64_t s_cand[64];
    __shared__ uint64_t s_exact[64];
    __shared__ double s_qn;
    __shared__ double s_eps;
    __shared__ uint64_t s_cut;
    __shared__ uint64_t s_lmin;
    __shared__ uint64_t s_st[7];
    const int tid = int(threadIdx.x), lane = lane_id(), wave = tid >> 6;
    const int c = a.c;
    auto stamp_at = [&](int i) {
        if (tid == 0) s_st[i] = __builtin_amdgcn_s_memrealtime();
    };
    stamp_at(0);
    uint64_t list = kEmptyKey, thr = kEmptyKey;
    if (a.n_lists > 0) {
        // A. the c (<= 64) best keys of the scan workgroups' lists
        list = merge_lists8(sh, a.part, a.n_lists, c, s_lmin, s_cut);
    } else {
        // A. the c best candidate keys (the finalize kernel's merge, 8 loads in flight per lane)
        const int n_part = int(*a.gcnt);
        const uint64_t gb = *a.gthr;             // the scan's final bound: the c best are <= it
        for (int base = wave * 64; base < n_part; base += kFinThreads * 8) {
            uint64_t x[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = base + j * kFinThreads + lane;
                x[j] = (i < n_part && a.part[i] <= gb) ? a.part[i] : kEmptyKey;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) wave_offer(list, thr, x[j], lane, c);
        }
        list = tree_merge(sh, list, c, n_part <= kFinThreads ? (n_part + 63) / 64 : kFinWaves);
    }
    stamp_at(1);
    // the query in the rescoring layout (every 16-lane group holds all of it); group 0 also
    // takes |q| (fp64) from its registers
    const int g = tid >> 4, sub = tid & 15;
    QF qf;
    qf.load(a.q, sub);
    if (wave == 0) s_cand[lane] = list;
    if (g == 0) {
        const double sq = row16_sum_f64(qf.norm2());
        if (sub == 0) s_qn = sqrt(sq);
    }
    __syncthreads();
    // B. exact rescoring: 16-lane group g takes candidate g
    const uint64_t ck = s_cand[g];
    uint64_t key = kEmptyKey;
    if (ck != kEmptyKey) {                       // uniform over the group
        const int32_t id = key_id(ck);
        const float dot = qf.dot(a.emb + int64_t(id) * a.d, sub);
        const QueryTerms t{a.t_q, a.lambda, a.mod_filter, -1, 0.0f};
        const float sc = fuse_score(row16_sum(dot), a.ts[id], (a.mod_filter >= 0) ? a.mods[id] : 0, -1, t);
        key = make_key(sc, uint32_t(id));
    }
    if (sub == 0) s_exact[g] = key;
    __syncthreads();
    if (wave == 0) {
    // C. the k best exact keys and the certificate
    const uint64_t x = wave_sort64(s_exact[lane], lane);
    const uint64_t cl = s_cand[lane];
    const uint64_t c_last = __shfl(cl, c - 1);
    const int kk = a.k < c ? a.k : c;
    const uint64_t kth = __shfl(x, kk - 1);
    bool ok = false;
    float margin = __builtin_inff();
    const double qn = s_qn, u = 0x1p-24;
    // eps: bound on |scan score - exact score| of any row (the interval BFS's half-width);
    // slack: what the certificate adds to the c-th candidate's key score; en: row norm bound
    double eps, slack, en;
    if (a.upper) {
        // int8 scan: keys are per-row upper bounds of the exact score (no slack), the
        // estimates in fin lie within |q| max c_r + tau plus the two products' rounding
        const double cm = double(__uint_as_float(a.nrm8[0]));
        en = double(__uint_as_float(a.nrm8[1]));
        // plus the scan's per-query term (query split remainder and roundings)
        const double tau = double(__uint_as_float(uint32_t(a.part[int64_t(kScan8MaxLists) * kScan8List])));
        eps = (cm * qn + 4.0 * u * (en + cm) * qn) * 1.01 + tau + 1e-30 * double(a.d);
        slack = 0.0;
    } else {
        const double e32 = double(__uint_as_float(a.nrm[0]));
        const double e16 = double(__uint_as_float(a.nrm[1]));
        const double de = double(__uint_as_float(a.nrm[2]));
        const double nq = double(a.d) / 16.0 + 4.0;
        const double gs = nq * u / (1.0 - nq * u);
        eps = (de * qn + gs * (e16 + e32) * qn + u * (e16 + e32) * qn * (1.0 + gs)) * 1.01 + 1e-30 * double(a.d);
        slack = eps;
        en = e16;
    }
    if (lane == 0) s_eps = eps;
    // every row outside the candidates has a key above bnd: the c-th candidate's (none when
    // fewer than c), and with per-workgroup lists the smallest last key of a full list
    const uint64_t bnd = (a.n_lists > 0 && s_lmin < c_last) ? s_lmin : c_last;
    if (a.k <= c) {
        if (bnd == kEmptyKey) {
            ok = true;                           // every live row was a candidate
        } else {
            const float s16 = key_score(bnd), s32 = key_score(kth);
            if (eps < 1e30) {                    // also false for NaN bounds
                if (s16 == -FLT_MAX) {
                    ok = en * qn * 2.0 < double(FLT_MAX);     // the c-th candidate is filtered
                } else {
                    const double mg = double(s32) - (double(s16) + slack);
                    ok = mg > 0.0;
                    margin = float(mg);
                }
            } else {
                margin = -__builtin_inff();
            }
        }
    }
    a.seeds[lane] = (ok && lane < kk) ? x : kEmptyKey;
    if (lane == 0) {
        *a.status = ok ? kMultiOk : kMultiUncertified;
        *a.margin = margin;
        *a.gcnt = 0u;                            // the scan's count and bound, for the next query
        *a.gthr = kEmptyKey;
        sh.s_misc[6] = ok ? 1 : 0;
    }
    }
    __threadfence_block();
    __syncthreads();
    // D. the certified seeds' BFS (visit set, hops, parents) in the same workgroup
    if (!a.finish) {
        flush_stamps(s_st, 2, a.stamps);
        if (sh.s_misc[6]) multi_bfs_query(sh, m, 0);
        return;
    }
    int n_st = 2;                                // stamps taken so far
    auto fail = [&](int32_t code) {
        if (tid == 0) {
            ResultHeader h;
            h.count = -1; h.visited = code; h.levels = 0; h.n_seeds = 0;
            m.res[0] = h;
        }
        flush_stamps(s_st, n_st, a.stamps);
        signal_done(a.done, a.seq);
    };
    stamp_at(2);
    n_st = 3;
    if (!sh.s_misc[6]) { fail(kMultiUncertified); return; }
    // E. the certified seeds' BFS in interval mode: every node's BFS score from the fp16
    // scan's fused scores (each within eps of the exact one) and a bound on its distance
    // to the exact BFS score. At least rc nodes have exact scores >= the rc-th largest
    // lower end, so a node whose upper end is below it cannot be a result; the others
    // (with their BFS ancestors) are rescored exactly and propagated in the finalize
    // kernel's arithmetic.
    FinalizeArgs v = multi_view(m, 0);
    v.fin = a.fin16;
    v.vdv = m.vfin;                              // bounds; later the exact fused scores
    v.eps = s_eps;
    v.mod_filter = a.mod_filter;
    const float dlt = m.hop_decay;               // in [0, 1] (checked by the caller)
    const int rk = m.rcap;                       // <= 64 (checked by the caller)
    uint64_t seedkey = kEmptyKey;
    if (wave == 0) {
        seedkey = lane < m.k ? a.seeds[lane] : kEmptyKey;
        const int nsd = __popcll(__ballot(seedkey != kEmptyKey));
        if (seedkey != kEmptyKey) {
            const int32_t id = key_id(seedkey);
            v.vlist[lane] = id;
            v.vhop[lane] = 0;
            v.vpar[lane] = -1;
            v.vscore[lane] = key_score(seedkey);
            v.vdv[lane] = 0.0f;
            v.vro[lane] = sh.ro_cache[lane] = v.ro[id];
            sh.seed_id[lane] = id;
        }
        if (lane == 0) { sh.s_misc[0] = nsd; sh.s_misc[7] = 0; }
    }
    __threadfence_block();
    __syncthreads();
    const int ns = sh.s_misc[0];
    int levels = 0;
    uint64_t best = (wave == 0 && lane < rk) ? seedkey : kEmptyKey;   // seeds: exact lower ends
    uint64_t bthr = __shfl(best, rk - 1);
    const int V = (v.hops < int(kClaimHop)) ? bfs_lds<kBfsInterval>(sh, v, ns, &levels, best, bthr, rk) : -1;
    if (V < 0) { fail(kMultiOverflow); return; }
    if (sh.s_misc[7]) { fail(kMultiUncertified); return; }
    stamp_at(3);
    n_st = 4;
    const int rc = min(m.rcap, V);
    best = tree_merge(sh, best, rk);
    if (wave == 0 && lane == rc - 1) sh.s_misc[5] = int(__float_as_uint(key_score(best)));
    __syncthreads();
    const double cut = double(__uint_as_float(uint32_t(sh.s_misc[5])));
    // positions p = tid + j kFinThreads (V <= kMultiVisit): each thread's visit data is
    // loaded once; parents and exact BFS scores live by position in the freed frontier arrays
    // (rstart + eoff: kMultiVisit words), marks and the marked list in the freed hash
    constexpr int kPer = kMultiVisit / kFinThreads;
    static_assert(kHashLimit + kFinThreads <= kMultiVisit && kMultiVisit <= 2 * kFrontierChunk + 1, "positions");
    float* dv = reinterpret_cast<float*>(&sh.u.bfs.rstart[0]);      // exact BFS scores by position
    int32_t* par_l = &sh.u.bfs.rstart[0];                            // parents by position (until dv)
    uint32_t* flag = sh.u.bfs.hkey;
    int32_t* rlist = reinterpret_cast<int32_t*>(sh.u.bfs.hval);
    // mark the candidates and their ancestors
    bool mk[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int p = tid + j * kFinThreads;
        mk[j] = false;
        if (p < V) {
            mk[j] = double(ld_coherent(v.vscore + p)) + double(ld_coherent(v.vdv + p)) >= cut;
            par_l[p] = ld_coherent(v.vpar + p);
            flag[p] = 0u;
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kPer; ++j)
        if (mk[j])
            for (int x = tid + j * kFinThreads; x >= 0; x = par_l[x]) flag[x] = 1u;
    __syncthreads();
    // compact the marked positions (ascending)
    int r = 0;
    for (int p0 = 0; p0 < V; p0 += kFinThreads) {
        const int p = p0 + tid;
        const int on = (p < V && flag[p]) ? 1 : 0;
        int tot = 0;
        const int o = block_excl_scan(on, sh.s_wave, &tot);
        if (on) rlist[r + o] = p;
        r += tot;
    }
    __syncthreads();
    stamp_at(4);
    // exact fused scores of the marked nodes past the seeds (one per 16-lane group)
    {
        QF qf;
        qf.load(a.q, sub);
        const QueryTerms t{a.t_q, a.lambda, a.mod_filter, -1, 0.0f};
        for (int i = g; i < r; i += kFinThreads / 16) {
            const int p = rlist[i];
            if (p < ns) continue;                // uniform over the group
            const int32_t id = ld_coherent(v.vlist + p);
            const float dot = qf.dot(a.emb + int64_t(id) * a.d, sub);
            const float sc = fuse_score(row16_sum(dot), a.ts[id], (a.mod_filter >= 0) ? a.mods[id] : 0, -1, t);
            if (sub == 0) m.vfin[p] = sc;
        }
    }
    __threadfence_block();
    __syncthreads();
    stamp_at(5);
    // the marked nodes (i = tid + j kFinThreads < r): position, hop, parent, id and the score
    // their exact BFS score starts from, loaded once
    int32_t mp[kPer], mh[kPer], mpar[kPer], mid[kPer];
    float mval[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int i = tid + j * kFinThreads;
        mh[j] = -1; mp[j] = 0; mpar[j] = -1; mid[j] = 0; mval[j] = 0.0f;
        if (i < r) {
            const int p = rlist[i];
            mp[j] = p;
            mh[j] = ld_coherent(v.vhop + p);
            mpar[j] = par_l[p];
            mid[j] = ld_coherent(v.vlist + p);
            mval[j] = p < ns ? ld_coherent(v.vscore + p) : ld_coherent(m.vfin + p);
        }
    }
    __syncthreads();                                                 // par_l read: dv may overwrite it
    // exact BFS scores over the marked set, level by level (parents are marked too)
    for (int h = 0; h <= levels; ++h) {
#pragma unroll
        for (int j = 0; j < kPer; ++j)
            if (mh[j] == h) dv[mp[j]] = (h == 0) ? mval[j] : fmaxf(dv[mpar[j]] * dlt, mval[j] * 0.8f);
        __syncthreads();
    }
    // the rc best exact keys among the marked nodes, and their hops
    best = kEmptyKey;
    bthr = kEmptyKey;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        if (j * kFinThreads + wave * 64 >= r) break;                 // uniform over the wave
        wave_offer(best, bthr, mh[j] >= 0 ? make_key(dv[mp[j]], uint32_t(mid[j])) : kEmptyKey, lane, rc);
    }
    best = tree_merge(sh, best, rc);
    // each result's hop from the one marked position that holds its node
    if (wave == 0) s_exact[lane] = best;
    __syncthreads();
    int32_t* s_hop = reinterpret_cast<int32_t*>(sh.lists[1]);        // free after the merge
#pragma unroll
    for (int j = 0; j < kPer; ++j)
        if (mh[j] >= 0)
            for (int x = 0; x < rc; ++x)
                if (key_id(s_exact[x]) == mid[j]) s_hop[x] = mh[j];
    __syncthreads();
    if (wave == 0 && lane < rc) write_result(v, lane, best, s_hop[lane]);
    if (tid == 0) {
        ResultHeader h;
        h.count = rc; h.visited = V; h.levels = levels; h.n_seeds = ns;
        m.res[0] = h;
    }
    stamp_at(6);
    flush_stamps(s_st, 7, a.stamps);
    signal_done(a.done, a.seq);
}

// ---- certified seeds of up to 16 queries after k_scan8m -----------------------------
// One workgroup per query j: the 64 best upper-bound keys of its scan lists (merge_lists8),
// rescored exactly (QF32 dot and 16-lane reduction as the fp32 scan; global queries then
// fuse_score with their time and the modality filter, plain queries keep the dot) and
// sorted; the K best are certified when the K-th exact key's score beats the score of the
// smallest key any row outside the candidates can hold (k_cert_bfs's int8 argument). A
// global query's seeds go to seeds[64 j ..] (ascending keys, kEmptyKey padded); a plain
// query's K = knn_k neighbour ids to knn_out[knn_k (j - n_glob) ..].
template <typename QF>
__global__ __launch_bounds__(kFinThreads) void k_cert_multi8(CertMArgs a) {
    __shared__ FinShared sh;
    __shared__ uint64_t s_cand[64];
    __shared__ uint64_t s_exact[64];
    __shared__ uint64_t s_lmin;
    __shared__ uint64_t s_cut;
    const int j = int(blockIdx.x);
    const int tid = int(threadIdx.x), lane = lane_id(), wave = tid >> 6, g = tid >> 4, sub = tid & 15;
    const bool plain = j >= a.n_glob;
    constexpr int c = 64;
    const uint64_t list = merge_lists8(sh, a.part + int64_t(j) * kScan8MPart, a.n_lists, c, s_lmin, s_cut);
    const float* q = plain ? a.q_plain + int64_t(j - a.n_glob) * a.d : a.q_glob + int64_t(j) * a.d;
    QF qf;
    qf.load(q, sub);
    if (wave == 0) s_cand[lane] = list;
    __syncthreads();
    const uint64_t ck = s_cand[g];
    uint64_t key = kEmptyKey;
    if (ck != kEmptyKey) {                       // uniform over the group
        const int32_t id = key_id(ck);
        const float dot = row16_sum(qf.dot(a.emb + int64_t(id) * a.d, sub));
        float sc = dot;
        if (!plain) {
            const QueryTerms t{a.tq ? a.tq[j] : a.tq_value, a.lambda, a.mod_filter, -1, 0.0f};
            sc = fuse_score(dot, a.ts[id], (a.mod_filter >= 0) ? a.mods[id] : 0, -1, t);
        }
        key = make_key(sc, uint32_t(id));
    }
    if (sub == 0) s_exact[g] = key;
    __syncthreads();
    if (wave != 0) return;
    const uint64_t x = wave_sort64(s_exact[lane], lane);
    const uint64_t c_last = __shfl(s_cand[lane], c - 1);
    const int K = plain ? a.knn_k : a.k;
    const int kk = K < c ? K : c;
    const uint64_t kth = __shfl(x, kk - 1);
    bool ok = false;
    float margin = __builtin_inff();
    // the bounds must be finite: the row bound maxima and this query's terms
    const double u = 0x1p-24;
    const double cm = double(__uint_as_float(a.nrm8[0])), en = double(__uint_as_float(a.nrm8[1]));
    const double qn = double(a.qp[4 * j + 3]), tau = double(a.qp[4 * j + 2]);
    const double eps = (cm * qn + 4.0 * u * (en + cm) * qn) * 1.01 + tau + 1e-30 * double(a.d);
    const uint64_t bnd = s_lmin < c_last ? s_lmin : c_last;
    if (K <= c) {
        if (bnd == kEmptyKey) {
            ok = true;                           // every row with a key was a candidate
        } else if (eps < 1e30) {                 // also false for NaN bounds
            const float s8 = key_score(bnd), s32 = key_score(kth);
            if (s8 == -FLT_MAX) {
                ok = en * qn * 2.0 < double(FLT_MAX);       // the bound key is a filtered row
            } else {
                const double mg = double(s32) - double(s8);
                ok = mg > 0.0;
                margin = float(mg);
            }
        } else {
            margin = -__builtin_inff();
        }
    }
    if (plain) {
        if (lane < kk) a.knn_out[int64_t(j - a.n_glob) * a.knn_k + lane] = (ok && x != kEmptyKey) ? key_id(x) : -1;
    } else {
        a.seeds[int64_t(j) * 64 + lane] = (ok && lane < kk) ? x : kEmptyKey;
    }
    if (lane == 0) {
        a.status[j] = ok ? kMultiOk : kMultiUncertified;
        a.margin[j] = margin;
    }
}

// NCH > 0 (d = 64 NCH, NCH <= 12): a member row's NCH 16-byte loads are all issued
// before its first FMA, and the query is read from LDS chunk by chunk (the same floats
// in the same fmaf order as the loop below, so the same scores). At most 64 VGPRs, so
// the kernel still fits on a CU beside a batched scan's workgroup.
template <int NCH>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(8))) void k_episode(EpisodeArgs a) {
    // latency-bound and short: its waves go first when they share a CU with a scan
    __builtin_amdgcn_s_setprio(3);
    __shared__ uint64_t s_lists[4][64];
    __shared__ int32_t s_ids[64];
    __shared__ uint64_t s_out[64];
    __shared__ int s_cnt[2];
    __shared__ f32x4 s_q[NCH > 0 ? NCH * 16 : 1];     // float4 i = floats 4i .. 4i+3
    const int lane = lane_id(), wave = int(threadIdx.x >> 6);
    const int sub = lane & 15, grp = lane >> 4;
    const int k = a.k;
    uint64_t list = kEmptyKey, thr = kEmptyKey;
    if constexpr (NCH > 0) {
        for (int i = int(threadIdx.x); i < NCH * 16; i += 256) s_q[i] = reinterpret_cast<const f32x4*>(a.q)[i];
        __syncthreads();
    }
    for (int base = 4 * wave; base < a.m; base += 16) {
        const int j = base + grp;
        const bool valid = j < a.m;
        const int32_t node = a.members[valid ? j : a.m - 1];
        float acc = 0.0f;
        const float* row = a.emb + int64_t(node) * a.d;
        if constexpr (NCH > 0) {
            const f32x4* r4 = reinterpret_cast<const f32x4*>(row) + sub;
            f32x4 x[NCH];
#pragma unroll
            for (int c = 0; c < NCH; ++c) x[c] = __builtin_nontemporal_load(r4 + c * 16);
            __builtin_amdgcn_sched_barrier(0);     // every load of the row before any FMA
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const f32x4 y = s_q[c * 16 + sub];
                acc = fmaf(x[c].x, y.x, acc); acc = fmaf(x[c].y, y.y, acc);
                acc = fmaf(x[c].z, y.z, acc); acc = fmaf(x[c].w, y.w, acc);
                if (c % 3 == 2) __builtin_amdgcn_sched_barrier(0);   // a few LDS reads in flight
            }
        } else if ((a.d & 3) == 0) {
            const float4* r4 = reinterpret_cast<const float4*>(row);
            const float4* q4 = reinterpret_cast<const float4*>(a.q);
            for (int i = sub; i < (a.d >> 2); i += 16) {
                const float4 x = r4[i], y = q4[i];
                acc = fmaf(x.x, y.x, acc); acc = fmaf(x.y, y.y, acc);
                acc = fmaf(x.z, y.z, acc); acc = fmaf(x.w, y.w, acc);
            }
        } else {
            for (int i = sub; i < a.d; i += 16) acc = fmaf(row[i], a.q[i], acc);
        }
        const float dot = row16_sum(acc);
        const bool filtered = a.mod_filter >= 0 && a.mods[node] != a.mod_filter;
        const float age = fmaxf(0.0f, a.t_q - a.ts[node]);
        const float s = dot * expf(-a.lambda * age);
        // filtered members score -FLT_MAX exactly like non-members (padding pool)
        const uint64_t key = (valid && !filtered) ? make_key(s, uint32_t(node)) : kEmptyKey;
        list_offer(list, thr, key, sub == 0, lane, k);
    }
    s_lists[wave][lane] = list;
    __syncthreads();
    if (wave == 0) {
        for (int w = 1; w < 4; ++w) list_offer(list, thr, s_lists[w][lane], true, lane, k);
        const int u = __popcll(__ballot(lane < k && list != kEmptyKey));
        s_out[lane] = list;
        if (lane < u) s_ids[lane] = key_id(list);
        if (lane == 0) s_cnt[0] = u;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const int u = s_cnt[0];
        const int kk = int(a.n < k ? a.n : k);          // seeds = min(K, N)
        // fewer unfiltered members than seeds: pad with the lowest ids whose
        // score is -FLT_MAX (everything but the unfiltered members), as the
        // reference's stable sort over the -FLT_MAX-filled score array does.
        if (u < kk) {
            for (int i = 1; i < u; ++i) {                 // sort member ids ascending
                const int32_t x = s_ids[i];
                int j = i - 1;
                while (j >= 0 && s_ids[j] > x) { s_ids[j + 1] = s_ids[j]; --j; }
                s_ids[j + 1] = x;
            }
            int need = kk - u, jm = 0, w = u;
            for (int32_t cand = 0; need > 0; ++cand) {
                if (jm < u && s_ids[jm] == cand) { ++jm; continue; }
                s_out[w++] = make_key(-FLT_MAX, uint32_t(cand));
                --need;
            }
        }
        s_cnt[1] = kk;
    }
    __syncthreads();
    const int kk = s_cnt[1];
    const int rc = min(a.rcap, kk);
    if (threadIdx.x < unsigned(kk)) {
        const uint64_t key = s_out[threadIdx.x];
        const int32_t id = key_id(key);
        a.seed_idx[threadIdx.x] = id;
        a.seed_val[threadIdx.x] = key_score(key);
        if (int(threadIdx.x) < rc) {
            mars_query_result r;
            r.node_id = id;
            r.score = key_score(key);
            r.modality = a.mods[id];
            r.hops_from_seed = 0;
            a.rec[threadIdx.x] = r;
        }
    }
    if (threadIdx.x == 0) {
        ResultHeader h;
        h.count = rc;
        h.visited = kk;
        h.levels = 0;
        h.n_seeds = kk;
        *a.res = h;
    }
    signal_done(a.done, a.seq);
}

__global__ void k_convert_f16(const float* __restrict__ in, __half* __restrict__ out, int64_t count) {
    const int64_t n8 = count >> 3;
    const int64_t stride = int64_t(gridDim.x) * blockDim.x;
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n8; i += stride) {
        const float4 a = reinterpret_cast<const float4*>(in)[2 * i];
        const float4 b = reinterpret_cast<const float4*>(in)[2 * i + 1];
        __half2 h[4] = {__floats2half2_rn(a.x, a.y), __floats2half2_rn(a.z, a.w),
                        __floats2half2_rn(b.x, b.y), __floats2half2_rn(b.z, b.w)};
        reinterpret_cast<uint4*>(out)[i] = *reinterpret_cast<const uint4*>(h);
    }
    for (int64_t i = (n8 << 3) + int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride)
        out[i] = __float2half_rn(in[i]);
}

// Tiled query (host-resident corpus, tiled_query.cu:174-314): after the scan of one
// tile, fold its candidate keys into the running K best and clear the count. Four
// waves sort-merge strided chunks of 64 keys, then wave 0 merges the four lists.
__global__ __launch_bounds__(256) void k_tile_merge(uint64_t* __restrict__ part, uint32_t* gcnt,
                                                    uint64_t* __restrict__ carry, int32_t k) {
    __shared__ uint64_t s_l[4][64];
    const int lane = lane_id(), wave = int(threadIdx.x >> 6);
    const uint32_t n = *gcnt;
    uint64_t list = (wave == 0 && lane < k) ? carry[lane] : kEmptyKey;
    for (uint32_t c0 = uint32_t(wave) * 64u; c0 < n; c0 += 256u) {
        const uint32_t i = c0 + uint32_t(lane);
        list = wave_merge64(list, wave_sort64(i < n ? part[i] : kEmptyKey, lane), lane, k);
    }
    s_l[wave][lane] = list;
    __syncthreads();
    if (wave == 0) {
        list = wave_merge64(list, s_l[1][lane], lane, k);
        list = wave_merge64(list, wave_merge64(s_l[2][lane], s_l[3][lane], lane, k), lane, k);
        if (lane < k) carry[lane] = list;
        if (lane == 0) *gcnt = 0u;
    }
}

// Plain streaming read of a row array, no arithmetic: the practical ceiling of the row
// scans. Each lane keeps 8 non-temporal 16-byte loads in flight (grid-stride); the words
// are folded so the loads stay live, and a workgroup writes its fold only if it equals
// the caller's sentinel.
__global__ __launch_bounds__(256) void k_read_rows(const u32x4* __restrict__ p, int64_t n16, uint32_t sentinel,
                                                   uint32_t* out) {
    uint32_t acc = 0u;
    const int64_t stride = int64_t(gridDim.x) * 256 * 8;
    for (int64_t base = int64_t(blockIdx.x) * 256 * 8 + threadIdx.x; base < n16; base += stride) {
        u32x4 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int64_t i = base + int64_t(j) * 256;
            v[j] = (i < n16) ? __builtin_nontemporal_load(p + i) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    }
    if (acc == sentinel && threadIdx.x == 0) out[blockIdx.x] = acc;
}

// The batched scan's fragment pattern, no arithmetic: each load instruction reads 16 rows
// x 64 bytes (lane l: row l % 16 of the tile, 16-byte piece l / 16 of the 64-byte k-chunk,
// the v_mfma_f32_16x16x32_f16 B operand), a tile's k-chunks back to back, tiles of 16 rows
// grid-strided over the waves. NT: non-temporal loads.
template <bool NT>
__global__ __launch_bounds__(256) void k_read_frags(const unsigned char* __restrict__ rows, int64_t n_tiles,
                                                    int32_t row_bytes, uint32_t sentinel, uint32_t* out) {
    const int lane = int(threadIdx.x) & 63;
    const int64_t nwaves = int64_t(gridDim.x) * 4;
    const int nchunks = row_bytes / 64;
    uint32_t acc = 0u;
    for (int64_t t = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6); t < n_tiles; t += nwaves) {
        const u32x4* p = reinterpret_cast<const u32x4*>(rows + (t * 16 + (lane & 15)) * row_bytes + (lane >> 4) * 16);
        int c = 0;
        for (; c + 4 <= nchunks; c += 4) {
            u32x4 v[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = NT ? __builtin_nontemporal_load(p + (c + j) * 4) : p[(c + j) * 4];
#pragma unroll
            for (int j = 0; j < 4; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
        }
        for (; c < nchunks; ++c) {
            const u32x4 v = NT ? __builtin_nontemporal_load(p + c * 4) : p[c * 4];
            acc ^= v.x ^ v.y ^ v.z ^ v.w;
        }
    }
    if (acc == sentinel && threadIdx.x == 0) out[blockIdx.x] = acc;
}

template <typename T, typename QF>
KernelLaunch scan_launch_t(const ScanArgs& a) {
    KernelLaunch l;
    const bool side = a.mod_filter >= 0 || (a.boost > 0.0f && a.ep_ids != nullptr);
    l.fn = side ? reinterpret_cast<const void*>(&k_scan<T, QF, true>)
                : reinterpret_cast<const void*>(&k_scan<T, QF, false>);
    l.grid = dim3(unsigned(a.num_wg));
    l.block = dim3(256);
    return l;
}

}  // namespace

void scan_grid(int64_t n, int32_t max_wg, int32_t* rows_per_wg, int32_t* num_wg) {
    // grid-stride scan: up to max_wg workgroups, each with at least one step of
    // 4 waves x kScanUnroll row groups of 4 rows
    const int64_t per_wg = int64_t(4) * 4 * kScanUnroll;
    int64_t wg = (n + per_wg - 1) / per_wg;
    if (wg > max_wg) wg = max_wg;
    *rows_per_wg = 0;
    *num_wg = int32_t(wg < 1 ? 1 : wg);
}

KernelLaunch scan_launch(const ScanArgs& a) {
    const bool f16 = a.fp16 != 0;
    if (!f16 && a.d % 64 == 0) {
        switch (a.d / 64) {
            case 4: return scan_launch_t<float, QF32<4>>(a);
            case 6: return scan_launch_t<float, QF32<6>>(a);
            case 8: return scan_launch_t<float, QF32<8>>(a);
            case 12: return scan_launch_t<float, QF32<12>>(a);
            case 16: return scan_launch_t<float, QF32<16>>(a);
            default: break;
        }
    }
    if (f16 && a.d % 128 == 0) {
        switch (a.d / 128) {
            case 2: return scan_launch_t<__half, QF16<2>>(a);
            case 3: return scan_launch_t<__half, QF16<3>>(a);
            case 4: return scan_launch_t<__half, QF16<4>>(a);
            case 6: return scan_launch_t<__half, QF16<6>>(a);
            case 8: return scan_launch_t<__half, QF16<8>>(a);
            default: break;
        }
    }
    if (f16) return scan_launch_t<__half, QGeneric>(a);
    return scan_launch_t<float, QGeneric>(a);
}

KernelLaunch finalize_launch() {
    KernelLaunch l;
    l.fn = reinterpret_cast<const void*>(&k_finalize);
    l.grid = dim3(1);
    l.block = dim3(kFinThreads);
    return l;
}

KernelLaunch episode_launch(int32_t d) {
    KernelLaunch l;
    l.fn = reinterpret_cast<const void*>(&k_episode<0>);
    if (d % 64 == 0) {
        switch (d / 64) {
            case 4: l.fn = reinterpret_cast<const void*>(&k_episode<4>); break;
            case 6: l.fn = reinterpret_cast<const void*>(&k_episode<6>); break;
            case 8: l.fn = reinterpret_cast<const void*>(&k_episode<8>); break;
            case 12: l.fn = reinterpret_cast<const void*>(&k_episode<12>); break;
            default: break;
        }
    }
    l.grid = dim3(1);
    l.block = dim3(256);
    return l;
}

int launch_scan(const ScanArgs& a, hipStream_t s) {
    const KernelLaunch l = scan_launch(a);
    void* args[] = {const_cast<ScanArgs*>(&a)};
    MARS_HIP(hipLaunchKernel(l.fn, l.grid, l.block, args, 0, s));
    return MARS_OK;
}

int launch_tile_merge(uint64_t* part, uint32_t* gcnt, uint64_t* carry, int32_t k, hipStream_t s) {
    MARS_LAUNCH(k_tile_merge, dim3(1), dim3(256), 0, s, part, gcnt, carry, k);
    return MARS_OK;
}

int launch_finalize(const FinalizeArgs& a, hipStream_t s) {
    MARS_LAUNCH(k_finalize, dim3(1), dim3(kFinThreads), 0, s, a);
    return MARS_OK;
}

int launch_cert_bfs(const CertArgs& a, const MultiArgs& m, hipStream_t s) {
    MARS_CHECK(a.n_lists <= kScan8MaxLists, MARS_ERR_INVALID, "certificate merge: %d lists", a.n_lists);
    if (a.d % 64 == 0) {
        switch (a.d / 64) {
            case 4: MARS_LAUNCH(k_cert_bfs<QF32<4>>, dim3(1), dim3(kFinThreads), 0, s, a, m); return MARS_OK;
            case 6: MARS_LAUNCH(k_cert_bfs<QF32<6>>, dim3(1), dim3(kFinThreads), 0, s, a, m); return MARS_OK;
            case 8: MARS_LAUNCH(k_cert_bfs<QF32<8>>, dim3(1), dim3(kFinThreads), 0, s, a, m); return MARS_OK;
            case 12: MARS_LAUNCH(k_cert_bfs<QF32<12>>, dim3(1), dim3(kFinThreads), 0, s, a, m); return MARS_OK;
            case 16: MARS_LAUNCH(k_cert_bfs<QF32<16>>, dim3(1), dim3(kFinThreads), 0, s, a, m); return MARS_OK;
            default: break;
        }
    }
    return set_error(MARS_ERR_UNSUPPORTED, "certified query: embedding_dim %d unsupported", a.d);
}

int launch_cert_multi8(const CertMArgs& a, hipStream_t s) {
    MARS_CHECK(a.q >= 1 && a.n_lists >= 1 && a.n_lists <= kScan8MaxLists && a.k <= 64 && a.knn_k <= 64,
               MARS_ERR_INVALID, "multi-query certificate: %d queries, %d lists", a.q, a.n_lists);
    switch (a.d) {
        case 256: MARS_LAUNCH(k_cert_multi8<QF32<4>>, dim3(unsigned(a.q)), dim3(kFinThreads), 0, s, a); return MARS_OK;
        case 512: MARS_LAUNCH(k_cert_multi8<QF32<8>>, dim3(unsigned(a.q)), dim3(kFinThreads), 0, s, a); return MARS_OK;
        case 768: MARS_LAUNCH(k_cert_multi8<QF32<12>>, dim3(unsigned(a.q)), dim3(kFinThreads), 0, s, a); return MARS_OK;
        case 1024: MARS_LAUNCH(k_cert_multi8<QF32<16>>, dim3(unsigned(a.q)), dim3(kFinThreads), 0, s, a); return MARS_OK;
        default: break;
    }
    return set_error(MARS_ERR_UNSUPPORTED, "multi-query certificate: embedding_dim %d", a.d);
}

int launch_multi_bfs(const MultiArgs& a, hipStream_t s) {
    MARS_LAUNCH(k_multi_bfs, dim3(unsigned(a.q)), dim3(kFinThreads), 0, s, a);
    return MARS_OK;
}

int launch_multi_select(const MultiArgs& a, hipStream_t s) {
    MARS_LAUNCH(k_multi_select, dim3(unsigned(a.q)), dim3(kFinThreads), 0, s, a);
    return MARS_OK;
}

int launch_episode(const EpisodeArgs& a, hipStream_t s) {
    const KernelLaunch l = episode_launch(a.d);
    void* args[] = {const_cast<EpisodeArgs*>(&a)};
    MARS_HIP(hipLaunchKernel(l.fn, l.grid, l.block, args, 0, s));
    return MARS_OK;
}

int launch_read_rows(const void* p, int64_t bytes, int32_t wg, uint32_t sentinel, uint32_t* out, hipStream_t s) {
    MARS_LAUNCH(k_read_rows, dim3(unsigned(wg)), dim3(256), 0, s, static_cast<const u32x4*>(p), bytes / 16,
                sentinel, out);
    return MARS_OK;
}

int launch_read_frags(const void* rows, int64_t n_rows, int32_t row_bytes, int32_t wg, bool nt, uint32_t sentinel,
                      uint32_t* out, hipStream_t s) {
    const int64_t tiles = n_rows / 16;
    const auto* r = static_cast<const unsigned char*>(rows);
    if (nt) MARS_LAUNCH(k_read_frags<true>, dim3(unsigned(wg)), dim3(256), 0, s, r, tiles, row_bytes, sentinel, out);
    else MARS_LAUNCH(k_read_frags<false>, dim3(unsigned(wg)), dim3(256), 0, s, r, tiles, row_bytes, sentinel, out);
    return MARS_OK;
}

int launch_convert_f16(const float* in, __half* out, int64_t count, hipStream_t s) {
    int64_t blocks = (count / 8 + 255) / 256;
    if (blocks < 1) blocks = 1;
    if (blocks > 65536) blocks = 65536;
    MARS_LAUNCH(k_convert_f16, dim3(unsigned(blocks)), dim3(256), 0, s, in, out, count);
    return MARS_OK;
}

}  // namespace mars
