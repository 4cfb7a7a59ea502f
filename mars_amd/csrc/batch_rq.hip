// ============================================================================
//  batch_rq.hip — k_batch_rq: batched scoring with the queries held in registers,
//  for batches of 65 .. 1023 queries (128 or 256 per workgroup, one corpus pass each).
//
//  A query tile of 256 fp16 queries x d does not fit in LDS (384 KiB at d = 768), but
//  it fits in the register files of one CU: each of the four waves (one per SIMD, the
//  whole 512-register file) holds 16 QT queries as MFMA A fragments for the whole kernel
//  (NS x QT fragments of 16 bytes per lane: 384 registers at d = 768 and QT = 4). Only
//  the corpus moves: 16-row tiles stream from HBM straight into LDS
//  (global_load_lds_dwordx4, each wave loading a quarter of every tile, whole rows
//  contiguous), five tile buffers deep, and all four waves read every tile's B fragments
//  from LDS. Each corpus row is read from HBM once per workgroup's 64 QT queries, and the
//  CU takes in nothing else.
//
//  Tile layout in LDS: row r's 16-byte piece p sits in slot r * P + (p ^ (r & 15)),
//  P = d / 8 pieces per row. A B-fragment read (lanes 16 g .. 16 g + 15: rows 0 .. 15,
//  the same piece) then touches 16 distinct 16-byte bank groups.
//
//  Scores: the same MFMA, operands and k order as k_batch_scan (queries the A operand,
//  rows the B operand, k-steps 0 .. NS - 1 accumulated in order from zero), so every raw
//  score is bit-identical to that kernel's, and so is every fused score. Selection: a tile
//  first goes through a test in the MFMA layout (a lane holds one row's scores for 4 QT
//  queries) against each query's floor (from the sampled pass of launch_batch_topk); only
//  a tile with a score at or above its floor goes through k_batch_scan's epilogue (a
//  per-wave LDS transpose after which lane j owns query j, the decay, filter and bound,
//  register lists), inserting only the rows that reach the bound, one per lane and
//  round. Output: K keys per (query, row range), the layout k_batch_merge reads.
//
//  Reference analogue: wmma_mma_similarity_kernel / wmma_similarity_kernel
//  (src/wmma_similarity.cu:55-138), which score one query and are never called.
// ============================================================================
#include "device.hpp"

#include <cfloat>

namespace mars {
namespace {

constexpr int kRWaves = 4;     // one per SIMD; each holds QT 16-query MFMA tiles
constexpr int kRThreads = kRWaves * 64;
constexpr int kRRows = 16;     // corpus rows per tile
constexpr int kRBuf = 5;       // tile buffers: tiles i + 1 .. i + 4 load while tile i computes
constexpr int kRqSparse = 4;   // at most this many lanes with one pair each: the pairs one at a time

template <int NS, int QT>
struct RqLds {
    u32x4 tile[kRBuf][kRRows * NS * 4];          // 16 rows x d / 8 pieces, swizzled
    uint32_t side[kRBuf][kRWaves][64];           // per wave: lanes 0-15 the rows' timestamps, 16-31 modalities
    float stage[kRWaves][kRRows][16 * QT + 1];   // per-wave score tile (+1: bank spread)
    float wrow[kRWaves][kRRows];                 // per wave: the tile rows' weights (or timestamps)
    float floorv[kRWaves][16 * QT];              // per wave: its queries' floors (-inf: none)
};

// s_waitcnt immediates (gfx9 encoding: vmcnt[3:0] and [15:14], expcnt[6:4], lgkmcnt[11:8])
constexpr int rq_wait_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int kRqWaitLgkm0 = 15 | (3 << 14) | (7 << 4);

// Orders this wave's LDS writes before its later LDS reads (the score stage is private
// to one wave).
__device__ inline void rq_wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One 16-byte (or 4-byte) piece per lane from global memory straight into LDS: lane l
// writes lds + l * bytes.
__device__ __attribute__((always_inline)) inline void dma16(const void* g, u32x4* lds) {
    __builtin_amdgcn_global_load_lds(g, lds, 16, 0, 0);
}
__device__ __attribute__((always_inline)) inline void dma4(const void* g, uint32_t* lds) {
    __builtin_amdgcn_global_load_lds(g, lds, 4, 0, 0);
}

// QT: 16-query MFMA tiles per wave (2 or 4: 128 or 256 queries per workgroup).
template <int NS, int K, int QT>
__global__ __launch_bounds__(kRThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void k_batch_rq(BatchArgs a) {
    __shared__ __attribute__((aligned(16))) RqLds<NS, QT> sh;
    constexpr int WQ = 16 * QT;                  // queries per wave
    constexpr int P = NS * 4;                    // 16-byte pieces per row
    constexpr int kLd = NS / 4;                  // tile loads per wave (64 slots each)
    static_assert(NS % 4 == 0 && P % 16 == 0, "tile layout");
    const int tid = int(threadIdx.x), lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int m = lane & 15, kg = lane >> 4;
    constexpr int d = NS * 32;
    const int r_id = int(blockIdx.x) % a.n_rranges;
    const int g = int(blockIdx.x) / a.n_rranges;                  // the workgroup's group of 64 QT queries
    const int wq0 = (g * kRWaves + wave) * WQ;                    // this wave's first query
    const int64_t r0 = int64_t(r_id) * (a.range_stride > 0 ? a.range_stride : a.rows_per_range);
    const int64_t r1 = (a.n < r0 + a.rows_per_range) ? a.n : r0 + a.rows_per_range;
    const int64_t ntiles = r1 > r0 ? (r1 - r0 + kRRows - 1) / kRRows : 0;

    // This lane's slots of a tile: load j of the wave fills slots s = (wave kLd + j) 64 +
    // lane, i.e. slot s % P of row s / P, which holds piece (s % P) ^ (row & 15); lin[j] is
    // that piece's offset from the tile's first row, in halves.
    int lin[kLd];
#pragma unroll
    for (int j = 0; j < kLd; ++j) {
        const int s = (wave * kLd + j) * 64 + lane;
        lin[j] = (s / P) * d + ((s % P) ^ ((s / P) & 15)) * 8;
    }
    const int side_row = lane & 15;
    const bool side_mod = lane >= 16 && lane < 32;
    // Tile tt (clamped: tiles past the last load the last one again, so every iteration
    // issues the same loads and the wait counts stay exact) into buffer b. Rows past the
    // range's end are only read in its last tile, and are clamped there.
    auto issue_tile = [&](int64_t tt, int b) {
        tt = tt < ntiles ? tt : ntiles - 1;
        const int64_t base = r0 + tt * kRRows;
        const __half* tp = a.emb16 + base * d;
        if (base + kRRows <= r1) {
#pragma unroll
            for (int j = 0; j < kLd; ++j)
                dma16(tp + lin[j], &sh.tile[b][(wave * kLd + j) * 64]);
        } else {
            const int last = int(r1 - 1 - base);
#pragma unroll
            for (int j = 0; j < kLd; ++j) {
                const int r = lin[j] / d;
                const int off = r <= last ? lin[j] : lin[j] - (r - last) * d;
                dma16(tp + off, &sh.tile[b][(wave * kLd + j) * 64]);
            }
        }
        int64_t srow = base + side_row;
        srow = srow < r1 ? srow : r1 - 1;
        const void* sp = side_mod ? static_cast<const void*>(a.mods + srow) : static_cast<const void*>(a.ts + srow);
        dma4(sp, &sh.side[b][wave][0]);
    };
    if (ntiles > 0) {
#pragma unroll
        for (int b = 0; b < kRBuf - 1; ++b) issue_tile(b, b);
    }

    // The wave's WQ queries as A fragments: af[qt][ks] = query wq0 + qt*16 + m,
    // halves ks*32 + kg*8 .. +7 (zero past the batch).
    f16x8 af[QT][NS];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int qrow = wq0 + qt * 16 + m;
        const bool ok = qrow < a.q;
        const u32x4* qp = reinterpret_cast<const u32x4*>(a.qh + int64_t(ok ? qrow : 0) * d + kg * 8);
#pragma unroll
        for (int ks = 0; ks < NS; ++ks) {
            const u32x4 v = ok ? qp[ks * 4] : u32x4{0u, 0u, 0u, 0u};
            af[qt][ks] = __builtin_bit_cast(f16x8, v);
        }
    }

    // lane j < WQ owns query wq0 + j
    const int myq = wq0 + lane;
    const bool qvalid = lane < WQ && myq < a.q;
    const bool wave_live = wq0 < a.q;            // uniform: the wave has queries to score
    const float tq = qvalid ? a.tq[myq] : 0.0f;
    const bool uni = a.uniform_tq != 0;
    const float tq0 = a.tq[0];
    const bool plain = myq >= a.q_plain;          // neighbour search: dot product only
    // the query's own row (a neighbour search of a corpus row), relative to the range: -1
    // when it is not in this range (one 32-bit register: the queries need the rest)
    int32_t self_rel = -1;
    if (a.self_base >= 0 && qvalid && plain) {
        const int64_t self_id = a.self_base + (myq - a.q_plain);
        if (self_id >= r0 && self_id < r1) self_rel = int32_t(self_id - r0);
    }
    uint64_t list[K];
#pragma unroll
    for (int j = 0; j < K; ++j) list[j] = kEmptyKey;
    uint32_t own = 0u;                           // ord32 of the bound: max(floor, list[K-1]'s score once full)
    if (a.floor_keys != nullptr && qvalid) {
        const uint64_t fk = a.floor_keys[int64_t(myq) * a.floor_k + a.floor_k - 1];
        if (fk != kEmptyKey) own = ord32(key_score(fk));
    }
    // per query: the floor its rows must reach (read after the loop's first barrier); past
    // the batch +inf, so no row reaches it
    if (lane < WQ) sh.floorv[wave][lane] = !qvalid ? INFINITY : own != 0u ? ord32_inv(own) : -INFINITY;
    const bool prefilter = uni || a.lambda >= 0.0f;

    // B-fragment slots: k-step ks reads piece 4 ks + kg of row m, i.e. slot
    // m P + ((4 ks + kg) ^ m) = m P + 16 (ks / 4) + ((4 (ks % 4)) ^ kg ^ m).
    int boff[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) boff[c] = m * P + ((4 * c) ^ kg ^ m);

    int b = 0;
    for (int64_t i = 0; i < ntiles; ++i) {
        // this wave's loads of tile i (tiles i + 1 .. i + 3 may stay in flight), then meet:
        // every wave's loads of tile i landed, every wave is done with tile i - 1's buffer
        __builtin_amdgcn_s_waitcnt(rq_wait_vm((kRBuf - 2) * (kLd + 1)));
        __builtin_amdgcn_s_waitcnt(kRqWaitLgkm0);
        __builtin_amdgcn_s_barrier();
        const int bn = b == 0 ? kRBuf - 1 : b - 1;                // tile i - 1's buffer
        issue_tile(i + kRBuf - 1, bn);
        const int64_t t0 = r0 + i * kRRows;
        if (wave_live) {
            const u32x4* tb = sh.tile[b];
            f32x4 acc[QT];
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) acc[qt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            auto bfrag = [&](int ks) { return __builtin_bit_cast(f16x8, tb[boff[ks & 3] + 16 * (ks >> 2)]); };
            if constexpr (QT == 4) {
            // B fragments two k-steps ahead in three registers (the 256-query form has no
            // room for a fourth: at 512 VGPRs it ran at half speed)
            f16x8 bf[3];
            bf[0] = bfrag(0);
            bf[1] = bfrag(1);
#pragma unroll
            for (int ks = 0; ks < NS; ++ks) {
                if (ks + 2 < NS) bf[(ks + 2) % 3] = bfrag(ks + 2);
#pragma unroll
                for (int qt = 0; qt < QT; ++qt)
                    acc[qt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[qt][ks], bf[ks % 3], acc[qt], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
            } else {
            // B fragments in pairs of k-steps, two pairs of registers: pair p + 1 is read
            // right after pair p's first MFMA, so each pair's reads have the 4 QT - 1 MFMAs
            // of a pair to land (every wait for them also waits for everything issued before)
            f16x8 bf[2][2];
            bf[0][0] = bfrag(0);
            bf[0][1] = bfrag(1);
#pragma unroll
            for (int p = 0; p < NS / 2; ++p) {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
#pragma unroll
                    for (int qt = 0; qt < QT; ++qt) {
                        acc[qt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[qt][2 * p + j], bf[p & 1][j], acc[qt], 0, 0, 0);
                        if (j == 0 && qt == 0 && p + 1 < NS / 2) {
                            __builtin_amdgcn_sched_barrier(0);
                            bf[(p + 1) & 1][0] = bfrag(2 * p + 2);
                            bf[(p + 1) & 1][1] = bfrag(2 * p + 3);
                            __builtin_amdgcn_sched_barrier(0);
                        }
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            }
            // Row m of the score tile (this lane's row): its weight (decay at the one query
            // time, else its timestamp) and filter flag.
            const float sts = __uint_as_float(sh.side[b][wave][m]);
            const int32_t smod = int32_t(sh.side[b][wave][16 + m]);
            const bool keep_m = a.mod_filter < 0 || smod == a.mod_filter;
            const float w_m = !uni ? sts : (a.lambda != 0.0f ? expf(-a.lambda * fmaxf(0.0f, tq0 - sts)) : 1.0f);
            const int nr = int((r1 - t0) < kRRows ? (r1 - t0) : kRRows);
            // Pre-filter in the MFMA layout (C[query qt*16 + 4*kg + v][row m]): bit 4 qt + v
            // of hb is set when this lane's row reaches query qt*16 + 4*kg + v's floor (from
            // the sampled pass; +inf past the batch). With one query time the score is the
            // selection's own (x * w_m); otherwise x, or 0 for x < 0, bounds x * w for any
            // weight in (0, 1]. NaN passes.
            uint32_t hb = 0xFFFFu;
            if (prefilter) {
                hb = 0u;
#pragma unroll
                for (int qt = 0; qt < QT; ++qt) {
                    const f32x4 fl = *reinterpret_cast<const f32x4*>(&sh.floorv[wave][qt * 16 + 4 * kg]);
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const float x = acc[qt][v];
                        float sv = uni ? x * w_m : (x < 0.0f ? 0.0f : x);
                        sv = keep_m ? sv : -FLT_MAX;
                        sv = (wq0 + qt * 16 + 4 * kg + v >= a.q_plain) ? x : sv;
                        hb = !(sv < fl[v]) ? (hb | (1u << (4 * qt + v))) : hb;
                    }
                }
            }
            hb = m < nr ? hb : 0u;
            const uint64_t hl = __ballot(hb != 0u);
            const bool any = hl != 0u;
            // sparse: a few lanes, one pair each; each pair's query lane then offers that
            // one row, instead of testing all 16
            const bool sparse = prefilter && __popcll(hl) <= kRqSparse && __ballot((hb & (hb - 1u)) != 0u) == 0;
            // The fused score of row j for this lane's query: dot * w (k_batch_scan's
            // arithmetic), filtered rows -FLT_MAX, neighbour searches the plain dot.
            // (Branch-free per lane: the uni / lambda tests are wave-uniform.)
            auto fuse = [&](float x, float wj, bool keep) {
                float sv = x;
                if (uni) sv = x * wj;
                else if (a.lambda != 0.0f) sv = x * expf(-a.lambda * fmaxf(0.0f, tq - wj));
                sv = keep ? sv : -FLT_MAX;
                return plain ? x : sv;
            };
            if (any) {
                if (lane < kRRows) sh.wrow[wave][lane] = w_m;
                const uint32_t keepm = uint32_t(__ballot(keep_m && lane < kRRows));
                uint32_t pass = 0u;                  // rows of this lane's query to offer
                // the tile, transposed: C[query = qt*16 + 4*kg + v][row = m]
#pragma unroll
                for (int qt = 0; qt < QT; ++qt)
#pragma unroll
                    for (int v = 0; v < 4; ++v) sh.stage[wave][m][qt * 16 + 4 * kg + v] = acc[qt][v];
                if (sparse) {
                    // each pair's row to the lane of its query (bit b: query (b / 4)*16 + 4*kg + b % 4)
                    const int bt = hb != 0u ? __builtin_ctz(hb) : 0;
                    for (uint64_t ln = hl; ln != 0; ln &= ln - 1) {
                        const int L = __builtin_ctzll(ln);
                        const int b1 = __builtin_amdgcn_readlane(bt, L);
                        if (lane == (b1 >> 2) * 16 + 4 * (L >> 4) + (b1 & 3)) pass |= 1u << (L & 15);
                    }
                }
                rq_wave_lds_sync();
                if (qvalid) {
                    const float bound_f = own != 0u ? ord32_inv(own) : -INFINITY;
                    if (!sparse) {
                        // The rows that may enter the list: not below its K-th score (a float
                        // test that never rejects a row the key test below accepts; NaN passes).
#pragma unroll
                        for (int j = 0; j < kRRows; ++j) {
                            const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w_m), j));
                            const float sv = fuse(sh.stage[wave][j][lane], wj, (keepm >> j) & 1u);
                            pass |= uint32_t(!(sv < bound_f)) << j;
                        }
                        pass &= 0xFFFFu >> (kRRows - nr);
                    }
                    const int32_t self_t = self_rel - int32_t(t0 - r0);
                    if (self_t >= 0 && self_t < kRRows) pass &= ~(1u << self_t);
                    // one row per lane and round (a round costs what one insertion does; most
                    // tiles need one or none), its fused score from the stage (the same
                    // operations, so the same bits)
                    while (pass) {
                        const int j = __builtin_ctz(pass);
                        pass &= pass - 1u;
                        const float sv = fuse(sh.stage[wave][j][lane], sh.wrow[wave][j], (keepm >> j) & 1u);
                        if (ord32(sv) >= own) {
                            const uint64_t key = make_key(sv, uint32_t(t0 + j));
                            if (key < list[K - 1]) {
                                reg_insert<K>(list, key);
                                if (list[K - 1] != kEmptyKey) {
                                    const uint32_t o = ord32(key_score(list[K - 1]));
                                    own = o > own ? o : own;
                                }
                            }
                        }
                    }
                }
                rq_wave_lds_sync();
            }
        }
        b = b == kRBuf - 1 ? 0 : b + 1;
    }
    // the last iterations' loads (clamped tiles nobody reads) must land before the
    // workgroup ends and its LDS is handed to another
    __builtin_amdgcn_s_waitcnt(rq_wait_vm(0));
    if (qvalid) {
        uint64_t* out = a.part + ((int64_t(myq / 64) * a.n_rranges + r_id) * 64 + myq % 64) * K;
#pragma unroll
        for (int j = 0; j < K; ++j) out[j] = list[j];
    }
}

template <int NS, int K, int QT>
int launch_rq_q(const BatchArgs& a, hipStream_t s) {
    constexpr int wgq = kRWaves * 16 * QT;       // queries per workgroup
    const unsigned grid = unsigned(a.n_rranges * ((a.q + wgq - 1) / wgq));
    MARS_LAUNCH((k_batch_rq<NS, K, QT>), dim3(grid), dim3(kRThreads), 0, s, a);
    return MARS_OK;
}

template <int NS, int K>
int launch_rq_t(const BatchArgs& a, hipStream_t s) {
    return batch_rq_tiles(a.q) == 2 ? launch_rq_q<NS, K, 2>(a, s) : launch_rq_q<NS, K, 4>(a, s);
}

template <int K>
int launch_rq_k(const BatchArgs& a, hipStream_t s) {
    switch (a.d / 32) {
        case 8: return launch_rq_t<8, K>(a, s);
        case 12: return launch_rq_t<12, K>(a, s);
        case 16: return launch_rq_t<16, K>(a, s);
        case 24: return launch_rq_t<24, K>(a, s);
        default: return set_error(MARS_ERR_UNSUPPORTED, "batched scoring: embedding_dim %d not in {256,384,512,768}", a.d);
    }
}

}  // namespace

int launch_batch_rq(const BatchArgs& a, hipStream_t s) {
    MARS_CHECK(a.k >= 1 && a.k <= 16, MARS_ERR_UNSUPPORTED, "batched scoring keeps at most 16 per query (asked %d)",
               a.k);
    MARS_CHECK(a.n_qblocks == (a.q + 63) / 64, MARS_ERR_INVALID, "batched scoring: %d query blocks for %d queries",
               a.n_qblocks, a.q);
    return a.k <= 8 ? launch_rq_k<8>(a, s) : launch_rq_k<16>(a, s);
}

}  // namespace mars
