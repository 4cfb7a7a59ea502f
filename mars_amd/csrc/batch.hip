// ============================================================================
//  batch.hip — batched scoring on MFMA (gfx950 v_mfma_f32_16x16x32_f16) with
//  fused temporal decay and per-query top-K; the k-NN graph builder on top.
//
//  k_batch_scan  C[q][row] = <Qh_q, E16_row> for 64 queries x 16-row tiles.
//                Queries live in LDS in MFMA A-fragment order (one 16-byte LDS
//                read per lane per fragment, conflict free); corpus fragments are
//                16-byte global loads straight into registers (the B operand is
//                K-contiguous, like the A operand, so no transpose is needed).
//                The 16x64 score tile goes through a per-wave LDS stage, after
//                which lane j owns query j: it applies the decay / filter and
//                keeps a sorted register list of the K best keys (score desc,
//                id asc). Workgroup (row range r, query block b) writes K keys per
//                query; the workgroup index puts all query blocks of a row range
//                on the same XCD (id % 8 == r % 8) so they share its L2.
//  k_batch_merge One wave per query merges the per-row-range keys.
//  k_knn_rerank  Exact fp32 rescoring of k-NN candidates (one wave per node).
//
//  Reference analogue: wmma_mma_similarity_kernel / wmma_similarity_kernel
//  (src/wmma_similarity.cu:55-138), which score one query and are never called.
// ============================================================================
#include "device.hpp"

#include <algorithm>
#include <cfloat>

namespace mars {
namespace {

constexpr int kBQ = 64;        // queries per workgroup (4 MFMA row tiles of 16)
constexpr int kBWaves = 8;     // waves per workgroup
constexpr int kTile = 16;      // corpus rows per MFMA tile

// Orders this wave's LDS writes before its later LDS reads (the staging buffers
// are private to one wave; waves run different trip counts, so no block barrier).
__device__ inline void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int KCH, int K>
struct BatchLds {
    static constexpr size_t kQBytes = size_t(4) * KCH * 64 * 16;
    static constexpr size_t kListBytes = size_t(kBWaves) * 64 * K * 8;
    static constexpr size_t kBytes = kQBytes > kListBytes ? kQBytes : kListBytes;
};

template <int KCH, int K>
__global__ __launch_bounds__(kBWaves * 64) void k_batch_scan(BatchArgs a) {
    // query A-fragments [4][KCH][64] (16 B each); after the scan, the per-wave lists
    __shared__ __attribute__((aligned(16))) unsigned char s_raw[BatchLds<KCH, K>::kBytes];
    u32x4 (*s_q)[KCH][64] = reinterpret_cast<u32x4 (*)[KCH][64]>(s_raw);
    __shared__ float s_stage[kBWaves][kTile][kBQ + 1];  // per-wave score tile (+1: bank spread)
    // Best known K-th score per query in this workgroup: a wave whose own list is full
    // publishes its K-th score here; a row scoring strictly below it cannot enter the
    // workgroup's top-K (K better rows are already held), so no wave keeps it.
    __shared__ uint32_t s_thr[kBQ];
    const int lane = int(threadIdx.x & 63u), wave = int(threadIdx.x >> 6);
    const int m = lane & 15, kg = lane >> 4;
    const int r_id = int(blockIdx.x) % a.n_rranges;
    const int qb = int(blockIdx.x) / a.n_rranges;
    const int d = KCH * 32;
    constexpr int H = KCH / 2;                 // k steps per half tile

    // stage this block's 64 queries (zero rows past the batch)
    for (int idx = int(threadIdx.x); idx < 4 * KCH * 64; idx += kBWaves * 64) {
        const int l = idx & 63, ks = (idx >> 6) % KCH, qt = idx / (64 * KCH);
        const int qrow = qb * kBQ + qt * 16 + (l & 15);
        u32x4 v = {0u, 0u, 0u, 0u};
        if (qrow < a.q)
            v = *reinterpret_cast<const u32x4*>(a.qh + int64_t(qrow) * d + ks * 32 + (l >> 4) * 8);
        s_q[qt][ks][l] = v;
    }
    if (threadIdx.x < kBQ) s_thr[threadIdx.x] = 0u;
    __syncthreads();

    // lane j owns query (qb*64 + j)
    const int myq = qb * kBQ + lane;
    const bool qvalid = myq < a.q;
    const float tq = qvalid ? a.tq[myq] : 0.0f;
    const bool uni = a.uniform_tq != 0;
    const float tq0 = a.tq[0];
    const bool plain = myq >= a.q_plain;       // neighbour search: dot product only
    const int64_t self_id = (a.self_base >= 0 && qvalid && plain) ? a.self_base + (myq - a.q_plain) : -1;
    uint64_t list[K];
#pragma unroll
    for (int j = 0; j < K; ++j) list[j] = kEmptyKey;
    uint32_t own = 0u;                         // ord32 of list[K-1]'s score once the list is full

    const int64_t r0 = int64_t(r_id) * (a.range_stride > 0 ? a.range_stride : a.rows_per_range);
    const int64_t r1 = (a.n < r0 + a.rows_per_range) ? a.n : r0 + a.rows_per_range;
    const int64_t step = int64_t(kBWaves) * kTile;
    // row fragments of a half tile (k steps half*H .. half*H + H - 1); the next half's
    // loads are issued before the current half's MFMAs
    auto load_half = [&](u32x4 (&b)[H], int64_t t, int half) {
        const int64_t row = t + m;
        const int64_t rr = row < r1 ? row : r1 - 1;
        const u32x4* bp = reinterpret_cast<const u32x4*>(a.emb16 + rr * d + kg * 8) + half * H * 4;
#pragma unroll
        for (int ks = 0; ks < H; ++ks) b[ks] = bp[ks * 4];
    };
    // Half 0 of a tile and its side values (timestamp, modality) load one half-tile
    // ahead; the side values are loaded first, so waiting for them never waits for
    // younger row loads. The kernel stays near 160 VGPRs, which leaves room on every
    // CU for the small kernels of other streams (episode queries, inserts).
    u32x4 b0[H], b1[H];
    float side_ts = 0.0f;
    int32_t side_mod = 0;
    auto load_head = [&](int64_t t) {
        if (lane < kTile) {
            const int64_t rl = (t + lane < r1) ? t + lane : r1 - 1;
            side_ts = a.ts[rl];
            side_mod = (a.mod_filter >= 0) ? a.mods[rl] : 0;
        }
        load_half(b0, t, 0);
    };
    int64_t t0 = r0 + int64_t(wave) * kTile;
    if (t0 < r1) load_head(t0);
    for (; t0 < r1; t0 += step) {
        load_half(b1, t0, 1);
        // lane j < 16: row j's weight (decay at the one query time, else its timestamp)
        // and filter flag, taken before the next tile's loads reuse the side registers
        float row_w = 0.0f;
        bool row_keep = true;
        if (lane < kTile) {
            row_keep = a.mod_filter < 0 || side_mod == a.mod_filter;
            row_w = !uni ? side_ts : (a.lambda != 0.0f ? expf(-a.lambda * fmaxf(0.0f, tq0 - side_ts)) : 1.0f);
        }
        const uint64_t keepm = __ballot(row_keep);
        f32x4 acc[4];
#pragma unroll
        for (int qt = 0; qt < 4; ++qt) acc[qt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < H; ++ks) {
            const f16x8 bf = __builtin_bit_cast(f16x8, b0[ks]);
#pragma unroll
            for (int qt = 0; qt < 4; ++qt) {
                const f16x8 af = __builtin_bit_cast(f16x8, s_q[qt][ks][lane]);
                acc[qt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf, acc[qt], 0, 0, 0);
            }
        }
        if (t0 + step < r1) load_head(t0 + step);
#pragma unroll
        for (int ks = 0; ks < H; ++ks) {
            const f16x8 bf = __builtin_bit_cast(f16x8, b1[ks]);
#pragma unroll
            for (int qt = 0; qt < 4; ++qt) {
                const f16x8 af = __builtin_bit_cast(f16x8, s_q[qt][H + ks][lane]);
                acc[qt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf, acc[qt], 0, 0, 0);
            }
        }
        // C[query = qt*16 + 4*kg + i][row = m]
#pragma unroll
        for (int qt = 0; qt < 4; ++qt)
#pragma unroll
            for (int i = 0; i < 4; ++i) s_stage[wave][m][qt * 16 + 4 * kg + i] = acc[qt][i];
        // the row weights as wave-uniform values (read in uniform control flow)
        float w[kTile];
#pragma unroll
        for (int j = 0; j < kTile; ++j) w[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(row_w), j));
        wave_lds_sync();
        if (qvalid) {
            uint32_t bound = own > s_thr[lane] ? own : s_thr[lane];
            const uint32_t own0 = own;
            const int nr = int((r1 - t0) < kTile ? (r1 - t0) : kTile);
            // the tile's 16 fused scores of this lane's query: dot * w (the reference's
            // order), filtered rows -FLT_MAX; all LDS reads issued before any is used
            float sc[kTile];
#pragma unroll
            for (int j = 0; j < kTile; ++j) sc[j] = s_stage[wave][j][lane];
            if (!plain) {
#pragma unroll
                for (int j = 0; j < kTile; ++j) {
                    float sv = sc[j];
                    if (uni) sv = sv * w[j];
                    else if (a.lambda != 0.0f) sv = sv * expf(-a.lambda * fmaxf(0.0f, tq - w[j]));
                    sc[j] = ((keepm >> j) & 1u) ? sv : -FLT_MAX;
                }
            }
            uint32_t top = 0u;
#pragma unroll
            for (int j = 0; j < kTile; ++j) {
                const uint32_t o = ord32(sc[j]);
                top = (j < nr && o > top) ? o : top;
            }
            if (top >= bound)
            for (int j = 0; j < nr; ++j) {
                const float sv = sc[j];
                if (ord32(sv) >= bound && t0 + j != self_id) {
                    const uint64_t key = make_key(sv, uint32_t(t0 + j));
                    if (key < list[K - 1]) {
                        reg_insert<K>(list, key);
                        if (list[K - 1] != kEmptyKey) {
                            own = ord32(key_score(list[K - 1]));
                            bound = bound > own ? bound : own;
                        }
                    }
                }
            }
            if (own > own0) atomicMax(&s_thr[lane], own);
        }
        wave_lds_sync();
    }

    // merge the 8 waves' lists of each query (the query LDS is reused as staging)
    __syncthreads();
    uint64_t* s_lists = reinterpret_cast<uint64_t*>(s_raw);   // [kBWaves][64][K]
#pragma unroll
    for (int j = 0; j < K; ++j) s_lists[(wave * 64 + lane) * K + j] = list[j];
    __syncthreads();
    if (wave == 0 && qvalid) {
        for (int w = 1; w < kBWaves; ++w)
#pragma unroll
            for (int j = 0; j < K; ++j) {
                const uint64_t x = s_lists[(w * 64 + lane) * K + j];
                if (x < list[K - 1]) reg_insert<K>(list, x);
            }
        uint64_t* out = a.part + ((int64_t(qb) * a.n_rranges + r_id) * kBQ + lane) * K;
#pragma unroll
        for (int j = 0; j < K; ++j) out[j] = list[j];
    }
}

// One workgroup of eight waves per query: merge n_rranges lists of K keys into the best
// k_out. Each wave takes every eighth round of 8 x 64 keys (loads in flight together; a
// chunk with many keys under the wave's bound is sorted and merged in registers, one with
// a few inserts them one by one), then wave 0 merges the eight lists. (One wave per
// query, inserting every key under its bound one at a time: 21 us for 256 queries of
// 4,096 keys; this form: 13 us.)
constexpr int kMergeWaves = 8;
constexpr int kRerankPieces = 3;  // k_knn_rerank: 16-byte pieces per lane and row (d <= 768)
__global__ __launch_bounds__(kMergeWaves * 64) void k_batch_merge(const uint64_t* __restrict__ part, int32_t n_rranges,
                                                                  int32_t kpart, int32_t q, int32_t k_out,
                                                                  uint64_t* __restrict__ out) {
    __shared__ uint64_t s_l[kMergeWaves][64];
    const int lane = int(threadIdx.x & 63u), wave = int(threadIdx.x >> 6);
    const int qi = int(blockIdx.x);
    if (qi >= q) return;                               // the whole workgroup
    const int qb = qi / kBQ, j = qi % kBQ;
    uint64_t list = kEmptyKey, thr = kEmptyKey;
    const int total = n_rranges * kpart;
    const int kshift = kpart == 8 ? 3 : 4;             // kpart is 8 or 16 (batch_kpart)
    constexpr int kMergeLd = 8;
    for (int base = wave * 64 * kMergeLd; base < total; base += kMergeWaves * 64 * kMergeLd) {
        uint64_t xs[kMergeLd];
#pragma unroll
        for (int c = 0; c < kMergeLd; ++c) {
            const int t = base + c * 64 + lane;
            xs[c] = kEmptyKey;
            if (t < total) {
                const int r = t >> kshift, s = t & (kpart - 1);
                xs[c] = part[((int64_t(qb) * n_rranges + r) * kBQ + j) * kpart + s];
            }
        }
#pragma unroll
        for (int c = 0; c < kMergeLd; ++c) wave_offer(list, thr, xs[c], lane, k_out);
    }
    s_l[wave][lane] = list;
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int w = 1; w < kMergeWaves; ++w) list = wave_merge64(list, s_l[w][lane], lane, k_out);
        if (lane < k_out) out[int64_t(qi) * k_out + lane] = list;
    }
}

// Exact fp32 rescoring of kc candidates per node; keeps k_out by (score desc, id asc).
// Nodes q0 .. q0+nq-1; cand / nbrs are indexed from q0.
// With nrm (the fp16 copy's row-norm maxima) and cert: cert[node] = 1 when the lists are
// certified exact. Every row outside the candidates has an fp16 score at most the kc-th
// candidate's, and its fp32 score (this kernel's arithmetic) exceeds its fp16 score by at
// most
//     eps = |e16| |ftz(e16) - e| + |e| |ftz(e16) - e|      (both fp16 roundings)
//           + g_mfma |e16|^2 + g_fp32 |e|^2 + u (|e16|^2 (1 + g_mfma) + |e|^2 (1 + g_fp32))
// (row maxima for the query row too; g_mfma = 2 d u / (1 - d u), doubled for the MFMA's
// unspecified order; g_fp32 = n u / (1 - n u) with n = 4 ceil(d / 256) + 6 for this
// kernel's per-lane chains and 64-lane butterfly), so a k_out-th exact score above (kc-th fp16 score
// + eps) leaves no row outside the candidates that could enter the list. Fewer than kc
// candidates: every other row was one.
__global__ __launch_bounds__(256) void k_knn_rerank(const float* __restrict__ emb, int64_t q0, int64_t nq,
                                                    int32_t d, const uint64_t* __restrict__ cand, int32_t kc,
                                                    int32_t k_out, int32_t* __restrict__ nbrs,
                                                    const uint32_t* __restrict__ nrm, int32_t* __restrict__ cert) {
    const int lane = int(threadIdx.x & 63u);
    const int64_t node = int64_t(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (node >= nq) return;                      // whole wave
    // lane l holds elements 4 l + 256 j .. + 3 of the node's row (d <= 768: j < 3)
    const int nj = (d + 255) >> 8;
    const float* x = emb + (q0 + node) * d;
    f32x4 xr[kRerankPieces];
#pragma unroll
    for (int j = 0; j < kRerankPieces; ++j) {
        const int i = 256 * j + 4 * lane;
        xr[j] = (j < nj && i < d) ? *reinterpret_cast<const f32x4*>(x + i) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    uint64_t keys[16];
#pragma unroll
    for (int c = 0; c < 16; ++c) keys[c] = kEmptyKey;
    const int nc = kc < 16 ? kc : 16;
    // four candidates at a time: their rows read in 1 KB pieces, one fmaf chain per lane and
    // candidate, then a butterfly over the wave (lane 0's association is the one kept)
    for (int c0 = 0; c0 < nc; c0 += 4) {
        uint64_t ck[4];
        float acc[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            ck[u] = c0 + u < nc ? cand[node * kc + c0 + u] : kEmptyKey;
            const float* y = ck[u] != kEmptyKey ? emb + int64_t(key_id(ck[u])) * d : x;
            acc[u] = 0.0f;
#pragma unroll
            for (int j = 0; j < kRerankPieces; ++j) {
                const int i = 256 * j + 4 * lane;
                if (j < nj && i < d) {
                    const f32x4 yv = *reinterpret_cast<const f32x4*>(y + i);
                    acc[u] = fmaf(xr[j].x, yv.x, acc[u]);
                    acc[u] = fmaf(xr[j].y, yv.y, acc[u]);
                    acc[u] = fmaf(xr[j].z, yv.z, acc[u]);
                    acc[u] = fmaf(xr[j].w, yv.w, acc[u]);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) acc[u] += __shfl_xor(acc[u], m);
            if (c0 + u < nc) keys[c0 + u] = ck[u] != kEmptyKey ? make_key(acc[u], uint32_t(key_id(ck[u]))) : kEmptyKey;
        }
    }
    if (lane == 0) {
        for (int i = 1; i < 16; ++i) {           // insertion sort of 16 keys
            const uint64_t v = keys[i];
            int j = i - 1;
            while (j >= 0 && keys[j] > v) { keys[j + 1] = keys[j]; --j; }
            keys[j + 1] = v;
        }
        for (int c = 0; c < k_out; ++c) nbrs[node * k_out + c] = (keys[c] != kEmptyKey) ? key_id(keys[c]) : -1;
        if (cert) {
            const uint64_t last = cand[node * kc + kc - 1];
            bool ok = last == kEmptyKey;
            if (!ok && nrm && keys[k_out - 1] != kEmptyKey) {
                const double e32 = double(__uint_as_float(nrm[0]));
                const double e16 = double(__uint_as_float(nrm[1]));
                const double de = double(__uint_as_float(nrm[2]));
                const double u = 0x1p-24, nm = double(d), nf = double(4 * nj + 6);
                const double g_mfma = 2.0 * nm * u / (1.0 - nm * u), g_f32 = nf * u / (1.0 - nf * u);
                const double eps = (e16 * de + e32 * de + g_mfma * e16 * e16 + g_f32 * e32 * e32 +
                                    u * (e16 * e16 * (1.0 + g_mfma) + e32 * e32 * (1.0 + g_f32))) * 1.01 + 1e-30 * nm;
                ok = eps < 1e30 && double(key_score(keys[k_out - 1])) > double(key_score(last)) + eps;
            }
            cert[node] = ok ? 1 : 0;
        }
    }
}

__global__ void k_f32_to_f16_rows(const float* __restrict__ in, __half* __restrict__ out, int64_t count) {
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += int64_t(gridDim.x) * blockDim.x)
        out[i] = __float2half_rn(in[i]);
}

template <int KCH, int K>
int launch_batch_t(const BatchArgs& a, hipStream_t s) {
    const unsigned grid = unsigned(a.n_rranges * a.n_qblocks);
    MARS_LAUNCH((k_batch_scan<KCH, K>), dim3(grid), dim3(kBWaves * 64), 0, s, a);
    return MARS_OK;
}

template <int K>
int launch_batch_k(const BatchArgs& a, hipStream_t s) {
    const bool plain = a.q_plain == 0;
    if (batch_uses_rq(a.q, plain)) return launch_batch_rq(a, s);
    if (batch_uses_gemm(a.q, plain)) return launch_batch_mm(a, s);
    MARS_CHECK(a.floor_keys == nullptr, MARS_ERR_INVALID, "k_batch_scan takes no score floor");
    switch (a.d / 32) {
        case 8: return launch_batch_t<8, K>(a, s);
        case 12: return launch_batch_t<12, K>(a, s);
        case 16: return launch_batch_t<16, K>(a, s);
        case 24: return launch_batch_t<24, K>(a, s);
        default: return set_error(MARS_ERR_UNSUPPORTED, "batched scoring: embedding_dim %d not in {256,384,512,768}", a.d);
    }
}

}  // namespace

bool batch_dim_supported(int32_t d) { return d == 256 || d == 384 || d == 512 || d == 768; }
bool batch_uses_gemm(int32_t q, bool plain) { return plain && q >= kGemmMinQ; }
bool batch_uses_rq(int32_t q, bool plain) { return q > kRqMaxScanQ && !batch_uses_gemm(q, plain); }
int batch_rq_tiles(int32_t q) { return q <= 128 ? 2 : 4; }
int batch_kpart(int32_t k) { return k <= 8 ? 8 : 16; }

int launch_batch_scan(const BatchArgs& a, hipStream_t s) {
    MARS_CHECK(a.k >= 1 && a.k <= 16, MARS_ERR_UNSUPPORTED, "batched scoring keeps at most 16 per query (asked %d)",
               a.k);
    return a.k <= 8 ? launch_batch_k<8>(a, s) : launch_batch_k<16>(a, s);
}

int launch_batch_merge(const uint64_t* part, int32_t n_rranges, int32_t kpart, int32_t q, int32_t k_out,
                       uint64_t* out, hipStream_t s) {
    MARS_CHECK(kpart == 8 || kpart == 16, MARS_ERR_INVALID, "batched merge: %d keys per range", kpart);
    MARS_LAUNCH(k_batch_merge, dim3(unsigned(q)), dim3(kMergeWaves * 64), 0, s, part, n_rranges, kpart, q, k_out, out);
    return MARS_OK;
}

int launch_batch_topk(BatchArgs a, int32_t k_out, uint64_t* out, hipStream_t s, hipEvent_t scanned) {
    MARS_CHECK(k_out >= 1 && k_out <= batch_kpart(a.k), MARS_ERR_INVALID, "batched top-K: %d of %d kept", k_out,
               batch_kpart(a.k));
    const int32_t kp = batch_kpart(a.k);
    a.range_stride = 0;
    a.floor_keys = nullptr;
    a.floor_k = 0;
    // The floor pays where a range is long: without it a query inserts about
    // K (1 + ln(rows / K)) rows per range (every new best of the rows seen so far), with
    // it about rows x K / sampled rows.
    if (a.q > kRqMaxScanQ && a.rows_per_range >= kSampleDiv * kSampleRowsMin) {
        BatchArgs b = a;
        b.rows_per_range = std::min<int64_t>(kSampleRowsMax, a.rows_per_range / kSampleDiv / 16 * 16);
        b.range_stride = a.rows_per_range;
        b.sample_pass = 1;
        MARS_TRY(launch_batch_scan(b, s));
        MARS_TRY(launch_batch_merge(a.part, a.n_rranges, kp, a.q, k_out, out, s));
        a.floor_keys = out;
        a.floor_k = k_out;
    }
    MARS_TRY(launch_batch_scan(a, s));
    if (scanned != nullptr) MARS_HIP(hipEventRecord(scanned, s));
    return launch_batch_merge(a.part, a.n_rranges, kp, a.q, k_out, out, s);
}

int launch_knn_rerank(const float* emb, int64_t q0, int64_t nq, int32_t d, const uint64_t* cand, int32_t kc,
                      int32_t k_out, int32_t* nbrs, hipStream_t s, const uint32_t* nrm, int32_t* cert) {
    MARS_CHECK(d >= 4 && d <= 256 * kRerankPieces && d % 4 == 0, MARS_ERR_UNSUPPORTED,
               "k-NN rescoring: embedding_dim %d not a multiple of 4 up to %d", d, 256 * kRerankPieces);
    const int64_t threads = nq * 64;
    MARS_LAUNCH(k_knn_rerank, dim3(unsigned((threads + 255) / 256)), dim3(256), 0, s, emb, q0, nq, d, cand, kc,
                k_out, nbrs, nrm, cert);
    return MARS_OK;
}

int launch_f32_to_f16_rows(const float* in, __half* out, int64_t count, hipStream_t s) {
    int64_t blocks = (count + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    MARS_LAUNCH(k_f32_to_f16_rows, dim3(unsigned(blocks)), dim3(256), 0, s, in, out, count);
    return MARS_OK;
}

}  // namespace mars
