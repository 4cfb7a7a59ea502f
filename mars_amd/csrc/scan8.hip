// ============================================================================
//  scan8.hip — the int8 candidate scan of the certified global query.
//
//  The certified query (MARS_CTX_CERTIFIED) needs, for every row, a cheap score and a
//  bound on its distance to the fp32 scan's score. Here the rows are read from an int8
//  copy (one byte per element, one fp32 scale per row: half the bytes of the fp16
//  copy, a quarter of the fp32 rows) and each row carries its own bound c_r (from its
//  quantisation residual and the two scans' rounding), so the scan ranks rows by an
//  upper bound of the fp32 scan's fused score,
//      U_r = fuse(dot8_r + |q| c_r + tau)  >=  fuse(dot32_r),
//  (fuse = dot * exp(-lambda age) is monotone in dot for the same row), and keeps the
//  64 best keys of U. k_cert_bfs rescores those candidates exactly: when the K-th exact
//  score beats the 64th candidate's U, no other row can reach the top K. Ranking by the
//  per-row bound instead of one global bound is what makes 64 candidates enough: rows
//  with large elements (coarse scales) are the only ones that pay for them.
//
//  k_scan8     the scan, on MFMA: the copy is tiled in blocks of 16 rows x 64 bytes
//              (i8_offset), each block one 1 KB load instruction and the B operand of
//              one v_mfma_i32_16x16x64_i8. The query is split into two int8 parts,
//              q = s_hi q_hi + s_lo q_lo + r2 (|r2| ~ 1e-4 |q|), the A operand's first two
//              rows, so the products are summed exactly in int32 and the row's dot is
//              s_r (s_hi A_hi + s_lo A_lo) in three fp32 operations; r2 and those three
//              roundings enter the bound as one per-query term tau. Lanes 0-15 of the
//              wave then hold one row each: fin[r] gets the estimate fuse(dot8) (within
//              |q| max c + tau of the exact score, used by the interval BFS); the key is
//              U_r. Each workgroup writes its 16 best keys to a slot of its own,
//              part[16 b ..] (no running bound: the workgroups finish together, so one
//              would filter little); k_cert_bfs merges them into the 64 candidates and
//              bounds the rows a list dropped by the smallest 16th key. (Rows are dealt
//              to the workgroups in blocks of 128 consecutive ids; on the benchmark corpus,
//              16 per workgroup certify as often as 64 would.)
//  k_convert_i8  one wave per row, the row read once: scale, bytes, c_r (quantize_row_i8's
//              arithmetic), and the maxima raised once per wave.
//
//  Reference analogue: none — the reference scores fp32 (cublasSgemv) or fp16 rows
//  (src/memory_cuda.cu:1207-1215, :155-201); the results here are its fp32 path's.
// ============================================================================
#include "device.hpp"

#include <algorithm>

namespace mars {
namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// 4 waves per workgroup, one tile of 16 rows per wave and step (d / 64 loads of 1 KB in
// flight, the next tile's issued before the current tile's scores are fused): 512
// workgroups put 2 waves on every SIMD of 256 CUs, with room beside them for a wave of
// another kernel (inserts, episode queries).
constexpr int kScan8Waves = 4;
constexpr int kScan8Ring = 2;
constexpr int kScan8Threads = kScan8Waves * 64;

// Block reductions of the query split (every thread gets the result).
__device__ inline float block_max8(float v, float* s_red) {
    v = wave_max_f(v);
    __syncthreads();                             // s_red free
    if (lane_id() == 0) s_red[threadIdx.x >> 6] = v;
    __syncthreads();
    float m = 0.0f;
#pragma unroll
    for (int w = 0; w < kScan8Waves; ++w) m = fmaxf(m, s_red[w]);
    return m;
}

// NK = d / 64 k-chunks. FILTER: the query has a modality filter (mods are read). The
// certified query never has a same-episode boost (ScanArgs boost = 0, query_ep = -1).
template <int NK, bool FILTER>
__global__ __launch_bounds__(kScan8Threads) void k_scan8(ScanArgs a) {
    __shared__ uint64_t s_lists[kScan8Waves][64];
    __shared__ i32x4 s_qa[NK][64];               // A operand per k-chunk: rows 0 / 1 = q_hi / q_lo
    __shared__ float s_red[kScan8Waves];
    __shared__ double s_sum[kScan8Waves][4];
    constexpr int D = NK * 64;
    constexpr int kPer = (D + kScan8Threads - 1) / kScan8Threads;
    const int tid = int(threadIdx.x), lane = lane_id(), wave = tid >> 6, m = lane & 15;
    const int k = a.k;
    const i32x4* blocks = static_cast<const i32x4*>(a.emb);        // 64 x 16 bytes per block
    const f32x2* meta = reinterpret_cast<const f32x2*>(a.meta8);
    const int64_t ntiles = (a.n + 15) / 16;
    const int64_t tstride = int64_t(gridDim.x) * kScan8Waves;
    int64_t t = int64_t(blockIdx.x) * kScan8Waves + wave;
    // kScan8Ring tiles in flight: a tile's row blocks and its rows' scale, bound, time and
    // modality (lane m: row 16 t + m)
    constexpr int R = NK <= 16 ? kScan8Ring : 1;  // d = 1536: one (the registers of two exceed a SIMD's share)
    i32x4 b[R][NK];
    f32x2 mt[R];
    float tsv[R];
    int32_t modv[R];
    auto load_tile = [&](int sl, int64_t tt) {
        int64_t rr = tt * 16 + m;
        rr = rr < a.n ? rr : a.n - 1;
        mt[sl] = meta[rr];
        tsv[sl] = a.ts[rr];
        modv[sl] = FILTER ? a.mods[rr] : 0;
        const i32x4* p = blocks + tt * NK * 64 + lane;
#pragma unroll
        for (int i = 0; i < NK; ++i) b[sl][i] = __builtin_nontemporal_load(p + i * 64);
    };
#pragma unroll
    for (int sl = 0; sl < R; ++sl)                // in flight while the query is split
        if (t + sl * tstride < ntiles) load_tile(sl, t + sl * tstride);
    // ---- q = s_hi q_hi + s_lo q_lo + r2, q_hi and q_lo in [-127, 127]
    float qv[kPer];
    float m1 = 0.0f;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int e = tid + j * kScan8Threads;
        qv[j] = e < D ? a.q[e] : 0.0f;
        m1 = fmaxf(m1, fabsf(qv[j]));
    }
    const float s_hi = block_max8(m1, s_red) / 127.0f;
    int32_t qh[kPer], ql[kPer];
    float r1[kPer];
    float m2 = 0.0f;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const float h = s_hi > 0.0f ? fminf(fmaxf(rintf(qv[j] / s_hi), -127.0f), 127.0f) : 0.0f;
        qh[j] = int32_t(h);
        r1[j] = fmaf(-s_hi, h, qv[j]);
        m2 = fmaxf(m2, fabsf(r1[j]));
    }
    const float s_lo = block_max8(m2, s_red) / 127.0f;
    double sr2 = 0.0, shi = 0.0, slo = 0.0, q2 = 0.0;
    int8_t* qa = reinterpret_cast<int8_t*>(&s_qa[0][0]);
    for (int i = tid; i < NK * 64 * 4; i += kScan8Threads) reinterpret_cast<int32_t*>(qa)[i] = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int e = tid + j * kScan8Threads;
        if (e < D) {
            ql[j] = s_lo > 0.0f ? int32_t(fminf(fmaxf(rintf(r1[j] / s_lo), -127.0f), 127.0f)) : 0;
            const double hq = double(s_hi) * double(qh[j]), lq = double(s_lo) * double(ql[j]);
            const double r2 = double(qv[j]) - hq - lq;
            sr2 += r2 * r2;
            shi += hq * hq;
            slo += lq * lq;
            q2 += double(qv[j]) * double(qv[j]);
            // chunk e / 64, lane 16 g + row (0: q_hi, 1: q_lo), byte e % 16
            const int blk = (e >> 6) * 64 + (((e & 63) >> 4) << 4);
            qa[size_t(blk) * 16 + (e & 15)] = int8_t(qh[j]);
            qa[size_t(blk + 1) * 16 + (e & 15)] = int8_t(ql[j]);
        }
    }
    sr2 = wave_sum_f64(sr2);
    shi = wave_sum_f64(shi);
    slo = wave_sum_f64(slo);
    q2 = wave_sum_f64(q2);
    if (lane == 0) { s_sum[wave][0] = sr2; s_sum[wave][1] = shi; s_sum[wave][2] = slo; s_sum[wave][3] = q2; }
    __syncthreads();
    sr2 = shi = slo = q2 = 0.0;
#pragma unroll
    for (int w = 0; w < kScan8Waves; ++w) {
        sr2 += s_sum[w][0]; shi += s_sum[w][1]; slo += s_sum[w][2]; q2 += s_sum[w][3];
    }
    // |q| rounded up
    const float qn = __uint_as_float(up_bits(sqrt(q2) * (1.0 + 1e-12)));
    // tau: |e^_r| (|r2| + 3.1 u (|q_hi| + |q_lo|)) with |e^_r| <= max |e| + max c_r
    const double en8 = double(__uint_as_float(a.nrm8[1])) + double(__uint_as_float(a.nrm8[0]));
    const float tau = __uint_as_float(up_bits(en8 * (sqrt(sr2) + 3.1 * 0x1p-24 * (sqrt(shi) + sqrt(slo))) *
                                              (1.0 + 1e-6) + 1e-30));
    if (blockIdx.x == 0 && tid == 0) a.part[int64_t(kScan8MaxLists) * kScan8List] = uint64_t(__float_as_uint(tau));
    uint64_t list = kEmptyKey, thr = kEmptyKey;
    for (int64_t t0 = t; t0 < ntiles; t0 += R * tstride)
#pragma unroll
    for (int sl = 0; sl < R; ++sl) {
        const int64_t t = t0 + sl * tstride;
        if (t >= ntiles) break;                  // uniform over the wave
        const f32x2 cmt = mt[sl];
        const float cts = tsv[sl];
        const int32_t cmod = modv[sl];
        i32x4 acc = i32x4{0, 0, 0, 0};
        // A fragments read from LDS four chunks ahead at most (16 VGPRs), not all at once
#pragma unroll
        for (int i0 = 0; i0 < NK; i0 += 4) {
#pragma unroll
            for (int i = i0; i < i0 + 4 && i < NK; ++i)
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(s_qa[i][lane], b[sl][i], acc, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        // the slot's next tile (R strides on) reuses its registers once the MFMAs read them
        if (t + R * tstride < ntiles) load_tile(sl, t + R * tstride);
        __builtin_amdgcn_sched_barrier(0);
        // lanes 0-15: C[0][m] = q_hi . row m, C[1][m] = q_lo . row m (exact int32 sums)
        const int64_t r = t * 16 + m;
        const bool valid = lane < 16 && r < a.n;
        const float dot = fmaf(s_lo, float(acc[1]), s_hi * float(acc[0])) * cmt.x;
        // dot + |q| c_r + tau, then raised past the roundings (and any underflow)
        float up = fmaf(qn, cmt.y, dot) + tau;
        up = up + fmaxf(fabsf(up) * 0x1p-20f, 1e-35f);
        // fuse_score's arithmetic with one exp: the filter, then dot * w
        const bool out = FILTER && cmod != a.mod_filter;
        const float w = decay_weight(cts, a);
        const float s8 = out ? -FLT_MAX : dot * w;
        const float su = out ? -FLT_MAX : up * w;
        if (valid) a.fin[r] = s8;
        const uint64_t key = valid ? make_key(su, uint32_t(a.id_base + r)) : kEmptyKey;
        list_offer(list, thr, key, valid, lane, k);
    }
    s_lists[wave][lane] = list;
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int w = 1; w < kScan8Waves; ++w) list = wave_merge64(list, s_lists[w][lane], lane, k);
        if (lane < kScan8List) a.part[int64_t(blockIdx.x) * kScan8List + lane] = list;
    }
}

// quantize_row_i8's arithmetic in one read of each row: one wave per row (grid-stride),
// lane l holding elements [16 g, 16 g + 16) for g = l and g = l + 64 (d a multiple of 16,
// at most 2048) as four 16-byte loads each; a group's 16 bytes are one 16-byte store into
// the tiled copy. The wave keeps the largest c_r and |e| of its rows and raises nrm8 once
// (an atomic per row on the same two words serialises the whole pass).
__global__ __launch_bounds__(256) void k_convert_i8(const float* __restrict__ emb, int64_t r0, int64_t r1, int32_t d,
                                                    int8_t* __restrict__ emb8, float* __restrict__ meta8,
                                                    uint32_t* __restrict__ nrm8) {
    const int wave = int(threadIdx.x >> 6), lane = lane_id();
    const int ng = d >> 4;
    uint32_t cmax = 0u, nmax = 0u;
    for (int64_t row = r0 + int64_t(blockIdx.x) * 4 + wave; row < r1; row += int64_t(gridDim.x) * 4) {
        f32x4 x[2][4];
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int g = lane + 64 * j;
            const f32x4* p = reinterpret_cast<const f32x4*>(emb + row * d + 16 * int64_t(g));
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                x[j][v] = g < ng ? __builtin_nontemporal_load(p + v) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                m = fmaxf(fmaxf(m, fabsf(x[j][v].x)), fabsf(x[j][v].y));
                m = fmaxf(fmaxf(m, fabsf(x[j][v].z)), fabsf(x[j][v].w));
            }
        }
        const float s = wave_max_f(m) / 127.0f;
        int8_t* tile = emb8 + i8_offset(row, 0, d);
        double s32 = 0.0, s8 = 0.0, sd = 0.0;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int g = lane + 64 * j;
            if (g >= ng) continue;
            uint32_t w[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float xs[4] = {x[j][v].x, x[j][v].y, x[j][v].z, x[j][v].w};
                uint32_t word = 0u;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    // I8Row::put's arithmetic
                    float t = s > 0.0f ? rintf(xs[b] / s) : 0.0f;
                    t = fminf(fmaxf(t, -127.0f), 127.0f);
                    const int vi = int(t);
                    word |= uint32_t(uint8_t(int8_t(vi))) << (8 * b);
                    const double eh = double(s) * double(vi);
                    s32 += double(xs[b]) * double(xs[b]);
                    s8 += eh * eh;
                    const double df = eh - double(xs[b]);
                    sd += df * df;
                }
                w[v] = word;
            }
            const int i0 = 16 * g;
            *reinterpret_cast<u32x4*>(tile + ((i0 >> 6) << 10) + (((i0 & 63) >> 4) << 8)) = u32x4{w[0], w[1], w[2], w[3]};
        }
        s32 = wave_sum_f64(s32);
        s8 = wave_sum_f64(s8);
        sd = wave_sum_f64(sd);
        const double c = (sqrt(sd) + i8_gamma(d) * (sqrt(s8) + sqrt(s32))) * (1.0 + 1e-9);
        const uint32_t cb = up_bits(c), nb = up_bits(sqrt(s32));
        if (lane == 0) {
            meta8[2 * row] = s;
            meta8[2 * row + 1] = __uint_as_float(cb);
        }
        cmax = cb > cmax ? cb : cmax;
        nmax = nb > nmax ? nb : nmax;
    }
    if (lane == 0 && (cmax | nmax)) {
        atomicMax(nrm8 + 0, cmax);
        atomicMax(nrm8 + 1, nmax);
    }
}

template <int NK>
int launch_scan8_t(const ScanArgs& a, hipStream_t s) {
    const dim3 grid(unsigned(a.num_wg)), block(kScan8Threads);
    if (a.mod_filter >= 0) MARS_LAUNCH((k_scan8<NK, true>), grid, block, 0, s, a);
    else MARS_LAUNCH((k_scan8<NK, false>), grid, block, 0, s, a);
    return MARS_OK;
}

}  // namespace

bool scan8_dim_supported(int32_t d) {
    if (d <= 0 || d % 256 != 0) return false;
    const int nch = d / 256;
    return nch == 1 || nch == 2 || nch == 3 || nch == 4 || nch == 6;
}

int launch_scan8(const ScanArgs& a, hipStream_t s) {
    MARS_CHECK(a.k == kScan8List, MARS_ERR_INVALID, "int8 scan keeps %d keys per workgroup (asked %d)", kScan8List,
               a.k);
    MARS_CHECK(a.boost == 0.0f && a.query_ep < 0, MARS_ERR_INVALID, "int8 scan: no same-episode boost");
    MARS_CHECK(a.num_wg >= 1 && a.num_wg <= kScan8MaxLists, MARS_ERR_INVALID, "int8 scan: %d workgroups", a.num_wg);
    MARS_CHECK(a.nrm8 != nullptr, MARS_ERR_INVALID, "int8 scan: no row bounds");
    switch (scan8_dim_supported(a.d) ? a.d / 64 : 0) {
        case 4: return launch_scan8_t<4>(a, s);
        case 8: return launch_scan8_t<8>(a, s);
        case 12: return launch_scan8_t<12>(a, s);
        case 16: return launch_scan8_t<16>(a, s);
        case 24: return launch_scan8_t<24>(a, s);
        default: break;
    }
    return set_error(MARS_ERR_UNSUPPORTED, "int8 scan: embedding_dim %d is not 256, 512, 768, 1024 or 1536", a.d);
}

int launch_convert_i8(const float* emb, int64_t r0, int64_t r1, int32_t d, int8_t* emb8, float* meta8,
                      uint32_t* nrm8, hipStream_t s) {
    if (r1 <= r0) return MARS_OK;
    MARS_CHECK(d % 16 == 0 && d <= 2048, MARS_ERR_UNSUPPORTED, "int8 copy: embedding_dim %d", d);
    const int64_t blocks = std::min<int64_t>((r1 - r0 + 3) / 4, 4096);
    MARS_LAUNCH(k_convert_i8, dim3(unsigned(blocks)), dim3(256), 0, s, emb, r0, r1, d, emb8, meta8, nrm8);
    return MARS_OK;
}

}  // namespace mars
