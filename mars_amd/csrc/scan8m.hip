// ============================================================================
//  scan8m.hip — the int8 candidate scan for up to 16 queries in one pass.
//
//  k_scan8 (scan8.hip) fills two of the sixteen rows of v_mfma_i32_16x16x64_i8's A
//  operand (the query split q = s_hi q_hi + s_lo q_lo + r2); the other fourteen multiply
//  zeros. Here the A operand holds eight queries (rows 2j, 2j + 1 = q_hi, q_lo of query
//  j), and with NA = 2 a second A operand eight more, so one pass over the int8 copy
//  ranks the rows for up to 16 queries: the bytes read per pass do not change, only the
//  epilogue grows (NA MFMAs per 1 KB block instead of one).
//
//  k_split8   one workgroup per query slot (8 NA): k_scan8's query split, written as the
//             A operands' bytes (zero rows for empty slots) and (s_hi, s_lo, tau, |q|).
//  k_scan8m   512 workgroups of 4 waves over 16-row tiles, two tiles in flight per wave
//             (k_scan8's loads). After the MFMAs, lane l holds C rows 4 (l >> 4) .. +3 of
//             tile row l & 15, i.e. queries 2 (l >> 4) and 2 (l >> 4) + 1 of each A
//             operand; it forms their upper-bound keys exactly as k_scan8 does (global
//             queries: decay and modality filter; plain queries, the k-NN of a node:
//             dot only, the node itself excluded) and offers them to 16-lane sorted
//             lists, one per query in each row of the wave (a bitonic sort of the row's
//             candidates, a mirror, a min and a half-cleaner merge). At the end the four
//             waves' lists of each query are sorted together and the 16 best keys go to
//             the query's slot of the workgroup: part[j][16 b ..], as k_scan8 writes.
//
//  Bounds: the keys are the per-row upper bounds of k_scan8 (same split, same per-query
//  tau, same roundings), so k_cert_multi8 certifies the seeds with k_cert_bfs's argument.
//
//  Reference analogue: none — the reference answers one query per call
//  (src/memory_cuda.cu:1351-1464) and scores rows with cublasSgemv.
// ============================================================================
#include "device.hpp"

#include <algorithm>

namespace mars {
namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;

__device__ inline float block_max_split(float v, float* s_red) {
    v = wave_max_f(v);
    __syncthreads();
    if (lane_id() == 0) s_red[threadIdx.x >> 6] = v;
    __syncthreads();
    float m = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) m = fmaxf(m, s_red[w]);
    return m;
}

// Query slot j = blockIdx.x: k_scan8's split of q_j into the A operand image qa
// ([NA][d / 64][64 lanes] x 16 bytes; slot j's rows are 2 (j % 8) and 2 (j % 8) + 1 of
// operand j / 8) and qp[4 j ..] = s_hi, s_lo, tau, |q| (tau and |q| rounded up). Slots
// >= nq write zero rows.
__global__ __launch_bounds__(kThreads) void k_split8(Split8Args a) {
    __shared__ float s_red[kWaves];
    __shared__ double s_sum[kWaves][4];
    const int j = int(blockIdx.x), tid = int(threadIdx.x), lane = lane_id(), wave = tid >> 6;
    const int d = a.d, nk = d >> 6;
    const float* q = j < a.n_glob ? a.q_glob + int64_t(j) * d : a.q_plain + int64_t(j - a.n_glob) * d;
    const bool on = j < a.nq;
    int8_t* qa = static_cast<int8_t*>(a.qa) + int64_t(j >> 3) * nk * 1024;
    const int r = 2 * (j & 7);
    float m1 = 0.0f;
    for (int e = tid; e < d; e += kThreads) m1 = fmaxf(m1, on ? fabsf(q[e]) : 0.0f);
    const float s_hi = block_max_split(m1, s_red) / 127.0f;
    float m2 = 0.0f;
    for (int e = tid; e < d; e += kThreads) {
        const float x = on ? q[e] : 0.0f;
        const float h = s_hi > 0.0f ? fminf(fmaxf(rintf(x / s_hi), -127.0f), 127.0f) : 0.0f;
        m2 = fmaxf(m2, fabsf(fmaf(-s_hi, h, x)));
    }
    const float s_lo = block_max_split(m2, s_red) / 127.0f;
    double sr2 = 0.0, shi = 0.0, slo = 0.0, q2 = 0.0;
    for (int e = tid; e < d; e += kThreads) {
        const float x = on ? q[e] : 0.0f;
        const float h = s_hi > 0.0f ? fminf(fmaxf(rintf(x / s_hi), -127.0f), 127.0f) : 0.0f;
        const float r1 = fmaf(-s_hi, h, x);
        const int32_t qh = int32_t(h);
        const int32_t ql = s_lo > 0.0f ? int32_t(fminf(fmaxf(rintf(r1 / s_lo), -127.0f), 127.0f)) : 0;
        const double hq = double(s_hi) * double(qh), lq = double(s_lo) * double(ql);
        const double r2 = double(x) - hq - lq;
        sr2 += r2 * r2;
        shi += hq * hq;
        slo += lq * lq;
        q2 += double(x) * double(x);
        // chunk e / 64, lane 16 g + row, byte e % 16 (k_scan8's A layout)
        const int64_t blk = int64_t(e >> 6) * 64 + (((e & 63) >> 4) << 4) + r;
        qa[blk * 16 + (e & 15)] = int8_t(qh);
        qa[(blk + 1) * 16 + (e & 15)] = int8_t(ql);
    }
    sr2 = wave_sum_f64(sr2);
    shi = wave_sum_f64(shi);
    slo = wave_sum_f64(slo);
    q2 = wave_sum_f64(q2);
    if (lane == 0) { s_sum[wave][0] = sr2; s_sum[wave][1] = shi; s_sum[wave][2] = slo; s_sum[wave][3] = q2; }
    __syncthreads();
    if (tid == 0) {
        sr2 = shi = slo = q2 = 0.0;
        for (int w = 0; w < kWaves; ++w) {
            sr2 += s_sum[w][0]; shi += s_sum[w][1]; slo += s_sum[w][2]; q2 += s_sum[w][3];
        }
        const double en8 = double(__uint_as_float(a.nrm8[1])) + double(__uint_as_float(a.nrm8[0]));
        const float tau = __uint_as_float(up_bits(en8 * (sqrt(sr2) + 3.1 * 0x1p-24 * (sqrt(shi) + sqrt(slo))) *
                                                  (1.0 + 1e-6) + 1e-30));
        const float qn = __uint_as_float(up_bits(sqrt(q2) * (1.0 + 1e-12)));
        a.qp[4 * j] = s_hi;
        a.qp[4 * j + 1] = s_lo;
        a.qp[4 * j + 2] = tau;
        a.qp[4 * j + 3] = qn;
    }
}

// Ascending sort of one key per lane within each 16-lane row.
__device__ inline uint64_t row_sort16(uint64_t x, int lane) {
    x = cmpx<1>(x, lane, (lane & 2) == 0);
    x = cmpx<2>(x, lane, (lane & 4) == 0);
    x = cmpx<1>(x, lane, (lane & 4) == 0);
    x = cmpx<4>(x, lane, (lane & 8) == 0);
    x = cmpx<2>(x, lane, (lane & 8) == 0);
    x = cmpx<1>(x, lane, (lane & 8) == 0);
    x = cmpx<8>(x, lane, true);
    x = cmpx<4>(x, lane, true);
    x = cmpx<2>(x, lane, true);
    x = cmpx<1>(x, lane, true);
    return x;
}

// Lane 15 - i of the lane's 16-lane row (DPP row_mirror).
__device__ inline uint64_t row_mirror64(uint64_t v) {
    const uint32_t hi = uint32_t(__builtin_amdgcn_mov_dpp(int(uint32_t(v >> 32)), 0x140, 0xF, 0xF, false));
    const uint32_t lo = uint32_t(__builtin_amdgcn_mov_dpp(int(uint32_t(v)), 0x140, 0xF, 0xF, false));
    return (uint64_t(hi) << 32) | lo;
}

// Each 16-lane row keeps the 16 smallest keys it was offered, ascending across its lanes;
// thr = the row's largest kept key (every lane of the row holds it).
__device__ inline void row_offer(uint64_t& list, uint64_t& thr, uint64_t key, int lane) {
    const bool in = key < thr;
    if (__ballot(in) == 0) return;               // wave-uniform
    const uint64_t c = row_sort16(in ? key : kEmptyKey, lane);
    const uint64_t r = row_mirror64(c);
    uint64_t m = list < r ? list : r;            // bitonic: the row's 16 smallest of both
    m = cmpx<8>(m, lane, true);
    m = cmpx<4>(m, lane, true);
    m = cmpx<2>(m, lane, true);
    m = cmpx<1>(m, lane, true);
    list = m;
    thr = __shfl(m, lane | 15);
}

template <int NK, int NA, bool FILTER>
__global__ __launch_bounds__(kThreads) void k_scan8m(Scan8MArgs a) {
    __shared__ i32x4 s_qa[NA][NK][64];
    __shared__ uint64_t s_rows[kWaves][2 * NA][64];
    const int tid = int(threadIdx.x), lane = lane_id(), wave = tid >> 6, m = lane & 15, G = lane >> 4;
    const i32x4* blocks = static_cast<const i32x4*>(a.emb8);
    const f32x2* meta = reinterpret_cast<const f32x2*>(a.meta8);
    const int64_t ntiles = (a.n + 15) / 16;
    const int64_t tstride = int64_t(gridDim.x) * kWaves;
    int64_t t = int64_t(blockIdx.x) * kWaves + wave;
    constexpr int R = 2;
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
    for (int sl = 0; sl < R; ++sl)
        if (t + sl * tstride < ntiles) load_tile(sl, t + sl * tstride);
    // the A operands (written by k_split8) into LDS; this lane's queries' terms
    {
        const i32x4* src = static_cast<const i32x4*>(a.qa);
        i32x4* dst = &s_qa[0][0][0];
        for (int i = tid; i < NA * NK * 64; i += kThreads) dst[i] = src[i];
    }
    float shi[2 * NA], slo[2 * NA], tau[2 * NA], qn[2 * NA], tq[2 * NA];
    int64_t self[2 * NA];
    bool qon[2 * NA], plain[2 * NA];
#pragma unroll
    for (int x = 0; x < 2 * NA; ++x) {
        const int j = 8 * (x >> 1) + 2 * G + (x & 1);
        const f32x4 p = reinterpret_cast<const f32x4*>(a.qp)[j];
        shi[x] = p.x; slo[x] = p.y; tau[x] = p.z; qn[x] = p.w;
        qon[x] = j < a.nq;
        plain[x] = j >= a.n_glob;
        tq[x] = (qon[x] && !plain[x]) ? (a.tq ? a.tq[j] : a.tq_value) : 0.0f;
        self[x] = plain[x] ? a.self_base + (j - a.n_glob) : -1;
    }
    __syncthreads();
    uint64_t list[2 * NA], thr[2 * NA];
#pragma unroll
    for (int x = 0; x < 2 * NA; ++x) { list[x] = kEmptyKey; thr[x] = kEmptyKey; }
    for (int64_t t0 = t; t0 < ntiles; t0 += R * tstride)
#pragma unroll
    for (int sl = 0; sl < R; ++sl) {
        const int64_t tt = t0 + sl * tstride;
        if (tt >= ntiles) break;                 // uniform over the wave
        const f32x2 cmt = mt[sl];
        const float cts = tsv[sl];
        const int32_t cmod = modv[sl];
        i32x4 acc[NA];
#pragma unroll
        for (int q = 0; q < NA; ++q) acc[q] = i32x4{0, 0, 0, 0};
#pragma unroll
        for (int i0 = 0; i0 < NK; i0 += 4) {
#pragma unroll
            for (int i = i0; i < i0 + 4 && i < NK; ++i)
#pragma unroll
                for (int q = 0; q < NA; ++q)
                    acc[q] = __builtin_amdgcn_mfma_i32_16x16x64_i8(s_qa[q][i][lane], b[sl][i], acc[q], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (tt + R * tstride < ntiles) load_tile(sl, tt + R * tstride);
        __builtin_amdgcn_sched_barrier(0);
        const int64_t r = tt * 16 + m;
        const bool row_ok = r < a.n;
#pragma unroll
        for (int x = 0; x < 2 * NA; ++x) {
            const int32_t hi = acc[x >> 1][2 * (x & 1)], lo = acc[x >> 1][2 * (x & 1) + 1];
            // k_scan8's arithmetic: the dot, then the upper bound raised past its roundings
            const float dot = fmaf(slo[x], float(lo), shi[x] * float(hi)) * cmt.x;
            float up = fmaf(qn[x], cmt.y, dot) + tau[x];
            up = up + fmaxf(fabsf(up) * 0x1p-20f, 1e-35f);
            float su;
            if (plain[x]) {
                su = up;
            } else {
                const bool out = FILTER && cmod != a.mod_filter;
                const float w = expf(-a.lambda * fmaxf(0.0f, tq[x] - cts));
                su = out ? -FLT_MAX : up * w;
            }
            const bool valid = row_ok && qon[x] && r != self[x];
            row_offer(list[x], thr[x], valid ? make_key(su, uint32_t(r)) : kEmptyKey, lane);
        }
    }
#pragma unroll
    for (int x = 0; x < 2 * NA; ++x) s_rows[wave][x][lane] = list[x];
    __syncthreads();
    // query j's lists: row (j % 8) / 2 of list slot 2 (j / 8) + (j % 2) in each wave
    for (int j = wave; j < a.nq; j += kWaves) {
        const int x = 2 * (j >> 3) + (j & 1), row = (j & 7) >> 1;
        const uint64_t v = s_rows[lane >> 4][x][16 * row + (lane & 15)];
        const uint64_t srt = wave_sort64(v, lane);
        if (lane < kScan8List)
            a.part[int64_t(j) * kScan8MaxLists * kScan8List + int64_t(blockIdx.x) * kScan8List + lane] = srt;
    }
}

template <int NK, int NA>
int launch_scan8m_t(const Scan8MArgs& a, hipStream_t s) {
    const dim3 grid(unsigned(a.num_wg)), block(kThreads);
    if (a.mod_filter >= 0) MARS_LAUNCH((k_scan8m<NK, NA, true>), grid, block, 0, s, a);
    else MARS_LAUNCH((k_scan8m<NK, NA, false>), grid, block, 0, s, a);
    return MARS_OK;
}

template <int NK>
int launch_scan8m_na(const Scan8MArgs& a, int na, hipStream_t s) {
    return na == 1 ? launch_scan8m_t<NK, 1>(a, s) : launch_scan8m_t<NK, 2>(a, s);
}

}  // namespace

int launch_split8(const Split8Args& a, hipStream_t s) {
    MARS_CHECK(a.na >= 1 && a.na <= kScan8MMaxA && a.nq >= 1 && a.nq <= 8 * a.na && a.n_glob >= 0 &&
                   a.n_glob <= a.nq && a.d % 64 == 0,
               MARS_ERR_INVALID, "int8 query split: %d queries in %d operands", a.nq, a.na);
    MARS_LAUNCH(k_split8, dim3(unsigned(8 * a.na)), dim3(kThreads), 0, s, a);
    return MARS_OK;
}

int launch_scan8m(const Scan8MArgs& a, int na, hipStream_t s) {
    MARS_CHECK(na >= 1 && na <= kScan8MMaxA && a.nq >= 1 && a.nq <= 8 * na, MARS_ERR_INVALID,
               "int8 multi-query scan: %d queries in %d operands", a.nq, na);
    MARS_CHECK(a.num_wg >= 1 && a.num_wg <= kScan8MaxLists, MARS_ERR_INVALID, "int8 scan: %d workgroups",
               a.num_wg);
    switch (a.d) {
        case 256: return launch_scan8m_na<4>(a, na, s);
        case 512: return launch_scan8m_na<8>(a, na, s);
        case 768: return launch_scan8m_na<12>(a, na, s);
        case 1024: return launch_scan8m_na<16>(a, na, s);
        default: break;
    }
    return set_error(MARS_ERR_UNSUPPORTED, "int8 multi-query scan: embedding_dim %d", a.d);
}

}  // namespace mars
