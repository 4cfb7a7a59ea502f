// ============================================================================
//  scan8.hip — the int8 candidate scan of the certified global query.
//
//  The certified query (MARS_CTX_CERTIFIED) needs, for every row, a cheap score and a
//  bound on its distance to the fp32 scan's score. Here the rows are read from an int8
//  copy (one byte per element, one fp32 scale per row: half the bytes of the fp16
//  copy, a quarter of the fp32 rows) and each row carries its own bound c_r (from its
//  quantisation residual and the two scans' rounding), so the scan ranks rows by an
//  upper bound of the fp32 scan's fused score,
//      U_r = fuse(dot8_r + |q| c_r)  >=  fuse(dot32_r),
//  (fuse = dot * exp(-lambda age) is monotone in dot for the same row), and keeps the
//  64 best keys of U. k_cert_bfs rescores those candidates exactly: when the K-th exact
//  score beats the 64th candidate's U, no other row can reach the top K. Ranking by the
//  per-row bound instead of one global bound is what makes 64 candidates enough: rows
//  with large elements (coarse scales) are the only ones that pay for them.
//
//  k_scan8     the scan: k_scan's 16-lane row layout (lane s of a group reads bytes
//              16s .. 16s+15 of each 256-byte chunk of its row), signed bytes
//              converted with one v_cvt_f32_i32 (SDWA byte select) each, fp32 fmaf
//              chain against the query in LDS, the 16-lane reduction, then the row scale. fin[r] gets the int8
//              estimate fuse(dot8) (within |q| max c_r of the exact score, used by the
//              interval BFS); the key is U_r. Each workgroup writes its 16 best keys to a
//              slot of its own, part[16 b ..] (no running bound: the workgroups finish
//              together, so one would filter little); k_cert_bfs merges them into the 64
//              candidates and bounds the rows a list dropped by the smallest 16th key.
//              (Rows are dealt to the workgroups in blocks of 64 consecutive ids; on the
//              benchmark corpus, 16 per workgroup certify as often as 64 would.)
//  k_convert_i8  one wave per row: scale, bytes, c_r and the maxima (quantize_row_i8).
//
//  Reference analogue: none — the reference scores fp32 (cublasSgemv) or fp16 rows
//  (src/memory_cuda.cu:1207-1215, :155-201); the results here are its fp32 path's.
// ============================================================================
#include "device.hpp"

#include <algorithm>

namespace mars {
namespace {

// 8 waves per workgroup and 2 row groups of 4 rows per wave and step: 100 VGPRs at d = 768,
// so 512 workgroups keep 4 waves on every SIMD and leave room for a wave of another kernel
// (1M x 768 rows on MI355X: 133 us; 145 us with 4 waves x 4 groups per workgroup, 2 waves
// per SIMD; 162 us with one group per wave; 127 us with the query in registers, which
// fills the SIMDs: a streaming insert's publication then waits for the scan, 150 us at p99
// instead of 65).
constexpr int kScan8Waves = 8;
constexpr int kScan8Unroll = 2;

// int8 rows: chunk c covers bytes [256c, 256c + 256); lane s of a 16-lane group reads the
// 16 bytes 256c + 16s .. + 15 of its row and multiplies them with the query floats of the
// same index, which the workgroup keeps in LDS (s_q[64 c + 4 s + j] = floats 256c + 16s +
// 4j .. + 3) and reads one chunk at a time: 16 query registers per lane instead of d / 16,
// which keeps the scan under 96 VGPRs so that other kernels (inserts, episode queries)
// still find room on a SIMD beside its 4 waves.
template <int NCH>
__device__ inline void fetch8(const int8_t* row, int sub, u32x4 (&x)[NCH]) {
    const u32x4* r = reinterpret_cast<const u32x4*>(row) + sub;
#pragma unroll
    for (int c = 0; c < NCH; ++c) x[c] = __builtin_nontemporal_load(r + c * 16);
}

// Per-lane partial dots of U rows (the fmaf chain over the lane's bytes in index order).
template <int NCH, int U>
__device__ inline void dot8(const f32x4* s_q, int sub, const u32x4 (&x)[U][NCH], float (&acc)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) acc[u] = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        f32x4 qv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) qv[j] = s_q[64 * c + 4 * sub + j];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t w[4] = {x[u][c].x, x[u][c].y, x[u][c].z, x[u][c].w};
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    acc[u] = fmaf(float(int8_t(w[j] >> (8 * b))), qv[j][b], acc[u]);
        }
    }
}

// FILTER: the query has a modality filter (mods are read). The certified query never
// has a same-episode boost (ScanArgs boost = 0, query_ep = -1).
template <int NCH, bool FILTER>
__global__ __launch_bounds__(kScan8Waves * 64) void k_scan8(ScanArgs a) {
    __shared__ uint64_t s_lists[kScan8Waves][64];
    __shared__ f32x4 s_q[NCH * 64];
    const int lane = lane_id(), wave = int(threadIdx.x >> 6);
    const int sub = lane & 15, grp = lane >> 4;
    const int k = a.k;
    for (int i = int(threadIdx.x); i < NCH * 64; i += kScan8Waves * 64) {
        // s_q[64 c + 4 s + j] = query floats 256c + 16s + 4j .. + 3: the same as float4 i
        s_q[i] = reinterpret_cast<const f32x4*>(a.q)[i];
    }
    __syncthreads();
    // |q| rounded up to fp32 (each 16-lane group sums the whole query)
    double q2 = 0.0;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const f32x4 v = s_q[64 * c + 4 * sub + j];
            q2 += double(v.x) * double(v.x) + double(v.y) * double(v.y) + double(v.z) * double(v.z) +
                  double(v.w) * double(v.w);
        }
    const float qn = __uint_as_float(up_bits(sqrt(row16_sum_f64(q2)) * (1.0 + 1e-12)));
    const int8_t* emb = static_cast<const int8_t*>(a.emb);
    const f32x2* meta = reinterpret_cast<const f32x2*>(a.meta8);
    uint64_t list = kEmptyKey, thr = kEmptyKey;
    const int64_t ngroups = (a.n + 3) / 4;
    const int64_t gstride = int64_t(gridDim.x) * kScan8Waves * kScan8Unroll;
    for (int64_t g0 = (int64_t(blockIdx.x) * kScan8Waves + wave) * kScan8Unroll; g0 < ngroups; g0 += gstride) {
        u32x4 x[kScan8Unroll][NCH];
        f32x2 mt[kScan8Unroll];
        float ts[kScan8Unroll];
        int32_t mod[kScan8Unroll];
#pragma unroll
        for (int u = 0; u < kScan8Unroll; ++u) {
            int64_t rr = (g0 + u) * 4 + grp;
            rr = rr < a.n ? rr : a.n - 1;
            ts[u] = a.ts[rr];
            mt[u] = meta[rr];
            mod[u] = FILTER ? a.mods[rr] : 0;
            fetch8<NCH>(emb + rr * a.d, sub, x[u]);
        }
        float acc[kScan8Unroll];
        dot8<NCH, kScan8Unroll>(s_q, sub, x, acc);
#pragma unroll
        for (int u = 0; u < kScan8Unroll; ++u) {
            const int64_t r = (g0 + u) * 4 + grp;
            const bool valid = r < a.n;
            const float dot = row16_sum(acc[u]) * mt[u].x;
            // dot + |q| c_r, then raised past the fmaf's rounding (and any underflow)
            float up = fmaf(qn, mt[u].y, dot);
            up = up + fmaxf(fabsf(up) * 0x1p-20f, 1e-35f);
            // fuse_score's arithmetic with one exp: the filter, then dot * w
            const bool out = FILTER && mod[u] != a.mod_filter;
            const float w = decay_weight(ts[u], a);
            const float s8 = out ? -FLT_MAX : dot * w;
            const float su = out ? -FLT_MAX : up * w;
            if (valid && sub == 0) a.fin[r] = s8;
            const uint64_t key = valid ? make_key(su, uint32_t(a.id_base + r)) : kEmptyKey;
            list_offer(list, thr, key, sub == 0, lane, k);
        }
    }
    s_lists[wave][lane] = list;
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int w = 1; w < kScan8Waves; ++w) list = wave_merge64(list, s_lists[w][lane], lane, k);
        if (lane < kScan8List) a.part[int64_t(blockIdx.x) * kScan8List + lane] = list;
    }
}

__global__ __launch_bounds__(256) void k_convert_i8(const float* __restrict__ emb, int64_t r0, int64_t r1, int32_t d,
                                                    int8_t* __restrict__ emb8, float* __restrict__ meta8,
                                                    uint32_t* __restrict__ nrm8) {
    const int wave = int(threadIdx.x >> 6);
    for (int64_t row = r0 + int64_t(blockIdx.x) * 4 + wave; row < r1; row += int64_t(gridDim.x) * 4)
        quantize_row_i8(emb + row * d, d, emb8 + row * d, meta8 + 2 * row, nrm8);
}

template <int NCH>
int launch_scan8_t(const ScanArgs& a, hipStream_t s) {
    const dim3 grid(unsigned(a.num_wg)), block(kScan8Waves * 64);
    if (a.mod_filter >= 0) MARS_LAUNCH((k_scan8<NCH, true>), grid, block, 0, s, a);
    else MARS_LAUNCH((k_scan8<NCH, false>), grid, block, 0, s, a);
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
    switch (scan8_dim_supported(a.d) ? a.d / 256 : 0) {
        case 1: return launch_scan8_t<1>(a, s);
        case 2: return launch_scan8_t<2>(a, s);
        case 3: return launch_scan8_t<3>(a, s);
        case 4: return launch_scan8_t<4>(a, s);
        case 6: return launch_scan8_t<6>(a, s);
        default: break;
    }
    return set_error(MARS_ERR_UNSUPPORTED, "int8 scan: embedding_dim %d is not 256, 512, 768, 1024 or 1536", a.d);
}

int launch_convert_i8(const float* emb, int64_t r0, int64_t r1, int32_t d, int8_t* emb8, float* meta8,
                      uint32_t* nrm8, hipStream_t s) {
    if (r1 <= r0) return MARS_OK;
    const int64_t blocks = std::min<int64_t>((r1 - r0 + 3) / 4, 4096);
    MARS_LAUNCH(k_convert_i8, dim3(unsigned(blocks)), dim3(256), 0, s, emb, r0, r1, d, emb8, meta8, nrm8);
    return MARS_OK;
}

}  // namespace mars
