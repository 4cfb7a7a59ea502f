// ============================================================================
//  multi.hip — batched global queries: Q global queries answered with one shared
//  fp16 MFMA scan of the corpus, each with the results the Q=1 global path gives.
//
//  1. The batched scan (batch.hip) keeps the C = 16 best fp16 keys per query.
//  2. k_multi_seed rescores the C candidates with the Q=1 scan's own arithmetic
//     (QF32 / QF16 dot in the same 16-lane layout, the same reduction and
//     fuse_score), sorts them and takes the K best as seeds, then certifies
//     them: every row outside the candidates has an fp16 score at most the C-th
//     candidate's, and its exact score exceeds its fp16 score by at most
//         eps = |e16|max |q16 - q| + |e16 - e|max |q| + accumulation terms,
//     so when the K-th exact seed beats (C-th fp16 score + eps) no other row can
//     enter the top K: the seeds are exactly the Q=1 scan's. Queries that miss
//     the certificate are answered by the Q=1 path.
//  3. k_multi_bfs (kernels.hip) runs the finalize kernel's LDS BFS without scores
//     (the visit order, hops and parents do not depend on them), k_visit_scores
//     computes the exact fused score of every visited node in parallel over the
//     whole batch, and k_multi_select propagates the BFS scores level by level in
//     the finalize kernel's arithmetic and writes the sorted results.
//
//  k_row_norms / k_query_norms give the norms the bound needs. Row norms are
//  kept per graph (maxima, raised as rows are converted to fp16); query norms are
//  computed per batch. Both in fp64, the row maxima rounded up to fp32.
//
//  Reference analogue: none — query_memory_fast (src/memory_cuda.cu:1351-1464)
//  answers one query per call; the results of each query here are that path's.
// ============================================================================
#include "device.hpp"

namespace mars {
namespace {

// One wave per row: |e|^2, |e16|^2 and |ftz(e16) - e|^2 in fp64; the block's maxima
// raise nrm[0..2] (fp32 bits of non-negative values order as unsigned integers).
__global__ __launch_bounds__(256) void k_row_norms(const float* __restrict__ emb, const __half* __restrict__ emb16,
                                                  int64_t r0, int64_t r1, int32_t d, uint32_t* nrm) {
    const int lane = int(threadIdx.x & 63u), wave = int(threadIdx.x >> 6);
    double m32 = 0.0, m16 = 0.0, md = 0.0;
    for (int64_t row = r0 + int64_t(blockIdx.x) * 4 + wave; row < r1; row += int64_t(gridDim.x) * 4) {
        double s32 = 0.0, s16 = 0.0, sd = 0.0;
        const float* e = emb + row * d;
        const __half* h = emb16 + row * d;
        for (int i = lane; i < d; i += 64) {
            const float x = e[i];
            const float hv = __half2float(h[i]);
            const float hf = fabsf(hv) < kHalfMinNormal ? 0.0f : hv;
            s32 += double(x) * double(x);
            s16 += double(hv) * double(hv);
            const double df = double(hf) - double(x);
            sd += df * df;
        }
        m32 = max_nan(m32, wave_sum_f64(s32));
        m16 = max_nan(m16, wave_sum_f64(s16));
        md = max_nan(md, wave_sum_f64(sd));
    }
    if (lane == 0) {
        atomicMax(nrm + 0, up_bits(sqrt(m32)));
        atomicMax(nrm + 1, up_bits(sqrt(m16)));
        atomicMax(nrm + 2, up_bits(sqrt(md)));
    }
}

// One wave per query: |q|, |q16|, |ftz(q16) - q| in fp64.
__global__ __launch_bounds__(256) void k_query_norms(const float* __restrict__ q32, const __half* __restrict__ q16,
                                                    int32_t q, int32_t d, double* __restrict__ out) {
    const int lane = int(threadIdx.x & 63u);
    const int j = int(blockIdx.x) * 4 + int(threadIdx.x >> 6);
    if (j >= q) return;                          // whole wave
    double s32 = 0.0, s16 = 0.0, sd = 0.0;
    for (int i = lane; i < d; i += 64) {
        const float x = q32[int64_t(j) * d + i];
        const float hv = __half2float(q16[int64_t(j) * d + i]);
        const float hf = fabsf(hv) < kHalfMinNormal ? 0.0f : hv;
        s32 += double(x) * double(x);
        s16 += double(hv) * double(hv);
        const double df = double(hf) - double(x);
        sd += df * df;
    }
    s32 = wave_sum_f64(s32);
    s16 = wave_sum_f64(s16);
    sd = wave_sum_f64(sd);
    if (lane == 0) {
        out[4 * j] = sqrt(s32);
        out[4 * j + 1] = sqrt(s16);
        out[4 * j + 2] = sqrt(sd);
        out[4 * j + 3] = 0.0;
    }
}

// Bound on |fp16 MFMA fused score - Q=1 fused score| of any row, for weights <= 1
// (lambda >= 0, no boost). MFMA: dot(e16, q16) accumulated in fp32; the Q=1 scan:
// dot(e, q) (fp32 rows) or dot(e16, q) (fp16 rows) as per-lane fma chains of d/16
// terms plus a 4-step reduction; both then rounded once by the product with w.
__device__ inline double score_bound(const SeedArgs& a, int j) {
    const double e32 = double(__uint_as_float(a.nrm[0]));
    const double e16 = double(__uint_as_float(a.nrm[1]));
    const double de = double(__uint_as_float(a.nrm[2]));
    const double qn = a.qn[4 * j], q16n = a.qn[4 * j + 1], dq = a.qn[4 * j + 2];
    const double u = 0x1p-24;
    const double nm = double(a.d), nq = double(a.d) / 16.0 + 4.0;
    const double g_mfma = 2.0 * nm * u / (1.0 - nm * u);     // doubled: the MFMA's internal order is not specified
    const double g_scan = nq * u / (1.0 - nq * u);
    const double et = a.fp16 ? e16 : e32;                     // rows the Q=1 path reads
    double e = e16 * dq + g_mfma * e16 * q16n + g_scan * et * qn +
               u * (e16 * q16n * (1.0 + g_mfma) + et * qn * (1.0 + g_scan));
    if (!a.fp16) e += de * qn;
    return e * 1.01 + 1e-30 * nm;
}

// One workgroup per query; 16-lane group g rescores candidate g.
template <typename T, typename QF>
__global__ __launch_bounds__(256) void k_multi_seed(SeedArgs a) {
    __shared__ uint64_t s_key[kMultiCand];
    const int j = int(blockIdx.x);
    const int tid = int(threadIdx.x), lane = tid & 63, sub = lane & 15, g = tid >> 4;
    const uint64_t* cand = a.cand + int64_t(j) * kMultiCand;
    const uint64_t ck = cand[g];
    uint64_t key = kEmptyKey;
    if (ck != kEmptyKey) {                       // uniform over the 16-lane group
        QF qf;
        if constexpr (std::is_same_v<QF, QGeneric>) qf.d = a.d;
        qf.load(a.queries + int64_t(j) * a.d, sub);
        const int32_t id = key_id(ck);
        const T* row = static_cast<const T*>(a.emb) + int64_t(id) * a.d;
        const float dot = qf.dot_all(row, sub);
        const QueryTerms t{a.tq[j], a.lambda, a.mod_filter, -1, 0.0f};
        const float s = fuse_score(row16_sum(dot), a.ts[id], (a.mod_filter >= 0) ? a.mods[id] : 0, -1, t);
        key = make_key(s, uint32_t(id));
    }
    if (sub == 0) s_key[g] = key;
    __syncthreads();
    if (tid >= 64) return;
    const uint64_t x = wave_sort64(lane < kMultiCand ? s_key[lane] : kEmptyKey, lane);
    const uint64_t cl = lane < kMultiCand ? cand[lane] : kEmptyKey;
    const int nc = __popcll(__ballot(cl != kEmptyKey));
    const uint64_t c_last = __shfl(cl, kMultiCand - 1);
    const int kk = a.k < kMultiCand ? a.k : kMultiCand;
    const uint64_t kth = __shfl(x, kk - 1);
    bool ok = false;
    float margin = __builtin_inff();
    if (a.k <= kMultiCand) {
        if (nc < kMultiCand) {
            ok = true;                           // every live row was a candidate
        } else {
            const double eps = score_bound(a, j);
            const float s16 = key_score(c_last), s32 = key_score(kth);
            const double e16 = double(__uint_as_float(a.nrm[1]));
            const double q16n = a.qn[4 * j + 1];
            if (eps < 1e30) {
                if (s16 == -FLT_MAX) {
                    // the C-th candidate is filtered, so every unfiltered row (|score| <
                    // FLT_MAX) is a candidate and the rest are filtered rows of larger id
                    ok = e16 * q16n * 2.0 < double(FLT_MAX);
                } else {
                    const double mg = double(s32) - (double(s16) + eps);
                    ok = mg > 0.0;
                    margin = float(mg);
                }
            } else {
                margin = -__builtin_inff();
            }
        }
    }
    if (lane < kMultiCand && ok) a.seeds[int64_t(j) * kMultiCand + lane] = lane < kk ? x : kEmptyKey;
    if (lane == 0) {
        a.status[j] = ok ? kMultiOk : kMultiUncertified;
        a.margin[j] = margin;
    }
}

// Exact fused score of every visited node past the seeds: block (x, j) covers visit
// positions 16x .. 16x+15 of query j, one per 16-lane group (blocks past the visit
// count exit at once).
template <typename T, typename QF>
__global__ __launch_bounds__(256) void k_visit_scores(VisitScoreArgs a) {
    const int j = int(blockIdx.y);
    if (a.status[j] != kMultiOk) return;
    const int V = a.info[4 * j], ns = a.info[4 * j + 2];
    const int p = int(blockIdx.x) * 16 + int(threadIdx.x >> 4);
    if (int(blockIdx.x) * 16 >= V) return;
    if (p < ns || p >= V) return;                // whole 16-lane group
    const int sub = int(threadIdx.x & 15u);
    QF qf;
    if constexpr (std::is_same_v<QF, QGeneric>) qf.d = a.d;
    qf.load(a.queries + int64_t(j) * a.d, sub);
    const QueryTerms t{a.tq ? a.tq[j] : a.t_q_value, a.lambda, a.mod_filter, -1, 0.0f};
    const int32_t id = a.vlist[int64_t(j) * kMultiVisit + p];
    const float dot = qf.dot_all(static_cast<const T*>(a.emb) + int64_t(id) * a.d, sub);
    const float s = fuse_score(row16_sum(dot), a.ts[id], (a.mod_filter >= 0) ? a.mods[id] : 0, -1, t);
    if (sub == 0) a.vfin[int64_t(j) * kMultiVisit + p] = s;
}

template <typename T, typename QF>
int launch_seed_t(const SeedArgs& a, hipStream_t s) {
    MARS_LAUNCH((k_multi_seed<T, QF>), dim3(unsigned(a.q)), dim3(256), 0, s, a);
    return MARS_OK;
}

template <typename T, typename QF>
int launch_visit_t(const VisitScoreArgs& a, hipStream_t s) {
    MARS_LAUNCH((k_visit_scores<T, QF>), dim3(unsigned(kMultiVisit / 16), unsigned(a.q)), dim3(256), 0, s, a);
    return MARS_OK;
}

// The row layout the Q=1 scan uses for (fp16, d): QF32<d/64> or QF16<d/128>.
template <template <typename, typename> class L, typename A>
int dispatch_rows(const A& a, hipStream_t s) {
    if (!a.fp16 && a.d % 64 == 0) {
        switch (a.d / 64) {
            case 4: return L<float, QF32<4>>::run(a, s);
            case 6: return L<float, QF32<6>>::run(a, s);
            case 8: return L<float, QF32<8>>::run(a, s);
            case 12: return L<float, QF32<12>>::run(a, s);
            case 16: return L<float, QF32<16>>::run(a, s);
            default: break;
        }
    }
    if (a.fp16 && a.d % 128 == 0) {
        switch (a.d / 128) {
            case 2: return L<__half, QF16<2>>::run(a, s);
            case 3: return L<__half, QF16<3>>::run(a, s);
            case 4: return L<__half, QF16<4>>::run(a, s);
            case 6: return L<__half, QF16<6>>::run(a, s);
            default: break;
        }
    }
    return set_error(MARS_ERR_UNSUPPORTED, "batched global queries: embedding_dim %d unsupported", a.d);
}

template <typename T, typename QF>
struct SeedL {
    static int run(const SeedArgs& a, hipStream_t s) { return launch_seed_t<T, QF>(a, s); }
};
template <typename T, typename QF>
struct VisitL {
    static int run(const VisitScoreArgs& a, hipStream_t s) { return launch_visit_t<T, QF>(a, s); }
};

}  // namespace

int launch_row_norms(const float* emb, const __half* emb16, int64_t r0, int64_t r1, int32_t d, uint32_t* nrm,
                     hipStream_t s) {
    if (r1 <= r0) return MARS_OK;
    int64_t blocks = (r1 - r0 + 3) / 4;
    if (blocks > 8192) blocks = 8192;
    MARS_LAUNCH(k_row_norms, dim3(unsigned(blocks)), dim3(256), 0, s, emb, emb16, r0, r1, d, nrm);
    return MARS_OK;
}

int launch_query_norms(const float* q32, const __half* q16, int32_t q, int32_t d, double* out, hipStream_t s) {
    MARS_LAUNCH(k_query_norms, dim3(unsigned((q + 3) / 4)), dim3(256), 0, s, q32, q16, q, d, out);
    return MARS_OK;
}

int launch_multi_seed(const SeedArgs& a, hipStream_t s) { return dispatch_rows<SeedL>(a, s); }

int launch_visit_scores(const VisitScoreArgs& a, hipStream_t s) { return dispatch_rows<VisitL>(a, s); }

}  // namespace mars
