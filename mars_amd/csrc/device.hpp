// ============================================================================
//  device.hpp — device-side building blocks shared by the scan, finalize and
//  batched-query kernels: wave lane exchanges, wave-held top-K lists of score
//  keys, and the per-row dot products + fused score of the Q=1 scan. Kernels
//  that must reproduce the scan's scores bit for bit (the batched global path
//  rescoring candidates and BFS nodes) call the same QF32 / QF16 dot, the same
//  16-lane reduction and the same fuse_score, in the same lane layout.
// ============================================================================
#pragma once

#include "internal.hpp"

#include <cfloat>
#include <type_traits>

namespace mars {
namespace {

__device__ inline int lane_id() { return int(threadIdx.x & 63u); }

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint64_t u64x2 __attribute__((ext_vector_type(2)));

// Insert key x into a register list of K keys kept ascending; x < list[K-1] is
// checked by the caller.
template <int K>
__device__ inline void reg_insert(uint64_t (&list)[K], uint64_t x) {
    uint64_t v = x;
#pragma unroll
    for (int j = 0; j < K; ++j) {
        const uint64_t lo = list[j] < v ? list[j] : v;
        const uint64_t hi = list[j] < v ? v : list[j];
        list[j] = lo;
        v = hi;
    }
}

// Ascending order-preserving code of a score (-0.0 folded onto +0.0): a < b as floats
// iff ord32(a) < ord32(b) as unsigned; 0 is below every score (no bound yet).
__device__ inline uint32_t ord32(float s) {
    const uint32_t u = __float_as_uint(s + 0.0f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// The score whose ord32 is o (o != 0; -0.0 comes back as +0.0).
__device__ inline float ord32_inv(uint32_t o) {
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}

// Loads of data written earlier in the same kernel by other threads: served by
// L2 (agent-coherent), never by a stale L1 line.
template <typename T>
__device__ inline T ld_coherent(const T* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- lane exchanges: value of lane (lane ^ J) -----------------------------------
// J = 1, 2: DPP quad_perm; J = 4: DPP row_shl/row_shr; J = 8: DPP row_ror:8 (within a
// 16-lane row i^8 == i+-8); J = 16: ds_swizzle (xor within 32 lanes); J = 32: bpermute.
template <int J>
__device__ inline uint32_t xor_lane(uint32_t v) {
    if constexpr (J == 1) return uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0xB1, 0xF, 0xF, false));
    else if constexpr (J == 2) return uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x4E, 0xF, 0xF, false));
    else if constexpr (J == 4) {
        const uint32_t up = uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x104, 0xF, 0xF, false));   // lane + 4
        const uint32_t dn = uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x114, 0xF, 0xF, false));   // lane - 4
        return (threadIdx.x & 4u) ? dn : up;
    } else if constexpr (J == 8) return uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x128, 0xF, 0xF, false));
    else if constexpr (J == 16) return uint32_t(__builtin_amdgcn_ds_swizzle(int(v), 0x401F));
    else return uint32_t(__shfl_xor(int(v), J));
}
template <int J>
__device__ inline uint64_t xor_lane64(uint64_t v) {
    return (uint64_t(xor_lane<J>(uint32_t(v >> 32))) << 32) | xor_lane<J>(uint32_t(v));
}
template <int J>
__device__ inline float xor_lanef(float v) {
    return __uint_as_float(xor_lane<J>(__float_as_uint(v)));
}

// Insert key x into the wave-held ascending list (lane i = i-th smallest; lanes
// >= k hold kEmptyKey). Caller guarantees x < list[k-1].
__device__ inline void list_insert(uint64_t& list, uint64_t x, int lane, int k) {
    const uint64_t below = __ballot(list < x);
    const int pos = __popcll(below);
    const uint64_t up = __shfl_up(list, 1u);
    uint64_t v = (lane < pos) ? list : ((lane == pos) ? x : up);
    list = (lane < k) ? v : kEmptyKey;
}

// Offer one candidate key per lane where `offer` holds; keeps thr = list[k-1].
__device__ inline void list_offer(uint64_t& list, uint64_t& thr, uint64_t key, bool offer,
                                  int lane, int k) {
    uint64_t m = __ballot(offer && key < thr);
    while (m) {
        const int src = __ffsll((unsigned long long)m) - 1;
        m &= m - 1;
        const uint64_t x = __shfl(key, src);
        if (x < thr) {
            list_insert(list, x, lane, k);
            thr = __shfl(list, k - 1);
        }
    }
}

template <int J>
__device__ inline uint64_t cmpx(uint64_t x, int lane, bool ascending_block) {
    const uint64_t y = xor_lane64<J>(x);
    const bool lower = (lane & J) == 0;
    const uint64_t lo = x < y ? x : y, hi = x < y ? y : x;
    return (lower == ascending_block) ? lo : hi;
}

// Ascending bitonic sort of one key per lane across the wave.
__device__ inline uint64_t wave_sort64(uint64_t x, int lane) {
    x = cmpx<1>(x, lane, (lane & 2) == 0);
    x = cmpx<2>(x, lane, (lane & 4) == 0);
    x = cmpx<1>(x, lane, (lane & 4) == 0);
    x = cmpx<4>(x, lane, (lane & 8) == 0);
    x = cmpx<2>(x, lane, (lane & 8) == 0);
    x = cmpx<1>(x, lane, (lane & 8) == 0);
    x = cmpx<8>(x, lane, (lane & 16) == 0);
    x = cmpx<4>(x, lane, (lane & 16) == 0);
    x = cmpx<2>(x, lane, (lane & 16) == 0);
    x = cmpx<1>(x, lane, (lane & 16) == 0);
    x = cmpx<16>(x, lane, (lane & 32) == 0);
    x = cmpx<8>(x, lane, (lane & 32) == 0);
    x = cmpx<4>(x, lane, (lane & 32) == 0);
    x = cmpx<2>(x, lane, (lane & 32) == 0);
    x = cmpx<1>(x, lane, (lane & 32) == 0);
    x = cmpx<32>(x, lane, true);
    x = cmpx<16>(x, lane, true);
    x = cmpx<8>(x, lane, true);
    x = cmpx<4>(x, lane, true);
    x = cmpx<2>(x, lane, true);
    x = cmpx<1>(x, lane, true);
    return x;
}

// Smallest k of two ascending wave lists (lanes >= k of the result hold kEmptyKey):
// min(a[i], b[63-i]) is bitonic and holds the 64 smallest; six half-cleaners sort it.
__device__ inline uint64_t wave_merge64(uint64_t a, uint64_t b, int lane, int k) {
    const uint64_t r = __shfl(b, 63 - lane);
    uint64_t c = a < r ? a : r;
    c = cmpx<32>(c, lane, true);
    c = cmpx<16>(c, lane, true);
    c = cmpx<8>(c, lane, true);
    c = cmpx<4>(c, lane, true);
    c = cmpx<2>(c, lane, true);
    c = cmpx<1>(c, lane, true);
    return lane < k ? c : kEmptyKey;
}

// Offer one key per lane: few winners are inserted one by one, many are sorted
// and merged in registers.
__device__ inline void wave_offer(uint64_t& list, uint64_t& thr, uint64_t key, int lane, int k) {
    const uint64_t m = __ballot(key < thr);
    if (m == 0) return;
    if (__popcll(m) <= 2) {
        list_offer(list, thr, key, true, lane, k);
        return;
    }
    const uint64_t xs = wave_sort64(key < thr ? key : kEmptyKey, lane);
    list = wave_merge64(list, xs, lane, k);
    thr = __shfl(list, k - 1);
}

// fp64 sum over the 16 lanes of a DPP row; every lane of the row gets the total.
__device__ inline double row16_sum_f64(double v) {
    auto x = [](double a, auto tag) {
        constexpr int J = decltype(tag)::value;
        const uint64_t b = uint64_t(__double_as_longlong(a));
        return __longlong_as_double((long long)xor_lane64<J>(b));
    };
    v += x(v, std::integral_constant<int, 8>{});
    v += x(v, std::integral_constant<int, 4>{});
    v += x(v, std::integral_constant<int, 2>{});
    v += x(v, std::integral_constant<int, 1>{});
    return v;
}

// Sum over the 16 lanes of a DPP row; every lane of the row gets the total.
__device__ inline float row16_sum(float v) {
    v += xor_lanef<8>(v);
    v += xor_lanef<4>(v);
    v += xor_lanef<2>(v);
    v += xor_lanef<1>(v);
    return v;
}

// ---- per-row dot products -------------------------------------------------------
// fp32 rows: chunk c covers floats [64c, 64c+64); lane s holds 4 of them.
template <int NCH>
struct QF32 {
    float v[NCH][4];
    __device__ void load(const float* q, int sub) {
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const float4 x = reinterpret_cast<const float4*>(q + c * 64)[sub];
            v[c][0] = x.x; v[c][1] = x.y; v[c][2] = x.z; v[c][3] = x.w;
        }
    }
    __device__ void fetch(const float* row, int sub, f32x4 (&x)[NCH]) const {
        const f32x4* r = reinterpret_cast<const f32x4*>(row) + sub;
#pragma unroll
        for (int c = 0; c < NCH; ++c) x[c] = __builtin_nontemporal_load(r + c * 16);
    }
    __device__ float dot_fetched(const f32x4 (&x)[NCH]) const {
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            acc = fmaf(x[c].x, v[c][0], acc);
            acc = fmaf(x[c].y, v[c][1], acc);
            acc = fmaf(x[c].z, v[c][2], acc);
            acc = fmaf(x[c].w, v[c][3], acc);
        }
        return acc;
    }
    __device__ float dot(const float* row, int sub) const {
        f32x4 x[NCH];
        fetch(row, sub, x);
        return dot_fetched(x);
    }
    // dot with every load of the row issued before the first FMA (latency-bound callers
    // that score one row per group; the arithmetic is dot's)
    __device__ float dot_all(const float* row, int sub) const {
        f32x4 x[NCH];
        fetch(row, sub, x);
        __builtin_amdgcn_sched_barrier(0);
        return dot_fetched(x);
    }
    // |q|^2 over the lane's elements, fp64
    __device__ double norm2() const {
        double s = 0.0;
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
            for (int j = 0; j < 4; ++j) s += double(v[c][j]) * double(v[c][j]);
        return s;
    }
};

// fp16 rows: chunk c covers halves [128c, 128c+128); lane s holds 8 of them.
template <int NCH>
struct QF16 {
    float v[NCH][8];
    __device__ void load(const float* q, int sub) {
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
            for (int j = 0; j < 8; ++j) v[c][j] = q[c * 128 + sub * 8 + j];
    }
    __device__ float dot(const __half* row, int sub) const {
        const u32x4* r = reinterpret_cast<const u32x4*>(row) + sub;
        u32x4 x[NCH];
#pragma unroll
        for (int c = 0; c < NCH; ++c) x[c] = __builtin_nontemporal_load(r + c * 16);
        return dot_fetched(x);
    }
    __device__ float dot_all(const __half* row, int sub) const {
        const u32x4* r = reinterpret_cast<const u32x4*>(row) + sub;
        u32x4 x[NCH];
#pragma unroll
        for (int c = 0; c < NCH; ++c) x[c] = __builtin_nontemporal_load(r + c * 16);
        __builtin_amdgcn_sched_barrier(0);
        return dot_fetched(x);
    }
    __device__ float dot_fetched(const u32x4 (&x)[NCH]) const {
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const uint32_t w[4] = {x[c].x, x[c].y, x[c].z, x[c].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const __half2 h2 = *reinterpret_cast<const __half2*>(&w[j]);
                const float2 f = __half22float2(h2);
                acc = fmaf(f.x, v[c][2 * j], acc);
                acc = fmaf(f.y, v[c][2 * j + 1], acc);
            }
        }
        return acc;
    }
};

// Any D: lane s of the group takes elements s, s+16, ... (q read through cache).
struct QGeneric {
    const float* q;
    int d;
    __device__ void load(const float* q_, int) { q = q_; }
    __device__ float dot(const float* row, int sub) const {
        float acc = 0.0f;
        for (int i = sub; i < d; i += 16) acc = fmaf(row[i], q[i], acc);
        return acc;
    }
    __device__ float dot(const __half* row, int sub) const {
        float acc = 0.0f;
        for (int i = sub; i < d; i += 16) acc = fmaf(__half2float(row[i]), q[i], acc);
        return acc;
    }
    template <typename T>
    __device__ float dot_all(const T* row, int sub) const { return dot(row, sub); }
};

// fused stage-1/2 epilogue (reference order of fp32 operations: dot * w, then
// * (1 + boost); filtered rows are -FLT_MAX and not decayed). A is any struct with
// the query terms t_q, lambda, mod_filter, query_ep, boost (ScanArgs, QueryTerms).
template <class A>
__device__ inline float decay_weight(float ts, const A& a) {
    const float age = fmaxf(0.0f, a.t_q - ts);
    return expf(-a.lambda * age);
}
template <class A>
__device__ inline float fuse_score(float dot, float ts, int32_t mod, int32_t ep, const A& a) {
    if (a.mod_filter >= 0 && mod != a.mod_filter) return -FLT_MAX;
    float s = dot * decay_weight(ts, a);
    if (a.boost > 0.0f && ep == a.query_ep && s > -FLT_MAX * 0.5f) s = s * (1.0f + a.boost);
    return s;
}


// End of a grid-stride scan: wave 0 merges the workgroup's four wave lists (s_lists,
// written by every wave and synchronised by the caller) and appends its keys that can
// still be among the global K best. Every key of the global top-K is <= the global K-th
// key <= any workgroup's K-th key, so keys above the running minimum of those are
// dropped here without changing the result. The bound is read first; only a workgroup
// that lowers it issues the atomicMin (about ln(#workgroups) of them), and only one with
// keys under it appends. A is any struct with part, gthr and gcnt (ScanArgs).
template <class A>
__device__ inline void wg_publish(const uint64_t (&s_lists)[4][64], int lane, int k, const A& a) {
    uint64_t list = s_lists[0][lane];
    list = wave_merge64(list, s_lists[1][lane], lane, k);
    list = wave_merge64(list, wave_merge64(s_lists[2][lane], s_lists[3][lane], lane, k), lane, k);
    const uint64_t kth = __shfl(list, k - 1);
    uint64_t cur = kEmptyKey;
    if (lane == 0) cur = ld_coherent(a.gthr);
    cur = __shfl(cur, 0);
    if (kth < cur && lane == 0) atomicMin(reinterpret_cast<unsigned long long*>(a.gthr), (unsigned long long)kth);
    const uint64_t bound = cur < kth ? cur : kth;
    const bool pass = lane < k && list != kEmptyKey && list <= bound;
    const uint64_t m = __ballot(pass);
    uint32_t base = 0;
    if (lane == 0 && m) base = atomicAdd(a.gcnt, uint32_t(__popcll(m)));
    base = __shfl(base, 0);
    if (pass) a.part[base + uint32_t(__popcll(m & ((1ull << lane) - 1ull)))] = list;
}

// Completion word of a Q=1 query (host-mapped): every thread's result writes are made
// visible system-wide, then one thread stores seq. Called by all threads of the
// workgroup that writes the query's last results, as its last action.
__device__ inline void signal_done(uint32_t* done, uint32_t seq) {
    if (done == nullptr) return;               // uniform
    __threadfence_system();
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(done, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// ---- row-norm bounds of the fp16 copy (batched global certificate) -------------------
constexpr float kHalfMinNormal = 6.103515625e-05f;   // 2^-14

// fp32 bit pattern of a value >= v (v >= 0); NaN stays NaN
__device__ inline uint32_t up_bits(double v) {
    if (!(v == v)) return 0x7fc00000u;
    float f = float(v);
    if (double(f) < v) f = nextafterf(f, __builtin_inff());
    return __float_as_uint(f);
}

__device__ inline double wave_sum_f64(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// max that lets a NaN through (the certificate must then fail)
__device__ inline double max_nan(double m, double v) { return (v <= m) ? m : v; }

// Raises nrm[0..2] to |e|, |e16| and |ftz(e16) - e| of one row whose per-lane sums of
// squares (fp64) the calling wave holds; lane 0 issues the atomics.
__device__ inline void raise_row_norms(double s32, double s16, double sd, uint32_t* nrm) {
    s32 = wave_sum_f64(s32);
    s16 = wave_sum_f64(s16);
    sd = wave_sum_f64(sd);
    if ((threadIdx.x & 63u) == 0) {
        atomicMax(nrm + 0, up_bits(sqrt(s32)));
        atomicMax(nrm + 1, up_bits(sqrt(s16)));
        atomicMax(nrm + 2, up_bits(sqrt(sd)));
    }
}

// ---- the int8 copy (certified global query) -------------------------------------------
// Row r is stored as bytes v_i in [-127, 127] with one scale s_r = fl(max_i |e_i| / 127),
// standing for e^_i = s_r v_i. The fp32 scan's dot of a row (per-lane fmaf chains of d/16
// steps, then the 16-lane reduction) lies within gamma_n |q| |e| of q.e, with n = d/16 + 6
// rounded operations per term at most. The int8 scan (k_scan8) splits the query into two
// int8 parts, q = s_hi q_hi + s_lo q_lo + r2, and sums q_hi.v and q_lo.v exactly in int32 on
// MFMA (|sum| <= 127 * 127 * d < 2^24 for d <= 1024, so the conversion to fp32 is exact as
// well); the split's remainder r2 and the three fp32 roundings of s_r (s_hi A_hi + s_lo A_lo)
// make up its per-query term tau. Hence
//     |dot8 - dot32| <= |q| (|e^ - e| + gamma_n (|e^| + |e|)) + tau = |q| c_r + tau,
// where the gamma_n |e^| term is slack the exact int32 sums no longer need.
__device__ inline double i8_gamma(int32_t d) {
    const double nu = (double(d) / 16.0 + 6.0) * 0x1p-24;
    return nu / (1.0 - nu);
}

__device__ inline float wave_max_f(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

// Quantizing one row (one wave): the scale from the row's max |e|, then per element its byte
// (into the tiled copy) and fp64 sums of squares of e, e^ and e^ - e; lane 0 stores (s_r, c_r)
// to meta and raises nrm8[0] to c_r and nrm8[1] to |e| (c_r rounded up to fp32). A NaN or
// infinite element makes c_r NaN or infinite, and with it nrm8[0]: the certificate then
// never holds.
struct I8Row {
    float s;                                  // the row's scale
    int8_t* tile;                             // the row's byte 0 in its tile
    double s32 = 0.0, s8 = 0.0, sd = 0.0;
    __device__ I8Row(float max_abs, int8_t* emb8, int64_t row, int32_t d)
        : s(max_abs / 127.0f), tile(emb8 + i8_offset(row, 0, d)) {}
    __device__ void put(int32_t i, float x) {
        float t = s > 0.0f ? rintf(x / s) : 0.0f;
        t = fminf(fmaxf(t, -127.0f), 127.0f);
        const int v = int(t);
        tile[((i >> 6) << 10) + (((i & 63) >> 4) << 8) + (i & 15)] = int8_t(v);   // i8_offset(row, i) - i8_offset(row, 0)
        const double eh = double(s) * double(v);
        s32 += double(x) * double(x);
        s8 += eh * eh;
        const double df = eh - double(x);
        sd += df * df;
    }
    __device__ void finish(int32_t d, float* meta, uint32_t* nrm8) {
        s32 = wave_sum_f64(s32);
        s8 = wave_sum_f64(s8);
        sd = wave_sum_f64(sd);
        if (lane_id() == 0) {
            const double c = (sqrt(sd) + i8_gamma(d) * (sqrt(s8) + sqrt(s32))) * (1.0 + 1e-9);
            const uint32_t cb = up_bits(c);
            meta[0] = s;
            meta[1] = __uint_as_float(cb);
            atomicMax(nrm8 + 0, cb);
            atomicMax(nrm8 + 1, up_bits(sqrt(s32)));
        }
    }
};

// One wave quantizes row `row` (d floats at e) into the tiled copy emb8, meta and nrm8.
// The row is read in chunks of 64 kPer floats held in registers (every load of a chunk issued
// at once), twice: one memory latency per chunk and pass.
// (kPer: floats per lane and chunk; every kPer visits each lane's elements in the same
// order, lane + 64 j, so it does not change the sums.)
template <int kPer = 8>
__device__ inline void quantize_row_i8(const float* e, int32_t d, int8_t* emb8, int64_t row, float* meta,
                                       uint32_t* nrm8) {
    const int lane = lane_id();
    float m = 0.0f;
    for (int base = 0; base < d; base += 64 * kPer) {
        float x[kPer];
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int i = base + lane + 64 * j;
            x[j] = i < d ? e[i] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < kPer; ++j) m = fmaxf(m, fabsf(x[j]));
    }
    I8Row q(wave_max_f(m), emb8, row, d);
    for (int base = 0; base < d; base += 64 * kPer) {
        float x[kPer];
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int i = base + lane + 64 * j;
            x[j] = i < d ? e[i] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int i = base + lane + 64 * j;
            if (i < d) q.put(i, x[j]);
        }
    }
    q.finish(d, meta, nrm8);
}

}  // namespace
}  // namespace mars
