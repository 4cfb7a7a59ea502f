// ============================================================================
//  batch_mm.hip — k_batch_mm: the neighbour searches of the k-NN builders, batches of
//  Q >= kGemmMinQ queries that are corpus rows (the score is the plain dot product and
//  the query's own row is excluded).
//
//  C = E_tile x Q_tile^T for 256 corpus rows x 256 queries per tile on
//  v_mfma_f32_32x32x16_f16 (fp16 operands, fp32 accumulation). Four waves, one per
//  SIMD with the whole register file: wave w holds rows 128 (w & 1) .. +127 against
//  queries 128 (w >> 1) .. +127, 4 x 4 tiles of 32 x 32 (256 accumulators per lane).
//  Each corpus row is read from HBM once per 256 queries, and the 384 KiB query tile
//  is read from L2 once per 256 rows.
//
//  Operands reach LDS in k-stages of 32 straight from global memory
//  (global_load_lds_dwordx4, no staging registers) through two rings: five corpus stage
//  buffers and four query stage buffers. Once stage g's fragments are in registers its
//  buffers refill, so the rows of stages g + 1 .. g + 5 and the queries of g + 1 .. g + 4
//  are in flight while stage g's MFMAs run. The stage pipeline waits for its own loads
//  by count (s_waitcnt vmcnt) and meets at plain s_barriers: the __syncthreads fence
//  would wait for every load in flight, the prefetches included.
//
//  Selection: thread t, the owner of query q0 + t, keeps its best K keys in registers.
//  Before each tile the owners publish a threshold per query (the larger of its sampled
//  floor and, once its list is full, its K-th score); after the tile each lane tests its
//  accumulators against it and offers the few (query, row) pairs that reach it into 8
//  slots per query in the tile's last stage buffers, and the owners insert those (the slot
//  selection). A tile where a query has no threshold or more candidates than slots goes
//  the full way instead: the raw accumulators pass through those buffers 32 rows
//  at a time ([query][row], 16-byte writes and reads) and the owners test all of their
//  scores. Output: K keys per (query, row range) in the layout k_batch_merge reads.
//  The sampled pass that gives the floors keeps no lists: per query and range it writes
//  the largest dot of each of the 16 row blocks a query's dots fall into (see gmx).
// ============================================================================
#include "device.hpp"

namespace mars {
namespace {

constexpr int kMQ = 256;        // queries per workgroup
constexpr int kMR = 256;        // rows per tile
constexpr int kMK = 32;         // k per LDS stage
constexpr int kMBC = 5;         // corpus stage buffers (a ring over the tile loop's stages)
constexpr int kMBQ = 4;         // query stage buffers
constexpr int kMThreads = 256;
constexpr int kMChunk = 32;     // rows per staged chunk of the full-way selection
constexpr int kPartQ = 64;      // queries per block of the partial-key layout
constexpr int kMDma = 4;        // load instructions per wave and operand per stage
constexpr int kMSlots = 8;      // candidate slots per query and tile (the slot selection)
constexpr int kMRec = 64;       // per wave and tile: 16-dot records of lanes that reach a threshold

typedef float f32x16 __attribute__((ext_vector_type(16)));

// The corpus stages in the first 80 KiB, the query stages in the next 64 KiB. The rows
// come from HBM (shared with the three other query tiles of the row range through L2) and
// get one more stage in flight than the L2-resident queries. (Same-box traces of the 1M
// k-NN chunks: full pass 1870 us with four buffers of each, 1828 us with this split.)
struct MmLds {
    u32x4 e[kMBC][kMR * 4];     // 5 x 16 KiB: 256 rows x 4 pieces per stage
    u32x4 q[kMBQ][kMQ * 4];     // 4 x 16 KiB: 256 queries x 4 pieces per stage
    float thr[kMQ];             // per query: raw dot products below it cannot enter its list
    uint32_t cnt[kMQ];          // per query: candidates offered in this tile
    uint32_t rhdr[kMThreads / 64][kMRec];  // per record: query << 8 | first row of the lane's 16
    uint32_t wfast[kMThreads / 64];  // per wave: every query it owns has a threshold
    uint32_t wover[kMThreads / 64];  // per wave: a query of its half got more than kMSlots
};
static_assert(sizeof(u32x4) * kMR * 4 == size_t(kMQ / 2) * kMChunk * sizeof(float), "half the queries per operand");
static_assert(sizeof(u32x4) * kMQ * 4 == size_t(kMQ) * kMSlots * 8, "the slots fill the query half of a stage buffer");
static_assert(sizeof(u32x4) * kMR * 4 == size_t(kMThreads / 64) * kMRec * 64, "the records fill its corpus half");
static_assert(kMThreads / 64 * kMDma * 64 == kMR * 4, "the waves' loads cover a stage");

// s_waitcnt immediates (gfx9 encoding: vmcnt[3:0] and [15:14], expcnt[6:4], lgkmcnt[11:8])
constexpr int wait_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int kWaitLgkm0 = 15 | (3 << 14) | (7 << 4);

// A pointer the wave holds in SGPRs (the same in every lane), so that loads take the
// scalar-base plus 32-bit vector-offset form.
__device__ inline const char* uniform_ptr(const char* p) {
    const uint64_t u = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(u)), hi = __builtin_amdgcn_readfirstlane(uint32_t(u >> 32));
    return reinterpret_cast<const char*>((uint64_t(hi) << 32) | lo);
}

// Workgroup barrier without the memory fence of __syncthreads (which waits for every
// load in flight, the stage prefetches included): callers wait for what they need first.
__device__ inline void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    __builtin_amdgcn_s_barrier();
}

template <int NS, int K>
__global__ __launch_bounds__(kMThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void k_batch_mm(BatchArgs a) {
    static_assert(NS > kMBC, "a tile has more stages than the corpus ring");
    __shared__ __attribute__((aligned(16))) MmLds sh;
    const int tid = int(threadIdx.x), lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = wave & 1, wq = wave >> 1;       // row half, query half
    const int lm = lane & 31, lh = lane >> 5;
    constexpr int d = NS * kMK;
    const int r_id = int(blockIdx.x) % a.n_rranges;
    const int q0 = (int(blockIdx.x) / a.n_rranges) * kMQ;
    const int64_t r0 = int64_t(r_id) * (a.range_stride > 0 ? a.range_stride : a.rows_per_range);
    const int64_t r1 = (a.n < r0 + a.rows_per_range) ? a.n : r0 + a.rows_per_range;
    const int64_t ntiles = r1 > r0 ? (r1 - r0 + kMR - 1) / kMR : 0;

    // Stage loads go straight from global memory to LDS (global_load_lds_dwordx4): load
    // j of a wave fills 64 consecutive 16-byte slots, s = (wave * kMDma + j) * 64 + lane,
    // i.e. slot s & 3 of row s >> 2, which holds piece (s & 3) ^ ((row >> 2) & 3) of the
    // row's 32 k. The fragment reads of 16 consecutive rows (a 16-lane group of a 16-byte
    // read) then hit the 16 distinct 16-byte bank groups of the 256-byte LDS row. Every
    // stage issues the same loads (rows clamped into range; stages past the last tile load
    // a clamped tile nobody reads), so the wait counts stay exact.
    const int srow = (wave * kMDma) * 16 + (lane >> 2);            // + 16 j
    const int spiece = (lane & 3) ^ ((srow >> 2) & 3);             // the same for every j
    // Addresses: a uniform base (the tile's first row; the query array) plus a 32-bit
    // byte offset per lane (within 256 rows, within the batch's queries).
    uint32_t qoff[kMDma];
#pragma unroll
    for (int j = 0; j < kMDma; ++j) {
        const int q = q0 + srow + 16 * j;
        qoff[j] = uint32_t(q < a.q ? q : a.q - 1) * uint32_t(d * 2) + uint32_t(spiece * 16);
    }
    // The loads of stage st of tile `tile` (st >= NS: stage st - NS of the next tile; tiles
    // past the last load the last one again) into query buffer bq / corpus buffer bc.
    auto issue_q = [&](int tile, int st, int bq) {
        if (st >= NS) { ++tile; st -= NS; }
        const char* const qb = uniform_ptr(reinterpret_cast<const char*>(a.qh) + st * kMK * 2);
#pragma unroll
        for (int j = 0; j < kMDma; ++j)
            __builtin_amdgcn_global_load_lds(qb + qoff[j], &sh.q[bq][(wave * kMDma + j) * 64], 16, 0, 0);
    };
    auto issue_c = [&](int tile, int st, int bc) {
        if (st >= NS) { ++tile; st -= NS; }
        tile = tile < int(ntiles) ? tile : int(ntiles) - 1;
        const int64_t trow = r0 + int64_t(tile) * kMR;
        const char* const tb = uniform_ptr(reinterpret_cast<const char*>(a.emb16 + trow * d) + st * kMK * 2);
        const uint32_t last = uint32_t(r1 - 1 - trow < kMR - 1 ? r1 - 1 - trow : kMR - 1);   // rows past r1 - 1 clamp
#pragma unroll
        for (int j = 0; j < kMDma; ++j) {
            const uint32_t rl = uint32_t(srow + 16 * j) < last ? uint32_t(srow + 16 * j) : last;
            __builtin_amdgcn_global_load_lds(tb + (rl * uint32_t(d * 2) + uint32_t(spiece * 16)),
                                             &sh.e[bc][(wave * kMDma + j) * 64], 16, 0, 0);
        }
    };

    uint64_t list[K];                              // query q0 + tid
#pragma unroll
    for (int j = 0; j < K; ++j) list[j] = kEmptyKey;
    const int my_q = q0 + tid;
    const int64_t my_self = a.self_base >= 0 ? a.self_base + my_q : -1;   // the query's own row
    // the sampled score floor (a lower bound of the query's final floor_k-th best score): no
    // row below it can be among the query's results, so none is kept
    float my_floor = -INFINITY;
    if (a.floor_keys != nullptr && my_q < a.q) {
        const uint64_t fk = a.floor_keys[int64_t(my_q) * a.floor_k + a.floor_k - 1];
        if (fk != kEmptyKey) my_floor = key_score(fk);
    }

    // Every stage issues its loads in one order, the queries kMBQ stages ahead, then the rows
    // kMBC stages ahead, so the wait counts below are exact in the steady state (and only
    // stricter in the first stages of the first tile).
    if (ntiles > 0) {
#pragma unroll
        for (int st = 0; st < kMBQ; ++st) {
            issue_q(0, st, st);
            issue_c(0, st, st);
        }
#pragma unroll
        for (int st = kMBQ; st < kMBC; ++st) issue_c(0, st, st);
    }
    // loads issued after stage g + 1's queries, when stage g waits for them: the rows of
    // stage g + 2 (issued with them), then two stages of loads
    constexpr int kStageWait = kMDma * (1 + 2 * (kMBQ - 2));
    // at a tile's first stage: also the deferred loads issued after the selection
    constexpr int kTileWait = kMDma * (1 + 2 * (kMBQ - 1));

    f32x16 acc[4][4];
    f16x8 fa0[4], fb0[4], fa1[4], fb1[4];          // fragments of k-step 0 / 1 of a stage
    auto read_frags = [&](int bc, int bq, int kk, f16x8 (&af)[4], f16x8 (&bf)[4]) {
        const int pc = (2 * kk + lh) ^ ((lm >> 2) & 3);        // swizzled slot of this lane's piece
#pragma unroll
        for (int x = 0; x < 4; ++x) {
            af[x] = __builtin_bit_cast(f16x8, sh.e[bc][(wr * 128 + x * 32 + lm) * 4 + pc]);
            bf[x] = __builtin_bit_cast(f16x8, sh.q[bq][(wq * 128 + x * 32 + lm) * 4 + pc]);
        }
    };
    auto mma = [&](const f16x8 (&af)[4], const f16x8 (&bf)[4]) {
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
#pragma unroll
            for (int qt = 0; qt < 4; ++qt)
                acc[rt][qt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[rt], bf[qt], acc[rt][qt], 0, 0, 0);
    };

    // Selection staging: a chunk's raw scores as [query][row] fp32, queries 0 .. 127 in the
    // tile's last corpus stage buffer and 128 .. 255 in its last query stage buffer. Query q's 32
    // rows are eight 16-byte slots; rows 4 s .. 4 s + 3 sit in slot s ^ ((q >> 1) & 7), so
    // the 16-byte writes and reads of 16 consecutive queries hit 16 distinct bank groups.
    // (the last stage's buffers of each tile: set before its selection)
    float* stg_lo = nullptr;
    float* stg_hi = nullptr;
    float* wbase = nullptr;                                         // this wave's 128 queries
    const float* obase = nullptr;
    const int oswz = (tid >> 1) & 7;
    // The owner's threshold for the next tile: the larger of its floor and, once its list is
    // full, its K-th score; a dot below it cannot enter the list. Without either the wave's
    // tiles go the full way. Queries past the batch offer nothing.
    auto publish = [&]() {
        float th = INFINITY;
        bool ok = true;
        if (my_q < a.q) {
            th = fmaxf(list[K - 1] != kEmptyKey ? key_score(list[K - 1]) : -INFINITY, my_floor);
            ok = th > -INFINITY;
        }
        int ut = tid;
        asm volatile("" : "+v"(ut));
        sh.thr[ut] = th;
        sh.cnt[ut] = 0u;
        const uint64_t bad = __ballot(!ok);
        if (lane == 0) sh.wfast[wave] = bad == 0u ? 1u : 0u;
    };
    // acc[rt][qt][v] = C[row wr*128 + rt*32 + 8*(v/4) + 4*lh + v%4][query wq*128 + qt*32 + lm]:
    // v = 4 g .. 4 g + 3 are rows 4 (2 g + lh) .. + 3 of the chunk, one 16-byte slot
    auto stage_rows = [&](const f32x16 (&ac)[4]) {
#pragma unroll
        for (int qt = 0; qt < 4; ++qt) {
            const int ql = qt * 32 + lm;
            const int sw = (ql >> 1) & 7;
#pragma unroll
            for (int g = 0; g < 4; ++g)
                *reinterpret_cast<float4*>(wbase + ql * kMChunk + ((2 * g + lh) ^ sw) * 4) =
                    float4{ac[qt][4 * g], ac[qt][4 * g + 1], ac[qt][4 * g + 2], ac[qt][4 * g + 3]};
        }
    };
    // The owner's pass over chunk c of the tile at row t0: its 32 dots, then the rows that
    // can enter its list.
    auto select_chunk = [&](int c, int64_t t0) {
        float x[kMChunk];
#pragma unroll
        for (int s4 = 0; s4 < kMChunk / 4; ++s4) {
            const float4 v4 = *reinterpret_cast<const float4*>(obase + (s4 ^ oswz) * 4);
            x[4 * s4] = v4.x; x[4 * s4 + 1] = v4.y; x[4 * s4 + 2] = v4.z; x[4 * s4 + 3] = v4.w;
        }
        // rows at or above the K-th score held and the floor (NaN passes to the key test)
        const float bound = fmaxf(list[K - 1] != kEmptyKey ? key_score(list[K - 1]) : -INFINITY, my_floor);
        uint32_t pass = 0u;
#pragma unroll
        for (int j = 0; j < kMChunk; ++j) pass |= uint32_t(!(x[j] < bound)) << j;
        const int64_t rbase = t0 + c * kMChunk;
        if (rbase + kMChunk > r1) pass &= (r1 > rbase) ? (0xFFFFFFFFu >> (kMChunk - int(r1 - rbase))) : 0u;
        if (my_self >= rbase && my_self < rbase + kMChunk) pass &= ~(1u << int(my_self - rbase));
        while (pass) {
            const int j = __builtin_ctz(pass);
            pass &= pass - 1u;
            const uint64_t key = make_key(obase[((j >> 2) ^ oswz) * 4 + (j & 3)], uint32_t(rbase + j));
            if (key < list[K - 1]) reg_insert<K>(list, key);
        }
    };

    // The sampled pass (its keys serve only as floors): each lane keeps, per block of the
    // accumulator layout, the largest dot of its 16 rows of that block over the tiles (rows
    // past the range and the query's own row left out). A query's 16 maxima per range are
    // 16 distinct dots of its sampled rows, so their k-th best is at most the k-th best of
    // those rows: a floor as sound as the best-K lists would give, and far cheaper (no
    // insertions). gmx[qt * 4 + rt]: block (rt, qt).
    const bool sample = a.sample_pass != 0;
    float gmx[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) gmx[i] = -INFINITY;
    auto sample_tile = [&](int64_t t0) {
        int ut = tid;
        asm volatile("" : "+v"(ut));
        const int ulm = ut & 31, ulh = (ut >> 5) & 1;
#pragma unroll 1
        for (int h = 0; h < 8; ++h) {
            f32x16 x0, x1;
            switch (h) {
                case 0: x0 = acc[0][0]; x1 = acc[0][1]; break;
                case 1: x0 = acc[0][2]; x1 = acc[0][3]; break;
                case 2: x0 = acc[1][0]; x1 = acc[1][1]; break;
                case 3: x0 = acc[1][2]; x1 = acc[1][3]; break;
                case 4: x0 = acc[2][0]; x1 = acc[2][1]; break;
                case 5: x0 = acc[2][2]; x1 = acc[2][3]; break;
                case 6: x0 = acc[3][0]; x1 = acc[3][1]; break;
                default: x0 = acc[3][2]; x1 = acc[3][3]; break;
            }
            // dot v of the lane's block is row rb + 8 (v >> 2) + (v & 3)
            const int64_t rb = t0 + wr * 128 + (h >> 1) * 32 + 4 * ulh;
            const int64_t lim64 = r1 - rb;
            const int lim = lim64 < 0 ? 0 : (lim64 > 32 ? 32 : int(lim64));   // offsets below it are in range
            const int ql0 = wq * 128 + (h & 1) * 64 + ulm;
            int s0 = -1, s1 = -1;                                             // the queries' own rows
            if (a.self_base >= 0) {
                const int64_t o0 = a.self_base + q0 + ql0 - rb, o1 = o0 + 32;
                s0 = (o0 >= 0 && o0 < 32) ? int(o0) : -1;
                s1 = (o1 >= 0 && o1 < 32) ? int(o1) : -1;
            }
            float m0 = -INFINITY, m1 = -INFINITY;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int o = 8 * (v >> 2) + (v & 3);
                m0 = (o < lim && o != s0) ? fmaxf(m0, x0[v]) : m0;
                m1 = (o < lim && o != s1) ? fmaxf(m1, x1[v]) : m1;
            }
            switch (h) {
                case 0: gmx[0] = fmaxf(gmx[0], m0); gmx[4] = fmaxf(gmx[4], m1); break;
                case 1: gmx[8] = fmaxf(gmx[8], m0); gmx[12] = fmaxf(gmx[12], m1); break;
                case 2: gmx[1] = fmaxf(gmx[1], m0); gmx[5] = fmaxf(gmx[5], m1); break;
                case 3: gmx[9] = fmaxf(gmx[9], m0); gmx[13] = fmaxf(gmx[13], m1); break;
                case 4: gmx[2] = fmaxf(gmx[2], m0); gmx[6] = fmaxf(gmx[6], m1); break;
                case 5: gmx[10] = fmaxf(gmx[10], m0); gmx[14] = fmaxf(gmx[14], m1); break;
                case 6: gmx[3] = fmaxf(gmx[3], m0); gmx[7] = fmaxf(gmx[7], m1); break;
                default: gmx[11] = fmaxf(gmx[11], m0); gmx[15] = fmaxf(gmx[15], m1); break;
            }
        }
    };

    publish();                                     // the first tile's thresholds (floors)
    for (int64_t t = 0; t < ntiles; ++t) {
        const int64_t t0 = r0 + t * kMR;
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
#pragma unroll
            for (int qt = 0; qt < 4; ++qt)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[rt][qt][v] = 0.0f;
        // stage 0's buffers (global stage t NS), its loads, then its k-step-0 fragments
        int bc = int((t * NS) % kMBC), bq = int((t * NS) % kMBQ);
        __builtin_amdgcn_s_waitcnt(wait_vm(kTileWait));
        lds_barrier();
        read_frags(bc, bq, 0, fa0, fb0);
        // Stage st, with its k-step-0 fragments already read:
        //   read k-step 1; MFMAs of k-step 0 (the reads land meanwhile);
        //   wait for stage st + 1's loads and meet: every wave's loads of st + 1 landed,
        //   every wave is done reading stage st; refill stage st's buffers with the queries
        //   of stage st + kMBQ and the rows of stage st + kMBC (the tile's last stage leaves
        //   that to after the selection, which needs the buffers); read k-step 0 of st + 1;
        //   MFMAs of k-step 1 (the reads land meanwhile).
        // (sched_barrier keeps each block of reads ahead of the MFMAs it overlaps: the
        // scheduler would otherwise sink the reads next to their uses. Unrolled whole: a
        // full pass of the 1M k-NN chunk took 1.72 ms against 1.76 ms unrolled by 4 on one
        // box; by 4 against by 2, 1.79 against 1.82 ms on another.)
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            read_frags(bc, bq, 1, fa1, fb1);
            __builtin_amdgcn_sched_barrier(0);
            mma(fa0, fb0);
            if (st + 1 < NS) {
                __builtin_amdgcn_s_waitcnt(wait_vm(kStageWait));
                lds_barrier();
                issue_q(int(t), st + kMBQ, bq);
                issue_c(int(t), st + kMBC, bc);
                bc = bc + 1 == kMBC ? 0 : bc + 1;
                bq = (bq + 1) & (kMBQ - 1);
                read_frags(bc, bq, 0, fa0, fb0);
                __builtin_amdgcn_sched_barrier(0);
            }
            mma(fa1, fb1);
        }
        // every wave is done with the tile's last stage's buffers (bc, bq): the selection's
        // LDS until the deferred loads refill them
        lds_barrier();
        stg_lo = reinterpret_cast<float*>(&sh.e[bc][0]);
        stg_hi = reinterpret_cast<float*>(&sh.q[bq][0]);
        wbase = wq ? stg_hi : stg_lo;
        obase = (tid < 128 ? stg_lo : stg_hi) + (tid & 127) * kMChunk;
        // (The order in which rows are offered does not change the result: the list keeps
        // the K least keys of a total order.)
        bool full_way = false;
        if (sample) sample_tile(t0);
        else full_way = (sh.wfast[0] & sh.wfast[1] & sh.wfast[2] & sh.wfast[3]) == 0u;
        if (!sample && !full_way) {
            // Slot selection, in three steps.
            // 1. Each lane tests its 16 dots of each 32 x 32 block at once: their maximum
            //    (NaN ignored) against the query's threshold, and their sum, NaN when a dot
            //    is NaN (offered, as the full way offers NaN). A lane that reaches it appends
            //    the block's 16 dots to its wave's records (ballot compaction).
            // 2. The wave's lanes take one record each and offer every dot not below the
            //    threshold: a slot index from the query's counter, then (row, dot).
            // 3. The owners insert their candidates.
            // More than kMRec records in a wave or kMSlots candidates for a query: the tile
            // goes the full way. The lane index is laundered so that the addresses and rows
            // derived from it are computed here rather than held across the tile loop.
            int ut = tid;
            asm volatile("" : "+v"(ut));
            const int ul = ut & 63, ulm = ut & 31;
            u32x4* const rec = &sh.e[bc][wave * 4 * kMRec];
            uint2* const slots = reinterpret_cast<uint2*>(&sh.q[bq][0]);
            const uint32_t rowb = uint32_t(wr * 128 + 4 * (ul >> 5));
            uint32_t nrec = 0;                                          // uniform
            // whether a lane's 16 dots of a block can reach threshold th: their maximum (NaN
            // ignored) is not below it, or their sum is NaN (a NaN dot), as trees
            auto block_hit = [](const f32x16& xv, float th) {
                const float m = fmaxf(fmaxf(fmaxf(fmaxf(xv[0], xv[1]), xv[2]), fmaxf(fmaxf(xv[3], xv[4]), xv[5])),
                                      fmaxf(fmaxf(fmaxf(xv[6], xv[7]), xv[8]), fmaxf(fmaxf(xv[9], xv[10]), xv[11])));
                const float m2 = fmaxf(fmaxf(fmaxf(xv[12], xv[13]), xv[14]), xv[15]);
                const float s0 = (xv[0] + xv[1]) + (xv[2] + xv[3]), s1 = (xv[4] + xv[5]) + (xv[6] + xv[7]);
                const float s2 = (xv[8] + xv[9]) + (xv[10] + xv[11]), s3 = (xv[12] + xv[13]) + (xv[14] + xv[15]);
                const float sum = (s0 + s1) + (s2 + s3);
                return !(fmaxf(m, m2) < th) || sum != sum;
            };
            // append the block of the lanes that hit to the wave's records
            auto put_records = [&](const f32x16& xv, bool hit, uint64_t hb, int ql, int rt) {
                const uint32_t idx = nrec + __builtin_amdgcn_mbcnt_hi(uint32_t(hb >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(hb), 0u));
                if (hit && idx < uint32_t(kMRec)) {
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        rec[c * kMRec + idx] = __builtin_bit_cast(u32x4, float4{xv[4 * c], xv[4 * c + 1], xv[4 * c + 2], xv[4 * c + 3]});
                    sh.rhdr[wave][idx] = (uint32_t(ql) << 8) | (rowb + uint32_t(rt * 32));
                }
                nrec += uint32_t(__popcll(hb));
            };
            // The 16 blocks unrolled, each block's accumulators passed through an empty asm
            // so that they are read from AGPRs once, where the block is tested. (A rolled
            // loop with a switch over the blocks compiled to a chain of cases that read up to
            // four blocks per iteration, twice each: 4.9-5.5 us per tile for this step.)
            auto one_block = [&](const f32x16& xa, int rt, int qt) {
                f32x16 x = xa;
                asm volatile("" : "+v"(x));
                const int ql = wq * 128 + qt * 32 + ulm;
                const bool hit = block_hit(x, sh.thr[ql]);
                const uint64_t hb = __ballot(hit);
                if (hb != 0u) put_records(x, hit, hb, ql, rt);
            };
#pragma unroll
            for (int rt = 0; rt < 4; ++rt)
#pragma unroll
                for (int qt = 0; qt < 4; ++qt) one_block(acc[rt][qt], rt, qt);
            bool over = nrec > uint32_t(kMRec);
            if (!over && uint32_t(ul) < nrec) {
                const uint32_t hdr = sh.rhdr[wave][ul];
                const uint32_t q = hdr >> 8, rb = hdr & 255u;
                const float th = sh.thr[q];
                float xv[16];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const float4 f4 = __builtin_bit_cast(float4, rec[c * kMRec + ul]);
                    xv[4 * c] = f4.x; xv[4 * c + 1] = f4.y; xv[4 * c + 2] = f4.z; xv[4 * c + 3] = f4.w;
                }
                // the record's dots not below the threshold: one slot reservation for all
                // of them, then each dot read back from the record by its index
                uint32_t hits = 0;
#pragma unroll
                for (int v = 0; v < 16; ++v) hits |= uint32_t(!(xv[v] < th)) << v;
                const uint32_t n = uint32_t(__popc(hits));
                uint32_t i = n != 0u ? atomicAdd(&sh.cnt[q], n) : 0u;
                if (i + n > uint32_t(kMSlots)) over = true;
                const uint32_t* const rw = reinterpret_cast<const uint32_t*>(rec);
                for (; hits != 0u && i < uint32_t(kMSlots); ++i) {
                    const uint32_t v = uint32_t(__builtin_ctz(hits));
                    hits &= hits - 1u;
                    slots[q * kMSlots + ((i + q) & (kMSlots - 1))] =
                        uint2{rb + 8u * (v >> 2) + (v & 3u), rw[((v >> 2) * kMRec + ul) * 4 + (v & 3u)]};
                }
            }
            const uint64_t ob = __ballot(over);
            if (lane == 0) sh.wover[wave] = ob != 0u ? 1u : 0u;
            lds_barrier();
            full_way = (sh.wover[0] | sh.wover[1] | sh.wover[2] | sh.wover[3]) != 0u;
            if (!full_way) {
                if (my_q < a.q) {
                    const uint32_t n = sh.cnt[ut];
                    for (uint32_t i = 0; i < n; ++i) {
                        const uint2 sl = slots[ut * kMSlots + ((i + uint32_t(ut)) & (kMSlots - 1))];
                        const int j = int(sl.x);
                        const int64_t row = t0 + j;
                        if (row >= r1 || row == my_self) continue;
                        const uint64_t key = make_key(__uint_as_float(sl.y), uint32_t(row));
                        if (key < list[K - 1]) reg_insert<K>(list, key);
                    }
                }
                // every owner has read its slots before the stage load below refills them
                lds_barrier();
            }
        }
        if (full_way) {
            // 32 rows at a time: the two waves holding them stage their raw scores, then the
            // owner of each query fuses its 32 scores and keeps its best K. Row half h is a
            // loop, not unrolled (the code then stays in the instruction cache); the four
            // 32-row tiles of a half are unrolled, so each stages a fixed accumulator.
#pragma unroll 1
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int rt = 0; rt < 4; ++rt) {
                    if (wr == h) stage_rows(acc[rt]);
                    lds_barrier();
                    if (my_q < a.q) select_chunk(4 * h + rt, t0);
                    lds_barrier();
                }
            }
        }
        if (!sample) publish();                // the next tile's thresholds
        // the deferred loads, into the buffers the selection used
        issue_q(int(t), NS - 1 + kMBQ, bq);
        issue_c(int(t), NS - 1 + kMBC, bc);
    }
    // the last stages' loads (past the last tile) must land before the workgroup ends
    __builtin_amdgcn_s_waitcnt(wait_vm(0));
    if (sample) {
        // query wq 128 + qt 32 + lm gets block (rt, qt)'s maximum in slot wr 8 + lh 4 + rt,
        // keyed with the block's first row (distinct per slot and range; only the score is used)
        static_assert(K == 16, "16 block maxima per query and range");
#pragma unroll
        for (int qt = 0; qt < 4; ++qt) {
            const int qg = q0 + wq * 128 + qt * 32 + lm;
            if (qg < a.q) {
                uint64_t* out = a.part + ((int64_t(qg / kPartQ) * a.n_rranges + r_id) * kPartQ + (qg % kPartQ)) * K +
                                wr * 8 + lh * 4;
#pragma unroll
                for (int rt = 0; rt < 4; ++rt)
                    out[rt] = make_key(gmx[qt * 4 + rt], uint32_t(r0 + wr * 128 + rt * 32 + 4 * lh));
            }
        }
    } else if (my_q < a.q) {
        uint64_t* out = a.part + ((int64_t(my_q / kPartQ) * a.n_rranges + r_id) * kPartQ + (my_q % kPartQ)) * K;
#pragma unroll
        for (int j = 0; j < K; ++j) out[j] = list[j];
    }
}

template <int NS, int K>
int launch_mm_t(const BatchArgs& a, hipStream_t s) {
    const unsigned grid = unsigned(a.n_rranges * ((a.q + kMQ - 1) / kMQ));
    MARS_LAUNCH((k_batch_mm<NS, K>), dim3(grid), dim3(kMThreads), 0, s, a);
    return MARS_OK;
}

template <int K>
int launch_mm_k(const BatchArgs& a, hipStream_t s) {
    switch (a.d / kMK) {
        case 8: return launch_mm_t<8, K>(a, s);
        case 12: return launch_mm_t<12, K>(a, s);
        case 16: return launch_mm_t<16, K>(a, s);
        case 24: return launch_mm_t<24, K>(a, s);
        default: return set_error(MARS_ERR_UNSUPPORTED, "batched scoring: embedding_dim %d not in {256,384,512,768}", a.d);
    }
}

}  // namespace

int launch_batch_mm(const BatchArgs& a, hipStream_t s) {
    // the k-NN builders keep 16 candidates per query and row range (batch_kpart(k) = 16)
    MARS_CHECK(a.k > 8 && a.k <= 16, MARS_ERR_UNSUPPORTED, "k_batch_mm keeps 16 keys per query (asked %d)", a.k);
    MARS_CHECK(a.q_plain == 0, MARS_ERR_INVALID, "k_batch_mm scores neighbour searches only (%d of %d queries fused)",
               a.q_plain, a.q);
    MARS_CHECK(a.floor_keys == nullptr || (a.floor_k >= 1 && a.floor_k <= 16), MARS_ERR_INVALID,
               "batched scoring: floor of %d keys per query", a.floor_k);
    return launch_mm_k<16>(a, s);
}

}  // namespace mars
