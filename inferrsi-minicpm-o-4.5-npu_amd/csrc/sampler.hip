// Fused token-sampling kernels for MI355X (gfx950) behind the C-ABI of include/mi355x_sampler.h.
//
// A row of V logits is cut into S vocabulary slices of at most ~10K elements,
// one 256-thread workgroup each.  Whole rows are assigned to XCDs, so a row's
// slices share an L2.
//
// sample_kernel, per slice workgroup:
//   1. issues the slice's 16-byte logit loads, its allowed-mask words and the
//      row's history, then reads the row's parameters,
//   2. counts the history ids that fall in the slice into an LDS table and
//      applies the row's pipeline element by element — EOS censor, repetition /
//      frequency / presence penalties, allowed-token bitmask, temperature, in
//      the order of engine/talker_sampler.py:142-156 — keeping the values in
//      registers,
//   3. publishes a summary (max, first argmax, sum of exp relative to its max,
//      per-sub-block sums) and, by row kind, its candidates (every value >= tau,
//      the c-th largest per-thread maximum, in vocabulary order) and for top-p
//      rows without top-k also a probability-mass histogram on a 1/8-logit grid,
//   4. counts itself in on the row's arrival word.  The last workgroup to arrive
//      finalises the row:
//        greedy rows: first index of the maximum;
//        top-k rows and small nuclei: sorts the candidate keys (rank sort or a
//          register bitonic network), reads the top-k threshold and the top-p
//          cut over the sorted masses, and draws by inverse CDF over the
//          candidates in vocabulary order;
//        unfiltered rows: walks the sub-block sums to the sub-block holding
//          u * total and rescans only that sub-block;
//        larger nuclei: merges the histograms and finds the bin that holds
//          the top-p boundary (see below);
//        anything the fast paths cannot prove exactly, or a row whose slices
//          ran on more than one XCD: streams the row again and selects by radix
//          over order-preserving keys.
//   5. a top-p row without top-k holds its other slices after they arrive: each
//      waits on the row's decision word, which the finaliser sets once it knows
//      whether the boundary bin is needed.  If it is, every slice (the finaliser
//      after re-reading its own) publishes from its registers the values inside
//      the bin and the sums of everything above it, and the last to arrive again
//      resolves the top-p threshold exactly and draws.  A waiting slice only ever
//      waits for the finaliser, which arrived last and is already running, so the
//      wait ends however the workgroups are scheduled.
// Apart from that wait, the only cross-workgroup protocol is publish / arrive /
// read on the per-row arrival word, which the finaliser resets for the next
// launch.

#include <hip/hip_runtime.h>

#include <climits>
#include <cstdarg>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <string>

#include "mi355x_sampler.h"

namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / 64;
constexpr int kNV = 40;              // register slots per thread in a slice
constexpr int kMaxGroups = 4;
constexpr int kMaxSlices = 64;
constexpr int kMaxSB = kNV / 4 * kWaves;  // sub-blocks per slice (fp32: 10 rounds x 4 waves)
constexpr int kCapSlice = 512;       // candidates one slice may publish
constexpr int kCapRow = 2048;        // candidates the finaliser sorts in LDS
constexpr int kCntWords = kBlock * kNV / 2;  // two u16 counts per word: covers every element of a slice
constexpr int kNB = 256;             // histogram bins below a slice's top bin
constexpr int kAlphaTable = 64;      // rep**n for n < 64 kept in LDS (larger counts take a slow call)
constexpr float kBinScale = 8.0f;    // bins of 1/8 logit
constexpr int kMaxRows = 16384;      // rows per launch
constexpr int kCounterStride = 32;  // u32 words between rows' counters: one 128-byte line each (no atomic contention)
constexpr int kDecisionWord = 2;    // in a row's counter line, after the 64-bit arrival word
constexpr int64_t kCounterBytes = 4 * kCounterStride * (int64_t)kMaxRows;
constexpr int64_t kPendingBytes = 64 * (int64_t)kMaxRows;
constexpr int64_t kPad = -1;
constexpr double kMassScale = 1099511627776.0;  // 2^40 fixed-point units of exp(x - max)

// The finaliser's decision for the held slices of a top-p row without top-k (0: not yet decided).
enum : uint32_t { kHeldDone = 1, kHeldBin = 2 };
constexpr int kSpinLimit = 1 << 22;  // bound on a held slice's wait (each try sleeps ~64 clocks): ~0.2 s

struct DevGroup {
    const char* logits;
    int64_t row_stride;
    int32_t es;        // element size in bytes (2 = bf16, 4 = f32)
    int32_t vocab;
    int32_t rows;
    int32_t semantics;
    int32_t flags;
    int32_t min_keep;
    const float* temperature;
    const int32_t* top_k;
    const float* top_p;
    const float* repetition;
    const float* presence;
    const float* frequency;
    float t_val, p_val, rep_val, pres_val, freq_val;
    int32_t k_val;
    const float* alpha_lut;
    int32_t alpha_lut_len;
    int32_t hist_len;
    const char* history;
    int64_t hist_stride;
    int32_t hist_i64;
    int32_t hist_mode;
    int32_t* hist_head;
    const uint32_t* allowed;
    int64_t allowed_stride;
    int32_t eos, min_new, max_new, rng;
    const int64_t* seeds;
    int64_t* steps;
    const int64_t* row_ids;
    const float* uniforms;
    const uint8_t* active;
    uint8_t* finished;
    int64_t* tokens;
    float* processed;
    int64_t processed_stride;
    float* probs;
    int64_t probs_stride;
    // derived by the host
    int32_t slices;
    int32_t slice_len;
    int32_t block_begin;
    int32_t row_begin;       // index of the group's first row among all rows of the launch
    char* ws;                // the group's row regions
    unsigned int* counters;  // arrival counters (fixed workspace prefix, zero between launches)
    char* pending;           // per-row pending records (fixed workspace region)
    int32_t gi;              // index of this group in the launch
    int32_t tiles;           // rows can be top-p without top-k: their row regions hold the processed-tile area
    int64_t ws_row_bytes;
};

// A pointer into global memory as such: accesses through it compile to global (not flat) instructions, which
// count only against the vector-memory counter.
template <class T>
__device__ __forceinline__ T* gp(T* p) {
    return (T*)(__attribute__((address_space(1))) T*)p;
}

// Whole rows are assigned to XCDs: block b runs on XCD b % 8 (the dispatcher's round-robin), as the (b / 8)-th
// slice of that XCD's rows, which are rows [seg_row[x][g], + seg_rows[x][g]) of each group g in turn.
struct KernelArgs {
    DevGroup g[kMaxGroups];
    int32_t n_groups;
    int32_t per_xcd;
    int32_t seg_row[8][kMaxGroups];
    int32_t seg_rows[8][kMaxGroups];
};

struct SliceSummary {
    float m;                 // max value of the slice (-inf if none finite)
    float g;                 // the published candidates hold every value >= g (+inf: none published)
    double z;                // sum of exp(x - m) over the slice
    int32_t argmax;          // first index of m
    int32_t ncand;
    int32_t overflow;
    int32_t hb;              // histogram: top bin floor(8 m)
    unsigned long long under_q;  // histogram: mass below the window (2^40 units of exp(x - m))
    int32_t under_n;
    int32_t n_hi;            // nucleus pass: values above the boundary bin
    double hi_mass;          // nucleus pass: their sum of exp(x - M); first pass of a top-p-only row: the sum of
                             // exp(x - m) over its published candidates
    int32_t pad_[2];
};
static_assert(sizeof(SliceSummary) == 64, "summary layout");

struct Pending {
    int32_t mode_;
    float lo_v, hi_v;        // boundary bin [lo_v, hi_v)
    float m;                 // row max
    double z;                // full-row sum of exp(x - m)
    double target;           // top_p * z
    int32_t pad_[8];
};
static_assert(sizeof(Pending) == 64, "pending layout");

struct Cand {
    float f;
    int32_t j;
};

// Row workspace: [S summaries][S x kMaxSB sub-block sums][S x kNB bin counts][S x kNB bin masses]
// [S x kCapSlice cands] and, for groups that can have top-p rows without top-k, [S x kNV x kBlock processed values]
// (a slice's tile as its threads hold it, slot-major: the boundary-bin draw reads one sub-block of it).
struct RowWs {
    SliceSummary* summ;
    double* sb;
    uint32_t* hcnt;
    unsigned long long* hmass;
    Cand* cand;
    float* tile;  // null without the tile area
};

__host__ __device__ __forceinline__ int64_t row_ws_bytes(int s, bool tiles) {
    int64_t b = (int64_t)s * (sizeof(SliceSummary) + 8 * kMaxSB + 12 * kNB + sizeof(Cand) * kCapSlice);
    if (tiles) b += (int64_t)s * kNV * kBlock * 4;
    return (b + 255) & ~(int64_t)255;
}

__device__ __forceinline__ RowWs row_ws(char* base, int s, bool tiles) {
    RowWs w;
    w.summ = (SliceSummary*)base;
    w.sb = (double*)(base + (int64_t)s * sizeof(SliceSummary));
    w.hcnt = (uint32_t*)((char*)w.sb + (int64_t)s * 8 * kMaxSB);
    w.hmass = (unsigned long long*)((char*)w.hcnt + (int64_t)s * 4 * kNB);
    w.cand = (Cand*)((char*)w.hmass + (int64_t)s * 8 * kNB);
    w.tile = tiles ? (float*)((char*)w.cand + (int64_t)s * sizeof(Cand) * kCapSlice) : nullptr;
    return w;
}

// The penalty of an element seen n times: x < 0 ? x * a : x / a, minus freq * n, minus pres (n > 0), with
// a = rep**n.  Entry 0 is the identity.  ra = RN(1 / a) serves the corrected-reciprocal division.
struct PenEntry {
    float a, ra, fn, pn;
};

// Allowed-bit words of a slice in LDS: word k covers elements [32 * (wb + k), +32) with wb = first >> 5.
constexpr int kMaskWords = kBlock * kNV / 32 + 2;

struct Smem {
    union alignas(16) {
        uint32_t cnt[kCntWords];  // history counts of a slice (u16 pairs)
        struct {
            float val[kCapRow];   // finaliser: candidate values, vocabulary order
            int32_t id[kCapRow];  //            their ids
            uint32_t key[kCapRow];  //          order keys, sorted descending
        } c;
        double sbs[kMaxSlices * kMaxSB];  // finaliser: sub-block totals
        struct {
            double mass[kNB];
            uint32_t cnt[kNB];
        } h;
    } u;
    float tmax[kBlock];
    uint32_t hcnt[kNB];
    unsigned long long hmass[kNB];
    double sbw[kMaxSB];
    PenEntry pen[kAlphaTable];
    uint32_t mask[kMaskWords];
    double red_d[kWaves];
    unsigned long long red_u[kWaves];
    float red_f[kWaves];
    int32_t red_i[kWaves];
    double tile_sum[kMaxSlices];  // streaming draw: slice sums; finaliser: per-slice scale exp(m_s - m)
    struct {
        double z, cmass;
        float m, gmax;
        int32_t am, ntot, overflow;
    } fin;  // the finaliser's merge of the slice summaries
    SliceSummary summ[kMaxSlices];
    Cand stage[kCapSlice];  // a slice's published candidates, copied out by wave 0
    int32_t coff[kMaxSlices + 1];  // finaliser: candidate offsets per slice
    int32_t sel_bin;
    int32_t sel_rem;
    int32_t is_last;
    int32_t foreign;  // the row's slices ran on more than one XCD: their publications are not readable here
    uint32_t decision;  // held slices: the finaliser's decision (kHeld*), 0 before it is made
    uint32_t kmin, kmax;  // boundary bin: the extreme keys of the sub-bucket holding the cut
    Pending held;       // held slices: the boundary bin
    unsigned long long sel_acc;
    float sel_tau;
};

__device__ __forceinline__ uint32_t ord_key(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_float(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__device__ __forceinline__ bool finite_f(float f) { return f > -INFINITY && f < INFINITY; }

__device__ __forceinline__ int bin_of(float f) {
    return (int)floorf(fminf(fmaxf(f * kBinScale, -1.0e9f), 1.0e9f));
}

// ---------------------------------------------------------------- cross-workgroup publication
// Data one workgroup publishes for another (summaries, sums, histograms, candidates) goes out as plain stores,
// which the CU's write-through L1 passes to the L2, and is read back with relaxed device-scope atomic loads, which
// bypass the reader's L1 and read the L2.  The publisher orders its stores before its arrival count by waiting
// for them.  Every workgroup of a row runs on one XCD (the block-to-row mapping groups a row's slices by
// blockIdx % 8, the stride of the dispatcher's round-robin over XCDs), so they share that L2: no cache writeback
// or invalidation is needed, and nothing is written through to HBM.

template <class T>
__device__ __forceinline__ void pub_st(T* p, T v) {
    *p = v;
}

template <class T>
__device__ __forceinline__ T pub_ld(const T* p) {
    return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void pub_st_cand(Cand* p, Cand v) {
    pub_st((unsigned long long*)p, ((unsigned long long)(uint32_t)v.j << 32) | __float_as_uint(v.f));
}

__device__ __forceinline__ Cand pub_ld_cand(const Cand* p) {
    const unsigned long long w = pub_ld((const unsigned long long*)p);
    return Cand{__uint_as_float((uint32_t)w), (int32_t)(uint32_t)(w >> 32)};
}

__device__ __forceinline__ void pub_st_summary(SliceSummary* d, const SliceSummary& v) {
    pub_st(&d->m, v.m);
    pub_st(&d->g, v.g);
    pub_st(&d->z, v.z);
    pub_st(&d->argmax, v.argmax);
    pub_st(&d->ncand, v.ncand);
    pub_st(&d->overflow, v.overflow);
    pub_st(&d->hb, v.hb);
    pub_st(&d->under_q, v.under_q);
    pub_st(&d->under_n, v.under_n);
    pub_st(&d->n_hi, v.n_hi);
    pub_st(&d->hi_mass, v.hi_mass);
}

__device__ __forceinline__ SliceSummary pub_ld_summary(const SliceSummary* d) {
    SliceSummary v;
    v.m = pub_ld(&d->m);
    v.g = pub_ld(&d->g);
    v.z = pub_ld(&d->z);
    v.argmax = pub_ld(&d->argmax);
    v.ncand = pub_ld(&d->ncand);
    v.overflow = pub_ld(&d->overflow);
    v.hb = pub_ld(&d->hb);
    v.under_q = pub_ld(&d->under_q);
    v.under_n = pub_ld(&d->under_n);
    v.n_hi = pub_ld(&d->n_hi);
    v.hi_mass = pub_ld(&d->hi_mass);
    v.pad_[0] = v.pad_[1] = 0;
    return v;
}

// ---------------------------------------------------------------- block primitives (every thread calls them)

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

// threadIdx.x through an opaque copy: index arithmetic derived from it is recomputed where it is used instead of
// being shared with (and kept live from) an earlier phase.
__device__ __forceinline__ int fresh_tid() {
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}
__device__ __forceinline__ int fresh_lane() { return fresh_tid() & 63; }

// Cross-lane moves.  The fixed xor partners are all VALU moves: DPP for 1 and 2 (quad permutes), 4 (row half
// mirror, then a quad reversal) and 8 (rotate by 8 in a row of 16), gfx950's permlane swaps for 16 and 32.  The
// dynamic ones use ds_bpermute and compute their own lane arithmetic, so no lane index is shared (and kept live)
// across the kernel.
__device__ __forceinline__ uint32_t lane_mbcnt() {
    return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}

template <int O>
__device__ __forceinline__ uint32_t xor_lane(uint32_t x) {
    static_assert(O >= 1 && O <= 32 && (O & (O - 1)) == 0, "power-of-two offset");
    if constexpr (O == 1) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    } else if constexpr (O == 2) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    } else if constexpr (O == 4) {
        const int m = __builtin_amdgcn_update_dpp(0, (int)x, 0x141, 0xF, 0xF, false);  // lane i <- 7 - i (in 8)
        return (uint32_t)__builtin_amdgcn_update_dpp(0, m, 0x1B, 0xF, 0xF, false);      // then i <- 3 - i (in 4)
    } else if constexpr (O == 8) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x128, 0xF, 0xF, false);  // row_ror:8 = lane ^ 8
    } else if constexpr (O == 16) {
        // odd rows of the first result hold the even rows' values and even rows of the second the odd rows'
        const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
        return (lane_mbcnt() & 16u) ? r[0] : r[1];
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        return lane_mbcnt() < 32u ? r[1] : r[0];
    }
}

__device__ __forceinline__ uint32_t xor_lane_dyn(uint32_t x, int o) {
    return (uint32_t)__builtin_amdgcn_ds_bpermute((fresh_lane() ^ o) << 2, (int)x);
}

// lane l receives lane l - o (lanes below o receive a lane of the upper half; callers ignore them)
__device__ __forceinline__ uint32_t up_lane(uint32_t x, int o) {
    return (uint32_t)__builtin_amdgcn_ds_bpermute(((fresh_lane() - o) & 63) << 2, (int)x);
}

template <class T>
struct Lanes;  // moves a value through 32-bit lane moves
template <>
struct Lanes<uint32_t> {
    template <class F>
    __device__ static uint32_t mv(uint32_t x, F f) { return f(x); }
};
template <>
struct Lanes<int> {
    template <class F>
    __device__ static int mv(int x, F f) { return (int)f((uint32_t)x); }
};
template <>
struct Lanes<float> {
    template <class F>
    __device__ static float mv(float x, F f) { return __uint_as_float(f(__float_as_uint(x))); }
};
template <>
struct Lanes<unsigned long long> {
    template <class F>
    __device__ static unsigned long long mv(unsigned long long x, F f) {
        return ((unsigned long long)f((uint32_t)(x >> 32)) << 32) | f((uint32_t)x);
    }
};
template <>
struct Lanes<double> {
    template <class F>
    __device__ static double mv(double x, F f) {
        return __longlong_as_double((long long)Lanes<unsigned long long>::mv((unsigned long long)__double_as_longlong(x), f));
    }
};

template <int O, class T>
__device__ __forceinline__ T shfl_xor_c(T x) {
    return Lanes<T>::mv(x, [](uint32_t v) { return xor_lane<O>(v); });
}

template <class T>
__device__ __forceinline__ T shfl_xor_d(T x, int o) {
    return Lanes<T>::mv(x, [o](uint32_t v) { return xor_lane_dyn(v, o); });
}

template <class T>
__device__ __forceinline__ T shfl_up_d(T x, int o) {
    return Lanes<T>::mv(x, [o](uint32_t v) { return up_lane(v, o); });
}

// All 64 lanes end with op over the wave (a symmetric butterfly: every lane computes the same sums).
template <class T, class Op>
__device__ __forceinline__ T wave_reduce(T x, Op op) {
    x = op(x, shfl_xor_c<32>(x));
    x = op(x, shfl_xor_c<16>(x));
    x = op(x, shfl_xor_c<8>(x));
    x = op(x, shfl_xor_c<4>(x));
    x = op(x, shfl_xor_c<2>(x));
    x = op(x, shfl_xor_c<1>(x));
    return x;
}

// A DPP move (lanes without a source in the pattern, or in rows outside ROW_MASK, read 0).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_or_zero(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, ROW_MASK, 0xF, false);
}

// Inclusive scan over the wave's lanes, all in DPP moves: Hillis-Steele inside each row of 16 lanes (row_shr 1, 2,
// 4, 8), then the row totals (row_bcast:15 into rows 1 and 3, row_bcast:31 into rows 2 and 3).
template <class T>
__device__ __forceinline__ T wave_incl_scan(T x) {
    x += Lanes<T>::mv(x, dpp_or_zero<0x111, 0xF>);
    x += Lanes<T>::mv(x, dpp_or_zero<0x112, 0xF>);
    x += Lanes<T>::mv(x, dpp_or_zero<0x114, 0xF>);
    x += Lanes<T>::mv(x, dpp_or_zero<0x118, 0xF>);
    x += Lanes<T>::mv(x, dpp_or_zero<0x142, 0xA>);
    x += Lanes<T>::mv(x, dpp_or_zero<0x143, 0xC>);
    return x;
}

__device__ __forceinline__ float block_max(float x, Smem& sm) {
    x = wave_reduce(x, [](float a, float b) { return fmaxf(a, b); });
    __syncthreads();
    if (lane_id() == 0) sm.red_f[wave_id()] = x;
    __syncthreads();
    float r = sm.red_f[0];
    for (int i = 1; i < kWaves; ++i) r = fmaxf(r, sm.red_f[i]);
    return r;
}

__device__ __forceinline__ int block_min_i(int x, Smem& sm) {
    x = wave_reduce(x, [](int a, int b) { return min(a, b); });
    __syncthreads();
    if (lane_id() == 0) sm.red_i[wave_id()] = x;
    __syncthreads();
    int r = sm.red_i[0];
    for (int i = 1; i < kWaves; ++i) r = min(r, sm.red_i[i]);
    return r;
}

__device__ __forceinline__ int block_max_i(int x, Smem& sm) {
    x = wave_reduce(x, [](int a, int b) { return max(a, b); });
    __syncthreads();
    if (lane_id() == 0) sm.red_i[wave_id()] = x;
    __syncthreads();
    int r = sm.red_i[0];
    for (int i = 1; i < kWaves; ++i) r = max(r, sm.red_i[i]);
    return r;
}

__device__ __forceinline__ int block_sum_i(int x, Smem& sm) {
    x = wave_reduce(x, [](int a, int b) { return a + b; });
    __syncthreads();
    if (lane_id() == 0) sm.red_i[wave_id()] = x;
    __syncthreads();
    int r = 0;
    for (int i = 0; i < kWaves; ++i) r += sm.red_i[i];
    return r;
}

// Fixed reduction tree: the result does not depend on scheduling.
__device__ __forceinline__ double wave_sum_d(double x) {
    return wave_reduce(x, [](double a, double b) { return a + b; });
}

__device__ __forceinline__ double block_sum_d(double x, Smem& sm) {
    x = wave_sum_d(x);
    __syncthreads();
    if (lane_id() == 0) sm.red_d[wave_id()] = x;
    __syncthreads();
    double r = 0.0;
    for (int i = 0; i < kWaves; ++i) r += sm.red_d[i];
    return r;
}

__device__ __forceinline__ unsigned long long block_sum_u(unsigned long long x, Smem& sm) {
    x = wave_reduce(x, [](unsigned long long a, unsigned long long b) { return a + b; });
    __syncthreads();
    if (lane_id() == 0) sm.red_u[wave_id()] = x;
    __syncthreads();
    unsigned long long r = 0;
    for (int i = 0; i < kWaves; ++i) r += sm.red_u[i];
    return r;
}

// Three sums with one barrier pair (double, u64, int).
__device__ __forceinline__ void block_sum3(double& a, unsigned long long& b, int& c, Smem& sm) {
    a = wave_sum_d(a);
    b = wave_reduce(b, [](unsigned long long x, unsigned long long y) { return x + y; });
    c = wave_reduce(c, [](int x, int y) { return x + y; });
    __syncthreads();
    if (lane_id() == 0) {
        sm.red_d[wave_id()] = a;
        sm.red_u[wave_id()] = b;
        sm.red_i[wave_id()] = c;
    }
    __syncthreads();
    a = 0.0;
    b = 0ull;
    c = 0;
    for (int i = 0; i < kWaves; ++i) {
        a += sm.red_d[i];
        b += sm.red_u[i];
        c += sm.red_i[i];
    }
}

// Exclusive prefix from the lane-shifted inclusive scan (no subtraction).
__device__ __forceinline__ double block_excl_scan_d(double x, double& total, Smem& sm) {
    const double incl = wave_incl_scan(x);
    double excl = shfl_up_d(incl, 1);
    if (lane_id() == 0) excl = 0.0;
    __syncthreads();
    if (lane_id() == 63) sm.red_d[wave_id()] = incl;
    __syncthreads();
    double off = 0.0;
    total = 0.0;
    for (int i = 0; i < kWaves; ++i) {
        if (i < wave_id()) off += sm.red_d[i];
        total += sm.red_d[i];
    }
    return off + excl;
}

__device__ __forceinline__ unsigned long long block_excl_scan_u(unsigned long long x, unsigned long long& total,
                                                               Smem& sm) {
    const unsigned long long incl = wave_incl_scan(x);
    __syncthreads();
    if (lane_id() == 63) sm.red_u[wave_id()] = incl;
    __syncthreads();
    unsigned long long off = 0;
    total = 0;
    for (int i = 0; i < kWaves; ++i) {
        if (i < wave_id()) off += sm.red_u[i];
        total += sm.red_u[i];
    }
    return off + incl - x;
}

// ---------------------------------------------------------------- per-row context

struct Ctx {
    int row, slice, S, V, slice_len, grow;  // grow: row index among all rows of the launch
    int64_t step;
    float tdiv;        // temperature divisor (1 for greedy rows)
    float rtdiv;       // RN(1 / tdiv)
    float top_p;
    float rep, pres, freq;
    int k_eff;
    int min_keep_eff;  // min(min_keep, k_eff)
    bool greedy, hf, later, censor, forced, live, want_out, p_active;
    bool counts;       // history penalties apply: build the count table
    bool full_draw;    // no filter: every finite value survives
    bool cand_mode;    // top-k bounded: slices publish candidates
    bool nucleus;      // top-p without top-k: slices publish mass histograms, second pass resolves
    bool need_mass;    // slices publish exp sums (full-vocabulary normaliser, sub-block sums)
    int cand_target;   // per-slice candidate count target
};

// A row's parameters as loaded; the loads are issued before the slice's tile so that waiting for them does not
// wait for the tile (vector loads complete in order).
struct RowParams {
    int64_t step;
    float t, p, rep, pres, freq;
    int k;
    uint8_t act, fin;
};

// Row-uniform values into scalar registers (they arrive from vector loads).
__device__ __forceinline__ int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ float uni(float x) { return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x))); }
__device__ __forceinline__ int64_t uni(int64_t x) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x), hi = __builtin_amdgcn_readfirstlane((uint32_t)(x >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ void load_params(const DevGroup& G, int row, RowParams& q) {
    q.step = gp(G.steps) ? gp(G.steps)[row] : 0;
    q.t = gp(G.temperature) ? gp(G.temperature)[row] : G.t_val;
    q.p = gp(G.top_p) ? gp(G.top_p)[row] : G.p_val;
    q.rep = gp(G.repetition) ? gp(G.repetition)[row] : G.rep_val;
    q.pres = gp(G.presence) ? gp(G.presence)[row] : G.pres_val;
    q.freq = gp(G.frequency) ? gp(G.frequency)[row] : G.freq_val;
    q.k = gp(G.top_k) ? gp(G.top_k)[row] : G.k_val;
    q.act = gp(G.active) ? gp(G.active)[row] : (uint8_t)1;
    q.fin = gp(G.finished) ? gp(G.finished)[row] : (uint8_t)0;
}

// The loaded parameters, once they are needed, as scalars.
__device__ __forceinline__ void settle_params(RowParams& q) {
    q.step = uni(q.step);
    q.t = uni(q.t);
    q.p = uni(q.p);
    q.rep = uni(q.rep);
    q.pres = uni(q.pres);
    q.freq = uni(q.freq);
    q.k = uni(q.k);
    q.act = (uint8_t)uni((int)q.act);
    q.fin = (uint8_t)uni((int)q.fin);
}

__device__ __forceinline__ void init_ctx(const DevGroup& G, int row, int slice, RowParams q, Ctx& c) {
    settle_params(q);
    c.row = row;
    c.slice = slice;
    c.grow = G.row_begin + row;
    c.S = G.slices;
    c.V = G.vocab;
    c.slice_len = G.slice_len;
    c.step = q.step;
    const float t = q.t;
    c.greedy = !(t > 0.f);
    c.tdiv = c.greedy ? 1.0f : t;
    c.rtdiv = 1.0f / c.tdiv;
    c.top_p = q.p;
    c.rep = q.rep;
    c.pres = q.pres;
    c.freq = q.freq;
    const int k = q.k;
    if ((G.flags & MIS_TOPK_ZERO_DISABLES) && k <= 0)
        c.k_eff = c.V;
    else
        c.k_eff = min(max(k, G.min_keep), c.V);
    c.min_keep_eff = min(G.min_keep, c.k_eff);
    c.p_active = !((G.flags & MIS_TOPP_ONE_DISABLES) && c.top_p >= 1.0f);
    c.hf = G.semantics == MIS_HF;
    c.later = c.step > 0;
    c.censor = G.eos >= 0 && c.step < (int64_t)G.min_new;
    c.forced = G.eos >= 0 && G.max_new > 0 && c.step >= (int64_t)G.max_new - 1;
    c.live = q.act != 0 && q.fin == 0;
    c.want_out = gp(G.processed) != nullptr || gp(G.probs) != nullptr;
    const bool pen = G.hist_len > 0 && gp(G.history) != nullptr &&
                     (c.rep != 1.0f || c.pres != 0.0f || c.freq != 0.0f || gp(G.alpha_lut) != nullptr);
    c.counts = pen && (!c.hf || c.later);
    const bool filters = !c.greedy && (!c.hf || c.later);
    c.full_draw = !c.greedy && (!filters || (c.k_eff >= c.V && !c.p_active));
    const int per_slice = (11 * c.k_eff + 10 * c.S - 1) / (10 * c.S) + 8;  // 1.1 k / S + 8
    c.cand_target = min(per_slice, kBlock);
    c.cand_mode = filters && !c.full_draw && per_slice <= kBlock && c.k_eff <= kCapRow / 2;
    c.nucleus = filters && !c.full_draw && !c.cand_mode && c.k_eff >= c.V && c.p_active;
    if (c.nucleus) c.cand_target = min(kBlock, kCapRow / (2 * c.S));  // a small nucleus resolves from these
    c.need_mass = c.full_draw || c.nucleus || (c.hf && filters && c.p_active);
}

__device__ __forceinline__ void init_ctx(const DevGroup& G, int row, int slice, Ctx& c) {
    RowParams q;
    load_params(G, row, q);
    init_ctx(G, row, slice, q, c);
}

// ---------------------------------------------------------------- the element pipeline

// rep**n by binary powering in double (<= 32 products, relative error < 4e-15) rounded once to float, or the
// caller's table where it covers n.
__device__ __forceinline__ float alpha_exact(const DevGroup& G, float rep, int n) {
    if (gp(G.alpha_lut) != nullptr && n < G.alpha_lut_len) return gp(G.alpha_lut)[n];
    double r = 1.0, b = (double)rep;
    for (unsigned e = (unsigned)n; e; e >>= 1) {
        if (e & 1u) r *= b;
        b *= b;
    }
    return (float)r;
}

__device__ __forceinline__ PenEntry pen_entry(const DevGroup& G, const Ctx& c, int n) {
    PenEntry e;
    if (n == 0) {
        e.a = 1.0f;
        e.ra = 1.0f;
        e.fn = 0.0f;
        e.pn = 0.0f;
    } else {
        e.a = alpha_exact(G, c.rep, n);
        e.ra = 1.0f / e.a;
        e.fn = c.freq * (float)n;  // built with -ffp-contract=off: product and difference round separately
        e.pn = c.pres;
    }
    return e;
}

// x / d rounded to nearest from r = RN(1/d): q = RN(x * r) is faithful, the residual x - q*d is exact in one
// fma, and one correction RN(q + r * residual) rounds the quotient correctly (Markstein).  The residual is formed
// as q*d - x so a zero x keeps its sign.  Checked bit-exact against IEEE division on 33.6 M pairs with
// 2^-100 <= |x| < 2^64 and 2^-16 <= d <= 2^16 (every divisor mantissa at one exponent); zero is exact too.
__device__ __forceinline__ float div_rn(float x, float d, float r) {
    const float q = x * r;
    const float e = fmaf(q, d, -x);
    return fmaf(-e, r, q);
}

// The raw logits the corrected-reciprocal pipeline takes: zero, or 2^-40 <= |x| < 2^40.  With the divisors in
// [2^-16, 2^16] and the penalty table's freq*n and presence zero or in [2^-60, 2^40] (checked per row), every
// operand a division then sees is zero or in [2^-100, 2^64).
__device__ __forceinline__ bool raw_in_range(float x) {
    const uint32_t u = __float_as_uint(x) & 0x7fffffffu;
    return u - 0x2b800000u < 0x28000000u || u == 0u;  // [2^-40, 2^40)
}

__device__ __forceinline__ bool table_term_ok(float v) {
    const float a = fabsf(v);
    return a == 0.f || (a >= 0x1p-60f && a <= 0x1p40f);
}

__device__ __forceinline__ bool divisor_in_range(float d) { return d >= 0x1p-16f && d <= 0x1p16f; }

__device__ __forceinline__ float pen_exact(float x, const PenEntry& e) {
    x = x < 0.f ? x * e.a : x / e.a;
    x = x - e.fn;
    return x - e.pn;
}

__device__ __forceinline__ float penalize(float x, int n, const DevGroup& G, const Ctx& c, const Smem& sm) {
    return pen_exact(x, n < kAlphaTable ? sm.pen[n] : pen_entry(G, c, n));
}

__device__ __forceinline__ float transform(float x, int j, int n, bool allowed, const DevGroup& G, const Ctx& c,
                                           const Smem& sm) {
    if (c.hf) {
        x = x / c.tdiv;
        if (n > 0) x = penalize(x, n, G, c, sm);
        if (!allowed) x = -INFINITY;
    } else {
        if (c.censor && j == G.eos) x = -INFINITY;
        if (n > 0) x = penalize(x, n, G, c, sm);
        if (!allowed) x = -INFINITY;
        x = x / c.tdiv;
    }
    return x;
}

// History counts of the elements [lo, hi) into sm.u.cnt as u16 pairs, element j at slot j - base (base <= lo;
// words [0, words) are cleared first), and the penalty table into sm.pen.  Entries < 0 (PAD) or >= V are empty.
// The history is loaded before the table is cleared, so the loads overlap the clearing barrier.  Ends with a
// barrier; returns nonzero (in every thread) when a table entry's rep**n lies outside [2^-16, 2^16].
__device__ __forceinline__ void count_id(Smem& sm, int64_t h, int base, int lo, int hi) {
    if (h >= lo && h < hi) {
        const int s = (int)(h - base);
        atomicAdd(&sm.u.cnt[s >> 1], 1u << (16 * (s & 1)));
    }
}

__device__ __forceinline__ int clear_counts(const DevGroup& G, const Ctx& c, int words, Smem& sm) {
    __syncthreads();  // the union may still be in use
    for (int w = threadIdx.x; w < words; w += kBlock) sm.u.cnt[w] = 0u;
    int bad = 0;
    if (threadIdx.x < kAlphaTable) {
        const PenEntry e = pen_entry(G, c, threadIdx.x);
        sm.pen[threadIdx.x] = e;
        bad = !divisor_in_range(e.a) || !table_term_ok(e.fn) || !table_term_ok(e.pn);
    }
    return bad;
}

__device__ __forceinline__ const char* hist_row(const DevGroup& G, int row) {
    return gp(G.history) + (int64_t)row * G.hist_stride * (G.hist_i64 ? 8 : 4);
}

// int32 ids, 16-byte aligned rows, W % 4 == 0: the history is read as int4.
__device__ __forceinline__ bool hist_vec(const DevGroup& G, const char* hrow) {
    return !G.hist_i64 && (((uintptr_t)hrow) & 15) == 0 && (G.hist_len & 3) == 0;
}

// pre: the first kBlock * 4 int4 of the row's history, already loaded (vector layout only), or null.
__device__ __forceinline__ int build_counts(const DevGroup& G, const Ctx& c, int base, int lo, int hi, int words,
                                            Smem& sm, const int4* pre = nullptr) {
    const char* hrow = hist_row(G, c.row);
    const int W = G.hist_len;
    const bool vec = hist_vec(G, hrow);
    int bad = 0;
    if (vec) {
        const int4* h4 = (const int4*)hrow;
        const int nv = W >> 2;
        for (int b0 = 0; b0 < nv || b0 == 0; b0 += kBlock * 4) {
            int4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = b0 + u * kBlock + threadIdx.x;
                v[u] = (b0 == 0 && pre != nullptr) ? pre[u] : i < nv ? h4[i] : make_int4(-1, -1, -1, -1);
            }
            if (b0 == 0) {
                bad = clear_counts(G, c, words, sm);
                __syncthreads();
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                count_id(sm, v[u].x, base, lo, hi);
                count_id(sm, v[u].y, base, lo, hi);
                count_id(sm, v[u].z, base, lo, hi);
                count_id(sm, v[u].w, base, lo, hi);
            }
        }
    } else {
        // one loop per id width, loads from clamped indices (a load under a branch would be waited for at the join)
        auto scan = [&](auto id_type) {
            using Id = decltype(id_type);
            const Id* hp = (const Id*)hrow;
            for (int b0 = 0; b0 < W || b0 == 0; b0 += kBlock * 8) {
                int64_t h[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) h[u] = (int64_t)hp[max(min(b0 + u * kBlock + (int)threadIdx.x, W - 1), 0)];
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (b0 + u * kBlock + (int)threadIdx.x >= W) h[u] = -1;
                if (b0 == 0) {
                    bad = clear_counts(G, c, words, sm);
                    __syncthreads();
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) count_id(sm, h[u], base, lo, hi);
            }
        };
        if (G.hist_i64)
            scan(int64_t{});
        else
            scan(int32_t{});
    }
    return __syncthreads_or(bad);
}

__device__ __forceinline__ int count_of(const Smem& sm, int slot) {
    return (int)((sm.u.cnt[slot >> 1] >> (16 * (slot & 1))) & 0xffffu);
}

// Placement of a slice in memory: 16-byte chunks from the aligned address at or below element lo.
struct Geo {
    uintptr_t base;
    int first;   // element index of the first byte of chunk 0 (may be < lo)
    int lo, hi;
    int nchunk;
};

template <int ES>
__device__ __forceinline__ Geo slice_geo_at(const DevGroup& G, int row, int s) {
    Geo g;
    g.lo = s * G.slice_len;
    g.hi = min(G.vocab, g.lo + G.slice_len);
    const char* rowp = gp(G.logits) + (int64_t)row * G.row_stride * ES;
    const uintptr_t lo_addr = (uintptr_t)(rowp + (int64_t)g.lo * ES);
    g.base = lo_addr & ~(uintptr_t)15;
    g.first = g.lo - (int)((lo_addr - g.base) / ES);
    g.nchunk = (int)(((uintptr_t)(rowp + (int64_t)g.hi * ES) - g.base + 15) / 16);
    return g;
}

template <int ES>
__device__ __forceinline__ Geo slice_geo(const DevGroup& G, const Ctx& c, int s) {
    return slice_geo_at<ES>(G, c.row, s);
}

template <int ES>
__device__ __forceinline__ float raw_elem(const uint4& r, int e) {
    const int w = ES == 2 ? (e >> 1) : e;
    const uint32_t v = w == 0 ? r.x : w == 1 ? r.y : w == 2 ? r.z : r.w;
    if (ES == 2) return __uint_as_float((e & 1) ? (v & 0xffff0000u) : (v << 16));
    return __uint_as_float(v);
}

// The allowed-mask words covering chunk elements [j0, j0 + E): word of max(j0, 0) and the next one.
struct MaskPair {
    uint32_t w0, w1;
    int base;  // word index of w0
};

__device__ __forceinline__ MaskPair mask_pair(const uint32_t* mrow, int nwords, int j0) {
    MaskPair p;
    p.base = max(j0, 0) >> 5;
    p.w0 = p.base < nwords ? mrow[p.base] : 0u;
    p.w1 = p.base + 1 < nwords ? mrow[p.base + 1] : 0u;
    return p;
}

__device__ __forceinline__ bool mask_bit(const MaskPair& p, int j) {
    const uint32_t w = (j >> 5) == p.base ? p.w0 : p.w1;
    return ((w >> (j & 31)) & 1u) != 0u;
}

// ---------------------------------------------------------------- slice phase: the slice in registers

// A slice's processed values in registers: thread t holds chunks t + kBlock * i (16 bytes each) in slots
// [E * i, E * i + E).  Elements outside the slice (the aligned chunks' overhang) hold -inf.
struct Tile {
    float v[kNV];
};

// Raw 16-byte chunks of a slice, loaded into registers before the prologue so the loads overlap it.
template <int ES>
struct RawTile {
    uint4 r[kNV / (16 / ES)];
};

template <int ES>
__device__ __forceinline__ void issue_tile(const Geo& g, RawTile<ES>& R) {
    constexpr int NCH = kNV / (16 / ES);
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        const int ch = threadIdx.x + kBlock * i;
        R.r[i] = ch < g.nchunk ? *(const uint4*)(g.base + (uintptr_t)ch * 16) : make_uint4(0u, 0u, 0u, 0u);
    }
}

// The slice's allowed bits into sm.mask: an element is allowed when it lies in [lo, hi), the row's bitmask (if
// any) allows it, and (omni order) it is not the censored EOS.  With the row's counts (sm.u.cnt, slot j - first)
// and penalty table when its penalties apply.  Ends with a barrier; returns nonzero when the table holds an
// alpha outside the corrected-reciprocal range.
// The slice's other inputs, loaded right after its tile (before the row's parameters are known): the allowed
// bits of the words covering it, limited to [lo, hi), and the first kBlock * 4 int4 of the row's history.
struct Preload {
    uint32_t mw[2];    // the slice's range bits of the two words
    uint32_t mraw[2];  // the row's mask words as loaded (used when the row has a mask)
    int4 h[4];
    bool hvec, masked;
};

__device__ __forceinline__ void preload(const DevGroup& G, int row, const Geo& g, Preload& P, bool history = true) {
    const uint32_t* mrow = gp(G.allowed) ? gp(G.allowed) + (int64_t)row * G.allowed_stride : nullptr;
    P.masked = mrow != nullptr;
    const int wb = g.first >> 5;  // arithmetic shift: first may be negative in slice 0
    const int wmax = (G.vocab - 1) >> 5;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int gw = wb + (int)threadIdx.x + u * kBlock;
        const int a = g.lo - 32 * gw, b = g.hi - 32 * gw;
        P.mw[u] = (a <= 0 ? ~0u : a >= 32 ? 0u : ~0u << a) & (b >= 32 ? ~0u : b <= 0 ? 0u : (1u << b) - 1u);
        // a clamped word (words outside [lo, hi) are masked off by mw), loaded with no branch around it (a row
        // without a mask reads the tile's first word instead) and combined only where it is used: a load under a
        // branch, or used at once, would be waited for together with the tile's loads before it
        P.mraw[u] = *(mrow != nullptr ? mrow + min(max(gw, 0), wmax) : (const uint32_t*)g.base);
    }
    const char* hrow = gp(G.history) != nullptr && G.hist_len > 0 ? hist_row(G, row) : nullptr;
    P.hvec = history && hrow != nullptr && hist_vec(G, hrow);
    if (P.hvec) {
        const int4* h4 = (const int4*)hrow;
        const int nv = G.hist_len >> 2;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = u * kBlock + threadIdx.x;
            P.h[u] = i < nv ? h4[i] : make_int4(-1, -1, -1, -1);
        }
    }
}

__device__ __forceinline__ int slice_prologue(const DevGroup& G, const Ctx& c, const Geo& g, int E, const Preload& P,
                                              Smem& sm) {
    const int wb = g.first >> 5;
    const int eos = (!c.hf && c.censor) ? G.eos : -1;
    uint32_t mw[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int gw = wb + (int)threadIdx.x + u * kBlock;
        mw[u] = P.masked ? P.mw[u] & P.mraw[u] : P.mw[u];
        if (eos >= 0 && (eos >> 5) == gw) mw[u] &= ~(1u << (eos & 31));
    }
    int pen_bad = 0;
    if (c.counts)  // ends with a barrier
        pen_bad = build_counts(G, c, g.first, g.lo, g.hi, g.nchunk * E / 2, sm, P.hvec ? P.h : nullptr);
    else
        __syncthreads();  // the previous use of sm.mask is over
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int i = threadIdx.x + u * kBlock;
        if (i < kMaskWords) sm.mask[i] = mw[u];
    }
    __syncthreads();
    return pen_bad;
}

// Division by the temperature: the corrected reciprocal (divisors in [2^-16, 2^16], powers of two included: there
// the product is exact and the correction zero), or IEEE division.
enum DivMode { kDivIeee = 0, kDivFast = 1 };

// One element of the row's pipeline with IEEE division, for the chunks the fast form does not cover.
template <bool HF, bool COUNTS>
__device__ __forceinline__ float elem_ieee(float x, int n, const DevGroup& G, const Ctx& c, const Smem& sm) {
    if (HF) x = x / c.tdiv;
    if (COUNTS) x = pen_exact(x, n < kAlphaTable ? sm.pen[n] : pen_entry(G, c, n));
    if (!HF) x = x / c.tdiv;
    return x;
}

// The row's pipeline on one tile.  HF: temperature, then penalties (engine/talker_sampler.py:149-154);
// otherwise penalties, then temperature (:145-146).  Masked, censored and out-of-slice elements become -inf
// at the end (-inf is absorbing under both orders).  Per chunk: one LDS read of its allowed bits, one of its
// counts; a chunk holding a count >= kAlphaTable or a division operand outside div_rn's range is recomputed
// with IEEE division.
template <int ES, bool HF, bool COUNTS, int DIV>
__device__ __forceinline__ void process_tile_t(const DevGroup& G, const Ctx& c, const Geo& g, const RawTile<ES>& R,
                                               Tile& T, const Smem& sm) {
    constexpr int E = 16 / ES;
    constexpr int NCH = kNV / E;
    const float d = c.tdiv, rd = c.rtdiv;
    const int wb = g.first >> 5;
    const int tid = fresh_tid();
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        const int ch = tid + kBlock * i;
        const int j0 = g.first + ch * E;
        const bool live = ch < g.nchunk;
        const int k = min((j0 >> 5) - wb, kMaskWords - 2);
        const uint32_t bits = live ? __builtin_amdgcn_alignbit(sm.mask[k + 1], sm.mask[k], (uint32_t)(j0 & 31)) : 0u;
        uint32_t cw[E / 2];
        bool slow = false;
        if (COUNTS) {
            if (ES == 2) {
                const uint4 v = *(const uint4*)&sm.u.cnt[ch * 4];
                cw[0] = v.x;
                cw[1] = v.y;
                cw[2] = v.z;
                cw[3] = v.w;
            } else {
                const uint2 v = *(const uint2*)&sm.u.cnt[ch * 2];
                cw[0] = v.x;
                cw[1] = v.y;
            }
            uint32_t any = 0u;
#pragma unroll
            for (int w = 0; w < E / 2; ++w) {
                cw[w] = live ? cw[w] : 0u;
                any |= cw[w];
            }
            slow = (any & 0xffc0ffc0u) != 0u;  // some count >= 64
        }
        float f[E];
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const float x = raw_elem<ES>(R.r[i], e);
            const int n = COUNTS ? (int)((cw[e >> 1] >> (16 * (e & 1))) & 63u) : 0;
            if (DIV == kDivIeee) {
                f[e] = elem_ieee<HF, COUNTS>(x, n, G, c, sm);
                continue;
            }
            float y = x;
            slow |= !raw_in_range(x);  // one check covers every division below
            if (HF) y = div_rn(y, d, rd);
            if (COUNTS) {
                const PenEntry pe = sm.pen[n];
                const float q = div_rn(y, pe.a, pe.ra);
                y = y < 0.f ? y * pe.a : q;
                y = (y - pe.fn) - pe.pn;
            }
            if (!HF) y = div_rn(y, d, rd);
            f[e] = y;
        }
        {
            if (slow) {
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    const int n = COUNTS ? (int)((cw[e >> 1] >> (16 * (e & 1))) & 0xffffu) : 0;
                    f[e] = elem_ieee<HF, COUNTS>(raw_elem<ES>(R.r[i], e), n, G, c, sm);
                }
            }
        }
#pragma unroll
        for (int e = 0; e < E; ++e) T.v[i * E + e] = ((bits >> e) & 1u) ? f[e] : -INFINITY;
    }
}

template <int ES, bool HF, bool COUNTS>
__device__ __forceinline__ void process_tile_d(const DevGroup& G, const Ctx& c, const Geo& g, const RawTile<ES>& R,
                                               Tile& T, const Smem& sm, int mode) {
    if (mode == kDivFast)
        process_tile_t<ES, HF, COUNTS, kDivFast>(G, c, g, R, T, sm);
    else
        process_tile_t<ES, HF, COUNTS, kDivIeee>(G, c, g, R, T, sm);
}

// The prologue and the element pipeline over a tile whose loads are in flight.
template <int ES>
__device__ __forceinline__ void finish_tile(const DevGroup& G, const Ctx& c, const Geo& g, const RawTile<ES>& R,
                                            const Preload& P, Tile& T, Smem& sm) {
    constexpr int E = 16 / ES;
    const int pen_bad = slice_prologue(G, c, g, E, P, sm);
    int mode = divisor_in_range(c.tdiv) ? kDivFast : kDivIeee;
    if (c.counts && pen_bad) mode = kDivIeee;
    if (c.hf) {
        if (c.counts)
            process_tile_d<ES, true, true>(G, c, g, R, T, sm, mode);
        else
            process_tile_d<ES, true, false>(G, c, g, R, T, sm, mode);
    } else {
        if (c.counts)
            process_tile_d<ES, false, true>(G, c, g, R, T, sm, mode);
        else
            process_tile_d<ES, false, false>(G, c, g, R, T, sm, mode);
    }
}

template <int ES>
__device__ __forceinline__ int tile_index(const Geo& g, int q) {
    constexpr int E = 16 / ES;
    return g.first + (int)(threadIdx.x + kBlock * (q / E)) * E + (q % E);
}

// Sub-block of element j of slice s: (round, wave) of the slice's chunk layout; a sub-block is 64 consecutive
// chunks, i.e. a contiguous vocabulary range.
template <int ES>
__device__ __forceinline__ int sub_block_of(const Geo& g, int j) {
    constexpr int E = 16 / ES;
    const int ch = (j - g.first) / E;
    return (ch / kBlock) * kWaves + (ch % kBlock) / 64;
}

// Per-(round, wave) sums of exp(v - ref) over the tile's finite values with v >= floor_v; lane 0 of each wave
// stores them to sm.sbw.  Returns the thread's total.
template <int ES>
__device__ __forceinline__ double tile_sub_sums(const Tile& T, float ref, float floor_v, Smem& sm) {
    constexpr int E = 16 / ES;
    constexpr int NCH = kNV / E;
    double tot = 0.0;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        double part = 0.0;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int q = i * E + e;
            const float f = T.v[q];
            if (f >= floor_v && finite_f(f)) part += (double)expf(f - ref);
        }
        tot += part;
        const double w = wave_sum_d(part);
        if (lane_id() == 0) sm.sbw[i * kWaves + wave_id()] = w;
    }
    return tot;
}

// Publishes the tile's values with lo_v <= v < hi_v (finite) in vocabulary order into cands (at most kCapSlice),
// staged in LDS and written out by wave 0 (so that wave's device-scope release covers them).  Returns the number
// found (may exceed kCapSlice).
template <int ES>
__device__ __forceinline__ int publish_range(const Tile& T, const Geo& geo, float lo_v, float hi_v, Cand* cands,
                                             Smem& sm) {
    constexpr int E = 16 / ES;
    constexpr int NCH = kNV / E;
    static_assert(NCH <= 10, "packed scan holds 5 rounds per word");
    // counts per round, packed 12 bits per round, 5 rounds per 64-bit word: one scan per word
    unsigned long long pk0 = 0ull, pk1 = 0ull;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        unsigned long long mine = 0;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int q = i * E + e;
            const float f = T.v[q];
            if (finite_f(f) && f >= lo_v && f < hi_v) ++mine;
        }
        if (i < 5)
            pk0 |= mine << (12 * i);
        else
            pk1 |= mine << (12 * (i - 5));
    }
    unsigned long long tot0, tot1 = 0ull;
    const unsigned long long ex0 = block_excl_scan_u(pk0, tot0, sm);
    unsigned long long ex1 = 0ull;
    if (NCH > 5) ex1 = block_excl_scan_u(pk1, tot1, sm);
    int run = 0;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        const unsigned long long ex = i < 5 ? ex0 : ex1;
        const unsigned long long tt = i < 5 ? tot0 : tot1;
        const int sh = 12 * (i < 5 ? i : i - 5);
        int pos = run + (int)((ex >> sh) & 0xfffull);
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int q = i * E + e;
            const float f = T.v[q];
            if (finite_f(f) && f >= lo_v && f < hi_v) {
                if (pos < kCapSlice) sm.stage[pos] = Cand{f, tile_index<ES>(geo, q)};
                ++pos;
            }
        }
        run += (int)((tt >> sh) & 0xfffull);
    }
    __syncthreads();
    if (threadIdx.x < 64)
        for (int p = threadIdx.x; p < min(run, kCapSlice); p += 64) pub_st_cand(&cands[p], sm.stage[p]);
    return run;
}

// ---------------------------------------------------------------- streaming (slow path and rescans)

// Streams slice s: fn(f, j) for every element.  Every thread runs the same number of iterations.
template <int ES, class F>
__device__ __forceinline__ void stream_slice(const DevGroup& G, const Ctx& c, int s, Smem& sm, F&& fn) {
    constexpr int E = 16 / ES;
    const Geo g = slice_geo<ES>(G, c, s);
    if (c.counts) build_counts(G, c, g.first, g.lo, g.hi, (g.hi - g.first + 1) >> 1, sm);
    const uint32_t* mrow = gp(G.allowed) ? gp(G.allowed) + (int64_t)c.row * G.allowed_stride : nullptr;
    const int nwords = (c.V + 31) >> 5;
    for (int ch = threadIdx.x; ch < g.nchunk; ch += kBlock) {
        const uint4 raw = *(const uint4*)(g.base + (uintptr_t)ch * 16);
        const MaskPair mk = mrow ? mask_pair(mrow, nwords, g.first + ch * E) : MaskPair{~0u, ~0u, 0};
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int j = g.first + ch * E + e;
            if (j >= g.lo && j < g.hi) {
                const int n = c.counts ? count_of(sm, j - g.first) : 0;
                fn(transform(raw_elem<ES>(raw, e), j, n, mrow ? mask_bit(mk, j) : true, G, c, sm), j);
            }
        }
    }
}

template <int ES, class F>
__device__ __forceinline__ void visit_row(const DevGroup& G, const Ctx& c, Smem& sm, F&& fn) {
    for (int s = 0; s < c.S; ++s) stream_slice<ES>(G, c, s, sm, fn);
}

// Wave 0 scans 256 count bins from the top for the bin holding the rem-th largest element.
__device__ __forceinline__ void pick_count_bin(int rem, Smem& sm) {
    if (threadIdx.x < 64) {
        const int l = threadIdx.x;
        uint32_t h[4];
        int sum = 0;
        for (int r = 0; r < 4; ++r) {
            h[r] = sm.hcnt[255 - (4 * l + r)];
            sum += (int)h[r];
        }
        const int incl = wave_incl_scan(sum);
        int before = incl - sum;
        for (int r = 0; r < 4; ++r) {
            if (before < rem && rem <= before + (int)h[r]) {
                sm.sel_bin = 255 - (4 * l + r);
                sm.sel_rem = rem - before;
            }
            before += (int)h[r];
        }
    }
}

// k-th largest finite value of the row (streamed); -inf when it holds fewer than k finite values.
template <int ES>
__device__ __forceinline__ float stream_kth(const DevGroup& G, const Ctx& c, Smem& sm, int k) {
    uint32_t prefix = 0u, pmask = 0u;
    int rem = k;
    for (int shift = 24; shift >= 0; shift -= 8) {
        __syncthreads();
        for (int b = threadIdx.x; b < 256; b += kBlock) sm.hcnt[b] = 0u;
        if (threadIdx.x == 0) sm.sel_bin = -1;
        __syncthreads();
        visit_row<ES>(G, c, sm, [&](float f, int) {
            if (finite_f(f)) {
                const uint32_t key = ord_key(f);
                if ((key & pmask) == prefix) atomicAdd(&sm.hcnt[(key >> shift) & 255u], 1u);
            }
        });
        __syncthreads();
        pick_count_bin(rem, sm);
        __syncthreads();
        const int bin = sm.sel_bin;
        if (bin < 0) return -INFINITY;
        rem = sm.sel_rem;
        prefix |= (uint32_t)bin << shift;
        pmask |= 255u << shift;
    }
    return key_float(prefix);
}

__device__ __forceinline__ unsigned long long mass_q(float f, float m) {
    return (unsigned long long)((double)expf(f - m) * kMassScale);
}

// Smallest value v >= lower of the row with sum{ q(x) : x > v, x >= lower } < target (q = fixed-point
// exp(x - m)); +inf when none qualifies.
template <int ES>
__device__ __forceinline__ float stream_mass(const DevGroup& G, const Ctx& c, Smem& sm, float lower, float m,
                                             double target) {
    const uint32_t lkey = ord_key(lower);
    uint32_t prefix = 0u, pmask = 0u;
    unsigned long long acc = 0ull;
    for (int shift = 24; shift >= 0; shift -= 8) {
        __syncthreads();
        for (int b = threadIdx.x; b < 256; b += kBlock) {
            sm.hcnt[b] = 0u;
            sm.hmass[b] = 0ull;
        }
        __syncthreads();
        visit_row<ES>(G, c, sm, [&](float f, int) {
            if (finite_f(f)) {
                const uint32_t key = ord_key(f);
                if (key >= lkey && (key & pmask) == prefix) {
                    const uint32_t b = (key >> shift) & 255u;
                    atomicAdd(&sm.hcnt[b], 1u);
                    atomicAdd(&sm.hmass[b], mass_q(f, m));
                }
            }
        });
        __syncthreads();
        if (threadIdx.x < 64) {
            const int l = threadIdx.x;
            unsigned long long hm[4];
            uint32_t hc[4];
            unsigned long long sum = 0ull;
            for (int r = 0; r < 4; ++r) {
                hm[r] = sm.hmass[255 - (4 * l + r)];
                hc[r] = sm.hcnt[255 - (4 * l + r)];
                sum += hm[r];
            }
            const unsigned long long incl = wave_incl_scan(sum);
            unsigned long long before = acc + (incl - sum);
            int mine = -1;
            unsigned long long mine_before = 0ull;
            for (int r = 0; r < 4; ++r) {  // descending bins: the last qualifying one is the lowest
                if (hc[r] > 0u && (double)before < target) {
                    mine = 255 - (4 * l + r);
                    mine_before = before;
                }
                before += hm[r];
            }
            int lowest = mine < 0 ? 1 << 20 : mine;
            lowest = wave_reduce(lowest, [](int a, int b) { return min(a, b); });
            if (mine >= 0 && mine == lowest) {
                sm.sel_bin = mine;
                sm.sel_acc = mine_before;
            }
            if (l == 0 && lowest == (1 << 20)) sm.sel_bin = -1;
        }
        __syncthreads();
        const int bin = sm.sel_bin;
        if (bin < 0) return INFINITY;
        acc = sm.sel_acc;
        prefix |= (uint32_t)bin << shift;
        pmask |= 255u << shift;
    }
    return key_float(prefix);
}

// The draw of engine/talker_sampler.py:168-172 over survivors (finite values >= thr, minus the EOS id when
// drop_eos), streaming the row: p = exp(x - m) * (1 / sum); the first survivor whose running sum, rounded to
// float, exceeds u * total; V - 1 when none does.
template <int ES>
__device__ __forceinline__ int stream_draw(const DevGroup& G, const Ctx& c, Smem& sm, float thr, float m,
                                           bool drop_eos, float u) {
    auto survives = [&](float f, int j) { return finite_f(f) && f >= thr && !(drop_eos && j == G.eos); };
    double zpart = 0.0;
    visit_row<ES>(G, c, sm, [&](float f, int j) {
        if (survives(f, j)) zpart += (double)expf(f - m);
    });
    const float inv = 1.0f / (float)block_sum_d(zpart, sm);
    double total = 0.0;
    for (int s = 0; s < c.S; ++s) {
        double part = 0.0;
        stream_slice<ES>(G, c, s, sm, [&](float f, int j) {
            if (survives(f, j)) part += (double)(expf(f - m) * inv);
        });
        const double ts = block_sum_d(part, sm);
        if (threadIdx.x == 0) sm.tile_sum[s] = ts;
        total += ts;
    }
    __syncthreads();
    const float target = u * (float)total;
    double base = 0.0;
    for (int s = 0; s < c.S; ++s) {
        const double ts = sm.tile_sum[s];
        if (!((float)(base + ts) > target)) {
            base += ts;
            continue;
        }
        constexpr int E = 16 / ES;
        const Geo g = slice_geo<ES>(G, c, s);
        if (c.counts) build_counts(G, c, g.first, g.lo, g.hi, (g.hi - g.first + 1) >> 1, sm);
        const uint32_t* mrow = gp(G.allowed) ? gp(G.allowed) + (int64_t)c.row * G.allowed_stride : nullptr;
        const int nwords = (c.V + 31) >> 5;
        int found = INT_MAX;
        double run_base = base;
        for (int r0 = 0; r0 < g.nchunk; r0 += kBlock) {
            const int ch = r0 + threadIdx.x;
            float pv[E];
            int jv[E];
            double mine = 0.0;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                pv[e] = 0.0f;
                jv[e] = 0;
            }
            if (ch < g.nchunk) {
                const uint4 raw = *(const uint4*)(g.base + (uintptr_t)ch * 16);
                const MaskPair mk = mrow ? mask_pair(mrow, nwords, g.first + ch * E) : MaskPair{~0u, ~0u, 0};
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    const int j = g.first + ch * E + e;
                    jv[e] = j;
                    if (j >= g.lo && j < g.hi) {
                        const int n = c.counts ? count_of(sm, j - g.first) : 0;
                        const float f = transform(raw_elem<ES>(raw, e), j, n, mrow ? mask_bit(mk, j) : true, G, c, sm);
                        if (survives(f, j)) pv[e] = expf(f - m) * inv;
                    }
                    mine += (double)pv[e];
                }
            }
            double tot;
            double run = run_base + block_excl_scan_d(mine, tot, sm);
#pragma unroll
            for (int e = 0; e < E; ++e) {
                if (pv[e] > 0.0f) {
                    run += (double)pv[e];
                    if ((float)run > target && found == INT_MAX) found = jv[e];
                }
            }
            run_base += tot;
            if (block_min_i(found, sm) != INT_MAX) break;
        }
        const int tok = block_min_i(found, sm);
        if (tok != INT_MAX) return tok;
        base += ts;
    }
    return c.V - 1;
}

// ---------------------------------------------------------------- rng

__device__ __forceinline__ uint32_t lowbias32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

// engine/talker_sampler.py:70-76
__device__ __forceinline__ float counter_uniform(int64_t seed, int64_t step) {
    const uint64_t s = (uint64_t)seed, t = (uint64_t)step;
    uint32_t h = lowbias32((uint32_t)s);
    h = lowbias32(h ^ (uint32_t)(s >> 32) ^ 0x9E3779B9u);
    h = lowbias32(h ^ (uint32_t)t ^ 0x632BE5ABu);
    return (float)(h >> 8) * (1.0f / 16777216.0f);
}

// Philox4x32-10 (Salmon et al., SC'11): key = seed, counter = (step, row id); word 0 -> U[0,1).
__device__ __forceinline__ float philox_uniform(int64_t seed, int64_t step, int64_t rid) {
    const uint64_t s = (uint64_t)seed, t = (uint64_t)step, r = (uint64_t)rid;
    uint32_t c0 = (uint32_t)t, c1 = (uint32_t)(t >> 32), c2 = (uint32_t)r, c3 = (uint32_t)(r >> 32);
    uint32_t k0 = (uint32_t)s, k1 = (uint32_t)(s >> 32);
#pragma unroll
    for (int rnd = 0; rnd < 10; ++rnd) {
        if (rnd) {
            k0 += 0x9E3779B9u;
            k1 += 0xBB67AE85u;
        }
        const uint32_t lo0 = 0xD2511F53u * c0, hi0 = __umulhi(0xD2511F53u, c0);
        const uint32_t lo1 = 0xCD9E8D57u * c2, hi1 = __umulhi(0xCD9E8D57u, c2);
        const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
        c0 = n0;
        c1 = lo1;
        c2 = n2;
        c3 = lo0;
    }
    return (float)(c0 >> 8) * (1.0f / 16777216.0f);
}

__device__ __forceinline__ float row_uniform(const DevGroup& G, const Ctx& c) {
    if (gp(G.uniforms)) return gp(G.uniforms)[c.row];
    const int64_t seed = gp(G.seeds) ? gp(G.seeds)[c.row] : 0;
    if (G.rng == MIS_RNG_PHILOX) return philox_uniform(seed, c.step, gp(G.row_ids) ? gp(G.row_ids)[c.row] : 0);
    return counter_uniform(seed, c.step);
}

// ---------------------------------------------------------------- outputs and state

// Processed logits (-inf where filtered) and softmax probabilities of the whole row (parity outputs).
template <int ES>
__device__ __forceinline__ void write_outputs(const DevGroup& G, const Ctx& c, Smem& sm, float thr, float m,
                                              bool drop_eos) {
    float* prow = gp(G.processed) ? gp(G.processed) + (int64_t)c.row * G.processed_stride : nullptr;
    float* qrow = gp(G.probs) ? gp(G.probs) + (int64_t)c.row * G.probs_stride : nullptr;
    if (c.forced) {
        for (int j = threadIdx.x; j < c.V; j += kBlock) {
            const bool e = j == G.eos;
            if (prow) prow[j] = e ? 0.0f : -INFINITY;
            if (qrow) qrow[j] = e ? 1.0f : 0.0f;
        }
        return;
    }
    auto keep = [&](float f, int j) { return f >= thr && !(drop_eos && j == G.eos); };
    double zpart = 0.0;
    if (qrow)
        visit_row<ES>(G, c, sm, [&](float f, int j) {
            if (finite_f(f) && keep(f, j)) zpart += (double)expf(f - m);
        });
    const float inv = 1.0f / (float)block_sum_d(zpart, sm);
    visit_row<ES>(G, c, sm, [&](float f, int j) {
        const bool k = keep(f, j);
        if (prow) prow[j] = k ? f : -INFINITY;
        if (qrow) qrow[j] = !(m > -INFINITY) ? NAN : (k && finite_f(f)) ? expf(f - m) * inv : 0.0f;
    });
}

// tokens[row]; for live rows with MIS_UPDATE_STATE: history append, steps + 1, finished |= (token == eos).
__device__ __forceinline__ void update_state(const DevGroup& G, const Ctx& c, int64_t tok) {
    if (!(G.flags & MIS_UPDATE_STATE) || !c.live) {
        if (threadIdx.x == 0 && gp(G.tokens)) gp(G.tokens)[c.row] = c.live ? tok : kPad;
        return;
    }
    if (gp(G.history) && G.hist_len > 0) {
        const int W = G.hist_len;
        char* hrow = (char*)gp(G.history) + (int64_t)c.row * G.hist_stride * (G.hist_i64 ? 8 : 4);
        if (G.hist_mode == MIS_HISTORY_RING) {
            if (threadIdx.x == 0) {
                const int pos = (int)((gp(G.hist_head)[c.row] % W + W) % W);
                if (G.hist_i64)
                    ((int64_t*)hrow)[pos] = tok;
                else
                    ((int32_t*)hrow)[pos] = (int32_t)tok;
                gp(G.hist_head)[c.row] = (pos + 1) % W;
            }
        } else {
            // shift left by one, append: each round reads [b+1, b+kBlock] before writing [b, b+kBlock)
            for (int b = 0; b < W; b += kBlock) {
                const int j = b + threadIdx.x;
                int64_t nxt = 0;
                if (j < W) {
                    if (j + 1 < W)
                        nxt = G.hist_i64 ? ((const int64_t*)hrow)[j + 1] : (int64_t)((const int32_t*)hrow)[j + 1];
                    else
                        nxt = tok;
                }
                __syncthreads();
                if (j < W) {
                    if (G.hist_i64)
                        ((int64_t*)hrow)[j] = nxt;
                    else
                        ((int32_t*)hrow)[j] = (int32_t)nxt;
                }
                __syncthreads();
            }
        }
    }
    if (threadIdx.x == 0) {
        if (gp(G.tokens)) gp(G.tokens)[c.row] = tok;
        if (gp(G.steps)) gp(G.steps)[c.row] = c.step + 1;
        if (gp(G.finished) && tok == (int64_t)G.eos) gp(G.finished)[c.row] = 1;
    }
}


// Appends key to sm.u.c.key at sm.sel_rem where pred holds (any order): one LDS atomic per wave, positions
// within the wave from the ballot.
__device__ __forceinline__ void append_key(bool pred, uint32_t key, Smem& sm) {
    const unsigned long long b = __ballot(pred);
    if (b == 0ull) return;
    const int leader = __ffsll((long long)b) - 1;
    int base = 0;
    if (lane_id() == leader) base = atomicAdd(&sm.sel_rem, __popcll(b));
    base = __builtin_amdgcn_readlane(base, leader);
    const int below = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
    if (pred) sm.u.c.key[base + below] = key;
}

// ---------------------------------------------------------------- cross-workgroup protocol

__device__ __forceinline__ unsigned xcc_id() {
    unsigned x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    return x & 7u;
}

// Every publication store of a slice is issued by wave 0 (threads 0..63).  Thread 0 waits until they have all
// completed, then counts the slice in with a device-scope atomic on the row's 64-bit arrival word, which holds
// one 7-bit count per XCD.  The slice that completes the count (S arrivals) is the row's last and finalises it.
// It also learns whether every slice ran on its own XCD: if one did not, the slices' publications may sit in
// another XCD's L2, and the finaliser must not read them (sm.foreign).  Returns true in the row's last workgroup
// (every thread).
__device__ __forceinline__ bool arrive_last(unsigned int* counter, int S, Smem& sm) {
    __syncthreads();
    if (threadIdx.x == 0) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        unsigned long long* word = (unsigned long long*)counter;
        const unsigned x = xcc_id();
        const unsigned long long old =
            __hip_atomic_fetch_add(word, 1ull << (7 * x), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        int total = 1;
        for (int f = 0; f < 8; ++f) total += (int)((old >> (7 * f)) & 127ull);
        const int last = total == S;
        if (last) __hip_atomic_store(word, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // for the next launch
        sm.is_last = last;
        sm.foreign = (old & ~(127ull << (7 * x))) != 0ull;
    }
    __syncthreads();
    return sm.is_last != 0;
}

// Held slices.  The slices of a top-p row without top-k (and S > 1) that are not last to arrive wait for the
// finaliser's decision word, kept next to the arrival word.  The finaliser is the row's last arrival, so it is
// running by the time anyone waits, and it sets the word on every path; the wait is bounded all the same.
__device__ __forceinline__ bool holds_slices(const Ctx& c) { return c.nucleus && c.S > 1; }

__device__ __forceinline__ unsigned int* row_counter(const DevGroup& G, const Ctx& c) {
    return gp(G.counters) + (int64_t)c.grow * kCounterStride;
}

// The finaliser's side (thread 0; the first call wins).  Stores issued before it (the pending record, the
// arrival word's reset) complete before the decision is visible.
__device__ __forceinline__ void release_held(const DevGroup& G, const Ctx& c, Smem& sm, uint32_t d) {
    if (!holds_slices(c) || threadIdx.x != 0 || sm.decision != 0u) return;
    sm.decision = d;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __hip_atomic_store(row_counter(G, c) + kDecisionWord, d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A held slice's side: the decision (0 if the bound ran out, which leaves the slice without a part to play).
__device__ __forceinline__ uint32_t await_decision(const DevGroup& G, const Ctx& c, Smem& sm) {
    if (threadIdx.x == 0) {
        unsigned int* word = row_counter(G, c) + kDecisionWord;
        uint32_t d = 0u;
        for (int i = 0; i < kSpinLimit; ++i) {
            d = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (d != 0u) break;
            __builtin_amdgcn_s_sleep(1);
        }
        sm.decision = d;
    }
    __syncthreads();
    return sm.decision;
}

// A held slice that is not needed counts itself out on the arrival word (which the finaliser reset); the last of
// the S - 1 clears the arrival and decision words for the next launch.
__device__ __forceinline__ void depart(const DevGroup& G, const Ctx& c) {
    if (threadIdx.x != 0) return;
    unsigned long long* word = (unsigned long long*)row_counter(G, c);
    const unsigned long long old =
        __hip_atomic_fetch_add(word, 1ull << (7 * xcc_id()), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int total = 1;
    for (int f = 0; f < 8; ++f) total += (int)((old >> (7 * f)) & 127ull);
    if (total == c.S - 1) {
        __hip_atomic_store(word, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(row_counter(G, c) + kDecisionWord, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// ---------------------------------------------------------------- finaliser pieces

// One compare-exchange step (block size K, partner distance J) of a descending bitonic sort over R keys per lane,
// element i = R * gl + r (gl: the lane's index among the sorting lanes).  Partners within a lane are in registers,
// within a wave across lanes, across waves through LDS.
template <int R, int K, int J>
__device__ __forceinline__ void bitonic_step(uint32_t (&a)[R], int gl, Smem& sm) {
    if constexpr (J < R) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (r & J) continue;
            bool desc;
            if constexpr (K >= R)
                desc = ((R * gl) & K) == 0;
            else
                desc = (r & K) == 0;
            const uint32_t lo = min(a[r], a[r | J]), hi = max(a[r], a[r | J]);
            a[r] = desc ? hi : lo;
            a[r | J] = desc ? lo : hi;
        }
    } else {
        constexpr int D = J / R;  // lane distance
        const bool keep_max = (((R * gl) & J) == 0) == (((R * gl) & K) == 0);  // lower of the pair in a desc block
        if constexpr (D < 64) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t b = xor_lane<D>(a[r]);
                a[r] = keep_max ? max(a[r], b) : min(a[r], b);
            }
        } else {
            __syncthreads();  // every wave sorts when partners cross waves
#pragma unroll
            for (int r = 0; r < R; ++r) sm.u.c.key[R * gl + r] = a[r];
            __syncthreads();
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t b = sm.u.c.key[(R * gl + r) ^ J];
                a[r] = keep_max ? max(a[r], b) : min(a[r], b);
            }
        }
    }
}

template <int R, int K, int J>
__device__ __forceinline__ void bitonic_merge(uint32_t (&a)[R], int gl, Smem& sm) {
    bitonic_step<R, K, J>(a, gl, sm);
    if constexpr (J > 1) bitonic_merge<R, K, J / 2>(a, gl, sm);
}

template <int N, int R, int K>
__device__ __forceinline__ void bitonic_stages(uint32_t (&a)[R], int gl, Smem& sm) {
    bitonic_merge<R, K, K / 2>(a, gl, sm);
    if constexpr (K < N) bitonic_stages<N, R, K * 2>(a, gl, sm);
}

// N keys (a power of two, 64..kCapRow) sorted descending in place: wave 0 alone up to 128 keys (no barrier),
// every wave beyond.  Fully unrolled.
template <int N>
__device__ __forceinline__ void sort_n(Smem& sm) {
    constexpr int NW = N <= 128 ? 1 : kWaves;
    constexpr int R = N / (64 * NW);
    static_assert(R >= 1 && R <= 8 && R * 64 * NW == N, "keys per lane");
    if (NW == kWaves || wave_id() == 0) {
        const int gl = fresh_tid();
        uint32_t a[R];
#pragma unroll
        for (int r = 0; r < R; ++r) a[r] = sm.u.c.key[R * gl + r];
        bitonic_stages<N, R, 2>(a, gl, sm);
        if constexpr (NW > 1) __syncthreads();  // the last cross-wave reads are done
#pragma unroll
        for (int r = 0; r < R; ++r) sm.u.c.key[R * gl + r] = a[r];
    }
    __syncthreads();
}

// Sorts sm.u.c.key[0, np) descending (np a power of two in [8, kCapRow]; the keys past the candidates are zero,
// below every real key).
__device__ __forceinline__ void sort_keys_desc(Smem& sm, int np) {
    if (np < 64) {
        for (int p = np + (int)threadIdx.x; p < 64; p += kBlock) sm.u.c.key[p] = 0u;
        __syncthreads();
    }
    switch (np) {
        case 8:
        case 16:
        case 32:
        case 64: sort_n<64>(sm); break;
        case 128: sort_n<128>(sm); break;
        case 256: sort_n<256>(sm); break;
        case 512: sort_n<512>(sm); break;
        case 1024: sort_n<1024>(sm); break;
        default: sort_n<2048>(sm); break;
    }
}

// The c-th largest (1 <= c <= 256) of the 256 per-thread values v: their order keys sorted by the bitonic network
// (all four waves, one key per lane), then read at rank c - 1.  Uses sm.u (the slice's count table is spent).
__device__ __forceinline__ float block_kth_of_256(float v, int c, Smem& sm) {
    __syncthreads();  // the union may still be in use
    sm.u.c.key[threadIdx.x] = ord_key(v);
    __syncthreads();
    sort_n<kBlock>(sm);  // ends with a barrier
    return key_float(sm.u.c.key[c - 1]);
}


// The top-k / top-p threshold from the sorted candidate keys (vocabulary counts n >= ...).  z_full is the
// full-row normaliser (hf order); omni normalises over the top k (engine/talker_sampler.py:112,129).
// kept_out: the ranks kept; ztop_out: the mass of the first min(k, n) ranks (top-p rows only).
__device__ __forceinline__ float sorted_threshold(const Ctx& c, Smem& sm, int n, float m, double z_full,
                                                  int* kept_out = nullptr, double* ztop_out = nullptr) {
    const int kk = min(c.k_eff, n);
    const float thr_k = c.k_eff <= n ? key_float(sm.u.c.key[c.k_eff - 1]) : -INFINITY;
    if (kept_out) *kept_out = min(c.k_eff, n);
    if (!c.p_active) return thr_k;
    // blocked layout: thread t owns sorted positions [t*per, (t+1)*per)
    const int per = (kk + kBlock - 1) / kBlock;
    double mine = 0.0;
    for (int r = threadIdx.x * per; r < min(kk, (int)(threadIdx.x + 1) * per); ++r)
        mine += (double)expf(key_float(sm.u.c.key[r]) - m);
    double ztop;
    double run = block_excl_scan_d(mine, ztop, sm);
    const double zp = (c.hf || c.nucleus) ? z_full : ztop;  // a row without top-k normalises over the full row
    const double target = (double)c.top_p * zp;
    int kp = 0;  // ranks whose exclusive mass is below top_p (a prefix)
    for (int r = threadIdx.x * per; r < min(kk, (int)(threadIdx.x + 1) * per); ++r) {
        if (run < target) ++kp;
        run += (double)expf(key_float(sm.u.c.key[r]) - m);
    }
    kp = block_sum_i(kp, sm);
    if (kp == kk && c.k_eff > n && zp < target) kp = c.k_eff;  // the top k's -inf ranks: exclusive mass = zp
    const int kept = min(max(kp, c.min_keep_eff), c.k_eff);
    if (kept_out) *kept_out = kept;
    if (ztop_out) *ztop_out = ztop;
    return kept <= n ? key_float(sm.u.c.key[kept - 1]) : -INFINITY;
}

// Inverse-CDF draw over the LDS candidates (vocabulary order), survivors >= thr: the first survivor whose
// inclusive running mass exceeds u times the survivors' total (engine/talker_sampler.py:168-173 searchsorted).
__device__ __forceinline__ int cand_draw(const DevGroup& G, const Ctx& c, Smem& sm, int n, float thr, float m,
                                         bool drop_eos, float u) {
    const int per = (n + kBlock - 1) / kBlock;
    const int lo = min(n, (int)threadIdx.x * per), hi = min(n, (int)(threadIdx.x + 1) * per);
    auto mass = [&](int p) {
        const float f = sm.u.c.val[p];
        return (f >= thr && !(drop_eos && sm.u.c.id[p] == G.eos)) ? (double)expf(f - m) : 0.0;
    };
    double mine = 0.0;
    for (int p = lo; p < hi; ++p) mine += mass(p);
    double total;
    double run = block_excl_scan_d(mine, total, sm);
    const double target = (double)u * total;
    int found = INT_MAX;
    for (int p = lo; p < hi; ++p) {
        const double e = mass(p);
        run += e;
        if (e > 0.0 && run > target) {
            found = sm.u.c.id[p];
            break;
        }
    }
    const int tok = block_min_i(found, sm);
    return tok == INT_MAX ? c.V - 1 : tok;
}

// Inverse-CDF draw from sub-block sums: sums[sbi] (already in units of exp(x - m), survivors only, flattened
// slice-major in vocabulary order) locate the sub-block holding u * total; that sub-block is rescanned element
// by element (survivors: finite values >= thr, minus EOS when drop_eos), from the published processed tiles when
// tile is given, else from the logits.
template <int ES>
__device__ __forceinline__ int sub_block_draw(const DevGroup& G, const Ctx& c, Smem& sm, int nsb_total, float thr,
                                              float m, bool drop_eos, float u, const float* tile = nullptr) {
    constexpr int E = 16 / ES;
    constexpr int NSB = kNV / E * kWaves;
    // wave 0 walks the sums (each lane a contiguous run of sub-blocks): no block-wide barrier until the result
    if (threadIdx.x < 64) {
        const int l = threadIdx.x;
        const int per = (nsb_total + 63) >> 6;
        const int lo = min(nsb_total, l * per), hi = min(nsb_total, lo + per);
        double zpart = 0.0;
        for (int i = lo; i < hi; ++i) zpart += sm.u.sbs[i];
        const double zs = wave_sum_d(zpart);
        const float inv = 1.0f / (float)zs;
        double mine = 0.0;
        for (int i = lo; i < hi; ++i) mine += sm.u.sbs[i] * (double)inv;
        const double incl = wave_incl_scan(mine);
        const double total = __longlong_as_double(
            (long long)(((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)((unsigned long long)__double_as_longlong(incl) >> 32), 63) << 32) |
                        (uint32_t)__builtin_amdgcn_readlane((int)__double_as_longlong(incl), 63)));
        double run = shfl_up_d(incl, 1);  // exclusive: the sub-blocks before this lane's run
        if (l == 0) run = 0.0;
        const float target = u * (float)total;
        int first = INT_MAX;
        for (int i = lo; i < hi; ++i) {
            const double nxt = run + sm.u.sbs[i] * (double)inv;
            if ((float)nxt > target) {
                first = i;
                break;
            }
            run = nxt;
        }
        const unsigned long long hit = __ballot(first != INT_MAX);
        if (l == 0) {
            sm.sel_rem = INT_MAX;
            sm.red_f[0] = inv;
            sm.red_f[1] = target;
        }
        if (hit != 0ull && l == __ffsll((long long)hit) - 1) {
            sm.sel_rem = first;
            sm.red_d[0] = run;
        }
    }
    __syncthreads();
    const float inv = sm.red_f[0], target = sm.red_f[1];
    const int first = sm.sel_rem;
    double before = first != INT_MAX ? sm.red_d[0] : 0.0;
    __syncthreads();  // (sel_rem and red_d are reused below)
    const uint32_t* mrow = gp(G.allowed) ? gp(G.allowed) + (int64_t)c.row * G.allowed_stride : nullptr;
    const int nwords = (c.V + 31) >> 5;
    int cur_slice = -1;
    for (int sbi = (first == INT_MAX ? nsb_total : first); sbi < nsb_total; ++sbi) {
        const int s = sbi / NSB, sb = sbi % NSB;
        const Geo g = slice_geo<ES>(G, c, s);
        if (tile == nullptr && c.counts && s != cur_slice)
            build_counts(G, c, g.first, g.lo, g.hi, (g.hi - g.first + 1) >> 1, sm);
        cur_slice = s;
        // 64 chunks: round sb / kWaves, wave sb % kWaves; wave 0 rescans them
        int found = INT_MAX;
        double sbsum = 0.0;
        if (threadIdx.x < 64) {
            const int ch = (sb / kWaves) * kBlock + (sb % kWaves) * 64 + (int)threadIdx.x;
            float pv[E];
            int jv[E];
            double mine2 = 0.0;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                pv[e] = 0.0f;
                jv[e] = 0;
            }
            if (tile != nullptr) {
                // slot (round, e) of thread (wave, lane): the tile's layout; out-of-slice slots hold -inf
                const float* tp = tile + ((int64_t)s * kNV + (sb / kWaves) * E) * kBlock + (sb % kWaves) * 64 +
                                  (int)threadIdx.x;
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    const int j = g.first + ch * E + e;
                    jv[e] = j;
                    const float f = pub_ld(&tp[e * kBlock]);
                    if (finite_f(f) && f >= thr && !(drop_eos && j == G.eos)) pv[e] = expf(f - m) * inv;
                    mine2 += (double)pv[e];
                }
            } else if (ch < g.nchunk) {
                const uint4 raw = *(const uint4*)(g.base + (uintptr_t)ch * 16);
                const MaskPair mk = mrow ? mask_pair(mrow, nwords, g.first + ch * E) : MaskPair{~0u, ~0u, 0};
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    const int j = g.first + ch * E + e;
                    jv[e] = j;
                    if (j >= g.lo && j < g.hi) {
                        const int n = c.counts ? count_of(sm, j - g.first) : 0;
                        const float f = transform(raw_elem<ES>(raw, e), j, n, mrow ? mask_bit(mk, j) : true, G, c, sm);
                        if (finite_f(f) && f >= thr && !(drop_eos && j == G.eos)) pv[e] = expf(f - m) * inv;
                    }
                    mine2 += (double)pv[e];
                }
            }
            // wave-level exclusive scan
            const double incl = wave_incl_scan(mine2);
            double ex = shfl_up_d(incl, 1);
            if (lane_id() == 0) ex = 0.0;
            double rr = before + ex;
#pragma unroll
            for (int e = 0; e < E; ++e)
                if (pv[e] > 0.0f) {
                    rr += (double)pv[e];
                    if ((float)rr > target && found == INT_MAX) found = jv[e];
                }
            sbsum = __longlong_as_double((long long)(((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)((unsigned long long)__double_as_longlong(incl) >> 32), 63) << 32) | (uint32_t)__builtin_amdgcn_readlane((int)__double_as_longlong(incl), 63)));
        }
        const int tok = block_min_i(found, sm);
        if (tok != INT_MAX) return tok;
        if (threadIdx.x == 0) sm.red_d[1] = sbsum;
        __syncthreads();
        before += sm.red_d[1];
    }
    return c.V - 1;
}

// ---------------------------------------------------------------- finaliser

template <int ES>
__device__ __forceinline__ void load_summaries(const Ctx& c, Smem& sm, const RowWs& w) {
    if ((int)threadIdx.x < c.S) sm.summ[threadIdx.x] = pub_ld_summary(&w.summ[threadIdx.x]);
    __syncthreads();
}

// The row's max, first argmax, normaliser, published-candidate count and gate from the slice summaries, one lane
// of wave 0 per slice; each slice's scale exp(m_s - m) stays in sm.tile_sum (0 for a slice with no finite value).
__device__ __forceinline__ void merge_summaries(const Ctx& c, Smem& sm, const RowWs& w) {
    if (threadIdx.x < 64) {
        const int l = threadIdx.x;
        const bool v = l < c.S;
        SliceSummary q;
        if (v) {
            q = pub_ld_summary(&w.summ[l]);
            sm.summ[l] = q;
        }
        const float qm = v ? q.m : -INFINITY;
        const float m = wave_reduce(qm, [](float a, float b) { return fmaxf(a, b); });
        const int am = wave_reduce(v && qm == m ? q.argmax : INT_MAX, [](int a, int b) { return min(a, b); });
        const bool fin = v && qm > -INFINITY;
        const double sc = fin ? exp((double)qm - (double)m) : 0.0;
        const double z = wave_sum_d(fin ? q.z * sc : 0.0);
        const double cmass = wave_sum_d(fin ? q.hi_mass * sc : 0.0);
        const float gmax = wave_reduce(v ? q.g : -INFINITY, [](float a, float b) { return fmaxf(a, b); });
        const int ntot = wave_reduce(v ? q.ncand : 0, [](int a, int b) { return a + b; });
        const int ovf = wave_reduce(v ? q.overflow : 0, [](int a, int b) { return a | b; });
        sm.tile_sum[l] = sc;
        if (l == 0) {
            sm.fin.z = z;
            sm.fin.cmass = cmass;
            sm.fin.m = m;
            sm.fin.gmax = gmax;
            sm.fin.am = am;
            sm.fin.ntot = ntot;
            sm.fin.overflow = ovf;
        }
    }
    __syncthreads();
}

// The slow, always-exact path: stream the row for every selection.
// The slices' published candidates into LDS in vocabulary order (slice s's at offset coff[s]) and the order keys
// of those >= gate, packed in no particular order (nkeys of them) and padded with zeros up to np, the returned
// power of two (>= 8).  ntot <= kCapRow.  The slice of each position comes from a map that every wave fills with
// plain stores, so the loads that follow are all issued before any is used.
__device__ __forceinline__ int gather_cands(const Ctx& c, Smem& sm, const RowWs& w, int ntot, float gate, int& nkeys) {
    if (threadIdx.x < 64) {
        const int l = threadIdx.x;
        const int x = l < c.S ? sm.summ[l].ncand : 0;
        const int incl = wave_incl_scan(x);
        sm.coff[l] = incl - x;
        if (l == 63) sm.coff[kMaxSlices] = incl;
        if (l == 0) sm.sel_rem = 0;  // key counter
    }
    __syncthreads();
    uint8_t* smap = (uint8_t*)sm.hmass;  // kCapRow bytes, idle while a finaliser runs
    for (int s = wave_id(); s < c.S; s += kWaves)
        for (int p = sm.coff[s] + lane_id(); p < sm.coff[s + 1]; p += 64) smap[p] = (uint8_t)s;
    __syncthreads();
    constexpr int U = kCapRow / kBlock;
    int sl[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int idx = threadIdx.x + u * kBlock;
        sl[u] = idx < ntot ? smap[idx] : 0;
    }
    Cand cd[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int idx = threadIdx.x + u * kBlock;
        cd[u] = Cand{-INFINITY, 0};
        if (idx < ntot) cd[u] = pub_ld_cand(&w.cand[(int64_t)sl[u] * kCapSlice + (idx - sm.coff[sl[u]])]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int idx = threadIdx.x + u * kBlock;
        if (idx < ntot) {
            sm.u.c.val[idx] = cd[u].f;
            sm.u.c.id[idx] = cd[u].j;
        }
        append_key(idx < ntot && cd[u].f >= gate, ord_key(cd[u].f), sm);
    }
    __syncthreads();
    nkeys = sm.sel_rem;
    int np = 8;  // at least 8: the rank sort reads keys eight at a time
    while (np < nkeys) np <<= 1;
    for (int p = nkeys + threadIdx.x; p < np; p += kBlock) sm.u.c.key[p] = 0u;
    __syncthreads();
    return np;
}

template <int ES>
__device__ __forceinline__ int slow_path(const DevGroup& G, const Ctx& c, Smem& sm, float m, double z, bool drop_eos,
                                         float& thr) {
    const float thr_k = stream_kth<ES>(G, c, sm, c.k_eff);
    thr = thr_k;
    if (c.p_active) {
        double zp;
        if (c.hf) {
            zp = z;
        } else {
            double part = 0.0;
            int ngt = 0;
            visit_row<ES>(G, c, sm, [&](float f, int) {
                if (finite_f(f) && f > thr_k) {
                    part += (double)expf(f - m);
                    ++ngt;
                }
            });
            zp = block_sum_d(part, sm);
            ngt = block_sum_i(ngt, sm);
            if (thr_k > -INFINITY) zp += (double)(c.k_eff - ngt) * (double)expf(thr_k - m);
        }
        const float thr_p = stream_mass<ES>(G, c, sm, thr_k, m, (double)c.top_p * zp * kMassScale);
        const float v_m = c.min_keep_eff <= 1 ? m : stream_kth<ES>(G, c, sm, c.min_keep_eff);
        thr = fmaxf(fminf(thr_p, v_m), thr_k);
    }
    return stream_draw<ES>(G, c, sm, thr, m, drop_eos, row_uniform(G, c));
}

// Exact processed value of the EOS id (every thread must call: its history count is a block reduction).
template <int ES>
__device__ __forceinline__ float eos_value(const DevGroup& G, const Ctx& c, Smem& sm) {
    int n = 0;
    if (c.counts) {
        const char* hrow = gp(G.history) + (int64_t)c.row * G.hist_stride * (G.hist_i64 ? 8 : 4);
        for (int i = threadIdx.x; i < G.hist_len; i += kBlock) {
            const int64_t h = G.hist_i64 ? ((const int64_t*)hrow)[i] : (int64_t)((const int32_t*)hrow)[i];
            n += h == (int64_t)G.eos;
        }
        n = block_sum_i(n, sm);
    }
    const char* rowp = gp(G.logits) + (int64_t)c.row * G.row_stride * ES;
    float x;
    if (ES == 2)
        x = __uint_as_float((uint32_t)(*(const uint16_t*)(rowp + (int64_t)G.eos * 2)) << 16);
    else
        x = *(const float*)(rowp + (int64_t)G.eos * 4);
    bool allowed = true;
    if (gp(G.allowed)) allowed = ((gp(G.allowed)[(int64_t)c.row * G.allowed_stride + (G.eos >> 5)] >> (G.eos & 31)) & 1u) != 0;
    return transform(x, G.eos, n, allowed, G, c, sm);
}

template <int ES>
__device__ __forceinline__ void finish_row(const DevGroup& G, const Ctx& c, Smem& sm, int64_t tok, float thr, float m,
                                           bool drop_eos) {
    if (c.want_out) write_outputs<ES>(G, c, sm, c.greedy ? -INFINITY : thr, m, drop_eos);
    update_state(G, c, tok);
}

// A top-p row without top-k from the slices' candidates: sorted, the nucleus cut over the full normaliser z is
// exact when it keeps only values >= gmax (every such value was published).  Returns false (LDS candidates
// spent) when the candidates do not settle it.
__device__ __forceinline__ bool nucleus_from_cands(const DevGroup& G, const Ctx& c, Smem& sm, const RowWs& w, int ntot,
                                                   bool overflow, float gmax, float m, double z, bool drop_eos,
                                                   bool need_tok, float& thr, int64_t& tok) {
    if (overflow || ntot <= 0 || ntot > kCapRow) return false;
    int nge = 0;
    const int np = gather_cands(c, sm, w, ntot, gmax, nge);
    if (nge <= 0) return false;
    sort_keys_desc(sm, np);
    int kept = 0;
    double zge = 0.0;
    const float t = sorted_threshold(c, sm, nge, m, z, &kept, &zge);
    // settled when the cut falls inside the values >= gmax: a kept rank past them, or their mass short of the
    // target, would need values that were not published
    const bool settled = gmax == -INFINITY || kept < nge || (kept == nge && zge >= (double)c.top_p * z);
    if (!settled) return false;
    release_held(G, c, sm, kHeldDone);
    thr = t;
    if (need_tok) tok = cand_draw(G, c, sm, ntot, thr, m, drop_eos, row_uniform(G, c));
    return true;
}

// The max, first argmax and full normaliser of the row straight from its logits (no published data), for a row
// whose slices did not all run on the finaliser's XCD.  An all -inf row answers index 0, like the slice path.
template <int ES>
__device__ __forceinline__ void stream_stats(const DevGroup& G, const Ctx& c, Smem& sm, float& m, int& am, double& z) {
    // max pass, then the first index of the max and the normaliser; plain loops over the row's 16-byte chunks
    constexpr int E = 16 / ES;
    float mx = -INFINITY;
    int ai = INT_MAX;
    double zpart = 0.0;
    for (int pass = 0; pass < 2; ++pass) {
        if (pass == 1) m = block_max(mx, sm);
        for (int s = 0; s < c.S; ++s) {
            const Geo g = slice_geo<ES>(G, c, s);
            if (c.counts) build_counts(G, c, g.first, g.lo, g.hi, (g.hi - g.first + 1) >> 1, sm);
            const uint32_t* mrow = gp(G.allowed) ? gp(G.allowed) + (int64_t)c.row * G.allowed_stride : nullptr;
            const int nwords = (c.V + 31) >> 5;
            for (int ch = threadIdx.x; ch < g.nchunk; ch += kBlock) {
                const uint4 raw = *(const uint4*)(g.base + (uintptr_t)ch * 16);
                const MaskPair mk = mrow ? mask_pair(mrow, nwords, g.first + ch * E) : MaskPair{~0u, ~0u, 0};
                for (int e = 0; e < E; ++e) {
                    const int j = g.first + ch * E + e;
                    if (j < g.lo || j >= g.hi) continue;
                    const int n = c.counts ? count_of(sm, j - g.first) : 0;
                    const float f = transform(raw_elem<ES>(raw, e), j, n, mrow ? mask_bit(mk, j) : true, G, c, sm);
                    if (pass == 0) {
                        mx = fmaxf(mx, f);
                    } else {
                        if (f == m && j < ai) ai = j;
                        if (finite_f(f)) zpart += (double)expf(f - m);
                    }
                }
            }
        }
    }
    am = m > -INFINITY ? block_min_i(ai, sm) : 0;  // an all -inf row answers index 0, like the slice path
    if (am == INT_MAX) am = 0;
    z = block_sum_d(zpart, sm);
}

// A top-p row without top-k whose nucleus the published candidates do not settle: the slices' mass histograms,
// merged on the global 1/8-logit grid below the row's top bin, locate the bin holding the top-p boundary.  When
// one does, its pending record is stored, the held slices are released to resolve it, and true is returned.
__device__ __forceinline__ bool pick_bin(const DevGroup& G, const Ctx& c, Smem& sm, const RowWs& w, float m, double z) {
    Pending* pend = (Pending*)(gp(G.pending) + (int64_t)c.grow * sizeof(Pending));
    const int HB = bin_of(m);
    double gm = 0.0;
    uint32_t gc = 0u;
    const int o = threadIdx.x;  // one global bin per thread (kNB == kBlock)
    for (int s0 = 0; s0 < c.S; s0 += 8) {  // 8 slices' loads in flight at a time
        unsigned long long hm[8];
        uint32_t hc[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int s = s0 + u;
            hm[u] = 0ull;
            hc[u] = 0u;
            if (s < c.S && sm.summ[s].m > -INFINITY) {
                const int os = o - (HB - sm.summ[s].hb);
                if (os >= 0 && os < kNB) {
                    hm[u] = pub_ld(&w.hmass[(int64_t)s * kNB + os]);
                    hc[u] = pub_ld(&w.hcnt[(int64_t)s * kNB + os]);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int s = s0 + u;
            if (hc[u] != 0u || hm[u] != 0ull)
                gm += (double)hm[u] * (1.0 / kMassScale) * sm.tile_sum[s];
            gc += hc[u];
        }
    }
    double ztot;
    const double before = block_excl_scan_d(gm, ztot, sm);
    const double target = (double)c.top_p * z;
    const int bstar = block_max_i((gc > 0u && before < target) ? o : -1, sm);
    int under = 0;
    for (int s = 0; s < c.S; ++s) under += sm.summ[s].under_n;
    const bool below_window = ztot < target && under > 0;  // the boundary may lie under the window
    if (bstar >= 0 && bstar < kNB - 1 && !below_window) {
        if (threadIdx.x == 0) {
            Pending p;
            p.mode_ = 0;
            p.lo_v = (float)(HB - bstar) / kBinScale;
            p.hi_v = (float)(HB - bstar + 1) / kBinScale;
            p.m = m;
            p.z = z;
            p.target = target;
            *pend = p;
        }
        release_held(G, c, sm, kHeldBin);
        return true;
    }
    return false;
}

// The finaliser of a top-p row without top-k, before anything else: when the published candidates cannot hold
// the nucleus (their mass is short of top_p), the boundary bin is chosen at once, while the finaliser's slice is
// still in registers.  Merges the summaries (the finaliser is then told so).
__device__ __forceinline__ bool early_bin(const DevGroup& G, const Ctx& c, Smem& sm, const RowWs& w) {
    if (sm.foreign != 0 || (G.flags & MIS_FINALIZE_STREAMING) != 0) return false;
    merge_summaries(c, sm, w);
    const float m = sm.fin.m;
    const double z = sm.fin.z;
    if (!(m > -INFINITY) || sm.fin.cmass >= (double)c.top_p * z) return false;
    if (threadIdx.x == 0) sm.decision = 0u;
    return pick_bin(G, c, sm, w, m, z);
}

// Returns true when the row's boundary bin is needed: the pending record is stored and the held slices released
// to publish it; the caller then resolves its own slice's part.
template <int ES>
__device__ __forceinline__ bool finalize(const DevGroup& G, const Ctx& c, Smem& sm, const RowWs& w, bool merged) {
    constexpr int E = 16 / ES;
    constexpr int NSB = kNV / E * kWaves;
    float m = -INFINITY, gmax = -INFINITY;
    double z = 0.0, cmass = 0.0;  // cmass: top-p-only rows, the published candidates' mass
    int am = INT_MAX, ntot = 0;
    bool overflow = false;
    // no published data: everything below streams the row
    const bool foreign = sm.foreign != 0 || (G.flags & MIS_FINALIZE_STREAMING) != 0;
    if (threadIdx.x == 0) sm.decision = 0u;
    if (foreign) {
        release_held(G, c, sm, kHeldDone);  // the held slices' publications would not be readable here
        stream_stats<ES>(G, c, sm, m, am, z);
    } else {
        if (!merged) merge_summaries(c, sm, w);
        m = sm.fin.m;
        am = sm.fin.am;
        z = sm.fin.z;
        cmass = sm.fin.cmass;
        gmax = sm.fin.gmax;
        ntot = sm.fin.ntot;
        overflow = sm.fin.overflow != 0;
    }
    const bool drop_eos = c.hf && c.censor;
    const bool need_tok = gp(G.tokens) != nullptr || (G.flags & MIS_UPDATE_STATE);
    int64_t tok = kPad;
    float thr = -INFINITY;
    if (c.greedy) {
        tok = am == INT_MAX ? c.V - 1 : am;
    } else if (!(m > -INFINITY)) {
        tok = c.V - 1;  // nothing allowed: the reference's clamp value
    } else if (c.full_draw && !foreign) {
        if (need_tok) {
            // survivors = every finite value (minus a censored EOS): the published sub-block sums
            const int nsb = c.S * NSB;
            for (int i = threadIdx.x; i < nsb; i += kBlock) {
                const int s = i / NSB;
                sm.u.sbs[i] = pub_ld(&w.sb[(int64_t)s * kMaxSB + (i % NSB)]) * sm.tile_sum[s];
            }
            __syncthreads();
            if (drop_eos) {
                const float fe = eos_value<ES>(G, c, sm);
                if (threadIdx.x == 0 && finite_f(fe)) {
                    const int s = G.eos / c.slice_len;
                    const Geo g = slice_geo<ES>(G, c, s);
                    const int i = s * NSB + sub_block_of<ES>(g, G.eos);
                    sm.u.sbs[i] = fmax(0.0, sm.u.sbs[i] - (double)expf(fe - m));
                }
                __syncthreads();
            }
            tok = sub_block_draw<ES>(G, c, sm, nsb, -INFINITY, m, drop_eos, row_uniform(G, c));
        }
    } else if (c.cand_mode && !foreign && !overflow && ntot <= kCapRow) {
        // candidates of all slices in vocabulary order; keys of those >= gmax
        int nge = 0;
        const int np = gather_cands(c, sm, w, ntot, gmax, nge);
        // every value >= gmax was published: the k-th largest is proven once k of them are >= gmax
        if (nge >= c.k_eff || gmax == -INFINITY) {
            sort_keys_desc(sm, np);
            thr = sorted_threshold(c, sm, nge, m, z);
            if (need_tok) tok = cand_draw(G, c, sm, ntot, thr, m, drop_eos, row_uniform(G, c));
        } else {
            tok = slow_path<ES>(G, c, sm, m, z, drop_eos, thr);
        }
    } else if (c.nucleus && !foreign && cmass >= (double)c.top_p * z &&  // else the candidates cannot settle it
               nucleus_from_cands(G, c, sm, w, ntot, overflow, gmax, m, z, drop_eos, need_tok, thr, tok)) {
        // resolved from the published candidates
    } else if (c.nucleus && !foreign) {
        if (pick_bin(G, c, sm, w, m, z)) return true;  // the row's slices resolve the bin, the last of them draws
        release_held(G, c, sm, kHeldDone);
        tok = slow_path<ES>(G, c, sm, m, z, drop_eos, thr);
    } else {
        release_held(G, c, sm, kHeldDone);
        tok = slow_path<ES>(G, c, sm, m, z, drop_eos, thr);
    }
    release_held(G, c, sm, kHeldDone);
    finish_row<ES>(G, c, sm, tok, thr, m, drop_eos);
    return false;
}

// ---------------------------------------------------------------- the slice phase

// The slice phase's results: max, first argmax (greedy rows), normaliser and, by row kind, the mass histogram,
// sub-block sums or candidates, then the slice's summary.
template <int ES>
__device__ __forceinline__ void publish_slice(const DevGroup& G, const Ctx& c, const Geo& geo, const Tile& T,
                                              const RowWs& w, const int slice, Smem& sm) {
    constexpr int E = 16 / ES;
    constexpr int NCH = kNV / E;
    float tm = -INFINITY;
#pragma unroll
    for (int q = 0; q < kNV; ++q) tm = fmaxf(tm, T.v[q]);
    const float m = block_max(tm, sm);
    int am = INT_MAX;
    if (c.greedy) {
        // lowest slot holding m; out-of-slice slots hold -inf, so an all -inf slice answers its first element
        int fq = kNV;
#pragma unroll
        for (int q = kNV - 1; q >= 0; --q) fq = T.v[q] == m ? q : fq;
        const int first = fq < kNV ? tile_index<ES>(geo, fq) : INT_MAX;
        am = m > -INFINITY ? block_min_i(first, sm) : geo.lo;
    }
    double z = 0.0;
    int ncand = 0, overflow = 0, hb = 0, under_n = 0;
    double cmass = 0.0;
    unsigned long long under_q = 0ull;
    float g = INFINITY;
    if (c.nucleus && m > -INFINITY) {
        // top-p without top-k: the sum of exp and the mass histogram in one pass, one exp per element
        hb = bin_of(m);
        for (int b = threadIdx.x; b < kNB; b += kBlock) {
            sm.hcnt[b] = 0u;
            sm.hmass[b] = 0ull;
        }
        __syncthreads();
        double part = 0.0;
        unsigned long long uq = 0ull;
        int un = 0;
#pragma unroll
        for (int q = 0; q < kNV; ++q) {
            const float f = T.v[q];
            if (finite_f(f)) {
                const float e = expf(f - m);
                part += (double)e;
                const int o = hb - bin_of(f);
                const unsigned long long mq = (unsigned long long)((double)e * kMassScale);  // mass_q(f, m)
                if (o < kNB) {
                    atomicAdd(&sm.hcnt[o], 1u);
                    if (mq) atomicAdd(&sm.hmass[o], mq);
                } else {
                    uq += mq;
                    ++un;
                }
            }
        }
        block_sum3(part, uq, un, sm);  // includes barriers: the histogram is complete
        z = part;
        under_q = uq;
        under_n = un;
        if (threadIdx.x < 64)
            for (int b = threadIdx.x; b < kNB; b += 64) {
                pub_st(&w.hcnt[(int64_t)slice * kNB + b], sm.hcnt[b]);
                pub_st(&w.hmass[(int64_t)slice * kNB + b], sm.hmass[b]);
            }
    } else if (c.full_draw && m > -INFINITY) {
        // unfiltered rows draw from the sub-block sums
        const double part = tile_sub_sums<ES>(T, m, -INFINITY, sm);
        z = block_sum_d(part, sm);  // includes a barrier: sm.sbw is complete
        if ((int)threadIdx.x < NCH * kWaves) pub_st(&w.sb[(int64_t)slice * kMaxSB + threadIdx.x], sm.sbw[threadIdx.x]);
    } else if (c.need_mass && m > -INFINITY) {
        // the full-row normaliser only
        double part = 0.0;
#pragma unroll
        for (int q = 0; q < kNV; ++q)
            if (finite_f(T.v[q])) part += (double)expf(T.v[q] - m);
        z = block_sum_d(part, sm);
    }
    if (c.cand_mode || c.nucleus) {
        // tau = the cand_target-th largest per-thread maximum: at least cand_target values are >= tau
        g = block_kth_of_256(tm, c.cand_target, sm);
        const int run = publish_range<ES>(T, geo, g, INFINITY, w.cand + (int64_t)slice * kCapSlice, sm);
        ncand = min(run, kCapSlice);
        overflow = run > kCapSlice;
        if (c.nucleus && threadIdx.x < 64) {  // wave 0 holds the staged candidates: their mass
            double part = 0.0;
            for (int p = threadIdx.x; p < ncand; p += 64) part += (double)expf(sm.stage[p].f - m);
            cmass = wave_sum_d(part);
        }
    }
    if (threadIdx.x == 0) {
        SliceSummary s;
        s.m = m;
        s.g = g;
        s.z = z;
        s.argmax = am;
        s.ncand = ncand;
        s.overflow = overflow;
        s.hb = hb;
        s.under_q = under_q;
        s.under_n = under_n;
        s.n_hi = 0;
        s.hi_mass = cmass;
        pub_st_summary(&w.summ[slice], s);
    }
}

template <int ES>
__device__ __forceinline__ void resolve_bin(const DevGroup& G, const Ctx& c, const Geo& geo, const Tile& T,
                                            const RowWs& w, const int slice, Smem& sm);

template <int ES>
__device__ __forceinline__ void run_row(const DevGroup& G, const int row, const int slice, Smem& sm) {
    // the slice's tile, mask words and history, then the row's parameters, go out before any of them is used
    const Geo geo = slice_geo_at<ES>(G, row, slice);
    RawTile<ES> R;
    issue_tile<ES>(geo, R);
    Preload P;
    preload(G, row, geo, P);
    RowParams q;
    load_params(G, row, q);
    Ctx c;
    init_ctx(G, row, slice, q, c);
    const RowWs w = row_ws(gp(G.ws) + (int64_t)row * G.ws_row_bytes, c.S, G.tiles != 0);
    if ((!c.live && !c.want_out) || c.forced) {
        if (slice != 0) return;
        if (!c.forced) {
            if (threadIdx.x == 0 && gp(G.tokens)) gp(G.tokens)[row] = kPad;
            return;
        }
        if (c.want_out) write_outputs<ES>(G, c, sm, -INFINITY, 0.0f, false);
        update_state(G, c, G.eos);
        return;
    }
    Tile T;
    finish_tile<ES>(G, c, geo, R, P, T, sm);
    publish_slice<ES>(G, c, geo, T, w, slice, sm);
    // the branches below are uniform: read through readfirstlane so the compiler keeps them as scalar branches
    // (a branch it takes for divergent would run both sides and keep T live across the finaliser)
    if (c.S > 1 && !uni((int)arrive_last(row_counter(G, c), c.S, sm))) {
        if (!holds_slices(c)) return;
        const uint32_t d = (uint32_t)uni((int)await_decision(G, c, sm));
        if (d == kHeldDone) depart(G, c);
        if (d != kHeldBin) return;
        // this slice's values are still in T
    } else {
        if (c.S == 1) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the slice's publications are in the L2
            if (threadIdx.x == 0) sm.foreign = 0;
            __syncthreads();
        }
        const bool merged = c.nucleus;
        if (!(c.nucleus && uni((int)early_bin(G, c, sm, w)))) {
            if (!uni((int)finalize<ES>(G, c, sm, w, merged))) return;
            // the bin after the candidates failed: the finaliser's registers did not keep its slice
            issue_tile<ES>(geo, R);
            preload(G, row, geo, P, false);  // (the counts then load the history themselves)
            finish_tile<ES>(G, c, geo, R, P, T, sm);
        }
    }
    resolve_bin<ES>(G, c, geo, T, w, slice, sm);
}

// ---------------------------------------------------------------- the boundary bin

// A held slice's part once the row needs its boundary bin [lo_v, hi_v) (the pending record): the sums per
// sub-block of its values above the bin and the values inside it, published; the last of the row's slices to
// arrive then finds the exact top-p threshold inside the bin and draws.
template <int ES>
__device__ __forceinline__ void resolve_bin(const DevGroup& G, const Ctx& c, const Geo& geo, const Tile& T,
                                            const RowWs& w, const int slice, Smem& sm) {
    constexpr int E = 16 / ES;
    constexpr int NCH = kNV / E;
    constexpr int NSB = NCH * kWaves;
    Pending* pend = (Pending*)(gp(G.pending) + (int64_t)c.grow * sizeof(Pending));
    if (threadIdx.x == 0) {
        Pending p;
        p.lo_v = pub_ld(&pend->lo_v);
        p.hi_v = pub_ld(&pend->hi_v);
        p.m = pub_ld(&pend->m);
        p.z = pub_ld(&pend->z);
        p.target = pub_ld(&pend->target);
        sm.held = p;
    }
    __syncthreads();
    const Pending P = sm.held;
    if (w.tile != nullptr) {  // the processed values, for the draw inside one sub-block (first: they drain meanwhile)
        float* tl = w.tile + (int64_t)slice * kNV * kBlock + threadIdx.x;
#pragma unroll
        for (int q = 0; q < kNV; ++q) pub_st(&tl[q * kBlock], T.v[q]);
    }
    // everything above the boundary bin survives: its sums per sub-block; the bin's values go to the finaliser
    const double part = tile_sub_sums<ES>(T, P.m, P.hi_v, sm);
    int nhi = 0;
#pragma unroll
    for (int q = 0; q < kNV; ++q)
        if (finite_f(T.v[q]) && T.v[q] >= P.hi_v) ++nhi;
    const double hi_mass = block_sum_d(part, sm);
    nhi = block_sum_i(nhi, sm);
    if ((int)threadIdx.x < NSB) pub_st(&w.sb[(int64_t)slice * kMaxSB + threadIdx.x], sm.sbw[threadIdx.x]);
    const int run = publish_range<ES>(T, geo, P.lo_v, P.hi_v, w.cand + (int64_t)slice * kCapSlice, sm);
    if (threadIdx.x == 0) {
        SliceSummary& s = w.summ[slice];
        pub_st(&s.ncand, min(run, kCapSlice));
        pub_st(&s.overflow, (int32_t)(run > kCapSlice));
        pub_st(&s.n_hi, nhi);
        pub_st(&s.hi_mass, hi_mass);
    }
    if (c.S > 1) {
        if (!arrive_last(row_counter(G, c), c.S, sm)) return;
        // every held slice has read the decision word: clear it for the next launch
        if (threadIdx.x == 0)
            __hip_atomic_store(row_counter(G, c) + kDecisionWord, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the slice's publications are in the L2
        if (threadIdx.x == 0) sm.foreign = 0;
        __syncthreads();
    }
    // ---- finalise: exact top-p inside the boundary bin, then the draw (a row split across XCDs streams instead)
    const bool foreign = sm.foreign != 0;
    if (!foreign) load_summaries<ES>(c, sm, w);
    const float m = P.m;
    const bool drop_eos = c.hf && c.censor;
    int ntot = 0, nabove = 0;
    bool overflow = false;
    double above = 0.0;
    for (int s = 0; s < c.S; ++s) {
        ntot += sm.summ[s].ncand;
        nabove += sm.summ[s].n_hi;
        above += sm.summ[s].hi_mass;
        overflow |= sm.summ[s].overflow != 0;
    }
    float thr = -INFINITY;
    int64_t tok = kPad;
    bool exact = !foreign && !overflow && ntot <= kCapRow && ntot > 0 && above < P.target;
    if (exact) {
        int nkeys = 0;
        gather_cands(c, sm, w, ntot, INFINITY, nkeys);  // the bin's values and ids in vocabulary order (no keys)
        // The cut inside the bin without sorting it: 256 sub-buckets of the bin, highest first, with fixed-point
        // masses; the sub-bucket where the running mass crosses the target is the only one sorted.
        const float scale = (float)kNB / (P.hi_v - P.lo_v);
        auto bucket = [&](float f) { return min(max((int)((P.hi_v - f) * scale), 0), kNB - 1); };
        for (int b = threadIdx.x; b < kNB; b += kBlock) {
            sm.hcnt[b] = 0u;
            sm.hmass[b] = 0ull;  // (the gather's slice map lived here)
        }
        __syncthreads();
        for (int q = threadIdx.x; q < ntot; q += kBlock) {
            const float f = sm.u.c.val[q];
            const int b = bucket(f);
            atomicAdd(&sm.hcnt[b], 1u);
            atomicAdd(&sm.hmass[b], mass_q(f, m));
        }
        __syncthreads();
        // one sub-bucket per thread (kNB == kBlock): exclusive scan of mass << 12 | count from the top (ntot <= 2048)
        const unsigned long long cq = sm.hcnt[threadIdx.x], mq = sm.hmass[threadIdx.x];
        unsigned long long tot_pk;
        const unsigned long long ex_pk = block_excl_scan_u((mq << 12) | cq, tot_pk, sm);
        const double tq = (P.target - above) * kMassScale;  // the bin's share of the target, in mass_q units
        const int bstar = block_max_i(cq > 0 && (double)(ex_pk >> 12) < tq ? (int)threadIdx.x : -1, sm);
        if ((int)threadIdx.x == bstar) {
            sm.sel_bin = (int)(ex_pk & 4095ull);  // bin values ranked above the sub-bucket
            sm.sel_acc = ex_pk >> 12;            // and their mass
        }
        if (threadIdx.x == 0) {
            sm.sel_rem = 0;
            sm.kmin = ~0u;
            sm.kmax = 0u;
        }
        __syncthreads();
        const int n_before = sm.sel_bin;
        const unsigned long long m_before = sm.sel_acc;
        if (bstar < 0 || (double)(tot_pk >> 12) < tq) {
            exact = false;  // the whole bin short of the target: the cut lies under the bin (streaming path)
        } else {
            // the sub-bucket's keys (bf16 inputs make many exact ties here), sorted descending
            uint32_t kmin = ~0u, kmax = 0u;
            for (int q0 = 0; q0 < ntot; q0 += kBlock) {  // block-uniform trip count (append_key ballots)
                const int q = q0 + threadIdx.x;
                const float f = q < ntot ? sm.u.c.val[q] : -INFINITY;
                const bool in = q < ntot && bucket(f) == bstar;
                const uint32_t k = ord_key(f);
                append_key(in, k, sm);
                kmin = in ? min(kmin, k) : kmin;
                kmax = in ? max(kmax, k) : kmax;
            }
            kmin = wave_reduce(kmin, [](uint32_t a, uint32_t b) { return min(a, b); });
            kmax = wave_reduce(kmax, [](uint32_t a, uint32_t b) { return max(a, b); });
            if (lane_id() == 0) {
                atomicMin(&sm.kmin, kmin);
                atomicMax(&sm.kmax, kmax);
            }
            __syncthreads();
            const int nbk = sm.sel_rem;
            int np = 8;
            while (np < nbk) np <<= 1;
            for (int q = nbk + threadIdx.x; q < np; q += kBlock) sm.u.c.key[q] = 0u;
            __syncthreads();
            // one distinct value (bf16 ties): the keys, then the zero padding, are in order already
            if (sm.kmin != sm.kmax) sort_keys_desc(sm, np);
            // ranks (blocked per thread) whose exclusive mass, above the sub-bucket included, is below the target
            const int per = (nbk + kBlock - 1) / kBlock;
            const int r0 = min(nbk, (int)threadIdx.x * per), r1 = min(nbk, r0 + per);
            unsigned long long mine = 0ull;
            for (int r = r0; r < r1; ++r) mine += mass_q(key_float(sm.u.c.key[r]), m);
            unsigned long long run_tot;
            unsigned long long run = m_before + block_excl_scan_u(mine, run_tot, sm);
            int kp = 0;
            for (int r = r0; r < r1; ++r) {
                if ((double)run < tq) ++kp;
                run += mass_q(key_float(sm.u.c.key[r]), m);
            }
            const int kept_in = block_sum_i(kp, sm);
            // ranks kept above the sub-bucket and in it; fewer than min_keep: the streaming path
            exact = kept_in >= 1 && nabove + n_before + kept_in >= c.min_keep_eff;
            if (exact) thr = key_float(sm.u.c.key[kept_in - 1]);
        }
    }
    const bool need_tok = gp(G.tokens) != nullptr || (G.flags & MIS_UPDATE_STATE);
    const float fe = drop_eos ? eos_value<ES>(G, c, sm) : -INFINITY;
    const int nsb = c.S * NSB;
    if (!exact) {
        tok = slow_path<ES>(G, c, sm, m, P.z, drop_eos, thr);
    } else if (need_tok && nsb <= kCapSlice) {
        // survivor sums per sub-block: the values above the bin (published) plus the bin's survivors, whose
        // fixed-point masses are added per sub-block (the sub-block of a candidate follows from its id)
        unsigned long long* sbq = (unsigned long long*)sm.stage;
        for (int i = threadIdx.x; i < nsb; i += kBlock) sbq[i] = 0ull;
        __syncthreads();
        for (int q = threadIdx.x; q < ntot; q += kBlock) {
            const float f = sm.u.c.val[q];
            const int id = sm.u.c.id[q];
            if (f >= thr && !(drop_eos && id == G.eos)) {
                const int s = id / c.slice_len;
                atomicAdd(&sbq[s * NSB + sub_block_of<ES>(slice_geo<ES>(G, c, s), id)], mass_q(f, m));
            }
        }
        __syncthreads();  // the candidates are spent: sm.u.sbs may overwrite them
        for (int i = threadIdx.x; i < nsb; i += kBlock) {
            const int s = i / NSB, sb = i % NSB;
            double v = pub_ld(&w.sb[(int64_t)s * kMaxSB + sb]) + (double)sbq[i] * (1.0 / kMassScale);
            if (drop_eos && finite_f(fe) && fe >= P.hi_v && G.eos / c.slice_len == s &&
                sub_block_of<ES>(slice_geo<ES>(G, c, s), G.eos) == sb)
                v = fmax(0.0, v - (double)expf(fe - m));
            sm.u.sbs[i] = v;
        }
        __syncthreads();
        tok = sub_block_draw<ES>(G, c, sm, nsb, thr, m, drop_eos, row_uniform(G, c), w.tile);
    } else if (need_tok) {
        // many sub-blocks: survivor sums per sub-block by binary search over the vocabulary-ordered candidates
        for (int i = threadIdx.x; i < nsb; i += kBlock) {
            const int s = i / NSB, sb = i % NSB;
            double v = pub_ld(&w.sb[(int64_t)s * kMaxSB + sb]);
            const Geo g = slice_geo<ES>(G, c, s);
            const int ch0 = (sb / kWaves) * kBlock + (sb % kWaves) * 64;
            const int jlo = max(g.lo, g.first + ch0 * E), jhi = min(g.hi, g.first + (ch0 + 64) * E);
            int a = 0, b = ntot;  // first candidate with id >= jlo
            while (a < b) {
                const int mid = (a + b) >> 1;
                if (sm.u.c.id[mid] < jlo)
                    a = mid + 1;
                else
                    b = mid;
            }
            for (int q = a; q < ntot && sm.u.c.id[q] < jhi; ++q) {
                const float f = sm.u.c.val[q];
                if (f >= thr && !(drop_eos && sm.u.c.id[q] == G.eos)) v += (double)expf(f - m);
            }
            if (drop_eos && G.eos >= jlo && G.eos < jhi && finite_f(fe) && fe >= P.hi_v)
                v = fmax(0.0, v - (double)expf(fe - m));
            pub_st(&w.sb[(int64_t)s * kMaxSB + sb], v);  // staged in global memory: LDS still holds the candidates
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // in the L2 before other threads read them back
        __syncthreads();
        for (int i = threadIdx.x; i < nsb; i += kBlock) sm.u.sbs[i] = pub_ld(&w.sb[(int64_t)(i / NSB) * kMaxSB + i % NSB]);
        __syncthreads();
        tok = sub_block_draw<ES>(G, c, sm, nsb, thr, m, drop_eos, row_uniform(G, c), w.tile);
    }
    finish_row<ES>(G, c, sm, tok, thr, m, drop_eos);
}

// The kernel arguments, read in place from the kernarg segment (a by-value parameter indexed with a run-time
// group index can be copied whole to scratch).
__device__ __forceinline__ const KernelArgs& kernel_args() {
    return *(const KernelArgs*)__builtin_amdgcn_kernarg_segment_ptr();
}



__device__ __forceinline__ bool locate(const KernelArgs& args, int& gi, int& row, int& slice) {
    const int x = blockIdx.x % 8;
    int i = blockIdx.x / 8;
    for (gi = 0; gi < args.n_groups; ++gi) {
        const int S = args.g[gi].slices;
        const int n = args.seg_rows[x][gi] * S;
        if (i < n) {
            row = args.seg_row[x][gi] + i / S;
            slice = i % S;
            return true;
        }
        i -= n;
    }
    return false;
}

__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(4, 8))) void sample_kernel(const KernelArgs args_in) {
    (void)args_in;
    const KernelArgs& args = kernel_args();
    __shared__ Smem sm;
    int gi, row, slice;
    if (!locate(args, gi, row, slice)) return;
    const DevGroup& G = args.g[gi];
    if (G.es == 2)
        run_row<2>(G, row, slice, sm);
    else
        run_row<4>(G, row, slice, sm);
}

__global__ void uniform_kernel(const int64_t* seeds, const int64_t* steps, const int64_t* rids, int64_t n, int rng,
                               float* out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int64_t s = seeds ? seeds[i] : 0, t = steps ? steps[i] : 0;
    out[i] = rng == MIS_RNG_PHILOX ? philox_uniform(s, t, rids ? rids[i] : 0) : counter_uniform(s, t);
}

// ---------------------------------------------------------------- host side

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int max_slice_elems(int es) { return kBlock * kNV - 16 / es; }

// Workspace: [arrival counters, kCounterBytes][pending records, kPendingBytes][per group: rows x row regions].
constexpr int64_t kFixedBytes = kCounterBytes + kPendingBytes;

// Whether some row of the group can be a top-p row without top-k (its row regions then hold the tile area).
bool may_hold_nucleus(const MisGroup& g) {
    const bool k_all = g.top_k != nullptr || ((g.flags & MIS_TOPK_ZERO_DISABLES) && g.top_k_value <= 0) ||
                       std::max(g.top_k_value, g.min_keep) >= g.vocab;
    const bool p_on = g.top_p != nullptr || !((g.flags & MIS_TOPP_ONE_DISABLES) && g.top_p_value >= 1.0f);
    const bool sampling = g.temperature != nullptr || g.temperature_value > 0.0f;
    return k_all && p_on && sampling;
}

int check_group(const MisGroup& g, int idx) {
    if (!g.logits && g.rows > 0) return fail(MIS_E_ARG, "group %d: logits is NULL", idx);
    if (g.dtype != MIS_F32 && g.dtype != MIS_BF16) return fail(MIS_E_ARG, "group %d: unknown dtype %d", idx, g.dtype);
    if (g.vocab < 1) return fail(MIS_E_ARG, "group %d: vocab must be >= 1 (got %d)", idx, g.vocab);
    if (g.rows < 0) return fail(MIS_E_ARG, "group %d: rows must be >= 0", idx);
    if (g.logits_row_stride < g.vocab) return fail(MIS_E_ARG, "group %d: logits row stride < vocab", idx);
    if (g.semantics != MIS_OMNI && g.semantics != MIS_HF)
        return fail(MIS_E_ARG, "unknown Talker sampling semantics: %d", g.semantics);
    if (g.min_keep < 1) return fail(MIS_E_ARG, "group %d: min_keep must be >= 1", idx);
    if (g.rng != MIS_RNG_COUNTER && g.rng != MIS_RNG_PHILOX) return fail(MIS_E_ARG, "unknown RNG mode: %d", g.rng);
    if (g.history_len < 0 || g.history_len > 65535)
        return fail(MIS_E_ARG, "group %d: history_len must be in [0, 65535]", idx);
    if (g.history_len > 0 && g.history) {
        if (g.history_row_stride < g.history_len) return fail(MIS_E_ARG, "group %d: history row stride < history_len", idx);
        if (g.history_mode != MIS_HISTORY_WINDOW && g.history_mode != MIS_HISTORY_RING)
            return fail(MIS_E_ARG, "group %d: unknown history mode %d", idx, g.history_mode);
        if (g.history_mode == MIS_HISTORY_RING && !g.history_head)
            return fail(MIS_E_ARG, "group %d: ring history needs history_head", idx);
    }
    if (g.allowed && g.allowed_row_stride < (g.vocab + 31) / 32)
        return fail(MIS_E_ARG, "group %d: allowed row stride < ceil(vocab / 32)", idx);
    if (g.eos >= g.vocab) return fail(MIS_E_ARG, "group %d: eos %d outside the vocabulary", idx, g.eos);
    if (g.alpha_lut_len < 0 || (g.alpha_lut_len > 0 && !g.alpha_lut))
        return fail(MIS_E_ARG, "group %d: alpha_lut_len without alpha_lut", idx);
    if (g.processed && g.processed_row_stride < g.vocab) return fail(MIS_E_ARG, "group %d: processed stride < vocab", idx);
    if (g.probs && g.probs_row_stride < g.vocab) return fail(MIS_E_ARG, "group %d: probs stride < vocab", idx);
    const int es = g.dtype == MIS_BF16 ? 2 : 4;
    const int s = (g.vocab + max_slice_elems(es) - 1) / max_slice_elems(es);
    if (s > kMaxSlices) return fail(MIS_E_UNSUPPORTED, "group %d: vocab %d exceeds %d slices", idx, g.vocab, kMaxSlices);
    return 0;
}

}  // namespace

extern "C" {

int mis_version(void) { return MIS_ABI_VERSION; }

const char* mis_last_error(void) { return g_err.c_str(); }

size_t mis_sizeof_group(void) { return sizeof(MisGroup); }

size_t mis_workspace_bytes(const MisGroup* groups, int n_groups) {
    if (!groups || n_groups < 1 || n_groups > kMaxGroups) return 0;
    size_t total = (size_t)kFixedBytes;
    for (int i = 0; i < n_groups; ++i) {
        if (check_group(groups[i], i)) return 0;
        const int es = groups[i].dtype == MIS_BF16 ? 2 : 4;
        const int s = (groups[i].vocab + max_slice_elems(es) - 1) / max_slice_elems(es);
        total += (size_t)row_ws_bytes(s, may_hold_nucleus(groups[i])) * (size_t)groups[i].rows;
    }
    return total;
}

int mis_sample(const MisGroup* groups, int n_groups, void* workspace, size_t workspace_bytes, void* stream) {
    g_err.clear();
    if (!groups || n_groups < 1 || n_groups > kMaxGroups)
        return fail(MIS_E_ARG, "n_groups must be in [1, %d]", kMaxGroups);
    KernelArgs a;
    memset(&a, 0, sizeof a);
    a.n_groups = n_groups;
    int blocks = 0, rows_total = 0;
    size_t ws_off = (size_t)kFixedBytes;
    for (int i = 0; i < n_groups; ++i) {
        const MisGroup& g = groups[i];
        if (int rc = check_group(g, i)) return rc;
        DevGroup& d = a.g[i];
        d.logits = (const char*)g.logits;
        d.row_stride = g.logits_row_stride;
        d.es = g.dtype == MIS_BF16 ? 2 : 4;
        d.vocab = g.vocab;
        d.rows = g.rows;
        d.semantics = g.semantics;
        d.flags = g.flags;
        d.min_keep = g.min_keep;
        d.temperature = g.temperature;
        d.top_k = g.top_k;
        d.top_p = g.top_p;
        d.repetition = g.repetition;
        d.presence = g.presence;
        d.frequency = g.frequency;
        d.t_val = g.temperature_value;
        d.p_val = g.top_p_value;
        d.rep_val = g.repetition_value;
        d.pres_val = g.presence_value;
        d.freq_val = g.frequency_value;
        d.k_val = g.top_k_value;
        d.alpha_lut = g.alpha_lut;
        d.alpha_lut_len = g.alpha_lut ? g.alpha_lut_len : 0;
        d.hist_len = g.history ? g.history_len : 0;
        d.history = (const char*)g.history;
        d.hist_stride = g.history_row_stride;
        d.hist_i64 = g.history_is_int64 ? 1 : 0;
        d.hist_mode = g.history_mode;
        d.hist_head = g.history_head;
        d.allowed = g.allowed;
        d.allowed_stride = g.allowed_row_stride;
        d.eos = g.eos < 0 ? -1 : g.eos;
        d.min_new = g.min_new_tokens;
        d.max_new = g.max_new_tokens;
        d.rng = g.rng;
        d.seeds = g.seeds;
        d.steps = g.steps;
        d.row_ids = g.row_ids;
        d.uniforms = g.uniforms;
        d.active = g.active;
        d.finished = g.finished;
        d.tokens = g.tokens;
        d.processed = g.processed;
        d.processed_stride = g.processed_row_stride;
        d.probs = g.probs;
        d.probs_stride = g.probs_row_stride;
        const int mx = max_slice_elems(d.es);
        d.slices = (g.vocab + mx - 1) / mx;
        d.slice_len = (g.vocab + d.slices - 1) / d.slices;
        d.block_begin = blocks;
        d.row_begin = rows_total;
        rows_total += g.rows;
        if (rows_total > kMaxRows) return fail(MIS_E_UNSUPPORTED, "more than %d rows in one launch", kMaxRows);
        d.tiles = may_hold_nucleus(g) ? 1 : 0;
        d.ws_row_bytes = row_ws_bytes(d.slices, d.tiles != 0);
        d.ws = (char*)workspace + ws_off;
        d.counters = (unsigned int*)workspace;
        d.pending = (char*)workspace + kCounterBytes;
        d.gi = i;
        ws_off += (size_t)d.ws_row_bytes * (size_t)g.rows;
        const int64_t nb = (int64_t)g.rows * d.slices;
        if (nb + blocks > (int64_t)1 << 30) return fail(MIS_E_UNSUPPORTED, "too many rows");
        blocks += (int)nb;
    }
    if (ws_off > workspace_bytes || (ws_off > 0 && !workspace))
        return fail(MIS_E_WORKSPACE, "workspace too small: need %zu bytes, got %zu", ws_off, workspace_bytes);
    if (blocks == 0) return 0;
    // whole rows to XCDs: contiguous in (group, row) order, balanced by slice count
    int64_t count[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int64_t prefix = 0;
    for (int gi = 0; gi < n_groups; ++gi) {
        const int S = a.g[gi].slices;
        for (int r = 0; r < groups[gi].rows; ++r) {
            const int x = (int)std::min<int64_t>(7, ((prefix + S / 2) * 8) / blocks);
            if (a.seg_rows[x][gi] == 0) a.seg_row[x][gi] = r;
            ++a.seg_rows[x][gi];
            count[x] += S;
            prefix += S;
        }
    }
    a.per_xcd = (int)*std::max_element(count, count + 8);
    const int grid = a.per_xcd * 8;
    hipLaunchKernelGGL(sample_kernel, dim3(grid), dim3(kBlock), 0, (hipStream_t)stream, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(-1, "launch failed: %s", hipGetErrorString(e));
    return 0;
}

int mis_uniform(const int64_t* seeds, const int64_t* steps, const int64_t* row_ids, int64_t n, int32_t rng, float* out,
                void* stream) {
    g_err.clear();
    if (n < 0 || (n > 0 && !out)) return fail(MIS_E_ARG, "uniform: bad output");
    if (rng != MIS_RNG_COUNTER && rng != MIS_RNG_PHILOX) return fail(MIS_E_ARG, "unknown RNG mode: %d", rng);
    if (n == 0) return 0;
    const int threads = 256;
    const int64_t grid = (n + threads - 1) / threads;
    if (grid > INT32_MAX) return fail(MIS_E_UNSUPPORTED, "uniform: too many elements");
    hipLaunchKernelGGL(uniform_kernel, dim3((unsigned)grid), dim3(threads), 0, (hipStream_t)stream, seeds, steps, row_ids,
                       n, rng, out);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(-1, "launch failed: %s", hipGetErrorString(e));
    return 0;
}

}  // extern "C"
