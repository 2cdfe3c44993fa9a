// Fused token-sampling kernel for MI355X (gfx950) behind the C-ABI of include/mi355x_sampler.h.
//
// One launch handles every row of every group.  A row of V logits is cut into
// S vocabulary slices of at most ~10K elements, one 256-thread workgroup each.
// A slice workgroup
//   1. counts its history ids into an LDS table (u16 per slice token),
//   2. reads its slice once with 16-byte aligned vector loads, applies the
//      row's pipeline element by element (EOS censor, repetition / frequency /
//      presence penalties, allowed-token bitmask, temperature, in the order of
//      engine/talker_sampler.py:142-156) and keeps the values in registers,
//   3. publishes a summary (max, first argmax, sum of exp relative to its max)
//      and, for top-k rows, its candidates: every value >= tau, the c-th
//      largest of the per-thread maxima, in vocabulary order,
//   4. increments the row's arrival counter.  The last workgroup to arrive
//      finalises the row: it merges the summaries, selects the top-k and top-p
//      thresholds exactly (radix select over order-preserving float keys, by
//      count and by fixed-point probability mass), draws by inverse CDF in
//      vocabulary order and updates the decode state in place.
// The finaliser works on the candidates in LDS when they provably contain the
// top-k (every value >= max_s tau_s was published and at least k of them are
// >= it); otherwise (a slice overflowed, the nucleus is not bounded by a
// top-k, a full-vocabulary draw) it streams the row again slice by slice and
// runs the same selections over every element.  Workgroups never wait for
// one another: the only cross-workgroup protocol is release / arrive /
// acquire on the per-row counter, which the finaliser resets to zero for the
// next launch.

#include <hip/hip_runtime.h>

#include <climits>
#include <cstdarg>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <string>

#include "mi355x_sampler.h"

namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / 64;
constexpr int kNV = 40;            // register slots per thread in the slice phase
constexpr int kMaxGroups = 4;
constexpr int kMaxSlices = 64;
constexpr int kCapSlice = 512;     // candidates one slice may publish
constexpr int kCapRow = 4096;      // candidates the finaliser holds in LDS
constexpr int kCntWords = kBlock * kNV / 2;  // two u16 counts per word: covers every element of a slice
constexpr int kAlphaTable = 256;   // rep**n for n < 256 kept in LDS
constexpr int kMaxRows = 16384;    // rows per launch (arrival counters live in a fixed prefix of the workspace)
constexpr int64_t kCounterBytes = 4 * (int64_t)kMaxRows;
constexpr int64_t kPad = -1;
constexpr double kMassScale = 1099511627776.0;  // 2^40 fixed-point units of exp(x - max)

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
    int32_t row_begin;      // index of the group's first row among all rows of the launch
    char* ws;               // the group's row regions
    unsigned int* counters; // the launch's arrival counters (fixed workspace prefix, all zero between launches)
    int64_t ws_row_bytes;
};

struct KernelArgs {
    DevGroup g[kMaxGroups];
    int32_t n_groups;
    int32_t total_blocks;
    int32_t per_xcd;
    int32_t pad_;
};

struct SliceSummary {
    float m;          // max value of the slice (-inf if none finite)
    float g;          // the published candidates hold every value >= g (+inf: none published)
    double z;         // sum of exp(x - m) over the slice
    int32_t argmax;   // first index of m
    int32_t ncand;
    int32_t overflow;
    int32_t pad_;
};

struct Cand {
    float f;
    int32_t j;
};

struct Smem {
    union {
        uint32_t cnt[kCntWords];  // slice phase and streaming: history counts (u16 pairs)
        struct {
            float val[kCapRow];   // finaliser: candidate values, vocabulary order
            int32_t id[kCapRow];
        } cand;
    } u;
    float alpha[kAlphaTable];
    float tmax[kBlock];
    uint32_t hcnt[256];
    unsigned long long hmass[256];
    double red_d[kWaves];
    unsigned long long red_u[kWaves];
    float red_f[kWaves];
    int32_t red_i[kWaves];
    double tile_sum[kMaxSlices];
    SliceSummary summ[kMaxSlices];
    int32_t sel_bin;
    int32_t sel_rem;
    int32_t is_last;
    int32_t pad_;
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

// ---------------------------------------------------------------- block primitives (every thread calls them)

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

__device__ __forceinline__ float block_max(float x, Smem& sm) {
    for (int o = 32; o; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
    __syncthreads();
    if (lane_id() == 0) sm.red_f[wave_id()] = x;
    __syncthreads();
    float r = sm.red_f[0];
    for (int i = 1; i < kWaves; ++i) r = fmaxf(r, sm.red_f[i]);
    return r;
}

__device__ __forceinline__ int block_min_i(int x, Smem& sm) {
    for (int o = 32; o; o >>= 1) x = min(x, __shfl_xor(x, o));
    __syncthreads();
    if (lane_id() == 0) sm.red_i[wave_id()] = x;
    __syncthreads();
    int r = sm.red_i[0];
    for (int i = 1; i < kWaves; ++i) r = min(r, sm.red_i[i]);
    return r;
}

__device__ __forceinline__ int block_sum_i(int x, Smem& sm) {
    for (int o = 32; o; o >>= 1) x += __shfl_xor(x, o);
    __syncthreads();
    if (lane_id() == 0) sm.red_i[wave_id()] = x;
    __syncthreads();
    int r = 0;
    for (int i = 0; i < kWaves; ++i) r += sm.red_i[i];
    return r;
}

// Fixed reduction tree: the result does not depend on scheduling.
__device__ __forceinline__ double block_sum_d(double x, Smem& sm) {
    for (int o = 32; o; o >>= 1) x += __shfl_xor(x, o);
    __syncthreads();
    if (lane_id() == 0) sm.red_d[wave_id()] = x;
    __syncthreads();
    double r = 0.0;
    for (int i = 0; i < kWaves; ++i) r += sm.red_d[i];
    return r;
}

// Exclusive prefix from the lane-shifted inclusive scan (no subtraction).
__device__ __forceinline__ double block_excl_scan_d(double x, double& total, Smem& sm) {
    double incl = x;
    for (int o = 1; o < 64; o <<= 1) {
        const double y = __shfl_up(incl, o);
        if (lane_id() >= o) incl += y;
    }
    double excl = __shfl_up(incl, 1);
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

__device__ __forceinline__ int block_excl_scan_i(int x, int& total, Smem& sm) {
    int incl = x;
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o);
        if (lane_id() >= o) incl += y;
    }
    __syncthreads();
    if (lane_id() == 63) sm.red_i[wave_id()] = incl;
    __syncthreads();
    int off = 0;
    total = 0;
    for (int i = 0; i < kWaves; ++i) {
        if (i < wave_id()) off += sm.red_i[i];
        total += sm.red_i[i];
    }
    return off + incl - x;
}

// ---------------------------------------------------------------- per-row context

struct Ctx {
    int row, slice, S, V, slice_len;
    int64_t step;
    float tdiv;        // temperature divisor (1 for greedy rows)
    float top_p;
    float rep, pres, freq;
    int k_eff;
    int min_keep_eff;  // min(min_keep, k_eff)
    bool greedy, hf, later, censor, forced, live, want_out, p_active;
    bool counts;       // history penalties apply: build the count table
    bool cand_mode;    // slices publish candidates
    bool full_draw;    // no filter: every finite value survives
    int cand_target;   // per-slice candidate count target
};

__device__ __forceinline__ void init_ctx(const DevGroup& G, int row, int slice, Ctx& c) {
    c.row = row;
    c.slice = slice;
    c.S = G.slices;
    c.V = G.vocab;
    c.slice_len = G.slice_len;
    c.step = G.steps ? G.steps[row] : 0;
    const float t = G.temperature ? G.temperature[row] : G.t_val;
    c.greedy = !(t > 0.f);
    c.tdiv = c.greedy ? 1.0f : t;
    c.top_p = G.top_p ? G.top_p[row] : G.p_val;
    c.rep = G.repetition ? G.repetition[row] : G.rep_val;
    c.pres = G.presence ? G.presence[row] : G.pres_val;
    c.freq = G.frequency ? G.frequency[row] : G.freq_val;
    const int k = G.top_k ? G.top_k[row] : G.k_val;
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
    const bool act = G.active ? G.active[row] != 0 : true;
    const bool fin = G.finished ? G.finished[row] != 0 : false;
    c.live = act && !fin;
    c.want_out = G.processed != nullptr || G.probs != nullptr;
    const bool pen = G.hist_len > 0 && G.history != nullptr &&
                     (c.rep != 1.0f || c.pres != 0.0f || c.freq != 0.0f || G.alpha_lut != nullptr);
    c.counts = pen && (!c.hf || c.later);
    const bool filters = !c.greedy && (!c.hf || c.later);
    c.full_draw = !c.greedy && (!filters || (c.k_eff >= c.V && !c.p_active));
    const int per_slice = (5 * c.k_eff + 4 * c.S - 1) / (4 * c.S) + 8;  // 1.25 k / S + 8
    c.cand_target = min(per_slice, kBlock);
    c.cand_mode = filters && !c.full_draw && per_slice <= kBlock && c.k_eff <= kCapRow / 2;
}

// ---------------------------------------------------------------- the element pipeline

// rep**n beyond the LDS table: binary powering in double (<= 32 products, relative error < 4e-15),
// rounded once to float.
__device__ __noinline__ float alpha_slow(float rep, int n) {
    double r = 1.0, b = (double)rep;
    for (unsigned e = (unsigned)n; e; e >>= 1) {
        if (e & 1u) r *= b;
        b *= b;
    }
    return (float)r;
}

__device__ __forceinline__ float penalize(float x, int n, const Ctx& c, const Smem& sm) {
    const float a = n < kAlphaTable ? sm.alpha[n] : alpha_slow(c.rep, n);
    x = (x < 0.f) ? x * a : x / a;
    x = x - c.freq * (float)n;  // built with -ffp-contract=off: product and difference round separately
    return x - c.pres;
}

__device__ __forceinline__ float transform(float x, int j, int n, bool allowed, const DevGroup& G, const Ctx& c,
                                           const Smem& sm) {
    if (c.hf) {
        x = x / c.tdiv;
        if (n > 0) x = penalize(x, n, c, sm);
        if (!allowed) x = -INFINITY;
    } else {
        if (c.censor && j == G.eos) x = -INFINITY;
        if (n > 0) x = penalize(x, n, c, sm);
        if (!allowed) x = -INFINITY;
        x = x / c.tdiv;
    }
    return x;
}

// History counts of the slice [lo, hi) into sm.u.cnt (u16 pairs) and the alpha table.  History entries < 0
// (PAD) or >= V are empty slots.
__device__ __forceinline__ void build_counts(const DevGroup& G, const Ctx& c, int lo, int hi, Smem& sm) {
    __syncthreads();  // the union may still be read by a previous pass
    for (int w = threadIdx.x; w < kCntWords; w += kBlock) sm.u.cnt[w] = 0u;
    if (threadIdx.x < kAlphaTable) {
        const int n = threadIdx.x;
        sm.alpha[n] = (G.alpha_lut != nullptr && n < G.alpha_lut_len) ? G.alpha_lut[n]
                                                                         : (float)pow((double)c.rep, (double)n);
    }
    __syncthreads();
    const char* hrow = G.history + (int64_t)c.row * G.hist_stride * (G.hist_i64 ? 8 : 4);
    for (int i = threadIdx.x; i < G.hist_len; i += kBlock) {
        const int64_t h = G.hist_i64 ? ((const int64_t*)hrow)[i] : (int64_t)((const int32_t*)hrow)[i];
        if (h >= lo && h < hi) {
            const int s = (int)(h - lo);
            atomicAdd(&sm.u.cnt[s >> 1], 1u << (16 * (s & 1)));
        }
    }
    __syncthreads();
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
__device__ __forceinline__ Geo slice_geo(const DevGroup& G, const Ctx& c, int s) {
    Geo g;
    g.lo = s * c.slice_len;
    g.hi = min(c.V, g.lo + c.slice_len);
    const char* rowp = G.logits + (int64_t)c.row * G.row_stride * ES;
    const uintptr_t lo_addr = (uintptr_t)(rowp + (int64_t)g.lo * ES);
    g.base = lo_addr & ~(uintptr_t)15;
    g.first = g.lo - (int)((lo_addr - g.base) / ES);
    g.nchunk = (int)(((uintptr_t)(rowp + (int64_t)g.hi * ES) - g.base + 15) / 16);
    return g;
}

template <int ES>
__device__ __forceinline__ float raw_elem(const uint4& r, int e) {
    const uint32_t w = (e >> (ES == 2 ? 1 : 0)) == 0 ? r.x : (e >> (ES == 2 ? 1 : 0)) == 1 ? r.y
                       : (e >> (ES == 2 ? 1 : 0)) == 2 ? r.z : r.w;
    if (ES == 2) return __uint_as_float((e & 1) ? (w & 0xffff0000u) : (w << 16));
    return __uint_as_float(w);
}

// Processed value of element j (in [lo, hi)) from its raw logit.
__device__ __forceinline__ float element(const DevGroup& G, const Ctx& c, const Smem& sm, const uint32_t* mrow, int lo,
                                         int j, float x) {
    const int n = c.counts ? count_of(sm, j - lo) : 0;
    const bool allowed = mrow ? ((mrow[j >> 5] >> (j & 31)) & 1u) != 0u : true;
    return transform(x, j, n, allowed, G, c, sm);
}

// ---------------------------------------------------------------- slice phase: the slice in registers

struct Tile {
    float v[kNV];
    unsigned long long valid;
};

template <int ES>
__device__ __forceinline__ void load_tile(const DevGroup& G, const Ctx& c, const Geo& g, Tile& T, const Smem& sm) {
    constexpr int E = 16 / ES;
    constexpr int NCH = kNV / E;
    const uint32_t* mrow = G.allowed ? G.allowed + (int64_t)c.row * G.allowed_stride : nullptr;
    T.valid = 0ull;
    uint4 raw[NCH];
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        const int ch = threadIdx.x + kBlock * i;
        raw[i] = ch < g.nchunk ? *(const uint4*)(g.base + (uintptr_t)ch * 16) : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        const int ch = threadIdx.x + kBlock * i;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int q = i * E + e;
            const int j = g.first + ch * E + e;
            const bool in = ch < g.nchunk && j >= g.lo && j < g.hi;
            T.v[q] = in ? element(G, c, sm, mrow, g.lo, j, raw_elem<ES>(raw[i], e)) : -INFINITY;
            if (in) T.valid |= 1ull << q;
        }
    }
}

template <int ES>
__device__ __forceinline__ int tile_index(const Geo& g, int q) {
    constexpr int E = 16 / ES;
    return g.first + (int)(threadIdx.x + kBlock * (q / E)) * E + (q % E);
}

// ---------------------------------------------------------------- finaliser sources

// The elements the finaliser selects from: the LDS candidates (n of them, vocabulary order) or the whole row,
// streamed slice by slice from global memory.
struct Src {
    bool cand;
    int n;
};

// Streams slice s: fn(f, j, round, e) for every element, chunk ch = round * kBlock + thread.  Every thread runs
// the same number of rounds (so fn may not synchronise, but callers may between slices).
template <int ES, class F>
__device__ __forceinline__ void stream_slice(const DevGroup& G, const Ctx& c, int s, Smem& sm, F&& fn) {
    constexpr int E = 16 / ES;
    const Geo g = slice_geo<ES>(G, c, s);
    if (c.counts) build_counts(G, c, g.lo, g.hi, sm);
    const uint32_t* mrow = G.allowed ? G.allowed + (int64_t)c.row * G.allowed_stride : nullptr;
    for (int ch = threadIdx.x; ch < g.nchunk; ch += kBlock) {
        const uint4 raw = *(const uint4*)(g.base + (uintptr_t)ch * 16);
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int j = g.first + ch * E + e;
            if (j >= g.lo && j < g.hi) fn(element(G, c, sm, mrow, g.lo, j, raw_elem<ES>(raw, e)), j);
        }
    }
}

template <int ES, class F>
__device__ __forceinline__ void visit(const DevGroup& G, const Ctx& c, Smem& sm, const Src& src, F&& fn) {
    if (src.cand) {
        for (int p = threadIdx.x; p < src.n; p += kBlock) fn(sm.u.cand.val[p], sm.u.cand.id[p]);
    } else {
        for (int s = 0; s < c.S; ++s) stream_slice<ES>(G, c, s, sm, fn);
    }
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
        int incl = sum;
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(incl, o);
            if (l >= o) incl += y;
        }
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

// k-th largest finite value of the source; -inf when it holds fewer than k finite values.
template <int ES>
__device__ __forceinline__ float select_kth(const DevGroup& G, const Ctx& c, Smem& sm, const Src& src, int k) {
    uint32_t prefix = 0u, pmask = 0u;
    int rem = k;
    for (int shift = 24; shift >= 0; shift -= 8) {
        __syncthreads();
        for (int b = threadIdx.x; b < 256; b += kBlock) sm.hcnt[b] = 0u;
        if (threadIdx.x == 0) sm.sel_bin = -1;
        __syncthreads();
        visit<ES>(G, c, sm, src, [&](float f, int) {
            if (finite_f(f)) {
                const uint32_t key = ord_key(f);
                if ((key & pmask) == prefix) atomicAdd(&sm.hcnt[(key >> shift) & 255u], 1u);
            }
        });
        __syncthreads();
        pick_count_bin(rem, sm);
        __syncthreads();
        const int bin = sm.sel_bin;
        if (bin < 0) return -INFINITY;  // fewer than k finite values (first round only)
        rem = sm.sel_rem;
        prefix |= (uint32_t)bin << shift;
        pmask |= 255u << shift;
    }
    return key_float(prefix);
}

__device__ __forceinline__ unsigned long long mass_q(float f, float m) {
    return (unsigned long long)((double)expf(f - m) * kMassScale);
}

// Smallest value v >= lower of the source with  sum{ q(x) : x > v, x >= lower } < target,  q = fixed-point
// exp(x - m); +inf when no value qualifies (target <= 0).
template <int ES>
__device__ __forceinline__ float select_mass(const DevGroup& G, const Ctx& c, Smem& sm, const Src& src, float lower,
                                             float m, double target) {
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
        visit<ES>(G, c, sm, src, [&](float f, int) {
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
            unsigned long long incl = sum;
            for (int o = 1; o < 64; o <<= 1) {
                const unsigned long long y = __shfl_up(incl, o);
                if (l >= o) incl += y;
            }
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
            for (int o = 32; o; o >>= 1) lowest = min(lowest, __shfl_xor(lowest, o));
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

// The draw of engine/talker_sampler.py:168-172 over the survivors (finite values >= thr, minus the EOS id when
// drop_eos): probabilities p = exp(x - m) * (1 / sum), their running sum in vocabulary order, the first survivor
// whose running sum (rounded to float) exceeds u * total, or V - 1 when none does.
template <int ES>
__device__ __forceinline__ int draw_token(const DevGroup& G, const Ctx& c, Smem& sm, const Src& src, float thr,
                                          float m, bool drop_eos, float u) {
    auto survives = [&](float f, int j) { return finite_f(f) && f >= thr && !(drop_eos && j == G.eos); };
    double zpart = 0.0;
    visit<ES>(G, c, sm, src, [&](float f, int j) {
        if (survives(f, j)) zpart += (double)expf(f - m);
    });
    const double zs = block_sum_d(zpart, sm);
    const float inv = 1.0f / (float)zs;
    const int ntiles = src.cand ? 1 : c.S;
    double total = 0.0;
    if (src.cand) {
        double part = 0.0;
        visit<ES>(G, c, sm, src, [&](float f, int j) {
            if (survives(f, j)) part += (double)(expf(f - m) * inv);
        });
        total = block_sum_d(part, sm);
        if (threadIdx.x == 0) sm.tile_sum[0] = total;
    } else {
        for (int s = 0; s < c.S; ++s) {
            double part = 0.0;
            stream_slice<ES>(G, c, s, sm, [&](float f, int j) {
                if (survives(f, j)) part += (double)(expf(f - m) * inv);
            });
            const double ts = block_sum_d(part, sm);
            if (threadIdx.x == 0) sm.tile_sum[s] = ts;
            total += ts;
        }
    }
    __syncthreads();
    const float target = u * (float)total;
    double base = 0.0;
    for (int s = 0; s < ntiles; ++s) {
        const double ts = sm.tile_sum[s];
        if (!((float)(base + ts) > target)) {
            base += ts;
            continue;
        }
        int found = INT_MAX;
        if (src.cand) {
            // vocabulary order = candidate order; rounds of kBlock consecutive candidates
            double run_base = base;
            for (int r0 = 0; r0 < src.n; r0 += kBlock) {
                const int p = r0 + threadIdx.x;
                const bool ok = p < src.n && survives(sm.u.cand.val[p], sm.u.cand.id[p]);
                const double x = ok ? (double)(expf(sm.u.cand.val[p] - m) * inv) : 0.0;
                double tot;
                const double run = run_base + block_excl_scan_d(x, tot, sm) + x;
                if (ok && (float)run > target) found = min(found, sm.u.cand.id[p]);
                run_base += tot;
                if (block_min_i(found, sm) != INT_MAX) break;
            }
        } else {
            constexpr int E = 16 / ES;
            const Geo g = slice_geo<ES>(G, c, s);
            if (c.counts) build_counts(G, c, g.lo, g.hi, sm);
            const uint32_t* mrow = G.allowed ? G.allowed + (int64_t)c.row * G.allowed_stride : nullptr;
            double run_base = base;
            for (int r0 = 0; r0 < g.nchunk; r0 += kBlock) {
                const int ch = r0 + threadIdx.x;
                float pv[E];
                int jv[E];
                double mine = 0.0;
                if (ch < g.nchunk) {
                    const uint4 raw = *(const uint4*)(g.base + (uintptr_t)ch * 16);
#pragma unroll
                    for (int e = 0; e < E; ++e) {
                        const int j = g.first + ch * E + e;
                        jv[e] = j;
                        pv[e] = 0.0f;
                        if (j >= g.lo && j < g.hi) {
                            const float f = element(G, c, sm, mrow, g.lo, j, raw_elem<ES>(raw, e));
                            if (survives(f, j)) pv[e] = expf(f - m) * inv;
                        }
                        mine += (double)pv[e];
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < E; ++e) {
                        pv[e] = 0.0f;
                        jv[e] = 0;
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
    if (G.uniforms) return G.uniforms[c.row];
    const int64_t seed = G.seeds ? G.seeds[c.row] : 0;
    if (G.rng == MIS_RNG_PHILOX) return philox_uniform(seed, c.step, G.row_ids ? G.row_ids[c.row] : 0);
    return counter_uniform(seed, c.step);
}

// ---------------------------------------------------------------- outputs and state

// Processed logits (-inf where filtered) and softmax probabilities of the whole row (parity outputs).
template <int ES>
__device__ __forceinline__ void write_outputs(const DevGroup& G, const Ctx& c, Smem& sm, float thr, float m,
                                              bool drop_eos) {
    float* prow = G.processed ? G.processed + (int64_t)c.row * G.processed_stride : nullptr;
    float* qrow = G.probs ? G.probs + (int64_t)c.row * G.probs_stride : nullptr;
    if (c.forced) {
        for (int j = threadIdx.x; j < c.V; j += kBlock) {
            const bool e = j == G.eos;
            if (prow) prow[j] = e ? 0.0f : -INFINITY;
            if (qrow) qrow[j] = e ? 1.0f : 0.0f;
        }
        return;
    }
    const Src src{false, 0};
    auto keep = [&](float f, int j) { return f >= thr && !(drop_eos && j == G.eos); };
    double zpart = 0.0;
    if (qrow)
        visit<ES>(G, c, sm, src, [&](float f, int j) {
            if (finite_f(f) && keep(f, j)) zpart += (double)expf(f - m);
        });
    const double zs = block_sum_d(zpart, sm);
    const float inv = 1.0f / (float)zs;
    visit<ES>(G, c, sm, src, [&](float f, int j) {
        const bool k = keep(f, j);
        if (prow) prow[j] = k ? f : -INFINITY;
        if (qrow) qrow[j] = !(m > -INFINITY) ? NAN : (k && finite_f(f)) ? expf(f - m) * inv : 0.0f;
    });
}

// tokens[row]; for live rows with MIS_UPDATE_STATE: history append, steps + 1, finished |= (token == eos).
__device__ __forceinline__ void update_state(const DevGroup& G, const Ctx& c, int64_t tok) {
    if (!(G.flags & MIS_UPDATE_STATE) || !c.live) {
        if (threadIdx.x == 0 && G.tokens) G.tokens[c.row] = c.live ? tok : kPad;
        return;
    }
    if (G.history && G.hist_len > 0) {
        const int W = G.hist_len;
        char* hrow = (char*)G.history + (int64_t)c.row * G.hist_stride * (G.hist_i64 ? 8 : 4);
        if (G.hist_mode == MIS_HISTORY_RING) {
            if (threadIdx.x == 0) {
                const int pos = (int)((G.hist_head[c.row] % W + W) % W);
                if (G.hist_i64)
                    ((int64_t*)hrow)[pos] = tok;
                else
                    ((int32_t*)hrow)[pos] = (int32_t)tok;
                G.hist_head[c.row] = (pos + 1) % W;
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
        if (G.tokens) G.tokens[c.row] = tok;
        if (G.steps) G.steps[c.row] = c.step + 1;
        if (G.finished && tok == (int64_t)G.eos) G.finished[c.row] = 1;
    }
}

// ---------------------------------------------------------------- finaliser

template <int ES>
__device__ __forceinline__ void finalize(const DevGroup& G, const Ctx& c, Smem& sm, char* rws) {
    if ((int)threadIdx.x < c.S) sm.summ[threadIdx.x] = ((const SliceSummary*)rws)[threadIdx.x];
    __syncthreads();
    float m = -INFINITY, gmax = -INFINITY;
    double z = 0.0;
    int am = INT_MAX, ntot = 0;
    bool overflow = false;
    for (int s = 0; s < c.S; ++s) m = fmaxf(m, sm.summ[s].m);
    for (int s = 0; s < c.S; ++s) {
        const SliceSummary q = sm.summ[s];
        if (q.m == m && q.argmax < am) am = q.argmax;
        if (q.m > -INFINITY) z += q.z * exp((double)q.m - (double)m);
        gmax = fmaxf(gmax, q.g);
        ntot += q.ncand;
        overflow |= q.overflow != 0;
    }
    const bool drop_eos = c.hf && c.censor;
    int64_t tok;
    float thr = -INFINITY;
    if (c.greedy) {
        tok = am == INT_MAX ? c.V - 1 : am;
    } else if (!(m > -INFINITY)) {
        tok = c.V - 1;  // nothing allowed: the reference's clamp value
    } else {
        Src src{false, 0};
        if (!c.full_draw) {
            if (c.cand_mode && !overflow && ntot <= kCapRow) {
                // candidates of all slices, in slice (= vocabulary) order
                const Cand* cands = (const Cand*)(rws + sizeof(SliceSummary) * c.S);
                int off = 0;
                for (int s = 0; s < c.S; ++s) {
                    const int n = sm.summ[s].ncand;
                    for (int p = threadIdx.x; p < n; p += kBlock) {
                        const Cand cd = cands[(int64_t)s * kCapSlice + p];
                        sm.u.cand.val[off + p] = cd.f;
                        sm.u.cand.id[off + p] = cd.j;
                    }
                    off += n;
                }
                __syncthreads();
                // every value >= gmax was published: the k-th largest is proven once k of them are >= gmax
                int nge = 0;
                for (int p = threadIdx.x; p < ntot; p += kBlock) nge += sm.u.cand.val[p] >= gmax ? 1 : 0;
                nge = block_sum_i(nge, sm);
                if (nge >= c.k_eff || gmax == -INFINITY) src = Src{true, ntot};
            }
            const float thr_k = select_kth<ES>(G, c, sm, src, c.k_eff);
            thr = thr_k;
            if (c.p_active) {
                double zp;
                if (c.hf) {
                    zp = z;  // full-vocabulary normaliser (engine/talker_sampler.py:112)
                } else {
                    // softmax over the top-k values (:129): those above thr_k plus (k - n_gt) copies of thr_k
                    double part = 0.0;
                    int ngt = 0;
                    visit<ES>(G, c, sm, src, [&](float f, int) {
                        if (finite_f(f) && f > thr_k) {
                            part += (double)expf(f - m);
                            ++ngt;
                        }
                    });
                    zp = block_sum_d(part, sm);
                    ngt = block_sum_i(ngt, sm);
                    if (thr_k > -INFINITY) zp += (double)(c.k_eff - ngt) * (double)expf(thr_k - m);
                }
                const double target = (double)c.top_p * zp * kMassScale;
                const float thr_p = select_mass<ES>(G, c, sm, src, thr_k, m, target);
                const float v_m = c.min_keep_eff <= 1 ? m : select_kth<ES>(G, c, sm, src, c.min_keep_eff);
                thr = fmaxf(fminf(thr_p, v_m), thr_k);
            }
        }
        const bool need_tok = G.tokens != nullptr || (G.flags & MIS_UPDATE_STATE);
        tok = need_tok ? draw_token<ES>(G, c, sm, src, thr, m, drop_eos, row_uniform(G, c)) : kPad;
    }
    if (c.want_out) write_outputs<ES>(G, c, sm, thr, m, drop_eos);
    update_state(G, c, tok);
}

// ---------------------------------------------------------------- the row

template <int ES>
__device__ __forceinline__ void run_row(const DevGroup& G, const int row, const int slice, Smem& sm) {
    Ctx c;
    init_ctx(G, row, slice, c);
    char* rws = G.ws + (int64_t)row * G.ws_row_bytes;
    if (!c.live && !c.want_out) {
        if (slice == 0 && threadIdx.x == 0 && G.tokens) G.tokens[row] = kPad;
        return;
    }
    if (c.forced) {
        if (slice != 0) return;
        if (c.want_out) write_outputs<ES>(G, c, sm, -INFINITY, 0.0f, false);
        update_state(G, c, G.eos);
        return;
    }
    const Geo geo = slice_geo<ES>(G, c, slice);
    if (c.counts) build_counts(G, c, geo.lo, geo.hi, sm);
    Tile T;
    load_tile<ES>(G, c, geo, T, sm);
    float tm = -INFINITY;
#pragma unroll
    for (int q = 0; q < kNV; ++q)
        if ((T.valid >> q) & 1ull) tm = fmaxf(tm, T.v[q]);
    const float m = block_max(tm, sm);
    int first = INT_MAX;
    if (c.greedy) {
#pragma unroll
        for (int q = 0; q < kNV; ++q)
            if (((T.valid >> q) & 1ull) && T.v[q] == m && first == INT_MAX) first = tile_index<ES>(geo, q);
    }
    const int am = block_min_i(first, sm);
    double z = 0.0;
    if (!c.greedy && m > -INFINITY) {
        double part = 0.0;
#pragma unroll
        for (int q = 0; q < kNV; ++q)
            if ((T.valid >> q) & 1ull) part += (double)expf(T.v[q] - m);
        z = block_sum_d(part, sm);
    }
    Cand* cands = (Cand*)(rws + sizeof(SliceSummary) * c.S) + (int64_t)slice * kCapSlice;
    int ncand = 0, overflow = 0;
    float g = INFINITY;
    if (c.cand_mode) {
        // tau = the cand_target-th largest per-thread maximum: at least cand_target values are >= tau
        sm.tmax[threadIdx.x] = tm;
        __syncthreads();
        int rank = 0;
        for (int u = 0; u < kBlock; ++u) {
            const float o = sm.tmax[u];
            rank += (o > tm) || (o == tm && u < (int)threadIdx.x);
        }
        if (rank == c.cand_target - 1) sm.sel_tau = tm;
        __syncthreads();
        const float tau = sm.sel_tau;
        g = tau;
        // ordered compaction: round i, thread, element = vocabulary order
        constexpr int E = 16 / ES;
        constexpr int NCH = kNV / E;
        int run = 0;
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            int mine = 0;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const int q = i * E + e;
                if (((T.valid >> q) & 1ull) && finite_f(T.v[q]) && T.v[q] >= tau) ++mine;
            }
            int tot;
            int pos = run + block_excl_scan_i(mine, tot, sm);
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const int q = i * E + e;
                if (((T.valid >> q) & 1ull) && finite_f(T.v[q]) && T.v[q] >= tau) {
                    if (pos < kCapSlice) cands[pos] = Cand{T.v[q], tile_index<ES>(geo, q)};
                    ++pos;
                }
            }
            run += tot;
        }
        ncand = min(run, kCapSlice);
        overflow = run > kCapSlice;
    }
    if (threadIdx.x == 0) {
        SliceSummary* summ = (SliceSummary*)rws + slice;
        summ->m = m;
        summ->g = g;
        summ->z = z;
        summ->argmax = am;
        summ->ncand = ncand;
        summ->overflow = overflow;
    }
    if (c.S > 1) {
        __threadfence();  // release this slice's summary and candidates
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned int* counter = G.counters + G.row_begin + row;
            const unsigned int old = atomicAdd(counter, 1u);
            const int last = old == (unsigned int)(c.S - 1);
            if (last) *counter = 0u;  // every slice has arrived: reset for the next launch
            sm.is_last = last;
        }
        __syncthreads();
        if (!sm.is_last) return;
        __threadfence();  // acquire the other slices' writes
    } else {
        __syncthreads();
    }
    finalize<ES>(G, c, sm, rws);
}

__global__ __launch_bounds__(kBlock) void sample_kernel(const KernelArgs args) {
    __shared__ Smem sm;
    const int bid = blockIdx.x;
    const int w = (bid % 8) * args.per_xcd + bid / 8;  // consecutive work items (a row's slices) share an XCD
    if (w >= args.total_blocks) return;
    int gi = 0;
    while (gi + 1 < args.n_groups && w >= args.g[gi + 1].block_begin) ++gi;
    const DevGroup& G = args.g[gi];
    const int local = w - G.block_begin;
    const int row = local / G.slices, slice = local % G.slices;
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

// Workspace: [arrival counters, kCounterBytes][per group: rows x (S summaries, S x kCapSlice candidates)].
int64_t row_ws_bytes(int slices) {
    const int64_t b = (int64_t)sizeof(SliceSummary) * slices + (int64_t)sizeof(Cand) * kCapSlice * slices;
    return (b + 255) & ~(int64_t)255;
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
    size_t total = (size_t)kCounterBytes;
    for (int i = 0; i < n_groups; ++i) {
        if (check_group(groups[i], i)) return 0;
        const int es = groups[i].dtype == MIS_BF16 ? 2 : 4;
        const int s = (groups[i].vocab + max_slice_elems(es) - 1) / max_slice_elems(es);
        total += (size_t)row_ws_bytes(s) * (size_t)groups[i].rows;
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
    size_t ws_off = (size_t)kCounterBytes;
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
        d.ws_row_bytes = row_ws_bytes(d.slices);
        d.ws = (char*)workspace + ws_off;
        d.counters = (unsigned int*)workspace;
        ws_off += (size_t)d.ws_row_bytes * (size_t)g.rows;
        const int64_t nb = (int64_t)g.rows * d.slices;
        if (nb + blocks > (int64_t)1 << 30) return fail(MIS_E_UNSUPPORTED, "too many rows");
        blocks += (int)nb;
    }
    if (ws_off > workspace_bytes || (ws_off > 0 && !workspace))
        return fail(MIS_E_WORKSPACE, "workspace too small: need %zu bytes, got %zu", ws_off, workspace_bytes);
    if (blocks == 0) return 0;
    a.total_blocks = blocks;
    a.per_xcd = (blocks + 7) / 8;
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
