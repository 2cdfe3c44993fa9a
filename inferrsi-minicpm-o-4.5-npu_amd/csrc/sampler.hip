// Fused token sampling for MI355X (gfx950) behind the C-ABI of include/mi355x_sampler.h.
//
// One launch samples every row of up to four row groups.  A row of V logits is cut into S vocabulary slices;
// one 1024-thread workgroup holds a slice in registers (at most 40 elements per thread, one workgroup per CU) and
// every slice of a row runs on one XCD, so the slices of a row share an L2.
//
// Per slice (engine/talker_sampler.py:136-172 and the per-row extensions):
//   * the history ids that fall in the slice are counted in LDS; those elements, and a censored EOS, become
//     "specials" whose processed value is computed element by element (penalties, mask, temperature in the
//     reference's order); every other element needs only the bitmask and the temperature, which preserves order,
//     so bf16 slices keep the raw logits and divide only the values they publish;
//   * by row kind the slice publishes: its first argmax (greedy rows); every element at or above a gate chosen so
//     that the slice's own top elements are all published (top-k and top-p rows), with the sum of exp over the
//     slice when the normaliser is the whole vocabulary; per-sub-block sums of exp (unfiltered rows);
//   * then it counts itself in on the row's arrival word.  The last slice to arrive finalises the row: greedy
//     rows take the first argmax; filtered rows select the k-th value and the top-p cut over the published
//     candidates (radix selection with fixed-point masses, so the result does not depend on scheduling) and draw
//     by inverse CDF in vocabulary order; unfiltered rows walk the sub-block sums and rescan one sub-block.
//   * A row the candidates cannot settle exactly (a nucleus wider than the candidates, top values packed into one
//     slice, a slice that ran on another XCD) is finalised by streaming the row again: the same selection, over
//     every element.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdarg>
#include <mutex>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <string>

#include "elem.h"
#include "mi355x_sampler.h"
#include "primitives.h"

namespace mis {
namespace {

// Phase timestamps (the 100 MHz real-time counter, thread 0 of each workgroup), for profiling the slice and
// finaliser phases; compiled in with -DMIS_PHASE_STAMPS only.
#ifdef MIS_PHASE_STAMPS
constexpr int kStampSlots = 32;
constexpr int kStampBlocks = 8192;
__device__ unsigned long long mis_stamps[kStampBlocks * kStampSlots];
#define MIS_STAMP(i)                                                                                         \
    do {                                                                                                     \
        if (threadIdx.x == 0 && blockIdx.x < kStampBlocks)                                                   \
            mis_stamps[blockIdx.x * kStampSlots + (i)] = __builtin_amdgcn_s_memrealtime();                   \
    } while (0)
#define MIS_STAMP_INFO(v)                                                                                    \
    do {                                                                                                     \
        if (threadIdx.x == 0 && blockIdx.x < kStampBlocks) mis_stamps[blockIdx.x * kStampSlots + 31] = (v); \
    } while (0)
#else
#define MIS_STAMP(i) ((void)0)
#define MIS_STAMP_INFO(v) ((void)0)
#endif

constexpr int kMaxGroups = 4;
constexpr int kMaxSlices = 64;
constexpr int kMaxRows = 16384;
constexpr int kMaxVocab = 1 << 21;               // token ids fit the 21-bit keys of the draw
constexpr int kRounds = 5;                       // 16-byte chunks per thread of a slice, at most
constexpr int kTileElems = 40;                   // elements per thread of a slice, at most (bf16; fp32: 20)
constexpr int kTileMax = kThreads * kTileElems;  // 40,960
constexpr int kCntWords = kTileMax / 2;          // history counts, u16 pairs
constexpr int kKeepWords = kTileMax / 32 + 3;    // keep bits of a slice (allowed, in range, not special)
constexpr int kSpecCap = 2048;                   // specials of one slice
constexpr int kCapWave = 512;                    // candidates one wave of a slice may publish
constexpr int kCapSpecSeg = 512;                 // candidates among a slice's specials
constexpr int kSegs = kWaves + 1;                // candidate segments of a slice: 16 waves + the specials
constexpr int kCapRow = 12288;                   // entries of the histogram path's weighted list
constexpr int kCapCand = 6144;                   // candidates a finaliser gathers (with their masses)
constexpr int kBins = 2048;                      // radix digit: 11 bits
constexpr int kMaxSB = kWaves * kRounds;         // (wave, round) sub-blocks of a slice
constexpr double kFx = 4398046511104.0;          // 2^42 fixed-point units of exp(q - max): V * 2^42 < 2^64
constexpr int kLineBytes = 128;                  // a row's arrival word has a cache line of its own
constexpr int64_t kHeaderBytes = 256;            // diagnostic counters (MIS_WS_PATH_OFFSET)
static_assert(MIS_WS_PATH_OFFSET + 4 * MIS_PATH_COUNT <= kHeaderBytes && MIS_WS_ERROR_OFFSET + 4 <= kHeaderBytes &&
                  MIS_WS_PATH_OFFSET + 4 * MIS_PATH_COUNT <= MIS_WS_ERROR_OFFSET,
              "workspace header");
// Arrival words live at fixed offsets (they must read zero at every launch, whatever the previous launch's shape).
constexpr int64_t kArriveBytes = (int64_t)kMaxRows * kLineBytes;
constexpr int kPad = -1;

enum Mode : int { kSkip = 0, kForced, kGreedy, kTopK, kNucleus, kFull, kStream };
enum EosRule : int { kEosNormal = 0, kEosExcluded, kEosSelOnly };
enum : int32_t { kRecOverflow = 1, kRecGateInf = 2 };
constexpr uint32_t kSelOnlyBit = 0x80000000u;  // candidate id flag: EOS that ranks but is not drawn
constexpr int kBufferWord3 = 0x00020000;       // raw buffer descriptor, word 3 (gfx9 family: 32-bit data format)

struct DevGroup {
    const char* logits;
    int64_t row_stride;
    int32_t es, vocab, rows, semantics, flags, min_keep;
    const float* temperature;
    const int32_t* top_k;
    const float* top_p;
    const float* repetition;
    const float* presence;
    const float* frequency;
    float t_val, p_val, rep_val, pres_val, freq_val;
    int32_t k_val;
    int64_t zero64;   // 0: what a missing steps / finished array reads as
    uint32_t one32;   // 1: what a missing active array reads as
    const float* alpha_lut;
    int32_t alpha_lut_len;
    int32_t hist_len;
    const char* history;
    int64_t hist_stride;
    int32_t hist_i64, hist_mode;
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
    // derived on the host
    int32_t S;          // slices per row
    int32_t R;          // 16-byte chunks per thread in a slice
    int32_t slice_len;  // elements per slice (the last one may be shorter)
    int32_t row_begin;  // index of the group's first row among the launch's rows
    char* recs;         // slice records: [rows][S] x kRecBytes
    uint32_t* paths;    // rows finalised per path (MIS_PATH_*), diagnostics
};

// Whole rows are assigned to XCDs: block b runs on XCD b % 8 (the dispatcher's round-robin) as the (b / 8)-th
// slice of that XCD's rows, which are rows [seg_row[x][g], + seg_rows[x][g]) of each group g in turn.
struct KernelArgs {
    DevGroup g[kMaxGroups];
    int32_t n_groups;
    int32_t seg_row[8][kMaxGroups];
    int32_t seg_rows[8][kMaxGroups];
    char* arrive;  // per launch row: a 64-bit arrival word, kLineBytes apart
};

// What a slice publishes for its row's finaliser.
struct SliceRec {
    float mq;        // max processed value of the slice (-inf if none)
    float mqd;       // max over the elements that can be drawn
    float gate;      // every element >= gate is among the slice's candidates (filtered rows)
    float mref;      // reference of z and of the sub-block sums
    int32_t argmax;  // first index of mqd (greedy rows)
    int32_t flags;   // kRec*
    int32_t hist;    // 1: the nucleus histogram and the specials list are published
    int32_t nspec;   // specials published
    double z;        // sum of exp(q - mref) (whole-vocabulary normaliser)
    double zc;       // the part of z over the published candidates
    int32_t ncand[kSegs];
    int32_t nhigh;   // histogram path: the first nhigh published specials lie at or above the value gate
    unsigned long long tinyfx;  // sum of exp(q) in fixed point over the tiny-magnitude lumps of the histogram
    unsigned long long zsurv;   // histogram path: the slice's survivor mass for the draw (after the cut)
};
constexpr int64_t kRecHead = 256;
static_assert(sizeof(SliceRec) <= kRecHead, "slice record");
constexpr int64_t kRecSbOff = kRecHead;
constexpr int64_t kRecCandOff = kRecSbOff + 8 * kMaxSB;
// Nucleus histogram of a bf16 slice: one key per bf16 value with |x| in [2^-7, 2^8) (1,920 per sign), zero, the
// tiny magnitudes of each sign (lumps) and the huge ones (lumps); keys increase with the value.
constexpr int kKeys = 3845;
constexpr int kKeyZero = 1922;
constexpr uint32_t kBfLo = 0x3C00u;  // 2^-7
constexpr uint32_t kBfHi = 0x4380u;  // 2^8
constexpr int kHistWords = (kKeys + 1) / 2;  // published as u16 pairs
constexpr int kHistReps = 4;                 // copies of a slice's counts while it builds them
constexpr int kHistStride = 3848;            // words per copy: kKeys + 1 rounded up to 8 (copies 8 banks apart)
static_assert(kHistReps * kHistStride <= kCntWords && kHistStride >= 2 * kHistWords, "histogram copies");
constexpr int64_t kRecHistOff = kRecCandOff + 8 * (kWaves * kCapWave + kCapSpecSeg);
constexpr int64_t kRecSpecOff = kRecHistOff + 4 * ((kHistWords + 63) / 64 * 64);
constexpr int64_t kRecSpecBinOff = kRecSpecOff + 8 * kSpecCap;  // the specials' histogram bins + 1 (u32)
constexpr int64_t kRecBytes = kRecSpecBinOff + 4 * kSpecCap;
constexpr float kHistMinT = 0.015625f;  // the histogram path serves temperatures >= 2^-6 (lumps stay near 0)

struct Special {
    int32_t j;    // token id
    int32_t n;    // history count
    float q;      // processed value
    int32_t sel;  // 1: ranks but is not drawn (censored EOS in the HF order)
};

struct Hist {
    unsigned long long w[kBins];
    unsigned long long scan[kWaves];
    int32_t sel;
    unsigned long long before;
};

constexpr int kSelBins = kBins;  // value bins of the candidate finaliser (their masses live in Hist::w)
constexpr int kSelCap = 1024;    // elements of one bin ranked exactly; specials of a row drawn from

// Candidate finaliser: bin counts, one bin ranked (compacted, then sorted), the specials in id order.
struct SelScratch {
    uint32_t bcnt[kSelBins];
    float cq[kSelCap];
    unsigned long long cw[kSelCap];
    float sq[kSelCap];
    unsigned long long sw[kSelCap];
};

// LDS of one workgroup.  The slice phase and the finaliser overlay the big arrays.
struct Lds {
    union {
        uint32_t cnt[kCntWords];  // slice phase / streaming: history counts by position (u16 pairs)
        struct {
            float q[kCapRow];
            uint32_t id[kCapRow];  // multiplicity (weighted lists)
        } c;                       // finaliser: histogram path, streaming
        struct {
            float q[kCapCand];
            uint32_t id[kCapCand];
            unsigned long long mass[kCapCand];  // efx(q, row max)
        } w;                       // finaliser: gathered candidates
    } a;
    Hist h;
    uint32_t keep[kKeepWords];
    union {
        Special spec[kSpecCap];  // slice phase
        SelScratch ss;           // finaliser: the candidate selection
    };
    double sb[kMaxSB];
    unsigned long long sbfx[kMaxSB];
    int32_t segoff[kMaxSlices * kSegs + 1];
    alignas(16) uint32_t gh[256];  // slice phase: histogram of the lane maxima (the gate)
    Red red;
    int32_t nspec;
    int32_t scnt;
    int32_t flags;
    int32_t is_last;
    int32_t nhi, nlo;  // slice phase of the histogram path: specials at or above the value gate, and below it
    int32_t foreign;
    int32_t token;
    float fscratch[4];
    double dscratch[4];
    unsigned long long tinyfx;               // slice phase: the histogram's tiny lumps
    unsigned long long uscratch[2];
    unsigned long long slice_u[kMaxSlices];  // finaliser: per-slice sums
    int32_t qbin[4];                         // candidate finaliser: the bin of each question (-1: none)
    unsigned long long qbefore[4];           // ... and the weight of the bins above it
    int32_t slice_n[kMaxSlices];             // finaliser (histogram path): specials each slice published
};
static_assert(sizeof(Lds) <= 160 * 1024, "LDS budget");

// ------------------------------------------------------------------ row context

struct Row {
    int gi, row, grow, slice;
    int S, V, lo, hi;
    int64_t step;
    float T;       // divisor (1 for greedy rows)
    double rT;     // RN64(1 / T)
    float top_p, rep, pres, freq;
    int kk;            // effective top-k (V when off)
    int min_keep_eff;  // min(min_keep, kk)
    int mode, eos_rule, c_gate;
    bool hf, greedy, filters, p_active, pen, live, want_out, needz;
};

struct Outcome {
    int64_t token;
    float thr;    // survivors: q >= thr (and drawable)
    float mdraw;  // reference of the survivors' masses
};

// The row's parameters as loaded (a slice issues these loads before its tile's: loads return in order).
struct RowIn {
    int64_t step;
    float t, p, rep, pres, freq;
    int k;
    bool act, fin;
};

// Row parameters through the scalar cache: every address is selected without a branch (a missing array reads the
// group's scalar value, which sits in the kernel arguments), so the loads issue back to back, ahead of the tile's,
// and are waited for on their own counter.
template <class T>
__device__ __forceinline__ T sload(const T* p) {
    return *(const __attribute__((address_space(4))) T*)p;
}
__device__ __forceinline__ bool sload_flag(const uint8_t* a, int row, const uint32_t* dflt) {
    const uintptr_t addr = a ? (uintptr_t)(a + row) : (uintptr_t)dflt;
    const uint32_t wd = sload((const uint32_t*)(addr & ~(uintptr_t)3));  // the aligned word holding the byte
    return ((wd >> (8 * (uint32_t)(addr & 3))) & 0xffu) != 0u;
}

__device__ __forceinline__ RowIn load_row_in(const DevGroup& G, int row) {
    RowIn I;
    I.step = sload(G.steps ? G.steps + row : (const int64_t*)&G.zero64);
    I.t = sload(G.temperature ? G.temperature + row : &G.t_val);
    I.p = sload(G.top_p ? G.top_p + row : &G.p_val);
    I.rep = sload(G.repetition ? G.repetition + row : &G.rep_val);
    I.pres = sload(G.presence ? G.presence + row : &G.pres_val);
    I.freq = sload(G.frequency ? G.frequency + row : &G.freq_val);
    I.k = sload(G.top_k ? G.top_k + row : &G.k_val);
    I.act = sload_flag(G.active, row, &G.one32);
    I.fin = sload_flag(G.finished, row, (const uint32_t*)&G.zero64);
    return I;
}

__device__ __forceinline__ Row make_row(const DevGroup& G, int gi, int row, int slice, const RowIn& I) {
    Row R;
    R.gi = gi;
    R.row = row;
    R.grow = G.row_begin + row;
    R.slice = slice;
    R.S = G.S;
    R.V = G.vocab;
    R.lo = slice * G.slice_len;
    R.hi = min(G.vocab, R.lo + G.slice_len);
    const int64_t step = I.step;
    const float t = I.t, p = I.p, rep = I.rep, pres = I.pres, freq = I.freq;
    const int k = I.k;
    const bool act = I.act, fin = I.fin;
    R.step = uni(step);
    R.greedy = !(uni(t) > 0.f);
    R.T = R.greedy ? 1.0f : uni(t);
    R.rT = 1.0 / (double)R.T;
    R.top_p = uni(p);
    R.rep = uni(rep);
    R.pres = uni(pres);
    R.freq = uni(freq);
    R.hf = G.semantics == MIS_HF;
    R.filters = !R.greedy && (!R.hf || R.step > 0);
    const int kv = uni(k);
    R.kk = ((G.flags & MIS_TOPK_ZERO_DISABLES) && kv <= 0) ? R.V : min(max(kv, G.min_keep), R.V);
    R.min_keep_eff = min(G.min_keep, R.kk);
    R.p_active = R.filters && !((G.flags & MIS_TOPP_ONE_DISABLES) && R.top_p >= 1.0f);
    const bool topk = R.filters && R.kk < R.V;
    R.pen = G.hist_len > 0 && G.history != nullptr && (!R.hf || R.step > 0) &&
            (R.rep != 1.0f || R.pres != 0.0f || R.freq != 0.0f || G.alpha_lut != nullptr);
    R.live = uni((int)act) && !uni((int)fin);
    R.want_out = G.processed != nullptr || G.probs != nullptr;
    const bool forced = G.eos >= 0 && G.max_new > 0 && R.step >= (int64_t)G.max_new - 1;
    if (forced)
        R.mode = kForced;
    else if (!R.live && !R.want_out)
        R.mode = kSkip;
    else if (R.greedy)
        R.mode = kGreedy;
    else if (!R.filters || (!topk && !R.p_active))
        R.mode = kFull;
    else if (topk)
        R.mode = R.kk <= 1024 ? kTopK : kStream;
    else
        R.mode = kNucleus;
    if ((G.flags & MIS_FINALIZE_STREAMING) && R.mode >= kGreedy) R.mode = kStream;
    const bool censor = G.eos >= 0 && R.step < (int64_t)G.min_new;
    R.eos_rule = !censor ? kEosNormal
                         : (!R.hf ? kEosExcluded : ((R.filters && (topk || R.p_active)) ? kEosSelOnly : kEosExcluded));
    R.needz = R.mode == kNucleus || (R.mode == kTopK && R.hf && R.p_active);
    // lane maxima of the slice its gate keeps: the row's k up to 64 (then the slice's own top k are all published),
    // else twice the slice's expected share of the top k plus 12; 64 for top-p rows without top-k
    if (R.mode == kTopK)
        R.c_gate = R.kk <= 64 ? R.kk : min(kThreads, (int)((2ll * R.kk * G.slice_len + R.V - 1) / R.V) + 12);
    else
        R.c_gate = 64;
    return R;
}

// ------------------------------------------------------------------ element pipeline

__device__ __forceinline__ float penalize(const Row& R, const DevGroup& G, float x, int n) {
    const float a = alpha_of(R.rep, n, G.alpha_lut, G.alpha_lut_len);
    x = x < 0.f ? x * a : div_rn(x, a, 1.0 / (double)a);
    x = x - R.freq * (float)n;
    return x - R.pres;
}

// The processed value of element j (before the top-k / top-p filters): engine/talker_sampler.py:142-156 with
// the per-row extensions (presence / frequency after the repetition penalty, the bitmask after the penalties).
__device__ __forceinline__ float elem_q(const Row& R, const DevGroup& G, float x, int n, bool allowed, int j) {
    if (R.eos_rule == kEosExcluded && j == G.eos) return -INFINITY;
    const bool pn = R.pen && n > 0;
    if (R.hf) {
        x = div_rn(x, R.T, R.rT);
        if (pn) x = penalize(R, G, x, n);
        if (!allowed) x = -INFINITY;
    } else {
        if (pn) x = penalize(R, G, x, n);
        if (!allowed) x = -INFINITY;
        x = div_rn(x, R.T, R.rT);
    }
    return x;
}

// exp(q - m) as fixed point (0 for q = -inf or m = -inf).
__device__ __forceinline__ unsigned long long efx(float q, float m) {
    if (!(q > -INFINITY) || !(m > -INFINITY)) return 0ull;
    return (unsigned long long)((double)exp_acc(q - m) * kFx);
}

__device__ __forceinline__ float row_uniform(const DevGroup& G, const Row& R) {
    if (G.uniforms) return gp(G.uniforms)[R.row];
    const int64_t seed = G.seeds ? gp(G.seeds)[R.row] : 0;
    if (G.rng == MIS_RNG_PHILOX) return philox_uniform(seed, R.step, G.row_ids ? gp(G.row_ids)[R.row] : 0);
    return counter_uniform(seed, R.step);
}

// ------------------------------------------------------------------ inputs

template <int ES>
__device__ __forceinline__ float load_elem(const DevGroup& G, int row, int j) {
    const char* p = G.logits + ((int64_t)row * G.row_stride + j) * ES;
    if (ES == 2) return __uint_as_float((uint32_t)*gp((const uint16_t*)p) << 16);
    return *gp((const float*)p);
}

__device__ __forceinline__ const char* hist_row(const DevGroup& G, int row) {
    return G.history + (int64_t)row * G.hist_stride * (G.hist_i64 ? 8 : 4);
}

// Keep words of positions [first, first + len): word k covers elements [jb + 32 k, + 32), jb = first rounded down
// to 32.  A bit is set for an element in [lo, hi) that the bitmask allows.  Words past the range are cleared.
__device__ __forceinline__ void build_keep(const DevGroup& G, int row, int first, int len, int lo, int hi, Lds& L) {
    const int jb = (first >> 5) << 5;
    const int nw_row = (G.vocab + 31) >> 5;
    const gptr<const uint32_t> mrow = G.allowed ? gp(G.allowed) + (int64_t)row * G.allowed_stride : nullptr;
    const int nkw = min(kKeepWords, ((first + len - jb) + 31) / 32 + 1);
    for (int k = threadIdx.x; k < kKeepWords; k += kThreads) {
        uint32_t w = 0u;
        if (k < nkw) {
            const int gw = (jb >> 5) + k;
            const uint32_t allowed = mrow ? ((gw >= 0 && gw < nw_row) ? mrow[gw] : 0u) : ~0u;
            const int a = lo - (jb + 32 * k), b = hi - (jb + 32 * k);
            const uint32_t lo_m = a <= 0 ? ~0u : (a >= 32 ? 0u : (~0u << a));
            const uint32_t hi_m = b >= 32 ? ~0u : (b <= 0 ? 0u : ((1u << b) - 1u));
            w = allowed & lo_m & hi_m;
        }
        L.keep[k] = w;
    }
}

__device__ __forceinline__ void clear_keep_bit(Lds& L, int first, int j) {
    const int o = j - ((first >> 5) << 5);
    atomicAnd(&L.keep[o >> 5], ~(1u << (o & 31)));
}

__device__ __forceinline__ int count_at(const Lds& L, int pos) {
    return (int)((L.a.cnt[pos >> 1] >> (16 * (pos & 1))) & 0xffffu);
}

// History counts of the ids in [lo, hi) by position j - first, and (with `specials`) the list of distinct ids in
// [lo, hi) other than `skip_id`.  Entries < 0 (PAD) or >= V are empty.  Ends with a barrier.
__device__ __forceinline__ void build_counts(const DevGroup& G, const Row& R, int first, int len, int lo, int hi,
                                             bool specials, int skip_id, Lds& L) {
    const int words = min(kCntWords, (len + 1) / 2 + 1);
    for (int w = threadIdx.x; w < words; w += kThreads) L.a.cnt[w] = 0u;
    if (threadIdx.x == 0) L.nspec = 0;
    __syncthreads();
    const char* hrow = hist_row(G, R.row);
    const int W = G.hist_len;
    for (int b = 0; b < W; b += kThreads * 4) {
        int64_t h[4];
        if (!G.hist_i64 && (((uintptr_t)hrow & 15) == 0) && b + 4 * kThreads <= W) {
            const int4 v = ld_i4((const int4*)hrow + (b >> 2) + threadIdx.x);
            h[0] = v.x;
            h[1] = v.y;
            h[2] = v.z;
            h[3] = v.w;
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = b + 4 * threadIdx.x + u;
                h[u] = i < W ? (G.hist_i64 ? gp((const int64_t*)hrow)[i] : (int64_t)gp((const int32_t*)hrow)[i]) : -1;
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const bool in = h[u] >= lo && h[u] < hi;
            uint32_t old = 0u;
            int pos = 0;
            if (in) {
                pos = (int)(h[u] - first);
                old = atomicAdd(&L.a.cnt[pos >> 1], 1u << (16 * (pos & 1)));
                old = (old >> (16 * (pos & 1))) & 0xffffu;
            }
            if (specials) {
                const bool first_seen = in && old == 0u && (int)h[u] != skip_id;
                const uint64_t bal = ballot(first_seen);
                if (bal) {
                    int base = 0;
                    if (lane_id() == __ffsll((long long)bal) - 1) base = atomicAdd(&L.nspec, __popcll(bal));
                    base = __builtin_amdgcn_readlane(base, __ffsll((long long)bal) - 1);
                    const int slot = base + (int)rank_below(bal);
                    if (first_seen && slot < kSpecCap) {
                        L.spec[slot].j = (int)h[u];
                        L.spec[slot].sel = 0;
                    }
                }
            }
        }
    }
    __syncthreads();
}

// ------------------------------------------------------------------ cross-workgroup protocol
//
// A slice publishes with plain stores (the CU's L1 writes through to the XCD's L2), waits until they are
// acknowledged, and counts itself in with an atomic on the row's arrival word.  The finaliser reads the records
// with device-scope atomic loads, which bypass its L1.  The slices of a row run on one XCD (block b on XCD b % 8),
// so they share the L2 that holds the records; the arrival word keeps one 8-bit count per XCD, and a finaliser
// that sees an arrival from another XCD streams the row instead of reading the records.

__device__ __forceinline__ unsigned xcc_id() {
    unsigned x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    return x & 7u;
}

template <class T>
__device__ __forceinline__ T pub_ld(const T* p) {
    return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Every thread: true in the row's last workgroup to arrive.  Sets L.foreign.
__device__ __forceinline__ bool arrive(const KernelArgs& A, const Row& R, Lds& L) {
    MIS_STAMP(5);
    if (R.S == 1) {
        wait_stores();
        __syncthreads();
        L.foreign = 0;
        return true;
    }
    wait_stores();
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long* word = (unsigned long long*)(A.arrive + (int64_t)R.grow * kLineBytes);
        const unsigned x = xcc_id();
        const unsigned long long old =
            __hip_atomic_fetch_add(word, 1ull << (8 * x), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        int total = 1;
#pragma unroll
        for (int f = 0; f < 8; ++f) total += (int)((old >> (8 * f)) & 255ull);
        const int last = total == R.S;
        if (last) __hip_atomic_store(word, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        L.is_last = last;
        L.foreign = (old & ~(255ull << (8 * x))) != 0ull;
    }
    __syncthreads();
    MIS_STAMP(6);
    return L.is_last != 0;
}

__device__ __forceinline__ char* rec_base(const DevGroup& G, int row, int s) {
    return G.recs + ((int64_t)row * G.S + s) * kRecBytes;
}

// ------------------------------------------------------------------ the slice phase

template <int ES>
struct Geo {
    static constexpr int E = 16 / ES;  // elements per 16-byte chunk
    const char* rowp;
    uintptr_t base;   // 16-byte aligned address at or below element lo
    int first;        // element index at base (may be < lo)
    uintptr_t row_end;
    // a raw buffer over [base, the row's end rounded up to 16 bytes): every chunk is wholly inside or wholly
    // outside it, and a load outside returns zeros without a memory access
    __amdgpu_buffer_rsrc_t rsrc;
};

template <int ES>
__device__ __forceinline__ Geo<ES> slice_geo(const DevGroup& G, int row, int lo) {
    Geo<ES> g;
    g.rowp = G.logits + (int64_t)row * G.row_stride * ES;
    const uintptr_t lo_addr = (uintptr_t)(g.rowp + (int64_t)lo * ES);
    g.base = lo_addr & ~(uintptr_t)15;
    g.first = lo - (int)((lo_addr - g.base) / ES);
    g.row_end = (uintptr_t)(g.rowp + (int64_t)G.vocab * ES);
    const uint32_t span = (uint32_t)(((g.row_end + 15) & ~(uintptr_t)15) - g.base);
    g.rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)g.base, (short)0, (int)span, kBufferWord3);
    return g;
}

// Chunk c of the slice: the 16 bytes at base + 16 c, elements first + E c + e; zeros for a chunk that starts at
// or past element hi.  The bytes read outside the row (before its first element, after its last) share a 16-byte
// block, and so a page, with an element of the row; the caller's range bits discard them.  No branches: the
// loads of a tile are issued back to back and counted in order.
template <int ES>
__device__ __forceinline__ uint4 load_chunk(const Geo<ES>& g, int c, int hi) {
    const int j0 = g.first + c * Geo<ES>::E;
    const int off = j0 < hi ? c * 16 : 0x7ffffff0;  // out of the buffer's range: no access, zeros
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(g.rsrc, off, 0, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// The keep bits of chunk c (E bits, element e at bit e).
template <int ES>
__device__ __forceinline__ uint32_t chunk_keep(const Lds& L, int first, int c) {
    constexpr int E = Geo<ES>::E;
    const int b0 = c * E + (first - ((first >> 5) << 5));
    const int k = b0 >> 5, sh = b0 & 31;
    const uint64_t w = (uint64_t)L.keep[k] | ((uint64_t)L.keep[k + 1] << 32);
    return (uint32_t)(w >> sh) & ((1u << E) - 1u);
}

// The first kThreads * 4 ids of the row's history, loaded with the tile (thread t: ids 4t .. 4t + 3).
struct HistPre {
    int32_t h[4];  // ids outside int32 are outside every vocabulary: -1
};

__device__ __forceinline__ void preload_history(const DevGroup& G, int row, HistPre& P) {
    const int W = G.hist_len;
    const char* hrow = G.history ? hist_row(G, row) : nullptr;
    if (hrow && !G.hist_i64 && (((uintptr_t)hrow & 15) == 0) && W >= 4 * kThreads) {
        const int4 v = ld_i4((const int4*)hrow + threadIdx.x);
        P.h[0] = v.x;
        P.h[1] = v.y;
        P.h[2] = v.z;
        P.h[3] = v.w;
    } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = 4 * (int)threadIdx.x + u;
            int64_t v = -1;
            if (hrow && i < W) v = G.hist_i64 ? gp((const int64_t*)hrow)[i] : (int64_t)gp((const int32_t*)hrow)[i];
            P.h[u] = (v >= 0 && v < INT_MAX) ? (int32_t)v : -1;
        }
    }
}

// Counts history id h (if it falls in [lo, hi)) and, on its first occurrence, lists it as a special.
__device__ __forceinline__ void count_id(int64_t h, int first, int lo, int hi, int skip_id, Lds& L) {
    const bool in = h >= lo && h < hi;
    uint32_t old = 1u;
    if (in) {
        const int pos = (int)(h - first);
        old = atomicAdd(&L.a.cnt[pos >> 1], 1u << (16 * (pos & 1)));
        old = (old >> (16 * (pos & 1))) & 0xffffu;
    }
    const bool first_seen = in && old == 0u && (int)h != skip_id;
    const uint64_t bal = ballot(first_seen);
    if (bal) {
        const int leader = __ffsll((long long)bal) - 1;
        int base = 0;
        if (lane_id() == leader) base = atomicAdd(&L.nspec, __popcll(bal));
        base = __builtin_amdgcn_readlane(base, leader);
        const int slot = base + (int)rank_below(bal);
        if (first_seen && slot < kSpecCap) {
            L.spec[slot].j = (int)h;
            L.spec[slot].sel = 0;
        }
    }
}

// count_id for the four preloaded ids of a thread at once: the four count increments issued together (an id outside
// [lo, hi) adds 0 to a word of the lane-maxima histogram, a no-op, so that no increment sits under a branch), then
// one reservation of list slots for all of the wave's first occurrences.
__device__ __forceinline__ void count_ids4(const HistPre& P, int first, int lo, int hi, int skip_id, Lds& L) {
    uint32_t old[4];
    bool in[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int h = P.h[u];
        in[u] = h >= lo && h < hi;
        const int pos = in[u] ? h - first : 0;
        uint32_t* word = in[u] ? &L.a.cnt[pos >> 1] : &L.gh[lane_id()];
        old[u] = atomicAdd(word, in[u] ? 1u << (16 * (pos & 1)) : 0u);
    }
    uint64_t bal[4];
    int total = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int h = P.h[u];
        const uint32_t prev = (old[u] >> (16 * ((h - first) & 1))) & 0xffffu;
        bal[u] = ballot(in[u] && prev == 0u && h != skip_id);
        total += __popcll(bal[u]);
    }
    if (total == 0) return;
    int base = 0;
    if (lane_id() == 0) base = atomicAdd(&L.nspec, total);
    base = __builtin_amdgcn_readfirstlane(base);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int slot = base + (int)rank_below(bal[u]);
        if (((bal[u] >> lane_id()) & 1ull) && slot < kSpecCap) {
            L.spec[slot].j = P.h[u];
            L.spec[slot].sel = 0;
        }
        base += __popcll(bal[u]);
    }
}

// The row's allowed word for keep word k of a slice whose keep words start at element jb (~0 without a mask).
__device__ __forceinline__ uint32_t mask_word(const DevGroup& G, int row, int jb, int k, int nkw) {
    if (k >= nkw) return 0u;
    if (!G.allowed) return ~0u;
    const int gw = (jb >> 5) + k;
    return (gw >= 0 && gw < (G.vocab + 31) >> 5) ? gp(G.allowed)[(int64_t)row * G.allowed_stride + gw] : 0u;
}

__device__ __forceinline__ uint32_t range_bits(int j0, int lo, int hi) {
    const int a = lo - j0, b = hi - j0;
    const uint32_t lo_m = a <= 0 ? ~0u : (a >= 32 ? 0u : (~0u << a));
    const uint32_t hi_m = b >= 32 ? ~0u : (b <= 0 ? 0u : ((1u << b) - 1u));
    return lo_m & hi_m;
}

// Room in an LDS list for the lanes where pred holds (wave-aggregated); -1 where it does not.
__device__ __forceinline__ int lds_reserve(bool pred, int* counter) {
    const uint64_t b = ballot(pred);
    if (b == 0ull) return -1;
    const int leader = __ffsll((long long)b) - 1;
    int base = 0;
    if (lane_id() == leader) base = atomicAdd(counter, __popcll(b));
    base = __builtin_amdgcn_readlane(base, leader);
    return pred ? base + (int)rank_below(b) : -1;
}

// bf16 pairs with the halves whose keep bit is clear set to -inf (0xFF80).
__device__ __forceinline__ uint32_t mask_pair(uint32_t v, uint32_t kb, int d) {
    const uint32_t lo = (kb >> (2 * d)) & 1u, hi = (kb >> (2 * d + 1)) & 1u;
    const uint32_t sel = (lo ? 0x0000ffffu : 0u) | (hi ? 0xffff0000u : 0u);
    return (v & sel) | (0xff80ff80u & ~sel);
}
__device__ __forceinline__ float bf_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

// Element e (0..E-1) of a chunk held as raw words, in the tile's domain (raw logits for bf16, processed values
// for fp32).
template <int ES>
__device__ __forceinline__ float tile_val(const uint4& v, int e) {
    if (ES == 2) {
        const uint32_t w = (e >> 1) == 0 ? v.x : (e >> 1) == 1 ? v.y : (e >> 1) == 2 ? v.z : v.w;
        return (e & 1) ? bf_hi(w) : bf_lo(w);
    }
    const uint32_t w = e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
    return __uint_as_float(w);
}

// tile_val for an element index known only at run time.
template <int ES>
__device__ __forceinline__ float tile_val_dyn(const uint4& v, int e) {
    if (ES == 2) {
        const int k = e >> 1;
        const uint32_t w = k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w;
        return (e & 1) ? bf_hi(w) : bf_lo(w);
    }
    const uint32_t w = e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
    return __uint_as_float(w);
}

template <int ES>
__device__ __forceinline__ float to_q(const Row& R, float x) {
    return ES == 2 ? div_rn(x, R.T, R.rT) : x;
}

// Histogram key of a finite bf16 value b (raw bits); -0 is zero.  Keys increase with the value.
__device__ __forceinline__ int bf_key(uint32_t b) {
    const uint32_t a = b & 0x7fffu;
    if (a == 0u) return kKeyZero;
    const bool neg = (b & 0x8000u) != 0u;
    if (a < kBfLo) return neg ? kKeyZero - 1 : kKeyZero + 1;
    if (a >= kBfHi) return neg ? 0 : kKeys - 1;
    const int m = (int)(a - kBfLo);
    return neg ? kKeyZero - 2 - m : kKeyZero + 2 + m;
}

// bf_key of the two bf16 values of word v (low half: the lower element), in 16-bit lanes; in tiny their magnitude
// patterns minus one (below kBfLo - 1 exactly for a magnitude in (0, 2^-7)).
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef short i16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t hist_key2(uint32_t v, uint32_t& tiny) {
    const u16x2 w = __builtin_bit_cast(u16x2, v);
    const u16x2 sg = __builtin_bit_cast(u16x2, __builtin_bit_cast(i16x2, v) >> (i16x2)15);  // 0xffff: negative
    const u16x2 a = w & (u16x2)0x7fff;
    u16x2 m = __builtin_elementwise_max(a, (u16x2)(kBfLo - 1));
    m = __builtin_elementwise_min(m, (u16x2)kBfHi) - (u16x2)(kBfLo - 1);  // 0 below 2^-7, 0x781 from 256 up
    const u16x2 u = __builtin_elementwise_min(a, (u16x2)1) + m;            // 0 for zero, 1 for the tiny lump
    tiny = __builtin_bit_cast(uint32_t, a - (u16x2)1);
    return __builtin_bit_cast(uint32_t, ((u ^ sg) - sg) + (u16x2)kKeyZero);
}

// A tile value the histogram counts: not the -inf of a masked element, not NaN.
__device__ __forceinline__ bool hist_counted(uint32_t b) { return b != 0xff80u && (b & 0x7fffu) <= 0x7f80u; }

// Keys that hold one value: every key but the lumps (0, kKeyZero - 1, kKeyZero + 1, kKeys - 1).
__device__ __forceinline__ bool key_exact(int k) {
    return k >= 1 && k <= kKeys - 2 && k != kKeyZero - 1 && k != kKeyZero + 1;
}

// The bf16 value of an exact key.
__device__ __forceinline__ float key_bf(int k) {
    uint32_t b;
    if (k == kKeyZero)
        b = 0u;
    else if (k > kKeyZero)
        b = kBfLo + (uint32_t)(k - kKeyZero - 2);
    else
        b = 0x8000u | (kBfLo + (uint32_t)(kKeyZero - 2 - k));
    return __uint_as_float(b << 16);
}

// The value of key k in the processed domain; a lump takes the value of the exact key below it, so the values
// never decrease with the key; -inf for key 0.
__device__ __forceinline__ float key_q(const Row& R, int k) {
    const int ke = key_exact(k) ? k : k - 1;
    return ke >= 1 ? to_q<2>(R, key_bf(ke)) : -INFINITY;
}

// Histogram bin of a processed value q (a special's): 2 k when q is the value of exact key k, 2 k + 1 when it lies
// strictly between that value and the next key's; -1 below every key.  qt(k) is key_q(R, k) (computed or from a
// table).  engine/talker_sampler.py:87-92 ranks values, so equal values share a bin.
template <class QT>
__device__ __forceinline__ int hist_bin(const Row& R, float q, float q1, QT&& qt) {
    if (!(q >= q1)) return -1;  // q1 = qt(1)
    // the largest key whose value is <= q: the bf16 value nearest q T is within a key or two of it (q is x / T
    // rounded once for the bf16 x of an exact key, and a special lies between two such values); its value and the
    // next key's are taken once, and a step away from the guess takes one more
    const uint32_t yb = __float_as_uint(q * R.T);
    int lo = min(max(bf_key((yb + 0x7fffu + ((yb >> 16) & 1u)) >> 16), 1), kKeys - 1);
    float qlo = qt(lo);
    int it = 0;
    for (; qlo > q && lo > 1 && it < 4; ++it) qlo = qt(--lo);
    float qhi = lo + 1 < kKeys ? qt(lo + 1) : INFINITY;
    for (; qhi <= q && it < 8; ++it) {
        ++lo;
        qlo = qhi;
        qhi = lo + 1 < kKeys ? qt(lo + 1) : INFINITY;
    }
    if (!(qlo <= q && q < qhi)) {
        lo = 1;
        int hi = kKeys;  // qt(lo) <= q < qt(hi)
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (qt(mid) <= q)
                lo = mid;
            else
                hi = mid;
        }
        qlo = qt(lo);
    }
    // a lump takes the value of the exact key below it, so qt(k) is qlo either way
    const int k = key_exact(lo) ? lo : lo - 1;
    return qlo == q ? 2 * k : 2 * k + 1;
}

// Top-p rows without top-k on bf16 logits are settled from value counts (the histogram path).
__device__ __forceinline__ bool nucleus_hist(const Row& R, int es) {
    return es == 2 && R.mode == kNucleus && R.T >= kHistMinT;
}

__device__ __forceinline__ unsigned long long readlane_u64(unsigned long long x, int lane);
__device__ __forceinline__ void write_outputs(const DevGroup& G, const Row& R, Lds& L, const Outcome& o, bool forced);
__device__ __forceinline__ void update_state(const DevGroup& G, const Row& R, int64_t tok);

// ------------------------------------------------------------------ the histogram path's draw
//
// After a top-p row's cut is settled from the value counts, the draw needs every slice's survivor mass, in token
// order.  The row's slices other than the finaliser keep their tiles in registers and wait on the row's line.  The
// finaliser first publishes the draw's reference md (the row's largest drawable value), so that they build the table
// of masses by value while it settles the cut; then the cut, md, x0 and the row's uniform.  Every slice then sums its
// survivors chunk by chunk (in LDS), publishes its total, and waits until all of the row's totals are out; the slice
// that holds the target then walks wave, chunk and value from its registers; the others leave.  A waiting slice waits
// only for slices of its row that have arrived and are running, so every wait ends whatever the scheduling; a slice
// that still gives up (after kR2SpinTicks) counts itself in with a failure mark and raises the workspace's error
// word; the row then comes out as PAD (written by the finaliser before its decision) with its state untouched.

constexpr int kLineDec = 64;   // u32 on the row's line: 0 pending, 3 md published, 1 settled by the finaliser (the
                               // row is streamed), 2 cut published: every slice sums its survivors
constexpr int kLineSeen = 68;  // u32: slices done with the line (the last clears it)
constexpr int kLineDat = 72;   // f32 thr, md, x0 (the least bf16 value x with x / T >= thr), u (the row's uniform)
constexpr int kLineSums = 88;  // u32: slices whose survivor mass is published (low 16 bits), failures (high 16 bits)
constexpr unsigned long long kR2SpinTicks = 200000ull;  // 2 ms of the 100 MHz real-time counter
static_assert(kLineSums + 4 <= kLineBytes, "row line");


// The holder's table of masses by bf16 value: entry kTabB + m for x >= 0 and kTabB - m for x < 0, where m = 0 for
// |x| < 2^-15 (the entry holds zero's mass; the other values there are weighed one by one), m = 1 + a - kTabLo for
// magnitude patterns a in [kTabLo, kBfHi), and m = kTabN for 256 and above, -inf and NaN (no mass: a row with
// values of 256 and above is streamed, and values of -256 and below are never drawn here).  Values below x0 weigh
// nothing.  The index is computed for two values at once in 16-bit lanes.
constexpr uint32_t kTabLo = 0x3800u;                // 2^-15
constexpr int kTabN = (int)(kBfHi - kTabLo) + 1;    // 2,945
constexpr int kTabB = kTabN;
constexpr int kTabSize = 2 * kTabN + 1;
constexpr int kTabMarkOff = 8 * (kTabSize + 1);     // the draw's chunk marks follow the table in L.a
constexpr int kChunkOff = 49152;                    // then the holder's chunk masses, [wave][round][lane]
static_assert(kTabMarkOff + 8 * 12 <= kChunkOff && kChunkOff + 8 * kWaves * kRounds * 64 <= (int)sizeof(Lds::a),
              "mass table");
static_assert(16 * (kKeys + 1) + 12 * 256 <= (int)sizeof(Lds::a), "the histogram finaliser's tables");

__device__ __forceinline__ char* row_line(const KernelArgs& A, const Row& R) {
    return A.arrive + (int64_t)R.grow * kLineBytes;
}

__device__ __forceinline__ unsigned long long* tab_of(Lds& L) { return (unsigned long long*)&L.a; }

// The table indexes of the two bf16 values of word v (low half: the lower element), and in tiny their magnitude
// patterns minus one (below kTabLo - 1 exactly for a magnitude in (0, 2^-15)).
__device__ __forceinline__ uint32_t tab_idx2(uint32_t v, uint32_t& tiny) {
    const u16x2 w = __builtin_bit_cast(u16x2, v);
    const u16x2 sg = __builtin_bit_cast(u16x2, __builtin_bit_cast(i16x2, v) >> (i16x2)15);  // 0xffff: negative
    const u16x2 a = w & (u16x2)0x7fff;
    u16x2 t = __builtin_elementwise_max(a, (u16x2)(kTabLo - 1));
    t = __builtin_elementwise_min(t, (u16x2)kBfHi);
    const u16x2 m = t - (u16x2)(kTabLo - 1);
    const u16x2 idx = ((m ^ sg) - sg) + (u16x2)kTabB;
    tiny = __builtin_bit_cast(uint32_t, a - (u16x2)1);
    return __builtin_bit_cast(uint32_t, idx);
}

// The bf16 value of table entry i (0 for the entry of zero; not called for the huge entries).
__device__ __forceinline__ float tab_val(int i) {
    const int d = i - kTabB;
    const uint32_t m = (uint32_t)(d < 0 ? -d : d);
    if (m == 0u) return 0.0f;
    const uint32_t b = (kTabLo - 1u + m) | (d < 0 ? 0x8000u : 0u);
    return __uint_as_float(b << 16);
}

// The table (every thread): efx(x / T, md) for the values x >= x0 with x / T <= md, 0 elsewhere.
__device__ __forceinline__ void r2_tab(const Row& R, Lds& L, float md, float x0) {
    unsigned long long* tab = tab_of(L);
    for (int i = threadIdx.x; i < kTabSize; i += kThreads) {
        unsigned long long v = 0ull;
        const int d = i - kTabB;
        if (d > -kTabN && d < kTabN) {
            const float x = tab_val(i);
            const float q = to_q<2>(R, x);
            if (x >= x0 && q <= md) v = efx(q, md);
        }
        tab[i] = v;
    }
}

// The values below x0 out of a table built without a bound.
__device__ __forceinline__ void r2_tab_cut(Lds& L, float x0) {
    unsigned long long* tab = tab_of(L);
    for (int i = threadIdx.x; i < kTabSize; i += kThreads) {
        const int d = i - kTabB;
        if (d > -kTabN && d < kTabN && tab_val(i) < x0) tab[i] = 0ull;
    }
}

// The finaliser's words (thread 0): dec 3 with md, then 1, or 2 with thr, md, x0 and u.
__device__ __forceinline__ void r2_decide(const KernelArgs& A, const Row& R, unsigned dec, float thr, float md, float x0,
                                          float u) {
    if (threadIdx.x != 0) return;
    char* line = row_line(A, R);
    float* d = (float*)(line + kLineDat);
    if (dec == 2u) {
        d[0] = thr;
        d[2] = x0;
        d[3] = u;
    }
    if (dec != 1u) d[1] = md;
    wait_stores();
    __hip_atomic_store((unsigned*)(line + kLineDec), dec, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A slice done with the row's line (thread 0; the finaliser once its decision is out): the last of the row's
// slices leaves the words zero for the next launch.  A slice that gave up raises the workspace's error word.
__device__ __forceinline__ void r2_seen(const KernelArgs& A, const DevGroup& G, const Row& R, bool gave_up) {
    if (threadIdx.x != 0) return;
    char* line = row_line(A, R);
    unsigned* sw = (unsigned*)(line + kLineSeen);
    const unsigned now = __hip_atomic_fetch_add(sw, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    if ((int)now == R.S) {
        __hip_atomic_store((unsigned*)(line + kLineDec), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store((unsigned*)(line + kLineSums), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(sw, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (gave_up && G.paths) atomicAdd(G.paths + (MIS_WS_ERROR_OFFSET - MIS_WS_PATH_OFFSET) / 4, 1u);
}

// A waiting slice: the decision (0 if it gave up waiting).  With 2, L.fscratch holds thr, md, x0, u; the table is
// built on the way (without its bound x0), as soon as md is out.
__device__ __forceinline__ unsigned r2_wait(const KernelArgs& A, const Row& R, Lds& L) {
    const char* line = row_line(A, R);
    unsigned* dw = (unsigned*)(line + kLineDec);
    const float* dat = (const float*)(line + kLineDat);
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    bool have_tab = false;
    for (;;) {
        if (threadIdx.x == 0) {
            unsigned d = __hip_atomic_load(dw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            while (d == 0u || (have_tab && d == 3u)) {
                if (__builtin_amdgcn_s_memrealtime() - t0 > kR2SpinTicks) {
                    d = 0u;
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
                d = __hip_atomic_load(dw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            if (d == 2u) {
                L.fscratch[0] = pub_ld(dat);
                L.fscratch[2] = pub_ld(dat + 2);
                L.fscratch[3] = pub_ld(dat + 3);
            }
            if (d >= 2u) L.fscratch[1] = pub_ld(dat + 1);
            L.token = (int)d;
        }
        __syncthreads();
        const unsigned d = (unsigned)L.token;
        if (d == 0u || d == 1u) return d;
        if (!have_tab) {
            r2_tab(R, L, L.fscratch[1], -INFINITY);
            have_tab = true;
        }
        __syncthreads();  // the table complete, and L.token read by every thread before thread 0 writes it again
        if (d == 2u) return d;
    }
}

// The survivor-mass exchange (every thread): this slice's total z (or a failure mark) goes to its record and the
// row's count; once all of the row's totals are out, the slice that holds the target floor(u Z) + 1 of the total Z
// and the target within it (L.token, L.uscratch[0]).  -1: no draw here (no mass, a failure, or a slice that gave
// up waiting).
__device__ __forceinline__ int r2_exchange(const KernelArgs& A, const DevGroup& G, const Row& R, Lds& L,
                                           unsigned long long z, bool failed, float u) {
    const int tid = threadIdx.x, l = lane_id();
    char* line = row_line(A, R);
    unsigned* cw = (unsigned*)(line + kLineSums);
    if (tid == 0) {
        ((SliceRec*)rec_base(G, R.row, R.slice))->zsurv = z;
        wait_stores();
        __hip_atomic_fetch_add(cw, failed ? 0x10001u : 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
        unsigned c = __hip_atomic_load(cw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        bool gave_up = false;
        while ((int)(c & 0xffffu) < R.S) {
            if (__builtin_amdgcn_s_memrealtime() - t0 > kR2SpinTicks) {
                gave_up = true;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
            c = __hip_atomic_load(cw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        L.flags = (gave_up || (c >> 16) != 0u) ? 1 : 0;
        r2_seen(A, G, R, gave_up);
        L.token = -1;
    }
    __syncthreads();
    if (L.flags) return -1;
    if (wave_id() == 0) {
        const unsigned long long zs = l < R.S ? pub_ld(&((const SliceRec*)rec_base(G, R.row, l))->zsurv) : 0ull;
        const unsigned long long incl = wave_incl_scan(zs);
        const unsigned long long Z = readlane_u64(incl, 63);
        if (Z) {
            const double pt = floor((double)u * (double)Z) + 1.0;
            const unsigned long long T2 = pt >= (double)Z ? Z : (unsigned long long)pt;
            const uint64_t h = ballot(incl >= T2);
            if (l == __ffsll((long long)h) - 1) {
                L.token = l;
                L.uscratch[0] = T2 - (incl - zs);
            }
        }
    }
    __syncthreads();
    return L.token;
}

// The least bf16 value x with x / T >= thr (finite thr), the same in every lane of the calling wave: x0 lies within
// a few bf16 steps of thr T, so the 64 values around it are tried at once; a binary search over the order of bf16
// bit patterns settles the rest.
__device__ __forceinline__ float r2_x0(const Row& R, float thr) {
    auto val = [](uint32_t o) {  // bf16 value of order index o (0x007f: -inf ... 0xff80: +inf)
        const uint32_t b = (o & 0x8000u) ? (o & 0x7fffu) : (~o & 0xffffu);
        return __uint_as_float(b << 16);
    };
    const uint32_t yb = __float_as_uint(thr * R.T) >> 16;
    const int oc = (int)((yb & 0x8000u) ? (~yb & 0xffffu) : (yb | 0x8000u));
    const int o = min(max(oc - 32 + lane_id(), 0x0080), 0xff80);
    const uint64_t hit = ballot(to_q<2>(R, val((uint32_t)o)) >= thr);
    if (hit && !(hit & 1ull)) return val((uint32_t)min(max(oc - 32 + __ffsll((long long)hit) - 1, 0x0080), 0xff80));
    uint32_t lo = 0x007fu, hi = 0xff80u;  // to_q(val(lo)) < thr <= to_q(val(hi))
    while (hi - lo > 1u) {
        const uint32_t mid = (lo + hi) >> 1;
        if (to_q<2>(R, val(mid)) >= thr)
            hi = mid;
        else
            lo = mid;
    }
    return val(hi);
}

// The mass of the 8 bf16 values of chunk v (survivors: x >= x0, by the table; the tiny ones weighed here), into m[].
__device__ __forceinline__ void r2_chunk_masses(const Row& R, const unsigned long long* tab, const uint4& v, float x0,
                                                float md, unsigned long long (&m)[8]) {
    const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
    uint32_t tmin = 0xffffffffu;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        uint32_t tn;
        const uint32_t ix = tab_idx2(wv[h], tn);
        tmin = __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(u16x2, tmin),
                                                                       __builtin_bit_cast(u16x2, tn)));
        m[2 * h] = tab[ix & 0xffffu];
        m[2 * h + 1] = tab[ix >> 16];
    }
    const bool tiny = (tmin & 0xffffu) < kTabLo - 1u || (tmin >> 16) < kTabLo - 1u;
    if (ballot(tiny)) {  // rare: magnitudes in (0, 2^-15)
        if (tiny) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t b = (wv[e >> 1] >> (16 * (e & 1))) & 0xffffu;
                const uint32_t a = b & 0x7fffu;
                const float x = __uint_as_float(b << 16);
                if (a != 0u && a < kTabLo) m[e] = x >= x0 ? efx(to_q<2>(R, x), md) : 0ull;
            }
        }
    }
}

// A slice's survivor mass.  Each lane's survivor mass per round (the 8 values of one 16-byte chunk) goes to LDS and
// the wave's total to one reduction; each drawable special's mass is added to its chunk and its wave.  Returns the
// slice's total.  The table must be built with its bound.
__device__ __forceinline__ unsigned long long r2_chunks(const Row& R, Lds& L, const uint4 (&t)[kRounds], int RR,
                                                        int first, int ns, float thr, float md, float x0) {
    const int tid = threadIdx.x, w = wave_id(), l = lane_id();
    const unsigned long long* tab = tab_of(L);
    unsigned long long* cs = (unsigned long long*)((char*)&L.a + kChunkOff);  // [wave][round][lane]
    unsigned long long tot = 0ull;
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
        if (r >= RR) continue;
        unsigned long long m[8];
        r2_chunk_masses(R, tab, t[r], x0, md, m);
        unsigned long long c = 0ull;
#pragma unroll
        for (int e = 0; e < 8; ++e) c += m[e];
        cs[(w * kRounds + r) * 64 + l] = c;
        tot += c;
    }
    tot = wave_reduce(tot, [](unsigned long long a, unsigned long long b) { return a + b; });
    if (l == 0) L.sbfx[w] = tot;
    __syncthreads();
    MIS_STAMP(17);
    // the specials (their chunks marked in L.keep, which the tile no longer needs)
    uint32_t* smark = L.keep;
    for (int i = tid; i < kKeepWords; i += kThreads) smark[i] = 0u;
    __syncthreads();
    for (int i = tid; i < ns; i += kThreads) {
        const Special sp = L.spec[i];
        const int c = (sp.j - first) >> 3;  // chunk (w RR + r) 64 + l
        atomicOr(&smark[c >> 5], 1u << (c & 31));
        if (!sp.sel && sp.q >= thr) {
            const int sw = c / (RR * 64), sr = (c >> 6) % RR;
            const unsigned long long f = efx(sp.q, md);
            atomicAdd(&cs[(sw * kRounds + sr) * 64 + (c & 63)], f);
            atomicAdd(&L.sbfx[sw], f);
        }
    }
    __syncthreads();
    MIS_STAMP(18);
    unsigned long long z = 0ull;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) z += L.sbfx[i];
    return z;
}

// The holder's walk: the wave that holds the target rem (1-based, within the slice's survivor mass), that wave's
// chunk (a scan over its lanes, round by round: chunks are in token order), then the chunk's value.  L keeps what
// r2_chunks left.
__device__ __forceinline__ int64_t r2_walk(const Row& R, Lds& L, const uint4 (&t)[kRounds], int RR, int first, int ns,
                                           float thr, float md, float x0, unsigned long long rem) {
    const int tid = threadIdx.x, w = wave_id(), l = lane_id();
    const unsigned long long* tab = tab_of(L);
    unsigned long long* cs = (unsigned long long*)((char*)&L.a + kChunkOff);
    const uint32_t* smark = L.keep;
    if (tid == 0) L.scnt = -1;
    __syncthreads();
    // the wave of the target (every wave finds it), then that wave's chunk, round by round
    int hw;
    unsigned long long rw;
    {
        const unsigned long long v = l < kWaves ? L.sbfx[l] : 0ull;
        const unsigned long long incl = wave_incl_scan(v);
        const uint64_t h = ballot(l < kWaves && incl >= rem);
        hw = h ? __ffsll((long long)h) - 1 : -1;
        rw = hw >= 0 ? rem - (readlane_u64(incl, hw) - readlane_u64(v, hw)) : 0ull;
    }
    if (hw < 0) return R.V - 1;  // cannot happen: rem is at most the holder's survivor mass
    if (w == hw) {
        unsigned long long rr = rw;
        for (int r = 0; r < RR; ++r) {
            const unsigned long long v = cs[(w * kRounds + r) * 64 + l];
            const unsigned long long incl = wave_incl_scan(v);
            const unsigned long long wt = readlane_u64(incl, 63);
            if (rr <= wt) {
                const uint64_t h = ballot(incl >= rr);
                if (l == __ffsll((long long)h) - 1) {
                    L.scnt = r * 64 + l;
                    L.uscratch[0] = rr - (incl - v);
                }
                break;
            }
            rr -= wt;
        }
    }
    __syncthreads();
    const int hc = L.scnt;
    if (hc < 0) return R.V - 1;
    const int hr = hc >> 6, hl = hc & 63;
    const int hcc = (hw * RR + hr) * 64 + hl;  // the chunk
    const int pos0 = hcc * 8;                  // its first position from first
    // the chunk's specials, when it has any: their masses (or 0), and marks that leave them out of the tile
    unsigned long long* om = (unsigned long long*)((char*)&L.a + kTabMarkOff);
    uint32_t* osp = (uint32_t*)(om + 8);
    const bool has_spec = (smark[hcc >> 5] >> (hcc & 31)) & 1u;
    if (tid < 8) {
        om[tid] = 0ull;
        osp[tid] = 0u;
    }
    if (tid == 0) L.uscratch[1] = (unsigned long long)(R.V - 1);
    if (has_spec) {
        __syncthreads();
        for (int i = tid; i < ns; i += kThreads) {
            const Special sp = L.spec[i];
            const int pos = sp.j - first - pos0;
            if (pos >= 0 && pos < 8) {
                om[pos] = (!sp.sel && sp.q >= thr) ? efx(sp.q, md) : 0ull;
                osp[pos] = 1u;
            }
        }
    }
    __syncthreads();
    MIS_STAMP(19);
    if (w == hw && l == hl) {
        const unsigned long long rc = L.uscratch[0];
#pragma unroll
        for (int r = 0; r < kRounds; ++r) {  // a constant index into the tile, which stays in registers
            if (r >= RR || r != hr) continue;
            unsigned long long m[8];
            r2_chunk_masses(R, tab, t[r], x0, md, m);
            unsigned long long c = 0ull;
            int last = -1;
            for (int e = 0; e < 8; ++e) {
                if (osp[e]) m[e] = om[e];  // a special's tile value is -inf: its mass comes from the list
                if (!m[e]) continue;
                last = e;
                if (c + m[e] >= rc) break;
                c += m[e];
            }
            if (last >= 0) L.uscratch[1] = (unsigned long long)(first + pos0 + last);
        }
    }
    __syncthreads();
    MIS_STAMP(20);
    return (int64_t)L.uscratch[1];
}

__device__ __forceinline__ int fin_hist(const KernelArgs& A, const DevGroup& G, const Row& R, Lds& L,
                                        Outcome& out);

enum : int { kActNone = 0, kActFinalize = 1, kActForced = 2, kActStream = 3 };

// One slice workgroup: loads, the row's pipeline on the tile, publication, arrival.  Returns kActFinalize in the
// row's last workgroup to arrive (R then holds the row), kActForced in slice 0 of a row whose EOS is forced.
template <int ES>
__device__ __forceinline__ int run(const KernelArgs& A, const DevGroup& G, int gi, int row, int slice, Lds& L,
                                   Row& Rout) {
    constexpr int E = Geo<ES>::E;
    constexpr int RMAX = kRounds;
    const int RR = G.R;
    const int lo = slice * G.slice_len, hi = min(G.vocab, lo + G.slice_len);
    const Geo<ES> geo = slice_geo<ES>(G, row, lo);
    const int w = wave_id(), l = lane_id(), tid = threadIdx.x;
    // the loads in the order their values are needed (loads return in order): the row's parameters, the history
    // head and the bitmask words (the LDS set-up runs on them while the tile is in flight), then the tile
    const RowIn rin = load_row_in(G, row);
    HistPre hp;
    preload_history(G, row, hp);
    const int tile_len = kThreads * E * RR;
    const int jb = (geo.first >> 5) << 5;
    const int nkw = min(kKeepWords, (geo.first + tile_len - jb + 31) / 32 + 1);
    uint32_t mw[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) mw[u] = mask_word(G, row, jb, tid + u * kThreads, nkw);
    uint4 t[RMAX];
#pragma unroll
    for (int r = 0; r < RMAX; ++r)
        t[r] = r < RR ? load_chunk<ES>(geo, (w * RR + r) * 64 + l, hi) : make_uint4(0u, 0u, 0u, 0u);
    const Row R = make_row(G, gi, row, slice, rin);
    Rout = R;
    MIS_STAMP(1);
    MIS_STAMP_INFO(((unsigned long long)(R.grow + 1) << 32) | ((unsigned long long)slice << 8) | (unsigned)R.mode);
    if (R.mode == kSkip) {
        if (slice == 0 && tid == 0 && G.tokens) gp(G.tokens)[row] = kPad;
        return kActNone;
    }
    if (R.mode == kForced) return slice == 0 ? kActForced : kActNone;
    SliceRec* rec = (SliceRec*)rec_base(G, R.row, R.slice);
    if (R.mode == kStream) return arrive(A, R, L) ? kActFinalize : kActNone;

    // keep bits (allowed and in range) and, with penalties, a cleared count table
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int k = tid + u * kThreads;
        if (k < kKeepWords) L.keep[k] = mw[u] & range_bits(jb + 32 * k, lo, hi);
    }
    if (R.pen) {
        uint4* cw = (uint4*)L.a.cnt;
        for (int i = tid; i < (tile_len / 2 + 4) / 4; i += kThreads) cw[i] = make_uint4(0u, 0u, 0u, 0u);
    }
    if (tid == 0) {
        L.flags = 0;
        L.nspec = 0;
        L.scnt = 0;
    }
    if (tid < kMaxSB) L.sbfx[tid] = 0ull;
    if (tid < 256) L.gh[tid] = 0u;
    __syncthreads();
    // the history: counts and first occurrences (specials); a censored EOS is taken out of the tile (listed as a
    // special when it ranks but is not drawn, which takes it out with the other specials)
    const int eos = G.eos;
    const bool eos_here = eos >= lo && eos < hi && R.eos_rule != kEosNormal;
    if (eos_here && tid == 0) {
        const int slot = R.eos_rule == kEosSelOnly ? atomicAdd(&L.nspec, 1) : kSpecCap;
        if (slot < kSpecCap) {
            L.spec[slot].j = eos;
            L.spec[slot].sel = 1;
        } else {  // beyond the list the row is flagged and finalised from its logits
            clear_keep_bit(L, geo.first, eos);
        }
    }
    if (R.pen) {
        const int skip = eos_here ? eos : -1;
        count_ids4(hp, geo.first, lo, hi, skip, L);
        if (G.hist_len > 4 * kThreads) {
            const char* hrow = hist_row(G, R.row);
            for (int b = 4 * kThreads; b < G.hist_len; b += kThreads) {
                const int i = b + tid;
                const int64_t h = i < G.hist_len
                                      ? (G.hist_i64 ? gp((const int64_t*)hrow)[i] : (int64_t)gp((const int32_t*)hrow)[i])
                                      : -1;
                count_id(h, geo.first, lo, hi, skip, L);
            }
        }
    }
    __syncthreads();
    MIS_STAMP(2);
    // specials: counts and allowed bits (the keep bit, which only the special's own thread clears), out of the
    // tile; the logits of the allowed ones loaded (the loads land during pass 1)
    const int ns = min(L.nspec, kSpecCap);
    if (tid == 0 && L.nspec > kSpecCap) L.flags |= kRecOverflow;
    float sx[2];
    bool sal[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int i = tid + u * kThreads;
        sx[u] = 0.f;
        sal[u] = false;
        if (i < ns) {
            const int j = L.spec[i].j;
            const int n = R.pen ? count_at(L, j - geo.first) : 0;
            L.spec[i].n = n;
            const int o = j - jb;
            sal[u] = (L.keep[o >> 5] >> (o & 31)) & 1u;
            clear_keep_bit(L, geo.first, j);
            if (sal[u]) sx[u] = load_elem<ES>(G, R.row, j);
        }
    }
    __syncthreads();
    MIS_STAMP(3);

    // pass 1: keep bits applied; lane max (and first argmax for greedy rows) in the tile's domain.  One loop per
    // kind of row, each taking a chunk's maximum as a tree.
    float lmax = -INFINITY;
    int larg = INT_MAX;
    auto masked = [&](int r, int c) {
        const uint32_t kb = chunk_keep<ES>(L, geo.first, c);
        uint4 v = t[r];
        if (ES == 2) {
            v.x = mask_pair(v.x, kb, 0);
            v.y = mask_pair(v.y, kb, 1);
            v.z = mask_pair(v.z, kb, 2);
            v.w = mask_pair(v.w, kb, 3);
        } else {
            float f[4] = {__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w)};
#pragma unroll
            for (int e = 0; e < 4; ++e) f[e] = ((kb >> e) & 1u) ? div_rn(f[e], R.T, R.rT) : -INFINITY;
            v = make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3]));
        }
        t[r] = v;
        return v;
    };
    auto chunk_max = [&](const uint4& v) {
        float m[E];
#pragma unroll
        for (int e = 0; e < E; ++e) m[e] = tile_val<ES>(v, e);
#pragma unroll
        for (int h = E / 2; h >= 1; h /= 2)
#pragma unroll
            for (int e = 0; e < h; ++e) m[e] = fmaxf(m[e], m[e + h]);
        return m[0];
    };
    if (R.mode == kGreedy) {
#pragma unroll
        for (int r = 0; r < RMAX; ++r) {
            if (r >= RR) continue;
            const int c = (w * RR + r) * 64 + l;
            const uint4 v = masked(r, c);
            const float cm = chunk_max(v);
            if (cm > lmax) {  // the chunk's first element at its maximum (NaN never wins)
                int e0 = E - 1;
#pragma unroll
                for (int e = E - 1; e >= 0; --e) e0 = tile_val<ES>(v, e) == cm ? e : e0;
                lmax = cm;
                larg = geo.first + c * E + e0;
            }
        }
    } else {
#pragma unroll
        for (int r = 0; r < RMAX; ++r) {
            if (r >= RR) continue;
            const int c = (w * RR + r) * 64 + l;
            lmax = fmaxf(lmax, chunk_max(masked(r, c)));
        }
    }
    // the specials' processed values
    float smax = -INFINITY, sdmax = -INFINITY;
    int sarg = INT_MAX;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int i = tid + u * kThreads;
        if (i < ns) {
            const int j = L.spec[i].j;
            const float q = elem_q(R, G, sx[u], L.spec[i].n, sal[u], j);
            L.spec[i].q = q;
            smax = fmaxf(smax, q);
            if (!L.spec[i].sel && (q > sdmax || (q == sdmax && j < sarg))) {
                sdmax = q;
                sarg = j;
            }
        }
    }

    MIS_STAMP(4);
    if (R.mode == kGreedy) {
        // greedy: q = x (no temperature); specials compete with their processed values
        float v = lmax;
        int idx = larg;
        if (sdmax > v || (sdmax == v && sarg < idx)) {
            v = sdmax;
            idx = sarg;
        }
        block_argmax(v, idx, L.red);
        if (tid == 0) {
            rec->mq = v;
            rec->mqd = v;
            rec->argmax = idx;
            rec->flags = L.flags;
        }
        return arrive(A, R, L) ? kActFinalize : kActNone;
    }

    const bool gated = R.mode == kTopK || R.mode == kNucleus;
    const float4 mx = block_max4(make_float4(lmax, smax, sdmax, (gated && lmax > -INFINITY) ? -lmax : -INFINITY), L.red);
    const float tmq = is_finite_f(mx.x) ? to_q<ES>(R, mx.x) : mx.x;  // tile max, processed domain
    const float mq = fmaxf(tmq, mx.y);
    const float mqd = fmaxf(tmq, mx.z);

    if (R.mode == kFull) {
        const float mref = mqd;
        // specials' exp into their sub-blocks (fixed point: independent of the order of the additions)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int i = tid + u * kThreads;
            if (i < ns) {
                const unsigned long long f = efx(L.spec[i].q, mref);
                if (f) atomicAdd(&L.sbfx[(L.spec[i].j - geo.first) / E >> 6], f);
            }
        }
#pragma unroll
        for (int r = 0; r < RMAX; ++r) {
            if (r >= RR) continue;
            double acc = 0.0;
            if (mref > -INFINITY) {
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    const float q = to_q<ES>(R, tile_val<ES>(t[r], e));
                    if (q > -INFINITY) acc += (double)exp_acc(q - mref);
                }
            }
            acc = wave_reduce(acc, [](double a, double b) { return a + b; });
            if (l == 0) L.sb[w * RR + r] = acc;
        }
        __syncthreads();
        const int nsb = kWaves * RR;
        double* sbg = (double*)((char*)rec + kRecSbOff);
        double sv = 0.0;
        if (tid < nsb) {
            sv = L.sb[tid] + (double)L.sbfx[tid] * (1.0 / kFx);
            sbg[tid] = sv;
        }
        const double z = block_sum_d(sv, L.red);
        if (tid == 0) {
            rec->mq = mq;
            rec->mqd = mqd;
            rec->mref = mref;
            rec->z = z;
            rec->flags = L.flags;
        }
        return arrive(A, R, L) ? kActFinalize : kActNone;
    }

    if constexpr (ES == 2) {
        if (nucleus_hist(R, ES)) {
            // the count of every value of the tile (the nucleus histogram), and for the specials a value gate: the
            // specials below mq - D weigh at most V e^-D of the row's largest, less than the 1 - top_p of the row the
            // cut leaves below it, so the cut lies above them whenever the row's largest is in the slice; they are
            // summed (z), and the finaliser checks that its cut lies above every slice's gate and streams the row
            // otherwise
            const float D = R.top_p < 1.0f ? __logf((float)R.V) - log1pf(-R.top_p) + 2.0f : INFINITY;
            const float gate_q = mq - D;
            const float hb = gate_q;  // every value left out is a special below it
            // kHistReps copies of the counts (lane l adds to copy l % kHistReps, so lanes of a wave that hold one
            // value spread their LDS atomics over several addresses and banks; the history counts are no longer
            // needed); the tiny-magnitude lumps also carry their sum of exp(q) (q within 2^-7 / T of 0), and their
            // values are listed
            uint4* hk4 = (uint4*)L.a.cnt;
            for (int i = tid; i < kHistReps * kHistStride / 4; i += kThreads) hk4[i] = make_uint4(0u, 0u, 0u, 0u);
            if (tid == 0) {
                L.tinyfx = 0ull;
                L.nhi = 0;
                L.nlo = 0;
            }
            __syncthreads();
            MIS_STAMP(26);
            uint32_t* hk = L.a.cnt + (l % kHistReps) * kHistStride;
            unsigned long long tf = 0ull;
            float zr = 0.0f;
#pragma unroll
            for (int r = 0; r < RMAX; ++r) {
                if (r >= RR) continue;
                const uint32_t wv[4] = {t[r].x, t[r].y, t[r].z, t[r].w};
                uint32_t tmin = 0xffffffffu;
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    uint32_t tn;
                    const uint32_t k2 = hist_key2(wv[h], tn);
                    tmin = __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(u16x2, tmin),
                                                                                   __builtin_bit_cast(u16x2, tn)));
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const uint32_t b = (wv[h] >> (16 * e)) & 0xffffu;
                        if (hist_counted(b)) atomicAdd(&hk[(k2 >> (16 * e)) & 0xffffu], 1u);
                    }
                }
                if (ballot((tmin & 0xffffu) < kBfLo - 1u || (tmin >> 16) < kBfLo - 1u)) {
                    // rare: magnitudes in (0, 2^-7), the lumps next to zero
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const uint32_t b = (wv[e >> 1] >> (16 * (e & 1))) & 0xffffu;
                        const uint32_t a = b & 0x7fffu;
                        if (a != 0u && a < kBfLo)
                            tf += (unsigned long long)((double)exp_acc(to_q<2>(R, __uint_as_float(b << 16))) * kFx);
                    }
                }
            }
            tf = wave_reduce(tf, [](unsigned long long a, unsigned long long b) { return a + b; });
            if (l == 0 && tf) atomicAdd(&L.tinyfx, tf);
            MIS_STAMP(27);
            // the specials with their bins, those at or above the gate first (their values are not in the counts;
            // the ones below the gate are listed only for the draw's pass over the slice)
            unsigned long long* sg = (unsigned long long*)((char*)rec + kRecSpecOff);
            uint32_t* sbin = (uint32_t*)((char*)rec + kRecSpecBinOff);
            const float q1 = key_q(R, 1);
            for (int i0 = 0; i0 < ns; i0 += kThreads) {
                const int i = i0 + tid;
                const float q = i < ns ? L.spec[i].q : -INFINITY;
                const bool high = i < ns && q > -INFINITY && q >= gate_q;
                const bool low = i < ns && !high;
                const int sh = lds_reserve(high, &L.nhi);
                const int sl = lds_reserve(low, &L.nlo);
                if (i < ns) {
                    const int slot = high ? sh : ns - 1 - sl;
                    sg[slot] = ((unsigned long long)((uint32_t)L.spec[i].j | (L.spec[i].sel ? kSelOnlyBit : 0u)) << 32) |
                               __float_as_uint(q);
                    int b = -1;
                    if (high) b = hist_bin(R, q, q1, [&](int k) { return key_q(R, k); });
                    sbin[slot] = (uint32_t)(b + 1);  // 0: below every key or -inf
                    if (low && q > -INFINITY) zr += exp_acc(q - mq);
                }
            }
            const double zrd = wave_reduce((double)zr, [](double a, double b) { return a + b; });
            if (l == 0) L.red.d[w] = zrd;
            __syncthreads();
            MIS_STAMP(28);
            uint32_t* hg = (uint32_t*)((char*)rec + kRecHistOff);
            for (int i = tid; i < kHistWords; i += kThreads) {
                uint32_t a = 0u, b = 0u;
#pragma unroll
                for (int c = 0; c < kHistReps; ++c) {
                    a += L.a.cnt[c * kHistStride + 2 * i];
                    b += L.a.cnt[c * kHistStride + 2 * i + 1];
                }
                hg[i] = a | (b << 16);
            }
            MIS_STAMP(29);
            if (tid == 0) {
                double z = 0.0;
#pragma unroll
                for (int i = 0; i < kWaves; ++i) z += L.red.d[i];
                rec->mq = mq;
                rec->mqd = mqd;
                rec->gate = hb;
                rec->mref = mq;
                rec->z = z;
                rec->flags = L.flags;
                rec->hist = 1;
                rec->nspec = ns;
                rec->nhigh = L.nhi;
                rec->tinyfx = L.tinyfx;
            }
            Outcome o;
            float x0 = 0.f, u = 0.f;
            const bool fin = arrive(A, R, L);
            if (!fin) {
                // held, the tile in registers, until the finaliser's cut
                const unsigned d = r2_wait(A, R, L);
                MIS_STAMP(9);
                if (d == 1u) {
                    r2_seen(A, G, R, false);
                    return kActNone;
                }
                if (d == 0u) {  // gave up: counted in with a failure mark, so that no slice waits for its total
                    if (tid == 0) {
                        __hip_atomic_fetch_add((unsigned*)(row_line(A, R) + kLineSums), 0x10001u, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
                        r2_seen(A, G, R, true);
                    }
                    return kActNone;
                }
                o.thr = L.fscratch[0];
                o.mdraw = L.fscratch[1];
                x0 = L.fscratch[2];
                u = L.fscratch[3];
                r2_tab_cut(L, x0);
            } else {
                // the row's finaliser, its tile still in registers: the cut from every slice's counts
                const int res = L.foreign ? 0 : fin_hist(A, G, R, L, o);
                MIS_STAMP(9);
                if (res != 2) {  // the row is streamed: the waiting slices are released
                    if (R.S > 1) {
                        r2_decide(A, R, 1u, 0.f, 0.f, 0.f, 0.f);
                        r2_seen(A, G, R, false);
                    }
                    return kActStream;
                }
                x0 = r2_x0(R, o.thr);
                u = L.fscratch[3];
                if (R.S > 1) {
                    if (tid == 0 && G.tokens) gp(G.tokens)[R.row] = kPad;  // until the holder writes the token
                    r2_decide(A, R, 2u, o.thr, o.mdraw, x0, u);
                }
                if (tid == 0 && G.paths) atomicAdd(G.paths + MIS_PATH_HISTOGRAM, 1u);
                r2_tab(R, L, o.mdraw, x0);
            }
            __syncthreads();
            MIS_STAMP(14);
            // every slice: its survivor mass; then the slice that holds the target walks to it
            const unsigned long long z = r2_chunks(R, L, t, RR, geo.first, ns, o.thr, o.mdraw, x0);
            int holder = 0;
            unsigned long long rem = 0ull;
            if (R.S > 1) {
                holder = r2_exchange(A, G, R, L, z, false, u);
                rem = L.uscratch[0];
            } else if (z) {
                const double pt = floor((double)u * (double)z) + 1.0;
                rem = pt >= (double)z ? z : (unsigned long long)pt;
            } else {
                holder = -1;
            }
            MIS_STAMP(15);
            if (holder == R.slice) {
                o.token = r2_walk(R, L, t, RR, geo.first, ns, o.thr, o.mdraw, x0, rem);
                update_state(G, R, o.token);
                MIS_STAMP(10);
                MIS_STAMP_INFO(((unsigned long long)(R.grow + 1) << 32) | ((unsigned long long)R.slice << 8) | 0x80u |
                               (unsigned)MIS_PATH_HISTOGRAM);
            }
            if (fin && R.want_out) write_outputs(G, R, L, o, false);
            return kActNone;
        }
    }

    // top-k and top-p rows: per-wave gates; every element of the wave at or above its gate is published
    // the slice's gate (tile domain): a value that at least c_gate of its lane maxima reach, the c-th largest lane max
    // to within one bin of a 256-bin histogram of them over [min, max]; each wave reads the histogram itself
    const float hi_l = mx.x, lo_l = -mx.w;
    const float span_l = hi_l - lo_l;
    const bool binned = span_l > 1e-6f * fmaxf(1.0f, fabsf(hi_l));
    const float scale_l = binned ? 256.0f / span_l : 0.0f;
    if (lmax > -INFINITY) atomicAdd(&L.gh[binned ? min(255, (int)((lmax - lo_l) * scale_l)) : 0], 1u);
    __syncthreads();
    float gate = -INFINITY;
    {
        const uint4 hv = *(const uint4*)&L.gh[252 - 4 * l];  // bins 255 - 4l .. 252 - 4l, from the top
        const int v0 = (int)hv.w, v1 = (int)hv.z, v2 = (int)hv.y, v3 = (int)hv.x;
        const int sum = v0 + v1 + v2 + v3;
        const int incl = wave_incl_scan(sum);
        const int c = R.c_gate;
        if (__builtin_amdgcn_readlane(incl, 63) >= c) {
            const int ex = incl - sum;
            const int ls = __ffsll((long long)ballot(ex < c && c <= incl)) - 1;
            const int t = ex + v0 >= c ? 0 : (ex + v0 + v1 >= c ? 1 : (ex + v0 + v1 + v2 >= c ? 2 : 3));
            const int b = 255 - (4 * ls + __builtin_amdgcn_readlane(t, ls));
            // one bin lower than the bin reached, so rounding in the binning cannot put a counted lane below it
            gate = (!binned || b <= 0) ? lo_l : lo_l + (float)(b - 1) * (span_l * (1.0f / 256.0f));
        }
    }
    MIS_STAMP(16);
    const float gate_q = (gate > -INFINITY) ? to_q<ES>(R, gate) : -INFINITY;
    unsigned long long* segs = (unsigned long long*)((char*)rec + kRecCandOff);
    unsigned long long* myseg = segs + (int64_t)w * kCapWave;
    int cnt = 0, flags = 0;
    double zacc = 0.0, cacc = 0.0;
    const float mref = mq;
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
        if (r >= RR) continue;
        const int c = (w * RR + r) * 64 + l;
        // the chunk's elements at or above the gate as a mask; one wave scan places every lane's candidates (in
        // token order) after the wave's previous ones
        uint32_t bits = 0u;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const float x = tile_val<ES>(t[r], e);
            bits |= (x >= gate && x > -INFINITY) ? (1u << e) : 0u;
            if (R.needz) {
                const float q = to_q<ES>(R, x);
                const double ex = q > -INFINITY ? (double)exp_acc(q - mref) : 0.0;
                zacc += ex;
                if (x >= gate) cacc += ex;
            }
        }
        const int nb = __popc(bits);
        const int incl = wave_incl_scan(nb);
        const int tot = __builtin_amdgcn_readlane(incl, 63);
        if (tot) {
            if (cnt + tot > kCapWave) {
                flags |= kRecOverflow;
                cnt = kCapWave;
            } else {
                int pos = cnt + incl - nb;
                const uint32_t j0 = (uint32_t)(geo.first + c * E);
                while (bits) {
                    const int e = __ffs(bits) - 1;
                    bits &= bits - 1u;
                    const float q = to_q<ES>(R, tile_val_dyn<ES>(t[r], e));
                    myseg[pos++] = ((unsigned long long)(j0 + (uint32_t)e) << 32) | __float_as_uint(q);
                }
                cnt += tot;
            }
        }
    }
    MIS_STAMP(17);
    // specials at or above the gate (every wave; slots of segment kWaves reserved in LDS)
    unsigned long long* sseg = segs + (int64_t)kWaves * kCapWave;
    for (int i0 = 0; i0 < ns; i0 += kThreads) {
        const int i = i0 + tid;
        const bool in = i < ns;
        const float q = in ? L.spec[i].q : -INFINITY;
        const uint32_t id = in ? ((uint32_t)L.spec[i].j | (L.spec[i].sel ? kSelOnlyBit : 0u)) : 0u;
        const bool pred = q >= gate_q && q > -INFINITY;
        if (R.needz && q > -INFINITY) {
            const double ex = (double)exp_acc(q - mref);
            zacc += ex;
            if (pred) cacc += ex;
        }
        const int slot = lds_reserve(pred, &L.scnt);
        if (pred) {
            if (slot < kCapSpecSeg)
                sseg[slot] = ((unsigned long long)id << 32) | __float_as_uint(q);
            else
                flags |= kRecOverflow;
        }
    }
    if (R.needz) {
        zacc = wave_reduce(zacc, [](double a, double b) { return a + b; });
        cacc = wave_reduce(cacc, [](double a, double b) { return a + b; });
    }
    flags = wave_reduce(flags, [](int a, int b) { return a | b; });
    MIS_STAMP(18);
    __syncthreads();
    MIS_STAMP(19);
    if (l == 0) {
        L.segoff[w] = cnt;
        L.red.d[w] = zacc;
        L.sb[w] = cacc;
        if (flags) atomicOr(&L.flags, flags);
    }
    __syncthreads();
    if (tid == 0) {
        double z = 0.0, zc = 0.0;
#pragma unroll
        for (int i = 0; i < kWaves; ++i) {
            z += L.red.d[i];
            zc += L.sb[i];
        }
        rec->zc = zc;
        rec->ncand[kWaves] = min(L.scnt, kCapSpecSeg);
        rec->mq = mq;
        rec->mqd = mqd;
        rec->gate = gate_q;
        rec->mref = mref;
        rec->z = z;
        rec->flags = L.flags | (gate_q > -INFINITY ? 0 : kRecGateInf);
        rec->hist = 0;
        rec->nspec = ns;
    }
    if (tid < kWaves) rec->ncand[tid] = L.segoff[tid];
    return arrive(A, R, L) ? kActFinalize : kActNone;
}

// ------------------------------------------------------------------ the finaliser
//
// The finaliser asks questions of a set of elements: the candidates its slices published, gathered into LDS, or
// the whole row, streamed in chunks with its processed values recomputed (history counts and keep bits rebuilt in
// LDS for each chunk).  One visiting routine serves every question (maxima, the histogram rounds of a selection,
// sums, the outputs), so the code that runs stays small.  Nothing here depends on the logits' dtype at compile
// time.

__device__ __forceinline__ float load_logit(const DevGroup& G, int row, int j) {
    const char* p = G.logits + ((int64_t)row * G.row_stride + j) * G.es;
    return G.es == 2 ? __uint_as_float((uint32_t)*gp((const uint16_t*)p) << 16) : *gp((const float*)p);
}

__device__ __forceinline__ int slice_first(const DevGroup& G, int row, int lo) {
    const char* rowp = G.logits + (int64_t)row * G.row_stride * G.es;
    const uintptr_t lo_addr = (uintptr_t)(rowp + (int64_t)lo * G.es);
    return lo - (int)((lo_addr & 15) / G.es);
}

enum : int { kSrcCands = 0, kSrcRow = 1 };
enum : int { kJobStats = 0, kJobHist, kJobSums, kJobSurvMax, kJobSurvSum, kJobOutZ, kJobOut, kJobPick };
enum : int { kSelCount = 0, kSelCut, kSelDraw };

struct Visit {
    int src, n;       // kSrcCands: n candidates in L.a.c (weighted: the id field holds a multiplicity)
    bool weighted;
    int lo, hi;       // kSrcRow: elements [lo, hi)
    int job, sel;
    uint32_t lo_k, hi_k;
    int sh;           // kJobHist: keys in [lo_k, hi_k], bins of 2^sh keys
    float kth, thr, m, md;
    gptr<float> prow;
    gptr<float> qrow;
    float inv;
    // per-thread results
    float f0, f1;
    int i0, i1;
    unsigned long long u0, u1;
    double d0;
};

__device__ __forceinline__ void consume(Visit& V, Lds& L, float q, int j, bool drawable,
                                        unsigned long long mult = 1ull) {
    switch (V.job) {
    case kJobStats:  // f0: max; f1: max drawable (i0: its first index); i1: finite count
        V.f0 = fmaxf(V.f0, q);
        if (q > -INFINITY) V.i1 += (int)mult;
        if (drawable && (q > V.f1 || (q == V.f1 && j < V.i0))) {
            V.f1 = q;
            V.i0 = j;
        }
        break;
    case kJobHist: {
        uint32_t key;
        unsigned long long w;
        if (V.sel == kSelCount) {
            key = ord_key(q);
            w = q > -INFINITY ? mult : 0ull;
        } else if (V.sel == kSelCut) {
            key = ord_key(q);
            w = q > V.kth ? mult * efx(q, V.m) : 0ull;
        } else {
            key = (uint32_t)j;
            w = (drawable && q >= V.thr) ? efx(q, V.md) : 0ull;
        }
        if (w && key >= V.lo_k && key <= V.hi_k) atomicAdd(&L.h.w[(key - V.lo_k) >> V.sh], w);
        break;
    }
    case kJobSums:  // u0: mass above kth; u1: all mass (relative to m)
        if (q > -INFINITY) {
            const unsigned long long e = mult * efx(q, V.m);
            if (q > V.kth) V.u0 += e;
            V.u1 += e;
        }
        break;
    case kJobSurvMax:
        if (drawable && q >= V.thr && q > -INFINITY) V.f0 = fmaxf(V.f0, q);
        break;
    case kJobSurvSum:
        if (drawable && q >= V.thr) V.u0 += mult * efx(q, V.md);
        break;
    case kJobOutZ:
        if (drawable && q >= V.thr && q > -INFINITY) V.d0 += (double)exp_acc(q - V.md);
        break;
    case kJobOut: {
        const bool keep = drawable && q >= V.thr;
        if (V.prow) V.prow[j] = keep ? q : -INFINITY;
        if (V.qrow)
            V.qrow[j] = !(V.md > -INFINITY) ? NAN : ((keep && q > -INFINITY) ? exp_acc(q - V.md) * V.inv : 0.0f);
        break;
    }
    case kJobPick:  // one element per thread
        V.d0 = (drawable && q > -INFINITY) ? (double)exp_acc(q - V.m) : 0.0;
        V.i0 = j;
        break;
    }
}

// Every thread calls visit.
__device__ __forceinline__ void visit(Visit& V, const DevGroup& G, const Row& R, Lds& L) {
    if (V.src == kSrcCands) {
        for (int i = threadIdx.x; i < V.n; i += kThreads) {
            const uint32_t id = L.a.c.id[i];
            const uint32_t v = id & ~kSelOnlyBit;
            consume(V, L, L.a.c.q[i], (int)v, !(id & kSelOnlyBit), V.weighted ? (unsigned long long)v : 1ull);
        }
        return;
    }
    const int chunk = kTileMax - 64;
    for (int c0 = V.lo; c0 < V.hi; c0 += chunk) {
        const int c1 = min(V.hi, c0 + chunk);
        __syncthreads();
        if (R.pen) build_counts(G, R, c0, c1 - c0, c0, c1, false, -1, L);
        build_keep(G, R.row, c0, c1 - c0, c0, c1, L);
        __syncthreads();
        for (int j = c0 + (int)threadIdx.x; j < c1; j += kThreads) {
            const float x = load_logit(G, R.row, j);
            const int n = R.pen ? count_at(L, j - c0) : 0;
            const int o = j - ((c0 >> 5) << 5);
            const bool allowed = (L.keep[o >> 5] >> (o & 31)) & 1u;
            const float q = elem_q(R, G, x, n, allowed, j);
            consume(V, L, q, j, !(R.eos_rule == kEosSelOnly && j == G.eos));
        }
    }
    __syncthreads();
}

// Scans keys in [klo, khi] in descending or ascending order and finds the first key at which the cumulative
// weight (the selection `sel` of the visited set, plus an optional virtual element vkey of weight vw) reaches T
// (T >= 1).  Each round histograms the keys of the current range into bins of a power-of-two width (at most kBins
// of them), finds the bin that reaches T and narrows the range to it, until the range is one key.  False when the
// total weight is below T; otherwise the key and the weight of every key strictly before it in scan order.
// Weights are integers, so the result does not depend on the order of the LDS additions.
__device__ __forceinline__ bool range_find(Visit& V, int sel, bool desc, unsigned long long T, uint32_t klo,
                                           uint32_t khi, uint32_t vkey, unsigned long long vw, const DevGroup& G,
                                           const Row& R, Lds& L, uint32_t& key_out, unsigned long long& before_out) {
    Hist& h = L.h;
    unsigned long long acc = 0;
    for (;;) {
        const uint64_t span = (uint64_t)khi - klo + 1;
        int sh = 0;
        while (((span - 1) >> sh) >= (uint64_t)kBins) ++sh;  // every key's bin (key - klo) >> sh < kBins
        const int nb = (int)((span + ((1ull << sh) - 1)) >> sh);
        for (int b = threadIdx.x; b < nb; b += kThreads) h.w[b] = 0ull;
        __syncthreads();
        V.job = kJobHist;
        V.sel = sel;
        V.lo_k = klo;
        V.hi_k = khi;
        V.sh = sh;
        visit(V, G, R, L);
        if (threadIdx.x == 0 && vw && vkey >= klo && vkey <= khi) atomicAdd(&h.w[(vkey - klo) >> sh], vw);
        __syncthreads();
        const int s0 = 2 * (int)threadIdx.x, s1 = s0 + 1;
        const int b0 = desc ? nb - 1 - s0 : s0, b1 = desc ? nb - 1 - s1 : s1;
        const unsigned long long v0 = s0 < nb ? h.w[b0] : 0ull, v1 = s1 < nb ? h.w[b1] : 0ull;
        unsigned long long tot;
        const unsigned long long ex = block_excl_scan(v0 + v1, tot, h.scan);
        if (tot < T) return false;
        if (s0 < nb && ex < T && T <= ex + v0) {
            h.sel = b0;
            h.before = ex;
        } else if (s1 < nb && ex + v0 < T && T <= ex + v0 + v1) {
            h.sel = b1;
            h.before = ex + v0;
        }
        __syncthreads();
        const int b = h.sel;
        const unsigned long long bf = h.before;
        T -= bf;
        acc += bf;
        const uint64_t a = (uint64_t)klo + ((uint64_t)b << sh);
        klo = (uint32_t)a;
        khi = (uint32_t)std::min<uint64_t>((uint64_t)khi, a + (1ull << sh) - 1);
        if (sh == 0) break;
    }
    key_out = klo;
    before_out = acc;
    return true;
}


// The top-k / top-p selection (engine/talker_sampler.py:95-133) and the draw (:161-172) over a visited set.
// m_sel: max over everything ranked; zfull_fx: the whole-vocabulary normaliser in fixed point relative to m_sel
// (HF order, or no top-k); n_fin: finite elements in the set; [klo, khi]: key range of its values.  From the
// candidates, every check that they hold what the selection needs is made (gate: every element >= gate is a
// candidate); false when one fails (the caller then streams the row).
__device__ __forceinline__ bool select_draw(const DevGroup& G, const Row& R, Lds& L, Visit& V, float m_sel,
                                            double zfull_fx, int n_fin, float gate, bool all_gate_inf,
                                            bool from_cands, uint32_t klo, uint32_t khi, Outcome& out) {
    const bool topk = R.kk < R.V;
    float kth = -INFINITY;
    unsigned long long cnt_gt = (unsigned long long)n_fin;
    uint32_t kkey = 0u;
    unsigned long long bf;
    if (topk) {
        if ((unsigned long long)R.kk <= (unsigned long long)n_fin) {
            range_find(V, kSelCount, true, (unsigned long long)R.kk, klo, khi, 0u, 0ull, G, R, L, kkey, bf);
            kth = key_float(kkey);
            cnt_gt = bf;
            if (from_cands && !(kth >= gate)) return false;
        } else if (from_cands && !all_gate_inf) {
            return false;
        }
    }
    float thr = kth;
    if (R.p_active) {
        V.m = m_sel;
        V.kth = kth;
        const unsigned long long ekth = efx(kth, m_sel);
        const unsigned long long vw = (topk && kth > -INFINITY) ? ((unsigned long long)R.kk - cnt_gt) * ekth : 0ull;
        double zn;
        if (topk && !R.hf) {
            V.job = kJobSums;
            V.u0 = V.u1 = 0ull;
            visit(V, G, R, L);
            zn = (double)(block_sum_u(V.u0, L.red) + vw);
        } else {
            zn = zfull_fx;
        }
        const double pt = ceil((double)R.top_p * zn);
        const unsigned long long T = pt < 1.0 ? 1ull : (unsigned long long)pt;
        uint32_t ckey = 0u;
        const uint32_t kthkey = ord_key(kth);
        const bool found = range_find(V, kSelCut, true, T, (kth > -INFINITY) ? max(klo, kthkey) : klo, khi, kthkey, vw,
                                      G, R, L, ckey, bf);
        float thr_p;
        if (found) {
            thr_p = key_float(ckey);
        } else {
            if (!topk && from_cands) return false;  // the nucleus reaches below the candidates
            thr_p = kth;
        }
        if (!topk && from_cands && !(thr_p >= gate)) return false;
        float vmk = m_sel;
        if (R.min_keep_eff >= 2) {
            uint32_t mk = 0u;
            if ((unsigned long long)R.min_keep_eff > (unsigned long long)n_fin) {
                vmk = -INFINITY;
            } else {
                range_find(V, kSelCount, true, (unsigned long long)R.min_keep_eff, klo, khi, 0u, 0ull, G, R, L, mk, bf);
                vmk = key_float(mk);
            }
            if (from_cands && !(vmk >= gate)) return false;
        }
        thr = fminf(thr_p, vmk);
        if (topk) thr = fmaxf(thr, kth);
    }
    // survivors: drawable, finite, q >= thr
    V.job = kJobSurvMax;
    V.thr = thr;
    V.f0 = -INFINITY;
    visit(V, G, R, L);
    const float md = block_max_f(V.f0, L.red);
    out.thr = thr;
    out.mdraw = md;
    out.token = R.V - 1;
    if (!(md > -INFINITY)) return true;
    V.job = kJobSurvSum;
    V.md = md;
    V.u0 = 0ull;
    visit(V, G, R, L);
    const unsigned long long zs = block_sum_u(V.u0, L.red);
    const float u = row_uniform(G, R);
    const unsigned long long T = (unsigned long long)floor((double)u * (double)zs) + 1ull;
    uint32_t tok = 0u;
    if (zs > 0ull && range_find(V, kSelDraw, false, T, 0u, (uint32_t)(R.V - 1), 0u, 0ull, G, R, L, tok, bf))
        out.token = (int64_t)tok;
    return true;
}

// Every element streamed: the reference path for any row.
__device__ __forceinline__ void fin_stream(const DevGroup& G, const Row& R, Lds& L, Outcome& out) {
    Visit V;
    V.weighted = false;
    V.src = kSrcRow;
    V.n = 0;
    V.lo = 0;
    V.hi = R.V;
    V.job = kJobStats;
    V.f0 = V.f1 = -INFINITY;
    V.i0 = INT_MAX;
    V.i1 = 0;
    V.kth = V.thr = V.m = V.md = -INFINITY;
    visit(V, G, R, L);
    float m_draw = V.f1;
    int arg = V.i0;
    block_argmax(m_draw, arg, L.red);
    const float m_sel = block_max_f(V.f0, L.red);
    const int nfin = block_sum_i(V.i1, L.red);
    out.thr = -INFINITY;
    out.mdraw = m_draw;
    if (R.greedy) {
        out.token = m_draw > -INFINITY ? arg : 0;
        return;
    }
    Row R2 = R;
    if (!R.filters) {
        R2.kk = R.V;
        R2.p_active = false;
    }
    double zfull = 0.0;
    if (R2.p_active && (R2.hf || R2.kk >= R2.V)) {
        V.job = kJobSums;
        V.m = m_sel;
        V.kth = INFINITY;
        V.u0 = V.u1 = 0ull;
        visit(V, G, R, L);
        zfull = (double)block_sum_u(V.u1, L.red);
    }
    select_draw(G, R2, L, V, m_sel, zfull, nfin, -INFINITY, true, false, 0u, 0xffffffffu, out);
}

// ------------------------------------------------------------------ the candidate finaliser (one wave)
//
// Once the candidates are in LDS (gathered by the whole workgroup, each with its mass relative to the row max), the
// selections run on wave 0 alone: no workgroup barriers, and each instruction costs one issue slot instead of
// sixteen.  The other waves wait at the barrier that follows.

__device__ __forceinline__ unsigned long long readlane_u64(unsigned long long x, int lane) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), lane);
    return ((unsigned long long)hi << 32) | lo;
}

#define MIS_LDS __attribute__((address_space(3)))

// A candidate set in LDS: value, id (with kSelOnlyBit), mass efx(q, row max).  The pointers carry the LDS address
// space so that every access is a DS instruction, not a flat one.
struct WSet {
    const MIS_LDS float* q;
    const MIS_LDS uint32_t* id;
    const MIS_LDS unsigned long long* mass;
    int n;
};

__device__ __forceinline__ WSet wset_of(float* q, uint32_t* id, unsigned long long* mass, int n) {
    WSet s;
    s.q = (const MIS_LDS float*)q;
    s.id = (const MIS_LDS uint32_t*)id;
    s.mass = (const MIS_LDS unsigned long long*)mass;
    s.n = n;
    return s;
}

template <class T>
__device__ __forceinline__ T wave_sum(T x) {
    return wave_reduce(x, [](T a, T b) { return a + b; });
}

// ------------------------------------------------------------------ small candidate sets: sorted in registers
//
// Up to 256 candidates: one bitonic sort by (value descending, index) puts them in rank order, after which the k-th
// value, the top-p cut and min_keep are rank lookups and one prefix scan; a second sort by token id (the id and
// the mass packed in one 64-bit key) gives the draw.  No LDS round trips between the steps.

__device__ __forceinline__ unsigned long long shfl_xor_u64(unsigned long long x, int j) {
    switch (j) {
    case 1: return shfl_xor<1>(x);
    case 2: return shfl_xor<2>(x);
    case 4: return shfl_xor<4>(x);
    case 8: return shfl_xor<8>(x);
    case 16: return shfl_xor<16>(x);
    default: return shfl_xor<32>(x);
    }
}

// v[p] is element p * 64 + lane of a bitonic network over 64 P keys; sorted ascending on return.
template <int P>
__device__ __forceinline__ void wave_bitonic(unsigned long long (&v)[P]) {
    const int lane = lane_id();
#pragma unroll
    for (int k = 2; k <= 64 * P; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            unsigned long long w[P];
#pragma unroll
            for (int p = 0; p < P; ++p) w[p] = j >= 64 ? v[p ^ (j >> 6)] : shfl_xor_u64(v[p], j);
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const int i = p * 64 + lane;
                const bool keep_min = ((i & j) == 0) == ((i & k) == 0);
                const bool lt = v[p] < w[p];
                v[p] = (lt == keep_min) ? v[p] : w[p];
            }
        }
    }
}

// The value of x[] at rank r (uniform r < 64 P): element r of the rank order.
// Each element is read out of its lane first and the pick is made among the scalar results, so no per-lane value is
// ever indexed by r.
template <int P, class T>
__device__ __forceinline__ T at_rank(const T (&x)[P], int r) {
    T y = (T)0;
#pragma unroll
    for (int p = 0; p < P; ++p) {
        T z;
        if constexpr (sizeof(T) == 8) z = (T)readlane_u64((unsigned long long)x[p], r & 63);
        else z = (T)__builtin_amdgcn_readlane((int)x[p], r & 63);
        if ((r >> 6) == p) y = z;
    }
    return y;
}

// select_draw for at most 64 P candidates (n >= 1), on wave 0.
template <int P>
__device__ __forceinline__ bool wsort_select_draw(const Row& R, const WSet& s, float m_sel, double zfull_fx, float gate,
                                                  bool all_gate_inf, float u, Outcome& out) {
    const int l = lane_id();
    const int n = s.n;
    unsigned long long v[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const int i = p * 64 + l;
        const float q = s.q[min(i, n - 1)];
        v[p] = i < n ? (((unsigned long long)~ord_key(q) << 32) | (uint32_t)i) : ~0ull;
    }
    wave_bitonic<P>(v);
    uint32_t key[P], id[P];
    unsigned long long mass[P];
    bool valid[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const int r = p * 64 + l;
        valid[p] = r < n;
        const int ix = valid[p] ? (int)(uint32_t)v[p] : 0;
        key[p] = ~(uint32_t)(v[p] >> 32);
        id[p] = s.id[ix];
        mass[p] = s.mass[ix];
    }
    const bool topk = R.kk < R.V;
    float kth = -INFINITY;
    unsigned long long cnt_gt = (unsigned long long)n;
    if (topk) {
        if (R.kk <= n) {
            kth = key_float(at_rank<P>(key, R.kk - 1));
            const uint32_t kk_key = ord_key(kth);
            cnt_gt = 0ull;
#pragma unroll
            for (int p = 0; p < P; ++p) cnt_gt += (unsigned long long)__popcll(ballot(valid[p] && key[p] > kk_key));
            if (!(kth >= gate)) return false;
        } else if (!all_gate_inf) {
            return false;
        }
    }
    const uint32_t kthkey = ord_key(kth);
    float thr = kth;
    if (R.p_active) {
        const unsigned long long ekth = efx(kth, m_sel);
        const unsigned long long vw = (topk && kth > -INFINITY) ? ((unsigned long long)R.kk - cnt_gt) * ekth : 0ull;
        unsigned long long wr[P];
        unsigned long long above = 0ull;
#pragma unroll
        for (int p = 0; p < P; ++p) {
            wr[p] = (valid[p] && key[p] > kthkey) ? mass[p] : 0ull;
            above += wr[p];
            if ((unsigned long long)(p * 64 + l) == cnt_gt) wr[p] += vw;  // the ties at kth, at its first rank
        }
        double zn;
        if (topk && !R.hf)
            zn = (double)(wave_sum(above) + vw);
        else
            zn = zfull_fx;
        const double pt = ceil((double)R.top_p * zn);
        const unsigned long long T = pt < 1.0 ? 1ull : (unsigned long long)pt;
        int rcut = -1;
        unsigned long long carry = 0ull;
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const unsigned long long incl = wave_incl_scan(wr[p]) + carry;
            const uint64_t hit = ballot(incl >= T);
            if (rcut < 0 && hit) rcut = p * 64 + __ffsll((long long)hit) - 1;
            carry = readlane_u64(incl, 63);
        }
        float thr_p;
        if (rcut >= 0) {
            thr_p = key_float(at_rank<P>(key, rcut));
        } else {
            if (!topk) return false;  // the nucleus reaches below the candidates
            thr_p = kth;
        }
        if (!topk && !(thr_p >= gate)) return false;
        float vmk = m_sel;
        if (R.min_keep_eff >= 2) {
            if (R.min_keep_eff > n) {
                vmk = -INFINITY;
            } else {
                vmk = key_float(at_rank<P>(key, R.min_keep_eff - 1));
                if (!(vmk >= gate)) return false;
            }
        }
        thr = fminf(thr_p, vmk);
        if (topk) thr = fmaxf(thr, kth);
    }
    // survivors: drawable, q >= thr; the first in rank order is the largest
    const uint32_t thrkey = ord_key(thr);
    bool surv[P];
    int first = -1;
#pragma unroll
    for (int p = 0; p < P; ++p) {
        surv[p] = valid[p] && key[p] >= thrkey && !(id[p] & kSelOnlyBit);  // candidates are finite
        const uint64_t b = ballot(surv[p]);
        if (first < 0 && b) first = p * 64 + __ffsll((long long)b) - 1;
    }
    const float md = first >= 0 ? key_float(at_rank<P>(key, first)) : -INFINITY;
    out.thr = thr;
    out.mdraw = md;
    out.token = R.V - 1;
    if (!(md > -INFINITY)) return true;
    const bool md_is_m = md == m_sel;
    unsigned long long zs = 0ull;
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const unsigned long long m2 = surv[p] ? (md_is_m ? mass[p] : efx(key_float(key[p]), md)) : 0ull;
        zs += m2;
        v[p] = surv[p] ? (((unsigned long long)(id[p] & ~kSelOnlyBit) << 43) | m2) : ~0ull;  // id < 2^21, mass < 2^43
    }
    zs = wave_sum(zs);
    if (zs == 0ull) return true;
    const unsigned long long T2 = (unsigned long long)floor((double)u * (double)zs) + 1ull;
    wave_bitonic<P>(v);  // survivors by token id
    constexpr unsigned long long kMassMask = (1ull << 43) - 1ull;
    unsigned long long carry = 0ull;
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const unsigned long long w = v[p] == ~0ull ? 0ull : (v[p] & kMassMask);
        const unsigned long long incl = wave_incl_scan(w) + carry;
        const uint64_t hit = ballot(v[p] != ~0ull && incl >= T2);
        if (hit) {
            out.token = (int64_t)(readlane_u64(v[p], __ffsll((long long)hit) - 1) >> 43);
            return true;
        }
        carry = readlane_u64(incl, 63);
    }
    return true;
}

// ------------------------------------------------------------------ the candidate finaliser (whole workgroup)
//
// The row's candidates (every element at or above its slice's gate, and the slices' specials at or above it) are
// gathered into LDS: the tile candidates first, in token order (slices in order, each slice's waves in order), then
// the specials.  Each question of the selection (the k-th value, the top-p cut, the min_keep floor) is one block
// scan over kSelBins value bins filled by one pass of LDS atomics; only the bin that holds the answer is ranked
// element by element, by every thread at once.  The draw is one block scan in token order.

// Value bins over [qmin, qmax]: monotone in the value, equal values share a bin.
struct SelBins {
    float qmin, scale;
};
__device__ __forceinline__ int sel_bin(float q, const SelBins& B) {
    const float f = fminf((q - B.qmin) * B.scale, (float)(kSelBins - 1));
    return max((int)f, 0);
}

// The elements of bin b sorted by value, descending (equal values in any order: they weigh alike): values in
// L.ss.sq, set indices in L.ss.sw; returns their count, or -1 when more than kSelCap.
__device__ __forceinline__ int sel_sort_bin(int b, int n, const SelBins& B, Lds& L) {
    const int tid = threadIdx.x;
    if (tid == 0) L.scnt = 0;
    __syncthreads();
    for (int i0 = 0; i0 < n; i0 += kThreads) {
        const int i = i0 + tid;
        const float q = i < n ? L.a.w.q[i] : 0.f;
        const bool in = i < n && sel_bin(q, B) == b;
        const int slot = lds_reserve(in, &L.scnt);
        if (in && slot < kSelCap) {
            L.ss.cq[slot] = q;
            L.ss.cw[slot] = (unsigned long long)i;
        }
    }
    __syncthreads();
    MIS_STAMP(23);
    const int m = L.scnt;
    if (m > kSelCap) return -1;
    // a bin of one value (the usual case: the bins are finer than the values' spacing) is sorted as it stands
    if (tid == 0) L.flags = 0;
    __syncthreads();
    if (tid < m && L.ss.cq[tid] != L.ss.cq[0]) L.flags = 1;
    __syncthreads();
    if (L.flags == 0) {
        if (tid < m) {
            L.ss.sq[tid] = L.ss.cq[tid];
            L.ss.sw[tid] = L.ss.cw[tid];
        }
        __syncthreads();
        return m;
    }
    if (tid < m) {
        const float q = L.ss.cq[tid];
        const uint32_t k = ord_key(q);
        int r = 0;
        // eight values per step, read together (the reads are broadcasts; one step waits once)
        for (int j0 = 0; j0 < m; j0 += 8) {
            float c[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) c[e] = L.ss.cq[min(j0 + e, m - 1)];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int j = j0 + e;
                const uint32_t kj = ord_key(c[e]);
                r += (j < m && (kj > k || (kj == k && j < tid))) ? 1 : 0;
            }
        }
        L.ss.sq[r] = q;
        L.ss.sw[r] = L.ss.cw[tid];
    }
    __syncthreads();
    return m;
}

// Position in the sorted bin (m elements) at which `before` plus the cumulative weight first reaches T; -1 if never.
__device__ __forceinline__ int sel_cross(int m, unsigned long long before, unsigned long long T, Lds& L) {
    const int tid = threadIdx.x;
    const unsigned long long w = tid < m ? L.ss.sw[tid] : 0ull;
    unsigned long long tot;
    const unsigned long long ex = block_excl_scan(w, tot, L.red.u) + before;
    if (tid == 0) L.token = -1;
    __syncthreads();
    if (tid < m && w && ex < T && T <= ex + w) L.token = tid;
    __syncthreads();
    const int r = L.token;
    __syncthreads();
    return r;
}

// The bins' counts and masses replaced by their sums over the bin and every bin above it (the highest bin first),
// in one pass: each question below then finds its bin with one check per thread and no further scan.
__device__ __forceinline__ void sel_prefix(Lds& L) {
    const int tid = threadIdx.x, w = wave_id();
    uint32_t* bc = L.ss.bcnt;
    unsigned long long* bm = L.h.w;
    const int b0 = kSelBins - 1 - 2 * tid, b1 = b0 - 1;
    const unsigned long long c0 = bc[b0], c1 = bc[b1], m0 = bm[b0], m1 = bm[b1];
    const unsigned long long ci = wave_incl_scan(c0 + c1), mi = wave_incl_scan(m0 + m1);
    __syncthreads();
    if (lane_id() == 63) {
        L.h.scan[w] = ci;
        L.red.u[w] = mi;
    }
    __syncthreads();
    unsigned long long co = 0ull, mo = 0ull;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
        co += i < w ? L.h.scan[i] : 0ull;
        mo += i < w ? L.red.u[i] : 0ull;
    }
    const unsigned long long ce = co + ci - (c0 + c1), me = mo + mi - (m0 + m1);  // the bins above b0
    bc[b0] = (uint32_t)(ce + c0);
    bc[b1] = (uint32_t)(ce + c0 + c1);
    bm[b0] = me + m0;
    bm[b1] = me + m0 + m1;
    __syncthreads();
}

// The bin at which the weight from the highest bin down first reaches T >= 1, from the inclusive sums incl(b): each
// thread checks its two bins; the answer (-1 if the total is below T) and the weight above it go to slot q of
// L.qbin / L.qbefore, which start at -1.  Every thread gets the result.
template <class INCL>
__device__ __forceinline__ int sel_find_prefix(INCL&& incl, unsigned long long T, unsigned long long& before, int q,
                                               Lds& L) {
    const int b0 = kSelBins - 1 - 2 * (int)threadIdx.x;
#pragma unroll
    for (int d = 0; d < 2; ++d) {
        const int b = b0 - d;
        const unsigned long long hi = incl(b), lo = b + 1 < kSelBins ? incl(b + 1) : 0ull;
        if (lo < T && T <= hi) {
            L.qbin[q] = b;
            L.qbefore[q] = lo;
        }
    }
    __syncthreads();
    before = L.qbefore[q];
    return L.qbin[q];
}

// The value at descending rank r (0-based) of the set (the k-th value, the min_keep floor), NaN if unresolved; its
// bin stays sorted in L.ss (m elements), `above` = how many elements of the set exceed the value, f = the first
// position of the value in the sorted bin.
__device__ __forceinline__ float sel_rank_value(int r, int n, const SelBins& B, Lds& L, int q, int& m, int& f,
                                                unsigned long long& above) {
    unsigned long long before;
    const uint32_t* bc = L.ss.bcnt;  // counts summed from the highest bin down (sel_prefix)
    const int b = sel_find_prefix([&](int x) { return (unsigned long long)bc[x]; }, (unsigned long long)r + 1ull,
                                  before, q, L);
    m = -1;
    MIS_STAMP(22);
    if (b < 0) return __uint_as_float(0x7fc00000u);
    m = sel_sort_bin(b, n, B, L);
    MIS_STAMP(24);
    if (m < 0) return __uint_as_float(0x7fc00000u);
    const int p = (int)((unsigned long long)r - before);
    if (p >= m) return __uint_as_float(0x7fc00000u);
    const float v = L.ss.sq[p];
    int lo = 0, hi = p;  // first position of v (the bin is sorted, descending)
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (L.ss.sq[mid] > v)
            lo = mid + 1;
        else
            hi = mid;
    }
    f = lo;
    above = before + (unsigned long long)f;
    return v;
}

__device__ __forceinline__ bool fin_sel(const DevGroup& G, const Row& R, Lds& L, Outcome& out) {
    const int S = R.S, tid = threadIdx.x, w = wave_id(), l = lane_id();
    const int ntile = S * kWaves, nseg = ntile + S;  // tile segments (slice-major), then one specials segment per slice
    if (w == 0) {
        // records (lane s: slice s) and segment counts (lane l: segments [l * per, (l + 1) * per)); the draw's
        // uniform after their loads are issued
        float mq = -INFINITY, mqd = -INFINITY, gt = -INFINITY, mr = -INFINITY;
        double zz = 0.0, zcc = 0.0;
        int over = 0, notinf = 0;
        if (l < S) {
            const SliceRec* rec = (const SliceRec*)rec_base(G, R.row, l);
            mq = pub_ld(&rec->mq);
            mqd = pub_ld(&rec->mqd);
            gt = pub_ld(&rec->gate);
            mr = pub_ld(&rec->mref);
            zz = pub_ld(&rec->z);
            zcc = pub_ld(&rec->zc);
            const int fl = pub_ld(&rec->flags);
            over = (fl & kRecOverflow) ? 1 : 0;
            notinf = (fl & kRecGateInf) ? 0 : 1;
        }
        const int per = (nseg + 63) >> 6;
        int c[kSegs];
        int mine = 0;
#pragma unroll
        for (int t = 0; t < kSegs; ++t) {
            const int i = l * per + t;
            int v = 0;
            if (t < per && i < nseg) {
                const int s = i < ntile ? i / kWaves : i - ntile;
                const int sg = i < ntile ? i % kWaves : kWaves;
                v = pub_ld(&((const SliceRec*)rec_base(G, R.row, s))->ncand[sg]);
            }
            c[t] = v;
            mine += v;
        }
        const float u = row_uniform(G, R);
        const float m_sel = wave_reduce(mq, [](float a, float b) { return fmaxf(a, b); });
        const float m_draw = wave_reduce(mqd, [](float a, float b) { return fmaxf(a, b); });
        const float gate = wave_reduce(gt, [](float a, float b) { return fmaxf(a, b); });
        const float gmin = wave_reduce(l < S ? gt : INFINITY, [](float a, float b) { return fminf(a, b); });
        const int anyover = wave_reduce(over, [](int a, int b) { return max(a, b); });
        const int anyfin = wave_reduce(notinf, [](int a, int b) { return max(a, b); });
        double zs = 0.0, zcs = 0.0;
        if (R.needz) {
            const double sc = (mr > -INFINITY && m_sel > -INFINITY) ? exp((double)mr - (double)m_sel) : 0.0;
            zs = wave_sum(zz * sc);
            zcs = wave_sum(zcc * sc);
        }
        // a top-p row without top-k whose candidates weigh clearly less than top_p of the row cannot be cut among
        // them
        const int short_mass = (R.mode == kNucleus && R.p_active && zcs < (double)R.top_p * zs * (1.0 - 1e-6)) ? 1 : 0;
        const int incl = wave_incl_scan(mine);
        int o = incl - mine;
#pragma unroll
        for (int t = 0; t < kSegs; ++t) {
            const int i = l * per + t;
            if (t < per && i < nseg) L.segoff[i] = o;
            o += c[t];
        }
        if (l == 0) {
            L.segoff[nseg] = __builtin_amdgcn_readlane(incl, 63);
            L.fscratch[0] = m_sel;
            L.fscratch[1] = gate;
            L.fscratch[2] = u;
            L.fscratch[3] = gmin;
            L.dscratch[0] = zs;
            L.dscratch[2] = (double)m_draw;
            L.token = anyover | short_mass;
#pragma unroll
            for (int q = 0; q < 4; ++q) L.qbin[q] = -1;
            L.is_last = anyfin;
        }
    }
    __syncthreads();
    MIS_STAMP(26);
    const int n = L.segoff[nseg], na = L.segoff[ntile];
    const bool ginf = L.is_last == 0;  // every slice published all its finite elements
    if (L.token || n > kCapCand || n - na > kSelCap) return false;
    const float m_sel = L.fscratch[0], gate = L.fscratch[1], u = L.fscratch[2];
    const double zfull_fx = L.dscratch[0] * kFx;
    out.thr = -INFINITY;
    out.mdraw = -INFINITY;
    out.token = R.V - 1;
    if (n == 0) return ginf;
    // gather: every load issued at once (at most kCapCand / kThreads per thread), each candidate with its mass
    // relative to the row max
    constexpr int kPer = kCapCand / kThreads;
    unsigned long long v[kPer];
#pragma unroll
    for (int u4 = 0; u4 < kPer; ++u4) {
        const int i = u4 * kThreads + tid;
        v[u4] = 0ull;
        if (i < n) {
            int lo = 0, hi = nseg;  // segment: segoff[lo] <= i < segoff[lo + 1]
            while (hi - lo > 1) {
                const int mid = (lo + hi) >> 1;
                if (L.segoff[mid] <= i)
                    lo = mid;
                else
                    hi = mid;
            }
            const int s = lo < ntile ? lo / kWaves : lo - ntile;
            const int sg = lo < ntile ? lo % kWaves : kWaves;
            const unsigned long long* seg =
                (const unsigned long long*)(rec_base(G, R.row, s) + kRecCandOff) + (int64_t)sg * kCapWave;
            v[u4] = pub_ld(seg + (i - L.segoff[lo]));
        }
    }
    // every candidate lies in [min gate, m_sel] (a slice with no gate published all its finite values: then the
    // range comes from the values)
    float qlo = L.fscratch[3], qhi = m_sel;
    const bool need_lo = !(qlo > -INFINITY);
    float vlo = INFINITY;
#pragma unroll
    for (int u4 = 0; u4 < kPer; ++u4) {
        const int i = u4 * kThreads + tid;
        if (i >= n) continue;
        const float q = __uint_as_float((uint32_t)v[u4]);
        L.a.w.q[i] = q;
        L.a.w.id[i] = (uint32_t)(v[u4] >> 32);
        L.a.w.mass[i] = efx(q, m_sel);
        vlo = fminf(vlo, q);
    }
    if (need_lo) qlo = -block_max4(make_float4(-vlo, -INFINITY, -INFINITY, -INFINITY), L.red).x;
    MIS_STAMP(27);
    if (n <= 256) {
        // a small set: wave 0 sorts it in registers, selects and draws (no workgroup barrier between the steps)
        __syncthreads();
        if (w == 0) {
            const WSet ws = wset_of(L.a.w.q, L.a.w.id, L.a.w.mass, n);
            Outcome o;
            bool ok;
            if (n <= 64)
                ok = wsort_select_draw<1>(R, ws, m_sel, zfull_fx, gate, ginf, u, o);
            else if (n <= 128)
                ok = wsort_select_draw<2>(R, ws, m_sel, zfull_fx, gate, ginf, u, o);
            else
                ok = wsort_select_draw<4>(R, ws, m_sel, zfull_fx, gate, ginf, u, o);
            if (l == 0) {
                L.token = ok ? 1 : 0;
                L.fscratch[3] = o.thr;
                L.dscratch[1] = o.mdraw;
                L.uscratch[0] = (unsigned long long)o.token;
            }
        }
        __syncthreads();
        if (!L.token) return false;
        out.thr = L.fscratch[3];
        out.mdraw = (float)L.dscratch[1];
        out.token = (int64_t)L.uscratch[0];
        return true;
    }
    SelBins B;
    B.qmin = qlo;
    B.scale = qhi > qlo ? fminf((float)kSelBins / (qhi - qlo), 1e30f) : 0.0f;
    // counts and masses by bin
    uint32_t* bc = L.ss.bcnt;
    unsigned long long* bm = L.h.w;
    for (int b = tid; b < kSelBins; b += kThreads) {
        bc[b] = 0u;
        bm[b] = 0ull;
    }
    __syncthreads();
#pragma unroll
    for (int u4 = 0; u4 < kPer; ++u4) {
        const int i = u4 * kThreads + tid;
        if (i >= n) continue;
        const float q = __uint_as_float((uint32_t)v[u4]);
        const int b = sel_bin(q, B);
        atomicAdd(&bc[b], 1u);
        const unsigned long long ms = efx(q, m_sel);
        if (ms) atomicAdd(&bm[b], ms);
    }
    __syncthreads();
    sel_prefix(L);
    MIS_STAMP(16);
    const bool topk = R.kk < R.V;
    // the k-th value (engine/talker_sampler.py:95-98, :119-133): ties at it count once per rank
    float kth = -INFINITY;
    unsigned long long cnt_gt = (unsigned long long)n;
    int bk = -1, mk = 0, fk = 0;
    if (topk) {
        if (R.kk <= n) {
            kth = sel_rank_value(R.kk - 1, n, B, L, 0, mk, fk, cnt_gt);
            if (!(kth >= gate)) return false;  // NaN (unresolved) included
            bk = sel_bin(kth, B);              // its sorted elements stay in L.ss
        } else if (!ginf) {
            return false;
        }
    }
    MIS_STAMP(17);
    float thr = kth;
    if (R.p_active) {
        // weights: the mass of every value above kth, and kk - cnt_gt copies of kth's at its first rank (the ranks
        // it fills)
        const unsigned long long ekth = efx(kth, m_sel);
        const unsigned long long vw = (topk && kth > -INFINITY) ? ((unsigned long long)R.kk - cnt_gt) * ekth : 0ull;
        unsigned long long gtk = 0ull;  // bin bk's mass above kth: its first fk sorted elements
        if (bk >= 0) {
            unsigned long long mine = 0ull;
            if (tid < fk) mine = L.a.w.mass[(int)L.ss.sw[tid]];
            gtk = block_sum_u(mine, L.red);
        }
        // the weight from the highest bin down: the masses above bin bk, then bk's weight, then nothing
        const unsigned long long above_k = bk >= 0 ? (bk + 1 < kSelBins ? bm[bk + 1] : 0ull) : 0ull;
        auto wincl = [&](int b) -> unsigned long long {
            if (bk < 0 || b > bk) return bm[b];
            return above_k + gtk + vw;
        };
        // the normaliser: the top-k mass (omni order with top-k), else the whole row's
        double zn;
        if (topk && !R.hf)
            zn = (double)(bk >= 0 ? above_k + gtk + vw : bm[0]);
        else
            zn = zfull_fx;
        const double pt = ceil((double)R.top_p * zn);
        const unsigned long long T = pt < 1.0 ? 1ull : (unsigned long long)pt;
        unsigned long long before;
        const int bp = sel_find_prefix(wincl, T, before, 1, L);
        float thr_p;
        if (bp >= 0) {
            // the bin's elements by value with their weights (bin bk is sorted already)
            const int m = bp == bk ? mk : sel_sort_bin(bp, n, B, L);
            if (m < 0) return false;
            if (tid < m) {
                const int i = (int)L.ss.sw[tid];
                unsigned long long wgt = L.ss.sq[tid] > kth ? L.a.w.mass[i] : 0ull;
                if (bp == bk && tid == fk) wgt += vw;
                L.ss.sw[tid] = wgt;
            }
            const int r = sel_cross(m, before, T, L);  // its first barrier publishes the weights
            if (r < 0) return false;
            thr_p = L.ss.sq[r];
        } else {
            if (!topk) return false;  // the nucleus reaches below the candidates
            thr_p = kth;
        }
        if (!topk && !(thr_p >= gate)) return false;
        MIS_STAMP(18);
        float vmk = m_sel;
        if (R.min_keep_eff >= 2) {
            if (R.min_keep_eff > n) {
                vmk = -INFINITY;
            } else {
                int m2, f2;
                unsigned long long a2;
                vmk = sel_rank_value(R.min_keep_eff - 1, n, B, L, 2, m2, f2, a2);
                if (!(vmk >= gate)) return false;
            }
        }
        thr = fminf(thr_p, vmk);
        if (topk) thr = fmaxf(thr, kth);
    }
    MIS_STAMP(19);
    // survivors: drawable, q >= thr; masses relative to the largest of them, the row's largest drawable value (a
    // slice's largest drawable value is at or above its gate, so it is among the candidates, and thr is at or above
    // every gate)
    const uint32_t thrkey = ord_key(thr);
    const float m_draw = (float)L.dscratch[2];
    const float md = m_draw >= thr ? m_draw : -INFINITY;
    out.thr = thr;
    out.mdraw = md;
    if (!(md > -INFINITY)) return true;
    const bool md_is_m = md == m_sel;
    auto wsurv = [&](int i) -> unsigned long long {
        const float q = L.a.w.q[i];
        if (!(ord_key(q) >= thrkey) || (L.a.w.id[i] & kSelOnlyBit)) return 0ull;
        return md_is_m ? L.a.w.mass[i] : efx(q, md);
    };
    // the draw (engine/talker_sampler.py:161-172) in token order: the surviving specials (ids in their slices'
    // ranges, in any order) are ranked by id; thread t then walks tile candidates [t c, (t + 1) c) merged with the
    // specials whose ids fall between its first candidate and the next thread's (thread 0 from the lowest id, the
    // last thread with candidates to the highest), from the mass of everything before them
    MIS_STAMP(20);
    const int nb = n - na;
    uint32_t* bids = (uint32_t*)L.ss.cq;  // the surviving specials' ids, ascending
    unsigned long long* bw = L.ss.cw;     // their masses in that order
    const unsigned long long wsp = tid < nb ? wsurv(na + tid) : 0ull;
    const uint32_t sid = tid < nb ? (L.a.w.id[na + tid] & ~kSelOnlyBit) : 0u;
    if (tid == 0) {
        L.scnt = 0;
        L.uscratch[0] = ~0ull;
    }
    __syncthreads();
    const int slot = lds_reserve(wsp != 0ull, &L.scnt);
    if (wsp) {
        L.ss.bcnt[slot] = sid;
        L.ss.sw[slot] = wsp;
    }
    __syncthreads();
    const int nbs = L.scnt;
    unsigned long long* bpe = L.ss.sw;  // (after the ranking) the mass of the surviving specials of lower id
    int myr = -1;
    unsigned long long below = 0ull;
    if (tid < nbs) {
        const uint32_t myid = L.ss.bcnt[tid];
        const unsigned long long myw = L.ss.sw[tid];
        int r = 0;
        for (int j0 = 0; j0 < nbs; j0 += 8) {  // ids are distinct; eight read together
            uint32_t c[8];
            unsigned long long cw8[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                c[e] = L.ss.bcnt[min(j0 + e, nbs - 1)];
                cw8[e] = L.ss.sw[min(j0 + e, nbs - 1)];
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const bool lt = j0 + e < nbs && c[e] < myid;
                r += lt ? 1 : 0;
                below += lt ? cw8[e] : 0ull;
            }
        }
        bids[r] = myid;
        bw[r] = myw;
        myr = r;
    }
    __syncthreads();
    if (myr >= 0) bpe[myr] = below;
    const int cpt = (na + kThreads - 1) / kThreads;
    const int i0 = tid * cpt, i1 = min(na, i0 + cpt);
    unsigned long long own = 0ull;
    for (int i = i0; i < i1; ++i) own += wsurv(i);
    unsigned long long zsa;
    const unsigned long long exa = block_excl_scan(own, zsa, L.red.u);  // its barriers also publish bids, bw, bpe
    const unsigned long long zsb = nbs ? bpe[nbs - 1] + bw[nbs - 1] : 0ull;
    const unsigned long long zs = zsa + zsb;
    if (zs == 0ull) return true;
    const unsigned long long T2 = (unsigned long long)floor((double)u * (double)zs) + 1ull;
    MIS_STAMP(21);
    // this thread's stretch of token order: its candidates and the specials with ids in [lo_id, hi_id)
    const bool first_t = tid == 0, last_t = i1 >= na;
    if (i0 < i1 || (first_t && na == 0)) {
        const uint32_t lo_id = first_t ? 0u : (L.a.w.id[i0] & ~kSelOnlyBit);
        const uint32_t hi_id = last_t ? 0xffffffffu : (L.a.w.id[i1] & ~kSelOnlyBit);
        int p = 0;  // the first special with id >= lo_id
        {
            int hi = nbs;
            while (p < hi) {
                const int mid = (p + hi) >> 1;
                if (bids[mid] < lo_id)
                    p = mid + 1;
                else
                    hi = mid;
            }
        }
        unsigned long long c = exa + (p < nbs ? bpe[p] : zsb);  // and the specials before the stretch
        bool hit = false;
        uint32_t tok = 0u;
        auto step = [&](unsigned long long wgt, uint32_t id) {
            if (!hit && wgt && c < T2 && T2 <= c + wgt) {
                hit = true;
                tok = id;
            }
            c += wgt;
        };
        for (int i = i0; i < i1; ++i) {
            const uint32_t id = L.a.w.id[i] & ~kSelOnlyBit;
            for (; p < nbs && bids[p] < id; ++p) step(bw[p], bids[p]);
            step(wsurv(i), id);
        }
        for (; p < nbs && bids[p] < hi_id; ++p) step(bw[p], bids[p]);
        if (hit) L.uscratch[0] = tok;
    }
    MIS_STAMP(25);
    __syncthreads();
    MIS_STAMP(13);
    if (L.uscratch[0] == ~0ull) return false;
    out.token = (int64_t)L.uscratch[0];
    return true;
}

// Top-p rows without top-k on bf16 logits whose nucleus the candidates do not hold.  The cut comes from every
// slice's value counts and specials, as a weighted selection (one entry per value present with its count, one per
// special; the tiny-magnitude lumps as one element at 0 with their summed mass, which may not be where the cut
// falls).  Each slice's survivor mass follows from its counts; the draw streams the one slice that holds it.
// False: the row is streamed instead.
// 0: the row must be streamed; 1: no survivor; 2: the cut (out.thr, out.mdraw) for the second round.
__device__ __forceinline__ int fin_hist(const KernelArgs& A, const DevGroup& G, const Row& R, Lds& L,
                                        Outcome& out) {
    const int S = R.S, tid = threadIdx.x, w = wave_id(), l = lane_id();
    // the first four slices' counts, loaded ahead of the records (their addresses need nothing from them)
    constexpr int kMI = (kHistWords + kThreads - 1) / kThreads;
    uint32_t hv[kMI][4];
#pragma unroll
    for (int mi = 0; mi < kMI; ++mi) {
        const int i = mi * kThreads + tid;
#pragma unroll
        for (int u4 = 0; u4 < 4; ++u4)
            hv[mi][u4] = (i < kHistWords && u4 < S)
                             ? pub_ld((const uint32_t*)(rec_base(G, R.row, u4) + kRecHistOff) + i)
                             : 0u;
    }
    if (tid == kThreads - 64) L.fscratch[3] = row_uniform(G, R);  // the draw's, off wave 0's path
    if (w == 0) {  // lane s reads slice s's record
        float mq = -INFINITY, mqd = -INFINITY, mr = -INFINITY, hb = -INFINITY;
        double zz = 0.0;
        int bad = 0, nsp = 0, nall = 0;
        unsigned long long tf = 0ull;
        if (l < S) {
            const SliceRec* rec = (const SliceRec*)rec_base(G, R.row, l);
            mq = pub_ld(&rec->mq);
            mqd = pub_ld(&rec->mqd);
            mr = pub_ld(&rec->mref);
            zz = pub_ld(&rec->z);
            hb = pub_ld(&rec->gate);
            bad = (!pub_ld(&rec->hist) || (pub_ld(&rec->flags) & kRecOverflow)) ? 1 : 0;
            nall = pub_ld(&rec->nspec);
            nsp = pub_ld(&rec->nhigh);
            tf = pub_ld(&rec->tinyfx);
        }
        const float m = wave_reduce(mq, [](float a, float b) { return fmaxf(a, b); });
        const float md = wave_reduce(mqd, [](float a, float b) { return fmaxf(a, b); });
        const float hbm = wave_reduce(hb, [](float a, float b) { return fmaxf(a, b); });
        const int anybad = wave_reduce(bad, [](int a, int b) { return max(a, b); });
        // the mass left out of the counts, relative to the row max, in the counts' fixed point
        const double zr = wave_reduce((mr > -INFINITY && m > -INFINITY) ? zz * exp((double)mr - (double)m) : 0.0,
                                      [](double a, double b) { return a + b; });
        const int incl = wave_incl_scan(nsp);
        if (l < S) {
            L.segoff[l] = incl - nsp;
            L.slice_u[l] = tf;
            L.slice_n[l] = nall;
        }
        if (l == 0) {
            L.segoff[S] = __builtin_amdgcn_readlane(incl, 63);
            L.fscratch[0] = m;
            L.fscratch[1] = md;
            L.fscratch[2] = hbm;
            L.dscratch[0] = zr * kFx;
            L.token = anybad;
            L.nspec = 0;
        }
    }
    __syncthreads();
    if (L.token) return 0;
    const float m = L.fscratch[0], mdraw = L.fscratch[1], hbound = L.fscratch[2];
    const double zrest = L.dscratch[0];
    const int ntot = L.segoff[S];
    out.thr = -INFINITY;
    out.mdraw = -INFINITY;
    out.token = R.V - 1;
    if (!(m > -INFINITY)) return 1;
    // md to the waiting slices, which build their mass tables while the cut is settled here
    if (S > 1 && mdraw > -INFINITY) r2_decide(A, R, 3u, 0.f, mdraw, 0.f, 0.f);
    // every slice's counts, merged
    uint32_t* cnt = (uint32_t*)L.h.w;
#pragma unroll
    for (int mi = 0; mi < kMI; ++mi) {
        const int i = mi * kThreads + tid;
        uint32_t a = 0u, b = 0u;
#pragma unroll
        for (int u4 = 0; u4 < 4; ++u4) {
            a += hv[mi][u4] & 0xffffu;
            b += hv[mi][u4] >> 16;
        }
        for (int s0 = 4; s0 < S; s0 += 4) {
            uint32_t v[4];
#pragma unroll
            for (int u4 = 0; u4 < 4; ++u4)
                v[u4] = (i < kHistWords && s0 + u4 < S)
                            ? pub_ld((const uint32_t*)(rec_base(G, R.row, s0 + u4) + kRecHistOff) + i)
                            : 0u;
#pragma unroll
            for (int u4 = 0; u4 < 4; ++u4) {
                a += v[u4] & 0xffffu;
                b += v[u4] >> 16;
            }
        }
        if (i < kHistWords) {
            cnt[2 * i] = a;
            cnt[2 * i + 1] = b;
        }
    }
    MIS_STAMP(22);
    // the value of every key (a lump takes the value of the exact key below it, so the table is monotone)
    char* const abase = (char*)&L.a;
    unsigned long long* mo = (unsigned long long*)abase;  // per key: mass of the specials strictly above its value
    uint32_t* co = (uint32_t*)(abase + 8 * (kKeys + 1));   // ... and their count
    float* qt = (float*)(abase + 12 * (kKeys + 1));
    for (int k = tid; k < kKeys; k += kThreads) {
        const int ke = key_exact(k) ? k : k - 1;
        qt[k] = ke >= 1 ? to_q<2>(R, key_bf(ke)) : -INFINITY;
        mo[k] = 0ull;
        co[k] = 0u;
    }
    __syncthreads();
    const uint32_t nlump = cnt[kKeyZero - 1] + cnt[kKeyZero + 1];
    if (cnt[kKeys - 1] != 0u) return 0;  // values of 256 and above are not resolved here
    // every special into the bin its slice found for it: the even bin of the exact key holding its value (counted
    // with that key), or the odd bin strictly between that key and the next exact one
    auto spec_at = [&](int i, unsigned long long& e, int& bin) {
        int lo = 0, hi = S;  // segoff[lo] <= i < segoff[lo + 1]
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (L.segoff[mid] <= i)
                lo = mid;
            else
                hi = mid;
        }
        const char* rb = rec_base(G, R.row, lo);
        const int o = i - L.segoff[lo];
        e = pub_ld((const unsigned long long*)(rb + kRecSpecOff) + o);
        bin = (int)pub_ld((const uint32_t*)(rb + kRecSpecBinOff) + o) - 1;
    };
    for (int i0 = 0; i0 < ntot; i0 += 4 * kThreads) {
        unsigned long long e[4];
        int bn[4];
#pragma unroll
        for (int u4 = 0; u4 < 4; ++u4) {
            const int i = i0 + u4 * kThreads + tid;
            e[u4] = 0ull;
            bn[u4] = -1;
            if (i < ntot) spec_at(i, e[u4], bn[u4]);
        }
#pragma unroll
        for (int u4 = 0; u4 < 4; ++u4) {
            const float q = __uint_as_float((uint32_t)e[u4]);
            if (i0 + u4 * kThreads + tid >= ntot || !(q > -INFINITY)) continue;
            const int b = bn[u4];
            if (b < 0) {
                atomicAdd(&co[0], 1u);  // below every key: ranks last, weighs nothing at these magnitudes
            } else if (b & 1) {
                atomicAdd(&mo[b >> 1], efx(q, m));
                atomicAdd(&co[b >> 1], 1u);
            } else {
                atomicAdd(&cnt[b >> 1], 1u);
            }
        }
    }
    MIS_STAMP(23);
    unsigned long long tiny0 = 0ull;
    for (int s = 0; s < S; ++s) tiny0 += L.slice_u[s];
    const unsigned long long lump_m = nlump ? (unsigned long long)((double)tiny0 * exp(-(double)m)) : 0ull;
    __syncthreads();
    // even-bin mass and count of key k (the tiny lumps' mass sits with the positive lump)
    auto even_mass = [&](int k) -> unsigned long long {
        if (key_exact(k)) return cnt[k] ? (unsigned long long)cnt[k] * efx(qt[k], m) : 0ull;
        return k == kKeyZero + 1 ? lump_m : 0ull;
    };
    // keys whose bins hold a lump, or the specials beside one (both tiny lumps' mass sits with the positive one):
    // their order is not resolved here
    auto near_lump = [&](int k) { return k == 0 || (nlump && k >= kKeyZero - 2 && k <= kKeyZero + 1); };
    // one descending pass over the keys: thread t holds keys kKeys - 1 - 4 t .. - 3; the first bin (odd bin of k,
    // then its even bin) at which the cumulative weight reaches T (T0, or with frac > 0 the target ceil(frac * total),
    // at least 1); false when the total is below T
    auto scan_cut = [&](unsigned long long T0, double frac, bool by_mass, int& key_out, bool& odd_out,
                        unsigned long long& before_out, unsigned long long& T_out) -> bool {
        unsigned long long wsum = 0ull;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const int k = kKeys - 1 - (4 * tid + d);
            if (k >= 0) wsum += by_mass ? mo[k] + even_mass(k) : (unsigned long long)co[k] + cnt[k];
        }
        unsigned long long tot;
        const unsigned long long ex = block_excl_scan(wsum, tot, L.red.u);
        unsigned long long T = T0;
        if (frac > 0.0) {
            const double pt = ceil(frac * ((double)tot + zrest));
            T = pt < 1.0 ? 1ull : (unsigned long long)pt;
        }
        T_out = T;
        if (tid == 0) L.token = -1;
        __syncthreads();
        if (ex < T && T <= ex + wsum) {
            unsigned long long c = ex;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const int k = kKeys - 1 - (4 * tid + d);
                if (k < 0) break;
                const unsigned long long wo = by_mass ? mo[k] : co[k];
                const unsigned long long we = by_mass ? even_mass(k) : cnt[k];
                if (c + wo >= T) {
                    L.token = 2 * k + 1;
                    L.uscratch[1] = c;
                    break;
                }
                c += wo;
                if (c + we >= T) {
                    L.token = 2 * k;
                    L.uscratch[1] = c;
                    break;
                }
                c += we;
            }
        }
        __syncthreads();
        const int b = L.token;
        before_out = L.uscratch[1];
        __syncthreads();
        if (b < 0) return 0;
        key_out = b >> 1;
        odd_out = (b & 1) != 0;
        return 1;
    };
    // the value at which the cumulative weight reaches T inside odd bin k: its specials sorted by value
    // (descending), walked from `before`; NaN when it cannot be resolved here
    auto resolve_odd = [&](int k, unsigned long long T, unsigned long long before, bool by_mass) -> float {
        float* rq = (float*)(abase + 16 * (kKeys + 1));
        unsigned long long* rm = (unsigned long long*)(abase + 16 * (kKeys + 1) + 4 * 256);
        if (tid == 0) L.scnt = 0;
        __syncthreads();
        for (int i0 = 0; i0 < ntot; i0 += kThreads) {
            const int i = i0 + tid;
            float q = -INFINITY;
            int b = -1;
            if (i < ntot) {
                unsigned long long e;
                spec_at(i, e, b);
                q = __uint_as_float((uint32_t)e);
            }
            const bool in = q > -INFINITY && b == 2 * k + 1;
            const int slot = lds_reserve(in, &L.scnt);
            if (in && slot < 256) {
                rq[slot] = q;
                rm[slot] = by_mass ? efx(q, m) : 1ull;
            }
        }
        __syncthreads();
        const int n = L.scnt;
        if (n > 256) return __uint_as_float(0x7fc00000u);
        if (wave_id() == 0) {
            unsigned long long v[4];
#pragma unroll
            for (int p4 = 0; p4 < 4; ++p4) {
                const int i = p4 * 64 + lane_id();
                v[p4] = i < n ? (((unsigned long long)(~ord_key(rq[i]))) << 32) | (unsigned long long)i : ~0ull;
            }
            wave_bitonic<4>(v);
            unsigned long long c = before;
            int hit = -1;
#pragma unroll
            for (int p4 = 0; p4 < 4; ++p4) {
                const int i = (int)(v[p4] & 0xffffffffull);
                const unsigned long long wgt = v[p4] != ~0ull ? rm[i] : 0ull;
                const unsigned long long incl = wave_incl_scan(wgt) + c;
                const uint64_t h = ballot(v[p4] != ~0ull && incl >= T);
                if (hit < 0 && h) hit = (int)__builtin_amdgcn_readlane((int)(v[p4] & 0xffffffffull), __ffsll((long long)h) - 1);
                c = __builtin_amdgcn_readlane((uint32_t)incl, 63) | ((unsigned long long)__builtin_amdgcn_readlane((uint32_t)(incl >> 32), 63) << 32);
            }
            if (lane_id() == 0) L.fscratch[2] = hit >= 0 ? rq[hit] : __uint_as_float(0x7fc00000u);
        }
        __syncthreads();
        const float r = L.fscratch[2];
        __syncthreads();
        return r;
    };
    // the top-p cut (engine/talker_sampler.py:87-92 through fixed-point masses: the target is top_p of the total
    // mass of every value in the row) and the min_keep floor
    int ck;
    bool codd;
    unsigned long long cbef, T, Tk;
    MIS_STAMP(12);
    if (!scan_cut(0ull, (double)R.top_p, true, ck, codd, cbef, T)) return 0;
    if (near_lump(ck)) return 0;
    const float thr_p = codd ? resolve_odd(ck, T, cbef, true) : qt[ck];
    if (!(thr_p > hbound)) return 0;  // the cut is not above every value the slices left out (or unresolved)
    float vmk = m;
    if (R.min_keep_eff >= 2) {
        if (scan_cut((unsigned long long)R.min_keep_eff, 0.0, false, ck, codd, cbef, Tk)) {
            if (near_lump(ck)) return 0;
            vmk = codd ? resolve_odd(ck, (unsigned long long)R.min_keep_eff, cbef, false) : qt[ck];
            if (!(vmk > hbound)) return 0;
        } else {
            vmk = -INFINITY;
        }
    }
    const float thr = fminf(thr_p, vmk);
    if (!(thr > hbound)) return 0;
    const float md = mdraw >= thr ? mdraw : -INFINITY;
    out.thr = thr;
    out.mdraw = md;
    MIS_STAMP(13);
    return md > -INFINITY ? 2 : 1;
}

// Greedy rows: the first argmax over the slices' maxima.  False when a slice's history ids overflowed its list of
// specials (some of its values went unpenalised): the row is then streamed.
__device__ __forceinline__ bool fin_greedy(const DevGroup& G, const Row& R, Lds& L, Outcome& out) {
    float v = -INFINITY;
    int idx = INT_MAX;
    bool over = false;
    if ((int)threadIdx.x < R.S) {
        const SliceRec* rec = (const SliceRec*)rec_base(G, R.row, threadIdx.x);
        v = pub_ld(&rec->mqd);
        idx = pub_ld(&rec->argmax);
        over = (pub_ld(&rec->flags) & kRecOverflow) != 0;
    }
    if (wave_id() == 0) {  // R.S <= 64: every slice on wave 0
        const uint64_t b = ballot(over);
        if (lane_id() == 0) L.token = b != 0;
    }
    block_argmax(v, idx, L.red);  // its barriers publish L.token
    if (L.token) return false;
    out.token = v > -INFINITY ? idx : 0;
    out.thr = -INFINITY;
    out.mdraw = v;
    return true;
}

// Unfiltered rows: walk the slices' totals, then the chosen slice's sub-block sums, to the sub-block holding
// u * Z, and rescan it element by element.
__device__ __forceinline__ double readlane_d(double x, int lane) {
    return __longlong_as_double((long long)readlane_u64((unsigned long long)__double_as_longlong(x), lane));
}

// Unfiltered rows: the slice that holds the target (from the slices' sums of exp), its sub-block (from the slice's
// sub-block sums), both on wave 0 without a workgroup barrier; then the sub-block's elements, one per thread, and the
// token from their masses on wave 0.  False (the row is streamed) when a slice's history ids overflowed its list of
// specials.
__device__ __forceinline__ bool fin_full(const DevGroup& G, const Row& R, Lds& L, Outcome& out) {
    const int E = 16 / G.es;
    const int nsb = kWaves * G.R;
    const int tid = threadIdx.x, l = lane_id();
    if (wave_id() == 0) {
        float mr = -INFINITY;
        double z = 0.0;
        bool over = false;
        if (l < R.S) {  // lane s: slice s
            const SliceRec* rec = (const SliceRec*)rec_base(G, R.row, l);
            mr = pub_ld(&rec->mref);
            z = pub_ld(&rec->z);
            over = (pub_ld(&rec->flags) & kRecOverflow) != 0;
        }
        const bool anyover = ballot(over) != 0;
        const float u = row_uniform(G, R);
        const float m = wave_reduce(mr, [](float a, float b) { return fmaxf(a, b); });
        const double sc = (mr > -INFINITY && m > -INFINITY) ? exp((double)mr - (double)m) : 0.0;
        const double zsl = z * sc;
        const double incl = wave_incl_scan(zsl);
        const double t = (double)u * readlane_d(incl, 63);
        const uint64_t hs = ballot(l < R.S && incl > t), hm = ballot(l < R.S && zsl > 0.0);
        // the first slice whose inclusive sum passes t, else (rounding) the last with mass
        const int ss = hs ? __ffsll((long long)hs) - 1 : (hm ? 63 - __clzll((long long)hm) : -1);
        int kb = -1;
        double rem2 = 0.0;
        float mref = -INFINITY;
        if (ss >= 0 && m > -INFINITY) {
            const double sc_s = readlane_d(sc, ss), zs = readlane_d(zsl, ss);
            const double rem = fmin((t - (readlane_d(incl, ss) - zs)) / sc_s, zs / sc_s);  // in the slice's units
            const SliceRec* rec = (const SliceRec*)rec_base(G, R.row, ss);
            mref = pub_ld(&rec->mref);
            const double* sbg = (const double*)((const char*)rec + kRecSbOff);
            const double v0 = l < nsb ? pub_ld(sbg + l) : 0.0;
            const double v1 = 64 + l < nsb ? pub_ld(sbg + 64 + l) : 0.0;
            const double i0 = wave_incl_scan(v0);
            const double i1 = wave_incl_scan(v1) + readlane_d(i0, 63);
            const uint64_t h0 = ballot(l < nsb && i0 > rem), h1 = ballot(64 + l < nsb && i1 > rem);
            const uint64_t g0 = ballot(l < nsb && v0 > 0.0), g1 = ballot(64 + l < nsb && v1 > 0.0);
            if (h0 || h1) {
                kb = h0 ? __ffsll((long long)h0) - 1 : 64 + __ffsll((long long)h1) - 1;
            } else if (g0 || g1) {  // rounding: the last sub-block with mass
                kb = g1 ? 64 + 63 - __clzll((long long)g1) : 63 - __clzll((long long)g0);
            }
            if (kb >= 0) {
                const double ik = kb < 64 ? readlane_d(i0, kb) : readlane_d(i1, kb - 64);
                const double vk = kb < 64 ? readlane_d(v0, kb) : readlane_d(v1, kb - 64);
                rem2 = rem - (ik - vk);
            }
        }
        if (l == 0) {
            L.token = anyover ? -2 : (kb >= 0 ? ss : -1);
            L.scnt = kb;
            L.dscratch[2] = rem2;
            L.fscratch[0] = m;
            L.fscratch[1] = mref;
        }
    }
    __syncthreads();
    const int ss = L.token, kb = L.scnt;
    const double rem = L.dscratch[2];
    const float m = L.fscratch[0], mref = L.fscratch[1];
    if (ss == -2) return false;
    out.thr = -INFINITY;
    out.mdraw = m;
    out.token = R.V - 1;
    if (!(m > -INFINITY) || ss < 0) return true;
    const int slo = ss * G.slice_len, shi = min(R.V, slo + G.slice_len);
    const int first = slice_first(G, R.row, slo);
    Visit V;
    V.weighted = false;
    V.src = kSrcRow;
    V.n = 0;
    V.lo = max(slo, first + kb * 64 * E);
    V.hi = min(shi, first + (kb + 1) * 64 * E);
    V.job = kJobPick;
    V.m = mref;
    V.d0 = 0.0;
    V.i0 = -1;
    visit(V, G, R, L);  // ends with a barrier
    // the sub-block's masses in element order (at most 512), then the token on wave 0: lane l sums elements
    // [8 l, 8 l + 8)
    double* pe = (double*)L.h.w;
    if (tid < 512) pe[tid] = (V.i0 >= 0) ? V.d0 : 0.0;
    if (tid == 0) L.uscratch[0] = ~0ull;
    __syncthreads();
    if (wave_id() == 0) {
        const int nel = V.hi - V.lo;
        double e8[8], own = 0.0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            e8[e] = 8 * l + e < nel ? pe[8 * l + e] : 0.0;
            own += e8[e];
        }
        const double incl = wave_incl_scan(own);
        const uint64_t hit = ballot(own > 0.0 && incl > rem);
        const uint64_t any = ballot(own > 0.0);
        const int hl = hit ? __ffsll((long long)hit) - 1 : (any ? 63 - __clzll((long long)any) : -1);
        if (l == hl) {
            double c = incl - own;
            int pick = -1;
            for (int e = 0; e < 8; ++e) {
                if (!(e8[e] > 0.0)) continue;
                pick = e;
                c += e8[e];
                if (hit && c > rem) break;  // else (rounding) the last with mass
            }
            if (pick >= 0) L.uscratch[0] = (unsigned long long)(V.lo + 8 * l + pick);
        }
    }
    __syncthreads();
    if (L.uscratch[0] != ~0ull) out.token = (int64_t)L.uscratch[0];
    return true;
}

// Processed logits and probabilities of the whole row (parity outputs), streamed.
__device__ __forceinline__ void write_outputs(const DevGroup& G, const Row& R, Lds& L, const Outcome& o, bool forced) {
    const gptr<float> prow = G.processed ? gp(G.processed) + (int64_t)R.row * G.processed_stride : nullptr;
    const gptr<float> qrow = G.probs ? gp(G.probs) + (int64_t)R.row * G.probs_stride : nullptr;
    if (forced) {
        for (int j = threadIdx.x; j < R.V; j += kThreads) {
            const bool e = j == G.eos;
            if (prow) prow[j] = e ? 0.0f : -INFINITY;
            if (qrow) qrow[j] = e ? 1.0f : 0.0f;
        }
        return;
    }
    Visit V;
    V.weighted = false;
    V.src = kSrcRow;
    V.n = 0;
    V.lo = 0;
    V.hi = R.V;
    V.thr = o.thr;
    V.md = o.mdraw;
    V.prow = prow;
    V.qrow = qrow;
    V.d0 = 0.0;
    double z = 0.0;
    if (qrow && o.mdraw > -INFINITY) {
        V.job = kJobOutZ;
        visit(V, G, R, L);
        z = block_sum_d(V.d0, L.red);
    }
    V.inv = (float)(1.0 / z);
    V.job = kJobOut;
    visit(V, G, R, L);
}

// tokens[row]; for live rows with MIS_UPDATE_STATE: history append, steps + 1, finished |= (token == eos).
__device__ __forceinline__ void update_state(const DevGroup& G, const Row& R, int64_t tok) {
    if (!(G.flags & MIS_UPDATE_STATE) || !R.live) {
        if (threadIdx.x == 0 && G.tokens) gp(G.tokens)[R.row] = R.live ? tok : (int64_t)kPad;
        return;
    }
    if (G.history && G.hist_len > 0) {
        const int W = G.hist_len;
        char* hrow = (char*)hist_row(G, R.row);
        if (G.hist_mode == MIS_HISTORY_RING) {
            if (threadIdx.x == 0) {
                const int pos = (int)((gp(G.hist_head)[R.row] % W + W) % W);
                if (G.hist_i64)
                    gp((int64_t*)hrow)[pos] = tok;
                else
                    gp((int32_t*)hrow)[pos] = (int32_t)tok;
                gp(G.hist_head)[R.row] = (pos + 1) % W;
            }
        } else {
            // shift left by one and append: each round reads [b + 1, b + 1024] before writing [b, b + 1024)
            for (int b = 0; b < W; b += kThreads) {
                const int j = b + (int)threadIdx.x;
                int64_t nxt = 0;
                if (j < W) {
                    if (j + 1 < W)
                        nxt = G.hist_i64 ? gp((const int64_t*)hrow)[j + 1] : (int64_t)gp((const int32_t*)hrow)[j + 1];
                    else
                        nxt = tok;
                }
                __syncthreads();
                if (j < W) {
                    if (G.hist_i64)
                        gp((int64_t*)hrow)[j] = nxt;
                    else
                        gp((int32_t*)hrow)[j] = (int32_t)nxt;
                }
                __syncthreads();
            }
        }
    }
    if (threadIdx.x == 0) {
        if (G.tokens) gp(G.tokens)[R.row] = tok;
        if (G.steps) gp(G.steps)[R.row] = R.step + 1;
        if (G.finished && tok == (int64_t)G.eos) gp(G.finished)[R.row] = 1;
    }
}

// The row's last workgroup (or slice 0 of a forced row).
__device__ __forceinline__ void finalize(const DevGroup& G, const Row& R, Lds& L, bool forced) {
    Outcome o;
    o.token = forced ? (int64_t)G.eos : 0;
    o.thr = -INFINITY;
    o.mdraw = -INFINITY;
    int path = MIS_PATH_FORCED;
    MIS_STAMP(7);

    if (!forced) {
        int mode = L.foreign ? kStream : R.mode;
        if (mode == kGreedy) {
            path = MIS_PATH_GREEDY;
            if (!fin_greedy(G, R, L, o)) mode = kStream;
        } else if (mode == kFull) {
            path = MIS_PATH_FULL;
            if (!fin_full(G, R, L, o)) mode = kStream;
        } else if (mode == kTopK || mode == kNucleus) {
            path = MIS_PATH_CANDIDATES;
            if (!fin_sel(G, R, L, o)) mode = kStream;
            MIS_STAMP(8);
        }
        if (mode == kStream) {
            fin_stream(G, R, L, o);
            path = MIS_PATH_STREAM;
            MIS_STAMP(10);
        }
    }
    if (threadIdx.x == 0 && G.paths) atomicAdd(G.paths + path, 1u);
    if (R.want_out) write_outputs(G, R, L, o, forced);
    update_state(G, R, o.token);
    MIS_STAMP(11);
    MIS_STAMP_INFO(((unsigned long long)(R.grow + 1) << 32) | ((unsigned long long)R.slice << 8) | 0x80u |
                   (unsigned)path);
}

__device__ __forceinline__ bool locate(const KernelArgs& A, int& gi, int& row, int& slice) {
    const int x = blockIdx.x % 8;
    int i = blockIdx.x / 8;
    for (gi = 0; gi < A.n_groups; ++gi) {
        const int S = A.g[gi].S;
        const int n = A.seg_rows[x][gi] * S;
        if (i < n) {
            row = A.seg_row[x][gi] + i / S;
            slice = i % S;
            return true;
        }
        i -= n;
    }
    return false;
}

__global__ __launch_bounds__(kThreads) void sample_kernel(const KernelArgs args) {
    (void)args;
    MIS_STAMP(0);
    // the arguments read in place from the kernarg segment: a by-value copy indexed by group would live in scratch
    const KernelArgs& A = *(const KernelArgs*)__builtin_amdgcn_kernarg_segment_ptr();
    __shared__ Lds L;
    int gi, row, slice;
    if (!locate(A, gi, row, slice)) return;
    const DevGroup& G = A.g[gi];
    Row R;
    const int act = G.es == 2 ? run<2>(A, G, gi, row, slice, L, R) : run<4>(A, G, gi, row, slice, L, R);
    if (act != kActNone) {
        if (act == kActForced) L.foreign = 0;
        if (act == kActStream) L.foreign = 1;  // finalised from the logits alone
        finalize(G, R, L, act == kActForced);
    }
}

__global__ void uniform_kernel(const int64_t* seeds, const int64_t* steps, const int64_t* rids, int64_t n, int rng,
                               float* out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int64_t s = seeds ? seeds[i] : 0, t = steps ? steps[i] : 0;
    out[i] = rng == MIS_RNG_PHILOX ? philox_uniform(s, t, rids ? rids[i] : 0) : counter_uniform(s, t);
}

// ------------------------------------------------------------------ host side

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

// The workspace of mis_sample_static: a file-scope device array, so that callers that cannot allocate (code under
// graph capture, serving loops) need not.  Every GPU the library runs on holds its own copy, zero when the code
// object loads, until the process ends; each launch leaves its arrival words zero again, so the next call on that
// GPU starts clean.  Host code uses the per-device address from hipGetSymbolAddress, never the array's name.
constexpr size_t kStaticWsBytes = (size_t)MIS_STATIC_WORKSPACE_BYTES;
__device__ __align__(256) unsigned char scratch[kStaticWsBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch` (looked up once per device, with that device current).
int static_workspace(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(-1, "hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return fail(MIS_E_UNSUPPORTED, "device %d: at most %d devices", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) return fail(-1, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return 0;
}

struct Plan {
    int S, R, slice_len;
};

// Slices per row: one workgroup per row when the row is small, otherwise enough slices to give the launch about
// one workgroup per CU, each holding at most 40 elements per thread.
Plan plan_group(const MisGroup& g, int rows_total) {
    const int es = g.dtype == MIS_BF16 ? 2 : 4;
    const int E = 16 / es;
    const int rmax = kRounds;
    auto len_of = [&](int r) { return kThreads * E * r - E; };
    Plan p;
    if ((int64_t)g.vocab * es <= 48 * 1024) {
        p.S = 1;
        p.R = std::max(1, (g.vocab + E + kThreads * E - 1) / (kThreads * E));
        p.slice_len = len_of(p.R);
        return p;
    }
    const int s_min = (g.vocab + len_of(rmax) - 1) / len_of(rmax);
    const int target = std::max(1, (256 + std::max(rows_total, 1) - 1) / std::max(rows_total, 1));
    int S = std::max(s_min, target);
    int R = (int)std::min<int64_t>(rmax, std::max<int64_t>(1, ((g.vocab + S - 1) / S + E + kThreads * E - 1) /
                                                                  (kThreads * E)));
    p.R = R;
    p.slice_len = len_of(R);
    p.S = (g.vocab + p.slice_len - 1) / p.slice_len;
    return p;
}

int check_group(const MisGroup& g, int idx) {
    if (!g.logits && g.rows > 0) return fail(MIS_E_ARG, "group %d: logits is NULL", idx);
    if (g.dtype != MIS_F32 && g.dtype != MIS_BF16) return fail(MIS_E_ARG, "group %d: unknown dtype %d", idx, g.dtype);
    if (g.vocab < 1) return fail(MIS_E_ARG, "group %d: vocab must be >= 1 (got %d)", idx, g.vocab);
    if (g.vocab > kMaxVocab) return fail(MIS_E_UNSUPPORTED, "group %d: vocab %d exceeds %d", idx, g.vocab, kMaxVocab);
    if (g.rows < 0) return fail(MIS_E_ARG, "group %d: rows must be >= 0", idx);
    if (g.logits_row_stride < g.vocab) return fail(MIS_E_ARG, "group %d: logits row stride < vocab", idx);
    if (g.semantics != MIS_OMNI && g.semantics != MIS_HF)
        return fail(MIS_E_ARG, "unknown Talker sampling semantics: %d", g.semantics);
    if (g.min_keep < 1) return fail(MIS_E_ARG, "group %d: min_keep must be >= 1", idx);
    if (g.rng != MIS_RNG_COUNTER && g.rng != MIS_RNG_PHILOX) return fail(MIS_E_ARG, "unknown RNG mode: %d", g.rng);
    if (g.history_len < 0 || g.history_len > 65535)
        return fail(MIS_E_ARG, "group %d: history_len must be in [0, 65535]", idx);
    if (g.history_len > 0 && g.history) {
        if (g.history_row_stride < g.history_len)
            return fail(MIS_E_ARG, "group %d: history row stride < history_len", idx);
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
    if (g.processed && g.processed_row_stride < g.vocab)
        return fail(MIS_E_ARG, "group %d: processed stride < vocab", idx);
    if (g.probs && g.probs_row_stride < g.vocab) return fail(MIS_E_ARG, "group %d: probs stride < vocab", idx);
    return 0;
}

int rows_total_of(const MisGroup* groups, int n_groups) {
    int64_t t = 0;
    for (int i = 0; i < n_groups; ++i) t += std::max(0, groups[i].rows);
    return (int)std::min<int64_t>(t, INT_MAX);
}

int64_t records_bytes(const MisGroup& g, int rows_total) {
    const Plan p = plan_group(g, rows_total);
    if (p.S > kMaxSlices) return -1;
    return (int64_t)g.rows * p.S * kRecBytes;
}

}  // namespace
}  // namespace mis

using namespace mis;

extern "C" {

int mis_version(void) { return MIS_ABI_VERSION; }

const char* mis_last_error(void) { return g_err.c_str(); }

size_t mis_sizeof_group(void) { return sizeof(MisGroup); }

size_t mis_workspace_bytes(const MisGroup* groups, int n_groups) {
    if (!groups || n_groups < 1 || n_groups > kMaxGroups) return 0;
    const int rows_total = rows_total_of(groups, n_groups);
    if (rows_total > kMaxRows) return 0;
    size_t total = (size_t)kHeaderBytes + (size_t)kArriveBytes;
    for (int i = 0; i < n_groups; ++i) {
        if (check_group(groups[i], i)) return 0;
        const int64_t b = records_bytes(groups[i], rows_total);
        if (b < 0) return 0;
        total += (size_t)b;
    }
    return (total + 255) & ~(size_t)255;
}

int mis_sample(const MisGroup* groups, int n_groups, void* workspace, size_t workspace_bytes, void* stream) {
    g_err.clear();
    if (!groups || n_groups < 1 || n_groups > kMaxGroups)
        return fail(MIS_E_ARG, "n_groups must be in [1, %d]", kMaxGroups);
    const int rows_total = rows_total_of(groups, n_groups);
    if (rows_total > kMaxRows) return fail(MIS_E_UNSUPPORTED, "more than %d rows in one launch", kMaxRows);
    KernelArgs a;
    memset(&a, 0, sizeof a);
    a.n_groups = n_groups;
    size_t off = (size_t)kHeaderBytes + (size_t)kArriveBytes;
    int row_begin = 0;
    int64_t blocks = 0;
    for (int i = 0; i < n_groups; ++i) {
        const MisGroup& g = groups[i];
        if (int rc = check_group(g, i)) return rc;
        const Plan p = plan_group(g, rows_total);
        if (p.S > kMaxSlices)
            return fail(MIS_E_UNSUPPORTED, "group %d: vocab %d needs %d slices (at most %d)", i, g.vocab, p.S, kMaxSlices);
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
        d.zero64 = 0;
        d.one32 = 1u;
        d.alpha_lut = g.alpha_lut_len > 0 ? g.alpha_lut : nullptr;
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
        d.S = p.S;
        d.R = p.R;
        d.slice_len = p.slice_len;
        d.row_begin = row_begin;
        d.recs = (char*)workspace + off;
        d.paths = (uint32_t*)((char*)workspace + MIS_WS_PATH_OFFSET);
        off += (size_t)g.rows * p.S * kRecBytes;
        row_begin += g.rows;
        blocks += (int64_t)g.rows * p.S;
    }
    off = (off + 255) & ~(size_t)255;
    if (blocks > 0 && (!workspace || off > workspace_bytes))
        return fail(MIS_E_WORKSPACE, "workspace too small: need %zu bytes, got %zu", off, workspace_bytes);
    if (blocks == 0) return 0;
    a.arrive = (char*)workspace + kHeaderBytes;
    // whole rows to XCDs: contiguous in (group, row) order, balanced by slice count
    int64_t count[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int64_t prefix = 0;
    for (int gi = 0; gi < n_groups; ++gi) {
        const int S = a.g[gi].S;
        for (int r = 0; r < groups[gi].rows; ++r) {
            const int x = (int)std::min<int64_t>(7, ((prefix + S / 2) * 8) / blocks);
            if (a.seg_rows[x][gi] == 0) a.seg_row[x][gi] = r;
            ++a.seg_rows[x][gi];
            count[x] += S;
            prefix += S;
        }
    }
    const int64_t per_xcd = *std::max_element(count, count + 8);
    const int64_t grid = per_xcd * 8;
    if (grid > INT32_MAX) return fail(MIS_E_UNSUPPORTED, "too many rows");
    hipLaunchKernelGGL(sample_kernel, dim3((unsigned)grid), dim3(kThreads), 0, (hipStream_t)stream, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(-1, "launch failed: %s", hipGetErrorString(e));
    return 0;
}

int mis_sample_static(const MisGroup* groups, int n_groups, void* stream) {
    g_err.clear();
    const size_t need = mis_workspace_bytes(groups, n_groups);
    if (need == 0) return mis_sample(groups, n_groups, nullptr, 0, stream);  // reports the argument error
    if (need > kStaticWsBytes)
        return fail(MIS_E_WORKSPACE, "these groups need %zu bytes of workspace; the static workspace holds %zu", need,
                    kStaticWsBytes);
    void* ws = nullptr;
    if (int rc = static_workspace(&ws)) return rc;
    return mis_sample(groups, n_groups, ws, kStaticWsBytes, stream);
}

#ifdef MIS_PHASE_STAMPS
// The phase timestamps of the last launches (profiling builds only): kStampBlocks x kStampSlots words.
int mis_debug_stamps(void* host, size_t bytes) {
    const size_t n = std::min(bytes, sizeof(mis_stamps));
    const hipError_t e = hipMemcpyFromSymbol(host, HIP_SYMBOL(mis_stamps), n, 0, hipMemcpyDeviceToHost);
    return e == hipSuccess ? 0 : -1;
}
int mis_debug_clear_stamps(void) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(mis_stamps)) != hipSuccess) return -1;
    return hipMemset(p, 0, sizeof(mis_stamps)) == hipSuccess ? 0 : -1;
}
#endif

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
