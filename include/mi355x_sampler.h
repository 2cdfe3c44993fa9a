/* C-ABI of the MI355X token-sampling path (libmi355x_sampler.so).
 *
 * Replaces the per-row logits pipeline and draw of the reference sampler,
 * engine/talker_sampler.py (Python + torch), with fused HIP kernels:
 *
 *   mis_sample   <- processed_logits (engine/talker_sampler.py:136-158)
 *                   + draw            (:161-172, incl. uniform_values injection)
 *                   + the state update of step (:234-249) and of the graph
 *                     bodies (engine/runtime/talker_post_graph.py:56-76,
 *                     engine/runtime/talker_decode.py:120-128)
 *                   + the filters used on their own (repetition_penalty :79-84,
 *                     top_p_filter :87-92, top_k_filter :95-98,
 *                     top_p_top_k_filter :101-116, top_k_top_p_filter :119-133)
 *                   + Thinker greedy argmax (engine/runtime/thinker_decode.py:107,
 *                     engine/runtime/backend_npu.py:890) as a row with T <= 0
 *   mis_uniform  <- uniform (engine/talker_sampler.py:70-76), and the Philox
 *                   draw key (no reference counterpart)
 *
 * All pointers are device pointers on the current HIP device.  Calls are
 * stream-ordered on the given hipStream_t (NULL = the null stream), allocate
 * nothing, never synchronise the host, and can be captured into a hipGraph.
 * The library keeps no global state besides the per-thread last-error string.
 *
 * Return codes: 0 success, > 0 invalid argument (MIS_E_*), < 0 HIP error.
 * mis_last_error() describes the last failure of the calling thread.
 */
#ifndef MI355X_SAMPLER_H
#define MI355X_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MIS_ABI_VERSION 1

enum { MIS_F32 = 0, MIS_BF16 = 1 };                        /* logits dtype */
enum { MIS_OMNI = 0, MIS_HF = 1 };                         /* pipeline order (engine/talker_sampler.py:142-156) */
enum { MIS_RNG_COUNTER = 0, MIS_RNG_PHILOX = 1 };          /* lowbias32 (seed, step) | Philox4x32-10 (seed, row id, step) */
enum { MIS_HISTORY_WINDOW = 0, MIS_HISTORY_RING = 1 };     /* shift-append (reference layout) | ring with a head index */

enum {
    MIS_TOPK_ZERO_DISABLES = 1, /* top_k <= 0 means "no top-k" (vLLM); otherwise k = min(max(top_k, min_keep), V) */
    MIS_TOPP_ONE_DISABLES = 2,  /* top_p >= 1 means "no top-p"; otherwise the reference formula is evaluated at p = 1 */
    MIS_UPDATE_STATE = 4,       /* live rows: append the token to history, steps += 1, finished |= (token == eos) */
    MIS_FINALIZE_STREAMING = 8, /* finalise every row from its logits alone (the path a row takes when its slice
                                   workgroups did not share an XCD); same results, slower; for validation */
};

enum { MIS_E_ARG = 1, MIS_E_WORKSPACE = 2, MIS_E_UNSUPPORTED = 3 };

/* Diagnostics (no reference counterpart): bytes [MIS_WS_PATH_OFFSET, + 4 * MIS_PATH_COUNT) of the workspace hold one
 * uint32 counter per finalisation path, incremented once per sampled row and never cleared by the library; a caller
 * that wants per-launch figures zeroes them before the launch.  Which path a row takes never changes its result. */
#define MIS_WS_PATH_OFFSET 64
/* Bytes [MIS_WS_ERROR_OFFSET, + 4): uint32 count of slice workgroups that gave up waiting (2 ms) for their row's
 * finaliser (a top-p row without top-k settled from value counts); never cleared by the library.  When the one that
 * gave up held the row's draw, the row came out as PAD with its state untouched.  It stays 0 unless the device
 * stalls a workgroup for milliseconds. */
#define MIS_WS_ERROR_OFFSET 128
enum {
    MIS_PATH_GREEDY = 0,     /* first argmax from the slices' maxima */
    MIS_PATH_FULL = 1,       /* no filter: the slices' sub-block sums, one sub-block rescanned */
    MIS_PATH_CANDIDATES = 2, /* top-k / top-p selection over the slices' candidates */
    MIS_PATH_HISTOGRAM = 3,  /* top-p without top-k, bf16: the slices' value histograms, one slice rescanned */
    MIS_PATH_STREAM = 4,     /* the whole row from its logits */
    MIS_PATH_FORCED = 5,     /* EOS forced at max_new_tokens */
    MIS_PATH_COUNT = 6
};

/* One group of rows that share a vocabulary size, dtype and pipeline order.
 * Per-row parameter arrays may be NULL, in which case the scalar *_value applies
 * to every row (the reference's single TalkerSampling). */
typedef struct MisGroup {
    const void* logits;            /* [rows, row_stride] f32 or bf16; only the first vocab entries of a row are read */
    int64_t logits_row_stride;     /* elements */
    int32_t dtype;                 /* MIS_F32 | MIS_BF16 */
    int32_t vocab;                 /* V >= 1 */
    int32_t rows;                  /* B >= 0 */
    int32_t semantics;             /* MIS_OMNI | MIS_HF */
    int32_t flags;                 /* MIS_TOPK_ZERO_DISABLES | MIS_TOPP_ONE_DISABLES | MIS_UPDATE_STATE | ... */
    int32_t min_keep;              /* >= 1 (reference: 3 for hf, 1 for omni) */

    const float* temperature;      /* [rows] or NULL; T <= 0 selects greedy (first index of the max) */
    const int32_t* top_k;          /* [rows] or NULL */
    const float* top_p;            /* [rows] or NULL */
    const float* repetition;       /* [rows] or NULL; alpha = rep**n, x<0 ? x*alpha : x/alpha */
    const float* presence;         /* [rows] or NULL; x -= presence * (n > 0) */
    const float* frequency;        /* [rows] or NULL; x -= frequency * n (before presence) */
    float temperature_value;
    float top_p_value;
    float repetition_value;
    float presence_value;
    float frequency_value;
    int32_t top_k_value;

    const float* alpha_lut;        /* optional [alpha_lut_len]: alpha for count n < len (e.g. torch.pow's values);
                                      otherwise alpha = fp32(pow(double(rep), n)), correctly rounded */
    int32_t alpha_lut_len;
    int32_t history_len;           /* W (0 = no history); <= 65535 */

    void* history;                 /* [rows, history_row_stride] int32 or int64 token ids; < 0 (PAD) or >= V: empty */
    int64_t history_row_stride;    /* elements */
    int32_t history_is_int64;
    int32_t history_mode;          /* MIS_HISTORY_WINDOW | MIS_HISTORY_RING */
    int32_t* history_head;         /* [rows] ring write position (MIS_HISTORY_RING only) */

    const uint32_t* allowed;       /* [rows, allowed_row_stride] packed bitmask or NULL; bit j of word w = token 32w+j, 1 = allowed */
    int64_t allowed_row_stride;    /* 32-bit words */

    int32_t eos;                   /* EOS id or -1 */
    int32_t min_new_tokens;        /* EOS censored while step < min_new_tokens */
    int32_t max_new_tokens;        /* EOS forced at step >= max_new_tokens - 1; 0 = never */
    int32_t rng;                   /* MIS_RNG_COUNTER | MIS_RNG_PHILOX */

    const int64_t* seeds;          /* [rows] (required unless uniforms given) */
    int64_t* steps;                /* [rows] frame index (NULL = all 0); advanced with MIS_UPDATE_STATE */
    const int64_t* row_ids;        /* [rows] request-stable ids for Philox (NULL = 0) */
    const float* uniforms;         /* [rows] injected U[0,1) draws or NULL */
    const uint8_t* active;         /* [rows] bool or NULL (= all active) */
    uint8_t* finished;             /* [rows] bool or NULL (= none finished) */

    int64_t* tokens;               /* [rows] out (or NULL): sampled id, PAD = -1 for inactive/finished rows */
    float* processed;              /* [rows, processed_row_stride] out (or NULL): processed logits, -inf where filtered */
    int64_t processed_row_stride;
    float* probs;                  /* [rows, probs_row_stride] out (or NULL): softmax of the processed logits */
    int64_t probs_row_stride;
} MisGroup;

/* Version of this ABI (MIS_ABI_VERSION). */
int mis_version(void);

/* sizeof(MisGroup) as compiled into the library: lets a binding check its struct layout (no reference
 * counterpart; an ABI guard for the ctypes / FFI side). */
size_t mis_sizeof_group(void);

/* Last error of the calling thread ("" if none). */
const char* mis_last_error(void);

/* Bytes of device workspace mis_sample needs for these groups (0 on invalid arguments). The workspace must
 * be zero-filled once when allocated; every launch leaves it zeroed again for the next. */
size_t mis_workspace_bytes(const MisGroup* groups, int n_groups);

/* The fused pipeline + draw (+ optional state update) for every row of every group: one kernel launch (a top-p
 * row without top-k whose nucleus the slices' candidates cannot hold resolves its boundary bin inside it).  Calls
 * that share a workspace must be ordered on one stream. */
int mis_sample(const MisGroup* groups, int n_groups, void* workspace, size_t workspace_bytes, void* stream);

/* mis_sample on a workspace the library owns, for callers that cannot allocate (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc).  No counterpart in the reference.  The workspace is a device
 * array of MIS_STATIC_WORKSPACE_BYTES in the library's code object (one copy per GPU, zero at load); this call
 * allocates nothing and fails with MIS_E_WORKSPACE when mis_workspace_bytes(groups) exceeds it.  Every call on a
 * GPU shares that GPU's array: calls that overlap on one GPU (different streams, concurrent graph replays) race
 * and must not be issued; calls ordered on one stream are safe. */
#define MIS_STATIC_WORKSPACE_BYTES (64u << 20)
int mis_sample_static(const MisGroup* groups, int n_groups, void* stream);

/* out[i] = U[0,1) of (seeds[i], steps[i], row_ids[i]) under MIS_RNG_COUNTER (row_ids ignored) or
 * MIS_RNG_PHILOX (row_ids NULL = 0): engine/talker_sampler.py:70-76 for the counter hash. */
int mis_uniform(const int64_t* seeds, const int64_t* steps, const int64_t* row_ids, int64_t n, int32_t rng, float* out,
                void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MI355X_SAMPLER_H */
