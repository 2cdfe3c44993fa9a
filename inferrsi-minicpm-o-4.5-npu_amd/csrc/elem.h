// Per-element arithmetic of the sampling pipeline and the draw's random numbers.
//
// Everything here is exact where the reference (engine/talker_sampler.py) is exact: divisions by the temperature
// and by rep**n round once, like torch's fp32 division, and products and differences round separately (the
// library is built with -ffp-contract=off).
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "primitives.h"

namespace mis {

// ------------------------------------------------------------------ the draw's uniforms

// lowbias32 (C. Wellons, hash-prospector), as engine/talker_sampler.py:60-67 applies it to 32-bit lanes.
__host__ __device__ __forceinline__ uint32_t lowbias32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

// engine/talker_sampler.py:70-76: U[0, 1) from (seed, frame index).
__host__ __device__ __forceinline__ float counter_uniform(int64_t seed, int64_t step) {
    const uint64_t s = (uint64_t)seed, t = (uint64_t)step;
    uint32_t h = lowbias32((uint32_t)s);
    h = lowbias32(h ^ (uint32_t)(s >> 32) ^ 0x9E3779B9u);
    h = lowbias32(h ^ (uint32_t)t ^ 0x632BE5ABu);
    return (float)(h >> 8) * (1.0f / 16777216.0f);
}

// Philox4x32-10 (Salmon et al., SC'11, "Parallel random numbers: as easy as 1, 2, 3"): key = seed, counter =
// (step, request id); word 0 -> U[0, 1) with 24 bits.  No reference counterpart.
__host__ __device__ __forceinline__ float philox_uniform(int64_t seed, int64_t step, int64_t rid) {
    const uint64_t s = (uint64_t)seed, t = (uint64_t)step, r = (uint64_t)rid;
    uint32_t c0 = (uint32_t)t, c1 = (uint32_t)(t >> 32), c2 = (uint32_t)r, c3 = (uint32_t)(r >> 32);
    uint32_t k0 = (uint32_t)s, k1 = (uint32_t)(s >> 32);
    for (int rnd = 0; rnd < 10; ++rnd) {
        if (rnd) {
            k0 += 0x9E3779B9u;
            k1 += 0xBB67AE85u;
        }
        const uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t lo0 = (uint32_t)p0, hi0 = (uint32_t)(p0 >> 32);
        const uint32_t lo1 = (uint32_t)p1, hi1 = (uint32_t)(p1 >> 32);
        const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
        c0 = n0;
        c1 = lo1;
        c2 = n2;
        c3 = lo0;
    }
    return (float)(c0 >> 8) * (1.0f / 16777216.0f);
}

// ------------------------------------------------------------------ element arithmetic

// x / d rounded once to float (IEEE division) for d > 0 given with rd = RN64(1 / d).  In the normal range the double
// product x * rd is within 2^-52 (relative) of x / d, while a quotient of two 24-bit significands is either a float
// or at least 2^-49 (relative) away from every float rounding midpoint, so rounding the product to float gives
// RN(x / d).  Below 2^-126 float midpoints are 2^-150 apart and a quotient can sit exactly on one, where the
// product may fall on either side: a result under 2^-125 in magnitude is therefore recomputed by IEEE division.
// Infinities, zeros (with their sign) and NaN pass through as IEEE division has them.
__device__ __forceinline__ float div_rn(float x, float d, double rd) {
    float q = (float)((double)x * rd);
    const bool tiny = fabsf(q) < 0x1p-125f && x != 0.0f;
    // a branch on the wave, not a select: the IEEE division runs only when some lane needs it (the empty asm
    // keeps the compiler from computing it ahead of the branch)
    if (__builtin_amdgcn_ballot_w64(tiny)) {
        float xs = x;
        asm volatile("" : "+v"(xs));
        if (tiny) q = xs / d;
    }
    return q;
}

// exp(x) within ~1.3 ulp: 2^(x log2 e) with the product's rounding error (and log2 e's own) folded back in
// first order, on the hardware exp2.
__device__ __forceinline__ float exp_acc(float x) {
    const float kL2e = 1.44269502f;           // RN(log2 e)
    const float kL2eLo = 1.925963033e-8f;     // log2 e - kL2e
    const float t = x * kL2e;
    float e = __builtin_fmaf(x, kL2e, -t);
    e = __builtin_fmaf(x, kL2eLo, e);
    const float r = __builtin_amdgcn_exp2f(t);
    return __builtin_fmaf(r, e * 0.693147182f, r);
}

// Order-preserving key of a float: keys compare as unsigned integers like the floats compare, with -0 and +0 one
// key (they compare equal).
__host__ __device__ __forceinline__ uint32_t ord_key(float f) {
    uint32_t u = __float_as_uint(f);
    if (u == 0x80000000u) u = 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__host__ __device__ __forceinline__ float key_float(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__device__ __forceinline__ bool is_finite_f(float f) { return f > -INFINITY && f < INFINITY; }

// rep**n rounded once to float: binary powering in double (at most 2 log2 n products, relative error < 1e-14),
// or the caller's table for n < len (the reference uses torch.pow, engine/talker_sampler.py:83).
__device__ __forceinline__ float alpha_of(float rep, int n, const float* lut, int lut_len) {
    if (lut != nullptr && n < lut_len) return gp(lut)[n];
    double r = 1.0, b = (double)rep;
    for (unsigned e = (unsigned)n; e; e >>= 1) {
        if (e & 1u) r *= b;
        b *= b;
    }
    return (float)r;
}

}  // namespace mis
