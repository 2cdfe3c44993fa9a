// Wave- and workgroup-level primitives for gfx950 (wave64, 1024-thread workgroups).
//
// Cross-lane moves are VALU moves wherever the partner is fixed: DPP quad permutes and row rotates inside a row
// of 16 lanes, gfx950's permlane swaps across rows.  Workgroup reductions combine the 16 wave results in a fixed
// order, so every result is independent of scheduling.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mis {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

// A pointer into global memory as such: accesses through it compile to global instructions.  A flat access
// would also count against the LDS wait counter, so every LDS wait after a flat load waits for that load too.
template <class T>
using gptr = __attribute__((address_space(1))) T*;
template <class T>
__device__ __forceinline__ gptr<T> gp(T* p) {
    return (gptr<T>)p;
}
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
// 16 bytes from global address a (16-byte aligned).
__device__ __forceinline__ uint4 ld_u4(uintptr_t a) {
    const u32x4_t v = *(gptr<const u32x4_t>)a;
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ int4 ld_i4(const void* p) {
    const u32x4_t v = *(gptr<const u32x4_t>)p;
    return make_int4((int)v.x, (int)v.y, (int)v.z, (int)v.w);
}

// Row-uniform values into scalar registers.
__device__ __forceinline__ int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ uint32_t uni(uint32_t x) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)x); }
__device__ __forceinline__ float uni(float x) {
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x)));
}
__device__ __forceinline__ int64_t uni(int64_t x) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)x >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ double uni(double x) {
    return __longlong_as_double(uni((int64_t)__double_as_longlong(x)));
}

__device__ __forceinline__ uint32_t lane_mbcnt() {
    return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}

// lane ^ O for a power of two O.
template <int O>
__device__ __forceinline__ uint32_t xor_lane(uint32_t x) {
    static_assert(O >= 1 && O <= 32 && (O & (O - 1)) == 0, "power-of-two offset");
    if constexpr (O == 1) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    } else if constexpr (O == 2) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    } else if constexpr (O == 4) {
        const int m = __builtin_amdgcn_update_dpp(0, (int)x, 0x141, 0xF, 0xF, false);  // row_half_mirror
        return (uint32_t)__builtin_amdgcn_update_dpp(0, m, 0x1B, 0xF, 0xF, false);      // quad_perm [3,2,1,0]
    } else if constexpr (O == 8) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x128, 0xF, 0xF, false);  // row_ror:8
    } else if constexpr (O == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
        return (lane_mbcnt() & 16u) ? r[0] : r[1];
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        return lane_mbcnt() < 32u ? r[1] : r[0];
    }
}

template <class T>
struct Lanes;
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
        return __longlong_as_double(
            (long long)Lanes<unsigned long long>::mv((unsigned long long)__double_as_longlong(x), f));
    }
};

template <int O, class T>
__device__ __forceinline__ T shfl_xor(T x) {
    return Lanes<T>::mv(x, [](uint32_t v) { return xor_lane<O>(v); });
}

// Every lane ends with op over the wave (a symmetric butterfly: each lane computes the same tree).
template <class T, class Op>
__device__ __forceinline__ T wave_reduce(T x, Op op) {
    x = op(x, shfl_xor<32>(x));
    x = op(x, shfl_xor<16>(x));
    x = op(x, shfl_xor<8>(x));
    x = op(x, shfl_xor<4>(x));
    x = op(x, shfl_xor<2>(x));
    x = op(x, shfl_xor<1>(x));
    return x;
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_or_zero(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, ROW_MASK, 0xF, false);
}

// Inclusive scan over the wave in DPP moves: Hillis-Steele within each row of 16 (row_shr 1, 2, 4, 8), then the
// row totals (row_bcast:15 into rows 1 and 3, row_bcast:31 into rows 2 and 3).
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

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

// Rank of this lane among the set lanes of b below it.
__device__ __forceinline__ uint32_t rank_below(uint64_t b) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
}

// Workgroup scratch for the reductions below (one slot per wave, 16-byte aligned so that a thread reads all 16
// partials with a few wide LDS loads).
struct alignas(16) Red {
    double d[kWaves];
    unsigned long long u[kWaves];
    float4 f4[kWaves];
    float f[kWaves];
    int32_t i[kWaves];
    int32_t j[kWaves];
};

// Workgroup reductions.  Each starts with a barrier (the scratch may still be read by the previous one) and ends
// with every thread holding the result.  The 16 wave partials are combined in a fixed order.
template <class T, int N>
__device__ __forceinline__ void load_partials(const T (&src)[N], T (&dst)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) dst[i] = src[i];
}

__device__ __forceinline__ float block_max_f(float x, Red& r) {
    x = wave_reduce(x, [](float a, float b) { return fmaxf(a, b); });
    __syncthreads();
    if (lane_id() == 0) r.f[wave_id()] = x;
    __syncthreads();
    float p[kWaves];
    load_partials(r.f, p);
    float m = p[0];
#pragma unroll
    for (int i = 1; i < kWaves; ++i) m = fmaxf(m, p[i]);
    return m;
}

__device__ __forceinline__ int block_min_i(int x, Red& r) {
    x = wave_reduce(x, [](int a, int b) { return min(a, b); });
    __syncthreads();
    if (lane_id() == 0) r.i[wave_id()] = x;
    __syncthreads();
    int p[kWaves];
    load_partials(r.i, p);
    int m = p[0];
#pragma unroll
    for (int i = 1; i < kWaves; ++i) m = min(m, p[i]);
    return m;
}

__device__ __forceinline__ int block_max_i(int x, Red& r) {
    x = wave_reduce(x, [](int a, int b) { return max(a, b); });
    __syncthreads();
    if (lane_id() == 0) r.i[wave_id()] = x;
    __syncthreads();
    int p[kWaves];
    load_partials(r.i, p);
    int m = p[0];
#pragma unroll
    for (int i = 1; i < kWaves; ++i) m = max(m, p[i]);
    return m;
}

__device__ __forceinline__ int block_sum_i(int x, Red& r) {
    x = wave_reduce(x, [](int a, int b) { return a + b; });
    __syncthreads();
    if (lane_id() == 0) r.i[wave_id()] = x;
    __syncthreads();
    int p[kWaves];
    load_partials(r.i, p);
    int m = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) m += p[i];
    return m;
}

__device__ __forceinline__ double block_sum_d(double x, Red& r) {
    x = wave_reduce(x, [](double a, double b) { return a + b; });
    __syncthreads();
    if (lane_id() == 0) r.d[wave_id()] = x;
    __syncthreads();
    double p[kWaves];
    load_partials(r.d, p);
    double m = 0.0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) m += p[i];
    return m;
}

__device__ __forceinline__ unsigned long long block_sum_u(unsigned long long x, Red& r) {
    x = wave_reduce(x, [](unsigned long long a, unsigned long long b) { return a + b; });
    __syncthreads();
    if (lane_id() == 0) r.u[wave_id()] = x;
    __syncthreads();
    unsigned long long p[kWaves];
    load_partials(r.u, p);
    unsigned long long m = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) m += p[i];
    return m;
}

// Four float maxima at once (one barrier pair).
__device__ __forceinline__ float4 block_max4(float4 v, Red& r) {
    auto mx = [](float a, float b) { return fmaxf(a, b); };
    v.x = wave_reduce(v.x, mx);
    v.y = wave_reduce(v.y, mx);
    v.z = wave_reduce(v.z, mx);
    v.w = wave_reduce(v.w, mx);
    __syncthreads();
    if (lane_id() == 0) r.f4[wave_id()] = v;
    __syncthreads();
    float4 p[kWaves];
    load_partials(r.f4, p);
    float4 m = p[0];
#pragma unroll
    for (int i = 1; i < kWaves; ++i) {
        m.x = fmaxf(m.x, p[i].x);
        m.y = fmaxf(m.y, p[i].y);
        m.z = fmaxf(m.z, p[i].z);
        m.w = fmaxf(m.w, p[i].w);
    }
    return m;
}

// Max of (value, first index): the largest value, and among equal values the smallest index.
__device__ __forceinline__ void block_argmax(float& v, int& idx, Red& r) {
    auto better = [](float a, int ia, float b, int ib) { return a > b || (a == b && ia < ib); };
    auto step = [&](float ov, int oi) {
        if (better(ov, oi, v, idx)) {
            v = ov;
            idx = oi;
        }
    };
    step(shfl_xor<32>(v), shfl_xor<32>(idx));
    step(shfl_xor<16>(v), shfl_xor<16>(idx));
    step(shfl_xor<8>(v), shfl_xor<8>(idx));
    step(shfl_xor<4>(v), shfl_xor<4>(idx));
    step(shfl_xor<2>(v), shfl_xor<2>(idx));
    step(shfl_xor<1>(v), shfl_xor<1>(idx));
    __syncthreads();
    if (lane_id() == 0) r.f4[wave_id()] = make_float4(v, __int_as_float(idx), 0.f, 0.f);
    __syncthreads();
    float4 p[kWaves];
    load_partials(r.f4, p);
    v = p[0].x;
    idx = __float_as_int(p[0].y);
#pragma unroll
    for (int i = 1; i < kWaves; ++i)
        if (better(p[i].x, __float_as_int(p[i].y), v, idx)) {
            v = p[i].x;
            idx = __float_as_int(p[i].y);
        }
}

// Exclusive prefix over the workgroup in thread order, and the total (integer types: the subtraction is exact).
template <class T>
__device__ __forceinline__ T block_excl_scan(T x, T& total, T* scratch /* kWaves */) {
    static_assert(__is_integral(T), "integer scan");
    const T incl = wave_incl_scan(x);
    __syncthreads();
    if (lane_id() == 63) scratch[wave_id()] = incl;
    __syncthreads();
    T p[kWaves];
#pragma unroll
    for (int i = 0; i < kWaves; ++i) p[i] = scratch[i];
    T off = T(0);
    total = T(0);
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
        off += (i < wave_id()) ? p[i] : T(0);
        total += p[i];
    }
    return off + incl - x;
}

}  // namespace mis
