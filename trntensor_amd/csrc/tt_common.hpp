// Shared device helpers for the gfx950 kernels: MFMA wrappers, 16-byte vector
// types, wavefront reductions, XCD-aware workgroup remapping, status plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/trntensor_hip.h"

namespace tt {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// MFMA 16x16x4 wrappers. One instruction computes a 16x16 block of
// D += A(16x4) * B(4x16) across the 64 lanes of a wavefront:
//   lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16];
//   lane l holds D[row(l / 16, r)][l % 16] in accumulator element r, where
//   row(g, r) = 4 g + r for f32 and g + 4 r for f64 (the f64 instruction
//   interleaves its four 4-row groups across the accumulator registers).
// ---------------------------------------------------------------------------
typedef double d4_t __attribute__((ext_vector_type(4)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef double d2_t __attribute__((ext_vector_type(2)));

template <typename T>
struct Mfma;

template <>
struct Mfma<double> {
    typedef d4_t acc_t;
    static __device__ __forceinline__ acc_t mma(double a, double b, acc_t c) {
        return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ int row(int g, int r) { return g + 4 * r; }
};

template <>
struct Mfma<float> {
    typedef f4_t acc_t;
    static __device__ __forceinline__ acc_t mma(float a, float b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ int row(int g, int r) { return 4 * g + r; }
};

// 16-byte vector of T (dwordx4 global/LDS access).
template <typename T>
struct Vec16;
template <>
struct Vec16<double> {
    typedef double type __attribute__((ext_vector_type(2)));
    static constexpr int n = 2;
};
template <>
struct Vec16<float> {
    typedef float type __attribute__((ext_vector_type(4)));
    static constexpr int n = 4;
};

// Vector of N values of T (N * sizeof(T) bytes).
template <typename T, int N>
struct VecN {
    typedef T type __attribute__((ext_vector_type(N)));
};

// ---------------------------------------------------------------------------
// Reductions
// ---------------------------------------------------------------------------
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Thread t's sum of p[t], p[t + 256], p[t + 512], ... (< n), in that order.
// Eight loads are issued before their sums (the order of the sums is
// unchanged): a single workgroup walking tens of thousands of partials with
// one load in flight per thread waits out a memory latency per element.
__device__ __forceinline__ double strided_sum256(const double* __restrict__ p, int64_t n) {
    double s = 0.0;
    int64_t k = threadIdx.x;
    for (; k + 7 * 256 < n; k += 8 * 256) {
        double x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = p[k + u * 256];
#pragma unroll
        for (int u = 0; u < 8; ++u) s += x[u];
    }
    for (; k < n; k += 256) s += p[k];
    return s;
}

// Sum over a 256-thread block; result valid in thread 0. `scratch` holds >= 4 doubles.
__device__ __forceinline__ double block256_sum(double v, double* scratch) {
    v = wave_sum(v);
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    double r = 0.0;
    if (threadIdx.x == 0) r = (scratch[0] + scratch[1]) + (scratch[2] + scratch[3]);
    return r;
}

// ---------------------------------------------------------------------------
// Double-double accumulation, after Ogita, Rump & Oishi, "Accurate sum and
// dot product", SIAM J. Sci. Comput. 26(6), 2005: TwoSum (Knuth) and
// TwoProduct (one FMA) are error-free transformations; Dot2 keeps the
// running sum p and the sum s of every rounding error, so p + s is the dot
// product as if accumulated in twice the working precision and rounded once.
// Contraction into FMAs is switched off inside these helpers: fusing the
// separate product into a following sum would change the values the error
// terms are computed from.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void two_sum(double a, double b, double& sum, double& err) {
#pragma clang fp contract(off)
    const double s = a + b;
    const double z = s - a;
    err = (a - (s - z)) + (b - z);
    sum = s;
}

struct Dot2 {
    double p = 0.0, s = 0.0;

    // p + s += a * b
    __device__ __forceinline__ void add_prod(double a, double b) {
#pragma clang fp contract(off)
        const double h = a * b;
        const double r = __builtin_fma(a, b, -h);
        double np, q;
        two_sum(p, h, np, q);
        p = np;
        s = s + (q + r);
    }
    // p + s += x
    __device__ __forceinline__ void add(double x) {
#pragma clang fp contract(off)
        double np, q;
        two_sum(p, x, np, q);
        p = np;
        s = s + q;
    }
    // p + s += o.p + o.s
    __device__ __forceinline__ void merge(double op, double os) {
#pragma clang fp contract(off)
        double np, q;
        two_sum(p, op, np, q);
        p = np;
        s = s + (q + os);
    }
    __device__ __forceinline__ double value() const { return p + s; }
};

// ---------------------------------------------------------------------------
// XCD-aware workgroup order. The dispatcher hands workgroup w to XCD w % 8,
// so consecutive ids land on different L2s. This maps the hardware id to a
// logical id such that each XCD walks a contiguous range of logical ids
// (neighbouring tiles share operand panels in that XCD's L2). The remainder
// (total % 8 ids at the end) keeps its identity mapping.
// ---------------------------------------------------------------------------
constexpr int kNumXcd = 8;

__device__ __forceinline__ int64_t xcd_remap(int64_t w, int64_t total) {
    const int64_t per = total / kNumXcd;
    if (w >= per * kNumXcd) return w;
    return (w % kNumXcd) * per + (w / kNumXcd);
}

// ---------------------------------------------------------------------------
// Fast unsigned division by a runtime constant (round-up multiplier method,
// Granlund & Montgomery 1994): for d >= 1, s = ceil(log2 d),
// m = floor(2^32 (2^s - d) / d) + 1, then n / d = (umulhi(n, m) + n) >> s
// for every n < 2^31 (the sum stays below 2^32).
// ---------------------------------------------------------------------------
struct FastDiv {
    uint32_t d, m, s;
};

inline FastDiv make_fastdiv(uint32_t d) {
    FastDiv f;
    f.d = d;
    uint32_t s = 0;
    while ((1ull << s) < d) ++s;
    f.s = s;
    f.m = (uint32_t)(((1ull << 32) * ((1ull << s) - d)) / d + 1);
    return f;
}

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
    return (__umulhi(n, f.m) + n) >> f.s;
}

// ---------------------------------------------------------------------------
// Status plumbing
// ---------------------------------------------------------------------------
int set_error(int code, const char* fmt, ...);

inline int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(TT_HIP_ERROR, "%s: %s", what, hipGetErrorString(e));
    return TT_OK;
}

}  // namespace tt
