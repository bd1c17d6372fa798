// Measurement aids: the MFMA rate this device sustains with no memory
// traffic, and the rate it streams HBM with no arithmetic; the denominators of
// the "fraction of the measured peak" next to each kernel's fraction of the
// datasheet peak.
//
// Every wavefront runs `iters` rounds of 8 independent accumulator chains of
// the MFMA the kernels use, from register operands only: 16x16x4 for f64 and
// f32 (8 * 2048 FLOP per round), 16x16x32 with fp32 accumulators for bf16 and
// f16 (8 * 16384 FLOP per round). One value per workgroup is written so
// the work cannot be removed.
#include <type_traits>

#include "tt_common.hpp"

namespace tt {

namespace {

template <typename T>
__global__ __launch_bounds__(256) void mfma_rate_kernel(int64_t iters, T* out) {
    typedef Mfma<T> MF;
    typename MF::acc_t acc[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = typename MF::acc_t{0, 0, 0, 0};
    // Small operands keep the sums finite for any iteration count.
    const T a = (T)((threadIdx.x & 7) + 1) * (T)1e-6;
    const T b = (T)((threadIdx.x >> 3 & 7) + 1) * (T)1e-6;
    for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[c] = MF::mma(a, b, acc[c]);
    }
    T s = T(0);
#pragma unroll
    for (int c = 0; c < 8; ++c) s += (acc[c][0] + acc[c][1]) + (acc[c][2] + acc[c][3]);
    if (threadIdx.x == 0) out[blockIdx.x] = s;
}

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

// The 16-bit kernels' MFMA (16x16x32 with fp32 accumulators), 16384 FLOP each.
template <typename T>
__global__ __launch_bounds__(256) void mfma16_rate_kernel(int64_t iters, unsigned short* out) {
    f32x4_t acc[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = f32x4_t{0, 0, 0, 0};
    const T a = (T)((float)((threadIdx.x & 7) + 1) * 1e-3f);
    const T b = (T)((float)((threadIdx.x >> 3 & 7) + 1) * 1e-3f);
    typedef typename std::conditional<std::is_same<T, __bf16>::value, bf16x8_t, f16x8_t>::type v8;
    const v8 va = {a, a, a, a, a, a, a, a}, vb = {b, b, b, b, b, b, b, b};
    for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            if constexpr (std::is_same<T, __bf16>::value)
                acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, vb, acc[c], 0, 0, 0);
            else
                acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, vb, acc[c], 0, 0, 0);
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) s += (acc[c][0] + acc[c][1]) + (acc[c][2] + acc[c][3]);
    if (threadIdx.x == 0) out[blockIdx.x] = __builtin_bit_cast(unsigned short, (T)s);
}

// ---------------------------------------------------------------------------
// HBM streaming probe: the rate at which this device moves bytes between HBM
// and the CUs with nothing else to do, the denominator of every "fraction of
// the measured HBM peak". Op 0 reads `n16` 16-byte pieces, op 1 writes them,
// op 2 copies them; every access is a 16-byte vector load or store,
// non-temporal (NT) or through the caches. Each thread walks the pieces
// grid-stride, kPieces at a time with all of a batch's loads issued before
// any of their uses, so every CU keeps many lines in flight.
// ---------------------------------------------------------------------------
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
constexpr int kPieces = 8;

template <bool NT>
__device__ __forceinline__ u32x4_t probe_load(const u32x4_t* p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    else return *p;
}

template <bool NT>
__device__ __forceinline__ void probe_store(u32x4_t v, u32x4_t* p) {
    if constexpr (NT) __builtin_nontemporal_store(v, p);
    else *p = v;
}

template <int OP, bool NT>
__global__ __launch_bounds__(256) void hbm_stream_kernel(const u32x4_t* __restrict__ src, u32x4_t* __restrict__ dst,
                                                         int64_t n16, uint32_t* flag) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    u32x4_t acc = {0, 0, 0, 0};
    const u32x4_t fill = {(uint32_t)i, 0x9e3779b9u, 0, 1};
    for (; i + (kPieces - 1) * stride < n16; i += kPieces * stride) {
        if constexpr (OP == 1) {
#pragma unroll
            for (int u = 0; u < kPieces; ++u) probe_store<NT>(fill, dst + i + u * stride);
        } else {
            u32x4_t v[kPieces];
#pragma unroll
            for (int u = 0; u < kPieces; ++u) v[u] = probe_load<NT>(src + i + u * stride);
#pragma unroll
            for (int u = 0; u < kPieces; ++u) {
                if constexpr (OP == 2) probe_store<NT>(v[u], dst + i + u * stride);
                else acc ^= v[u];
            }
        }
    }
    for (; i < n16; i += stride) {
        if constexpr (OP == 1) {
            probe_store<NT>(fill, dst + i);
        } else {
            const u32x4_t v = probe_load<NT>(src + i);
            if constexpr (OP == 2) probe_store<NT>(v, dst + i);
            else acc ^= v;
        }
    }
    // Read op: the loads feed a value the kernel may store, so they stay.
    if constexpr (OP == 0)
        if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x5a17c0deu) flag[0] = 1;
}

}  // namespace

}  // namespace tt

extern "C" int tt_hbm_probe(int mode, const void* src, void* dst, int64_t bytes, int64_t workgroups, void* flag,
                            void* stream) {
    using namespace tt;
    const int op = mode & 3;
    const bool cached = (mode & 4) != 0;
    if (mode < 0 || mode > 6 || op == 3)
        return set_error(TT_INVALID, "tt_hbm_probe: mode %d (0 read, 1 write, 2 copy; +4 cached)", mode);
    if (bytes < 0 || bytes % 16 != 0)
        return set_error(TT_INVALID, "tt_hbm_probe: %lld bytes (a non-negative multiple of 16)", (long long)bytes);
    if (workgroups <= 0 || workgroups > 0x7fffffffLL)
        return set_error(TT_INVALID, "tt_hbm_probe: workgroups %lld", (long long)workgroups);
    if ((op != 1 && !src) || (op != 0 && !dst) || (op == 0 && !flag))
        return set_error(TT_INVALID, "tt_hbm_probe: NULL pointer");
    if (((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) != 0)
        return set_error(TT_INVALID, "tt_hbm_probe: buffers must be 16-byte aligned");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid((unsigned)workgroups), block(256);
    const u32x4_t* s = static_cast<const u32x4_t*>(src);
    u32x4_t* d = static_cast<u32x4_t*>(dst);
    uint32_t* f = static_cast<uint32_t*>(flag);
    const int64_t n16 = bytes / 16;
#define TT_HBM_CASE(O, C) \
    if (op == O && cached == C) hipLaunchKernelGGL((hbm_stream_kernel<O, !C>), grid, block, 0, st, s, d, n16, f);
    TT_HBM_CASE(0, false)
    TT_HBM_CASE(1, false)
    TT_HBM_CASE(2, false)
    TT_HBM_CASE(0, true)
    TT_HBM_CASE(1, true)
    TT_HBM_CASE(2, true)
#undef TT_HBM_CASE
    return check_launch("tt_hbm_probe");
}

extern "C" int tt_mfma_rate_probe(int dtype, int64_t workgroups, int64_t iters, void* out, void* stream) {
    using namespace tt;
    if (workgroups <= 0 || workgroups > 0x7fffffffLL || iters < 0)
        return set_error(TT_INVALID, "tt_mfma_rate_probe: workgroups %lld, iters %lld", (long long)workgroups,
                         (long long)iters);
    if (!out) return set_error(TT_INVALID, "tt_mfma_rate_probe: out is NULL");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid((unsigned)workgroups), block(256);
    if (dtype == TT_F64)
        hipLaunchKernelGGL(mfma_rate_kernel<double>, grid, block, 0, st, iters, static_cast<double*>(out));
    else if (dtype == TT_F32)
        hipLaunchKernelGGL(mfma_rate_kernel<float>, grid, block, 0, st, iters, static_cast<float*>(out));
    else if (dtype == TT_BF16)
        hipLaunchKernelGGL(mfma16_rate_kernel<__bf16>, grid, block, 0, st, iters, static_cast<unsigned short*>(out));
    else if (dtype == TT_F16)
        hipLaunchKernelGGL(mfma16_rate_kernel<_Float16>, grid, block, 0, st, iters, static_cast<unsigned short*>(out));
    else
        return set_error(TT_UNSUPPORTED, "tt_mfma_rate_probe: dtype %d (TT_F32, TT_F64, TT_BF16, TT_F16)", dtype);
    return check_launch("tt_mfma_rate_probe");
}
