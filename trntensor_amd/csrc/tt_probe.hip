// Measurement aid: the MFMA rate this device sustains with no memory traffic,
// the denominator of the "fraction of the measured peak" next to each
// kernel's fraction of the datasheet peak.
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

}  // namespace

}  // namespace tt

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
