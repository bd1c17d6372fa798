// Measurement aid: the MFMA rate this device sustains with no memory traffic,
// the denominator of the "fraction of the measured peak" next to each
// kernel's fraction of the datasheet peak.
//
// Every wavefront runs `iters` rounds of 8 independent accumulator chains of
// the same 16x16x4 MFMA the kernels use (f64 or f32), i.e. 8 * 2048 FLOP per
// round, from register operands only. One value per workgroup is written so
// the work cannot be removed.
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
    else
        return set_error(TT_UNSUPPORTED, "tt_mfma_rate_probe: dtype %d (only TT_F32, TT_F64)", dtype);
    return check_launch("tt_mfma_rate_probe");
}
