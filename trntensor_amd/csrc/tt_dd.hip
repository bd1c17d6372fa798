// Double-double GEMM on the vector ALUs: the kernel behind precision="dd".
//   D[b][m, n] = alpha * dd_sum_k op(A)[m, k] op(B)[k, n]  (+ beta * C[b][m, n])
// Each product is formed exactly (TwoProduct) and summed into a (p, s) pair
// per output (Dot2, see tt_common.hpp), so an output is the dot product
// accumulated in about twice double precision and rounded to double once.
//
// Tile: 64 x 64 outputs per 256-thread workgroup, 4 x 4 per thread
// (rows 4 ty + i, columns 4 tx + j with tx = t % 16, ty = t / 16), K staged
// through LDS 16 at a time as As[k][m] and Bs[k][n]. The work is VALU-bound
// (10 double-precision VALU operations per multiply-add against 2 LDS reads
// of 32 bytes per 16 multiply-adds), so the global loads are plain
// bounds-checked element loads: 4 consecutive elements per thread along the
// operand's contiguous direction, the next stage prefetched into registers
// while the current one is computed.
#include "tt_gemm.hpp"

namespace tt {

namespace {

constexpr int kDdTile = 64;
constexpr int kDdK = 16;
constexpr int kDdPitch = kDdTile + 4;  // rows stay 32-byte aligned; k rows start on different banks

template <bool TA, bool TB>
__global__ __launch_bounds__(256) void gemm_dd_kernel(GemmArgs g) {
    __shared__ __attribute__((aligned(32))) double As[kDdK][kDdPitch];
    __shared__ __attribute__((aligned(32))) double Bs[kDdK][kDdPitch];
    const int t = threadIdx.x;
    const int64_t tiles = g.tiles_m * g.tiles_n;
    const int64_t w = blockIdx.x;
    const int64_t bat = w / tiles;
    const int64_t rem = w - bat * tiles;
    const int64_t tm = rem / g.tiles_n;
    const int64_t tn = rem - tm * g.tiles_n;
    const int64_t m0 = tm * kDdTile, n0 = tn * kDdTile;
    const double* A = static_cast<const double*>(g.A) + bat * g.sA;
    const double* B = static_cast<const double*>(g.B) + bat * g.sB;

    // op(A)[m, k] = TA ? A[k * lda + m] : A[m * lda + k]
    // op(B)[k, n] = TB ? B[n * ldb + k] : B[k * ldb + n]
    const int a_k = TA ? t / 16 : (t % 4) * 4;
    const int a_m = TA ? (t % 16) * 4 : t / 4;
    const int b_k = TB ? (t % 4) * 4 : t / 16;
    const int b_n = TB ? t / 4 : (t % 16) * 4;
    double ra[4], rb[4];

    auto load = [&](int64_t k0) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int64_t m = m0 + a_m + (TA ? e : 0);
            const int64_t k = k0 + a_k + (TA ? 0 : e);
            const bool ok = m < g.M && k < g.K;
            const int64_t off = ok ? (TA ? k * g.lda + m : m * g.lda + k) : 0;
            const double v = A[off];
            ra[e] = ok ? v : 0.0;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int64_t n = n0 + b_n + (TB ? 0 : e);
            const int64_t k = k0 + b_k + (TB ? e : 0);
            const bool ok = n < g.N && k < g.K;
            const int64_t off = ok ? (TB ? n * g.ldb + k : k * g.ldb + n) : 0;
            const double v = B[off];
            rb[e] = ok ? v : 0.0;
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int e = 0; e < 4; ++e) As[a_k + (TA ? 0 : e)][a_m + (TA ? e : 0)] = ra[e];
#pragma unroll
        for (int e = 0; e < 4; ++e) Bs[b_k + (TB ? e : 0)][b_n + (TB ? 0 : e)] = rb[e];
    };

    const int tx = t % 16, ty = t / 16;
    Dot2 acc[4][4];
    if (g.K > 0) load(0);
    for (int64_t k0 = 0; k0 < g.K; k0 += kDdK) {
        __syncthreads();  // the previous stage's LDS reads are done
        stage();
        __syncthreads();
        if (k0 + kDdK < g.K) load(k0 + kDdK);
#pragma unroll 2
        for (int kk = 0; kk < kDdK; ++kk) {
            const d4_t a = *reinterpret_cast<const d4_t*>(&As[kk][ty * 4]);
            const d4_t b = *reinterpret_cast<const d4_t*>(&Bs[kk][tx * 4]);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j].add_prod(a[i], b[j]);
        }
    }

    double* D = static_cast<double*>(g.D) + bat * g.sD;
    const double* C = g.C ? static_cast<const double*>(g.C) + bat * g.sC : nullptr;
    // All 16 C values are loaded (clamped addresses, branch-free) before the
    // first store: D may alias C, so loads placed between stores could not be
    // moved ahead of them and would each wait out a memory latency.
    double cv[4][4];
    if (C) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t m = m0 + ty * 4 + i, n = n0 + tx * 4 + j;
                const bool ok = m < g.M && n < g.N;
                const double c = C[ok ? m * g.ldc + n : 0];
                cv[i][j] = ok ? c : 0.0;
            }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t m = m0 + ty * 4 + i;
        if (m >= g.M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t n = n0 + tx * 4 + j;
            if (n >= g.N) continue;
            double v = acc[i][j].value();
            if (g.alpha != 1.0) v = g.alpha * v;
            if (C) v = v + g.beta * cv[i][j];
            D[m * g.ldd + n] = v;
        }
    }
}

}  // namespace

int gemm_dd_dispatch(bool ta, bool tb, GemmArgs& g, hipStream_t st) {
    g.tiles_m = (g.M + kDdTile - 1) / kDdTile;
    g.tiles_n = (g.N + kDdTile - 1) / kDdTile;
    const int64_t total = g.tiles_m * g.tiles_n * g.batch;
    if (total > 0x7fffffffLL)
        return set_error(TT_UNSUPPORTED, "tt_gemm: %lld tiles exceed one launch", (long long)total);
    const dim3 grid((unsigned)total), block(256);
    if (!ta && !tb) hipLaunchKernelGGL((gemm_dd_kernel<false, false>), grid, block, 0, st, g);
    if (!ta && tb) hipLaunchKernelGGL((gemm_dd_kernel<false, true>), grid, block, 0, st, g);
    if (ta && !tb) hipLaunchKernelGGL((gemm_dd_kernel<true, false>), grid, block, 0, st, g);
    if (ta && tb) hipLaunchKernelGGL((gemm_dd_kernel<true, true>), grid, block, 0, st, g);
    return check_launch("tt_gemm (double-double)");
}

}  // namespace tt
