// Host-side interface of the MFMA GEMM core shared by the C-ABI sources.
#pragma once

#include "tt_common.hpp"

namespace tt {

struct GemmArgs {
    const void* A;
    const void* B;
    const void* C;
    void* D;
    int64_t M, N, K;
    int64_t lda, ldb, ldc, ldd;
    int64_t sA, sB, sC, sD;
    int64_t batch;
    int64_t tiles_m, tiles_n;
    double alpha, beta;
    // Dot epilogue: instead of storing D, each workgroup writes
    // sum_{m,n} D[m,n] * E(m,n) to partial[workgroup], with
    // E(m,n) = E1[off1] * (E2 ? E2[off2] : 1), off = m_hi*s[0] + m_lo*s[1] +
    // n_hi*s[2] + n_lo*s[3] + batch*s[4], (m_hi, m_lo) = divmod(m, mdiv.d),
    // (n_hi, n_lo) = divmod(n, ndiv.d).
    const void* E1;
    const void* E2;
    int64_t e1s[5], e2s[5];
    FastDiv mdiv, ndiv;
    double* partial;
};

// tt_gemm after argument checks (store epilogue).
int gemm_dispatch(int dtype, bool ta, bool tb, GemmArgs& g, hipStream_t st);
// Double-double GEMM (dtype TT_F64_DD) on the vector ALUs; same arguments.
int gemm_dd_dispatch(bool ta, bool tb, GemmArgs& g, hipStream_t st);
// 16-bit GEMM (dtype TT_BF16 / TT_F16) on the 16x16x32 MFMA; same arguments.
int gemm16_dispatch(int dtype, bool ta, bool tb, GemmArgs& g, hipStream_t st);
// Its direct-load variant: 16-byte aligned operands (A, B, lda, ldb and
// batch strides multiples of 8 elements), whole tiles of gemm16_dma_tile,
// K a multiple of 32. gemm16_dma_rows: the tile height for a layout and K.
int gemm16_dma_dispatch(int dtype, bool ta, bool tb, GemmArgs& g, hipStream_t st);
int gemm16_dma_rows(bool ta, bool tb, int64_t K);
// Its tile (bm x bn) for an M x N x K problem of `batch` products.
void gemm16_dma_tile(bool ta, bool tb, int64_t M, int64_t N, int64_t K, int64_t batch, int& bm, int& bn);
// fp32 on 256 x 256 tiles (tt_gemm_big.hip): whether it takes the problem,
// and its launch.
bool gemm_big_f32_fits(bool ta, bool tb, const GemmArgs& g);
int gemm_big_f32_launch(GemmArgs& g, hipStream_t st);
// Dot epilogue; writes one double per workgroup to g.partial and returns the
// number of workgroups in *nparts.
int gemm_dot_dispatch(int dtype, bool ta, bool tb, GemmArgs& g, hipStream_t st, int64_t* nparts);

}  // namespace tt
