// C-ABI housekeeping (version, status strings, per-thread error text) and the
// AO->MO transform composed from two MFMA GEMM launches.
#include <stdarg.h>
#include <string.h>

#include "tt_gemm.hpp"

namespace tt {



static thread_local char g_err[512];

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

static GemmArgs gemm_args(int64_t M, int64_t N, int64_t K, const void* A, int64_t lda, int64_t sA, const void* B,
                          int64_t ldb, int64_t sB, void* D, int64_t ldd, int64_t sD, int64_t batch) {
    GemmArgs g;
    memset(&g, 0, sizeof(g));
    g.A = A;
    g.B = B;
    g.C = nullptr;
    g.D = D;
    g.M = M;
    g.N = N;
    g.K = K;
    g.lda = lda;
    g.ldb = ldb;
    g.ldd = ldd;
    g.sA = sA;
    g.sB = sB;
    g.sD = sD;
    g.batch = batch;
    g.alpha = 1.0;
    g.beta = 0.0;
    return g;
}

}  // namespace tt

extern "C" int tt_abi_version(void) { return TT_ABI_VERSION; }

extern "C" const char* tt_status_string(int status) {
    switch (status) {
        case TT_OK:
            return "ok";
        case TT_INVALID:
            return "invalid argument";
        case TT_UNSUPPORTED:
            return "unsupported dtype or shape";
        case TT_HIP_ERROR:
            return "HIP runtime error";
        default:
            return "unknown status";
    }
}

extern "C" const char* tt_last_error(void) { return tt::g_err; }

extern "C" size_t tt_ao_to_mo_workspace_bytes(int dtype, int64_t nbasis, int64_t nocc, int64_t nvir, int64_t naux) {
    (void)nvir;
    if (nbasis < 0 || nocc < 0 || naux < 0) return 0;
    const size_t es = dtype == TT_F64 ? 8 : 4;
    return ((size_t)(nocc * nbasis * naux) * es + 255) / 256 * 256;
}

extern "C" int tt_ao_to_mo_transform(int dtype, int64_t nbasis, int64_t nocc, int64_t nvir, int64_t naux,
                                     const void* eri, const void* C_occ, const void* C_vir, void* B_out,
                                     void* workspace, size_t workspace_bytes, void* stream) {
    using namespace tt;
    if (nbasis < 0 || nocc < 0 || nvir < 0 || naux < 0)
        return set_error(TT_INVALID, "tt_ao_to_mo_transform: negative extent");
    if (dtype != TT_F32 && dtype != TT_F64)
        return set_error(TT_UNSUPPORTED, "tt_ao_to_mo_transform: dtype %d (only TT_F32, TT_F64)", dtype);
    if (nocc == 0 || nvir == 0 || naux == 0) return TT_OK;
    if (!B_out || (nbasis > 0 && (!eri || !C_occ || !C_vir)))
        return set_error(TT_INVALID, "tt_ao_to_mo_transform: NULL pointer");
    const size_t need = tt_ao_to_mo_workspace_bytes(dtype, nbasis, nocc, nvir, naux);
    if (!workspace || workspace_bytes < need)
        return set_error(TT_INVALID, "tt_ao_to_mo_transform: workspace of %zu bytes, need %zu", workspace_bytes, need);
    hipStream_t st = static_cast<hipStream_t>(stream);
    // Step 1: X[i, (nu, P)] = sum_mu C_occ[mu, i] eri[mu, (nu, P)]  (A = C_occ^T, B = eri as (nbasis, nbasis*naux)).
    const int64_t NP = nbasis * naux;
    GemmArgs g1 = gemm_args(nocc, NP, nbasis, C_occ, nocc, 0, eri, NP, 0, workspace, NP, 0, 1);
    int rc = gemm_dispatch(dtype, true, false, g1, st);
    if (rc != TT_OK) return rc;
    // Step 2: B[i] (nvir, naux) = sum_nu C_vir[nu, a] X[i][nu, P], batched over i.
    GemmArgs g2 = gemm_args(nvir, naux, nbasis, C_vir, nvir, 0, workspace, naux, NP, B_out, naux, nvir * naux, nocc);
    return gemm_dispatch(dtype, true, false, g2, st);
}
