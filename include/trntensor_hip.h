/*
 * trntensor_hip.h — C ABI of libtrntensor_hip.so, the gfx950 (MI355X) kernel
 * library behind trntensor_amd's fused-contraction path.
 *
 * The reference (trntensor 0.4.0) has no native code; its device boundary is
 * the Python module trntensor/nki/dispatch.py, which hands padded, contiguous
 * tensors to four NKI kernels in trntensor/nki/_kernels.py. Each entry point
 * below replaces one of those kernels plus its dispatcher; the citation on
 * each declaration names the reference code it stands in for.
 *
 * Conventions (all entry points):
 *  - Plain pointers and sizes only. Every pointer named "device" is device
 *    memory on the current HIP device; the library never allocates or frees
 *    memory. Every entry point except tt_mp2_energy_noalloc keeps no mutable
 *    global state, so those calls are re-entrant; tt_mp2_energy_noalloc
 *    works in a per-device static array, so its calls that overlap on one
 *    device race (see its declaration).
 *  - `stream` is a hipStream_t passed as void*; NULL is the null stream.
 *    Work is enqueued on it and the call returns without synchronising.
 *  - dtype codes: TT_F32 = 0 (float), TT_F64 = 1 (double). TT_F64_DD = 2
 *    (tt_gemm, tt_strided_contract only): double data, every product formed
 *    exactly and summed in double-double (Ogita-Rump-Oishi Dot2), rounded
 *    to double once per output. TT_BF16 = 3, TT_F16 = 4 (tt_gemm only):
 *    16-bit A, B, C, D; products and sums in fp32 on the 16-bit MFMA, alpha
 *    and beta applied in fp32, one rounding at the store. TT_I64 = 5
 *    (tt_strided_contract only): int64 data, products and sums with
 *    two's-complement wraparound, integral alpha and beta.
 *  - Return codes: TT_OK 0; TT_INVALID 1 (bad argument: the Python layer
 *    raises ValueError); TT_UNSUPPORTED 2 (dtype/shape the kernels do not
 *    cover: NotImplementedError); TT_HIP_ERROR 3 (launch failure:
 *    RuntimeError). tt_last_error() returns a message for the calling
 *    thread's last failure.
 */
#ifndef TRNTENSOR_HIP_H
#define TRNTENSOR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TT_ABI_VERSION 4
#define TT_MAX_DIMS 8

enum { TT_OK = 0, TT_INVALID = 1, TT_UNSUPPORTED = 2, TT_HIP_ERROR = 3 };
enum { TT_F32 = 0, TT_F64 = 1, TT_F64_DD = 2, TT_BF16 = 3, TT_F16 = 4, TT_I64 = 5 };

/* ABI version of the loaded library (TT_ABI_VERSION at build time). */
int tt_abi_version(void);

/* Static name of a status code. */
const char* tt_status_string(int status);

/* Message for the calling thread's last non-OK return. */
const char* tt_last_error(void);

/*
 * Batched strided GEMM on the MFMA core, row-major:
 *   op(A)[m,k] = transA ? A[k*lda + m] : A[m*lda + k]
 *   op(B)[k,n] = transB ? B[n*ldb + k] : B[k*ldb + n]
 *   D[m*ldd + n] = alpha * sum_k op(A)[m,k] op(B)[k,n]  (+ beta * C[m*ldc + n])
 * for every batch b, each operand offset by b*stride. C is read iff it is
 * non-NULL (so beta*C is added whenever C is given, like torch's
 * add(out, alpha=beta)). D may alias C exactly. K may be 0.
 *
 * Replaces matmul_kernel (trntensor/nki/_kernels.py:35-75) behind
 * nki_matmul (trntensor/nki/dispatch.py:187-237) and batched_matmul_kernel
 * (_kernels.py:77-117) behind nki_batched_matmul (dispatch.py:339-387), and
 * additionally folds einsum's alpha/beta epilogue (trntensor/einsum.py:99-102)
 * into the store. No padding: edge tiles are masked in the kernel.
 *
 * dtype TT_F64_DD runs a double-double GEMM on the vector ALUs (no MFMA):
 * D = alpha * round(sum_k in double-double) (+ beta * C). It is the kernel
 * behind precision="dd", which the reference declares but rejects with
 * NotImplementedError (trntensor/einsum.py:112-116, plan.py:155).
 */
int tt_gemm(int dtype, int transA, int transB, int64_t M, int64_t N, int64_t K,
            double alpha, const void* A, int64_t lda, int64_t strideA,
            const void* B, int64_t ldb, int64_t strideB,
            double beta, const void* C, int64_t ldc, int64_t strideC,
            void* D, int64_t ldd, int64_t strideD, int64_t batch, void* stream);

/*
 * tt_gemm with its integer launch parameters in one array, for callers that
 * launch the same contraction shape many times and keep the array: params =
 * {dtype, transA, transB, M, N, K, lda, strideA, ldb, strideB, ldc, strideC,
 * ldd, strideD, batch} (15 values). Same checks, kernels and results as
 * tt_gemm. No counterpart in the reference: it shortens the host path of a
 * small device-resident einsum on a plan-cache hit (the Python front-end
 * passes 8 arguments instead of 22 through its FFI).
 */
int tt_gemm_packed(const int64_t* params, double alpha, double beta, const void* A, const void* B,
                   const void* C, void* D, void* stream);

/*
 * Workspace (device bytes) that tt_gemm_dot needs.
 */
size_t tt_gemm_dot_workspace_bytes(int dtype, int64_t M, int64_t N, int64_t batch);

/*
 * GEMM whose product is contracted on the spot instead of stored:
 *   out[0] = alpha * sum_{b,m,n} (sum_k op(A)[m,k] op(B)[k,n]) * E(b,m,n)  (+ beta * C[0])
 *   E(b,m,n) = E1[o(e1_strides)] * (E2 ? E2[o(e2_strides)] : 1),
 *   o(s) = m_hi*s[0] + m_lo*s[1] + n_hi*s[2] + n_lo*s[3] + b*s[4],
 *   (m_hi, m_lo) = divmod(m, m_lo_extent), (n_hi, n_lo) = divmod(n, n_lo_extent).
 * op(A), op(B), batch strides as in tt_gemm. E1 alone is a tensor with the
 * product's letters (any strides); E1 * E2 is an outer product of two factors
 * that is never materialised. Each workgroup contributes one partial, summed
 * in a fixed order. C (one element) is read iff non-NULL; out is one element.
 *
 * Replaces the last two steps of the reference's path executor when the final
 * step is a full dot of a GEMM-shaped step's result
 * (trntensor/einsum.py:151-193, each step a torch.einsum call at :188), e.g.
 * the 'abP,ijP->abij' and 'iajb,abij->' steps of 'ia,jb,abP,ijP->'.
 */
int tt_gemm_dot(int dtype, int transA, int transB, int64_t M, int64_t N, int64_t K,
                const void* A, int64_t lda, int64_t strideA,
                const void* B, int64_t ldb, int64_t strideB, int64_t batch,
                int64_t m_lo_extent, int64_t n_lo_extent,
                const void* E1, const int64_t* e1_strides,
                const void* E2, const int64_t* e2_strides,
                double alpha, double beta, const void* C, void* out,
                void* workspace, size_t workspace_bytes, void* stream);

/*
 * Workspace (device bytes) for tt_mp2_energy and tt_mp2_energy_shard: one
 * double per work unit plus one, and, when naux is not a multiple of 16, a
 * copy of B with each row padded with zeros to the next multiple of 16
 * elements (nocc * nvir * that many elements of dtype). Both calls accept any
 * workspace that holds the partials (this function's value for naux rounded
 * up to a multiple of 16); they make the padded copy, and then run at the
 * rate of an aligned naux, only when the workspace holds it too and starts
 * on a 256-byte boundary. The energy is the same, bitwise, either way.
 */
size_t tt_mp2_energy_workspace_bytes(int dtype, int64_t nocc, int64_t nvir, int64_t naux);

/*
 * Density-fitted MP2 correlation energy
 *   E = sum_{ijab} T_ijab (2 T_ijab - T_ijba) / (e_i + e_j - e_a - e_b),
 *   T_ijab = sum_P B[i,a,P] B[j,b,P]
 * with B contiguous (nocc, nvir, naux), eps_occ (nocc), eps_vir (nvir), all
 * of `dtype`. Writes one element of `dtype` to energy_out (device). T never
 * reaches memory: each workgroup forms a 64x64 block of T_ij and its
 * exchange partner on MFMA, applies the denominator and exchange term in
 * registers and reduces to one double. deterministic != 0 writes one partial
 * per workgroup and sums them in a fixed order in a second kernel;
 * deterministic == 0 adds each workgroup's value with one atomic.
 *
 * Replaces mp2_energy_kernel (trntensor/nki/_kernels.py:119-207) behind
 * _nki_mp2_energy (trntensor/nki/dispatch.py:240-283), without its
 * nvir <= 128 / naux <= 128 limits (trntensor/quantum.py:72-76).
 */
int tt_mp2_energy(int dtype, int64_t nocc, int64_t nvir, int64_t naux,
                  const void* B, const void* eps_occ, const void* eps_vir,
                  void* energy_out, void* workspace, size_t workspace_bytes,
                  int deterministic, void* stream);

/*
 * Number of MP2 work units for nocc, nvir: one per occupied pair i <= j and
 * pair of 64-row virtual blocks p <= q, numbered pair-major
 * (nocc(nocc+1)/2 * nblk(nblk+1)/2, nblk = ceil(nvir/64)).
 */
int64_t tt_mp2_energy_unit_count(int64_t nocc, int64_t nvir);

/*
 * The part of the MP2 energy that work units [first_unit, first_unit +
 * n_units) contribute, written to energy_out (one element of dtype); the
 * units of any partition of [0, tt_mp2_energy_unit_count) sum to the
 * tt_mp2_energy result (up to the rounding of that final sum). Arguments and
 * workspace as tt_mp2_energy. No counterpart in the reference: it is the
 * single-GPU piece of a sharded MP2 (each GPU takes a contiguous range of
 * units with B replicated, then one scalar all-reduce).
 */
int tt_mp2_energy_shard(int dtype, int64_t nocc, int64_t nvir, int64_t naux,
                        const void* B, const void* eps_occ, const void* eps_vir,
                        int64_t first_unit, int64_t n_units,
                        void* energy_out, void* workspace, size_t workspace_bytes,
                        int deterministic, void* stream);

/*
 * tt_mp2_energy without a workspace, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). No counterpart in the reference. Same arguments,
 * kernels and result as tt_mp2_energy, bitwise; the partials (deterministic
 * != 0: nocc(nocc+1)/2 * nblk(nblk+1)/2 + 1 doubles, nblk = ceil(nvir/64))
 * or the atomic accumulator (deterministic == 0: one double) live in a
 * static device array of 2^21 doubles (16 MiB) that each device holds until
 * the process ends. A deterministic problem needing more returns TT_INVALID.
 * The call allocates nothing. Every call on one device shares that array,
 * so calls that overlap on one device (different streams, or threads) race;
 * calls ordered on one stream do not. The first call on each device looks
 * up the array's device address (a runtime call, not a stream operation),
 * so it must be made outside stream capture: a first call while `stream`
 * is capturing returns TT_INVALID. Make one eager call on each device before
 * capturing; later calls record only kernel launches.
 */
int tt_mp2_energy_noalloc(int dtype, int64_t nocc, int64_t nvir, int64_t naux,
                          const void* B, const void* eps_occ, const void* eps_vir,
                          void* energy_out, int deterministic, void* stream);

/*
 * Workspace (device bytes) that tt_ao_to_mo_transform needs.
 */
size_t tt_ao_to_mo_workspace_bytes(int dtype, int64_t nbasis, int64_t nocc, int64_t nvir, int64_t naux);

/*
 * Full AO->MO transform B[i,a,P] = sum_{mu,nu} C_occ[mu,i] C_vir[nu,a] eri[mu,nu,P]
 * with eri contiguous (nbasis, nbasis, naux), C_occ (nbasis, nocc),
 * C_vir (nbasis, nvir), B_out contiguous (nocc, nvir, naux). Two MFMA GEMMs:
 * X[i,(nu,P)] = C_occ^T eri viewed (nbasis, nbasis*naux) into the workspace,
 * then B[i] = C_vir^T X[i] batched over i. All loads are P-contiguous.
 *
 * Replaces ao_to_mo_transform_kernel (trntensor/nki/_kernels.py:209-296)
 * behind _nki_ao_to_mo_transform (trntensor/nki/dispatch.py:286-336),
 * without its nbasis/nocc/nvir limits (trntensor/quantum.py:161-177).
 */
int tt_ao_to_mo_transform(int dtype, int64_t nbasis, int64_t nocc, int64_t nvir, int64_t naux,
                          const void* eri, const void* C_occ, const void* C_vir,
                          void* B_out, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Workspace (device bytes) that tt_strided_contract needs for these extents.
 */
size_t tt_strided_contract_workspace_bytes(int dtype, int n_out, const int64_t* out_shape,
                                           int n_red, const int64_t* red_shape);

/*
 * Strided multiply-reduce for contractions that have no GEMM shape (outer
 * products, traces, dots, permutations, letters summed away):
 *   D[o] = alpha * sum_r A[a_off(o) + a_roff(r)] * B[b_off(o) + b_roff(r)]  (+ beta * C[o])
 * o runs over out_shape (n_out <= 8 dims, row-major), r over red_shape
 * (n_red <= 8 dims); offsets are dot products of the multi-index with the
 * given element strides (0 broadcasts). B may be NULL (single operand:
 * the factor is 1). D and C are contiguous in out_shape order; C is read iff
 * non-NULL. Accumulation is in `dtype`; TT_F64_DD accumulates double data
 * in double-double (partial sums travel as pairs) and rounds once. TT_I64
 * accumulates int64 with wraparound (so any integer dtype widened to int64
 * and truncated back equals its own wrapping accumulation); it requires
 * integral alpha and beta (TT_INVALID otherwise).
 *
 * No counterpart kernel in the reference: these contractions are the
 * "torch" strategy, which the reference hands to torch.einsum
 * (trntensor/einsum.py:117-118) and its path executor's steps
 * (trntensor/einsum.py:188).
 */
int tt_strided_contract(int dtype, int n_out, const int64_t* out_shape,
                        const int64_t* a_out_strides, const int64_t* b_out_strides,
                        int n_red, const int64_t* red_shape,
                        const int64_t* a_red_strides, const int64_t* b_red_strides,
                        const void* A, const void* B, double alpha, double beta,
                        const void* C, void* D, void* workspace, size_t workspace_bytes,
                        void* stream);

/*
 * Measurement aid with no counterpart in the reference: `workgroups`
 * workgroups of 4 wavefronts each run `iters` rounds of 8 independent MFMA
 * accumulator chains from register operands and write one value per
 * workgroup to out (device, `workgroups` elements of dtype). TT_F32/TT_F64:
 * 16x16x4 MFMA, 8 * 2048 FLOP per wavefront per round; TT_BF16/TT_F16:
 * 16x16x32 MFMA with fp32 accumulators, 8 * 16384 FLOP per wavefront per round. Timing it gives
 * the MFMA rate the device sustains without memory traffic, the measured
 * peak that the benchmark reports next to the datasheet peak.
 */
int tt_mfma_rate_probe(int dtype, int64_t workgroups, int64_t iters, void* out, void* stream);

/*
 * Measurement aid with no counterpart in the reference: streams `bytes`
 * (a multiple of 16) through HBM with 16-byte accesses from `workgroups`
 * workgroups of 256 threads, grid-stride. mode 0 reads src (device; `flag`,
 * one device uint32, is written only if the data's XOR equals a fixed word,
 * so the loads cannot be dropped), mode 1 writes dst, mode 2 copies src to
 * dst (the two must not overlap). Modes 0-2 use non-temporal accesses;
 * modes 4-6 are the same through the caches. src and dst 16-byte aligned.
 * Timing it on
 * buffers well beyond the 256 MB MALL gives the HBM rate the device
 * sustains, the measured peak the benchmark reports beside the 8 TB/s
 * datasheet figure.
 */
int tt_hbm_probe(int mode, const void* src, void* dst, int64_t bytes, int64_t workgroups, void* flag,
                 void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TRNTENSOR_HIP_H */
