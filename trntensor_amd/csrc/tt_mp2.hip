// Fused DF-MP2 correlation energy for gfx950.
//
//   E = sum_{ij} sum_{ab} T_ab (2 T_ab - T_ba) / (e_i + e_j - e_a - e_b),
//   T = T^{ij} = B_i B_j^T,  B_i = B[i] : (nvir, naux), P contiguous.
//
// Work unit: occupied pair i <= j and virtual 64-blocks p <= q. Because
// T^{ij}_{ba} = (B_j[p] B_i[q]^T)_{ab} for a in block p and b in block q,
// one workgroup forms
//   X = B_i[p] B_j[q]^T    (T_ab for a in p, b in q)
//   Y = B_j[p] B_i[q]^T    (T_ba at the same (a, b) position)
// in the same register layout, so the exchange term pairs X and Y element by
// element. Y comes from MFMA only for i < j, p < q; for p = q it is X^T
// (one transpose through LDS), for i = j, p < q it is X itself. For p < q
// the unit also accounts for the mirrored block (q, p), whose terms are
// Y (2Y - X) / Delta_ba. For i < j the unit's sum is doubled, since the
// (j, i) pair contributes the same amount (Delta is symmetric).
// T never leaves registers and LDS; each workgroup reduces to one double with
// wavefront shuffles and either stores it (deterministic mode, summed later
// in a fixed order) or adds it with one atomic.
//
// Per-element arithmetic follows the reference's operation order
// (trntensor/quantum.py:97-99): denominator ((e_i + e_j) - e_a) - e_b with a
// the row index, term (T * (2T - T^T)) / denominator with IEEE division, in
// the input dtype; the energy is accumulated in double.
#include <mutex>
#include <type_traits>

#include "tt_common.hpp"

namespace tt {

constexpr int kMp2Threads = 256;
constexpr int kMp2Tile = 64;
// Occupied pairs per group of the unit order (see mp2_energy_kernel). Same
// box, one process, alternating, against one pair per group: config 4 fp64
// 7.366 against 7.477 ms and 7.393 against 7.500 ms, fp32 3.932 against
// 3.961 ms, naux 2400 fp64 15.33 against 15.42 ms, nocc 128 / nvir 640 /
// naux 2400 243.0 against 243.2 ms (groups of 8: 7.401, 3.960, 15.26, 241.8;
// of 64: 7.389, 3.902, 15.31, 243.4).
constexpr int kMp2PairGroup = 16;
#ifndef TT_MP2_STAGE_K
#define TT_MP2_STAGE_K 16
#endif
constexpr int kMp2StageK = TT_MP2_STAGE_K;  // k per LDS stage

// One 64-row x BK stage of a B_i block, k contiguous in memory and in LDS
// (row pitch BK + 16 bytes). Thread t stages row t / 4, elements
// [(t % 4) E, (t % 4) E + E) with E = BK / 4: four consecutive threads read
// one row's BK contiguous values. MFMA step s of a stage gives lane group
// g = lane / 16 the k index E g + s, so a lane's E values per stage are
// adjacent in LDS and one vector read feeds E MFMAs.
//
// AW is the global access width in elements: each thread's E values are
// E / AW loads of AW consecutive elements. The launcher picks the widest AW
// (16, 8 or 4 bytes) that every row start (a multiple of naux from B's base)
// keeps naturally aligned, so rows of any naux take the branch-free
// interior loop; only the access width narrows.
template <typename T, int BK, int AW>
struct Panel {
    static constexpr int E = BK / 4;  // elements per thread, = MFMA steps per stage
    static constexpr int NP = E / AW;  // global loads per thread per stage
    static constexpr int PITCH = BK + 16 / sizeof(T);
    static constexpr int ELEMS = kMp2Tile * PITCH;
    static_assert(BK == 8 || BK == 16, "stage depth");
    static_assert(AW >= 1 && E % AW == 0 && AW * sizeof(T) <= 16, "access width");
    typedef typename VecN<T, E>::type vec_t;
    typedef typename VecN<T, AW>::type piece_t;

    vec_t reg;

    __device__ __forceinline__ void put(int c, piece_t x) {
#pragma unroll
        for (int e = 0; e < AW; ++e) reg[c * AW + e] = x[e];
    }

    // FAST (interior stage: BK k in range): NP unconditional loads; in a
    // block with fewer than 64 rows the rows past its end read its last row
    // again (their products are never used: the energy loop skips rows and
    // columns past the block). Otherwise (the K tail) each AW-piece is one
    // load when it lies inside, zero without a load when it lies outside,
    // and element loads from clamped addresses only when it straddles the
    // end of the row.
    template <bool FAST>
    __device__ __forceinline__ void load(const T* __restrict__ base, int rows, int64_t naux, int64_t k0) {
        const int r = FAST ? min((int)(threadIdx.x >> 2), rows - 1) : (int)(threadIdx.x >> 2);
        const int k = (threadIdx.x & 3) * E;
        const T* row = base + (int64_t)r * naux;
        if (FAST) {
#pragma unroll
            for (int c = 0; c < NP; ++c) put(c, *reinterpret_cast<const piece_t*>(row + k0 + k + c * AW));
            return;
        }
#pragma unroll
        for (int c = 0; c < NP; ++c) {
            const int64_t gk = k0 + k + c * AW;
            if (r < rows && gk + AW <= naux) {
                put(c, *reinterpret_cast<const piece_t*>(row + gk));
            } else if (r >= rows || gk >= naux) {
#pragma unroll
                for (int e = 0; e < AW; ++e) reg[c * AW + e] = T(0);
            } else {
#pragma unroll
                for (int e = 0; e < AW; ++e) {
                    const bool ok = gk + e < naux;
                    const T x = *(ok ? row + gk + e : row);
                    reg[c * AW + e] = ok ? x : T(0);
                }
            }
        }
    }

    __device__ __forceinline__ void store(T* s) const {
        *reinterpret_cast<vec_t*>(s + (threadIdx.x >> 2) * PITCH + (threadIdx.x & 3) * E) = reg;
    }

    // Lane's E k values (MFMA steps 0..E-1) for rows rb..rb+15.
    __device__ __forceinline__ static vec_t frag(const T* s, int rb, int lane) {
        return *reinterpret_cast<const vec_t*>(s + (rb + (lane & 15)) * PITCH + E * (lane >> 4));
    }
};

struct Mp2Args {
    const void* B;
    const void* eo;
    const void* ev;
    double* partial;  // one per workgroup (deterministic) or nullptr
    double* accum;    // atomic accumulator (non-deterministic) or nullptr
    int64_t naux;
    int nocc, nvir, nblk;
    int64_t npq;     // nblk * (nblk + 1) / 2
    int64_t first;   // first work unit of this launch
    int64_t ntasks;  // work units in this launch (of npq * nocc * (nocc + 1) / 2)
};

// Index of (x, y), x <= y < n, in row-major upper-triangle order -> (x, y).
__device__ __forceinline__ void tri_decode(int64_t idx, int n, int& x, int& y) {
    int r = 0;
    while (idx >= n - r) {
        idx -= n - r;
        ++r;
    }
    x = r;
    y = r + (int)idx;
}

// K loop of one work unit: X = P0 Q0^T and, if NEED_Y, Y = P2 Q3^T, BK k per
// stage. Stages whose successor is interior run in the first loop with
// unconditional prefetch; the rest (edge rows, the K remainder, the last
// stage) run in the second loop.
template <typename T, int BK, int AW, bool NEED_Y>
__device__ __forceinline__ void mp2_kloop(T* lds_base, const T* base0, const T* base1,
                                          const T* base2, const T* base3, int rows_p, int rows_q, int64_t naux,
                                          typename Mfma<T>::acc_t (&X)[2][2], typename Mfma<T>::acc_t (&Y)[2][2]) {
    typedef Mfma<T> MF;
    typedef Panel<T, BK, AW> PN;
    constexpr int KS = PN::E;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wr = (wave >> 1) * 32;
    const int wc = (wave & 1) * 32;
    const int64_t nk = (naux + BK - 1) / BK;
    // Stages 0 .. nfull-1 are interior (all BK k in range). Ragged blocks (fewer than 64 rows) take this loop too, their missing
    // rows reading the block's last row: config 4's shape with nvir 300
    // (44-row last block) ran 5.0 ms fp32 with those units in the guarded
    // loop.
    const int64_t nfull = naux / BK;

    // DQ (with Y): each wave's two column fragments (B_j[q] for the X
    // waves, B_i[q] for the Y waves) go from memory straight into registers: a
    // lane's fragment is E consecutive k of one row, the same values the LDS
    // fragment read gives, so energies are bitwise those of staging all four
    // panels. Only the row panels B_i[p] and B_j[p] pass through LDS, which
    // halves the LDS stores and cuts the fragment reads per wave from six to
    // four per stage. A fragment is reloaded for the next stage as soon as its
    // MFMAs have issued. Config 4 (fp64), same box, alternating: 7.73-7.74
    // against 7.95-7.98 ms (naux 1199: 7.77 against 8.05 ms). Double-buffering
    // the two row panels (one barrier per stage, same LDS) measured the same
    // (7.72-7.77 ms); four waves per SIMD would spill 137 registers. fp32
    // (the same split, 100 VGPRs, four workgroups per CU instead of five with
    // quadrants): 4.00-4.02 against 4.11-4.12 ms, naux 1199 4.05 against 4.13
    // ms, energies bitwise equal.
    constexpr bool DQ = NEED_Y;
    // Stage buffer b, panel k at lds_base + (4 b + k) * ELEMS; with DQ only
    // panels 0 and 2 are staged, at lds_base + (2 b + k / 2) * ELEMS.
    auto lds = [&](int b, int k) -> T* { return lds_base + (DQ ? 2 * b + (k >> 1) : 4 * b + k) * PN::ELEMS; };
    const int qmat = wave >> 1;
    const int qch = (wave & 1) * 32;
    const T* qbase = qmat ? base3 : base1;
    typename PN::vec_t fq[2];
    auto qload = [&](int b, int64_t k0, auto fast) __attribute__((always_inline)) {
        constexpr bool F = decltype(fast)::value;
        const int r = F ? min(qch + 16 * b + (lane & 15), rows_q - 1) : qch + 16 * b + (lane & 15);
        const int64_t k = k0 + PN::E * (lane >> 4);
        const T* row = qbase + (int64_t)r * naux;
#pragma unroll
        for (int c = 0; c < PN::NP; ++c) {
            const int64_t gk = k + c * AW;
            typename PN::piece_t x;
            if (F || (r < rows_q && gk + AW <= naux)) {
                x = *reinterpret_cast<const typename PN::piece_t*>(row + gk);
            } else {
#pragma unroll
                for (int e = 0; e < AW; ++e) {
                    const bool ok = r < rows_q && gk + e < naux;
                    const T v = *(ok ? row + gk + e : qbase);
                    x[e] = ok ? v : T(0);
                }
            }
#pragma unroll
            for (int e = 0; e < AW; ++e) fq[b][c * AW + e] = x[e];
        }
    };
    PN s0, s1, s2, s3;
    auto load = [&](int64_t k0, auto fast) {
        constexpr bool F = decltype(fast)::value;
        s0.template load<F>(base0, rows_p, naux, k0);
        if (!DQ) s1.template load<F>(base1, rows_q, naux, k0);
        if (NEED_Y) {
            s2.template load<F>(base2, rows_p, naux, k0);
            if (!DQ) s3.template load<F>(base3, rows_q, naux, k0);
        }
    };
    auto store = [&](int buf) {
        s0.store(lds(buf, 0));
        if (!DQ) s1.store(lds(buf, 1));
        if (NEED_Y) {
            s2.store(lds(buf, 2));
            if (!DQ) s3.store(lds(buf, 3));
        }
    };
    // next: 0 = no next stage, 1 = interior next stage, 2 = edge next stage
    // (the column fragments of stage k0n are loaded right after their MFMAs).
    auto compute = [&](int buf, int64_t k0n, int next) {
        if (DQ) {
            // Waves 0, 1 form X = P0 P1^T and waves 2, 3 Y = P2 P3^T, each a
            // 64 x 32 half (columns qch .. qch + 31; row blocks 0, 1 in
            // X[.][.], 2, 3 in Y[.][.]); the epilogue pairs X and Y through
            // LDS. With all four panels staged, this split read six fragments
            // per stage for a wave's 32 MFMAs instead of eight for quadrants
            // of both (fp64 166 -> 158 VGPRs; config 4 7.86-7.87 against 7.93
            // ms; fp32 measured the same at 104 VGPRs).
            const T* rp = lds(buf, qmat ? 2 : 0);
            typename PN::vec_t fr[4];
#pragma unroll
            for (int a = 0; a < 4; ++a) fr[a] = PN::frag(rp, 16 * a, lane);
#pragma unroll
            for (int b = 0; b < 2; ++b) {
#pragma unroll
                for (int st = 0; st < KS; ++st)
#pragma unroll
                    for (int a = 0; a < 2; ++a) {
                        X[a][b] = MF::mma(fr[a][st], fq[b][st], X[a][b]);
                        Y[a][b] = MF::mma(fr[a + 2][st], fq[b][st], Y[a][b]);
                    }
                if (next == 1) qload(b, k0n, std::true_type{});
                else if (next == 2) qload(b, k0n, std::false_type{});
            }
            return;
        }
        // X only (i = j or p = q): quadrants, both panels through LDS.
        typename PN::vec_t f0[2], f1[2];
#pragma unroll
        for (int a = 0; a < 2; ++a) f0[a] = PN::frag(lds(buf, 0), wr + 16 * a, lane);
#pragma unroll
        for (int b = 0; b < 2; ++b) f1[b] = PN::frag(lds(buf, 1), wc + 16 * b, lane);
#pragma unroll
        for (int st = 0; st < KS; ++st)
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b) X[a][b] = MF::mma(f0[a][st], f1[b][st], X[a][b]);
    };

    // One LDS stage buffer and one register prefetch set: while stage k is
    // multiplied out of LDS, stage k+1 is in flight in registers; after a
    // barrier it replaces stage k. Half the LDS of double buffering buys a
    // third workgroup per CU, whose MFMAs cover the extra barrier. The
    // scheduling barrier keeps the wait for the prefetch behind the MFMAs.
    // All waves run at the default priority. With all four panels staged,
    // raising the fp64 wave's priority over its stage's MFMAs gained 5 points
    // of MFMA utilisation; with the column fragments loaded directly it costs
    // 0.7% (config 4, same box, alternating: 7.65 against 7.70 ms; fp32 4.10
    // against 4.00 ms), so neither dtype raises it.
    if (nk == 0) return;
    if (nfull > 0) {
        load(0, std::true_type{});
        if (DQ) qload(0, 0, std::true_type{}), qload(1, 0, std::true_type{});
    } else {
        load(0, std::false_type{});
        if (DQ) qload(0, 0, std::false_type{}), qload(1, 0, std::false_type{});
    }
    store(0);
    __syncthreads();
    int64_t kt = 0;
    for (; kt + 1 < nfull; ++kt) {
        load((kt + 1) * BK, std::true_type{});
        compute(0, (kt + 1) * BK, 1);
        if constexpr (DQ && sizeof(T) == 4) {
            // fp32: one of the stage's four loads (two staged panels, then
            // the two column fragments) after every 8 MFMAs; left alone the
            // compiler bunched all four after the 28th. Config 4 fp32, same
            // box, alternating, bitwise equal: 3.900-3.913 against 3.942-3.970
            // ms (nvir 300: 4.91 against 5.01 ms). The staged panels' loads
            // after the 4th and 8th MFMA instead: 4.11-4.13 ms; the same
            // spacing in fp64 (eight loads): -0.6% at naux 1200, +0.7% at 2400.
            constexpr int NL = 4 * PN::NP;  // loads per thread per stage
            constexpr int NM = 8 * KS;      // MFMAs per wave per stage
#pragma unroll
            for (int l = 0; l < NL; ++l) {
                __builtin_amdgcn_sched_group_barrier(0x008, NM / NL, 0);
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        store(0);
        __syncthreads();
    }
    for (; kt < nk; ++kt) {
        const bool more = kt + 1 < nk;
        if (more) load((kt + 1) * BK, std::false_type{});
        compute(0, (kt + 1) * BK, more ? 2 : 0);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        if (more) store(0);
        __syncthreads();
    }
}

template <typename T, int BK, int AW>
__global__ __launch_bounds__(kMp2Threads) void mp2_energy_kernel(Mp2Args g) {
    typedef Mfma<T> MF;
    typedef typename MF::acc_t acc_t;
    typedef Panel<T, BK, AW> PN;

    __shared__ __attribute__((aligned(16))) T lds[1][4][PN::ELEMS];
    __shared__ double red[4];

    const int64_t local = xcd_remap(blockIdx.x, g.ntasks);
    const int64_t task = g.first + local;
    // Unit order: groups of kMp2PairGroup occupied pairs; within a group, the
    // off-diagonal units (p < q) of all its pairs first, pair-major and
    // row-major over p < q, then its diagonal units (p = q). A diagonal unit
    // issues half the MFMAs per stage and runs ahead of the off-diagonal
    // units that read the same panels; grouped, each kind keeps the pace of
    // the units it shares panels with, and short units end each group.
    const int64_t noff = (int64_t)g.nblk * (g.nblk - 1) / 2;  // off-diagonal units per pair
    int64_t pair, u;
    {
        const int64_t npairs = (int64_t)g.nocc * (g.nocc + 1) / 2;
        const int64_t grp = task / (kMp2PairGroup * g.npq);
        const int64_t gp = min((int64_t)kMp2PairGroup, npairs - grp * kMp2PairGroup);  // pairs in this group
        const int64_t r = task - grp * kMp2PairGroup * g.npq;
        if (r < gp * noff) {
            pair = grp * kMp2PairGroup + r / noff;
            u = r % noff;
        } else {
            const int64_t r2 = r - gp * noff;
            pair = grp * kMp2PairGroup + r2 / g.nblk;
            u = noff + r2 % g.nblk;
        }
    }
    int i, j, p, q;
    tri_decode(pair, g.nocc, i, j);
    // u < noff: the off-diagonal units in row-major order over p < q; then
    // the diagonal ones.
    if (u < noff) {
        tri_decode(u, g.nblk - 1, p, q);
        q += 1;
    } else {
        p = q = (int)(u - noff);
    }
    // Y source: 0 = MFMA (i < j, p < q), 1 = X itself (i = j, p < q), 2 = X^T (p = q).
    const int ymode = (p == q) ? 2 : (i == j ? 1 : 0);

    const T* B = static_cast<const T*>(g.B);
    const int64_t nvir = g.nvir;
    const int rows_p = min(kMp2Tile, g.nvir - p * kMp2Tile);
    const int rows_q = min(kMp2Tile, g.nvir - q * kMp2Tile);
    // Panels: 0 = B_i[p], 1 = B_j[q], 2 = B_j[p], 3 = B_i[q].
    const T* base0 = B + ((int64_t)i * nvir + (int64_t)p * kMp2Tile) * g.naux;
    const T* base1 = B + ((int64_t)j * nvir + (int64_t)q * kMp2Tile) * g.naux;
    const T* base2 = B + ((int64_t)j * nvir + (int64_t)p * kMp2Tile) * g.naux;
    const T* base3 = B + ((int64_t)i * nvir + (int64_t)q * kMp2Tile) * g.naux;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wr = (wave >> 1) * 32;  // quadrant row offset (a within p)
    const int wc = (wave & 1) * 32;   // quadrant col offset (b within q)

    acc_t X[2][2], Y[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            X[a][b] = acc_t{0, 0, 0, 0};
            Y[a][b] = acc_t{0, 0, 0, 0};
        }

    if (ymode == 0)
        mp2_kloop<T, BK, AW, true>(&lds[0][0][0], base0, base1, base2, base3, rows_p, rows_q, g.naux, X, Y);
    else
        mp2_kloop<T, BK, AW, false>(&lds[0][0][0], base0, base1, base2, base3, rows_p, rows_q, g.naux, X, Y);

    const int lg = lane >> 4;
    // Rows and columns of the quadrant the energy loop below reads from X and Y.
    int rb = wr, cb0 = wc;
    if (ymode == 0) {
        // The K loop left each X wave with X rows 0-63 of its columns
        // and each Y wave with Y rows 0-63 of the same columns. The X wave
        // keeps rows 0-31 and hands rows 32-63 to the Y wave, which keeps its
        // rows 32-63 and hands rows 0-31 back, through LDS (free after the K
        // loop's last barrier); each then holds X and Y of one quadrant.
        const int mat = wave >> 1;
        const int ch = (wave & 1) * 32;
        constexpr int TP = kMp2Tile + 1;
        T* xs = &lds[0][0][0];  // X rows 32-63
        T* ys = xs + 32 * TP;   // Y rows 0-31
        static_assert(kMp2Tile * TP <= 4 * PN::ELEMS, "exchange fits in the staging buffers");
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int o = (16 * a + MF::row(lg, r)) * TP + ch + 16 * b + (lane & 15);
                    if (mat == 0) xs[o] = Y[a][b][r];
                    else ys[o] = X[a][b][r];
                }
        __syncthreads();
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int o = (16 * a + MF::row(lg, r)) * TP + ch + 16 * b + (lane & 15);
                    if (mat == 0) Y[a][b][r] = ys[o];
                    else X[a][b][r] = xs[o];
                }
        rb = mat ? 32 : 0;
        cb0 = ch;
    }
    if (ymode == 2) {
        // Y = X^T through LDS (the staging buffers are free after the last barrier).
        constexpr int TP = kMp2Tile + 1;
        T* tr = &lds[0][0][0];
        static_assert(kMp2Tile * TP <= 4 * PN::ELEMS, "transpose fits in the staging buffers");
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    tr[(wr + 16 * a + MF::row(lg, r)) * TP + wc + 16 * b + (lane & 15)] = X[a][b][r];
        __syncthreads();
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    Y[a][b][r] = tr[(wc + 16 * b + (lane & 15)) * TP + wr + 16 * a + MF::row(lg, r)];
    }

    // Epilogue: denominators and exchange term in registers.
    const T* eo = static_cast<const T*>(g.eo);
    const T* ev = static_cast<const T*>(g.ev);
    const T eij = eo[i] + eo[j];
    const bool mirror = (p != q);
    // The lane's orbital energies are all loaded first, branch-free (a row
    // outside the block loads ev[0]; its terms are skipped below): loads
    // inside the per-element bounds branches each waited out a latency.
    T e_bv[2], e_av[2][4];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const int cb = cb0 + 16 * b + (lane & 15);
        e_bv[b] = ev[cb < rows_q ? q * kMp2Tile + cb : 0];
    }
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int ra = rb + 16 * a + MF::row(lg, r);
            e_av[a][r] = ev[ra < rows_p ? p * kMp2Tile + ra : 0];
        }
    double sum = 0.0;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const int cb = cb0 + 16 * b + (lane & 15);
        const bool okb = cb < rows_q;
        const T e_b = e_bv[b];
#pragma unroll
        for (int a = 0; a < 2; ++a) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int ra = rb + 16 * a + MF::row(lg, r);
                if (okb && ra < rows_p) {
                    const T e_a = e_av[a][r];
                    const T x = X[a][b][r];
                    const T y = ymode == 1 ? x : Y[a][b][r];
                    const T d_ab = (eij - e_a) - e_b;
                    T term = (x * (T(2) * x - y)) / d_ab;
                    sum += (double)term;
                    if (mirror) {
                        const T d_ba = (eij - e_b) - e_a;
                        T term2 = (y * (T(2) * y - x)) / d_ba;
                        sum += (double)term2;
                    }
                }
            }
        }
    }
    double blk = block256_sum(sum, red);
    if (threadIdx.x == 0) {
        if (i != j) blk *= 2.0;
        if (g.partial) g.partial[local] = blk;
        else atomicAdd(g.accum, blk);
    }
}

// Fixed-order sum of the per-workgroup partials (or the atomic accumulator)
// into one element of T.
template <typename T>
__global__ __launch_bounds__(256) void mp2_finalize_kernel(const double* partial, int64_t n, T* out) {
    __shared__ double red[4];
    const double s = strided_sum256(partial, n);
    double tot = block256_sum(s, red);
    if (threadIdx.x == 0) out[0] = (T)tot;
}

__global__ void zero_double_kernel(double* p) {
    if (threadIdx.x == 0) p[0] = 0.0;
}

// Largest of 16 / sizeof(T), ..., 2, 1 elements such that B's base and every
// row start (multiples of naux elements from it) are aligned to that many
// elements' bytes.
static int mp2_access_width(size_t elem, int64_t naux, const void* B) {
    int aw = (int)(16 / elem);
    while (aw > 1 && ((naux % aw) != 0 || (reinterpret_cast<uintptr_t>(B) % (aw * elem)) != 0)) aw >>= 1;
    return aw;
}

static int64_t mp2_ntasks(int64_t nocc, int64_t nvir) {
    const int64_t nblk = (nvir + kMp2Tile - 1) / kMp2Tile;
    return (nblk * (nblk + 1) / 2) * (nocc * (nocc + 1) / 2);
}

// Workspace layout: the per-unit partials (plus one double), then, when naux
// is not a multiple of the stage depth, a copy of B whose rows are padded
// with zeros to mp2_pitch(naux) elements.
//
// The stages of a row start at multiples of 16 elements from the row start.
// With naux a multiple of 16 (and B's base so aligned) every stage is a whole
// 128-byte (fp64) or 64-byte (fp32) aligned chunk; otherwise each straddles
// cache lines and the kernel runs 5-7% slower (nocc 64, nvir 320: naux 1199
// fp64 8.58 ms against 8.06 ms on the padded copy, which itself takes
// 0.07 ms; fp32 4.38 against 4.13 + 0.03 ms). The zero columns add nothing
// to any product, and the unpadded kernel masks the same columns to zero in
// its last stage, so both give the same energy, bitwise.
static size_t mp2_partials_bytes(int64_t nocc, int64_t nvir) {
    const size_t n = (size_t)mp2_ntasks(nocc, nvir) + 1;
    return ((n * sizeof(double) + 255) / 256) * 256;
}

static int64_t mp2_pitch(int64_t naux) { return (naux + kMp2StageK - 1) / kMp2StageK * kMp2StageK; }

static size_t mp2_pad_bytes(int dtype, int64_t nocc, int64_t nvir, int64_t naux) {
    if (naux <= 0 || naux % kMp2StageK == 0 || nocc <= 0 || nvir <= 0) return 0;
    const unsigned __int128 b =
        (unsigned __int128)nocc * (unsigned __int128)nvir * (unsigned __int128)mp2_pitch(naux) * (dtype == TT_F32 ? 4u : 8u);
    if (b > (unsigned __int128)(SIZE_MAX / 4)) return SIZE_MAX / 4;
    return (((size_t)b + 255) / 256) * 256;
}

// src (rows x naux, contiguous) -> dst (rows x pitch), zero in columns naux
// and beyond. One workgroup per row (grid-stride); each thread forms V
// elements from element loads (clamped addresses, so no load leaves the row)
// and writes them with one 16-byte store (every dst row starts on a
// 16-element boundary).
template <typename T>
__global__ __launch_bounds__(256) void mp2_pad_rows_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                           int64_t rows, int64_t naux, int64_t pitch) {
    constexpr int V = 16 / sizeof(T);
    typedef typename VecN<T, V>::type vec_t;
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const T* s = src + r * naux;
        vec_t* d = reinterpret_cast<vec_t*>(dst + r * pitch);
        for (int64_t c = (int64_t)threadIdx.x * V; c < pitch; c += 256 * V) {
            vec_t v;
#pragma unroll
            for (int e = 0; e < V; ++e) {
                const bool ok = c + e < naux;
                const T x = s[ok ? c + e : naux - 1];
                v[e] = ok ? x : T(0);
            }
            d[c / V] = v;
        }
    }
}

template <typename T>
static int mp2_typed(int64_t nocc, int64_t nvir, int64_t naux, const void* B, const void* eo, const void* ev,
                     void* out, void* ws, size_t ws_bytes, int det, hipStream_t st, int64_t first, int64_t count) {
    // Row-padded copy of B when the workspace holds it (and is 256-byte
    // aligned, which the copy's 16-byte stores and the stage alignment need).
    const size_t part = mp2_partials_bytes(nocc, nvir);
    const size_t pad = mp2_pad_bytes(sizeof(T) == 4 ? TT_F32 : TT_F64, nocc, nvir, naux);
    if (pad > 0 && ws_bytes >= part && ws_bytes - part >= pad && (reinterpret_cast<uintptr_t>(ws) & 255) == 0) {
        T* Bp = reinterpret_cast<T*>(static_cast<char*>(ws) + part);
        const int64_t rows = nocc * nvir, pitch = mp2_pitch(naux);
        hipLaunchKernelGGL(mp2_pad_rows_kernel<T>, dim3((unsigned)(rows < 65536 ? rows : 65536)), dim3(256), 0, st,
                           static_cast<const T*>(B), Bp, rows, naux, pitch);
        B = Bp;
        naux = pitch;
    }
    Mp2Args g;
    g.B = B;
    g.eo = eo;
    g.ev = ev;
    g.naux = naux;
    g.nocc = (int)nocc;
    g.nvir = (int)nvir;
    g.nblk = (int)((nvir + kMp2Tile - 1) / kMp2Tile);
    g.npq = (int64_t)g.nblk * (g.nblk + 1) / 2;
    g.first = first;
    g.ntasks = count;
    double* w = static_cast<double*>(ws);
    if (det) {
        g.partial = w;
        g.accum = nullptr;
    } else {
        g.partial = nullptr;
        g.accum = w;
        hipLaunchKernelGGL(zero_double_kernel, dim3(1), dim3(64), 0, st, w);
    }
    constexpr int BK = kMp2StageK;
    // Widest access (elements) that keeps every row start naturally aligned.
    const int aw = mp2_access_width(sizeof(T), naux, B);
    if (g.ntasks > 0) {
        const dim3 grid((unsigned)g.ntasks), block(kMp2Threads);
        constexpr int V = 16 / sizeof(T);
        if (aw == V)
            hipLaunchKernelGGL((mp2_energy_kernel<T, BK, V>), grid, block, 0, st, g);
        else if (aw == 2)
            hipLaunchKernelGGL((mp2_energy_kernel<T, BK, 2>), grid, block, 0, st, g);
        else
            hipLaunchKernelGGL((mp2_energy_kernel<T, BK, 1>), grid, block, 0, st, g);
    }
    hipLaunchKernelGGL(mp2_finalize_kernel<T>, dim3(1), dim3(256), 0, st, (const double*)w,
                       det ? g.ntasks : (int64_t)1, static_cast<T*>(out));
    return check_launch("tt_mp2_energy");
}

}  // namespace tt

extern "C" size_t tt_mp2_energy_workspace_bytes(int dtype, int64_t nocc, int64_t nvir, int64_t naux) {
    if (nocc < 0 || nvir < 0) return 0;
    return tt::mp2_partials_bytes(nocc, nvir) + tt::mp2_pad_bytes(dtype, nocc, nvir, naux);
}

namespace tt {

// Argument checks shared by both entry points (no HIP call).
static int mp2_check(const char* what, int dtype, int64_t nocc, int64_t nvir, int64_t naux, const void* B,
                     const void* eps_occ, const void* eps_vir, const void* energy_out) {
    if (nocc < 0 || nvir < 0 || naux < 0)
        return set_error(TT_INVALID, "%s: negative extent (nocc=%lld nvir=%lld naux=%lld)", what, (long long)nocc,
                         (long long)nvir, (long long)naux);
    if (nocc > (1 << 20) || nvir > (1 << 24))
        return set_error(TT_UNSUPPORTED, "%s: nocc=%lld nvir=%lld beyond the kernel's index range", what,
                         (long long)nocc, (long long)nvir);
    if (mp2_ntasks(nocc, nvir) > 0x7fffffffLL)
        return set_error(TT_UNSUPPORTED, "%s: too many work units for one launch", what);
    if (!energy_out || (nocc > 0 && nvir > 0 && (!B || !eps_occ || !eps_vir)))
        return set_error(TT_INVALID, "%s: NULL pointer", what);
    if (dtype != TT_F64 && dtype != TT_F32)
        return set_error(TT_UNSUPPORTED, "%s: dtype %d (only TT_F32, TT_F64)", what, dtype);
    return TT_OK;
}

static int mp2_dispatch(int dtype, int64_t nocc, int64_t nvir, int64_t naux, const void* B, const void* eo,
                        const void* ev, void* out, void* ws, size_t ws_bytes, int det, hipStream_t st,
                        int64_t first = 0, int64_t count = -1) {
    if (count < 0) count = mp2_ntasks(nocc, nvir);
    if (dtype == TT_F64)
        return mp2_typed<double>(nocc, nvir, naux, B, eo, ev, out, ws, ws_bytes, det, st, first, count);
    return mp2_typed<float>(nocc, nvir, naux, B, eo, ev, out, ws, ws_bytes, det, st, first, count);
}

// Scratch of the allocation-free entry point: the per-workgroup partials
// (deterministic mode) or the atomic accumulator (element 0). One copy per
// device, resident until the process ends. Host code never passes this
// name to a kernel: it is a host-side stand-in, and the device address comes
// from hipGetSymbolAddress (mp2_scratch_ptr below).
constexpr int64_t kMp2ScratchDoubles = int64_t(1) << 21;  // 16 MiB
static __device__ __align__(256) double scratch[kMp2ScratchDoubles];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept. The lookup is a runtime call
// that may load the code object, which a stream capture must not record: a
// first call on a device while `st` is capturing is refused (the caller makes
// one eager call on each device before capturing).
static int mp2_scratch_ptr(hipStream_t st, void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(TT_HIP_ERROR, "tt_mp2_energy_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices)
        return set_error(TT_UNSUPPORTED, "tt_mp2_energy_noalloc: device index %d beyond %d", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(st, &cs);
        if (e != hipSuccess)
            return set_error(TT_HIP_ERROR, "tt_mp2_energy_noalloc: hipStreamIsCapturing: %s", hipGetErrorString(e));
        if (cs != hipStreamCaptureStatusNone)
            return set_error(TT_INVALID,
                             "tt_mp2_energy_noalloc: first call on device %d made under stream capture; make one "
                             "call on each device before capturing (it looks up the scratch address)",
                             dev);
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return set_error(TT_HIP_ERROR, "tt_mp2_energy_noalloc: hipGetSymbolAddress(scratch): %s",
                             hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return TT_OK;
}

}  // namespace tt

extern "C" int tt_mp2_energy(int dtype, int64_t nocc, int64_t nvir, int64_t naux, const void* B, const void* eps_occ,
                             const void* eps_vir, void* energy_out, void* workspace, size_t workspace_bytes,
                             int deterministic, void* stream) {
    using namespace tt;
    int rc = mp2_check("tt_mp2_energy", dtype, nocc, nvir, naux, B, eps_occ, eps_vir, energy_out);
    if (rc != TT_OK) return rc;
    const size_t need = mp2_partials_bytes(nocc, nvir);
    if (!workspace || workspace_bytes < need)
        return set_error(TT_INVALID, "tt_mp2_energy: workspace of %zu bytes, need %zu", workspace_bytes, need);
    return mp2_dispatch(dtype, nocc, nvir, naux, B, eps_occ, eps_vir, energy_out, workspace, workspace_bytes,
                        deterministic, static_cast<hipStream_t>(stream));
}

extern "C" int tt_mp2_energy_noalloc(int dtype, int64_t nocc, int64_t nvir, int64_t naux, const void* B,
                                     const void* eps_occ, const void* eps_vir, void* energy_out, int deterministic,
                                     void* stream) {
    using namespace tt;
    int rc = mp2_check("tt_mp2_energy_noalloc", dtype, nocc, nvir, naux, B, eps_occ, eps_vir, energy_out);
    if (rc != TT_OK) return rc;
    // Deterministic mode keeps one partial per work unit; the atomic mode
    // needs only the accumulator.
    const int64_t need = deterministic ? mp2_ntasks(nocc, nvir) + 1 : 1;
    if (need > kMp2ScratchDoubles)
        return set_error(TT_INVALID,
                         "tt_mp2_energy_noalloc: nocc=%lld nvir=%lld needs %lld partials, the static scratch holds "
                         "%lld (use tt_mp2_energy with a workspace, or deterministic=0)",
                         (long long)nocc, (long long)nvir, (long long)need, (long long)kMp2ScratchDoubles);
    void* ws = nullptr;
    rc = mp2_scratch_ptr(static_cast<hipStream_t>(stream), &ws);
    if (rc != TT_OK) return rc;
    // The scratch holds the partials only: no padded copy of B.
    return mp2_dispatch(dtype, nocc, nvir, naux, B, eps_occ, eps_vir, energy_out, ws, 0, deterministic,
                        static_cast<hipStream_t>(stream));
}

extern "C" int64_t tt_mp2_energy_unit_count(int64_t nocc, int64_t nvir) {
    if (nocc < 0 || nvir < 0) return 0;
    return tt::mp2_ntasks(nocc, nvir);
}

extern "C" int tt_mp2_energy_shard(int dtype, int64_t nocc, int64_t nvir, int64_t naux, const void* B,
                                   const void* eps_occ, const void* eps_vir, int64_t first_unit, int64_t n_units,
                                   void* energy_out, void* workspace, size_t workspace_bytes, int deterministic,
                                   void* stream) {
    using namespace tt;
    int rc = mp2_check("tt_mp2_energy_shard", dtype, nocc, nvir, naux, B, eps_occ, eps_vir, energy_out);
    if (rc != TT_OK) return rc;
    const int64_t total = mp2_ntasks(nocc, nvir);
    if (first_unit < 0 || n_units < 0 || first_unit > total || n_units > total - first_unit)
        return set_error(TT_INVALID, "tt_mp2_energy_shard: units [%lld, %lld) outside [0, %lld)", (long long)first_unit,
                         (long long)(first_unit + n_units), (long long)total);
    const size_t need = mp2_partials_bytes(nocc, nvir);
    if (!workspace || workspace_bytes < need)
        return set_error(TT_INVALID, "tt_mp2_energy_shard: workspace of %zu bytes, need %zu", workspace_bytes, need);
    return mp2_dispatch(dtype, nocc, nvir, naux, B, eps_occ, eps_vir, energy_out, workspace, workspace_bytes,
                        deterministic, static_cast<hipStream_t>(stream), first_unit, n_units);
}
