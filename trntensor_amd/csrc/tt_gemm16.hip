// 16-bit GEMM for bf16 / fp16 operands (dtype TT_BF16 / TT_F16 of tt_gemm):
//   D = alpha * op(A) op(B) (+ beta * C), products and sums in fp32 on
//   v_mfma_f32_16x16x32_{bf16,f16}, alpha/beta applied in fp32, one rounding
//   to the 16-bit type at the store.
//
// Workgroup: 256 threads = 4 wavefronts in a 2 x 2 grid over a BM x BN
// output tile (128 x 128 or 256 x 128), each wave (BM / 2) x (BN / 2) of
// 16 x 16 MFMA blocks with fp32 accumulators. K advances BK (64 or 32) per
// stage through two LDS buffers (one barrier per stage), the next stage's
// global loads held in registers during the current stage's MFMAs.
//
// MFMA operand layout (16x16x32): lane l holds A[l % 16][8 (l / 16) + j] and
// B[8 (l / 16) + j][l % 16], j = 0..7; accumulator element r holds
// D[4 (l / 16) + r][l % 16].
//
// Each operand is staged in its memory order, so staging is a plain copy:
//   k-contiguous operand: LDS [row][k], row pitch BK + 8 elements; a lane's
//     MFMA operand (8 consecutive k of one row) is one 16-byte read;
//   row-contiguous operand: LDS [k][row], k-row pitch ROWS + 16 elements;
//     a lane's MFMA operand is gathered across k-rows by two transposing
//     reads h = 0, 1 (ds_read_b64_tr_b16: within each 16 lanes, lane
//     16 g + 4 j + a supplies
//     the address of rows 4 a .. 4 a + 3 of k-row 8 g + 4 h + j, and lane
//     16 g + 4 a + b receives element b of the blocks of lanes 16 g + 4 j + a,
//     j = 0..3, i.e. k 8 g + 4 h .. 8 g + 4 h + 3 of row 4 a + b).
#include <string.h>
#include <type_traits>

#include "tt_gemm.hpp"

namespace tt {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct Mfma16;
template <>
struct Mfma16<__bf16> {
    static __device__ __forceinline__ f32x4 mma(u16x8 a, u16x8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       c, 0, 0, 0);
    }
};
template <>
struct Mfma16<_Float16> {
    static __device__ __forceinline__ f32x4 mma(u16x8 a, u16x8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
    }
};

// One operand's ROWS x BK stage: global -> registers -> LDS, plus MFMA operand
// reads. KC: element (row, k) at p[row * ld + k], LDS [row][k]; otherwise at
// p[k * ld + row], LDS [k][row]. Each of the 256 threads copies NP 16-byte
// pieces that are consecutive in memory.
template <bool KC, int ROWS, int BK>
struct Stage16 {
    static constexpr int PITCH = KC ? BK + 8 : ROWS + 16;  // elements (16-byte multiple)
    static constexpr int ELEMS = KC ? ROWS * PITCH : BK * PITCH;
    static constexpr int LINE = KC ? BK / 8 : ROWS / 8;    // 16-byte pieces per LDS line
    static constexpr int NP = ROWS * BK / 8 / 256;         // pieces per thread
    static constexpr int TPL = LINE / NP;                  // threads per line
    static_assert(NP >= 1 && LINE % NP == 0 && BK % 32 == 0 && ROWS % 32 == 0, "stage split");
    u16x8 reg[NP];

    // Line (row for KC, k-row otherwise) and first element along it for this thread.
    __device__ __forceinline__ static void place(int& line, int& off) {
        line = threadIdx.x / TPL;
        off = (threadIdx.x % TPL) * NP * 8;
    }

    // FAST: interior stage, 16-byte aligned lines: unconditional vector loads.
    // Otherwise (a tile crossing the matrix edge, the K tail, or unaligned
    // lines) piece by piece: a piece wholly inside is one vector load (VEC:
    // aligned lines), one wholly outside is zero without a load, and only a
    // piece that straddles the edge is loaded element by element from clamped
    // addresses. (Element loads for every piece made edge tiles, and so whole
    // ragged launches, 4-7x slower than aligned ones of the same size.)
    template <bool FAST, bool VEC>
    __device__ __forceinline__ void load(const unsigned short* __restrict__ p, int64_t ld, int64_t row0, int64_t rows,
                                         int64_t k0, int64_t kdim) {
        int line, off;
        place(line, off);
        if (FAST) {
            const unsigned short* src = KC ? p + (row0 + line) * ld + k0 + off : p + (k0 + line) * ld + row0 + off;
#pragma unroll
            for (int c = 0; c < NP; ++c) reg[c] = *reinterpret_cast<const u16x8*>(src + 8 * c);
        } else {
#pragma unroll
            for (int c = 0; c < NP; ++c) {
                // Piece start (gr, gk) and its extent along the contiguous direction.
                const int64_t gr = row0 + (KC ? line : off + 8 * c);
                const int64_t gk = k0 + (KC ? off + 8 * c : line);
                const bool inside = KC ? (gr < rows && gk + 8 <= kdim) : (gk < kdim && gr + 8 <= rows);
                const bool outside = gr >= rows || gk >= kdim;
                if (VEC && inside) {
                    reg[c] = *reinterpret_cast<const u16x8*>(KC ? p + gr * ld + gk : p + gk * ld + gr);
                } else if (outside) {
                    reg[c] = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const int64_t r = gr + (KC ? 0 : e), k = gk + (KC ? e : 0);
                        const bool ok = r < rows && k < kdim;
                        const unsigned short x = *(ok ? (KC ? p + r * ld + k : p + k * ld + r) : p);
                        reg[c][e] = ok ? x : (unsigned short)0;
                    }
                }
            }
        }
    }

    __device__ __forceinline__ void store(unsigned short* s) const {
        int line, off;
        place(line, off);
        unsigned short* dst = s + line * PITCH + off;
#pragma unroll
        for (int c = 0; c < NP; ++c) *reinterpret_cast<u16x8*>(dst + 8 * c) = reg[c];
    }

    // This lane's MFMA operand for the 16 rows from rb, k step ks (k 32 ks .. 32 ks + 31).
    __device__ __forceinline__ static u16x8 frag(const unsigned short* s, int rb, int ks, int lane) {
        if (KC) return *reinterpret_cast<const u16x8*>(s + (rb + (lane & 15)) * PITCH + 32 * ks + 8 * (lane >> 4));
        const int g = lane >> 4, j = (lane & 15) >> 2, a = lane & 3;
        const unsigned short* base = s + (32 * ks + 8 * g + j) * PITCH + rb + 4 * a;
        typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base + 4 * PITCH));
        return u16x8{(unsigned short)lo[0], (unsigned short)lo[1], (unsigned short)lo[2], (unsigned short)lo[3],
                     (unsigned short)hi[0], (unsigned short)hi[1], (unsigned short)hi[2], (unsigned short)hi[3]};
    }
};

template <typename T>
__device__ __forceinline__ float to_f32(unsigned short x) {
    return (float)__builtin_bit_cast(T, x);
}
template <typename T>
__device__ __forceinline__ unsigned short from_f32(float x) {
    return __builtin_bit_cast(unsigned short, (T)x);
}

template <typename T, bool TA, bool TB, bool VEC, int BM, int BN, int BK>
__global__ __launch_bounds__(256) void gemm16_kernel(GemmArgs g) {
    // A rows are m: k-contiguous unless transposed. B rows are n: k-contiguous iff transposed.
    typedef Stage16<!TA, BM, BK> SA;
    typedef Stage16<TB, BN, BK> SB;
    // Four wavefronts in a 2 x 2 grid, each FM x FN MFMA blocks of 16 x 16.
    constexpr int WM = BM / 2, WN = BN / 2, FM = WM / 16, FN = WN / 16;
    __shared__ __attribute__((aligned(16))) unsigned short lds[2 * (SA::ELEMS + SB::ELEMS)];
    auto bufA = [&](int b) -> unsigned short* { return lds + b * SA::ELEMS; };
    auto bufB = [&](int b) -> unsigned short* { return lds + 2 * SA::ELEMS + b * SB::ELEMS; };

    const int64_t tiles = g.tiles_m * g.tiles_n;
    const int64_t total = tiles * g.batch;
    const int64_t id = xcd_remap(blockIdx.x, total);
    const int64_t bat = id / tiles;
    const int64_t t = id - bat * tiles;
    constexpr int64_t GROUP = 8;
    const int64_t grp = t / (GROUP * g.tiles_n);
    const int64_t first_m = grp * GROUP;
    const int64_t gsize = min(g.tiles_m - first_m, GROUP);
    const int64_t rem = t - grp * GROUP * g.tiles_n;
    const int64_t m0 = (first_m + rem % gsize) * BM;
    const int64_t n0 = (rem / gsize) * BN;

    const unsigned short* A = static_cast<const unsigned short*>(g.A) + bat * g.sA;
    const unsigned short* B = static_cast<const unsigned short*>(g.B) + bat * g.sB;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm0 = (wave >> 1) * WM;
    const int wn0 = (wave & 1) * WN;
    const int lrow = lane & 15;
    const int lg = lane >> 4;

    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0, 0, 0, 0};

    SA sa;
    SB sb;
    const int64_t nk = (g.K + BK - 1) / BK;
    const int64_t nfull = (VEC && m0 + BM <= g.M && n0 + BN <= g.N) ? g.K / BK : 0;
    auto load = [&](int64_t k0, auto fast) {
        constexpr bool F = decltype(fast)::value;
        sa.template load<F, VEC>(A, g.lda, m0, g.M, k0, g.K);
        sb.template load<F, VEC>(B, g.ldb, n0, g.N, k0, g.K);
    };
    auto compute = [&](int buf) {
        const unsigned short* a = bufA(buf);
        const unsigned short* b = bufB(buf);
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            u16x8 fa[FM], fb[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) fa[i] = SA::frag(a, wm0 + 16 * i, ks, lane);
#pragma unroll
            for (int j = 0; j < FN; ++j) fb[j] = SB::frag(b, wn0 + 16 * j, ks, lane);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) acc[i][j] = Mfma16<T>::mma(fa[i], fb[j], acc[i][j]);
        }
    };
    int64_t kt = 0;
    if (nk > 0) {
        if (nfull > 0) load(0, std::true_type{});
        else load(0, std::false_type{});
        sa.store(bufA(0));
        sb.store(bufB(0));
    }
    __syncthreads();
    for (; kt + 1 < nfull; ++kt) {
        load((kt + 1) * BK, std::true_type{});
        compute(kt & 1);
        __builtin_amdgcn_sched_barrier(0);
        sa.store(bufA((kt & 1) ^ 1));
        sb.store(bufB((kt & 1) ^ 1));
        __syncthreads();
    }
    // Buffer kt & 1 holds stage kt; the remaining stages load one ahead.
    for (; kt < nk; ++kt) {
        const bool more = kt + 1 < nk;
        if (more) load((kt + 1) * BK, std::false_type{});
        compute(kt & 1);
        __builtin_amdgcn_sched_barrier(0);
        if (more) {
            sa.store(bufA((kt & 1) ^ 1));
            sb.store(bufB((kt & 1) ^ 1));
        }
        __syncthreads();
    }

    // Epilogue through LDS (free after the last barrier): each wave writes one
    // 16-row slab of its tile as fp32 with alpha applied, then each lane
    // finishes 8 consecutive columns of one row with a 16-byte load of C and a
    // 16-byte store of D (element-wise at ragged or unaligned edges).
    const unsigned short* C = g.C ? static_cast<const unsigned short*>(g.C) + bat * g.sC : nullptr;
    unsigned short* D = static_cast<unsigned short*>(g.D) + bat * g.sD;
    const float alpha = (float)g.alpha;
    const float beta = (float)g.beta;
    constexpr int SP = WN + 4;  // slab pitch in floats (16-byte multiple)
    static_assert(4 * 16 * SP * sizeof(float) <= sizeof(lds), "epilogue slabs fit in the stage buffers");
    float* slab = reinterpret_cast<float*>(lds) + wave * 16 * SP;
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    const bool vout = a16(D) && g.ldd % 8 == 0 && (!C || (a16(C) && g.ldc % 8 == 0));
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        // This slab's C chunks are loaded before any of its stores (and before the
        // slab exchange, whose barrier then covers their latency): D may
        // alias C, so the compiler cannot move a load of C past a store of D,
        // and chunk-by-chunk loads would each wait out a full memory latency.
        u16x8 cc[WN / 32];
#pragma unroll
        for (int h = 0; h < WN / 32; ++h) {
            const int v = lane + 64 * h;
            const int rr = v / (WN / 8), cb = v % (WN / 8);
            const int64_t row = m0 + wm0 + 16 * i + rr;
            const int64_t col = n0 + wn0 + 8 * cb;
            cc[h] = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
            if (C && vout && row < g.M && col + 8 <= g.N) cc[h] = *reinterpret_cast<const u16x8*>(C + row * g.ldc + col);
        }
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v = acc[i][j][r];
                if (g.alpha != 1.0) v = alpha * v;
                slab[(4 * lg + r) * SP + 16 * j + lrow] = v;
            }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < WN / 32; ++h) {
            const int v = lane + 64 * h;
            const int rr = v / (WN / 8), cb = v % (WN / 8);
            const int64_t row = m0 + wm0 + 16 * i + rr;
            const int64_t col = n0 + wn0 + 8 * cb;
            const f32x4 lo = *reinterpret_cast<const f32x4*>(slab + rr * SP + 8 * cb);
            const f32x4 hi = *reinterpret_cast<const f32x4*>(slab + rr * SP + 8 * cb + 4);
            float x[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            if (row < g.M) {
                if (vout && col + 8 <= g.N) {
                    if (C) {
#pragma unroll
                        for (int e = 0; e < 8; ++e) x[e] = x[e] + beta * to_f32<T>(cc[h][e]);
                    }
                    u16x8 d;
#pragma unroll
                    for (int e = 0; e < 8; ++e) d[e] = from_f32<T>(x[e]);
                    *reinterpret_cast<u16x8*>(D + row * g.ldd + col) = d;
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (col + e < g.N) {
                            float y = x[e];
                            if (C) y = y + beta * to_f32<T>(C[row * g.ldc + col + e]);
                            D[row * g.ldd + col + e] = from_f32<T>(y);
                        }
                }
            }
        }
        __syncthreads();
    }
}

template <typename T, int BM, int BN, int BK>
int launch16(bool ta, bool tb, bool vec, GemmArgs& g, hipStream_t st) {
    g.tiles_m = (g.M + BM - 1) / BM;
    g.tiles_n = (g.N + BN - 1) / BN;
    const int64_t total = g.tiles_m * g.tiles_n * g.batch;
    if (total > 0x7fffffffLL) return set_error(TT_UNSUPPORTED, "tt_gemm: %lld tiles exceed one launch", (long long)total);
    const dim3 grid((unsigned)total), block(256);
#define TT_GEMM16_CASE(TA, TB, VC)           \
    if (ta == TA && tb == TB && vec == VC) \
        hipLaunchKernelGGL((gemm16_kernel<T, TA, TB, VC, BM, BN, BK>), grid, block, 0, st, g);
    TT_GEMM16_CASE(false, false, false)
    TT_GEMM16_CASE(false, false, true)
    TT_GEMM16_CASE(false, true, false)
    TT_GEMM16_CASE(false, true, true)
    TT_GEMM16_CASE(true, false, false)
    TT_GEMM16_CASE(true, false, true)
    TT_GEMM16_CASE(true, true, false)
    TT_GEMM16_CASE(true, true, true)
#undef TT_GEMM16_CASE
    return check_launch("tt_gemm (16-bit)");
}

// Register-staged kernel (any shape, alignment and K).
template <typename T>
int gemm16_staged(bool ta, bool tb, GemmArgs& g, hipStream_t st) {
    auto ok16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    bool vec = ok16(g.A) && ok16(g.B) && g.lda % 8 == 0 && g.ldb % 8 == 0;
    if (g.batch > 1) vec = vec && g.sA % 8 == 0 && g.sB % 8 == 0;
    // Measured at 4096^3 (bf16): with A row-contiguous (transposed), 256 x 128
    // tiles of depth 32 run at 934-939 TFLOP/s against 840-862 for 128 x 128 x 64;
    // with A k-contiguous the 128 x 128 x 64 tile is the faster (857-872 against
    // 827-871). 128 x 256 x 32 and 128 x 128 x 32 tiles measured 802-922 and
    // 710-868; 128 x 256 x 64 (one workgroup per CU) 500. On smaller grids the
    // 256 x 128 tile leaves CUs idle: 8 x 384 x 1024^2 41 against 282-288,
    // 2048^3 252 against 394-399, 4096 x 256 x 4096 68 against 113-115.
    if (ta && ((g.M + 255) / 256) * ((g.N + 127) / 128) * g.batch >= 512)
        return launch16<T, 256, 128, 32>(ta, tb, vec, g, st);
    return launch16<T, 128, 128, 64>(ta, tb, vec, g, st);
}

template <typename T>
int gemm16_typed(bool ta, bool tb, GemmArgs& g, hipStream_t st) {
    auto ok16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    bool vec = ok16(g.A) && ok16(g.B) && g.lda % 8 == 0 && g.ldb % 8 == 0;
    if (g.batch > 1) vec = vec && g.sA % 8 == 0 && g.sB % 8 == 0;
    // The direct-load kernel needs K deep enough to amortise its prologue and
    // epilogue. With its 128 x 256 tiles
    // it is level or ahead from K = 256 in every layout (bf16, 64 x 512^2 x 256:
    // NN 370-374 against 338-342 TFLOP/s, NT 389-409 against 338-346, TN
    // 398-403 against 400-401, TT 419 against 392-396; 64 x 512^3: 588-669
    // against 508-562).
    const int64_t kmin = 256;
    // It also needs a full grid, and the ragged strips run as separate,
    // serial launches: against the register-staged kernel alone it lost with
    // 96-128 whole tiles (8 x 384 x 1024^2: 228-241 against 282-298 TFLOP/s;
    // 2048^3: 359-387 against 394-411), tied at 192-256 (16 x 512 x 1024^2:
    // 572-602 against 574-612) and won at 512 (4096^3 NN: 1104 against 850);
    // with strips of a tenth of the outputs (2000 x 3000 x 320) it ran at
    // 31-43 against 71-74. Its 128 x 128 tile (three workgroups per CU) takes
    // the grids too small for 128 x 256 and beats the register-staged kernel
    // on the same grid from 64 tiles (2048^3: 512-544 against 397-406;
    // 8 x 384 x 1024^2: 320-335 against 293-302; 4096 x 256 x 4096: 151-162
    // against 113-117, NT 112 against 113); with strips of 5.8% of the
    // outputs (2000 x 3000 x 320) it lost again, 42-48 against 71-75, so
    // strips are limited to 1/64.
    int bm_, bn_;
    gemm16_dma_tile(ta, tb, g.M, g.N, g.K, g.batch, bm_, bn_);
    const int64_t bm = bm_, bn = bn_;
    const int64_t Mi = g.M & ~(bm - 1), Ni = g.N & ~(bn - 1);
    const int64_t tiles = (Mi / bm) * (Ni / bn) * g.batch;
    const bool small_strips = (g.M - Mi) * g.N + Mi * (g.N - Ni) <= g.M * g.N / 64;
    if (!vec || g.M < bm || g.N < bn || g.K < kmin || g.K % 32 != 0 || tiles < 64 || !small_strips)
        return gemm16_staged<T>(ta, tb, g, st);
    // Whole bm x bn tiles by the direct-load kernel; the ragged row and
    // column strips (if any) by the register-staged kernel on sub-matrices.
    const unsigned short* A = static_cast<const unsigned short*>(g.A);
    const unsigned short* B = static_cast<const unsigned short*>(g.B);
    const unsigned short* C = static_cast<const unsigned short*>(g.C);
    unsigned short* D = static_cast<unsigned short*>(g.D);
    GemmArgs gi = g;
    gi.M = Mi;
    gi.N = Ni;
    int rc = gemm16_dma_dispatch(std::is_same<T, __bf16>::value ? TT_BF16 : TT_F16, ta, tb, gi, st);
    if (rc == TT_OK && Mi < g.M) {
        GemmArgs ge = g;
        ge.M = g.M - Mi;
        ge.A = ta ? A + Mi : A + Mi * g.lda;
        ge.C = C ? C + Mi * g.ldc : nullptr;
        ge.D = D + Mi * g.ldd;
        rc = gemm16_staged<T>(ta, tb, ge, st);
    }
    if (rc == TT_OK && Ni < g.N) {
        GemmArgs ge = g;
        ge.M = Mi;
        ge.N = g.N - Ni;
        ge.B = tb ? B + Ni * g.ldb : B + Ni;
        ge.C = C ? C + Ni : nullptr;
        ge.D = D + Ni;
        rc = gemm16_staged<T>(ta, tb, ge, st);
    }
    return rc;
}

}  // namespace

int gemm16_dispatch(int dtype, bool ta, bool tb, GemmArgs& g, hipStream_t st) {
    if (dtype == TT_BF16) return gemm16_typed<__bf16>(ta, tb, g, st);
    return gemm16_typed<_Float16>(ta, tb, g, st);
}

}  // namespace tt
