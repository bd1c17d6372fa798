// 16-bit GEMM for bf16 / fp16 operands (dtype TT_BF16 / TT_F16 of tt_gemm):
//   D = alpha * op(A) op(B) (+ beta * C), products and sums in fp32 on
//   v_mfma_f32_16x16x32_{bf16,f16}, alpha/beta applied in fp32, one rounding
//   to the 16-bit type at the store.
//
// Workgroup: 256 threads = 4 wavefronts, 128 x 128 output tile, each wave a
// 64 x 64 sub-tile (4 x 4 MFMA blocks of 16 x 16, fp32 accumulators). K
// advances 64 per stage through two LDS buffers (one barrier per stage).
//
// MFMA operand layout (16x16x32): lane l holds A[l % 16][8 (l / 16) + j] and
// B[8 (l / 16) + j][l % 16], j = 0..7; accumulator element r holds
// D[4 (l / 16) + r][l % 16].
//
// Each operand is staged in its memory order, so staging is a plain copy:
//   k-contiguous operand: LDS [row][k], 144-byte row pitch; thread t copies
//     32 consecutive k of row t / 2; a lane's MFMA operand (8 consecutive k of
//     one row) is one 16-byte read;
//   row-contiguous operand: LDS [k][row], 288-byte k-row pitch; thread t
//     copies 32 consecutive rows of k-row t / 4; a lane's MFMA operand is
//     gathered across k-rows by two transposing reads h = 0, 1
//     (ds_read_b64_tr_b16: within each 16 lanes, lane 16 g + 4 j + a supplies
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

constexpr int kT = 128;      // output tile rows and columns
constexpr int kK = 64;       // k per stage
constexpr int kP = kK + 8;   // [row][k] pitch in elements (144 bytes)
constexpr int kPR = kT + 16; // [k][row] pitch in elements (288 bytes)
constexpr int kStage = kT * kP;
static_assert(kK * kPR == kStage, "both stage layouts fill the same buffer");

template <bool KC>
struct Stage16 {
    u16x8 reg[4];

    // FAST: interior stage, 16-byte aligned rows: unconditional vector loads.
    // Otherwise element loads from clamped addresses, zero outside.
    template <bool FAST>
    __device__ __forceinline__ void load(const unsigned short* __restrict__ p, int64_t ld, int64_t row0, int64_t rows,
                                         int64_t k0, int64_t kdim) {
        const int t = threadIdx.x;
        if (KC) {
            const int r = t >> 1;
            const int kb = (t & 1) * 32;
            if (FAST) {
                const unsigned short* src = p + (row0 + r) * ld + k0 + kb;
#pragma unroll
                for (int c = 0; c < 4; ++c) reg[c] = *reinterpret_cast<const u16x8*>(src + 8 * c);
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c)
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const int64_t gr = row0 + r, gk = k0 + kb + 8 * c + e;
                        const bool ok = gr < rows && gk < kdim;
                        const unsigned short x = *(ok ? p + gr * ld + gk : p);
                        reg[c][e] = ok ? x : (unsigned short)0;
                    }
            }
        } else {
            const int k = t >> 2;
            const int rb = (t & 3) * 32;
            if (FAST) {
                const unsigned short* src = p + (k0 + k) * ld + row0 + rb;
#pragma unroll
                for (int c = 0; c < 4; ++c) reg[c] = *reinterpret_cast<const u16x8*>(src + 8 * c);
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c)
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const int64_t gr = row0 + rb + 8 * c + e, gk = k0 + k;
                        const bool ok = gr < rows && gk < kdim;
                        const unsigned short x = *(ok ? p + gk * ld + gr : p);
                        reg[c][e] = ok ? x : (unsigned short)0;
                    }
            }
        }
    }

    __device__ __forceinline__ void store(unsigned short* s) const {
        const int t = threadIdx.x;
        unsigned short* dst = KC ? s + (t >> 1) * kP + (t & 1) * 32 : s + (t >> 2) * kPR + (t & 3) * 32;
#pragma unroll
        for (int c = 0; c < 4; ++c) *reinterpret_cast<u16x8*>(dst + 8 * c) = reg[c];
    }

    // This lane's MFMA operand for the 16 rows from rb, k step ks (k 32 ks .. 32 ks + 31).
    __device__ __forceinline__ static u16x8 frag(const unsigned short* s, int rb, int ks, int lane) {
        if (KC) return *reinterpret_cast<const u16x8*>(s + (rb + (lane & 15)) * kP + 32 * ks + 8 * (lane >> 4));
        const int g = lane >> 4, j = (lane & 15) >> 2, a = lane & 3;
        const unsigned short* base = s + (32 * ks + 8 * g + j) * kPR + rb + 4 * a;
        typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base + 4 * kPR));
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

template <typename T, bool TA, bool TB, bool VEC>
__global__ __launch_bounds__(256) void gemm16_kernel(GemmArgs g) {
    // A rows are m: k-contiguous unless transposed. B rows are n: k-contiguous iff transposed.
    typedef Stage16<!TA> SA;
    typedef Stage16<TB> SB;
    __shared__ __attribute__((aligned(16))) unsigned short lds[2 * 2 * kStage];
    auto bufA = [&](int b) -> unsigned short* { return lds + b * kStage; };
    auto bufB = [&](int b) -> unsigned short* { return lds + (2 + b) * kStage; };

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
    const int64_t m0 = (first_m + rem % gsize) * kT;
    const int64_t n0 = (rem / gsize) * kT;

    const unsigned short* A = static_cast<const unsigned short*>(g.A) + bat * g.sA;
    const unsigned short* B = static_cast<const unsigned short*>(g.B) + bat * g.sB;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm0 = (wave >> 1) * 64;
    const int wn0 = (wave & 1) * 64;
    const int lrow = lane & 15;
    const int lg = lane >> 4;

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0, 0, 0, 0};

    SA sa;
    SB sb;
    const int64_t nk = (g.K + kK - 1) / kK;
    const int64_t nfull = (VEC && m0 + kT <= g.M && n0 + kT <= g.N) ? g.K / kK : 0;
    auto load = [&](int64_t k0, auto fast) {
        constexpr bool F = decltype(fast)::value;
        sa.template load<F>(A, g.lda, m0, g.M, k0, g.K);
        sb.template load<F>(B, g.ldb, n0, g.N, k0, g.K);
    };
    auto compute = [&](int buf) {
        const unsigned short* a = bufA(buf);
        const unsigned short* b = bufB(buf);
#pragma unroll
        for (int ks = 0; ks < kK / 32; ++ks) {
            u16x8 fa[4], fb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) fa[i] = SA::frag(a, wm0 + 16 * i, ks, lane);
#pragma unroll
            for (int j = 0; j < 4; ++j) fb[j] = SB::frag(b, wn0 + 16 * j, ks, lane);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = Mfma16<T>::mma(fa[i], fb[j], acc[i][j]);
        }
    };
    if (nk > 0) {
        if (nfull > 0) load(0, std::true_type{});
        else load(0, std::false_type{});
        sa.store(bufA(0));
        sb.store(bufB(0));
    }
    __syncthreads();
    int64_t kt = 0;
    for (; kt + 1 < nfull; ++kt) {
        load((kt + 1) * kK, std::true_type{});
        compute(kt & 1);
        __builtin_amdgcn_sched_barrier(0);
        sa.store(bufA((kt & 1) ^ 1));
        sb.store(bufB((kt & 1) ^ 1));
        __syncthreads();
    }
    for (; kt < nk; ++kt) {
        const bool more = kt + 1 < nk;
        if (more) load((kt + 1) * kK, std::false_type{});
        compute(kt & 1);
        __builtin_amdgcn_sched_barrier(0);
        if (more) {
            sa.store(bufA((kt & 1) ^ 1));
            sb.store(bufB((kt & 1) ^ 1));
        }
        __syncthreads();
    }

    const unsigned short* C = g.C ? static_cast<const unsigned short*>(g.C) + bat * g.sC : nullptr;
    unsigned short* D = static_cast<unsigned short*>(g.D) + bat * g.sD;
    const float alpha = (float)g.alpha;
    const float beta = (float)g.beta;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t col = n0 + wn0 + 16 * j + lrow;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = m0 + wm0 + 16 * i + 4 * lg + r;
                if (row < g.M && col < g.N) {
                    float v = acc[i][j][r];
                    if (g.alpha != 1.0) v = alpha * v;
                    if (C) v = v + beta * to_f32<T>(C[row * g.ldc + col]);
                    D[row * g.ldd + col] = from_f32<T>(v);
                }
            }
        }
}

template <typename T>
int gemm16_typed(bool ta, bool tb, GemmArgs& g, hipStream_t st) {
    auto ok16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    bool vec = ok16(g.A) && ok16(g.B) && g.lda % 8 == 0 && g.ldb % 8 == 0;
    if (g.batch > 1) vec = vec && g.sA % 8 == 0 && g.sB % 8 == 0;
    g.tiles_m = (g.M + kT - 1) / kT;
    g.tiles_n = (g.N + kT - 1) / kT;
    const int64_t total = g.tiles_m * g.tiles_n * g.batch;
    if (total > 0x7fffffffLL) return set_error(TT_UNSUPPORTED, "tt_gemm: %lld tiles exceed one launch", (long long)total);
    const dim3 grid((unsigned)total), block(256);
#define TT_GEMM16_CASE(TA, TB, VC) \
    if (ta == TA && tb == TB && vec == VC) hipLaunchKernelGGL((gemm16_kernel<T, TA, TB, VC>), grid, block, 0, st, g);
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

}  // namespace

int gemm16_dispatch(int dtype, bool ta, bool tb, GemmArgs& g, hipStream_t st) {
    if (dtype == TT_BF16) return gemm16_typed<__bf16>(ta, tb, g, st);
    return gemm16_typed<_Float16>(ta, tb, g, st);
}

}  // namespace tt
