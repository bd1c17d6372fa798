// 16-bit GEMM, large-tile variant (dtype TT_BF16 / TT_F16 of tt_gemm when
// M, N >= 256): the same arithmetic as gemm16_kernel (v_mfma_f32_16x16x32,
// fp32 accumulators, alpha/beta in fp32, one rounding at the store) with
//  - BM x BN workgroup tiles, four wavefronts of (BM / 2) x (BN / 2);
//    256 x 256: 8 x 8 MFMA blocks per wave, 256 fp32 accumulators per lane
//    (AGPRs; this file is built without the VGPR-accumulator option the other
//    kernels use), one workgroup per CU; 128 x 256: 4 x 8 blocks, two
//    workgroups per CU, whose independent barriers let one workgroup's MFMAs
//    run while the other waits; 128 x 128 (small grids): 4 x 4 blocks, three
//    workgroups per CU,
//  - operands copied global -> LDS by the direct-load path
//    (global_load_lds_dwordx4: no VGPR staging and no ds_write), 16 bytes per
//    lane, one kilobyte of LDS per wavefront instruction,
//  - an LDS ring of 32-deep stages, one barrier per stage: four slots with
//    three stages in flight (256 x 256, 128 KB) or three slots with two in
//    flight (128 x 256, 72 KB; 128 x 128, 48 KB).
// BM = 256: per stage a wave issues 64 MFMAs (1024 MFMA cycles) against 16 KB
// of LDS reads; the four waves together read 64 KB and the direct loads write
// 32 KB, 96 bytes per clock at the full MFMA rate, of the 256 the LDS serves
// when every 16-lane quarter of a 16-byte access covers one 256-byte run
// (BM = 128 moves half as many bytes again per MFMA).
//
// Stage layouts in LDS (unpadded; 16-byte pieces XOR-swizzled against LDS
// bank conflicts, the swizzles chosen by measurement):
//   k-contiguous operand: row r (32 k = four pieces, 64 bytes) at r * 64,
//     global piece p at position p ^ ((r >> 1) & 3) (bitwise-equal
//     measurements, 4096^3 and 8192^3: +2.2-2.9% against (r >> 2) & 3;
//     r & 3 and no swizzle no better);
//   row-contiguous operand: k-row kr (ROWS rows = ROWS / 8 pieces, 2 ROWS
//     bytes) at kr * 2 ROWS, global piece p at position p ^ (2 (kr & 3)).
// Direct load q (0..ROWS/16 - 1) of an operand fills bytes [1024 q, 1024 q +
// 1024); wave w issues q = w, w + 4, ..., and lane l writes position l.
// The host launches this kernel on whole tiles only (K a multiple of 32,
// 16-byte aligned operands); ragged row and column strips run on the
// register-staged kernel.
#include <type_traits>

#include "tt_gemm.hpp"

namespace tt {

namespace {

typedef __bf16 dbf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 df16x8 __attribute__((ext_vector_type(8)));
typedef float df32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short du16x8 __attribute__((ext_vector_type(8)));
typedef short ds16x4 __attribute__((ext_vector_type(4)));

constexpr int kDK = 32;                   // k per stage
constexpr int kSlots = 4;                 // LDS ring slots (three stages in flight)

template <typename T>
__device__ __forceinline__ df32x4 mma16(du16x8 a, du16x8 b, df32x4 c) {
    if constexpr (std::is_same<T, __bf16>::value)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(dbf16x8, a), __builtin_bit_cast(dbf16x8, b), c,
                                                       0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(df16x8, a), __builtin_bit_cast(df16x8, b), c, 0,
                                                      0, 0);
}

// The direct loads are issued as inline assembly (M0 = this instruction's LDS
// kilobyte, then global_load_lds_dwordx4). Issued through the compiler
// builtin, they are LDS writes the compiler cannot tell apart from any LDS
// read, so every operand read would wait for all of them, including the
// stages still in flight. As assembly they are invisible to the compiler; the
// loop's own s_waitcnt and barrier order them against the reads, and the
// compiler keeps tracking the reads themselves. Nothing else in the kernel
// uses M0.
__device__ __forceinline__ unsigned lds_off(const void* p) {
    return (unsigned)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
__device__ __forceinline__ void dma16(const unsigned short* g, unsigned lds_kilobyte) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(lds_kilobyte)), "v"(g)
                 : "memory", "m0");
}

template <bool KC, int ROWS = 256>
struct DStage {
    static_assert(ROWS == 256 || ROWS == 128, "stage rows");
    static constexpr int KRB = ROWS * 2;  // bytes per k-row of a row-contiguous stage
    // Row and k offsets (relative to the tile's row0 and the stage's k0) of
    // the 8 elements lane `lane` of direct load q fetches.
    __device__ __forceinline__ static void src(int q, int lane, int& row, int& k) {
        if (KC) {
            const int r = 16 * q + (lane >> 2);
            row = r;
            k = 8 * ((lane & 3) ^ ((r >> 1) & 3));
        } else {
            const int kr = (1024 / KRB) * q + lane / (KRB / 16);
            k = kr;
            row = 8 * ((lane % (KRB / 16)) ^ (2 * (kr & 3)));
        }
    }

    // Interior stage: this wave's four direct loads (all addresses in range);
    // slot_off is the stage's LDS byte address, uniform across the wave.
    __device__ __forceinline__ static void dma(const unsigned short* p, int64_t ld, int64_t row0, int64_t k0,
                                               unsigned slot_off, int wave, int lane) {
#pragma unroll
        for (int i = 0; i < ROWS / 64; ++i) {
            const int q = wave + 4 * i;
            int r, k;
            src(q, lane, r, k);
            const unsigned short* g = KC ? p + (row0 + r) * ld + k0 + k : p + (k0 + k) * ld + row0 + r;
            dma16(g, slot_off + 1024 * q);
        }
    }

    // This lane's MFMA operand for the 16 rows from rb: rows rb + (lane % 16),
    // k 8 (lane / 16) .. 8 (lane / 16) + 7 (layout of the 16x16x32 MFMA).
    __device__ __forceinline__ static du16x8 frag(const unsigned char* slot, int rb, int lane) {
        if (KC) {
            const int r = rb + (lane & 15), c = lane >> 4;
            return *reinterpret_cast<const du16x8*>(slot + r * 64 + 16 * (c ^ ((r >> 1) & 3)));
        }
        // Transposing reads: within 16 lanes, lane 4 j + a supplies the 8-byte
        // block of rows 4 b .. 4 b + 3 (b = rb / 4 + a) of k-row 8 g + 4 h + j,
        // and lane 4 a + e receives element e of the blocks of lanes 4 j + a.
        const int g = lane >> 4, j = (lane & 15) >> 2, a = lane & 3;
        const int b = (rb >> 2) + a;
        ds16x4 h[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int kr = 8 * g + 4 * hh + j;
            const int pos = (b >> 1) ^ (2 * (kr & 3));
            typedef __attribute__((address_space(3))) ds16x4 lds_s16x4;
            h[hh] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(slot + kr * KRB + 16 * pos + 8 * (b & 1)));
        }
        return du16x8{(unsigned short)h[0][0], (unsigned short)h[0][1], (unsigned short)h[0][2], (unsigned short)h[0][3],
                      (unsigned short)h[1][0], (unsigned short)h[1][1], (unsigned short)h[1][2], (unsigned short)h[1][3]};
    }
};

template <typename T>
__device__ __forceinline__ float dto_f32(unsigned short x) {
    return (float)__builtin_bit_cast(T, x);
}
template <typename T>
__device__ __forceinline__ unsigned short dfrom_f32(float x) {
    return __builtin_bit_cast(unsigned short, (T)x);
}

template <typename T, bool TA, bool TB, int BM, int BN>
__global__ __launch_bounds__(256, BN == 128 ? 3 : (BM == 128 ? 2 : 1)) void gemm16_dma_kernel(GemmArgs g) {
    // A rows are m: k-contiguous unless transposed. B rows are n: k-contiguous iff transposed.
    typedef DStage<!TA, BM> SA;
    typedef DStage<TB, BN> SB;
    constexpr int FM = BM / 32;                 // 16-row MFMA blocks per wave
    constexpr int FN = BN / 32;                 // 16-column MFMA blocks per wave
    constexpr int WN = BN / 2;                  // wave tile columns
    constexpr int NS = BM == 256 ? kSlots : 3;  // ring slots
    constexpr int AB = BM * kDK * 2;            // A bytes per stage
    constexpr int SB_ = AB + BN * kDK * 2;      // slot bytes
    constexpr int DPW = BM / 64 + BN / 64;      // direct loads per wave per stage
    __shared__ __attribute__((aligned(1024))) unsigned char lds[NS * SB_];

    const int64_t tiles = g.tiles_m * g.tiles_n;
    const int64_t total = tiles * g.batch;
    const int64_t id = xcd_remap(blockIdx.x, total);
    const int64_t bat = id / tiles;
    const int64_t t = id - bat * tiles;
    constexpr int64_t GROUP = 4;
    const int64_t grp = t / (GROUP * g.tiles_n);
    const int64_t first_m = grp * GROUP;
    const int64_t gsize = min(g.tiles_m - first_m, GROUP);
    const int64_t rem = t - grp * GROUP * g.tiles_n;
    const int64_t m0 = (first_m + rem % gsize) * BM;
    const int64_t n0 = (rem / gsize) * BN;

    const unsigned short* A = static_cast<const unsigned short*>(g.A) + bat * g.sA;
    const unsigned short* B = static_cast<const unsigned short*>(g.B) + bat * g.sB;
    const int lane = threadIdx.x & 63;
    // Uniform by construction; as a scalar it keeps every direct load's LDS
    // offset (M0) in scalar registers.
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm0 = (wave >> 1) * (BM / 2);
    const int wn0 = (wave & 1) * WN;

    // The host launches this kernel on whole tiles only (M, N multiples of
    // 256 within the launch, K a multiple of 32, 16-byte aligned operands).
    const int64_t nk = g.K / kDK;
    auto slot = [&](int64_t s) __attribute__((always_inline)) -> unsigned char* { return lds + ((int)s % NS) * SB_; };

    df32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = df32x4{0, 0, 0, 0};

    auto read = [&](du16x8 (&fa)[FM], du16x8 (&fb)[FN], int64_t s) __attribute__((always_inline)) {
        const unsigned char* sl = slot(s);
#pragma unroll
        for (int j = 0; j < FN; ++j) fb[j] = SB::frag(sl + AB, wn0 + 16 * j, lane);
#pragma unroll
        for (int i = 0; i < FM; ++i) fa[i] = SA::frag(sl, wm0 + 16 * i, lane);
    };
    auto mfma = [&](du16x8 (&fa)[FM], du16x8 (&fb)[FN]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) acc[i][j] = mma16<T>(fa[i], fb[j], acc[i][j]);
    };
    // Make stage s readable by every wave, with `ahead` direct-loaded stages
    // issued after it: this wave's direct loads of stage s are its oldest
    // outstanding ones (vector-memory ops complete in order), so those of the
    // later stages may stay in flight; lgkmcnt(0) also retires this wave's LDS
    // reads of earlier stages and register-staged writes. A plain barrier then
    // publishes stage s and frees the slot every wave has finished reading (a
    // fenced barrier would also wait for the later stages).
    auto ready = [&](int64_t ahead) __attribute__((always_inline)) {
        // s_waitcnt immediate: vmcnt in bits 3:0 and 15:14, expcnt 6:4 (7: no
        // wait), lgkmcnt 11:8.
        constexpr auto imm = [](int vm) { return (vm & 15) | ((vm >> 4) << 14) | 0x70; };  // lgkmcnt(0), no expcnt wait
        if (ahead >= 3) __builtin_amdgcn_s_waitcnt(imm(3 * DPW));
        else if (ahead == 2) __builtin_amdgcn_s_waitcnt(imm(2 * DPW));
        else if (ahead == 1) __builtin_amdgcn_s_waitcnt(imm(DPW));
        else __builtin_amdgcn_s_waitcnt(imm(0));
        asm volatile("s_barrier" ::: "memory");
    };
    // One stage at a time: after the barrier that publishes stage kt, stage
    // kt + 3 is loaded into the slot stage kt - 1 used, then stage kt's
    // operands are read and its MFMAs run.
    // Slot offsets are integer LDS addresses: converting a generic pointer per
    // load cost a null check and a vector-to-scalar move on every one.
    const unsigned lds0 = lds_off(lds);
    auto dma = [&](int64_t s) __attribute__((always_inline)) {
        const unsigned so = lds0 + (unsigned)((int)s % NS) * SB_;
        SA::dma(A, g.lda, m0, s * kDK, so, wave, lane);
        SB::dma(B, g.ldb, n0, s * kDK, so + AB, wave, lane);
    };
    for (int64_t s = 0; s < NS - 1 && s < nk; ++s) dma(s);
    for (int64_t kt = 0; kt < nk; ++kt) {
        // Stages issued after stage kt: those below min(nk, kt + NS - 1).
        ready(min<int64_t>(nk, kt + NS - 1) - (kt + 1));
        if (kt + NS - 1 < nk) dma(kt + NS - 1);
        du16x8 fa[FM], fb[FN];
        read(fa, fb, kt);
        mfma(fa, fb);
        // Software pipeline for the scheduler: the B fragments and the first
        // two A fragments are read up front, then each row's 8 MFMAs are
        // followed by the read of the A fragment two rows ahead, so every
        // read has a row of MFMAs to land in (left alone, the scheduler put
        // each A read right before its row, behind a full wait).
        constexpr int RA = TA ? 2 : 1;  // LDS read instructions per A fragment
        constexpr int RB = TB ? 1 : 2;  // per B fragment
        __builtin_amdgcn_sched_group_barrier(0x100, FN * RB + 2 * RA, 0);
#pragma unroll
        for (int i = 0; i < FM - 2; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, FN, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, RA, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 2 * FN, 0);
    }
    __syncthreads();

    // Epilogue through LDS, one 16-row slab of the wave's tile at a time (fp32,
    // alpha applied); each lane then finishes 8 consecutive columns of one row
    // with a 16-byte load of C and a 16-byte store of D.
    const unsigned short* C = g.C ? static_cast<const unsigned short*>(g.C) + bat * g.sC : nullptr;
    unsigned short* D = static_cast<unsigned short*>(g.D) + bat * g.sD;
    const float alpha = (float)g.alpha;
    const float beta = (float)g.beta;
    constexpr int SP = WN + 4;  // slab pitch in floats
    constexpr int CPR = WN / 8;  // 8-column chunks per slab row
    static_assert(4 * 16 * SP * sizeof(float) <= sizeof(lds), "epilogue slabs fit in the ring");
    float* slab = reinterpret_cast<float*>(lds) + wave * 16 * SP;
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    const bool vout = a16(D) && g.ldd % 8 == 0 && (!C || (a16(C) && g.ldc % 8 == 0));
    const int lrow = lane & 15, lg = lane >> 4;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        // This slab's C chunks are loaded before any of its stores (and before the
        // slab exchange, whose barrier then covers their latency): D may
        // alias C, so the compiler cannot move a load of C past a store of D,
        // and chunk-by-chunk loads would each wait out a full memory latency.
        du16x8 cc[16 * CPR / 64];
#pragma unroll
        for (int h = 0; h < 16 * CPR / 64; ++h) {
            const int v = lane + 64 * h;
            const int rr = v / CPR, cb = v % CPR;
            const int64_t row = m0 + wm0 + 16 * i + rr;
            const int64_t col = n0 + wn0 + 8 * cb;
            cc[h] = du16x8{0, 0, 0, 0, 0, 0, 0, 0};
            if (C && vout && row < g.M && col + 8 <= g.N) cc[h] = *reinterpret_cast<const du16x8*>(C + row * g.ldc + col);
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
        for (int h = 0; h < 16 * CPR / 64; ++h) {
            const int v = lane + 64 * h;
            const int rr = v / CPR, cb = v % CPR;
            const int64_t row = m0 + wm0 + 16 * i + rr;
            const int64_t col = n0 + wn0 + 8 * cb;
            const df32x4 lo = *reinterpret_cast<const df32x4*>(slab + rr * SP + 8 * cb);
            const df32x4 hi = *reinterpret_cast<const df32x4*>(slab + rr * SP + 8 * cb + 4);
            float x[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            if (row < g.M) {
                if (vout && col + 8 <= g.N) {
                    if (C) {
#pragma unroll
                        for (int e = 0; e < 8; ++e) x[e] = x[e] + beta * dto_f32<T>(cc[h][e]);
                    }
                    du16x8 d;
#pragma unroll
                    for (int e = 0; e < 8; ++e) d[e] = dfrom_f32<T>(x[e]);
                    *reinterpret_cast<du16x8*>(D + row * g.ldd + col) = d;
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (col + e < g.N) {
                            float y = x[e];
                            if (C) y = y + beta * dto_f32<T>(C[row * g.ldc + col + e]);
                            D[row * g.ldd + col + e] = dfrom_f32<T>(y);
                        }
                }
            }
        }
        __syncthreads();
    }
}

template <typename T>
int launch16_dma(bool ta, bool tb, GemmArgs& g, hipStream_t st) {
    // Tile height, measured at bf16 (TFLOP/s, 128 against 256 rows): NN 4096^3
    // 1104 against 1029, 4096^2 x 1024 855 against 704-740; TN 4096^3
    // 1169-1172 against 1030-1034, x 1024 902-911 against 725-732; NT
    // 4096^2 x 1024 797 against 734-748, x 2048 931 against 905-917, x 3072
    // 987-989 against 980-992, 4096^3 1013 against 1043; TT x 1024 846-850
    // against 747-754, x 2048 993-995 against 921-946, 4096^3 1088-1091
    // against 1070-1077.
    int bm, bn;
    gemm16_dma_tile(ta, tb, g.M, g.N, g.K, g.batch, bm, bn);
    const bool rows128 = bm == 128;
    g.tiles_m = (g.M + bm - 1) / bm;
    g.tiles_n = (g.N + bn - 1) / bn;
    const int64_t total = g.tiles_m * g.tiles_n * g.batch;
    if (total > 0x7fffffffLL) return set_error(TT_UNSUPPORTED, "tt_gemm: %lld tiles exceed one launch", (long long)total);
    const dim3 grid((unsigned)total), block(256);
    if (bn == 128) {
        if (!ta && !tb) hipLaunchKernelGGL((gemm16_dma_kernel<T, false, false, 128, 128>), grid, block, 0, st, g);
        if (!ta && tb) hipLaunchKernelGGL((gemm16_dma_kernel<T, false, true, 128, 128>), grid, block, 0, st, g);
        if (ta && !tb) hipLaunchKernelGGL((gemm16_dma_kernel<T, true, false, 128, 128>), grid, block, 0, st, g);
        if (ta && tb) hipLaunchKernelGGL((gemm16_dma_kernel<T, true, true, 128, 128>), grid, block, 0, st, g);
        return check_launch("tt_gemm (16-bit, direct loads)");
    }
    if (!ta && !tb) hipLaunchKernelGGL((gemm16_dma_kernel<T, false, false, 128, 256>), grid, block, 0, st, g);
    if (!ta && tb && rows128) hipLaunchKernelGGL((gemm16_dma_kernel<T, false, true, 128, 256>), grid, block, 0, st, g);
    if (!ta && tb && !rows128) hipLaunchKernelGGL((gemm16_dma_kernel<T, false, true, 256, 256>), grid, block, 0, st, g);
    if (ta && !tb) hipLaunchKernelGGL((gemm16_dma_kernel<T, true, false, 128, 256>), grid, block, 0, st, g);
    if (ta && tb) hipLaunchKernelGGL((gemm16_dma_kernel<T, true, true, 128, 256>), grid, block, 0, st, g);
    return check_launch("tt_gemm (16-bit, direct loads)");
}

}  // namespace

int gemm16_dma_rows(bool ta, bool tb, int64_t K) { return ta || !tb || K <= 2048 ? 128 : 256; }

// Tile of the direct-load kernel: bm rows as above; 128 columns instead of 256
// (three workgroups per CU) when fewer than 256 tiles of 128 x 256 would run.
void gemm16_dma_tile(bool ta, bool tb, int64_t M, int64_t N, int64_t K, int64_t batch, int& bm, int& bn) {
    bm = gemm16_dma_rows(ta, tb, K);
    bn = 256;
    if (bm == 128 && (M / 128) * (N / 256) * batch < 256) bn = 128;
}

int gemm16_dma_dispatch(int dtype, bool ta, bool tb, GemmArgs& g, hipStream_t st) {
    if (dtype == TT_BF16) return launch16_dma<__bf16>(ta, tb, g, st);
    return launch16_dma<_Float16>(ta, tb, g, st);
}

}  // namespace tt
