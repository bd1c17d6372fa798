// fp32 GEMM and batched GEMM on 256 x 256 tiles with both operands staged
// through LDS (tt_gemm, TT_F32, both operands not transposed, whole tiles, K
// a multiple of 32, 16-byte aligned; the dispatcher takes it in whole rounds
// of one tile per CU, without C or with K >= 1024).
//
// Four waves of 128 x 128 (8 x 8 blocks of v_mfma_f32_16x16x4f32), one wave
// per SIMD, one workgroup per CU (144 KiB of LDS). The 256 fp32 accumulators
// per lane live in AGPRs: this file is built without the VGPR-accumulator
// option the other kernels use, which leaves the wave its 256 VGPRs for two
// sets of fragments and the staging registers.
//
// Stages of 32 k (two 16-k chunks), double-buffered in LDS, one barrier per
// stage; A rows padded by 8 floats, B k-rows unpadded (no LDS bank conflicts;
// B k-rows padded by 4 floats conflicted in 3/8 of the LDS-active cycles).
// With one wave per SIMD nothing else covers a stall, so the loop is
// software-pipelined and every memory instruction is spread among the MFMAs:
//  - chunk 0's MFMAs run with chunk 1's fragment reads and the next stage's
//    global loads interleaved, one of each per 16 MFMAs;
//  - chunk 1's first three MFMA steps run with the next stage's LDS stores
//    (into the other buffer, which the previous barrier released), one per
//    12 MFMAs;
//  - the barrier comes before chunk 1's last step, whose 64 MFMAs run with
//    the next stage's chunk-0 fragment reads, one per 4 MFMAs.
// Same box, alternating, fraction of the fp32 peak: 4096^3 0.933, 8192^2 x
// 2048 0.934, 2048 x 8192 x 4096 0.929, 4096^2 x 1024 0.892, against 0.920,
// 0.924, 0.919, 0.876 for eight waves of 64 x 128 at two waves per SIMD
// (accumulators in VGPRs, no room for a second fragment set) and 0.88 or
// less for the 64 x 256 direct-B tiles.
//
// Fragments (the layout of gemm_directb_kernel, whose results this kernel
// reproduces bitwise): chunk h of a stage is 16 k; MFMA step p of chunk h
// gives lane group g = lane / 16 the k index 16 h + 4 g + p. A lane's A
// operand for row block a is row 16 a + lane % 16, four consecutive k (one
// 16-byte LDS read feeds steps 0..3); its B operand piece for step p is four
// consecutive columns 4 (lane % 16) .. + 3 of one k-row (one 16-byte read),
// one column for each of the four MFMA column blocks of a 64-column set.
#include "tt_gemm.hpp"

namespace tt {

namespace {

typedef float f4_v __attribute__((ext_vector_type(4)));

constexpr int kBigM = 256, kBigN = 256, kBigK = 32;  // tile and stage
constexpr int kBigThreads = 256;

__global__ __launch_bounds__(kBigThreads, 1) void gemm_big_f32_kernel(GemmArgs g) {
    constexpr int T = kBigThreads, BK = kBigK;
    constexpr int AP = BK + 8;          // floats per A row in LDS
    constexpr int BP = kBigN;           // floats per B k-row in LDS
    constexpr int AE = kBigM * AP;      // A floats per stage buffer
    constexpr int BE = BK * BP;         // B floats per stage buffer
    constexpr int LA = BK / 4;          // threads per A row (16 bytes each)
    constexpr int RA = kBigM * LA / T;  // A loads per thread per stage
    constexpr int RB = BK * 64 / T;     // B loads per thread per stage (64 threads per k-row)
    constexpr int NL = RA + RB;
    static_assert(NL == 16, "the schedule below spreads 16 loads, stores and fragment reads");
    __shared__ __attribute__((aligned(16))) float lds[2 * (AE + BE)];

    // Batch-major; within a product, rows of tiles in groups of four, each
    // group column-major: an XCD's contiguous range of tiles is a block four
    // tile rows high.
    const int64_t tiles = g.tiles_m * g.tiles_n;
    const int64_t id0 = xcd_remap(blockIdx.x, tiles * g.batch);
    const int64_t bat = id0 / tiles, id = id0 - bat * tiles;
    const int64_t grp = id / (4 * g.tiles_n);
    const int64_t gm = min((int64_t)4, g.tiles_m - grp * 4);
    const int64_t rr = id - grp * 4 * g.tiles_n;
    const int64_t tn = rr / gm, tm = grp * 4 + rr % gm;
    const int64_t m0 = tm * kBigM, n0 = tn * kBigN;
    const float* A = static_cast<const float*>(g.A) + bat * g.sA;
    const float* B = static_cast<const float*>(g.B) + bat * g.sB;

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int w = t >> 6;
    const int lg = lane >> 4, c = lane & 15;
    const int wm = w >> 1, wn = w & 1;  // rows 128 wm .., columns 128 wn ..

    // Global -> registers: A rows t / LA + (T / LA) i, k (t % LA) 4; B k-rows
    // t / 64 + (T / 64) i, columns (t % 64) 4. Every instruction covers whole
    // rows of the stage (BK floats of A, 256 of B).
    f4_v ra[RA], rb[RB];
    const float* ag = A + (m0 + t / LA) * g.lda + (t % LA) * 4;
    const float* bg = B + (int64_t)(t >> 6) * g.ldb + n0 + (t & 63) * 4;
    auto gload = [&](int64_t k0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < RA; ++i) ra[i] = *reinterpret_cast<const f4_v*>(ag + (T / LA) * i * g.lda + k0);
#pragma unroll
        for (int i = 0; i < RB; ++i) rb[i] = *reinterpret_cast<const f4_v*>(bg + (k0 + (T / 64) * i) * g.ldb);
    };
    auto sstore = [&](int buf) __attribute__((always_inline)) {
        float* as = lds + buf * (AE + BE);
        float* bs = as + AE;
#pragma unroll
        for (int i = 0; i < RA; ++i)
            *reinterpret_cast<f4_v*>(as + (t / LA + (T / LA) * i) * AP + (t % LA) * 4) = ra[i];
#pragma unroll
        for (int i = 0; i < RB; ++i)
            *reinterpret_cast<f4_v*>(bs + ((t >> 6) + (T / 64) * i) * BP + (t & 63) * 4) = rb[i];
    };
    // Chunk h's fragments of stage buffer buf: eight A pieces, then the B
    // pieces of both 64-column sets for steps 0..3.
    auto reads = [&](int buf, int h, f4_v (&fa)[8], f4_v (&fb)[2][4]) __attribute__((always_inline)) {
        const float* as = lds + buf * (AE + BE);
        const float* bs = as + AE;
#pragma unroll
        for (int a = 0; a < 8; ++a)
            fa[a] = *reinterpret_cast<const f4_v*>(as + (128 * wm + 16 * a + c) * AP + 16 * h + 4 * lg);
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int p = 0; p < 4; ++p)
                fb[s][p] = *reinterpret_cast<const f4_v*>(bs + (16 * h + 4 * lg + p) * BP + 128 * wn + 64 * s + 4 * c);
    };

    f4_v acc[8][8];
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[a][j] = f4_v{0, 0, 0, 0};
    // MFMA steps p0 .. p1 - 1 of one chunk: 64 MFMAs per step.
    auto mfma = [&](const f4_v (&fa)[8], const f4_v (&fb)[2][4], int p0, int p1) __attribute__((always_inline)) {
#pragma unroll
        for (int p = p0; p < p1; ++p)
#pragma unroll
            for (int a = 0; a < 8; ++a)
#pragma unroll
                for (int s = 0; s < 2; ++s)
#pragma unroll
                    for (int b = 0; b < 4; ++b)
                        acc[a][4 * s + b] =
                            __builtin_amdgcn_mfma_f32_16x16x4f32(fa[a][p], fb[s][p][b], acc[a][4 * s + b], 0, 0, 0);
    };

    // Scheduling-group masks: 0x008 MFMA, 0x020 global load, 0x100 LDS read,
    // 0x200 LDS write.
    f4_v fa0[8], fb0[2][4], fa1[8], fb1[2][4];
    const int64_t nk = g.K / BK;
    gload(0);
    sstore(0);
    __syncthreads();
    reads(0, 0, fa0, fb0);
    int64_t st = 0;
    for (; st + 1 < nk; ++st) {
        const int buf = (int)(st & 1);
        reads(buf, 1, fa1, fb1);
        gload((st + 1) * BK);
        mfma(fa0, fb0, 0, 4);
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        sstore(buf ^ 1);
        mfma(fa1, fb1, 0, 3);
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 12, 0);
            __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        reads(buf ^ 1, 0, fa0, fb0);
        mfma(fa1, fb1, 3, 4);
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    reads((int)(st & 1), 1, fa1, fb1);
    mfma(fa0, fb0, 0, 4);
    mfma(fa1, fb1, 0, 4);

    // D = alpha acc (+ beta C): acc[a][4 s + b][r] is row m0 + 128 wm + 16 a +
    // 4 lg + r, column n0 + 128 wn + 64 s + 4 c + b; a lane's four columns
    // are one 16-byte piece.
    float* D = static_cast<float*>(g.D) + bat * g.sD;
    const float* C = g.C ? static_cast<const float*>(g.C) + bat * g.sC : nullptr;
    const float alpha = (float)g.alpha, beta = (float)g.beta;
    // C of row blocks a and a + 1 in flight: block a + 2's loads are issued
    // after block a's stores (they read other rows, so D may alias C).
    f4_v cv[2][4][2];
    auto cload = [&](int a, f4_v (&dst)[4][2]) __attribute__((always_inline)) {
        const int64_t row0 = m0 + 128 * wm + 16 * a + 4 * lg;
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int s = 0; s < 2; ++s)
                dst[r][s] = *reinterpret_cast<const f4_v*>(C + (row0 + r) * g.ldc + n0 + 128 * wn + 64 * s + 4 * c);
    };
    if (C) {
        cload(0, cv[0]);
        cload(1, cv[1]);
    }
#pragma unroll
    for (int a = 0; a < 8; ++a) {
        const int64_t row0 = m0 + 128 * wm + 16 * a + 4 * lg;
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                f4_v v;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    v[b] = acc[a][4 * s + b][r];
                    if (g.alpha != 1.0) v[b] = alpha * v[b];
                    if (C) v[b] = v[b] + beta * cv[a & 1][r][s][b];
                }
                *reinterpret_cast<f4_v*>(D + (row0 + r) * g.ldd + n0 + 128 * wn + 64 * s + 4 * c) = v;
            }
        if (C && a + 2 < 8) cload(a + 2, cv[a & 1]);
    }
}

}  // namespace

// Whether gemm_big_f32 takes this problem (see the file comment).
bool gemm_big_f32_fits(bool ta, bool tb, const GemmArgs& g) {
    auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    const bool batch_ok =
        g.batch == 1 || (g.sA % 4 == 0 && g.sB % 4 == 0 && g.sD % 4 == 0 && (!g.C || g.sC % 4 == 0));
    return !ta && !tb && batch_ok && g.M % kBigM == 0 && g.N % kBigN == 0 && g.K >= kBigK && g.K % kBigK == 0 &&
           g.lda % 4 == 0 && g.ldb % 4 == 0 && g.ldd % 4 == 0 && al(g.A) && al(g.B) && al(g.D) &&
           (!g.C || (al(g.C) && g.ldc % 4 == 0));
}

int gemm_big_f32_launch(GemmArgs& g, hipStream_t st) {
    g.tiles_m = g.M / kBigM;
    g.tiles_n = g.N / kBigN;
    const int64_t tiles = g.tiles_m * g.tiles_n * g.batch;
    hipLaunchKernelGGL(gemm_big_f32_kernel, dim3((unsigned)tiles), dim3(kBigThreads), 0, st, g);
    return check_launch("tt_gemm");
}

}  // namespace tt
