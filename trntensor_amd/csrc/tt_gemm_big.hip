// fp32 GEMM on 256 x 256 tiles with both operands staged through LDS
// (tt_gemm, TT_F32, both operands not transposed, whole tiles, K a multiple
// of 32, 16-byte aligned; the dispatcher takes it in whole rounds of one
// tile per CU).
//
// Eight waves of 64 x 128 (4 x 8 blocks of v_mfma_f32_16x16x4f32, 128 fp32
// accumulators per lane), two waves per SIMD, one workgroup per CU (144 KiB
// of LDS). Stages of 32 k, double-buffered, one barrier per stage. The next
// stage's global loads are spread over the first half of the stage's first
// 16-k chunk (one per 8 MFMAs; one per 16: -0.5 points, per 4 or all first:
// -0.4) and its LDS stores over the second chunk (one per 16 MFMAs, into the
// other buffer, which the previous barrier released). Measured against the direct-B kernel's
// 64 x 256 tiles at four workgroups per CU (same box, alternating): 4096^3
// fp32 0.968 against 0.996 ms; the template's other shape, 128 x 256 tiles
// with 16-k stages at two workgroups per CU, 0.996 ms; B read one MFMA step
// ahead, 0.977 ms. LDS pitches (floats of padding per A row / B k-row, 4096^3
// fraction of the fp32 peak, one box): 8 / 0 0.914, 4 / 0 0.908, 12 / 0
// 0.908, 4 / 4 0.900, 4 / 16 0.909, 8 / 8 0.892, unpadded A 0.882; A pieces
// XOR-swizzled instead of padded 0.898.
//
// Fragments (the layout of gemm_directb_kernel, whose results this kernel
// reproduces bitwise): chunk h of a stage is 16 k; MFMA step p of chunk h
// gives lane group g = lane / 16 the k index 16 h + 4 g + p. A lane's A
// operand for row block a is row 16 a + lane % 16, four consecutive k (one
// 16-byte LDS read feeds steps 0..3); its B operand piece for step p is four
// consecutive columns 4 (lane % 16) .. + 3 of one k-row (one 16-byte read),
// one column for each of the four MFMA column blocks of a 64-column set.
#include <type_traits>

#include "tt_gemm.hpp"

namespace tt {

namespace {

constexpr int kBigN = 256;
typedef float f4_v __attribute__((ext_vector_type(4)));

template <int TM, int BK>
struct BigCfg {
    static constexpr int NW = TM / 64 * 2;  // waves
    static constexpr int T = 64 * NW;       // threads
    static constexpr int CH = BK / 16;      // 16-k chunks per stage
    static constexpr int AP = BK + 8;       // floats per A row in LDS
    static constexpr int BP = kBigN;        // floats per B k-row in LDS (unpadded)
    static constexpr int AE = TM * AP;      // A floats per stage buffer
    static constexpr int BE = BK * BP;      // B floats per stage buffer
    static constexpr int LA = BK / 4;       // threads per A row (16 bytes each)
    static constexpr int RA = TM * LA / T;  // A loads per thread per stage
    static constexpr int RB = BK * 64 / T;  // B loads per thread per stage (64 threads per k-row)
    static constexpr int NL = RA + RB;
    static constexpr int WG_PER_CU = TM == 256 ? 1 : 2;
    static_assert(RA >= 1 && RB >= 1 && TM * LA % T == 0 && BK * 64 % T == 0, "staging split");
};

constexpr int big_threads(int tm) { return tm / 64 * 2 * 64; }
constexpr int big_wgs_per_cu(int tm) { return tm == 256 ? 1 : 2; }

template <int TM, int BK>
__global__ __launch_bounds__(big_threads(TM), big_wgs_per_cu(TM)) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_big_f32_kernel(GemmArgs g) {
    typedef BigCfg<TM, BK> C_;
    constexpr int T = C_::T, AP = C_::AP, BP = C_::BP, AE = C_::AE, BE = C_::BE, LA = C_::LA, RA = C_::RA, RB = C_::RB,
                  NL = C_::NL, CH = C_::CH;
    constexpr int MC = 4 * 8 * 4;  // MFMAs per wave per chunk
    __shared__ __attribute__((aligned(16))) float lds[2 * (AE + BE)];

    // Rows of tiles in groups of four, each group column-major: an XCD's
    // contiguous range of tiles is a block four tile rows high.
    const int64_t tiles = g.tiles_m * g.tiles_n;
    const int64_t id = xcd_remap(blockIdx.x, tiles);
    const int64_t grp = id / (4 * g.tiles_n);
    const int64_t gm = min((int64_t)4, g.tiles_m - grp * 4);
    const int64_t rr = id - grp * 4 * g.tiles_n;
    const int64_t tn = rr / gm, tm = grp * 4 + rr % gm;
    const int64_t m0 = tm * TM, n0 = tn * kBigN;
    const float* A = static_cast<const float*>(g.A);
    const float* B = static_cast<const float*>(g.B);

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int w = t >> 6;
    const int lg = lane >> 4, c = lane & 15;
    const int wm = w >> 1, wn = w & 1;  // rows 64 wm .., columns 128 wn ..

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

    f4_v acc[4][8];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[a][j] = f4_v{0, 0, 0, 0};

    auto chunk = [&](int buf, int h) __attribute__((always_inline)) {
        const float* as = lds + buf * (AE + BE);
        const float* bs = as + AE;
        f4_v fa[4], fb[2][4];
#pragma unroll
        for (int a = 0; a < 4; ++a)
            fa[a] = *reinterpret_cast<const f4_v*>(as + (64 * wm + 16 * a + c) * AP + 16 * h + 4 * lg);
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int p = 0; p < 4; ++p)
                fb[s][p] = *reinterpret_cast<const f4_v*>(bs + (16 * h + 4 * lg + p) * BP + 128 * wn + 64 * s + 4 * c);
#pragma unroll
        for (int p = 0; p < 4; ++p)
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int s = 0; s < 2; ++s)
#pragma unroll
                    for (int b = 0; b < 4; ++b)
                        acc[a][4 * s + b] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[a][p], fb[s][p][b],
                                                                                 acc[a][4 * s + b], 0, 0, 0);
    };
    // Scheduling of a stage's loads (mask 0x020) and stores (0x200) among
    // MFMAs (0x008).
    auto spread_loads = [&](auto per) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, decltype(per)::value, 0);
        }
    };
    auto spread_stores = [&](auto per) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, decltype(per)::value, 0);
            __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
        }
    };
    constexpr std::integral_constant<int, MC / 2 / NL> HALF{};
    constexpr std::integral_constant<int, MC / NL> FULL{};

    const int64_t nk = g.K / BK;
    gload(0);
    sstore(0);
    __syncthreads();
    int64_t st = 0;
    for (; st + 1 < nk; ++st) {
        const int buf = (int)(st & 1);
        gload((st + 1) * BK);
        if constexpr (CH == 1) {
            chunk(buf, 0);
            sstore(buf ^ 1);
            spread_loads(HALF);
            spread_stores(HALF);
            __builtin_amdgcn_sched_barrier(0);
        } else {
            chunk(buf, 0);
            spread_loads(HALF);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int h = 1; h + 1 < CH; ++h) chunk(buf, h);
            __builtin_amdgcn_sched_barrier(0);
            chunk(buf, CH - 1);
            sstore(buf ^ 1);
            spread_stores(FULL);
            __builtin_amdgcn_sched_barrier(0);
        }
        __syncthreads();
    }
#pragma unroll
    for (int h = 0; h < CH; ++h) chunk((int)(st & 1), h);

    // D = alpha acc (+ beta C): acc[a][4 s + b][r] is row m0 + 64 wm + 16 a +
    // 4 lg + r, column n0 + 128 wn + 64 s + 4 c + b; a lane's four columns
    // are one 16-byte piece. Each row block's C pieces are loaded before its
    // stores (D may alias C).
    float* D = static_cast<float*>(g.D);
    const float* C = static_cast<const float*>(g.C);
    const float alpha = (float)g.alpha, beta = (float)g.beta;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
        const int64_t row0 = m0 + 64 * wm + 16 * a + 4 * lg;
        f4_v cv[4][2];
        if (C) {
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int s = 0; s < 2; ++s)
                    cv[r][s] = *reinterpret_cast<const f4_v*>(C + (row0 + r) * g.ldc + n0 + 128 * wn + 64 * s + 4 * c);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                f4_v v;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    v[b] = acc[a][4 * s + b][r];
                    if (g.alpha != 1.0) v[b] = alpha * v[b];
                    if (C) v[b] = v[b] + beta * cv[r][s][b];
                }
                *reinterpret_cast<f4_v*>(D + (row0 + r) * g.ldd + n0 + 128 * wn + 64 * s + 4 * c) = v;
            }
    }
}

}  // namespace

constexpr int kBigTM = 256, kBigBK = 32;

// Whether gemm_big_f32 takes this problem (see the file comment).
bool gemm_big_f32_fits(bool ta, bool tb, const GemmArgs& g) {
    auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    return !ta && !tb && g.batch == 1 && g.M % kBigTM == 0 && g.N % kBigN == 0 && g.K >= kBigBK &&
           g.K % kBigBK == 0 && g.lda % 4 == 0 && g.ldb % 4 == 0 && g.ldd % 4 == 0 && al(g.A) && al(g.B) &&
           al(g.D) && (!g.C || (al(g.C) && g.ldc % 4 == 0));
}

int gemm_big_f32_launch(GemmArgs& g, hipStream_t st) {
    g.tiles_m = g.M / kBigTM;
    g.tiles_n = g.N / kBigN;
    const int64_t tiles = g.tiles_m * g.tiles_n;
    hipLaunchKernelGGL((gemm_big_f32_kernel<kBigTM, kBigBK>), dim3((unsigned)tiles),
                       dim3(BigCfg<kBigTM, kBigBK>::T), 0, st, g);
    return check_launch("tt_gemm");
}

}  // namespace tt
