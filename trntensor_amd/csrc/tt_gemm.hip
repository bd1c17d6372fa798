// MFMA GEMM core for gfx950: batched, strided, transposed operands in place,
// fused alpha/beta epilogue. fp64 on v_mfma_f64_16x16x4f64, fp32 on
// v_mfma_f32_16x16x4f32.
//
// Workgroup: 256 threads = 4 wavefronts, output tile BM x BN, each wavefront
// a 64x64 sub-tile (4 x 4 MFMA blocks, 64 accumulators per lane).
// K advances in stages of 16 through two LDS buffers: while the MFMAs consume
// one stage, the next stage's global loads are in flight in registers and are
// written to the other buffer afterwards (one barrier per stage).
//
// LDS layouts follow the operand's contiguous direction so every global load
// and LDS store is a 16-byte vector:
//   k-contiguous operand   -> [row][k],  row pitch 16 + 16 B of padding
//   row-contiguous operand -> [k][row],  k-row pitch ROWS + 16 B of padding
// Inside a 16-wide stage, MFMA step s (0..3) gives lane-group g = lane / 16
// the k index 4 g + s for both operands, so a lane's four k values are
// adjacent in the [row][k] layout and one 32-byte read feeds four MFMAs.
#include <string.h>
#include <type_traits>

#include "tt_gemm.hpp"

namespace tt {

constexpr int kBK = 16;
constexpr int kThreads = 256;


// One operand's ROWS x BK stage: global -> registers -> LDS, plus fragment reads.
// KC: element (row, k) at p[row * ld + k]; otherwise at p[k * ld + row].
// Each thread stages E = ROWS * BK / 256 elements as NC 16-byte pieces:
//   KC: row t / (BK / E), one contiguous chunk from k = (t % (BK / E)) E;
//   RC: 16 threads per k-row, k-rows t / 16 + 16 j; within a k-row a
//       thread's pieces are (t % 16) + 16 c, so every instruction covers 256
//       contiguous bytes of the k-row (coalesced loads, conflict-free stores).
// RC k-rows are padded by 4 elements: the four lane groups of a fragment read
// (k-rows 4 g + s) then land on disjoint LDS banks.
template <typename T, int ROWS, bool KC, bool VEC, int BK, bool NT = false>
struct Stage {
    static constexpr int V = Vec16<T>::n;
    static constexpr int E = ROWS * BK / kThreads;
    static constexpr int NC = E / V;  // 16-byte pieces per thread
    static constexpr int NCR = KC ? NC : ROWS / (16 * V);  // RC: pieces per k-row and thread
    static constexpr int PAD = 16 / sizeof(T);
    static constexpr int PITCH = KC ? (BK + PAD) : (ROWS + 4);
    static constexpr int ELEMS = KC ? ROWS * PITCH : BK * PITCH;
    static_assert(BK % 16 == 0 && E % V == 0 && (KC ? BK % E == 0 : (NC % NCR == 0 && NCR >= 1)), "stage split");
    typedef typename Vec16<T>::type vec_t;

    vec_t reg[NC];

    __device__ __forceinline__ static void place(int& row, int& k) {
        const int t = threadIdx.x;
        if (KC) {
            row = t / (BK / E);
            k = (t % (BK / E)) * E;
        } else {
            k = t / 16;
            row = (t % 16) * V;
        }
    }
    // Offsets of piece c relative to piece 0: along the rows and along k.
    __device__ __forceinline__ static constexpr int prow(int c) { return KC ? 0 : (c % NCR) * 16 * V; }
    __device__ __forceinline__ static constexpr int pk(int c) { return KC ? c * V : (c / NCR) * 16; }

    // FAST (interior stage: tile inside the matrix, 16-byte aligned):
    // unconditional vector loads. Otherwise (edge tiles, the K tail, unaligned
    // operands) piece by piece: a piece wholly inside is one vector load (VEC),
    // one wholly outside is zero without a load, and only a piece straddling
    // the edge is loaded element-wise from clamped addresses. Measured against
    // element-wise loads for every piece (fp32, fp64 TFLOP/s): 2000 x 3000 x
    // 2000 106.5 and 57.3 against 77.0 and 51.0; 4000^3 TN 123.4 and 58.4
    // against 95.7 and 53.6; aligned shapes unchanged.
    template <bool FAST>
    __device__ __forceinline__ void load(const T* __restrict__ p, int64_t ld, int64_t row0, int64_t rows,
                                         int64_t k0, int64_t kdim) {
        int r, k;
        place(r, k);
        if (FAST) {
            const T* src = KC ? p + (row0 + r) * ld + (k0 + k) : p + (k0 + k) * ld + (row0 + r);
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const vec_t* q = reinterpret_cast<const vec_t*>(KC ? src + pk(c) : src + pk(c) * ld + prow(c));
                reg[c] = NT ? __builtin_nontemporal_load(q) : *q;
            }
        } else {
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const int64_t pr = row0 + r + prow(c);
                const int64_t pkk = k0 + k + pk(c);
                const bool inside = KC ? (pr < rows && pkk + V <= kdim) : (pkk < kdim && pr + V <= rows);
                const bool outside = pr >= rows || pkk >= kdim;
                if (VEC && inside) {
                    reg[c] = *reinterpret_cast<const vec_t*>(KC ? p + pr * ld + pkk : p + pkk * ld + pr);
                } else if (outside) {
#pragma unroll
                    for (int e = 0; e < V; ++e) reg[c][e] = T(0);
                } else {
#pragma unroll
                    for (int e = 0; e < V; ++e) {
                        const int64_t gr = pr + (KC ? 0 : e);
                        const int64_t gk = pkk + (KC ? e : 0);
                        const bool ok = gr < rows && gk < kdim;
                        const T x = *(ok ? (KC ? p + gr * ld + gk : p + gk * ld + gr) : p);
                        reg[c][e] = ok ? x : T(0);
                    }
                }
            }
        }
    }

    __device__ __forceinline__ void store(T* s) const {
        int r, k;
        place(r, k);
        T* dst = KC ? (s + r * PITCH + k) : (s + k * PITCH + r);
#pragma unroll
        for (int c = 0; c < NC; ++c)
            *reinterpret_cast<vec_t*>(KC ? dst + pk(c) : dst + pk(c) * PITCH + prow(c)) = reg[c];
    }

    // The four k values (MFMA steps 0..3 of 16-k pass kk) this lane feeds for
    // the 16-row block at rb.
    __device__ __forceinline__ static void frag(const T* s, int rb, int lane, int kk, T out[4]) {
        const int r = rb + (lane & 15);
        const int g = lane >> 4;
        if (KC) {
            typedef typename VecN<T, 4>::type v4_t;
            const v4_t x = *reinterpret_cast<const v4_t*>(s + r * PITCH + 16 * kk + 4 * g);
#pragma unroll
            for (int st = 0; st < 4; ++st) out[st] = x[st];
        } else {
#pragma unroll
            for (int st = 0; st < 4; ++st) out[st] = s[(16 * kk + 4 * g + st) * PITCH + r];
        }
    }
};

template <typename T, int BM, int BN, int FM, int FN, bool TA, bool TB, bool VEC, bool DOT, int NBUF, int BK,
          bool PRIO>
__global__ __launch_bounds__(kThreads) void gemm_kernel(GemmArgs g) {
    typedef Mfma<T> MF;
    typedef typename MF::acc_t acc_t;
    // A rows are m: k-contiguous unless transposed. B rows are n: k-contiguous iff transposed.
    typedef Stage<T, BM, !TA, VEC, BK> SA;
    // The single-buffer small-M tile reads B once (one tile row; the launcher
    // sends a batch-broadcast B elsewhere), so B's loads are non-temporal and
    // leave the L2 to A, which every workgroup re-reads: AO->MO half
    // transform 0.909-0.920 -> 0.899-0.900 ms, results bitwise equal.
    // Non-temporal loads of A as well, or on tiles that re-read B, cost 7-18%.
    typedef Stage<T, BN, TB, VEC, BK, NBUF == 1 && PRIO> SB;
    // Each wavefront owns an (16 FM) x (16 FN) sub-tile: FM x FN MFMA blocks.
    constexpr int WM = 16 * FM, WN = 16 * FN;
    constexpr int WAVES_N = BN / WN;
    static_assert((BM / WM) * WAVES_N == 4, "four wavefront tiles per workgroup");

    static_assert(NBUF == 1 || NBUF == 2, "stage buffers");
    __shared__ __attribute__((aligned(16))) T lds[NBUF * (SA::ELEMS + SB::ELEMS)];
    // Stage buffers: A0 (A1) B0 (B1).
    auto bufA = [&](int b) -> T* { return lds + b * SA::ELEMS; };
    auto bufB = [&](int b) -> T* { return lds + NBUF * SA::ELEMS + b * SB::ELEMS; };

    const int64_t tiles = g.tiles_m * g.tiles_n;
    const int64_t total = tiles * g.batch;
    const int64_t id = xcd_remap(blockIdx.x, total);
    const int64_t bat = id / tiles;
    int64_t t = id - bat * tiles;
    // Grouped order: 8 tile-rows sweep each tile-column, so concurrently
    // running workgroups share A panels and B panels.
    constexpr int64_t GROUP = 8;
    const int64_t grp = t / (GROUP * g.tiles_n);
    const int64_t first_m = grp * GROUP;
    const int64_t gsize = min(g.tiles_m - first_m, GROUP);
    const int64_t rem = t - grp * GROUP * g.tiles_n;
    const int64_t tm = first_m + rem % gsize;
    const int64_t tn = rem / gsize;
    const int64_t m0 = tm * BM;
    const int64_t n0 = tn * BN;

    const T* A = static_cast<const T*>(g.A) + bat * g.sA;
    const T* B = static_cast<const T*>(g.B) + bat * g.sB;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm0 = (wave / WAVES_N) * WM;
    const int wn0 = (wave % WAVES_N) * WN;

    acc_t acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = acc_t{0, 0, 0, 0};

    SA sa;
    SB sb;
    const int64_t nk = (g.K + BK - 1) / BK;
    // Stages 0 .. nfull-1 are interior for both operands.
    const int64_t nfull = (VEC && m0 + BM <= g.M && n0 + BN <= g.N) ? g.K / BK : 0;
    // The lambdas below are always inlined: left as calls (which the inliner
    // chose for 64-deep stages), they capture acc by reference and the
    // accumulators go to scratch memory.
    auto load = [&](int64_t k0, auto fast) __attribute__((always_inline)) {
        constexpr bool F = decltype(fast)::value;
        sa.template load<F>(A, g.lda, m0, g.M, k0, g.K);
        sb.template load<F>(B, g.ldb, n0, g.N, k0, g.K);
    };
    auto compute = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int kk = 0; kk < BK / 16; ++kk) {
            T fa[FM][4], fb[FN][4];
#pragma unroll
            for (int i = 0; i < FM; ++i) SA::frag(bufA(buf), wm0 + 16 * i, lane, kk, fa[i]);
#pragma unroll
            for (int j = 0; j < FN; ++j) SB::frag(bufB(buf), wn0 + 16 * j, lane, kk, fb[j]);
#pragma unroll
            for (int st = 0; st < 4; ++st)
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j) acc[i][j] = MF::mma(fa[i][st], fb[j][st], acc[i][j]);
        }
    };
    if (nk > 0) {
        if (nfull > 0) load(0, std::true_type{});
        else load(0, std::false_type{});
        sa.store(bufA(0));
        sb.store(bufB(0));
    }
    __syncthreads();

    // The scheduling barrier keeps the prefetch's LDS stores (and the wait for
    // its global loads) behind this stage's MFMAs. With two buffers the next
    // stage goes to the other buffer (one barrier per stage); with one, it
    // replaces the current stage after a second barrier (half the LDS, so
    // more workgroups per CU).
    auto next = [&](int64_t kt) -> int { return NBUF == 2 ? (int)((kt & 1) ^ 1) : 0; };
    auto cur = [&](int64_t kt) -> int { return NBUF == 2 ? (int)(kt & 1) : 0; };
    int64_t kt = 0;
    // PRIO (fp64): the wave issuing a stage's MFMAs runs at raised priority
    // for the burst, so co-resident waves in their load/store phase do not
    // delay the MFMA stream.
    auto mfma_stage = [&](int b) __attribute__((always_inline)) {
        if (PRIO && sizeof(T) == 8) __builtin_amdgcn_s_setprio(1);
        compute(b);
        if (PRIO && sizeof(T) == 8) __builtin_amdgcn_s_setprio(0);
    };
    for (; kt + 1 < nfull; ++kt) {
        load((kt + 1) * BK, std::true_type{});
        mfma_stage(cur(kt));
        __builtin_amdgcn_sched_barrier(0);
        if (NBUF == 1) __syncthreads();
        sa.store(bufA(next(kt)));
        sb.store(bufB(next(kt)));
        __syncthreads();
    }
    for (; kt < nk; ++kt) {
        const bool more = kt + 1 < nk;
        if (more) load((kt + 1) * BK, std::false_type{});
        mfma_stage(cur(kt));
        __builtin_amdgcn_sched_barrier(0);
        if (NBUF == 1) __syncthreads();
        if (more) {
            sa.store(bufA(next(kt)));
            sb.store(bufB(next(kt)));
        }
        __syncthreads();
    }

    const int col_l = lane & 15;
    const int lgrp = lane >> 4;
    if (DOT) {
        // Dot epilogue: sum of D .* E over this tile, one double per workgroup.
        __shared__ double red[4];
        const T* E1 = static_cast<const T*>(g.E1) + bat * g.e1s[4];
        const T* E2 = g.E2 ? static_cast<const T*>(g.E2) + bat * g.e2s[4] : nullptr;
        double sum = 0.0;
        if constexpr (NBUF == 2) {
            // Each 16x16 block's eight E loads (branch-free: rows and columns
            // outside the matrix read element (0, 0)) go out together before
            // its sums, which keep the order below. Loaded under the
            // per-element bounds branches, every load waited out a full
            // latency before its sum: 128 waits per lane at 128 x 128, and
            // config 5's greedy path took 69.4 ms against 68.4 ms this way
            // (results bitwise equal). The single-buffer small-M tile keeps
            // the form below: the batches would cost it a wave per SIMD.
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int64_t col = n0 + wn0 + 16 * j + col_l;
                const bool cok = col < g.N;
                const uint32_t nh = fdiv((uint32_t)(cok ? col : 0), g.ndiv);
                const uint32_t nl = (uint32_t)(cok ? col : 0) - nh * g.ndiv.d;
                const int64_t o1n = nh * g.e1s[2] + nl * g.e1s[3];
                const int64_t o2n = nh * g.e2s[2] + nl * g.e2s[3];
#pragma unroll
                for (int i = 0; i < FM; ++i) {
                    T e1v[4], e2v[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int64_t row = m0 + wm0 + 16 * i + MF::row(lgrp, r);
                        const bool ok = cok && row < g.M;
                        const uint32_t mh = fdiv((uint32_t)(ok ? row : 0), g.mdiv);
                        const uint32_t ml = (uint32_t)(ok ? row : 0) - mh * g.mdiv.d;
                        e1v[r] = E1[ok ? mh * g.e1s[0] + ml * g.e1s[1] + o1n : 0];
                        if (E2) e2v[r] = E2[ok ? mh * g.e2s[0] + ml * g.e2s[1] + o2n : 0];
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int64_t row = m0 + wm0 + 16 * i + MF::row(lgrp, r);
                        if (cok && row < g.M) {
                            T e = e1v[r];
                            if (E2) e = e * e2v[r];
                            sum += (double)(acc[i][j][r] * e);
                        }
                    }
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int64_t col = n0 + wn0 + 16 * j + col_l;
                const uint32_t nh = fdiv((uint32_t)col, g.ndiv);
                const uint32_t nl = (uint32_t)col - nh * g.ndiv.d;
                const int64_t o1n = nh * g.e1s[2] + nl * g.e1s[3];
                const int64_t o2n = nh * g.e2s[2] + nl * g.e2s[3];
#pragma unroll
                for (int i = 0; i < FM; ++i) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int64_t row = m0 + wm0 + 16 * i + MF::row(lgrp, r);
                        if (row < g.M && col < g.N) {
                            const uint32_t mh = fdiv((uint32_t)row, g.mdiv);
                            const uint32_t ml = (uint32_t)row - mh * g.mdiv.d;
                            T e = E1[mh * g.e1s[0] + ml * g.e1s[1] + o1n];
                            if (E2) e = e * E2[mh * g.e2s[0] + ml * g.e2s[1] + o2n];
                            sum += (double)(acc[i][j][r] * e);
                        }
                    }
                }
            }
        }
        const double tot = block256_sum(sum, red);
        if (threadIdx.x == 0) g.partial[blockIdx.x] = tot;
        return;
    }

    // Store epilogue: D = alpha * acc (+ beta * C), masked at the matrix edge.
    // D may alias C, so the compiler cannot move a load of C past a store of
    // D: loaded element by element, every element would wait out a full
    // memory latency before its store. Each 16-row block's C values are
    // therefore loaded (from clamped addresses, branch-free) before any of
    // its stores, which keeps FN * 4 loads in flight together.
    const T alpha = (T)g.alpha;
    const T beta = (T)g.beta;
    const T* C = g.C ? static_cast<const T*>(g.C) + bat * g.sC : nullptr;
    T* D = static_cast<T*>(g.D) + bat * g.sD;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        T cv[FN][4];
        if (C) {
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int64_t col = n0 + wn0 + 16 * j + col_l;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t row = m0 + wm0 + 16 * i + MF::row(lgrp, r);
                    const bool ok = row < g.M && col < g.N;
                    const T c = C[ok ? row * g.ldc + col : 0];
                    cv[j][r] = ok ? c : T(0);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int64_t col = n0 + wn0 + 16 * j + col_l;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = m0 + wm0 + 16 * i + MF::row(lgrp, r);
                if (row < g.M && col < g.N) {
                    T v = acc[i][j][r];
                    if (g.alpha != 1.0) v = alpha * v;
                    if (C) v = v + beta * cv[j][r];
                    D[row * g.ldd + col] = v;
                }
            }
        }
    }
}

// Store epilogue of the direct-B kernels: D = alpha * acc (+ beta * C) for
// the 64 x BN tile at rows m0.., column tile tn of batch entry bat.
// acc[a][b][r] is row m0 + 16 a + MF::row(lg, r), column col + b. When D's
// (and C's) rows start 16-byte aligned (checked below), a lane's NB columns
// are one 16-byte piece. The lane indices are formed again here rather than
// held through the K loop.
// PLAIN: no C, D's rows 16-byte aligned and the tile inside N (the caller
// checked), so every row is one unconditional 16-byte store per lane.
template <typename T, bool FULLM, bool PLAIN = false>
__device__ __forceinline__ void directb_store(const GemmArgs& g, typename Mfma<T>::acc_t (&acc)[4][16 / sizeof(T)],
                                              int64_t bat, int64_t m0, int64_t tn) {
    typedef Mfma<T> MF;
    constexpr int NB = 16 / sizeof(T);
    constexpr int BN = 64 * NB;
    typedef typename VecN<T, 16 / sizeof(T)>::type v16_t;
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int lg = (tid & 63) >> 4;
    const int64_t col = tn * BN + (tid >> 6) * (16 * NB) + NB * (tid & 15);
    const T alpha = (T)g.alpha;
    const T beta = (T)g.beta;
    T* D = static_cast<T*>(g.D) + bat * g.sD;
    if constexpr (PLAIN) {
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                v16_t v;
#pragma unroll
                for (int b = 0; b < NB; ++b) v[b] = g.alpha != 1.0 ? alpha * acc[a][b][r] : acc[a][b][r];
                *reinterpret_cast<v16_t*>(D + (m0 + 16 * a + MF::row(lg, r)) * g.ldd + col) = v;
            }
        return;
    }
    const T* C = g.C ? static_cast<const T*>(g.C) + bat * g.sC : nullptr;
    const bool vecd = ((reinterpret_cast<uintptr_t>(D) | (uintptr_t)(g.ldd * sizeof(T))) & 15) == 0 &&
                      (!C || ((reinterpret_cast<uintptr_t>(C) | (uintptr_t)(g.ldc * sizeof(T))) & 15) == 0);
    const bool colok = col < g.N;  // N is a multiple of NB: all NB columns or none
    if (C && vecd) {
        // A lane's NB columns of a row are one 16-byte piece of C and of D.
        // The C pieces of two row blocks (eight rows) go out together before
        // their stores: two memory round trips per tile instead of four, and
        // one load per row instead of NB. D may alias C exactly: every row's
        // C piece is loaded before that row's store. Same box, alternating,
        // bitwise equal: 64 x 512^3 with alpha/beta and C 0.1362-0.1366
        // against 0.1429-0.1432 ms fp32, 0.2615-0.2618 against 0.2646-0.2661
        // ms fp64; 4096^3 fp32 0.993 against 0.999 ms.
#pragma unroll
        for (int a2 = 0; a2 < 4; a2 += 2) {
            v16_t cv[2][4];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t row = m0 + 16 * (a2 + h) + MF::row(lg, r);
                    const bool ok = (FULLM || row < g.M) && colok;
                    const v16_t x = *reinterpret_cast<const v16_t*>(C + (ok ? row * g.ldc + col : 0));
#pragma unroll
                    for (int b = 0; b < NB; ++b) cv[h][r][b] = ok ? x[b] : T(0);
                }
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t row = m0 + 16 * (a2 + h) + MF::row(lg, r);
                    if ((!FULLM && row >= g.M) || !colok) continue;
                    v16_t v;
#pragma unroll
                    for (int b = 0; b < NB; ++b) {
                        v[b] = acc[a2 + h][b][r];
                        if (g.alpha != 1.0) v[b] = alpha * v[b];
                        v[b] = v[b] + beta * cv[h][r][b];
                    }
                    *reinterpret_cast<v16_t*>(D + row * g.ldd + col) = v;
                }
        }
        return;
    }
#pragma unroll
    for (int a = 0; a < 4; ++a) {
        T cv[4][NB];
        if (C) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = m0 + 16 * a + MF::row(lg, r);
                const bool ok = (FULLM || row < g.M) && colok;
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    const T x = C[ok ? row * g.ldc + col + b : 0];
                    cv[r][b] = ok ? x : T(0);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t row = m0 + 16 * a + MF::row(lg, r);
            if ((!FULLM && row >= g.M) || !colok) continue;
            v16_t v;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                v[b] = acc[a][b][r];
                if (g.alpha != 1.0) v[b] = alpha * v[b];
                if (C) v[b] = v[b] + beta * cv[r][b];
            }
            T* d = D + row * g.ldd + col;
            if (vecd) {
                *reinterpret_cast<v16_t*>(d) = v;
            } else {
#pragma unroll
                for (int b = 0; b < NB; ++b) d[b] = v[b];
            }
        }
    }
}

// GEMM (or dot epilogue, DOT): fp64 on 64 x 128 tiles, fp32 on 64 x 256 tiles,
// four waves each; N a multiple of NB (below), the last column tile may be
// partial (not with DOT).
// A (either layout) is staged through LDS one 64-row slab per workgroup,
// double-buffered, one barrier per 16-k stage; rows from M up and k from K up
// read as zero. B goes from memory straight into the MFMA operand registers:
// wave w owns all 64 rows and 16 NB columns (NB = 16 bytes / element: 2 for
// fp64, 4 for fp32), and lane (g, c) feeds MFMA block b (0 .. NB - 1) with
// column n0 + 16 NB w + NB c + b, so one 16-byte load per k-row gives it every
// block's operand and B never passes through LDS. With B k-contiguous (TB)
// the lane's 16-byte piece is NB consecutive k of one column instead, and its
// four pieces cover its NB columns over the stage's 4 k. MFMA step s of stage t gives
// lane group g the k index 16 t + 4 g + s, the order of gemm_kernel, whose
// results it reproduces bitwise. 118-128 VGPRs: four waves per SIMD. NT: B is
// read once (M <= 64, e.g. the AO->MO half transform), so its loads bypass the
// caches. AO->MO half transform (64 x 786432 x 512) against the LDS-staged
// small-M tile: 0.877-0.883 against 0.893-0.900 ms on one box and 0.885-0.886
// against 0.913-0.915 ms on another, alternating; M < 64 (48 x 65536 x 256,
// four batches) measured the same.
template <typename T, bool FULLM, bool TA, bool TB, bool NT, bool DOT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) void gemm_directb_kernel(GemmArgs g) {
    typedef Mfma<T> MF;
    typedef typename MF::acc_t acc_t;
    constexpr int NB = 16 / sizeof(T);  // MFMA column blocks per wave: one 16-byte B piece per lane
    constexpr int BN = 64 * NB;         // tile columns: 128 (fp64), 256 (fp32)
    constexpr int SPL = TB ? 16 / sizeof(T) : 1;  // MFMA steps one B load feeds (TB: k-contiguous piece)
    typedef typename VecN<T, 16 / sizeof(T)>::type v16_t;
    typedef Stage<T, 64, !TA, true, kBK> SA;  // A: a 64-row slab, [k][m] (TA) or [m][k] in LDS
    __shared__ __attribute__((aligned(16))) T lds[2 * SA::ELEMS];

    // Tile order: the 64-row slabs of one column tile are adjacent (they
    // share its B panel in L2). With more than 64 row tiles, the rows go in
    // groups of 16 slabs that sweep every column tile before the next group,
    // so a group's A slabs stay cached instead of A streaming from HBM once
    // per column tile. Config 5's fused GEMM (2500 x 128 tiles, A 1 GB):
    // 60.36 and 60.01 against 60.92 and 61.10 ms on one box (groups of 32:
    // 60.28 and 60.31 ms; of 64: 60.83 and 60.98 ms).
    const int64_t tiles = g.tiles_m * g.tiles_n;
    const int64_t id = xcd_remap(blockIdx.x, tiles * g.batch);
    const int64_t bat = id / tiles;
    const int64_t rem = id - bat * tiles;
    constexpr int64_t kRowGroup = 16;
    int64_t tn, tm;
    if (g.tiles_m > 4 * kRowGroup) {
        const int64_t grp = rem / (kRowGroup * g.tiles_n);
        const int64_t gm = min(kRowGroup, g.tiles_m - grp * kRowGroup);  // row tiles in this group
        const int64_t r = rem - grp * kRowGroup * g.tiles_n;
        tn = r / gm;
        tm = grp * kRowGroup + r % gm;
    } else {
        tn = rem / g.tiles_m;
        tm = rem - tn * g.tiles_m;
    }
    const int64_t m0 = tm * 64;
    const T* A = static_cast<const T*>(g.A) + bat * g.sA;
    const int64_t nk = (g.K + kBK - 1) / kBK;
    const int64_t nfull = g.K / kBK;

    acc_t acc[4][NB];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[a][b] = acc_t{0, 0, 0, 0};
    if (nk > 0) {
        const int lane = threadIdx.x & 63;
        const int lg = lane >> 4;
        const int c = lane & 15;
        // The lane's first column, clamped into the matrix: in a last, partial
        // column tile the lanes past N read column N - NB instead, and their
        // results are never stored (a column of D depends on that column of B
        // only).
        const int64_t col0 = min(tn * BN + (threadIdx.x >> 6) * (16 * NB) + NB * c, g.N - NB);
        // B row-major: piece p (0..3) is k-row 16 t + 4 g + p, all NB columns.
        // B k-contiguous: piece p is column col0 + p % NB, k 16 t + 4 g +
        // SPL (p / NB) .. + SPL - 1 (MFMA steps SPL (p / NB) ..).
        const T* B = TB ? static_cast<const T*>(g.B) + bat * g.sB + col0 * g.ldb + 4 * lg
                        : static_cast<const T*>(g.B) + bat * g.sB + col0 + (int64_t)(4 * lg) * g.ldb;
        auto bptr = [&](int64_t t, int p) __attribute__((always_inline)) -> const T* {
            return TB ? B + (int64_t)(p % NB) * g.ldb + 16 * t + SPL * (p / NB) : B + (16 * t + p) * g.ldb;
        };
        SA sa;
        v16_t rb[4];  // B pieces of the current stage
        auto bload = [&](int64_t t, int p) __attribute__((always_inline)) {
            const v16_t* q = reinterpret_cast<const v16_t*>(bptr(t, p));
            rb[p] = NT ? __builtin_nontemporal_load(q) : *q;
        };
        // Stage t's B where it may pass K: k from K up reads as zero.
        auto bload_tail = [&](int64_t t, int p) __attribute__((always_inline)) {
#pragma unroll
            for (int e = 0; e < 16 / (int)sizeof(T); ++e) {
                const int64_t k = 16 * t + 4 * lg + (TB ? SPL * (p / NB) + e : p);
                const bool ok = k < g.K;
                const T* q = TB ? bptr(t, p) + e : bptr(t, p) + e;
                const T x = *(ok ? q : static_cast<const T*>(g.B));
                rb[p][e] = ok ? x : T(0);
            }
        };
        auto aload = [&](int64_t t) __attribute__((always_inline)) {
            if (FULLM && t < nfull) sa.template load<true>(A, g.lda, m0, g.M, t * kBK, g.K);
            else sa.template load<false>(A, g.lda, m0, g.M, t * kBK, g.K);
        };
        auto afrag = [&](const T* sbuf, int a, int s) __attribute__((always_inline)) -> T {
            return TA ? sbuf[(4 * lg + s) * SA::PITCH + 16 * a + c] : sbuf[(16 * a + c) * SA::PITCH + 4 * lg + s];
        };
        // The MFMAs piece p feeds. Every accumulator still takes MFMA steps
        // 0, 1, 2, 3 in order.
        T fa[4][SPL];
        auto piece = [&](const T* sbuf, int p) __attribute__((always_inline)) {
            if (!TB) {
#pragma unroll
                for (int a = 0; a < 4; ++a) fa[a][0] = afrag(sbuf, a, p);
#pragma unroll
                for (int a = 0; a < 4; ++a)
#pragma unroll
                    for (int b = 0; b < NB; ++b) acc[a][b] = MF::mma(fa[a][0], rb[p][b], acc[a][b]);
            } else {
                const int h = p / NB, b = p % NB;
                if (b == 0) {
#pragma unroll
                    for (int a = 0; a < 4; ++a)
#pragma unroll
                        for (int e = 0; e < SPL; ++e) fa[a][e] = afrag(sbuf, a, SPL * h + e);
                }
#pragma unroll
                for (int e = 0; e < SPL; ++e)
#pragma unroll
                    for (int a = 0; a < 4; ++a) acc[a][b] = MF::mma(fa[a][e], rb[p][e], acc[a][b]);
            }
        };
        // A wave whose columns all lie past N (in a last, partial column tile)
        // only helps stage A: the same loads, stores and barriers as the
        // loop below, no B loads and no MFMAs, so its SIMD's MFMA pipe serves
        // the other workgroups. Its accumulators stay zero and are never
        // stored (not with DOT, whose column tiles are full). Config 5's
        // optimal-order step 'jb,abP->jaP' (N = 800): 0.828 against 0.830 and
        // 0.836 ms for the whole path, 12% fewer executed MFMA FLOP there.
        const int wave_u = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        if (!DOT && tn * BN + (int64_t)wave_u * (16 * NB) >= g.N) {
            aload(0);
            sa.store(lds);
            __syncthreads();
            for (int64_t t = 0; t + 1 < nk; ++t) {
                aload(t + 1);
                sa.store(lds + ((t + 1) & 1) * SA::ELEMS);
                __syncthreads();
            }
        } else {
        aload(0);
        sa.store(lds);
        int64_t t = 0;
        // Only the vector loads of B lead into the main loop: with the
        // element-wise tail loads joining them there, the compiler's wait at
        // the top of each stage covered every outstanding load (same box,
        // alternating, bitwise equal: 4096^3 fp32 1.0135 against 1.0172 ms,
        // 64 x 512^3 with alpha/beta 0.1441 against 0.1456 ms fp32 and 0.2639
        // against 0.2669 ms fp64).
        if (nfull == 0) {
#pragma unroll
            for (int p = 0; p < 4; ++p) bload_tail(0, p);
            __syncthreads();
        } else {  // the main loop below is this branch's (closed after it)
#pragma unroll
            for (int p = 0; p < 4; ++p) bload(0, p);
            __syncthreads();
        for (; t + 1 < nfull; ++t) {
            // Stage t + 1 of A goes to the other buffer; B piece p is reloaded
            // for stage t + 1 as soon as its MFMAs have issued. With B
            // k-contiguous the fp64 wave issuing the MFMAs runs at raised
            // priority for the burst (0.4-0.5% faster); with B row-major the
            // default priority is faster (same box, alternating, bitwise
            // equal: AO->MO half transform 0.865 against 0.890 ms, 4096^3 1.883
            // against 1.924 ms, 64 x 512^3 with alpha/beta 0.266 against 0.275
            // ms, the transform's batched GEMM 0.479 against 0.511 ms).
            aload(t + 1);
            const T* cur = lds + (t & 1) * SA::ELEMS;
            if (sizeof(T) == 8 && TB) __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                piece(cur, p);
                bload(t + 1, p);
            }
            if (sizeof(T) == 8 && TB) __builtin_amdgcn_s_setprio(0);
            if constexpr (sizeof(T) == 4 && !TB) {
                // A's loads, then each piece's MFMAs followed by its
                // next-stage B load; left to itself the compiler issued the
                // four B loads together near the end of the stage (same box,
                // alternating, bitwise equal: 4096^3 1.0036 against 1.0135
                // ms, 64 x 512^3 with alpha/beta 0.1437 against 0.1441 ms; in
                // fp64 4096^3 measured 1% slower with it).
                __builtin_amdgcn_sched_group_barrier(0x020, SA::NC, 0);
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 4 * NB, 0);
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            sa.store(lds + ((t + 1) & 1) * SA::ELEMS);
            __syncthreads();
        }
        }  // nfull > 0
        if (t + 1 < nk) {
            // The partial last stage (K not a multiple of 16).
            aload(t + 1);
            const T* cur = lds + (t & 1) * SA::ELEMS;
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                piece(cur, p);
                bload_tail(t + 1, p);
            }
            sa.store(lds + ((t + 1) & 1) * SA::ELEMS);
            __syncthreads();
            ++t;
        }
        const T* cur = lds + (t & 1) * SA::ELEMS;
#pragma unroll
        for (int p = 0; p < 4; ++p) piece(cur, p);
        }  // live wave
    }

    if constexpr (DOT) {
        // acc[a][b][r] is row m0 + 16 a + MF::row(lg, r), column col + b. The
        // lane indices are formed again here rather than held through the K
        // loop.
        int tid = threadIdx.x;
        asm volatile("" : "+v"(tid));
        const int lg = (tid & 63) >> 4;
        const int64_t col = tn * BN + (tid >> 6) * (16 * NB) + NB * (tid & 15);
        // Dot epilogue: sum of D .* E over this tile, one double per
        // workgroup (see gemm_kernel's), in a fixed order: column blocks,
        // row blocks, then rows; each block's eight E loads go out together.
        __shared__ double red[4];
        const T* E1 = static_cast<const T*>(g.E1) + bat * g.e1s[4];
        const T* E2 = g.E2 ? static_cast<const T*>(g.E2) + bat * g.e2s[4] : nullptr;
        double sum = 0.0;
        // E2 present or not: two straight-line copies of the loop below.
        auto dot = [&](auto has_e2) __attribute__((always_inline)) {
            constexpr bool HE2 = decltype(has_e2)::value;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                // The row parts below are formed again for every column block
                // (the empty asm hides that they repeat): held across the
                // blocks, they would not fit the registers of four waves per
                // SIMD.
                int lgb = lg;
                asm volatile("" : "+v"(lgb));
                const uint32_t cb = (uint32_t)(col + b);
                const uint32_t nh = fdiv(cb, g.ndiv);
                const uint32_t nl = cb - nh * g.ndiv.d;
                const int64_t o1n = nh * g.e1s[2] + nl * g.e1s[3];
                const int64_t o2n = nh * g.e2s[2] + nl * g.e2s[3];
#pragma unroll
                for (int a = 0; a < 4; ++a) {
                    T e1v[4], e2v[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int64_t row = m0 + 16 * a + MF::row(lgb, r);
                        const bool ok = FULLM || row < g.M;
                        const uint32_t rr = (uint32_t)(ok ? row : 0);
                        const uint32_t mh = fdiv(rr, g.mdiv);
                        const uint32_t ml = rr - mh * g.mdiv.d;
                        e1v[r] = E1[ok ? mh * g.e1s[0] + ml * g.e1s[1] + o1n : 0];
                        if (HE2) e2v[r] = E2[ok ? mh * g.e2s[0] + ml * g.e2s[1] + o2n : 0];
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int64_t row = m0 + 16 * a + MF::row(lgb, r);
                        if (FULLM || row < g.M) {
                            T e = e1v[r];
                            if (HE2) e = e * e2v[r];
                            sum += (double)(acc[a][b][r] * e);
                        }
                    }
                    // One block's loads in flight at a time.
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        };
        if (E2) dot(std::true_type{});
        else dot(std::false_type{});
        const double tot = block256_sum(sum, red);
        if (tid == 0) g.partial[blockIdx.x] = tot;
        return;
    } else {
        directb_store<T, FULLM>(g, acc, bat, m0, tn);
    }
}

// Persistent form of gemm_directb_kernel (store epilogue, no C, D 16-byte
// aligned, whole 64-row and BN-column tiles, K a positive multiple of 16): each workgroup walks a list of tiles
// and the stages of consecutive tiles form one software pipeline. The next
// tile's first stage (A slab into LDS, B pieces into registers) is loaded
// during the current tile's last MFMAs, and the current tile's stores are
// issued while those loads are in flight, so no workgroup waits out a
// memory latency between tiles. Hardware workgroup w runs on XCD w % 8; the
// tiles are split into eight contiguous ranges, one per XCD, and the
// workgroups of an XCD take that range's tiles round-robin. The MFMA order
// per accumulator is gemm_directb_kernel's: results are bitwise equal.
template <typename T, bool TA, bool TB, bool NT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) void gemm_directb_persistent_kernel(
    GemmArgs g) {
    typedef Mfma<T> MF;
    typedef typename MF::acc_t acc_t;
    constexpr int NB = 16 / sizeof(T);
    constexpr int BN = 64 * NB;
    constexpr int SPL = TB ? 16 / sizeof(T) : 1;
    typedef typename VecN<T, 16 / sizeof(T)>::type v16_t;
    typedef Stage<T, 64, !TA, true, kBK> SA;
    __shared__ __attribute__((aligned(16))) T lds[2 * SA::ELEMS];

    const int64_t tiles = g.tiles_m * g.tiles_n;
    const int64_t total = tiles * g.batch;
    const int64_t x = blockIdx.x % kNumXcd;
    const int64_t per = gridDim.x / kNumXcd;  // the grid is a multiple of 8
    const int64_t hi = total * (x + 1) / kNumXcd;
    int64_t id = total * x / kNumXcd + blockIdx.x / kNumXcd;
    if (id >= hi) return;  // the whole workgroup: no barrier is left waiting
    const int64_t nk = g.K / kBK;

    const int lane = threadIdx.x & 63;
    const int lg = lane >> 4;
    const int c = lane & 15;
    // The lane's offset into a tile's B panel (N is a multiple of BN: no
    // column clamp), the same for every tile; the tile bases are uniform.
    const int64_t wcol = (threadIdx.x >> 6) * (16 * NB) + NB * c;
    const int64_t boff = TB ? wcol * g.ldb + 4 * lg : wcol + (int64_t)(4 * lg) * g.ldb;
    struct Tile {
        const T* A;
        const T* B;
        int64_t bat, tn, m0;
    };
    auto tile = [&](int64_t tid) __attribute__((always_inline)) -> Tile {
        Tile u;
        u.bat = tid / tiles;
        const int64_t rem = tid - u.bat * tiles;
        u.tn = rem / g.tiles_m;
        u.m0 = (rem - u.tn * g.tiles_m) * 64;
        u.A = static_cast<const T*>(g.A) + u.bat * g.sA;
        u.B = static_cast<const T*>(g.B) + u.bat * g.sB + (TB ? u.tn * BN * g.ldb : u.tn * BN);
        return u;
    };
    SA sa;
    v16_t rb[4];
    auto bload = [&](const T* B, int64_t t, int p) __attribute__((always_inline)) {
        const T* q = (TB ? B + (int64_t)(p % NB) * g.ldb + 16 * t + SPL * (p / NB) : B + (16 * t + p) * g.ldb) + boff;
        rb[p] = NT ? __builtin_nontemporal_load(reinterpret_cast<const v16_t*>(q)) : *reinterpret_cast<const v16_t*>(q);
    };
    auto afrag = [&](const T* sbuf, int a, int s) __attribute__((always_inline)) -> T {
        return TA ? sbuf[(4 * lg + s) * SA::PITCH + 16 * a + c] : sbuf[(16 * a + c) * SA::PITCH + 4 * lg + s];
    };
    acc_t acc[4][NB];
    T fa[4][SPL];
    auto piece = [&](const T* sbuf, int p) __attribute__((always_inline)) {
        if (!TB) {
#pragma unroll
            for (int a = 0; a < 4; ++a) fa[a][0] = afrag(sbuf, a, p);
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int b = 0; b < NB; ++b) acc[a][b] = MF::mma(fa[a][0], rb[p][b], acc[a][b]);
        } else {
            const int h = p / NB, b = p % NB;
            if (b == 0) {
#pragma unroll
                for (int a = 0; a < 4; ++a)
#pragma unroll
                    for (int e = 0; e < SPL; ++e) fa[a][e] = afrag(sbuf, a, SPL * h + e);
            }
#pragma unroll
            for (int e = 0; e < SPL; ++e)
#pragma unroll
                for (int a = 0; a < 4; ++a) acc[a][b] = MF::mma(fa[a][e], rb[p][e], acc[a][b]);
        }
    };

    Tile cur = tile(id);
    sa.template load<true>(cur.A, g.lda, cur.m0, g.M, 0, g.K);
    sa.store(lds);
#pragma unroll
    for (int p = 0; p < 4; ++p) bload(cur.B, 0, p);
    __syncthreads();
    int buf = 0;
    for (;;) {
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int b = 0; b < NB; ++b) acc[a][b] = acc_t{0, 0, 0, 0};
        for (int64_t t = 0; t + 1 < nk; ++t) {
            sa.template load<true>(cur.A, g.lda, cur.m0, g.M, (t + 1) * kBK, g.K);
            const T* sb = lds + buf * SA::ELEMS;
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                piece(sb, p);
                bload(cur.B, t + 1, p);
            }
            __builtin_amdgcn_sched_barrier(0);
            sa.store(lds + (buf ^ 1) * SA::ELEMS);
            __syncthreads();
            buf ^= 1;
        }
        // Last stage: the next tile's first stage goes out behind its MFMAs.
        const int64_t nid = id + per;
        const bool more = nid < hi;
        const Tile nxt = tile(more ? nid : id);
        if (more) sa.template load<true>(nxt.A, g.lda, nxt.m0, g.M, 0, g.K);
        const T* sb = lds + buf * SA::ELEMS;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            piece(sb, p);
            if (more) bload(nxt.B, 0, p);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (more) sa.store(lds + (buf ^ 1) * SA::ELEMS);
        directb_store<T, true, true>(g, acc, cur.bat, cur.m0, cur.tn);
        if (!more) break;
        __syncthreads();
        buf ^= 1;
        id = nid;
        cur = nxt;
    }
}


// Streaming direct-B GEMM (fp64, A transposed, B row-major, no C, at most two
// 64-row tiles: the AO->MO half transform's shape, where B streams from HBM
// once and feeds at most 128 rows). Persistent like
// gemm_directb_persistent_kernel, but 64 x 256 tiles of four waves of 64 x 64
// (NB = 4 column blocks), two workgroups per CU (two waves per SIMD), so
// each A fragment read from LDS feeds 16 MFMAs instead of 8. Column block
// 2 j + e of a lane is column 32 j + 2 c + e of its wave's 64: every 16-byte
// B load and D store of a lane group covers 256 contiguous bytes. Per
// 16-k stage: the next piece's A fragments are read ahead, the next stage's B
// pieces are loaded one per 8 MFMAs, and the barrier comes before the last
// piece, whose MFMAs cover the next stage's first fragment reads. The stages
// of consecutive tiles form one pipeline (the next tile's first stage is
// loaded during the current tile's last). MFMA order per output as
// gemm_directb_kernel's: bitwise equal. Same box, alternating, against the
// persistent 64 x 128 kernel: 64 x 786432 x 512 0.842-0.851 against
// 0.880 ms, 64 x 393216 x 1024 0.819 against 0.855 ms, 128 x 393216 x 512
// 0.775 against 0.803 ms; with five row tiles (the transform's batched
// GEMM, 320 x 1536 x 512 x 64) it lost (0.490 against 0.483 ms), with 1.5
// tiles per workgroup it tied. One wave per SIMD with NB = 8 (AGPR
// accumulators) ran 0.951 against 0.914 ms on another box, and B two stages
// ahead (238 VGPRs) 0.907 against 0.852 ms.
template <bool NT>
__global__ __launch_bounds__(kThreads, 2) void gemm_directb_stream_kernel(GemmArgs g) {
    typedef Mfma<double> MF;
    typedef typename MF::acc_t acc_t;
    constexpr int NB = 4;
    constexpr int BN = 64 * NB;
    typedef typename Vec16<double>::type v16_t;
    typedef Stage<double, 64, false, true, kBK> SA;
    __shared__ __attribute__((aligned(16))) double lds[2 * SA::ELEMS];

    // Hardware workgroup w runs on XCD w % 8; the tiles are split into eight
    // contiguous ranges, one per XCD, taken round-robin by its workgroups.
    const int64_t tiles = g.tiles_m * g.tiles_n;
    const int64_t total = tiles * g.batch;
    const int64_t x = blockIdx.x % kNumXcd;
    const int64_t per = gridDim.x / kNumXcd;  // the grid is a multiple of 8
    const int64_t hi = total * (x + 1) / kNumXcd;
    int64_t id = total * x / kNumXcd + blockIdx.x / kNumXcd;
    if (id >= hi) return;  // the whole workgroup: no barrier is left waiting
    const int64_t nk = g.K / kBK;

    const int lane = threadIdx.x & 63;
    const int lg = lane >> 4;
    const int c = lane & 15;
    const int64_t wcol = (threadIdx.x >> 6) * (16 * NB) + 2 * c;
    const int64_t boff = wcol + (int64_t)(4 * lg) * g.ldb;
    struct Tile {
        const double* A;
        const double* B;
        int64_t bat, tn, m0;
    };
    auto tile = [&](int64_t tid) __attribute__((always_inline)) -> Tile {
        Tile u;
        u.bat = tid / tiles;
        const int64_t rem = tid - u.bat * tiles;
        u.tn = rem / g.tiles_m;
        u.m0 = (rem - u.tn * g.tiles_m) * 64;
        u.A = static_cast<const double*>(g.A) + u.bat * g.sA;
        u.B = static_cast<const double*>(g.B) + u.bat * g.sB + u.tn * BN;
        return u;
    };
    SA sa;
    v16_t rb[4][NB / 2];  // [piece p][j]: k-row 16 t + 4 lg + p, columns 32 j + 2 c, + 1
    auto bload = [&](const double* B, int64_t t, int p) __attribute__((always_inline)) {
        const double* q = B + (16 * t + p) * g.ldb + boff;
#pragma unroll
        for (int j = 0; j < NB / 2; ++j) {
            const v16_t* qq = reinterpret_cast<const v16_t*>(q + 32 * j);
            rb[p][j] = NT ? __builtin_nontemporal_load(qq) : *qq;
        }
    };
    auto afrag = [&](const double* sbuf, int a, int s) __attribute__((always_inline)) -> double {
        return sbuf[(4 * lg + s) * SA::PITCH + 16 * a + c];
    };
    acc_t acc[4][NB];
    double fa[2][4];
    auto piece = [&](int p, const double (&f)[4]) __attribute__((always_inline)) {
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int b = 0; b < NB; ++b) acc[a][b] = MF::mma(f[a], rb[p][b >> 1][b & 1], acc[a][b]);
    };
    // Scheduling groups: the piece's A reads first (0x100), then one B load
    // (0x020) after every 8 MFMAs (0x008).
    auto spread = [&]() __attribute__((always_inline)) {
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
        for (int i = 0; i < NB / 2; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // One stage of the current tile from LDS buffer buf; stage tn1 of tile
    // nxt is loaded behind it when `more`.
    auto stage = [&](int buf, bool more, const Tile& nxt, int64_t tn1) __attribute__((always_inline)) {
        if (more) sa.template load<true>(nxt.A, g.lda, nxt.m0, g.M, tn1 * kBK, g.K);
        const double* sb = lds + buf * SA::ELEMS;
#pragma unroll
        for (int p = 0; p < 3; ++p) {
#pragma unroll
            for (int a = 0; a < 4; ++a) fa[(p + 1) & 1][a] = afrag(sb, a, p + 1);
            piece(p, fa[p & 1]);
            if (more) bload(nxt.B, tn1, p);
            spread();
        }
        if (more) sa.store(lds + (buf ^ 1) * SA::ELEMS);
        __syncthreads();
        if (more) {
#pragma unroll
            for (int a = 0; a < 4; ++a) fa[0][a] = afrag(lds + (buf ^ 1) * SA::ELEMS, a, 0);
        }
        piece(3, fa[1]);
        if (more) bload(nxt.B, tn1, 3);
        spread();
    };
    // D is written once and not read here: non-temporal stores (64 x 786432
    // x 512, same box, alternating, three runs: 0.838-0.845 against
    // 0.844-0.849 ms; K 1024 with N / 2: 0.818 against 0.813 ms).
    auto store = [&](const Tile& u) __attribute__((always_inline)) {
        double* D = static_cast<double*>(g.D) + u.bat * g.sD;
        const int64_t col = u.tn * BN + wcol;
        const double alpha = g.alpha;
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = u.m0 + 16 * a + MF::row(lg, r);
#pragma unroll
                for (int j = 0; j < NB / 2; ++j) {
                    v16_t v;
                    v[0] = acc[a][2 * j][r];
                    v[1] = acc[a][2 * j + 1][r];
                    if (alpha != 1.0) v = v * alpha;
                    __builtin_nontemporal_store(v, reinterpret_cast<v16_t*>(D + row * g.ldd + col + 32 * j));
                }
            }
    };

    Tile cur = tile(id);
    sa.template load<true>(cur.A, g.lda, cur.m0, g.M, 0, g.K);
    sa.store(lds);
#pragma unroll
    for (int p = 0; p < 4; ++p) bload(cur.B, 0, p);
    __syncthreads();
#pragma unroll
    for (int a = 0; a < 4; ++a) fa[0][a] = afrag(lds, a, 0);
    int buf = 0;
    for (;;) {
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int b = 0; b < NB; ++b) acc[a][b] = acc_t{0, 0, 0, 0};
        for (int64_t t = 0; t + 1 < nk; ++t) {
            stage(buf, true, cur, t + 1);
            buf ^= 1;
        }
        const int64_t nid = id + per;
        const bool more = nid < hi;
        const Tile nxt = tile(more ? nid : id);
        stage(buf, more, nxt, 0);
        buf ^= 1;
        store(cur);
        if (!more) break;
        id = nid;
        cur = nxt;
    }
}

// Compute units of the current device (cached per device).
static int device_cus() {
    static int cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

template <typename T, bool DOT>
static int launch_directb(GemmArgs& g, bool ta, bool tb, bool nt, hipStream_t st) {
    constexpr int BN = 64 * (16 / sizeof(T));
    g.tiles_m = (g.M + 63) / 64;
    g.tiles_n = (g.N + BN - 1) / BN;
    const int64_t total = g.tiles_m * g.tiles_n * g.batch;
    if (total > 0x7fffffffLL) return set_error(TT_UNSUPPORTED, "tt_gemm: %lld tiles exceed one launch", (long long)total);
    const bool full = g.M % 64 == 0;
    // Three or more rounds of tiles (four workgroups per CU) with A
    // transposed and B row-major (the AO->MO transform's two GEMMs): the
    // persistent kernel. Same box, alternating, bitwise equal: AO->MO half
    // transform (64 x 786432 x 512) 0.8646 against 0.8787 ms, the transform's
    // batched GEMM (64 x 320 x 1536 x 512) 0.4702 against 0.4830 ms. At two
    // rounds (4096^3, 64 x 512^3 without C) it measured 1-2% slower, and its
    // other layouts spill registers.
    const int64_t slots = (int64_t)device_cus() / kNumXcd * 4;
    const bool vecd = ((reinterpret_cast<uintptr_t>(g.D) | (uintptr_t)(g.ldd * sizeof(T)) |
                        (uintptr_t)(g.sD * sizeof(T))) & 15) == 0;
    // fp64 with at most two row tiles and at least three 64 x 256 tiles per
    // workgroup at two per CU: the streaming kernel.
    if constexpr (sizeof(T) == 8 && !DOT) {
        const int64_t stiles = g.tiles_m * (g.N / 256) * g.batch;
        const int64_t sgrid = (int64_t)device_cus() / kNumXcd * kNumXcd * 2;
        if (ta && !tb && full && !g.C && vecd && g.N % 256 == 0 && g.K >= kBK && g.K % kBK == 0 &&
            g.tiles_m <= 2 && stiles >= 3 * sgrid) {
            g.tiles_n = g.N / 256;
            const dim3 grid((unsigned)sgrid), block(kThreads);
            if (nt) hipLaunchKernelGGL((gemm_directb_stream_kernel<true>), grid, block, 0, st, g);
            else hipLaunchKernelGGL((gemm_directb_stream_kernel<false>), grid, block, 0, st, g);
            return check_launch("tt_gemm");
        }
    }
    if (!DOT && ta && !tb && full && !g.C && vecd && g.N % BN == 0 && g.K >= kBK && g.K % kBK == 0 &&
        total >= 3 * slots * kNumXcd) {
        const dim3 grid((unsigned)(slots * kNumXcd)), block(kThreads);
        if (nt) hipLaunchKernelGGL((gemm_directb_persistent_kernel<T, true, false, true>), grid, block, 0, st, g);
        else hipLaunchKernelGGL((gemm_directb_persistent_kernel<T, true, false, false>), grid, block, 0, st, g);
        return check_launch("tt_gemm");
    }
    const dim3 grid((unsigned)total), block(kThreads);
#define TT_DIRECTB_CASE(F, A_T, B_T, N_T)                         \
    if (full == F && ta == A_T && tb == B_T && nt == N_T)         \
        hipLaunchKernelGGL((gemm_directb_kernel<T, F, A_T, B_T, N_T, DOT>), grid, block, 0, st, g);
#define TT_DIRECTB_NT(F, A_T, B_T) TT_DIRECTB_CASE(F, A_T, B_T, true) TT_DIRECTB_CASE(F, A_T, B_T, false)
#define TT_DIRECTB_TB(F, A_T) TT_DIRECTB_NT(F, A_T, false) TT_DIRECTB_NT(F, A_T, true)
    TT_DIRECTB_TB(true, true)
    TT_DIRECTB_TB(false, true)
    TT_DIRECTB_TB(true, false)
    TT_DIRECTB_TB(false, false)
#undef TT_DIRECTB_TB
#undef TT_DIRECTB_NT
#undef TT_DIRECTB_CASE
    return check_launch("tt_gemm");
}

template <typename T, int BM, int BN, int FM, int FN, bool DOT, int NBUF = 2, int BK = kBK, bool PRIO = false>
static int launch_tile(GemmArgs& g, bool ta, bool tb, bool vec, hipStream_t st) {
    g.tiles_m = (g.M + BM - 1) / BM;
    g.tiles_n = (g.N + BN - 1) / BN;
    const int64_t total = g.tiles_m * g.tiles_n * g.batch;
    if (total > 0x7fffffffLL) return set_error(TT_UNSUPPORTED, "tt_gemm: %lld tiles exceed one launch", (long long)total);
    dim3 grid((unsigned)total), block(kThreads);
#define TT_GEMM_CASE(TA, TB, VC) \
    if (ta == TA && tb == TB && vec == VC) hipLaunchKernelGGL((gemm_kernel<T, BM, BN, FM, FN, TA, TB, VC, DOT, NBUF, BK, PRIO>), grid, block, 0, st, g);
    TT_GEMM_CASE(false, false, false)
    TT_GEMM_CASE(false, false, true)
    TT_GEMM_CASE(false, true, false)
    TT_GEMM_CASE(false, true, true)
    TT_GEMM_CASE(true, false, false)
    TT_GEMM_CASE(true, false, true)
    TT_GEMM_CASE(true, true, false)
    TT_GEMM_CASE(true, true, true)
#undef TT_GEMM_CASE
    return check_launch("tt_gemm");
}

// Small problems: 32 x 32 tiles (four 16 x 16 wave tiles) and one stage that
// holds all of K, so a launch makes one round trip to memory instead of one
// per 16-deep stage. Both operands k-contiguous (A not transposed, B
// transposed), the layouts whose 32-row stage the staging supports. The k
// order per output is the other tiles' (16-deep passes in order).
template <typename T, int BK>
static int launch_small(GemmArgs& g, bool vec, hipStream_t st) {
    g.tiles_m = (g.M + 31) / 32;
    g.tiles_n = (g.N + 31) / 32;
    const int64_t total = g.tiles_m * g.tiles_n * g.batch;
    if (total > 0x7fffffffLL) return set_error(TT_UNSUPPORTED, "tt_gemm: %lld tiles exceed one launch", (long long)total);
    const dim3 grid((unsigned)total), block(kThreads);
    if (vec) hipLaunchKernelGGL((gemm_kernel<T, 32, 32, 1, 1, false, true, true, false, 1, BK, false>), grid, block, 0, st, g);
    else hipLaunchKernelGGL((gemm_kernel<T, 32, 32, 1, 1, false, true, false, false, 1, BK, false>), grid, block, 0, st, g);
    return check_launch("tt_gemm");
}

template <typename T, bool DOT>
static int gemm_typed(GemmArgs& g, bool ta, bool tb, hipStream_t st) {
    constexpr int V = Vec16<T>::n;
    auto ok16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    // 16-byte vectors need aligned bases, leading dimensions and batch strides.
    bool vec = ok16(g.A) && ok16(g.B) && g.lda % V == 0 && g.ldb % V == 0;
    if (g.batch > 1) vec = vec && g.sA % V == 0 && g.sB % V == 0;
    // One 32 x 32 tile per batch entry and K within one deep stage (the
    // DF-MP2 pair block 'ap,bp->ab' of config 1: 32 x 32 x 96).
    constexpr int64_t KS = 512 / sizeof(T);  // 128 fp32, 64 fp64
    if (!DOT && !ta && tb && g.M <= 32 && g.N <= 32 && g.K <= KS) {
        if (g.K <= KS / 2) return launch_small<T, KS / 2>(g, vec, st);
        return launch_small<T, KS>(g, vec, st);
    }
    // Small-M (e.g. the AO->MO half transform, M = nocc): 64 x 128 tiles of
    // four 32 x 64 wavefront tiles keep registers and LDS low enough for
    // several workgroups per CU, i.e. more loads in flight on a long stream.
    // Batched short-K fp64 (e.g. 64 x 512^3): three 64 x 128 workgroups per
    // CU instead of two 128 x 128 ones overlap one workgroup's prologue and
    // epilogue with the others' MFMAs (measured 62% -> 70% of fp64 peak;
    // unbatched and fp32 cases measured no gain).
    // fp64 small-M (the AO->MO half transform: M = nocc, K = nbasis, N =
    // nbasis * naux): one LDS stage buffer (26 KB) gives four workgroups per
    // CU instead of three, and the wave issuing a stage's MFMAs raises its
    // priority for the burst. Same box, results bitwise equal: 64 x 786432 x
    // 512 0.928-0.952 -> 0.895-0.927 ms (+2-3%). Raised priority measured
    // slower for the batched and large fp64 tiles (64 x 512^3: +12% time), so
    // it stays on this tile only. This tile streams B (non-temporal loads), so
    // a B broadcast over the batch (stride 0, re-read per batch entry) takes
    // the two-buffer tile below.
    // fp64: A through LDS, B straight into the MFMA registers
    // (gemm_directb_kernel above), non-temporal when B is read once (M <= 64).
    // With B row-major and N a multiple of 128, same box, alternating,
    // bitwise equal, against the LDS-staged tiles below: 4096^3 with alpha/beta 1.952 against 2.082
    // ms (NN 1.944 against 2.069, TN 1.965 against 2.171), 4096^2 x 512 0.258
    // against 0.274 ms, 64 x 512^3 with alpha/beta and C 0.275 against 0.292
    // ms, the AO->MO transform's two GEMMs 0.885 against 0.914 and 0.492
    // against 0.520 ms. With N % 128 columns left over, a second launch for
    // them ran alone after the first (nocc 50, N = 100002: 0.198 against
    // 0.146 ms); a partial last tile in the same launch (below) takes 0.144.
    // B k-contiguous (NT, TT) takes the same kernel, and so does the dot
    // epilogue when M is a multiple of 64 (with row masking its epilogue
    // spills). Same box, alternating: 4096^3 NT 2.026 against 2.130 ms and TT
    // 2.025 against 2.104 ms (bitwise equal); the fused contraction of config
    // 5 (dot GEMM 160000 x 16384 x 800, B k-contiguous) 66.2-66.4 against
    // 67.9-68.0 ms, the sum equal to 2e-15 (another order of the per-tile
    // sums).
    // Any even N (a last, partial column tile clamps its columns; the dot
    // epilogue keeps N a multiple of 128, any M: rows past M read A as zero
    // and are left out of the sum). Same box, alternating, bitwise
    // equal, against the LDS-staged tiles: 3000 x 3000 x 1000 with alpha/beta
    // 0.331 against 0.438 ms, NT 0.382 against 0.426 ms, 8192 x 200 x 2048
    // 0.145 against 0.186 ms, config 5's optimal-order GEMM (400 x 128 x 800
    // x 400) 0.580 against 0.629 ms. The fp32 tile lost on such shapes (3000
    // x 3000 x 1000 0.221 against 0.212 ms), so fp32 keeps whole tiles.
    if constexpr (sizeof(T) == 8)
        if (vec && (DOT ? g.N % 128 == 0 : g.N % 2 == 0))
            return launch_directb<T, DOT>(g, ta, tb, g.M <= 64 && (g.batch == 1 || g.sB != 0), st);
    // fp32 on 64 x 256 tiles (four 16-column MFMA blocks per wave, so a lane's
    // B piece is still 16 bytes): within 1-2% of the LDS-staged tiles, ahead
    // on short K (same box, alternating, bitwise equal: 4096^2 x 512 0.1345
    // against 0.1364 ms, 64 x 512^3 with alpha/beta and C 0.1397 against
    // 0.1414 ms, 4096^3 0.988 against 0.990 ms).
    // fp32, both operands not transposed, whole 256 x 256 tiles in whole
    // rounds of one tile per CU (at least 95% of the last round busy), without
    // C or with K >= 1024: the 256 x 256 LDS tile (tt_gemm_big.hip), bitwise
    // equal to the tiles below. Same box, alternating, fraction of the fp32
    // peak against the 64 x 256 direct-B tile: 4096^3 with alpha/beta and C
    // 0.93 against 0.88; 64 x 512^3 without C 0.834 against 0.806, 16 x
    // 1024^3 with C 0.866 against 0.845. A partial last round loses (6144^2 x
    // 2048, 2.25 rounds: 1.444 against 1.118 ms), and so does a short K with
    // C, whose epilogue one wave per SIMD cannot hide (64 x 512^3 with C
    // 0.785 against 0.801, 128 x 512^3 with C 0.760 against 0.799).
    if constexpr (sizeof(T) == 4 && !DOT)
        if (gemm_big_f32_fits(ta, tb, g) && (!g.C || g.K >= 1024)) {
            const int64_t tiles = (g.M / 256) * (g.N / 256) * g.batch, cus = device_cus();
            const int64_t rounds = (tiles + cus - 1) / cus;
            if (tiles >= cus && 100 * tiles >= 95 * rounds * cus) return gemm_big_f32_launch(g, st);
        }
    if constexpr (sizeof(T) == 4 && !DOT)
        if (!tb && vec && g.N % 256 == 0)
            return launch_directb<T, DOT>(g, ta, false, g.M <= 64 && (g.batch == 1 || g.sB != 0), st);
    if (sizeof(T) == 8 && !DOT && g.M <= 64 && (g.batch == 1 || g.sB != 0))
        return launch_tile<T, 64, 128, 2, 4, DOT, 1, kBK, true>(g, ta, tb, vec, st);
    if (g.M <= 64 || (sizeof(T) == 8 && g.batch > 1 && g.K <= 1024))
        return launch_tile<T, 64, 128, 2, 4, DOT>(g, ta, tb, vec, st);
    if (g.N <= 64) return launch_tile<T, 256, 64, 4, 4, DOT>(g, ta, tb, vec, st);
    // Small grids: fewer than 448 128 x 128 tiles leave CUs idle; 64 x 128
    // tiles double the grid (fp32, fp64 TFLOP/s against 128 x 128: 1024^3 41.9
    // and 25.9 against 21.9 and 14.6; 2000 x 3000 x 2000 77.2 and 50.9 against
    // 59.5 and 39.4; 2048^3 112.4 and 60.3 against 90.8 and 59.8; at 484 tiles,
    // 2816^3, 120.4 and 60.7 against 131.3 and 62.0). Results are identical
    // (the k order per output does not depend on the tile).
    if (((g.M + 127) / 128) * ((g.N + 127) / 128) * g.batch < 448)
        return launch_tile<T, 64, 128, 2, 4, DOT>(g, ta, tb, vec, st);
    return launch_tile<T, 128, 128, 4, 4, DOT>(g, ta, tb, vec, st);
}

int gemm_dispatch(int dtype, bool ta, bool tb, GemmArgs& g, hipStream_t st) {
    g.E1 = g.E2 = nullptr;
    g.partial = nullptr;
    if (dtype == TT_F64) return gemm_typed<double, false>(g, ta, tb, st);
    if (dtype == TT_F32) return gemm_typed<float, false>(g, ta, tb, st);
    if (dtype == TT_F64_DD) return gemm_dd_dispatch(ta, tb, g, st);
    if (dtype == TT_BF16 || dtype == TT_F16) return gemm16_dispatch(dtype, ta, tb, g, st);
    return set_error(TT_UNSUPPORTED, "tt_gemm: dtype %d (only TT_F32, TT_F64, TT_F64_DD, TT_BF16, TT_F16)", dtype);
}

int gemm_dot_dispatch(int dtype, bool ta, bool tb, GemmArgs& g, hipStream_t st, int64_t* nparts) {
    int rc;
    if (dtype == TT_F64) rc = gemm_typed<double, true>(g, ta, tb, st);
    else if (dtype == TT_F32) rc = gemm_typed<float, true>(g, ta, tb, st);
    else return set_error(TT_UNSUPPORTED, "tt_gemm_dot: dtype %d (only TT_F32, TT_F64)", dtype);
    *nparts = g.tiles_m * g.tiles_n * g.batch;
    return rc;
}

// out[0] = alpha * (fixed-order sum of the partials) (+ beta * C[0]).
template <typename T>
__global__ __launch_bounds__(256) void dot_finalize_kernel(const double* partial, int64_t n, double alpha, double beta,
                                                           const T* C, T* out) {
    __shared__ double red[4];
    const double s = strided_sum256(partial, n);
    const double tot = block256_sum(s, red);
    if (threadIdx.x == 0) {
        T v = (T)tot;
        if (alpha != 1.0) v = (T)alpha * v;
        if (C) v = v + (T)beta * C[0];
        out[0] = v;
    }
}

}  // namespace tt

extern "C" int tt_gemm(int dtype, int transA, int transB, int64_t M, int64_t N, int64_t K, double alpha,
                       const void* A, int64_t lda, int64_t strideA, const void* B, int64_t ldb, int64_t strideB,
                       double beta, const void* C, int64_t ldc, int64_t strideC, void* D, int64_t ldd,
                       int64_t strideD, int64_t batch, void* stream) {
    using namespace tt;
    if (M < 0 || N < 0 || K < 0 || batch < 0)
        return set_error(TT_INVALID, "tt_gemm: negative extent (M=%lld N=%lld K=%lld batch=%lld)", (long long)M,
                         (long long)N, (long long)K, (long long)batch);
    if (M == 0 || N == 0 || batch == 0) return TT_OK;
    if (!D) return set_error(TT_INVALID, "tt_gemm: D is NULL");
    if (K > 0 && (!A || !B)) return set_error(TT_INVALID, "tt_gemm: A or B is NULL");
    const int64_t rowsA = transA ? K : M, colsA = transA ? M : K;
    const int64_t rowsB = transB ? N : K, colsB = transB ? K : N;
    if (K > 0 && ((rowsA > 1 && lda < colsA) || (rowsB > 1 && ldb < colsB)))
        return set_error(TT_INVALID, "tt_gemm: leading dimension smaller than a row (lda=%lld ldb=%lld)",
                         (long long)lda, (long long)ldb);
    if ((M > 1 && ldd < N) || (C && M > 1 && ldc < N))
        return set_error(TT_INVALID, "tt_gemm: ldd/ldc smaller than N");
    GemmArgs g;
    g.A = A;
    g.B = B;
    g.C = C;
    g.D = D;
    g.M = M;
    g.N = N;
    g.K = K;
    g.lda = lda;
    g.ldb = ldb;
    g.ldc = ldc;
    g.ldd = ldd;
    g.sA = strideA;
    g.sB = strideB;
    g.sC = strideC;
    g.sD = strideD;
    g.batch = batch;
    g.alpha = alpha;
    g.beta = beta;
    return gemm_dispatch(dtype, transA != 0, transB != 0, g, static_cast<hipStream_t>(stream));
}

extern "C" int tt_gemm_packed(const int64_t* params, double alpha, double beta, const void* A, const void* B,
                              const void* C, void* D, void* stream) {
    if (!params) return tt::set_error(TT_INVALID, "tt_gemm_packed: params is NULL");
    const int64_t* p = params;
    return tt_gemm((int)p[0], (int)p[1], (int)p[2], p[3], p[4], p[5], alpha, A, p[6], p[7], B, p[8], p[9], beta, C,
                   p[10], p[11], D, p[12], p[13], p[14], stream);
}

extern "C" size_t tt_gemm_dot_workspace_bytes(int dtype, int64_t M, int64_t N, int64_t batch) {
    (void)dtype;
    if (M <= 0 || N <= 0 || batch <= 0) return 256;
    // One double per workgroup; every tile configuration is at least 64 x 64.
    const size_t parts = (size_t)((M + 63) / 64) * (size_t)((N + 63) / 64) * (size_t)batch;
    return ((parts * sizeof(double) + 255) / 256) * 256;
}

extern "C" int tt_gemm_dot(int dtype, int transA, int transB, int64_t M, int64_t N, int64_t K, const void* A,
                           int64_t lda, int64_t strideA, const void* B, int64_t ldb, int64_t strideB, int64_t batch,
                           int64_t m_lo, int64_t n_lo, const void* E1, const int64_t* e1_strides, const void* E2,
                           const int64_t* e2_strides, double alpha, double beta, const void* C, void* out,
                           void* workspace, size_t workspace_bytes, void* stream) {
    using namespace tt;
    if (M < 0 || N < 0 || K < 0 || batch < 0)
        return set_error(TT_INVALID, "tt_gemm_dot: negative extent (M=%lld N=%lld K=%lld batch=%lld)", (long long)M,
                         (long long)N, (long long)K, (long long)batch);
    if (dtype != TT_F32 && dtype != TT_F64)
        return set_error(TT_UNSUPPORTED, "tt_gemm_dot: dtype %d (only TT_F32, TT_F64)", dtype);
    if (!out || !workspace) return set_error(TT_INVALID, "tt_gemm_dot: out or workspace is NULL");
    if (M >= (1LL << 31) || N >= (1LL << 31))
        return set_error(TT_UNSUPPORTED, "tt_gemm_dot: M or N reaches 2^31");
    const int64_t mlo = m_lo > 0 ? m_lo : 1, nlo = n_lo > 0 ? n_lo : 1;
    const size_t need = tt_gemm_dot_workspace_bytes(dtype, M, N, batch);
    if (workspace_bytes < need)
        return set_error(TT_INVALID, "tt_gemm_dot: workspace of %zu bytes, need %zu", workspace_bytes, need);
    hipStream_t st = static_cast<hipStream_t>(stream);
    int64_t nparts = 0;
    if (M > 0 && N > 0 && batch > 0) {
        if (K > 0 && (!A || !B)) return set_error(TT_INVALID, "tt_gemm_dot: A or B is NULL");
        if (!E1 || !e1_strides || (E2 && !e2_strides)) return set_error(TT_INVALID, "tt_gemm_dot: E1 is NULL");
        const int64_t rowsA = transA ? K : M, colsA = transA ? M : K;
        const int64_t rowsB = transB ? N : K, colsB = transB ? K : N;
        if (K > 0 && ((rowsA > 1 && lda < colsA) || (rowsB > 1 && ldb < colsB)))
            return set_error(TT_INVALID, "tt_gemm_dot: leading dimension smaller than a row (lda=%lld ldb=%lld)",
                             (long long)lda, (long long)ldb);
        GemmArgs g;
        memset(&g, 0, sizeof(g));
        g.A = A;
        g.B = B;
        g.M = M;
        g.N = N;
        g.K = K;
        g.lda = lda;
        g.ldb = ldb;
        g.sA = strideA;
        g.sB = strideB;
        g.batch = batch;
        g.alpha = 1.0;
        g.E1 = E1;
        g.E2 = E2;
        for (int k = 0; k < 5; ++k) {
            g.e1s[k] = e1_strides[k];
            g.e2s[k] = E2 ? e2_strides[k] : 0;
        }
        g.mdiv = make_fastdiv((uint32_t)mlo);
        g.ndiv = make_fastdiv((uint32_t)nlo);
        g.partial = static_cast<double*>(workspace);
        const int rc = gemm_dot_dispatch(dtype, transA != 0, transB != 0, g, st, &nparts);
        if (rc != TT_OK) return rc;
    }
    if (dtype == TT_F64)
        hipLaunchKernelGGL(dot_finalize_kernel<double>, dim3(1), dim3(256), 0, st, (const double*)workspace, nparts,
                           alpha, beta, static_cast<const double*>(C), static_cast<double*>(out));
    else
        hipLaunchKernelGGL(dot_finalize_kernel<float>, dim3(1), dim3(256), 0, st, (const double*)workspace, nparts,
                           alpha, beta, static_cast<const float*>(C), static_cast<float*>(out));
    return check_launch("tt_gemm_dot");
}
