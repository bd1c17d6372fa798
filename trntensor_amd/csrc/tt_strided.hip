// Strided multiply-reduce for contractions without a GEMM shape:
//   D[o] = alpha * sum_r A[a_off(o) + a_roff(r)] * B[b_off(o) + b_roff(r)] (+ beta * C[o])
//
// Four schedules, chosen on the host from extents and strides:
//  - per output: one thread per output element, grid-stride (many outputs:
//    outer products, elementwise products, short per-output reductions);
//  - per block: one workgroup per (output, reduction slice) (few outputs,
//    long reductions over the operands' contiguous dimension: dots, traces):
//    256 threads stride the slice, reduce with wavefront shuffles, and either
//    finish the output or write a partial that a second kernel sums in a
//    fixed order;
//  - column tiles: 256 consecutive outputs per workgroup times reduction
//    slices, when the output's innermost dimension is the operands'
//    contiguous one ('ijk->k'): each thread reduces one output over a slice,
//    so every load instruction reads consecutive addresses; partials as above;
//  - transpose tiles: a single-operand permutation whose output innermost
//    dimension is not the operand's contiguous one ('ijk->kji'): 64 x 64
//    tiles pass through LDS so both the reads and the writes are coalesced.
// Multi-indices are decoded with precomputed fast-division multipliers; the
// host splits any launch whose index range would reach 2^31.
#include "tt_common.hpp"

namespace tt {

struct Dims {
    int n;
    FastDiv div[TT_MAX_DIMS];  // extents, innermost last
    int64_t sa[TT_MAX_DIMS];
    int64_t sb[TT_MAX_DIMS];
};

// Offsets of linear index `lin` (< 2^31) into A and B.
__device__ __forceinline__ void decode(uint32_t lin, const Dims& d, int64_t& oa, int64_t& ob) {
    oa = 0;
    ob = 0;
    for (int k = d.n - 1; k >= 0; --k) {
        const uint32_t q = fdiv(lin, d.div[k]);
        const uint32_t idx = lin - q * d.div[k].d;
        oa += (int64_t)idx * d.sa[k];
        ob += (int64_t)idx * d.sb[k];
        lin = q;
    }
}

struct StridedArgs {
    const void* A;
    const void* B;  // nullptr: factor 1
    const void* C;  // nullptr: no beta term
    void* D;
    void* partial;  // nsplit * n_out elements of T, or nullptr
    Dims out, red;
    int64_t n_out;  // outputs in this launch (< 2^31)
    int64_t n_red;  // reduction length (< 2^31)
    int64_t nsplit;
    double alpha, beta;
};

// Accumulator of one output: plain sum in T, or double-double (Dot2) for
// TT_F64_DD, whose partial sums travel as (p, s) pairs.
template <typename T, bool DD>
struct Acc;

template <typename T>
struct Acc<T, false> {
    T v = T(0);
    __device__ __forceinline__ void add_prod(T x, T y) { v += x * y; }
    __device__ __forceinline__ void add(T x) { v += x; }
    __device__ __forceinline__ void wave_reduce() {
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    }
    __device__ __forceinline__ void put(double* red, int w) const { red[w] = (double)v; }
    // Four wave totals in a fixed order.
    __device__ __forceinline__ void take4(const double* red) { v = ((T)red[0] + (T)red[1]) + ((T)red[2] + (T)red[3]); }
    __device__ __forceinline__ void store_partial(void* P, int64_t idx, int64_t plane) const {
        (void)plane;
        static_cast<T*>(P)[idx] = v;
    }
    __device__ __forceinline__ void add_partial(const void* P, int64_t idx, int64_t plane) {
        (void)plane;
        v += static_cast<const T*>(P)[idx];
    }
    __device__ __forceinline__ T value() const { return v; }
};

// int64: two's-complement wraparound (unsigned arithmetic), so every
// integer dtype computed through int64 and truncated back equals its own
// wrapping accumulation. Wave totals travel bit-exactly through the double
// scratch slots.
template <>
struct Acc<int64_t, false> {
    uint64_t v = 0;
    __device__ __forceinline__ void add_prod(int64_t x, int64_t y) { v += (uint64_t)x * (uint64_t)y; }
    __device__ __forceinline__ void add(int64_t x) { v += (uint64_t)x; }
    __device__ __forceinline__ void wave_reduce() {
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v += (uint64_t)__shfl_xor((long long)v, off, 64);
    }
    __device__ __forceinline__ void put(double* red, int w) const { red[w] = __longlong_as_double((long long)v); }
    __device__ __forceinline__ void take4(const double* red) {
        v = ((uint64_t)__double_as_longlong(red[0]) + (uint64_t)__double_as_longlong(red[1])) +
            ((uint64_t)__double_as_longlong(red[2]) + (uint64_t)__double_as_longlong(red[3]));
    }
    __device__ __forceinline__ void store_partial(void* P, int64_t idx, int64_t plane) const {
        (void)plane;
        static_cast<int64_t*>(P)[idx] = (int64_t)v;
    }
    __device__ __forceinline__ void add_partial(const void* P, int64_t idx, int64_t plane) {
        (void)plane;
        v += (uint64_t) static_cast<const int64_t*>(P)[idx];
    }
    __device__ __forceinline__ int64_t value() const { return (int64_t)v; }
};

template <>
struct Acc<double, true> : Dot2 {
    __device__ __forceinline__ void wave_reduce() {
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const double op = __shfl_xor(p, off, 64);
            const double os = __shfl_xor(s, off, 64);
            merge(op, os);
        }
    }
    __device__ __forceinline__ void put(double* red, int w) const {
        red[w] = p;
        red[4 + w] = s;
    }
    __device__ __forceinline__ void take4(const double* red) {
        p = red[0];
        s = red[4];
        for (int w = 1; w < 4; ++w) merge(red[w], red[4 + w]);
    }
    // p in plane 0, s in plane 1 (plane = nsplit * n_out doubles).
    __device__ __forceinline__ void store_partial(void* P, int64_t idx, int64_t plane) const {
        static_cast<double*>(P)[idx] = p;
        static_cast<double*>(P)[plane + idx] = s;
    }
    __device__ __forceinline__ void add_partial(const void* P, int64_t idx, int64_t plane) {
        merge(static_cast<const double*>(P)[idx], static_cast<const double*>(P)[plane + idx]);
    }
};

// acc += sum over r = r0, r0 + step, ... < r1 of A[oa + a_roff(r)] (* B[ob + b_roff(r)]),
// in that order. The loads of four consecutive terms are issued before their
// sums (the order of the sums is unchanged, so results are bit-identical to a
// plain loop): each thread keeps four loads in flight instead of one on these
// memory-bound loops ('ijk->i' and 'ijk->k' on 1 GiB: +13%).
template <typename T, bool DD>
__device__ __forceinline__ void reduce_range(Acc<T, DD>& acc, const T* __restrict__ A, const T* __restrict__ B,
                                             int64_t oa, int64_t ob, const Dims& red, int64_t r0, int64_t r1,
                                             int64_t step) {
    int64_t r = r0;
    for (; r + 3 * step < r1; r += 4 * step) {
        T x[4], y[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            int64_t ra, rb;
            decode((uint32_t)(r + u * step), red, ra, rb);
            x[u] = A[oa + ra];
            if (B) y[u] = B[ob + rb];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (B) acc.add_prod(x[u], y[u]);
            else acc.add(x[u]);
        }
    }
    for (; r < r1; r += step) {
        int64_t ra, rb;
        decode((uint32_t)r, red, ra, rb);
        const T x = A[oa + ra];
        if (B) acc.add_prod(x, B[ob + rb]);
        else acc.add(x);
    }
}

// alpha * v (+ beta * c). For int64 the host admits only integral alpha and
// beta, applied with wraparound.
__device__ __forceinline__ int64_t scale(int64_t v, double alpha) {
    return (int64_t)((uint64_t)v * (uint64_t)(int64_t)alpha);
}
template <typename T>
__device__ __forceinline__ T scale(T v, double alpha) {
    return (T)alpha * v;
}
__device__ __forceinline__ int64_t add_scaled(int64_t v, double beta, int64_t c) {
    return (int64_t)((uint64_t)v + (uint64_t)(int64_t)beta * (uint64_t)c);
}
template <typename T>
__device__ __forceinline__ T add_scaled(T v, double beta, T c) {
    return v + (T)beta * c;
}

template <typename T, bool DD>
__device__ __forceinline__ T finish(const StridedArgs& g, int64_t o, const Acc<T, DD>& acc) {
    T v = acc.value();
    if (g.alpha != 1.0) v = scale(v, g.alpha);
    if (g.C) v = add_scaled(v, g.beta, static_cast<const T*>(g.C)[o]);
    return v;
}

template <typename T, bool DD>
__global__ __launch_bounds__(256) void strided_per_output_kernel(StridedArgs g) {
    const T* A = static_cast<const T*>(g.A);
    const T* B = static_cast<const T*>(g.B);
    T* D = static_cast<T*>(g.D);
    for (int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x; o < g.n_out; o += (int64_t)gridDim.x * 256) {
        int64_t oa, ob;
        decode((uint32_t)o, g.out, oa, ob);
        Acc<T, DD> acc;
        reduce_range<T, DD>(acc, A, B, oa, ob, g.red, 0, g.n_red, 1);
        D[o] = finish<T, DD>(g, o, acc);
    }
}

// Grid: (n_out, nsplit). Workgroup (o, s) reduces r = s*256 + t + k*nsplit*256.
template <typename T, bool DD>
__global__ __launch_bounds__(256) void strided_per_block_kernel(StridedArgs g) {
    __shared__ double red[8];
    const T* A = static_cast<const T*>(g.A);
    const T* B = static_cast<const T*>(g.B);
    const int64_t o = blockIdx.x;
    const int64_t s = blockIdx.y;
    int64_t oa, ob;
    decode((uint32_t)o, g.out, oa, ob);
    Acc<T, DD> acc;
    reduce_range<T, DD>(acc, A, B, oa, ob, g.red, s * 256 + threadIdx.x, g.n_red, g.nsplit * 256);
    // Block sum: wavefront shuffles, then the four wave totals in order.
    acc.wave_reduce();
    if ((threadIdx.x & 63) == 0) acc.put(red, threadIdx.x >> 6);
    __syncthreads();
    if (threadIdx.x == 0) {
        Acc<T, DD> tot;
        tot.take4(red);
        if (g.nsplit == 1) static_cast<T*>(g.D)[o] = finish<T, DD>(g, o, tot);
        else tot.store_partial(g.partial, s * g.n_out + o, g.nsplit * g.n_out);
    }
}

template <typename T, bool DD>
__global__ __launch_bounds__(256) void strided_finish_kernel(StridedArgs g) {
    __shared__ double red[8];
    const int64_t o = blockIdx.x;
    Acc<T, DD> acc;
    for (int64_t s = threadIdx.x; s < g.nsplit; s += 256) acc.add_partial(g.partial, s * g.n_out + o, g.nsplit * g.n_out);
    acc.wave_reduce();
    if ((threadIdx.x & 63) == 0) acc.put(red, threadIdx.x >> 6);
    __syncthreads();
    if (threadIdx.x == 0) {
        Acc<T, DD> tot;
        tot.take4(red);
        static_cast<T*>(g.D)[o] = finish<T, DD>(g, o, tot);
    }
}

// Grid: (ceil(n_out / 256), nsplit). Thread t of workgroup (x, s) reduces
// output 256 x + t over the s-th contiguous slice of the reduction range.
template <typename T, bool DD>
__global__ __launch_bounds__(256) void strided_coltile_kernel(StridedArgs g) {
    const int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (o >= g.n_out) return;
    const T* A = static_cast<const T*>(g.A);
    const T* B = static_cast<const T*>(g.B);
    int64_t oa, ob;
    decode((uint32_t)o, g.out, oa, ob);
    const int64_t chunk = (g.n_red + g.nsplit - 1) / g.nsplit;
    const int64_t r0 = (int64_t)blockIdx.y * chunk;
    const int64_t r1 = min(g.n_red, r0 + chunk);
    Acc<T, DD> acc;
    reduce_range<T, DD>(acc, A, B, oa, ob, g.red, r0, r1, 1);
    if (g.nsplit == 1) static_cast<T*>(g.D)[o] = finish<T, DD>(g, o, acc);
    else acc.store_partial(g.partial, (int64_t)blockIdx.y * g.n_out + o, g.nsplit * g.n_out);
}

// Permutation through LDS. Output dimension u is the output's innermost
// (D stride 1), v the dimension along which A is contiguous; the remaining
// output dimensions form `bat` (A and D strides). Workgroup: one TS (u) x TS
// (v) tile of one batch index; threads read along v and write along u.
struct TransArgs {
    int64_t U, V;      // extents of u and v
    int64_t sa_u, sa_v, sd_v;
    int64_t tiles_u, tiles_v;
    Dims bat;          // sa = A strides, sb = D strides
};

template <typename T, int TS>
__global__ __launch_bounds__(256) void strided_transpose_kernel(StridedArgs g, TransArgs t) {
    constexpr int RP = 256 / TS;       // tile rows per pass of the 256 threads
    constexpr int NE = TS * TS / 256;  // elements per thread
    __shared__ T tile[TS][TS + 1];
    const int64_t per = t.tiles_u * t.tiles_v;
    const int64_t z = blockIdx.x / per;
    const int64_t rem = blockIdx.x - z * per;
    const int64_t u0 = (rem % t.tiles_u) * TS;
    const int64_t v0 = (rem / t.tiles_u) * TS;
    int64_t za, zd;
    decode((uint32_t)z, t.bat, za, zd);
    const T* A = static_cast<const T*>(g.A);
    const int lo = threadIdx.x % TS;
    const int hi = threadIdx.x / TS;
    // All loads of a thread are issued before its LDS stores, branch-free
    // (an element outside the tensor loads the batch's first element, which
    // always exists, into a tile cell that is never stored): loads inside
    // per-element bounds branches were each followed by a wait, one memory
    // latency per element.
    T x[NE];
#pragma unroll
    for (int i = 0; i < NE; ++i) {
        const int ul = hi + RP * i;
        const int64_t u = u0 + ul, v = v0 + lo;
        const bool ok = u < t.U && v < t.V;
        x[i] = A[ok ? za + u * t.sa_u + v * t.sa_v : za];
    }
#pragma unroll
    for (int i = 0; i < NE; ++i) tile[hi + RP * i][lo] = x[i];
    __syncthreads();
    T* D = static_cast<T*>(g.D);
    const T* C = static_cast<const T*>(g.C);
    // The beta term's C values are likewise loaded before the first store (D
    // may alias C element for element).
    T c[NE];
    if (C) {
#pragma unroll
        for (int i = 0; i < NE; ++i) {
            const int vl = hi + RP * i;
            const int64_t u = u0 + lo, v = v0 + vl;
            const bool ok = u < t.U && v < t.V;
            c[i] = C[ok ? zd + v * t.sd_v + u : zd];
        }
    }
#pragma unroll
    for (int i = 0; i < NE; ++i) {
        const int vl = hi + RP * i;
        const int64_t u = u0 + lo, v = v0 + vl;
        if (u < t.U && v < t.V) {
            T y = tile[lo][vl];
            if (g.alpha != 1.0) y = scale(y, g.alpha);
            if (C) y = add_scaled(y, g.beta, c[i]);
            D[zd + v * t.sd_v + u] = y;
        }
    }
}

// Host-side schedule choice. The workspace query sees only extents, so it
// reserves the larger partial buffer of the two split schedules the extents
// allow; the launch then picks with the strides.
enum Kind { PER_OUTPUT, PER_BLOCK, COLTILE, TRANSPOSE };

struct Plan {
    Kind kind;
    int64_t nsplit;
};

static int64_t per_block_split(int64_t n_out, int64_t n_red) {
    // Enough workgroups to fill 256 CUs several times, each at least 2K elements.
    int64_t want = (4096 + n_out - 1) / n_out;
    int64_t cap = (n_red + 2047) / 2048;
    int64_t n = want < cap ? want : cap;
    return n < 1 ? 1 : (n > 65535 ? 65535 : n);
}

static int64_t coltile_split(int64_t n_out, int64_t n_red) {
    // ~2048 workgroups in all, each thread at least 64 reduction elements.
    const int64_t bx = (n_out + 255) / 256;
    int64_t want = (2048 + bx - 1) / bx;
    int64_t cap = (n_red + 63) / 64;
    int64_t n = want < cap ? want : cap;
    return n < 1 ? 1 : (n > 65535 ? 65535 : n);
}

constexpr int64_t kColtileMaxOut = 1 << 18;

static bool per_block_fits(int64_t n_out, int64_t n_red) { return n_red > 1 && n_out < 8192; }
static bool coltile_fits(int64_t n_out, int64_t n_red) { return n_red > 1 && n_out < kColtileMaxOut; }

static Plan choose(const StridedArgs& g) {
    const int last = g.out.n - 1;
    const bool out_contig = last >= 0 && g.out.sa[last] == 1 && (!g.B || g.out.sb[last] == 0 || g.out.sb[last] == 1);
    if (g.red.n == 0 && !g.B && g.out.n >= 2 && g.n_out >= 4096 && g.out.sa[last] != 1) {
        for (int k = 0; k < last; ++k)
            if (g.out.sa[k] == 1) return Plan{TRANSPOSE, 1};
    }
    if (out_contig && coltile_fits(g.n_out, g.n_red)) return Plan{COLTILE, coltile_split(g.n_out, g.n_red)};
    if (per_block_fits(g.n_out, g.n_red)) return Plan{PER_BLOCK, per_block_split(g.n_out, g.n_red)};
    return Plan{PER_OUTPUT, 1};
}

static int64_t prod(int n, const int64_t* s) {
    int64_t r = 1;
    for (int k = 0; k < n; ++k) r *= s[k];
    return r;
}

template <typename T>
static int launch_transpose(StridedArgs& g, const int64_t* out_shape, hipStream_t st) {
    const int last = g.out.n - 1;
    int v = -1;
    for (int k = 0; k < last; ++k)
        if (g.out.sa[k] == 1) {
            v = k;
            break;
        }
    int64_t dstride[TT_MAX_DIMS];
    int64_t acc = 1;
    for (int k = last; k >= 0; --k) {
        dstride[k] = acc;
        acc *= out_shape[k];
    }
    TransArgs t;
    t.U = out_shape[last];
    t.V = out_shape[v];
    t.sa_u = g.out.sa[last];
    t.sa_v = g.out.sa[v];
    t.sd_v = dstride[v];
    // 4-byte elements on 128 x 128 tiles (512-byte rows on both sides; 'ij->ji'
    // f32 16384^2, same box, alternating: 0.416 against 0.469 ms on 64 x 64,
    // 0.626 ms on 32 x 32); 8-byte ones on 64 x 64 (already 512-byte rows).
    constexpr int TS = sizeof(T) == 4 ? 128 : 64;
    t.tiles_u = (t.U + TS - 1) / TS;
    t.tiles_v = (t.V + TS - 1) / TS;
    t.bat.n = 0;
    int64_t nbat = 1;
    for (int k = 0; k < last; ++k) {
        if (k == v) continue;
        const int b = t.bat.n++;
        t.bat.div[b] = make_fastdiv((uint32_t)out_shape[k]);
        t.bat.sa[b] = g.out.sa[k];
        t.bat.sb[b] = dstride[k];
        nbat *= out_shape[k];
    }
    const int64_t blocks = t.tiles_u * t.tiles_v * nbat;
    if (blocks > 0x7fffffffLL) return set_error(TT_UNSUPPORTED, "tt_strided_contract: %lld tiles", (long long)blocks);
    hipLaunchKernelGGL((strided_transpose_kernel<T, TS>), dim3((unsigned)blocks), dim3(256), 0, st, g, t);
    return TT_OK;
}

template <typename T, bool DD>
static int run_typed(StridedArgs g, const int64_t* out_shape, hipStream_t st) {
    const Plan pl = choose(g);
    g.nsplit = pl.nsplit;
    if (pl.kind == TRANSPOSE) {
        const int rc = launch_transpose<T>(g, out_shape, st);
        if (rc != TT_OK) return rc;
    } else if (pl.kind == PER_OUTPUT) {
        int64_t blocks = (g.n_out + 255) / 256;
        if (blocks > 1 << 20) blocks = 1 << 20;
        if (blocks > 0) hipLaunchKernelGGL((strided_per_output_kernel<T, DD>), dim3((unsigned)blocks), dim3(256), 0, st, g);
    } else if (pl.kind == COLTILE) {
        const unsigned bx = (unsigned)((g.n_out + 255) / 256);
        hipLaunchKernelGGL((strided_coltile_kernel<T, DD>), dim3(bx, (unsigned)g.nsplit), dim3(256), 0, st, g);
        if (g.nsplit > 1) hipLaunchKernelGGL((strided_finish_kernel<T, DD>), dim3((unsigned)g.n_out), dim3(256), 0, st, g);
    } else {
        hipLaunchKernelGGL((strided_per_block_kernel<T, DD>), dim3((unsigned)g.n_out, (unsigned)g.nsplit), dim3(256), 0, st, g);
        if (g.nsplit > 1) hipLaunchKernelGGL((strided_finish_kernel<T, DD>), dim3((unsigned)g.n_out), dim3(256), 0, st, g);
    }
    return check_launch("tt_strided_contract");
}

}  // namespace tt

extern "C" size_t tt_strided_contract_workspace_bytes(int dtype, int n_out, const int64_t* out_shape, int n_red,
                                                      const int64_t* red_shape) {
    using namespace tt;
    if (n_out < 0 || n_red < 0 || n_out > TT_MAX_DIMS || n_red > TT_MAX_DIMS) return 0;
    const int64_t no = prod(n_out, out_shape), nr = prod(n_red, red_shape);
    int64_t parts = 0;
    if (per_block_fits(no, nr)) parts = per_block_split(no, nr);
    if (coltile_fits(no, nr)) {
        const int64_t c = coltile_split(no, nr);
        parts = c > parts ? c : parts;
    }
    if (parts <= 1) return 0;
    // TT_F64_DD partials are (p, s) pairs of doubles.
    const size_t es = dtype == TT_F64_DD ? 16 : (dtype == TT_F64 || dtype == TT_I64) ? 8 : 4;
    return ((size_t)(parts * no) * es + 255) / 256 * 256;
}

extern "C" int tt_strided_contract(int dtype, int n_out, const int64_t* out_shape, const int64_t* a_out_strides,
                                   const int64_t* b_out_strides, int n_red, const int64_t* red_shape,
                                   const int64_t* a_red_strides, const int64_t* b_red_strides, const void* A,
                                   const void* B, double alpha, double beta, const void* C, void* D, void* workspace,
                                   size_t workspace_bytes, void* stream) {
    using namespace tt;
    if (n_out < 0 || n_red < 0 || n_out > TT_MAX_DIMS || n_red > TT_MAX_DIMS)
        return set_error(TT_INVALID, "tt_strided_contract: dims out=%d red=%d (max %d)", n_out, n_red, TT_MAX_DIMS);
    if (dtype != TT_F32 && dtype != TT_F64 && dtype != TT_F64_DD && dtype != TT_I64)
        return set_error(TT_UNSUPPORTED, "tt_strided_contract: dtype %d (only TT_F32, TT_F64, TT_F64_DD, TT_I64)",
                         dtype);
    if (dtype == TT_I64) {
        auto integral = [](double x) { return x >= -9.2e18 && x <= 9.2e18 && x == (double)(int64_t)x; };
        if (!integral(alpha) || !integral(beta))
            return set_error(TT_INVALID, "tt_strided_contract: TT_I64 takes integral alpha and beta (got %g, %g)",
                             alpha, beta);
    }
    for (int k = 0; k < n_out; ++k)
        if (out_shape[k] < 0) return set_error(TT_INVALID, "tt_strided_contract: negative output extent");
    for (int k = 0; k < n_red; ++k)
        if (red_shape[k] < 0) return set_error(TT_INVALID, "tt_strided_contract: negative reduction extent");
    const int64_t no = prod(n_out, out_shape), nr = prod(n_red, red_shape);
    if (no == 0) return TT_OK;
    if (!A || !D) return set_error(TT_INVALID, "tt_strided_contract: A or D is NULL");
    if (no >= (1LL << 31) || nr >= (1LL << 31))
        return set_error(TT_UNSUPPORTED, "tt_strided_contract: index range %lld x %lld reaches 2^31; split the call",
                         (long long)no, (long long)nr);
    const size_t need = tt_strided_contract_workspace_bytes(dtype, n_out, out_shape, n_red, red_shape);
    if (need > 0 && (!workspace || workspace_bytes < need))
        return set_error(TT_INVALID, "tt_strided_contract: workspace of %zu bytes, need %zu", workspace_bytes, need);

    StridedArgs g;
    g.A = A;
    g.B = B;
    g.C = C;
    g.D = D;
    g.partial = workspace;
    g.n_out = no;
    g.n_red = nr;
    g.alpha = alpha;
    g.beta = beta;
    g.out.n = n_out;
    for (int k = 0; k < n_out; ++k) {
        g.out.div[k] = make_fastdiv((uint32_t)(out_shape[k] > 0 ? out_shape[k] : 1));
        g.out.sa[k] = a_out_strides[k];
        g.out.sb[k] = B ? b_out_strides[k] : 0;
    }
    g.red.n = n_red;
    for (int k = 0; k < n_red; ++k) {
        g.red.div[k] = make_fastdiv((uint32_t)(red_shape[k] > 0 ? red_shape[k] : 1));
        g.red.sa[k] = a_red_strides[k];
        g.red.sb[k] = B ? b_red_strides[k] : 0;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (nr == 0) {
        // Empty reduction: every output is alpha * 0 (+ beta * C).
        g.n_red = 0;
    }
    if (dtype == TT_F64_DD) return run_typed<double, true>(g, out_shape, st);
    if (dtype == TT_F64) return run_typed<double, false>(g, out_shape, st);
    if (dtype == TT_I64) return run_typed<int64_t, false>(g, out_shape, st);
    return run_typed<float, false>(g, out_shape, st);
}
