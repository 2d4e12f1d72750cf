// MI355X (gfx950) neighbor-list library: device geometry, binning, counting
// and emission kernels plus the C ABI declared in include/tonari_hip.h.
//
// Pipeline of one request (all on the caller's stream):
//   tnr_count: k_zero -> k_setup (per structure: batch_ptr checks, active
//              pseudo-inverse, image repeats, grid frame) -> k_atoms (per atom:
//              wraps, wrapped position, bounds) -> k_plan (per structure:
//              margins, algorithm, bin grid) -> scan(bins per structure) ->
//              k_bin -> scan(bin counts) -> k_scatter -> k_cell<count> +
//              k_brute<count> -> scan(pairs per source) -> k_finish -> one
//              4-word device-to-host copy and a stream sync (E).
//   tnr_emit:  k_cell<emit> + k_brute<emit> write i/j/P/S/d/D in place.
//
// Reference semantics (songfeitong/tonari):
//   the public predicate             csrc/core/neighbors_cpu.cpp:247-261
//   S = image - wrap_t + wrap_s      csrc/core/neighbors_cpu.cpp:236-241
//   identity policy                  csrc/core/pair_policy.h:42-79
//   periodic metadata                csrc/core/geometry.cpp:123-219
//   error messages and types         csrc/torch/bindings_cuda.cpp:69-118,
//                                    csrc/torch/neighbors_cuda.cu:513-521
//
// Every kernel is compiled with -ffp-contract=off; the broad phase asks for
// fused multiply-adds explicitly, the exact predicate uses the _rn
// intrinsics so that its rounding sequence is the reference's.

#include "nl_device.h"

#include "../../include/tonari_hip.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <limits>

namespace tnr {

// --------------------------------------------------------------- scalar ops

template <typename T>
struct Ops;

template <>
struct Ops<float> {
    static constexpr double eps = 1.1920928955078125e-07;
    static constexpr double max = 3.4028234663852886e+38;
    __device__ static float add(float a, float b) { return __fadd_rn(a, b); }
    __device__ static float sub(float a, float b) { return __fsub_rn(a, b); }
    __device__ static float mul(float a, float b) { return __fmul_rn(a, b); }
    __device__ static float fma_(float a, float b, float c) { return __fmaf_rn(a, b, c); }
    __device__ static float sqrt_(float a) { return __fsqrt_rn(a); }
    // Nearest float not below / not above x.
    __device__ static float down(double x) {
        float f = (float)x;
        if ((double)f > x) f = nextafterf(f, -INFINITY);
        return f;
    }
    __device__ static float up(double x) {
        float f = (float)x;
        if ((double)f < x) f = nextafterf(f, INFINITY);
        return f;
    }
};

template <>
struct Ops<double> {
    static constexpr double eps = 2.220446049250313e-16;
    static constexpr double max = 1.7976931348623157e+308;
    __device__ static double add(double a, double b) { return __dadd_rn(a, b); }
    __device__ static double sub(double a, double b) { return __dsub_rn(a, b); }
    __device__ static double mul(double a, double b) { return __dmul_rn(a, b); }
    __device__ static double fma_(double a, double b, double c) { return __fma_rn(a, b, c); }
    __device__ static double sqrt_(double a) { return __dsqrt_rn(a); }
    __device__ static double down(double x) { return x; }
    __device__ static double up(double x) { return x; }
};

template <typename T>
struct alignas(4 * sizeof(T)) Vec4 {
    T x, y, z, w;
};

__device__ __forceinline__ float idx_as(int i, float) { return __int_as_float(i); }
__device__ __forceinline__ double idx_as(int i, double) { return (double)i; }
__device__ __forceinline__ int as_idx(float v) { return __float_as_int(v); }
__device__ __forceinline__ int as_idx(double v) { return (int)v; }

__device__ __forceinline__ unsigned long long load_status(const unsigned long long* s) {
    return __atomic_load_n(s, __ATOMIC_RELAXED);
}

__device__ __forceinline__ long long floor_div(long long a, long long b) {
    long long q = a / b;
    if ((a % b != 0) && ((a < 0) != (b < 0))) --q;
    return q;
}

// The public predicate of the reference (neighbors_cpu.cpp:247-261): every
// product and sum rounded in T, in this order.  Returns d2 and writes D.
template <typename T>
__device__ __forceinline__ T public_vector(const T ps[3], const T pt[3], long long S0,
                                           long long S1, long long S2, const T* cell,
                                           T D[3]) {
    using O = Ops<T>;
    const T s0 = (T)S0, s1 = (T)S1, s2 = (T)S2;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        T comp = O::sub(pt[c], ps[c]);
        comp = O::add(comp, O::mul(s0, cell[c]));
        comp = O::add(comp, O::mul(s1, cell[3 + c]));
        comp = O::add(comp, O::mul(s2, cell[6 + c]));
        D[c] = comp;
    }
    T d2 = O::mul(D[0], D[0]);
    d2 = O::add(d2, O::mul(D[1], D[1]));
    d2 = O::add(d2, O::mul(D[2], D[2]));
    return d2;
}

// ----------------------------------------------------------- block helpers

__device__ __forceinline__ long long wave_inclusive_scan(long long x) {
    const int lane = lane_id();
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const long long y = __shfl_up(x, d);
        if (lane >= d) x += y;
    }
    return x;
}

__device__ __forceinline__ long long wave_sum(long long x) {
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1) x += __shfl_xor(x, d);
    return x;
}

// Exclusive scan over the 256 threads of a block; *total receives the sum.
__device__ __forceinline__ long long block_exclusive_scan(long long x, long long* total) {
    __shared__ long long wave_tot[kWavesPerBlock];
    const int lane = lane_id();
    const int w = threadIdx.x / kWave;
    const long long inc = wave_inclusive_scan(x);
    if (lane == kWave - 1) wave_tot[w] = inc;
    __syncthreads();
    long long before = 0, all = 0;
#pragma unroll
    for (int i = 0; i < kWavesPerBlock; ++i) {
        if (i < w) before += wave_tot[i];
        all += wave_tot[i];
    }
    __syncthreads();
    *total = all;
    return before + inc - x;
}

// ------------------------------------------------------------- fill / scan

__global__ void k_fill_i64(long long* p, int64_t n, long long v) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

__global__ void k_fill_i32(int* p, int64_t n, int v) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

template <typename In>
__global__ __launch_bounds__(kBlock) void k_scan_reduce(const In* in, int64_t n,
                                                         long long* partial) {
    const int64_t base = (int64_t)blockIdx.x * kScanChunk;
    long long s = 0;
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        const int64_t i = base + threadIdx.x + (int64_t)j * kBlock;
        if (i < n) s += (long long)in[i];
    }
    long long total;
    block_exclusive_scan(s, &total);
    if (threadIdx.x == 0) partial[blockIdx.x] = total;
}

// One block: exclusive scan of partial[0..np) in place, partial[np] = total.
__global__ __launch_bounds__(kBlock) void k_scan_partials(long long* partial, int64_t np) {
    __shared__ long long carry_s;
    if (threadIdx.x == 0) carry_s = 0;
    __syncthreads();
    for (int64_t base = 0; base < np; base += kBlock) {
        const int64_t i = base + threadIdx.x;
        const long long v = i < np ? partial[i] : 0;
        long long total;
        const long long ex = block_exclusive_scan(v, &total);
        const long long carry = carry_s;
        if (i < np) partial[i] = carry + ex;
        __syncthreads();
        if (threadIdx.x == 0) carry_s = carry + total;
        __syncthreads();
    }
    if (threadIdx.x == 0) partial[np] = carry_s;
}

template <typename In, typename Out>
__global__ __launch_bounds__(kBlock) void k_scan_apply(const In* in, int64_t n,
                                                        const long long* partial,
                                                        int64_t np, Out* out) {
    const int64_t base = (int64_t)blockIdx.x * kScanChunk + (int64_t)threadIdx.x * kScanItems;
    long long v[kScanItems];
    long long s = 0;
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        const int64_t i = base + j;
        v[j] = i < n ? (long long)in[i] : 0;
        s += v[j];
    }
    long long total;
    long long run = block_exclusive_scan(s, &total) +
                    (blockIdx.x < np ? partial[blockIdx.x] : 0);
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        const int64_t i = base + j;
        if (i < n) out[i] = (Out)run;
        run += v[j];
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) out[n] = (Out)partial[np];
}

template <typename In, typename Out>
static hipError_t device_scan(const In* in, int64_t n, Out* out, long long* partial,
                              hipStream_t stream) {
    const int64_t np = (n + kScanChunk - 1) / kScanChunk;
    if (np > 0) k_scan_reduce<In><<<dim3((unsigned)np), dim3(kBlock), 0, stream>>>(in, n, partial);
    k_scan_partials<<<1, kBlock, 0, stream>>>(partial, np);
    k_scan_apply<In, Out><<<dim3((unsigned)(np > 0 ? np : 1)), dim3(kBlock), 0, stream>>>(
        in, n, partial, np, out);
    return hipGetLastError();
}

// ----------------------------------------------------------------- geometry

// Active-row pseudo-inverse by one-sided (Hestenes) Jacobi in float64, the
// algorithm of geometry.cpp:15-118 carried out in double instead of long
// double.  Returns false when the active rows are linearly dependent.
__device__ bool active_pinv(const double* cell, const int* axes, int k, double dual[3][3]) {
    double w[3][3] = {}, v[3][3] = {};
    for (int j = 0; j < k; ++j) {
        v[j][j] = 1.0;
        for (int c = 0; c < 3; ++c) w[c][j] = cell[3 * axes[j] + c];
    }
    const double eps = 2.220446049250313e-16;
    for (int sweep = 0; sweep < 64; ++sweep) {
        bool rotated = false;
        for (int p = 0; p < k; ++p)
            for (int q = p + 1; q < k; ++q) {
                double app = 0, aqq = 0, apq = 0;
                for (int c = 0; c < 3; ++c) {
                    app += w[c][p] * w[c][p];
                    aqq += w[c][q] * w[c][q];
                    apq += w[c][p] * w[c][q];
                }
                if (fabs(apq) <= 8 * eps * sqrt(app * aqq)) continue;
                rotated = true;
                const double zeta = (aqq - app) / (2 * apq);
                const double t = zeta == 0.0
                                     ? 1.0
                                     : copysign(1.0, zeta) / (fabs(zeta) + hypot(1.0, zeta));
                const double cs = 1.0 / hypot(1.0, t);
                const double sn = cs * t;
                for (int c = 0; c < 3; ++c) {
                    const double a = w[c][p], b = w[c][q];
                    w[c][p] = cs * a - sn * b;
                    w[c][q] = sn * a + cs * b;
                }
                for (int r = 0; r < k; ++r) {
                    const double a = v[r][p], b = v[r][q];
                    v[r][p] = cs * a - sn * b;
                    v[r][q] = sn * a + cs * b;
                }
            }
        if (!rotated) break;
    }
    double sig[3] = {}, smax = 0, smin = INFINITY;
    for (int j = 0; j < k; ++j) {
        double s2 = 0;
        for (int c = 0; c < 3; ++c) s2 += w[c][j] * w[c][j];
        sig[j] = sqrt(s2);
        smax = fmax(smax, sig[j]);
        smin = fmin(smin, sig[j]);
    }
    if (!(smin > eps * 3 * fmax(smax, 1.0))) return false;
    for (int c = 0; c < 3; ++c)
        for (int a = 0; a < k; ++a) {
            double acc = 0;
            for (int j = 0; j < k; ++j) acc += w[c][j] * v[a][j] / (sig[j] * sig[j]);
            dual[c][a] = acc;
        }
    return true;
}

__device__ inline void cross3(const double* a, const double* b, double* o) {
    o[0] = a[1] * b[2] - a[2] * b[1];
    o[1] = a[2] * b[0] - a[0] * b[2];
    o[2] = a[0] * b[1] - a[1] * b[0];
}

__device__ inline bool normalize3(double* v) {
    const double n = sqrt(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
    if (!(n > 0) || !isfinite(n)) return false;
    v[0] /= n;
    v[1] /= n;
    v[2] /= n;
    return true;
}

// One thread per structure: batch_ptr checks, periodic metadata and the grid
// frame used for binning.  Grid rows: dual columns on periodic axes (so the
// grid coordinate is the fractional coordinate), orthonormal complements of
// the periodic rows on the other axes.
template <typename T>
__global__ void k_setup(const int64_t* bp, const T* cells, const uint8_t* pbc, int64_t nb,
                        int64_t n_atoms, double cutoff, StructRec* recs,
                        unsigned long long* status) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    unsigned long long* flags = status + SS_FLAGS;
    if (nb == 0) {
        if (b == 0) {
            unsigned long long st = 0;
            if (bp[0] != 0) st |= ST_BP_START;
            if (bp[0] != n_atoms) st |= ST_BP_END;
            if (st) atomicOr(flags, st);
        }
        return;
    }
    if (b >= nb) return;
    unsigned long long st = 0;
    const int64_t lo = bp[b], hi = bp[b + 1];
    if (b == 0 && lo != 0) st |= ST_BP_START;
    if (b == nb - 1 && hi != n_atoms) st |= ST_BP_END;
    if (hi < lo) st |= ST_BP_ORDER;

    StructRec r;
    memset(&r, 0, sizeof(r));
    r.atom0 = lo;
    r.natoms = hi > lo ? hi - lo : 0;
    for (int a = 0; a < 3; ++a) {
        r.umin[a] = r.cmin[a] = ~0ull;
        r.umax[a] = r.cmax[a] = 0ull;
    }
    double cell[9];
    bool finite = true;
    for (int e = 0; e < 9; ++e) {
        cell[e] = (double)cells[9 * b + e];
        finite = finite && isfinite(cell[e]);
    }
    if (!finite) st |= ST_CELL_NONFINITE;
    int axes[3], k = 0;
    for (int a = 0; a < 3; ++a)
        if (pbc[3 * b + a]) {
            axes[k++] = a;
            r.active |= 1 << a;
        }
    r.nimages = 1;
    if (finite && r.natoms > 0) {
        double dual[3][3] = {};
        if (k > 0 && !active_pinv(cell, axes, k, dual)) st |= ST_CELL_RANK;
        int64_t reps[3] = {0, 0, 0};
        for (int j = 0; j < k && !(st & ST_CELL_RANK); ++j) {
            double n2 = 0;
            for (int c = 0; c < 3; ++c) {
                const double x = dual[c][j];
                if (!isfinite(x)) st |= ST_DUAL_RANGE;
                r.dual[3 * c + axes[j]] = x;
                n2 += x * x;
            }
            const double rep = ceil(cutoff * sqrt(n2));
            if (!(rep <= 2147483647.0)) {
                st |= ST_REPEAT_RANGE;
            } else {
                reps[axes[j]] = (int64_t)rep;
            }
        }
        int64_t count = 1;
        for (int a = 0; a < 3 && !(st & (ST_REPEAT_RANGE | ST_CELL_RANK | ST_DUAL_RANGE)); ++a) {
            const int64_t f = 2 * reps[a] + 1;
            if (count > kImageCap / f) {
                st |= ST_IMAGE_CAP;
                break;
            }
            count *= f;
        }
        if (!(st & (ST_IMAGE_CAP | ST_REPEAT_RANGE | ST_CELL_RANK | ST_DUAL_RANGE))) {
            r.nimages = count;
            for (int a = 0; a < 3; ++a) r.reps[a] = (int32_t)reps[a];
            atomicAdd((unsigned long long*)(status + SS_TOTAL_IMAGES), (unsigned long long)count);
        }
        // Grid frame.
        double g[3][3] = {{1, 0, 0}, {0, 1, 0}, {0, 0, 1}};
        if (k >= 1) {
            for (int j = 0; j < k; ++j)
                for (int c = 0; c < 3; ++c) g[axes[j]][c] = dual[c][j];
        }
        if (k == 2) {
            int ic = 3 - axes[0] - axes[1];
            cross3(cell + 3 * axes[0], cell + 3 * axes[1], g[ic]);
            normalize3(g[ic]);
        } else if (k == 1) {
            double rr[3] = {cell[3 * axes[0]], cell[3 * axes[0] + 1], cell[3 * axes[0] + 2]};
            normalize3(rr);
            int e = 0;
            for (int c = 1; c < 3; ++c)
                if (fabs(rr[c]) < fabs(rr[e])) e = c;
            double unit[3] = {0, 0, 0};
            unit[e] = 1;
            double e1[3], e2[3];
            cross3(rr, unit, e1);
            normalize3(e1);
            cross3(rr, e1, e2);
            normalize3(e2);
            int i1 = -1, i2 = -1;
            for (int a = 0; a < 3; ++a)
                if (a != axes[0]) {
                    if (i1 < 0) i1 = a; else i2 = a;
                }
            for (int c = 0; c < 3; ++c) {
                g[i1][c] = e1[c];
                g[i2][c] = e2[c];
            }
        }
        for (int a = 0; a < 3; ++a)
            for (int c = 0; c < 3; ++c) r.grid[3 * a + c] = g[a][c];
    }
    recs[b] = r;
    if (st) atomicOr(flags, st);
}

// Structure of atom i: the b with bp[b] <= i < bp[b + 1] (batch_ptr valid).
__device__ __forceinline__ int structure_of(const int64_t* bp, int64_t nb, int64_t i) {
    int64_t lo = 0, hi = nb;  // answer in [lo, hi)
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) >> 1;
        if (bp[mid] <= i) lo = mid; else hi = mid;
    }
    return (int)lo;
}

// floor(sum_c x_c * y_c) with double-double accumulation (nearly exact), as
// the reference's long-double fractional coordinate; *ok false when the
// value is non-finite or outside [-2^31, 2^31).
__device__ __forceinline__ int wrap_of(const double x[3], const double y[3], bool* ok) {
    double hi = 0, lo = 0;
    for (int c = 0; c < 3; ++c) {
        const double p = x[c] * y[c];
        const double pe = fma(x[c], y[c], -p);
        const double s = hi + p;
        const double bb = s - hi;
        const double se = (hi - (s - bb)) + (p - bb);
        lo += pe + se;
        hi = s;
    }
    const double s = hi + lo;
    lo = lo - (s - hi);
    hi = s;
    if (!isfinite(hi)) {
        *ok = false;
        return 0;
    }
    double f = floor(hi);
    if (hi == f && lo < 0) f -= 1.0;
    if (!(f >= -2147483648.0 && f <= 2147483647.0)) {
        *ok = false;
        return 0;
    }
    return (int)f;
}

template <typename T>
__device__ __forceinline__ void grid_coords(const StructRec& r, const T q[3], double u[3]) {
    for (int a = 0; a < 3; ++a)
        u[a] = r.grid[3 * a] * (double)q[0] + r.grid[3 * a + 1] * (double)q[1] +
               r.grid[3 * a + 2] * (double)q[2];
}

__device__ __forceinline__ unsigned long long wave_min_u64(unsigned long long x) {
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1) {
        const unsigned long long y = __shfl_xor(x, d);
        x = y < x ? y : x;
    }
    return x;
}
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long x) {
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1) {
        const unsigned long long y = __shfl_xor(x, d);
        x = y > x ? y : x;
    }
    return x;
}

// One thread per atom: finiteness, representative wraps, wrapped positions
// (neighbors_cpu.cpp:92-133) and per-structure bounds.
template <typename T>
__global__ __launch_bounds__(kBlock) void k_atoms(const T* pos, const int64_t* bp, const T* cells,
                                                   int64_t nb, int64_t n_atoms, StructRec* recs,
                                                   int* atom_struct, int4* atom_wrap,
                                                   Vec4<T>* atom_q, unsigned long long* status) {
    if (load_status(status + SS_FLAGS) & kAbortBits) return;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const bool valid = i < n_atoms;
    int b = 0;
    bool good = false;
    T q[3] = {T(0), T(0), T(0)};
    int w[3] = {0, 0, 0};
    double u[3] = {0, 0, 0};
    T p[3] = {T(0), T(0), T(0)};
    unsigned long long st = 0;
    if (valid) {
        b = structure_of(bp, nb, i);
        atom_struct[i] = b;
        const StructRec& r = recs[b];
        bool finite = true;
        for (int c = 0; c < 3; ++c) {
            p[c] = pos[3 * i + c];
            finite = finite && isfinite((double)p[c]);
        }
        if (!finite) {
            st |= ST_POS_NONFINITE;
        } else {
            double pd[3] = {(double)p[0], (double)p[1], (double)p[2]};
            bool ok = true;
            for (int a = 0; a < 3; ++a) {
                double dcol[3];
                for (int c = 0; c < 3; ++c) dcol[c] = (double)(T)r.dual[3 * c + a];
                w[a] = wrap_of(pd, dcol, &ok);
            }
            if (!ok) {
                st |= ST_WRAP_RANGE;
            } else {
                const T* cell = cells + 9 * b;
                for (int c = 0; c < 3; ++c) {
                    T x = p[c];
                    for (int a = 0; a < 3; ++a)
                        x = Ops<T>::sub(x, Ops<T>::mul((T)w[a], cell[3 * a + c]));
                    q[c] = x;
                }
                grid_coords(r, q, u);
                good = true;
            }
        }
        atom_wrap[i] = make_int4(w[0], w[1], w[2], 0);
        atom_q[i] = Vec4<T>{q[0], q[1], q[2], idx_as((int)i, T(0))};
    }
    if (st) atomicOr(status + SS_FLAGS, st);

    // Per-structure reductions, aggregated over the wave when it lies in
    // one structure (the common case: structures are contiguous ranges).
    unsigned long long umin[3], umax[3], cmin[3], cmax[3], mp[3];
    unsigned mw[3];
    for (int a = 0; a < 3; ++a) {
        umin[a] = good ? order_key(u[a]) : ~0ull;
        umax[a] = good ? order_key(u[a]) : 0ull;
        cmin[a] = good ? order_key((double)q[a]) : ~0ull;
        cmax[a] = good ? order_key((double)q[a]) : 0ull;
        mp[a] = good ? (unsigned long long)__double_as_longlong(fabs((double)p[a])) : 0ull;
        mw[a] = good ? (unsigned)llabs((long long)w[a]) : 0u;
    }
    const int b0 = __shfl(b, 0);
    const bool uniform = __all(!valid || b == b0);
    if (uniform) {
        for (int a = 0; a < 3; ++a) {
            umin[a] = wave_min_u64(umin[a]);
            umax[a] = wave_max_u64(umax[a]);
            cmin[a] = wave_min_u64(cmin[a]);
            cmax[a] = wave_max_u64(cmax[a]);
            mp[a] = wave_max_u64(mp[a]);
            mw[a] = (unsigned)wave_max_u64((unsigned long long)mw[a]);
        }
    }
    if ((uniform && lane_id() == 0 && valid) || (!uniform && good)) {
        StructRec& r = recs[uniform ? b0 : b];
        for (int a = 0; a < 3; ++a) {
            if (umin[a] != ~0ull) atomicMin(&r.umin[a], umin[a]);
            if (umax[a] != 0ull) atomicMax(&r.umax[a], umax[a]);
            if (cmin[a] != ~0ull) atomicMin(&r.cmin[a], cmin[a]);
            if (cmax[a] != 0ull) atomicMax(&r.cmax[a], cmax[a]);
            if (mp[a]) atomicMax(&r.maxp[a], mp[a]);
            if (mw[a]) atomicMax(&r.maxw[a], mw[a]);
        }
    }
}

// One thread per structure: broad-phase margin, algorithm choice and the bin
// grid.  The margin pad = 64 eps_T max(scale, rc) bounds the difference
// between the fused broad-phase distance and the public predicate, with
// scale = max_c (2 max|p_c| + sum_a (R_a + 2 max|w_a|) |cell_ac|) as in
// neighbors_cpu.cpp:156-219.
template <typename T>
__global__ void k_plan(const T* cells, int64_t nb, double cutoff, int requested,
                       StructRec* recs, long long* struct_bins, unsigned long long* status) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b == 0 && status[SS_TOTAL_IMAGES] > (unsigned long long)kImageCap)
        atomicOr(status + SS_FLAGS, ST_BATCH_IMAGE_CAP);
    if (b >= nb) return;
    if (load_status(status + SS_FLAGS) & kAbortBits) {
        struct_bins[b] = 0;
        return;
    }
    StructRec r = recs[b];
    r.algo = ALGO_NONE;
    r.nbins = 0;
    if (r.natoms == 0) {
        recs[b] = r;
        struct_bins[b] = 0;
        return;
    }
    double cell[9];
    for (int e = 0; e < 9; ++e) cell[e] = (double)cells[9 * b + e];
    double maxp[3];
    for (int c = 0; c < 3; ++c) maxp[c] = __longlong_as_double((long long)r.maxp[c]);
    double scale = 0;
    for (int c = 0; c < 3; ++c) {
        double sc = 2 * maxp[c];
        for (int a = 0; a < 3; ++a)
            sc += ((double)r.reps[a] + 2.0 * (double)r.maxw[a]) * fabs(cell[3 * a + c]);
        scale = fmax(scale, sc);
    }
    const double rc = cutoff;
    const double pad = 64.0 * Ops<T>::eps * fmax(scale, rc);
    r.pad = pad;
    r.any_wrap = (r.maxw[0] | r.maxw[1] | r.maxw[2]) != 0;
    const double inner = rc - pad;
    r.inner2 = inner > 0 ? (double)Ops<T>::down(inner * inner) : 0.0;
    r.outer2 = (double)Ops<T>::up((rc + pad) * (rc + pad));
    r.cut2 = (double)(T)(cutoff * cutoff);
    const bool safe = isfinite(rc + pad) && rc + pad <= 2 * rc && rc + pad <= Ops<T>::max;

    const int64_t n = r.natoms;
    const bool large = n > kAutoBruteCandidates / r.nimages;
    bool want_cell = requested == TNR_CELL_LIST || (requested == TNR_AUTO && large);
    unsigned long long st = 0;
    if (requested == TNR_CELL_LIST) {
        // The reference CPU layout rule (neighbors_cpu.cpp:379-430): bins of
        // the padded cutoff over the wrapped bounding box.
        const double size = rc + pad;
        double count = 1;
        bool ok = safe;
        for (int c = 0; c < 3 && ok; ++c) {
            const double span = key_value(r.cmax[c]) - key_value(r.cmin[c]) + 2 * size;
            const double dim = span / size;
            if (!isfinite(dim) || dim > 67108864.0) ok = false;
            count *= fmax(1.0, ceil(dim));
        }
        if (!ok || count > 67108864.0 ||
            ceil(count / 64.0) > (double)n * (double)r.nimages)
            st |= ST_CELL_UNSAFE;
    }
    if (want_cell && !safe) want_cell = false;
    if (want_cell) {
        const double rcu0 = rc + 2 * pad;
        const double kt = (double)kStencilReach;
        double ext[3], w[3], nbf[3], rcu[3];
        for (int a = 0; a < 3; ++a) {
            const double gn = sqrt(r.grid[3 * a] * r.grid[3 * a] +
                                   r.grid[3 * a + 1] * r.grid[3 * a + 1] +
                                   r.grid[3 * a + 2] * r.grid[3 * a + 2]);
            rcu[a] = rcu0 * gn;
            if (r.active >> a & 1) {
                ext[a] = 1.0;
                nbf[a] = fmin(fmax(ceil(kt / rcu[a]) - 1.0, 1.0), 1048576.0);
                w[a] = 1.0 / nbf[a];
            } else {
                const double lo = key_value(r.umin[a]), hi = key_value(r.umax[a]);
                ext[a] = fmax(hi - lo, 0.0);
                if (!isfinite(ext[a]) || !isfinite(lo)) want_cell = false;
                w[a] = rcu[a] / kt * (1.0 + 1e-9);
                if (ext[a] / w[a] > 1048575.0) w[a] = ext[a] / 1048575.0 * (1.0 + 1e-9);
                if (!(w[a] > 0) || !isfinite(w[a])) w[a] = 1.0;
                nbf[a] = fmin(floor(ext[a] / w[a]) + 1.0, 1048576.0);
                r.lo[a] = lo;
            }
        }
        const double capb = 2.0 * (double)n + 64.0;
        for (int it = 0; it < 200 && nbf[0] * nbf[1] * nbf[2] > capb; ++it) {
            int a = 0;
            for (int c = 1; c < 3; ++c)
                if (nbf[c] > nbf[a]) a = c;
            if (r.active >> a & 1) {
                nbf[a] = ceil(nbf[a] / 2.0);
                w[a] = 1.0 / nbf[a];
            } else {
                w[a] *= 2.0;
                nbf[a] = fmin(floor(ext[a] / w[a]) + 1.0, 1048576.0);
            }
        }
        int reach[3];
        bool reach_ok = true;
        for (int a = 0; a < 3; ++a) {
            const double rd = floor(rcu[a] / w[a] * (1.0 + 1e-12)) + 1.0;
            reach_ok = reach_ok && rd < 256.0;
            reach[a] = reach_ok ? (int)rd : 1;
            r.nb[a] = (int32_t)nbf[a];
            r.inv_w[a] = (r.active >> a & 1) ? nbf[a] : 1.0 / w[a];
            r.reach[a] = reach[a];
        }
        const int rows = (2 * reach[0] + 1) * (2 * reach[1] + 1);
        int zs = 1;
        if (r.active >> 2 & 1) {
            const int span = 2 * reach[2] + 1;
            zs = min(span, (span + r.nb[2] - 1) / r.nb[2] + 1);
        }
        r.zseg = zs;
        const bool fits = want_cell && reach_ok && nbf[0] * nbf[1] * nbf[2] <= capb &&
                          (long long)rows * zs <= kPieceCap &&
                          (double)n * (double)(rows * zs) < 2147483647.0;
        if (fits) {
            r.algo = ALGO_CELL;
            r.nbins = (int64_t)(nbf[0] * nbf[1] * nbf[2]);
        }
    }
    if (r.algo == ALGO_NONE) r.algo = ALGO_BRUTE;
    recs[b] = r;
    struct_bins[b] = r.nbins;
    if (st) atomicOr(status + SS_FLAGS, st);
}

__global__ void k_struct_bin0(StructRec* recs, const long long* off, int64_t nb,
                              unsigned long long* status, int64_t cap_bins) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b < nb) recs[b].bin0 = off[b];
    if (b == 0) {
        status[SS_TOTAL_BINS] = (unsigned long long)off[nb];
        if (off[nb] > cap_bins) atomicOr(status + SS_FLAGS, ST_CAPACITY);
    }
}

template <typename T>
__device__ __forceinline__ int64_t local_bin(const StructRec& r, const T q[3]) {
    double u[3];
    grid_coords(r, q, u);
    int64_t k[3];
    for (int a = 0; a < 3; ++a) {
        const double x = (u[a] - r.lo[a]) * r.inv_w[a];
        double f = floor(x);
        f = fmin(fmax(f, 0.0), (double)(r.nb[a] - 1));
        k[a] = isfinite(f) ? (int64_t)f : 0;
    }
    return (k[0] * r.nb[1] + k[1]) * r.nb[2] + k[2];
}

template <typename T>
__global__ __launch_bounds__(kBlock) void k_bin(int64_t n_atoms, const StructRec* recs,
                                                 const int* atom_struct, const Vec4<T>* atom_q,
                                                 int* atom_bin, int* atom_rank, int* bin_count,
                                                 const unsigned long long* status) {
    if (load_status(status + SS_FLAGS) & kAbortBits) return;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_atoms) return;
    const StructRec& r = recs[atom_struct[i]];
    if (r.algo != ALGO_CELL) {
        atom_bin[i] = -1;
        return;
    }
    const Vec4<T> v = atom_q[i];
    const T q[3] = {v.x, v.y, v.z};
    const int64_t g = r.bin0 + local_bin(r, q);
    atom_bin[i] = (int)g;
    atom_rank[i] = atomicAdd(bin_count + g, 1);
}

template <typename T>
__global__ __launch_bounds__(kBlock) void k_scatter(int64_t n_atoms, const Vec4<T>* atom_q,
                                                     const int* atom_bin, const int* atom_rank,
                                                     const int* bin_start, Vec4<T>* binned,
                                                     const unsigned long long* status) {
    if (load_status(status + SS_FLAGS) & kAbortBits) return;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_atoms) return;
    const int g = atom_bin[i];
    if (g < 0) return;
    binned[bin_start[g] + atom_rank[i]] = atom_q[i];
}

// ----------------------------------------------------------- query kernels

template <typename T>
struct QueryArgs {
    const T* pos;
    const T* cells;
    const StructRec* recs;
    const int64_t* struct_bin_off;  // B + 1
    const int* atom_struct;
    const int4* atom_wrap;
    const Vec4<T>* atom_q;
    const int* bin_start;
    const Vec4<T>* binned;
    long long* counts;
    const long long* offsets;
    unsigned long long* status;
    int64_t n_atoms;
    int64_t nb;
    int64_t limit;  // E: emit never writes at or beyond it
    // outputs (emit)
    int64_t* pairs;
    int32_t* shifts;
    T* dist;
    T* vec;
    int64_t* src;
    int64_t* dst;
};

template <typename T>
__device__ __forceinline__ void write_hit(const QueryArgs<T>& a, long long o, int s, int t,
                                          long long S0, long long S1, long long S2,
                                          const T ps[3], const T pt[3], const T* cell) {
    if (o < 0 || o >= a.limit) {
        atomicOr(a.status + SS_FLAGS, ST_CAPACITY);
        return;
    }
    if (a.pairs) {
        long2 v;
        v.x = s;
        v.y = t;
        *reinterpret_cast<long2*>(a.pairs + 2 * o) = v;
    }
    if (a.src) a.src[o] = s;
    if (a.dst) a.dst[o] = t;
    if (a.shifts) {
        a.shifts[3 * o] = (int32_t)S0;
        a.shifts[3 * o + 1] = (int32_t)S1;
        a.shifts[3 * o + 2] = (int32_t)S2;
    }
    if (a.vec || a.dist) {
        T D[3];
        const T d2 = public_vector(ps, pt, S0, S1, S2, cell, D);
        if (a.vec) {
            a.vec[3 * o] = D[0];
            a.vec[3 * o + 1] = D[1];
            a.vec[3 * o + 2] = D[2];
        }
        if (a.dist) a.dist[o] = Ops<T>::sqrt_(d2);
    }
}

__device__ __forceinline__ bool fits_i32(long long v) {
    return v >= -2147483648ll && v <= 2147483647ll;
}

// One wave per source atom of a brute-force structure (grid-stride).  Lanes
// hold 64 targets; the wave walks the image box of the structure in the
// reference order (x-major, z fastest).  Broad phase: fused distance of the
// wrapped positions plus the image translation against [inner2, outer2);
// the band in between is decided by the public predicate.
template <typename T, int MODE, bool EMIT>
__global__ __launch_bounds__(kBlock) void k_brute(QueryArgs<T> a) {
    using O = Ops<T>;
    if (load_status(a.status + SS_FLAGS) & kAbortBits) return;
    const int lane = lane_id();
    const int64_t wave0 = ((int64_t)blockIdx.x * kBlock + threadIdx.x) / kWave;
    const int64_t nwaves = (int64_t)gridDim.x * kWavesPerBlock;
    for (int64_t s64 = wave0; s64 < a.n_atoms; s64 += nwaves) {
        const int s = (int)s64;
        const int b = a.atom_struct[s];
        const StructRec& r = a.recs[b];
        if (r.algo != ALGO_BRUTE) continue;
        const int a0 = (int)r.atom0;
        const int a1 = (int)(r.atom0 + r.natoms);
        const int R0 = r.reps[0], R1 = r.reps[1], R2 = r.reps[2];
        const T* cell = a.cells + 9 * b;
        T c[9];
#pragma unroll
        for (int e = 0; e < 9; ++e) c[e] = cell[e];
        const T inner2 = (T)r.inner2, outer2 = (T)r.outer2, cut2 = (T)r.cut2;
        const bool any_wrap = r.any_wrap != 0;
        const Vec4<T> qs4 = a.atom_q[s];
        const int4 ws = a.atom_wrap[s];
        const T ps[3] = {a.pos[3 * s], a.pos[3 * s + 1], a.pos[3 * s + 2]};
        long long total = 0;
        long long cursor = EMIT ? a.offsets[s] : 0;
        const int tstart = (MODE & 2) ? s : a0;
        for (int tb = tstart; tb < a1; tb += kWave) {
            const int t = tb + lane;
            const bool vt = t < a1;
            T bx = T(0), by = T(0), bz = T(0);
            T pt[3] = {T(0), T(0), T(0)};
            int4 wt = make_int4(0, 0, 0, 0);
            if (vt) {
                const Vec4<T> qt = a.atom_q[t];
                bx = O::sub(qt.x, qs4.x);
                by = O::sub(qt.y, qs4.y);
                bz = O::sub(qt.z, qs4.z);
                pt[0] = a.pos[3 * t];
                pt[1] = a.pos[3 * t + 1];
                pt[2] = a.pos[3 * t + 2];
                wt = a.atom_wrap[t];
            }
            for (int i0 = -R0; i0 <= R0; ++i0) {
                const T f0 = (T)i0;
                for (int i1 = -R1; i1 <= R1; ++i1) {
                    const T f1 = (T)i1;
                    const T ex = O::fma_(f1, c[3], O::fma_(f0, c[0], bx));
                    const T ey = O::fma_(f1, c[4], O::fma_(f0, c[1], by));
                    const T ez = O::fma_(f1, c[5], O::fma_(f0, c[2], bz));
                    for (int i2 = -R2; i2 <= R2; ++i2) {
                        const T f2 = (T)i2;
                        const T dx = O::fma_(f2, c[6], ex);
                        const T dy = O::fma_(f2, c[7], ey);
                        const T dz = O::fma_(f2, c[8], ez);
                        const T d2 = O::fma_(dz, dz, O::fma_(dy, dy, O::mul(dx, dx)));
                        const bool zs = t == s && i0 == 0 && i1 == 0 && i2 == 0;
                        bool ok = vt && (d2 < outer2 || zs) &&
                                  keep_identity<MODE>(s, t, i0, i1, i2);
                        const long long S0 = (long long)i0 - wt.x + ws.x;
                        const long long S1 = (long long)i1 - wt.y + ws.y;
                        const long long S2 = (long long)i2 - wt.z + ws.z;
                        if (ok && !zs && !(d2 < inner2)) {
                            T D[3];
                            ok = public_vector(ps, pt, S0, S1, S2, c, D) < cut2;
                        }
                        const unsigned long long m = ballot(ok);
                        if (m == 0) continue;
                        if (!EMIT) {
                            if (any_wrap && ok && !(fits_i32(S0) && fits_i32(S1) && fits_i32(S2)))
                                atomicOr(a.status + SS_FLAGS, ST_SHIFT_RANGE);
                            total += __popcll(m);
                        } else {
                            if (ok)
                                write_hit(a, cursor + lanes_below(m), s, t, S0, S1, S2, ps, pt, c);
                            cursor += __popcll(m);
                        }
                    }
                }
            }
        }
        if (!EMIT && lane == 0) a.counts[s] = total;
    }
}

// One wave per bin of a cell-list structure (grid-stride over all bins,
// XCD-grouped).  The wave builds the stencil of its bin as pieces: runs of
// consecutive z-bins of one (x, y) row with one periodic image k.  Pieces
// with |k_a| > R_a are dropped, which keeps exactly the reference's image
// box.  Lanes then hold 64 consecutive candidates of the flattened stencil;
// the sources of the bin are broadcast one at a time.
template <typename T, int MODE, bool EMIT>
__global__ __launch_bounds__(kBlock) void k_cell(QueryArgs<T> a) {
    using O = Ops<T>;
    __shared__ int s_start[kWavesPerBlock][kPieceCap];
    __shared__ int s_pre[kWavesPerBlock][kPieceCap + 1];
    __shared__ int s_k[kWavesPerBlock][kPieceCap];
    __shared__ T s_tr[kWavesPerBlock][3][kPieceCap];

    if (load_status(a.status + SS_FLAGS) & kAbortBits) return;
    const int lane = lane_id();
    const int wv = threadIdx.x / kWave;
    // XCD-grouped block order: the hardware deals blocks round-robin over 8
    // XCDs; give each XCD a contiguous range of logical blocks.
    const unsigned nblk = gridDim.x;
    unsigned lb = blockIdx.x;
    if ((nblk & 7u) == 0) lb = (blockIdx.x & 7u) * (nblk >> 3) + (blockIdx.x >> 3);
    const int64_t wave0 = (int64_t)lb * kWavesPerBlock + wv;
    const int64_t nwaves = (int64_t)nblk * kWavesPerBlock;
    const int64_t total_bins = a.struct_bin_off[a.nb];
    int* pstart = s_start[wv];
    int* pre = s_pre[wv];
    int* pk = s_k[wv];

    for (int64_t g = wave0; g < total_bins; g += nwaves) {
        const int sb = a.bin_start[g], se = a.bin_start[g + 1];
        if (sb == se) continue;
        // structure of bin g
        int64_t lo = 0, hi = a.nb;
        while (hi - lo > 1) {
            const int64_t mid = (lo + hi) >> 1;
            if (a.struct_bin_off[mid] <= g) lo = mid; else hi = mid;
        }
        const int b = (int)lo;
        const StructRec& r = a.recs[b];
        const T* cell = a.cells + 9 * b;
        T c[9];
#pragma unroll
        for (int e = 0; e < 9; ++e) c[e] = cell[e];
        const T outer2 = (T)r.outer2, inner2 = (T)r.inner2, cut2 = (T)r.cut2;
        const bool wrapped = r.any_wrap != 0;
        const int nx = r.nb[0], ny = r.nb[1], nz = r.nb[2];
        const int Kx = r.reach[0], Ky = r.reach[1], Kz = r.reach[2];
        const int R0 = r.reps[0], R1 = r.reps[1], R2 = r.reps[2];
        const bool perx = r.active & 1, pery = r.active >> 1 & 1, perz = r.active >> 2 & 1;
        const int zs = r.zseg;
        const int64_t lbin = g - r.bin0;
        const int iz = (int)(lbin % nz);
        const int iy = (int)((lbin / nz) % ny);
        const int ix = (int)(lbin / ((int64_t)nz * ny));
        const int RY = 2 * Ky + 1;
        const int rows = (2 * Kx + 1) * RY;
        const int npieces = rows * zs;
        const int* bstart = a.bin_start + r.bin0;

        // ---- stencil pieces
        for (int row = lane; row < rows; row += kWave) {
            const int ox = row / RY - Kx, oy = row % RY - Ky;
            int jx = ix + ox, jy = iy + oy, kx = 0, ky = 0;
            bool okr = true;
            if (perx) {
                kx = (int)floor_div(jx, nx);
                jx -= kx * nx;
                okr = okr && abs(kx) <= R0;
            } else {
                okr = okr && jx >= 0 && jx < nx;
            }
            if (pery) {
                ky = (int)floor_div(jy, ny);
                jy -= ky * ny;
                okr = okr && abs(ky) <= R1;
            } else {
                okr = okr && jy >= 0 && jy < ny;
            }
            const int rowbase = (jx * ny + jy) * nz;
            int seg = 0;
            if (okr) {
                if (perz) {
                    int z = iz - Kz;
                    const int zhi = iz + Kz;
                    while (z <= zhi && seg < zs) {
                        const int kz = (int)floor_div(z, nz);
                        const int top = min(zhi, (kz + 1) * nz - 1);
                        const int z0 = z - kz * nz, z1 = top - kz * nz;
                        const int slot = row * zs + seg;
                        if (abs(kz) <= R2) {
                            pstart[slot] = bstart[rowbase + z0];
                            pre[slot + 1] = bstart[rowbase + z1 + 1] - bstart[rowbase + z0];
                        } else {
                            pstart[slot] = 0;
                            pre[slot + 1] = 0;
                        }
                        pk[slot] = (kx + 512) | ((ky + 512) << 10) | ((kz + 512) << 20);
                        s_tr[wv][0][slot] = O::fma_((T)kz, c[6], O::fma_((T)ky, c[3], O::mul((T)kx, c[0])));
                        s_tr[wv][1][slot] = O::fma_((T)kz, c[7], O::fma_((T)ky, c[4], O::mul((T)kx, c[1])));
                        s_tr[wv][2][slot] = O::fma_((T)kz, c[8], O::fma_((T)ky, c[5], O::mul((T)kx, c[2])));
                        ++seg;
                        z = top + 1;
                    }
                } else {
                    const int z0 = max(0, iz - Kz), z1 = min(nz - 1, iz + Kz);
                    const int slot = row * zs;
                    pstart[slot] = bstart[rowbase + z0];
                    pre[slot + 1] = bstart[rowbase + z1 + 1] - bstart[rowbase + z0];
                    pk[slot] = (kx + 512) | ((ky + 512) << 10) | (512 << 20);
                    s_tr[wv][0][slot] = O::fma_((T)ky, c[3], O::mul((T)kx, c[0]));
                    s_tr[wv][1][slot] = O::fma_((T)ky, c[4], O::mul((T)kx, c[1]));
                    s_tr[wv][2][slot] = O::fma_((T)ky, c[5], O::mul((T)kx, c[2]));
                    seg = 1;
                }
            }
            for (; seg < zs; ++seg) {
                const int slot = row * zs + seg;
                pstart[slot] = 0;
                pre[slot + 1] = 0;
                pk[slot] = 512 | (512 << 10) | (512 << 20);
                s_tr[wv][0][slot] = T(0);
                s_tr[wv][1][slot] = T(0);
                s_tr[wv][2][slot] = T(0);
            }
        }
        __builtin_amdgcn_wave_barrier();
        // prefix sum of piece lengths: pre[0] = 0, pre[i + 1] = sum_{j <= i} len_j
        if (lane == 0) pre[0] = 0;
        int carry = 0;
        for (int base = 0; base < npieces; base += kWave) {
            const int i = base + lane;
            const long long len = i < npieces ? pre[i + 1] : 0;
            const long long inc = wave_inclusive_scan(len);
            if (i < npieces) pre[i + 1] = carry + (int)inc;
            carry += (int)read_lane((long long)inc, kWave - 1);
        }
        __builtin_amdgcn_wave_barrier();
        const int C = carry;

        // ---- sources of this bin, 64 at a time
        for (int sg = sb; sg < se; sg += kWave) {
            const int ns = min(kWave, se - sg);
            Vec4<T> sq = {T(0), T(0), T(0), T(0)};
            int sidx_l = 0;
            if (lane < ns) {
                sq = a.binned[sg + lane];
                sidx_l = as_idx(sq.w);
            }
            long long acc = 0;
            long long cur = 0;
            if (EMIT && lane < ns) cur = a.offsets[sidx_l];
            for (int cb = 0; cb < C; cb += kWave) {
                const int v = cb + lane;
                const bool valid = v < C;
                int piece = 0;
                T tx = T(0), ty = T(0), tz = T(0);
                T rx = T(0), ry = T(0), rz = T(0);
                int tidx = -1;
                int kx = 0, ky = 0, kz = 0;
                if (valid) {
                    int plo = 0, phi = npieces;
                    while (phi - plo > 1) {
                        const int mid = (plo + phi) >> 1;
                        if (pre[mid] <= v) plo = mid; else phi = mid;
                    }
                    piece = plo;
                    const Vec4<T> rec = a.binned[pstart[piece] + (v - pre[piece])];
                    rx = rec.x;
                    ry = rec.y;
                    rz = rec.z;
                    tidx = as_idx(rec.w);
                    tx = O::add(rx, s_tr[wv][0][piece]);
                    ty = O::add(ry, s_tr[wv][1][piece]);
                    tz = O::add(rz, s_tr[wv][2][piece]);
                    const int kk = pk[piece];
                    kx = (kk & 1023) - 512;
                    ky = ((kk >> 10) & 1023) - 512;
                    kz = ((kk >> 20) & 1023) - 512;
                }
                const bool k0 = kx == 0 && ky == 0 && kz == 0;
                for (int gi = 0; gi < ns; ++gi) {
                    const T sx = read_lane(sq.x, gi), sy = read_lane(sq.y, gi),
                            sz = read_lane(sq.z, gi);
                    const int si = read_lane(sidx_l, gi);
                    const T dx = O::sub(tx, sx), dy = O::sub(ty, sy), dz = O::sub(tz, sz);
                    const T d2 = O::fma_(dz, dz, O::fma_(dy, dy, O::mul(dx, dx)));
                    const bool zsf = tidx == si && k0;
                    bool ok = valid && (d2 < outer2 || zsf) &&
                              keep_identity<MODE>(si, tidx, kx, ky, kz);
                    long long S0 = kx, S1 = ky, S2 = kz;
                    T ps[3], pt[3];
                    const bool need_exact = ok && !zsf && !(d2 < inner2);
                    if ((need_exact || (EMIT && ok)) || (wrapped && ok)) {
                        if (wrapped) {
                            const int4 wt = a.atom_wrap[tidx];
                            const int4 ws = a.atom_wrap[si];
                            S0 = (long long)kx - wt.x + ws.x;
                            S1 = (long long)ky - wt.y + ws.y;
                            S2 = (long long)kz - wt.z + ws.z;
                            for (int cc = 0; cc < 3; ++cc) {
                                ps[cc] = a.pos[3 * (int64_t)si + cc];
                                pt[cc] = a.pos[3 * (int64_t)tidx + cc];
                            }
                        } else {
                            ps[0] = sx;
                            ps[1] = sy;
                            ps[2] = sz;
                            pt[0] = rx;
                            pt[1] = ry;
                            pt[2] = rz;
                        }
                        if (need_exact) {
                            T D[3];
                            ok = public_vector(ps, pt, S0, S1, S2, c, D) < cut2;
                        }
                    }
                    const unsigned long long m = ballot(ok);
                    if (m == 0) continue;
                    if (!EMIT) {
                        if (wrapped && ok && !(fits_i32(S0) && fits_i32(S1) && fits_i32(S2)))
                            atomicOr(a.status + SS_FLAGS, ST_SHIFT_RANGE);
                        if (lane == gi) acc += __popcll(m);
                    } else {
                        const long long base = read_lane(cur, gi);
                        if (ok) write_hit(a, base + lanes_below(m), si, tidx, S0, S1, S2, ps, pt, c);
                        if (lane == gi) cur += __popcll(m);
                    }
                }
            }
            if (!EMIT && lane < ns) a.counts[sidx_l] = acc;
        }
    }
}

__global__ void k_finish(const long long* offsets, int64_t n_atoms, unsigned long long* status) {
    if (blockIdx.x == 0 && threadIdx.x == 0) status[SS_PAIRS] = (unsigned long long)offsets[n_atoms];
}

// ------------------------------------------------------------------- host

struct Views {
    unsigned long long* status;
    StructRec* recs;
    long long* struct_bins;
    long long* struct_bin_off;
    int* atom_struct;
    int4* atom_wrap;
    void* atom_q;
    int* atom_bin;
    int* atom_rank;
    int* bin_count;
    int* bin_start;
    void* binned;
    long long* counts;
    long long* offsets;
    long long* partials;
};

static Views views(void* ws, const Layout& L) {
    char* base = (char*)ws;
    Views v;
    v.status = (unsigned long long*)(base + L.status);
    v.recs = (StructRec*)(base + L.structs);
    v.struct_bins = (long long*)(base + L.struct_bins);
    v.struct_bin_off = (long long*)(base + L.struct_bin_off);
    v.atom_struct = (int*)(base + L.atom_struct);
    v.atom_wrap = (int4*)(base + L.atom_wrap);
    v.atom_q = base + L.atom_q;
    v.atom_bin = (int*)(base + L.atom_bin);
    v.atom_rank = (int*)(base + L.atom_rank);
    v.bin_count = (int*)(base + L.bin_count);
    v.bin_start = (int*)(base + L.bin_start);
    v.binned = base + L.binned;
    v.counts = (long long*)(base + L.counts);
    v.offsets = (long long*)(base + L.offsets);
    v.partials = (long long*)(base + L.partials);
    return v;
}

static unsigned blocks_for(int64_t n, int per = kBlock) {
    const int64_t b = (n + per - 1) / per;
    return (unsigned)(b > 0 ? b : 1);
}

// Waves of a grid-stride query kernel: enough for ~8 waves per SIMD.
static unsigned query_blocks(int64_t work_waves) {
    const int64_t want = (work_waves + kWavesPerBlock - 1) / kWavesPerBlock;
    int64_t cap = 8192;
    int64_t b = want < cap ? want : cap;
    if (b > 8) b = (b + 7) / 8 * 8;
    return (unsigned)(b > 0 ? b : 1);
}

template <typename T>
static QueryArgs<T> query_args(const tnr_request* req, const Views& v) {
    QueryArgs<T> q{};
    q.pos = (const T*)req->positions;
    q.cells = (const T*)req->cell;
    q.recs = v.recs;
    q.struct_bin_off = (const int64_t*)v.struct_bin_off;
    q.atom_struct = v.atom_struct;
    q.atom_wrap = v.atom_wrap;
    q.atom_q = (const Vec4<T>*)v.atom_q;
    q.bin_start = v.bin_start;
    q.binned = (const Vec4<T>*)v.binned;
    q.counts = v.counts;
    q.offsets = v.offsets;
    q.status = v.status;
    q.n_atoms = req->n_atoms;
    q.nb = req->n_structures;
    return q;
}

template <typename T, int MODE, bool EMIT>
static void launch_queries(const tnr_request* req, const Layout& L, const QueryArgs<T>& q,
                           hipStream_t stream) {
    const int64_t n = req->n_atoms;
    if (n == 0) return;
    if (req->algorithm != TNR_BRUTE_FORCE)
        k_cell<T, MODE, EMIT><<<query_blocks(L.cap_bins), kBlock, 0, stream>>>(q);
    k_brute<T, MODE, EMIT><<<query_blocks(n), kBlock, 0, stream>>>(q);
}

template <typename T, bool EMIT>
static void dispatch_queries(const tnr_request* req, const Layout& L, const QueryArgs<T>& q,
                             hipStream_t stream) {
    const int mode = (req->half_list ? 2 : 0) | (req->include_self ? 1 : 0);
    switch (mode) {
        case 0: launch_queries<T, 0, EMIT>(req, L, q, stream); break;
        case 1: launch_queries<T, 1, EMIT>(req, L, q, stream); break;
        case 2: launch_queries<T, 2, EMIT>(req, L, q, stream); break;
        default: launch_queries<T, 3, EMIT>(req, L, q, stream); break;
    }
}

template <typename T>
static hipError_t run_count(const tnr_request* req, void* ws, const Layout& L,
                            hipStream_t stream) {
    const Views v = views(ws, L);
    const int64_t n = req->n_atoms, nb = req->n_structures;
    k_fill_i64<<<1, 64, 0, stream>>>((long long*)v.status, SS_SLOTS, 0);
    k_setup<T><<<blocks_for(nb > 0 ? nb : 1, 64), 64, 0, stream>>>(
        req->batch_ptr, (const T*)req->cell, req->pbc, nb, n, req->cutoff, v.recs, v.status);
    if (n > 0)
        k_atoms<T><<<blocks_for(n), kBlock, 0, stream>>>(
            (const T*)req->positions, req->batch_ptr, (const T*)req->cell, nb, n, v.recs,
            v.atom_struct, v.atom_wrap, (Vec4<T>*)v.atom_q, v.status);
    k_plan<T><<<blocks_for(nb > 0 ? nb : 1, 64), 64, 0, stream>>>(
        (const T*)req->cell, nb, req->cutoff, req->algorithm, v.recs, v.struct_bins, v.status);
    (void)device_scan<long long, long long>(v.struct_bins, nb, v.struct_bin_off, v.partials,
                                            stream);
    k_struct_bin0<<<blocks_for(nb > 0 ? nb : 1, 64), 64, 0, stream>>>(
        v.recs, v.struct_bin_off, nb, v.status, L.cap_bins);
    if (n > 0 && req->algorithm != TNR_BRUTE_FORCE) {
        k_fill_i32<<<blocks_for(L.cap_bins + 1), kBlock, 0, stream>>>(v.bin_count,
                                                                      L.cap_bins + 1, 0);
        k_bin<T><<<blocks_for(n), kBlock, 0, stream>>>(n, v.recs, v.atom_struct,
                                                       (const Vec4<T>*)v.atom_q, v.atom_bin,
                                                       v.atom_rank, v.bin_count, v.status);
        (void)device_scan<int, int>(v.bin_count, L.cap_bins, v.bin_start, v.partials, stream);
        k_scatter<T><<<blocks_for(n), kBlock, 0, stream>>>(n, (const Vec4<T>*)v.atom_q,
                                                           v.atom_bin, v.atom_rank,
                                                           v.bin_start, (Vec4<T>*)v.binned,
                                                           v.status);
    }
    const QueryArgs<T> q = query_args<T>(req, v);
    dispatch_queries<T, false>(req, L, q, stream);
    (void)device_scan<long long, long long>(v.counts, n, v.offsets, v.partials, stream);
    k_finish<<<1, 1, 0, stream>>>(v.offsets, n, v.status);
    return hipGetLastError();
}

template <typename T>
static hipError_t run_emit(const tnr_request* req, void* ws, const Layout& L,
                           const tnr_outputs* out, hipStream_t stream) {
    const Views v = views(ws, L);
    QueryArgs<T> q = query_args<T>(req, v);
    q.pairs = out->pairs;
    q.shifts = out->shifts;
    q.dist = (T*)out->distances;
    q.vec = (T*)out->vectors;
    q.src = out->sources;
    q.dst = out->targets;
    q.limit = out->n_pairs;
    dispatch_queries<T, true>(req, L, q, stream);
    return hipGetLastError();
}

struct StatusMessage {
    unsigned long long bit;
    int code;
    const char* text;
};

// Priority follows the order in which the reference raises: host-side
// batch_ptr checks, periodic metadata, then device status words.
static const StatusMessage kMessages[] = {
    {ST_BP_START, TNR_INPUT_ERROR, "batch_ptr must start at zero"},
    {ST_BP_END, TNR_INPUT_ERROR, "batch_ptr must end at N_total"},
    {ST_BP_ORDER, TNR_INPUT_ERROR, "batch_ptr must be nondecreasing"},
    {ST_CELL_NONFINITE, TNR_INPUT_ERROR, "cell must contain only finite values"},
    {ST_CELL_RANK, TNR_INPUT_ERROR, "active periodic cell vectors must be linearly independent"},
    {ST_DUAL_RANGE, TNR_INPUT_ERROR, "active periodic cell dual is outside the float64 range"},
    {ST_REPEAT_RANGE, TNR_INPUT_ERROR, "periodic image range exceeds int32 cell shifts"},
    {ST_IMAGE_CAP, TNR_INPUT_ERROR, "periodic image count exceeds the 2^24 resource limit"},
    {ST_BATCH_IMAGE_CAP, TNR_INPUT_ERROR,
     "batched periodic image count exceeds the 2^24 resource limit"},
    {ST_POS_NONFINITE, TNR_SEARCH_ERROR, "positions must contain only finite values"},
    {ST_WRAP_RANGE, TNR_SEARCH_ERROR,
     "atom representatives require periodic wraps outside the int32 range"},
    {ST_CELL_UNSAFE, TNR_SEARCH_ERROR,
     "cell_list cannot safely process this structure; use algorithm='auto' or 'brute_force'"},
    {ST_SHIFT_RANGE, TNR_SEARCH_ERROR,
     "a cell shift required by the neighbor list exceeds the int32 output range"},
    {ST_CAPACITY, TNR_SEARCH_ERROR, "neighbor-list workspace capacity exceeded"},
};

static int put_error(char* err, size_t len, int code, const char* msg) {
    if (err && len > 0) {
        std::strncpy(err, msg, len - 1);
        err[len - 1] = 0;
    }
    return code;
}

static int check_request(const tnr_request* req, size_t ws_bytes, const void* ws, char* err,
                         size_t err_len, Layout* L) {
    if (!req) return put_error(err, err_len, TNR_INPUT_ERROR, "request is null");
    if (req->dtype != TNR_FLOAT32 && req->dtype != TNR_FLOAT64)
        return put_error(err, err_len, TNR_INPUT_ERROR,
                         "positions must have dtype float32 or float64");
    if (req->algorithm < TNR_AUTO || req->algorithm > TNR_CELL_LIST)
        return put_error(err, err_len, TNR_INPUT_ERROR,
                         "algorithm must be 'auto', 'brute_force', or 'cell_list'");
    if (!(std::isfinite(req->cutoff) && req->cutoff > 0))
        return put_error(err, err_len, TNR_INPUT_ERROR, "cutoff must be finite and positive");
    if (req->n_atoms < 0 || req->n_structures < 0)
        return put_error(err, err_len, TNR_INPUT_ERROR, "invalid sizes");
    if (req->n_atoms >= (int64_t{1} << 31))
        return put_error(err, err_len, TNR_INPUT_ERROR,
                         "the current implementation supports fewer than 2^31 atoms");
    *L = make_layout(req->n_atoms, req->n_structures,
                     req->dtype == TNR_FLOAT32 ? sizeof(float) : sizeof(double));
    if (L->cap_bins >= (int64_t{1} << 31))
        return put_error(err, err_len, TNR_INPUT_ERROR,
                         "the current implementation supports fewer than 2^31 atoms");
    if (!ws || ws_bytes < L->total || ((uintptr_t)ws & 255) != 0)
        return put_error(err, err_len, TNR_INPUT_ERROR,
                         "workspace is missing, too small or not 256-byte aligned");
    return TNR_OK;
}

}  // namespace tnr

// ----------------------------------------------------------------- C ABI

extern "C" {

int tnr_abi_version(void) { return TNR_ABI_VERSION; }

const char* tnr_device_arch(void) { return "gfx950"; }

size_t tnr_workspace_size(const tnr_request* req) {
    if (!req || req->n_atoms < 0 || req->n_structures < 0) return 0;
    return tnr::make_layout(req->n_atoms, req->n_structures,
                            req->dtype == TNR_FLOAT32 ? sizeof(float) : sizeof(double))
        .total;
}

int tnr_count(const tnr_request* req, void* workspace, size_t workspace_bytes,
              int64_t* host_result, void* stream, int64_t* n_pairs, char* err, size_t err_len) {
    tnr::Layout L;
    const int rc = tnr::check_request(req, workspace_bytes, workspace, err, err_len, &L);
    if (rc != TNR_OK) return rc;
    if (!host_result || !n_pairs)
        return tnr::put_error(err, err_len, TNR_INPUT_ERROR, "result pointers are null");
    hipStream_t s = (hipStream_t)stream;
    hipError_t e = req->dtype == TNR_FLOAT32 ? tnr::run_count<float>(req, workspace, L, s)
                                             : tnr::run_count<double>(req, workspace, L, s);
    if (e == hipSuccess) {
        const tnr::Views v = tnr::views(workspace, L);
        e = hipMemcpyAsync(host_result, v.status, 4 * sizeof(int64_t), hipMemcpyDeviceToHost, s);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return tnr::put_error(err, err_len, TNR_DEVICE_ERROR, hipGetErrorString(e));
    const unsigned long long flags = (unsigned long long)host_result[tnr::SS_FLAGS];
    if (flags) {
        for (const auto& m : tnr::kMessages)
            if (flags & m.bit) return tnr::put_error(err, err_len, m.code, m.text);
        return tnr::put_error(err, err_len, TNR_SEARCH_ERROR, "invalid neighbor-list status");
    }
    *n_pairs = host_result[tnr::SS_PAIRS];
    return TNR_OK;
}

int tnr_emit(const tnr_request* req, void* workspace, size_t workspace_bytes,
             const tnr_outputs* out, void* stream, char* err, size_t err_len) {
    tnr::Layout L;
    const int rc = tnr::check_request(req, workspace_bytes, workspace, err, err_len, &L);
    if (rc != TNR_OK) return rc;
    if (!out) return tnr::put_error(err, err_len, TNR_INPUT_ERROR, "outputs are null");
    if (out->n_pairs == 0) return TNR_OK;
    hipStream_t s = (hipStream_t)stream;
    const hipError_t e = req->dtype == TNR_FLOAT32
                             ? tnr::run_emit<float>(req, workspace, L, out, s)
                             : tnr::run_emit<double>(req, workspace, L, out, s);
    if (e != hipSuccess) return tnr::put_error(err, err_len, TNR_DEVICE_ERROR, hipGetErrorString(e));
    return TNR_OK;
}

}  // extern "C"
