// Prologue kernels of a neighbor-list request: per-structure periodic
// metadata (k_setup), per-atom wraps and reductions (k_atoms), per-structure
// margins / algorithm / bin grid (k_plan), and the counting sort of cell-list
// atoms into bins (k_bin, k_scatter; the scans are in nl_scan.h).
#pragma once

#include "nl_math.h"
#include "nl_scan.h"

namespace tnr {

// ------------------------------------------------------------------ geometry

// Moore-Penrose pseudo-inverse of the k active cell rows (stored in columns
// 0..k-1 of w) by one-sided (Hestenes) Jacobi in float64: the algorithm of
// geometry.cpp:15-118, carried out in double instead of long double.  Loops
// run over all three columns with guards so every index is static (no
// scratch memory).  Returns false when the active rows are linearly dependent.
__device__ __forceinline__ bool active_pinv(double w[3][3], int k, double dual[3][3]) {
    double v[3][3] = {{1, 0, 0}, {0, 1, 0}, {0, 0, 1}};
    const double eps = 2.220446049250313e-16;
    bool any_rotation = false;
    for (int sweep = 0; sweep < 64; ++sweep) {
        bool rotated = false;
#pragma unroll
        for (int p = 0; p < 3; ++p) {
#pragma unroll
            for (int q = p + 1; q < 3; ++q) {
                if (q >= k) continue;
                double app = 0, aqq = 0, apq = 0;
#pragma unroll
                for (int c = 0; c < 3; ++c) {
                    app += w[c][p] * w[c][p];
                    aqq += w[c][q] * w[c][q];
                    apq += w[c][p] * w[c][q];
                }
                if (fabs(apq) <= 8 * eps * sqrt(app * aqq)) continue;
                rotated = true;
                any_rotation = true;
                const double zeta = (aqq - app) / (2 * apq);
                // hypot(1, x) as sqrt(fma(x, x, 1)) (one rounding before the
                // root) wherever x^2 cannot overflow; |t| <= 1 always
                const double az = fabs(zeta);
                const double hz = az < 1e150 ? sqrt(fma(zeta, zeta, 1.0)) : hypot(1.0, zeta);
                const double t = zeta == 0.0 ? 1.0 : copysign(1.0, zeta) / (az + hz);
                const double cs = 1.0 / sqrt(fma(t, t, 1.0));
                const double sn = cs * t;
#pragma unroll
                for (int c = 0; c < 3; ++c) {
                    const double a = w[c][p], b = w[c][q];
                    w[c][p] = cs * a - sn * b;
                    w[c][q] = sn * a + cs * b;
                }
#pragma unroll
                for (int r = 0; r < 3; ++r) {
                    const double a = v[r][p], b = v[r][q];
                    v[r][p] = cs * a - sn * b;
                    v[r][q] = sn * a + cs * b;
                }
            }
        }
        if (!rotated) break;
    }
    double sig2[3], smax = 0, smin = INFINITY;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        sig2[j] = w[0][j] * w[0][j] + w[1][j] * w[1][j] + w[2][j] * w[2][j];
        if (j < k) {
            const double s = sqrt(sig2[j]);
            smax = fmax(smax, s);
            smin = fmin(smin, s);
        }
    }
    if (!(smin > eps * 3 * fmax(smax, 1.0))) return false;
    if (!any_rotation) {
        // Orthogonal active rows (a diagonal cell among them): v is the
        // identity, so every term of the sum below but j = a is a signed
        // zero and the sum is 0 + w[c][a] / sig2[a], bit for bit.
#pragma unroll
        for (int c = 0; c < 3; ++c)
#pragma unroll
            for (int a = 0; a < 3; ++a) dual[c][a] = a < k ? 0.0 + w[c][a] / sig2[a] : 0.0;
        return true;
    }
#pragma unroll
    for (int c = 0; c < 3; ++c)
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            double acc = 0;
#pragma unroll
            for (int j = 0; j < 3; ++j)
                if (j < k) acc += w[c][j] * v[a][j] / sig2[j];
            dual[c][a] = a < k ? acc : 0.0;
        }
    return true;
}

__device__ inline void cross3(const double a[3], const double b[3], double o[3]) {
    o[0] = a[1] * b[2] - a[2] * b[1];
    o[1] = a[2] * b[0] - a[0] * b[2];
    o[2] = a[0] * b[1] - a[1] * b[0];
}

__device__ inline void normalize3(double v[3]) {
    const double n = sqrt(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
    if (n > 0 && isfinite(n)) {
        v[0] /= n;
        v[1] /= n;
        v[2] /= n;
    }
}

// Structure b (one thread): batch_ptr checks, periodic metadata
// (geometry.cpp:123-219) and the grid frame used for binning, into r.  Grid rows:
// dual columns on periodic axes (the grid coordinate is the fractional
// coordinate) and orthonormal complements of the periodic rows elsewhere.
// Per-structure errors go to the record's flags.  OPEN (the molecule plan of
// a plan hint): only structures without periodic axes are set up; any other
// raises ST_PLAN_HINT and gets no geometry, and the pseudo-inverse is not
// compiled in.
template <typename T, bool OPEN = false>
__device__ __forceinline__ void setup_structure(const int64_t* bp, const T* cells,
                                                const uint8_t* pbc, int64_t nb, int64_t n_atoms,
                                                double cutoff, int mw, int64_t b, StructRec& r) {
    unsigned long long st = 0;
    const int64_t lo = bp[b], hi = bp[b + 1];
    if (b == 0 && lo != 0) st |= ST_BP_START;
    if (b == nb - 1 && hi != n_atoms) st |= ST_BP_END;
    if (hi < lo) st |= ST_BP_ORDER;
    const int64_t natoms = hi > lo ? hi - lo : 0;
    r.atom0 = lo;
    r.natoms = natoms;
    r.bin0 = 0;
    r.nbins = 0;
    r.unit0 = 0;
    r.mask0 = 0;
    r.bgroup = 1;
    r.bslices = 1;
    r.bwidth = 1;
    r.mwords = mw;
    r.mneed = 0;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        r.lo[a] = 0.0;
        r.inv_w[a] = 1.0;
        r.reps[a] = 0;
        r.nb[a] = 1;
        r.reach[a] = 1;
    }
#pragma unroll
    for (int e = 0; e < kRedCount; ++e) r.red[e] = 0;
    r.maxp = 0;
    r.maxw = 0;
    r.algo = ALGO_NONE;
    r.any_wrap = 0;
    r.img_total = 0;

    double cell[3][3];
    bool finite = true;
#pragma unroll
    for (int a = 0; a < 3; ++a)
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            cell[a][c] = (double)cells[9 * b + 3 * a + c];
            finite = finite && isfinite(cell[a][c]);
        }
    r.diagonal = cell[0][1] == 0 && cell[0][2] == 0 && cell[1][0] == 0 && cell[1][2] == 0 &&
                 cell[2][0] == 0 && cell[2][1] == 0;
    if (!finite) st |= ST_CELL_NONFINITE;
    const bool px = pbc[3 * b] != 0, py = pbc[3 * b + 1] != 0, pz = pbc[3 * b + 2] != 0;
    const int k = (int)px + (int)py + (int)pz;
    r.active = (px ? 1 : 0) | (py ? 2 : 0) | (pz ? 4 : 0);
    // slot j holds the j-th periodic axis, then the non-periodic ones, in
    // increasing axis order (a lookup on the 3-bit mask keeps indices static)
    int slot_axis[3] = {0, 1, 2};
    switch (r.active) {
        case 2: slot_axis[0] = 1; slot_axis[1] = 0; slot_axis[2] = 2; break;
        case 4: slot_axis[0] = 2; slot_axis[1] = 0; slot_axis[2] = 1; break;
        case 5: slot_axis[0] = 0; slot_axis[1] = 2; slot_axis[2] = 1; break;
        case 6: slot_axis[0] = 1; slot_axis[1] = 2; slot_axis[2] = 0; break;
        default: break;
    }
    r.nimages = 1;
    double dual_slot[3][3] = {{0, 0, 0}, {0, 0, 0}, {0, 0, 0}};
    if (OPEN && k > 0) st |= ST_PLAN_HINT;
    if (finite && natoms > 0 && !(OPEN && k > 0)) {
        double w[3][3];
#pragma unroll
        for (int j = 0; j < 3; ++j)
#pragma unroll
            for (int c = 0; c < 3; ++c)
                w[c][j] = j >= k ? 0.0
                                 : (slot_axis[j] == 0 ? cell[0][c]
                                                      : (slot_axis[j] == 1 ? cell[1][c] : cell[2][c]));
        if constexpr (!OPEN) {
            if (k > 0 && !active_pinv(w, k, dual_slot)) st |= ST_CELL_RANK;
        }
        int64_t reps[3] = {0, 0, 0};
        if (!(st & ST_CELL_RANK)) {
#pragma unroll
            for (int j = 0; j < 3; ++j) {
                if (j >= k) continue;
                const double n2 = dual_slot[0][j] * dual_slot[0][j] +
                                  dual_slot[1][j] * dual_slot[1][j] +
                                  dual_slot[2][j] * dual_slot[2][j];
                if (!isfinite(n2) || !isfinite(dual_slot[0][j]) || !isfinite(dual_slot[1][j]) ||
                    !isfinite(dual_slot[2][j]))
                    st |= ST_DUAL_RANGE;
                const double rep = ceil(cutoff * sqrt(n2));
                if (!(rep <= 2147483647.0))
                    st |= ST_REPEAT_RANGE;
                else
                    reps[j] = (int64_t)rep;
            }
        }
        // per-axis repeats and duals, image count with the 2^24 cap
        int64_t rep_axis[3] = {0, 0, 0};
        double dual_axis[3][3] = {{0, 0, 0}, {0, 0, 0}, {0, 0, 0}};
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            if (j >= k) continue;
            const int a = slot_axis[j];
#pragma unroll
            for (int aa = 0; aa < 3; ++aa)
                if (aa == a) {
                    rep_axis[aa] = reps[j];
#pragma unroll
                    for (int c = 0; c < 3; ++c) dual_axis[c][aa] = dual_slot[c][j];
                }
        }
        const bool geometry_ok = !(st & (ST_REPEAT_RANGE | ST_CELL_RANK | ST_DUAL_RANGE));
        int64_t count = 1;
        if (geometry_ok) {
#pragma unroll
            for (int a = 0; a < 3; ++a) {
                const int64_t f = 2 * rep_axis[a] + 1;
                if (!(st & ST_IMAGE_CAP)) {
                    // count > floor(cap / f) without an integer division
                    // (count <= 2^24 and f <= 2^32 + 1, so the product fits)
                    if (count * f > kImageCap)
                        st |= ST_IMAGE_CAP;
                    else
                        count *= f;
                }
            }
        }
        if (geometry_ok && !(st & ST_IMAGE_CAP)) {
            r.nimages = count;
#pragma unroll
            for (int a = 0; a < 3; ++a) r.reps[a] = (int32_t)rep_axis[a];
            r.img_total = count;
        }
#pragma unroll
        for (int e = 0; e < 9; ++e) r.dual[e] = dual_axis[e / 3][e % 3];
        // grid frame
        double g[3][3] = {{1, 0, 0}, {0, 1, 0}, {0, 0, 1}};
#pragma unroll
        for (int a = 0; a < 3; ++a)
            if (r.active >> a & 1)
#pragma unroll
                for (int c = 0; c < 3; ++c) g[a][c] = dual_axis[c][a];
        if (OPEN) {
            // no periodic axis: the grid frame is the identity
        } else if (k == 2) {
            const int i0 = slot_axis[0], i1 = slot_axis[1], ic = slot_axis[2];
            double r0[3], r1[3], nrm[3];
#pragma unroll
            for (int c = 0; c < 3; ++c) {
                r0[c] = i0 == 0 ? cell[0][c] : (i0 == 1 ? cell[1][c] : cell[2][c]);
                r1[c] = i1 == 0 ? cell[0][c] : (i1 == 1 ? cell[1][c] : cell[2][c]);
            }
            cross3(r0, r1, nrm);
            normalize3(nrm);
#pragma unroll
            for (int a = 0; a < 3; ++a)
                if (a == ic)
#pragma unroll
                    for (int c = 0; c < 3; ++c) g[a][c] = nrm[c];
        } else if (k == 1) {
            const int i0 = slot_axis[0], i1 = slot_axis[1], i2 = slot_axis[2];
            double rr[3];
#pragma unroll
            for (int c = 0; c < 3; ++c)
                rr[c] = i0 == 0 ? cell[0][c] : (i0 == 1 ? cell[1][c] : cell[2][c]);
            normalize3(rr);
            double unit[3] = {0, 0, 0};
            if (fabs(rr[0]) <= fabs(rr[1]) && fabs(rr[0]) <= fabs(rr[2]))
                unit[0] = 1;
            else if (fabs(rr[1]) <= fabs(rr[2]))
                unit[1] = 1;
            else
                unit[2] = 1;
            double e1[3], e2[3];
            cross3(rr, unit, e1);
            normalize3(e1);
            cross3(rr, e1, e2);
            normalize3(e2);
#pragma unroll
            for (int a = 0; a < 3; ++a) {
                if (a == i1)
#pragma unroll
                    for (int c = 0; c < 3; ++c) g[a][c] = e1[c];
                if (a == i2)
#pragma unroll
                    for (int c = 0; c < 3; ++c) g[a][c] = e2[c];
            }
        }
#pragma unroll
        for (int e = 0; e < 9; ++e) r.grid[e] = g[e / 3][e % 3];
    } else {
#pragma unroll
        for (int e = 0; e < 9; ++e) {
            r.dual[e] = 0.0;
            r.grid[e] = (e % 4 == 0) ? 1.0 : 0.0;
        }
    }
    r.flags = st;
}

// Structures per workgroup of the per-structure set-up kernels.
constexpr int kSetupBlock = 64;

// Copies the records of structures [b0, b0 + count) from the workgroup's
// LDS copies to recs (16-byte words, consecutive threads on consecutive
// words); every thread calls it.
__device__ __forceinline__ void store_records(const StructRec* s_recs, StructRec* recs,
                                              int64_t b0, int64_t count) {
    static_assert(sizeof(StructRec) % sizeof(int4) == 0, "records copy as 16-byte words");
    __syncthreads();
    const int64_t words = count * (int64_t)(sizeof(StructRec) / sizeof(int4));
    const int4* src = reinterpret_cast<const int4*>(s_recs);
    int4* dst = reinterpret_cast<int4*>(recs + b0);
    for (int64_t k = threadIdx.x; k < words; k += blockDim.x) dst[k] = src[k];
}

// One thread per structure (setup_structure), kSetupBlock per workgroup,
// each record built in LDS and stored with the workgroup's others
// (store_records).  Block 0 first zeroes the status block of the request
// (every later kernel reads it).  Per-structure errors go to the record
// (k_plan folds them into the status words), so no thread races the zeroing.
// Key word e < kMemoKey of structure b of a request, for a memo entry of
// kind `tag` (kMemoPeriodic with the request's algorithm and reach, or
// kMemoSetup).
template <typename T>
__device__ __forceinline__ unsigned long long memo_key_word(int e, const int64_t* bp,
                                                            const T* cells, const uint8_t* pbc,
                                                            int64_t nb, int64_t b,
                                                            int64_t n_atoms, double cutoff, int mw,
                                                            int requested, int reach_target,
                                                            unsigned long long tag) {
    if (e < 2) return (unsigned long long)bp[b + e];
    if (e < 11) return (unsigned long long)__double_as_longlong((double)cells[9 * b + e - 2]);
    switch (e) {
        case 11:
            return (unsigned long long)(pbc[3 * b] != 0) |
                   (unsigned long long)(pbc[3 * b + 1] != 0) << 8 |
                   (unsigned long long)(pbc[3 * b + 2] != 0) << 16;
        case 12: return (unsigned long long)n_atoms;
        case 13: return (unsigned long long)__double_as_longlong(cutoff);
        case 14: return (unsigned long long)(unsigned)mw;
        case 15: return (unsigned long long)(unsigned)requested;
        case 16: return (unsigned long long)(unsigned)reach_target;
        case 17: return (unsigned long long)sizeof(T);
        case 18: return (unsigned long long)sizeof(StructRec);
        case 19: return (unsigned long long)b;
        case 20: return (unsigned long long)nb;
        default: return tag;
    }
}

// Word i < kMemoWords of the memo's checksum cover (key, flag, record).
__device__ __forceinline__ unsigned long long memo_word(const PeriodicMemo* m, int i) {
    if (i < kMemoKey) return m->key[i];
    if (i == kMemoKey) return m->fast;
    return reinterpret_cast<const unsigned long long*>(&m->rec)[i - kMemoKey - 1];
}

// Word i of the checksum cover, made position-dependent: plus a constant of
// i, rotated by an amount of i (a bijection of the word, so a single changed
// word always changes the checksum); the checksum is the XOR of these.
__device__ __forceinline__ unsigned long long memo_mix(unsigned long long x, int i) {
    x += (unsigned long long)(i + 1) * 0x9e3779b97f4a7c15ull;
    const int r = (i * 7 + 1) & 63;
    return (x << r) | (x >> ((64 - r) & 63));
}

__device__ __forceinline__ unsigned long long wave_xor(unsigned long long x) {
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1) x ^= __shfl_xor(x, d);
    return x;
}

// One thread: whether memo entry m holds the set-up of structure b (every
// key word equal, the flag set and the checksum right); copies the record
// into r when it does.  The key, checksum and flag load together (twelve
// 16-byte loads), the record only when the key matches, eleven 16-byte
// loads at a time.
template <typename T>
__device__ __forceinline__ bool memo_take_setup(const PeriodicMemo* m, const int64_t* bp,
                                                const T* cells, const uint8_t* pbc, int64_t nb,
                                                int64_t b, int64_t n_atoms, double cutoff, int mw,
                                                StructRec& r) {
    static_assert(kMemoKey == 22 && offsetof(PeriodicMemo, check) == 22 * 8 &&
                      offsetof(PeriodicMemo, fast) == 23 * 8 &&
                      offsetof(PeriodicMemo, rec) == 24 * 8,
                  "key, checksum and flag fill the first twelve 16-byte words");
    const ulonglong2* head = reinterpret_cast<const ulonglong2*>(m);
    ulonglong2 kw[12];
#pragma unroll
    for (int q = 0; q < 12; ++q) kw[q] = head[q];
    bool same = kw[11].y == 1ull;
    unsigned long long h = memo_mix(1ull, kMemoKey);
#pragma unroll
    for (int i = 0; i < kMemoKey; ++i) {
        const unsigned long long w = (i & 1) ? kw[i / 2].y : kw[i / 2].x;
        same = same && w == memo_key_word<T>(i, bp, cells, pbc, nb, b, n_atoms, cutoff, mw, 0, 0,
                                              kMemoSetup);
        h ^= memo_mix(w, i);
    }
    if (!same) return false;
    constexpr int kRecWords = (int)(sizeof(StructRec) / sizeof(ulonglong2));
    static_assert(kRecWords == 33, "the record loads in three batches of eleven");
    const ulonglong2* src = reinterpret_cast<const ulonglong2*>(&m->rec);
    ulonglong2* dst = reinterpret_cast<ulonglong2*>(&r);
#pragma unroll
    for (int q0 = 0; q0 < kRecWords; q0 += 11) {
        ulonglong2 x[11];
#pragma unroll
        for (int q = 0; q < 11; ++q) x[q] = src[q0 + q];
#pragma unroll
        for (int q = 0; q < 11; ++q) {
            h ^= memo_mix(x[q].x, kMemoKey + 1 + 2 * (q0 + q));
            h ^= memo_mix(x[q].y, kMemoKey + 2 + 2 * (q0 + q));
            dst[q0 + q] = x[q];
        }
    }
    return h == kw[11].x;
}

// One thread: stores record r (the set-up of structure b) into memo entry m.
template <typename T>
__device__ __forceinline__ void memo_put_setup(PeriodicMemo* m, const StructRec& r,
                                               const int64_t* bp, const T* cells,
                                               const uint8_t* pbc, int64_t nb, int64_t b,
                                               int64_t n_atoms, double cutoff, int mw) {
    unsigned long long h = 0;
    for (int i = 0; i < kMemoKey; ++i) {
        const unsigned long long k =
            memo_key_word<T>(i, bp, cells, pbc, nb, b, n_atoms, cutoff, mw, 0, 0, kMemoSetup);
        m->key[i] = k;
        h ^= memo_mix(k, i);
    }
    m->fast = 1ull;
    h ^= memo_mix(1ull, kMemoKey);
    const unsigned long long* rw = reinterpret_cast<const unsigned long long*>(&r);
    unsigned long long* mr = reinterpret_cast<unsigned long long*>(&m->rec);
    for (int j = 0; j < kMemoRecWords; ++j) {
        mr[j] = rw[j];
        h ^= memo_mix(rw[j], kMemoKey + 1 + j);
    }
    m->check = h;
}

template <typename T>
__global__ __launch_bounds__(kSetupBlock) void k_setup(const int64_t* bp, const T* cells,
                                                       const uint8_t* pbc, int64_t nb,
                                                       int64_t n_atoms, double cutoff, int mw,
                                                       StructRec* recs,
                                                       unsigned long long* status,
                                                       PeriodicMemo* memo) {
    __shared__ StructRec s_recs[kSetupBlock];
    const int64_t b0 = (int64_t)blockIdx.x * kSetupBlock;
    const int64_t b = b0 + threadIdx.x;
    if (blockIdx.x == 0) {
        for (int k = threadIdx.x; k < SS_SLOTS; k += blockDim.x) status[k] = 0;
        __syncthreads();
        if (nb == 0 && threadIdx.x == 0) {
            unsigned long long st = 0;
            if (bp[0] != 0) st |= ST_BP_START;
            if (bp[0] != n_atoms) st |= ST_BP_END;
            status[SS_FLAGS] = st;
        }
    }
    // the set-up of an earlier request with the same inputs, when the memo
    // holds it; otherwise derived and stored there for the next request
    if (b < nb && !memo_take_setup<T>(memo + b, bp, cells, pbc, nb, b, n_atoms, cutoff, mw,
                                       s_recs[threadIdx.x])) {
        setup_structure<T>(bp, cells, pbc, nb, n_atoms, cutoff, mw, b, s_recs[threadIdx.x]);
        memo_put_setup<T>(memo + b, s_recs[threadIdx.x], bp, cells, pbc, nb, b, n_atoms, cutoff,
                          mw);
    }
    if (b0 < nb) store_records(s_recs, recs, b0, min((int64_t)kSetupBlock, nb - b0));
}

// Structure of atom i: the b in [lo, hi) with bp[b] <= i < bp[b + 1]
// (batch_ptr valid, the answer known to lie in [lo, hi)).
__device__ __forceinline__ int structure_of(const int64_t* bp, int64_t lo, int64_t hi, int64_t i) {
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) >> 1;
        if (bp[mid] <= i) lo = mid; else hi = mid;
    }
    return (int)lo;
}

// The same for a wave-uniform i, by the whole wave: 64 candidates per step
// (one load per lane), so a batch of B structures takes log64(B) loads.
__device__ __forceinline__ int structure_of_wave(const int64_t* bp, int64_t nb, int64_t i) {
    const int lane = lane_id();
    int64_t lo = 0, len = nb;
    while (len > 1) {
        const int64_t step = (len + kWave - 1) / kWave;
        const int64_t at = (int64_t)lane * step;
        const bool le = at < len && bp[lo + at] <= i;
        const unsigned long long m = ballot(le) | 1ull;
        const int64_t last = 63 - __builtin_clzll(m);
        lo += last * step;
        len = min(step, len - last * step);
    }
    return (int)lo;
}

// floor(sum_c x_c * y_c) with double-double accumulation (nearly exact), as
// the reference's long-double fractional coordinate (neighbors_cpu.cpp:110-
// 122); *ok becomes false when the value is non-finite or outside
// [-2^31, 2^31).
__device__ __forceinline__ int wrap_of(const double x[3], const double y[3], bool* ok) {
    double hi = 0, lo = 0;
#pragma unroll
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
#pragma unroll
    for (int a = 0; a < 3; ++a)
        u[a] = r.grid[3 * a] * (double)q[0] + r.grid[3 * a + 1] * (double)q[1] +
               r.grid[3 * a + 2] * (double)q[2];
}

// One thread per atom: finiteness, representative wraps and wrapped
// positions (neighbors_cpu.cpp:92-133), and the per-structure reductions the
// planner needs (grid-coordinate and Cartesian bounds, max |p|, max |wrap|).
// A block whose atoms all lie in one structure writes one BlockPartial
// without atomics; a block spanning several structures uses atomics on the
// structure records (each such structure is small, so contention is low).
// The grid also zeroes the bin counters, the tile states of the two
// single-pass scans and the per-source pair counts (sliced brute-force
// sources add theirs), which later kernels of the request use.
//
// SINGLE (a request of one structure with atoms): the grid also does the
// work of k_setup.  Every block derives the structure's record in LDS
// (thread 0) and block 0 stores it; the atoms' error bits go to the block's
// partial instead of the status words, which k_single_bin writes.
template <typename T, bool SINGLE>
__global__ __launch_bounds__(kBlock) void k_atoms(const T* pos, const int64_t* bp,
                                                   const T* cells, const uint8_t* pbc,
                                                   double cutoff, int mw, int64_t nb,
                                                   int64_t n_atoms,
                                                   StructRec* recs, BlockPartial* partials,
                                                   int* atom_struct, int4* atom_wrap,
                                                   Vec4<T>* atom_q, unsigned long long* status,
                                                   int* bin_count, int64_t n_bin_count,
                                                   unsigned long long* tiles, int64_t n_tiles,
                                                   long long* counts) {
    __shared__ unsigned long long s_red[kWavesPerBlock][kRedCount];
    __shared__ unsigned long long s_flags, s_atom_flags;
    __shared__ StructRec s_rec;
    {
        const int64_t stride = (int64_t)gridDim.x * kBlock;
        if ((int64_t)blockIdx.x * kBlock + threadIdx.x < n_atoms)
            counts[(int64_t)blockIdx.x * kBlock + threadIdx.x] = 0;
        for (int64_t k = (int64_t)blockIdx.x * kBlock + threadIdx.x; k < n_bin_count; k += stride)
            bin_count[k] = 0;
        for (int64_t k = (int64_t)blockIdx.x * kBlock + threadIdx.x; k < n_tiles; k += stride)
            tiles[k] = 0;
    }
    // the atom's position loads while thread 0 derives the record
    const int64_t ia = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    const int64_t ic = ia < n_atoms ? ia : (n_atoms > 0 ? n_atoms - 1 : 0);
    T p_pre[3] = {T(0), T(0), T(0)};
    if (n_atoms > 0)
#pragma unroll
        for (int c = 0; c < 3; ++c) p_pre[c] = pos[3 * ic + c];
    // Block-uniform early exit (the barrier below needs every thread).
    if (threadIdx.x == 0) {
        if constexpr (SINGLE) {
            setup_structure<T>(bp, cells, pbc, 1, n_atoms, cutoff, mw, 0, s_rec);
            if (blockIdx.x == 0) recs[0] = s_rec;
            s_flags = s_rec.flags;
            s_atom_flags = 0;
        } else {
            s_flags = load_status(status + SS_FLAGS);
        }
    }
    __syncthreads();
    if (s_flags & kAbortBits) {
        if (SINGLE && threadIdx.x == 0) partials[blockIdx.x].flags = 0;
        return;
    }
    const int64_t first = (int64_t)blockIdx.x * kBlock;
    const int64_t last = (first + kBlock < n_atoms ? first + kBlock : n_atoms) - 1;
    const int64_t i = first + threadIdx.x;
    const bool valid = i < n_atoms;
    const int bfirst = SINGLE ? 0 : __builtin_amdgcn_readfirstlane(structure_of_wave(bp, nb, first));
    const int blast = SINGLE ? 0 : __builtin_amdgcn_readfirstlane(structure_of_wave(bp, nb, last));
    const bool uniform = bfirst == blast;
    int b = bfirst;
    bool good = false;
    T q[3] = {T(0), T(0), T(0)};
    int w[3] = {0, 0, 0};
    double u[3] = {0, 0, 0};
    double pabs[3] = {0, 0, 0};
    unsigned long long st = 0;
    if (valid) {
        b = uniform ? bfirst : structure_of(bp, bfirst, (int64_t)blast + 1, i);
        atom_struct[i] = b;
        const StructRec& r = SINGLE ? s_rec : recs[b];
        T p[3];
        bool finite = true;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            p[c] = p_pre[c];
            finite = finite && isfinite((double)p[c]);
        }
        if (r.flags & kAbortBits) {
            // a structure with input errors: the request fails, nothing to compute
        } else if (!finite) {
            st |= ST_POS_NONFINITE;
        } else {
            const double pd[3] = {(double)p[0], (double)p[1], (double)p[2]};
            bool ok = true;
#pragma unroll
            for (int a = 0; a < 3; ++a) {
                const double dcol[3] = {(double)(T)r.dual[a], (double)(T)r.dual[3 + a],
                                        (double)(T)r.dual[6 + a]};
                w[a] = wrap_of(pd, dcol, &ok);
            }
            if (!ok) {
                st |= ST_WRAP_RANGE;
            } else {
                const T* cell = cells + 9 * b;
#pragma unroll
                for (int c = 0; c < 3; ++c) {
                    T x = p[c];
#pragma unroll
                    for (int a = 0; a < 3; ++a)
                        x = Ops<T>::sub(x, Ops<T>::mul((T)w[a], cell[3 * a + c]));
                    q[c] = x;
                }
                grid_coords(r, q, u);
#pragma unroll
                for (int c = 0; c < 3; ++c) pabs[c] = fabs(pd[c]);
                good = true;
            }
        }
        atom_wrap[i] = make_int4(w[0], w[1], w[2], 0);
        atom_q[i] = Vec4<T>{q[0], q[1], q[2], idx_as((int)i, T(0))};
    }
    if (st) {
        if constexpr (SINGLE)
            atomicOr(&s_atom_flags, st);
        else
            atomicOr(status + SS_FLAGS, st);
    }

    // the 18 reductions as max-keys (0 = identity for atoms that contribute nothing)
    using K = RedKeys<T>;
    unsigned long long v[kRedCount];
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        v[kRedUlo + a] = good ? K::lower(u[a]) : 0ull;
        v[kRedUhi + a] = good ? K::upper(u[a]) : 0ull;
        v[kRedClo + a] = good ? K::lower_exact(q[a]) : 0ull;
        v[kRedChi + a] = good ? K::upper_exact(q[a]) : 0ull;
    }
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        v[kRedP + c] = good ? K::magnitude(pabs[c]) : 0ull;
        v[kRedW + c] = good ? (unsigned long long)abs(w[c]) : 0ull;
    }
    if (uniform) {
        const int wv = threadIdx.x / kWave;
#pragma unroll
        for (int e = 0; e < kRedCount; ++e) v[e] = K::wave_max(v[e]);
        if (lane_id() == 0)
#pragma unroll
            for (int e = 0; e < kRedCount; ++e) s_red[wv][e] = v[e];
        __syncthreads();
        if (threadIdx.x < kRedCount) {
            const int e = threadIdx.x;
            unsigned long long x = s_red[0][e];
#pragma unroll
            for (int k = 1; k < kWavesPerBlock; ++k) x = s_red[k][e] > x ? s_red[k][e] : x;
            partials[blockIdx.x].red[e] = x;
        }
        if (threadIdx.x == kRedCount) partials[blockIdx.x].flags = SINGLE ? s_atom_flags : 0ull;
    } else {
        // several structures: a segmented maximum per wave, then one atomic
        // per (wave, structure, reduction) from the segment's last lane
        const int lane = lane_id();
        const int bprev = __shfl_up(b, 1);
        const unsigned long long heads = __builtin_amdgcn_ballot_w64(lane == 0 || bprev != b);
        const unsigned long long below = heads & (lane == kWave - 1 ? ~0ull : ((2ull << lane) - 1));
        const int head = kWave - 1 - __builtin_clzll(below);
        const unsigned long long next_head = heads >> 1;  // bit l: lane l + 1 starts a segment
        const bool tail = lane == kWave - 1 || ((next_head >> lane) & 1ull);
#pragma unroll
        for (int e = 0; e < kRedCount; ++e) v[e] = segment_max_u64(v[e], head);
        if (tail && valid) {
            StructRec& r = recs[b];
#pragma unroll
            for (int e = 0; e < kRedCount; ++e)
                if (v[e]) atomicMax(&r.red[e], v[e]);
        }
    }
}


// Margins of a structure from the reductions of its atoms (max |p|, max
// |wrap|): the broad-phase margin pad = 64 eps_T max(scale, rc), with scale =
// 2 max|p| + sum_a (R_a + 2 max|w|) max_c |cell_ac| the operation scale of
// neighbors_cpu.cpp:156-219, which sizes the bins, and the half-width of the
// band the public predicate decides.  With wrapped atoms the band is the
// padding above.  Without (every wrap zero, so the wrapped positions are the
// positions): per component, the broad-phase D of the cell-list walk (p_t +
// k.cell, minus p_s) and of the brute-force walk ((p_t - p_s) + k.cell,
// fused) differ from the exact value by at most u (5 |D| + |p| + 4 B) and u
// (4 |D| + 7 B), the public D by u (4 |D| + 8 B), with u = eps / 2 and B =
// max_c sum_a R_a |cell_ac| the largest image translation; over three
// components and the d2 roundings (at most 4 u d together), |d_broad -
// d_public| <= u (17.9 rc + 1.74 max|p| + 26 B) near the cutoff, first
// order.  Twice that bound is the band.
struct Margins {
    double pad, band, maxp;
    unsigned maxw;
    bool safe;  // the padded cutoff is finite and at most 2 rc (bins of it are usable)
};

template <typename T>
__device__ __forceinline__ Margins plan_margins(const double cell[9], const StructRec& r,
                                                double maxp, unsigned maxw_u, double rc) {
    Margins m;
    const double maxw = (double)maxw_u;
    const int R0 = r.reps[0], R1 = r.reps[1], R2 = r.reps[2];
    double scale = 0, bmax = 0;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        const double sc = 2 * maxp + ((double)R0 + 2 * maxw) * fabs(cell[c]) +
                          ((double)R1 + 2 * maxw) * fabs(cell[3 + c]) +
                          ((double)R2 + 2 * maxw) * fabs(cell[6 + c]);
        scale = fmax(scale, sc);
        bmax = fmax(bmax, (double)R0 * fabs(cell[c]) + (double)R1 * fabs(cell[3 + c]) +
                              (double)R2 * fabs(cell[6 + c]));
    }
    m.pad = 64.0 * Ops<T>::eps * fmax(scale, rc);
    m.band = maxw_u == 0 ? fmin(m.pad, Ops<T>::eps * (18.0 * rc + 1.75 * maxp + 26.0 * bmax))
                         : m.pad;
    m.maxp = maxp;
    m.maxw = maxw_u;
    m.safe = isfinite(rc + m.pad) && rc + m.pad <= 2 * rc && rc + m.pad <= Ops<T>::max;
    return m;
}

// The record's thresholds from the margins (one writer).
template <typename T>
__device__ __forceinline__ void write_margins(StructRec& r, const Margins& m, double cutoff) {
    const double rc = cutoff;
    const double inner = rc - m.band;
    r.pad = m.pad;
    r.maxp = (unsigned long long)__double_as_longlong(m.maxp);
    r.maxw = m.maxw;
    r.any_wrap = m.maxw != 0;
    r.inner2 = inner > 0 ? (double)Ops<T>::down(inner * inner) : 0.0;
    r.outer2 = (double)Ops<T>::up((rc + m.band) * (rc + m.band));
    r.cut2 = (double)(T)(cutoff * cutoff);
}

// Largest |p_c| over the components and largest |wrap_a| over the axes,
// from the per-component reductions (the keys order as the values do).
template <typename T>
__device__ __forceinline__ double red_pmax(const unsigned long long red[kRedCount]) {
    unsigned long long k = red[kRedP];
    k = red[kRedP + 1] > k ? red[kRedP + 1] : k;
    k = red[kRedP + 2] > k ? red[kRedP + 2] : k;
    return RedKeys<T>::magnitude_value(k);
}
__device__ __forceinline__ unsigned red_wmax(const unsigned long long red[kRedCount]) {
    unsigned long long k = red[kRedW];
    k = red[kRedW + 1] > k ? red[kRedW + 1] : k;
    k = red[kRedW + 2] > k ? red[kRedW + 2] : k;
    return (unsigned)k;
}

// The reference's CPU refusal of an explicit cell_list ("cell_list cannot
// safely process this structure"), evaluated as it does.  The padded search
// cutoff (neighbors_cpu.cpp:157-218): the operation scale, max over c of
// 2 max|p_c| + sum_a (R_a + 2 max|w_a|) |cell_ac|, and cutoff + 64 eps_T
// scale in x87 long double (emulated, Ext), rounded to T and moved up one
// ulp; refused when that is not finite or exceeds 2 cutoff or T's maximum.
// Then the dense bin layout over the wrapped positions' bounding box in T
// arithmetic (neighbors_cpu.cpp:379-430): per axis span = (max - min) + 2
// size and span / size bins, refused beyond 2^26 bins in all or more than
// 64 bins per atom image.  cell holds the structure's cell entries (values
// of T); n atoms, r.nimages images.  True when refused.
template <typename T>
__device__ __forceinline__ bool cell_unsafe(const unsigned long long red[kRedCount],
                                            const StructRec& r, const double cell[9],
                                            double cutoff, int64_t n) {
    using K = RedKeys<T>;
    using O = Ops<T>;
    constexpr int64_t kDenseBins = int64_t{1} << 26;
    const T rc = (T)cutoff;
    {
        // Far from the limits, as nearly every structure is: the search
        // cutoff is at least rc (the pad is not negative and the rounding
        // monotone), so the bins per axis are at most ceil((max - min) / rc
        // + 2), widened by 1e-6 for T's roundings; with the padding bounded
        // above in double (1e-9 beyond its roundings), a layout that fits
        // the limits is accepted without the long double evaluation.
        double scale_hi = 0.0;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            double comp = 2.0 * K::magnitude_value(red[kRedP + c]);
#pragma unroll
            for (int a = 0; a < 3; ++a)
                comp += ((double)r.reps[a] + 2.0 * (double)(unsigned)red[kRedW + a]) *
                        fabs(cell[3 * a + c]);
            scale_hi = fmax(scale_hi, comp);
        }
        const double padded_hi = ((double)rc + 64.0 * O::eps * scale_hi) * (1.0 + 1e-9);
        if (padded_hi < 2.0 * (double)rc && padded_hi <= (double)O::max) {
            double bins = 1.0;
#pragma unroll
            for (int c = 0; c < 3; ++c) {
                const double span = K::upper_value(red[kRedChi + c]) - K::lower_value(red[kRedClo + c]);
                bins *= fmax(1.0, ceil((span / (double)rc + 2.0) * (1.0 + 1e-6)));
            }
            if (bins <= (double)kDenseBins && ceil(bins / 64.0) <= (double)n * (double)r.nimages)
                return false;
        }
    }
    Ext scale = ext_exact(0.0);
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        Ext comp = ext_exact(2.0 * K::magnitude_value(red[kRedP + c]));
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            const double shift = (double)r.reps[a] + 2.0 * (double)(unsigned)red[kRedW + a];
            comp = ext_add(comp, ext_mul(shift, fabs(cell[3 * a + c])));
        }
        if (ext_less(scale, comp)) scale = comp;
    }
    // 64 eps_T = 2^-17 (float) or 2^-46 (double): the product is exact
    const Ext padded = ext_add(ext_exact((double)rc), ext_scale(scale, sizeof(T) == 4 ? -17 : -46));
    if (!isfinite(padded.hi) || ext_less(ext_exact(2.0 * (double)rc), padded) ||
        ext_less(ext_exact((double)O::max), padded))
        return true;
    const T size = nextafter(ext_to<T>(padded), (T)INFINITY);
    if (!isfinite((double)size)) return true;
    int64_t count = 1;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        const T lo = (T)K::lower_value(red[kRedClo + c]);
        const T hi = (T)K::upper_value(red[kRedChi + c]);
        const T span = O::add(O::sub(hi, lo), O::mul(T(2), size));
        const T dim = span / size;  // correctly rounded (IEEE division)
        if (!isfinite((double)dim) || (double)dim > (double)kDenseBins) return true;
        const int64_t d = max((int64_t)1, (int64_t)ceil((double)dim));
        if (count > kDenseBins / d) return true;
        count *= d;
    }
    return !(count <= kDenseBins && (count + 63) / 64 <= n * r.nimages);
}

// A bin grid of a cell-list structure: bins per axis, bins per grid unit,
// origin, stencil reach and z segments per stencil row.
struct GridPlan {
    double inv_w[3], lo[3];
    int nb[3], reach[3];
    int zs;
    int64_t nbins;
};

// z segments per stencil row for a z reach of Kz bins over nz bins.
__device__ __forceinline__ int stencil_zseg(bool perz, int Kz, int nz) {
    if (!perz) return 1;
    const int span = 2 * Kz + 1;
    return min(span, (span + nz - 1) / nz + 1);
}

// Bin grid for a stencil reach of kt bins per padded cutoff, run by all lanes
// of one wave.  With reach_target 0 the reach is chosen per structure by an
// estimated cost per source: the stencil candidates (distance tests) times
// 1 + kBinOverhead / (sources per bin), since every bin builds and stages its
// stencil once for all of its sources; stencils beyond the mask capacity take
// the slow path and count four times.  The candidate reaches are evaluated
// one per lane.  red (the reduced bounds) is read for non-periodic axes only.
// Returns false, in every lane, when no grid fits (the structure then stays
// with brute force, whose pairs are the same set): where the cutoff spans two
// or more cell widths on every periodic axis (one bin per axis, a reach of
// three bins: 7^3 stencil pieces, beyond kPieceCap), or beyond about 2^24
// atoms.
template <typename T>
__device__ __forceinline__ bool choose_grid(const StructRec& r, const unsigned long long* red,
                                            double rc, double pad, int64_t n, int reach_target,
                                            GridPlan& gp) {
    using K = RedKeys<T>;
    const int active = r.active;
    const double rcu0 = rc + 2 * pad;
    const int k_lo = reach_target > 0 ? reach_target : 1;
    const int k_hi = reach_target > 0 ? reach_target : 4;
    const int lane = lane_id();
    const int kt_i = min(k_lo + lane, k_hi);
    const double kt = (double)kt_i;
    double ext[3], wdt[3], nbf[3], rcu[3], lo[3];
    bool ok = k_lo + lane <= k_hi;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        const double gn = sqrt(r.grid[3 * a] * r.grid[3 * a] + r.grid[3 * a + 1] * r.grid[3 * a + 1] +
                               r.grid[3 * a + 2] * r.grid[3 * a + 2]);
        rcu[a] = rcu0 * gn;
        lo[a] = 0.0;
        if (active >> a & 1) {
            ext[a] = 1.0;
            nbf[a] = fmin(fmax(ceil(kt / rcu[a]) - 1.0, 1.0), 1048576.0);
            wdt[a] = 1.0 / nbf[a];
        } else {
            lo[a] = K::lower_value(red[kRedUlo + a]);
            const double hi = K::upper_value(red[kRedUhi + a]);
            ext[a] = fmax(hi - lo[a], 0.0);
            if (!isfinite(ext[a]) || !isfinite(lo[a])) ok = false;
            wdt[a] = rcu[a] / kt * (1.0 + 1e-9);
            if (ext[a] / wdt[a] > 1048575.0) wdt[a] = ext[a] / 1048575.0 * (1.0 + 1e-9);
            if (!(wdt[a] > 0) || !isfinite(wdt[a])) wdt[a] = 1.0;
            nbf[a] = fmin(floor(ext[a] / wdt[a]) + 1.0, 1048576.0);
        }
    }
    const double capb = 2.0 * (double)n + 64.0;
    for (int it = 0; it < 200 && nbf[0] * nbf[1] * nbf[2] > capb; ++it) {
        const int a = (nbf[0] >= nbf[1] && nbf[0] >= nbf[2]) ? 0 : (nbf[1] >= nbf[2] ? 1 : 2);
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            if (c != a) continue;
            if (active >> c & 1) {
                nbf[c] = ceil(nbf[c] / 2.0);
                wdt[c] = 1.0 / nbf[c];
            } else {
                wdt[c] *= 2.0;
                nbf[c] = fmin(floor(ext[c] / wdt[c]) + 1.0, 1048576.0);
            }
        }
    }
    int reach[3];
    bool reach_ok = true;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        const double rd = floor(rcu[a] / wdt[a] * (1.0 + 1e-12)) + 1.0;
        reach_ok = reach_ok && rd < 256.0;
        reach[a] = rd < 256.0 ? (int)rd : 1;
    }
    const int rows = (2 * reach[0] + 1) * (2 * reach[1] + 1);
    const int zs = stencil_zseg(active >> 2 & 1, reach[2], (int)nbf[2]);
    const bool fits = ok && reach_ok && nbf[0] * nbf[1] * nbf[2] <= capb &&
                      (long long)rows * zs <= kPieceCap &&
                      (double)n * (double)(rows * zs) < 2147483647.0;
    // estimated candidates of a stencil and sources of a bin
    const double bins_f = nbf[0] * nbf[1] * nbf[2];
    const double per_bin = (double)n / bins_f;
    double span_bins = 1.0;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        const double w = 2.0 * reach[a] + 1.0;
        span_bins *= (active >> a & 1) ? w : fmin(w, nbf[a]);
    }
    const double cand = span_bins * per_bin;
    double cost = cand * (1.0 + kBinOverhead / fmax(per_bin, 1e-9)) *
                  (cand > (double)(kMaskWords * kWave) ? 4.0 : 1.0);
    // the cheapest fitting reach, the smallest on ties
    cost = fits ? fmin(cost, 1.7976931348623157e308) : INFINITY;
    int best = lane;
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1) {
        const double oc = __shfl_xor(cost, d);
        const int ob = __shfl_xor(best, d);
        if (oc < cost || (oc == cost && ob < best)) {
            cost = oc;
            best = ob;
        }
    }
    best = __builtin_amdgcn_readfirstlane(best);
    if (!(cost < INFINITY)) return false;
    gp.nbins = (int64_t)__shfl(bins_f, best);
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        gp.nb[a] = (int)__shfl(nbf[a], best);
        gp.inv_w[a] = __shfl((active >> a & 1) ? nbf[a] : 1.0 / wdt[a], best);
        gp.lo[a] = __shfl(lo[a], best);
        gp.reach[a] = __shfl(reach[a], best);
    }
    gp.zs = __shfl(zs, best);
    return true;
}

// Brute-force work units of a structure of n atoms (one writer): units of
// bgroup consecutive sources, and for periodic structures k0 slices.
__device__ __forceinline__ int64_t plan_brute_units(StructRec& r, int64_t n) {
    int64_t units = 0;
    if (molecule_path(r.active, n)) r.mneed = molecule_words(n);
    if (molecule_rec(r)) {
        // a molecule: sources x chunks of 64 targets per unit
        const int chunks = (int)((n + kWave - 1) / kWave);
        const int g = (int)min((int64_t)max(kMolUnitWork / chunks, 1), n);
        r.bgroup = g;
        units = (n + g - 1) / g;
    } else {
        // a round: 64 (source, k0, target) triples, each walking the
        // K1 x K2 images of its k0 plane, costing about 1 + K1 K2 / 4.
        // A source whose K0 planes exceed a unit's work is split into
        // slices of k0 (at most kMaxSlices, and no more than the words of
        // an atom's hit-mask row: their counts are kept in the source's
        // row).
        const int64_t K0 = 2 * (int64_t)r.reps[0] + 1;
        const double round = 1.0 + 0.25 * (double)r.nimages / (double)K0;
        const double want = fmax(kBruteUnitWork / round, 1.0);     // rounds per unit
        const double per_source = (double)n * (double)K0 / kWave;  // rounds per source
        double g = floor(want / per_source);
        int64_t nsl = 1, width = K0;
        if (g < 1.0) {
            g = 1.0;
            const int64_t cap = K0 < kMaxSlices ? K0 : kMaxSlices;
            const int64_t wanted = (int64_t)fmin(ceil(per_source / want), (double)cap);
            if (wanted > 1) r.mneed = max(r.mneed, (int32_t)wanted);
            nsl = min(wanted, (int64_t)r.mwords);
            width = (K0 + nsl - 1) / nsl;
            nsl = (K0 + width - 1) / width;
        }
        g = fmin(fmin(g, (double)n), (double)kBruteGroupCap);
        r.bgroup = (int32_t)g;
        r.bslices = (int32_t)nsl;
        r.bwidth = (int32_t)width;
        units = (n + (int64_t)g - 1) / (int64_t)g * nsl;
    }
    return units;
}

// Planner of one structure, run by all lanes of one wave (lane 0 writes the
// record and the per-structure arrays): from the reduced bounds red (see
// k_plan) the margins (plan_margins), the algorithm and the bin grid
// (choose_grid) or the brute-force work units.
template <typename T>
__device__ __forceinline__ void plan_structure(const T* cells, int64_t b, StructRec& r,
                                               const unsigned long long red[kRedCount],
                                               double cutoff, int requested, int reach_target,
                                               long long* struct_bins, long long* struct_units) {
    using K = RedKeys<T>;
    const bool writer = lane_id() == 0;
    const int64_t n = r.natoms;
    if (n == 0) {
        if (writer) {
            r.algo = ALGO_NONE;
            r.nbins = 0;
            struct_bins[b] = 0;
            struct_units[b] = 0;
        }
        return;
    }
    double cell[9];
#pragma unroll
    for (int e = 0; e < 9; ++e) cell[e] = (double)cells[9 * b + e];
    const double rc = cutoff;
    const Margins m = plan_margins<T>(cell, r, red_pmax<T>(red), red_wmax(red), rc);
    if (writer) write_margins<T>(r, m, cutoff);
    const int64_t nimages = r.nimages;
    // n > floor(limit / nimages), as a product (nimages <= 2^24)
    const bool large = r.active != 0 ? n * nimages > kAutoBrutePeriodic : n > kAutoBruteIsolated;
    bool want_cell = requested == TNR_CELL_LIST || (requested == TNR_AUTO && large);
    unsigned long long st = 0;
    if (requested == TNR_CELL_LIST && cell_unsafe<T>(red, r, cell, cutoff, n)) st |= ST_CELL_UNSAFE;
    if (!m.safe) want_cell = false;
    int algo = ALGO_BRUTE;
    int64_t nbins = 0;
    GridPlan gp;
    // An explicit cell_list request whose structure no grid fits has its
    // brute-force structures counted by the cell-list counting kernel.
    if (want_cell && choose_grid<T>(r, red, rc, m.pad, n, reach_target, gp)) {
        algo = ALGO_CELL;
        nbins = gp.nbins;
        if (writer) {
#pragma unroll
            for (int a = 0; a < 3; ++a) {
                r.nb[a] = (int32_t)gp.nb[a];
                r.inv_w[a] = gp.inv_w[a];
                r.lo[a] = gp.lo[a];
                r.reach[a] = gp.reach[a];
            }
            r.zseg = gp.zs;
        }
    }
    if (writer) {
        r.algo = algo;
        r.nbins = nbins;
        struct_bins[b] = nbins;
        struct_units[b] = algo == ALGO_BRUTE ? plan_brute_units(r, n) : 0;
        r.flags |= st;
    }
}

// The grid of the periodic fast prologue, run by all lanes of one wave: for a
// fully periodic structure planned as a cell list (an explicit cell_list, or
// auto above the brute-force crossover), the grid choose_grid picks with the
// margin of atoms inside the cell (max |p_c| <= sum_a |cell_ac|, no wraps).
// False, in every lane, when the fast prologue does not apply.  k_single_bin
// runs it too, so that the plan bit it reports is exactly this condition.
template <typename T>
__device__ __forceinline__ bool periodic_grid(const StructRec& r, const T* cells, double cutoff,
                                              int requested, int reach_target, GridPlan& gp) {
    const int64_t n = r.natoms;
    if ((r.flags & kAbortBits) || r.active != 7 || n <= 0 || requested == TNR_BRUTE_FORCE)
        return false;
    if (requested == TNR_AUTO && !(n * r.nimages > kAutoBrutePeriodic)) return false;
    double cell[9];
#pragma unroll
    for (int e = 0; e < 9; ++e) cell[e] = (double)cells[e];
    double maxp = 0;
#pragma unroll
    for (int c = 0; c < 3; ++c) maxp = fmax(maxp, fabs(cell[c]) + fabs(cell[3 + c]) + fabs(cell[6 + c]));
    const Margins m = plan_margins<T>(cell, r, maxp, 0u, cutoff);
    if (!m.safe) return false;
    return choose_grid<T>(r, nullptr, cutoff, m.pad, n, reach_target, gp);
}

// One workgroup per structure: combines the block partials of k_atoms (all
// loads in flight at once) with the atomics of shared blocks, and plans the
// structure (plan_structure).  Results stay in the structure's record and
// the per-structure arrays; k_struct_scan combines them for the batch (for a
// single structure, with `fused_scan`, this workgroup does it itself).
template <typename T>
__global__ __launch_bounds__(kBlock) void k_plan(const T* cells, int64_t nb, int64_t n_atoms,
                                                  double cutoff, int requested, int reach_target,
                                                  StructRec* recs, const BlockPartial* partials,
                                                  long long* struct_bins, long long* bin_off,
                                                  long long* struct_units, long long* unit_off,
                                                  int64_t cap_bins, unsigned long long* status,
                                                  int fused_scan, PlanSummary* meta) {
    using K = RedKeys<T>;
    __shared__ unsigned long long s_red[kWavesPerBlock][kRedCount];
    const int64_t b = blockIdx.x;
    const int tid = threadIdx.x, lane = lane_id(), wv = tid / kWave;
    if (b < nb) {
        StructRec& r = recs[b];
        const unsigned long long flags = r.flags;
        if ((flags & kAbortBits) || (load_status(status + SS_FLAGS) & kAbortBits)) {
            if (tid == 0) {
                struct_bins[b] = 0;
                struct_units[b] = 0;
            }
        } else {
            const int64_t n = r.natoms;
            unsigned long long v[kRedCount];
#pragma unroll
            for (int e = 0; e < kRedCount; ++e) v[e] = r.red[e];
            if (n > 0) {
                // partials of the k_atoms blocks that lie inside this structure
                const int64_t k0 = r.atom0 / kBlock, k1 = (r.atom0 + n - 1) / kBlock;
#pragma unroll 4
                for (int64_t kb = k0 + tid; kb <= k1; kb += kBlock) {
                    const int64_t first = kb * kBlock;
                    const int64_t last = (first + kBlock < n_atoms ? first + kBlock : n_atoms) - 1;
                    const bool inside = first >= r.atom0 && last < r.atom0 + n;
#pragma unroll
                    for (int e = 0; e < kRedCount; ++e) {
                        const unsigned long long x = partials[kb].red[e];
                        if (inside) v[e] = x > v[e] ? x : v[e];
                    }
                }
            }
#pragma unroll
            for (int e = 0; e < kRedCount; ++e) v[e] = K::wave_max(v[e]);
            if (lane == 0)
#pragma unroll
                for (int e = 0; e < kRedCount; ++e) s_red[wv][e] = v[e];
            __syncthreads();
            if (wv == 0) {
#pragma unroll
                for (int e = 0; e < kRedCount; ++e) {
                    v[e] = s_red[0][e];
#pragma unroll
                    for (int w = 1; w < kWavesPerBlock; ++w)
                        v[e] = s_red[w][e] > v[e] ? s_red[w][e] : v[e];
                }
                plan_structure<T>(cells, b, r, v, cutoff, requested, reach_target, struct_bins,
                                  struct_units);
            }
        }
        // thread 0 wrote the record's plan (or k_setup did, for an aborted
        // structure), so it reads it back in program order
        if (tid == 0) write_summary(meta + b, recs[b]);
    }
    if (fused_scan) {
        __syncthreads();
        struct_scan_block(struct_bins, struct_units, meta, nb, n_atoms, bin_off, unit_off,
                          recs, status, cap_bins, 0);
    }
}

// The batch-wide step of the planner (one workgroup, after k_plan).
__global__ __launch_bounds__(kBlock) void k_struct_scan(const long long* struct_bins,
                                                         const long long* struct_units,
                                                         const PlanSummary* meta,
                                                         int64_t nb, int64_t n_atoms,
                                                         long long* bin_off, long long* unit_off,
                                                         StructRec* recs,
                                                         unsigned long long* status,
                                                         int64_t cap_bins, int brute_hint) {
    struct_scan_block(struct_bins, struct_units, meta, nb, n_atoms, bin_off, unit_off, recs,
                      status, cap_bins, brute_hint);
}

// The set-up and plan of structure b of a request whose structures are all
// molecules (a plan hint from an earlier count of the same shape): the
// set-up of k_setup, then the molecule plan (brute force with hit masks
// needs no wraps, no bounds and no bin grid, so k_atoms, k_plan and the
// cell-list kernels have nothing to do).  A structure that is not a molecule
// under the request's algorithm raises ST_PLAN_HINT in its record, which the
// batch scan folds into the status words.
template <typename T>
__device__ __forceinline__ long long molecule_setup_one(const int64_t* bp, const T* cells,
                                                        const uint8_t* pbc, int64_t nb,
                                                        int64_t n_atoms, double cutoff, int mw,
                                                        int requested, StructRec& r,
                                                        long long* struct_bins,
                                                        long long* struct_units,
                                                        PlanSummary* meta, int64_t b) {
    setup_structure<T, true>(bp, cells, pbc, nb, n_atoms, cutoff, mw, b, r);
    // no cell-list atoms share the hit-mask rows: each atom takes its own
    r.mask0 = r.atom0;
    const int64_t n = r.natoms;
    long long units = 0;
    if (!(r.flags & kAbortBits) && n > 0) {
        if (molecule_path(r.active, n)) r.mneed = molecule_words(n);
        const bool molecule = molecule_rec(r) &&
                              (requested == TNR_BRUTE_FORCE || n <= kAutoBruteIsolated);
        if (molecule) {
            r.algo = ALGO_BRUTE;
            r.pad = 0.0;
            r.maxp = 0;
            r.maxw = 0;
            r.any_wrap = 0;
            r.cut2 = (double)(T)(cutoff * cutoff);
            r.inner2 = 0.0;  // the molecule passes decide by the public predicate
            r.outer2 = r.cut2;
            const int chunks = (int)((n + kWave - 1) / kWave);
            const int g = (int)min((int64_t)max(kMolUnitWork / chunks, 1), n);
            r.bgroup = g;
            r.bslices = 1;
            r.bwidth = 1;
            units = (n + g - 1) / g;
        } else {
            r.flags |= ST_PLAN_HINT;
        }
    }
    struct_bins[b] = 0;
    struct_units[b] = units;
    if (meta) write_summary(meta + b, r);
    return units;
}

// Molecule plan, one thread per structure (molecule_setup_one), kSetupBlock
// (one wave) per workgroup with the records built in LDS (store_records);
// block 0 first zeroes the status words and the pair scan's tile states.
// k_struct_scan follows, unless `local`: then each workgroup writes its
// structures' block-local unit offsets to local_off and its summary to
// blocks[blockIdx.x], block 0 writes the plan, and the molecule counting
// kernel finishes the offsets and the status words (MoleculeBlock).
template <typename T>
__global__ __launch_bounds__(kSetupBlock) void k_molecule_setup(
    const int64_t* bp, const T* cells, const uint8_t* pbc, int64_t nb, int64_t n_atoms,
    double cutoff, int mw, int requested, StructRec* recs, long long* struct_bins,
    long long* struct_units, PlanSummary* meta, unsigned long long* status,
    unsigned long long* tiles, int64_t n_tiles, int local, long long* local_off) {
    static_assert(kSetupBlock == kWave, "the local scan is one wave's");
    static_assert(kMolLocalMax == (int64_t)kSetupBlock * kWave, "one summary per lane");
    __shared__ StructRec s_recs[kSetupBlock];
    const int64_t b0 = (int64_t)blockIdx.x * kSetupBlock;
    const int64_t b = b0 + threadIdx.x;
    if (blockIdx.x == 0) {
        for (int k = threadIdx.x; k < SS_SLOTS; k += blockDim.x) status[k] = 0;
        for (int64_t k = threadIdx.x; k < n_tiles; k += blockDim.x) tiles[k] = 0;
        if (local && threadIdx.x == 0) status[SS_PLAN] = 1ull | kPlanMolecules;
    }
    long long units = 0;
    if (b < nb)
        units = molecule_setup_one<T>(bp, cells, pbc, nb, n_atoms, cutoff, mw, requested,
                                      s_recs[threadIdx.x], struct_bins, struct_units,
                                      local ? nullptr : meta, b);
    if (local) {
        // the workgroup's exclusive scan of units (its structures' offsets
        // within it) and its summary
        const int inc = wave_inclusive_scan_i32((int)units);
        unsigned long long fl = b < nb ? s_recs[threadIdx.x].flags : 0ull;
        long long img = b < nb ? (long long)s_recs[threadIdx.x].img_total : 0ll;
#pragma unroll
        for (int d = kWave / 2; d > 0; d >>= 1) {
            fl |= __shfl_xor(fl, d);
            img += __shfl_xor(img, d);
        }
        if (b < nb) local_off[b] = (long long)(inc - (int)units);
        if (threadIdx.x == kWave - 1) {
            MoleculeBlock mb;
            mb.units = (long long)inc;
            mb.flags = fl;
            mb.images = img;
            mb.pad = 0;
            reinterpret_cast<MoleculeBlock*>(meta)[blockIdx.x] = mb;
        }
    }
    if (b0 < nb) store_records(s_recs, recs, b0, min((int64_t)kSetupBlock, nb - b0));
}

template <typename T>
__device__ __forceinline__ int64_t local_bin(const StructRec& r, const T q[3]) {
    double u[3];
    grid_coords(r, q, u);
    int64_t k[3];
#pragma unroll
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
    // the status, the structure index and the position in one round trip;
    // the record (indexed by the structure) only once the status is clean
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t ic = i < n_atoms ? i : n_atoms - 1;
    const unsigned long long st = load_status(status + SS_FLAGS);
    const int b = atom_struct[ic];
    const Vec4<T> v = atom_q[ic];
    if ((st & kAbortBits) || i >= n_atoms) return;
    const StructRec& r = recs[b];
    const int algo = r.algo;
    const T q[3] = {v.x, v.y, v.z};
    const int64_t g = r.bin0 + local_bin(r, q);
    if (algo != ALGO_CELL) {
        atom_bin[i] = -1;
        return;
    }
    atom_bin[i] = (int)g;
    atom_rank[i] = atomicAdd(bin_count + g, 1);
}

// Single-structure request: k_plan, the planner's batch step and k_bin in
// one kernel.  Every block combines the partials of k_atoms<T, true> (the
// reductions and the atoms' error bits, all loads in flight at once) and
// plans the structure itself (thread 0, into an LDS copy of the record), so
// no block waits for another; block 0 stores the plan and writes the status
// words (all zero first: nothing has written them yet in this request).
// Then every block bins its atoms as k_bin does.
template <typename T>
__global__ __launch_bounds__(kBlock) void k_single_bin(
    const T* cells, int64_t n_atoms, double cutoff, int requested, int reach_target,
    StructRec* recs, const BlockPartial* partials, int64_t n_partials, const Vec4<T>* atom_q,
    int* atom_bin, int* atom_rank, int* bin_count, long long* struct_bins, long long* bin_off,
    long long* struct_units, long long* unit_off, int64_t cap_bins, unsigned long long* status,
    int brute_hint) {
    using K = RedKeys<T>;
    __shared__ StructRec s_rec;
    __shared__ unsigned long long s_red[kWavesPerBlock][kRedCount + 1];
    __shared__ long long s_bins, s_units;
    __shared__ int s_fast;
    const int tid = threadIdx.x, lane = lane_id(), wv = tid / kWave;
    // the record (16-byte words) and this thread's partials in one round trip
    constexpr int kRecWords = (int)(sizeof(StructRec) / sizeof(int4));
    static_assert(sizeof(StructRec) % sizeof(int4) == 0 && kRecWords <= kBlock, "record copy");
    if (tid < kRecWords)
        reinterpret_cast<int4*>(&s_rec)[tid] = reinterpret_cast<const int4*>(recs)[tid];
    const int64_t i = (int64_t)blockIdx.x * kBlock + tid;
    const Vec4<T> qv = atom_q[i < n_atoms ? i : n_atoms - 1];
    unsigned long long v[kRedCount + 1];
#pragma unroll
    for (int e = 0; e <= kRedCount; ++e) v[e] = 0;
    static_assert(kRedCount % 2 == 0 && sizeof(BlockPartial) == 8 * (kRedCount + 2),
                  "partials load as 16-byte words");
#pragma unroll 2
    for (int64_t kb = tid; kb < n_partials; kb += kBlock) {
        const ulonglong2* w = reinterpret_cast<const ulonglong2*>(partials + kb);
        ulonglong2 x[kRedCount / 2 + 1];
#pragma unroll
        for (int e = 0; e <= kRedCount / 2; ++e) x[e] = w[e];
#pragma unroll
        for (int e = 0; e < kRedCount / 2; ++e) {
            v[2 * e] = x[e].x > v[2 * e] ? x[e].x : v[2 * e];
            v[2 * e + 1] = x[e].y > v[2 * e + 1] ? x[e].y : v[2 * e + 1];
        }
        v[kRedCount] |= x[kRedCount / 2].x;
    }
#pragma unroll
    for (int e = 0; e < kRedCount; ++e) v[e] = K::wave_max(v[e]);
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1) v[kRedCount] |= __shfl_xor(v[kRedCount], d);
    if (lane == 0)
#pragma unroll
        for (int e = 0; e <= kRedCount; ++e) s_red[wv][e] = v[e];
    __syncthreads();
    if (wv == 0) {
#pragma unroll
        for (int e = 0; e <= kRedCount; ++e) v[e] = s_red[0][e];
#pragma unroll
        for (int w = 1; w < kWavesPerBlock; ++w) {
#pragma unroll
            for (int e = 0; e < kRedCount; ++e) v[e] = s_red[w][e] > v[e] ? s_red[w][e] : v[e];
            v[kRedCount] |= s_red[w][kRedCount];
        }
        StructRec& r = s_rec;
        const unsigned long long flags = r.flags | v[kRedCount];
        if (lane == 0) {
            r.flags = flags;
            s_bins = 0;
            s_units = 0;
            s_fast = 0;
            r.algo = ALGO_NONE;
        }
        if (!(flags & kAbortBits))
            plan_structure<T>(cells, 0, r, v, cutoff, requested, reach_target, &s_bins,
                              &s_units);
        if (blockIdx.x == 0) {
            // whether the next count of this shape may take the periodic fast
            // prologue (the plan bit kPlanPeriodicGrid); lane 0's writes to the
            // record above are visible to the wave
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            GridPlan gp;
            const bool fast = r.algo == ALGO_CELL &&
                              periodic_grid<T>(r, cells, cutoff, requested, reach_target, gp);
            if (lane == 0) s_fast = fast ? 1 : 0;
        }
    }
    __syncthreads();
    if (tid == 0) {
        StructRec& r = s_rec;
        r.bin0 = 0;
        r.unit0 = 0;
        if (blockIdx.x == 0) {
            recs[0] = r;
            struct_bins[0] = s_bins;
            bin_off[0] = 0;
            bin_off[1] = s_bins;
            struct_units[0] = s_units;
            unit_off[0] = 0;
            unit_off[1] = s_units;
            for (int k = 0; k < SS_SLOTS; ++k) status[k] = 0;
            const unsigned long long images = (unsigned long long)r.img_total;
            unsigned long long st = r.flags;
            if (s_bins > cap_bins) st |= ST_CAPACITY;
            if (images > (unsigned long long)kImageCap) st |= ST_BATCH_IMAGE_CAP;
            if (brute_hint && r.algo == ALGO_CELL) st |= ST_PLAN_HINT;
            status[SS_TOTAL_BINS] = (unsigned long long)s_bins;
            status[SS_TOTAL_UNITS] = (unsigned long long)s_units;
            status[SS_ANY_WRAP] = r.algo == ALGO_CELL && r.any_wrap ? 1ull : 0ull;
            status[SS_PLAN] = r.algo == ALGO_CELL
                                  ? (s_fast ? 2ull | kPlanPeriodicGrid : 2ull)
                                  : (r.algo == ALGO_BRUTE
                                         ? (molecule_rec(r) ? 1ull | kPlanMolecules
                                                                              : 1ull)
                                         : 0ull);
            status[SS_TOTAL_IMAGES] = images;
            status[SS_FLAGS] = st;
        }
    }
    __syncthreads();
    const StructRec& r = s_rec;
    if ((r.flags & kAbortBits) || s_bins > cap_bins || i >= n_atoms) return;
    if (r.algo != ALGO_CELL) {
        atom_bin[i] = -1;
        return;
    }
    const T q[3] = {qv.x, qv.y, qv.z};
    const int64_t g = local_bin(r, q);
    atom_bin[i] = (int)g;
    atom_rank[i] = atomicAdd(bin_count + g, 1);
}

// Counting sort, last step: atom i goes to binned position
// bin_start[bin] + rank (with its wraps and original position when some
// cell-list structure has wrapped atoms).
template <typename T>
__global__ __launch_bounds__(kBlock) void k_scatter(int64_t n_atoms, const Vec4<T>* atom_q,
                                                     const int* atom_bin, const int* atom_rank,
                                                     const int* bin_start, Vec4<T>* binned,
                                                     const T* pos, const int4* atom_wrap,
                                                     int4* binned_w, Vec4<T>* binned_p,
                                                     const unsigned long long* status) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_atoms) return;
    // the atom's own words load alongside the status words (in bounds for
    // every i < n_atoms); the bin is used only once the request is known good
    const int g = atom_bin[i];
    const int rank = atom_rank[i];
    const Vec4<T> q = atom_q[i];
    if (load_status(status + SS_FLAGS) & kAbortBits) return;
    const bool wrapped = load_status(status + SS_ANY_WRAP) != 0;
    if (g < 0) return;
    const int at = bin_start[g] + rank;
    binned[at] = q;
    if (wrapped) {
        // the emitting pass of a wrapped structure reads each candidate's
        // wraps and original position (with the atom index of the record) at
        // its binned position
        binned_w[at] = atom_wrap[i];
        binned_p[at] = Vec4<T>{pos[3 * i], pos[3 * i + 1], pos[3 * i + 2], q.w};
    }
}

// ------------------------------------------------ periodic fast prologue
// A request of one fully periodic structure whose previous count of the same
// shape planned it as a cell list (plan bit kPlanPeriodicGrid) bins its atoms
// without waiting for their reductions: the bin grid of a fully periodic
// structure depends on the cell, the cutoff and the margin pad only, so it is
// chosen from a margin estimate before any atom is reduced (periodic_grid)
// and every atom is binned in the first kernel.  The margins are finished
// from the atom reductions beside the placing of the atoms, where the
// stencil reach is refitted to the true margin (periodic_finish).
//   k_periodic_atoms  set-up and grid per block; per atom: wraps, wrapped
//                     position, block reductions, bin;
//   k_periodic_place  in one workgroup the finished plan and the status
//                     words; in the others the ranking atomics, a grid
//                     barrier, the bin scan and the binned atoms.
// Two launches against four for the general single-structure prologue
// (k_atoms, k_single_bin, the bin scan, k_scatter): the reductions and the
// planning do not sit between the atom pass and the atomics (every
// k_single_bin block re-reduces all partials and plans before it bins), and
// the bin scan and the scatter wait on a barrier instead of a launch.

// One whole wave: whether the memo holds the set-up of this request (every
// key word equal to the request's, the flag set and the checksum right).
template <typename T>
__device__ __forceinline__ bool memo_hit(const PeriodicMemo* m, const int64_t* bp,
                                         const T* cells, const uint8_t* pbc, int64_t n_atoms,
                                         double cutoff, int mw, int requested, int reach_target) {
    const int lane = lane_id();
    bool differs = false;
    if (lane < kMemoKey)
        differs = m->key[lane] != memo_key_word<T>(lane, bp, cells, pbc, 1, 0, n_atoms, cutoff,
                                                   mw, requested, reach_target, kMemoPeriodic);
    unsigned long long h = 0;
    for (int i = lane; i < kMemoWords; i += kWave) h ^= memo_mix(memo_word(m, i), i);
    h = wave_xor(h);
    return !__builtin_amdgcn_ballot_w64(differs) && m->fast == 1ull && h == m->check;
}

// One whole wave: stores record r (the set-up of this request, in LDS) into
// the memo with the request's key and the checksum.
template <typename T>
__device__ __forceinline__ void memo_store(PeriodicMemo* m, const StructRec& r, const int64_t* bp,
                                           const T* cells, const uint8_t* pbc, int64_t n_atoms,
                                           double cutoff, int mw, int requested,
                                           int reach_target) {
    const int lane = lane_id();
    const unsigned long long* rw = reinterpret_cast<const unsigned long long*>(&r);
    unsigned long long h = 0;
    if (lane < kMemoKey) {
        const unsigned long long k = memo_key_word<T>(lane, bp, cells, pbc, 1, 0, n_atoms, cutoff,
                                                      mw, requested, reach_target, kMemoPeriodic);
        m->key[lane] = k;
        h ^= memo_mix(k, lane);
    }
    if (lane == 0) {
        m->fast = 1ull;
        h ^= memo_mix(1ull, kMemoKey);
    }
    unsigned long long* mr = reinterpret_cast<unsigned long long*>(&m->rec);
    for (int j = lane; j < kMemoRecWords; j += kWave) {
        mr[j] = rw[j];
        h ^= memo_mix(rw[j], kMemoKey + 1 + j);
    }
    h = wave_xor(h);
    if (lane == 0) m->check = h;
}

// First kernel of the periodic fast prologue (one thread per atom).  As
// k_atoms<T, true> (every block derives the record in LDS, thread 0; per
// atom the wraps, the wrapped position and the block reductions, written as
// the block's partial with its atoms' error bits), and wave 0 of every block
// chooses the grid (periodic_grid), so each atom's bin is known here.  Block
// 0 stores the record and the status words: all zero but the bin total, or
// ST_PLAN_HINT when the fast prologue does not apply (every later kernel then
// skips its work and the caller counts again without the hint).  The grid
// also zeroes the bin counters (k_periodic_place's, kPlaceStride ints
// apart) and its barrier counters, the pair scan's tile states and the
// per-source pair counts, and each block flags whether one of its atoms is
// wrapped (place_flags).
template <typename T>
__global__ __launch_bounds__(kBlock) void k_periodic_atoms(
    const T* pos, const int64_t* bp, const T* cells, const uint8_t* pbc, double cutoff, int mw,
    int64_t n_atoms, int requested, int reach_target, StructRec* recs, BlockPartial* partials,
    int* atom_struct, int4* atom_wrap, Vec4<T>* atom_q, int* atom_bin,
    unsigned long long* status, int* bin_count, int64_t n_bin_count, unsigned long long* tiles,
    int64_t n_tiles, long long* counts, long long* struct_bins, long long* bin_off,
    long long* struct_units, long long* unit_off, unsigned long long* place, int* place_flags,
    const PeriodicMemo* memo) {
    __shared__ unsigned long long s_red[kWavesPerBlock][kRedCount];
    __shared__ unsigned long long s_atom_flags;
    __shared__ int s_fast, s_hit;
    __shared__ StructRec s_rec;
    const int tid = threadIdx.x, lane = lane_id(), wv = tid / kWave;
    {
        const int64_t stride = (int64_t)gridDim.x * kBlock;
        const int64_t k0 = (int64_t)blockIdx.x * kBlock + tid;
        if (k0 < n_atoms) counts[k0] = 0;
        if (k0 < kPlaceCounters) place[k0 * kPlaceLine] = 0;
        for (int64_t k = k0; k < n_bin_count; k += stride) bin_count[k] = 0;
        for (int64_t k = k0; k < n_tiles; k += stride) tiles[k] = 0;
    }
    const int64_t i = (int64_t)blockIdx.x * kBlock + tid;
    const int64_t ic = i < n_atoms ? i : n_atoms - 1;
    T p_pre[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) p_pre[c] = pos[3 * ic + c];
    // the set-up of an earlier request with the same inputs, when the memo
    // holds it (the record loads beside the key check)
    constexpr int kRecWords = (int)(sizeof(StructRec) / sizeof(int4));
    if (tid < kRecWords)
        reinterpret_cast<int4*>(&s_rec)[tid] = reinterpret_cast<const int4*>(&memo->rec)[tid];
    if (wv == 0) {
        const bool hit = memo_hit<T>(memo, bp, cells, pbc, n_atoms, cutoff, mw, requested,
                                     reach_target);
        if (lane == 0) {
            s_hit = hit ? 1 : 0;
            s_fast = hit ? 1 : 0;
            s_atom_flags = 0;
        }
    }
    __syncthreads();
    if (!s_hit) {
        if (tid == 0) setup_structure<T>(bp, cells, pbc, 1, n_atoms, cutoff, mw, 0, s_rec);
        __syncthreads();
        if (wv == 0) {
            GridPlan gp;
            const bool fast = periodic_grid<T>(s_rec, cells, cutoff, requested, reach_target, gp);
            if (lane == 0) {
                StructRec& r = s_rec;
                r.bin0 = 0;
                r.unit0 = 0;
                r.algo = fast ? ALGO_CELL : ALGO_NONE;
                r.nbins = fast ? gp.nbins : 0;
                if (fast) {
#pragma unroll
                    for (int a = 0; a < 3; ++a) {
                        r.nb[a] = (int32_t)gp.nb[a];
                        r.inv_w[a] = gp.inv_w[a];
                        r.lo[a] = gp.lo[a];
                        r.reach[a] = gp.reach[a];
                    }
                    r.zseg = gp.zs;
                }
                s_fast = fast ? 1 : 0;
            }
        }
        __syncthreads();
    }
    if (wv == 0) {
        if (lane == 0) {
            const StructRec& r = s_rec;
            const bool fast = s_fast != 0;
            if (blockIdx.x == 0) {
                recs[0] = r;
                const long long nbins = fast ? (long long)r.nbins : 0;
                struct_bins[0] = nbins;
                bin_off[0] = 0;
                bin_off[1] = nbins;
                struct_units[0] = 0;
                unit_off[0] = 0;
                unit_off[1] = 0;
                for (int k = 0; k < SS_SLOTS; ++k) status[k] = 0;
                status[SS_TOTAL_BINS] = (unsigned long long)nbins;
                status[SS_FLAGS] = fast ? 0ull : ST_PLAN_HINT;
            }
        }
    }
    __syncthreads();
    const bool valid = i < n_atoms;
    if (!s_fast) {
        if (valid) atom_bin[i] = -1;
        if (tid == 0) partials[blockIdx.x].flags = 0;
        return;
    }
    const StructRec& r = s_rec;
    bool good = false;
    T q[3] = {T(0), T(0), T(0)};
    int w[3] = {0, 0, 0};
    double u[3] = {0, 0, 0};
    double pabs[3] = {0, 0, 0};
    unsigned long long st = 0;
    if (valid) {
        atom_struct[i] = 0;
        bool finite = true;
#pragma unroll
        for (int c = 0; c < 3; ++c) finite = finite && isfinite((double)p_pre[c]);
        if (!finite) {
            st |= ST_POS_NONFINITE;
        } else {
            const double pd[3] = {(double)p_pre[0], (double)p_pre[1], (double)p_pre[2]};
            bool ok = true;
#pragma unroll
            for (int a = 0; a < 3; ++a) {
                const double dcol[3] = {(double)(T)r.dual[a], (double)(T)r.dual[3 + a],
                                        (double)(T)r.dual[6 + a]};
                w[a] = wrap_of(pd, dcol, &ok);
            }
            if (!ok) {
                st |= ST_WRAP_RANGE;
            } else {
#pragma unroll
                for (int c = 0; c < 3; ++c) {
                    T x = p_pre[c];
#pragma unroll
                    for (int a = 0; a < 3; ++a)
                        x = Ops<T>::sub(x, Ops<T>::mul((T)w[a], cells[3 * a + c]));
                    q[c] = x;
                }
                grid_coords(r, q, u);
#pragma unroll
                for (int c = 0; c < 3; ++c) pabs[c] = fabs(pd[c]);
                good = true;
            }
        }
        atom_wrap[i] = make_int4(w[0], w[1], w[2], 0);
        atom_q[i] = Vec4<T>{q[0], q[1], q[2], idx_as((int)i, T(0))};
        atom_bin[i] = good ? (int)local_bin(r, q) : -1;
    }
    if (st) atomicOr(&s_atom_flags, st);
    using K = RedKeys<T>;
    unsigned long long v[kRedCount];
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        v[kRedUlo + a] = good ? K::lower(u[a]) : 0ull;
        v[kRedUhi + a] = good ? K::upper(u[a]) : 0ull;
        v[kRedClo + a] = good ? K::lower_exact(q[a]) : 0ull;
        v[kRedChi + a] = good ? K::upper_exact(q[a]) : 0ull;
    }
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        v[kRedP + c] = good ? K::magnitude(pabs[c]) : 0ull;
        v[kRedW + c] = good ? (unsigned long long)abs(w[c]) : 0ull;
    }
#pragma unroll
    for (int e = 0; e < kRedCount; ++e) v[e] = K::wave_max(v[e]);
    if (lane == 0)
#pragma unroll
        for (int e = 0; e < kRedCount; ++e) s_red[wv][e] = v[e];
    __syncthreads();
    if (tid < kRedCount) {
        const int e = tid;
        unsigned long long x = s_red[0][e];
#pragma unroll
        for (int k = 1; k < kWavesPerBlock; ++k) x = s_red[k][e] > x ? s_red[k][e] : x;
        partials[blockIdx.x].red[e] = x;
    }
    if (tid == kRedCount) partials[blockIdx.x].flags = s_atom_flags;
    if (tid == kRedCount + 1) {
        unsigned long long w = 0;
#pragma unroll
        for (int k = 0; k < kWavesPerBlock; ++k)
            w |= s_red[k][kRedW] | s_red[k][kRedW + 1] | s_red[k][kRedW + 2];
        place_flags[blockIdx.x] = w != 0ull ? 1 : 0;
    }
}

// Workgroup 0 of k_periodic_place: the reductions of every k_periodic_atoms
// block, the margins (plan_margins), the reference's layout rule for an
// explicit cell_list, and the stencil reach refitted to the true margin
// (bins of the chosen grid, a padded cutoff of rc + 2 pad); a structure whose
// refitted stencil no longer fits is planned as brute force (the same pair
// set).  Then the record, the per-structure arrays and the status words.
template <typename T>
__device__ __forceinline__ void periodic_finish(const T* cells, int64_t n_atoms, double cutoff,
                                                int requested, StructRec* recs,
                                                const BlockPartial* partials, int64_t n_partials,
                                                long long* struct_bins, long long* bin_off,
                                                long long* struct_units, long long* unit_off,
                                                int64_t cap_bins, unsigned long long* status,
                                                const int64_t* bp, const uint8_t* pbc, int mw,
                                                int reach_target, PeriodicMemo* memo) {
    using K = RedKeys<T>;
    __shared__ StructRec s_rec;
    __shared__ unsigned long long s_red[kWavesPerBlock][kRedCount + 1];
    const int tid = threadIdx.x, lane = lane_id(), wv = tid / kWave;
    constexpr int kRecWords = (int)(sizeof(StructRec) / sizeof(int4));
    if (tid < kRecWords)
        reinterpret_cast<int4*>(&s_rec)[tid] = reinterpret_cast<const int4*>(recs)[tid];
    const unsigned long long st0 = load_status(status + SS_FLAGS);
    unsigned long long v[kRedCount + 1];
#pragma unroll
    for (int e = 0; e <= kRedCount; ++e) v[e] = 0;
#pragma unroll 2
    for (int64_t kb = tid; kb < n_partials; kb += kBlock) {
        const ulonglong2* wp = reinterpret_cast<const ulonglong2*>(partials + kb);
        ulonglong2 x[kRedCount / 2 + 1];
#pragma unroll
        for (int e = 0; e <= kRedCount / 2; ++e) x[e] = wp[e];
#pragma unroll
        for (int e = 0; e < kRedCount / 2; ++e) {
            v[2 * e] = x[e].x > v[2 * e] ? x[e].x : v[2 * e];
            v[2 * e + 1] = x[e].y > v[2 * e + 1] ? x[e].y : v[2 * e + 1];
        }
        v[kRedCount] |= x[kRedCount / 2].x;
    }
    if (st0 & kAbortBits) return;  // the hint did not hold (block-uniform)
#pragma unroll
    for (int e = 0; e < kRedCount; ++e) v[e] = K::wave_max(v[e]);
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1) v[kRedCount] |= __shfl_xor(v[kRedCount], d);
    if (lane == 0)
#pragma unroll
        for (int e = 0; e <= kRedCount; ++e) s_red[wv][e] = v[e];
    __syncthreads();
    if (wv != 0) return;
    // the record as k_periodic_atoms derived it, for the next request with
    // the same inputs (read here before this wave changes it)
    memo_store<T>(memo, s_rec, bp, cells, pbc, n_atoms, cutoff, mw,
                  requested, reach_target);
#pragma unroll
    for (int e = 0; e <= kRedCount; ++e) v[e] = s_red[0][e];
#pragma unroll
    for (int w = 1; w < kWavesPerBlock; ++w) {
#pragma unroll
        for (int e = 0; e < kRedCount; ++e) v[e] = s_red[w][e] > v[e] ? s_red[w][e] : v[e];
        v[kRedCount] |= s_red[w][kRedCount];
    }
    StructRec& r = s_rec;
    const int64_t n = r.natoms;
    unsigned long long st = r.flags | v[kRedCount];
    int algo = ALGO_CELL;
    long long nbins = r.nbins, units = 0;
    if (!(st & kAbortBits)) {
        double cell[9];
#pragma unroll
        for (int e = 0; e < 9; ++e) cell[e] = (double)cells[e];
        const double rc = cutoff;
        const Margins m = plan_margins<T>(cell, r, red_pmax<T>(v), red_wmax(v), rc);
        if (requested == TNR_CELL_LIST && cell_unsafe<T>(v, r, cell, cutoff, n))
            st |= ST_CELL_UNSAFE;
        // the reach that bins of the chosen grid need for the true margin
        bool fits = m.safe;
        int reach[3];
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            const double gn = sqrt(r.grid[3 * a] * r.grid[3 * a] + r.grid[3 * a + 1] * r.grid[3 * a + 1] +
                                   r.grid[3 * a + 2] * r.grid[3 * a + 2]);
            const double rcu = (rc + 2 * m.pad) * gn;
            const double rd = floor(rcu * (double)r.nb[a] * (1.0 + 1e-12)) + 1.0;
            fits = fits && rd < 256.0;
            reach[a] = rd < 256.0 ? (int)rd : 1;
        }
        const int zs = stencil_zseg(true, reach[2], r.nb[2]);
        const int rows = (2 * reach[0] + 1) * (2 * reach[1] + 1);
        fits = fits && (long long)rows * zs <= kPieceCap &&
               (double)n * (double)(rows * zs) < 2147483647.0;
        if (lane == 0) {
            write_margins<T>(r, m, cutoff);
            if (fits) {
#pragma unroll
                for (int a = 0; a < 3; ++a) r.reach[a] = reach[a];
                r.zseg = zs;
            } else {
                algo = ALGO_BRUTE;
                nbins = 0;
                r.nbins = 0;
                units = plan_brute_units(r, n);
            }
        }
    }
    if (lane != 0) return;
    r.algo = (st & kAbortBits) ? ALGO_NONE : algo;
    r.flags = st;
    recs[0] = r;
    struct_bins[0] = nbins;
    bin_off[1] = nbins;
    struct_units[0] = units;
    unit_off[1] = units;
    const unsigned long long images = (unsigned long long)r.img_total;
    if (nbins > cap_bins) st |= ST_CAPACITY;
    if (images > (unsigned long long)kImageCap) st |= ST_BATCH_IMAGE_CAP;
    // the bin total stays the grid's (the bin scan beside this workgroup
    // reads it); a structure planned as brute force has no cell-list work
    status[SS_TOTAL_UNITS] = (unsigned long long)units;
    status[SS_ANY_WRAP] = algo == ALGO_CELL && r.any_wrap ? 1ull : 0ull;
    status[SS_PLAN] = algo == ALGO_CELL ? 2ull | kPlanPeriodicGrid : 1ull;
    status[SS_TOTAL_IMAGES] = images;
    if (st) atomicOr(status + SS_FLAGS, st);
}

// Grid barrier of k_periodic_place, for its nblk workgroups blk = 0 ..
// nblk - 1 (all resident at once): every wave first waits for its own
// memory operations (its atomics have been performed, its stores written),
// then thread 0 adds the workgroup to its group's counter (blk % 8), the
// group's last arrival adds the group to the groups' counter, and thread 0
// waits for that counter to reach round x groups (the counters only grow:
// round is the barrier's number, from 1).  Everything that crosses
// workgroups inside the kernel is read with device-scope atomic loads
// (place_load), so no fence writes back or invalidates the XCD's L2 (an
// agent-scope fence does both, and one per wave on each side cost tens of
// microseconds on C4).  The wait is bounded by `ticks` of the constant-rate
// clock (s_memrealtime); false when it expired.
__device__ __forceinline__ bool place_barrier(unsigned long long* ctr, unsigned nblk, unsigned blk,
                                              unsigned round, long long ticks) {
    __shared__ int s_ok;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned x = blk & 7u;
        const unsigned long long members = (nblk - x + 7u) / 8u;
        const unsigned long long groups = nblk < 8u ? nblk : 8u;
        const unsigned long long old = atomicAdd(ctr + x * kPlaceLine, 1ull);
        if (old + 1ull == round * members) atomicAdd(ctr + 8 * kPlaceLine, 1ull);
        const unsigned long long want = round * groups;
        const long long t0 = (long long)wall_clock64();
        int ok = 1;
        while (__hip_atomic_load(ctr + 8 * kPlaceLine, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT) < want) {
            if ((long long)wall_clock64() - t0 > ticks) {
                ok = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        s_ok = ok;
    }
    __syncthreads();
    return s_ok != 0;
}

template <typename V>
__device__ __forceinline__ V place_load(const V* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename V>
__device__ __forceinline__ void place_store(V* p, V v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Atom i (record q) to binned position `at`, with its wraps and original
// position when some atom of the request is wrapped.
template <typename T>
__device__ __forceinline__ void place_atom(int64_t i, int at, Vec4<T> q, bool wrapped,
                                           const T* pos, const int4* atom_wrap, Vec4<T>* binned,
                                           int4* binned_w, Vec4<T>* binned_p) {
    binned[at] = q;
    if (wrapped) {
        binned_w[at] = atom_wrap[i];
        binned_p[at] = Vec4<T>{pos[3 * i], pos[3 * i + 1], pos[3 * i + 2], q.w};
    }
}

// Second and last kernel of the periodic fast prologue: ranks, bin starts
// and the binned atoms in one launch.  Workgroup 0 finishes the plan
// (periodic_finish: it leaves the bin total alone), workgroups 1 .. 7 leave
// at once, and workgroups 8 + blk, blk = 0 .. G - 1 (G no more than the
// device holds at once beside them), take the atoms i = (blk + k G) 256 +
// thread: for k = 0 the atoms k_periodic_atoms block blk wrote, on the
// same XCD (workgroup b runs on XCD b % 8), so their records are read from
// that XCD's L2 (read from another XCD's writes, the loads took a median
// 8 us on C4 against under 1 us):
//   1. one returning atomic per binned atom on its bin's counter (its rank
//      in the bin), and whether any atom is wrapped (the flags of the
//      k_periodic_atoms workgroups);
//   2. grid barrier; up to kPlaceScanMax bins every workgroup scans the bin
//      counts whole into LDS and writes its share of bin_start; beyond,
//      each workgroup sums a slice of the bins, and after a second barrier
//      scans its slice behind the sums of the slices before it (bin_start
//      from memory after a third);
//   3. each atom to binned[bin start + rank] (with its wraps and original
//      position when some atom is wrapped).
// A wait that expires (`ticks`; the workgroups could not all be resident)
// raises ST_PLAN_HINT, so the caller counts again without the hint, and the
// workgroup leaves: every wave exits.
template <typename T>
__global__ __launch_bounds__(kBlock) void k_periodic_place(
    const T* cells, int64_t n_atoms, double cutoff, int requested, StructRec* recs,
    const BlockPartial* partials, int64_t n_partials, long long* struct_bins, long long* bin_off,
    long long* struct_units, long long* unit_off, int64_t cap_bins, unsigned long long* status,
    const int* atom_bin, int* atom_rank, int* place_cnt, int* bin_start, const Vec4<T>* atom_q,
    Vec4<T>* binned, const T* pos, const int4* atom_wrap, int4* binned_w, Vec4<T>* binned_p,
    unsigned long long* place, const int* place_flags, long long ticks, const int64_t* bp,
    const uint8_t* pbc, int mw, int reach_target, PeriodicMemo* memo) {
    if (blockIdx.x < kPlaceFirst) {
        if (blockIdx.x == 0)
            periodic_finish<T>(cells, n_atoms, cutoff, requested, recs, partials, n_partials,
                               struct_bins, bin_off, struct_units, unit_off, cap_bins, status,
                               bp, pbc, mw, reach_target, memo);
        return;
    }
    // bin starts of the whole scan, entry k at k + k / 32 (each thread's 32
    // consecutive bins fall in 32 different banks)
    __shared__ int s_start[kPlaceScanMax + kPlaceScanMax / 32 + 1];
    const int tid = threadIdx.x;
    const unsigned G = gridDim.x - kPlaceFirst, blk = blockIdx.x - kPlaceFirst;
    // ST_PLAN_HINT here comes from k_periodic_atoms (the same for every
    // workgroup) or from an expired wait; the finishing workgroup's error
    // bits are left to the later kernels
    if (load_status(status + SS_FLAGS) & ST_PLAN_HINT) return;
    const int64_t stride = (int64_t)G * kBlock;
    const int64_t i0 = (int64_t)blk * kBlock + tid;
    int g0 = -1, r0 = 0;
    Vec4<T> q0{T(0), T(0), T(0), T(0)};
    if (i0 < n_atoms) {
        g0 = atom_bin[i0];
        q0 = atom_q[i0];
    }
    if (g0 >= 0) r0 = atomicAdd(place_cnt + (int64_t)g0 * kPlaceStride, 1);
    for (int64_t i = i0 + stride; i < n_atoms; i += stride) {
        const int g = atom_bin[i];
        if (g >= 0) atom_rank[i] = atomicAdd(place_cnt + (int64_t)g * kPlaceStride, 1);
    }
    int wf = 0;
    for (int64_t k = tid; k < n_partials; k += kBlock) wf |= place_flags[k];
    const bool wrapped = __syncthreads_or(wf) != 0;
    unsigned long long* ctr = place;
    if (!place_barrier(ctr, G, blk, 1u, ticks)) {
        if (tid == 0) atomicOr(status + SS_FLAGS, ST_PLAN_HINT);
        return;
    }
    const int64_t nbins = (int64_t)load_status(status + SS_TOTAL_BINS);
    const bool whole = nbins <= kPlaceScanMax;
    auto lds = [](int64_t k) { return (int)(k + (k >> 5)); };
    if (whole) {
        // the counts into LDS, 256 consecutive bins per load (all loads
        // issued before the first is stored); then each thread scans 32
        // consecutive bins
        constexpr int kPer = (int)(kPlaceScanMax / kBlock);
        int c[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int64_t g = (int64_t)k * kBlock + tid;
            c[k] = g < nbins ? place_load(place_cnt + g * kPlaceStride) : 0;
        }
#pragma unroll
        for (int k = 0; k < kPer; ++k) s_start[lds((int64_t)k * kBlock + tid)] = c[k];
        __syncthreads();
        const int64_t base = (int64_t)tid * kPer;
        long long sum = 0;
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            c[k] = s_start[lds(base + k)];
            sum += c[k];
        }
        long long total;
        long long run = block_exclusive_scan(sum, &total);
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            s_start[lds(base + k)] = (int)run;
            run += c[k];
        }
        if (tid == 0) s_start[lds(nbins)] = (int)total;
        __syncthreads();
        for (int64_t k = (int64_t)blk * kBlock + tid; k <= nbins; k += stride)
            bin_start[k] = s_start[lds(k)];
    } else {
        long long* slice = reinterpret_cast<long long*>(place + kPlaceCounters * kPlaceLine);
        const int64_t S = (nbins + G - 1) / G;
        const int64_t b0 = min((int64_t)blk * S, nbins), b1 = min(nbins, b0 + S);
        long long sum = 0, total;
        for (int64_t k = b0 + tid; k < b1; k += kBlock) sum += place_load(place_cnt + k * kPlaceStride);
        (void)block_exclusive_scan(sum, &total);
        if (tid == 0) place_store(slice + blk, total);
        if (!place_barrier(ctr, G, blk, 2u, ticks)) {
            if (tid == 0) atomicOr(status + SS_FLAGS, ST_PLAN_HINT);
            return;
        }
        long long before = 0;
        for (int64_t k = tid; k < (int64_t)blk; k += kBlock) before += place_load(slice + k);
        (void)block_exclusive_scan(before, &total);
        long long run = total;
        for (int64_t k0 = b0; k0 < b1; k0 += kBlock) {
            const int64_t k = k0 + tid;
            const long long x = k < b1 ? place_load(place_cnt + k * kPlaceStride) : 0;
            const long long ex = block_exclusive_scan(x, &total);
            if (k < b1) place_store(bin_start + k, (int)(run + ex));
            run += total;
        }
        if (blk == G - 1 && tid == 0) place_store(bin_start + nbins, (int)run);
        if (!place_barrier(ctr, G, blk, 3u, ticks)) {
            if (tid == 0) atomicOr(status + SS_FLAGS, ST_PLAN_HINT);
            return;
        }
    }
    // the records stay in registers (place_atom takes them by value): an
    // atom record whose address was taken (a by-reference lambda, or a
    // select between it and a load) was kept in LDS at a 12-byte stride,
    // whose misaligned 8-byte writes held the loads up by about 7 us per
    // workgroup on C4, or in scratch memory
    if (g0 >= 0)
        place_atom<T>(i0, (whole ? s_start[lds(g0)] : place_load(bin_start + g0)) + r0, q0,
                      wrapped, pos, atom_wrap, binned, binned_w, binned_p);
    for (int64_t i = i0 + stride; i < n_atoms; i += stride) {
        const int g = atom_bin[i];
        if (g < 0) continue;
        place_atom<T>(i, (whole ? s_start[lds(g)] : place_load(bin_start + g)) + atom_rank[i],
                      atom_q[i], wrapped, pos, atom_wrap, binned, binned_w, binned_p);
    }
}

}  // namespace tnr
