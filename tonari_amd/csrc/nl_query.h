// Query arguments, pair output, the pair identity policy and the
// brute-force image walk (k_brute / brute_source) in a counting and an
// emitting flavour.  The cell-list walk is in nl_cell.h.
//
// Both apply the reference's pair identity policy and public predicate
// (neighbors_cpu.cpp:222-273): a fused broad-phase distance classifies a
// candidate as inside (d2 < inner2), outside (d2 >= outer2) or in the thin
// band between, which the public predicate decides.  The margin between the
// thresholds covers the rounding difference of the two formulas.
#pragma once

#include "nl_math.h"

namespace tnr {

template <typename T>
struct QueryArgs {
    const T* pos;
    const T* cells;
    const StructRec* recs;
    const int64_t* struct_bin_off;    // B + 1: first cell-list bin of each structure
    const int* atom_struct;
    const int4* atom_wrap;
    const Vec4<T>* atom_q;
    const int* bin_start;
    const Vec4<T>* binned;
    long long* counts;
    const long long* offsets;
    unsigned long long* status;
    unsigned long long* masks;      // kMaskWords hit masks per binned cell-list source
    int64_t n_atoms;
    int64_t nb;
    // without `sorted`: when every structure is searched with a cell list
    // (status plan 2), pair counts and output offsets are indexed by binned
    // position, so sources take the outputs in binned order and every
    // emitting workgroup writes one contiguous range; otherwise by atom index
    int by_bin;
    int64_t limit;  // E: emit never writes at or beyond it
    int64_t n_bins; // emit: cell-list bins covered by the grid (at least the batch's)
    // outputs (emit)
    int64_t* pairs;
    int32_t* shifts;
    T* dist;
    T* vec;
    int64_t* src;
    int64_t* dst;
};

// Value of x held by the first active lane, as a wave-uniform (scalar) value.
__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

template <typename T>
struct Triple {
    T x, y, z;
};

// Writes pair o.  Only the emitting passes call this, after the counting
// pass has proved that every output shift fits in int32.
template <typename T>
__device__ __forceinline__ void write_hit(const QueryArgs<T>& a, long long o, int s, int t,
                                          int S0, int S1, int S2, const T ps[3], const T pt[3],
                                          const T* cell, bool diagonal) {
    if (o < 0 || o >= a.limit) {
        atomicOr(a.status + SS_FLAGS, ST_OUTPUT_RANGE);
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
        Triple<int32_t> v;
        v.x = S0;
        v.y = S1;
        v.z = S2;
        *reinterpret_cast<Triple<int32_t>*>(a.shifts + 3 * o) = v;
    }
    if (a.vec || a.dist) {
        T D[3];
        const T d2 = diagonal ? public_vector_diag(ps, pt, S0, S1, S2, cell, D)
                              : public_vector(ps, pt, S0, S1, S2, cell, D);
        if (a.vec) {
            Triple<T> v;
            v.x = D[0];
            v.y = D[1];
            v.z = D[2];
            *reinterpret_cast<Triple<T>*>(a.vec + 3 * o) = v;
        }
        if (a.dist) a.dist[o] = Ops<T>::sqrt_(d2);
    }
}

// Output shift S = k - wrap_t + wrap_s in int32 (wrapping arithmetic; exact
// whenever the counting pass raised no shift-range error).
__device__ __forceinline__ int shift_i32(int k, int wt, int ws) {
    return (int)((unsigned)k - (unsigned)wt + (unsigned)ws);
}

// Identity filter of pair_policy.h:42-79 for a candidate whose output shift
// equals the image shift k when s == t.
template <int MODE>
__device__ __forceinline__ bool identity_ok(int s, int t, bool kzero, bool kneg) {
    if (s == t && kzero) return (MODE & 1) != 0;
    if constexpr ((MODE & 2) != 0) return s < t || (s == t && kneg);
    return true;
}

// The same filter as one unsigned comparison against a per-candidate key:
//   MODE 0 (full list):             key = k == 0 ? t : ~0u,   keep iff key != s
//   MODE 1 (full list, self pairs): keep every candidate
//   MODE 2 (half list):             key = 2t + [k < 0],       keep iff key > 2s
//   MODE 3 (half list, self pairs): key = 2t + [k <= 0],      keep iff key > 2s
// where k < 0 is lexicographic order of (kx, ky, kz).  For the half list,
// t > s gives key >= 2s + 2, t < s gives key <= 2s - 1, and t == s keeps the
// candidate exactly when the flag is set.  Indices are below 2^31, so 2t + 1
// fits in 32 bits.
template <int MODE>
__device__ __forceinline__ unsigned identity_key(int t, bool kzero, bool kneg) {
    if constexpr (MODE == 0) return kzero ? (unsigned)t : ~0u;
    if constexpr (MODE == 2) return 2u * (unsigned)t + (kneg ? 1u : 0u);
    if constexpr (MODE == 3) return 2u * (unsigned)t + ((kneg || kzero) ? 1u : 0u);
    return 0u;
}
template <int MODE>
__device__ __forceinline__ bool identity_pass(unsigned key, int s) {
    if constexpr (MODE == 0) return key != (unsigned)s;
    if constexpr ((MODE & 2) != 0) return key > 2u * (unsigned)s;
    return true;
}

// -------------------------------------------------------------------- brute

// One source atom s of brute-force structure b, walked by one wave.  Lanes
// hold 64 targets; the wave walks the image box of the structure in the
// reference order (x-major, z fastest).  Counting writes counts[s]; emitting
// writes the pairs of s from offsets[s] on.
template <typename T, int MODE, bool EMIT>
__device__ __forceinline__ void brute_source(const QueryArgs<T>& a, int s, int b,
                                             const StructRec& r) {
    using O = Ops<T>;
    const int lane = lane_id();
    {
        const int a0 = (int)r.atom0;
        const int a1 = (int)(r.atom0 + r.natoms);
        const int R0 = r.reps[0], R1 = r.reps[1], R2 = r.reps[2];
        const T* cell = a.cells + 9 * b;
        T c[9];
#pragma unroll
        for (int e = 0; e < 9; ++e) c[e] = cell[e];
        const T inner2 = (T)r.inner2, outer2 = (T)r.outer2, cut2 = (T)r.cut2;
        const bool any_wrap = r.any_wrap != 0;
        const bool diagonal = r.diagonal != 0;
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
                        const bool kzero = i0 == 0 && i1 == 0 && i2 == 0;
                        const bool zs = t == s && kzero;
                        bool ok = vt && (d2 < outer2 || zs) &&
                                  identity_ok<MODE>(s, t, kzero, lex_negative(i0, i1, i2));
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
                                write_hit(a, cursor + lanes_below(m), s, t, (int)S0, (int)S1,
                                          (int)S2, ps, pt, c, diagonal);
                            cursor += __popcll(m);
                        }
                    }
                }
            }
        }
        if (!EMIT && lane == 0) a.counts[s] = total;
    }
}

// One wave per source atom of the brute-force structures (grid-stride).
template <typename T, int MODE, bool EMIT>
__global__ __launch_bounds__(kBlock) void k_brute(QueryArgs<T> a) {
    if ((load_status(a.status + SS_FLAGS) & kAbortBits) ||
        !(load_status(a.status + SS_PLAN) & 1))
        return;
    const int64_t wave0 = (int64_t)blockIdx.x * kWavesPerBlock + uniform(threadIdx.x / kWave);
    const int64_t nwaves = (int64_t)gridDim.x * kWavesPerBlock;
    for (int64_t s64 = wave0; s64 < a.n_atoms; s64 += nwaves) {
        const int s = (int)s64;
        const int b = a.atom_struct[s];
        const StructRec& r = a.recs[b];
        if (r.algo != ALGO_BRUTE) continue;
        brute_source<T, MODE, EMIT>(a, s, b, r);
    }
}

}  // namespace tnr
