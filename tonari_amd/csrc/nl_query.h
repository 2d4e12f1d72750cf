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
    const int64_t* struct_unit_off;   // B + 1: first brute-force work unit of each structure
    const int* atom_struct;
    const int4* atom_wrap;
    const Vec4<T>* atom_q;
    const int* bin_start;
    const Vec4<T>* binned;
    const int4* binned_w;       // wraps in binned order (status SS_ANY_WRAP)
    const Vec4<T>* binned_p;    // original positions (and the records' atom index) in binned order
    long long* counts;
    const long long* offsets;
    unsigned long long* status;
    unsigned long long* masks;      // mask_words hit masks per atom slot
    int64_t n_atoms;
    int64_t nb;
    int mask_words;  // words of an atom's hit-mask row (1 to kMaskWords)
    // count of a molecules-only request planned without the batch scan
    // (k_molecule_setup with `local`): struct_bin_off holds block-local unit
    // offsets and mol_blocks the workgroups' summaries; the counting kernel
    // makes the offsets global for the emitting pass
    int mol_local;
    const MoleculeBlock* mol_blocks;
    // without `sorted`: when every structure is searched with a cell list
    // (status plan 2), pair counts and output offsets are indexed by binned
    // position, so sources take the outputs in binned order and every
    // emitting workgroup writes one contiguous range; otherwise by atom index
    int by_bin;
    // count: the cell-list counting kernel also counts the brute-force
    // structures (an explicit cell_list request, whose count launches no
    // brute-force kernel; the planner gives such a request brute-force
    // structures only where no bin grid fits)
    int brute_in_cell;
    int64_t limit;  // E: emit never writes at or beyond it
    int64_t n_bins; // emit: cell-list bins covered by the grid (at least the batch's)
    // outputs (emit)
    int64_t* pairs;
    int32_t* shifts;
    T* dist;
    T* vec;
    int64_t* src;
    int64_t* dst;
    int64_t* edge;  // edge-first i/j (tnr_outputs::edge_index); place_edge_index sets src, dst
};

// Edge-first outputs: sources at edge[0, E), targets at edge[E, 2E), with E
// from the count's status words, so an emit launched before the host read E
// writes the layout too.  When E exceeds the output length the targets are
// not written (the sources' rows stay below the length); the caller sees E
// and emits again into a larger buffer.
template <typename T>
__device__ __forceinline__ void place_edge_index(QueryArgs<T>& a) {
    if (!a.edge) return;
    const long long E = (long long)load_status(a.status + SS_PAIRS);
    a.src = a.edge;
    a.dst = E <= a.limit ? a.edge + E : nullptr;
}

// Value of x held by the first active lane, as a wave-uniform (scalar) value.
__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// A counting wave's longest wanted hit-mask row (wave-uniform) into the
// status word SS_MASK_NEED, by one atomic maximum from the waves that raise it.
__device__ __forceinline__ void report_mask_need(unsigned long long* status, int need) {
    if (need <= 0 || lane_id() != 0) return;
    unsigned long long* slot = status + SS_MASK_NEED;
    if ((unsigned long long)need >
        __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
        atomicMax(slot, (unsigned long long)need);
}

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

// Structure of the last item (cell-list bin or brute-force unit) looked up
// by this workgroup: items [lo, hi) belong to structure b.  Consecutive items
// usually share a structure.
struct StructCache {
    int b;
    int64_t lo, hi;
};

// Structure of unit u: the largest b with off[b] <= u, found by the whole
// wave (every lane with the same u), 64 candidates per step (one load per
// lane): one round trip for up to 64 structures, two up to 4,096.
__device__ __forceinline__ int unit_structure(const int64_t* off, int64_t nb, int64_t u) {
    const int lane = lane_id();
    int64_t lo = 0, len = nb;
    while (len > 1) {
        const int64_t step = (len + kWave - 1) / kWave;
        const int64_t at = (int64_t)lane * step;
        const bool le = at < len && off[lo + at] <= u;
        const unsigned long long m = ballot(le) | 1ull;
        const int64_t last = 63 - __builtin_clzll(m);
        lo += last * step;
        len = min(step, len - last * step);
    }
    return (int)lo;
}

// Structure of item g (the whole wave calls it with the same g): the wave
// search of unit_structure, unless g lies in the item range cached in sc
// by the previous call (callers that walk consecutive items).
__device__ __forceinline__ int structure_of_item(const int64_t* off, int64_t nb, int64_t g,
                                                 StructCache& sc) {
    if (nb == 1) return 0;  // every item belongs to the only structure
    if (g >= sc.lo && g < sc.hi) return sc.b;
    sc.b = uniform(unit_structure(off, nb, g));
    sc.lo = off[sc.b];
    sc.hi = off[sc.b + 1];
    return sc.b;
}

// -------------------------------------------------------------------- brute
//
// Brute-force structures (neighbors_cuda.cu:89-279,443-556 and the brute path
// of neighbors_cpu.cpp): every (source, target) pair of a structure with every
// periodic image k of the box |k_a| <= R_a.  Here each lane takes one
// (source, k0, target) triple; the wave walks the rows k1 of the box, and
// each lane visits only the k2 of a row whose translate can lie within the
// padded cutoff (pair_images): a superset of the images the public predicate
// can keep, widened far beyond its rounding and clipped to the reference's
// box.  Every visited image is then decided as everywhere else: fused broad
// phase, identity, and the public predicate in the band.  A wave takes one
// work unit: bgroup consecutive sources of one structure and one slice of
// bwidth consecutive k0 values (the planner sizes units to similar work and
// slices k0 only where one source's planes exceed a unit).

// The integers k in [-R, R] within c - h .. c + h, each end widened by 1/256
// plus 2^-16 of the magnitudes (the rounding of the float evaluations that
// produce c and h is far smaller).  A NaN end keeps the box's end.
template <typename T>
__device__ __forceinline__ void axis_range(T c, T h, int R, int& lo, int& hi) {
    const T slack = (T)(1.0 / 256.0) + (fabs(c) + h) * (T)(1.0 / 65536.0);
    const T fr = (T)R;
    lo = (int)fmin(fmax(ceil(c - h - slack), -fr), fr + (T)1);
    hi = (int)fmax(fmin(floor(c + h + slack), fr), -fr - (T)1);
}

// The integers k in [-R, R] for which |p + k v|^2 < rho2 may hold: the
// closest approach of the line p + x v lies at x = c = -(p.v)/|v|^2, at
// distance |q| with q = p + c v, and |p + x v|^2 = |q|^2 + (x - c)^2 |v|^2.
// rho2 is widened by 2^-20 |p|^2, which covers the cancellation in |q|.  The
// half-width comes from the hardware square root in float (within an ulp;
// axis_range widens each end by far more).
__device__ __forceinline__ float range_sqrt(float x) { return __builtin_amdgcn_sqrtf(x); }
__device__ __forceinline__ double range_sqrt(double x) { return sqrt(x); }
template <typename T>
__device__ __forceinline__ void line_range(T px, T py, T pz, T vx, T vy, T vz, T inv_vv, T rho2,
                                           int R, int& lo, int& hi) {
    const T c = -(px * vx + py * vy + pz * vz) * inv_vv;
    const T qx = px + c * vx, qy = py + c * vy, qz = pz + c * vz;
    const T pp = px * px + py * py + pz * pz;
    const T h2 = (rho2 + pp * (T)(1.0 / 1048576.0) - (qx * qx + qy * qy + qz * qz)) * inv_vv;
    if (h2 < (T)0) {
        lo = 1;
        hi = 0;
        return;
    }
    axis_range(c, range_sqrt(h2), R, lo, hi);
}

// Wave-uniform geometry of a brute-force structure.
template <typename T>
struct BruteGeom {
    T c[9];  // cell rows
    T inv2;  // 1/|c2|^2
    T rho2, inner2, outer2, cut2;
    int R0, R1, R2;
    bool any_wrap, diagonal;
};

// The search radius rho2 is outer2 widened by 2^-8, so every image with a
// broad-phase distance below outer2 is visited.
template <typename T>
__device__ __forceinline__ void brute_geom(const QueryArgs<T>& a, const StructRec& r, int b,
                                           BruteGeom<T>& g) {
    const T* cell = a.cells + 9 * b;
#pragma unroll
    for (int e = 0; e < 9; ++e) g.c[e] = cell[e];
    g.R0 = r.reps[0];
    g.R1 = r.reps[1];
    g.R2 = r.reps[2];
    g.inner2 = (T)r.inner2;
    g.outer2 = (T)r.outer2;
    g.cut2 = (T)r.cut2;
    g.any_wrap = r.any_wrap != 0;
    g.diagonal = r.diagonal != 0;
    g.rho2 = g.outer2 * (T)(1.0 + 1.0 / 256.0);
    g.inv2 = g.R2 > 0 ? (T)1 / (g.c[6] * g.c[6] + g.c[7] * g.c[7] + g.c[8] * g.c[8]) : T(0);
}

// Decision for image (k0, k1, k2) of the pair (s, t), whose broad-phase
// displacement before the k2 term is (ex, ey, ez): broad phase, identity,
// and the public predicate in the band.  dw = wrap_s - wrap_t in double
// (exact), so the output shift k + dw is exact in double and rounds to T as
// the integer itself would.
template <typename T, int MODE>
__device__ __forceinline__ bool image_decide(const BruteGeom<T>& g, int k0, int k1, int k2, T ex,
                                             T ey, T ez, int s, int t, const double dw[3],
                                             const T ps[3], const T pt[3]) {
    using O = Ops<T>;
    const T f2 = (T)k2;
    const T dx = O::fma_(f2, g.c[6], ex);
    const T dy = O::fma_(f2, g.c[7], ey);
    const T dz = O::fma_(f2, g.c[8], ez);
    const T d2 = O::fma_(dz, dz, O::fma_(dy, dy, O::mul(dx, dx)));
    const bool kzero = k0 == 0 && k1 == 0 && k2 == 0;
    const bool zs = t == s && kzero;
    if (!((d2 < g.outer2 || zs) && identity_ok<MODE>(s, t, kzero, lex_negative(k0, k1, k2))))
        return false;
    if (zs || d2 < g.inner2) return true;
    const T S0 = (T)((double)k0 + dw[0]), S1 = (T)((double)k1 + dw[1]),
            S2 = (T)((double)k2 + dw[2]);
    T D[3];
    return public_vector(ps, pt, S0, S1, S2, g.c, D) < g.cut2;
}

// An atom's data for pair_images: wrapped position, wraps, position.
template <typename T>
struct WalkAtom {
    Vec4<T> q;
    int4 w;
    T p[3];
};

template <typename T>
__device__ __forceinline__ WalkAtom<T> walk_atom(const QueryArgs<T>& a, int i) {
    WalkAtom<T> x;
    x.q = a.atom_q[i];
    x.w = a.atom_wrap[i];
#pragma unroll
    for (int e = 0; e < 3; ++e) x.p[e] = a.pos[3 * i + e];
    return x;
}

// The images of the lane's (source, target) pair in the lane's plane k0, row
// by row: the rows k1 of the box are walked by the whole wave, and each lane
// restricts k2 to the integers where |e + k2 c2| can fall below the search
// radius (line_range; k2 = 0 when axis 2 is not periodic), so only the
// images near the cutoff sphere are decided.
//   PASS 0 (count): returns the kept pairs, raising the int32 shift-range
//                   error where a kept shift does not fit.
//   PASS 1 (write): writes the kept pairs.  Every lane runs every step of a
//                   row (as long as the row's longest range); the hits of a
//                   step are placed by ballot after the earlier hits of the
//                   same source: `seg` marks the lanes of the lane's source,
//                   and `cursor` (equal on those lanes) is the source's next
//                   output position, advanced here.
template <typename T, int MODE, int PASS>
__device__ __forceinline__ int pair_images(const QueryArgs<T>& a, const BruteGeom<T>& g, bool valid,
                                           int s, int t, int k0, const WalkAtom<T>& xs,
                                           const WalkAtom<T>& xt, unsigned long long seg,
                                           long long& cursor) {
    using O = Ops<T>;
    const T bx = O::sub(xt.q.x, xs.q.x), by = O::sub(xt.q.y, xs.q.y), bz = O::sub(xt.q.z, xs.q.z);
    const double dw[3] = {(double)xs.w.x - (double)xt.w.x, (double)xs.w.y - (double)xt.w.y,
                          (double)xs.w.z - (double)xt.w.z};
    const unsigned long long below = (1ull << lane_id()) - 1ull;
    int hits = 0;
    {
        const T f0 = (T)k0;
        const T e0x = O::fma_(f0, g.c[0], bx), e0y = O::fma_(f0, g.c[1], by),
                e0z = O::fma_(f0, g.c[2], bz);
        for (int k1 = -g.R1; k1 <= g.R1; ++k1) {
            const T f1 = (T)k1;
            const T ex = O::fma_(f1, g.c[3], e0x), ey = O::fma_(f1, g.c[4], e0y),
                    ez = O::fma_(f1, g.c[5], e0z);
            int lo2 = 0, hi2 = 0;
            if (g.R2 > 0)
                line_range(ex, ey, ez, g.c[6], g.c[7], g.c[8], g.inv2, g.rho2, g.R2, lo2, hi2);
            if (!valid) hi2 = lo2 - 1;
            if (PASS == 0) {
                for (int k2 = lo2; k2 <= hi2; ++k2) {
                    if (image_decide<T, MODE>(g, k0, k1, k2, ex, ey, ez, s, t, dw, xs.p, xt.p)) {
                        ++hits;
                        if (g.any_wrap && !(fits_i32d((double)k0 + dw[0]) &&
                                            fits_i32d((double)k1 + dw[1]) &&
                                            fits_i32d((double)k2 + dw[2])))
                            atomicOr(a.status + SS_FLAGS, ST_SHIFT_RANGE);
                    }
                }
            } else {
                const int len = max(hi2 - lo2 + 1, 0);
                const int steps = read_lane(wave_inclusive_max_i32(len), kWave - 1);
                for (int j = 0; j < steps; ++j) {
                    const int k2 = lo2 + j;
                    const bool hit = j < len && image_decide<T, MODE>(g, k0, k1, k2, ex, ey, ez,
                                                                      s, t, dw, xs.p, xt.p);
                    const unsigned long long m = ballot(hit) & seg;
                    if (hit)
                        write_hit(a, cursor + __popcll(m & below), s, t,
                                  shift_i32(k0, xt.w.x, xs.w.x), shift_i32(k1, xt.w.y, xs.w.y),
                                  shift_i32(k2, xt.w.z, xs.w.z), xs.p, xt.p, g.c, g.diagonal);
                    cursor += __popcll(m);
                }
            }
        }
    }
    return hits;
}

// Atoms of a structure staged in LDS per wave (structures up to this size).
// 120 float atoms make 7,808 bytes per wave, 31,232 per workgroup: five
// workgroups per CU fit in the 160 KiB of LDS with room to spare.  At
// exactly 32 KiB per workgroup (128 atoms) only four were resident at once,
// although the occupancy query reported five, so a grid sized by the query
// left a fifth of its workgroups waiting for the first ones to finish.
constexpr int kBruteStage = 120;

// Per source of a brute-force work unit: its pair count (counting) or its
// next output (emitting).
union BruteCursor {
    int cnt[kBruteGroupCap];
    long long cur[kBruteGroupCap];
};

// Per-wave LDS of the brute-force kernels: the structure's atoms and the
// unit's per-source cursors.
template <typename T>
struct BruteLds {
    Vec4<T> q[kBruteStage];
    int4 w[kBruteStage];
    Vec4<T> p[kBruteStage];
    BruteCursor c;
};

__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
}

// Pairs of the unit's sources before source x (0 <= x <= G) when the unit
// starts at local source f of a structure of n atoms: x n for a full list;
// for a half list (targets t >= s) sum_{k < x} (n - f - k).
template <int MODE>
__device__ __forceinline__ int64_t unit_pairs_before(int x, int n, int f) {
    if constexpr ((MODE & 2) != 0) return (int64_t)x * (2 * (int64_t)(n - f) - x + 1) / 2;
    return (int64_t)x * n;
}

// Source offset x of triple p within a unit of W k0 values: the largest x
// with W unit_pairs_before(x) <= p, from a double estimate (off by at most
// one) corrected in integers.
template <int MODE>
__device__ __forceinline__ int unit_source_of(int64_t p, int n, int f, int G, int W) {
    int x;
    if constexpr ((MODE & 2) != 0) {
        const double A = (double)(2 * (int64_t)(n - f) + 1);
        x = (int)((A - sqrt(fmax(A * A - 8.0 * ((double)p / (double)W), 0.0))) * 0.5);
    } else {
        x = (int)(((double)p + 0.5) / ((double)n * (double)W));
    }
    x = min(max(x, 0), G - 1);
    if (x + 1 < G && (int64_t)W * unit_pairs_before<MODE>(x + 1, n, f) <= p) ++x;
    if (x > 0 && (int64_t)W * unit_pairs_before<MODE>(x, n, f) > p) --x;
    return x;
}

// q / d (returned) and q mod d (rem) for 0 <= q < 2^24 and d >= 1, from a
// float estimate: (float)q is exact and q * inv_d (inv_d = 1 / d rounded)
// is within one of q / d, so one correction step gives the quotient.
__device__ __forceinline__ int div_small(int q, int d, float inv_d, int& rem) {
    int x = (int)((float)q * inv_d);
    int r = q - x * d;
    if (r < 0) {
        --x;
        r += d;
    } else if (r >= d) {
        ++x;
        r -= d;
    }
    rem = r;
    return x;
}

// Work unit u of the brute-force structures, of structure b: sources
// [first, first + G) and the k0 values of one slice.  Their (source, k0,
// target) triples (targets t >= s for a half list), in source order, then
// k0, then target, are taken 64 per round, lane l taking triple 64 r + l;
// the atoms of a structure of up to kBruteStage atoms are staged in the
// wave's LDS first.  Counting adds each lane's pairs to its source's count
// (one LDS add per source run of the round); at the end it stores counts[s],
// or, for a sliced source, adds it to counts[s] (zeroed by k_atoms) and
// keeps the slice's count in the source's hit-mask slot.  Emitting places a
// source's pairs from offsets[s] plus the counts of its earlier slices on,
// carrying its next output position from round to round in LDS.  Without
// STAGE (L null) the atoms are always read from global memory and only the
// cursors C live in LDS: the form the cell-list counting kernel runs for the
// structures of an explicit cell_list request that no bin grid fits.
template <typename T, int MODE, bool EMIT, bool STAGE = true>
__device__ __forceinline__ void brute_unit(const QueryArgs<T>& a, int64_t u, int b,
                                           BruteLds<T>* L, BruteCursor& C) {
    const StructRec& r = a.recs[b];
    BruteGeom<T> g;
    brute_geom(a, r, b, g);
    const int a0 = (int)r.atom0, n = (int)r.natoms;
    const int nsl = r.bslices;
    const int64_t ul = u - r.unit0;
    const int grp = (int)(ul / nsl), sl = (int)(ul - (int64_t)grp * nsl);
    const int f = grp * r.bgroup;
    const int G = min(r.bgroup, n - f);
    const int k0a = -g.R0 + sl * r.bwidth;
    const int W = min(r.bwidth, g.R0 - k0a + 1);  // k0 values of the slice
    // slice counts of the unit's sources: hit-mask slot words
    unsigned long long* slice_cnt = a.masks + (r.mask0 + f) * a.mask_words;
    const int lane = lane_id();
    const bool staged = STAGE && n <= kBruteStage;
    if (staged) {
        for (int i = lane; i < n; i += kWave) {
            const WalkAtom<T> x = walk_atom(a, a0 + i);
            L->q[i] = x.q;
            L->w[i] = x.w;
            L->p[i] = Vec4<T>{x.p[0], x.p[1], x.p[2], T(0)};
        }
    }
    for (int x = lane; x < G; x += kWave) {
        if (EMIT) {
            long long o = a.offsets[a0 + f + x];
            for (int j = 0; j < sl; ++j) o += (long long)slice_cnt[(int64_t)x * a.mask_words + j];
            C.cur[x] = o;
        } else {
            C.cnt[x] = 0;
        }
    }
    wave_lds_fence();
    // the atoms of the unit's pairs: from LDS when staged, else from global
    // memory (two instances of the round loop below, so that each one's
    // loads keep their own address space)
    auto atom = [&](auto from_lds, int i) {
        WalkAtom<T> x;
        if constexpr (decltype(from_lds)::value) {
            x.q = L->q[i];
            x.w = L->w[i];
            const Vec4<T> p = L->p[i];
            x.p[0] = p.x;
            x.p[1] = p.y;
            x.p[2] = p.z;
        } else {
            x = walk_atom(a, a0 + i);
        }
        return x;
    };
    const int64_t total = (int64_t)W * unit_pairs_before<MODE>(G, n, f);
    // a full list of fewer than 2^24 triples: (source, k0, target) by two
    // small divisions (the unit's triples are source-major blocks of n W)
    const bool small = (MODE & 2) == 0 && total < (int64_t{1} << 24);
    const int nW = small ? n * W : 1;
    const float inv_nW = 1.0f / (float)nW, inv_n = 1.0f / (float)n;
    auto rounds = [&](auto from_lds) {
        for (int64_t base = 0; base < total; base += kWave) {
            const int64_t p = base + lane;
            const bool valid = p < total;
            const int64_t pc = min(p, total - 1);
            int x, k0i, tr;
            int64_t q0;
            if (small) {
                int rem;
                x = div_small((int)pc, nW, inv_nW, rem);
                k0i = div_small(rem, n, inv_n, tr);
                q0 = (int64_t)x * nW;
            } else {
                x = unit_source_of<MODE>(pc, n, f, G, W);
                q0 = (int64_t)W * unit_pairs_before<MODE>(x, n, f);
                // (k0, target) of the triple: q = k0i * len + t, len targets per k0
                const int len = (MODE & 2) ? n - (f + x) : n;
                const int64_t q = pc - q0;
                k0i = (int)((double)q / (double)len);
                tr = (int)(q - (int64_t)k0i * len);
                if (tr < 0) {
                    --k0i;
                    tr += len;
                } else if (tr >= len) {
                    ++k0i;
                    tr -= len;
                }
            }
            const int li = f + x;
            const int tl = ((MODE & 2) ? li : 0) + tr;
            // lanes of this round that hold triples of the same source
            const int seg_lo = (int)max(q0 - base, (int64_t)0);
            const int64_t q1 = small ? q0 + nW : (int64_t)W * unit_pairs_before<MODE>(x + 1, n, f);
            const int seg_hi = (int)min(q1 - base, (int64_t)kWave);
            const unsigned long long seg =
                (seg_hi >= kWave ? ~0ull : ((1ull << seg_hi) - 1ull)) & ~((1ull << seg_lo) - 1ull);
            const WalkAtom<T> xs = atom(from_lds, li), xt = atom(from_lds, tl);
            const int k0 = k0a + k0i;
            if constexpr (EMIT) {
                long long cursor = C.cur[x];
                pair_images<T, MODE, 1>(a, g, valid, a0 + li, a0 + tl, k0, xs, xt, seg, cursor);
                wave_lds_fence();
                if (valid && lane == seg_hi - 1) C.cur[x] = cursor;
            } else {
                long long unused = 0;
                const int h = pair_images<T, MODE, 0>(a, g, valid, a0 + li, a0 + tl, k0, xs, xt,
                                                      seg, unused);
                const int incl = wave_inclusive_scan_i32(h);
                const int before = __shfl(incl, max(seg_lo - 1, 0));
                if (valid && lane == seg_hi - 1) C.cnt[x] += incl - (seg_lo > 0 ? before : 0);
            }
            wave_lds_fence();
        }
    };
    if (staged)
        rounds(std::true_type{});
    else
        rounds(std::false_type{});
    if (!EMIT) {
        for (int x = lane; x < G; x += kWave) {
            const int c = C.cnt[x];
            if (nsl == 1) {
                a.counts[a0 + f + x] = c;
            } else {
                slice_cnt[(int64_t)x * a.mask_words + sl] = (unsigned long long)c;
                atomicAdd(reinterpret_cast<unsigned long long*>(a.counts + a0 + f + x),
                          (unsigned long long)c);
            }
        }
    }
    wave_lds_fence();
}

// ---------------------------------------------------------------- molecules
//
// Brute-force structures with no periodic axis and at most kMoleculeCap
// atoms (molecule_path).  They have one image, k = 0, and no wraps, so the
// output shift is zero and the public predicate is the whole test: with
// S = 0 every product S_a * cell_ac of the public formula is a signed zero,
// and adding a signed zero leaves a nonzero value unchanged (a zero
// component can only change sign), so d2 = ((dx dx + dy dy) + dz dz) with
// d = p_t - p_s, rounded after every operation, is the public d2 bit for
// bit.  The passes read the positions themselves (every wrap is zero).
// The identity policy reduces to t != s (full list) or t > s (half list),
// and include_self keeps t == s.  A work unit holds bgroup consecutive
// sources, bgroup x chunks <= kMolUnitWork (chunk c: targets 64 c .. 64 c +
// 63).
//   Counting: lane l holds target 64 c + l of each chunk c of a register
//   pass; each source is read from the lane that holds it, and one ballot
//   per (source, chunk) gives the hit mask, stored in the hit-mask buffer
//   from the structure's slot mask0 on (a row of mask_words words per atom).
//   Emitting: the unit's masks are decoded into a list of (source, target)
//   entries in the wave's LDS, in source and target order, and written 64
//   pairs per round.  The unit's sources are consecutive atoms, so their
//   pairs form one contiguous output range from offsets[first source].

constexpr int kMolPass = 8;                   // chunks per register pass (counting)
constexpr int kMolList = kMolUnitWork * kWave;  // hits of one unit, at most
static_assert(kMoleculeCap <= 2048 && kMoleculeCap <= kMaskWords * kWave,
              "molecule list entries: 11 bits of target; one mask word per chunk");

template <typename T, int MODE>
__device__ __forceinline__ void molecule_count(const QueryArgs<T>& a, const StructRec& r,
                                               int64_t u, int64_t unit0) {
    using O = Ops<T>;
    const int lane = lane_id();
    const int a0 = (int)r.atom0, n = (int)r.natoms;
    const int f = (int)(u - unit0) * r.bgroup;
    const int G = min(r.bgroup, n - f);  // <= kMolUnitWork
    const int nch = (n + kWave - 1) / kWave;
    const T cut2 = (T)r.cut2;
    T sx = 0, sy = 0, sz = 0;  // lane g: source f + g
    if (lane < G) {
        const int64_t i = 3 * (int64_t)(a0 + f + lane);
        sx = a.pos[i];
        sy = a.pos[i + 1];
        sz = a.pos[i + 2];
        // every atom is a source of one unit: the check of the atom pass,
        // which a request planned by k_molecule_setup does not run
        if (!(isfinite((double)sx) && isfinite((double)sy) && isfinite((double)sz)))
            atomicOr(a.status + SS_FLAGS, ST_POS_NONFINITE);
    }
    int cnt = 0;  // lane g: pairs of source f + g
    for (int c0 = 0; c0 < nch; c0 += kMolPass) {
        const int np = min(kMolPass, nch - c0);
        // targets beyond the structure sit at infinity: d2 is never below cut2
        T tx[kMolPass], ty[kMolPass], tz[kMolPass];
        static_for<kMolPass>([&](auto J) {
            constexpr int j = decltype(J)::value;
            const int t = (c0 + j) * kWave + lane;
            tx[j] = ty[j] = tz[j] = (T)__builtin_inf();
            if (j < np && t < n) {
                const int64_t i = 3 * (int64_t)(a0 + t);
                tx[j] = a.pos[i];
                ty[j] = a.pos[i + 1];
                tz[j] = a.pos[i + 2];
            }
        });
        for (int g = 0; g < G; ++g) {
            const int s = f + g;
            const T px = read_lane(sx, g), py = read_lane(sy, g), pz = read_lane(sz, g);
            int mlo = 0, mhi = 0;  // lane j: the mask of chunk c0 + j
            int hits = 0;
            static_for<kMolPass>([&](auto J) {
                constexpr int j = decltype(J)::value;
                if (j < np) {
                    unsigned long long m = 0;
                    // a half list has no target below s
                    if ((MODE & 2) == 0 || (c0 + j + 1) * kWave > s) {
                        const int t = (c0 + j) * kWave + lane;
                        const T dx = O::sub(tx[j], px), dy = O::sub(ty[j], py),
                                dz = O::sub(tz[j], pz);
                        const T d2 = O::add(O::add(O::mul(dx, dx), O::mul(dy, dy)), O::mul(dz, dz));
                        bool keep = d2 < cut2 && ((MODE & 2) != 0 ? t > s : t != s);
                        if constexpr ((MODE & 1) != 0) keep = keep || t == s;
                        m = ballot(keep);
                    }
                    hits += __popcll(m);
                    mlo = write_lane<j>(mlo, (int)(unsigned)m);
                    mhi = write_lane<j>(mhi, (int)(unsigned)(m >> 32));
                }
            });
            if (lane < np)
                a.masks[(r.mask0 + s) * a.mask_words + c0 + lane] =
                    ((unsigned long long)(unsigned)mhi << 32) | (unsigned)mlo;
            cnt += lane == g ? hits : 0;
        }
    }
    if (lane < G) a.counts[a0 + f + lane] = cnt;
}

template <typename T, int MODE>
__device__ __forceinline__ void molecule_emit(const QueryArgs<T>& a, const StructRec& r, int b,
                                              int64_t u, int* list) {
    const int lane = lane_id();
    const int a0 = (int)r.atom0, n = (int)r.natoms;
    const int f = (int)(u - r.unit0) * r.bgroup;
    const int G = min(r.bgroup, n - f);
    const int nch = (n + kWave - 1) / kWave;
    const int nw = G * nch;  // mask words of the unit, <= kMolUnitWork
    const long long base = a.offsets[a0 + f];
    unsigned long long mw = 0;  // lane g * nch + j: mask of source f + g, chunk j
    if (lane < nw) {
        const int g = lane / nch;
        mw = a.masks[(r.mask0 + f + g) * a.mask_words + (lane - g * nch)];
    }
    const T* cell = a.cells + 9 * b;
    T c[9];
#pragma unroll
    for (int e = 0; e < 9; ++e) c[e] = cell[e];
    const bool diagonal = r.diagonal != 0;
    // entries (g << 11) | t in output order
    int len = 0;
    for (int g = 0, w = 0; g < G; ++g) {
        for (int j = 0; j < nch; ++j, ++w) {
            const unsigned long long m = (unsigned long long)read_lane((long long)mw, w);
            if ((m >> lane) & 1ull) list[len + lanes_below(m)] = (g << 11) | (j * kWave + lane);
            len += __popcll(m);
        }
    }
    wave_lds_fence();
    for (int k = lane; k < len; k += kWave) {
        const int e = list[k];
        const int s = a0 + f + (e >> 11), t = a0 + (e & 2047);
        T ps[3], pt[3];
#pragma unroll
        for (int x = 0; x < 3; ++x) {
            ps[x] = a.pos[3 * (int64_t)s + x];
            pt[x] = a.pos[3 * (int64_t)t + x];
        }
        write_hit(a, base + k, s, t, 0, 0, 0, ps, pt, c, diagonal);
    }
    wave_lds_fence();  // the next unit rewrites the list
}

// Per-wave LDS of the brute-force kernels: the image walk's atoms and
// cursors, or a molecule unit's hit list.
template <typename T>
union BruteWaveLds {
    BruteLds<T> walk;
    int mol[kMolList];
};

// Counting (EMIT false) or emitting pass of the brute-force structures: one
// wave per work unit (grid-stride).  Exits at once when the request has no
// brute-force structure.
template <typename T, int MODE, bool EMIT>
__global__ __launch_bounds__(kBlock) void k_brute(QueryArgs<T> a) {
    if ((load_status(a.status + SS_FLAGS) & kAbortBits) ||
        !(load_status(a.status + SS_PLAN) & 1))
        return;
    if constexpr (EMIT) place_edge_index(a);
    __shared__ BruteWaveLds<T> s_lds[kWavesPerBlock];
    const int64_t units = (int64_t)load_status(a.status + SS_TOTAL_UNITS);
    const int wv = uniform(threadIdx.x / kWave);
    const int64_t wave0 = (int64_t)blockIdx.x * kWavesPerBlock + wv;
    const int64_t nwaves = (int64_t)gridDim.x * kWavesPerBlock;
    int need = 0;  // counting: the longest hit-mask row the wave's structures want
    for (int64_t u = wave0; u < units; u += nwaves) {
        const int b = uniform(unit_structure(a.struct_unit_off, a.nb, u));
        const StructRec& r = a.recs[b];
        if constexpr (!EMIT) need = max(need, r.mneed);
        if (molecule_rec(r)) {
            if constexpr (EMIT)
                molecule_emit<T, MODE>(a, r, b, u, s_lds[wv].mol);
            else
                molecule_count<T, MODE>(a, r, u, r.unit0);
        } else {
            brute_unit<T, MODE, EMIT>(a, u, b, &s_lds[wv].walk, s_lds[wv].walk.c);
        }
    }
    if constexpr (!EMIT) report_mask_need(a.status, need);
}

// The workgroup summaries of a molecule prologue without the batch scan
// (QueryArgs::mol_local), as every counting wave reads them: lane l holds
// workgroup l's exclusive unit offset.
struct MolScan {
    int off;                   // lane l: units of workgroups before l
    int total;                 // units of the request
    int nblk;                  // workgroups of the prologue (at most kWave)
    unsigned long long flags;  // every structure's error bits
    long long images;
};

template <typename T>
__device__ __forceinline__ MolScan mol_scan(const QueryArgs<T>& a) {
    const int lane = lane_id();
    MolScan m;
    m.nblk = (int)((a.nb + kWave - 1) / kWave);
    MoleculeBlock mb{0, 0ull, 0, 0};
    if (lane < m.nblk) mb = a.mol_blocks[lane];
    const int inc = wave_inclusive_scan_i32((int)mb.units);
    m.off = inc - (int)mb.units;
    m.total = __builtin_amdgcn_readlane(inc, kWave - 1);
    unsigned long long fl = mb.flags;
    long long img = mb.images;
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1) {
        fl |= __shfl_xor(fl, d);
        img += __shfl_xor(img, d);
    }
    m.flags = fl;
    m.images = img;
    return m;
}

// Structure of unit u and its first unit under mol_local: the workgroup
// from the lanes' offsets, then the structure from its block-local offsets
// (one load per lane).
template <typename T>
__device__ __forceinline__ int mol_unit_structure(const QueryArgs<T>& a, const MolScan& m,
                                                  int64_t u, int64_t& unit0) {
    const int lane = lane_id();
    const unsigned long long mb = ballot(lane < m.nblk && (int64_t)m.off <= u);
    const int B = 63 - __builtin_clzll(mb | 1ull);
    const int64_t base = (int64_t)__builtin_amdgcn_readlane(m.off, B);
    const int64_t b0 = (int64_t)B * kWave;
    const int cnt = (int)min((int64_t)kWave, a.nb - b0);
    const long long lo = lane < cnt ? a.struct_bin_off[b0 + lane] : 0ll;
    const unsigned long long ms = ballot(lane < cnt && base + lo <= u);
    const int k = 63 - __builtin_clzll(ms | 1ull);
    unit0 = base + (int64_t)__builtin_amdgcn_readlane((int)lo, k);
    return (int)(b0 + k);
}

// Counting or emitting pass of a request whose brute-force structures are
// all molecules (plan bit kPlanMolecules, or a molecule plan hint): the
// molecule passes alone, without the registers of the periodic image walk
// that k_brute also holds, so every unit of a large batch is resident at
// once.  Exits at once when the request has no brute-force structure, or
// when the count found one that is not a molecule (an emit launched with an
// earlier call's plan: it writes nothing, and the caller, seeing the
// count's plan, emits again).  Counting under mol_local, each wave first
// scans the prologue's workgroup summaries (mol_scan); the first waves then
// write the global unit offsets (struct_unit_off and each record's unit0)
// for the emitting pass, and wave 0 the status words the batch scan would
// have written.
template <typename T, int MODE, bool EMIT>
__global__ __launch_bounds__(kBlock) void k_molecules(QueryArgs<T> a) {
    const unsigned long long plan = load_status(a.status + SS_PLAN);
    if ((load_status(a.status + SS_FLAGS) & kAbortBits) || !(plan & 1) ||
        !(plan & kPlanMolecules))
        return;
    if constexpr (EMIT) place_edge_index(a);
    __shared__ int s_list[kWavesPerBlock][EMIT ? kMolList : 1];
    const int wv = uniform(threadIdx.x / kWave);
    const int64_t wave0 = (int64_t)blockIdx.x * kWavesPerBlock + wv;
    const int64_t nwaves = (int64_t)gridDim.x * kWavesPerBlock;
    int64_t units = 0;
    MolScan ms{0, 0, 0, 0ull, 0};
    if (!EMIT && a.mol_local) {
        ms = mol_scan(a);
        if (wave0 == 0 && lane_id() == 0) {
            a.status[SS_TOTAL_UNITS] = (unsigned long long)ms.total;
            a.status[SS_TOTAL_IMAGES] = (unsigned long long)ms.images;
            if (ms.flags) atomicOr(a.status + SS_FLAGS, ms.flags);
        }
        if (ms.flags & kAbortBits) return;
        // global unit offsets for the emitting pass (workgroup w of the
        // prologue by wave w, striding when the grid holds fewer waves)
        for (int64_t w = wave0; w < ms.nblk; w += nwaves) {
            const int base = __builtin_amdgcn_readlane(ms.off, (int)w);
            const int64_t b = w * kWave + lane_id();
            if (b < a.nb) {
                const long long off = a.struct_bin_off[b] + (long long)base;
                const_cast<int64_t*>(a.struct_unit_off)[b] = off;
                const_cast<StructRec*>(a.recs)[b].unit0 = off;
            }
            if (w == ms.nblk - 1 && lane_id() == 0)
                const_cast<int64_t*>(a.struct_unit_off)[a.nb] = (int64_t)ms.total;
        }
        units = ms.total;
    } else {
        units = (int64_t)load_status(a.status + SS_TOTAL_UNITS);
    }
    int need = 0;  // counting: the longest hit-mask row the wave's molecules want
    for (int64_t u = wave0; u < units; u += nwaves) {
        int b;
        int64_t unit0;
        if (!EMIT && a.mol_local) {
            b = uniform(mol_unit_structure(a, ms, u, unit0));
        } else {
            b = uniform(unit_structure(a.struct_unit_off, a.nb, u));
            unit0 = a.recs[b].unit0;
        }
        const StructRec& r = a.recs[b];
        if constexpr (EMIT) {
            molecule_emit<T, MODE>(a, r, b, u, s_list[wv]);
        } else {
            need = max(need, r.mneed);
            molecule_count<T, MODE>(a, r, u, unit0);
        }
    }
    if constexpr (!EMIT) report_mask_need(a.status, need);
}

}  // namespace tnr
