// Query kernels: the cell-list stencil walk (k_cell) and the brute-force
// image walk (k_brute), each in a counting and an emitting flavour.
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
    const int64_t* struct_bin_off;  // B + 1
    const int* atom_struct;
    const int4* atom_wrap;
    const Vec4<T>* atom_q;
    const int* bin_start;
    const Vec4<T>* binned;
    long long* counts;
    const long long* offsets;
    unsigned long long* masks;      // kMaxChunks per binned source
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
                                          const T ps[3], const T pt[3], const T* cell,
                                          bool diagonal) {
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
        const T d2 = diagonal ? public_vector_diag(ps, pt, S0, S1, S2, cell, D)
                              : public_vector(ps, pt, S0, S1, S2, cell, D);
        if (a.vec) {
            a.vec[3 * o] = D[0];
            a.vec[3 * o + 1] = D[1];
            a.vec[3 * o + 2] = D[2];
        }
        if (a.dist) a.dist[o] = Ops<T>::sqrt_(d2);
    }
}

// Identity filter of pair_policy.h:42-79 for a candidate whose output shift
// equals the image shift k when s == t.
template <int MODE>
__device__ __forceinline__ bool identity_ok(int s, int t, bool kzero, bool kneg) {
    if (s == t && kzero) return (MODE & 1) != 0;
    if constexpr ((MODE & 2) != 0) return s < t || (s == t && kneg);
    return true;
}

// -------------------------------------------------------------------- brute

// One wave per source atom of a brute-force structure (grid-stride).  Lanes
// hold 64 targets; the wave walks the image box of the structure in the
// reference order (x-major, z fastest).
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
                                write_hit(a, cursor + lanes_below(m), s, t, S0, S1, S2, ps, pt, c,
                                          diagonal);
                            cursor += __popcll(m);
                        }
                    }
                }
            }
        }
        if (!EMIT && lane == 0) a.counts[s] = total;
    }
}

// --------------------------------------------------------------------- cell

// Per-wave stencil table in LDS.
constexpr int kMapCap = kMaxChunks * kWave;  // candidates with a direct piece map

template <typename T>
struct Stencil {
    int pre[kPieceCap + 1];   // exclusive prefix of piece lengths
    int delta[kPieceCap];     // binned index = candidate index + delta
    int kid[kPieceCap];       // packed image shift (k + 512 per 10 bits)
    T tr[3][kPieceCap];       // broad-phase translation k . cell
    unsigned char piece[kMapCap];  // piece of each candidate (when C <= kMapCap)
};

__device__ __forceinline__ int pack_k(int kx, int ky, int kz) {
    return (kx + 512) | ((ky + 512) << 10) | ((kz + 512) << 20);
}
__device__ __forceinline__ void unpack_k(int v, int& kx, int& ky, int& kz) {
    kx = (v & 1023) - 512;
    ky = ((v >> 10) & 1023) - 512;
    kz = ((v >> 20) & 1023) - 512;
}

// The band between inner2 and outer2: decided by the public predicate on the
// original positions and the output shift.
template <typename T>
__device__ __forceinline__ bool cell_band(const QueryArgs<T>& a, int tid, int kx, int ky,
                                                    int kz, int bidx, T sx, T sy, T sz, int si,
                                                    T cut2, bool wrapped, const T* gcell) {
    bool ok;
    {
        T ps[3], pt[3];
        long long S0 = kx, S1 = ky, S2 = kz;
        if (wrapped) {
            const int4 wt = a.atom_wrap[tid];
            const int4 ws = a.atom_wrap[si];
            S0 += (long long)ws.x - wt.x;
            S1 += (long long)ws.y - wt.y;
            S2 += (long long)ws.z - wt.z;
#pragma unroll
            for (int cc = 0; cc < 3; ++cc) {
                ps[cc] = a.pos[3 * (int64_t)si + cc];
                pt[cc] = a.pos[3 * (int64_t)tid + cc];
            }
        } else {
            const Vec4<T> rec = a.binned[bidx];
            ps[0] = sx; ps[1] = sy; ps[2] = sz;
            pt[0] = rec.x; pt[1] = rec.y; pt[2] = rec.z;
        }
        T c[9];
#pragma unroll
        for (int e = 0; e < 9; ++e) c[e] = gcell[e];
        T D[3];
        ok = public_vector(ps, pt, S0, S1, S2, c, D) < cut2;
    }
    return ok;
}

// Broad-phase + identity + band decision for one candidate lane against one
// source; returns whether the pair is kept.  `bidx` is the candidate's
// binned index (its untranslated record, for the band case).
template <typename T, int MODE>
__device__ __forceinline__ bool cell_keep(const QueryArgs<T>& a, T tx, T ty, T tz, int tid, int kk,
                                          int bidx, T sx, T sy, T sz, int si, T outer2,
                                          T inner2, T cut2, bool wrapped, const T* gcell) {
    using O = Ops<T>;
    int kx, ky, kz;
    unpack_k(kk, kx, ky, kz);
    const bool kzero = kk == pack_k(0, 0, 0);
    const T dx = O::sub(tx, sx), dy = O::sub(ty, sy), dz = O::sub(tz, sz);
    const T d2 = O::fma_(dz, dz, O::fma_(dy, dy, O::mul(dx, dx)));
    const bool zsf = tid == si && kzero;
    bool ok = tid >= 0 && (d2 < outer2 || zsf) &&
              identity_ok<MODE>(si, tid, kzero, lex_negative(kx, ky, kz));
    if (ok && !zsf && !(d2 < inner2))
        ok = cell_band(a, tid, kx, ky, kz, bidx, sx, sy, sz, si, cut2, wrapped, gcell);
    return ok;
}

// Writes one kept candidate of source si: the output shift is the image k
// corrected by the representatives' wraps; D uses the original positions.
template <typename T>
__device__ __forceinline__ void cell_write(const QueryArgs<T>& a, long long o, int si, int tid,
                                           int kk, T rx, T ry, T rz, T sx, T sy, T sz,
                                           bool wrapped, bool diagonal, const T* c) {
    int kx, ky, kz;
    unpack_k(kk, kx, ky, kz);
    long long S0 = kx, S1 = ky, S2 = kz;
    T ps[3] = {sx, sy, sz}, pt[3] = {rx, ry, rz};
    if (wrapped) {
        const int4 wt = a.atom_wrap[tid];
        const int4 ws = a.atom_wrap[si];
        S0 += (long long)ws.x - wt.x;
        S1 += (long long)ws.y - wt.y;
        S2 += (long long)ws.z - wt.z;
#pragma unroll
        for (int cc = 0; cc < 3; ++cc) {
            ps[cc] = a.pos[3 * (int64_t)si + cc];
            pt[cc] = a.pos[3 * (int64_t)tid + cc];
        }
    }
    write_hit(a, o, si, tid, S0, S1, S2, ps, pt, c, diagonal);
}

template <typename T>
__device__ __forceinline__ void shift_check(const QueryArgs<T>& a, int tid, int kk, int si) {
    int kx, ky, kz;
    unpack_k(kk, kx, ky, kz);
    const int4 wt = a.atom_wrap[tid];
    const int4 ws = a.atom_wrap[si];
    if (!(fits_i32((long long)kx - wt.x + ws.x) && fits_i32((long long)ky - wt.y + ws.y) &&
          fits_i32((long long)kz - wt.z + ws.z)))
        atomicOr(a.status + SS_FLAGS, ST_SHIFT_RANGE);
}

constexpr int kSourceGroup = kWave / kMaxChunks;  // sources per mask load

// Returns x unchanged but hides its value from the optimiser, so values
// derived from it inside a loop are recomputed rather than hoisted into
// registers for every unrolled chunk.
__device__ __forceinline__ int opaque(int x) {
    asm volatile("" : "+v"(x));
    return x;
}

// Candidate v of the stencil: binned index and piece (map or binary search).
template <typename T>
__device__ __forceinline__ int stencil_piece(const Stencil<T>& st, int v, int C, int npieces,
                                             int top) {
    if (C <= kMapCap) return st.piece[v];
    int p = 0;
    for (int step = top; step > 0; step >>= 1) {
        const int q = p + step;
        if (q < npieces && st.pre[q] <= v) p = q;
    }
    return p;
}

// Band candidates of one source (d2 in [inner2, outer2)): decide each with
// the public predicate, OR the accepted lanes into the stored masks and
// return how many were added.  Rare: the band is ~1e-4 of the cutoff wide.
template <typename T, int MODE>
__device__ __forceinline__ long long cell_band_fixup(
    const QueryArgs<T>& a, const Stencil<T>& st, unsigned long long* mrow, unsigned chunks, T sx,
    T sy, T sz, int si, int C, T outer2, T inner2, T cut2, bool wrapped, const T* gcell) {
    using O = Ops<T>;
    const int lane = lane_id();
    long long added = 0;
#pragma unroll 1
    for (int j = 0; j < kMaxChunks; ++j) {
        if (!((chunks >> j) & 1u)) continue;
        const int v = j * kWave + lane;
        bool ok = false;
        if (v < C) {
            const int p = st.piece[v];
            const int bidx = v + st.delta[p];
            const Vec4<T> rec = a.binned[bidx];
            const int tid = as_idx(rec.w);
            int kx, ky, kz;
            unpack_k(st.kid[p], kx, ky, kz);
            const bool kzero = kx == 0 && ky == 0 && kz == 0;
            const T tx = O::add(rec.x, st.tr[0][p]), ty = O::add(rec.y, st.tr[1][p]),
                    tz = O::add(rec.z, st.tr[2][p]);
            const T dx = O::sub(tx, sx), dy = O::sub(ty, sy), dz = O::sub(tz, sz);
            const T d2 = O::fma_(dz, dz, O::fma_(dy, dy, O::mul(dx, dx)));
            const bool zsf = tid == si && kzero;
            const bool keep = (d2 < outer2 || zsf) &&
                              identity_ok<MODE>(si, tid, kzero, lex_negative(kx, ky, kz));
            if (keep && !zsf && !(d2 < inner2)) {
                ok = cell_band(a, tid, kx, ky, kz, bidx, sx, sy, sz, si, cut2, wrapped, gcell);
                if (ok && wrapped) shift_check(a, tid, st.kid[p], si);
            }
        }
        const unsigned long long m = ballot(ok);
        if (m) {
            if (lane == 0) mrow[j] |= m;
            added += __popcll(m);
        }
    }
    return added;
}

// Stencils with more than kMaxChunks chunks (coarse grids): one chunk at a
// time, decisions recomputed in both passes (no masks).
template <typename T, int MODE, bool EMIT>
__device__ __forceinline__ void cell_slow(const QueryArgs<T>& a, const Stencil<T>& st,
                                                    int sb, int se, int C, int nch, int npieces,
                                                    int top, T outer2, T inner2, T cut2,
                                                    bool wrapped, bool diagonal, const T* c,
                                                    const T* gcell) {
    using O = Ops<T>;
    const int lane = lane_id();
    for (int sg = sb; sg < se; sg += kWave) {
        const int ns = min(kWave, se - sg);
        Vec4<T> sq = {T(0), T(0), T(0), T(0)};
        int sidx = 0;
        if (lane < ns) {
            sq = a.binned[sg + lane];
            sidx = as_idx(sq.w);
        }
        long long acc = 0, cur = 0;
        if (EMIT && lane < ns) cur = a.offsets[sidx];
        for (int j = 0; j < nch; ++j) {
            const int v = j * kWave + lane;
            int tid = -1, kk = pack_k(0, 0, 0), bidx = 0;
            T tx = T(0), ty = T(0), tz = T(0), rx = T(0), ry = T(0), rz = T(0);
            if (v < C) {
                const int p = stencil_piece(st, v, C, npieces, top);
                bidx = v + st.delta[p];
                const Vec4<T> rec = a.binned[bidx];
                tid = as_idx(rec.w);
                kk = st.kid[p];
                rx = rec.x;
                ry = rec.y;
                rz = rec.z;
                tx = O::add(rec.x, st.tr[0][p]);
                ty = O::add(rec.y, st.tr[1][p]);
                tz = O::add(rec.z, st.tr[2][p]);
            }
            for (int gi = 0; gi < ns; ++gi) {
                const T sx = read_lane(sq.x, gi), sy = read_lane(sq.y, gi),
                        sz = read_lane(sq.z, gi);
                const int si = read_lane(sidx, gi);
                const bool ok = cell_keep<T, MODE>(a, tx, ty, tz, tid, kk, bidx, sx, sy, sz, si,
                                                   outer2, inner2, cut2, wrapped, gcell);
                const unsigned long long m = ballot(ok);
                if (!EMIT) {
                    if (wrapped && ok) shift_check(a, tid, kk, si);
                    if (lane == gi) acc += __popcll(m);
                } else if (m) {
                    const long long base = read_lane(cur, gi);
                    if (ok)
                        cell_write(a, base + lanes_below(m), si, tid, kk, rx, ry, rz, sx, sy, sz,
                                   wrapped, diagonal, c);
                    if (lane == gi) cur += __popcll(m);
                }
            }
        }
        if (!EMIT && lane < ns) a.counts[sidx] = acc;
    }
}

// One wave per bin of a cell-list structure (grid-stride over all bins,
// XCD-grouped).  The stencil of the bin is cut into pieces: runs of
// consecutive z-bins of one (x, y) row with one periodic image k (one lane
// per piece).  Pieces with |k_a| > R_a are dropped, which keeps exactly the
// reference's image box.  When the flattened stencil has at most
// kMaxChunks chunks of 64 candidates (the common case) they are gathered
// into registers once and the bin's sources are broadcast one at a time;
// the counting pass stores one 64-bit hit mask per (source, chunk) and the
// emitting pass replays those masks, so both passes see identical pairs and
// the emitting pass does no distance tests.  Larger stencils (coarse grids)
// take a chunk-at-a-time path that recomputes the decisions.
template <typename T, int MODE, bool EMIT>
__global__ __launch_bounds__(kBlock) void k_cell(QueryArgs<T> a) {
    using O = Ops<T>;
    __shared__ Stencil<T> s_st[kWavesPerBlock];

    if (load_status(a.status + SS_FLAGS) & kAbortBits) return;
    const int lane = lane_id();
    const int wv = threadIdx.x / kWave;
    Stencil<T>& st = s_st[wv];
    // XCD-grouped block order: the hardware deals blocks round-robin over 8
    // XCDs; give each XCD a contiguous range of logical blocks.
    const unsigned nblk = gridDim.x;
    unsigned lb = blockIdx.x;
    if ((nblk & 7u) == 0) lb = (blockIdx.x & 7u) * (nblk >> 3) + (blockIdx.x >> 3);
    const int64_t wave0 = (int64_t)lb * kWavesPerBlock + wv;
    const int64_t nwaves = (int64_t)nblk * kWavesPerBlock;
    const int64_t total_bins = a.struct_bin_off[a.nb];

    for (int64_t g = wave0; g < total_bins; g += nwaves) {
        const int sb = a.bin_start[g], se = a.bin_start[g + 1];
        if (sb == se) continue;
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
        const bool diagonal = r.diagonal != 0;
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
        const int npieces = (2 * Kx + 1) * RY * zs;
        const int* bstart = a.bin_start + r.bin0;

        // ---- stencil pieces, one lane per piece
        int carry = 0;
        for (int base = 0; base < npieces; base += kWave) {
            const int p = base + lane;
            int len = 0, start = 0, kx = 0, ky = 0, kz = 0;
            if (p < npieces) {
                const int row = p / zs, seg = p - row * zs;
                const int ox = row / RY - Kx, oy = row % RY - Ky;
                int jx = ix + ox, jy = iy + oy;
                bool ok = true;
                if (perx) {
                    kx = floor_div(jx, nx);
                    jx -= kx * nx;
                    ok = ok && abs(kx) <= R0;
                } else {
                    ok = ok && jx >= 0 && jx < nx;
                }
                if (pery) {
                    ky = floor_div(jy, ny);
                    jy -= ky * ny;
                    ok = ok && abs(ky) <= R1;
                } else {
                    ok = ok && jy >= 0 && jy < ny;
                }
                int z0, z1;
                const int zlo = iz - Kz, zhi = iz + Kz;
                if (perz) {
                    const int k0 = floor_div(zlo, nz);
                    kz = k0 + seg;
                    const int zbeg = seg == 0 ? zlo : kz * nz;
                    const int zend = min(zhi, (kz + 1) * nz - 1);
                    ok = ok && zbeg <= zhi && abs(kz) <= R2;
                    z0 = zbeg - kz * nz;
                    z1 = zend - kz * nz;
                } else {
                    z0 = max(0, zlo);
                    z1 = min(nz - 1, zhi);
                    ok = ok && seg == 0 && z0 <= z1;
                }
                if (ok) {
                    const int rowbase = (jx * ny + jy) * nz;
                    start = bstart[rowbase + z0];
                    len = bstart[rowbase + z1 + 1] - start;
                }
            }
            const int inc = wave_inclusive_scan_i32(len);
            if (p < npieces) {
                const int ex = carry + inc - len;
                st.pre[p] = ex;
                st.delta[p] = start - ex;
                st.kid[p] = pack_k(kx, ky, kz);
                st.tr[0][p] = O::fma_((T)kz, c[6], O::fma_((T)ky, c[3], O::mul((T)kx, c[0])));
                st.tr[1][p] = O::fma_((T)kz, c[7], O::fma_((T)ky, c[4], O::mul((T)kx, c[1])));
                st.tr[2][p] = O::fma_((T)kz, c[8], O::fma_((T)ky, c[5], O::mul((T)kx, c[2])));
            }
            carry += __shfl(inc, kWave - 1);
        }
        if (lane == 0) st.pre[npieces] = carry;
        const int C = carry;
        const int nch = (C + kWave - 1) / kWave;
        const bool mapped = C <= kMapCap;
        const bool use_masks = nch <= kMaxChunks;
        if (mapped) {
            // candidate -> piece map: lane p fills the slots of piece p
            for (int base = 0; base < npieces; base += kWave) {
                const int p = base + lane;
                if (p < npieces) {
                    const int b0 = st.pre[p];
                    const int len = (p + 1 < npieces ? st.pre[p + 1] : C) - b0;
                    for (int i = 0; i < len; ++i) st.piece[b0 + i] = (unsigned char)p;
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        int top = 1;
        while (top * 2 <= npieces) top *= 2;

        // ---- sources of this bin
        if (nch > kMaxChunks) {
            cell_slow<T, MODE, EMIT>(a, st, sb, se, C, nch, npieces, top, outer2, inner2, cut2,
                                     wrapped, diagonal, c, cell);
            continue;
        }
        // gather every candidate chunk into registers (one round trip)
        T px[kMaxChunks], py[kMaxChunks], pz[kMaxChunks];
        int tid[kMaxChunks], kk[kMaxChunks];
#pragma unroll
        for (int j = 0; j < kMaxChunks; ++j) {
            const int v = j * kWave + lane;
            tid[j] = -1;
            kk[j] = pack_k(0, 0, 0);
            px[j] = py[j] = pz[j] = T(0);
            if (j < nch && v < C) {
                const int p = st.piece[v];
                const Vec4<T> rec = a.binned[v + st.delta[p]];
                tid[j] = as_idx(rec.w);
                kk[j] = st.kid[p];
                if (EMIT) {  // original positions (for D)
                    px[j] = rec.x;
                    py[j] = rec.y;
                    pz[j] = rec.z;
                } else {     // image positions (for the broad phase)
                    px[j] = O::add(rec.x, st.tr[0][p]);
                    py[j] = O::add(rec.y, st.tr[1][p]);
                    pz[j] = O::add(rec.z, st.tr[2][p]);
                }
            }
        }
        for (int sg = sb; sg < se; sg += kSourceGroup) {
            const int ns = min(kSourceGroup, se - sg);
            // lane l < ns: source sg + l; lane l < ns * kMaxChunks (emit): mask
            // (source sg + l / kMaxChunks, chunk l % kMaxChunks)
            Vec4<T> sq = {T(0), T(0), T(0), T(0)};
            int sidx = 0;
            if (lane < ns) {
                sq = a.binned[sg + lane];
                sidx = as_idx(sq.w);
            }
            unsigned long long mreg = 0;
            if (EMIT && lane < ns * kMaxChunks) mreg = a.masks[(int64_t)sg * kMaxChunks + lane];
            long long cur = 0;
            if (EMIT && lane < ns) cur = a.offsets[sidx];
            long long acc = 0;
#pragma unroll 1
            for (int gi = 0; gi < ns; ++gi) {
                const T sx = read_lane(sq.x, gi), sy = read_lane(sq.y, gi),
                        sz = read_lane(sq.z, gi);
                const int si = read_lane(sidx, gi);
                unsigned long long* mrow = a.masks + (int64_t)(sg + gi) * kMaxChunks;
                if (!EMIT) {
                    long long cnt = 0;
                    unsigned band_chunks = 0;
#pragma unroll
                    for (int j = 0; j < kMaxChunks; ++j) {
                        if (j >= nch) continue;
                        const int kj = opaque(kk[j]);
                        const int tj = opaque(tid[j]);
                        const bool kzero = kj == pack_k(0, 0, 0);
                        const T dx = O::sub(px[j], sx), dy = O::sub(py[j], sy),
                                dz = O::sub(pz[j], sz);
                        const T d2 = O::fma_(dz, dz, O::fma_(dy, dy, O::mul(dx, dx)));
                        const bool zsf = tj == si && kzero;
                        bool keep = tj >= 0 && (d2 < outer2 || zsf);
                        if (MODE != 0) {
                            int kx, ky, kz;
                            unpack_k(kj, kx, ky, kz);
                            keep = keep && identity_ok<MODE>(si, tj, kzero,
                                                             lex_negative(kx, ky, kz));
                        } else {
                            keep = keep && !zsf;
                        }
                        const bool band = keep && !zsf && !(d2 < inner2);
                        const unsigned long long m = ballot(keep && !band);
                        if (ballot(band)) band_chunks |= 1u << j;
                        if (wrapped && keep && !band) shift_check(a, tj, kj, si);
                        if (lane == 0) mrow[j] = m;
                        cnt += __popcll(m);
                    }
                    if (band_chunks)
                        cnt += cell_band_fixup<T, MODE>(a, st, mrow, band_chunks, sx, sy, sz, si,
                                                        C, outer2, inner2, cut2, wrapped, cell);
                    if (lane == gi) acc = cnt;
                } else {
                    long long base = read_lane(cur, gi);
#pragma unroll
                    for (int j = 0; j < kMaxChunks; ++j) {
                        if (j >= nch) continue;
                        const unsigned long long m =
                            (unsigned long long)read_lane((long long)mreg, gi * kMaxChunks + j);
                        if (m == 0) continue;
                        if ((m >> lane) & 1ull)
                            cell_write(a, base + lanes_below(m), si, opaque(tid[j]),
                                       opaque(kk[j]), px[j], py[j], pz[j], sx, sy, sz, wrapped,
                                       diagonal, c);
                        base += __popcll(m);
                    }
                }
            }
            if (!EMIT && lane < ns) a.counts[sidx] = acc;
        }
    }
}

}  // namespace tnr
