// Query kernels: the cell-list stencil walk (k_cell_count / k_cell_emit) and
// the brute-force image walk (k_brute), each in a counting and an emitting
// flavour.
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

// One wave per source atom of a brute-force structure (grid-stride).  Lanes
// hold 64 targets; the wave walks the image box of the structure in the
// reference order (x-major, z fastest).
template <typename T, int MODE, bool EMIT>
__global__ __launch_bounds__(kBlock) void k_brute(QueryArgs<T> a) {
    using O = Ops<T>;
    if ((load_status(a.status + SS_FLAGS) & kAbortBits) ||
        !(load_status(a.status + SS_PLAN) & 1))
        return;
    const int lane = lane_id();
    const int64_t wave0 = (int64_t)blockIdx.x * kWavesPerBlock + uniform(threadIdx.x / kWave);
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

// --------------------------------------------------------------------- cell

constexpr int kMapCap = kMaxChunks * kWave;        // candidates of the register path
constexpr int kSourceGroup = kWave / kMaxChunks;   // sources per mask load
constexpr int kListCap = 1024;                     // emit: compacted hits per flush

// Stencil of one source bin, one per wave in LDS.
struct StencilLds {
    int pre[kPieceCap + 1];        // exclusive prefix of piece lengths
    int delta[kPieceCap];          // binned index = candidate index + delta
    int kid[kPieceCap];            // packed image shift (k + 512 per 10 bits)
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

// Broad-phase translation k . cell of image k; every pass that needs it
// evaluates this same expression, so the broad-phase decisions agree.
template <typename T>
__device__ __forceinline__ void image_translation(int kk, const T c[9], T& tx, T& ty, T& tz) {
    using O = Ops<T>;
    int kx, ky, kz;
    unpack_k(kk, kx, ky, kz);
    const T fx = (T)kx, fy = (T)ky, fz = (T)kz;
    tx = O::fma_(fz, c[6], O::fma_(fy, c[3], O::mul(fx, c[0])));
    ty = O::fma_(fz, c[7], O::fma_(fy, c[4], O::mul(fx, c[1])));
    tz = O::fma_(fz, c[8], O::fma_(fy, c[5], O::mul(fx, c[2])));
}

// Wave-uniform description of one source bin of a cell-list structure.
template <typename T>
struct CellBin {
    int b;            // structure
    int sb, se;       // binned sources [sb, se)
    int C;            // flattened stencil candidates
    int npieces;
    T c[9];           // cell (rows are cell vectors)
    T outer2, inner2, cut2;
    bool wrapped, diagonal;
};

// Loads the structure of bin g and builds its stencil: pieces are runs of
// consecutive z-bins of one (x, y) row with one periodic image k, one lane
// per piece; pieces with |k_a| > R_a are dropped, which keeps exactly the
// reference's image box.  Fills the piece table of st (and, when TR, the
// per-piece broad-phase translations) and marks the first candidate of every
// non-empty piece in st.piece for stencil_resolve.  Returns false when the
// bin holds no source.
template <typename T, bool TR>
__device__ __forceinline__ bool cell_bin(const QueryArgs<T>& a, int64_t g, CellBin<T>& cb,
                                         StencilLds& st, T (*tr)[kPieceCap]) {
    const int lane = lane_id();
    // issued first, consumed after the piece loads
    const int sb = a.bin_start[g], se = a.bin_start[g + 1];
    int64_t lo = 0, hi = a.nb;
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) >> 1;
        if (a.struct_bin_off[mid] <= g) lo = mid; else hi = mid;
    }
    cb.b = (int)lo;
    const StructRec& r = a.recs[cb.b];
    const T* cell = a.cells + 9 * cb.b;
#pragma unroll
    for (int e = 0; e < 9; ++e) cb.c[e] = cell[e];
    cb.outer2 = (T)r.outer2;
    cb.inner2 = (T)r.inner2;
    cb.cut2 = (T)r.cut2;
    cb.wrapped = r.any_wrap != 0;
    cb.diagonal = r.diagonal != 0;
    const int nx = r.nb[0], ny = r.nb[1], nz = r.nb[2];  // each at least 1
    const int Kx = r.reach[0], Ky = r.reach[1], Kz = r.reach[2];
    const int R0 = r.reps[0], R1 = r.reps[1], R2 = r.reps[2];
    const bool perx = r.active & 1, pery = r.active >> 1 & 1, perz = r.active >> 2 & 1;
    const int zs = r.zseg;
    // the bins of all structures number fewer than 2^31
    const unsigned lbin = (unsigned)(g - r.bin0);
    const int iz = (int)(lbin % (unsigned)nz);
    const unsigned rest = lbin / (unsigned)nz;
    const int iy = (int)(rest % (unsigned)ny);
    const int ix = (int)(rest / (unsigned)ny);
    const int RY = 2 * Ky + 1;
    const int npieces = (2 * Kx + 1) * RY * zs;
    cb.npieces = npieces;
    const int* bstart = a.bin_start + r.bin0;
    // p / zs and row / RY through a float reciprocal: p < 2^8 and divisors
    // below 2^8, so (p + 1/2) / d lies at least 1/512 from an integer while
    // the float error stays below 2^-15.
    const float rzs = 1.0f / (float)zs, rry = 1.0f / (float)RY;
    const int zlo = iz - Kz, zhi = iz + Kz;
    int kz0 = 0;  // image of the lowest stencil z-bin (zlo < nz)
    if (perz)
        for (int zz = zlo; zz < 0; zz += nz) --kz0;
    // clear the piece marks: kMapCap bytes, 8 per lane
    reinterpret_cast<unsigned long long*>(st.piece)[lane] = 0ull;

    int carry = 0;
    for (int base = 0; base < npieces; base += kWave) {
        const int p = base + lane;
        int len = 0, start = 0, kx = 0, ky = 0, kz = 0;
        if (p < npieces) {
            const int row = (int)(((float)p + 0.5f) * rzs);
            const int seg = p - row * zs;
            const int rx = (int)(((float)row + 0.5f) * rry);
            int jx = ix + rx - Kx, jy = iy + (row - rx * RY) - Ky;
            bool ok;
            if (perx) {
                while (jx < 0) { jx += nx; --kx; }
                while (jx >= nx) { jx -= nx; ++kx; }
                ok = abs(kx) <= R0;
            } else {
                ok = jx >= 0 && jx < nx;
            }
            if (pery) {
                while (jy < 0) { jy += ny; --ky; }
                while (jy >= ny) { jy -= ny; ++ky; }
                ok = ok && abs(ky) <= R1;
            } else {
                ok = ok && jy >= 0 && jy < ny;
            }
            int z0, z1;
            if (perz) {
                kz = kz0 + seg;
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
            const int kk = pack_k(kx, ky, kz);
            st.pre[p] = ex;
            st.delta[p] = start - ex;
            st.kid[p] = kk;
            if (len > 0 && ex < kMapCap) st.piece[ex] = (unsigned char)p;
            if constexpr (TR) image_translation(kk, cb.c, tr[0][p], tr[1][p], tr[2][p]);
        }
        carry += __builtin_amdgcn_readlane(inc, kWave - 1);
    }
    if (lane == 0) st.pre[npieces] = carry;
    cb.C = uniform(carry);
    cb.sb = uniform(sb);
    cb.se = uniform(se);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    return cb.sb != cb.se;
}

// Piece of candidate v = 64 j + lane (C <= kMapCap): the running maximum of
// the piece marks up to v, chunks resolved in increasing j with `carry` the
// previous chunk's last piece.  Stores it in st.piece[v] for random access.
// Called by the whole wave.
__device__ __forceinline__ int stencil_resolve(StencilLds& st, int j, int& carry) {
    const int v = j * kWave + lane_id();
    const int p = max(wave_inclusive_max_i32((int)st.piece[v]), carry);
    carry = __builtin_amdgcn_readlane(p, kWave - 1);
    st.piece[v] = (unsigned char)p;
    return p;
}

// The band between inner2 and outer2: decided by the public predicate on the
// original positions and the output shift.
template <typename T>
__device__ __forceinline__ bool cell_band(const QueryArgs<T>& a, int tid, int kk, int bidx,
                                          T sx, T sy, T sz, int si, const CellBin<T>& cb) {
    int kx, ky, kz;
    unpack_k(kk, kx, ky, kz);
    T ps[3], pt[3];
    long long S0 = kx, S1 = ky, S2 = kz;
    if (cb.wrapped) {
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
    T D[3];
    return public_vector(ps, pt, S0, S1, S2, cb.c, D) < cb.cut2;
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

// Full decision for candidate v (piece p) of the stencil against the source
// at (sx, sy, sz) with index si: broad phase, identity and band.  Used by the
// rare paths; its broad phase is the register path's, operation for operation.
template <typename T, int MODE>
__device__ __forceinline__ bool cell_decide(const QueryArgs<T>& a, const StencilLds& st,
                                            const CellBin<T>& cb, int p, int v, T sx, T sy,
                                            T sz, int si, int* tid_out, int* kk_out,
                                            Vec4<T>* rec_out) {
    using O = Ops<T>;
    const int bidx = v + st.delta[p];
    const Vec4<T> rec = a.binned[bidx];
    const int tid = as_idx(rec.w);
    const int kk = st.kid[p];
    *tid_out = tid;
    *kk_out = kk;
    *rec_out = rec;
    int kx, ky, kz;
    unpack_k(kk, kx, ky, kz);
    T trx, trY, trz;
    image_translation(kk, cb.c, trx, trY, trz);
    const T dx = O::sub(O::add(rec.x, trx), sx), dy = O::sub(O::add(rec.y, trY), sy),
            dz = O::sub(O::add(rec.z, trz), sz);
    const T d2 = O::fma_(dz, dz, O::fma_(dy, dy, O::mul(dx, dx)));
    const bool kzero = kk == pack_k(0, 0, 0);
    const bool zsf = tid == si && kzero;
    bool ok = (d2 < cb.outer2 || zsf) &&
              identity_ok<MODE>(si, tid, kzero, lex_negative(kx, ky, kz));
    if (ok && !zsf && !(d2 < cb.inner2)) ok = cell_band(a, tid, kk, bidx, sx, sy, sz, si, cb);
    return ok;
}

// Candidate v of a stencil too large for the piece map: its piece by binary
// search over the piece starts.
__device__ __forceinline__ int stencil_piece(const StencilLds& st, int v, int npieces) {
    int top = 1;
    while (top * 2 <= npieces) top *= 2;
    int p = 0;
    for (int step = top; step > 0; step >>= 1) {
        const int q = p + step;
        if (q < npieces && st.pre[q] <= v) p = q;
    }
    return p;
}

// Writes one kept candidate of source si: the output shift is the image k
// corrected by the representatives' wraps; D uses the original positions.
template <typename T>
__device__ __forceinline__ void cell_write(const QueryArgs<T>& a, long long o, int si, int tid,
                                           int kk, T rx, T ry, T rz, T sx, T sy, T sz,
                                           const CellBin<T>& cb) {
    int kx, ky, kz;
    unpack_k(kk, kx, ky, kz);
    T ps[3] = {sx, sy, sz}, pt[3] = {rx, ry, rz};
    if (cb.wrapped) {
        const int4 wt = a.atom_wrap[tid];
        const int4 ws = a.atom_wrap[si];
        kx = shift_i32(kx, wt.x, ws.x);
        ky = shift_i32(ky, wt.y, ws.y);
        kz = shift_i32(kz, wt.z, ws.z);
#pragma unroll
        for (int cc = 0; cc < 3; ++cc) {
            ps[cc] = a.pos[3 * (int64_t)si + cc];
            pt[cc] = a.pos[3 * (int64_t)tid + cc];
        }
    }
    write_hit(a, o, si, tid, kx, ky, kz, ps, pt, cb.c, cb.diagonal);
}

// Stencils with more than kMaxChunks chunks (coarse grids): one chunk at a
// time, decisions recomputed in both passes (no masks).
template <typename T, int MODE, bool EMIT>
__device__ __forceinline__ void cell_slow(const QueryArgs<T>& a, const StencilLds& st,
                                          const CellBin<T>& cb) {
    const int lane = lane_id();
    const int nch = (cb.C + kWave - 1) / kWave;
    for (int sg = cb.sb; sg < cb.se; sg += kWave) {
        const int ns = min(kWave, cb.se - sg);
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
            const bool valid = v < cb.C;
            const int p = valid ? stencil_piece(st, v, cb.npieces) : 0;
            for (int gi = 0; gi < ns; ++gi) {
                const T sx = read_lane(sq.x, gi), sy = read_lane(sq.y, gi),
                        sz = read_lane(sq.z, gi);
                const int si = read_lane(sidx, gi);
                int tid = 0, kk = 0;
                Vec4<T> rec = {T(0), T(0), T(0), T(0)};
                const bool ok = valid && cell_decide<T, MODE>(a, st, cb, p, v, sx, sy, sz, si,
                                                              &tid, &kk, &rec);
                const unsigned long long m = ballot(ok);
                if (!EMIT) {
                    if (cb.wrapped && ok) shift_check(a, tid, kk, si);
                    if (lane == gi) acc += __popcll(m);
                } else if (m) {
                    const long long base = read_lane(cur, gi);
                    if (ok)
                        cell_write(a, base + lanes_below(m), si, tid, kk, rec.x, rec.y, rec.z, sx,
                                   sy, sz, cb);
                    if (lane == gi) cur += __popcll(m);
                }
            }
        }
        if (!EMIT && lane < ns) a.counts[sidx] = acc;
    }
}

// Band candidates of one source (d2 in [inner2, outer2)) in the chunks set
// in `chunks`: every candidate of such a chunk is decided in full and the
// accepted ones are ORed into lane j of the mask register mv.  Returns how
// many were added.  Rare: the band is about 1e-4 of the cutoff wide.
template <typename T, int MODE>
__device__ __forceinline__ int cell_band_fixup(const QueryArgs<T>& a, const StencilLds& st,
                                               const CellBin<T>& cb, unsigned long long& mv,
                                               unsigned chunks, T sx, T sy, T sz, int si) {
    const int lane = lane_id();
    int added = 0;
#pragma unroll 1
    for (int j = 0; j < kMaxChunks; ++j) {
        if (!((chunks >> j) & 1u)) continue;
        const int v = j * kWave + lane;
        bool ok = false;
        if (v < cb.C) {
            int tid, kk;
            Vec4<T> rec;
            ok = cell_decide<T, MODE>(a, st, cb, st.piece[v], v, sx, sy, sz, si, &tid, &kk, &rec);
            if (ok && cb.wrapped) shift_check(a, tid, kk, si);
        }
        const unsigned long long m = ballot(ok);
        const unsigned long long cur = (unsigned long long)read_lane((long long)mv, j);
        added += __popcll(m & ~cur);
        if (lane == j) mv = cur | m;
    }
    return added;
}

// XCD-grouped wave order of a grid-stride query kernel: the hardware deals
// blocks round-robin over 8 XCDs; give each XCD a contiguous range of
// logical blocks so that neighbouring bins share an L2.
__device__ __forceinline__ int64_t xcd_wave(int wv) {
    const unsigned nblk = gridDim.x;
    unsigned lb = blockIdx.x;
    if ((nblk & 7u) == 0) lb = (blockIdx.x & 7u) * (nblk >> 3) + (blockIdx.x >> 3);
    return (int64_t)lb * kWavesPerBlock + wv;
}

// Counting pass: one wave per bin of a cell-list structure (grid-stride over
// all bins).  When the flattened stencil has at most kMaxChunks chunks of 64
// candidates (the common case) their image positions and identity keys are
// gathered into registers once and the bin's sources are broadcast one at a
// time; one 64-bit hit mask per (source, chunk) is stored for the emitting
// pass, so both passes see identical pairs and the emitting pass does no
// distance tests.  Larger stencils (coarse grids) take a chunk-at-a-time
// path that recomputes the decisions in both passes.
template <typename T, int MODE>
__global__ __launch_bounds__(kBlock) void k_cell_count(QueryArgs<T> a) {
    using O = Ops<T>;
    __shared__ StencilLds s_st[kWavesPerBlock];
    __shared__ T s_tr[kWavesPerBlock][3][kPieceCap];

    const unsigned long long st0 = load_status(a.status + SS_FLAGS);
    if ((st0 & kAbortBits) || !(load_status(a.status + SS_PLAN) & 2)) return;
    const int lane = lane_id();
    const int wv = uniform(threadIdx.x / kWave);
    StencilLds& st = s_st[wv];
    T(*tr)[kPieceCap] = s_tr[wv];
    const int64_t nwaves = (int64_t)gridDim.x * kWavesPerBlock;
    const int64_t total_bins = a.struct_bin_off[a.nb];
    const T far = T(1e18);  // position of an empty candidate slot: fails every test
    const Vec4<T> zero4 = {T(0), T(0), T(0), T(0)};

    for (int64_t g = xcd_wave(wv); g < total_bins; g += nwaves) {
        CellBin<T> cb;
        if (!cell_bin<T, true>(a, g, cb, st, tr)) continue;
        const int nch = (cb.C + kWave - 1) / kWave;
        if (nch > kMaxChunks) {
            cell_slow<T, MODE, false>(a, st, cb);
            continue;
        }
        // first source group: its load overlaps the gather below
        Vec4<T> sq_next = zero4;
        if (lane < min(kSourceGroup, cb.se - cb.sb)) sq_next = a.binned[cb.sb + lane];
        // gather the candidate chunks (image positions, identity keys)
        T px[kMaxChunks], py[kMaxChunks], pz[kMaxChunks];
        unsigned key[kMaxChunks];
        int carry = 0;
#pragma unroll
        for (int j = 0; j < kMaxChunks; ++j) {
            px[j] = py[j] = pz[j] = far;
            key[j] = MODE == 0 ? ~0u : 0u;
            if (j < nch) {
                const int p = stencil_resolve(st, j, carry);
                const int v = j * kWave + lane;
                if (v < cb.C) {
                    const Vec4<T> rec = a.binned[v + st.delta[p]];
                    const int kk = st.kid[p];
                    int kx, ky, kz;
                    unpack_k(kk, kx, ky, kz);
                    key[j] = identity_key<MODE>(as_idx(rec.w), kk == pack_k(0, 0, 0),
                                                lex_negative(kx, ky, kz));
                    px[j] = O::add(rec.x, tr[0][p]);
                    py[j] = O::add(rec.y, tr[1][p]);
                    pz[j] = O::add(rec.z, tr[2][p]);
                }
            }
        }
        for (int sg = cb.sb; sg < cb.se; sg += kSourceGroup) {
            const int ns = min(kSourceGroup, cb.se - sg);
            const Vec4<T> sq = sq_next;
            const int sidx = as_idx(sq.w);
            if (sg + kSourceGroup < cb.se) {
                sq_next = zero4;
                if (lane < min(kSourceGroup, cb.se - sg - kSourceGroup))
                    sq_next = a.binned[sg + kSourceGroup + lane];
            }
            long long acc = 0;
#pragma unroll 1
            for (int gi = 0; gi < ns; ++gi) {
                const T sx = read_lane(sq.x, gi), sy = read_lane(sq.y, gi),
                        sz = read_lane(sq.z, gi);
                const int si = read_lane(sidx, gi);
                unsigned long long mv = 0;  // lane j: hit mask of chunk j
                int cnt = 0;
                unsigned band_chunks = 0;
#pragma unroll
                for (int j = 0; j < kMaxChunks; ++j) {
                    if (j >= nch) break;
                    const T dx = O::sub(px[j], sx), dy = O::sub(py[j], sy),
                            dz = O::sub(pz[j], sz);
                    const T d2 = O::fma_(dz, dz, O::fma_(dy, dy, O::mul(dx, dx)));
                    const bool keep = d2 < cb.outer2 && identity_pass<MODE>(key[j], si);
                    const bool in = d2 < cb.inner2;
                    const unsigned long long m = ballot(keep && in);
                    if (ballot(keep && !in)) band_chunks |= 1u << j;
                    if (lane == j) mv = m;
                    cnt += __popcll(m);
                    if (cb.wrapped && keep && in) {
                        const int v = j * kWave + lane;
                        const int p = st.piece[v];
                        shift_check(a, as_idx(a.binned[v + st.delta[p]].w), st.kid[p], si);
                    }
                }
                if (band_chunks)
                    cnt += cell_band_fixup<T, MODE>(a, st, cb, mv, band_chunks, sx, sy, sz, si);
                if (lane < nch) a.masks[(int64_t)(sg + gi) * kMaxChunks + lane] = mv;
                if (lane == gi) acc = cnt;
            }
            if (lane < ns) a.counts[sidx] = acc;
        }
    }
}

// Emitting pass: the same bins and stencils as the counting pass.  The hit
// masks of a group of sources are compacted into an LDS list of (source,
// candidate) entries, which the wave then writes 64 pairs at a time: every
// lane is busy and consecutive lanes write consecutive pairs of a source.
template <typename T, int MODE>
__global__ __launch_bounds__(kBlock) void k_cell_emit(QueryArgs<T> a) {
    __shared__ StencilLds s_st[kWavesPerBlock];
    __shared__ unsigned short s_list[kWavesPerBlock][kListCap];

    if (load_status(a.status + SS_FLAGS) & kAbortBits) return;
    const int lane = lane_id();
    const int wv = uniform(threadIdx.x / kWave);
    StencilLds& st = s_st[wv];
    unsigned short* list = s_list[wv];
    const int64_t nwaves = (int64_t)gridDim.x * kWavesPerBlock;
    const int64_t total_bins = a.struct_bin_off[a.nb];
    const Vec4<T> zero4 = {T(0), T(0), T(0), T(0)};

    for (int64_t g = xcd_wave(wv); g < total_bins; g += nwaves) {
        CellBin<T> cb;
        if (!cell_bin<T, false>(a, g, cb, st, nullptr)) continue;
        const int nch = (cb.C + kWave - 1) / kWave;
        if (nch > kMaxChunks) {
            cell_slow<T, MODE, true>(a, st, cb);
            continue;
        }
        // lane l < ns: source sg + l; lane l < ns * kMaxChunks: mask
        // (source sg + l / kMaxChunks, chunk l % kMaxChunks).  The first
        // group is loaded before the piece map is resolved.
        Vec4<T> sq_next = zero4;
        unsigned long long m_next = 0;
        {
            const int ns = min(kSourceGroup, cb.se - cb.sb);
            if (lane < ns) sq_next = a.binned[cb.sb + lane];
            if (lane < ns * kMaxChunks) m_next = a.masks[(int64_t)cb.sb * kMaxChunks + lane];
        }
        int carry = 0;
#pragma unroll
        for (int j = 0; j < kMaxChunks; ++j)
            if (j < nch) (void)stencil_resolve(st, j, carry);
        for (int sg = cb.sb; sg < cb.se; sg += kSourceGroup) {
            const int ns = min(kSourceGroup, cb.se - sg);
            const Vec4<T> sq = sq_next;
            const unsigned long long mreg = m_next;
            const int sidx = as_idx(sq.w);
            long long cur = 0;
            if (lane < ns) cur = a.offsets[sidx];
            if (sg + kSourceGroup < cb.se) {
                const int nn = min(kSourceGroup, cb.se - sg - kSourceGroup);
                sq_next = zero4;
                m_next = 0;
                if (lane < nn) sq_next = a.binned[sg + kSourceGroup + lane];
                if (lane < nn * kMaxChunks)
                    m_next = a.masks[(int64_t)(sg + kSourceGroup) * kMaxChunks + lane];
            }
            long long ob = 0;  // lane gi: output index of list entry 0 for source gi
            int L = 0;         // entries in the list
            auto flush = [&]() {
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
                for (int r0 = 0; r0 < L; r0 += kWave) {
                    const int r = r0 + lane;
                    const int e = r < L ? (int)list[r] : 0;
                    const int gi = e >> 9, v = e & (kMapCap - 1);
                    const T sx = __shfl(sq.x, gi), sy = __shfl(sq.y, gi), sz = __shfl(sq.z, gi);
                    const int si = __shfl(sidx, gi);
                    const long long o = __shfl(ob, gi) + r;
                    if (r < L) {
                        const int p = st.piece[v];
                        const Vec4<T> rec = a.binned[v + st.delta[p]];
                        cell_write(a, o, si, as_idx(rec.w), st.kid[p], rec.x, rec.y, rec.z, sx,
                                   sy, sz, cb);
                    }
                }
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            };
#pragma unroll 1
            for (int gi = 0; gi < ns; ++gi) {
                unsigned long long m[kMaxChunks];
                int c = 0;
#pragma unroll
                for (int j = 0; j < kMaxChunks; ++j) {
                    m[j] = j < nch ? (unsigned long long)read_lane((long long)mreg,
                                                                   gi * kMaxChunks + j)
                                   : 0ull;
                    c += __popcll(m[j]);
                }
                if (L + c > kListCap) {
                    flush();
                    L = 0;
                }
                if (lane == gi) ob = cur - L;
                int at = L;
#pragma unroll
                for (int j = 0; j < kMaxChunks; ++j) {
                    if (j >= nch) break;
                    if ((m[j] >> lane) & 1ull)
                        list[at + lanes_below(m[j])] =
                            (unsigned short)((gi << 9) | (j * kWave + lane));
                    at += __popcll(m[j]);
                }
                L = at;
            }
            flush();
        }
    }
}

}  // namespace tnr
