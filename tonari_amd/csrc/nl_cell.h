// Cell-list query: the stencil of a bin, its pieces and exact decisions,
// shared by the counting pass (k_cell_count, nl_count.h), and the emitting
// pass (k_cell_emit: writes i/j/P/S/d/D at the scanned offsets).
//
// A bin's stencil is the neighbouring bins with their periodic images, cut
// into pieces (runs of consecutive z-bins of one (x, y) row with one image
// k) and flattened into candidates.  The emitting pass takes one source bin
// per workgroup: the four waves build the stencil once in LDS and, when it
// holds at most EmitStageCap<T> candidates, stage their records (wrapped
// position and atom index) in LDS too.  It runs no distance tests: the hit
// masks of the counting pass are decoded into an LDS list of (source,
// candidate) entries that are written 64 pairs per round, every lane busy
// and consecutive lanes writing consecutive pairs.
//
// Stencils with more chunks of 64 candidates than an atom's hit-mask row
// holds (so always those of more than kMapCap candidates) take a slow path
// that decides every candidate in both passes.
//
// Reference: the cell-list query of csrc/torch/neighbors_cell_cuda.cu:294-442
// (one warp per source walking linked lists) and csrc/core/neighbors_cpu.cpp:
// 515-584; both apply the public predicate of neighbors_cpu.cpp:247-261.
// Here a fused broad-phase distance classifies a candidate as inside
// (d2 < inner2), outside (d2 >= outer2) or in the thin band between, which
// the public predicate decides (cell_decide, cell_band).
#pragma once

#include "nl_query.h"

namespace tnr {

constexpr int kMapCap = kMaskWords * kWave;  // candidates whose piece is mapped in LDS
constexpr int kMarkWords = kMapCap / (8 * kBlock);  // 8-byte words of the piece map per thread
constexpr int kListCap = 512;                // emit: compacted hits per flush

// Stencil of the workgroup's current bin in LDS.
struct StencilLds {
    int pre[kPieceCap + 1];             // exclusive prefix of piece lengths
    int delta[kPieceCap];               // binned index = candidate index + delta
    int kid[kPieceCap];                 // packed image shift (pack_k)
    unsigned char kfl[kPieceCap];       // bit 0: k == 0, bit 1: k < 0 (lexicographic)
    unsigned char piece[kMapCap];       // piece of each candidate (when C <= kMapCap)
    int wtot[kWavesPerBlock];           // block scan: wave totals
    int wmax[kWavesPerBlock];           // block running maximum: wave maxima
};

// Candidates of a stencil staged in LDS by the emitting pass (at most); a
// multiple of kBlock.  Smaller than the counting pass's so that more
// emitting workgroups fit on a CU.
template <typename T>
struct EmitStageCap;
template <>
struct EmitStageCap<float> {
    static constexpr int value = 768;
};
template <>
struct EmitStageCap<double> {
    static constexpr int value = 1280;
};

// Image shift k packed as three signed 10-bit fields (|k_a| <= 511).
__device__ __forceinline__ int pack_k(int kx, int ky, int kz) {
    return (kx & 1023) | ((ky & 1023) << 10) | ((kz & 1023) << 20);
}
__device__ __forceinline__ void unpack_k(int v, int& kx, int& ky, int& kz) {
    kx = (int)__builtin_amdgcn_sbfe((unsigned)v, 0u, 10u);
    ky = (int)__builtin_amdgcn_sbfe((unsigned)v, 10u, 10u);
    kz = (int)__builtin_amdgcn_sbfe((unsigned)v, 20u, 10u);
}

// Candidate held by lane l of chunk j of a stencil with nch chunks: the
// chunks interleave the flattened stencil (chunk j takes candidates j,
// j + nch, j + 2 nch, ...), so every chunk samples all pieces alike and
// the hits of a source spread evenly over its mask words.  Both passes map
// mask bits to candidates through this function.
__device__ __forceinline__ int chunk_cand(int j, int l, int nch) {
    return (int)__umul24((unsigned)l, (unsigned)nch) + j;
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

// Workgroup-uniform description of one source bin of a cell-list structure;
// sb, se hold the sources of the calling wave once they are split.
template <typename T>
struct CellBin {
    int b;            // structure
    int sb, se;       // binned sources [sb, se)
    int C;            // flattened stencil candidates
    int nch;          // chunks of 64 candidates
    int npieces;
    bool by_bin;      // counts and offsets indexed by binned position (QueryArgs::by_bin)
    int dself;        // delta of the piece holding the bin itself with k = 0 (a source
                      // s at binned index b is its own candidate b - dself)
    T c[9];           // cell (rows are cell vectors)
    T outer2, inner2, cut2;
    bool wrapped, diagonal;
    bool shiftcheck;  // wrapped, and R + 2 max|wrap| may exceed int32: check kept shifts
    bool kwpack;      // wrapped, and every k - w_t packs (max_a R_a + max|wrap| <= 511)
};

// Geometry of the stencil of one bin, decoded from its structure record.
struct BinGeom {
    int ix, iy, iz;         // the bin
    int nx, ny, nz;         // bins per axis (each at least 1)
    int Kx, Kz, RY, zs;     // reach in x and z, rows per x step, z segments per row
    int R0, R1, R2;         // image repeats
    bool perx, pery, perz;
    int kz0;                // image of the lowest stencil z-bin
    int npieces;            // (2 Kx + 1) * RY * zs, at most kPieceCap
};

__device__ __forceinline__ BinGeom bin_geom(const StructRec& r, unsigned lbin) {
    BinGeom G;
    G.nx = r.nb[0];
    G.ny = r.nb[1];
    G.nz = r.nb[2];
    G.Kx = r.reach[0];
    const int Ky = r.reach[1];
    G.Kz = r.reach[2];
    G.R0 = r.reps[0];
    G.R1 = r.reps[1];
    G.R2 = r.reps[2];
    G.perx = r.active & 1;
    G.pery = r.active >> 1 & 1;
    G.perz = r.active >> 2 & 1;
    G.zs = r.zseg;
    G.iz = (int)(lbin % (unsigned)G.nz);
    const unsigned rest = lbin / (unsigned)G.nz;
    G.iy = (int)(rest % (unsigned)G.ny);
    G.ix = (int)(rest / (unsigned)G.ny);
    G.RY = 2 * Ky + 1;
    G.npieces = (2 * G.Kx + 1) * G.RY * G.zs;
    G.kz0 = 0;
    if (G.perz)
        for (int zz = G.iz - G.Kz; zz < 0; zz += G.nz) --G.kz0;
    return G;
}

// Piece p < npieces of the stencil: a run of consecutive z-bins of one (x, y)
// row with one periodic image k.  Pieces with |k_a| > R_a are dropped, which
// keeps exactly the reference's image box.  Returns whether the piece is
// kept and writes the image shift and the indices i0, i1 (relative to the
// structure's first bin) whose bin starts bound the run; dropped pieces get
// i0 = i1 = 0, so callers may load both unconditionally (every load of a
// thread in flight at once) and take len = ok ? start(i1) - start(i0) : 0.
__device__ __forceinline__ bool stencil_piece_rows(const BinGeom& G, int p, int& i0, int& i1,
                                                   int& kx, int& ky, int& kz) {
    kx = ky = kz = 0;
    // p / zs and row / RY through a float reciprocal: p < 2^8 and divisors
    // below 2^8, so (p + 1/2) / d lies at least 1/512 from an integer while
    // the float error stays below 2^-15.
    const float rzs = 1.0f / (float)G.zs, rry = 1.0f / (float)G.RY;
    const int row = (int)(((float)p + 0.5f) * rzs);
    const int seg = p - row * G.zs;
    const int rx = (int)(((float)row + 0.5f) * rry);
    int jx = G.ix + rx - G.Kx, jy = G.iy + (row - rx * G.RY) - (G.RY >> 1);
    bool ok;
    if (G.perx) {
        while (jx < 0) { jx += G.nx; --kx; }
        while (jx >= G.nx) { jx -= G.nx; ++kx; }
        ok = abs(kx) <= G.R0;
    } else {
        ok = jx >= 0 && jx < G.nx;
    }
    if (G.pery) {
        while (jy < 0) { jy += G.ny; --ky; }
        while (jy >= G.ny) { jy -= G.ny; ++ky; }
        ok = ok && abs(ky) <= G.R1;
    } else {
        ok = ok && jy >= 0 && jy < G.ny;
    }
    const int zlo = G.iz - G.Kz, zhi = G.iz + G.Kz;
    int z0, z1;
    if (G.perz) {
        kz = G.kz0 + seg;
        const int zbeg = seg == 0 ? zlo : kz * G.nz;
        const int zend = min(zhi, (kz + 1) * G.nz - 1);
        ok = ok && zbeg <= zhi && abs(kz) <= G.R2;
        z0 = zbeg - kz * G.nz;
        z1 = zend - kz * G.nz;
    } else {
        z0 = max(0, zlo);
        z1 = min(G.nz - 1, zhi);
        ok = ok && seg == 0 && z0 <= z1;
    }
    const int rowbase = (jx * G.ny + jy) * G.nz;
    i0 = ok ? rowbase + z0 : 0;
    i1 = ok ? rowbase + z1 + 1 : 0;
    return ok;
}

// Builds the stencil of global bin g with the whole workgroup (every thread
// calls it; it holds workgroup barriers), one thread per piece
// (stencil_piece_rows).  Fills the piece tables of st and, when C <= kMapCap, the piece
// of every candidate in st.piece (a workgroup running maximum of the marks
// left at every piece start).  Returns false, before any barrier, when the
// bin holds no source.  The caller separates two calls with a barrier.
template <typename T>
__device__ __forceinline__ bool block_bin(const QueryArgs<T>& a, int64_t g, StructCache& sc,
                                          CellBin<T>& cb, StencilLds& st,
                                          Vec4<T>* src_pre = nullptr) {
    const int tid = threadIdx.x;
    const int lane = lane_id();
    const int wv = tid / kWave;
    // the bin's sources load with the structure search
    const int sb_raw = a.bin_start[g], se_raw = a.bin_start[g + 1];
    cb.b = structure_of_item(a.struct_bin_off, a.nb, g, sc);
    const StructRec& r = a.recs[cb.b];
    const unsigned lbin = (unsigned)(g - r.bin0);  // bins of a structure fit in 32 bits
    const T* cell = a.cells + 9 * cb.b;
#pragma unroll
    for (int e = 0; e < 9; ++e) cb.c[e] = cell[e];
    cb.outer2 = (T)r.outer2;
    cb.inner2 = (T)r.inner2;
    cb.cut2 = (T)r.cut2;
    cb.wrapped = r.any_wrap != 0;
    // |S| = |k - w_t + w_s| <= max_a R_a + 2 max|w|: no shift of the
    // structure can leave int32 unless that bound does
    cb.shiftcheck = cb.wrapped && (double)max(max(r.reps[0], r.reps[1]), r.reps[2]) +
                                         2.0 * (double)r.maxw >= 2147483647.0;
    cb.kwpack = cb.wrapped && (double)max(max(r.reps[0], r.reps[1]), r.reps[2]) +
                                      (double)r.maxw <= 511.0;
    cb.diagonal = r.diagonal != 0;
    cb.by_bin = a.by_bin && (load_status(a.status + SS_PLAN) & kPlanFamilies) == 2ull;
    const BinGeom G = bin_geom(r, lbin);
    const int npieces = G.npieces;  // at most kPieceCap < kBlock
    cb.npieces = npieces;
    const int p = tid;
    int kx = 0, ky = 0, kz = 0, i0 = 0, i1 = 0;
    const bool pok = p < npieces && stencil_piece_rows(G, p, i0, i1, kx, ky, kz);
    const int* bstart = a.bin_start + r.bin0;
    const int start = bstart[i0];
    const int len = pok ? bstart[i1] - start : 0;
    cb.sb = uniform(sb_raw);
    cb.se = uniform(se_raw);
    if (cb.sb >= cb.se) return false;
    // clear the piece marks (the previous bin's users passed a barrier)
    static_assert(kMapCap == kMarkWords * 8 * kBlock, "kMarkWords 8-byte words of marks per thread");
#pragma unroll
    for (int k = 0; k < kMarkWords; ++k)
        reinterpret_cast<unsigned long long*>(st.piece)[kMarkWords * tid + k] = 0ull;
    // workgroup exclusive scan of the piece lengths
    const int inc = wave_inclusive_scan_i32(len);
    if (src_pre) {
        // lane l: record of the bin's source l (l < 64), in flight during the
        // rest of the stencil build (issued after the piece bounds were used)
        const Vec4<T> zero4 = {T(0), T(0), T(0), T(0)};
        *src_pre = zero4;
        if (lane < cb.se - cb.sb) *src_pre = a.binned[cb.sb + lane];
    }
    if (lane == kWave - 1) st.wtot[wv] = inc;
    __syncthreads();  // also orders the mark clearing before the marks
    int before = 0, total = 0;
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) {
        const int t = st.wtot[w];
        before += w < wv ? t : 0;
        total += t;
    }
    if (p < npieces) {
        const int ex = before + inc - len;
        const int kk = pack_k(kx, ky, kz);
        st.pre[p] = ex;
        st.delta[p] = start - ex;
        st.kid[p] = kk;
        st.kfl[p] = (unsigned char)((kx == 0 && ky == 0 && kz == 0 ? 1 : 0) |
                                    (lex_negative(kx, ky, kz) ? 2 : 0));
        if (len > 0 && ex < kMapCap) st.piece[ex] = (unsigned char)p;
    }
    if (tid == 0) st.pre[npieces] = total;
    cb.C = uniform(total);
    cb.nch = (cb.C + kWave - 1) / kWave;
    __syncthreads();
    // the bin itself with image 0: row (Kx, Ky), the z segment with kz = 0
    cb.dself = st.delta[(G.Kx * G.RY + (G.RY >> 1)) * G.zs + (G.perz ? -G.kz0 : 0)];
    if (cb.C <= kMapCap) {
        // piece of candidate v: running maximum of the marks up to v,
        // 8 kMarkWords consecutive candidates per thread
        unsigned long long w8[kMarkWords];
#pragma unroll
        for (int k = 0; k < kMarkWords; ++k)
            w8[k] = reinterpret_cast<const unsigned long long*>(st.piece)[kMarkWords * tid + k];
        int run = 0;
        int m[8 * kMarkWords];
#pragma unroll
        for (int k = 0; k < 8 * kMarkWords; ++k) {
            run = max(run, (int)((w8[k / 8] >> (8 * (k % 8))) & 0xffull));
            m[k] = run;
        }
        const int incm = wave_inclusive_max_i32(run);
        int exm = __shfl_up(incm, 1);
        if (lane == 0) exm = 0;
        if (lane == kWave - 1) st.wmax[wv] = incm;
        __syncthreads();
        int carry = exm;
#pragma unroll
        for (int w = 0; w < kWavesPerBlock; ++w)
            if (w < wv) carry = max(carry, st.wmax[w]);
#pragma unroll
        for (int k = 0; k < kMarkWords; ++k) {
            unsigned long long w = 0;
#pragma unroll
            for (int e = 0; e < 8; ++e)
                w |= (unsigned long long)max(carry, m[8 * k + e]) << (8 * e);
            reinterpret_cast<unsigned long long*>(st.piece)[kMarkWords * tid + k] = w;
        }
        __syncthreads();
    }
    return true;
}

// Copies the records of the C <= CAP candidates into LDS (every
// thread calls it; ends with a workgroup barrier).
template <typename T, int CAP>
__device__ __forceinline__ void stage_candidates(const QueryArgs<T>& a, const StencilLds& st,
                                                 int C, Vec4<T>* cand) {
    constexpr int NS = CAP / kBlock;
    const int tid = threadIdx.x;
    Vec4<T> rec[NS];
    // every load is issued before the first is needed: slots past C re-read
    // candidate 0 (C >= 1) and are not stored
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        const int v0 = tid + k * kBlock;
        const int v = v0 < C ? v0 : 0;
        rec[k] = a.binned[v + st.delta[st.piece[v]]];
    }
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        const int v = tid + k * kBlock;
        if (v < C) cand[v] = rec[k];
    }
    __syncthreads();
}

// Staged candidates of a wrapped structure: the original position, the atom
// index and the image shift k of the candidate's piece minus its wraps w_t,
// packed (pack_k).  Float64 keeps the index in the low and k - w_t in the
// high half of the fourth word; float32 keeps the index in the fourth word
// and k - w_t in an array behind WrapStageCap<float> records, inside the
// same staging area.  Taken when max_a R_a + max|w| <= 511 (every k - w_t
// packs).
template <typename T>
struct WrapStageCap;
template <>
struct WrapStageCap<float> {
    static constexpr int value = 512;
};
template <>
struct WrapStageCap<double> {
    static constexpr int value = 1280;
};
static_assert(WrapStageCap<float>::value * (16 + 4) <= EmitStageCap<float>::value * 16 &&
                  WrapStageCap<double>::value <= EmitStageCap<double>::value,
              "the wrapped staging fits the staging area");

__device__ __forceinline__ void wstage_put(Vec4<float>* cand, int v, const Vec4<float>& p,
                                           int kw) {
    cand[v] = p;
    reinterpret_cast<int*>(cand + WrapStageCap<float>::value)[v] = kw;
}
__device__ __forceinline__ void wstage_put(Vec4<double>* cand, int v, Vec4<double> p, int kw) {
    p.w = __hiloint2double(kw, as_idx(p.w));
    cand[v] = p;
}
__device__ __forceinline__ int wstage_kw(const Vec4<float>* cand, int v, const Vec4<float>&) {
    return reinterpret_cast<const int*>(cand + WrapStageCap<float>::value)[v];
}
__device__ __forceinline__ int wstage_kw(const Vec4<double>*, int, const Vec4<double>& rec) {
    return __double2hiint(rec.w);
}
__device__ __forceinline__ int wstage_idx(const Vec4<float>& rec) { return as_idx(rec.w); }
__device__ __forceinline__ int wstage_idx(const Vec4<double>& rec) {
    return __double2loint(rec.w);
}

// Stages the C <= WrapStageCap<T> candidates of a wrapped structure (every
// thread calls it; ends with a workgroup barrier): original positions (whose
// fourth word holds the atom index) and wraps in binned order.
template <typename T>
__device__ __forceinline__ void stage_wrapped(const QueryArgs<T>& a, const StencilLds& st, int C,
                                              Vec4<T>* cand) {
    constexpr int NS = WrapStageCap<T>::value / kBlock;
    static_assert(WrapStageCap<T>::value % kBlock == 0, "whole rounds");
    const int tid = threadIdx.x;
    Vec4<T> rp[NS];
    int4 rw[NS];
    int kk[NS];
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        const int v0 = tid + k * kBlock;
        const int v = v0 < C ? v0 : 0;
        const int p = st.piece[v];
        const int at = v + st.delta[p];
        kk[k] = st.kid[p];
        rp[k] = a.binned_p[at];
        rw[k] = a.binned_w[at];
    }
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        const int v = tid + k * kBlock;
        int kx, ky, kz;
        unpack_k(kk[k], kx, ky, kz);
        if (v < C) wstage_put(cand, v, rp[k], pack_k(kx - rw[k].x, ky - rw[k].y, kz - rw[k].z));
    }
    __syncthreads();
}

// Sources of the calling wave: the wv-th quarter of the bin's sources.
template <typename T>
__device__ __forceinline__ void wave_sources(CellBin<T>& cb) {
    const int wv = uniform(threadIdx.x / kWave);
    const int n = cb.se - cb.sb;
    const int q = (n + kWavesPerBlock - 1) / kWavesPerBlock;
    const int s0 = cb.sb + wv * q;
    cb.se = min(cb.se, s0 + q);
    cb.sb = s0;
}

// Record of candidate v in piece p: from LDS when staged.
template <typename T, bool STAGED>
__device__ __forceinline__ Vec4<T> cand_record(const QueryArgs<T>& a, const StencilLds& st,
                                               const Vec4<T>* cand, int p, int v) {
    if constexpr (STAGED) return cand[v];
    return a.binned[v + st.delta[p]];
}

// The band between inner2 and outer2: decided by the public predicate on the
// original positions and the output shift.
template <typename T>
__device__ __forceinline__ bool cell_band(const QueryArgs<T>& a, int tid, int kk,
                                          const Vec4<T>& rec, T sx, T sy, T sz, int si,
                                          const CellBin<T>& cb) {
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
// The candidate's record comes from `cand` (the LDS staging) when given.
// ST: any stencil table with pre, delta and kid (StencilLds, WaveStencil).
template <typename T, int MODE, typename ST>
__device__ __forceinline__ bool cell_decide(const QueryArgs<T>& a, const ST& st,
                                            const CellBin<T>& cb, int p, int v, T sx, T sy,
                                            T sz, int si, int* tid_out, int* kk_out,
                                            Vec4<T>* rec_out, const Vec4<T>* cand = nullptr) {
    using O = Ops<T>;
    const Vec4<T> rec = cand ? cand[v] : a.binned[v + st.delta[p]];
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
    if (ok && !zsf && !(d2 < cb.inner2)) ok = cell_band(a, tid, kk, rec, sx, sy, sz, si, cb);
    return ok;
}

// Piece of candidate v: the last piece whose start is at most v, by binary
// search over the piece starts.
template <typename ST>
__device__ __forceinline__ int stencil_piece(const ST& st, int v, int npieces) {
    int top = 1;
    while (top * 2 <= npieces) top *= 2;
    int p = 0;
    for (int step = top; step > 0; step >>= 1) {
        const int q = p + step;
        if (q < npieces && st.pre[q] <= v) p = q;
    }
    return p;
}

// Writes one kept candidate of source si from values in registers: the
// output shift is the image k corrected by the wraps ws, wt (zero for an
// unwrapped structure); D uses the original positions ps, pt.
template <typename T>
__device__ __forceinline__ void cell_write_regs(const QueryArgs<T>& a, long long o, int si, int tid,
                                                int kk, const T ps[3], const T pt[3],
                                                const int4& ws, const int4& wt,
                                                const CellBin<T>& cb) {
    int kx, ky, kz;
    unpack_k(kk, kx, ky, kz);
    kx = shift_i32(kx, wt.x, ws.x);
    ky = shift_i32(ky, wt.y, ws.y);
    kz = shift_i32(kz, wt.z, ws.z);
    write_hit(a, o, si, tid, kx, ky, kz, ps, pt, cb.c, cb.diagonal);
}

// Writes one kept candidate of source si: the output shift is the image k
// corrected by the representatives' wraps; D uses the original positions
// (loaded here for a wrapped structure).
template <typename T, bool WRAPPED>
__device__ __forceinline__ void cell_write(const QueryArgs<T>& a, long long o, int si, int tid,
                                           int kk, T rx, T ry, T rz, T sx, T sy, T sz,
                                           const CellBin<T>& cb) {
    int kx, ky, kz;
    unpack_k(kk, kx, ky, kz);
    T ps[3] = {sx, sy, sz}, pt[3] = {rx, ry, rz};
    if (WRAPPED) {
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

// Stencils with more than kMapCap candidates (coarse grids): one chunk at a
// time, the piece of each candidate found by binary search.
template <typename T, int MODE, bool EMIT, typename ST>
__device__ __forceinline__ void cell_slow(const QueryArgs<T>& a, const ST& st,
                                       const CellBin<T>& cb) {
    const int lane = lane_id();
    for (int sg = cb.sb; sg < cb.se; sg += kWave) {
        const int ns = min(kWave, cb.se - sg);
        Vec4<T> sq = {T(0), T(0), T(0), T(0)};
        int sidx = 0;
        if (lane < ns) {
            sq = a.binned[sg + lane];
            sidx = as_idx(sq.w);
        }
        long long acc = 0, cur = 0;
        if (EMIT && lane < ns) cur = a.offsets[cb.by_bin ? sg + lane : sidx];
        for (int j = 0; j < cb.nch; ++j) {
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
                    if (cb.shiftcheck && ok) shift_check(a, tid, kk, si);
                    if (lane == gi) acc += __popcll(m);
                } else if (m) {
                    const long long base = read_lane(cur, gi);
                    if (ok) {
                        if (cb.wrapped)
                            cell_write<T, true>(a, base + lanes_below(m), si, tid, kk, rec.x,
                                                rec.y, rec.z, sx, sy, sz, cb);
                        else
                            cell_write<T, false>(a, base + lanes_below(m), si, tid, kk, rec.x,
                                                 rec.y, rec.z, sx, sy, sz, cb);
                    }
                    if (lane == gi) cur += __popcll(m);
                }
            }
        }
        if (!EMIT && lane < ns) a.counts[cb.by_bin ? sg + lane : sidx] = acc;
    }
}

// Emitting, register path of the wave's sources: no distance tests, the hit
// masks of the counting pass are decoded.  Sources are taken S = 64 / nch at
// a time, lane (s, j) holding the mask of chunk j of source s; a wave scan of
// the mask popcounts places every hit in the wave's LDS list (entry = owner
// lane << 6 | bit), which is written out in rounds of 64 consecutive pairs.
// With STAGED the candidates come from LDS: the records (unwrapped) or the
// wrapped staging (stage_wrapped), so that a round holds no global load and
// the pair stores stream without waits (a wait for a load also waits for
// every earlier store).  With WRAPPED and not STAGED each candidate's
// original position (carrying its index) and wraps are loaded in binned
// order.
template <typename T, bool STAGED, bool WRAPPED>
__device__ __forceinline__ void emit_bin(const QueryArgs<T>& a, const StencilLds& st,
                                         const Vec4<T>* cand, const CellBin<T>& cb,
                                         unsigned short* list) {
    const int lane = lane_id();
    const Vec4<T> zero4 = {T(0), T(0), T(0), T(0)};
    const int nch = cb.nch;
    const int S = kWave / nch;
    // lane = sl * nch + j
    const int sl = (int)(((float)lane + 0.5f) / (float)nch);
    const int j = lane - sl * nch;
    for (int sg = cb.sb; sg < cb.se; sg += kWave) {
        const int ns = min(kWave, cb.se - sg);
        Vec4<T> sq = zero4;
        if (lane < ns) sq = a.binned[sg + lane];
        const int sidx = as_idx(sq.w);
        // wrapped: the sources' wraps and original positions (binned order)
        int4 sw = make_int4(0, 0, 0, 0);
        Vec4<T> sp = sq;
        if (WRAPPED && lane < ns) {
            sw = a.binned_w[sg + lane];
            sp = a.binned_p[sg + lane];
        }
        // lane gi: first output of source gi
        const long long cur = lane < ns ? a.offsets[cb.by_bin ? sg + lane : sidx] : 0;
        auto mask_of = [&](int s0_) -> unsigned long long {
            const int gi_ = s0_ + sl;
            return sl < S && gi_ < ns ? a.masks[(int64_t)(sg + gi_) * a.mask_words + j] : 0ull;
        };
        unsigned long long m_next = mask_of(0);
        for (int s0 = 0; s0 < ns; s0 += S) {
            const int gi = s0 + sl;
            const unsigned long long m = m_next;
            if (s0 + S < ns) m_next = mask_of(s0 + S);
            const int c = __popcll(m);
            const int incl = wave_inclusive_scan_i32(c);
            const int pos = incl - c;  // list position of this lane's first hit
            const int total = __builtin_amdgcn_readlane(incl, kWave - 1);
            // output of list entry r owned by this lane: cur[gi] + (pos - first) + (r - pos)
            const int first = __shfl(pos, min(sl, S - 1) * nch);
            const long long ob = __shfl(cur, min(gi, kWave - 1)) - first;
            const int tag = (min(gi, kWave - 1) << 6) | j;  // owner data: source lane, chunk
            for (int base = 0; base < total; base += kListCap) {
                const int L = min(kListCap, total - base);
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
                {
                    unsigned long long mm = m;
                    int r = pos - base;
                    while (mm) {
                        const int bit = __builtin_ctzll(mm);
                        mm &= mm - 1;
                        if (r >= 0 && r < L) list[r] = (unsigned short)((lane << 6) | bit);
                        ++r;
                    }
                }
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
                // rounds of 64 entries; the next round's record is loaded ahead.
                // The owner lookup (a lane shuffle) runs with every lane active.
                // A wrapped structure's candidates also bring their wraps and
                // original positions (binned order), loaded with the record.
                struct Entry {
                    int e, tg, kk;
                    Vec4<T> rec, rp;
                    int4 rw;
                };
                auto fetch = [&](int r) {
                    Entry x;
                    x.kk = 0;
                    x.rec = x.rp = Vec4<T>{T(0), T(0), T(0), T(0)};
                    x.rw = make_int4(0, 0, 0, 0);
                    x.e = r < L ? (int)list[r] : 0;
                    x.tg = __shfl(tag, x.e >> 6);
                    if (r < L) {
                        const int v = chunk_cand(x.tg & 63, x.e & 63, nch);
                        if (STAGED && WRAPPED) {
                            x.rp = cand[v];
                            x.kk = wstage_kw(cand, v, x.rp);
                        } else {
                            const int p = st.piece[v];
                            x.kk = st.kid[p];
                            if (WRAPPED) {
                                x.rw = a.binned_w[v + st.delta[p]];
                                x.rp = a.binned_p[v + st.delta[p]];
                            } else {
                                x.rec = cand_record<T, STAGED>(a, st, cand, p, v);
                            }
                        }
                    }
                    return x;
                };
                Entry cur = fetch(lane);
                for (int r0 = 0; r0 < L; r0 += kWave) {
                    // past the end, fetch returns zeros that no lane writes
                    const Entry nxt = fetch(r0 + kWave + lane);
                    const int g = cur.tg >> 6;
                    const long long o = __shfl(ob, cur.e >> 6) + base + r0 + lane;
                    const int si = __shfl(sidx, g);
                    if (WRAPPED) {
                        const T ps[3] = {__shfl(sp.x, g), __shfl(sp.y, g), __shfl(sp.z, g)};
                        const int4 ws = make_int4(__shfl(sw.x, g), __shfl(sw.y, g),
                                                  __shfl(sw.z, g), 0);
                        const T pt[3] = {cur.rp.x, cur.rp.y, cur.rp.z};
                        if (r0 + lane < L) {
                            if (STAGED) {
                                // kk holds k - w_t: S = kk + w_s
                                int kx, ky, kz;
                                unpack_k(cur.kk, kx, ky, kz);
                                write_hit(a, o, si, wstage_idx(cur.rp), shift_i32(kx, 0, ws.x),
                                          shift_i32(ky, 0, ws.y), shift_i32(kz, 0, ws.z), ps, pt,
                                          cb.c, cb.diagonal);
                            } else {
                                cell_write_regs<T>(a, o, si, as_idx(cur.rp.w), cur.kk, ps, pt,
                                                   ws, cur.rw, cb);
                            }
                        }
                    } else {
                        const T sx = __shfl(sq.x, g), sy = __shfl(sq.y, g), sz = __shfl(sq.z, g);
                        if (r0 + lane < L)
                            cell_write<T, false>(a, o, si, as_idx(cur.rec.w), cur.kk, cur.rec.x,
                                                 cur.rec.y, cur.rec.z, sx, sy, sz, cb);
                    }
                    cur = nxt;
                }
            }
        }
    }
}

// Sources per decode group of the emitting fast path: at most 64 / nch (one
// mask word per lane), and so many groups (a multiple of the wave count,
// dealt round-robin) that every wave of the workgroup gets an equal share
// of the bin's sources.
__device__ __forceinline__ int emit_group_size(int nsrc, int nch) {
    const int S = kWave / nch;
    const int per_pass = kWavesPerBlock * S;
    const int groups = kWavesPerBlock * ((nsrc + per_pass - 1) / per_pass);
    return (nsrc + groups - 1) / groups;
}

// Largest pair count whose every output byte offset fits in 32 bits: the
// widest requested row is P (16 bytes) or, for float64, D (24 bytes).
template <typename T>
__device__ __forceinline__ int64_t off32_limit(const QueryArgs<T>& a) {
    const int64_t widest = a.vec != nullptr && 3 * sizeof(T) > 16 ? 3 * sizeof(T) : 16;
    return (int64_t)0xffffffffll / widest;
}

// Emitting fast path: staged candidates, no wrapped representative (the
// output shift is the image shift k and positions are the records).  The
// decode of emit_bin, except that a list entry holds the source's lane in
// the group and the candidate index itself; a round reads only LDS (the
// entry, the candidate record, its piece and the piece's shift) and
// evaluates D with the public formula's operation order.  Each source's output range
// [offsets[s], offsets[s] + hits) is checked against E once; a source that
// does not fit raises ST_OUTPUT_RANGE and writes nothing.
template <typename T, bool OFF32, bool WRAPPED>
__device__ __forceinline__ void emit_fast(const QueryArgs<T>& a, const StencilLds& st,
                                          const Vec4<T>* cand,
                                          const CellBin<T>& cb, unsigned short* list,
                                          const Vec4<T>& src_all, const int4& sw_all,
                                          long long cur_all, unsigned long long m_pre0,
                                          unsigned long long m_pre1) {
    using O = Ops<T>;
    const int lane = lane_id();
    const Vec4<T> zero4 = {T(0), T(0), T(0), T(0)};
    const int nch = cb.nch;
    const int S = emit_group_size(cb.se - cb.sb, nch);
    const int sl = (int)(((float)lane + 0.5f) / (float)nch);  // lane = sl * nch + j
    const int j = lane - sl * nch;
    const bool want_d = a.dist != nullptr;
    const bool want_vec = a.vec != nullptr || want_d;
    // bits of the candidate index in a list entry
    const unsigned vb = cb.C > 1 ? 32u - (unsigned)__builtin_clz((unsigned)(cb.C - 1)) : 1u;
    const unsigned vmask = (1u << vb) - 1u;
    // groups of S sources of the bin (emit_group_size), dealt round-robin to the waves
    const int wv = uniform(threadIdx.x / kWave);
    const int nsrc = cb.se - cb.sb;  // at most kWave: sources and offsets come preloaded
    int it = 0;
    for (int s0g = wv * S; s0g < nsrc; s0g += kWavesPerBlock * S, ++it) {
        const int ns = min(S, nsrc - s0g);
        const int sg = cb.sb + s0g;
        // lane gi: the group's source gi and its first output
        const int from = min(s0g + lane, kWave - 1);
        Vec4<T> sq;
        sq.x = __shfl(src_all.x, from);
        sq.y = __shfl(src_all.y, from);
        sq.z = __shfl(src_all.z, from);
        sq.w = __shfl(src_all.w, from);
        const int sidx = as_idx(sq.w);
        int4 sw = make_int4(0, 0, 0, 0);
        if (WRAPPED) {
            sw.x = __shfl(sw_all.x, from);
            sw.y = __shfl(sw_all.y, from);
            sw.z = __shfl(sw_all.z, from);
        }
        const long long cur = __shfl(cur_all, from);
        {
            const int s0 = 0;
            const int gi = min(sl, kWave - 1);
            unsigned long long m =
                it == 0 ? m_pre0
                        : it == 1 ? m_pre1
                                  : (sl < ns ? a.masks[(int64_t)(sg + sl) * a.mask_words + j] : 0ull);
            int c = __popcll(m);
            int incl = wave_inclusive_scan_i32(c);
            // output range check of each source of the group (lane sl * nch)
            {
                const int first = __shfl(incl - c, min(sl, S - 1) * nch);
                const int last = __shfl(incl, min(sl, S - 1) * nch + nch - 1);
                const long long o0 = __shfl(cur, gi);
                const bool bad = sl < S && s0 + sl < ns &&
                                 (o0 < 0 || o0 + (last - first) > a.limit);
                if (__builtin_amdgcn_ballot_w64(bad)) {
                    if (bad) {
                        m = 0;
                        atomicOr(a.status + SS_FLAGS, ST_OUTPUT_RANGE);
                    }
                    c = __popcll(m);
                    incl = wave_inclusive_scan_i32(c);
                }
            }
            const int pos = incl - c;  // list position of this lane's first hit
            const int total = __builtin_amdgcn_readlane(incl, kWave - 1);
            const int first = __shfl(pos, min(sl, S - 1) * nch);
            // lane g: output base of the group's source g (its first output
            // minus the list position of its first hit)
            const long long ob = __shfl(__shfl(cur, gi) - first, min(lane, S - 1) * nch);
            const unsigned ob32 = (unsigned)ob;  // o = ob + list position (mod 2^32)
            // list entry: source lane g << vb | candidate v, with vb bits for
            // v < C; g < 64 / nch and C <= 64 nch keep it below 2^13
            static_assert(EmitStageCap<float>::value <= kMapCap &&
                              EmitStageCap<double>::value <= kMapCap,
                          "entries fit 16 bits");
            const unsigned ebase = ((unsigned)gi << vb) + (unsigned)j;  // + bit * nch
            for (int base = 0; base < total; base += kListCap) {
                const int L = min(kListCap, total - base);
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
                if (total <= kListCap) {
                    // every entry fits: the two mask halves, no range checks
                    unsigned lo = (unsigned)m, hi = (unsigned)(m >> 32);
                    int r = pos;
                    while (lo) {
                        const unsigned bit = __builtin_ctz(lo);
                        lo &= lo - 1;
                        list[r++] = (unsigned short)(ebase + __umul24(bit, (unsigned)nch));
                    }
                    while (hi) {
                        const unsigned bit = __builtin_ctz(hi) + 32;
                        hi &= hi - 1;
                        list[r++] = (unsigned short)(ebase + __umul24(bit, (unsigned)nch));
                    }
                } else {
                    unsigned long long mm = m;
                    int r = pos - base;
                    while (mm) {
                        const unsigned bit = __builtin_ctzll(mm);
                        mm &= mm - 1;
                        if (r >= 0 && r < L)
                            list[r] = (unsigned short)(ebase + __umul24(bit, (unsigned)nch));
                        ++r;
                    }
                }
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
                // rounds of 64 entries; the next round's LDS reads are issued ahead
                auto fetch = [&](int r, int& g_, Vec4<T>& rec_, int4& k_) {
                    const unsigned e_ = list[min(r, L - 1)];
                    g_ = (int)(e_ >> vb);
                    const int v = (int)(e_ & vmask);
                    rec_ = cand[v];
                    if (WRAPPED)
                        unpack_k(wstage_kw(cand, v, rec_), k_.x, k_.y, k_.z);  // k - w_t
                    else
                        unpack_k(st.kid[st.piece[v]], k_.x, k_.y, k_.z);
                };
                // pair r0 + lane of the list; byte offsets of output o in 32
                // bits when OFF32 (every offset below 2^32)
                auto put = [&](int r0, int g, const Vec4<T>& rec, int4 k) {
                    const T sx = __shfl(sq.x, g), sy = __shfl(sq.y, g), sz = __shfl(sq.z, g);
                    const int si = __shfl(sidx, g);
                    if (WRAPPED) {
                        // S = (k - w_t) + w_s
                        k.x = shift_i32(k.x, 0, __shfl(sw.x, g));
                        k.y = shift_i32(k.y, 0, __shfl(sw.y, g));
                        k.z = shift_i32(k.z, 0, __shfl(sw.z, g));
                    }
                    long long o;
                    if constexpr (OFF32)
                        o = (long long)(unsigned)(__shfl(ob32, g) + (unsigned)(base + r0 + lane));
                    else
                        o = __shfl(ob, g) + base + r0 + lane;
                    auto at = [&](auto* ptr, unsigned width) {
                        using P = std::remove_pointer_t<decltype(ptr)>;
                        // widths 12 and 24 by shifts (a full-rate add, not a
                        // 32-bit multiply)
                        const unsigned u = (unsigned)o;
                        const unsigned off = width == 12u   ? (u << 3) + (u << 2)
                                             : width == 24u ? (u << 4) + (u << 3)
                                                            : u * width;
                        if constexpr (OFF32)
                            return reinterpret_cast<P*>(reinterpret_cast<char*>(ptr) + (size_t)off);
                        else
                            return reinterpret_cast<P*>(reinterpret_cast<char*>(ptr) +
                                                        (size_t)o * width);
                    };
                    if (r0 + lane >= L) return;
                    const int t = WRAPPED ? wstage_idx(rec) : as_idx(rec.w);
                    if (a.pairs) {
                        long2 v;
                        v.x = (long long)(unsigned)si;
                        v.y = (long long)(unsigned)t;
                        *reinterpret_cast<long2*>(at(a.pairs, 16u)) = v;
                    }
                    if (a.src) *at(a.src, 8u) = (long long)(unsigned)si;
                    if (a.dst) *at(a.dst, 8u) = (long long)(unsigned)t;
                    if (a.shifts) {
                        Triple<int32_t> v;
                        v.x = k.x;
                        v.y = k.y;
                        v.z = k.z;
                        *reinterpret_cast<Triple<int32_t>*>(at(a.shifts, 12u)) = v;
                    }
                    if (want_vec) {
                        // D = (p_t - p_s) + S0 c0 + S1 c1 + S2 c2, rounded in T
                        // after every operation (public_vector)
                        const T f0 = (T)k.x, f1 = (T)k.y, f2 = (T)k.z;
                        T D0 = O::sub(rec.x, sx), D1 = O::sub(rec.y, sy), D2 = O::sub(rec.z, sz);
                        if (cb.diagonal) {
                            D0 = O::add(D0, O::mul(f0, cb.c[0]));
                            D1 = O::add(D1, O::mul(f1, cb.c[4]));
                            D2 = O::add(D2, O::mul(f2, cb.c[8]));
                        } else {
                            D0 = O::add(O::add(O::add(D0, O::mul(f0, cb.c[0])), O::mul(f1, cb.c[3])),
                                        O::mul(f2, cb.c[6]));
                            D1 = O::add(O::add(O::add(D1, O::mul(f0, cb.c[1])), O::mul(f1, cb.c[4])),
                                        O::mul(f2, cb.c[7]));
                            D2 = O::add(O::add(O::add(D2, O::mul(f0, cb.c[2])), O::mul(f1, cb.c[5])),
                                        O::mul(f2, cb.c[8]));
                        }
                        if (a.vec) {
                            Triple<T> v;
                            v.x = D0;
                            v.y = D1;
                            v.z = D2;
                            *reinterpret_cast<Triple<T>*>(at(a.vec, 3u * sizeof(T))) = v;
                        }
                        if (want_d) {
                            T d2 = O::mul(D0, D0);
                            d2 = O::add(d2, O::mul(D1, D1));
                            d2 = O::add(d2, O::mul(D2, D2));
                            *at(a.dist, (unsigned)sizeof(T)) = O::sqrt_(d2);
                        }
                    }
                };
                // two register sets alternate: round r + 1's LDS reads are in
                // flight while round r writes
                int gA, gB;
                Vec4<T> recA, recB;
                int4 kA, kB;
                fetch(lane, gA, recA, kA);
                for (int r0 = 0; r0 < L; r0 += 2 * kWave) {
                    fetch(r0 + kWave + lane, gB, recB, kB);
                    put(r0, gA, recA, kA);
                    if (r0 + kWave >= L) break;
                    fetch(r0 + 2 * kWave + lane, gA, recA, kA);
                    put(r0 + kWave, gB, recB, kB);
                }
            }
        }
    }
}

// XCD-aware deal of work items: workgroup b runs on XCD b % 8 (the hardware
// deals workgroups round-robin).  Items go to the XCDs in chunks of K
// consecutive items, chunk c to XCD c % 8, so the bins of one region mostly
// share an L2 while a region of heavy bins (a dense, skewed or large
// structure of a batch) spreads over every XCD instead of holding up one.
// Chunks of bins: 16 for the emitting pass (one workgroup per bin: on C5,
// 2.83 ms against 3.05 ms at 64 and 3.68 ms at 256), 64 for the counting
// pass (its waves stride over their XCD's tasks: 1.12 ms against 1.15 ms
// at 16).
constexpr int64_t kEmitChunk = 16;
constexpr int64_t kCountChunk = 64;

// Chunk length of the emitting pass for n bins: kEmitChunk, or n / 8
// rounded up for fewer than 8 kEmitChunk bins (so that a grid of
// 8 ceil(n / 8) workgroups covers them).
__device__ __host__ __forceinline__ int64_t xcd_chunk(int64_t n) {
    return n >= 8 * kEmitChunk ? kEmitChunk : (n + 7) / 8 > 0 ? (n + 7) / 8 : 1;
}
// Items of XCD x among W, in chunks of K.
__device__ __forceinline__ int64_t xcd_items(int64_t W, int64_t K, int64_t x) {
    const int64_t nc = W / K, rem = W - nc * K;
    const int64_t full = nc / 8 + (x < nc % 8 ? 1 : 0);
    return full * K + (x == nc % 8 ? rem : 0);
}
// The j-th item of XCD x, in chunks of K.
__device__ __forceinline__ int64_t xcd_item(int64_t x, int64_t j, int64_t K) {
    const int64_t c = j / K;
    return (c * 8 + x) * K + (j - c * K);
}

// The items of the calling workgroup: j = first, first + step, ... < end,
// item(j) the j-th.  A grid whose size is not a multiple of 8 strides over
// the items in order.
struct ItemRange {
    int64_t x, first, end, step, K;
    bool dealt;
    __device__ __forceinline__ int64_t item(int64_t j) const {
        return dealt ? xcd_item(x, j, K) : j;
    }
};
// W items, chunks of K (xcd_chunk of the count the grid was sized for).
__device__ __forceinline__ ItemRange xcd_block_range(int64_t W, int64_t K) {
    const unsigned nblk = gridDim.x;
    ItemRange r;
    r.K = K;
    if ((nblk & 7u) != 0) {
        r.dealt = false;
        r.x = 0;
        r.first = blockIdx.x;
        r.end = W;
        r.step = nblk;
        return r;
    }
    r.dealt = true;
    r.x = blockIdx.x & 7u;
    r.first = (int64_t)(blockIdx.x >> 3);
    r.end = xcd_items(W, K, r.x);
    r.step = (int64_t)(nblk >> 3);
    return r;
}

static_assert(kMapCap == kMaskWords * kWave, "one mask word per chunk of the piece map");

// Emitting pass for one bin with staged candidates: the fast path (at most
// 64 sources) or the decode path.  WRAPPED: the wrapped staging
// (stage_wrapped), and the sources' original positions and wraps.
template <typename T, bool WRAPPED>
__device__ __forceinline__ void emit_staged(const QueryArgs<T>& a, StencilLds& s_st,
                                            Vec4<T>* s_cand, unsigned short* list,
                                            CellBin<T>& cb, Vec4<T> src_all, int wv, int lane) {
    const int nsrc = cb.se - cb.sb;
    // the wrapped fast path needs six more VGPRs than the kernel's other
    // paths: float32 (seven workgroups per CU, at most 72 VGPRs) leaves it
    // to the decode path
    const bool fast = nsrc <= kWave && (!WRAPPED || sizeof(T) == 8);
    long long cur_all = 0;
    unsigned long long m0 = 0, m1 = 0;
    int4 sw_all = make_int4(0, 0, 0, 0);
    if (fast) {
        // sources, offsets and the masks of the wave's first two groups load
        // with the staging
        if (WRAPPED && lane < nsrc) {
            src_all = a.binned_p[cb.sb + lane];
            sw_all = a.binned_w[cb.sb + lane];
        }
        cur_all = lane < nsrc ? a.offsets[cb.by_bin ? cb.sb + lane : as_idx(src_all.w)] : 0;
        const int S = emit_group_size(nsrc, cb.nch);
        const int sl = (int)(((float)lane + 0.5f) / (float)cb.nch);
        const int j = lane - sl * cb.nch;
        const int s0 = wv * S + sl, s1 = (wv + kWavesPerBlock) * S + sl;
        if (sl < S && s0 < min(nsrc, wv * S + S))
            m0 = a.masks[(int64_t)(cb.sb + s0) * a.mask_words + j];
        if (sl < S && s1 < min(nsrc, (wv + kWavesPerBlock) * S + S))
            m1 = a.masks[(int64_t)(cb.sb + s1) * a.mask_words + j];
    }
    if (WRAPPED)
        stage_wrapped<T>(a, s_st, cb.C, s_cand);
    else
        stage_candidates<T, EmitStageCap<T>::value>(a, s_st, cb.C, s_cand);
    if (fast) {
        // every output's byte offset below 2^32: 32-bit offsets
        if (a.limit <= off32_limit(a))
            emit_fast<T, true, WRAPPED>(a, s_st, s_cand, cb, list, src_all, sw_all, cur_all, m0,
                                        m1);
        else
            emit_fast<T, false, WRAPPED>(a, s_st, s_cand, cb, list, src_all, sw_all, cur_all,
                                         m0, m1);
    } else {
        wave_sources(cb);
        emit_bin<T, true, WRAPPED>(a, s_st, s_cand, cb, list);
    }
}

// Emitting pass for one bin whose stencil block_bin has built: staged
// candidates (emit_staged), the decode path with candidates loaded from
// global memory (emit_bin) or, beyond the hit-mask row, the slow path.
template <typename T, int MODE>
__device__ __forceinline__ void emit_one_bin(const QueryArgs<T>& a, StencilLds& s_st,
                                             Vec4<T>* s_cand, unsigned short* list,
                                             CellBin<T>& cb, const Vec4<T>& src_all, int wv,
                                             int lane) {
    // the count stored hit masks for this bin when its row held them
    if (cb.nch > a.mask_words) {
        wave_sources(cb);
        cell_slow<T, MODE, true>(a, s_st, cb);
    } else if (!cb.wrapped && cb.C <= EmitStageCap<T>::value) {
        emit_staged<T, false>(a, s_st, s_cand, list, cb, src_all, wv, lane);
    } else if (cb.kwpack && cb.C <= WrapStageCap<T>::value) {
        emit_staged<T, true>(a, s_st, s_cand, list, cb, src_all, wv, lane);
    } else {
        wave_sources(cb);
        if (cb.wrapped)
            emit_bin<T, false, true>(a, s_st, s_cand, cb, list);
        else
            emit_bin<T, false, false>(a, s_st, s_cand, cb, list);
    }
}

// Emitting pass: one workgroup per bin, dealt to the XCDs in chunks of bins
// (xcd_block_range).  The grid is sized
// for out->n_tasks bins; the kernel reads the batch's bin count from the
// status words and only trusts the smaller of the two, and it can run again
// on the same workspace.  STRIDED: the workgroups of a grid of any size
// stride over the bins, for a launch that does not know the bin count.
template <typename T, int MODE, bool STRIDED = false>
__global__ __launch_bounds__(kBlock) void k_cell_emit(
    QueryArgs<T> a) {
    __shared__ StencilLds s_st;
    __shared__ Vec4<T> s_cand[EmitStageCap<T>::value];
    __shared__ unsigned short s_list[kWavesPerBlock][kListCap];

    if (load_status(a.status + SS_FLAGS) & kAbortBits) return;
    place_edge_index(a);
    // the batch's bins from the count's status words; the grid may cover
    // more (a launch sized before the count finished)
    const int64_t bins = (int64_t)load_status(a.status + SS_TOTAL_BINS);
    const ItemRange br = xcd_block_range(min(a.n_bins, bins), xcd_chunk(a.n_bins));
    StructCache sc{0, 0, 0};
    const int wv = uniform(threadIdx.x / kWave);
    const int lane = lane_id();
    if constexpr (!STRIDED) {
        // one bin per workgroup (the grid covers the bins)
        if (br.first >= br.end) return;
        const int64_t g = br.item(br.first);
        CellBin<T> cb;
        Vec4<T> src_all;
        if (block_bin<T>(a, g, sc, cb, s_st, &src_all))
            emit_one_bin<T, MODE>(a, s_st, s_cand, s_list[wv], cb, src_all, wv, lane);
    } else {
        // a grid of any size strides over the bins (a launch that does not
        // know the bin count)
        for (int64_t j = br.first; j < br.end; j += br.step) {
            const int64_t g = br.item(j);
            CellBin<T> cb;
            Vec4<T> src_all;
            if (block_bin<T>(a, g, sc, cb, s_st, &src_all))
                emit_one_bin<T, MODE>(a, s_st, s_cand, s_list[wv], cb, src_all, wv, lane);
            __syncthreads();  // the bin's LDS is free
        }
    }
}

}  // namespace tnr
