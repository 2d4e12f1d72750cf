// Verlet-skin lists: a list searched at a larger cutoff (cutoff + skin),
// filtered to the cutoff at the current positions.  No counterpart in the
// reference, which lists a Verlet skin as unsupported
// (docs/design.md:125-127).
//
// A pair (i, j, S) of the reference's list is identified by its atoms and
// its output shift; its displacement D = x_j - x_i + S cell depends on the
// atoms' positions as given, not on their wraps.  While the cells, pbc and
// batch_ptr equal those of the build and every atom has moved by at most m
// since, a pair within the cutoff now was within cutoff + 2m then, so
// filtering the stored list with the reference's public predicate
// (neighbors_cpu.cpp:247-261) at the current positions gives the
// reference's list for those positions, provided 2m plus a rounding margin
// stays below the skin (tnr_skin_finish decides that from the reductions
// below).  The filter keeps the stored order, so a sorted or source-grouped
// list stays so.
//
//   k_skin_clear   zeroes the filter's status words and scan tiles
//   k_skin_count   per atom: max |x - x_ref|^2 and max |x|_1; per structure:
//                  whether cell / pbc / batch_ptr changed, and the bound K_b
//                  on the shift terms; per stored pair: the keep decision,
//                  kept pairs per workgroup
//   (k_scan_lookback over the workgroup counts: offsets, E, status words
//   to the host)
//   k_skin_emit    writes the kept pairs from their workgroup's offset on,
//                  in stored order
#pragma once

#include "nl_query.h"
#include "nl_scan.h"

namespace tnr {

// Status words of the filter (a status block of its own, kHostResultSlots
// of which reach the host).  The maxima are bits of non-negative doubles,
// whose unsigned order is their numeric order.
enum SkinSlot : int {
    SK_FLAGS = 0,      // ST_SCAN_STALL / ST_OUTPUT_RANGE
    SK_PAIRS = 1,      // kept pairs E (SS_PAIRS, read by place_edge_index)
    SK_MAX_DISP2 = 2,  // max over atoms of |x - x_ref|_2^2
    SK_CHANGED = 3,    // nonzero: a cell, pbc or batch_ptr entry differs from the build's
    SK_MAX_COORD = 4,  // max over atoms of |x|_1
    SK_MAX_COND = 5,   // max over structures of K_b (skin_condition)
    SK_TICKET = 6,     // tile tickets of the scan
};
static_assert(SK_PAIRS == SS_PAIRS, "place_edge_index reads E from SS_PAIRS");
static_assert(SK_TICKET < kHostResultSlots, "filter status words reach the host");

struct SkinArgs {
    int64_t n_pairs;  // stored pairs
    int64_t n_atoms;
    int64_t nb;
    const int64_t* pairs;   // int64[n_pairs][2]
    const int32_t* shifts;  // int32[n_pairs][3]
    const int64_t* bp;      // batch_ptr now
    const uint8_t* pbc;
    const void* ref_pos;    // build-time inputs
    const void* ref_cell;
    const uint8_t* ref_pbc;
    const int64_t* ref_bp;
    double cutoff;          // filter cutoff
};

// Structure of atom i: the last b with bp[b] <= i, clamped to [0, nb - 1]
// (in bounds for any batch_ptr; a batch_ptr that differs from the build's
// forces a rebuild, which discards the filter's results).
__device__ __forceinline__ int skin_structure(const int64_t* bp, int64_t nb, int64_t i) {
    int64_t lo = 0, hi = nb;
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) >> 1;
        if (bp[mid] <= i) lo = mid; else hi = mid;
    }
    return (int)lo;
}

// Bound K_b on the shift terms of structure b: for any shift S of its
// periodic axes P, sum_k |S_k| |c_k|_1 <= |S cell|_2 K_b.  With G the Gram
// matrix of the periodic rows, S_k = (S cell) . b_k for the dual rows b_k,
// |b_k|_2^2 = (G^-1)_kk, so K_b = sum_{k in P} sqrt((G^-1)_kk) |c_k|_1,
// inflated by 1% for the rounding of the inverse.  A singular or non-finite
// cell gives infinity (the caller then rebuilds, and the rebuild reports the
// cell).
struct SkinRow {
    double x, y, z, l1;
};

__device__ __forceinline__ double skin_dot(const SkinRow& a, const SkinRow& b) {
    return a.x * b.x + a.y * b.y + a.z * b.z;
}

template <typename T>
__device__ double skin_condition(const T* cell, const uint8_t* pbc) {
    // the periodic rows, in axis order, in r0 .. r(p-1)
    SkinRow r0{}, r1{}, r2{};
    int p = 0;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        if (!pbc[k]) continue;
        SkinRow r;
        r.x = (double)cell[3 * k];
        r.y = (double)cell[3 * k + 1];
        r.z = (double)cell[3 * k + 2];
        r.l1 = fabs(r.x) + fabs(r.y) + fabs(r.z);
        if (p == 0) r0 = r; else if (p == 1) r1 = r; else r2 = r;
        ++p;
    }
    double K;
    if (p == 0) {
        return 0.0;
    } else if (p == 1) {
        const double g = skin_dot(r0, r0);
        if (!(g > 0.0)) return INFINITY;
        K = r0.l1 / sqrt(g);
    } else if (p == 2) {
        const double g00 = skin_dot(r0, r0), g11 = skin_dot(r1, r1), g01 = skin_dot(r0, r1);
        const double det = g00 * g11 - g01 * g01;
        if (!(det > 0.0)) return INFINITY;
        K = sqrt(g11 / det) * r0.l1 + sqrt(g00 / det) * r1.l1;
    } else {
        const double g00 = skin_dot(r0, r0), g11 = skin_dot(r1, r1), g22 = skin_dot(r2, r2);
        const double g01 = skin_dot(r0, r1), g02 = skin_dot(r0, r2), g12 = skin_dot(r1, r2);
        const double m00 = g11 * g22 - g12 * g12;
        const double m11 = g00 * g22 - g02 * g02;
        const double m22 = g00 * g11 - g01 * g01;
        const double det = g00 * m00 - g01 * (g01 * g22 - g12 * g02) + g02 * (g01 * g12 - g11 * g02);
        if (!(det > 0.0) || !(m00 > 0.0) || !(m11 > 0.0) || !(m22 > 0.0)) return INFINITY;
        K = sqrt(m00 / det) * r0.l1 + sqrt(m11 / det) * r1.l1 + sqrt(m22 / det) * r2.l1;
    }
    K *= 1.01;
    return K == K ? K : INFINITY;
}

// Stored pair e at the current positions: its atoms, shift and the public
// predicate's D and d^2; true when d^2 is below the filter cutoff's square,
// rounded to T as the search rounds it.
template <typename T>
__device__ __forceinline__ bool skin_keep(const SkinArgs& k, const T* pos, const T* cells,
                                         int64_t e, int64_t& s, int64_t& t, int S[3], T D[3],
                                         T& d2) {
    const long2 st = *reinterpret_cast<const long2*>(k.pairs + 2 * e);
    s = st.x;
    t = st.y;
    S[0] = k.shifts[3 * e];
    S[1] = k.shifts[3 * e + 1];
    S[2] = k.shifts[3 * e + 2];
    const int b = k.nb == 1 ? 0 : skin_structure(k.bp, k.nb, s);
    const T ps[3] = {pos[3 * s], pos[3 * s + 1], pos[3 * s + 2]};
    const T pt[3] = {pos[3 * t], pos[3 * t + 1], pos[3 * t + 2]};
    d2 = public_vector(ps, pt, S[0], S[1], S[2], cells + 9 * b, D);
    return d2 < (T)(k.cutoff * k.cutoff);
}

// Largest non-negative double of the wave into status[slot].
__device__ __forceinline__ void skin_max(unsigned long long* status, int slot, double v) {
    const unsigned long long key = wave_max_u64((unsigned long long)__double_as_longlong(v));
    if (lane_id() == 0 && key) atomicMax(status + slot, key);
}

__global__ void k_skin_clear(unsigned long long* status, unsigned long long* tiles,
                             int64_t n_tiles) {
    for (int64_t i = threadIdx.x; i < SS_SLOTS; i += blockDim.x) status[i] = 0;
    for (int64_t i = threadIdx.x; i < n_tiles; i += blockDim.x) tiles[i] = 0;
}

// Thread g of the grid takes atom g, structure g (and cell entry g, pbc
// entry g, batch_ptr entry g) and stored pair g; workgroup w writes its kept
// pairs to counts[w].
template <typename T>
__global__ __launch_bounds__(kBlock) void k_skin_count(SkinArgs k, const T* pos, const T* cells,
                                                       long long* counts,
                                                       unsigned long long* status) {
    __shared__ int s_kept[kWavesPerBlock];
    const int64_t g = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    const int64_t wave0 = g - lane_id();
    const int wv = threadIdx.x / kWave;
    if (wave0 < k.n_atoms) {
        double d2 = 0.0, l1 = 0.0;
        if (g < k.n_atoms) {
            const T* ref = (const T*)k.ref_pos;
#pragma unroll
            for (int c = 0; c < 3; ++c) {
                const double x = (double)pos[3 * g + c];
                const double dx = x - (double)ref[3 * g + c];
                d2 += dx * dx;
                l1 += fabs(x);
            }
            if (!(d2 == d2)) d2 = INFINITY;
            if (!(l1 == l1)) l1 = INFINITY;
        }
        skin_max(status, SK_MAX_DISP2, d2);
        skin_max(status, SK_MAX_COORD, l1);
    }
    if (wave0 < 9 * k.nb + 1) {
        bool changed = false;
        if (g < 9 * k.nb) changed |= !(cells[g] == ((const T*)k.ref_cell)[g]);
        if (g < 3 * k.nb) changed |= k.pbc[g] != k.ref_pbc[g];
        if (g <= k.nb) changed |= k.bp[g] != k.ref_bp[g];
        if (ballot(changed) && lane_id() == 0) atomicOr(status + SK_CHANGED, 1ull);
        double K = 0.0;
        if (g < k.nb) K = skin_condition<T>(cells + 9 * g, k.pbc + 3 * g);
        skin_max(status, SK_MAX_COND, K);
    }
    bool keep = false;
    if (g < k.n_pairs) {
        int64_t s, t;
        int S[3];
        T D[3], d2;
        keep = skin_keep<T>(k, pos, cells, g, s, t, S, D, d2);
    }
    const int kept = __popcll(ballot(keep));  // every lane takes part in the ballot
    if (lane_id() == 0) s_kept[wv] = kept;
    __syncthreads();
    if (threadIdx.x == 0) {
        long long total = 0;
#pragma unroll
        for (int w = 0; w < kWavesPerBlock; ++w) total += s_kept[w];
        counts[blockIdx.x] = total;
    }
}

// Workgroup w writes the kept pairs among stored pairs [w kBlock, (w + 1)
// kBlock) from offsets[w] on, in stored order.
template <typename T>
__global__ __launch_bounds__(kBlock) void k_skin_emit(SkinArgs k, QueryArgs<T> a,
                                                      const long long* offsets) {
    __shared__ int s_kept[kWavesPerBlock];
    place_edge_index(a);
    const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    const int wv = threadIdx.x / kWave;
    int64_t s = 0, t = 0;
    int S[3] = {0, 0, 0};
    T D[3] = {T(0), T(0), T(0)}, d2 = T(0);
    const bool keep = e < k.n_pairs && skin_keep<T>(k, a.pos, a.cells, e, s, t, S, D, d2);
    const unsigned long long m = ballot(keep);
    if (lane_id() == 0) s_kept[wv] = __popcll(m);
    __syncthreads();
    long long o = offsets[blockIdx.x] + lanes_below(m);
    for (int w = 0; w < wv; ++w) o += s_kept[w];
    if (!keep) return;
    if (o >= a.limit) {
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
        v.x = S[0];
        v.y = S[1];
        v.z = S[2];
        *reinterpret_cast<Triple<int32_t>*>(a.shifts + 3 * o) = v;
    }
    if (a.vec) {
        Triple<T> v;
        v.x = D[0];
        v.y = D[1];
        v.z = D[2];
        *reinterpret_cast<Triple<T>*>(a.vec + 3 * o) = v;
    }
    if (a.dist) a.dist[o] = Ops<T>::sqrt_(d2);
}

}  // namespace tnr
