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
// stays below the skin (skin_valid on the host decides that from the
// reductions of k_skin_place).  The filter keeps the stored order, so a
// sorted or source-grouped list stays so.
//
// The stored list is compact: 8 bytes per pair, the target's place and the
// packed shift, in the order of the build's output, where the pairs of one
// source form one run.  Atoms are renumbered into places: the source of run
// r takes place r, atoms that start no run the places after.  The build's
// output comes in cell-list bin order when it is not sorted, so
// neighbouring sources, and their targets, sit in nearby places: the filter
// reads positions gathered into place order (one 16- or 32-byte load per
// atom, the atom index riding in the fourth lane) instead of scattered
// gathers from the input order.
//
// Every wave owns a wave tile of kSkinWaveTile consecutive stored pairs
// (item it of lane l is pair tile kSkinWaveTile + it 64 + l): a run-start
// bit marks each run's first pair and the store keeps the run of each wave
// tile's first pair, so a wave finds its pairs' runs with ballots; its kept
// pairs are counted per wave tile and written from the scan of those counts
// on.  Waves share no data: no workgroup barrier and no LDS, and the
// writing pass writes each item as soon as it is decided.
//
//   store:  k_skin_clear -> k_skin_pack (records, run starts per wave tile,
//           copies of the build's inputs) -> k_scan_lookback (runs before
//           each wave tile) -> k_skin_runs (run table, first run of each
//           wave tile, places of the sources) -> k_scan_lookback (atoms that
//           start no run) -> k_skin_ranks (their places) -> k_skin_retarget
//           (records: target atom -> target place)
//   filter: k_skin_place (positions in place order; per atom: max
//           |x - x_ref|^2 and max |x|_1; per structure: changed inputs and
//           the bound K_b; maxima per workgroup) -> k_skin_count (kept pairs per wave tile) ->
//           k_scan_lookback (their offsets, E) -> k_skin_emit (the kept
//           pairs in stored order) -> k_skin_publish (the maxima reduced,
//           status words to the host, then zeroes them and the scan tiles
//           for the next filter)
//   Tiles are indexed by the block and wave index, not by tickets:
//   same-address atomics serialise at about 12 ns each on this device, and
//   a 100,000-atom list has 28,000 wave tiles.
#pragma once

#include "nl_query.h"
#include "nl_scan.h"

namespace tnr {

constexpr int kSkinItems = 8;  // stored pairs per lane and wave tile
constexpr int64_t kSkinWaveTile = (int64_t)kWave * kSkinItems;
constexpr int64_t kSkinBlockPairs = kSkinWaveTile * kWavesPerBlock;
constexpr int kSkinShiftMin = -512, kSkinShiftMax = 511;  // 10-bit shift fields
constexpr unsigned kSkinRunStart = 1u << 30;              // in the record's high word

// Status words of the filter (a status block of its own; the first
// kHostResultSlots reach the host).  The maxima are bits of non-negative
// doubles, whose unsigned order is their numeric order.
enum SkinSlot : int {
    SK_FLAGS = 0,      // ST_SCAN_STALL / ST_OUTPUT_RANGE
    // (slots 2 to 5 are filled by k_skin_publish from the place kernel's
    // per-workgroup maxima)
    SK_PAIRS = 1,      // kept pairs E (the scan of the wave-tile counts)
    SK_MAX_DISP2 = 2,  // max over atoms of |x - x_ref|_2^2
    SK_CHANGED = 3,    // nonzero: a cell, pbc or batch_ptr entry differs from the build's
    SK_MAX_COORD = 4,  // max over atoms of |x|_1
    SK_MAX_COND = 5,   // max over structures of K_b (skin_condition)
    SK_TICKET = 6,     // tile tickets of that scan
    SK_STORE = 7,      // nonzero: the stored list cannot be filtered (SkinStoreBit)
};
static_assert((int)SK_STORE < (int)kHostResultSlots, "filter status words reach the host");

// Words that persist from the store to every filter of it.  The store's
// scans use them as their status block (a stall raises ST_SCAN_STALL in
// SP_FLAGS) and tickets.
enum SkinPersist : int { SP_FLAGS = 0, SP_RUNS = 1, SP_TICKET = 2, SP_TICKET2 = 3, SP_WORDS = 4 };
enum SkinStoreBit : unsigned long long {
    SKB_RANGE = 1,  // an atom index out of range, or a shift beyond the 10-bit fields
    SKB_RUNS = 2,   // more runs than atoms: the pairs of a source are not contiguous
};
static_assert((int)SS_FLAGS == (int)SP_FLAGS,
              "the store's scans raise their stall flag in SP_FLAGS");

// ------------------------------------------------------------ helpers

__device__ __forceinline__ unsigned skin_pack_shift(int s0, int s1, int s2) {
    return ((unsigned)s0 & 0x3ffu) | (((unsigned)s1 & 0x3ffu) << 10) |
           (((unsigned)s2 & 0x3ffu) << 20);
}

// Field c (0..2) of a packed shift, sign-extended (one bit-field extract).
__device__ __forceinline__ int skin_shift(unsigned code, int c) {
    return __builtin_amdgcn_sbfe((int)code, 10 * c, 10);
}

// Structure of atom i: the last b with bp[b] <= i, clamped to [0, nb - 1].
__device__ __forceinline__ int skin_structure(const int64_t* bp, int64_t nb, int64_t i) {
    int64_t lo = 0, hi = nb;
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) >> 1;
        if (bp[mid] <= i) lo = mid; else hi = mid;
    }
    return (int)lo;
}

// Largest non-negative double of the wave into status[slot].
__device__ __forceinline__ void skin_max(unsigned long long* status, int slot, double v) {
    const unsigned long long key = wave_max_u64((unsigned long long)__double_as_longlong(v));
    if (lane_id() == 0 && key) atomicMax(status + slot, key);
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

// ------------------------------------------------------------------ store

struct SkinStore {
    int64_t n_pairs, n_atoms, nb, n_wtiles, cap_runs;
    const int64_t* pairs;   // int64[n_pairs][2] of the build
    const int32_t* shifts;  // int32[n_pairs][3]
    const void* pos;        // the build's inputs
    const void* cell;
    const uint8_t* pbc;
    const int64_t* bp;
    unsigned long long* records;
    int2* runs;             // per run: source atom, structure
    int* wtile_run0;        // per wave tile: the run of its first pair
    long long* wtile_starts;               // per wave tile: run starts in it
    const long long* wtile_runs_before;    // their exclusive scan
    int* rank;              // per atom: its place
    int* perm;              // per place: the atom
    int* nonsrc;            // per atom: 1 when it starts no run
    const int* nonsrc_before;  // their exclusive scan
    void* ref_pos;          // copies of the build's inputs
    void* ref_cell;
    uint8_t* ref_pbc;
    int64_t* ref_bp;
    unsigned long long* persist;
};

__global__ void k_skin_clear(unsigned long long* status, unsigned long long* tiles,
                             int64_t n_tiles, unsigned long long* persist,
                             unsigned long long* tiles2, int64_t n_tiles2) {
    for (int64_t i = threadIdx.x; i < SS_SLOTS; i += blockDim.x) status[i] = 0;
    for (int64_t i = threadIdx.x; i < n_tiles; i += blockDim.x) tiles[i] = 0;
    for (int64_t i = threadIdx.x; i < n_tiles2; i += blockDim.x) tiles2[i] = 0;
    if (persist)
        for (int64_t i = threadIdx.x; i < SP_WORDS; i += blockDim.x) persist[i] = 0;
}

// Wave w of workgroup b packs the records of wave tile 4 b + w (the low word
// holds the target atom until k_skin_retarget replaces it by the target's
// place) and counts its run starts; every thread copies a grid-stride share
// of the build's inputs and marks its share of the atoms as starting no run.
template <typename T>
__global__ __launch_bounds__(kBlock) void k_skin_pack(SkinStore k) {
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    const int64_t g0 = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    for (int64_t i = g0; i < 3 * k.n_atoms; i += stride) ((T*)k.ref_pos)[i] = ((const T*)k.pos)[i];
    for (int64_t i = g0; i < k.n_atoms; i += stride) {
        k.nonsrc[i] = 1;
        k.perm[i] = 0;
    }
    for (int64_t i = g0; i < 9 * k.nb; i += stride) ((T*)k.ref_cell)[i] = ((const T*)k.cell)[i];
    for (int64_t i = g0; i < 3 * k.nb; i += stride) k.ref_pbc[i] = k.pbc[i];
    for (int64_t i = g0; i <= k.nb; i += stride) k.ref_bp[i] = k.bp[i];
    const int64_t wt = (int64_t)blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
    if (wt >= k.n_wtiles) return;
    const int lane = lane_id();
    int starts = 0;
    bool bad = false;
#pragma unroll
    for (int it = 0; it < kSkinItems; ++it) {
        const int64_t e = wt * kSkinWaveTile + it * kWave + lane;
        bool start = false;
        if (e < k.n_pairs) {
            const long2 st = *reinterpret_cast<const long2*>(k.pairs + 2 * e);
            const long long prev = e > 0 ? k.pairs[2 * e - 2] : -1;
            const int s0 = k.shifts[3 * e], s1 = k.shifts[3 * e + 1], s2 = k.shifts[3 * e + 2];
            const bool ok = st.x >= 0 && st.x < k.n_atoms && st.y >= 0 && st.y < k.n_atoms &&
                            s0 >= kSkinShiftMin && s0 <= kSkinShiftMax && s1 >= kSkinShiftMin &&
                            s1 <= kSkinShiftMax && s2 >= kSkinShiftMin && s2 <= kSkinShiftMax;
            bad |= !ok;
            start = st.x != prev;
            const unsigned hi = skin_pack_shift(s0, s1, s2) | (start ? kSkinRunStart : 0u);
            const unsigned lo = ok ? (unsigned)st.y : 0u;
            k.records[e] = (unsigned long long)lo | ((unsigned long long)hi << 32);
        }
        starts += __popcll(ballot(start));
    }
    if (ballot(bad) && lane == 0) atomicOr(k.persist + SP_FLAGS, (unsigned long long)SKB_RANGE);
    if (lane == 0) k.wtile_starts[wt] = starts;
}

// Wave w of workgroup b writes the run table entries of the runs that start
// in wave tile 4 b + w, the run of its first pair, and the places of their
// sources: the source of run r takes place r.
__global__ __launch_bounds__(kBlock) void k_skin_runs(SkinStore k) {
    const int64_t wt = (int64_t)blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
    if (wt >= k.n_wtiles) return;
    const int lane = lane_id();
    long long before = k.wtile_runs_before[wt];
    bool first = false, overflow = false;
#pragma unroll
    for (int it = 0; it < kSkinItems; ++it) {
        const int64_t e = wt * kSkinWaveTile + it * kWave + lane;
        const bool start = e < k.n_pairs && ((k.records[e] >> 32) & kSkinRunStart) != 0;
        const unsigned long long m = ballot(start);
        if (it == 0) first = (m & 1ull) != 0;
        if (start) {
            const long long run = before + lanes_below(m);
            const long long s = k.pairs[2 * e];
            if (run >= k.cap_runs || s < 0 || s >= k.n_atoms) {
                overflow = true;
            } else {
                int2 r;
                r.x = (int)s;
                r.y = k.nb == 1 ? 0 : skin_structure(k.ref_bp, k.nb, s);
                k.runs[run] = r;
                k.rank[s] = (int)run;
                k.perm[run] = (int)s;
                k.nonsrc[s] = 0;
            }
        }
        before += __popcll(m);
    }
    if (ballot(overflow) && lane == 0)
        atomicOr(k.persist + SP_FLAGS, (unsigned long long)SKB_RUNS);
    if (lane == 0)
        k.wtile_run0[wt] = (int)(k.wtile_runs_before[wt] + (first ? 1 : 0) - 1);
}

// Atoms that start no run take the places after the runs, in index order.
__global__ __launch_bounds__(kBlock) void k_skin_ranks(SkinStore k) {
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i >= k.n_atoms || !k.nonsrc[i]) return;
    const long long r = (long long)k.persist[SP_RUNS] + k.nonsrc_before[i];
    if (r >= k.n_atoms) {
        atomicOr(k.persist + SP_FLAGS, (unsigned long long)SKB_RUNS);
        return;
    }
    k.rank[i] = (int)r;
    k.perm[r] = (int)i;
}

// The records' low words: target atom -> target place.
__global__ __launch_bounds__(kBlock) void k_skin_retarget(SkinStore k) {
    const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (e >= k.n_pairs) return;
    const unsigned long long r = k.records[e];
    const int t = (int)(unsigned)r;
    k.records[e] = (r & 0xffffffff00000000ull) | (unsigned)k.rank[t];
}

// ----------------------------------------------------------------- filter

struct SkinFilter {
    int64_t n_pairs, n_atoms, nb, n_wtiles, cap_runs;
    const unsigned long long* records;
    const int2* runs;
    const int* wtile_run0;
    const int* perm;
    const void* ref_pos;
    const void* ref_cell;
    const uint8_t* ref_pbc;
    const int64_t* ref_bp;
    const int64_t* bp;   // now
    const uint8_t* pbc;  // now
    const unsigned long long* persist;
    void* placed;                    // Vec4<T>[n_atoms]: current positions by place
    long long* wtile_kept;           // count pass: kept pairs per wave tile
    const long long* wtile_offsets;  // emit pass: their exclusive scan
    double cutoff;
};

// Thread g: place g's current position (the atom index in the fourth lane;
// one 16- or 32-byte record per atom, and the targets of nearby sources sit
// close together), atom g's displacement since the build and coordinate
// magnitude (in double), and cell, pbc and batch_ptr entry g against the
// build's with structure g's shift bound.  Workgroup b writes its maxima to
// parts[b][0..3] (bits of max |x - x_ref|^2, max |x|_1, max K_b, changed);
// k_skin_publish reduces them (one atomic per workgroup or wave on shared
// words would serialise).
template <typename T>
__global__ __launch_bounds__(kBlock) void k_skin_place(SkinFilter k, const T* pos, const T* cells,
                                                       unsigned long long* parts) {
    __shared__ unsigned long long s_part[kWavesPerBlock][4];
    const int64_t g = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    double d2 = 0.0, l1 = 0.0, K = 0.0;
    bool changed = false;
    if (g < k.n_atoms) {
        int i = k.perm[g];
        i = i < 0 ? 0 : (i >= k.n_atoms ? (int)k.n_atoms - 1 : i);
        Vec4<T> v;
        v.x = pos[3 * (int64_t)i];
        v.y = pos[3 * (int64_t)i + 1];
        v.z = pos[3 * (int64_t)i + 2];
        v.w = idx_as(i, T());
        reinterpret_cast<Vec4<T>*>(k.placed)[g] = v;
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
    if (g < 9 * k.nb) changed |= !(cells[g] == ((const T*)k.ref_cell)[g]);
    if (g < 3 * k.nb) changed |= k.pbc[g] != k.ref_pbc[g];
    if (g <= k.nb) changed |= k.bp[g] != k.ref_bp[g];
    if (g < k.nb) K = skin_condition<T>(cells + 9 * g, k.pbc + 3 * g);
    const int w = threadIdx.x / kWave;
    const unsigned long long md = wave_max_u64((unsigned long long)__double_as_longlong(d2));
    const unsigned long long ml = wave_max_u64((unsigned long long)__double_as_longlong(l1));
    const unsigned long long mk = wave_max_u64((unsigned long long)__double_as_longlong(K));
    const unsigned long long mc = ballot(changed) ? 1ull : 0ull;
    if (lane_id() == 0) {
        s_part[w][0] = md;
        s_part[w][1] = ml;
        s_part[w][2] = mk;
        s_part[w][3] = mc;
    }
    __syncthreads();
    if (threadIdx.x < 4) {
        unsigned long long m = 0;
#pragma unroll
        for (int q = 0; q < kWavesPerBlock; ++q) m = max(m, s_part[q][threadIdx.x]);
        parts[4 * (int64_t)blockIdx.x + threadIdx.x] = m;
    }
}

// The cell of one structure, its rows in registers, and whether its
// off-diagonal entries are all zero (then the diagonal form of the public
// predicate applies, as in the search kernels).
template <typename T>
struct SkinCell {
    T c[9];
    bool diagonal;
};

template <typename T>
__device__ __forceinline__ SkinCell<T> skin_cell(const T* p) {
    SkinCell<T> r;
#pragma unroll
    for (int q = 0; q < 9; ++q) r.c[q] = p[q];
    r.diagonal = r.c[1] == T(0) && r.c[2] == T(0) && r.c[3] == T(0) && r.c[5] == T(0) &&
                 r.c[6] == T(0) && r.c[7] == T(0);
    return r;
}

// One stored pair at the current positions.
template <typename T>
struct SkinPair {
    int src, tgt;
    unsigned code;
    T D[3], d2;
};

// Visits the stored pairs of wave tile `wt` in order, item by item, calling
// visit(pair, keep mask of the item) in every lane (the pair's own keep bit
// is the lane's bit of the mask).  FULL: the wave tile holds kSkinWaveTile
// pairs, so no item needs a bounds check.  The records are loaded first, all
// eight at once, then the runs follow from ballots of their run-start bits;
// positions are loaded four items at a time.
template <typename T, bool FULL, typename Visit>
__device__ __forceinline__ void skin_wave(const SkinFilter& k, const QueryArgs<T>& a, int64_t wt,
                                          Visit visit) {
    const int lane = lane_id();
    const Vec4<T>* placed = reinterpret_cast<const Vec4<T>*>(k.placed);
    const unsigned long long* recs = k.records + wt * kSkinWaveTile;
    const int valid = FULL ? (int)kSkinWaveTile : (int)(k.n_pairs - wt * kSkinWaveTile);
    unsigned long long rec[kSkinItems];
#pragma unroll
    for (int it = 0; it < kSkinItems; ++it) {
        const int o = it * kWave + lane;
        rec[it] = recs[FULL ? o : min(o, valid - 1)];
    }
    const int last_run = (int)k.cap_runs - 1, last_atom = (int)k.n_atoms - 1;
    int run[kSkinItems], tp[kSkinItems];
    int run_base = k.wtile_run0[wt];  // run of the tile's first pair
#pragma unroll
    for (int it = 0; it < kSkinItems; ++it) {
        if (!FULL && it * kWave + lane >= valid) rec[it] = 0ull;
        const unsigned long long m = ballot(((unsigned)(rec[it] >> 32) & kSkinRunStart) != 0);
        // the first pair's own start is already counted in run_base
        const unsigned long long mm = it == 0 ? (m & ~1ull) : m;
        run[it] = min(max(run_base + lanes_below(mm) + (int)((mm >> lane) & 1ull), 0), last_run);
        run_base += __popcll(mm);
        tp[it] = min(max((int)(unsigned)rec[it], 0), last_atom);
    }
    const bool single = k.nb == 1;
    int sb[kSkinItems];
#pragma unroll
    for (int it = 0; it < kSkinItems; ++it)
        sb[it] = single ? 0 : min(max(k.runs[run[it]].y, 0), (int)k.nb - 1);
    const T cut2 = (T)(k.cutoff * k.cutoff);
    SkinCell<T> c1;
    if (single) c1 = skin_cell(a.cells);
    constexpr int kGroup = 4;
#pragma unroll
    for (int g0 = 0; g0 < kSkinItems; g0 += kGroup) {
        Vec4<T> vs[kGroup], vt[kGroup];
#pragma unroll
        for (int j = 0; j < kGroup; ++j) {
            vs[j] = placed[run[g0 + j]];
            vt[j] = placed[tp[g0 + j]];
        }
#pragma unroll
        for (int j = 0; j < kGroup; ++j) {
            const int it = g0 + j;
            SkinPair<T> p;
            p.code = (unsigned)(rec[it] >> 32);
            const T ps[3] = {vs[j].x, vs[j].y, vs[j].z};
            const T pt[3] = {vt[j].x, vt[j].y, vt[j].z};
            const int S0 = skin_shift(p.code, 0), S1 = skin_shift(p.code, 1),
                      S2 = skin_shift(p.code, 2);
            if (single) {
                p.d2 = c1.diagonal ? public_vector_diag(ps, pt, S0, S1, S2, c1.c, p.D)
                                   : public_vector(ps, pt, S0, S1, S2, c1.c, p.D);
            } else {
                // scalar loads when the wave's pairs share a structure
                const int b0 = __builtin_amdgcn_readfirstlane(sb[it]);
                const SkinCell<T> cl = ballot(sb[it] != b0)
                                           ? skin_cell(a.cells + 9 * (int64_t)sb[it])
                                           : skin_cell(a.cells + 9 * (int64_t)b0);
                p.d2 = cl.diagonal ? public_vector_diag(ps, pt, S0, S1, S2, cl.c, p.D)
                                   : public_vector(ps, pt, S0, S1, S2, cl.c, p.D);
            }
            const bool keep = (FULL || it * kWave + lane < valid) && p.d2 < cut2;
            p.src = as_idx(vs[j].w);
            p.tgt = as_idx(vt[j].w);
            visit(p, ballot(keep));
        }
    }
}

// Counting pass: wave w of workgroup b counts the kept pairs of wave tile
// 4 b + w into wtile_kept.
template <typename T>
__global__ __launch_bounds__(kBlock) void k_skin_count(SkinFilter k, QueryArgs<T> a) {
    const int64_t wt = (int64_t)blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
    if (wt >= k.n_wtiles || k.persist[SP_FLAGS] != 0) return;
    int kept = 0;
    auto visit = [&](const SkinPair<T>&, unsigned long long m) { kept += __popcll(m); };
    if ((wt + 1) * kSkinWaveTile <= k.n_pairs)
        skin_wave<T, true>(k, a, wt, visit);
    else
        skin_wave<T, false>(k, a, wt, visit);
    if (lane_id() == 0) k.wtile_kept[wt] = kept;
}

// Emitting pass: wave w of workgroup b writes the kept pairs of wave tile
// 4 b + w from wtile_offsets on, in stored order; rows at or beyond a.limit
// are dropped and flagged.
template <typename T>
__global__ __launch_bounds__(kBlock) void k_skin_emit(SkinFilter k, QueryArgs<T> a) {
    const int64_t wt = (int64_t)blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
    if (wt >= k.n_wtiles || k.persist[SP_FLAGS] != 0) return;
    long long next = k.wtile_offsets[wt];
    bool dropped = false;
    auto visit = [&](const SkinPair<T>& p, unsigned long long m) {
        const long long o = next + lanes_below(m);
        next += __popcll(m);
        if (!((m >> lane_id()) & 1ull)) return;
        if (o >= a.limit) {
            dropped = true;
            return;
        }
        if (a.pairs) {
            long2 v;
            v.x = p.src;
            v.y = p.tgt;
            *reinterpret_cast<long2*>(a.pairs + 2 * o) = v;
        }
        if (a.src) a.src[o] = p.src;
        if (a.dst) a.dst[o] = p.tgt;
        if (a.shifts) {
            Triple<int32_t> v;
            v.x = skin_shift(p.code, 0);
            v.y = skin_shift(p.code, 1);
            v.z = skin_shift(p.code, 2);
            *reinterpret_cast<Triple<int32_t>*>(a.shifts + 3 * o) = v;
        }
        if (a.vec) {
            Triple<T> v;
            v.x = p.D[0];
            v.y = p.D[1];
            v.z = p.D[2];
            *reinterpret_cast<Triple<T>*>(a.vec + 3 * o) = v;
        }
        if (a.dist) a.dist[o] = Ops<T>::sqrt_(p.d2);
    };
    if ((wt + 1) * kSkinWaveTile <= k.n_pairs)
        skin_wave<T, true>(k, a, wt, visit);
    else
        skin_wave<T, false>(k, a, wt, visit);
    if (ballot(dropped) && lane_id() == 0) atomicOr(a.status + SK_FLAGS, ST_OUTPUT_RANGE);
}

// After the filter: the maxima of the place kernel's `parts` (n_parts
// workgroups) into their status words, the store's flags into SK_STORE, and
// the first kHostResultSlots status words into `copy` and, when it is
// mapped, the caller's pinned buffer (otherwise the host copies `copy`
// behind this kernel).  Then the status words and scan tiles go back to zero
// for the next filter.
__global__ __launch_bounds__(kBlock) void k_skin_publish(unsigned long long* status,
                                                         const unsigned long long* persist,
                                                         const unsigned long long* parts,
                                                         int64_t n_parts, long long* host_out,
                                                         long long* copy,
                                                         unsigned long long* tiles,
                                                         int64_t n_tiles) {
    __shared__ unsigned long long s_max[kWavesPerBlock][4];
    unsigned long long m[4] = {0, 0, 0, 0};
    for (int64_t b = threadIdx.x; b < n_parts; b += blockDim.x)
#pragma unroll
        for (int q = 0; q < 4; ++q) m[q] = max(m[q], parts[4 * b + q]);
#pragma unroll
    for (int q = 0; q < 4; ++q) m[q] = wave_max_u64(m[q]);
    if (lane_id() == 0)
#pragma unroll
        for (int q = 0; q < 4; ++q) s_max[threadIdx.x / kWave][q] = m[q];
    __syncthreads();
    if (threadIdx.x < kHostResultSlots) {
        unsigned long long r[4] = {0, 0, 0, 0};
#pragma unroll
        for (int w = 0; w < kWavesPerBlock; ++w)
#pragma unroll
            for (int q = 0; q < 4; ++q) r[q] = max(r[q], s_max[w][q]);
        long long v;
        switch (threadIdx.x) {
            case SK_MAX_DISP2: v = (long long)r[0]; break;
            case SK_MAX_COORD: v = (long long)r[1]; break;
            case SK_MAX_COND: v = (long long)r[2]; break;
            case SK_CHANGED: v = (long long)r[3]; break;
            case SK_STORE: v = (long long)persist[SP_FLAGS]; break;
            default: v = (long long)status[threadIdx.x]; break;
        }
        copy[threadIdx.x] = v;
        if (host_out) host_out[threadIdx.x] = v;
    }
    __syncthreads();
    for (int64_t i = threadIdx.x; i < SS_SLOTS; i += blockDim.x) status[i] = 0;
    for (int64_t i = threadIdx.x; i < n_tiles; i += blockDim.x) tiles[i] = 0;
}

}  // namespace tnr
