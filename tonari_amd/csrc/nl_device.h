// Device-side building blocks shared by the neighbor-list kernels: wave64
// primitives, pair-identity policy, per-structure records and the workspace
// layout.  Target: gfx950 (CDNA4), wave64 only.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/tonari_hip.h"

#include <cstddef>
#include <cstdint>
#include <type_traits>

namespace tnr {

constexpr int kWave = 64;
constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int kPieceCap = 192;            // stencil pieces per source bin

// Automatic stencil reach: weight of the per-bin work (stencil build,
// staging, register gather) against the per-source distance tests.
constexpr double kBinOverhead = 6.0;
constexpr int64_t kImageCap = int64_t{1} << 24;   // geometry.cpp:12
// algorithm='auto', per structure: brute force at or below these sizes, the
// crossovers measured on gfx950 (bench.py --auto-sweep, batches of ~16k atoms
// of equal structures): periodic structures by atoms x images (brute force
// faster up to 1,296, the cell list from 1,728, in cubic and skewed cells
// alike), non-periodic ones by atoms (the molecule form of brute force is
// faster at every size it takes, up to kMoleculeCap = 2,048 atoms).
constexpr int64_t kAutoBrutePeriodic = 1500;
constexpr int64_t kAutoBruteIsolated = 2048;
// Brute force: a work unit takes about this many rounds of one image walk
// per lane, a round (64 (source, k0, target) triples) costing 1 + (images
// of one k0 plane) / 4 (most images fall outside the cutoff sphere and are
// never visited).
constexpr double kBruteUnitWork = 16.0;
constexpr int kBruteGroupCap = 256;  // sources per brute-force work unit (at most)

// Status bits.  Input errors map to ValueError, search errors to RuntimeError.
enum StatusBit : unsigned long long {
    ST_BP_START = 1ull << 0,
    ST_BP_END = 1ull << 1,
    ST_BP_ORDER = 1ull << 2,
    ST_CELL_NONFINITE = 1ull << 3,
    ST_CELL_RANK = 1ull << 4,
    ST_DUAL_RANGE = 1ull << 5,
    ST_REPEAT_RANGE = 1ull << 6,
    ST_IMAGE_CAP = 1ull << 7,
    ST_BATCH_IMAGE_CAP = 1ull << 8,
    ST_POS_NONFINITE = 1ull << 9,
    ST_WRAP_RANGE = 1ull << 10,
    ST_SHIFT_RANGE = 1ull << 11,
    ST_CELL_UNSAFE = 1ull << 12,
    ST_CAPACITY = 1ull << 13,
    ST_SCAN_STALL = 1ull << 14,
    // emitting pass: a pair index at or beyond the caller's output length
    // (outputs sized for another pair count); not an abort bit, so the pass
    // can run again on the same workspace with larger outputs
    ST_OUTPUT_RANGE = 1ull << 15,
    // a count launched with a brute-force-only plan hint (no cell-list
    // kernels) met a structure planned as a cell list: nothing of the count
    // is valid, the caller counts again without the hint
    ST_PLAN_HINT = 1ull << 16,
};
// Bits that make every later kernel skip its work (inputs are unusable).
constexpr unsigned long long kAbortBits =
    ST_BP_START | ST_BP_END | ST_BP_ORDER | ST_CELL_NONFINITE | ST_CELL_RANK | ST_DUAL_RANGE |
    ST_REPEAT_RANGE | ST_IMAGE_CAP | ST_POS_NONFINITE | ST_WRAP_RANGE | ST_CAPACITY |
    ST_PLAN_HINT;

// Slots of the status block (int64 each).
enum StatusSlot : int {
    SS_FLAGS = 0,
    SS_PAIRS = 1,
    SS_TOTAL_IMAGES = 2,
    SS_PLAN = 3,          // bit 0: some brute-force structure, bit 1: some cell-list one,
                          // bit 2: every brute-force structure is a molecule,
                          // bit 3: the periodic fast prologue applies
    SS_TOTAL_BINS = 4,
    SS_MASK_NEED = 5,     // hit-mask words per atom the count's sources wanted (maximum)
    SS_TICKET_PAIRS = 6,  // tile tickets of the pair-count scan
    SS_TOTAL_UNITS = 7,   // brute-force work units of the batch
    SS_ANY_WRAP = 8,      // some cell-list atom has a nonzero wrap: binned_w / binned_p are written
    SS_TICKET_BINS = 9,   // tile tickets of the bin-count scan
    SS_SLOTS = 64,
    kHostResultSlots = 8,  // status words copied to the caller's host buffer
};

enum Algo : int { ALGO_NONE = 0, ALGO_BRUTE = 1, ALGO_CELL = 2 };
constexpr unsigned long long kPlanFamilies = 3;   // plan bits 0-1: the kernel families
constexpr unsigned long long kPlanMolecules = 4;  // plan bit 2
// plan bit 3: one fully periodic cell-list structure whose grid the periodic
// fast prologue chooses (periodic_grid holds), a hint for the next count
constexpr unsigned long long kPlanPeriodicGrid = 8;

// The 18 per-structure reductions over atoms, all kept as maxima of
// "max-keys": kRedUlo + a / kRedUhi + a are the lower / upper bounds of the
// grid coordinate on axis a, kRedClo + c / kRedChi + c those of the wrapped
// Cartesian coordinate c, kRedP + c is max |p_c| and kRedW + a max |wrap_a|
// (per component and axis, as the reference's cell-list padding takes them).
// Lower bounds are stored complemented so that every reduction is a
// maximum and 0 is the identity.  For float inputs the keys are 32-bit
// (grid bounds rounded outward; Cartesian bounds and |p| exact); for double
// inputs they are 64-bit and exact.
enum RedSlot : int { kRedUlo = 0, kRedUhi = 3, kRedClo = 6, kRedChi = 9, kRedP = 12, kRedW = 15,
                     kRedCount = 18 };

// One record per structure.  Filled by k_setup (geometry), k_atoms
// (reductions of atoms in blocks that span several structures) and k_plan
// (margins, algorithm and bin grid).
struct alignas(16) StructRec {
    int64_t atom0;
    int64_t natoms;
    int64_t nimages;
    int64_t bin0;
    int64_t nbins;
    int64_t unit0;       // first brute-force work unit of the structure
    int64_t mask0;       // brute force: hit-mask slot of the structure's first atom
    double dual[9];      // [cartesian][axis] pseudo-inverse columns, 0 for inactive axes
    double grid[9];      // [axis][cartesian]: grid coordinate u_a = grid[a] . q
    double lo[3];        // grid origin (inactive axes)
    double inv_w[3];     // bins per grid unit
    double pad;          // broad-phase margin (length units)
    double inner2;       // broad d2 below this: inside for sure
    double outer2;       // broad d2 at or above this: outside for sure
    double cut2;         // (T)(cutoff * cutoff) as double
    unsigned long long red[kRedCount];  // max-keys of the atom reductions of shared blocks
    unsigned long long maxp;     // bits of max_c |p_c| (non-negative double), set by k_plan
    unsigned long long flags;   // input-error bits found by k_setup for this structure
    int64_t img_total;   // images this structure adds to the batch total (0 if invalid)
    uint32_t maxw;       // max_a |wrap_a| (2^31 fits)
    int32_t reps[3];     // image repeats R_a
    int32_t nb[3];       // bins per axis
    int32_t reach[3];    // stencil reach K_a in bins
    int32_t zseg;        // maximum z segments per stencil row
    int32_t active;      // bit a set: axis a periodic
    int32_t algo;
    int32_t any_wrap;
    int32_t diagonal;    // every off-diagonal cell entry is zero
    int32_t bgroup;      // brute force: sources per work unit
    int32_t bslices;     // brute force: work units per source group (slices of k0)
    int32_t bwidth;      // brute force: k0 values per slice
    int32_t mwords;      // hit-mask words per atom of the request's workspace (1-kMaskWords)
    int32_t mneed;       // brute force: hit-mask words per atom the structure wants
};

// Memo of a structure's set-up: a record with every input it depends on as
// the key (batch_ptr, the cell, pbc, atoms, cutoff, mask words, algorithm,
// reach, dtype, the structure's index and the batch size, and a tag for
// the kind of record) and a checksum over key, flag and record.  Two kinds:
//   the periodic fast prologue's record (setup_structure, then the grid of
//   periodic_grid), in entry 0: written by k_periodic_place's finishing
//   workgroup (after k_periodic_atoms has finished, before the next
//   request's starts) and read by the next request's k_periodic_atoms;
//   a batch's records (setup_structure), one entry per structure: read and
//   written by the k_setup thread of that structure.
// A record is taken from the memo when every key word and the checksum
// match, and derived otherwise.
constexpr int kMemoKey = 22;
constexpr unsigned long long kMemoPeriodic = 0x544e52504552494full;  // tags of the two kinds
constexpr unsigned long long kMemoSetup = 0x544e525345545550ull;
struct alignas(16) PeriodicMemo {
    unsigned long long key[kMemoKey];
    unsigned long long check;
    unsigned long long fast;
    StructRec rec;
};
constexpr int kMemoRecWords = (int)(sizeof(StructRec) / sizeof(unsigned long long));
constexpr int kMemoWords = kMemoKey + 1 + kMemoRecWords;  // words the checksum covers

// Per-block reduction record written by k_atoms for blocks whose atoms all
// lie in one structure (k_plan combines them without atomics); for a
// single-structure request also the block's atom error bits.
struct alignas(16) BlockPartial {
    unsigned long long red[kRedCount];
    unsigned long long flags;
};

// What the batch scan of the plans reads of a structure's record, in one
// 32-byte line per structure (records are several hundred bytes apart).
// Written by whoever plans the structure, right after its record.
struct alignas(32) PlanSummary {
    unsigned long long flags;
    long long img_total;
    long long natoms;
    long long kind;  // algo | any_wrap << 8 | molecule << 9
};

// Workspace layout.  Sub-buffers are 256-byte aligned from a 256-byte
// aligned base.  Depends only on N, B and the scalar size.
struct Layout {
    size_t status, structs, struct_bins, struct_bin_off, struct_units, struct_unit_off,
        atom_struct, atom_wrap, atom_q, binned_w, binned_p,
        atom_bin, atom_rank, bin_count, bin_start, binned, counts, offsets,
        block_partials, masks, tiles_bins, tiles_pairs, struct_meta, place, place_flags,
        place_cnt, memo, total;
    int64_t cap_bins, n_atom_blocks, n_tiles_bins, n_tiles_pairs;
};

// Hit masks stored per cell-list source: one 64-bit word per chunk of 64
// stencil candidates, in a row of `mask words` (the request's, 1 to
// kMaskWords, kMaskWords by default) per atom.  A bin whose stencil has more chunks
// than a row holds takes the slow path, which stores no masks, in both
// passes.  Brute-force structures use the same buffer, in slots counted
// down from the top: the cell-list sources of a request fill slots [0,
// cell-list atoms) by binned position, its brute-force atoms slots [n -
// brute-force atoms, n), so the two never meet.  A molecule (below) stores
// its hit masks there, one word per chunk of 64 targets; a periodic
// structure whose sources are split into k0 slices (no more than a row's
// words) stores each slice's pair count.  The counting passes report the
// largest row any source wanted (SS_MASK_NEED), so that a caller can size
// the next call's rows to it.
constexpr int kMaskWords = 64;
constexpr int kDefaultMaskWords = kMaskWords;

// Molecules: brute-force structures with no periodic axis and at most
// kMoleculeCap atoms.  They take the hit-mask form of the brute-force
// passes (molecule_unit): work units of bgroup consecutive sources, with
// bgroup x (chunks of 64 targets) at most kMolUnitWork, so that the
// emitting pass's list of one unit's hits fits its LDS.
constexpr int kMoleculeCap = 2048;
constexpr int kMolUnitWork = 28;
__host__ __device__ inline bool molecule_path(int active, int64_t natoms) {
    return active == 0 && natoms <= (int64_t)kMoleculeCap;
}
// Words of a molecule's hit-mask row (chunks of 64 targets).
__host__ __device__ inline int molecule_words(int64_t natoms) {
    return (int)((natoms + 63) / 64);
}
// A planned structure takes the molecule passes: a molecule whose row of
// hit masks fits the request's (otherwise the general brute-force passes).
__host__ __device__ inline bool molecule_rec(const StructRec& r) {
    return molecule_path(r.active, r.natoms) && molecule_words(r.natoms) <= r.mwords;
}

// Summary of one workgroup of the molecule prologue (kSetupBlock structures):
// their work units, periodic images and error bits.  A molecules-only request
// of at most kMolLocalMax structures is planned without the batch scan: the
// set-up leaves block-local unit offsets and one summary per workgroup (in the
// plan-summary area), and the molecule counting kernel, whose waves scan the
// summaries, makes the offsets global.
struct alignas(32) MoleculeBlock {
    long long units;
    unsigned long long flags;
    long long images;
    long long pad;
};
static_assert(sizeof(MoleculeBlock) == sizeof(PlanSummary), "one summary per plan-summary slot");
constexpr int64_t kMolLocalMax = 64 * 64;  // 64 workgroups of 64 structures: one wave's lanes

// k0 slices of a periodic brute-force structure, at most (each source's
// slice pair counts fill the first words of its hit-mask slot).
constexpr int kMaxSlices = 32;

// Placing kernel of the periodic fast prologue (k_periodic_place): grid
// barrier counters, one per group of workgroups (blockIdx % 8) and one for
// the groups, each alone in a 128-byte line, followed by one slice sum per
// workgroup (place); one flag per k_periodic_atoms workgroup, set when one
// of its atoms is wrapped (place_flags); and the bin counters of the
// ranking atomics, kPlaceStride ints apart (place_cnt: returning atomics on
// adjacent 4-byte counters took about three times as long on gfx950 as on
// counters 8 bytes apart, 100,000 atomics on 4,096 bins; wider spacing
// gained nothing more).  The barrier and bin counters are zeroed by
// k_periodic_atoms.  Up to kPlaceScanMax bins every workgroup scans the bin
// counts whole (one barrier); beyond, slices of the bins are summed and
// scanned (three).
constexpr int kPlaceLine = 16;
constexpr int kPlaceCounters = 9;
constexpr int kPlaceStride = 2;
constexpr unsigned kPlaceFirst = 8;  // workgroups of k_periodic_place before the placing ones
constexpr int64_t kPlaceScanMax = 8192;

constexpr int64_t kScanItems = 8;
constexpr int64_t kScanChunk = kBlock * kScanItems;
// Items per thread of the single-pass scan.
constexpr int64_t kTileItems = 8;
constexpr int64_t kScanTile = kBlock * kTileItems;

inline size_t align_up(size_t x) { return (x + 255) & ~size_t(255); }

inline Layout make_layout(int64_t n, int64_t b, size_t tsize, int mask_words) {
    Layout L{};
    L.cap_bins = 2 * n + 64 * b + 64;
    size_t o = 0;
    auto take = [&](size_t bytes) {
        const size_t at = o;
        o = align_up(o + bytes);
        return at;
    };
    L.status = take(sizeof(int64_t) * SS_SLOTS);
    L.structs = take(sizeof(StructRec) * (size_t)(b > 0 ? b : 1));
    L.struct_bins = take(sizeof(int64_t) * (size_t)(b + 1));
    L.struct_bin_off = take(sizeof(int64_t) * (size_t)(b + 2));
    L.struct_units = take(sizeof(int64_t) * (size_t)(b + 1));
    L.struct_unit_off = take(sizeof(int64_t) * (size_t)(b + 2));
    L.atom_struct = take(sizeof(int32_t) * (size_t)(n + 1));
    L.atom_wrap = take(sizeof(int32_t) * 4 * (size_t)(n + 1));
    L.atom_q = take(tsize * 4 * (size_t)(n + 1));
    L.atom_bin = take(sizeof(int32_t) * (size_t)(n + 1));
    L.atom_rank = take(sizeof(int32_t) * (size_t)(n + 1));
    L.bin_count = take(sizeof(int32_t) * (size_t)(L.cap_bins + 1));
    L.bin_start = take(sizeof(int32_t) * (size_t)(L.cap_bins + 2));
    L.binned = take(tsize * 4 * (size_t)(n + 1));
    L.binned_w = take(sizeof(int32_t) * 4 * (size_t)(n + 1));
    L.binned_p = take(tsize * 4 * (size_t)(n + 1));
    L.counts = take(sizeof(int64_t) * (size_t)(n + 1));
    L.offsets = take(sizeof(int64_t) * (size_t)(n + 2));
    L.n_atom_blocks = (n + kBlock - 1) / kBlock;
    L.block_partials = take(sizeof(BlockPartial) * (size_t)(L.n_atom_blocks + 1));
    L.masks = take(sizeof(unsigned long long) * (size_t)mask_words * (size_t)(n + 1));
    L.n_tiles_bins = (L.cap_bins + kScanTile - 1) / kScanTile + 1;
    L.n_tiles_pairs = (n + kScanTile - 1) / kScanTile + 1;
    L.tiles_bins = take(sizeof(unsigned long long) * (size_t)L.n_tiles_bins);
    L.tiles_pairs = take(sizeof(unsigned long long) * (size_t)L.n_tiles_pairs);
    L.struct_meta = take(sizeof(PlanSummary) * (size_t)(b + 1));
    // the periodic fast prologue's regions (one structure only)
    const size_t one = b == 1 ? 1 : 0;
    L.place = take(one * sizeof(unsigned long long) *
                   (size_t)(kPlaceCounters * kPlaceLine + L.n_atom_blocks + 1));
    L.place_flags = take(one * sizeof(int32_t) * (size_t)(L.n_atom_blocks + 1));
    L.place_cnt = take(one * sizeof(int32_t) * kPlaceStride * (size_t)(L.cap_bins + 1));
    L.memo = take(sizeof(PeriodicMemo) * (size_t)(b > 1 ? b : 1));
    L.total = o;
    return L;
}

// ------------------------------------------------------------ wave helpers

__device__ __forceinline__ int lane_id() { return (int)__lane_id(); }

__device__ __forceinline__ unsigned long long ballot(bool p) { return __ballot(p); }

// Number of set bits of `mask` below this lane.
__device__ __forceinline__ int lanes_below(unsigned long long mask) {
    return (int)__builtin_amdgcn_mbcnt_hi((unsigned)(mask >> 32),
                                          __builtin_amdgcn_mbcnt_lo((unsigned)mask, 0u));
}

__device__ __forceinline__ int read_lane(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ __forceinline__ float read_lane(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ double read_lane(double v, int l) {
    const long long bits = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)(bits & 0xffffffffll), l);
    const int hi = __builtin_amdgcn_readlane((int)(bits >> 32), l);
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}
__device__ __forceinline__ long long read_lane(long long v, int l) {
    const int lo = __builtin_amdgcn_readlane((int)(v & 0xffffffffll), l);
    const int hi = __builtin_amdgcn_readlane((int)(v >> 32), l);
    return ((long long)hi << 32) | (unsigned int)lo;
}

// Copy of `old` whose lane L holds the wave-uniform value `v`
// (v_writelane_b32 with an immediate lane: one VALU instruction).
template <int L>
__device__ __forceinline__ int write_lane(int old, int v) {
    int r;
    asm("v_writelane_b32 %0, %1, %2" : "=v"(r) : "s"(v), "n"(L), "0"(old));
    return r;
}

// f(std::integral_constant<int, j>) for j = 0 .. N - 1, unrolled at compile
// time (lane indices and register array indices become immediates).
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (N > 0) {
        static_for<N - 1>(f);
        f(std::integral_constant<int, N - 1>{});
    }
}

// Ordered 64-bit key of a double: key order == numeric order.
__device__ __forceinline__ unsigned long long order_key(double x) {
    const unsigned long long b = (unsigned long long)__double_as_longlong(x);
    return (b >> 63) ? ~b : (b | (1ull << 63));
}
__host__ __device__ inline double key_value(unsigned long long k) {
    const unsigned long long b = (k >> 63) ? (k & ~(1ull << 63)) : ~k;
    double x;
    __builtin_memcpy(&x, &b, sizeof(x));
    return x;
}

// ------------------------------------------------------------ pair policy
// Reference: csrc/core/pair_policy.h:42-79.  A zero-shift self pair is kept
// only with include_self; a half list keeps the lexicographically smaller of
// (s, t, S) and (t, s, -S).  When s == t the output shift equals the image
// shift, so the identity tests below take the image shift.

__device__ __forceinline__ bool lex_negative(int kx, int ky, int kz) {
    return kx < 0 || (kx == 0 && (ky < 0 || (ky == 0 && kz < 0)));
}

template <int MODE>
__device__ __forceinline__ bool keep_identity(int s, int t, int kx, int ky, int kz) {
    const bool self0 = s == t && kx == 0 && ky == 0 && kz == 0;
    if (self0) return (MODE & 1) != 0;
    if constexpr ((MODE & 2) != 0) {
        if (s != t) return s < t;
        return lex_negative(kx, ky, kz);
    }
    return true;
}

}  // namespace tnr
