// MI355X (gfx950) neighbor-list library: host orchestration and the C ABI
// declared in include/tonari_hip.h.  Kernels live in nl_prologue.h (device
// geometry, wraps, bin grid, counting sort), nl_query.h (cell-list and
// brute-force count/emit), nl_scan.h (device-wide scans), nl_skin.h (the
// Verlet-skin filter) and nl_backward.h (the geometry backward).
//
// Pipeline of one request (all on the caller's stream):
//   tnr_count, one structure: k_atoms<T, true> (every block derives the
//              structure's periodic metadata in LDS; per atom: wraps, wrapped
//              position, block reductions; zeroes the bin counters and scan
//              tiles) -> k_single_bin (plan: margins, algorithm, bin grid,
//              status words; then binning);
//   tnr_count, one fully periodic structure with the plan hint of an
//              earlier count: k_periodic_atoms (grid from the cell and
//              cutoff; per atom also its bin) -> k_periodic_place (the
//              plan finished from the atom reductions; beside it the bin
//              atomics, a grid barrier, bin starts and binned atoms);
//   tnr_count, a batch: k_setup (zeroes the status words; per structure:
//              batch_ptr checks, active pseudo-inverse, image repeats, grid
//              frame) -> k_atoms<T, false> -> k_plan (one workgroup per
//              structure: margins, algorithm, bin grid or brute-force work
//              units) -> k_struct_scan (their scans over the batch, batch
//              status) -> k_bin;
//   then       k_scan_lookback (bin counts -> bin starts) -> k_scatter
//              (binned atoms) -> k_cell_count and/or k_brute<count> ->
//              k_scan_lookback (pairs per source -> offsets and E; its last
//              block copies the status words into the caller's pinned host
//              buffer).
//   tnr_emit:  k_cell_emit and/or k_brute<emit> write i/j/P/S/d/D in place.
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

#include "nl_count.h"
#include "nl_prologue.h"
#include "nl_query.h"
#include "nl_scan.h"
#include "nl_backward.h"
#include "nl_skin.h"

#include "../../include/tonari_hip.h"

#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <mutex>

namespace tnr {

static_assert(kHostResultSlots == TNR_HOST_RESULT_SLOTS, "host result slots");


// ------------------------------------------------------------------- host

struct Views {
    unsigned long long* status;
    StructRec* recs;
    long long* struct_bins;
    long long* struct_bin_off;
    long long* struct_units;
    long long* struct_unit_off;
    int* atom_struct;
    int4* atom_wrap;
    void* atom_q;
    int* atom_bin;
    int* atom_rank;
    int* bin_count;
    int* bin_start;
    void* binned;
    int4* binned_w;
    void* binned_p;
    long long* counts;
    long long* offsets;
    BlockPartial* block_partials;
    unsigned long long* masks;
    unsigned long long* tiles_bins;
    unsigned long long* tiles_pairs;
    PlanSummary* struct_meta;
    unsigned long long* place;
    int* place_flags;
    int* place_cnt;
    PeriodicMemo* memo;
};

static Views views(void* ws, const Layout& L) {
    char* base = (char*)ws;
    Views v;
    v.status = (unsigned long long*)(base + L.status);
    v.recs = (StructRec*)(base + L.structs);
    v.struct_bins = (long long*)(base + L.struct_bins);
    v.struct_bin_off = (long long*)(base + L.struct_bin_off);
    v.struct_units = (long long*)(base + L.struct_units);
    v.struct_unit_off = (long long*)(base + L.struct_unit_off);
    v.atom_struct = (int*)(base + L.atom_struct);
    v.atom_wrap = (int4*)(base + L.atom_wrap);
    v.atom_q = base + L.atom_q;
    v.atom_bin = (int*)(base + L.atom_bin);
    v.atom_rank = (int*)(base + L.atom_rank);
    v.bin_count = (int*)(base + L.bin_count);
    v.bin_start = (int*)(base + L.bin_start);
    v.binned = base + L.binned;
    v.binned_w = (int4*)(base + L.binned_w);
    v.binned_p = base + L.binned_p;
    v.counts = (long long*)(base + L.counts);
    v.offsets = (long long*)(base + L.offsets);
    v.block_partials = (BlockPartial*)(base + L.block_partials);
    v.masks = (unsigned long long*)(base + L.masks);
    v.tiles_bins = (unsigned long long*)(base + L.tiles_bins);
    v.tiles_pairs = (unsigned long long*)(base + L.tiles_pairs);
    v.struct_meta = (PlanSummary*)(base + L.struct_meta);
    v.place = (unsigned long long*)(base + L.place);
    v.place_flags = (int*)(base + L.place_flags);
    v.place_cnt = (int*)(base + L.place_cnt);
    v.memo = (PeriodicMemo*)(base + L.memo);
    return v;
}

static unsigned blocks_for(int64_t n, int per = kBlock) {
    const int64_t b = (n + per - 1) / per;
    return (unsigned)(b > 0 ? b : 1);
}

// Workgroups a kernel keeps resident on the whole device (occupancy x
// CUs).  Looked up once per device and kernel (one cache per template
// argument, that is per kernel) and cached: the only state the library
// keeps; it is idempotent and safe under concurrent use.
template <auto Kernel>
static int64_t resident_blocks() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    int v = cache[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, Kernel, kBlock, 0) != hipSuccess ||
        per_cu <= 0)
        per_cu = 2;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
        cus = 256;
    v = per_cu * cus;
    cache[dev].store(v, std::memory_order_relaxed);
    return v;
}

// Bound of k_periodic_place's barrier waits, in ticks of the device's
// constant-rate clock: TNR_PLACE_WAIT_US microseconds (read on every call;
// default 20,000).  The wait only runs out when the placing workgroups cannot
// all be resident (other kernels holding the device), and then the request
// is counted again without the periodic plan hint; the variable lets a test
// force that path.
static long long barrier_ticks() {
    static std::atomic<int> rate_khz[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    int r = rate_khz[dev].load(std::memory_order_relaxed);
    if (r <= 0) {
        if (hipDeviceGetAttribute(&r, hipDeviceAttributeWallClockRate, dev) != hipSuccess ||
            r <= 0)
            r = 100000;
        rate_khz[dev].store(r, std::memory_order_relaxed);
    }
    long long us = 20000;
    if (const char* e = std::getenv("TNR_PLACE_WAIT_US")) {
        char* end = nullptr;
        const long long x = std::strtoll(e, &end, 10);
        if (end != e && x >= 0 && x <= 60000000) us = x;
    }
    return us * (long long)r / 1000;
}

// Blocks of the persistent counting kernel: as many as the device holds at
// once, rounded down to a multiple of 8 so that every XCD gets the same
// number, and no more than the work needs.
template <typename T, int MODE>
static unsigned count_blocks(int64_t work_waves) {
    const int64_t want = (work_waves + kWavesPerBlock - 1) / kWavesPerBlock;
    const int64_t cap = resident_blocks<k_cell_count<T, MODE>>() / 8 * 8;
    int64_t b = want < cap ? want : cap;
    b = (b + 7) / 8 * 8;
    return (unsigned)(b > 0 ? b : 8);
}

// Workgroups of the emitting cell-list kernel: one per bin, the bins dealt
// to the XCDs in chunks of K = xcd_chunk(bins) (every XCD gets the same
// number of workgroups, enough for its share of whole chunks).
static unsigned emit_blocks(int64_t bins) {
    const int64_t K = xcd_chunk(bins);
    const int64_t b = 8 * K * ((bins + 8 * K - 1) / (8 * K));
    return (unsigned)(b > 0 ? b : 8);
}

// Workgroups of the brute-force kernels (K: k_brute or k_molecules): one
// wave per work unit (a batch has at most one unit per atom), no more than
// the device holds at once (the waves stride over the units; surplus
// workgroups would only cost dispatch).
template <auto K>
static unsigned unit_blocks(int64_t n) {
    const int64_t want = (n + kWavesPerBlock - 1) / kWavesPerBlock;
    const int64_t cap = resident_blocks<K>();
    const int64_t b = want < cap ? want : cap;
    return (unsigned)(b > 0 ? b : 1);
}
template <typename T, int MODE, bool EMIT>
static unsigned brute_blocks(int64_t n) {
    return unit_blocks<k_brute<T, MODE, EMIT>>(n);
}

// The brute-force pass of a request: k_molecules when every brute-force
// structure is known to be a molecule, else k_brute.
template <typename T, int MODE, bool EMIT>
static void launch_brute(const QueryArgs<T>& q, int64_t n, bool molecules, hipStream_t stream) {
    if (molecules)
        k_molecules<T, MODE, EMIT><<<unit_blocks<k_molecules<T, MODE, EMIT>>(n), kBlock, 0,
                                     stream>>>(q);
    else
        k_brute<T, MODE, EMIT><<<brute_blocks<T, MODE, EMIT>(n), kBlock, 0, stream>>>(q);
}

// Words of an atom's hit-mask row: the request's, or the default.
static int mask_words(const tnr_request* req) {
    return req->mask_words > 0 ? (int)req->mask_words : kDefaultMaskWords;
}

template <typename T>
static QueryArgs<T> query_args(const tnr_request* req, const Views& v) {
    QueryArgs<T> q{};
    q.pos = (const T*)req->positions;
    q.cells = (const T*)req->cell;
    q.recs = v.recs;
    q.struct_bin_off = (const int64_t*)v.struct_bin_off;
    q.struct_unit_off = (const int64_t*)v.struct_unit_off;
    q.atom_struct = v.atom_struct;
    q.atom_wrap = v.atom_wrap;
    q.atom_q = (const Vec4<T>*)v.atom_q;
    q.bin_start = v.bin_start;
    q.binned = (const Vec4<T>*)v.binned;
    q.binned_w = v.binned_w;
    q.binned_p = (const Vec4<T>*)v.binned_p;
    q.counts = v.counts;
    q.offsets = v.offsets;
    q.status = v.status;
    q.masks = v.masks;
    q.mask_words = mask_words(req);
    q.n_atoms = req->n_atoms;
    q.nb = req->n_structures;
    q.by_bin = req->sorted ? 0 : 1;
    q.brute_in_cell = req->algorithm == TNR_CELL_LIST ? 1 : 0;
    return q;
}

// Counting: the plan is only known on the device, so with auto both
// families are launched and each exits at once when the plan has none of
// its structures, unless plan is 1 (a hint that there is no cell-list
// structure, checked by the planner) or 5 (every structure a molecule:
// k_molecules counts).  An explicit brute_force request launches the brute-force
// kernel only, an explicit cell_list request the cell-list kernel only,
// which also counts the structures that no bin grid fits (brute force,
// QueryArgs::brute_in_cell).  Emitting: plan bit 0 launches the
// brute-force family, bit 1 the cell-list family over n_tasks bins (one
// workgroup each).
template <typename T, int MODE, bool EMIT>
static void launch_queries(const tnr_request* req, const Layout& L, const QueryArgs<T>& q,
                           int64_t plan, int64_t n_tasks, hipStream_t stream) {
    const int64_t n = req->n_atoms;
    if (n == 0) return;
    // every brute-force structure a molecule (plan bit 2 with brute force only)
    const bool molecules = plan >= 0 && (plan & (int64_t)kPlanMolecules) != 0;
    if constexpr (!EMIT) {
        // plan 1: brute force only (an explicit request or a plan hint);
        // plan 5: molecules only (the molecule plan hint)
        (void)n_tasks;
        if (req->algorithm != TNR_BRUTE_FORCE && (plan & (int64_t)kPlanFamilies) != 1)
            k_cell_count<T, MODE><<<count_blocks<T, MODE>(2 * (L.cap_bins > n ? L.cap_bins : n)),
                                    kBlock, 0, stream>>>(q);
        if (req->algorithm != TNR_CELL_LIST) launch_brute<T, MODE, false>(q, n, molecules, stream);
    } else if (plan < 0) {
        // plan and bins unknown on the host: both families, grids the device
        // holds at once, the kernels reading plan and bins from the status
        if (req->algorithm != TNR_BRUTE_FORCE) {
            const int64_t cap = resident_blocks<k_cell_emit<T, MODE, true>>() / 8 * 8;
            k_cell_emit<T, MODE, true><<<(unsigned)(cap > 8 ? cap : 8), kBlock, 0, stream>>>(q);
        }
        k_brute<T, MODE, true><<<brute_blocks<T, MODE, true>(n), kBlock, 0, stream>>>(q);
    } else {
        if ((plan & 2) && n_tasks > 0)
            k_cell_emit<T, MODE><<<emit_blocks(n_tasks), kBlock, 0, stream>>>(q);
        if (plan & 1) launch_brute<T, MODE, true>(q, n, molecules, stream);
    }
}

template <typename T, bool EMIT>
static void dispatch_queries(const tnr_request* req, const Layout& L, const QueryArgs<T>& q,
                             int64_t plan, int64_t n_tasks, hipStream_t stream) {
    const int mode = (req->half_list ? 2 : 0) | (req->include_self ? 1 : 0);
    switch (mode) {
        case 0: launch_queries<T, 0, EMIT>(req, L, q, plan, n_tasks, stream); break;
        case 1: launch_queries<T, 1, EMIT>(req, L, q, plan, n_tasks, stream); break;
        case 2: launch_queries<T, 2, EMIT>(req, L, q, plan, n_tasks, stream); break;
        default: launch_queries<T, 3, EMIT>(req, L, q, plan, n_tasks, stream); break;
    }
}

// The count pipeline.  Its last kernel copies the status words into
// host_out (a device-visible pointer to the caller's pinned buffer) when
// given.
// Plan hints of a count (from an earlier count of the same request shape):
//   HINT_BRUTE      no cell-list structure: the cell-list kernels are not
//                   launched, and the planner raises ST_PLAN_HINT if a
//                   structure is planned as a cell list after all;
//   HINT_MOLECULES  every structure a molecule: k_molecule_setup is the
//                   whole prologue (ST_PLAN_HINT for any other structure),
//                   followed by k_struct_scan only for more than
//                   kMolLocalMax structures (below that the molecule
//                   counting kernel finishes the plan from the workgroups'
//                   summaries);
//   HINT_PERIODIC   one fully periodic structure planned as a cell list
//                   whose grid periodic_grid chooses: the periodic fast
//                   prologue (k_periodic_atoms, k_periodic_place;
//                   ST_PLAN_HINT if it does not apply, or if the placing
//                   kernel's workgroups could not all be resident).
enum CountHint : int { HINT_NONE = 0, HINT_BRUTE = 1, HINT_MOLECULES = 2, HINT_PERIODIC = 3 };

template <typename T>
static hipError_t run_count(const tnr_request* req, void* ws, const Layout& L,
                            hipStream_t stream, long long* host_out, int hint) {
    const bool brute_hint = hint == HINT_BRUTE;
    const bool periodic = hint == HINT_PERIODIC;
    const bool cell_kernels =
        req->algorithm != TNR_BRUTE_FORCE && (hint == HINT_NONE || periodic);
    const Views v = views(ws, L);
    const int64_t n = req->n_atoms, nb = req->n_structures;
    const int reach = req->stencil_reach;  // 0: chosen per structure
    const int mw = mask_words(req);
    const int64_t n_tiles =
        (int64_t)((L.tiles_pairs - L.tiles_bins) / sizeof(unsigned long long)) + L.n_tiles_pairs;
    // a molecules-only batch of up to kMolLocalMax structures: no batch scan
    // (the molecule counting kernel finishes the plan, MoleculeBlock)
    const bool mol_local = hint == HINT_MOLECULES && nb >= 1 && nb <= kMolLocalMax;
    if (hint == HINT_MOLECULES) {
        k_molecule_setup<T><<<blocks_for(nb, kSetupBlock), kSetupBlock, 0, stream>>>(
            req->batch_ptr, (const T*)req->cell, req->pbc, nb, n, req->cutoff, mw, req->algorithm,
            v.recs, v.struct_bins, v.struct_units, v.struct_meta, v.status, v.tiles_pairs,
            L.n_tiles_pairs, mol_local ? 1 : 0, v.struct_bin_off);
        if (!mol_local)
            k_struct_scan<<<1, kBlock, 0, stream>>>(v.struct_bins, v.struct_units,
                                                    v.struct_meta, nb, n, v.struct_bin_off,
                                                    v.struct_unit_off, v.recs, v.status,
                                                    L.cap_bins, 0);
    } else if (periodic) {
        // one fully periodic structure: set-up, grid, atoms and bins; then
        // the finished plan beside ranks, bin starts and binned atoms
        const unsigned nblk = blocks_for(n);
        k_periodic_atoms<T><<<nblk, kBlock, 0, stream>>>(
            (const T*)req->positions, req->batch_ptr, (const T*)req->cell, req->pbc, req->cutoff,
            mw, n, req->algorithm, reach, v.recs, v.block_partials, v.atom_struct, v.atom_wrap,
            (Vec4<T>*)v.atom_q, v.atom_bin, v.status, v.place_cnt,
            kPlaceStride * (L.cap_bins + 1), v.tiles_bins, n_tiles, v.counts, v.struct_bins,
            v.struct_bin_off, v.struct_units, v.struct_unit_off, v.place, v.place_flags, v.memo);
        // the placing workgroups (behind the finishing one and seven that
        // leave at once) are no more than the device holds at once, so that
        // every one reaches the barrier
        const int64_t cap = resident_blocks<k_periodic_place<T>>() - (int64_t)kPlaceFirst;
        const int64_t place_blocks = (int64_t)nblk < cap ? (int64_t)nblk : (cap > 1 ? cap : 1);
        k_periodic_place<T><<<(unsigned)(place_blocks + kPlaceFirst), kBlock, 0, stream>>>(
            (const T*)req->cell, n, req->cutoff, req->algorithm, v.recs, v.block_partials,
            (int64_t)nblk, v.struct_bins, v.struct_bin_off, v.struct_units, v.struct_unit_off,
            L.cap_bins, v.status, v.atom_bin, v.atom_rank, v.place_cnt, v.bin_start,
            (const Vec4<T>*)v.atom_q, (Vec4<T>*)v.binned, (const T*)req->positions,
            v.atom_wrap, v.binned_w, (Vec4<T>*)v.binned_p, v.place, v.place_flags,
            barrier_ticks(), req->batch_ptr, req->pbc, mw, reach, v.memo);
    } else if (nb == 1 && n > 0) {
        // one structure: set-up and atoms, then plan and binning, in two
        // launches; k_single_bin writes the status words
        k_atoms<T, true><<<blocks_for(n), kBlock, 0, stream>>>(
            (const T*)req->positions, req->batch_ptr, (const T*)req->cell, req->pbc, req->cutoff,
            mw, nb, n, v.recs, v.block_partials, v.atom_struct, v.atom_wrap, (Vec4<T>*)v.atom_q,
            v.status, v.bin_count, L.cap_bins + 1, v.tiles_bins, n_tiles, v.counts);
        k_single_bin<T><<<blocks_for(n), kBlock, 0, stream>>>(
            (const T*)req->cell, n, req->cutoff, req->algorithm, reach, v.recs, v.block_partials,
            (int64_t)blocks_for(n), (const Vec4<T>*)v.atom_q, v.atom_bin, v.atom_rank,
            v.bin_count, v.struct_bins, v.struct_bin_off, v.struct_units, v.struct_unit_off,
            L.cap_bins, v.status, brute_hint ? 1 : 0);
    } else {
        // k_setup zeroes the status words; k_atoms zeroes the bin counters and
        // the tile states of both single-pass scans.
        k_setup<T><<<blocks_for(nb > 0 ? nb : 1, kSetupBlock), kSetupBlock, 0, stream>>>(
            req->batch_ptr, (const T*)req->cell, req->pbc, nb, n, req->cutoff, mw, v.recs,
            v.status, v.memo);
        if (n > 0)
            k_atoms<T, false><<<blocks_for(n), kBlock, 0, stream>>>(
                (const T*)req->positions, req->batch_ptr, (const T*)req->cell, req->pbc,
                req->cutoff, mw, nb, n, v.recs, v.block_partials, v.atom_struct, v.atom_wrap,
                (Vec4<T>*)v.atom_q, v.status, v.bin_count, L.cap_bins + 1, v.tiles_bins, n_tiles,
                v.counts);
        // a single structure is planned and scanned by one workgroup
        const int fused_scan = nb <= 1 ? 1 : 0;
        k_plan<T><<<(unsigned)(nb > 0 ? nb : 1), kBlock, 0, stream>>>(
            (const T*)req->cell, nb, n, req->cutoff, req->algorithm, reach, v.recs,
            v.block_partials, v.struct_bins, v.struct_bin_off, v.struct_units, v.struct_unit_off,
            L.cap_bins, v.status, fused_scan, v.struct_meta);
        if (!fused_scan)
            k_struct_scan<<<1, kBlock, 0, stream>>>(
                v.struct_bins, v.struct_units, v.struct_meta, nb, n, v.struct_bin_off,
                v.struct_unit_off, v.recs, v.status, L.cap_bins, brute_hint ? 1 : 0);
        if (n > 0 && cell_kernels)
            k_bin<T><<<blocks_for(n), kBlock, 0, stream>>>(n, v.recs, v.atom_struct,
                                                           (const Vec4<T>*)v.atom_q, v.atom_bin,
                                                           v.atom_rank, v.bin_count, v.status);
    }
    if (n > 0 && cell_kernels && !periodic) {
        k_scan_lookback<int, int><<<(unsigned)(L.n_tiles_bins), kBlock, 0, stream>>>(
            v.bin_count, L.cap_bins, v.status + SS_TOTAL_BINS, v.bin_start, v.tiles_bins,
            v.status + SS_TICKET_BINS, v.status, nullptr);
        k_scatter<T><<<blocks_for(n), kBlock, 0, stream>>>(n, (const Vec4<T>*)v.atom_q,
                                                           v.atom_bin, v.atom_rank,
                                                           v.bin_start, (Vec4<T>*)v.binned,
                                                           (const T*)req->positions, v.atom_wrap,
                                                           v.binned_w, (Vec4<T>*)v.binned_p,
                                                           v.status);
    }
    QueryArgs<T> q = query_args<T>(req, v);
    if (mol_local) {
        q.mol_local = 1;
        q.mol_blocks = reinterpret_cast<const MoleculeBlock*>(v.struct_meta);
    }
    dispatch_queries<T, false>(
        req, L, q, cell_kernels ? 0 : (hint == HINT_MOLECULES ? 1 | (int64_t)kPlanMolecules : 1), 0,
        stream);
    // pairs per source -> offsets; the total (E) goes to the status words
    k_scan_lookback<long long, long long>
        <<<(unsigned)((n + kScanTile - 1) / kScanTile > 0 ? (n + kScanTile - 1) / kScanTile : 1),
           kBlock, 0, stream>>>(v.counts, n, nullptr, v.offsets, v.tiles_pairs,
                                v.status + SS_TICKET_PAIRS, v.status, v.status + SS_PAIRS,
                                host_out);
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
    q.edge = out->edge_index;
    q.limit = out->n_pairs;
    q.n_bins = out->plan < 0 ? L.cap_bins : out->n_tasks;
    dispatch_queries<T, true>(req, L, q, out->plan, out->n_tasks, stream);
    return hipGetLastError();
}

struct StatusMessage {
    unsigned long long bit;
    int code;
    const char* text;
};

// Priority follows the order in which the reference raises: host-side
// batch_ptr checks, periodic metadata, then device status words; a plan
// hint that did not hold comes first (the count is retried without it).
static const StatusMessage kMessages[] = {
    {ST_PLAN_HINT, TNR_RETRY,
     "the plan hint does not hold for this request; count again without it"},
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
    {ST_SCAN_STALL, TNR_SEARCH_ERROR, "a device-wide scan of the neighbor search did not complete"},
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
    if (req->stencil_reach < 0 || req->stencil_reach > 4)
        return put_error(err, err_len, TNR_INPUT_ERROR, "stencil_reach must be in [0, 4]");
    if (req->mask_words < 0 || req->mask_words > kMaskWords)
        return put_error(err, err_len, TNR_INPUT_ERROR, "mask_words must be in [0, 64]");
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
                     req->dtype == TNR_FLOAT32 ? sizeof(float) : sizeof(double),
                     mask_words(req));
    if (L->cap_bins >= (int64_t{1} << 31))
        return put_error(err, err_len, TNR_INPUT_ERROR,
                         "the current implementation supports fewer than 2^31 atoms");
    if (!ws || ws_bytes < L->total || ((uintptr_t)ws & 255) != 0)
        return put_error(err, err_len, TNR_INPUT_ERROR,
                         "workspace is missing, too small or not 256-byte aligned");
    return TNR_OK;
}

// ------------------------------------------------------- static scratch
// Device memory of tnr_search_static, for callers that cannot allocate: one
// array per GPU the library runs on (the runtime gives each device its own
// copy, at its own address), held until the process ends.  Host code never
// passes the array's name to a kernel or a copy: it is a host-side stand-in,
// not a device address.  scratch_address() looks up the device address once
// per device (with that device current) and every later use goes through it.
constexpr size_t kStaticScratchBytes = size_t{64} << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_lock;
static void* g_scratch_ptr[kMaxDevices];

static int scratch_address(void** out, char* err, size_t err_len) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return put_error(err, err_len, TNR_DEVICE_ERROR, hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices)
        return put_error(err, err_len, TNR_DEVICE_ERROR, "device index beyond the library's table");
    std::lock_guard<std::mutex> guard(g_scratch_lock);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return put_error(err, err_len, TNR_DEVICE_ERROR, hipGetErrorString(e));
        if (!ptr || ((uintptr_t)ptr & 255) != 0)
            return put_error(err, err_len, TNR_DEVICE_ERROR, "static scratch has no usable address");
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return TNR_OK;
}

// ------------------------------------------------------- Verlet-skin lists

struct SkinLayout {
    int64_t n_wtiles, cap_runs, n_scan_tiles, n_scan_tiles2;
    int64_t n_parts;
    size_t status, persist, copy, parts, tiles, tiles2, wtile_starts, wtile_runs_before, wtile_kept,
        wtile_offsets, wtile_run0, runs, rank, perm, nonsrc, nonsrc_before, placed, records,
        ref_pos, ref_cell, ref_pbc, ref_bp, total;
};

// The skin workspace: the filter's status block, the store's persistent
// words, the host copy of the status, look-back tile states of the scans
// over wave tiles and over atoms, per-wave-tile run data and counts, the run
// table (at most one run per atom), places, positions in place order, the
// 8-byte records and copies of the build's inputs.
static SkinLayout skin_layout(int64_t n_pairs, int64_t n_atoms, int64_t nb, size_t tsize) {
    SkinLayout L;
    L.n_wtiles = (n_pairs + kSkinWaveTile - 1) / kSkinWaveTile;
    L.cap_runs = n_atoms > 0 ? n_atoms : 1;
    L.n_scan_tiles = (L.n_wtiles + kScanTile - 1) / kScanTile;
    L.n_scan_tiles2 = (n_atoms + kScanTile - 1) / kScanTile;
    size_t o = 0;
    auto take = [&](size_t bytes) {
        const size_t at = o;
        o = align_up(o + bytes);
        return at;
    };
    const size_t wtiles = (size_t)(L.n_wtiles > 0 ? L.n_wtiles : 1);
    const size_t atoms = (size_t)(n_atoms > 0 ? n_atoms : 1);
    L.status = take(sizeof(int64_t) * SS_SLOTS);
    L.persist = take(sizeof(int64_t) * SP_WORDS);
    L.copy = take(sizeof(int64_t) * kHostResultSlots);
    // one workgroup of the place kernel per 256 atoms or cell entries
    const int64_t place = n_atoms > 9 * nb + 1 ? n_atoms : 9 * nb + 1;
    L.n_parts = (place + kBlock - 1) / kBlock;
    L.parts = take(sizeof(int64_t) * 4 * (size_t)L.n_parts);
    L.tiles = take(sizeof(int64_t) * (size_t)(L.n_scan_tiles > 0 ? L.n_scan_tiles : 1));
    L.tiles2 = take(sizeof(int64_t) * (size_t)(L.n_scan_tiles2 > 0 ? L.n_scan_tiles2 : 1));
    L.wtile_starts = take(sizeof(int64_t) * (wtiles + 1));
    L.wtile_runs_before = take(sizeof(int64_t) * (wtiles + 1));
    L.wtile_kept = take(sizeof(int64_t) * (wtiles + 1));
    L.wtile_offsets = take(sizeof(int64_t) * (wtiles + 1));
    L.wtile_run0 = take(sizeof(int32_t) * wtiles);
    L.runs = take(sizeof(int32_t) * 2 * (size_t)L.cap_runs);
    L.rank = take(sizeof(int32_t) * atoms);
    L.perm = take(sizeof(int32_t) * atoms);
    L.nonsrc = take(sizeof(int32_t) * atoms);
    L.nonsrc_before = take(sizeof(int32_t) * (atoms + 1));
    L.placed = take(tsize * 4 * atoms);
    L.records = take(sizeof(int64_t) * (size_t)(n_pairs > 0 ? n_pairs : 1));
    L.ref_pos = take(tsize * 3 * atoms);
    L.ref_cell = take(tsize * 9 * (size_t)(nb > 0 ? nb : 1));
    L.ref_pbc = take(3 * (size_t)(nb > 0 ? nb : 1));
    L.ref_bp = take(sizeof(int64_t) * (size_t)(nb + 1));
    L.total = o;
    return L;
}

static size_t dtype_size(int32_t dtype) { return dtype == TNR_FLOAT32 ? sizeof(float) : sizeof(double); }

// Checks shared by the store and the filter: the request (dtype, cutoff,
// sizes, input pointers) and the workspace.
static int check_skin_request(const tnr_request* req, int64_t n_pairs, size_t ws_bytes,
                              const void* ws, char* err, size_t err_len, SkinLayout* L) {
    if (!req) return put_error(err, err_len, TNR_INPUT_ERROR, "request is null");
    if (req->dtype != TNR_FLOAT32 && req->dtype != TNR_FLOAT64)
        return put_error(err, err_len, TNR_INPUT_ERROR,
                         "positions must have dtype float32 or float64");
    if (!(std::isfinite(req->cutoff) && req->cutoff > 0))
        return put_error(err, err_len, TNR_INPUT_ERROR, "cutoff must be finite and positive");
    if (req->n_atoms < 0 || req->n_structures < 1 || n_pairs < 0 ||
        req->n_atoms >= (int64_t{1} << 31))
        return put_error(err, err_len, TNR_INPUT_ERROR, "invalid sizes");
    if (!req->batch_ptr || !req->cell || !req->pbc || (req->n_atoms > 0 && !req->positions))
        return put_error(err, err_len, TNR_INPUT_ERROR, "required pointers are null");
    *L = skin_layout(n_pairs, req->n_atoms, req->n_structures, dtype_size(req->dtype));
    if (!ws || ws_bytes < L->total || ((uintptr_t)ws & 255) != 0)
        return put_error(err, err_len, TNR_INPUT_ERROR,
                         "workspace is missing, too small or not 256-byte aligned");
    return TNR_OK;
}

// The pair mode of a request as tnr_skin_list::pair_mode records it.
static int32_t pair_mode(const tnr_request* req) {
    return (req->half_list ? 2 : 0) | (req->include_self ? 1 : 0);
}

static int check_skin_list(const tnr_request* req, const tnr_skin_list* list, char* err,
                           size_t err_len) {
    if (!list) return put_error(err, err_len, TNR_INPUT_ERROR, "list is null");
    if (list->dtype != req->dtype || list->n_atoms != req->n_atoms ||
        list->n_structures != req->n_structures)
        return put_error(err, err_len, TNR_INPUT_ERROR,
                         "the request's dtype, N or B differ from the stored list's");
    // a list stored in one pair mode holds other pairs than another mode's
    if (list->pair_mode != pair_mode(req))
        return put_error(err, err_len, TNR_INPUT_ERROR,
                         "the request's half_list or include_self differ from the stored list's");
    if (!(std::isfinite(list->build_cutoff) && list->build_cutoff >= req->cutoff))
        return put_error(err, err_len, TNR_INPUT_ERROR,
                         "the list's build cutoff must be finite and at least the cutoff");
    return TNR_OK;
}

static unsigned skin_blocks(int64_t n_wtiles) {
    const int64_t b = (n_wtiles + kWavesPerBlock - 1) / kWavesPerBlock;
    return (unsigned)(b > 0 ? b : 1);
}

template <typename T>
static hipError_t run_skin_store(const tnr_request* req, const int64_t* pairs,
                                 const int32_t* shifts, int64_t n_pairs, void* ws,
                                 const SkinLayout& L, hipStream_t stream) {
    char* base = (char*)ws;
    auto* status = (unsigned long long*)(base + L.status);
    auto* persist = (unsigned long long*)(base + L.persist);
    auto* tiles = (unsigned long long*)(base + L.tiles);
    auto* tiles2 = (unsigned long long*)(base + L.tiles2);
    const int64_t n_tiles = L.n_scan_tiles > 0 ? L.n_scan_tiles : 1;
    const int64_t n_tiles2 = L.n_scan_tiles2 > 0 ? L.n_scan_tiles2 : 1;
    SkinStore k{};
    k.n_pairs = n_pairs;
    k.n_atoms = req->n_atoms;
    k.nb = req->n_structures;
    k.n_wtiles = L.n_wtiles;
    k.cap_runs = L.cap_runs;
    k.pairs = pairs;
    k.shifts = shifts;
    k.pos = req->positions;
    k.cell = req->cell;
    k.pbc = req->pbc;
    k.bp = req->batch_ptr;
    k.records = (unsigned long long*)(base + L.records);
    k.runs = (int2*)(base + L.runs);
    k.wtile_run0 = (int*)(base + L.wtile_run0);
    k.wtile_starts = (long long*)(base + L.wtile_starts);
    k.wtile_runs_before = (const long long*)(base + L.wtile_runs_before);
    k.rank = (int*)(base + L.rank);
    k.perm = (int*)(base + L.perm);
    k.nonsrc = (int*)(base + L.nonsrc);
    k.nonsrc_before = (const int*)(base + L.nonsrc_before);
    k.ref_pos = base + L.ref_pos;
    k.ref_cell = base + L.ref_cell;
    k.ref_pbc = (uint8_t*)(base + L.ref_pbc);
    k.ref_bp = (int64_t*)(base + L.ref_bp);
    k.persist = persist;
    k_skin_clear<<<1, kBlock, 0, stream>>>(status, tiles, n_tiles, persist, tiles2, n_tiles2);
    // the copies need about one block per 2048 input words; the records one
    // per four wave tiles
    int64_t grid = skin_blocks(L.n_wtiles);
    const int64_t copy = (3 * req->n_atoms + kSkinBlockPairs - 1) / kSkinBlockPairs;
    if (copy > grid) grid = copy;
    k_skin_pack<T><<<(unsigned)grid, kBlock, 0, stream>>>(k);
    if (L.n_wtiles > 0) {
        k_scan_lookback<long long, long long><<<(unsigned)L.n_scan_tiles, kBlock, 0, stream>>>(
            (const long long*)k.wtile_starts, L.n_wtiles, nullptr,
            (long long*)(base + L.wtile_runs_before), tiles, persist + SP_TICKET, persist,
            persist + SP_RUNS, nullptr);
        k_skin_runs<<<skin_blocks(L.n_wtiles), kBlock, 0, stream>>>(k);
    }
    if (req->n_atoms > 0) {
        k_scan_lookback<int, int><<<(unsigned)L.n_scan_tiles2, kBlock, 0, stream>>>(
            k.nonsrc, req->n_atoms, nullptr, (int*)(base + L.nonsrc_before), tiles2,
            persist + SP_TICKET2, persist, nullptr, nullptr);
        k_skin_ranks<<<blocks_for(req->n_atoms), kBlock, 0, stream>>>(k);
    }
    if (n_pairs > 0) k_skin_retarget<<<blocks_for(n_pairs), kBlock, 0, stream>>>(k);
    // the filter starts from zeroed status words and scan tiles
    k_skin_clear<<<1, kBlock, 0, stream>>>(status, tiles, n_tiles, nullptr, tiles2, 0);
    return hipGetLastError();
}

template <typename T>
static hipError_t run_skin_filter(const tnr_request* req, const tnr_skin_list* list, void* ws,
                                  const SkinLayout& L, const tnr_outputs* out,
                                  hipStream_t stream, long long* host_out) {
    char* base = (char*)ws;
    auto* status = (unsigned long long*)(base + L.status);
    auto* persist = (unsigned long long*)(base + L.persist);
    auto* tiles = (unsigned long long*)(base + L.tiles);
    SkinFilter k{};
    k.n_pairs = list->n_pairs;
    k.n_atoms = req->n_atoms;
    k.nb = req->n_structures;
    k.n_wtiles = L.n_wtiles;
    k.cap_runs = L.cap_runs;
    k.records = (const unsigned long long*)(base + L.records);
    k.runs = (const int2*)(base + L.runs);
    k.wtile_run0 = (const int*)(base + L.wtile_run0);
    k.perm = (const int*)(base + L.perm);
    k.ref_pos = base + L.ref_pos;
    k.ref_cell = base + L.ref_cell;
    k.ref_pbc = (const uint8_t*)(base + L.ref_pbc);
    k.ref_bp = (const int64_t*)(base + L.ref_bp);
    k.bp = req->batch_ptr;
    k.pbc = req->pbc;
    k.persist = persist;
    k.placed = base + L.placed;
    k.wtile_kept = (long long*)(base + L.wtile_kept);
    k.wtile_offsets = (const long long*)(base + L.wtile_offsets);
    k.cutoff = req->cutoff;
    QueryArgs<T> q{};
    q.pos = (const T*)req->positions;
    q.cells = (const T*)req->cell;
    q.status = status;
    q.n_atoms = req->n_atoms;
    q.nb = req->n_structures;
    q.limit = out->n_pairs;
    q.pairs = out->pairs;
    q.shifts = out->shifts;
    q.dist = (T*)out->distances;
    q.vec = (T*)out->vectors;
    q.src = out->sources;
    q.dst = out->targets;
    auto* parts = (unsigned long long*)(base + L.parts);
    k_skin_place<T><<<(unsigned)L.n_parts, kBlock, 0, stream>>>(k, (const T*)req->positions,
                                                               (const T*)req->cell, parts);
    if (L.n_wtiles > 0) {
        k_skin_count<T><<<skin_blocks(L.n_wtiles), kBlock, 0, stream>>>(k, q);
        k_scan_lookback<long long, long long><<<(unsigned)L.n_scan_tiles, kBlock, 0, stream>>>(
            (const long long*)k.wtile_kept, L.n_wtiles, nullptr,
            (long long*)(base + L.wtile_offsets), tiles, status + SK_TICKET, status,
            status + SK_PAIRS, nullptr);
        if (out->n_pairs > 0) k_skin_emit<T><<<skin_blocks(L.n_wtiles), kBlock, 0, stream>>>(k, q);
    }
    k_skin_publish<<<1, kBlock, 0, stream>>>(status, persist, parts, L.n_parts, host_out,
                                             (long long*)(base + L.copy), tiles,
                                             L.n_scan_tiles > 0 ? L.n_scan_tiles : 1);
    return hipGetLastError();
}

static double bits_double(int64_t v) {
    double d;
    std::memcpy(&d, &v, sizeof d);
    return d;
}

// Whether the filtered list equals a search at `cutoff` for the current
// positions.  With eps the input type's machine epsilon, m the largest atom
// displacement, A the largest |x|_1, K the largest skin_condition and
// Cb the build cutoff: every pair within the cutoff now has
// |S cell|_2 <= 3 (cutoff + 2A) (when 2 eps K <= 1/3), so the terms of its
// public D sum to at most M = 2A + 3 (cutoff + 2A) K in 1-norm and its
// rounded D lies within 2 eps M of the exact one; the exact D moved by at
// most 2m since the build, and the rounded d^2 and squared cutoffs add
// relative errors of a few eps.  The pair was then in the stored list when
//   cutoff (1 + 2e) + 2m (1 + 4e) + 2e M + 2e (M + 4m) < Cb (1 - 3e),
// here with e = 2 eps, twice the error bounds.
static bool skin_valid(int32_t dtype, double cutoff, double build_cutoff, const int64_t* h) {
    if (h[SK_CHANGED]) return false;
    const double eps = dtype == TNR_FLOAT32 ? 0x1p-23 : 0x1p-52;
    const double e = 2 * eps;
    const double m = std::sqrt(bits_double(h[SK_MAX_DISP2])) * (1 + 1e-12);
    const double A = bits_double(h[SK_MAX_COORD]) * (1 + 1e-12);
    const double K = bits_double(h[SK_MAX_COND]);
    if (!(2 * eps * K <= 1.0 / 3.0)) return false;
    const double M = 2 * A + 3 * (cutoff + 2 * A) * K;
    const double lhs = cutoff * (1 + 2 * e) + 2 * m * (1 + 4 * e) + 2 * e * M + 2 * e * (M + 4 * m);
    return lhs < build_cutoff * (1 - 3 * e);
}

}  // namespace tnr

// ----------------------------------------------------------------- C ABI

extern "C" {

int tnr_abi_version(void) { return TNR_ABI_VERSION; }

#ifndef TNR_OFFLOAD_ARCH
#error "build with -DTNR_OFFLOAD_ARCH=\"<offload target>\" (tonari_amd/build.py)"
#endif

const char* tnr_device_arch(void) { return TNR_OFFLOAD_ARCH; }

int tnr_hip_version(void) { return HIP_VERSION_MAJOR * 100 + HIP_VERSION_MINOR; }

size_t tnr_workspace_size(const tnr_request* req) {
    if (!req || req->n_atoms < 0 || req->n_structures < 0 || req->mask_words < 0 ||
        req->mask_words > tnr::kMaskWords)
        return 0;
    return tnr::make_layout(req->n_atoms, req->n_structures,
                            req->dtype == TNR_FLOAT32 ? sizeof(float) : sizeof(double),
                            tnr::mask_words(req))
        .total;
}

int tnr_count_async(const tnr_request* req, void* workspace, size_t workspace_bytes,
                    int64_t* host_result, void* stream, char* err, size_t err_len) {
    return tnr_count_async_hinted(req, workspace, workspace_bytes, host_result, stream, -1, err,
                                  err_len);
}

int tnr_count_async_hinted(const tnr_request* req, void* workspace, size_t workspace_bytes,
                           int64_t* host_result, void* stream, int64_t plan_hint, char* err,
                           size_t err_len) {
    tnr::Layout L;
    const int rc = tnr::check_request(req, workspace_bytes, workspace, err, err_len, &L);
    if (rc != TNR_OK) return rc;
    if (!host_result) return tnr::put_error(err, err_len, TNR_INPUT_ERROR, "host_result is null");
    hipStream_t s = (hipStream_t)stream;
    // Pinned host memory is written by the count's last kernel directly;
    // other memory gets a copy behind it.
    void* mapped = nullptr;
    if (hipHostGetDevicePointer(&mapped, host_result, 0) != hipSuccess) {
        mapped = nullptr;
        (void)hipGetLastError();
    }
    // a hint of brute force only (plan bits 0-1 equal to 1) from an earlier
    // count; with bit 2 every structure was a molecule
    int hint = tnr::HINT_NONE;
    // a hint of one fully periodic cell-list structure (plan bit 3)
    if (plan_hint >= 0 && (plan_hint & (int64_t)tnr::kPlanPeriodicGrid) &&
        (plan_hint & (int64_t)tnr::kPlanFamilies) == 2 && req->n_structures == 1 &&
        req->n_atoms > 0 && req->algorithm != TNR_BRUTE_FORCE)
        hint = tnr::HINT_PERIODIC;
    if (plan_hint >= 0 && (plan_hint & (int64_t)tnr::kPlanFamilies) == 1 && req->n_structures > 0 &&
        (req->algorithm == TNR_AUTO || req->algorithm == TNR_BRUTE_FORCE)) {
        if (plan_hint & (int64_t)tnr::kPlanMolecules)
            hint = tnr::HINT_MOLECULES;
        else if (req->algorithm == TNR_AUTO)
            hint = tnr::HINT_BRUTE;
    }
    hipError_t e =
        req->dtype == TNR_FLOAT32
            ? tnr::run_count<float>(req, workspace, L, s, (long long*)mapped, hint)
            : tnr::run_count<double>(req, workspace, L, s, (long long*)mapped, hint);
    if (e == hipSuccess && !mapped) {
        const tnr::Views v = tnr::views(workspace, L);
        e = hipMemcpyAsync(host_result, v.status, TNR_HOST_RESULT_SLOTS * sizeof(int64_t),
                           hipMemcpyDeviceToHost, s);
    }
    if (e != hipSuccess) return tnr::put_error(err, err_len, TNR_DEVICE_ERROR, hipGetErrorString(e));
    return TNR_OK;
}

int tnr_count_finish(const int64_t* host_result, int64_t* n_pairs, char* err, size_t err_len) {
    if (!host_result || !n_pairs)
        return tnr::put_error(err, err_len, TNR_INPUT_ERROR, "result pointers are null");
    const unsigned long long flags = (unsigned long long)host_result[tnr::SS_FLAGS];
    if (flags) {
        for (const auto& m : tnr::kMessages)
            if (flags & m.bit) return tnr::put_error(err, err_len, m.code, m.text);
        return tnr::put_error(err, err_len, TNR_SEARCH_ERROR, "invalid neighbor-list status");
    }
    *n_pairs = host_result[tnr::SS_PAIRS];
    return TNR_OK;
}

int tnr_count(const tnr_request* req, void* workspace, size_t workspace_bytes,
              int64_t* host_result, void* stream, int64_t* n_pairs, char* err, size_t err_len) {
    if (!n_pairs) return tnr::put_error(err, err_len, TNR_INPUT_ERROR, "n_pairs is null");
    const int rc = tnr_count_async(req, workspace, workspace_bytes, host_result, stream, err,
                                   err_len);
    if (rc != TNR_OK) return rc;
    const hipError_t e = hipStreamSynchronize((hipStream_t)stream);
    if (e != hipSuccess) return tnr::put_error(err, err_len, TNR_DEVICE_ERROR, hipGetErrorString(e));
    return tnr_count_finish(host_result, n_pairs, err, err_len);
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

int tnr_search_static(const tnr_request* req, const tnr_outputs* out, int64_t* host_result,
                      void* stream, char* err, size_t err_len) {
    if (!req) return tnr::put_error(err, err_len, TNR_INPUT_ERROR, "request is null");
    const size_t need = tnr_workspace_size(req);
    if (need > tnr::kStaticScratchBytes) {
        char msg[192];
        std::snprintf(msg, sizeof(msg),
                      "request needs %zu bytes of scratch; the static scratch holds %zu "
                      "bytes (use tnr_count / tnr_emit with a workspace)",
                      need, tnr::kStaticScratchBytes);
        return tnr::put_error(err, err_len, TNR_INPUT_ERROR, msg);
    }
    void* ws = nullptr;
    int rc = tnr::scratch_address(&ws, err, err_len);
    if (rc != TNR_OK) return rc;
    rc = tnr_count_async(req, ws, tnr::kStaticScratchBytes, host_result, stream, err, err_len);
    if (rc != TNR_OK || !out || out->n_pairs <= 0) return rc;
    // the emit reads the plan and the bins from the count's status words on
    // the device (no host wait), and drops pairs beyond out->n_pairs rows
    tnr_outputs o = *out;
    o.plan = -1;
    o.n_tasks = 0;
    return tnr_emit(req, ws, tnr::kStaticScratchBytes, &o, stream, err, err_len);
}

size_t tnr_skin_workspace_size(const tnr_request* req, int64_t n_pairs) {
    if (!req || req->n_atoms < 0 || req->n_structures < 0 || n_pairs < 0) return 0;
    return tnr::skin_layout(n_pairs, req->n_atoms, req->n_structures, tnr::dtype_size(req->dtype))
        .total;
}

int tnr_skin_store(const tnr_request* req, double build_cutoff, const int64_t* pairs,
                   const int32_t* shifts, int64_t n_pairs, void* workspace,
                   size_t workspace_bytes, tnr_skin_list* list, void* stream, char* err,
                   size_t err_len) {
    tnr::SkinLayout L;
    const int rc =
        tnr::check_skin_request(req, n_pairs, workspace_bytes, workspace, err, err_len, &L);
    if (rc != TNR_OK) return rc;
    if (!list) return tnr::put_error(err, err_len, TNR_INPUT_ERROR, "list is null");
    if (!(std::isfinite(build_cutoff) && build_cutoff >= req->cutoff))
        return tnr::put_error(err, err_len, TNR_INPUT_ERROR,
                              "the list's build cutoff must be finite and at least the cutoff");
    if (n_pairs > 0 && (!pairs || !shifts))
        return tnr::put_error(err, err_len, TNR_INPUT_ERROR, "required pointers are null");
    hipStream_t s = (hipStream_t)stream;
    const hipError_t e =
        req->dtype == TNR_FLOAT32
            ? tnr::run_skin_store<float>(req, pairs, shifts, n_pairs, workspace, L, s)
            : tnr::run_skin_store<double>(req, pairs, shifts, n_pairs, workspace, L, s);
    if (e != hipSuccess) return tnr::put_error(err, err_len, TNR_DEVICE_ERROR, hipGetErrorString(e));
    list->n_pairs = n_pairs;
    list->n_atoms = req->n_atoms;
    list->n_structures = req->n_structures;
    list->dtype = req->dtype;
    list->pair_mode = tnr::pair_mode(req);
    list->build_cutoff = build_cutoff;
    return TNR_OK;
}

int tnr_skin_filter_async(const tnr_request* req, const tnr_skin_list* list, void* workspace,
                          size_t workspace_bytes, const tnr_outputs* out, int64_t* host_result,
                          void* stream, char* err, size_t err_len) {
    tnr::SkinLayout L;
    if (!list) return tnr::put_error(err, err_len, TNR_INPUT_ERROR, "list is null");
    int rc = tnr::check_skin_request(req, list->n_pairs, workspace_bytes, workspace, err,
                                     err_len, &L);
    if (rc != TNR_OK) return rc;
    rc = tnr::check_skin_list(req, list, err, err_len);
    if (rc != TNR_OK) return rc;
    if (!out || !host_result)
        return tnr::put_error(err, err_len, TNR_INPUT_ERROR, "outputs or host_result are null");
    if (out->edge_index)
        return tnr::put_error(err, err_len, TNR_INPUT_ERROR,
                              "the skin filter does not write the edge-first layout");
    if (out->n_pairs < 0) return tnr::put_error(err, err_len, TNR_INPUT_ERROR, "invalid sizes");
    hipStream_t s = (hipStream_t)stream;
    void* mapped = nullptr;
    if (hipHostGetDevicePointer(&mapped, host_result, 0) != hipSuccess) {
        mapped = nullptr;
        (void)hipGetLastError();
    }
    hipError_t e =
        req->dtype == TNR_FLOAT32
            ? tnr::run_skin_filter<float>(req, list, workspace, L, out, s, (long long*)mapped)
            : tnr::run_skin_filter<double>(req, list, workspace, L, out, s, (long long*)mapped);
    if (e == hipSuccess && !mapped)
        e = hipMemcpyAsync(host_result, (char*)workspace + L.copy,
                           TNR_HOST_RESULT_SLOTS * sizeof(int64_t), hipMemcpyDeviceToHost, s);
    if (e != hipSuccess) return tnr::put_error(err, err_len, TNR_DEVICE_ERROR, hipGetErrorString(e));
    return TNR_OK;
}

int tnr_skin_finish(const tnr_request* req, const tnr_skin_list* list, const int64_t* host_result,
                    int64_t* n_pairs, int32_t* rebuild, char* err, size_t err_len) {
    if (!req || !list || !host_result || !n_pairs || !rebuild)
        return tnr::put_error(err, err_len, TNR_INPUT_ERROR, "result pointers are null");
    if ((unsigned long long)host_result[tnr::SK_FLAGS] & tnr::ST_SCAN_STALL)
        return tnr::put_error(err, err_len, TNR_SEARCH_ERROR,
                              "a device-wide scan of the neighbor search did not complete");
    const bool ok = host_result[tnr::SK_STORE] == 0 &&
                    tnr::skin_valid(req->dtype, req->cutoff, list->build_cutoff, host_result);
    *rebuild = ok ? 0 : 1;
    *n_pairs = ok ? host_result[tnr::SK_PAIRS] : 0;
    return TNR_OK;
}

int tnr_geometry_backward(int32_t dtype, int64_t n_pairs, int64_t n_atoms, int64_t n_structures,
                          const int64_t* batch_ptr, const int64_t* pairs, const int32_t* shifts,
                          const void* vectors, const void* distances, const void* grad_vectors,
                          const void* grad_distances, void* grad_positions, void* grad_cell,
                          void* stream, char* err, size_t err_len) {
    if (dtype != TNR_FLOAT32 && dtype != TNR_FLOAT64)
        return tnr::put_error(err, err_len, TNR_INPUT_ERROR, "dtype must be float32 or float64");
    if (n_pairs < 0 || n_atoms < 0 || n_structures < 1)
        return tnr::put_error(err, err_len, TNR_INPUT_ERROR, "invalid sizes");
    if (n_pairs == 0) return TNR_OK;
    if (!batch_ptr || !pairs || !shifts || !grad_positions || !grad_cell)
        return tnr::put_error(err, err_len, TNR_INPUT_ERROR, "required pointers are null");
    if (grad_distances && (!distances || !vectors))
        return tnr::put_error(err, err_len, TNR_INPUT_ERROR,
                              "the gradient of d needs the distances and vectors");
    if (!grad_vectors && !grad_distances) return TNR_OK;
    hipStream_t s = (hipStream_t)stream;
    // at most kBwdPairsPerBlock pairs per workgroup (32 rounds of 64 per
    // wave): the targets of that many consecutive pairs fit its hash table
    const int64_t blocks_wanted = (n_pairs + tnr::kBwdPairsPerBlock - 1) / tnr::kBwdPairsPerBlock;
    if (blocks_wanted > 0x7fffffff)
        return tnr::put_error(err, err_len, TNR_INPUT_ERROR, "invalid sizes");
    const unsigned blocks = (unsigned)blocks_wanted;
    if (dtype == TNR_FLOAT32)
        tnr::k_geometry_backward<float><<<blocks, tnr::kBlock, 0, s>>>(
            n_pairs, n_structures, batch_ptr, pairs, shifts, (const float*)vectors,
            (const float*)distances, (const float*)grad_vectors, (const float*)grad_distances,
            (float*)grad_positions, (float*)grad_cell);
    else
        tnr::k_geometry_backward<double><<<blocks, tnr::kBlock, 0, s>>>(
            n_pairs, n_structures, batch_ptr, pairs, shifts, (const double*)vectors,
            (const double*)distances, (const double*)grad_vectors, (const double*)grad_distances,
            (double*)grad_positions, (double*)grad_cell);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return tnr::put_error(err, err_len, TNR_DEVICE_ERROR, hipGetErrorString(e));
    return TNR_OK;
}

}  // extern "C"
