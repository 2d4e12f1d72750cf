// Device-wide exclusive scans: a single-pass scan with decoupled look-back
// (k_scan_lookback) and the one-workgroup scan of the bins per structure
// (struct_scan_block, run by k_plan for one structure or k_struct_scan).
#pragma once

#include "nl_math.h"

namespace tnr {

// ----------------------------------------------------------- block helpers

// Exclusive scan over the 256 threads of a block; *total receives the sum.
__device__ __forceinline__ long long block_exclusive_scan(long long x, long long* total) {
    __shared__ long long wave_tot[kWavesPerBlock];
    const int lane = lane_id();
    const int w = threadIdx.x / kWave;
    const long long inc = wave_inclusive_scan(x);
    if (lane == kWave - 1) wave_tot[w] = inc;
    __syncthreads();
    long long before = 0, all = 0;
#pragma unroll
    for (int i = 0; i < kWavesPerBlock; ++i) {
        if (i < w) before += wave_tot[i];
        all += wave_tot[i];
    }
    __syncthreads();
    *total = all;
    return before + inc - x;
}

// ------------------------------------------------------- single-pass scan

// Tile state of the single-pass scan: bits 62-63 hold the flag (0 not ready,
// 1 tile aggregate, 2 inclusive prefix), bits 0-61 the value.
constexpr unsigned long long kTileAggregate = 1ull << 62;
constexpr unsigned long long kTilePrefix = 2ull << 62;
constexpr unsigned long long kTileValue = (1ull << 62) - 1;
constexpr int kLookbackSpins = 1 << 22;

// Tile words are relaxed device-scope atomics: a tile word carries
// everything its readers use (flag and value in one 64-bit word), and no
// block reads another block's other outputs, so no ordering with other
// memory is needed.  Release / acquire at device scope would write back /
// invalidate the XCD's L2 on every publish and poll.
__device__ __forceinline__ void tile_publish(unsigned long long* t, unsigned long long w) {
    __hip_atomic_store(t, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long tile_read(const unsigned long long* t) {
    return __hip_atomic_load(t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Decoupled look-back of tile `tile` with aggregate `total`, run by one
// whole wave: publishes the aggregate, then looks back over the 64
// preceding tiles at a time (one read per lane) and adds the aggregates
// down to the nearest inclusive prefix, publishes its own inclusive prefix
// and returns the exclusive prefix (in every lane).  The wait on an earlier
// tile is bounded (kLookbackSpins polls); on expiry ST_SCAN_STALL is raised
// and the wave goes on, so every wave exits.
__device__ __forceinline__ long long lookback_exclusive(unsigned long long* tiles, int64_t tile,
                                                        long long total,
                                                        unsigned long long* status) {
    const int lane = lane_id();
    long long excl = 0;
    if (tile > 0) {
        if (lane == 0) tile_publish(tiles + tile, kTileAggregate | (unsigned long long)total);
        for (int64_t hi = tile - 1;; hi -= kWave) {
            const int64_t t = hi - lane;
            // tiles before the first count as an inclusive prefix of 0
            unsigned long long w = t >= 0 ? tile_read(tiles + t) : kTilePrefix;
            for (int spin = 0; spin < kLookbackSpins; ++spin) {
                if (!__builtin_amdgcn_ballot_w64((w >> 62) == 0)) break;
                __builtin_amdgcn_s_sleep(1);
                if ((w >> 62) == 0) w = tile_read(tiles + t);
            }
            if (__builtin_amdgcn_ballot_w64((w >> 62) == 0)) {
                if (lane == 0) atomicOr(status + SS_FLAGS, ST_SCAN_STALL);
                break;
            }
            const unsigned long long pm =
                __builtin_amdgcn_ballot_w64((w & ~kTileValue) == kTilePrefix);
            const int stop = pm ? __builtin_ctzll(pm) : kWave - 1;
            long long part = lane <= stop ? (long long)(w & kTileValue) : 0;
#pragma unroll
            for (int d = kWave / 2; d > 0; d >>= 1) part += __shfl_xor(part, d);
            excl += part;
            if (pm) break;
        }
    }
    if (lane == 0) tile_publish(tiles + tile, kTilePrefix | (unsigned long long)(excl + total));
    return excl;
}

// Exclusive scan of n (min(n, *n_dev) when n_dev is given) non-negative values of
// `in` (which holds at least one element) into out[0..n], out[n] = total, in
// one launch.  Blocks take tiles of
// kScanTile items in the order they start (an atomic ticket), so every
// earlier tile belongs to a block that is already running; a block publishes
// its tile aggregate, then its first wave looks back over the 64 preceding
// tiles at a time (one read per lane) and adds the aggregates down to the
// nearest inclusive prefix (decoupled look-back).  The wait on an earlier
// tile is bounded (kLookbackSpins polls); on expiry the block raises
// ST_SCAN_STALL and finishes, so every wave exits.  `tiles` must hold zeros
// and `ticket` zero.  When total_slot is given the total is also stored there,
// and when host_out is given the block of the last tile then copies the
// first kHostResultSlots status words (total included) into it: the caller's
// pinned host buffer, which the caller reads after synchronising with the
// stream.
template <typename In, typename Out>
__device__ __forceinline__ void scan_lookback_block(const In* in, int64_t n,
                                                    const unsigned long long* n_dev, Out* out,
                                                    unsigned long long* tiles,
                                                    unsigned long long* ticket,
                                                    unsigned long long* status,
                                                    unsigned long long* total_slot,
                                                    long long* host_out) {
    __shared__ long long s_tile, s_excl;
    if (n_dev) n = min(n, (int64_t)*n_dev);
    const int64_t ntiles = n > 0 ? (n + kScanTile - 1) / kScanTile : 1;
    // blocks beyond the tiles (a grid sized for a capacity) leave without a
    // ticket; the first ntiles blocks take tickets 0 .. ntiles - 1
    if ((int64_t)blockIdx.x >= ntiles) return;
    if (threadIdx.x == 0) s_tile = (long long)atomicAdd(ticket, 1ull);
    __syncthreads();
    const int64_t tile = s_tile;
    const int64_t base = tile * kScanTile + (int64_t)threadIdx.x * kTileItems;
    // every load is issued before the first is used (slots past n re-read
    // in[0], which every caller's input holds, and count as 0)
    In raw[kTileItems];
#pragma unroll
    for (int k = 0; k < kTileItems; ++k) raw[k] = in[base + k < n ? base + k : 0];
    long long v[kTileItems];
    long long s = 0;
#pragma unroll
    for (int k = 0; k < kTileItems; ++k) {
        v[k] = base + k < n ? (long long)raw[k] : 0;
        s += v[k];
    }
    long long total;
    const long long ex = block_exclusive_scan(s, &total);
    if (threadIdx.x < kWave) {
        const long long excl = lookback_exclusive(tiles, tile, total, status);
        if (lane_id() == 0) s_excl = excl;
    }
    __syncthreads();
    long long run = s_excl + ex;
#pragma unroll
    for (int k = 0; k < kTileItems; ++k) {
        const int64_t i = base + k;
        if (i < n) out[i] = (Out)run;
        run += v[k];
    }
    if (tile == ntiles - 1 && threadIdx.x == 0) {
        out[n] = (Out)(s_excl + total);
        if (total_slot) *total_slot = (unsigned long long)(s_excl + total);
        if (host_out) {
#pragma unroll
            for (int k = 0; k < kHostResultSlots; ++k)
                host_out[k] = (long long)__hip_atomic_load(status + k, __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

template <typename In, typename Out>
__global__ __launch_bounds__(kBlock) void k_scan_lookback(const In* in, int64_t n,
                                                           const unsigned long long* n_dev,
                                                           Out* out, unsigned long long* tiles,
                                                           unsigned long long* ticket,
                                                           unsigned long long* status,
                                                           unsigned long long* total_slot,
                                                           long long* host_out = nullptr) {
    scan_lookback_block<In, Out>(in, n, n_dev, out, tiles, ticket, status, total_slot, host_out);
}

// The summary of record r for the batch scan.
__device__ __forceinline__ void write_summary(PlanSummary* s, const StructRec& r) {
    PlanSummary x;
    x.flags = r.flags;
    x.img_total = r.img_total;
    x.natoms = r.natoms;
    x.kind = (long long)r.algo | (r.any_wrap ? 1ll << 8 : 0ll) |
             (molecule_rec(r) ? 1ll << 9 : 0ll);
    *s = x;
}

// One workgroup, from the plans' summaries (meta): exclusive scans of the
// bins and of the brute-force work units per structure into bin_off and
// unit_off ([0..nb]; each structure's first bin and unit also go to its
// record), of the brute-force atoms (each brute-force structure's hit-mask
// slots, counted down from n_atoms, go to its record), their totals, and
// the batch checks that need every structure's plan: total periodic images,
// bin capacity and, for a count launched without the cell-list kernels
// (brute_hint), the absence of cell-list structures.  Every load of a chunk
// is issued at once (indices clamped to the last structure, values masked),
// and the batch reductions go through wave reductions and one LDS slot per
// wave, without atomics.
__device__ __forceinline__ void struct_scan_block(const long long* struct_bins,
                                                  const long long* struct_units,
                                                  const PlanSummary* meta, int64_t nb,
                                                  int64_t n_atoms, long long* bin_off,
                                                  long long* unit_off, StructRec* recs,
                                                  unsigned long long* status, int64_t cap_bins,
                                                  int brute_hint) {
    __shared__ long long s_carry, s_ucarry, s_mcarry;
    __shared__ unsigned long long s_red[4][kWavesPerBlock];
    if (threadIdx.x == 0) {
        s_carry = 0;
        s_ucarry = 0;
        s_mcarry = 0;
    }
    __syncthreads();
    unsigned long long flags = 0, plan = 0, images = 0, wrap = 0, nonmol = 0;
    for (int64_t base = 0; base < nb; base += kScanChunk) {
        const int64_t i0 = base + (int64_t)threadIdx.x * kScanItems;
        // every load of the chunk is issued before the first is used
        // (indices clamped to the last structure, values masked below)
        PlanSummary sm[kScanItems];
        long long bv[kScanItems], uv[kScanItems];
#pragma unroll
        for (int k = 0; k < kScanItems; ++k) {
            const int64_t ic = i0 + k < nb ? i0 + k : nb - 1;
            sm[k] = meta[ic];
            bv[k] = struct_bins[ic];
            uv[k] = struct_units[ic];
        }
        long long v[kScanItems], u[kScanItems], m[kScanItems];
        long long sum = 0, usum = 0, msum = 0;
#pragma unroll
        for (int k = 0; k < kScanItems; ++k) {
            const bool in = i0 + k < nb;
            const unsigned long long fl = sm[k].flags;
            const int algo = (int)(sm[k].kind & 0xff);
            const bool aw = (sm[k].kind >> 8) & 1, mol = (sm[k].kind >> 9) & 1;
            const long long img = sm[k].img_total, na = sm[k].natoms;
            v[k] = in ? bv[k] : 0;
            u[k] = in ? uv[k] : 0;
            m[k] = in && algo == ALGO_BRUTE ? na : 0;
            sum += v[k];
            usum += u[k];
            msum += m[k];
            flags |= in ? fl : 0ull;
            plan |= !in ? 0ull : (algo == ALGO_CELL ? 2ull : (algo == ALGO_BRUTE ? 1ull : 0ull));
            wrap |= in && algo == ALGO_CELL && aw ? 1ull : 0ull;
            nonmol |= in && algo == ALGO_BRUTE && !mol ? 1ull : 0ull;
            images += in ? (unsigned long long)img : 0ull;
        }
        long long tot, utot, mtot;
        long long run = block_exclusive_scan(sum, &tot) + s_carry;
        long long urun = block_exclusive_scan(usum, &utot) + s_ucarry;
        long long mrun = block_exclusive_scan(msum, &mtot) + s_mcarry;
#pragma unroll
        for (int k = 0; k < kScanItems; ++k) {
            const int64_t i = i0 + k;
            mrun += m[k];
            if (i < nb) {
                bin_off[i] = run;
                recs[i].bin0 = run;
                unit_off[i] = urun;
                recs[i].unit0 = urun;
                recs[i].mask0 = n_atoms - mrun;
            }
            run += v[k];
            urun += u[k];
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            s_carry += tot;
            s_ucarry += utot;
            s_mcarry += mtot;
        }
        __syncthreads();
    }
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1) {
        flags |= __shfl_xor(flags, d);
        plan |= __shfl_xor(plan, d);
        wrap |= __shfl_xor(wrap, d);
        nonmol |= __shfl_xor(nonmol, d);
        images += __shfl_xor(images, d);
    }
    const int w = threadIdx.x / kWave;
    if (lane_id() == 0) {
        s_red[0][w] = flags;
        s_red[1][w] = plan;
        s_red[2][w] = images;
        s_red[3][w] = wrap | (nonmol << 1);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long all_flags = 0, all_plan = 0, all_images = 0, all_wrap = 0;
#pragma unroll
        for (int x = 0; x < kWavesPerBlock; ++x) {
            all_flags |= s_red[0][x];
            all_plan |= s_red[1][x];
            all_images += s_red[2][x];
            all_wrap |= s_red[3][x];
        }
        const long long total = s_carry;
        bin_off[nb] = total;
        unit_off[nb] = s_ucarry;
        status[SS_TOTAL_BINS] = (unsigned long long)total;
        status[SS_TOTAL_UNITS] = (unsigned long long)s_ucarry;
        status[SS_PLAN] =
            all_plan | ((all_plan & 1ull) && !(all_wrap & 2ull) ? kPlanMolecules : 0ull);
        status[SS_TOTAL_IMAGES] = all_images;
        status[SS_ANY_WRAP] = all_wrap & 1ull;
        unsigned long long st = all_flags;
        if (total > cap_bins) st |= ST_CAPACITY;
        if (all_images > (unsigned long long)kImageCap) st |= ST_BATCH_IMAGE_CAP;
        if (brute_hint && (all_plan & 2ull)) st |= ST_PLAN_HINT;
        if (st) atomicOr(status + SS_FLAGS, st);
    }
}

}  // namespace tnr
