// Device-wide exclusive scans: a single-pass scan with decoupled look-back
// (k_scan_lookback), the one-block scan of the bins per structure
// (k_struct_scan), the three-kernel scan (reduce, scan of block totals,
// apply) and small fill kernels.
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

// ------------------------------------------------------------- fill / scan

__global__ void k_fill_i64(long long* p, int64_t n, long long v) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

__global__ void k_fill_i32(int* p, int64_t n, int v) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

template <typename In>
__global__ __launch_bounds__(kBlock) void k_scan_reduce(const In* in, int64_t n,
                                                         long long* partial) {
    const int64_t base = (int64_t)blockIdx.x * kScanChunk;
    long long s = 0;
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        const int64_t i = base + threadIdx.x + (int64_t)j * kBlock;
        if (i < n) s += (long long)in[i];
    }
    long long total;
    block_exclusive_scan(s, &total);
    if (threadIdx.x == 0) partial[blockIdx.x] = total;
}

// One block: exclusive scan of partial[0..np) in place, partial[np] = total.
__global__ __launch_bounds__(kBlock) void k_scan_partials(long long* partial, int64_t np) {
    __shared__ long long carry_s;
    if (threadIdx.x == 0) carry_s = 0;
    __syncthreads();
    for (int64_t base = 0; base < np; base += kBlock) {
        const int64_t i = base + threadIdx.x;
        const long long v = i < np ? partial[i] : 0;
        long long total;
        const long long ex = block_exclusive_scan(v, &total);
        const long long carry = carry_s;
        if (i < np) partial[i] = carry + ex;
        __syncthreads();
        if (threadIdx.x == 0) carry_s = carry + total;
        __syncthreads();
    }
    if (threadIdx.x == 0) partial[np] = carry_s;
}

template <typename In, typename Out>
__global__ __launch_bounds__(kBlock) void k_scan_apply(const In* in, int64_t n,
                                                        const long long* partial,
                                                        int64_t np, Out* out) {
    const int64_t base = (int64_t)blockIdx.x * kScanChunk + (int64_t)threadIdx.x * kScanItems;
    long long v[kScanItems];
    long long s = 0;
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        const int64_t i = base + j;
        v[j] = i < n ? (long long)in[i] : 0;
        s += v[j];
    }
    long long total;
    long long run = block_exclusive_scan(s, &total) +
                    (blockIdx.x < np ? partial[blockIdx.x] : 0);
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        const int64_t i = base + j;
        if (i < n) out[i] = (Out)run;
        run += v[j];
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) out[n] = (Out)partial[np];
}

// ------------------------------------------------------- single-pass scan

// Tile state of the single-pass scan: bits 62-63 hold the flag (0 not ready,
// 1 tile aggregate, 2 inclusive prefix), bits 0-61 the value.
constexpr unsigned long long kTileAggregate = 1ull << 62;
constexpr unsigned long long kTilePrefix = 2ull << 62;
constexpr unsigned long long kTileValue = (1ull << 62) - 1;
constexpr int kLookbackSpins = 1 << 22;

__device__ __forceinline__ void tile_publish(unsigned long long* t, unsigned long long w) {
    __hip_atomic_store(t, w, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long tile_read(const unsigned long long* t) {
    return __hip_atomic_load(t, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
}

// Exclusive scan of n (min(n, *n_dev) when n_dev is given) non-negative values of
// `in` into out[0..n], out[n] = total, in one launch.  Blocks take tiles of
// kScanTile items in the order they start (an atomic ticket), so every
// earlier tile belongs to a block that is already running; a block publishes
// its tile aggregate, then walks back over the earlier tiles until it meets
// an inclusive prefix (decoupled look-back).  The wait on an earlier tile is
// bounded (kLookbackSpins polls); on expiry the block raises ST_SCAN_STALL
// and finishes, so every wave exits.  `tiles` must hold zeros and `ticket`
// zero.  When total_slot is given the total is also stored there.
template <typename In, typename Out>
__global__ __launch_bounds__(kBlock) void k_scan_lookback(const In* in, int64_t n,
                                                           const unsigned long long* n_dev,
                                                           Out* out, unsigned long long* tiles,
                                                           unsigned long long* ticket,
                                                           unsigned long long* status,
                                                           unsigned long long* total_slot) {
    __shared__ long long s_tile, s_excl;
    if (threadIdx.x == 0) s_tile = (long long)atomicAdd(ticket, 1ull);
    __syncthreads();
    if (n_dev) n = min(n, (int64_t)*n_dev);
    const int64_t tile = s_tile;
    const int64_t ntiles = n > 0 ? (n + kScanTile - 1) / kScanTile : 1;
    if (tile >= ntiles) return;
    const int64_t base = tile * kScanTile + (int64_t)threadIdx.x * kScanItems;
    long long v[kScanItems];
    long long s = 0;
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        const int64_t i = base + k;
        v[k] = i < n ? (long long)in[i] : 0;
        s += v[k];
    }
    long long total;
    const long long ex = block_exclusive_scan(s, &total);
    if (threadIdx.x == 0) {
        long long excl = 0;
        if (tile > 0) {
            tile_publish(tiles + tile, kTileAggregate | (unsigned long long)total);
            for (int64_t t = tile - 1; t >= 0; --t) {
                unsigned long long w = tile_read(tiles + t);
                for (int spin = 0; (w >> 62) == 0 && spin < kLookbackSpins; ++spin) {
                    __builtin_amdgcn_s_sleep(1);
                    w = tile_read(tiles + t);
                }
                if ((w >> 62) == 0) {
                    atomicOr(status + SS_FLAGS, ST_SCAN_STALL);
                    break;
                }
                excl += (long long)(w & kTileValue);
                if ((w & ~kTileValue) == kTilePrefix) break;
            }
        }
        tile_publish(tiles + tile, kTilePrefix | (unsigned long long)(excl + total));
        s_excl = excl;
    }
    __syncthreads();
    long long run = s_excl + ex;
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        const int64_t i = base + k;
        if (i < n) out[i] = (Out)run;
        run += v[k];
    }
    if (tile == ntiles - 1 && threadIdx.x == 0) {
        out[n] = (Out)(s_excl + total);
        if (total_slot) *total_slot = (unsigned long long)(s_excl + total);
    }
}

// One block: exclusive scans of the bins, the emitting tasks and the
// counting tasks per structure into bin_off, task_off and ctask_off
// ([0..nb]; each structure's first bin and tasks go to its record), their
// totals, and the batch checks that need every structure's plan: total
// periodic images and bin capacity.
__global__ __launch_bounds__(kBlock) void k_struct_scan(const long long* struct_bins,
                                                         const long long* struct_tasks,
                                                         const long long* struct_ctasks,
                                                         int64_t nb, long long* bin_off,
                                                         long long* task_off,
                                                         long long* ctask_off, StructRec* recs,
                                                         unsigned long long* status,
                                                         int64_t cap_bins) {
    __shared__ long long carry[3];
    if (threadIdx.x < 3) carry[threadIdx.x] = 0;
    __syncthreads();
    const long long* in[3] = {struct_bins, struct_tasks, struct_ctasks};
    long long* out[3] = {bin_off, task_off, ctask_off};
    for (int64_t base = 0; base < nb; base += kScanChunk) {
        const int64_t i0 = base + (int64_t)threadIdx.x * kScanItems;
#pragma unroll
        for (int q = 0; q < 3; ++q) {
            long long v[kScanItems];
            long long sum = 0;
#pragma unroll
            for (int k = 0; k < kScanItems; ++k) {
                v[k] = i0 + k < nb ? in[q][i0 + k] : 0;
                sum += v[k];
            }
            long long tot;
            long long run = block_exclusive_scan(sum, &tot) + carry[q];
#pragma unroll
            for (int k = 0; k < kScanItems; ++k) {
                if (i0 + k < nb) {
                    out[q][i0 + k] = run;
                    if (q == 0) recs[i0 + k].bin0 = run;
                    if (q == 1) recs[i0 + k].task0 = run;
                    if (q == 2) recs[i0 + k].ctask0 = run;
                }
                run += v[k];
            }
            __syncthreads();
            if (threadIdx.x == 0) carry[q] += tot;
            __syncthreads();
        }
    }
    if (threadIdx.x == 0) {
#pragma unroll
        for (int q = 0; q < 3; ++q) out[q][nb] = carry[q];
        status[SS_TOTAL_BINS] = (unsigned long long)carry[0];
        status[SS_TOTAL_TASKS] = (unsigned long long)carry[1];
        status[SS_TOTAL_CTASKS] = (unsigned long long)carry[2];
        unsigned long long st = 0;
        if (carry[0] > cap_bins) st |= ST_CAPACITY;
        if (status[SS_TOTAL_IMAGES] > (unsigned long long)kImageCap) st |= ST_BATCH_IMAGE_CAP;
        if (st) atomicOr(status + SS_FLAGS, st);
    }
}

template <typename In, typename Out>
static hipError_t device_scan(const In* in, int64_t n, Out* out, long long* partial,
                              hipStream_t stream) {
    const int64_t np = (n + kScanChunk - 1) / kScanChunk;
    if (np > 0) k_scan_reduce<In><<<dim3((unsigned)np), dim3(kBlock), 0, stream>>>(in, n, partial);
    k_scan_partials<<<1, kBlock, 0, stream>>>(partial, np);
    k_scan_apply<In, Out><<<dim3((unsigned)(np > 0 ? np : 1)), dim3(kBlock), 0, stream>>>(
        in, n, partial, np, out);
    return hipGetLastError();
}

}  // namespace tnr
