// Device-wide exclusive scans (reduce, scan of block totals, apply) and
// small fill kernels.
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
