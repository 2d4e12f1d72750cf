// Backward of the fused d/D outputs: the gradients of positions and cell
// from the gradients of D (pairs x 3) and d (pairs), for the pairs written by
// the emitting kernels.  It replaces the autograd of the reference's Torch
// expression (src/tonari/_torch_frontend.py:92-104)
//   D_e = pos[j_e] - pos[i_e] + S_e @ cell[b_e],   d_e = |D_e|,
// whose gradient is, with g_e = dL/dD_e + dL/dd_e * D_e / d_e (0 when
// d_e = 0, as torch's vector_norm backward):
//   dL/dpos[j_e] += g_e,  dL/dpos[i_e] -= g_e,  dL/dcell[b_e][a][c] += S_e[a] g_e[c].
//
// One thread per pair.  The pairs of a source are contiguous, so the source
// side is reduced per run of equal sources inside a wave (segmented scan) and
// added once per run; the target side takes one atomic add per component;
// the cell side is reduced per run of equal structures and added once per
// run (9 atomics).  Float atomics make the summation order vary between runs
// (the same holds for torch's index_add on the device).
#pragma once

#include "nl_math.h"

namespace tnr {

// Inclusive sum over the lanes of the calling lane's segment up to it; seg0
// is the first lane of that segment (every lane active).
template <typename V>
__device__ __forceinline__ V segment_inclusive_sum(V x, int seg0) {
    const int lane = lane_id();
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const V y = __shfl_up(x, d);
        if (lane - d >= seg0) x += y;
    }
    return x;
}

template <typename T>
__global__ __launch_bounds__(kBlock) void k_geometry_backward(
    int64_t n_pairs, int64_t nb, const int64_t* bp, const int64_t* pairs, const int32_t* shifts,
    const T* vec, const T* dist, const T* grad_vec, const T* grad_dist, T* grad_pos,
    T* grad_cell) {
    const int lane = lane_id();
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t e0 = (int64_t)blockIdx.x * kBlock; e0 < n_pairs; e0 += stride) {
        const int64_t e = e0 + threadIdx.x;
        const bool valid = e < n_pairs;
        long long s = -1 - lane, t = 0;  // invalid lanes: keys no other lane has
        int b = -1 - lane;
        T g[3] = {T(0), T(0), T(0)};
        int S[3] = {0, 0, 0};
        if (valid) {
            const long2 st = *reinterpret_cast<const long2*>(pairs + 2 * e);
            s = st.x;
            t = st.y;
#pragma unroll
            for (int c = 0; c < 3; ++c) S[c] = shifts[3 * e + c];
            if (grad_vec) {
#pragma unroll
                for (int c = 0; c < 3; ++c) g[c] = grad_vec[3 * e + c];
            }
            if (grad_dist) {
                const T gd = grad_dist[e], d = dist[e];
                if (d != T(0)) {
                    const T k = gd / d;
#pragma unroll
                    for (int c = 0; c < 3; ++c) g[c] += k * vec[3 * e + c];
                }
            }
            // structure of the source: the b with bp[b] <= s < bp[b + 1]
            int64_t lo = 0, hi = nb;
            while (hi - lo > 1) {
                const int64_t mid = (lo + hi) >> 1;
                if (bp[mid] <= s) lo = mid; else hi = mid;
            }
            b = (int)lo;
        }
        // target side
        if (valid) {
#pragma unroll
            for (int c = 0; c < 3; ++c) unsafeAtomicAdd(grad_pos + 3 * t + c, g[c]);
        }
        // source side: runs of equal sources
        {
            const long long sp = __shfl_up(s, 1);
            const unsigned long long heads = ballot(lane == 0 || sp != s);
            const unsigned long long le = lane == kWave - 1 ? ~0ull : ((2ull << lane) - 1ull);
            const int seg0 = 63 - __builtin_clzll(heads & le);
            const bool tail = lane == kWave - 1 || ((heads >> (lane + 1)) & 1ull);
            T sum[3];
#pragma unroll
            for (int c = 0; c < 3; ++c) sum[c] = segment_inclusive_sum(g[c], seg0);
            if (valid && tail) {
#pragma unroll
                for (int c = 0; c < 3; ++c) unsafeAtomicAdd(grad_pos + 3 * s + c, -sum[c]);
            }
        }
        // cell side: runs of equal structures
        {
            const int bpv = __shfl_up(b, 1);
            const unsigned long long heads = ballot(lane == 0 || bpv != b);
            const unsigned long long le = lane == kWave - 1 ? ~0ull : ((2ull << lane) - 1ull);
            const int seg0 = 63 - __builtin_clzll(heads & le);
            const bool tail = lane == kWave - 1 || ((heads >> (lane + 1)) & 1ull);
#pragma unroll
            for (int a = 0; a < 3; ++a) {
#pragma unroll
                for (int c = 0; c < 3; ++c) {
                    const T v = segment_inclusive_sum((T)S[a] * g[c], seg0);
                    if (valid && tail) unsafeAtomicAdd(grad_cell + 9 * b + 3 * a + c, v);
                }
            }
        }
    }
}

}  // namespace tnr
