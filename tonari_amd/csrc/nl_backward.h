// Backward of the fused d/D outputs: the gradients of positions and cell
// from the gradients of D (pairs x 3) and d (pairs), for the pairs written by
// the emitting kernels.  It replaces the autograd of the reference's Torch
// expression (src/tonari/_torch_frontend.py:92-104)
//   D_e = pos[j_e] - pos[i_e] + S_e @ cell[b_e],   d_e = |D_e|,
// whose gradient is, with g_e = dL/dD_e + dL/dd_e * D_e / d_e (0 when
// d_e = 0, as torch's vector_norm backward):
//   dL/dpos[j_e] += g_e,  dL/dpos[i_e] -= g_e,  dL/dcell[b_e][a][c] += S_e[a] g_e[c].
//
// One thread per pair, each wave a contiguous range of pairs.  The pairs of
// a source are contiguous, so the source side is reduced per run of equal
// sources inside a wave (segmented scan) and added once per run.  The target
// side is accumulated in an LDS hash table of the workgroup (open
// addressing, keyed by target atom, LDS atomics) and added to grad_pos once
// per distinct target at the end: the targets of a workgroup's consecutive
// pairs are few when the list comes in bin order (a few hundred stencil
// atoms for 8,192 pairs), where one global atomic per pair and component
// serialised (27 M on a 100,000-atom list: 1.25 ms of a 1.39 ms kernel).
// A target that finds no slot within kBwdProbes probes takes the global
// atomics directly.  The pairs of a structure are
// contiguous too (sources come in index or bin order, both grouped by
// structure), so each wave keeps a running sum of the cell gradient of its
// current structure, adds it when the structure changes, and the waves of
// a block merge their last sums: a structure's 9 entries take a few atomics
// per block, not per pair.  Float atomics make the summation order vary
// between runs (the same holds for torch's index_add on the device).
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

constexpr int kBwdSlots = 2048;  // LDS hash slots per workgroup (power of two)
constexpr int kBwdProbes = 8;
constexpr int kBwdPairsPerBlock = 8192;  // the launcher's grid: at most this many pairs per workgroup

template <typename T>
__global__ __launch_bounds__(kBlock) void k_geometry_backward(
    int64_t n_pairs, int64_t nb, const int64_t* bp, const int64_t* pairs, const int32_t* shifts,
    const T* vec, const T* dist, const T* grad_vec, const T* grad_dist, T* grad_pos,
    T* grad_cell) {
    __shared__ T s_acc[kWavesPerBlock][9];
    __shared__ int s_b[kWavesPerBlock];
    __shared__ int s_key[kBwdSlots];
    __shared__ T s_val[3][kBwdSlots];
    for (int i = threadIdx.x; i < kBwdSlots; i += kBlock) {
        s_key[i] = -1;
        s_val[0][i] = s_val[1][i] = s_val[2][i] = T(0);
    }
    __syncthreads();
    const int lane = lane_id();
    const int wv = uniform(threadIdx.x / kWave);
    // a contiguous range of pairs per wave
    const int64_t nwaves = (int64_t)gridDim.x * kWavesPerBlock;
    const int64_t per = ((n_pairs + nwaves - 1) / nwaves + kWave - 1) / kWave * kWave;
    const int64_t w_lo = min(((int64_t)blockIdx.x * kWavesPerBlock + wv) * per, n_pairs);
    const int64_t w_hi = min(w_lo + per, n_pairs);
    // per-lane partial cell-gradient sums of structure cur_b (wave-uniform)
    T acc[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) acc[k] = T(0);
    int cur_b = -1;
    // adds the wave's sums of structure cur_b to grad_cell (lanes 0..8)
    auto flush = [&]() {
        if (cur_b < 0) return;
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            T x = acc[k];
#pragma unroll
            for (int d = kWave / 2; d > 0; d >>= 1) x += __shfl_xor(x, d);
            if (lane == k) unsafeAtomicAdd(grad_cell + 9 * cur_b + k, x);
            acc[k] = T(0);
        }
    };
    for (int64_t e0 = w_lo; e0 < w_hi; e0 += kWave) {
        const int64_t e = e0 + lane;
        const bool valid = e < w_hi;
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
        // target side: the workgroup's hash table, else global atomics
        if (valid) {
            const int key = (int)t;
            unsigned h = ((unsigned)key * 2654435761u) >> (32 - 11);
            static_assert(kBwdSlots == 1 << 11, "hash width");
            bool placed = false;
            for (int p = 0; p < kBwdProbes; ++p) {
                const int old = atomicCAS(&s_key[h], -1, key);
                if (old == -1 || old == key) {
#pragma unroll
                    for (int c = 0; c < 3; ++c) atomicAdd(&s_val[c][h], g[c]);
                    placed = true;
                    break;
                }
                h = (h + 1) & (kBwdSlots - 1);
            }
            if (!placed) {
#pragma unroll
                for (int c = 0; c < 3; ++c) unsafeAtomicAdd(grad_pos + 3 * t + c, g[c]);
            }
        }
        const unsigned long long le = lane == kWave - 1 ? ~0ull : ((2ull << lane) - 1ull);
        // source side: runs of equal sources
        {
            const long long sp = __shfl_up(s, 1);
            const unsigned long long heads = ballot(lane == 0 || sp != s);
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
        // cell side: lanes of structure cur_b add to their partial sums; a
        // round that holds another structure (rare: the pairs of a structure
        // are contiguous) flushes the sums and takes that structure's runs
        // one by one
        {
            T v[9];
#pragma unroll
            for (int a = 0; a < 3; ++a)
#pragma unroll
                for (int c = 0; c < 3; ++c) v[3 * a + c] = (T)S[a] * g[c];
            if (ballot(valid && b != cur_b) == 0) {
#pragma unroll
                for (int k = 0; k < 9; ++k) acc[k] += v[k];
            } else {
                flush();
                // runs of equal structures: all but the last are added now,
                // the last one becomes the running structure
                const int bpv = __shfl_up(b, 1);
                const unsigned long long heads = ballot(lane == 0 || bpv != b);
                const unsigned long long vmask = ballot(valid);
                const int last_valid = 63 - __builtin_clzll(vmask);
                const int b_last = __builtin_amdgcn_readfirstlane(__shfl(b, last_valid));
                const int seg0 = 63 - __builtin_clzll(heads & le);
                const bool tail = valid && lane != last_valid &&
                                  (lane == kWave - 1 || ((heads >> (lane + 1)) & 1ull)) &&
                                  b != b_last;
#pragma unroll
                for (int k = 0; k < 9; ++k) {
                    const T x = segment_inclusive_sum(v[k], seg0);
                    if (tail) unsafeAtomicAdd(grad_cell + 9 * b + k, x);
                    acc[k] = valid && b == b_last ? v[k] : T(0);
                }
                cur_b = b_last;
            }
        }
    }
    // the block's waves merge their last sums when they share a structure
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        T x = acc[k];
#pragma unroll
        for (int d = kWave / 2; d > 0; d >>= 1) x += __shfl_xor(x, d);
        if (lane == k) s_acc[wv][k] = x;
    }
    if (lane == 0) s_b[wv] = cur_b;
    __syncthreads();
    // the table's targets, once each
    for (int i = threadIdx.x; i < kBwdSlots; i += kBlock) {
        const int key = s_key[i];
        if (key < 0) continue;
#pragma unroll
        for (int c = 0; c < 3; ++c) unsafeAtomicAdd(grad_pos + 3 * (int64_t)key + c, s_val[c][i]);
    }
    if (threadIdx.x < 9) {
        const int k = threadIdx.x;
        for (int w = 0; w < kWavesPerBlock; ++w) {
            const int bw = s_b[w];
            if (bw < 0) continue;
            bool first = true;
            for (int u = 0; u < w; ++u) first = first && s_b[u] != bw;
            if (!first) continue;
            T sum = T(0);
            for (int u = w; u < kWavesPerBlock; ++u)
                if (s_b[u] == bw) sum += s_acc[u][k];
            unsafeAtomicAdd(grad_cell + 9 * bw + k, sum);
        }
    }
}

}  // namespace tnr
