// Counting pass of the cell-list structures: pairs per source and the hit
// masks the emitting pass replays (k_cell_count).
//
// Work unit: one source bin per wave.  A wave builds its bin's stencil on
// its own (no workgroup barrier): the neighbouring bins with their periodic
// images cut into pieces (stencil_piece_rows), their lengths scanned across
// the lanes, and the piece tables written to the wave's slice of LDS.  Lane
// l then takes the candidates l * nch + j of the chunks j it holds (the
// interleave chunk_cand shares with the emitting pass), loads their records
// straight from the binned array into registers and adds the piece's image
// translation.  The bin's sources are broadcast one at a time and tested
// against every chunk: per chunk and source, six VALU operations
// for the broad-phase distance, two compares whose lane masks land in scalar
// registers, and two lane writes that assemble the 64-bit hit masks of the
// chunks for one vector store.  Identity, self exclusion and the band
// between the broad-phase thresholds are scalar mask operations; candidates
// in the band are decided by the public predicate (cell_band), rarely.
//
// Reference: the counting flavour of the cell-list query,
// csrc/torch/neighbors_cell_cuda.cu:294-442 (one warp per source walking
// linked lists of image nodes), and csrc/core/neighbors_cpu.cpp:515-584.
#pragma once

#include "nl_cell.h"

namespace tnr {

// Chunks of 64 candidates a counting wave holds in registers (one pass);
// stencils with more chunks take several passes.
template <typename T>
struct CountChunks;
template <>
struct CountChunks<float> {
    static constexpr int value = 12;
};
template <>
struct CountChunks<double> {
    static constexpr int value = 8;
};

// Counting tasks per bin: the bin's sources are split into this many equal
// parts, one wave each, and each part builds the bin's stencil.  Measured:
// C4 (float32, bins of about 24 sources) 94 us with two parts against
// 97.5 us with one; C5 (float64, bins of 12 to 16 sources, a float64
// stencil costing more to build) 0.66 ms with one against 0.72 ms with two.
template <typename T>
struct CountParts;
template <>
struct CountParts<float> {
    static constexpr int value = 2;
};
template <>
struct CountParts<double> {
    static constexpr int value = 1;
};

// Stencil tables of one counting wave's bin.
template <typename T>
struct WaveStencil {
    int pre[kPieceCap + 1];        // exclusive prefix of piece lengths
    int delta[kPieceCap];          // binned index = candidate index + delta
    int kid[kPieceCap];            // packed image shift (pack_k)
    T tr[3][kPieceCap];            // broad-phase translation of the piece's image
    unsigned char kfl[kPieceCap];  // bit 0: k == 0, bit 1: k < 0 (lexicographic)
};

// Per-wave LDS of the counting kernel: the stencil tables, or the
// per-source cursors of a brute-force work unit.
template <typename T>
union CountLds {
    WaveStencil<T> st;
    BruteCursor cur;
};

// Builds the stencil of global bin g with one wave: the bin's geometry and
// thresholds into cb, the piece tables into st.  Returns false when the bin
// holds no source.
template <typename T>
__device__ __forceinline__ bool wave_bin(const QueryArgs<T>& a, int64_t g, StructCache& sc,
                                         CellBin<T>& cb, WaveStencil<T>& st) {
    const int lane = lane_id();
    // the bin's sources load with the structure search
    const int sb_raw = a.bin_start[g], se_raw = a.bin_start[g + 1];
    cb.b = structure_of_item(a.struct_bin_off, a.nb, g, sc);
    const StructRec& r = a.recs[cb.b];
    const unsigned lbin = (unsigned)(g - r.bin0);  // bins of a structure fit in 32 bits
    cb.sb = uniform(sb_raw);
    cb.se = uniform(se_raw);
    if (cb.sb >= cb.se) return false;
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
    cb.diagonal = r.diagonal != 0;
    cb.by_bin = a.by_bin && (load_status(a.status + SS_PLAN) & kPlanFamilies) == 2ull;
    const BinGeom G = bin_geom(r, lbin);
    cb.npieces = G.npieces;  // at most kPieceCap
    const int* bstart = a.bin_start + r.bin0;
    // earlier reads of the tables (the previous bin) are done
    wave_lds_fence();
    int total = 0;
    for (int p0 = 0; p0 < G.npieces; p0 += kWave) {
        const int p = p0 + lane;
        int kx = 0, ky = 0, kz = 0, i0 = 0, i1 = 0;
        const bool pok = p < G.npieces && stencil_piece_rows(G, p, i0, i1, kx, ky, kz);
        const int start = bstart[i0];
        const int len = pok ? bstart[i1] - start : 0;
        const int inc = wave_inclusive_scan_i32(len);
        if (p < G.npieces) {
            const int ex = total + inc - len;
            const int kk = pack_k(kx, ky, kz);
            st.pre[p] = ex;
            st.delta[p] = start - ex;
            st.kid[p] = kk;
            st.kfl[p] = (unsigned char)((kx == 0 && ky == 0 && kz == 0 ? 1 : 0) |
                                        (lex_negative(kx, ky, kz) ? 2 : 0));
            image_translation(kk, cb.c, st.tr[0][p], st.tr[1][p], st.tr[2][p]);
        }
        total += __builtin_amdgcn_readlane(inc, kWave - 1);
    }
    if (lane == 0) st.pre[G.npieces] = total;
    cb.C = uniform(total);
    cb.nch = (cb.C + kWave - 1) / kWave;
    wave_lds_fence();
    // the bin itself with image 0: row (Kx, Ky), the z segment with kz = 0
    cb.dself = uniform(st.delta[(G.Kx * G.RY + (G.RY >> 1)) * G.zs + (G.perz ? -G.kz0 : 0)]);
    return true;
}

// band |= 1 << J when mk has a lane that mi has not: three scalar
// operations (s_andn2_b64 sets SCC when its result is nonzero).
template <int J>
__device__ __forceinline__ void band_flag(unsigned long long mk, unsigned long long mi,
                                          unsigned& band) {
    unsigned long long t;
    unsigned x;
    asm volatile(
        "s_andn2_b64 %[t], %[mk], %[mi]\n\t"
        "s_cselect_b32 %[x], %[bit], 0\n\t"
        "s_or_b32 %[band], %[band], %[x]"
        : [t] "=&s"(t), [x] "=&s"(x), [band] "+s"(band)
        : [mk] "s"(mk), [mi] "s"(mi), [bit] "i"(1u << J)
        : "scc");
}

// Candidates of one register pass: NC chunks from chunk c0 of the stencil,
// lane l of chunk j holding candidate chunk_cand(c0 + j, l, nch).  Slots past
// the last candidate hold a far position that fails every test.
template <typename T, int NC>
struct WaveChunks {
    T x[NC], y[NC], z[NC];  // image positions (broad phase)
    unsigned key[NC];       // identity keys (half lists)
};

// Image position (broad phase) and identity key of candidate v < C.
template <typename T, int MODE>
__device__ __forceinline__ void candidate_at(const QueryArgs<T>& a, const WaveStencil<T>& st,
                                             int v, int p, T& x, T& y, T& z, unsigned& key,
                                             Vec4<T>* rec_out = nullptr) {
    using O = Ops<T>;
    const Vec4<T> rec = a.binned[v + st.delta[p]];
    if constexpr (MODE >= 2) {
        const int f = st.kfl[p];
        key = identity_key<MODE>(as_idx(rec.w), (f & 1) != 0, (f & 2) != 0);
    }
    x = O::add(rec.x, st.tr[0][p]);
    y = O::add(rec.y, st.tr[1][p]);
    z = O::add(rec.z, st.tr[2][p]);
    if (rec_out) *rec_out = rec;
}

template <typename T, int MODE, int NC>
__device__ __forceinline__ void wave_gather(const QueryArgs<T>& a, const WaveStencil<T>& st,
                                            const CellBin<T>& cb, int c0,
                                            WaveChunks<T, NC>& cd) {
    const int lane = lane_id();
    const T far = T(1e18);
    // the lane's candidates are consecutive: the piece of the first by
    // binary search over the piece starts, later ones by stepping forward
    const int v0 = (int)__umul24((unsigned)lane, (unsigned)cb.nch) + c0;
    int p = v0 < cb.C ? stencil_piece(st, v0, cb.npieces) : 0;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        cd.x[j] = cd.y[j] = cd.z[j] = far;
        cd.key[j] = 0u;
        const int v = v0 + j;
        if (v < cb.C) {
            while (st.pre[p + 1] <= v) ++p;
            candidate_at<T, MODE>(a, st, v, p, cd.x[j], cd.y[j], cd.z[j], cd.key[j]);
        }
    }
}

// Broad-phase distance of a candidate's image position to the source.
template <typename T>
__device__ __forceinline__ T broad_d2(T x, T y, T z, T sx, T sy, T sz) {
    using O = Ops<T>;
    const T dx = O::sub(x, sx), dy = O::sub(y, sy), dz = O::sub(z, sz);
    return O::fma_(dz, dz, O::fma_(dy, dy, O::mul(dx, dx)));
}

// Candidates of chunk c0 + j between the broad-phase thresholds, for the
// source (sx, sy, sz, si): decided by the public predicate, and the ones it
// keeps added to the source's stored hit mask.  Returns how many it kept.
// Runs after a pass's source loop, when the pass's chunk registers are free.
template <typename T, int MODE>
__device__ __forceinline__ int band_fixup(const QueryArgs<T>& a, const WaveStencil<T>& st,
                                          const CellBin<T>& cb, int c0, int j, T sx, T sy, T sz,
                                          int si, int sj, int sl, unsigned long long* mask) {
    const int lane = lane_id();
    const int v = (int)__umul24((unsigned)lane, (unsigned)cb.nch) + c0 + j;
    bool ok = false;
    if (v < cb.C) {
        const int p = stencil_piece(st, v, cb.npieces);
        T x, y, z;
        unsigned key = 0;
        Vec4<T> rec;
        candidate_at<T, MODE>(a, st, v, p, x, y, z, key, &rec);
        const T d2 = broad_d2(x, y, z, sx, sy, sz);
        bool band = d2 < cb.outer2 && !(d2 < cb.inner2);
        if constexpr (MODE >= 2) band = band && identity_pass<MODE>(key, si);
        if constexpr (MODE == 0) band = band && !(j == sj && lane == sl);
        if (band) ok = cell_band(a, as_idx(rec.w), st.kid[p], rec, sx, sy, sz, si, cb);
    }
    const unsigned long long kept = __builtin_amdgcn_ballot_w64(ok);
    if (kept && lane == 0) *mask |= kept;
    return __popcll(kept);
}

// One register pass of NC chunks (from chunk c0) over the sources [sg, sg +
// ns) of the wave's bin: per source, the hit masks of the chunks go to
// masks[binned index][c0 ..] and the hit count is added to lane gi of acc.
// selfp (full list without self pairs): lane gi holds the chunk and bit of
// source gi's own candidate.  The candidates in the band between the
// thresholds are left out of the masks in the loop and decided afterwards
// (band_fixup), so the loop holds only the chunk registers.
template <typename T, int MODE, int NC>
__device__ __forceinline__ void count_pass(const QueryArgs<T>& a, const WaveStencil<T>& st,
                                           const CellBin<T>& cb, int sg, int ns, int c0,
                                           const Vec4<T>& own, int selfp, int& acc) {
    const int lane = lane_id();
    WaveChunks<T, NC> cd;
    wave_gather<T, MODE, NC>(a, st, cb, c0, cd);
    unsigned long long bandsrc = 0;  // bit gi: source gi has band candidates
    int bandv = 0;                   // lane gi: the chunks of source gi with band candidates
#pragma unroll 1
    for (int gi = 0; gi < ns; ++gi) {
        const T sx = read_lane(own.x, gi), sy = read_lane(own.y, gi), sz = read_lane(own.z, gi);
        const int si = as_idx(read_lane(own.w, gi));
        unsigned band = 0;
        int cnt = 0;
        int mlo = 0, mhi = 0;  // lane j: the two halves of the mask of chunk c0 + j
        static_for<NC>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            const T d2 = broad_d2(cd.x[j], cd.y[j], cd.z[j], sx, sy, sz);
            unsigned long long mk = __builtin_amdgcn_ballot_w64(d2 < cb.outer2);
            const unsigned long long mi = __builtin_amdgcn_ballot_w64(d2 < cb.inner2);
            // inside: within the inner threshold (and, for a half list,
            // passing identity); the band: within the outer one only
            unsigned long long m = mi;
            if constexpr (MODE >= 2) {
                mk &= __builtin_amdgcn_ballot_w64(identity_pass<MODE>(cd.key[j], si));
                m = mk & mi;
            }
            band_flag<j>(mk, mi, band);
            cnt += __popcll(m);
            mlo = write_lane<j>(mlo, (int)(unsigned)m);
            mhi = write_lane<j>(mhi, (int)(unsigned)(m >> 32));
        });
        unsigned long long mv = ((unsigned long long)(unsigned)mhi << 32) | (unsigned)mlo;
        if (band) {
            bandsrc |= 1ull << gi;
            bandv = lane == gi ? (int)band : bandv;
        }
        // full list without self pairs: the source itself, at distance 0,
        // is inside whenever the inner threshold is positive (otherwise it
        // sits in the band, where band_fixup leaves it out)
        if constexpr (MODE == 0) {
            const int sp = __builtin_amdgcn_readlane(selfp, gi);
            const int sj = (sp & 0xffff) - c0;
            if (sj >= 0 && sj < NC && cb.inner2 > T(0)) {
                --cnt;
                if (lane == sj) mv &= ~(1ull << (sp >> 16));
            }
        }
        if (lane < NC) a.masks[(int64_t)(sg + gi) * a.mask_words + c0 + lane] = mv;
        acc += lane == gi ? cnt : 0;
    }
    if (bandsrc) {
        // the masks stored above are complete before they are amended
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        for (unsigned long long bs = bandsrc; bs != 0ull; bs &= bs - 1ull) {
            const int gi = __builtin_ctzll(bs);
            const T sx = read_lane(own.x, gi), sy = read_lane(own.y, gi), sz = read_lane(own.z, gi);
            const int si = as_idx(read_lane(own.w, gi));
            int sj = -1, sl = 0;
            if constexpr (MODE == 0) {
                const int sp = __builtin_amdgcn_readlane(selfp, gi);
                sj = (sp & 0xffff) - c0;
                sl = sp >> 16;
            }
            int kept = 0;
            for (unsigned b = (unsigned)__builtin_amdgcn_readlane(bandv, gi); b != 0u; b &= b - 1u) {
                const int j = __builtin_ctz(b);
                kept += band_fixup<T, MODE>(a, st, cb, c0, j, sx, sy, sz, si, sj, sl,
                                            a.masks + (int64_t)(sg + gi) * a.mask_words + c0 + j);
            }
            acc += lane == gi ? kept : 0;
        }
    }
    if (cb.shiftcheck) {
        // kept shifts of a wrapped structure with a huge image range: each
        // must fit in int32 (read back the completed masks)
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
        for (int gi = 0; gi < ns; ++gi) {
            const int si = as_idx(read_lane(own.w, gi));
            for (int j = 0; j < NC; ++j) {
                const unsigned long long m = a.masks[(int64_t)(sg + gi) * a.mask_words + c0 + j];
                if ((m >> lane) & 1ull) {
                    const int v = (int)__umul24((unsigned)lane, (unsigned)cb.nch) + c0 + j;
                    const int p = stencil_piece(st, v, cb.npieces);
                    shift_check(a, as_idx(a.binned[v + st.delta[p]].w), st.kid[p], si);
                }
            }
        }
    }
}

// Counting, register path of one wave's bin (stencil of at most kMapCap
// candidates): counts[s] and masks[binned index][chunk] of every source.
// Passes of CountChunks<T> chunks, the last one with exactly the chunks left.
template <typename T, int MODE>
__device__ __forceinline__ void count_wave_bin(const QueryArgs<T>& a, const WaveStencil<T>& st,
                                               const CellBin<T>& cb, int s_begin, int s_end) {
    constexpr int CH = CountChunks<T>::value;
    const int lane = lane_id();
    const int nch = cb.nch;
    for (int sg = s_begin; sg < s_end; sg += kWave) {
        const int ns = min(kWave, s_end - sg);
        const Vec4<T> zero4 = {T(0), T(0), T(0), T(0)};
        const Vec4<T> own = lane < ns ? a.binned[sg + lane] : zero4;
        // lane gi, full list without self pairs: chunk and bit of source
        // gi's own candidate (binned index minus dself, k = 0)
        int selfp = 0;
        if constexpr (MODE == 0) {
            const int vs = sg + lane - cb.dself;
            const int ls = (int)(((float)vs + 0.5f) / (float)nch);
            selfp = (vs - ls * nch) | (ls << 16);
        }
        int acc = 0;  // lane gi: pairs of source gi
        for (int c0 = 0; c0 < nch; c0 += CH) {
            switch (min(CH, nch - c0)) {
#define TNR_COUNT_NC(n)                                                                    \
    case n:                                                                                \
        if constexpr (n <= CH) count_pass<T, MODE, n>(a, st, cb, sg, ns, c0, own, selfp, acc); \
        break;
                TNR_COUNT_NC(1) TNR_COUNT_NC(2) TNR_COUNT_NC(3) TNR_COUNT_NC(4)
                TNR_COUNT_NC(5) TNR_COUNT_NC(6) TNR_COUNT_NC(7) TNR_COUNT_NC(8)
                TNR_COUNT_NC(9) TNR_COUNT_NC(10) TNR_COUNT_NC(11) TNR_COUNT_NC(12)
#undef TNR_COUNT_NC
                default: break;
            }
        }
        if (lane < ns) a.counts[cb.by_bin ? sg + lane : as_idx(own.w)] = acc;
    }
}

// Counting pass, persistent grid of waves.  A task is one of the
// CountParts<T> equal parts of a bin's sources; the tasks are dealt to the
// XCDs (workgroup b runs on XCD b % 8) in chunks of kCountChunk bins' tasks,
// chunk c to XCD c % 8, and the waves of an XCD take its tasks round robin,
// the four waves of a workgroup four consecutive tasks.  Each task builds
// its bin's stencil itself.
// Writes counts[s] for each source s of a cell-list structure.  The status
// word is read once: abort bits only come from earlier kernels.
template <typename T, int MODE>
__global__ __launch_bounds__(kBlock) void k_cell_count(QueryArgs<T> a) {
    __shared__ CountLds<T> s_lds[kWavesPerBlock];

    if (load_status(a.status + SS_FLAGS) & kAbortBits) return;
    const unsigned long long plan = load_status(a.status + SS_PLAN);
    const int wv = uniform(threadIdx.x / kWave);
    int need = 0;  // the longest hit-mask row this wave's sources wanted
    if (plan & 2) {
        constexpr int kCountParts = CountParts<T>::value;
        const int64_t W = a.struct_bin_off[a.nb] * kCountParts;
        const int64_t K = kCountChunk * kCountParts;
        const int64_t x = (int64_t)(blockIdx.x & 7u);
        const int64_t nw = (int64_t)(gridDim.x / 8) * kWavesPerBlock;  // grid: a multiple of 8
        const int64_t end = xcd_items(W, K, x);
        StructCache sc{0, 0, 0};
        for (int64_t j = (int64_t)(blockIdx.x >> 3) * kWavesPerBlock + wv; j < end; j += nw) {
            const int64_t t = xcd_item(x, j, K);
            CellBin<T> cb;
            if (!wave_bin<T>(a, t / kCountParts, sc, cb, s_lds[wv].st)) continue;
            const int part = (int)(t % kCountParts);
            const int h = (cb.se - cb.sb + kCountParts - 1) / kCountParts;
            const int s0 = cb.sb + part * h, s1 = min(cb.se, s0 + h);
            if (s0 >= s1) continue;
            if (cb.C <= kMapCap) need = max(need, cb.nch);
            if (cb.nch <= a.mask_words) {
                count_wave_bin<T, MODE>(a, s_lds[wv].st, cb, s0, s1);
            } else {
                cb.sb = s0;
                cb.se = s1;
                cell_slow<T, MODE, false>(a, s_lds[wv].st, cb);
            }
        }
    }
    if ((plan & 1) && a.brute_in_cell) {
        // brute-force structures of an explicit cell_list request (no bin
        // grid fits them): one wave per work unit, atoms read from global
        // memory, the per-source cursors in the wave's LDS
        wave_lds_fence();
        const int64_t units = (int64_t)load_status(a.status + SS_TOTAL_UNITS);
        const int64_t nwaves = (int64_t)gridDim.x * kWavesPerBlock;
        for (int64_t u = (int64_t)blockIdx.x * kWavesPerBlock + wv; u < units; u += nwaves) {
            const int b = uniform(unit_structure(a.struct_unit_off, a.nb, u));
            const StructRec& r = a.recs[b];
            need = max(need, r.mneed);
            if (molecule_rec(r))
                molecule_count<T, MODE>(a, r, u, r.unit0);
            else
                brute_unit<T, MODE, false, false>(a, u, b, nullptr, s_lds[wv].cur);
        }
    }
    report_mask_need(a.status, need);
}

}  // namespace tnr
