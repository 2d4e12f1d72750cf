// CPU oracle for the tonari neighbor-list hot path.
//
// TEST INFRASTRUCTURE ONLY.  This file restates, in plain C++20, the
// algorithm of the reference CPU search so that tests, smoke() and the
// benchmark's cpu_baseline leg can check the HIP product path against it.
// The product library (tonari_amd) never loads or links it.
//
// Reference behaviour followed (file:line in songfeitong/tonari):
//   periodic metadata / active pseudo-inverse  csrc/core/geometry.cpp:15-219
//   pair identity policy                       csrc/core/pair_policy.h:17-79
//   representative wraps (long double)         csrc/core/neighbors_cpu.cpp:92-133
//   image translations                         csrc/core/neighbors_cpu.cpp:136-153
//   conservative cell-list cutoff              csrc/core/neighbors_cpu.cpp:156-219
//   public predicate (append_candidate)        csrc/core/neighbors_cpu.cpp:222-273
//   wrapped broad phase (append_cell_candidate) csrc/core/neighbors_cpu.cpp:276-327
//   brute force                                csrc/core/neighbors_cpu.cpp:330-361
//   per-structure auto selection (16384)       csrc/core/neighbors_cpu.cpp:21,82-89,364-376
//   bin layout / image-node cell list          csrc/core/neighbors_cpu.cpp:379-584
//   prepare + fallback                         csrc/core/neighbors_cpu.cpp:625-680
//   task split (2^18 candidates / 128 sources) csrc/core/neighbors_cpu.cpp:26-27,683-697,700-865
//   input checks                               csrc/core/neighbors_cpu.cpp:976-1030
//   worker pool semantics                      csrc/core/thread_pool.cpp:22-191
//
// Pinned by (all in tests/test_oracle.py): the reference test suite's
// known-answer tests restated as test_kat_*, the error contract
// (test_error_contract), an independent numpy enumeration
// (test_port_matches_numpy_enumeration, test_batched_structures_match_numpy),
// closed forms and invariants (test_half_and_self_algebra,
// test_cell_list_equals_brute_force, test_thread_count_invariance,
// test_quantities_closed_form), golden key hashes written by the compiled
// reference core (test_port_matches_golden*, tests/golden/) and that core
// itself when it builds here (test_port_matches_reference_core, oracle/_ref).

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <exception>
#include <limits>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

namespace orc {

struct input_error : std::invalid_argument {
    using std::invalid_argument::invalid_argument;
};
struct search_error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

static void need_input(bool ok, const char* what) {
    if (!ok) throw input_error(what);
}
static void need_search(bool ok, const char* what) {
    if (!ok) throw search_error(what);
}

constexpr int64_t kImageCap = int64_t{1} << 24;          // geometry.cpp:12
constexpr int64_t kBruteLimit = 16384;                   // neighbors_cpu.cpp:21
constexpr int64_t kDenseBinCap = int64_t{1} << 26;       // neighbors_cpu.cpp:23
constexpr int64_t kBinsPerImage = 64;                    // neighbors_cpu.cpp:24
constexpr int kRoundoff = 64;                            // neighbors_cpu.cpp:25
constexpr int64_t kBruteTaskCandidates = int64_t{1} << 18;  // neighbors_cpu.cpp:26
constexpr int64_t kCellTaskSources = 128;                // neighbors_cpu.cpp:27

enum Mode : int { FULL = 0, FULL_SELF = 1, HALF = 2, HALF_SELF = 3 };
enum Algo : int { AUTO = 0, BRUTE = 1, CELL = 2 };

// ---------------------------------------------------------------- geometry

// Moore-Penrose pseudo-inverse of the k active cell rows by one-sided
// (Hestenes) Jacobi in long double.  Output: dual[c][j] for active slot j.
static void hestenes_pinv(const double* cell, const int* axes, int k,
                          long double dual[3][3]) {
    long double w[3][3] = {};  // w[c][j]: column j = active row j
    long double v[3][3] = {};  // accumulated right rotations
    for (int j = 0; j < k; ++j) {
        v[j][j] = 1.0L;
        for (int c = 0; c < 3; ++c) w[c][j] = (long double)cell[3 * axes[j] + c];
    }
    const long double eps = std::numeric_limits<double>::epsilon();
    for (int sweep = 0; sweep < 64; ++sweep) {
        bool rotated = false;
        for (int p = 0; p < k; ++p) {
            for (int q = p + 1; q < k; ++q) {
                long double app = 0.0L, aqq = 0.0L, apq = 0.0L;
                for (int c = 0; c < 3; ++c) {
                    app += w[c][p] * w[c][p];
                    aqq += w[c][q] * w[c][q];
                    apq += w[c][p] * w[c][q];
                }
                if (std::abs(apq) <= 8 * eps * std::sqrt(app * aqq)) continue;
                rotated = true;
                const long double zeta = (aqq - app) / (2 * apq);
                const long double t =
                    zeta == 0.0L ? 1.0L
                                 : std::copysign(1.0L, zeta) /
                                       (std::abs(zeta) + std::hypot(1.0L, zeta));
                const long double cs = 1.0L / std::hypot(1.0L, t);
                const long double sn = cs * t;
                for (int c = 0; c < 3; ++c) {
                    const long double a = w[c][p], b = w[c][q];
                    w[c][p] = cs * a - sn * b;
                    w[c][q] = sn * a + cs * b;
                }
                for (int r = 0; r < k; ++r) {
                    const long double a = v[r][p], b = v[r][q];
                    v[r][p] = cs * a - sn * b;
                    v[r][q] = sn * a + cs * b;
                }
            }
        }
        if (!rotated) break;
    }
    long double sigma[3] = {};
    long double smax = 0.0L, smin = std::numeric_limits<long double>::infinity();
    for (int j = 0; j < k; ++j) {
        long double s2 = 0.0L;
        for (int c = 0; c < 3; ++c) s2 += w[c][j] * w[c][j];
        sigma[j] = std::sqrt(s2);
        smax = std::max(smax, sigma[j]);
        smin = std::min(smin, sigma[j]);
    }
    const long double tol = eps * 3 * std::max(smax, 1.0L);
    need_input(smin > tol, "active periodic cell vectors must be linearly independent");
    for (int c = 0; c < 3; ++c) {
        for (int a = 0; a < k; ++a) {
            long double acc = 0.0L;
            for (int j = 0; j < k; ++j) acc += w[c][j] * v[a][j] / (sigma[j] * sigma[j]);
            dual[c][a] = acc;
        }
    }
}

struct Metadata {
    std::vector<double> duals;       // (B, 3, 3): [b][cartesian][axis]
    std::vector<int32_t> shifts;     // (I_total, 3)
    std::vector<int64_t> offsets;    // (B + 1)
};

static Metadata periodic_metadata(const std::vector<double>& cells, const uint8_t* pbc,
                                  const std::vector<int64_t>& counts, double cutoff) {
    const int64_t nb = (int64_t)counts.size();
    Metadata md;
    md.duals.assign(9 * nb, 0.0);
    md.offsets.push_back(0);
    for (int64_t b = 0; b < nb; ++b) {
        const double* cell = cells.data() + 9 * b;
        for (int e = 0; e < 9; ++e)
            need_input(std::isfinite(cell[e]), "cell must contain only finite values");
        if (counts[b] == 0) {
            md.offsets.push_back((int64_t)md.shifts.size() / 3);
            continue;
        }
        int axes[3];
        int k = 0;
        for (int a = 0; a < 3; ++a)
            if (pbc[3 * b + a]) axes[k++] = a;
        int64_t reps[3] = {0, 0, 0};
        if (k > 0) {
            long double dual[3][3] = {};
            hestenes_pinv(cell, axes, k, dual);
            for (int j = 0; j < k; ++j) {
                long double n2 = 0.0L;
                for (int c = 0; c < 3; ++c) {
                    const long double x = dual[c][j];
                    need_input(std::isfinite(x) &&
                                   std::abs(x) <= std::numeric_limits<double>::max(),
                               "active periodic cell dual is outside the float64 range");
                    md.duals[9 * b + 3 * c + axes[j]] = (double)x;
                    n2 += x * x;
                }
                const long double r = std::ceil(cutoff * std::sqrt(n2));
                need_input(r <= std::numeric_limits<int32_t>::max(),
                           "periodic image range exceeds int32 cell shifts");
                reps[axes[j]] = (int64_t)r;
            }
        }
        int64_t count = 1;
        for (int a = 0; a < 3; ++a) {
            const int64_t f = 2 * reps[a] + 1;
            need_input(count <= kImageCap / f,
                       "periodic image count exceeds the 2^24 resource limit");
            count *= f;
        }
        const int64_t have = (int64_t)md.shifts.size() / 3;
        need_input(have <= kImageCap - count,
                   "batched periodic image count exceeds the 2^24 resource limit");
        for (int64_t x = -reps[0]; x <= reps[0]; ++x)
            for (int64_t y = -reps[1]; y <= reps[1]; ++y)
                for (int64_t z = -reps[2]; z <= reps[2]; ++z) {
                    md.shifts.push_back((int32_t)x);
                    md.shifts.push_back((int32_t)y);
                    md.shifts.push_back((int32_t)z);
                }
        md.offsets.push_back((int64_t)md.shifts.size() / 3);
    }
    return md;
}

// ------------------------------------------------------------ pair policy

static inline bool zero_shift_self(int64_t s, int64_t t, const int64_t S[3]) {
    return s == t && S[0] == 0 && S[1] == 0 && S[2] == 0;
}
static inline bool canonical_half(int64_t s, int64_t t, const int64_t S[3]) {
    if (s != t) return s < t;
    for (int a = 0; a < 3; ++a)
        if (S[a] != 0) return S[a] < 0;
    return true;
}
template <int M>
static inline bool keep_identity(int64_t s, int64_t t, const int64_t S[3]) {
    if (zero_shift_self(s, t, S)) return (M & 1) != 0;
    if constexpr ((M & 2) != 0) return canonical_half(s, t, S);
    return true;
}

// -------------------------------------------------------------- buffers

struct Chunk {
    std::vector<int64_t> idx;
    std::vector<int32_t> sh;
};

// ----------------------------------------------------------- structures

template <typename T>
struct Bins {
    T origin[3];
    T size;
    int64_t dim[3];
    int64_t count;
};

struct Node {
    int32_t target;
    int32_t image;
    int32_t next;
};

template <typename T>
struct Structure {
    int64_t offset = 0, n = 0, shift0 = 0, ns = 0;
    int algo = AUTO;
    const T* pos = nullptr;
    const T* cell = nullptr;
    const T* dual = nullptr;
    const int32_t* img = nullptr;
    std::vector<T> wpos;
    std::vector<int32_t> wrap;
    std::vector<T> trans;
    Bins<T> bins{};
    std::vector<int32_t> heads;
    std::vector<Node> nodes;
    T search2 = T(0), inner2 = T(0);
};

static bool brute_small(int64_t n, int64_t ns, int64_t limit) {
    if (n == 0 || ns == 0) return true;
    return n <= limit / n && ns <= limit / (n * n);
}

template <typename T>
static void wrap_positions(Structure<T>& st) {
    const T upper = (T)2147483648.0;
    st.wpos.resize(3 * st.n);
    st.wrap.resize(3 * st.n);
    for (int64_t i = 0; i < st.n; ++i) {
        const T* p = st.pos + 3 * i;
        for (int c = 0; c < 3; ++c)
            need_search(std::isfinite(p[c]), "positions must contain only finite values");
        for (int a = 0; a < 3; ++a) {
            long double f = 0.0L;
            for (int c = 0; c < 3; ++c)
                f += (long double)p[c] * (long double)st.dual[3 * c + a];
            need_search(std::isfinite(f) && f >= -(long double)upper && f < (long double)upper,
                        "atom representatives require periodic wraps outside the int32 range");
            st.wrap[3 * i + a] = (int32_t)std::floor(f);
        }
        for (int c = 0; c < 3; ++c) {
            T q = p[c];
            for (int a = 0; a < 3; ++a) q -= (T)st.wrap[3 * i + a] * st.cell[3 * a + c];
            st.wpos[3 * i + c] = q;
        }
    }
}

template <typename T>
static bool padded_search_cutoff(const Structure<T>& st, T cutoff, T& search) {
    long double maxp[3] = {};
    int64_t maxw[3] = {}, maxi[3] = {};
    for (int64_t i = 0; i < st.n; ++i) {
        for (int c = 0; c < 3; ++c) {
            if (!std::isfinite(st.wpos[3 * i + c])) return false;
            maxp[c] = std::max(maxp[c], std::abs((long double)st.pos[3 * i + c]));
        }
        for (int a = 0; a < 3; ++a)
            maxw[a] = std::max(maxw[a], std::abs((int64_t)st.wrap[3 * i + a]));
    }
    for (int64_t s = 0; s < st.ns; ++s)
        for (int a = 0; a < 3; ++a)
            maxi[a] = std::max(maxi[a], std::abs((int64_t)st.img[3 * s + a]));
    long double scale = 0.0L;
    for (int c = 0; c < 3; ++c) {
        long double sc = 2 * maxp[c];
        for (int a = 0; a < 3; ++a)
            sc += (long double)(maxi[a] + 2 * maxw[a]) * std::abs((long double)st.cell[3 * a + c]);
        scale = std::max(scale, sc);
    }
    const long double pad = kRoundoff * std::numeric_limits<T>::epsilon() * scale;
    const long double padded = (long double)cutoff + pad;
    if (!std::isfinite(padded) || padded > 2 * (long double)cutoff ||
        padded > std::numeric_limits<T>::max())
        return false;
    search = std::nextafter((T)padded, std::numeric_limits<T>::infinity());
    return std::isfinite(search);
}

template <typename T>
static bool make_bins(Structure<T>& st, T size, T lo[3], T hi[3]) {
    if (size == T(0)) return false;
    st.bins.size = size;
    for (int c = 0; c < 3; ++c) {
        lo[c] = std::numeric_limits<T>::infinity();
        hi[c] = -std::numeric_limits<T>::infinity();
    }
    for (int64_t i = 0; i < st.n; ++i)
        for (int c = 0; c < 3; ++c) {
            lo[c] = std::min(lo[c], st.wpos[3 * i + c]);
            hi[c] = std::max(hi[c], st.wpos[3 * i + c]);
        }
    st.bins.count = 1;
    for (int c = 0; c < 3; ++c) {
        const T span = hi[c] - lo[c] + 2 * size;
        const T dim = span / size;
        if (!std::isfinite(dim) || dim > kDenseBinCap) return false;
        st.bins.origin[c] = lo[c] - size;
        st.bins.dim[c] = std::max<int64_t>(1, (int64_t)std::ceil(dim));
        if (st.bins.count > kDenseBinCap / st.bins.dim[c]) return false;
        st.bins.count *= st.bins.dim[c];
    }
    if (st.n > std::numeric_limits<int64_t>::max() / st.ns) return false;
    const int64_t images = st.n * st.ns;
    return st.bins.count <= kDenseBinCap &&
           (st.bins.count + kBinsPerImage - 1) / kBinsPerImage <= images;
}

template <typename T>
static int64_t bin_of(const T x[3], const Bins<T>& b) {
    int64_t k[3];
    for (int c = 0; c < 3; ++c)
        k[c] = std::clamp((int64_t)std::floor((x[c] - b.origin[c]) / b.size), int64_t{0},
                          b.dim[c] - 1);
    return (k[0] * b.dim[1] + k[1]) * b.dim[2] + k[2];
}

template <typename T>
static bool build_cell_list(Structure<T>& st, T search, T inner2) {
    need_search(st.n < std::numeric_limits<int32_t>::max() &&
                    st.ns < std::numeric_limits<int32_t>::max(),
                "cell-list atoms and image shifts must fit int32 indexing");
    T lo[3], hi[3];
    if (!make_bins(st, search, lo, hi)) return false;
    st.heads.assign(st.bins.count, -1);
    st.nodes.clear();
    st.nodes.reserve((size_t)std::min(st.n * st.ns, 4 * st.n));
    for (int64_t t = 0; t < st.n; ++t) {
        for (int64_t s = 0; s < st.ns; ++s) {
            T x[3];
            bool inside = true;
            for (int c = 0; c < 3; ++c) {
                x[c] = st.wpos[3 * t + c] + st.trans[3 * s + c];
                inside = inside && std::isfinite(x[c]) && x[c] >= lo[c] - search &&
                         x[c] <= hi[c] + search;
            }
            if (!inside) continue;
            const int64_t bin = bin_of(x, st.bins);
            need_search(st.nodes.size() < (size_t)std::numeric_limits<int32_t>::max(),
                        "cell-list node count exceeds int32 indexing");
            const int32_t id = (int32_t)st.nodes.size();
            st.nodes.push_back({(int32_t)t, (int32_t)s, st.heads[bin]});
            st.heads[bin] = id;
        }
    }
    st.search2 = search * search;
    st.inner2 = inner2;
    return true;
}

template <typename T>
static void prepare(Structure<T>& st, T cutoff, int requested) {
    if (st.n == 0) return;
    wrap_positions(st);
    st.algo = requested != AUTO ? requested
                                : (brute_small(st.n, st.ns, kBruteLimit) ? BRUTE : CELL);
    if (st.algo == BRUTE) return;
    st.trans.assign(3 * st.ns, T(0));
    for (int64_t s = 0; s < st.ns; ++s)
        for (int c = 0; c < 3; ++c) {
            T acc = T(0);
            for (int a = 0; a < 3; ++a) acc += (T)st.img[3 * s + a] * st.cell[3 * a + c];
            st.trans[3 * s + c] = acc;
        }
    T search = T(0);
    const bool safe = padded_search_cutoff(st, cutoff, search);
    const T inner = std::max(T(0), 2 * cutoff - search);
    if (safe && build_cell_list(st, search, inner * inner)) return;
    need_search(requested != CELL,
                "cell_list cannot safely process this structure; use "
                "algorithm='auto' or 'brute_force'");
    st.algo = BRUTE;
}

// The public predicate: D = (p_t - p_s) + S0*c0 + S1*c1 + S2*c2 (each step
// rounded in T), d2 = D0^2 + D1^2 + D2^2 left to right, strict d2 < rc^2.
template <typename T, int M>
static inline void candidate(const Structure<T>& st, int64_t s, int64_t t, int64_t image,
                             bool known_inside, T cut2, Chunk& out) {
    const int32_t* I = st.img + 3 * image;
    int64_t S[3];
    for (int a = 0; a < 3; ++a)
        S[a] = (int64_t)I[a] - (int64_t)st.wrap[3 * t + a] + (int64_t)st.wrap[3 * s + a];
    const bool self0 = zero_shift_self(s, t, S);
    if (!keep_identity<M>(s, t, S)) return;
    if (!self0 && !known_inside) {
        T d2 = T(0);
        for (int c = 0; c < 3; ++c) {
            T comp = st.pos[3 * t + c] - st.pos[3 * s + c];
            for (int a = 0; a < 3; ++a) comp += (T)S[a] * st.cell[3 * a + c];
            d2 += comp * comp;
        }
        if (d2 >= cut2) return;
    }
    for (int a = 0; a < 3; ++a)
        need_search(S[a] >= std::numeric_limits<int32_t>::min() &&
                        S[a] <= std::numeric_limits<int32_t>::max(),
                    "a cell shift required by the cutoff pairs exceeds the int32 output range");
    out.idx.push_back(st.offset + s);
    out.idx.push_back(st.offset + t);
    for (int a = 0; a < 3; ++a) out.sh.push_back((int32_t)S[a]);
}

template <typename T, int M>
static void search_brute(const Structure<T>& st, int64_t s0, int64_t s1, T cut2, Chunk& out) {
    for (int64_t s = s0; s < s1; ++s)
        for (int64_t t = 0; t < st.n; ++t)
            for (int64_t i = 0; i < st.ns; ++i) candidate<T, M>(st, s, t, i, false, cut2, out);
}

template <typename T, int M>
static void search_cell(const Structure<T>& st, int64_t s0, int64_t s1, T cut2, Chunk& out) {
    const Bins<T>& b = st.bins;
    for (int64_t s = s0; s < s1; ++s) {
        const T* q = st.wpos.data() + 3 * s;
        int64_t k[3];
        for (int c = 0; c < 3; ++c)
            k[c] = std::clamp((int64_t)std::floor((q[c] - b.origin[c]) / b.size), int64_t{0},
                              b.dim[c] - 1);
        for (int ox = -1; ox <= 1; ++ox) {
            const int64_t x = k[0] + ox;
            if (x < 0 || x >= b.dim[0]) continue;
            for (int oy = -1; oy <= 1; ++oy) {
                const int64_t y = k[1] + oy;
                if (y < 0 || y >= b.dim[1]) continue;
                for (int oz = -1; oz <= 1; ++oz) {
                    const int64_t z = k[2] + oz;
                    if (z < 0 || z >= b.dim[2]) continue;
                    for (int32_t nd = st.heads[(x * b.dim[1] + y) * b.dim[2] + z]; nd >= 0;
                         nd = st.nodes[nd].next) {
                        const int64_t t = st.nodes[nd].target;
                        const int64_t im = st.nodes[nd].image;
                        if constexpr ((M & 2) != 0) {
                            int64_t S[3];
                            for (int a = 0; a < 3; ++a)
                                S[a] = (int64_t)st.img[3 * im + a] - st.wrap[3 * t + a] +
                                       st.wrap[3 * s + a];
                            if (!keep_identity<M>(s, t, S)) continue;
                        }
                        T d2 = T(0);
                        for (int c = 0; c < 3; ++c) {
                            const T comp = st.wpos[3 * t + c] - q[c] + st.trans[3 * im + c];
                            d2 += comp * comp;
                        }
                        if (d2 >= st.search2) continue;
                        candidate<T, M>(st, s, t, im, d2 < st.inner2, cut2, out);
                    }
                }
            }
        }
    }
}

template <typename T, int M>
static void search(const Structure<T>& st, int64_t s0, int64_t s1, T cut2, Chunk& out) {
    if (st.algo == BRUTE)
        search_brute<T, M>(st, s0, s1, cut2, out);
    else
        search_cell<T, M>(st, s0, s1, cut2, out);
}

// ---------------------------------------------------------------- threads

// Dynamic task counter shared by `threads` participants (the caller included);
// the first exception cancels the remaining tasks and is rethrown.
template <typename F>
static void parallel_for(int64_t tasks, int64_t threads, F&& fn) {
    if (tasks <= 0) return;
    const int64_t parts = std::min(tasks, threads);
    if (parts <= 1) {
        for (int64_t i = 0; i < tasks; ++i) fn(i);
        return;
    }
    std::atomic<int64_t> next{0};
    std::atomic<bool> cancel{false};
    std::exception_ptr first;
    std::mutex mu;
    auto body = [&]() {
        while (!cancel.load(std::memory_order_relaxed)) {
            const int64_t i = next.fetch_add(1, std::memory_order_relaxed);
            if (i >= tasks) break;
            try {
                fn(i);
            } catch (...) {
                std::lock_guard<std::mutex> g(mu);
                if (!first) first = std::current_exception();
                cancel.store(true);
            }
        }
    };
    std::vector<std::thread> pool;
    pool.reserve(parts - 1);
    for (int64_t w = 0; w + 1 < parts; ++w) pool.emplace_back(body);
    body();
    for (auto& th : pool) th.join();
    if (first) std::rethrow_exception(first);
}

static int64_t chunk_size(int algo, int64_t n, int64_t ns) {
    if (algo == CELL) return kCellTaskSources;
    if (n == 0 || ns == 0 || n > std::numeric_limits<int64_t>::max() / ns) return 1;
    return std::max<int64_t>(1, kBruteTaskCandidates / (n * ns));
}

struct Result {
    std::vector<Chunk> chunks;
    int64_t pairs = 0;
};

template <typename T, int M>
static void build(const T* pos, const int64_t* bp, int64_t nb, const T* cells,
                  const std::vector<T>& duals, const Metadata& md, double cutoff, int requested,
                  int64_t threads, Result& res) {
    const T rc = (T)cutoff;
    const T cut2 = (T)(cutoff * cutoff);
    std::vector<Structure<T>> sts((size_t)nb);
    for (int64_t b = 0; b < nb; ++b) {
        auto& st = sts[b];
        st.offset = bp[b];
        st.n = bp[b + 1] - bp[b];
        st.shift0 = md.offsets[b];
        st.ns = md.offsets[b + 1] - md.offsets[b];
        st.pos = pos + 3 * st.offset;
        st.cell = cells + 9 * b;
        st.dual = duals.data() + 9 * b;
        st.img = md.shifts.data() + 3 * st.shift0;
    }
    if (threads == 1) {
        res.chunks.emplace_back();
        for (int64_t b = 0; b < nb; ++b) {
            prepare(sts[b], rc, requested);
            search<T, M>(sts[b], 0, sts[b].n, cut2, res.chunks.back());
            sts[b] = Structure<T>();
        }
    } else {
        std::vector<char> split((size_t)nb, 0);
        std::vector<int64_t> split_ids;
        for (int64_t b = 0; b < nb; ++b) {
            auto& st = sts[b];
            st.algo = requested != AUTO
                          ? requested
                          : (brute_small(st.n, st.ns, kBruteLimit) ? BRUTE : CELL);
            if (st.n > chunk_size(st.algo, st.n, st.ns)) {
                split[b] = 1;
                split_ids.push_back(b);
            }
        }
        parallel_for((int64_t)split_ids.size(), threads,
                     [&](int64_t i) { prepare(sts[split_ids[i]], rc, requested); });
        struct Task {
            int64_t b, s0, s1;
            bool prep;
        };
        std::vector<Task> tasks;
        for (int64_t b = 0; b < nb; ++b) {
            const auto& st = sts[b];
            if (st.n == 0) continue;
            if (!split[b]) {
                tasks.push_back({b, 0, st.n, true});
                continue;
            }
            const int64_t cs = chunk_size(st.algo, st.n, st.ns);
            for (int64_t s = 0; s < st.n; s += cs) tasks.push_back({b, s, std::min(st.n, s + cs), false});
        }
        res.chunks.resize(tasks.size());
        parallel_for((int64_t)tasks.size(), threads, [&](int64_t i) {
            const Task& tk = tasks[i];
            auto& st = sts[tk.b];
            if (tk.prep) prepare(st, rc, requested);
            search<T, M>(st, tk.s0, tk.s1, cut2, res.chunks[i]);
            if (tk.prep) st = Structure<T>();
        });
    }
    for (const auto& c : res.chunks) res.pairs += (int64_t)c.idx.size() / 2;
}

template <typename T>
static void run(const T* pos, int64_t n, const int64_t* bp, int64_t blen, const T* cells,
                const uint8_t* pbc, double cutoff, int mode, int algo, int64_t threads,
                Result& res) {
    need_input(blen >= 1, "batch_ptr must have shape (B + 1,)");
    const int64_t nb = blen - 1;
    need_input(std::isfinite(cutoff) && cutoff > 0, "cutoff must be finite and positive");
    need_input(threads > 0, "num_threads must be a positive integer");
    need_input(bp[0] == 0, "batch_ptr must start at zero");
    need_input(bp[nb] == n, "batch_ptr must end at N_total");
    need_input(n < std::numeric_limits<int32_t>::max(),
               "the current implementation supports fewer than 2^31 atoms");
    std::vector<int64_t> counts;
    counts.reserve(nb);
    for (int64_t b = 0; b < nb; ++b) {
        need_input(bp[b + 1] >= bp[b], "batch_ptr must be nondecreasing");
        counts.push_back(bp[b + 1] - bp[b]);
    }
    std::vector<double> cd(cells, cells + 9 * nb);
    const Metadata md = periodic_metadata(cd, pbc, counts, cutoff);
    std::vector<T> duals(md.duals.begin(), md.duals.end());
    switch (mode) {
        case FULL: build<T, FULL>(pos, bp, nb, cells, duals, md, cutoff, algo, threads, res); break;
        case FULL_SELF: build<T, FULL_SELF>(pos, bp, nb, cells, duals, md, cutoff, algo, threads, res); break;
        case HALF: build<T, HALF>(pos, bp, nb, cells, duals, md, cutoff, algo, threads, res); break;
        default: build<T, HALF_SELF>(pos, bp, nb, cells, duals, md, cutoff, algo, threads, res); break;
    }
}

}  // namespace orc

// ---------------------------------------------------------------- C ABI
//
// Return codes: 0 ok, 1 input error (ValueError), 2 search error
// (RuntimeError), 3 other failure.  The message is NUL-terminated in `err`.

extern "C" {

int orc_neighbor_list(int dtype, const void* positions, int64_t n_atoms, const int64_t* batch_ptr,
                      int64_t batch_len, const void* cells, const uint8_t* pbc, double cutoff,
                      int half_list, int include_self, int algorithm, int64_t threads,
                      void** handle, int64_t* n_pairs, char* err, int64_t errlen) {
    auto* res = new orc::Result();
    auto fail = [&](int code, const char* msg) {
        if (err && errlen > 0) {
            std::strncpy(err, msg, (size_t)errlen - 1);
            err[errlen - 1] = 0;
        }
        delete res;
        *handle = nullptr;
        *n_pairs = 0;
        return code;
    };
    try {
        const int mode = (half_list ? 2 : 0) | (include_self ? 1 : 0);
        if (dtype == 0)
            orc::run<float>((const float*)positions, n_atoms, batch_ptr, batch_len,
                            (const float*)cells, pbc, cutoff, mode, algorithm, threads, *res);
        else
            orc::run<double>((const double*)positions, n_atoms, batch_ptr, batch_len,
                             (const double*)cells, pbc, cutoff, mode, algorithm, threads, *res);
    } catch (const orc::input_error& e) {
        return fail(1, e.what());
    } catch (const orc::search_error& e) {
        return fail(2, e.what());
    } catch (const std::exception& e) {
        return fail(3, e.what());
    }
    *handle = res;
    *n_pairs = res->pairs;
    return 0;
}

void orc_copy(void* handle, int64_t* pairs, int32_t* shifts) {
    const auto* res = (const orc::Result*)handle;
    int64_t o = 0;
    for (const auto& c : res->chunks) {
        const int64_t m = (int64_t)c.idx.size() / 2;
        if (m) {
            std::memcpy(pairs + 2 * o, c.idx.data(), sizeof(int64_t) * 2 * m);
            std::memcpy(shifts + 3 * o, c.sh.data(), sizeof(int32_t) * 3 * m);
        }
        o += m;
    }
}

void orc_free(void* handle) { delete (orc::Result*)handle; }

}  // extern "C"
