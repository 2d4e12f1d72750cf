// Host (CPU) neighbor-list provider: the C ABI of include/tonari_cpu.h.
//
// The same search as the device pipeline (tonari_hip.hip), on host threads:
// per-structure periodic metadata (the pseudo-inverse of the active cell
// rows by one-sided Jacobi, repeats, image counts and their caps), per-atom
// representative wraps (double-double, as the reference's long double) and
// wrapped positions, the per-structure operation scale and broad-phase
// margin, the reference's cell_list layout rule, then a search that decides
// every candidate with the reference's public predicate
// (neighbors_cpu.cpp:247-261), so the pair set is the reference's.
//
// Candidates:
//   brute force  every target of the structure in every image of the
//                reference's image box [-R, R] on the periodic axes
//                (neighbors_cpu.cpp:136-153, 330-361);
//   cell list    bins over the grid coordinates of the wrapped positions
//                (fractional coordinates on periodic axes, an orthonormal
//                complement elsewhere), at least rc + 2 pad wide in every
//                grid direction; a source visits the unwrapped bins within
//                its reach, each giving a bin and an image shift, so every
//                target within rc + 2 pad of it is visited once per image.
// Pairs come grouped by structure and by source in index order, as the
// reference's CPU path returns them (neighbors_cpu.cpp:700-865).
//
// Compiled with -ffp-contract=off and SSE arithmetic: every operation of
// the predicate is rounded in the input type, in the reference's order.

#include "../../../include/tonari_cpu.h"

#include <pthread.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <deque>
#include <exception>
#include <functional>
#include <limits>
#include <mutex>
#include <new>
#include <thread>
#include <vector>

namespace tnr_cpu {

constexpr int kOk = 0, kInputError = 1, kSearchError = 2;
constexpr int kFloat32 = 0, kFloat64 = 1;
constexpr int kAuto = 0, kBruteForce = 1, kCellList = 2;
constexpr int64_t kImageCap = int64_t{1} << 24;        // geometry.cpp:12
constexpr int64_t kAutoCandidates = 4096;              // this provider's brute/cell crossover
constexpr int64_t kSourcesPerTask = 256;  // at most; fewer when that leaves threads idle

// Error bits, decoded in the reference's priority order (kMessages).
enum Err : uint32_t {
    E_BP_START = 1u << 0,
    E_BP_END = 1u << 1,
    E_BP_ORDER = 1u << 2,
    E_CELL_NONFINITE = 1u << 3,
    E_CELL_RANK = 1u << 4,
    E_DUAL_RANGE = 1u << 5,
    E_REPEAT_RANGE = 1u << 6,
    E_IMAGE_CAP = 1u << 7,
    E_BATCH_IMAGE_CAP = 1u << 8,
    E_POS_NONFINITE = 1u << 9,
    E_WRAP_RANGE = 1u << 10,
    E_CELL_UNSAFE = 1u << 11,
    E_SHIFT_RANGE = 1u << 12,
};

struct Message {
    uint32_t bit;
    int code;
    const char* text;
};

// The reference's messages and exception classes (bindings_cuda.cpp:69-118,
// neighbors_cpu.cpp:976-1030, geometry.cpp), in its order of precedence.
const Message kMessages[] = {
    {E_BP_START, kInputError, "batch_ptr must start at zero"},
    {E_BP_END, kInputError, "batch_ptr must end at N_total"},
    {E_BP_ORDER, kInputError, "batch_ptr must be nondecreasing"},
    {E_CELL_NONFINITE, kInputError, "cell must contain only finite values"},
    {E_CELL_RANK, kInputError, "active periodic cell vectors must be linearly independent"},
    {E_DUAL_RANGE, kInputError, "active periodic cell dual is outside the float64 range"},
    {E_REPEAT_RANGE, kInputError, "periodic image range exceeds int32 cell shifts"},
    {E_IMAGE_CAP, kInputError, "periodic image count exceeds the 2^24 resource limit"},
    {E_BATCH_IMAGE_CAP, kInputError,
     "batched periodic image count exceeds the 2^24 resource limit"},
    {E_POS_NONFINITE, kSearchError, "positions must contain only finite values"},
    {E_WRAP_RANGE, kSearchError,
     "atom representatives require periodic wraps outside the int32 range"},
    {E_CELL_UNSAFE, kSearchError,
     "cell_list cannot safely process this structure; use algorithm='auto' or 'brute_force'"},
    {E_SHIFT_RANGE, kSearchError,
     "a cell shift required by the cutoff pairs exceeds the int32 output range"},
};

int put_error(char* err, size_t len, int code, const char* msg) {
    if (err && len > 0) {
        std::strncpy(err, msg, len - 1);
        err[len - 1] = 0;
    }
    return code;
}

// Machine epsilon and largest finite value of T.
template <typename T>
struct Limits {
    static constexpr double eps = std::numeric_limits<T>::epsilon();
    static constexpr double max = (double)std::numeric_limits<T>::max();
};

// ------------------------------------------------------------- geometry

// Moore-Penrose pseudo-inverse of the k active cell rows (columns 0..k-1 of
// w) by one-sided (Hestenes) Jacobi in float64, the steps of
// geometry.cpp:15-118; false when the rows are linearly dependent.
bool active_pinv(double w[3][3], int k, double dual[3][3]) {
    double v[3][3] = {{1, 0, 0}, {0, 1, 0}, {0, 0, 1}};
    const double eps = 2.220446049250313e-16;
    for (int sweep = 0; sweep < 64; ++sweep) {
        bool rotated = false;
        for (int p = 0; p < 3; ++p) {
            for (int q = p + 1; q < 3; ++q) {
                if (q >= k) continue;
                double app = 0, aqq = 0, apq = 0;
                for (int c = 0; c < 3; ++c) {
                    app += w[c][p] * w[c][p];
                    aqq += w[c][q] * w[c][q];
                    apq += w[c][p] * w[c][q];
                }
                if (std::fabs(apq) <= 8 * eps * std::sqrt(app * aqq)) continue;
                rotated = true;
                const double zeta = (aqq - app) / (2 * apq);
                const double t = zeta == 0.0 ? 1.0
                                             : std::copysign(1.0, zeta) /
                                                   (std::fabs(zeta) + std::hypot(1.0, zeta));
                const double cs = 1.0 / std::hypot(1.0, t);
                const double sn = cs * t;
                for (int c = 0; c < 3; ++c) {
                    const double a = w[c][p], b = w[c][q];
                    w[c][p] = cs * a - sn * b;
                    w[c][q] = sn * a + cs * b;
                }
                for (int r = 0; r < 3; ++r) {
                    const double a = v[r][p], b = v[r][q];
                    v[r][p] = cs * a - sn * b;
                    v[r][q] = sn * a + cs * b;
                }
            }
        }
        if (!rotated) break;
    }
    double sig2[3], smax = 0, smin = INFINITY;
    for (int j = 0; j < 3; ++j) {
        sig2[j] = w[0][j] * w[0][j] + w[1][j] * w[1][j] + w[2][j] * w[2][j];
        if (j < k) {
            const double s = std::sqrt(sig2[j]);
            smax = std::fmax(smax, s);
            smin = std::fmin(smin, s);
        }
    }
    if (!(smin > eps * 3 * std::fmax(smax, 1.0))) return false;
    for (int c = 0; c < 3; ++c)
        for (int a = 0; a < 3; ++a) {
            double acc = 0;
            for (int j = 0; j < 3; ++j)
                if (j < k) acc += w[c][j] * v[a][j] / sig2[j];
            dual[c][a] = a < k ? acc : 0.0;
        }
    return true;
}

void cross3(const double a[3], const double b[3], double o[3]) {
    o[0] = a[1] * b[2] - a[2] * b[1];
    o[1] = a[2] * b[0] - a[0] * b[2];
    o[2] = a[0] * b[1] - a[1] * b[0];
}

void normalize3(double v[3]) {
    const double n = std::sqrt(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
    if (n > 0 && std::isfinite(n)) {
        v[0] /= n;
        v[1] /= n;
        v[2] /= n;
    }
}

// One structure: metadata, then its atoms' representatives and the plan.
struct Structure {
    int64_t atom0 = 0, n = 0;
    int active = 0;            // bit a: axis a periodic
    int32_t reps[3] = {0, 0, 0};
    int64_t nimages = 1;
    double dual[3][3] = {};    // column a: dual vector of axis a (0 on non-periodic axes)
    double grid[3][3] = {};    // row a: grid direction of axis a
    uint32_t flags = 0;
    // planning
    bool cell_list = false;
    int nb[3] = {1, 1, 1};
    int reach[3] = {1, 1, 1};
    double lo[3] = {0, 0, 0};
    double inv_w[3] = {1, 1, 1};
    std::vector<int64_t> bin_start;  // nb0*nb1*nb2 + 1
    std::vector<int32_t> binned;     // atoms (structure-local) in bin order
};

// Metadata of structure b (geometry.cpp:123-219), after setup_structure of
// the device pipeline.
void setup_structure(const int64_t* bp, const double cell[3][3], const uint8_t* pbc,
                     int64_t nb, int64_t n_atoms, double cutoff, int64_t b, Structure& r) {
    uint32_t st = 0;
    const int64_t lo = bp[b], hi = bp[b + 1];
    if (b == 0 && lo != 0) st |= E_BP_START;
    if (b == nb - 1 && hi != n_atoms) st |= E_BP_END;
    if (hi < lo) st |= E_BP_ORDER;
    r.atom0 = lo;
    r.n = hi > lo ? hi - lo : 0;
    bool finite = true;
    for (int a = 0; a < 3; ++a)
        for (int c = 0; c < 3; ++c) finite = finite && std::isfinite(cell[a][c]);
    if (!finite) st |= E_CELL_NONFINITE;
    const bool px = pbc[3 * b] != 0, py = pbc[3 * b + 1] != 0, pz = pbc[3 * b + 2] != 0;
    const int k = (int)px + (int)py + (int)pz;
    r.active = (px ? 1 : 0) | (py ? 2 : 0) | (pz ? 4 : 0);
    int slot_axis[3];  // the periodic axes first, then the others, in axis order
    {
        int j = 0;
        for (int a = 0; a < 3; ++a)
            if (r.active >> a & 1) slot_axis[j++] = a;
        for (int a = 0; a < 3; ++a)
            if (!(r.active >> a & 1)) slot_axis[j++] = a;
    }
    for (int e = 0; e < 9; ++e) {
        r.dual[e / 3][e % 3] = 0.0;
        r.grid[e / 3][e % 3] = (e % 4 == 0) ? 1.0 : 0.0;
    }
    if (finite && r.n > 0) {
        double w[3][3], dual_slot[3][3] = {};
        for (int j = 0; j < 3; ++j)
            for (int c = 0; c < 3; ++c) w[c][j] = j >= k ? 0.0 : cell[slot_axis[j]][c];
        if (k > 0 && !active_pinv(w, k, dual_slot)) st |= E_CELL_RANK;
        int64_t reps[3] = {0, 0, 0};
        if (!(st & E_CELL_RANK)) {
            for (int j = 0; j < k; ++j) {
                const double n2 = dual_slot[0][j] * dual_slot[0][j] +
                                  dual_slot[1][j] * dual_slot[1][j] +
                                  dual_slot[2][j] * dual_slot[2][j];
                if (!std::isfinite(n2) || !std::isfinite(dual_slot[0][j]) ||
                    !std::isfinite(dual_slot[1][j]) || !std::isfinite(dual_slot[2][j]))
                    st |= E_DUAL_RANGE;
                const double rep = std::ceil(cutoff * std::sqrt(n2));
                if (!(rep <= 2147483647.0))
                    st |= E_REPEAT_RANGE;
                else
                    reps[j] = (int64_t)rep;
            }
        }
        int64_t rep_axis[3] = {0, 0, 0};
        for (int j = 0; j < k; ++j) {
            const int a = slot_axis[j];
            rep_axis[a] = reps[j];
            for (int c = 0; c < 3; ++c) r.dual[c][a] = dual_slot[c][j];
        }
        const bool geometry_ok = !(st & (E_REPEAT_RANGE | E_CELL_RANK | E_DUAL_RANGE));
        int64_t count = 1;
        if (geometry_ok) {
            for (int a = 0; a < 3; ++a) {
                const int64_t f = 2 * rep_axis[a] + 1;
                if (!(st & E_IMAGE_CAP)) {
                    if (count > kImageCap / f)
                        st |= E_IMAGE_CAP;
                    else
                        count *= f;
                }
            }
        }
        if (geometry_ok && !(st & E_IMAGE_CAP)) {
            r.nimages = count;
            for (int a = 0; a < 3; ++a) r.reps[a] = (int32_t)rep_axis[a];
        }
        // grid frame: duals on periodic axes, orthonormal complements elsewhere
        double g[3][3] = {{1, 0, 0}, {0, 1, 0}, {0, 0, 1}};
        for (int a = 0; a < 3; ++a)
            if (r.active >> a & 1)
                for (int c = 0; c < 3; ++c) g[a][c] = r.dual[c][a];
        if (k == 2) {
            double nrm[3];
            cross3(cell[slot_axis[0]], cell[slot_axis[1]], nrm);
            normalize3(nrm);
            for (int c = 0; c < 3; ++c) g[slot_axis[2]][c] = nrm[c];
        } else if (k == 1) {
            double rr[3] = {cell[slot_axis[0]][0], cell[slot_axis[0]][1], cell[slot_axis[0]][2]};
            normalize3(rr);
            double unit[3] = {0, 0, 0};
            if (std::fabs(rr[0]) <= std::fabs(rr[1]) && std::fabs(rr[0]) <= std::fabs(rr[2]))
                unit[0] = 1;
            else if (std::fabs(rr[1]) <= std::fabs(rr[2]))
                unit[1] = 1;
            else
                unit[2] = 1;
            double e1[3], e2[3];
            cross3(rr, unit, e1);
            normalize3(e1);
            cross3(rr, e1, e2);
            normalize3(e2);
            for (int c = 0; c < 3; ++c) {
                g[slot_axis[1]][c] = e1[c];
                g[slot_axis[2]][c] = e2[c];
            }
        }
        for (int e = 0; e < 9; ++e) r.grid[e / 3][e % 3] = g[e / 3][e % 3];
    }
    r.flags = st;
}

// floor(sum_c x_c y_c) with double-double accumulation (nearly exact), as
// the reference's long-double fractional coordinate (neighbors_cpu.cpp:110-
// 122); *ok becomes false when the value is non-finite or outside
// [-2^31, 2^31).
int wrap_of(const double x[3], const double y[3], bool* ok) {
    double hi = 0, lo = 0;
    for (int c = 0; c < 3; ++c) {
        const double p = x[c] * y[c];
        const double pe = std::fma(x[c], y[c], -p);
        const double s = hi + p;
        const double bb = s - hi;
        const double se = (hi - (s - bb)) + (p - bb);
        lo += pe + se;
        hi = s;
    }
    const double s = hi + lo;
    lo = lo - (s - hi);
    hi = s;
    if (!std::isfinite(hi)) {
        *ok = false;
        return 0;
    }
    double f = std::floor(hi);
    if (hi == f && lo < 0) f -= 1.0;
    if (!(f >= -2147483648.0 && f <= 2147483647.0)) {
        *ok = false;
        return 0;
    }
    return (int)f;
}

// ------------------------------------------------------------- threads
//
// One worker pool per process, as the reference's CPU provider keeps
// (thread_pool.cpp:22-191): workers are started on demand, kept, and reused
// by every later call, so a small search with several threads does not pay
// for starting them.  A job hands out tickets, one per helper it asks for;
// a worker that takes a ticket runs the job's items with the caller until
// none are left.  Tickets still queued when the caller has run out of items
// are withdrawn, so a job never waits for workers busy with another one.
// A worker that cannot be started leaves the pool smaller (the job runs on
// fewer threads); an exception thrown by an item stops the job's other
// items and is rethrown to the caller.  After fork() the child starts a new
// pool (its parent's workers do not exist in it).

class WorkerPool {
  public:
    static WorkerPool& instance();

    // f(i) for i in [0, n) on the calling thread and up to `helpers` workers.
    void run(int64_t n, int64_t helpers, const std::function<void(int64_t)>& f);

  private:
    struct Job {
        const std::function<void(int64_t)>* f;
        int64_t n;
        std::atomic<int64_t> next{0};
        std::atomic<bool> stop{false};
        std::exception_ptr error;  // the first item's exception (under mu_)
        int running = 0;           // workers inside this job (under mu_)
        std::condition_variable idle;
    };

    void grow(int64_t workers);
    void work(Job& job);
    void loop();

    std::mutex mu_;
    std::condition_variable wake_;
    std::deque<Job*> tickets_;
    int64_t workers_ = 0;
};

namespace {
std::mutex g_pool_mu;
WorkerPool* g_pool = nullptr;
bool g_atfork = false;

void pool_prepare() { g_pool_mu.lock(); }
void pool_parent() { g_pool_mu.unlock(); }
void pool_child() {
    // the parent's workers do not exist here: the old pool is left as it is
    // (its state may be mid-update) and a new one is made on demand
    g_pool = nullptr;
    g_pool_mu.unlock();
}

// Workers at most: a few per hardware thread.
int64_t worker_cap() {
    const int64_t hw = (int64_t)std::thread::hardware_concurrency();
    return std::max<int64_t>(1, std::min<int64_t>(4 * std::max<int64_t>(hw, 1), 1024));
}
}  // namespace

WorkerPool& WorkerPool::instance() {
    std::lock_guard<std::mutex> guard(g_pool_mu);
    if (!g_atfork) g_atfork = pthread_atfork(pool_prepare, pool_parent, pool_child) == 0;
    // held until the process ends: workers wait on it until then
    if (!g_pool) g_pool = new WorkerPool();
    return *g_pool;
}

// Workers run with 1 MiB stacks (the search keeps its data on the heap),
// detached: the pool outlives them.
void WorkerPool::grow(int64_t workers) {
    std::lock_guard<std::mutex> guard(mu_);
    if (workers_ >= workers) return;
    pthread_attr_t attr;
    if (pthread_attr_init(&attr) != 0) return;
    pthread_attr_setstacksize(&attr, size_t{1} << 20);
    pthread_attr_setdetachstate(&attr, PTHREAD_CREATE_DETACHED);
    while (workers_ < workers) {
        pthread_t id;
        auto entry = [](void* self) -> void* {
            static_cast<WorkerPool*>(self)->loop();
            return nullptr;
        };
        // a worker that cannot start leaves the pool smaller
        if (pthread_create(&id, &attr, entry, this) != 0) break;
        ++workers_;
    }
    pthread_attr_destroy(&attr);
}

void WorkerPool::work(Job& job) {
    while (!job.stop.load(std::memory_order_relaxed)) {
        const int64_t i = job.next.fetch_add(1, std::memory_order_relaxed);
        if (i >= job.n) break;
        try {
            (*job.f)(i);
        } catch (...) {
            std::lock_guard<std::mutex> guard(mu_);
            if (!job.error) job.error = std::current_exception();
            job.stop.store(true, std::memory_order_relaxed);
        }
    }
}

void WorkerPool::loop() {
    for (;;) {
        Job* job;
        {
            std::unique_lock<std::mutex> lock(mu_);
            wake_.wait(lock, [this] { return !tickets_.empty(); });
            job = tickets_.front();
            tickets_.pop_front();
            ++job->running;
        }
        work(*job);
        std::lock_guard<std::mutex> guard(mu_);
        if (--job->running == 0) job->idle.notify_all();
    }
}

void WorkerPool::run(int64_t n, int64_t helpers, const std::function<void(int64_t)>& f) {
    Job job;
    job.f = &f;
    job.n = n;
    grow(helpers);
    {
        std::lock_guard<std::mutex> guard(mu_);
        helpers = std::min(helpers, workers_);
        for (int64_t k = 0; k < helpers; ++k) tickets_.push_back(&job);
    }
    if (helpers == 1)
        wake_.notify_one();
    else if (helpers > 1)
        wake_.notify_all();
    work(job);
    std::unique_lock<std::mutex> lock(mu_);
    tickets_.erase(std::remove(tickets_.begin(), tickets_.end(), &job), tickets_.end());
    job.idle.wait(lock, [&job] { return job.running == 0; });
    if (job.error) std::rethrow_exception(job.error);
}

// Runs f(i) for i in [0, n) on `threads` threads (the calling one included,
// the others from the process's worker pool), items taken in order from a
// shared counter.
template <typename F>
void parallel_for(int64_t n, int64_t threads, F f) {
    if (n <= 0) return;
    const int64_t nt = std::max<int64_t>(1, std::min({threads, n, worker_cap() + 1}));
    if (nt == 1) {
        for (int64_t i = 0; i < n; ++i) f(i);
        return;
    }
    const std::function<void(int64_t)> fn = [&f](int64_t i) { f(i); };
    WorkerPool::instance().run(n, nt - 1, fn);
}

// ------------------------------------------------------------- search

struct Pairs {
    std::vector<int64_t> idx;  // (source, target) per pair
    std::vector<int32_t> sh;   // S per pair
    uint32_t flags = 0;
};

template <typename T>
struct Atoms {
    std::vector<int32_t> w;  // wraps, 3 per atom
    std::vector<T> q;        // wrapped positions, 3 per atom
    std::vector<double> u;   // grid coordinates, 3 per atom
};

// The public predicate: D = (((p_t - p_s) + S0 c0) + S1 c1) + S2 c2 and
// d^2 = (D0^2 + D1^2) + D2^2, every operation rounded in T.
template <typename T>
inline T public_d2(const T* ps, const T* pt, const int64_t S[3], const T* cell) {
    const T s0 = (T)S[0], s1 = (T)S[1], s2 = (T)S[2];
    T D[3];
    for (int c = 0; c < 3; ++c) {
        T comp = pt[c] - ps[c];
        comp = comp + s0 * cell[c];
        comp = comp + s1 * cell[3 + c];
        comp = comp + s2 * cell[6 + c];
        D[c] = comp;
    }
    T d2 = D[0] * D[0];
    d2 = d2 + D[1] * D[1];
    d2 = d2 + D[2] * D[2];
    return d2;
}

// Identity rule of pair_policy.h:42-79 for the output shift S.
inline bool identity_ok(int64_t s, int64_t t, const int64_t S[3], bool half, bool self) {
    const bool zero = S[0] == 0 && S[1] == 0 && S[2] == 0;
    if (s == t && zero) return self;
    if (!half) return true;
    if (s < t) return true;
    if (s > t) return false;
    // s == t: keep the lexicographically negative shift of (S, -S)
    for (int c = 0; c < 3; ++c)
        if (S[c] != 0) return S[c] < 0;
    return false;
}

template <typename T>
inline void consider(const T* pos, const T* cell, int64_t s, int64_t t, const int64_t S[3],
                     T cut2, bool half, bool self, Pairs& out) {
    if (!identity_ok(s, t, S, half, self)) return;
    if (!(public_d2(pos + 3 * s, pos + 3 * t, S, cell) < cut2)) return;
    for (int c = 0; c < 3; ++c) {
        if (S[c] < INT32_MIN || S[c] > INT32_MAX) {
            out.flags |= E_SHIFT_RANGE;
            return;
        }
    }
    out.idx.push_back(s);
    out.idx.push_back(t);
    out.sh.push_back((int32_t)S[0]);
    out.sh.push_back((int32_t)S[1]);
    out.sh.push_back((int32_t)S[2]);
}

inline int64_t floor_div(int64_t a, int64_t b) {
    int64_t q = a / b;
    if ((a % b != 0) && ((a < 0) != (b < 0))) --q;
    return q;
}

// Sources [s0, s1) (global indices) of structure r.
template <typename T>
void search_sources(const Structure& r, const T* pos, const T* cell, const Atoms<T>& at,
                    T cut2, bool half, bool self, int64_t s0, int64_t s1, Pairs& out) {
    const int64_t a0 = r.atom0, n = r.n;
    if (!r.cell_list) {
        const int R0 = (r.active & 1) ? r.reps[0] : 0, R1 = (r.active & 2) ? r.reps[1] : 0,
                  R2 = (r.active & 4) ? r.reps[2] : 0;
        for (int64_t s = s0; s < s1; ++s) {
            const int32_t* ws = &at.w[3 * s];
            for (int64_t t = a0; t < a0 + n; ++t) {
                const int32_t* wt = &at.w[3 * t];
                for (int k0 = -R0; k0 <= R0; ++k0)
                    for (int k1 = -R1; k1 <= R1; ++k1)
                        for (int k2 = -R2; k2 <= R2; ++k2) {
                            const int64_t S[3] = {(int64_t)k0 - wt[0] + ws[0],
                                                  (int64_t)k1 - wt[1] + ws[1],
                                                  (int64_t)k2 - wt[2] + ws[2]};
                            consider(pos, cell, s, t, S, cut2, half, self, out);
                        }
            }
        }
        return;
    }
    const int nb0 = r.nb[0], nb1 = r.nb[1], nb2 = r.nb[2];
    for (int64_t s = s0; s < s1; ++s) {
        int ib[3];
        for (int a = 0; a < 3; ++a) {
            const double x = (at.u[3 * s + a] - r.lo[a]) * r.inv_w[a];
            const double f = std::floor(x);
            ib[a] = f < 0 ? 0 : (f >= r.nb[a] ? r.nb[a] - 1 : (int)f);
        }
        const int32_t* ws = &at.w[3 * s];
        // unwrapped bin ranges per axis
        int lo[3], hi[3];
        for (int a = 0; a < 3; ++a) {
            if (r.active >> a & 1) {
                lo[a] = ib[a] - r.reach[a];
                hi[a] = ib[a] + r.reach[a];
            } else {
                lo[a] = std::max(ib[a] - r.reach[a], 0);
                hi[a] = std::min(ib[a] + r.reach[a], r.nb[a] - 1);
            }
        }
        for (int J0 = lo[0]; J0 <= hi[0]; ++J0) {
            const int64_t k0 = (r.active & 1) ? floor_div(J0, nb0) : 0;
            const int j0 = (int)(J0 - k0 * nb0);
            for (int J1 = lo[1]; J1 <= hi[1]; ++J1) {
                const int64_t k1 = (r.active & 2) ? floor_div(J1, nb1) : 0;
                const int j1 = (int)(J1 - k1 * nb1);
                for (int J2 = lo[2]; J2 <= hi[2]; ++J2) {
                    const int64_t k2 = (r.active & 4) ? floor_div(J2, nb2) : 0;
                    const int j2 = (int)(J2 - k2 * nb2);
                    const int64_t bin = ((int64_t)j0 * nb1 + j1) * nb2 + j2;
                    for (int64_t x = r.bin_start[bin]; x < r.bin_start[bin + 1]; ++x) {
                        const int64_t t = a0 + r.binned[x];
                        const int32_t* wt = &at.w[3 * t];
                        const int64_t S[3] = {k0 - wt[0] + ws[0], k1 - wt[1] + ws[1],
                                              k2 - wt[2] + ws[2]};
                        consider(pos, cell, s, t, S, cut2, half, self, out);
                    }
                }
            }
        }
    }
}

// Whether the reference's CPU path refuses an explicit cell_list for
// structure r ("cell_list cannot safely process this structure"), evaluated
// as it does: the operation scale and padding in long double from the
// largest |position| per component and the largest |wrap| and |image shift|
// per axis (neighbors_cpu.cpp:157-218), the search cutoff rounded to T and
// moved up one ulp, then the dense bin layout over the wrapped positions in
// T arithmetic, with its caps on bins and bins per atom image
// (neighbors_cpu.cpp:380-430).
template <typename T>
bool reference_refuses_cell_list(const Structure& r, const T* pos, const double cell[3][3],
                                 const Atoms<T>& at, T cutoff) {
    constexpr int64_t kDenseBins = int64_t{1} << 26;
    constexpr int64_t kBinsPerImage = 64;
    const int64_t a0 = r.atom0, n = r.n;
    long double maxp[3] = {0.0L, 0.0L, 0.0L};
    int64_t maxw[3] = {0, 0, 0};
    T lo[3], hi[3];
    for (int c = 0; c < 3; ++c) {
        lo[c] = std::numeric_limits<T>::infinity();
        hi[c] = -std::numeric_limits<T>::infinity();
    }
    for (int64_t i = a0; i < a0 + n; ++i)
        for (int c = 0; c < 3; ++c) {
            const T q = at.q[3 * i + c];
            if (!std::isfinite(q)) return true;
            maxp[c] = std::max(maxp[c], std::fabs((long double)pos[3 * i + c]));
            maxw[c] = std::max<int64_t>(maxw[c], std::llabs((long long)at.w[3 * i + c]));
            lo[c] = std::min(lo[c], q);
            hi[c] = std::max(hi[c], q);
        }
    long double scale = 0.0L;
    for (int c = 0; c < 3; ++c) {
        long double comp = 2 * maxp[c];
        for (int a = 0; a < 3; ++a)
            comp += (long double)((int64_t)r.reps[a] + 2 * maxw[a]) *
                    std::fabs((long double)(T)cell[a][c]);
        scale = std::max(scale, comp);
    }
    const long double padded =
        (long double)cutoff + 64 * (long double)std::numeric_limits<T>::epsilon() * scale;
    if (!std::isfinite(padded) || padded > 2 * (long double)cutoff ||
        padded > (long double)std::numeric_limits<T>::max())
        return true;
    const T size = std::nextafter((T)padded, std::numeric_limits<T>::infinity());
    if (!std::isfinite(size) || size == T(0)) return true;
    int64_t count = 1;
    for (int c = 0; c < 3; ++c) {
        const T span = hi[c] - lo[c] + 2 * size;
        const T dim = span / size;
        if (!std::isfinite(dim) || dim > (T)kDenseBins) return true;
        const int64_t d = std::max<int64_t>(1, (int64_t)std::ceil(dim));
        if (count > kDenseBins / d) return true;
        count *= d;
    }
    if (n > std::numeric_limits<int64_t>::max() / r.nimages) return true;
    return !(count <= kDenseBins && (count + kBinsPerImage - 1) / kBinsPerImage <= n * r.nimages);
}

// Plans structure r from its atoms: the broad-phase margin pad = 64 eps_T
// max(scale, rc) with the operation scale of neighbors_cpu.cpp:156-219
// (2 max|p| + sum_a (R_a + 2 max|w|) |cell_ac|, maximised over c), the
// reference's cell_list layout rule for an explicit cell_list request
// (neighbors_cpu.cpp:379-430: bins of rc + pad over the bounding box of the
// wrapped positions), the algorithm and the bins.
template <typename T>
void plan_structure(Structure& r, const T* pos, const double cell[3][3], const Atoms<T>& at,
                    double cutoff, int algorithm) {
    const int64_t a0 = r.atom0, n = r.n;
    double maxp = 0;
    int64_t maxw = 0;
    double qlo[3] = {INFINITY, INFINITY, INFINITY}, qhi[3] = {-INFINITY, -INFINITY, -INFINITY};
    double ulo[3] = {INFINITY, INFINITY, INFINITY}, uhi[3] = {-INFINITY, -INFINITY, -INFINITY};
    for (int64_t i = a0; i < a0 + n; ++i) {
        for (int c = 0; c < 3; ++c) {
            maxp = std::fmax(maxp, std::fabs((double)pos[3 * i + c]));
            maxw = std::max<int64_t>(maxw, std::llabs((long long)at.w[3 * i + c]));
            const double q = (double)at.q[3 * i + c], u = at.u[3 * i + c];
            qlo[c] = std::fmin(qlo[c], q);
            qhi[c] = std::fmax(qhi[c], q);
            ulo[c] = std::fmin(ulo[c], u);
            uhi[c] = std::fmax(uhi[c], u);
        }
    }
    const double rc = cutoff;
    double scale = 0;
    for (int c = 0; c < 3; ++c) {
        double sc = 2 * maxp;
        for (int a = 0; a < 3; ++a)
            sc += ((double)r.reps[a] + 2 * (double)maxw) * std::fabs(cell[a][c]);
        scale = std::fmax(scale, sc);
    }
    const double pad = 64.0 * Limits<T>::eps * std::fmax(scale, rc);
    const bool safe = std::isfinite(rc + pad) && rc + pad <= 2 * rc && rc + pad <= Limits<T>::max;
    if (algorithm == kCellList && reference_refuses_cell_list<T>(r, pos, cell, at, (T)cutoff))
        r.flags |= E_CELL_UNSAFE;
    const bool large = (double)n * (double)r.nimages > (double)kAutoCandidates;
    bool want_cell = algorithm == kCellList || (algorithm == kAuto && large);
    if (!safe) want_cell = false;
    r.cell_list = false;
    if (!want_cell || (r.flags & E_CELL_UNSAFE)) return;
    // bins at least rc + 2 pad wide along every grid direction
    const double rcu = rc + 2 * pad;
    double rad[3], w[3], ext[3];
    for (int a = 0; a < 3; ++a) {
        const double gn = std::sqrt(r.grid[a][0] * r.grid[a][0] + r.grid[a][1] * r.grid[a][1] +
                                    r.grid[a][2] * r.grid[a][2]);
        rad[a] = rcu * gn * (1.0 + 1e-9);
        if (!(rad[a] > 0) || !std::isfinite(rad[a])) return;
        if (r.active >> a & 1) {
            r.lo[a] = 0.0;
            r.nb[a] = (int)std::fmin(std::fmax(std::floor(1.0 / rad[a]), 1.0), 1048576.0);
            r.inv_w[a] = r.nb[a];
            r.reach[a] = (int)std::floor(rad[a] * r.nb[a]) + 1;
            ext[a] = 1.0;
            w[a] = 1.0 / r.nb[a];
        } else {
            r.lo[a] = ulo[a];
            ext[a] = std::fmax(uhi[a] - ulo[a], 0.0);
            if (!std::isfinite(ext[a]) || !std::isfinite(ulo[a])) return;
            w[a] = rad[a];
            if (ext[a] / w[a] > 1048575.0) w[a] = ext[a] / 1048575.0 * (1.0 + 1e-9);
            r.nb[a] = (int)std::fmin(std::floor(ext[a] / w[a]) + 1.0, 1048576.0);
            r.inv_w[a] = 1.0 / w[a];
            r.reach[a] = 1;
        }
    }
    // at most 2 n + 64 bins: coarsen the axis with the most bins
    const double capb = 2.0 * (double)n + 64.0;
    for (int it = 0; it < 200 && (double)r.nb[0] * r.nb[1] * r.nb[2] > capb; ++it) {
        const int a = (r.nb[0] >= r.nb[1] && r.nb[0] >= r.nb[2]) ? 0 : (r.nb[1] >= r.nb[2] ? 1 : 2);
        if (r.nb[a] == 1) break;
        if (r.active >> a & 1) {
            r.nb[a] = (r.nb[a] + 1) / 2;
            r.inv_w[a] = r.nb[a];
            r.reach[a] = (int)std::floor(rad[a] * r.nb[a]) + 1;
        } else {
            w[a] *= 2.0;
            r.nb[a] = (int)std::fmin(std::floor(ext[a] / w[a]) + 1.0, 1048576.0);
            r.inv_w[a] = 1.0 / w[a];
        }
    }
    const int64_t nbins = (int64_t)r.nb[0] * r.nb[1] * r.nb[2];
    if ((double)nbins > capb + 1.0 || r.reach[0] > 1 << 20 || r.reach[1] > 1 << 20 ||
        r.reach[2] > 1 << 20)
        return;
    // counting sort of the structure's atoms by bin
    std::vector<int64_t> bin_of((size_t)n);
    r.bin_start.assign((size_t)nbins + 1, 0);
    for (int64_t x = 0; x < n; ++x) {
        const int64_t i = a0 + x;
        int ib[3];
        for (int a = 0; a < 3; ++a) {
            const double f = std::floor((at.u[3 * i + a] - r.lo[a]) * r.inv_w[a]);
            ib[a] = f < 0 ? 0 : (f >= r.nb[a] ? r.nb[a] - 1 : (int)f);
        }
        const int64_t bin = ((int64_t)ib[0] * r.nb[1] + ib[1]) * r.nb[2] + ib[2];
        bin_of[(size_t)x] = bin;
        ++r.bin_start[(size_t)bin + 1];
    }
    for (int64_t b = 0; b < nbins; ++b) r.bin_start[(size_t)b + 1] += r.bin_start[(size_t)b];
    std::vector<int64_t> fill(r.bin_start.begin(), r.bin_start.end() - 1);
    r.binned.assign((size_t)n, 0);
    for (int64_t x = 0; x < n; ++x) r.binned[(size_t)fill[(size_t)bin_of[(size_t)x]]++] = (int32_t)x;
    r.cell_list = true;
}

// Representative wraps floor(p . dual_a) (duals rounded to T, as the
// reference stores them), wrapped positions q = p - sum_a w_a cell_a rounded
// in T in that order, and grid coordinates of the atoms [i0, i1) of
// structure r; returns the atoms' error bits.
template <typename T>
uint32_t prepare_atoms(const Structure& r, const T* pos, const T* cell, int64_t i0, int64_t i1,
                       Atoms<T>& at) {
    uint32_t st = 0;
    for (int64_t i = i0; i < i1; ++i) {
        const T* p = pos + 3 * i;
        bool finite = std::isfinite((double)p[0]) && std::isfinite((double)p[1]) &&
                      std::isfinite((double)p[2]);
        int w[3] = {0, 0, 0};
        T q[3] = {T(0), T(0), T(0)};
        if (!finite) {
            st |= E_POS_NONFINITE;
        } else {
            const double pd[3] = {(double)p[0], (double)p[1], (double)p[2]};
            bool ok = true;
            for (int a = 0; a < 3; ++a) {
                const double dcol[3] = {(double)(T)r.dual[0][a], (double)(T)r.dual[1][a],
                                        (double)(T)r.dual[2][a]};
                w[a] = wrap_of(pd, dcol, &ok);
            }
            if (!ok) {
                st |= E_WRAP_RANGE;
                w[0] = w[1] = w[2] = 0;
            } else {
                for (int c = 0; c < 3; ++c) {
                    T x = p[c];
                    for (int a = 0; a < 3; ++a) x = x - (T)w[a] * cell[3 * a + c];
                    q[c] = x;
                }
            }
        }
        for (int a = 0; a < 3; ++a) {
            at.w[3 * i + a] = w[a];
            at.q[3 * i + a] = q[a];
            at.u[3 * i + a] = r.grid[a][0] * (double)q[0] + r.grid[a][1] * (double)q[1] +
                              r.grid[a][2] * (double)q[2];
        }
    }
    return st;
}

struct Task {
    int64_t structure, s0, s1;
};

}  // namespace tnr_cpu

struct tnr_cpu_result {
    std::vector<tnr_cpu::Pairs> parts;
    int64_t n_pairs = 0;
};

namespace tnr_cpu {

uint32_t first_flag_message(uint32_t flags, int* code, const char** text) {
    for (const auto& m : kMessages)
        if (flags & m.bit) {
            *code = m.code;
            *text = m.text;
            return m.bit;
        }
    *code = kSearchError;
    *text = "invalid neighbor-list status";
    return 0;
}

template <typename T>
int search(const T* pos, int64_t n_atoms, const int64_t* bp, int64_t nb, const T* cells,
           const uint8_t* pbc, double cutoff, bool half, bool self, int algorithm,
           int64_t threads, tnr_cpu_result* res, char* err, size_t err_len) {
    // batch_ptr (neighbors_cpu.cpp:1000-1014), then per-structure metadata
    uint32_t flags = 0;
    if (bp[0] != 0) flags |= E_BP_START;
    if (bp[nb] != n_atoms) flags |= E_BP_END;
    for (int64_t b = 0; b < nb; ++b)
        if (bp[b + 1] < bp[b]) flags |= E_BP_ORDER;
    std::vector<Structure> st((size_t)nb);
    std::vector<double> cell_d((size_t)(9 * nb));
    for (int64_t e = 0; e < 9 * nb; ++e) cell_d[(size_t)e] = (double)cells[e];
    if (!(flags & (E_BP_START | E_BP_END | E_BP_ORDER))) {
        parallel_for(nb, threads, [&](int64_t b) {
            const double(*c)[3] = reinterpret_cast<const double(*)[3]>(&cell_d[(size_t)(9 * b)]);
            setup_structure(bp, c, pbc, nb, n_atoms, cutoff, b, st[(size_t)b]);
        });
        int64_t images = 0;
        for (const auto& r : st) {
            flags |= r.flags;
            if (r.n > 0 && !(r.flags & (E_CELL_RANK | E_DUAL_RANGE | E_REPEAT_RANGE | E_IMAGE_CAP)))
                images += r.nimages;
        }
        if (images > kImageCap) flags |= E_BATCH_IMAGE_CAP;
    }
    if (flags) {
        int code;
        const char* text;
        first_flag_message(flags, &code, &text);
        return put_error(err, err_len, code, text);
    }
    // atoms: representatives, wrapped positions, grid coordinates
    Atoms<T> at;
    at.w.assign((size_t)(3 * n_atoms), 0);
    at.q.assign((size_t)(3 * n_atoms), T(0));
    at.u.assign((size_t)(3 * n_atoms), 0.0);
    constexpr int64_t kAtomChunk = 4096;
    const int64_t n_chunks = (n_atoms + kAtomChunk - 1) / kAtomChunk;
    std::vector<uint32_t> chunk_flags((size_t)std::max<int64_t>(n_chunks, 1), 0);
    parallel_for(n_chunks, threads, [&](int64_t c) {
        const int64_t i0 = c * kAtomChunk, i1 = std::min(n_atoms, i0 + kAtomChunk);
        // the structures of [i0, i1): from the last b with bp[b] <= i0
        int64_t lo = 0, hi = nb;
        while (hi - lo > 1) {
            const int64_t mid = (lo + hi) / 2;
            if (bp[mid] <= i0) lo = mid; else hi = mid;
        }
        uint32_t f = 0;
        for (int64_t b = lo; b < nb && bp[b] < i1; ++b) {
            const int64_t a = std::max(i0, bp[b]), z = std::min(i1, bp[b + 1]);
            if (a < z) f |= prepare_atoms(st[(size_t)b], pos, cells + 9 * b, a, z, at);
        }
        chunk_flags[(size_t)c] = f;
    });
    for (uint32_t f : chunk_flags) flags |= f;
    if (!flags) {
        parallel_for(nb, threads, [&](int64_t b) {
            Structure& r = st[(size_t)b];
            if (r.n == 0) return;
            const double(*c)[3] = reinterpret_cast<const double(*)[3]>(&cell_d[(size_t)(9 * b)]);
            plan_structure<T>(r, pos, c, at, cutoff, algorithm);
        });
        for (const auto& r : st) flags |= r.flags;
    }
    if (flags) {
        int code;
        const char* text;
        first_flag_message(flags, &code, &text);
        return put_error(err, err_len, code, text);
    }
    // tasks: runs of sources, in structure and source order; about eight
    // per thread, of 16 to kSourcesPerTask sources
    const int64_t per_task =
        std::max<int64_t>(16, std::min<int64_t>(kSourcesPerTask, n_atoms / (8 * threads)));
    std::vector<Task> tasks;
    for (int64_t b = 0; b < nb; ++b) {
        const Structure& r = st[(size_t)b];
        for (int64_t s = 0; s < r.n; s += per_task)
            tasks.push_back({b, r.atom0 + s, r.atom0 + std::min(r.n, s + per_task)});
    }
    res->parts.assign(tasks.size(), Pairs());
    const T cut2 = (T)(cutoff * cutoff);
    parallel_for((int64_t)tasks.size(), threads, [&](int64_t k) {
        const Task& tk = tasks[(size_t)k];
        search_sources<T>(st[(size_t)tk.structure], pos, cells + 9 * tk.structure, at, cut2, half,
                          self, tk.s0, tk.s1, res->parts[(size_t)k]);
    });
    int64_t total = 0;
    for (const auto& part : res->parts) {
        flags |= part.flags;
        total += (int64_t)(part.idx.size() / 2);
    }
    if (flags) {
        int code;
        const char* text;
        first_flag_message(flags, &code, &text);
        return put_error(err, err_len, code, text);
    }
    res->n_pairs = total;
    return kOk;
}

}  // namespace tnr_cpu

extern "C" {

int tnr_cpu_abi_version(void) { return TNR_CPU_ABI_VERSION; }

int tnr_cpu_search(int32_t dtype, const void* positions, int64_t n_atoms,
                   const int64_t* batch_ptr, int64_t n_structures, const void* cell,
                   const uint8_t* pbc, double cutoff, int32_t half_list, int32_t include_self,
                   int32_t algorithm, int64_t threads, tnr_cpu_result** result,
                   int64_t* n_pairs, char* err, size_t err_len) {
    using namespace tnr_cpu;
    if (!result || !n_pairs) return put_error(err, err_len, kInputError, "result pointers are null");
    *result = nullptr;
    *n_pairs = 0;
    if (dtype != kFloat32 && dtype != kFloat64)
        return put_error(err, err_len, kInputError, "positions must have dtype float32 or float64");
    if (algorithm < kAuto || algorithm > kCellList)
        return put_error(err, err_len, kInputError,
                         "algorithm must be 'auto', 'brute_force', or 'cell_list'");
    if (!(std::isfinite(cutoff) && cutoff > 0))
        return put_error(err, err_len, kInputError, "cutoff must be finite and positive");
    if (threads <= 0)
        return put_error(err, err_len, kInputError, "num_threads must be a positive integer");
    if (n_atoms < 0 || n_structures < 0) return put_error(err, err_len, kInputError, "invalid sizes");
    if (!batch_ptr || (n_structures > 0 && (!cell || !pbc)) || (n_atoms > 0 && !positions))
        return put_error(err, err_len, kInputError, "required pointers are null");
    if (n_atoms >= (int64_t)std::numeric_limits<int32_t>::max())
        return put_error(err, err_len, kInputError,
                         "the current implementation supports fewer than 2^31 atoms");
    tnr_cpu_result* res = new (std::nothrow) tnr_cpu_result();
    if (!res) return put_error(err, err_len, kSearchError, "out of host memory");
    int rc;
    try {
        rc = dtype == kFloat32
                 ? search<float>((const float*)positions, n_atoms, batch_ptr, n_structures,
                                 (const float*)cell, pbc, cutoff, half_list != 0,
                                 include_self != 0, algorithm, threads, res, err, err_len)
                 : search<double>((const double*)positions, n_atoms, batch_ptr, n_structures,
                                  (const double*)cell, pbc, cutoff, half_list != 0,
                                  include_self != 0, algorithm, threads, res, err, err_len);
    } catch (const std::bad_alloc&) {
        rc = put_error(err, err_len, kSearchError, "out of host memory");
    } catch (...) {
        rc = put_error(err, err_len, kSearchError, "the host search failed");
    }
    if (rc != kOk) {
        delete res;
        return rc;
    }
    *result = res;
    *n_pairs = res->n_pairs;
    return kOk;
}

void tnr_cpu_copy(const tnr_cpu_result* result, int64_t* pairs, int32_t* shifts,
                  int64_t threads) {
    if (!result) return;
    const auto& parts = result->parts;
    std::vector<int64_t> off(parts.size() + 1, 0);
    for (size_t k = 0; k < parts.size(); ++k) off[k + 1] = off[k] + (int64_t)(parts[k].idx.size() / 2);
    auto copy = [&](int64_t k) {
        const auto& part = parts[(size_t)k];
        if (part.idx.empty()) return;
        if (pairs)
            std::memcpy(pairs + 2 * off[(size_t)k], part.idx.data(), part.idx.size() * sizeof(int64_t));
        if (shifts)
            std::memcpy(shifts + 3 * off[(size_t)k], part.sh.data(), part.sh.size() * sizeof(int32_t));
    };
    try {
        tnr_cpu::parallel_for((int64_t)parts.size(), threads < 1 ? 1 : threads, copy);
    } catch (...) {
        // the pool could not be reached (out of memory): copy on this thread
        for (int64_t k = 0; k < (int64_t)parts.size(); ++k) copy(k);
    }
}

void tnr_cpu_free(tnr_cpu_result* result) { delete result; }

}  // extern "C"
