// Thin C-ABI driver over the compiled reference CPU core.
//
// TEST INFRASTRUCTURE ONLY.  oracle/Makefile compiles this file together with
// the reference's own sources where they lie (csrc/core/{geometry,
// neighbors_cpu,thread_pool}.cpp under the reference checkout) into
// oracle/_ref/libtonari_ref.so.  It exposes the same orc_* entry points as
// oracle/nl_oracle.cpp so tests can run the restatement and the real
// reference side by side.  Calls: neighbor_search::neighbor_list_cpu<T>
// (csrc/core/neighbors_cpu.cpp:976-1030) and copy_pair_buffers (:908-973).

#include "neighbors_cpu.h"
#include "errors.h"

#include <cstdint>
#include <cstring>
#include <exception>
#include <span>

namespace {

struct Held {
    neighbor_search::PairBuffers buffers;
    int64_t threads = 1;
};

template <typename T>
neighbor_search::PairBuffers call(const void* positions, int64_t n, const int64_t* bp,
                                  int64_t blen, const void* cells, const uint8_t* pbc,
                                  double cutoff, int half, int self, int algorithm,
                                  int64_t threads) {
    const int64_t nb = blen - 1;
    const auto mode = neighbor_search::pair_mode(half != 0, self != 0);
    const auto algo = algorithm == 1   ? neighbor_search::Algorithm::BruteForce
                      : algorithm == 2 ? neighbor_search::Algorithm::CellList
                                       : neighbor_search::Algorithm::Auto;
    return neighbor_search::neighbor_list_cpu<T>(
        std::span<const T>((const T*)positions, (size_t)(3 * n)),
        std::span<const int64_t>(bp, (size_t)blen),
        std::span<const T>((const T*)cells, (size_t)(9 * (nb > 0 ? nb : 0))),
        std::span<const uint8_t>(pbc, (size_t)(3 * (nb > 0 ? nb : 0))), cutoff, mode, algo,
        threads);
}

void put(char* err, int64_t errlen, const char* msg) {
    if (err && errlen > 0) {
        std::strncpy(err, msg, (size_t)errlen - 1);
        err[errlen - 1] = 0;
    }
}

}  // namespace

extern "C" {

int orc_neighbor_list(int dtype, const void* positions, int64_t n_atoms, const int64_t* batch_ptr,
                      int64_t batch_len, const void* cells, const uint8_t* pbc, double cutoff,
                      int half_list, int include_self, int algorithm, int64_t threads,
                      void** handle, int64_t* n_pairs, char* err, int64_t errlen) {
    *handle = nullptr;
    *n_pairs = 0;
    auto* held = new Held();
    held->threads = threads;
    try {
        if (dtype == 0)
            held->buffers = call<float>(positions, n_atoms, batch_ptr, batch_len, cells, pbc,
                                        cutoff, half_list, include_self, algorithm, threads);
        else
            held->buffers = call<double>(positions, n_atoms, batch_ptr, batch_len, cells, pbc,
                                         cutoff, half_list, include_self, algorithm, threads);
    } catch (const neighbor_search::InputError& e) {
        put(err, errlen, e.what());
        delete held;
        return 1;
    } catch (const neighbor_search::SearchError& e) {
        put(err, errlen, e.what());
        delete held;
        return 2;
    } catch (const std::exception& e) {
        put(err, errlen, e.what());
        delete held;
        return 3;
    }
    *handle = held;
    *n_pairs = (int64_t)held->buffers.pair_count;
    return 0;
}

void orc_copy(void* handle, int64_t* pairs, int32_t* shifts) {
    auto* held = (Held*)handle;
    const size_t m = held->buffers.pair_count;
    neighbor_search::copy_pair_buffers(held->buffers, std::span<int64_t>(pairs, 2 * m),
                                       std::span<int32_t>(shifts, 3 * m), held->threads);
}

void orc_free(void* handle) { delete (Held*)handle; }

}  // extern "C"
