/*
 * tonari_cpu.h - C ABI of the host (CPU) neighbor-list provider
 * (libtonari_cpu.so), the CPU counterpart of include/tonari_hip.h.
 *
 * This ABI replaces the reference's pybind11 CPU providers
 *   _torch_cpu.neighbor_list(positions, batch_ptr, cell, pbc, cutoff,
 *                            half_list, include_self, algorithm, num_threads)
 *       -> [P (E,2) int64, S (E,3) int32]
 *   _numpy_cpu.neighbor_list(...)   (the same arguments and result)
 * (songfeitong/tonari csrc/torch/bindings_cpu.cpp:73-122 and
 * csrc/numpy/bindings.cpp, called from src/tonari/_torch_frontend.py:
 * 147-156 and src/tonari/_numpy_frontend.py:119-140; the search itself is
 * csrc/core/neighbors_cpu.cpp, its worker pool csrc/core/thread_pool.cpp).
 *
 * All pointers are host pointers.  The search runs on `threads` threads
 * (the calling thread included).  Pairs come grouped by structure, and by
 * source in increasing index order inside a structure, as the reference's
 * CPU path returns them; the order of targets within a source is
 * unspecified.
 *
 * Return codes and messages are those of tonari_hip.h: TNR_OK,
 * TNR_INPUT_ERROR (ValueError), TNR_SEARCH_ERROR (RuntimeError), with the
 * reference's message copied into `err`.
 */
#ifndef TONARI_CPU_H
#define TONARI_CPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TNR_CPU_ABI_VERSION 1

/* Opaque search result: the pairs of one call. */
typedef struct tnr_cpu_result tnr_cpu_result;

int tnr_cpu_abi_version(void);

/*
 * Searches on the CPU.  dtype is TNR_FLOAT32 (0) or TNR_FLOAT64 (1);
 * positions T[n_atoms][3], batch_ptr int64[n_structures + 1], cell
 * T[n_structures][3][3] (rows are cell vectors), pbc uint8[n_structures][3];
 * algorithm 0 auto, 1 brute_force, 2 cell_list.  On success *result owns the
 * pairs (free it with tnr_cpu_free) and *n_pairs is E.
 */
int tnr_cpu_search(int32_t dtype, const void* positions, int64_t n_atoms,
                   const int64_t* batch_ptr, int64_t n_structures, const void* cell,
                   const uint8_t* pbc, double cutoff, int32_t half_list, int32_t include_self,
                   int32_t algorithm, int64_t threads, tnr_cpu_result** result,
                   int64_t* n_pairs, char* err, size_t err_len);

/* Copies the pairs into P (int64[E][2]) and S (int32[E][3]). */
void tnr_cpu_copy(const tnr_cpu_result* result, int64_t* pairs, int32_t* shifts,
                  int64_t threads);

void tnr_cpu_free(tnr_cpu_result* result);

#ifdef __cplusplus
}
#endif

#endif /* TONARI_CPU_H */
