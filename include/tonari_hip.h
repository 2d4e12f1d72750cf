/*
 * tonari_hip.h - C ABI of the MI355X (gfx950) neighbor-list library
 * (libtonari_hip.so).
 *
 * This ABI replaces the reference's pybind11 CUDA provider entry point
 *   _torch_cuda.neighbor_list(positions, batch_ptr, cell, pbc, cutoff,
 *                             half_list, include_self, algorithm, sorted)
 *       -> [P (E,2) int64, S (E,3) int32]
 * (songfeitong/tonari csrc/torch/bindings_cuda.cpp:59-228, registered at
 * :233-238; internal launchers declared in csrc/torch/neighbors_cuda.h:9-38,
 * called from src/tonari/_torch_frontend.py:138-145).
 *
 * The single pybind call is split in two so that the caller owns every device
 * allocation (the library never calls hipMalloc):
 *   1. tnr_workspace_size()  - bytes of device scratch for this request
 *   2. tnr_count()           - geometry, binning and the counting pass; the only
 *                              host synchronisation: returns E
 *   3. tnr_emit()            - writes the requested quantities (i, j, P, S, d,
 *                              D) into caller buffers sized for E pairs
 * The frontend calls them in this order with the same request, workspace and
 * stream.  Quantity assembly that the reference does in Torch
 * (src/tonari/_torch_frontend.py:78-105) is fused into tnr_emit.
 *
 * All pointers are device pointers unless stated otherwise.  Every launch and
 * copy goes on `stream`, on the current HIP device.  The library keeps no
 * mutable global state: concurrent calls with distinct workspaces are safe.
 *
 * Return codes: TNR_OK, TNR_INPUT_ERROR (reference InputError -> Python
 * ValueError), TNR_SEARCH_ERROR (reference SearchError / TORCH_CHECK ->
 * Python RuntimeError), TNR_DEVICE_ERROR (HIP failure -> RuntimeError).  A
 * NUL-terminated message is written to `err` (capacity `err_len`).
 */
#ifndef TONARI_HIP_H
#define TONARI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TNR_ABI_VERSION 7

#define TNR_OK 0
#define TNR_INPUT_ERROR 1
#define TNR_SEARCH_ERROR 2
#define TNR_DEVICE_ERROR 3
#define TNR_RETRY 4 /* tnr_count_finish: a plan hint did not hold; count again without it */

/* Slots of host_result: status flags, E, total periodic images, plan mask,
 * total cell-list bins, hit-mask words per atom the count wanted (the
 * longest row any source or brute-force structure would store; 0 when none
 * stores masks), one internal ticket, brute-force work units. */
#define TNR_HOST_RESULT_SLOTS 8

#define TNR_FLOAT32 0
#define TNR_FLOAT64 1

/* Algorithm enum of the reference (csrc/core/algorithm.h:10-29). */
#define TNR_AUTO 0
#define TNR_BRUTE_FORCE 1
#define TNR_CELL_LIST 2

/* One neighbor-list request: the arguments of bindings_cuda.cpp:59-68. */
typedef struct tnr_request {
    int32_t dtype;            /* TNR_FLOAT32 or TNR_FLOAT64 */
    int32_t algorithm;        /* TNR_AUTO / TNR_BRUTE_FORCE / TNR_CELL_LIST */
    int64_t n_atoms;          /* N_total */
    int64_t n_structures;     /* B (batch_ptr has B + 1 entries) */
    const void* positions;    /* T[N][3], contiguous */
    const int64_t* batch_ptr; /* int64[B + 1] */
    const void* cell;         /* T[B][3][3], rows are cell vectors */
    const uint8_t* pbc;       /* uint8 (bool) [B][3] */
    double cutoff;            /* strict, finite, positive */
    int32_t half_list;        /* 0 / 1 */
    int32_t include_self;     /* 0 / 1 */
    int32_t sorted;           /* 0 / 1: sources in index order (see tnr_emit) */
    int32_t stencil_reach;    /* cell-list bins per cutoff along each axis, 1-4; 0 = chosen per structure */
    int32_t mask_words;       /* 64-bit hit-mask words of workspace per atom, 0-64; 0 = 64.  A
                                 cell-list bin whose stencil has more chunks of 64 candidates,
                                 a molecule of more than 64 x mask_words atoms, and k0 slices
                                 beyond mask_words take paths that store no masks: the results
                                 are the same, only slower.  host_result[5] of a count gives the
                                 value that avoids them for the same inputs.  Count and emit
                                 of one workspace must use the same value. */
} tnr_request;

/* Output buffers for tnr_emit; any pointer may be NULL (not requested). */
typedef struct tnr_outputs {
    int64_t n_pairs;    /* E returned by tnr_count, or the rows the outputs hold (see plan) */
    int64_t plan;       /* host_result[3] of tnr_count (kernel families in use), or -1: the
                           emit reads plan and bins from the count's status words on the
                           device, for callers that do not wait for the count (graph
                           capture); pairs beyond n_pairs rows are then dropped and flagged */
    int64_t n_tasks;    /* host_result[4] of tnr_count (cell-list bins of the batch) */
    int64_t* pairs;     /* P: int64[E][2] (source, target) */
    int32_t* shifts;    /* S: int32[E][3] */
    void* distances;    /* d: T[E] */
    void* vectors;      /* D: T[E][3] = pos[j] - pos[i] + S @ cell[b] */
    int64_t* sources;   /* i: int64[E] */
    int64_t* targets;   /* j: int64[E] */
    int64_t* edge_index; /* edge-first layout int64[2][E]: sources, then targets from row E on,
                            with E taken from the count on the device (so a buffer of
                            2 x n_pairs rows serves a launch made before E is read); when
                            given, `sources` and `targets` are ignored.  No counterpart in the
                            reference, whose design leaves (2, E) layouts to graph adapters
                            (docs/design.md:61,127). */
} tnr_outputs;

/* ABI version compiled into the library (TNR_ABI_VERSION). */
int tnr_abi_version(void);

/* Offload target the library was compiled for ("gfx950"). */
const char* tnr_device_arch(void);

/* HIP version of the headers the library was compiled with, as
 * major * 100 + minor.  The library calls only the C API of the HIP runtime
 * (libamdhip64.so.<major>) loaded in the process, so the loader requires the
 * same major version as the runtime torch loaded (replaces the CUDA runtime
 * check of src/tonari/_extensions.py:42-48). */
int tnr_hip_version(void);

/* Device scratch bytes for `req`; depends only on dtype, N, B and mask_words
 * (0 when mask_words is out of range). */
size_t tnr_workspace_size(const tnr_request* req);

/*
 * Validates the request on the device, builds per-structure geometry and the
 * cell-list bins, counts pairs per source and scans the counts.  Copies the
 * status words into `host_result` (pinned host memory of
 * TNR_HOST_RESULT_SLOTS int64) and synchronises
 * `stream`; *n_pairs receives E.  Equivalent to tnr_count_async followed by
 * hipStreamSynchronize(stream) and tnr_count_finish.
 */
int tnr_count(const tnr_request* req, void* workspace, size_t workspace_bytes,
              int64_t* host_result, void* stream, int64_t* n_pairs, char* err,
              size_t err_len);

/* The counting pass without the synchronisation: everything is enqueued on
 * `stream`; `host_result` is valid once the stream has reached this point. */
int tnr_count_async(const tnr_request* req, void* workspace, size_t workspace_bytes,
                    int64_t* host_result, void* stream, char* err, size_t err_len);

/*
 * No counterpart in the reference (its binding plans on the host and reads
 * the plan back, bindings_cuda.cpp:96-98,161-185).  tnr_count_async with a
 * plan hint: host_result[3] (the plan mask: bit 0 brute-force structures,
 * bit 1 cell-list structures, bit 2 every brute-force structure a
 * molecule, i.e. without periodic axes and of at most 2,048 atoms and
 * 64 x mask_words atoms, bit 3
 * one fully periodic structure whose bin grid follows from its cell and
 * cutoff) of an earlier count of a request of the same shape, or -1 for
 * none.  Hint 1 (brute force only) with algorithm TNR_AUTO: the cell-list
 * kernels are not launched.  Hint 5 (molecules only) with TNR_AUTO or
 * TNR_BRUTE_FORCE: one kernel plans the whole batch in place of the set-up,
 * atom and planning kernels.  Hint 10 (one periodic cell-list structure)
 * with TNR_AUTO or TNR_CELL_LIST: the bin grid is chosen before the atoms
 * are reduced and the prologue takes two launches instead of four, the
 * second ranking, scanning and placing the atoms behind a grid barrier
 * whose waits are bounded by the environment variable TNR_PLACE_WAIT_US
 * (microseconds of the device clock, default 20,000; a wait that expires
 * makes the hint fail).  The device checks the hint: if a structure does
 * not fit it,
 * nothing of this count is valid and tnr_count_finish returns TNR_RETRY;
 * the caller counts again without the hint.  Other hints launch the full
 * count.
 */
int tnr_count_async_hinted(const tnr_request* req, void* workspace, size_t workspace_bytes,
                           int64_t* host_result, void* stream, int64_t plan_hint, char* err,
                           size_t err_len);

/* Decodes `host_result` written by a completed tnr_count_async: maps the
 * status flags to the reference's error types and messages, sets *n_pairs. */
int tnr_count_finish(const int64_t* host_result, int64_t* n_pairs, char* err, size_t err_len);

/* Writes every non-NULL output of `out` for the request last counted in
 * `workspace`.  The pairs of one source are contiguous; with `sorted` the
 * sources come in increasing index order, otherwise in an order of the
 * library's choosing (the cell-list bin order when every structure of the
 * request is searched with a cell list, index order otherwise). */
int tnr_emit(const tnr_request* req, void* workspace, size_t workspace_bytes,
             const tnr_outputs* out, void* stream, char* err, size_t err_len);

/*
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): tnr_count_async followed by tnr_emit, on a static
 * scratch array of 64 MiB per GPU inside the library instead of a caller
 * workspace.  It allocates nothing and does not wait on the host.  The
 * caller passes the inputs (req) and outputs of a chosen capacity
 * (out->n_pairs rows; out->plan and out->n_tasks are ignored: the emit reads
 * them from the count on the device).  Once `stream` has completed,
 * tnr_count_finish(host_result) reports errors and E; when E exceeds the
 * capacity, the rows beyond it were not written and the call must be
 * repeated with larger outputs.  Requests whose tnr_workspace_size exceeds
 * 64 MiB (one structure of more than about 105,000 float32 or 98,000
 * float64 atoms) are rejected with TNR_INPUT_ERROR before any device work.
 * Every call on one GPU uses that GPU's one array: calls that overlap on a
 * GPU (two streams, two threads) race and must be serialised by the caller.
 */
int tnr_search_static(const tnr_request* req, const tnr_outputs* out, int64_t* host_result,
                      void* stream, char* err, size_t err_len);

/*
 * Verlet-skin lists.  No counterpart in the reference, which lists a Verlet
 * skin as unsupported (docs/design.md:125-127); for molecular-dynamics
 * loops that search every step.  The caller searches once at
 * build_cutoff = cutoff + skin (tnr_count / tnr_emit, P and S) and stores
 * that list with tnr_skin_store, which packs it into a workspace (8 bytes per
 * pair) together with copies of the request's positions, cell, pbc and
 * batch_ptr.  At a later step, tnr_skin_filter_async re-decides every stored
 * pair with the reference's public predicate at the current positions and
 * writes the kept pairs in stored order, in one pass; tnr_skin_finish says
 * whether the result equals a fresh search at req->cutoff (every atom moved
 * less than about skin / 2, less a rounding margin, and cell, pbc and
 * batch_ptr unchanged).  If not, the caller rebuilds.
 */
typedef struct tnr_skin_list {
    int64_t n_pairs;      /* stored pairs */
    int64_t n_atoms;      /* N of the stored list's request */
    int64_t n_structures; /* B */
    int32_t dtype;
    int32_t pair_mode;    /* the stored list's half_list << 1 | include_self */
    double build_cutoff;  /* cutoff the stored list was searched with */
} tnr_skin_list;

/* Device bytes of a skin workspace for `req` (dtype, N, B) and n_pairs
 * stored pairs. */
size_t tnr_skin_workspace_size(const tnr_request* req, int64_t n_pairs);

/* Stores the list (pairs, shifts: the n_pairs rows that tnr_emit wrote for
 * `req` at build_cutoff, 16-byte aligned pairs) and the request's positions,
 * cell, pbc and batch_ptr in `workspace`, on `stream`; fills `list`.  Shifts
 * beyond [-512, 511] or pairs whose sources are not contiguous make the list
 * unfilterable: every later tnr_skin_finish then asks for a rebuild. */
int tnr_skin_store(const tnr_request* req, double build_cutoff, const int64_t* pairs,
                   const int32_t* shifts, int64_t n_pairs, void* workspace,
                   size_t workspace_bytes, tnr_skin_list* list, void* stream, char* err,
                   size_t err_len);

/* Filters the stored list at req's positions, cell and cutoff (dtype, N, B,
 * half_list and include_self as stored; any other request is refused with
 * TNR_INPUT_ERROR) into `out` (P, S, d, D, i, j; no edge_index), rows at and
 * beyond out->n_pairs being dropped: out->n_pairs = list->n_pairs always
 * suffices.  The status words reach `host_result` (pinned,
 * TNR_HOST_RESULT_SLOTS int64) when the stream has reached this point. */
int tnr_skin_filter_async(const tnr_request* req, const tnr_skin_list* list, void* workspace,
                          size_t workspace_bytes, const tnr_outputs* out, int64_t* host_result,
                          void* stream, char* err, size_t err_len);

/* Decodes a completed tnr_skin_filter_async: *rebuild = 1 when the filtered
 * list may differ from a fresh search (the caller rebuilds); otherwise
 * *rebuild = 0 and *n_pairs receives E (when E exceeds the out->n_pairs of
 * the filter, rows beyond it were dropped: filter again into larger
 * outputs). */
int tnr_skin_finish(const tnr_request* req, const tnr_skin_list* list, const int64_t* host_result,
                    int64_t* n_pairs, int32_t* rebuild, char* err, size_t err_len);

/*
 * Backward of the d/D outputs of tnr_emit: adds the gradients of positions
 * (T[N][3]) and cell (T[B][3][3]) into grad_positions and grad_cell (set to
 * zero by the caller) from grad_vectors (dL/dD, T[E][3]) and grad_distances
 * (dL/dd, T[E]); either may be NULL.  pairs, shifts, vectors and distances
 * are the E rows tnr_emit wrote (vectors and distances are needed only with
 * grad_distances).  Replaces the autograd of the reference's Torch
 * expression for D and d (src/tonari/_torch_frontend.py:92-104): with
 * g = dL/dD + dL/dd * D / d (0 where d = 0), pos[j] += g, pos[i] -= g and
 * cell[b][a][c] += S[a] g[c].  Float atomics: the summation order varies.
 */
int tnr_geometry_backward(int32_t dtype, int64_t n_pairs, int64_t n_atoms, int64_t n_structures,
                          const int64_t* batch_ptr, const int64_t* pairs, const int32_t* shifts,
                          const void* vectors, const void* distances, const void* grad_vectors,
                          const void* grad_distances, void* grad_positions, void* grad_cell,
                          void* stream, char* err, size_t err_len);

#ifdef __cplusplus
}
#endif

#endif /* TONARI_HIP_H */
