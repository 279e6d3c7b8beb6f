/*
 * welder_solver_capi.h -- tile search entry point, same symbol and signature
 * as the reference's backend/welder/compiler/solver/WelderSolverCAPI.h:19-24
 * (implemented there at WelderSolverCAPI.cpp:104-196).  The caller dlopens
 * the library and dlsym's this name (reference caller:
 * compiler/scheduler/SearchBackendApi.cpp:45-60).
 *
 * Here the search enumerates the tile variants the gfx950 kernel library is
 * built with (tile_k counts input elements of one 128-byte k-tile; the thread
 * tile is one lane's accumulator footprint, rows x columns) and ranks them
 * with a roofline cost model of MI355X: MFMA time per wave of resident
 * tiles, HBM bytes, and the softmax pass (row exchange or rescale).
 *
 * Returns 0 on success, 1 bad arguments, 2 input unreadable / not a
 * Matmul->row-Softmax chain, 3 no candidate fits, 4 output I/O error.
 * On success writes best_summary_json_path (keys problem{m,n,k},
 * arch{smemBytes,numSM,warpSize,elementBytes}, best{tileM,tileN,tileK,
 * threadTileM,threadTileN,score,estimatedLatency,profiledMs,bytesCut}), the
 * sorted 13-column candidates_tsv_path, and the best tile fields.  The error
 * buffer is cleared first and receives a NUL-terminated, truncated message.
 * Not thread-safe with respect to concurrent calls writing the same paths.
 */
#ifndef WTC_WELDER_SOLVER_CAPI_H
#define WTC_WELDER_SOLVER_CAPI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int welder_solver_solve_typical_chain(
    const char *input_mlir_path, const char *best_summary_json_path,
    const char *candidates_tsv_path, int64_t max_connect_level, int verbose,
    int64_t *out_tile_m, int64_t *out_tile_n, int64_t *out_tile_k,
    int64_t *out_thread_tile_m, int64_t *out_thread_tile_n,
    char *error_buffer, size_t error_buffer_size);

#ifdef __cplusplus
}
#endif

#endif /* WTC_WELDER_SOLVER_CAPI_H */
