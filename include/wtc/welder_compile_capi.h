/*
 * welder_compile_capi.h -- compile entry point, same symbol and signature as
 * the reference's backend/welder/compiler/driver/WelderCompileCAPI.h:19-25
 * (implemented there at WelderCompileCAPI.cpp:20-71).  The reference caller
 * dlopens the library once and dlsym's this name
 * (compiler/transform/CompileApiSession.cpp:24-72).
 *
 * Here "compiling" selects and plans the hand-written gfx950 kernel for the
 * chain (no code generation happens at run time): the chain is recognised
 * from the MLIR text, the tile parameters are checked against the kernel
 * variants the library is built with, and out_dir receives, under the names
 * the reference's header lists (WelderCompileCAPI.h:12-16) and its callers
 * and scripts read:
 *   03.after_postbufferize.mlir     the decomposed chain the kernel implements
 *   04.after_workgroup_launch.mlir  one gpu.launch per HIP kernel: grid,
 *                                   block, LDS as the workgroup(...) attribution
 *   04c.after_linalg_to_loops.mlir  the loop structure of the path's kernels
 *                                   (scf loops with this problem's bounds)
 *   05.out.nvvm.runnable.mlir       the runnable module: one gpu.launch_func
 *                                   per kernel of the gfx950 code object, with
 *                                   the entry point and its arguments as
 *                                   attributes (no NVVM is involved)
 * and this build's own:
 *   03.chain.canonical.mlir   the same chain as 03.after_postbufferize.mlir
 *   04.kernel.plan.json       kernel variant, path, grid / block / LDS
 *   05.out.hip.launch.json    the runnable artefact: library, C entry point
 *                             (wtc_matmul_softmax_tiles) and its arguments
 *   05.out.gfx950.hsaco       the gfx950 device code object of the chain
 *                             kernels (plus 05.out.rows.gfx950.hsaco for the
 *                             unfused path's row kernels)
 *   kernel_report.txt         key=value artifact report (kernel count, MFMA /
 *                             LDS-DMA / scratch instruction counts, spills)
 *                             and one line per kernel (registers, LDS)
 * workgroup_pass_plugin_path and welder_compiler_bin_path are accepted and
 * ignored (no MLIR pass plugin or external compiler exists in this build).
 * fused != 0 selects the fused kernel (exchange or split path), fused == 0
 * the unfused five-kernel lowering.
 *
 * Returns 0 on success, 1 for empty paths or non-positive tiles, 2 for any
 * failure of the compile session (unreadable input, not a Matmul->row-Softmax
 * chain, tile parameters no kernel variant implements, output I/O).  The
 * error buffer is cleared first and receives a NUL-terminated, truncated
 * message (driver/WelderCompileCAPI.cpp:10-16).  Calls are reentrant: the
 * function keeps no state between calls.
 */
#ifndef WTC_WELDER_COMPILE_CAPI_H
#define WTC_WELDER_COMPILE_CAPI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int welder_compile_typical_chain_to_nvvm(
    const char *input_mlir_path, const char *out_dir,
    const char *workgroup_pass_plugin_path,
    const char *welder_compiler_bin_path, int64_t tile_m, int64_t tile_n,
    int64_t tile_k, int64_t thread_tile_m, int64_t thread_tile_n,
    int64_t max_connect_level, int fused, int verbose, char *error_buffer,
    size_t error_buffer_size);

/* The same entry point under a name that says what it produces. */
int welder_compile_typical_chain_to_hip(
    const char *input_mlir_path, const char *out_dir,
    const char *workgroup_pass_plugin_path,
    const char *welder_compiler_bin_path, int64_t tile_m, int64_t tile_n,
    int64_t tile_k, int64_t thread_tile_m, int64_t thread_tile_n,
    int64_t max_connect_level, int fused, int verbose, char *error_buffer,
    size_t error_buffer_size);

#ifdef __cplusplus
}
#endif

#endif /* WTC_WELDER_COMPILE_CAPI_H */
