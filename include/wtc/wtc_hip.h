/*
 * wtc_hip.h -- launcher C-ABI of the MI355X (gfx950) fused Matmul->row-Softmax
 * kernels:  out[b] = softmax_row(logit_scale * scale_a * scale_b * (A[b] . B[b])).
 *
 * Replaces the reference's launch boundary, which is the welder-profiler
 * runtime: it text-parses `gpu.launch_func` lines of the NVVM artifact
 * (backend/welder/compiler/solver/WelderProfilerParsing.h:211-282), binds
 * memref descriptors (WelderProfilerRuntime.h:1-102), and launches with
 * cuLaunchKernel (backend/welder/compiler/solver/WelderProfiler.cpp:752-792).
 * A HIP code object has no such text form, so the launch is a C call taking
 * device pointers.  All buffers are owned by the caller; the library owns
 * only the default workspaces (one per stream that passed a NULL
 * `workspace`; they grow when a larger problem needs it, keeping the smaller
 * buffer too, since a captured graph may hold its address, and are freed by
 * wtc_release_stream or at process end) and one small pinned host array per
 * device (the timeout mailbox: one word per stream).
 *
 * Layouts are dense row-major: A [batch][m][k], B [batch][k][n],
 * out [batch][m][n] (the reference's strides [K,1] / [N,1] / [N,1],
 * bench/run_ab.sh:30-33).  Pointers must be 16-byte aligned; k*elem_bytes
 * must be a multiple of 16 and n a multiple of 8.  m, n, batch may be 0
 * (nothing to do); k may be 0 (every row is uniform 1/n).
 *
 * Thread safety: calls may come from any host thread.  One lock per process
 * covers the library's shared state (plans, default workspaces, the timeout
 * mailbox) and is released before the ROWS, SPLIT and UNFUSED launches, so
 * such calls from several threads enqueue in parallel; EXCHANGE-path calls
 * hold it through their launch (see below).  Calls that share a
 * caller workspace must not overlap on the GPU (the default workspaces are
 * per stream, so NULL-workspace calls on different streams never share one).
 * An EXCHANGE-path call needs all of its tiles resident at once: the library
 * orders the exchange calls it makes on different streams of one device (an
 * event recorded after each, waited for by the next on another stream;
 * not for streams being captured into a graph).  If other work -- another
 * process, or a replayed graph -- holds the CUs its tiles wait for, the wait
 * ends after a bounded time and the call's output is wrong: that is reported
 * as WTC_ERR_TIMEOUT to the same stream, by its next call of any entry point
 * made after the kernel finished (which then does nothing else) or by
 * wtc_check_status of that stream; calls on other streams are not affected
 * (see also wtc_read_error_flags).  A graph's call reports to the stream it
 * was captured on.  The wait limit defaults to 200 times the cost model's
 * estimate of the call, between 5 ms and 2 s (wtc_set_exchange_wait_limit).
 */
#ifndef WTC_HIP_H
#define WTC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define WTC_OK 0
#define WTC_ERR_ARG 1          /* bad pointer, size, dtype or alignment */
#define WTC_ERR_WORKSPACE 2    /* caller workspace too small */
#define WTC_ERR_HIP 3          /* a HIP runtime call failed */
#define WTC_ERR_UNSUPPORTED 4  /* shape / path combination not available */
#define WTC_ERR_TIMEOUT 5      /* an earlier exchange-path call on this stream timed out
                                  waiting for its tiles; its output is wrong (reported
                                  once; the call that reports it does nothing else) */

/* Element types. */
#define WTC_DTYPE_F32 0
#define WTC_DTYPE_F16 1
#define WTC_DTYPE_BF16 2
#define WTC_DTYPE_FP8_E4M3 3 /* OCP e4m3 ("fn"), inputs only */

/* Execution paths. */
#define WTC_PATH_AUTO 0      /* the fused path and kernel variant that the library's
                                cost model (calibrated on MI355X) ranks fastest for
                                the problem: EXCHANGE, SPLIT or ROWS */
#define WTC_PATH_EXCHANGE 1  /* one kernel, row statistics exchanged between tiles */
#define WTC_PATH_SPLIT 2     /* two kernels: tile pass + row rescale (online two-pass) */
#define WTC_PATH_UNFUSED 3   /* five kernels: matmul, max, exp, sum, divide */
#define WTC_PATH_ROWS 4      /* one kernel, one workgroup per 128 rows over all of n:
                                row statistics in a first pass, outputs in a second
                                (16-bit inputs, k <= 128) */

/* The fused chain.  in_dtype is one of F32/F16/BF16/FP8_E4M3; out_dtype one of
 * F32/F16/BF16.  scale_a / scale_b are the per-tensor dequantisation scales
 * of fp8 inputs (pass 1 otherwise); logit_scale multiplies A.B before the
 * softmax (1/sqrt(d) for attention scores).  `stream` is a hipStream_t
 * (NULL = the null stream).  Asynchronous: returns after enqueueing. */
int wtc_matmul_softmax(const void *a, const void *b, void *out, int64_t batch,
                       int64_t m, int64_t n, int64_t k, int in_dtype,
                       int out_dtype, float logit_scale, float scale_a,
                       float scale_b, int path, void *workspace,
                       size_t workspace_bytes, void *stream);

/* Tile parameters of one kernel variant, in the fields and units of the
 * reference's best.json (compiler/scheduler/Search.cpp:62-86): a tile_m x
 * tile_n output tile per workgroup, tile_k elements of K per pipeline stage,
 * thread_tile_m x thread_tile_n accumulators per lane. */
typedef struct wtc_tiles {
  int64_t tile_m, tile_n, tile_k, thread_tile_m, thread_tile_n;
} wtc_tiles;

/* wtc_matmul_softmax on exactly the kernel variant `tiles` (NULL: the
 * variant the cost model ranks first, as wtc_matmul_softmax does).  Replaces
 * the reference's launch of the kernel it generated for best.json's tiles
 * (welder_compile_typical_chain_to_nvvm's tile arguments,
 * backend/welder/compiler/driver/WelderCompileCAPI.h:19-25, launched by
 * WelderProfiler.cpp:752-792): here the variant is chosen among the built
 * ones at call time.  With path AUTO the variant runs the fused path the
 * cost model ranks first for it.  WTC_ERR_UNSUPPORTED when no variant has
 * these tiles for in_dtype, or when the variant cannot run `path` for this
 * problem (wtc_last_error says why). */
int wtc_matmul_softmax_tiles(const void *a, const void *b, void *out, int64_t batch,
                             int64_t m, int64_t n, int64_t k, int in_dtype,
                             int out_dtype, float logit_scale, float scale_a,
                             float scale_b, const wtc_tiles *tiles, int path,
                             void *workspace, size_t workspace_bytes, void *stream);

/* The kernel variants built for an input type, the candidates the solver
 * ranks (the reference's tile space, WelderSolverSolveEntrypoints.h:157-265).
 * Writes up to `capacity` entries -- tiles, a bit (1 << WTC_PATH_x) per
 * path the variant runs, a static name (any array may be NULL) -- and
 * returns the number of variants, or -1 for an unknown dtype. */
int wtc_list_variants(int in_dtype, wtc_tiles *tiles, unsigned *paths,
                      const char **names, int capacity);

/* Times one variant on one path on the current device: allocates A, B, out
 * and a workspace, fills A and B with finite pseudo-random values (from
 * `seed`), runs `warmup` untimed calls and then `iters` back-to-back calls
 * between two HIP events on a stream of its own, frees everything and
 * writes the mean microseconds per call.  `tiles` NULL = the cost model's
 * choice.  The counterpart of the reference's profile step, which compiles
 * and times top-ranked candidates with welder-profiler
 * (backend/welder/compiler/solver/WelderSolverProfileCompileAndRun.h,
 * WelderProfiler.cpp:752-792).  Synchronous; allocates. */
int wtc_profile_tiles(int64_t batch, int64_t m, int64_t n, int64_t k, int in_dtype,
                      int out_dtype, const wtc_tiles *tiles, int path, int warmup,
                      int iters, uint64_t seed, double *us_per_call);

/* Size of the device scratch array behind wtc_matmul_softmax_noalloc. */
#define WTC_NOALLOC_SCRATCH_BYTES (8u << 20)

/* No counterpart in the reference: an allocation-free variant of
 * wtc_matmul_softmax for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, paths and results as wtc_matmul_softmax,
 * except that the workspace is a fixed array of WTC_NOALLOC_SCRATCH_BYTES
 * that the library holds on each GPU until the process ends (its address is
 * looked up once per device).  It calls no hipMalloc, hipFree or other
 * allocating routine, so it also creates no timeout mailbox or exchange
 * event itself.  Set-up: call wtc_check_status once on the device, outside
 * graph capture, before the first call of this entry point there: that call
 * makes the device's set-up (kernel attributes, the array's address, the
 * mailbox, the exchange event), after which calls of this entry point do
 * none and may be captured.  Without it the first call on a device does the
 * set-up other than the mailbox and event (it must then not be captured),
 * and a timed-out exchange wait is reported only through the array's
 * diagnostic words (wtc_read_error_flags(NULL, ...)).  Problems whose
 * workspace (wtc_matmul_softmax_workspace_size) exceeds the array get
 * WTC_ERR_WORKSPACE.  Every call on a GPU shares that GPU's array: calls
 * that overlap on one GPU (other streams, other host threads) race and must
 * not be made. */
int wtc_matmul_softmax_noalloc(const void *a, const void *b, void *out,
                               int64_t batch, int64_t m, int64_t n, int64_t k,
                               int in_dtype, int out_dtype, float logit_scale,
                               float scale_a, float scale_b, int path,
                               void *stream);

/* Bytes of workspace wtc_matmul_softmax needs for this problem and path
 * (AUTO, EXCHANGE and SPLIT need the same amount).  Negative on bad args. */
int64_t wtc_matmul_softmax_workspace_size(int64_t batch, int64_t m, int64_t n,
                                          int64_t k, int in_dtype,
                                          int out_dtype, int path);

/* Zero a caller workspace with a kernel on `stream` (required once, before
 * its first use; safe inside graph capture). */
int wtc_workspace_init(void *workspace, size_t workspace_bytes, void *stream);

/* The launch plan for a device with `cu_count` compute units of which each
 * holds `wg_per_cu` chain workgroups: grid size, chosen path and workspace
 * bytes.  Pure host arithmetic (no GPU needed). */
int wtc_plan(int64_t batch, int64_t m, int64_t n, int64_t k, int in_dtype,
             int out_dtype, int path, int cu_count, int wg_per_cu,
             int64_t *grid, int *chosen_path, int64_t *workspace_bytes);

/* wtc_plan for one variant (`tiles`; NULL = every variant): the variant and
 * path the cost model ranks first (for path AUTO, among the fused paths),
 * its grid, its workspace bytes and the model's estimate of microseconds
 * per back-to-back call.  Any output pointer may be NULL.  Pure host
 * arithmetic (no GPU needed). */
int wtc_plan_tiles(int64_t batch, int64_t m, int64_t n, int64_t k, int in_dtype,
                   int out_dtype, int path, const wtc_tiles *tiles, int cu_count,
                   int wg_per_cu, wtc_tiles *chosen_tiles, int *chosen_path,
                   int64_t *grid, int64_t *workspace_bytes, double *estimated_us);

/* Reads (and with clear != 0, resets) the three diagnostic words of a
 * workspace (NULL = all default workspaces of the current device and the
 * scratch array of wtc_matmul_softmax_noalloc, or-ed / max-ed / summed) into
 * flags[0..2]: flags[0] bit 0 = an exchange-path wait
 * timed out, flags[1] = longest exchange-path wait in 100 MHz ticks,
 * flags[2] = number of timed-out waits.  Synchronises the device. */
int wtc_read_error_flags(void *workspace, uint32_t *flags, int clear);

/* Synchronises `stream` (a hipStream_t, NULL = the null stream) and returns
 * WTC_ERR_TIMEOUT if an exchange-path wait of a call on that stream timed out
 * since the last report, else WTC_OK.  Also makes the current device's
 * set-up (see wtc_matmul_softmax_noalloc). */
int wtc_check_status(void *stream);

/* Limit of every exchange-path wait, in ticks of the 100 MHz real-time clock
 * (0 = automatic: 200 times the cost model's estimate of the call, at least
 * 5 ms, at most 2 s).  Applies to calls made after it. */
int wtc_set_exchange_wait_limit(uint64_t ticks);

/* Synchronises `stream`, frees its default workspace (and the smaller ones it
 * replaced) and gives back its timeout-mailbox word; call it before
 * destroying a stream that made NULL-workspace calls.  Graphs captured on the
 * stream with its default workspace must not be replayed afterwards.  Returns
 * WTC_ERR_TIMEOUT if a timeout of the stream was still unreported (the
 * resources are freed all the same).  No counterpart in the reference, whose
 * launches take caller buffers only. */
int wtc_release_stream(void *stream);

/* Message of the last failing call on this thread ("" if none). */
const char *wtc_last_error(void);

/* Library version string. */
const char *wtc_version(void);

#ifdef __cplusplus
}
#endif

#endif /* WTC_HIP_H */
