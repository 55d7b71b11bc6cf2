/*
 * pjrtx_hip.h — the thin C ABI between the pjrtx runtime and HIP.
 *
 * The reference's Zig runtime reaches its device backend through a private
 * C ABI over MLX (`pjrtx_mlx_metal_*`, reference:
 * src/backend/mlx_metal/api.h:198-477) and a generated-kernel runner
 * (`pjrtx_metalcpp_*`, reference: src/backend/mlx_metal/metalcpp_api.cc:
 * 1165-1335). This header is the HIP replacement: plain pointers, sizes and
 * integer status codes, no C++ or torch types, so that a Zig, Python
 * (ctypes) or C caller can bind it unchanged. Every function returns 0 on
 * success; on failure it returns a PJRT_Error_Code value and the message is
 * available from pjrtx_hip_last_error() on the same thread.
 *
 * The PJRT entry point (GetPjrtApi) is declared in pjrt_c_api.h; the plugin
 * itself is built on the functions below.
 */
#ifndef PJRTX_AMD_PJRTX_HIP_H_
#define PJRTX_AMD_PJRTX_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PJRTX_HIP_API __attribute__((visibility("default")))

/* Thread-local message of the last failing call. */
PJRTX_HIP_API const char* pjrtx_hip_last_error(void);

/* ---------------------------------------------------------------- devices */

/* Number of visible HIP devices (0 when none). Replaces
 * pjrtx_mlx_metal_copy_devices (api.h:198, api.cc:1753). */
PJRTX_HIP_API int pjrtx_hip_device_count(int* count);

/* Device memory from the per-device caching allocator. Replaces the buffer
 * creation / destroy entries of api.h (pjrtx_mlx_metal_buffer_from_host_typed
 * api.cc:1781-1852, pjrtx_mlx_metal_buffer_destroy). */
PJRTX_HIP_API int pjrtx_hip_malloc(int device, size_t bytes, void** ptr);
PJRTX_HIP_API int pjrtx_hip_free(int device, void* ptr);

/* Stream-ordered copies on this ABI's stream of the device; each returns
 * after the copy completed. pjrtx_hip_synchronize waits for all work queued
 * on the device, on every stream (PJRT clients queue on streams of their
 * own). Replace buffer_from_host_typed (api.cc:1781-1852) and
 * pjrtx_mlx_metal_buffer_copy_to_host (api.cc:5685-5731). */
PJRTX_HIP_API int pjrtx_hip_copy_h2d(int device, void* dst, const void* src, size_t bytes);
PJRTX_HIP_API int pjrtx_hip_copy_d2h(int device, void* dst, const void* src, size_t bytes);
PJRTX_HIP_API int pjrtx_hip_synchronize(int device);

/* Calibration: the dense bf16 matrix-core throughput the device sustains,
 * in TFLOP/s (two waves per SIMD on every CU issuing independent
 * v_mfma_f32_16x16x32_bf16 for shape 0, v_mfma_f32_32x32x16_bf16 for
 * shape 1; best of five timed runs). Lets MFMA-bound roofline fractions be
 * quoted against a measured peak beside the published one. No counterpart
 * in the reference (its benchmarks quote Apple GPU figures). */
PJRTX_HIP_API int pjrtx_mfma_peak_tflops(int device, int shape, double* tflops);

/* --------------------------------------------------- compiler (host only) */

/* Compile-cache counters of this process: compiles that reused a cached
 * parsed and planned program, compiles that built one, entries held (any
 * pointer may be NULL). Replaces the reference's executable-cache stats
 * (src/runtime/executable_cache.zig:9-25, hits / misses / resident_entries). */
PJRTX_HIP_API int pjrtx_compile_cache_stats(int64_t* hits, int64_t* misses, int64_t* entries);

/* Host bytes the compile cache holds (program texts and constant literals)
 * and entries it evicted; the cap is PJRTX_COMPILE_CACHE_BYTES (default
 * 256 MiB) and 32 entries. Replaces the reference's cache byte accounting
 * (src/runtime/executable_cache.zig:9-25, resident_bytes / evictions). */
PJRTX_HIP_API int pjrtx_compile_cache_usage(int64_t* bytes, int64_t* evictions);

/* The compile-cache key of a program text under the current PJRTX_*
 * environment ("pjrtx-" and 32 hex digits). Replaces
 * executable_fingerprint.zig:9-24 (alloc). */
PJRTX_HIP_API int pjrtx_compile_fingerprint(const char* text, size_t len, char* out, size_t cap, size_t* needed);

/* ------------------------------------------- residency (needs a device) */

/* Device residency budget: the cap, in bytes, on the device memory that
 * loaded executables hold (code objects, resident constants, kernel
 * scratch); 0 removes it (the default, or PJRTX_MAX_RESIDENT_BYTES).
 * Loading past the cap first evicts idle executables, largest first, then
 * least recently used; an evicted executable loads again when next run.
 * Replaces Residency.setMaxResidentBytes (executable_cache.zig:118-122,
 * 233-300) and client_residency.zig:58-92. */
PJRTX_HIP_API int pjrtx_set_max_resident_bytes(int device, int64_t bytes);

/* out = {resident bytes, peak resident bytes, resident executables,
 * evictions, evicted bytes, cap} of the device's residency budget.
 * Replaces executable_cache.zig:9-25 (Stats). */
PJRTX_HIP_API int pjrtx_residency_stats(int device, int64_t out[6]);

/* --------------------------------------------------- plans (host only) */

/* Parses a StableHLO text module, runs the fusion planner and code
 * generator, and writes a JSON description of the plan to `out` (at most
 * `cap` bytes; `*needed` gets the full size). Needs no GPU. Replaces the
 * compile-time half of pjrtx_metalcpp_executable_program_create
 * (metalcpp_api.cc:1296) together with the Zig planner
 * (program_build.zig:10-207). */
PJRTX_HIP_API int pjrtx_plan_json(const char* text, size_t len, char* out, size_t cap, size_t* needed);

/* As pjrtx_plan_json, and also compiles the generated fusion kernels with
 * hiprtc for `arch` (e.g. "gfx950"); `code_size` gets the code-object size.
 * Needs no GPU. Replaces the MSL pipeline compile (metalcpp_api.cc:459-540). */
PJRTX_HIP_API int pjrtx_compile_check(const char* text, size_t len, const char* arch, size_t* code_size);

/* Writes the full hiprtc translation unit of the plan's generated kernels
 * (device header + bodies) to `out`, for inspection. Needs no GPU. */
PJRTX_HIP_API int pjrtx_kernel_source(const char* text, size_t len, char* out, size_t cap, size_t* needed);

/* ------------------------------------------------------ executable timing */

struct PJRT_LoadedExecutable;
struct PJRT_Buffer;

/* Replays each launch unit of a compiled executable `iters` times between
 * two hipEvents on the device stream and writes the mean milliseconds per
 * launch to ms[0..steps). A launch unit is one step, except that a split
 * reduction is two units (its main kernel, then its combine kernel). Used by
 * the benchmark's roofline figure. Replaces
 * PJRTX_METALCPP_EXECUTABLE_STEP_PROFILE (metalcpp_api.cc:399-416). */
PJRTX_HIP_API int pjrtx_executable_time_steps(struct PJRT_LoadedExecutable* exe, struct PJRT_Buffer* const* args,
                                size_t num_args, int iters, double* ms, size_t cap, size_t* steps);

/* Executes the executable `iters` times back to back on its device stream,
 * through the same path as PJRT_LoadedExecutable_Execute (argument checks,
 * graph capture and replay, output allocation; nothing donated), dropping
 * each call's outputs, and writes the wall milliseconds from a synchronized
 * start to the synchronized end of the last call to *ms_total. This is the
 * steady-state execute loop without a host language's per-call binding cost.
 * Replaces the reference's steady-execute measurement
 * (src/plugin/jax/jax_llama_like_inference.py:291-296, timing
 * execute_executable_program, metalcpp_api.cc:961-1161). */
PJRTX_HIP_API int pjrtx_executable_run(struct PJRT_LoadedExecutable* exe, struct PJRT_Buffer* const* args,
                                       size_t num_args, int iters, double* ms_total);

/* The same loop through this plugin's PJRT C API table (GetPjrtApi): each
 * iteration is one PJRT_LoadedExecutable_Execute with a completion event,
 * followed by PJRT_Event_Destroy and PJRT_Buffer_Destroy of its outputs, as
 * a C PJRT client does, so the figure includes the PJRT layer's host work
 * per call (argument structs, output buffer and event objects). Writes the
 * wall milliseconds from a synchronized start to the synchronized end of the
 * last call to *ms_total. Replaces the reference's steady-execute
 * measurement (src/plugin/jax/jax_llama_like_inference.py:291-296) at the
 * C-API level. */
PJRTX_HIP_API int pjrtx_executable_run_pjrt(struct PJRT_LoadedExecutable* exe, struct PJRT_Buffer* const* args,
                                            size_t num_args, int iters, double* ms_total);

/* Allocation-free execute. No counterpart in the reference: it is for
 * callers that cannot allocate device memory while they run (tight serving
 * loops, harnesses that forbid hipMalloc). Its launches record no memset
 * and make no host-synchronizing call, but capturing them into a HIP graph
 * is not tested. Runs a compiled,
 * loaded executable (PJRT_Client_Compile loads it on device 0) on
 * caller-owned device memory: args[i] and outputs[i] are device addresses of
 * the i-th parameter / result, dense row-major, of the program's sizes.
 * Every intermediate value, every copy of a parameter the plan writes in
 * place (the caller's inputs are never modified), and every kernel scratch
 * block (split-reduction partials, split-K partials, sort keys, scatter
 * segments) is carved from one fixed device block per GPU of
 * pjrtx_noalloc_scratch_bytes() bytes (64 MiB), held from the first call on
 * that GPU until the process ends. A program whose needs exceed it fails with
 * PJRT_Error_Code_RESOURCE_EXHAUSTED (outputs then unspecified); programs with
 * a while loop fail with UNIMPLEMENTED. The call calls no hipMalloc or
 * hipFree and no allocating library routine; the work is queued on the
 * device's stream and the call returns without waiting
 * (pjrtx_hip_synchronize waits). Every call on one GPU shares that GPU's
 * block (one per process) and finds the previous call's contents in it.
 * Calls on one GPU, from any thread, take the device's execute lock and
 * queue their work on the one device stream, so they run one after another
 * and never overlap on the block; work the caller queues on other streams
 * never touches it.
 * `scratch_used` (may be NULL) gets the bytes of the block the call used. */
PJRTX_HIP_API int pjrtx_executable_execute_noalloc(struct PJRT_LoadedExecutable* exe, int device,
                                                   const void* const* args, size_t num_args,
                                                   void* const* outputs, size_t num_outputs,
                                                   size_t* scratch_used);
PJRTX_HIP_API size_t pjrtx_noalloc_scratch_bytes(void);

/* Names of the executable's launch units, in the order of
 * pjrtx_executable_time_steps, '\n'-separated: the kernel name, or
 * "lib:<kind>" for a library step, "-" for a view that launches nothing. */
PJRTX_HIP_API int pjrtx_executable_step_names(struct PJRT_LoadedExecutable* exe, char* out, size_t cap, size_t* needed);

/* Counters of the executable: executions, kernel launches, library calls,
 * released intermediate values. */
PJRTX_HIP_API int pjrtx_executable_stats(struct PJRT_LoadedExecutable* exe, int64_t out[4]);

/* Graph counters of the executable: hipGraph captures and replays.
 * Repeated executions with the same large argument buffers are captured
 * once into a hipGraph and replayed (PJRTX_GRAPHS=0 turns this off). The
 * reference replays an MLX compiled trace instead
 * (execution_compiled_program.zig:18-67, api.cc:5425-5674). */
PJRTX_HIP_API int pjrtx_executable_graph_stats(struct PJRT_LoadedExecutable* exe, int64_t out[2]);

#ifdef __cplusplus
}
#endif

#endif /* PJRTX_AMD_PJRTX_HIP_H_ */
