/*
 * warpir_rt -- the C-ABI launcher of the WarpIR MI355X (gfx950) backend.
 *
 * The reference has no native launcher of its own: its harness JIT-builds a
 * pybind wrapper around each generated kernel and launches it with the
 * triple-chevron syntax on the default stream
 * (reference tests/test_modal_gpu.py:24-50, tests/test_modal_attention.py:25-39,
 * built by tests/test_modal_gpu.py:80-99).  This library replaces that
 * wrapper with a fixed, kernel-independent C ABI: a code object produced by
 * the CDNA4 lowering is loaded once, its kernel looked up by the IR kernel's
 * name, and launched with a packed kernel-argument buffer whose layout is the
 * kernel's globals struct (inputs then outputs, in IR order; the reference's
 * `global_vars`, warpir/lowering/lowering.py:291-298).
 *
 * Conventions
 *   - Every function returns 0 on success or a hipError_t code; the message of
 *     any code is available from wir_error_string().
 *   - Plain pointers and sizes only.  Device buffers are owned by the caller
 *     (PyTorch in the Python host); the library allocates no user memory.
 *   - Streams are passed as opaque `void*` (a hipStream_t; NULL = the null
 *     stream).  Launches are asynchronous on that stream.
 */
#ifndef WARPIR_RT_H
#define WARPIR_RT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* wir_module_t;   /* a loaded code object (hipModule_t)      */
typedef void* wir_function_t; /* a kernel inside a module (hipFunction_t) */
typedef void* wir_event_t;    /* a timing event (hipEvent_t)              */

/* ABI version of this header; bumped on any signature change. */
#define WIR_RT_ABI_VERSION 4
int wir_abi_version(void);

/* Make `device` current for the calling thread. */
int wir_set_device(int device);

/* Device facts used by the lowering and by roofline reporting:
 * compute-unit count, peak shader clock (kHz), LDS bytes per workgroup and
 * the gfx architecture name (NUL-terminated, truncated to arch_len). */
int wir_device_info(int device, int* num_cus, int* clock_khz, int* lds_per_block,
                    char* arch, size_t arch_len);

/* Load a code object image (an ELF .hsaco as bytes).  Replaces the
 * reference's load_inline build-and-dlopen step (tests/test_modal_gpu.py:80-99). */
int wir_module_load(const void* image, size_t size, wir_module_t* module);
int wir_module_unload(wir_module_t module);

/* Look up the kernel named `name` (the IR Kernel.name) in a loaded module. */
int wir_module_get_function(wir_module_t module, const char* name, wir_function_t* function);

/* Launch `function` on `stream` with grid (gx, gy, gz) of workgroups of
 * (bx, by, bz) work-items and `dyn_lds` bytes of dynamic LDS.  `kernarg`
 * points at `kernarg_size` bytes laid out as the kernel's globals struct.
 * Replaces the reference launch wrappers (`gemm<<<grid, 128[, smem]>>>(g)`,
 * tests/test_modal_gpu.py:24-50). */
int wir_launch(wir_function_t function, unsigned gx, unsigned gy, unsigned gz,
               unsigned bx, unsigned by, unsigned bz, unsigned dyn_lds, void* stream,
               const void* kernarg, size_t kernarg_size);

/* Kernel resource facts (from the code object's metadata): registers per
 * work-item, static LDS bytes and the maximum work-group size. */
int wir_function_attrs(wir_function_t function, int* num_regs, int* static_lds,
                       int* max_threads);

/* Wait for all work queued on `stream`, or on the whole device. */
int wir_stream_sync(void* stream);
int wir_device_sync(void);

/* Timing events on a stream (the reference times with CUDA events,
 * tests/test_modal_gpu.py:138-151). */
int wir_event_create(wir_event_t* event);
int wir_event_destroy(wir_event_t event);
int wir_event_record(wir_event_t event, void* stream);
int wir_event_elapsed_ms(wir_event_t start, wir_event_t end, float* ms);

/* Human-readable message for a code returned by any function in this header
 * (hipError_t codes and the WIR_ERROR_* codes below). */
const char* wir_error_string(int code);

/* Returned when an input needs more device scratch than the library holds. */
#define WIR_ERROR_SCRATCH_LIMIT 20001

/* Floats of device scratch held by wir_gemm_splitk_noalloc: 8 Mi fp32 values
 * (32 MiB) on every device the library runs on, until the process ends. */
#define WIR_NOALLOC_SCRATCH_FLOATS (8 * 1024 * 1024)

/* out[M][N] (bf16) = a[M][K] @ b[K][N] (bf16, row-major, contiguous) as
 * `splits` K slices plus an fp32 reduction, the partials in `workspace`
 * (fp32, at least splits * M * N of its `workspace_floats`, 16-byte
 * aligned): both launches of one product in one call, on `stream`.  The
 * reference has no split-K path; this is the host side of
 * warpir_amd.api.gemm_split_k, whose short-M products would otherwise be
 * bound by per-launch host work.  gemm and reduce as below. */
int wir_gemm_splitk(wir_function_t gemm, wir_function_t reduce, const void* a, const void* b,
                    void* out, void* workspace, size_t workspace_floats, int m, int n, int k,
                    int splits, void* stream);

/* out[M][N] (bf16) = a[M][K] @ b[K][N] (bf16, row-major, contiguous) as
 * `splits` K slices in ONE launch: `gemm` is a fused split-K variant
 * (gemm_128_splitk_fused) whose last slice to store a 128x128 output tile
 * sums the tile's fp32 partials (in `workspace`, as for wir_gemm_splitk) in
 * slice order and writes the bf16 tile.  `arrivals` holds one 32-bit
 * counter per output tile, at least ceil(M/128) * ceil(N/128) of its
 * `arrival_count`, all zero before the call; the kernel leaves them zero.
 * Calls that share `workspace` or `arrivals` must be ordered (one stream).
 * The reference has no split-K path; this is the host side of
 * warpir_amd.api.gemm_split_k with its fused variant.  Same limits as
 * wir_gemm_splitk. */
int wir_gemm_splitk_fused(wir_function_t gemm, const void* a, const void* b, void* out, void* workspace,
                          size_t workspace_floats, void* arrivals, size_t arrival_count, int m, int n,
                          int k, int splits, void* stream);

/* out[M][N] (bf16) = a[M][K] @ b[K][N] (bf16, row-major, contiguous) as
 * `splits` K slices plus an fp32 reduction, with no device allocation: the
 * fp32 partials live in the library's own device scratch instead of a
 * workspace.  No counterpart in the reference; it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).
 *   gemm   -- a split-K GEMM variant (128x128 tiles, 4 wavefronts:
 *             gemm_128_splitk*), loaded from its code object;
 *   reduce -- wir_splitk_reduce, loaded from splitk_reduce.hsaco.
 * Requires 1 <= splits <= 16, K % (64 * splits) == 0, N % 8 == 0 and 16-byte
 * aligned a, b, out; returns WIR_ERROR_SCRATCH_LIMIT when
 * splits * M * N > WIR_NOALLOC_SCRATCH_FLOATS.  Runs on the current device,
 * which must own `stream`.  Every call on one device shares that device's
 * scratch: calls that overlap on one device race, so order them on one
 * stream. */
int wir_gemm_splitk_noalloc(wir_function_t gemm, wir_function_t reduce, const void* a,
                            const void* b, void* out, int m, int n, int k, int splits,
                            void* stream);

#ifdef __cplusplus
}
#endif

#endif /* WARPIR_RT_H */
