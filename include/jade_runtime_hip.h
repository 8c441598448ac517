/*
 * libjade_runtime_hip.so — the Jade native-runtime C ABI for AMD Instinct
 * MI355X (gfx950). A drop-in third backend next to Metal: it exports the
 * reference's jr_* set from native/jade_runtime_corex.h:9-31 with identical
 * signatures, return codes and error-text conventions, and replaces the
 * CoreX backend's runtime compilation of emitted .cu modules
 * (src/runtime/corex.rs:439-542) with precompiled gfx950 kernels selected
 * from a checked KernelSpec (jr_compile / jr_execute_dispatches).
 *
 * Conventions (unchanged from ABI 1):
 *   return 0 = success, 1 = invalid input/state, 2 = runtime, 3 = allocation;
 *   `err`/`cap` is caller storage, always NUL-terminated when cap > 0;
 *   every call on one context is serial; transfers and execute synchronise
 *   before returning, so no caller pointer is retained.
 * Additions in ABI 2 (jr_version() == 2): the context owns a registry of its
 * live allocations and compiled kernels, so ownership, exact transfer sizes,
 * binding lengths and write aliasing are validated here, before any GPU work,
 * for every caller (the reference did these checks only in its Rust layer:
 * src/runtime/corex.rs:322-332, 389-394, 556-569; src/runtime/ir.rs:340-367).
 */
#ifndef JADE_RUNTIME_HIP_H
#define JADE_RUNTIME_HIP_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* native/jade_runtime_corex.h:9-14: a raw launcher and its device pointers. */
typedef int (*jr_launch_fn)(void *stream, void **buffers);
typedef struct jr_job {
    jr_launch_fn launch;
    void **buffers;
    size_t buffer_count;
} jr_job;

/* native/jade_runtime_corex.h:18 (corex.rs:263-266 checks it). Returns 2. */
uint32_t jr_version(void);

/* native/jade_runtime_corex.h:19: opens a context on `device`: one ordered
 * non-blocking queue (default priority), an event pair for timing and an
 * empty region table. */
int jr_create(int device, void **out, char *err, size_t cap);

/* native/jade_runtime_corex.h:20: synchronises, releases kernels, allocations,
 * events and the stream. Null-safe. */
void jr_destroy(void *ctx);

/* native/jade_runtime_corex.h:21: one line naming the device, e.g.
 * "hip:0 AMD Instinct MI355X isa=gfx950:sramecc+:xnack- cus=256
 * hbm_bytes=... hip_runtime=... hip_driver=...". The text is informational
 * (the reference's caller stores it verbatim: corex.rs:305). */
int jr_info(void *ctx, char *out, size_t out_cap, char *err, size_t cap);

/* native/jade_runtime_corex.h:22: a nonempty device region that reads as
 * zeros before its first upload, recorded in this context's region table. */
int jr_alloc(void *ctx, size_t bytes, void **out, char *err, size_t cap);

/* native/jade_runtime_corex.h:23: synchronises, then frees. Pointers this
 * context did not allocate are ignored. */
void jr_free(void *ctx, void *ptr);

/* native/jade_runtime_corex.h:24-27: synchronous transfers. ABI 2 requires
 * `device_ptr` to be a live allocation of this context and `bytes` to equal
 * its size exactly (corex.rs:391-394). */
int jr_upload(void *ctx, void *device_ptr, const void *host_ptr, size_t bytes, char *err, size_t cap);
int jr_download(void *ctx, const void *device_ptr, void *host_ptr, size_t bytes, char *err, size_t cap);

/* native/jade_runtime_corex.h:28-31: raw launchers, whole sequence replayed
 * `repeats` times between two events; gpu_ms covers the whole sequence. */
int jr_execute(void *ctx, const jr_job *jobs, size_t job_count, uint32_t repeats, double *gpu_ms, char *err,
               size_t cap);

/* ---- ABI 2: precompiled kernels from a KernelSpec --------------------- */

/* Context-free and GPU-free: parses a KernelSpec JSON document (the serde
 * format of src/runtime/ir.rs:6-84), validates it under the HIP rules and
 * writes a JSON description: canonical spec, name, bindings (ir.rs:269-339),
 * the HIP launch shape, whether the reference's own rules (ir.rs:193-268)
 * accept it, and whether this backend runs it. */
int jr_spec_describe(const char *spec_json, size_t len, char *out, size_t out_cap, char *err, size_t cap);

/* KernelSpec::validate_bindings, src/runtime/ir.rs:340-367, context-free:
 * `lengths` are f32 element counts and `ids` buffer identities, one per
 * binding in order. 0 when the binding count and every length match and no
 * write binding shares an identity with another binding; 1 otherwise. */
int jr_spec_validate_bindings(const char *spec_json, size_t len, const uint64_t *lengths, const uint64_t *ids,
                              size_t count, char *err, size_t cap);

/* Replaces CorexRuntime::compile (corex.rs:439-542): validates the spec and
 * returns a kernel handle owned by this context. Identical canonical specs
 * share one cached pipeline (the reference caches by source text). */
int jr_compile(void *ctx, const char *spec_json, size_t len, void **kernel, char *err, size_t cap);

/* Releases one jr_compile reference; the pipeline is destroyed with its last. */
void jr_kernel_release(void *ctx, void *kernel);

/* Same JSON description as jr_spec_describe, for a compiled kernel. */
int jr_kernel_describe(void *ctx, void *kernel, char *out, size_t out_cap, char *err, size_t cap);

/* One dispatch of a compiled kernel over device buffers in binding order
 * (Dispatch{kernel, buffers}, src/runtime/mod.rs:30-33). */
typedef struct jr_dispatch {
    void *kernel;
    void **buffers;
    size_t buffer_count;
} jr_dispatch;

/* Replaces CorexRuntime::execute (corex.rs:544-612): validates every job
 * (kernel and buffers owned by this context, binding count, exact lengths,
 * no write aliasing) before anything is enqueued, then records the start
 * event, launches `repeats` x jobs in order on the context stream, records
 * the stop event and synchronises. */
int jr_execute_dispatches(void *ctx, const jr_dispatch *jobs, size_t job_count, uint32_t repeats, double *gpu_ms,
                          char *err, size_t cap);

/* Element count (f32) of a live allocation of this context. */
int jr_buffer_elements(void *ctx, const void *device_ptr, size_t *elements, char *err, size_t cap);

/* Synthetic inputs on the host (the harness generators the reference's
 * experiments use). workloads::values, src/runtime/workloads.rs:17-27:
 * xorshift32 (13,17,5) then ((s>>8)/2^24*2-1)*scale; scale 1 reproduces
 * validation::inputs (src/validation.rs:6-21). */
int jr_fill_values(float *out, size_t len, uint32_t seed, float scale);
/* No reference counterpart (its experiments are uniform only): Box-Muller over
 * the same xorshift32 stream, two draws per value, u1=((s>>8)+1)/2^24,
 * u2=(s>>8)/2^24, mean + sigma*sqrt(-2 ln u1)*cos(2 pi u2) in FP64. */
int jr_fill_normal(float *out, size_t len, uint32_t seed, float mean, float sigma);

/* No counterpart in the reference (introspection of jr_execute_dispatches):
 * validates the batch exactly as jr_execute_dispatches does, enqueues
 * nothing, and writes the launches it would make, in order, as
 * space-separated "form:first_job" items, form one of single, pair
 * (two GEMMs of one shape in one launch), gate_up_swiglu (gate and up GEMMs
 * with their SwiGLU) or gemm_residual (a GEMM with the Add of its output).
 * Codes as above (1 invalid, 2 runtime). */
int jr_plan_dispatches(void *ctx, const jr_dispatch *jobs, size_t job_count, char *out, size_t out_cap, char *err,
                       size_t cap);

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): C = A B for device pointers A [m,k], B [k,n], C [m,n]
 * (16-byte aligned A and B), the same kernels and results as a compiled
 * {"op":"gemm"} pipeline run by jr_execute_dispatches, launched
 * asynchronously on `stream` (a hipStream_t of the current device; NULL is
 * the null stream). Nothing is allocated: the split-K partials of small grids
 * use a static 8 MiB device array that each GPU holds until the process
 * ends, enough for every plan of the current planner; a shape needing more
 * is rejected with code 1. Calls that overlap on one GPU race on that array.
 * The array's device address is looked up by jr_create for its device, or
 * else by the first call on a device that needs it; a caller that captures
 * calls into a HIP graph creates a context on that device (or makes one
 * uncaptured call) first. Codes as above (1 invalid, 2 runtime). */
int jr_gemm_f32_noalloc(void *stream, const float *a, const float *b, float *c, uint32_t m, uint32_t n, uint32_t k,
                        char *err, size_t cap);

#ifdef __cplusplus
}
#endif
#endif
