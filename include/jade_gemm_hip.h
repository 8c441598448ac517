/*
 * GEMM-plan C ABI for MI355X (gfx950), exported by libjade_runtime_hip.so.
 * The symbol set, signatures and return codes are those of the reference's
 * per-shape GEMM bridge, native/jade_corex.h:11-29, so the reference's loader
 * (src/corex.rs:57-137, behind `jade-compute --backend corex --corex-library`)
 * binds this library unchanged. The matrix product is this library's FP32
 * MFMA kernel, not a vendor BLAS (the reference called cublasSgemm at
 * native/jade_corex.cpp:91-95).
 *
 * 0 = success; 1 = invalid input/state; 2 = runtime; 3 = BLAS (unused here);
 * 4 = allocation. Every matrix is dense, row-major. Upload/run/download
 * synchronise before returning. precision 0 = FP32 only: precision 1 (FP16
 * A/B) is rejected with code 1.
 */
#ifndef JADE_GEMM_HIP_H
#define JADE_GEMM_HIP_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* native/jade_corex.h:17 */
uint32_t jade_corex_abi_version(void);
/* native/jade_corex.h:18-19 */
int jade_corex_create(uint32_t m, uint32_t n, uint32_t k, int device, uint32_t precision, void **out, char *err,
                      size_t cap);
/* native/jade_corex.h:20-21: exact element counts. */
int jade_corex_upload(void *ctx, const float *a, size_t a_len, const float *b, size_t b_len, char *err, size_t cap);
/* native/jade_corex.h:22-24: elapsed_ms is GPU-event time of all iterations. */
int jade_corex_run(void *ctx, uint32_t iterations, double *elapsed_ms, char *err, size_t cap);
/* native/jade_corex.h:25-26 */
int jade_corex_download(void *ctx, float *out, size_t out_len, char *err, size_t cap);
/* native/jade_corex.h:27-28 */
int jade_corex_device_info(void *ctx, char *out, size_t out_cap, char *err, size_t cap);
/* native/jade_corex.h:29 */
void jade_corex_destroy(void *ctx);

#ifdef __cplusplus
}
#endif
#endif
