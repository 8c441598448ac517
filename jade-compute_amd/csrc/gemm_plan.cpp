// Per-shape GEMM-plan ABI (native/jade_corex.h:11-29) over this library's FP32
// MFMA GEMM: one context holds M,N,K, device A/B/C, a non-blocking stream and
// two events; run() replays the product `iterations` times between events.
// Mirrors the state machine of native/jade_corex.cpp:113-291 (upload before
// run, run before download, exact element counts).
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <limits>
#include <new>

#include "jade_gemm_hip.h"
#include "kernels.hpp"

namespace {

struct Plan {
    int m = 0, n = 0, k = 0, device = 0;
    size_t a_len = 0, b_len = 0, c_len = 0;
    float *a = nullptr, *b = nullptr, *c = nullptr;
    float *workspace = nullptr;  // split-K partials for small output grids
    hipStream_t stream = nullptr;
    hipEvent_t start = nullptr, stop = nullptr;
    bool uploaded = false, computed = false;
};

void clear_error(char *err, size_t cap) {
    if (err && cap) err[0] = '\0';
}
int fail(int code, char *err, size_t cap, const char *format, ...) {
    if (err && cap) {
        va_list args;
        va_start(args, format);
        std::vsnprintf(err, cap, format, args);
        va_end(args);
        err[cap - 1] = '\0';
    }
    return code;
}
int runtime_error(hipError_t status, char *err, size_t cap, const char *op) {
    return fail(2, err, cap, "%s: %s (runtime code %d)", op, hipGetErrorString(status), static_cast<int>(status));
}
int select(Plan *p, char *err, size_t cap) {
    if (!p) return fail(1, err, cap, "null context");
    const auto status = hipSetDevice(p->device);
    return status == hipSuccess ? 0 : runtime_error(status, err, cap, "hipSetDevice");
}
bool matrix_size(uint32_t x, uint32_t y, size_t &count) {
    const auto maximum = std::numeric_limits<size_t>::max();
    if (!x || !y || static_cast<size_t>(x) > maximum / y) return false;
    count = static_cast<size_t>(x) * y;
    return count <= maximum / sizeof(float);
}
void cleanup(Plan *p) {
    if (!p) return;
    (void)hipSetDevice(p->device);
    if (p->stream) (void)hipStreamSynchronize(p->stream);
    if (p->start) (void)hipEventDestroy(p->start);
    if (p->stop) (void)hipEventDestroy(p->stop);
    if (p->a) (void)hipFree(p->a);
    if (p->b) (void)hipFree(p->b);
    if (p->c) (void)hipFree(p->c);
    if (p->workspace) (void)hipFree(p->workspace);
    if (p->stream) (void)hipStreamDestroy(p->stream);
    delete p;
}

}  // namespace

extern "C" uint32_t jade_corex_abi_version(void) { return 1; }

extern "C" int jade_corex_create(uint32_t m, uint32_t n, uint32_t k, int device, uint32_t precision, void **out,
                                 char *err, size_t cap) {
    clear_error(err, cap);
    if (!out) return fail(1, err, cap, "null output handle");
    *out = nullptr;
    if (!m || !n || !k || m > INT_MAX || n > INT_MAX || k > INT_MAX || device < 0 || precision > 1)
        return fail(1, err, cap, "dimensions must be 1..INT_MAX; device >= 0; precision 0 or 1");
    if (precision == 1)
        return fail(1, err, cap, "precision 1 (FP16 inputs) is not provided by the HIP backend; use precision 0");
    auto *p = new (std::nothrow) Plan();
    if (!p) return fail(4, err, cap, "context allocation failed");
    p->m = int(m);
    p->n = int(n);
    p->k = int(k);
    p->device = device;
    if (!matrix_size(m, k, p->a_len) || !matrix_size(k, n, p->b_len) || !matrix_size(m, n, p->c_len) ||
        p->a_len > size_t(INT_MAX) || p->b_len > size_t(INT_MAX) || p->c_len > size_t(INT_MAX)) {
        delete p;
        return fail(1, err, cap, "each matrix must hold at most INT_MAX elements");
    }
    const auto initialize = [&]() -> int {
        int count = 0;
        auto status = hipGetDeviceCount(&count);
        if (status != hipSuccess) return runtime_error(status, err, cap, "hipGetDeviceCount");
        if (device >= count) return fail(1, err, cap, "device %d outside detected count %d", device, count);
        int rc = select(p, err, cap);
        if (rc) return rc;
        status = hipStreamCreateWithFlags(&p->stream, hipStreamNonBlocking);
        if (status != hipSuccess) return runtime_error(status, err, cap, "hipStreamCreateWithFlags");
        status = hipEventCreate(&p->start);
        if (status != hipSuccess) return runtime_error(status, err, cap, "hipEventCreate(start)");
        status = hipEventCreate(&p->stop);
        if (status != hipSuccess) return runtime_error(status, err, cap, "hipEventCreate(stop)");
        status = hipMalloc(&p->a, p->a_len * sizeof(float));
        if (status != hipSuccess) return fail(4, err, cap, "hipMalloc(A): %s", hipGetErrorString(status));
        status = hipMalloc(&p->b, p->b_len * sizeof(float));
        if (status != hipSuccess) return fail(4, err, cap, "hipMalloc(B): %s", hipGetErrorString(status));
        status = hipMalloc(&p->c, p->c_len * sizeof(float));
        if (status != hipSuccess) return fail(4, err, cap, "hipMalloc(C): %s", hipGetErrorString(status));
        const size_t ws = jade::hipk::gemm_f32_workspace_bytes(m, n, k);
        if (ws) {
            status = hipMalloc(&p->workspace, ws);
            if (status != hipSuccess) return fail(4, err, cap, "hipMalloc(workspace): %s", hipGetErrorString(status));
        }
        return 0;
    };
    const int rc = initialize();
    if (rc) {
        cleanup(p);
        return rc;
    }
    *out = p;
    return 0;
}

extern "C" int jade_corex_upload(void *handle, const float *a, size_t a_len, const float *b, size_t b_len, char *err,
                                 size_t cap) {
    clear_error(err, cap);
    auto *p = static_cast<Plan *>(handle);
    if (!p || !a || !b || a_len != p->a_len || b_len != p->b_len)
        return fail(1, err, cap, "upload requires non-null buffers and exact A/B element counts");
    p->uploaded = false;
    p->computed = false;
    const int rc = select(p, err, cap);
    if (rc) return rc;
    auto status = hipMemcpyAsync(p->a, a, a_len * sizeof(float), hipMemcpyHostToDevice, p->stream);
    if (status == hipSuccess) status = hipMemcpyAsync(p->b, b, b_len * sizeof(float), hipMemcpyHostToDevice, p->stream);
    const auto sync = hipStreamSynchronize(p->stream);
    if (status != hipSuccess) return runtime_error(status, err, cap, "hipMemcpyAsync(upload)");
    if (sync != hipSuccess) return runtime_error(sync, err, cap, "hipStreamSynchronize(upload)");
    p->uploaded = true;
    return 0;
}

extern "C" int jade_corex_run(void *handle, uint32_t iterations, double *elapsed_ms, char *err, size_t cap) {
    clear_error(err, cap);
    if (elapsed_ms) *elapsed_ms = 0;
    auto *p = static_cast<Plan *>(handle);
    if (!p || !iterations || !elapsed_ms)
        return fail(1, err, cap, "run requires context, iterations > 0 and elapsed output");
    p->computed = false;
    if (!p->uploaded) return fail(1, err, cap, "upload A/B before running");
    const int rc = select(p, err, cap);
    if (rc) return rc;
    auto status = hipEventRecord(p->start, p->stream);
    if (status != hipSuccess) return runtime_error(status, err, cap, "hipEventRecord(start)");
    for (uint32_t i = 0; i < iterations; ++i) {
        status = jade::hipk::gemm_f32(p->stream, p->a, p->b, p->c, uint32_t(p->m), uint32_t(p->n), uint32_t(p->k),
                                      p->workspace);
        if (status != hipSuccess) {
            (void)hipStreamSynchronize(p->stream);
            return runtime_error(status, err, cap, "matrix multiplication");
        }
    }
    status = hipEventRecord(p->stop, p->stream);
    if (status != hipSuccess) {
        (void)hipStreamSynchronize(p->stream);
        return runtime_error(status, err, cap, "hipEventRecord(stop)");
    }
    status = hipEventSynchronize(p->stop);
    if (status != hipSuccess) return runtime_error(status, err, cap, "hipEventSynchronize");
    float milliseconds = 0;
    status = hipEventElapsedTime(&milliseconds, p->start, p->stop);
    if (status != hipSuccess) return runtime_error(status, err, cap, "hipEventElapsedTime");
    if (!std::isfinite(milliseconds) || milliseconds < 0) return fail(2, err, cap, "invalid GPU event duration");
    *elapsed_ms = static_cast<double>(milliseconds);
    p->computed = true;
    return 0;
}

extern "C" int jade_corex_download(void *handle, float *out, size_t out_len, char *err, size_t cap) {
    clear_error(err, cap);
    auto *p = static_cast<Plan *>(handle);
    if (!p || !out || out_len != p->c_len) return fail(1, err, cap, "download requires exact C element count");
    if (!p->computed) return fail(1, err, cap, "run successfully before downloading C");
    const int rc = select(p, err, cap);
    if (rc) return rc;
    const auto status = hipMemcpyAsync(out, p->c, p->c_len * sizeof(float), hipMemcpyDeviceToHost, p->stream);
    const auto sync = hipStreamSynchronize(p->stream);
    if (status != hipSuccess) return runtime_error(status, err, cap, "hipMemcpyAsync(download)");
    return sync == hipSuccess ? 0 : runtime_error(sync, err, cap, "hipStreamSynchronize(download)");
}

extern "C" int jade_corex_device_info(void *handle, char *out, size_t out_cap, char *err, size_t cap) {
    clear_error(err, cap);
    if (out && out_cap) out[0] = '\0';
    auto *p = static_cast<Plan *>(handle);
    if (!p || !out || !out_cap) return fail(1, err, cap, "device info requires context and output buffer");
    const int rc = select(p, err, cap);
    if (rc) return rc;
    hipDeviceProp_t prop{};
    auto status = hipGetDeviceProperties(&prop, p->device);
    if (status != hipSuccess) return runtime_error(status, err, cap, "hipGetDeviceProperties");
    int runtime = 0, driver = 0;
    status = hipRuntimeGetVersion(&runtime);
    if (status != hipSuccess) return runtime_error(status, err, cap, "hipRuntimeGetVersion");
    status = hipDriverGetVersion(&driver);
    if (status != hipSuccess) return runtime_error(status, err, cap, "hipDriverGetVersion");
    const int needed = std::snprintf(out, out_cap,
                                     "device=%d name=%.255s memory_bytes=%llu multiprocessors=%d runtime_api=%d "
                                     "driver_api=%d blas_api=0 precision=fp32 arch=%.63s gemm=jade_mfma_f32",
                                     p->device, prop.name, static_cast<unsigned long long>(prop.totalGlobalMem),
                                     prop.multiProcessorCount, runtime, driver, prop.gcnArchName);
    if (needed < 0 || static_cast<size_t>(needed) >= out_cap) {
        out[out_cap - 1] = '\0';
        return fail(1, err, cap, "device info output buffer too small");
    }
    return 0;
}

extern "C" void jade_corex_destroy(void *handle) { cleanup(static_cast<Plan *>(handle)); }
