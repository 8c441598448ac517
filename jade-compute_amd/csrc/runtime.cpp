// jr_* ABI 2 for gfx950: the device layer of the reference's native runtime
// (native/jade_runtime_corex.cpp:1-189) plus the checks its Rust CoreX backend
// did before calling it (src/runtime/corex.rs:322-612), re-designed around
// precompiled HIP kernels instead of runtime-compiled modules.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "jade_runtime_hip.h"
#include "kernels.hpp"
#include "spec.hpp"

namespace {

using jade::Binding;
using jade::KernelSpec;
using jade::Op;

struct Context;

// A compiled pipeline: a validated spec bound to one precompiled kernel.
struct Pipeline {
    Context *owner = nullptr;
    KernelSpec spec;
    std::string canonical;
    std::vector<Binding> binds;
    jade::Instr *program = nullptr;  // device copy of an Elementwise program
    uint32_t program_len = 0;
    float *workspace = nullptr;      // split-K / split-key partials of a small GEMM or attention grid
    bool copy = false;  // Elementwise whose expression is input0
    int refs = 0;
};

struct Allocation {
    size_t bytes;
    uint64_t id;
};

struct Context {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t start = nullptr, stop = nullptr;
    std::unordered_map<const void *, Allocation> allocations;
    std::unordered_map<std::string, Pipeline *> cache;
    std::unordered_set<Pipeline *> pipelines;
    uint64_t next_id = 1;
};

std::mutex g_registry_mutex;
std::unordered_set<Context *> g_contexts;

Context *lookup(void *handle) {
    std::lock_guard<std::mutex> lock(g_registry_mutex);
    auto *ctx = static_cast<Context *>(handle);
    return g_contexts.count(ctx) ? ctx : nullptr;
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
void clear(char *err, size_t cap) {
    if (err && cap) err[0] = '\0';
}
int hip_fail(hipError_t status, char *err, size_t cap, const char *operation) {
    return fail(2, err, cap, "%s: %s (%d)", operation, hipGetErrorString(status), static_cast<int>(status));
}
int select(Context *ctx, char *err, size_t cap) {
    if (!ctx) return fail(1, err, cap, "null or unknown runtime context");
    const auto status = hipSetDevice(ctx->device);
    return status == hipSuccess ? 0 : hip_fail(status, err, cap, "hipSetDevice");
}

void release_pipeline(Context *ctx, Pipeline *p) {
    if (p->program) (void)hipFree(p->program);
    if (p->workspace) (void)hipFree(p->workspace);
    ctx->cache.erase(p->canonical);
    ctx->pipelines.erase(p);
    delete p;
}

void destroy(Context *ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    for (Pipeline *p : std::vector<Pipeline *>(ctx->pipelines.begin(), ctx->pipelines.end())) release_pipeline(ctx, p);
    for (auto &a : ctx->allocations) (void)hipFree(const_cast<void *>(a.first));
    ctx->allocations.clear();
    if (ctx->start) (void)hipEventDestroy(ctx->start);
    if (ctx->stop) (void)hipEventDestroy(ctx->stop);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

jade::hipk::LaunchShape launch_shape(const KernelSpec &s) {
    using namespace jade::hipk;
    switch (s.op) {
        case Op::Elementwise: {
            const auto &e = *s.expression;
            if (e.kind == jade::Expr::Kind::Input && e.binding == 0) {
                auto shape = stream_shape(s.len);
                shape.kernel = "copy_stream";
                return shape;
            }
            return elementwise_shape(s.len);
        }
        case Op::Axpy:
        case Op::Add:
        case Op::SwiGlu: return stream_shape(s.len);
        case Op::Gemm:
        case Op::GemmSimd: return gemm_f32_shape(s.m, s.n, s.k);
        case Op::AttentionOnline: return attention_online_shape(s.heads, s.seq, s.dim, s.causal);
        case Op::AttentionScores: return attention_scores_shape(s.heads, s.seq, s.dim, s.causal);
        case Op::AttentionApply: return attention_apply_shape(s.heads, s.seq, s.dim);
        case Op::RmsNorm: return rms_norm_shape(s.rows, s.cols);
        case Op::Softmax: return softmax_shape(s.rows, s.cols);
        case Op::GemmMps: break;
    }
    return {nullptr, {0, 0, 0}, {0, 0, 0}, 0};
}

hipError_t launch(const Pipeline &p, hipStream_t st, void *const *b) {
    using namespace jade::hipk;
    const KernelSpec &s = p.spec;
    auto in = [&](size_t i) { return static_cast<const float *>(b[i]); };
    auto out = [&](size_t i) { return static_cast<float *>(b[i]); };
    switch (s.op) {
        case Op::Elementwise: {
            if (p.copy) return copy_f32(st, in(0), out(s.inputs), s.len);
            const float *inputs[jade::kMaxElementwiseInputs] = {};
            for (uint32_t i = 0; i < s.inputs; ++i) inputs[i] = in(i);
            return elementwise_f32(st, inputs, s.inputs, out(s.inputs), s.len, p.program, p.program_len);
        }
        case Op::Axpy: return axpy_f32(st, s.alpha, in(0), in(1), out(2), s.len);
        case Op::Add: return add_f32(st, in(0), in(1), out(2), s.len);
        case Op::SwiGlu: return swiglu_f32(st, in(0), in(1), out(2), s.len);
        case Op::Gemm:
        case Op::GemmSimd: return gemm_f32(st, in(0), in(1), out(2), s.m, s.n, s.k, p.workspace);
        case Op::AttentionOnline:
            return attention_online_f32(st, in(0), in(1), in(2), out(3), s.heads, s.seq, s.dim, s.causal,
                                        p.workspace);
        case Op::AttentionScores:
            return attention_scores_f32(st, in(0), in(1), out(2), s.heads, s.seq, s.dim, s.causal);
        case Op::AttentionApply: return attention_apply_f32(st, in(0), in(1), out(2), s.heads, s.seq, s.dim);
        case Op::RmsNorm: return rms_norm_f32(st, in(0), in(1), out(2), s.rows, s.cols, s.epsilon);
        case Op::Softmax: return softmax_f32(st, in(0), out(1), s.rows, s.cols);
        case Op::GemmMps: break;
    }
    return hipErrorInvalidValue;
}

// Device workspace a pipeline allocates at jr_compile (split-K partial
// products of small GEMM grids, split-key partial rows of small attention
// grids); 0 for every other launch.
size_t workspace_bytes_for(const KernelSpec &spec) {
    if (spec.op == Op::Gemm || spec.op == Op::GemmSimd)
        return jade::hipk::gemm_f32_workspace_bytes(spec.m, spec.n, spec.k);
    if (spec.op == Op::AttentionOnline)
        return jade::hipk::attention_online_workspace_bytes(spec.heads, spec.seq, spec.dim, spec.causal);
    return 0;
}

std::string describe(const KernelSpec &spec) {
    std::string ref_error, hip_error;
    const bool reference_valid = jade::validate(spec, jade::Rules::Reference, ref_error);
    const bool supported = jade::hip_supported(spec, hip_error);
    std::string out = "{\"name\":" + jade::json::quote(jade::spec_name(spec)) +
                      ",\"spec\":" + jade::canonical_json(spec) + ",\"bindings\":[";
    const auto binds = jade::bindings(spec);
    for (size_t i = 0; i < binds.size(); ++i) {
        if (i) out += ",";
        out += "{\"name\":" + jade::json::quote(binds[i].name) +
               ",\"elements\":" + std::to_string(binds[i].elements) +
               ",\"write\":" + (binds[i].write ? "true" : "false") + "}";
    }
    out += std::string("],\"reference_valid\":") + (reference_valid ? "true" : "false");
    out += ",\"reference_error\":" + (reference_valid ? std::string("null") : jade::json::quote(ref_error));
    out += std::string(",\"hip_supported\":") + (supported ? "true" : "false");
    out += ",\"hip_error\":" + (supported ? std::string("null") : jade::json::quote(hip_error));
    if (supported) {
        const auto shape = launch_shape(spec);
        out += ",\"launch\":{\"kernel\":" + jade::json::quote(shape.kernel) + ",\"grid\":[" +
               std::to_string(shape.grid[0]) + "," + std::to_string(shape.grid[1]) + "," +
               std::to_string(shape.grid[2]) + "],\"block\":[" + std::to_string(shape.block[0]) + "," +
               std::to_string(shape.block[1]) + "," + std::to_string(shape.block[2]) +
               "],\"lds_bytes\":" + std::to_string(shape.lds_bytes) + "}";
        out += ",\"workspace_bytes\":" + std::to_string(workspace_bytes_for(spec));
    } else {
        out += ",\"launch\":null,\"workspace_bytes\":0";
    }
    return out + "}";
}

int write_text(const std::string &text, char *out, size_t out_cap, char *err, size_t cap) {
    if (text.size() + 1 > out_cap) {
        out[out_cap - 1] = '\0';
        return fail(1, err, cap, "description output buffer too small (%zu bytes needed)", text.size() + 1);
    }
    std::memcpy(out, text.c_str(), text.size() + 1);
    return 0;
}

int parse_checked(const char *spec_json, size_t len, KernelSpec &spec, char *err, size_t cap) {
    if (!spec_json || !len) return fail(1, err, cap, "empty kernel spec");
    std::string error;
    if (!jade::parse_spec(std::string(spec_json, len), spec, error))
        return fail(1, err, cap, "kernel spec: %s", error.c_str());
    if (!jade::validate(spec, jade::Rules::Hip, error))
        return fail(1, err, cap, "%s: %s", jade::spec_name(spec), error.c_str());
    return 0;
}

}  // namespace

extern "C" uint32_t jr_version(void) { return 2; }

extern "C" int jr_create(int device, void **out, char *err, size_t cap) {
    clear(err, cap);
    if (!out) return fail(1, err, cap, "null output handle");
    *out = nullptr;
    if (device < 0) return fail(1, err, cap, "negative device index");
    int count = 0;
    auto status = hipGetDeviceCount(&count);
    if (status != hipSuccess) return hip_fail(status, err, cap, "hipGetDeviceCount");
    if (device >= count) return fail(1, err, cap, "device %d outside device count %d", device, count);
    auto *ctx = new (std::nothrow) Context;
    if (!ctx) return fail(3, err, cap, "runtime context allocation failed");
    ctx->device = device;
    int rc = select(ctx, err, cap);
    if (rc) {
        destroy(ctx);
        return rc;
    }
    status = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (status == hipSuccess) status = hipEventCreate(&ctx->start);
    if (status == hipSuccess) status = hipEventCreate(&ctx->stop);
    if (status != hipSuccess) {
        rc = hip_fail(status, err, cap, "create stream/timing events");
        destroy(ctx);
        return rc;
    }
    {
        std::lock_guard<std::mutex> lock(g_registry_mutex);
        g_contexts.insert(ctx);
    }
    *out = ctx;
    return 0;
}

extern "C" void jr_destroy(void *handle) {
    Context *ctx = lookup(handle);
    if (!ctx) return;
    {
        std::lock_guard<std::mutex> lock(g_registry_mutex);
        g_contexts.erase(ctx);
    }
    destroy(ctx);
}

extern "C" int jr_info(void *handle, char *out, size_t out_cap, char *err, size_t cap) {
    clear(err, cap);
    if (out && out_cap) out[0] = '\0';
    if (!out || !out_cap) return fail(1, err, cap, "missing device-info output");
    Context *ctx = lookup(handle);
    const int rc = select(ctx, err, cap);
    if (rc) return rc;
    hipDeviceProp_t prop{};
    auto status = hipGetDeviceProperties(&prop, ctx->device);
    if (status != hipSuccess) return hip_fail(status, err, cap, "hipGetDeviceProperties");
    int runtime = 0, driver = 0;
    status = hipRuntimeGetVersion(&runtime);
    if (status == hipSuccess) status = hipDriverGetVersion(&driver);
    if (status != hipSuccess) return hip_fail(status, err, cap, "runtime/driver version");
    const int n = std::snprintf(out, out_cap,
                                "device=%d name=%.255s memory_bytes=%llu runtime_api=%d driver_api=%d arch=%.63s "
                                "compute_units=%d",
                                ctx->device, prop.name, static_cast<unsigned long long>(prop.totalGlobalMem), runtime,
                                driver, prop.gcnArchName, prop.multiProcessorCount);
    if (n < 0 || static_cast<size_t>(n) >= out_cap) {
        out[out_cap - 1] = '\0';
        return fail(1, err, cap, "device-info output too small");
    }
    return 0;
}

extern "C" int jr_alloc(void *handle, size_t bytes, void **out, char *err, size_t cap) {
    clear(err, cap);
    if (!out) return fail(1, err, cap, "null allocation output");
    *out = nullptr;
    if (!bytes) return fail(1, err, cap, "allocation must be nonempty");
    Context *ctx = lookup(handle);
    const int rc = select(ctx, err, cap);
    if (rc) return rc;
    auto status = hipMalloc(out, bytes);
    if (status != hipSuccess) {
        *out = nullptr;
        const int code = status == hipErrorOutOfMemory ? 3 : 2;
        return fail(code, err, cap, "hipMalloc(%zu): %s (%d)", bytes, hipGetErrorString(status), int(status));
    }
    // Public allocations contain defined zeros, even before the first upload.
    status = hipMemsetAsync(*out, 0, bytes, ctx->stream);
    const auto sync = hipStreamSynchronize(ctx->stream);
    if (status != hipSuccess || sync != hipSuccess) {
        (void)hipFree(*out);
        *out = nullptr;
        return hip_fail(status != hipSuccess ? status : sync, err, cap, "initialize allocation");
    }
    try {
        ctx->allocations.emplace(*out, Allocation{bytes, ctx->next_id++});
    } catch (...) {
        (void)hipFree(*out);
        *out = nullptr;
        return fail(3, err, cap, "allocation registry insert failed");
    }
    return 0;
}

extern "C" void jr_free(void *handle, void *ptr) {
    Context *ctx = lookup(handle);
    if (!ctx || !ptr) return;
    auto it = ctx->allocations.find(ptr);
    if (it == ctx->allocations.end()) return;
    if (hipSetDevice(ctx->device) != hipSuccess) return;
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipFree(ptr);
    ctx->allocations.erase(it);
}

static int transfer_check(Context *ctx, const void *device_ptr, size_t bytes, const char *what, char *err,
                          size_t cap) {
    auto it = ctx->allocations.find(device_ptr);
    if (it == ctx->allocations.end())
        return fail(1, err, cap, "%s: buffer belongs to another runtime/device context or is not live", what);
    if (it->second.bytes != bytes)
        return fail(1, err, cap, "%s element count must match buffer exactly (%zu bytes, buffer holds %zu)", what,
                    bytes, it->second.bytes);
    return 0;
}

extern "C" int jr_upload(void *handle, void *device_ptr, const void *host_ptr, size_t bytes, char *err, size_t cap) {
    clear(err, cap);
    if (!device_ptr || !host_ptr || !bytes) return fail(1, err, cap, "invalid upload buffers/size");
    Context *ctx = lookup(handle);
    int rc = select(ctx, err, cap);
    if (rc) return rc;
    rc = transfer_check(ctx, device_ptr, bytes, "upload", err, cap);
    if (rc) return rc;
    const auto status = hipMemcpyAsync(device_ptr, host_ptr, bytes, hipMemcpyHostToDevice, ctx->stream);
    const auto sync = hipStreamSynchronize(ctx->stream);
    if (status != hipSuccess) return hip_fail(status, err, cap, "upload");
    return sync == hipSuccess ? 0 : hip_fail(sync, err, cap, "upload synchronization");
}

extern "C" int jr_download(void *handle, const void *device_ptr, void *host_ptr, size_t bytes, char *err,
                           size_t cap) {
    clear(err, cap);
    if (!device_ptr || !host_ptr || !bytes) return fail(1, err, cap, "invalid download buffers/size");
    Context *ctx = lookup(handle);
    int rc = select(ctx, err, cap);
    if (rc) return rc;
    rc = transfer_check(ctx, device_ptr, bytes, "download", err, cap);
    if (rc) return rc;
    const auto status = hipMemcpyAsync(host_ptr, device_ptr, bytes, hipMemcpyDeviceToHost, ctx->stream);
    const auto sync = hipStreamSynchronize(ctx->stream);
    if (status != hipSuccess) return hip_fail(status, err, cap, "download");
    return sync == hipSuccess ? 0 : hip_fail(sync, err, cap, "download synchronization");
}

extern "C" int jr_buffer_elements(void *handle, const void *device_ptr, size_t *elements, char *err, size_t cap) {
    clear(err, cap);
    if (!elements) return fail(1, err, cap, "null elements output");
    *elements = 0;
    Context *ctx = lookup(handle);
    if (!ctx) return fail(1, err, cap, "null or unknown runtime context");
    auto it = ctx->allocations.find(device_ptr);
    if (it == ctx->allocations.end()) return fail(1, err, cap, "not a live allocation of this context");
    *elements = it->second.bytes / sizeof(float);
    return 0;
}

// Records events around `repeats` passes of `submit()`; `submit` returns a HIP status.
template <typename Submit>
static int timed_sequence(Context *ctx, uint32_t repeats, double *gpu_ms, Submit submit, char *err, size_t cap) {
    auto status = hipEventRecord(ctx->start, ctx->stream);
    if (status != hipSuccess) return hip_fail(status, err, cap, "record start event");
    for (uint32_t repeat = 0; repeat < repeats; ++repeat) {
        status = submit();
        if (status != hipSuccess) {
            (void)hipStreamSynchronize(ctx->stream);
            return hip_fail(status, err, cap, "kernel launch");
        }
    }
    status = hipEventRecord(ctx->stop, ctx->stream);
    if (status != hipSuccess) {
        (void)hipStreamSynchronize(ctx->stream);
        return hip_fail(status, err, cap, "record stop event");
    }
    status = hipEventSynchronize(ctx->stop);
    if (status != hipSuccess) return hip_fail(status, err, cap, "kernel synchronization");
    float elapsed = 0;
    status = hipEventElapsedTime(&elapsed, ctx->start, ctx->stop);
    if (status != hipSuccess) return hip_fail(status, err, cap, "event elapsed time");
    if (!std::isfinite(elapsed) || elapsed < 0) return fail(2, err, cap, "invalid GPU-event duration");
    *gpu_ms = static_cast<double>(elapsed);
    return 0;
}

extern "C" int jr_execute(void *handle, const jr_job *jobs, size_t job_count, uint32_t repeats, double *gpu_ms,
                          char *err, size_t cap) {
    clear(err, cap);
    if (gpu_ms) *gpu_ms = 0;
    if (!jobs || !job_count || !repeats || !gpu_ms)
        return fail(1, err, cap, "empty dispatch sequence or missing timing output");
    for (size_t j = 0; j < job_count; ++j) {
        if (!jobs[j].launch || !jobs[j].buffers || !jobs[j].buffer_count) return fail(1, err, cap, "invalid job %zu", j);
        for (size_t b = 0; b < jobs[j].buffer_count; ++b)
            if (!jobs[j].buffers[b]) return fail(1, err, cap, "null buffer in job %zu", j);
    }
    Context *ctx = lookup(handle);
    const int rc = select(ctx, err, cap);
    if (rc) return rc;
    return timed_sequence(
        ctx, repeats, gpu_ms,
        [&]() -> hipError_t {
            for (size_t j = 0; j < job_count; ++j) {
                const int status = jobs[j].launch(static_cast<void *>(ctx->stream), jobs[j].buffers);
                if (status != 0) return static_cast<hipError_t>(status);
            }
            return hipSuccess;
        },
        err, cap);
}

extern "C" int jr_spec_describe(const char *spec_json, size_t len, char *out, size_t out_cap, char *err,
                                size_t cap) {
    clear(err, cap);
    if (out && out_cap) out[0] = '\0';
    if (!out || !out_cap) return fail(1, err, cap, "missing description output");
    KernelSpec spec;
    const int rc = parse_checked(spec_json, len, spec, err, cap);
    if (rc) return rc;
    return write_text(describe(spec), out, out_cap, err, cap);
}

extern "C" int jr_spec_validate_bindings(const char *spec_json, size_t len, const uint64_t *lengths,
                                         const uint64_t *ids, size_t count, char *err, size_t cap) {
    clear(err, cap);
    if ((!lengths || !ids) && count) return fail(1, err, cap, "null binding arrays");
    KernelSpec spec;
    const int rc = parse_checked(spec_json, len, spec, err, cap);
    if (rc) return rc;
    std::string error;
    if (!jade::validate_bindings(spec, lengths, ids, count, error)) return fail(1, err, cap, "%s", error.c_str());
    return 0;
}

extern "C" int jr_compile(void *handle, const char *spec_json, size_t len, void **kernel, char *err, size_t cap) {
    clear(err, cap);
    if (!kernel) return fail(1, err, cap, "null kernel output");
    *kernel = nullptr;
    Context *ctx = lookup(handle);
    int rc = select(ctx, err, cap);
    if (rc) return rc;
    KernelSpec spec;
    rc = parse_checked(spec_json, len, spec, err, cap);
    if (rc) return rc;
    std::string error;
    if (!jade::hip_supported(spec, error)) return fail(1, err, cap, "%s", error.c_str());
    const std::string canonical = jade::canonical_json(spec);
    auto hit = ctx->cache.find(canonical);
    if (hit != ctx->cache.end()) {
        hit->second->refs += 1;
        *kernel = hit->second;
        return 0;
    }
    auto *p = new (std::nothrow) Pipeline;
    if (!p) return fail(3, err, cap, "pipeline allocation failed");
    p->owner = ctx;
    p->spec = spec;
    p->canonical = canonical;
    p->binds = jade::bindings(spec);
    if (spec.op == Op::Elementwise) {
        const auto code = jade::compile_expression(*spec.expression);
        p->copy = code.size() == 1 && code[0].op == uint32_t(jade::Opcode::Input) && code[0].arg == 0;
        p->program_len = uint32_t(code.size());
        auto status = hipMalloc(&p->program, code.size() * sizeof(jade::Instr));
        if (status == hipSuccess)
            status = hipMemcpyAsync(p->program, code.data(), code.size() * sizeof(jade::Instr), hipMemcpyHostToDevice,
                                    ctx->stream);
        const auto sync = hipStreamSynchronize(ctx->stream);
        if (status != hipSuccess || sync != hipSuccess) {
            if (p->program) (void)hipFree(p->program);
            delete p;
            return hip_fail(status != hipSuccess ? status : sync, err, cap, "upload expression program");
        }
    }
    const size_t workspace_bytes = workspace_bytes_for(spec);
    if (workspace_bytes) {
        const auto status = hipMalloc(&p->workspace, workspace_bytes);
        if (status != hipSuccess) {
            p->workspace = nullptr;
            delete p;
            return fail(status == hipErrorOutOfMemory ? 3 : 2, err, cap, "kernel workspace (%zu bytes): %s",
                        workspace_bytes, hipGetErrorString(status));
        }
    }
    p->refs = 1;
    ctx->cache.emplace(canonical, p);
    ctx->pipelines.insert(p);
    *kernel = p;
    return 0;
}

extern "C" void jr_kernel_release(void *handle, void *kernel) {
    Context *ctx = lookup(handle);
    if (!ctx || !kernel) return;
    auto *p = static_cast<Pipeline *>(kernel);
    if (!ctx->pipelines.count(p)) return;
    if (--p->refs > 0) return;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    release_pipeline(ctx, p);
}

extern "C" int jr_kernel_describe(void *handle, void *kernel, char *out, size_t out_cap, char *err, size_t cap) {
    clear(err, cap);
    if (out && out_cap) out[0] = '\0';
    if (!out || !out_cap) return fail(1, err, cap, "missing description output");
    Context *ctx = lookup(handle);
    if (!ctx) return fail(1, err, cap, "null or unknown runtime context");
    auto *p = static_cast<Pipeline *>(kernel);
    if (!kernel || !ctx->pipelines.count(p)) return fail(1, err, cap, "kernel belongs to another runtime/device context");
    return write_text(describe(p->spec), out, out_cap, err, cap);
}

// Two consecutive jobs run as one paired GEMM launch when both are GEMMs of
// the same shape whose plan pairs, and neither touches the other's output:
// job y must not read or write x's C (read-after-write, write-after-write) and
// x must not read y's C (write-after-read). Each output is then bit-identical
// to ordered launches.
static bool pairable(const jr_dispatch &x, const jr_dispatch &y) {
    const KernelSpec &a = static_cast<Pipeline *>(x.kernel)->spec;
    const KernelSpec &b = static_cast<Pipeline *>(y.kernel)->spec;
    auto gemm = [](const KernelSpec &s) { return s.op == Op::Gemm || s.op == Op::GemmSimd; };
    if (!gemm(a) || !gemm(b) || a.m != b.m || a.n != b.n || a.k != b.k) return false;
    if (x.buffer_count != 3 || y.buffer_count != 3) return false;
    if (!jade::hipk::gemm_f32_pairable(a.m, a.n, a.k)) return false;
    for (int i = 0; i < 3; ++i)
        if (y.buffers[i] == x.buffers[2] || x.buffers[i] == y.buffers[2]) return false;
    return true;
}

// Three consecutive jobs run as one fused launch when they are the residual
// MLP's gate and up projections and their SwiGLU (src/runtime/workloads.rs:
// 440-465): two pairable GEMMs on the same A, then swi_glu(x's C, y's C -> D)
// over m*n elements, with D none of the GEMMs' inputs, a shape whose plan is
// whole 128x64 tiles and 16-byte aligned inputs. The three outputs are
// bit-identical to the ordered launches (gemm_f32_dual_swiglu).
static bool fusable_gate_up_swiglu(const jr_dispatch &x, const jr_dispatch &y, const jr_dispatch &z) {
    if (!pairable(x, y) || z.buffer_count != 3) return false;
    const KernelSpec &g = static_cast<Pipeline *>(x.kernel)->spec;
    const KernelSpec &f = static_cast<Pipeline *>(z.kernel)->spec;
    if (f.op != Op::SwiGlu || uint64_t(f.len) != uint64_t(g.m) * g.n) return false;
    if (x.buffers[0] != y.buffers[0] || z.buffers[0] != x.buffers[2] || z.buffers[1] != y.buffers[2]) return false;
    void *const d = z.buffers[2];
    if (d == x.buffers[0] || d == x.buffers[1] || d == y.buffers[1]) return false;
    const uintptr_t bits = reinterpret_cast<uintptr_t>(x.buffers[0]) | reinterpret_cast<uintptr_t>(x.buffers[1]) |
                           reinterpret_cast<uintptr_t>(y.buffers[1]);
    return (bits & 15u) == 0 && jade::hipk::gemm_f32_dual_swiglu_fits(g.m, g.n, g.k);
}

extern "C" int jr_execute_dispatches(void *handle, const jr_dispatch *jobs, size_t job_count, uint32_t repeats,
                                     double *gpu_ms, char *err, size_t cap) {
    clear(err, cap);
    if (gpu_ms) *gpu_ms = 0;
    if (!jobs || !job_count || !repeats || !gpu_ms)
        return fail(1, err, cap, "execution requires jobs, positive repeats and a timing output");
    Context *ctx = lookup(handle);
    if (!ctx) return fail(1, err, cap, "null or unknown runtime context");
    // Whole-batch validation before any submission (corex.rs:556-569).
    std::vector<uint64_t> lengths, ids;
    for (size_t j = 0; j < job_count; ++j) {
        auto *p = static_cast<Pipeline *>(jobs[j].kernel);
        if (!p || !ctx->pipelines.count(p))
            return fail(1, err, cap, "job %zu: kernel belongs to another runtime/device context", j);
        if (!jobs[j].buffers && jobs[j].buffer_count) return fail(1, err, cap, "job %zu: null buffer array", j);
        lengths.assign(jobs[j].buffer_count, 0);
        ids.assign(jobs[j].buffer_count, 0);
        for (size_t b = 0; b < jobs[j].buffer_count; ++b) {
            auto it = ctx->allocations.find(jobs[j].buffers[b]);
            if (!jobs[j].buffers[b] || it == ctx->allocations.end())
                return fail(1, err, cap, "job %zu: buffer %zu belongs to another runtime/device context", j, b);
            if (it->second.bytes % sizeof(float))
                return fail(1, err, cap, "job %zu: buffer %zu is not a whole number of floats", j, b);
            lengths[b] = it->second.bytes / sizeof(float);
            ids[b] = it->second.id;
        }
        std::string error;
        if (!jade::validate_bindings(p->spec, lengths.data(), ids.data(), jobs[j].buffer_count, error))
            return fail(1, err, cap, "job %zu: %s", j, error.c_str());
    }
    const int rc = select(ctx, err, cap);
    if (rc) return rc;
    // The MLP's gate/up GEMMs and SwiGLU fuse into one launch
    // (fusable_gate_up_swiglu()); other adjacent independent GEMMs of one
    // shape share a launch (pairable()).
    std::vector<bool> paired(job_count, false), fused(job_count, false);
    for (size_t j = 0; j + 1 < job_count; ++j) {
        if (j + 2 < job_count && fusable_gate_up_swiglu(jobs[j], jobs[j + 1], jobs[j + 2])) {
            fused[j] = true;
            j += 2;
        } else if (pairable(jobs[j], jobs[j + 1])) {
            paired[j] = true;
            ++j;
        }
    }
    return timed_sequence(
        ctx, repeats, gpu_ms,
        [&]() -> hipError_t {
            for (size_t j = 0; j < job_count; ++j) {
                hipError_t status;
                if (fused[j]) {
                    const KernelSpec &s = static_cast<Pipeline *>(jobs[j].kernel)->spec;
                    void *const *x = jobs[j].buffers;
                    void *const *y = jobs[j + 1].buffers;
                    status = jade::hipk::gemm_f32_dual_swiglu(
                        ctx->stream, static_cast<const float *>(x[0]), static_cast<const float *>(x[1]),
                        static_cast<const float *>(y[1]), static_cast<float *>(x[2]), static_cast<float *>(y[2]),
                        static_cast<float *>(jobs[j + 2].buffers[2]), s.m, s.n, s.k);
                    j += 2;
                } else if (paired[j]) {
                    const KernelSpec &s = static_cast<Pipeline *>(jobs[j].kernel)->spec;
                    void *const *x = jobs[j].buffers;
                    void *const *y = jobs[j + 1].buffers;
                    status = jade::hipk::gemm_f32_pair(
                        ctx->stream, static_cast<const float *>(x[0]), static_cast<const float *>(x[1]),
                        static_cast<float *>(x[2]), static_cast<const float *>(y[0]), static_cast<const float *>(y[1]),
                        static_cast<float *>(y[2]), s.m, s.n, s.k);
                    ++j;
                } else {
                    status = launch(*static_cast<Pipeline *>(jobs[j].kernel), ctx->stream, jobs[j].buffers);
                }
                if (status != hipSuccess) return status;
            }
            return hipSuccess;
        },
        err, cap);
}
