// The jr_* C ABI of libjade_runtime_hip.so (ABI 2: the reference's
// native/jade_runtime_corex.h:9-31 entry points plus precompiled kernels from
// a KernelSpec). Each handle is a RuntimeContext: one dev::Session (device,
// queue, event clock, region table) and the session's pipeline cache. Every
// entry point is a short body run under dev::abi_entry, which maps the
// failure kinds onto this ABI's codes: 1 invalid, 2 device, 3 memory.
//
// The Rust CoreX backend made its ownership, exact-length and alias checks
// before calling into C (src/runtime/corex.rs:322-332, 389-394, 556-569); here
// the C layer makes them itself, from the session's region table, for every
// caller.
#include <hip/hip_runtime.h>

#include <memory>
#include <string>
#include <vector>

#include "batch.hpp"
#include "jade_runtime_hip.h"
#include "kernels.hpp"
#include "pipeline.hpp"
#include "session.hpp"
#include "spec.hpp"

namespace {

using jade::KernelSpec;
using jade::Op;
using jade::Pipeline;
using jade::dev::Kind;
using jade::dev::refuse_invalid;
using jade::dev::text_of;

int jr_code(Kind kind) {
    switch (kind) {
        case Kind::Invalid: return 1;
        case Kind::Device: return 2;
        case Kind::Memory: return 3;
    }
    return 2;
}

template <class Body>
int entry(char *err, size_t cap, Body &&body) {
    return jade::dev::abi_entry(err, cap, jr_code, body);
}

struct RuntimeContext {
    explicit RuntimeContext(int ordinal) : session(ordinal), pipelines(session) {}
    jade::dev::Session session;       // destroyed last: frees the regions and the queue
    jade::PipelineCache pipelines;    // destroyed first: frees programs and workspaces
};

jade::dev::HandleSet<RuntimeContext> g_contexts;

RuntimeContext &context_of(void *handle) {
    RuntimeContext *c = g_contexts.find(handle);
    if (!c) refuse_invalid("unknown runtime context handle (null, destroyed, or not from jr_create)");
    return *c;
}

Pipeline &pipeline_of(RuntimeContext &c, void *kernel, const char *where) {
    if (!kernel || !c.pipelines.holds(kernel))
        refuse_invalid(text_of("%s: the kernel handle was not compiled by this context", where));
    return *static_cast<Pipeline *>(kernel);
}

void emit(const std::string &text, char *out, size_t out_cap) {
    if (text.size() + 1 > out_cap)
        refuse_invalid(text_of("output buffer holds %zu bytes; the text needs %zu", out_cap, text.size() + 1));
    jade::dev::copy_text(text, out, out_cap);
}

// ---- batches: checks and planning in batch.cpp, launches here --------------

using jade::batch::Step;

// The context's pipelines and region table, as the batch unit sees them.
class BatchView final : public jade::batch::Context {
public:
    explicit BatchView(RuntimeContext &c) : c_(c) {}
    const KernelSpec *kernel(const void *handle) const override {
        void *h = const_cast<void *>(handle);
        return h && c_.pipelines.holds(h) ? &static_cast<Pipeline *>(h)->spec : nullptr;
    }
    bool region(const void *ptr, size_t &bytes, uint64_t &serial) const override {
        const auto *r = c_.session.region(ptr);
        if (!r) return false;
        bytes = r->bytes;
        serial = r->serial;
        return true;
    }

private:
    RuntimeContext &c_;
};

const jade::batch::LaunchRules kLaunchRules{jade::hipk::gemm_f32_pairable, jade::hipk::gemm_f32_dual_swiglu_fits,
                                            jade::hipk::gemm_f32_residual_fits};

const KernelSpec &spec_of(const jr_dispatch &d) { return static_cast<Pipeline *>(d.kernel)->spec; }

hipError_t run_step(const Step &step, const jr_dispatch *jobs, hipStream_t q) {
    const jr_dispatch &x = jobs[step.first];
    auto f = [](void *p) { return static_cast<float *>(p); };
    auto cf = [](void *p) { return static_cast<const float *>(p); };
    switch (step.form) {
        case Step::Form::Single: return jade::enqueue(*static_cast<Pipeline *>(x.kernel), q, x.buffers);
        case Step::Form::Pair: {
            const KernelSpec &s = spec_of(x);
            const jr_dispatch &y = jobs[step.first + 1];
            return jade::hipk::gemm_f32_pair(q, cf(x.buffers[0]), cf(x.buffers[1]), f(x.buffers[2]),
                                             cf(y.buffers[0]), cf(y.buffers[1]), f(y.buffers[2]), s.m, s.n, s.k);
        }
        case Step::Form::GateUpSwiglu: {
            const KernelSpec &s = spec_of(x);
            const jr_dispatch &y = jobs[step.first + 1];
            const jr_dispatch &z = jobs[step.first + 2];
            return jade::hipk::gemm_f32_dual_swiglu(q, cf(x.buffers[0]), cf(x.buffers[1]), cf(y.buffers[1]),
                                                    f(x.buffers[2]), f(y.buffers[2]), f(z.buffers[2]), s.m, s.n,
                                                    s.k);
        }
        case Step::Form::GemmResidual: {
            const KernelSpec &s = spec_of(x);
            const jr_dispatch &y = jobs[step.first + 1];
            void *const residual = y.buffers[0] == x.buffers[2] ? y.buffers[1] : y.buffers[0];
            return jade::hipk::gemm_f32_residual(q, cf(x.buffers[0]), cf(x.buffers[1]), f(x.buffers[2]),
                                                 cf(residual), f(y.buffers[2]), s.m, s.n, s.k);
        }
    }
    return hipErrorInvalidValue;
}

}  // namespace

extern "C" uint32_t jr_version(void) { return 2; }

extern "C" int jr_create(int device, void **out, char *err, size_t cap) {
    if (out) *out = nullptr;
    return entry(err, cap, [&] {
        if (!out) refuse_invalid("jr_create needs somewhere to return the handle");
        std::unique_ptr<RuntimeContext> c(new RuntimeContext(device));
        // The allocation-free GEMM's per-device scratch address, looked up
        // here (the context's device is current) rather than inside a call
        // that may run under stream capture.
        jade::hipk::noalloc_prepare(device);
        g_contexts.add(c.get());
        *out = c.release();
    });
}

extern "C" void jr_destroy(void *handle) {
    RuntimeContext *c = g_contexts.find(handle);
    if (!c || !g_contexts.remove(c)) return;
    (void)hipSetDevice(c->session.ordinal());
    delete c;
}

extern "C" int jr_info(void *handle, char *out, size_t out_cap, char *err, size_t cap) {
    if (out && out_cap) out[0] = '\0';
    return entry(err, cap, [&] {
        if (!out || !out_cap) refuse_invalid("jr_info needs an output buffer");
        emit(context_of(handle).session.device_summary(), out, out_cap);
    });
}

extern "C" int jr_alloc(void *handle, size_t bytes, void **out, char *err, size_t cap) {
    if (out) *out = nullptr;
    return entry(err, cap, [&] {
        if (!out) refuse_invalid("jr_alloc needs somewhere to return the pointer");
        RuntimeContext &c = context_of(handle);
        *out = c.session.allocate_zeroed(bytes);
    });
}

extern "C" void jr_free(void *handle, void *ptr) {
    RuntimeContext *c = g_contexts.find(handle);
    if (c && ptr) (void)c->session.give_back(ptr);
}

extern "C" int jr_upload(void *handle, void *device_ptr, const void *host_ptr, size_t bytes, char *err, size_t cap) {
    return entry(err, cap, [&] { context_of(handle).session.write_region(device_ptr, host_ptr, bytes); });
}

extern "C" int jr_download(void *handle, const void *device_ptr, void *host_ptr, size_t bytes, char *err,
                           size_t cap) {
    return entry(err, cap, [&] { context_of(handle).session.read_region(host_ptr, device_ptr, bytes); });
}

extern "C" int jr_buffer_elements(void *handle, const void *device_ptr, size_t *elements, char *err, size_t cap) {
    if (elements) *elements = 0;
    return entry(err, cap, [&] {
        if (!elements) refuse_invalid("jr_buffer_elements needs an output");
        const auto *r = context_of(handle).session.region(device_ptr);
        if (!r) refuse_invalid("the pointer is not a live region of this context");
        *elements = r->bytes / sizeof(float);
    });
}

extern "C" int jr_execute(void *handle, const jr_job *jobs, size_t job_count, uint32_t repeats, double *gpu_ms,
                          char *err, size_t cap) {
    if (gpu_ms) *gpu_ms = 0;
    return entry(err, cap, [&] {
        jade::batch::check_batch(jobs, job_count, repeats, gpu_ms);
        for (size_t j = 0; j < job_count; ++j) {
            if (!jobs[j].launch) refuse_invalid(text_of("job %zu has no launcher", j));
            if (!jobs[j].buffers || !jobs[j].buffer_count) refuse_invalid(text_of("job %zu binds no buffers", j));
            for (size_t b = 0; b < jobs[j].buffer_count; ++b)
                if (!jobs[j].buffers[b]) refuse_invalid(text_of("job %zu: buffer %zu is null", j, b));
        }
        RuntimeContext &c = context_of(handle);
        c.session.make_current();
        *gpu_ms = c.session.clocked(repeats, [&](hipStream_t q) -> hipError_t {
            for (size_t j = 0; j < job_count; ++j) {
                const int status = jobs[j].launch(static_cast<void *>(q), jobs[j].buffers);
                if (status) return static_cast<hipError_t>(status);
            }
            return hipSuccess;
        });
    });
}

extern "C" int jr_spec_describe(const char *spec_json, size_t len, char *out, size_t out_cap, char *err,
                                size_t cap) {
    if (out && out_cap) out[0] = '\0';
    return entry(err, cap, [&] {
        if (!out || !out_cap) refuse_invalid("jr_spec_describe needs an output buffer");
        emit(jade::describe_spec(jade::read_spec(spec_json, len)), out, out_cap);
    });
}

extern "C" int jr_spec_validate_bindings(const char *spec_json, size_t len, const uint64_t *lengths,
                                         const uint64_t *ids, size_t count, char *err, size_t cap) {
    return entry(err, cap, [&] {
        if ((!lengths || !ids) && count) refuse_invalid("binding lengths and identities are missing");
        const KernelSpec spec = jade::read_spec(spec_json, len);
        std::string error;
        if (!jade::validate_bindings(spec, lengths, ids, count, error)) refuse_invalid(error);
    });
}

extern "C" int jr_compile(void *handle, const char *spec_json, size_t len, void **kernel, char *err, size_t cap) {
    if (kernel) *kernel = nullptr;
    return entry(err, cap, [&] {
        if (!kernel) refuse_invalid("jr_compile needs somewhere to return the kernel");
        RuntimeContext &c = context_of(handle);
        const KernelSpec spec = jade::read_spec(spec_json, len);
        *kernel = c.pipelines.obtain(spec);
    });
}

extern "C" void jr_kernel_release(void *handle, void *kernel) {
    RuntimeContext *c = g_contexts.find(handle);
    if (c && kernel) c->pipelines.drop(static_cast<Pipeline *>(kernel));
}

extern "C" int jr_kernel_describe(void *handle, void *kernel, char *out, size_t out_cap, char *err, size_t cap) {
    if (out && out_cap) out[0] = '\0';
    return entry(err, cap, [&] {
        if (!out || !out_cap) refuse_invalid("jr_kernel_describe needs an output buffer");
        RuntimeContext &c = context_of(handle);
        emit(jade::describe_spec(pipeline_of(c, kernel, "jr_kernel_describe").spec), out, out_cap);
    });
}

extern "C" int jr_execute_dispatches(void *handle, const jr_dispatch *jobs, size_t job_count, uint32_t repeats,
                                     double *gpu_ms, char *err, size_t cap) {
    if (gpu_ms) *gpu_ms = 0;
    return entry(err, cap, [&] {
        jade::batch::check_batch(jobs, job_count, repeats, gpu_ms);
        RuntimeContext &c = context_of(handle);
        const BatchView view(c);
        // The whole batch is checked before anything is enqueued.
        jade::batch::validate(jobs, job_count, view);
        const std::vector<Step> steps = jade::batch::plan_steps(jobs, job_count, view, kLaunchRules);
        c.session.make_current();
        *gpu_ms = c.session.clocked(repeats, [&](hipStream_t q) -> hipError_t {
            for (const Step &s : steps) {
                const hipError_t status = run_step(s, jobs, q);
                if (status != hipSuccess) return status;
            }
            return hipSuccess;
        });
    });
}

extern "C" int jr_plan_dispatches(void *handle, const jr_dispatch *jobs, size_t job_count, char *out, size_t out_cap,
                                  char *err, size_t cap) {
    if (out && out_cap) out[0] = '\0';
    return entry(err, cap, [&] {
        if (!out || !out_cap) refuse_invalid("jr_plan_dispatches needs an output buffer");
        double unused = 0;
        jade::batch::check_batch(jobs, job_count, 1, &unused);
        RuntimeContext &c = context_of(handle);
        const BatchView view(c);
        jade::batch::validate(jobs, job_count, view);
        std::string text;
        for (const Step &s : jade::batch::plan_steps(jobs, job_count, view, kLaunchRules)) {
            static const char *const forms[] = {"single", "pair", "gate_up_swiglu", "gemm_residual"};
            text += text_of("%s%s:%zu", text.empty() ? "" : " ", forms[int(s.form)], s.first);
        }
        emit(text, out, out_cap);
    });
}
