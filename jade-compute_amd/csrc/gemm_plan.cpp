// The per-shape GEMM-plan C ABI (names, signatures and codes of
// native/jade_corex.h:11-29), written as a client of this library's own jr_*
// runtime rather than as a second device layer. A plan is:
//   - one runtime context (jr_create),
//   - three regions A [m,k], B [k,n], C [m,n] (jr_alloc),
//   - one compiled `gemm` pipeline (jr_compile of the KernelSpec
//     {"op":"gemm","m":m,"n":n,"k":k,"tiled":true}, so the IR's shape rules
//     and its 31-bit element bound per matrix apply unchanged),
// and run() is one jr_execute_dispatches batch of that single job replayed
// `iterations` times. The product is this library's FP32 MFMA kernel.
//
// Codes: 1 invalid input or order of calls, 2 device, 4 allocation. Code 3
// (a BLAS failure in the reference) cannot occur: no BLAS is called.
#include <memory>
#include <string>

#include "jade_gemm_hip.h"
#include "jade_runtime_hip.h"
#include "session.hpp"

namespace {

using jade::dev::Kind;
using jade::dev::refuse;
using jade::dev::refuse_invalid;
using jade::dev::text_of;

int plan_code(Kind kind) {
    switch (kind) {
        case Kind::Invalid: return 1;
        case Kind::Device: return 2;
        case Kind::Memory: return 4;
    }
    return 2;
}

template <class Body>
int entry(char *err, size_t cap, Body &&body) {
    return jade::dev::abi_entry(err, cap, plan_code, body);
}

// Rethrows a failed jr_* call (codes 1/2/3) as this ABI's refusal, keeping
// the runtime's message.
void forward(int jr_status, const char *why) {
    if (jr_status == 0) return;
    const Kind kind = jr_status == 1 ? Kind::Invalid : jr_status == 3 ? Kind::Memory : Kind::Device;
    refuse(kind, why);
}

struct GemmPlan {
    uint32_t m = 0, n = 0, k = 0;
    void *runtime = nullptr;
    void *kernel = nullptr;
    void *a = nullptr, *b = nullptr, *c = nullptr;
    // What the device regions hold: nothing usable, the operands of the last
    // successful upload, or those operands and their product.
    enum class Holds { Nothing, Operands, Product } holds = Holds::Nothing;

    size_t a_len() const { return size_t(m) * k; }
    size_t b_len() const { return size_t(k) * n; }
    size_t c_len() const { return size_t(m) * n; }

    ~GemmPlan() {
        if (!runtime) return;
        jr_kernel_release(runtime, kernel);
        jr_destroy(runtime);  // frees A, B and C with the context
    }
};

jade::dev::HandleSet<GemmPlan> g_plans;

GemmPlan &plan_of(void *handle) {
    GemmPlan *p = g_plans.find(handle);
    if (!p) refuse_invalid("unknown GEMM plan handle (null, destroyed, or not from jade_corex_create)");
    return *p;
}

}  // namespace

extern "C" uint32_t jade_corex_abi_version(void) { return 1; }

extern "C" int jade_corex_create(uint32_t m, uint32_t n, uint32_t k, int device, uint32_t precision, void **out,
                                 char *err, size_t cap) {
    if (out) *out = nullptr;
    return entry(err, cap, [&] {
        if (!out) refuse_invalid("jade_corex_create needs somewhere to return the plan");
        if (precision == 1)
            refuse_invalid("precision 1 (FP16 operands) is not offered by the HIP backend; use precision 0 (FP32)");
        if (precision != 0) refuse_invalid(text_of("unknown precision %u (0 = FP32)", precision));
        if (!m || !n || !k) refuse_invalid(text_of("GEMM plan %ux%ux%u has an empty dimension", m, n, k));
        char why[512];
        std::unique_ptr<GemmPlan> p(new GemmPlan);
        p->m = m;
        p->n = n;
        p->k = k;
        forward(jr_create(device, &p->runtime, why, sizeof why), why);
        const std::string spec = text_of("{\"op\":\"gemm\",\"m\":%u,\"n\":%u,\"k\":%u,\"tiled\":true}", m, n, k);
        forward(jr_compile(p->runtime, spec.data(), spec.size(), &p->kernel, why, sizeof why), why);
        forward(jr_alloc(p->runtime, p->a_len() * sizeof(float), &p->a, why, sizeof why), why);
        forward(jr_alloc(p->runtime, p->b_len() * sizeof(float), &p->b, why, sizeof why), why);
        forward(jr_alloc(p->runtime, p->c_len() * sizeof(float), &p->c, why, sizeof why), why);
        g_plans.add(p.get());
        *out = p.release();
    });
}

extern "C" int jade_corex_upload(void *handle, const float *a, size_t a_len, const float *b, size_t b_len, char *err,
                                 size_t cap) {
    return entry(err, cap, [&] {
        GemmPlan &p = plan_of(handle);
        if (!a || !b) refuse_invalid("upload needs both host operands");
        if (a_len != p.a_len() || b_len != p.b_len())
            refuse_invalid(text_of("upload of a %ux%ux%u plan takes exactly %zu A and %zu B elements (got %zu, %zu)",
                                   p.m, p.n, p.k, p.a_len(), p.b_len(), a_len, b_len));
        p.holds = GemmPlan::Holds::Nothing;
        char why[512];
        forward(jr_upload(p.runtime, p.a, a, a_len * sizeof(float), why, sizeof why), why);
        forward(jr_upload(p.runtime, p.b, b, b_len * sizeof(float), why, sizeof why), why);
        p.holds = GemmPlan::Holds::Operands;
    });
}

extern "C" int jade_corex_run(void *handle, uint32_t iterations, double *elapsed_ms, char *err, size_t cap) {
    if (elapsed_ms) *elapsed_ms = 0;
    return entry(err, cap, [&] {
        GemmPlan &p = plan_of(handle);
        if (!iterations) refuse_invalid("run needs at least one iteration");
        if (!elapsed_ms) refuse_invalid("run needs somewhere to write the elapsed milliseconds");
        if (p.holds == GemmPlan::Holds::Nothing) refuse_invalid("nothing to multiply: upload A and B first");
        void *buffers[3] = {p.a, p.b, p.c};
        const jr_dispatch job{p.kernel, buffers, 3};
        p.holds = GemmPlan::Holds::Operands;  // C is undefined until this run succeeds
        char why[512];
        forward(jr_execute_dispatches(p.runtime, &job, 1, iterations, elapsed_ms, why, sizeof why), why);
        p.holds = GemmPlan::Holds::Product;
    });
}

extern "C" int jade_corex_download(void *handle, float *out, size_t out_len, char *err, size_t cap) {
    return entry(err, cap, [&] {
        GemmPlan &p = plan_of(handle);
        if (!out) refuse_invalid("download needs a host destination");
        if (out_len != p.c_len())
            refuse_invalid(text_of("C of a %ux%ux%u plan holds %zu elements, not %zu", p.m, p.n, p.k, p.c_len(),
                                   out_len));
        if (p.holds != GemmPlan::Holds::Product) refuse_invalid("no product yet: a run must succeed before download");
        char why[512];
        forward(jr_download(p.runtime, p.c, out, out_len * sizeof(float), why, sizeof why), why);
    });
}

extern "C" int jade_corex_device_info(void *handle, char *out, size_t out_cap, char *err, size_t cap) {
    if (out && out_cap) out[0] = '\0';
    return entry(err, cap, [&] {
        GemmPlan &p = plan_of(handle);
        if (!out || !out_cap) refuse_invalid("device info needs an output buffer");
        char device[768];
        char why[512];
        forward(jr_info(p.runtime, device, sizeof device, why, sizeof why), why);
        const std::string text =
            text_of("%s gemm=jade_mfma_f32 precision=fp32 plan=%ux%ux%u", device, p.m, p.n, p.k);
        if (text.size() + 1 > out_cap)
            refuse_invalid(text_of("output buffer holds %zu bytes; the device info needs %zu", out_cap,
                                   text.size() + 1));
        jade::dev::copy_text(text, out, out_cap);
    });
}

extern "C" void jade_corex_destroy(void *handle) {
    GemmPlan *p = g_plans.find(handle);
    if (p && g_plans.remove(p)) delete p;
}
