// Host-only part of jr_execute_dispatches: see batch.hpp.
#include "batch.hpp"

#include <string>

#include "refusal.hpp"

namespace jade {
namespace batch {
namespace {

using dev::refuse_invalid;
using dev::text_of;

const KernelSpec &spec_of(const jr_dispatch &d, const Context &context) {
    const KernelSpec *s = context.kernel(d.kernel);
    if (!s) refuse_invalid("the batch was planned before it was validated");
    return *s;
}

bool is_gemm(const KernelSpec &s) { return s.op == Op::Gemm || s.op == Op::GemmSimd; }

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Two consecutive jobs run as one paired GEMM launch when both are GEMMs of
// the same shape whose plan pairs, and neither touches the other's output:
// job y must not read or write x's C (read-after-write, write-after-write) and
// x must not read y's C (write-after-read). Each output is then bit-identical
// to ordered launches.
bool pairable(const jr_dispatch &x, const jr_dispatch &y, const Context &context, const LaunchRules &rules) {
    const KernelSpec &a = spec_of(x, context), &b = spec_of(y, context);
    if (!is_gemm(a) || !is_gemm(b) || a.m != b.m || a.n != b.n || a.k != b.k) return false;
    if (x.buffer_count != 3 || y.buffer_count != 3) return false;
    if (!rules.pairable(a.m, a.n, a.k)) return false;
    for (int i = 0; i < 3; ++i)
        if (y.buffers[i] == x.buffers[2] || x.buffers[i] == y.buffers[2]) return false;
    return true;
}

// Three consecutive jobs run as one fused launch when they are the residual
// MLP's gate and up projections and their SwiGLU (src/runtime/workloads.rs:
// 440-465): two GEMMs of one shape on the same A that could share a launch,
// then swi_glu(x's C, y's C -> D) over m*n elements, with D none of the GEMMs'
// inputs, a shape the fused kernel takes and 16-byte aligned inputs. The
// three outputs are bit-identical to the ordered launches
// (gemm_f32_dual_swiglu).
bool fusable_gate_up_swiglu(const jr_dispatch &x, const jr_dispatch &y, const jr_dispatch &z,
                            const Context &context, const LaunchRules &rules) {
    const KernelSpec &g = spec_of(x, context), &h = spec_of(y, context), &f = spec_of(z, context);
    if (!is_gemm(g) || !is_gemm(h) || g.m != h.m || g.n != h.n || g.k != h.k) return false;
    if (x.buffer_count != 3 || y.buffer_count != 3 || z.buffer_count != 3) return false;
    for (int i = 0; i < 3; ++i)
        if (y.buffers[i] == x.buffers[2] || x.buffers[i] == y.buffers[2]) return false;
    if (f.op != Op::SwiGlu || uint64_t(f.len) != uint64_t(g.m) * g.n) return false;
    if (x.buffers[0] != y.buffers[0] || z.buffers[0] != x.buffers[2] || z.buffers[1] != y.buffers[2]) return false;
    void *const d = z.buffers[2];
    if (d == x.buffers[0] || d == x.buffers[1] || d == y.buffers[1]) return false;
    return aligned16(x.buffers[0]) && aligned16(x.buffers[1]) && aligned16(y.buffers[1]) &&
           rules.dual_swiglu_fits(g.m, g.n, g.k);
}

// A GEMM and the Add that follows it run as one launch when the GEMM's output
// P is one operand of the Add (add(P, X -> O) or add(X, P -> O) over m*n
// elements), X is not P, and O is neither of the GEMM's inputs (the epilogue
// writes O while other workgroups still read them): the residual MLP's down
// projection and residual add (src/runtime/workloads.rs:440-465). P and O are
// bit-identical to the ordered launches (gemm_f32_residual).
bool fusable_gemm_residual(const jr_dispatch &x, const jr_dispatch &y, const Context &context,
                           const LaunchRules &rules) {
    const KernelSpec &g = spec_of(x, context), &a = spec_of(y, context);
    if (!is_gemm(g) || a.op != Op::Add || x.buffer_count != 3 || y.buffer_count != 3) return false;
    if (uint64_t(a.len) != uint64_t(g.m) * g.n) return false;
    void *const p = x.buffers[2];
    if (y.buffers[0] != p && y.buffers[1] != p) return false;
    void *const residual = y.buffers[0] == p ? y.buffers[1] : y.buffers[0];
    void *const o = y.buffers[2];
    if (residual == p || o == x.buffers[0] || o == x.buffers[1]) return false;
    return aligned16(x.buffers[0]) && aligned16(x.buffers[1]) && rules.residual_fits(g.m, g.n, g.k);
}

}  // namespace

void check_batch(const void *jobs, size_t job_count, uint32_t repeats, const double *gpu_ms) {
    if (!jobs || !job_count) refuse_invalid("the batch holds no jobs");
    if (!repeats) refuse_invalid("repeats must be at least 1");
    if (!gpu_ms) refuse_invalid("no place to write the measured milliseconds");
}

void validate(const jr_dispatch *jobs, size_t job_count, const Context &context) {
    std::vector<uint64_t> lengths, ids;
    for (size_t j = 0; j < job_count; ++j) {
        const std::string where = text_of("job %zu", j);
        const KernelSpec *spec = context.kernel(jobs[j].kernel);
        if (!spec) refuse_invalid(where + ": the kernel handle was not compiled by this context");
        if (!jobs[j].buffers && jobs[j].buffer_count) refuse_invalid(where + ": null buffer list");
        lengths.assign(jobs[j].buffer_count, 0);
        ids.assign(jobs[j].buffer_count, 0);
        for (size_t b = 0; b < jobs[j].buffer_count; ++b) {
            size_t bytes = 0;
            uint64_t serial = 0;
            if (!context.region(jobs[j].buffers[b], bytes, serial))
                refuse_invalid(text_of("job %zu: buffer %zu is not a live region of this context", j, b));
            if (bytes % sizeof(float))
                refuse_invalid(text_of("job %zu: buffer %zu is not a whole number of f32 elements", j, b));
            lengths[b] = bytes / sizeof(float);
            ids[b] = serial;
        }
        std::string error;
        if (!validate_bindings(*spec, lengths.data(), ids.data(), jobs[j].buffer_count, error))
            refuse_invalid(where + ": " + error);
    }
}

std::vector<Step> plan_steps(const jr_dispatch *jobs, size_t job_count, const Context &context,
                             const LaunchRules &rules) {
    std::vector<Step> steps;
    for (size_t j = 0; j < job_count;) {
        if (j + 2 < job_count && fusable_gate_up_swiglu(jobs[j], jobs[j + 1], jobs[j + 2], context, rules)) {
            steps.push_back({Step::Form::GateUpSwiglu, j});
            j += 3;
        } else if (j + 1 < job_count && pairable(jobs[j], jobs[j + 1], context, rules)) {
            steps.push_back({Step::Form::Pair, j});
            j += 2;
        } else if (j + 1 < job_count && fusable_gemm_residual(jobs[j], jobs[j + 1], context, rules)) {
            steps.push_back({Step::Form::GemmResidual, j});
            j += 2;
        } else {
            steps.push_back({Step::Form::Single, j});
            j += 1;
        }
    }
    return steps;
}

}  // namespace batch
}  // namespace jade
