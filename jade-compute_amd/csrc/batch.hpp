// Host-only part of jr_execute_dispatches (no HIP): the checks a batch passes
// before anything is enqueued, and the planner that turns adjacent jobs into
// paired or fused launches. runtime.cpp supplies the context (its pipelines
// and region table) and the GEMM planner's shape rules; the CPU tests build
// this unit with the spec parser under AddressSanitizer and UBSan and drive it
// with fake contexts (tests/sanitize/).
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

#include "jade_runtime_hip.h"
#include "spec.hpp"

namespace jade {
namespace batch {

// What a batch needs to know about the context that runs it.
class Context {
public:
    // The spec of a kernel handle compiled by this context, else nullptr.
    virtual const KernelSpec *kernel(const void *handle) const = 0;
    // Size in bytes and serial number of a live region of this context;
    // false when `ptr` is not one.
    virtual bool region(const void *ptr, size_t &bytes, uint64_t &serial) const = 0;

protected:
    ~Context() = default;
};

// The GEMM planner's rules that decide whether adjacent jobs may share a
// launch (gemm_f32_pairable, gemm_f32_dual_swiglu_fits,
// gemm_f32_residual_fits in kernels.hpp).
struct LaunchRules {
    bool (*pairable)(uint32_t m, uint32_t n, uint32_t k);
    bool (*dual_swiglu_fits)(uint32_t m, uint32_t n, uint32_t k);
    bool (*residual_fits)(uint32_t m, uint32_t n, uint32_t k);
};

// One launch of the batch: job `first` alone, or it and the one or two jobs
// after it as one paired or fused launch.
struct Step {
    enum class Form { Single, Pair, GateUpSwiglu, GemmResidual } form;
    size_t first;
};

// The arguments every batch entry point checks first (throws Refusal).
void check_batch(const void *jobs, size_t job_count, uint32_t repeats, const double *gpu_ms);

// Every job of the batch, before anything is enqueued (corex.rs:556-569):
// a kernel compiled by this context, a buffer list when it binds buffers,
// live regions of whole f32 elements, the spec's binding count and exact
// lengths, no write aliasing. Throws Refusal (Kind::Invalid) naming the job.
void validate(const jr_dispatch *jobs, size_t job_count, const Context &context);

// The launches of a validated batch, in order.
std::vector<Step> plan_steps(const jr_dispatch *jobs, size_t job_count, const Context &context,
                             const LaunchRules &rules);

}  // namespace batch
}  // namespace jade
