// Compiled pipelines: a checked KernelSpec bound to one precompiled gfx950
// kernel, plus the device memory that kernel needs besides its bindings (an
// Elementwise program, split-K / split-key partials). This replaces the
// reference's run-time compilation of emitted modules
// (src/runtime/corex.rs:439-542); identical canonical specs share one cached
// pipeline, as the reference shares modules by source text (corex.rs:442-460).
#pragma once

#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "kernels.hpp"
#include "session.hpp"
#include "spec.hpp"

namespace jade {

struct Pipeline {
    KernelSpec spec;
    std::string canonical;
    std::vector<Binding> binds;
    Instr *program = nullptr;    // device copy of an Elementwise program
    uint32_t program_len = 0;
    bool copy = false;           // Elementwise whose expression is input0
    float *workspace = nullptr;  // split-K / split-key partials of a small grid
    size_t workspace_bytes = 0;
    int holders = 0;
};

// Parses and validates (HIP rules) a KernelSpec document; Kind::Invalid with
// the reference's validation text otherwise.
KernelSpec read_spec(const char *json, size_t len);

// JSON description: name, canonical spec, bindings, whether the reference's
// rules accept it, whether this backend runs it, launch shape and workspace.
std::string describe_spec(const KernelSpec &spec);

// Device workspace the spec's kernel needs (0 for most).
size_t workspace_bytes_of(const KernelSpec &spec);

// Launches one pipeline over device buffers in binding order.
hipError_t enqueue(const Pipeline &p, hipStream_t queue, void *const *buffers);

// The pipelines of one session, shared by canonical spec and counted.
class PipelineCache {
public:
    explicit PipelineCache(dev::Session &session) : session_(session) {}
    ~PipelineCache();
    PipelineCache(const PipelineCache &) = delete;
    PipelineCache &operator=(const PipelineCache &) = delete;

    // A pipeline for `spec` (built on first use, shared afterwards).
    Pipeline *obtain(const KernelSpec &spec);
    // Drops one holder; the last one frees the pipeline's device memory.
    void drop(Pipeline *p);
    bool holds(const void *p) const { return all_.count(static_cast<Pipeline *>(const_cast<void *>(p))) != 0; }

private:
    void destroy(Pipeline *p);

    dev::Session &session_;
    std::unordered_map<std::string, Pipeline *> by_spec_;
    std::unordered_set<Pipeline *> all_;
};

}  // namespace jade
