// Drives the host-only batch unit of libjade_runtime_hip.so (csrc/batch.cpp:
// the checks jr_execute_dispatches makes before it enqueues anything, and its
// launch planner) with fake contexts, for a build under AddressSanitizer and
// UBSan (tests/test_sanitize_batch.py). Buffer pointers are addresses that
// are never mapped, so a planner that dereferenced one would fault; buffer
// lists are heap arrays of exactly buffer_count entries, so a read past one
// is a reported overflow.
//
// Prints one line per case: "<case>: <plan>" with the plan as
// jr_plan_dispatches writes it, or "<case>: refused <message>". Exits 1 on a
// failed invariant.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <memory>
#include <random>
#include <string>
#include <vector>

#include "batch.hpp"
#include "refusal.hpp"
#include "spec.hpp"

using jade::KernelSpec;
using jade::batch::LaunchRules;
using jade::batch::Step;

namespace {

class Fake final : public jade::batch::Context {
public:
    // A kernel handle for the spec (handles are distinct, never-mapped
    // addresses in a high range).
    const void *kernel_for(const std::string &json) {
        KernelSpec spec;
        std::string error;
        if (!jade::parse_spec(json, spec, error)) {
            std::printf("bad spec %s: %s\n", json.c_str(), error.c_str());
            std::exit(1);
        }
        const void *h = reinterpret_cast<const void *>(uintptr_t(0x7e0000000000ull) + 0x1000 * kernels_.size());
        kernels_[h] = spec;
        return h;
    }
    // A region of `elements` floats (a 256-byte aligned, never-mapped address).
    void *buffer(uint64_t elements) {
        void *p = reinterpret_cast<void *>(uintptr_t(0x7f0000000000ull) + (uintptr_t(regions_.size()) << 32));
        regions_[p] = {elements * 4, uint64_t(regions_.size()) + 1};
        return p;
    }
    const KernelSpec *kernel(const void *handle) const override {
        auto it = kernels_.find(handle);
        return it == kernels_.end() ? nullptr : &it->second;
    }
    bool region(const void *ptr, size_t &bytes, uint64_t &serial) const override {
        auto it = regions_.find(ptr);
        if (it == regions_.end()) return false;
        bytes = it->second.first;
        serial = it->second.second;
        return true;
    }

private:
    std::map<const void *, KernelSpec> kernels_;
    std::map<const void *, std::pair<size_t, uint64_t>> regions_;
};

// A batch whose buffer lists are separate heap arrays of exactly
// buffer_count pointers.
struct Batch {
    std::vector<std::unique_ptr<void *[]>> lists;
    std::vector<jr_dispatch> jobs;
    void add(const void *kernel, std::vector<void *> buffers) {
        std::unique_ptr<void *[]> list;
        if (!buffers.empty()) {
            list.reset(new void *[buffers.size()]);
            for (size_t i = 0; i < buffers.size(); ++i) list[i] = buffers[i];
        }
        jobs.push_back({const_cast<void *>(kernel), list.get(), buffers.size()});
        lists.push_back(std::move(list));
    }
};

bool yes(uint32_t, uint32_t, uint32_t) { return true; }
bool no(uint32_t, uint32_t, uint32_t) { return false; }
const LaunchRules kAll{yes, yes, yes}, kNone{no, no, no}, kPairOnly{yes, no, no}, kFuseOnly{no, yes, yes};

std::string text(const std::vector<Step> &steps) {
    static const char *const forms[] = {"single", "pair", "gate_up_swiglu", "gemm_residual"};
    std::string out;
    for (const Step &s : steps)
        out += (out.empty() ? "" : " ") + std::string(forms[int(s.form)]) + ":" + std::to_string(s.first);
    return out;
}

// Checks and plans a batch as jr_plan_dispatches does, printing the result.
std::string run(const char *name, const Fake &ctx, const Batch &b, const LaunchRules &rules, uint32_t repeats = 1,
                bool null_ms = false, bool null_jobs = false) {
    std::string line;
    try {
        double ms = 0;
        jade::batch::check_batch(null_jobs ? nullptr : b.jobs.data(), b.jobs.size(), repeats,
                                 null_ms ? nullptr : &ms);
        jade::batch::validate(b.jobs.data(), b.jobs.size(), ctx);
        line = text(jade::batch::plan_steps(b.jobs.data(), b.jobs.size(), ctx, rules));
    } catch (const jade::dev::Refusal &r) {
        line = "refused " + r.text;
    }
    std::printf("%s: %s\n", name, line.c_str());
    return line;
}

std::string gemm(int m, int n, int k) {
    return "{\"op\":\"gemm\",\"m\":" + std::to_string(m) + ",\"n\":" + std::to_string(n) + ",\"k\":" +
           std::to_string(k) + ",\"tiled\":true}";
}
std::string unary(const char *op, uint64_t len) { return std::string("{\"op\":\"") + op + "\",\"len\":" + std::to_string(len) + "}"; }

int failures = 0;
void expect(bool ok, const char *what) {
    if (!ok) {
        std::printf("invariant failed: %s\n", what);
        ++failures;
    }
}

}  // namespace

int main() {
    // The C4 block (src/runtime/workloads.rs:440-465): x[4096x1024] ->
    // RMSNorm -> gate/up GEMMs 1024->2816 -> SwiGLU -> down GEMM -> + x.
    const int batch = 4096, width = 1024, hidden = 2816;
    Fake ctx;
    const void *norm = ctx.kernel_for("{\"op\":\"rms_norm\",\"rows\":4096,\"cols\":1024,\"epsilon\":1e-6}");
    const void *up = ctx.kernel_for(gemm(batch, hidden, width));
    const void *down = ctx.kernel_for(gemm(batch, width, hidden));
    const void *act = ctx.kernel_for(unary("swi_glu", uint64_t(batch) * hidden));
    const void *add = ctx.kernel_for(unary("add", uint64_t(batch) * width));
    void *x = ctx.buffer(uint64_t(batch) * width), *gamma = ctx.buffer(width);
    void *wg = ctx.buffer(uint64_t(width) * hidden), *wu = ctx.buffer(uint64_t(width) * hidden);
    void *wd = ctx.buffer(uint64_t(hidden) * width), *normalized = ctx.buffer(uint64_t(batch) * width);
    void *gate = ctx.buffer(uint64_t(batch) * hidden), *upv = ctx.buffer(uint64_t(batch) * hidden);
    void *a = ctx.buffer(uint64_t(batch) * hidden), *proj = ctx.buffer(uint64_t(batch) * width);
    void *out = ctx.buffer(uint64_t(batch) * width);
    Batch c4;
    c4.add(norm, {x, gamma, normalized});
    c4.add(up, {normalized, wg, gate});
    c4.add(up, {normalized, wu, upv});
    c4.add(act, {gate, upv, a});
    c4.add(down, {a, wd, proj});
    c4.add(add, {proj, x, out});
    expect(run("c4_all", ctx, c4, kAll) == "single:0 gate_up_swiglu:1 gemm_residual:4", "c4 fuses");
    expect(run("c4_none", ctx, c4, kNone) == "single:0 single:1 single:2 single:3 single:4 single:5", "c4 alone");
    expect(run("c4_pair_only", ctx, c4, kPairOnly) == "single:0 pair:1 single:3 single:4 single:5", "c4 pairs");
    expect(run("c4_fuse_only", ctx, c4, kFuseOnly) == "single:0 gate_up_swiglu:1 gemm_residual:4",
           "fusion does not need a paired plan");

    // Hazards (tests/test_gpu_mlp.py): the SwiGLU writes the gate weights;
    // the Add writes the GEMM's A; dependent GEMMs; one job twice.
    const void *sq = ctx.kernel_for(gemm(2048, 2048, 2048));
    const void *sq_act = ctx.kernel_for(unary("swi_glu", 2048u * 2048u));
    const void *sq_add = ctx.kernel_for(unary("add", 2048u * 2048u));
    void *p = ctx.buffer(2048u * 2048u), *q = ctx.buffer(2048u * 2048u), *r = ctx.buffer(2048u * 2048u);
    void *s = ctx.buffer(2048u * 2048u), *t = ctx.buffer(2048u * 2048u), *u = ctx.buffer(2048u * 2048u);
    Batch h1;
    h1.add(sq, {p, q, s});
    h1.add(sq, {p, r, t});
    h1.add(sq_act, {s, t, q});
    expect(run("swiglu_writes_gate_weights", ctx, h1, kAll) == "pair:0 single:2", "no fusion over a hazard");
    Batch h2;
    h2.add(sq, {p, q, s});
    h2.add(sq_add, {s, t, p});
    expect(run("add_writes_gemm_input", ctx, h2, kAll) == "single:0 single:1", "no residual fusion over a hazard");
    Batch h3;
    h3.add(sq, {p, q, s});
    h3.add(sq, {s, q, t});
    expect(run("read_after_write", ctx, h3, kAll) == "single:0 single:1", "raw");
    Batch h4;
    h4.add(sq, {u, q, s});
    h4.add(sq, {p, q, u});
    expect(run("write_after_read", ctx, h4, kAll) == "single:0 single:1", "war");
    Batch h5;
    h5.add(sq, {p, q, s});
    h5.add(sq, {p, q, s});
    expect(run("one_job_twice", ctx, h5, kAll) == "single:0 single:1", "waw");
    Batch h6;
    h6.add(sq, {p, q, s});
    h6.add(sq_add, {s, s, t});
    expect(run("residual_is_the_product", ctx, h6, kAll) == "single:0 single:1", "add(P, P)");

    // Malformed batches: each refused before any planning.
    const void *copy = ctx.kernel_for("{\"op\":\"elementwise\",\"len\":4194304,\"inputs\":1,"
                                      "\"expression\":{\"kind\":\"input\",\"binding\":0}}");
    Batch m1;
    m1.add(sq, {p, q});
    expect(run("short_buffer_list", ctx, m1, kAll).rfind("refused", 0) == 0, "short list");
    Batch m2;
    m2.add(sq, {p, nullptr, s});
    expect(run("null_buffer", ctx, m2, kAll).rfind("refused", 0) == 0, "null buffer");
    Batch m3;
    m3.jobs.push_back({const_cast<void *>(sq), nullptr, 3});
    expect(run("null_buffer_list", ctx, m3, kAll).rfind("refused", 0) == 0, "null list");
    Batch m4;
    m4.add(reinterpret_cast<const void *>(uintptr_t(0x12345000)), {p, q, s});
    expect(run("foreign_kernel", ctx, m4, kAll).rfind("refused", 0) == 0, "foreign kernel");
    Batch m5;
    m5.add(sq, {p, q, reinterpret_cast<void *>(uintptr_t(0x5000))});
    expect(run("foreign_buffer", ctx, m5, kAll).rfind("refused", 0) == 0, "foreign buffer");
    Batch m6;
    m6.add(sq, {p, q, gamma});
    expect(run("wrong_length", ctx, m6, kAll).rfind("refused", 0) == 0, "length");
    Batch m7;
    m7.add(sq, {p, q, p});
    expect(run("output_aliases_input", ctx, m7, kAll).rfind("refused", 0) == 0, "write alias");
    Batch m8;
    m8.add(sq, {p, q, s});
    m8.add(copy, {s, t});
    m8.add(sq, {p, q, s, t});
    expect(run("bad_later_job", ctx, m8, kAll).rfind("refused job 2", 0) == 0, "later job named");
    Batch m9;
    expect(run("empty_batch", ctx, m9, kAll).rfind("refused", 0) == 0, "empty");
    Batch m10;
    m10.add(sq, {p, q, s});
    expect(run("zero_repeats", ctx, m10, kAll, 0).rfind("refused", 0) == 0, "repeats");
    expect(run("no_time_output", ctx, m10, kAll, 1, true).rfind("refused", 0) == 0, "gpu_ms");
    expect(run("null_jobs", ctx, m10, kAll, 1, false, true).rfind("refused", 0) == 0, "jobs");
    Batch m11;
    m11.add(copy, {s, t});
    m11.add(sq, {p, q, s});
    m11.add(sq_add, {s, t, u});
    expect(run("mixed_counts", ctx, m11, kAll) == "single:0 gemm_residual:1", "one-input job then fusion");

    // Seeded random batches over this pool of kernels and buffers: every
    // valid batch's plan covers each job once, in order, and each fused step
    // keeps the hazard rules.
    std::mt19937 rng(20261202);
    const void *kernels[] = {sq, sq_act, sq_add, copy};
    void *bufs[] = {p, q, r, s, t, u};
    const LaunchRules rules[] = {kAll, kNone, kPairOnly, kFuseOnly};
    int valid = 0, fused = 0;
    for (int trial = 0; trial < 20000; ++trial) {
        Batch b;
        const int jobs = 1 + int(rng() % 6);
        for (int j = 0; j < jobs; ++j) {
            const int which = int(rng() % 4);
            const size_t count = which == 3 ? 2 : 3;
            std::vector<void *> list;
            for (size_t i = 0; i < count; ++i) list.push_back(bufs[rng() % 6]);
            b.add(kernels[which], list);
        }
        std::vector<Step> steps;
        try {
            jade::batch::validate(b.jobs.data(), b.jobs.size(), ctx);
            steps = jade::batch::plan_steps(b.jobs.data(), b.jobs.size(), ctx, rules[trial % 4]);
        } catch (const jade::dev::Refusal &) {
            continue;
        }
        ++valid;
        size_t next = 0;
        for (const Step &st : steps) {
            expect(st.first == next, "steps in order");
            const size_t span = st.form == Step::Form::Single ? 1 : st.form == Step::Form::GateUpSwiglu ? 3 : 2;
            if (span > 1) {
                ++fused;
                const jr_dispatch &x = b.jobs[st.first], &y = b.jobs[st.first + 1];
                // The later job never reads or writes the earlier one's output
                // before it is produced, except through the fused operand.
                if (st.form == Step::Form::Pair || st.form == Step::Form::GateUpSwiglu)
                    for (int i = 0; i < 3; ++i)
                        expect(y.buffers[i] != x.buffers[2] && x.buffers[i] != y.buffers[2], "pair hazard");
                if (st.form == Step::Form::GemmResidual)
                    expect(y.buffers[2] != x.buffers[0] && y.buffers[2] != x.buffers[1], "residual hazard");
            }
            next += span;
        }
        expect(next == b.jobs.size(), "every job planned once");
    }
    std::printf("random: %d valid batches, %d fused steps\n", valid, fused);
    expect(valid > 1000 && fused > 100, "random batches exercise the planner");
    std::printf("%s\n", failures ? "FAILED" : "ok");
    return failures ? 1 : 0;
}
