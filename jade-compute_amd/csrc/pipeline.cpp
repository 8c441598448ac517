// Compiled pipelines: see pipeline.hpp.
#include "pipeline.hpp"

#include <cstring>

namespace jade {

using dev::Kind;
using dev::refuse;
using dev::refuse_invalid;
using dev::text_of;

namespace {

hipk::LaunchShape launch_shape(const KernelSpec &s) {
    using namespace hipk;
    switch (s.op) {
        case Op::Elementwise: {
            const auto &e = *s.expression;
            if (e.kind == Expr::Kind::Input && e.binding == 0) {
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

std::string shape_json(const hipk::LaunchShape &shape) {
    return "{\"kernel\":" + json::quote(shape.kernel) + ",\"grid\":[" + std::to_string(shape.grid[0]) + "," +
           std::to_string(shape.grid[1]) + "," + std::to_string(shape.grid[2]) + "],\"block\":[" +
           std::to_string(shape.block[0]) + "," + std::to_string(shape.block[1]) + "," +
           std::to_string(shape.block[2]) + "],\"lds_bytes\":" + std::to_string(shape.lds_bytes) +
           (shape.epilogue_k ? ",\"epilogue_k\":" + std::to_string(shape.epilogue_k) : std::string()) + "}";
}

}  // namespace

KernelSpec read_spec(const char *text, size_t len) {
    if (!text || !len) refuse_invalid("no kernel spec document was given");
    KernelSpec spec;
    std::string error;
    if (!parse_spec(std::string(text, len), spec, error)) refuse_invalid("kernel spec: " + error);
    if (!validate(spec, Rules::Hip, error)) refuse_invalid(std::string(spec_name(spec)) + ": " + error);
    return spec;
}

size_t workspace_bytes_of(const KernelSpec &spec) {
    if (spec.op == Op::Gemm || spec.op == Op::GemmSimd) return hipk::gemm_f32_workspace_bytes(spec.m, spec.n, spec.k);
    if (spec.op == Op::AttentionOnline)
        return hipk::attention_online_workspace_bytes(spec.heads, spec.seq, spec.dim, spec.causal);
    return 0;
}

std::string describe_spec(const KernelSpec &spec) {
    std::string ref_error, hip_error;
    const bool reference_valid = validate(spec, Rules::Reference, ref_error);
    bool supported = hip_supported(spec, hip_error);
    const hipk::LaunchShape shape = supported ? launch_shape(spec) : hipk::LaunchShape{nullptr, {0, 0, 0}, {0, 0, 0}, 0};
    if (supported && !shape.kernel) {
        supported = false;
        hip_error = "no gfx950 kernel instantiation covers this shape";
    }
    std::string out =
        "{\"name\":" + json::quote(spec_name(spec)) + ",\"spec\":" + canonical_json(spec) + ",\"bindings\":[";
    const auto binds = bindings(spec);
    for (size_t i = 0; i < binds.size(); ++i) {
        if (i) out += ",";
        out += "{\"name\":" + json::quote(binds[i].name) + ",\"elements\":" + std::to_string(binds[i].elements) +
               ",\"write\":" + (binds[i].write ? "true" : "false") + "}";
    }
    out += std::string("],\"reference_valid\":") + (reference_valid ? "true" : "false");
    out += ",\"reference_error\":" + (reference_valid ? std::string("null") : json::quote(ref_error));
    out += std::string(",\"hip_supported\":") + (supported ? "true" : "false");
    out += ",\"hip_error\":" + (supported ? std::string("null") : json::quote(hip_error));
    if (supported)
        out += ",\"launch\":" + shape_json(shape) +
               ",\"workspace_bytes\":" + std::to_string(workspace_bytes_of(spec));
    else
        out += ",\"launch\":null,\"workspace_bytes\":0";
    return out + "}";
}

hipError_t enqueue(const Pipeline &p, hipStream_t st, void *const *b) {
    using namespace hipk;
    const KernelSpec &s = p.spec;
    auto in = [&](size_t i) { return static_cast<const float *>(b[i]); };
    auto out = [&](size_t i) { return static_cast<float *>(b[i]); };
    switch (s.op) {
        case Op::Elementwise: {
            if (p.copy) return copy_f32(st, in(0), out(s.inputs), s.len);
            const float *inputs[kMaxElementwiseInputs] = {};
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

PipelineCache::~PipelineCache() {
    (void)hipSetDevice(session_.ordinal());
    for (Pipeline *p : std::vector<Pipeline *>(all_.begin(), all_.end())) destroy(p);
}

void PipelineCache::destroy(Pipeline *p) {
    if (p->program) (void)hipFree(p->program);
    if (p->workspace) (void)hipFree(p->workspace);
    by_spec_.erase(p->canonical);
    all_.erase(p);
    delete p;
}

void PipelineCache::drop(Pipeline *p) {
    if (!all_.count(p) || --p->holders > 0) return;
    // A queued launch may still use the pipeline's workspace or program.
    (void)hipSetDevice(session_.ordinal());
    (void)hipStreamSynchronize(session_.queue());
    destroy(p);
}

Pipeline *PipelineCache::obtain(const KernelSpec &spec) {
    std::string unsupported;
    if (!hip_supported(spec, unsupported)) refuse_invalid(unsupported);
    if (!launch_shape(spec).kernel)
        refuse_invalid(std::string(spec_name(spec)) + ": no gfx950 kernel instantiation covers this shape");
    std::string canonical = canonical_json(spec);
    auto hit = by_spec_.find(canonical);
    if (hit != by_spec_.end()) {
        ++hit->second->holders;
        return hit->second;
    }
    session_.make_current();
    auto *p = new Pipeline;
    p->spec = spec;
    p->canonical = std::move(canonical);
    p->binds = bindings(spec);
    try {
        if (spec.op == Op::Elementwise) {
            const std::vector<Instr> code = compile_expression(*spec.expression);
            p->copy = code.size() == 1 && code[0].op == uint32_t(Opcode::Input) && code[0].arg == 0;
            p->program_len = uint32_t(code.size());
            const size_t bytes = code.size() * sizeof(Instr);
            dev::expect(hipMalloc(&p->program, bytes), "allocating the expression program");
            dev::expect(hipMemcpyAsync(p->program, code.data(), bytes, hipMemcpyHostToDevice, session_.queue()),
                        "uploading the expression program");
            session_.drain();
        }
        p->workspace_bytes = workspace_bytes_of(spec);
        if (p->workspace_bytes) {
            const hipError_t status = hipMalloc(&p->workspace, p->workspace_bytes);
            if (status != hipSuccess) {
                p->workspace = nullptr;
                refuse(status == hipErrorOutOfMemory ? Kind::Memory : Kind::Device,
                       text_of("%s needs %zu bytes of device workspace: %s", spec_name(spec), p->workspace_bytes,
                               hipGetErrorString(status)));
            }
        }
    } catch (...) {
        if (p->program) (void)hipFree(p->program);
        delete p;
        throw;
    }
    p->holders = 1;
    by_spec_.emplace(p->canonical, p);
    all_.insert(p);
    return p;
}

}  // namespace jade
