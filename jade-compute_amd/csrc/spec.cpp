#include "spec.hpp"

#include <cmath>
#include <cstring>

namespace jade {
namespace {

using json::Value;

constexpr uint64_t kIntMax = 2147483647ull;  // i32::MAX, the reference's index bound
// HIP grid limits of the attention launches. Heads: grid.y of the batched
// P.V launch and grid.z of the score launches may not exceed 65535 (the
// online kernel puts heads on grid.x, but all attention ops share the cap).
// Sequence: the online kernel's query blocks (at least 128 queries each) sit
// on grid.y, so seq may not exceed 65535 * 128.
constexpr uint32_t kHipMaxHeads = 65535;
constexpr uint32_t kHipMaxOnlineSeq = 65535u * 128u;

struct OpName {
    const char *tag;
    Op op;
};
constexpr OpName kOps[] = {
    {"elementwise", Op::Elementwise},
    {"axpy", Op::Axpy},
    {"add", Op::Add},
    {"gemm", Op::Gemm},
    {"gemm_simd", Op::GemmSimd},
    {"gemm_mps", Op::GemmMps},
    {"attention_scores", Op::AttentionScores},
    {"attention_apply", Op::AttentionApply},
    {"attention_online", Op::AttentionOnline},
    {"rms_norm", Op::RmsNorm},
    {"swi_glu", Op::SwiGlu},
    {"softmax", Op::Softmax},
};

const char *tag_of(Op op) {
    for (const auto &o : kOps)
        if (o.op == op) return o.tag;
    return "?";
}

bool get_u32(const Value &obj, const char *key, uint32_t &out, std::string &error) {
    const Value *v = obj.find(key);
    if (!v) { error = std::string("missing field `") + key + "`"; return false; }
    if (!json::as_u32(*v, out)) { error = std::string("field `") + key + "` must be a u32"; return false; }
    return true;
}
bool get_bool(const Value &obj, const char *key, bool &out, std::string &error) {
    const Value *v = obj.find(key);
    if (!v) { error = std::string("missing field `") + key + "`"; return false; }
    if (v->kind != Value::Kind::Bool) { error = std::string("field `") + key + "` must be a boolean"; return false; }
    out = v->boolean;
    return true;
}
bool get_f32(const Value &obj, const char *key, float &out, std::string &error) {
    const Value *v = obj.find(key);
    if (!v) { error = std::string("missing field `") + key + "`"; return false; }
    if (!json::as_f32(*v, out)) { error = std::string("field `") + key + "` must be a number"; return false; }
    return true;
}

bool parse_expr(const Value &v, Expr &out, std::string &error, int depth) {
    // Structural guard only; the reference's depth/node limits apply in validate.
    if (depth > 64) { error = "expression nesting exceeds parser limit"; return false; }
    if (v.kind != Value::Kind::Object) { error = "expression must be an object"; return false; }
    const Value *kind = v.find("kind");
    if (!kind || kind->kind != Value::Kind::String) { error = "expression missing string tag `kind`"; return false; }
    const std::string &k = kind->text;
    auto child = [&](const char *key, std::unique_ptr<Expr> &slot) -> bool {
        const Value *c = v.find(key);
        if (!c) { error = std::string("missing field `") + key + "`"; return false; }
        slot.reset(new Expr);
        return parse_expr(*c, *slot, error, depth + 1);
    };
    if (k == "input") {
        out.kind = Expr::Kind::Input;
        return get_u32(v, "binding", out.binding, error);
    }
    if (k == "constant") {
        out.kind = Expr::Kind::Constant;
        return get_f32(v, "value", out.value, error);
    }
    if (k == "add" || k == "multiply" || k == "maximum") {
        out.kind = k == "add" ? Expr::Kind::Add : k == "multiply" ? Expr::Kind::Multiply : Expr::Kind::Maximum;
        return child("left", out.left) && child("right", out.right);
    }
    if (k == "negate" || k == "exp") {
        out.kind = k == "negate" ? Expr::Kind::Negate : Expr::Kind::Exp;
        return child("value", out.left);
    }
    error = "unknown expression kind `" + k + "`";
    return false;
}

bool expr_validate(const Expr &e, uint32_t inputs, uint32_t depth, uint32_t &nodes, std::string &error) {
    nodes += 1;
    if (!(depth <= kMaxExprDepth && nodes <= kMaxExprNodes)) {
        error = "expression exceeds compiler complexity limit";
        return false;
    }
    switch (e.kind) {
        case Expr::Kind::Input:
            if (!(e.binding < inputs)) { error = "expression input binding out of range"; return false; }
            return true;
        case Expr::Kind::Constant:
            if (!std::isfinite(e.value)) { error = "expression constant must be finite"; return false; }
            return true;
        case Expr::Kind::Add:
        case Expr::Kind::Multiply:
        case Expr::Kind::Maximum:
            return expr_validate(*e.left, inputs, depth + 1, nodes, error) &&
                   expr_validate(*e.right, inputs, depth + 1, nodes, error);
        case Expr::Kind::Negate:
        case Expr::Kind::Exp:
            return expr_validate(*e.left, inputs, depth + 1, nodes, error);
    }
    return false;
}

bool dim_ok(uint64_t v, std::string &error) {
    if (!(v > 0 && v <= kIntMax)) { error = "dimension must be in 1..=INT_MAX"; return false; }
    return true;
}
bool matrix_ok(uint64_t x, uint64_t y, std::string &error) {
    if (!dim_ok(x, error) || !dim_ok(y, error)) return false;
    if (x * y > kIntMax) { error = "tensor exceeds checked 31-bit indexing"; return false; }
    return true;
}

void expr_json(const Expr &e, std::string &out) {
    switch (e.kind) {
        case Expr::Kind::Input:
            out += "{\"kind\":\"input\",\"binding\":" + std::to_string(e.binding) + "}";
            return;
        case Expr::Kind::Constant:
            out += "{\"kind\":\"constant\",\"value\":" + json::format_f32(e.value) + "}";
            return;
        case Expr::Kind::Add:
        case Expr::Kind::Multiply:
        case Expr::Kind::Maximum:
            out += std::string("{\"kind\":\"") +
                   (e.kind == Expr::Kind::Add ? "add" : e.kind == Expr::Kind::Multiply ? "multiply" : "maximum") +
                   "\",\"left\":";
            expr_json(*e.left, out);
            out += ",\"right\":";
            expr_json(*e.right, out);
            out += "}";
            return;
        case Expr::Kind::Negate:
        case Expr::Kind::Exp:
            out += std::string("{\"kind\":\"") + (e.kind == Expr::Kind::Negate ? "negate" : "exp") + "\",\"value\":";
            expr_json(*e.left, out);
            out += "}";
            return;
    }
}

void lower(const Expr &e, std::vector<Instr> &code) {
    switch (e.kind) {
        case Expr::Kind::Input:
            code.push_back({uint32_t(Opcode::Input), e.binding});
            return;
        case Expr::Kind::Constant: {
            uint32_t bits;
            std::memcpy(&bits, &e.value, sizeof bits);
            code.push_back({uint32_t(Opcode::Constant), bits});
            return;
        }
        case Expr::Kind::Add:
        case Expr::Kind::Multiply:
        case Expr::Kind::Maximum:
            lower(*e.left, code);
            lower(*e.right, code);
            code.push_back({uint32_t(e.kind == Expr::Kind::Add ? Opcode::Add
                                     : e.kind == Expr::Kind::Multiply ? Opcode::Multiply
                                                                      : Opcode::Maximum),
                            0});
            return;
        case Expr::Kind::Negate:
        case Expr::Kind::Exp:
            lower(*e.left, code);
            code.push_back({uint32_t(e.kind == Expr::Kind::Negate ? Opcode::Negate : Opcode::Exp), 0});
            return;
    }
}

}  // namespace

bool parse_spec(const std::string &text, KernelSpec &out, std::string &error) {
    if (text.size() > 65536) { error = "kernel JSON exceeds 64 KiB"; return false; }
    Value root;
    if (!json::parse(text, root, error)) return false;
    if (root.kind != Value::Kind::Object) { error = "kernel spec must be a JSON object"; return false; }
    const Value *tag = root.find("op");
    if (!tag || tag->kind != Value::Kind::String) { error = "missing string tag `op`"; return false; }
    bool known = false;
    for (const auto &o : kOps)
        if (tag->text == o.tag) { out.op = o.op; known = true; }
    if (!known) { error = "unknown variant `" + tag->text + "`"; return false; }
    switch (out.op) {
        case Op::Elementwise: {
            if (!get_u32(root, "len", out.len, error) || !get_u32(root, "inputs", out.inputs, error)) return false;
            const Value *e = root.find("expression");
            if (!e) { error = "missing field `expression`"; return false; }
            auto expr = std::make_shared<Expr>();
            if (!parse_expr(*e, *expr, error, 0)) return false;
            out.expression = expr;
            return true;
        }
        case Op::Axpy:
            return get_u32(root, "len", out.len, error) && get_f32(root, "alpha", out.alpha, error);
        case Op::Add:
        case Op::SwiGlu:
            return get_u32(root, "len", out.len, error);
        case Op::Gemm:
            return get_u32(root, "m", out.m, error) && get_u32(root, "n", out.n, error) &&
                   get_u32(root, "k", out.k, error) && get_bool(root, "tiled", out.tiled, error);
        case Op::GemmSimd:
        case Op::GemmMps:
            return get_u32(root, "m", out.m, error) && get_u32(root, "n", out.n, error) &&
                   get_u32(root, "k", out.k, error);
        case Op::AttentionScores:
        case Op::AttentionOnline:
            return get_u32(root, "heads", out.heads, error) && get_u32(root, "seq", out.seq, error) &&
                   get_u32(root, "dim", out.dim, error) && get_bool(root, "causal", out.causal, error);
        case Op::AttentionApply:
            return get_u32(root, "heads", out.heads, error) && get_u32(root, "seq", out.seq, error) &&
                   get_u32(root, "dim", out.dim, error);
        case Op::RmsNorm:
            return get_u32(root, "rows", out.rows, error) && get_u32(root, "cols", out.cols, error) &&
                   get_f32(root, "epsilon", out.epsilon, error);
        case Op::Softmax:
            return get_u32(root, "rows", out.rows, error) && get_u32(root, "cols", out.cols, error);
    }
    return false;
}

const char *spec_name(const KernelSpec &spec) {
    switch (spec.op) {
        case Op::Elementwise: return "elementwise";
        case Op::Axpy: return "axpy";
        case Op::Add: return "add";
        case Op::Gemm: return spec.tiled ? "gemm_register32" : "gemm_naive";
        case Op::GemmSimd: return "gemm_simdgroup_fp32";
        case Op::GemmMps: return "gemm_mps_fp32";
        case Op::AttentionScores: return "attention_scores";
        case Op::AttentionApply: return "attention_apply";
        case Op::AttentionOnline: return "attention_online";
        case Op::RmsNorm: return "rms_norm";
        case Op::SwiGlu: return "swi_glu";
        case Op::Softmax: return "softmax";
    }
    return "?";
}

bool validate(const KernelSpec &s, Rules rules, std::string &error) {
    switch (s.op) {
        case Op::Elementwise: {
            if (!dim_ok(s.len, error)) return false;
            if (!(s.inputs > 0 && s.inputs <= kMaxElementwiseInputs)) {
                error = "elementwise input count must be 1..8";
                return false;
            }
            if (!s.expression) { error = "missing expression"; return false; }
            uint32_t nodes = 0;
            return expr_validate(*s.expression, s.inputs, 0, nodes, error);
        }
        case Op::Axpy:
            if (!dim_ok(s.len, error)) return false;
            if (!std::isfinite(s.alpha)) { error = "alpha must be finite"; return false; }
            return true;
        case Op::Add:
        case Op::SwiGlu:
            return dim_ok(s.len, error);
        case Op::Gemm:
        case Op::GemmSimd:
        case Op::GemmMps:
            return matrix_ok(s.m, s.k, error) && matrix_ok(s.k, s.n, error) && matrix_ok(s.m, s.n, error);
        case Op::AttentionScores:
        case Op::AttentionApply:
        case Op::AttentionOnline: {
            if (rules == Rules::Reference) {
                if (!(s.heads >= 1 && s.heads <= 32)) { error = "attention heads must be 1..=32"; return false; }
                if (!(s.seq >= 1 && s.seq <= 2048)) { error = "attention sequence must be 1..=2048"; return false; }
                if (!(s.dim >= 1 && s.dim <= 128)) { error = "attention head dimension must be 1..=128"; return false; }
                const uint64_t hs = uint64_t(s.heads) * s.seq;  // cannot exceed u32 under the caps
                return matrix_ok(hs, s.dim, error) && matrix_ok(hs, s.seq, error);
            }
            if (!(s.heads >= 1 && s.heads <= kHipMaxHeads)) { error = "attention heads must be 1..=65535"; return false; }
            if (!(s.seq >= 1)) { error = "attention sequence must be positive"; return false; }
            if (!(s.dim >= 1 && s.dim <= 128)) { error = "attention head dimension must be 1..=128"; return false; }
            const uint64_t hs = uint64_t(s.heads) * s.seq;
            if (!matrix_ok(hs, s.dim, error)) return false;
            if (s.op != Op::AttentionOnline) return matrix_ok(hs, s.seq, error);
            if (s.seq > kHipMaxOnlineSeq) {
                error = "online attention sequence must be at most 8388480 (65535 query blocks of 128)";
                return false;
            }
            return true;
        }
        case Op::RmsNorm:
            if (!matrix_ok(s.rows, s.cols, error)) return false;
            if (!(std::isfinite(s.epsilon) && s.epsilon > 0.0f)) {
                error = "epsilon must be finite and positive";
                return false;
            }
            return true;
        case Op::Softmax:
            return matrix_ok(s.rows, s.cols, error);
    }
    error = "unknown op";
    return false;
}

bool hip_supported(const KernelSpec &spec, std::string &error) {
    if (spec.op == Op::GemmMps) {
        error = "gemm_mps is an Apple MPS library operation; use gemm or gemm_simd on the HIP backend";
        return false;
    }
    return true;
}

std::vector<Binding> bindings(const KernelSpec &s) {
    static const char *kInputNames[] = {"input0", "input1", "input2", "input3",
                                        "input4", "input5", "input6", "input7"};
    const uint64_t hsd = uint64_t(s.heads) * s.seq * s.dim;
    const uint64_t hss = uint64_t(s.heads) * s.seq * s.seq;
    switch (s.op) {
        case Op::Elementwise: {
            std::vector<Binding> out;
            for (uint32_t i = 0; i < s.inputs && i < kMaxElementwiseInputs; ++i)
                out.push_back({kInputNames[i], s.len, false});
            out.push_back({"out", s.len, true});
            return out;
        }
        case Op::Axpy:
        case Op::Add:
            return {{"a", s.len, false}, {"b", s.len, false}, {"out", s.len, true}};
        case Op::SwiGlu:
            return {{"gate", s.len, false}, {"up", s.len, false}, {"out", s.len, true}};
        case Op::Gemm:
        case Op::GemmSimd:
        case Op::GemmMps:
            return {{"a", uint64_t(s.m) * s.k, false},
                    {"b", uint64_t(s.k) * s.n, false},
                    {"out", uint64_t(s.m) * s.n, true}};
        case Op::AttentionScores:
            return {{"q", hsd, false}, {"k", hsd, false}, {"scores", hss, true}};
        case Op::AttentionApply:
            return {{"probabilities", hss, false}, {"v", hsd, false}, {"out", hsd, true}};
        case Op::AttentionOnline:
            return {{"q", hsd, false}, {"k", hsd, false}, {"v", hsd, false}, {"out", hsd, true}};
        case Op::RmsNorm:
            return {{"x", uint64_t(s.rows) * s.cols, false},
                    {"weight", s.cols, false},
                    {"out", uint64_t(s.rows) * s.cols, true}};
        case Op::Softmax:
            return {{"x", uint64_t(s.rows) * s.cols, false}, {"out", uint64_t(s.rows) * s.cols, true}};
    }
    return {};
}

bool validate_bindings(const KernelSpec &spec, const uint64_t *lengths, const uint64_t *ids, size_t count,
                       std::string &error) {
    const auto expected = bindings(spec);
    if (count != expected.size()) {
        error = std::string(spec_name(spec)) + " expects " + std::to_string(expected.size()) + " bindings";
        return false;
    }
    for (size_t i = 0; i < expected.size(); ++i) {
        if (lengths[i] != expected[i].elements) {
            error = std::string(spec_name(spec)) + " binding " + expected[i].name + " expected " +
                    std::to_string(expected[i].elements) + " floats, got " + std::to_string(lengths[i]);
            return false;
        }
        if (expected[i].write) {
            for (size_t j = 0; j < count; ++j) {
                if (i != j && ids[i] == ids[j]) {
                    error = "output binding must not alias another binding";
                    return false;
                }
            }
        }
    }
    return true;
}

std::string canonical_json(const KernelSpec &s) {
    std::string out = std::string("{\"op\":\"") + tag_of(s.op) + "\"";
    auto u = [&](const char *k, uint32_t v) { out += std::string(",\"") + k + "\":" + std::to_string(v); };
    auto b = [&](const char *k, bool v) { out += std::string(",\"") + k + "\":" + (v ? "true" : "false"); };
    auto f = [&](const char *k, float v) { out += std::string(",\"") + k + "\":" + json::format_f32(v); };
    switch (s.op) {
        case Op::Elementwise:
            u("len", s.len);
            u("inputs", s.inputs);
            out += ",\"expression\":";
            if (s.expression) expr_json(*s.expression, out);
            else out += "null";
            break;
        case Op::Axpy: u("len", s.len); f("alpha", s.alpha); break;
        case Op::Add:
        case Op::SwiGlu: u("len", s.len); break;
        case Op::Gemm: u("m", s.m); u("n", s.n); u("k", s.k); b("tiled", s.tiled); break;
        case Op::GemmSimd:
        case Op::GemmMps: u("m", s.m); u("n", s.n); u("k", s.k); break;
        case Op::AttentionScores:
        case Op::AttentionOnline: u("heads", s.heads); u("seq", s.seq); u("dim", s.dim); b("causal", s.causal); break;
        case Op::AttentionApply: u("heads", s.heads); u("seq", s.seq); u("dim", s.dim); break;
        case Op::RmsNorm: u("rows", s.rows); u("cols", s.cols); f("epsilon", s.epsilon); break;
        case Op::Softmax: u("rows", s.rows); u("cols", s.cols); break;
    }
    return out + "}";
}

std::vector<Instr> compile_expression(const Expr &expr) {
    std::vector<Instr> code;
    lower(expr, code);
    return code;
}

}  // namespace jade
