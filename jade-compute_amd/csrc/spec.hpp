// KernelSpec / Expr: the reference's checked operation IR (src/runtime/ir.rs:6-84)
// restated in C++ for the HIP backend. Parsing accepts the reference's serde JSON
// (internally tagged, `op` / `kind`, snake_case); validation applies the
// reference's rules (ir.rs:86-110, 193-268) with the HIP relaxations listed at
// `validate`. This translation unit has no HIP dependency so it is CPU-testable.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "json.hpp"

namespace jade {

enum class Op {
    Elementwise,
    Axpy,
    Add,
    Gemm,
    GemmSimd,
    GemmMps,
    AttentionScores,
    AttentionApply,
    AttentionOnline,
    RmsNorm,
    SwiGlu,
    Softmax,
};

// Expression tree, ir.rs:74-84.
struct Expr {
    enum class Kind { Input, Constant, Add, Multiply, Maximum, Negate, Exp } kind = Kind::Input;
    uint32_t binding = 0;
    float value = 0.0f;
    std::unique_ptr<Expr> left, right;  // unary nodes use `left`
};

// Postfix program evaluated by the elementwise interpreter kernel.
enum class Opcode : uint32_t { Input = 0, Constant = 1, Add = 2, Multiply = 3, Maximum = 4, Negate = 5, Exp = 6 };
struct Instr {
    uint32_t op;   // Opcode
    uint32_t arg;  // binding index, or the f32 bits of a constant
};
constexpr uint32_t kMaxExprNodes = 512;     // ir.rs:89
constexpr uint32_t kMaxExprDepth = 32;      // ir.rs:89
constexpr uint32_t kMaxExprStack = kMaxExprDepth + 2;
constexpr uint32_t kMaxElementwiseInputs = 8;  // ir.rs:218

struct KernelSpec {
    Op op = Op::Add;
    uint32_t len = 0, inputs = 0;
    uint32_t m = 0, n = 0, k = 0;
    uint32_t heads = 0, seq = 0, dim = 0;
    uint32_t rows = 0, cols = 0;
    bool tiled = false, causal = false;
    float alpha = 0.0f, epsilon = 0.0f;
    std::shared_ptr<Expr> expression;
};

// ir.rs:146-151. Elements are f32 counts.
struct Binding {
    const char *name;
    uint64_t elements;
    bool write;
};

enum class Rules { Reference, Hip };

// serde-compatible parse; unknown members are ignored as serde does by default.
bool parse_spec(const std::string &text, KernelSpec &out, std::string &error);

// ir.rs:176-192 (`KernelSpec::name`).
const char *spec_name(const KernelSpec &spec);

// ir.rs:193-268. Rules::Reference reproduces the reference exactly. Rules::Hip
// lifts the Metal-era attention caps (heads <= 32, seq <= 2048, and the
// heads*seq*seq <= INT_MAX check for the online op, which keeps no S*S
// buffer) while keeping every per-tensor 31-bit element bound.
bool validate(const KernelSpec &spec, Rules rules, std::string &error);

// True when the HIP backend has a kernel for the op (everything except the
// Apple-library gemm_mps op).
bool hip_supported(const KernelSpec &spec, std::string &error);

// ir.rs:269-339. Caller must validate first.
std::vector<Binding> bindings(const KernelSpec &spec);

// ir.rs:340-367: exact lengths; a write binding must not share identity with
// any other binding; read/read aliasing is allowed.
bool validate_bindings(const KernelSpec &spec, const uint64_t *lengths, const uint64_t *ids,
                       size_t count, std::string &error);

// Compact serde-shaped JSON (tag first, fields in declaration order).
std::string canonical_json(const KernelSpec &spec);

// Postfix lowering of an Elementwise expression (depth-first, left first).
std::vector<Instr> compile_expression(const Expr &expr);

}  // namespace jade
