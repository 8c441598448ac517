// Minimal JSON reader/writer for KernelSpec documents (<= 64 KiB, as the
// reference's `emit` command caps them: src/bin/jade-runtime.rs:205-209).
// Objects keep member order; numbers keep their source text so integer fields
// can be range-checked exactly the way serde checks a u32.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <utility>
#include <vector>

namespace jade {
namespace json {

struct Value {
    enum class Kind { Null, Bool, Number, String, Array, Object } kind = Kind::Null;
    bool boolean = false;
    std::string text;  // number source text or string contents
    std::vector<Value> items;
    std::vector<std::pair<std::string, Value>> members;

    const Value *find(const std::string &key) const {
        for (const auto &m : members)
            if (m.first == key) return &m.second;
        return nullptr;
    }
};

// Parses `source`; on failure returns false and sets `error`.
bool parse(const std::string &source, Value &out, std::string &error);

// Exact u32 from a JSON number (no sign, fraction or exponent), as serde does.
bool as_u32(const Value &v, uint32_t &out);
// Finite or non-finite f32 from a JSON number, rounded once from its decimal text.
bool as_f32(const Value &v, float &out);

// Shortest round-trip decimal for an f32 (used for canonical cache keys).
std::string format_f32(float value);
std::string quote(const std::string &s);

}  // namespace json
}  // namespace jade
