// Failure handling shared by every entry point: see refusal.hpp.
#include "refusal.hpp"

#include <cstdarg>
#include <cstdio>
#include <cstring>

namespace jade {
namespace dev {

std::string text_of(const char *format, ...) {
    va_list args;
    va_start(args, format);
    va_list again;
    va_copy(again, args);
    const int n = std::vsnprintf(nullptr, 0, format, args);
    va_end(args);
    std::string out;
    if (n > 0) {
        out.resize(size_t(n) + 1);
        std::vsnprintf(&out[0], out.size(), format, again);
        out.resize(size_t(n));
    }
    va_end(again);
    return out;
}

void refuse(Kind kind, std::string text) { throw Refusal{kind, std::move(text)}; }

void copy_text(const std::string &text, char *out, size_t cap) {
    if (!out || !cap) return;
    const size_t n = text.size() < cap - 1 ? text.size() : cap - 1;
    std::memcpy(out, text.data(), n);
    out[n] = '\0';
}

}  // namespace dev
}  // namespace jade
