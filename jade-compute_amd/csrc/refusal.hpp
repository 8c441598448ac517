// Failure handling shared by every entry point of this library, with no
// HIP dependency (the host-only units include it too): failures are thrown
// as `Refusal` values and turned into a status code and NUL-terminated
// message exactly once, at the ABI edge (`abi_entry`). Each ABI maps the
// three failure kinds onto its own numeric codes.
#pragma once

#include <cstddef>
#include <cstdint>
#include <mutex>
#include <new>
#include <string>
#include <unordered_set>

namespace jade {
namespace dev {

// Why an entry point stopped: a caller error, a failed device step, or memory
// that could not be had (host or device).
enum class Kind { Invalid, Device, Memory };

struct Refusal {
    Kind kind;
    std::string text;
};

// printf-style message builder.
std::string text_of(const char *format, ...) __attribute__((format(printf, 1, 2)));

[[noreturn]] void refuse(Kind kind, std::string text);
[[noreturn]] inline void refuse_invalid(std::string text) { refuse(Kind::Invalid, std::move(text)); }

// Copies `text` into caller storage, truncating, always NUL-terminated when
// cap > 0. A null `out` or zero `cap` writes nothing.
void copy_text(const std::string &text, char *out, size_t cap);

// Runs `body` under the ABI error convention: clears `err`, returns 0 when
// the body returns normally, otherwise writes the message and returns
// `code_of(kind)`.
template <class CodeOf, class Body>
int abi_entry(char *err, size_t cap, CodeOf code_of, Body &&body) {
    if (err && cap) err[0] = '\0';
    try {
        body();
        return 0;
    } catch (const Refusal &r) {
        copy_text(r.text, err, cap);
        return code_of(r.kind);
    } catch (const std::bad_alloc &) {
        copy_text("host memory exhausted", err, cap);
        return code_of(Kind::Memory);
    }
}

// A set of live opaque handles of one type, so that an entry point can tell
// its own handles from stale or foreign pointers.
template <class T>
class HandleSet {
public:
    void add(T *h) {
        std::lock_guard<std::mutex> guard(mutex_);
        live_.insert(h);
    }
    bool remove(T *h) {
        std::lock_guard<std::mutex> guard(mutex_);
        return live_.erase(h) != 0;
    }
    T *find(void *h) {
        std::lock_guard<std::mutex> guard(mutex_);
        auto *t = static_cast<T *>(h);
        return live_.count(t) ? t : nullptr;
    }

private:
    std::mutex mutex_;
    std::unordered_set<T *> live_;
};

}  // namespace dev
}  // namespace jade
