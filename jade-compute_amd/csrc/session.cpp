// Device layer: see session.hpp.
#include "session.hpp"

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

namespace jade {
namespace dev {

void expect(hipError_t status, const char *step) {
    if (status == hipSuccess) return;
    const Kind kind = status == hipErrorOutOfMemory ? Kind::Memory : Kind::Device;
    refuse(kind, text_of("%s failed with %s (HIP status %d: %s)", step, hipGetErrorName(status), int(status),
                         hipGetErrorString(status)));
}

Session::Session(int ordinal) {
    if (ordinal < 0) refuse_invalid(text_of("device ordinal %d is negative", ordinal));
    int devices = 0;
    expect(hipGetDeviceCount(&devices), "counting HIP devices");
    if (ordinal >= devices)
        refuse_invalid(text_of("device ordinal %d does not exist (%d HIP device(s) visible)", ordinal, devices));
    ordinal_ = ordinal;
    try {
        make_current();
        // Default priority on purpose: every queue of this library runs at the
        // same priority.
        expect(hipStreamCreateWithFlags(&queue_, hipStreamNonBlocking), "creating the session queue");
        expect(hipEventCreate(&clock_[0]), "creating the start event");
        expect(hipEventCreate(&clock_[1]), "creating the stop event");
    } catch (...) {
        release_all();
        throw;
    }
}

Session::~Session() { release_all(); }

void Session::release_all() {
    if (ordinal_ >= 0) (void)hipSetDevice(ordinal_);
    if (queue_) (void)hipStreamSynchronize(queue_);
    for (auto &entry : regions_) (void)hipFree(const_cast<void *>(entry.first));
    regions_.clear();
    for (hipEvent_t &e : clock_) {
        if (e) (void)hipEventDestroy(e);
        e = nullptr;
    }
    if (queue_) (void)hipStreamDestroy(queue_);
    queue_ = nullptr;
}

void Session::make_current() const { expect(hipSetDevice(ordinal_), "selecting the session's device"); }

void Session::drain() const { expect(hipStreamSynchronize(queue_), "waiting for the session queue"); }

void *Session::allocate_zeroed(size_t bytes) {
    if (!bytes) refuse_invalid("a device region must hold at least one byte");
    make_current();
    void *ptr = nullptr;
    const hipError_t status = hipMalloc(&ptr, bytes);
    if (status != hipSuccess)
        refuse(status == hipErrorOutOfMemory ? Kind::Memory : Kind::Device,
               text_of("no device region of %zu bytes: %s", bytes, hipGetErrorString(status)));
    try {
        // The region reads as zeros before its first upload.
        expect(hipMemsetAsync(ptr, 0, bytes, queue_), "zero-filling a new region");
        drain();
        regions_.emplace(ptr, Region{bytes, next_serial_++});
    } catch (...) {
        (void)hipFree(ptr);
        throw;
    }
    return ptr;
}

bool Session::give_back(void *ptr) {
    auto it = regions_.find(ptr);
    if (it == regions_.end()) return false;
    if (hipSetDevice(ordinal_) != hipSuccess) return false;
    // A kernel still queued may read the region.
    (void)hipStreamSynchronize(queue_);
    (void)hipFree(ptr);
    regions_.erase(it);
    return true;
}

const Session::Region *Session::region(const void *ptr) const {
    auto it = regions_.find(ptr);
    return it == regions_.end() ? nullptr : &it->second;
}

namespace {
const Session::Region &whole_region(const Session &s, const void *ptr, size_t bytes, const char *direction) {
    const Session::Region *r = s.region(ptr);
    if (!r) refuse_invalid(text_of("%s: %p is not a live region of this session", direction, ptr));
    if (r->bytes != bytes)
        refuse_invalid(text_of("%s: transfers move whole regions; this one holds %zu bytes, %zu were given",
                               direction, r->bytes, bytes));
    return *r;
}
}  // namespace

void Session::write_region(void *dst, const void *host, size_t bytes) {
    if (!host) refuse_invalid("upload: null host source");
    whole_region(*this, dst, bytes, "upload");
    make_current();
    expect(hipMemcpyAsync(dst, host, bytes, hipMemcpyHostToDevice, queue_), "host-to-device copy");
    drain();
}

void Session::read_region(void *host, const void *src, size_t bytes) {
    if (!host) refuse_invalid("download: null host destination");
    whole_region(*this, src, bytes, "download");
    make_current();
    expect(hipMemcpyAsync(host, src, bytes, hipMemcpyDeviceToHost, queue_), "device-to-host copy");
    drain();
}

double Session::stop_clock() {
    const hipError_t recorded = hipEventRecord(clock_[1], queue_);
    if (recorded != hipSuccess) {
        (void)hipStreamSynchronize(queue_);
        expect(recorded, "stop event");
    }
    expect(hipEventSynchronize(clock_[1]), "waiting for the stop event");
    float ms = 0.0f;
    expect(hipEventElapsedTime(&ms, clock_[0], clock_[1]), "reading the event clock");
    if (!(ms >= 0.0f) || !std::isfinite(ms)) refuse(Kind::Device, text_of("event clock read %g ms", double(ms)));
    return double(ms);
}

std::string Session::device_summary() const {
    make_current();
    hipDeviceProp_t prop{};
    expect(hipGetDeviceProperties(&prop, ordinal_), "reading device properties");
    int runtime = 0, driver = 0;
    expect(hipRuntimeGetVersion(&runtime), "reading the HIP runtime version");
    expect(hipDriverGetVersion(&driver), "reading the driver version");
    // The reference's info names the device (native/jade_runtime_corex.cpp:
    // 88-89). Some drivers report no product name; the ISA name (without its
    // feature suffixes) stands in for it then.
    std::string name(prop.name);
    if (name.find_first_not_of(" \t") == std::string::npos) {
        name = prop.gcnArchName;
        name = name.substr(0, name.find(':'));
    }
    return text_of("hip:%d name=%s isa=%s cus=%d hbm_bytes=%llu hip_runtime=%d hip_driver=%d", ordinal_, name.c_str(),
                   prop.gcnArchName, prop.multiProcessorCount, static_cast<unsigned long long>(prop.totalGlobalMem),
                   runtime, driver);
}

}  // namespace dev
}  // namespace jade
