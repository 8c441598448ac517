// jr_gemm_f32_noalloc: the FP32 GEMM of a compiled `gemm` pipeline, launched
// on the caller's stream with no allocation of any kind, for callers that
// cannot allocate device memory (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc).
//
// The only device memory the GEMM needs besides A, B and C is the split-K
// partial products of small output grids. Here they live in `scratch`, a
// file-scope device array of kScratchBytes that every GPU the library runs on
// holds until the process ends. Its device address differs per GPU and is
// looked up once per device with hipGetSymbolAddress (the array's name is a
// host-side stand-in, not a device address); creating a runtime context on a
// device (jr_create) does that lookup, so calls on that device made later,
// for example under stream capture, only read the kept address. Every call on one GPU shares
// that GPU's array: calls that overlap on one GPU (two streams, or two
// threads) race on it. No clearing is needed: each split slice writes every
// element the reduce reads.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "jade_runtime_hip.h"
#include "kernels.hpp"
#include "session.hpp"
#include "spec.hpp"

namespace {

constexpr size_t kScratchBytes = size_t(8) << 20;
__device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float *g_scratch[kMaxDevices] = {};

// This device's address of `scratch`, looked up with the device current on
// the first call that needs it and kept afterwards.
float *scratch_on(int device) {
    using jade::dev::refuse;
    using jade::dev::text_of;
    if (device < 0 || device >= kMaxDevices)
        refuse(jade::dev::Kind::Invalid, text_of("device %d is outside the %d devices this entry serves", device,
                                                 kMaxDevices));
    std::lock_guard<std::mutex> guard(g_scratch_mutex);
    if (!g_scratch[device]) {
        void *ptr = nullptr;
        jade::dev::expect(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "looking up the scratch array");
        if (!ptr) refuse(jade::dev::Kind::Device, "the scratch array has no device address");
        g_scratch[device] = static_cast<float *>(ptr);
    }
    return g_scratch[device];
}

}  // namespace

namespace jade {
namespace hipk {
// Looks up this device's address of the scratch array (the device must be
// current). jr_create calls it for its device, so that calls made later
// under stream capture need no lookup there.
void noalloc_prepare(int device) { (void)scratch_on(device); }
}  // namespace hipk
}  // namespace jade

namespace {

int jr_code(jade::dev::Kind kind) {
    return kind == jade::dev::Kind::Invalid ? 1 : kind == jade::dev::Kind::Memory ? 3 : 2;
}

}  // namespace

extern "C" int jr_gemm_f32_noalloc(void *stream, const float *a, const float *b, float *c, uint32_t m, uint32_t n,
                                   uint32_t k, char *err, size_t cap) {
    using jade::dev::refuse_invalid;
    using jade::dev::text_of;
    return jade::dev::abi_entry(err, cap, jr_code, [&] {
        if (!a || !b || !c) refuse_invalid("jr_gemm_f32_noalloc needs device pointers for A, B and C");
        jade::KernelSpec spec;
        spec.op = jade::Op::Gemm;
        spec.m = m;
        spec.n = n;
        spec.k = k;
        spec.tiled = true;
        std::string error;
        if (!jade::validate(spec, jade::Rules::Hip, error)) refuse_invalid("gemm: " + error);
        if (((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15u) != 0)
            refuse_invalid("A and B must start on 16-byte boundaries (whole device allocations do)");
        const size_t need = jade::hipk::gemm_f32_workspace_bytes(m, n, k);
        if (need > kScratchBytes)
            refuse_invalid(text_of("a %ux%ux%u product needs %zu bytes of split-K scratch; this entry holds %zu",
                                   m, n, k, need, kScratchBytes));
        float *work = nullptr;
        if (need) {
            int device = -1;
            jade::dev::expect(hipGetDevice(&device), "reading the current device");
            work = scratch_on(device);
        }
        jade::dev::expect(jade::hipk::gemm_f32(static_cast<hipStream_t>(stream), a, b, c, m, n, k, work),
                          "launching the GEMM");
    });
}
