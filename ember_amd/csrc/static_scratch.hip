// ember_hip_paged_decode_static: ember_hip_paged_decode for callers that
// cannot allocate device memory (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc). The split scratch (partials of
// every (token, head, split) and their (max, sum)) and the per-(run, kv head)
// merge counters come from `scratch`, a file-scope device array of this
// library, instead of caller memory; the splits are always merged in the
// kernel (the same merge arithmetic and order as the separate merge kernel,
// so results are bit-identical to ember_hip_paged_decode's).
//
// Every GPU holds its own copy of `scratch` (EMBER_STATIC_SCRATCH_BYTES) until
// the process ends. Its address is looked up once per device, with that
// device current, by hipGetSymbolAddress: in host code the array's name is
// only a host-side stand-in, so kernels receive the looked-up pointer. Calls
// on one GPU share the array and keep the last call's contents; the counters
// are cleared by a fill kernel at the start of each call (no hipMemsetAsync,
// so the call can be captured). Calls that overlap on one GPU (two streams,
// two host threads) race on the array.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "capi_errors.hpp"
#include "ember_hip.h"
#include "kernels.hpp"

namespace {

constexpr size_t kCounterBytes = sizeof(uint32_t) * EMBER_STATIC_MAX_COUNTERS;
constexpr size_t kMlBytes = sizeof(float) * 2 * static_cast<size_t>(EMBER_STATIC_MAX_PARTIALS);
constexpr size_t kAccBytes = sizeof(float) * 128 * static_cast<size_t>(EMBER_STATIC_MAX_PARTIALS);
static_assert(kCounterBytes % 256 == 0 && kMlBytes % 256 == 0, "regions stay 256-byte aligned");
static_assert(kCounterBytes + kMlBytes + kAccBytes == EMBER_STATIC_SCRATCH_BYTES, "scratch layout");

// Layout: counters [EMBER_STATIC_MAX_COUNTERS] u32, then part_ml
// [EMBER_STATIC_MAX_PARTIALS][2] f32, then part_acc [EMBER_STATIC_MAX_PARTIALS][128] f32.
__device__ __align__(256) unsigned char scratch[EMBER_STATIC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_mutex;
void *g_scratch[kMaxDevices] = {};  // per device: scratch's device address

__global__ void __launch_bounds__(256) clear_counters_kernel(uint32_t *counters, int n) {
    const int i = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
    if (i < n) counters[i] = 0u;
}

// The current device's copy of `scratch`, looked up on the device's first call.
int device_scratch(void **out) {
    int dev = -1;
    if (hipError_t e = hipGetDevice(&dev); e != hipSuccess)
        return ember::hip::hip_status(e, "paged_decode_static: hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices)
        return ember::hip::set_error(EMBER_ERR_INVALID, "paged_decode_static: device %d beyond %d", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!g_scratch[dev]) {
        void *p = nullptr;
        if (hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)); e != hipSuccess)
            return ember::hip::hip_status(e, "paged_decode_static: hipGetSymbolAddress(scratch)");
        if (!p) return ember::hip::set_error(EMBER_ERR_INVALID, "paged_decode_static: scratch has no device address");
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return EMBER_OK;
}

}  // namespace

extern "C" int ember_hip_paged_decode_static(const EmberAttnArgs *args, void *stream) {
    using ember::hip::set_error;
    if (!args) return set_error(EMBER_ERR_INVALID, "paged_decode_static: null arguments");
    if (args->part_acc || args->part_ml || args->merge_counters)
        return set_error(EMBER_ERR_INVALID,
                         "paged_decode_static: part_acc, part_ml and merge_counters must be NULL (the library's "
                         "static scratch replaces them)");
    if (args->T <= 0 || args->num_splits < 1 || args->n_heads <= 0 || args->n_kv <= 0)
        return ember::hip::paged_decode(args, static_cast<hipStream_t>(stream), nullptr, nullptr);  // its own errors
    const long long partials = static_cast<long long>(args->T) * args->n_heads * args->num_splits;
    const long long runs = args->run_first ? args->num_runs : args->T;
    const long long counters = runs * args->n_kv;
    if (partials > EMBER_STATIC_MAX_PARTIALS)
        return set_error(EMBER_ERR_INVALID,
                         "paged_decode_static: %lld (token, head, split) partials exceed the static scratch's %d",
                         partials, EMBER_STATIC_MAX_PARTIALS);
    if (runs < 0 || counters > EMBER_STATIC_MAX_COUNTERS)
        return set_error(EMBER_ERR_INVALID, "paged_decode_static: %lld (run, kv head) counters exceed the static "
                         "scratch's %d", counters, EMBER_STATIC_MAX_COUNTERS);
    void *base = nullptr;
    if (int e = device_scratch(&base)) return e;
    auto *bytes = static_cast<unsigned char *>(base);
    EmberAttnArgs a = *args;
    a.merge_counters = reinterpret_cast<uint32_t *>(bytes);
    a.part_ml = reinterpret_cast<float *>(bytes + kCounterBytes);
    a.part_acc = reinterpret_cast<float *>(bytes + kCounterBytes + kMlBytes);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (counters > 0) {
        const int n = static_cast<int>(counters);
        hipLaunchKernelGGL(clear_counters_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s,
                           a.merge_counters, n);
        if (hipError_t e = hipGetLastError(); e != hipSuccess)
            return ember::hip::hip_status(e, "paged_decode_static: clearing the merge counters");
    }
    return ember::hip::paged_decode(&a, s, nullptr, nullptr);
}
