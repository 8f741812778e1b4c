// Internal launchers of the gfx950 kernels. The C ABI (capi.hip) validates
// arguments and calls these; each enqueues on `stream` and returns the launch
// status.
#pragma once

#include <hip/hip_runtime.h>

#include "ember_hip.h"

namespace ember::hip {

hipError_t launch_kv_append(const EmberQkvArgs &a, hipStream_t stream);

// Decode attention (+ the split merge when a.num_splits > 1). `rows` is the
// kernel's query-row capacity, G * max_run rounded up to a built instance.
// Given events, the attention kernel's own dispatch is timed into them
// (hipExtLaunchKernel: the start and end of that kernel, the merge excluded).
hipError_t launch_paged_decode(const EmberAttnArgs &a, int rows, hipStream_t stream, hipEvent_t start = nullptr,
                               hipEvent_t stop = nullptr);

// The fused append + decode launch (ember_hip_decode_step).
hipError_t launch_decode_step(const EmberQkvArgs &qa, const EmberAttnArgs &a, int rows, hipStream_t stream,
                              hipEvent_t start = nullptr, hipEvent_t stop = nullptr);

// Validation + launch behind ember_hip_paged_decode / ember_hip_decode_step
// (qkv == nullptr: the unfused kernel), for in-library callers that time the
// kernel. Returns an EMBER_* / hipError_t code.
int paged_decode(const EmberAttnArgs *a, hipStream_t stream, hipEvent_t start, hipEvent_t stop,
                 const EmberQkvArgs *qkv = nullptr);

// Given events, the prefill kernel's own dispatch is timed into them.
hipError_t launch_prefill(const EmberPrefillArgs &a, hipStream_t stream, hipEvent_t start = nullptr,
                          hipEvent_t stop = nullptr);

// Validation + launch behind ember_hip_prefill_attn, for in-library callers
// that time the kernel. Returns an EMBER_* / hipError_t code.
int prefill_attn(const EmberPrefillArgs *a, hipStream_t stream, hipEvent_t start, hipEvent_t stop);

hipError_t launch_copy_pages(const EmberCopyArgs &a, hipStream_t stream);

hipError_t launch_gemv(const EmberGemvArgs &a, hipStream_t stream);
int64_t gemv_workspace_bytes(int M, int N, int K);  // 0: no K split for this shape
int64_t gemv_packed_bytes(int N, int K);
hipError_t launch_gemv_pack(const void *W, int N, int K, void *out, hipStream_t stream);

hipError_t launch_rmsnorm_rows(const EmberNormArgs &a, hipStream_t stream);

hipError_t launch_embed(const EmberEmbedArgs &a, hipStream_t stream);
hipError_t launch_sample(const EmberSampleArgs &a, hipStream_t stream);
hipError_t launch_token_probs(const EmberProbArgs &a, hipStream_t stream);

// Row capacities with a built decode kernel, ascending.
constexpr int kDecodeRowInstances[] = {1, 2, 4, 8, 10, 16};

// The built row capacity that serves G query heads per kv head and runs of up
// to max_run tokens; 0 if none does.
int decode_rows(int G, int max_run);

}  // namespace ember::hip
