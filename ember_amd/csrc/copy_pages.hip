// Whole-page copies: the device half of copy-on-write (no counterpart in the
// reference, which never writes a shared page). One work-group per
// (page pair, layer, K or V) moves the kv-head-contiguous page span
// (n_kv x 16 x head_dim elements; 32 KiB at 8 kv heads in f16) with 16-byte
// loads and stores. It doubles as the known-size copy that calibrates the
// HBM byte counters.
#include "device.hpp"
#include "kernels.hpp"

namespace ember::hip {
namespace {

constexpr int kCopyThreads = 256;

__global__ void __launch_bounds__(kCopyThreads) copy_pages_kernel(EmberCopyArgs a, int64_t page_vec16) {
    const int pair = blockIdx.x, layer = blockIdx.y, which = blockIdx.z;
    const int src = a.src_blocks[pair], dst = a.dst_blocks[pair];
    if (src < 0 || src >= a.num_blocks || dst < 0 || dst >= a.num_blocks || src == dst) return;
    char *pool = static_cast<char *>(which == 0 ? a.k_cache : a.v_cache);
    const int64_t elem = a.dtype == EMBER_DTYPE_F16 ? 2 : 4;
    char *layer_base = pool + static_cast<int64_t>(layer) * a.layer_stride * elem;
    const uint4 *from = reinterpret_cast<const uint4 *>(layer_base) + static_cast<int64_t>(src) * page_vec16;
    uint4 *to = reinterpret_cast<uint4 *>(layer_base) + static_cast<int64_t>(dst) * page_vec16;
    for (int64_t i = threadIdx.x; i < page_vec16; i += kCopyThreads) to[i] = from[i];
}

}  // namespace

hipError_t launch_copy_pages(const EmberCopyArgs &a, hipStream_t stream) {
    if (a.n <= 0 || a.n_layers <= 0) return hipSuccess;
    const int64_t elem = a.dtype == EMBER_DTYPE_F16 ? 2 : 4;
    const int64_t page_vec16 = static_cast<int64_t>(a.n_kv) * kPage * a.head_dim * elem / 16;
    const dim3 grid(static_cast<unsigned>(a.n), static_cast<unsigned>(a.n_layers), 2);
    hipLaunchKernelGGL(copy_pages_kernel, grid, dim3(kCopyThreads), 0, stream, a, page_vec16);
    return hipGetLastError();
}

}  // namespace ember::hip
