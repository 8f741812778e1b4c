// Fused QK-RMSNorm + rotate-half RoPE + K/V page write, gfx950.
//
// Replaces the reference's qk_norm_rope_store_kernel
// (src/backend/cuda/k_elementwise.cu:67-126); the arithmetic follows its f32
// CPU backend (src/backend/cpu/cpu_backend.cpp:34-39 rmsnorm, :155-172 the
// append loop, :262-272 rope) so that the f32 path reproduces it to the last
// bit almost everywhere.
//
// One wave64 per head vector of one token. Lane l holds elements l and l + 64:
// exactly a rotary pair (x_i, x_{i + D/2}), so the rotation needs no lane
// exchange, and each half-vector is one coalesced 128-byte (f16) or 256-byte
// (f32) access. The sum of squares is taken in double (products of f32 values
// are exact in double), matching the CPU's double accumulator; the angle's
// sine and cosine are evaluated in double and rounded once to f32.
#include "device.hpp"
#include "kernels.hpp"

namespace ember::hip {
namespace {

constexpr int kWavesPerBlock = 4;

template <typename T>
__global__ void __launch_bounds__(kWavesPerBlock * kWave) kv_append_kernel(EmberQkvArgs a) {
    constexpr int D = kHeadDim, HALF = D / 2;
    const int t = blockIdx.x;
    const int head = blockIdx.y * kWavesPerBlock + static_cast<int>(threadIdx.x) / kWave;
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const int total = a.n_heads + 2 * a.n_kv;
    if (head >= total) return;  // whole wave

    const T *src = static_cast<const T *>(a.qkv) + (static_cast<int64_t>(t) * total + head) * D;
    float x0 = to_f32(src[lane]), x1 = to_f32(src[lane + HALF]);
    if (a.bias) {
        x0 = x0 + a.bias[head * D + lane];
        x1 = x1 + a.bias[head * D + lane + HALF];
    }

    const int pos = a.positions[t];
    const bool is_q = head < a.n_heads, is_k = !is_q && head < a.n_heads + a.n_kv;
    if (is_q || is_k) qk_norm_rope(x0, x1, is_q ? a.q_norm : a.k_norm, a.eps, pos, a.inv_freq, lane);

    if (is_q) {
        T *dst = static_cast<T *>(a.q_out) + (static_cast<int64_t>(t) * a.n_heads + head) * D;
        dst[lane] = from_f32<T>(x0);
        dst[lane + HALF] = from_f32<T>(x1);
        return;
    }
    const int kvh = is_k ? head - a.n_heads : head - a.n_heads - a.n_kv;
    const int page = pos / kPage;
    if (pos < 0 || page >= a.max_blocks) return;
    const int block = a.block_tables[static_cast<int64_t>(a.token_seq[t]) * a.max_blocks + page];
    if (block < 0 || block >= a.num_blocks) return;  // never write outside the pool
    T *pool = static_cast<T *>(is_k ? a.k_cache : a.v_cache);
    T *dst = pool + ((static_cast<int64_t>(block) * a.n_kv + kvh) * kPage + pos % kPage) * D;
    dst[lane] = to_page<T>(x0);
    dst[lane + HALF] = to_page<T>(x1);
}

}  // namespace

hipError_t launch_kv_append(const EmberQkvArgs &a, hipStream_t stream) {
    if (a.T <= 0) return hipSuccess;
    const int heads = a.n_heads + 2 * a.n_kv;
    const dim3 grid(static_cast<unsigned>(a.T), static_cast<unsigned>((heads + kWavesPerBlock - 1) / kWavesPerBlock));
    const dim3 block(kWavesPerBlock * kWave);
    if (a.dtype == EMBER_DTYPE_F16)
        hipLaunchKernelGGL(kv_append_kernel<f16>, grid, block, 0, stream, a);
    else
        hipLaunchKernelGGL(kv_append_kernel<float>, grid, block, 0, stream, a);
    return hipGetLastError();
}

}  // namespace ember::hip
