// Fused QK-RMSNorm + rotate-half RoPE + K/V page write, gfx950.
//
// Replaces the reference's qk_norm_rope_store_kernel
// (src/backend/cuda/k_elementwise.cu:67-126); the arithmetic follows its f32
// CPU backend (src/backend/cpu/cpu_backend.cpp:34-39 rmsnorm, :155-172 the
// append loop, :262-272 rope) so that the f32 path reproduces it to the last
// bit almost everywhere.
//
// One wave64 per token and group of 8 heads: lane l serves head 8 * group +
// l / 8 and, of its 128 elements, the 8 from 8 * (l % 8) on and their rotary
// partners 64 elements further, so every access is 16 bytes wide and a wave
// moves 2 KiB (f16) per instruction pair. The angle's sine and cosine are
// evaluated in double once per frequency (lane f takes frequency f) and rounded
// once to f32, then shuffled to the lanes that use them; the sum of squares is
// taken in double (products of f32 values are exact in double), matching the
// CPU's double accumulator, in the same pairing order as the one-pair-per-lane
// form the fused decode step uses (elements 32 apart first, then 16, 8, 4, 2,
// 1), so both write bit-identical pages.
#include "device.hpp"
#include "kernels.hpp"

namespace ember::hip {
namespace {

constexpr int kWavesPerBlock = 4;
constexpr int kLanesPerHead = 8;
constexpr int kHeadsPerWave = kWave / kLanesPerHead;
constexpr int kElems = kHeadDim / 2 / kLanesPerHead;  // elements per lane in each half

// Eight elements as loaded (one 16-byte load for f16, two for f32), widened to
// f32 later, so that nothing waits for them where they are loaded.
template <typename T>
struct Raw8 {
    f16x8 v;
};
template <>
struct Raw8<float> {
    f32x4 lo, hi;
};

template <typename T>
__device__ __forceinline__ Raw8<T> load8(const T *src) {
    if constexpr (sizeof(T) == 2) {
        return Raw8<T>{*reinterpret_cast<const f16x8 *>(src)};
    } else {
        return Raw8<T>{*reinterpret_cast<const f32x4 *>(src), *reinterpret_cast<const f32x4 *>(src + 4)};
    }
}

template <typename T>
__device__ __forceinline__ void widen8(const Raw8<T> &r, float (&x)[kElems]) {
    if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int e = 0; e < kElems; e++) x[e] = static_cast<float>(r.v[e]);
    } else {
#pragma unroll
        for (int e = 0; e < 4; e++) x[e] = r.lo[e], x[e + 4] = r.hi[e];
    }
}

template <typename T, bool PAGE>
__device__ __forceinline__ void store8(T *dst, const float (&x)[kElems]) {
    if constexpr (sizeof(T) == 2) {
        f16x8 v;
#pragma unroll
        for (int e = 0; e < kElems; e++) v[e] = PAGE ? to_page<T>(x[e]) : from_f32<T>(x[e]);
        *reinterpret_cast<f16x8 *>(dst) = v;
    } else {
        *reinterpret_cast<f32x4 *>(dst) = f32x4{x[0], x[1], x[2], x[3]};
        *reinterpret_cast<f32x4 *>(dst + 4) = f32x4{x[4], x[5], x[6], x[7]};
    }
}

// The arguments that the first loads need come first and are preloaded into
// scalar registers at launch (build.py: -amdgpu-kernarg-preload-count=8), and
// every load that depends on nothing else goes out at once, unguarded (indices
// clamped into their arrays; a lane past the heads stores nothing): the
// token's position and sequence, this lane's frequency and the head's
// elements, then the page's block id, which needs the first two. The wave
// meets the memory's latency about twice instead of once per dependent load.
template <typename T>
__global__ void __launch_bounds__(kWavesPerBlock * kWave)
    kv_append_kernel(const int32_t *positions, const int32_t *token_seq, const float *inv_freq, const void *qkv,
                     const int32_t *block_tables, int n_heads, int n_kv, int max_blocks, EmberQkvArgs a) {
    constexpr int D = kHeadDim, HALF = D / 2;
    const int t = blockIdx.x;
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const int group = static_cast<int>(blockIdx.y) * kWavesPerBlock + static_cast<int>(threadIdx.x) / kWave;
    const int total = n_heads + 2 * n_kv;
    const int head = group * kHeadsPerWave + lane / kLanesPerHead;
    const int e0 = (lane % kLanesPerHead) * kElems;
    const bool live = head < total;

    // The frequency first: vector loads complete in issue order, so the angle's
    // sine and cosine can start before the head's elements arrive.
    const float freq = inv_freq[lane];
    __builtin_amdgcn_sched_barrier(0);
    const int pos = positions[t];
    const int seq = token_seq[t];
    const T *src = static_cast<const T *>(qkv) + (static_cast<int64_t>(t) * total + min(head, total - 1)) * D;
    const Raw8<T> r0 = load8(src + e0), r1 = load8(src + HALF + e0);
    __builtin_amdgcn_sched_barrier(0);
    const bool is_q = head < n_heads, is_k = !is_q && head < n_heads + n_kv;
    const int page = pos / kPage;
    const bool slot_ok = pos >= 0 && page < max_blocks;
    // The index is clamped into the row (a position outside the table stores nothing) and a negative
    // sequence reads row 0, so the load needs no branch: a select here made the compiler load the
    // sequence inside a branch, one more round trip.
    const int block =
        block_tables[static_cast<int64_t>(max(seq, 0)) * max_blocks + min(max(page, 0), max_blocks - 1)];
    // Taken here, while the head's elements are still in flight: left to itself the
    // compiler issued this load after the sine and cosine, where the shuffles' LDS
    // waits (lgkmcnt, which counts scalar loads too) then waited for it.
    __asm__ volatile("" ::"s"(block));

    // Sine and cosine of frequency `lane`, then the lane's own eight: they need
    // only the position and the frequency, so they run while the head's
    // elements are still in flight.
    const float angle = static_cast<float>(pos) * freq;
    double sd, cd;
    sincos(static_cast<double>(angle), &sd, &cd);
    const float s_f = static_cast<float>(sd), c_f = static_cast<float>(cd);
    float sn[kElems], cs[kElems];
#pragma unroll
    for (int e = 0; e < kElems; e++) sn[e] = __shfl(s_f, e0 + e, kWave), cs[e] = __shfl(c_f, e0 + e, kWave);

    float x0[kElems], x1[kElems];
    widen8(r0, x0);
    widen8(r1, x1);
    if (a.bias) {
        const float *b = a.bias + min(head, total - 1) * D;
#pragma unroll
        for (int e = 0; e < kElems; e++) x0[e] = x0[e] + b[e0 + e], x1[e] = x1[e] + b[HALF + e0 + e];
    }

    // Sum of squares over the head, every lane of the 8 taking part (the head
    // groups never mix): element bits 5, 4, 3 are lane bits 2, 1, 0; bits 2, 1, 0
    // are the register index.
    double ss[kElems];
#pragma unroll
    for (int e = 0; e < kElems; e++)
        ss[e] = static_cast<double>(x0[e]) * x0[e] + static_cast<double>(x1[e]) * x1[e];
#pragma unroll
    for (int o = kLanesPerHead / 2; o > 0; o >>= 1) {
#pragma unroll
        for (int e = 0; e < kElems; e++) ss[e] += __shfl_xor(ss[e], o, kLanesPerHead);
    }
#pragma unroll
    for (int o = kElems / 2; o > 0; o >>= 1) {
#pragma unroll
        for (int e = 0; e < o; e++) ss[e] += ss[e + o];
    }

    if (is_q || is_k) {
        const float *w = is_q ? a.q_norm : a.k_norm;
        if (w) {
            const float scale = static_cast<float>(1.0 / sqrt(ss[0] / kHeadDim + static_cast<double>(a.eps)));
#pragma unroll
            for (int e = 0; e < kElems; e++) {
                x0[e] = w[e0 + e] * (x0[e] * scale);
                x1[e] = w[HALF + e0 + e] * (x1[e] * scale);
            }
        }
#pragma unroll
        for (int e = 0; e < kElems; e++) {
            const float lo = x0[e], hi = x1[e];
            x0[e] = lo * cs[e] - hi * sn[e];
            x1[e] = hi * cs[e] + lo * sn[e];
        }
    }
    if (!live) return;

    if (is_q) {
        T *dst = static_cast<T *>(a.q_out) + (static_cast<int64_t>(t) * n_heads + head) * D;
        store8<T, false>(dst + e0, x0);
        store8<T, false>(dst + HALF + e0, x1);
        return;
    }
    const int kvh = is_k ? head - n_heads : head - n_heads - n_kv;
    if (!slot_ok || block < 0 || block >= a.num_blocks) return;  // never write outside the pool
    T *pool = static_cast<T *>(is_k ? a.k_cache : a.v_cache);
    T *dst = pool + ((static_cast<int64_t>(block) * n_kv + kvh) * kPage + pos % kPage) * D;
    store8<T, true>(dst + e0, x0);
    store8<T, true>(dst + HALF + e0, x1);
}

}  // namespace

hipError_t launch_kv_append(const EmberQkvArgs &a, hipStream_t stream) {
    if (a.T <= 0) return hipSuccess;
    const int groups = (a.n_heads + 2 * a.n_kv + kHeadsPerWave - 1) / kHeadsPerWave;
    const dim3 grid(static_cast<unsigned>(a.T), static_cast<unsigned>((groups + kWavesPerBlock - 1) / kWavesPerBlock));
    const dim3 block(kWavesPerBlock * kWave);
    if (a.dtype == EMBER_DTYPE_F16)
        hipLaunchKernelGGL(kv_append_kernel<f16>, grid, block, 0, stream, a.positions, a.token_seq, a.inv_freq, a.qkv,
                           a.block_tables, a.n_heads, a.n_kv, a.max_blocks, a);
    else
        hipLaunchKernelGGL(kv_append_kernel<float>, grid, block, 0, stream, a.positions, a.token_seq, a.inv_freq, a.qkv,
                           a.block_tables, a.n_heads, a.n_kv, a.max_blocks, a);
    return hipGetLastError();
}

}  // namespace ember::hip
