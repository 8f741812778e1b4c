// Device-side helpers shared by the gfx950 kernels of the paged-KV path.
//
// Everything here is written for CDNA4's 64-wide waves: cross-lane traffic
// inside a 16-lane row uses DPP (row/quad permutations folded into the VALU
// op), wider exchanges use ds_bpermute through __shfl_xor.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ember::hip {

constexpr int kPage = 16;         // tokens per KV page (kBlockSize)
constexpr int kHeadDim = 128;     // the only head_dim the kernels are built for
constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kHalfMax = 65504.0f;

using f16 = _Float16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// DPP move of a float (row_mask, bank_mask all on; every source lane exists
// for the quad / mirror / row broadcast patterns used here, so no lane keeps
// an old value and none needs initialising).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xf, 0xf, true));
}

constexpr int kDppQuadXor1 = 0xb1;     // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4e;     // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

// Sum over the 16 lanes of a DPP row; every lane of the row gets the same,
// bit-identical result (each step adds two values that both partner lanes
// hold, and float addition is commutative).
__device__ __forceinline__ float row16_sum(float x) {
    x = x + dpp_mov<kDppQuadXor1>(x);
    x = x + dpp_mov<kDppQuadXor2>(x);
    x = x + dpp_mov<kDppRowHalfMirror>(x);
    x = x + dpp_mov<kDppRowMirror>(x);
    return x;
}

__device__ __forceinline__ double wave_sum_f64(double x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, kWave);
    return x;
}

__device__ __forceinline__ float clamp_half(float x) { return fminf(fmaxf(x, -kHalfMax), kHalfMax); }

// QK-RMSNorm (optional) and rotate-half RoPE of one 128-dim head vector held
// by a wave64: lane l holds x0 = x[l] and x1 = x[l + 64], exactly one rotary
// pair. Follows the reference's f32 CPU backend (src/backend/cpu/cpu_backend.cpp
// :34-39 rmsnorm with a double sum of squares, :262-272 rope): the sum of
// squares is taken in double (f32 products are exact there), sine and cosine
// in double rounded once to f32, and the rest in f32 as the CPU writes it.
// Every lane of the wave must call it (the sum is a wave reduction).
// The lane's operands from memory, loadable ahead of the arithmetic: its two
// norm weights (unused without a norm) and its rotary frequency.
struct NormRopeLane {
    float w0, w1, inv_freq;
};

__device__ __forceinline__ NormRopeLane norm_rope_lane(const float *w, const float *inv_freq, int lane) {
    NormRopeLane n;
    n.w0 = w ? w[lane] : 1.0f;
    n.w1 = w ? w[lane + kHeadDim / 2] : 1.0f;
    n.inv_freq = inv_freq[lane];
    return n;
}

__device__ __forceinline__ void qk_norm_rope(float &x0, float &x1, bool norm, const NormRopeLane &n, float eps,
                                             int pos) {
    if (norm) {
        double ss = static_cast<double>(x0) * x0 + static_cast<double>(x1) * x1;
        ss = wave_sum_f64(ss);
        const float scale = static_cast<float>(1.0 / sqrt(ss / kHeadDim + static_cast<double>(eps)));
        x0 = n.w0 * (x0 * scale);
        x1 = n.w1 * (x1 * scale);
    }
    const float angle = static_cast<float>(pos) * n.inv_freq;
    double sd, cd;
    sincos(static_cast<double>(angle), &sd, &cd);
    const float s = static_cast<float>(sd), c = static_cast<float>(cd);
    const float lo = x0, hi = x1;
    x0 = lo * c - hi * s;
    x1 = hi * c + lo * s;
}

__device__ __forceinline__ void qk_norm_rope(float &x0, float &x1, const float *w, float eps, int pos,
                                             const float *inv_freq, int lane) {
    qk_norm_rope(x0, x1, w != nullptr, norm_rope_lane(w, inv_freq, lane), eps, pos);
}

// The value a K/V element is stored as: f16 pages clamp to the finite range
// first (as the reference's store does, k_elementwise.cu:125); f32 pages keep it.
template <typename T>
__device__ __forceinline__ T to_page(float x) {
    if constexpr (sizeof(T) == 2) return static_cast<T>(clamp_half(x));
    else return x;
}

// f16 <-> f32 element conversion for the templated (f16 / f32) kernels.
template <typename T>
__device__ __forceinline__ float to_f32(T x) {
    return static_cast<float>(x);
}
template <typename T>
__device__ __forceinline__ T from_f32(float x) {
    return static_cast<T>(x);  // f16: v_cvt_f16_f32, round to nearest even
}

}  // namespace ember::hip
