// The layer's linear layers either side of the paged-KV path on gfx950: the
// input RMSNorm, and decode-sized linear layers (the qkv projection that feeds
// the append, the output projection that adds attention into the residual).
//
// rmsnorm_rows_kernel replaces the reference's rmsnorm_kernel
// (src/backend/cuda/k_elementwise.cu:52-65) with the CPU backend's arithmetic
// (src/backend/cpu/cpu_backend.cpp:34-39): the sum of squares in double, the
// scale 1/sqrt(ss/n + eps) in double rounded once to f32, out = w * (x *
// scale), stored as f16 clamped to the finite range.
//
// gemv_kernel replaces gemv_tc_kernel (src/backend/cuda/k_gemm.cu:302-425):
// C[M, N] = A[M, K] . W[N, K]^T for M <= 64 with the same four epilogues. The
// time is spent streaming W once, so the kernel is built around its loads: a
// work-group owns 16 output features and its 8 waves split K, each wave
// issuing all of its W loads before its first MFMA. Per 32-wide k step one
// v_mfma_f32_16x16x32_f16 per 16-token tile takes W as the A operand (lane l:
// feature l % 16, k 8 (l / 16) .. + 7, one 16-byte load of a W row) and the
// activations as the B operand (lane l: token l % 16, the same k), so
// D = W X^T holds C^T: lane l ends with token l % 16 and features 4 (l / 16)
// + 0..3. The waves' partial sums meet in LDS and are added in wave order.
#include "device.hpp"
#include "kernels.hpp"

namespace ember::hip {
namespace {

constexpr int kGemvWaves = 8;
constexpr int kGemvThreads = kGemvWaves * kWave;
constexpr int kGemvUnroll = 8;  // k steps whose W loads are in flight together, per wave

__device__ __forceinline__ f16x8 load_w(const f16 *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const f16x8 *>(p));  // W is read once per launch
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

template <int MT, int EP>  // MT tiles of 16 tokens (M <= 16 MT); EP an EMBER_EPILOGUE_*
__global__ void __launch_bounds__(kGemvThreads) gemv_kernel(const f16 *__restrict__ A, int lda,
                                                            const f16 *__restrict__ W, int M, int N, int K,
                                                            void *__restrict__ C, int ldc) {
    __shared__ f32x4 red[kGemvWaves - 1][MT][kWave];
    const int lane = static_cast<int>(threadIdx.x) % kWave, wave = static_cast<int>(threadIdx.x) / kWave;
    const int c = lane % 16, g = lane / 16;
    const int n0 = static_cast<int>(blockIdx.x) * 16;
    const f16 *w = W + static_cast<int64_t>(min(n0 + c, N - 1)) * K + 8 * g;  // rows past N repeat the last
    const f16 *x[MT];
    bool xok[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int tok = 16 * mt + c;
        xok[mt] = tok < M;
        x[mt] = A + static_cast<int64_t>(min(tok, M - 1)) * lda + 8 * g;
    }
    f32x4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) acc[mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // Wave w takes k steps w, w + 8, ...; kGemvUnroll of them per round, every
    // W load of the round issued before its MFMAs.
    const int steps = K / 32;
    int s = wave;
    for (; s + (kGemvUnroll - 1) * kGemvWaves < steps; s += kGemvUnroll * kGemvWaves) {
        f16x8 wv[kGemvUnroll], xv[kGemvUnroll][MT];
#pragma unroll
        for (int u = 0; u < kGemvUnroll; u++) wv[u] = load_w(w + 32 * (s + u * kGemvWaves));
#pragma unroll
        for (int u = 0; u < kGemvUnroll; u++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
                xv[u][mt] = xok[mt] ? *reinterpret_cast<const f16x8 *>(x[mt] + 32 * (s + u * kGemvWaves)) : f16x8{};
#pragma unroll
        for (int u = 0; u < kGemvUnroll; u++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++) acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wv[u], xv[u][mt], acc[mt], 0, 0, 0);
    }
    for (; s < steps; s += kGemvWaves) {
        const f16x8 wv = load_w(w + 32 * s);
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const f16x8 xv = xok[mt] ? *reinterpret_cast<const f16x8 *>(x[mt] + 32 * s) : f16x8{};
            acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wv, xv, acc[mt], 0, 0, 0);
        }
    }

    if (wave > 0) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++) red[wave - 1][mt][lane] = acc[mt];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int v = 0; v < kGemvWaves - 1; v++) acc[mt] = acc[mt] + red[v][mt][lane];

    // acc[mt][i] = C[token 16 mt + c][feature n0 + 4 g + i].
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int tok = 16 * mt + c;
        if (tok >= M) continue;
        if constexpr (EP == EMBER_EPILOGUE_SILU_MUL) {
            // gate rows even, up rows odd: this lane holds the pairs (4g, 4g+1), (4g+2, 4g+3)
#pragma unroll
            for (int i = 0; i < 4; i += 2) {
                const int n = n0 + 4 * g + i;
                if (n + 1 < N)
                    static_cast<f16 *>(C)[static_cast<int64_t>(tok) * ldc + n / 2] =
                        static_cast<f16>(clamp_half(silu(acc[mt][i]) * acc[mt][i + 1]));
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int n = n0 + 4 * g + i;
                if (n >= N) continue;
                const int64_t at = static_cast<int64_t>(tok) * ldc + n;
                if constexpr (EP == EMBER_EPILOGUE_STORE_F16)
                    static_cast<f16 *>(C)[at] = static_cast<f16>(clamp_half(acc[mt][i]));
                else if constexpr (EP == EMBER_EPILOGUE_STORE_F32)
                    static_cast<float *>(C)[at] = acc[mt][i];
                else
                    static_cast<float *>(C)[at] += acc[mt][i];
            }
        }
    }
}

template <int EP>
hipError_t launch_gemv_ep(const EmberGemvArgs &a, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((a.N + 15) / 16));
    const f16 *A = static_cast<const f16 *>(a.A);
    const f16 *W = static_cast<const f16 *>(a.W);
    switch ((a.M + 15) / 16) {
        case 1: hipLaunchKernelGGL((gemv_kernel<1, EP>), grid, dim3(kGemvThreads), 0, stream, A, a.lda, W, a.M, a.N, a.K, a.C, a.ldc); break;
        case 2: hipLaunchKernelGGL((gemv_kernel<2, EP>), grid, dim3(kGemvThreads), 0, stream, A, a.lda, W, a.M, a.N, a.K, a.C, a.ldc); break;
        case 3: hipLaunchKernelGGL((gemv_kernel<3, EP>), grid, dim3(kGemvThreads), 0, stream, A, a.lda, W, a.M, a.N, a.K, a.C, a.ldc); break;
        case 4: hipLaunchKernelGGL((gemv_kernel<4, EP>), grid, dim3(kGemvThreads), 0, stream, A, a.lda, W, a.M, a.N, a.K, a.C, a.ldc); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

constexpr int kNormThreads = 256;

// One work-group per row: the sum of squares in double, reduced in a fixed
// order (each thread's stride, then the wave, then the waves in order).
__global__ void __launch_bounds__(kNormThreads) rmsnorm_rows_kernel(const float *__restrict__ x,
                                                                    const int32_t *__restrict__ rows, int hidden,
                                                                    const float *__restrict__ w, float eps,
                                                                    f16 *__restrict__ out) {
    __shared__ double part[kNormThreads / kWave];
    const int r = static_cast<int>(blockIdx.x);
    const float *xr = x + static_cast<int64_t>(rows ? rows[r] : r) * hidden;
    double ss = 0.0;
    for (int i = static_cast<int>(threadIdx.x); i < hidden; i += kNormThreads)
        ss += static_cast<double>(xr[i]) * xr[i];
    for (int o = kWave / 2; o > 0; o >>= 1) ss += __shfl_xor(ss, o, kWave);
    if (threadIdx.x % kWave == 0) part[threadIdx.x / kWave] = ss;
    __syncthreads();
    double total = part[0];
    for (int v = 1; v < kNormThreads / kWave; v++) total += part[v];
    const float scale = static_cast<float>(1.0 / sqrt(total / hidden + static_cast<double>(eps)));
    f16 *o = out + static_cast<int64_t>(r) * hidden;
    for (int i = static_cast<int>(threadIdx.x); i < hidden; i += kNormThreads)
        o[i] = static_cast<f16>(clamp_half(w[i] * (xr[i] * scale)));
}

}  // namespace

hipError_t launch_gemv(const EmberGemvArgs &a, hipStream_t stream) {
    switch (a.epilogue) {
        case EMBER_EPILOGUE_STORE_F16: return launch_gemv_ep<EMBER_EPILOGUE_STORE_F16>(a, stream);
        case EMBER_EPILOGUE_STORE_F32: return launch_gemv_ep<EMBER_EPILOGUE_STORE_F32>(a, stream);
        case EMBER_EPILOGUE_ADD_F32: return launch_gemv_ep<EMBER_EPILOGUE_ADD_F32>(a, stream);
        case EMBER_EPILOGUE_SILU_MUL: return launch_gemv_ep<EMBER_EPILOGUE_SILU_MUL>(a, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_rmsnorm_rows(const EmberNormArgs &a, hipStream_t stream) {
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(static_cast<unsigned>(a.R)), dim3(kNormThreads), 0, stream, a.x,
                       a.rows, a.hidden, a.w, a.eps, static_cast<f16 *>(a.out));
    return hipGetLastError();
}

}  // namespace ember::hip
