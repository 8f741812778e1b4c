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
//
// A launch wants one work-group per CU at least: with few features (N / 16
// below 256, e.g. the output projection's 2048), and a caller workspace, KS =
// 2 or 4 work-groups share each 16 features, each taking a K slice (grid y).
// Each stores its slice sum; the last to count in adds the KS sums in slice
// order and applies the epilogue. KS depends on N and K only.
#include <type_traits>

#include "device.hpp"
#include "kernels.hpp"

namespace ember::hip {
namespace {

constexpr int kGemvWaves = 8;
constexpr int kGemvThreads = kGemvWaves * kWave;
constexpr int kGemvUnroll = 8;  // k steps whose W loads are in flight together, per wave
constexpr int kGemvTargetGroups = 256;  // work-groups a launch should reach: one per CU
constexpr int kGemvMaxSplit = 4;
// Packed W (ember_hip_gemv_pack): for each 16-feature tile and 32-wide k step,
// the MFMA A operand as the 64 lanes take it, 8 halves per lane (lane 16 g + c:
// row 16 tile + c, k 32 step + 8 g ..): one contiguous 1 KiB per load
// instruction of a wave instead of 16 rows of 64 bytes. Rows past N are zero.
constexpr int kPackBlock = 64 * 8;  // halves per (tile, k step)

// Split slices are written and read with device-scope relaxed atomics (sc1
// global stores and loads on gfx950, coherent across the XCDs' L2s), under
// the same protocol as the decode kernel's split merge: each work-group waits
// for its slice stores (s_waitcnt vmcnt(0), then a barrier) before it counts
// in, and the merging work-group loads the slices only after its count has
// returned. So every slice counted before the last count is visible.
__device__ __forceinline__ void put_slice(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float get_slice(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ f16x8 load_w(const f16 *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const f16x8 *>(p));  // W is read once per launch
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// MT tiles of 16 tokens (M <= 16 MT); EP an EMBER_EPILOGUE_*; SPLIT: K split
// over gridDim.y work-groups (a separate instance, so the unsplit one keeps
// its constant-stride loads and no merge code).
template <int MT, int EP, bool SPLIT, bool PACKED>
__global__ void __launch_bounds__(kGemvThreads) gemv_kernel(const f16 *__restrict__ A, int lda,
                                                            const f16 *__restrict__ W, int M, int N, int K,
                                                            void *__restrict__ C, int ldc,
                                                            float *__restrict__ slices, uint32_t *__restrict__ counters) {
    __shared__ f32x4 red[kGemvWaves - 1][MT][kWave];
    __shared__ int merge_here;
    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid % kWave, wave = tid / kWave;
    const int c = lane % 16, g = lane / 16;
    const int fb = static_cast<int>(blockIdx.x), nfb = static_cast<int>(gridDim.x);
    const int ks = SPLIT ? static_cast<int>(blockIdx.y) : 0, KS = SPLIT ? static_cast<int>(gridDim.y) : 1;
    const int n0 = fb * 16;
    const int k0 = ks * (K / KS);  // this work-group's K slice: K / KS, a multiple of 32
    // Row-major W: this lane's row (rows past N repeat the last), k step s at
    // +32 s. Packed W: the tile's k steps are 1 KiB blocks in lane order.
    const f16 *w = PACKED ? W + (static_cast<int64_t>(fb) * (K / 32) + k0 / 32) * kPackBlock + 8 * lane
                          : W + static_cast<int64_t>(min(n0 + c, N - 1)) * K + k0 + 8 * g;
    constexpr int wstep = PACKED ? kPackBlock : 32;  // halves per k step
    const f16 *x[MT];
    bool xok[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int tok = 16 * mt + c;
        xok[mt] = tok < M;
        x[mt] = A + static_cast<int64_t>(min(tok, M - 1)) * lda + k0 + 8 * g;
    }
    f32x4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) acc[mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // Up to kGemvUnroll k steps per round, every W load of the round issued
    // before its MFMAs.
    auto round = [&](auto unroll, int s0, int stride) {
        constexpr int U = decltype(unroll)::value;
        f16x8 wv[U], xv[U][MT];
#pragma unroll
        for (int u = 0; u < U; u++) wv[u] = load_w(w + wstep * (s0 + u * stride));
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
                xv[u][mt] = xok[mt] ? *reinterpret_cast<const f16x8 *>(x[mt] + 32 * (s0 + u * stride)) : f16x8{};
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++) acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wv[u], xv[u][mt], acc[mt], 0, 0, 0);
    };
    using Full = std::integral_constant<int, kGemvUnroll>;
    using Half = std::integral_constant<int, kGemvUnroll / 2>;
    // A tail of n = 1..4 steps (wave-uniform) as one round of exactly n: the
    // same steps in the same order, their loads issued together. (A form with
    // every step of the round guarded by u < n, its unused operands left
    // unset, gave wrong sums in one accumulator element of some lanes at 4-way
    // splits; rounds of a fixed size have no guarded MFMAs.)
    auto tail = [&](int s0, int stride, int n) {
        switch (n) {
            case 1: round(std::integral_constant<int, 1>{}, s0, stride); break;
            case 2: round(std::integral_constant<int, 2>{}, s0, stride); break;
            case 3: round(std::integral_constant<int, 3>{}, s0, stride); break;
            default: round(Half{}, s0, stride); break;
        }
    };
    const int steps = K / KS / 32;
    if constexpr (SPLIT) {
        // A slice has few steps per wave: each wave takes a contiguous run, so
        // its consecutive loads read whole 128-byte lines of W.
        int s = wave * steps / kGemvWaves;
        const int end = (wave + 1) * steps / kGemvWaves;
        for (; s + kGemvUnroll <= end; s += kGemvUnroll) round(Full{}, s, 1);
        if (s + kGemvUnroll / 2 <= end) {
            round(Half{}, s, 1);
            s += kGemvUnroll / 2;
        }
        if (s < end) tail(s, 1, end - s);
    } else {
        // Wave w takes k steps w, w + 8, ...
        int s = wave;
        for (; s + (kGemvUnroll - 1) * kGemvWaves < steps; s += kGemvUnroll * kGemvWaves) round(Full{}, s, kGemvWaves);
        for (int left = (steps - s + kGemvWaves - 1) / kGemvWaves; left > 0;) {
            const int n = min(left, kGemvUnroll / 2);
            tail(s, kGemvWaves, n);
            s += n * kGemvWaves;
            left -= n;
        }
    }

    if (wave > 0) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++) red[wave - 1][mt][lane] = acc[mt];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int v = 0; v < kGemvWaves - 1; v++) acc[mt] = acc[mt] + red[v][mt][lane];
    }
    if constexpr (SPLIT) {
        // Slice sums: [ks][fb][mt][element i][lane], one 256-byte row per store.
        auto slice = [&](int q, int mt) { return slices + ((static_cast<int64_t>(q) * nfb + fb) * MT + mt) * 256 + lane; };
        if (wave == 0) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int i = 0; i < 4; i++) put_slice(slice(ks, mt) + 64 * i, acc[mt][i]);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) {
            const uint32_t before = __hip_atomic_fetch_add(counters + fb, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            merge_here = before + 1 == static_cast<uint32_t>(KS);
            if (merge_here) __hip_atomic_store(counters + fb, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!merge_here || wave != 0) return;
        // The slices in slice order, this work-group's own included, so the sum
        // does not depend on which work-group merges.
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            float part[kGemvMaxSplit][4];
#pragma unroll
            for (int q = 0; q < kGemvMaxSplit; q++)
#pragma unroll
                for (int i = 0; i < 4; i++) part[q][i] = q < KS ? get_slice(slice(q, mt) + 64 * i) : 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float t = part[0][i];
#pragma unroll
                for (int q = 1; q < kGemvMaxSplit; q++)
                    if (q < KS) t += part[q][i];
                acc[mt][i] = t;
            }
        }
    } else if (wave != 0) {
        return;
    }

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

// Very wide launches (an LM head's 151,936 features) at up to 16 tokens: each
// work-group takes kWideTiles 16-feature tiles that share every activation
// load, so the launch runs a quarter of the work-groups, each with four times
// the W loads in flight. Per tile the arithmetic is gemv_kernel's (the same k
// steps per wave in the same order, the waves summed in wave order), so the
// results are the same bits.
constexpr int kWideTiles = 4;
constexpr int kWideMinTiles = 4096;  // 16-feature tiles at which a launch goes wide

template <int EP, bool PACKED>
__global__ void __launch_bounds__(kGemvThreads) gemv_wide_kernel(const f16 *__restrict__ A, int lda,
                                                                 const f16 *__restrict__ W, int M, int N, int K,
                                                                 void *__restrict__ C, int ldc) {
    __shared__ f32x4 red[kGemvWaves - 1][kWideTiles][kWave];
    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid % kWave, wave = tid / kWave;
    const int c = lane % 16, g = lane / 16;
    const int n0 = static_cast<int>(blockIdx.x) * 16 * kWideTiles;
    const f16 *w[kWideTiles];
#pragma unroll
    for (int f = 0; f < kWideTiles; f++)
        w[f] = PACKED ? W + static_cast<int64_t>(min(n0 / 16 + f, (N + 15) / 16 - 1)) * (K / 32) * kPackBlock + 8 * lane
                      : W + static_cast<int64_t>(min(n0 + 16 * f + c, N - 1)) * K + 8 * g;
    constexpr int wstep = PACKED ? kPackBlock : 32;
    const bool xok = c < M;
    const f16 *x = A + static_cast<int64_t>(min(c, M - 1)) * lda + 8 * g;
    f32x4 acc[kWideTiles];
#pragma unroll
    for (int f = 0; f < kWideTiles; f++) acc[f] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // Wave w takes k steps w, w + 8, ..., up to four per round.
    auto round = [&](auto unroll, int s0) {
        constexpr int U = decltype(unroll)::value;
        f16x8 wv[U][kWideTiles], xv[U];
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int f = 0; f < kWideTiles; f++) wv[u][f] = load_w(w[f] + wstep * (s0 + u * kGemvWaves));
#pragma unroll
        for (int u = 0; u < U; u++)
            xv[u] = xok ? *reinterpret_cast<const f16x8 *>(x + 32 * (s0 + u * kGemvWaves)) : f16x8{};
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int f = 0; f < kWideTiles; f++) acc[f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wv[u][f], xv[u], acc[f], 0, 0, 0);
    };
    const int steps = K / 32;
    int s = wave;
    for (; s + 3 * kGemvWaves < steps; s += 4 * kGemvWaves) round(std::integral_constant<int, 4>{}, s);
    switch ((steps - s + kGemvWaves - 1) / kGemvWaves) {
        case 1: round(std::integral_constant<int, 1>{}, s); break;
        case 2: round(std::integral_constant<int, 2>{}, s); break;
        case 3: round(std::integral_constant<int, 3>{}, s); break;
        default: break;
    }

    if (wave > 0) {
#pragma unroll
        for (int f = 0; f < kWideTiles; f++) red[wave - 1][f][lane] = acc[f];
    }
    __syncthreads();
    if (wave != 0 || !xok) return;
#pragma unroll
    for (int f = 0; f < kWideTiles; f++) {
#pragma unroll
        for (int v = 0; v < kGemvWaves - 1; v++) acc[f] = acc[f] + red[v][f][lane];
        // acc[f][i] = C[token c][feature n0 + 16 f + 4 g + i].
        if constexpr (EP == EMBER_EPILOGUE_SILU_MUL) {
#pragma unroll
            for (int i = 0; i < 4; i += 2) {
                const int n = n0 + 16 * f + 4 * g + i;
                if (n + 1 < N)
                    static_cast<f16 *>(C)[static_cast<int64_t>(c) * ldc + n / 2] =
                        static_cast<f16>(clamp_half(silu(acc[f][i]) * acc[f][i + 1]));
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int n = n0 + 16 * f + 4 * g + i;
                if (n >= N) continue;
                const int64_t at = static_cast<int64_t>(c) * ldc + n;
                if constexpr (EP == EMBER_EPILOGUE_STORE_F16)
                    static_cast<f16 *>(C)[at] = static_cast<f16>(clamp_half(acc[f][i]));
                else if constexpr (EP == EMBER_EPILOGUE_STORE_F32)
                    static_cast<float *>(C)[at] = acc[f][i];
                else
                    static_cast<float *>(C)[at] += acc[f][i];
            }
        }
    }
}

// Work-groups per 16 features: doubled while the launch has fewer than
// kGemvTargetGroups and each slice keeps at least one 32-wide k step per wave.
int gemv_split(int N, int K) {
    const int nfb = (N + 15) / 16;
    int ks = 1;
    while (ks < kGemvMaxSplit && nfb * ks < kGemvTargetGroups && K % (2 * ks * 32) == 0 &&
           K / (2 * ks) >= 32 * kGemvWaves)
        ks *= 2;
    return ks;
}

// Workspace of a split launch: the merge counters (one per 16 features,
// padded to 256 bytes), then the slice sums.
int64_t gemv_workspace(int M, int N, int K) {
    const int ks = gemv_split(N, K);
    if (ks == 1) return 0;
    const int64_t nfb = (N + 15) / 16, mt = (M + 15) / 16;
    return (nfb * 4 + 255) / 256 * 256 + ks * nfb * mt * 256 * 4;
}

template <int EP>
hipError_t launch_gemv_ep(const EmberGemvArgs &a, hipStream_t stream) {
    const int64_t need = gemv_workspace(a.M, a.N, a.K);
    const bool split = need > 0 && a.workspace && a.workspace_bytes >= need;
    const int nfb = (a.N + 15) / 16;
    const dim3 grid(static_cast<unsigned>(nfb), static_cast<unsigned>(split ? gemv_split(a.N, a.K) : 1));
    uint32_t *counters = split ? static_cast<uint32_t *>(a.workspace) : nullptr;
    float *slices = split ? reinterpret_cast<float *>(static_cast<char *>(a.workspace) + (nfb * 4 + 255) / 256 * 256)
                          : nullptr;
    const f16 *A = static_cast<const f16 *>(a.A);
    const f16 *W = static_cast<const f16 *>(a.W);
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, dim3(kGemvThreads), 0, stream, A, a.lda, W, a.M, a.N, a.K, a.C, a.ldc, slices,
                           counters);
        return hipGetLastError();
    };
    if (!split && a.M <= 16 && nfb >= kWideMinTiles) {
        const dim3 wide(static_cast<unsigned>((nfb + kWideTiles - 1) / kWideTiles));
        if (a.w_packed)
            hipLaunchKernelGGL((gemv_wide_kernel<EP, true>), wide, dim3(kGemvThreads), 0, stream, A, a.lda, W, a.M, a.N,
                               a.K, a.C, a.ldc);
        else
            hipLaunchKernelGGL((gemv_wide_kernel<EP, false>), wide, dim3(kGemvThreads), 0, stream, A, a.lda, W, a.M, a.N,
                               a.K, a.C, a.ldc);
        return hipGetLastError();
    }
    switch ((a.M + 15) / 16 + (split ? 4 : 0) + (a.w_packed ? 8 : 0)) {
        case 1: return go(gemv_kernel<1, EP, false, false>);
        case 2: return go(gemv_kernel<2, EP, false, false>);
        case 3: return go(gemv_kernel<3, EP, false, false>);
        case 4: return go(gemv_kernel<4, EP, false, false>);
        case 5: return go(gemv_kernel<1, EP, true, false>);
        case 6: return go(gemv_kernel<2, EP, true, false>);
        case 7: return go(gemv_kernel<3, EP, true, false>);
        case 8: return go(gemv_kernel<4, EP, true, false>);
        case 9: return go(gemv_kernel<1, EP, false, true>);
        case 10: return go(gemv_kernel<2, EP, false, true>);
        case 11: return go(gemv_kernel<3, EP, false, true>);
        case 12: return go(gemv_kernel<4, EP, false, true>);
        case 13: return go(gemv_kernel<1, EP, true, true>);
        case 14: return go(gemv_kernel<2, EP, true, true>);
        case 15: return go(gemv_kernel<3, EP, true, true>);
        case 16: return go(gemv_kernel<4, EP, true, true>);
        default: return hipErrorInvalidValue;
    }
}

// One thread per 16-byte piece of packed W: piece q is lane q % 64 of k step
// (q / 64) % (K / 32) of tile q / (64 K / 32).
__global__ void __launch_bounds__(256) gemv_pack_kernel(const f16 *__restrict__ W, int N, int K, int64_t pieces,
                                                        f16 *__restrict__ out) {
    const int64_t q = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (q >= pieces) return;
    const int lane = static_cast<int>(q % 64);
    const int64_t ks = K / 32, step = (q / 64) % ks, tile = q / (64 * ks);
    const int64_t row = 16 * tile + lane % 16;
    f16x8 v = {};
    if (row < N) v = *reinterpret_cast<const f16x8 *>(W + row * K + 32 * step + 8 * (lane / 16));
    *reinterpret_cast<f16x8 *>(out + 8 * q) = v;
}

constexpr int kNormThreads = 256;
constexpr int kNormPer = 16;  // elements of a row per thread held in registers (hidden <= 4096)

// One work-group per row: the sum of squares in double, reduced in a fixed
// order (each thread's elements t, t + 256, ..., then the wave, then the
// waves in order). Rows up to kNormThreads * kNormPer wide keep the thread's
// elements of x and w in registers, all loaded up front: one memory round
// trip per row instead of one for x and another for w and x again.
template <bool HELD>
__global__ void __launch_bounds__(kNormThreads) rmsnorm_rows_kernel(const float *__restrict__ x,
                                                                    const int32_t *__restrict__ rows, int hidden,
                                                                    const float *__restrict__ w, float eps,
                                                                    f16 *__restrict__ out) {
    __shared__ double part[kNormThreads / kWave];
    const int r = static_cast<int>(blockIdx.x), t = static_cast<int>(threadIdx.x);
    const float *xr = x + static_cast<int64_t>(rows ? rows[r] : r) * hidden;
    f16 *o = out + static_cast<int64_t>(r) * hidden;
    float xv[HELD ? kNormPer : 1], wv[HELD ? kNormPer : 1];
    double ss = 0.0;
    if constexpr (HELD) {
#pragma unroll
        for (int j = 0; j < kNormPer; j++) {
            const int i = t + j * kNormThreads;
            xv[j] = i < hidden ? xr[i] : 0.0f;
            wv[j] = i < hidden ? w[i] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < kNormPer; j++) ss += static_cast<double>(xv[j]) * xv[j];  // + 0.0 past the row: exact
    } else {
        for (int i = t; i < hidden; i += kNormThreads) ss += static_cast<double>(xr[i]) * xr[i];
    }
    for (int off = kWave / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off, kWave);
    if (t % kWave == 0) part[t / kWave] = ss;
    __syncthreads();
    double total = part[0];
    for (int v = 1; v < kNormThreads / kWave; v++) total += part[v];
    const float scale = static_cast<float>(1.0 / sqrt(total / hidden + static_cast<double>(eps)));
    if constexpr (HELD) {
#pragma unroll
        for (int j = 0; j < kNormPer; j++) {
            const int i = t + j * kNormThreads;
            if (i < hidden) o[i] = static_cast<f16>(clamp_half(wv[j] * (xv[j] * scale)));
        }
    } else {
        for (int i = t; i < hidden; i += kNormThreads) o[i] = static_cast<f16>(clamp_half(w[i] * (xr[i] * scale)));
    }
}

}  // namespace

int64_t gemv_workspace_bytes(int M, int N, int K) { return gemv_workspace(M, N, K); }

int64_t gemv_packed_bytes(int N, int K) { return static_cast<int64_t>((N + 15) / 16) * 16 * K * 2; }

hipError_t launch_gemv_pack(const void *W, int N, int K, void *out, hipStream_t stream) {
    const int64_t pieces = static_cast<int64_t>((N + 15) / 16) * (K / 32) * 64;
    hipLaunchKernelGGL(gemv_pack_kernel, dim3(static_cast<unsigned>((pieces + 255) / 256)), dim3(256), 0, stream,
                       static_cast<const f16 *>(W), N, K, pieces, static_cast<f16 *>(out));
    return hipGetLastError();
}

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
    if (a.hidden <= kNormThreads * kNormPer)
        hipLaunchKernelGGL(rmsnorm_rows_kernel<true>, dim3(static_cast<unsigned>(a.R)), dim3(kNormThreads), 0, stream,
                           a.x, a.rows, a.hidden, a.w, a.eps, static_cast<f16 *>(a.out));
    else
        hipLaunchKernelGGL(rmsnorm_rows_kernel<false>, dim3(static_cast<unsigned>(a.R)), dim3(kNormThreads), 0, stream,
                           a.x, a.rows, a.hidden, a.w, a.eps, static_cast<f16 *>(a.out));
    return hipGetLastError();
}

}  // namespace ember::hip
