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
#include <algorithm>
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
constexpr int kGemvSplitAbove = 4096;  // K slices at most this wide are not split further
// A staged first round's W loads issued before its activation copies: one
// for a single 16-token tile (8 KiB of copies per wave at K 2048), two for
// more (16 KiB at two tiles). Measured at K 2048: qkv (two tiles) 6.32 us
// with none, 6.14 with one, 5.96 with two, 6.02 with three, 6.20 with four;
// o (one tile) 4.70, 4.65, 4.71, 4.77, 4.83.
constexpr int gemv_early_w(int mt) { return mt == 1 ? 1 : 2; }
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

// Activations staged in LDS (when the launcher passes staged): the
// work-group's rows of A over its K slice, copied by buffer_load_dwordx4 ...
// lds, each load writing 1 KiB of LDS (lane l's 16 bytes at 16 l). Slot t
// (16 bytes) holds piece (t % P) ^ (r & 15) of row r = t / P, P = 16-byte
// pieces per row (a multiple of 16). Every global load then reads whole
// 128-byte lines of consecutive pieces; read straight from A, a wave's
// operand load reads 64 bytes from each of 16 rows, 4 KiB apart at K = 2048,
// and the qkv projection at 32 tokens took 9.4 instead of 7.1 us. The operand
// read of step s (row 16 mt + c, piece 4 s + g) is one ds_read_b128 whose 16
// lanes of a given g hit 16 different slots modulo 16: no bank conflicts.
// Rows past M read as zeros (offsets past the descriptor's records).
constexpr int kGemvMaxStage = 128 * 1024;  // bytes of staged activations a work-group may hold
constexpr int kGemvRedBytes = kGemvWaves * kWave * 16;  // one f32x4 per lane and wave, per 16-token tile
constexpr int kDescWord3 = 0x00020000;  // gfx9 raw buffer: 32-bit data format, no swizzle

// MT tiles of 16 tokens (M <= 16 MT); EP an EMBER_EPILOGUE_*; SPLIT: K split
// over gridDim.y work-groups (a separate instance, so the unsplit one keeps
// its constant-stride loads and no merge code). Dynamic LDS: the staged
// activations (staged) or nothing, and afterwards the waves' partial sums.
template <int MT, int EP, bool SPLIT, bool PACKED, bool STAGED>
__global__ void __launch_bounds__(kGemvThreads) gemv_kernel(const f16 *__restrict__ A, int lda,
                                                            const f16 *__restrict__ W, int M, int N, int K,
                                                            void *__restrict__ C, int ldc,
                                                            uint32_t piece_magic, float *__restrict__ slices,
                                                            uint32_t *__restrict__ counters) {
    extern __shared__ __align__(16) unsigned char gemv_lds[];
    constexpr bool staged = STAGED;
    __shared__ int merge_here;
    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid % kWave, wave = tid / kWave;
    const int c = lane % 16, g = lane / 16;
    const int fb = static_cast<int>(blockIdx.x), nfb = static_cast<int>(gridDim.x);
    const int ks = SPLIT ? static_cast<int>(blockIdx.y) : 0, KS = SPLIT ? static_cast<int>(gridDim.y) : 1;
    const int n0 = fb * 16;
    // An unsplit launch may give its work-groups one group of MT token tiles
    // each (blockIdx.z): rows 16 MT z ... of A and C. A row's arithmetic does
    // not depend on the group, so the bits are those of one wider group.
    if constexpr (!SPLIT) {
        const int m0 = 16 * MT * static_cast<int>(blockIdx.z);
        constexpr int out_bytes = EP == EMBER_EPILOGUE_STORE_F32 || EP == EMBER_EPILOGUE_ADD_F32 ? 4 : 2;
        A += static_cast<int64_t>(m0) * lda;
        C = static_cast<char *>(C) + static_cast<int64_t>(m0) * ldc * out_bytes;
        M -= m0;
    }
    const int kw = K / KS, k0 = ks * kw;  // this work-group's K slice, a multiple of 32 wide
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
    const uint32_t pieces = kw / 8;  // 16-byte pieces per staged row
    // The f32 residual this work-group's epilogue adds to, read now so that
    // its latency hides behind the W loads (wave mt ends with token tile mt).
    // A lane's four outputs (features n0 + 4 g .. + 3 of one token) are
    // adjacent: with a 16-byte aligned C, ldc a multiple of 4 and the whole
    // tile inside N, they go out as one store (and come in as one load).
    const bool vec_out = ((reinterpret_cast<uintptr_t>(C) & 15) | (ldc & 3)) == 0 && n0 + 16 <= N;
    f32x4 prev = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (EP == EMBER_EPILOGUE_ADD_F32) {
        const int tok = 16 * wave + c;
        if (wave < MT && tok < M) {
            const float *row = static_cast<const float *>(C) + static_cast<int64_t>(tok) * ldc;
            if (vec_out) {
                prev = *reinterpret_cast<const f32x4 *>(row + n0 + 4 * g);
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int n = n0 + 4 * g + i;
                    if (n < N) prev[i] = row[n];
                }
            }
        }
    }
    f32x4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) acc[mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // The MFMAs of U k steps s0, s0 + stride, ... whose W operands are in wv,
    // with the activations from LDS (staged) or from A.
    auto compute = [&](auto unroll, const f16x8 *wv, int s0, int stride) {
        constexpr int U = decltype(unroll)::value;
        f16x8 xv[U][MT];
        if constexpr (staged) {
#pragma unroll
            for (int u = 0; u < U; u++)
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    const uint32_t r = 16 * mt + c, q = 4 * (s0 + u * stride) + g;
                    xv[u][mt] = *reinterpret_cast<const f16x8 *>(gemv_lds + 16 * (r * pieces + (q ^ (r & 15u))));
                }
        } else {
#pragma unroll
            for (int u = 0; u < U; u++)
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
                    xv[u][mt] = xok[mt] ? *reinterpret_cast<const f16x8 *>(x[mt] + 32 * (s0 + u * stride)) : f16x8{};
        }
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++) acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wv[u], xv[u][mt], acc[mt], 0, 0, 0);
    };
    // One round: U k steps, every W load issued before the MFMAs.
    auto round = [&](auto unroll, int s0, int stride) {
        constexpr int U = decltype(unroll)::value;
        f16x8 wv[U];
#pragma unroll
        for (int u = 0; u < U; u++) wv[u] = load_w(w + wstep * (s0 + u * stride));
        compute(unroll, wv, s0, stride);
    };
    using Full = std::integral_constant<int, kGemvUnroll>;
    using Half = std::integral_constant<int, kGemvUnroll / 2>;
    // A round of n = 1..4 steps (wave-uniform) as one round of exactly n: the
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
    // This wave's k steps (local to the slice): unsplit, w, w + 8, ...; split,
    // a contiguous run, so its consecutive loads read whole 128-byte lines of
    // a row-major W. A wave accumulates its steps in that order whatever the
    // rounds they are issued in, so the rounds do not change the sums.
    const int steps = kw / 32;
    const int stride = SPLIT ? 1 : kGemvWaves;
    int s = SPLIT ? wave * steps / kGemvWaves : wave;
    int left = SPLIT ? (wave + 1) * steps / kGemvWaves - s : (steps - wave + kGemvWaves - 1) / kGemvWaves;
    // The first round has the same size in every wave (8 when every wave has
    // 8 steps, else up to 4 and at most the fewest any wave has: steps / 8 in
    // both schemes), so it and the staging barrier inside it are uniform
    // across the work-group. The copies into LDS go out first, then the
    // round's W loads; the wave then waits for its copies only (vector memory
    // operations complete in issue order), so the W loads stay in flight
    // across the barrier. The barrier orders LDS alone (the copies are
    // already complete), so it does not wait for them either.
    auto issue_stage = [&]() {
        const uint32_t records = static_cast<uint32_t>((static_cast<int64_t>(M - 1) * lda + K) * 2);
        const __amdgpu_buffer_rsrc_t d = __builtin_amdgcn_make_buffer_rsrc(const_cast<f16 *>(A), 0, records, kDescWord3);
        const int blocks = 16 * MT * pieces / 64;
        for (int b = wave; b < blocks; b += kGemvWaves) {
            // slot t = r * pieces + q': r = t / pieces by one multiply-high
            // (exact here: t * pieces < 2^32)
            const uint32_t t = 64u * b + lane, r = __umulhi(t, piece_magic);
            const uint32_t q = (t - r * pieces) ^ (r & 15u);
            const uint32_t off = static_cast<int>(r) < M ? (r * lda + k0 + 8 * q) * 2 : records;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(d, (__attribute__((address_space(3))) void *)(gemv_lds + 1024 * b), 16,
                                                     off, 0, 0, 0);
        }
    };
    auto stage_barrier = [&]() {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    };
    auto first_round = [&](auto unroll) {
        constexpr int U = decltype(unroll)::value;
        constexpr int E = staged ? (U < gemv_early_w(MT) ? U : gemv_early_w(MT)) : 0;  // W loads ahead of the copies
        f16x8 wv[U];
#pragma unroll
        for (int u = 0; u < E; u++) wv[u] = load_w(w + wstep * (s + u * stride));
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (staged) issue_stage();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = E; u < U; u++) wv[u] = load_w(w + wstep * (s + u * stride));
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (staged) {
            // s_waitcnt vmcnt(U - E), expcnt and lgkmcnt left alone: every
            // copy (issued before the last U - E W loads) has landed
            __builtin_amdgcn_s_waitcnt(0x0F70 | (U - E));
            stage_barrier();
        }
        compute(unroll, wv, s, stride);
    };
    const int least = steps / kGemvWaves;
    const int first = least >= kGemvUnroll ? kGemvUnroll : min(least, kGemvUnroll / 2);
    switch (first) {
        case kGemvUnroll: first_round(Full{}); break;
        case 4: first_round(Half{}); break;
        case 3: first_round(std::integral_constant<int, 3>{}); break;
        case 2: first_round(std::integral_constant<int, 2>{}); break;
        case 1: first_round(std::integral_constant<int, 1>{}); break;
        default:
            if constexpr (staged) {
                issue_stage();
                __builtin_amdgcn_s_waitcnt(0);
                stage_barrier();
            }
            break;
    }
    s += first * stride;
    left -= first;
    for (; left >= kGemvUnroll; left -= kGemvUnroll, s += kGemvUnroll * stride) round(Full{}, s, stride);
    while (left > 0) {
        const int n = min(left, kGemvUnroll / 2);
        tail(s, stride, n);
        s += n * stride;
        left -= n;
    }

    // The waves' partial sums meet in LDS (over the staged activations, once
    // every wave is done with them); wave mt adds token tile mt's in wave order.
    f32x4 *red = reinterpret_cast<f32x4 *>(gemv_lds);  // [wave][mt][lane]
    if constexpr (staged) __syncthreads();
#pragma unroll
    for (int mt = 0; mt < MT; mt++) red[(wave * MT + mt) * kWave + lane] = acc[mt];
    __syncthreads();
    const int mt = wave;
    f32x4 sum = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (mt < MT) {
        sum = red[mt * kWave + lane];
#pragma unroll
        for (int v = 1; v < kGemvWaves; v++) sum = sum + red[(v * MT + mt) * kWave + lane];
    }
    if constexpr (SPLIT) {
        // Slice sums: [ks][fb][mt][element i][lane], one 256-byte row per store.
        auto slice = [&](int q) { return slices + ((static_cast<int64_t>(q) * nfb + fb) * MT + mt) * 256 + lane; };
        if (mt < MT) {
#pragma unroll
            for (int i = 0; i < 4; i++) put_slice(slice(ks) + 64 * i, sum[i]);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) {
            const uint32_t before = __hip_atomic_fetch_add(counters + fb, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            merge_here = before + 1 == static_cast<uint32_t>(KS);
            if (merge_here) __hip_atomic_store(counters + fb, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!merge_here || mt >= MT) return;
        // The slices in slice order, this work-group's own included, so the sum
        // does not depend on which work-group merges.
        float part[kGemvMaxSplit][4];
#pragma unroll
        for (int q = 0; q < kGemvMaxSplit; q++)
#pragma unroll
            for (int i = 0; i < 4; i++) part[q][i] = q < KS ? get_slice(slice(q) + 64 * i) : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float t = part[0][i];
#pragma unroll
            for (int q = 1; q < kGemvMaxSplit; q++)
                if (q < KS) t += part[q][i];
            sum[i] = t;
        }
    } else if (mt >= MT) {
        return;
    }

    // sum[i] = C[token 16 mt + c][feature n0 + 4 g + i].
    const int tok = 16 * mt + c;
    if (tok >= M) return;
    if constexpr (EP == EMBER_EPILOGUE_SILU_MUL) {
        // gate rows even, up rows odd: this lane holds the pairs (4g, 4g+1), (4g+2, 4g+3),
        // whose outputs are adjacent: one 4-byte store when vec_out holds
        if (vec_out) {
            const f16x2 h = {static_cast<f16>(clamp_half(silu(sum[0]) * sum[1])),
                             static_cast<f16>(clamp_half(silu(sum[2]) * sum[3]))};
            *reinterpret_cast<f16x2 *>(static_cast<f16 *>(C) + static_cast<int64_t>(tok) * ldc + (n0 + 4 * g) / 2) = h;
            return;
        }
#pragma unroll
        for (int i = 0; i < 4; i += 2) {
            const int n = n0 + 4 * g + i;
            if (n + 1 < N)
                static_cast<f16 *>(C)[static_cast<int64_t>(tok) * ldc + n / 2] =
                    static_cast<f16>(clamp_half(silu(sum[i]) * sum[i + 1]));
        }
    } else if (vec_out) {
        const int64_t at = static_cast<int64_t>(tok) * ldc + n0 + 4 * g;
        if constexpr (EP == EMBER_EPILOGUE_STORE_F16) {
            f16x4 h;
#pragma unroll
            for (int i = 0; i < 4; i++) h[i] = static_cast<f16>(clamp_half(sum[i]));
            *reinterpret_cast<f16x4 *>(static_cast<f16 *>(C) + at) = h;
        } else if constexpr (EP == EMBER_EPILOGUE_STORE_F32) {
            *reinterpret_cast<f32x4 *>(static_cast<float *>(C) + at) = sum;
        } else {
            *reinterpret_cast<f32x4 *>(static_cast<float *>(C) + at) = prev + sum;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = n0 + 4 * g + i;
            if (n >= N) continue;
            const int64_t at = static_cast<int64_t>(tok) * ldc + n;
            if constexpr (EP == EMBER_EPILOGUE_STORE_F16)
                static_cast<f16 *>(C)[at] = static_cast<f16>(clamp_half(sum[i]));
            else if constexpr (EP == EMBER_EPILOGUE_STORE_F32)
                static_cast<float *>(C)[at] = sum[i];
            else
                static_cast<float *>(C)[at] = prev[i] + sum[i];
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
// kGemvTargetGroups, the slice is wider than kGemvSplitAbove, and each slice
// keeps at least one 32-wide k step per wave. A slice of 4096 or less runs in
// at most two rounds of W loads per wave, and there the split's slice stores,
// count-in and merge cost more than the spread over more CUs saves (per
// launch, unsplit against split: 1024 x 2048 at 8 tokens 4.32 against 5.82 us
// in 4 slices; 2048 x 2048 at 32 tokens 5.62 against 6.65 us in 2; 1024 x
// 3072 at 8 tokens 5.78 against 6.14 in 4). At 2048 x 6144, 2 slices still
// win (9.08 against 9.88 us).
int gemv_split(int N, int K) {
    const int nfb = (N + 15) / 16;
    int ks = 1;
    while (ks < kGemvMaxSplit && nfb * ks < kGemvTargetGroups && K / ks > kGemvSplitAbove && K % (2 * ks * 32) == 0 &&
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
    const int ks = split ? gemv_split(a.N, a.K) : 1;
    // With fewer 16-feature blocks than kGemvTargetGroups and no K split, each
    // work-group takes one 16-token tile (grid z): twice the work-groups at 17
    // to 32 tokens, each staging half the activations. Blocks z and z + 1 of
    // one feature block are nfb apart in launch order, on one XCD when nfb is
    // a multiple of 8, so the second read of W can come from its L2.
    const int tiles = (a.M + 15) / 16;
    const int mt = !split && tiles > 1 && nfb < kGemvTargetGroups ? 1 : tiles;  // token tiles per work-group
    const dim3 grid(static_cast<unsigned>(nfb), static_cast<unsigned>(ks), static_cast<unsigned>(tiles / mt));
    uint32_t *counters = split ? static_cast<uint32_t *>(a.workspace) : nullptr;
    float *slices = split ? reinterpret_cast<float *>(static_cast<char *>(a.workspace) + (nfb * 4 + 255) / 256 * 256)
                          : nullptr;
    const f16 *A = static_cast<const f16 *>(a.A);
    const f16 *W = static_cast<const f16 *>(a.W);
    // Stage the activations when the slice's rows fit and their 16-byte
    // pieces per row are a multiple of 16 (the swizzle's period).
    const int kw = a.K / ks;
    const int stage = 16 * mt * kw * 2;
    const bool staged = kw % 128 == 0 && stage <= kGemvMaxStage;
    const int lds = staged ? std::max(stage, mt * kGemvRedBytes) : mt * kGemvRedBytes;
    // ceil(2^32 / pieces): r = t / pieces as one multiply-high for every slot t
    // of the stage (t * pieces < 2^32 since the stage is at most 128 KiB).
    const uint32_t magic = staged ? static_cast<uint32_t>(((uint64_t{1} << 32) + kw / 8 - 1) / (kw / 8)) : 0;
    // Dynamic LDS up to the device's 160 KiB per work-group launches without
    // raising a per-kernel limit on gfx950 (hipDeviceProp_t::sharedMemPerBlock).
    auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, dim3(kGemvThreads), static_cast<unsigned>(lds), stream, A, a.lda, W, a.M, a.N,
                           a.K, a.C, a.ldc, magic, slices, counters);
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
    switch (mt + (split ? 4 : 0) + (a.w_packed ? 8 : 0) + (staged ? 16 : 0)) {
        case 1: return go(gemv_kernel<1, EP, false, false, false>);
        case 2: return go(gemv_kernel<2, EP, false, false, false>);
        case 3: return go(gemv_kernel<3, EP, false, false, false>);
        case 4: return go(gemv_kernel<4, EP, false, false, false>);
        case 5: return go(gemv_kernel<1, EP, true, false, false>);
        case 6: return go(gemv_kernel<2, EP, true, false, false>);
        case 7: return go(gemv_kernel<3, EP, true, false, false>);
        case 8: return go(gemv_kernel<4, EP, true, false, false>);
        case 9: return go(gemv_kernel<1, EP, false, true, false>);
        case 10: return go(gemv_kernel<2, EP, false, true, false>);
        case 11: return go(gemv_kernel<3, EP, false, true, false>);
        case 12: return go(gemv_kernel<4, EP, false, true, false>);
        case 13: return go(gemv_kernel<1, EP, true, true, false>);
        case 14: return go(gemv_kernel<2, EP, true, true, false>);
        case 15: return go(gemv_kernel<3, EP, true, true, false>);
        case 16: return go(gemv_kernel<4, EP, true, true, false>);
        case 17: return go(gemv_kernel<1, EP, false, false, true>);
        case 18: return go(gemv_kernel<2, EP, false, false, true>);
        case 19: return go(gemv_kernel<3, EP, false, false, true>);
        case 20: return go(gemv_kernel<4, EP, false, false, true>);
        case 21: return go(gemv_kernel<1, EP, true, false, true>);
        case 22: return go(gemv_kernel<2, EP, true, false, true>);
        case 23: return go(gemv_kernel<3, EP, true, false, true>);
        case 24: return go(gemv_kernel<4, EP, true, false, true>);
        case 25: return go(gemv_kernel<1, EP, false, true, true>);
        case 26: return go(gemv_kernel<2, EP, false, true, true>);
        case 27: return go(gemv_kernel<3, EP, false, true, true>);
        case 28: return go(gemv_kernel<4, EP, false, true, true>);
        case 29: return go(gemv_kernel<1, EP, true, true, true>);
        case 30: return go(gemv_kernel<2, EP, true, true, true>);
        case 31: return go(gemv_kernel<3, EP, true, true, true>);
        case 32: return go(gemv_kernel<4, EP, true, true, true>);
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
// order (each thread's elements in the order it holds them, then the wave,
// then the waves in order). Rows up to kNormThreads * kNormPer wide keep the
// thread's elements of x and w in registers, all loaded up front: one memory
// round trip per row instead of one for x and another for w and x again.
// FORM: kNormLoop (any width: elements t, t + 256, ... re-read for the
// output), kNormHeld (held, elements t, t + 256, ...), kNormHeld4 (held, a
// width that is a multiple of 4 with 16-byte aligned rows: runs of 4
// adjacent elements 4 (t + 256 j) .. + 3, each one load of x, one of w and
// one 8-byte store).
constexpr int kNormLoop = 0, kNormHeld = 1, kNormHeld4 = 2;

template <int FORM>
__global__ void __launch_bounds__(kNormThreads) rmsnorm_rows_kernel(const float *__restrict__ x,
                                                                    const int32_t *__restrict__ rows, int hidden,
                                                                    const float *__restrict__ w, float eps,
                                                                    f16 *__restrict__ out) {
    __shared__ double part[kNormThreads / kWave];
    const int r = static_cast<int>(blockIdx.x), t = static_cast<int>(threadIdx.x);
    const float *xr = x + static_cast<int64_t>(rows ? rows[r] : r) * hidden;
    f16 *o = out + static_cast<int64_t>(r) * hidden;
    constexpr bool HELD = FORM != kNormLoop;
    float xv[HELD ? kNormPer : 1], wv[HELD ? kNormPer : 1];
    double ss = 0.0;
    if constexpr (FORM == kNormHeld4) {
#pragma unroll
        for (int j = 0; j < kNormPer / 4; j++) {
            const int i = 4 * (t + j * kNormThreads);
            const f32x4 xq = i < hidden ? *reinterpret_cast<const f32x4 *>(xr + i) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            const f32x4 wq = i < hidden ? *reinterpret_cast<const f32x4 *>(w + i) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                xv[4 * j + e] = xq[e];
                wv[4 * j + e] = wq[e];
            }
        }
#pragma unroll
        for (int j = 0; j < kNormPer; j++) ss += static_cast<double>(xv[j]) * xv[j];  // + 0.0 past the row: exact
    } else if constexpr (FORM == kNormHeld) {
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
    if constexpr (FORM == kNormHeld4) {
#pragma unroll
        for (int j = 0; j < kNormPer / 4; j++) {
            const int i = 4 * (t + j * kNormThreads);
            if (i >= hidden) continue;
            f16x4 h;
#pragma unroll
            for (int e = 0; e < 4; e++) h[e] = static_cast<f16>(clamp_half(wv[4 * j + e] * (xv[4 * j + e] * scale)));
            *reinterpret_cast<f16x4 *>(o + i) = h;
        }
    } else if constexpr (FORM == kNormHeld) {
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
    const bool aligned = a.hidden % 4 == 0 && ((reinterpret_cast<uintptr_t>(a.x) | reinterpret_cast<uintptr_t>(a.w)) & 15) == 0 &&
                         (reinterpret_cast<uintptr_t>(a.out) & 7) == 0;
    const auto kernel = a.hidden > kNormThreads * kNormPer ? rmsnorm_rows_kernel<kNormLoop>
                        : aligned                          ? rmsnorm_rows_kernel<kNormHeld4>
                                                           : rmsnorm_rows_kernel<kNormHeld>;
    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(a.R)), dim3(kNormThreads), 0, stream, a.x, a.rows, a.hidden,
                       a.w, a.eps, static_cast<f16 *>(a.out));
    return hipGetLastError();
}

}  // namespace ember::hip
