// Causal prefill attention over the paged cache on gfx950 MFMA.
//
// Replaces the reference's prefill_attention_kernel (src/backend/cuda/
// k_attention.cu:214-370): a query tile of up to 64 consecutive tokens of one
// sequence attends to every cached key up to each token's own position
// (keys 0..pos, the tile's own keys included: the append kernel has stored
// them). Semantics kept: 16-token pages gathered through the block table,
// keys past a query's position masked, online softmax, f16 in, f32
// accumulation, f16 out.
//
// Shape on MI355X: one work-group per (tile, pair of query heads of one kv
// head), so each K/V block is read once for both heads of a GQA pair (the
// reference's block serves one head): 4 waves per head, wave w owning tokens
// 16 (w % 4) .. + 15 of the tile for head w / 4. Keys go in blocks of 32 (two
// pages): the work-group stages a block's K rows and V transposed (dims x
// keys) in LDS, double-buffered (every thread fetches its part of block k + 1
// into registers while block k computes, then stores it to the other buffer),
// and every wave runs
//   S^T = K Q^T   16 keys x 16 queries per v_mfma_f32_16x16x32_f16, four
//                 32-dim chunks; lane l ends with query l % 16 and keys
//                 4 (l / 16) + 0..3 of each 16-key half;
//   softmax       per query in base 2, the block max reduced over the four
//                 lanes that hold a query; each lane sums its own keys' p;
//   O += P V      P is the A operand as the S^T lanes hold it: lane l's eight
//                 k-slots are keys {4g..4g+3, 16+4g..16+4g+3} (g = l / 16),
//                 and V^T in LDS serves exactly those keys per dim, so the
//                 products pair up (k order inside one MFMA is free).
// P is rounded to f16 for the MFMA and the row sum adds the same rounded
// values, so numerator and denominator agree.
#include "device.hpp"
#include "kernels.hpp"

namespace ember::hip {
namespace {

constexpr int kTileTokens = EMBER_PREFILL_TILE;  // 64
constexpr int kKeyBlock = 32;                     // keys per LDS block: two pages
template <int HG>
constexpr int kThreadsFor = 256 * HG;  // 4 waves per query head
constexpr int kKRow = kHeadDim + 8;               // LDS row of K, halves (272 B: rows land on distinct banks)
constexpr int kVRow = kKeyBlock + 4;              // LDS row of V^T (one dim), halves: 18 dwords, rows 2 apart 4 banks apart

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

// 2^x by the hardware instruction (v_exp_f32); 0 at -inf.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

template <int HG>  // query heads per work-group (1 or 2), all of one kv head
__global__ void __launch_bounds__(kThreadsFor<HG>) prefill_kernel(EmberPrefillArgs a, float scale_log2) {
    constexpr int kPThreads = kThreadsFor<HG>;
    constexpr int kWavesP = kPThreads / kWave;         // 4 x HG: wave w takes tokens 16 (w % 4).. and head w / 4
    __shared__ __align__(16) f16 k_lds[2][kKeyBlock * kKRow];
    __shared__ __align__(16) f16 v_lds[2][kHeadDim * kVRow];
    __shared__ int wave_max[kWavesP];

    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid % kWave, wave = tid / kWave;
    const int ql = lane % 16, g = lane / 16;
    const int tile = static_cast<int>(blockIdx.x);
    const int head = static_cast<int>(blockIdx.y) * HG + wave / 4;
    const int G = a.n_heads / a.n_kv;
    const int kvh = static_cast<int>(blockIdx.y) * HG / G;
    const int t0 = a.tile_start[tile];
    const int nt = min(a.tile_end[tile] - t0, kTileTokens);
    const int32_t *table = a.block_tables + static_cast<int64_t>(a.tile_seq[tile]) * a.max_blocks;
    const f16 *q = static_cast<const f16 *>(a.q);
    const f16 *kc = static_cast<const f16 *>(a.k_cache);
    const f16 *vc = static_cast<const f16 *>(a.v_cache);

    // This lane's query (token 16 (wave % 4) + ql of the tile) and the tile's key range.
    const int my_i = 16 * (wave % 4) + ql;
    const bool my_ok = my_i < nt;
    const int my_pos = my_ok ? a.positions[t0 + my_i] : -1;
    int mx = my_pos;
    for (int o = 32; o > 0; o >>= 1) mx = max(mx, __shfl_xor(mx, o, kWave));
    if (lane == 0) wave_max[wave] = mx;
    __syncthreads();
    int max_pos = wave_max[0];
    for (int w = 1; w < kWavesP; w++) max_pos = max(max_pos, wave_max[w]);
    max_pos = min(max_pos, a.max_blocks * kPage - 1);
    const int n_blocks = (max_pos + kKeyBlock) / kKeyBlock;

    // Q^T operands: for 32-dim chunk c, dims 32c + 8g .. + 8 of this lane's query.
    f16x8 qb[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        f16x8 v = {};
        if (my_ok)
            v = *reinterpret_cast<const f16x8 *>(q + (static_cast<int64_t>(t0 + my_i) * a.n_heads + head) * kHeadDim +
                                                 32 * c + 8 * g);
        qb[c] = v;
    }

    float m = -INFINITY, l = 0.0f;
    f32x4v o_acc[8];
#pragma unroll
    for (int dt = 0; dt < 8; dt++) o_acc[dt] = f32x4v{0.0f, 0.0f, 0.0f, 0.0f};

    // A key block's K and V, fetched into registers and later stored to LDS;
    // keys past the tile's last position or in a block outside the pool are
    // zeros. K: 512 chunks of 8 dims of one key (one or two per thread), stored
    // as rows. V: 512 pieces of 4 keys x 2 dims (dims 2 dp, 2 dp + 1 of keys
    // 4 kq .. 4 kq + 3), each one 4-byte load per key - a wave's load reads one
    // 256-byte key row - regrouped into two 8-byte rows of V^T (dims x keys),
    // so V is transposed without sub-dword LDS stores.
    constexpr int kChunks = kKeyBlock * kHeadDim / 8 / kPThreads;
    auto fetch = [&](int kb, uint4 (&kv4)[kChunks], uint4 (&vq)[kChunks]) {
#pragma unroll
        for (int j = 0; j < kChunks; j++) {
            const int chunk = tid + j * kPThreads;
            {
                const int key = chunk / 16, d8 = (chunk % 16) * 8;
                kv4[j] = make_uint4(0, 0, 0, 0);
                const int pos = kb * kKeyBlock + key;
                if (kb < n_blocks && pos <= max_pos) {
                    const int blk = table[pos / kPage];
                    if (blk >= 0 && blk < a.num_blocks) {
                        const int64_t off =
                            ((static_cast<int64_t>(blk) * a.n_kv + kvh) * kPage + pos % kPage) * kHeadDim + d8;
                        kv4[j] = *reinterpret_cast<const uint4 *>(kc + off);
                    }
                }
            }
            {
                const int kq = chunk / 64, dp = chunk % 64;
                const int pos0 = kb * kKeyBlock + 4 * kq;  // the quad's 4 keys share a page
                uint32_t w[4] = {0, 0, 0, 0};
                if (kb < n_blocks && pos0 <= max_pos) {
                    const int blk = table[pos0 / kPage];
                    if (blk >= 0 && blk < a.num_blocks) {
                        const int64_t off =
                            ((static_cast<int64_t>(blk) * a.n_kv + kvh) * kPage + pos0 % kPage) * kHeadDim + 2 * dp;
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            if (pos0 + e <= max_pos) w[e] = *reinterpret_cast<const uint32_t *>(vc + off + e * kHeadDim);
                    }
                }
                vq[j] = make_uint4(w[0], w[1], w[2], w[3]);
            }
        }
    };
    auto stage = [&](int buf, const uint4 (&kv4)[kChunks], const uint4 (&vq)[kChunks]) {
#pragma unroll
        for (int j = 0; j < kChunks; j++) {
            const int chunk = tid + j * kPThreads;
            const int key = chunk / 16, d8 = (chunk % 16) * 8;
            *reinterpret_cast<uint4 *>(&k_lds[buf][key * kKRow + d8]) = kv4[j];
            // vq = (key e: dim 2dp | dim 2dp+1 << 16), e = 0..3; v_perm picks halves.
            const int kq = chunk / 64, dp = chunk % 64;
            const uint2 lo = make_uint2(__builtin_amdgcn_perm(vq[j].y, vq[j].x, 0x05040100u),
                                        __builtin_amdgcn_perm(vq[j].w, vq[j].z, 0x05040100u));
            const uint2 hi = make_uint2(__builtin_amdgcn_perm(vq[j].y, vq[j].x, 0x07060302u),
                                        __builtin_amdgcn_perm(vq[j].w, vq[j].z, 0x07060302u));
            *reinterpret_cast<uint2 *>(&v_lds[buf][(2 * dp) * kVRow + 4 * kq]) = lo;
            *reinterpret_cast<uint2 *>(&v_lds[buf][(2 * dp + 1) * kVRow + 4 * kq]) = hi;
        }
    };

    uint4 nk[kChunks], nv[kChunks];
    fetch(0, nk, nv);
    stage(0, nk, nv);
    __syncthreads();
    for (int kb = 0; kb < n_blocks; kb++) {
        const int buf = kb & 1;
        fetch(kb + 1, nk, nv);  // in flight while this block computes

        // Keys of this lane in the block: 16 st + 4g + r (st = half, r = 0..3).
        const int key_base = kb * kKeyBlock + 4 * g;
        const bool full = kb * kKeyBlock + kKeyBlock - 1 <= my_pos;  // every key of the block visible
        f32x4v s[2];
#pragma unroll
        for (int st = 0; st < 2; st++) {
            f32x4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const f16x8 ka = *reinterpret_cast<const f16x8 *>(&k_lds[buf][(16 * st + ql) * kKRow + 32 * c + 8 * g]);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qb[c], acc, 0, 0, 0);
            }
            s[st] = acc;
        }
        float sv[8];
        float bm = -INFINITY;
#pragma unroll
        for (int st = 0; st < 2; st++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float x = s[st][r] * scale_log2;
                if (!full && key_base + 16 * st + r > my_pos) x = -INFINITY;
                sv[4 * st + r] = x;
                bm = fmaxf(bm, x);
            }
        bm = fmaxf(bm, __shfl_xor(bm, 16, kWave));
        bm = fmaxf(bm, __shfl_xor(bm, 32, kWave));
        const float mn = fmaxf(m, bm);
        const float ref = mn == -INFINITY ? 0.0f : mn;
        const float corr = m == mn ? 1.0f : exp2_fast(m - ref);
        f16x8 pa;
        float psum = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const f16 ph = static_cast<f16>(exp2_fast(sv[i] - ref));
            pa[i] = ph;
            psum += static_cast<float>(ph);
        }
        l = l * corr + psum;
        m = mn;
        // O rows are queries 4g + r: their correction factors live in lanes 4g + r.
        float cq[4];
#pragma unroll
        for (int r = 0; r < 4; r++) cq[r] = __shfl(corr, 4 * g + r, kWave);
#pragma unroll
        for (int dt = 0; dt < 8; dt++) {
            const f16 *vrow = &v_lds[buf][(16 * dt + ql) * kVRow];
            const f16x4 lo = *reinterpret_cast<const f16x4 *>(vrow + 4 * g);
            const f16x4 hi = *reinterpret_cast<const f16x4 *>(vrow + 16 + 4 * g);
            const f16x8 vb = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            f32x4v acc = o_acc[dt];
#pragma unroll
            for (int r = 0; r < 4; r++) acc[r] = acc[r] * cq[r];
            o_acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, vb, acc, 0, 0, 0);
        }
        // The next block goes into the other buffer, which nobody reads any more:
        // the barrier that ended the previous block separated its readers.
        if (kb + 1 < n_blocks) stage(buf ^ 1, nk, nv);
        __syncthreads();
    }

    // Row sums over the four lanes of each query, then out = O / l for the
    // queries 4g + r this lane's O rows hold.
    float lt = l;
    lt = lt + __shfl_xor(lt, 16, kWave);
    lt = lt + __shfl_xor(lt, 32, kWave);
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    float iq[4];
#pragma unroll
    for (int r = 0; r < 4; r++) iq[r] = __shfl(inv, 4 * g + r, kWave);
    f16 *out = static_cast<f16 *>(a.out);
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int i = 16 * (wave % 4) + 4 * g + r;
        if (i >= nt) continue;
        f16 *row = out + (static_cast<int64_t>(t0 + i) * a.n_heads + head) * kHeadDim;
#pragma unroll
        for (int dt = 0; dt < 8; dt++) row[16 * dt + ql] = static_cast<f16>(o_acc[dt][r] * iq[r]);
    }
}

}  // namespace

hipError_t launch_prefill(const EmberPrefillArgs &a, hipStream_t stream) {
    const int G = a.n_heads / a.n_kv;
    const int hg = G % 2 == 0 ? 2 : 1;
    const dim3 grid(static_cast<unsigned>(a.num_tiles), static_cast<unsigned>(a.n_heads / hg));
    const float scale_log2 = a.scale * kLog2e;
    if (hg == 2)
        hipLaunchKernelGGL(prefill_kernel<2>, grid, dim3(kThreadsFor<2>), 0, stream, a, scale_log2);
    else
        hipLaunchKernelGGL(prefill_kernel<1>, grid, dim3(kThreadsFor<1>), 0, stream, a, scale_log2);
    return hipGetLastError();
}

}  // namespace ember::hip
