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
// reference's block serves one head). The work-group is two key groups of 4
// waves per head: group 0 takes key blocks 0, 2, 4, ..., group 1 blocks 1, 3,
// 5, ..., and in each group wave w owns tokens 16 (w % 4) .. + 15 of the tile
// for head w / 4 - four waves per SIMD, so one wave's LDS and MFMA latency
// hides behind the others'. Keys go in blocks of 32 (two pages): each group
// stages its block's K and V rows (one key each) in its own
// double-buffered LDS, with the loads of its next two blocks in flight while
// the current one computes; both groups pass one barrier per step. At the end group 1 hands
// its partial (reference max, row sums, O) through LDS to the group 0 wave
// with the same rows, which merges them. Every wave runs
//   S^T = K Q^T   16 keys x 16 queries per v_mfma_f32_16x16x32_f16, four
//                 32-dim chunks; lane l ends with query l % 16 and keys
//                 4 (l / 16) + 0..3 of each 16-key half;
//   softmax       per query in base 2, the block max reduced over the four
//                 lanes that hold a query; the causal mask only where a key
//                 of the block passes some row's position; O rescaled only
//                 when a row's max passes its reference by more than 2^8;
//   O += P V      P is the A operand as the S^T lanes hold it: lane l's eight
//                 k-slots are keys {4g..4g+3, 16+4g..16+4g+3} (g = l / 16),
//                 and the transposing LDS read (ds_read_b64_tr_b16) of
//                 the V rows gives lane l exactly those keys of dim l % 16,
//                 so the products pair up (k order inside one MFMA is free).
// P is rounded to f16 for the MFMA and the row sums are one more MFMA of the
// same P against ones, so numerator and denominator agree.
#include <hip/hip_ext.h>

#include "device.hpp"
#include "kernels.hpp"

namespace ember::hip {
namespace {

constexpr int kTileTokens = EMBER_PREFILL_TILE;  // 64
constexpr int kKeyBlock = 32;                     // keys per LDS block: two pages
template <int HG>
constexpr int kThreadsFor = 512 * HG;  // two key groups of 4 waves per query head
constexpr int kMergeSlots = 10;        // float4 slots per lane of a key group's partial: O (8), l, m
// LDS row of K, halves. 288 B: the score operand's 16-byte reads (rows 16 h + ql,
// chunk 4 c + g) measured free of bank conflicts, where 272 B rows cost 2.7
// conflict cycles per read.
constexpr int kKRow = kHeadDim + 16;
constexpr int kVRow = kHeadDim + 16;              // LDS row of V (one key), halves: 72 dwords, rows 8 banks apart
constexpr int kVAhead = 2;                        // V operand reads in flight ahead of their MFMAs
constexpr int kDescWord3 = 0x00020000;            // gfx9 raw buffer: 32-bit data format, no swizzle

typedef float f32x4v __attribute__((ext_vector_type(4)));
// The transposing LDS read's operand type. Its v4i16 form, with each element
// bit-cast to f16 after the read, came out of hipcc keeping only the first
// dword of each read; this form goes straight into the MFMA operand.
typedef __fp16 tr16x4 __attribute__((__vector_size__(4 * sizeof(__fp16))));

// How far a block's max may pass the running reference max (base 2) before
// the reference moves: P stays below 2^8.
constexpr float kLazyLog2 = 8.0f;

// 2^x by the hardware instruction (v_exp_f32); 0 at -inf.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

template <int HG>  // query heads per work-group (1 or 2), all of one kv head
__global__ void __launch_bounds__(kThreadsFor<HG>) prefill_kernel(const int32_t *tile_start, const int32_t *tile_end,
                                                                  const int32_t *tile_seq, const int32_t *positions,
                                                                  const int32_t *block_tables, int n_heads,
                                                                  int n_kv, int max_blocks, float scale_log2_arg,
                                                                  EmberPrefillArgs a) {
    // The leading arguments (what the first loads need, and the softmax scale) are preloaded into scalar
    // registers at launch (build.py: -amdgpu-kernarg-preload-count=9); `a` carries the rest. The scale
    // loaded from the argument segment instead went out just before the key loop, and its pending scalar
    // load made the compiler wait for all of a step's first LDS reads (lgkmcnt(0)) at the loop's head.
    // Kernel arguments used inside the key loop are taken into scalar registers once: left as they are, the
    // compiler reloads them from the argument segment every step, and each reload is one more scalar round
    // trip ahead of the step's LDS waits (lgkmcnt counts both).
    const float scale_log2 = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, scale_log2_arg)));
    const int pool_blocks = __builtin_amdgcn_readfirstlane(a.num_blocks);
    constexpr int kPThreads = kThreadsFor<HG>;
    constexpr int kGroupThreads = kPThreads / 2;       // one key group
    constexpr int kGroupWaves = kGroupThreads / kWave; // 4 x HG: wave w takes tokens 16 (w % 4).. and head w / 4
    constexpr int kWavesP = 2 * kGroupWaves;
    constexpr int kKBytes = kKeyBlock * kKRow * 2, kVBytes = kKeyBlock * kVRow * 2;
    constexpr int kStageBytes = 2 * 2 * (kKBytes + kVBytes);           // [group][buffer] K and V
    constexpr int kMergeBytes = kGroupWaves * kMergeSlots * kWave * 16;  // group 1's partials, one float4 per slot
    __shared__ __align__(16) unsigned char lds[kStageBytes > kMergeBytes ? kStageBytes : kMergeBytes];
    __shared__ int wave_max[kWavesP];

    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid % kWave, wave = tid / kWave;
    const int grp = __builtin_amdgcn_readfirstlane(wave / kGroupWaves);  // key blocks grp, grp + 2, ...
    const int wl = wave % kGroupWaves, tg = tid % kGroupThreads;
    const int ql = lane % 16, g = lane / 16;
    // Work-group id -> (tile, head pair), head pairs fastest: ids that differ by
    // a multiple of 8 run on one XCD, so with 8 head pairs every tile of one
    // (sequence, kv head) shares that XCD's L2 for the keys they all read.
    const int n_pairs = n_heads / HG;
    const int tile = static_cast<int>(blockIdx.x) / n_pairs;
    const int pair = static_cast<int>(blockIdx.x) % n_pairs;
    const int head = pair * HG + wl / 4;
    const int G = n_heads / n_kv;
    const int kvh = pair * HG / G;
    const int t0 = tile_start[tile], t_end = tile_end[tile], seq = tile_seq[tile];
    const int nt = min(t_end - t0, kTileTokens);
    const int32_t *table = block_tables + static_cast<int64_t>(seq) * max_blocks;
    const f16 *q = static_cast<const f16 *>(a.q);
    const f16 *kc = static_cast<const f16 *>(a.k_cache);
    const f16 *vc = static_cast<const f16 *>(a.v_cache);
    auto k_lds = [&](int buf) { return reinterpret_cast<f16 *>(lds + (grp * 2 + buf) * kKBytes); };
    auto v_lds = [&](int buf) { return reinterpret_cast<f16 *>(lds + 4 * kKBytes + (grp * 2 + buf) * kVBytes); };

    // This lane's query (token 16 (wl % 4) + ql of the tile) and the tile's key range.
    const int my_i = 16 * (wl % 4) + ql;
    const bool my_ok = my_i < nt;
    // One query head per work-group (launches of one round, where every work-group's prologue is on the
    // launch's critical path): every load the first blocks need goes out here, before the positions'
    // reduction and its barrier, unguarded: this lane's position and Q (a row past the tile reads the
    // tile's last token; its position still counts as -1 and its Q as 0), and the block ids of the first
    // three fetches, clamped into the table's row (the fetches test the page against the last one
    // later). Config 3: 55.4-55.6 against 56.3-56.4 us per launch. Two heads per work-group keep their
    // loads after the barrier: early, they cost config 4's many-round launches 1.7%.
    constexpr bool kEarly = HG == 1;
    const int my_row = t0 + min(my_i, nt - 1);
    const int wl_pre = __builtin_amdgcn_readfirstlane(wl);
    constexpr int kChunks = kKeyBlock * kHeadDim / 8 / kGroupThreads;  // 16-byte chunks per thread and tensor
    f16x8 qb[4];  // Q^T operands: for 32-dim chunk c, dims 32c + 8g .. + 8 of this lane's query
    int ids_pre[3][kChunks];
    int my_pos;
    if constexpr (kEarly) {
        const int pos_raw = positions[my_row];
#pragma unroll
        for (int c = 0; c < 4; c++)
            qb[c] = *reinterpret_cast<const f16x8 *>(q + (static_cast<int64_t>(my_row) * n_heads + head) * kHeadDim +
                                                     32 * c + 8 * g);
#pragma unroll
        for (int b = 0; b < 3; b++)
#pragma unroll
            for (int j = 0; j < kChunks; j++)
                ids_pre[b][j] = table[min(2 * (grp + 2 * b) + (wl_pre * kWave + j * kGroupThreads) / (kPage * 16),
                                          max_blocks - 1)];
        my_pos = my_ok ? pos_raw : -1;
    } else {
        my_pos = my_ok ? positions[t0 + my_i] : -1;
    }
    int mx = my_pos, mn_pos = my_pos;
    for (int o = 32; o > 0; o >>= 1) {
        mx = max(mx, __shfl_xor(mx, o, kWave));
        mn_pos = min(mn_pos, __shfl_xor(mn_pos, o, kWave));
    }
    // The wave's lowest position: a block every key of which is at or below it
    // needs no causal mask in this wave (a tile's unused rows hold -1: masked).
    const int wave_min_pos = __builtin_amdgcn_readfirstlane(mn_pos);
    if (lane == 0) wave_max[wave] = mx;
    __syncthreads();
    int max_pos = wave_max[0];
    for (int w = 1; w < kWavesP; w++) max_pos = max(max_pos, wave_max[w]);
    max_pos = __builtin_amdgcn_readfirstlane(min(max_pos, max_blocks * kPage - 1));
    const int n_blocks = (max_pos + kKeyBlock) / kKeyBlock;

    if constexpr (kEarly) {
#pragma unroll
        for (int c = 0; c < 4; c++) qb[c] = my_ok ? qb[c] : f16x8{};
    } else {
#pragma unroll
        for (int c = 0; c < 4; c++) {
            f16x8 v = {};
            if (my_ok)
                v = *reinterpret_cast<const f16x8 *>(q + (static_cast<int64_t>(t0 + my_i) * n_heads + head) * kHeadDim +
                                                     32 * c + 8 * g);
            qb[c] = v;
        }
    }

    float m = -INFINITY;  // the reference max of this lane's query (base 2, scaled)
    f32x4v o_acc[8];
#pragma unroll
    for (int dt = 0; dt < 8; dt++) o_acc[dt] = f32x4v{0.0f, 0.0f, 0.0f, 0.0f};
    // Row sums by the MFMA: P times a ones operand, so lane l holds the sums of
    // exactly the query rows 4g + r its O values belong to, in the same f32
    // accumulation as O and of the same f16-rounded P.
    f32x4v l_acc = {0.0f, 0.0f, 0.0f, 0.0f};
    f16x8 ones;
#pragma unroll
    for (int i = 0; i < 8; i++) ones[i] = static_cast<f16>(1.0f);

    // A key block's K and V, fetched by its group into registers and later
    // stored to the group's LDS buffer. K and V alike: 512 chunks of 8 dims of
    // one key (one or two per thread, 16-byte loads), stored as rows; the PV
    // product transposes V as it reads it from LDS. A chunk's page (the
    // block's first or second) is the same for a whole wave, so the block ids
    // are scalar loads and each thread's offsets inside a page are fixed.
    // Pages past the tile's last position or outside the pool give zeros, and
    // so do V slots past the last position (an unwritten slot may hold
    // anything, and P = 0 must not meet a NaN).
    // Each load goes through a buffer descriptor of the kv head's page (built
    // in scalar registers from the wave-uniform block id): a page past the
    // tile's keys or outside the pool gets a descriptor with no records, and
    // V's covers only the slots up to the last position, so those loads
    // return zeros with no branch and no register cleared beforehand.
    const int wl_u = wl_pre;
    const int64_t page_elems = static_cast<int64_t>(n_kv) * kPage * kHeadDim;
    const int64_t head_elems = static_cast<int64_t>(kvh) * kPage * kHeadDim;
    const int last_page = max_pos / kPage;
    uint32_t koff[kChunks];  // bytes from the kv head's page start
#pragma unroll
    for (int j = 0; j < kChunks; j++) {
        const int chunk = tg + j * kGroupThreads;
        koff[j] = static_cast<uint32_t>((((chunk / 16) % kPage) * kHeadDim + (chunk % 16) * 8) * 2);
    }
    // The block ids of block kb's pages for this wave's chunks (scalar loads), read one step before the
    // fetch that uses them, next to the step's LDS stores: their round trip then ends inside the wait that
    // precedes the barrier instead of at the top of the next step.
    auto fetch_ids = [&](int kb, int (&ids)[kChunks]) {
#pragma unroll
        for (int j = 0; j < kChunks; j++)
            ids[j] = table[min(2 * kb + (wl_u * kWave + j * kGroupThreads) / (kPage * 16), last_page)];
    };
    auto fetch = [&](int kb, const int (&ids)[kChunks], uint4 (&kv4)[kChunks], uint4 (&vq)[kChunks]) {
#pragma unroll
        for (int j = 0; j < kChunks; j++) {
            const int pg = 2 * kb + (wl_u * kWave + j * kGroupThreads) / (kPage * 16);  // wave-uniform
            const int blk = ids[j];
            // Bitwise, not short-circuit: a branch here let the compiler sink the second id's load past the
            // first chunk's loads, two scalar round trips per step instead of one.
            const bool live = (kb < n_blocks) & (pg <= last_page) & (blk >= 0) & (blk < pool_blocks);
            const int64_t at = (live ? blk : 0) * page_elems + head_elems;
            const int vslots = live ? min(kPage, max_pos - pg * kPage + 1) : 0;  // V slots up to the last position
            const __amdgpu_buffer_rsrc_t kd = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<f16 *>(kc + at), 0, live ? kPage * kHeadDim * 2 : 0, kDescWord3);
            const __amdgpu_buffer_rsrc_t vd =
                __builtin_amdgcn_make_buffer_rsrc(const_cast<f16 *>(vc + at), 0, vslots * kHeadDim * 2, kDescWord3);
            kv4[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(kd, koff[j], 0, 0));
            vq[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(vd, koff[j], 0, 0));
        }
    };
    auto stage = [&](int buf, const uint4 (&kv4)[kChunks], const uint4 (&vq)[kChunks]) {
        f16 *kl = k_lds(buf), *vl = v_lds(buf);
#pragma unroll
        for (int j = 0; j < kChunks; j++) {
            const int chunk = tg + j * kGroupThreads;
            const int key = chunk / 16, d8 = (chunk % 16) * 8;
            *reinterpret_cast<uint4 *>(&kl[key * kKRow + d8]) = kv4[j];
            *reinterpret_cast<uint4 *>(&vl[key * kVRow + d8]) = vq[j];
        }
    };

    // The two groups step together, one barrier per step: at step s group
    // grp computes block 2 s + grp from its buffer s % 2, and at the end of
    // the step stores block 2 (s + 1) + grp into its other buffer (whose
    // readers all finished before the previous barrier). The loads run kAhead
    // steps ahead of that store: with two, block 2 (s + 1) + grp was fetched
    // during step s - 1 into one register set while the other set, staged at
    // the end of step s - 1, now takes block 2 (s + 2) + grp. The two sets
    // alternate, so the loop is unrolled by two to keep them in registers.
    // Measured at config 3: 64.0 -> 61.9 us with two steps ahead (two query
    // heads per work-group, 120 VGPRs). One query head per work-group runs
    // two ahead as well at 128 VGPRs (four waves per SIMD still).
    constexpr int kAhead = 2;
    const int n_steps = (n_blocks + 1) / 2;
    uint4 nk0[kChunks], nv0[kChunks], nk1[kChunks], nv1[kChunks];
    int idn[kChunks];
    if constexpr (kEarly) {
        fetch(grp, ids_pre[0], nk0, nv0);
        fetch(grp + 2, ids_pre[1], nk1, nv1);
#pragma unroll
        for (int j = 0; j < kChunks; j++) idn[j] = ids_pre[2][j];  // the first step's fetch
    } else {
        fetch_ids(grp, idn);
        fetch(grp, idn, nk0, nv0);
        fetch_ids(grp + 2, idn);
        fetch(grp + 2, idn, nk1, nv1);
        fetch_ids(grp + 2 * kAhead, idn);  // the first step's fetch
    }
    stage(0, nk0, nv0);
    __syncthreads();
    auto step = [&](int st, uint4 (&nk_free)[kChunks], uint4 (&nv_free)[kChunks], uint4 (&nk_next)[kChunks],
                    uint4 (&nv_next)[kChunks]) {
        const int buf = st & 1, kb = 2 * st + grp;
        fetch(kb + 2 * kAhead, idn, nk_free, nv_free);  // in flight while this block and the next compute
        if (kb < n_blocks) {
            const f16 *kl = k_lds(buf), *vl = v_lds(buf);
            // S^T: lane l holds query ql and keys 16 h + 4g + r (h = half, r = 0..3).
            float sv[8];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                f16x8 ka[4];
#pragma unroll
                for (int c = 0; c < 4; c++)
                    ka[c] = *reinterpret_cast<const f16x8 *>(&kl[(16 * h + ql) * kKRow + 32 * c + 8 * g]);
                f32x4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int c = 0; c < 4; c++) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[c], qb[c], acc, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++) sv[4 * h + r] = acc[r];
            }
            if (kb * kKeyBlock + kKeyBlock - 1 > wave_min_pos) {  // some key of the block is past some row's position
                const int key_base = kb * kKeyBlock + 4 * g;
#pragma unroll
                for (int i = 0; i < 8; i++)
                    if (key_base + 16 * (i / 4) + i % 4 > my_pos) sv[i] = -INFINITY;
            }
            // The reference max moves only when a block's max passes it by more
            // than kLazyLog2, so P stays below 2^kLazyLog2 (f16 holds it) and O is
            // rescaled in few blocks; O / l is the same for any reference. Each
            // lane first checks its own eight keys: only when one of them passes
            // does the wave reduce to the query max over its four lanes.
            float lmax = sv[0];
#pragma unroll
            for (int i = 1; i < 8; i++) lmax = fmaxf(lmax, sv[i]);
            if (__builtin_amdgcn_ballot_w64(lmax * scale_log2 > m + kLazyLog2) != 0) {
                float bm = fmaxf(lmax, __shfl_xor(lmax, 16, kWave));
                bm = fmaxf(bm, __shfl_xor(bm, 32, kWave));
                const float bx = bm * scale_log2;
                const bool grow = bx > m + kLazyLog2;
                const float corr = grow ? exp2_fast(m - bx) : 1.0f;  // 0 from an empty row
                m = grow ? bx : m;
                float cq[4];
#pragma unroll
                for (int r = 0; r < 4; r++) cq[r] = __shfl(corr, 4 * g + r, kWave);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    l_acc[r] = l_acc[r] * cq[r];
#pragma unroll
                    for (int dt = 0; dt < 8; dt++) o_acc[dt][r] = o_acc[dt][r] * cq[r];
                }
            }
            const float neg_ref = m == -INFINITY ? 0.0f : -m;  // a row with no visible key yet has only -inf scores
            f16x8 pa;
#pragma unroll
            for (int i = 0; i < 8; i++) pa[i] = static_cast<f16>(exp2_fast(fmaf(sv[i], scale_log2, neg_ref)));
            l_acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, ones, l_acc, 0, 0, 0);
            // The V operand of dim tile dt; reads run kVAhead tiles ahead of
            // their MFMAs. Left to itself the scheduler issues each read next to
            // its MFMA, one LDS round trip per tile; the scheduling barriers keep
            // the reads ahead (3-4% of the launch at configs 3 and 4).
            // ds_read_b64_tr_b16: in each 16-lane block, lane r reads 4 halves
            // (row r of a 16 x 4 matrix M) and lane i receives M[4 m + i / 4][i % 4],
            // m = 0..3. Lane r reading key 4 g + r / 4, dims 16 dt + 4 (r % 4) + 0..3
            // so hands lane i dim 16 dt + i of keys 4 g + 0..3; the second read
            // is the same 16 keys on. A half-wave's 8 key rows sit 8 banks apart.
            auto vread = [&](int dt) {
                const f16 *p = &vl[(4 * g + ql / 4) * kVRow + 16 * dt + 4 * (ql % 4)];
                typedef __attribute__((address_space(3))) tr16x4 lds_tr16x4;
                const f16x4 lo = __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_tr16x4 *)(p)));
                const f16x4 hi =
                    __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_tr16x4 *)(p + 16 * kVRow)));
                return f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            };
            f16x8 vb[kVAhead];
#pragma unroll
            for (int i = 0; i < kVAhead; i++) vb[i] = vread(i);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int dt = 0; dt < 8; dt++) {
                o_acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, vb[dt % kVAhead], o_acc[dt], 0, 0, 0);
                if (dt + kVAhead < 8) vb[dt % kVAhead] = vread(dt + kVAhead);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        fetch_ids(kb + 2 * kAhead + 2, idn);  // the next step's fetch
        if (kb + 2 < n_blocks) stage(buf ^ 1, nk_next, nv_next);
        __syncthreads();
    };
    for (int st = 0; st < n_steps; st += 2) {
        step(st, nk0, nv0, nk1, nv1);
        if (st + 1 < n_steps) step(st + 1, nk1, nv1, nk0, nv0);
    }

    // Group 1 hands its partial (reference max, row sums, O) to the group 0
    // wave with the same rows, through LDS (the staging buffers are free after
    // the last barrier); that wave merges the two and writes out = O / l.
    f32x4v *slot = reinterpret_cast<f32x4v *>(lds) + (wl * kMergeSlots) * kWave + lane;
    if (grp == 1) {
#pragma unroll
        for (int dt = 0; dt < 8; dt++) slot[dt * kWave] = o_acc[dt];
        slot[8 * kWave] = l_acc;
        slot[9 * kWave] = f32x4v{m, 0.0f, 0.0f, 0.0f};
    }
    __syncthreads();
    if (grp == 1) return;
    const float m1 = slot[9 * kWave][0];
    const float mm = fmaxf(m, m1);
    const float f0 = mm == -INFINITY ? 0.0f : exp2_fast(m - mm);   // per query ql
    const float f1 = mm == -INFINITY ? 0.0f : exp2_fast(m1 - mm);
    float c0[4], c1[4];
#pragma unroll
    for (int r = 0; r < 4; r++) c0[r] = __shfl(f0, 4 * g + r, kWave), c1[r] = __shfl(f1, 4 * g + r, kWave);
    const f32x4v l1 = slot[8 * kWave];
    f16 *out = static_cast<f16 *>(a.out);
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int i = 16 * (wl % 4) + 4 * g + r;
        const float l = l_acc[r] * c0[r] + l1[r] * c1[r];
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        if (i >= nt) continue;
        f16 *row = out + (static_cast<int64_t>(t0 + i) * n_heads + head) * kHeadDim;
#pragma unroll
        for (int dt = 0; dt < 8; dt++) {
            const float o = o_acc[dt][r] * c0[r] + slot[dt * kWave][r] * c1[r];
            row[16 * dt + ql] = static_cast<f16>(o * inv);
        }
    }
}
}  // namespace

hipError_t launch_prefill(const EmberPrefillArgs &a, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    const int G = a.n_heads / a.n_kv;
    const int hg = a.heads_per_group == 1 || G % 2 != 0 ? 1 : 2;
    const dim3 grid(static_cast<unsigned>(a.num_tiles * (a.n_heads / hg)));
    const float scale_log2 = a.scale * kLog2e;
    if (hg == 2)
        hipExtLaunchKernelGGL(prefill_kernel<2>, grid, dim3(kThreadsFor<2>), 0, stream, start, stop, 0, a.tile_start,
                              a.tile_end, a.tile_seq, a.positions, a.block_tables, a.n_heads, a.n_kv, a.max_blocks,
                              scale_log2, a);
    else
        hipExtLaunchKernelGGL(prefill_kernel<1>, grid, dim3(kThreadsFor<1>), 0, stream, start, stop, 0, a.tile_start,
                              a.tile_end, a.tile_seq, a.positions, a.block_tables, a.n_heads, a.n_kv, a.max_blocks,
                              scale_log2, a);
    return hipGetLastError();
}

}  // namespace ember::hip
