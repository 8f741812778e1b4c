// Paged decode attention on gfx950: a bandwidth-bound gather whose page
// arithmetic runs on MFMA for f16 pages (VALU for f32 pages).
//
// Replaces the reference's paged_attention_kernel + combine_splits_kernel
// (src/backend/cuda/k_attention.cu:29-201), and in its fused form also its
// qk_norm_rope_store_kernel (k_elementwise.cu:67-126) for decode steps.
// Semantics kept: GQA with the G query heads of a kv head in one work-group
// (each page is read once for all of them), softmax in base 2 with the scale
// folded in, fixed context splits merged in a fixed order (batch invariance),
// slots past a query's position never contribute.
//
// Work-group = 4 waves per (query run, kv head, context split). A run is 1..8
// consecutive tokens of one sequence (decode: 1; speculative verify: k + 1);
// all of them are served by the same page reads. Its query rows (token, head
// of the kv head's G) number at most 16.
//
// Page walk: wave w takes pages first + w, first + w + 4, ... A page of one kv
// head is 16 keys x 128 dims, contiguous (4 KiB in f16), read with four
// dwordx4 loads per lane for K and four for V.
//
// f16 pages (MFMA): lane l = 16 g + c serves query column c, the run's row c
// (columns past the last row repeat it).
//   scores: S^T = K Q^T, four v_mfma_f32_16x16x32_f16 over 32 dims each. The A
//           operand is K (lane l: key c, dims 32 s + 8 g .. + 7 of step s), the
//           B operand q (lane l: row c, the same dims), so lane l ends with
//           row c's raw scores of keys 4 g .. 4 g + 3.
//   softmax: per column, the max over the 16 keys (its four lane groups meet
//           through v_permlane16_swap / v_permlane32_swap), then one
//           exponential per score; the weights, rounded to f16, are already
//           the B operand of the value products, and each lane keeps the sum
//           of its own four (the groups' sums meet once, at the end).
//   values: O^T += V^T P^T, eight v_mfma_f32_16x16x16_f16, one per dim tile
//           t: lane l loads keys 4 g .. 4 g + 3, dims 8 c .. 8 c + 7 of V
//           (each load instruction reads four whole 256-byte key rows), and
//           two v_perm per tile give it the A operand (dim 8 c + t of its four
//           keys). Lane l accumulates row c's dims 32 g .. 32 g + 31.
// f32 pages (VALU): lane l = 16 r + c holds dims [8c, 8c + 8) of keys 4i + r
// (i = 0..3), for K and for V, and computes every row itself:
//   scores: an 8-dim partial dot per key, reduced over the 16 lanes of DPP row
//           r so that quad q of the row holds key q's score;
//   softmax: each DPP row keeps its own running max / sum over its keys;
//   values: each lane accumulates its 8 dims over its 4 keys.
// Latency: a work-group's first page loads depend on one descriptor load only
// (the descriptor carries the first block ids), the split's other block ids
// arrive in one vector load next to them, and each wave loads the next page's
// keys while it computes the current page's values, and the next page's values
// while it computes the next page's scores.
// At the end: lanes merge (f32: two lane exchanges; f16: the row sums over
// the lane groups), waves through LDS, and splits either in the separate merge
// kernel or, with merge counters, in the last work-group of the (run, kv head)
// to finish - all in one fixed order.
//
// Fused form (decode steps): the work-group computes its rows' q from qkv
// (QK-RMSNorm + RoPE, the append kernel's arithmetic), and the K/V of the
// run's new tokens that fall in its split; it stores them to the pool and uses
// them in place of those slots of the pages it reads. Only this work-group
// reads those slots in this launch, so nothing waits for another work-group.
//
// Exactness of runs: a query row's arithmetic is the same whether its token is
// alone or in a run: each MFMA output element is its own row's dot product,
// and every per-row step is done per column. Pages entirely below the run's
// lowest position take a path with no masking at all; later pages set the
// scores of keys past a row's position to -inf (weight 0, and the max ignores
// them), which gives a fully visible page the same bits as the fast path and
// makes a page with no visible key an exact no-op for that row (correction
// factor 1 exactly, zero weights). On those pages the V slots past the run's
// last position, which may hold anything (pool slots never written), are read
// as 0, so a zero weight never meets an inf or NaN. Hence verify of k + 1
// tokens equals k + 1 single-token decode steps bit-exactly (f16 pages written
// by the append kernels are finite: it clamps them).
#include <climits>
#include <type_traits>

#include <hip/hip_ext.h>

#include "device.hpp"
#include "kernels.hpp"

namespace ember::hip {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * kWave;

// A work item as the host plan describes it (EmberAttnArgs::work_desc): run,
// split, first list entry, count, sequence, lowest position, highest position,
// the first entry's token when the run's tokens and positions both count up by
// one (else -1), then the block ids of the split's first 8 pages (-1 past its
// last page). One s_load_dwordx16 gives a work-group everything it needs to
// issue its first page loads. The descriptors' address and n_kv, and the
// pools, block tables, qkv and rotary frequencies that the first page and
// query loads need, come as the kernel's leading arguments, which build.py has
// the compiler preload into scalar registers at launch
// (-amdgpu-kernarg-preload-count=7): the descriptor load then goes out at
// once, beside the first kernel-argument loads, instead of after their round
// trip.
typedef int32_t WorkDesc __attribute__((ext_vector_type(16)));
constexpr int kDescTok = 7, kDescBlocks = 8;

struct DecodeParams {
    const void *q, *k, *v;
    const int32_t *positions, *token_seq, *tables, *token_index, *run_first, *run_count, *work, *work_desc;
    void *out;
    float *part_acc, *part_ml;
    uint32_t *counters;
    int max_blocks, n_heads, n_kv, G, num_blocks, num_splits, split_len, num_runs;
    float scale_log2;
    // fused form
    const void *qkv;
    const float *q_norm, *k_norm, *bias, *inv_freq;
    float eps;
};

// A load through the constant address space: with a wave-uniform address the
// compiler emits s_load (scalar cache, lgkmcnt), which never waits for the
// vector page loads in flight. Only for data the kernel does not write.
template <class T>
__device__ __forceinline__ T uniform_load(const T *p) {
    return *(const __attribute__((address_space(4))) T *)(p);  // an address-space cast
}

__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// One page of K and V as this lane holds it: 4 x 8 dims of K and of V (which
// keys and dims depends on the path: see the top of the file).
template <typename T>
struct PageRegs;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
template <>
struct PageRegs<f16> {  // V only: f16 pages stage K in LDS
    u32x4 v[4];
};

template <>
struct PageRegs<float> {
    float4 k[4][2], v[4][2];
};

// Page data is read once per launch and never again before it leaves the
// caches, so it is loaded non-temporally (nt): on MI355X a page gather of this
// shape then reaches about 6.2 TB/s instead of about 5.6 TB/s with ordinary
// loads, which fill the caches with dead lines.
// Loads one page of one kv head through a buffer descriptor built from the
// wave-uniform page address (scalar registers): each load is
// buffer_load_dwordx4 v, v_lane_off, s[desc] offen offset:imm nt, with no
// per-page vector address arithmetic. A descriptor with no records (live =
// false) makes the loads return 0 without touching memory.
constexpr int kDescWord3 = 0x00020000;  // gfx9 raw buffer: 32-bit data format, no swizzle
constexpr int kNonTemporal = 2;         // cache-policy bit nt of a gfx950 buffer load

__device__ __forceinline__ u32x4 load_desc(__amdgpu_buffer_rsrc_t d, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(d, off, 0, kNonTemporal));
}

// One half of a page of one kv head (its 16 keys, or its 16 values) into
// regs[4]: four loads per lane, load i at byte lane_off + step * i of the half.
template <typename T, typename R>
__device__ __forceinline__ void load_half(R (&regs)[4], const T *base, uint32_t lane_off, uint32_t step, bool live) {
    constexpr int kBytes = kPage * kHeadDim * sizeof(T);  // one half-page of one kv head
    const __amdgpu_buffer_rsrc_t d = __builtin_amdgcn_make_buffer_rsrc(const_cast<T *>(base), 0, live ? kBytes : 0,
                                                                       kDescWord3);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if constexpr (sizeof(T) == 2) {
            regs[i] = load_desc(d, lane_off + step * i);
        } else {
            const u32x4 x = load_desc(d, lane_off + step * i), y = load_desc(d, lane_off + step * i + 16);
            regs[i][0] = make_float4(__uint_as_float(x.x), __uint_as_float(x.y), __uint_as_float(x.z), __uint_as_float(x.w));
            regs[i][1] = make_float4(__uint_as_float(y.x), __uint_as_float(y.y), __uint_as_float(y.z), __uint_as_float(y.w));
        }
    }
}

// Replaces key i of a page with the 8 dims this lane holds, read from LDS, in
// the lanes where `take` holds: the LDS rows are read by every lane (the
// caller passes an in-range row) and kept by selects, with no divergent branch.
__device__ __forceinline__ u32x4 select4(bool take, const u32x4 &a, const u32x4 &b) { return take ? a : b; }
__device__ __forceinline__ float4 select4(bool take, const float4 &a, const float4 &b) {
    return make_float4(take ? a.x : b.x, take ? a.y : b.y, take ? a.z : b.z, take ? a.w : b.w);
}

// f32 pages: key i of a page replaced by the 8 dims this lane holds.
__device__ __forceinline__ void put_key(PageRegs<float> &pr, int i, bool take, const float *k8, const float *v8) {
    pr.k[i][0] = select4(take, *reinterpret_cast<const float4 *>(k8), pr.k[i][0]);
    pr.k[i][1] = select4(take, *reinterpret_cast<const float4 *>(k8 + 4), pr.k[i][1]);
    pr.v[i][0] = select4(take, *reinterpret_cast<const float4 *>(v8), pr.v[i][0]);
    pr.v[i][1] = select4(take, *reinterpret_cast<const float4 *>(v8 + 4), pr.v[i][1]);
}

// f32 pages: a row's weights for the page's four keys of this lane's DPP row,
// and the query slice a lane needs (dims [8c, 8c + 8) of one row).
struct Weights {
    float w[4];
};
struct QSlice {
    float f[8];
};

__device__ __forceinline__ void load_q(QSlice &q, const float *qp) {
    const float4 a = *reinterpret_cast<const float4 *>(qp);
    const float4 b = *reinterpret_cast<const float4 *>(qp + 4);
    q.f[0] = a.x;
    q.f[1] = a.y;
    q.f[2] = a.z;
    q.f[3] = a.w;
    q.f[4] = b.x;
    q.f[5] = b.y;
    q.f[6] = b.z;
    q.f[7] = b.w;
}

__device__ __forceinline__ float dot8(const QSlice &q, const float4 (&k)[2]) {
    float s = 0.0f;
    s = fmaf(q.f[0], k[0].x, s);
    s = fmaf(q.f[1], k[0].y, s);
    s = fmaf(q.f[2], k[0].z, s);
    s = fmaf(q.f[3], k[0].w, s);
    s = fmaf(q.f[4], k[1].x, s);
    s = fmaf(q.f[5], k[1].y, s);
    s = fmaf(q.f[6], k[1].z, s);
    s = fmaf(q.f[7], k[1].w, s);
    return s;
}

__device__ __forceinline__ void unpack8(const float4 (&v)[2], float (&out)[8]) {
    out[0] = v[0].x;
    out[1] = v[0].y;
    out[2] = v[0].z;
    out[3] = v[0].w;
    out[4] = v[1].x;
    out[5] = v[1].y;
    out[6] = v[1].z;
    out[7] = v[1].w;
}

// 2^x by the hardware instruction (v_exp_f32): exact powers of two at
// integers, 0 at -inf; results below 2^-126 may flush to 0, which only drops
// weights that cannot move an f32 sum.
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// The page's scores in a DPP row (16 lanes, c = lane % 16, each holding an
// 8-dim partial dot product for the row's keys i = 0..3): reduced so that
// the lanes of quad q = c / 4 hold key q's full score, with 11 instructions
// instead of the 16 that give every lane all four. Two exchange steps halve
// the keys a lane carries (c pairs with 15 - c, keys {0,1} staying with c < 8;
// then c with its row-half mirror, keys q staying with quad q), and two quad
// steps finish the sums. The 16 lanes' partials of a key meet in a fixed tree,
// and the quad steps add values both partners hold, so the four lanes of a
// quad end bit-identical.
__device__ __forceinline__ float key_sums(const float (&x)[4], bool upper_half, bool odd_quad) {
    const float keep0 = upper_half ? x[2] : x[0], give0 = upper_half ? x[0] : x[2];
    const float keep1 = upper_half ? x[3] : x[1], give1 = upper_half ? x[1] : x[3];
    const float a0 = keep0 + dpp_mov<kDppRowMirror>(give0);
    const float a1 = keep1 + dpp_mov<kDppRowMirror>(give1);
    const float keep = odd_quad ? a1 : a0, give = odd_quad ? a0 : a1;
    float b = keep + dpp_mov<kDppRowHalfMirror>(give);
    b = b + dpp_mov<kDppQuadXor1>(b);
    return b + dpp_mov<kDppQuadXor2>(b);
}

// Max and sum over the four quads of a DPP row; every lane gets the same bits
// (quads q and q ^ 1 meet first, then the pairs, and both operations are
// commutative). The sum is (v0 + v1) + (v2 + v3).
__device__ __forceinline__ float quads_max(float v) {
    v = fmaxf(v, dpp_mov<kDppRowHalfMirror>(v));
    return fmaxf(v, dpp_mov<kDppRowMirror>(v));
}
__device__ __forceinline__ float quads_sum(float v) {
    v = v + dpp_mov<kDppRowHalfMirror>(v);
    return v + dpp_mov<kDppRowMirror>(v);
}

// Lane 4 q of each DPP row to every lane of the row: quad q's value (row_newbcast).
template <int Q>
__device__ __forceinline__ float quad_value(float v) {
    return dpp_mov<0x150 + 4 * Q>(v);
}

// f16 pages: max and sum over the four lane groups of a query column (lanes
// c, c + 16, c + 32, c + 48). Groups 0 and 1, and 2 and 3, meet through
// v_permlane16_swap, then the pairs through v_permlane32_swap. Both operations
// are commutative, so every lane of the column gets the same bits; the sum is
// (x0 + x1) + (x2 + x3).
__device__ __forceinline__ float groups_max(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float groups_sum(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// f16 pages: the A operand of the value products' dim tile TILE, dim
// 8 c + TILE of this lane's keys 4 g .. 4 g + 3 (its four 8-dim slices of V,
// one per key): two v_perm, each pairing one half of a word of two keys.
template <int TILE>
__device__ __forceinline__ f16x4 value_tile(const u32x4 (&v)[4]) {
    constexpr uint32_t sel = (TILE & 1) ? 0x07060302u : 0x05040100u;  // high or low halves of (b, a)
    constexpr int w = TILE / 2;
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 pair = {__builtin_amdgcn_perm(v[1][w], v[0][w], sel),   // keys 4g, 4g + 1
                        __builtin_amdgcn_perm(v[3][w], v[2][w], sel)};  // keys 4g + 2, 4g + 3
    return __builtin_bit_cast(f16x4, pair);
}

__device__ __forceinline__ f16x8 as_f16x8(const u32x4 &x) { return __builtin_bit_cast(f16x8, x); }

// Merges this lane's (m, l, acc) with the lane `mask` away; both lanes end
// with the same values.
// The running max of a row before any visible key: finite and far below any
// score (|q.k| * scale of f16 vectors is below 1e12), so a row's first visible
// key gives corr = 2^(kNoMax - max) = 0 exactly, as -inf would, while an empty
// row keeps l = 0 and O = 0; the merges below treat it like -inf (weight 0
// against any real max, and zeros when every part is empty).
constexpr float kNoMax = -1.0e30f;

__device__ __forceinline__ void merge_lanes(float &m, float &l, float (&acc)[8], int mask) {
    const float mo = __shfl_xor(m, mask, kWave), lo = __shfl_xor(l, mask, kWave);
    const float M = fmaxf(m, mo);
    const float fa = m == -INFINITY ? 0.0f : exp2_hw(m - M);
    const float fb = mo == -INFINITY ? 0.0f : exp2_hw(mo - M);
    l = l * fa + lo * fb;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float ao = __shfl_xor(acc[e], mask, kWave);
        acc[e] = acc[e] * fa + ao * fb;
    }
    m = M;
}

// Split partials are written and read with device-scope (agent) relaxed
// atomics: on gfx950 these are global_store / global_load with sc1, coherent
// across the XCDs' L2s by themselves, so the in-kernel merge needs no
// cache-wide write-back or invalidate (an agent-scope fence is buffer_wbl2 of
// the whole L2 per work-group, which serializes).
//
// Why the merge reads complete partials although every access is relaxed:
// the compiler lowers an agent-scope release as "buffer_wbl2 sc1; s_waitcnt
// vmcnt(0)" before the releasing store, and an acquire as "s_waitcnt
// vmcnt(0); buffer_inv sc1" after the acquiring load (LLVM AMDGPU memory
// model, GFX942 family, which gfx950 follows). The wbl2 / inv halves only
// write back or drop cached lines of non-atomic accesses; the partials are
// atomic sc1 accesses that bypass the non-coherent caches, so what ordering
// needs is the waits. They are here by hand: each work-group waits for its
// partial stores (s_waitcnt vmcnt(0), then a barrier) before its counter
// increment, and the merging work-group issues its partial loads only after
// the increment has returned (a barrier behind the returned value's branch).
// So every partial counted before the last increment is visible to the
// merge. The order is the hardware's, not the HIP source's: a port to another
// target must use release / acquire orderings instead.
__device__ __forceinline__ void put_partial(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float get_partial(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A split's (M, L), stored as two adjacent floats, with one 8-byte load.
__device__ __forceinline__ float2 get_partial_pair(const float *p) {
    const uint64_t v = __hip_atomic_load(reinterpret_cast<const uint64_t *>(p), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    return __builtin_bit_cast(float2, v);
}

// The split merge of one output element (token list entry li, head, dim d):
// out = sum_s O_s 2^(M_s - M) / sum_s L_s 2^(M_s - M) over the ns splits that
// hold the token's keys, in split order; splits without a visible key skipped.
// Used by the merge kernel and by the in-kernel merge alike. The partials of
// up to kMergeChunk splits are requested together and waited for once: a
// merge costs one memory round trip per chunk instead of one per split.
constexpr int kMergeChunk = 8;

template <typename T>
__device__ __forceinline__ void merge_one(const DecodeParams &p, int li, int head, int d, int ctx, T *out) {
    constexpr int D = kHeadDim;
    const int ns = min(p.num_splits, max(1, (ctx + p.split_len - 1) / p.split_len));
    const int64_t base = (static_cast<int64_t>(li) * p.n_heads + head) * p.num_splits;
    const float *ml = p.part_ml + base * 2;
    const float *acc = p.part_acc + base * D + d;
    float M = -INFINITY;
    float mv[kMergeChunk], lv[kMergeChunk], ov[kMergeChunk];
    // Pass 1 (only when there are more splits than one chunk holds): the max.
    if (ns > kMergeChunk) {
        for (int s0 = 0; s0 < ns; s0 += kMergeChunk) {
#pragma unroll
            for (int k = 0; k < kMergeChunk; k++) mv[k] = get_partial(ml + 2 * min(s0 + k, ns - 1));
#pragma unroll
            for (int k = 0; k < kMergeChunk; k++) M = fmaxf(M, mv[k]);  // repeats of the last split change nothing
        }
    }
    // Pass 2: the sums, in split order.
    float L = 0.0f, O = 0.0f;
    bool any = false;
    for (int s0 = 0; s0 < ns; s0 += kMergeChunk) {
#pragma unroll
        for (int k = 0; k < kMergeChunk; k++) {
            const int s = min(s0 + k, ns - 1);
            mv[k] = get_partial(ml + 2 * s);
            lv[k] = get_partial(ml + 2 * s + 1);
            ov[k] = get_partial(acc + static_cast<int64_t>(s) * D);
        }
        if (ns <= kMergeChunk) {
#pragma unroll
            for (int k = 0; k < kMergeChunk; k++) M = fmaxf(M, mv[k]);
        }
#pragma unroll
        for (int k = 0; k < kMergeChunk; k++) {
            if (s0 + k >= ns || mv[k] == -INFINITY) continue;
            const float f = mv[k] == M ? 1.0f : exp2_hw(mv[k] - M);  // one split: exactly O / L, as a direct write
            const float ls = lv[k] * f;
            const float os = ov[k] * f;
            L = any ? L + ls : ls;
            O = any ? O + os : os;
            any = true;
        }
    }
    out[d] = from_f32<T>(L > 0.0f ? O / L : 0.0f);
}

// Keeps the compiler's scheduler from moving instructions across this point:
// the page loop is written as load-next / use-current phases, and letting the
// scheduler hoist a phase's arithmetic above the next page's loads would leave
// fewer pages in flight.
__device__ __forceinline__ void phase_break() { __builtin_amdgcn_sched_barrier(0); }

// One work item: (run, kv head, split) = work-group `bid` of the dense grid or
// entry `bid` of the work list (item bid / n_kv, kv head bid % n_kv). tid is
// the thread's index in the work-group.
struct Preloaded {  // the kernel's leading arguments, in scalar registers from launch on
    const WorkDesc *descs;
    int n_kv;
    const void *k, *v;
    const int32_t *tables;
    const void *qkv;
    const float *inv_freq;
};

template <typename T, int ROWS, bool FUSED>
__device__ __forceinline__ void decode_item(const DecodeParams &p, const Preloaded &pre, const int bid, const int tid) {
    const WorkDesc *descs = pre.descs;
    const int n_kv_pre = pre.n_kv;
    constexpr int D = kHeadDim;
    constexpr int NEW = FUSED ? EMBER_MAX_RUN : 1;
    const int lane = tid % kWave;
    const int wave = uniform(tid / kWave);
    const int r = lane >> 4, c = lane & 15;
    const int G = p.G;
    // Until its page walk starts, a work-group runs at raised wave priority: a
    // CU's older waves, streaming pages, otherwise win the issue arbitration
    // and a late work-group's first loads wait behind them for microseconds.
    __builtin_amdgcn_s_setprio(3);

    // descs: the work list's descriptors (preloaded argument), or null when the
    // launch has none; n_kv_pre = p.n_kv, preloaded too.
    int run, kvh, split;
    WorkDesc desc = {};
    const bool have_desc = descs != nullptr;
    if (have_desc) {
        const int item = bid / n_kv_pre;
        kvh = bid % n_kv_pre;
        desc = uniform_load(descs + item);  // one s_load_dwordx16
        run = desc[0];
        split = desc[1];
        if (run < 0 || run >= p.num_runs || split < 0 || split >= p.num_splits) return;  // whole work-group
    } else if (p.work) {
        const int item = bid / p.n_kv;
        kvh = bid % p.n_kv;
        run = uniform_load(p.work + 2 * item);
        split = uniform_load(p.work + 2 * item + 1);
        if (run < 0 || run >= p.num_runs || split < 0 || split >= p.num_splits) return;  // whole work-group
    } else {
        run = bid;
        kvh = blockIdx.y;
        split = blockIdx.z;
    }

    // f16 pages run on MFMA (MF); f32 pages on the VALU.
    constexpr bool MF = sizeof(T) == 2;
    // Each wave's region of LDS: its partial (ROWS x D floats) at the end of
    // its page walk, and on f16 pages, before that, the staged keys of its
    // current page (16 x 128 f16 = 4 KiB).
    // On MFMA the 16 lanes of a lane group store 16 rows' float4s at one dim: a
    // row pitch of D + 4 floats puts them on distinct banks (measured: at a
    // pitch of D, 32 conflict cycles per store at 10 rows, none at D + 4).
    constexpr int RP = MF ? D + 4 : D;                              // floats per row
    constexpr int RW = MF && ROWS * RP < 1024 ? 1024 : ROWS * RP;  // floats per wave
    __shared__ __align__(16) float red_acc[kWaves * RW];
    __shared__ float red_m[ROWS][kWaves], red_l[ROWS][kWaves];
    auto red_row = [&](int row, int w) { return &red_acc[w * RW + row * RP]; };
    // q passes through LDS for MF (each lane then loads its column's operand),
    // and for f32 pages with many rows (a verify run), where each row's slice is
    // read again per page: holding every row's q in registers as well would
    // push the kernel past 256 VGPRs (one wave per SIMD).
    constexpr bool Q_LDS = MF || ROWS > 4;
    __shared__ __align__(16) T q_lds[(FUSED || Q_LDS) ? ROWS : 1][D];
    __shared__ __align__(16) T new_k[NEW][D], new_v[NEW][D];
    __shared__ int merge_here;
    __shared__ int merge_ctx[ROWS];  // the keys each row sees, for the in-kernel merge

    // The run: list entries first .. first + nq - 1, one sequence. Its rows are
    // (token i, head kvh * G + g) for row = i * G + g < nrows; rows nrows ..
    // ROWS - 1 repeat the last real row, so the page loop always computes ROWS
    // rows with no per-row tests (their results are never stored).
    const int first = have_desc ? desc[2] : p.run_first ? uniform_load(p.run_first + run) : run;
    int nq = have_desc ? desc[3] : p.run_count ? uniform_load(p.run_count + run) : 1;
    nq = max(1, min(min(nq, ROWS / G), FUSED ? NEW : ROWS));  // FUSED: new_k / new_v hold NEW tokens
    const int nrows = nq * G;
    auto src_row = [&](int row) { return min(row, nrows - 1); };
    // Token and position of the run's entry i: with a counting descriptor both
    // are arithmetic, otherwise two dependent scalar loads.
    const bool counting = have_desc && desc[kDescTok] >= 0;
    auto token_of = [&](int i) {
        if (counting) return desc[kDescTok] + i;
        return p.token_index ? uniform_load(p.token_index + first + i) : first + i;
    };
    auto pos_of = [&](int i) { return counting ? desc[5] + i : uniform_load(p.positions + token_of(i)); };
    const int seq = have_desc ? desc[4] : uniform_load(p.token_seq + token_of(0));
    const int32_t *table = pre.tables + static_cast<int64_t>(seq) * p.max_blocks;

    // Per-row positions (for masking and RoPE); the page range needs only the
    // lowest and highest, which the descriptor already holds.
    int row_pos[ROWS];
    int min_pos = INT_MAX, max_pos = -1;
#pragma unroll
    for (int row = 0; row < ROWS; row++) {
        row_pos[row] = pos_of(src_row(row) / G);
        min_pos = min(min_pos, row_pos[row]);
        max_pos = max(max_pos, row_pos[row]);
    }
    if (have_desc) {
        min_pos = desc[5];
        max_pos = desc[6];
    }
    const int ctx_max = min(max_pos + 1, p.max_blocks * kPage);
    const int begin = split * p.split_len;
    if (begin >= ctx_max) return;  // a split past the run's context: nothing reads its partial
    const int end = min(ctx_max, begin + p.split_len);
    const int run_splits = (ctx_max + p.split_len - 1) / p.split_len;

    const T *kbase = static_cast<const T *>(pre.k);
    const T *vbase = static_cast<const T *>(pre.v);
    const int64_t head_off = static_cast<int64_t>(kvh) * (kPage * kHeadDim);
    const int64_t block_stride = static_cast<int64_t>(p.n_kv) * (kPage * kHeadDim);

    // The page walk: wave w takes pages first_page + w, first_page + w + 4, ...
    // (n of them). Every page of the loop is fetched the same way, so each use
    // waits at a fixed vmcnt: a fetch past the wave's last page gets a
    // descriptor with no records (its loads return 0 and touch no memory), and
    // a block id outside the pool is read as a page of zeros the same way (the
    // host plan never hands such an id to the kernel).
    const int first_page = begin / kPage, last_page = (end - 1) / kPage;
    const int n = first_page + wave <= last_page ? (last_page - first_page - wave) / kWaves + 1 : 0;
    auto page_of = [&](int j) { return first_page + wave + j * kWaves; };
    auto in_pool = [&](int blk) { return blk >= 0 && blk < p.num_blocks; };
    // Lane offsets and load steps within a half page. f32: lane l at 32 l,
    // loads 2 KiB apart (keys 4 i + r, dims 8 c .. 8 c + 7), K and V alike.
    // f16: V four whole key rows per load (keys 4 r + i, dims 8 c .. 8 c + 7).
    const uint32_t k_off = 32u * lane, k_step = 2048u;
    const uint32_t v_off = MF ? 1024u * r + 16u * c : 32u * lane, v_step = MF ? 256u : 2048u;
    // f16 keys go through this wave's LDS region, 16-byte chunks swizzled so
    // that both sides are conflict-free: LDS slot 16 k + (q ^ k) holds chunk q
    // (dims 8 q .. 8 q + 7) of key k. Load i (buffer_load_dwordx4 ... lds,
    // lane l to slot 64 i + l) then reads four whole key rows (keys 4 i + r,
    // each row's 16 chunks in a permuted order), and the scores' A operand of
    // step s (key c, chunk 4 s + r) is one ds_read_b128 whose 16 lanes of a
    // given r hit 16 different slots modulo 16.
    uint32_t *const kstage = reinterpret_cast<uint32_t *>(&red_acc[wave * RW]);
    uint32_t k_dma[4], k_rd[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        k_dma[i] = 1024u * i + 256u * r + 16u * ((c ^ (4 * i + r)) & 15);
        k_rd[i] = 64u * c + 4u * (((4 * i + r) ^ c) & 15);  // dwords
    }
    // Keys of one page of one kv head into kstage: four loads, each writing
    // 1 KiB of LDS (lane l's 16 bytes at 16 l); a descriptor with no records
    // (live = false) writes zeros.
    auto stage_keys = [&](const T *base, bool live) {
        const __amdgpu_buffer_rsrc_t d = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<T *>(base), 0, live ? kPage * D * static_cast<int>(sizeof(T)) : 0, kDescWord3);
#pragma unroll
        for (int i = 0; i < 4; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(d, (__attribute__((address_space(3))) void *)(kstage + 256 * i),
                                                     16, k_dma[i], 0, 0, kNonTemporal);
    };
    // The split's block ids, lane k holding page first_page + k: one vector
    // load, issued before any page load and read back per page with
    // v_readlane, so no page load waits on a scalar load of the table (under a
    // full memory queue each such round trip costs microseconds). A split has
    // at most 64 pages (split_len <= 1024, checked by the launcher).
    const int tv = first_page + lane <= last_page ? table[first_page + lane] : -1;
    auto block_at = [&](int page) { return __builtin_amdgcn_readlane(tv, page - first_page); };  // page in the split
    // The wave's page j: its keys, its values, or both, into pr.
    auto fetch_block = [&](PageRegs<T> &pr, int j, int blk, bool keys, bool values) {
        const bool live = j < n && in_pool(blk);
        const int64_t off = static_cast<int64_t>(live ? blk : 0) * block_stride + head_off;
        if constexpr (MF) {
            if (keys) stage_keys(kbase + off, live);
        } else {
            if (keys) load_half(pr.k, kbase + off, k_off, k_step, live);
        }
        if (values) load_half(pr.v, vbase + off, v_off, v_step, live);
    };
    auto block_of = [&](int j) { return block_at(min(page_of(j), last_page)); };
    auto fetch = [&](PageRegs<T> &pr, int j) { fetch_block(pr, j, block_of(j), true, true); };
    auto fetch_keys = [&](PageRegs<T> &pr, int j) { fetch_block(pr, j, block_of(j), true, false); };
    auto fetch_values = [&](PageRegs<T> &pr, int j) { fetch_block(pr, j, block_of(j), false, true); };
    // A wave's first page, whose block id the descriptor holds: the work-group
    // issues it right after the descriptor load.
    auto fetch_first = [&](PageRegs<T> &pr) {
        if (!have_desc) return fetch(pr, 0);
        const int rel = min(wave, last_page - first_page);
        int blk = desc[kDescBlocks];
        blk = rel == 1 ? desc[kDescBlocks + 1] : blk;
        blk = rel == 2 ? desc[kDescBlocks + 2] : blk;
        blk = rel == 3 ? desc[kDescBlocks + 3] : blk;
        fetch_block(pr, 0, blk, true, true);
    };

    // f32 pages: every row's state in every lane (its q slice when q is not in
    // LDS, running max, sum and 8 accumulated dims). f16 pages keep one
    // column's state per lane, declared with their page walk below.
    constexpr int FR = MF ? 1 : ROWS;
    QSlice q[Q_LDS ? 1 : FR];
    float m[FR], l[FR], acc[FR][8];
#pragma unroll
    for (int row = 0; row < FR; row++) {
        m[row] = kNoMax;
        l[row] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) acc[row][e] = 0.0f;
    }
    PageRegs<T> A;

    if constexpr (!FUSED) {
        if constexpr (Q_LDS) {
            // rows' q vectors into LDS, 8 elements per thread at a time
            for (int idx = tid; idx < nrows * (D / 8); idx += kThreads) {
                const int row = idx / (D / 8), d8 = (idx % (D / 8)) * 8;
                const int li = first + row / G;  // per thread: a vector load when looked up
                const int t = counting ? desc[kDescTok] + row / G : p.token_index ? p.token_index[li] : li;
                const T *src = static_cast<const T *>(p.q) + (static_cast<int64_t>(t) * p.n_heads + kvh * G + row % G) * D + d8;
#pragma unroll
                for (int e = 0; e < 8; e++) q_lds[row][d8 + e] = src[e];
            }
        } else {
#pragma unroll
            for (int row = 0; row < ROWS; row++) {
                const int t = token_of(src_row(row) / G);
                const int head = kvh * G + src_row(row) % G;
                load_q(q[row], static_cast<const T *>(p.q) + (static_cast<int64_t>(t) * p.n_heads + head) * D + 8 * c);
            }
        }
        fetch_first(A);
        if constexpr (Q_LDS) __syncthreads();
    } else {
        // q of every row and the new K/V in this split, one head vector per
        // wave at a time; lane l holds dims l and l + 64 (a rotary pair). Wave
        // w takes rows w, w + 4, ... and new tokens w, w + 4, ...; all of
        // their loads are issued before the first is used, and before the
        // wave's first pages, so the prologue costs one memory round trip (a
        // verify run of 5 tokens gives a wave up to 3 rows and 2 tokens: one
        // after another, under a full memory queue, they took about 4 round
        // trips) and the arithmetic overlaps the page loads. The barrier after
        // it waits for LDS only, not for the pages.
        const int n_total = p.n_heads + 2 * p.n_kv;
        const T *qkv = static_cast<const T *>(pre.qkv);
        auto vec = [&](int t, int head) { return qkv + (static_cast<int64_t>(t) * n_total + head) * D; };
        const int kh = p.n_heads + kvh, vh = p.n_heads + p.n_kv + kvh;

        constexpr int RQ = (ROWS + kWaves - 1) / kWaves;                        // rows per wave, at most
        constexpr int NT = ((NEW < ROWS ? NEW : ROWS) + kWaves - 1) / kWaves;  // new tokens per wave, at most
        T qa[RQ], qb[RQ], ka[NT], kb[NT], va[NT], vb[NT];  // a row or token past the run loads the last again
#pragma unroll
        for (int k = 0; k < RQ; k++) {
            const int row = min(wave + k * kWaves, nrows - 1);
            const T *qs = vec(token_of(row / G), kvh * G + row % G);
            qa[k] = qs[lane];
            qb[k] = qs[lane + D / 2];
        }
#pragma unroll
        for (int k = 0; k < NT; k++) {
            const int t = token_of(min(wave + k * kWaves, nq - 1));
            const T *ks = vec(t, kh), *vs = vec(t, vh);
            ka[k] = ks[lane];
            kb[k] = ks[lane + D / 2];
            va[k] = vs[lane];
            vb[k] = vs[lane + D / 2];
        }
        const NormRopeLane qn = norm_rope_lane(p.q_norm, pre.inv_freq, lane);
        const NormRopeLane kn = norm_rope_lane(p.k_norm, pre.inv_freq, lane);

        fetch_first(A);

        auto put_q = [&](int row, float x0, float x1, int pos) {
            const int head = kvh * G + row % G;
            if (p.bias) {
                x0 = x0 + p.bias[head * D + lane];
                x1 = x1 + p.bias[head * D + lane + D / 2];
            }
            qk_norm_rope(x0, x1, p.q_norm != nullptr, qn, p.eps, pos);
            q_lds[row][lane] = from_f32<T>(x0);
            q_lds[row][lane + D / 2] = from_f32<T>(x1);
        };
        auto put_kv = [&](int i, float k0, float k1, float v0, float v1, int pos) {
            if (p.bias) {
                k0 = k0 + p.bias[kh * D + lane];
                k1 = k1 + p.bias[kh * D + lane + D / 2];
                v0 = v0 + p.bias[vh * D + lane];
                v1 = v1 + p.bias[vh * D + lane + D / 2];
            }
            qk_norm_rope(k0, k1, p.k_norm != nullptr, kn, p.eps, pos);
            const T ek0 = to_page<T>(k0), ek1 = to_page<T>(k1), ev0 = to_page<T>(v0), ev1 = to_page<T>(v1);
            new_k[i][lane] = ek0;
            new_k[i][lane + D / 2] = ek1;
            new_v[i][lane] = ev0;
            new_v[i][lane + D / 2] = ev1;
            const int blk = block_at(pos / kPage);  // the token's page lies in this split
            if (in_pool(blk)) {
                const int64_t off = static_cast<int64_t>(blk) * block_stride + head_off + (pos % kPage) * D;
                T *kd = const_cast<T *>(kbase) + off;
                T *vd = const_cast<T *>(vbase) + off;
                kd[lane] = ek0;
                kd[lane + D / 2] = ek1;
                vd[lane] = ev0;
                vd[lane + D / 2] = ev1;
            }
        };
        // A new token is appended by the work-group whose split holds its position.
        auto in_split = [&](int pos) { return pos >= begin && pos < end; };

#pragma unroll
        for (int k = 0; k < RQ; k++) {
            const int row = wave + k * kWaves;
            if (row < nrows) put_q(row, to_f32(qa[k]), to_f32(qb[k]), pos_of(row / G));
        }
#pragma unroll
        for (int k = 0; k < NT; k++) {
            const int i = wave + k * kWaves;
            if (i >= nq) continue;
            const int pos = pos_of(i);
            if (in_split(pos)) put_kv(i, to_f32(ka[k]), to_f32(kb[k]), to_f32(va[k]), to_f32(vb[k]), pos);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        if constexpr (!Q_LDS) {
#pragma unroll
            for (int row = 0; row < ROWS; row++) load_q(q[row], &q_lds[src_row(row)][8 * c]);
        }
    }

    // The page walk: each wave holds one page in registers and loads the next
    // page's keys once this page's scores are done, its values once this
    // page's values are done, so half a page is in flight while the wave
    // computes. With 16 waves per CU that keeps the memory system as busy as
    // two whole pages per wave did, with shorter queues.
    // The wave's fast pages come first (pages below min_pos / 16 hold no new key
    // and only keys every row sees); they run through a loop with no masking.
    // The rest (the run's positions, at most EMBER_MAX_RUN and consecutive, lie
    // in at most two adjacent pages, of which a wave at stride 4 gets at most
    // one) goes through the masked path.
    const int fast_end = min_pos / kPage;
    const int n_fast = first_page + wave < fast_end ? min(n, (fast_end - 1 - first_page - wave) / kWaves + 1) : 0;
    using Fast = std::false_type;
    using Masked = std::true_type;
    __builtin_amdgcn_s_setprio(0);
    if constexpr (MF) {
        // Lane (r, c) serves query column c, the run's row src_row(c): its q
        // operand (dims 32 i + 8 r .. + 7 for score step i), its position, and
        // its running max m, its own keys' weight sum l and 32 accumulated dims
        // (o[t][v]: dim 32 r + 8 v + t).
        u32x4 qf[4];
#pragma unroll
        for (int i = 0; i < 4; i++) qf[i] = *reinterpret_cast<const u32x4 *>(&q_lds[src_row(c)][32 * i + 8 * r]);
        int my_pos = row_pos[0];
#pragma unroll
        for (int k = 1; k < ROWS; k++) my_pos = src_row(c) == k ? row_pos[k] : my_pos;
        float mc = kNoMax, lc = 0.0f;
        f32x4 o[8];
#pragma unroll
        for (int t = 0; t < 8; t++) o[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

        // One page: the scores and the online softmax (which rescales o), then
        // the value products with the page's weights. MASKED = false: every key
        // is visible to every row (the page lies below the run's lowest
        // position). MASKED = true: a key past the column's position scores
        // -inf, so it weighs 0 and leaves the max alone; for a fully visible
        // page both forms compute the same bits. The two halves read only pr.k
        // and only pr.v, so a wave can load the next page's keys between them.
        // The staged keys as the scores' A operand: key c, dims 32 i + 8 r .. + 7.
        auto read_keys = [&](u32x4 (&kf)[4]) {
#pragma unroll
            for (int i = 0; i < 4; i++) kf[i] = *reinterpret_cast<const u32x4 *>(kstage + k_rd[i]);
        };
        auto scores = [&](const u32x4 (&kf)[4], int page, auto masked_tag) {
            constexpr bool MASKED = decltype(masked_tag)::value;
            // s[v]: the raw score of key 4 r + v against row src_row(c); the
            // softmax scale is applied in the exponent.
            f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int i = 0; i < 4; i++) s = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_f16x8(kf[i]), as_f16x8(qf[i]), s, 0, 0, 0);
            if constexpr (MASKED) {
                const int key0 = page * kPage + 4 * r;
#pragma unroll
                for (int v = 0; v < 4; v++) s[v] = key0 + v > my_pos ? -INFINITY : s[v];
            }
            // The running max is in scaled units: round(scale * max s) is the
            // max of the rounded scaled scores (scale > 0, rounding monotonic).
            // m starts at kNoMax, not -inf, so mn is always finite, and corr is
            // 2^0 = 1 exactly when the max stays. The weights are rounded to
            // f16 (to nearest), the value products' operand; the sum takes the
            // same rounded weights, so numerator and denominator agree.
            const float mn = fmaxf(mc, groups_max(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]))) * p.scale_log2);
            f16x4 w;
#pragma unroll
            for (int v = 0; v < 4; v++) w[v] = static_cast<f16>(exp2_hw(__builtin_fmaf(s[v], p.scale_log2, -mn)));
            const float corr = exp2_hw(mc - mn);
            const f16x2 ones = {static_cast<f16>(1.0f), static_cast<f16>(1.0f)};
            lc = __builtin_amdgcn_fdot2(w.zw, ones, __builtin_amdgcn_fdot2(w.xy, ones, lc * corr, false), false);
#pragma unroll
            for (int t = 0; t < 8; t++) o[t] = o[t] * corr;
            mc = mn;
            return w;
        };
        auto values = [&](const PageRegs<T> &pr, f16x4 w) {
            o[0] = __builtin_amdgcn_mfma_f32_16x16x16f16(value_tile<0>(pr.v), w, o[0], 0, 0, 0);
            o[1] = __builtin_amdgcn_mfma_f32_16x16x16f16(value_tile<1>(pr.v), w, o[1], 0, 0, 0);
            o[2] = __builtin_amdgcn_mfma_f32_16x16x16f16(value_tile<2>(pr.v), w, o[2], 0, 0, 0);
            o[3] = __builtin_amdgcn_mfma_f32_16x16x16f16(value_tile<3>(pr.v), w, o[3], 0, 0, 0);
            o[4] = __builtin_amdgcn_mfma_f32_16x16x16f16(value_tile<4>(pr.v), w, o[4], 0, 0, 0);
            o[5] = __builtin_amdgcn_mfma_f32_16x16x16f16(value_tile<5>(pr.v), w, o[5], 0, 0, 0);
            o[6] = __builtin_amdgcn_mfma_f32_16x16x16f16(value_tile<6>(pr.v), w, o[6], 0, 0, 0);
            o[7] = __builtin_amdgcn_mfma_f32_16x16x16f16(value_tile<7>(pr.v), w, o[7], 0, 0, 0);
        };
        // A page of the masked part: the fused form first puts this launch's
        // new keys into the page they land in (in place: the registers are
        // reloaded after use anyway); then V slots past the run's last
        // position read as 0.
        auto consume = [&](PageRegs<T> &pr, int page) {
            u32x4 kf[4];
            read_keys(kf);
            if constexpr (FUSED) {
                if (page * kPage <= max_pos && (page + 1) * kPage > min_pos) {
                    const int jk = page * kPage + c - min_pos;  // this lane's key; the run's positions are consecutive
                    const int jkc = min(max(jk, 0), nq - 1);
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        kf[i] = select4(jk >= 0 && jk < nq, *reinterpret_cast<const u32x4 *>(&new_k[jkc][32 * i + 8 * r]), kf[i]);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int jv = page * kPage + 4 * r + i - min_pos;  // this lane's value key i
                        const int jvc = min(max(jv, 0), nq - 1);
                        pr.v[i] = select4(jv >= 0 && jv < nq, *reinterpret_cast<const u32x4 *>(&new_v[jvc][8 * c]), pr.v[i]);
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < 4; i++) pr.v[i] = select4(page * kPage + 4 * r + i > max_pos, u32x4{0, 0, 0, 0}, pr.v[i]);
            const f16x4 w = scores(kf, page, Masked{});
            values(pr, w);
        };

        int j = 0;
        for (; j < n_fast; j++) {
            u32x4 kf[4];
            read_keys(kf);
            const f16x4 w = scores(kf, page_of(j), Fast{});
            phase_break();
            fetch_keys(A, j + 1);
            phase_break();
            values(A, w);
            phase_break();
            fetch_values(A, j + 1);
            phase_break();
        }
        for (; j < n; j++) {
            consume(A, page_of(j));
            phase_break();
            fetch(A, j + 1);
            phase_break();
        }

        // The wave's last key fetch (past its last page: a descriptor with no
        // records) still writes zeros into its stage, the LDS its partial goes
        // to next, so every load of the wave completes first.
        __builtin_amdgcn_s_waitcnt(0);
        // The column's sum over its lane groups; its lanes write its partial.
        lc = groups_sum(lc);
        if (c < nrows) {
#pragma unroll
            for (int v = 0; v < 4; v++) {
                float *dst = red_row(c, wave) + 32 * r + 8 * v;
                *reinterpret_cast<float4 *>(dst) = make_float4(o[0][v], o[1][v], o[2][v], o[3][v]);
                *reinterpret_cast<float4 *>(dst + 4) = make_float4(o[4][v], o[5][v], o[6][v], o[7][v]);
            }
            if (r == 0) {
                red_m[c][wave] = mc;
                red_l[c][wave] = lc;
            }
        }
    } else {
        // One page: scores and online softmax for every row, then the values key by
        // key (each key's 8 dims converted once, used by every row). Per row the
        // operations and their order are: rescale by corr, then fma over keys 0..3.
        // MASKED = false: every key of the page is visible to every row (the page
        // lies below the run's lowest position). MASKED = true: per-row visibility,
        // with selects, so a hidden key leaves a row's state bit-for-bit unchanged;
        // for a fully visible page both forms compute the same bits. The two halves
        // read only pr.k and only pr.v, so a wave can load the next page's keys
        // between them.
        const int quad = c >> 2;
        const bool upper_half = c >= 8, odd_quad = (c & 4) != 0;
        auto scores = [&](const PageRegs<T> &pr, int page, auto masked_tag, Weights (&pj)[ROWS], bool (&vis)[ROWS][4]) {
            constexpr bool MASKED = decltype(masked_tag)::value;
            const int key0 = page * kPage + r;  // position of this lane's key i = 0; key i is key0 + 4 i
#pragma unroll
            for (int row = 0; row < ROWS; row++) {
                QSlice qrow;
                if constexpr (Q_LDS) load_q(qrow, &q_lds[src_row(row)][8 * c]);
                else qrow = q[row];
                float x[4];
#pragma unroll
                for (int i = 0; i < 4; i++) x[i] = dot8(qrow, pr.k[i]);
                // This lane's key (quad q of the DPP row: key 4 q + r of the page),
                // its raw score; the softmax scale is applied in the exponent.
                float sq = key_sums(x, upper_half, odd_quad);
                if constexpr (MASKED) {
#pragma unroll
                    for (int i = 0; i < 4; i++) vis[row][i] = key0 + 4 * i <= row_pos[row];
                    if (key0 + 4 * quad > row_pos[row]) sq = -INFINITY;
                }
                // The running max m is in scaled units: round(scale * max s) is the
                // max of the rounded scaled scores (scale > 0, rounding monotonic).
                // m starts at kNoMax, not -inf, so mn is always finite: no select
                // guards the subtraction, and corr is 2^0 = 1 exactly when the max
                // stays. One exponential per lane: its own key's weight.
                const float mn = fmaxf(m[row], quads_max(sq) * p.scale_log2);
                const float pq = exp2_hw(__builtin_fmaf(sq, p.scale_log2, -mn));  // 2^-inf = 0 for a hidden key
                pj[row].w[0] = quad_value<0>(pq);
                pj[row].w[1] = quad_value<1>(pq);
                pj[row].w[2] = quad_value<2>(pq);
                pj[row].w[3] = quad_value<3>(pq);
                const float corr = exp2_hw(m[row] - mn);
                l[row] = l[row] * corr + quads_sum(pq);
#pragma unroll
                for (int e = 0; e < 8; e++) acc[row][e] = acc[row][e] * corr;
                m[row] = mn;
            }
        };
        auto values = [&](const PageRegs<T> &pr, auto masked_tag, const Weights (&pj)[ROWS], const bool (&vis)[ROWS][4]) {
            constexpr bool MASKED = decltype(masked_tag)::value;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float vf[8];
                unpack8(pr.v[i], vf);
#pragma unroll
                for (int row = 0; row < ROWS; row++) {
                    if constexpr (!MASKED) {
#pragma unroll
                        for (int e = 0; e < 8; e++) acc[row][e] = fmaf(pj[row].w[i], vf[e], acc[row][e]);
                    } else {
#pragma unroll
                        for (int e = 0; e < 8; e++)
                            acc[row][e] = vis[row][i] ? fmaf(pj[row].w[i], vf[e], acc[row][e]) : acc[row][e];
                    }
                }
            }
        };
        // A page of the masked part: the fused form first puts this launch's new
        // keys into the page they land in (in place: the registers are reloaded
        // after use anyway).
        auto consume = [&](PageRegs<T> &pr, int page) {
            if constexpr (FUSED) {
                if (page * kPage <= max_pos && (page + 1) * kPage > min_pos) {
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int j = page * kPage + r + 4 * i - min_pos;  // the run's positions are consecutive
                        const int jc = min(max(j, 0), nq - 1);
                        put_key(pr, i, j >= 0 && j < nq, &new_k[jc][8 * c], &new_v[jc][8 * c]);
                    }
                }
            }
            Weights pj[ROWS];
            bool vis[ROWS][4];
            scores(pr, page, Masked{}, pj, vis);
            values(pr, Masked{}, pj, vis);
        };

        int j = 0;
        for (; j < n_fast; j++) {
            Weights pj[ROWS];
            bool vis[ROWS][4];
            scores(A, page_of(j), Fast{}, pj, vis);
            phase_break();
            fetch_keys(A, j + 1);
            phase_break();
            values(A, Fast{}, pj, vis);
            phase_break();
            fetch_values(A, j + 1);
            phase_break();
        }
        for (; j < n; j++) {
            consume(A, page_of(j));
            phase_break();
            fetch(A, j + 1);
            phase_break();
        }

        // Merge the four DPP rows of the wave (rows 0+1 and 2+3, then the pairs).
#pragma unroll
        for (int row = 0; row < ROWS; row++) {
            if (row >= nrows) continue;
            merge_lanes(m[row], l[row], acc[row], 16);
            merge_lanes(m[row], l[row], acc[row], 32);
            if (r == 0) {
#pragma unroll
                for (int e = 0; e < 8; e++) red_row(row, wave)[8 * c + e] = acc[row][e];
                if (c == 0) {
                    red_m[row][wave] = m[row];
                    red_l[row][wave] = l[row];
                }
            }
        }
    }
    __syncthreads();

    // Merge the waves in order 0..3, then write the output (a run with one
    // split) or this split's partial.
    const bool direct = p.counters ? run_splits == 1 : p.num_splits == 1;
    for (int idx = tid; idx < nrows * D; idx += kThreads) {
        const int row = idx / D, d = idx % D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; w++) M = fmaxf(M, red_m[row][w]);
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; w++) {
            const float mw = red_m[row][w];
            const float f = mw == -INFINITY ? 0.0f : exp2_hw(mw - M);
            L = L + red_l[row][w] * f;
            O = O + red_row(row, w)[d] * f;
        }
        const int li = first + row / G;
        const int head = kvh * G + row % G;
        if (direct) {
            const int t = counting ? desc[kDescTok] + row / G : p.token_index ? p.token_index[li] : li;
            T *o = static_cast<T *>(p.out) + (static_cast<int64_t>(t) * p.n_heads + head) * D;
            o[d] = from_f32<T>(L > 0.0f ? O / L : 0.0f);
        } else {
            const int64_t slot = (static_cast<int64_t>(li) * p.n_heads + head) * p.num_splits + split;
            put_partial(p.part_acc + slot * D + d, O);
            if (d == 0) {
                put_partial(p.part_ml + slot * 2, M);
                put_partial(p.part_ml + slot * 2 + 1, L);
            }
        }
    }
    if (direct || !p.counters) return;

    // In-kernel split merge: every work-group of this (run, kv head) counts in
    // once its partial stores have completed (they are device-coherent sc1
    // stores, so completion is visibility); the last one merges, reading the
    // partials with device-coherent loads, and resets the counter for the next
    // launch. Nothing waits on another work-group.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        uint32_t *counter = p.counters + static_cast<int64_t>(run) * p.n_kv + kvh;
        const uint32_t before = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        merge_here = before + 1 == static_cast<uint32_t>(run_splits);
        if (merge_here) {
            __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int row = 0; row < ROWS; row++) merge_ctx[row] = min(row_pos[row] + 1, p.max_blocks * kPage);
        }
    }
    __syncthreads();
    if (!merge_here) return;
    auto ns_of = [&](int row) { return min(p.num_splits, max(1, (merge_ctx[row] + p.split_len - 1) / p.split_len)); };
    auto out_of = [&](int row) {
        const int li = first + row / G, head = kvh * G + row % G;
        const int t = counting ? desc[kDescTok] + row / G : p.token_index ? p.token_index[li] : li;
        return static_cast<T *>(p.out) + (static_cast<int64_t>(t) * p.n_heads + head) * D;
    };
    constexpr int E = (ROWS * D + kThreads - 1) / kThreads;  // elements per thread
    const int nsm = min(p.num_splits, run_splits);            // no row holds keys in more splits
    // Element by element (merge_one) where that costs one round trip (one
    // element per thread, the splits in one chunk), or where the splits are
    // too many to stage in LDS; the batched merge below otherwise.
    if ((E == 1 && nsm <= kMergeChunk) || 2 * nrows * nsm > kWaves * RW) {
        for (int idx = tid; idx < nrows * D; idx += kThreads) {
            const int row = idx / D;
            merge_one<T>(p, first + row / G, kvh * G + row % G, idx % D, merge_ctx[row], out_of(row));
        }
        return;
    }

    // The run's merge with merge_one's arithmetic in merge_one's order (the
    // same bits), its loads batched over the work-group: thread i < nrows * nsm
    // brings (M, L) of (row i / nsm, split i % nsm) into LDS with one load,
    // and every thread requests the O partials of all its elements for MS
    // splits before the first wait. Up to MS splits then cost one memory round
    // trip, where merge_one costs up to three per element and a thread merges
    // ROWS / 2 elements one after another. One thread per row then turns its
    // (M, L) pairs into weights (-1: a split without a key of the row) and L,
    // and the elements' sums read the weights with no branch. red_acc is free:
    // the partials are stored.
    constexpr int MS = E >= 12 ? 4 : 48 / E < 16 ? 48 / E : 16;
    constexpr int RC = 8;                     // splits per LDS batch of the row pass
    float *const sm = red_acc;                // M per (row, split)
    float *const sw = red_acc + nrows * nsm;  // L per (row, split), then its weight
    auto slot_of = [&](int row, int s) {
        const int li = first + row / G, head = kvh * G + row % G;
        return (static_cast<int64_t>(li) * p.n_heads + head) * p.num_splits + s;
    };
    float O[E];
    bool any[E];
#pragma unroll
    for (int e = 0; e < E; e++) {
        O[e] = 0.0f;
        any[e] = false;
    }
    for (int s0 = 0; s0 < nsm; s0 += MS) {
        // Unconditional loads, one straight run and one wait: an element past
        // the rows reads the last row, a split past the run's last reads that
        // one again, and a split past a row's last reads that row's partial of
        // the split (stored, holding no key of the row); none of them is used.
        float ov[E][MS];
#pragma unroll
        for (int e = 0; e < E; e++) {
            const int row = min((tid + e * kThreads) / D, nrows - 1);
#pragma unroll
            for (int k = 0; k < MS; k++)
                ov[e][k] = get_partial(p.part_acc + slot_of(row, min(s0 + k, nsm - 1)) * D + tid % D);
        }
        if (s0 == 0) {
            for (int i = tid; i < nrows * nsm; i += kThreads) {
                const float2 ml = get_partial_pair(p.part_ml + slot_of(i / nsm, i % nsm) * 2);
                sm[i] = ml.x;
                sw[i] = ml.y;
            }
            __syncthreads();
            if (tid < nrows) {  // per row: M, then each split's weight and L in split order
                const int row = tid, ns = ns_of(row);
                const float *rm = sm + row * nsm;
                float *rw = sw + row * nsm;
                float M = -INFINITY;
                for (int c0 = 0; c0 < ns; c0 += RC) {
                    float mv[RC];
#pragma unroll
                    for (int k = 0; k < RC; k++) mv[k] = rm[min(c0 + k, ns - 1)];
#pragma unroll
                    for (int k = 0; k < RC; k++) M = fmaxf(M, mv[k]);  // repeats of the last split change nothing
                }
                float L = 0.0f;
                bool seen = false;
                for (int c0 = 0; c0 < ns; c0 += RC) {
                    float mv[RC], lv[RC], w[RC];
#pragma unroll
                    for (int k = 0; k < RC; k++) {
                        mv[k] = rm[min(c0 + k, ns - 1)];
                        lv[k] = rw[min(c0 + k, ns - 1)];
                    }
#pragma unroll
                    for (int k = 0; k < RC; k++) {
                        const bool use = c0 + k < ns && mv[k] != -INFINITY;
                        const float f = mv[k] == M ? 1.0f : exp2_hw(mv[k] - M);
                        const float ls = lv[k] * f;
                        L = use ? (seen ? L + ls : ls) : L;
                        seen = seen || use;
                        w[k] = use ? f : -1.0f;
                    }
#pragma unroll
                    for (int k = 0; k < RC; k++)
                        if (c0 + k < ns) rw[c0 + k] = w[k];
                }
                for (int s = ns; s < nsm; s++) rw[s] = -1.0f;
                red_l[row][0] = L;
            }
            __syncthreads();
        }
#pragma unroll
        for (int e = 0; e < E; e++) {
            const int row = min((tid + e * kThreads) / D, nrows - 1);
#pragma unroll
            for (int k = 0; k < MS; k++) {
                const float w = sw[row * nsm + min(s0 + k, nsm - 1)];
                const bool use = s0 + k < nsm && w >= 0.0f;
                const float os = ov[e][k] * w;
                O[e] = use ? (any[e] ? O[e] + os : os) : O[e];
                any[e] = any[e] || use;
            }
        }
    }
#pragma unroll
    for (int e = 0; e < E; e++) {
        const int idx = tid + e * kThreads, row = idx / D;
        if (idx >= nrows * D) continue;
        const float L = red_l[row][0];
        out_of(row)[idx % D] = from_f32<T>(L > 0.0f ? O[e] / L : 0.0f);
    }
}

template <typename T, int ROWS, bool FUSED>
__global__ void __launch_bounds__(kThreads)
    paged_decode_kernel(const WorkDesc *descs, int n_kv, const void *k, const void *v, const int32_t *tables,
                        const void *qkv, const float *inv_freq, DecodeParams p) {
    decode_item<T, ROWS, FUSED>(p, Preloaded{descs, n_kv, k, v, tables, qkv, inv_freq}, static_cast<int>(blockIdx.x),
                                static_cast<int>(threadIdx.x));
}

// The split merge as its own launch: one work-group per (token, head).
template <typename T>
__global__ void __launch_bounds__(kHeadDim) merge_splits_kernel(DecodeParams p) {
    const int li = static_cast<int>(blockIdx.x), head = static_cast<int>(blockIdx.y);
    const int t = p.token_index ? p.token_index[li] : li;
    const int ctx = min(p.positions[t] + 1, p.max_blocks * kPage);
    T *o = static_cast<T *>(p.out) + (static_cast<int64_t>(t) * p.n_heads + head) * kHeadDim;
    merge_one<T>(p, li, head, static_cast<int>(threadIdx.x), ctx, o);
}

template <typename T, int ROWS, bool FUSED>
hipError_t launch_rows(const DecodeParams &p, int runs, int num_work, hipStream_t stream, hipEvent_t start,
                       hipEvent_t stop) {
    const dim3 grid = p.work ? dim3(static_cast<unsigned>(num_work * p.n_kv))
                             : dim3(static_cast<unsigned>(runs), static_cast<unsigned>(p.n_kv),
                                    static_cast<unsigned>(p.num_splits));
    // The descriptors go with the work list only (a launch without one indexes by grid position).
    const WorkDesc *descs = p.work && p.work_desc ? reinterpret_cast<const WorkDesc *>(p.work_desc) : nullptr;
    if (start || stop)
        hipExtLaunchKernelGGL((paged_decode_kernel<T, ROWS, FUSED>), grid, dim3(kThreads), 0, stream, start, stop, 0,
                              descs, p.n_kv, p.k, p.v, p.tables, p.qkv, p.inv_freq, p);
    else
        hipLaunchKernelGGL((paged_decode_kernel<T, ROWS, FUSED>), grid, dim3(kThreads), 0, stream, descs, p.n_kv, p.k,
                           p.v, p.tables, p.qkv, p.inv_freq, p);
    return hipGetLastError();
}

template <typename T, bool FUSED>
hipError_t launch_typed(const DecodeParams &p, int runs, int num_work, int rows, hipStream_t stream, hipEvent_t start,
                        hipEvent_t stop) {
    switch (rows) {
        case 1: return launch_rows<T, 1, FUSED>(p, runs, num_work, stream, start, stop);
        case 2: return launch_rows<T, 2, FUSED>(p, runs, num_work, stream, start, stop);
        case 4: return launch_rows<T, 4, FUSED>(p, runs, num_work, stream, start, stop);
        case 8: return launch_rows<T, 8, FUSED>(p, runs, num_work, stream, start, stop);
        case 10: return launch_rows<T, 10, FUSED>(p, runs, num_work, stream, start, stop);
        case 16: return launch_rows<T, 16, FUSED>(p, runs, num_work, stream, start, stop);
        default: return hipErrorInvalidValue;
    }
}

DecodeParams params_of(const EmberAttnArgs &a) {
    DecodeParams p{};
    p.q = a.q;
    p.k = a.k_cache;
    p.v = a.v_cache;
    p.positions = a.positions;
    p.token_seq = a.token_seq;
    p.tables = a.block_tables;
    p.token_index = a.token_index;
    p.run_first = a.run_first;
    p.run_count = a.run_count;
    p.work = a.work;
    p.work_desc = a.work_desc;
    p.out = a.out;
    p.part_acc = a.part_acc;
    p.part_ml = a.part_ml;
    p.counters = a.merge_counters;
    p.max_blocks = a.max_blocks;
    p.n_heads = a.n_heads;
    p.n_kv = a.n_kv;
    p.G = a.n_heads / a.n_kv;
    p.num_blocks = a.num_blocks;
    p.num_splits = a.num_splits;
    p.split_len = a.split_len;
    p.num_runs = a.run_first ? a.num_runs : a.T;
    p.scale_log2 = a.scale * kLog2e;
    return p;
}

hipError_t launch(const DecodeParams &p, const EmberAttnArgs &a, int rows, bool fused, hipStream_t stream,
                  hipEvent_t start, hipEvent_t stop) {
    if (p.num_runs <= 0 || (a.work && a.num_work <= 0)) return hipSuccess;
    hipError_t e;
    if (a.dtype == EMBER_DTYPE_F16)
        e = fused ? launch_typed<f16, true>(p, p.num_runs, a.num_work, rows, stream, start, stop)
                  : launch_typed<f16, false>(p, p.num_runs, a.num_work, rows, stream, start, stop);
    else
        e = fused ? launch_typed<float, true>(p, p.num_runs, a.num_work, rows, stream, start, stop)
                  : launch_typed<float, false>(p, p.num_runs, a.num_work, rows, stream, start, stop);
    if (e != hipSuccess || a.num_splits == 1 || a.merge_counters) return e;
    const dim3 grid(static_cast<unsigned>(a.T), static_cast<unsigned>(a.n_heads));
    if (a.dtype == EMBER_DTYPE_F16)
        hipLaunchKernelGGL(merge_splits_kernel<f16>, grid, dim3(kHeadDim), 0, stream, p);
    else
        hipLaunchKernelGGL(merge_splits_kernel<float>, grid, dim3(kHeadDim), 0, stream, p);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_paged_decode(const EmberAttnArgs &a, int rows, hipStream_t stream, hipEvent_t start,
                               hipEvent_t stop) {
    if (a.T <= 0) return hipSuccess;
    return launch(params_of(a), a, rows, false, stream, start, stop);
}

hipError_t launch_decode_step(const EmberQkvArgs &qa, const EmberAttnArgs &a, int rows, hipStream_t stream,
                              hipEvent_t start, hipEvent_t stop) {
    if (a.T <= 0) return hipSuccess;
    DecodeParams p = params_of(a);
    p.qkv = qa.qkv;
    p.q_norm = qa.q_norm;
    p.k_norm = qa.k_norm;
    p.bias = qa.bias;
    p.inv_freq = qa.inv_freq;
    p.eps = qa.eps;
    return launch(p, a, rows, true, stream, start, stop);
}

}  // namespace ember::hip
