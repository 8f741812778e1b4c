// HipBackend: the reference's Backend (src/backend/backend.hpp:94-123) on one
// MI355X, built around this library's paged-KV path (HipPagedKv) and kernels.
//
// Structure follows the reference's CudaBackend (src/backend/cuda/cuda_backend.cu
// :84-205 forward, :288-374 the layer sequence, :586-704 weight loading):
//   - weights in f16 on the device: q/k/v projections concatenated into one
//     [Q + 2KV, H] matrix, gate and up interleaved row by row into [2I, H]
//     (so the GEMV's silu_mul epilogue sees gate_j, up_j side by side), norms
//     in f32; a tied model's LM head is its embedding;
//   - per step: embedding, then per layer the input RMSNorm, the qkv GEMV, the
//     path's append + attention (decode runs, prefill tiles, fused decode),
//     the o GEMV into the f32 residual, the post-attention RMSNorm, gate/up
//     with silu_mul and the down GEMV into the residual; the final RMSNorm of
//     the logit rows and the LM head into f32 logits, kept on the device;
//   - sampling and token probabilities on the device (ember_hip_sample /
//     ember_hip_token_probs), logits copied out on request.
// Every launch goes to one stream of default priority. Decode-sized GEMVs
// take up to 64 rows; larger steps (prompt chunks) run them 64 rows at a time.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <initializer_list>
#include <memory>
#include <string>
#include <tuple>
#include <utility>
#include <unordered_map>
#include <vector>

#include "backend/backend.hpp"
#include "backend/hip_paged_kv.hpp"
#include "common/error.hpp"
#include "ember_hip.h"
#include "model/safetensors.hpp"

#define HIPB_CHECK(expr)                                                                            \
    do {                                                                                            \
        hipError_t err_ = (expr);                                                                   \
        if (err_ != hipSuccess) ::ember::fail("{} failed: {}", #expr, hipGetErrorString(err_));       \
    } while (0)

namespace ember {

namespace {

std::atomic<int64_t> g_graph_replays{0};   // whole-step graphs launched, every backend of the process
std::atomic<int64_t> g_graph_captures{0};  // whole-step graphs captured and instantiated

void check_abi(int code, const char *what) {
    if (code != EMBER_OK) fail("{}: {}", what, ember_hip_last_error());
}

// IEEE binary16 bits of a float, round to nearest even, clamped to the finite
// range first (as the reference's weight conversion clamps).
uint16_t half_bits(float f) {
    f = std::min(std::max(f, -65504.0f), 65504.0f);
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t absx = x & 0x7fffffffu;
    if (absx > 0x7f800000u) return static_cast<uint16_t>(sign | 0x7e00u);  // NaN
    const int exp = static_cast<int>(absx >> 23) - 127;
    if (exp < -24) {  // below half the smallest subnormal (or exactly zero): signed zero, or the smallest subnormal
        if (exp == -25 && (absx & 0x7fffffu)) return static_cast<uint16_t>(sign | 1u);  // above 2^-25: rounds up
        return static_cast<uint16_t>(sign);
    }
    uint32_t mant = (absx & 0x7fffffu) | 0x800000u;  // 24 significant bits
    if (exp < -14) {                                  // subnormal half: keep 24 - (-14 - exp) - 13 bits
        const int shift = 13 + (-14 - exp);
        const uint32_t kept = mant >> shift, rest = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
        const uint32_t r = kept + (rest > half || (rest == half && (kept & 1u)));
        return static_cast<uint16_t>(sign | r);  // a carry into the exponent field is the right normal value
    }
    const uint32_t kept = mant >> 13, rest = mant & 0x1fffu;
    uint32_t r = (static_cast<uint32_t>(exp + 15) << 10) | (kept & 0x3ffu);
    r += rest > 0x1000u || (rest == 0x1000u && (kept & 1u));  // a carry rolls into the exponent, as it should
    return static_cast<uint16_t>(sign | r);
}

float bf16_to_float(uint16_t b) {
    const uint32_t x = static_cast<uint32_t>(b) << 16;
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}

float half_to_float(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu, x;
    if (exp == 0x1f) {
        x = sign | 0x7f800000u | (mant << 13);
    } else if (exp == 0) {
        if (mant == 0) {
            x = sign;
        } else {  // subnormal: normalize
            int e = -1;
            do {
                mant <<= 1;
                e++;
            } while (!(mant & 0x400u));
            x = sign | (static_cast<uint32_t>(127 - 15 - e) << 23) | ((mant & 0x3ffu) << 13);
        }
    } else {
        x = sign | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}

float element(const TensorView &t, int64_t i) {
    switch (t.dtype) {
        case DType::f32: return static_cast<const float *>(t.data)[i];
        case DType::f16: return half_to_float(static_cast<const uint16_t *>(t.data)[i]);
        case DType::bf16: return bf16_to_float(static_cast<const uint16_t *>(t.data)[i]);
        default: fail("tensor {}: weights must be F32, F16 or BF16 (got {})", t.name, dtype_name(t.dtype));
    }
}

// Device memory, freed on destruction.
class DeviceMem {
public:
    DeviceMem() = default;
    explicit DeviceMem(size_t bytes) : bytes_(bytes) { HIPB_CHECK(hipMalloc(&p_, std::max<size_t>(bytes, 1))); }
    ~DeviceMem() {
        if (p_) (void)hipFree(p_);
    }
    DeviceMem(DeviceMem &&o) noexcept : p_(std::exchange(o.p_, nullptr)), bytes_(std::exchange(o.bytes_, 0)) {}
    DeviceMem &operator=(DeviceMem &&o) noexcept {
        if (this != &o) {
            if (p_) (void)hipFree(p_);
            p_ = std::exchange(o.p_, nullptr);
            bytes_ = std::exchange(o.bytes_, 0);
        }
        return *this;
    }
    template <class T = void>
    T *get() const {
        return static_cast<T *>(p_);
    }
    size_t bytes() const { return bytes_; }

private:
    void *p_ = nullptr;
    size_t bytes_ = 0;
};

struct Linear {
    int N = 0, K = 0;
    const void *w = nullptr;  // f16 [N, K], or packed for the GEMV (ember_hip_gemv_pack's layout)
    bool packed = false;
};

struct LayerWeights {
    Linear qkv, o, gate_up, down;
    const float *in_norm = nullptr, *post_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr, *qkv_bias = nullptr;
};

class HipBackend final : public Backend {
public:
    HipBackend(const std::string &dir, const BackendOptions &opt) : cfg_(ModelConfig::load(dir)), opt_(opt) {
        int count = 0;
        if (hipGetDeviceCount(&count) != hipSuccess || count == 0) fail("no HIP device found");
        EMBER_CHECK(opt_.gpu >= 0 && opt_.gpu < count, "GPU {} does not exist ({} found)", opt_.gpu, count);
        HIPB_CHECK(hipSetDevice(opt_.gpu));
        EMBER_CHECK(opt_.weights == WeightFormat::f16, "the hip backend takes f16 weights (got {})",
                    weight_format_name(opt_.weights));
        EMBER_CHECK(opt_.max_batch_tokens > 0 && opt_.max_seqs > 0, "bad batch limits");
        if (opt_.max_logit_rows <= 0) opt_.max_logit_rows = opt_.max_seqs;
        EMBER_CHECK(cfg_.hidden % 32 == 0 && cfg_.intermediate % 32 == 0 && cfg_.q_dim() % 32 == 0,
                    "hidden, intermediate and q widths must be multiples of 32 (the GEMV's k step)");
        HIPB_CHECK(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));  // default priority
        load_weights(dir);
        allocate_activations();
        create_kv();
    }

    ~HipBackend() override {
        if (stream_) (void)hipStreamSynchronize(stream_);
        for (auto &[key, exec] : graphs_) (void)hipGraphExecDestroy(exec);
        kv_.reset();
        if (host_params_) (void)hipHostFree(host_params_);
        if (host_ints_) (void)hipHostFree(host_ints_);
        if (stream_) (void)hipStreamDestroy(stream_);
    }

    std::string name() const override { return "hip"; }
    const ModelConfig &config() const override { return cfg_; }
    const BackendOptions &options() const override { return opt_; }
    int num_kv_blocks() const override { return num_blocks_; }

    MemoryInfo memory() const override {
        MemoryInfo m;
        m.weights = static_cast<int64_t>(weights_.bytes());
        m.kv_cache = kv_bytes_;
        m.activations = static_cast<int64_t>(act_bytes_);
        size_t free = 0, total = 0;
        (void)hipMemGetInfo(&free, &total);
        m.device_free = static_cast<int64_t>(free);
        m.device_total = static_cast<int64_t>(total);
        return m;
    }

    void forward(const StepBatch &b) override {
        const ModelConfig &c = cfg_;
        const int T = b.num_tokens(), S = b.num_seqs(), R = static_cast<int>(b.logit_rows.size());
        EMBER_CHECK(T > 0 && T <= opt_.max_batch_tokens, "batch of {} tokens (limit {})", T, opt_.max_batch_tokens);
        EMBER_CHECK(S <= opt_.max_seqs && R <= opt_.max_logit_rows,
                    "batch of {} sequences / {} logit rows exceeds the limits", S, R);
        EMBER_CHECK(static_cast<int>(b.positions.size()) == T, "malformed batch: {} positions for {} tokens",
                    b.positions.size(), T);
        for (int32_t t : b.tokens) EMBER_CHECK(t >= 0 && t < c.vocab_size, "token id {} outside the vocabulary", t);
        for (int32_t r : b.logit_rows) EMBER_CHECK(r >= 0 && r < T, "logit row {} outside the batch", r);
        rows_ = 0;  // until this step's logits exist
        // A pure decode step (one token per sequence, every token a logit row in
        // order) replays one hipGraph of the whole step, as the reference does
        // (cuda_backend.cu:145-149): the step's ~200 launches become one.
        bool decode_only = opt_.cuda_graphs && !capture_ && R == T && T == S;
        for (int i = 0; decode_only && i < R; i++) decode_only = b.logit_rows[static_cast<size_t>(i)] == i;
        if (decode_only && forward_graph(b)) {
            rows_ = R;
            return;
        }
        kv_->plan(b);  // validates the tables, uploads tokens, positions, tables and logit rows in one copy
        enqueue_step(T, R, kv_->d_logit_rows());
        rows_ = R;
    }

    void sample(std::span<const SampleRequest> reqs, std::span<int32_t> out) override {
        EMBER_CHECK(static_cast<int>(reqs.size()) == rows_ && out.size() == reqs.size(),
                    "sample: {} requests for {} rows", reqs.size(), rows_);
        if (reqs.empty()) return;
        upload_params(reqs);
        EmberSampleArgs a{};
        a.logits = logits_.get<float>();
        a.R = rows_;
        a.vocab = cfg_.vocab_size;
        a.params = dev_params_.get<EmberSampleParams>();
        a.out = dev_tokens_.get<int32_t>();
        check_abi(ember_hip_sample(&a, stream_), "sample");
        HIPB_CHECK(hipMemcpyAsync(host_ints_, dev_tokens_.get(), reqs.size() * sizeof(int32_t), hipMemcpyDeviceToHost,
                                  stream_));
        HIPB_CHECK(hipStreamSynchronize(stream_));
        std::memcpy(out.data(), host_ints_, reqs.size() * sizeof(int32_t));
    }

    void token_probs(std::span<const SampleRequest> reqs, std::span<const int32_t> rows,
                     std::span<const int32_t> tokens, std::span<float> out) override {
        EMBER_CHECK(static_cast<int>(reqs.size()) == rows_, "token_probs: params must cover every logit row");
        const size_t n = rows.size();
        EMBER_CHECK(tokens.size() == n && out.size() >= n, "token_probs: {} rows, {} tokens, {} outputs", n,
                    tokens.size(), out.size());
        if (n == 0) return;
        EMBER_CHECK(n <= static_cast<size_t>(opt_.max_logit_rows), "token_probs: too many queries");
        for (size_t i = 0; i < n; i++)
            EMBER_CHECK(rows[i] >= 0 && rows[i] < rows_ && tokens[i] >= 0 && tokens[i] < cfg_.vocab_size,
                        "token_probs: query {} (row {}, token {}) out of range", i, rows[i], tokens[i]);
        upload_params(reqs);
        std::copy(rows.begin(), rows.end(), host_ints_);
        std::copy(tokens.begin(), tokens.end(), host_ints_ + n);
        HIPB_CHECK(hipMemcpyAsync(dev_queries_.get(), host_ints_, 2 * n * sizeof(int32_t), hipMemcpyHostToDevice,
                                  stream_));
        EmberProbArgs a{};
        a.logits = logits_.get<float>();
        a.vocab = cfg_.vocab_size;
        a.params = dev_params_.get<EmberSampleParams>();
        a.rows = dev_queries_.get<int32_t>();
        a.tokens = dev_queries_.get<int32_t>() + n;
        a.n = static_cast<int32_t>(n);
        a.out = dev_probs_.get<float>();
        a.R = rows_;
        check_abi(ember_hip_token_probs(&a, stream_), "token_probs");
        HIPB_CHECK(hipMemcpyAsync(out.data(), dev_probs_.get(), n * sizeof(float), hipMemcpyDeviceToHost, stream_));
        HIPB_CHECK(hipStreamSynchronize(stream_));
    }

    void logits(int row, std::span<float> out) override {
        EMBER_CHECK(row >= 0 && row < rows_ && static_cast<int>(out.size()) >= cfg_.vocab_size, "logits: bad row {}",
                    row);
        HIPB_CHECK(hipMemcpyAsync(out.data(), logits_.get<float>() + static_cast<size_t>(row) * cfg_.vocab_size,
                                  sizeof(float) * cfg_.vocab_size, hipMemcpyDeviceToHost, stream_));
        HIPB_CHECK(hipStreamSynchronize(stream_));
    }

    void set_capture_hidden(bool on) override {
        capture_ = on;
        if (on && !captured_.bytes())
            captured_ = DeviceMem(static_cast<size_t>(cfg_.n_layers + 1) * cfg_.hidden * sizeof(float));
    }

    std::vector<float> captured_hidden() override {
        std::vector<float> out(captured_.bytes() / sizeof(float));
        if (!out.empty()) {
            HIPB_CHECK(hipMemcpyAsync(out.data(), captured_.get(), captured_.bytes(), hipMemcpyDeviceToHost, stream_));
            HIPB_CHECK(hipStreamSynchronize(stream_));
        }
        return out;
    }

private:
    // C[M, N] (+)= A[M, K] . W^T with an epilogue, 64 rows per GEMV launch.
    // Every launch of a planned step of T tokens: embedding, the layers, then
    // the final norm and LM head of R logit rows (rows: the planned step's
    // logit rows on the device, or null for rows 0..R-1).
    void enqueue_step(int T, int R, const int32_t *rows) {
        const ModelConfig &c = cfg_;
        const int H = c.hidden, Q = c.q_dim(), KV = c.kv_dim(), I = c.intermediate;
        EmberEmbedArgs e{};
        e.tokens = kv_->d_tokens();
        e.T = T;
        e.table = embed_;
        e.vocab = c.vocab_size;
        e.hidden = H;
        e.out = h_.get<float>();
        check_abi(ember_hip_embed(&e, stream_), "embed");
        capture(0, T);

        for (int l = 0; l < c.n_layers; l++) {
            const LayerWeights &L = layers_[static_cast<size_t>(l)];
            rmsnorm(nullptr, T, L.in_norm);
            gemm(xn_.get(), H, L.qkv, T, qkv_.get(), Q + 2 * KV, EMBER_EPILOGUE_STORE_F16);
            kv_->layer(l, qkv_.get(), L.q_norm, L.k_norm, L.qkv_bias, att_.get());
            gemm(att_.get(), Q, L.o, T, h_.get(), H, EMBER_EPILOGUE_ADD_F32);
            rmsnorm(nullptr, T, L.post_norm);
            gemm(xn_.get(), H, L.gate_up, T, act_.get(), I, EMBER_EPILOGUE_SILU_MUL);
            gemm(act_.get(), I, L.down, T, h_.get(), H, EMBER_EPILOGUE_ADD_F32);
            capture(l + 1, T);
        }
        if (R > 0) {
            rmsnorm(rows, R, final_norm_);
            gemm(xn_.get(), H, lm_head_, R, logits_.get(), c.vocab_size, EMBER_EPILOGUE_STORE_F32);
        }
    }

    // The step padded to the path's token bucket and planned once
    // (HipPagedKv::plan_graph: padding tokens sit at position 0 on the spare
    // block), then every launch of the padded step, logits for all its rows,
    // replayed from a graph kept per planned layout (cuda_backend.cu:402-454).
    // The per-token arithmetic is the eager step's, so the real rows' logits
    // are the same bits. False, with nothing enqueued, when the padded step
    // would not fit the activation buffers.
    bool forward_graph(const StepBatch &b) {
        const int TB = kv_->graph_bucket(b);
        if (TB == 0 || TB > opt_.max_logit_rows || TB > opt_.max_batch_tokens) return false;
        EMBER_CHECK(kv_->plan_graph(b) == TB, "internal: the graph bucket changed while planning");
        const uint64_t key = kv_->graph_key();
        auto it = graphs_.find(key);
        if (it == graphs_.end()) {
            hipGraph_t graph = nullptr;
            HIPB_CHECK(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
            try {
                enqueue_step(TB, TB, nullptr);
            } catch (...) {
                (void)hipStreamEndCapture(stream_, &graph);
                if (graph) (void)hipGraphDestroy(graph);
                throw;
            }
            HIPB_CHECK(hipStreamEndCapture(stream_, &graph));
            hipGraphExec_t exec = nullptr;
            const hipError_t inst = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
            (void)hipGraphDestroy(graph);
            HIPB_CHECK(inst);
            it = graphs_.emplace(key, exec).first;
            g_graph_captures.fetch_add(1, std::memory_order_relaxed);
        }
        HIPB_CHECK(hipGraphLaunch(it->second, stream_));
        g_graph_replays.fetch_add(1, std::memory_order_relaxed);
        return true;
    }

    void gemm(const void *A, int lda, const Linear &W, int M, void *C, int ldc, int ep) {
        const size_t out_elem = ep == EMBER_EPILOGUE_STORE_F32 || ep == EMBER_EPILOGUE_ADD_F32 ? 4 : 2;
        for (int m0 = 0; m0 < M; m0 += 64) {
            EmberGemvArgs g{};
            g.A = static_cast<const char *>(A) + static_cast<size_t>(m0) * lda * 2;
            g.lda = lda;
            g.W = W.w;
            g.M = std::min(64, M - m0);
            g.N = W.N;
            g.K = W.K;
            g.C = static_cast<char *>(C) + static_cast<size_t>(m0) * ldc * out_elem;
            g.ldc = ldc;
            g.epilogue = ep;
            g.workspace = gemv_ws_.get();
            g.workspace_bytes = static_cast<int64_t>(gemv_ws_.bytes());
            g.w_packed = W.packed ? 1 : 0;
            check_abi(ember_hip_gemv(&g, stream_), "gemv");
        }
    }

    void rmsnorm(const int32_t *rows, int R, const float *w) {
        EmberNormArgs n{};
        n.x = h_.get<float>();
        n.rows = rows;
        n.R = R;
        n.hidden = cfg_.hidden;
        n.w = w;
        n.eps = cfg_.rms_eps;
        n.out = xn_.get();
        check_abi(ember_hip_rmsnorm_rows(&n, stream_), "rmsnorm_rows");
    }

    void capture(int index, int T) {
        if (!capture_) return;
        const int H = cfg_.hidden;
        HIPB_CHECK(hipMemcpyAsync(captured_.get<float>() + static_cast<size_t>(index) * H,
                                  h_.get<float>() + static_cast<size_t>(T - 1) * H, H * sizeof(float),
                                  hipMemcpyDeviceToDevice, stream_));
    }

    void upload_params(std::span<const SampleRequest> reqs) {
        for (size_t i = 0; i < reqs.size(); i++) {
            const SamplingParams &p = reqs[i].params;
            host_params_[i] = EmberSampleParams{p.temperature, p.top_p, p.min_p, p.top_k, p.seed, reqs[i].counter};
        }
        HIPB_CHECK(hipMemcpyAsync(dev_params_.get(), host_params_, reqs.size() * sizeof(EmberSampleParams),
                                  hipMemcpyHostToDevice, stream_));
    }

    // ---- loading ----------------------------------------------------------------------------

    void load_weights(const std::string &dir) {
        const SafeTensors st = SafeTensors::open_dir(dir);
        const ModelConfig &c = cfg_;
        const int64_t H = c.hidden, Q = c.q_dim(), KV = c.kv_dim(), I = c.intermediate, D = c.head_dim,
                      V = c.vocab_size;
        const bool tied = c.tie_embeddings || !st.has("lm_head.weight");
        auto al = [](int64_t bytes) { return static_cast<size_t>((bytes + 255) & ~int64_t(255)); };
        auto prow = [](int64_t rows) { return (rows + 15) / 16 * 16; };  // a packed matrix's rows
        const size_t per_layer = al(2 * prow(Q + 2 * KV) * H) + al(2 * prow(H) * Q) + al(2 * prow(2 * I) * H) +
                                 al(2 * prow(H) * I) + 2 * al(4 * H) + 2 * al(4 * D) + al(4 * (Q + 2 * KV));
        // The LM head is kept packed for the GEMV; a tied head is a packed copy of the embedding, which the
        // embedding gather reads row-major (memory is cheap here: 311 MB for a 0.6B model's table).
        const size_t bytes = al(2 * V * H) + al(2 * prow(V) * H) + al(4 * H) + per_layer * static_cast<size_t>(c.n_layers);
        size_t free = 0, total = 0;
        HIPB_CHECK(hipMemGetInfo(&free, &total));
        EMBER_CHECK(bytes + (256u << 20) < free, "the model needs {} MiB of GPU memory, {} MiB are free",
                    bytes >> 20, free >> 20);
        weights_ = DeviceMem(bytes);
        size_t used = 0;
        auto take = [&](int64_t n_bytes) {
            void *p = weights_.get<char>() + used;
            used += al(n_bytes);
            EMBER_CHECK(used <= bytes, "internal: weight arena overflow");
            return p;
        };
        // A device matrix is assembled on the host as f16 rows and uploaded with one copy: `parts` are
        // (tensor, first destination row, destination row stride) for tensors of `cols` columns.
        // With `packed`, the matrix goes up in ember_hip_gemv_pack's layout instead (its rows rounded up to 16,
        // the extra rows zero): for 16-row tile t and 32-wide k step s, lane l = 16 g + c's 8 halves are row
        // 16 t + c, columns 32 s + 8 g ..., the 64 lanes in order.
        std::vector<uint16_t> staging, packed;
        auto upload_matrix = [&](void *dst, int64_t rows, int64_t cols,
                                 std::initializer_list<std::tuple<const TensorView *, int64_t, int64_t>> parts,
                                 bool pack = false) {
            staging.assign(static_cast<size_t>(rows * cols), 0);
            for (const auto &[t, first, stride] : parts) {
                const int64_t n = t->shape.size() == 1 ? 1 : t->shape[0];
                EMBER_CHECK(t->shape.back() == cols && first + (n - 1) * stride < rows, "tensor {} does not fit", t->name);
                for (int64_t r = 0; r < n; r++)
                    for (int64_t k = 0; k < cols; k++)
                        staging[static_cast<size_t>((first + r * stride) * cols + k)] = half_bits(element(*t, r * cols + k));
            }
            if (!pack) {
                HIPB_CHECK(hipMemcpy(dst, staging.data(), staging.size() * 2, hipMemcpyHostToDevice));
                return;
            }
            EMBER_CHECK(cols % 32 == 0, "a packed matrix needs a multiple of 32 columns (got {})", cols);
            const int64_t steps = cols / 32;
            packed.assign(static_cast<size_t>(prow(rows) * cols), 0);
            size_t q = 0;
            for (int64_t tile = 0; tile < prow(rows) / 16; tile++)
                for (int64_t s = 0; s < steps; s++)
                    for (int lane = 0; lane < 64; lane++, q += 8) {
                        const int64_t row = 16 * tile + lane % 16;
                        if (row < rows)
                            std::copy_n(&staging[static_cast<size_t>(row * cols + 32 * s + 8 * (lane / 16))], 8, &packed[q]);
                    }
            HIPB_CHECK(hipMemcpy(dst, packed.data(), packed.size() * 2, hipMemcpyHostToDevice));
        };
        auto upload_vector = [&](const TensorView &t) {
            std::vector<float> v(static_cast<size_t>(t.numel()));
            for (int64_t i = 0; i < t.numel(); i++) v[static_cast<size_t>(i)] = element(t, i);
            void *p = take(4 * t.numel());
            HIPB_CHECK(hipMemcpy(p, v.data(), v.size() * 4, hipMemcpyHostToDevice));
            return static_cast<const float *>(p);
        };
        embed_ = take(2 * V * H);
        upload_matrix(const_cast<void *>(embed_), V, H, {{&st.get("model.embed_tokens.weight", {V, H}), 0, 1}});
        lm_head_.N = static_cast<int>(V);
        lm_head_.K = static_cast<int>(H);
        {
            void *w = take(2 * prow(V) * H);
            const std::string head = tied ? "model.embed_tokens.weight" : "lm_head.weight";
            upload_matrix(w, V, H, {{&st.get(head, {V, H}), 0, 1}}, true);
            lm_head_.w = w;
            lm_head_.packed = true;
        }
        final_norm_ = upload_vector(st.get("model.norm.weight", {H}));
        layers_.resize(static_cast<size_t>(c.n_layers));
        for (int l = 0; l < c.n_layers; l++) {
            const std::string p = "model.layers." + std::to_string(l) + ".";
            LayerWeights &L = layers_[static_cast<size_t>(l)];
            void *qkv = take(2 * prow(Q + 2 * KV) * H);
            upload_matrix(qkv, Q + 2 * KV, H,
                          {{&st.get(p + "self_attn.q_proj.weight", {Q, H}), 0, 1},
                           {&st.get(p + "self_attn.k_proj.weight", {KV, H}), Q, 1},
                           {&st.get(p + "self_attn.v_proj.weight", {KV, H}), Q + KV, 1}}, true);
            L.qkv = {static_cast<int>(Q + 2 * KV), static_cast<int>(H), qkv, true};
            void *o = take(2 * prow(H) * Q);
            upload_matrix(o, H, Q, {{&st.get(p + "self_attn.o_proj.weight", {H, Q}), 0, 1}}, true);
            L.o = {static_cast<int>(H), static_cast<int>(Q), o, true};
            void *gu = take(2 * prow(2 * I) * H);
            upload_matrix(gu, 2 * I, H,
                          {{&st.get(p + "mlp.gate_proj.weight", {I, H}), 0, 2},    // even rows
                           {&st.get(p + "mlp.up_proj.weight", {I, H}), 1, 2}}, true);    // odd rows
            L.gate_up = {static_cast<int>(2 * I), static_cast<int>(H), gu, true};
            void *down = take(2 * prow(H) * I);
            upload_matrix(down, H, I, {{&st.get(p + "mlp.down_proj.weight", {H, I}), 0, 1}}, true);
            L.down = {static_cast<int>(H), static_cast<int>(I), down, true};
            L.in_norm = upload_vector(st.get(p + "input_layernorm.weight", {H}));
            L.post_norm = upload_vector(st.get(p + "post_attention_layernorm.weight", {H}));
            if (c.qk_norm) {
                L.q_norm = upload_vector(st.get(p + "self_attn.q_norm.weight", {D}));
                L.k_norm = upload_vector(st.get(p + "self_attn.k_norm.weight", {D}));
            }
            if (c.qkv_bias) {
                const TensorView *parts[3] = {&st.get(p + "self_attn.q_proj.bias", {Q}),
                                              &st.get(p + "self_attn.k_proj.bias", {KV}),
                                              &st.get(p + "self_attn.v_proj.bias", {KV})};
                std::vector<float> bias;
                for (const TensorView *t : parts)
                    for (int64_t i = 0; i < t->numel(); i++) bias.push_back(element(*t, i));
                void *b = take(4 * (Q + 2 * KV));
                HIPB_CHECK(hipMemcpy(b, bias.data(), bias.size() * 4, hipMemcpyHostToDevice));
                L.qkv_bias = static_cast<const float *>(b);
            }
        }
    }

    void allocate_activations() {
        const ModelConfig &c = cfg_;
        const size_t T = static_cast<size_t>(opt_.max_batch_tokens), R = static_cast<size_t>(opt_.max_logit_rows);
        const size_t H = c.hidden, Q = c.q_dim(), KV = c.kv_dim(), I = c.intermediate;
        h_ = DeviceMem(T * H * 4);
        xn_ = DeviceMem(std::max(T, R) * H * 2);
        qkv_ = DeviceMem(T * (Q + 2 * KV) * 2);
        att_ = DeviceMem(T * Q * 2);
        act_ = DeviceMem(T * I * 2);
        logits_ = DeviceMem(std::max<size_t>(R, 1) * c.vocab_size * 4);
        dev_params_ = DeviceMem(R * sizeof(EmberSampleParams));
        dev_tokens_ = DeviceMem(R * sizeof(int32_t));
        dev_queries_ = DeviceMem(2 * R * sizeof(int32_t));
        dev_probs_ = DeviceMem(R * sizeof(float));
        HIPB_CHECK(hipHostMalloc(reinterpret_cast<void **>(&host_params_), R * sizeof(EmberSampleParams), 0));
        HIPB_CHECK(hipHostMalloc(reinterpret_cast<void **>(&host_ints_), 2 * R * sizeof(int32_t), 0));
        // One zeroed GEMV workspace, for the largest split among the model's projections at 64 tokens;
        // the projections run one after another on stream_, so they share it.
        int64_t ws = 0;
        const int64_t shapes[][2] = {{static_cast<int64_t>(Q + 2 * KV), static_cast<int64_t>(H)},
                                     {static_cast<int64_t>(H), static_cast<int64_t>(Q)},
                                     {static_cast<int64_t>(2 * I), static_cast<int64_t>(H)},
                                     {static_cast<int64_t>(H), static_cast<int64_t>(I)},
                                     {static_cast<int64_t>(c.vocab_size), static_cast<int64_t>(H)}};
        for (const auto &sh : shapes)
            ws = std::max(ws, ember_hip_gemv_workspace_bytes(64, static_cast<int32_t>(sh[0]), static_cast<int32_t>(sh[1])));
        gemv_ws_ = DeviceMem(static_cast<size_t>(ws));
        HIPB_CHECK(hipMemset(gemv_ws_.get(), 0, gemv_ws_.bytes()));
        act_bytes_ = h_.bytes() + xn_.bytes() + qkv_.bytes() + att_.bytes() + act_.bytes() + logits_.bytes() +
                     gemv_ws_.bytes();
    }

    void create_kv() {
        const ModelConfig &c = cfg_;
        const int64_t block_bytes = 2LL * c.n_layers * c.n_kv_heads * kBlockSize * c.head_dim * 2;  // K + V, f16
        int64_t blocks;
        if (opt_.kv_cache_tokens > 0) {
            blocks = (opt_.kv_cache_tokens + kBlockSize - 1) / kBlockSize;
        } else if (opt_.kv_cache_bytes > 0) {
            blocks = opt_.kv_cache_bytes / block_bytes - 1;  // one spare block for graph padding
        } else {
            size_t free = 0, total = 0;
            HIPB_CHECK(hipMemGetInfo(&free, &total));
            const size_t keep = static_cast<size_t>((1.0 - opt_.memory_fraction) * static_cast<double>(total)) + (512u << 20);
            blocks = free > keep ? static_cast<int64_t>((free - keep) / static_cast<size_t>(block_bytes)) - 1 : 0;
        }
        EMBER_CHECK(blocks >= 4 && blocks < (1LL << 31), "KV cache of {} blocks is not usable", blocks);
        num_blocks_ = static_cast<int>(blocks);
        kv_bytes_ = (blocks + 1) * block_bytes;
        PagedKvOptions po;
        po.num_blocks = num_blocks_;
        po.max_batch_tokens = opt_.max_batch_tokens;
        po.max_seqs = opt_.max_seqs;
        po.dtype = EMBER_DTYPE_F16;
        kv_ = std::make_unique<HipPagedKv>(cfg_, po, stream_);
    }

    ModelConfig cfg_;
    BackendOptions opt_;
    hipStream_t stream_ = nullptr;
    DeviceMem weights_;
    const void *embed_ = nullptr;
    Linear lm_head_;
    const float *final_norm_ = nullptr;
    std::vector<LayerWeights> layers_;
    DeviceMem h_, xn_, qkv_, att_, act_, logits_, captured_, gemv_ws_;
    DeviceMem dev_params_, dev_tokens_, dev_queries_, dev_probs_;
    EmberSampleParams *host_params_ = nullptr;
    int32_t *host_ints_ = nullptr;
    size_t act_bytes_ = 0;
    int64_t kv_bytes_ = 0;
    int num_blocks_ = 0;
    int rows_ = 0;
    bool capture_ = false;
    std::unordered_map<uint64_t, hipGraphExec_t> graphs_;  // whole decode steps, per planned layout
    std::unique_ptr<HipPagedKv> kv_;
};

}  // namespace

int64_t hip_backend_graph_replays() { return g_graph_replays.load(std::memory_order_relaxed); }
int64_t hip_backend_graph_captures() { return g_graph_captures.load(std::memory_order_relaxed); }

std::unique_ptr<Backend> create_hip_backend(const std::string &dir, const BackendOptions &opt) {
    return std::make_unique<HipBackend>(dir, opt);
}

}  // namespace ember
