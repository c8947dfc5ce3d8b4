// qmoe_layer.hpp -- header-only C++ drop-in over the C ABI of qmoe.h.
//
// Mirrors the reference's layer module (rye-001/Qwenium src/layers/moe.h:32-75):
// the same Hparams fields, the same constructor slot order and the same
// exception behaviour (std::runtime_error from the constructor when the shared
// expert is requested without its weights, moe.cpp:47-52).  build() appended
// ggml nodes; forward() here enqueues the layer on a HIP stream instead.
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "qmoe.h"

namespace qmoe {

// layer.h:19-22; accepted by forward() for interface symmetry (no effect,
// as in the reference, moe.h:55-57).
enum class Phase { Prefill, Decode };

inline void check(int rc) {
    if (rc != QMOE_OK) throw std::runtime_error(qmoe_last_error());
}

class MoELayer {
public:
    struct Hparams {
        int n_experts;
        int top_k;
        int ffn_dim;
        bool has_shared_expert;
    };

    // All tensors are borrowed device views in GGUF block layout; the w_sh_*
    // slots may be nullptr when !hp.has_shared_expert.  prefill_copies (no
    // counterpart in the reference; opt-in, so the reference's nine arguments
    // keep one copy of the weights): also keep chunk-major copies of the expert
    // matrices for the prefill GEMMs (qmoe_layer_build_prefill_copies), read from
    // the tensors here, so their data must be in place; one more copy of the
    // expert weights in device memory (455 MB for a Qwen3.6-35B-A3B layer in
    // Q4_0, 18.2 GB for its 40 layers).  Without them the prefill GEMMs read the
    // GGUF rows (same results, slower prefill).
    MoELayer(const qmoe_tensor* w_router, const qmoe_tensor* w_exp_gate, const qmoe_tensor* w_exp_up,
             const qmoe_tensor* w_exp_down, const qmoe_tensor* w_sh_gate, const qmoe_tensor* w_sh_up,
             const qmoe_tensor* w_sh_down, const qmoe_tensor* w_sh_norm, const Hparams& hp,
             bool prefill_copies = false)
        : hp_(hp) {
        const qmoe_hparams c{hp.n_experts, hp.top_k, hp.ffn_dim, hp.has_shared_expert ? 1 : 0};
        check(qmoe_layer_create(w_router, w_exp_gate, w_exp_up, w_exp_down, w_sh_gate, w_sh_up, w_sh_down,
                                w_sh_norm, &c, &layer_));
        if (prefill_copies) {
            const int rc = qmoe_layer_build_prefill_copies(layer_);
            if (rc != QMOE_OK) {
                const std::string msg = qmoe_last_error();
                qmoe_layer_destroy(layer_);
                throw std::runtime_error(msg);
            }
        }
    }
    ~MoELayer() { qmoe_layer_destroy(layer_); }
    MoELayer(const MoELayer&) = delete;
    MoELayer& operator=(const MoELayer&) = delete;

    int n_embd() const { return qmoe_layer_n_embd(layer_); }
    // Chunk-major copies of the expert matrices for the prefill GEMMs, read from
    // the tensors now (their data in place); one more copy of the expert weights.
    void build_prefill_copies() { check(qmoe_layer_build_prefill_copies(layer_)); }
    // Device histogram u64[n_experts] that every later forward adds its
    // per-expert dispatch counts to (nullptr stops it).
    void set_expert_counts(uint64_t* device_counts) { check(qmoe_layer_set_expert_counts(layer_, device_counts)); }
    const Hparams& hparams() const { return hp_; }
    qmoe_layer* handle() const { return layer_; }

    // y[n_tokens][n_embd] = MoE(x) (+ residual).  Device pointers; work is
    // enqueued on `stream` (a hipStream_t, nullptr = default stream).
    void forward(const float* x, int n_tokens, float* y, Phase /*phase*/ = Phase::Prefill, int /*il*/ = 0,
                 void* stream = nullptr, qmoe_workspace* ws = nullptr, const float* residual = nullptr,
                 const qmoe_debug* dbg = nullptr) {
        check(qmoe_layer_forward(layer_, ws, x, n_tokens, y, residual, dbg, stream));
    }
    // The block's caller slice (qwen36.cpp:297-304): y = x + MoE(RMSNorm(x) * norm_w).
    // x_ssq / y_ssq (optional, [n_tokens][ceil(n_embd/32)] doubles): x's RMSNorm
    // partial sums in, y's out, for a chain of blocks; the bits do not change.
    void forward_norm(const float* x, const float* norm_w, float eps, int n_tokens, float* y, void* stream = nullptr,
                      qmoe_workspace* ws = nullptr, const double* x_ssq = nullptr, double* y_ssq = nullptr,
                      const qmoe_debug* dbg = nullptr) {
        if (x_ssq || y_ssq)
            check(qmoe_layer_forward_norm_chain(layer_, ws, x, x_ssq, norm_w, eps, n_tokens, y, y_ssq, dbg, stream));
        else
            check(qmoe_layer_forward_norm(layer_, ws, x, norm_w, eps, n_tokens, y, dbg, stream));
    }

private:
    Hparams hp_;
    qmoe_layer* layer_ = nullptr;
};

// Gemma 4 GeGLU MoE (replaces Gemma4ForwardPass::build_moe_geglu,
// src/models/gemma4.cpp:367-445): fused gate_up tensor, GeGLU-tanh, no shared
// expert, the router on its own input.
class GeGLUMoELayer {
public:
    using Hparams = MoELayer::Hparams;

    // prefill_copies: as MoELayer's.
    GeGLUMoELayer(const qmoe_tensor* w_router, const qmoe_tensor* w_gate_up_exps, const qmoe_tensor* w_down_exps,
                  const Hparams& hp, bool prefill_copies = false)
        : hp_(hp) {
        const qmoe_hparams c{hp.n_experts, hp.top_k, hp.ffn_dim, hp.has_shared_expert ? 1 : 0};
        check(qmoe_geglu_layer_create(w_router, w_gate_up_exps, w_down_exps, &c, &layer_));
        if (prefill_copies) {
            const int rc = qmoe_layer_build_prefill_copies(layer_);
            if (rc != QMOE_OK) {
                const std::string msg = qmoe_last_error();
                qmoe_layer_destroy(layer_);
                throw std::runtime_error(msg);
            }
        }
    }
    ~GeGLUMoELayer() { qmoe_layer_destroy(layer_); }
    GeGLUMoELayer(const GeGLUMoELayer&) = delete;
    GeGLUMoELayer& operator=(const GeGLUMoELayer&) = delete;

    int n_embd() const { return qmoe_layer_n_embd(layer_); }
    const Hparams& hparams() const { return hp_; }
    qmoe_layer* handle() const { return layer_; }

    // build_moe_geglu(expert_in, router_in): y[n_tokens][n_embd], device pointers.
    void forward(const float* expert_in, const float* router_in, int n_tokens, float* y, void* stream = nullptr,
                 qmoe_workspace* ws = nullptr, const qmoe_debug* dbg = nullptr) {
        check(qmoe_layer_forward_routed(layer_, ws, expert_in, router_in, n_tokens, y, dbg, stream));
    }
    // The MoE branch from the residual rows x (gemma4.cpp:555-565): both inputs
    // (pre_ffw_norm_2, ffn_gate_inp.scale) prepared in one pass, then the layer.
    void forward_gemma4(const float* x, const float* pre_norm_w, const float* router_scale_w, float eps, int n_tokens,
                        float* y, void* stream = nullptr, qmoe_workspace* ws = nullptr,
                        const qmoe_debug* dbg = nullptr) {
        check(qmoe_layer_forward_gemma4(layer_, ws, x, pre_norm_w, router_scale_w, eps, n_tokens, y, dbg, stream));
    }

private:
    Hparams hp_;
    qmoe_layer* layer_ = nullptr;
};

// GGUF ingestion (replaces GGUFLoader, src/loader/gguf_loader.cpp): failures
// throw std::runtime_error with the loader's message, as GGUFLoadError does.
class GGUF {
public:
    explicit GGUF(const std::string& path) { check(qmoe_gguf_open(path.c_str(), &g_)); }
    ~GGUF() { qmoe_gguf_close(g_); }
    GGUF(const GGUF&) = delete;
    GGUF& operator=(const GGUF&) = delete;

    uint32_t get_u32(const std::string& key) const {
        uint32_t v = 0;
        check(qmoe_gguf_get_u32(g_, key.c_str(), &v));
        return v;
    }
    float get_f32(const std::string& key) const {
        float v = 0.0f;
        check(qmoe_gguf_get_f32(g_, key.c_str(), &v));
        return v;
    }
    std::string get_str(const std::string& key) const {
        const char* v = nullptr;
        check(qmoe_gguf_get_str(g_, key.c_str(), &v));
        return v;
    }
    qmoe_gguf_tensor find(const std::string& name) const {
        qmoe_gguf_tensor t{};
        check(qmoe_gguf_find(g_, name.c_str(), &t));
        return t;
    }
    // Copies tensor `name` into device memory `dst` (at least find(name).nbytes)
    // and returns its ggml view there.
    qmoe_tensor upload(const std::string& name, void* dst, uint64_t dst_bytes, void* stream = nullptr) const {
        const qmoe_gguf_tensor t = find(name);
        check(qmoe_gguf_upload(g_, name.c_str(), dst, dst_bytes, stream));
        qmoe_tensor v{};
        check(qmoe_gguf_tensor_view(&t, dst, &v));
        return v;
    }
    const qmoe_gguf* handle() const { return g_; }

private:
    qmoe_gguf* g_ = nullptr;
};

// MoE expert-dispatch telemetry (replaces MoEResidencyTracker,
// src/layers/moe_residency.h:35-69, and MoEMetrics, src/telemetry/metrics.h:15-17):
// the same methods and the same std::runtime_error messages.
struct MoEMetrics {
    uint64_t cold_dispatch_count = 0;
};

class MoEResidencyTracker {
public:
    MoEResidencyTracker(int n_experts, int resident_k) : n_(n_experts) {
        check(qmoe_residency_create(n_experts, resident_k, &r_));
        freq_.resize((size_t)n_experts);
    }
    ~MoEResidencyTracker() { qmoe_residency_destroy(r_); }
    MoEResidencyTracker(const MoEResidencyTracker&) = delete;
    MoEResidencyTracker& operator=(const MoEResidencyTracker&) = delete;

    void record_dispatch(int expert_id) {
        const int32_t id = expert_id;
        check(qmoe_residency_record(r_, &id, 1));
    }
    // n dispatches in order (e.g. a forward's top-k ids, token-major).
    void record_dispatches(const int32_t* expert_ids, int64_t n) { check(qmoe_residency_record(r_, expert_ids, n)); }
    // One batch from a per-expert dispatch histogram (n_experts counts).
    void record_counts(const uint64_t* counts) { check(qmoe_residency_record_counts(r_, counts, n_)); }
    bool is_resident(int expert_id) const { return qmoe_residency_is_resident(r_, expert_id) != 0; }
    uint64_t cold_dispatch_count() const { return snapshot_metrics().cold_dispatch_count; }
    MoEMetrics snapshot_metrics() const {
        qmoe_moe_metrics m{};
        check(qmoe_residency_metrics(r_, &m));
        return MoEMetrics{m.cold_dispatch_count};
    }
    const std::vector<int>& resident_set() const {
        resident_.resize((size_t)n_);
        const int32_t k = qmoe_residency_resident_set(r_, resident_.data(), n_);
        resident_.resize((size_t)k);
        return resident_;
    }
    const std::vector<uint64_t>& frequencies() const {
        check(qmoe_residency_frequencies(r_, freq_.data(), n_));
        return freq_;
    }
    void reset() { qmoe_residency_reset(r_); }

private:
    int n_;
    qmoe_residency* r_ = nullptr;
    mutable std::vector<int> resident_;
    mutable std::vector<uint64_t> freq_;
};

// A contiguous ggml-style view (ne[0] fastest) of device data.
inline qmoe_tensor make_tensor(const void* data, int type, int n_dims, long long ne0, long long ne1 = 1,
                               long long ne2 = 1) {
    qmoe_tensor t{};
    t.data = data;
    t.type = type;
    t.n_dims = n_dims;
    t.ne[0] = ne0; t.ne[1] = ne1; t.ne[2] = ne2; t.ne[3] = 1;
    const unsigned long long bb = type == QMOE_TYPE_Q4_0 ? 18 : type == QMOE_TYPE_Q8_0 ? 34 : 4;
    t.nb[0] = bb;
    t.nb[1] = type == QMOE_TYPE_F32 ? 4ull * ne0 : bb * (unsigned long long)(ne0 / 32);
    t.nb[2] = t.nb[1] * ne1;
    t.nb[3] = t.nb[2] * ne2;
    return t;
}

}  // namespace qmoe
