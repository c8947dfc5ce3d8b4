// test_moe_layer.cpp -- the reference's MoE unit tests (tests/unit/test_moe.cpp)
// re-run through the C++ drop-in (include/qmoe_layer.hpp) on the HIP path.
//
// Same cases and constant fills as the reference (router 0.1, experts 0.05,
// shared 0.02, shared gate 0.5, input 0.5), at the smallest widths Q8_0 rows
// allow (n_embd 32, ffn 32: one block each; the layer runs them on its
// zero-padded copies), 8 experts, top-2, 2 tokens, with Q8_0 expert weights.  TopKGatingCorrectness feeds the reference's KAT
// logits {1,3,0.5,2,-1,0,4,1.5} through the real router (one-hot input, so
// logits equal the router column exactly) and checks ids [6,1] and weights
// 0.7310586 / 0.2689414.
//
// The Res* cases restate the reference's MoEResidencyTracker tests
// (tests/unit/test_moe_residency.cpp:17-182) through the C++ wrapper.
//
// Usage: test_moe_layer [--host-only]   (--host-only: checks that need no GPU)
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include <unistd.h>

#include "qmoe_layer.hpp"

static int g_failures = 0;
#define EXPECT(cond, msg)                                                       \
    do {                                                                        \
        if (!(cond)) {                                                          \
            std::printf("    FAILED: %s (%s:%d)\n", msg, __FILE__, __LINE__);   \
            ++g_failures;                                                       \
        }                                                                       \
    } while (0)
#define HIP_OK(x)                                                                            \
    do {                                                                                     \
        hipError_t e_ = (x);                                                                 \
        if (e_ != hipSuccess) {                                                              \
            std::printf("HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
            std::exit(2);                                                                    \
        }                                                                                    \
    } while (0)

constexpr int N_EMBD = 32, N_EXPERTS = 8, TOP_K = 2, FFN_DIM = 32, N_TOKENS = 2;

// Q8_0 bytes of n values all equal to v (quantize_row_q8_0_ref of a constant block).
static std::vector<uint8_t> q8_const(float v, size_t n) {
    const float amax = std::fabs(v);
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const _Float16 dh = (_Float16)d;
    const int8_t q = (int8_t)std::roundf(v * id);
    std::vector<uint8_t> out(n / 32 * 34);
    for (size_t b = 0; b < n / 32; ++b) {
        std::memcpy(&out[b * 34], &dh, 2);
        std::memset(&out[b * 34 + 2], (uint8_t)q, 32);
    }
    return out;
}

struct DevBuf {
    void* p = nullptr;
    explicit DevBuf(size_t bytes) { HIP_OK(hipMalloc(&p, bytes)); }
    template <typename T>
    DevBuf(const std::vector<T>& h) {
        HIP_OK(hipMalloc(&p, h.size() * sizeof(T)));
        HIP_OK(hipMemcpy(p, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
    }
    ~DevBuf() { (void)hipFree(p); }
};

struct Fixture {
    DevBuf router, gate, up, down, sh_gate, sh_up, sh_down, sh_norm;
    qmoe_tensor t_router, t_gate, t_up, t_down, t_sh_gate, t_sh_up, t_sh_down, t_sh_norm;
    Fixture(const std::vector<float>& router_vals, float expert_v)
        : router(router_vals),
          gate(q8_const(expert_v, (size_t)N_EXPERTS * FFN_DIM * N_EMBD)),
          up(q8_const(expert_v, (size_t)N_EXPERTS * FFN_DIM * N_EMBD)),
          down(q8_const(expert_v, (size_t)N_EXPERTS * N_EMBD * FFN_DIM)),
          sh_gate(q8_const(0.02f, (size_t)FFN_DIM * N_EMBD)),
          sh_up(q8_const(0.02f, (size_t)FFN_DIM * N_EMBD)),
          sh_down(q8_const(0.02f, (size_t)N_EMBD * FFN_DIM)),
          sh_norm(std::vector<float>(N_EMBD, 0.5f)) {
        t_router = qmoe::make_tensor(router.p, QMOE_TYPE_F32, 2, N_EMBD, N_EXPERTS);
        t_gate = qmoe::make_tensor(gate.p, QMOE_TYPE_Q8_0, 3, N_EMBD, FFN_DIM, N_EXPERTS);
        t_up = qmoe::make_tensor(up.p, QMOE_TYPE_Q8_0, 3, N_EMBD, FFN_DIM, N_EXPERTS);
        t_down = qmoe::make_tensor(down.p, QMOE_TYPE_Q8_0, 3, FFN_DIM, N_EMBD, N_EXPERTS);
        t_sh_gate = qmoe::make_tensor(sh_gate.p, QMOE_TYPE_Q8_0, 2, N_EMBD, FFN_DIM);
        t_sh_up = qmoe::make_tensor(sh_up.p, QMOE_TYPE_Q8_0, 2, N_EMBD, FFN_DIM);
        t_sh_down = qmoe::make_tensor(sh_down.p, QMOE_TYPE_Q8_0, 2, FFN_DIM, N_EMBD);
        t_sh_norm = qmoe::make_tensor(sh_norm.p, QMOE_TYPE_F32, 1, N_EMBD);
    }
};

static qmoe::MoELayer::Hparams hparams(bool shared) { return {N_EXPERTS, TOP_K, FFN_DIM, shared}; }

static std::vector<float> run_forward(bool use_shared, int n_tokens = N_TOKENS, float x_val = 0.5f) {
    Fixture f(std::vector<float>((size_t)N_EMBD * N_EXPERTS, 0.1f), 0.05f);
    qmoe::MoELayer layer(&f.t_router, &f.t_gate, &f.t_up, &f.t_down, use_shared ? &f.t_sh_gate : nullptr,
                         use_shared ? &f.t_sh_up : nullptr, use_shared ? &f.t_sh_down : nullptr,
                         use_shared ? &f.t_sh_norm : nullptr, hparams(use_shared));
    DevBuf x(std::vector<float>((size_t)n_tokens * N_EMBD, x_val));
    DevBuf y((size_t)n_tokens * N_EMBD * sizeof(float));
    layer.forward((const float*)x.p, n_tokens, (float*)y.p, qmoe::Phase::Prefill, 0);
    HIP_OK(hipDeviceSynchronize());
    std::vector<float> out((size_t)n_tokens * N_EMBD);
    HIP_OK(hipMemcpy(out.data(), y.p, out.size() * sizeof(float), hipMemcpyDeviceToHost));
    return out;
}

static void BuildSucceedsNoSharedExpert() { EXPECT(run_forward(false).size() == (size_t)N_EMBD * N_TOKENS, "size"); }
static void BuildSucceedsWithSharedExpert() { EXPECT(run_forward(true).size() == (size_t)N_EMBD * N_TOKENS, "size"); }

static void OutputIsFinite() {
    for (float v : run_forward(false)) EXPECT(std::isfinite(v), "finite");
}
static void OutputIsFiniteWithSharedExpert() {
    for (float v : run_forward(true)) EXPECT(std::isfinite(v), "finite");
}

static void TopKGatingCorrectness() {
    const float kat[N_EXPERTS] = {1.0f, 3.0f, 0.5f, 2.0f, -1.0f, 0.0f, 4.0f, 1.5f};
    std::vector<float> router((size_t)N_EMBD * N_EXPERTS, 0.0f);
    for (int e = 0; e < N_EXPERTS; ++e) router[(size_t)e * N_EMBD] = kat[e];  // row e = [kat[e], 0, ...]
    Fixture f(router, 0.05f);
    qmoe::MoELayer layer(&f.t_router, &f.t_gate, &f.t_up, &f.t_down, nullptr, nullptr, nullptr, nullptr,
                         hparams(false));
    std::vector<float> xh(N_EMBD, 0.0f);
    xh[0] = 1.0f;  // one-hot: logits == kat exactly
    DevBuf x(xh);
    DevBuf y(N_EMBD * sizeof(float));
    DevBuf logits(N_EXPERTS * sizeof(float)), idx(TOP_K * sizeof(int32_t)), w(TOP_K * sizeof(float));
    qmoe_debug dbg{};
    dbg.logits = (float*)logits.p;
    dbg.topk_idx = (int32_t*)idx.p;
    dbg.topk_w = (float*)w.p;
    layer.forward((const float*)x.p, 1, (float*)y.p, qmoe::Phase::Decode, 0, nullptr, nullptr, nullptr, &dbg);
    HIP_OK(hipDeviceSynchronize());
    int32_t ih[TOP_K];
    float wh[TOP_K], lh[N_EXPERTS];
    HIP_OK(hipMemcpy(ih, idx.p, sizeof(ih), hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(wh, w.p, sizeof(wh), hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(lh, logits.p, sizeof(lh), hipMemcpyDeviceToHost));
    for (int e = 0; e < N_EXPERTS; ++e) EXPECT(lh[e] == kat[e], "router logits equal the KAT logits");
    EXPECT(ih[0] == 6 && ih[1] == 1, "top-2 ids [6, 1]");
    const float e6 = std::exp(4.0f), e1 = std::exp(3.0f);
    EXPECT(std::fabs(wh[0] - e6 / (e6 + e1)) < 1e-5f, "weight 0");
    EXPECT(std::fabs(wh[1] - e1 / (e6 + e1)) < 1e-5f, "weight 1");
    EXPECT(std::fabs(wh[0] - 0.7310586f) < 1e-6f && std::fabs(wh[1] - 0.2689414f) < 1e-6f, "KAT weights");
}

// The prefill path (300 tokens: the f16-MFMA expert GEMMs and the batched
// router) of the drop-in constructor, which builds the chunk-major weight copies
// by default, gives the same bits as a layer constructed without them.
static void PrefillCopiesGiveTheSameOutput() {
    std::vector<float> router((size_t)N_EMBD * N_EXPERTS);
    for (size_t i = 0; i < router.size(); ++i) router[i] = 0.01f * (float)((i * 37) % 23) - 0.1f;
    Fixture f(router, 0.05f);
    const int n_tok = 300;
    std::vector<float> xh((size_t)n_tok * N_EMBD);
    for (size_t i = 0; i < xh.size(); ++i) xh[i] = 0.25f * (float)((i * 13) % 11) - 1.0f;
    DevBuf x(xh);
    DevBuf y0((size_t)n_tok * N_EMBD * sizeof(float)), y1((size_t)n_tok * N_EMBD * sizeof(float));
    {
        qmoe::MoELayer with(&f.t_router, &f.t_gate, &f.t_up, &f.t_down, &f.t_sh_gate, &f.t_sh_up, &f.t_sh_down,
                            &f.t_sh_norm, hparams(true), true);
        qmoe::MoELayer without(&f.t_router, &f.t_gate, &f.t_up, &f.t_down, &f.t_sh_gate, &f.t_sh_up, &f.t_sh_down,
                               &f.t_sh_norm, hparams(true), false);
        with.forward((const float*)x.p, n_tok, (float*)y0.p);
        without.forward((const float*)x.p, n_tok, (float*)y1.p);
        HIP_OK(hipDeviceSynchronize());
    }
    std::vector<float> a(xh.size()), b(xh.size());
    HIP_OK(hipMemcpy(a.data(), y0.p, a.size() * 4, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(b.data(), y1.p, b.size() * 4, hipMemcpyDeviceToHost));
    EXPECT(std::memcmp(a.data(), b.data(), a.size() * 4) == 0, "same bits with and without the prefill copies");
    bool finite = true;
    for (float v : a) finite = finite && std::isfinite(v);
    EXPECT(finite, "finite");
}

static void SharedExpertChangesOutput() {
    const std::vector<float> a = run_forward(false), b = run_forward(true);
    bool any = false;
    for (size_t i = 0; i < a.size(); ++i) any |= std::fabs(a[i] - b[i]) > 1e-6f;
    EXPECT(any, "shared expert had no effect on output");
}

static void OutputShapeMatchesInput() {
    Fixture f(std::vector<float>((size_t)N_EMBD * N_EXPERTS, 0.1f), 0.01f);
    qmoe::MoELayer layer(&f.t_router, &f.t_gate, &f.t_up, &f.t_down, nullptr, nullptr, nullptr, nullptr,
                         hparams(false));
    EXPECT(layer.n_embd() == N_EMBD, "n_embd");
    const int n_tok = 5;
    DevBuf x(std::vector<float>((size_t)n_tok * N_EMBD, 0.5f));
    DevBuf y((size_t)n_tok * N_EMBD * sizeof(float));
    layer.forward((const float*)x.p, n_tok, (float*)y.p);
    HIP_OK(hipDeviceSynchronize());
}

// Host-only: the constructor's fail-loud contract (moe.cpp:47-52), fake pointers,
// at widths on the kernels' grid (256, 64): such a layer reads its weights in
// place, so constructing it without the prefill copies touches no device memory
// (a padded one, or the copies, read them).
static void ConstructorThrowsWithoutSharedWeights() {
    const void* fake = (const void*)0x10000000;
    constexpr int kEmbd = 256, kFfn = 64;
    qmoe_tensor r = qmoe::make_tensor(fake, QMOE_TYPE_F32, 2, kEmbd, N_EXPERTS);
    qmoe_tensor g = qmoe::make_tensor(fake, QMOE_TYPE_Q8_0, 3, kEmbd, kFfn, N_EXPERTS);
    qmoe_tensor d = qmoe::make_tensor(fake, QMOE_TYPE_Q8_0, 3, kFfn, kEmbd, N_EXPERTS);
    const qmoe::MoELayer::Hparams hp_shared{N_EXPERTS, TOP_K, kFfn, true}, hp_plain{N_EXPERTS, TOP_K, kFfn, false};
    std::string msg;
    try {
        qmoe::MoELayer layer(&r, &g, &g, &d, nullptr, nullptr, nullptr, nullptr, hp_shared, false);
    } catch (const std::runtime_error& e) {
        msg = e.what();
    }
    EXPECT(msg == "moe_layer: has_shared_expert=true but shared expert weights are null", "reference message");
    bool threw = false;
    try {
        qmoe::MoELayer ok(&r, &g, &g, &d, nullptr, nullptr, nullptr, nullptr, hp_plain, false);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    EXPECT(!threw, "valid layer constructs");
}

// GGUF ingestion through the C++ wrapper (no GPU): a hand-built v3 file with
// the architecture string, one u32 hparam and one Q8_0 tensor [64, 2].
static void GGUFLoaderReadsBlockTensors() {
    std::vector<uint8_t> b;
    auto put = [&](const void* p, size_t n) { b.insert(b.end(), (const uint8_t*)p, (const uint8_t*)p + n); };
    auto u32 = [&](uint32_t v) { put(&v, 4); };
    auto u64 = [&](uint64_t v) { put(&v, 8); };
    auto str = [&](const std::string& s) { u64(s.size()); put(s.data(), s.size()); };
    u32(0x46554747u); u32(3); u64(1); u64(2);
    str("general.architecture"); u32(8); str("qwen35moe");
    str("qwen35moe.expert_count"); u32(4); u32(256);
    str("blk.0.ffn_down_exps.weight"); u32(2); u64(64); u64(2); u32(QMOE_TYPE_Q8_0); u64(0);
    const size_t data_start = (b.size() + 31) / 32 * 32;
    b.resize(data_start, 0);
    std::vector<uint8_t> data(2 * 2 * 34);
    for (size_t i = 0; i < data.size(); ++i) data[i] = (uint8_t)(i * 7 + 3);
    put(data.data(), data.size());
    const std::string path = "/tmp/qmoe_cpp_test_" + std::to_string((long long)getpid()) + ".gguf";
    FILE* f = std::fopen(path.c_str(), "wb");
    EXPECT(f != nullptr, "temp file");
    if (!f) return;
    std::fwrite(b.data(), 1, b.size(), f);
    std::fclose(f);
    {
        qmoe::GGUF g(path);
        EXPECT(g.get_str("general.architecture") == "qwen35moe", "architecture");
        EXPECT(g.get_u32("qwen35moe.expert_count") == 256, "expert_count");
        const qmoe_gguf_tensor t = g.find("blk.0.ffn_down_exps.weight");
        EXPECT(t.type == QMOE_TYPE_Q8_0 && t.n_dims == 2 && t.ne[0] == 64 && t.ne[1] == 2, "inventory entry");
        EXPECT(t.file_offset == data_start && t.nbytes == data.size(), "data offset and size");
        std::vector<uint8_t> got(t.nbytes);
        qmoe::check(qmoe_gguf_read(g.handle(), "blk.0.ffn_down_exps.weight", got.data(), got.size()));
        EXPECT(got == data, "tensor bytes");
        bool threw = false;
        try {
            g.find("blk.0.ffn_up_exps.weight");
        } catch (const std::runtime_error& e) {
            threw = std::string(e.what()).find("expected present, got absent") != std::string::npos;
        }
        EXPECT(threw, "missing tensor throws");
    }
    std::remove(path.c_str());
}

// ---- Gemma 4 GeGLU MoE through qmoe::GeGLUMoELayer ----
static void GeGLUConstructorRejectsSharedExpert() {
    const qmoe_tensor r = qmoe::make_tensor(nullptr, QMOE_TYPE_F32, 2, N_EMBD, N_EXPERTS);
    const qmoe_tensor gu = qmoe::make_tensor(nullptr, QMOE_TYPE_Q8_0, 3, N_EMBD, 2 * FFN_DIM, N_EXPERTS);
    const qmoe_tensor d = qmoe::make_tensor(nullptr, QMOE_TYPE_Q8_0, 3, FFN_DIM, N_EMBD, N_EXPERTS);
    bool threw = false;
    try {
        qmoe::GeGLUMoELayer layer(&r, &gu, &d, hparams(true));
    } catch (const std::runtime_error& e) {
        threw = std::string(e.what()).find("has_shared_expert") != std::string::npos;
    }
    EXPECT(threw, "shared expert rejected");
}

// Constant weights (router 0.1, gate/up 0.05, down 0.05, input 0.5 as the
// reference's MoE tests): the Gemma 4 one-call slice equals its two inputs fed
// to forward(expert_in, router_in), and the output is finite and non-zero.
static void GeGLUGemma4SliceMatchesRoutedForward() {
    std::vector<float> router((size_t)N_EMBD * N_EXPERTS, 0.1f);
    std::vector<uint8_t> gu = q8_const(0.05f, (size_t)N_EXPERTS * 2 * FFN_DIM * N_EMBD);
    std::vector<uint8_t> dn = q8_const(0.05f, (size_t)N_EXPERTS * N_EMBD * FFN_DIM);
    std::vector<float> x((size_t)N_TOKENS * N_EMBD), ones(N_EMBD, 1.0f);
    for (size_t i = 0; i < x.size(); ++i) x[i] = 0.5f + 0.001f * (float)(i % 7);
    void *d_r, *d_gu, *d_dn, *d_x, *d_w, *d_ei, *d_ri, *d_y0, *d_y1;
    HIP_OK(hipMalloc(&d_r, router.size() * 4));
    HIP_OK(hipMalloc(&d_gu, gu.size()));
    HIP_OK(hipMalloc(&d_dn, dn.size()));
    for (void** p : {&d_x, &d_ei, &d_ri, &d_y0, &d_y1}) HIP_OK(hipMalloc(p, x.size() * 4));
    HIP_OK(hipMalloc(&d_w, N_EMBD * 4));
    HIP_OK(hipMemcpy(d_r, router.data(), router.size() * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_gu, gu.data(), gu.size(), hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_dn, dn.data(), dn.size(), hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_x, x.data(), x.size() * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_w, ones.data(), N_EMBD * 4, hipMemcpyHostToDevice));
    const qmoe_tensor r = qmoe::make_tensor(d_r, QMOE_TYPE_F32, 2, N_EMBD, N_EXPERTS);
    const qmoe_tensor tgu = qmoe::make_tensor(d_gu, QMOE_TYPE_Q8_0, 3, N_EMBD, 2 * FFN_DIM, N_EXPERTS);
    const qmoe_tensor tdn = qmoe::make_tensor(d_dn, QMOE_TYPE_Q8_0, 3, FFN_DIM, N_EMBD, N_EXPERTS);
    {
        qmoe::GeGLUMoELayer layer(&r, &tgu, &tdn, hparams(false));
        layer.forward_gemma4((const float*)d_x, (const float*)d_w, (const float*)d_w, 1e-6f, N_TOKENS, (float*)d_y0);
        qmoe::check(qmoe_gemma4_moe_inputs((const float*)d_x, (const float*)d_w, (const float*)d_w, 1e-6f, N_TOKENS,
                                           N_EMBD, (float*)d_ei, (float*)d_ri, nullptr));
        layer.forward((const float*)d_ei, (const float*)d_ri, N_TOKENS, (float*)d_y1);
        HIP_OK(hipDeviceSynchronize());
        std::vector<float> y0(x.size()), y1(x.size());
        HIP_OK(hipMemcpy(y0.data(), d_y0, y0.size() * 4, hipMemcpyDeviceToHost));
        HIP_OK(hipMemcpy(y1.data(), d_y1, y1.size() * 4, hipMemcpyDeviceToHost));
        EXPECT(std::memcmp(y0.data(), y1.data(), y0.size() * 4) == 0, "one-call slice == inputs + routed forward");
        bool finite = true, nonzero = false;
        for (float v : y0) {
            finite = finite && std::isfinite(v);
            nonzero = nonzero || v != 0.0f;
        }
        EXPECT(finite && nonzero, "finite, non-zero output");
    }
    for (void* p : {d_r, d_gu, d_dn, d_x, d_w, d_ei, d_ri, d_y0, d_y1}) HIP_OK(hipFree(p));
}

// ---- MoEResidencyTracker: the reference's cases (tests/unit/test_moe_residency.cpp:17-182) ----
template <class F>
static bool throws_runtime(F f, const char* needle) {
    try {
        f();
    } catch (const std::runtime_error& e) {
        return std::string(e.what()).find(needle) != std::string::npos;
    }
    return false;
}

static void dispatch_n(qmoe::MoEResidencyTracker& t, int id, int n) {
    for (int i = 0; i < n; ++i) t.record_dispatch(id);
}

static void ResConstructionSucceeds() {
    qmoe::MoEResidencyTracker t(8, 3);
    EXPECT(t.cold_dispatch_count() == 0 && t.resident_set().empty(), "fresh tracker");
}
static void ResFrequenciesStartAtZero() {
    qmoe::MoEResidencyTracker t(4, 2);
    bool zero = t.frequencies().size() == 4;
    for (uint64_t f : t.frequencies()) zero = zero && f == 0;
    EXPECT(zero, "zero frequencies");
}
static void ResInvalidNExpertsThrows() {
    EXPECT(throws_runtime([] { qmoe::MoEResidencyTracker t(0, 1); }, "n_experts must be > 0; got 0"), "n_experts 0");
}
static void ResInvalidResidentKThrows() {
    EXPECT(throws_runtime([] { qmoe::MoEResidencyTracker t(8, 0); }, "resident_k must be > 0; got 0"), "resident_k 0");
}
static void ResResidentSetTracksTopKByFrequency() {
    qmoe::MoEResidencyTracker t(8, 2);
    dispatch_n(t, 0, 4);
    dispatch_n(t, 1, 3);
    dispatch_n(t, 2, 2);
    dispatch_n(t, 3, 1);
    EXPECT(t.resident_set().size() == 2, "two resident");
    EXPECT(t.is_resident(0) && t.is_resident(1) && !t.is_resident(2) && !t.is_resident(3), "experts 0 and 1");
    EXPECT(t.resident_set()[0] == 0 && t.resident_set()[1] == 1, "descending frequency");
}
static void ResResidentSetRespectsClamping() {
    qmoe::MoEResidencyTracker t(3, 10);
    for (int e = 0; e < 3; ++e) t.record_dispatch(e);
    EXPECT(t.resident_set().size() == 3 && t.is_resident(0) && t.is_resident(1) && t.is_resident(2), "k clamped to 3");
}
static void ResResidentSetExcludesZeroFrequencyExperts() {
    qmoe::MoEResidencyTracker t(8, 3);
    t.record_dispatch(4);
    EXPECT(t.resident_set().size() == 1 && t.is_resident(4), "only expert 4");
}
static void ResColdCounterIncrementsOnNonResidentDispatch() {
    qmoe::MoEResidencyTracker t(8, 3);
    dispatch_n(t, 0, 5);
    dispatch_n(t, 1, 4);
    dispatch_n(t, 2, 3);
    EXPECT(t.is_resident(0) && t.is_resident(1) && t.is_resident(2), "0, 1, 2 resident");
    const uint64_t before = t.cold_dispatch_count();
    t.record_dispatch(7);
    EXPECT(t.cold_dispatch_count() == before + 1, "cold +1");
}
static void ResColdCounterStaysStableOnResidentDispatch() {
    qmoe::MoEResidencyTracker t(8, 3);
    dispatch_n(t, 0, 5);
    dispatch_n(t, 1, 4);
    dispatch_n(t, 2, 3);
    const uint64_t before = t.cold_dispatch_count();
    t.record_dispatch(0);
    EXPECT(t.cold_dispatch_count() == before, "cold unchanged");
}
static void ResColdCounterEarlyDispatchesAreAllCold() {
    qmoe::MoEResidencyTracker t(4, 2);
    t.record_dispatch(0);
    EXPECT(t.cold_dispatch_count() == 1, "first dispatch cold");
}
static void ResSnapshotMetricsMatchesColdCount() {
    qmoe::MoEResidencyTracker t(8, 3);
    dispatch_n(t, 0, 5);
    t.record_dispatch(5);
    EXPECT(t.snapshot_metrics().cold_dispatch_count == t.cold_dispatch_count(), "snapshot");
}
static void ResResetClearsAllState() {
    qmoe::MoEResidencyTracker t(8, 3);
    dispatch_n(t, 0, 4);
    t.record_dispatch(5);
    t.reset();
    bool zero = t.cold_dispatch_count() == 0 && t.resident_set().empty();
    for (uint64_t f : t.frequencies()) zero = zero && f == 0;
    EXPECT(zero, "reset");
}
static void ResResetAllowsReuseFromCleanState() {
    qmoe::MoEResidencyTracker t(4, 1);
    t.record_dispatch(0);
    t.reset();
    t.record_dispatch(2);
    EXPECT(t.cold_dispatch_count() == 1 && t.is_resident(2), "clean reuse");
}
static void ResOutOfRangeExpertIdThrowsLow() {
    qmoe::MoEResidencyTracker t(8, 3);
    EXPECT(throws_runtime([&] { t.record_dispatch(-1); }, "expert_id=-1 out of range [0, 8)"), "id -1");
}
static void ResOutOfRangeExpertIdThrowsHigh() {
    qmoe::MoEResidencyTracker t(8, 3);
    EXPECT(throws_runtime([&] { t.record_dispatch(8); }, "expert_id=8 out of range [0, 8)"), "id 8");
}
static void ResFrequenciesAccumulateCorrectly() {
    qmoe::MoEResidencyTracker t(4, 2);
    t.record_dispatch(0);
    t.record_dispatch(0);
    t.record_dispatch(1);
    const std::vector<uint64_t> want{2, 1, 0, 0};
    EXPECT(t.frequencies() == want, "frequencies");
}

int main(int argc, char** argv) {
    const bool host_only = argc > 1 && std::string(argv[1]) == "--host-only";
    struct Case { const char* name; void (*fn)(); bool gpu; } cases[] = {
        {"ConstructorThrowsWithoutSharedWeights", ConstructorThrowsWithoutSharedWeights, false},
        {"GGUFLoaderReadsBlockTensors", GGUFLoaderReadsBlockTensors, false},
        {"GeGLUConstructorRejectsSharedExpert", GeGLUConstructorRejectsSharedExpert, false},
        {"GeGLUGemma4SliceMatchesRoutedForward", GeGLUGemma4SliceMatchesRoutedForward, true},
        {"ResConstructionSucceeds", ResConstructionSucceeds, false},
        {"ResFrequenciesStartAtZero", ResFrequenciesStartAtZero, false},
        {"ResInvalidNExpertsThrows", ResInvalidNExpertsThrows, false},
        {"ResInvalidResidentKThrows", ResInvalidResidentKThrows, false},
        {"ResResidentSetTracksTopKByFrequency", ResResidentSetTracksTopKByFrequency, false},
        {"ResResidentSetRespectsClamping", ResResidentSetRespectsClamping, false},
        {"ResResidentSetExcludesZeroFrequencyExperts", ResResidentSetExcludesZeroFrequencyExperts, false},
        {"ResColdCounterIncrementsOnNonResidentDispatch", ResColdCounterIncrementsOnNonResidentDispatch, false},
        {"ResColdCounterStaysStableOnResidentDispatch", ResColdCounterStaysStableOnResidentDispatch, false},
        {"ResColdCounterEarlyDispatchesAreAllCold", ResColdCounterEarlyDispatchesAreAllCold, false},
        {"ResSnapshotMetricsMatchesColdCount", ResSnapshotMetricsMatchesColdCount, false},
        {"ResResetClearsAllState", ResResetClearsAllState, false},
        {"ResResetAllowsReuseFromCleanState", ResResetAllowsReuseFromCleanState, false},
        {"ResOutOfRangeExpertIdThrowsLow", ResOutOfRangeExpertIdThrowsLow, false},
        {"ResOutOfRangeExpertIdThrowsHigh", ResOutOfRangeExpertIdThrowsHigh, false},
        {"ResFrequenciesAccumulateCorrectly", ResFrequenciesAccumulateCorrectly, false},
        {"BuildSucceedsNoSharedExpert", BuildSucceedsNoSharedExpert, true},
        {"BuildSucceedsWithSharedExpert", BuildSucceedsWithSharedExpert, true},
        {"OutputIsFinite", OutputIsFinite, true},
        {"OutputIsFiniteWithSharedExpert", OutputIsFiniteWithSharedExpert, true},
        {"TopKGatingCorrectness", TopKGatingCorrectness, true},
        {"SharedExpertChangesOutput", SharedExpertChangesOutput, true},
        {"OutputShapeMatchesInput", OutputShapeMatchesInput, true},
        {"PrefillCopiesGiveTheSameOutput", PrefillCopiesGiveTheSameOutput, true},
    };
    int run = 0;
    for (const auto& c : cases) {
        if (host_only && c.gpu) continue;
        const int before = g_failures;
        std::printf("[ RUN      ] MoELayerTest.%s\n", c.name);
        std::fflush(stdout);
        c.fn();
        std::printf("[ %s ] MoELayerTest.%s\n", g_failures == before ? "      OK" : " FAILED ", c.name);
        ++run;
    }
    std::printf("%d tests, %d failures\n", run, g_failures);
    return g_failures ? 1 : 0;
}
