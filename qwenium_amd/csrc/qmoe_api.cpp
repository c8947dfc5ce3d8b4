// qmoe_api.cpp -- the C ABI of include/qmoe.h: argument validation, workspace
// management and the per-layer launch sequence.
//
// Validation mirrors the reference's fail-loud contract (src/qinf_error.h:1-29:
// "<slot> expected <value>, got <value>") and the one check MoELayer's
// constructor performs (src/layers/moe.cpp:47-52).  Everything is checked on
// the host before any launch; kernels never see a shape they do not support.
#include "qmoe.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <string>

#include "qmoe_internal.h"

using qmoe::LayerDesc;
using qmoe::Workspace;

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

std::string slot_error(const char* slot, const std::string& expected, const std::string& got) {
    return std::string("qmoe: slot \"") + slot + "\" expected " + expected + ", got " + got;
}

const char* type_name(int t) {
    switch (t) {
        case QMOE_TYPE_F32: return "F32";
        case QMOE_TYPE_Q4_0: return "Q4_0";
        case QMOE_TYPE_Q8_0: return "Q8_0";
        default: return "unsupported";
    }
}

std::string type_str(int t) { return std::string(type_name(t)) + " (ggml type " + std::to_string(t) + ")"; }

std::string shape_str(const qmoe_tensor* t) {
    std::string s = "[";
    for (int i = 0; i < t->n_dims; ++i) {
        if (i) s += ",";
        s += std::to_string(t->ne[i]);
    }
    return s + "]";
}

uint64_t block_bytes(int type) {
    switch (type) {
        case QMOE_TYPE_Q4_0: return 18;
        case QMOE_TYPE_Q8_0: return 34;
        case QMOE_TYPE_F32: return 4;
        default: return 0;
    }
}

// Checks type, rank, ne (ne_expect[i] < 0 means "any"), contiguous rows and
// (aligned) 4-byte aligned data/strides: the kernels read the rows in place;
// tensors that are copied first (padded widths) may have any byte strides.
// Returns 0 or an error code (message set).
int check_tensor(const char* slot, const qmoe_tensor* t, int n_dims, const int64_t* ne_expect,
                 bool quantized, bool aligned = true) {
    if (!t) return fail(QMOE_ERR_NULL, slot_error(slot, "a tensor", "null"));
    if (!t->data) return fail(QMOE_ERR_NULL, slot_error(slot, "device data", "null data pointer"));
    if (quantized) {
        if (t->type != QMOE_TYPE_Q4_0 && t->type != QMOE_TYPE_Q8_0)
            return fail(QMOE_ERR_TYPE, slot_error(slot, "type Q4_0 or Q8_0", type_str(t->type)));
    } else if (t->type != QMOE_TYPE_F32) {
        return fail(QMOE_ERR_TYPE, slot_error(slot, "type F32", type_str(t->type)));
    }
    if (t->n_dims != n_dims) {
        return fail(QMOE_ERR_SHAPE, slot_error(slot, std::to_string(n_dims) + " dims",
                                               std::to_string(t->n_dims) + " dims " + shape_str(t)));
    }
    for (int i = 0; i < n_dims; ++i) {
        if (ne_expect[i] >= 0 && t->ne[i] != ne_expect[i]) {
            std::string exp = "ne[" + std::to_string(i) + "]=" + std::to_string(ne_expect[i]);
            return fail(QMOE_ERR_SHAPE, slot_error(slot, exp, "shape " + shape_str(t)));
        }
    }
    const uint64_t bb = block_bytes(t->type);
    const uint64_t row = quantized ? (uint64_t)(t->ne[0] / 32) * bb : (uint64_t)t->ne[0] * 4;
    if (t->nb[0] != bb)
        return fail(QMOE_ERR_SHAPE, slot_error(slot, "nb[0]=" + std::to_string(bb), "nb[0]=" + std::to_string(t->nb[0])));
    if (n_dims >= 2 && t->nb[1] < row)
        return fail(QMOE_ERR_SHAPE, slot_error(slot, "nb[1]>=" + std::to_string(row), "nb[1]=" + std::to_string(t->nb[1])));
    if (n_dims >= 3 && t->nb[2] < t->nb[1] * (uint64_t)t->ne[1])
        return fail(QMOE_ERR_SHAPE, slot_error(slot, "nb[2]>=" + std::to_string(t->nb[1] * (uint64_t)t->ne[1]),
                                               "nb[2]=" + std::to_string(t->nb[2])));
    if (!aligned) return QMOE_OK;
    if (((uintptr_t)t->data & 3u) != 0)
        return fail(QMOE_ERR_SHAPE, slot_error(slot, "4-byte aligned data", "misaligned pointer"));
    for (int i = 1; i < n_dims; ++i)
        if (t->nb[i] & 3u)
            return fail(QMOE_ERR_SHAPE, slot_error(slot, "nb[" + std::to_string(i) + "] multiple of 4",
                                                   "nb[" + std::to_string(i) + "]=" + std::to_string(t->nb[i])));
    return QMOE_OK;
}

int hip_fail(hipError_t err, const char* what) {
    return fail(QMOE_ERR_HIP, std::string("qmoe: ") + what + " failed: " + hipGetErrorString(err));
}

}  // namespace

namespace qmoe {

// Error reporting for the other host sources of the library (same thread-local text).
void clear_error() { g_last_error.clear(); }
int set_error(int code, const std::string& msg) { return fail(code, msg); }
int hip_error(hipError_t err, const char* what) { return hip_fail(err, what); }

static size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Carves the workspace buffers out of `base` (when non-null) and returns the byte size.
size_t workspace_bytes(int T, int H, int E, int K, int F, Workspace* w, void* base, bool pad) {
    const size_t A = (size_t)T * K;
    const size_t R = A + (size_t)T;  // room for a shared expert
    const int nblk = (T + kTopkMinTokensPerBlock - 1) / kTopkMinTokensPerBlock;  // top-k blocks, at most
    const int max_tiles = (int)((A + kMfmaTileM - 1) / kMfmaTileM) + std::min<int>(E, (int)A) +
                          (T + kMfmaTileM - 1) / kMfmaTileM + 1;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off = align_up(off + bytes, 256);
        return base ? (void*)((char*)base + o) : nullptr;
    };
    Workspace tmp;
    Workspace& ws = w ? *w : tmp;
    ws.xq_qs = (int8_t*)take((size_t)T * H);
    ws.xq_ds = (float2*)take((size_t)T * (H / 32) * sizeof(float2));
    ws.logits = (float*)take((size_t)T * (E + 1) * sizeof(float));
    ws.logit_bound = (float*)take((size_t)T * E * sizeof(float));
    ws.topk_idx = (int32_t*)take(A * sizeof(int32_t));
    ws.topk_w = (float*)take(A * sizeof(float));
    ws.sh_gate = (float*)take((size_t)T * sizeof(float));
    ws.local_rank = (int32_t*)take(A * sizeof(int32_t));
    ws.hist = (int32_t*)take((size_t)(nblk + kTotalCopies) * E * sizeof(int32_t));  // + the per-expert totals
    ws.jslot = (uint64_t*)take((size_t)nblk * E * sizeof(uint64_t));
    ws.offsets = (int32_t*)take((size_t)(E + 2) * sizeof(int32_t));
    ws.rows = (int32_t*)take(R * sizeof(int32_t));
    ws.row_token = (int32_t*)take(R * sizeof(int32_t));
    ws.pos = (int32_t*)take(A * sizeof(int32_t));
    ws.active = (int32_t*)take((size_t)(E + 1) * sizeof(int32_t));
    ws.expert_slot = (int32_t*)take((size_t)E * sizeof(int32_t));
    ws.slot_info = (int4*)take((size_t)(E + 1) * sizeof(int4));
    ws.dslots = (int4*)take((size_t)(E + 2) * sizeof(int4));
    ws.counters = (int32_t*)take(qmoe::kCounters * sizeof(int32_t));
    ws.sync = (int32_t*)take(kSyncWords * sizeof(int32_t));
    ws.tiles = (int4*)take((size_t)max_tiles * sizeof(int4));
    ws.gubuf = (float2*)take(R * F * sizeof(float2));
    ws.h_q = (_Float16*)ws.gubuf;  // R*F*2 bytes of the R*F*8 (the rest is its padding)
    // built with 128-wide k chunks, the prefill GEMMs stage whole chunks: a
    // 64-wide last chunk reads up to 128 bytes of quants and 4 bytes of scales
    // past a row, so the four A buffers end in 256 bytes of padding
    ws.h_d = (uint16_t*)take(R * (F / 32) * sizeof(uint16_t) + 256);
    ws.x_q = (_Float16*)take((size_t)T * H * sizeof(_Float16) + 256);
    ws.x_d = (uint16_t*)take((size_t)T * (H / 32) * sizeof(uint16_t) + 256);
    ws.rx_split = (uint16_t*)take((size_t)2 * T * H * sizeof(uint16_t));
    ws.rw_split = (uint16_t*)take((size_t)2 * E * H * sizeof(uint16_t));
    ws.rnorm = (float*)take((size_t)(T + E) * sizeof(float));
    ws.fix_max = (int)std::min<size_t>(R * (F / 32), (size_t)1 << 30);  // every h block, at worst
    ws.fix = (int4*)take((size_t)ws.fix_max * sizeof(int4));
    ws.fix_h = (float*)take((size_t)ws.fix_max * kFixStride * sizeof(float));
    ws.hq_qs = (int8_t*)take(R * F);
    ws.hq_ds = (float2*)take(R * (F / 32) * sizeof(float2));
    ws.ybuf = (float*)take(R * H * sizeof(float));
    ws.ysh = (float*)take((size_t)T * H * sizeof(float));
    ws.xn = (float*)take((size_t)T * H * sizeof(float));
    ws.xr = (float*)take((size_t)T * H * sizeof(float));
    ws.x_scale = (float*)take((size_t)T * sizeof(float));
    ws.yp = pad ? (float*)take((size_t)T * H * sizeof(float)) : nullptr;
    ws.max_tiles = max_tiles;
    ws.cap_T = T; ws.H = H; ws.E = E; ws.K = K; ws.F = F;
    ws.base = base;
    ws.bytes = off;
    return off;
}

}  // namespace qmoe

struct qmoe_layer {
    LayerDesc d;
    int Hu = 0, Fu = 0;         // the caller's widths; d.H, d.F are larger when the weights were padded
    void* pad_base = nullptr;   // the padded weight copies (owned), or null
    int device = 0;
    qmoe_workspace* own_ws = nullptr;
    hipEvent_t phase_events[QMOE_N_PHASE_EVENTS] = {};
    bool record_phases = false;
};

struct qmoe_workspace {
    Workspace w;
    int device = 0;
};

namespace {

// Zero-padded copies of the layer's weights at widths Hp >= H, Fp >= F (one
// allocation, owned by the layer); the descriptor then points at them.
hipError_t build_padded(qmoe_layer& L, int Hp, int Fp) {
    LayerDesc& d = L.d;
    const int H = d.H, F = d.F, E = d.E;
    const uint64_t bg = block_bytes(d.gu_type), bd = block_bytes(d.dn_type);
    const uint64_t row_g = (uint64_t)(Hp / 32) * bg, row_d = (uint64_t)(Fp / 32) * bd;  // padded row bytes
    const uint64_t n_router = qmoe::align_up((uint64_t)E * Hp * 4, 256), n_gu = qmoe::align_up((uint64_t)E * Fp * row_g, 256);
    const uint64_t n_dn = qmoe::align_up((uint64_t)E * Hp * row_d, 256);
    const uint64_t n_sgu = d.S ? qmoe::align_up((uint64_t)Fp * row_g, 256) : 0, n_sdn = d.S ? qmoe::align_up((uint64_t)Hp * row_d, 256) : 0;
    const uint64_t n_snorm = d.S ? qmoe::align_up((uint64_t)Hp * 4, 256) : 0;
    const uint64_t total = n_router + 2 * n_gu + n_dn + 2 * n_sgu + n_sdn + n_snorm;
    void* base = nullptr;
    hipError_t err = hipMalloc(&base, total);
    if (err != hipSuccess) return err;
    uint8_t* p = (uint8_t*)base;
    float* router = (float*)p; p += n_router;
    uint8_t* gate = p; p += n_gu;
    uint8_t* up = p; p += n_gu;
    uint8_t* down = p; p += n_dn;
    uint8_t* sgate = p; p += n_sgu;
    uint8_t* sup = p; p += n_sgu;
    uint8_t* sdown = p; p += n_sdn;
    float* snorm = (float*)p;
    err = hipMemset(base, 0, total);
    const hipMemcpyKind k = hipMemcpyDeviceToDevice;
    if (err == hipSuccess)
        err = hipMemcpy2D(router, (size_t)Hp * 4, d.w_router, (size_t)d.router_ld * 4, (size_t)H * 4, E, k);
    const uint64_t wg = (uint64_t)(H / 32) * bg, wd = (uint64_t)(F / 32) * bd;  // real row bytes
    for (int e = 0; e < E && err == hipSuccess; ++e) {
        err = hipMemcpy2D(gate + e * Fp * row_g, row_g, d.w_gate + e * d.gate_nb2, d.gate_nb1, wg, F, k);
        if (err == hipSuccess) err = hipMemcpy2D(up + e * Fp * row_g, row_g, d.w_up + e * d.up_nb2, d.up_nb1, wg, F, k);
        if (err == hipSuccess)
            err = hipMemcpy2D(down + e * Hp * row_d, row_d, d.w_down + e * d.down_nb2, d.down_nb1, wd, H, k);
    }
    if (d.S && err == hipSuccess) {
        err = hipMemcpy2D(sgate, row_g, d.w_sh_gate, d.sh_gate_nb1, wg, F, k);
        if (err == hipSuccess) err = hipMemcpy2D(sup, row_g, d.w_sh_up, d.sh_up_nb1, wg, F, k);
        if (err == hipSuccess) err = hipMemcpy2D(sdown, row_d, d.w_sh_down, d.sh_down_nb1, wd, H, k);
        if (err == hipSuccess) err = hipMemcpy(snorm, d.w_sh_norm, (size_t)H * 4, k);
    }
    if (err == hipSuccess) err = hipDeviceSynchronize();
    if (err != hipSuccess) {
        (void)hipFree(base);
        return err;
    }
    d.H = Hp;
    d.F = Fp;
    d.w_router = router;
    d.router_ld = Hp;
    d.w_gate = gate; d.gate_nb1 = row_g; d.gate_nb2 = Fp * row_g;
    d.w_up = up; d.up_nb1 = row_g; d.up_nb2 = Fp * row_g;
    d.w_down = down; d.down_nb1 = row_d; d.down_nb2 = Hp * row_d;
    if (d.S) {
        d.w_sh_gate = sgate; d.sh_gate_nb1 = row_g;
        d.w_sh_up = sup; d.sh_up_nb1 = row_g;
        d.w_sh_down = sdown; d.sh_down_nb1 = row_d;
        d.w_sh_norm = snorm;
    }
    L.pad_base = base;
    return hipSuccess;
}

}  // namespace

extern "C" {

const char* qmoe_last_error(void) { return g_last_error.c_str(); }

int qmoe_layer_create(const qmoe_tensor* w_router, const qmoe_tensor* w_exp_gate, const qmoe_tensor* w_exp_up,
                      const qmoe_tensor* w_exp_down, const qmoe_tensor* w_sh_gate, const qmoe_tensor* w_sh_up,
                      const qmoe_tensor* w_sh_down, const qmoe_tensor* w_sh_norm, const qmoe_hparams* hp,
                      qmoe_layer** out) {
    g_last_error.clear();
    if (!out) return fail(QMOE_ERR_NULL, "qmoe: out expected a non-null qmoe_layer**, got null");
    *out = nullptr;
    if (!hp) return fail(QMOE_ERR_NULL, "qmoe: hp expected non-null hparams, got null");
    // moe.cpp:47-52: the shared expert matrices are required when has_shared_expert
    if (hp->has_shared_expert && (!w_sh_gate || !w_sh_up || !w_sh_down))
        return fail(QMOE_ERR_NULL, "moe_layer: has_shared_expert=true but shared expert weights are null");
    if (hp->n_experts < 1 || hp->n_experts > 1024)
        return fail(QMOE_ERR_VALUE, "qmoe: hparam \"n_experts\" expected 1..1024, got " + std::to_string(hp->n_experts));
    if (hp->top_k < 1 || hp->top_k > hp->n_experts || hp->top_k > 64)
        return fail(QMOE_ERR_VALUE, "qmoe: hparam \"top_k\" expected 1..min(n_experts, 64) (n_experts=" +
                                        std::to_string(hp->n_experts) + "), got " + std::to_string(hp->top_k));
    if (hp->ffn_dim < 32 || hp->ffn_dim > 4096 || hp->ffn_dim % 32 != 0)
        return fail(QMOE_ERR_VALUE, "qmoe: hparam \"ffn_dim\" expected a multiple of 32 in [32, 4096], got " +
                                        std::to_string(hp->ffn_dim));
    if (!w_router) return fail(QMOE_ERR_NULL, slot_error("w_router", "a tensor", "null"));
    const int64_t H = w_router->ne[0];
    if (H < 32 || H > 4096 || H % 32 != 0)
        return fail(QMOE_ERR_SHAPE, slot_error("w_router", "ne[0]=n_embd a multiple of 32 in [32, 4096]",
                                               "ne[0]=" + std::to_string(H)));
    const int64_t E = hp->n_experts, F = hp->ffn_dim;
    const bool al = H % 256 == 0 && F % 64 == 0;  // else padded copies are read, not these rows
    int rc;
    {
        const int64_t ne[2] = {H, E};
        if ((rc = check_tensor("w_router", w_router, 2, ne, false))) return rc;
    }
    {
        const int64_t ne[3] = {H, F, E};
        if ((rc = check_tensor("w_exp_gate", w_exp_gate, 3, ne, true, al))) return rc;
        if ((rc = check_tensor("w_exp_up", w_exp_up, 3, ne, true, al))) return rc;
        if (w_exp_up->type != w_exp_gate->type)
            return fail(QMOE_ERR_TYPE, slot_error("w_exp_up", "type " + type_str(w_exp_gate->type) + " (as w_exp_gate)",
                                                  type_str(w_exp_up->type)));
    }
    {
        const int64_t ne[3] = {F, H, E};
        if ((rc = check_tensor("w_exp_down", w_exp_down, 3, ne, true, al))) return rc;
    }
    if (hp->has_shared_expert) {
        const int64_t ne_gu[2] = {H, F};
        const int64_t ne_d[2] = {F, H};
        const int64_t ne_n[1] = {H};
        if ((rc = check_tensor("w_sh_gate", w_sh_gate, 2, ne_gu, true, al))) return rc;
        if ((rc = check_tensor("w_sh_up", w_sh_up, 2, ne_gu, true, al))) return rc;
        if ((rc = check_tensor("w_sh_down", w_sh_down, 2, ne_d, true, al))) return rc;
        if ((rc = check_tensor("w_sh_norm", w_sh_norm, 1, ne_n, false))) return rc;
        if (w_sh_gate->type != w_exp_gate->type)
            return fail(QMOE_ERR_TYPE, slot_error("w_sh_gate", "type " + type_str(w_exp_gate->type) + " (as w_exp_gate)",
                                                  type_str(w_sh_gate->type)));
        if (w_sh_up->type != w_exp_gate->type)
            return fail(QMOE_ERR_TYPE, slot_error("w_sh_up", "type " + type_str(w_exp_gate->type) + " (as w_exp_gate)",
                                                  type_str(w_sh_up->type)));
        if (w_sh_down->type != w_exp_down->type)
            return fail(QMOE_ERR_TYPE, slot_error("w_sh_down", "type " + type_str(w_exp_down->type) + " (as w_exp_down)",
                                                  type_str(w_sh_down->type)));
    }
    qmoe_layer* L = new (std::nothrow) qmoe_layer();
    if (!L) return fail(QMOE_ERR_VALUE, "qmoe: host allocation failed");
    LayerDesc& d = L->d;
    d.H = (int)H; d.E = (int)E; d.K = hp->top_k; d.F = (int)F; d.S = hp->has_shared_expert ? 1 : 0;
    d.gu_type = w_exp_gate->type;
    d.dn_type = w_exp_down->type;
    d.w_router = (const float*)w_router->data;
    d.router_ld = w_router->nb[1] / 4;
    d.w_gate = (const uint8_t*)w_exp_gate->data; d.gate_nb1 = w_exp_gate->nb[1]; d.gate_nb2 = w_exp_gate->nb[2];
    d.w_up = (const uint8_t*)w_exp_up->data; d.up_nb1 = w_exp_up->nb[1]; d.up_nb2 = w_exp_up->nb[2];
    d.w_down = (const uint8_t*)w_exp_down->data; d.down_nb1 = w_exp_down->nb[1]; d.down_nb2 = w_exp_down->nb[2];
    if (d.S) {
        d.w_sh_gate = (const uint8_t*)w_sh_gate->data; d.sh_gate_nb1 = w_sh_gate->nb[1];
        d.w_sh_up = (const uint8_t*)w_sh_up->data; d.sh_up_nb1 = w_sh_up->nb[1];
        d.w_sh_down = (const uint8_t*)w_sh_down->data; d.sh_down_nb1 = w_sh_down->nb[1];
        d.w_sh_norm = (const float*)w_sh_norm->data;
    }
    (void)hipGetDevice(&L->device);
    int n_cu = 0;
    if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, L->device) == hipSuccess && n_cu > 0)
        d.n_cu = n_cu;
    // token count from which the grouped f16-MFMA GEMMs replace the streaming GEMVs:
    // where an expert averages about 5.5 rows (T * top_k / n_experts), and from 128
    // tokens at least (measured: the 35B-A3B shape crosses over near 176 tokens,
    // Gemma 4's below 128)
    {
        const int64_t t = (11 * (int64_t)d.E + 2 * d.K - 1) / (2 * d.K);  // ceil(5.5 E / K)
        d.mfma_min_tokens = (int)std::max<int64_t>(128, std::min<int64_t>(4096, (t + 15) / 16 * 16));
    }
    // token count from which routing runs the batched bf16-MFMA router: its cost is
    // nearly flat in T (its tiles split over more workgroups at small T), the exact
    // grouped router's grows with T * n_experts * n_embd; measured crossovers (whole
    // layer, same box): about 140 tokens at the 35B-A3B shape, about 270 at Gemma 4's;
    // this rule puts them at 224 and 272
    {
        const double t = 216.0 * std::sqrt(524288.0 / ((double)d.E * (double)d.H));
        d.big_router_min_tokens = (int)std::max(128.0, std::min(1024.0, std::ceil(t / 16.0) * 16.0));
    }
    if (const char* env = std::getenv("QMOE_MFMA_MIN_TOKENS")) {
        const long v = std::strtol(env, nullptr, 10);
        if (v >= 1) d.mfma_min_tokens = (int)std::min<long>(v, 1 << 30);
    }
    // decode down+combine prefetch depth (tuning)
    if (const char* env = std::getenv("QMOE_DC_AHEAD")) {
        const long v = std::strtol(env, nullptr, 10);
        if (v >= 1) d.dc_ahead = (int)std::min<long>(v, 4);
    }
    // token count from which routing runs the batched bf16-MFMA router
    if (const char* env = std::getenv("QMOE_BIG_ROUTER_MIN_TOKENS")) {
        const long v = std::strtol(env, nullptr, 10);
        if (v >= 1) d.big_router_min_tokens = (int)std::min<long>(v, 1 << 30);
    }
    L->Hu = d.H;
    L->Fu = d.F;
    if (d.H % 256 != 0 || d.F % 64 != 0) {
        // widths off the kernels' grid: zero-padded copies (n_embd to a multiple of
        // 256, ffn_dim of 64); the padded columns and rows meet zero weights and
        // zero activations, so every real dot, sum and Q8_0 block keeps its value
        const hipError_t err = build_padded(*L, (d.H + 255) / 256 * 256, (d.F + 63) / 64 * 64);
        if (err != hipSuccess) {
            delete L;
            return hip_fail(err, "padded weight copies");
        }
    }
    *out = L;
    return QMOE_OK;
}

int qmoe_layer_build_prefill_copies(qmoe_layer* layer) {
    g_last_error.clear();
    if (!layer) return fail(QMOE_ERR_NULL, "qmoe: layer expected non-null, got null");
    if (layer->d.pk_base) return QMOE_OK;
    const hipError_t err = qmoe::build_prefill_copies(layer->d);
    return err == hipSuccess ? QMOE_OK : hip_fail(err, "prefill weight copies");
}

int qmoe_geglu_layer_create(const qmoe_tensor* w_router, const qmoe_tensor* w_gate_up_exps,
                            const qmoe_tensor* w_down_exps, const qmoe_hparams* hp, qmoe_layer** out) {
    g_last_error.clear();
    if (!out) return fail(QMOE_ERR_NULL, "qmoe: out expected a non-null qmoe_layer**, got null");
    *out = nullptr;
    if (!hp) return fail(QMOE_ERR_NULL, "qmoe: hp expected non-null hparams, got null");
    if (hp->has_shared_expert)
        return fail(QMOE_ERR_VALUE, "qmoe: hparam \"has_shared_expert\" expected 0 for the GeGLU MoE (Gemma 4 has none), got " +
                                        std::to_string(hp->has_shared_expert));
    if (!w_router) return fail(QMOE_ERR_NULL, slot_error("w_router", "a tensor", "null"));
    if (hp->ffn_dim < 32 || hp->ffn_dim > 4096 || hp->ffn_dim % 32 != 0)
        return fail(QMOE_ERR_VALUE, "qmoe: hparam \"ffn_dim\" expected a multiple of 32 in [32, 4096], got " +
                                        std::to_string(hp->ffn_dim));
    const int64_t H = w_router->ne[0], E = hp->n_experts, F = hp->ffn_dim;
    {
        // [n_embd, 2*ffn_dim, n_experts]: gate rows 0..F-1, up rows F..2F-1 of each expert (gemma4.cpp:397-409)
        const int64_t ne[3] = {H, 2 * F, E};
        int rc = check_tensor("w_gate_up_exps", w_gate_up_exps, 3, ne, true, H % 256 == 0 && F % 64 == 0);
        if (rc) return rc;
    }
    qmoe_tensor gate = *w_gate_up_exps, up = *w_gate_up_exps;
    gate.ne[1] = up.ne[1] = F;
    up.data = (const uint8_t*)w_gate_up_exps->data + (uint64_t)F * w_gate_up_exps->nb[1];
    int rc = qmoe_layer_create(w_router, &gate, &up, w_down_exps, nullptr, nullptr, nullptr, nullptr, hp, out);
    if (rc) return rc;
    const uint16_t* tab = nullptr;
    hipError_t err = qmoe::gelu_table_device(&tab);
    if (err != hipSuccess) {
        qmoe_layer_destroy(*out);
        *out = nullptr;
        return hip_fail(err, "gelu table upload");
    }
    (*out)->d.act = qmoe::kActGeluTanh;
    (*out)->d.gelu_tab = tab;
    return QMOE_OK;
}

int qmoe_layer_destroy(qmoe_layer* layer) {
    if (!layer) return QMOE_OK;
    if (layer->own_ws) qmoe_workspace_destroy(layer->own_ws);
    if (layer->d.pk_base) (void)hipFree(layer->d.pk_base);
    if (layer->pad_base) (void)hipFree(layer->pad_base);
    delete layer;
    return QMOE_OK;
}

int qmoe_layer_n_embd(const qmoe_layer* layer) { return layer ? layer->Hu : 0; }

int qmoe_workspace_create(const qmoe_layer* like, int32_t max_tokens, qmoe_workspace** out) {
    g_last_error.clear();
    if (!out) return fail(QMOE_ERR_NULL, "qmoe: out expected a non-null qmoe_workspace**, got null");
    *out = nullptr;
    if (!like) return fail(QMOE_ERR_NULL, "qmoe: like expected a layer, got null");
    if (max_tokens < 1 || max_tokens > (1 << 20))
        return fail(QMOE_ERR_VALUE, "qmoe: max_tokens expected 1..1048576, got " + std::to_string(max_tokens));
    const LayerDesc& d = like->d;
    qmoe_workspace* ws = new (std::nothrow) qmoe_workspace();
    if (!ws) return fail(QMOE_ERR_VALUE, "qmoe: host allocation failed");
    const bool pad = like->pad_base != nullptr;
    const size_t bytes = qmoe::workspace_bytes(max_tokens, d.H, d.E, d.K, d.F, nullptr, nullptr, pad);
    void* base = nullptr;
    hipError_t err = hipMalloc(&base, bytes);
    if (err != hipSuccess) {
        delete ws;
        return hip_fail(err, "hipMalloc(workspace)");
    }
    qmoe::workspace_bytes(max_tokens, d.H, d.E, d.K, d.F, &ws->w, base, pad);
    // the signalling area (the merged top-k's finished-workgroup counter) starts at zero
    err = hipMemset(ws->w.sync, 0, qmoe::kSyncWords * sizeof(int32_t));
    if (err == hipSuccess) err = hipDeviceSynchronize();
    if (err != hipSuccess) {
        (void)hipFree(base);
        delete ws;
        return hip_fail(err, "hipMemset(workspace sync area)");
    }
    (void)hipGetDevice(&ws->device);
    *out = ws;
    return QMOE_OK;
}

int qmoe_workspace_destroy(qmoe_workspace* ws) {
    if (!ws) return QMOE_OK;
    if (ws->w.base) (void)hipFree(ws->w.base);
    delete ws;
    return QMOE_OK;
}

int32_t qmoe_workspace_capacity(const qmoe_workspace* ws) { return ws ? ws->w.cap_T : 0; }

int qmoe_workspace_check(qmoe_workspace* ws, int32_t* fault) {
    g_last_error.clear();
    if (!ws || !fault) return fail(QMOE_ERR_NULL, "qmoe: ws and fault expected non-null, got null");
    // no kernel waits on another workgroup, so no forward can fail that way: the
    // check synchronizes (surfacing any device error) and reports no fault
    hipError_t err = hipDeviceSynchronize();
    if (err != hipSuccess) return hip_fail(err, "workspace check");
    *fault = 0;
    return QMOE_OK;
}

// Scratch of the allocation-free forward: one copy of this array per GPU, held
// until the process ends.  Host code never passes `scratch` itself to a kernel
// (in host code the name is a stand-in, not a device address): it uses the
// address hipGetSymbolAddress returns on each device, kept in g_scratch.
static __device__ __align__(256) uint8_t scratch[QMOE_STATIC_SCRATCH_BYTES];
// The decode routing's signalling area sits at the start of the array.
constexpr size_t kStaticSyncBytes = 4096;
static_assert(kStaticSyncBytes >= qmoe::kSyncWords * sizeof(int32_t), "signalling area fits");

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

// The device address of this GPU's scratch (dev current), set up on first use.
// The signalling area (the merged top-k's last-workgroup counter) must start
// at zero: device globals are zero when the code object loads, the top-k
// returns its counter to zero after each use, and a first use on a stream
// that is not being captured also clears the area with a fill kernel and
// waits for it, so the array is published only after the clear has run.
int static_scratch(int dev, hipStream_t stream, void** out) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (dev < 0 || dev >= kMaxDevices)
        return fail(QMOE_ERR_VALUE, "qmoe: device expected 0.." + std::to_string(kMaxDevices - 1) + ", got " +
                                        std::to_string(dev));
    if (!g_scratch[dev]) {
        void* p = nullptr;
        hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess) return hip_fail(err, "hipGetSymbolAddress(scratch)");
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        err = hipStreamIsCapturing(stream, &cs);
        if (err != hipSuccess) return hip_fail(err, "hipStreamIsCapturing");
        if (cs == hipStreamCaptureStatusNone) {
            err = qmoe::launch_fill_i32((int32_t*)p, (int)(kStaticSyncBytes / sizeof(int32_t)), 0, stream);
            if (err == hipSuccess) err = hipStreamSynchronize(stream);
            if (err != hipSuccess) return hip_fail(err, "scratch signalling area clear");
        }
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return QMOE_OK;
}

}  // namespace

// What feeds one forward: x and optional residual, or x as the residual row of
// a fused caller slice (norm_w: the Qwen pre-MoE RMSNorm; g4_pre_w + g4_rs_w:
// the Gemma 4 expert and router inputs), or a separate router input xr.
struct ForwardIn {
    const float* x = nullptr;
    const float* xr = nullptr;        // router input (null: the experts' input)
    const float* residual = nullptr;
    const float* norm_w = nullptr;    // y = x + MoE(RMSNorm(x) * norm_w)
    const float* g4_pre_w = nullptr;  // y = MoE(rms(x)*pre_w) routed on (rms(x)/sqrt(H))*rs_w
    const float* g4_rs_w = nullptr;
    float eps = 0.0f;
    const double* x_ssq = nullptr;  // x's RMSNorm partial sums (norm_w only; optional)
    double* y_ssq = nullptr;        // receives y's RMSNorm partial sums (optional)
    bool padded_rows = false;       // x (and xr) already at the layer's padded width, y too
};

static int forward_impl(qmoe_layer* layer, qmoe_workspace* ws, const ForwardIn& in, int32_t n_tokens, float* y,
                        const qmoe_debug* dbg, void* hip_stream);

// A layer with padded widths: the caller's rows (n_embd = Hu) are prepared at
// that width (RMSNorm, the Gemma 4 inputs), zero-padded to the layer's width
// into the workspace, run there, and the first Hu columns of each output row
// written back with the residual added (the same single f32 add the combine
// ends with).
static int forward_padded(qmoe_layer* layer, qmoe_workspace* ws, const ForwardIn& in, int32_t T, float* y,
                          const qmoe_debug* dbg, void* hip_stream) {
    const LayerDesc& d = layer->d;
    const Workspace& w = ws->w;
    if (!w.yp)
        return fail(QMOE_ERR_SHAPE, "qmoe: workspace expected one created for this layer (padded widths), got one "
                                    "without padded output rows");
    const int Hu = layer->Hu, Hp = d.H;
    hipStream_t stream = (hipStream_t)hip_stream;
    // scratch rows in ybuf (at least 2 T rows; the down stage writes it later)
    float* t0 = w.ybuf;
    float* t1 = w.ybuf + (size_t)T * Hp;
    ForwardIn pin;
    pin.padded_rows = true;
    pin.x = w.xn;
    const float* res = in.residual;
    hipError_t err;
    if (in.norm_w) {
        err = qmoe::launch_rms_norm(in.x, in.norm_w, T, Hu, in.eps, t0, stream);
        if (err == hipSuccess) err = qmoe::launch_pad_rows(t0, T, Hu, Hp, w.xn, stream);
        res = in.x;
    } else if (in.g4_pre_w) {
        const float s = 1.0f / std::sqrt((float)Hu);  // gemma4.cpp:561-562, the caller's n_embd
        err = qmoe::launch_gemma4_inputs(in.x, in.g4_pre_w, in.g4_rs_w, T, Hu, in.eps, s, t0, t1, stream);
        if (err == hipSuccess) err = qmoe::launch_pad_rows(t0, T, Hu, Hp, w.xn, stream);
        if (err == hipSuccess) err = qmoe::launch_pad_rows(t1, T, Hu, Hp, w.xr, stream);
        pin.xr = w.xr;
    } else {
        err = qmoe::launch_pad_rows(in.x, T, Hu, Hp, w.xn, stream);
        if (in.xr && err == hipSuccess) {
            err = qmoe::launch_pad_rows(in.xr, T, Hu, Hp, w.xr, stream);
            pin.xr = w.xr;
        }
    }
    if (err != hipSuccess) return hip_fail(err, "padded input rows");
    const int rc = forward_impl(layer, ws, pin, T, w.yp, dbg, hip_stream);
    if (rc) return rc;
    err = qmoe::launch_unpad_rows(w.yp, T, Hp, Hu, res, y, stream);
    if (err == hipSuccess && in.y_ssq) err = qmoe::launch_rms_partials(y, T, Hu, in.y_ssq, stream);
    return err == hipSuccess ? QMOE_OK : hip_fail(err, "padded output rows");
}

static int forward_impl(qmoe_layer* layer, qmoe_workspace* ws, const ForwardIn& in, int32_t n_tokens, float* y,
                        const qmoe_debug* dbg, void* hip_stream) {
    const float* x = in.x;
    const float* residual = in.residual;
    g_last_error.clear();
    if (!layer) return fail(QMOE_ERR_NULL, "qmoe: layer expected non-null, got null");
    if (n_tokens < 0)
        return fail(QMOE_ERR_VALUE, "qmoe: n_tokens expected >= 0, got " + std::to_string(n_tokens));
    if (n_tokens == 0) return QMOE_OK;
    if (!x) return fail(QMOE_ERR_NULL, "qmoe: x expected a device pointer, got null");
    if (!y) return fail(QMOE_ERR_NULL, "qmoe: y expected a device pointer, got null");
    if (x == y) return fail(QMOE_ERR_VALUE, "qmoe: y expected a buffer distinct from x, got x");
    if (in.xr == y) return fail(QMOE_ERR_VALUE, "qmoe: y expected a buffer distinct from router_in, got router_in");
    if (((uintptr_t)x & 15u) || ((uintptr_t)y & 15u) || ((uintptr_t)residual & 15u) || ((uintptr_t)in.norm_w & 15u) ||
        ((uintptr_t)in.xr & 15u))
        return fail(QMOE_ERR_VALUE,
                    "qmoe: x/y/residual/norm_w/router_in expected 16-byte aligned device pointers, got a misaligned one");
    const LayerDesc& d = layer->d;
    if (!ws) {
        if (!layer->own_ws || layer->own_ws->w.cap_T < n_tokens) {
            // growing the layer's own workspace allocates and synchronises the
            // device: not allowed while the stream is being captured into a graph
            hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
            if (hipStreamIsCapturing((hipStream_t)hip_stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
                return fail(QMOE_ERR_CAPACITY,
                            "qmoe: n_tokens expected <= the layer's own workspace capacity " +
                                std::to_string(layer->own_ws ? layer->own_ws->w.cap_T : 0) +
                                " while the stream is capturing (pass a workspace), got " + std::to_string(n_tokens));
            if (layer->own_ws) {
                (void)hipDeviceSynchronize();
                qmoe_workspace_destroy(layer->own_ws);
                layer->own_ws = nullptr;
            }
            int rc = qmoe_workspace_create(layer, n_tokens, &layer->own_ws);
            if (rc) return rc;
        }
        ws = layer->own_ws;
    }
    const Workspace& w = ws->w;
    if (n_tokens > w.cap_T)
        return fail(QMOE_ERR_CAPACITY, "qmoe: n_tokens expected <= workspace capacity " + std::to_string(w.cap_T) +
                                           ", got " + std::to_string(n_tokens));
    if (w.H < d.H || w.E < d.E || w.K < d.K || w.F < d.F)
        return fail(QMOE_ERR_SHAPE, "qmoe: workspace expected dims >= layer (H,E,K,F)=(" + std::to_string(d.H) + "," +
                                        std::to_string(d.E) + "," + std::to_string(d.K) + "," + std::to_string(d.F) +
                                        "), got (" + std::to_string(w.H) + "," + std::to_string(w.E) + "," +
                                        std::to_string(w.K) + "," + std::to_string(w.F) + ")");
    if (layer->pad_base && !in.padded_rows) return forward_padded(layer, ws, in, n_tokens, y, dbg, hip_stream);
    // buffers are sized for the workspace's (larger or equal) dims; kernels index with the layer's
    const Workspace& v = w;
    hipStream_t stream = (hipStream_t)hip_stream;
    auto mark = [&](int i) -> hipError_t {
        return layer->record_phases ? hipEventRecord(layer->phase_events[i], stream) : hipSuccess;
    };
    hipError_t err = mark(0);
    qmoe::RouteDebug rdbg;
    if (dbg) {
        rdbg.exact_logits = dbg->logits != nullptr;
        rdbg.approx = dbg->router_approx;
        rdbg.bound = dbg->router_bound;
    }
    const float* xin = x;                    // the experts' input
    const float* xr = in.xr ? in.xr : x;     // the router's input
    // the prefill GEMMs address their A operands (x and h quants as f16) with
    // 32-bit byte offsets
    const uint64_t R = (uint64_t)n_tokens * (d.K + d.S);
    const bool mfma = n_tokens >= d.mfma_min_tokens && !qmoe::gateup_q_fused(d, n_tokens) &&
                      R * d.F * 2 + 256 < (1ull << 32) && (uint64_t)n_tokens * d.H * 2 + 256 < (1ull << 32);
    // decode: the routing normalizes x on the fly (no RMSNorm launch, no normalized copy)
    const float* route_norm_w = nullptr;
    if (in.norm_w) {
        // the residual add is the combine epilogue
        residual = x;
        if (!mfma && qmoe::route_norm_fused(d, n_tokens)) {
            route_norm_w = in.norm_w;
        } else if (mfma && qmoe::route_uses_mfma(d, n_tokens) && !dbg && d.H <= 4096) {
            // prefill: the batched router's preparation normalizes the rows (the
            // scale from x_ssq when carried) into every operand it writes, the
            // exact refinement normalizes on the fly: no normalized copy of x
            route_norm_w = in.norm_w;
        } else {
            // the normalized rows go to the workspace
            if (err == hipSuccess) err = qmoe::launch_rms_norm(x, in.norm_w, n_tokens, d.H, in.eps, v.xn, stream);
            xin = xr = v.xn;
        }
    } else if (in.g4_pre_w) {
        const float s = 1.0f / std::sqrt((float)d.H);  // gemma4.cpp:561-562
        if (err == hipSuccess)
            err = qmoe::launch_gemma4_inputs(x, in.g4_pre_w, in.g4_rs_w, n_tokens, d.H, in.eps, s, v.xn, v.xr, stream);
        xin = v.xn;
        xr = v.xr;
    }
    if (err == hipSuccess)
        err = qmoe::launch_route(d, v, xin, xr, n_tokens, rdbg, mfma, stream, route_norm_w, in.eps, in.x_ssq);
    if (err != hipSuccess) return hip_fail(err, "route kernels");
    // events [1] and [2] are taken by the gate/up launch itself (its own start and end)
    hipEvent_t e1 = layer->record_phases ? layer->phase_events[1] : nullptr;
    hipEvent_t e2 = layer->record_phases ? layer->phase_events[2] : nullptr;
    if (qmoe::gateup_q_fused(d, n_tokens)) {
        // decode: SwiGLU and the Q8_0 of h run in the gate/up kernel
        err = qmoe::launch_gateup_q(d, v, n_tokens, stream, e1, e2);
        if (err != hipSuccess) return hip_fail(err, "gate/up+quant expert kernel");
    } else if (mfma) {
        // prefill: SwiGLU and the Q8_0 of h (as the down GEMM's f16 planes) run in the gate/up epilogue
        err = qmoe::launch_gateup_mfma(d, v, n_tokens, stream, e1, e2);
        if (err != hipSuccess) return hip_fail(err, "gate/up expert kernel");
    } else {
        err = qmoe::launch_experts_gateup(d, v, n_tokens, stream, e1, e2);
        if (err != hipSuccess) return hip_fail(err, "gate/up expert kernel");
        err = qmoe::launch_quant_h(d, v, n_tokens, stream);
    }
    bool ssq_done = false;
    if (qmoe::down_combine_fused(d, n_tokens)) {
        // decode: the combine runs in the down kernel's epilogue (and y's partial sums with it)
        if (err == hipSuccess) err = qmoe::launch_down_combine(d, v, n_tokens, y, residual, stream, in.y_ssq, &ssq_done);
        if (err != hipSuccess) return hip_fail(err, "down+combine kernel");
        err = mark(3);
    } else {
        if (err == hipSuccess)
            err = mfma ? qmoe::launch_down_mfma(d, v, n_tokens, stream) : qmoe::launch_experts_down(d, v, n_tokens, stream);
        if (err != hipSuccess) return hip_fail(err, "down expert kernel");
        err = mark(3);
        if (err == hipSuccess) err = qmoe::launch_combine(d, v, n_tokens, y, residual, stream, in.y_ssq);
        if (err != hipSuccess) return hip_fail(err, "combine kernel");
        ssq_done = in.y_ssq != nullptr && d.H % 32 == 0;
    }
    if (in.y_ssq && !ssq_done) {
        err = qmoe::launch_rms_partials(y, n_tokens, d.H, in.y_ssq, stream);
        if (err != hipSuccess) return hip_fail(err, "RMSNorm partial sums");
    }
    err = mark(4);
    if (err != hipSuccess) return hip_fail(err, "phase event record");
    if (dbg) {
        const size_t T = (size_t)n_tokens;
        if (dbg->logits) {
            err = hipMemcpy2DAsync(dbg->logits, d.E * sizeof(float), v.logits, (d.E + 1) * sizeof(float),
                                   d.E * sizeof(float), T, hipMemcpyDeviceToDevice, stream);
            if (err != hipSuccess) return hip_fail(err, "debug copy (logits)");
        }
        struct { void* dst; const void* src; size_t bytes; const char* what; } cp[] = {
            {dbg->topk_idx, v.topk_idx, T * d.K * 4, "topk_idx"},
            {dbg->topk_w, v.topk_w, T * d.K * 4, "topk_w"},
            {d.S ? dbg->sh_gate : nullptr, v.sh_gate, T * 4, "sh_gate"},
            {dbg->offsets, v.offsets, (size_t)(d.E + 1) * 4, "offsets"},
            {dbg->rows, v.rows, T * d.K * 4, "rows"},
        };
        for (auto& c : cp) {
            if (!c.dst) continue;
            err = hipMemcpyAsync(c.dst, c.src, c.bytes, hipMemcpyDeviceToDevice, stream);
            if (err != hipSuccess) return hip_fail(err, c.what);
        }
        // per-row intermediates in assignment order, at the caller's widths
        const int A = n_tokens * d.K, R = A + d.S * n_tokens;
        const int Fo = layer->Fu ? layer->Fu : d.F, Ho = layer->Hu ? layer->Hu : d.H;
        if (dbg->h_qs && dbg->h_d) {
            err = mfma ? qmoe::launch_debug_h(v.rows, A, R, d.F, Fo, nullptr, nullptr, v.h_q, v.h_d, dbg->h_qs, dbg->h_d,
                                              stream)
                       : qmoe::launch_debug_h(v.rows, A, R, d.F, Fo, v.hq_qs, v.hq_ds, nullptr, nullptr, dbg->h_qs,
                                              dbg->h_d, stream);
            if (err != hipSuccess) return hip_fail(err, "debug copy (h)");
        }
        if (dbg->h_fixed) {
            err = mfma ? hipMemcpyAsync(dbg->h_fixed, v.counters + qmoe::kCounterFix, 4, hipMemcpyDeviceToDevice, stream)
                       : qmoe::launch_fill_i32(dbg->h_fixed, 1, 0, stream);
            if (err != hipSuccess) return hip_fail(err, "debug copy (h_fixed)");
        }
        if (dbg->exp_down && !qmoe::down_combine_fused(d, n_tokens)) {
            err = qmoe::launch_debug_rows(v.rows, A, R, d.H, Ho, v.ybuf, dbg->exp_down, stream);
            if (err != hipSuccess) return hip_fail(err, "debug copy (exp_down)");
        }
    }
    return QMOE_OK;
}

int qmoe_layer_forward(qmoe_layer* layer, qmoe_workspace* ws, const float* x, int32_t n_tokens, float* y,
                       const float* residual, const qmoe_debug* dbg, void* hip_stream) {
    ForwardIn in;
    in.x = x;
    in.residual = residual;
    return forward_impl(layer, ws, in, n_tokens, y, dbg, hip_stream);
}

int qmoe_layer_forward_static(qmoe_layer* layer, const float* x, int32_t n_tokens, float* y, const float* residual,
                              void* hip_stream) {
    g_last_error.clear();
    if (!layer) return fail(QMOE_ERR_NULL, "qmoe: layer expected non-null, got null");
    if (n_tokens < 0) return fail(QMOE_ERR_VALUE, "qmoe: n_tokens expected >= 0, got " + std::to_string(n_tokens));
    if (n_tokens == 0) return QMOE_OK;
    const LayerDesc& d = layer->d;
    const bool pad = layer->pad_base != nullptr;
    const size_t need =
        kStaticSyncBytes + qmoe::workspace_bytes(n_tokens, d.H, d.E, d.K, d.F, nullptr, nullptr, pad);
    if (need > QMOE_STATIC_SCRATCH_BYTES)
        return fail(QMOE_ERR_CAPACITY, "qmoe: n_tokens expected a scratch of at most " +
                                           std::to_string(QMOE_STATIC_SCRATCH_BYTES) + " bytes (the static scratch), got " +
                                           std::to_string(n_tokens) + " tokens needing " + std::to_string(need));
    int dev = -1;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return hip_fail(err, "hipGetDevice");
    if (dev != layer->device)
        return fail(QMOE_ERR_VALUE, "qmoe: current device expected the layer's device " + std::to_string(layer->device) +
                                        ", got " + std::to_string(dev));
    void* base = nullptr;
    int rc = static_scratch(dev, (hipStream_t)hip_stream, &base);
    if (rc) return rc;
    // the signalling area keeps its place at the start of the array from call to
    // call; the rest is carved for this call's token count
    qmoe_workspace ws;
    ws.device = dev;
    qmoe::workspace_bytes(n_tokens, d.H, d.E, d.K, d.F, &ws.w, (char*)base + kStaticSyncBytes, pad);
    ws.w.sync = (int32_t*)base;
    ForwardIn in;
    in.x = x;
    in.residual = residual;
    return forward_impl(layer, &ws, in, n_tokens, y, nullptr, hip_stream);
}

int qmoe_layer_forward_norm(qmoe_layer* layer, qmoe_workspace* ws, const float* x, const float* norm_w, float eps,
                            int32_t n_tokens, float* y, const qmoe_debug* dbg, void* hip_stream) {
    g_last_error.clear();
    if (!norm_w) return fail(QMOE_ERR_NULL, "qmoe: norm_w expected a device pointer, got null");
    if (!(eps >= 0.0f)) return fail(QMOE_ERR_VALUE, "qmoe: eps expected >= 0, got " + std::to_string(eps));
    ForwardIn in;
    in.x = x;
    in.norm_w = norm_w;
    in.eps = eps;
    return forward_impl(layer, ws, in, n_tokens, y, dbg, hip_stream);
}

int qmoe_layer_forward_norm_chain(qmoe_layer* layer, qmoe_workspace* ws, const float* x, const double* x_ssq,
                                  const float* norm_w, float eps, int32_t n_tokens, float* y, double* y_ssq,
                                  const qmoe_debug* dbg, void* hip_stream) {
    g_last_error.clear();
    if (!norm_w) return fail(QMOE_ERR_NULL, "qmoe: norm_w expected a device pointer, got null");
    if (!(eps >= 0.0f)) return fail(QMOE_ERR_VALUE, "qmoe: eps expected >= 0, got " + std::to_string(eps));
    if (((uintptr_t)x_ssq & 15u) || ((uintptr_t)y_ssq & 15u))
        return fail(QMOE_ERR_VALUE, "qmoe: x_ssq/y_ssq expected 16-byte aligned device pointers, got a misaligned one");
    ForwardIn in;
    in.x = x;
    in.norm_w = norm_w;
    in.eps = eps;
    in.x_ssq = x_ssq;
    in.y_ssq = y_ssq;
    return forward_impl(layer, ws, in, n_tokens, y, dbg, hip_stream);
}

int qmoe_rms_partials(const float* x, int32_t n_tokens, int32_t n_embd, double* out, void* hip_stream) {
    g_last_error.clear();
    if (n_tokens < 0 || n_embd <= 0)
        return fail(QMOE_ERR_VALUE, "qmoe: n_tokens >= 0 and n_embd > 0 expected, got " + std::to_string(n_tokens) +
                                        ", " + std::to_string(n_embd));
    if (n_tokens == 0) return QMOE_OK;
    if (!x || !out) return fail(QMOE_ERR_NULL, "qmoe: x/out expected device pointers, got null");
    if ((uintptr_t)out & 7u) return fail(QMOE_ERR_VALUE, "qmoe: out expected an 8-byte aligned device pointer");
    const hipError_t err = qmoe::launch_rms_partials(x, n_tokens, n_embd, out, (hipStream_t)hip_stream);
    return err == hipSuccess ? QMOE_OK : hip_fail(err, "RMSNorm partial sums");
}

int qmoe_layer_forward_routed(qmoe_layer* layer, qmoe_workspace* ws, const float* expert_in, const float* router_in,
                              int32_t n_tokens, float* y, const qmoe_debug* dbg, void* hip_stream) {
    g_last_error.clear();
    if (n_tokens > 0 && !router_in)
        return fail(QMOE_ERR_NULL, "qmoe: router_in expected a device pointer, got null");
    ForwardIn in;
    in.x = expert_in;
    in.xr = router_in;
    return forward_impl(layer, ws, in, n_tokens, y, dbg, hip_stream);
}

int qmoe_layer_forward_gemma4(qmoe_layer* layer, qmoe_workspace* ws, const float* x, const float* pre_norm_w,
                              const float* router_scale_w, float eps, int32_t n_tokens, float* y, const qmoe_debug* dbg,
                              void* hip_stream) {
    g_last_error.clear();
    if (!pre_norm_w || !router_scale_w)
        return fail(QMOE_ERR_NULL, "qmoe: pre_norm_w and router_scale_w expected device pointers, got null");
    if (((uintptr_t)pre_norm_w & 3u) || ((uintptr_t)router_scale_w & 3u))
        return fail(QMOE_ERR_VALUE, "qmoe: pre_norm_w/router_scale_w expected 4-byte aligned, got a misaligned one");
    if (!(eps >= 0.0f)) return fail(QMOE_ERR_VALUE, "qmoe: eps expected >= 0, got " + std::to_string(eps));
    ForwardIn in;
    in.x = x;
    in.g4_pre_w = pre_norm_w;
    in.g4_rs_w = router_scale_w;
    in.eps = eps;
    return forward_impl(layer, ws, in, n_tokens, y, dbg, hip_stream);
}

int qmoe_gemma4_moe_inputs(const float* x, const float* pre_norm_w, const float* router_scale_w, float eps,
                           int32_t n_tokens, int32_t n_embd, float* expert_in, float* router_in, void* hip_stream) {
    g_last_error.clear();
    if (n_tokens < 0) return fail(QMOE_ERR_VALUE, "qmoe: n_tokens expected >= 0, got " + std::to_string(n_tokens));
    if (n_tokens == 0) return QMOE_OK;
    if (!x || !pre_norm_w || !router_scale_w || !expert_in || !router_in)
        return fail(QMOE_ERR_NULL, "qmoe: x/pre_norm_w/router_scale_w/expert_in/router_in expected device pointers, got null");
    if (n_embd < 1 || n_embd > 4096)
        return fail(QMOE_ERR_VALUE, "qmoe: n_embd expected 1..4096, got " + std::to_string(n_embd));
    if (!(eps >= 0.0f)) return fail(QMOE_ERR_VALUE, "qmoe: eps expected >= 0, got " + std::to_string(eps));
    const float s = 1.0f / std::sqrt((float)n_embd);
    hipError_t err = qmoe::launch_gemma4_inputs(x, pre_norm_w, router_scale_w, n_tokens, n_embd, eps, s, expert_in,
                                                router_in, (hipStream_t)hip_stream);
    return err == hipSuccess ? QMOE_OK : hip_fail(err, "gemma4 inputs kernel");
}

int qmoe_layer_set_expert_counts(qmoe_layer* layer, uint64_t* device_counts) {
    g_last_error.clear();
    if (!layer) return fail(QMOE_ERR_NULL, "qmoe: layer expected non-null, got null");
    if ((uintptr_t)device_counts & 7u)
        return fail(QMOE_ERR_VALUE, "qmoe: device_counts expected 8-byte aligned, got a misaligned pointer");
    layer->d.expert_counts = (unsigned long long*)device_counts;
    return QMOE_OK;
}

int qmoe_layer_set_phase_events(qmoe_layer* layer, void* const* events) {
    g_last_error.clear();
    if (!layer) return fail(QMOE_ERR_NULL, "qmoe: layer expected non-null, got null");
    if (!events) {
        layer->record_phases = false;
        return QMOE_OK;
    }
    for (int i = 0; i < QMOE_N_PHASE_EVENTS; ++i) {
        if (!events[i])
            return fail(QMOE_ERR_NULL, "qmoe: events[" + std::to_string(i) + "] expected a hipEvent_t, got null");
        layer->phase_events[i] = (hipEvent_t)events[i];
    }
    layer->record_phases = true;
    return QMOE_OK;
}

int qmoe_rms_norm(const float* x, const float* w, int32_t n_tokens, int32_t n_embd, float eps, float* y,
                  void* hip_stream) {
    g_last_error.clear();
    if (n_tokens < 0) return fail(QMOE_ERR_VALUE, "qmoe: n_tokens expected >= 0, got " + std::to_string(n_tokens));
    if (n_tokens == 0) return QMOE_OK;
    if (!x || !y) return fail(QMOE_ERR_NULL, "qmoe: x/y expected device pointers, got null");
    if (n_embd < 1 || n_embd > 256 * qmoe::kRmsMaxChunks)
        return fail(QMOE_ERR_VALUE, "qmoe: n_embd expected 1.." + std::to_string(256 * qmoe::kRmsMaxChunks) + ", got " +
                                        std::to_string(n_embd));
    hipError_t err = qmoe::launch_rms_norm(x, w, n_tokens, n_embd, eps, y, (hipStream_t)hip_stream);
    return err == hipSuccess ? QMOE_OK : hip_fail(err, "rms_norm kernel");
}

int qmoe_synth_f32(float* dst, int64_t n, uint64_t seed, uint64_t stream, double mean, double sigma,
                   void* hip_stream) {
    g_last_error.clear();
    if (n < 0) return fail(QMOE_ERR_VALUE, "qmoe: n expected >= 0, got " + std::to_string(n));
    if (n == 0) return QMOE_OK;
    if (!dst) return fail(QMOE_ERR_NULL, "qmoe: dst expected a device pointer, got null");
    hipError_t err = qmoe::launch_synth_f32(dst, n, seed, stream, mean, sigma, (hipStream_t)hip_stream);
    return err == hipSuccess ? QMOE_OK : hip_fail(err, "synth_f32 kernel");
}

int qmoe_synth_quant(void* dst, int32_t type, int64_t n_rows, int64_t row_len, uint64_t seed, uint64_t stream,
                     double sigma, void* hip_stream) {
    g_last_error.clear();
    if (type != QMOE_TYPE_Q4_0 && type != QMOE_TYPE_Q8_0)
        return fail(QMOE_ERR_TYPE, "qmoe: type expected Q4_0 or Q8_0, got " + type_str(type));
    if (n_rows < 0 || row_len < 0 || row_len % 32 != 0)
        return fail(QMOE_ERR_VALUE, "qmoe: rows x row_len expected n_rows >= 0 and row_len a multiple of 32, got " +
                                        std::to_string(n_rows) + " x " + std::to_string(row_len));
    if (n_rows == 0 || row_len == 0) return QMOE_OK;
    if (!dst) return fail(QMOE_ERR_NULL, "qmoe: dst expected a device pointer, got null");
    if ((uintptr_t)dst & 1u) return fail(QMOE_ERR_VALUE, "qmoe: dst expected 2-byte alignment, got odd address");
    hipError_t err = qmoe::launch_synth_quant(dst, type, n_rows, row_len, seed, stream, sigma, (hipStream_t)hip_stream);
    return err == hipSuccess ? QMOE_OK : hip_fail(err, "synth_quant kernel");
}

}  // extern "C"
