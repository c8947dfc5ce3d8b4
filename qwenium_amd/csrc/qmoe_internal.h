// qmoe_internal.h -- host-side layer/workspace structures and kernel launchers.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <string>
#include <stdint.h>

namespace qmoe {

// Tokens handled by one top-k block; the per-block histogram granularity of
// the stable counting sort.
constexpr int kTopkTokensPerBlock = 16;
constexpr int kTopkMinTokensPerBlock = 4;  // the unmerged top-k's smallest blocks (more blocks to fill the CUs)
// Cross-block signalling area of a workspace: the merged top-k's
// finished-workgroup counter (back to 0 after each use).
constexpr int kSyncWords = 64;
constexpr int kSyncTopk = 1;
constexpr int kTopkMergeMax = 4096;  // top-k blocks x experts the merged top-k keeps in LDS
// Copies of the per-expert totals that the top-k blocks add into (block b into
// copy b % kTotalCopies: fewer atomics on one address).
constexpr int kTotalCopies = 8;
// RMSNorm: 256-column chunks of a row whose sums fit a workgroup's LDS (rows of
// at most 65536 columns).
constexpr int kRmsMaxChunks = 256;
// Row tile of the prefill grouped GEMM (rows of one expert per tile).
constexpr int kMfmaTileM = 128;
// k values per LDS chunk of the prefill GEMMs.
constexpr int kF16ChunkK = 64;
// Workspace counters (kCounters ints): [0] active slots, [1] tiles,
// [kCounterFix] listed h blocks.
constexpr int kCounters = 32;
constexpr int kCounterFix = 4;
constexpr int kFixStride = 36;  // floats per listed h block: 32 values, amax's error estimate, padding
// Expert activations: SwiGLU (moe.cpp:117) or GeGLU-tanh (gemma4.cpp:423).
constexpr int kActSilu = 0;
constexpr int kActGeluTanh = 1;

struct LayerDesc {
    int H = 0, E = 0, K = 0, F = 0, S = 0;  // n_embd, n_experts, top_k, ffn_dim, shared (0/1)
    int gu_type = 0, dn_type = 0;           // gate/up type, down type (Q4_0 or Q8_0)
    const float* w_router = nullptr;
    uint64_t router_ld = 0;                 // row stride in floats
    const uint8_t* w_gate = nullptr;
    const uint8_t* w_up = nullptr;
    uint64_t gate_nb1 = 0, gate_nb2 = 0, up_nb1 = 0, up_nb2 = 0;
    const uint8_t* w_down = nullptr;
    uint64_t down_nb1 = 0, down_nb2 = 0;
    const uint8_t* w_sh_gate = nullptr;
    const uint8_t* w_sh_up = nullptr;
    const uint8_t* w_sh_down = nullptr;
    uint64_t sh_gate_nb1 = 0, sh_up_nb1 = 0, sh_down_nb1 = 0;
    const float* w_sh_norm = nullptr;
    int n_cu = 256;                         // compute units of the layer's device
    int mfma_min_tokens = 128;              // token count from which the f16-MFMA GEMMs run (set per shape)
    int big_router_min_tokens = 256;        // token count from which the bf16-MFMA router runs (set per shape)
    int dc_ahead = 2;                       // decode down+combine: steps with loads in flight (2 or 4)
    unsigned long long* expert_counts = nullptr;  // optional device [E]: += each forward's per-expert dispatches
    int act = 0;                            // 0 SwiGLU (silu(g)*u), 1 GeGLU-tanh (gelu(g)*u, ggml's fp16 table)
    const uint16_t* gelu_tab = nullptr;     // device [65536] fp16 gelu table of the layer's device (GeGLU)
    // Chunk-major copies of the expert matrices for the prefill GEMMs (null: they
    // read the GGUF rows): [expert][block pair p][row r] raw block pairs, so the
    // lanes of a wave read consecutive pairs of one k chunk (a few cache lines
    // per load instead of one per lane).  Built once at creation; pk_base owns them.
    const uint8_t* pk_gate = nullptr;
    const uint8_t* pk_up = nullptr;
    const uint8_t* pk_down = nullptr;
    const uint8_t* pk_sh_gate = nullptr;
    const uint8_t* pk_sh_up = nullptr;
    const uint8_t* pk_sh_down = nullptr;
    void* pk_base = nullptr;
};
// The chunk-major copies (LayerDesc::pk_*) of a layer's expert matrices.
hipError_t build_prefill_copies(LayerDesc& d);

// Device scratch.  R = T*K + S*T rows: routed assignments sorted by expert,
// then the shared expert's rows in token order.
struct Workspace {
    int cap_T = 0, H = 0, E = 0, K = 0, F = 0;
    void* base = nullptr;
    size_t bytes = 0;
    int8_t* xq_qs = nullptr;      // [T][H]   Q8_0 activation quants
    float2* xq_ds = nullptr;      // [T][H/32] {d, bitcast(sum q)}
    float* logits = nullptr;      // [T][E+1] (column E: shared gate logit)
    float* logit_bound = nullptr; // [T][E] error bound of the approximate (MFMA) logits
    int32_t* topk_idx = nullptr;  // [T][K]
    float* topk_w = nullptr;      // [T][K]
    float* sh_gate = nullptr;     // [T]
    int32_t* local_rank = nullptr;  // [T*K]
    int32_t* hist = nullptr;      // [nblk + kTotalCopies][E] per top-k block counts or token masks, then the totals
    uint64_t* jslot = nullptr;    // [nblk][E] the slot of each masked token, four bits each
    int32_t* offsets = nullptr;   // [E+2]
    int32_t* rows = nullptr;      // [R] assignment id (t*K+j); shared rows: -1
    int32_t* row_token = nullptr; // [R]
    int32_t* pos = nullptr;       // [T*K] position of assignment
    int32_t* active = nullptr;    // [E+1] active experts (ascending), shared (=E) last
    int32_t* expert_slot = nullptr; // [E] slot of each active expert
    int4* slot_info = nullptr;    // [E+1] per active slot {expert, first row, rows, 0}
    int4* dslots = nullptr;       // [E+2] decode slot list {expert, first row, rows, token mask}:
                                  // active routed experts, then expert -1 up to min(E, T*K)
    int32_t* counters = nullptr;  // [kCounters] n_active, n_tiles, ...
    int32_t* sync = nullptr;      // [kSyncWords] zeroed at creation: the merged top-k's finished-workgroup counter
    int4* tiles = nullptr;        // [max tiles] {expert, row0, nrows, 0}
    float2* gubuf = nullptr;      // [R][F] (gate, up) projections
    int8_t* hq_qs = nullptr;      // [R][F]   Q8_0 quants of h = silu(g)*u
    float2* hq_ds = nullptr;      // [R][F/32] {d, bitcast(sum q)}
    // prefill GEMM operands: Q8_0 quants as exact f16 values and fp16 block scales
    _Float16* x_q = nullptr;      // [T][H] x (the experts' input)
    uint16_t* x_d = nullptr;      // [T][H/32]
    _Float16* h_q = nullptr;      // [R][F] h (aliases gubuf: the prefill path writes no (g, u))
    uint16_t* h_d = nullptr;      // [R][F/32]
    // batched router operands: bf16 hi/lo splits of the router input and weights, row norms
    uint16_t* rx_split = nullptr; // [2][T][H] (hi, lo)
    uint16_t* rw_split = nullptr; // [2][E][H]
    float* rnorm = nullptr;       // [T + E] |x_t|, |w_e|
    int4* fix = nullptr;          // [fix_max] h blocks whose rounding the f32 values do not settle
    float* fix_h = nullptr;       // [fix_max][kFixStride] their 32 f32 h values and amax's error estimate
    int fix_max = 0;
    float* xn = nullptr;          // [T][H] RMSNorm(x)*w for fused-norm forwards (the experts' input)
    float* xr = nullptr;          // [T][H] the router's own input when it differs (Gemma 4 slice)
    float* x_scale = nullptr;     // [T] RMSNorm scales of a forward that normalizes in its routing
    float* ybuf = nullptr;        // [R][H] down outputs (unweighted)
    float* ysh = nullptr;         // [T][H] the shared expert's down rows (fused decode)
    float* yp = nullptr;          // [T][H] output rows of a layer with padded widths (null otherwise)
    int max_tiles = 0;
};

size_t workspace_bytes(int T, int H, int E, int K, int F, Workspace* carve, void* base, bool pad = false);

// Launch with optional start/stop events recorded by the launch itself.
template <typename K, typename... Args>
inline void launch_timed(K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t stream, hipEvent_t ev_start,
                         hipEvent_t ev_stop, Args... args) {
    if (ev_start || ev_stop)
        hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, stream, ev_start, ev_stop, 0u, args...);
    else
        hipLaunchKernelGGL(kernel, grid, block, lds, stream, args...);
}

// Error reporting shared by the host sources (qmoe_last_error() text, status code).
void clear_error();
int set_error(int code, const std::string& msg);
int hip_error(hipError_t err, const char* what);

// --- launchers (each enqueues on `stream`, returns hipError_t of the launch) ---
// Routing: logits, top-k + softmax + shared gate, counting sort.  Large T
// routes through the bf16-MFMA router with exact refinement; exact_logits
// additionally leaves the exact logits of every expert in ws.logits.
struct RouteDebug {
    bool exact_logits = false;      // leave exact logits of all experts in ws.logits
    float* approx = nullptr;        // [T][E] MFMA-router approximate logits (MFMA router only)
    float* bound = nullptr;         // [T][E] their error bounds
};
bool route_uses_mfma(const LayerDesc& L, int T);
// One-launch decode routing (T <= 16); it also writes ws.dslots.
bool route_decode_fused(const LayerDesc& L, int T);
// x: the experts' input (quantized to Q8_0); xr: the router's input (x for
// the Qwen layer; the scaled norm for Gemma 4); the shared gate reads xr.
// x_f16: also write x's Q8_0 quants as f16 and its fp16 block scales (ws.x_q,
// ws.x_d), the prefill GEMMs' A operand (inside the batched router's launch,
// else a launch of its own).
// norm_w: x (== xr) is the residual row and the routing normalizes it on the
// fly, x_in = (x * rms scale) * norm_w, for the router and for x's Q8_0: at
// decode (T <= 16 without x_f16, route_norm_fused says when) and in the batched
// router (route_uses_mfma, with x_f16); x_ssq (optional): x's partial sums.
hipError_t launch_route(const LayerDesc& L, const Workspace& ws, const float* x, const float* xr, int T,
                        const RouteDebug& dbg, bool x_f16, hipStream_t stream, const float* norm_w = nullptr,
                        float eps = 0.0f, const double* x_ssq = nullptr);
bool route_norm_fused(const LayerDesc& L, int T);
// ev_start / ev_stop (optional): events recorded at the kernel's own start and
// end (profiling of the dominant kernel without marker overhead).
hipError_t launch_experts_gateup(const LayerDesc& L, const Workspace& ws, int T, hipStream_t stream,
                                 hipEvent_t ev_start = nullptr, hipEvent_t ev_stop = nullptr);
hipError_t launch_experts_down(const LayerDesc& L, const Workspace& ws, int T, hipStream_t stream);
hipError_t launch_quant_h(const LayerDesc& L, const Workspace& ws, int T, hipStream_t stream);
// Decode: gate/up + SwiGLU + Q8_0 of h of the routed experts in one launch
// over ws.dslots (replaces launch_experts_gateup + launch_quant_h when
// gateup_q_fused(); the decode routing launch computes the shared expert's h).
bool gateup_q_fused(const LayerDesc& L, int T);
hipError_t launch_gateup_q(const LayerDesc& L, const Workspace& ws, int T, hipStream_t stream,
                           hipEvent_t ev_start = nullptr, hipEvent_t ev_stop = nullptr);
hipError_t launch_gateup_mfma(const LayerDesc& L, const Workspace& ws, int T, hipStream_t stream,
                              hipEvent_t ev_start = nullptr, hipEvent_t ev_stop = nullptr);
hipError_t launch_down_mfma(const LayerDesc& L, const Workspace& ws, int T, hipStream_t stream);
// y_ssq (optional): y's RMSNorm partial sums, written with the rows (n_embd a
// multiple of 32; otherwise ignored and left to the caller).
hipError_t launch_combine(const LayerDesc& L, const Workspace& ws, int T, float* y, const float* residual,
                          hipStream_t stream, double* y_ssq = nullptr);
// Decode sizes: token-major down projection with the combine in its epilogue
// (replaces launch_experts_down + launch_combine when down_combine_fused()).
bool down_combine_fused(const LayerDesc& L, int T);
// The token-per-workgroup down+combine kernel takes the layer's K + S steps.
bool down_combine_tok_fits(const LayerDesc& L);
// Fused decode with a shared expert of F = 512 (down rows of the gate/up type):
// its down projection runs in the gate/up launch, on workgroups of their own,
// into ws.ysh; the down+combine kernel adds ysh * sh_gate as its last step
// instead of computing it.
bool shared_down_in_gateup(const LayerDesc& L, int T);
// y_ssq (optional): y's RMSNorm partial sums, written by the epilogue where the
// kernel's rows allow it (*ssq_done set), otherwise left to the caller.
hipError_t launch_down_combine(const LayerDesc& L, const Workspace& ws, int T, float* y, const float* residual,
                               hipStream_t stream, double* y_ssq = nullptr, bool* ssq_done = nullptr);
hipError_t launch_rms_norm(const float* x, const float* w, int T, int H, float eps, float* y, hipStream_t stream);
// out[T][ssq_parts(H)]: the RMSNorm partial sums of the rows x[T][H].
hipError_t launch_rms_partials(const float* x, int T, int H, double* out, hipStream_t stream);
// dst[0..n) = v on `stream` (a kernel, never a memset node).
hipError_t launch_fill_i32(int32_t* dst, int n, int32_t v, hipStream_t stream);
// Debug copies in assignment order (workspace row p -> row rows[p] for p < A,
// p for the shared rows after them): h's Q8_0 from either representation
// (qs8/ds8: int8 quants and {d, sum}; q16/d16: f16 quants and fp16 scale bits),
// the first fo columns of f; and f32 rows, the first ho columns of h.
hipError_t launch_debug_h(const int32_t* rows, int A, int R, int f, int fo, const int8_t* qs8, const float2* ds8,
                          const _Float16* q16, const uint16_t* d16, int8_t* out_q, float* out_d, hipStream_t stream);
hipError_t launch_debug_rows(const int32_t* rows, int A, int R, int h, int ho, const float* src, float* out,
                             hipStream_t stream);
// Rows of hs floats -> rows of hd >= hs floats, zeros after column hs (the
// input of a layer whose widths were padded); and back: the first hd of each
// hs-wide row, plus residual (when non-null) as one f32 add per value.
hipError_t launch_pad_rows(const float* src, int T, int hs, int hd, float* dst, hipStream_t stream);
hipError_t launch_unpad_rows(const float* src, int T, int hs, int hd, const float* residual, float* dst,
                             hipStream_t stream);
// Gemma 4 MoE inputs from one pass over x (H <= 4096): expert_in = (x*scale)*w_pre,
// router_in = ((x*scale)*s)*w_rs with scale = 1/sqrtf(mean(x^2) + eps).
hipError_t launch_gemma4_inputs(const float* x, const float* w_pre, const float* w_rs, int T, int H, float eps, float s,
                                float* expert_in, float* router_in, hipStream_t stream);
// ggml's CPU fp16 gelu table (65536 entries): host copy, and the current device's copy.
void gelu_table_host(uint16_t* out);
hipError_t gelu_table_device(const uint16_t** out);
hipError_t launch_synth_f32(float* dst, int64_t n, uint64_t seed, uint64_t stream_id, double mean, double sigma,
                            hipStream_t stream);
hipError_t launch_synth_quant(void* dst, int type, int64_t n_rows, int64_t row_len, uint64_t seed,
                              uint64_t stream_id, double sigma, hipStream_t stream);

}  // namespace qmoe
