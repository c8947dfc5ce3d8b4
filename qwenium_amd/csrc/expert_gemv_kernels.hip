// expert_gemv_kernels.hip -- grouped expert SwiGLU for small token counts
// (decode): bandwidth-bound GEMV over the per-expert row lists, then the
// k-ordered weighted combine with the sigmoid-gated shared expert.
//
// Semantics restated from src/layers/moe.cpp:105-127 (3x ggml_mul_mat_id with
// Q8_0-quantized activations), :117 (silu(g)*u), :134-151 (weights times
// outputs, summed in slot order), :161-174 (shared expert, sigmoid gate, add).
//
// Weight rows are read straight from GGUF block layout: a lane owns a pair of
// 32-value blocks (36 B Q4_0 / 68 B Q8_0) and loads it with dword-aligned
// 16-byte loads; lanes of a row cover it contiguously, so each wave streams
// whole rows.  Nibbles are unpacked in registers; dots use v_dot4_i32_i8.
#include "qmoe_device.h"
#include "qmoe_internal.h"

#include <algorithm>

namespace qmoe {

struct ExpertArgs {
    int H, F, E, K, S, T;
    const uint8_t* w_gate; const uint8_t* w_up; uint64_t gate_nb1, gate_nb2, up_nb1, up_nb2;
    const uint8_t* w_down; uint64_t down_nb1, down_nb2;
    const uint8_t* w_sh_gate; const uint8_t* w_sh_up; const uint8_t* w_sh_down;
    uint64_t sh_gate_nb1, sh_up_nb1, sh_down_nb1;
    const int32_t* counters;   // [0] n_active
    const int4* slot_info;     // [E+1] {expert, first row, rows, token of first row}
    const int32_t* offsets;    // [E+2]
    const int32_t* row_token;  // [R]
    const int8_t* xq_qs; const float2* xq_ds;  // [T][H], [T][H/32]
    float2* gubuf;                             // [R][F] (gate, up) projections (f32)
    int8_t* hq_qs; float2* hq_ds;              // [R][F], [R][F/32] Q8_0 of hbuf
    float* ybuf;                               // [R][H] down outputs (unweighted)
    int act;                                   // kActSilu or kActGeluTanh
    const uint16_t* gelu_tab;                  // [65536] fp16 gelu table (GeGLU layers)
    float* ysh;                                // [T][H] the shared expert's down rows (fused decode)
    int sd_blocks;                             // fused decode gate/up: leading workgroups computing ysh
};

// Loads the slot table into LDS (all E+1 entries; those past n_active are
// never read) and returns n_active.  One latency at kernel start.
__device__ __forceinline__ int stage_slots(const ExpertArgs& a, int4* s_slots, int* s_nact) {
    for (int i = threadIdx.x; i <= a.E; i += blockDim.x) s_slots[i] = a.slot_info[i];
    if (threadIdx.x == 0) *s_nact = a.counters[0];
    __syncthreads();
    return *s_nact;
}

// ---------------------------------------------------------------------------
// G1: gate + up projections -> gubuf (f32 pairs), persistent streaming.
// Work item = (active slot, group of RPW consecutive ffn rows of gate and up).
// Items are strided over all waves (consecutive waves take consecutive row
// groups of one expert); each wave prefetches the next item's weights and
// first-token activations while it computes the current item.  LPR lanes
// cover one H row (lane lp owns 64-value pair lp); RPI = 64/LPR rows per load
// instruction, NI = RPW/RPI loads per matrix.
// ---------------------------------------------------------------------------
template <int WT, int LPR, int RPW>
struct GuItem {
    static constexpr int RPI = 64 / LPR;
    static constexpr int NI = RPW / RPI;
    WPair<WT> wg[NI], wu[NI];
    XPair x;
    int e, p0, nrows, f0, t0;  // t0: the shared expert's first token (its rows are tokens t0, t0 + 1, ...)
};

// The shared expert's rows (one per token) go to items of kShChunk rows each, so
// that no item walks all T rows one after another.
constexpr int kShChunk = 8;
__device__ __forceinline__ int sh_chunks(const ExpertArgs& a) { return a.S ? (a.T + kShChunk - 1) / kShChunk : 0; }
// Slot entry of item `item` (ips items per slot or shared chunk): the shared
// expert's chunks first (the heaviest items), then the routed experts' slots.
__device__ __forceinline__ int4 item_slot_info(const ExpertArgs& a, const int4* slots, int item, int ips, int n_act) {
    const int k = item / ips, nsh = sh_chunks(a);
    if (k < nsh) {
        const int c0 = k * kShChunk;
        return make_int4(a.E, a.T * a.K + c0, min(kShChunk, a.T - c0), c0);
    }
    return slots[k - nsh];
}

// Activation source of the gate/up kernel: the quantized token rows and the
// row -> token map, in LDS (decode: staged once per block) or in global memory.
struct XSrc {
    const int8_t* qs;     // [T][H]
    const float2* ds;     // [T][H/32]
    const int32_t* rtok;  // [R]
};

// Weights of one item (RPW rows of gate and of up of the slot's expert).
template <int WT, int LPR, int RPW>
__device__ __forceinline__ void gu_load_w(const ExpertArgs& a, const int4 si, int item, int ips, int sub, int lp,
                                          GuItem<WT, LPR, RPW>& it) {
    constexpr int RPI = 64 / LPR;
    constexpr int NI = RPW / RPI;
    it.e = si.x; it.p0 = si.y; it.nrows = si.z; it.t0 = si.w;
    it.f0 = (item % ips) * RPW;
    const bool sh = it.e >= a.E;
    const uint8_t* gb = sh ? a.w_sh_gate : a.w_gate + (uint64_t)it.e * a.gate_nb2;
    const uint8_t* ub = sh ? a.w_sh_up : a.w_up + (uint64_t)it.e * a.up_nb2;
    const uint64_t gnb1 = sh ? a.sh_gate_nb1 : a.gate_nb1;
    const uint64_t unb1 = sh ? a.sh_up_nb1 : a.up_nb1;
    const int pair = min(lp, (a.H >> 6) - 1);  // lanes past the row re-read the last pair; their sums are dropped
#pragma unroll
    for (int m = 0; m < NI; ++m) {
        const int f = it.f0 + m * RPI + sub;
        it.wg[m].load(gb + (uint64_t)f * gnb1, pair);
        it.wu[m].load(ub + (uint64_t)f * unb1, pair);
    }
}

// Activations of the item's first row (token tok).
template <int WT, int LPR, int RPW>
__device__ __forceinline__ void gu_load_x(const ExpertArgs& a, const XSrc& xs, int tok, int lp,
                                          GuItem<WT, LPR, RPW>& it) {
    it.x.load(xs.qs + (uint64_t)tok * a.H, xs.ds + (uint64_t)tok * (a.H >> 5), min(lp, (a.H >> 6) - 1));
}

template <int WT, int LPR, int RPW>
__device__ __forceinline__ void gu_load(const ExpertArgs& a, const XSrc& xs, const int4* s_slots, int n_act, int item,
                                        int ips, int sub, int lp, GuItem<WT, LPR, RPW>& it) {
    const int4 si = item_slot_info(a, s_slots, item, ips, n_act);
    gu_load_w(a, si, item, ips, sub, lp, it);
    gu_load_x(a, xs, si.w, lp, it);
}

template <int WT, int LPR, int RPW>
__device__ __forceinline__ void gu_compute(const ExpertArgs& a, const XSrc& xs, const GuItem<WT, LPR, RPW>& it,
                                           int sub, int lp) {
    constexpr int RPI = 64 / LPR;
    constexpr int NI = RPW / RPI;
    const bool live = lp < (a.H >> 6);
    XPair x = it.x, xn;
    for (int c = 0; c < it.nrows; ++c) {
        if (c + 1 < it.nrows) {  // the next row's activations, requested before this row's dots
            const int tok = it.e >= a.E ? it.t0 + c + 1 : xs.rtok[it.p0 + c + 1];
            xn.load(xs.qs + (uint64_t)tok * a.H, xs.ds + (uint64_t)tok * (a.H >> 5), min(lp, (a.H >> 6) - 1));
        }
#pragma unroll
        for (int m = 0; m < NI; ++m) {
            double g, u;
            group_sum2_f64<LPR>(live ? pair_dot<WT>(it.wg[m], x) : 0.0, live ? pair_dot<WT>(it.wu[m], x) : 0.0, g, u);
            float2& o = a.gubuf[(uint64_t)(it.p0 + c) * a.F + it.f0 + m * RPI + sub];
            if constexpr (LPR >= 32) {
                if (lp == LPR / 2 - 1) o.x = (float)g;
                if (lp == LPR - 1) o.y = (float)u;
            } else {
                if (lp == LPR - 1) o = make_float2((float)g, (float)u);
            }
        }
        x = xn;
    }
}

// Token rows staged in LDS by the gate/up kernel: at most 32 KiB of quants
// (8 chunks of 16 bytes per thread of a 256-thread block).
constexpr int kGuStageChunks = 8;

// LDS layout of the gate/up kernel: slot table, then (XLDS) the T quantized
// token rows, their scales and the row -> token map.
__host__ __device__ constexpr size_t gu_lds_slots(int E) { return (size_t)(E + 1) * 16; }
__host__ __device__ constexpr size_t gu_lds_bytes(int E, int T, int H, int R, bool xlds) {
    return gu_lds_slots(E) + (xlds ? (size_t)T * H + (size_t)T * (H / 32) * 8 + (size_t)((R + 3) & ~3) * 4 : 0);
}

// Copies n (>= 1) 16-byte chunks global -> LDS with all of a thread's loads
// (at most MAXC) issued before its first store: one memory round trip.  Loads
// past n re-read the last chunk (unconditional loads keep v[] in registers).
template <int MAXC>
__device__ __forceinline__ void stage_chunks(u32x4* dst, const u32x4* src, int n) {
    u32x4 v[MAXC];
#pragma unroll
    for (int u = 0; u < MAXC; ++u) v[u] = src[min((int)threadIdx.x + 256 * u, n - 1)];
#pragma unroll
    for (int u = 0; u < MAXC; ++u) {
        const int i = threadIdx.x + 256 * u;
        if (i < n) dst[i] = v[u];
    }
}

template <int WT, int LPR, int RPW, bool XLDS>
__global__ __launch_bounds__(256) void k_gateup_stream(ExpertArgs a) {
    extern __shared__ __align__(16) uint8_t s_dyn[];
    int4* s_slots = (int4*)s_dyn;
    // routed slots (the table's last slot is the shared expert's, which goes to chunks)
    const int n_act = __builtin_amdgcn_readfirstlane(a.counters[0]) - a.S;
    const int ips = a.F / RPW;
    const int n_items = (n_act + sh_chunks(a)) * ips;
    const int lane = threadIdx.x & 63;
    const int sub = lane / LPR, lp = lane % LPR;
    const int tw = gridDim.x * (blockDim.x >> 6);
    int item = blockIdx.x * (blockDim.x >> 6) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // ping-pong: while one buffer is computed the other one's loads are in flight.  The
    // first two items' weights are requested before the block stages its tables, with
    // their slot entries read from global memory.
    GuItem<WT, LPR, RPW> b0, b1;
    int4 si0 = make_int4(0, 0, 0, 0), si1 = si0;
    if (item < n_items) {
        si0 = item_slot_info(a, a.slot_info, item, ips, n_act);
        gu_load_w(a, si0, item, ips, sub, lp, b0);
        if (item + tw < n_items) {
            si1 = item_slot_info(a, a.slot_info, item + tw, ips, n_act);
            gu_load_w(a, si1, item + tw, ips, sub, lp, b1);
        }
    }
    XSrc xs{a.xq_qs, a.xq_ds, a.row_token};
    if (XLDS) {
        // the T token rows (16-byte chunks), their scales and the row map
        int8_t* lq = (int8_t*)(s_dyn + gu_lds_slots(a.E));
        float2* ld = (float2*)(lq + (size_t)a.T * a.H);
        int32_t* lr = (int32_t*)(ld + (size_t)a.T * (a.H >> 5));
        const int nq = a.T * a.H / 16, nd = a.T * (a.H >> 5) / 2, R = a.offsets[a.E + 1];
        stage_chunks<kGuStageChunks>((u32x4*)lq, (const u32x4*)a.xq_qs, nq);
        stage_chunks<2>((u32x4*)ld, (const u32x4*)a.xq_ds, nd);
        for (int i = threadIdx.x; i < R; i += blockDim.x) lr[i] = a.row_token[i];
        xs = XSrc{lq, ld, lr};
    }
    for (int i = threadIdx.x; i < n_act; i += blockDim.x) s_slots[i] = a.slot_info[i];
    __syncthreads();
    if (item >= n_items) return;
    gu_load_x(a, xs, si0.w, lp, b0);
    if (item + tw < n_items) gu_load_x(a, xs, si1.w, lp, b1);
    for (;;) {
        int nitem = item + tw;
        gu_compute(a, xs, b0, sub, lp);
        if (nitem >= n_items) break;
        item = nitem;
        nitem = item + tw;
        if (nitem < n_items) gu_load(a, xs, s_slots, n_act, nitem, ips, sub, lp, b0);
        gu_compute(a, xs, b1, sub, lp);
        if (nitem >= n_items) break;
        item = nitem;
        nitem = item + tw;
        if (nitem < n_items) gu_load(a, xs, s_slots, n_act, nitem, ips, sub, lp, b1);
    }
}

// ---------------------------------------------------------------------------
// Q: h = silu(g)*u (SwiGLU) or gelu(g)*u (GeGLU) of each (row, ffn index), then Q8_0 quantization of
// the h rows (the activation quantization ggml applies to src1 of the down
// mul_mat_id).  Each lane takes 4 consecutive values; the 8 lanes of a 32-value
// block reduce with DPP (quad xor 1, quad xor 2, half-row mirror) and store
// their quants as one dword each.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_quant_h(ExpertArgs a) {
    const int nrows = a.offsets[a.E + 1];
    const int nq = a.F >> 2;  // quads per row (a multiple of 16: blocks never straddle rows or waves)
    const int gq = blockIdx.x * 256 + threadIdx.x;
    if ((gq & ~63) >= nrows * nq) return;  // whole waves past the end
    const bool live = gq < nrows * nq;     // uniform over each 8-lane block
    const int gqc = live ? gq : 0;
    const int p = gqc / nq, q = gqc - p * nq;
    const f32x4* src = (const f32x4*)(a.gubuf + (uint64_t)p * a.F + 4 * q);
    const f32x4 v0 = src[0], v1 = src[1];  // (g0, u0, g1, u1), (g2, u2, g3, u3)
    float h[4];
    h[0] = act_mul(a.act, a.gelu_tab, v0.x, v0.y);
    h[1] = act_mul(a.act, a.gelu_tab, v0.z, v0.w);
    h[2] = act_mul(a.act, a.gelu_tab, v1.x, v1.y);
    h[3] = act_mul(a.act, a.gelu_tab, v1.z, v1.w);
    float amax = fmaxf(fmaxf(__builtin_fabsf(h[0]), __builtin_fabsf(h[1])),
                       fmaxf(__builtin_fabsf(h[2]), __builtin_fabsf(h[3])));
    amax = dpp8_max<kDppQuadXor1>(amax);
    amax = dpp8_max<kDppQuadXor2>(amax);
    amax = dpp8_max<kDppRowHalfMirror>(amax);
    const float d = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    uint32_t word = 0;
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int qv = (int)__builtin_rintf(h[i] * id);
        sum += qv;
        word |= ((uint32_t)qv & 0xffu) << (8 * i);
    }
    sum = dpp8_add<kDppQuadXor1>(sum);
    sum = dpp8_add<kDppQuadXor2>(sum);
    sum = dpp8_add<kDppRowHalfMirror>(sum);
    if (!live) return;
    *(uint32_t*)(a.hq_qs + (uint64_t)p * a.F + 4 * q) = word;
    if ((q & 7) == 0)
        a.hq_ds[(uint64_t)p * (a.F >> 5) + (q >> 3)] = make_float2(fp16_to_f32(f32_to_fp16(d)), __builtin_bit_cast(float, sum));
}

// ---------------------------------------------------------------------------
// G1+Q at decode sizes: gate/up, SwiGLU and the Q8_0 quantization of h of the
// routed experts in one launch (the decode routing launch does the shared
// expert's).  Block = (slot v of the decode slot list, 32 consecutive ffn rows:
// one Q8_0 block of h per token row); NW waves of 32/NW rows of gate and of up.
// The block stages its slot's token rows (Q8_0 of x) in LDS -- loads issued
// before the weight loads, so they land first -- computes g and u for every
// row into LDS, then one lane per value does h = silu(g)*u and 32 lanes
// quantize a row's block: the same operations as k_quant_h, so the same bits.
// ---------------------------------------------------------------------------

#ifndef GQ_Q4_WAVES
#define GQ_Q4_WAVES 8
#endif
#ifndef GQ_MIN_WAVES
#define GQ_MIN_WAVES 1
#endif
template <int WT> constexpr int kGqWaves = GQ_Q4_WAVES;  // waves per block (rows per wave: 32 / waves)
template <> constexpr int kGqWaves<kTypeQ8_0> = 8;

__host__ __device__ constexpr size_t gq_lds_bytes(int T, int H) { return (size_t)T * H + (size_t)T * (H / 32) * 8; }

// The shared expert's down projection in the fused decode gate/up launch (its h
// rows were written by the routing launch): ysh[t][n] = the dot of down row n
// with token t's Q8_0 h over 8 lanes of one block pair each (F = 512) and the
// same f64 tree as the down+combine kernel's shared step, so the same f32 value.
// Wave gw of these workgroups takes the 8 rows of group gw / kSdSplit and the
// tokens t = gw (mod kSdSplit), two tokens' h rows in flight.
constexpr int kSdLanes = 8;
constexpr int kSdSplit = 2;
template <int WT, int NW>
__device__ void gu_shared_down(const ExpertArgs& a, int j) {
#pragma clang fp contract(off)
    constexpr int RPI = 64 / kSdLanes;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane / kSdLanes, lp = lane % kSdLanes;
    const int gw = j * NW + wave;
    const int g = gw / kSdSplit;
    if (g >= a.H / RPI) return;
    const int n = g * RPI + sub;
    WPair<WT> w;
    w.load(a.w_sh_down + (uint64_t)n * a.sh_down_nb1, lp);
    const int nfb = a.F >> 5;
    for (int t = gw % kSdSplit; t < a.T; t += 2 * kSdSplit) {
        const uint64_t p0 = (uint64_t)a.T * a.K + t, p1 = p0 + kSdSplit;  // the shared expert's h rows
        const bool has1 = t + kSdSplit < a.T;
        XPair x0, x1;
        x0.load(a.hq_qs + p0 * a.F, a.hq_ds + p0 * nfb, lp);
        if (has1) x1.load(a.hq_qs + p1 * a.F, a.hq_ds + p1 * nfb, lp);
        const double y0 = dpp_sum_f64<kSdLanes>(pair_dot<WT>(w, x0));
        if (lp == kSdLanes - 1) a.ysh[(uint64_t)t * a.H + n] = (float)y0;
        if (has1) {
            const double y1 = dpp_sum_f64<kSdLanes>(pair_dot<WT>(w, x1));
            if (lp == kSdLanes - 1) a.ysh[(uint64_t)(t + kSdSplit) * a.H + n] = (float)y1;
        }
    }
}

// PPL: Q8_0 block pairs per lane of a row (pairs lp, lp + LPR, ...): LPR * PPL >= H / 64.
// Each pair's contribution is exact in f64, so any split sums to the same bits.
template <int WT, int LPR, int NW, int PPL>
__global__ __launch_bounds__(NW * 64, GQ_MIN_WAVES) void k_gateup_q(ExpertArgs a, const int4* dslots) {
#pragma clang fp contract(off)
    constexpr int RPI = 64 / LPR;
    constexpr int RPW = 32 / NW;  // ffn rows per wave
    constexpr int NI = RPW / RPI;
    constexpr int NT = NW * 64;
    static_assert(NI >= 1 && NI * RPI == RPW, "rows per wave");
    extern __shared__ __align__(16) uint8_t s_dyn[];
    __shared__ float2 s_gu[kTopkTokensPerBlock][32];
    if ((int)blockIdx.x < a.sd_blocks) {  // dispatched first: no dependence on the slot list
        gu_shared_down<WT, NW>(a, blockIdx.x);
        return;
    }
    const int bid = (int)blockIdx.x - a.sd_blocks;
    const int nfb = a.F >> 5;
    const int v = bid / nfb;
    const int fb = bid - v * nfb;
    const int4 si = dslots[v];
    if (si.x < 0) return;  // past the forward's active slots (whole block)
    const int e = si.x, p0 = si.y, nrows = si.z;
    const uint32_t mask = (uint32_t)si.w;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int sub = lane / LPR, lp = lane % LPR;
    // lanes past the row re-read the last pair; their sums are dropped
    int pairk[PPL];
    bool livek[PPL];
#pragma unroll
    for (int k = 0; k < PPL; ++k) {
        livek[k] = lp + k * LPR < (a.H >> 6);
        pairk[k] = min(lp + k * LPR, (a.H >> 6) - 1);
    }
    // token rows of the slot -> LDS: quants [nrows][H], then {d, sum} [nrows][H/32]
    int8_t* lq = (int8_t*)s_dyn;
    float2* ld = (float2*)(lq + (size_t)nrows * a.H);
    const int cq = a.H >> 4, cpr = cq + (a.H >> 6);  // 16-byte chunks per row
    const int nc = nrows * cpr;
    constexpr int kStage = 2;  // chunks per thread per round (a round covers 2 rows at H = 2048)
    u32x4 xv[kStage];
    u32x4* xdst[kStage];
    auto stage_load = [&](int base) {
#pragma unroll
        for (int u = 0; u < kStage; ++u) {
            const int i = min(base + NT * u + tid, nc - 1);
            const int c = i / cpr, k = i - c * cpr;
            uint32_t m = mask;  // token of row c: the c-th set bit
            for (int b = 0; b < c; ++b) m &= m - 1u;
            const int tok = __builtin_ctz(m);
            const bool q = k < cq;
            const u32x4* src = q ? (const u32x4*)(a.xq_qs + (uint64_t)tok * a.H) + k
                                 : (const u32x4*)(a.xq_ds + (uint64_t)tok * (a.H >> 5)) + (k - cq);
            xv[u] = *src;
            xdst[u] = q ? (u32x4*)(lq + (size_t)c * a.H) + k : (u32x4*)(ld + (size_t)c * (a.H >> 5)) + (k - cq);
        }
    };
    auto stage_store = [&](int base) {
#pragma unroll
        for (int u = 0; u < kStage; ++u)
            if (base + NT * u + tid < nc) *xdst[u] = xv[u];
    };
    stage_load(0);
    // weights: rows fb*32 + wave*4 + m*RPI + sub of gate and up
    const bool sh = e >= a.E;
    const uint8_t* gb = sh ? a.w_sh_gate : a.w_gate + (uint64_t)e * a.gate_nb2;
    const uint8_t* ub = sh ? a.w_sh_up : a.w_up + (uint64_t)e * a.up_nb2;
    const uint64_t gnb1 = sh ? a.sh_gate_nb1 : a.gate_nb1;
    const uint64_t unb1 = sh ? a.sh_up_nb1 : a.up_nb1;
    const int fw = fb * 32 + wave * RPW;
    WPair<WT> wg[NI][PPL], wu[NI][PPL];
#pragma unroll
    for (int m = 0; m < NI; ++m) {
        const int f = fw + m * RPI + sub;
#pragma unroll
        for (int k = 0; k < PPL; ++k) {
            wg[m][k].load(gb + (uint64_t)f * gnb1, pairk[k]);
            wu[m][k].load(ub + (uint64_t)f * unb1, pairk[k]);
        }
    }
    stage_store(0);
    for (int base = kStage * NT; base < nc; base += kStage * NT) {  // rows past the first round
        stage_load(base);
        stage_store(base);
    }
    __syncthreads();
    for (int c = 0; c < nrows; ++c) {
        // unpack the weights per row: hoisting the unpacked nibbles out of the
        // loop costs registers (residency) that single-row slots never repay
#pragma unroll
        for (int m = 0; m < NI; ++m) {
#pragma unroll
            for (int k = 0; k < PPL; ++k) {
#pragma unroll
                for (int i = 0; i < (int)(sizeof(wg[m][k].w) / 4); ++i) {
                    asm volatile("" : "+v"(wg[m][k].w[i]));
                    asm volatile("" : "+v"(wu[m][k].w[i]));
                }
            }
        }
        // activations stream through 4 registers, one 16-byte chunk at a time,
        // re-read from LDS for each row group so its weights die after use
#pragma unroll
        for (int m = 0; m < NI; ++m) {
            double pg = 0.0, pu = 0.0;
#pragma unroll
            for (int k = 0; k < PPL; ++k) {
                const u32x4* xq = (const u32x4*)(lq + (size_t)c * a.H + 64 * pairk[k]);
                const u32x4 xd = *(const u32x4*)(ld + (size_t)c * (a.H >> 5) + 2 * pairk[k]);  // {dA, sumA, dB, sumB}
                const int za = -WPair<WT>::kZero * (int)xd.y, zb = -WPair<WT>::kZero * (int)xd.w;
                const float dxa = __builtin_bit_cast(float, (uint32_t)xd.x), dxb = __builtin_bit_cast(float, (uint32_t)xd.z);
                const WPair<WT>& g = wg[m][k];
                const WPair<WT>& u = wu[m][k];
                u32x4 xc = xq[0];
                int ga = g.template dot_chunk<0>(xc, za), ua = u.template dot_chunk<0>(xc, za);
                xc = xq[1];
                ga = g.template dot_chunk<1>(xc, ga); ua = u.template dot_chunk<1>(xc, ua);
                xc = xq[2];
                int gbs = g.template dot_chunk<2>(xc, zb), ubs = u.template dot_chunk<2>(xc, zb);
                xc = xq[3];
                gbs = g.template dot_chunk<3>(xc, gbs); ubs = u.template dot_chunk<3>(xc, ubs);
                const double tg = __builtin_fma((double)(g.dA() * dxa), (double)ga, (double)(g.dB() * dxb) * (double)gbs);
                const double tu = __builtin_fma((double)(u.dA() * dxa), (double)ua, (double)(u.dB() * dxb) * (double)ubs);
                if (k == 0) {  // dead lanes contribute +0.0, as a single-pair lane always did
                    pg = livek[0] ? tg : 0.0;
                    pu = livek[0] ? tu : 0.0;
                } else if (livek[k]) {
                    pg = pg + tg;
                    pu = pu + tu;
                }
            }
            double gs, us;
            group_sum2_f64<LPR>(pg, pu, gs, us);
            float2& o = s_gu[c][wave * RPW + m * RPI + sub];
            if constexpr (LPR >= 32) {
                if (lp == LPR / 2 - 1) o.x = (float)gs;
                if (lp == LPR - 1) o.y = (float)us;
            } else {
                if (lp == LPR - 1) o = make_float2((float)gs, (float)us);
            }
        }
    }
    __syncthreads();
    for (int i = tid; i < nrows * 32; i += NT) {  // whole 32-lane groups: row c = i / 32, value fl
        const int c = i >> 5, fl = i & 31;
        const float2 gu = s_gu[c][fl];
        const int p = p0 + c;
        swiglu_q8_block32(gu.x, gu.y, fl, a.hq_qs + (uint64_t)p * a.F + fb * 32, a.hq_ds + (uint64_t)p * nfb + fb,
                          a.act, a.gelu_tab);
    }
}

// ---------------------------------------------------------------------------
// G2: down projection, persistent streaming.  Work item = (active slot, group
// of RPW consecutive output rows n).  LPR lanes per F row.  Writes ybuf[p][n].
// ---------------------------------------------------------------------------
template <int WT, int LPR, int RPW>
struct DnItem {
    static constexpr int RPI = 64 / LPR;
    static constexpr int NI = RPW / RPI;
    WPair<WT> w[NI];
    XPair x;
    int e, p0, nrows, n0, t0;  // t0: the shared expert's first token
};

template <int WT, int LPR, int RPW>
__device__ __forceinline__ void dn_load(const ExpertArgs& a, const XSrc& hs, const int4* s_slots, int item, int ips,
                                        int sub, int lp, int n_act, DnItem<WT, LPR, RPW>& it) {
    constexpr int RPI = 64 / LPR;
    constexpr int NI = RPW / RPI;
    const int4 si = item_slot_info(a, s_slots, item, ips, n_act);
    it.e = si.x; it.p0 = si.y; it.nrows = si.z; it.t0 = si.w;
    it.n0 = (item % ips) * RPW;
    const bool sh = it.e >= a.E;
    const uint8_t* db = sh ? a.w_sh_down : a.w_down + (uint64_t)it.e * a.down_nb2;
    const uint64_t dnb1 = sh ? a.sh_down_nb1 : a.down_nb1;
    const int pair = min(lp, (a.F >> 6) - 1);
#pragma unroll
    for (int m = 0; m < NI; ++m) it.w[m].load(db + (uint64_t)(it.n0 + m * RPI + sub) * dnb1, pair);
    if (sh && hs.qs) it.x.load(hs.qs + (uint64_t)it.t0 * a.F, hs.ds + (uint64_t)it.t0 * (a.F >> 5), pair);  // uniform branches keep the address spaces known
    else it.x.load(a.hq_qs + (uint64_t)it.p0 * a.F, a.hq_ds + (uint64_t)it.p0 * (a.F >> 5), pair);
}

template <int WT, int LPR, int RPW>
__device__ __forceinline__ void dn_compute(const ExpertArgs& a, const XSrc& hs, const DnItem<WT, LPR, RPW>& it,
                                           int sub, int lp) {
    constexpr int RPI = 64 / LPR;
    constexpr int NI = RPW / RPI;
    const bool live = lp < (a.F >> 6);
    const bool sh = it.e >= a.E;
    XPair x = it.x, xn;
    for (int c = 0; c < it.nrows; ++c) {
        const int p = it.p0 + c;
        if (c + 1 < it.nrows) {
            // the next row, requested before this row's dots: shared-expert rows from
            // the block's LDS copy (hs), routed rows from global memory
            const int pair = min(lp, (a.F >> 6) - 1);
            const int tn = it.t0 + c + 1;
            if (sh && hs.qs) xn.load(hs.qs + (uint64_t)tn * a.F, hs.ds + (uint64_t)tn * (a.F >> 5), pair);
            else xn.load(a.hq_qs + (uint64_t)(p + 1) * a.F, a.hq_ds + (uint64_t)(p + 1) * (a.F >> 5), pair);
        }
#pragma unroll
        for (int m = 0; m < NI; ++m) {
            const double y = dpp_sum_f64<LPR>(live ? pair_dot<WT>(it.w[m], x) : 0.0);
            if (lp == LPR - 1) a.ybuf[(uint64_t)p * a.H + it.n0 + m * RPI + sub] = (float)y;
        }
        x = xn;
    }
}

// LDS of the down kernel: slot table, then (SHLDS) the shared expert's T rows
// of quantized h (the slot with the most rows at decode sizes).
__host__ __device__ constexpr size_t dn_lds_bytes(int E, int T, int F, bool shlds) {
    return (size_t)(E + 1) * 16 + (shlds ? (size_t)T * F + (size_t)T * (F / 32) * 8 : 0);
}

template <int WT, int LPR, int RPW, bool SHLDS>
__global__ __launch_bounds__(256) void k_down_stream(ExpertArgs a) {
    extern __shared__ __align__(16) uint8_t s_dyn[];
    __shared__ int s_nact;
    int4* s_slots = (int4*)s_dyn;
    XSrc hs{nullptr, nullptr, nullptr};
    if (SHLDS) {
        int8_t* lq = (int8_t*)(s_dyn + (size_t)(a.E + 1) * 16);
        float2* ld = (float2*)(lq + (size_t)a.T * a.F);
        const int A = a.T * a.K;  // the shared rows follow the T*K routed rows
        const int nq = a.T * a.F / 16, nd = a.T * (a.F >> 5) / 2;
        const u32x4* gq = (const u32x4*)(a.hq_qs + (uint64_t)A * a.F);
        const u32x4* gd = (const u32x4*)(a.hq_ds + (uint64_t)A * (a.F >> 5));
        for (int i = threadIdx.x; i < nq; i += blockDim.x) ((u32x4*)lq)[i] = gq[i];
        for (int i = threadIdx.x; i < nd; i += blockDim.x) ((u32x4*)ld)[i] = gd[i];
        hs = XSrc{lq, ld, nullptr};
    }
    const int n_act = stage_slots(a, s_slots, &s_nact) - a.S;  // routed slots; the shared expert goes to chunks
    const int ips = a.H / RPW;
    const int n_items = (n_act + sh_chunks(a)) * ips;
    const int lane = threadIdx.x & 63;
    const int sub = lane / LPR, lp = lane % LPR;
    const int tw = gridDim.x * (blockDim.x >> 6);
    int item = blockIdx.x * (blockDim.x >> 6) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (item >= n_items) return;
    DnItem<WT, LPR, RPW> b0, b1;
    dn_load(a, hs, s_slots, item, ips, sub, lp, n_act, b0);
    for (;;) {
        int nitem = item + tw;
        if (nitem < n_items) dn_load(a, hs, s_slots, nitem, ips, sub, lp, n_act, b1);
        dn_compute(a, hs, b0, sub, lp);
        if (nitem >= n_items) break;
        item = nitem;
        nitem = item + tw;
        if (nitem < n_items) dn_load(a, hs, s_slots, nitem, ips, sub, lp, n_act, b0);
        dn_compute(a, hs, b1, sub, lp);
        if (nitem >= n_items) break;
        item = nitem;
    }
}

// ---------------------------------------------------------------------------
// G2+G3 at decode sizes (T <= kTopkTokensPerBlock, K + S <= kDcMaxSteps):
// token-major down projection with the combine in its epilogue.  Work item =
// (token t, RPI consecutive output rows n); a wave walks t's selected experts
// in slot order j = 0..K-1, then the shared expert, and accumulates
//     acc = w_0*y_0;  acc = acc + w_j*y_j;  acc = acc + y_sh*sigma_t;  (+ residual)
// in f32, each product and sum separately rounded -- the combine of
// moe.cpp:134-151,169-174, in the same order as k_combine, so the outputs are
// the same bits.  Each step's weights (RPI rows of W_down[e_j]) and activation
// row (Q8_0 of h for assignment (t, j)) are loaded kDcAhead steps ahead.  An
// expert used by several tokens (the shared one by all) is read once per
// token; those repeats hit the L2.
// ---------------------------------------------------------------------------
constexpr int kDcMaxSteps = 16;

struct DownCombineArgs {
    int H, F, E, K, S, T;
    const uint8_t* w_down; uint64_t down_nb1, down_nb2;
    const uint8_t* w_sh_down; uint64_t sh_down_nb1;
    const int32_t* topk_idx; const float* topk_w; const int32_t* pos; const float* sh_gate;
    const int8_t* hq_qs; const float2* hq_ds;
    const float* residual; float* y;
    const float* ysh;  // [T][H] the shared expert's down rows, computed by the gate/up launch (or null)
    double* y_ssq;     // [T][ssq_parts(H)] y's RMSNorm partial sums (token-per-block kernel, LPR <= 8), or null
};

template <int WT>
struct DcStep {
    WPair<WT> w;
    XPair x;
};

// Step tables of the block's tokens: expert (E = shared), activation row and
// combine weight (sigma_t for the shared step) of step j of token t.
struct DcTables {
    int32_t e[kTopkTokensPerBlock][kDcMaxSteps];
    int32_t p[kTopkTokensPerBlock][kDcMaxSteps];
    float w[kTopkTokensPerBlock][kDcMaxSteps];
};

__device__ __forceinline__ void dc_fill_tables(const DownCombineArgs& a, DcTables& s, int t_lo, int t_hi) {
    const int nj = a.K + a.S;
    const int A = a.T * a.K;
    for (int i = threadIdx.x; i < (t_hi - t_lo) * nj; i += blockDim.x) {
        const int t = t_lo + i / nj, j = i % nj;
        const bool routed = j < a.K;
        s.e[t][j] = routed ? a.topk_idx[t * a.K + j] : a.E;
        s.p[t][j] = routed ? a.pos[t * a.K + j] : A + t;
        s.w[t][j] = routed ? a.topk_w[t * a.K + j] : a.sh_gate[t];
    }
}

// Combine order of the reference's ggml graph: w_0*y_0, then + w_j*y_j, then + y_sh*sigma_t.
__device__ __forceinline__ void dc_combine(float& acc, int j, int K, float wj, double yd) {
#pragma clang fp contract(off)
    const float yv = (float)yd;
    if (j == 0) acc = wj * yv;
    else if (j < K) acc = acc + wj * yv;
    else acc = acc + yv * wj;
}

template <int WT, int LPR, int kDcAhead>  // kDcAhead: steps whose loads are in flight
__global__ __launch_bounds__(256) void k_down_combine(DownCombineArgs a) {
#pragma clang fp contract(off)
    constexpr int RPI = 64 / LPR;
    __shared__ DcTables s;
    dc_fill_tables(a, s, 0, a.T);
    __syncthreads();
    const int nj = a.K + a.S;
    const int lane = threadIdx.x & 63;
    const int sub = lane / LPR, lp = lane % LPR;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int n_items = a.T * (a.H / RPI);
    if (item >= n_items) return;
    const int t = item % a.T;          // tokens fastest: neighbouring waves share experts' rows in L2
    const int n = (item / a.T) * RPI + sub;
    const int pair = min(lp, (a.F >> 6) - 1);
    const bool live = lp < (a.F >> 6);
    auto load = [&](int j, DcStep<WT>& st) {
        const int e = s.e[t][j];
        const uint8_t* row = e >= a.E ? a.w_sh_down + (uint64_t)n * a.sh_down_nb1
                                      : a.w_down + (uint64_t)e * a.down_nb2 + (uint64_t)n * a.down_nb1;
        st.w.load(row, pair);
        const int p = s.p[t][j];
        st.x.load(a.hq_qs + (uint64_t)p * a.F, a.hq_ds + (uint64_t)p * (a.F >> 5), pair);
    };
    DcStep<WT> buf[kDcAhead];
#pragma unroll
    for (int j = 0; j < kDcAhead; ++j)
        if (j < nj) load(j, buf[j]);
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < kDcMaxSteps; ++j) {
        if (j < nj) {
            const double yd = dpp_sum_f64<LPR>(live ? pair_dot<WT>(buf[j % kDcAhead].w, buf[j % kDcAhead].x) : 0.0);
            if (j + kDcAhead < nj) load(j + kDcAhead, buf[j % kDcAhead]);
            dc_combine(acc, j, a.K, s.w[t][j], yd);
        }
    }
    if (lp == LPR - 1) {
        if (a.residual) acc = acc + a.residual[(uint64_t)t * a.H + n];
        a.y[(uint64_t)t * a.H + n] = acc;
    }
}

// Token-per-block variant: the block's 4 waves take 4*RPI consecutive output
// rows of one token, whose nj (<= NJ) activation rows (Q8_0 h: quants, then
// {scale, sum} pairs) are staged once in LDS.  Loads are issued in the order
// they are consumed -- the staging chunks (MAXC per thread), then every step's
// weight pair -- so step j computes while the later steps' weights arrive.
__host__ __device__ constexpr size_t dc_lds_bytes(int F, int nj) {
    return (size_t)nj * F + (size_t)nj * (F / 32) * 8;
}
__host__ __device__ constexpr int dc_stage_chunks(int F, int nj) { return nj * (F / 16 + F / 64); }

template <int WT, int LPR, int NJ, int MAXC>
__global__ __launch_bounds__(256) void k_down_combine_tok(DownCombineArgs a) {
#pragma clang fp contract(off)
    constexpr int RPI = 64 / LPR;
    extern __shared__ __align__(16) uint8_t s_dyn[];
    // Workgroups are dealt round-robin to the 8 XCDs (block b to XCD b % 8), each
    // with its own L2.  Logical block g = (b % 8) * (G / 8) + b / 8 gives every
    // XCD a contiguous run of row groups with all their tokens, dispatched
    // together: the tokens of a row group read the same expert rows (shared
    // expert always, routed experts often) through one L2.
    const int G = gridDim.x;
    const int b = blockIdx.x;
    const int g = (G & 7) == 0 ? (b & 7) * (G >> 3) + (b >> 3) : b;
    const int rg = g / a.T;
    const int t = g - rg * a.T;  // tokens fastest within an XCD's run
    const int nj = a.K + (a.ysh ? 0 : a.S);  // steps with weights here (the shared one may come precomputed)
    // the token's steps (wave-uniform: scalar loads); steps past nj repeat the last one
    int se[NJ], sp[NJ];
    float sw[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int jj = min(j, nj - 1);
        const bool routed = jj < a.K;
        se[j] = routed ? a.topk_idx[t * a.K + jj] : a.E;
        sp[j] = routed ? a.pos[t * a.K + jj] : a.T * a.K + t;
        sw[j] = routed ? a.topk_w[t * a.K + jj] : a.sh_gate[t];
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane / LPR, lp = lane % LPR;
    const int n_raw = (rg * 4 + wave) * RPI + sub;
    const int n = min(n_raw, a.H - 1);
    const int pair = min(lp, (a.F >> 6) - 1);
    const bool live = lp < (a.F >> 6);
    const float ysh = a.ysh ? a.ysh[(uint64_t)t * a.H + n] : 0.0f;
    // staging loads (chunks past nc re-read the last one; only chunks < nc are stored)
    int8_t* lq = (int8_t*)s_dyn;
    float2* ld = (float2*)(lq + (size_t)nj * a.F);
    const int qc = a.F >> 4, dc = a.F >> 6;  // 16-byte chunks per row: quants, {scale, sum} pairs
    const int nc = nj * (qc + dc);
    u32x4 v[MAXC];
    u32x4* dst[MAXC];
#pragma unroll
    for (int u = 0; u < MAXC; ++u) {
        const int i = min((int)threadIdx.x + 256 * u, nc - 1);
        const int j = i / (qc + dc), c = i - j * (qc + dc);
        int p = sp[0];
#pragma unroll
        for (int k = 1; k < NJ; ++k) p = j == k ? sp[k] : p;
        const bool q = c < qc;
        const u32x4* src = q ? (const u32x4*)(a.hq_qs + (uint64_t)p * a.F) + c
                             : (const u32x4*)(a.hq_ds + (uint64_t)p * (a.F >> 5)) + (c - qc);
        v[u] = *src;
        dst[u] = q ? (u32x4*)(lq + (size_t)j * a.F) + c : (u32x4*)(ld + (size_t)j * (a.F >> 5)) + (c - qc);
    }
    WPair<WT> w[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const uint8_t* row = se[j] >= a.E ? a.w_sh_down + (uint64_t)n * a.sh_down_nb1
                                          : a.w_down + (uint64_t)se[j] * a.down_nb2 + (uint64_t)n * a.down_nb1;
        w[j].load(row, pair);
    }
#pragma unroll
    for (int u = 0; u < MAXC; ++u)
        if ((int)threadIdx.x + 256 * u < nc) *dst[u] = v[u];
    __syncthreads();
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        if (j < nj) {
            XPair x;
            x.load(lq + (size_t)j * a.F, ld + (size_t)j * (a.F >> 5), pair);
            dc_combine(acc, j, a.K, sw[j], dpp_sum_f64<LPR>(live ? pair_dot<WT>(w[j], x) : 0.0));
        }
    }
    if (a.ysh) acc = acc + ysh * a.sh_gate[t];  // the shared step, last (as dc_combine orders it)
    if (lp == LPR - 1 && n_raw < a.H) {
        if (a.residual) acc = acc + a.residual[(uint64_t)t * a.H + n];
        a.y[(uint64_t)t * a.H + n] = acc;
    }
    if constexpr (LPR <= 8) {
        // y's RMSNorm partial sums: the block's 4 RPI rows are RPI runs of four,
        // RPI / 8 whole entries (run sums in row order, then the 8-lane trees)
        if (a.y_ssq) {  // uniform
            __shared__ float s_y[4 * RPI];
            if (lp == LPR - 1) s_y[wave * RPI + sub] = acc;
            __syncthreads();
            if (wave == 0) {
                const int r0 = rg * 4 * RPI + 4 * lane;  // first row of run `lane`
                double s = 0.0;
                if (lane < RPI)
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        if (r0 + k < a.H) s += (double)(s_y[4 * lane + k] * s_y[4 * lane + k]);
                s = dpp_sum_f64<8>(s);
                const int np = ssq_parts(a.H);
                const int c = rg * (RPI / 8) + (lane >> 3);
                if (lane < RPI && (lane & 7) == 7 && c < np) a.y_ssq[(uint64_t)t * np + c] = s;
            }
        }
    }
}

bool shared_down_in_gateup(const LayerDesc& L, int T) {
    return L.S && gateup_q_fused(L, T) && L.F == 64 * kSdLanes && L.dn_type == L.gu_type && down_combine_tok_fits(L);
}

bool down_combine_tok_fits(const LayerDesc& L) {
    const int nj = L.K + L.S;
    return nj <= 9 && dc_lds_bytes(L.F, nj) <= 64 * 1024 && dc_stage_chunks(L.F, nj) <= 1024 && L.dc_ahead <= 2;
}

// Up to 16 tokens either down+combine kernel; beyond, below the MFMA path, the
// token-per-workgroup one (its step tables are per token; measured faster than
// the streaming down + k_combine from 24 to 127 tokens: 99 -> 86 us at 24 tokens,
// 156 -> 146 at 64, 221 -> 215 at 127).
bool down_combine_fused(const LayerDesc& L, int T) {
    return T < L.mfma_min_tokens && L.K + L.S <= kDcMaxSteps &&
           (T <= kTopkTokensPerBlock || down_combine_tok_fits(L));
}

// Up to 9 steps (8 routed + shared) whose activation rows fit in 64 KiB of
// LDS and 1024 staging chunks: the token-per-block kernel (9 Q4_0 weight pairs
// are 81 VGPRs).  Otherwise steps stream with `ahead` (2 or 4) in flight.
template <int WT, int LPR>
static hipError_t launch_down_combine_v(const DownCombineArgs& a, int ahead, hipStream_t stream) {
    constexpr int RPI = 64 / LPR;
    const int nj = a.K + (a.ysh ? 0 : a.S);
    const int nc = dc_stage_chunks(a.F, nj);
    if (nj <= 9 && dc_lds_bytes(a.F, nj) <= 64 * 1024 && nc <= 1024 && ahead <= 2) {
        const dim3 g(a.T * ((a.H + 4 * RPI - 1) / (4 * RPI))), b(256);
        const size_t lds = dc_lds_bytes(a.F, nj);
        // 8 steps (top-8 with the shared row precomputed): no ninth weight pair in registers
        if (nj <= 8 && nc <= 512) hipLaunchKernelGGL((k_down_combine_tok<WT, LPR, 8, 2>), g, b, lds, stream, a);
        else if (nc <= 512) hipLaunchKernelGGL((k_down_combine_tok<WT, LPR, 9, 2>), g, b, lds, stream, a);
        else hipLaunchKernelGGL((k_down_combine_tok<WT, LPR, 9, 4>), g, b, lds, stream, a);
        return hipGetLastError();
    }
    if (a.ysh) return hipErrorInvalidValue;  // only the token-per-workgroup kernel takes a precomputed shared step
    const int n_items = a.T * (a.H / RPI);
    const dim3 g((n_items + 3) / 4), b(256);
    if (ahead <= 2) hipLaunchKernelGGL((k_down_combine<WT, LPR, 2>), g, b, 0, stream, a);
    else hipLaunchKernelGGL((k_down_combine<WT, LPR, 4>), g, b, 0, stream, a);
    return hipGetLastError();
}

template <int WT>
static hipError_t launch_down_combine_t(const DownCombineArgs& a, int ahead, hipStream_t stream) {
    const int npairs = a.F / 64;
    if (npairs <= 4) return launch_down_combine_v<WT, 4>(a, ahead, stream);
    if (npairs <= 8) return launch_down_combine_v<WT, 8>(a, ahead, stream);
    if (npairs <= 16) return launch_down_combine_v<WT, 16>(a, ahead, stream);
    if (npairs <= 32) return launch_down_combine_v<WT, 32>(a, ahead, stream);
    return launch_down_combine_v<WT, 64>(a, ahead, stream);
}

hipError_t launch_down_combine(const LayerDesc& L, const Workspace& ws, int T, float* y, const float* residual,
                               hipStream_t stream, double* y_ssq, bool* ssq_done) {
    DownCombineArgs a;
    a.H = L.H; a.F = L.F; a.E = L.E; a.K = L.K; a.S = L.S; a.T = T;
    a.w_down = L.w_down; a.down_nb1 = L.down_nb1; a.down_nb2 = L.down_nb2;
    a.w_sh_down = L.w_sh_down; a.sh_down_nb1 = L.sh_down_nb1;
    a.topk_idx = ws.topk_idx; a.topk_w = ws.topk_w; a.pos = ws.pos; a.sh_gate = ws.sh_gate;
    a.hq_qs = ws.hq_qs; a.hq_ds = ws.hq_ds;
    a.residual = residual; a.y = y;
    a.ysh = shared_down_in_gateup(L, T) ? ws.ysh : nullptr;
    // the token-per-block kernel with whole entries per block (LPR <= 8: F <= 512)
    const bool ssq = y_ssq && down_combine_tok_fits(L) && L.F <= 512 && L.H % kSsqCols == 0;
    a.y_ssq = ssq ? y_ssq : nullptr;
    if (ssq_done) *ssq_done = ssq;
    return (L.dn_type == kTypeQ4_0) ? launch_down_combine_t<kTypeQ4_0>(a, L.dc_ahead, stream)
                                    : launch_down_combine_t<kTypeQ8_0>(a, L.dc_ahead, stream);
}

// Persistent grid: every block resident at once (blocks per CU from the
// occupancy calculator), never more waves than items.
template <typename KernelT>
static int stream_blocks(KernelT kernel, size_t lds, int n_items_max, int n_cu) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 256, lds) != hipSuccess || per_cu < 1) per_cu = 1;
    const int want = (n_items_max + 3) / 4;
    return std::max(1, std::min(want, n_cu * per_cu));
}

// Token rows are staged in LDS when they take at most this many bytes per block.
constexpr size_t kGuXLdsMax = 32 * 1024;

template <int WT, int LPR, int RPW>
static hipError_t launch_gateup_v(const ExpertArgs& a, int max_slots, int n_cu, hipStream_t stream, hipEvent_t e0,
                                  hipEvent_t e1) {
    const int R = a.T * a.K + a.S * a.T;
    const bool xlds = gu_lds_bytes(a.E, a.T, a.H, R, true) - gu_lds_slots(a.E) <= kGuXLdsMax;
    const size_t lds = gu_lds_bytes(a.E, a.T, a.H, R, xlds);
    if (xlds) {
        auto kern = k_gateup_stream<WT, LPR, RPW, true>;
        const int g = stream_blocks(kern, lds, max_slots * (a.F / RPW), n_cu);
        launch_timed(kern, dim3(g), dim3(256), lds, stream, e0, e1, a);
    } else {
        auto kern = k_gateup_stream<WT, LPR, RPW, false>;
        const int g = stream_blocks(kern, lds, max_slots * (a.F / RPW), n_cu);
        launch_timed(kern, dim3(g), dim3(256), lds, stream, e0, e1, a);
    }
    return hipGetLastError();
}

template <int WT>
static hipError_t launch_gateup(const ExpertArgs& a, int max_slots, int n_cu, hipStream_t stream, hipEvent_t e0,
                                hipEvent_t e1) {
    const int npairs = a.H / 64;
    if (npairs <= 16) return launch_gateup_v<WT, 16, 4>(a, max_slots, n_cu, stream, e0, e1);
    if (npairs <= 32) return launch_gateup_v<WT, 32, 4>(a, max_slots, n_cu, stream, e0, e1);  // 4 rows: twice the bytes per request (2 rows: +14%, 8 rows: +19% at 64 tokens)
    return launch_gateup_v<WT, 64, 2>(a, max_slots, n_cu, stream, e0, e1);
}

template <int WT, int LPR>
static hipError_t launch_down_v(const ExpertArgs& a, int max_slots, int n_cu, hipStream_t stream) {
    constexpr int RPW = 4 * (64 / LPR);  // four load instructions per item (at 64 tokens: two +8%, one +40%, eight +25%)
    const bool shlds = a.S && dn_lds_bytes(a.E, a.T, a.F, true) - dn_lds_bytes(a.E, a.T, a.F, false) <= kGuXLdsMax;
    const size_t lds = dn_lds_bytes(a.E, a.T, a.F, shlds);
    if (shlds) {
        auto kern = k_down_stream<WT, LPR, RPW, true>;
        const int g = stream_blocks(kern, lds, max_slots * (a.H / RPW), n_cu);
        hipLaunchKernelGGL(kern, dim3(g), dim3(256), lds, stream, a);
    } else {
        auto kern = k_down_stream<WT, LPR, RPW, false>;
        const int g = stream_blocks(kern, lds, max_slots * (a.H / RPW), n_cu);
        hipLaunchKernelGGL(kern, dim3(g), dim3(256), lds, stream, a);
    }
    return hipGetLastError();
}

template <int WT>
static hipError_t launch_down(const ExpertArgs& a, int max_slots, int n_cu, hipStream_t stream) {
    const int npairs = a.F / 64;
    if (npairs <= 4) return launch_down_v<WT, 4>(a, max_slots, n_cu, stream);
    if (npairs <= 8) return launch_down_v<WT, 8>(a, max_slots, n_cu, stream);
    if (npairs <= 16) return launch_down_v<WT, 16>(a, max_slots, n_cu, stream);
    if (npairs <= 32) return launch_down_v<WT, 32>(a, max_slots, n_cu, stream);
    return launch_down_v<WT, 64>(a, max_slots, n_cu, stream);
}

static ExpertArgs make_expert_args(const LayerDesc& L, const Workspace& ws, int T) {
    ExpertArgs a;
    a.H = L.H; a.F = L.F; a.E = L.E; a.K = L.K; a.S = L.S; a.T = T;
    a.w_gate = L.w_gate; a.w_up = L.w_up;
    a.gate_nb1 = L.gate_nb1; a.gate_nb2 = L.gate_nb2; a.up_nb1 = L.up_nb1; a.up_nb2 = L.up_nb2;
    a.w_down = L.w_down; a.down_nb1 = L.down_nb1; a.down_nb2 = L.down_nb2;
    a.w_sh_gate = L.w_sh_gate; a.w_sh_up = L.w_sh_up; a.w_sh_down = L.w_sh_down;
    a.sh_gate_nb1 = L.sh_gate_nb1; a.sh_up_nb1 = L.sh_up_nb1; a.sh_down_nb1 = L.sh_down_nb1;
    a.counters = ws.counters; a.slot_info = ws.slot_info; a.offsets = ws.offsets; a.row_token = ws.row_token;
    a.xq_qs = ws.xq_qs; a.xq_ds = ws.xq_ds; a.gubuf = ws.gubuf; a.hq_qs = ws.hq_qs; a.hq_ds = ws.hq_ds;
    a.ybuf = ws.ybuf;
    a.act = L.act;
    a.gelu_tab = L.gelu_tab;
    a.ysh = ws.ysh;
    a.sd_blocks = 0;
    return a;
}

hipError_t launch_experts_gateup(const LayerDesc& L, const Workspace& ws, int T, hipStream_t stream,
                                 hipEvent_t ev_start, hipEvent_t ev_stop) {
    const ExpertArgs a = make_expert_args(L, ws, T);
    const int max_slots = min(L.E, T * L.K) + L.S;
    return (L.gu_type == kTypeQ4_0) ? launch_gateup<kTypeQ4_0>(a, max_slots, L.n_cu, stream, ev_start, ev_stop)
                                    : launch_gateup<kTypeQ8_0>(a, max_slots, L.n_cu, stream, ev_start, ev_stop);
}

// The fused decode gate/up needs the decode slot list (the decode routing),
// 16..64 lanes per H row (H in (512, 4096]) and the token rows within 64 KiB of LDS.
bool gateup_q_fused(const LayerDesc& L, int T) {
    return route_decode_fused(L, T) && down_combine_fused(L, T) && L.H > 512 && L.H <= 4096 &&
           gq_lds_bytes(T, L.H) <= 64 * 1024;
}

template <int WT>
static hipError_t launch_gateup_q_t(const ExpertArgs& a, const int4* dslots, int max_v, hipStream_t stream,
                                    hipEvent_t e0, hipEvent_t e1) {
    const int npairs = a.H / 64;
    const dim3 g(a.sd_blocks + max_v * (a.F / 32));
    const size_t lds = gq_lds_bytes(a.T, a.H);
    constexpr int NW = kGqWaves<WT>;
    // lanes x pairs per row: 16 x 1, 32 x 1, 16 x 3 (H = 2816: 44 of 48 slots live), 64 x 1
    if (npairs <= 16) launch_timed(k_gateup_q<WT, 16, NW, 1>, g, dim3(NW * 64), lds, stream, e0, e1, a, dslots);
    else if (npairs <= 32) launch_timed(k_gateup_q<WT, 32, NW, 1>, g, dim3(NW * 64), lds, stream, e0, e1, a, dslots);
    else if (npairs <= 48) launch_timed(k_gateup_q<WT, 16, NW, 3>, g, dim3(NW * 64), lds, stream, e0, e1, a, dslots);
    else launch_timed(k_gateup_q<WT, 64, 8, 1>, g, dim3(512), lds, stream, e0, e1, a, dslots);
    return hipGetLastError();
}

hipError_t launch_gateup_q(const LayerDesc& L, const Workspace& ws, int T, hipStream_t stream, hipEvent_t ev_start,
                           hipEvent_t ev_stop) {
    ExpertArgs a = make_expert_args(L, ws, T);
    const int max_v = min(L.E, T * L.K);  // routed slots; the routing launch does the shared expert's h
    if (shared_down_in_gateup(L, T)) {
        constexpr int NW = 8;  // waves per workgroup of the Q4_0 and Q8_0 instances
        static_assert(kGqWaves<kTypeQ4_0> == NW && kGqWaves<kTypeQ8_0> == NW, "shared-down workgroup size");
        a.sd_blocks = ((L.H / (64 / kSdLanes)) * kSdSplit + NW - 1) / NW;
    }
    return (L.gu_type == kTypeQ4_0) ? launch_gateup_q_t<kTypeQ4_0>(a, ws.dslots, max_v, stream, ev_start, ev_stop)
                                    : launch_gateup_q_t<kTypeQ8_0>(a, ws.dslots, max_v, stream, ev_start, ev_stop);
}

hipError_t launch_quant_h(const LayerDesc& L, const Workspace& ws, int T, hipStream_t stream) {
    const ExpertArgs a = make_expert_args(L, ws, T);
    const int max_rows = T * L.K + L.S * T;
    const int qblocks = (max_rows * (L.F / 4) + 255) / 256;
    hipLaunchKernelGGL(k_quant_h, dim3(qblocks), dim3(256), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_experts_down(const LayerDesc& L, const Workspace& ws, int T, hipStream_t stream) {
    const ExpertArgs a = make_expert_args(L, ws, T);
    const int max_slots = min(L.E, T * L.K) + L.S;
    return (L.dn_type == kTypeQ4_0) ? launch_down<kTypeQ4_0>(a, max_slots, L.n_cu, stream)
                                    : launch_down<kTypeQ8_0>(a, max_slots, L.n_cu, stream);
}

// ---------------------------------------------------------------------------
// G3: combine.  out[t] = ((w0*y0 + w1*y1) + ...) + sigma_t * y_shared (+ residual),
// each product and sum a separately rounded f32 operation, in slot order.
// ---------------------------------------------------------------------------
struct CombineArgs {
    int H, K, S, T;
    const float* ybuf; const int32_t* pos; const float* topk_w; const float* sh_gate;
    const float* residual; float* y;
    double* y_ssq;  // [T][ssq_parts(H)] y's RMSNorm partial sums (H a multiple of 32), or null
};

__global__ __launch_bounds__(256) void k_combine(CombineArgs a) {
#pragma clang fp contract(off)
    const int t = blockIdx.y;
    const int n = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (!a.y_ssq && n >= a.H) return;
    const bool live = n < a.H;  // (with y_ssq every lane takes part in the 8-lane trees)
    const int A = a.T * a.K;
    f32x4 acc = {};
    if (live) {
        const int32_t* pt = a.pos + (uint64_t)t * a.K;
        const float* wt = a.topk_w + (uint64_t)t * a.K;
        {
            const float w = wt[0];
            const f32x4 v = *(const f32x4*)(a.ybuf + (uint64_t)pt[0] * a.H + n);
            acc = f32x4{w * v.x, w * v.y, w * v.z, w * v.w};
        }
        for (int j = 1; j < a.K; ++j) {
            const float w = wt[j];
            const f32x4 v = *(const f32x4*)(a.ybuf + (uint64_t)pt[j] * a.H + n);
            const f32x4 term = f32x4{w * v.x, w * v.y, w * v.z, w * v.w};
            acc = acc + term;
        }
        if (a.S) {
            const float s = a.sh_gate[t];
            const f32x4 v = *(const f32x4*)(a.ybuf + (uint64_t)(A + t) * a.H + n);
            const f32x4 term = f32x4{v.x * s, v.y * s, v.z * s, v.w * s};
            acc = acc + term;
        }
        if (a.residual) {
            const f32x4 r = *(const f32x4*)(a.residual + (uint64_t)t * a.H + n);
            acc = acc + r;
        }
        *(f32x4*)(a.y + (uint64_t)t * a.H + n) = acc;
    }
    if (a.y_ssq) {
        // this thread's 4 columns are run n / 4 of the row (f64 of each f32
        // square, in column order); 8 consecutive lanes hold the 8 runs of entry
        // n / 32, whose adjacent-pairs tree is dpp_sum_f64<8>
        double s = 0.0;
        if (live)
#pragma unroll
            for (int c = 0; c < 4; ++c) s += (double)(acc[c] * acc[c]);
        s = dpp_sum_f64<8>(s);
        if (live && (threadIdx.x & 7) == 7) a.y_ssq[(uint64_t)t * ssq_parts(a.H) + (n >> 5)] = s;
    }
}

hipError_t launch_combine(const LayerDesc& L, const Workspace& ws, int T, float* y, const float* residual,
                          hipStream_t stream, double* y_ssq) {
    CombineArgs a;
    a.H = L.H; a.K = L.K; a.S = L.S; a.T = T;
    a.ybuf = ws.ybuf; a.pos = ws.pos; a.topk_w = ws.topk_w; a.sh_gate = ws.sh_gate;
    a.residual = residual; a.y = y;
    a.y_ssq = (L.H % 32 == 0) ? y_ssq : nullptr;
    const dim3 grid((L.H / 4 + 255) / 256, T);
    hipLaunchKernelGGL(k_combine, grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace qmoe
