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

namespace qmoe {

struct ExpertArgs {
    int H, F, E, K, S, T;
    const uint8_t* w_gate; const uint8_t* w_up; uint64_t gate_nb1, gate_nb2, up_nb1, up_nb2;
    const uint8_t* w_down; uint64_t down_nb1, down_nb2;
    const uint8_t* w_sh_gate; const uint8_t* w_sh_up; const uint8_t* w_sh_down;
    uint64_t sh_gate_nb1, sh_up_nb1, sh_down_nb1;
    const int32_t* active;     // [E+1]
    const int32_t* counters;   // [0] n_active
    const int32_t* offsets;    // [E+2]
    const int32_t* row_token;  // [R]
    const int8_t* xq_qs; const float2* xq_ds;  // [T][H], [T][H/32]
    int8_t* hq_qs; float2* hq_ds;              // [R][F], [R][F/32]
    float* ybuf;                               // [R][H]
};

// ---------------------------------------------------------------------------
// G1: gate + up + SwiGLU + Q8_0 quantization of h.
// Block = 4 waves = 32 consecutive ffn rows of one active expert (one Q8_0
// block of h).  Wave w owns rows f0+8w .. f0+8w+7 of gate and of up.
// LPR lanes cover one H row (LPR = min(64, H/64) pairs); RPI = 64/LPR rows
// are loaded per instruction.
// ---------------------------------------------------------------------------
constexpr int kGuRowsPerWave = 8;
constexpr int kGuTokChunk = 2;

template <int WT, int LPR>
__global__ __launch_bounds__(256) void k_gateup_gemv(ExpertArgs a) {
    constexpr int RPI = 64 / LPR;
    constexpr int NI = kGuRowsPerWave / RPI;   // loads per matrix per wave
    const int slot = blockIdx.x;
    if (slot >= a.counters[0]) return;
    const int e = a.active[slot];
    const int f0 = blockIdx.y * 32;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int sub = lane / LPR;       // row inside an instruction
    const int lp = lane % LPR;        // lane inside the row
    const int npairs = a.H >> 6;

    const uint8_t* gbase; const uint8_t* ubase; uint64_t gnb1, unb1;
    if (e < a.E) {
        gbase = a.w_gate + (uint64_t)e * a.gate_nb2; gnb1 = a.gate_nb1;
        ubase = a.w_up + (uint64_t)e * a.up_nb2; unb1 = a.up_nb1;
    } else {
        gbase = a.w_sh_gate; gnb1 = a.sh_gate_nb1;
        ubase = a.w_sh_up; unb1 = a.sh_up_nb1;
    }
    const int p0 = a.offsets[e];
    const int nrows = a.offsets[e + 1] - p0;

    __shared__ float s_h[kGuTokChunk][32];

    // rows of this wave: f = f0 + 8*wave + m*RPI + sub, m < NI
    const int npass = (npairs + LPR - 1) / LPR;  // pair groups per lane (1 for H <= 64*LPR)

    for (int c0 = 0; c0 < nrows; c0 += kGuTokChunk) {
        const int nc = min(kGuTokChunk, nrows - c0);
        double acc_g[NI][kGuTokChunk];
        double acc_u[NI][kGuTokChunk];
#pragma unroll
        for (int m = 0; m < NI; ++m)
#pragma unroll
            for (int c = 0; c < kGuTokChunk; ++c) { acc_g[m][c] = 0.0; acc_u[m][c] = 0.0; }

        for (int ps = 0; ps < npass; ++ps) {
            const int pair = lp + ps * LPR;
            if (pair < npairs) {
                WPair<WT> wg[NI], wu[NI];
#pragma unroll
                for (int m = 0; m < NI; ++m) {
                    const int f = f0 + kGuRowsPerWave * wave + m * RPI + sub;
                    wg[m].load(gbase + (uint64_t)f * gnb1, pair);
                    wu[m].load(ubase + (uint64_t)f * unb1, pair);
                }
#pragma unroll
                for (int c = 0; c < kGuTokChunk; ++c) {
                    if (c < nc) {
                        const int t = a.row_token[p0 + c0 + c];
                        XPair xp;
                        xp.load(a.xq_qs + (uint64_t)t * a.H, a.xq_ds + (uint64_t)t * (a.H >> 5), pair);
#pragma unroll
                        for (int m = 0; m < NI; ++m) {
                            acc_g[m][c] += pair_dot<WT>(wg[m], xp);
                            acc_u[m][c] += pair_dot<WT>(wu[m], xp);
                        }
                    }
                }
            }
        }
        // reduce over the LPR lanes of each row; SwiGLU into LDS
#pragma unroll
        for (int c = 0; c < kGuTokChunk; ++c) {
#pragma unroll
            for (int m = 0; m < NI; ++m) {
                const double g = group_sum_f64<LPR>(acc_g[m][c]);
                const double u = group_sum_f64<LPR>(acc_u[m][c]);
                if (lp == 0 && c < nc) {
                    const int fl = kGuRowsPerWave * wave + m * RPI + sub;
                    s_h[c][fl] = silu_mul_det((float)g, (float)u);
                }
            }
        }
        __syncthreads();
        // Q8_0 quantization of each h row block (wave c handles token c)
        if (wave < nc) {
            const int c = wave;
            const float v = lane < 32 ? s_h[c][lane] : 0.0f;
            const float amax = group_max_f32<32>(__builtin_fabsf(v));
            const float d = amax / 127.0f;
            const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
            const int q = (int)__builtin_rintf(v * id);
            const int sum = group_sum_i32<32>(q);
            const int p = p0 + c0 + c;
            if (lane < 32) a.hq_qs[(uint64_t)p * a.F + f0 + lane] = (int8_t)q;
            if (lane == 0)
                a.hq_ds[(uint64_t)p * (a.F >> 5) + blockIdx.y] =
                    make_float2(fp16_to_f32(f32_to_fp16(d)), __builtin_bit_cast(float, sum));
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// G2: down projection for every row of an active expert.  Block = 4 waves =
// 64 consecutive output rows n; each wave owns 16 of them.  LPR lanes cover one
// F row.  Writes ybuf[p][n] (unweighted expert output).
// ---------------------------------------------------------------------------
constexpr int kDnRowsPerWave = 16;
constexpr int kDnTokChunk = 4;

template <int WT, int LPR>
__global__ __launch_bounds__(256) void k_down_gemv(ExpertArgs a) {
    constexpr int RPI = 64 / LPR;
    constexpr int NI = kDnRowsPerWave / RPI;
    const int slot = blockIdx.x;
    if (slot >= a.counters[0]) return;
    const int e = a.active[slot];
    const int n0 = blockIdx.y * 64;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int sub = lane / LPR;
    const int lp = lane % LPR;
    const int npairs = a.F >> 6;
    const int npass = (npairs + LPR - 1) / LPR;

    const uint8_t* dbase; uint64_t dnb1;
    if (e < a.E) { dbase = a.w_down + (uint64_t)e * a.down_nb2; dnb1 = a.down_nb1; }
    else { dbase = a.w_sh_down; dnb1 = a.sh_down_nb1; }
    const int p0 = a.offsets[e];
    const int nrows = a.offsets[e + 1] - p0;

    for (int c0 = 0; c0 < nrows; c0 += kDnTokChunk) {
        const int nc = min(kDnTokChunk, nrows - c0);
        double acc[NI][kDnTokChunk];
#pragma unroll
        for (int m = 0; m < NI; ++m)
#pragma unroll
            for (int c = 0; c < kDnTokChunk; ++c) acc[m][c] = 0.0;
        for (int ps = 0; ps < npass; ++ps) {
            const int pair = lp + ps * LPR;
            if (pair < npairs) {
                WPair<WT> wd[NI];
#pragma unroll
                for (int m = 0; m < NI; ++m) {
                    const int n = n0 + kDnRowsPerWave * wave + m * RPI + sub;
                    wd[m].load(dbase + (uint64_t)n * dnb1, pair);
                }
#pragma unroll
                for (int c = 0; c < kDnTokChunk; ++c) {
                    if (c < nc) {
                        const int p = p0 + c0 + c;
                        XPair xp;
                        xp.load(a.hq_qs + (uint64_t)p * a.F, a.hq_ds + (uint64_t)p * (a.F >> 5), pair);
#pragma unroll
                        for (int m = 0; m < NI; ++m) acc[m][c] += pair_dot<WT>(wd[m], xp);
                    }
                }
            }
        }
#pragma unroll
        for (int c = 0; c < kDnTokChunk; ++c) {
#pragma unroll
            for (int m = 0; m < NI; ++m) {
                const double y = group_sum_f64<LPR>(acc[m][c]);
                if (lp == 0 && c < nc) {
                    const int n = n0 + kDnRowsPerWave * wave + m * RPI + sub;
                    a.ybuf[(uint64_t)(p0 + c0 + c) * a.H + n] = (float)y;
                }
            }
        }
    }
}

template <int WT>
static hipError_t launch_gateup(const ExpertArgs& a, int max_slots, hipStream_t stream) {
    const dim3 grid(max_slots, a.F / 32), block(256);
    const int npairs = a.H / 64;
    if (npairs >= 32) hipLaunchKernelGGL((k_gateup_gemv<WT, 32>), grid, block, 0, stream, a);
    else if (npairs >= 16) hipLaunchKernelGGL((k_gateup_gemv<WT, 16>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((k_gateup_gemv<WT, 8>), grid, block, 0, stream, a);
    return hipGetLastError();
}

template <int WT>
static hipError_t launch_down(const ExpertArgs& a, int max_slots, hipStream_t stream) {
    const dim3 grid(max_slots, a.H / 64), block(256);
    const int npairs = a.F / 64;
    if (npairs >= 16) hipLaunchKernelGGL((k_down_gemv<WT, 16>), grid, block, 0, stream, a);
    else if (npairs >= 8) hipLaunchKernelGGL((k_down_gemv<WT, 8>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((k_down_gemv<WT, 4>), grid, block, 0, stream, a);
    return hipGetLastError();
}

static ExpertArgs make_expert_args(const LayerDesc& L, const Workspace& ws, int T) {
    ExpertArgs a;
    a.H = L.H; a.F = L.F; a.E = L.E; a.K = L.K; a.S = L.S; a.T = T;
    a.w_gate = L.w_gate; a.w_up = L.w_up;
    a.gate_nb1 = L.gate_nb1; a.gate_nb2 = L.gate_nb2; a.up_nb1 = L.up_nb1; a.up_nb2 = L.up_nb2;
    a.w_down = L.w_down; a.down_nb1 = L.down_nb1; a.down_nb2 = L.down_nb2;
    a.w_sh_gate = L.w_sh_gate; a.w_sh_up = L.w_sh_up; a.w_sh_down = L.w_sh_down;
    a.sh_gate_nb1 = L.sh_gate_nb1; a.sh_up_nb1 = L.sh_up_nb1; a.sh_down_nb1 = L.sh_down_nb1;
    a.active = ws.active; a.counters = ws.counters; a.offsets = ws.offsets; a.row_token = ws.row_token;
    a.xq_qs = ws.xq_qs; a.xq_ds = ws.xq_ds; a.hq_qs = ws.hq_qs; a.hq_ds = ws.hq_ds; a.ybuf = ws.ybuf;
    return a;
}

hipError_t launch_experts_gemv(const LayerDesc& L, const Workspace& ws, int T, hipStream_t stream) {
    const ExpertArgs a = make_expert_args(L, ws, T);
    const int max_slots = min(L.E, T * L.K) + L.S;
    hipError_t err = (L.gu_type == kTypeQ4_0) ? launch_gateup<kTypeQ4_0>(a, max_slots, stream)
                                              : launch_gateup<kTypeQ8_0>(a, max_slots, stream);
    if (err != hipSuccess) return err;
    return (L.dn_type == kTypeQ4_0) ? launch_down<kTypeQ4_0>(a, max_slots, stream)
                                    : launch_down<kTypeQ8_0>(a, max_slots, stream);
}

// ---------------------------------------------------------------------------
// G3: combine.  out[t] = ((w0*y0 + w1*y1) + ...) + sigma_t * y_shared (+ residual),
// each product and sum a separately rounded f32 operation, in slot order.
// ---------------------------------------------------------------------------
struct CombineArgs {
    int H, K, S, T;
    const float* ybuf; const int32_t* pos; const float* topk_w; const float* sh_gate;
    const float* residual; float* y;
};

__global__ __launch_bounds__(256) void k_combine(CombineArgs a) {
#pragma clang fp contract(off)
    const int t = blockIdx.y;
    const int n = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (n >= a.H) return;
    const int A = a.T * a.K;
    const int32_t* pt = a.pos + (uint64_t)t * a.K;
    const float* wt = a.topk_w + (uint64_t)t * a.K;
    f32x4 acc;
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

hipError_t launch_combine(const LayerDesc& L, const Workspace& ws, int T, float* y, const float* residual,
                          hipStream_t stream) {
    CombineArgs a;
    a.H = L.H; a.K = L.K; a.S = L.S; a.T = T;
    a.ybuf = ws.ybuf; a.pos = ws.pos; a.topk_w = ws.topk_w; a.sh_gate = ws.sh_gate;
    a.residual = residual; a.y = y;
    const dim3 grid((L.H / 4 + 255) / 256, T);
    hipLaunchKernelGGL(k_combine, grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace qmoe
