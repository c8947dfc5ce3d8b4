// route_kernels.hip -- router GEMV + Q8_0 activation quantization, top-k +
// softmax, and the stable token->expert counting sort.
//
// Semantics restated from the reference's MoELayer::build
// (src/layers/moe.cpp:72 router mul_mat, :77-82 argsort DESC + view,
// :88-94 get_rows + soft_max, :169-172 shared-expert gate) and from the row
// mapping that ggml_mul_mat_id builds for :105-127 (per expert, ascending
// (token, slot)).  Ties in the top-k go to the lowest expert index.
#include "qmoe_device.h"
#include "qmoe_internal.h"

namespace qmoe {

// ---------------------------------------------------------------------------
// R1: router logits (one wave per router row, all tokens) + activation quant
// ---------------------------------------------------------------------------
struct RouterArgs {
    const float* x;         // [T][H]
    const float* w_router;  // [E][ld]
    uint64_t router_ld;
    const float* w_sh_norm; // [H] or null
    int T, H, E, S;
    int n_router_blocks;
    float* logits;          // [T][E+1]
    int8_t* xq_qs;          // [T][H]
    float2* xq_ds;          // [T][H/32]
};

constexpr int kRouterMaxChunks = 64;  // H <= 4096 keeps the router row in registers

__global__ __launch_bounds__(256) void k_router_quant(RouterArgs a) {
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    if ((int)blockIdx.x < a.n_router_blocks) {
        const int e = blockIdx.x * 4 + wave;
        if (e >= a.E + a.S) return;
        const float* wrow = (e < a.E) ? a.w_router + (uint64_t)e * a.router_ld : a.w_sh_norm;
        const int nch = a.H >> 6;  // values per lane
        if (nch <= kRouterMaxChunks) {
            float w[kRouterMaxChunks];
#pragma unroll
            for (int i = 0; i < kRouterMaxChunks; ++i)
                if (i < nch) w[i] = wrow[i * 64 + lane];
            for (int t = 0; t < a.T; ++t) {
                const float* xr = a.x + (uint64_t)t * a.H;
                double acc = 0.0;
#pragma unroll
                for (int i = 0; i < kRouterMaxChunks; ++i)
                    if (i < nch) acc = __builtin_fma((double)w[i], (double)xr[i * 64 + lane], acc);
                acc = group_sum_f64<64>(acc);
                if (lane == 0) a.logits[(uint64_t)t * (a.E + 1) + e] = (float)acc;
            }
        } else {
            for (int t = 0; t < a.T; ++t) {
                const float* xr = a.x + (uint64_t)t * a.H;
                double acc = 0.0;
                for (int i = lane; i < a.H; i += 64) acc = __builtin_fma((double)wrow[i], (double)xr[i], acc);
                acc = group_sum_f64<64>(acc);
                if (lane == 0) a.logits[(uint64_t)t * (a.E + 1) + e] = (float)acc;
            }
        }
        return;
    }
    // activation quantization: one wave per token, one 32-value block per lane step
    const int t = (blockIdx.x - a.n_router_blocks) * 4 + wave;
    if (t >= a.T) return;
    const float* xr = a.x + (uint64_t)t * a.H;
    const int nb = a.H >> 5;
    for (int b = lane; b < nb; b += 64) {
        const f32x4* src = (const f32x4*)(xr + 32 * b);
        float v[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const f32x4 q = src[i];
            v[4 * i + 0] = q.x; v[4 * i + 1] = q.y; v[4 * i + 2] = q.z; v[4 * i + 3] = q.w;
        }
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) amax = fmaxf(amax, __builtin_fabsf(v[i]));
        const float d = amax / 127.0f;
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        const float df = fp16_to_f32(f32_to_fp16(d));
        uint32_t packed[8];
        int sum = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            uint32_t word = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int q = (int)__builtin_rintf(v[4 * i + j] * id);
                sum += q;
                word |= ((uint32_t)(q & 0xff)) << (8 * j);
            }
            packed[i] = word;
        }
        u32x4* dst = (u32x4*)(a.xq_qs + (uint64_t)t * a.H + 32 * b);
        dst[0] = u32x4{packed[0], packed[1], packed[2], packed[3]};
        dst[1] = u32x4{packed[4], packed[5], packed[6], packed[7]};
        a.xq_ds[(uint64_t)t * nb + b] = make_float2(df, __builtin_bit_cast(float, sum));
    }
}

// ---------------------------------------------------------------------------
// R2: top-k + softmax + shared gate; per-block histogram and local ranks;
// then (single block, or a second launch) scan + stable scatter.
// ---------------------------------------------------------------------------
struct TopkArgs {
    const float* logits;  // [T][E+1]
    int T, E, K, S;
    int32_t* topk_idx;    // [T][K]
    float* topk_w;        // [T][K]
    float* sh_gate;       // [T]
    int32_t* local_rank;  // [T*K]
    int32_t* hist;        // [nblk][E]
    int32_t* offsets;     // [E+2]
    int32_t* rows;        // [R]
    int32_t* row_token;   // [R]
    int32_t* pos;         // [T*K]
    int32_t* active;      // [E+1]
    int32_t* counters;    // [0] n_active, [1] n_tiles
    int4* tiles;
    int max_tiles;
    int nblk;
};

constexpr int kMaxExpertsPerLane = 16;  // E <= 1024
constexpr int kMaxTopK = 64;

// (v, i) beats (v2, i2): larger logit first, ties to the lower expert id.
__device__ __forceinline__ bool better(float v, int i, float v2, int i2) {
    return v > v2 || (v == v2 && i < i2);
}

__device__ void topk_one_token(const TopkArgs& a, int t, int lane, int32_t* s_idx_row, float* s_val_row) {
    const float* l = a.logits + (uint64_t)t * (a.E + 1);
    float v[kMaxExpertsPerLane];
    const int per_lane = (a.E + 63) >> 6;
#pragma unroll
    for (int i = 0; i < kMaxExpertsPerLane; ++i) {
        const int e = i * 64 + lane;
        v[i] = (i < per_lane && e < a.E) ? l[e] : -__builtin_huge_valf();
    }
    uint32_t taken = 0;
    for (int j = 0; j < a.K; ++j) {
        float bv = -__builtin_huge_valf();
        int bi = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < kMaxExpertsPerLane; ++i) {
            const int e = i * 64 + lane;
            if (i < per_lane && e < a.E && !((taken >> i) & 1u) && better(v[i], e, bv, bi)) { bv = v[i]; bi = e; }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int oi = __shfl_xor(bi, o, 64);
            if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
        }
        if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
        if (lane == 0) {
            s_idx_row[j] = bi;
            s_val_row[j] = bv;
            a.topk_idx[(uint64_t)t * a.K + j] = bi;
        }
    }
    if (lane == 0) {
#pragma clang fp contract(off)
        // softmax over the selected logits; slot 0 holds the maximum
        const double m = (double)s_val_row[0];
        double sum = 0.0;
        for (int j = 0; j < a.K; ++j) sum = sum + exp_det((double)s_val_row[j] - m);
        for (int j = 0; j < a.K; ++j)
            a.topk_w[(uint64_t)t * a.K + j] = (float)(exp_det((double)s_val_row[j] - m) / sum);
        if (a.S) a.sh_gate[t] = sigmoid_det(l[a.E]);
    }
}

// Scan of per-block histograms, expert offsets, active list, MFMA tile list and
// the stable scatter.  Runs in ONE block (any blockDim multiple of 64).
__device__ void scan_and_scatter(const TopkArgs& a, int32_t* s_scan /* >= E+1 ints */) {
    const int tid = threadIdx.x;
    const int nthr = blockDim.x;
    // 1. per-expert exclusive base per top-k block (in place) and totals
    for (int e = tid; e < a.E; e += nthr) {
        int run = 0;
        for (int b = 0; b < a.nblk; ++b) {
            const int c = a.hist[(uint64_t)b * a.E + e];
            a.hist[(uint64_t)b * a.E + e] = run;
            run += c;
        }
        s_scan[e] = run;
    }
    __syncthreads();
    // 2. serial-in-wave exclusive scans (E <= 1024; done by wave 0)
    if (tid < 64) {
        int carry = 0;
        int carry_act = 0;
        int carry_tiles = 0;
        for (int base = 0; base < a.E; base += 64) {
            const int e = base + tid;
            const int c = e < a.E ? s_scan[e] : 0;
            const int act = c > 0 ? 1 : 0;
            const int nt = (c + kMfmaTileM - 1) / kMfmaTileM;
            int inc = c, inc_act = act, inc_t = nt;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int u = __shfl_up(inc, o, 64);
                const int ua = __shfl_up(inc_act, o, 64);
                const int ut = __shfl_up(inc_t, o, 64);
                if (tid >= o) { inc += u; inc_act += ua; inc_t += ut; }
            }
            if (e < a.E) {
                const int off = carry + inc - c;
                a.offsets[e] = off;
                if (act) a.active[carry_act + inc_act - 1] = e;
                int t0 = carry_tiles + inc_t - nt;
                for (int i = 0; i < nt && t0 + i < a.max_tiles; ++i) {
                    const int r0 = off + i * kMfmaTileM;
                    const int nr = min(kMfmaTileM, c - i * kMfmaTileM);
                    a.tiles[t0 + i] = make_int4(e, r0, nr, 0);
                }
            }
            carry += __shfl(inc, 63, 64);
            carry_act += __shfl(inc_act, 63, 64);
            carry_tiles += __shfl(inc_t, 63, 64);
        }
        const int A = a.T * a.K;
        if (tid == 0) {
            a.offsets[a.E] = A;
            a.offsets[a.E + 1] = A + a.S * a.T;
            int n_act = carry_act;
            int n_tiles = carry_tiles;
            if (a.S) {
                a.active[n_act++] = a.E;
                const int nt = (a.T + kMfmaTileM - 1) / kMfmaTileM;
                for (int i = 0; i < nt && n_tiles < a.max_tiles; ++i) {
                    a.tiles[n_tiles++] = make_int4(a.E, A + i * kMfmaTileM, min(kMfmaTileM, a.T - i * kMfmaTileM), 0);
                }
            }
            a.counters[0] = n_act;
            a.counters[1] = n_tiles;
        }
    }
    __syncthreads();
    // 3. stable scatter: position = offset[e] + block base + rank inside block
    const int A = a.T * a.K;
    for (int asg = tid; asg < A; asg += nthr) {
        const int t = asg / a.K;
        const int e = a.topk_idx[asg];
        const int blk = t / kTopkTokensPerBlock;
        const int p = a.offsets[e] + a.hist[(uint64_t)blk * a.E + e] + a.local_rank[asg];
        a.rows[p] = asg;
        a.row_token[p] = t;
        a.pos[asg] = p;
    }
    if (a.S) {
        for (int t = tid; t < a.T; t += nthr) {
            a.rows[A + t] = -1;
            a.row_token[A + t] = t;
        }
    }
}

// blockDim = 256 (4 waves), kTopkTokensPerBlock tokens per block.
__global__ __launch_bounds__(256) void k_topk(TopkArgs a, int fused_scan) {
    __shared__ int32_t s_idx[kTopkTokensPerBlock][kMaxTopK];
    __shared__ float s_val[kTopkTokensPerBlock][kMaxTopK];
    __shared__ int32_t s_cnt[1024 + 1];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int t0 = blockIdx.x * kTopkTokensPerBlock;
    const int ntok = min(kTopkTokensPerBlock, a.T - t0);
    for (int i = wave; i < ntok; i += 4) topk_one_token(a, t0 + i, lane, s_idx[i], s_val[i]);
    for (int e = threadIdx.x; e < a.E; e += blockDim.x) s_cnt[e] = 0;
    __syncthreads();
    // local ranks (stable by token inside the block) and block histogram
    for (int asg = threadIdx.x; asg < ntok * a.K; asg += blockDim.x) {
        const int ti = asg / a.K;
        const int j = asg % a.K;
        const int e = s_idx[ti][j];
        int rank = 0;
        for (int tp = 0; tp < ti; ++tp)
            for (int jj = 0; jj < a.K; ++jj) rank += (s_idx[tp][jj] == e) ? 1 : 0;
        a.local_rank[(uint64_t)(t0 + ti) * a.K + j] = rank;
        atomicAdd(&s_cnt[e], 1);
    }
    __syncthreads();
    for (int e = threadIdx.x; e < a.E; e += blockDim.x) a.hist[(uint64_t)blockIdx.x * a.E + e] = s_cnt[e];
    if (fused_scan) {
        __syncthreads();
        scan_and_scatter(a, s_cnt);
    }
}

__global__ __launch_bounds__(1024) void k_scan_scatter(TopkArgs a) {
    __shared__ int32_t s_cnt[1024 + 1];
    scan_and_scatter(a, s_cnt);
}

hipError_t launch_route(const LayerDesc& L, const Workspace& ws, const float* x, int T, hipStream_t stream) {
    RouterArgs ra;
    ra.x = x;
    ra.w_router = L.w_router;
    ra.router_ld = L.router_ld;
    ra.w_sh_norm = L.w_sh_norm;
    ra.T = T; ra.H = L.H; ra.E = L.E; ra.S = L.S;
    ra.n_router_blocks = (L.E + L.S + 3) / 4;
    ra.logits = ws.logits;
    ra.xq_qs = ws.xq_qs;
    ra.xq_ds = ws.xq_ds;
    const int nq = (T + 3) / 4;
    hipLaunchKernelGGL(k_router_quant, dim3(ra.n_router_blocks + nq), dim3(256), 0, stream, ra);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;

    TopkArgs ta;
    ta.logits = ws.logits;
    ta.T = T; ta.E = L.E; ta.K = L.K; ta.S = L.S;
    ta.topk_idx = ws.topk_idx;
    ta.topk_w = ws.topk_w;
    ta.sh_gate = ws.sh_gate;
    ta.local_rank = ws.local_rank;
    ta.hist = ws.hist;
    ta.offsets = ws.offsets;
    ta.rows = ws.rows;
    ta.row_token = ws.row_token;
    ta.pos = ws.pos;
    ta.active = ws.active;
    ta.counters = ws.counters;
    ta.tiles = ws.tiles;
    ta.max_tiles = ws.max_tiles;
    ta.nblk = (T + kTopkTokensPerBlock - 1) / kTopkTokensPerBlock;
    const int fused = ta.nblk == 1 ? 1 : 0;
    hipLaunchKernelGGL(k_topk, dim3(ta.nblk), dim3(256), 0, stream, ta, fused);
    err = hipGetLastError();
    if (err != hipSuccess || fused) return err;
    hipLaunchKernelGGL(k_scan_scatter, dim3(1), dim3(1024), 0, stream, ta);
    return hipGetLastError();
}

}  // namespace qmoe
