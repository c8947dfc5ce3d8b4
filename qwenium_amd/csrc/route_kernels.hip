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

// Router GEMV for small token counts: one 256-thread block per router row
// (row E is the shared-expert gate vector).  Wave w owns float4 chunks
// c = w + 4i of the row (chunk = 64 float4 = 256 values); every load is
// unconditional (clamped index, zeroed weight) so a token chunk's loads issue
// back to back.  Products are exact in f64; the sum is exact-order-free f64.
constexpr int kRouterTokChunk = 8;

template <int NCH>
__device__ __forceinline__ void router_row(const RouterArgs& a, int e, float* s_part) {
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const float* wrow = (e < a.E) ? a.w_router + (uint64_t)e * a.router_ld : a.w_sh_norm;
    const int nchunks = a.H >> 8;
    f32x4 w[NCH];
    int off[NCH];
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        const int c = wave + 4 * i;
        const int cc = c < nchunks ? c : nchunks - 1;
        off[i] = (cc * 64 + lane) * 4;
        const f32x4 v = *(const f32x4*)(wrow + off[i]);
        w[i] = c < nchunks ? v : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    for (int t0 = 0; t0 < a.T; t0 += kRouterTokChunk) {
        f32x4 xv[kRouterTokChunk][NCH];
#pragma unroll
        for (int c = 0; c < kRouterTokChunk; ++c) {
            const int t = min(t0 + c, a.T - 1);
            const float* xr = a.x + (uint64_t)t * a.H;
#pragma unroll
            for (int i = 0; i < NCH; ++i) xv[c][i] = *(const f32x4*)(xr + off[i]);
        }
#pragma unroll
        for (int c = 0; c < kRouterTokChunk; ++c) {
            double acc = 0.0;
#pragma unroll
            for (int i = 0; i < NCH; ++i) {
                acc = __builtin_fma((double)w[i].x, (double)xv[c][i].x, acc);
                acc = __builtin_fma((double)w[i].y, (double)xv[c][i].y, acc);
                acc = __builtin_fma((double)w[i].z, (double)xv[c][i].z, acc);
                acc = __builtin_fma((double)w[i].w, (double)xv[c][i].w, acc);
            }
            acc = group_sum_f64<64>(acc);
            if (lane == 0) ((double*)s_part)[wave * kRouterTokChunk + c] = acc;
        }
        __syncthreads();
        if (threadIdx.x < kRouterTokChunk && t0 + (int)threadIdx.x < a.T) {
            const double* p = (const double*)s_part;
            const int c = threadIdx.x;
            const double sum = (p[0 * kRouterTokChunk + c] + p[1 * kRouterTokChunk + c]) +
                               (p[2 * kRouterTokChunk + c] + p[3 * kRouterTokChunk + c]);
            a.logits[(uint64_t)(t0 + c) * (a.E + 1) + e] = (float)sum;
        }
        __syncthreads();
    }
}

template <int NCH>
__global__ __launch_bounds__(256) void k_router_quant(RouterArgs a) {
    __shared__ double s_part[4 * kRouterTokChunk];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    if ((int)blockIdx.x < a.n_router_blocks) {
        router_row<NCH>(a, blockIdx.x, (float*)s_part);
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
    int4* slot_info;      // [E+1] {expert, first row, rows, 0}
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

template <int EPL>
__device__ void topk_one_token(const TopkArgs& a, int t, int lane, int32_t* s_idx_row, float* s_val_row,
                               double* s_ex_row) {
    const float* l = a.logits + (uint64_t)t * (a.E + 1);
    // this lane's candidates e = i*64 + lane, sorted by (logit desc, id asc)
    float v[EPL];
    int id[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        const int e = i * 64 + lane;
        const float lv = l[min(e, a.E - 1)];  // unconditional load, masked below
        v[i] = e < a.E ? lv : -__builtin_huge_valf();
        id[i] = e < a.E ? e : 0x7fffffff;
    }
#pragma unroll
    for (int i = 1; i < EPL; ++i)
#pragma unroll
        for (int j = i; j > 0; --j) {
            if (better(v[j], id[j], v[j - 1], id[j - 1])) {
                const float tv = v[j]; v[j] = v[j - 1]; v[j - 1] = tv;
                const int ti = id[j]; id[j] = id[j - 1]; id[j - 1] = ti;
            }
        }
    for (int j = 0; j < a.K; ++j) {
        float bv = v[0];
        int bi = id[0];
        wave_argmax(bv, bi);
        if (id[0] == bi) {  // the winning lane pops its head
#pragma unroll
            for (int i = 0; i + 1 < EPL; ++i) { v[i] = v[i + 1]; id[i] = id[i + 1]; }
            v[EPL - 1] = -__builtin_huge_valf();
            id[EPL - 1] = 0x7fffffff;
        }
        if (lane == 0) {
            s_idx_row[j] = bi;
            s_val_row[j] = bv;
            a.topk_idx[(uint64_t)t * a.K + j] = bi;
        }
    }
    // lanes below read what lane 0 wrote to LDS: order the wave's LDS accesses
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    // softmax over the selected logits (slot 0 holds the maximum): exps in
    // parallel lanes, the sum in slot order, the divisions in parallel lanes
    {
#pragma clang fp contract(off)
        const double m = (double)s_val_row[0];
        double ex = 0.0;
        if (lane < a.K) {
            ex = exp_det((double)s_val_row[lane] - m);
            s_ex_row[lane] = ex;
        }
        if (lane == a.K && a.S) a.sh_gate[t] = sigmoid_det(l[a.E]);
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        double sum = 0.0;
        if (lane == 0) {
            for (int j = 0; j < a.K; ++j) sum = sum + s_ex_row[j];
            s_ex_row[kMaxTopK] = sum;
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        sum = s_ex_row[kMaxTopK];
        if (lane < a.K) a.topk_w[(uint64_t)t * a.K + lane] = (float)(ex / sum);
    }
}

__device__ __forceinline__ void topk_dispatch(const TopkArgs& a, int t, int lane, int32_t* s_idx_row,
                                              float* s_val_row, double* s_ex_row) {
    const int epl = (a.E + 63) >> 6;
    if (epl <= 1) topk_one_token<1>(a, t, lane, s_idx_row, s_val_row, s_ex_row);
    else if (epl <= 2) topk_one_token<2>(a, t, lane, s_idx_row, s_val_row, s_ex_row);
    else if (epl <= 4) topk_one_token<4>(a, t, lane, s_idx_row, s_val_row, s_ex_row);
    else if (epl <= 8) topk_one_token<8>(a, t, lane, s_idx_row, s_val_row, s_ex_row);
    else topk_one_token<16>(a, t, lane, s_idx_row, s_val_row, s_ex_row);
}

// Scan of per-block histograms, expert offsets, active list, slot table, MFMA
// tile list and the stable scatter.  Runs in ONE block (blockDim a multiple of
// 64, at least 256).
__device__ void scan_and_scatter(const TopkArgs& a, int32_t* s_scan /* >= E+1 ints */, int32_t* s_misc /* >= 64 */) {
    const int tid = threadIdx.x;
    const int nthr = blockDim.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int nwaves = nthr >> 6;
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
    // 2. exclusive scans over experts: rows, active flags, MFMA tiles.  Chunks of
    //    64 experts are scanned by separate waves, then chunk totals are combined.
    const int nchunk = (a.E + 63) >> 6;  // <= 16
    int c_rows = 0, c_act = 0, c_tiles = 0, inc = 0, inc_act = 0, inc_t = 0, e = 0;
    if (wave < nchunk) {
        e = wave * 64 + lane;
        c_rows = e < a.E ? s_scan[e] : 0;
        c_act = c_rows > 0 ? 1 : 0;
        c_tiles = (c_rows + kMfmaTileM - 1) / kMfmaTileM;
        inc = wave_incl_scan_i32(c_rows);
        inc_act = wave_incl_scan_i32(c_act);
        inc_t = wave_incl_scan_i32(c_tiles);
        if (lane == 63) { s_misc[3 * wave] = inc; s_misc[3 * wave + 1] = inc_act; s_misc[3 * wave + 2] = inc_t; }
    }
    __syncthreads();
    if (wave < nchunk) {
        int base = 0, base_act = 0, base_t = 0;
        for (int w = 0; w < wave; ++w) { base += s_misc[3 * w]; base_act += s_misc[3 * w + 1]; base_t += s_misc[3 * w + 2]; }
        if (e < a.E) {
            const int off = base + inc - c_rows;
            a.offsets[e] = off;
            s_scan[e] = off;  // offsets kept in LDS for the scatter
            if (c_act) {
                const int slot = base_act + inc_act - 1;
                a.active[slot] = e;
                a.slot_info[slot] = make_int4(e, off, c_rows, 0);
            }
            const int t0 = base_t + inc_t - c_tiles;
            for (int i = 0; i < c_tiles && t0 + i < a.max_tiles; ++i)
                a.tiles[t0 + i] = make_int4(e, off + i * kMfmaTileM, min(kMfmaTileM, c_rows - i * kMfmaTileM), 0);
        }
        if (wave == nchunk - 1 && lane == 63) {
            const int A = a.T * a.K;
            int n_act = base_act + inc_act;
            int n_tiles = base_t + inc_t;
            a.offsets[a.E] = A;
            a.offsets[a.E + 1] = A + a.S * a.T;
            if (a.S) {
                a.active[n_act] = a.E;
                a.slot_info[n_act] = make_int4(a.E, A, a.T, 0);
                n_act++;
                const int nt = (a.T + kMfmaTileM - 1) / kMfmaTileM;
                for (int i = 0; i < nt && n_tiles < a.max_tiles; ++i)
                    a.tiles[n_tiles++] = make_int4(a.E, A + i * kMfmaTileM, min(kMfmaTileM, a.T - i * kMfmaTileM), 0);
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
        const int ex = a.topk_idx[asg];
        const int blk = t / kTopkTokensPerBlock;
        const int p = s_scan[ex] + a.hist[(uint64_t)blk * a.E + ex] + a.local_rank[asg];
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
    __syncthreads();
    // 4. token of each slot's first row (lets the expert kernels fetch it without a lookup)
    const int n_act = a.counters[0];
    for (int i = tid; i < n_act; i += nthr) {
        int4 si = a.slot_info[i];
        si.w = a.row_token[si.y];
        a.slot_info[i] = si;
    }
}

// blockDim = 64 * kTopkTokensPerBlock: one wave per token.
__global__ __launch_bounds__(64 * kTopkTokensPerBlock) void k_topk(TopkArgs a, int fused_scan) {
    __shared__ int32_t s_idx[kTopkTokensPerBlock][kMaxTopK];
    __shared__ float s_val[kTopkTokensPerBlock][kMaxTopK];
    __shared__ double s_ex[kTopkTokensPerBlock][kMaxTopK + 1];
    __shared__ uint32_t s_mask[1024];  // per expert: bit ti set if block token ti chose it
    __shared__ int32_t s_cnt[1024 + 1];
    __shared__ int32_t s_misc[64];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int t0 = blockIdx.x * kTopkTokensPerBlock;
    const int ntok = min(kTopkTokensPerBlock, a.T - t0);
    for (int e = threadIdx.x; e < a.E; e += blockDim.x) s_mask[e] = 0;
    __syncthreads();
    if (wave < ntok) {
        topk_dispatch(a, t0 + wave, lane, s_idx[wave], s_val[wave], s_ex[wave]);
        if (lane < a.K) atomicOr(&s_mask[s_idx[wave][lane]], 1u << wave);
    }
    __syncthreads();
    // local rank of (token ti, slot j) = earlier block tokens that chose the same expert
    for (int asg = threadIdx.x; asg < ntok * a.K; asg += blockDim.x) {
        const int ti = asg / a.K;
        const int j = asg % a.K;
        const int ex = s_idx[ti][j];
        a.local_rank[(uint64_t)(t0 + ti) * a.K + j] = __builtin_popcount(s_mask[ex] & ((1u << ti) - 1u));
    }
    for (int e = threadIdx.x; e < a.E; e += blockDim.x)
        a.hist[(uint64_t)blockIdx.x * a.E + e] = __builtin_popcount(s_mask[e]);
    if (fused_scan) {
        __syncthreads();
        scan_and_scatter(a, s_cnt, s_misc);
    }
}

// Whole routing for T <= kTopkTokensPerBlock in ONE block, everything in LDS:
// top-k per token (one wave each), per-expert token masks, counts, offsets,
// active slots (with the token of each slot's first row = lowest mask bit),
// stable scatter (rank = earlier tokens in the expert's mask) and tiles.
__global__ __launch_bounds__(64 * kTopkTokensPerBlock) void k_route_small(TopkArgs a) {
    __shared__ int32_t s_idx[kTopkTokensPerBlock][kMaxTopK];
    __shared__ float s_val[kTopkTokensPerBlock][kMaxTopK];
    __shared__ double s_ex[kTopkTokensPerBlock][kMaxTopK + 1];
    __shared__ uint32_t s_mask[1024];
    __shared__ int32_t s_off[1024];
    __shared__ int32_t s_misc[64];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int A = a.T * a.K;
    for (int e = tid; e < a.E; e += blockDim.x) s_mask[e] = 0;
    __syncthreads();
    if (wave < a.T) {
        topk_dispatch(a, wave, lane, s_idx[wave], s_val[wave], s_ex[wave]);
        if (lane < a.K) atomicOr(&s_mask[s_idx[wave][lane]], 1u << wave);
    }
    __syncthreads();
    const int nchunk = (a.E + 63) >> 6;
    int cnt = 0, act = 0, nt = 0, inc = 0, inc_act = 0, inc_t = 0, e = 0;
    if (wave < nchunk) {
        e = wave * 64 + lane;
        cnt = e < a.E ? __builtin_popcount(s_mask[e]) : 0;
        act = cnt > 0 ? 1 : 0;
        nt = (cnt + kMfmaTileM - 1) / kMfmaTileM;
        inc = wave_incl_scan_i32(cnt);
        inc_act = wave_incl_scan_i32(act);
        inc_t = wave_incl_scan_i32(nt);
        if (lane == 63) { s_misc[3 * wave] = inc; s_misc[3 * wave + 1] = inc_act; s_misc[3 * wave + 2] = inc_t; }
    }
    __syncthreads();
    if (wave < nchunk) {
        int base = 0, base_act = 0, base_t = 0;
        for (int w = 0; w < wave; ++w) { base += s_misc[3 * w]; base_act += s_misc[3 * w + 1]; base_t += s_misc[3 * w + 2]; }
        if (e < a.E) {
            const int off = base + inc - cnt;
            a.offsets[e] = off;
            s_off[e] = off;
            if (act) {
                const int slot = base_act + inc_act - 1;
                a.active[slot] = e;
                a.slot_info[slot] = make_int4(e, off, cnt, __builtin_ctz(s_mask[e]));
            }
            if (nt) {
                const int t0 = base_t + inc_t - nt;
                if (t0 < a.max_tiles) a.tiles[t0] = make_int4(e, off, cnt, 0);  // cnt <= T <= 16 < tile rows
            }
        }
        if (wave == nchunk - 1 && lane == 63) {
            int n_act = base_act + inc_act;
            int n_tiles = base_t + inc_t;
            a.offsets[a.E] = A;
            a.offsets[a.E + 1] = A + a.S * a.T;
            if (a.S) {
                a.active[n_act] = a.E;
                a.slot_info[n_act] = make_int4(a.E, A, a.T, 0);
                n_act++;
                if (n_tiles < a.max_tiles) a.tiles[n_tiles++] = make_int4(a.E, A, a.T, 0);
            }
            a.counters[0] = n_act;
            a.counters[1] = n_tiles;
        }
    }
    __syncthreads();
    for (int asg = tid; asg < A; asg += blockDim.x) {
        const int t = asg / a.K, j = asg % a.K;
        const int ex = s_idx[t][j];
        const int p = s_off[ex] + __builtin_popcount(s_mask[ex] & ((1u << t) - 1u));
        a.rows[p] = asg;
        a.row_token[p] = t;
        a.pos[asg] = p;
    }
    if (a.S && tid < a.T) {
        a.rows[A + tid] = -1;
        a.row_token[A + tid] = tid;
    }
}

__global__ __launch_bounds__(1024) void k_scan_scatter(TopkArgs a) {
    __shared__ int32_t s_cnt[1024 + 1];
    __shared__ int32_t s_misc[64];
    scan_and_scatter(a, s_cnt, s_misc);
}

hipError_t launch_route(const LayerDesc& L, const Workspace& ws, const float* x, int T, hipStream_t stream) {
    RouterArgs ra;
    ra.x = x;
    ra.w_router = L.w_router;
    ra.router_ld = L.router_ld;
    ra.w_sh_norm = L.w_sh_norm;
    ra.T = T; ra.H = L.H; ra.E = L.E; ra.S = L.S;
    ra.logits = ws.logits;
    ra.xq_qs = ws.xq_qs;
    ra.xq_ds = ws.xq_ds;
    const int nq = (T + 3) / 4;
    ra.n_router_blocks = L.E + L.S;
    const dim3 grid(ra.n_router_blocks + nq);
    const int nch_per_wave = (L.H / 256 + 3) / 4;  // float4 chunks of 256 values per wave
    if (nch_per_wave <= 1) hipLaunchKernelGGL((k_router_quant<1>), grid, dim3(256), 0, stream, ra);
    else if (nch_per_wave <= 2) hipLaunchKernelGGL((k_router_quant<2>), grid, dim3(256), 0, stream, ra);
    else if (nch_per_wave <= 4) hipLaunchKernelGGL((k_router_quant<4>), grid, dim3(256), 0, stream, ra);
    else hipLaunchKernelGGL((k_router_quant<8>), grid, dim3(256), 0, stream, ra);
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
    ta.slot_info = ws.slot_info;
    ta.counters = ws.counters;
    ta.tiles = ws.tiles;
    ta.max_tiles = ws.max_tiles;
    ta.nblk = (T + kTopkTokensPerBlock - 1) / kTopkTokensPerBlock;
    if (ta.nblk == 1) {
        hipLaunchKernelGGL(k_route_small, dim3(1), dim3(64 * kTopkTokensPerBlock), 0, stream, ta);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_topk, dim3(ta.nblk), dim3(64 * kTopkTokensPerBlock), 0, stream, ta, 0);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(k_scan_scatter, dim3(1), dim3(1024), 0, stream, ta);
    return hipGetLastError();
}

}  // namespace qmoe
