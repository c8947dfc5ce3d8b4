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

#include <algorithm>

namespace qmoe {

// ---------------------------------------------------------------------------
// R1: exact router logits of every token, for the debug copy when the batched
// router runs (its own logits are approximate); the forward paths compute
// theirs in k_route_decode (up to the batched router's threshold) or refine
// the batched router's candidates in k_topk
// ---------------------------------------------------------------------------
struct RouterArgs {
    const float* x;         // [T][H] router input
    const float* xe;        // [T][H] expert input (quantized to Q8_0 here)
    const float* w_router;  // [E][ld]
    uint64_t router_ld;
    const float* w_sh_norm; // [H] or null
    int T, H, E, S;
    int n_router_blocks;
    float* logits;          // [T][E+1]
    int8_t* xq_qs;          // [T][H]
    float2* xq_ds;          // [T][H/32]
};

// One 256-thread block per router row (row E is the shared-expert gate
// vector).  Wave w owns float4 chunks c = w + 4i of the row (chunk = 64 float4
// = 256 values); every load is unconditional (clamped index, zeroed weight) so
// a token chunk's loads issue back to back.  Products are exact in f64, summed
// in f64 and rounded once to f32.
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

// Q8_0 quantization of one token row (one wave; lane b handles 32-value
// blocks b, b+64, ...): d = fp16(amax/127), q = rint(x * 127/amax), and the
// block's quant sum for the Q4_0 offset term.  With nw, the row is first
// normalized as RMSNorm writes it: x = (x * nscale) * nw (f32, two roundings).
__device__ __forceinline__ void quant_x_row(const float* xr, int H, int lane, int8_t* qs, float2* ds,
                                            const float* nw = nullptr, float nscale = 1.0f) {
    const int nb = H >> 5;
    for (int b = lane; b < nb; b += 64) {
        const f32x4* src = (const f32x4*)(xr + 32 * b);
        float v[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const f32x4 q = src[i];
            v[4 * i + 0] = q.x; v[4 * i + 1] = q.y; v[4 * i + 2] = q.z; v[4 * i + 3] = q.w;
        }
        if (nw) {
            const f32x4* wsrc = (const f32x4*)(nw + 32 * b);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const f32x4 w4 = wsrc[i];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float u = v[4 * i + k] * nscale;
                    v[4 * i + k] = u * w4[k];
                }
            }
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
        u32x4* dst = (u32x4*)(qs + 32 * b);
        dst[0] = u32x4{packed[0], packed[1], packed[2], packed[3]};
        dst[1] = u32x4{packed[4], packed[5], packed[6], packed[7]};
        ds[b] = make_float2(df, __builtin_bit_cast(float, sum));
    }
}

__device__ __forceinline__ void quant_token_row(const float* x, int H, int t, int lane, int8_t* xq_qs,
                                                float2* xq_ds, const float* nw = nullptr, float nscale = 1.0f) {
    quant_x_row(x + (uint64_t)t * H, H, lane, xq_qs + (uint64_t)t * H, xq_ds + (uint64_t)t * (H >> 5), nw, nscale);
}

// The same Q8_0 quantization of one token row (one wave; lane b handles blocks
// b, b+64, ...), written as the prefill GEMMs' A operand (the quants as exact
// f16 values, the block scales as fp16 bits) and in the int8 layout above (for
// the exact recomputation of uncertain h values).
__device__ void quant_x_row_f16(const float* xr, int H, int lane, _Float16* q, uint16_t* d, int8_t* qs, float2* ds) {
    const int nb = H >> 5;
    for (int b = lane; b < nb; b += 64) {
        const f32x4* src = (const f32x4*)(xr + 32 * b);
        float v[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const f32x4 x = src[i];
            v[4 * i + 0] = x.x; v[4 * i + 1] = x.y; v[4 * i + 2] = x.z; v[4 * i + 3] = x.w;
        }
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) amax = fmaxf(amax, __builtin_fabsf(v[i]));
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        uint32_t w[16], packed[8] = {};
        int sum = 0;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float r0 = __builtin_rintf(v[2 * i] * id), r1 = __builtin_rintf(v[2 * i + 1] * id);
            w[i] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)r0) |
                   ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)r1) << 16);
            const int i0 = (int)r0, i1 = (int)r1;
            sum += i0 + i1;
            packed[i >> 1] |= (((uint32_t)(i0 & 0xff)) | ((uint32_t)(i1 & 0xff) << 8)) << (16 * (i & 1));
        }
        u32x4* dst = (u32x4*)(q + 32 * b);
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[i] = u32x4{w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]};
        const uint32_t dh = f32_to_fp16(amax / 127.0f);
        d[b] = (uint16_t)dh;
        u32x4* qdst = (u32x4*)(qs + 32 * b);
        qdst[0] = u32x4{packed[0], packed[1], packed[2], packed[3]};
        qdst[1] = u32x4{packed[4], packed[5], packed[6], packed[7]};
        ds[b] = make_float2(fp16_to_f32(dh), __builtin_bit_cast(float, sum));
    }
}

// x's f16 quants and scales for the prefill GEMMs, four tokens per block (one wave each).
__global__ __launch_bounds__(256) void k_x_f16(const float* x, int T, int H, _Float16* q, uint16_t* d, int8_t* qs,
                                               float2* ds) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t < T)
        quant_x_row_f16(x + (uint64_t)t * H, H, threadIdx.x & 63, q + (uint64_t)t * H, d + (uint64_t)t * (H >> 5),
                        qs + (uint64_t)t * H, ds + (uint64_t)t * (H >> 5));
}

// Blocks [0, n_router_blocks) compute router rows; any further blocks
// quantize x, four tokens per block.
template <int NCH>
__global__ __launch_bounds__(256) void k_router_quant(RouterArgs a) {
    __shared__ double s_part[4 * kRouterTokChunk];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    if ((int)blockIdx.x < a.n_router_blocks) {
        router_row<NCH>(a, blockIdx.x, (float*)s_part);
        return;
    }
    const int t = (blockIdx.x - a.n_router_blocks) * 4 + wave;
    if (t < a.T) quant_token_row(a.xe, a.H, t, lane, a.xq_qs, a.xq_ds);
}

// ---------------------------------------------------------------------------
// R1': batched router for large token counts: approximate logits from bf16
// MFMAs with a rigorous per-logit error bound; the top-k then recomputes
// exactly every expert the bound cannot rule out.
//
// x = xh + xl + rx and w = wh + wl + rw with xh = bf16(x), xl = bf16(x - xh)
// (round to nearest, 8-bit significands): |rx| <= 2^-16 |x|.  The MFMAs sum
// xh*wh + xh*wl + xl*wh; the dropped terms are <= 3.05 * 2^-16 |x||w| per
// product.  Each 64-wide k step accumulates its 192 products in a fresh f32
// accumulator (error <= 191 * 2^-23 * sum|p|, valid for any summation order
// and rounding no worse than truncation) and is then added in f64.  Summing
// both over k and using sum |x||w| <= |x|_2 |w|_2:
//     |approx - exact| <= 7.2e-5 * |x_t|_2 * |w_e|_2,
// charged as kRouterBoundRel (8e-5, which also covers the f32 norms) plus
// 2^-21 |approx| for the f32 roundings of the logits and of approx +- bound.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kRtTile = 64;          // tokens and experts per router tile
constexpr int kRtK = 64;             // k step
constexpr int kRtLd = kRtK + 8;      // LDS row stride in bf16: conflict-free 16-byte reads
constexpr float kRouterBoundRel = 8.0e-5f;

struct RouterMfmaArgs {
    const float* x;         // [T][H] router input
    const float* xe;        // [T][H] expert input (quantized to Q8_0 by the preparation)
    const float* w;         // [E][ld]
    uint64_t ld;
    int T, H, E;
    int n_etiles, n_tiles;  // router tiles
    float* logits;          // [T][E+1] approximate logits (column E untouched)
    float* bound;           // [T][E]
    int8_t* xq_qs;
    float2* xq_ds;
    _Float16* x_q;          // non-null: the preparation also writes x's f16 quants and scales
    uint16_t* x_d;
    uint16_t* rx;           // [2][T][H] bf16 hi, lo of the router input
    uint16_t* rw;           // [2][E][H] bf16 hi, lo of the router weights
    float* rnorm;           // [T + E]
    // pre-MoE RMSNorm on the fly (norm_w non-null; then x == xe is the residual
    // row): every operand is of (x * scale) * norm_w, scale = 1/sqrtf(mean(x^2)
    // + eps) from the row's sum of squares (x_ssq: its carried partial sums);
    // the scales go to x_scale for the exact refinement
    const float* norm_w;
    float eps;
    const double* x_ssq;    // [T][ssq_parts(H)] or null
    float* x_scale;         // [T]
    int32_t* ecount;        // [kTotalCopies][E] per-expert totals, zeroed here for the top-k blocks to add into
    int ksplit;             // k ranges per tile (1: logits and bounds; 2, 4: f64 partial sums into part)
    double* part;           // [ksplit][T][E] when ksplit > 1
};

// bf16 split of 8 floats (round to nearest both times): hi = bf16(v), lo = bf16(v - hi);
// returns their sum of squares
__device__ float split8(const f32x4 a, const f32x4 b, u32x4& hi, u32x4& lo) {
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const __bf16 h0 = (__bf16)v[2 * i], h1 = (__bf16)v[2 * i + 1];
        const __bf16 l0 = (__bf16)(v[2 * i] - (float)h0), l1 = (__bf16)(v[2 * i + 1] - (float)h1);
        h[i] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
        l[i] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
    }
    hi = u32x4{h[0], h[1], h[2], h[3]};
    lo = u32x4{l[0], l[1], l[2], l[3]};
    float sq = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) sq += v[i] * v[i];
    return sq;
}

// The split of one row (one wave; lane l takes 8-float groups l, l + 64, ...)
// and its f32 norm.
__device__ __forceinline__ float split_row(const float* src, int H, int lane, uint16_t* hi, uint16_t* lo) {
    float sq = 0.0f;
    for (int c = lane; c < (H >> 3); c += 64) {
        const f32x4 a = *(const f32x4*)(src + 8 * c), b = *(const f32x4*)(src + 8 * c + 4);
        u32x4 h, l;
        sq += split8(a, b, h, l);
        *(u32x4*)(hi + 8 * c) = h;
        *(u32x4*)(lo + 8 * c) = l;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sq += __shfl_xor(sq, o, 64);
    return __builtin_sqrtf(sq);
}

typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));

// The Q8_0 of one row (as quant_x_row / quant_x_row_f16: the same quants,
// scales and sums) with coalesced accesses: lanes 8j..8j+7 take block
// 8 i + j, four values each, the block's amax and quant sum over the 8 lanes.
// Writes the f16 quants when q is non-null; with hi non-null also the row's
// bf16 hi/lo split and returns this lane's sum of squares.
__device__ float quant_split_row(const float* xr, int H, int lane, _Float16* q, uint16_t* d, int8_t* qs, float2* ds,
                                 uint16_t* hi, uint16_t* lo, const float* nw = nullptr, float scale = 1.0f) {
#pragma clang fp contract(off)
    const int nb = H >> 5;
    const int sub = lane & 7;
    float sq = 0.0f;
    for (int b0 = 0; b0 < nb; b0 += 8) {
        const int b = b0 + (lane >> 3);
        const int o = 32 * b + 4 * sub;
        f32x4 v = *(const f32x4*)(xr + o);
        if (nw) {  // the RMSNorm output (x * scale) * w, as k_rms_norm writes it
            const f32x4 w4 = *(const f32x4*)(nw + o);
            v = f32x4{(v.x * scale) * w4.x, (v.y * scale) * w4.y, (v.z * scale) * w4.z, (v.w * scale) * w4.w};
        }
        float amax = fmaxf(fmaxf(__builtin_fabsf(v.x), __builtin_fabsf(v.y)), fmaxf(__builtin_fabsf(v.z), __builtin_fabsf(v.w)));
        amax = dpp8_max<kDppQuadXor1>(amax);
        amax = dpp8_max<kDppQuadXor2>(amax);
        amax = dpp8_max<kDppRowHalfMirror>(amax);
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        const float r0 = __builtin_rintf(v.x * id), r1 = __builtin_rintf(v.y * id), r2 = __builtin_rintf(v.z * id),
                    r3 = __builtin_rintf(v.w * id);
        const int i0 = (int)r0, i1 = (int)r1, i2 = (int)r2, i3 = (int)r3;
        int sum = i0 + i1 + i2 + i3;
        sum = dpp8_add<kDppQuadXor1>(sum);
        sum = dpp8_add<kDppQuadXor2>(sum);
        sum = dpp8_add<kDppRowHalfMirror>(sum);
        if (q) {
            const uint32_t w0 = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)r0) |
                                ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)r1) << 16);
            const uint32_t w1 = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)r2) |
                                ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)r3) << 16);
            *(u32x2v*)(q + o) = u32x2v{w0, w1};
        }
        *(uint32_t*)(qs + o) = ((uint32_t)(i0 & 0xff)) | ((uint32_t)(i1 & 0xff) << 8) | ((uint32_t)(i2 & 0xff) << 16) |
                               ((uint32_t)(i3 & 0xff) << 24);
        if (sub == 0) {
            const uint32_t dh = f32_to_fp16(amax / 127.0f);
            if (q) d[b] = (uint16_t)dh;
            ds[b] = make_float2(fp16_to_f32(dh), __builtin_bit_cast(float, sum));
        }
        if (hi) {
            const float vv[4] = {v.x, v.y, v.z, v.w};
            uint32_t hw[2], lw[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const __bf16 h0 = (__bf16)vv[2 * i], h1 = (__bf16)vv[2 * i + 1];
                const __bf16 l0 = (__bf16)(vv[2 * i] - (float)h0), l1 = (__bf16)(vv[2 * i + 1] - (float)h1);
                hw[i] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
                lw[i] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
            }
            *(u32x2v*)(hi + o) = u32x2v{hw[0], hw[1]};
            *(u32x2v*)(lo + o) = u32x2v{lw[0], lw[1]};
            sq += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
    }
    return sq;
}

// Batched-router preparation, one wave per row: blocks [0, ceil(T/4)) take
// tokens (the experts' Q8_0 of x, the router input's split and norm), the
// rest take router rows (split and norm); the first of those also zeroes the
// per-expert totals that the top-k blocks add into.
__global__ __launch_bounds__(256) void k_router_prep(RouterMfmaArgs a) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int ntb = (a.T + 3) / 4;
    if ((int)blockIdx.x < ntb) {
        const int t = (int)blockIdx.x * 4 + wave;
        if (t >= a.T) return;
        uint16_t* hi = a.rx + (uint64_t)t * a.H;
        uint16_t* lo = a.rx + ((uint64_t)a.T + t) * a.H;
        const bool same = a.x == a.xe;  // one pass over the row: quants and the router operand
        float scale = 1.0f;
        if (a.norm_w) {
            const double ssq = a.x_ssq ? ssq_from_parts(a.x_ssq + (uint64_t)t * ssq_parts(a.H), ssq_parts(a.H), lane)
                                       : ssq_row(a.xe + (uint64_t)t * a.H, a.H, lane);
            scale = rms_scale_from_ssq(ssq, a.H, a.eps);
            if (lane == 0) a.x_scale[t] = scale;
        }
        float sq = quant_split_row(a.xe + (uint64_t)t * a.H, a.H, lane, a.x_q ? a.x_q + (uint64_t)t * a.H : nullptr,
                                   a.x_d + (uint64_t)t * (a.H >> 5), a.xq_qs + (uint64_t)t * a.H,
                                   a.xq_ds + (uint64_t)t * (a.H >> 5), same ? hi : nullptr, same ? lo : nullptr,
                                   a.norm_w, scale);
        if (same) {
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) sq += __shfl_xor(sq, o, 64);
            if (lane == 0) a.rnorm[t] = __builtin_sqrtf(sq);
        } else {
            const float n = split_row(a.x + (uint64_t)t * a.H, a.H, lane, hi, lo);
            if (lane == 0) a.rnorm[t] = n;
        }
        return;
    }
    if ((int)blockIdx.x == ntb)
        for (int i = threadIdx.x; i < kTotalCopies * a.E; i += 256) a.ecount[i] = 0;
    const int e = ((int)blockIdx.x - ntb) * 4 + wave;
    if (e >= a.E) return;
    const float n = split_row(a.w + (uint64_t)e * a.ld, a.H, lane, a.rw + (uint64_t)e * a.H,
                              a.rw + ((uint64_t)a.E + e) * a.H);
    if (lane == 0) a.rnorm[a.T + e] = n;
}

// Router tiles of 64 tokens x 64 experts, one 32x32 MFMA tile per wave.  The
// four split operands of each 64-wide k step are loaded straight into LDS
// (NST buffers, issued NST - 1 steps ahead: a fixed 9 loads per wave and step;
// three buffers take 110 KB, one workgroup per CU, two take 74 KB, two per CU).
// Where the tiles alone would not give every CU two workgroups, each tile's k
// steps are split into ksplit ranges on separate workgroups, which write their
// f64 sums; the top-k adds them (in f64, then rounds to f32) and forms the
// bound itself.
constexpr int kRtRowUnits = kRtLd / 8;                   // 16-byte units per LDS row (8 + 1 padding)
constexpr int kRtSlots = 4 * kRtTile * kRtRowUnits;      // per stage
constexpr int kRtDma = kRtSlots / 256;                   // loads per thread and step
static_assert(kRtSlots % 256 == 0 && (kRtTile * kRtRowUnits) % 64 == 0, "router staging slots");
constexpr int kRtStageHalfs = 4 * kRtTile * kRtLd;

template <int NST>
__global__ __launch_bounds__(256) void k_router_mfma(RouterMfmaArgs a) {
    extern __shared__ __align__(16) uint8_t s_dyn[];
    __bf16* s_op = (__bf16*)s_dyn;  // [stage][xh, xl, wh, wl][64][kRtLd]
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // XCD-aware order: blocks are dealt round-robin to the 8 XCDs, so block b
    // takes logical tile (b % 8) * (n/8) + b / 8 and the expert tiles of one
    // token tile run on one XCD and share its L2.
    const int b = blockIdx.x;
    const int nwg = a.n_tiles * a.ksplit;
    const int gk = (nwg & 7) == 0 ? (b & 7) * (nwg >> 3) + (b >> 3) : b;
    const int g = gk / a.ksplit, kp = gk - g * a.ksplit;
    const int t0 = (g / a.n_etiles) * kRtTile;
    const int e0 = (g % a.n_etiles) * kRtTile;
    // this thread's staging slots: slot s = (array, row, unit); unit 8 (the
    // padding) reloads unit 0 into a slot that is never read
    uint32_t soff[kRtDma];       // byte offset of the slot's source from its array base (k step 0)
    const uint16_t* sbase[kRtDma];
#pragma unroll
    for (int i = 0; i < kRtDma; ++i) {
        const int sl = i * 256 + tid;
        const int arr = sl / (kRtTile * kRtRowUnits);
        const int rem = sl - arr * (kRtTile * kRtRowUnits);
        const int r = rem / kRtRowUnits, u = rem - r * kRtRowUnits;
        const bool isx = arr < 2;
        const int row = isx ? min(t0 + r, a.T - 1) : min(e0 + r, a.E - 1);
        // the array is wave-uniform (576 slots per array, a multiple of 64): scalar base
        const uint64_t base =
            (uint64_t)(isx ? a.rx + (uint64_t)(arr & 1) * a.T * a.H : a.rw + (uint64_t)(arr & 1) * a.E * a.H);
        sbase[i] = (const uint16_t*)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(base >> 32)) << 32) |
                                     (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)base));
        soff[i] = (uint32_t)row * (uint32_t)a.H * 2u + (u < 8 ? 16u * u : 0u);
    }
    // this workgroup's k steps [s0, s0 + nstep)
    const int s0 = kp * (a.H / kRtK) / a.ksplit;
    const int nstep = (kp + 1) * (a.H / kRtK) / a.ksplit - s0;
    auto stage = [&](int st) {
        const int stc = s0 + min(st, nstep - 1);  // past the end: a repeat into a buffer that is not read
        __bf16* dst = s_op + (st % NST) * kRtStageHalfs;
#pragma unroll
        for (int i = 0; i < kRtDma; ++i) {
            // the wave's 64 slots are contiguous in LDS: base = the first slot of the wave
            const uint32_t lds = lds_addr(dst) + (uint32_t)(i * 256 + wave * 64) * 16u;
            dma_lds16(sbase[i], soff[i] + (uint32_t)stc * kRtK * 2u, __builtin_amdgcn_readfirstlane(lds));
        }
    };
    double acc64[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) acc64[r] = 0.0;
    const int ms = wave & 1, ns = wave >> 1;
    const int arow = (ms * 32 + (lane & 31)) * kRtLd + (lane >> 5) * 8;
    const int brow = (ns * 32 + (lane & 31)) * kRtLd + (lane >> 5) * 8;
    stage(0);
    if (NST == 3) stage(1);
    for (int st = 0; st < nstep; ++st) {
        __builtin_amdgcn_s_waitcnt(NST == 3 ? kRtDma : 0);  // step st's loads have landed
        __syncthreads();                     // ... for every wave; the buffer read at st - 1 is free
        stage(st + NST - 1);
        const __bf16* op = s_op + (st % NST) * kRtStageHalfs;
        const __bf16* xh = op;
        const __bf16* xl = op + kRtTile * kRtLd;
        const __bf16* wh = op + 2 * kRtTile * kRtLd;
        const __bf16* wl = op + 3 * kRtTile * kRtLd;
        f32x16 acc = {};
#pragma unroll
        for (int s16 = 0; s16 < kRtK / 16; ++s16) {
            const bf16x8 ah = *(const bf16x8*)(xh + arow + 16 * s16);
            const bf16x8 al = *(const bf16x8*)(xl + arow + 16 * s16);
            const bf16x8 bh = *(const bf16x8*)(wh + brow + 16 * s16);
            const bf16x8 bl = *(const bf16x8*)(wl + brow + 16 * s16);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh, acc, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) acc64[r] += (double)acc[r];
    }
    __builtin_amdgcn_s_waitcnt(0);  // the repeated loads past the end have landed
    // D[row][col]: row = 8 (r / 4) + 4 (lane / 32) + r % 4, col = lane % 32
    const int col = ns * 32 + (lane & 31);
    const int e = e0 + col;
    if (a.ksplit > 1) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = t0 + ms * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (t < a.T && e < a.E) a.part[((uint64_t)kp * a.T + t) * a.E + e] = acc64[r];
        }
        return;
    }
    const float nw = a.rnorm[a.T + min(e, a.E - 1)];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int row = ms * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const int t = t0 + row;
        if (t < a.T && e < a.E) {
            const float L = (float)acc64[r];
            const float d = kRouterBoundRel * a.rnorm[t] * nw + 0x1p-21f * __builtin_fabsf(L) + 1e-30f;
            a.logits[(uint64_t)t * (a.E + 1) + e] = L;
            a.bound[(uint64_t)t * a.E + e] = d;
        }
    }
}

// ---------------------------------------------------------------------------
// R2: top-k + softmax + shared gate; per-block histogram and local ranks;
// then (single block, or a second launch) scan + stable scatter.
// ---------------------------------------------------------------------------
struct TopkArgs {
    const float* logits;       // [T][E+1] (approximate on the refined path)
    const float* logit_bound;  // [T][E]   refined path only
    const double* rpart;       // [rsplit][T][E] refined path with rsplit > 1: the router's k-range sums
    const float* rnorm;        // [T + E] ... and the row norms for their bound
    int rsplit;
    const float* x;            // [T][H]   router input: exact logits (refined path), decode router
    const float* xe;           // [T][H]   expert input: its Q8_0 (decode routing launch)
    const float* w_router;     // [E][router_ld]
    uint64_t router_ld;
    const float* w_sh_norm;    // [H] or null
    int T, E, K, S, H;
    const float* norm_w;  // x is normalized on the fly, (x * x_scale[t]) * norm_w (null: not)
    float norm_eps;
    float* x_scale;       // [T] the rows' RMSNorm scales (router block 0 writes them for the table launch)
    const double* x_ssq;  // [T][ssq_parts(H)] x's RMSNorm partial sums, or null (the router sums x itself)
    int quant_rows;       // router launch over token groups: its blocks also write x's Q8_0 ...
    int8_t* xq_qs;        // ... quants [T][H]
    float2* xq_ds;        // ... and {d, sum} [T][H/32]
    int32_t* topk_idx;    // [T][K]
    float* topk_w;        // [T][K]
    float* sh_gate;       // [T]
    int32_t* local_rank;  // [T*K]
    int32_t* hist;        // [nblk + kTotalCopies][E] per top-k block counts (merged top-k) or token masks, then the totals
    uint64_t* jslot;      // [nblk][E] the masked tokens' slots j, four bits each (top_k <= 16)
    int32_t* offsets;     // [E+2]
    int32_t* rows;        // [R]
    int32_t* row_token;   // [R]
    int32_t* pos;         // [T*K]
    int32_t* active;      // [E+1]
    int32_t* expert_slot; // [E]
    int4* slot_info;      // [E+1] {expert, first row, rows, token of first row}
    int4* dslots;         // [E+2] decode slot list (decode routing only, else null)
    unsigned long long* expert_counts;  // optional [E]: per-expert dispatch counts accumulated
    int defer_softmax;    // 1: the selection leaves the softmax to the caller (token_softmax)
    int32_t* counters;    // [0] n_active, [1] n_tiles
    int4* tiles;
    int max_tiles;
    int nblk;             // top-k blocks
    int tpb;              // tokens per top-k block (a wave each): 16, or 8 / 4 where fewer tokens fill the CUs
};

constexpr int kMaxExpertsPerLane = 16;  // E <= 1024
constexpr int kMaxTopK = 64;

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_max_step(float v) {
    const float o = __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), CTRL, ROW_MASK,
                                           0xF, false));
    return fmaxf(v, o);
}

// Whole-wave maximum, returned to every lane.
__device__ __forceinline__ float wave_max_f32(float v) {
    v = dpp_max_step<kDppQuadXor1, 0xF>(v);
    v = dpp_max_step<kDppQuadXor2, 0xF>(v);
    v = dpp_max_step<kDppRowHalfMirror, 0xF>(v);
    v = dpp_max_step<kDppRowMirror, 0xF>(v);
    v = dpp_max_step<kDppRowBcast15, 0xA>(v);
    v = dpp_max_step<kDppRowBcast31, 0xC>(v);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}


__device__ __forceinline__ double dot4_f64(const f32x4 w, const f32x4 v, double acc) {
    acc = __builtin_fma((double)w.x, (double)v.x, acc);
    acc = __builtin_fma((double)w.y, (double)v.y, acc);
    acc = __builtin_fma((double)w.z, (double)v.z, acc);
    return __builtin_fma((double)w.w, (double)v.w, acc);
}

// Exact router logits of one token against NR router rows (one wave; f32
// products are exact in f64, each row's sum is f64 in column order), rounded
// once to f32.  The router input is x itself or, with NORM, the RMSNorm output
// (x * scale) * nw as k_rms_norm writes it.  Each step loads two 256-column
// chunks of x and of every row before any arithmetic (no branch between the
// loads: a step past the last chunk reloads it and multiplies it by x = 0,
// which leaves the f64 sums' bits unchanged, as they are never -0).
template <int NR, bool NORM>
__device__ __forceinline__ void exact_dots(const float* const (&w)[NR], const float* xr, int H, int lane,
                                           float (&r)[NR], const float* nw, float scale) {
#pragma clang fp contract(off)
    double acc[NR];
#pragma unroll
    for (int k = 0; k < NR; ++k) acc[k] = 0.0;
    const int nch = H >> 8;
    for (int c = 0; c < nch; c += 2) {
        f32x4 xv[2], nv[2], v[NR][2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int o = min(c + i, nch - 1) * 256 + 4 * lane;
            xv[i] = *(const f32x4*)(xr + o);
            if (NORM) nv[i] = *(const f32x4*)(nw + o);
#pragma unroll
            for (int k = 0; k < NR; ++k) v[k][i] = *(const f32x4*)(w[k] + o);
        }
        __builtin_amdgcn_sched_barrier(0);  // every load of the step in flight before the arithmetic
#pragma unroll
        for (int i = 0; i < 2; ++i)
            if (NORM)
                xv[i] = f32x4{(xv[i].x * scale) * nv[i].x, (xv[i].y * scale) * nv[i].y, (xv[i].z * scale) * nv[i].z,
                              (xv[i].w * scale) * nv[i].w};
        if (c + 1 >= nch) xv[1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int k = 0; k < NR; ++k) acc[k] = dot4_f64(v[k][i], xv[i], acc[k]);
    }
#pragma unroll
    for (int k = 0; k < NR; ++k) r[k] = (float)wave_sum_f64(acc[k]);
}

// Selection keys: the float's bits mapped to an unsigned order (negative values
// flipped, positive values with the sign bit set) in the high word, ~id in the
// low word, so the larger key is the larger logit and, among equal logits,
// the lower expert id.  Key 0 is below every real entry (no candidate).
__device__ __forceinline__ uint64_t sel_key(float v, int id) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)o << 32) | (uint32_t)~(uint32_t)id;
}
__device__ __forceinline__ int sel_id(uint64_t k) { return (int)~(uint32_t)k; }
__device__ __forceinline__ float sel_val(uint64_t k) {
    const uint32_t o = (uint32_t)(k >> 32);
    return __builtin_bit_cast(float, (o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint64_t dpp_max_u64_step(uint64_t k) {
    const uint32_t lo = (uint32_t)k, hi = (uint32_t)(k >> 32);
    const uint32_t olo = (uint32_t)__builtin_amdgcn_update_dpp((int)lo, (int)lo, CTRL, ROW_MASK, 0xF, false);
    const uint32_t ohi = (uint32_t)__builtin_amdgcn_update_dpp((int)hi, (int)hi, CTRL, ROW_MASK, 0xF, false);
    const uint64_t o = ((uint64_t)ohi << 32) | olo;
    return o > k ? o : k;
}

// Whole-wave maximum key, returned to every lane (branch-free).
__device__ __forceinline__ uint64_t wave_max_key(uint64_t k) {
    k = dpp_max_u64_step<kDppQuadXor1, 0xF>(k);
    k = dpp_max_u64_step<kDppQuadXor2, 0xF>(k);
    k = dpp_max_u64_step<kDppRowHalfMirror, 0xF>(k);
    k = dpp_max_u64_step<kDppRowMirror, 0xF>(k);
    k = dpp_max_u64_step<kDppRowBcast15, 0xA>(k);
    k = dpp_max_u64_step<kDppRowBcast31, 0xC>(k);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(k >> 32), 63);
    return ((uint64_t)hi << 32) | lo;
}

// Whole-wave maximum of a u32 in every lane: four in-row DPP steps (the DPP
// moves fold into the maximum), then the 16- and 32-lane swaps; no scalar
// round trip.
__device__ __forceinline__ uint32_t wave_allmax_u32(uint32_t v) {
#define QMOE_MAXU32_STEP(CTRL) v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false))
    QMOE_MAXU32_STEP(kDppQuadXor1);
    QMOE_MAXU32_STEP(kDppQuadXor2);
    QMOE_MAXU32_STEP(kDppRowHalfMirror);
    QMOE_MAXU32_STEP(kDppRowMirror);
#undef QMOE_MAXU32_STEP
    const auto r16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = max((uint32_t)r16[0], (uint32_t)r16[1]);
    const auto r32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return max((uint32_t)r32[0], (uint32_t)r32[1]);
}

// Softmax over a token's selected logits (s_val_row[0..K-1], slot 0 holds the
// maximum): exps in parallel lanes, the sum in slot order, the divisions in
// parallel lanes; and the shared-expert gate.  One wave.
__device__ void token_softmax(const TopkArgs& a, int t, int lane, const float* s_val_row, double* s_ex_row,
                              float sg_logit) {
#pragma clang fp contract(off)
    const double m = (double)s_val_row[0];
    double ex = 0.0;
    if (lane < a.K) {
        ex = exp_det((double)s_val_row[lane] - m);
        s_ex_row[lane] = ex;
    }
    if (lane == a.K && a.S) a.sh_gate[t] = sigmoid_det(sg_logit);
    wave_lds_sync();
    double sum = 0.0;
    if (lane == 0) {
        for (int j = 0; j < a.K; ++j) sum = sum + s_ex_row[j];
        s_ex_row[kMaxTopK] = sum;
    }
    wave_lds_sync();
    sum = s_ex_row[kMaxTopK];
    if (lane < a.K) a.topk_w[(uint64_t)t * a.K + lane] = (float)(ex / sum);
}

// Top-k of one token from per-lane candidates (expert e = i*64 + lane in
// v[i]/id[i], id INT_MAX for none), softmax over the selected logits and the
// shared-expert gate.  One wave.  Each lane sorts its keys (compare-exchange
// network), then K rounds take the wave maximum of the lanes' heads and the
// winning lane pops its head.
template <int EPL>
__device__ void select_softmax(const TopkArgs& a, int t, int lane, float (&v)[EPL], int (&id)[EPL], float sg_logit,
                               int32_t* s_idx_row, float* s_val_row, double* s_ex_row, float* s_sg) {
    uint64_t key[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) key[i] = id[i] == 0x7fffffff ? 0ull : sel_key(v[i], id[i]);
#pragma unroll
    for (int i = 1; i < EPL; ++i)
#pragma unroll
        for (int j = i; j > 0; --j) {
            const uint64_t hi = key[j - 1] > key[j] ? key[j - 1] : key[j];
            const uint64_t lo = key[j - 1] > key[j] ? key[j] : key[j - 1];
            key[j - 1] = hi;
            key[j] = lo;
        }
    for (int j = 0; j < a.K; ++j) {
        // the largest head: the value word's maximum first; the full keys (lowest
        // expert id among equal values) only when several lanes hold that value
        const uint32_t hi = (uint32_t)(key[0] >> 32);
        bool pop = hi == wave_allmax_u32(hi);
        const uint64_t at = __ballot(pop);
        if (at & (at - 1)) pop = key[0] == wave_max_key(pop ? key[0] : 0ull);  // a value tie: keys are distinct
        if (pop) {  // the winning lane records its head
            const int bi = sel_id(key[0]);
            s_idx_row[j] = bi;
            s_val_row[j] = sel_val(key[0]);
            a.topk_idx[(uint64_t)t * a.K + j] = bi;
        }
        // the pop as one select per key word (element-wise selects of an array
        // get rewritten into an indexed access, a chain of selects per key)
        typedef uint64_t KeyVec __attribute__((ext_vector_type(EPL)));
        KeyVec cur, nxt;
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
            cur[i] = key[i];
            nxt[i] = i + 1 < EPL ? key[i + 1 < EPL ? i + 1 : i] : 0ull;
        }
        cur = pop ? nxt : cur;
#pragma unroll
        for (int i = 0; i < EPL; ++i) key[i] = cur[i];
    }
    // every lane reads what the winning lanes wrote to LDS: order the wave's LDS accesses
    wave_lds_sync();
    if (a.defer_softmax) {
        if (lane == 0 && s_sg) *s_sg = sg_logit;
        return;
    }
    token_softmax(a, t, lane, s_val_row, s_ex_row, sg_logit);
}

// Top-k from exact logits.
template <int EPL>
__device__ void topk_one_token(const TopkArgs& a, int t, int lane, int32_t* s_idx_row, float* s_val_row,
                               double* s_ex_row, float* s_sg) {
    const float* l = a.logits + (uint64_t)t * (a.E + 1);
    float v[EPL];
    int id[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        const int e = i * 64 + lane;
        const float lv = l[min(e, a.E - 1)];  // unconditional load, masked below
        v[i] = e < a.E ? lv : -__builtin_huge_valf();
        id[i] = e < a.E ? e : 0x7fffffff;
    }
    select_softmax<EPL>(a, t, lane, v, id, a.S ? l[a.E] : 0.0f, s_idx_row, s_val_row, s_ex_row, s_sg);
}

// Top-k from approximate logits L~ with bounds d (|L~ - L| <= d): thr = the
// K-th largest lower bound L~ - d is <= the K-th largest exact logit, so every
// expert with L~ + d < thr is strictly below the K-th selected value and
// cannot be selected (whatever the tie rule).  The rest are recomputed
// exactly and ranked as on the exact path; the selection is identical.
template <int EPL, bool NORM>
__device__ void topk_refine_token(const TopkArgs& a, int t, int lane, int32_t* s_idx_row, float* s_val_row,
                                  double* s_ex_row) {
    const float* l = a.logits + (uint64_t)t * (a.E + 1);
    const float* bd = a.logit_bound + (uint64_t)t * a.E;
    float lo[EPL], up[EPL];
    if (a.rsplit > 1) {
        // the router's k-range sums (f64, added in range order), its bound formed here
        double ps[EPL];
        float nw[EPL];
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
            const int ec = min(i * 64 + lane, a.E - 1);
            ps[i] = a.rpart[(uint64_t)t * a.E + ec];
            nw[i] = a.rnorm[a.T + ec];
        }
        for (int p = 1; p < a.rsplit; ++p)
#pragma unroll
            for (int i = 0; i < EPL; ++i)
                ps[i] += a.rpart[((uint64_t)p * a.T + t) * a.E + min(i * 64 + lane, a.E - 1)];
        const float nx = a.rnorm[t];
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
            const int e = i * 64 + lane;
            const float L = (float)ps[i];
            const float d = kRouterBoundRel * nx * nw[i] + 0x1p-21f * __builtin_fabsf(L) + 1e-30f;
            lo[i] = e < a.E ? L - d : -__builtin_huge_valf();
            up[i] = e < a.E ? L + d : -__builtin_huge_valf();
        }
    } else {
#pragma unroll
        for (int i = 0; i < EPL; ++i) {
            const int e = i * 64 + lane;
            const int ec = min(e, a.E - 1);
            const float L = l[ec], d = bd[ec];
            lo[i] = e < a.E ? L - d : -__builtin_huge_valf();
            up[i] = e < a.E ? L + d : -__builtin_huge_valf();
        }
    }
    // K-th largest lower bound (with multiplicity)
    float s[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) s[i] = lo[i];
#pragma unroll
    for (int i = 1; i < EPL; ++i)
#pragma unroll
        for (int j = i; j > 0; --j)
            if (s[j] > s[j - 1]) { const float tv = s[j]; s[j] = s[j - 1]; s[j - 1] = tv; }
    float thr = -__builtin_huge_valf();
    int removed = 0;
    for (int j = 0; j < a.K; ++j) {
        const float mx = wave_max_f32(s[0]);
        const bool pop = s[0] == mx;
        removed += __builtin_popcountll(__ballot(pop));
        if (pop) {
#pragma unroll
            for (int i = 0; i + 1 < EPL; ++i) s[i] = s[i + 1];
            s[EPL - 1] = -__builtin_huge_valf();
        }
        if (removed >= a.K) { thr = mx; break; }
    }
    // exact logits of the candidates and of the shared gate: one queue over
    // every group, eight rows per pass, then four, then two (as the registers
    // allow: eight up to 256 experts, four up to 512)
    const float* xr = a.x + (uint64_t)t * a.H;
    // prefill with the pre-MoE RMSNorm on the fly: x is the residual row
    const float* nw = a.norm_w;
    const float xscale = NORM ? a.x_scale[t] : 1.0f;
    float v[EPL];
    int id[EPL];
    uint64_t mk[EPL];
    int n = a.S ? 1 : 0;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        const int e = i * 64 + lane;
        v[i] = -__builtin_huge_valf();
        id[i] = e < a.E ? e : 0x7fffffff;
        mk[i] = __ballot(e < a.E && up[i] >= thr);
        n += __builtin_popcountll(mk[i]);
    }
    bool sh = a.S != 0;
    float sg = 0.0f;
    // next queue entry: group g (EPL = the shared gate) and lane b
    auto pop = [&](int& g, int& b) {
        g = -1;
        b = 0;
#pragma unroll
        for (int i = 0; i < EPL; ++i)
            if (g < 0 && mk[i]) { g = i; b = __builtin_ctzll(mk[i]); mk[i] &= mk[i] - 1; }
        if (g < 0 && sh) { g = EPL; sh = false; }
    };
    auto row = [&](int g, int b) {
        return g == EPL ? a.w_sh_norm : a.w_router + (uint64_t)(g * 64 + b) * a.router_ld;
    };
    auto put = [&](int g, int b, float r) {
        if (g == EPL) sg = r;
#pragma unroll
        for (int i = 0; i < EPL; ++i)
            if (g == i && lane == b) v[i] = r;
    };
    // eight rows per pass where the registers allow (up to 256 experts)
    for (; EPL <= 4 && n >= 7; n -= 8) {
        int g[8], b[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) pop(g[k], b[k]);
        const float* w[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) w[k] = row(g[k] < 0 ? g[0] : g[k], g[k] < 0 ? b[0] : b[k]);
        float r[8];
        exact_dots<8, NORM>(w, xr, a.H, lane, r, nw, xscale);
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (g[k] >= 0) put(g[k], b[k], r[k]);
    }
    for (; EPL <= 8 && n >= 3; n -= 4) {
        int g[4], b[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) pop(g[k], b[k]);
        const float* w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) w[k] = row(g[k] < 0 ? g[0] : g[k], g[k] < 0 ? b[0] : b[k]);
        float r[4];
        exact_dots<4, NORM>(w, xr, a.H, lane, r, nw, xscale);
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (g[k] >= 0) put(g[k], b[k], r[k]);
    }
    for (; n > 0; n -= 2) {
        int g0, b0, g1, b1;
        pop(g0, b0);
        pop(g1, b1);
        if (g1 < 0) { g1 = g0; b1 = b0; }
        const float* w[2] = {row(g0, b0), row(g1, b1)};
        float r[2];
        exact_dots<2, NORM>(w, xr, a.H, lane, r, nw, xscale);
        put(g0, b0, r[0]);
        put(g1, b1, r[1]);
    }
    select_softmax<EPL>(a, t, lane, v, id, sg, s_idx_row, s_val_row, s_ex_row, nullptr);
}

// s_sg (deferred softmax only): where the shared-gate logit is kept for token_softmax.
// EPL: experts per lane (1, 2, 4, 8 or 16; 0: chosen here from E).
template <bool REFINE, int EPL = 0>
__device__ __forceinline__ void topk_dispatch(const TopkArgs& a, int t, int lane, int32_t* s_idx_row,
                                              float* s_val_row, double* s_ex_row, float* s_sg = nullptr) {
    if constexpr (EPL > 0) {
        if (REFINE) {
            if (a.norm_w) topk_refine_token<EPL, true>(a, t, lane, s_idx_row, s_val_row, s_ex_row);
            else topk_refine_token<EPL, false>(a, t, lane, s_idx_row, s_val_row, s_ex_row);
        }
        else topk_one_token<EPL>(a, t, lane, s_idx_row, s_val_row, s_ex_row, s_sg);
    } else {
        const int epl = (a.E + 63) >> 6;
        if (epl <= 1) topk_dispatch<REFINE, 1>(a, t, lane, s_idx_row, s_val_row, s_ex_row, s_sg);
        else if (epl <= 2) topk_dispatch<REFINE, 2>(a, t, lane, s_idx_row, s_val_row, s_ex_row, s_sg);
        else if (epl <= 4) topk_dispatch<REFINE, 4>(a, t, lane, s_idx_row, s_val_row, s_ex_row, s_sg);
        else if (epl <= 8) topk_dispatch<REFINE, 8>(a, t, lane, s_idx_row, s_val_row, s_ex_row, s_sg);
        else topk_dispatch<REFINE, 16>(a, t, lane, s_idx_row, s_val_row, s_ex_row, s_sg);
    }
}

// Experts per lane of a top-k over E experts: 1, 2, 4, 8 or 16.
static inline int topk_epl(int E) {
    const int epl = (E + 63) >> 6;
    return epl <= 1 ? 1 : epl <= 2 ? 2 : epl <= 4 ? 4 : epl <= 8 ? 8 : 16;
}

__device__ void scan_experts(const TopkArgs& a, const int32_t* s_cnt, const uint32_t* first_token, int32_t* s_off,
                             int32_t* s_misc);

// blockDim = 64 * a.tpb: one wave per token.  Writes the selection and, per
// expert, the mask of the block's tokens that chose it.
// MERGE (blocks x experts <= kTopkMergeMax): the per-block counts and each
// assignment's rank among the block's assignments to the same expert (token
// order) are written through, and the last block to finish (a counter in sync)
// runs the expert scan and the stable scatter.  Otherwise the masks go to hist
// (with the slot j of each token whose mask bit is set, four bits each, in
// jslot when top_k <= 16) and the block adds its counts into the per-expert
// totals (hist's rows from nblk on, zeroed by the router launch) for k_lists.  EPL:
// experts per lane (an instance per expert count class, so each gets its own
// registers).
template <bool REFINE, bool MERGE, int EPL>
__global__ __launch_bounds__(64 * kTopkTokensPerBlock) void k_topk(TopkArgs a, int32_t* sync) {
    __shared__ int32_t s_idx[kTopkTokensPerBlock][kMaxTopK];
    __shared__ float s_val[kTopkTokensPerBlock][kMaxTopK];
    __shared__ double s_ex[kTopkTokensPerBlock][kMaxTopK + 1];
    __shared__ uint32_t s_mask[1024];  // per expert: bit ti set if block token ti chose it
    __shared__ uint64_t s_jslot[MERGE ? 1 : 1024];  // per expert: nibble ti = the slot j of token ti
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int t0 = blockIdx.x * a.tpb;
    const int ntok = min(a.tpb, a.T - t0);
    const bool jslot = !MERGE && a.K <= 16;
    for (int e = threadIdx.x; e < a.E; e += blockDim.x) {
        s_mask[e] = 0;
        if (jslot) s_jslot[e] = 0;
    }
    __syncthreads();
    if (wave < ntok) {
        topk_dispatch<REFINE, EPL>(a, t0 + wave, lane, s_idx[wave], s_val[wave], s_ex[wave]);
        if (lane < a.K) {
            atomicOr(&s_mask[s_idx[wave][lane]], 1u << wave);
            if (jslot) atomicOr((unsigned long long*)&s_jslot[s_idx[wave][lane]], (unsigned long long)lane << (4 * wave));
        }
    }
    __syncthreads();
    if constexpr (MERGE) {
        for (int asg = threadIdx.x; asg < ntok * a.K; asg += blockDim.x) {
            const int ti = asg / a.K;
            const int j = asg % a.K;
            const int ex = s_idx[ti][j];
            const int rank = __builtin_popcount(s_mask[ex] & ((1u << ti) - 1u));
            const uint64_t i = (uint64_t)(t0 + ti) * a.K + j;
            // written through: the last block reads them
            __hip_atomic_store(a.local_rank + i, rank, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(a.topk_idx + i, ex, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    for (int e = threadIdx.x; e < a.E; e += blockDim.x) {
        const uint32_t m = s_mask[e];
        const uint64_t h = (uint64_t)blockIdx.x * a.E + e;
        if constexpr (MERGE) {
            __hip_atomic_store(a.hist + h, (int)__builtin_popcount(m), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            a.hist[h] = (int32_t)m;
            if (m) {
                if (jslot) a.jslot[h] = s_jslot[e];
                __hip_atomic_fetch_add(a.hist + ((uint64_t)a.nblk + blockIdx.x % kTotalCopies) * a.E + e,
                                       (int)__builtin_popcount(m),
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    if constexpr (MERGE) {
        __shared__ int32_t s_base[kTopkMergeMax];  // [block][expert]: the block's first rank in the expert's rows
        __shared__ int32_t s_cnt[1024], s_off[1024], s_misc[64];
        __shared__ int s_last;
        const int tid = threadIdx.x;
        __builtin_amdgcn_s_waitcnt(0);  // this block's write-through stores have completed
        __syncthreads();
        // the counter's add releases this block's stores (barrier, then an
        // agent-scope release by thread 0) and acquires the other blocks'
        if (tid == 0)
            s_last = __hip_atomic_fetch_add(sync + kSyncTopk, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) ==
                     (int)gridDim.x - 1;
        __syncthreads();
        if (!s_last) return;
        if (tid == 0) __hip_atomic_store(sync + kSyncTopk, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // per expert: the blocks' bases (exclusive prefix of their counts) and the total
        for (int e = tid; e < a.E; e += blockDim.x) {
            int run = 0;
            for (int b = 0; b < (int)gridDim.x; ++b) {
                const int c = __hip_atomic_load(a.hist + (uint64_t)b * a.E + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                s_base[b * a.E + e] = run;
                run += c;
            }
            s_cnt[e] = run;
        }
        __syncthreads();
        scan_experts(a, s_cnt, nullptr, s_off, s_misc);
        __syncthreads();
        // the stable scatter: assignment i of expert e to row offsets[e] + its block's
        // base + its rank in the block; the first row's token into the slot table;
        // the shared expert's rows in token order
        const int A = a.T * a.K;
        for (int i = tid; i < A + a.S * a.T; i += blockDim.x) {
            if (i < A) {
                const int t = i / a.K;
                const int ex = __hip_atomic_load(a.topk_idx + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const int off = s_off[ex];
                const int p = off + s_base[(t / a.tpb) * a.E + ex] +
                              __hip_atomic_load(a.local_rank + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                a.rows[p] = i;
                a.row_token[p] = t;
                a.pos[i] = p;
                if (p == off) ((int*)(a.slot_info + a.expert_slot[ex]))[3] = t;
            } else {
                a.rows[i] = -1;
                a.row_token[i] = i - A;
            }
        }
    }
}

// Exclusive scans over experts of the per-expert counts in s_cnt: offsets,
// active slots, expert->slot map, MFMA tiles, counters.  In one block of at
// least E threads rounded to waves (E <= 1024).  first_token (optional, LDS)
// gives the token of each expert's first row; otherwise the scatter sets it.
__device__ void scan_experts(const TopkArgs& a, const int32_t* s_cnt, const uint32_t* first_token,
                             int32_t* s_off, int32_t* s_misc) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int nchunk = (a.E + 63) >> 6;
    int cnt = 0, act = 0, nt = 0, inc = 0, inc_act = 0, inc_t = 0, e = 0;
    if (wave < nchunk) {
        e = wave * 64 + lane;
        cnt = e < a.E ? s_cnt[e] : 0;
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
            if (s_off) s_off[e] = off;
            if (act) {
                const int slot = base_act + inc_act - 1;
                if (a.expert_counts) atomicAdd(a.expert_counts + e, (unsigned long long)cnt);
                a.active[slot] = e;
                a.expert_slot[e] = slot;
                a.slot_info[slot] = make_int4(e, off, cnt, first_token ? (int)__builtin_ctz(first_token[e]) : 0);
                if (a.dslots && first_token) a.dslots[slot] = make_int4(e, off, cnt, (int)first_token[e]);
            }
            const int tb = base_t + inc_t - nt;
            for (int i = 0; i < nt && tb + i < a.max_tiles; ++i)
                a.tiles[tb + i] = make_int4(e, off + i * kMfmaTileM, min(kMfmaTileM, cnt - i * kMfmaTileM), 0);
        }
        if (wave == nchunk - 1 && a.dslots && first_token) {
            // decode slot list: the active routed experts, then "none" up to the
            // most a forward can have (the shared expert is not in it)
            const int n_routed = __builtin_amdgcn_readlane(base_act + inc_act, 63);
            const int max_v = min(a.E, a.T * a.K);
            for (int i = n_routed + lane; i < max_v; i += 64) a.dslots[i] = make_int4(-1, 0, 0, 0);
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
                const int ntt = (a.T + kMfmaTileM - 1) / kMfmaTileM;
                for (int i = 0; i < ntt && n_tiles < a.max_tiles; ++i)
                    a.tiles[n_tiles++] = make_int4(a.E, A + i * kMfmaTileM, min(kMfmaTileM, a.T - i * kMfmaTileM), 0);
            }
            a.counters[0] = n_act;
            a.counters[1] = n_tiles;
            a.counters[kCounterFix] = 0;  // the prefill gate/up's list of uncertain h blocks starts empty
        }
    }
}

// Whole routing for T <= kTopkTokensPerBlock in ONE block of 1024 threads,
// everything in LDS: top-k per token (one wave each), per-expert token masks,
// then wave 0 alone (no further barrier): counts, offsets, active slots (with
// the token of each slot's first row = lowest mask bit), tiles, and the stable
// scatter (rank = earlier tokens in the expert's mask), while the other waves
// run the deferred softmax.  Reads the exact logits from a.logits.
struct SmallRouteLds {
    int32_t idx[kTopkTokensPerBlock][kMaxTopK];
    float val[kTopkTokensPerBlock][kMaxTopK];
    double ex[kTopkTokensPerBlock][kMaxTopK + 1];
    float sg[kTopkTokensPerBlock];  // shared-gate logits (deferred softmax)
    uint32_t mask[1024];
    int32_t off[1024];
};

// The expert scans of scan_experts (same tables) for the masks of at most 32
// tokens, by one wave: lane l takes experts l * epl .. l * epl + epl - 1 in
// order, three wave scans give each lane its bases.  Writes the offsets to
// s_off as well.
static_assert(kTopkTokensPerBlock <= 32, "token masks are 32-bit");
__device__ void scan_experts_wave(const TopkArgs& a, const uint32_t* mask, int32_t* s_off) {
    const int lane = threadIdx.x & 63;
    const int epl = (a.E + 63) >> 6;
    const int e0 = lane * epl, e1 = min(a.E, e0 + epl);
    int c = 0, ac = 0, tc = 0;
    for (int e = e0; e < e1; ++e) {
        const int n = __builtin_popcount(mask[e]);
        c += n;
        ac += n > 0 ? 1 : 0;
        tc += (n + kMfmaTileM - 1) / kMfmaTileM;
    }
    const int ic = wave_incl_scan_i32(c), ia = wave_incl_scan_i32(ac), it = wave_incl_scan_i32(tc);
    int off = ic - c, slot = ia - ac, tile = it - tc;
    for (int e = e0; e < e1; ++e) {
        const uint32_t m = mask[e];
        const int n = __builtin_popcount(m);
        a.offsets[e] = off;
        s_off[e] = off;
        if (n > 0) {
            if (a.expert_counts) atomicAdd(a.expert_counts + e, (unsigned long long)n);
            a.active[slot] = e;
            a.expert_slot[e] = slot;
            a.slot_info[slot] = make_int4(e, off, n, (int)__builtin_ctz(m));
            if (a.dslots) a.dslots[slot] = make_int4(e, off, n, (int)m);
            const int nt = (n + kMfmaTileM - 1) / kMfmaTileM;
            for (int i = 0; i < nt && tile + i < a.max_tiles; ++i)
                a.tiles[tile + i] = make_int4(e, off + i * kMfmaTileM, min(kMfmaTileM, n - i * kMfmaTileM), 0);
            tile += nt;
            ++slot;
        }
        off += n;
    }
    const int A = a.T * a.K;
    const int n_routed = __builtin_amdgcn_readlane(ia, 63);
    if (a.dslots) {
        // decode slot list: the active routed experts, then "none" up to the
        // most a forward can have (the shared expert is not in it)
        const int max_v = min(a.E, A);
        for (int i = n_routed + lane; i < max_v; i += 64) a.dslots[i] = make_int4(-1, 0, 0, 0);
    }
    if (lane == 0) {
        int n_act = n_routed;
        int n_tiles = __builtin_amdgcn_readlane(it, 63);
        a.offsets[a.E] = A;
        a.offsets[a.E + 1] = A + a.S * a.T;
        if (a.S) {
            a.active[n_act] = a.E;
            a.slot_info[n_act] = make_int4(a.E, A, a.T, 0);
            n_act++;
            const int ntt = (a.T + kMfmaTileM - 1) / kMfmaTileM;
            for (int i = 0; i < ntt && n_tiles < a.max_tiles; ++i)
                a.tiles[n_tiles++] = make_int4(a.E, A + i * kMfmaTileM, min(kMfmaTileM, a.T - i * kMfmaTileM), 0);
        }
        a.counters[0] = n_act;
        a.counters[1] = n_tiles;
        a.counters[kCounterFix] = 0;
    }
}

__device__ void route_small_body(const TopkArgs& a, SmallRouteLds& L) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int A = a.T * a.K;
    for (int e = tid; e < a.E; e += blockDim.x) L.mask[e] = 0;
    __syncthreads();
    if (wave < a.T) {
        topk_dispatch<false>(a, wave, lane, L.idx[wave], L.val[wave], L.ex[wave], &L.sg[wave]);
        if (lane < a.K) atomicOr(&L.mask[L.idx[wave][lane]], 1u << wave);
    }
    __syncthreads();
    if (wave == 0) {
        scan_experts_wave(a, L.mask, L.off);
        wave_lds_sync();  // the offsets written by the other lanes
        for (int asg = lane; asg < A; asg += 64) {
            const int t = asg / a.K, j = asg % a.K;
            const int ex = L.idx[t][j];
            const int p = L.off[ex] + __builtin_popcount(L.mask[ex] & ((1u << t) - 1u));
            a.rows[p] = asg;
            a.row_token[p] = t;
            a.pos[asg] = p;
        }
        if (a.S && lane < a.T) {
            a.rows[A + lane] = -1;
            a.row_token[A + lane] = lane;
        }
    } else if (a.defer_softmax) {
        // the softmax of every token on the other waves: off the path from the
        // top-k to the end of the routing
        for (int t = wave - 1; t < a.T; t += 15) token_softmax(a, t, lane, L.val[t], L.ex[t], L.sg[t]);
    }
}

// Decode routing (T <= kTopkTokensPerBlock), two launches.  The router launch:
// block b computes router rows 2b, 2b+1 (row E is the shared-expert gate) for
// all tokens.  Wave (g, p) takes the 256-column slabs p, p+4, ... of both rows
// for the tokens t = g (mod 4), loading its x columns straight from memory
// (each x column once per block); the four partial sums of a (row, token) are
// added in order.  The routing-table launch (after the launch boundary, so no
// workgroup waits on another) runs the whole routing on the exact logits in
// one workgroup while the others compute the shared expert's h or x's Q8_0.
constexpr int kRdRows = 2;                                     // router rows per block
constexpr int kRdGroups = 4;                                   // token groups (t = g mod kRdGroups)
constexpr int kRdParts = 16 / kRdGroups;                       // waves per token group
constexpr int kRdTokSlots = kTopkTokensPerBlock / kRdGroups;   // token slots per wave
constexpr int kRdSlab = 256;        // columns per lane-float4 sweep
constexpr int kMaxRdSlabs = 16;     // decode routing for H <= 4096
// dynamic LDS: block 0's routing tables, the shared-expert blocks' token rows
constexpr int kRdLdsBytes = 96 * 1024;

// Wave sums of N per-lane f64 values at once (reduce-scatter): after the 32-
// and 16-lane swap steps every lane holds N/4 values, of slots
// j + (N/4) * (lane >> 4), and a 16-lane tree completes them (every lane of
// the row ends with the sums).
template <int N>
__device__ __forceinline__ void wave_sum_rs_f64(const double (&v)[N], double (&out)[N / 4]) {
    static_assert(N >= 4 && N % 4 == 0, "slots");
    double h[N / 2];
#pragma unroll
    for (int i = 0; i < N / 2; ++i) h[i] = swap_add_f64<32>(v[i], v[i + N / 2]);
#pragma unroll
    for (int i = 0; i < N / 4; ++i) out[i] = dpp_sum_f64<16>(swap_add_f64<16>(h[i], h[i + N / 4]));
}

static_assert(sizeof(SmallRouteLds) <= kRdLdsBytes, "the routing tables fit the dynamic LDS");
static_assert(kTopkTokensPerBlock * (kMaxRdSlabs * kRdSlab * 5 / 4 + 32 * 8) <= kRdLdsBytes,
              "the shared-expert blocks' token rows fit the dynamic LDS");

// Shared expert at decode: its gate/up, SwiGLU and Q8_0 of h do not depend on
// the routing, so blocks after the router blocks compute them meanwhile on
// otherwise idle CUs.  Block j takes ffn rows 32*(j % nfb) .. +32 (one Q8_0
// block of h) for tokens tpg*(j / nfb) .. +tpg: it quantizes those x rows into
// LDS (quant_x_row, as the router blocks do for the workspace), computes g and
// u with one wave per RPW rows, then 32 lanes per token do silu(g)*u and the
// block's Q8_0 (swiglu_q8_block32, as the routed experts) into h rows T*K + t.
struct SharedGuArgs {
    const uint8_t* w_gate; const uint8_t* w_up;  // shared expert gate/up [F] rows
    uint64_t gate_nb1, up_nb1;
    int F;
    int n_blocks;  // shared-expert blocks after the router blocks (0: none)
    int tpg;       // tokens per block
    int8_t* hq_qs; float2* hq_ds;
    int act; const uint16_t* gelu_tab;  // the layer's activation
};

template <int WT, int LPR>
__device__ __forceinline__ void shared_gateup_block(const TopkArgs& a, const SharedGuArgs& sg, int j, uint8_t* s_dyn,
                                                    int8_t* xq_qs, float2* xq_ds) {
#pragma clang fp contract(off)
    constexpr int RPI = 64 / LPR;
    constexpr int RPW = RPI > 2 ? RPI : 2;  // ffn rows per wave
    constexpr int NI = RPW / RPI;
    constexpr int NWA = 32 / RPW;           // waves with rows (of 16)
    const int nfb = sg.F >> 5;
    const int fb = j % nfb, t0 = (j / nfb) * sg.tpg;
    const int nt = min(sg.tpg, a.T - t0);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int sub = lane / LPR, lp = lane % LPR;
    const int pair = min(lp, (a.H >> 6) - 1);
    const bool live = lp < (a.H >> 6);
    WPair<WT> wg[NI], wu[NI];
    if (wave < NWA) {
#pragma unroll
        for (int m = 0; m < NI; ++m) {
            const int f = fb * 32 + wave * RPW + m * RPI + sub;
            wg[m].load(sg.w_gate + (uint64_t)f * sg.gate_nb1, pair);
            wu[m].load(sg.w_up + (uint64_t)f * sg.up_nb1, pair);
        }
    }
    int8_t* lq = (int8_t*)s_dyn;                              // [tpg][H] quants
    float2* ld = (float2*)(lq + (size_t)sg.tpg * a.H);        // [tpg][H/32] {d, sum}
    float2* lgu = ld + (size_t)sg.tpg * (a.H >> 5);           // [tpg][32] (g, u)
    if (wave < nt)
        quant_x_row(a.xe + (uint64_t)(t0 + wave) * a.H, a.H, lane, lq + (size_t)wave * a.H,
                    ld + (size_t)wave * (a.H >> 5), a.norm_w, a.norm_w ? a.x_scale[t0 + wave] : 1.0f);
    __syncthreads();
    if (fb == 0) {
        // the workspace copy of these tokens' Q8_0 rows (the routed experts read it),
        // so the router blocks raise their flags without quantizing
        const int cq = a.H >> 4, cd = a.H >> 6;  // 16-byte chunks per row: quants, {d, sum} pairs
        for (int i = tid; i < nt * (cq + cd); i += blockDim.x) {
            const int c = i / (cq + cd), k = i - c * (cq + cd);
            if (k < cq)
                ((u32x4*)(xq_qs + (uint64_t)(t0 + c) * a.H))[k] = ((const u32x4*)(lq + (size_t)c * a.H))[k];
            else
                ((u32x4*)(xq_ds + (uint64_t)(t0 + c) * (a.H >> 5)))[k - cq] =
                    ((const u32x4*)(ld + (size_t)c * (a.H >> 5)))[k - cq];
        }
    }
    if (wave < NWA) {
        for (int c = 0; c < nt; ++c) {
            XPair x;
            x.load(lq + (size_t)c * a.H, ld + (size_t)c * (a.H >> 5), pair);
#pragma unroll
            for (int m = 0; m < NI; ++m) {
                double g, u;
                group_sum2_f64<LPR>(live ? pair_dot<WT>(wg[m], x) : 0.0, live ? pair_dot<WT>(wu[m], x) : 0.0, g, u);
                float2& o = lgu[c * 32 + wave * RPW + m * RPI + sub];
                if constexpr (LPR >= 32) {
                    if (lp == LPR / 2 - 1) o.x = (float)g;
                    if (lp == LPR - 1) o.y = (float)u;
                } else {
                    if (lp == LPR - 1) o = make_float2((float)g, (float)u);
                }
            }
        }
    }
    __syncthreads();
    if (tid < nt * 32) {
        const int c = tid >> 5, fl = tid & 31;
        const float2 gu = lgu[c * 32 + fl];
        const uint64_t p = (uint64_t)a.T * a.K + t0 + c;
        swiglu_q8_block32(gu.x, gu.y, fl, sg.hq_qs + p * sg.F + fb * 32, sg.hq_ds + p * nfb + fb, sg.act, sg.gelu_tab);
    }
}

// NORM (H <= 2048: a wave's slabs are one load pair): x is the residual row.
// The rows' RMSNorm scales come from the x values loaded for the dots: a 256-
// column slab is one 64-run chunk of the order every RMSNorm here uses (lane i
// holds run 64 slab + i), so each wave takes its slabs' chunk trees for its
// tokens (dpp_sum_f64<64>), the chunk sums meet in LDS, and each wave forms its
// tokens' scales (the tree over the chunks; the same bits in every block and in
// the standalone RMSNorm).  Block 0 stores them for the table launch's Q8_0 of
// x; the router input is (x * scale) * norm_w.
template <int NSW, bool NORM, int RR = kRdRows>  // NSW: router slabs per wave (ceil(H/256/4)); RR: rows per block
__global__ __launch_bounds__(1024) void k_route_decode(TopkArgs a0, float* logits0) {
#pragma clang fp contract(off)
    constexpr int RVALS = RR * kRdTokSlots;  // (row, token) sums per wave
    __shared__ double s_part[RR][kRdParts][kTopkTokensPerBlock];
    __shared__ double s_chunk[NORM ? kTopkTokensPerBlock : 1][8];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    static_assert(!NORM || NSW <= 2, "the fused norm takes rows of at most 8 slabs");
    // more than 16 tokens run in groups of 16: workgroup b takes router rows of
    // block b % nbr for the tokens of group b / nbr; with quant_rows, router block
    // rb of a group also writes the Q8_0 rows of its tokens rb + nbr * w (at the end)
    const int nbr = (a0.E + a0.S + RR - 1) / RR;
    const int gi = (int)blockIdx.x / nbr, rb = (int)blockIdx.x - gi * nbr;
    const int tb = gi * kTopkTokensPerBlock;
    if (a0.quant_rows && blockIdx.x == 0)  // the per-expert totals that the top-k blocks add into
        for (int i = tid; i < kTotalCopies * a0.E; i += 1024) a0.hist[(uint64_t)a0.nblk * a0.E + i] = 0;
    TopkArgs a = a0;  // this group's tokens
    a.T = min(kTopkTokensPerBlock, a0.T - tb);
    a.x = a0.x + (uint64_t)tb * a0.H;
    a.x_scale = a0.x_scale + tb;
    if (a0.x_ssq) a.x_ssq = a0.x_ssq + (uint64_t)tb * ssq_parts(a0.H);
    float* logits = logits0 + (uint64_t)tb * (a0.E + 1);
    const int E1 = a.E + a.S;
    const int nslab = a.H / kRdSlab;
    const int part = wave % kRdParts;
    auto router_row = [&](int e) {
        return e < a.E ? a.w_router + (uint64_t)min(e, a.E - 1) * a.router_ld : (a.S ? a.w_sh_norm : a.w_router);
    };
    const int grp = wave / kRdParts;
    const int e0 = rb * RR;
    double acc[RVALS];  // [row q][i]: token kRdGroups * i + grp
#pragma unroll
    for (int k = 0; k < RVALS; ++k) acc[k] = 0.0;
    // two slabs at a time: every load of the pair issued before its FMAs (the
    // first pair's before the RMSNorm scales, whose row loads then overlap them)
    constexpr int kPair = NSW > 1 ? 2 : 1;
    f32x4 w[kPair][RR], xv[kPair][kRdTokSlots], wn[kPair];
    float xs[kRdTokSlots];  // NORM: the RMSNorm scales of this wave's tokens
    auto load_pair = [&](int s0) {
#pragma unroll
        for (int u = 0; u < kPair; ++u) {
            const int c = min(part + kRdParts * (s0 + u), nslab - 1);  // this wave's slab (clamped)
#pragma unroll
            for (int q = 0; q < RR; ++q)
                w[u][q] = *(const f32x4*)(router_row(e0 + q) + c * kRdSlab + 4 * lane);
            if constexpr (NORM) wn[u] = *(const f32x4*)(a.norm_w + c * kRdSlab + 4 * lane);
#pragma unroll
            for (int i = 0; i < kRdTokSlots; ++i)
                if (kRdGroups * i + grp < a.T)
                    xv[u][i] = *(const f32x4*)(a.x + (uint64_t)(kRdGroups * i + grp) * a.H + c * kRdSlab + 4 * lane);
        }
    };
    auto compute_pair = [&](int s0) {
#pragma unroll
        for (int u = 0; u < kPair; ++u) {
            if (s0 + u >= NSW || e0 >= E1 || part + kRdParts * (s0 + u) >= nslab) continue;  // uniform
#pragma unroll
            for (int i = 0; i < kRdTokSlots; ++i) {
                if (kRdGroups * i + grp < a.T) {
                    f32x4 xx = xv[u][i];
                    if constexpr (NORM) {
                        const float sc = xs[i];
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const float v = xx[k] * sc;
                            xx[k] = v * wn[u][k];
                        }
                    }
                    const double x0 = xx.x, x1 = xx.y, x2 = xx.z, x3 = xx.w;
#pragma unroll
                    for (int q = 0; q < RR; ++q) {
                        double& d = acc[q * kRdTokSlots + i];
                        d = __builtin_fma((double)w[u][q].x, x0, d);
                        d = __builtin_fma((double)w[u][q].y, x1, d);
                        d = __builtin_fma((double)w[u][q].z, x2, d);
                        d = __builtin_fma((double)w[u][q].w, x3, d);
                    }
                }
            }
        }
    };
    // x's RMSNorm partial sums when the caller has them (one per lane, loaded
    // ahead of the slabs): each wave finishes its tokens' trees itself
    // x's partial sums (NORM with x_ssq): lane l takes entries 8j .. 8j+7
    // (j = l & 7) of slot l >> 3, so that one pass of 8-lane trees covers every
    // slot (a row has at most 64 entries: n_embd <= 2048, a multiple of 256)
    f64x2 pq[NORM ? 4 : 1];
    const int np = ssq_parts(a.H);
    const int qs = min(lane >> 3, kRdTokSlots - 1), qj = lane & 7;
    const int qt = kRdGroups * qs + grp;
    if constexpr (NORM) {
        if (a.x_ssq) {  // clamped addresses, masked where the sums are taken
            const f64x2* src = (const f64x2*)(a.x_ssq + (uint64_t)min(qt, a.T - 1) * np + 8 * min(qj, np / 8 - 1));
#pragma unroll
            for (int k = 0; k < 4; ++k) pq[k] = src[k];
        }
    }
    load_pair(0);
    if constexpr (NORM) {
      if (a.x_ssq) {
        // the adjacent-pairs tree of the entries: 8 in registers, then the 8
        // lanes of a slot; one divide and square-root chain for all the slots
        double s = ((pq[0].x + pq[0].y) + (pq[1].x + pq[1].y)) + ((pq[2].x + pq[2].y) + (pq[3].x + pq[3].y));
        s = (lane >> 3) < kRdTokSlots && qt < a.T && 8 * qj < np ? s : 0.0;
        s = dpp_sum_f64<8>(s);
        const float sc = rms_scale_from_ssq(s, a.H, a.norm_eps);
#pragma unroll
        for (int i = 0; i < kRdTokSlots; ++i)
            xs[i] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sc), 8 * i));
      } else {
#pragma unroll
        for (int u = 0; u < kPair; ++u) {
            const int c = part + kRdParts * u;  // slab = chunk
            if (c >= nslab) continue;           // uniform
#pragma unroll
            for (int i = 0; i < kRdTokSlots; ++i) {
                const int t = kRdGroups * i + grp;
                if (t >= a.T) continue;  // uniform
                double run = 0.0;        // run 64 c + lane: its four columns in order
#pragma unroll
                for (int k = 0; k < 4; ++k) run += (double)(xv[u][i][k] * xv[u][i][k]);
                const double cs = dpp_sum_f64<64>(run);
                if (lane == 63) s_chunk[t][c] = cs;
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kRdTokSlots; ++i) {
            const int t = kRdGroups * i + grp;
            xs[i] = 1.0f;
            if (t >= a.T) continue;
            double cv[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) cv[k] = k < nslab ? s_chunk[t][k] : 0.0;
#pragma unroll
            for (int w2 = 4; w2 >= 1; w2 >>= 1)
#pragma unroll
                for (int k = 0; k < w2; ++k) cv[k] = cv[2 * k] + cv[2 * k + 1];
            xs[i] = rms_scale_from_ssq(cv[0], a.H, a.norm_eps);
        }
      }
    }
    compute_pair(0);
#pragma unroll
    for (int s0 = 2; s0 < NSW; s0 += 2) {
        if (part + kRdParts * s0 >= nslab) break;  // uniform: no slab left for this wave
        load_pair(s0);
        compute_pair(s0);
    }
    // wave sums of the (row, token) values: one reduce-scatter, a fixed cost
    // below the trees of 6 steps per live value (each slot's sum in the same
    // order for any row count)
    {
        double sums[RVALS / 4];
        wave_sum_rs_f64<RVALS>(acc, sums);
        const int j = lane & 15, k = j + (RVALS / 4) * (lane >> 4);
        const int t = kRdGroups * (k % kRdTokSlots) + grp;
        double v = sums[0];
#pragma unroll
        for (int m = 1; m < RVALS / 4; ++m) v = j == m ? sums[m] : v;
        if (j < RVALS / 4 && t < a.T) s_part[k / kRdTokSlots][part][t] = v;
    }
    __syncthreads();
    if (tid < RR * a.T) {
        const int rr = tid / a.T, t = tid % a.T;
        const int er = e0 + rr;
        if (er < E1) {
            double sum = s_part[rr][0][t];
#pragma unroll
            for (int q = 1; q < kRdParts; ++q) sum = sum + s_part[rr][q][t];
            logits[(uint64_t)t * (a.E + 1) + er] = (float)sum;
        }
    }
    // the scales for the table launch's quantization of x (after every load)
    if constexpr (NORM) {
        if (rb == 0 && part == 0 && lane == 0)
#pragma unroll
            for (int i = 0; i < kRdTokSlots; ++i)
                if (kRdGroups * i + grp < a.T) a.x_scale[kRdGroups * i + grp] = xs[i];
    }
    if (a0.quant_rows) {  // wave w: the group's token rb + nbr * w (at most one per block when nbr >= 16)
        const int t = rb + nbr * wave;
        if (t < a.T) quant_token_row(a0.xe, a0.H, tb + t, lane, a0.xq_qs, a0.xq_ds);
    }
}

// Decode routing on the router launch's logits (complete and visible at the
// launch boundary): workgroup 0 runs the top-k, softmax, counts, scan and the
// row and slot tables; the other workgroups meanwhile compute the shared
// expert's h (SWT: its weight type) or, without one, x's Q8_0 (one wave per token).
template <int SWT, int SLPR>
__global__ __launch_bounds__(1024) void k_route_decode_tables(TopkArgs a, int8_t* xq_qs, float2* xq_ds, SharedGuArgs sg) {
    extern __shared__ __align__(16) uint8_t s_dyn[];
    if (blockIdx.x == 0) {
        route_small_body(a, *(SmallRouteLds*)s_dyn);
        return;
    }
    if constexpr (SWT != 0) {
        shared_gateup_block<SWT, SLPR>(a, sg, blockIdx.x - 1, s_dyn, xq_qs, xq_ds);
    } else {
        const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
        if (wave < a.T)
            quant_token_row(a.xe, a.H, wave, lane, xq_qs, xq_ds, a.norm_w, a.norm_w ? a.x_scale[wave] : 1.0f);
    }
}

// The expert lists from the top-k blocks' token masks, one workgroup per
// expert and one more (index E) for the shared expert's rows and the totals.
// The top-k blocks added their counts into the per-expert totals, so each
// workgroup finds its expert's first row, active slot and first tile by
// summing the totals below it, and none waits for another.  It then scans its
// column of masks (threads own consecutive blocks) and writes the expert's rows
// in token order: the same offsets, slots, tiles, rows and positions as
// scan_experts followed by the stable scatter.
constexpr int kListThreads = 256;
constexpr int kListRegs = 4;  // masks per thread held in registers (nblk <= 1024); beyond, loaded twice

__global__ __launch_bounds__(kListThreads) void k_lists(TopkArgs a) {
    __shared__ int32_t s_red[3][kListThreads / 64];
    __shared__ int32_t s_wtot[kListThreads / 64];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int e = (int)blockIdx.x;
    const bool routed = e < a.E;
    const uint32_t* masks = (const uint32_t*)a.hist;
    const int32_t* total = a.hist + (uint64_t)a.nblk * a.E;
    const bool jslot = a.K <= 16;
    const int per = (a.nblk + kListThreads - 1) / kListThreads;
    const int b0 = min(a.nblk, tid * per), b1 = min(a.nblk, b0 + per);
    // this thread's masks (and slots), issued with the totals' loads
    uint32_t mk[kListRegs];
    uint64_t js[kListRegs];
#pragma unroll
    for (int i = 0; i < kListRegs; ++i) {
        mk[i] = 0;
        js[i] = 0;
        if (routed && b0 + i < b1) {
            const uint64_t h = (uint64_t)(b0 + i) * a.E + e;
            mk[i] = masks[h];
            if (jslot) js[i] = a.jslot[h];
        }
    }
    // rows, active experts and tiles of the experts below e (all of them for e = E)
    int below = 0, below_act = 0, below_t = 0;
    for (int i = tid; i < a.E; i += kListThreads) {
        int cp[kTotalCopies];
#pragma unroll
        for (int r = 0; r < kTotalCopies; ++r) cp[r] = total[r * a.E + i];
        int c = 0;
#pragma unroll
        for (int r = 0; r < kTotalCopies; ++r) c += cp[r];
        if (i < e) {
            below += c;
            below_act += c > 0 ? 1 : 0;
            below_t += (c + kMfmaTileM - 1) / kMfmaTileM;
        }
    }
    int here = 0;
#pragma unroll
    for (int i = 0; i < kListRegs; ++i) here += __builtin_popcount(mk[i]);
    if (routed)
        for (int b = b0 + kListRegs; b < b1; ++b) here += __builtin_popcount(masks[(uint64_t)b * a.E + e]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        below += __shfl_xor(below, o, 64);
        below_act += __shfl_xor(below_act, o, 64);
        below_t += __shfl_xor(below_t, o, 64);
    }
    const int inc = wave_incl_scan_i32(here);
    if (lane == 63) s_wtot[wave] = inc;
    if (lane == 0) {
        s_red[0][wave] = below;
        s_red[1][wave] = below_act;
        s_red[2][wave] = below_t;
    }
    __syncthreads();
    int off = 0, slot = 0, tb = 0, wbase = 0, cnt = 0;
#pragma unroll
    for (int w = 0; w < kListThreads / 64; ++w) {
        off += s_red[0][w];
        slot += s_red[1][w];
        tb += s_red[2][w];
        wbase += w < wave ? s_wtot[w] : 0;
        cnt += s_wtot[w];
    }
    if (!routed) {
        // the shared expert's rows in token order, the slot and tile totals, the counters
        const int A = a.T * a.K;
        if (a.S)
            for (int t = tid; t < a.T; t += kListThreads) {
                a.rows[A + t] = -1;
                a.row_token[A + t] = t;
            }
        if (tid == 0) {
            int n_act = slot, n_tiles = tb;
            a.offsets[a.E] = A;
            a.offsets[a.E + 1] = A + a.S * a.T;
            if (a.S) {
                a.active[n_act] = a.E;
                a.slot_info[n_act] = make_int4(a.E, A, a.T, 0);
                n_act++;
                const int ntt = (a.T + kMfmaTileM - 1) / kMfmaTileM;
                for (int i = 0; i < ntt && n_tiles < a.max_tiles; ++i)
                    a.tiles[n_tiles++] = make_int4(a.E, A + i * kMfmaTileM, min(kMfmaTileM, a.T - i * kMfmaTileM), 0);
            }
            a.counters[0] = n_act;
            a.counters[1] = n_tiles;
            a.counters[kCounterFix] = 0;  // the prefill gate/up's list of uncertain h blocks starts empty
        }
        return;
    }
    if (tid == 0) a.offsets[e] = off;
    if (cnt == 0) return;
    const int nt = (cnt + kMfmaTileM - 1) / kMfmaTileM;
    for (int i = tid; i < nt && tb + i < a.max_tiles; i += kListThreads)
        a.tiles[tb + i] = make_int4(e, off + i * kMfmaTileM, min(kMfmaTileM, cnt - i * kMfmaTileM), 0);
    if (tid == 0) {
        a.active[slot] = e;
        a.expert_slot[e] = slot;
        if (a.expert_counts) atomicAdd(a.expert_counts + e, (unsigned long long)cnt);
    }
    // this thread's rows start after the rows of the blocks before its own
    int p = off + wbase + inc - here;
    auto put = [&](int b, uint32_t m, uint64_t jw) {
        while (m) {
            const int ti = __builtin_ctz(m);
            m &= m - 1;
            const int t = b * a.tpb + ti;
            int j = (int)((jw >> (4 * ti)) & 15u);
            if (!jslot) {  // top_k > 16: find e in the token's selection
                const int32_t* ir = a.topk_idx + (uint64_t)t * a.K;
                for (int j0 = 0; j0 < a.K; j0 += 8) {
                    int v[8];
#pragma unroll
                    for (int q = 0; q < 8; ++q) v[q] = ir[min(j0 + q, a.K - 1)];
#pragma unroll
                    for (int q = 0; q < 8; ++q)
                        if (j0 + q < a.K && v[q] == e) j = j0 + q;
                }
            }
            const int i = t * a.K + j;
            if (p == off) a.slot_info[slot] = make_int4(e, off, cnt, t);
            a.rows[p] = i;
            a.row_token[p] = t;
            a.pos[i] = p;
            ++p;
        }
    };
#pragma unroll
    for (int i = 0; i < kListRegs; ++i) put(b0 + i, mk[i], js[i]);
    for (int b = b0 + kListRegs; b < b1; ++b) {
        const uint64_t h = (uint64_t)b * a.E + e;
        put(b, masks[h], jslot ? a.jslot[h] : 0);
    }
}

bool route_uses_mfma(const LayerDesc& L, int T) {
    return T > kTopkTokensPerBlock && T >= L.big_router_min_tokens;
}

bool route_decode_fused(const LayerDesc& L, int T) {
    return !route_uses_mfma(L, T) && T <= kTopkTokensPerBlock && L.H <= kMaxRdSlabs * kRdSlab;
}

// The decode router instance for nsw slabs per wave; the routing-table launch
// for shared-expert type swt (0 none, 1 Q4_0, 2 Q8_0) and the shared blocks'
// lanes per row (16 for H <= 1024, 32 for H <= 2048, else 64).
template <bool REFINE, bool MERGE>
static const void* topk_kernel(int E) {
    switch (topk_epl(E)) {
        case 1: return (const void*)k_topk<REFINE, MERGE, 1>;
        case 2: return (const void*)k_topk<REFINE, MERGE, 2>;
        case 4: return (const void*)k_topk<REFINE, MERGE, 4>;
        case 8: return (const void*)k_topk<REFINE, MERGE, 8>;
        default: return (const void*)k_topk<REFINE, MERGE, 16>;
    }
}

static hipError_t launch_topk(const void* kern, TopkArgs& ta, int32_t* sync, hipStream_t stream) {
    void* args[] = {&ta, &sync};
    hipError_t err = hipLaunchKernel(kern, dim3(ta.nblk), dim3(64 * ta.tpb), args, 0, stream);
    return err != hipSuccess ? err : hipGetLastError();
}

static const void* route_decode_kernel(int nsw, bool norm) {
    static_assert(kRdParts == 4, "slabs per wave: 1 at H <= 1024, 2 at H <= 2048, 3-4 at H <= 4096");
    if (norm) return nsw == 1 ? (const void*)k_route_decode<1, true> : nsw == 2 ? (const void*)k_route_decode<2, true> : nullptr;
    switch (nsw) {
        case 1: return (const void*)k_route_decode<1, false>;
        case 2: return (const void*)k_route_decode<2, false>;
        case 3: return (const void*)k_route_decode<3, false>;
        case 4: return (const void*)k_route_decode<4, false>;
        default: return nullptr;
    }
}
// The router over groups of 16 tokens: five rows per block for rows of at most
// 2048 columns (a 256-expert layer's 52 blocks per group fill the CUs in one
// round up to 64 tokens), two for wider rows (five would spill registers).
static const void* route_group_kernel(int nsw, int* rows) {
    *rows = nsw <= 2 ? 5 : kRdRows;
    switch (nsw) {
        case 1: return (const void*)k_route_decode<1, false, 5>;
        case 2: return (const void*)k_route_decode<2, false, 5>;
        case 3: return (const void*)k_route_decode<3, false>;
        case 4: return (const void*)k_route_decode<4, false>;
        default: return nullptr;
    }
}
template <int SLPR>
static const void* route_tables_for(int swt) {
    return swt == 0 ? (const void*)k_route_decode_tables<0, SLPR>
                    : swt == 1 ? (const void*)k_route_decode_tables<kTypeQ4_0, SLPR>
                               : (const void*)k_route_decode_tables<kTypeQ8_0, SLPR>;
}
static const void* route_tables_kernel(int swt, int lpr) {
    return lpr == 16 ? route_tables_for<16>(swt) : lpr == 32 ? route_tables_for<32>(swt) : route_tables_for<64>(swt);
}

static hipError_t launch_router_exact(const LayerDesc& L, const Workspace& ws, const float* xr, const float* xe, int T,
                                      bool quant, hipStream_t stream) {
    RouterArgs ra;
    ra.x = xr;
    ra.xe = xe;
    ra.w_router = L.w_router;
    ra.router_ld = L.router_ld;
    ra.w_sh_norm = L.w_sh_norm;
    ra.T = T; ra.H = L.H; ra.E = L.E; ra.S = L.S;
    ra.logits = ws.logits;
    ra.xq_qs = ws.xq_qs;
    ra.xq_ds = ws.xq_ds;
    ra.n_router_blocks = L.E + L.S;
    const int nq = quant ? (T + 3) / 4 : 0;
    const dim3 grid(ra.n_router_blocks + nq);
    const int nch_per_wave = (L.H / 256 + 3) / 4;  // float4 chunks of 256 values per wave
    if (nch_per_wave <= 1) hipLaunchKernelGGL((k_router_quant<1>), grid, dim3(256), 0, stream, ra);
    else if (nch_per_wave <= 2) hipLaunchKernelGGL((k_router_quant<2>), grid, dim3(256), 0, stream, ra);
    else if (nch_per_wave <= 4) hipLaunchKernelGGL((k_router_quant<4>), grid, dim3(256), 0, stream, ra);
    else hipLaunchKernelGGL((k_router_quant<8>), grid, dim3(256), 0, stream, ra);
    return hipGetLastError();
}

static hipError_t launch_route_tables(const LayerDesc& L, const Workspace& ws, const float* x, const float* xr, int T,
                                      const RouteDebug& dbg, bool& x_f16, hipStream_t stream, const float* norm_w,
                                      float eps, const double* x_ssq) {
    TopkArgs ta;
    ta.norm_w = nullptr;
    ta.x_ssq = nullptr;
    ta.quant_rows = 0;
    ta.xq_qs = ws.xq_qs;
    ta.xq_ds = ws.xq_ds;
    ta.norm_eps = eps;
    ta.x_scale = ws.x_scale;
    ta.logits = ws.logits;
    ta.logit_bound = ws.logit_bound;
    ta.rpart = nullptr;
    ta.rnorm = ws.rnorm;
    ta.rsplit = 1;
    ta.x = xr;
    ta.xe = x;
    ta.w_router = L.w_router;
    ta.router_ld = L.router_ld;
    ta.w_sh_norm = L.w_sh_norm;
    ta.T = T; ta.E = L.E; ta.K = L.K; ta.S = L.S; ta.H = L.H;
    ta.topk_idx = ws.topk_idx;
    ta.topk_w = ws.topk_w;
    ta.sh_gate = ws.sh_gate;
    ta.local_rank = ws.local_rank;
    ta.hist = ws.hist;
    ta.jslot = ws.jslot;
    ta.offsets = ws.offsets;
    ta.rows = ws.rows;
    ta.row_token = ws.row_token;
    ta.pos = ws.pos;
    ta.active = ws.active;
    ta.expert_slot = ws.expert_slot;
    ta.slot_info = ws.slot_info;
    ta.dslots = nullptr;
    ta.expert_counts = L.expert_counts;
    ta.defer_softmax = 0;
    ta.counters = ws.counters;
    ta.tiles = ws.tiles;
    ta.max_tiles = ws.max_tiles;
    // the merged top-k keeps 16 tokens per block; otherwise blocks of 8 or 4 tokens
    // where blocks of 16 would leave CUs idle (a block's tokens run one after another
    // on its four SIMDs)
    ta.tpb = kTopkTokensPerBlock;
    ta.nblk = (T + ta.tpb - 1) / ta.tpb;
    const bool merge = !route_uses_mfma(L, T) && !route_decode_fused(L, T) && ta.nblk * L.E <= kTopkMergeMax;
    if (!merge && T > kTopkTokensPerBlock) {
        while (ta.tpb > kTopkMinTokensPerBlock && (T + ta.tpb - 1) / ta.tpb < L.n_cu) ta.tpb >>= 1;
        ta.nblk = (T + ta.tpb - 1) / ta.tpb;
    }
    hipError_t err;
    if (route_uses_mfma(L, T)) {
        RouterMfmaArgs ma;
        ma.x = xr;
        ma.xe = x;
        ma.w = L.w_router;
        ma.ld = L.router_ld;
        ma.T = T; ma.H = L.H; ma.E = L.E;
        ma.n_etiles = (L.E + kRtTile - 1) / kRtTile;
        ma.n_tiles = ((T + kRtTile - 1) / kRtTile) * ma.n_etiles;
        ma.logits = ws.logits;
        ma.bound = ws.logit_bound;
        ma.xq_qs = ws.xq_qs;
        ma.xq_ds = ws.xq_ds;
        ma.x_q = x_f16 ? ws.x_q : nullptr;
        ma.x_d = ws.x_d;
        ma.rx = ws.rx_split;
        ma.rw = ws.rw_split;
        ma.rnorm = ws.rnorm;
        // k ranges per tile where the tiles alone would leave CUs idle (up to 4,
        // at least 4 steps each); their f64 sums go to the expert-row buffer, free
        // until the down projection, and the top-k adds them.  The debug copies of
        // the approximate logits and bounds take the unsplit form.
        ma.ksplit = 1;
        ma.part = (double*)ws.ybuf;
        if (!dbg.approx && !dbg.bound)
            while (ma.ksplit < 4 && ma.n_tiles * ma.ksplit < L.n_cu && L.H / kRtK >= 8 * ma.ksplit &&
                   (size_t)2 * ma.ksplit * T * L.E * sizeof(double) <= (size_t)T * (L.K + L.S) * L.H * sizeof(float))
                ma.ksplit *= 2;
        ta.rsplit = ma.ksplit;
        ta.rpart = ma.part;
        // the pre-MoE RMSNorm on the fly (x == xr is the residual row): the
        // preparation normalizes (and writes the scales), the refinement too
        ma.norm_w = norm_w;
        ma.eps = eps;
        ma.x_ssq = norm_w ? x_ssq : nullptr;
        ma.x_scale = ws.x_scale;
        ma.ecount = ws.hist + (uint64_t)ta.nblk * L.E;
        ta.norm_w = norm_w;
        x_f16 = false;  // written by the preparation
        hipLaunchKernelGGL(k_router_prep, dim3((T + 3) / 4 + (L.E + 3) / 4), dim3(256), 0, stream, ma);
        if ((err = hipGetLastError()) != hipSuccess) return err;
        // tiles that fill the CUs once: split in two on two-buffer workgroups, two per CU
        int nst = 3;
        if (ma.ksplit == 1 && !dbg.approx && !dbg.bound && ma.n_tiles <= L.n_cu && L.H / kRtK >= 8 &&
            (size_t)2 * 2 * T * L.E * sizeof(double) <= (size_t)T * (L.K + L.S) * L.H * sizeof(float)) {
            nst = 2;
            ma.ksplit = 2;
            ta.rsplit = 2;
        }
        const void* rk = nst == 2 ? (const void*)k_router_mfma<2> : (const void*)k_router_mfma<3>;
        const size_t lds = (size_t)nst * kRtStageHalfs * 2;
        if ((err = hipFuncSetAttribute(rk, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds)) != hipSuccess)
            return err;
        void* rargs[] = {&ma};
        if ((err = hipLaunchKernel(rk, dim3(ma.n_tiles * ma.ksplit), dim3(256), rargs, lds, stream)) != hipSuccess)
            return err;
        if ((err = hipGetLastError()) != hipSuccess) return err;
        if ((err = launch_topk(topk_kernel<true, false>(L.E), ta, nullptr, stream)) != hipSuccess) return err;
        if (dbg.approx &&
            (err = hipMemcpy2DAsync(dbg.approx, L.E * sizeof(float), ws.logits, (L.E + 1) * sizeof(float),
                                    L.E * sizeof(float), T, hipMemcpyDeviceToDevice, stream)) != hipSuccess)
            return err;
        if (dbg.bound && (err = hipMemcpyAsync(dbg.bound, ws.logit_bound, (size_t)T * L.E * sizeof(float),
                                               hipMemcpyDeviceToDevice, stream)) != hipSuccess)
            return err;
        if (dbg.exact_logits && (err = launch_router_exact(L, ws, xr, x, T, false, stream)) != hipSuccess) return err;
    } else if (route_decode_fused(L, T)) {
        // decode: the router launch, then the routing-table launch (it also writes
        // the decode slot list and, when the fused gate/up runs next, computes
        // the shared expert's h on other CUs meanwhile)
        ta.dslots = ws.dslots;
        ta.defer_softmax = 1;
        ta.norm_w = norm_w;
        ta.x_ssq = norm_w ? x_ssq : nullptr;
        const int nb = (L.E + L.S + kRdRows - 1) / kRdRows;
        const int nslab = L.H / kRdSlab;
        SharedGuArgs sg{};
        if (L.S && gateup_q_fused(L, T)) {
            const int nfb = L.F / 32;
            const int groups = std::max(1, std::min(T, (L.n_cu - nb) / nfb));
            sg.tpg = (T + groups - 1) / groups;
            sg.n_blocks = nfb * ((T + sg.tpg - 1) / sg.tpg);
            sg.w_gate = L.w_sh_gate; sg.w_up = L.w_sh_up;
            sg.gate_nb1 = L.sh_gate_nb1; sg.up_nb1 = L.sh_up_nb1;
            sg.F = L.F;
            sg.hq_qs = ws.hq_qs; sg.hq_ds = ws.hq_ds;
            sg.act = L.act; sg.gelu_tab = L.gelu_tab;
        }
        // above the 64 KiB default window: raise it
        const size_t lds = kRdLdsBytes;
        const int lpr = L.H <= 1024 ? 16 : (L.H <= 2048 ? 32 : 64);
        const int nsw = (nslab + kRdParts - 1) / kRdParts;  // slabs per wave
        const int swt = !sg.n_blocks ? 0 : (L.gu_type == kTypeQ4_0 ? 1 : 2);
        const void* kern = route_decode_kernel(nsw, ta.norm_w != nullptr);
        if (!kern) return hipErrorInvalidValue;
        float* logits = ws.logits;
        void* args[] = {&ta, &logits};
        if ((err = hipLaunchKernel(kern, dim3(nb), dim3(64 * kTopkTokensPerBlock), args, 0, stream)) != hipSuccess)
            return err;
        const void* tk = route_tables_kernel(swt, lpr);
        if ((err = hipFuncSetAttribute(tk, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds)) != hipSuccess)
            return err;
        int8_t* xq_qs = ws.xq_qs;
        float2* xq_ds = ws.xq_ds;
        void* targs[] = {&ta, &xq_qs, &xq_ds, &sg};
        if ((err = hipLaunchKernel(tk, dim3(1 + (sg.n_blocks ? sg.n_blocks : 1)), dim3(1024), targs, lds, stream)) !=
            hipSuccess)
            return err;
        return hipGetLastError();
    } else {
        // the decode router over groups of 16 tokens, x's Q8_0 on the same launch
        // (after each block's logits); then the top-k
        ta.quant_rows = 1;
        const int ngr = (T + kTopkTokensPerBlock - 1) / kTopkTokensPerBlock;
        const int nsw = (L.H / kRdSlab + kRdParts - 1) / kRdParts;
        int rows = 0;
        const void* kern = route_group_kernel(nsw, &rows);
        if (!kern) return hipErrorInvalidValue;
        const int nb = (L.E + L.S + rows - 1) / rows;
        float* logits = ws.logits;
        void* args[] = {&ta, &logits};
        if ((err = hipLaunchKernel(kern, dim3(nb * ngr), dim3(64 * kTopkTokensPerBlock), args, 0, stream)) !=
            hipSuccess)
            return err;
        ta.quant_rows = 0;
        if (merge) {
            // the last top-k block runs the expert scan and the scatter: no more launches
            return launch_topk(topk_kernel<false, true>(L.E), ta, ws.sync, stream);
        }
        if ((err = launch_topk(topk_kernel<false, false>(L.E), ta, nullptr, stream)) != hipSuccess) return err;
    }
    hipLaunchKernelGGL(k_lists, dim3(L.E + 1), dim3(kListThreads), 0, stream, ta);
    return hipGetLastError();
}

bool route_norm_fused(const LayerDesc& L, int T) { return route_decode_fused(L, T) && L.H <= 8 * kRdSlab; }

hipError_t launch_route(const LayerDesc& L, const Workspace& ws, const float* x, const float* xr, int T,
                        const RouteDebug& dbg, bool x_f16, hipStream_t stream, const float* norm_w, float eps,
                        const double* x_ssq) {
    // norm_w: decode routing (route_norm_fused, no f16 operands) or the batched
    // router (its preparation writes the f16 operands), with x == xr
    if (norm_w && (x != xr || (route_uses_mfma(L, T) ? !x_f16 : (x_f16 || !route_norm_fused(L, T)))))
        return hipErrorInvalidValue;
    hipError_t err = launch_route_tables(L, ws, x, xr, T, dbg, x_f16, stream, norm_w, eps, x_ssq);
    if (err != hipSuccess || !x_f16) return err;
    // the routing launch did not write x's f16 quants (only the batched router's does)
    hipLaunchKernelGGL(k_x_f16, dim3((T + 3) / 4), dim3(256), 0, stream, x, T, L.H, ws.x_q, ws.x_d, ws.xq_qs, ws.xq_ds);
    return hipGetLastError();
}

}  // namespace qmoe
