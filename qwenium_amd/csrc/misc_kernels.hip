// misc_kernels.hip -- RMSNorm (the MoE layer's pre-norm caller slice) and the
// seeded synthetic-data generators used by tests and benchmarks.
#include "qmoe_device.h"
#include "qmoe_internal.h"

#include <algorithm>

namespace qmoe {

// ---------------------------------------------------------------------------
// RMSNorm, restating ggml_rms_norm + ggml_mul as used by build_rms_norm
// (src/layers/norm.cpp:15-26): sum of f32 squares accumulated in f64,
// mean rounded to f32, scale = 1/sqrtf(mean + eps), y = (x*scale)*w.
// One block per token; the sum of squares in the order rms_scale_row fixes
// (runs of four columns, then a pairwise tree), as the fused decode router
// computes it.
// ---------------------------------------------------------------------------
// one 1024-thread block per row: each 256-column chunk's tree in its own wave (one
// round of row loads), the same order as with fewer waves
__global__ __launch_bounds__(1024) void k_rms_norm(const float* x, const float* w, int H, float eps, float* y) {
#pragma clang fp contract(off)
    __shared__ double s_chunk[kRmsMaxChunks];
    __shared__ float s_scale;
    const int t = blockIdx.x;
    const float* xr = x + (uint64_t)t * H;
    const float scale = rms_scale_row(xr, H, eps, s_chunk, &s_scale);
    for (int i = threadIdx.x; i < H; i += 1024) {
        const float v = xr[i] * scale;
        y[(uint64_t)t * H + i] = w ? v * w[i] : v;
    }
}

hipError_t launch_rms_norm(const float* x, const float* w, int T, int H, float eps, float* y, hipStream_t stream) {
    if (H > 256 * kRmsMaxChunks) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_rms_norm, dim3(T), dim3(1024), 0, stream, x, w, H, eps, y);
    return hipGetLastError();
}

// The RMSNorm partial sums of the rows x[T][H] (ssq_parts(H) per row, each the
// subtree over 8 runs of four columns): one block per row, lane i of a wave
// takes run 64 m + i of its windows m, the 8-lane trees give the entries.
__global__ __launch_bounds__(256) void k_rms_partials(const float* x, int H, double* out) {
#pragma clang fp contract(off)
    const int t = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const float* xr = x + (uint64_t)t * H;
    const int np = ssq_parts(H);
    for (int base = 64 * wave; base < 8 * np; base += 256) {
        const double s = dpp_sum_f64<8>(ssq_run4(xr, H, base + lane));
        const int c = (base + lane) >> 3;
        if ((lane & 7) == 7 && c < np) out[(uint64_t)t * np + c] = s;
    }
}

hipError_t launch_rms_partials(const float* x, int T, int H, double* out, hipStream_t stream) {
    if (T <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_rms_partials, dim3(T), dim3(256), 0, stream, x, H, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Gemma 4 MoE inputs (src/models/gemma4.cpp:555-563): from the residual row x,
//   expert_in = rms_norm(x) * pre_ffw_norm_2            (build_rms_norm)
//   router_in = (rms_norm(x) * s) * ffn_gate_inp.scale  (ggml_rms_norm, ggml_scale, ggml_mul)
// with s = 1/sqrtf(n_embd): the scale computed once, in k_rms_norm's
// summation order (so rms_norm(x) has the same bits).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void k_gemma4_inputs(const float* x, const float* w_pre, const float* w_rs, int H,
                                                       float eps, float s, float* ei, float* ri) {
#pragma clang fp contract(off)
    __shared__ double s_chunk[kRmsMaxChunks];
    __shared__ float s_scale;
    const int t = blockIdx.x;
    const float* xr = x + (uint64_t)t * H;
    const float scale = rms_scale_row(xr, H, eps, s_chunk, &s_scale);
    for (int i = threadIdx.x; i < H; i += 1024) {
        const float u = xr[i] * scale;
        ei[(uint64_t)t * H + i] = u * w_pre[i];
        const float r = u * s;
        ri[(uint64_t)t * H + i] = r * w_rs[i];
    }
}

hipError_t launch_gemma4_inputs(const float* x, const float* w_pre, const float* w_rs, int T, int H, float eps, float s,
                                float* expert_in, float* router_in, hipStream_t stream) {
    hipLaunchKernelGGL(k_gemma4_inputs, dim3(T), dim3(1024), 0, stream, x, w_pre, w_rs, H, eps, s, expert_in, router_in);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Synthetic data: N(mean, sigma) from (seed, stream, index); quantized rows
// use ggml's reference quantizers (quantize_row_q4_0_ref / _q8_0_ref).
// ---------------------------------------------------------------------------
// Plain fill of n words (clears flags and counters; unlike hipMemsetAsync it
// records as an ordinary kernel node when a caller captures the stream).
__global__ __launch_bounds__(256) void k_fill_i32(int32_t* dst, int n, int32_t v) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = v;
}

hipError_t launch_fill_i32(int32_t* dst, int n, int32_t v, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_fill_i32, dim3((n + 255) / 256), dim3(256), 0, stream, dst, n, v);
    return hipGetLastError();
}

// Debug copies of per-row intermediates in assignment order.  Workspace row p
// holds routed assignment rows[p] for p < A (rows grouped by expert) and the
// shared expert's row of token p - A after them; output row = rows[p] or p.
// h: from the int8 quants + {d, sum} records of the decode and streaming paths
// (qs8, ds8) or the f16 quants + fp16 scale bits of the MFMA path (q16, d16);
// the first fo of each f-wide row (fo: the caller's ffn width).
__global__ __launch_bounds__(256) void k_debug_h(const int32_t* rows, int A, int R, int f, int fo, const int8_t* qs8,
                                                 const float2* ds8, const _Float16* q16, const uint16_t* d16,
                                                 int8_t* out_q, float* out_d) {
    const uint64_t n = (uint64_t)R * fo;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256) {
        const int p = (int)(i / (uint64_t)fo), c = (int)(i - (uint64_t)p * fo);
        const uint64_t dst = p < A ? (uint64_t)rows[p] : (uint64_t)p;
        const uint64_t s = (uint64_t)p * f + c;
        out_q[dst * fo + c] = qs8 ? qs8[s] : (int8_t)(float)q16[s];
        if ((c & 31) == 0) {
            const uint64_t b = (uint64_t)p * (f >> 5) + (c >> 5);
            out_d[dst * (fo >> 5) + (c >> 5)] = ds8 ? ds8[b].x : fp16_to_f32(d16[b]);
        }
    }
}

// The unweighted down rows (ybuf, h-wide) in assignment order, first ho columns.
__global__ __launch_bounds__(256) void k_debug_rows(const int32_t* rows, int A, int R, int h, int ho, const float* src,
                                                    float* out) {
    const uint64_t n = (uint64_t)R * ho;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256) {
        const int p = (int)(i / (uint64_t)ho), c = (int)(i - (uint64_t)p * ho);
        const uint64_t dst = p < A ? (uint64_t)rows[p] : (uint64_t)p;
        out[dst * ho + c] = src[(uint64_t)p * h + c];
    }
}

hipError_t launch_debug_h(const int32_t* rows, int A, int R, int f, int fo, const int8_t* qs8, const float2* ds8,
                          const _Float16* q16, const uint16_t* d16, int8_t* out_q, float* out_d, hipStream_t stream) {
    const uint64_t n = (uint64_t)R * fo;
    if (n == 0) return hipSuccess;
    const unsigned g = (unsigned)std::min<uint64_t>((n + 255) / 256, 65536);
    hipLaunchKernelGGL(k_debug_h, dim3(g), dim3(256), 0, stream, rows, A, R, f, fo, qs8, ds8, q16, d16, out_q, out_d);
    return hipGetLastError();
}

hipError_t launch_debug_rows(const int32_t* rows, int A, int R, int h, int ho, const float* src, float* out,
                             hipStream_t stream) {
    const uint64_t n = (uint64_t)R * ho;
    if (n == 0) return hipSuccess;
    const unsigned g = (unsigned)std::min<uint64_t>((n + 255) / 256, 65536);
    hipLaunchKernelGGL(k_debug_rows, dim3(g), dim3(256), 0, stream, rows, A, R, h, ho, src, out);
    return hipGetLastError();
}

// Zero padding of rows for layers built with padded widths (the padded
// columns meet zero weights, so every dot and every Q8_0 block of the real
// columns keeps its value).
__global__ __launch_bounds__(256) void k_pad_rows(const float* src, int T, int hs, int hd, float* dst) {
    const uint64_t n = (uint64_t)T * hd;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256) {
        const uint64_t t = i / (uint64_t)hd, c = i - t * (uint64_t)hd;
        dst[i] = c < (uint64_t)hs ? src[t * hs + c] : 0.0f;
    }
}

__global__ __launch_bounds__(256) void k_unpad_rows(const float* src, int T, int hs, int hd, const float* residual,
                                                    float* dst) {
#pragma clang fp contract(off)
    const uint64_t n = (uint64_t)T * hd;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256) {
        const uint64_t t = i / (uint64_t)hd, c = i - t * (uint64_t)hd;
        const float v = src[t * hs + c];
        dst[i] = residual ? v + residual[i] : v;
    }
}

static int pad_grid(int T, int hd) { return (int)std::min<uint64_t>(((uint64_t)T * hd + 255) / 256, 1u << 16); }

hipError_t launch_pad_rows(const float* src, int T, int hs, int hd, float* dst, hipStream_t stream) {
    if (T <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_pad_rows, dim3(pad_grid(T, hd)), dim3(256), 0, stream, src, T, hs, hd, dst);
    return hipGetLastError();
}

hipError_t launch_unpad_rows(const float* src, int T, int hs, int hd, const float* residual, float* dst,
                             hipStream_t stream) {
    if (T <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_unpad_rows, dim3(pad_grid(T, hd)), dim3(256), 0, stream, src, T, hs, hd, residual, dst);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_synth_f32(float* dst, int64_t n, uint64_t key, double mean, double sigma) {
#pragma clang fp contract(off)
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        dst[i] = (float)(mean + sigma * normal_det(key, (uint64_t)i));
}

template <int WT>
__global__ __launch_bounds__(256) void k_synth_quant(uint8_t* dst, int64_t n_rows, int64_t row_len, uint64_t key,
                                                      double sigma) {
#pragma clang fp contract(off)
    const int64_t nb = row_len / 32;
    const int64_t total = n_rows * nb;
    constexpr int BS = BlockTraits<WT>::kBytes;
    for (int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x; g < total; g += (int64_t)gridDim.x * 256) {
        const int64_t row = g / nb, b = g % nb;
        const uint64_t i0 = (uint64_t)(row * row_len + 32 * b);
        float v[32];
#pragma unroll
        for (int j = 0; j < 32; ++j) v[j] = (float)(0.0 + sigma * normal_det(key, i0 + j));
        uint16_t* out = (uint16_t*)(dst + row * nb * BS + b * BS);
        if (WT == kTypeQ4_0) {
            float amax = 0.0f, vmax = 0.0f;
            for (int j = 0; j < 32; ++j) {
                if (amax < __builtin_fabsf(v[j])) { amax = __builtin_fabsf(v[j]); vmax = v[j]; }
            }
            const float d = vmax / -8.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            out[0] = (uint16_t)f32_to_fp16(d);
#pragma unroll
            for (int j = 0; j < 16; j += 2) {
                uint32_t pair = 0;
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {
                    const float x0 = v[j + jj] * id;
                    const float x1 = v[16 + j + jj] * id;
                    const int xi0 = min(15, (int)(x0 + 8.5f));
                    const int xi1 = min(15, (int)(x1 + 8.5f));
                    pair |= (uint32_t)(xi0 | (xi1 << 4)) << (8 * jj);
                }
                out[1 + j / 2] = (uint16_t)pair;
            }
        } else {
            float amax = 0.0f;
            for (int j = 0; j < 32; ++j) amax = fmaxf(amax, __builtin_fabsf(v[j]));
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            out[0] = (uint16_t)f32_to_fp16(d);
#pragma unroll
            for (int j = 0; j < 32; j += 2) {
                const int q0 = (int)__builtin_roundf(v[j] * id);
                const int q1 = (int)__builtin_roundf(v[j + 1] * id);
                out[1 + j / 2] = (uint16_t)((q0 & 0xff) | ((q1 & 0xff) << 8));
            }
        }
    }
}

hipError_t launch_synth_f32(float* dst, int64_t n, uint64_t seed, uint64_t stream_id, double mean, double sigma,
                            hipStream_t stream) {
    const int64_t blocks = n <= 0 ? 1 : (n + 255) / 256;
    const int grid = (int)(blocks < 65536 ? blocks : 65536);
    hipLaunchKernelGGL(k_synth_f32, dim3(grid), dim3(256), 0, stream, dst, n, stream_key(seed, stream_id), mean,
                       sigma);
    return hipGetLastError();
}

hipError_t launch_synth_quant(void* dst, int type, int64_t n_rows, int64_t row_len, uint64_t seed,
                              uint64_t stream_id, double sigma, hipStream_t stream) {
    const int64_t total = n_rows * (row_len / 32);
    const int64_t blocks = total <= 0 ? 1 : (total + 255) / 256;
    const int grid = (int)(blocks < 65536 ? blocks : 65536);
    const uint64_t key = stream_key(seed, stream_id);
    if (type == kTypeQ4_0)
        hipLaunchKernelGGL((k_synth_quant<kTypeQ4_0>), dim3(grid), dim3(256), 0, stream, (uint8_t*)dst, n_rows,
                           row_len, key, sigma);
    else
        hipLaunchKernelGGL((k_synth_quant<kTypeQ8_0>), dim3(grid), dim3(256), 0, stream, (uint8_t*)dst, n_rows,
                           row_len, key, sigma);
    return hipGetLastError();
}

}  // namespace qmoe
