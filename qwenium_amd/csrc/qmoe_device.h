// qmoe_device.h -- device helpers shared by the qmoe HIP kernels (gfx950).
//
// Numeric contract (matches the CPU restatement in oracle/ exactly):
//   * exp_det / log_det / cospi2_det are fixed sequences of separately
//     rounded IEEE f64 operations (contraction disabled), so they return the
//     same bits as any IEEE CPU running the same sequence.
//   * Quantized block dots accumulate d_w*d_x*isum in f64.  Each term is
//     exact in f64 (22-bit scale product x <= 19-bit integer) and the row sum
//     stays exact for the scale ranges of these layers, so the result does
//     not depend on summation order (lane split, butterfly, MFMA tiling).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qmoe_internal.h"

namespace qmoe {

constexpr int kTypeF32 = 0;
constexpr int kTypeQ4_0 = 2;
constexpr int kTypeQ8_0 = 8;

template <int WT> struct BlockTraits;
template <> struct BlockTraits<kTypeQ4_0> { static constexpr int kBytes = 18; static constexpr int kPairDwords = 9; };
template <> struct BlockTraits<kTypeQ8_0> { static constexpr int kBytes = 34; static constexpr int kPairDwords = 17; };

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef double f64x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// fp16 <-> fp32 (IEEE binary16, round to nearest even)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float fp16_to_f32(uint32_t h16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(h16 & 0xffffu));
}
__device__ __forceinline__ uint32_t f32_to_fp16(float f) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

// ---------------------------------------------------------------------------
// Deterministic f64 elementary functions
// ---------------------------------------------------------------------------
constexpr double kLn2Hi = 6.93147180369123816490e-01;  // 32 significant bits
constexpr double kLn2Lo = 1.90821492927058770002e-10;
constexpr double kLog2e = 1.44269504088896338700e+00;

__device__ __forceinline__ double exp_det(double x) {
#pragma clang fp contract(off)
    if (x != x) return x;
    if (x > 709.78) return __builtin_huge_val();
    if (x < -745.2) return 0.0;
    const double k = __builtin_rint(x * kLog2e);
    double r = x - k * kLn2Hi;
    r = r - k * kLn2Lo;
    // Taylor series of exp(r), |r| <= 0.347, degree 13
    double p = 1.0 / 6227020800.0;
    p = p * r + 1.0 / 479001600.0;
    p = p * r + 1.0 / 39916800.0;
    p = p * r + 1.0 / 3628800.0;
    p = p * r + 1.0 / 362880.0;
    p = p * r + 1.0 / 40320.0;
    p = p * r + 1.0 / 5040.0;
    p = p * r + 1.0 / 720.0;
    p = p * r + 1.0 / 120.0;
    p = p * r + 1.0 / 24.0;
    p = p * r + 1.0 / 6.0;
    p = p * r + 0.5;
    p = p * r + 1.0;
    p = p * r + 1.0;
    return __builtin_ldexp(p, (int)k);
}

__device__ __forceinline__ double log_det(double x) {
#pragma clang fp contract(off)
    int e;
    double m = __builtin_frexp(x, &e);
    if (m < 0.70710678118654752440) { m = m * 2.0; e = e - 1; }
    const double s = (m - 1.0) / (m + 1.0);
    const double s2 = s * s;
    double p = 1.0 / 23.0;
    p = p * s2 + 1.0 / 21.0;
    p = p * s2 + 1.0 / 19.0;
    p = p * s2 + 1.0 / 17.0;
    p = p * s2 + 1.0 / 15.0;
    p = p * s2 + 1.0 / 13.0;
    p = p * s2 + 1.0 / 11.0;
    p = p * s2 + 1.0 / 9.0;
    p = p * s2 + 1.0 / 7.0;
    p = p * s2 + 1.0 / 5.0;
    p = p * s2 + 1.0 / 3.0;
    p = p * s2 + 1.0;
    const double de = (double)e;
    return de * kLn2Hi + (de * kLn2Lo + 2.0 * s * p);
}

__device__ __forceinline__ double cospi2_det(double u) {
#pragma clang fp contract(off)
    const double t = u * 4.0;
    double q = __builtin_floor(t);
    double f = t - q;
    if (f > 0.5) { f = f - 1.0; q = q + 1.0; }
    const double a = f * 1.57079632679489661923;
    const double a2 = a * a;
    double c = 1.0 / 20922789888000.0;
    c = c * a2 - 1.0 / 87178291200.0;
    c = c * a2 + 1.0 / 479001600.0;
    c = c * a2 - 1.0 / 3628800.0;
    c = c * a2 + 1.0 / 40320.0;
    c = c * a2 - 1.0 / 720.0;
    c = c * a2 + 1.0 / 24.0;
    c = c * a2 - 0.5;
    c = c * a2 + 1.0;
    double s = 1.0 / 355687428096000.0;
    s = s * a2 - 1.0 / 1307674368000.0;
    s = s * a2 + 1.0 / 6227020800.0;
    s = s * a2 - 1.0 / 39916800.0;
    s = s * a2 + 1.0 / 362880.0;
    s = s * a2 - 1.0 / 5040.0;
    s = s * a2 + 1.0 / 120.0;
    s = s * a2 - 1.0 / 6.0;
    s = s * a2 + 1.0;
    s = s * a;
    switch (((int)q) & 3) {
        case 0: return c;
        case 1: return -s;
        case 2: return -c;
        default: return s;
    }
}

// h = silu(g) * u, evaluated in f64 and rounded once to f32.
__device__ __forceinline__ float silu_mul_det(float g, float u) {
#pragma clang fp contract(off)
    const double gd = (double)g;
    const double s = gd / (1.0 + exp_det(-gd));
    return (float)(s * (double)u);
}

// gelu(g)*u as ggml's CPU backend computes it: g <= -10 -> 0, g >= 10 -> g,
// else the fp16 table entry of fp16(g) (tab: 65536 fp16 values, built on the
// host from the tanh formula), widened, times u in f32.
__device__ __forceinline__ float geglu_mul_tab(float g, float u, const uint16_t* tab) {
    float gl;
    if (g <= -10.0f) gl = 0.0f;
    else if (g >= 10.0f) gl = g;
    else gl = fp16_to_f32(tab[f32_to_fp16(g) & 0xffffu]);
    return gl * u;
}

__device__ __forceinline__ float act_mul(int act, const uint16_t* gelu_tab, float g, float u) {
    return act == kActGeluTanh ? geglu_mul_tab(g, u, gelu_tab) : silu_mul_det(g, u);
}

__device__ __forceinline__ float sigmoid_det(float g) {
#pragma clang fp contract(off)
    return (float)(1.0 / (1.0 + exp_det(-(double)g)));
}

// ---------------------------------------------------------------------------
// Counter-based normal generator (splitmix64 finalizer + Box-Muller)
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__host__ __device__ __forceinline__ uint64_t stream_key(uint64_t seed, uint64_t stream) {
    return mix64(seed ^ mix64(stream + 0x632BE59BD9B4E019ull));
}
__device__ __forceinline__ double normal_det(uint64_t key, uint64_t idx) {
#pragma clang fp contract(off)
    const uint64_t h1 = mix64(key ^ (2 * idx));
    const uint64_t h2 = mix64(key ^ (2 * idx + 1));
    const double u1 = (double)((h1 >> 11) + 1) * (1.0 / 9007199254740992.0);
    const double u2 = (double)(h2 >> 11) * (1.0 / 9007199254740992.0);
    const double r = __builtin_sqrt(-2.0 * log_det(u1));
    return r * cospi2_det(u2);
}

// ---------------------------------------------------------------------------
// DPP reductions (wave64).  Groups of WIDTH aligned lanes (WIDTH = 2..64);
// the group result lands in the group's LAST lane (lane WIDTH-1 of the group).
// Steps: quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror,
// row_mirror, row_bcast:15 (rows 1,3), row_bcast:31 (rows 2,3).  All VALU; no
// LDS round trip.
// ---------------------------------------------------------------------------
constexpr int kDppQuadXor1 = 0xB1;
constexpr int kDppQuadXor2 = 0x4E;
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;
constexpr int kDppRowBcast15 = 0x142;
constexpr int kDppRowBcast31 = 0x143;

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ double dpp_f64_or_zero(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    uint32_t lo, hi;
    if constexpr (ROW_MASK == 0xF) {
        // every lane is written from a lane of its own row: no old value needed
        lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)b, CTRL, 0xF, 0xF, false);
        hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(b >> 32), CTRL, 0xF, 0xF, false);
    } else {
        lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, ROW_MASK, 0xF, false);
        hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, ROW_MASK, 0xF, false);
    }
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

template <int WIDTH>
__device__ __forceinline__ double dpp_sum_f64(double v) {
    static_assert(WIDTH == 2 || WIDTH == 4 || WIDTH == 8 || WIDTH == 16 || WIDTH == 32 || WIDTH == 64, "width");
    v += dpp_f64_or_zero<kDppQuadXor1, 0xF>(v);
    if (WIDTH >= 4) v += dpp_f64_or_zero<kDppQuadXor2, 0xF>(v);
    if (WIDTH >= 8) v += dpp_f64_or_zero<kDppRowHalfMirror, 0xF>(v);
    if (WIDTH >= 16) v += dpp_f64_or_zero<kDppRowMirror, 0xF>(v);
    if (WIDTH >= 32) v += dpp_f64_or_zero<kDppRowBcast15, 0xA>(v);
    if (WIDTH >= 64) v += dpp_f64_or_zero<kDppRowBcast31, 0xC>(v);
    return v;
}

// Direct global->LDS loads (lane i's 16 or 4 bytes to LDS byte address
// lds + 16 i or + 4 i; lds wave-uniform).  Issued as assembly so that the
// compiler does not order every later LDS read after them: the kernel waits
// for them itself (s_waitcnt vmcnt at the chunk boundary, then a barrier).
// M0 takes the LDS base; the LDS-DMA read of M0 needs one wait state.
// Source: a wave-uniform base plus this lane's 32-bit byte offset.
__device__ __forceinline__ void dma_lds16(const void* base, uint32_t off, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds)
                 : "memory", "m0");
}
__device__ __forceinline__ void dma_lds4(const void* base, uint32_t off, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "s"(lds)
                 : "memory", "m0");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// RMSNorm's sum of squares in the one order every RMSNorm here uses (the
// standalone kernels and the decode router that normalizes on the fly): the
// columns in runs of four (run r: columns 4r .. 4r+3 below H), each run's
// f64(f32(v * v)) added in column order; then an adjacent-pairs tree over the
// run sums zero-padded to a power of two (a longer zero padding changes no
// bits: its subtrees are exact zeros).  A wave reads 64 consecutive runs with
// one coalesced load per lane, and dpp_sum_f64<64> is exactly the adjacent-pairs
// tree over its lanes (xor 1, xor 2, then half-row, row, 16- and 32-lane steps
// over uniform groups; a + b == b + a).  ggml adds all columns one after another
// in f64 (src/layers/norm.cpp:15-26 -> ggml_rms_norm); the orders round
// differently only where the f64 sum lands within a few f64 ulps of an f32
// rounding boundary of the mean.
__device__ __forceinline__ double ssq_run4(const float* xr, int H, int r) {
#pragma clang fp contract(off)
    const int c0 = 4 * r;
    float v[4];
    if (c0 + 4 <= H && ((uintptr_t)(xr + c0) & 15u) == 0) {
        const f32x4 q = *(const f32x4*)(xr + c0);
        v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
    } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) v[c] = c0 + c < H ? xr[c0 + c] : 0.0f;
    }
    double s = 0.0;
#pragma unroll
    for (int c = 0; c < 4; ++c)
        if (c0 + c < H) s += (double)(v[c] * v[c]);
    return s;
}
// The tree over runs 64 c .. 64 c + 63 (lane i: run 64 c + i), in lane 63.
__device__ __forceinline__ double ssq_chunk64(const float* xr, int H, int c, int lane) {
    return dpp_sum_f64<64>(ssq_run4(xr, H, 64 * c + lane));
}
// Partial sums carried from a layer's output to the next layer's RMSNorm: entry
// c of a row is the subtree over runs 8c .. 8c+7 (columns 32c .. 32c+31), so
// the adjacent-pairs tree over a row's entries, zero-padded, is the row's sum.
constexpr int kSsqCols = 32;
__host__ __device__ constexpr int ssq_parts(int H) { return (H + kSsqCols - 1) / kSsqCols; }
// f32 RMSNorm scale from the f64 sum of squares (ggml_rms_norm: mean in f32).
__device__ __forceinline__ float rms_scale_from_ssq(double ssq, int H, float eps) {
    // a power-of-two H divides by exact scaling (one instruction, the same bits)
    const float mean = (float)((H & (H - 1)) == 0 ? __builtin_ldexp(ssq, -__builtin_ctz(H)) : ssq / (double)H);
    return 1.0f / __builtin_sqrtf(mean + eps);
}
// scale = 1/sqrtf(fp32(ssq / H) + eps) of one row (H <= 256 kRmsMaxChunks), by
// the whole workgroup (every thread calls it): the waves take the chunks in
// turn, their trees go to s_chunk (LDS, kRmsMaxChunks doubles), then the tree
// over the chunk sums level by level.
__device__ inline float rms_scale_row(const float* xr, int H, float eps, double* s_chunk, float* s_scale) {
#pragma clang fp contract(off)
    const int nc = (H + 255) >> 8;
    const int nw = (int)blockDim.x >> 6, wave = (int)threadIdx.x >> 6, lane = (int)threadIdx.x & 63;
    int L = 1;
    while (L < nc) L <<= 1;
    for (int c = wave; c < L; c += nw) {
        const double v = c < nc ? ssq_chunk64(xr, H, c, lane) : 0.0;
        if (lane == 63) s_chunk[c] = v;
    }
    __syncthreads();
    for (int w = L >> 1; w >= 1; w >>= 1) {
        const int i = threadIdx.x;
        const double v = i < w ? s_chunk[2 * i] + s_chunk[2 * i + 1] : 0.0;
        __syncthreads();
        if (i < w) s_chunk[i] = v;
        __syncthreads();
    }
    if (threadIdx.x == 0) *s_scale = rms_scale_from_ssq(s_chunk[0], H, eps);
    __syncthreads();
    return *s_scale;
}

// The whole wave's f64 sum in every lane (dpp_sum_f64<64> leaves it in lane 63).
__device__ __forceinline__ double wave_sum_f64(double v) {
    v = dpp_sum_f64<64>(v);
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), 63);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// A row's sum of squares by one wave (every lane gets it), in the order every
// RMSNorm here uses: the trees of 64-run chunks, then the adjacent-pairs tree
// over the chunks, zero-padded to 16 leaves (H <= 4096; a longer zero padding
// changes no bits).
__device__ inline double ssq_row(const float* xr, int H, int lane) {
    const int nc = (H + 255) >> 8;
    double c[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) c[i] = i < nc ? wave_sum_f64(ssq_run4(xr, H, 64 * i + lane)) : 0.0;
#pragma unroll
    for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
        for (int i = 0; i < w; ++i) c[i] = c[2 * i] + c[2 * i + 1];
    return c[0];
}
// The same sum from a row's carried partial sums (np <= 128 entries, each the
// subtree of 8 runs): the adjacent-pairs tree over the entries zero-padded,
// 64-entry chunks by DPP trees, then the chunks' pair.
__device__ inline double ssq_from_parts(const double* parts, int np, int lane) {
    double c[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int e = 64 * i + lane;
        c[i] = 64 * i < np ? wave_sum_f64(e < np ? parts[e] : 0.0) : 0.0;
    }
    return c[0] + c[1];
}

// One reduce-scatter step over an f64 pair (x, y): the 32-lane swap (W = 32)
// leaves lanes 0..31 with x[l] + x[l + 32] and lanes 32..63 with y[l - 32] + y[l];
// the 16-lane swap (W = 16) does the same between the even and odd rows of 16.
template <int W>
__device__ __forceinline__ double swap_add_f64(double x, double y) {
    const uint64_t bx = __builtin_bit_cast(uint64_t, x), by = __builtin_bit_cast(uint64_t, y);
    uint32_t a_lo, a_hi, b_lo, b_hi;
    if constexpr (W == 32) {
        const auto lo = __builtin_amdgcn_permlane32_swap((uint32_t)bx, (uint32_t)by, false, false);
        const auto hi = __builtin_amdgcn_permlane32_swap((uint32_t)(bx >> 32), (uint32_t)(by >> 32), false, false);
        a_lo = lo[0]; b_lo = lo[1]; a_hi = hi[0]; b_hi = hi[1];
    } else {
        const auto lo = __builtin_amdgcn_permlane16_swap((uint32_t)bx, (uint32_t)by, false, false);
        const auto hi = __builtin_amdgcn_permlane16_swap((uint32_t)(bx >> 32), (uint32_t)(by >> 32), false, false);
        a_lo = lo[0]; b_lo = lo[1]; a_hi = hi[0]; b_hi = hi[1];
    }
    return __builtin_bit_cast(double, ((uint64_t)a_hi << 32) | a_lo) +
           __builtin_bit_cast(double, ((uint64_t)b_hi << 32) | b_lo);
}

// Sums of two per-lane f64 values g and u over aligned groups of LPR lanes.
// LPR >= 32: one swap step folds u into the upper half of each group and g
// into the lower, then one tree of LPR/2 lanes finishes both; the sum of g is
// then in lane LPR/2 - 1 of the group and the sum of u in lane LPR - 1 (returned
// by those lanes).  Narrower groups: two trees, g and u both in lane LPR - 1.
template <int LPR>
__device__ __forceinline__ void group_sum2_f64(double g, double u, double& gs, double& us) {
    if constexpr (LPR >= 32) {
        const double s = dpp_sum_f64<LPR / 2>(swap_add_f64<LPR / 2>(g, u));
        gs = s;
        us = s;
    } else {
        gs = dpp_sum_f64<LPR>(g);
        us = dpp_sum_f64<LPR>(u);
    }
}

// (value, index) arg-max step: keep the better of own and the DPP source
// (larger value; ties to the lower index).  Masked rows keep their own pair.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ void dpp_argmax_step(float& bv, int& bi) {
    const float ov = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, bv),
                                                                           __builtin_bit_cast(int, bv), CTRL,
                                                                           ROW_MASK, 0xF, false));
    const int oi = __builtin_amdgcn_update_dpp(bi, bi, CTRL, ROW_MASK, 0xF, false);
    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
}

// Whole-wave inclusive prefix sum of an int (row_shr 1,2,4,8 then row
// broadcasts); lane i receives sum of lanes 0..i.
__device__ __forceinline__ int wave_incl_scan_i32(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, kDppRowBcast15, 0xA, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, kDppRowBcast31, 0xC, 0xF, false);
    return v;
}

// Orders one wave's LDS accesses across its lanes (a lane reads what another
// lane of the same wave wrote): compiler barrier, LDS counter drained, wave
// barrier.  Unlike a memory fence it does not wait for the wave's global
// stores.
__device__ __forceinline__ void wave_lds_sync() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left at their maxima
    __builtin_amdgcn_wave_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Whole-wave arg-max; the winner is returned to every lane.
__device__ __forceinline__ void wave_argmax(float& bv, int& bi) {
    dpp_argmax_step<kDppQuadXor1, 0xF>(bv, bi);
    dpp_argmax_step<kDppQuadXor2, 0xF>(bv, bi);
    dpp_argmax_step<kDppRowHalfMirror, 0xF>(bv, bi);
    dpp_argmax_step<kDppRowMirror, 0xF>(bv, bi);
    dpp_argmax_step<kDppRowBcast15, 0xA>(bv, bi);
    dpp_argmax_step<kDppRowBcast31, 0xC>(bv, bi);
    bv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, bv), 63));
    bi = __builtin_amdgcn_readlane(bi, 63);
}

// ---------------------------------------------------------------------------
// Shuffle-based reductions (wave64; WIDTH lanes per independent group; result
// in every lane of the group)
// ---------------------------------------------------------------------------
template <int WIDTH>
__device__ __forceinline__ double group_sum_f64(double v) {
#pragma unroll
    for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
template <int WIDTH>
__device__ __forceinline__ int group_sum_i32(int v) {
#pragma unroll
    for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
template <int WIDTH>
__device__ __forceinline__ float group_max_f32(float v) {
#pragma unroll
    for (int o = WIDTH / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// ---------------------------------------------------------------------------
// Quantized weight pair loaders.  A "pair" is two consecutive 32-value blocks
// of one row: 36 bytes (Q4_0) or 68 bytes (Q8_0), starting 4-byte aligned
// when the row starts 4-byte aligned.  Loads are dword-aligned dwordx4.
// ---------------------------------------------------------------------------
template <int WT> struct WPair;

template <> struct WPair<kTypeQ4_0> {
    uint32_t w[9];
    __device__ __forceinline__ void load(const uint8_t* row, int pair) {
        const uint32_t* b = (const uint32_t*)(row + 36 * pair);
        const u32x4a4 a0 = *(const u32x4a4*)(b);
        const u32x4a4 a1 = *(const u32x4a4*)(b + 4);
        w[0] = a0.x; w[1] = a0.y; w[2] = a0.z; w[3] = a0.w;
        w[4] = a1.x; w[5] = a1.y; w[6] = a1.z; w[7] = a1.w;
        w[8] = b[8];
    }
    // pair at byte offset `off` (32-bit) from a wave-uniform base: saddr loads
    __device__ __forceinline__ void load32(const uint8_t* base, uint32_t off) {
        const u32x4a4 a0 = *(const u32x4a4*)(base + off);
        const u32x4a4 a1 = *(const u32x4a4*)(base + (off + 16u));
        w[0] = a0.x; w[1] = a0.y; w[2] = a0.z; w[3] = a0.w;
        w[4] = a1.x; w[5] = a1.y; w[6] = a1.z; w[7] = a1.w;
        w[8] = *(const uint32_t*)(base + (off + 32u));
    }
    // scales (as f32) of block A and block B
    __device__ __forceinline__ float dA() const { return fp16_to_f32(w[0]); }
    __device__ __forceinline__ float dB() const { return fp16_to_f32(w[4] >> 16); }
    // integer dot of block A / B against 32 int8 activations xs[0..7] (dwords);
    // returns sum_j (q_j - 8) * x_j given xsum = sum_j x_j
    __device__ __forceinline__ int dotA(const uint32_t* xs, int xsum) const {
        int acc = -8 * xsum;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t q = __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2);
            acc = __builtin_amdgcn_sdot4((int)(q & 0x0f0f0f0fu), (int)xs[i], acc, false);
            acc = __builtin_amdgcn_sdot4((int)((q >> 4) & 0x0f0f0f0fu), (int)xs[4 + i], acc, false);
        }
        return acc;
    }
    __device__ __forceinline__ int dotB(const uint32_t* xs, int xsum) const {
        int acc = -8 * xsum;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t q = w[5 + i];
            acc = __builtin_amdgcn_sdot4((int)(q & 0x0f0f0f0fu), (int)xs[i], acc, false);
            acc = __builtin_amdgcn_sdot4((int)((q >> 4) & 0x0f0f0f0fu), (int)xs[4 + i], acc, false);
        }
        return acc;
    }
    // The same dots split by 16-byte chunk c of the pair's 64 activation quants
    // (chunks 0, 1: block A; 2, 3: block B), for callers that stream the
    // activations through a few registers.  dot_chunk<0>(..., -8*sumA) then
    // dot_chunk<1> equals dotA; <2> and <3> likewise dotB.
    template <int C>
    __device__ __forceinline__ int dot_chunk(u32x4 x, int acc) const {
        const uint32_t xv[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t q = C < 2 ? __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2) : w[5 + i];
            const uint32_t n = (C & 1) ? (q >> 4) & 0x0f0f0f0fu : q & 0x0f0f0f0fu;
            acc = __builtin_amdgcn_sdot4((int)n, (int)xv[i], acc, false);
        }
        return acc;
    }
    static constexpr int kZero = 8;  // quant offset: value = q - 8
};

template <> struct WPair<kTypeQ8_0> {
    uint32_t w[17];
    __device__ __forceinline__ void load(const uint8_t* row, int pair) {
        const uint32_t* b = (const uint32_t*)(row + 68 * pair);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4a4 a = *(const u32x4a4*)(b + 4 * i);
            w[4 * i + 0] = a.x; w[4 * i + 1] = a.y; w[4 * i + 2] = a.z; w[4 * i + 3] = a.w;
        }
        w[16] = b[16];
    }
    __device__ __forceinline__ void load32(const uint8_t* base, uint32_t off) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4a4 a = *(const u32x4a4*)(base + (off + 16u * i));
            w[4 * i + 0] = a.x; w[4 * i + 1] = a.y; w[4 * i + 2] = a.z; w[4 * i + 3] = a.w;
        }
        w[16] = *(const uint32_t*)(base + (off + 64u));
    }
    __device__ __forceinline__ float dA() const { return fp16_to_f32(w[0]); }
    __device__ __forceinline__ float dB() const { return fp16_to_f32(w[8] >> 16); }
    __device__ __forceinline__ int dotA(const uint32_t* xs, int /*xsum*/) const {
        int acc = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t q = __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2);
            acc = __builtin_amdgcn_sdot4((int)q, (int)xs[i], acc, false);
        }
        return acc;
    }
    __device__ __forceinline__ int dotB(const uint32_t* xs, int /*xsum*/) const {
        int acc = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc = __builtin_amdgcn_sdot4((int)w[9 + i], (int)xs[i], acc, false);
        return acc;
    }
    template <int C>
    __device__ __forceinline__ int dot_chunk(u32x4 x, int acc) const {
        const uint32_t xv[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t q = C < 2 ? __builtin_amdgcn_alignbyte(w[4 * C + i + 1], w[4 * C + i], 2) : w[9 + 4 * (C - 2) + i];
            acc = __builtin_amdgcn_sdot4((int)q, (int)xv[i], acc, false);
        }
        return acc;
    }
    static constexpr int kZero = 0;
};

// Activation pair in the workspace layout: qs[64] int8 + {dA, sumA, dB, sumB}.
struct XPair {
    uint32_t xs[16];
    float dA, dB;
    int sA, sB;
    __device__ __forceinline__ void load(const int8_t* qs_row, const float2* ds_row, int pair) {
        const u32x4* q = (const u32x4*)(qs_row + 64 * pair);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4 v = q[i];
            xs[4 * i + 0] = v.x; xs[4 * i + 1] = v.y; xs[4 * i + 2] = v.z; xs[4 * i + 3] = v.w;
        }
        // {dA, sumA, dB, sumB}: loaded as integers and bit-cast as scalars (a
        // bit_cast of an ext-vector element reads element 0 in this compiler)
        const u32x4 d = *(const u32x4*)(ds_row + 2 * pair);
        const uint32_t da = d.x, sa = d.y, db = d.z, sb = d.w;
        dA = __builtin_bit_cast(float, da);
        sA = (int)sa;
        dB = __builtin_bit_cast(float, db);
        sB = (int)sb;
    }
};

// Within-row reductions for the h quantization (CTRL moves within a row of 16
// lanes, so every lane has a source and no old value is needed), and the step
// between the two rows of a 32-lane group: the 16-lane swap hands each lane its
// partner's value, the pair is combined in both lanes.
template <int CTRL>
__device__ __forceinline__ float dpp8_max(float v) {
    const float o = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
    return fmaxf(v, o);
}
template <int CTRL>
__device__ __forceinline__ int dpp8_add(int v) {
    return v + __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float xor16_max(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                    false, false);
    return fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}
__device__ __forceinline__ int xor16_add(int v) {
    const auto r = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
    return (int)r[0] + (int)r[1];
}

// h = silu(g)*u (or gelu(g)*u) of one value per lane and the Q8_0 quantization of the 32-value
// block held by a whole aligned 32-lane group (lane fl = value fl): ggml's
// quantize_row_q8_0 (d = fp16(amax/127), q = rint(h*127/amax)) plus the block's
// quant sum.  Writes the lane's quant to qs[fl] and, from lane 0, {d, sum}.
__device__ __forceinline__ void swiglu_q8_block32(float g, float u, int fl, int8_t* qs, float2* ds, int act = kActSilu,
                                                  const uint16_t* gelu_tab = nullptr) {
    const float h = act_mul(act, gelu_tab, g, u);
    float amax = __builtin_fabsf(h);
    amax = dpp8_max<kDppQuadXor1>(amax);
    amax = dpp8_max<kDppQuadXor2>(amax);
    amax = dpp8_max<kDppRowHalfMirror>(amax);
    amax = dpp8_max<kDppRowMirror>(amax);
    amax = xor16_max(amax);
    const float d = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    const int qv = (int)__builtin_rintf(h * id);
    int sum = qv;
    sum = dpp8_add<kDppQuadXor1>(sum);
    sum = dpp8_add<kDppQuadXor2>(sum);
    sum = dpp8_add<kDppRowHalfMirror>(sum);
    sum = dpp8_add<kDppRowMirror>(sum);
    sum = xor16_add(sum);
    qs[fl] = (int8_t)qv;
    if (fl == 0) *ds = make_float2(fp16_to_f32(f32_to_fp16(d)), __builtin_bit_cast(float, sum));
}

// Exact contribution of one weight pair against one activation pair (f64).
template <int WT>
__device__ __forceinline__ double pair_dot(const WPair<WT>& w, const XPair& x) {
    const int ia = w.dotA(x.xs, x.sA);
    const int ib = w.dotB(x.xs + 8, x.sB);
    const float ca = w.dA() * x.dA;  // exact: two 11-bit significands
    const float cb = w.dB() * x.dB;
    return __builtin_fma((double)ca, (double)ia, (double)cb * (double)ib);
}

}  // namespace qmoe
