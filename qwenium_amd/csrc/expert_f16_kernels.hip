// expert_f16_kernels.hip -- grouped expert GEMMs for large token counts
// (prefill) on f16 MFMA (gfx950), plus the exact fixup of h's quantization.
//
// Semantics as the reference's mul_mat_id with Q8_0 activations
// (src/layers/moe.cpp:105-127, shared expert :161-165): per 32-value quant
// block b, y[p][n] += fp32(dw[n][b]) * fp32(dx[p][b]) * isum_b[p][n], with
// isum_b the exact integer dot of the block's quants.
//
// Per block and 32x32 output tile, on the MFMA pipe:
//   isum: two v_mfma_f32_32x32x16_f16 over the quants as f16 (the activation
//         quants q in [-127, 127] and the weights' q - 8 (Q4_0) or q (Q8_0) are
//         exact in f16, and so is every partial sum, < 2^24), exact in f32;
//   scale: one v_mfma_f32_32x32x16_f16 outer product dx (rows) x dw (columns),
//         exact in f32 (two 11-bit significands);
// then one FMA per output, acc += scale * isum, in f32 (as ggml's CPU dot
// accumulates its block terms in f32).  The work per tile is 3 MFMAs (96
// cycles) + ~21 VALU instructions (the 16 FMAs and the weight unpack shared by
// four row tiles); the two pipes overlap only partly (about four independent
// VALU instructions hide under each MFMA), so the loop runs at ~160 SIMD-cycles
// per tile and block with three waves per SIMD.
//
// Tiles come from the routing: tiles[i] = {expert, first row, rows <= 128}.
// A workgroup (4 waves) computes 128 rows x 128 weight columns of one tile;
// each wave owns all 128 rows (four 32-row MFMA tiles) and 32 columns:
//   gate/up: wave w takes gate (w < 2) or up (w >= 2) rows f = 64 y + 32 (w & 1) + lane % 32;
//   down:    output columns n = 128 y + 32 w + lane % 32.
// Activation rows (f16 quants and f16 block scales) are staged in LDS by
// direct global->LDS loads, kF16ChunkK (64) k values per chunk, double
// buffered; weights are read per lane one chunk ahead, from the chunk-major
// copies of the expert matrices when the layer has them (each lane's block pair
// of a chunk next to its neighbours'), else straight from the GGUF rows.
//
// Gate/up epilogue: h = act(g) * u in f32 and the Q8_0 of h per 32-wide block
// (ggml's activation quantizer: d = fp16(amax / 127), q = rint(h * 127 / amax)),
// written as the down GEMM's f16 quants and scales.  The f32 sums differ from
// the exact ones by rounding errors proportional to the partial sums, not to
// the result: each value gets an error estimate from max(|g|, rms of the
// block's 32 g) (likewise u), carried through the activation and the scaling
// by 127 / amax.  A value whose quant is not settled by it (h * 127 / amax
// within the error of a rounding tie; for GeGLU, g within it of an fp16 tie,
// which selects the table entry; a candidate for the block's largest |h| when
// the top two are not clear of each other or amax / 127 is near an fp16 tie)
// is listed with the block's amax candidates, and k_fix_h recomputes them
// exactly (the f64 block sum, rounded once, and the deterministic activation,
// as the CPU restatement does) and requantizes the block with the exact amax
// before the down GEMM reads it.
// Down epilogue: the unweighted expert rows into ybuf for the k-ordered combine.
#include "qmoe_device.h"
#include "qmoe_internal.h"

#include <algorithm>
#include <type_traits>

namespace qmoe {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));
// 4-byte aligned (block pairs are only dword aligned): dwordx3 / dwordx2 loads, nothing wider
typedef uint32_t u32x3 __attribute__((ext_vector_type(3), aligned(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2), aligned(4)));

constexpr int kTM = kMfmaTileM;             // 128 rows per tile
constexpr int kNM = kTM / 32;               // 32-row MFMA tiles per tile
constexpr int kKC = kF16ChunkK;             // k values per LDS chunk
constexpr int kPPC = kKC / 64;              // quant block pairs per chunk
static_assert(kPPC == 1 || kPPC == 2, "chunks of 64 or 128");
constexpr int kLd = kKC + 8;                // LDS row stride in f16 (144 or 272 bytes: conflict-free 16-byte reads)
constexpr int kSlotsPerRow = kLd / 8;       // sixteen-byte slots per row, the last one padding
constexpr int kASlots = kTM * kSlotsPerRow;
constexpr int kAHalfs = kASlots * 8;
constexpr int kDmaIters = (kASlots + 255) / 256;
constexpr int kSinkBytes = 64 * 16;        // the last round's spare waves all land here
static_assert(kASlots % 64 == 0, "a wave's staging slots are all real or all spare");
constexpr int kScaleRounds = kTM * 4 / 256;  // scale dword slots per thread
static_assert(kTM * 4 % 256 == 0, "scale slots");
static_assert(kNM == 4, "the main loop instantiates 1..4 row tiles");
constexpr int kScaleBytes = kTM * 16;       // per row and chunk: its 4 f16 block scales, twice
constexpr int kStageBytes = kAHalfs * 2 + kScaleBytes;
constexpr int kHLd = 64 + 4;                // gate/up epilogue: g and u rows in LDS, f32
constexpr size_t kF16LdsBytes = 2 * (size_t)kStageBytes + kSinkBytes + kTM * 8;
static_assert(2 * 64 * kHLd * 4 <= 2 * (size_t)kStageBytes, "an epilogue pass's g and u rows fit the stage buffers");
// Error model of the gate/up epilogue's f32 values.  The accumulation error of
// g (n block terms summed by fma in f32) relative to max(|g|, rms of the
// block's g) is at most 1.2e-6 over 0.5M emulated values at n = 64; it is
// charged as kAccErr * sqrt(n) (3e-6 at n = 64).  The activation's slope is
// below kActSlope (SiLU 1.10, GELU 1.13; SiLU charges its local slope instead,
// from sigma(g)); the f32 SiLU (within 3.6e-7 (1 + |g|)
// relative) and the product (half an ulp) are within kActRel * (1 + |g|) * |h|
// of the exact ones.
constexpr float kAccErr = 3.75e-7f;
constexpr float kActSlope = 1.13f;
constexpr float kActRel = 4.5e-7f;

struct F16Args {
    int H, F, E;
    const uint8_t* w0; uint64_t w0_nb2;  // gate (gate/up) or down; expert stride
    const uint8_t* w1; uint64_t w1_nb2;  // up (gate/up)
    const uint8_t* sh0;                  // shared gate or shared down
    const uint8_t* sh1;                  // shared up
    // byte strides of a weight row (a GEMM column) and of a block pair: the GGUF
    // rows (nb1, pair bytes) or the chunk-major copies (pair bytes, rows * pair bytes)
    uint32_t w0_cs, w0_ps, w1_cs, w1_ps, sh0_cs, sh0_ps, sh1_cs, sh1_ps;
    const int32_t* counters;                     // [1] n_tiles
    const int4* tiles;
    const int32_t* row_token;                    // gate/up: the token of each output row
    const _Float16* a_q;                         // A quants [rows][K] as f16
    const uint16_t* a_d;                         // A block scales [rows][K/32] (fp16 bits)
    int K;                                       // reduction length (H or F)
    int n_y;                                     // column chunks per tile
    // gate/up: h's quants and scales, the fixup list
    _Float16* h_q; uint16_t* h_d;
    int4* fix;                                   // [max] {row, f block | expert << 16, uncertain values, amax candidates}
    float* fix_h;                                // [max][kFixStride] the block's f32 h values, amax's error
    int32_t* fix_count;
    int fix_max;
    float acc_err;                               // kAccErr * sqrt(K / 32)
    int act; const uint16_t* gelu_tab;
    // down
    float* ybuf;
};

// The bytes of a GGUF block pair (two consecutive 32-value blocks of one
// weight row; pairs start 4-byte aligned) that one lane needs: its k half kh
// of each block's quants and both block scales.
//   Q4_0 (36 bytes): w[0..2] = bytes 8kh .. 8kh+11 (block 0: d0 for kh = 0,
//     quants at 2 + 8kh), w[3] = bytes 16 (kh = 0: d1) or 0 (kh = 1: d0),
//     w[4..5] = bytes 20 + 8kh .. (block 1 quants); kh = 1 finds d1 in w[2].
//   Q8_0 (68 bytes): w[0..2] = bytes 8kh .. (d0 / first quant half of block 0),
//     w[3..5] = bytes 16 + 8kh .. (second half; kh = 1 also d1 at bytes 34-35),
//     w[6] = bytes 32 (kh = 0: d1) or 0 (kh = 1: d0), w[7..8] = bytes 36 + 8kh,
//     w[9..10] = bytes 52 + 8kh (block 1's quant halves).
template <int WT> struct RawPair;
template <> struct RawPair<kTypeQ4_0> {
    uint32_t w[6];
    __device__ __forceinline__ void load(const uint8_t* base, uint32_t off, bool kh) {
        const uint8_t* p = base + off;
        const uint32_t h8 = kh ? 8u : 0u;
        const u32x3 a = *(const u32x3*)(p + h8);
        const u32x2 b = *(const u32x2*)(p + 20 + h8);
        w[0] = a.x; w[1] = a.y; w[2] = a.z;
        w[3] = *(const uint32_t*)(p + (kh ? 0 : 16));
        w[4] = b.x; w[5] = b.y;
    }
};
template <> struct RawPair<kTypeQ8_0> {
    uint32_t w[11];
    __device__ __forceinline__ void load(const uint8_t* base, uint32_t off, bool kh) {
        const uint8_t* p = base + off;
        const uint32_t h8 = kh ? 8u : 0u;
        const u32x3 a = *(const u32x3*)(p + h8);
        const u32x3 b = *(const u32x3*)(p + 16 + h8);
        const u32x2 c = *(const u32x2*)(p + 36 + h8);
        const u32x2 d = *(const u32x2*)(p + 52 + h8);
        w[0] = a.x; w[1] = a.y; w[2] = a.z;
        w[3] = b.x; w[4] = b.y; w[5] = b.z;
        w[6] = *(const uint32_t*)(p + (kh ? 0 : 32));
        w[7] = c.x; w[8] = c.y;
        w[9] = d.x; w[10] = d.y;
    }
};

// Two f16 (1024 + byte) values from two bytes of u (v_perm: 0x64 = the f16
// exponent bits of 1024 in the high byte of each half).
__device__ __forceinline__ uint32_t bytes_1024(uint32_t u, uint32_t sel) {
    return __builtin_amdgcn_perm(0x64646464u, u, sel);
}
constexpr uint32_t kSelB01 = 0x04010400u;  // [b0, 0x64, b1, 0x64]
constexpr uint32_t kSelB23 = 0x04030402u;  // [b2, 0x64, b3, 0x64]

__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }
__device__ __forceinline__ uint32_t as_u32(h2 v) { return __builtin_bit_cast(uint32_t, v); }

// Q4_0 quants of this lane as exact f16 q - 8 (8 bytes u0, u1 = qs[8kh..8kh+7]):
// half 0 = low nibbles (k = 8kh + i), half 1 = high nibbles (k = 16 + 8kh + i).
__device__ __forceinline__ void quants_q4(uint32_t u0, uint32_t u1, v8h (&b)[2]) {
#pragma clang fp contract(off)
    const h2 c1032 = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const h2 c72 = {(_Float16)-72.0f, (_Float16)-72.0f};
    const h2 c16th = {(_Float16)0.0625f, (_Float16)0.0625f};
    const uint32_t p[4] = {bytes_1024(u0, kSelB01), bytes_1024(u0, kSelB23), bytes_1024(u1, kSelB01),
                           bytes_1024(u1, kSelB23)};
    u32x4 lo, hi;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // (1024 + lo) - 1032 = lo - 8; (1024 + 16 hi) / 16 - 72 = hi - 8: both exact
        lo[i] = as_u32(as_h2(p[i] & 0xFF0FFF0Fu) + c1032);
        hi[i] = as_u32(__builtin_elementwise_fma(as_h2(p[i] & 0xFFF0FFF0u), c16th, c72));
    }
    b[0] = __builtin_bit_cast(v8h, lo);
    b[1] = __builtin_bit_cast(v8h, hi);
}

// Q8_0 quants (8 signed bytes) as exact f16: (1024 + (q ^ 0x80)) - 1152 = q.
__device__ __forceinline__ v8h quants_q8(uint32_t u0, uint32_t u1) {
#pragma clang fp contract(off)
    const h2 c1152 = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const uint32_t a = u0 ^ 0x80808080u, b = u1 ^ 0x80808080u;
    const uint32_t p[4] = {bytes_1024(a, kSelB01), bytes_1024(a, kSelB23), bytes_1024(b, kSelB01),
                           bytes_1024(b, kSelB23)};
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = as_u32(as_h2(p[i]) + c1152);
    return __builtin_bit_cast(v8h, r);
}

// Quants (two MFMA halves) and the fp16 scale bits of block j (0/1) of a raw pair.
template <int WT>
__device__ __forceinline__ uint32_t block_quants(const RawPair<WT>& r, int j, bool kh, v8h (&b)[2]);

template <>
__device__ __forceinline__ uint32_t block_quants<kTypeQ4_0>(const RawPair<kTypeQ4_0>& r, int j, bool kh, v8h (&b)[2]) {
    if (j == 0) {
        // block 0: quants at bytes 2 + 8kh .. 9 + 8kh = bytes 2..9 of w[0..2]
        quants_q4(__builtin_amdgcn_alignbyte(r.w[1], r.w[0], 2), __builtin_amdgcn_alignbyte(r.w[2], r.w[1], 2), b);
        return (kh ? r.w[3] : r.w[0]) & 0xffffu;
    }
    quants_q4(r.w[4], r.w[5], b);
    return (kh ? r.w[2] : r.w[3]) >> 16;
}

template <>
__device__ __forceinline__ uint32_t block_quants<kTypeQ8_0>(const RawPair<kTypeQ8_0>& r, int j, bool kh, v8h (&b)[2]) {
    if (j == 0) {
        b[0] = quants_q8(__builtin_amdgcn_alignbyte(r.w[1], r.w[0], 2), __builtin_amdgcn_alignbyte(r.w[2], r.w[1], 2));
        b[1] = quants_q8(__builtin_amdgcn_alignbyte(r.w[4], r.w[3], 2), __builtin_amdgcn_alignbyte(r.w[5], r.w[4], 2));
        return (kh ? r.w[6] : r.w[0]) & 0xffffu;
    }
    b[0] = quants_q8(r.w[7], r.w[8]);
    b[1] = quants_q8(r.w[9], r.w[10]);
    return (kh ? r.w[5] : r.w[6]) >> 16;
}

// fp16 bit patterns: -0 as +0, and the next value up of a finite one (toward
// zero for negatives; -min subnormal's next is 0).
__device__ __forceinline__ uint32_t fp16_canon(uint32_t h) { return h == 0x8000u ? 0u : h; }
__device__ __forceinline__ uint32_t fp16_next_up(uint32_t h) { return fp16_canon((h & 0x8000u) ? h - 1u : h + 1u); }

__device__ __forceinline__ v16f mfma16(v8h a, v8h b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// silu(g) (moe.cpp:117) or ggml's tabled gelu(g) (gemma4.cpp:423) in f32.
// SiLU: exp (argument error |g| 6e-8 relative, 1 ulp), 1 + e, a 1-ulp
// reciprocal and the product: within 3.6e-7 (1 + |g|) of silu(g) relative.
template <int ACT>
__device__ __forceinline__ float act_f32(const uint16_t* tab, float g) {
    if (ACT == kActGeluTanh) {
        if (g <= -10.0f) return 0.0f;
        if (g >= 10.0f) return g;
        return fp16_to_f32(tab[f32_to_fp16(g) & 0xffffu]);
    }
    return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}

// One 32-wide block of h from its 32 g and u values in LDS (pg, pu; h and its
// error bound overwrite them): the Q8_0 of h into h_q / h_d, and the block into
// the fixup list when a quant (or the amax) is not settled by the error bound.
// Row p of the tile lists, f block fb, expert e.
template <int ACT>
__device__ __forceinline__ void h_block(const F16Args& a, f32x4* pg, f32x4* pu, uint64_t p, int fb, int e) {
    const int nfb = a.F >> 5;
    float sg = 0.0f, su = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const f32x4 g4 = pg[i], u4 = pu[i];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            sg = __builtin_fmaf(g4[k], g4[k], sg);
            su = __builtin_fmaf(u4[k], u4[k], su);
        }
    }
    const float rg = __builtin_sqrtf(sg * (1.0f / 32.0f)), ru = __builtin_sqrtf(su * (1.0f / 32.0f));
    // h and its error bound eh (over g and u in LDS); the exact block amax
    // lies within amax +- emax (emax: the block's largest eh)
    float amax = 0.0f, emax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const f32x4 g4 = pg[i], u4 = pu[i];
        f32x4 h4, e4;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float gv = g4[k], uv = u4[k];
            const float ag = __builtin_fabsf(gv), au = __builtin_fabsf(uv);
            // GeGLU: the table entries at fp16(g) and at the ends of g's error
            // range, loaded unconditionally (16-bit indices) so that no load waits
            // behind a branch
            float av, tl = 0.0f, th = 0.0f, lo = 0.0f, hi = 0.0f, eg = 0.0f, sgm = 0.0f;
            uint32_t l16 = 0, h16 = 0;
            if (ACT == kActGeluTanh) {
                eg = a.acc_err * fmaxf(ag, rg);
                lo = gv - eg;
                hi = gv + eg;
                l16 = f32_to_fp16(lo) & 0xffffu;
                h16 = f32_to_fp16(hi) & 0xffffu;
                const float tv = fp16_to_f32(a.gelu_tab[f32_to_fp16(gv) & 0xffffu]);
                tl = fp16_to_f32(a.gelu_tab[l16]);
                th = fp16_to_f32(a.gelu_tab[h16]);
                av = gv <= -10.0f ? 0.0f : (gv >= 10.0f ? gv : tv);
            } else {
                sgm = __builtin_amdgcn_rcpf(1.0f + __expf(-gv));  // act_f32's SiLU, its sigma kept
                av = gv * sgm;
            }
            const float h = av * uv;
            const float ah = __builtin_fabsf(h);
            // g and u are within eg = acc_err max(|g|, rg) and eu = acc_err
            // max(|u|, ru); the activation's error: SiLU's from g's error through
            // its slope.  GeGLU's: at g >= 10 the activation is g itself (error
            // eg), at g <= -10 it is 0; between, it is the table entry at fp16(g),
            // and the exact g's fp16 lies in [fp16(g - eg), fp16(g + eg)]: one
            // value leaves the entry exact, two adjacent values leave it one of
            // two entries (within their difference), a wider range or one
            // crossing +-10 is bounded through the slope
            float eh;
            if (ACT == kActGeluTanh) {
                const uint32_t cl = fp16_canon(l16), ch = fp16_canon(h16);
                const bool near = lo > -10.0f && hi < 10.0f && (cl == ch || fp16_next_up(cl) == ch);
                const float wide = kActSlope * (fp16_to_f32(h16) - fp16_to_f32(l16) + 2.0f * eg) + 2e-3f * __builtin_fabsf(av);
                const float eav = lo >= 10.0f ? eg : (hi <= -10.0f ? 0.0f : (near ? __builtin_fabsf(th - tl) : wide));
                eh = au * eav + __builtin_fabsf(av) * (a.acc_err * fmaxf(au, ru));
            } else {
                // |u| slope eg + |av| eu, the slope over g's error range from sigma(g):
                // |silu'(g)| = |s + silu(g) (1 - s)|, plus 0.5 eg (|silu''| <= 0.5) and
                // 1e-3 for the f32 sigma
                const float egs = a.acc_err * fmaxf(ag, rg);
                const float sl = __builtin_fabsf(__builtin_fmaf(av, 1.0f - sgm, sgm)) + __builtin_fmaf(0.5f, egs, 1e-3f);
                eh = __builtin_fmaf(au * sl, egs, __builtin_fabsf(av) * (a.acc_err * fmaxf(au, ru)));
            }
            eh = __builtin_fmaf(kActRel, __builtin_fmaf(ag, ah, ah), eh);
            h4[k] = h;
            e4[k] = eh;
            amax = fmaxf(amax, ah);
            emax = fmaxf(emax, eh);
        }
        pg[i] = h4;
        pu[i] = e4;
    }
    // error bound of the f32 amax: the largest error bound among the values that
    // could be the largest |h| (|h| + eh >= amax - emax); the exact amax lies
    // within amax +- ea.  GeGLU only: there one value whose fp16(g) is open can
    // carry a bound far above the rest, and the block max would widen every
    // value's quant test with it (a CPU emulation of the flags: 15.5% of the
    // blocks listed against 5.2%); with SiLU the extra pass costs more than the
    // few fixups it saves.
    float ea = emax;
    if constexpr (ACT == kActGeluTanh) {
        const float thr0 = amax - emax;
        ea = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const f32x4 h4 = pg[i], e4 = pu[i];
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (__builtin_fabsf(h4[k]) + e4[k] >= thr0) ea = fmaxf(ea, e4[k]);
        }
    }
    const float amax_lo = amax - ea;
    const float d = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    // t = h * 127 / amax is within et = eh id + |t| (ea id / 127 + 2.5e-7) of
    // the exact one (amax's own error and the product's rounding included)
    const float c1 = __builtin_fmaf(ea * id, 1.0f / 127.0f, 2.5e-7f);
    // quants; a value whose t lies within et of a rounding tie is uncertain;
    // a value whose range reaches amax_lo could be the exact largest |h|
    uint32_t unsure = 0, cand = 0;
    u32x4* hq = (u32x4*)(a.h_q + p * a.F + 32 * fb);
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
        uint32_t packed[4];
#pragma unroll
        for (int ii = 0; ii < 2; ++ii) {
            const f32x4 h4 = pg[i + ii], e4 = pu[i + ii];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int v = 4 * (i + ii) + k;
                const float t = h4[k] * id;
                const float q = __builtin_rintf(t);
                const float et = __builtin_fmaf(e4[k], id, __builtin_fabsf(t) * c1);
                if (__builtin_fabsf(__builtin_fabsf(t - q) - 0.5f) <= et) unsure |= 1u << v;
                if (__builtin_fabsf(h4[k]) + e4[k] >= amax_lo) cand |= 1u << v;
                const uint32_t qb = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)q);
                packed[2 * ii + (k >> 1)] = (k & 1) ? (packed[2 * ii + (k >> 1)] | (qb << 16)) : qb;
            }
        }
        hq[i >> 1] = u32x4{packed[0], packed[1], packed[2], packed[3]};
    }
    a.h_d[p * nfb + fb] = (uint16_t)f32_to_fp16(d);
    // the block's largest |h| is open when several values could be it or
    // amax / 127 is near an fp16 tie (then its candidates are uncertain values too)
    const bool amax_open = __builtin_popcount(cand) > 1 ||
                           f32_to_fp16(amax_lo / 127.0f) != f32_to_fp16((amax + ea) / 127.0f);
    const uint32_t mask = unsure | (amax_open ? cand : 0u);
    if (mask) {
        const int slot = atomicAdd(a.fix_count, 1);
        if (slot < a.fix_max) {
            f32x4* fh = (f32x4*)(a.fix_h + (uint64_t)slot * kFixStride);
#pragma unroll
            for (int i = 0; i < 8; ++i) fh[i] = pg[i];
            fh[8] = f32x4{ea, 0.0f, 0.0f, 0.0f};
            a.fix[slot] = make_int4((int)p, fb | (e << 16), (int)mask, (int)cand);
        }
    }
}

template <int WT, bool GATEUP, int ACT>
__global__ __launch_bounds__(256, 3) void k_expert_f16(F16Args a) {
    extern __shared__ __align__(16) uint8_t s_dyn[];
    // [2 stages] {A quants [128][kLd] f16, block scale records [128][8] f16 (the
    // 4 scales twice)}, the sink, A row offsets [128], scale row offsets [128]
    uint8_t* s_stage = s_dyn;
    uint32_t* s_rowoff = (uint32_t*)(s_dyn + 2 * kStageBytes + kSinkBytes);
    uint32_t* s_doff = s_rowoff + kTM;
    // XCD-aware mapping (workgroups are dealt to the 8 XCDs round-robin): XCD x
    // takes tiles x, x + 8, ... and all column chunks of each, so a tile's
    // activation rows are read into one L2 and the XCDs get statistically
    // equal shares of the (unequal) tiles.  (Contiguous work-balanced expert
    // ranges per XCD fetch less past the L2s but run slower, most of all under
    // skewed routing.)
    const int jb = (int)(blockIdx.x >> 3);
    const int tile_local = jb / a.n_y, y = jb - tile_local * a.n_y;
    const int tile_id = (int)(blockIdx.x & 7) + 8 * tile_local;
    if (tile_id >= a.counters[1]) return;
    const int4 tile = a.tiles[tile_id];
    const int e = tile.x, p0 = tile.y, nr = tile.z;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;  // wave: scalar
    const int col = lane & 31;
    const bool kh = lane >= 32;
    const bool sh = e >= a.E;
    const int nm = (nr + 31) >> 5;  // 32-row MFMA tiles with rows (wave-uniform)
    const int nblk = a.K >> 5;

    if (tid < kTM) {
        const int pr = p0 + min(tid, nr - 1);
        const int arow = GATEUP ? a.row_token[pr] : pr;
        s_rowoff[tid] = (uint32_t)arow * (uint32_t)a.K;
        s_doff[tid] = (uint32_t)arow * (uint32_t)nblk;
    }
    __syncthreads();

    // this lane's weight row (wave-uniform slab base + 32-bit row offset: an
    // expert's slab is far below 4 GiB)
    const uint8_t* wbase;
    uint32_t woff, wps;
    int out_col;
    if (GATEUP) {
        const bool up = wave >= 2;
        const int f = y * 64 + 32 * (wave & 1) + col;
        wbase = up ? (sh ? a.sh1 : a.w1 + (uint64_t)e * a.w1_nb2) : (sh ? a.sh0 : a.w0 + (uint64_t)e * a.w0_nb2);
        woff = (uint32_t)f * (up ? (sh ? a.sh1_cs : a.w1_cs) : (sh ? a.sh0_cs : a.w0_cs));
        wps = up ? (sh ? a.sh1_ps : a.w1_ps) : (sh ? a.sh0_ps : a.w0_ps);
        out_col = f;
    } else {
        out_col = y * 128 + 32 * wave + col;
        wbase = sh ? a.sh0 : a.w0 + (uint64_t)e * a.w0_nb2;
        woff = (uint32_t)out_col * (sh ? a.sh0_cs : a.w0_cs);
        wps = sh ? a.sh0_ps : a.w0_ps;
    }
    constexpr uint32_t kPairBytes = 2 * BlockTraits<WT>::kBytes;
    const int npairs = nblk >> 1;
    const int nchunk = (nblk + 2 * kPPC - 1) / (2 * kPPC);

    // direct global->LDS staging of chunk c.  Quants: slot s = row * kSlotsPerRow
    // + unit (the last unit is the row's padding); every wave issues exactly kDmaIters
    // unconditional loads (a count the wait counters can track): slots past
    // the buffer land in the sink, the padding unit reloads the chunk's first
    // 16 bytes of the row into a slot that is never read.  K is a multiple of
    // 64; with 128-wide chunks a last chunk holds 2 or 4 blocks, and a 2-block
    // one reads up to 128 bytes of quants and 4 bytes of scales past a row (the
    // A buffers end in padding) into slots that are never read.  This lane's
    // source offsets (row offset + 8 unit) are computed once.
    uint32_t soff[kDmaIters];
#pragma unroll
    for (int it = 0; it < kDmaIters; ++it) {
        const int s = min(it * 256 + wave * 64 + lane, kASlots - 1);
        const int r = s / kSlotsPerRow;
        const int u = s - r * kSlotsPerRow;
        soff[it] = s_rowoff[r] + (u < kSlotsPerRow - 1 ? 8 * u : 0);
    }
    // Scales: each row's 16-byte record holds the chunk's block scales: with
    // 128-wide chunks its 4 scales twice (dword d = blocks 2 (d & 1), + 1), with
    // 64-wide chunks its 2 scales four times; lane slot sl = (row, dword) =
    // (sl / 4, sl % 4), two rounds of 64 slots per wave.  The scale MFMA's B
    // operand is zero at k >= 2 kPPC, so the copies (finite) add nothing.
    uint32_t doff[kScaleRounds];
#pragma unroll
    for (int rd = 0; rd < kScaleRounds; ++rd) {
        const int sl = 256 * rd + wave * 64 + lane;
        doff[rd] = s_doff[sl >> 2] + (kPPC == 2 ? 2 * (sl & 1) : 0);
    }
    auto stage = [&](int c, int buf) {
        uint8_t* st = s_stage + buf * kStageBytes;
        const uint32_t k0 = (uint32_t)(c * kKC);
#pragma unroll
        for (int it = 0; it < kDmaIters; ++it) {
            const int s0 = it * 256 + wave * 64;
            const void* dst = s0 < kASlots ? (const void*)(st + s0 * 16) : (const void*)(s_stage + 2 * kStageBytes);
            dma_lds16(a.a_q + k0, 2u * soff[it], __builtin_amdgcn_readfirstlane(lds_addr(dst)));  // wave-uniform
        }
        // a 2-block last chunk: the odd dwords (blocks 2, 3, past the row) reload
        // blocks 0, 1, so every scale the MFMA multiplies (by 0 or not) is finite
        const uint32_t back = (kPPC == 2 && 4 * c + 4 > nblk && (lane & 1)) ? 4u : 0u;
#pragma unroll
        for (int rd = 0; rd < kScaleRounds; ++rd)
            dma_lds4(a.a_d + 2 * kPPC * c, 2u * doff[rd] - back,
                     __builtin_amdgcn_readfirstlane(lds_addr(st + kAHalfs * 2 + (256 * rd + wave * 64) * 4)));
    };

    v16f acc[kNM];
#pragma unroll
    for (int m = 0; m < kNM; ++m) acc[m] = v16f{};

    // weights one whole chunk ahead: chunk c's kPPC pairs live in wa (c even) or
    // wb (c odd), so nothing inside a chunk waits on memory.  The second pair
    // of a 2-block last 128-wide chunk reloads the first (never used).
    RawPair<WT> wa[kPPC], wb[kPPC];  // [pair of the chunk]
    auto fetch = [&](int c, RawPair<WT>(&dst)[kPPC]) {
#pragma unroll
        for (int pp = 0; pp < kPPC; ++pp) {
            const int pair = min(kPPC * c + pp, npairs - 1);
            dst[pp].load(wbase, woff + (uint32_t)pair * wps, kh);
        }
    };
    // this lane's A fragment: row col of each 32-row tile, k offset 8 kh (+ 16 for half 1)
    const int arow0 = col * kLd + (kh ? 8 : 0);
    // the main loop for NM row tiles with rows (a wave-uniform count)
    auto run = [&](auto nm_c) {
        constexpr int NM = decltype(nm_c)::value;
        auto chunk = [&](int c, const RawPair<WT>(&cur)[kPPC], RawPair<WT>(&nxt)[kPPC]) {
            __builtin_amdgcn_s_waitcnt(0);  // chunk c's LDS loads and weights (issued a chunk ago) have landed
            __syncthreads();                // ... for every wave; stage (c + 1) & 1 is no longer read
            if (c + 1 < nchunk) {
                fetch(c + 1, nxt);
                stage(c + 1, (c + 1) & 1);
            }
            const uint8_t* st = s_stage + (c & 1) * kStageBytes;
            const _Float16* aq = (const _Float16*)st;
            const uint8_t* srec = st + kAHalfs * 2 + col * 16;  // this lane's row (32 m + col) scale record
            const int np = min(kPPC, npairs - kPPC * c);
#pragma unroll
            for (int pp = 0; pp < kPPC; ++pp) {
                if (pp >= np) break;  // uniform
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int bl = 2 * pp + j;  // block within the chunk
                    v8h bq[2];
                    const uint32_t dw = block_quants<WT>(cur[pp], j, kh, bq);
                    // the outer product's B: dw at element bl of lanes 0..31 (k = bl),
                    // zero elsewhere; its A is the row's record {dx0..dx3, dx0..dx3}:
                    // D = dx_bl * dw, exact
                    const uint32_t dwl = kh ? 0u : dw;
                    u32x4 bsw = {0u, 0u, 0u, 0u};
                    bsw[bl >> 1] = (bl & 1) ? (dwl << 16) : dwl;
                    const v8h bs = __builtin_bit_cast(v8h, bsw);
#pragma unroll
                    for (int m = 0; m < NM; ++m) {
                        const int o = arow0 + 32 * m * kLd + 32 * bl;
                        const v8h aq0 = *(const v8h*)(aq + o);
                        const v8h aq1 = *(const v8h*)(aq + o + 16);
                        const v8h as = *(const v8h*)(srec + 32 * m * 16);
                        const v16f sc = mfma16(as, bs, v16f{});
                        v16f P = mfma16(aq0, bq[0], v16f{});
                        P = mfma16(aq1, bq[1], P);
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[m][r] = __builtin_fmaf(sc[r], P[r], acc[m][r]);
                    }
                }
            }
        };
        for (int c = 0; c < nchunk; c += 2) {
            chunk(c, wa, wb);
            if (c + 1 < nchunk) chunk(c + 1, wb, wa);
        }
    };
    fetch(0, wa);
    stage(0, 0);
    switch (nm) {
        case 1: run(std::integral_constant<int, 1>{}); break;
        case 2: run(std::integral_constant<int, 2>{}); break;
        case 3: run(std::integral_constant<int, 3>{}); break;
        default: run(std::integral_constant<int, 4>{}); break;
    }

    if (!GATEUP) {
        // unweighted expert rows (lane: column out_col, rows 32 m + 8 (r / 4) + 4 kh + r % 4)
#pragma unroll
        for (int m = 0; m < kNM; ++m)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = 32 * m + 8 * (r >> 2) + (kh ? 4 : 0) + (r & 3);
                if (row < nr) a.ybuf[(uint64_t)(p0 + row) * a.H + out_col] = acc[m][r];
            }
        return;
    }

    // gate/up epilogue, in passes of kEH rows (the g and u rows of a pass in
    // LDS, over the stage buffers: free once every wave is done).
    // 1) g (waves 0, 1) and u (waves 2, 3) of the pass's row tiles into LDS;
    // 2) one thread per (row, 32-wide f block): the thread's 32 g and u values
    //    stay in LDS, h and its error estimate overwrite them there (three
    //    passes of 16-byte reads, few registers).
    constexpr int kEH = 64;
    float* s_g = (float*)s_dyn;
    float* s_u = s_g + kEH * kHLd;
    const int nfb = a.F >> 5;
    auto epi = [&](int row, int lrow, int jb2) {
        const int fb = y * 2 + jb2;  // f block of h
        if (row >= nr || fb >= nfb) return;
        h_block<ACT>(a, (f32x4*)(s_g + lrow * kHLd + 32 * jb2), (f32x4*)(s_u + lrow * kHLd + 32 * jb2),
                     (uint64_t)(p0 + row), fb, e);
    };
#pragma unroll
    for (int half = 0; half < kTM / kEH; ++half) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        {
            float* dst = wave >= 2 ? s_u : s_g;
            const int fl = 32 * (wave & 1) + col;
#pragma unroll
            for (int mm = 0; mm < kEH / 32; ++mm)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int lrow = 32 * mm + 8 * (r >> 2) + (kh ? 4 : 0) + (r & 3);
                    dst[lrow * kHLd + fl] = acc[half * (kEH / 32) + mm][r];
                }
        }
        __syncthreads();
        if (tid < 2 * kEH) epi(half * kEH + (tid & (kEH - 1)), tid & (kEH - 1), tid / kEH);
    }
}

// Exact recomputation of listed h blocks (one wave per block): each uncertain
// value gets g and u as the exact f64 sum of its block terms fp32(dw) *
// fp32(dx) * isum rounded once to f32 and the deterministic activation (the
// CPU restatement's values); the block is then requantized from its 32 values.
struct FixArgs {
    int H, F, E;
    const uint8_t* wg; uint64_t wg_nb1, wg_nb2;
    const uint8_t* wu; uint64_t wu_nb1, wu_nb2;
    const uint8_t* sg; uint64_t sg_nb1;
    const uint8_t* su; uint64_t su_nb1;
    const int32_t* row_token;
    const int8_t* xq_qs; const float2* xq_ds;  // x's Q8_0 quants [T][H], {scale, quant sum} [T][H/32]
    const int4* fix; const float* fix_h; const int32_t* fix_count; int fix_max;
    _Float16* h_q; uint16_t* h_d;
    int act; const uint16_t* gelu_tab;
};

// The exact gate and up dots of weight rows rg, ru with one token's int8
// quants over the lanes of a 32-lane half (lane l32 takes block pairs l32,
// l32 + 32, ...): each block term fp32(dw) * fp32(dx) * isum is exact in f64
// (a 22-bit scale product times a 19-bit integer); the caller sums them over
// the half.
template <int WT>
__device__ void exact_gu_part(const uint8_t* rg, const uint8_t* ru, const int8_t* xqs, const float2* xds, int npairs,
                              int l32, double& g, double& u) {
    g = 0.0;
    u = 0.0;
    for (int pr = l32; pr < npairs; pr += 32) {
        WPair<WT> wg, wu;
        wg.load(rg, pr);
        wu.load(ru, pr);
        XPair xp;
        xp.load(xqs, xds, pr);
        // fp32(dw) * fp32(dx) is exact in f32
        g += (double)(wg.dA() * xp.dA) * (double)wg.dotA(xp.xs, xp.sA) +
             (double)(wg.dB() * xp.dB) * (double)wg.dotB(xp.xs + 8, xp.sB);
        u += (double)(wu.dA() * xp.dA) * (double)wu.dotA(xp.xs, xp.sA) +
             (double)(wu.dB() * xp.dB) * (double)wu.dotB(xp.xs + 8, xp.sB);
    }
}

__device__ __forceinline__ double readlane_f64(double v, int l) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), l);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// One 32-lane half per listed block, its uncertain values one at a time (lane
// l takes weight block pairs l, l + 32, ...), each from the exact f64 gate and
// up sums rounded once to f32 and the deterministic activation.  The block is
// then requantized with the f32 amax if every recomputed value's quant is
// settled despite amax's error, else with the exact amax (its candidates
// recomputed as well).
template <int WT>
__device__ __forceinline__ void fix_values(const FixArgs& a, uint32_t todo, int fb, int e, bool sh, const int8_t* xqs,
                                           const float2* xds, float& h) {
    const int l32 = threadIdx.x & 31;
    const bool upper = (threadIdx.x & 63) >= 32;
    while (todo) {
        const int v = __builtin_ctz(todo);
        todo &= todo - 1;
        const int f = 32 * fb + v;
        const uint8_t* rg = sh ? a.sg + (uint64_t)f * a.sg_nb1 : a.wg + (uint64_t)e * a.wg_nb2 + (uint64_t)f * a.wg_nb1;
        const uint8_t* ru = sh ? a.su + (uint64_t)f * a.su_nb1 : a.wu + (uint64_t)e * a.wu_nb2 + (uint64_t)f * a.wu_nb1;
        double gd, ud;
        exact_gu_part<WT>(rg, ru, xqs, xds, a.H >> 6, l32, gd, ud);
        gd = dpp_sum_f64<32>(gd);  // half sums in lanes 31 and 63
        ud = dpp_sum_f64<32>(ud);
        const double g = upper ? readlane_f64(gd, 63) : readlane_f64(gd, 31);
        const double u = upper ? readlane_f64(ud, 63) : readlane_f64(ud, 31);
        const float hv = act_mul(a.act, a.gelu_tab, (float)g, (float)u);
        if (l32 == v) h = hv;
    }
}

__device__ __forceinline__ float half_max(float v) {
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

template <int WT>
__global__ __launch_bounds__(256) void k_fix_h(FixArgs a) {
    const int l32 = threadIdx.x & 31;
    const bool upper = (threadIdx.x & 63) >= 32;
    const int n = min(*a.fix_count, a.fix_max);
    const int nblk = a.H >> 5;
    for (int i = blockIdx.x * 8 + (int)(threadIdx.x >> 5); i < n; i += gridDim.x * 8) {
        const int4 ent = a.fix[i];
        const int p = ent.x, fb = ent.y & 0xffff, e = ent.y >> 16;
        const uint32_t unsure = (uint32_t)ent.z, cand = (uint32_t)ent.w;
        const bool sh = e >= a.E;
        const int t = a.row_token[p];
        const int8_t* xqs = a.xq_qs + (uint64_t)t * a.H;
        const float2* xds = a.xq_ds + (uint64_t)t * nblk;
        const float* fh = a.fix_h + (uint64_t)i * kFixStride;
        float h = fh[l32];  // value l32 of the block
        const float ea = fh[32];
        fix_values<WT>(a, unsure, fb, e, sh, xqs, xds, h);
        float amax = half_max(__builtin_fabsf(h));
        const uint32_t rest = cand & ~unsure;
        if (rest) {
            // amax is one of the f32 candidates: is every recomputed quant settled
            // under amax's error?
            const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
            const float tv = h * id, at = __builtin_fabsf(tv);
            const bool open = ((unsure >> l32) & 1u) &&
                              __builtin_fabsf(__builtin_fabsf(tv - __builtin_rintf(tv)) - 0.5f) <=
                                  at * (ea * 1.01f / amax + 2.5e-7f);
            const uint64_t ball = __ballot(open);
            if ((upper ? (ball >> 32) : (ball & 0xffffffffull)) != 0) {
                fix_values<WT>(a, rest, fb, e, sh, xqs, xds, h);
                amax = half_max(__builtin_fabsf(h));
            }
        }
        // requantize the block from its 32 values
        const float d = amax / 127.0f;
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        a.h_q[(uint64_t)p * a.F + 32 * fb + l32] = (_Float16)__builtin_rintf(h * id);
        if (l32 == 0) a.h_d[(uint64_t)p * (a.F >> 5) + fb] = (uint16_t)f32_to_fp16(d);
    }
}

// Chunk-major copy of one expert matrix: pair p of row r of expert e (GGUF rows
// of nb1 bytes, experts nb2 apart) to dst + ((e * npairs + p) * rows + r) * pb.
// One thread per dword of the copy (pairs and rows are 4-byte aligned).
__global__ __launch_bounds__(256) void k_repack_pairs(const uint8_t* src, uint64_t nb1, uint64_t nb2, int rows,
                                                      int npairs, int pb, uint64_t n_dwords, uint8_t* dst) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n_dwords) return;
    const int pd = pb >> 2;
    const uint64_t q = i / (uint64_t)pd;  // pair index in the copy: (e * npairs + p) * rows + r
    const int w = (int)(i - q * pd);
    const uint64_t r = q % (uint64_t)rows, ep = q / (uint64_t)rows;
    const uint64_t p = ep % (uint64_t)npairs, e = ep / (uint64_t)npairs;
    ((uint32_t*)dst)[i] = *(const uint32_t*)(src + e * nb2 + r * nb1 + p * (uint64_t)pb + 4u * (uint32_t)w);
}

static size_t pk_bytes(int type, int rows, int k, int nexp) {
    const int pb = 2 * (type == kTypeQ4_0 ? BlockTraits<kTypeQ4_0>::kBytes : BlockTraits<kTypeQ8_0>::kBytes);
    return (size_t)nexp * (size_t)(k / 64) * (size_t)rows * (size_t)pb;
}

static hipError_t repack(const uint8_t* src, uint64_t nb1, uint64_t nb2, int type, int rows, int k, int nexp,
                         uint8_t* dst) {
    const int pb = 2 * (type == kTypeQ4_0 ? BlockTraits<kTypeQ4_0>::kBytes : BlockTraits<kTypeQ8_0>::kBytes);
    const uint64_t n = (uint64_t)pk_bytes(type, rows, k, nexp) / 4;
    hipLaunchKernelGGL(k_repack_pairs, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, nullptr, src, nb1, nb2, rows,
                       k / 64, pb, n, dst);
    return hipGetLastError();
}

hipError_t build_prefill_copies(LayerDesc& d) {
    const size_t g = pk_bytes(d.gu_type, d.F, d.H, d.E), dn = pk_bytes(d.dn_type, d.H, d.F, d.E);
    const size_t sg = d.S ? pk_bytes(d.gu_type, d.F, d.H, 1) : 0, sd = d.S ? pk_bytes(d.dn_type, d.H, d.F, 1) : 0;
    void* base = nullptr;
    hipError_t err = hipMalloc(&base, 2 * g + dn + 2 * sg + sd);
    if (err != hipSuccess) return err;
    uint8_t* p = (uint8_t*)base;
    uint8_t* pg = p; p += g;
    uint8_t* pu = p; p += g;
    uint8_t* pd = p; p += dn;
    uint8_t* psg = d.S ? p : nullptr; p += sg;
    uint8_t* psu = d.S ? p : nullptr; p += sg;
    uint8_t* psd = d.S ? p : nullptr;
    if (err == hipSuccess) err = repack(d.w_gate, d.gate_nb1, d.gate_nb2, d.gu_type, d.F, d.H, d.E, pg);
    if (err == hipSuccess) err = repack(d.w_up, d.up_nb1, d.up_nb2, d.gu_type, d.F, d.H, d.E, pu);
    if (err == hipSuccess) err = repack(d.w_down, d.down_nb1, d.down_nb2, d.dn_type, d.H, d.F, d.E, pd);
    if (d.S) {
        if (err == hipSuccess) err = repack(d.w_sh_gate, d.sh_gate_nb1, 0, d.gu_type, d.F, d.H, 1, psg);
        if (err == hipSuccess) err = repack(d.w_sh_up, d.sh_up_nb1, 0, d.gu_type, d.F, d.H, 1, psu);
        if (err == hipSuccess) err = repack(d.w_sh_down, d.sh_down_nb1, 0, d.dn_type, d.H, d.F, 1, psd);
    }
    if (err == hipSuccess) err = hipDeviceSynchronize();
    if (err != hipSuccess) {
        (void)hipFree(base);
        return err;
    }
    d.pk_base = base;
    d.pk_gate = pg; d.pk_up = pu; d.pk_down = pd;
    d.pk_sh_gate = psg; d.pk_sh_up = psu; d.pk_sh_down = psd;
    return hipSuccess;
}

// A weight operand of the prefill GEMMs: its chunk-major copy when the layer has
// one (rows of the matrix, k its reduction length), else the GGUF rows.
static void set_weights(const uint8_t*& w, uint64_t& nb2, uint32_t& cs, uint32_t& ps, const uint8_t* pk,
                        const uint8_t* gguf, uint64_t gguf_nb1, uint64_t gguf_nb2, int type, int rows, int k) {
    const uint32_t pb = 2 * (type == kTypeQ4_0 ? BlockTraits<kTypeQ4_0>::kBytes : BlockTraits<kTypeQ8_0>::kBytes);
    if (pk) {
        w = pk;
        nb2 = (uint64_t)(k / 64) * (uint64_t)rows * pb;
        cs = pb;
        ps = (uint32_t)rows * pb;
    } else {
        w = gguf;
        nb2 = gguf_nb2;
        cs = (uint32_t)gguf_nb1;
        ps = pb;
    }
}

static F16Args base_f16_args(const LayerDesc& L, const Workspace& ws) {
    F16Args a{};
    a.H = L.H; a.F = L.F; a.E = L.E;
    a.counters = ws.counters;
    a.tiles = ws.tiles;
    a.row_token = ws.row_token;
    a.h_q = ws.h_q; a.h_d = ws.h_d;
    a.fix = ws.fix; a.fix_h = ws.fix_h; a.fix_count = ws.counters + kCounterFix; a.fix_max = ws.fix_max;
    a.acc_err = kAccErr * sqrtf((float)(L.H / 32));
    a.ybuf = ws.ybuf;
    a.act = L.act;
    a.gelu_tab = L.gelu_tab;
    return a;
}

static int f16_max_tiles(const LayerDesc& L, const Workspace& ws, int T) {
    return min(ws.max_tiles, (T * L.K + kTM - 1) / kTM + min(L.E, T * L.K) + (L.S ? (T + kTM - 1) / kTM : 0));
}

template <typename Kern>
static hipError_t launch_f16(Kern kern, dim3 grid, hipStream_t stream, hipEvent_t ev_start, hipEvent_t ev_stop,
                             const F16Args& a) {
    // above the 64 KiB default dynamic LDS window: raise it (idempotent)
    hipError_t err = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kF16LdsBytes);
    if (err != hipSuccess) return err;
    launch_timed(kern, grid, dim3(256), kF16LdsBytes, stream, ev_start, ev_stop, a);
    return hipGetLastError();
}

hipError_t launch_gateup_mfma(const LayerDesc& L, const Workspace& ws, int T, hipStream_t stream,
                              hipEvent_t ev_start, hipEvent_t ev_stop) {
    F16Args a = base_f16_args(L, ws);
    set_weights(a.w0, a.w0_nb2, a.w0_cs, a.w0_ps, L.pk_gate, L.w_gate, L.gate_nb1, L.gate_nb2, L.gu_type, L.F, L.H);
    set_weights(a.w1, a.w1_nb2, a.w1_cs, a.w1_ps, L.pk_up, L.w_up, L.up_nb1, L.up_nb2, L.gu_type, L.F, L.H);
    uint64_t nb2_unused = 0;
    set_weights(a.sh0, nb2_unused, a.sh0_cs, a.sh0_ps, L.pk_sh_gate, L.w_sh_gate, L.sh_gate_nb1, 0, L.gu_type, L.F, L.H);
    set_weights(a.sh1, nb2_unused, a.sh1_cs, a.sh1_ps, L.pk_sh_up, L.w_sh_up, L.sh_up_nb1, 0, L.gu_type, L.F, L.H);
    a.a_q = ws.x_q; a.a_d = ws.x_d;
    a.K = L.H;
    a.n_y = L.F / 64;
    // the fixup list starts empty: the routing's expert scan clears its counter
    hipError_t err = hipSuccess;
    const dim3 grid(8 * ((f16_max_tiles(L, ws, T) + 7) / 8) * a.n_y);
    const bool gelu = L.act == kActGeluTanh;
    if (L.gu_type == kTypeQ4_0)
        err = gelu ? launch_f16(k_expert_f16<kTypeQ4_0, true, kActGeluTanh>, grid, stream, ev_start, ev_stop, a)
                   : launch_f16(k_expert_f16<kTypeQ4_0, true, kActSilu>, grid, stream, ev_start, ev_stop, a);
    else
        err = gelu ? launch_f16(k_expert_f16<kTypeQ8_0, true, kActGeluTanh>, grid, stream, ev_start, ev_stop, a)
                   : launch_f16(k_expert_f16<kTypeQ8_0, true, kActSilu>, grid, stream, ev_start, ev_stop, a);
    if (err != hipSuccess) return err;
    FixArgs f{};
    f.H = L.H; f.F = L.F; f.E = L.E;
    f.wg = L.w_gate; f.wg_nb1 = L.gate_nb1; f.wg_nb2 = L.gate_nb2;
    f.wu = L.w_up; f.wu_nb1 = L.up_nb1; f.wu_nb2 = L.up_nb2;
    f.sg = L.w_sh_gate; f.sg_nb1 = L.sh_gate_nb1;
    f.su = L.w_sh_up; f.su_nb1 = L.sh_up_nb1;
    f.row_token = ws.row_token;
    f.xq_qs = ws.xq_qs; f.xq_ds = ws.xq_ds;
    f.fix = ws.fix; f.fix_h = ws.fix_h; f.fix_count = ws.counters + kCounterFix; f.fix_max = ws.fix_max;
    f.h_q = ws.h_q; f.h_d = ws.h_d;
    f.act = L.act; f.gelu_tab = L.gelu_tab;
    // one 32-lane half per listed block, enough waves in flight to hide the row reads
    const dim3 fgrid(std::max(1, std::min(8 * L.n_cu, (ws.fix_max + 7) / 8)));
    if (L.gu_type == kTypeQ4_0) hipLaunchKernelGGL(k_fix_h<kTypeQ4_0>, fgrid, dim3(256), 0, stream, f);
    else hipLaunchKernelGGL(k_fix_h<kTypeQ8_0>, fgrid, dim3(256), 0, stream, f);
    return hipGetLastError();
}

hipError_t launch_down_mfma(const LayerDesc& L, const Workspace& ws, int T, hipStream_t stream) {
    F16Args a = base_f16_args(L, ws);
    set_weights(a.w0, a.w0_nb2, a.w0_cs, a.w0_ps, L.pk_down, L.w_down, L.down_nb1, L.down_nb2, L.dn_type, L.H, L.F);
    uint64_t nb2_unused = 0;
    set_weights(a.sh0, nb2_unused, a.sh0_cs, a.sh0_ps, L.pk_sh_down, L.w_sh_down, L.sh_down_nb1, 0, L.dn_type, L.H, L.F);
    a.a_q = ws.h_q; a.a_d = ws.h_d;
    a.K = L.F;
    a.n_y = L.H / 128;
    const dim3 grid(8 * ((f16_max_tiles(L, ws, T) + 7) / 8) * a.n_y);
    return L.dn_type == kTypeQ4_0 ? launch_f16(k_expert_f16<kTypeQ4_0, false, kActSilu>, grid, stream, nullptr, nullptr, a)
                                  : launch_f16(k_expert_f16<kTypeQ8_0, false, kActSilu>, grid, stream, nullptr, nullptr, a);
}

}  // namespace qmoe
