// expert_mfma_kernels.hip -- grouped expert GEMMs for large token counts
// (prefill) on int8 MFMA (v_mfma_i32_32x32x32_i8, gfx950).
//
// Semantics as the decode kernels (src/layers/moe.cpp:105-127 mul_mat_id with
// Q8_0 activations): per 32-value quant block the MFMA produces the exact
// integer dot of a 32x32 (rows x outputs) tile; the block term
// fp32(d_w)*fp32(d_x) * isum is then accumulated in f64, exactly, so results
// equal the GEMV path and the CPU restatement bit for bit.
//
// Tiles come from the routing kernels: tiles[i] = {expert, first row, rows <= 64}.
// Block = 4 waves: wave (ms, ns) owns the 32x32 sub-tile of rows
// 32*ms..+32 of the row tile and outputs ns*32..+32 of the block's 64 outputs.
//   gate/up mode: ns = 0 -> 32 gate rows, ns = 1 -> the same 32 up rows;
//                 results go to gubuf[p][f] as (g, u).
//   down mode:    64 consecutive W_down rows; results go to ybuf[p][n].
// Activation rows (int8 Q8_0 + f64 scales) are staged in LDS (row stride padded
// to 272 bytes: conflict-free 16-byte fragment reads); weights are read per
// lane straight from GGUF block layout (dword-aligned block pairs) and
// unpacked to int8 in registers.
#include "qmoe_device.h"
#include "qmoe_internal.h"

#include <algorithm>

namespace qmoe {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kTileM = kMfmaTileM;  // 64 rows per tile
constexpr int kKC = 256;            // k values staged per LDS round (8 quant blocks)
constexpr int kRowStride = kKC + 16;

struct MfmaArgs {
    int H, F, E;
    const uint8_t* w0; uint64_t w0_nb1, w0_nb2;  // gate (gate/up mode) or down
    const uint8_t* w1; uint64_t w1_nb1, w1_nb2;  // up (gate/up mode)
    const uint8_t* sh0; uint64_t sh0_nb1;        // shared gate or shared down
    const uint8_t* sh1; uint64_t sh1_nb1;        // shared up
    const int32_t* counters;                     // [1] n_tiles
    const int4* tiles;
    const int32_t* row_token;                    // A-row indirection (gate/up)
    const int8_t* a_qs; const float2* a_ds;      // A rows: [.][K] int8, [.][K/32] {d, sum}
    int K;                                       // reduction length (H or F)
    float2* gubuf;                               // gate/up output [R][F]
    float* ybuf;                                 // down output [R][H]
    int n_out;                                   // outputs per row (F or H)
};

// 16 int8 weights of block `blk` (0 = first of the pair, 1 = second), k-half kh,
// as signed int8 in 4 dwords.
template <int WT>
__device__ __forceinline__ v4i weight_frag(const WPair<WT>& w, int blk, int kh);

template <>
__device__ __forceinline__ v4i weight_frag<kTypeQ4_0>(const WPair<kTypeQ4_0>& w, int blk, int kh) {
    v4i r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t q = blk == 0 ? __builtin_amdgcn_alignbyte(w.w[i + 1], w.w[i], 2) : w.w[5 + i];
        const uint32_t nib = kh == 0 ? (q & 0x0f0f0f0fu) : ((q >> 4) & 0x0f0f0f0fu);
        // nibble v in [0,15] -> v - 8 as int8, per byte, no inter-byte carry
        r[i] = (int)((nib + 0x78787878u) ^ 0x80808080u);
    }
    return r;
}

template <>
__device__ __forceinline__ v4i weight_frag<kTypeQ8_0>(const WPair<kTypeQ8_0>& w, int blk, int kh) {
    v4i r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // dword i (kh = 0) or 4 + i (kh = 1) of the block's 8 quant dwords; static register indices
        const uint32_t lo = blk == 0 ? __builtin_amdgcn_alignbyte(w.w[i + 1], w.w[i], 2) : w.w[9 + i];
        const uint32_t hi = blk == 0 ? __builtin_amdgcn_alignbyte(w.w[i + 5], w.w[i + 4], 2) : w.w[13 + i];
        r[i] = (int)(kh == 0 ? lo : hi);
    }
    return r;
}

template <int WT, bool GATEUP>
__global__ __launch_bounds__(256) void k_expert_mfma(MfmaArgs a) {
    __shared__ __align__(16) int8_t s_x[kTileM * kRowStride];
    __shared__ __align__(16) double s_d[(kKC / 32) * kTileM];  // [block][row]
    const int tile_id = blockIdx.x;
    if (tile_id >= a.counters[1]) return;
    const int4 tile = a.tiles[tile_id];
    const int e = tile.x, p0 = tile.y, nr = tile.z;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int ms = wave & 1, ns = wave >> 1;
    const int col = lane & 31, kh = lane >> 5;
    const int out0 = blockIdx.y * 64;

    // weight row of this lane's output column
    const uint8_t* wrow;
    int out_idx;
    if (GATEUP) {
        const bool sh = e >= a.E;
        const uint8_t* base = ns == 0 ? (sh ? a.sh0 : a.w0 + (uint64_t)e * a.w0_nb2)
                                      : (sh ? a.sh1 : a.w1 + (uint64_t)e * a.w1_nb2);
        const uint64_t nb1 = ns == 0 ? (sh ? a.sh0_nb1 : a.w0_nb1) : (sh ? a.sh1_nb1 : a.w1_nb1);
        out_idx = blockIdx.y * 32 + col;  // ffn index f
        wrow = base + (uint64_t)out_idx * nb1;
    } else {
        const bool sh = e >= a.E;
        const uint8_t* base = sh ? a.sh0 : a.w0 + (uint64_t)e * a.w0_nb2;
        const uint64_t nb1 = sh ? a.sh0_nb1 : a.w0_nb1;
        out_idx = out0 + ns * 32 + col;  // output row n
        wrow = base + (uint64_t)out_idx * nb1;
    }

    double acc[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0;

    const int nblk_k = a.K >> 5;
    for (int kc = 0; kc < a.K; kc += kKC) {
        const int kcn = min(kKC, a.K - kc);  // multiple of 64
        __syncthreads();
        // stage A rows: kTileM rows x kcn bytes (16-byte chunks) + per-block scales
        const int chunks = kcn / 16;
        for (int i = threadIdx.x; i < kTileM * chunks; i += 256) {
            const int m = i / chunks, c = i % chunks;
            u32x4 v = u32x4{0u, 0u, 0u, 0u};
            if (m < nr) {
                const int p = p0 + m;
                const int arow = GATEUP ? a.row_token[p] : p;
                v = *(const u32x4*)(a.a_qs + (uint64_t)arow * a.K + kc + 16 * c);
            }
            *(u32x4*)(s_x + m * kRowStride + 16 * c) = v;
        }
        const int nbk = kcn / 32;
        for (int i = threadIdx.x; i < kTileM * nbk; i += 256) {
            const int m = i % kTileM, b = i / kTileM;
            double d = 0.0;
            if (m < nr) {
                const int p = p0 + m;
                const int arow = GATEUP ? a.row_token[p] : p;
                d = (double)a.a_ds[(uint64_t)arow * nblk_k + (kc >> 5) + b].x;
            }
            s_d[b * kTileM + m] = d;
        }
        __syncthreads();
        const int8_t* xrow = s_x + (32 * ms + col) * kRowStride + 16 * kh;
        for (int bp = 0; bp < nbk; bp += 2) {
            WPair<WT> w;
            w.load(wrow, ((kc >> 5) + bp) >> 1);
#pragma unroll
            for (int sub = 0; sub < 2; ++sub) {
                const int b = bp + sub;
                const v4i bf = weight_frag<WT>(w, sub, kh);
                const v4i af = *(const v4i*)(xrow + 32 * b);
                const v16i z = {};
                const v16i isum = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bf, z, 0, 0, 0);
                const double dw = (double)(sub == 0 ? w.dA() : w.dB());
                const double* drow = s_d + b * kTileM + 32 * ms + 4 * kh;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int r = 4 * i + j;
                        // fp32(d_w)*fp32(d_x) is exact in f32 and in f64
                        acc[r] = __builtin_fma(dw * drow[8 * i + j], (double)isum[r], acc[r]);
                    }
                }
            }
        }
    }
    // output tile: lane holds column `col`, rows 8i + 4kh + j of the sub-tile
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int m = 32 * ms + 8 * i + 4 * kh + j;
            if (m < nr) {
                const int p = p0 + m;
                const float v = (float)acc[4 * i + j];
                if (GATEUP) {
                    float* dst = (float*)(a.gubuf + (uint64_t)p * a.n_out + out_idx);
                    dst[ns] = v;
                } else {
                    a.ybuf[(uint64_t)p * a.n_out + out_idx] = v;
                }
            }
        }
    }
}

static MfmaArgs base_args(const LayerDesc& L, const Workspace& ws) {
    MfmaArgs a{};
    a.H = L.H; a.F = L.F; a.E = L.E;
    a.counters = ws.counters;
    a.tiles = ws.tiles;
    a.row_token = ws.row_token;
    a.gubuf = ws.gubuf;
    a.ybuf = ws.ybuf;
    return a;
}

hipError_t launch_gateup_mfma(const LayerDesc& L, const Workspace& ws, int T, hipStream_t stream) {
    MfmaArgs a = base_args(L, ws);
    a.w0 = L.w_gate; a.w0_nb1 = L.gate_nb1; a.w0_nb2 = L.gate_nb2;
    a.w1 = L.w_up; a.w1_nb1 = L.up_nb1; a.w1_nb2 = L.up_nb2;
    a.sh0 = L.w_sh_gate; a.sh0_nb1 = L.sh_gate_nb1;
    a.sh1 = L.w_sh_up; a.sh1_nb1 = L.sh_up_nb1;
    a.a_qs = ws.xq_qs; a.a_ds = ws.xq_ds;
    a.K = L.H;
    a.n_out = L.F;
    const int max_tiles = min(ws.max_tiles, (T * L.K + kTileM - 1) / kTileM + min(L.E, T * L.K) +
                                                (L.S ? (T + kTileM - 1) / kTileM : 0));
    const dim3 grid(max_tiles, L.F / 32);
    if (L.gu_type == kTypeQ4_0) hipLaunchKernelGGL((k_expert_mfma<kTypeQ4_0, true>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((k_expert_mfma<kTypeQ8_0, true>), grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_down_mfma(const LayerDesc& L, const Workspace& ws, int T, hipStream_t stream) {
    MfmaArgs a = base_args(L, ws);
    a.w0 = L.w_down; a.w0_nb1 = L.down_nb1; a.w0_nb2 = L.down_nb2;
    a.sh0 = L.w_sh_down; a.sh0_nb1 = L.sh_down_nb1;
    a.a_qs = ws.hq_qs; a.a_ds = ws.hq_ds;
    a.K = L.F;
    a.n_out = L.H;
    const int max_tiles = min(ws.max_tiles, (T * L.K + kTileM - 1) / kTileM + min(L.E, T * L.K) +
                                                (L.S ? (T + kTileM - 1) / kTileM : 0));
    const dim3 grid(max_tiles, L.H / 64);
    if (L.dn_type == kTypeQ4_0) hipLaunchKernelGGL((k_expert_mfma<kTypeQ4_0, false>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((k_expert_mfma<kTypeQ8_0, false>), grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace qmoe
