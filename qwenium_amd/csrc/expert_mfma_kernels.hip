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
// A block computes 64 rows x 64 output columns of one tile with 4 waves; wave
// (ms, ws) owns rows 32*ms..+32 and two 32-column MFMA tiles:
//   gate/up mode: the gate rows and the up rows of the same 32 ffn indices
//                 f (block columns 32*ws..+32), written to gubuf[p][f] as (g, u);
//   down mode:    64 consecutive W_down rows (block columns 64*ws..+64 of 128).
// The two column tiles share the wave's activation fragment and its per-row
// activation scales.  Activation rows (int8 Q8_0 + f64 scales) are staged in
// LDS (row stride padded to 272 bytes: conflict-free 16-byte fragment reads),
// the next chunk is prefetched through registers while the current one is
// consumed; weights are read per lane straight from GGUF block layout
// (dword-aligned block pairs, one pair ahead) and unpacked in registers.
//
// Block order: logical block g = (tile, y) with y fastest; the blocks of each
// XCD (hardware deals workgroups round-robin over the 8 XCDs) take one
// contiguous range of g, so the tiles of an expert and their column chunks
// share one L2.
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
    int n_y;                                     // column chunks per tile
};

// 16 int8 weights of block `blk` (0 = first of the pair, 1 = second), k-half kh,
// as 4 dwords of int8 operands.  Q4_0 lanes get 16 * (nibble - 8): with
// x = q ^ 0x88888888 (flips bit 3 of every nibble), (x << 4*(1-kh)) & 0xF0F0F0F0
// puts the wanted nibble, as a two's complement value, in each byte's high
// half, so the MFMA sums 16 * isum (the 1/16 is folded into the staged
// activation scales, exactly).  Q8_0 lanes get the quants as stored.
template <int WT>
__device__ __forceinline__ v4i weight_frag(const WPair<WT>& w, int blk, int sh);

template <>
__device__ __forceinline__ v4i weight_frag<kTypeQ4_0>(const WPair<kTypeQ4_0>& w, int blk, int sh) {
    v4i r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t q = blk == 0 ? __builtin_amdgcn_alignbyte(w.w[i + 1], w.w[i], 2) : w.w[5 + i];
        r[i] = (int)(((q ^ 0x88888888u) << sh) & 0xF0F0F0F0u);
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
__global__ __launch_bounds__(256, 2) void k_expert_mfma(MfmaArgs a) {
    __shared__ __align__(16) int8_t s_x[kTileM * kRowStride];
    __shared__ __align__(16) double s_d[(kKC / 32) * kTileM];  // [block][row]
    // XCD-aware logical block (see the file comment); the grid has >= 8 spare blocks
    const int total = a.counters[1] * a.n_y;
    const int share = (total + 7) >> 3;
    const int jb = (int)(blockIdx.x >> 3);
    if (jb >= share) return;
    const int g = (int)(blockIdx.x & 7) * share + jb;
    if (g >= total) return;
    const int tile_id = g / a.n_y, y = g - tile_id * a.n_y;
    const int4 tile = a.tiles[tile_id];
    const int e = tile.x, p0 = tile.y, nr = tile.z;
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int ms = wave & 1, ws = wave >> 1;
    const int col = lane & 31, kh = lane >> 5;
    const bool sh = e >= a.E;

    // weight rows of this lane's two output columns: wave-uniform slab base +
    // 32-bit row offset (an expert's slab is far below 4 GiB)
    const uint8_t* wbase[2];
    uint32_t woff[2];
    int out_idx[2];
    if (GATEUP) {
        const int f = y * 64 + ws * 32 + col;
        wbase[0] = sh ? a.sh0 : a.w0 + (uint64_t)e * a.w0_nb2;
        wbase[1] = sh ? a.sh1 : a.w1 + (uint64_t)e * a.w1_nb2;
        woff[0] = (uint32_t)(f * (sh ? a.sh0_nb1 : a.w0_nb1));
        woff[1] = (uint32_t)(f * (sh ? a.sh1_nb1 : a.w1_nb1));
        out_idx[0] = out_idx[1] = f;
    } else {
        const uint8_t* base = sh ? a.sh0 : a.w0 + (uint64_t)e * a.w0_nb2;
        const uint64_t nb1 = sh ? a.sh0_nb1 : a.w0_nb1;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            out_idx[c] = y * 128 + ws * 64 + c * 32 + col;
            wbase[c] = base;
            woff[c] = (uint32_t)(out_idx[c] * nb1);
        }
    }
    constexpr uint32_t kPairBytes = 2 * BlockTraits<WT>::kBytes;

    // staging assignment: 16-byte chunk (m = tid/16 + 16q, c16 = tid%16), q < 4;
    // scales (m = tid%64, block tid/64 + 4q), q < 2.  The row lookups are
    // issued together, before any of them is used.
    const int nblk_k = a.K >> 5;
    int srow[5];
#pragma unroll
    for (int q = 0; q < 5; ++q) {
        const int m = q < 4 ? (tid >> 4) + 16 * q : (tid & 63);
        const int pr = p0 + min(m, nr - 1);
        srow[q] = GATEUP ? a.row_token[pr] : pr;
    }
    // activation sources as 32-bit offsets from the uniform a_qs / a_ds bases
    // (R*K and R*K/32 stay far below 2^32); rows past the tile read as zero
    uint32_t xoff[4];
    bool xlive[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        xlive[q] = (tid >> 4) + 16 * q < nr;
        xoff[q] = (uint32_t)srow[q] * (uint32_t)a.K + 16u * (tid & 15);
    }
    const bool dlive = (tid & 63) < nr;
    const uint32_t doff = (uint32_t)srow[4] * (uint32_t)nblk_k;
    // Q4_0 fragments carry 16x the weight quants (see weight_frag)
    constexpr double kDxScale = WT == kTypeQ4_0 ? 0.0625 : 1.0;
    u32x4 px[4];
    float pd[2];  // raw f32 scales: converted when stored, so the loads are not waited on early
    auto stage_load = [&](int kc) {
        const int kcn = min(kKC, a.K - kc);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            px[q] = (xlive[q] && 16 * (tid & 15) < kcn) ? *(const u32x4*)(a.a_qs + (xoff[q] + (uint32_t)kc))
                                                        : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int bb = (tid >> 6) + 4 * q;
            pd[q] = (dlive && 32 * bb < kcn) ? a.a_ds[doff + (uint32_t)((kc >> 5) + bb)].x : 0.0f;
        }
    };
    stage_load(0);

    double acc[2][16];
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[c][r] = 0.0;

    const int frag_sel = WT == kTypeQ4_0 ? 4 * (1 - kh) : kh;
    const bool active = 32 * ms < nr;  // wave-uniform: rows 32*ms.. of the tile exist
    const int npairs = a.K >> 6;
    constexpr int kPairsPerChunk = kKC / 64;
    const int8_t* xrow = s_x + (32 * ms + col) * kRowStride + 16 * kh;

    // one pair (two quant blocks) of the wave's two column tiles
    auto pair_step = [&](const WPair<WT> (&w)[2], int pidx) {
        const int bp = 2 * (pidx % kPairsPerChunk);
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
            const int b = bp + sub;
            const v4i af = *(const v4i*)(xrow + 32 * b);
            const v16i z = {};
            const v16i is0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, weight_frag<WT>(w[0], sub, frag_sel), z, 0, 0, 0);
            const v16i is1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, weight_frag<WT>(w[1], sub, frag_sel), z, 0, 0, 0);
            const double* drow = s_d + b * kTileM + 32 * ms + 4 * kh;
            double dx[16];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) dx[4 * i + j] = drow[8 * i + j];
            const double dw0 = (double)(sub == 0 ? w[0].dA() : w[0].dB());
            const double dw1 = (double)(sub == 0 ? w[1].dA() : w[1].dB());
            // fp32(d_w)*fp32(d_x) (times 1/16 for Q4_0) is exact in f64; the block term and the sum are exact
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[0][r] = __builtin_fma(dw0 * dx[r], (double)is0[r], acc[0][r]);
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[1][r] = __builtin_fma(dw1 * dx[r], (double)is1[r], acc[1][r]);
        }
    };
    // chunk boundary: publish the prefetched activation chunk, prefetch the next
    auto stage_chunk = [&](int kc) {
        __syncthreads();  // the previous chunk's LDS reads are done
#pragma unroll
        for (int q = 0; q < 4; ++q) *(u32x4*)(s_x + ((tid >> 4) + 16 * q) * kRowStride + 16 * (tid & 15)) = px[q];
#pragma unroll
        for (int q = 0; q < 2; ++q) s_d[((tid >> 6) + 4 * q) * kTileM + (tid & 63)] = (double)pd[q] * kDxScale;
        __syncthreads();
        if (kc + kKC < a.K) stage_load(kc + kKC);
    };

    // Weight pairs one ahead: wn loads while wc computes.  The next chunk is
    // published at the end of the iteration that finishes the current one.
    WPair<WT> wc[2], wn[2];
    if (active) {
        wc[0].load32(wbase[0], woff[0]);
        wc[1].load32(wbase[1], woff[1]);
    }
    stage_chunk(0);
    for (int pidx = 0; pidx < npairs; ++pidx) {
        if (active) {
            if (pidx + 1 < npairs) {
                wn[0].load32(wbase[0], woff[0] + (pidx + 1) * kPairBytes);
                wn[1].load32(wbase[1], woff[1] + (pidx + 1) * kPairBytes);
            }
            pair_step(wc, pidx);
        }
        if ((pidx + 1) % kPairsPerChunk == 0 && pidx + 1 < npairs) stage_chunk((pidx + 1) * 64);
        wc[0] = wn[0];
        wc[1] = wn[1];
    }
    if (!active) return;
    // output: lane holds column `col` of each MFMA tile, rows 8i + 4kh + j of the wave's 32
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int m = 32 * ms + 8 * i + 4 * kh + j;
            if (m < nr) {
                const int p = p0 + m;
                const int r = 4 * i + j;
                if (GATEUP) {
                    a.gubuf[(uint64_t)p * a.n_out + out_idx[0]] = make_float2((float)acc[0][r], (float)acc[1][r]);
                } else {
                    a.ybuf[(uint64_t)p * a.n_out + out_idx[0]] = (float)acc[0][r];
                    a.ybuf[(uint64_t)p * a.n_out + out_idx[1]] = (float)acc[1][r];
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

static int mfma_max_tiles(const LayerDesc& L, const Workspace& ws, int T) {
    return min(ws.max_tiles, (T * L.K + kTileM - 1) / kTileM + min(L.E, T * L.K) +
                                 (L.S ? (T + kTileM - 1) / kTileM : 0));
}

hipError_t launch_gateup_mfma(const LayerDesc& L, const Workspace& ws, int T, hipStream_t stream,
                              hipEvent_t ev_start, hipEvent_t ev_stop) {
    MfmaArgs a = base_args(L, ws);
    a.w0 = L.w_gate; a.w0_nb1 = L.gate_nb1; a.w0_nb2 = L.gate_nb2;
    a.w1 = L.w_up; a.w1_nb1 = L.up_nb1; a.w1_nb2 = L.up_nb2;
    a.sh0 = L.w_sh_gate; a.sh0_nb1 = L.sh_gate_nb1;
    a.sh1 = L.w_sh_up; a.sh1_nb1 = L.sh_up_nb1;
    a.a_qs = ws.xq_qs; a.a_ds = ws.xq_ds;
    a.K = L.H;
    a.n_out = L.F;
    a.n_y = L.F / 64;
    const dim3 grid(mfma_max_tiles(L, ws, T) * a.n_y + 8);
    if (L.gu_type == kTypeQ4_0)
        launch_timed(k_expert_mfma<kTypeQ4_0, true>, grid, dim3(256), 0, stream, ev_start, ev_stop, a);
    else
        launch_timed(k_expert_mfma<kTypeQ8_0, true>, grid, dim3(256), 0, stream, ev_start, ev_stop, a);
    return hipGetLastError();
}

hipError_t launch_down_mfma(const LayerDesc& L, const Workspace& ws, int T, hipStream_t stream) {
    MfmaArgs a = base_args(L, ws);
    a.w0 = L.w_down; a.w0_nb1 = L.down_nb1; a.w0_nb2 = L.down_nb2;
    a.sh0 = L.w_sh_down; a.sh0_nb1 = L.sh_down_nb1;
    a.a_qs = ws.hq_qs; a.a_ds = ws.hq_ds;
    a.K = L.F;
    a.n_out = L.H;
    a.n_y = L.H / 128;
    const dim3 grid(mfma_max_tiles(L, ws, T) * a.n_y + 8);
    if (L.dn_type == kTypeQ4_0) hipLaunchKernelGGL((k_expert_mfma<kTypeQ4_0, false>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((k_expert_mfma<kTypeQ8_0, false>), grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace qmoe
