// Tile rasterisation and fused epilogues shared by the 16-bit GEMM kernels.
#pragma once
#include "ltx_device.h"

#define GM 4  // M-tiles per rasterisation group

struct TileIdx {
    int tm, tn;
};

// Hardware places workgroup b on XCD b % 8. Hand each XCD a contiguous run of
// the tile sequence, and walk that sequence in groups of GM M-tiles x all
// N-tiles, so the ~32 workgroups resident on one XCD share A rows and B
// columns in that XCD's L2.
__device__ __forceinline__ TileIdx tile_of(int bid, int tiles_m, int tiles_n) {
    int nt = tiles_m * tiles_n;
    int t = bid;
    if ((nt & 7) == 0) t = (bid & 7) * (nt >> 3) + (bid >> 3);
    int gsz = GM * tiles_n;
    int g = t / gsz, r = t - g * gsz;
    int gm0 = g * GM;
    int gcnt = min(GM, tiles_m - gm0);
    TileIdx ti;
    ti.tm = gm0 + r % gcnt;
    ti.tn = r / gcnt;
    return ti;
}

// Epilogue of one wave's NI x NJ blocks of 32 x 32. acc[i][j][r] holds row
// rb + 32 i + 8 (r / 4) + r % 4 and column cb + 32 j, where rb already
// includes 4 (lane / 32) and cb includes lane % 32. n0 is the workgroup's
// first column (the QKV split point is a multiple of the tile width).
template <typename T, int EPI, int NI, int NJ>
__device__ __forceinline__ void gemm_epilogue(const LtxGemmArgs& a, const f32x16 (&acc)[NI][NJ], int rb, int cb,
                                              int n0) {
    unsigned bad = 0;  // 16-bit stores out of range (range guard)
#pragma unroll
    for (int i = 0; i < NI; i++) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = rb + 32 * i + 8 * (r >> 2) + (r & 3);
            if (m >= a.M) continue;
            const float* gt = nullptr;
            const float* gs = nullptr;
            if (EPI == LTX_EPI_RESID_GATE) {  // ada row of the gate: sst[i] + tstab[tidx[m]][i]
                gt = a.ada.tstab + ((size_t)ada_row(a.ada, m) * 9 + a.igate) * LTX_D;
                gs = a.ada.sst + (size_t)a.igate * LTX_D;
            }
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const int n = cb + 32 * j;
                float v = acc[i][j][r] + (a.bias ? a.bias[n] : 0.0f);
                if (EPI == LTX_EPI_STORE) {
                    if (a.gelu) v = gelu_tanh(v);
                    if (a.out_f32) {
                        ((float*)a.out)[(size_t)m * a.ldo + n] = v;
                    } else {
                        ((uint16_t*)a.out)[(size_t)m * a.ldo + n] = Op<T>::bits(v);
                        bad += out_of_range<T>(v);
                    }
                } else if (EPI == LTX_EPI_RESID_GATE) {
                    size_t o = (size_t)m * a.ldo + n;
                    ((float*)a.out)[o] = a.resid[o] + v * (gt[n] + gs[n]);
                } else {  // QKV
                    if (n0 < a.nsplit) {
                        ((uint16_t*)a.out)[(size_t)m * a.nsplit + n] = Op<T>::bits(v);
                        bad += out_of_range<T>(v);
                    } else {
                        int c = n - a.nsplit;  // = h * 128 + d
                        ((uint16_t*)a.out2)[(size_t)c * a.M + m] = Op<T>::bits(v);
                        bad += out_of_range<T>(v);
                    }
                }
            }
        }
    }
    range_report(a.sat, bad);
}

// LDS-staged epilogue: the same outputs as gemm_epilogue, for one wave's
// (32 NI) x (32 NJ) tile at rows mw.., columns nw... Each 32-row block is
// written to a wave-private LDS patch [32][32 NJ + 8] f32 and read back so
// that every global load and store moves 16 contiguous bytes: f32 rows 4
// columns a lane, 16-bit rows 8 columns a lane, V^T columns 8 rows a lane.
// The patch is only touched by this wave (LDS operations of a wave complete in
// order), so no barrier is needed; the caller guarantees no other wave still
// reads that LDS. The residual rows and the 16-bit and gated-residual outputs
// move with non-temporal loads and stores: each is touched once here, and
// kept out of the way of the A and W tiles in L2 they took o1 and o2 1.2-1.6 %
// faster and the RMSNorm + modulate that reads x_sa 1.6 % faster.
//
// The patch is filled by fill(i, patch, LD) with the wave's accumulators of
// 32-row block i (row r of the block at patch[r * LD + column]), so kernels
// with other MFMA layouts share everything after it; gemm_epilogue_lds below
// is the form for NI x NJ blocks of 32 x 32.
//
// The body is compiled per output form (OUT: 0 16-bit rows, 1 f32 rows, 2
// V^T), GELU and whether every row of the wave's tile is inside M (FULL, and M
// a multiple of 8), and the per-column values (bias, gate shift) are loaded
// once before the blocks. On full tiles the stores are issued in batches
// from registers that nothing reuses before they have gone out: the 16-bit
// outputs of HOLD blocks (the whole wave tile where registers allow) are
// formed first and then stored, the f32 rows block by block. (Stored pass by pass, each patch read reused the
// registers of the store before it, and the wait-insertion pass made the
// read wait for that store to complete: 32 store round trips a tile.) The
// range guard takes each block's largest |value| (v_maximum3, which
// propagates NaN: half an instruction per value) and counts the block's
// values one by one from the patch only when that exceeds the type's range.
template <typename T, int EPI, int NI, int NJ, int OUT, bool GELU, bool FULL, int HOLD, typename Fill>
__device__ __forceinline__ void gemm_epilogue_body(const LtxGemmArgs& a, Fill fill, float* patch, int mw, int nw) {
    constexpr int WN = 32 * NJ, LD = WN + 8;
    const int lane = opaque_tid() & 63;
    const int ldo = EPI == LTX_EPI_QKV ? a.nsplit : a.ldo;  // 16-bit rows: q | k [M][nsplit] or [M][ldo]
    unsigned bad = 0;  // 16-bit stores out of range (range guard)
    // f32 rows (and the gated residual): 4 columns a lane, RPP rows a pass
    constexpr int RLPR = WN / 4, RRPP = 64 / RLPR, RNP = 32 / RRPP;
    // 16-bit rows: 8 columns a lane
    constexpr int HLPR = WN / 8, HRPP = 64 / HLPR, HNP = 32 / HRPP;
    // V^T: 4 lanes cover one column's 32 rows (64 contiguous bytes)
    constexpr int VNP = WN / 16;
    constexpr bool RES = EPI == LTX_EPI_RESID_GATE;
    constexpr int TNP = RES ? RNP : 1;
    constexpr int BNP = OUT == 0 ? HNP : OUT == 2 ? VNP : 1;  // batched 16-bit stores per block
    // per-column values, loaded once for the wave's tile
    f32x4 cb0 = {0, 0, 0, 0}, cb1 = {0, 0, 0, 0}, gs = {0, 0, 0, 0};
    float bn[OUT == 2 ? VNP : 1];
    if (OUT == 0) {
        const int n = nw + 8 * (lane % HLPR);
        if (a.bias) {
            cb0 = *(const f32x4*)(a.bias + n);
            cb1 = *(const f32x4*)(a.bias + n + 4);
        }
    } else if (OUT == 1) {
        const int n = nw + 4 * (lane % RLPR);
        if (a.bias) cb0 = *(const f32x4*)(a.bias + n);
        if (RES) gs = *(const f32x4*)(a.ada.sst + (size_t)a.igate * LTX_D + n);
    } else {
#pragma unroll
        for (int p = 0; p < VNP; p++) bn[p] = a.bias ? a.bias[nw + 16 * p + (lane >> 2)] : 0.0f;
    }
    auto row = [&](int m) { return FULL ? m : min(m, a.M - 1); };
    auto act = [&](float v) { return GELU ? gelu_tanh(v) : v; };
    // gated residual: lane rows r0 + RRPP p of each 32-row block. The
    // timestep rows of block i + 1 are looked up with block i's loads, so
    // that a block's gate-row loads do not wait out a round trip for them.
    int tixn[TNP];
    if (RES)
#pragma unroll
        for (int p = 0; p < TNP; p++) tixn[p] = ada_row(a.ada, row(mw + lane / RLPR + RRPP * p));
    static_assert(NI % HOLD == 0, "HOLD divides the blocks");
    u32x4 ob[HOLD][BNP];  // full tiles: the 16-bit outputs of HOLD blocks, stored together
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int mb = mw + 32 * i;
        // this block's residual rows and gate rows are loaded before
        // anything is stored
        f32x4 rs[TNP], gt[TNP];
        if (RES) {
            const int n = nw + 4 * (lane % RLPR), r0 = lane / RLPR;
#pragma unroll
            for (int p = 0; p < RNP; p++) {
                const int m = row(mb + r0 + RRPP * p);
                rs[p] = __builtin_nontemporal_load((const f32x4*)(a.resid + (size_t)m * a.ldo + n));
                gt[p] = *(const f32x4*)(a.ada.tstab + ((size_t)tixn[p] * 9 + a.igate) * LTX_D + n);
            }
            if (i + 1 < NI)
#pragma unroll
                for (int p = 0; p < RNP; p++) tixn[p] = ada_row(a.ada, row(mb + 32 + r0 + RRPP * p));
        }
        fill(i, patch, LD);
        if (OUT == 2) {
            const int rg = lane & 3;
            float mx = 0.0f;
#pragma unroll
            for (int p = 0; p < VNP; p++) {
                const int cc = 16 * p + (lane >> 2);
                const int c = nw + cc - a.nsplit;
                float v[8];
#pragma unroll
                for (int e = 0; e < 8; e++) v[e] = patch[(8 * rg + e) * LD + cc] + bn[p];
                const int m = mb + 8 * rg;
                const u32x4 pk = {pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3]), pack2<T>(v[4], v[5]),
                                  pack2<T>(v[6], v[7])};
                if (FULL) {
                    ob[i % HOLD][p] = pk;
#pragma unroll
                    for (int e = 0; e < 8; e++) mx = __builtin_elementwise_maximum(mx, __builtin_fabsf(v[e]));
                } else {
                    uint16_t* dst = (uint16_t*)a.out2 + (size_t)c * a.M + m;
#pragma unroll
                    for (int e = 0; e < 8; e++) bad += m + e < a.M ? out_of_range<T>(v[e]) : 0u;
                    if ((a.M & 7) == 0 && m + 8 <= a.M) {
                        __builtin_nontemporal_store(pk, (u32x4*)dst);
                    } else {
#pragma unroll
                        for (int e = 0; e < 8; e++)
                            if (m + e < a.M) dst[e] = Op<T>::bits(v[e]);
                    }
                }
            }
            if (FULL && !(mx <= RangeMax<T>::v))  // rare: count this block's values from the patch
#pragma unroll
                for (int p = 0; p < VNP; p++)
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        bad += out_of_range<T>(patch[(8 * rg + e) * LD + 16 * p + (lane >> 2)] + bn[p]);
        } else if (OUT == 1) {
            const int c4 = 4 * (lane % RLPR), r0 = lane / RLPR;
            const int n = nw + c4;
            // the block's rows formed first, then stored (HOLD > 1: the
            // kernels with registers to spare), or row by row
            constexpr int BO = FULL && HOLD > 1 ? RNP : 1;
            f32x4 o[BO];
#pragma unroll
            for (int p = 0; p < RNP; p++) {
                const int rr = r0 + RRPP * p;
                f32x4 v = *(const f32x4*)(patch + rr * LD + c4) + cb0;
                if (!RES) {
                    if (GELU) v = f32x4{gelu_tanh(v[0]), gelu_tanh(v[1]), gelu_tanh(v[2]), gelu_tanh(v[3])};
                    o[p % BO] = v;
                } else {  // gated residual
                    o[p % BO] = rs[p] + v * (gt[p] + gs);
                }
#pragma unroll
                for (int q = p + 1 - BO; q <= p; q++) {
                    if (BO > 1 && p != RNP - 1) break;
                    const int m = mb + r0 + RRPP * q;
                    if (!FULL && m >= a.M) continue;
                    float* dst = (float*)a.out + (size_t)m * a.ldo + n;
                    if (RES)
                        __builtin_nontemporal_store(o[q % BO], (f32x4*)dst);
                    else
                        *(f32x4*)dst = o[q % BO];
                }
            }
        } else {  // 16-bit rows: 8 columns a lane
            const int c8 = 8 * (lane % HLPR), r0 = lane / HLPR;
            const int n = nw + c8;
            float mx = 0.0f;
#pragma unroll
            for (int p = 0; p < HNP; p++) {
                const int rr = r0 + HRPP * p, m = mb + rr;
                if (!FULL && m >= a.M) continue;
                f32x4 v0 = *(const f32x4*)(patch + rr * LD + c8) + cb0;
                f32x4 v1 = *(const f32x4*)(patch + rr * LD + c8 + 4) + cb1;
                if (GELU) {
                    v0 = f32x4{gelu_tanh(v0[0]), gelu_tanh(v0[1]), gelu_tanh(v0[2]), gelu_tanh(v0[3])};
                    v1 = f32x4{gelu_tanh(v1[0]), gelu_tanh(v1[1]), gelu_tanh(v1[2]), gelu_tanh(v1[3])};
                }
                const u32x4 pk = {pack2<T>(v0[0], v0[1]), pack2<T>(v0[2], v0[3]), pack2<T>(v1[0], v1[1]),
                                  pack2<T>(v1[2], v1[3])};
                if (FULL) {
                    ob[i % HOLD][p] = pk;
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        mx = __builtin_elementwise_maximum(
                            mx, __builtin_elementwise_maximum(__builtin_fabsf(v0[e]), __builtin_fabsf(v1[e])));
                } else {
                    __builtin_nontemporal_store(pk, (u32x4*)((uint16_t*)a.out + (size_t)m * ldo + n));
#pragma unroll
                    for (int e = 0; e < 4; e++) bad += out_of_range<T>(v0[e]) + out_of_range<T>(v1[e]);
                }
            }
            if (FULL && !(mx <= RangeMax<T>::v))  // rare: count this block's values from the patch
#pragma unroll
                for (int p = 0; p < HNP; p++)
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        bad += out_of_range<T>(act(patch[(r0 + HRPP * p) * LD + c8 + e] + (e < 4 ? cb0[e] : cb1[e - 4])));
        }
        if (FULL && OUT != 1 && i % HOLD == HOLD - 1) {
#pragma unroll
            for (int h = 0; h < HOLD; h++) {
                const int bb = mw + 32 * (i + 1 - HOLD + h);
#pragma unroll
                for (int p = 0; p < BNP; p++) {
                    if (OUT == 2) {
                        const int c = nw + 16 * p + (lane >> 2) - a.nsplit;
                        __builtin_nontemporal_store(
                            ob[h][p], (u32x4*)((uint16_t*)a.out2 + (size_t)c * a.M + bb + 8 * (lane & 3)));
                    } else {
                        const int m = bb + lane / HLPR + HRPP * p;
                        __builtin_nontemporal_store(
                            ob[h][p], (u32x4*)((uint16_t*)a.out + (size_t)m * ldo + nw + 8 * (lane % HLPR)));
                    }
                }
            }
        }
    }
    range_report(a.sat, bad);
}

template <typename T, int EPI, int NI, int NJ, int OUT, bool GELU, int HOLD, typename Fill>
__device__ __forceinline__ void gemm_epilogue_rows(const LtxGemmArgs& a, Fill fill, float* patch, int mw, int nw) {
    if (mw + 32 * NI <= a.M && (a.M & 7) == 0)
        gemm_epilogue_body<T, EPI, NI, NJ, OUT, GELU, true, HOLD>(a, fill, patch, mw, nw);
    else
        gemm_epilogue_body<T, EPI, NI, NJ, OUT, GELU, false, 1>(a, fill, patch, mw, nw);
}

// SF: the STORE epilogue's form fixed at compile time (bit 0 GELU, bit 1 f32
// output), or -1 to take a.gelu and a.out_f32 at run time. HOLD: the blocks
// of 16-bit outputs held in registers before they are stored.
template <typename T, int EPI, int NI, int NJ, typename Fill, int SF = -1, int HOLD = 1>
__device__ __forceinline__ void gemm_epilogue_patch(const LtxGemmArgs& a, Fill fill, float* patch, int mw, int nw,
                                                    int n0) {
    if (EPI == LTX_EPI_STORE && SF >= 0) {
        gemm_epilogue_rows<T, EPI, NI, NJ, (SF & 2) ? 1 : 0, (SF & 1) != 0, HOLD>(a, fill, patch, mw, nw);
    } else if (EPI == LTX_EPI_QKV) {
        if (n0 >= a.nsplit)
            gemm_epilogue_rows<T, EPI, NI, NJ, 2, false, HOLD>(a, fill, patch, mw, nw);
        else
            gemm_epilogue_rows<T, EPI, NI, NJ, 0, false, HOLD>(a, fill, patch, mw, nw);
    } else if (EPI == LTX_EPI_RESID_GATE) {
        gemm_epilogue_rows<T, EPI, NI, NJ, 1, false, HOLD>(a, fill, patch, mw, nw);
    } else if (a.out_f32) {
        if (a.gelu)
            gemm_epilogue_rows<T, EPI, NI, NJ, 1, true, HOLD>(a, fill, patch, mw, nw);
        else
            gemm_epilogue_rows<T, EPI, NI, NJ, 1, false, HOLD>(a, fill, patch, mw, nw);
    } else {
        if (a.gelu)
            gemm_epilogue_rows<T, EPI, NI, NJ, 0, true, HOLD>(a, fill, patch, mw, nw);
        else
            gemm_epilogue_rows<T, EPI, NI, NJ, 0, false, HOLD>(a, fill, patch, mw, nw);
    }
}

template <typename T, int EPI, int NI, int NJ>
__device__ __forceinline__ void gemm_epilogue_lds(const LtxGemmArgs& a, const f32x16 (&acc)[NI][NJ], float* patch,
                                                  int mw, int nw, int n0) {
    const int lane = opaque_tid() & 63;
    gemm_epilogue_patch<T, EPI, NI, NJ>(
        a,
        [&](int i, float* p, int LD) {
#pragma unroll
            for (int j = 0; j < NJ; j++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    p[(8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * LD + 32 * j + (lane & 31)] = acc[i][j][r];
        },
        patch, mw, nw, n0);
}

// Split-K partial sums: one wave's (32 NI) x (32 NJ) f32 accumulators to
// part[m][n] (row stride N), through the same wave-private LDS patch as the
// epilogues so that every store is 16 contiguous bytes of a row.
template <int NI, int NJ>
__device__ __forceinline__ void gemm_store_partial(const f32x16 (&acc)[NI][NJ], float* patch, float* part, int M,
                                                   int N, int mw, int nw) {
    constexpr int WN = 32 * NJ, LD = WN + 8;
    constexpr int LPR = WN / 4, RPP = 64 / LPR;  // lanes per row, rows per pass
    const int lane = threadIdx.x & 63;
    const int c4 = 4 * (lane % LPR), r0 = lane / LPR;
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int mb = mw + 32 * i;
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int r = 0; r < 16; r++)
                patch[(8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * LD + 32 * j + (lane & 31)] = acc[i][j][r];
#pragma unroll
        for (int p = 0; p < 32 / RPP; p++) {
            const int rr = r0 + RPP * p, m = mb + rr;
            if (m < M) *(f32x4*)(part + (size_t)m * N + nw + c4) = *(const f32x4*)(patch + rr * LD + c4);
        }
    }
}
