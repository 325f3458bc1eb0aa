// Tile rasterisation and fused epilogues shared by the 16-bit GEMM kernels.
#pragma once
#include "ltx_device.h"

#define GM 8  // M-tiles per rasterisation group

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
#pragma unroll
    for (int i = 0; i < NI; i++) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = rb + 32 * i + 8 * (r >> 2) + (r & 3);
            if (m >= a.M) continue;
            const float* gt = nullptr;
            const float* gs = nullptr;
            if (EPI == LTX_EPI_RESID_GATE) {  // ada row of the gate: sst[i] + tstab[tidx[m]][i]
                gt = a.ada.tstab + ((size_t)a.ada.tidx[m] * 9 + a.igate) * LTX_D;
                gs = a.ada.sst + (size_t)a.igate * LTX_D;
            }
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const int n = cb + 32 * j;
                float v = acc[i][j][r] + (a.bias ? a.bias[n] : 0.0f);
                if (EPI == LTX_EPI_STORE) {
                    if (a.gelu) v = gelu_tanh(v);
                    if (a.out_f32)
                        ((float*)a.out)[(size_t)m * a.ldo + n] = v;
                    else
                        ((uint16_t*)a.out)[(size_t)m * a.ldo + n] = Op<T>::bits(v);
                } else if (EPI == LTX_EPI_RESID_GATE) {
                    size_t o = (size_t)m * a.ldo + n;
                    ((float*)a.out)[o] = a.resid[o] + v * (gt[n] + gs[n]);
                } else {  // QKV
                    if (n0 < a.nsplit) {
                        ((float*)a.out)[(size_t)m * a.nsplit + n] = v;
                    } else {
                        int c = n - a.nsplit;  // = h * 128 + d
                        ((uint16_t*)a.out2)[(size_t)c * a.M + m] = Op<T>::bits(v);
                    }
                }
            }
        }
    }
}
