// f32 reference-precision kernels (mode LTX_MODE_F32): a SIMT tiled GEMM with
// in-register dequant (f32(q) * s, exactly dq4 at ltx/block.zig:462-471) and a
// SIMT online-softmax attention. These carry the <= 1e-5 parity mode; they
// are correctness paths, not the throughput path.
#include "ltx_device.h"

// 64 x 64 output tile, 256 threads, 4 x 4 outputs per thread, K step 16.
extern "C" __global__ void __launch_bounds__(256) ltx_gemm_f32(const LtxGemm32Args a) {
    __shared__ float sA[16][64 + 1];
    __shared__ float sB[16][64 + 1];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    const int G = a.K / LTX_GROUP;
    float acc[4][4] = {};
    for (int k0 = 0; k0 < a.K; k0 += 16) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int id = tid + 256 * i, r = id >> 4, k = id & 15;
            int m = min(m0 + r, a.M - 1);
            sA[k][r] = a.a[(size_t)m * a.K + k0 + k];
            int n = min(n0 + r, a.N - 1);
            size_t bi = (size_t)n * a.K + k0 + k;
            float bv;
            if (a.bkind == 2) {
                bv = bf16_bits_to_f32(((const uint16_t*)a.b)[bi]);
            } else {
                size_t si = (size_t)n * G + (k0 + k) / LTX_GROUP;
                float s = a.bkind == 1 ? f16_bits_to_f32(((const uint16_t*)a.scales)[si]) : ((const float*)a.scales)[si];
                bv = (float)((int)(((const uint8_t*)a.b)[bi] ^ (a.qxor & 0xffu)) - 128) * s;
            }
            sB[k][r] = bv;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 16; k++) {
            float av[4], bv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) av[i] = sA[k][ty * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; j++) bv[j] = sB[k][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = __builtin_fmaf(av[i], bv[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        int m = m0 + ty * 4 + i;
        if (m >= a.M) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int n = n0 + tx * 4 + j;
            if (n >= a.N) continue;
            float v = acc[i][j] + (a.bias ? a.bias[n] : 0.0f);
            size_t o = (size_t)m * a.N + n;
            if (a.epi == LTX_EPI_RESID_GATE) {
                a.out[o] = a.resid[o] + v * ada_val(a.ada, m, a.igate, n);
            } else {
                a.out[o] = a.gelu ? gelu_tanh(v) : v;
            }
        }
    }
}

// One wave = 64 queries of one head, one query per lane; keys streamed
// through LDS in tiles of 32. q/k/v/out are [L][D] f32 (merged heads).
extern "C" __global__ void __launch_bounds__(64) ltx_attn_f32(const LtxAttn32Args a) {
    __shared__ float sK[32][LTX_HD + 1];
    __shared__ float sV[32][LTX_HD + 1];
    const int h = blockIdx.y, lane = threadIdx.x;
    const int q = blockIdx.x * 64 + lane;
    const int qc = min(q, a.lq - 1);
    float qr[LTX_HD], acc[LTX_HD];
#pragma unroll
    for (int e = 0; e < LTX_HD; e++) {
        qr[e] = a.q[(size_t)qc * LTX_D + h * LTX_HD + e];
        acc[e] = 0.f;
    }
    float m = -3.402823466e38f, l = 0.f;
    for (int kv0 = 0; kv0 < a.lkv; kv0 += 32) {
        for (int i = lane; i < 32 * LTX_HD; i += 64) {
            int r = i / LTX_HD, e = i % LTX_HD;
            int key = min(kv0 + r, a.lkv - 1);
            sK[r][e] = a.k[(size_t)key * LTX_D + h * LTX_HD + e];
            sV[r][e] = a.v[(size_t)key * LTX_D + h * LTX_HD + e];
        }
        __syncthreads();
        const int nk = min(32, a.lkv - kv0);
        float s[32];
        float mx = m;
        for (int j = 0; j < nk; j++) {
            float d = 0.f;
#pragma unroll
            for (int e = 0; e < LTX_HD; e++) d = __builtin_fmaf(qr[e], sK[j][e] * a.scale, d);
            s[j] = d;
            mx = fmaxf(mx, d);
        }
        const float corr = expf(m - mx);
        float ps = 0.f;
#pragma unroll
        for (int e = 0; e < LTX_HD; e++) acc[e] *= corr;
        for (int j = 0; j < nk; j++) {
            float p = expf(s[j] - mx);
            ps += p;
#pragma unroll
            for (int e = 0; e < LTX_HD; e++) acc[e] = __builtin_fmaf(p, sV[j][e], acc[e]);
        }
        l = l * corr + ps;
        m = mx;
        __syncthreads();
    }
    if (q >= a.lq) return;
    const float g = a.glog ? 2.0f / (1.0f + expf(-a.glog[(size_t)q * LTX_H + h])) : 1.0f;
#pragma unroll
    for (int e = 0; e < LTX_HD; e++) a.out[(size_t)q * LTX_D + h * LTX_HD + e] = acc[e] / l * g;
}
