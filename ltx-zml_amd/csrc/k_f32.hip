// f32 reference-precision kernels (mode LTX_MODE_F32): a SIMT tiled GEMM with
// in-register dequant (f32(q) * s, exactly dq4 at ltx/block.zig:462-471) and an
// online-softmax attention on f32 MFMAs. These carry the <= 1e-5 parity mode.
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

// f32 flash attention on v_mfma_f32_16x16x4_f32 (the f32 arithmetic of
// ltx/block.zig:105-154: K scaled by 1/sqrt(128) once, in f32; running max
// and sum per query; out = acc / l, then the gate). A workgroup of 8 waves
// takes 128 queries of one head, 16 per wave; keys go through LDS in tiles
// of 64, the next tile held in registers while the current one is used.
// q/k/v/out are [L][D] f32 (merged heads), glog [L][H].
//
// Operand layouts (lane l; lr = l % 16, lg = l / 16):
// - S^T = K Q^T per 16-key block kb: the A operand is K (key 16 kb + lr),
//   the B operand Q^T (query lr), and in MFMA step s the k index lg stands
//   for head dim 32 lg + s, so a lane's K and Q operands are 32 contiguous
//   dims. The result holds keys 16 kb + 4 lg + r (r = 0..3) of query lr.
// - O^T = V^T P^T per 16-dim block db: step (kb, i) multiplies keys
//   16 kb + 4 g + i (g = 0..3, the k index), so its B operand is register i
//   of kb's S^T result, unmoved. Row m of block db is dim 4 m + db (db < 4)
//   or 64 + 4 m + db - 4, so a lane's V operands are two float4 of one key
//   row and its outputs two runs of 16 dims.
// K rows in LDS are padded to 132 floats: the 16 lanes of a fragment read
// (16 keys, one column) then cover all 64 banks.
extern "C" __global__ void __launch_bounds__(512) ltx_attn_f32(const LtxAttn32Args a) {
    constexpr int KLD = LTX_HD + 4;
    __shared__ __attribute__((aligned(16))) float sK[64 * KLD];
    __shared__ __attribute__((aligned(16))) float sV[64 * LTX_HD];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int h = blockIdx.y;
    const int q0 = blockIdx.x * 128 + 16 * w;
    const size_t hoff = (size_t)h * LTX_HD;
    float qf[32];  // Q^T operand: query q0 + lr, dims 32 lg .. +31
    {
        const float* src = a.q + (size_t)min(q0 + lr, a.lq - 1) * LTX_D + hoff + 32 * lg;
#pragma unroll
        for (int t = 0; t < 8; t++) *(f32x4*)(qf + 4 * t) = *(const f32x4*)(src + 4 * t);
    }
    f32x4 o[8];
#pragma unroll
    for (int db = 0; db < 8; db++) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    // running max of query lr (equal in its four lanes); this lane's part
    // of the row sum (its keys), added over the four lanes at the end
    float m = -3.402823466e38f, lsum = 0.f;
    const int ntile = (a.lkv + 63) / 64;
    // staging: thread tid moves float4 f = tid + 512 j of each 64 x 128 tile
    // (row f / 32, chunk f % 32); rows past lkv repeat row lkv - 1
    f32x4 pk[4], pv[4];
    auto load_tile = [&](int t) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int f = tid + 512 * j, r = f >> 5, c = f & 31;
            const size_t off = (size_t)min(64 * t + r, a.lkv - 1) * LTX_D + hoff + 4 * c;
            pk[j] = *(const f32x4*)(a.k + off);
            pv[j] = *(const f32x4*)(a.v + off);
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int f = tid + 512 * j, r = f >> 5, c = f & 31;
            *(f32x4*)(sK + r * KLD + 4 * c) = pk[j] * a.scale;
            *(f32x4*)(sV + r * LTX_HD + 4 * c) = pv[j];
        }
    };
    load_tile(0);
    store_tile();
    __syncthreads();
    for (int t = 0; t < ntile; t++) {
        if (t + 1 < ntile) load_tile(t + 1);
        f32x4 s[4];
#pragma unroll
        for (int kb = 0; kb < 4; kb++) s[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < 8; u++) {
            f32x4 kf[4];
#pragma unroll
            for (int kb = 0; kb < 4; kb++) kf[kb] = *(const f32x4*)(sK + (16 * kb + lr) * KLD + 32 * lg + 4 * u);
#pragma unroll
            for (int e = 0; e < 4; e++)
#pragma unroll
                for (int kb = 0; kb < 4; kb++)
                    s[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[kb][e], qf[4 * u + e], s[kb], 0, 0, 0);
        }
        float mx = m;
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                if (64 * t + 16 * kb + 4 * lg + r >= a.lkv) s[kb][r] = -__builtin_inff();
                mx = fmaxf(mx, s[kb][r]);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float corr = expf(m - mx);
        m = mx;
        float ps = 0.f;
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float p = expf(s[kb][r] - mx);
                s[kb][r] = p;
                ps += p;
            }
        lsum = lsum * corr + ps;
#pragma unroll
        for (int db = 0; db < 8; db++) o[db] *= corr;
#pragma unroll
        for (int kb = 0; kb < 4; kb++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float* vr = sV + (16 * kb + 4 * lg + i) * LTX_HD + 4 * lr;
                const f32x4 v0 = *(const f32x4*)vr, v1 = *(const f32x4*)(vr + 64);
#pragma unroll
                for (int db = 0; db < 4; db++) {
                    o[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(v0[db], s[kb][i], o[db], 0, 0, 0);
                    o[4 + db] = __builtin_amdgcn_mfma_f32_16x16x4f32(v1[db], s[kb][i], o[4 + db], 0, 0, 0);
                }
            }
        __syncthreads();
        if (t + 1 < ntile) {
            store_tile();
            __syncthreads();
        }
    }
    lsum += __shfl_xor(lsum, 16, 64);
    lsum += __shfl_xor(lsum, 32, 64);
    const int q = q0 + lr;
    if (q >= a.lq) return;
    const float g = a.glog ? 2.0f / (1.0f + expf(-a.glog[(size_t)q * LTX_H + h])) : 1.0f;
    float* dst = a.out + (size_t)q * LTX_D + hoff + 16 * lg;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        *(f32x4*)(dst + 4 * r) = f32x4{o[0][r] / lsum * g, o[1][r] / lsum * g, o[2][r] / lsum * g, o[3][r] / lsum * g};
        *(f32x4*)(dst + 64 + 4 * r) =
            f32x4{o[4][r] / lsum * g, o[5][r] / lsum * g, o[6][r] / lsum * g, o[7][r] / lsum * g};
    }
}
