// f32 reference-precision kernels (mode LTX_MODE_F32): a GEMM that dequantises
// in f32 (f32(q) * s, exactly dq4 at ltx/block.zig:462-471) and an
// online-softmax attention, both on f32 MFMAs. These carry the <= 1e-5 parity
// mode.
#include "ltx_device.h"

// y[M][N] = A[M][K] . W[N][K]^T (+ bias, GELU or the gated residual) in f32
// on v_mfma_f32_16x16x4_f32. Workgroup: 4 waves, output tile 128 x 128, wave
// w owns rows 64 (w / 2) .. +63 and columns 64 (w % 2) .. +63 (4 x 4 blocks
// of 16 x 16). K goes in tiles of 32 through two LDS buffers: each tile's A
// and W rows are loaded into registers while the previous tile is
// multiplied, W dequantised as they are written to LDS (int8: f32(q) * s,
// one f32 rounding, exactly dq4 at ltx/block.zig:462-471; bf16: widened).
// In MFMA step s (0..7) the k index lg = lane / 16 stands for k = 8 lg + s,
// so a lane's A and W operands of a tile are two float4 of one row. Rows are
// padded to 36 floats: the 16 rows of a fragment read cover all 64 banks.
// K must be a multiple of 32. BK is the weight kind (0: int8 + f32 scales,
// 1: int8 + f16 scales, 2: bf16), RG the gated-residual epilogue; both are
// compile-time so that no load in the main loop is conditional.
__shared__ __attribute__((aligned(16))) float g32_sa[2][128 * 36];
__shared__ __attribute__((aligned(16))) float g32_sb[2][128 * 36];

template <int BK, bool RG>
__device__ __forceinline__ void gemm32_body(const LtxGemm32Args& a) {
    constexpr int LD = 36;
    float(&sA)[2][128 * LD] = g32_sa;
    float(&sB)[2][128 * LD] = g32_sb;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int m0 = blockIdx.y * 128, n0 = blockIdx.x * 128;
    const int wm = (w >> 1) * 64, wn = (w & 1) * 64;
    const int G = a.K / LTX_GROUP, ntile = a.K / 32;
    // staging: A float4 f = tid + 256 j (row f / 8, chunk f % 8); W row
    // tid / 2, k 16 (tid % 2) .. +15. Rows past M or N repeat the last one.
    const int wr = tid >> 1, wk = 16 * (tid & 1);
    const int wrow = min(n0 + wr, a.N - 1);
    f32x4 pa[4];
    u32x4 pw[BK == 2 ? 2 : 1];
    uint32_t sraw = 0;  // the tile's scale, bits as stored
    auto load = [&](int kt) {
        const int k0 = 32 * kt;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int f = tid + 256 * j, r = f >> 3, c = f & 7;
            pa[j] = *(const f32x4*)(a.a + (size_t)min(m0 + r, a.M - 1) * a.K + k0 + 4 * c);
        }
        const size_t bi = (size_t)wrow * a.K + k0 + wk;
        if constexpr (BK == 2) {
            pw[0] = *(const u32x4*)((const uint16_t*)a.b + bi);
            pw[1] = *(const u32x4*)((const uint16_t*)a.b + bi + 8);
        } else {
            pw[0] = *(const u32x4*)((const uint8_t*)a.b + bi);
            const size_t si = (size_t)wrow * G + k0 / LTX_GROUP;
            if constexpr (BK == 1)
                sraw = ((const uint16_t*)a.scales)[si];
            else
                sraw = ((const uint32_t*)a.scales)[si];
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int f = tid + 256 * j, r = f >> 3, c = f & 7;
            *(f32x4*)(sA[buf] + r * LD + 4 * c) = pa[j];
        }
        float wv[16];
        if constexpr (BK == 2) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint32_t x = pw[i >> 2][i & 3];
                wv[2 * i] = bf16_bits_to_f32((uint16_t)(x & 0xffffu));
                wv[2 * i + 1] = bf16_bits_to_f32((uint16_t)(x >> 16));
            }
        } else {
            const float sc = BK == 1 ? f16_bits_to_f32((uint16_t)sraw) : __builtin_bit_cast(float, sraw);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const uint32_t byte = (pw[0][i >> 2] >> (8 * (i & 3))) & 0xffu;
                wv[i] = (float)((int)(byte ^ (a.qxor & 0xffu)) - 128) * sc;
            }
        }
        float* d = sB[buf] + wr * LD + wk;
#pragma unroll
        for (int i = 0; i < 4; i++) *(f32x4*)(d + 4 * i) = f32x4{wv[4 * i], wv[4 * i + 1], wv[4 * i + 2], wv[4 * i + 3]};
    };
    f32x4 acc[4][4];
#pragma unroll
    for (int rb = 0; rb < 4; rb++)
#pragma unroll
        for (int cb = 0; cb < 4; cb++) acc[rb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
    load(0);
    store(0);
    __syncthreads();
    for (int kt = 0; kt < ntile; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < ntile) load(kt + 1);
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            f32x4 af[4], bf[4];
#pragma unroll
            for (int rb = 0; rb < 4; rb++) af[rb] = *(const f32x4*)(sA[buf] + (wm + 16 * rb + lr) * LD + 8 * lg + 4 * hh);
#pragma unroll
            for (int cb = 0; cb < 4; cb++) bf[cb] = *(const f32x4*)(sB[buf] + (wn + 16 * cb + lr) * LD + 8 * lg + 4 * hh);
#pragma unroll
            for (int e = 0; e < 4; e++)
#pragma unroll
                for (int rb = 0; rb < 4; rb++)
#pragma unroll
                    for (int cb = 0; cb < 4; cb++)
                        acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[rb][e], bf[cb][e], acc[rb][cb], 0, 0, 0);
        }
        // the other buffer was last read in the previous trip, before its
        // closing barrier
        if (kt + 1 < ntile) store(buf ^ 1);
        __syncthreads();
    }
    // acc[rb][cb][r]: row wm + 16 rb + 4 lg + r, column wn + 16 cb + lr.
    // The residual and gate values of a row block are loaded before its
    // first store (rows and columns past M and N load the last ones).
    int nc[4];
    float bv[4], sv[4];
#pragma unroll
    for (int cb = 0; cb < 4; cb++) {
        nc[cb] = min(n0 + wn + 16 * cb + lr, a.N - 1);
        bv[cb] = a.bias ? a.bias[nc[cb]] : 0.0f;
        if constexpr (RG) sv[cb] = a.ada.sst[(size_t)a.igate * LTX_D + nc[cb]];
    }
    const bool full = m0 + 128 <= a.M && n0 + 128 <= a.N;
    int trow[4][4];  // timestep-table row of each output row
    if constexpr (RG) {
#pragma unroll
        for (int rb = 0; rb < 4; rb++)
#pragma unroll
            for (int r = 0; r < 4; r++) trow[rb][r] = ada_row(a.ada, min(m0 + wm + 16 * rb + 4 * lg + r, a.M - 1));
    }
#pragma unroll
    for (int rb = 0; rb < 4; rb++) {
        float rv[4][4], gv[4][4];
        if constexpr (RG) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int mc = min(m0 + wm + 16 * rb + 4 * lg + r, a.M - 1);
                const float* tr = a.ada.tstab + ((size_t)trow[rb][r] * 9 + a.igate) * LTX_D;
#pragma unroll
                for (int cb = 0; cb < 4; cb++) {
                    rv[r][cb] = a.resid[(size_t)mc * a.N + nc[cb]];
                    gv[r][cb] = tr[nc[cb]] + sv[cb];  // the AdaLN gate value, as ada_val
                }
            }
        }
        float val[4][4];
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int cb = 0; cb < 4; cb++) {
                const float v = acc[rb][cb][r] + bv[cb];
                if constexpr (RG)
                    val[r][cb] = rv[r][cb] + v * gv[r][cb];
                else
                    val[r][cb] = a.gelu ? gelu_tanh(v) : v;
            }
        // whole tiles store without per-element branches (each branch join
        // would otherwise wait for the stores before it)
        float* orow = a.out + (size_t)(m0 + wm + 16 * rb + 4 * lg) * a.N + n0 + wn + lr;
        if (full) {
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int cb = 0; cb < 4; cb++) orow[(size_t)r * a.N + 16 * cb] = val[r][cb];
        } else {
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int cb = 0; cb < 4; cb++)
                    if (m0 + wm + 16 * rb + 4 * lg + r < a.M && n0 + wn + 16 * cb + lr < a.N)
                        orow[(size_t)r * a.N + 16 * cb] = val[r][cb];
        }
    }
}

extern "C" __global__ void __launch_bounds__(256) ltx_gemm_f32(const LtxGemm32Args a) {
    const bool rg = a.epi == LTX_EPI_RESID_GATE;
    if (a.bkind == 0)
        rg ? gemm32_body<0, true>(a) : gemm32_body<0, false>(a);
    else if (a.bkind == 1)
        rg ? gemm32_body<1, true>(a) : gemm32_body<1, false>(a);
    else
        rg ? gemm32_body<2, true>(a) : gemm32_body<2, false>(a);
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
