// Blockwise online-softmax attention for gfx950 (the production attention of
// ltx/block.zig:105-154, whileSdpaC), fused with the per-(token, head) gate
// 2*sigmoid(glog) and the head merge (ltx/block.zig:237-242).
//
// Workgroup = 4 waves = 256 queries of one head; each wave owns 64 queries
// (two 32-query column blocks). K and V^T are streamed through LDS in tiles
// of 64 keys, double-buffered (global -> registers -> LDS, one barrier per
// tile). Scores are computed TRANSPOSED, S^T = K . Q^T, and the output as
// O^T = V^T . P^T, with v_mfma_f32_32x32x16: the query is then the MFMA column
// index, so lane l always holds query l % 32 — its running max m, partial sum
// l and its O^T column stay lane-local, and only the tile max needs one
// exchange with lane l ^ 32. The P^T operand comes straight from the S^T
// accumulators (no LDS round trip): within every 16-key chunk the keys are
// consumed in the order 0-3, 8-11, 4-7, 12-15, which is exactly the order the
// accumulator layout hands them to each lane, and the V^T tile is stored in
// LDS permuted the same way.
//
// Statistics are f32. Softmax uses exp2 with the 1/sqrt(128) scale folded
// into the exponent (s * C - m * C, C = scale * log2 e); m starts at -FLT_MAX
// as in the reference, and keys past lkv are masked to -inf.
#include "ltx_device.h"

#define QT 256         // queries per workgroup
#define KT 64          // keys per tile
#define KROW (128 + 8) // padded K row (16-bit elements)
#define VROW (KT + 8)  // padded V^T row

// QB = 32-query column blocks per wave: 2 -> 4 waves of 64 queries (one wave
// per SIMD), 1 -> 8 waves of 32 queries (two waves per SIMD, so one wave's
// softmax VALU work overlaps the other's MFMAs).
template <typename T, int QB>
__device__ void attn_body(const LtxAttnArgs& a) {
    typedef typename Op<T>::v8 v8;
    constexpr int NT = 256 * (2 / QB);  // threads per workgroup
    constexpr int QW = 32 * QB;         // queries per wave
    __shared__ __attribute__((aligned(16))) uint16_t sK[2][KT * KROW];
    __shared__ __attribute__((aligned(16))) uint16_t sV[2][LTX_HD * VROW];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int nblk = a.q_tiles * LTX_H;
    int t = blockIdx.x;
    if ((nblk & 7) == 0) t = (t & 7) * (nblk >> 3) + (t >> 3);  // one XCD per run of tiles (same head)
    const int h = t / a.q_tiles, qt = t - h * a.q_tiles;
    const int q0 = qt * QT + w * QW;
    const int lq = a.lq, lkv = a.lkv;

    const uint16_t* Q = (const uint16_t*)a.q + (size_t)h * lq * LTX_HD;
    const uint16_t* K = (const uint16_t*)a.k + (size_t)h * lkv * LTX_HD;
    const uint16_t* V = (const uint16_t*)a.vt + (size_t)h * LTX_HD * lkv;

    // Q^T operand: lane holds Q[q][16 c + 8 (lane / 32) .. + 8] for its query.
    const int fr = lane & 31, hi = lane >> 5;
    v8 qf[QB][8];
#pragma unroll
    for (int qb = 0; qb < QB; qb++) {
        const int q = min(q0 + 32 * qb + fr, lq - 1);
#pragma unroll
        for (int c = 0; c < 8; c++) qf[qb][c] = __builtin_bit_cast(v8, *(const u32x4*)(Q + (size_t)q * LTX_HD + 16 * c + 8 * hi));
    }

    f32x16 o[QB][4];
#pragma unroll
    for (int qb = 0; qb < QB; qb++)
#pragma unroll
        for (int db = 0; db < 4; db++) o[qb][db] = f32x16{0};
    float m[QB], l[QB];
#pragma unroll
    for (int qb = 0; qb < QB; qb++) {
        m[qb] = -3.402823466e38f;
        l[qb] = 0.f;
    }
    const float C = a.scale_log2;

    // Global -> register staging of one K tile (64 x 128) and one V^T tile
    // (128 x 64): 1024 + 1024 chunks of 16 B per workgroup.
    constexpr int NCH = 1024 / NT;
    u32x4 rk[NCH], rv[NCH];
    auto gload = [&](int kv0) {
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            int id = tid + NT * i, row = id >> 4, c16 = id & 15;
            int key = min(kv0 + row, lkv - 1);
            rk[i] = *(const u32x4*)(K + (size_t)key * LTX_HD + 8 * c16);
        }
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            int id = tid + NT * i, d = id >> 3, kc = id & 7;
            int key = kv0 + 8 * kc;
            const uint16_t* src = V + (size_t)d * lkv + key;
            if (key + 8 <= lkv && (lkv & 7) == 0) {  // 16-byte aligned row chunk
                rv[i] = *(const u32x4*)src;
            } else {  // ragged tail / unaligned rows: element loads, zero-fill (0 * p stays finite)
                uint16_t e[8];
#pragma unroll
                for (int j = 0; j < 8; j++) e[j] = key + j < lkv ? src[j] : (uint16_t)0;
                rv[i] = u32x4{e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16),
                              e[4] | ((uint32_t)e[5] << 16), e[6] | ((uint32_t)e[7] << 16)};
            }
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            int id = tid + NT * i, row = id >> 4, c16 = id & 15;
            *(u32x4*)(sK[buf] + row * KROW + 8 * c16) = rk[i];
        }
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            int id = tid + NT * i, d = id >> 3, kc = id & 7;
            int base = 16 * (kc >> 1), odd = kc & 1;
            uint16_t* row = sV[buf] + d * VROW + base;
            *(u32x2*)(row + (odd ? 4 : 0)) = u32x2{rv[i][0], rv[i][1]};   // keys 0-3 / 8-11
            *(u32x2*)(row + (odd ? 12 : 8)) = u32x2{rv[i][2], rv[i][3]};  // keys 4-7 / 12-15
        }
    };

    const int ntiles = (lkv + KT - 1) / KT;
    gload(0);
    sstore(0);
    __syncthreads();

    for (int tix = 0; tix < ntiles; tix++) {
        const int buf = tix & 1, kv0 = tix * KT;
        if (tix + 1 < ntiles) gload(kv0 + KT);

        // S^T blocks: s[kb][qb] = K[32 kb .. +32] . Q^T[qb]
        f32x16 s[2][QB];
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
            for (int qb = 0; qb < QB; qb++) s[kb][qb] = f32x16{0};
        const uint16_t* pk = sK[buf] + fr * KROW + 8 * hi;
#pragma unroll
        for (int c = 0; c < 8; c++) {
#pragma unroll
            for (int kb = 0; kb < 2; kb++) {
                v8 kf = __builtin_bit_cast(v8, *(const u32x4*)(pk + 32 * kb * KROW + 16 * c));
#pragma unroll
                for (int qb = 0; qb < QB; qb++) s[kb][qb] = Op<T>::mfma32(kf, qf[qb][c], s[kb][qb]);
            }
        }

        // Online softmax per query column (lane-local), P^T operands.
        v8 pf[QB][4];
#pragma unroll
        for (int qb = 0; qb < QB; qb++) {
            if (kv0 + KT > lkv) {
#pragma unroll
                for (int kb = 0; kb < 2; kb++)
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        int key = kv0 + 32 * kb + 8 * (r >> 2) + 4 * hi + (r & 3);
                        if (key >= lkv) s[kb][qb][r] = -__builtin_inff();
                    }
            }
            float mx = s[0][qb][0];
#pragma unroll
            for (int r = 1; r < 16; r++) mx = fmaxf(mx, s[0][qb][r]);
#pragma unroll
            for (int r = 0; r < 16; r++) mx = fmaxf(mx, s[1][qb][r]);
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float mn = fmaxf(m[qb], mx);
            const float corr = __builtin_amdgcn_exp2f((m[qb] - mn) * C);
            const float mc = mn * C;
            m[qb] = mn;
            float ps = 0.f;
#pragma unroll
            for (int kb = 0; kb < 2; kb++) {
#pragma unroll
                for (int half = 0; half < 2; half++) {
                    float p[8];
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][qb][8 * half + e], C, -mc));
                        ps += p[e];
                    }
                    u32x4 pk4 = {pack2<T>(p[0], p[1]), pack2<T>(p[2], p[3]), pack2<T>(p[4], p[5]), pack2<T>(p[6], p[7])};
                    pf[qb][2 * kb + half] = __builtin_bit_cast(v8, pk4);
                }
            }
            l[qb] = l[qb] * corr + ps;
#pragma unroll
            for (int db = 0; db < 4; db++) o[qb][db] *= corr;
        }

        // O^T[db][qb] += V^T[32 db .. +32][chunk] . P^T[chunk][qb]
        const uint16_t* pv = sV[buf] + fr * VROW + 8 * hi;
#pragma unroll
        for (int kc = 0; kc < 4; kc++) {
#pragma unroll
            for (int db = 0; db < 4; db++) {
                v8 vf = __builtin_bit_cast(v8, *(const u32x4*)(pv + 32 * db * VROW + 16 * kc));
#pragma unroll
                for (int qb = 0; qb < QB; qb++) o[qb][db] = Op<T>::mfma32(vf, pf[qb][kc], o[qb][db]);
            }
        }

        if (tix + 1 < ntiles) sstore(buf ^ 1);
        __syncthreads();
    }

    // out[q][h * 128 + d] = O^T[d][q] / l * 2 sigmoid(glog[q][h])
    uint16_t* out = (uint16_t*)a.out;
#pragma unroll
    for (int qb = 0; qb < QB; qb++) {
        const float lt = l[qb] + __shfl_xor(l[qb], 32, 64);
        const int q = q0 + 32 * qb + fr;
        if (q >= lq) continue;
        const float g = a.glog ? 2.0f * sigmoid_f(a.glog[(size_t)q * LTX_H + h]) : 1.0f;
        const float sc = g / lt;
#pragma unroll
        for (int db = 0; db < 4; db++) {
#pragma unroll
            for (int rg = 0; rg < 4; rg++) {
                int d = 32 * db + 8 * rg + 4 * hi;
                u32x2 pk2 = {pack2<T>(o[qb][db][4 * rg] * sc, o[qb][db][4 * rg + 1] * sc),
                             pack2<T>(o[qb][db][4 * rg + 2] * sc, o[qb][db][4 * rg + 3] * sc)};
                *(u32x2*)(out + (size_t)q * LTX_D + h * LTX_HD + d) = pk2;
            }
        }
    }
}

extern "C" __global__ void __launch_bounds__(256, 1) ltx_attn_f16(const LtxAttnArgs a) { attn_body<_Float16, 2>(a); }
extern "C" __global__ void __launch_bounds__(256, 1) ltx_attn_bf16(const LtxAttnArgs a) { attn_body<__bf16, 2>(a); }
extern "C" __global__ void __launch_bounds__(512, 1) ltx_attn_f16_w8(const LtxAttnArgs a) { attn_body<_Float16, 1>(a); }
extern "C" __global__ void __launch_bounds__(512, 1) ltx_attn_bf16_w8(const LtxAttnArgs a) { attn_body<__bf16, 1>(a); }
