// Blockwise online-softmax attention for gfx950 (the production attention of
// ltx/block.zig:105-154, whileSdpaC), fused with the per-(token, head) gate
// 2*sigmoid(glog) and the head merge (ltx/block.zig:237-242).
//
// A workgroup owns QT queries of one head; each wave owns QW = 32 * QB of
// them. K and V^T are streamed through LDS in tiles of 64 keys (global ->
// registers -> LDS, one barrier per tile). Scores are computed TRANSPOSED,
// S^T = K . Q^T, and the output as O^T = V^T . P^T, with v_mfma_f32_32x32x16:
// the query is then the MFMA column index, so lane l always holds query
// l % 32 — its running max m, partial sum l and its O^T column stay
// lane-local, and only the tile max needs one exchange with lane l ^ 32.
// The P^T operand comes straight from the S^T accumulators (no LDS round
// trip): within every 16-key chunk the keys are consumed in the order 0-3,
// 8-11, 4-7, 12-15, which is the order the accumulator layout hands them to
// each lane, and the V^T tile is stored in LDS permuted the same way.
//
// Eight-wave variant (two waves per SIMD) runs the two halves of the
// workgroup half a tile apart: waves 0-3 do S(j), softmax(j), PV(j) while
// waves 4-7 do softmax(j-1), PV(j-1), S(j). Within one barrier interval one
// half issues MFMAs while the other half runs the softmax VALU work, instead
// of both contending for the same unit at the same time. This needs the V
// tile of j-1 alive during iteration j: K/V use three LDS buffers.
//
// Statistics are f32. Softmax uses exp2 with the 1/sqrt(128) scale folded
// into the exponent (s * C - m * C, C = scale * log2 e); m starts at -FLT_MAX
// as in the reference, and keys past lkv are masked to -inf. The running max
// moves only when a query's tile max exceeds it by more than 2^8 in p; the
// stale max is otherwise kept for numerator and denominator alike.
#include "ltx_device.h"

#define KT 64              // keys per tile
#define KROW (128 + 8)     // padded K row (16-bit elements)
#define VROW (KT + 8)      // padded V^T row
#define RESCALE_LOG2 8.0f  // rescale threshold, in log2 units of p

// QB: 32-query column blocks per wave. NW: waves per workgroup. FULL: lkv is
// a multiple of 64 (no tail handling, no masking). PS: phase-shifted halves.
template <typename T, int QB, bool FULL, int NW, bool PS>
__device__ void attn_body(const LtxAttnArgs& a) {
    typedef typename Op<T>::v8 v8;
    constexpr int NT = 64 * NW;         // threads per workgroup
    constexpr int QT = NW * 32 * QB;    // queries per workgroup
    constexpr int QW = 32 * QB;         // queries per wave
    constexpr int NBUF = PS ? 3 : 2;    // LDS tile buffers
    __shared__ __attribute__((aligned(16))) uint16_t sK[NBUF][KT * KROW];
    __shared__ __attribute__((aligned(16))) uint16_t sV[NBUF][LTX_HD * VROW];

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
        for (int c = 0; c < 8; c++)
            qf[qb][c] = __builtin_bit_cast(v8, *(const u32x4*)(Q + (size_t)q * LTX_HD + 16 * c + 8 * hi));
    }

    f32x16 o[QB][4];
    float m[QB], l[QB];
#pragma unroll
    for (int qb = 0; qb < QB; qb++) {
#pragma unroll
        for (int db = 0; db < 4; db++) o[qb][db] = f32x16{0};
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
            int key = FULL ? kv0 + row : min(kv0 + row, lkv - 1);
            rk[i] = *(const u32x4*)(K + (size_t)key * LTX_HD + 8 * c16);
        }
#pragma unroll
        for (int i = 0; i < NCH; i++) {
            int id = tid + NT * i, d = id >> 3, kc = id & 7;
            int key = kv0 + 8 * kc;
            const uint16_t* src = V + (size_t)d * lkv + key;
            if (FULL || (key + 8 <= lkv && (lkv & 7) == 0)) {  // 16-byte aligned row chunk
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

    // S^T blocks of one tile: s[kb][qb] = K[32 kb .. +32] . Q^T[qb]
    typedef f32x16 STile[2][QB];
    auto scores = [&](const int buf, STile& s) {
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
    };

    // Online softmax of one tile (lane-local per query) -> P^T operands.
    typedef v8 PTile[QB][4];
    auto softmax = [&](STile& s, PTile& pf, const int kv0, const bool last) {
#pragma unroll
        for (int qb = 0; qb < QB; qb++) {
            if (!FULL && last && kv0 + KT > lkv) {
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
            if (__builtin_amdgcn_ballot_w64(mx > m[qb] + RESCALE_LOG2 / C) != 0) {
                const float mn = fmaxf(m[qb], mx);
                const float corr = __builtin_amdgcn_exp2f((m[qb] - mn) * C);
                m[qb] = mn;
                l[qb] *= corr;
#pragma unroll
                for (int db = 0; db < 4; db++) o[qb][db] *= corr;
            }
            const float mc = m[qb] * C;
            float ps = 0.f;
#pragma unroll
            for (int kb = 0; kb < 2; kb++) {
#pragma unroll
                for (int half = 0; half < 2; half++) {
                    float p[8];
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][qb][8 * half + e], C, -mc));
                    // pack to the 16-bit operand and sum exactly those rounded
                    // weights into l, so O and l use identical P
                    u32x4 pk4 = {Op<T>::cvt2(p[0], p[1]), Op<T>::cvt2(p[2], p[3]), Op<T>::cvt2(p[4], p[5]),
                                 Op<T>::cvt2(p[6], p[7])};
#pragma unroll
                    for (int e = 0; e < 4; e++) ps = Op<T>::sum2(pk4[e], ps);
                    pf[qb][2 * kb + half] = __builtin_bit_cast(v8, pk4);
                }
            }
            l[qb] += ps;
        }
    };

    // O^T[db][qb] += V^T[32 db .. +32][chunk] . P^T[chunk][qb]
    auto pv = [&](const int buf, PTile& pf) {
        const uint16_t* pvp = sV[buf] + fr * VROW + 8 * hi;
#pragma unroll
        for (int kc = 0; kc < 4; kc++) {
#pragma unroll
            for (int db = 0; db < 4; db++) {
                v8 vf = __builtin_bit_cast(v8, *(const u32x4*)(pvp + 32 * db * VROW + 16 * kc));
#pragma unroll
                for (int qb = 0; qb < QB; qb++) o[qb][db] = Op<T>::mfma32(vf, pf[qb][kc], o[qb][db]);
            }
        }
    };

    const int ntiles = (lkv + KT - 1) / KT;
    gload(0);
    sstore(0);
    __syncthreads();

    STile s;
    PTile pf;
    if (!PS || w < NW / 2) {
        // in-phase: S(j), softmax(j), PV(j)
        for (int j = 0; j + 1 < ntiles; j++) {
            gload((j + 1) * KT);
            scores(j % NBUF, s);
            softmax(s, pf, j * KT, false);
            pv(j % NBUF, pf);
            sstore((j + 1) % NBUF);
            __syncthreads();
        }
        const int jl = ntiles - 1;
        scores(jl % NBUF, s);
        softmax(s, pf, jl * KT, true);
        pv(jl % NBUF, pf);
    } else {
        // half a tile behind: softmax(j-1), PV(j-1), S(j)
        for (int j = 0; j + 1 < ntiles; j++) {
            gload((j + 1) * KT);
            if (j > 0) {
                softmax(s, pf, (j - 1) * KT, false);
                pv((j - 1) % NBUF, pf);
            }
            scores(j % NBUF, s);
            sstore((j + 1) % NBUF);
            __syncthreads();
        }
        const int jl = ntiles - 1;
        if (jl > 0) {
            softmax(s, pf, (jl - 1) * KT, false);
            pv((jl - 1) % NBUF, pf);
        }
        scores(jl % NBUF, s);
        softmax(s, pf, jl * KT, true);
        pv(jl % NBUF, pf);
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
                u32x2 pk2 = {Op<T>::cvt2(o[qb][db][4 * rg] * sc, o[qb][db][4 * rg + 1] * sc),
                             Op<T>::cvt2(o[qb][db][4 * rg + 2] * sc, o[qb][db][4 * rg + 3] * sc)};
                *(u32x2*)(out + (size_t)q * LTX_D + h * LTX_HD + d) = pk2;
            }
        }
    }
}

#define ATTN_KERNEL(NAME, T, QB, FULL, NW, PS)                                                      \
    extern "C" __global__ void __launch_bounds__(64 * NW, 1) NAME(const LtxAttnArgs a) {           \
        attn_body<T, QB, FULL, NW, PS>(a);                                                          \
    }

ATTN_KERNEL(ltx_attn_f16, _Float16, 2, false, 4, false)
ATTN_KERNEL(ltx_attn_bf16, __bf16, 2, false, 4, false)
ATTN_KERNEL(ltx_attn_f16_w8, _Float16, 1, false, 8, false)
ATTN_KERNEL(ltx_attn_bf16_w8, __bf16, 1, false, 8, false)
ATTN_KERNEL(ltx_attn_f16_w8_full, _Float16, 1, true, 8, false)
ATTN_KERNEL(ltx_attn_bf16_w8_full, __bf16, 1, true, 8, false)
ATTN_KERNEL(ltx_attn_f16_ps, _Float16, 1, false, 8, true)
ATTN_KERNEL(ltx_attn_bf16_ps, __bf16, 1, false, 8, true)
ATTN_KERNEL(ltx_attn_f16_ps_full, _Float16, 1, true, 8, true)
ATTN_KERNEL(ltx_attn_bf16_ps_full, __bf16, 1, true, 8, true)
