// Blockwise online-softmax attention for gfx950 (the production attention of
// ltx/block.zig:105-154, whileSdpaC), fused with the per-(token, head) gate
// 2*sigmoid(glog) and the head merge (ltx/block.zig:237-242). Two kernels:
//
// - ltx_attn_{f16,bf16}_pp (the ping-pong kernel, below): whole 64-key tiles
//   (lkv % 64 == 0, at least two), K and V^T streamed global -> LDS by DMA;
//   the block's self- and cross-attention take it;
// - ltx_attn_{f16,bf16}_w8[_full] (any key count): 8 waves of 32 queries, K
//   and V^T staged through registers into LDS, keys past lkv masked.
//
// Both compute the scores TRANSPOSED, S^T = K . Q^T, and the output as
// O^T = V^T . P^T: the query is then the MFMA column index, so a query's
// running max m, partial sums l and O^T column stay in the few lanes that
// hold that column, and only the tile max needs an exchange between them.
// The P^T operand comes straight from the S^T accumulators (no LDS round
// trip): the K tile is stored in LDS with its rows permuted so that the
// accumulator layout hands each lane the keys of its P^T operand in order.
// The w8 kernel uses v_mfma_f32_32x32x16 (lane l holds query l % 32; within
// every 16-key chunk the keys are consumed in the order 0-3, 8-11, 4-7,
// 12-15), the ping-pong kernel v_mfma_f32_16x16x32 (below).
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
// a multiple of 64 (no tail handling, no masking).
template <typename T, int QB, bool FULL, int NW>
__device__ void attn_body(const LtxAttnArgs& a) {
    typedef typename Op<T>::v8 v8;
    constexpr int NT = 64 * NW;         // threads per workgroup
    constexpr int QT = NW * 32 * QB;    // queries per workgroup
    constexpr int QW = 32 * QB;         // queries per wave
    constexpr int NBUF = 2;             // LDS tile buffers
    __shared__ __attribute__((aligned(16))) uint16_t sK[NBUF][KT * KROW];
    __shared__ __attribute__((aligned(16))) uint16_t sV[NBUF][LTX_HD * VROW];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int nblk = a.q_tiles * LTX_H;
    int t = blockIdx.x;
    if ((nblk & 7) == 0) t = (t & 7) * (nblk >> 3) + (t >> 3);  // one XCD per run of tiles (same head)
    const int h = t / a.q_tiles, qt = t - h * a.q_tiles;
    const int q0 = qt * QT + w * QW;
    const int lq = a.lq, lkv = a.lkv;

    const uint16_t* Q = (const uint16_t*)a.q + (size_t)h * a.q_hs;
    const uint16_t* K = (const uint16_t*)a.k + (size_t)h * a.k_hs;
    const uint16_t* V = (const uint16_t*)a.vt + (size_t)h * LTX_HD * lkv;

    // Q^T operand: lane holds Q[q][16 c + 8 (lane / 32) .. + 8] for its query.
    const int fr = lane & 31, hi = lane >> 5;
    v8 qf[QB][8];
#pragma unroll
    for (int qb = 0; qb < QB; qb++) {
        const int q = min(q0 + 32 * qb + fr, lq - 1);
#pragma unroll
        for (int c = 0; c < 8; c++)
            qf[qb][c] = __builtin_bit_cast(v8, *(const u32x4*)(Q + (size_t)q * a.q_rs + 16 * c + 8 * hi));
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
            rk[i] = *(const u32x4*)(K + (size_t)key * a.k_rs + 8 * c16);
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
    // S(j), softmax(j), PV(j)
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

    // out[q][h * 128 + d] = O^T[d][q] / l * 2 sigmoid(glog[q][h])
    uint16_t* out = (uint16_t*)a.out;
    unsigned bad = 0;  // 16-bit outputs out of range (range guard)
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
#pragma unroll
                for (int e = 0; e < 4; e++) bad += out_of_range<T>(o[qb][db][4 * rg + e] * sc);
            }
        }
    }
    range_report(a.sat, bad);
}

#define ATTN_KERNEL(NAME, T, QB, FULL, NW)                                                          \
    extern "C" __global__ void __launch_bounds__(64 * NW, 1) NAME(const LtxAttnArgs a) {           \
        attn_body<T, QB, FULL, NW>(a);                                                              \
    }

// the any-length kernels: 8 waves of 32 queries, registers-staged K/V
ATTN_KERNEL(ltx_attn_f16_w8, _Float16, 1, false, 8)
ATTN_KERNEL(ltx_attn_bf16_w8, __bf16, 1, false, 8)
ATTN_KERNEL(ltx_attn_f16_w8_full, _Float16, 1, true, 8)
ATTN_KERNEL(ltx_attn_bf16_w8_full, __bf16, 1, true, 8)

// ---------------------------------------------------------------------------
// Helpers of the LDS-DMA kernel below.
typedef __attribute__((address_space(3))) void* attn_lds_ptr;
#define ASP_WAIT_VM(n) ((((n) & 15) | (((n) >> 4) << 14)) | (7 << 4) | (15 << 8))
#define ASP_WAIT_LGKM0 (15 | (3 << 14) | (7 << 4))
#define ASP_RSRC_W3 0x00020000

// max of x and the same register in the other half of the wave (lane ^ 32)
__device__ __forceinline__ float asp_xhalf_max(float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return fmaxf(x, fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1])));
}

// ---------------------------------------------------------------------------
// max of x over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (one query's lanes
// in the 16 x 16 layout)
__device__ __forceinline__ float asp_quad_max(float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    x = fmaxf(x, fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1])));
    return asp_xhalf_max(x);
}

// ---------------------------------------------------------------------------
// Ping-pong kernel for whole 64-key tiles (lkv % 64 == 0, at least two
// tiles), on v_mfma_f32_16x16x32: 8 waves of 32 queries; waves w and w + 4
// share a SIMD and run one phase apart. A wave alternates an MFMA phase
// (PV(t-1) then S(t), fragments from LDS) with a softmax phase (softmax(t),
// the rare output rescale, and the DMA of K(t+2) and V(t+1)), so at any time
// one wave of each SIMD feeds the matrix core while the other runs the VALU
// work. One s_barrier per phase keeps the pairing. At equal flops the
// 16 x 16 x 32 MFMA runs faster than 32 x 32 x 16 at the board's
// power-limited clock (self-attention at 28,672 tokens: 10.15 against
// 10.88 ms on one box), with the same LDS bytes per flop: every 1 KB K or
// V^T fragment feeds the MFMAs of both query blocks.
//
// Layout (16 x 16 x 32: A lane l = row l % 16, k 8 (l / 16) .. + 7; B lane l
// = column l % 16, same k; D lane l = column l % 16, rows 4 (l / 16) .. + 3):
// - a wave's 32 queries are two column blocks qb; lane l holds queries
//   16 qb + l % 16, so each query's scores live in the four lanes l % 16 +
//   16 j, which share its running max (one exchange over l ^ 16, l ^ 32);
// - S^T = K . Q^T in four 16-key blocks kb, four 32-dim steps;
// - O^T = V^T . P^T in eight 16-dim blocks db, two 32-key steps kc. The P^T
//   operand of step kc is the lane's own accumulators of key blocks 2 kc and
//   2 kc + 1 (4 + 4 values): LDS row R of a K tile holds key
//   32 R5 + 16 R3 + 8 R2 + 4 R4 + 2 R1 + R0 (bits of R), so that these
//   8 values are keys 8 (l / 16) .. + 7 of the step, in V^T's natural order.
//
// LDS: K tiles of 64 rows x 256 B, 16-byte chunk c of row r in slot
// c ^ (r & 15); V^T tiles of 128 rows x 128 B with chunk c of row d in slot
// c ^ ((d >> 1) & 7). Four stages each (streaming form), distinct objects.
//
// DMA and waits (G0 = waves 0-3 lead, G1 = waves 4-7 follow one phase
// later): G0 issues all of K(t+2) and V(t+2) (its slices and G1's) at the
// start of its softmax phase t, and at the end of softmax phase t waits for
// what it issued one softmax phase earlier: K(t+1) and V(t+1) are complete
// before the barrier after which G0's MFMA phase t+1 (and, half a step
// later, G1's) reads K(t+1); V(t+1) is read from the softmax phase t+1 on
// (the first fragments of PV(t+1)). G1 issues no DMA: its softmax phase runs
// one phase after G0's, so slices it issued would have only one phase to
// land (measured 1 % slower on the whole kernel).
//
// The softmax state (running max m, partial sums l) is held in vector
// values: as arrays in the kernel's state the compiler placed them in LDS,
// which added LDS round trips and waits to every phase (10 % slower).
__shared__ __attribute__((aligned(1024))) uint8_t app_k0[16384];
__shared__ __attribute__((aligned(1024))) uint8_t app_k1[16384];
__shared__ __attribute__((aligned(1024))) uint8_t app_k2[16384];
__shared__ __attribute__((aligned(1024))) uint8_t app_k3[16384];
__shared__ __attribute__((aligned(1024))) uint8_t app_v0[16384];
__shared__ __attribute__((aligned(1024))) uint8_t app_v1[16384];
__shared__ __attribute__((aligned(1024))) uint8_t app_v2[16384];
__shared__ __attribute__((aligned(1024))) uint8_t app_v3[16384];

template <int S>
__device__ __forceinline__ uint8_t* app_k() {
    return S == 0 ? app_k0 : S == 1 ? app_k1 : S == 2 ? app_k2 : app_k3;
}
template <int S>
__device__ __forceinline__ uint8_t* app_v() {
    return S == 0 ? app_v0 : S == 1 ? app_v1 : S == 2 ? app_v2 : app_v3;
}


// PS: Q arrives multiplied by the exponent scale C = log2(e)/sqrt(128) (the
// block's qk-norm kernel writes it so), so a score is already in exp2 units.
template <typename T, bool PS>
struct AttnPP {
    typedef typename Op<T>::v8 v8;
    const LtxAttnArgs& a;
    __amdgpu_buffer_rsrc_t rk, rv;
    uint32_t gk[2], gv[2];  // per-lane DMA source offsets in tile 0
    uint32_t kr;            // bytes between consecutive K rows
    int lw;                 // this wave's 2 KB slice of a stage
    uint32_t ok[4];         // K fragment offsets per 32-dim step ks (kb adds 4096)
    uint32_t ov[2];         // V^T fragment offsets per 32-key step kc (db adds 2048)
    v8 qf[2][4];            // Q^T operand [qb][ks]
    f32x4 o[8][2];          // O^T [db][qb]
    f32x4 s[4][2];          // S^T [kb][qb]
    v8 pf[2][2];            // P^T operand [kc][qb]
    v8 vpre[4];             // V^T fragments kc = 0, db = 0..3 of the next PV, read in the softmax phase (resident form)
    f32x4 sb[2];            // -m of the lane's query in block qb: the S MFMAs start from it
    f32x2 m, l;             // running max and partial sum per query block (vectors, not arrays: kept in registers)
    float C;
    int nt, g;

    __device__ __forceinline__ AttnPP(const LtxAttnArgs& args) : a(args) {}

    // Group 0 (waves 0-3) issues every DMA: wave w fills its own 2 KB slice
    // of a stage and that of wave w + 4 (8 KB further, K rows + 32 = keys
    // + 32, V^T rows + 64), 4 instructions per K or V tile.
    template <int S>
    __device__ __forceinline__ void dma_k(int t) {
        uint8_t* d = app_k<S>() + lw;
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int i = 0; i < 2; i++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (attn_lds_ptr)(d + 8192 * h + 1024 * i), 16, gk[i],
                                                         (uint32_t)(64 * t + 32 * h) * kr, 0, 0);
    }
    template <int S>
    __device__ __forceinline__ void dma_v(int t) {
        uint8_t* d = app_v<S>() + lw;
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int i = 0; i < 2; i++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (attn_lds_ptr)(d + 8192 * h + 1024 * i), 16, gv[i],
                                                         t * 128 + 128 * a.lkv * h, 0, 0);
    }

    // MFMA phase t: PV(t-1) from the V^T tile at sv, then S(t) from the K tile
    // at sk; each fragment feeds the MFMAs of both query blocks. PRE: the
    // first four V^T fragments were read into vpre at the end of the softmax
    // phase before (prefetch_v), so the phase opens with MFMAs instead of
    // waiting out its first LDS reads (the resident form: its K/V never
    // change, so any phase may read them).
    template <bool PRE = false>
    __device__ __forceinline__ void mfma_phase(const uint8_t* sk, const uint8_t* sv, bool ds, bool dp) {
        if (dp) {
#pragma unroll
            for (int kc = 0; kc < 2; kc++)
#pragma unroll
                for (int db = 0; db < 8; db++) {
                    const v8 vf = PRE && kc == 0 && db < 4
                                      ? vpre[db & 3]
                                      : __builtin_bit_cast(v8, *(const u32x4*)(sv + ov[kc] + 2048 * db));
                    o[db][0] = Op<T>::mfma16(vf, pf[kc][0], o[db][0]);
                    o[db][1] = Op<T>::mfma16(vf, pf[kc][1], o[db][1]);
                }
        }
        if (ds) {
#pragma unroll
            for (int kb = 0; kb < 4; kb++) {
                s[kb][0] = sb[0];
                s[kb][1] = sb[1];
            }
#pragma unroll
            for (int ks = 0; ks < 4; ks++)
#pragma unroll
                for (int kb = 0; kb < 4; kb++) {
                    const v8 kf = __builtin_bit_cast(v8, *(const u32x4*)(sk + ok[ks] + 4096 * kb));
                    s[kb][0] = Op<T>::mfma16(kf, qf[0][ks], s[kb][0]);
                    s[kb][1] = Op<T>::mfma16(kf, qf[1][ks], s[kb][1]);
                }
        }
        // fragment reads eight MFMAs (four reads) ahead (masks: 0x100 DS
        // read, 0x008 MFMA); with PRE the first four are already in registers
        if (!PRE) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
        for (int i = 0; i < 32; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            if (i < 28) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
    }

    // the first four V^T fragments of the next MFMA phase's PV (tile at sv)
    __device__ __forceinline__ void prefetch_v(const uint8_t* sv) {
#pragma unroll
        for (int db = 0; db < 4; db++) vpre[db] = __builtin_bit_cast(v8, *(const u32x4*)(sv + ov[0] + 2048 * db));
    }

    // P^T operands and their row sums, per query block. s holds score - m
    // (the MFMAs start from sb = -m), so the weight is exp2(s) with Q
    // pre-scaled (PS), else exp2(s C); ADJ subtracts a further max shift
    // delta. The row sum adds exactly the rounded 16-bit weights that feed
    // the MFMA, on the VALU.
    template <bool ADJ>
    __device__ __forceinline__ f32x2 exps(f32x2 delta) {
        f32x2 ps = {0.f, 0.f};
#pragma unroll
        for (int kc = 0; kc < 2; kc++)
#pragma unroll
            for (int qb = 0; qb < 2; qb++) {
                float p[8];
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    float x = s[2 * kc + (e >> 2)][qb][e & 3];
                    if (ADJ) x -= delta[qb];
                    p[e] = __builtin_amdgcn_exp2f(PS ? x : x * C);
                }
                const uint32_t w0 = Op<T>::cvt2(p[0], p[1]), w1 = Op<T>::cvt2(p[2], p[3]),
                               w2 = Op<T>::cvt2(p[4], p[5]), w3 = Op<T>::cvt2(p[6], p[7]);
                float t = ps[qb];
                t = Op<T>::sum2(w0, t);
                t = Op<T>::sum2(w1, t);
                t = Op<T>::sum2(w2, t);
                t = Op<T>::sum2(w3, t);
                ps[qb] = t;
                pf[kc][qb] = __builtin_bit_cast(v8, (u32x4){w0, w1, w2, w3});
            }
        return ps;
    }

    // softmax phase: S^T accumulators -> P^T operands. The weights are first
    // formed with the running max; only if some lane's sum of its rounded
    // weights exceeds 2^8 (a weight above 2^8, or an f16 overflow, which sums
    // to inf) is the tile max taken (over the query's four lanes), the max
    // moved, the output and row sum rescaled (after PV(t-1), before PV(t))
    // and the weights formed again. The first tile always takes that path
    // and sets m to its max.
    __device__ __forceinline__ void softmax(bool first) {
        f32x2 ps = exps<false>(f32x2{0.f, 0.f});
        if (first || __builtin_amdgcn_ballot_w64(!(ps[0] <= 256.0f) || !(ps[1] <= 256.0f)) != 0) {
            f32x2 delta;
#pragma unroll
            for (int qb = 0; qb < 2; qb++) {
                float mx = s[0][qb][0];
#pragma unroll
                for (int kb = 0; kb < 4; kb++)
#pragma unroll
                    for (int r = 0; r < 4; r++) mx = fmaxf(mx, s[kb][qb][r]);
                mx = asp_quad_max(mx);  // tile max relative to m
                delta[qb] = first ? mx : fmaxf(mx, 0.f);
                const float corr = first ? 0.f : __builtin_amdgcn_exp2f(PS ? -delta[qb] : -delta[qb] * C);
                m[qb] += delta[qb];
                l[qb] *= corr;
#pragma unroll
                for (int db = 0; db < 8; db++) o[db][qb] *= corr;
                sb[qb] = f32x4{0} - m[qb];
            }
            ps = exps<true>(delta);
        }
        l += ps;
    }

    __device__ __forceinline__ void barrier() {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(ASP_WAIT_LGKM0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    }

    // MFMA phase t then softmax phase t (T4 = t mod 4); returns after the
    // softmax phase's barrier (or after the MFMA phase's when t == nt).
    // FULL: 1 <= t and t + 2 < nt, every operation present. The wave in its
    // MFMA phase takes issue priority over the other wave of its SIMD.
    //
    // K and V^T both run two tiles ahead in four stages each: the softmax
    // phase t issues K(t + 2) and V(t + 2) and waits for K(t + 1) and V(t + 1),
    // so V(t) is complete one phase before the PV(t) that reads it, and the
    // softmax phase reads PV(t)'s first four V^T fragments (prefetch_v): the
    // MFMA phase opens with MFMAs instead of waiting out those reads. (With V one tile ahead in three stages, V(t) completed
    // only at the barrier before PV(t).)
    template <int T4, bool FULL>
    __device__ __forceinline__ void step(int t) {
        __builtin_amdgcn_s_setprio(1);
        mfma_phase<true>(app_k<T4>(), app_v<(T4 + 3) % 4>(), FULL || t < nt, FULL || t >= 1);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
        barrier();
        if (!FULL && t >= nt) return;
        // read first, before this phase's DMA is in flight (the compiler's
        // LDS-DMA tracking made reads behind it wait for it)
        prefetch_v(app_v<T4>());
        __builtin_amdgcn_sched_barrier(0);
        const bool dkv = FULL || t + 2 < nt;
        if (g == 0 && dkv) {
            dma_k<(T4 + 2) % 4>(t + 2);
            dma_v<(T4 + 2) % 4>(t + 2);
        }
        __builtin_amdgcn_sched_barrier(0);
        softmax(!FULL && t == 0);
        pin_softmax_pre();
        __builtin_amdgcn_sched_barrier(0);
        if (g == 0) {
            if (dkv)
                __builtin_amdgcn_s_waitcnt(ASP_WAIT_VM(8));
            else
                __builtin_amdgcn_s_waitcnt(ASP_WAIT_VM(0));
        }
        barrier();
    }

    // Buffers, DMA sources and fragment offsets of head h (wave w)
    __device__ __forceinline__ void setup(int h, int w, int lane) {
        const int lkv = a.lkv;
        nt = lkv / 64;
        C = a.scale_log2;
        // K rows are kr bytes apart (head-major: 256; token rows: 8 KB)
        kr = 2u * (uint32_t)a.k_rs;
        rk = __builtin_amdgcn_make_buffer_rsrc((void*)((const uint16_t*)a.k + (size_t)h * a.k_hs), 0,
                                               (int)((uint32_t)(lkv - 1) * kr + 2u * LTX_HD), ASP_RSRC_W3);
        rv = __builtin_amdgcn_make_buffer_rsrc((void*)((const uint16_t*)a.vt + (size_t)h * LTX_HD * lkv), 0,
                                               lkv * LTX_HD * 2, ASP_RSRC_W3);
        lw = 2048 * w;
        // DMA sources: K instruction i of wave w fills LDS rows 4 (2 w + i) ..
        // +3 (16 lanes a row; row R holds key perm(R), the +32 half likewise);
        // V^T rows 8 (2 w + i) .. +7 (8 lanes a row)
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int r = 4 * (2 * w + i) + (lane >> 4);  // LDS row within the first 32
            const int key = (r & 3) | ((r & 16) >> 2) | ((r & 4) << 1) | ((r & 8) << 1);
            const int c = (lane & 15) ^ (r & 15);
            gk[i] = (uint32_t)key * kr + 16u * c;
            const int d = 8 * (2 * w + i) + (lane >> 3);
            const int cv = (lane & 7) ^ ((d >> 1) & 7);
            gv[i] = (uint32_t)d * (uint32_t)lkv * 2u + 16u * cv;
        }
        const int j = lane >> 4, r = lane & 15;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) ok[ks] = r * 256 + 16 * ((4 * ks + j) ^ r);
#pragma unroll
        for (int kc = 0; kc < 2; kc++) ov[kc] = r * 128 + 16 * ((4 * kc + j) ^ (r >> 1));
    }

    // Q^T operands of the wave's queries q0 .. q0 + 31 of head h (rows past
    // lq read row lq - 1)
    __device__ __forceinline__ void load_q(v8 (&dst)[2][4], int h, int q0, int lane) const {
        const uint16_t* Q = (const uint16_t*)a.q + (size_t)h * a.q_hs;
        const int j = lane >> 4, r = lane & 15;
#pragma unroll
        for (int qb = 0; qb < 2; qb++) {
            const int q = min(q0 + 16 * qb + r, a.lq - 1);
#pragma unroll
            for (int ks = 0; ks < 4; ks++)
                dst[qb][ks] = __builtin_bit_cast(v8, *(const u32x4*)(Q + (size_t)q * a.q_rs + 32 * ks + 8 * j));
        }
    }

    __device__ __forceinline__ void reset() {
#pragma unroll
        for (int db = 0; db < 8; db++) o[db][0] = o[db][1] = f32x4{0};
        m = f32x2{0.f, 0.f};
        sb[0] = sb[1] = f32x4{0};
        l = f32x2{0.f, 0.f};
    }

    // gate logits glog[q][h] of the lane's two queries (rows past lq read
    // row lq - 1; gl is left as it is without gate)
    __device__ __forceinline__ void load_glog(float (&gl)[2], int h, int q0, int lane) const {
        if (a.glog)
#pragma unroll
            for (int qb = 0; qb < 2; qb++)
                gl[qb] = a.glog[(size_t)min(q0 + 16 * qb + (lane & 15), a.lq - 1) * LTX_H + h];
    }

    // out[q][h * 128 + d] = O^T[d][q] / l * 2 sigmoid(glog[q][h]) for the
    // wave's queries q0 .. q0 + 31, through a wave-private LDS patch
    // [32 q][DPP d] (pitch DPP + 8 elements) per DPP dims
    template <int DPP>
    __device__ __forceinline__ void store_out(uint16_t* patch, int h, int q0, int lane, const float (&gl)[2],
                                              unsigned& bad) const {
        constexpr int LD = DPP + 8, LPR = DPP / 8, RPI = 64 / LPR;  // lanes per row, rows per instruction
        const int j = lane >> 4, r = lane & 15;
        float sc[2];
        bool qok[2];
#pragma unroll
        for (int qb = 0; qb < 2; qb++) {
            float lt = l[qb] + __shfl_xor(l[qb], 16, 64);
            lt += __shfl_xor(lt, 32, 64);
            qok[qb] = q0 + 16 * qb + r < a.lq;
            const float gg = a.glog ? 2.0f * sigmoid_f(gl[qb]) : 1.0f;
            sc[qb] = gg / lt;
        }
        uint16_t* out = (uint16_t*)a.out;
#pragma unroll
        for (int part = 0; part < 128 / DPP; part++) {
#pragma unroll
            for (int dbh = 0; dbh < DPP / 16; dbh++) {
                const int db = (DPP / 16) * part + dbh;
#pragma unroll
                for (int qb = 0; qb < 2; qb++) {
                    const f32x4 v = o[db][qb] * sc[qb];
                    *(u32x2*)(patch + (16 * qb + r) * LD + 16 * dbh + 4 * j) =
                        u32x2{Op<T>::cvt2(v[0], v[1]), Op<T>::cvt2(v[2], v[3])};
                    if (qok[qb])
#pragma unroll
                        for (int e = 0; e < 4; e++) bad += out_of_range<T>(v[e]);
                }
            }
#pragma unroll
            for (int it = 0; it < 32 / RPI; it++) {
                const int row = RPI * it + lane / LPR, c = lane % LPR;  // LPR lanes x 16 B per row
                const u32x4 v = *(const u32x4*)(patch + row * LD + 8 * c);
                const int q = q0 + row;
                if (q < a.lq) *(u32x4*)(out + (size_t)q * LTX_D + h * LTX_HD + DPP * part + 8 * c) = v;
            }
        }
    }

    __device__ __forceinline__ void run() {
        const int tid = threadIdx.x, lane = tid & 63;
        const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
        g = w >> 2;
        const int nblk = a.q_tiles * LTX_H;
        int t = blockIdx.x;
        if ((nblk & 7) == 0) t = (t & 7) * (nblk >> 3) + (t >> 3);
        const int h = t / a.q_tiles, qt = t - h * a.q_tiles;
        const int q0 = qt * 256 + w * 32;
        setup(h, w, lane);
        load_q(qf, h, q0, lane);
        reset();
        if (g == 0) {  // K(0) and V(0) complete, K(1) and V(1) in flight
            dma_k<0>(0);
            dma_v<0>(0);
            dma_k<1>(1);
            dma_v<1>(1);
            __builtin_amdgcn_s_waitcnt(ASP_WAIT_VM(8));
        }
        __builtin_amdgcn_s_barrier();
        if (g == 1) __builtin_amdgcn_s_barrier();
        step<0, false>(0);
        int u = 1;
        for (; u + 5 < nt; u += 4) {
            step<1, true>(u);
            step<2, true>(u + 1);
            step<3, true>(u + 2);
            step<0, true>(u + 3);
        }
        for (; u <= nt; u += 4) {
            step<1, false>(u);
            if (u + 1 <= nt) step<2, false>(u + 1);
            if (u + 2 <= nt) step<3, false>(u + 2);
            if (u + 3 <= nt) step<0, false>(u + 3);
        }
        if (g == 0) __builtin_amdgcn_s_barrier();
        // every wave has passed its last barrier: the K stages hold the
        // wave-private patches
        uint16_t* patch = (uint16_t*)(w < 3 ? app_k0 + 4608 * w : w < 6 ? app_k1 + 4608 * (w - 3) : app_k2 + 4608 * (w - 6));
        unsigned bad = 0;  // 16-bit outputs out of range (range guard)
        float gl[2] = {0.f, 0.f};
        load_glog(gl, h, q0, lane);
        store_out<64>(patch, h, q0, lane, gl, bad);
        range_report(a.sat, bad);
    }

    // the softmax phase's results stay in registers (not rematerialised in
    // the next phase)
    __device__ __forceinline__ void pin_softmax() {
#pragma unroll
        for (int kc = 0; kc < 2; kc++)
#pragma unroll
            for (int qb = 0; qb < 2; qb++) asm volatile("" ::"v"(__builtin_bit_cast(u32x4, pf[kc][qb])));
        asm volatile("" ::"v"(l), "v"(m));
        asm volatile("" ::"v"(sb[0]), "v"(sb[1]));
    }

    // as pin_softmax, and the prefetched V^T fragments of the next PV
    __device__ __forceinline__ void pin_softmax_pre() {
        pin_softmax();
#pragma unroll
        for (int db = 0; db < 4; db++) asm volatile("" ::"v"(__builtin_bit_cast(u32x4, vpre[db])));
    }

    // after the last softmax of a query tile: the next MFMA phase starts the
    // next tile (S(0) from a zero max, with its Q)
    __device__ __forceinline__ void next_tile(const v8 (&qn)[2][4]) {
        m = f32x2{0.f, 0.f};
        sb[0] = sb[1] = f32x4{0};
#pragma unroll
        for (int qb = 0; qb < 2; qb++)
#pragma unroll
            for (int ks = 0; ks < 4; ks++) qf[qb][ks] = qn[qb][ks];
    }

    template <bool PRE>
    __device__ __forceinline__ void rphase(const uint8_t* sk, const uint8_t* sv, bool ds, bool dp) {
        __builtin_amdgcn_s_setprio(1);
        mfma_phase<PRE>(sk, sv, ds, dp);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
        barrier();
    }

    // Resident K/V (lkv = 64 nt, 1 <= nt <= 4): the workgroup loads head h's
    // whole K and V^T into LDS once (kres, vres: nt tiles of 16 KB each, the
    // stage layouts above), then runs query tiles qt0, qt0 + wph, ... of that
    // head with no DMA, as one continuous ping-pong over the (query tile, key
    // tile) sequence: the MFMA phase after the last softmax of tile i runs
    // PV_i(nt - 1) and S_i+1(0), and tile i's output is stored in the next
    // softmax phase, before softmax_i+1(0) clears O and l. The running max
    // and the Q^T operands switch to tile i + 1 at the end of softmax_i(nt -
    // 1). The next tile's Q and the tile's gate logits load while it runs.
    // Every query tile takes 2 nt barriers in both groups (group 1 keeps its
    // one-phase lag), plus one after the final PV.
    __device__ __forceinline__ void run_resident(uint8_t* kres, uint8_t* vres, uint16_t* patches) {
        const int tid = threadIdx.x, lane = tid & 63;
        const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
        g = w >> 2;
        const int wph = gridDim.x / LTX_H;  // workgroups per head
        const int h = blockIdx.x / wph, qt0 = blockIdx.x - h * wph;
        if (h >= LTX_H || qt0 >= a.q_tiles) return;  // uniform over the workgroup
        setup(h, w, lane);
        // group 0 loads every K and V^T tile (its slices and group 1's)
        if (g == 0) {
            for (int t = 0; t < nt; t++) {
#pragma unroll
                for (int hh = 0; hh < 2; hh++)
#pragma unroll
                    for (int i = 0; i < 2; i++) {
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(
                            rk, (attn_lds_ptr)(kres + 16384 * t + lw + 8192 * hh + 1024 * i), 16, gk[i],
                            (uint32_t)(64 * t + 32 * hh) * kr, 0, 0);
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(
                            rv, (attn_lds_ptr)(vres + 16384 * t + lw + 8192 * hh + 1024 * i), 16, gv[i],
                            t * 128 + 128 * a.lkv * hh, 0, 0);
                    }
            }
        }
        int q0 = qt0 * 256 + w * 32;
        load_q(qf, h, q0, lane);
        float gl[2] = {0.f, 0.f};  // gate logits of the tile being computed, until its output is stored
        load_glog(gl, h, q0, lane);
        reset();
        __builtin_amdgcn_s_waitcnt(ASP_WAIT_VM(0));
        __builtin_amdgcn_s_barrier();
        if (g == 1) __builtin_amdgcn_s_barrier();
        uint16_t* patch = patches + 1280 * w;  // [32 q][40]: 32 dims per pass
        unsigned bad = 0;  // 16-bit outputs out of range (range guard)
        v8 qn[2][4];       // the next tile's Q^T operands
        for (int qt = qt0; qt < a.q_tiles; qt += wph) {
            const bool prev = qt > qt0;
            // t = 0: PV of the previous tile's last key tile, S(0); then the
            // previous tile's output, this tile's gate logits and the next
            // tile's Q (read at t = nt - 1)
            if (prev)
                rphase<true>(kres, vres + 16384 * (nt - 1), true, true);
            else
                rphase<false>(kres, vres + 16384 * (nt - 1), true, false);
            // unconditional (rows past lq read row lq - 1), so that every
            // path waits for these loads where qf takes them; issued before
            // the output stores, which would otherwise queue ahead of them
            load_q(qn, h, q0 + 256 * wph, lane);
            if (prev) {
                store_out<32>(patch, h, q0 - 256 * wph, lane, gl, bad);
                load_glog(gl, h, q0, lane);
            }
            softmax(true);
            if (nt == 1) next_tile(qn);
            prefetch_v(vres);
            pin_softmax_pre();
            barrier();
            for (int t = 1; t < nt - 1; t++) {
                rphase<true>(kres + 16384 * t, vres + 16384 * (t - 1), true, true);
                softmax(false);
                prefetch_v(vres + 16384 * t);
                pin_softmax_pre();
                barrier();
            }
            if (nt > 1) {
                rphase<true>(kres + 16384 * (nt - 1), vres + 16384 * (nt - 2), true, true);
                softmax(false);
                next_tile(qn);
                prefetch_v(vres + 16384 * (nt - 1));
                pin_softmax_pre();
                barrier();
            }
            q0 += 256 * wph;
        }
        // the last tile's last PV, then its output
        rphase<true>(kres, vres + 16384 * (nt - 1), false, true);
        store_out<32>(patch, h, q0 - 256 * wph, lane, gl, bad);
        if (g == 0) __builtin_amdgcn_s_barrier();
        range_report(a.sat, bad);
    }
};

// _pp: Q pre-scaled by scale_log2 (the block's layout); _pp_uq: plain Q.
extern "C" __global__ void __launch_bounds__(512, 1) ltx_attn_f16_pp(const LtxAttnArgs a) {
    AttnPP<_Float16, true> k(a);
    k.run();
}
extern "C" __global__ void __launch_bounds__(512, 1) ltx_attn_bf16_pp(const LtxAttnArgs a) {
    AttnPP<__bf16, true> k(a);
    k.run();
}
extern "C" __global__ void __launch_bounds__(512, 1) ltx_attn_f16_pp_uq(const LtxAttnArgs a) {
    AttnPP<_Float16, false> k(a);
    k.run();
}
extern "C" __global__ void __launch_bounds__(512, 1) ltx_attn_bf16_pp_uq(const LtxAttnArgs a) {
    AttnPP<__bf16, false> k(a);
    k.run();
}

// _kv: resident K/V (a multiple of 64 keys, at most 256), persistent over
// query tiles: grid = LTX_H x workgroups per head
__shared__ __attribute__((aligned(1024))) uint8_t arx_k[65536];
__shared__ __attribute__((aligned(1024))) uint8_t arx_v[65536];
__shared__ __attribute__((aligned(1024))) uint16_t arx_patch[8 * 1280];
extern "C" __global__ void __launch_bounds__(512, 1) ltx_attn_f16_kv(const LtxAttnArgs a) {
    AttnPP<_Float16, true> k(a);
    k.run_resident(arx_k, arx_v, arx_patch);
}
extern "C" __global__ void __launch_bounds__(512, 1) ltx_attn_bf16_kv(const LtxAttnArgs a) {
    AttnPP<__bf16, true> k(a);
    k.run_resident(arx_k, arx_v, arx_patch);
}
extern "C" __global__ void __launch_bounds__(512, 1) ltx_attn_f16_kv_uq(const LtxAttnArgs a) {
    AttnPP<_Float16, false> k(a);
    k.run_resident(arx_k, arx_v, arx_patch);
}
extern "C" __global__ void __launch_bounds__(512, 1) ltx_attn_bf16_kv_uq(const LtxAttnArgs a) {
    AttnPP<__bf16, false> k(a);
    k.run_resident(arx_k, arx_v, arx_patch);
}
