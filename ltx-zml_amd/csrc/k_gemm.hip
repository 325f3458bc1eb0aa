// W8A16 / W16A16 GEMM for gfx950: y[M][N] = A[M][K] . W[N][K]^T with fused
// epilogues (bias, GELU-tanh, gated residual, QKV split with V^T store).
//
// Tile 256 x 256 x 64 per workgroup of NW waves: NW = 4 (a 2 x 2 grid of
// 128 x 128 wave tiles, one wave per SIMD) or NW = 8 (2 x 4 grid of 128 x 64
// wave tiles, two waves per SIMD so one wave's dequant/LDS work overlaps the
// other's MFMAs). v_mfma_f32_32x32x16_{f16,bf16}, fp32 accumulate.
// Global -> register -> LDS staging with two LDS buffers and one barrier per
// K-tile; MFMA fragments double-buffered in registers. int8 weights are dequantised ONCE per workgroup
// while staging into LDS: v = fma(u, s, -128 s) with u = q + 128 (an unsigned
// byte), which is the single-rounding f32 value q * s of dq4
// (ltx/block.zig:462-471), then rounded to the 16-bit operand type.
// LDS rows are padded by 16 bytes.
#include "gemm_common.h"
#include "gemm_q8.h"
#include "gemm_w16.h"
#include "gemm_x4.h"

#define BM 256
#define BN 256
#define BK 64
#define LDSW (BK + 8)  // 16-bit elements per padded LDS row
template <typename T, int BKIND, int NT>
struct Stage {
    static constexpr int NA = BM * (BK / 8) / NT;    // 16-byte A chunks per thread
    static constexpr int NB8 = BN * (BK / 16) / NT;  // 16-byte int8 B chunks per thread
    static constexpr int NB16 = BN * (BK / 8) / NT;  // 16-byte 16-bit B chunks per thread
    static constexpr int NBR = BKIND == LTX_B_W16 ? NB16 : NB8;
    u32x4 ra[NA];
    u32x4 rb[NBR];
    float sc[NB8];

    __device__ __forceinline__ void load(const LtxGemmArgs& a, int m0, int n0, int k0, int tid) {
        const uint16_t* A = (const uint16_t*)a.a;
        const int c = tid & 7;
#pragma unroll
        for (int i = 0; i < NA; i++) {
            int r = min(m0 + (tid >> 3) + (NT / 8) * i, a.M - 1);
            ra[i] = *(const u32x4*)(A + (size_t)r * a.lda + k0 + 8 * c);
        }
        if (BKIND == LTX_B_W16) {
            const uint16_t* B = (const uint16_t*)a.b;
#pragma unroll
            for (int i = 0; i < NB16; i++) {
                int r = n0 + (tid >> 3) + (NT / 8) * i;
                rb[i] = *(const u32x4*)(B + (size_t)r * a.K + k0 + 8 * c);
            }
        } else {
            const int8_t* B = (const int8_t*)a.b;
            const int cb = tid & 3;
            const int G = a.K / LTX_GROUP;
#pragma unroll
            for (int i = 0; i < NB8; i++) {
                int r = n0 + (tid >> 2) + (NT / 4) * i;
                rb[i] = *(const u32x4*)(B + (size_t)r * a.K + k0 + 16 * cb) ^ a.qxor;  // -> bytes q + 128
                size_t si = (size_t)r * G + (k0 + 16 * cb) / LTX_GROUP;
                sc[i] = BKIND == LTX_B_I8_F16S ? f16_bits_to_f32(((const uint16_t*)a.scales)[si])
                                              : ((const float*)a.scales)[si];
            }
        }
    }

    __device__ __forceinline__ void store(uint16_t* sA, uint16_t* sB, int tid) {
        const int c = tid & 7;
#pragma unroll
        for (int i = 0; i < NA; i++) *(u32x4*)(sA + ((tid >> 3) + (NT / 8) * i) * LDSW + 8 * c) = ra[i];
        if (BKIND == LTX_B_W16) {
#pragma unroll
            for (int i = 0; i < NB16; i++) *(u32x4*)(sB + ((tid >> 3) + (NT / 8) * i) * LDSW + 8 * c) = rb[i];
        } else {
            const int cb = tid & 3;
#pragma unroll
            for (int i = 0; i < NB8; i++) {
                const float s = sc[i], nb = -128.0f * s;
                uint32_t o[8];
#pragma unroll
                for (int d = 0; d < 4; d++) {
                    const uint32_t w = rb[i][d];  // bytes q + 128
                    o[2 * d] = deq_pack2<T>((float)(w & 0xffu), (float)((w >> 8) & 0xffu), s, nb);
                    o[2 * d + 1] = deq_pack2<T>((float)((w >> 16) & 0xffu), (float)(w >> 24), s, nb);
                }
                uint16_t* dst = sB + ((tid >> 2) + (NT / 4) * i) * LDSW + 16 * cb;
                *(u32x4*)dst = u32x4{o[0], o[1], o[2], o[3]};
                *(u32x4*)(dst + 8) = u32x4{o[4], o[5], o[6], o[7]};
            }
        }
    }
};

template <typename T, int BKIND, int EPI, int NW>
__device__ void gemm_body(const LtxGemmArgs& a) {
    typedef typename Op<T>::v8 v8;
    constexpr int NT = 64 * NW;
    constexpr int WNW = NW / 2;          // waves along N
    constexpr int WN = BN / WNW;         // wave tile N extent (128 or 64)
    constexpr int NI = 4, NJ = WN / 32;  // 32 x 32 MFMA blocks per wave
    __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM * LDSW];
    __shared__ __attribute__((aligned(16))) uint16_t sB[2][BN * LDSW];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int wm = w / WNW, wn = w % WNW;
    // split-K: workgroup b computes slice b % ksplit of K for tile b / ksplit
    const int ks_n = a.ksplit > 1 ? a.ksplit : 1;
    TileIdx ti = tile_of(blockIdx.x / ks_n, a.tiles_m, a.tiles_n);
    const int m0 = ti.tm * BM, n0 = ti.tn * BN;
    const int kc = a.K / ks_n, kb = (blockIdx.x % ks_n) * kc;  // this slice: k in [kb, kb + kc)

    f32x16 acc[NI][NJ];
#pragma unroll
    for (int i = 0; i < NI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[i][j] = f32x16{0};

    Stage<T, BKIND, NT> st;
    const int nk = kc / BK;
    st.load(a, m0, n0, kb, tid);
    st.store(sA[0], sB[0], tid);
    __syncthreads();

    // Fragments are double-buffered in registers: the LDS reads for k-step
    // kk + 1 are issued before the MFMAs of step kk; the next K-tile's global
    // loads are issued at the top of the tile and written to the other LDS
    // buffer after the MFMAs.
    const int fr = lane & 31, fk = 8 * (lane >> 5);
    const int offa = (wm * 128 + fr) * LDSW + fk, offb = (wn * WN + fr) * LDSW + fk;
    v8 fa[2][NI], fb[2][NJ];
    auto frags = [&](int buf, int kk, int slot) {
#pragma unroll
        for (int i = 0; i < NI; i++)
            fa[slot][i] = __builtin_bit_cast(v8, *(const u32x4*)(sA[buf] + offa + 32 * i * LDSW + 16 * kk));
#pragma unroll
        for (int j = 0; j < NJ; j++)
            fb[slot][j] = __builtin_bit_cast(v8, *(const u32x4*)(sB[buf] + offb + 32 * j * LDSW + 16 * kk));
    };
    frags(0, 0, 0);
    for (int kt = 0; kt < nk; kt++) {
        const int buf = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) st.load(a, m0, n0, kb + (kt + 1) * BK, tid);
#pragma unroll
        for (int kk = 0; kk < BK / 16; kk++) {
            const int cur = kk & 1;
            if (kk + 1 < BK / 16) frags(buf, kk + 1, cur ^ 1);
#pragma unroll
            for (int i = 0; i < NI; i++)
#pragma unroll
                for (int j = 0; j < NJ; j++) acc[i][j] = Op<T>::mfma32(fa[cur][i], fb[cur][j], acc[i][j]);
        }
        if (more) st.store(sA[buf ^ 1], sB[buf ^ 1], tid);
        __syncthreads();
        if (more) frags(buf ^ 1, 0, 0);
    }

    // acc[i][j][r]: row 32 i + 8 (r / 4) + 4 (lane / 32) + r % 4, column 32 j + lane % 32
    if (ks_n > 1) {  // the slice's partial sums; ltx_gemm_reduce_* applies the epilogue
        float* part = a.part + (size_t)(blockIdx.x % ks_n) * a.M * a.N;
        const int mr = m0 + wm * 128 + 4 * (lane >> 5), nc = n0 + wn * WN + (lane & 31);
#pragma unroll
        for (int i = 0; i < NI; i++)
#pragma unroll
            for (int j = 0; j < NJ; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int m = mr + 32 * i + 8 * (r >> 2) + (r & 3);
                    if (m < a.M) part[(size_t)m * a.N + nc + 32 * j] = acc[i][j][r];
                }
        return;
    }
    gemm_epilogue<T, EPI, NI, NJ>(a, acc, m0 + wm * 128 + 4 * (lane >> 5), n0 + wn * WN + (lane & 31), n0);
}

#define GEMM_KERNEL(NAME, T, BK_, EPI_)                                                        \
    extern "C" __global__ void __launch_bounds__(512, 1) NAME(const LtxGemmArgs a) {           \
        gemm_body<T, BK_, EPI_, 8>(a);                                                         \
    }

GEMM_KERNEL(ltx_gemm_f16_i8f32_store, _Float16, LTX_B_I8_F32S, LTX_EPI_STORE)
GEMM_KERNEL(ltx_gemm_f16_i8f32_resid, _Float16, LTX_B_I8_F32S, LTX_EPI_RESID_GATE)
GEMM_KERNEL(ltx_gemm_f16_i8f32_qkv, _Float16, LTX_B_I8_F32S, LTX_EPI_QKV)
GEMM_KERNEL(ltx_gemm_f16_i8f16_store, _Float16, LTX_B_I8_F16S, LTX_EPI_STORE)
GEMM_KERNEL(ltx_gemm_f16_i8f16_resid, _Float16, LTX_B_I8_F16S, LTX_EPI_RESID_GATE)
GEMM_KERNEL(ltx_gemm_f16_i8f16_qkv, _Float16, LTX_B_I8_F16S, LTX_EPI_QKV)
GEMM_KERNEL(ltx_gemm_f16_w16_store, _Float16, LTX_B_W16, LTX_EPI_STORE)
GEMM_KERNEL(ltx_gemm_f16_w16_resid, _Float16, LTX_B_W16, LTX_EPI_RESID_GATE)
GEMM_KERNEL(ltx_gemm_f16_w16_qkv, _Float16, LTX_B_W16, LTX_EPI_QKV)
GEMM_KERNEL(ltx_gemm_bf16_i8f32_store, __bf16, LTX_B_I8_F32S, LTX_EPI_STORE)
GEMM_KERNEL(ltx_gemm_bf16_i8f32_resid, __bf16, LTX_B_I8_F32S, LTX_EPI_RESID_GATE)
GEMM_KERNEL(ltx_gemm_bf16_i8f32_qkv, __bf16, LTX_B_I8_F32S, LTX_EPI_QKV)
GEMM_KERNEL(ltx_gemm_bf16_i8f16_store, __bf16, LTX_B_I8_F16S, LTX_EPI_STORE)
GEMM_KERNEL(ltx_gemm_bf16_i8f16_resid, __bf16, LTX_B_I8_F16S, LTX_EPI_RESID_GATE)
GEMM_KERNEL(ltx_gemm_bf16_i8f16_qkv, __bf16, LTX_B_I8_F16S, LTX_EPI_QKV)
GEMM_KERNEL(ltx_gemm_bf16_w16_store, __bf16, LTX_B_W16, LTX_EPI_STORE)
GEMM_KERNEL(ltx_gemm_bf16_w16_resid, __bf16, LTX_B_W16, LTX_EPI_RESID_GATE)
GEMM_KERNEL(ltx_gemm_bf16_w16_qkv, __bf16, LTX_B_W16, LTX_EPI_QKV)

// LDS-DMA W8A16 kernels (ping-pong schedule): ltx_gemm_q8_[bf16_][s32_]{store,
// resid,qkv} for f16 (bf16_: bf16) operands with f16 (s32_: f32) scales.
Q8_GEMM_KERNEL(ltx_gemm_q8_store, _Float16, false, LTX_EPI_STORE)
Q8_GEMM_KERNEL(ltx_gemm_q8_resid, _Float16, false, LTX_EPI_RESID_GATE)
Q8_GEMM_KERNEL(ltx_gemm_q8_qkv, _Float16, false, LTX_EPI_QKV)
Q8_GEMM_KERNEL(ltx_gemm_q8_bf16_store, __bf16, false, LTX_EPI_STORE)
Q8_GEMM_KERNEL(ltx_gemm_q8_bf16_resid, __bf16, false, LTX_EPI_RESID_GATE)
Q8_GEMM_KERNEL(ltx_gemm_q8_bf16_qkv, __bf16, false, LTX_EPI_QKV)
Q8_GEMM_KERNEL(ltx_gemm_q8_s32_store, _Float16, true, LTX_EPI_STORE)
Q8_GEMM_KERNEL(ltx_gemm_q8_s32_resid, _Float16, true, LTX_EPI_RESID_GATE)
Q8_GEMM_KERNEL(ltx_gemm_q8_s32_qkv, _Float16, true, LTX_EPI_QKV)
Q8_GEMM_KERNEL(ltx_gemm_q8_bf16_s32_store, __bf16, true, LTX_EPI_STORE)
Q8_GEMM_KERNEL(ltx_gemm_q8_bf16_s32_resid, __bf16, true, LTX_EPI_RESID_GATE)
Q8_GEMM_KERNEL(ltx_gemm_q8_bf16_s32_qkv, __bf16, true, LTX_EPI_QKV)

// LDS-DMA W16A16 kernels (unquantised weights): ltx_gemm_w16dma_{f16,bf16}_
// {store,resid,qkv}, 256 x 128 output tiles.
W16_GEMM_KERNEL(ltx_gemm_w16dma_f16_store, _Float16, LTX_EPI_STORE)
W16_GEMM_KERNEL(ltx_gemm_w16dma_f16_resid, _Float16, LTX_EPI_RESID_GATE)
W16_GEMM_KERNEL(ltx_gemm_w16dma_f16_qkv, _Float16, LTX_EPI_QKV)
W16_GEMM_KERNEL(ltx_gemm_w16dma_bf16_store, __bf16, LTX_EPI_STORE)
W16_GEMM_KERNEL(ltx_gemm_w16dma_bf16_resid, __bf16, LTX_EPI_RESID_GATE)
W16_GEMM_KERNEL(ltx_gemm_w16dma_bf16_qkv, __bf16, LTX_EPI_QKV)

// Four-wave 16-bit kernels (256 x 256 tiles, 16 x 16 x 32 MFMAs):
// ltx_gemm_x4_{f16,bf16}_{store,store_gelu,store32,store32_gelu,resid,qkv}
// (store32: f32 output), and the per-forward dequantisation of the int8
// weights they take: ltx_gemm_dq16_{f16,bf16} (fp16 scale pairs), _s32 (f32
// scales).
X4_GEMM_KERNEL(ltx_gemm_x4_f16_store, _Float16, LTX_EPI_STORE, 0)
X4_GEMM_KERNEL(ltx_gemm_x4_f16_store_gelu, _Float16, LTX_EPI_STORE, 1)
X4_GEMM_KERNEL(ltx_gemm_x4_f16_store32, _Float16, LTX_EPI_STORE, 2)
X4_GEMM_KERNEL(ltx_gemm_x4_f16_store32_gelu, _Float16, LTX_EPI_STORE, 3)
X4_GEMM_KERNEL(ltx_gemm_x4_f16_resid, _Float16, LTX_EPI_RESID_GATE, 0)
X4_GEMM_KERNEL(ltx_gemm_x4_f16_qkv, _Float16, LTX_EPI_QKV, 0)
X4_GEMM_KERNEL(ltx_gemm_x4_bf16_store, __bf16, LTX_EPI_STORE, 0)
X4_GEMM_KERNEL(ltx_gemm_x4_bf16_store_gelu, __bf16, LTX_EPI_STORE, 1)
X4_GEMM_KERNEL(ltx_gemm_x4_bf16_store32, __bf16, LTX_EPI_STORE, 2)
X4_GEMM_KERNEL(ltx_gemm_x4_bf16_store32_gelu, __bf16, LTX_EPI_STORE, 3)
X4_GEMM_KERNEL(ltx_gemm_x4_bf16_resid, __bf16, LTX_EPI_RESID_GATE, 0)
X4_GEMM_KERNEL(ltx_gemm_x4_bf16_qkv, __bf16, LTX_EPI_QKV, 0)
extern "C" __global__ void __launch_bounds__(256) ltx_gemm_dq16_f16(const LtxDq16Args a) { dq16_body<_Float16, false>(a); }
extern "C" __global__ void __launch_bounds__(256) ltx_gemm_dq16_f16_s32(const LtxDq16Args a) {
    dq16_body<_Float16, true>(a);
}
extern "C" __global__ void __launch_bounds__(256) ltx_gemm_dq16_bf16(const LtxDq16Args a) { dq16_body<__bf16, false>(a); }
extern "C" __global__ void __launch_bounds__(256) ltx_gemm_dq16_bf16_s32(const LtxDq16Args a) {
    dq16_body<__bf16, true>(a);
}

// Gate logits (ltx/block.zig:238, 526, 564): glog[t][h] = a[t] . gw[h] + gb[h].
// One wave per 32 token rows: 256 MFMAs over K = 4096, operands straight
// from global memory (the 32 x 4096 weight stays L2-resident).
template <typename T>
__device__ void gate_body(const LtxGateArgs& a) {
    typedef typename Op<T>::v8 v8;
    const int lane = threadIdx.x & 63;
    const int m0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 32;
    if (m0 >= a.M) return;
    const int fr = lane & 31, fk = 8 * (lane >> 5);
    const uint16_t* pa = (const uint16_t*)a.a + (size_t)min(m0 + fr, a.M - 1) * LTX_D + fk;
    const uint16_t* pb = (const uint16_t*)a.gw + (size_t)fr * LTX_D + fk;
    f32x16 acc = f32x16{0};
#pragma unroll 8
    for (int k = 0; k < LTX_D; k += 16) {
        v8 fa = __builtin_bit_cast(v8, *(const u32x4*)(pa + k));
        v8 fb = __builtin_bit_cast(v8, *(const u32x4*)(pb + k));
        acc = Op<T>::mfma32(fa, fb, acc);
    }
    const float bias = a.gb[fr];
#pragma unroll
    for (int r = 0; r < 16; r++) {
        int m = m0 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m < a.M) a.out[(size_t)m * LTX_H + fr] = acc[r] + bias;
    }
}

extern "C" __global__ void __launch_bounds__(256) ltx_gate_f16(const LtxGateArgs a) { gate_body<_Float16>(a); }
extern "C" __global__ void __launch_bounds__(256) ltx_gate_bf16(const LtxGateArgs a) { gate_body<__bf16>(a); }

// The same logits for few rows: one workgroup per 32 rows, wave q sums
// k in [1024 q, 1024 q + 1024) over two alternating accumulators (two
// independent MFMA chains), and wave 0 adds the four partial sums in wave
// order through LDS.
template <typename T>
__device__ void gate_ks_body(const LtxGateArgs& a) {
    typedef typename Op<T>::v8 v8;
    __shared__ f32x16 red[3][64];
    const int lane = threadIdx.x & 63, q = threadIdx.x >> 6;
    const int m0 = blockIdx.x * 32;
    const int fr = lane & 31, fk = 8 * (lane >> 5) + q * (LTX_D / 4);
    const uint16_t* pa = (const uint16_t*)a.a + (size_t)min(m0 + fr, a.M - 1) * LTX_D + fk;
    const uint16_t* pb = (const uint16_t*)a.gw + (size_t)fr * LTX_D + fk;
    f32x16 acc0 = f32x16{0}, acc1 = f32x16{0};
#pragma unroll 8
    for (int k = 0; k < LTX_D / 4; k += 32) {
        acc0 = Op<T>::mfma32(__builtin_bit_cast(v8, *(const u32x4*)(pa + k)),
                             __builtin_bit_cast(v8, *(const u32x4*)(pb + k)), acc0);
        acc1 = Op<T>::mfma32(__builtin_bit_cast(v8, *(const u32x4*)(pa + k + 16)),
                             __builtin_bit_cast(v8, *(const u32x4*)(pb + k + 16)), acc1);
    }
    const f32x16 acc = acc0 + acc1;
    if (q > 0) red[q - 1][lane] = acc;
    __syncthreads();
    if (q > 0) return;
    const f32x16 sum = ((acc + red[0][lane]) + red[1][lane]) + red[2][lane];
    const float bias = a.gb[fr];
#pragma unroll
    for (int r = 0; r < 16; r++) {
        int m = m0 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m < a.M) a.out[(size_t)m * LTX_H + fr] = sum[r] + bias;
    }
}

extern "C" __global__ void __launch_bounds__(256) ltx_gate_ks_f16(const LtxGateArgs a) { gate_ks_body<_Float16>(a); }
extern "C" __global__ void __launch_bounds__(256) ltx_gate_ks_bf16(const LtxGateArgs a) { gate_ks_body<__bf16>(a); }

// Split-K completion: v = sum over s = 0 .. S-1 of part[s][m][n] (in that
// order) + bias[n], then the GEMM's epilogue. A workgroup of 256 threads owns
// a 64 x 64 block: thread t row t / 4, columns 16 (t % 4) .. + 15 (four
// threads read a row's 256 contiguous bytes). V^T blocks of the QKV split
// are transposed through LDS so that their rows (64 tokens) store whole.
template <typename T, int EPI>
__device__ void reduce_body(const LtxGemmArgs& a) {
    __shared__ uint16_t tr[64][64 + 8];
    const int t = threadIdx.x, r = t >> 2, cq = 16 * (t & 3);
    const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    const int m = m0 + r, n = n0 + cq;
    const bool row_ok = m < a.M;
    const size_t MN = (size_t)a.M * a.N;
    float v[16];
#pragma unroll
    for (int e = 0; e < 16; e++) v[e] = 0.0f;
    if (row_ok) {
        for (int s = 0; s < a.ksplit; s++) {
            const float* p = a.part + s * MN + (size_t)m * a.N + n;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const f32x4 x = *(const f32x4*)(p + 4 * c);
#pragma unroll
                for (int e = 0; e < 4; e++) v[4 * c + e] += x[e];
            }
        }
        if (a.bias) {
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const f32x4 b = *(const f32x4*)(a.bias + n + 4 * c);
#pragma unroll
                for (int e = 0; e < 4; e++) v[4 * c + e] += b[e];
            }
        }
    }
    unsigned bad = 0;  // 16-bit stores out of range (range guard)
    if (EPI == LTX_EPI_RESID_GATE) {
        if (row_ok) {
            const float* gt = a.ada.tstab + ((size_t)ada_row(a.ada, m) * 9 + a.igate) * LTX_D + n;
            const float* gs = a.ada.sst + (size_t)a.igate * LTX_D + n;
            const float* rs = a.resid + (size_t)m * a.ldo + n;
            float* o = (float*)a.out + (size_t)m * a.ldo + n;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const f32x4 x = *(const f32x4*)(rs + 4 * c), g0 = *(const f32x4*)(gt + 4 * c),
                            g1 = *(const f32x4*)(gs + 4 * c);
                f32x4 y;
#pragma unroll
                for (int e = 0; e < 4; e++) y[e] = x[e] + v[4 * c + e] * (g0[e] + g1[e]);
                *(f32x4*)(o + 4 * c) = y;
            }
        }
    } else if (EPI == LTX_EPI_QKV && n0 >= a.nsplit) {
        // V^T [c][m], c = n - nsplit: through LDS, then 64-token rows
#pragma unroll
        for (int e = 0; e < 16; e++) tr[cq + e][r] = Op<T>::bits(v[e]);
        if (row_ok)
#pragma unroll
            for (int e = 0; e < 16; e++) bad += out_of_range<T>(v[e]);
        __syncthreads();
        const int c = n0 - a.nsplit + r, mm = m0 + cq;  // row r of the transposed block, tokens cq ..
        uint16_t* dst = (uint16_t*)a.out2 + (size_t)c * a.M + mm;
        if (mm + 16 <= a.M && (a.M & 7) == 0) {
            const u32x4* src = (const u32x4*)&tr[r][cq];
            *(u32x4*)dst = src[0];
            *(u32x4*)(dst + 8) = src[1];
        } else {
            for (int e = 0; e < 16; e++)
                if (mm + e < a.M) dst[e] = tr[r][cq + e];
        }
    } else if (row_ok) {  // STORE, or the q | k rows of the QKV split
        const bool gelu = EPI == LTX_EPI_STORE && a.gelu;
        if (gelu)
#pragma unroll
            for (int e = 0; e < 16; e++) v[e] = gelu_tanh(v[e]);
        if (EPI == LTX_EPI_STORE && a.out_f32) {
            float* o = (float*)a.out + (size_t)m * a.ldo + n;
#pragma unroll
            for (int c = 0; c < 4; c++) *(f32x4*)(o + 4 * c) = f32x4{v[4 * c], v[4 * c + 1], v[4 * c + 2], v[4 * c + 3]};
        } else {
            const int ld = EPI == LTX_EPI_QKV ? a.nsplit : a.ldo;
            uint16_t* o = (uint16_t*)a.out + (size_t)m * ld + n;
#pragma unroll
            for (int c = 0; c < 2; c++)
                *(u32x4*)(o + 8 * c) = u32x4{pack2<T>(v[8 * c], v[8 * c + 1]), pack2<T>(v[8 * c + 2], v[8 * c + 3]),
                                             pack2<T>(v[8 * c + 4], v[8 * c + 5]), pack2<T>(v[8 * c + 6], v[8 * c + 7])};
#pragma unroll
            for (int e = 0; e < 16; e++) bad += out_of_range<T>(v[e]);
        }
    }
    range_report(a.sat, bad);
}

#define REDUCE_KERNEL(NAME, T, EPI_) \
    extern "C" __global__ void __launch_bounds__(256) NAME(const LtxGemmArgs a) { reduce_body<T, EPI_>(a); }

REDUCE_KERNEL(ltx_gemm_reduce_f16_store, _Float16, LTX_EPI_STORE)
REDUCE_KERNEL(ltx_gemm_reduce_f16_resid, _Float16, LTX_EPI_RESID_GATE)
REDUCE_KERNEL(ltx_gemm_reduce_f16_qkv, _Float16, LTX_EPI_QKV)
REDUCE_KERNEL(ltx_gemm_reduce_bf16_store, __bf16, LTX_EPI_STORE)
REDUCE_KERNEL(ltx_gemm_reduce_bf16_resid, __bf16, LTX_EPI_RESID_GATE)
REDUCE_KERNEL(ltx_gemm_reduce_bf16_qkv, __bf16, LTX_EPI_QKV)
