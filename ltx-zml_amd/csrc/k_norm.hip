// Bandwidth-bound kernels: fused RMSNorm + AdaLN modulate, the cross-attention
// K/V modulation, and the full-row qk RMSNorm + split-half 3D RoPE.
// 256-thread workgroups over token rows of D = 4096 channels.
#include "ltx_device.h"

// RMSNorm + modulate (ltx/block.zig:28-30, 36-38, 248-252, 548-552, 569-572):
// y = x * rsqrt(mean(x^2) + 1e-6) * (1 + ada[isc]) + ada[ish].
// Each thread owns 4 float4 columns c = 4*tid + 1024*i. A workgroup takes
// NORM_ROWS consecutive rows; when their timestep rows agree (the usual case:
// runs of tokens share one), the scale and shift rows (tstab + sst) are
// formed once for all of them, which quarters their L2 reads (64 KB per row
// otherwise, four times the row's own bytes).
#define NORM_ROWS 4
template <int OUT>  // 0: f16, 1: bf16, 2: f32
__device__ void norm_mod_body(const LtxNormArgs& a) {
    __shared__ float red[4];
    const int row0 = blockIdx.x * NORM_ROWS;
    if (row0 >= a.rows) return;
    const int nr = min(NORM_ROWS, a.rows - row0);
    const bool mod = a.isc >= 0;
    bool shared_mod = mod;
    if (mod) {
        const int r0 = ada_row(a.ada, row0);
        for (int k = 1; k < nr; k++) shared_mod = shared_mod && ada_row(a.ada, row0 + k) == r0;
    }
    float4 sc1[4], sh[4];  // 1 + scale, shift
    auto load_mod = [&](int r) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = 4 * (threadIdx.x + 256 * i);
            const float4 sct = *(const float4*)(a.ada.tstab + ((size_t)r * 9 + a.isc) * LTX_D + c);
            const float4 scs = *(const float4*)(a.ada.sst + (size_t)a.isc * LTX_D + c);
            const float4 sht = *(const float4*)(a.ada.tstab + ((size_t)r * 9 + a.ish) * LTX_D + c);
            const float4 shs = *(const float4*)(a.ada.sst + (size_t)a.ish * LTX_D + c);
            sc1[i] = make_float4((sct.x + scs.x) + 1.0f, (sct.y + scs.y) + 1.0f, (sct.z + scs.z) + 1.0f,
                                 (sct.w + scs.w) + 1.0f);
            sh[i] = make_float4(sht.x + shs.x, sht.y + shs.y, sht.z + shs.z, sht.w + shs.w);
        }
    };
    if (shared_mod) load_mod(ada_row(a.ada, row0));
    unsigned bad = 0;  // 16-bit stores out of range (range guard)
    if (a.sat_add && blockIdx.x == 0 && threadIdx.x == 0 && a.sat) atomicAdd(a.sat, *a.sat_add);
    for (int k = 0; k < nr; k++) {
        const int row = row0 + k;
        const float4* x = (const float4*)(a.x + (size_t)row * LTX_D);
        float4 v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = x[threadIdx.x + 256 * i];
        // rows with their own timestep row: its modulation rows load before
        // the reduction so their latency overlaps it
        if (mod && !shared_mod) load_mod(ada_row(a.ada, row));
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
        ss = block_sum256(ss, red);
        const float inv = 1.0f / sqrtf(ss * (1.0f / LTX_D) + 1e-6f);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = 4 * (threadIdx.x + 256 * i);
            float o[4] = {v[i].x * inv, v[i].y * inv, v[i].z * inv, v[i].w * inv};
            if (mod) {
                const float s1[4] = {sc1[i].x, sc1[i].y, sc1[i].z, sc1[i].w}, s0[4] = {sh[i].x, sh[i].y, sh[i].z, sh[i].w};
#pragma unroll
                for (int j = 0; j < 4; j++) o[j] = o[j] * s1[j] + s0[j];
            }
            const size_t off = (size_t)row * LTX_D + c;
            if (OUT == 2) {
                *(float4*)((float*)a.y + off) = make_float4(o[0], o[1], o[2], o[3]);
            } else if (OUT == 0) {
                u32x2 p = {pack2<_Float16>(o[0], o[1]), pack2<_Float16>(o[2], o[3])};
                *(u32x2*)((uint16_t*)a.y + off) = p;
#pragma unroll
                for (int j = 0; j < 4; j++) bad += out_of_range<_Float16>(o[j]);
            } else {
                u32x2 p = {pack2<__bf16>(o[0], o[1]), pack2<__bf16>(o[2], o[3])};
                *(u32x2*)((uint16_t*)a.y + off) = p;
#pragma unroll
                for (int j = 0; j < 4; j++) bad += out_of_range<__bf16>(o[j]);
            }
        }
    }
    range_report(a.sat, bad);
}

extern "C" __global__ void __launch_bounds__(256) ltx_norm_mod_f16(const LtxNormArgs a) { norm_mod_body<0>(a); }
extern "C" __global__ void __launch_bounds__(256) ltx_norm_mod_bf16(const LtxNormArgs a) { norm_mod_body<1>(a); }
extern "C" __global__ void __launch_bounds__(256) ltx_norm_mod_f32(const LtxNormArgs a) { norm_mod_body<2>(a); }

// enc = ctx * (1 + (psst[1] + pts2[1])) + (psst[0] + pts2[0])  (ltx/block.zig:553-556)
template <int OUT>
__device__ void enc_body(const LtxEncArgs& a) {
    int row = blockIdx.x;
    if (row >= a.rows) return;
    unsigned bad = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        int c = 4 * (threadIdx.x + 256 * i);
        float4 x = *(const float4*)(a.ctx + (size_t)row * LTX_D + c);
        float4 s0 = *(const float4*)(a.psst + c), s1 = *(const float4*)(a.psst + LTX_D + c);
        float4 p0 = *(const float4*)(a.pts2 + c), p1 = *(const float4*)(a.pts2 + LTX_D + c);
        float o[4] = {x.x * ((s1.x + p1.x) + 1.0f) + (s0.x + p0.x), x.y * ((s1.y + p1.y) + 1.0f) + (s0.y + p0.y),
                      x.z * ((s1.z + p1.z) + 1.0f) + (s0.z + p0.z), x.w * ((s1.w + p1.w) + 1.0f) + (s0.w + p0.w)};
        size_t off = (size_t)row * LTX_D + c;
        if (OUT == 2) {
            *(float4*)((float*)a.y + off) = make_float4(o[0], o[1], o[2], o[3]);
        } else if (OUT == 0) {
            u32x2 p = {pack2<_Float16>(o[0], o[1]), pack2<_Float16>(o[2], o[3])};
            *(u32x2*)((uint16_t*)a.y + off) = p;
#pragma unroll
            for (int j = 0; j < 4; j++) bad += out_of_range<_Float16>(o[j]);
        } else {
            u32x2 p = {pack2<__bf16>(o[0], o[1]), pack2<__bf16>(o[2], o[3])};
            *(u32x2*)((uint16_t*)a.y + off) = p;
#pragma unroll
            for (int j = 0; j < 4; j++) bad += out_of_range<__bf16>(o[j]);
        }
    }
    range_report(a.sat, bad);
}

extern "C" __global__ void __launch_bounds__(256) ltx_enc_f16(const LtxEncArgs a) { enc_body<0>(a); }
extern "C" __global__ void __launch_bounds__(256) ltx_enc_bf16(const LtxEncArgs a) { enc_body<1>(a); }
extern "C" __global__ void __launch_bounds__(256) ltx_enc_f32(const LtxEncArgs a) { enc_body<2>(a); }

// 8 consecutive 16-bit values (one 16-byte load) widened to f32 (exact).
template <typename T>
__device__ __forceinline__ void load8(const uint16_t* p, float* out) {
    const u32x4 v = *(const u32x4*)p;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        out[2 * i] = Op<T>::to_f32((uint16_t)(v[i] & 0xffffu));
        out[2 * i + 1] = Op<T>::to_f32((uint16_t)(v[i] >> 16));
    }
}

// qk norm + RoPE (ltx/block.zig:32-34, 69-77, 214-226): y = rope(rms(x) * w).
// Thread t owns head h = t / 8 and rotary slots f0 = 8 * (t % 8) .. f0 + 8, so
// each RoPE pair (f, f + 64) lives in one thread. Output rows [rows][D]: each
// token's 8 KB leaves as one contiguous row (head-major [H][rows][HD] wrote
// 256-byte pieces 32 rows apart and ran at 4.2 TB/s).
template <typename T>
__device__ void qknorm_body(const LtxQkNormArgs& a) {
    __shared__ float red[4];
    // a contiguous range of tokens per XCD, as in qknorm2_body
    const int row = (gridDim.x & 7) == 0 ? (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3) : blockIdx.x;
    if (row >= a.rows) return;
    int h = threadIdx.x >> 3, f0 = (threadIdx.x & 7) * 8;
    const uint16_t* xr = (const uint16_t*)a.x + (size_t)row * a.ldx + h * LTX_HD;
    float lo[8], hi[8];
    float ss = 0.f;
    load8<T>(xr + f0, lo);
    load8<T>(xr + 64 + f0, hi);
    // norm weights and RoPE rows do not depend on the row statistics: loaded
    // before the reduction so their latency overlaps it
    const float* wl = a.w + h * LTX_HD + f0;
    float wlo[8], whi[8], cs[8], sn[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        wlo[j] = wl[j];
        whi[j] = wl[64 + j];
    }
    if (a.cos) {
        const float* cr = a.cos + ((size_t)row * LTX_H + h) * 64 + f0;
        const float* sr = a.sin + ((size_t)row * LTX_H + h) * 64 + f0;
#pragma unroll
        for (int j = 0; j < 8; j += 4) {
            *(float4*)(cs + j) = *(const float4*)(cr + j);
            *(float4*)(sn + j) = *(const float4*)(sr + j);
        }
    }
#pragma unroll
    for (int j = 0; j < 8; j++) ss += lo[j] * lo[j] + hi[j] * hi[j];
    ss = block_sum256(ss, red);
    float inv = 1.0f / sqrtf(ss * (1.0f / LTX_D) + 1e-6f);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        lo[j] = lo[j] * inv * wlo[j];
        hi[j] = hi[j] * inv * whi[j];
    }
    if (a.cos) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            float c = cs[j], s = sn[j], x0 = lo[j], x1 = hi[j];
            lo[j] = x0 * c - x1 * s;
            hi[j] = x1 * c + x0 * s;
        }
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
        lo[j] *= a.oscale;
        hi[j] *= a.oscale;
    }
    uint16_t* y = (uint16_t*)a.y + (size_t)row * LTX_D + h * LTX_HD;
    u32x4 plo = {pack2<T>(lo[0], lo[1]), pack2<T>(lo[2], lo[3]), pack2<T>(lo[4], lo[5]), pack2<T>(lo[6], lo[7])};
    u32x4 phi = {pack2<T>(hi[0], hi[1]), pack2<T>(hi[2], hi[3]), pack2<T>(hi[4], hi[5]), pack2<T>(hi[6], hi[7])};
    *(u32x4*)(y + f0) = plo;
    *(u32x4*)(y + 64 + f0) = phi;
    unsigned bad = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) bad += out_of_range<T>(lo[j]) + out_of_range<T>(hi[j]);
    range_report(a.sat, bad);
}

// q and k of one token together (same thread layout as qknorm_body), the
// cos / sin rows loaded once for both.
template <typename T>
__device__ void qknorm2_body(const LtxQkNorm2Args& a) {
    __shared__ float red[8];
    // workgroups go round-robin to the 8 XCDs: give each XCD a contiguous
    // range of tokens, so that its L2 sees whole runs of consecutive rows of
    // every head-major output (measured: qknorm2 -1.5 %, and the gate logits
    // beside it on the side stream 0.245 -> 0.170 ms)
    const int row = (gridDim.x & 7) == 0 ? (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3) : blockIdx.x;
    if (row >= a.rows) return;
    const int h = threadIdx.x >> 3, f0 = (threadIdx.x & 7) * 8;
    float lo[2][8], hi[2][8], cs[8], sn[8], wlo[2][8], whi[2][8];
#pragma unroll
    for (int p = 0; p < 2; p++) {
        const uint16_t* xr = (const uint16_t*)a.x + (size_t)row * a.ldx + p * LTX_D + h * LTX_HD;
        load8<T>(xr + f0, lo[p]);
        load8<T>(xr + 64 + f0, hi[p]);
        const float* wl = (p ? a.wk : a.wq) + h * LTX_HD + f0;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            wlo[p][j] = wl[j];
            whi[p][j] = wl[64 + j];
        }
    }
    const float* cr = a.cos + ((size_t)row * LTX_H + h) * 64 + f0;
    const float* sr = a.sin + ((size_t)row * LTX_H + h) * 64 + f0;
#pragma unroll
    for (int j = 0; j < 8; j += 4) {
        *(float4*)(cs + j) = *(const float4*)(cr + j);
        *(float4*)(sn + j) = *(const float4*)(sr + j);
    }
    float ss[2] = {0.f, 0.f};
#pragma unroll
    for (int p = 0; p < 2; p++)
#pragma unroll
        for (int j = 0; j < 8; j++) ss[p] += lo[p][j] * lo[p][j] + hi[p][j] * hi[p][j];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        ss[0] += __shfl_xor(ss[0], o, 64);
        ss[1] += __shfl_xor(ss[1], o, 64);
    }
    const int wv = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        red[wv] = ss[0];
        red[4 + wv] = ss[1];
    }
    __syncthreads();
#pragma unroll
    for (int p = 0; p < 2; p++) {
        const float tot = red[4 * p] + red[4 * p + 1] + red[4 * p + 2] + red[4 * p + 3];
        const float inv = 1.0f / sqrtf(tot * (1.0f / LTX_D) + 1e-6f);
        const float osc = p ? a.oscale_k : a.oscale_q;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float x0 = lo[p][j] * inv * wlo[p][j], x1 = hi[p][j] * inv * whi[p][j];
            lo[p][j] = (x0 * cs[j] - x1 * sn[j]) * osc;
            hi[p][j] = (x1 * cs[j] + x0 * sn[j]) * osc;
        }
        uint16_t* y = (uint16_t*)(p ? a.yk : a.yq) + (size_t)row * LTX_D + h * LTX_HD;
        const float* l = lo[p];
        const float* u = hi[p];
        *(u32x4*)(y + f0) = u32x4{pack2<T>(l[0], l[1]), pack2<T>(l[2], l[3]), pack2<T>(l[4], l[5]), pack2<T>(l[6], l[7])};
        *(u32x4*)(y + 64 + f0) =
            u32x4{pack2<T>(u[0], u[1]), pack2<T>(u[2], u[3]), pack2<T>(u[4], u[5]), pack2<T>(u[6], u[7])};
    }
    unsigned bad = 0;
#pragma unroll
    for (int p = 0; p < 2; p++)
#pragma unroll
        for (int j = 0; j < 8; j++) bad += out_of_range<T>(lo[p][j]) + out_of_range<T>(hi[p][j]);
    range_report(a.sat, bad);
}

extern "C" __global__ void __launch_bounds__(256) ltx_qknorm2_f16(const LtxQkNorm2Args a) { qknorm2_body<_Float16>(a); }
extern "C" __global__ void __launch_bounds__(256) ltx_qknorm2_bf16(const LtxQkNorm2Args a) { qknorm2_body<__bf16>(a); }

extern "C" __global__ void __launch_bounds__(256) ltx_qknorm_f16(const LtxQkNormArgs a) { qknorm_body<_Float16>(a); }
extern "C" __global__ void __launch_bounds__(256) ltx_qknorm_bf16(const LtxQkNormArgs a) { qknorm_body<__bf16>(a); }

// f32 mode: in place on [rows][ldx] f32, merged-head layout kept.
extern "C" __global__ void __launch_bounds__(256) ltx_qknorm_f32(const LtxQkNorm32Args a) {
    __shared__ float red[4];
    int row = blockIdx.x;
    if (row >= a.rows) return;
    int h = threadIdx.x >> 3, f0 = (threadIdx.x & 7) * 8;
    float* xr = a.x + (size_t)row * a.ldx + h * LTX_HD;
    float lo[8], hi[8];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        lo[j] = xr[f0 + j];
        hi[j] = xr[64 + f0 + j];
        ss += lo[j] * lo[j] + hi[j] * hi[j];
    }
    ss = block_sum256(ss, red);
    float inv = 1.0f / sqrtf(ss * (1.0f / LTX_D) + 1e-6f);
    const float* wl = a.w + h * LTX_HD + f0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        lo[j] = lo[j] * inv * wl[j];
        hi[j] = hi[j] * inv * wl[64 + j];
    }
    if (a.cos) {
        const float* cr = a.cos + ((size_t)row * LTX_H + h) * 64 + f0;
        const float* sr = a.sin + ((size_t)row * LTX_H + h) * 64 + f0;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            float c = cr[j], s = sr[j], x0 = lo[j], x1 = hi[j];
            lo[j] = x0 * c - x1 * s;
            hi[j] = x1 * c + x0 * s;
        }
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
        xr[f0 + j] = lo[j];
        xr[64 + f0 + j] = hi[j];
    }
}

// Dequantisation probe: the exact f32 value q * s (one rounding, as dq4 at
// ltx/block.zig:462-471) and the 16-bit operand the GEMM feeds the MFMA.
// Same arithmetic as the GEMM's staging path: fma(u, s, -128 s) with
// u = q + 128 read as an unsigned byte, which equals round(q * s).
// Each thread handles a pair of adjacent elements (K is a multiple of 128).
template <typename T>
__device__ void dequant_body(const LtxDequantArgs& a) {
    size_t i = 2 * ((size_t)blockIdx.x * blockDim.x + threadIdx.x);
    size_t n = (size_t)a.N * a.K;
    if (i >= n) return;
    int row = (int)(i / a.K), k = (int)(i % a.K);
    size_t si = (size_t)row * (a.K / LTX_GROUP) + k / LTX_GROUP;
    float s = a.scale_f16 ? f16_bits_to_f32(((const uint16_t*)a.scales)[si]) : ((const float*)a.scales)[si];
    float nb = -128.0f * s;
    float u0 = (float)(uint8_t)((uint8_t)a.q[i] ^ 0x80u);
    float u1 = (float)(uint8_t)((uint8_t)a.q[i + 1] ^ 0x80u);
    a.out32[i] = __builtin_fmaf(u0, s, nb);
    a.out32[i + 1] = __builtin_fmaf(u1, s, nb);
    *(uint32_t*)((uint16_t*)a.out16 + i) = deq_pack2<T>(u0, u1, s, nb);
}

extern "C" __global__ void __launch_bounds__(256) ltx_dequant_f16(const LtxDequantArgs a) { dequant_body<_Float16>(a); }
extern "C" __global__ void __launch_bounds__(256) ltx_dequant_bf16(const LtxDequantArgs a) { dequant_body<__bf16>(a); }

// Scale pairs for the LDS-DMA int8 GEMM: out[g][n] = s[n][g] in both halves.
extern "C" __global__ void __launch_bounds__(256) ltx_cvt_bf16(const LtxCvtArgs a) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= a.n) return;
    const float v = __builtin_bit_cast(float, (uint32_t)a.in[i] << 16);
    if (a.to_f16) {
        const _Float16 h = (_Float16)v;
        ((_Float16*)a.out)[i] = h;
        range_report(a.over, __builtin_isfinite((float)h) ? 0u : 1u);
    } else {
        ((float*)a.out)[i] = v;
    }
}

extern "C" __global__ void __launch_bounds__(256) ltx_q8_flip(const LtxFlipArgs a) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < a.n) a.out[i] = a.in[i] ^ 0x80808080u;
}

extern "C" __global__ void __launch_bounds__(256) ltx_scale_pairs(const LtxPairArgs a) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= a.N * a.G) return;
    const int g = i / a.N, n = i - g * a.N;
    const size_t j = (size_t)n * a.G + g;
    a.out[i] = a.f32 ? ((const uint32_t*)a.s)[j] : (uint32_t)((const uint16_t*)a.s)[j] * 0x10001u;
}
