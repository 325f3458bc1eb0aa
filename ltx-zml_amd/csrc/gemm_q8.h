// W8A16 GEMM for gfx950 with LDS-DMA staging: y[M][N] = A[M][K] . W[N][K]^T,
// A f16 (or bf16) activations, W int8 with one f16 (or f32) scale per 128
// consecutive k (ltx/block.zig:462-471), fused epilogues as in gemm_common.h.
// The scales arrive as words: a.scales is u32 [K / 128][N], each word an f16
// scale in both halves or an f32 scale's bits (laid out once at upload).
//
// Workgroup: 8 waves (two per SIMD), output tile 256 x 256; wave w owns rows
// 128 (w / 4) .. +127 and columns 64 (w % 4) .. +63 (4 x 2 blocks of 32 x 32,
// v_mfma_f32_32x32x16_f16 or _bf16, f32 accumulate).
//
// K is walked in tiles of 64. Each tile's A (256 x 64 f16, 32 KB) and W
// (256 x 64 int8, 16 KB) go straight from global memory into LDS with
// global_load_lds_dwordx4 (no register staging) into one of three stages, two
// tiles ahead of the tile being multiplied. The weight tile stays int8 in LDS:
// every wave dequantises the fragments it reads (half the LDS bytes of an f16
// tile, no second LDS pass).
//
// Dequantisation is exact. The weight bytes are stored as u = q + 128 (q XOR
// 0x80, done once at upload); the operand is the one the register-staged
// kernels and the dequant probe produce: for f16, q * s rounded once to
// nearest even; for bf16, the f32 value f32(q) * s (the reference's
// dequantised weight) rounded to nearest even. Per operand and scale type:
// - f16, f16 scales: the f16 with bits 0x6400 | u is 1024 + u; subtracting
//   1152 gives q exactly, one v_pk_mul_f16 by the scale rounds q * s once
//   (v_perm, v_pk_add_f16, v_pk_mul_f16: 3 VALU instructions per MFMA).
// - f16, f32 scales: the f16 with bits u is the subnormal u 2^-24;
//   v_fma_mixlo/hi_f16 reads it and rounds fma(u 2^-24, s 2^24, -128 s) =
//   q * s once (3 per MFMA; s 2^24 is finite for |s| < 2^104, and above
//   65504 / 128 every nonzero q * s is beyond the f16 range anyway).
// - bf16, f16 scales: the same subnormal read by v_fma_mix_f32 gives q * s
//   in f32 (exact: at most 19 significant bits), one v_cvt_pk_bf16_f32
//   rounds a pair (4 per MFMA).
// - bf16, f32 scales: v_cvt_f32_ubyteN and v_fma_f32 (u, s, -128 s) give
//   f32(q) * s, then v_cvt_pk_bf16_f32 (5 per MFMA). -128 s is finite for
//   |s| < 2^120; uploads refuse f32 scales of magnitude 2^100 or more.
//
// LDS layout: A rows of 128 B (8 chunks of 8 k), chunk c of row r stored in
// slot c ^ ((r >> 1) & 7) (16 consecutive rows, one ds_read_b128 lane group,
// then cover all 64 banks once); W rows of 64 B (4 chunks of 16 k), chunk c of row n in
// slot c ^ ((n >> 2) & 3). The DMA writes 64 consecutive 16-byte slots per
// instruction; each lane picks the global chunk that belongs in its slot.
//
// k order inside a tile: for MFMA step t (0..3), lanes 0-31 multiply
// k = 8 t + 0..7 and lanes 32-63 k = 32 + 8 t + 0..7 (A and W alike), so a
// lane's A operands for the whole tile are 64 contiguous bytes of its row and
// its W operands 32 contiguous bytes.
//
// Synchronisation: waits are explicit (s_waitcnt vmcnt for this wave's DMA,
// lgkmcnt for its LDS reads) followed by s_barrier. Each stage is its own
// __shared__ object, so the compiler's alias tracking of LDS DMA sees that a
// read of one stage does not depend on DMA into another and adds no
// vmcnt(0) of its own. The two waves of a SIMD run half a tile
// apart: while one multiplies, the other reads fragments, dequantises and
// issues DMA.
#pragma once
#include "gemm_common.h"

typedef __attribute__((address_space(3))) void* lds_vptr;

// s_waitcnt immediates (vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
#define Q8_WAIT_VM(n) ((((n) & 15) | (((n) >> 4) << 14)) | (7 << 4) | (15 << 8))
#define Q8_WAIT_LGKM0 (15 | (3 << 14) | (7 << 4))

__shared__ __attribute__((aligned(1024))) uint8_t q8_sa0[32768];
__shared__ __attribute__((aligned(1024))) uint8_t q8_sa1[32768];
__shared__ __attribute__((aligned(1024))) uint8_t q8_sa2[32768];
__shared__ __attribute__((aligned(1024))) uint8_t q8_sb0[16384];
__shared__ __attribute__((aligned(1024))) uint8_t q8_sb1[16384];
__shared__ __attribute__((aligned(1024))) uint8_t q8_sb2[16384];

template <int S>
__device__ __forceinline__ uint8_t* q8_stage_a() {
    return S == 0 ? q8_sa0 : S == 1 ? q8_sa1 : q8_sa2;
}
template <int S>
__device__ __forceinline__ uint8_t* q8_stage_b() {
    return S == 0 ? q8_sb0 : S == 1 ? q8_sb1 : q8_sb2;
}

// 8 weights (two dwords of an LDS chunk, bytes q + 128) -> one f16x8
// operand, times the scale pair s2.
__device__ __forceinline__ f16x8 q8_dequant8(uint32_t w0, uint32_t w1, f16x2 s2) {
    const f16x2 off = {(_Float16)1152.0f, (_Float16)1152.0f};
    uint32_t o[4];
#pragma unroll
    for (int d = 0; d < 2; d++) {
        const uint32_t x = d ? w1 : w0;
        const f16x2 p0 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u));
        const f16x2 p1 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u));
        o[2 * d] = __builtin_bit_cast(uint32_t, (p0 - off) * s2);
        o[2 * d + 1] = __builtin_bit_cast(uint32_t, (p1 - off) * s2);
    }
    return __builtin_bit_cast(f16x8, u32x4{o[0], o[1], o[2], o[3]});
}

// The operand type's and scale type's part of the kernel: the scale form a
// lane keeps for one column (from its scale word), the dequantisation of 8
// weights and the MFMA.
template <typename T, bool SF32>
struct Q8Op;

template <typename T>
struct Q8Mfma;
template <>
struct Q8Mfma<_Float16> {
    typedef f16x8 V8;
    static __device__ __forceinline__ f32x16 mfma(u32x4 a, V8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), b, c, 0, 0, 0);
    }
};
template <>
struct Q8Mfma<__bf16> {
    typedef bf16x8 V8;
    static __device__ __forceinline__ f32x16 mfma(u32x4 a, V8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), b, c, 0, 0, 0);
    }
};

struct Q8ScaleF32 {
    float s, c;  // the scale and -128 times it (exact: a power of two)
};

// 8 weights to bf16 through f32: fma(u, s, -128 s) = f32(q * s), then one
// v_cvt_pk_bf16_f32 per pair.
__device__ __forceinline__ bf16x8 q8_dequant8_bf16_f32(uint32_t w0, uint32_t w1, Q8ScaleF32 s) {
    uint32_t o[4];
#pragma unroll
    for (int d = 0; d < 2; d++) {
        const uint32_t x = d ? w1 : w0;
        o[2 * d] = Op<__bf16>::cvt2(__builtin_fmaf((float)(x & 0xffu), s.s, s.c),
                                    __builtin_fmaf((float)((x >> 8) & 0xffu), s.s, s.c));
        o[2 * d + 1] = Op<__bf16>::cvt2(__builtin_fmaf((float)((x >> 16) & 0xffu), s.s, s.c),
                                        __builtin_fmaf((float)(x >> 24), s.s, s.c));
    }
    return __builtin_bit_cast(bf16x8, u32x4{o[0], o[1], o[2], o[3]});
}

// bf16 operands, f32 scales: through f32 without a prescaled form, since
// q * s may reach far beyond the f16 range (|s| < 2^100, as uploads require)
template <>
struct Q8Op<__bf16, true> : Q8Mfma<__bf16> {
    typedef Q8ScaleF32 Scale;
    static __device__ __forceinline__ Scale scale(uint32_t word) {
        const float s = __builtin_bit_cast(float, word);
        return Scale{s, -128.0f * s};
    }
    static __device__ __forceinline__ V8 deq8(uint32_t w0, uint32_t w1, Scale s) {
        return q8_dequant8_bf16_f32(w0, w1, s);
    }
};

// f16 operands, f32 scales: each byte u enters as the f16 subnormal u 2^-24
// (one v_perm per pair, exact), and fma(u 2^-24, s 2^24, -128 s) = q s is
// rounded once to f16 by v_fma_mix reading that f16 directly: the rounding
// of the exact q * s that the register-staged kernels make, in 3 VALU
// instructions per MFMA. s 2^24 is finite for |s| < 2^104; above
// 65504 / 128 every nonzero q * s is beyond the f16 range anyway.
template <>
struct Q8Op<_Float16, true> : Q8Mfma<_Float16> {
    typedef Q8ScaleF32 Scale;  // s 2^24 and -128 s
    static __device__ __forceinline__ Scale scale(uint32_t word) {
        const float s = __builtin_bit_cast(float, word);
        return Scale{s * 16777216.0f, -128.0f * s};
    }
    static __device__ __forceinline__ V8 deq8(uint32_t w0, uint32_t w1, Scale s) {
        uint32_t o[4];
#pragma unroll
        for (int d = 0; d < 2; d++) {
            const uint32_t x = d ? w1 : w0;
            const f16x2 p0 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0u, x, 0x04010400u));
            const f16x2 p1 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0u, x, 0x04030402u));
            const f16x2 r0 = {(_Float16)__builtin_fmaf((float)p0[0], s.s, s.c),
                              (_Float16)__builtin_fmaf((float)p0[1], s.s, s.c)};
            const f16x2 r1 = {(_Float16)__builtin_fmaf((float)p1[0], s.s, s.c),
                              (_Float16)__builtin_fmaf((float)p1[1], s.s, s.c)};
            o[2 * d] = __builtin_bit_cast(uint32_t, r0);
            o[2 * d + 1] = __builtin_bit_cast(uint32_t, r1);
        }
        return __builtin_bit_cast(f16x8, u32x4{o[0], o[1], o[2], o[3]});
    }
};

template <>
struct Q8Op<_Float16, false> : Q8Mfma<_Float16> {
    typedef f16x2 Scale;  // the f16 scale in both halves
    static __device__ __forceinline__ Scale scale(uint32_t pair) { return __builtin_bit_cast(f16x2, pair); }
    static __device__ __forceinline__ V8 deq8(uint32_t w0, uint32_t w1, Scale s) { return q8_dequant8(w0, w1, s); }
};

// bf16 operands, f16 scales: each byte u as the f16 subnormal u 2^-24 (one
// v_perm per pair), v_fma_mix_f32 reads it directly and forms
// fma(u 2^-24, s 2^24, -128 s) = q s (exact in f32: at most 19 significant
// bits), one v_cvt_pk_bf16_f32 rounds the pair; 4 VALU instructions per
// MFMA. s 2^24 of an f16 scale is at most 1.1e12.
template <>
struct Q8Op<__bf16, false> : Q8Mfma<__bf16> {
    typedef Q8ScaleF32 Scale;  // s 2^24 and -128 s
    static __device__ __forceinline__ Scale scale(uint32_t pair) {
        const float s = (float)__builtin_bit_cast(_Float16, (uint16_t)(pair & 0xffffu));
        return Scale{s * 16777216.0f, -128.0f * s};
    }
    static __device__ __forceinline__ V8 deq8(uint32_t w0, uint32_t w1, Scale s) {
        uint32_t o[4];
#pragma unroll
        for (int d = 0; d < 2; d++) {
            const uint32_t x = d ? w1 : w0;
            const f16x2 p0 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0u, x, 0x04010400u));
            const f16x2 p1 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0u, x, 0x04030402u));
            o[2 * d] = Op<__bf16>::cvt2(__builtin_fmaf((float)p0[0], s.s, s.c), __builtin_fmaf((float)p0[1], s.s, s.c));
            o[2 * d + 1] =
                Op<__bf16>::cvt2(__builtin_fmaf((float)p1[0], s.s, s.c), __builtin_fmaf((float)p1[1], s.s, s.c));
        }
        return __builtin_bit_cast(bf16x8, u32x4{o[0], o[1], o[2], o[3]});
    }
};

// Raw buffer descriptor word 3 for gfx9-family parts (untyped dword access).
#define Q8_RSRC_W3 0x00020000

template <typename T, bool SF32, int EPI>
struct Q8Gemm {
    typedef Q8Op<T, SF32> QO;
    static constexpr int NI = 4, NJ = 2;
    const LtxGemmArgs& a;
    f32x16 acc[NI][NJ];
    __amdgpu_buffer_rsrc_t ra_, rb_, rs_;  // A, W and scale-pair buffers
    int g, nk, ng;
    uint32_t ga[4], gb[2];  // per-lane byte offsets of this wave's DMA sources (k-tile 0)
    int la, lb;             // this wave's DMA destinations within a stage (uniform)
    uint32_t offa[4], offb[2];
    uint32_t so;            // byte offset of the lane's first scale pair in group 0
    typename QO::Scale s2[NJ];

    __device__ __forceinline__ Q8Gemm(const LtxGemmArgs& args) : a(args) {}

    template <int S>
    __device__ __forceinline__ void dma(int k) {
        uint8_t* da = q8_stage_a<S>() + la;
        uint8_t* db = q8_stage_b<S>() + lb;
#pragma unroll
        for (int i = 0; i < 4; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra_, (lds_vptr)(da + 1024 * i), 16, ga[i], k * 128, 0, 0);
#pragma unroll
        for (int i = 0; i < 2; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb_, (lds_vptr)(db + 1024 * i), 16, gb[i], k * 64, 0, 0);
    }

    __device__ __forceinline__ void wait_dma(bool more2) {
        if (more2)
            __builtin_amdgcn_s_waitcnt(Q8_WAIT_VM(6));
        else
            __builtin_amdgcn_s_waitcnt(Q8_WAIT_VM(0));
    }

    // One K-tile: tile k sits in stage S; DMA of tile k + 2 (when more2) goes
    // to stage (S + 2) % 3, the stage tile k - 1 was read from.
    template <int S>
    __device__ __forceinline__ void step(int k, bool more2) {
        const uint8_t* sa = q8_stage_a<S>();
        const uint8_t* sb = q8_stage_b<S>();
        u32x4 fa[NI][4], wb[NJ][2];
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int c = 0; c < 2; c++) wb[j][c] = *(const u32x4*)(sb + offb[c] + 2048 * j);
#pragma unroll
        for (int i = 0; i < NI; i++)
#pragma unroll
            for (int t = 0; t < 4; t++) fa[i][t] = *(const u32x4*)(sa + offa[t] + 4096 * i);
        // scale pairs of the next tile, issued before this step's DMA so the
        // DMA wait below also covers them
        uint32_t sn[NJ];
        const int gnext = min((k + 1) >> 1, ng - 1) * a.N * 4;
#pragma unroll
        for (int j = 0; j < NJ; j++) sn[j] = __builtin_amdgcn_raw_buffer_load_b32(rs_, so + 128 * j, gnext, 0);
        __builtin_amdgcn_sched_barrier(0);
        if (more2) dma<(S + 2) % 3>(k + 2);
        __builtin_amdgcn_sched_barrier(0);
        // ping-pong: the first DQ k-steps are dequantised in this (memory)
        // phase, so the MFMA phase opens with MFMAs; the rest interleave with it
        constexpr int DQ = 2;
        typename QO::V8 fb0[DQ][NJ];
        {
            __builtin_amdgcn_s_waitcnt(Q8_WAIT_LGKM0);
#pragma unroll
            for (int t = 0; t < DQ; t++)
#pragma unroll
                for (int j = 0; j < NJ; j++) {
                    const u32x4 w = wb[j][t >> 1];
                    fb0[t][j] = (t & 1) ? QO::deq8(w[2], w[3], s2[j]) : QO::deq8(w[0], w[1], s2[j]);
                }
            if (g == 1) wait_dma(more2);
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            // the wave in its MFMA phase takes issue priority over the other
            // wave of its SIMD (without it the lower-numbered waves win)
            __builtin_amdgcn_s_setprio(1);
        }
#pragma unroll
        for (int t = 0; t < 4; t++) {
            typename QO::V8 fb[NJ];
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const u32x4 w = wb[j][t >> 1];
                if (t < DQ)
                    fb[j] = fb0[t < DQ ? t : 0][j];
                else
                    fb[j] = (t & 1) ? QO::deq8(w[2], w[3], s2[j]) : QO::deq8(w[0], w[1], s2[j]);
            }
#pragma unroll
            for (int i = 0; i < NI; i++)
#pragma unroll
                for (int j = 0; j < NJ; j++)
                    acc[i][j] = QO::mfma(fa[i][t], fb[j], acc[i][j]);
        }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
        if (g == 0) wait_dma(more2);
        __builtin_amdgcn_s_waitcnt(Q8_WAIT_LGKM0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < NJ; j++) s2[j] = QO::scale(sn[j]);
    }

    // One output tile per trip of a persistent loop: the grid is at most one
    // workgroup per CU, and workgroup b takes tiles b, b + grid, ... (the same
    // XCD and order as one workgroup per tile, without a dispatch and a drain
    // of the epilogue's stores between tiles).
    __device__ __forceinline__ void run() {
        const int tid = threadIdx.x, lane = tid & 63;
        const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
        g = w >> 2;
        const int q = w & 3;
        // split-K: each work item is one output tile and one of ksplit slices
        // of K (kc = K / ksplit, a multiple of 128); offsets below add the
        // slice's first k
        const int ks_n = a.ksplit > 1 ? a.ksplit : 1;
        const int kc = a.K / ks_n;
        nk = kc / 64;
        ng = kc / LTX_GROUP;
        ra_ = __builtin_amdgcn_make_buffer_rsrc((void*)a.a, 0, (int)((uint32_t)a.M * (uint32_t)a.lda * 2u), Q8_RSRC_W3);
        rb_ = __builtin_amdgcn_make_buffer_rsrc((void*)a.b, 0, (int)((uint32_t)a.N * (uint32_t)a.K), Q8_RSRC_W3);
        rs_ = __builtin_amdgcn_make_buffer_rsrc((void*)a.scales, 0,
                                                (int)((uint32_t)(a.K / LTX_GROUP) * (uint32_t)a.N * 4u), Q8_RSRC_W3);
        la = 4096 * w;
        lb = 2048 * w;
        // fragment reads: A row 128 g + 32 i + lane % 32, chunks 4 h + t;
        // W row 64 q + 32 j + lane % 32, chunks 2 h + c (h = lane / 32)
        {
            const int h = lane >> 5, r = lane & 31;
#pragma unroll
            for (int t = 0; t < 4; t++) offa[t] = (128 * g + r) * 128 + 16 * ((4 * h + t) ^ ((r >> 1) & 7));
#pragma unroll
            for (int c = 0; c < 2; c++) offb[c] = (64 * q + r) * 64 + 16 * ((2 * h + c) ^ ((r >> 2) & 3));
        }
        const int ntiles = a.tiles_m * a.tiles_n * ks_n;
        for (int item = blockIdx.x; item < ntiles; item += gridDim.x) {
            const int ks = item % ks_n;
            const TileIdx ti = tile_of(item / ks_n, a.tiles_m, a.tiles_n);
            const int m0 = ti.tm * 256, n0 = ti.tn * 256;
            const uint32_t k0 = (uint32_t)(ks * kc);  // first k of this slice
            // DMA sources. A: instruction i of wave w fills rows 8 (4 w + i) ..
            // +7, 8 lanes a row; W: rows 16 (2 w + i) .. +15, 4 lanes a row.
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int tr = 8 * (4 * w + i) + (lane >> 3);  // row within the tile
                const int c = (lane & 7) ^ ((tr >> 1) & 7);
                const int row = min(m0 + tr, a.M - 1);
                ga[i] = (uint32_t)row * (uint32_t)a.lda * 2u + 2u * k0 + 16u * c;
            }
            {
                const int nr = lane >> 2, nc = (lane & 3) ^ ((lane >> 4) & 3);
#pragma unroll
                for (int i = 0; i < 2; i++)
                    gb[i] = (uint32_t)(n0 + 16 * (2 * w + i) + nr) * (uint32_t)a.K + k0 + 16u * nc;
            }
            so = 4u * ((k0 / LTX_GROUP) * (uint32_t)a.N + (uint32_t)(n0 + 64 * q + (lane & 31)));
#pragma unroll
            for (int i = 0; i < NI; i++)
#pragma unroll
                for (int j = 0; j < NJ; j++) acc[i][j] = f32x16{0};

            // scale pairs first: the wait for tile 0 below then covers them too
#pragma unroll
            for (int j = 0; j < NJ; j++)
                s2[j] = QO::scale(__builtin_amdgcn_raw_buffer_load_b32(rs_, so + 128 * j, 0, 0));
            __builtin_amdgcn_sched_barrier(0);
            dma<0>(0);
            dma<1>(1);  // K is a multiple of 128: nk >= 2
            wait_dma(true);
            __builtin_amdgcn_s_barrier();
            if (g == 1) __builtin_amdgcn_s_barrier();
            // Main loop: three tiles per trip, every one with a DMA two tiles
            // ahead; the last 2 to 4 tiles follow unrolled.
            const int trips = (nk - 2) / 3;
            for (int it = 0; it < trips; it++) {
                const int k = 3 * it;
                step<0>(k, true);
                step<1>(k + 1, true);
                step<2>(k + 2, true);
            }
            {
                const int k = 3 * trips;  // nk - k is 2, 3 or 4
                step<0>(k, k + 2 < nk);
                step<1>(k + 1, k + 3 < nk);
                if (k + 2 < nk) step<2>(k + 2, k + 4 < nk);
                if (k + 3 < nk) step<0>(k + 3, false);
            }
            if (g == 0) __builtin_amdgcn_s_barrier();
            // Every wave has passed its last barrier: no stage is read or DMA'd
            // any more, and each wave stages its epilogue in a private 9 KB patch.
            uint8_t* patch = w < 3 ? q8_sa0 + 9216 * w : w < 6 ? q8_sa1 + 9216 * (w - 3) : q8_sa2 + 9216 * (w - 6);
            if (ks_n > 1)  // a slice's partial sums; ltx_gemm_reduce_* applies the epilogue
                gemm_store_partial<NI, NJ>(acc, (float*)patch, a.part + (size_t)ks * a.M * a.N, a.M, a.N,
                                           m0 + 128 * g, n0 + 64 * q);
            else
                gemm_epilogue_lds<T, EPI, NI, NJ>(a, acc, (float*)patch, m0 + 128 * g, n0 + 64 * q, n0);
            // every patch has been read back before the next tile's DMA fills
            // the stages it lives in
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(Q8_WAIT_LGKM0);
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
        }
    }
};

#define Q8_GEMM_KERNEL(NAME, T_, SF32_, EPI_)                                                \
    extern "C" __global__ void __launch_bounds__(512, 1) NAME(const LtxGemmArgs a) {         \
        Q8Gemm<T_, SF32_, EPI_> k(a);                                                  \
        k.run();                                                                             \
    }
