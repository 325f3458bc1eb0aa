// 16-bit GEMM for gfx950 on four waves: y[M][N] = A[M][K] . W[N][K]^T, A and
// W in the 16-bit operand type (f16 or bf16), f32 accumulate, the fused
// epilogues of gemm_common.h. It serves the unquantised projections
// (Block.wBlockOut, ltx/block.zig:351-353) directly and the int8 ones after
// ltx_gemm_dq16_* has dequantised their weights for the forward (the same
// operand bits as the W8A16 kernel's in-register dequantisation).
//
// Workgroup: 4 waves, one per SIMD, output tile 256 x 256; wave w owns rows
// 128 (w / 2) .. +127 and columns 128 (w % 2) .. +127 as 8 x 8 blocks of
// 16 x 16 on v_mfma_f32_16x16x32_{f16,bf16}: 256 accumulator registers
// (AGPRs), every fragment read from LDS feeds 8 MFMAs (0.25 KB of LDS per
// MFMA of 16 K flops, half the W8A16 kernel's bytes per flop), and the
// 16 x 16 x 32 shape runs at a higher rate than 32 x 32 x 16 at the board's
// power-limited clock.
//
// K is walked in tiles of 64: A (256 x 64) and W (256 x 64) go global -> LDS
// by LDS DMA (buffer_load_dwordx4 ... lds) into one of two stages of 64 KB,
// rows of 128 B with 16-byte chunk c of row r in slot c ^ ((r >> 1) & 7) (16
// consecutive rows of one chunk then cover the 64 banks once). A tile is
// multiplied in two steps of 32 k: in step s lanes 16 h .. 16 h + 15 read
// chunk 4 s + h of their row (A and W alike).
//
// Schedule (one barrier per K-tile, at the middle of the pair of steps that
// straddles two tiles): after the barrier that follows tile k's step 0, the
// waves issue the DMA of tile k + 2 into the stage tile k came from (every
// wave has read it), multiply tile k's step 1 while reading tile k + 1's
// step-0 fragments (landed: each wave waited for its own DMA before the
// barrier), then multiply tile k + 1's step 0 while reading its step 1, wait
// for their DMA and LDS reads, and meet at the next barrier. The DMA of a
// tile has one tile's MFMAs (2 x 64 per wave) to land. Fragment reads and
// DMA instructions are spread between the MFMAs (one of each after every
// fourth MFMA), in the order the next step needs them.
//
// Grid: persistent, one workgroup per CU, tiles in the XCD-grouped order of
// tile_of. After the last K-tile every stage is free and each wave stages
// its epilogue through a private 17 KB patch in one of the four stage
// objects.
#pragma once
#include "gemm_q8.h"

__shared__ __attribute__((aligned(1024))) uint8_t x4_a0[32768];
__shared__ __attribute__((aligned(1024))) uint8_t x4_a1[32768];
__shared__ __attribute__((aligned(1024))) uint8_t x4_b0[32768];
__shared__ __attribute__((aligned(1024))) uint8_t x4_b1[32768];

template <int S>
__device__ __forceinline__ uint8_t* x4_stage_a() {
    return S == 0 ? x4_a0 : x4_a1;
}
template <int S>
__device__ __forceinline__ uint8_t* x4_stage_b() {
    return S == 0 ? x4_b0 : x4_b1;
}

// s_waitcnt: vmcnt(0) and lgkmcnt(0)
#define X4_WAIT_ALL0 (7 << 4)

// A per-lane (v) or wave-uniform (s) offset through an empty volatile asm, at
// the point of use: the LDS addresses derived from it are formed there (one
// add, the rest in the instructions' offset fields) instead of being hoisted
// out of the tile loop as one register per fragment and DMA slice (which ran
// out of registers and spilled around the epilogue).
__device__ __forceinline__ uint32_t x4_vofs(uint32_t x) {
    asm volatile("" : "+v"(x));
    return x;
}
__device__ __forceinline__ int x4_sofs(int x) {
    asm volatile("" : "+s"(x));
    return x;
}

// SF: the STORE epilogue's form (bit 0 GELU, bit 1 f32 output), one kernel
// each, so that a kernel holds only the epilogue it runs.
template <typename T, int EPI, int SF = 0>
struct X4Gemm {
    typedef typename Op<T>::v8 V8;
    const LtxGemmArgs& a;
    f32x4 acc[8][8];
    __amdgpu_buffer_rsrc_t ra_, rb_;
    uint32_t ga[8];     // A: per-lane source offset of DMA instruction i (rows clamped to M - 1), k-tile 0
    uint32_t gb[2];     // W: of even and odd instructions; instruction i adds (i & ~1) 8-row steps
    uint32_t wstep;     // bytes of 8 W rows
    int lw;             // this wave's DMA destination within a stage
    uint32_t offa[2], offb[2];  // fragment reads of step s (row block i adds 2048 i)
    u32x4 fa0[8], fb0[8], fa1[8], fb1[8];

    __device__ __forceinline__ X4Gemm(const LtxGemmArgs& args) : a(args) {}

    __device__ __forceinline__ void mfma(const u32x4& x, const u32x4& y, f32x4& c) {
        c = Op<T>::mfma16(__builtin_bit_cast(V8, x), __builtin_bit_cast(V8, y), c);
    }

    template <int RS, int RSTEP>
    __device__ __forceinline__ void read_all(u32x4 (&ya)[8], u32x4 (&yb)[8]) {
        const uint8_t* sa = x4_stage_a<RS>() + x4_vofs(offa[RSTEP]);
        const uint8_t* sb = x4_stage_b<RS>() + x4_vofs(offb[RSTEP]);
#pragma unroll
        for (int i = 0; i < 8; i++) ya[i] = *(const u32x4*)(sa + 2048 * i);
#pragma unroll
        for (int j = 0; j < 8; j++) yb[j] = *(const u32x4*)(sb + 2048 * j);
    }

    template <int DS>
    __device__ __forceinline__ void dma(int k) {
        const int l = x4_sofs(lw);
        uint8_t* da = x4_stage_a<DS>() + l;
        uint8_t* db = x4_stage_b<DS>() + l;
#pragma unroll
        for (int i = 0; i < 8; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra_, (lds_vptr)(da + 1024 * i), 16, ga[i], k * 128, 0, 0);
#pragma unroll
        for (int i = 0; i < 8; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb_, (lds_vptr)(db + 1024 * i), 16, gb[i & 1],
                                                     k * 128 + (i & ~1) * wstep, 0, 0);
    }

    __device__ __forceinline__ void mfma_all(const u32x4 (&xa)[8], const u32x4 (&xb)[8]) {
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int j = 0; j < 8; j++) mfma(xa[i], xb[j], acc[i][j]);
    }

    // The 64 MFMAs of one step (xa, xb) with the 16 fragment reads of another
    // (stage RS, step RSTEP, into ya, yb) and, when DMA, the 16 DMA
    // instructions of tile kd into stage DS, one of each after every fourth
    // MFMA; reads in the order the next step needs them (A0, W0..W7, A1..A7).
    // Measured against one after every third MFMA: 1-3 % faster at 28,672
    // rows; every second: 10 % slower; all DMA at the region's start: 10-14 %
    // slower.
    template <int RS, int RSTEP, int DS, bool DMA>
    __device__ __forceinline__ void region(const u32x4 (&xa)[8], const u32x4 (&xb)[8], u32x4 (&ya)[8],
                                           u32x4 (&yb)[8], int kd) {
        const uint8_t* sa = x4_stage_a<RS>() + x4_vofs(offa[RSTEP]);
        const uint8_t* sb = x4_stage_b<RS>() + x4_vofs(offb[RSTEP]);
        const int l = DMA ? x4_sofs(lw) : 0;
        uint8_t* da = x4_stage_a<DS>() + l;
        uint8_t* db = x4_stage_b<DS>() + l;
#pragma unroll
        for (int m = 0; m < 64; m++) {
            mfma(xa[m >> 3], xb[m & 7], acc[m >> 3][m & 7]);
            if (m % 4 == 3) {
                const int g = m / 4;
                __builtin_amdgcn_sched_barrier(0);
                if (g == 0)
                    ya[0] = *(const u32x4*)sa;
                else if (g <= 8)
                    yb[g - 1] = *(const u32x4*)(sb + 2048 * (g - 1));
                else
                    ya[g - 8] = *(const u32x4*)(sa + 2048 * (g - 8));
                if (DMA) {
                    if (g < 8)
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(ra_, (lds_vptr)(da + 1024 * g), 16, ga[g], kd * 128,
                                                                 0, 0);
                    else
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(rb_, (lds_vptr)(db + 1024 * (g - 8)), 16, gb[g & 1],
                                                                 kd * 128 + ((g - 8) & ~1) * wstep, 0, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }

    __device__ __forceinline__ void meet() {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(X4_WAIT_ALL0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    }

    // Entered after a barrier: tile k in stage S with its step-1 fragments in
    // fa1/fb1, tile k + 1 landed in stage S ^ 1, no DMA pending, stage S read
    // by every wave. DMA of tile k + 2 into stage S (when DMA); tile k step 1;
    // tile k + 1 step 0; barrier.
    template <int S, bool DMA>
    __device__ __forceinline__ void pair(int k) {
        region<S ^ 1, 0, S, DMA>(fa1, fb1, fa0, fb0, k + 2);
        __builtin_amdgcn_sched_barrier(0);
        region<S ^ 1, 1, S, false>(fa0, fb0, fa1, fb1, 0);
        meet();
    }

    __device__ __forceinline__ void run() {
        const int tid = threadIdx.x, lane = tid & 63;
        const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int wm = 128 * (w >> 1), wn = 128 * (w & 1);
        const int nk = a.K / 64;  // even: K is a multiple of 128
        ra_ = __builtin_amdgcn_make_buffer_rsrc((void*)a.a, 0, (int)((uint32_t)a.M * (uint32_t)a.lda * 2u), Q8_RSRC_W3);
        rb_ = __builtin_amdgcn_make_buffer_rsrc((void*)a.b, 0, (int)((uint32_t)a.N * (uint32_t)a.K * 2u), Q8_RSRC_W3);
        lw = 8192 * w;
        wstep = 16u * (uint32_t)a.K;
        {
            const int h = lane >> 4, r = lane & 15;
#pragma unroll
            for (int s = 0; s < 2; s++) {
                offa[s] = (wm + r) * 128 + 16 * ((4 * s + h) ^ ((r >> 1) & 7));
                offb[s] = (wn + r) * 128 + 16 * ((4 * s + h) ^ ((r >> 1) & 7));
            }
        }
        uint8_t* patch = w == 0 ? x4_a0 : w == 1 ? x4_a1 : w == 2 ? x4_b0 : x4_b1;
        const int ntiles = a.tiles_m * a.tiles_n;
        for (int item = blockIdx.x; item < ntiles; item += gridDim.x) {
            const TileIdx ti = tile_of(item, a.tiles_m, a.tiles_n);
            const int m0 = ti.tm * 256, n0 = ti.tn * 256;
            // DMA instruction i of wave w fills tile rows 8 (8 w + i) .. +7,
            // 8 lanes a row; the row's swizzle (row / 2) & 7 is (4 i + lane / 16) & 7
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int tr = 8 * (8 * w + i) + (lane >> 3);
                const int c = (lane & 7) ^ ((tr >> 1) & 7);
                ga[i] = (uint32_t)min(m0 + tr, a.M - 1) * (uint32_t)a.lda * 2u + 16u * c;
            }
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int tr = 8 * (8 * w + i) + (lane >> 3);
                const int c = (lane & 7) ^ ((tr >> 1) & 7);
                gb[i] = (uint32_t)(n0 + tr) * (uint32_t)a.K * 2u + 16u * c;
            }
#pragma unroll
            for (int i = 0; i < 8; i++)
#pragma unroll
                for (int j = 0; j < 8; j++) acc[i][j] = f32x4{0, 0, 0, 0};
            dma<0>(0);
            __builtin_amdgcn_s_waitcnt(Q8_WAIT_VM(0));
            __builtin_amdgcn_s_barrier();
            dma<1>(1);
            read_all<0, 0>(fa0, fb0);
            read_all<0, 1>(fa1, fb1);
            mfma_all(fa0, fb0);  // tile 0, step 0
            meet();
            for (int k = 0; k < nk - 2; k += 2) {
                pair<0, true>(k);
                pair<1, true>(k + 1);
            }
            pair<0, false>(nk - 2);
            mfma_all(fa1, fb1);  // tile nk - 1, step 1
            meet();
            // every wave has passed the last barrier: the stages are free
            const int el = opaque_tid() & 63;
            auto fill = [&](int b, float* p, int LD) {
#pragma unroll
                for (int e = 0; e < 2; e++)
#pragma unroll
                    for (int j = 0; j < 8; j++)
#pragma unroll
                        for (int r = 0; r < 4; r++)
                            p[(16 * e + 4 * (el >> 4) + r) * LD + 16 * j + (el & 15)] = acc[2 * b + e][j][r];
            };
            gemm_epilogue_patch<T, EPI, 4, 4, decltype(fill), EPI == LTX_EPI_STORE ? SF : -1, 4>(
                a, fill, (float*)patch, m0 + wm, n0 + wn, n0);
            // every patch has been read back before the next tile's DMA
            meet();
        }
    }
};

#define X4_GEMM_KERNEL(NAME, T_, EPI_, SF_)                                          \
    extern "C" __global__ void __launch_bounds__(256, 1) NAME(const LtxGemmArgs a) { \
        X4Gemm<T_, EPI_, SF_> k(a);                                                  \
        k.run();                                                                     \
    }

// Dequantisation of int8 projections for the forward: W16[n][k] = the
// operand the W8A16 kernel forms in registers (Q8Op::deq8) from the bytes
// q + 128 [N][K] and the scale words [K / 128][N]. Up to LTX_DQ_JOBS
// projections per launch; workgroup b of job j (start[j] <= b < start[j + 1])
// covers 32 rows of one 128-k group, 16 k per thread (16 bytes in, 32 out).
template <typename T, bool SF32>
__device__ __forceinline__ void dq16_body(const LtxDq16Args& a) {
    typedef Q8Op<T, SF32> QO;
    const int b = blockIdx.x;
    int j = 0;
#pragma unroll
    for (int t = 1; t < LTX_DQ_JOBS; t++) j += (t < a.njobs && b >= a.start[t]) ? 1 : 0;
    const int local = b - a.start[j];
    const int G = a.K[j] / LTX_GROUP;
    const int g = local % G, nb = local / G;
    const int n = 32 * nb + (threadIdx.x >> 3);
    const int k = LTX_GROUP * g + 16 * (threadIdx.x & 7);
    if (n >= a.N[j]) return;
    const u32x4 w = *(const u32x4*)(a.q[j] + (size_t)n * a.K[j] + k);
    const typename QO::Scale s = QO::scale(a.s2[j][(size_t)g * a.N[j] + n]);
    const typename QO::V8 lo = QO::deq8(w[0], w[1], s), hi = QO::deq8(w[2], w[3], s);
    u32x4* out = (u32x4*)((uint16_t*)a.out[j] + (size_t)n * a.K[j] + k);
    out[0] = __builtin_bit_cast(u32x4, lo);
    out[1] = __builtin_bit_cast(u32x4, hi);
}
