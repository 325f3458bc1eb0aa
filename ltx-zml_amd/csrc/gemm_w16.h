// W16A16 GEMM for gfx950 with LDS-DMA staging: y[M][N] = A[M][K] . W[N][K]^T,
// A and W both in the 16-bit operand type (f16 or bf16): the unquantised
// projections of Block.wBlockOut (ltx/block.zig:22-26, 351-353), fused
// epilogues as in gemm_common.h.
//
// Workgroup: 8 waves (two per SIMD), output tile 256 x 128; wave w owns rows
// 64 (w / 2) .. +63 and columns 64 (w % 2) .. +63 (2 x 2 blocks of 32 x 32,
// v_mfma_f32_32x32x16_f16 or _bf16, f32 accumulate). A 16-bit W tile of 256
// columns would need 32 KB per stage beside A's 32 KB; with 128 columns a
// stage is A 32 KB + W 16 KB, the same 48 KB as the int8 kernel, so three
// stages fit and the DMA runs two tiles ahead as there. The price is LDS
// bytes per MFMA: 1 KB (each A and W fragment feeds two MFMAs) against the
// int8 kernel's 0.625 KB, with no dequantisation.
//
// K is walked in tiles of 64: A (256 x 64) and W (128 x 64) go global -> LDS
// with buffer_load ... lds into one of three stages, rows of 128 B with
// 16-byte chunk c of row r in slot c ^ ((r >> 1) & 7) (the int8 kernel's A
// layout, for both). k order inside a tile: for MFMA step t (0..3), lanes
// 0-31 multiply k = 8 t + 0..7 and lanes 32-63 k = 32 + 8 t + 0..7, for A and
// W alike. Ping-pong, waits and the persistent grid as in gemm_q8.h.
#pragma once
#include "gemm_q8.h"

template <typename T, int EPI>
struct W16Gemm {
    typedef typename Op<T>::v8 V8;
    static constexpr int NI = 2, NJ = 2;
    const LtxGemmArgs& a;
    f32x16 acc[NI][NJ];
    __amdgpu_buffer_rsrc_t ra_, rb_;  // A and W buffers
    int grp, nk;
    uint32_t ga[4], gb[2];  // per-lane byte offsets of this wave's DMA sources (k-tile 0)
    int la, lb;             // this wave's DMA destinations within a stage (uniform)
    uint32_t offa[4], offb[4];  // fragment reads per MFMA step (row block i / column block j adds 4096)

    __device__ __forceinline__ W16Gemm(const LtxGemmArgs& args) : a(args) {}

    template <int S>
    __device__ __forceinline__ void dma(int k) {
        uint8_t* da = q8_stage_a<S>() + la;
        uint8_t* db = q8_stage_b<S>() + lb;
#pragma unroll
        for (int i = 0; i < 4; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra_, (lds_vptr)(da + 1024 * i), 16, ga[i], k * 128, 0, 0);
#pragma unroll
        for (int i = 0; i < 2; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb_, (lds_vptr)(db + 1024 * i), 16, gb[i], k * 128, 0, 0);
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
    __device__ __forceinline__ void step(bool more2, int k) {
        const uint8_t* sa = q8_stage_a<S>();
        const uint8_t* sb = q8_stage_b<S>();
        u32x4 fa[NI][4], fb[NJ][4];
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int t = 0; t < 4; t++) fb[j][t] = *(const u32x4*)(sb + offb[t] + 4096 * j);
#pragma unroll
        for (int i = 0; i < NI; i++)
#pragma unroll
            for (int t = 0; t < 4; t++) fa[i][t] = *(const u32x4*)(sa + offa[t] + 4096 * i);
        __builtin_amdgcn_sched_barrier(0);
        if (more2) dma<(S + 2) % 3>(k + 2);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(Q8_WAIT_LGKM0);
        if (grp == 1) wait_dma(more2);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        // the wave in its MFMA phase takes issue priority over the other wave
        // of its SIMD
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int i = 0; i < NI; i++)
#pragma unroll
                for (int j = 0; j < NJ; j++)
                    acc[i][j] = Op<T>::mfma32(__builtin_bit_cast(V8, fa[i][t]), __builtin_bit_cast(V8, fb[j][t]),
                                              acc[i][j]);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
        if (grp == 0) wait_dma(more2);
        __builtin_amdgcn_s_waitcnt(Q8_WAIT_LGKM0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    }

    // One output tile (or split-K slice) per trip of a persistent loop, as in
    // Q8Gemm::run.
    __device__ __forceinline__ void run() {
        const int tid = threadIdx.x, lane = tid & 63;
        const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
        grp = w >> 2;
        const int wm = 64 * (w >> 1), wn = 64 * (w & 1);  // this wave's tile within the workgroup's
        const int ks_n = a.ksplit > 1 ? a.ksplit : 1;
        const int kc = a.K / ks_n;
        nk = kc / 64;
        ra_ = __builtin_amdgcn_make_buffer_rsrc((void*)a.a, 0, (int)((uint32_t)a.M * (uint32_t)a.lda * 2u), Q8_RSRC_W3);
        rb_ = __builtin_amdgcn_make_buffer_rsrc((void*)a.b, 0, (int)((uint32_t)a.N * (uint32_t)a.K * 2u), Q8_RSRC_W3);
        la = 4096 * w;
        lb = 2048 * w;
        // fragment reads: A row wm + 32 i + lane % 32, W row wn + 32 j + lane % 32,
        // chunk 4 h + t (h = lane / 32)
        {
            const int h = lane >> 5, r = lane & 31;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                offa[t] = (wm + r) * 128 + 16 * ((4 * h + t) ^ ((r >> 1) & 7));
                offb[t] = (wn + r) * 128 + 16 * ((4 * h + t) ^ ((r >> 1) & 7));
            }
        }
        const int ntiles = a.tiles_m * a.tiles_n * ks_n;
        for (int item = blockIdx.x; item < ntiles; item += gridDim.x) {
            const int ks = item % ks_n;
            const TileIdx ti = tile_of(item / ks_n, a.tiles_m, a.tiles_n);
            const int m0 = ti.tm * 256, n0 = ti.tn * 128;
            const uint32_t k0 = (uint32_t)(ks * kc);  // first k of this slice
            // DMA sources. A: instruction i of wave w fills rows 8 (4 w + i) ..
            // +7; W: rows 8 (2 w + i) .. +7 (8 lanes a row, 16 B each)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int tr = 8 * (4 * w + i) + (lane >> 3);
                const int c = (lane & 7) ^ ((tr >> 1) & 7);
                const int row = min(m0 + tr, a.M - 1);
                ga[i] = (uint32_t)row * (uint32_t)a.lda * 2u + 2u * k0 + 16u * c;
            }
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int tr = 8 * (2 * w + i) + (lane >> 3);
                const int c = (lane & 7) ^ ((tr >> 1) & 7);
                gb[i] = (uint32_t)(n0 + tr) * (uint32_t)a.K * 2u + 2u * k0 + 16u * c;
            }
#pragma unroll
            for (int i = 0; i < NI; i++)
#pragma unroll
                for (int j = 0; j < NJ; j++) acc[i][j] = f32x16{0};
            dma<0>(0);
            dma<1>(1);  // K is a multiple of 128: nk >= 2
            wait_dma(true);
            __builtin_amdgcn_s_barrier();
            if (grp == 1) __builtin_amdgcn_s_barrier();
            const int trips = (nk - 2) / 3;
            for (int it = 0; it < trips; it++) {
                const int k = 3 * it;
                step<0>(true, k);
                step<1>(true, k + 1);
                step<2>(true, k + 2);
            }
            {
                const int k = 3 * trips;  // nk - k is 2, 3 or 4
                step<0>(k + 2 < nk, k);
                step<1>(k + 3 < nk, k + 1);
                if (k + 2 < nk) step<2>(k + 4 < nk, k + 2);
                if (k + 3 < nk) step<0>(false, k + 3);
            }
            if (grp == 0) __builtin_amdgcn_s_barrier();
            // every wave has passed its last barrier: stages are free for the
            // wave-private epilogue patches
            uint8_t* patch = w < 3 ? q8_sa0 + 9216 * w : w < 6 ? q8_sa1 + 9216 * (w - 3) : q8_sa2 + 9216 * (w - 6);
            if (ks_n > 1)
                gemm_store_partial<NI, NJ>(acc, (float*)patch, a.part + (size_t)ks * a.M * a.N, a.M, a.N, m0 + wm,
                                           n0 + wn);
            else
                gemm_epilogue_lds<T, EPI, NI, NJ>(a, acc, (float*)patch, m0 + wm, n0 + wn, n0);
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(Q8_WAIT_LGKM0);
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
        }
    }
};

#define W16_GEMM_KERNEL(NAME, T_, EPI_)                                              \
    extern "C" __global__ void __launch_bounds__(512, 1) NAME(const LtxGemmArgs a) { \
        W16Gemm<T_, EPI_> k(a);                                                      \
        k.run();                                                                     \
    }
