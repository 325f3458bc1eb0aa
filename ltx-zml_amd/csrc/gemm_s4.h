// Small-grid GEMM for gfx950: y[M][N] = A[M][K] . W[N][K]^T on 128 x 128
// output tiles, for the shapes whose 256 x 256 tiles would leave CUs idle
// (fewer rows than 4,096: the 1,024-token block, the 256-row context k|v
// projection), where the 256 x 256 kernels otherwise split K and add the
// slices in a second launch.
//
// Workgroup: 4 waves in a 2 x 2 grid of 64 x 64 wave tiles, each 4 x 4
// blocks of 16 x 16 on v_mfma_f32_16x16x32_{f16,bf16} (64 f32 accumulators);
// two workgroups share a CU, so one's barrier and epilogue overlap the
// other's MFMAs.
//
// W is int8 (bytes q + 128 [N][K] and scale words [K / 128][N], the layout of
// the W8A16 kernel; each 16 x 32 fragment is dequantised in registers after
// its LDS read by the same Q8Op arithmetic, so the operand bits are that
// kernel's) or 16-bit. K goes in tiles of 64 through LDS by LDS DMA
// (buffer_load_dwordx4 ... lds) into NS stages, one barrier per tile: int8
// NS = 3, the DMA two tiles ahead (74 KB of LDS); 16-bit NS = 2, one tile
// ahead (64 KB). A rows of 128 B with 16-byte chunk c of row r in slot
// c ^ ((r >> 1) & 7); 16-bit W the same; int8 W rows of 64 B with chunk c of
// row n in slot c ^ ((n >> 2) & 3). Each stage is a __shared__ object of its
// own, so the compiler's LDS-DMA alias tracking waits only for the stage a
// read touches.
//
// Split-K as in the 256 x 256 kernels: a work item is one tile and one of
// ksplit K slices, whose f32 partial sums go to part[S][M][N] for
// ltx_gemm_reduce_* to finish with the epilogue.
#pragma once
#include "gemm_common.h"
#include "gemm_q8.h"

// s_waitcnt lgkmcnt(n) alone (vmcnt and expcnt at their maxima)
#define Q8_WAIT_LGKM(n) (15 | (3 << 14) | (7 << 4) | ((n) << 8))

#include <type_traits>

// One __shared__ object per stage, A at 0 and W at 16384 (int8: 8 KB of
// weights, then the tile's scale words, 256 B a wave for the 64 columns of
// its wave tile). With an object per operand and stage (six), the compiler's
// LDS-DMA tracking no longer told the stages apart and waited for the DMA two
// tiles ahead before reading the current one.
__shared__ __attribute__((aligned(1024))) uint8_t s4q_st0[25600];
__shared__ __attribute__((aligned(1024))) uint8_t s4q_st1[25600];
__shared__ __attribute__((aligned(1024))) uint8_t s4q_st2[25600];
__shared__ __attribute__((aligned(1024))) uint8_t s4w_st0[32768];
__shared__ __attribute__((aligned(1024))) uint8_t s4w_st1[32768];
__shared__ __attribute__((aligned(1024))) uint8_t s4w_st2[32768];

template <bool Q, int S>
__device__ __forceinline__ uint8_t* s4_stage_a() {
    if constexpr (Q)
        return S == 0 ? s4q_st0 : S == 1 ? s4q_st1 : s4q_st2;
    else
        return S == 0 ? s4w_st0 : S == 1 ? s4w_st1 : s4w_st2;
}
template <bool Q, int S>
__device__ __forceinline__ uint8_t* s4_stage_b() {
    return s4_stage_a<Q, S>() + 16384;
}

// One dword read from LDS by an instruction the compiler does not track
// (its result has no wait of its own): used for the int8 scale words, each
// read just before an ordinary LDS read whose wait then covers it (LDS reads
// complete in order). Tracked, the first scale read after the tile loop's
// head made the compiler wait for the LDS DMA two tiles ahead (it could not
// tell that DMA's stage from the one read).
__device__ __forceinline__ uint32_t s4_lds_u32(const uint8_t* p) {
    uint32_t x;
    const uint32_t addr = (uint32_t)(uintptr_t)(lds_vptr)p;
    asm volatile("ds_read_b32 %0, %1" : "=v"(x) : "v"(addr) : "memory");
    return x;
}

// Split-K partial sums of one wave's (32 NI) x (32 NJ) tile, filled block by
// block into the wave-private patch (fill(i, patch, LD) as for
// gemm_epilogue_patch) and stored as 16-byte row segments of part[m][n].
template <int NI, int NJ, typename Fill>
__device__ __forceinline__ void gemm_store_partial_patch(Fill fill, float* patch, float* part, int M, int N, int mw,
                                                         int nw) {
    constexpr int WN = 32 * NJ, LD = WN + 8;
    constexpr int LPR = WN / 4, RPP = 64 / LPR;  // lanes per row, rows per pass
    const int lane = opaque_tid() & 63;
    const int c4 = 4 * (lane % LPR), r0 = lane / LPR;
#pragma unroll
    for (int i = 0; i < NI; i++) {
        fill(i, patch, LD);
#pragma unroll
        for (int p = 0; p < 32 / RPP; p++) {
            const int rr = r0 + RPP * p, m = mw + 32 * i + rr;
            if (m < M) *(f32x4*)(part + (size_t)m * N + nw + c4) = *(const f32x4*)(patch + rr * LD + c4);
        }
    }
}

template <typename T, int BK, int EPI>
struct S4Gemm {
    static constexpr bool Q = BK != LTX_B_W16;
    static constexpr bool SF32 = BK == LTX_B_I8_F32S;
    static constexpr int NDB = Q ? 2 : 4;             // W DMA instructions per wave and tile (A: 4)
    static constexpr int NV = 4 + NDB + (Q ? 1 : 0);  // DMA instructions per wave and tile (+1: scale words)
    typedef Q8Op<T, SF32> QO;
    typedef typename Op<T>::v8 V8;
    typedef typename std::conditional<Q, u32x2, u32x4>::type WF;  // a W fragment as read from LDS
    const LtxGemmArgs& a;
    f32x4 acc[4][4];
    __amdgpu_buffer_rsrc_t ra_, rb_, rs_;
    uint32_t ga[4], gb[4];  // per-lane DMA source offsets, K-tile 0 of the slice
    uint32_t so;            // byte offset of scale word n0 + wn + lane, first group of the slice
    uint32_t lsc;           // LDS offset of the lane's scale word (column block 0) within a W stage
    int la, lb, ls;         // this wave's DMA destinations within a stage (A, W, int8 scale words)
    uint32_t offa[2], offb[2];  // fragment reads of step s (block i adds 2048 i; int8 W 1024 i)
    // fragments of one 32-k step (A, W as read, W's scale words): step 0 of
    // the next tile and step 1 of the current one
    u32x4 fa0[4], fa1[4];
    WF fw0[4], fw1[4];
    uint32_t sc0[4], sc1[4];

    __device__ __forceinline__ S4Gemm(const LtxGemmArgs& args) : a(args) {}

    // DMA instruction d (0 .. NV - 1) of K-tile kt into stage S: with int8
    // weights first the scale words of the tile's group for the wave's 64
    // columns (one dword a lane, read back by the wave itself), then A, then W
    template <int S>
    __device__ __forceinline__ void dma1(int d, int kt) {
        constexpr int Q1 = Q ? 1 : 0;
        if (Q && d == 0)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_, (lds_vptr)(s4_stage_b<Q, S>() + ls), 4, so,
                                                     (kt >> 1) * a.N * 4, 0, 0);
        else if (d < Q1 + 4)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra_, (lds_vptr)(s4_stage_a<Q, S>() + la + 1024 * (d - Q1)), 16,
                                                     ga[d - Q1], kt * 128, 0, 0);
        else
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb_, (lds_vptr)(s4_stage_b<Q, S>() + lb + 1024 * (d - Q1 - 4)),
                                                     16, gb[d - Q1 - 4], kt * (Q ? 64 : 128), 0, 0);
    }
    template <int S>
    __device__ __forceinline__ void dma(int kt) {
#pragma unroll
        for (int d = 0; d < NV; d++) dma1<S>(d, kt);
    }

    // read r (0 .. 7) of step STEP from stage S: W blocks 0 .. 3 (int8, step
    // 0: each after its scale word), then A blocks 0 .. 3, the order the
    // step's MFMAs take them
    template <int S, int STEP>
    __device__ __forceinline__ void read1(int r, u32x4 (&ya)[4], WF (&yw)[4], uint32_t (&ysc)[4]) {
        const uint8_t* sa = s4_stage_a<Q, S>();
        const uint8_t* sb = s4_stage_b<Q, S>();
        if (r < 4) {
            if (Q && STEP == 0) ysc[r] = s4_lds_u32(sb + lsc + 64 * r);
            yw[r] = *(const WF*)(sb + offb[STEP] + (Q ? 1024 : 2048) * r);
        } else {
            ya[r - 4] = *(const u32x4*)(sa + offa[STEP] + 2048 * (r - 4));
        }
    }
    template <int S, int STEP>
    __device__ __forceinline__ void read_all(u32x4 (&ya)[4], WF (&yw)[4], uint32_t (&ysc)[4]) {
#pragma unroll
        for (int r = 0; r < 8; r++) read1<S, STEP>(r, ya, yw, ysc);
    }

    // the W fragments as MFMA operands (int8: dequantised with their scales)
    __device__ __forceinline__ void operands(const WF (&w)[4], const uint32_t (&sc)[4], V8 (&xb)[4]) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if constexpr (Q)
                xb[j] = QO::deq8(w[j][0], w[j][1], QO::scale(sc[j]));
            else
                xb[j] = __builtin_bit_cast(V8, w[j]);
        }
    }

    __device__ __forceinline__ void mfma1(int m, const u32x4 (&xa)[4], const V8 (&xb)[4]) {
        acc[m >> 2][m & 3] = Op<T>::mfma16(__builtin_bit_cast(V8, xa[m >> 2]), xb[m & 3], acc[m >> 2][m & 3]);
    }

    // The 16 MFMAs of one step (xa, xb) with the 8 fragment reads of step
    // STEP of stage RS (after every odd MFMA) and, when DMA, the NV DMA
    // instructions of tile kd into stage DS (after every even one).
    template <int RS, int STEP, int DS, bool DMA>
    __device__ __forceinline__ void region(const u32x4 (&xa)[4], const V8 (&xb)[4], u32x4 (&ya)[4], WF (&yw)[4],
                                           uint32_t (&ysc)[4], int kd) {
#pragma unroll
        for (int m = 0; m < 16; m++) {
            mfma1(m, xa, xb);
            __builtin_amdgcn_sched_barrier(0);
            if (m & 1)
                read1<RS, STEP>(m >> 1, ya, yw, ysc);
            else if (DMA && (m >> 1) < NV)
                dma1<DS>(m >> 1, kd);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // s_waitcnt vmcnt(n) lgkmcnt(0)
    __device__ __forceinline__ void wait_vm_lds(bool more) {
        if (more)
            __builtin_amdgcn_s_waitcnt(Q8_WAIT_VM(NV) & ~(15 << 8));
        else
            __builtin_amdgcn_s_waitcnt(7 << 4);
    }
    __device__ __forceinline__ void meet_lds() {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(Q8_WAIT_LGKM0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    }

    // Entered after a barrier: tile k's step-1 fragments in fa1/fw1/sc1, tile
    // k + 1 landed in stage (S + 1) % 3, the DMA of tile k + 2 in flight,
    // stage S (tile k) read by every wave. DMA of tile k + 3 into stage S;
    // tile k step 1 while reading tile k + 1 step 0; tile k + 1 step 0 while
    // reading its step 1; wait for tile k + 2; barrier. Past the last tile the
    // DMA repeats tile nk - 1 into the free stage: with no branch around the
    // DMA or the wait, the compiler's LDS-DMA tracking keeps the stages apart
    // at the loop head (with one, the first read of every third tile waited
    // for the DMA two tiles ahead).
    template <int S>
    __device__ __forceinline__ void pair(int k, int nk) {
        constexpr int R = (S + 1) % 3;
        V8 xb[4];
        operands(fw1, sc1, xb);
        region<R, 0, S, true>(fa1, xb, fa0, fw0, sc0, min(k + 3, nk - 1));
        __builtin_amdgcn_sched_barrier(0);
        // step 0's scale words and W fragments landed (its A fragments, read
        // last, may still be in flight)
        __builtin_amdgcn_s_waitcnt(Q8_WAIT_LGKM(4));
        // nothing that reads the scale words may move above that wait
        __builtin_amdgcn_sched_barrier(0);
        operands(fw0, sc0, xb);
#pragma unroll
        for (int j = 0; j < 4; j++) sc1[j] = sc0[j];
        region<R, 1, S, false>(fa0, xb, fa1, fw1, sc1, 0);
        __builtin_amdgcn_sched_barrier(0);
        wait_vm_lds(true);
        meet_lds();
    }

    __device__ __forceinline__ void run() {
        const int tid = threadIdx.x, lane = tid & 63;
        const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int wm = 64 * (w >> 1), wn = 64 * (w & 1);
        const int ks_n = a.ksplit > 1 ? a.ksplit : 1;
        const int kc = a.K / ks_n;  // a multiple of 128: nk is even and at least 2
        const int nk = kc / 64;
        ra_ = __builtin_amdgcn_make_buffer_rsrc((void*)a.a, 0, (int)((uint32_t)a.M * (uint32_t)a.lda * 2u), Q8_RSRC_W3);
        rb_ = __builtin_amdgcn_make_buffer_rsrc((void*)a.b, 0, (int)((uint32_t)a.N * (uint32_t)a.K * (Q ? 1u : 2u)),
                                                Q8_RSRC_W3);
        if constexpr (Q)
            rs_ = __builtin_amdgcn_make_buffer_rsrc((void*)a.scales, 0,
                                                    (int)((uint32_t)(a.K / LTX_GROUP) * (uint32_t)a.N * 4u), Q8_RSRC_W3);
        // wave w's DMA fills A rows 32 w .. 32 w + 31 (4 KB), int8 W rows
        // 32 w .. + 31 (2 KB), 16-bit W rows 32 w .. + 31 (4 KB); int8 scale
        // words of columns wn .. wn + 63 at 8192 + 256 w
        la = 4096 * w;
        lb = (Q ? 2048 : 4096) * w;
        ls = 8192 + 256 * w;
        lsc = ls + 4 * (lane & 15);
        {
            const int h = lane >> 4, r = lane & 15;
#pragma unroll
            for (int s = 0; s < 2; s++) {
                offa[s] = (wm + r) * 128 + 16 * ((4 * s + h) ^ ((r >> 1) & 7));
                // int8: the lane's 8 bytes k = 32 s + 8 h .. + 7 are half h & 1 of chunk 2 s + h / 2
                offb[s] = Q ? (wn + r) * 64 + 16 * ((2 * s + (h >> 1)) ^ ((r >> 2) & 3)) + 8 * (h & 1)
                            : (wn + r) * 128 + 16 * ((4 * s + h) ^ ((r >> 1) & 7));
            }
        }
        // epilogue patches (32 rows of 72 floats, 9 KB): waves 0-2 at the start
        // of stages 0-2, wave 3 at 16384 in stage 0
        uint8_t* patch = w == 0 ? s4_stage_a<Q, 0>() : w == 1 ? s4_stage_a<Q, 1>()
                       : w == 2 ? s4_stage_a<Q, 2>() : s4_stage_b<Q, 0>();
        const int ntiles = a.tiles_m * a.tiles_n * ks_n;
        for (int item = blockIdx.x; item < ntiles; item += gridDim.x) {
            const int ks = item % ks_n;
            const TileIdx ti = tile_of(item / ks_n, a.tiles_m, a.tiles_n);
            const int m0 = ti.tm * 128, n0 = ti.tn * 128;
            const uint32_t k0 = (uint32_t)(ks * kc);  // first k of this slice
            // A and 16-bit W: instruction i of wave w fills rows 8 (4 w + i) ..
            // + 7, 8 lanes a row (16-byte slot lane % 8 of the row, which holds
            // the row's chunk slot ^ ((row >> 1) & 7)); A rows past M repeat row M - 1
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int tr = 8 * (4 * w + i) + (lane >> 3);
                const int c = (lane & 7) ^ ((tr >> 1) & 7);
                ga[i] = (uint32_t)min(m0 + tr, a.M - 1) * (uint32_t)a.lda * 2u + 2u * k0 + 16u * c;
                if constexpr (!Q) gb[i] = (uint32_t)(n0 + tr) * (uint32_t)a.K * 2u + 2u * k0 + 16u * c;
            }
            if constexpr (Q) {
                // int8 W: instruction i of wave w fills rows 16 (2 w + i) .. + 15,
                // 4 lanes a row (slot lane % 4 holds chunk slot ^ ((row >> 2) & 3))
                const int nr = lane >> 2, nc = (lane & 3) ^ ((lane >> 4) & 3);
#pragma unroll
                for (int i = 0; i < 2; i++) gb[i] = (uint32_t)(n0 + 16 * (2 * w + i) + nr) * (uint32_t)a.K + k0 + 16u * nc;
                so = 4u * ((k0 / LTX_GROUP) * (uint32_t)a.N + (uint32_t)(n0 + wn + lane));
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = f32x4{0, 0, 0, 0};
            // tiles 0 and 1 landed (tile 2 in flight), both steps of tile 0 read,
            // its step 0 multiplied; the barrier frees stage 0 for tile 3
            dma<0>(0);
            dma<1>(1);
            dma<2>(min(2, nk - 1));
            wait_vm_lds(true);
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            read_all<0, 0>(fa0, fw0, sc0);
            read_all<0, 1>(fa1, fw1, sc1);
            {
                V8 xb[4];
                // step 0's scale words and W fragments landed (12 reads after them)
                __builtin_amdgcn_s_waitcnt(Q8_WAIT_LGKM(12));
                __builtin_amdgcn_sched_barrier(0);
                operands(fw0, sc0, xb);
#pragma unroll
                for (int m = 0; m < 16; m++) mfma1(m, fa0, xb);
            }
#pragma unroll
            for (int j = 0; j < 4; j++) sc1[j] = sc0[j];
            meet_lds();
            int k = 0;
            for (; k + 3 < nk; k += 3) {
                pair<0>(k, nk);
                pair<1>(k + 1, nk);
                pair<2>(k + 2, nk);
            }
            // nk - 1 - k (0, 1 or 2) pairs left, then tile nk - 1 step 1
            if (k + 1 < nk) pair<0>(k, nk);
            if (k + 2 < nk) pair<1>(k + 1, nk);
            {
                V8 xb[4];
                operands(fw1, sc1, xb);
#pragma unroll
                for (int m = 0; m < 16; m++) mfma1(m, fa1, xb);
            }
            // every wave past this barrier has finished its MFMAs and its DMA
            // (the repeats of tile nk - 1): the stages are free
            wait_vm_lds(false);
            meet_lds();
            const int el = opaque_tid() & 63;
            auto fill = [&](int b, float* p, int LD) {
#pragma unroll
                for (int e = 0; e < 2; e++)
#pragma unroll
                    for (int j = 0; j < 4; j++)
#pragma unroll
                        for (int r = 0; r < 4; r++)
                            p[(16 * e + 4 * (el >> 4) + r) * LD + 16 * j + (el & 15)] = acc[2 * b + e][j][r];
            };
            if (ks_n > 1)
                gemm_store_partial_patch<2, 2>(fill, (float*)patch, a.part + (size_t)ks * a.M * a.N, a.M, a.N, m0 + wm,
                                               n0 + wn);
            else
                gemm_epilogue_patch<T, EPI, 2, 2, decltype(fill)>(a, fill, (float*)patch, m0 + wm, n0 + wn, n0);
            // every patch has been read back before the next tile's DMA (the
            // epilogue's global stores may still be in flight: the next tile's
            // first wait covers them)
            meet_lds();
        }
    }
};

#define S4_GEMM_KERNEL(NAME, T_, BK_, EPI_)                                          \
    extern "C" __global__ void __launch_bounds__(256, 2) NAME(const LtxGemmArgs a) { \
        S4Gemm<T_, BK_, EPI_> k(a);                                                  \
        k.run();                                                                     \
    }
