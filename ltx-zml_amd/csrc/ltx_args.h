// Kernel argument blocks shared by the host orchestrator (g++) and the gfx950
// code objects (hipcc --genco). Every kernel takes exactly one of these by
// value, so hipModuleLaunchKernel passes a single pointer in kernelParams.
// Plain C layout only: pointers, 32/64-bit integers, floats.
#pragma once
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// Range guard: kernels that store 16-bit activations add to *sat the number of
// stored values that are not finite or exceed the type's largest finite value
// (65504 for f16), when sat is not NULL.

// Model geometry of the LTX-2.5 video block (ltx/block.zig:14-18).
#define LTX_D 4096
#define LTX_H 32
#define LTX_HD 128
#define LTX_FF 16384
#define LTX_GROUP 128

// AdaLN gather (ltx/block.zig:47-67): ada_i[t][c] = tstab[row(t)][i][c] + sst[i][c],
// row(t) = tidx[t] when it lies in 1 .. K-1, else 0 (the reference's select
// chain starts from row 0 and replaces it only for k = 1 .. K-1).
typedef struct {
    const float* sst;    // [9][D] per-block table
    const float* tstab;  // [K][9][D] timestep table
    const int32_t* tidx; // [T] row of tstab per token
    int K;               // rows of tstab
} LtxAda;

// Fused RMSNorm + AdaLN modulate: y = rms(x) * (1 + ada[isc]) + ada[ish].
typedef struct {
    const float* x;  // [rows][D] f32
    void* y;         // [rows][D] f16 / bf16 / f32 (by kernel)
    LtxAda ada;
    int rows;
    int ish, isc;    // ada row indices for shift and scale; isc < 0: plain rms
    unsigned long long* sat;  // range guard counter (16-bit outputs) or NULL
    const unsigned long long* sat_add;  // or NULL: a count the first workgroup adds to sat
} LtxNormArgs;

// Cross-attention K/V modulation (ltx/block.zig:553-556):
// enc = ctx * (1 + (psst[1] + pts2[1])) + (psst[0] + pts2[0]).
typedef struct {
    const float* ctx;   // [S][D]
    const float* psst;  // [2][D]
    const float* pts2;  // [2][D]
    void* y;            // [S][D]
    int rows;
    unsigned long long* sat;  // range guard counter (16-bit outputs) or NULL
} LtxEncArgs;

// Epilogue kinds of the W8A16 / W16A16 GEMM.
enum {
    LTX_EPI_STORE = 0,      // y = acc (+ bias); out f32 or 16-bit; optional GELU
    LTX_EPI_RESID_GATE = 1, // out32 = resid + (acc (+ bias)) * ada[igate]
    LTX_EPI_QKV = 2,        // cols < nsplit: 16-bit [M][nsplit] (+bias); cols >= nsplit: 16-bit V^T [H][HD][M]
};

// B operand kinds.
enum {
    LTX_B_I8_F32S = 0,  // int8 [N][K] + f32 scales [N][K/128]
    LTX_B_I8_F16S = 1,  // int8 [N][K] + f16 scales [N][K/128]
    LTX_B_W16 = 2,      // 16-bit weights [N][K] in the operand type
};

typedef struct {
    const void* a;        // [M][K] activations, row stride lda (elements)
    const void* b;        // [N][K] weights (int8 or 16-bit), row stride K
    const void* scales;   // [N][K/128] f32 or f16 (int8 kinds)
    const float* bias;    // [N] or NULL
    void* out;            // output (meaning per epilogue)
    const float* resid;   // [M][N] f32 residual (RESID_GATE)
    void* out2;           // V^T output (QKV)
    LtxAda ada;           // RESID_GATE gate table
    int M, N, K;
    int lda;
    int ldo;              // output row stride (elements)
    int nsplit;           // QKV: first V column
    int igate;            // RESID_GATE ada row
    int gelu;             // STORE: apply GELU-tanh
    int out_f32;          // STORE: 1 = f32 output, 0 = 16-bit output
    int tiles_m, tiles_n; // grid geometry (filled by host)
    uint32_t qxor;        // int8 kinds: XOR taking each weight byte to q + 128 (0x80808080 for plain int8,
                          // 0 for bytes stored as q + 128); the LDS-DMA kernels take the latter only
    unsigned long long* sat;  // range guard counter of the 16-bit outputs (V^T, 16-bit stores) or NULL
    int ksplit;           // split-K (LDS-DMA kernel): 1, or S slices of K / S each, whose f32 partial sums
    float* part;          // go to part [S][M][N] for ltx_gemm_reduce_* to finish with the epilogue
} LtxGemmArgs;

// Dequantisation of int8 projections into 16-bit weights for the four-wave
// 16-bit GEMM: out[j] [N][K] = the W8A16 kernel's operands, from the bytes
// q + 128 [N][K] and the scale words [K / 128][N]. Workgroups start[j] ..
// start[j + 1] - 1 cover job j, 32 rows of one 128-k group each.
#define LTX_DQ_JOBS 8
typedef struct {
    const uint8_t* q[LTX_DQ_JOBS];
    const uint32_t* s2[LTX_DQ_JOBS];
    void* out[LTX_DQ_JOBS];
    int N[LTX_DQ_JOBS], K[LTX_DQ_JOBS];
    int start[LTX_DQ_JOBS + 1];
    int njobs;
} LtxDq16Args;

// Full-row qk RMSNorm (weighted, over all 4096 channels) + optional split-half
// RoPE, writing 16-bit rows [rows][D] (head h at columns h * HD ..), the
// layout of its input: every token's output is one contiguous 8 KB row.
typedef struct {
    const void* x;      // [rows][ldx] pre-norm projections, in the 16-bit operand type
    const float* w;     // [D] norm weight (f32 copy of the bf16 tensor)
    const float* cos;   // [rows][H][64] or NULL (no RoPE)
    const float* sin;
    void* y;            // [rows][D]
    int rows;
    int ldx;
    float oscale;       // applied before the 16-bit rounding (1, or the attention's exponent scale for Q)
    unsigned long long* sat;  // range guard counter or NULL
} LtxQkNormArgs;

// The self-attention's q and k rows of one token in one pass (the RoPE rows
// read once): q = x[row][0 .. D), k = x[row][D .. 2D).
typedef struct {
    const void* x;      // [rows][ldx] q | k, in the 16-bit operand type
    const float* wq;    // [D] norm weights (f32)
    const float* wk;
    const float* cos;   // [rows][H][64]
    const float* sin;
    void* yq;           // [rows][D]
    void* yk;
    int rows;
    int ldx;
    float oscale_q, oscale_k;
    unsigned long long* sat;  // range guard counter or NULL
} LtxQkNorm2Args;

// Blockwise online-softmax attention with per-(token, head) gate.
// q, k: 16-bit, element (h, l, d) at h * hs + l * rs + d: head-major
// [H][L][HD] (hs = L HD, rs = HD) or token rows [L][D] (hs = HD, rs = D);
// vt: [H][HD][Lkv] 16-bit; glog: [Lq][H] f32 gate logits (gate =
// 2*sigmoid); out: [Lq][D] 16-bit merged heads.
typedef struct {
    const void* q;
    const void* k;
    const void* vt;
    const float* glog;
    void* out;
    int lq, lkv;
    int q_hs, q_rs;     // element strides of q: head, row
    int k_hs, k_rs;     // of k
    float scale_log2;   // softmax scale * log2(e)
    int q_tiles;        // ceil(lq / q-tile)
    unsigned long long* sat;  // range guard counter of the 16-bit output or NULL
} LtxAttnArgs;

// Gate logits: glog[t][h] = a[t] . gw[h] + gb[h] (N = 32 heads).
typedef struct {
    const void* a;      // [M][D] 16-bit
    const void* gw;     // [H][D] 16-bit
    const float* gb;    // [H]
    float* out;         // [M][H]
    int M;
} LtxGateArgs;

// Dequantisation probe: out[n][k] = f32(q[n][k]) * scale[n][k/128], exactly
// as the GEMM's in-register dequant computes it before the 16-bit rounding.
typedef struct {
    const int8_t* q;
    const void* scales;
    float* out32;       // f32 value
    void* out16;        // the 16-bit MFMA operand
    int N, K;
    int scale_f16;
} LtxDequantArgs;

// bf16 -> f32 (to_f16 = 0) or f16 (to_f16 = 1, round to nearest even), n
// elements. over (f16 only, or NULL): counts the values whose f16 is not
// finite (beyond 65504, or not finite already).
typedef struct {
    const uint16_t* in;
    void* out;
    size_t n;
    int to_f16;
    unsigned long long* over;
} LtxCvtArgs;

// int8 weights -> bytes q + 128 (XOR 0x80 per byte), n words of 4 bytes.
typedef struct {
    const uint32_t* in;
    uint32_t* out;
    size_t n;
} LtxFlipArgs;

// Scales [N][G] -> scale words u32 [G][N] for the LDS-DMA int8 GEMM: f16
// scales as pairs (s | s << 16), f32 scales (f32 != 0) as their bits.
typedef struct {
    const void* s;
    uint32_t* out;
    int N, G;
    int f32;
} LtxPairArgs;

// f32 reference-precision kernels (mode LTX_MODE_F32).
typedef struct {
    const float* a;     // [M][K]
    const void* b;      // int8 [N][K] or bf16 [N][K]
    const void* scales;
    int bkind;          // 0: int8+f32s, 1: int8+f16s, 2: bf16
    const float* bias;
    float* out;
    const float* resid;
    LtxAda ada;
    int M, N, K;
    int epi;            // LTX_EPI_STORE / RESID_GATE
    int gelu;
    int igate;
    uint32_t qxor;      // int8 kinds: as LtxGemmArgs.qxor
} LtxGemm32Args;

typedef struct {
    const float* q;     // [Lq][D] (roped / normed)
    const float* k;     // [Lkv][D]
    const float* v;     // [Lkv][D]
    const float* glog;  // [Lq][H]
    float* out;         // [Lq][D]
    int lq, lkv;
    float scale;
} LtxAttn32Args;

typedef struct {
    float* x;           // [rows][D] in place
    const float* w;     // [D]
    const float* cos;   // [rows][H][64] or NULL
    const float* sin;
    int rows;
    int ldx;
} LtxQkNorm32Args;

// Parts around the blocks (ltx/core_parts.zig) and the scheduler
// (ltx/scheduler.zig).
typedef struct {
    const float* t;     // [rows] timestep values
    float* out;         // [rows][256]
    int rows;
} LtxSinArgs;

typedef struct {
    const float* x;
    float* y;
    size_t n;
} LtxEltArgs;

typedef struct {
    const float* x;       // [T][D]
    const float* fsst;    // [2][D] (shift row, scale row)
    const float* emb;     // [K][D] embedded timestep per distinct t
    const int32_t* tidx;  // [T]
    float* y;             // [T][D]
} LtxTailNormArgs;

typedef struct {
    const float* x;       // latent [T][stride]
    const float* v;       // velocity [T][stride]
    const float* clean;   // clean latent [T][stride]
    const float* tk;      // [K] mask * sigma
    const float* maskk;   // [K] mask values
    const int32_t* tidx;  // [T]
    float* y;
    size_t n;             // T * stride
    int stride;
    float sigma, sigma_next;
} LtxSchedArgs;

typedef struct {
    const float* clean;
    const float* noise;
    const float* maskk;
    const int32_t* tidx;
    float* y;
    size_t n;
    int stride;
    float noise_scale;
} LtxNoiseArgs;

typedef struct {
    const float* maskk;
    float* tk;
    int K;
    float sigma;
} LtxTimestepArgs;

#ifdef __cplusplus
}
#endif
