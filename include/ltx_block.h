/*
 * ltx_block.h — C ABI of the MI355X-native LTX-2.5 DiT block forward.
 *
 * Drop-in for the one hot path the reference builds with ZML/XLA: the int8
 * block QBlock.qBlockOutAll (ltx/block.zig:544-574) and its f32 twin
 * Block.wBlockOut (ltx/block.zig:351-353), the packed int8-g128 blob format
 * (tools/pack_block.py, tools/quantize_block.py) and the streaming loader
 * (ltx/loader.zig).
 *
 * Conventions follow the reference's only C ABI (coli-zml/coli/abi.zig:1-10):
 *   - every entry point returns an int status, NON-ZERO = success (LTX_OK);
 *   - C++ exceptions never cross this boundary;
 *   - objects are opaque handles; error text via ltx_last_error();
 *   - fault injection: environment LTX_FAIL_AFTER=N makes the N-th checked
 *     HIP runtime call of the process fail, so every HIP-error path can be
 *     driven from the host.
 * All tensors are device pointers owned by the caller unless stated; calls
 * are asynchronous on the given stream (NULL = the null stream). A context is
 * not thread-safe (one consumer thread, as in ltx/e2e_prod.zig:382-399).
 */
#ifndef LTX_BLOCK_H
#define LTX_BLOCK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LTX_OK 1
#define LTX_FAIL 0

/* Model geometry (ltx/block.zig:14-18). */
#define LTX_DIM 4096
#define LTX_HEADS 32
#define LTX_HEAD_DIM 128
#define LTX_FF_DIM 16384

/* Arithmetic modes. F16/BF16: 16-bit MFMA operands, f32 accumulation, f32
 * residual stream, norms, AdaLN values and softmax statistics. F32: f32
 * everywhere (the reference graph's own precision). */
enum { LTX_MODE_F16 = 0, LTX_MODE_BF16 = 1, LTX_MODE_F32 = 2 };

typedef struct ltx_ctx ltx_ctx;
typedef struct ltx_block_weights ltx_block_weights;

/* Base weight tensors in WEIGHT_SPECS order (ltx/block.zig:377-406): bf16
 * except sst [9][4096] and psst [2][4096] (f32). */
enum {
    LTX_W_Q1_W, LTX_W_Q1_B, LTX_W_K1_W, LTX_W_K1_B, LTX_W_V1_W, LTX_W_V1_B, LTX_W_O1_W, LTX_W_O1_B,
    LTX_W_QN1, LTX_W_KN1, LTX_W_G1_W, LTX_W_G1_B, LTX_W_Q2_W, LTX_W_Q2_B, LTX_W_K2_W, LTX_W_K2_B,
    LTX_W_V2_W, LTX_W_V2_B, LTX_W_O2_W, LTX_W_O2_B, LTX_W_QN2, LTX_W_KN2, LTX_W_G2_W, LTX_W_G2_B,
    LTX_W_FF1_W, LTX_W_FF2_W, LTX_W_SST, LTX_W_PSST, LTX_W_COUNT
};

/* int8 companions in Q8_SPECS order (ltx/loader.zig:147-156), plus the two
 * output projections (tools/quantize_block.py:23, class "out"). */
enum { LTX_Q_Q1, LTX_Q_K1, LTX_Q_V1, LTX_Q_Q2, LTX_Q_K2, LTX_Q_V2, LTX_Q_F1, LTX_Q_F2, LTX_Q_O1, LTX_Q_O2, LTX_Q_COUNT };

/* ---- context ----------------------------------------------------------- */

/* Select `device`, load the gfx950 code objects (hipModuleLoadData), create
 * the context. Replaces zml.Platform.auto + platform.compile
 * (ltx/e2e_prod.zig:187-189, 297-299). */
int ltx_init(int device, ltx_ctx** out);
void ltx_destroy(ltx_ctx* ctx);
/* Last error of `ctx`, or of the calling thread when ctx is NULL. */
const char* ltx_last_error(const ltx_ctx* ctx);
/* Library / code-object build identification. */
const char* ltx_version(void);

/* ---- weights ----------------------------------------------------------- */

/* Upload one block from a blob image laid out per its manifest
 * (ltx/loader.zig:133-172, buildBlockBufs + buildQuantBufs): entries are
 * found by normalised name "transformer_blocks_{i}_{stem}[_q8|_q8scale]"
 * (ltx/loader.zig:100-129). `mem` is the blob bytes (an mmap or a ring slot),
 * `manifest_json` the text of blob_manifest.json. q8scale entries may be F32
 * (the reference format) or F16. Missing q8 entries fall back to the bf16
 * base weight for that projection. Entries must lie inside `mem` at offsets
 * that are multiples of the manifest's alignment, and F32 scales must be
 * finite with magnitude below 2^100 (error "ScaleRange"; absmax / 127 of any
 * bf16 weight below 1e32 is). */
int ltx_block_weights_from_blob(ltx_ctx* ctx, const void* mem, uint64_t mem_bytes, const char* manifest_json,
                                int64_t block_idx, ltx_block_weights** out);

/* Streaming form of ltx_block_weights_from_blob for a ring consumer
 * (ltx/loader.zig:133-172 and the ring of :176-321, with one DMA per blob):
 * enqueues on `stream` one hipMemcpyAsync of the whole blob image `mem`
 * (pinned host memory such as a ring slot, for the copy to be asynchronous)
 * into the context's staging buffer, then kernels that carve it into the
 * device form (fused projections, weights as q + 128, scale pairs, widened
 * biases and norm weights), and returns at once. The manifest is parsed and
 * checked on the host first, with the same errors as the synchronous call.
 * `reuse`: NULL for a new handle, or a handle of the same layout whose
 * buffers are overwritten with no allocation (the caller orders this after
 * the last kernel reading it). The caller keeps `mem` unchanged until
 * `stream` has passed this call (record an event after it), and does not run
 * two streaming uploads of one context on different streams at once (they
 * share the staging buffer). */
int ltx_block_weights_from_blob_async(ltx_ctx* ctx, const void* mem, uint64_t mem_bytes, const char* manifest_json,
                                      int64_t block_idx, ltx_block_weights* reuse, void* stream,
                                      ltx_block_weights** out);

/* Upload one block from host pointers: base[LTX_W_COUNT] (bf16 bits / f32),
 * q8[LTX_Q_COUNT] int8 [O][I] or NULL, q8s[LTX_Q_COUNT] scales [O][I/128]
 * (f32, or f16 when scale_f16). */
int ltx_block_weights_from_host(ltx_ctx* ctx, const void* const* base, const int8_t* const* q8,
                                const void* const* q8s, int scale_f16, ltx_block_weights** out);
void ltx_block_weights_free(ltx_ctx* ctx, ltx_block_weights* w);
/* Device bytes held by one uploaded block. */
uint64_t ltx_block_weights_bytes(const ltx_block_weights* w);

/* ---- the block forward ------------------------------------------------- */

/* y = QBlock.qBlockOutAll(x, tstab, tidx, ctx, pts2, cos, sin)
 * (ltx/block.zig:544-574), self-attention blockwise (ltx/block.zig:105-154).
 *   x      [T][4096] f32         tstab [K][9][4096] f32   tidx [T] i32
 *   ctx_tokens [S][4096] f32     pts2  [2][4096] f32
 *   cos, sin [T][32][64] f32 (graph layout, ltx/block_conformance.zig:255-267)
 *   y      [T][4096] f32 (may not alias x)
 * Argument order follows the reference method (ltx/e2e_prod.zig:238-247). */
int ltx_block_forward(ltx_ctx* ctx, const ltx_block_weights* w, const float* x, const float* tstab, int K,
                      const int32_t* tidx, const float* ctx_tokens, int S, const float* pts2, const float* cos,
                      const float* sin, int T, float* y, int mode, void* stream);

/* The same forward captured once and replayed: the pair the reference's
 * caller uses, platform.compile binding the method into an executable
 * (ltx/e2e_prod.zig:297-299) and exe.call per block (ltx/e2e_prod.zig:377-399),
 * here as a HIP graph with the buffers bound at creation.
 * ltx_block_graph_create runs no kernel: it sizes the context's workspace and
 * records one ltx_block_forward with these arguments (same meanings) into a
 * graph. ltx_block_graph_launch enqueues that forward on `stream` with one
 * host call, asynchronously, with the same results bit for bit (measured:
 * no faster than ltx_block_forward at 28,672 tokens; for callers that
 * replay or capture).
 * The graph binds the weights, every buffer and the context's workspace:
 * they must outlive it, and while a graph lives, a forward on the context
 * that needs a larger workspace fails. Launches share the workspace with
 * every other forward on the context: in order on one stream, racing on
 * different streams. Event profiling must be off at creation, and graph
 * launches are not profiled. After a launch, ltx_block_stage reads the
 * intermediates of the captured forward. Destroy graphs before their
 * context. */
typedef struct ltx_block_graph ltx_block_graph;
int ltx_block_graph_create(ltx_ctx* ctx, const ltx_block_weights* w, const float* x, const float* tstab, int K,
                           const int32_t* tidx, const float* ctx_tokens, int S, const float* pts2, const float* cos,
                           const float* sin, int T, float* y, int mode, ltx_block_graph** out);
int ltx_block_graph_launch(ltx_block_graph* g, void* stream);
void ltx_block_graph_destroy(ltx_block_graph* g);

/* Intermediate tensors of the last forward, for staged parity checks
 * (the staged methods of ltx/block.zig:248-338), and the velocity of the last
 * ltx_denoise step (ltx/e2e_denoise.zig:314 gates it per step). Device
 * pointer + bytes, valid until the next forward on this context; a stage the
 * last call did not produce reads NULL / 0. */
enum {
    LTX_ST_NORM_MSA,    /* s1NormMsa: modulated norm, operand dtype [T][4096] */
    LTX_ST_Q1,          /* normed+roped q times log2(e)/sqrt(128), [T][4096] (f32 mode: unscaled) */
    LTX_ST_K1,          /* normed+roped k, same layout */
    LTX_ST_V1,          /* v: [32][128][T] (f32 mode: [T][4096]) */
    LTX_ST_GLOG1,       /* gate logits [T][32] f32 */
    LTX_ST_ATTN1,       /* gated merged attention before out-proj [T][4096] */
    LTX_ST_X_SA,        /* s4AfterSa [T][4096] f32 */
    LTX_ST_ATTN_IN,     /* cross-attention query input [T][4096] */
    LTX_ST_ATTN2,       /* gated merged cross-attention [T][4096] */
    LTX_ST_X_CA,        /* x after cross-attention [T][4096] f32 */
    LTX_ST_FF_IN,       /* s6FfIn [T][4096] */
    LTX_ST_FF_H,        /* gelu(ff1) [T][16384] */
    LTX_ST_GLOG2,       /* cross-attention gate logits [T][32] f32 */
    LTX_ST_Q2,          /* normed cross q times log2(e)/sqrt(128), [T][4096] (f32 mode: unscaled) */
    LTX_ST_K2,          /* normed cross k [S][4096] */
    LTX_ST_V2,          /* cross v: [32][128][S] (f32 mode: [S][4096]) */
    LTX_ST_VELOCITY,    /* ltx_denoise: the last step's velocity [T][128] f32 */
    LTX_ST_COUNT
};
int ltx_block_stage(ltx_ctx* ctx, int stage, void** dev_ptr, uint64_t* bytes);

/* Range guard of the 16-bit modes. The reference computes in f32; here the
 * MFMA operands (the modulated norms, Q, K, V, the attention outputs, the
 * GELU hidden, the modulated context) are stored as f16 (LTX_MODE_F16) or
 * bf16. Every block forward in those modes counts, on the device, the values
 * it stored in 16 bits that were not finite or beyond the type's largest
 * finite value (65504 for f16), in a counter of the context that accumulates
 * over forwards (and ltx_denoise) until reset. This call waits for `stream`,
 * returns the count and, when `reset`, sets it to 0 (the context starts at
 * 0). A non-zero count means some activation left the 16-bit range: rerun in
 * LTX_MODE_BF16 (the f32 exponent range) or LTX_MODE_F32. Weight operands
 * are checked at upload instead: a forward in LTX_MODE_F16 refuses a block
 * whose dequantised weights (128 |s|) or f16 copies exceed 65504. Weights
 * from ltx_block_weights_from_blob_async are checked the same way except the
 * f16 copies of unquantised projections, which are made on the device: the
 * copies that are not finite are counted there, and every LTX_MODE_F16
 * forward with those weights adds that count to this counter. */
int ltx_range_count(ltx_ctx* ctx, void* stream, uint64_t* count, int reset);

/* ---- isolated operators (the microbenchmark surface, ltx/smoke.zig) ---- */

/* y[M][N] = a[M][K] . dq4(q, s)^T (+ bias) with optional GELU-tanh.
 * a: 16-bit [M][K] (mode F16/BF16) or f32 (mode F32); q int8 [N][K];
 * scales [N][K/128] f32 or f16 (f32: finite, magnitude below 2^100, not
 * checked here); y f32 (out_f32) or 16-bit. Mirrors linQ
 * (ltx/block.zig:473-477). In the 16-bit modes with N a multiple of 256 the
 * call first lays the weights out as bytes q + 128 and the scales as words
 * [K/128][N] in scratch the context owns (allocated on first use, grown as
 * needed) and then runs the GEMM, all on `stream`: two calls of one context on
 * different streams may overwrite each other's scratch, so keep one context's
 * calls on one stream. A shape with M, N or K not positive or K not a
 * multiple of 128, or an unknown mode, is refused (status 0, ltx_last_error)
 * before any scratch is sized or allocated. */
int ltx_op_linear_q8(ltx_ctx* ctx, const void* a, const int8_t* q, const void* scales, int scale_f16,
                     const float* bias, void* y, int out_f32, int M, int N, int K, int gelu, int mode,
                     void* stream);

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): ltx_op_linear_q8 with the same arguments and results,
 * calling no hipMalloc / hipFree. Its scratch (the weights as bytes q + 128,
 * N * K bytes rounded up to 256, then the scale words, 4 N K / 128 bytes,
 * and for the shapes ltx_op_linear_q8 runs on the four-wave GEMM, from 4,096
 * rows, the weights dequantised to the operand type, 2 N K bytes) is
 * a static device array of LTX_NOALLOC_SCRATCH_BYTES on each GPU the library
 * runs on, held until the process ends; a shape needing more is refused with
 * an error. The kernels write all of the scratch they read on each call, so
 * nothing carries over between calls, but every call on one GPU shares the
 * array: calls that overlap on one GPU (other streams, contexts or threads)
 * race. */
#define LTX_NOALLOC_SCRATCH_BYTES (66u << 20)
int ltx_op_linear_q8_noalloc(ltx_ctx* ctx, const void* a, const int8_t* q, const void* scales, int scale_f16,
                             const float* bias, void* y, int out_f32, int M, int N, int K, int gelu, int mode,
                             void* stream);

/* Attention with per-(token, head) gate (gate logits glog [Lq][32] f32, or
 * NULL for no gate). F16/BF16: q, k [32][L][128] 16-bit, vt [32][128][Lkv]
 * 16-bit, out [Lq][4096] 16-bit. F32: q, k, v, out [L][4096] f32.
 * mode | LTX_ATTN_Q_SCALED (16-bit modes): q already holds
 * q * log2(e) / sqrt(128), as the block's qk-norm writes it (LTX_ST_Q1). */
#define LTX_ATTN_Q_SCALED 0x100
int ltx_op_attention(ltx_ctx* ctx, const void* q, const void* k, const void* v, const float* glog, void* out,
                     int lq, int lkv, int mode, void* stream);

/* Dequantisation probe: out32 = f32(q) * s (bit-exact dq4, ltx/block.zig:
 * 462-471) and out16 = that value rounded to the mode's operand type. */
int ltx_op_dequant(ltx_ctx* ctx, const int8_t* q, const void* scales, int scale_f16, int N, int K, float* out32,
                   void* out16, int mode, void* stream);

/* ---- host utilities ---------------------------------------------------- */

/* 3D RoPE tables, host f64 (ltx/block_conformance.zig:87-126). grid
 * [3][T][2] f32 (start, end); outputs f32 in the bundle layout [32][T][64]
 * when graph_layout == 0, or the graph layout [T][32][64] when 1. */
int ltx_rope_tables(const float* grid, int T, float* cos_out, float* sin_out, int graph_layout);

/* Per-kernel timing with HIP events on the launch stream. */
int ltx_profile_enable(ltx_ctx* ctx, int enable);
/* Total milliseconds and launch count of kernels whose name contains
 * `substr` (all recorded launches when substr is NULL or empty). Synchronises. */
int ltx_profile_read(ltx_ctx* ctx, const char* substr, double* total_ms, int* count);
int ltx_profile_reset(ltx_ctx* ctx);

/* ---- parts around the blocks (ltx/core_parts.zig) ---------------------- */

#define LTX_IN_CH 128 /* latent channels (ltx/core_parts.zig:15) */

typedef struct ltx_core_weights ltx_core_weights;

/* Core tensors in CORE_SPECS order (ltx/core_parts.zig:53-72): bf16 bits
 * [O][I] / [O], except fsst, f32 [2][4096]. */
enum {
    LTX_C_ADA_L1_W, LTX_C_ADA_L1_B, LTX_C_ADA_L2_W, LTX_C_ADA_L2_B, LTX_C_ADA_OUT_W, LTX_C_ADA_OUT_B,
    LTX_C_PADA_L1_W, LTX_C_PADA_L1_B, LTX_C_PADA_L2_W, LTX_C_PADA_L2_B, LTX_C_PADA_OUT_W, LTX_C_PADA_OUT_B,
    LTX_C_PAT_W, LTX_C_PAT_B, LTX_C_PO_W, LTX_C_PO_B, LTX_C_FSST, LTX_C_COUNT
};

/* Upload the core tensors from host memory (the role of loadCoreBufs,
 * ltx/e2e_denoise.zig:73-84). Weights stay bf16; biases are widened to f32. */
int ltx_core_weights_from_host(ltx_ctx* ctx, const void* const* tensors, ltx_core_weights** out);
void ltx_core_weights_free(ltx_ctx* ctx, ltx_core_weights* cw);

/* CoreParts.ts9r + emb + pts2r (ltx/core_parts.zig:112-141), f32:
 *   t [K] raw timesteps (mask * sigma), sigma [1]   (device pointers)
 *   tstab [K][9][4096], emb [K][4096] (embedded_timestep), pts2 [2][4096]. */
int ltx_core_conditioning(ltx_ctx* ctx, const ltx_core_weights* cw, const float* t, int K, const float* sigma,
                          float* tstab, float* emb, float* pts2, void* stream);
/* CoreParts.patchify (ltx/core_parts.zig:143-145): latent [T][128] -> x [T][4096]. */
int ltx_core_patchify(ltx_ctx* ctx, const ltx_core_weights* cw, const float* latent, int T, float* x, void* stream);
/* CoreParts.tailFromEmb (ltx/core_parts.zig:147-166): LayerNorm, modulation
 * by fsst + emb[tidx[t]], proj_out. x [T][4096] -> vel [T][128]. */
int ltx_core_tail(ltx_ctx* ctx, const ltx_core_weights* cw, const float* x, const float* emb, const int32_t* tidx,
                  int T, float* vel, void* stream);

/* ---- distilled scheduler (ltx/scheduler.zig) ---------------------------- */

/* SIGMAS_STAGE1 (stage 1, 9 values) or SIGMAS_STAGE2 (stage 2, 4 values),
 * ltx/scheduler.zig:15-18. `out` may be NULL to read the count only. */
int ltx_sched_sigmas(int stage, float* out, int* count);
/* noiseInit (ltx/scheduler.zig:37-46) on device, bit-exact: latent [T][C],
 * mask of token t = maskk[tidx[t]]. */
int ltx_sched_noise_init(ltx_ctx* ctx, const float* clean, const float* noise, const float* maskk,
                         const int32_t* tidx, int T, int C, float noise_scale, float* out, void* stream);
/* toDenoised -> postProcess -> eulerStep (ltx/scheduler.zig:53-80) fused,
 * bit-exact: ts of token t = tk[tidx[t]], mask maskk[tidx[t]]. out may
 * equal x. */
int ltx_sched_step(ltx_ctx* ctx, const float* x, const float* vel, const float* tk, const float* maskk,
                   const int32_t* tidx, const float* clean, int T, int C, float sigma, float sigma_next, float* out,
                   void* stream);

/* The denoising loop (ltx/e2e_denoise.zig:218-336; one pass: ltx/e2e_prod.zig:302-430):
 * per step, timesteps -> ts9r/emb/pts2r -> patchify -> every block ->
 * tail -> scheduler step, with the latent [T][128] updated in place on the
 * device. sigmas: host array of nsteps + 1 values. K distinct mask values
 * maskk [K] (device), K < 64. blocks: nblocks resident block weights. */
int ltx_denoise(ltx_ctx* ctx, const ltx_block_weights* const* blocks, int nblocks, const ltx_core_weights* cw,
                float* latent, const float* clean, const float* maskk, const int32_t* tidx, int K,
                const float* ctx_tokens, int S, const float* cos, const float* sin, int T, const float* sigmas,
                int nsteps, int mode, void* stream);

#ifdef __cplusplus
}
#endif
#endif
