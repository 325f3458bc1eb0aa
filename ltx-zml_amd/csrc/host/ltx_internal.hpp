// Internal declarations of the host runtime (not part of the C ABI).
#pragma once
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "../ltx_args.h"
#include "ltx_block.h"

namespace ltx {

// Error carried across internal calls; converted to a status + message at
// the C boundary and never propagated through it.
struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// Checked HIP call, with the LTX_FAIL_AFTER fault-injection counter.
void hip_check(hipError_t e, const char* what);
// LTX_FAIL_CAPTURE=1 (fault injection, like LTX_FAIL_AFTER; read at every
// call): a block forward being captured into a graph throws right after it
// forks its second stream into the capture, so that the capture's error path
// can be tested.
bool fail_in_capture();
#define HIPC(x) ::ltx::hip_check((x), #x)

// A device allocation owned by the runtime.
struct DevBuf {
    void* p = nullptr;
    size_t bytes = 0;
    void alloc(size_t n);
    void free_();
    ~DevBuf() { free_(); }
    DevBuf() = default;
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
};

struct ProfRec {
    const char* name;
    hipEvent_t a, b;
};

}  // namespace ltx

// One projection's weights on device, in the form the kernels consume.
struct LtxProj {
    int N = 0, K = 0;
    bool q8 = false;          // int8 + scales available
    bool qflip = false;       // q holds the bytes q + 128 (q XOR 0x80)
    int scale_f16 = 0;
    ltx::DevBuf q;            // int8 [N][K]
    ltx::DevBuf s;            // [N][K/128] f32 or f16
    ltx::DevBuf s2;           // scale words u32 [K/128][N]: an f16 scale in both halves, or f32 bits
    ltx::DevBuf w_bf16;       // bf16 [N][K] (base tensor)
    ltx::DevBuf w_f16;        // f16 copy of the base tensor (F16 mode, non-q8)
    ltx::DevBuf bias;         // f32 [N] (may be empty)
};

struct ltx_block_weights {
    LtxProj qkv1;             // q1 | k1 | v1, N = 12288
    LtxProj o1;
    LtxProj q2;
    LtxProj kv2;              // k2 | v2, N = 8192
    LtxProj o2;
    LtxProj f1, f2;
    LtxProj g1, g2;           // gate logits, N = 32 (16-bit only)
    ltx::DevBuf qn1, kn1, qn2, kn2;  // f32 [4096]
    ltx::DevBuf sst, psst;    // f32 [9][4096], [2][4096]
    float f16_max = 0.0f;     // largest |weight operand| of mode F16 (above 65504: refused in F16)
    // async blob uploads: the count of unquantised weights whose f16 copy is
    // not finite, formed on the device (u64; unallocated for host uploads,
    // whose f16_max covers them); an F16 forward adds it to the range guard
    ltx::DevBuf f16_over;
    // f32-mode views of the fused projections' parts (bf16 originals / q8)
    uint64_t bytes = 0;
};

struct ltx_ctx {
    int device = 0;
    // kernel selection: the int8 GEMM's LDS-DMA ping-pong kernel (true) or
    // the register-staged one; the ping-pong attention for whole 64-key tiles
    // (true) or the any-length kernel everywhere; for 64-256 keys the
    // resident-K/V form of the ping-pong kernel (true) or its streaming form
    // (all kept for testing)
    bool gemm_dma = true;
    // the four-wave 16-bit GEMM (int8 projections dequantised per forward):
    // 0 never, 1 where its tiles fill the CUs (M >= 4,096 and no split-K),
    // 2 wherever the shape allows (tests)
    int gemm_x4 = 1;
    // the small-grid GEMM (128 x 128 tiles): 0 never, 1 for int8 weights
    // where the 256 x 256 kernels would split K over at most 4,096 (M below
    // 4,096), 2 wherever the shape allows (tests)
    int gemm_s4 = 1;
    int num_cu = 256;             // compute units: the persistent GEMM's grid bound
    bool gemm_persistent = true;  // LDS-DMA GEMM: at most one workgroup per CU, looping over tiles
    bool attn_pp = true;
    bool attn_kv = true;
    // side stream of a forward: work off the main chain (gate logits, the
    // cross-attention K/V) overlaps it, ordered by the events
    hipStream_t side = nullptr;
    hipEvent_t side_ev[5] = {};
    // the small-T schedule of the side stream (block forward): 0 never, 1
    // below kEarlySideRows tokens, 2 at every size (tests)
    int side_early = 1;
    // markers recorded after each launch inside a MarkScope (see launch),
    // cycled; no timing, no system-scope fence
    hipEvent_t marks[16] = {};
    unsigned mark_i = 0;
    bool marks_on = false;
    std::vector<hipModule_t> modules;
    std::map<std::string, hipFunction_t> fns;
    std::string err;
    // workspace
    ltx::DevBuf ws;
    ltx::DevBuf range_ctr;  // range guard: 16-bit stores out of range (u64), see ltx_range_count
    ltx::DevBuf op_pairs;  // scale pairs of the last ltx_op_linear_q8 call (f16 scales)
    ltx::DevBuf op_q;      // its weights as bytes q + 128
    ltx::DevBuf op_w16;    // and dequantised to 16 bits (four-wave GEMM)
    ltx::DevBuf blob_stage;  // device copy of the blob image of the last streaming upload
    ltx::DevBuf core_ws;   // conditioning MLP rows
    ltx::DevBuf tail_ws;   // normed rows of ltx_core_tail
    ltx::DevBuf dn_ws;     // the denoising loop's activations
    size_t ws_T = 0, ws_S = 0;
    int ws_mode = -1;
    int ws_pins = 0;  // live block graphs: their kernels hold workspace addresses
    void* stage_ptr[LTX_ST_COUNT] = {};
    uint64_t stage_bytes[LTX_ST_COUNT] = {};
    // profiling
    bool prof = false;
    std::vector<ltx::ProfRec> prof_recs;
    std::vector<hipEvent_t> ev_pool;
    hipFunction_t fn(const char* name);
    // `label` names the launch in the event profile (defaults to the kernel name).
    void launch(const char* name, unsigned gx, unsigned gy, unsigned gz, unsigned bx, void* args, hipStream_t st,
                const char* label = nullptr);
};

namespace ltx {
// Markers after each launch for the duration of a scope: the stretch of a
// block forward (from 8,192 tokens) in which the second stream's gate logits
// run beside the context k|v GEMM (ltx_ctx::launch).
struct MarkScope {
    ltx_ctx* c;
    bool prev;
    MarkScope(ltx_ctx* ctx, bool on) : c(ctx), prev(ctx->marks_on) { c->marks_on = on; }
    ~MarkScope() { c->marks_on = prev; }
    MarkScope(const MarkScope&) = delete;
    MarkScope& operator=(const MarkScope&) = delete;
};
constexpr int kMarkRows = 8192;
// below this many tokens the block's GEMM and attention grids leave CUs idle:
// the side stream starts at the first RMSNorm + modulate (block_forward)
constexpr int kEarlySideRows = 4096;

void set_thread_error(const std::string& e);
void block_forward(ltx_ctx* c, const ltx_block_weights* w, const float* x, const float* tstab, int K,
                   const int32_t* tidx, const float* ctxv, int S, const float* pts2, const float* cs,
                   const float* sn, int T, float* y, int mode, hipStream_t st);
uint16_t f32_to_f16_bits(float f);
float bf16_bits_to_f32(uint16_t b);
float f16_bits_to_f32(uint16_t h);

// Device scratch of the isolated int8 GEMM: the weights as bytes q + 128
// (N * K bytes) and the scale words [K/128][N] (4 N K / 128 bytes).
struct LinearScratch {
    uint32_t* q;
    uint32_t* pairs;
    void* w16 = nullptr;  // N * K 16-bit weights for the four-wave GEMM, or NULL (the W8A16 kernel)
};
// Whether the four-wave 16-bit GEMM takes an M x N x K product with A rows of
// lda elements (shape, 32-bit buffer offsets and the context's setting).
bool x4_shape(const ltx_ctx* c, int mode, int M, int N, int K, int lda);
// Whether the small-grid GEMM takes it (q8: int8 weights, else 16-bit).
bool s4_shape(const ltx_ctx* c, int mode, int M, int N, int K, int lda, bool q8);
// Shape and mode checks of the isolated int8 GEMM (throws Error), made before
// any scratch is sized from N and K.
void check_linear_q8(int M, int N, int K, int mode);
bool linear_q8_needs_scratch(const ltx_ctx* c, int N, int K, int mode);
void linear_q8(ltx_ctx* c, const void* a, const int8_t* q, const void* scales, int scale_f16, const float* bias,
               void* y, int out_f32, int M, int N, int K, int gelu, int mode, const LinearScratch& sc,
               hipStream_t st);

// The static scratch array of ltx_op_linear_q8_noalloc (ltx_noalloc.hip):
// noalloc_setup resolves its address on `device` (which must be current),
// once per device; noalloc_scratch returns it (NULL before setup).
void noalloc_setup(int device);
void* noalloc_scratch(int device);
}  // namespace ltx

// Runs a body at the C boundary: exceptions become LTX_FAIL + error text.
#define LTX_GUARD(ctxp, ...)                                    \
    try {                                                       \
        __VA_ARGS__;                                            \
        return LTX_OK;                                          \
    } catch (const std::exception& ex) {                        \
        if (ctxp) (ctxp)->err = ex.what();                      \
        ::ltx::set_thread_error(ex.what());                     \
        return LTX_FAIL;                                        \
    } catch (...) {                                             \
        if (ctxp) (ctxp)->err = "unknown C++ exception";        \
        ::ltx::set_thread_error("unknown C++ exception");       \
        return LTX_FAIL;                                        \
    }
