// Block forward orchestration: QBlock.qBlockOutAll (ltx/block.zig:544-574)
// as a sequence of gfx950 kernel launches on one stream, plus the isolated
// operator entry points.
#include <cmath>
#include <algorithm>
#include <cstring>
#include <new>

#include "ltx_internal.hpp"

namespace ltx {

static const char* msuffix(int mode) { return mode == LTX_MODE_BF16 ? "bf16" : "f16"; }

static size_t al(size_t n) { return (n + 255) & ~(size_t)255; }

// Bump allocator over the context workspace.
struct Carve {
    char* base;
    size_t off = 0;
    size_t total = 0;
    bool dry;
    void* take(size_t n) {
        void* p = dry ? nullptr : base + off;
        off += al(n);
        return p;
    }
};

struct Ws16 {
    void *n_msa, *qk16, *vt1, *qh1, *kh1, *glog1, *o1, *x_sa, *attn_in, *q2_16, *glog2, *enc, *k2_16, *vt2, *qh2,
        *kh2, *o2, *x_ca, *ff_in, *h, *part, *part2;
    void* dq[6];  // 16-bit weights of qkv1, o1, q2, o2, ff1, ff2 for the four-wave GEMM (NULL: not used)
};

// The projections the four-wave GEMM may take, as (N, K) with A rows of K
// elements and M = T: qkv1, o1, q2, o2, ff1, ff2.
static const int kX4Shapes[6][2] = {{3 * LTX_D, LTX_D}, {LTX_D, LTX_D}, {LTX_D, LTX_D},
                                    {LTX_D, LTX_D},     {LTX_FF, LTX_D}, {LTX_D, LTX_FF}};

// Split-K slices of a GEMM whose 256 x tn output tiles would fill at most
// half the CUs: the largest power of two S <= 8 with tiles * S <= CUs and
// K / S a multiple of 128 of at least 512 (eight K-tiles per slice).
static int gemm_ksplit(int num_cu, int M, int N, int K, int tn = 256, int tm = 256) {
    const int tiles = ((M + tm - 1) / tm) * (N / tn);
    int s = 1;
    while (s < 8 && tiles * s * 2 <= num_cu && K % (256 * s) == 0 && K / (s * 2) >= 512) s *= 2;
    return s;
}

bool x4_shape(const ltx_ctx* c, int mode, int M, int N, int K, int lda) {
    if (mode != LTX_MODE_F16 && mode != LTX_MODE_BF16) return false;
    if (!c->gemm_x4 || !c->gemm_dma) return false;
    if (M <= 0 || N % 256 || K % 128 || lda < K || lda % 8) return false;
    if ((uint64_t)M * lda * 2 >= (1ull << 31) || (uint64_t)N * K * 2 >= (1ull << 31)) return false;
    if (c->gemm_x4 == 2) return true;
    // where its 256 x 256 tiles fill the CUs: the sizes that need no split-K
    return M >= 4096 && gemm_ksplit(c->num_cu, M, N, K) == 1;
}

bool s4_shape(const ltx_ctx* c, int mode, int M, int N, int K, int lda, bool q8) {
    if (mode != LTX_MODE_F16 && mode != LTX_MODE_BF16) return false;
    if (!c->gemm_s4 || !c->gemm_dma) return false;
    if (M <= 0 || N % 128 || K % 128 || lda < K || lda % 8) return false;
    if ((uint64_t)M * lda * 2 >= (1ull << 31) || (uint64_t)N * K * (q8 ? 1 : 2) >= (1ull << 31)) return false;
    if (c->gemm_s4 == 2) return true;
    // int8 weights where the 256 x 256 kernels would split K (their tiles
    // fill at most half the CUs) over at most 4,096: there it needs no
    // split-K reduce (the context k|v projection, the 4096-wide projections
    // below 4,096 rows). With 16-bit weights, or K = 16,384, its 128 x 128
    // tiles (half the flops per byte moved) measured slower than the split
    // 256 x 256 kernels; with no split (q|k|v at 1,024 rows) slower too.
    return q8 && M < 4096 && K <= 4096 && gemm_ksplit(c->num_cu, M, N, K) > 1;
}

// The small-T schedule of the block forward (side stream from the first
// RMSNorm + modulate on).
static bool side_early(const ltx_ctx* c, size_t T) {
    return c->side_early == 2 || (c->side_early == 1 && T < (size_t)kEarlySideRows);
}

static void carve16(Carve& c, Ws16& w, size_t T, size_t S, const ltx_ctx* ctx, int mode) {
    const size_t D = LTX_D;
    const int num_cu = ctx->num_cu;
    w.n_msa = c.take(T * D * 2);
    w.qk16 = c.take(T * 2 * D * 2);
    w.vt1 = c.take(T * D * 2);
    w.qh1 = c.take(T * D * 2);
    w.kh1 = c.take(T * D * 2);
    w.glog1 = c.take(T * LTX_H * 4);
    w.o1 = c.take(T * D * 2);
    w.x_sa = c.take(T * D * 4);
    w.attn_in = c.take(T * D * 2);
    w.q2_16 = c.take(T * D * 2);
    w.glog2 = c.take(T * LTX_H * 4);
    w.enc = c.take(S * D * 2);
    w.k2_16 = c.take(S * D * 2);
    w.vt2 = c.take(S * D * 2);
    w.qh2 = c.take(T * D * 2);
    w.kh2 = c.take(S * D * 2);
    w.o2 = c.take(T * D * 2);
    w.x_ca = c.take(T * D * 4);
    w.ff_in = c.take(T * D * 2);
    w.h = c.take(T * LTX_FF * 2);
    // f32 partial sums of the split-K GEMMs: the largest slices * M * N over
    // the block's seven projections (none at large T)
    size_t part = 0;
    const int shapes[6][3] = {{(int)T, 3 * LTX_D, LTX_D}, {(int)T, LTX_D, LTX_D}, {(int)S, 2 * LTX_D, LTX_D},
                              {(int)T, LTX_FF, LTX_D}, {(int)T, LTX_D, LTX_FF}, {(int)T, LTX_D, LTX_D}};
    for (const auto& sh : shapes) {
        const int k = gemm_ksplit(num_cu, sh[0], sh[1], sh[2]);
        if (k > 1) part = std::max(part, (size_t)k * sh[0] * sh[1] * 4);
    }
    w.part = part ? c.take(part) : nullptr;
    // the context k|v GEMM's own partial sums when it runs on the side
    // stream beside the main chain's split GEMMs
    w.part2 = nullptr;
    if (side_early(ctx, T)) {
        const int k = gemm_ksplit(num_cu, (int)S, 2 * LTX_D, LTX_D);
        if (k > 1) w.part2 = c.take((size_t)k * S * 2 * LTX_D * 4);
    }
    for (int i = 0; i < 6; i++) {
        const int N = kX4Shapes[i][0], K = kX4Shapes[i][1];
        w.dq[i] = x4_shape(ctx, mode, (int)T, N, K, K) ? c.take((size_t)N * K * 2) : nullptr;
    }
}

struct Ws32 {
    void *n_msa, *q, *k, *v, *glog1, *o1, *x_sa, *attn_in, *q2, *enc, *k2, *v2, *glog2, *o2, *x_ca, *ff_in, *h;
};

static void carve32(Carve& c, Ws32& w, size_t T, size_t S) {
    const size_t D = LTX_D;
    w.n_msa = c.take(T * D * 4);
    w.q = c.take(T * D * 4);
    w.k = c.take(T * D * 4);
    w.v = c.take(T * D * 4);
    w.glog1 = c.take(T * LTX_H * 4);
    w.o1 = c.take(T * D * 4);
    w.x_sa = c.take(T * D * 4);
    w.attn_in = c.take(T * D * 4);
    w.q2 = c.take(T * D * 4);
    w.enc = c.take(S * D * 4);
    w.k2 = c.take(S * D * 4);
    w.v2 = c.take(S * D * 4);
    w.glog2 = c.take(T * LTX_H * 4);
    w.o2 = c.take(T * D * 4);
    w.x_ca = c.take(T * D * 4);
    w.ff_in = c.take(T * D * 4);
    w.h = c.take(T * LTX_FF * 4);
}

static void ensure_ws(ltx_ctx* c, size_t T, size_t S, int mode) {
    Carve cv{nullptr, 0, 0, true};
    if (mode == LTX_MODE_F32) {
        Ws32 w;
        carve32(cv, w, T, S);
    } else {
        Ws16 w;
        carve16(cv, w, T, S, c, mode);
    }
    if (c->ws.bytes < cv.off) {
        if (c->ws_pins)
            throw Error("the workspace is bound by " + std::to_string(c->ws_pins) +
                        " live block graph(s) and this forward needs a larger one; destroy them first");
        HIPC(hipDeviceSynchronize());
        c->ws.alloc(cv.off);
    }
}

// ---- launch helpers -------------------------------------------------------

static LtxAda make_ada(const ltx_block_weights* w, const float* tstab, const int32_t* tidx, int K) {
    LtxAda a;
    a.sst = (const float*)w->sst.p;
    a.tstab = tstab;
    a.tidx = tidx;
    a.K = K;
    return a;
}

// The range guard's counter for the 16-bit modes (NULL in mode F32).
static unsigned long long* sat_of(ltx_ctx* c, int mode) {
    return mode == LTX_MODE_F32 ? nullptr : (unsigned long long*)c->range_ctr.p;
}

// sat_add: a device count the kernel adds to the range guard (the weights'
// f16_over in mode F16), or NULL.
static void norm_mod(ltx_ctx* c, int mode, const float* x, void* y, LtxAda ada, int rows, int ish, int isc,
                     hipStream_t st, const unsigned long long* sat_add = nullptr) {
    LtxNormArgs a{x, y, ada, rows, ish, isc, sat_of(c, mode), sat_add};
    const char* k = mode == LTX_MODE_F32 ? "ltx_norm_mod_f32" : mode == LTX_MODE_BF16 ? "ltx_norm_mod_bf16" : "ltx_norm_mod_f16";
    c->launch(k, (rows + 3) / 4, 1, 1, 256, &a, st);  // four rows per workgroup (NORM_ROWS)
}

// 16-bit GEMM: y = A . W^T with the given epilogue. w16: the int8
// projection's weights dequantised to the operand type for this call (by
// dequant16), which routes it to the four-wave kernel, or NULL.
static void gemm16(ltx_ctx* c, int mode, const LtxProj& p, const void* A, int M, int lda, int epi, LtxGemmArgs g,
                   hipStream_t st, const char* label = nullptr, const void* w16 = nullptr) {
    if (p.N % 256 != 0 || p.K % 64 != 0) throw Error("gemm16: N must be a multiple of 256 and K of 64");
    g.a = A;
    g.M = M;
    g.N = p.N;
    g.K = p.K;
    g.lda = lda;
    g.bias = (const float*)p.bias.p;
    const char* bk;
    if (p.q8) {
        g.b = p.q.p;
        g.scales = p.s.p;
        g.qxor = p.qflip ? 0u : 0x80808080u;
        bk = p.scale_f16 ? "i8f16" : "i8f32";
    } else {
        g.b = mode == LTX_MODE_BF16 ? p.w_bf16.p : p.w_f16.p;
        g.scales = nullptr;
        bk = "w16";
    }
    if (!g.b) throw Error("gemm16: weight not resident for this mode");
    g.tiles_m = (M + 255) / 256;
    g.tiles_n = p.N / 256;
    char name[64];
    auto al16 = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
    const char* es = epi == LTX_EPI_STORE ? "store" : epi == LTX_EPI_RESID_GATE ? "resid" : "qkv";
    // Four-wave 16-bit kernel: unquantised weights, or int8 weights
    // dequantised for this call; 16-byte aligned operands (its DMA and
    // epilogue move 16-byte vectors)
    {
        const void* wb = p.q8 ? w16 : (mode == LTX_MODE_BF16 ? p.w_bf16.p : p.w_f16.p);
        if (wb && x4_shape(c, mode, M, p.N, p.K, lda) && g.ldo % 8 == 0 && al16(A) && al16(wb) && al16(g.out) &&
            al16(g.out2) && al16(g.resid) && al16(g.bias) && al16(g.ada.tstab) && al16(g.ada.sst)) {
            g.b = wb;
            g.scales = nullptr;
            g.ksplit = 1;
            std::snprintf(name, sizeof(name), "ltx_gemm_x4_%s_%s%s%s", msuffix(mode), es,
                          epi == LTX_EPI_STORE && g.out_f32 ? "32" : "", epi == LTX_EPI_STORE && g.gelu ? "_gelu" : "");
            const int nitems = g.tiles_m * g.tiles_n;
            c->launch(name, c->gemm_persistent ? std::min(nitems, c->num_cu) : nitems, 1, 1, 256, &g, st, label);
            return;
        }
    }
    // Small grids: 128 x 128 tiles, two workgroups a CU, int8 weights laid
    // out for the LDS-DMA kernels (bytes q + 128, scale words) or 16-bit
    // weights; split K only while even those tiles fill at most half the CUs
    {
        const void* wb = p.q8 ? (p.qflip && p.s2.p ? p.q.p : nullptr) : (mode == LTX_MODE_BF16 ? p.w_bf16.p : p.w_f16.p);
        if (wb && s4_shape(c, mode, M, p.N, p.K, lda, p.q8) && g.ldo % 8 == 0 && al16(A) && al16(wb) && al16(g.out) &&
            al16(g.out2) && al16(g.resid) && al16(g.bias) && al16(g.ada.tstab) && al16(g.ada.sst)) {
            g.b = wb;
            g.scales = p.q8 ? p.s2.p : nullptr;
            g.tiles_m = (M + 127) / 128;
            g.tiles_n = p.N / 128;
            g.ksplit = g.part ? gemm_ksplit(c->num_cu, M, p.N, p.K, 128, 128) : 1;
            std::snprintf(name, sizeof(name), "ltx_gemm_s4_%s_%s_%s", msuffix(mode),
                          p.q8 ? (p.scale_f16 ? "i8f16" : "i8f32") : "w16", es);
            const int nitems = g.tiles_m * g.tiles_n * g.ksplit;
            c->launch(name, c->gemm_persistent ? std::min(nitems, 2 * c->num_cu) : nitems, 1, 1, 256, &g, st, label);
            if (g.ksplit > 1) {
                std::snprintf(name, sizeof(name), "ltx_gemm_reduce_%s_%s", msuffix(mode), es);
                c->launch(name, p.N / 64, (M + 63) / 64, 1, 256, &g, st, "splitk_reduce");
            }
            return;
        }
    }
    // LDS-DMA int8 kernel: f16 or bf16 operands, f16 scales, K a multiple of
    // 128, and byte offsets of A and W within 31 bits (32-bit buffer offsets)
    if ((mode == LTX_MODE_F16 || mode == LTX_MODE_BF16) && p.q8 && p.qflip && p.s2.p &&
        c->gemm_dma && p.K % 128 == 0 && (uint64_t)M * lda * 2 < (1ull << 31) && (uint64_t)p.N * p.K < (1ull << 31) && g.ldo % 8 == 0 &&
        al16(g.out) && al16(g.out2) && al16(g.resid) && al16(g.bias) && al16(g.ada.tstab) && al16(g.ada.sst)) {
        // (its epilogue moves 16-byte vectors: outputs, residual and bias 16-byte aligned)
        g.scales = p.s2.p;
        std::snprintf(name, sizeof(name), "ltx_gemm_q8_%s%s%s", mode == LTX_MODE_BF16 ? "bf16_" : "",
                      p.scale_f16 ? "" : "s32_", es);
        // few output tiles: split K over more workgroups (when the caller
        // gave a buffer for the partial sums), then reduce + epilogue
        g.ksplit = g.part ? gemm_ksplit(c->num_cu, M, p.N, p.K) : 1;
        const int nitems = g.tiles_m * g.tiles_n * g.ksplit;
        c->launch(name, c->gemm_persistent ? std::min(nitems, c->num_cu) : nitems, 1, 1, 512, &g, st, label);
        if (g.ksplit > 1) {
            std::snprintf(name, sizeof(name), "ltx_gemm_reduce_%s_%s", msuffix(mode), es);
            c->launch(name, p.N / 64, (M + 63) / 64, 1, 256, &g, st, "splitk_reduce");
        }
        return;
    }
    // LDS-DMA 16-bit-weight kernel (256 x 128 tiles): the same conditions
    if ((mode == LTX_MODE_F16 || mode == LTX_MODE_BF16) && !p.q8 && c->gemm_dma && p.K % 128 == 0 &&
        p.N % 128 == 0 && (uint64_t)M * lda * 2 < (1ull << 31) && (uint64_t)p.N * p.K * 2 < (1ull << 31) &&
        g.ldo % 8 == 0 && al16(g.out) && al16(g.out2) && al16(g.resid) && al16(g.bias) && al16(g.ada.tstab) &&
        al16(g.ada.sst) && al16(g.b)) {
        std::snprintf(name, sizeof(name), "ltx_gemm_w16dma_%s_%s", msuffix(mode), es);
        g.tiles_n = p.N / 128;
        g.ksplit = g.part ? gemm_ksplit(c->num_cu, M, p.N, p.K, 128) : 1;
        const int nitems = g.tiles_m * g.tiles_n * g.ksplit;
        c->launch(name, c->gemm_persistent ? std::min(nitems, c->num_cu) : nitems, 1, 1, 512, &g, st, label);
        if (g.ksplit > 1) {
            std::snprintf(name, sizeof(name), "ltx_gemm_reduce_%s_%s", msuffix(mode), es);
            c->launch(name, p.N / 64, (M + 63) / 64, 1, 256, &g, st, "splitk_reduce");
        }
        return;
    }
    std::snprintf(name, sizeof(name), "ltx_gemm_%s_%s_%s", msuffix(mode), bk, es);
    // split-K as above; the reduce kernel moves 16-byte vectors, so only with
    // aligned operands
    const bool aligned = g.ldo % 8 == 0 && al16(g.out) && al16(g.out2) && al16(g.resid) && al16(g.bias) &&
                         al16(g.ada.tstab) && al16(g.ada.sst);
    g.ksplit = g.part && aligned ? gemm_ksplit(c->num_cu, M, p.N, p.K) : 1;
    c->launch(name, g.tiles_m * g.tiles_n * g.ksplit, 1, 1, 512, &g, st, label);
    if (g.ksplit > 1) {
        std::snprintf(name, sizeof(name), "ltx_gemm_reduce_%s_%s", msuffix(mode), es);
        c->launch(name, p.N / 64, (M + 63) / 64, 1, 256, &g, st, "splitk_reduce");
    }
}

// Dequantises the int8 projections p[i] whose buffer out[i] is set (and whose
// weights are laid out for the LDS-DMA kernels: bytes q + 128, scale words)
// into out[i], one launch per scale type; done[i] = out[i] for those, NULL
// for the rest.
static void dequant16(ltx_ctx* c, int mode, const LtxProj* const* p, void* const* out, int n, const void** done,
                      hipStream_t st) {
    for (int sf = 0; sf < 2; sf++) {  // f16 scale pairs, then f32 scales
        LtxDq16Args a{};
        int nb = 0;
        for (int i = 0; i < n; i++) {
            if (sf == 0) done[i] = nullptr;
            const LtxProj& q = *p[i];
            if (!out[i] || !q.q8 || !q.qflip || !q.s2.p || (q.scale_f16 ? 0 : 1) != sf) continue;
            const int j = a.njobs++;
            a.q[j] = (const uint8_t*)q.q.p;
            a.s2[j] = (const uint32_t*)q.s2.p;
            a.out[j] = out[i];
            a.N[j] = q.N;
            a.K[j] = q.K;
            a.start[j] = nb;
            nb += (q.K / LTX_GROUP) * ((q.N + 31) / 32);
            done[i] = out[i];
        }
        if (!a.njobs) continue;
        a.start[a.njobs] = nb;
        char name[48];
        std::snprintf(name, sizeof(name), "ltx_gemm_dq16_%s%s", msuffix(mode), sf ? "_s32" : "");
        c->launch(name, nb, 1, 1, 256, &a, st, "dq16");
    }
}

static void gate16(ltx_ctx* c, int mode, const LtxProj& p, const void* A, int M, float* out, hipStream_t st) {
    LtxGateArgs g{A, mode == LTX_MODE_BF16 ? p.w_bf16.p : p.w_f16.p, (const float*)p.bias.p, out, M};
    // one wave per 32 rows while that gives every CU at least one wave
    // (each wave's 256 MFMAs form one dependent chain); below that, K split
    // over the four waves of a workgroup per 32 rows
    if ((M + 31) / 32 >= c->num_cu)
        c->launch(mode == LTX_MODE_BF16 ? "ltx_gate_bf16" : "ltx_gate_f16", (M + 127) / 128, 1, 1, 256, &g, st);
    else
        c->launch(mode == LTX_MODE_BF16 ? "ltx_gate_ks_bf16" : "ltx_gate_ks_f16", (M + 31) / 32, 1, 1, 256, &g, st);
}

// The attention's exponent scale: softmax scale 1/sqrt(128) times log2(e).
static const float kAttnC = (float)(1.4426950408889634 / 11.313708498984761);

// oscale multiplies the normed (and roped) rows before the 16-bit rounding:
// kAttnC for Q, so the attention reads scores in exp2 units, 1 for K.
static void qknorm16(ltx_ctx* c, int mode, const void* x, int ldx, const void* w, const float* cs, const float* sn,
                     void* y, int rows, float oscale, hipStream_t st) {
    LtxQkNormArgs a{x, (const float*)w, cs, sn, y, rows, ldx, oscale, sat_of(c, mode)};
    c->launch(mode == LTX_MODE_BF16 ? "ltx_qknorm_bf16" : "ltx_qknorm_f16", rows, 1, 1, 256, &a, st);
}

// q_scaled: Q already carries kAttnC (the block path); else plain Q.
// qk_rows: Q and K as token rows [L][4096] (the block's qk-norm output);
// else head-major [32][L][128] (ltx_op_attention).
static void attn16(ltx_ctx* c, int mode, const void* q, const void* k, const void* vt, const float* glog, void* out,
                   int lq, int lkv, bool q_scaled, hipStream_t st, const char* label = nullptr,
                   unsigned long long* sat = nullptr, bool qk_rows = false) {
    LtxAttnArgs a{};
    a.sat = sat;
    a.q = q;
    a.k = k;
    a.q_hs = qk_rows ? LTX_HD : lq * LTX_HD;
    a.q_rs = qk_rows ? LTX_D : LTX_HD;
    a.k_hs = qk_rows ? LTX_HD : lkv * LTX_HD;
    a.k_rs = qk_rows ? LTX_D : LTX_HD;
    a.vt = vt;
    a.glog = glog;
    a.out = out;
    a.lq = lq;
    a.lkv = lkv;
    a.scale_log2 = q_scaled ? 1.0f : kAttnC;
    a.q_tiles = (lq + 255) / 256;  // 256 queries per workgroup
    char name[48];
    const int wph = std::max(1, std::min(c->num_cu / LTX_H, a.q_tiles));  // workgroups per head
    if (c->attn_kv && lkv % 64 == 0 && lkv >= 64 && lkv <= 256 && (a.q_tiles >= 2 * wph || lkv < 128)) {
        // resident K/V: each workgroup loads one head's K and V^T once and
        // runs every wph-th query tile of that head (with fewer than two
        // tiles per workgroup the streaming kernel, which overlaps the K/V
        // loads with the first tiles, is faster)
        std::snprintf(name, sizeof(name), "ltx_attn_%s_kv%s", msuffix(mode), q_scaled ? "" : "_uq");
        c->launch(name, LTX_H * wph, 1, 1, 512, &a, st, label);
        return;
    }
    if (c->attn_pp && lkv % 64 == 0 && lkv >= 128) {
        // ping-pong kernel: whole 64-key tiles, at least two
        std::snprintf(name, sizeof(name), "ltx_attn_%s_pp%s", msuffix(mode), q_scaled ? "" : "_uq");
        c->launch(name, a.q_tiles * LTX_H, 1, 1, 512, &a, st, label);
        return;
    }
    // any key count: 8 waves of 32 queries (whole 64-key tiles: no masking)
    std::snprintf(name, sizeof(name), "ltx_attn_%s_w8%s", msuffix(mode), lkv % 64 == 0 ? "_full" : "");
    c->launch(name, a.q_tiles * LTX_H, 1, 1, 512, &a, st, label);
}

// f32-mode GEMM over rows [r0, r0 + N) of a (possibly fused) projection.
static void gemm32(ltx_ctx* c, const LtxProj& p, int r0, int N, const float* A, int M, float* out, int epi,
                   const float* resid, LtxAda ada, int igate, int gelu, hipStream_t st,
                   const char* label = nullptr) {
    LtxGemm32Args g{};
    g.a = A;
    const size_t G = p.K / LTX_GROUP;
    if (p.q8) {
        g.bkind = p.scale_f16 ? 1 : 0;
        g.qxor = p.qflip ? 0u : 0x80808080u;
        g.b = (const int8_t*)p.q.p + (size_t)r0 * p.K;
        g.scales = (const char*)p.s.p + (size_t)r0 * G * (p.scale_f16 ? 2 : 4);
    } else {
        g.bkind = 2;
        g.b = (const uint16_t*)p.w_bf16.p + (size_t)r0 * p.K;
    }
    g.bias = p.bias.p ? (const float*)p.bias.p + r0 : nullptr;
    g.out = out;
    g.resid = resid;
    g.ada = ada;
    g.M = M;
    g.N = N;
    g.K = p.K;
    g.epi = epi;
    g.gelu = gelu;
    g.igate = igate;
    if (p.K % 32) throw Error("mode F32 GEMM: K must be a multiple of 32");
    c->launch("ltx_gemm_f32", (N + 127) / 128, (M + 127) / 128, 1, 256, &g, st, label);
}

static void qknorm32(ltx_ctx* c, float* x, const void* w, const float* cs, const float* sn, int rows, hipStream_t st) {
    LtxQkNorm32Args a{x, (const float*)w, cs, sn, rows, LTX_D};
    c->launch("ltx_qknorm_f32", rows, 1, 1, 256, &a, st);
}

static void attn32(ltx_ctx* c, const float* q, const float* k, const float* v, const float* glog, float* out, int lq,
                   int lkv, hipStream_t st, const char* label = nullptr) {
    LtxAttn32Args a{q, k, v, glog, out, lq, lkv, 1.0f / std::sqrt(128.0f)};
    c->launch("ltx_attn_f32", (lq + 127) / 128, LTX_H, 1, 512, &a, st, label);
}

// `to` runs what it is given next only after everything enqueued so far on
// `from` (event e).
static void stream_after(hipStream_t to, hipStream_t from, hipEvent_t e) {
    HIPC(hipEventRecord(e, from));
    HIPC(hipStreamWaitEvent(to, e, 0));
}

static void set_stage(ltx_ctx* c, int id, void* p, size_t bytes) {
    c->stage_ptr[id] = p;
    c->stage_bytes[id] = bytes;
}

// ---- the block ------------------------------------------------------------

void block_forward(ltx_ctx* c, const ltx_block_weights* w, const float* x, const float* tstab, int K,
                   const int32_t* tidx, const float* ctxv, int S, const float* pts2, const float* cs, const float* sn,
                   int T, float* y, int mode, hipStream_t st) {
    if (!w) throw Error("NULL weights");
    if (T <= 0 || S <= 0 || K <= 0) throw Error("T, S and K must be positive");
    if (!x || !tstab || !tidx || !ctxv || !pts2 || !cs || !sn || !y) throw Error("NULL tensor argument");
    if ((const void*)x == (const void*)y) throw Error("y may not alias x");
    if (mode != LTX_MODE_F16 && mode != LTX_MODE_BF16 && mode != LTX_MODE_F32) throw Error("unknown mode");
    HIPC(hipSetDevice(c->device));
    ensure_ws(c, (size_t)T, (size_t)S, mode);
    std::memset(c->stage_ptr, 0, sizeof(c->stage_ptr));
    const size_t TD = (size_t)T * LTX_D, SD = (size_t)S * LTX_D;
    LtxAda ada = make_ada(w, tstab, tidx, K);
    Carve cv{(char*)c->ws.p, 0, 0, false};

    if (mode == LTX_MODE_F32) {
        Ws32 b;
        carve32(cv, b, T, S);
        // self-attention (ltx/block.zig:546-547, qAttn1 520-530)
        norm_mod(c, mode, x, b.n_msa, ada, T, 0, 1, st,
             mode == LTX_MODE_F16 ? (const unsigned long long*)w->f16_over.p : nullptr);
        gemm32(c, w->qkv1, 0, LTX_D, (const float*)b.n_msa, T, (float*)b.q, LTX_EPI_STORE, nullptr, ada, 0, 0, st, "gemm:qkv1");
        gemm32(c, w->qkv1, LTX_D, LTX_D, (const float*)b.n_msa, T, (float*)b.k, LTX_EPI_STORE, nullptr, ada, 0, 0, st, "gemm:qkv1");
        gemm32(c, w->qkv1, 2 * LTX_D, LTX_D, (const float*)b.n_msa, T, (float*)b.v, LTX_EPI_STORE, nullptr, ada, 0, 0, st, "gemm:qkv1");
        gemm32(c, w->g1, 0, LTX_H, (const float*)b.n_msa, T, (float*)b.glog1, LTX_EPI_STORE, nullptr, ada, 0, 0, st, "ltx_gate:1");
        qknorm32(c, (float*)b.q, w->qn1.p, cs, sn, T, st);
        qknorm32(c, (float*)b.k, w->kn1.p, cs, sn, T, st);
        attn32(c, (const float*)b.q, (const float*)b.k, (const float*)b.v, (const float*)b.glog1, (float*)b.o1, T, T, st, "attn:self");
        gemm32(c, w->o1, 0, LTX_D, (const float*)b.o1, T, (float*)b.x_sa, LTX_EPI_RESID_GATE, x, ada, 2, 0, st, "gemm:o1");
        // cross-attention (ltx/block.zig:548-568)
        norm_mod(c, mode, (const float*)b.x_sa, b.attn_in, ada, T, 6, 7, st);
        LtxEncArgs ea{ctxv, (const float*)w->psst.p, pts2, b.enc, S};
        c->launch("ltx_enc_f32", S, 1, 1, 256, &ea, st);
        gemm32(c, w->q2, 0, LTX_D, (const float*)b.attn_in, T, (float*)b.q2, LTX_EPI_STORE, nullptr, ada, 0, 0, st, "gemm:q2");
        gemm32(c, w->kv2, 0, LTX_D, (const float*)b.enc, S, (float*)b.k2, LTX_EPI_STORE, nullptr, ada, 0, 0, st, "gemm:kv2");
        gemm32(c, w->kv2, LTX_D, LTX_D, (const float*)b.enc, S, (float*)b.v2, LTX_EPI_STORE, nullptr, ada, 0, 0, st, "gemm:kv2");
        gemm32(c, w->g2, 0, LTX_H, (const float*)b.attn_in, T, (float*)b.glog2, LTX_EPI_STORE, nullptr, ada, 0, 0, st, "ltx_gate:2");
        qknorm32(c, (float*)b.q2, w->qn2.p, nullptr, nullptr, T, st);
        qknorm32(c, (float*)b.k2, w->kn2.p, nullptr, nullptr, S, st);
        attn32(c, (const float*)b.q2, (const float*)b.k2, (const float*)b.v2, (const float*)b.glog2, (float*)b.o2, T, S, st, "attn:cross");
        gemm32(c, w->o2, 0, LTX_D, (const float*)b.o2, T, (float*)b.x_ca, LTX_EPI_RESID_GATE, (const float*)b.x_sa, ada, 8, 0, st, "gemm:o2");
        // feed-forward (ltx/block.zig:569-573)
        norm_mod(c, mode, (const float*)b.x_ca, b.ff_in, ada, T, 3, 4, st);
        gemm32(c, w->f1, 0, LTX_FF, (const float*)b.ff_in, T, (float*)b.h, LTX_EPI_STORE, nullptr, ada, 0, 1, st, "gemm:ff1");
        gemm32(c, w->f2, 0, LTX_D, (const float*)b.h, T, y, LTX_EPI_RESID_GATE, (const float*)b.x_ca, ada, 5, 0, st, "gemm:ff2");
        set_stage(c, LTX_ST_NORM_MSA, b.n_msa, TD * 4);
        set_stage(c, LTX_ST_Q1, b.q, TD * 4);
        set_stage(c, LTX_ST_K1, b.k, TD * 4);
        set_stage(c, LTX_ST_V1, b.v, TD * 4);
        set_stage(c, LTX_ST_GLOG1, b.glog1, (size_t)T * LTX_H * 4);
        set_stage(c, LTX_ST_ATTN1, b.o1, TD * 4);
        set_stage(c, LTX_ST_X_SA, b.x_sa, TD * 4);
        set_stage(c, LTX_ST_ATTN_IN, b.attn_in, TD * 4);
        set_stage(c, LTX_ST_ATTN2, b.o2, TD * 4);
        set_stage(c, LTX_ST_X_CA, b.x_ca, TD * 4);
        set_stage(c, LTX_ST_FF_IN, b.ff_in, TD * 4);
        set_stage(c, LTX_ST_FF_H, b.h, (size_t)T * LTX_FF * 4);
        set_stage(c, LTX_ST_GLOG2, b.glog2, (size_t)T * LTX_H * 4);
        set_stage(c, LTX_ST_Q2, b.q2, TD * 4);
        set_stage(c, LTX_ST_K2, b.k2, SD * 4);
        set_stage(c, LTX_ST_V2, b.v2, SD * 4);
        return;
    }

    if (mode == LTX_MODE_F16 && !(w->f16_max <= 65504.0f))
        throw Error("mode F16: weight operands beyond the f16 range (largest |q s| or |w| " +
                    std::to_string(w->f16_max) + " > 65504); run LTX_MODE_BF16");
    unsigned long long* sat = sat_of(c, mode);
    Ws16 b;
    carve16(cv, b, T, S, c, mode);
    // the int8 weights of the projections on the four-wave GEMM, dequantised
    // for this forward (qkv1, o1, q2, o2, ff1, ff2)
    const void* dq[6];
    {
        const LtxProj* ps[6] = {&w->qkv1, &w->o1, &w->q2, &w->o2, &w->f1, &w->f2};
        dequant16(c, mode, ps, b.dq, 6, dq, st);
    }
    // self-attention: n = modulate(rms(x), ada1, ada0); fused q|k|v GEMM
    norm_mod(c, mode, x, b.n_msa, ada, T, 0, 1, st,
             mode == LTX_MODE_F16 ? (const unsigned long long*)w->f16_over.p : nullptr);
    hipStream_t sd = c->side;
    auto fail_check = [&]() {
        if (fail_in_capture()) {
            hipStreamCaptureStatus cst = hipStreamCaptureStatusNone;
            if (hipStreamIsCapturing(st, &cst) == hipSuccess && cst == hipStreamCaptureStatusActive)
                throw Error("injected failure inside a graph capture, after the second stream joined it [LTX_FAIL_CAPTURE]");
        }
    };
    // The context side of the cross-attention: K/V modulation, fused k|v
    // GEMM (split-K partial sums in `part`), on stream s.
    auto ctx_side = [&](hipStream_t s, void* part) {
        LtxEncArgs ea{ctxv, (const float*)w->psst.p, pts2, b.enc, S, sat};
        c->launch(mode == LTX_MODE_BF16 ? "ltx_enc_bf16" : "ltx_enc_f16", S, 1, 1, 256, &ea, s);
        LtxGemmArgs gk{};
        gk.out = b.k2_16;
        gk.out2 = b.vt2;
        gk.nsplit = LTX_D;
        gk.sat = sat;
        gk.part = (float*)part;
        gemm16(c, mode, w->kv2, b.enc, S, LTX_D, LTX_EPI_QKV, gk, s, "gemm:kv2");
    };
    // Small T (early): the 256-row GEMM tiles and attention query tiles
    // leave CUs idle, and the side stream fills them from here on: the
    // self-attention gate logits beside the q|k|v GEMM, then the whole
    // context side (K/V modulation, k|v GEMM with its own partial sums, k
    // norm) beside the self-attention branch; later the cross-attention
    // gate logits beside the q2 GEMM. Large T: side work starts only after
    // the persistent GEMMs, whose one-workgroup-per-CU grids it would
    // otherwise hold back, and ends before the attentions, which it would
    // slow as much as it gains.
    const bool early = side_early(c, (size_t)T);
    if (early) {
        stream_after(sd, st, c->side_ev[0]);
        fail_check();
        gate16(c, mode, w->g1, b.n_msa, T, (float*)b.glog1, sd);
        HIPC(hipEventRecord(c->side_ev[1], sd));  // glog1 ready
        ctx_side(sd, b.part2);
        qknorm16(c, mode, b.k2_16, LTX_D, w->kn2.p, nullptr, nullptr, b.kh2, S, 1.0f, sd);
    }
    LtxGemmArgs g{};
    g.out = b.qk16;
    g.out2 = b.vt1;
    g.nsplit = 2 * LTX_D;
    g.sat = sat;
    g.part = (float*)b.part;  // split-K partial sums (small grids)
    gemm16(c, mode, w->qkv1, b.n_msa, T, LTX_D, LTX_EPI_QKV, g, st, "gemm:qkv1", dq[0]);
    if (!early) {
        // the self-attention gate logits beside the q/k norms (both read
        // only what the GEMMs above wrote)
        stream_after(sd, st, c->side_ev[0]);
        fail_check();
        gate16(c, mode, w->g1, b.n_msa, T, (float*)b.glog1, sd);
        HIPC(hipEventRecord(c->side_ev[1], sd));  // glog1 ready
    }
    {  // q and k norms + RoPE in one pass (the RoPE rows read once)
        LtxQkNorm2Args qa{b.qk16, (const float*)w->qn1.p, (const float*)w->kn1.p, cs, sn, b.qh1, b.kh1,
                          T, 2 * LTX_D, kAttnC, 1.0f, sat};
        c->launch(mode == LTX_MODE_BF16 ? "ltx_qknorm2_bf16" : "ltx_qknorm2_f16", T, 1, 1, 256, &qa, st);
    }
    HIPC(hipStreamWaitEvent(st, c->side_ev[1], 0));
    attn16(c, mode, b.qh1, b.kh1, b.vt1, (const float*)b.glog1, b.o1, T, T, true, st, "attn:self", sat, true);
    g = LtxGemmArgs{};
    g.out = b.x_sa;
    g.resid = x;
    g.ada = ada;
    g.igate = 2;
    g.ldo = LTX_D;
    g.part = (float*)b.part;  // split-K partial sums (small grids)
    gemm16(c, mode, w->o1, b.o1, T, LTX_D, LTX_EPI_RESID_GATE, g, st, "gemm:o1", dq[1]);
    // cross-attention
    norm_mod(c, mode, (const float*)b.x_sa, b.attn_in, ada, T, 6, 7, st);
    if (early) {
        stream_after(sd, st, c->side_ev[2]);
        gate16(c, mode, w->g2, b.attn_in, T, (float*)b.glog2, sd);
    }
    g = LtxGemmArgs{};
    g.out = b.q2_16;
    g.ldo = LTX_D;
    g.sat = sat;
    g.part = (float*)b.part;  // split-K partial sums (small grids)
    gemm16(c, mode, w->q2, b.attn_in, T, LTX_D, LTX_EPI_STORE, g, st, "gemm:q2", dq[2]);
    {
        // A marker after each launch from here to the cross-attention (see
        // ltx_ctx::launch): without them the gate logits below and the k|v
        // GEMM's split-K reduce beside them interleaved so badly that they
        // took 0.57 and 0.39 ms instead of 0.09 and 0.01 (28,672 tokens).
        MarkScope marks(c, T >= kMarkRows);
        if (early) {
            qknorm16(c, mode, b.q2_16, LTX_D, w->qn2.p, nullptr, nullptr, b.qh2, T, kAttnC, st);
        } else {
            // the cross-attention gate logits on the side stream, beside the
            // context side (K/V modulation, k|v GEMM) and the q and k norms
            stream_after(sd, st, c->side_ev[2]);
            gate16(c, mode, w->g2, b.attn_in, T, (float*)b.glog2, sd);
            ctx_side(st, b.part);
            qknorm16(c, mode, b.q2_16, LTX_D, w->qn2.p, nullptr, nullptr, b.qh2, T, kAttnC, st);
            qknorm16(c, mode, b.k2_16, LTX_D, w->kn2.p, nullptr, nullptr, b.kh2, S, 1.0f, st);
        }
        stream_after(st, sd, c->side_ev[3]);  // glog2 (and, early, the context side) ready
        attn16(c, mode, b.qh2, b.kh2, b.vt2, (const float*)b.glog2, b.o2, T, S, true, st, "attn:cross", sat, true);
    }
    g = LtxGemmArgs{};
    g.out = b.x_ca;
    g.resid = (const float*)b.x_sa;
    g.ada = ada;
    g.igate = 8;
    g.ldo = LTX_D;
    g.part = (float*)b.part;  // split-K partial sums (small grids)
    gemm16(c, mode, w->o2, b.o2, T, LTX_D, LTX_EPI_RESID_GATE, g, st, "gemm:o2", dq[3]);
    // feed-forward
    norm_mod(c, mode, (const float*)b.x_ca, b.ff_in, ada, T, 3, 4, st);
    g = LtxGemmArgs{};
    g.out = b.h;
    g.ldo = LTX_FF;
    g.gelu = 1;
    g.sat = sat;
    g.part = (float*)b.part;  // split-K partial sums (small grids)
    gemm16(c, mode, w->f1, b.ff_in, T, LTX_D, LTX_EPI_STORE, g, st, "gemm:ff1", dq[4]);
    g = LtxGemmArgs{};
    g.out = y;
    g.resid = (const float*)b.x_ca;
    g.ada = ada;
    g.igate = 5;
    g.ldo = LTX_D;
    g.part = (float*)b.part;  // split-K partial sums (small grids)
    gemm16(c, mode, w->f2, b.h, T, LTX_FF, LTX_EPI_RESID_GATE, g, st, "gemm:ff2", dq[5]);

    set_stage(c, LTX_ST_NORM_MSA, b.n_msa, TD * 2);
    set_stage(c, LTX_ST_Q1, b.qh1, TD * 2);
    set_stage(c, LTX_ST_K1, b.kh1, TD * 2);
    set_stage(c, LTX_ST_V1, b.vt1, TD * 2);
    set_stage(c, LTX_ST_GLOG1, b.glog1, (size_t)T * LTX_H * 4);
    set_stage(c, LTX_ST_ATTN1, b.o1, TD * 2);
    set_stage(c, LTX_ST_X_SA, b.x_sa, TD * 4);
    set_stage(c, LTX_ST_ATTN_IN, b.attn_in, TD * 2);
    set_stage(c, LTX_ST_ATTN2, b.o2, TD * 2);
    set_stage(c, LTX_ST_X_CA, b.x_ca, TD * 4);
    set_stage(c, LTX_ST_FF_IN, b.ff_in, TD * 2);
    set_stage(c, LTX_ST_FF_H, b.h, (size_t)T * LTX_FF * 2);
    set_stage(c, LTX_ST_GLOG2, b.glog2, (size_t)T * LTX_H * 4);
    set_stage(c, LTX_ST_Q2, b.qh2, TD * 2);
    set_stage(c, LTX_ST_K2, b.kh2, SD * 2);
    set_stage(c, LTX_ST_V2, b.vt2, SD * 2);
}

bool linear_q8_needs_scratch(const ltx_ctx* c, int N, int K, int mode) {
    (void)K;
    return mode != LTX_MODE_F32 && c->gemm_dma && N % 256 == 0;
}

// ltx_op_linear_q8 / _noalloc: in the 16-bit modes with the LDS-DMA kernel the
// weights are first laid out as bytes q + 128 in sc.q and the scales as words
// [K/128][N] in sc.pairs (both written whole before the GEMM reads them).
void check_linear_q8(int M, int N, int K, int mode) {
    if (M <= 0 || N <= 0 || K <= 0 || K % 128) throw Error("bad GEMM shape (K must be a multiple of 128)");
    if (mode != LTX_MODE_F16 && mode != LTX_MODE_BF16 && mode != LTX_MODE_F32) throw Error("unknown mode");
}

void linear_q8(ltx_ctx* c, const void* a, const int8_t* q, const void* scales, int scale_f16, const float* bias,
               void* y, int out_f32, int M, int N, int K, int gelu, int mode, const LinearScratch& sc,
               hipStream_t st) {
    check_linear_q8(M, N, K, mode);
    if (!a || !q || !scales || !y) throw Error("NULL tensor argument");
    // Borrow the caller's buffers through a non-owning projection view.
    LtxProj p;
    p.N = N;
    p.K = K;
    p.q8 = true;
    p.scale_f16 = scale_f16;
    p.q.p = (void*)q;
    p.s.p = (void*)scales;
    p.bias.p = (void*)bias;
    try {
        if (mode == LTX_MODE_F32) {
            if (!out_f32) throw Error("mode F32 writes f32 output");
            LtxAda ada{};
            gemm32(c, p, 0, N, (const float*)a, M, (float*)y, LTX_EPI_STORE, nullptr, ada, 0, gelu, st);
        } else {
            if (linear_q8_needs_scratch(c, N, K, mode)) {
                if (!sc.q || !sc.pairs) throw Error("linear_q8: no scratch");
                // the LDS-DMA kernel reads scale words [K/128][N]
                const size_t n2 = (size_t)N * (K / LTX_GROUP);
                LtxPairArgs pa{scales, sc.pairs, N, K / LTX_GROUP, scale_f16 ? 0 : 1};
                c->launch("ltx_scale_pairs", (unsigned)((n2 + 255) / 256), 1, 1, 256, &pa, st);
                p.s2.p = sc.pairs;
                // and its weights as the bytes q + 128
                const size_t nq = (size_t)N * K / 4;
                LtxFlipArgs fa{(const uint32_t*)q, sc.q, nq};
                c->launch("ltx_q8_flip", (unsigned)((nq + 255) / 256), 1, 1, 256, &fa, st);
                p.q.p = sc.q;
                p.qflip = true;
            }
            // the four-wave kernel on the weights dequantised into sc.w16
            const void* w16 = nullptr;
            if (sc.w16 && p.qflip && x4_shape(c, mode, M, N, K, K)) {
                const LtxProj* ps[1] = {&p};
                void* outs[1] = {sc.w16};
                dequant16(c, mode, ps, outs, 1, &w16, st);
            }
            LtxGemmArgs g{};
            g.out = y;
            g.ldo = N;
            g.gelu = gelu;
            g.out_f32 = out_f32;
            gemm16(c, mode, p, a, M, K, LTX_EPI_STORE, g, st, nullptr, w16);
        }
    } catch (...) {
        p.q.p = p.s.p = p.s2.p = p.bias.p = nullptr;
        throw;
    }
    p.q.p = p.s.p = p.s2.p = p.bias.p = nullptr;
}

}  // namespace ltx


extern "C" {

int ltx_block_forward(ltx_ctx* c, const ltx_block_weights* w, const float* x, const float* tstab, int K,
                      const int32_t* tidx, const float* ctx_tokens, int S, const float* pts2, const float* cos,
                      const float* sin, int T, float* y, int mode, void* stream) {
    LTX_GUARD(c, {
        if (!c) throw ltx::Error("NULL context");
        ltx::block_forward(c, w, x, tstab, K, tidx, ctx_tokens, S, pts2, cos, sin, T, y, mode, (hipStream_t)stream);
    })
}

// A block forward captured once into a HIP graph, with its buffers bound.
struct ltx_block_graph {
    ltx_ctx* c = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    // the captured forward's intermediates, restored for ltx_block_stage at
    // every launch
    void* stage_ptr[LTX_ST_COUNT] = {};
    uint64_t stage_bytes[LTX_ST_COUNT] = {};
};

int ltx_block_graph_create(ltx_ctx* c, const ltx_block_weights* w, const float* x, const float* tstab, int K,
                           const int32_t* tidx, const float* ctx_tokens, int S, const float* pts2, const float* cos,
                           const float* sin, int T, float* y, int mode, ltx_block_graph** out) {
    LTX_GUARD(c, {
        if (!c) throw ltx::Error("NULL context");
        if (!out) throw ltx::Error("NULL output handle");
        *out = nullptr;
        if (c->prof) throw ltx::Error("event profiling is on; a graph cannot capture its events");
        if (T <= 0 || S <= 0) throw ltx::Error("bad token counts");
        HIPC(hipSetDevice(c->device));
        // the workspace is sized (and allocated) before the capture, which
        // may only record launches and event waits
        ltx::ensure_ws(c, (size_t)T, (size_t)S, mode);
        hipStream_t cs = nullptr;
        HIPC(hipStreamCreateWithFlags(&cs, hipStreamNonBlocking));
        hipGraph_t graph = nullptr;
        const hipError_t eb = hipStreamBeginCapture(cs, hipStreamCaptureModeRelaxed);
        if (eb != hipSuccess) {
            (void)hipStreamDestroy(cs);
            throw ltx::Error(std::string("graph capture could not start: ") + hipGetErrorString(eb));
        }
        try {
            ltx::block_forward(c, w, x, tstab, K, tidx, ctx_tokens, S, pts2, cos, sin, T, y, mode, cs);
        } catch (...) {
            // A throw after the forward forked the context's second stream
            // into the capture leaves that stream capturing: join it back
            // into cs, or the capture cannot end and every later forward
            // would find the second stream still in capture mode.
            hipStreamCaptureStatus sst = hipStreamCaptureStatusNone;
            if (hipStreamIsCapturing(c->side, &sst) == hipSuccess && sst == hipStreamCaptureStatusActive &&
                hipEventRecord(c->side_ev[1], c->side) == hipSuccess)
                (void)hipStreamWaitEvent(cs, c->side_ev[1], 0);
            (void)hipStreamEndCapture(cs, &graph);
            if (graph) (void)hipGraphDestroy(graph);
            (void)hipStreamDestroy(cs);
            throw;
        }
        const hipError_t ec = hipStreamEndCapture(cs, &graph);
        (void)hipStreamDestroy(cs);
        if (ec != hipSuccess || !graph) {
            if (graph) (void)hipGraphDestroy(graph);
            throw ltx::Error(std::string("graph capture of the block forward failed: ") + hipGetErrorString(ec));
        }
        hipGraphExec_t exec = nullptr;
        const hipError_t ei = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        if (ei != hipSuccess) {
            (void)hipGraphDestroy(graph);
            throw ltx::Error(std::string("graph instantiation failed: ") + hipGetErrorString(ei));
        }
        ltx_block_graph* g = new (std::nothrow) ltx_block_graph;
        if (!g) {
            (void)hipGraphExecDestroy(exec);
            (void)hipGraphDestroy(graph);
            throw ltx::Error("out of host memory");
        }
        g->c = c;
        g->graph = graph;
        g->exec = exec;
        std::memcpy(g->stage_ptr, c->stage_ptr, sizeof(g->stage_ptr));
        std::memcpy(g->stage_bytes, c->stage_bytes, sizeof(g->stage_bytes));
        c->ws_pins++;
        *out = g;
    })
}

int ltx_block_graph_launch(ltx_block_graph* g, void* stream) {
    ltx_ctx* c = g ? g->c : nullptr;
    LTX_GUARD(c, {
        if (!g) throw ltx::Error("NULL graph");
        HIPC(hipSetDevice(c->device));
        HIPC(hipGraphLaunch(g->exec, (hipStream_t)stream));
        std::memcpy(c->stage_ptr, g->stage_ptr, sizeof(c->stage_ptr));
        std::memcpy(c->stage_bytes, g->stage_bytes, sizeof(c->stage_bytes));
    })
}

void ltx_block_graph_destroy(ltx_block_graph* g) {
    if (!g) return;
    (void)hipSetDevice(g->c->device);
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    g->c->ws_pins--;
    delete g;
}

int ltx_op_linear_q8(ltx_ctx* c, const void* a, const int8_t* q, const void* scales, int scale_f16, const float* bias,
                     void* y, int out_f32, int M, int N, int K, int gelu, int mode, void* stream) {
    LTX_GUARD(c, {
        if (!c) throw ltx::Error("NULL context");
        ltx::check_linear_q8(M, N, K, mode);  // before N and K size the scratch
        HIPC(hipSetDevice(c->device));
        ltx::LinearScratch sc{};
        if (ltx::linear_q8_needs_scratch(c, N, K, mode)) {
            // scratch owned by the context, grown as needed
            const size_t nq = (size_t)N * K, np = (size_t)N * (K / LTX_GROUP) * 4;
            if (c->op_q.bytes < nq) c->op_q.alloc(nq);
            if (c->op_pairs.bytes < np) c->op_pairs.alloc(np);
            sc.q = (uint32_t*)c->op_q.p;
            sc.pairs = (uint32_t*)c->op_pairs.p;
            if (ltx::x4_shape(c, mode, M, N, K, K)) {
                if (c->op_w16.bytes < 2 * nq) c->op_w16.alloc(2 * nq);
                sc.w16 = c->op_w16.p;
            }
        }
        ltx::linear_q8(c, a, q, scales, scale_f16, bias, y, out_f32, M, N, K, gelu, mode, sc, (hipStream_t)stream);
    })
}

int ltx_op_attention(ltx_ctx* c, const void* q, const void* k, const void* v, const float* glog, void* out, int lq,
                     int lkv, int mode, void* stream) {
    LTX_GUARD(c, {
        if (!c) throw ltx::Error("NULL context");
        if (lq <= 0 || lkv <= 0) throw ltx::Error("bad attention lengths");
        const bool q_scaled = (mode & LTX_ATTN_Q_SCALED) != 0;
        mode &= ~LTX_ATTN_Q_SCALED;
        if (q_scaled && mode == LTX_MODE_F32) throw ltx::Error("LTX_ATTN_Q_SCALED applies to the 16-bit modes");
        HIPC(hipSetDevice(c->device));
        if (mode == LTX_MODE_F32)
            ltx::attn32(c, (const float*)q, (const float*)k, (const float*)v, glog, (float*)out, lq, lkv,
                        (hipStream_t)stream);
        else
            ltx::attn16(c, mode, q, k, v, glog, out, lq, lkv, q_scaled, (hipStream_t)stream);
    })
}

int ltx_op_dequant(ltx_ctx* c, const int8_t* q, const void* scales, int scale_f16, int N, int K, float* out32,
                   void* out16, int mode, void* stream) {
    LTX_GUARD(c, {
        if (!c) throw ltx::Error("NULL context");
        if (N <= 0 || K <= 0 || K % 128) throw ltx::Error("bad dequant shape");
        HIPC(hipSetDevice(c->device));
        LtxDequantArgs a{q, scales, out32, out16, N, K, scale_f16};
        size_t n = (size_t)N * K;
        c->launch(mode == LTX_MODE_BF16 ? "ltx_dequant_bf16" : "ltx_dequant_f16", (unsigned)((n / 2 + 255) / 256), 1,
                  1, 256, &a, (hipStream_t)stream);
    })
}

}  // extern "C"
