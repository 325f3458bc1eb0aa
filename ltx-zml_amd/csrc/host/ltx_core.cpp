// Parts around the blocks (ltx/core_parts.zig), the distilled scheduler
// (ltx/scheduler.zig) and the denoising loop that drives a stack of resident
// blocks (ltx/e2e_denoise.zig:218-336). Everything here is f32, as in the
// reference; the linear layers use the f32 GEMM kernel with bf16 weights.
#include <cstring>
#include <vector>

#include "ltx_internal.hpp"

using ltx::DevBuf;
using ltx::Error;

namespace {

// CORE_SPECS order (ltx/core_parts.zig:55-74): bf16 weights [O][I], bf16
// biases [O], and the f32 scale_shift_table [2][D].
struct CoreSpec {
    const char* name;
    int o, i;  // i == 0: a bias / vector of o elements
};
const CoreSpec kCore[LTX_C_COUNT] = {
    {"ada_l1_w", LTX_DIM, 256},      {"ada_l1_b", LTX_DIM, 0},         {"ada_l2_w", LTX_DIM, LTX_DIM},
    {"ada_l2_b", LTX_DIM, 0},        {"ada_out_w", 9 * LTX_DIM, LTX_DIM}, {"ada_out_b", 9 * LTX_DIM, 0},
    {"pada_l1_w", LTX_DIM, 256},     {"pada_l1_b", LTX_DIM, 0},        {"pada_l2_w", LTX_DIM, LTX_DIM},
    {"pada_l2_b", LTX_DIM, 0},       {"pada_out_w", 2 * LTX_DIM, LTX_DIM}, {"pada_out_b", 2 * LTX_DIM, 0},
    {"pat_w", LTX_DIM, 128},         {"pat_b", LTX_DIM, 0},            {"po_w", 128, LTX_DIM},
    {"po_b", 128, 0},                {"fsst", 2, LTX_DIM},
};

// The distilled sigma lists (ltx/scheduler.zig:15-18).
const float kStage1[] = {1.0f, 0.99375f, 0.9875f, 0.98125f, 0.975f, 0.909375f, 0.725f, 0.421875f, 0.0f};
const float kStage2[] = {0.909375f, 0.725f, 0.421875f, 0.0f};

}  // namespace

struct ltx_core_weights {
    DevBuf t[LTX_C_COUNT];  // weights bf16 as given; biases and fsst f32
};

namespace ltx {

// y[M][N] = A[M][K] . W[N][K]^T + b, W bf16, f32 everywhere else.
static void lin32(ltx_ctx* c, const ltx_core_weights* cw, int wi, const float* A, int M, float* out, hipStream_t st) {
    const CoreSpec& s = kCore[wi];
    LtxGemm32Args g{};
    g.a = A;
    g.b = cw->t[wi].p;
    g.bkind = 2;
    g.bias = (const float*)cw->t[wi + 1].p;
    g.out = out;
    g.M = M;
    g.N = s.o;
    g.K = s.i;
    g.epi = LTX_EPI_STORE;
    if (s.i % 32) throw Error("core GEMM: K must be a multiple of 32");
    c->launch("ltx_gemm_f32", (s.o + 127) / 128, (M + 127) / 128, 1, 256, &g, st);
}

static void silu(ltx_ctx* c, const float* x, float* y, size_t n, hipStream_t st) {
    LtxEltArgs a{x, y, n};
    c->launch("ltx_core_silu", (unsigned)((n + 255) / 256), 1, 1, 256, &a, st);
}

static void sinusoid(ltx_ctx* c, const float* t, int rows, float* out, hipStream_t st) {
    LtxSinArgs a{t, out, rows};
    c->launch("ltx_core_sinusoid", rows, 1, 1, 128, &a, st);
}

// Scratch of the conditioning MLPs for K timestep rows, carved from one
// context buffer: sin [K+1][256], h [K][D], silu(emb) [K][D], and the prompt
// branch's own rows.
static float* core_scratch(ltx_ctx* c, int K) {
    const size_t need = ((size_t)(K + 1) * 256 + (size_t)(3 * K + 4) * LTX_DIM + 64) * sizeof(float);
    if (c->core_ws.bytes < need) c->core_ws.alloc(need);
    return (float*)c->core_ws.p;
}

// ts9r, embedded_timestep and pts2r (ltx/core_parts.zig:112-141).
static void conditioning(ltx_ctx* c, const ltx_core_weights* cw, const float* t, int K, const float* sigma_dev,
                         float* tstab, float* emb, float* pts2, hipStream_t st) {
    float* ws = core_scratch(c, K);
    float* sn = ws;                                   // [K][256]
    float* psn = sn + (size_t)K * 256;                // [1][256]
    float* h = psn + 256;                             // [K][D]
    float* se = h + (size_t)K * LTX_DIM;              // [K][D]
    float* ph = se + (size_t)K * LTX_DIM;             // [1][D]
    float* pe = ph + LTX_DIM;                         // [1][D]
    float* pse = pe + LTX_DIM;                        // [1][D]
    // emb = lin2(silu(lin1(sinusoid(t))));  ts9 = lin_out(silu(emb))
    sinusoid(c, t, K, sn, st);
    lin32(c, cw, LTX_C_ADA_L1_W, sn, K, h, st);
    silu(c, h, h, (size_t)K * LTX_DIM, st);
    lin32(c, cw, LTX_C_ADA_L2_W, h, K, emb, st);
    silu(c, emb, se, (size_t)K * LTX_DIM, st);
    lin32(c, cw, LTX_C_ADA_OUT_W, se, K, tstab, st);
    // pts2 = p_out(silu(p_lin2(silu(p_lin1(sinusoid(sigma))))))
    sinusoid(c, sigma_dev, 1, psn, st);
    lin32(c, cw, LTX_C_PADA_L1_W, psn, 1, ph, st);
    silu(c, ph, ph, LTX_DIM, st);
    lin32(c, cw, LTX_C_PADA_L2_W, ph, 1, pe, st);
    silu(c, pe, pse, LTX_DIM, st);
    lin32(c, cw, LTX_C_PADA_OUT_W, pse, 1, pts2, st);
}

static void tail(ltx_ctx* c, const ltx_core_weights* cw, const float* x, const float* emb, const int32_t* tidx, int T,
                 float* normed, float* vel, hipStream_t st) {
    LtxTailNormArgs a{x, (const float*)cw->t[LTX_C_FSST].p, emb, tidx, normed};
    c->launch("ltx_core_tail_norm", T, 1, 1, 256, &a, st);
    lin32(c, cw, LTX_C_PO_W, normed, T, vel, st);
}

}  // namespace ltx

extern "C" {

int ltx_core_weights_from_host(ltx_ctx* c, const void* const* tensors, ltx_core_weights** out) {
    LTX_GUARD(c, {
        if (!c || !tensors || !out) throw Error("NULL argument");
        *out = nullptr;
        HIPC(hipSetDevice(c->device));
        auto* cw = new ltx_core_weights();
        try {
            for (int i = 0; i < LTX_C_COUNT; i++) {
                if (!tensors[i]) throw Error(std::string("missing core tensor ") + kCore[i].name);
                const CoreSpec& s = kCore[i];
                if (i == LTX_C_FSST) {  // f32 [2][D]
                    cw->t[i].alloc((size_t)2 * LTX_DIM * 4);
                    HIPC(hipMemcpy(cw->t[i].p, tensors[i], (size_t)2 * LTX_DIM * 4, hipMemcpyHostToDevice));
                } else if (s.i == 0) {  // bf16 bias -> f32
                    std::vector<float> b(s.o);
                    for (int k = 0; k < s.o; k++) b[k] = ltx::bf16_bits_to_f32(((const uint16_t*)tensors[i])[k]);
                    cw->t[i].alloc(b.size() * 4);
                    HIPC(hipMemcpy(cw->t[i].p, b.data(), b.size() * 4, hipMemcpyHostToDevice));
                } else {  // bf16 weight [O][I] as given
                    const size_t n = (size_t)s.o * s.i * 2;
                    cw->t[i].alloc(n);
                    HIPC(hipMemcpy(cw->t[i].p, tensors[i], n, hipMemcpyHostToDevice));
                }
            }
        } catch (...) {
            delete cw;
            throw;
        }
        *out = cw;
    })
}

void ltx_core_weights_free(ltx_ctx* c, ltx_core_weights* cw) {
    if (c) (void)hipSetDevice(c->device);
    delete cw;
}

int ltx_core_conditioning(ltx_ctx* c, const ltx_core_weights* cw, const float* t, int K, const float* sigma,
                          float* tstab, float* emb, float* pts2, void* stream) {
    LTX_GUARD(c, {
        if (!c || !cw || !t || !sigma || !tstab || !emb || !pts2) throw Error("NULL argument");
        if (K <= 0) throw Error("K must be positive");
        HIPC(hipSetDevice(c->device));
        ltx::conditioning(c, cw, t, K, sigma, tstab, emb, pts2, (hipStream_t)stream);
    })
}

int ltx_core_patchify(ltx_ctx* c, const ltx_core_weights* cw, const float* latent, int T, float* x, void* stream) {
    LTX_GUARD(c, {
        if (!c || !cw || !latent || !x) throw Error("NULL argument");
        if (T <= 0) throw Error("T must be positive");
        HIPC(hipSetDevice(c->device));
        ltx::lin32(c, cw, LTX_C_PAT_W, latent, T, x, (hipStream_t)stream);
    })
}

int ltx_core_tail(ltx_ctx* c, const ltx_core_weights* cw, const float* x, const float* emb, const int32_t* tidx, int T,
                  float* vel, void* stream) {
    LTX_GUARD(c, {
        if (!c || !cw || !x || !emb || !tidx || !vel) throw Error("NULL argument");
        if (T <= 0) throw Error("T must be positive");
        HIPC(hipSetDevice(c->device));
        const size_t need = (size_t)T * LTX_DIM * 4;
        if (c->tail_ws.bytes < need) c->tail_ws.alloc(need);
        ltx::tail(c, cw, x, emb, tidx, T, (float*)c->tail_ws.p, vel, (hipStream_t)stream);
    })
}

int ltx_sched_sigmas(int stage, float* out, int* count) {
    const float* v = stage == 2 ? kStage2 : kStage1;
    const int n = stage == 2 ? 4 : 9;
    if (stage != 1 && stage != 2) {
        ltx::set_thread_error("stage must be 1 or 2");
        return LTX_FAIL;
    }
    if (count) *count = n;
    if (out) std::memcpy(out, v, n * sizeof(float));
    return LTX_OK;
}

int ltx_sched_noise_init(ltx_ctx* c, const float* clean, const float* noise, const float* maskk, const int32_t* tidx,
                         int T, int C, float noise_scale, float* out, void* stream) {
    LTX_GUARD(c, {
        if (!c || !clean || !noise || !maskk || !tidx || !out) throw Error("NULL argument");
        if (T <= 0 || C <= 0) throw Error("bad latent shape");
        HIPC(hipSetDevice(c->device));
        const size_t n = (size_t)T * C;
        LtxNoiseArgs a{clean, noise, maskk, tidx, out, n, C, noise_scale};
        c->launch("ltx_sched_noise_init", (unsigned)((n + 255) / 256), 1, 1, 256, &a, (hipStream_t)stream);
    })
}

int ltx_sched_step(ltx_ctx* c, const float* x, const float* vel, const float* tk, const float* maskk,
                   const int32_t* tidx, const float* clean, int T, int C, float sigma, float sigma_next, float* out,
                   void* stream) {
    LTX_GUARD(c, {
        if (!c || !x || !vel || !tk || !maskk || !tidx || !clean || !out) throw Error("NULL argument");
        if (T <= 0 || C <= 0) throw Error("bad latent shape");
        HIPC(hipSetDevice(c->device));
        const size_t n = (size_t)T * C;
        LtxSchedArgs a{x, vel, clean, tk, maskk, tidx, out, n, C, sigma, sigma_next};
        c->launch("ltx_sched_step", (unsigned)((n + 255) / 256), 1, 1, 256, &a, (hipStream_t)stream);
    })
}

int ltx_denoise(ltx_ctx* c, const ltx_block_weights* const* blocks, int nblocks, const ltx_core_weights* cw,
                float* latent, const float* clean, const float* maskk, const int32_t* tidx, int K,
                const float* ctx_tokens, int S, const float* cos, const float* sin, int T, const float* sigmas,
                int nsteps, int mode, void* stream) {
    LTX_GUARD(c, {
        if (!c || !blocks || !cw || !latent || !clean || !maskk || !tidx || !ctx_tokens || !cos || !sin || !sigmas)
            throw Error("NULL argument");
        if (nblocks <= 0 || nsteps <= 0 || K <= 0 || K > 63 || T <= 0 || S <= 0) throw Error("bad denoise shape");
        for (int b = 0; b < nblocks; b++)
            if (!blocks[b]) throw Error("NULL block weights");
        HIPC(hipSetDevice(c->device));
        hipStream_t st = (hipStream_t)stream;
        // workspace: x ping-pong [T][D] x 2, tail norm [T][D], tstab [K][9][D],
        // emb [K][D], pts2 [2][D], velocity [T][128], tk [K] + sigma
        const size_t xd = (size_t)T * LTX_DIM;
        const size_t need = (3 * xd + (size_t)K * 10 * LTX_DIM + 2 * LTX_DIM + (size_t)T * 128 + 64) * 4;
        if (c->dn_ws.bytes < need) c->dn_ws.alloc(need);
        float* xa = (float*)c->dn_ws.p;
        float* xb = xa + xd;
        float* normed = xb + xd;
        float* tstab = normed + xd;
        float* emb = tstab + (size_t)K * 9 * LTX_DIM;
        float* pts2 = emb + (size_t)K * LTX_DIM;
        float* vel = pts2 + 2 * LTX_DIM;
        float* tk = vel + (size_t)T * 128;
        const size_t n = (size_t)T * LTX_IN_CH;
        for (int s = 0; s < nsteps; s++) {
            const float sigma = sigmas[s], sigma_next = sigmas[s + 1];
            LtxTimestepArgs ta{maskk, tk, K, sigma};
            c->launch("ltx_sched_timesteps", 1, 1, 1, 64, &ta, st);
            ltx::conditioning(c, cw, tk, K, tk + K, tstab, emb, pts2, st);
            ltx::lin32(c, cw, LTX_C_PAT_W, latent, T, xa, st);
            for (int b = 0; b < nblocks; b++) {
                ltx::block_forward(c, blocks[b], xa, tstab, K, tidx, ctx_tokens, S, pts2, cos, sin, T, xb, mode, st);
                std::swap(xa, xb);
            }
            ltx::tail(c, cw, xa, emb, tidx, T, normed, vel, st);
            // elementwise, so the latent is updated in place
            LtxSchedArgs sa{latent, vel, clean, tk, maskk, tidx, latent, n, LTX_IN_CH, sigma, sigma_next};
            c->launch("ltx_sched_step", (unsigned)((n + 255) / 256), 1, 1, 256, &sa, st);
        }
        c->stage_ptr[LTX_ST_VELOCITY] = vel;
        c->stage_bytes[LTX_ST_VELOCITY] = (uint64_t)T * LTX_IN_CH * 4;
    })
}

}  // extern "C"
