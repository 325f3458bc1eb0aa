/*
 * CPU restatement of the LTX-2.5 DiT block forward (the int8 QBlock path)
 * — TEST INFRASTRUCTURE ONLY. Nothing in the product links or calls this
 * file; tests, the smoke check and the CPU-baseline leg of the benchmark use
 * it as the checker / baseline.
 *
 * Compiled twice: REAL=double (the parity oracle) and REAL=float (the timed
 * CPU baseline). Every function cites the reference file:line it restates.
 *
 *   block forward ........ ltx/block.zig:544-574 (QBlock.qBlockOutAll)
 *   lin / linQ / dq4 ..... ltx/block.zig:22-26, 462-477
 *   rmsNoW / rmsW ........ ltx/block.zig:28-34
 *   modulate / adaVal .... ltx/block.zig:36-67
 *   rope ................. ltx/block.zig:69-77 (split-half), 220-226
 *   whileSdpaC ........... ltx/block.zig:110-154 (online softmax, K scaled)
 *   dense sdpa ........... zml.nn.sdpa as used at ltx/block.zig:525,563
 *   rope tables .......... ltx/block_conformance.zig:87-126
 *   quantizer ............ tools/quantize_block.py:51-59 (int8, group 128)
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifndef REAL
#define REAL double
#endif
typedef REAL real;

#define D 4096
#define H 32
#define HD 128
#define FF 16384
#define EPS 1e-6

/* ---- scalar helpers ----------------------------------------------------- */

static inline float bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline float f16_to_f32(uint16_t h) {
    uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff, u;
    if (e == 0) {
        if (m == 0) {
            u = s;
        } else { /* subnormal: renormalise */
            int k = -1;
            do { k++; m <<= 1; } while (!(m & 0x400));
            u = s | ((uint32_t)(127 - 15 - k) << 23) | ((m & 0x3ff) << 13);
        }
    } else if (e == 31) {
        u = s | 0x7f800000u | (m << 13);
    } else {
        u = s | ((e + 127 - 15) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* Weight element access: base tensors are bf16 bit patterns. */
static inline real bfr(const uint16_t* p, size_t i) { return (real)bf16_to_f32(p[i]); }

/* ---- dequant (ltx/block.zig:462-471): one f32 rounding of f32(q)*s ------- */

void orc_dequant(const int8_t* q, const void* s, int scale_f16, int O, int I, float* out) {
    int G = I / 128;
    for (int o = 0; o < O; o++)
        for (int i = 0; i < I; i++) {
            float sc = scale_f16 ? f16_to_f32(((const uint16_t*)s)[(size_t)o * G + i / 128])
                                 : ((const float*)s)[(size_t)o * G + i / 128];
            out[(size_t)o * I + i] = (float)q[(size_t)o * I + i] * sc;
        }
}

/* ---- quantizer (tools/quantize_block.py:51-59), f64 arithmetic ---------- */

void orc_quantize(const uint16_t* w_bf16, int O, int I, int gs, int bits, int8_t* q, float* s) {
    int qmax = bits == 4 ? 7 : 127, lo = bits == 4 ? -8 : -128;
    int G = I / gs;
    for (int o = 0; o < O; o++)
        for (int g = 0; g < G; g++) {
            double am = 0;
            for (int e = 0; e < gs; e++) {
                double v = fabs((double)bf16_to_f32(w_bf16[(size_t)o * I + g * gs + e]));
                if (v > am) am = v;
            }
            double sc = am > 0 ? am / qmax : 1.0;
            for (int e = 0; e < gs; e++) {
                double r = nearbyint((double)bf16_to_f32(w_bf16[(size_t)o * I + g * gs + e]) / sc);
                if (r < lo) r = lo;
                if (r > qmax) r = qmax;
                q[(size_t)o * I + g * gs + e] = (int8_t)r;
            }
            s[(size_t)o * G + g] = (float)sc;
        }
}

/* ---- RoPE tables (ltx/block_conformance.zig:87-126) ----------------------
 * grid [3][T][2] f32 (start,end) per axis; out cos/sin in the bundle layout
 * [H][T][64] f32. Frequencies: theta^linspace(0,1,682)*pi/2 evaluated in
 * f64 and rounded to f32 (the numpy grid generator returns f32), then
 * promoted back for the position product; trig in f64, one cast to f32. */

#define NF 682
static const double MAXPOS[3] = {20.0, 2048.0, 2048.0};

void orc_rope_freqs(double* freqs /* [NF] */) {
    double step = 1.0 / (double)(NF - 1);
    for (int k = 0; k < NF; k++) {
        double x = k == NF - 1 ? 1.0 : (double)k * step; /* numpy linspace */
        double v = pow(10000.0, x) * (M_PI / 2.0);
        freqs[k] = (double)(float)v;
    }
}

void orc_rope_tables(const float* grid, int T, float* cos_out, float* sin_out) {
    double freqs[NF];
    orc_rope_freqs(freqs);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; t++) {
        double arg[3];
        for (int a = 0; a < 3; a++) {
            double s0 = grid[((size_t)a * T + t) * 2], s1 = grid[((size_t)a * T + t) * 2 + 1];
            double mid = (s0 + s1) / 2.0;
            arg[a] = (mid / MAXPOS[a]) * 2.0 - 1.0;
        }
        for (int h = 0; h < H; h++)
            for (int f = 0; f < 64; f++) {
                int j = h * 64 + f;
                double c = 1.0, s = 0.0;
                if (j >= 2) {
                    int sl = j - 2;
                    double th = freqs[sl / 3] * arg[sl % 3];
                    c = cos(th);
                    s = sin(th);
                }
                size_t idx = ((size_t)h * T + t) * 64 + f;
                cos_out[idx] = (float)c;
                sin_out[idx] = (float)s;
            }
    }
}

/* ---- dense linear algebra ---------------------------------------------- */

/* C[M][N] = A[M][K] * Bt[K][N]; saxpy form, sequential k order per output. */
static void gemm_kn(const real* A, int M, int K, const real* Bt, int N, real* C) {
    enum { MB = 4, NB = 64 };
    int nnb = (N + NB - 1) / NB;
#pragma omp parallel for schedule(dynamic, 1)
    for (int nb = 0; nb < nnb; nb++) {
        int n0 = nb * NB, nn = N - n0 < NB ? N - n0 : NB;
        for (int m0 = 0; m0 < M; m0 += MB) {
            int mm = M - m0 < MB ? M - m0 : MB;
            real acc[MB][NB];
            memset(acc, 0, sizeof(acc));
            for (int k = 0; k < K; k++) {
                const real* b = Bt + (size_t)k * N + n0;
                for (int i = 0; i < mm; i++) {
                    real a = A[(size_t)(m0 + i) * K + k];
                    for (int j = 0; j < nn; j++) acc[i][j] += a * b[j];
                }
            }
            for (int i = 0; i < mm; i++)
                for (int j = 0; j < nn; j++) C[(size_t)(m0 + i) * N + n0 + j] = acc[i][j];
        }
    }
}

/* Transposed weight [K][N] from a bf16 [N][K] tensor or an int8 [N][K] +
 * scale [N][K/128] pair (dq4 semantics: f32(q)*s rounded once to f32). */
static real* weight_t(const uint16_t* wbf, const int8_t* q, const void* s, int scale_f16, int N, int K) {
    real* wt = (real*)malloc(sizeof(real) * (size_t)N * K);
    int G = K / 128;
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++)
        for (int k = 0; k < K; k++) {
            real v;
            if (q) {
                float sc = scale_f16 ? f16_to_f32(((const uint16_t*)s)[(size_t)n * G + k / 128])
                                     : ((const float*)s)[(size_t)n * G + k / 128];
                v = (real)((float)q[(size_t)n * K + k] * sc);
            } else {
                v = bfr(wbf, (size_t)n * K + k);
            }
            wt[(size_t)k * N + n] = v;
        }
    return wt;
}

/* lin / linQ (ltx/block.zig:22-26, 473-477): y = x W^T (+ b) */
static void linear(const real* x, int M, int K, const uint16_t* wbf, const int8_t* q, const void* s,
                   int scale_f16, const uint16_t* b, int N, real* y) {
    real* wt = weight_t(wbf, q, s, scale_f16, N, K);
    gemm_kn(x, M, K, wt, N, y);
    free(wt);
    if (b) {
#pragma omp parallel for schedule(static)
        for (int m = 0; m < M; m++)
            for (int n = 0; n < N; n++) y[(size_t)m * N + n] += bfr(b, n);
    }
}

/* rmsNoW (ltx/block.zig:28-30): x * rsqrt(mean(x^2) + eps) over the row */
static void rms_rows(const real* x, int M, int N, const uint16_t* w, real* y) {
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; m++) {
        const real* r = x + (size_t)m * N;
        real ss = 0;
        for (int n = 0; n < N; n++) ss += r[n] * r[n];
        real inv = (real)1 / (real)sqrt((double)(ss / N + (real)EPS));
        for (int n = 0; n < N; n++) {
            real v = r[n] * inv;
            if (w) v *= bfr(w, n); /* rmsW (ltx/block.zig:32-34) */
            y[(size_t)m * N + n] = v;
        }
    }
}

/* adaVal (ltx/block.zig:47-67): ada_i[t] = sst[i] + tstab[tidx[t], i] */
static inline real ada(const float* sst, const float* tstab, const int32_t* tidx, int t, int i, int c) {
    return (real)tstab[((size_t)tidx[t] * 9 + i) * D + c] + (real)sst[(size_t)i * D + c];
}

/* modulate(rms(x), ada[isc], ada[ish]) (ltx/block.zig:36-38, 248-252) */
static void norm_mod(const real* x, int T, const float* sst, const float* tstab, const int32_t* tidx,
                     int ish, int isc, real* y) {
    rms_rows(x, T, D, NULL, y);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; t++)
        for (int c = 0; c < D; c++) {
            real n = y[(size_t)t * D + c];
            y[(size_t)t * D + c] = n * (ada(sst, tstab, tidx, t, isc, c) + 1) + ada(sst, tstab, tidx, t, ish, c);
        }
}

/* rope (ltx/block.zig:69-77): per head, a = x[0:64], b = x[64:128];
 * out = [a cos - b sin, b cos + a sin]; cos/sin in graph layout [T][H][64] */
static void rope_apply(real* x, int T, const float* cs, const float* sn) {
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; t++)
        for (int h = 0; h < H; h++) {
            real* r = x + (size_t)t * D + h * HD;
            const float* c = cs + ((size_t)t * H + h) * 64;
            const float* s = sn + ((size_t)t * H + h) * 64;
            for (int f = 0; f < 64; f++) {
                real a = r[f], b = r[64 + f];
                r[f] = a * (real)c[f] - b * (real)s[f];
                r[64 + f] = b * (real)c[f] + a * (real)s[f];
            }
        }
}

/* Attention. q [Lq][D], k/v [Lkv][D] (head h at columns h*128..). Output in
 * merged layout [Lq][D]. chunk > 0: whileSdpaC (ltx/block.zig:110-154):
 * K pre-scaled by f32(1/sqrt(128)), running (m, l, acc) with m0 = -FLT_MAX,
 * corr = exp(m - m'), p = exp(s - m'). chunk == 0: dense softmax (zml
 * nn.sdpa: same K scaling, max-subtracted softmax). */
int orc_sdpa(const real* q, int Lq, const real* k, const real* v, int Lkv, int chunk, real* out) {
    if (chunk > 0 && Lkv % chunk != 0) return 0; /* whileSdpaC asserts divisibility (ltx/block.zig:112) */
    const real scale = (real)(1.0f / sqrtf(128.0f));
    real* ks = (real*)malloc(sizeof(real) * (size_t)Lkv * D);
    for (size_t i = 0; i < (size_t)Lkv * D; i++) ks[i] = k[i] * scale;
#pragma omp parallel
    {
        real* s = (real*)malloc(sizeof(real) * (size_t)(chunk > 0 ? chunk : Lkv));
#pragma omp for schedule(dynamic, 16) collapse(2)
        for (int h = 0; h < H; h++)
            for (int i = 0; i < Lq; i++) {
                const real* qr = q + (size_t)i * D + h * HD;
                real acc[HD];
                memset(acc, 0, sizeof(acc));
                if (chunk > 0) {
                    real m = (real)-FLT_MAX, l = 0;
                    for (int c0 = 0; c0 < Lkv; c0 += chunk) {
                        real cmax = (real)-INFINITY;
                        for (int j = 0; j < chunk; j++) {
                            const real* kr = ks + (size_t)(c0 + j) * D + h * HD;
                            real d = 0;
                            for (int e = 0; e < HD; e++) d += qr[e] * kr[e];
                            s[j] = d;
                            if (d > cmax) cmax = d;
                        }
                        real mn = m > cmax ? m : cmax;
                        real corr = (real)exp((double)(m - mn));
                        real psum = 0;
                        for (int e = 0; e < HD; e++) acc[e] *= corr;
                        for (int j = 0; j < chunk; j++) {
                            real p = (real)exp((double)(s[j] - mn));
                            psum += p;
                            const real* vr = v + (size_t)(c0 + j) * D + h * HD;
                            for (int e = 0; e < HD; e++) acc[e] += p * vr[e];
                        }
                        l = l * corr + psum;
                        m = mn;
                    }
                    for (int e = 0; e < HD; e++) out[(size_t)i * D + h * HD + e] = acc[e] / l;
                } else {
                    real mx = (real)-INFINITY;
                    for (int j = 0; j < Lkv; j++) {
                        const real* kr = ks + (size_t)j * D + h * HD;
                        real d = 0;
                        for (int e = 0; e < HD; e++) d += qr[e] * kr[e];
                        s[j] = d;
                        if (d > mx) mx = d;
                    }
                    real l = 0;
                    for (int j = 0; j < Lkv; j++) {
                        s[j] = (real)exp((double)(s[j] - mx));
                        l += s[j];
                    }
                    for (int j = 0; j < Lkv; j++) {
                        const real* vr = v + (size_t)j * D + h * HD;
                        real p = s[j] / l;
                        for (int e = 0; e < HD; e++) acc[e] += p * vr[e];
                    }
                    for (int e = 0; e < HD; e++) out[(size_t)i * D + h * HD + e] = acc[e];
                }
            }
        free(s);
    }
    free(ks);
    return 1;
}

static inline real sigmoid_r(real x) { return (real)1 / ((real)1 + (real)exp(-(double)x)); }

/* Tensor.gelu, tanh form (used at ltx/block.zig:332, 533) */
static inline real gelu_tanh(real x) {
    const double c = 0.7978845608028654; /* sqrt(2/pi) */
    double xd = (double)x;
    return (real)(0.5 * xd * (1.0 + tanh(c * (xd + 0.044715 * xd * xd * xd))));
}

/* ---- the block --------------------------------------------------------- */

/* Base tensor order (ltx/block.zig:377-406, WEIGHT_SPECS). */
enum {
    W_Q1_W, W_Q1_B, W_K1_W, W_K1_B, W_V1_W, W_V1_B, W_O1_W, W_O1_B, W_QN1, W_KN1, W_G1_W, W_G1_B,
    W_Q2_W, W_Q2_B, W_K2_W, W_K2_B, W_V2_W, W_V2_B, W_O2_W, W_O2_B, W_QN2, W_KN2, W_G2_W, W_G2_B,
    W_FF1_W, W_FF2_W, W_SST, W_PSST, W_COUNT
};
/* Quantized companions (ltx/loader.zig:147-156, plus the out-projections). */
enum { Q_Q1, Q_K1, Q_V1, Q_Q2, Q_K2, Q_V2, Q_F1, Q_F2, Q_O1, Q_O2, Q_COUNT };

/* Stage dumps, in forward order. */
enum {
    ST_S1_NORM_MSA, ST_Q1_ROPED, ST_K1_ROPED, ST_V1, ST_ATTN1_MERGED, ST_S3_ATTN1, ST_S4_AFTER_SA,
    ST_S4_NORMED, ST_ATTN_IN, ST_ENC, ST_Q2_NORMED, ST_K2_NORMED, ST_V2, ST_ATTN2_MERGED, ST_S5_CA_OUT,
    ST_X_CA, ST_S6_FF_IN, ST_FF_H, ST_S7_FF_OUT, ST_COUNT
};

static void dump(real* const* stages, int id, const real* src, size_t n) {
    if (stages && stages[id]) memcpy(stages[id], src, sizeof(real) * n);
}

#define BW(i) ((const uint16_t*)base[i])
#define QW(i) (q8 ? q8[i] : NULL)
#define QS(i) (q8s ? q8s[i] : NULL)

/* One attention (Block.attention, ltx/block.zig:212-244 / QBlock,
 * ltx/block.zig:500-530, 557-567): q = rmsW(lin(x)), k = rmsW(lin(ctx)),
 * v = lin(ctx), optional RoPE, sdpa, gate 2*sigmoid(lin(x, gw, gb)) per
 * (token, head) from the attention input, merge heads, output projection.
 * Weight slot ids: qi/ki/vi/oi index both base (bf16) and q8 tables. */
static void attention(const void* const* base, const int8_t* const* q8, const void* const* q8s, int sf16,
                      const real* x, int T, const real* ctxv, int S, int bq, int bk, int bv, int bo, int iqn,
                      int ikn, int igw, int qq, int qk, int qv, int qo, const float* cs, const float* sn,
                      int chunk, real* out, real* const* stages, int st_q, int st_k, int st_v, int st_merged) {
    real* q = (real*)malloc(sizeof(real) * (size_t)T * D);
    real* k = (real*)malloc(sizeof(real) * (size_t)S * D);
    real* v = (real*)malloc(sizeof(real) * (size_t)S * D);
    real* o = (real*)malloc(sizeof(real) * (size_t)T * D);
    linear(x, T, D, BW(bq), QW(qq), QS(qq), sf16, BW(bq + 1), D, q);
    rms_rows(q, T, D, BW(iqn), q);
    linear(ctxv, S, D, BW(bk), QW(qk), QS(qk), sf16, BW(bk + 1), D, k);
    rms_rows(k, S, D, BW(ikn), k);
    linear(ctxv, S, D, BW(bv), QW(qv), QS(qv), sf16, BW(bv + 1), D, v);
    if (cs) {
        rope_apply(q, T, cs, sn);
        rope_apply(k, S, cs, sn);
    }
    dump(stages, st_q, q, (size_t)T * D);
    dump(stages, st_k, k, (size_t)S * D);
    dump(stages, st_v, v, (size_t)S * D);
    if (!orc_sdpa(q, T, k, v, S, chunk, o)) { /* chunk must divide the key count */
        memset(o, 0xff, sizeof(real) * (size_t)T * D); /* NaN: fails loudly */
    }
    real* glog = (real*)malloc(sizeof(real) * (size_t)T * H);
    linear(x, T, D, BW(igw), NULL, NULL, 0, BW(igw + 1), H, glog);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; t++)
        for (int h = 0; h < H; h++) {
            real g = sigmoid_r(glog[(size_t)t * H + h]) * 2;
            for (int e = 0; e < HD; e++) o[(size_t)t * D + h * HD + e] *= g;
        }
    dump(stages, st_merged, o, (size_t)T * D);
    linear(o, T, D, BW(bo), QW(qo), QS(qo), sf16, BW(bo + 1), D, out);
    free(glog);
    free(q);
    free(k);
    free(v);
    free(o);
}

/* QBlock.qBlockOutAll (ltx/block.zig:544-574) with the self-attention
 * computed blockwise (chunk) — the production attention algorithm
 * (ltx/block.zig:105-154); cross-attention dense (cross_chunk 0) as in the
 * reference, or blockwise. q8[i] == NULL selects the bf16 base weight. */
int orc_block_forward(const void* const* base, const int8_t* const* q8, const void* const* q8s, int scale_f16,
                      const float* x_in, const float* tstab, int K, const int32_t* tidx, const float* ctx_in,
                      int S, const float* pts2, const float* cs, const float* sn, int T, int chunk,
                      int cross_chunk, real* out, real* const* stages) {
    (void)K;
    const float* sst = (const float*)base[W_SST];
    const float* psst = (const float*)base[W_PSST];
    size_t TD = (size_t)T * D;
    real* x = (real*)malloc(sizeof(real) * TD);
    real* n = (real*)malloc(sizeof(real) * TD);
    real* a = (real*)malloc(sizeof(real) * TD);
    real* x_sa = (real*)malloc(sizeof(real) * TD);
    for (size_t i = 0; i < TD; i++) x[i] = x_in[i];

    /* self-attention: n = modulate(rms(x), ada1, ada0) */
    norm_mod(x, T, sst, tstab, tidx, 0, 1, n);
    dump(stages, ST_S1_NORM_MSA, n, TD);
    attention(base, q8, q8s, scale_f16, n, T, n, T, W_Q1_W, W_K1_W, W_V1_W, W_O1_W, W_QN1, W_KN1, W_G1_W, Q_Q1,
              Q_K1, Q_V1, Q_O1, cs, sn, chunk, a, stages, ST_Q1_ROPED, ST_K1_ROPED, ST_V1, ST_ATTN1_MERGED);
    dump(stages, ST_S3_ATTN1, a, TD);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; t++)
        for (int c = 0; c < D; c++)
            x_sa[(size_t)t * D + c] = x[(size_t)t * D + c] + a[(size_t)t * D + c] * ada(sst, tstab, tidx, t, 2, c);
    dump(stages, ST_S4_AFTER_SA, x_sa, TD);

    /* cross-attention (ltx/block.zig:548-568) */
    rms_rows(x_sa, T, D, NULL, n);
    dump(stages, ST_S4_NORMED, n, TD);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; t++)
        for (int c = 0; c < D; c++) {
            real v = n[(size_t)t * D + c];
            n[(size_t)t * D + c] = v * (ada(sst, tstab, tidx, t, 7, c) + 1) + ada(sst, tstab, tidx, t, 6, c);
        }
    dump(stages, ST_ATTN_IN, n, TD);
    real* enc = (real*)malloc(sizeof(real) * (size_t)S * D);
    for (int t = 0; t < S; t++)
        for (int c = 0; c < D; c++) {
            real sh = (real)psst[c] + (real)pts2[c];
            real sc = (real)psst[D + c] + (real)pts2[D + c];
            enc[(size_t)t * D + c] = (real)ctx_in[(size_t)t * D + c] * (sc + 1) + sh;
        }
    dump(stages, ST_ENC, enc, (size_t)S * D);
    attention(base, q8, q8s, scale_f16, n, T, enc, S, W_Q2_W, W_K2_W, W_V2_W, W_O2_W, W_QN2, W_KN2, W_G2_W, Q_Q2,
              Q_K2, Q_V2, Q_O2, NULL, NULL, cross_chunk, a, stages, ST_Q2_NORMED, ST_K2_NORMED, ST_V2,
              ST_ATTN2_MERGED);
    free(enc);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; t++)
        for (int c = 0; c < D; c++) a[(size_t)t * D + c] *= ada(sst, tstab, tidx, t, 8, c);
    dump(stages, ST_S5_CA_OUT, a, TD);
    real* x_ca = x; /* reuse */
    for (size_t i = 0; i < TD; i++) x_ca[i] = x_sa[i] + a[i];
    dump(stages, ST_X_CA, x_ca, TD);

    /* feed-forward (ltx/block.zig:569-573, qFf 532-534) */
    norm_mod(x_ca, T, sst, tstab, tidx, 3, 4, n);
    dump(stages, ST_S6_FF_IN, n, TD);
    real* h = (real*)malloc(sizeof(real) * (size_t)T * FF);
    linear(n, T, D, BW(W_FF1_W), QW(Q_F1), QS(Q_F1), scale_f16, NULL, FF, h);
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < (size_t)T * FF; i++) h[i] = gelu_tanh(h[i]);
    dump(stages, ST_FF_H, h, (size_t)T * FF);
    linear(h, T, FF, BW(W_FF2_W), QW(Q_F2), QS(Q_F2), scale_f16, NULL, D, a);
    free(h);
    dump(stages, ST_S7_FF_OUT, a, TD);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; t++)
        for (int c = 0; c < D; c++)
            out[(size_t)t * D + c] = x_ca[(size_t)t * D + c] + a[(size_t)t * D + c] * ada(sst, tstab, tidx, t, 5, c);
    free(x);
    free(n);
    free(a);
    free(x_sa);
    return 1;
}

/* Isolated linear for GEMM parity: y = x W^T (+ b), weight from bf16 or q8. */
void orc_linear(const real* x, int M, int K, const uint16_t* wbf, const int8_t* q, const void* s, int scale_f16,
                const uint16_t* b, int N, real* y) {
    linear(x, M, K, wbf, q, s, scale_f16, b, N, y);
}

/* Isolated rms/rmsW rows (w may be NULL). */
void orc_rms(const real* x, int M, int N, const uint16_t* w, real* y) { rms_rows(x, M, N, w, y); }

int orc_real_size(void) { return (int)sizeof(real); }
