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

/* C[M][N] = A[M][K] * Bt[K][N]. Every output is one chain of fused
 * multiply-adds over k in ascending order (the accumulator goes to C and back
 * between k-blocks, which does not change the chain), so a row's result does
 * not depend on the blocking or on which other rows are computed with it.
 * Blocked for the caches: k-blocks of KC, micro-tiles of MR x NR outputs
 * held in registers. */
#include <immintrin.h>
#ifdef REAL_F32
typedef __m256 vreal;
#define VW 8
#define V_LOAD _mm256_loadu_ps
#define V_STORE _mm256_storeu_ps
#define V_BCAST _mm256_broadcast_ss
#define V_FMA _mm256_fmadd_ps
#else
typedef __m256d vreal;
#define VW 4
#define V_LOAD _mm256_loadu_pd
#define V_STORE _mm256_storeu_pd
#define V_BCAST _mm256_broadcast_sd
#define V_FMA _mm256_fmadd_pd
#endif
#define MR 6
#define NR (2 * VW)
#define KC 256
#define MC 48
#define NC 256

static inline real fma_r(real a, real b, real c) {
    return sizeof(real) == sizeof(double) ? (real)__builtin_fma((double)a, (double)b, (double)c)
                                          : (real)__builtin_fmaf((float)a, (float)b, (float)c);
}

/* A full MR x NR tile: twelve vector accumulators, one broadcast of A per
 * row and k (vfmadd: one rounding, as fma_r). */
static inline void gemm_micro_full(const real* A, int lda, const real* B, int ldb, real* C, int ldc, int kc) {
#define ROW_LOAD(i) vreal c##i##0 = V_LOAD(C + (size_t)(i) * ldc), c##i##1 = V_LOAD(C + (size_t)(i) * ldc + VW);
#define ROW_FMA(i)                                              \
    {                                                           \
        const vreal a = V_BCAST(A + (size_t)(i) * lda + k);     \
        c##i##0 = V_FMA(a, b0, c##i##0);                        \
        c##i##1 = V_FMA(a, b1, c##i##1);                        \
    }
#define ROW_STORE(i)                                  \
    V_STORE(C + (size_t)(i) * ldc, c##i##0);          \
    V_STORE(C + (size_t)(i) * ldc + VW, c##i##1);
    ROW_LOAD(0) ROW_LOAD(1) ROW_LOAD(2) ROW_LOAD(3) ROW_LOAD(4) ROW_LOAD(5)
    for (int k = 0; k < kc; k++) {
        const vreal b0 = V_LOAD(B + (size_t)k * ldb), b1 = V_LOAD(B + (size_t)k * ldb + VW);
        ROW_FMA(0) ROW_FMA(1) ROW_FMA(2) ROW_FMA(3) ROW_FMA(4) ROW_FMA(5)
    }
    ROW_STORE(0) ROW_STORE(1) ROW_STORE(2) ROW_STORE(3) ROW_STORE(4) ROW_STORE(5)
#undef ROW_LOAD
#undef ROW_FMA
#undef ROW_STORE
}

static inline void gemm_micro(const real* A, int lda, const real* B, int ldb, real* C, int ldc, int mr, int nr,
                              int kc) {
    if (mr == MR && nr == NR) {
        gemm_micro_full(A, lda, B, ldb, C, ldc, kc);
        return;
    }
    real acc[MR][NR];
    for (int i = 0; i < mr; i++)
        for (int j = 0; j < nr; j++) acc[i][j] = C[(size_t)i * ldc + j];
    for (int k = 0; k < kc; k++) {
        const real* b = B + (size_t)k * ldb;
        for (int i = 0; i < mr; i++) {
            const real a = A[(size_t)i * lda + k];
            for (int j = 0; j < nr; j++) acc[i][j] = fma_r(a, b[j], acc[i][j]);
        }
    }
    for (int i = 0; i < mr; i++)
        for (int j = 0; j < nr; j++) C[(size_t)i * ldc + j] = acc[i][j];
}

static void gemm_kn(const real* A, int M, int K, const real* Bt, int N, real* C) {
    const int nmb = (M + MC - 1) / MC, nnb = (N + NC - 1) / NC;
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; m++) memset(C + (size_t)m * N, 0, sizeof(real) * (size_t)N);
    for (int k0 = 0; k0 < K; k0 += KC) {
        const int kc = K - k0 < KC ? K - k0 : KC;
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
        for (int nb = 0; nb < nnb; nb++)
            for (int mb = 0; mb < nmb; mb++) {
                const int n0 = nb * NC, m0 = mb * MC;
                const int n1 = N < n0 + NC ? N : n0 + NC, m1 = M < m0 + MC ? M : m0 + MC;
                for (int n = n0; n < n1; n += NR)
                    for (int m = m0; m < m1; m += MR)
                        gemm_micro(A + (size_t)m * K + k0, K, Bt + (size_t)k0 * N + n, N, C + (size_t)m * N + n, N,
                                   m1 - m < MR ? m1 - m : MR, n1 - n < NR ? n1 - n : NR, kc);
            }
    }
}

/* Transposed weight [K][N] from a bf16 [N][K] tensor or an int8 [N][K] +
 * scale [N][K/128] pair (dq4 semantics: f32(q)*s rounded once to f32). */
static real* weight_t(const uint16_t* wbf, const int8_t* q, const void* s, int scale_f16, int N, int K) {
    real* wt = (real*)malloc(sizeof(real) * (size_t)N * K);
    const int G = K / 128, TB = 64;
    const int ntn = (N + TB - 1) / TB, ntk = (K + TB - 1) / TB;
    /* 64 x 64 tiles, so the transposed stores stay within a few cache lines */
#pragma omp parallel for collapse(2) schedule(static)
    for (int tn = 0; tn < ntn; tn++)
        for (int tk = 0; tk < ntk; tk++) {
            const int n1 = N < (tn + 1) * TB ? N : (tn + 1) * TB, k1 = K < (tk + 1) * TB ? K : (tk + 1) * TB;
            for (int n = tn * TB; n < n1; n++)
                for (int k = tk * TB; k < k1; k++) {
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
        }
    return wt;
}

/* Few rows (M <= SMALL_M): the weight is dequantised panel by panel (NP
 * columns x KC k at a time) into a per-thread buffer and multiplied with the
 * same micro-kernels; the whole transposed weight (and the page faults of
 * allocating it per call) is never built. Each output is still one chain of
 * fused multiply-adds over k in ascending order from 0, the accumulator
 * passing through C between k-blocks unchanged, so the result is bit-identical
 * to gemm_kn's for every row. */
#define SMALL_M 256
#define NP 64
static void linear_small(const real* x, int M, int K, const uint16_t* wbf, const int8_t* q, const void* s,
                         int scale_f16, int N, real* y) {
    const int G = K / 128;
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; m++) memset(y + (size_t)m * N, 0, sizeof(real) * (size_t)N);
#pragma omp parallel
    {
        real* pan = (real*)malloc(sizeof(real) * (size_t)KC * NP);
#pragma omp for schedule(dynamic, 1)
        for (int n0 = 0; n0 < N; n0 += NP) {
            const int np = N - n0 < NP ? N - n0 : NP;
            for (int k0 = 0; k0 < K; k0 += KC) {
                const int kc = K - k0 < KC ? K - k0 : KC;
                for (int j = 0; j < np; j++) {
                    const size_t n = (size_t)(n0 + j);
                    for (int k = 0; k < kc; k++) {
                        const size_t kk = (size_t)(k0 + k);
                        real v;
                        if (q) {
                            float sc = scale_f16 ? f16_to_f32(((const uint16_t*)s)[n * G + kk / 128])
                                                 : ((const float*)s)[n * G + kk / 128];
                            v = (real)((float)q[n * K + kk] * sc);
                        } else {
                            v = bfr(wbf, n * K + kk);
                        }
                        pan[(size_t)k * NP + j] = v;
                    }
                }
                for (int m = 0; m < M; m += MR)
                    for (int j = 0; j < np; j += NR)
                        gemm_micro(x + (size_t)m * K + k0, K, pan + j, NP, y + (size_t)m * N + n0 + j, N,
                                   M - m < MR ? M - m : MR, np - j < NR ? np - j : NR, kc);
            }
        }
        free(pan);
    }
}

/* lin / linQ (ltx/block.zig:22-26, 473-477): y = x W^T (+ b) */
static void linear(const real* x, int M, int K, const uint16_t* wbf, const int8_t* q, const void* s,
                   int scale_f16, const uint16_t* b, int N, real* y) {
    if (M <= SMALL_M) {
        linear_small(x, M, K, wbf, q, s, scale_f16, N, y);
    } else {
        real* wt = weight_t(wbf, q, s, scale_f16, N, K);
        gemm_kn(x, M, K, wt, N, y);
        free(wt);
    }
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

/* adaVal (ltx/block.zig:47-67): ada_i[t] = tstab[row(t), i] + sst[i]. The
 * reference selects the row with a chain over k = 1 .. K-1 starting from row
 * 0, so an index outside 1 .. K-1 takes row 0 (ada_rows resolves that once
 * per token; `trow` below holds the resolved rows). */
static int32_t* ada_rows(const int32_t* tidx, const int* rows, int n, int K) {
    int32_t* r = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n > 0 ? n : 1));
    for (int i = 0; i < n; i++) {
        const int32_t k = tidx[rows ? rows[i] : i];
        r[i] = (k >= 1 && k < K) ? k : 0;
    }
    return r;
}

static inline real ada(const float* sst, const float* tstab, const int32_t* trow, int t, int i, int c) {
    return (real)tstab[((size_t)trow[t] * 9 + i) * D + c] + (real)sst[(size_t)i * D + c];
}

/* modulate(rms(x), ada[isc], ada[ish]) (ltx/block.zig:36-38, 248-252) */
static void norm_mod(const real* x, int T, const float* sst, const float* tstab, const int32_t* trow,
                     int ish, int isc, real* y) {
    rms_rows(x, T, D, NULL, y);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; t++)
        for (int c = 0; c < D; c++) {
            real n = y[(size_t)t * D + c];
            y[(size_t)t * D + c] = n * (ada(sst, tstab, trow, t, isc, c) + 1) + ada(sst, tstab, trow, t, ish, c);
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

/* Stage dumps, in forward order (glog1 / glog2, the gate logits, last). */
enum {
    ST_S1_NORM_MSA, ST_Q1_ROPED, ST_K1_ROPED, ST_V1, ST_ATTN1_MERGED, ST_S3_ATTN1, ST_S4_AFTER_SA,
    ST_S4_NORMED, ST_ATTN_IN, ST_ENC, ST_Q2_NORMED, ST_K2_NORMED, ST_V2, ST_ATTN2_MERGED, ST_S5_CA_OUT,
    ST_X_CA, ST_S6_FF_IN, ST_FF_H, ST_S7_FF_OUT, ST_GLOG1, ST_GLOG2, ST_COUNT
};

static void dump(real* const* stages, int id, const real* src, size_t n) {
    if (stages && stages[id]) memcpy(stages[id], src, sizeof(real) * n);
}

#define BW(i) ((const uint16_t*)base[i])
#define QW(i) (q8 ? q8[i] : NULL)
#define QS(i) (q8s ? q8s[i] : NULL)

/* One attention (Block.attention, ltx/block.zig:212-244 / QBlock,
 * ltx/block.zig:500-530, 557-567): q = rmsW(lin(xq)), k = rmsW(lin(xkv)),
 * v = lin(xkv), RoPE on q and k when tables are given (rows of q and k each
 * with their own [rows][H][64] tables), sdpa, gate 2*sigmoid(lin(xq, gw, gb))
 * per (token, head) from the attention input, merge heads, output
 * projection. Every op but the sdpa is row-local, so xq may be any subset of
 * the query rows. Weight slot ids index both base (bf16) and q8 tables. */
static void attention(const void* const* base, const int8_t* const* q8, const void* const* q8s, int sf16,
                      const real* xq, int Tq, const float* csq, const float* snq, const real* xkv, int S,
                      const float* cskv, const float* snkv, int bq, int bk, int bv, int bo, int iqn, int ikn, int igw,
                      int qq, int qk, int qv, int qo, int chunk, real* out, real* const* stages, int st_q, int st_k,
                      int st_v, int st_merged, int st_glog) {
    real* q = (real*)malloc(sizeof(real) * (size_t)Tq * D);
    real* k = (real*)malloc(sizeof(real) * (size_t)S * D);
    real* v = (real*)malloc(sizeof(real) * (size_t)S * D);
    real* o = (real*)malloc(sizeof(real) * (size_t)Tq * D);
    linear(xq, Tq, D, BW(bq), QW(qq), QS(qq), sf16, BW(bq + 1), D, q);
    rms_rows(q, Tq, D, BW(iqn), q);
    linear(xkv, S, D, BW(bk), QW(qk), QS(qk), sf16, BW(bk + 1), D, k);
    rms_rows(k, S, D, BW(ikn), k);
    linear(xkv, S, D, BW(bv), QW(qv), QS(qv), sf16, BW(bv + 1), D, v);
    if (csq) {
        rope_apply(q, Tq, csq, snq);
        rope_apply(k, S, cskv, snkv);
    }
    dump(stages, st_q, q, (size_t)Tq * D);
    dump(stages, st_k, k, (size_t)S * D);
    dump(stages, st_v, v, (size_t)S * D);
    if (!orc_sdpa(q, Tq, k, v, S, chunk, o)) { /* chunk must divide the key count */
        memset(o, 0xff, sizeof(real) * (size_t)Tq * D); /* NaN: fails loudly */
    }
    real* glog = (real*)malloc(sizeof(real) * (size_t)Tq * H);
    linear(xq, Tq, D, BW(igw), NULL, NULL, 0, BW(igw + 1), H, glog);
    dump(stages, st_glog, glog, (size_t)Tq * H);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < Tq; t++)
        for (int h = 0; h < H; h++) {
            real g = sigmoid_r(glog[(size_t)t * H + h]) * 2;
            for (int e = 0; e < HD; e++) o[(size_t)t * D + h * HD + e] *= g;
        }
    dump(stages, st_merged, o, (size_t)Tq * D);
    linear(o, Tq, D, BW(bo), QW(qo), QS(qo), sf16, BW(bo + 1), D, out);
    free(glog);
    free(q);
    free(k);
    free(v);
    free(o);
}

/* Rows `rows[0 .. nr)` of a [T][w] table (every row when rows is NULL). */
static float* gather_f32(const float* src, const int* rows, int nr, size_t w) {
    float* d = (float*)malloc(sizeof(float) * (size_t)nr * w);
    for (int i = 0; i < nr; i++) memcpy(d + (size_t)i * w, src + (size_t)rows[i] * w, sizeof(float) * w);
    return d;
}

/* QBlock.qBlockOutAll (ltx/block.zig:544-574) with the self-attention
 * computed blockwise (chunk) — the production attention algorithm
 * (ltx/block.zig:105-154); cross-attention dense (cross_chunk 0) as in the
 * reference, or blockwise. q8[i] == NULL selects the bf16 base weight.
 *
 * Output rows: all T tokens (rows == NULL), or only the tokens rows[0 .. nr)
 * (out is [nr][D]). Every op except the self-attention is token-local, so a
 * subset computes the modulated norm, K and V of every token (the keys) and
 * everything else for its own rows only; each of its rows equals that row of
 * the whole block (the same operations in the same order). Stage dumps
 * follow the computed rows: K1 / V1 have T rows, ENC / K2 / V2 have S, the
 * rest nr. */
static int block_rows(const void* const* base, const int8_t* const* q8, const void* const* q8s, int scale_f16,
                      const float* x_in, const float* tstab, int K, const int32_t* tidx, const float* ctx_in, int S,
                      const float* pts2, const float* cs, const float* sn, int T, int chunk, int cross_chunk,
                      const int* rows, int nr, real* out, real* const* stages) {
    if (K <= 0 || T <= 0 || S <= 0) return 0;
    if (rows) {
        if (nr <= 0) return 0;
        for (int i = 0; i < nr; i++)
            if (rows[i] < 0 || rows[i] >= T) return 0;
    } else {
        nr = T;
    }
    const float* sst = (const float*)base[W_SST];
    const float* psst = (const float*)base[W_PSST];
    const size_t TD = (size_t)T * D, RD = (size_t)nr * D;
    int32_t* trow_all = ada_rows(tidx, NULL, T, K);
    int32_t* trow = rows ? ada_rows(tidx, rows, nr, K) : trow_all;
    real* x = (real*)malloc(sizeof(real) * RD);  /* the output rows' x, later x_ca */
    real* n_all = (real*)malloc(sizeof(real) * TD);
    real* a = (real*)malloc(sizeof(real) * RD);
    real* x_sa = (real*)malloc(sizeof(real) * RD);
    {
        real* x_all = (real*)malloc(sizeof(real) * TD);
        for (size_t i = 0; i < TD; i++) x_all[i] = x_in[i];
        /* self-attention: n = modulate(rms(x), ada1, ada0), for every token */
        norm_mod(x_all, T, sst, tstab, trow_all, 0, 1, n_all);
        for (int i = 0; i < nr; i++)
            memcpy(x + (size_t)i * D, x_all + (size_t)(rows ? rows[i] : i) * D, sizeof(real) * D);
        free(x_all);
    }
    real* n = (real*)malloc(sizeof(real) * RD);  /* the output rows' modulated norm */
    for (int i = 0; i < nr; i++) memcpy(n + (size_t)i * D, n_all + (size_t)(rows ? rows[i] : i) * D, sizeof(real) * D);
    dump(stages, ST_S1_NORM_MSA, n, RD);
    float* csq = rows ? gather_f32(cs, rows, nr, (size_t)H * 64) : NULL;
    float* snq = rows ? gather_f32(sn, rows, nr, (size_t)H * 64) : NULL;
    attention(base, q8, q8s, scale_f16, n, nr, rows ? csq : cs, rows ? snq : sn, n_all, T, cs, sn, W_Q1_W, W_K1_W,
              W_V1_W, W_O1_W, W_QN1, W_KN1, W_G1_W, Q_Q1, Q_K1, Q_V1, Q_O1, chunk, a, stages, ST_Q1_ROPED,
              ST_K1_ROPED, ST_V1, ST_ATTN1_MERGED, ST_GLOG1);
    free(csq);
    free(snq);
    free(n_all);
    dump(stages, ST_S3_ATTN1, a, RD);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < nr; t++)
        for (int c = 0; c < D; c++)
            x_sa[(size_t)t * D + c] = x[(size_t)t * D + c] + a[(size_t)t * D + c] * ada(sst, tstab, trow, t, 2, c);
    dump(stages, ST_S4_AFTER_SA, x_sa, RD);

    /* cross-attention (ltx/block.zig:548-568) */
    rms_rows(x_sa, nr, D, NULL, n);
    dump(stages, ST_S4_NORMED, n, RD);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < nr; t++)
        for (int c = 0; c < D; c++) {
            real v = n[(size_t)t * D + c];
            n[(size_t)t * D + c] = v * (ada(sst, tstab, trow, t, 7, c) + 1) + ada(sst, tstab, trow, t, 6, c);
        }
    dump(stages, ST_ATTN_IN, n, RD);
    real* enc = (real*)malloc(sizeof(real) * (size_t)S * D);
    for (int t = 0; t < S; t++)
        for (int c = 0; c < D; c++) {
            real sh = (real)psst[c] + (real)pts2[c];
            real sc = (real)psst[D + c] + (real)pts2[D + c];
            enc[(size_t)t * D + c] = (real)ctx_in[(size_t)t * D + c] * (sc + 1) + sh;
        }
    dump(stages, ST_ENC, enc, (size_t)S * D);
    attention(base, q8, q8s, scale_f16, n, nr, NULL, NULL, enc, S, NULL, NULL, W_Q2_W, W_K2_W, W_V2_W, W_O2_W, W_QN2,
              W_KN2, W_G2_W, Q_Q2, Q_K2, Q_V2, Q_O2, cross_chunk, a, stages, ST_Q2_NORMED, ST_K2_NORMED, ST_V2,
              ST_ATTN2_MERGED, ST_GLOG2);
    free(enc);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < nr; t++)
        for (int c = 0; c < D; c++) a[(size_t)t * D + c] *= ada(sst, tstab, trow, t, 8, c);
    dump(stages, ST_S5_CA_OUT, a, RD);
    real* x_ca = x; /* reuse */
    for (size_t i = 0; i < RD; i++) x_ca[i] = x_sa[i] + a[i];
    dump(stages, ST_X_CA, x_ca, RD);

    /* feed-forward (ltx/block.zig:569-573, qFf 532-534) */
    norm_mod(x_ca, nr, sst, tstab, trow, 3, 4, n);
    dump(stages, ST_S6_FF_IN, n, RD);
    real* h = (real*)malloc(sizeof(real) * (size_t)nr * FF);
    linear(n, nr, D, BW(W_FF1_W), QW(Q_F1), QS(Q_F1), scale_f16, NULL, FF, h);
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < (size_t)nr * FF; i++) h[i] = gelu_tanh(h[i]);
    dump(stages, ST_FF_H, h, (size_t)nr * FF);
    linear(h, nr, FF, BW(W_FF2_W), QW(Q_F2), QS(Q_F2), scale_f16, NULL, D, a);
    free(h);
    dump(stages, ST_S7_FF_OUT, a, RD);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < nr; t++)
        for (int c = 0; c < D; c++)
            out[(size_t)t * D + c] = x_ca[(size_t)t * D + c] + a[(size_t)t * D + c] * ada(sst, tstab, trow, t, 5, c);
    free(x);
    free(n);
    free(a);
    free(x_sa);
    if (trow != trow_all) free(trow);
    free(trow_all);
    return 1;
}

/* The whole block: every token (out [T][D]). */
int orc_block_forward(const void* const* base, const int8_t* const* q8, const void* const* q8s, int scale_f16,
                      const float* x_in, const float* tstab, int K, const int32_t* tidx, const float* ctx_in,
                      int S, const float* pts2, const float* cs, const float* sn, int T, int chunk,
                      int cross_chunk, real* out, real* const* stages) {
    return block_rows(base, q8, q8s, scale_f16, x_in, tstab, K, tidx, ctx_in, S, pts2, cs, sn, T, chunk, cross_chunk,
                      NULL, 0, out, stages);
}

/* Output rows rows[0 .. nr) of the block (out [nr][D]); each equals that row
 * of orc_block_forward. */
int orc_block_rows(const void* const* base, const int8_t* const* q8, const void* const* q8s, int scale_f16,
                   const float* x_in, const float* tstab, int K, const int32_t* tidx, const float* ctx_in, int S,
                   const float* pts2, const float* cs, const float* sn, int T, int chunk, int cross_chunk,
                   const int* rows, int nr, real* out, real* const* stages) {
    if (!rows) return 0;
    return block_rows(base, q8, q8s, scale_f16, x_in, tstab, K, tidx, ctx_in, S, pts2, cs, sn, T, chunk, cross_chunk,
                      rows, nr, out, stages);
}

/* Isolated linear for GEMM parity: y = x W^T (+ b), weight from bf16 or q8. */
void orc_linear(const real* x, int M, int K, const uint16_t* wbf, const int8_t* q, const void* s, int scale_f16,
                const uint16_t* b, int N, real* y) {
    linear(x, M, K, wbf, q, s, scale_f16, b, N, y);
}

/* Isolated rms/rmsW rows (w may be NULL). */
void orc_rms(const real* x, int M, int N, const uint16_t* w, real* y) { rms_rows(x, M, N, w, y); }

int orc_real_size(void) { return (int)sizeof(real); }

/* Isolated split-half RoPE application, in place on x [T][4096] with cos/sin
 * in graph layout [T][32][64] (ltx/block.zig:69-77). */
void orc_rope_apply(real* x, int T, const float* cs, const float* sn) { rope_apply(x, T, cs, sn); }

/* Isolated GELU, tanh form (ltx/block.zig:332), elementwise over n values. */
void orc_gelu(const real* x, long n, real* y) {
    for (long i = 0; i < n; i++) y[i] = gelu_tanh(x[i]);
}
