// Kernels of the parts around the blocks (ltx/core_parts.zig) and of the
// distilled scheduler (ltx/scheduler.zig). All f32; the linear layers run on
// the f32 GEMM (k_f32.hip).
#include "ltx_device.h"

// DDPM/PixArt sinusoid of t * 1000, cos half first, divisor HALF = 128
// (ltx/core_parts.zig:36-49): freq[k] = exp(k * (-ln(1e4) / 128)) in f32,
// arg = (t * 1000) * freq, out = [cos(arg) | sin(arg)].
extern "C" __global__ void __launch_bounds__(128) ltx_core_sinusoid(const LtxSinArgs a) {
    const int r = blockIdx.x, k = threadIdx.x;
    if (r >= a.rows) return;
    const float freq = expf((float)k * (-9.210340371976184f / 128.0f));
    const float arg = (a.t[r] * 1000.0f) * freq;
    a.out[(size_t)r * 256 + k] = cosf(arg);
    a.out[(size_t)r * 256 + 128 + k] = sinf(arg);
}

// y = x * sigmoid(x) (ltx/core_parts.zig:22-24), elementwise.
extern "C" __global__ void __launch_bounds__(256) ltx_core_silu(const LtxEltArgs a) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= a.n) return;
    const float x = a.x[i];
    a.y[i] = x * (1.0f / (1.0f + expf(-x)));
}

// Output tail norm (ltx/core_parts.zig:26-35, 143-147): mean-subtracting
// LayerNorm without weight, biased variance, eps 1e-6, then
// n * (1 + (fsst[1] + e)) + (fsst[0] + e) with e = emb[tidx[t]]. One
// workgroup of 256 threads per row.
extern "C" __global__ void __launch_bounds__(256) ltx_core_tail_norm(const LtxTailNormArgs a) {
    __shared__ float red[4];
    const int t = blockIdx.x;
    const float* x = a.x + (size_t)t * LTX_D;
    float v[16];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        v[i] = x[threadIdx.x + 256 * i];
        s += v[i];
    }
    const float mean = block_sum256(s, red) / (float)LTX_D;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        v[i] -= mean;
        q += v[i] * v[i];
    }
    const float var = block_sum256(q, red) / (float)LTX_D;
    const float r = 1.0f / sqrtf(var + 1e-6f);
    const float* e = a.emb + (size_t)a.tidx[t] * LTX_D;
    float* y = a.y + (size_t)t * LTX_D;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int c = threadIdx.x + 256 * i;
        const float scl = a.fsst[LTX_D + c] + e[c], shift = a.fsst[c] + e[c];
        y[c] = v[i] * r * (1.0f + scl) + shift;
    }
}

// One Euler step of the distilled sampler on the latent [T][C], in the
// reference's exact f32 operation order and without fused multiply-adds
// (ltx/scheduler.zig:54-80):
//   den  = x - v * ts                       (toDenoised, per-token ts)
//   post = den * m + c * (1 - m)            (postProcess)
//   next = x + ((x - post) / sigma) * dt    (eulerStep, dt = sigma_next - sigma)
// with ts = tk[tidx[t]], m = maskk[tidx[t]] for token t.
extern "C" __global__ void __launch_bounds__(256) ltx_sched_step(const LtxSchedArgs a) {
#pragma clang fp contract(off)
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= a.n) return;
    const int k = a.tidx[i / a.stride];
    const float ts = a.tk[k], m = a.maskk[k];
    const float x = a.x[i];
    const float vts = a.v[i] * ts;
    const float den = x - vts;
    const float dm = den * m;
    const float om = 1.0f - m;
    const float cm = a.clean[i] * om;
    const float post = dm + cm;
    const float dt = a.sigma_next - a.sigma;
    const float vel = (x - post) / a.sigma;
    const float step = vel * dt;
    a.y[i] = x + step;
}

// torch.lerp as the reference computes it (ltx/scheduler.zig:21-33): the
// branch on |w| < 0.5 and one fused multiply-add in either branch.
__device__ __forceinline__ float sched_lerp(float a, float b, float w) {
#pragma clang fp contract(off)
    const float d = b - a;
    if (fabsf(w) < 0.5f) return __builtin_fmaf(w, d, a);
    return __builtin_fmaf(-d, 1.0f - w, b);
}

// GaussianNoiser at state initialisation (ltx/scheduler.zig:38-46):
// x = lerp(clean, noise, noise_scale); out = lerp(clean, x, mask[token]).
extern "C" __global__ void __launch_bounds__(256) ltx_sched_noise_init(const LtxNoiseArgs a) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= a.n) return;
    const float c = a.clean[i];
    const float x = sched_lerp(c, a.noise[i], a.noise_scale);
    a.y[i] = sched_lerp(c, x, a.maskk[a.tidx[i / a.stride]]);
}

// t[k] = mask[k] * sigma (ltx/scheduler.zig:48-51), one value per distinct
// mask value, and t[K] = sigma itself (the prompt conditioning's input), so a
// step needs no host-to-device copy. K < 64.
extern "C" __global__ void __launch_bounds__(64) ltx_sched_timesteps(const LtxTimestepArgs a) {
#pragma clang fp contract(off)
    const int k = threadIdx.x;
    if (k < a.K) a.tk[k] = a.maskk[k] * a.sigma;
    else if (k == a.K) a.tk[k] = a.sigma;
}
