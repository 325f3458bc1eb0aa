// Practical MFMA ceiling of one MI355X: the rate of v_mfma_f32_32x32x16_{f16,bf16}
// loops on random operands, with the A operand from registers, from one
// ds_read_b128 per MFMA (the GEMMs' and the 32x32x16 attention's fragment
// rate) or from one read per two MFMAs; and of v_mfma_f32_16x16x32_f16 (the
// attention's shape) from registers and from one read per two MFMAs (the same
// LDS bytes per flop as one read per 32x32x16). The published dense peak assumes the top clock; under a
// sustained MFMA load the board's power limit sets a lower clock, and that
// clock depends on the operand type and on the operands' bits.
//
// Shape: 1024 workgroups of 8 waves (two per SIMD), 96 KB of LDS each so that
// one workgroup holds a CU; each wave runs ITERS x 16 MFMAs over four
// accumulators, fragments read four MFMAs ahead. LDS reads stay in the first
// 16 KB (index < 1024 of u32x4). Prints one JSON line: TFLOP/s per variant,
// the median of 7 timed launches after one warm-up round.
//
// Build: part of ltx-zml_amd/build.py (-> ltx-zml_amd/mfma_ceiling).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <vector>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

enum { SRC_REGS = 0, SRC_LDS = 1, SRC_LDS_HALF = 2 };

__device__ __forceinline__ uint32_t mix(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

// two random 16-bit values in (-1, 1): random sign and significand, exponent
// drawn from the top 7 binades below 1
template <bool BF>
__device__ __forceinline__ uint32_t rand_pair(uint32_t x) {
    uint32_t r = 0;
    for (int h = 0; h < 2; h++) {
        const uint32_t b = mix(x * 2u + (uint32_t)h + 0x9e3779b9u);
        const uint32_t v = BF ? ((b & 0x807fu) | ((120u + (b >> 7) % 7u) << 7))
                              : ((b & 0x83ffu) | ((8u + (b >> 10) % 7u) << 10));
        r |= v << (16 * h);
    }
    return r;
}

template <bool BF, int SRC>
__global__ void __launch_bounds__(512) ceiling(float* out, int iters) {
    using V = typename std::conditional<BF, bf16x8, f16x8>::type;
    __shared__ u32x4 lds[6144];  // 96 KB: one workgroup per CU
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    for (int i = threadIdx.x; i < 1024; i += 512)
        lds[i] = u32x4{rand_pair<BF>(4 * i), rand_pair<BF>(4 * i + 1), rand_pair<BF>(4 * i + 2),
                       rand_pair<BF>(4 * i + 3)};
    __syncthreads();
    const uint32_t s0 = 4096u + 8u * (uint32_t)lane;
    const V b = __builtin_bit_cast(V, u32x4{rand_pair<BF>(s0), rand_pair<BF>(s0 + 1), rand_pair<BF>(s0 + 2),
                                            rand_pair<BF>(s0 + 3)});
    const V areg = __builtin_bit_cast(V, u32x4{rand_pair<BF>(s0 + 4), rand_pair<BF>(s0 + 5),
                                               rand_pair<BF>(s0 + 6), rand_pair<BF>(s0 + 7)});
    f32x16 acc[4];
    for (int i = 0; i < 4; i++)
        for (int e = 0; e < 16; e++) acc[i][e] = 0.0f;
    // fragment q: 1 KB of the 16 KB, rotating per wave
    auto load = [&](int q) -> V {
        if (SRC == SRC_REGS) return areg;
        return __builtin_bit_cast(V, lds[((w + q) & 15) * 64 + lane]);
    };
    V fr[4];
    for (int j = 0; j < 4; j++) fr[j] = load(j);
    int q = 4;
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const int f = SRC == SRC_LDS_HALF ? (j >> 1) & 3 : j & 3;
            if (BF)
                acc[j & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fr[f], b, acc[j & 3], 0, 0, 0);
            else
                acc[j & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fr[f], b, acc[j & 3], 0, 0, 0);
            if (SRC != SRC_LDS_HALF || (j & 1)) fr[f] = load(q++);
            __builtin_amdgcn_sched_barrier(0);  // keep MFMA j before the read for MFMA j + 4
        }
    }
    float t = 0.0f;
    for (int i = 0; i < 4; i++)
        for (int e = 0; e < 16; e++) t += acc[i][e];
    out[(size_t)blockIdx.x * 512 + threadIdx.x] = t;
}

// 16x16x32 f16: 32 MFMAs per iteration (the flops of 16 of 32x32x16) over
// eight accumulators; SRC_LDS_HALF reads one fragment per two MFMAs
template <int SRC>
__global__ void __launch_bounds__(512) ceiling16(float* out, int iters) {
    __shared__ u32x4 lds[6144];  // 96 KB: one workgroup per CU
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    for (int i = threadIdx.x; i < 1024; i += 512)
        lds[i] = u32x4{rand_pair<false>(4 * i), rand_pair<false>(4 * i + 1), rand_pair<false>(4 * i + 2),
                       rand_pair<false>(4 * i + 3)};
    __syncthreads();
    const uint32_t s0 = 4096u + 8u * (uint32_t)lane;
    const f16x8 b = __builtin_bit_cast(f16x8, u32x4{rand_pair<false>(s0), rand_pair<false>(s0 + 1),
                                                    rand_pair<false>(s0 + 2), rand_pair<false>(s0 + 3)});
    const f16x8 areg = __builtin_bit_cast(f16x8, u32x4{rand_pair<false>(s0 + 4), rand_pair<false>(s0 + 5),
                                                       rand_pair<false>(s0 + 6), rand_pair<false>(s0 + 7)});
    f32x4 acc[8];
    for (int i = 0; i < 8; i++)
        for (int e = 0; e < 4; e++) acc[i][e] = 0.0f;
    auto load = [&](int q) -> f16x8 {
        if (SRC == SRC_REGS) return areg;
        return __builtin_bit_cast(f16x8, lds[((w + q) & 15) * 64 + lane]);
    };
    f16x8 fr[4];
    for (int j = 0; j < 4; j++) fr[j] = load(j);
    int q = 4;
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int j = 0; j < 32; j++) {
            const int f = (j >> 1) & 3;
            acc[j & 7] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fr[f], b, acc[j & 7], 0, 0, 0);
            if (SRC != SRC_REGS && (j & 1)) fr[f] = load(q++);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    float t = 0.0f;
    for (int i = 0; i < 8; i++)
        for (int e = 0; e < 4; e++) t += acc[i][e];
    out[(size_t)blockIdx.x * 512 + threadIdx.x] = t;
}

struct Variant {
    const char* name;
    void (*kern)(float*, int);
};

int main(int argc, char** argv) {
    const int nwg = 1024, iters = argc > 1 ? std::max(1, atoi(argv[1])) : 500;
    float* out = nullptr;
    if (hipMalloc(&out, (size_t)nwg * 512 * sizeof(float)) != hipSuccess) {
        fprintf(stderr, "hipMalloc failed\n");
        return 1;
    }
    const Variant vars[] = {
        {"f16_regs", ceiling<false, SRC_REGS>},         {"f16_lds_per_mfma", ceiling<false, SRC_LDS>},
        {"f16_lds_per_2mfma", ceiling<false, SRC_LDS_HALF>}, {"bf16_regs", ceiling<true, SRC_REGS>},
        {"bf16_lds_per_mfma", ceiling<true, SRC_LDS>},   {"bf16_lds_per_2mfma", ceiling<true, SRC_LDS_HALF>},
        {"f16_16x16x32_regs", ceiling16<SRC_REGS>},      {"f16_16x16x32_lds_per_2mfma", ceiling16<SRC_LDS_HALF>},
    };
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return 1;
    const double flop = (double)nwg * 8 * iters * 16 * (32.0 * 32 * 16 * 2);
    printf("{\"tool\": \"mfma_ceiling\", \"workgroups\": %d, \"waves_per_simd\": 2, \"iters\": %d, \"tflops\": {", nwg,
           iters);
    // variants interleaved launch by launch, so that a drift of the clock
    // over the run (temperature, power state) spreads over all of them
    constexpr int NV = sizeof(vars) / sizeof(vars[0]), REPS = 7;
    std::vector<float> ms[NV];
    for (int rep = 0; rep <= REPS; rep++)
        for (int i = 0; i < NV; i++) {
            hipEventRecord(e0);
            hipLaunchKernelGGL(vars[i].kern, dim3(nwg), dim3(512), 0, 0, out, iters);
            hipEventRecord(e1);
            if (hipEventSynchronize(e1) != hipSuccess) return 2;
            float t = 0.0f;
            hipEventElapsedTime(&t, e0, e1);
            if (rep) ms[i].push_back(t);  // the first repetition warms up
        }
    for (int i = 0; i < NV; i++) {
        std::sort(ms[i].begin(), ms[i].end());
        printf("%s\"%s\": %.1f", i ? ", " : "", vars[i].name, flop / (ms[i][REPS / 2] * 1e-3) / 1e12);
    }
    printf("}}\n");
    if (hipGetLastError() != hipSuccess) return 2;
    return hipFree(out) == hipSuccess ? 0 : 1;
}
