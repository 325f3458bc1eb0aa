// Device-side helpers shared by the gfx950 kernels: 16-bit operand traits,
// MFMA wrappers, conversions, the AdaLN gather and block reductions.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "ltx_args.h"

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Operand traits: the MFMA operand type (f16 or bf16), its 8-wide vector,
// f32 -> 16-bit rounding (round-to-nearest-even) and the 32x32x16 MFMA.
template <typename T>
struct Op;

template <>
struct Op<_Float16> {
    typedef f16x8 v8;
    static __device__ __forceinline__ uint16_t bits(float f) {
        _Float16 h = (_Float16)f;
        return __builtin_bit_cast(uint16_t, h);
    }
    static __device__ __forceinline__ float to_f32(uint16_t b) {
        return (float)__builtin_bit_cast(_Float16, b);
    }
    static __device__ __forceinline__ f32x16 mfma32(v8 a, v8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ f32x4 mfma16(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
    // two f32 -> packed pair, one v_cvt_pk_f16_f32 (round to nearest even)
    static __device__ __forceinline__ uint32_t cvt2(float a, float b) {
        return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
    }
    // acc + lo + hi of a packed pair, each half widened exactly (two
    // v_fma_mix_f32 with 1.0). The dot2 forms would do this in one
    // instruction, but they issue to the matrix pipeline and wait behind
    // another wave's MFMAs.
    static __device__ __forceinline__ float sum2(uint32_t p, float acc) {
        asm("v_fma_mix_f32 %0, %1, 1.0, %0 op_sel_hi:[1,0,0]\n\t"
            "v_fma_mix_f32 %0, %1, 1.0, %0 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
            : "+v"(acc)
            : "v"(p));
        return acc;
    }
};

template <>
struct Op<__bf16> {
    typedef bf16x8 v8;
    static __device__ __forceinline__ uint16_t bits(float f) {
        __bf16 h = (__bf16)f;
        return __builtin_bit_cast(uint16_t, h);
    }
    static __device__ __forceinline__ float to_f32(uint16_t b) {
        return __builtin_bit_cast(float, (uint32_t)b << 16);
    }
    static __device__ __forceinline__ f32x16 mfma32(v8 a, v8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ f32x4 mfma16(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t cvt2(float a, float b) {
        return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
    }
    // acc + lo + hi of a packed pair, widened exactly on the VALU (see the
    // f16 form)
    static __device__ __forceinline__ float sum2(uint32_t p, float acc) {
        return (acc + __builtin_bit_cast(float, p << 16)) + __builtin_bit_cast(float, p & 0xffff0000u);
    }
};

// Range guard of the 16-bit stores: 1 when v is not finite or beyond the
// operand type's largest finite value (its 16-bit rounding saturates to inf).
template <typename T>
struct RangeMax;
template <>
struct RangeMax<_Float16> {
    static constexpr float v = 65504.0f;
};
template <>
struct RangeMax<__bf16> {
    static constexpr float v = 3.38953139e38f;
};
template <typename T>
__device__ __forceinline__ unsigned out_of_range(float v) {
    return __builtin_fabsf(v) <= RangeMax<T>::v ? 0u : 1u;
}
// One vector atomic per lane that saw any (none in the ordinary case).
__device__ __forceinline__ void range_report(unsigned long long* sat, unsigned n) {
    if (n && sat) atomicAdd(sat, (unsigned long long)n);
}

// threadIdx.x through an empty volatile asm: values derived from it cannot be
// hoisted out of the loop that contains the call. Epilogues inside a
// persistent tile loop take their lane from it, so that their address
// arithmetic is recomputed per tile instead of living across the main loop,
// where registers are short (the hoisted values were spilled and their
// reloads waited behind the tile's stores).
__device__ __forceinline__ int opaque_tid() {
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

// Pack two f32 into two 16-bit lanes of one dword (lo = a).
template <typename T>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    return (uint32_t)Op<T>::bits(a) | ((uint32_t)Op<T>::bits(b) << 16);
}

// Dequantised 16-bit weight operands for two int8 values. u = q + 128 is the
// byte read as unsigned (q ^ 0x80), nb = -128 s; fma(u, s, nb) is the exact
// q * s rounded once to f32 — the dq4 value of ltx/block.zig:462-471. The
// 16-bit operand is then: f16 — the compiler fuses fma + convert into
// v_fma_mix, a single round-to-nearest-even of the exact q * s to f16; bf16 —
// round-to-nearest-even of that f32 value. Shared by the GEMM staging path and
// the dequantisation probe, so the probe reports exactly what the MFMA sees.
template <typename T>
__device__ __forceinline__ uint32_t deq_pack2(float u0, float u1, float s, float nb) {
    return pack2<T>(__builtin_fmaf(u0, s, nb), __builtin_fmaf(u1, s, nb));
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
    return __builtin_bit_cast(float, (uint32_t)b << 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
    return (float)__builtin_bit_cast(_Float16, b);
}

// The timestep-table row of token t (ltx/block.zig:47-67): tidx[t] when it is
// in 0 .. K-1, else 0, so no index reads outside the table.
__device__ __forceinline__ int ada_row(const LtxAda& a, int t) {
    const int r = a.tidx[t];
    return (unsigned)r < (unsigned)a.K ? r : 0;
}

// AdaLN value (ltx/block.zig:47-67): f32 add of the timestep-table row and
// the table row.
__device__ __forceinline__ float ada_val(const LtxAda& a, int t, int i, int c) {
    const int r = ada_row(a, t);
    return a.tstab[((size_t)r * 9 + i) * LTX_D + c] + a.sst[(size_t)i * LTX_D + c];
}

// Sum over a 256-thread block (4 waves). `red` holds 4 floats of LDS.
__device__ __forceinline__ float block_sum256(float v, float* red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float s = red[0] + red[1] + red[2] + red[3];
    __syncthreads();
    return s;
}

// GELU, tanh form: 0.5 x (1 + tanh(u)), u = sqrt(2/pi) (x + 0.044715 x^3),
// evaluated through the exact identity 0.5 (1 + tanh u) = 1 / (1 + exp(-2u)):
// x / (1 + 2^(-2u log2 e)). No subtraction, so no cancellation for negative
// x (the form 1 - 2 / (exp(2u) + 1) lost most digits of 1 + tanh u there),
// and 8 VALU operations against 12 (the ff1 GEMM 1.2 % faster). Large
// negative x gives -0 (exp overflows to inf), large positive x gives x.
__device__ __forceinline__ float gelu_tanh(float x) {
    const float c = 0.7978845608028654f;
    const float a = x * __builtin_fmaf(0.044715f * x, x, 1.0f);  // x + 0.044715 x^3
    const float e = __builtin_amdgcn_exp2f(a * (-2.0f * c * 1.4426950408889634f));
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + __expf(-x)); }
