// ltx_op_linear_q8_noalloc: the isolated int8 GEMM with its scratch in a
// static device array instead of memory the context allocates, for callers
// that may not allocate device memory (code under HIP graph capture, serving
// loops, harnesses that forbid hipMalloc).
//
// `scratch` is one file-scope array per GPU (the code object holding it is
// loaded on each device the library runs on, and stays until the process
// ends). Its host-side name is only a stand-in: the device address comes from
// hipGetSymbolAddress, resolved once per device with that device current
// (ltx_init), and only that address is handed to kernels.
//
// Compiled by hipcc as a host object (with the array's gfx950 code object
// embedded and registered when the library loads); the kernels that use the
// scratch live in the library's own code objects and take its address as an
// argument.
#include <hip/hip_runtime.h>

#include <mutex>

#include "ltx_internal.hpp"

static __device__ __align__(256) unsigned char scratch[LTX_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch[kMaxDevices] = {};
}  // namespace

namespace ltx {

void noalloc_setup(int device) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (device < 0 || device >= kMaxDevices) throw Error("noalloc: device index beyond the supported 64");
    if (g_scratch[device]) return;
    void* p = nullptr;
    HIPC(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) throw Error("noalloc: hipGetSymbolAddress returned no address for the scratch array");
    g_scratch[device] = p;
}

void* noalloc_scratch(int device) {
    std::lock_guard<std::mutex> lk(g_mu);
    return device >= 0 && device < kMaxDevices ? g_scratch[device] : nullptr;
}

}  // namespace ltx

extern "C" int ltx_op_linear_q8_noalloc(ltx_ctx* c, const void* a, const int8_t* q, const void* scales, int scale_f16,
                                        const float* bias, void* y, int out_f32, int M, int N, int K, int gelu,
                                        int mode, void* stream) {
    LTX_GUARD(c, {
        if (!c) throw ltx::Error("NULL context");
        ltx::check_linear_q8(M, N, K, mode);
        ltx::LinearScratch sc{};
        if (ltx::linear_q8_needs_scratch(c, N, K, mode)) {
            // weights as bytes q + 128, then the scale words, then (where
            // ltx_op_linear_q8 runs the four-wave kernel) the weights
            // dequantised to the operand type, each 256-byte aligned
            auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
            const size_t nq = al((size_t)N * K), np = al((size_t)N * (K / LTX_GROUP) * 4);
            const size_t nw = ltx::x4_shape(c, mode, M, N, K, K) ? (size_t)N * K * 2 : 0;
            if (nq + np + nw > LTX_NOALLOC_SCRATCH_BYTES)
                throw ltx::Error(std::string("ltx_op_linear_q8_noalloc: ") +
                                 (nw ? "N * K + 4 N K / 128 + 2 N K bytes (the 16-bit weight copy of the "
                                       "four-wave GEMM, from 4,096 rows)"
                                     : "N * K + 4 N K / 128 bytes") +
                                 " exceed the " + std::to_string(LTX_NOALLOC_SCRATCH_BYTES) + "-byte scratch");
            char* base = (char*)ltx::noalloc_scratch(c->device);
            if (!base) throw ltx::Error("ltx_op_linear_q8_noalloc: scratch not set up on this device");
            sc.q = (uint32_t*)base;
            sc.pairs = (uint32_t*)(base + nq);
            sc.w16 = nw ? base + nq + np : nullptr;
        }
        HIPC(hipSetDevice(c->device));
        ltx::linear_q8(c, a, q, scales, scale_f16, bias, y, out_f32, M, N, K, gelu, mode, sc, (hipStream_t)stream);
    })
}
