// Context, code-object loading, kernel launch, errors and event profiling.
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cmath>
#include <cstring>

#include "ltx_internal.hpp"

// gfx950 code objects, embedded at build time (ltx_codeobjects.S).
extern "C" {
extern const unsigned char ltx_co_k_gemm[], ltx_co_k_gemm_s4[], ltx_co_k_attn[], ltx_co_k_norm[], ltx_co_k_f32[],
    ltx_co_k_core[];
}

namespace ltx {

static thread_local std::string g_thread_err;
static std::atomic<long> g_hip_calls{0};
static long g_fail_after = [] {
    const char* e = std::getenv("LTX_FAIL_AFTER");
    return e ? std::atol(e) : 0L;
}();

void set_thread_error(const std::string& e) { g_thread_err = e; }

bool fail_in_capture() {  // read at every call (once per forward), so a process can switch it
    const char* e = std::getenv("LTX_FAIL_CAPTURE");
    return e && std::atoi(e) != 0;
}

void hip_check(hipError_t e, const char* what) {
    long n = ++g_hip_calls;
    if (g_fail_after > 0 && n >= g_fail_after && e == hipSuccess) e = hipErrorUnknown;  // injected
    if (e != hipSuccess) {
        char buf[512];
        std::snprintf(buf, sizeof(buf), "%s failed: %s (%d)%s", what, hipGetErrorString(e), (int)e,
                      (g_fail_after > 0 && n >= g_fail_after) ? " [LTX_FAIL_AFTER]" : "");
        throw Error(buf);
    }
}

void DevBuf::alloc(size_t n) {
    free_();
    if (n == 0) return;
    HIPC(hipMalloc(&p, n));
    bytes = n;
}

void DevBuf::free_() {
    if (p) (void)hipFree(p);
    p = nullptr;
    bytes = 0;
}

uint16_t f32_to_f16_bits(float f) {  // round to nearest even, IEEE binary16
    uint32_t x;
    std::memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // rounds to >= 65520 -> inf
    if (ax < 0x38800000u) {                                    // subnormal or zero in f16
        if (ax < 0x33000000u) return (uint16_t)sign;           // < 2^-25 -> 0
        uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u;
        int shift = 126 - (int)e;  // f16 subnormal ulp 2^-24
        uint32_t q = m >> shift, rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((ax - 0x38000000u) >> 13);  // rebias 127 -> 15
    uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) q++;
    return (uint16_t)(sign | q);
}

float bf16_bits_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// f16 bits -> f32 (exact): subnormals as m 2^-24, inf and NaN kept.
float f16_bits_to_f32(uint16_t h) {
    const uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
    const float sign = (h & 0x8000u) ? -1.0f : 1.0f;
    if (e == 0) return sign * std::ldexp((float)m, -24);
    if (e == 31) return m ? NAN : sign * INFINITY;
    return sign * std::ldexp((float)(m | 0x400u), (int)e - 25);
}

}  // namespace ltx

hipFunction_t ltx_ctx::fn(const char* name) {
    auto it = fns.find(name);
    if (it != fns.end()) return it->second;
    for (hipModule_t m : modules) {
        hipFunction_t f;
        if (hipModuleGetFunction(&f, m, name) == hipSuccess) {
            fns[name] = f;
            return f;
        }
        (void)hipGetLastError();  // a miss in this module is not an error: clear it for later callers
    }
    throw ltx::Error(std::string("kernel not found in code objects: ") + name);
}

void ltx_ctx::launch(const char* name, unsigned gx, unsigned gy, unsigned gz, unsigned bx, void* args, hipStream_t st,
                     const char* label) {
    hipFunction_t f = fn(name);
    void* params[] = {args};
    hipEvent_t ea = nullptr, eb = nullptr;
    if (prof) {
        if (ev_pool.size() < 2) {
            for (int i = 0; i < 64; i++) {
                hipEvent_t e;
                HIPC(hipEventCreate(&e));
                ev_pool.push_back(e);
            }
        }
        ea = ev_pool.back();
        ev_pool.pop_back();
        eb = ev_pool.back();
        ev_pool.pop_back();
        HIPC(hipEventRecord(ea, st));
    }
    HIPC(hipModuleLaunchKernel(f, gx, gy, gz, bx, 1, 1, 0, st, params, nullptr));
    if (prof) {
        HIPC(hipEventRecord(eb, st));
        prof_recs.push_back({label ? label : fns.find(name)->first.c_str(), ea, eb});
    } else if (marks_on) {
        // A marker after each kernel inside a MarkScope: the stretch of the
        // block forward from the q2 GEMM to the cross-attention. Without them
        // (kernel traces of the 28,672-token block) the cross-attention gate
        // logits on the second stream and the context k|v GEMM's split-K
        // reduce beside them took 0.568 and 0.394 ms instead of 0.089 and
        // 0.014 ms; every other kernel ran within 1 %. The block took
        // 1-2.3 % less time with markers on six of seven boxes, whether they
        // carried a timing stamp, a system-scope fence or neither; markers on
        // the second stream alone, or one marker just before or after the
        // reduce, did not help, and markers on every launch of the forward
        // helped no more than on this stretch. At 1,024 tokens (kernels of
        // 4-130 us) markers on every launch cost 2 %, hence the size switch.
        HIPC(hipEventRecord(marks[mark_i++ & 15], st));
    }
}


extern "C" {

const char* ltx_version(void) { return "ltx-mi355x 0.1 gfx950"; }

const char* ltx_last_error(const ltx_ctx* ctx) {
    if (ctx) return ctx->err.c_str();
    return ltx::g_thread_err.c_str();
}

int ltx_init(int device, ltx_ctx** out) {
    ltx_ctx* c = nullptr;
    try {
        if (!out) throw ltx::Error("ltx_init: out is NULL");
        *out = nullptr;
        int n = 0;
        HIPC(hipGetDeviceCount(&n));
        if (device < 0 || device >= n) throw ltx::Error("ltx_init: device index out of range");
        HIPC(hipSetDevice(device));
        hipDeviceProp_t prop;
        HIPC(hipGetDeviceProperties(&prop, device));
        if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
            throw ltx::Error(std::string("ltx_init: code objects are gfx950-only, device is ") + prop.gcnArchName);
        // the static scratch of ltx_op_linear_q8_noalloc, resolved on this device
        ltx::noalloc_setup(device);
        c = new ltx_ctx();
        c->device = device;
        // the range guard's counter, zero at creation
        c->range_ctr.alloc(256);
        HIPC(hipMemset(c->range_ctr.p, 0, 256));
        c->num_cu = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
        // LTX_GEMM_GRID=tile: one workgroup per output tile instead of the
        // persistent grid of one per CU; LTX_GEMM_Q8=reg: the register-staged
        // int8 GEMM everywhere; LTX_GEMM_X4=off / all: the four-wave 16-bit
        // GEMM nowhere / wherever the shape allows; LTX_GEMM_S4=off / all: the
        // small-grid GEMM likewise; LTX_ATTN_VARIANT=w8: the any-length attention
        // everywhere, =pp: the streaming ping-pong attention also for 64-256
        // keys; LTX_SIDE_EARLY=off / all: the small-T side-stream schedule
        // of the block forward nowhere / at every size (the kernels and
        // schedules each test exercises beside the defaults)
        if (const char* e = std::getenv("LTX_GEMM_GRID")) c->gemm_persistent = std::strcmp(e, "tile") != 0;
        if (const char* e = std::getenv("LTX_GEMM_Q8")) c->gemm_dma = std::strcmp(e, "reg") != 0;
        if (const char* e = std::getenv("LTX_GEMM_X4"))
            c->gemm_x4 = std::strcmp(e, "off") == 0 ? 0 : std::strcmp(e, "all") == 0 ? 2 : 1;
        if (const char* e = std::getenv("LTX_GEMM_S4"))
            c->gemm_s4 = std::strcmp(e, "off") == 0 ? 0 : std::strcmp(e, "all") == 0 ? 2 : 1;
        if (const char* e = std::getenv("LTX_SIDE_EARLY"))
            c->side_early = std::strcmp(e, "off") == 0 ? 0 : std::strcmp(e, "all") == 0 ? 2 : 1;
        if (const char* e = std::getenv("LTX_ATTN_VARIANT")) {
            c->attn_pp = std::strcmp(e, "w8") != 0;
            c->attn_kv = c->attn_pp && std::strcmp(e, "pp") != 0;
        }
        HIPC(hipStreamCreateWithFlags(&c->side, hipStreamNonBlocking));  // default priority
        for (auto& e : c->side_ev) HIPC(hipEventCreateWithFlags(&e, hipEventDisableTiming));
        for (auto& e : c->marks) HIPC(hipEventCreateWithFlags(&e, hipEventDisableTiming | hipEventDisableSystemFence));
        for (const unsigned char* co :
             {ltx_co_k_gemm, ltx_co_k_gemm_s4, ltx_co_k_attn, ltx_co_k_norm, ltx_co_k_f32, ltx_co_k_core}) {
            hipModule_t m;
            HIPC(hipModuleLoadData(&m, co));
            c->modules.push_back(m);
        }
        *out = c;
        return LTX_OK;
    } catch (const std::exception& ex) {
        ltx::set_thread_error(ex.what());
        if (c) ltx_destroy(c);
        return LTX_FAIL;
    }
}

void ltx_destroy(ltx_ctx* c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    (void)hipDeviceSynchronize();
    for (auto& r : c->prof_recs) {
        (void)hipEventDestroy(r.a);
        (void)hipEventDestroy(r.b);
    }
    for (auto e : c->ev_pool) (void)hipEventDestroy(e);
    for (auto e : c->side_ev)
        if (e) (void)hipEventDestroy(e);
    for (auto e : c->marks)
        if (e) (void)hipEventDestroy(e);
    if (c->side) (void)hipStreamDestroy(c->side);
    c->ws.free_();
    c->op_pairs.free_();
    c->op_q.free_();
    c->blob_stage.free_();
    c->core_ws.free_();
    c->tail_ws.free_();
    c->dn_ws.free_();
    for (hipModule_t m : c->modules) (void)hipModuleUnload(m);
    delete c;
}

int ltx_profile_enable(ltx_ctx* c, int enable) {
    LTX_GUARD(c, {
        if (!c) throw ltx::Error("NULL context");
        c->prof = enable != 0;
    })
}

int ltx_profile_reset(ltx_ctx* c) {
    LTX_GUARD(c, {
        if (!c) throw ltx::Error("NULL context");
        HIPC(hipDeviceSynchronize());
        for (auto& r : c->prof_recs) {
            c->ev_pool.push_back(r.a);
            c->ev_pool.push_back(r.b);
        }
        c->prof_recs.clear();
    })
}

int ltx_profile_read(ltx_ctx* c, const char* substr, double* total_ms, int* count) {
    LTX_GUARD(c, {
        if (!c) throw ltx::Error("NULL context");
        HIPC(hipDeviceSynchronize());
        double tot = 0;
        int n = 0;
        for (auto& r : c->prof_recs) {
            if (substr && *substr && !std::strstr(r.name, substr)) continue;
            float ms = 0;
            HIPC(hipEventElapsedTime(&ms, r.a, r.b));
            tot += ms;
            n++;
        }
        if (total_ms) *total_ms = tot;
        if (count) *count = n;
    })
}

int ltx_range_count(ltx_ctx* c, void* stream, uint64_t* count, int reset) {
    LTX_GUARD(c, {
        if (!c || !count) throw ltx::Error("NULL argument");
        HIPC(hipSetDevice(c->device));
        HIPC(hipStreamSynchronize((hipStream_t)stream));
        unsigned long long v = 0;
        HIPC(hipMemcpy(&v, c->range_ctr.p, sizeof(v), hipMemcpyDeviceToHost));
        *count = v;
        if (reset) {
            v = 0;
            HIPC(hipMemcpy(c->range_ctr.p, &v, sizeof(v), hipMemcpyHostToDevice));
        }
    })
}

int ltx_block_stage(ltx_ctx* c, int stage, void** dev_ptr, uint64_t* bytes) {
    LTX_GUARD(c, {
        if (!c) throw ltx::Error("NULL context");
        if (stage < 0 || stage >= LTX_ST_COUNT) throw ltx::Error("stage id out of range");
        if (!c->stage_ptr[stage]) throw ltx::Error("stage not available (no forward yet, or not in this mode)");
        if (dev_ptr) *dev_ptr = c->stage_ptr[stage];
        if (bytes) *bytes = c->stage_bytes[stage];
    })
}

}  // extern "C"
