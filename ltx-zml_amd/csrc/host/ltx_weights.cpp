// Weight upload: host pointers or a blob image + manifest -> the device form
// the kernels consume (ltx/loader.zig:100-172: normalizeName, findEntry,
// buildBlockBufs, buildQuantBufs).
#include <cmath>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "json.hpp"
#include "ltx_internal.hpp"

namespace ltx {

// File stems of WEIGHT_SPECS (ltx/block.zig:377-406), in LTX_W_* order.
static const char* const kBaseStems[LTX_W_COUNT] = {
    "attn1_to_q_weight", "attn1_to_q_bias", "attn1_to_k_weight", "attn1_to_k_bias",
    "attn1_to_v_weight", "attn1_to_v_bias", "attn1_to_out_0_weight", "attn1_to_out_0_bias",
    "attn1_q_norm_weight", "attn1_k_norm_weight", "attn1_to_gate_logits_weight", "attn1_to_gate_logits_bias",
    "attn2_to_q_weight", "attn2_to_q_bias", "attn2_to_k_weight", "attn2_to_k_bias",
    "attn2_to_v_weight", "attn2_to_v_bias", "attn2_to_out_0_weight", "attn2_to_out_0_bias",
    "attn2_q_norm_weight", "attn2_k_norm_weight", "attn2_to_gate_logits_weight", "attn2_to_gate_logits_bias",
    "ff_net_0_proj_weight", "ff_net_2_weight", "scale_shift_table", "prompt_scale_shift_table"};

static size_t base_numel(int i) {
    switch (i) {
        case LTX_W_G1_W: case LTX_W_G2_W: return (size_t)LTX_H * LTX_D;
        case LTX_W_G1_B: case LTX_W_G2_B: return LTX_H;
        case LTX_W_FF1_W: case LTX_W_FF2_W: return (size_t)LTX_FF * LTX_D;
        case LTX_W_SST: return 9 * (size_t)LTX_D;
        case LTX_W_PSST: return 2 * (size_t)LTX_D;
        case LTX_W_Q1_W: case LTX_W_K1_W: case LTX_W_V1_W: case LTX_W_O1_W:
        case LTX_W_Q2_W: case LTX_W_K2_W: case LTX_W_V2_W: case LTX_W_O2_W: return (size_t)LTX_D * LTX_D;
        default: return LTX_D;  // biases and norm weights
    }
}

// Q8 companions: the base weight each one quantises, and its [O, I].
static const int kQBase[LTX_Q_COUNT] = {LTX_W_Q1_W, LTX_W_K1_W, LTX_W_V1_W, LTX_W_Q2_W, LTX_W_K2_W,
                                        LTX_W_V2_W, LTX_W_FF1_W, LTX_W_FF2_W, LTX_W_O1_W, LTX_W_O2_W};

static void q_dims(int qi, int& O, int& I) {
    O = LTX_D;
    I = LTX_D;
    if (qi == LTX_Q_F1) O = LTX_FF;
    if (qi == LTX_Q_F2) I = LTX_FF;
}

static void h2d(DevBuf& d, const void* src, size_t n) {
    d.alloc(n);
    HIPC(hipMemcpy(d.p, src, n, hipMemcpyHostToDevice));
}

static std::vector<float> bf16v_to_f32(const uint16_t* p, size_t n) {
    std::vector<float> o(n);
    for (size_t i = 0; i < n; i++) o[i] = bf16_bits_to_f32(p[i]);
    return o;
}

static std::vector<uint16_t> bf16v_to_f16(const uint16_t* p, size_t n) {
    std::vector<uint16_t> o(n);
    for (size_t i = 0; i < n; i++) o[i] = f32_to_f16_bits(bf16_bits_to_f32(p[i]));
    return o;
}

// One projection from parts (fused along N when several are given).
static void build_proj(LtxProj& p, const void* const* base, const int8_t* const* q8, const void* const* q8s, int sf16,
                       std::initializer_list<int> qids, int K, bool want_f16_copy) {
    std::vector<int> ids(qids);
    bool all_q8 = q8 != nullptr && q8s != nullptr;
    if (all_q8)
        for (int qi : ids) all_q8 = all_q8 && q8[qi] && q8s[qi];
    p.K = K;
    p.N = 0;
    std::vector<int> Ns;
    for (int qi : ids) {
        int O, I;
        q_dims(qi, O, I);
        Ns.push_back(O);
        p.N += O;
    }
    p.q8 = all_q8;
    p.scale_f16 = sf16;
    const size_t G = K / LTX_GROUP;
    if (all_q8) {
        // weights stored as the bytes q + 128 (XOR 0x80): the LDS-DMA GEMM
        // then needs no per-byte flip (K is a multiple of 128, so of 8)
        std::vector<uint64_t> q((size_t)p.N * K / 8);
        std::vector<char> s((size_t)p.N * G * (sf16 ? 2 : 4));
        size_t r = 0;
        for (size_t j = 0; j < ids.size(); j++) {
            int qi = ids[j];
            const size_t nw = (size_t)Ns[j] * K / 8;
            uint64_t* dst = q.data() + r * K / 8;
            for (size_t i = 0; i < nw; i++) {
                uint64_t v;
                std::memcpy(&v, (const char*)q8[qi] + 8 * i, 8);
                dst[i] = v ^ 0x8080808080808080ull;
            }
            std::memcpy(s.data() + r * G * (sf16 ? 2 : 4), q8s[qi], (size_t)Ns[j] * G * (sf16 ? 2 : 4));
            r += Ns[j];
        }
        h2d(p.q, q.data(), q.size() * 8);
        p.qflip = true;
        h2d(p.s, s.data(), s.size());
        {  // the scales also as words u32 [G][N] for the LDS-DMA kernels: f16 pairs (s | s << 16) or f32 bits
            std::vector<uint32_t> s2((size_t)G * p.N);
            for (size_t n = 0; n < (size_t)p.N; n++)
                for (size_t g = 0; g < G; g++) {
                    uint32_t w = 0;
                    if (sf16) {
                        uint16_t h;
                        std::memcpy(&h, s.data() + 2 * (n * G + g), 2);
                        w = (uint32_t)h * 0x10001u;
                    } else {
                        std::memcpy(&w, s.data() + 4 * (n * G + g), 4);
                    }
                    s2[g * p.N + n] = w;
                }
            h2d(p.s2, s2.data(), s2.size() * 4);
        }
    } else {
        std::vector<uint16_t> w((size_t)p.N * K);
        size_t r = 0;
        for (size_t j = 0; j < ids.size(); j++) {
            std::memcpy(w.data() + r * K, base[kQBase[ids[j]]], (size_t)Ns[j] * K * 2);
            r += Ns[j];
        }
        h2d(p.w_bf16, w.data(), w.size() * 2);
        if (want_f16_copy) {
            auto h = bf16v_to_f16(w.data(), w.size());
            h2d(p.w_f16, h.data(), h.size() * 2);
        }
    }
    // biases: weight slot + 1 in WEIGHT_SPECS order for the attention projections
    std::vector<float> b;
    bool has_bias = false;
    for (int qi : ids) {
        int bw = kQBase[qi];
        bool biased = bw != LTX_W_FF1_W && bw != LTX_W_FF2_W;  // the video FFN is bias-free
        int O, I;
        q_dims(qi, O, I);
        if (biased) {
            has_bias = true;
            auto v = bf16v_to_f32((const uint16_t*)base[bw + 1], O);
            b.insert(b.end(), v.begin(), v.end());
        } else {
            b.insert(b.end(), O, 0.0f);
        }
    }
    if (has_bias) h2d(p.bias, b.data(), b.size() * 4);
}

static void build_gate(LtxProj& p, const void* const* base, int wi) {
    p.N = LTX_H;
    p.K = LTX_D;
    const uint16_t* w = (const uint16_t*)base[wi];
    h2d(p.w_bf16, w, (size_t)LTX_H * LTX_D * 2);
    auto h = bf16v_to_f16(w, (size_t)LTX_H * LTX_D);
    h2d(p.w_f16, h.data(), h.size() * 2);
    auto b = bf16v_to_f32((const uint16_t*)base[wi + 1], LTX_H);
    h2d(p.bias, b.data(), b.size() * 4);
}

static uint64_t proj_bytes(const LtxProj& p) {
    return p.q.bytes + p.s.bytes + p.s2.bytes + p.w_bf16.bytes + p.w_f16.bytes + p.bias.bytes;
}

// f32 scales must be finite and below 2^100 in magnitude: the dequantising
// GEMMs form q * s as fma(q + 128, s, -128 s), and for fp16 operands from
// (q + 128) 2^-24 times s 2^24, which stay finite only below that. A scale
// absmax / 127 of bf16 weights reaches 2^100 only for weights above 1e32.
static void check_f32_scales(const void* s, size_t n, const char* what) {
    const uint32_t* u = (const uint32_t*)s;
    for (size_t i = 0; i < n; i++)
        if ((u[i] & 0x7fffffffu) >= 0x71800000u)  // |s| >= 2^100, inf or NaN
            throw Error(std::string("ScaleRange: f32 scale of ") + what + " is not finite or has magnitude >= 2^100");
}

// The largest magnitude among the 16-bit weight operands of mode F16: 128 max
// |s| for each int8 projection (|q s| <= 128 |s|), max |w| for each bf16
// weight converted to f16 (projections without int8 companions, gate logits).
// Above 65504 those operands would round to inf.
static float f16_operand_max(const void* const* base, const int8_t* const* q8, const void* const* q8s, int sf16,
                             bool unquantised = true) {
    float m = 0.0f;
    auto bf16_max = [&](int wi, size_t n) {
        const uint16_t* w = (const uint16_t*)base[wi];
        uint16_t mx = 0;
        for (size_t i = 0; i < n; i++) mx = std::max<uint16_t>(mx, w[i] & 0x7fffu);
        m = std::max(m, mx >= 0x7f80u ? INFINITY : bf16_bits_to_f32(mx));
    };
    for (int qi = 0; qi < LTX_Q_COUNT; qi++) {
        int O, I;
        q_dims(qi, O, I);
        const size_t G = (size_t)O * (I / LTX_GROUP);
        if (q8 && q8s && q8[qi] && q8s[qi]) {
            float smax = 0.0f;
            for (size_t g = 0; g < G; g++) {
                float v;
                if (sf16) {
                    uint16_t h;
                    std::memcpy(&h, (const char*)q8s[qi] + 2 * g, 2);
                    v = f16_bits_to_f32(h);
                } else {
                    std::memcpy(&v, (const char*)q8s[qi] + 4 * g, 4);
                }
                v = std::fabs(v);
                smax = std::isnan(v) ? INFINITY : std::max(smax, v);
            }
            m = std::max(m, 128.0f * smax);
        } else if (unquantised) {
            bf16_max(kQBase[qi], (size_t)O * I);
        }
    }
    bf16_max(LTX_W_G1_W, (size_t)LTX_H * LTX_D);
    bf16_max(LTX_W_G2_W, (size_t)LTX_H * LTX_D);
    return m;
}

static void check_scales(const void* const* q8s, const int8_t* const* q8, int sf16) {
    if (sf16 || !q8 || !q8s) return;
    for (int qi = 0; qi < LTX_Q_COUNT; qi++) {
        if (!q8[qi] || !q8s[qi]) continue;
        int O, I;
        q_dims(qi, O, I);
        check_f32_scales(q8s[qi], (size_t)O * (I / LTX_GROUP), kBaseStems[kQBase[qi]]);
    }
}

ltx_block_weights* upload(ltx_ctx* c, const void* const* base, const int8_t* const* q8, const void* const* q8s, int sf16) {
    if (!base) throw Error("NULL base weight table");
    for (int i = 0; i < LTX_W_COUNT; i++)
        if (!base[i]) throw Error(std::string("missing base weight ") + kBaseStems[i]);
    check_scales(q8s, q8, sf16);
    const float f16max = f16_operand_max(base, q8, q8s, sf16);
    HIPC(hipSetDevice(c->device));
    auto* w = new ltx_block_weights();
    w->f16_max = f16max;
    try {
        build_proj(w->qkv1, base, q8, q8s, sf16, {LTX_Q_Q1, LTX_Q_K1, LTX_Q_V1}, LTX_D, true);
        build_proj(w->o1, base, q8, q8s, sf16, {LTX_Q_O1}, LTX_D, true);
        build_proj(w->q2, base, q8, q8s, sf16, {LTX_Q_Q2}, LTX_D, true);
        build_proj(w->kv2, base, q8, q8s, sf16, {LTX_Q_K2, LTX_Q_V2}, LTX_D, true);
        build_proj(w->o2, base, q8, q8s, sf16, {LTX_Q_O2}, LTX_D, true);
        build_proj(w->f1, base, q8, q8s, sf16, {LTX_Q_F1}, LTX_D, true);
        build_proj(w->f2, base, q8, q8s, sf16, {LTX_Q_F2}, LTX_FF, true);
        build_gate(w->g1, base, LTX_W_G1_W);
        build_gate(w->g2, base, LTX_W_G2_W);
        auto up_f32 = [&](DevBuf& d, int wi) {
            auto v = bf16v_to_f32((const uint16_t*)base[wi], LTX_D);
            h2d(d, v.data(), v.size() * 4);
        };
        up_f32(w->qn1, LTX_W_QN1);
        up_f32(w->kn1, LTX_W_KN1);
        up_f32(w->qn2, LTX_W_QN2);
        up_f32(w->kn2, LTX_W_KN2);
        h2d(w->sst, base[LTX_W_SST], 9 * (size_t)LTX_D * 4);
        h2d(w->psst, base[LTX_W_PSST], 2 * (size_t)LTX_D * 4);
        w->bytes = proj_bytes(w->qkv1) + proj_bytes(w->o1) + proj_bytes(w->q2) + proj_bytes(w->kv2) +
                   proj_bytes(w->o2) + proj_bytes(w->f1) + proj_bytes(w->f2) + proj_bytes(w->g1) + proj_bytes(w->g2) +
                   w->qn1.bytes * 4 + w->sst.bytes + w->psst.bytes;
    } catch (...) {
        delete w;
        throw;
    }
    return w;
}

// '.' -> '_', "::" -> '_' (ltx/loader.zig:100-119)
std::string normalize_name(const std::string& n) {
    std::string o;
    for (size_t i = 0; i < n.size(); i++) {
        if (n[i] == ':' && i + 1 < n.size() && n[i + 1] == ':') {
            o.push_back('_');
            i++;
        } else if (n[i] == '.') {
            o.push_back('_');
        } else {
            o.push_back(n[i]);
        }
    }
    return o;
}

struct Entry {
    std::string dtype;
    uint64_t offset, nbytes;
};

// packer_version 1 is the reference format (F32 scales; int8 companions for
// q/k/v and ff only); version 2 adds F16 scale entries and int8
// out-projections. A version-1 manifest carrying either is refused.
void check_format_version(const json::Value& m) {
    const json::Value* pv = m.get("packer_version");
    const int64_t v = pv ? pv->as_int() : 1;
    if (v != 1 && v != 2) throw Error("FormatVersion: unsupported packer_version " + std::to_string(v));
    if (v == 2) return;
    for (const auto& e : m.at("entries").arr) {
        const std::string& n = e.at("name").as_str();
        auto ends = [&](const std::string& suf) {
            return n.size() >= suf.size() && n.compare(n.size() - suf.size(), suf.size(), suf) == 0;
        };
        if (ends("::q8scale") && e.at("dtype").as_str() == "F16")
            throw Error("FormatVersion: version-1 manifest with F16 scales (" + n + ")");
        if (ends("attn1.to_out.0.weight::q8") || ends("attn2.to_out.0.weight::q8"))
            throw Error("FormatVersion: version-1 manifest with an int8 out-projection (" + n + ")");
    }
}

// Offsets of one block's entries within its blob image (findEntry,
// ltx/loader.zig:100-129, with the dtype and size checks of buildBlockBufs /
// buildQuantBufs). q8 offsets are -1 where the companion is absent.
struct BlobLayout {
    uint64_t base[LTX_W_COUNT];
    int64_t q8[LTX_Q_COUNT], q8s[LTX_Q_COUNT];
    int sf16;
};

static BlobLayout parse_layout(uint64_t mem_bytes, const char* manifest, int64_t block) {
    if (!manifest) throw Error("NULL manifest");
    json::Value m = json::parse(manifest);
    check_format_version(m);
    // alignment of every entry (checkLayout, ltx/loader.zig:56-74); the upload
    // kernels read entries as 16-byte vectors
    const json::Value* jal = m.get("align");
    const int64_t align = jal ? jal->as_int() : 64;
    if (align <= 0 || align % 16) throw Error("Misaligned: manifest align " + std::to_string(align));
    std::unordered_map<std::string, Entry> ents;
    for (const auto& e : m.at("entries").arr) {
        const std::string& name = e.at("name").as_str();
        const int64_t off = e.at("offset").as_int(), nb = e.at("nbytes").as_int();
        // no sum that can wrap: nbytes fits, then offset fits before it
        if (off < 0 || nb < 0 || (uint64_t)nb > mem_bytes || (uint64_t)off > mem_bytes - (uint64_t)nb)
            throw Error("manifest entry beyond the blob: " + name);
        if (off % align) throw Error("Misaligned: " + name);
        ents[normalize_name(name)] = Entry{e.at("dtype").as_str(), (uint64_t)off, (uint64_t)nb};
    }
    auto find = [&](const std::string& want) -> const Entry* {
        auto it = ents.find(want);
        return it == ents.end() ? nullptr : &it->second;
    };
    BlobLayout L;
    const std::string pre = "transformer_blocks_" + std::to_string(block) + "_";
    for (int i = 0; i < LTX_W_COUNT; i++) {
        const Entry* e = find(pre + kBaseStems[i]);
        if (!e) throw Error("blob " + std::to_string(block) + ": no entry named " + pre + kBaseStems[i]);
        bool f32 = i == LTX_W_SST || i == LTX_W_PSST;
        if (e->dtype != (f32 ? "F32" : "BF16")) throw Error("unexpected dtype " + e->dtype + " for " + kBaseStems[i]);
        if (e->nbytes != base_numel(i) * (f32 ? 4 : 2)) throw Error(std::string("size mismatch for ") + kBaseStems[i]);
        L.base[i] = e->offset;
    }
    int sf16 = -1;
    for (int qi = 0; qi < LTX_Q_COUNT; qi++) {
        L.q8[qi] = L.q8s[qi] = -1;
        std::string stem = pre + kBaseStems[kQBase[qi]];
        const Entry* eq = find(stem + "_q8");
        const Entry* es = find(stem + "_q8scale");
        if (!eq || !es) continue;
        int O, I;
        q_dims(qi, O, I);
        if (eq->dtype != "I8" || eq->nbytes != (uint64_t)O * I) throw Error("bad q8 entry " + stem);
        int f16 = es->dtype == "F16" ? 1 : es->dtype == "F32" ? 0 : -1;
        if (f16 < 0) throw Error("bad q8scale dtype " + es->dtype);
        if (sf16 >= 0 && f16 != sf16) throw Error("mixed q8scale dtypes in one blob");
        sf16 = f16;
        if (es->nbytes != (uint64_t)O * (I / LTX_GROUP) * (f16 ? 2 : 4)) throw Error("bad q8scale size " + stem);
        L.q8[qi] = (int64_t)eq->offset;
        L.q8s[qi] = (int64_t)es->offset;
    }
    L.sf16 = sf16 < 0 ? 0 : sf16;
    return L;
}

ltx_block_weights* upload_blob(ltx_ctx* c, const void* mem, uint64_t mem_bytes, const char* manifest, int64_t block) {
    if (!mem || !manifest) throw Error("NULL blob or manifest");
    const BlobLayout L = parse_layout(mem_bytes, manifest, block);
    const char* bytes = (const char*)mem;
    const void* base[LTX_W_COUNT];
    for (int i = 0; i < LTX_W_COUNT; i++) base[i] = bytes + L.base[i];
    const int8_t* q8[LTX_Q_COUNT] = {};
    const void* q8s[LTX_Q_COUNT] = {};
    for (int qi = 0; qi < LTX_Q_COUNT; qi++)
        if (L.q8[qi] >= 0) {
            q8[qi] = (const int8_t*)(bytes + L.q8[qi]);
            q8s[qi] = bytes + L.q8s[qi];
        }
    return upload(c, base, q8, q8s, L.sf16);
}

// ---- streaming upload: one DMA of the blob image, carved on the device ----
//
// The same device form as upload(), built by kernels from the blob image in
// the context's staging area: int8 parts flipped to q + 128 into the fused
// projection, scales copied and paired, bf16 biases / norm weights widened,
// f16 copies converted. Everything is enqueued on one stream.
struct DevCarve {
    ltx_ctx* c;
    hipStream_t st;
    const char* img;  // device copy of the blob
    bool reuse;
    unsigned long long* over;  // counts f16 copies that are not finite (the weights' f16_over)

    void ensure(DevBuf& d, size_t n) {
        if (reuse) {
            if (d.bytes != n) throw Error("the reused weights handle has a different layout");
        } else {
            d.alloc(n);
        }
    }
    void copy(void* dst, uint64_t off, size_t n) {
        HIPC(hipMemcpyAsync(dst, img + off, n, hipMemcpyDeviceToDevice, st));
    }
    void flip(void* dst, uint64_t off, size_t n) {  // n bytes, a multiple of 4
        LtxFlipArgs a{(const uint32_t*)(img + off), (uint32_t*)dst, n / 4};
        c->launch("ltx_q8_flip", (unsigned)((n / 4 + 255) / 256), 1, 1, 256, &a, st);
    }
    void cvt(const void* src, void* dst, size_t n, int to_f16) {  // bf16 -> f32 (0) or f16 (1)
        LtxCvtArgs a{(const uint16_t*)src, dst, n, to_f16, to_f16 ? over : nullptr};
        c->launch("ltx_cvt_bf16", (unsigned)((n + 255) / 256), 1, 1, 256, &a, st);
    }

    void proj(LtxProj& p, const BlobLayout& L, std::initializer_list<int> qids, int K, bool want_f16_copy) {
        std::vector<int> ids(qids);
        bool all_q8 = true;
        for (int qi : ids) all_q8 = all_q8 && L.q8[qi] >= 0;
        if (reuse && (p.q8 != all_q8 || (all_q8 && p.scale_f16 != L.sf16)))
            throw Error("the reused weights handle has a different layout");
        std::vector<int> Ns;
        p.K = K;
        p.N = 0;
        for (int qi : ids) {
            int O, I;
            q_dims(qi, O, I);
            Ns.push_back(O);
            p.N += O;
        }
        p.q8 = all_q8;
        p.scale_f16 = L.sf16;
        const size_t G = K / LTX_GROUP, ss = L.sf16 ? 2 : 4;
        if (all_q8) {
            ensure(p.q, (size_t)p.N * K);
            ensure(p.s, (size_t)p.N * G * ss);
            size_t r = 0;
            for (size_t j = 0; j < ids.size(); j++) {
                flip((char*)p.q.p + r * K, (uint64_t)L.q8[ids[j]], (size_t)Ns[j] * K);
                copy((char*)p.s.p + r * G * ss, (uint64_t)L.q8s[ids[j]], (size_t)Ns[j] * G * ss);
                r += Ns[j];
            }
            p.qflip = true;
            ensure(p.s2, G * p.N * 4);
            LtxPairArgs pa{p.s.p, (uint32_t*)p.s2.p, p.N, (int)G, L.sf16 ? 0 : 1};
            c->launch("ltx_scale_pairs", (unsigned)((G * p.N + 255) / 256), 1, 1, 256, &pa, st);
        } else {
            ensure(p.w_bf16, (size_t)p.N * K * 2);
            size_t r = 0;
            for (size_t j = 0; j < ids.size(); j++) {
                copy((char*)p.w_bf16.p + r * K * 2, L.base[kQBase[ids[j]]], (size_t)Ns[j] * K * 2);
                r += Ns[j];
            }
            if (want_f16_copy) {
                ensure(p.w_f16, (size_t)p.N * K * 2);
                cvt(p.w_bf16.p, p.w_f16.p, (size_t)p.N * K, 1);
            }
        }
        bool has_bias = false;
        for (int qi : ids) has_bias = has_bias || (kQBase[qi] != LTX_W_FF1_W && kQBase[qi] != LTX_W_FF2_W);
        if (has_bias) {
            ensure(p.bias, (size_t)p.N * 4);
            size_t r = 0;
            for (size_t j = 0; j < ids.size(); j++) {
                const int bw = kQBase[ids[j]];
                if (bw == LTX_W_FF1_W || bw == LTX_W_FF2_W) throw Error("mixed biased and bias-free parts");
                cvt(img + L.base[bw + 1], (float*)p.bias.p + r, (size_t)Ns[j], 0);
                r += Ns[j];
            }
        }
    }
    void gate(LtxProj& p, const BlobLayout& L, int wi) {
        p.N = LTX_H;
        p.K = LTX_D;
        const size_t n = (size_t)LTX_H * LTX_D;
        ensure(p.w_bf16, n * 2);
        copy(p.w_bf16.p, L.base[wi], n * 2);
        ensure(p.w_f16, n * 2);
        cvt(p.w_bf16.p, p.w_f16.p, n, 1);
        ensure(p.bias, LTX_H * 4);
        cvt(img + L.base[wi + 1], p.bias.p, LTX_H, 0);
    }
};

ltx_block_weights* upload_blob_async(ltx_ctx* c, const void* mem, uint64_t mem_bytes, const char* manifest,
                                     int64_t block, ltx_block_weights* reuse, hipStream_t st) {
    if (!mem || !manifest) throw Error("NULL blob or manifest");
    const BlobLayout L = parse_layout(mem_bytes, manifest, block);
    if (!L.sf16)  // the scale entries are read on the host before the copy
        for (int qi = 0; qi < LTX_Q_COUNT; qi++)
            if (L.q8s[qi] >= 0) {
                int O, I;
                q_dims(qi, O, I);
                check_f32_scales((const char*)mem + L.q8s[qi], (size_t)O * (I / LTX_GROUP), kBaseStems[kQBase[qi]]);
            }
    HIPC(hipSetDevice(c->device));
    if (c->blob_stage.bytes < mem_bytes) c->blob_stage.alloc(mem_bytes);
    // the one DMA of the whole image (asynchronous when `mem` is pinned)
    HIPC(hipMemcpyAsync(c->blob_stage.p, mem, mem_bytes, hipMemcpyHostToDevice, st));
    float f16max;
    {  // the range of the int8 products (scales) and gate weights, read from
       // the host image; the unquantised projections' f16 copies are counted
       // on the device as they are made (f16_over), with no host pass over
       // their ~0.5 GB
        const char* bytes = (const char*)mem;
        const void* base[LTX_W_COUNT];
        for (int i = 0; i < LTX_W_COUNT; i++) base[i] = bytes + L.base[i];
        const int8_t* q8[LTX_Q_COUNT] = {};
        const void* q8s[LTX_Q_COUNT] = {};
        for (int qi = 0; qi < LTX_Q_COUNT; qi++)
            if (L.q8[qi] >= 0) {
                q8[qi] = (const int8_t*)(bytes + L.q8[qi]);
                q8s[qi] = bytes + L.q8s[qi];
            }
        f16max = f16_operand_max(base, q8, q8s, L.sf16, false);
    }
    ltx_block_weights* w = reuse ? reuse : new ltx_block_weights();
    w->f16_max = f16max;
    try {
        if (!w->f16_over.p) w->f16_over.alloc(sizeof(unsigned long long));
        HIPC(hipMemsetAsync(w->f16_over.p, 0, sizeof(unsigned long long), st));
        DevCarve d{c, st, (const char*)c->blob_stage.p, reuse != nullptr, (unsigned long long*)w->f16_over.p};
        d.proj(w->qkv1, L, {LTX_Q_Q1, LTX_Q_K1, LTX_Q_V1}, LTX_D, true);
        d.proj(w->o1, L, {LTX_Q_O1}, LTX_D, true);
        d.proj(w->q2, L, {LTX_Q_Q2}, LTX_D, true);
        d.proj(w->kv2, L, {LTX_Q_K2, LTX_Q_V2}, LTX_D, true);
        d.proj(w->o2, L, {LTX_Q_O2}, LTX_D, true);
        d.proj(w->f1, L, {LTX_Q_F1}, LTX_D, true);
        d.proj(w->f2, L, {LTX_Q_F2}, LTX_FF, true);
        d.gate(w->g1, L, LTX_W_G1_W);
        d.gate(w->g2, L, LTX_W_G2_W);
        auto norm = [&](DevBuf& b, int wi) {
            d.ensure(b, (size_t)LTX_D * 4);
            d.cvt(d.img + L.base[wi], b.p, LTX_D, 0);
        };
        norm(w->qn1, LTX_W_QN1);
        norm(w->kn1, LTX_W_KN1);
        norm(w->qn2, LTX_W_QN2);
        norm(w->kn2, LTX_W_KN2);
        d.ensure(w->sst, 9 * (size_t)LTX_D * 4);
        d.copy(w->sst.p, L.base[LTX_W_SST], 9 * (size_t)LTX_D * 4);
        d.ensure(w->psst, 2 * (size_t)LTX_D * 4);
        d.copy(w->psst.p, L.base[LTX_W_PSST], 2 * (size_t)LTX_D * 4);
        w->bytes = proj_bytes(w->qkv1) + proj_bytes(w->o1) + proj_bytes(w->q2) + proj_bytes(w->kv2) +
                   proj_bytes(w->o2) + proj_bytes(w->f1) + proj_bytes(w->f2) + proj_bytes(w->g1) + proj_bytes(w->g2) +
                   w->qn1.bytes * 4 + w->sst.bytes + w->psst.bytes;
    } catch (...) {
        if (!reuse) delete w;
        throw;
    }
    return w;
}

}  // namespace ltx


extern "C" {

int ltx_block_weights_from_host(ltx_ctx* c, const void* const* base, const int8_t* const* q8, const void* const* q8s,
                                int scale_f16, ltx_block_weights** out) {
    LTX_GUARD(c, {
        if (!c || !out) throw ltx::Error("NULL context or out");
        *out = ltx::upload(c, base, q8, q8s, scale_f16);
    })
}

int ltx_block_weights_from_blob(ltx_ctx* c, const void* mem, uint64_t mem_bytes, const char* manifest_json,
                                int64_t block_idx, ltx_block_weights** out) {
    LTX_GUARD(c, {
        if (!c || !out) throw ltx::Error("NULL context or out");
        *out = ltx::upload_blob(c, mem, mem_bytes, manifest_json, block_idx);
    })
}

int ltx_block_weights_from_blob_async(ltx_ctx* c, const void* mem, uint64_t mem_bytes, const char* manifest_json,
                                      int64_t block_idx, ltx_block_weights* reuse, void* stream,
                                      ltx_block_weights** out) {
    LTX_GUARD(c, {
        if (!c || !out) throw ltx::Error("NULL context or out");
        *out = ltx::upload_blob_async(c, mem, mem_bytes, manifest_json, block_idx, reuse, (hipStream_t)stream);
    })
}

void ltx_block_weights_free(ltx_ctx* c, ltx_block_weights* w) {
    if (c) (void)hipSetDevice(c->device);
    delete w;
}

uint64_t ltx_block_weights_bytes(const ltx_block_weights* w) { return w ? w->bytes : 0; }

}  // extern "C"
