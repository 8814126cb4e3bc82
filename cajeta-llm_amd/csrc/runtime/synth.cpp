// synth.cpp — seeded random-init models as GGUF images (the synthetic
// inputs of every benchmark config), with this repository's quantizers.
//
// Values: w = 0.02·z with z an Irwin–Hall(4) normal approximation drawn
// from splitmix64(seed, tensor, element) — integer arithmetic plus one
// rounding, so every run and host produces the same bytes. Norm weights are
// 1 + 0.02·z; the MoE router (f32) is z/sqrt(hidden) so router logits are
// ~N(0, 1). Quantizers (own min/max designs; the bytes are valid GGUF
// blocks that the reference's decoders read):
//   Q8_0  d = amax/127, q = round(x/d)
//   Q4_0  d = m/−8 (m the value of largest |x|), q = min(15, trunc(x/d + 8.5))
//   Q4_K  per 32: scale (max−min)/15 and min offset, both 6-bit against the
//         block's fp16 d/dmin; q = round((x + min)/scale) in 0..15
//   Q6_K  per 16: scale amax/31 as int8 against the block's fp16 d;
//         q = round(x/scale) in −32..31, stored +32
//   MXFP4 per 32: E8M0 e = floor(log2 amax) − 2 + 127, nearest E2M1 code
#include "gguf.h"
#include "rt.h"
#include <cmath>
#include <cstring>
#include <algorithm>
#include <sstream>
#include <thread>
#include <vector>

namespace cj {

namespace {

inline uint64_t splitmix(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}
uint64_t name_hash(const std::string &s) {
    uint64_t h = 1469598103934665603ull;
    for (unsigned char c : s) h = (h ^ c) * 1099511628211ull;
    return h;
}
// Irwin–Hall(4) over 16-bit uniforms, scaled to unit variance.
inline float gauss(uint64_t key, uint64_t i) {
    uint64_t r = splitmix(key ^ (i * 0xD1B54A32D192ED03ull));
    int64_t s = (int64_t)(r & 0xffff) + (int64_t)((r >> 16) & 0xffff) + (int64_t)((r >> 32) & 0xffff) + (int64_t)(r >> 48);
    return (float)(s - 131070) * (1.0f / 37837.23f);
}

inline uint16_t f2h(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return sign | 0x7e00;
    if (ax >= 0x477ff000u) return sign | 0x7c00;
    if (ax < 0x38800000u) {
        uint32_t e = ax >> 23;
        if (e < 102) return sign;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u, sh = 126 - e;
        uint32_t q = m >> sh, rem = m & ((1u << sh) - 1), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return sign | (uint16_t)q;
    }
    uint32_t r = ax + 0xfffu + ((ax >> 13) & 1u);
    return sign | (uint16_t)((r >> 13) - (112u << 10));
}
inline float h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000) << 16, e = (h >> 10) & 31, m = h & 1023, b;
    if (e == 31) b = sign | 0x7f800000u | (m << 13);
    else if (e == 0) { float v = (float)m * (1.0f / 16777216.0f); return sign ? -v : v; }
    else b = sign | ((e + 112) << 23) | (m << 13);
    float f; memcpy(&f, &b, 4); return f;
}

void q8_0_block(const float *x, uint8_t *o) {
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) amax = std::max(amax, std::fabs(x[j]));
    const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    uint16_t h = f2h(d); memcpy(o, &h, 2);
    for (int j = 0; j < 32; j++) o[2 + j] = (uint8_t)(int8_t)std::lround(x[j] * id);
}
void q4_0_block(const float *x, uint8_t *o) {
    float amax = 0.0f, mx = 0.0f;
    for (int j = 0; j < 32; j++) if (std::fabs(x[j]) > amax) { amax = std::fabs(x[j]); mx = x[j]; }
    const float d = mx / -8.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    uint16_t h = f2h(d); memcpy(o, &h, 2);
    for (int j = 0; j < 16; j++) {
        int a = std::min(15, (int)(x[j] * id + 8.5f)), b = std::min(15, (int)(x[j + 16] * id + 8.5f));
        a = std::max(a, 0); b = std::max(b, 0);
        o[2 + j] = (uint8_t)(a | (b << 4));
    }
}
void q4_k_block(const float *x, uint8_t *o) {
    float sc[8], mn[8];
    for (int s = 0; s < 8; s++) {
        float lo = x[32 * s], hi = x[32 * s];
        for (int j = 1; j < 32; j++) { lo = std::min(lo, x[32 * s + j]); hi = std::max(hi, x[32 * s + j]); }
        lo = std::min(lo, 0.0f);
        sc[s] = (hi - lo) / 15.0f;
        mn[s] = -lo;
    }
    float ms = 0.0f, mm = 0.0f;
    for (int s = 0; s < 8; s++) { ms = std::max(ms, sc[s]); mm = std::max(mm, mn[s]); }
    const uint16_t dh = f2h(ms / 63.0f), mh = f2h(mm / 63.0f);
    const float d = h2f(dh), dmin = h2f(mh);
    int isc[8], imn[8];
    for (int s = 0; s < 8; s++) {
        isc[s] = d > 0.0f ? std::min(63, (int)std::lround(sc[s] / d)) : 0;
        imn[s] = dmin > 0.0f ? std::min(63, (int)std::lround(mn[s] / dmin)) : 0;
    }
    memcpy(o, &dh, 2); memcpy(o + 2, &mh, 2);
    uint8_t *s12 = o + 4;
    for (int j = 0; j < 4; j++) {
        s12[j] = (uint8_t)(isc[j] | ((isc[j + 4] >> 4) << 6));
        s12[j + 4] = (uint8_t)(imn[j] | ((imn[j + 4] >> 4) << 6));
        s12[j + 8] = (uint8_t)((isc[j + 4] & 15) | ((imn[j + 4] & 15) << 4));
    }
    uint8_t q[256];
    for (int e = 0; e < 256; e++) {
        const int s = e / 32;
        const float es = d * (float)isc[s], em = dmin * (float)imn[s];
        int v = es > 0.0f ? (int)std::lround((x[e] + em) / es) : 0;
        q[e] = (uint8_t)std::min(15, std::max(0, v));
    }
    for (int g = 0; g < 4; g++)
        for (int l = 0; l < 32; l++) o[16 + 32 * g + l] = (uint8_t)(q[64 * g + l] | (q[64 * g + 32 + l] << 4));
}
void q6_k_block(const float *x, uint8_t *o) {
    float sc[16], ms = 0.0f;
    for (int s = 0; s < 16; s++) {
        float amax = 0.0f;
        for (int j = 0; j < 16; j++) amax = std::max(amax, std::fabs(x[16 * s + j]));
        sc[s] = amax / 31.0f;
        ms = std::max(ms, sc[s]);
    }
    const uint16_t dh = f2h(ms / 127.0f);
    const float d = h2f(dh);
    int isc[16];
    for (int s = 0; s < 16; s++) isc[s] = d > 0.0f ? std::min(127, (int)std::lround(sc[s] / d)) : 0;
    memset(o, 0, 210);
    for (int e = 0; e < 256; e++) {
        const float es = d * (float)isc[e / 16];
        int v = es > 0.0f ? (int)std::lround(x[e] / es) : 0;
        v = std::min(31, std::max(-32, v)) + 32;
        const int g = e / 128, r = e % 128, sl = r / 64, l64 = r % 64, sh = r / 32, l32 = r % 32;
        o[64 * g + l64] |= (uint8_t)((v & 15) << (4 * sl));
        o[128 + 32 * g + l32] |= (uint8_t)(((v >> 4) & 3) << (2 * sh));
    }
    for (int s = 0; s < 16; s++) o[192 + s] = (uint8_t)(int8_t)isc[s];
    memcpy(o + 208, &dh, 2);
}
void mxfp4_block(const float *x, uint8_t *o) {
    static const float kv[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) amax = std::max(amax, std::fabs(x[j]));
    int e = amax > 0.0f ? (int)std::floor(std::log2(amax)) - 2 + 127 : 0;
    e = std::max(0, std::min(254, e));
    uint32_t bits = e < 2 ? (0x00200000u << e) : ((uint32_t)(e - 1) << 23);
    float d; memcpy(&d, &bits, 4);
    o[0] = (uint8_t)e;
    auto best = [&](float v) {
        int bi = 0; float be = std::fabs(v - kv[0] * d);
        for (int k = 1; k < 16; k++) { float er = std::fabs(v - kv[k] * d); if (er < be) { be = er; bi = k; } }
        return bi;
    };
    for (int j = 0; j < 16; j++) o[1 + j] = (uint8_t)(best(x[j]) | (best(x[j + 16]) << 4));
}

struct Spec {
    int layers = 4, hidden = 512, heads = 8, kv = 2, hd = 64, ffn = 1408, vocab = 32000, ctx = 4096;
    float eps = 1e-5f, theta = 10000.0f;
    int wtype = CJ_Q8_0, head = CJ_Q8_0, embd = CJ_F32;
    int experts = 0, used = 0, expert_ffn = 0, expert_type = CJ_MXFP4, norm_topk = 1, swa = 0, eos = -1;
    int rope_freqs = 0;   // 1: a rope_freqs.weight tensor of hd/2 factors (Llama-3.1's scaled RoPE)
};

int type_of(const std::string &s) {
    if (s == "f32") return CJ_F32;
    if (s == "f16") return CJ_F16;
    if (s == "q8_0") return CJ_Q8_0;
    if (s == "q4_0") return CJ_Q4_0;
    if (s == "q4_k") return CJ_Q4_K;
    if (s == "q6_k") return CJ_Q6_K;
    if (s == "mxfp4") return CJ_MXFP4;
    return -1;
}

bool parse_spec(const std::string &in, Spec &sp, std::string &err) {
    std::string s = in;
    if (s == "c1") s = "layers=4;hidden=512;heads=8;kv=2;hd=64;ffn=1408;vocab=32000;eps=1e-5;theta=10000;wtype=q8_0;head=q8_0;embd=f32";
    else if (s == "c3") s = "layers=32;hidden=4096;heads=32;kv=8;hd=128;ffn=14336;vocab=128256;eps=1e-5;theta=500000;wtype=q4_k;head=q6_k;embd=q4_k;ctx=8192";
    else if (s == "c4") s = "layers=32;hidden=4096;heads=32;kv=8;hd=128;ffn=14336;vocab=128256;eps=1e-5;theta=500000;wtype=q8_0;head=q8_0;embd=q8_0;ctx=8192";
    else if (s == "c5") s = "layers=24;hidden=2880;heads=64;kv=8;hd=64;ffn=2880;vocab=201088;eps=1e-5;theta=150000;wtype=q8_0;head=q8_0;embd=q8_0;experts=32;used=4;expert_ffn=2880;expert_type=mxfp4;swa=128;ctx=8192";
    std::stringstream ss(s);
    std::string kvp;
    while (std::getline(ss, kvp, ';')) {
        if (kvp.empty()) continue;
        size_t eq = kvp.find('=');
        if (eq == std::string::npos) { err = "spec item without '=': " + kvp; return false; }
        std::string k = kvp.substr(0, eq), v = kvp.substr(eq + 1);
        auto I = [&]() { return std::stoi(v); };
        if (k == "layers") sp.layers = I();
        else if (k == "hidden") sp.hidden = I();
        else if (k == "heads") sp.heads = I();
        else if (k == "kv") sp.kv = I();
        else if (k == "hd") sp.hd = I();
        else if (k == "ffn") sp.ffn = I();
        else if (k == "vocab") sp.vocab = I();
        else if (k == "ctx") sp.ctx = I();
        else if (k == "eps") sp.eps = std::stof(v);
        else if (k == "theta") sp.theta = std::stof(v);
        else if (k == "wtype") sp.wtype = type_of(v);
        else if (k == "head") sp.head = type_of(v);
        else if (k == "embd") sp.embd = type_of(v);
        else if (k == "experts") sp.experts = I();
        else if (k == "used") sp.used = I();
        else if (k == "expert_ffn") sp.expert_ffn = I();
        else if (k == "expert_type") sp.expert_type = type_of(v);
        else if (k == "norm_topk") sp.norm_topk = I();
        else if (k == "swa") sp.swa = I();
        else if (k == "eos") sp.eos = I();
        else if (k == "rope_freqs") sp.rope_freqs = I();
        else { err = "unknown spec key " + k; return false; }
    }
    if (sp.wtype < 0 || sp.head < 0 || sp.embd < 0 || sp.expert_type < 0) { err = "unknown weight type in spec"; return false; }
    return true;
}

struct Job { std::string name; int type; int64_t rows, cols; int kind; };  // kind 0 weight, 1 norm, 2 router, 3 rope factors

void fill_tensor(uint8_t *dst, const Job &j, uint64_t seed, int hidden, int nthreads) {
    const uint64_t key = splitmix(seed ^ name_hash(j.name));
    const int be = ggml_block_elems(j.type), bb = ggml_block_bytes(j.type);
    const int64_t rb = ggml_row_bytes(j.type, j.cols);
    auto work = [&](int64_t r0, int64_t r1) {
        std::vector<float> row((size_t)j.cols);
        for (int64_t r = r0; r < r1; r++) {
            for (int64_t c = 0; c < j.cols; c++) {
                const float z = gauss(key, (uint64_t)(r * j.cols + c));
                // rope factors: 1 on the fast dimensions rising to 8 on the
                // slow ones, with a seeded wobble (the shape of Llama-3.1's)
                const float fr = 1.0f + 7.0f * (float)c / (float)std::max<int64_t>(1, j.cols - 1);
                row[(size_t)c] = j.kind == 1   ? 1.0f + 0.02f * z
                                 : j.kind == 2 ? z / std::sqrt((float)hidden)
                                 : j.kind == 3 ? fr * (1.0f + 0.05f * z)
                                               : 0.02f * z;
            }
            uint8_t *o = dst + r * rb;
            if (j.type == CJ_F32) { memcpy(o, row.data(), (size_t)j.cols * 4); continue; }
            if (j.type == CJ_F16) { for (int64_t c = 0; c < j.cols; c++) { uint16_t h = f2h(row[(size_t)c]); memcpy(o + 2 * c, &h, 2); } continue; }
            for (int64_t b = 0; b < j.cols / be; b++) {
                const float *x = row.data() + b * be;
                uint8_t *ob = o + b * bb;
                switch (j.type) {
                case CJ_Q8_0: q8_0_block(x, ob); break;
                case CJ_Q4_0: q4_0_block(x, ob); break;
                case CJ_Q4_K: q4_k_block(x, ob); break;
                case CJ_Q6_K: q6_k_block(x, ob); break;
                case CJ_MXFP4: mxfp4_block(x, ob); break;
                }
            }
        }
    };
    const int64_t nt = std::max<int64_t>(1, std::min<int64_t>(nthreads, j.rows / 16));
    std::vector<std::thread> th;
    for (int64_t t = 0; t < nt; t++) th.emplace_back(work, j.rows * t / nt, j.rows * (t + 1) / nt);
    for (auto &t : th) t.join();
}

}  // namespace

int synth_gguf(const std::string &spec, const std::string &path, int64_t seed) {
    Spec sp;
    std::string err;
    if (!parse_spec(spec, sp, err)) return fail(CJ_ERR_ARG, "cj_synth_gguf: %s", err.c_str());
    GgufWriter w;
    w.kv_str("general.architecture", "llama");
    w.kv_str("general.name", "cajeta-mi355x synthetic " + spec.substr(0, 32));
    w.kv_u32("general.alignment", 32);
    w.kv_u32("llama.context_length", (uint32_t)sp.ctx);
    w.kv_u32("llama.embedding_length", (uint32_t)sp.hidden);
    w.kv_u32("llama.block_count", (uint32_t)sp.layers);
    w.kv_u32("llama.feed_forward_length", (uint32_t)sp.ffn);
    w.kv_u32("llama.attention.head_count", (uint32_t)sp.heads);
    w.kv_u32("llama.attention.head_count_kv", (uint32_t)sp.kv);
    w.kv_u32("llama.attention.key_length", (uint32_t)sp.hd);
    w.kv_u32("llama.attention.value_length", (uint32_t)sp.hd);
    w.kv_u32("llama.rope.dimension_count", (uint32_t)sp.hd);
    w.kv_f32("llama.rope.freq_base", sp.theta);
    w.kv_f32("llama.attention.layer_norm_rms_epsilon", sp.eps);
    w.kv_u32("llama.vocab_size", (uint32_t)sp.vocab);
    if (sp.experts > 0) {
        w.kv_u32("llama.expert_count", (uint32_t)sp.experts);
        w.kv_u32("llama.expert_used_count", (uint32_t)sp.used);
        w.kv_u32("llama.expert_feed_forward_length", (uint32_t)sp.expert_ffn);
        w.kv_u32("llama.expert_weights_norm", (uint32_t)sp.norm_topk);
        w.kv_u32("llama.expert_gating_func", 1);
    }
    if (sp.swa > 0) {
        w.kv_u32("llama.attention.sliding_window", (uint32_t)sp.swa);
        w.kv_u32("llama.attention.sliding_window_pattern", 2);
    }
    if (sp.eos >= 0) w.kv_u32("tokenizer.ggml.eos_token_id", (uint32_t)sp.eos);

    std::vector<Job> jobs;
    const int64_t h = sp.hidden, qd = (int64_t)sp.heads * sp.hd, kvd = (int64_t)sp.kv * sp.hd;
    jobs.push_back({"token_embd.weight", sp.embd, sp.vocab, h, 0});
    for (int l = 0; l < sp.layers; l++) {
        const std::string p = "blk." + std::to_string(l) + ".";
        jobs.push_back({p + "attn_norm.weight", CJ_F32, 1, h, 1});
        jobs.push_back({p + "attn_q.weight", sp.wtype, qd, h, 0});
        jobs.push_back({p + "attn_k.weight", sp.wtype, kvd, h, 0});
        jobs.push_back({p + "attn_v.weight", sp.wtype, kvd, h, 0});
        jobs.push_back({p + "attn_output.weight", sp.wtype, h, qd, 0});
        jobs.push_back({p + "ffn_norm.weight", CJ_F32, 1, h, 1});
        if (sp.experts > 0) {
            jobs.push_back({p + "ffn_gate_inp.weight", CJ_F32, sp.experts, h, 2});
            jobs.push_back({p + "ffn_gate_exps.weight", sp.expert_type, (int64_t)sp.experts * sp.expert_ffn, h, 0});
            jobs.push_back({p + "ffn_up_exps.weight", sp.expert_type, (int64_t)sp.experts * sp.expert_ffn, h, 0});
            jobs.push_back({p + "ffn_down_exps.weight", sp.expert_type, (int64_t)sp.experts * h, sp.expert_ffn, 0});
        } else {
            jobs.push_back({p + "ffn_gate.weight", sp.wtype, sp.ffn, h, 0});
            jobs.push_back({p + "ffn_up.weight", sp.wtype, sp.ffn, h, 0});
            jobs.push_back({p + "ffn_down.weight", sp.wtype, h, sp.ffn, 0});
        }
    }
    jobs.push_back({"output_norm.weight", CJ_F32, 1, h, 1});
    jobs.push_back({"output.weight", sp.head, sp.vocab, h, 0});
    if (sp.rope_freqs) jobs.push_back({"rope_freqs.weight", CJ_F32, 1, sp.hd / 2, 3});
    for (auto &j : jobs) {
        if (ggml_row_bytes(j.type, j.cols) < 0)
            return fail(CJ_ERR_ARG, "cj_synth_gguf: %s has %lld columns, not whole blocks of its type", j.name.c_str(), (long long)j.cols);
        if (sp.experts > 0 && (j.name.find("_exps") != std::string::npos)) {
            const int64_t per = j.name.find("down") != std::string::npos ? h : sp.expert_ffn;
            w.tensor(j.name, j.type, {j.cols, per, (int64_t)sp.experts});
        } else if (j.rows == 1) {
            w.tensor(j.name, j.type, {j.cols});
        } else {
            w.tensor(j.name, j.type, {j.cols, j.rows});
        }
    }
    std::vector<size_t> offs;
    const size_t total = w.layout(offs);
    const bool mem = path.rfind("mem:", 0) == 0;
    uint8_t *img = nullptr;
    std::unique_ptr<uint8_t[]> tmp;
    if (mem) {
        img = image_create(path.substr(4), total);
    } else {
        tmp.reset(new (std::nothrow) uint8_t[total]);
        img = tmp.get();
    }
    if (!img) return fail(CJ_ERR_IO, "cj_synth_gguf: cannot allocate %zu bytes", total);
    memset(img, 0, offs.empty() ? total : offs[0]);
    w.write_header(img);
    const int nthreads = (int)std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    for (size_t i = 0; i < jobs.size(); i++) fill_tensor(img + offs[i], jobs[i], (uint64_t)seed, sp.hidden, nthreads);
    if (!mem) {
        FILE *f = fopen(path.c_str(), "wb");
        if (!f) return fail(CJ_ERR_IO, "cj_synth_gguf: cannot write %s", path.c_str());
        size_t wr = fwrite(img, 1, total, f);
        fclose(f);
        if (wr != total) return fail(CJ_ERR_IO, "cj_synth_gguf: short write to %s", path.c_str());
    }
    return CJ_OK;
}

}  // namespace cj

extern "C" {
int32_t cj_synth_gguf(const int8_t *spec, const int8_t *path, int64_t seed) {
    if (!spec || !path) return cj::fail(CJ_ERR_ARG, "cj_synth_gguf: null argument");
    return cj::synth_gguf((const char *)spec, (const char *)path, seed);
}
int32_t cj_image_info(const int8_t *name, int64_t *addr, int64_t *size) {
    const uint8_t *p; size_t n;
    if (!name || !cj::image_get((const char *)name, &p, &n)) return cj::fail(CJ_ERR_ARG, "cj_image_info: no image");
    *addr = (int64_t)(uintptr_t)p;
    *size = (int64_t)n;
    return CJ_OK;
}
int32_t cj_image_free(const int8_t *name) {
    return name && cj::image_free((const char *)name) ? CJ_OK : cj::fail(CJ_ERR_ARG, "cj_image_free: no image");
}
int32_t cj_gguf_info(const int8_t *path, int64_t *n_tensors, int64_t *n_shards) {
    if (!path || !n_tensors || !n_shards) return cj::fail(CJ_ERR_ARG, "cj_gguf_info: null argument");
    try {
        cj::Gguf f;
        std::string err;
        if (!f.open((const char *)path, err)) return cj::fail(CJ_ERR_IO, "%s", err.c_str());
        *n_tensors = (int64_t)f.tensors().size();
        *n_shards = f.shards();
        return CJ_OK;
    } catch (const std::exception &x) {   // nothing may unwind through the C-ABI
        return cj::fail(CJ_ERR_IO, "gguf: %s", x.what());
    }
}
}
