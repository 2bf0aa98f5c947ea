// synth.cpp — synthetic GGUF images.
//
// mode 0 restates SyntheticSpec::build (testing.rs:229-383) byte for byte: one
// xorshift Rng stream (testing.rs:10-30) fills the block bytes of every matrix
// and draws its fp16 scales (random_weight, testing.rs:46-91); norms are
// 1 + 0.1·U(-1,1); the metadata, vocabulary and tensor order are the same, and
// the image layout is GgufWriter::to_bytes (gguf.rs:407-436, 32-byte alignment).
//
// mode 1 is the benchmark workload definition: weights drawn N(0, 0.02) (normal
// quantiles looked up with 16-bit uniforms, see Normal below) and quantized
// with the reference's own quantize::q4_0 / quantize::q8_0 (quant/mod.rs:
// 262-298) or, for Q4_K and Q6_K (which the reference cannot produce,
// quant/mod.rs:259-261), with the min/max quantizers below; unit norms, a
// chosen RoPE base, a chosen output-head type, and optionally the Q4_K_M
// per-tensor mix.  Each tensor is cut into 64-row chunks with independent Rng
// streams seeded by splitmix64(seed, tensor index, chunk index), so the image
// is generated in parallel and is the same for any thread count.
#include "synth.hpp"

#include "../common.hpp"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <algorithm>
#include <atomic>
#include <thread>

namespace rie {

namespace {

struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s((seed * 0x9E3779B97F4A7C15ULL) | 1ULL) {}
    uint64_t next() {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        return s;
    }
    float f32() { return (float)(next() >> 40) / (float)(1ULL << 24); }
    float sym() { return f32() * 2.0f - 1.0f; }
};

uint16_t f2h(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, exp = (x >> 23) & 0xffu, man = x & 0x7fffffu;
    if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x0200u | (man >> 13) : 0u));
    int e = (int)exp - 112;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m = man | 0x800000u;
        int shift = 14 - e;
        uint32_t half = 1u << (shift - 1), rem = m & ((1u << shift) - 1u), r = m >> shift;
        if (rem > half || (rem == half && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((uint32_t)e << 10) | (man >> 13), rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t)(sign | r);
}

uint16_t f2bf(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    if ((x & 0x8000u) && (x & 0x17fffu)) return (uint16_t)((x >> 16) + 1);
    return (uint16_t)(x >> 16);
}

void put16(uint8_t *p, uint16_t v) {
    p[0] = (uint8_t)v;
    p[1] = (uint8_t)(v >> 8);
}

// testing.rs:46-91
void random_weight(Rng &r, int ty, size_t rows, size_t cols, uint8_t *out) {
    const size_t n = rows * cols;
    if (ty == T_F32 || ty == T_F16 || ty == T_BF16) {
        const float sc = 0.1f;
        for (size_t i = 0; i < n; i++) {
            float v = r.sym() * sc;
            if (ty == T_F32) std::memcpy(out + 4 * i, &v, 4);
            else put16(out + 2 * i, ty == T_F16 ? f2h(v) : f2bf(v));
        }
        return;
    }
    const size_t nblocks = n / block_size(ty), bb = block_bytes(ty), total = nblocks * bb;
    size_t i = 0;
    for (; i + 8 <= total; i += 8) {
        uint64_t v = r.next();
        std::memcpy(out + i, &v, 8);
    }
    if (i < total) {
        uint64_t v = r.next();
        std::memcpy(out + i, &v, total - i);
    }
    float k = 0.01f;
    switch (ty) {
    case T_Q5_0: case T_Q5_1: k = 0.005f; break;
    case T_Q8_0: k = 0.001f; break;
    case T_Q2_K: k = 0.004f; break;
    case T_Q3_K: k = 0.003f; break;
    case T_Q4_K: k = 0.001f; break;
    case T_Q5_K: k = 0.0007f; break;
    case T_Q6_K: k = 0.0001f; break;
    default: break;
    }
    const float scale = 1.0f * k;
    size_t offs[2];
    size_t nofs = 0;
    switch (ty) {
    case T_Q4_0: case T_Q5_0: case T_Q8_0: offs[0] = 0; nofs = 1; break;
    case T_Q4_1: case T_Q5_1: case T_Q4_K: case T_Q5_K: offs[0] = 0; offs[1] = 2; nofs = 2; break;
    case T_Q2_K: offs[0] = 80; offs[1] = 82; nofs = 2; break;
    case T_Q3_K: offs[0] = 108; nofs = 1; break;
    case T_Q6_K: offs[0] = 208; nofs = 1; break;
    default: break;
    }
    const bool signed_first = ty == T_Q4_0 || ty == T_Q5_0 || ty == T_Q8_0 || ty == T_Q3_K || ty == T_Q6_K;
    const bool min_second = ty == T_Q4_1 || ty == T_Q5_1;
    for (size_t b = 0; b < nblocks; b++)
        for (size_t si = 0; si < nofs; si++) {
            float v = (r.f32() * 0.5f + 0.5f) * scale;
            if (si == 0 && signed_first && r.f32() < 0.3f) v = -v;
            if (si == 1 && min_second) v = -v * 8.0f;
            put16(out + b * bb + offs[si], f2h(v));
        }
}

// quantize::q4_0 (quant/mod.rs:279-298)
void quantize_q4_0(const float *x, size_t n, uint8_t *out) {
    for (size_t b = 0; b < n / 32; b++) {
        const float *xb = x + b * 32;
        float max = 0.0f;
        for (int i = 0; i < 32; i++)
            if (std::fabs(xb[i]) > std::fabs(max)) max = xb[i];
        const float d = max / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint8_t *o = out + b * 18;
        put16(o, f2h(d));
        for (int j = 0; j < 16; j++) {
            int q0 = (int)(xb[j] * id + 8.5f), q1 = (int)(xb[j + 16] * id + 8.5f);
            q0 = q0 < 0 ? 0 : (q0 > 15 ? 15 : q0);
            q1 = q1 < 0 ? 0 : (q1 > 15 ? 15 : q1);
            o[2 + j] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}

// quantize::q8_0 (quant/mod.rs:265-277)
void quantize_q8_0(const float *x, size_t n, uint8_t *out) {
    for (size_t b = 0; b < n / 32; b++) {
        const float *xb = x + b * 32;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) amax = std::fmax(amax, std::fabs(xb[i]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint8_t *o = out + b * 34;
        put16(o, f2h(d));
        for (int j = 0; j < 32; j++) {
            int r = (int)std::round(xb[j] * id);
            r = r < -127 ? -127 : (r > 127 ? 127 : r);
            o[2 + j] = (uint8_t)(int8_t)r;
        }
    }
}

int nearest_int(float v) { return (int)std::nearbyint(v); }  // round half to even

float h2f_host(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1fu, man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) bits = sign;
        else {  // subnormal: renormalize
            int e = -1;
            uint32_t m = man;
            do { m <<= 1; e++; } while (!(m & 0x400u));
            bits = sign | ((uint32_t)(112 - e) << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (exp == 0x1f) bits = sign | 0x7f800000u | (man << 13);
    else bits = sign | ((exp + 112) << 23) | (man << 13);
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// Q4_K (256 values: 8 sub-blocks of 32, 6-bit scale and min each, f16 d and
// dmin; layout of dequantize_block, quant/reference.rs:8-27, 160-176).  Per
// sub-block: min = −min(0, x), scale = (max − min(0, x)) / 15; d and dmin are the
// largest scale and min over 63, the 6-bit sub-block values the nearest
// multiples of the stored f16 d and dmin, and each code the nearest level
// d·sc·q − dmin·m, q in 0..15.
void quantize_q4_k(const float *x, size_t n, uint8_t *out) {
    for (size_t b = 0; b < n / 256; b++) {
        const float *xb = x + b * 256;
        uint8_t *o = out + b * 144;
        float scale[8], mn[8];
        float max_scale = 0.0f, max_min = 0.0f;
        for (int j = 0; j < 8; j++) {
            float lo = 0.0f, hi = -INFINITY;
            for (int l = 0; l < 32; l++) {
                lo = std::fmin(lo, xb[32 * j + l]);
                hi = std::fmax(hi, xb[32 * j + l]);
            }
            scale[j] = (hi - lo) / 15.0f;
            mn[j] = -lo;
            max_scale = std::fmax(max_scale, scale[j]);
            max_min = std::fmax(max_min, mn[j]);
        }
        const uint16_t dh = f2h(max_scale / 63.0f), mh = f2h(max_min / 63.0f);
        const float d = h2f_host(dh), dmin = h2f_host(mh);
        uint8_t sc[8], m[8];
        for (int j = 0; j < 8; j++) {
            sc[j] = (uint8_t)std::min(63, std::max(0, d > 0.0f ? nearest_int(scale[j] / d) : 0));
            m[j] = (uint8_t)std::min(63, std::max(0, dmin > 0.0f ? nearest_int(mn[j] / dmin) : 0));
        }
        put16(o, dh);
        put16(o + 2, mh);
        // the 12-byte field as get_scale_min_k4 reads it: bytes 0-3 scales 0-3 with the top
        // two bits of scales 4-7, bytes 4-7 mins 0-3 with the top bits of mins 4-7, bytes
        // 8-11 the low nibbles of scales 4-7 (low) and mins 4-7 (high)
        for (int j = 0; j < 4; j++) {
            o[4 + j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
            o[8 + j] = (uint8_t)(m[j] | ((m[j + 4] >> 4) << 6));
            o[12 + j] = (uint8_t)((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
        }
        uint8_t q[256];
        for (int j = 0; j < 8; j++) {
            const float ds = d * (float)sc[j], dm = dmin * (float)m[j];
            for (int l = 0; l < 32; l++) {
                const int v = ds > 0.0f ? nearest_int((xb[32 * j + l] + dm) / ds) : 0;
                q[32 * j + l] = (uint8_t)std::min(15, std::max(0, v));
            }
        }
        // byte 32j + l: value 64j + l (low nibble), value 64j + 32 + l (high nibble)
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 32; l++) o[16 + 32 * j + l] = (uint8_t)(q[64 * j + l] | (q[64 * j + 32 + l] << 4));
    }
}

// Q6_K (256 values: 16 sub-blocks of 16 with signed 8-bit scales, f16 d; layout
// of quant/reference.rs:190-212).  Per sub-block the value of largest
// magnitude maps to code −32 (scale = that value / −32); d is the largest |scale|
// over 127, the sub-block scales the nearest multiples of the stored f16 d, and
// each code the nearest d·sc·q, q in −32..31 (stored +32).
void quantize_q6_k(const float *x, size_t n, uint8_t *out) {
    for (size_t b = 0; b < n / 256; b++) {
        const float *xb = x + b * 256;
        uint8_t *o = out + b * 210;
        float scale[16];
        float amax_scale = 0.0f;
        for (int k = 0; k < 16; k++) {
            float mx = 0.0f;
            for (int l = 0; l < 16; l++)
                if (std::fabs(xb[16 * k + l]) > std::fabs(mx)) mx = xb[16 * k + l];
            scale[k] = mx / -32.0f;
            amax_scale = std::fmax(amax_scale, std::fabs(scale[k]));
        }
        const uint16_t dh = f2h(amax_scale / 127.0f);
        const float d = h2f_host(dh);
        int8_t sc[16];
        for (int k = 0; k < 16; k++) sc[k] = (int8_t)std::min(127, std::max(-127, d > 0.0f ? nearest_int(scale[k] / d) : 0));
        uint8_t q[256];
        for (int k = 0; k < 16; k++) {
            const float ds = d * (float)sc[k];
            for (int l = 0; l < 16; l++) {
                const int v = ds != 0.0f ? nearest_int(xb[16 * k + l] / ds) : 0;
                q[16 * k + l] = (uint8_t)(std::min(31, std::max(-32, v)) + 32);
            }
        }
        uint8_t *ql = o, *qh = o + 128;
        for (int h = 0; h < 2; h++)
            for (int l = 0; l < 32; l++) {
                const uint8_t q1 = q[128 * h + l], q2 = q[128 * h + l + 32], q3 = q[128 * h + l + 64], q4 = q[128 * h + l + 96];
                ql[64 * h + l] = (uint8_t)((q1 & 0xF) | ((q3 & 0xF) << 4));
                ql[64 * h + l + 32] = (uint8_t)((q2 & 0xF) | ((q4 & 0xF) << 4));
                qh[32 * h + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
            }
        for (int k = 0; k < 16; k++) o[192 + k] = (uint8_t)sc[k];
        put16(o + 208, dh);
    }
}

// llama.cpp's choice of the layers that get the larger type in a Q4_K_M file
bool more_bits_layer(uint32_t i, uint32_t n) { return i < n / 8 || i >= 7 * n / 8 || (i - n / 8) % 3 == 2; }

uint64_t splitmix(uint64_t z) {
    z += 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

// Inverse normal CDF (Acklam's rational approximation, |rel err| < 1.2e-9,
// polished by one Newton step on erfc).
double norm_ppf(double p) {
    static const double a[6] = {-3.969683028665376e+01, 2.209460984245205e+02, -2.759285104469687e+02,
                                1.383577518672690e+02, -3.066479806614716e+01, 2.506628277459239e+00};
    static const double b[5] = {-5.447609879822406e+01, 1.615858368580409e+02, -1.556989798598866e+02,
                                6.680131188771972e+01, -1.328068155288572e+01};
    static const double c[6] = {-7.784894002430293e-03, -3.223964580411365e-01, -2.400758277161838e+00,
                                -2.549732539343734e+00, 4.374664141464968e+00, 2.938163982698783e+00};
    static const double d[4] = {7.784695709041462e-03, 3.224671290700398e-01, 2.445134137142996e+00, 3.754408661907416e+00};
    double x;
    if (p < 0.02425) {
        const double q = std::sqrt(-2 * std::log(p));
        x = (((((c[0] * q + c[1]) * q + c[2]) * q + c[3]) * q + c[4]) * q + c[5]) / ((((d[0] * q + d[1]) * q + d[2]) * q + d[3]) * q + 1);
    } else if (p > 1 - 0.02425) {
        const double q = std::sqrt(-2 * std::log(1 - p));
        x = -(((((c[0] * q + c[1]) * q + c[2]) * q + c[3]) * q + c[4]) * q + c[5]) / ((((d[0] * q + d[1]) * q + d[2]) * q + d[3]) * q + 1);
    } else {
        const double q = p - 0.5, r = q * q;
        x = (((((a[0] * r + a[1]) * r + a[2]) * r + a[3]) * r + a[4]) * r + a[5]) * q /
            (((((b[0] * r + b[1]) * r + b[2]) * r + b[3]) * r + b[4]) * r + 1);
    }
    const double e = 0.5 * std::erfc(-x / std::sqrt(2.0)) - p;
    const double u = e * std::sqrt(2 * M_PI) * std::exp(x * x / 2);
    return x - u / (1 + x * u / 2);
}

// N(0,1) samples: each 16-bit slice of an Rng output indexes a table of the
// normal quantiles at the midpoints of 65536 equal-probability cells.
struct Normal {
    static const float *table() {
        static std::vector<float> t = [] {
            std::vector<float> v(65536);
            for (int i = 0; i < 65536; i++) v[i] = (float)norm_ppf((i + 0.5) / 65536.0);
            return v;
        }();
        return t.data();
    }
    Rng r;
    uint64_t bits = 0;
    int left = 0;
    explicit Normal(uint64_t seed) : r(seed) {}
    float next() {
        if (left == 0) {
            bits = r.next();
            left = 4;
        }
        const float z = table()[bits & 0xffff];
        bits >>= 16;
        left--;
        return z;
    }
};

// one planned tensor of the image
struct Plan {
    std::string name;
    std::vector<uint64_t> dims;
    int ty;
    size_t rows, cols, bytes;
    int kind;  // 0 matrix, 1 norm (ones / 1+0.1·U), 2 f32 vector U·scale, 3 router
    float vscale;
    uint64_t data_off = 0;
};

struct Writer {
    std::vector<uint8_t> kv;
    uint64_t n_kv = 0;
    void raw(const void *p, size_t n) { kv.insert(kv.end(), (const uint8_t *)p, (const uint8_t *)p + n); }
    void u32(uint32_t v) { raw(&v, 4); }
    void u64(uint64_t v) { raw(&v, 8); }
    void str(const std::string &s) {
        u64(s.size());
        raw(s.data(), s.size());
    }
    void key(const std::string &k, uint32_t ty) {
        str(k);
        u32(ty);
        n_kv++;
    }
    void kv_u32(const std::string &k, uint32_t v) {
        key(k, 4);
        u32(v);
    }
    void kv_f32(const std::string &k, float v) {
        key(k, 6);
        raw(&v, 4);
    }
    void kv_str(const std::string &k, const std::string &v) {
        key(k, 8);
        str(v);
    }
};

bool is_kq(int t) { return t == T_Q4_K || t == T_Q5_K || t == T_Q6_K || t == T_Q2_K || t == T_Q3_K; }

}  // namespace

int32_t synth_tiny(const char *arch, int32_t wtype, rie_hip_synth_spec *s) {
    std::memset(s, 0, sizeof(*s));
    std::snprintf(s->arch, sizeof(s->arch), "%s", arch);
    const std::string a = arch;
    s->n_vocab = 384; s->n_embd = 256; s->n_layer = 2; s->n_head = 4; s->n_head_kv = 2; s->head_dim = 64;
    s->n_ff = 512; s->rope_dim = 64; s->ctx = 256;
    s->wtype = wtype;
    s->embd_type = block_size(wtype) > 1 ? T_Q8_0 : wtype;
    s->qkv_bias = a == "qwen2";
    s->qk_norm = a == "qwen3" || a == "gemma3";
    s->post_norms = a == "gemma2" || a == "gemma3";
    s->fused = a == "phi3";
    s->swa_window = (a == "gemma2" || a == "gemma3") ? 5 : 0;
    s->n_expert = (a == "qwen3moe" || a == "qwen2moe") ? 8 : 0;
    s->n_expert_used = 2;
    s->n_ff_exp = 256;
    s->n_ff_shexp = a == "qwen2moe" ? 256 : 0;
    s->seed = 1;
    s->mode = 0;
    s->rope_base = 10000.0f;
    s->output_type = -1;
    return 0;
}

int32_t synth_preset(const char *name, int32_t wtype, rie_hip_synth_spec *s) {
    struct P {
        const char *name, *arch;
        uint32_t v, e, l, h, kv, hd, ff;
        int tied;
    };
    static const P presets[] = {
        {"llama-3.2-1b", "llama", 128256, 2048, 16, 32, 8, 64, 8192, 1},
        {"llama-3.2-3b", "llama", 128256, 3072, 28, 24, 8, 128, 8192, 1},
        {"qwen2.5-0.5b", "qwen2", 151936, 896, 24, 14, 2, 64, 4864, 1},
        {"qwen2.5-1.5b", "qwen2", 151936, 1536, 28, 12, 2, 128, 8960, 1},
        {"qwen3-0.6b", "qwen3", 151936, 1024, 28, 16, 8, 128, 3072, 1},
        {"qwen3-1.7b", "qwen3", 151936, 2048, 28, 16, 8, 128, 6144, 1},
        {"qwen3-4b", "qwen3", 151936, 2560, 36, 32, 8, 128, 9728, 1},
        {"gemma-3-1b", "gemma3", 262144, 1152, 26, 4, 1, 256, 6912, 1},
        {"phi-4-mini", "phi3", 200064, 3072, 32, 24, 8, 128, 8192, 1},
        {"smollm2-360m", "llama", 49152, 960, 32, 15, 5, 64, 2560, 1},
        {"qwen3-30b-a3b", "qwen3moe", 151936, 2048, 48, 32, 4, 128, 6144, 0},
        // benchmark workload shapes that are not presets of the reference
        {"llama-3.1-8b", "llama", 128256, 4096, 32, 32, 8, 128, 14336, 0},
    };
    for (const P &p : presets) {
        if (std::strcmp(p.name, name) != 0) continue;
        synth_tiny(p.arch, wtype, s);
        s->n_vocab = p.v; s->n_embd = p.e; s->n_layer = p.l; s->n_head = p.h; s->n_head_kv = p.kv; s->head_dim = p.hd; s->n_ff = p.ff;
        s->rope_dim = std::strcmp(p.arch, "phi3") == 0 ? 96 : p.hd;
        s->ctx = 4096;
        s->swa_window = std::strcmp(p.arch, "gemma3") == 0 ? 512 : 0;
        if (std::strcmp(p.arch, "qwen3moe") == 0) {
            s->n_expert = 128;
            s->n_expert_used = 8;
            s->n_ff_exp = 768;
        }
        s->tied_output = p.tied;
        s->embd_type = block_size(wtype) > 1 ? T_Q6_K : wtype;
        if (p.e % 256 != 0 || p.ff % 256 != 0) {
            if (is_kq(wtype)) s->wtype = T_Q8_0;
            if (s->embd_type == T_Q6_K) s->embd_type = T_Q8_0;
        }
        return 0;
    }
    return -1;
}

uint8_t *synth_build(const rie_hip_synth_spec &sp, int n_threads, size_t *out_len) {
    const std::string a = sp.arch;
    const bool m1 = sp.mode == 1;
    Writer w;
    w.kv_str("general.architecture", a);
    w.kv_str("general.name", "synthetic-" + a);
    w.kv_u32(a + ".embedding_length", sp.n_embd);
    w.kv_u32(a + ".block_count", sp.n_layer);
    w.kv_u32(a + ".attention.head_count", sp.n_head);
    w.kv_u32(a + ".attention.head_count_kv", sp.n_head_kv);
    w.kv_u32(a + ".attention.key_length", sp.head_dim);
    w.kv_u32(a + ".attention.value_length", sp.head_dim);
    w.kv_u32(a + ".feed_forward_length", sp.n_ff);
    w.kv_u32(a + ".context_length", sp.ctx);
    w.kv_u32(a + ".rope.dimension_count", sp.rope_dim);
    w.kv_f32(a + ".rope.freq_base", m1 ? sp.rope_base : 10000.0f);
    w.kv_f32(a + ".attention.layer_norm_rms_epsilon", 1e-6f);
    if (sp.n_expert > 0) {
        w.kv_u32(a + ".expert_count", sp.n_expert);
        w.kv_u32(a + ".expert_used_count", sp.n_expert_used);
        w.kv_u32(a + ".expert_feed_forward_length", sp.n_ff_exp);
    }
    if (sp.swa_window > 0) w.kv_u32(a + ".attention.sliding_window", sp.swa_window);
    if (a == "granite") {
        w.kv_f32("granite.embedding_scale", 12.0f);
        w.kv_f32("granite.residual_scale", 0.22f);
        w.kv_f32("granite.logit_scale", 8.0f);
        w.kv_f32("granite.attention.scale", 0.0078125f * 8.0f);
    }
    if (a == "gemma3") w.kv_f32("gemma3.rope.freq_base", 1000000.0f);
    // mode 1 records the weight mix as llama.cpp's general.file_type (2 Q4_0, 7 Q8_0, 15 Q4_K_M, 14 Q4_K_S)
    if (m1) w.kv_u32("general.file_type", sp.mix == 1 ? 15u : sp.wtype == T_Q4_K ? 14u : sp.wtype == T_Q8_0 ? 7u : 2u);
    // vocabulary (testing.rs:264-300)
    std::vector<std::string> toks = {"<unk>", "<s>", "</s>"};
    std::vector<int32_t> types = {2, 3, 3};
    char buf[32];
    for (int b = 0; b < 256; b++) {
        std::snprintf(buf, sizeof(buf), "<0x%02X>", b);
        toks.push_back(buf);
        types.push_back(6);
    }
    if (sp.chat_template == 1) {
        for (const char *t : {"<|im_start|>", "<|im_end|>"}) { toks.push_back(t); types.push_back(3); }
    } else if (sp.chat_template == 2) {
        for (const char *t : {"<|start_header_id|>", "<|end_header_id|>", "<|eot_id|>"}) { toks.push_back(t); types.push_back(3); }
    }
    static const char *pieces[] = {"\xe2\x96\x81the", "\xe2\x96\x81" "a", "\xe2\x96\x81phone", "\xe2\x96\x81" "fast", "in", "er",
                                   "\xe2\x96\x81", "e", "t", "h", "o", "n"};
    for (const char *p : pieces)
        if (toks.size() < sp.n_vocab) { toks.push_back(p); types.push_back(1); }
    while (toks.size() < sp.n_vocab) {
        std::snprintf(buf, sizeof(buf), "[tok%zu]", toks.size());
        toks.push_back(buf);
        types.push_back(1);
    }
    toks.resize(sp.n_vocab);
    types.resize(sp.n_vocab);
    w.kv_str("tokenizer.ggml.model", "llama");
    w.key("tokenizer.ggml.tokens", 9);
    w.u32(toks.empty() ? 4 : 8);
    w.u64(toks.size());
    for (auto &t : toks) w.str(t);
    w.key("tokenizer.ggml.scores", 9);
    w.u32(sp.n_vocab ? 6 : 4);
    w.u64(sp.n_vocab);
    for (uint32_t i = 0; i < sp.n_vocab; i++) {
        float f = -(float)i;
        w.raw(&f, 4);
    }
    w.key("tokenizer.ggml.token_type", 9);
    w.u32(types.empty() ? 4 : 5);
    w.u64(types.size());
    for (auto t : types) w.raw(&t, 4);
    w.kv_u32("tokenizer.ggml.bos_token_id", 1);
    w.kv_u32("tokenizer.ggml.eos_token_id", 2);
    w.kv_u32("tokenizer.ggml.unknown_token_id", 0);
    if (sp.chat_template == 1)
        w.kv_str("tokenizer.chat_template", "{% for m in messages %}<|im_start|>{{ m.role }}\n{{ m.content }}<|im_end|>\n{% endfor %}");
    else if (sp.chat_template == 2)
        w.kv_str("tokenizer.chat_template", "<|start_header_id|>{{ role }}<|end_header_id|>\n\n{{ content }}<|eot_id|>");

    // ---- tensor plan (testing.rs:314-381) ----
    const uint64_t e = sp.n_embd, ff = sp.n_ff, qd = (uint64_t)sp.n_head * sp.head_dim, kvd = (uint64_t)sp.n_head_kv * sp.head_dim,
                   hd = sp.head_dim;
    const int wt = sp.wtype;
    std::vector<Plan> plans;
    auto add = [&](const std::string &name, std::vector<uint64_t> dims, int ty, size_t rows, size_t cols, int kind, float vs) {
        uint64_t n = 1;
        for (auto d : dims) n *= d;
        Plan p{name, dims, ty, rows, cols, (size_t)(n / block_size(ty) * block_bytes(ty)), kind, vs};
        plans.push_back(p);
    };
    const int out_ty = (m1 && sp.output_type >= 0) ? sp.output_type : sp.embd_type;
    add("token_embd.weight", {e, sp.n_vocab}, sp.embd_type, sp.n_vocab, e, 0, 0);
    add("output_norm.weight", {e}, T_F32, 1, e, 1, 0);
    if (!sp.tied_output) add("output.weight", {e, sp.n_vocab}, out_ty, sp.n_vocab, e, 0, 0);
    for (uint32_t il = 0; il < sp.n_layer; il++) {
        const std::string p = "blk." + std::to_string(il) + ".";
        add(p + "attn_norm.weight", {e}, T_F32, 1, e, 1, 0);
        if (sp.fused) add(p + "attn_qkv.weight", {e, qd + 2 * kvd}, wt, qd + 2 * kvd, e, 0, 0);
        else {
            add(p + "attn_q.weight", {e, qd}, wt, qd, e, 0, 0);
            add(p + "attn_k.weight", {e, kvd}, wt, kvd, e, 0, 0);
            add(p + "attn_v.weight", {e, kvd}, (m1 && sp.mix == 1) ? T_Q6_K : wt, kvd, e, 0, 0);
        }
        if (sp.qkv_bias) {
            add(p + "attn_q.bias", {qd}, T_F32, 1, qd, 2, 0.1f);
            add(p + "attn_k.bias", {kvd}, T_F32, 1, kvd, 2, 0.1f);
            add(p + "attn_v.bias", {kvd}, T_F32, 1, kvd, 2, 0.1f);
        }
        if (sp.qk_norm) {
            add(p + "attn_q_norm.weight", {hd}, T_F32, 1, hd, 1, 0);
            add(p + "attn_k_norm.weight", {hd}, T_F32, 1, hd, 1, 0);
        }
        add(p + "attn_output.weight", {qd, e}, wt, e, qd, 0, 0);
        const int down_ty = (m1 && sp.mix == 1 && more_bits_layer(il, sp.n_layer)) ? T_Q6_K : wt;
        if (sp.post_norms) {
            add(p + "post_attention_norm.weight", {e}, T_F32, 1, e, 1, 0);
            add(p + "post_ffw_norm.weight", {e}, T_F32, 1, e, 1, 0);
        }
        add(p + "ffn_norm.weight", {e}, T_F32, 1, e, 1, 0);
        if (sp.n_expert > 0) {
            const uint64_t ne = sp.n_expert, fx = sp.n_ff_exp;
            add(p + "ffn_gate_inp.weight", {e, ne}, T_F32, ne, e, 3, 0.5f);
            add(p + "ffn_gate_exps.weight", {e, fx, ne}, wt, fx * ne, e, 0, 0);
            add(p + "ffn_up_exps.weight", {e, fx, ne}, wt, fx * ne, e, 0, 0);
            add(p + "ffn_down_exps.weight", {fx, e, ne}, wt, e * ne, fx, 0, 0);
            if (sp.n_ff_shexp > 0) {
                const uint64_t fs = sp.n_ff_shexp;
                add(p + "ffn_gate_shexp.weight", {e, fs}, wt, fs, e, 0, 0);
                add(p + "ffn_up_shexp.weight", {e, fs}, wt, fs, e, 0, 0);
                add(p + "ffn_down_shexp.weight", {fs, e}, wt, e, fs, 0, 0);
                add(p + "ffn_gate_inp_shexp.weight", {e}, T_F32, 1, e, 2, 0.3f);
            }
        } else if (sp.fused) {
            add(p + "ffn_up.weight", {e, 2 * ff}, wt, 2 * ff, e, 0, 0);
            add(p + "ffn_down.weight", {ff, e}, wt, e, ff, 0, 0);
        } else {
            add(p + "ffn_gate.weight", {e, ff}, wt, ff, e, 0, 0);
            add(p + "ffn_up.weight", {e, ff}, wt, ff, e, 0, 0);
            add(p + "ffn_down.weight", {ff, e}, down_ty, e, ff, 0, 0);
        }
    }
    if (m1)
        for (auto &p : plans)
            if ((p.kind == 0) && !(p.ty == T_Q4_0 || p.ty == T_Q8_0 || p.ty == T_Q4_K || p.ty == T_Q6_K || p.ty == T_F32 || p.ty == T_F16))
                throw Error{E_UNSUPPORTED, std::string("unsupported: N(0,0.02) synthesis of type ") + type_name(p.ty)};
    // ---- layout (gguf.rs:407-436) ----
    std::vector<uint8_t> hdr;
    auto hput = [&](const void *p, size_t n) { hdr.insert(hdr.end(), (const uint8_t *)p, (const uint8_t *)p + n); };
    uint32_t magic = 0x46554747u, version = 3;
    uint64_t nt = plans.size();
    hput(&magic, 4);
    hput(&version, 4);
    hput(&nt, 8);
    hput(&w.n_kv, 8);
    hput(w.kv.data(), w.kv.size());
    uint64_t offset = 0;
    for (auto &p : plans) {
        uint64_t l = p.name.size();
        hput(&l, 8);
        hput(p.name.data(), p.name.size());
        uint32_t nd = (uint32_t)p.dims.size();
        hput(&nd, 4);
        for (auto d : p.dims) hput(&d, 8);
        uint32_t id = (uint32_t)p.ty;
        hput(&id, 4);
        hput(&offset, 8);
        p.data_off = offset;
        offset += (p.bytes + 31) / 32 * 32;
    }
    const size_t data_start = (hdr.size() + 31) / 32 * 32;
    const size_t total = data_start + offset;
    uint8_t *img = (uint8_t *)std::malloc(total);
    if (!img) throw Error{E_RUNTIME, "out of host memory for the synthetic image"};
    std::memcpy(img, hdr.data(), hdr.size());
    std::memset(img + hdr.size(), 0, data_start - hdr.size());
    uint8_t *data = img + data_start;
    for (auto &p : plans) {  // alignment padding after each tensor
        const size_t padded = (p.bytes + 31) / 32 * 32;
        std::memset(data + p.data_off + p.bytes, 0, padded - p.bytes);
    }
    *out_len = total;

    if (!m1) {
        // one sequential Rng stream over all tensors, in order
        Rng rng(sp.seed);
        for (auto &p : plans) {
            uint8_t *o = data + p.data_off;
            if (p.kind == 0) random_weight(rng, p.ty, p.rows, p.cols, o);
            else if (p.kind == 1) {
                for (size_t i = 0; i < p.cols; i++) {
                    float v = 1.0f + 0.1f * rng.sym();
                    std::memcpy(o + 4 * i, &v, 4);
                }
            } else {
                const size_t n = p.rows * p.cols;
                for (size_t i = 0; i < n; i++) {
                    float v = rng.sym() * p.vscale;
                    std::memcpy(o + 4 * i, &v, 4);
                }
            }
        }
        return img;
    }
    // mode 1: parallel chunks of 64 rows, independent streams
    struct Job {
        size_t plan, r0, r1;
    };
    std::vector<Job> jobs;
    for (size_t i = 0; i < plans.size(); i++)
        for (size_t r0 = 0; r0 < plans[i].rows; r0 += 64) jobs.push_back({i, r0, std::min(plans[i].rows, r0 + 64)});
    std::atomic<size_t> next{0};
    auto worker = [&]() {
        std::vector<float> vals;
        for (;;) {
            const size_t j = next.fetch_add(1);
            if (j >= jobs.size()) break;
            const Job &jb = jobs[j];
            const Plan &p = plans[jb.plan];
            Normal nrm(splitmix(sp.seed ^ splitmix((uint64_t)jb.plan * 0x100000001B3ULL + jb.r0)));
            const size_t n = (jb.r1 - jb.r0) * p.cols;
            vals.resize(n);
            const float sigma = p.kind == 3 ? 1.0f : 0.02f;
            if (p.kind == 1) {
                for (size_t i = 0; i < n; i++) vals[i] = 1.0f;
            } else {
                for (size_t i = 0; i < n; i++) vals[i] = sigma * nrm.next();
            }
            const size_t rb = row_bytes(p.ty, p.cols);
            uint8_t *o = data + p.data_off + jb.r0 * rb;
            switch (p.ty) {
            case T_Q4_0: quantize_q4_0(vals.data(), n, o); break;
            case T_Q8_0: quantize_q8_0(vals.data(), n, o); break;
            case T_Q4_K: quantize_q4_k(vals.data(), n, o); break;
            case T_Q6_K: quantize_q6_k(vals.data(), n, o); break;
            case T_F16:
                for (size_t i = 0; i < n; i++) put16(o + 2 * i, f2h(vals[i]));
                break;
            default: std::memcpy(o, vals.data(), n * 4); break;
            }
        }
    };
    Normal::table();  // build the quantile table before the workers start
    const int nth = std::max(1, n_threads > 0 ? n_threads : (int)std::thread::hardware_concurrency());
    std::vector<std::thread> th;
    for (int i = 1; i < nth; i++) th.emplace_back(worker);
    worker();
    for (auto &t : th) t.join();
    return img;
}

bool synth_quantize(int ty, const float *x, size_t n, uint8_t *out) {
    switch (ty) {
    case T_Q4_0: if (n % 32) return false; quantize_q4_0(x, n, out); return true;
    case T_Q8_0: if (n % 32) return false; quantize_q8_0(x, n, out); return true;
    case T_Q4_K: if (n % 256) return false; quantize_q4_k(x, n, out); return true;
    case T_Q6_K: if (n % 256) return false; quantize_q6_k(x, n, out); return true;
    default: return false;
    }
}

}  // namespace rie
