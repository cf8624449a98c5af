// quants.cpp — weight encoders (F32 -> Q4_K / Q6_K / Q8_0 / F16, GGUF block layouts)
// and the tensor-type mixture of diffuse-quantize (tools/quantize.cpp:31-110).
//
// The encoders are this library's own: per-sub-block min/max (Q4_K) or signed
// max (Q6_K) scaling with 6/8-bit scale quantisation.  They emit the standard
// GGML block layouts, so the files load anywhere GGUF does; the bytes need not
// equal GGML's quantizer output (the oracle and the GPU both read the file).
#include <cmath>
#include <cstring>
#include <string>

#include "quants.h"

static inline uint16_t f16_bits(float f) {
    _Float16 h = (_Float16)f;
    uint16_t u;
    memcpy(&u, &h, 2);
    return u;
}
static inline float f16_val(uint16_t u) {
    _Float16 h;
    memcpy(&h, &u, 2);
    return (float)h;
}
static inline int iround(float x) { return (int)lrintf(x); }
static inline int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

static void enc_q8_0(const float * x, uint8_t * out, int64_t n) {
    for (int64_t b = 0; b < n / 32; b++) {
        const float * v = x + b * 32;
        uint8_t * o = out + b * 34;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(v[j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t dh = f16_bits(d);
        memcpy(o, &dh, 2);
        for (int j = 0; j < 32; j++) o[2 + j] = (uint8_t)(int8_t)clampi((int)roundf(v[j] * id), -127, 127);
    }
}

static void enc_q4_K(const float * x, uint8_t * out, int64_t n) {
    for (int64_t b = 0; b < n / 256; b++) {
        const float * v = x + b * 256;
        uint8_t * o = out + b * 144;
        float scale[8], mn[8];
        float max_scale = 0.0f, max_min = 0.0f;
        for (int j = 0; j < 8; j++) {
            float lo = 0.0f, hi = -INFINITY;
            for (int l = 0; l < 32; l++) {
                lo = fminf(lo, v[32 * j + l]);
                hi = fmaxf(hi, v[32 * j + l]);
            }
            scale[j] = hi > lo ? (hi - lo) / 15.0f : 0.0f;
            mn[j] = -lo;   // >= 0
            max_scale = fmaxf(max_scale, scale[j]);
            max_min = fmaxf(max_min, mn[j]);
        }
        const uint16_t dh = f16_bits(max_scale / 63.0f), mh = f16_bits(max_min / 63.0f);
        const float d = f16_val(dh), dmin = f16_val(mh);
        memcpy(o, &dh, 2);
        memcpy(o + 2, &mh, 2);
        uint8_t sc[8], m[8];
        for (int j = 0; j < 8; j++) {
            sc[j] = (uint8_t)(d > 0.0f ? clampi(iround(scale[j] / d), 0, 63) : 0);
            // round the min up so x + min stays >= 0 after quantisation
            m[j] = (uint8_t)(dmin > 0.0f ? clampi((int)ceilf(mn[j] / dmin), 0, 63) : 0);
        }
        uint8_t * s = o + 4;
        memset(s, 0, 12);
        for (int j = 0; j < 4; j++) {
            s[j] = sc[j] & 63;
            s[j + 4] = m[j] & 63;
        }
        for (int j = 4; j < 8; j++) {
            s[j + 4] = (uint8_t)((sc[j] & 0x0F) | ((m[j] & 0x0F) << 4));
            s[j - 4] |= (uint8_t)((sc[j] >> 4) << 6);
            s[j] |= (uint8_t)((m[j] >> 4) << 6);
        }
        uint8_t q[256];
        for (int j = 0; j < 8; j++) {
            const float es = d * sc[j], em = dmin * m[j];
            for (int l = 0; l < 32; l++)
                q[32 * j + l] = (uint8_t)(es > 0.0f ? clampi(iround((v[32 * j + l] + em) / es), 0, 15) : 0);
        }
        uint8_t * qs = o + 16;
        for (int g = 0; g < 4; g++)
            for (int l = 0; l < 32; l++) qs[32 * g + l] = (uint8_t)(q[64 * g + l] | (q[64 * g + 32 + l] << 4));
    }
}

static void enc_q6_K(const float * x, uint8_t * out, int64_t n) {
    for (int64_t b = 0; b < n / 256; b++) {
        const float * v = x + b * 256;
        uint8_t * o = out + b * 210;
        float scale[16];
        float max_abs_scale = 0.0f;
        for (int j = 0; j < 16; j++) {
            float amax = 0.0f, mx = 0.0f;
            for (int l = 0; l < 16; l++) {
                const float a = fabsf(v[16 * j + l]);
                if (a > amax) { amax = a; mx = v[16 * j + l]; }
            }
            scale[j] = mx / -32.0f;   // the extreme value lands on q = -32
            max_abs_scale = fmaxf(max_abs_scale, fabsf(scale[j]));
        }
        const uint16_t dh = f16_bits(max_abs_scale / 127.0f);
        const float d = f16_val(dh);
        int8_t sc[16];
        for (int j = 0; j < 16; j++) sc[j] = (int8_t)(d > 0.0f ? clampi(iround(scale[j] / d), -127, 127) : 0);
        uint8_t q[256];
        for (int j = 0; j < 16; j++) {
            const float es = d * sc[j];
            for (int l = 0; l < 16; l++)
                q[16 * j + l] = (uint8_t)((es != 0.0f ? clampi(iround(v[16 * j + l] / es), -32, 31) : 0) + 32);
        }
        uint8_t * ql = o, * qh = o + 128;
        int8_t * scales = (int8_t *)(o + 192);
        for (int half = 0; half < 2; half++)
            for (int l = 0; l < 32; l++) {
                const uint8_t q1 = q[128 * half + l], q2 = q[128 * half + 32 + l], q3 = q[128 * half + 64 + l],
                              q4 = q[128 * half + 96 + l];
                ql[64 * half + l] = (uint8_t)((q1 & 15) | ((q3 & 15) << 4));
                ql[64 * half + 32 + l] = (uint8_t)((q2 & 15) | ((q4 & 15) << 4));
                qh[32 * half + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
            }
        for (int j = 0; j < 16; j++) scales[j] = sc[j];
        memcpy(o + 208, &dh, 2);
    }
}

int64_t quant_row_bytes(int type, int64_t n) {
    switch (type) {
        case QT_F32: return n * 4;
        case QT_F16: return n * 2;
        case QT_Q8_0: return n % 32 ? -1 : n / 32 * 34;
        case QT_Q4_K: return n % 256 ? -1 : n / 256 * 144;
        case QT_Q6_K: return n % 256 ? -1 : n / 256 * 210;
    }
    return -1;
}

bool quantize_rows(int type, const float * src, int64_t n_rows, int64_t n_cols, void * dst) {
    const int64_t rb = quant_row_bytes(type, n_cols);
    if (rb < 0) return false;
    uint8_t * d = (uint8_t *)dst;
    for (int64_t r = 0; r < n_rows; r++) {
        const float * x = src + r * n_cols;
        uint8_t * o = d + r * rb;
        switch (type) {
            case QT_F32: memcpy(o, x, (size_t)n_cols * 4); break;
            case QT_F16:
                for (int64_t i = 0; i < n_cols; i++) {
                    const uint16_t h = f16_bits(x[i]);
                    memcpy(o + 2 * i, &h, 2);
                }
                break;
            case QT_Q8_0: enc_q8_0(x, o, n_cols); break;
            case QT_Q4_K: enc_q4_K(x, o, n_cols); break;
            case QT_Q6_K: enc_q6_K(x, o, n_cols); break;
        }
    }
    return true;
}

// ---- diffuse-quantize mixture (tools/quantize.cpp:31-110) ----
tensor_class classify_tensor(const char * name, int n_layers) {
    if (strstr(name, "_norm") || strstr(name, "norm.")) return TC_NORM;
    if (strstr(name, ".bias")) return TC_NORM;
    if (strstr(name, "token_embd") || strstr(name, "embed")) return TC_EMBED;
    int layer = -1;
    if (const char * blk = strstr(name, "blk.")) layer = atoi(blk + 4);
    if (strstr(name, "attn_q") || strstr(name, "attn_k") || strstr(name, "attn_v") || strstr(name, "attn_output"))
        return TC_ATTN;
    if (strstr(name, "ffn_gate") || strstr(name, "ffn_up") || strstr(name, "ffn_down"))
        return (layer == 0 || layer == n_layers - 1) ? TC_FFN_EDGE : TC_FFN;
    if (strstr(name, "output.weight") || strstr(name, "lm_head")) return TC_OUTPUT;
    return TC_ATTN;
}

bool scheme_for(const char * s, quant_scheme & out) {
    const std::string t = s;
    if (t == "q8_0") { out = {"Q8_0", QT_F32, QT_F16, QT_Q8_0, QT_Q8_0, QT_Q8_0, QT_Q8_0}; return true; }
    if (t == "q4_k_m" || t == "q4_k") { out = {"Q4_K_M", QT_F32, QT_F16, QT_Q6_K, QT_Q4_K, QT_Q4_K, QT_Q6_K}; return true; }
    if (t == "q6_k") { out = {"Q6_K", QT_F32, QT_F16, QT_Q6_K, QT_Q6_K, QT_Q6_K, QT_Q6_K}; return true; }
    if (t == "f16") { out = {"F16", QT_F16, QT_F16, QT_F16, QT_F16, QT_F16, QT_F16}; return true; }
    return false;
}

int target_type(tensor_class tc, const quant_scheme & s) {
    switch (tc) {
        case TC_NORM: return s.norm;
        case TC_EMBED: return s.embed;
        case TC_OUTPUT: return s.output;
        case TC_ATTN: return s.attn;
        case TC_FFN: return s.ffn;
        case TC_FFN_EDGE: return s.ffn_edge;
    }
    return QT_F32;
}

bool is_quantized(int type) { return type == QT_Q8_0 || type == QT_Q4_K || type == QT_Q6_K; }

// Keep rules of tools/quantize.cpp:197-207 and 269-280 (block-size check).
int resolve_type(int src_type, int dst_type, int64_t n_per_row) {
    if (dst_type == src_type || (!is_quantized(dst_type) && dst_type >= src_type)) return src_type;
    if (quant_row_bytes(dst_type, n_per_row) < 0) return src_type;
    return dst_type;
}
