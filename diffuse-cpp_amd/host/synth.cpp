// synth.cpp — GGUF quantizer (diffuse-quantize) and the deterministic random-init
// model generator used for tests and benchmarks.
//
// Quantizer: tools/quantize.cpp:126-357 — per tensor classify -> target type ->
// keep / convert to F32 / quantize row-wise along ne0, metadata copied.
//
// Generator: writes what tools/convert-llada.py / convert-dream.py (--type f16)
// followed by diffuse-quantize would produce for a random-init checkpoint, in one
// pass: every value is drawn, rounded to f16 (the converter's output type), then
// converted with the scheme's mixture.  Keys and tensor names follow the
// converters (convert-llada.py:185-202, 43-60; convert-dream.py:180-195, 43-63).
//   value(name, i) = sigma * N(0,1), pairs (2k, 2k+1) from one splitmix64 draw of
//   key = splitmix64(seed ^ fnv1a64(name)) + k through Box-Muller (logf/cosf/sinf);
//   norm weights are 1.0.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include "dfx.h"
#include "gguf.h"
#include "quants.h"

extern "C" void dfx_set_error(const char * fmt, ...);

namespace {

uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

uint64_t fnv1a64(const std::string & s) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (unsigned char c : s) {
        h ^= c;
        h *= 0x100000001b3ull;
    }
    return h;
}

int pick_threads(int n) {
    if (n > 0) return n;
    const unsigned hc = std::thread::hardware_concurrency();
    return (int)std::min<unsigned>(hc ? hc : 4, 16);
}

template <typename F> void parallel_rows(int64_t n_rows, int n_threads, F fn) {
    const int nt = (int)std::min<int64_t>(n_threads, std::max<int64_t>(n_rows / 8, 1));
    if (nt <= 1) {
        fn(0, n_rows);
        return;
    }
    std::atomic<int64_t> next(0);
    const int64_t chunk = std::max<int64_t>(1, n_rows / (nt * 16));
    std::vector<std::thread> th;
    for (int t = 0; t < nt; t++)
        th.emplace_back([&]() {
            for (;;) {
                const int64_t r0 = next.fetch_add(chunk);
                if (r0 >= n_rows) break;
                fn(r0, std::min(n_rows, r0 + chunk));
            }
        });
    for (auto & t : th) t.join();
}

float f16_round(float x) { return (float)(_Float16)x; }

// Random values of rows [r0, r1) of a tensor with ne0 = cols, already f16-rounded.
void draw_rows(uint64_t stream, float sigma, int64_t cols, int64_t r0, int64_t r1, float * out) {
    const int64_t i0 = r0 * cols, i1 = r1 * cols;
    for (int64_t i = i0 & ~1ll; i < i1; i += 2) {
        const uint64_t z = splitmix64(stream + (uint64_t)(i >> 1));
        const float u1 = (float)((z >> 40) + 1) * (1.0f / 16777216.0f);
        const float u2 = (float)(z & 0xFFFFFF) * (1.0f / 16777216.0f);
        const float r = sqrtf(-2.0f * logf(u1));
        const float a = 6.283185307179586f * u2;
        if (i >= i0) out[i - i0] = f16_round(sigma * r * cosf(a));
        if (i + 1 < i1) out[i + 1 - i0] = f16_round(sigma * r * sinf(a));
    }
}

struct blob {
    std::string name;
    int type;
    int n_dims;
    int64_t ne[2];
    std::vector<uint8_t> data;
};

}  // namespace

extern "C" int dfx_quantize_rows(int type, const float * src, int64_t n_rows, int64_t n_cols, void * dst) {
    if (!quantize_rows(type, src, n_rows, n_cols, dst)) {
        dfx_set_error("dfx_quantize_rows: type %d with %lld columns not supported", type, (long long)n_cols);
        return DFX_ERR_UNSUPPORTED;
    }
    return DFX_OK;
}

extern "C" int dfx_synth_model(const char * path, const dfx_synth_spec * s) {
    quant_scheme sch;
    const char * scheme = s && s->scheme ? s->scheme : "f16";
    if (path && s && !strcmp(scheme, "f32")) {
        // the converters' default output type (tools/convert-llada.py --type f32): every
        // tensor F32 (the generator's f16-rounded draws are exact in it)
        sch = {"F32", QT_F32, QT_F32, QT_F32, QT_F32, QT_F32, QT_F32};
    } else if (!path || !s || !scheme_for(scheme, sch)) {
        dfx_set_error("dfx_synth_model: bad arguments or unknown scheme");
        return DFX_ERR_ARG;
    }
    if (!s->n_head || !s->n_head_kv || s->n_head % s->n_head_kv || s->n_embd % s->n_head) {
        dfx_set_error("dfx_synth_model: inconsistent head counts");
        return DFX_ERR_ARG;
    }
    const int nt = pick_threads(s->n_threads);
    const int64_t d = s->n_embd, F = s->n_ff, V = s->n_vocab, L = s->n_layer;
    const int64_t dkv = d / s->n_head * s->n_head_kv;

    std::vector<std::unique_ptr<blob>> blobs;
    auto add = [&](const std::string & name, int64_t cols, int64_t rows, bool is_norm, bool is_bias) -> bool {
        std::unique_ptr<blob> b(new blob);
        b->name = name;
        b->n_dims = rows > 1 || !(is_norm || is_bias) ? 2 : 1;
        b->ne[0] = cols;
        b->ne[1] = rows;
        const int dst = resolve_type(QT_F16, target_type(classify_tensor(name.c_str(), (int)L), sch), cols);
        b->type = dst;
        const int64_t rb = quant_row_bytes(dst, cols);
        if (rb < 0) {
            dfx_set_error("dfx_synth_model: cannot encode %s", name.c_str());
            return false;
        }
        b->data.resize((size_t)(rb * rows));
        const uint64_t stream = splitmix64(s->seed ^ fnv1a64(name));
        parallel_rows(rows, nt, [&](int64_t r0, int64_t r1) {
            std::vector<float> buf((size_t)((r1 - r0) * cols));
            if (is_norm) std::fill(buf.begin(), buf.end(), 1.0f);
            else draw_rows(stream, s->sigma, cols, r0, r1, buf.data());
            quantize_rows(dst, buf.data(), r1 - r0, cols, b->data.data() + r0 * rb);
        });
        blobs.push_back(std::move(b));
        return true;
    };

    bool ok = add("token_embd.weight", d, V, false, false) && add("output_norm.weight", d, 1, true, false) &&
              (s->tied_output || add("output.weight", d, V, false, false));
    for (int64_t il = 0; ok && il < L; il++) {
        const std::string p = "blk." + std::to_string(il) + ".";
        ok = add(p + "attn_norm.weight", d, 1, true, false) && add(p + "attn_q.weight", d, d, false, false) &&
             add(p + "attn_k.weight", d, dkv, false, false) && add(p + "attn_v.weight", d, dkv, false, false);
        if (ok && s->is_dream)
            ok = add(p + "attn_q.bias", d, 1, false, true) && add(p + "attn_k.bias", dkv, 1, false, true) &&
                 add(p + "attn_v.bias", dkv, 1, false, true);
        ok = ok && add(p + "attn_output.weight", d, d, false, false) && add(p + "ffn_norm.weight", d, 1, true, false) &&
             add(p + "ffn_gate.weight", d, F, false, false) && add(p + "ffn_up.weight", d, F, false, false) &&
             add(p + "ffn_down.weight", F, d, false, false);
    }
    if (!ok) return DFX_ERR_UNSUPPORTED;

    gguf::writer w;
    w.set_str("general.architecture", "diffuse");
    w.set_str("general.name", s->is_dream ? "Dream-synthetic" : "LLaDA-synthetic");
    w.set_u32("diffuse.block_count", s->n_layer);
    w.set_u32("diffuse.context_length", s->n_ctx_max ? s->n_ctx_max : 4096);
    w.set_u32("diffuse.embedding_length", s->n_embd);
    w.set_u32("diffuse.feed_forward_length", s->n_ff);
    w.set_u32("diffuse.attention.head_count", s->n_head);
    w.set_u32("diffuse.attention.head_count_kv", s->n_head_kv);
    w.set_f32("diffuse.rope.freq_base", s->rope_theta);
    w.set_f32("diffuse.attention.layer_norm_rms_epsilon", s->rms_norm_eps);
    w.set_u32("diffuse.vocab_size", s->n_vocab);
    w.set_u32("diffuse.mask_token_id", s->mask_token_id);
    w.set_str("diffuse.model_type", s->is_dream ? "dream" : "llada");
    for (auto & b : blobs) w.add_tensor(b->name, b->type, b->n_dims, b->ne, b->data.data(), b->data.size());
    std::string err;
    if (!w.write(path, err)) {
        dfx_set_error("%s", err.c_str());
        return DFX_ERR_IO;
    }
    return DFX_OK;
}

extern "C" int dfx_quantize_file(const char * in_path, const char * out_path, const char * scheme_str, int n_threads) {
    quant_scheme sch;
    if (!in_path || !out_path || !scheme_str || !scheme_for(scheme_str, sch)) {
        dfx_set_error("dfx_quantize_file: unknown type '%s' (supported: q8_0, q4_k_m, q6_k, f16)",
                      scheme_str ? scheme_str : "");
        return DFX_ERR_ARG;
    }
    gguf::reader rd;
    std::string err;
    if (!rd.open(in_path, err)) {
        dfx_set_error("%s", err.c_str());
        return DFX_ERR_IO;
    }
    uint32_t n_layers = 32;   // tools/quantize.cpp:156-159
    if (const gguf::value * v = rd.find("diffuse.block_count")) n_layers = (uint32_t)v->u;
    const int nt = pick_threads(n_threads);
    gguf::writer w;
    for (const auto & kv : rd.kvs()) w.set_value(kv.first, kv.second);
    std::vector<std::vector<uint8_t>> bufs;
    bufs.reserve(rd.tensors().size());
    for (const auto & t : rd.tensors()) {
        const int dst = target_type(classify_tensor(t.name.c_str(), (int)n_layers), sch);
        const int64_t per_row = t.n_dims > 1 ? t.ne[0] : t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3];
        const int64_t nrows = t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3] / per_row;
        const bool src_float = t.type == QT_F32 || t.type == QT_F16 || t.type == 30;
        const int out_type = src_float ? resolve_type(t.type, dst, per_row) : t.type;
        if (out_type == t.type) {
            w.add_tensor(t.name, t.type, t.n_dims, t.ne, t.data, t.nbytes);
            continue;
        }
        const int64_t rb = quant_row_bytes(out_type, per_row);
        bufs.emplace_back((size_t)(rb * nrows));
        std::vector<uint8_t> & out = bufs.back();
        parallel_rows(nrows, nt, [&](int64_t r0, int64_t r1) {
            std::vector<float> f((size_t)((r1 - r0) * per_row));
            for (int64_t i = 0; i < (int64_t)f.size(); i++) {
                const int64_t e = r0 * per_row + i;
                if (t.type == QT_F32) f[i] = ((const float *)t.data)[e];
                else if (t.type == QT_F16) f[i] = (float)((const _Float16 *)t.data)[e];
                else {
                    const uint32_t u = (uint32_t)((const uint16_t *)t.data)[e] << 16;
                    memcpy(&f[i], &u, 4);
                }
            }
            quantize_rows(out_type, f.data(), r1 - r0, per_row, out.data() + r0 * rb);
        });
        w.add_tensor(t.name, out_type, t.n_dims, t.ne, out.data(), out.size());
    }
    if (!w.write(out_path, err)) {
        dfx_set_error("%s", err.c_str());
        return DFX_ERR_IO;
    }
    return DFX_OK;
}
