// model.cpp — GGUF -> HBM model loader.
//
// Follows diffuse_model_load_impl (src/diffuse-model.cpp:83-185): the same
// multi-prefix metadata keys and defaults, model_type resolution, tensor names,
// optional Q/K/V biases and the tied lm_head fallback.  Instead of keeping the
// file in host RAM for a CPU graph, every matrix is repacked into the device
// layout of dfx.h and uploaded once; Q|K|V and gate|up are stacked so one GEMM
// reads each group's shared input.
#include <cstring>
#include <memory>

#include "engine.h"
#include "gguf.h"

namespace {

struct loader {
    gguf::reader rd;
    diffuse_model * m = nullptr;
    std::string err;

    // get_u32_multi / get_f32_multi (src/diffuse-model.cpp:27-57)
    bool u32_multi(const char * suffix, uint32_t & out, uint32_t def, bool required) {
        static const char * prefixes[] = {"diffuse", "qwen2", "llama"};
        for (const char * p : prefixes)
            if (rd.get_u32(std::string(p) + "." + suffix, out)) return true;
        if (required) {
            err = std::string("missing GGUF metadata key: *.") + suffix + " (tried diffuse/qwen2/llama)";
            return false;
        }
        out = def;
        return true;
    }
    float f32_multi(const char * suffix, float def) {
        static const char * prefixes[] = {"diffuse", "qwen2", "llama"};
        float v;
        for (const char * p : prefixes)
            if (rd.get_f32(std::string(p) + "." + suffix, v)) return v;
        return def;
    }
    // detect_arch_prefix (src/diffuse-model.cpp:60-71)
    std::string arch_prefix() {
        std::string s;
        if (rd.get_str("general.architecture", s)) return s;
        uint32_t v;
        if (rd.get_u32("diffuse.block_count", v)) return "diffuse";
        if (rd.get_u32("qwen2.block_count", v)) return "qwen2";
        if (rd.get_u32("llama.block_count", v)) return "llama";
        return "unknown";
    }

    void * dalloc(size_t bytes) {
        void * p = nullptr;
        if (hipMalloc(&p, bytes ? bytes : 1) != hipSuccess) {
            err = "hipMalloc of " + std::to_string(bytes) + " bytes failed";
            return nullptr;
        }
        m->allocs.push_back(p);
        m->device_bytes += bytes;
        return p;
    }
    // Uploads go through a non-blocking stream of the loader's own (waited for): the legacy
    // stream is never used, so a load may run while another thread captures a context's stream.
    hipStream_t st = nullptr;
    ~loader() {
        if (st) (void)hipStreamDestroy(st);
    }
    bool upload(void * dst, const void * src, size_t bytes) {
        if (!st && hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess) {
            st = nullptr;
            err = "hipStreamCreate failed";
            return false;
        }
        if (hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st) != hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess) {
            err = "hipMemcpy upload failed";
            return false;
        }
        return true;
    }

    const gguf::tensor_info * need(const std::string & name) {
        const gguf::tensor_info * t = rd.tensor(name);
        if (!t) err = "tensor not found: " + name;
        return t;
    }

    // Vector (norm weight / bias) as f32: ggml_cast to F32 (src/diffuse-graph.cpp:54-56, 4-8).
    bool to_f32(const gguf::tensor_info * t, int64_t n, std::vector<float> & out) {
        if (t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3] != n) {
            err = "tensor " + t->name + " has " + std::to_string(t->ne[0]) + " elements, expected " + std::to_string(n);
            return false;
        }
        out.resize((size_t)n);
        if (t->type == DFX_TYPE_F32) {
            memcpy(out.data(), t->data, (size_t)n * 4);
        } else if (t->type == DFX_TYPE_F16) {
            const _Float16 * h = (const _Float16 *)t->data;
            for (int64_t i = 0; i < n; i++) out[i] = (float)h[i];
        } else if (t->type == 30) {  // BF16
            const uint16_t * b = (const uint16_t *)t->data;
            for (int64_t i = 0; i < n; i++) {
                const uint32_t u = (uint32_t)b[i] << 16;
                memcpy(&out[i], &u, 4);
            }
        } else {
            err = "tensor " + t->name + ": unsupported type " + gguf::type_name(t->type) + " for a vector";
            return false;
        }
        return true;
    }
    float * vec_f32(const gguf::tensor_info * t, int64_t n) {
        std::vector<float> v;
        if (!to_f32(t, n, v)) return nullptr;
        float * d = (float *)dalloc((size_t)n * 4);
        if (!d || !upload(d, v.data(), (size_t)n * 4)) return nullptr;
        return d;
    }

    bool check_matrix(const gguf::tensor_info * t, int64_t cols, int64_t rows) {
        if (t->ne[0] != cols || t->ne[1] != rows || t->ne[2] != 1 || t->ne[3] != 1) {
            err = "tensor " + t->name + " has shape [" + std::to_string(t->ne[0]) + ", " + std::to_string(t->ne[1]) +
                  "], expected [" + std::to_string(cols) + ", " + std::to_string(rows) + "]";
            return false;
        }
        if (dfx_device_row_bytes(t->type, cols) < 0) {
            err = "tensor " + t->name + ": type " + gguf::type_name(t->type) + " with row length " +
                  std::to_string(cols) + " is not supported (Q4_K, Q6_K, Q8_0, F16, F32; rows a multiple of 256)";
            return false;
        }
        return true;
    }

    // Repack a GGUF matrix into dst (device) in the device layout.
    bool put_matrix(const gguf::tensor_info * t, uint8_t * dst, dev_matrix & dm) {
        dm.type = dfx_device_type(t->type);
        dm.cols = t->ne[0];
        dm.rows = t->ne[1];
        dm.data = dst;
        const int64_t drb = dfx_device_row_bytes(t->type, dm.cols);
        std::vector<uint8_t> host((size_t)(drb * dm.rows));
        if (dfx_repack_rows(t->type, t->data, dm.rows, dm.cols, host.data()) != DFX_OK) {
            err = dfx_last_error();
            return false;
        }
        return upload(dst, host.data(), host.size());
    }

    // gate and up (same type and shape, rows a multiple of 16) repacked with their rows
    // interleaved in blocks of 16, so that one 32-column tile of the GEMM holds the gate and
    // up values of 16 F-indices and its epilogue forms silu(gate) * up.
    bool swiglu_group(const gguf::tensor_info * gate, const gguf::tensor_info * up, proj_group & g) {
        const int64_t F = gate->ne[1], K = gate->ne[0];
        const int64_t drb = dfx_device_row_bytes(gate->type, K);
        std::vector<uint8_t> hg((size_t)(drb * F)), hu((size_t)(drb * F)), both((size_t)(2 * drb * F));
        if (dfx_repack_rows(gate->type, gate->data, F, K, hg.data()) != DFX_OK ||
            dfx_repack_rows(up->type, up->data, F, K, hu.data()) != DFX_OK) {
            err = dfx_last_error();
            return false;
        }
        for (int64_t j = 0; j < F / 16; j++) {
            memcpy(both.data() + (size_t)(32 * j) * drb, hg.data() + (size_t)(16 * j) * drb, (size_t)(16 * drb));
            memcpy(both.data() + (size_t)(32 * j + 16) * drb, hu.data() + (size_t)(16 * j) * drb, (size_t)(16 * drb));
        }
        uint8_t * base = (uint8_t *)dalloc(both.size());
        if (!base || !upload(base, both.data(), both.size())) return false;
        g.all.type = dfx_device_type(gate->type);
        g.all.rows = 2 * F;
        g.all.cols = K;
        g.all.data = base;
        g.n_out = 2 * F;   // parts stay empty: the two matrices are not contiguous
        g.fused = true;
        g.swiglu = true;
        return true;
    }

    // Q|K|V (one device type; head size hd a multiple of 32) stacked into one matrix with the
    // rows of every Q and K head permuted: row 32j + i of a head is dim 16j + i (i < 16) or
    // dim hd/2 + 16j + i - 16 (i >= 16), so that one 32-column tile of the GEMM holds both
    // dims of 16 NEOX pairs and its epilogue can rotate them.  Biases follow the rows.
    bool rope_group(const gguf::tensor_info * wq, const gguf::tensor_info * wk, const gguf::tensor_info * wv,
                    const gguf::tensor_info * bq, const gguf::tensor_info * bk, const gguf::tensor_info * bv,
                    int64_t hd, proj_group & g) {
        const int64_t K = wq->ne[0];
        const int64_t drb = dfx_device_row_bytes(wq->type, K);
        const int64_t nq = wq->ne[1], nk = wk->ne[1], nv = wv->ne[1], n = nq + nk + nv;
        std::vector<uint8_t> plain((size_t)(drb * n)), both((size_t)(drb * n));
        if (dfx_repack_rows(wq->type, wq->data, nq, K, plain.data()) != DFX_OK ||
            dfx_repack_rows(wk->type, wk->data, nk, K, plain.data() + (size_t)(drb * nq)) != DFX_OK ||
            dfx_repack_rows(wv->type, wv->data, nv, K, plain.data() + (size_t)(drb * (nq + nk))) != DFX_OK) {
            err = dfx_last_error();
            return false;
        }
        // source row of every device row
        std::vector<int64_t> src((size_t)n);
        for (int64_t r = 0; r < n; r++) {
            if (r >= nq + nk) {
                src[(size_t)r] = r;
                continue;
            }
            const int64_t head = r / hd, i = r % hd, j = i / 32, c = i % 32;
            src[(size_t)r] = head * hd + (c < 16 ? 16 * j + c : hd / 2 + 16 * j + c - 16);
        }
        for (int64_t r = 0; r < n; r++)
            memcpy(both.data() + (size_t)(r * drb), plain.data() + (size_t)(src[(size_t)r] * drb), (size_t)drb);
        uint8_t * base = (uint8_t *)dalloc(both.size());
        if (!base || !upload(base, both.data(), both.size())) return false;
        g.all.type = dfx_device_type(wq->type);
        g.all.rows = n;
        g.all.cols = K;
        g.all.data = base;
        g.n_out = n;   // parts stay empty: the rows are not in Q|K|V order
        g.fused = true;
        g.rope = true;
        if (bq || bk || bv) {
            std::vector<float> bias((size_t)n, 0.0f), perm((size_t)n);
            const gguf::tensor_info * bs[3] = {bq, bk, bv};
            const int64_t off[3] = {0, nq, nq + nk}, rows[3] = {nq, nk, nv};
            for (int i = 0; i < 3; i++) {
                if (!bs[i]) continue;
                std::vector<float> v;
                if (!to_f32(bs[i], rows[i], v)) return false;
                memcpy(bias.data() + off[i], v.data(), v.size() * 4);
            }
            for (int64_t r = 0; r < n; r++) perm[(size_t)r] = bias[(size_t)src[(size_t)r]];
            g.bias = (float *)dalloc(perm.size() * 4);
            if (!g.bias || !upload(g.bias, perm.data(), perm.size() * 4)) return false;
        }
        return true;
    }

    bool group(const std::vector<const gguf::tensor_info *> & ts, const std::vector<const gguf::tensor_info *> & biases,
               proj_group & g) {
        size_t total = 0;
        bool same = true;
        for (auto * t : ts) {
            total += (size_t)(dfx_device_row_bytes(t->type, t->ne[0]) * t->ne[1]);
            if (dfx_device_type(t->type) != dfx_device_type(ts[0]->type)) same = false;
        }
        uint8_t * base = (uint8_t *)dalloc(total);
        if (!base) return false;
        size_t off = 0;
        g.n_out = 0;
        for (auto * t : ts) {
            dev_matrix dm;
            if (!put_matrix(t, base + off, dm)) return false;
            off += (size_t)(dfx_device_row_bytes(t->type, t->ne[0]) * t->ne[1]);
            g.col_off.push_back(g.n_out);
            g.n_out += dm.rows;
            g.parts.push_back(dm);
        }
        g.fused = same;
        if (same) {
            g.all = g.parts[0];
            g.all.rows = g.n_out;
        }
        bool any_bias = false;
        for (auto * b : biases) any_bias |= b != nullptr;
        if (any_bias) {
            std::vector<float> bias((size_t)g.n_out, 0.0f);
            for (size_t i = 0; i < ts.size(); i++) {
                if (!biases[i]) continue;
                std::vector<float> v;
                if (!to_f32(biases[i], g.parts[i].rows, v)) return false;
                memcpy(bias.data() + g.col_off[i], v.data(), v.size() * 4);
            }
            g.bias = (float *)dalloc(bias.size() * 4);
            if (!g.bias || !upload(g.bias, bias.data(), bias.size() * 4)) return false;
        }
        return true;
    }

    bool load(const std::string & path) {
        if (!rd.open(path, err)) return false;
        auto & hp = m->hparams;
        const std::string arch = arch_prefix();
        DIFFUSE_LOG("  detected arch prefix: %s", arch.c_str());
        if (!u32_multi("block_count", hp.n_layer, 0, true)) return false;
        if (!u32_multi("attention.head_count", hp.n_head, 0, true)) return false;
        if (!u32_multi("attention.head_count_kv", hp.n_head_kv, 0, true)) return false;
        if (!u32_multi("embedding_length", hp.n_embd, 0, true)) return false;
        if (!u32_multi("feed_forward_length", hp.n_ff, 0, true)) return false;
        if (!u32_multi("context_length", hp.n_ctx_max, 4096, true)) return false;
        u32_multi("vocab_size", hp.n_vocab, 0, false);
        u32_multi("mask_token_id", hp.mask_token_id, 0, false);
        hp.rope_theta = f32_multi("rope.freq_base", 1000000.0f);
        hp.rms_norm_eps = f32_multi("attention.layer_norm_rms_epsilon", 1e-6f);

        // model_type (src/diffuse-model.cpp:116-128)
        if (!rd.get_str("diffuse.model_type", m->model_type)) {
            m->model_type = arch == "qwen2" ? "qwen2" : arch == "llama" ? "llama" : "llada";
        }
        m->is_dream = m->model_type == "dream";
        const char * arch_name = m->model_type == "llada" ? "LLaDA (Llama backbone, diffusion)"
                               : m->model_type == "dream" ? "Dream (Qwen2.5 backbone, diffusion)"
                               : m->model_type == "qwen2" ? "Qwen2.5 (autoregressive)"
                               : m->model_type == "llama" ? "Llama (autoregressive)" : "unknown";
        DIFFUSE_LOG("  arch: %s", arch_name);

        if (hp.n_head == 0 || hp.n_head_kv == 0 || hp.n_head % hp.n_head_kv || hp.n_embd % hp.n_head) {
            err = "inconsistent head counts";
            return false;
        }
        const int64_t d = hp.n_embd, F = hp.n_ff, hd = d / hp.n_head, dkv = hd * hp.n_head_kv;

        const gguf::tensor_info * te = need("token_embd.weight");
        const gguf::tensor_info * tn = te ? need("output_norm.weight") : nullptr;
        if (!te || !tn) return false;
        if (hp.n_vocab == 0) {
            hp.n_vocab = (uint32_t)te->ne[1];
            DIFFUSE_LOG("  n_vocab inferred from token_embd: %u", hp.n_vocab);
        }
        DIFFUSE_LOG("  n_vocab=%u, n_embd=%u, n_head=%u/%u(kv), n_layer=%u, n_ff=%u", hp.n_vocab, hp.n_embd, hp.n_head,
                    hp.n_head_kv, hp.n_layer, hp.n_ff);
        DIFFUSE_LOG("  rope_theta=%.0f, rms_norm_eps=%.1e, mask_token=%u", hp.rope_theta, hp.rms_norm_eps,
                    hp.mask_token_id);
        if (hd != 64 && hd != 128) {
            err = "head_dim " + std::to_string(hd) + " not supported (64 or 128)";
            return false;
        }

        // token embedding table
        if (te->ne[0] != d || te->ne[1] < hp.n_vocab) { err = "token_embd.weight shape mismatch"; return false; }
        if (!check_matrix(te, d, te->ne[1])) return false;
        {
            uint8_t * p = (uint8_t *)dalloc((size_t)(dfx_device_row_bytes(te->type, d) * te->ne[1]));
            if (!p || !put_matrix(te, p, m->tok_embd)) return false;
        }
        if (!(m->output_norm = vec_f32(tn, d))) return false;

        // lm_head, or tied to token_embd (src/diffuse-model.cpp:156-158)
        const gguf::tensor_info * to = rd.tensor("output.weight");
        if (to) {
            if (!check_matrix(to, d, hp.n_vocab)) return false;
            uint8_t * p = (uint8_t *)dalloc((size_t)(dfx_device_row_bytes(to->type, d) * hp.n_vocab));
            if (!p || !put_matrix(to, p, m->output)) return false;
        } else {
            m->output = m->tok_embd;
            m->output.rows = hp.n_vocab;
        }

        m->layers.resize(hp.n_layer);
        char name[128];
        auto T = [&](const char * pat, int il, bool required) -> const gguf::tensor_info * {
            snprintf(name, sizeof(name), pat, il);
            return required ? need(name) : rd.tensor(name);
        };
        for (uint32_t il = 0; il < hp.n_layer; il++) {
            dev_layer & L = m->layers[il];
            const gguf::tensor_info *an = T("blk.%d.attn_norm.weight", il, true), *wq = an ? T("blk.%d.attn_q.weight", il, true) : nullptr,
                                    *wk = wq ? T("blk.%d.attn_k.weight", il, true) : nullptr,
                                    *wv = wk ? T("blk.%d.attn_v.weight", il, true) : nullptr,
                                    *wo = wv ? T("blk.%d.attn_output.weight", il, true) : nullptr,
                                    *fn = wo ? T("blk.%d.ffn_norm.weight", il, true) : nullptr,
                                    *wg = fn ? T("blk.%d.ffn_gate.weight", il, true) : nullptr,
                                    *wu = wg ? T("blk.%d.ffn_up.weight", il, true) : nullptr,
                                    *wd = wu ? T("blk.%d.ffn_down.weight", il, true) : nullptr;
            if (!wd) return false;
            const gguf::tensor_info *bq = T("blk.%d.attn_q.bias", il, false), *bk = T("blk.%d.attn_k.bias", il, false),
                                    *bv = T("blk.%d.attn_v.bias", il, false);
            if (!check_matrix(wq, d, d) || !check_matrix(wk, d, dkv) || !check_matrix(wv, d, dkv) ||
                !check_matrix(wo, d, d) || !check_matrix(wg, d, F) || !check_matrix(wu, d, F) || !check_matrix(wd, F, d))
                return false;
            if (!(L.attn_norm = vec_f32(an, d)) || !(L.ffn_norm = vec_f32(fn, d))) return false;
            const int dq = dfx_device_type(wq->type);
            if (dq == dfx_device_type(wk->type) && dq == dfx_device_type(wv->type) && hd % 32 == 0) {
                if (!rope_group(wq, wk, wv, bq, bk, bv, hd, L.qkv)) return false;
            } else if (!group({wq, wk, wv}, {bq, bk, bv}, L.qkv)) {
                return false;
            }
            if (dfx_device_type(wg->type) == dfx_device_type(wu->type) && wg->ne[1] % 16 == 0) {
                if (!swiglu_group(wg, wu, L.gu)) return false;
            } else if (!group({wg, wu}, {nullptr, nullptr}, L.gu)) {
                return false;
            }
            uint8_t * p = (uint8_t *)dalloc((size_t)(dfx_device_row_bytes(wo->type, d) * d));
            if (!p || !put_matrix(wo, p, L.o)) return false;
            p = (uint8_t *)dalloc((size_t)(dfx_device_row_bytes(wd->type, F) * d));
            if (!p || !put_matrix(wd, p, L.down)) return false;
        }
        DIFFUSE_LOG("model loaded: %zu tensors, %.2f GB in HBM", rd.tensors().size(), m->device_bytes / 1e9);
        return true;
    }
};

}  // namespace

int engine_model_load(const std::string & path, diffuse_model ** out) {
    DIFFUSE_LOG("loading model from %s", path.c_str());
    std::unique_ptr<loader> L(new loader);
    L->m = new diffuse_model();
    if (!L->load(path)) {
        dfx_set_error("%s", L->err.c_str());
        engine_model_free(L->m);
        return L->err.rfind("cannot open", 0) == 0 ? DFX_ERR_IO : DFX_ERR_FORMAT;
    }
    *out = L->m;
    return DFX_OK;
}

void engine_model_free(diffuse_model * m) {
    if (!m) return;
    for (void * p : m->allocs) (void)hipFree(p);
    delete m;
}
