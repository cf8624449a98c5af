// dump-logits — one forward pass, logits written as [int32 n_tokens, int32 n_vocab,
// f32 logits row-major by position] (the file format of tools/dump-logits.cpp:81-86).
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

#include "diffuse.h"

static std::vector<int32_t> split_ids(const char * s) {
    std::vector<int32_t> v;
    while (*s) {
        v.push_back(atoi(s));
        while (*s && *s != ',') s++;
        if (*s == ',') s++;
    }
    return v;
}

int main(int argc, char ** argv) {
    std::string model_path, out_path = "logits.bin";
    std::vector<int32_t> ids;
    int n_threads = 4;
    for (int i = 1; i < argc; i++) {
        if (!strcmp(argv[i], "-m") && i + 1 < argc) model_path = argv[++i];
        else if (!strcmp(argv[i], "-o") && i + 1 < argc) out_path = argv[++i];
        else if (!strcmp(argv[i], "--tokens") && i + 1 < argc) ids = split_ids(argv[++i]);
        else if (!strcmp(argv[i], "-t") && i + 1 < argc) n_threads = atoi(argv[++i]);
    }
    if (model_path.empty() || ids.empty()) {
        fprintf(stderr, "Usage: dump-logits -m MODEL.gguf --tokens 1,2,3 [-o logits.bin] [-t threads]\n");
        return 1;
    }
    fprintf(stderr, "Loading model: %s\n", model_path.c_str());
    diffuse_model * model = diffuse_model_load(model_path, n_threads);
    if (!model) return 1;
    const diffuse_hparams & hp = diffuse_model_hparams(model);
    const int n = (int)ids.size();
    diffuse_context * ctx = diffuse_context_new(model, n, n_threads);
    std::vector<float> logits((size_t)n * hp.n_vocab);
    const auto t0 = std::chrono::steady_clock::now();
    const bool ok = diffuse_forward(ctx, ids.data(), n, logits.data());
    const auto t1 = std::chrono::steady_clock::now();
    if (!ok) {
        fprintf(stderr, "Forward pass failed\n");
        return 1;
    }
    fprintf(stderr, "Forward pass: %.1f ms\n", std::chrono::duration<double, std::milli>(t1 - t0).count());
    FILE * f = fopen(out_path.c_str(), "wb");
    if (!f) {
        fprintf(stderr, "Failed to open %s for writing\n", out_path.c_str());
        return 1;
    }
    const int32_t header[2] = {n, (int32_t)hp.n_vocab};
    fwrite(header, sizeof(int32_t), 2, f);
    fwrite(logits.data(), sizeof(float), logits.size(), f);
    fclose(f);
    fprintf(stderr, "Logits saved: %s (%d x %u)\n", out_path.c_str(), n, hp.n_vocab);
    for (int i = 0; i < n && i < 8; i++) {
        const float * row = logits.data() + (size_t)i * hp.n_vocab;
        std::vector<std::pair<float, int>> s(hp.n_vocab);
        for (uint32_t v = 0; v < hp.n_vocab; v++) s[v] = {row[v], (int)v};
        const int k = std::min<int>(5, (int)hp.n_vocab);
        std::partial_sort(s.begin(), s.begin() + k, s.end(),
                          [](const std::pair<float, int> & a, const std::pair<float, int> & b) { return a.first > b.first; });
        fprintf(stderr, "  pos %d (in=%d): ", i, ids[i]);
        for (int j = 0; j < k; j++) fprintf(stderr, "%d(%.2f) ", s[j].second, s[j].first);
        fprintf(stderr, "\n");
    }
    diffuse_context_free(ctx);
    diffuse_model_free(model);
    return 0;
}
