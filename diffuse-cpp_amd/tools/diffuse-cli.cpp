// diffuse-cli — generate with a masked-diffusion model on the GPU.
// Command-line contract of tools/main-cli.cpp (flags 9-27, generated ids on
// stdout as comma-separated integers, progress and logs on stderr).
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "diffuse.h"

static void usage(const char * prog) {
    fprintf(stderr,
            "Usage: %s [options]\n\nOptions:\n"
            "  -m PATH     Model file (GGUF)\n"
            "  -p TEXT     Prompt text\n"
            "  -n INT      Tokens to generate (default: 128)\n"
            "  -s INT      Diffusion steps (default: 32)\n"
            "  -t INT      Threads (default: 4; host-side only)\n"
            "  --temp F    Temperature (default: 0 = argmax)\n"
            "  --seed INT  Random seed (default: 42)\n"
            "  --schedule  cosine|linear (default: cosine)\n"
            "  --remasking low_confidence|random|entropy_exit|maskgit_plus|topk_margin (default: low_confidence)\n"
            "  --entropy-threshold F  Entropy threshold for entropy_exit (default: 1.5)\n"
            "  --no-cache             Disable the inter-step KV cache\n"
            "  --cache-refresh INT    Force full forward every N steps (default: 0 = never)\n"
            "  --cache-keep-active INT  Keep recently-changed positions active N extra steps (default: 0)\n"
            "\nTokenization is external: pass pre-tokenized input with\n"
            "  --tokens IDs  Comma-separated token IDs (bypasses prompt)\n",
            prog);
}

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
    std::string model_path, prompt;
    std::vector<int32_t> ids;
    int n_generate = 128, n_threads = 4;
    diffuse_sampler_params sp;
    for (int i = 1; i < argc; i++) {
        const char * a = argv[i];
        const bool has = i + 1 < argc;
        if (!strcmp(a, "-m") && has) model_path = argv[++i];
        else if (!strcmp(a, "-p") && has) prompt = argv[++i];
        else if (!strcmp(a, "-n") && has) n_generate = atoi(argv[++i]);
        else if (!strcmp(a, "-s") && has) sp.n_steps = atoi(argv[++i]);
        else if (!strcmp(a, "-t") && has) n_threads = atoi(argv[++i]);
        else if (!strcmp(a, "--temp") && has) sp.temperature = (float)atof(argv[++i]);
        else if (!strcmp(a, "--seed") && has) sp.seed = (uint32_t)atoi(argv[++i]);
        else if (!strcmp(a, "--tokens") && has) ids = split_ids(argv[++i]);
        else if (!strcmp(a, "--schedule") && has) {
            if (!strcmp(argv[++i], "linear")) sp.schedule = diffuse_schedule::LINEAR;
        } else if (!strcmp(a, "--entropy-threshold") && has) sp.entropy_threshold = (float)atof(argv[++i]);
        else if (!strcmp(a, "--remasking") && has) {
            const char * r = argv[++i];
            if (!strcmp(r, "random")) sp.remasking = diffuse_remasking::RANDOM;
            else if (!strcmp(r, "entropy_exit")) sp.remasking = diffuse_remasking::ENTROPY_EXIT;
            else if (!strcmp(r, "maskgit_plus")) sp.remasking = diffuse_remasking::MASKGIT_PLUS;
            else if (!strcmp(r, "topk_margin")) sp.remasking = diffuse_remasking::TOPK_MARGIN;
        } else if (!strcmp(a, "--no-cache")) sp.use_cache = false;
        else if (!strcmp(a, "--cache-refresh") && has) sp.cache_refresh = atoi(argv[++i]);
        else if (!strcmp(a, "--cache-keep-active") && has) sp.cache_keep_active = atoi(argv[++i]);
        else if (!strcmp(a, "-h") || !strcmp(a, "--help")) {
            usage(argv[0]);
            return 0;
        }
    }
    if (model_path.empty()) {
        fprintf(stderr, "Error: model path required (-m)\n");
        usage(argv[0]);
        return 1;
    }
    if (ids.empty() && prompt.empty()) {
        fprintf(stderr, "Error: prompt (-p) or tokens (--tokens) required\n");
        return 1;
    }
    if (ids.empty()) {
        fprintf(stderr, "Warning: native tokenizer not yet integrated. Use --tokens with pre-tokenized input.\n");
        return 1;
    }
    fprintf(stderr, "Loading model...\n");
    diffuse_model * model = diffuse_model_load(model_path, n_threads);
    if (!model) {
        fprintf(stderr, "Failed to load model\n");
        return 1;
    }
    diffuse_context * ctx = diffuse_context_new(model, (int)ids.size() + n_generate, n_threads);
    fprintf(stderr, "Generating %d tokens with %d diffusion steps...\n", n_generate, sp.n_steps);
    std::vector<int32_t> out = diffuse_generate(ctx, ids, n_generate, sp,
        [](int step, int total, const std::vector<int32_t> &) { fprintf(stderr, "\r  step %d/%d", step, total); });
    fprintf(stderr, "\n\nGenerated token IDs:\n");
    for (size_t i = 0; i < out.size(); i++) printf(i ? ",%d" : "%d", out[i]);
    printf("\n");
    diffuse_context_free(ctx);
    diffuse_model_free(model);
    return 0;
}
