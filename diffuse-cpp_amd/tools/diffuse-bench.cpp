// diffuse-bench — throughput sweep over schedulers x steps x threads.
// Contract of tools/main-bench.cpp: same flags and defaults (82-93), dummy prompt of
// --prompt-len ids = 1 without --tokens (104), COSINE / T=0 / seed 42 with the
// default cache setting (155-161), warmup + timed reps, tok/s = n_generate / s,
// same JSON and markdown output.  Extra: --schedulers LIST restricts the sweep.
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "diffuse.h"

static std::vector<int> split_ints(const char * s) {
    std::vector<int> v;
    while (*s) {
        v.push_back(atoi(s));
        while (*s && *s != ',') s++;
        if (*s == ',') s++;
    }
    return v;
}

struct result {
    int steps, threads;
    std::string sched;
    double ms, tps;
    int actual;
};

int main(int argc, char ** argv) {
    std::string model_path, sched_filter;
    std::vector<int32_t> ids;
    int n_generate = 256, n_reps = 3, n_warmup = 1, prompt_len = 32;
    std::vector<int> steps_list = {8, 16, 32}, threads_list = {1, 4, 12};
    bool json = false;
    float tau = 1.5f;
    for (int i = 1; i < argc; i++) {
        const char * a = argv[i];
        const bool has = i + 1 < argc;
        if (!strcmp(a, "-m") && has) model_path = argv[++i];
        else if (!strcmp(a, "--tokens") && has) {
            for (int v : split_ints(argv[++i])) ids.push_back(v);
        } else if (!strcmp(a, "-n") && has) n_generate = atoi(argv[++i]);
        else if (!strcmp(a, "-s") && has) steps_list = split_ints(argv[++i]);
        else if (!strcmp(a, "-t") && has) threads_list = split_ints(argv[++i]);
        else if (!strcmp(a, "-r") && has) n_reps = atoi(argv[++i]);
        else if (!strcmp(a, "--warmup") && has) n_warmup = atoi(argv[++i]);
        else if (!strcmp(a, "--json")) json = true;
        else if (!strcmp(a, "--entropy-threshold") && has) tau = (float)atof(argv[++i]);
        else if (!strcmp(a, "--prompt-len") && has) prompt_len = atoi(argv[++i]);
        else if (!strcmp(a, "--schedulers") && has) sched_filter = argv[++i];
        else if (!strcmp(a, "-h") || !strcmp(a, "--help")) {
            fprintf(stderr,
                    "Usage: %s -m MODEL [options]\n"
                    "  --tokens IDs   Pre-tokenized input (comma-separated)\n"
                    "  --prompt-len N Dummy prompt length if no --tokens (default: 32)\n"
                    "  -n INT         Tokens to generate (default: 256)\n"
                    "  -s LIST        Step counts (default: 8,16,32)\n"
                    "  -t LIST        Thread counts (default: 1,4,12)\n"
                    "  -r INT         Repetitions (default: 3)\n"
                    "  --warmup INT   Warmup runs (default: 1)\n"
                    "  --json         Output JSON instead of table\n"
                    "  --entropy-threshold F  (default: 1.5)\n"
                    "  --schedulers LIST  subset of low_confidence,entropy_exit,maskgit_plus,topk_margin\n",
                    argv[0]);
            return 0;
        }
    }
    if (model_path.empty()) {
        fprintf(stderr, "Error: -m MODEL required\n");
        return 1;
    }
    if (ids.empty()) {
        ids.assign(prompt_len, 1);
        fprintf(stderr, "No --tokens given, using dummy prompt (%d tokens)\n", prompt_len);
    }
    struct sched { const char * name; diffuse_remasking r; };
    const sched all[] = {{"low_confidence", diffuse_remasking::LOW_CONFIDENCE},
                         {"entropy_exit", diffuse_remasking::ENTROPY_EXIT},
                         {"maskgit_plus", diffuse_remasking::MASKGIT_PLUS},
                         {"topk_margin", diffuse_remasking::TOPK_MARGIN}};
    std::vector<sched> scheds;
    for (const sched & s : all)
        if (sched_filter.empty() || strstr(sched_filter.c_str(), s.name)) scheds.push_back(s);

    int max_threads = 1;
    for (int t : threads_list) max_threads = t > max_threads ? t : max_threads;
    fprintf(stderr, "Loading model: %s\n", model_path.c_str());
    diffuse_model * model = diffuse_model_load(model_path, max_threads);
    if (!model) {
        fprintf(stderr, "Failed to load model\n");
        return 1;
    }
    const diffuse_hparams & hp = diffuse_model_hparams(model);
    const int n_ctx = (int)ids.size() + n_generate;
    fprintf(stderr, "  n_vocab=%d n_embd=%d n_layer=%d\n", hp.n_vocab, hp.n_embd, hp.n_layer);
    fprintf(stderr, "  prompt=%d gen=%d\n", (int)ids.size(), n_generate);
    fprintf(stderr, "  steps=%zu configs, threads=%zu configs, reps=%d, warmup=%d\n\n", steps_list.size(),
            threads_list.size(), n_reps, n_warmup);

    std::vector<result> results;
    const int total = (int)(scheds.size() * steps_list.size() * threads_list.size());
    int idx = 0;
    for (const sched & s : scheds)
        for (int steps : steps_list)
            for (int threads : threads_list) {
                fprintf(stderr, "[%d/%d] %s s=%d t=%d ...", ++idx, total, s.name, steps, threads);
                fflush(stderr);
                diffuse_context * ctx = diffuse_context_new(model, n_ctx, threads);
                diffuse_sampler_params sp;
                sp.n_steps = steps;
                sp.temperature = 0.0f;
                sp.seed = 42;
                sp.schedule = diffuse_schedule::COSINE;
                sp.remasking = s.r;
                sp.entropy_threshold = tau;
                for (int w = 0; w < n_warmup; w++) diffuse_generate(ctx, ids, n_generate, sp);
                double sum = 0;
                int last = 0;
                for (int r = 0; r < n_reps; r++) {
                    int actual = 0;
                    const auto t0 = std::chrono::high_resolution_clock::now();
                    diffuse_generate(ctx, ids, n_generate, sp,
                                     [&actual](int step, int, const std::vector<int32_t> &) { actual = step; });
                    const auto t1 = std::chrono::high_resolution_clock::now();
                    const double ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
                    sum += ms;
                    last = actual;
                    results.push_back({steps, threads, s.name, ms, n_generate / (ms / 1000.0), actual});
                }
                const double avg = sum / n_reps;
                fprintf(stderr, " %.0fms (%.2f tok/s, %d steps)\n", avg, n_generate / (avg / 1000.0), last);
                diffuse_context_free(ctx);
            }
    if (json) {
        printf("{\n  \"model\": \"%s\",\n  \"n_prompt\": %d,\n  \"n_generate\": %d,\n  \"n_reps\": %d,\n  \"results\": [\n",
               model_path.c_str(), (int)ids.size(), n_generate, n_reps);
        for (size_t i = 0; i < results.size(); i++) {
            const result & r = results[i];
            printf("    {\"scheduler\": \"%s\", \"steps\": %d, \"threads\": %d, \"elapsed_ms\": %.1f, "
                   "\"tok_per_sec\": %.2f, \"actual_steps\": %d}%s\n",
                   r.sched.c_str(), r.steps, r.threads, r.ms, r.tps, r.actual, i + 1 < results.size() ? "," : "");
        }
        printf("  ]\n}\n");
    } else {
        printf("\n## Benchmark Results\n\n| Scheduler | Steps | Threads | Avg Time (ms) | tok/s | Actual Steps |\n"
               "|---|---|---|---|---|---|\n");
        for (const sched & s : scheds)
            for (int steps : steps_list)
                for (int threads : threads_list) {
                    double sum = 0;
                    int cnt = 0, actual = 0;
                    for (const result & r : results)
                        if (r.sched == s.name && r.steps == steps && r.threads == threads) {
                            sum += r.ms;
                            actual = r.actual;
                            cnt++;
                        }
                    if (cnt)
                        printf("| %s | %d | %d | %.0f | %.2f | %d |\n", s.name, steps, threads, sum / cnt,
                               n_generate / (sum / cnt / 1000.0), actual);
                }
    }
    diffuse_model_free(model);
    return 0;
}
