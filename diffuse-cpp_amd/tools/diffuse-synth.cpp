// diffuse-synth — write a deterministic random-init model as GGUF.
//   diffuse-synth OUT.gguf {llada-8b|dream-7b|tiny} [scheme=q4_k_m] [seed=0]
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "dfx.h"

int main(int argc, char ** argv) {
    if (argc < 3) {
        fprintf(stderr, "Usage: %s OUT.gguf {llada-8b|dream-7b|tiny} [q4_k_m|q8_0|q6_k|f16] [seed]\n", argv[0]);
        return 1;
    }
    dfx_synth_spec s = {};
    s.sigma = 0.02f;
    s.scheme = argc > 3 ? argv[3] : "q4_k_m";
    s.seed = argc > 4 ? strtoull(argv[4], nullptr, 10) : 0;
    s.n_ctx_max = 4096;
    if (!strcmp(argv[2], "llada-8b")) {
        s.n_vocab = 126464; s.n_embd = 4096; s.n_head = 32; s.n_head_kv = 32; s.n_layer = 32; s.n_ff = 12288;
        s.rope_theta = 500000.0f; s.rms_norm_eps = 1e-5f; s.mask_token_id = 126336;
    } else if (!strcmp(argv[2], "dream-7b")) {
        s.n_vocab = 152064; s.n_embd = 3584; s.n_head = 28; s.n_head_kv = 4; s.n_layer = 28; s.n_ff = 18944;
        s.rope_theta = 1000000.0f; s.rms_norm_eps = 1e-6f; s.mask_token_id = 151666; s.is_dream = 1;
    } else if (!strcmp(argv[2], "tiny")) {
        s.n_vocab = 1024; s.n_embd = 512; s.n_head = 4; s.n_head_kv = 4; s.n_layer = 2; s.n_ff = 1024;
        s.rope_theta = 500000.0f; s.rms_norm_eps = 1e-5f; s.mask_token_id = 1000;
    } else {
        fprintf(stderr, "unknown architecture %s\n", argv[2]);
        return 1;
    }
    if (dfx_synth_model(argv[1], &s) != DFX_OK) {
        fprintf(stderr, "Error: %s\n", dfx_last_error());
        return 1;
    }
    fprintf(stderr, "wrote %s\n", argv[1]);
    return 0;
}
