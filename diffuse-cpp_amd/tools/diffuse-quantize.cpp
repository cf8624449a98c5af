// diffuse-quantize — F16/F32 GGUF -> quantized GGUF with the Q4_K_M / Q8_0 mixture of
// tools/quantize.cpp (usage: diffuse-quantize in.gguf out.gguf q4_k_m|q8_0|q6_k|f16).
#include <cstdio>

#include "dfx.h"

int main(int argc, char ** argv) {
    if (argc != 4) {
        fprintf(stderr, "Usage: %s <input.gguf> <output.gguf> <type>\n\nTypes: q8_0, q4_k_m, q6_k, f16\n", argv[0]);
        return 1;
    }
    fprintf(stderr, "Quantizing: %s -> %s [%s]\n", argv[1], argv[2], argv[3]);
    if (dfx_quantize_file(argv[1], argv[2], argv[3], 0) != DFX_OK) {
        fprintf(stderr, "Error: %s\n", dfx_last_error());
        return 1;
    }
    fprintf(stderr, "Done!\n");
    return 0;
}
