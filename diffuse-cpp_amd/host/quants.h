// quants.h — weight encoders and the diffuse-quantize type mixture.
#pragma once
#include <cstdint>

// GGML type ids
enum { QT_F32 = 0, QT_F16 = 1, QT_Q8_0 = 8, QT_Q4_K = 12, QT_Q6_K = 14 };

int64_t quant_row_bytes(int type, int64_t n);   // GGUF bytes of one row, -1 if unsupported
bool    quantize_rows(int type, const float * src, int64_t n_rows, int64_t n_cols, void * dst);

// tools/quantize.cpp:39-46
enum tensor_class { TC_NORM, TC_EMBED, TC_OUTPUT, TC_ATTN, TC_FFN, TC_FFN_EDGE };

struct quant_scheme {
    const char * name;
    int norm, embed, output, attn, ffn, ffn_edge;
};

tensor_class classify_tensor(const char * name, int n_layers);
bool scheme_for(const char * type_str, quant_scheme & out);
int  target_type(tensor_class tc, const quant_scheme & s);
bool is_quantized(int type);
int  resolve_type(int src_type, int dst_type, int64_t n_per_row);
