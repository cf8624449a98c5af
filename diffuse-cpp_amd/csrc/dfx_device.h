// dfx_device.h — device-side helpers shared by the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dfx.h"
#include "dfx_epi.h"

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));   // value type for 16-byte loads/stores

#define WAVE 64

// Device super-block sizes (256 elements) of each storage type.
#define SB_Q4_K 144
#define SB_Q6_K 224
#define SB_Q8_0 272
#define SB_F16  512

__device__ __forceinline__ float h2f(uint16_t h) {
    half_t v = __builtin_bit_cast(half_t, h);
    return (float)v;
}
__device__ __forceinline__ uint16_t f2h(float f) {
    half_t v = (half_t)f;   // v_cvt_f16_f32: round to nearest even
    return __builtin_bit_cast(uint16_t, v);
}

// 6-bit scale / min of sub-block j (0..7) of a Q4_K block (GGML get_scale_min_k4).
__device__ __forceinline__ void q4k_scale_min(int j, const uint8_t * s, int & sc, int & m) {
    if (j < 4) {
        sc = s[j] & 63;
        m  = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4);
        m  = (s[j + 4] >> 4)   | ((s[j]     >> 6) << 4);
    }
}

// ---- wave reductions (64 lanes) ----
// Maximum over the (fully active) wave, in every lane: within each row of 16 lanes by DPP
// moves (lane ^ 1, lane ^ 2, the mirrored quads, the mirrored halves), then over the four
// rows' results read out of lanes 0, 16, 32 and 48.  A maximum is exact in any order.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, true)));
    const int b = __float_as_int(v);
    return fmaxf(fmaxf(__int_as_float(__builtin_amdgcn_readlane(b, 0)), __int_as_float(__builtin_amdgcn_readlane(b, 16))),
                 fmaxf(__int_as_float(__builtin_amdgcn_readlane(b, 32)), __int_as_float(__builtin_amdgcn_readlane(b, 48))));
}
__device__ __forceinline__ float wave_sum(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}

// ---- converted activations (the GEMM input) ----
// GGML's mul_mat converts activations to the weight's vec_dot_type; the buffer holds
// that conversion so the GEMM can reproduce GGML's integer block dot products:
//   q   f16 [M][K]        Q8_K / Q8_0: the int8 quants (exact in f16); F16: the values
//   d   f32 [M][K/blk]    block scale (Q8_K: blk 256, f32; Q8_0: blk 32, the f16 scale)
//   bs  f16 [M][K/16]     Q8_K only: sums of q over 16-element groups (GGML bsums)
// For Q4_K weights (CONV_Q8_K_P4) q is stored in the order in which the GEMM unpacks
// Q4_K nibbles: inside every 64-element group, slot 8i+s holds element
//   s < 4:  4i + P[s]        s >= 4:  32 + 4i + P[s-4]        P = {0, 2, 1, 3}
// (one 32-bit word of packed nibbles gives the 8 operands of slots 8i..8i+7).
// For Q6_K weights (CONV_Q8_K_P6), inside every 128-element half super-block, slot
// 64*g + 8*(i + 4*p) + s holds element 32*q + 16*g + 4*i + P[s % 4] with quarter
// q = p + 2*(s >= 4) (g, p in 0..1, i in 0..3): one word of low bits (4 bytes l..l+3)
// carries quarters p and p+2.
// For F32 weights (CONV_F32) q holds the f32 activations themselves, [M][K] (GGML's
// vec_dot_type of F32 is F32: no conversion).
enum { CONV_Q8_K = 0, CONV_Q8_0 = 1, CONV_F16 = 2, CONV_Q8_K_P4 = 3, CONV_Q8_K_P6 = 4, CONV_F32 = 5 };

// Quantised GEMMs sum the scaled block dot products of each chunk of DFX_DOT_CHUNK
// K elements from zero, in K order, and add the chunk sums in order (T = T + S).
// The order does not depend on the launch, so a GEMM may split K at chunk borders.
#define DFX_DOT_CHUNK 2048
__host__ __device__ inline int dot_chunks(int64_t K) { return (int)((K + DFX_DOT_CHUNK - 1) / DFX_DOT_CHUNK); }

__host__ __device__ inline int conv_mode(int wtype) {
    return wtype == DFX_TYPE_Q4_K ? CONV_Q8_K_P4
         : wtype == DFX_TYPE_Q6_K ? CONV_Q8_K_P6
         : wtype == DFX_TYPE_Q8_0 ? CONV_Q8_0
         : wtype == DFX_TYPE_F32 ? CONV_F32 : CONV_F16;
}
__host__ __device__ inline bool conv_is_q8k(int mode) {
    return mode == CONV_Q8_K || mode == CONV_Q8_K_P4 || mode == CONV_Q8_K_P6;
}

// For both permuted modes q is stored in MFMA fragment order, rows padded to a
// multiple of 32.  The slot sl = 256*sb + 128*h + 64*hl + 8*kk + j (slot order as
// above) of row m is at half index
//   (((m/32) * (K/128) + 2*sb + h) * 8 + kk) * 512 + (m%32 + 32*hl) * 8 + j
// so that the eight A operands (32 rows x 16 slots, 1 KB each) of one 128-slot K
// step of a 32-row tile are 8 KB of consecutive memory, the 16 bytes of MFMA lane
// m%32 + 32*hl at byte 16*lane of operand kk.
__host__ __device__ inline bool conv_is_frag(int mode) { return mode == CONV_Q8_K_P4 || mode == CONV_Q8_K_P6; }
__host__ __device__ inline int64_t act_q_rows(int mode, int64_t M) { return conv_is_frag(mode) ? (M + 31) & ~(int64_t)31 : M; }
__host__ __device__ inline int64_t act_frag_off(int64_t m, int64_t sl, int64_t K) {
    const int64_t step = sl >> 7, w = sl & 127, hl = w >> 6, kk = (w >> 3) & 7, j = w & 7;
    return ((((m >> 5) * (K >> 7) + step) * 8 + kk) * 64 + (m & 31) + 32 * hl) * 8 + j;
}

// The d of the permuted modes is stored super-block major, d[K/256][ceil(M/32)*32]
// (the scales of consecutive rows of one super-block are adjacent).
// With at most DFX_GEMV_M rows, the permuted modes also keep the int8 quants in natural
// order, i8 [M][K], for the matrix-vector kernels (integer dot products).
#define DFX_GEMV_M 4
struct act_layout {
    size_t q, d, bs, i8, bytes;   // i8 = 0: no int8 plane
    int64_t mq;   // rows of q (and, for the permuted modes, the row stride of d)
};
__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }
__host__ __device__ inline act_layout act_layout_of(int mode, int64_t M, int64_t K) {
    act_layout L;
    L.q = 0;
    L.mq = act_q_rows(mode, M);
    L.d = align256((size_t)L.mq * K * (mode == CONV_F32 ? 4 : 2));
    const size_t nd = conv_is_q8k(mode) ? (size_t)L.mq * (K / 256) : mode == CONV_Q8_0 ? (size_t)M * (K / 32) : 0;
    L.bs = align256(L.d + nd * 4);
    const size_t nbs = conv_is_q8k(mode) ? (size_t)M * (K / 16) : 0;
    L.bytes = align256(L.bs + nbs * 2);
    L.i8 = 0;
    if (conv_is_frag(mode) && M <= DFX_GEMV_M) {
        L.i8 = L.bytes;
        L.bytes = align256(L.i8 + (size_t)M * K);
    }
    return L;
}


// exp inside GGML ops (silu, soft_max) is taken correctly rounded: (float)exp((double)x).
__device__ __forceinline__ float exp_cr(float x) { return (float)exp((double)x); }
// GGML ggml_silu_f32 (x / (1 + exp(-x))) times the up value, as the reference graph's
// ggml_silu + ggml_mul (src/diffuse-graph.cpp:138-139).
__device__ __forceinline__ float silu_mul(float g, float u) {
    const float e = exp_cr(-g);
    const float d = 1.0f + e;
    const float sg = g / d;   // the compiler's correctly rounded f32 division
    return sg * u;
}

// Error plumbing shared by the host-side launch wrappers.
extern "C" void dfx_set_error(const char * fmt, ...);
#define DFX_CHECK_LAUNCH(name)                                                     \
    do {                                                                           \
        hipError_t e_ = hipGetLastError();                                         \
        if (e_ != hipSuccess) {                                                    \
            dfx_set_error("%s: launch failed: %s", name, hipGetErrorString(e_));   \
            return DFX_ERR_HIP;                                                    \
        }                                                                          \
    } while (0)
