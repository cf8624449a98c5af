// dfx_epi.h — GEMM epilogue selection, shared by the kernels and the host code.
#pragma once
#include <stdint.h>

// Epilogues:
//   DFX_EPI_PLAIN   y = (v + bias) + residual, written to Y[ymap[m] * ldy + n].
//   DFX_EPI_SWIGLU  gate|up columns interleaved in blocks of 32 (columns 32j + i, i < 16: gate
//                   of F-index 16j + i; i >= 16: up of 16j + i - 16), written as
//                   h[m][f] = silu(gate) * up with row stride ldy.
//   DFX_EPI_ROPE    the columns are Q|K|V heads (H, Hkv and Hkv heads of hd columns; this GEMM's
//                   column 0 is column col0 of that layout).  Within a Q or K head the columns
//                   come in blocks of 32: block j holds dims 16j..16j+15, then the dims
//                   hd/2 + 16j.. of the same NEOX pairs.  v = acc (+ bias) is rotated at
//                   position pos[m] with tab[pos][hd/2][cos, sin] and stored as q_out[m][H][hd]
//                   (Q) or kc[pos][Hkv][hd] (K); V is stored transposed, vt[Hkv][hd][v_ld] at
//                   column pos[m].  Nothing is written to Y.
#define DFX_EPI_PLAIN 0
#define DFX_EPI_SWIGLU 1
#define DFX_EPI_ROPE 2

struct dfx_epi {
    int kind;
    int col0, H, Hkv, hd;
    const int32_t * pos;
    const float * tab;
    float * q_out;
    float * kc;
    float * vt;
    int64_t v_ld;
    // Completion counters of tiles whose K range is split over two workgroups inside one
    // launch (the later of the two adds the halves and applies the epilogue); one int per
    // tile, 128 bytes apart, zero before the call and left zero after it.  Null: no such
    // split (any epilogue kind may use it).
    int32_t * tile_cnt;
};
