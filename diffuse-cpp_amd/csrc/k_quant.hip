// k_quant.hip — dequantisation, embedding gather and the activation-side
// conversions that feed the MFMA GEMMs (RMSNorm, SwiGLU, plain convert).
//
// Activation conversion restates what GGML's mul_mat does to src1 before the
// dot products: rows are converted to the weight's vec_dot_type (Q8_K blocks of
// 256 for Q4_K/Q6_K, Q8_0 blocks of 32 for Q8_0, F16 for F16).  The GEMM then
// consumes f16(d*q), so the activation rounding of the reference is reproduced
// value for value (up to the final f16 rounding of d*q).
#include "dfx_device.h"

// ---------------------------------------------------------------------------
// Dequantisation of one element of a device-layout row (bit-exact with GGML
// dequantize_row_q4_K / _q6_K / _q8_0 / fp16_to_fp32: no FMA contraction, same
// association order).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float dequant_elem(int type, const uint8_t * row, int64_t e) {
#pragma clang fp contract(off)
    const int64_t sb = e >> 8;
    const int i = (int)(e & 255);
    if (type == DFX_TYPE_Q4_K) {
        const uint8_t * b = row + sb * SB_Q4_K;
        const float d = h2f(*(const uint16_t *)(b + 0));
        const float dmin = h2f(*(const uint16_t *)(b + 2));
        const int g = i >> 6, r = i & 63, sub = 2 * g + (r >> 5), l = r & 31;
        const uint8_t byte = b[16 + 32 * g + l];
        const int q = (r < 32) ? (byte & 0x0F) : (byte >> 4);
        int sc, m;
        q4k_scale_min(sub, b + 4, sc, m);
        const float d1 = d * (float)sc;
        const float m1 = dmin * (float)m;
        return d1 * (float)q - m1;
    } else if (type == DFX_TYPE_Q6_K) {
        const uint8_t * b = row + sb * SB_Q6_K;
        const float d = h2f(*(const uint16_t *)(b + 208));
        const int half = i >> 7, r = i & 127, quarter = r >> 5, l = r & 31;
        const uint8_t lo = b[64 * half + l + 32 * (quarter & 1)];
        const int low4 = (quarter < 2) ? (lo & 0x0F) : (lo >> 4);
        const int hi2 = (b[128 + 32 * half + l] >> (2 * quarter)) & 3;
        const int q = (low4 | (hi2 << 4)) - 32;
        const float sc = (float)(int8_t)b[192 + (i >> 4)];
        return (d * sc) * (float)q;
    } else if (type == DFX_TYPE_Q8_0) {
        const uint8_t * b = row + sb * SB_Q8_0;
        const float d = h2f(*(const uint16_t *)(b + 2 * (i >> 5)));
        return (float)(int8_t)b[16 + i] * d;
    } else if (type == DFX_TYPE_F32) {
        return *(const float *)(row + e * 4);
    } else {  // F16
        return h2f(*(const uint16_t *)(row + e * 2));
    }
}

__device__ __forceinline__ int64_t dev_row_bytes(int type, int64_t n) {
    const int64_t nsb = n >> 8;
    switch (type) {
        case DFX_TYPE_Q4_K: return nsb * SB_Q4_K;
        case DFX_TYPE_Q6_K: return nsb * SB_Q6_K;
        case DFX_TYPE_Q8_0: return nsb * SB_Q8_0;
        case DFX_TYPE_F32: return n * 4;
        default: return n * 2;
    }
}

__global__ void k_dequant(int type, const uint8_t * w, int64_t n_rows, int64_t n_cols, float * out) {
    const int64_t total = n_rows * n_cols;
    const int64_t rb = dev_row_bytes(type, n_cols);
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = idx / n_cols, e = idx - r * n_cols;
        out[idx] = dequant_elem(type, w + r * rb, e);
    }
}

__global__ void k_embed(int type, const uint8_t * table, int64_t n_embd, const int32_t * tokens,
                        int64_t M, float * x) {
    const int64_t total = M * n_embd;
    const int64_t rb = dev_row_bytes(type, n_embd);
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t m = idx / n_embd, e = idx - m * n_embd;
        x[idx] = dequant_elem(type, table + (int64_t)tokens[m] * rb, e);
    }
}

// ---------------------------------------------------------------------------
// Conversion of one 256-element block held by a wave (lane owns elements
// 4*lane .. 4*lane+3) into the activation buffer (layout in dfx_device.h).
// ---------------------------------------------------------------------------
__device__ __forceinline__ void store_q4(uint16_t * dst, const uint16_t o[4]) {
    const uint64_t packed = (uint64_t)o[0] | ((uint64_t)o[1] << 16) | ((uint64_t)o[2] << 32) | ((uint64_t)o[3] << 48);
    *(uint64_t *)dst = packed;
}

// Lane-to-lane moves inside rows of 16 lanes (DPP: no LDS round trip).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
#define DPP_QUAD_1032 0xB1   // quad_perm [1, 0, 3, 2]: lane ^ 1
#define DPP_QUAD_2301 0x4E   // quad_perm [2, 3, 0, 1]: lane ^ 2
#define DPP_ROW_HALF_MIRROR 0x141
#define DPP_ROW_MIRROR 0x140

// row m, block b (256 elements) of a [M][K] activation
__device__ __forceinline__ void convert_block256(const float v[4], int lane, int mode, uint8_t * act,
                                                 const act_layout & Lay, int64_t m, int64_t K, int64_t b) {
#pragma clang fp contract(off)
    if (mode == CONV_F32) {   // F32 weights: the activations go in unchanged
        *(float4 *)((float *)(act + Lay.q) + m * K + b * 256 + 4 * lane) = make_float4(v[0], v[1], v[2], v[3]);
        return;
    }
    uint16_t * q = (uint16_t *)(act + Lay.q) + m * K + b * 256 + 4 * lane;
    uint16_t o[4];
    if (conv_is_q8k(mode)) {
        // GGML quantize_row_q8_K_ref: max = the signed value of the first element
        // with the largest |x|; iscale = -127/max; q = min(127, nearest_int(iscale*x));
        // d = 1/iscale; bsums over 16.  All-zero block -> d = 0, q = 0.
        // amax = the largest |x| over the block (a NaN never compares greater, as in the
        // reference's |x| > amax scan: it counts as 0); max = the element with the lowest
        // index among those with |x| = amax: the lowest lane holding one (ballot), its lowest j
        uint32_t ab[4];
        float a4 = 0.0f;
        for (int j = 0; j < 4; j++) {
            ab[j] = __float_as_uint(v[j]) & 0x7fffffffu;
            if (ab[j] > 0x7f800000u) ab[j] = 0u;
            a4 = fmaxf(a4, __uint_as_float(ab[j]));
        }
        const float amax = wave_max(a4);
        const uint32_t amax_bits = __float_as_uint(amax);
        bool has = false;
        int sign = 0;
        for (int j = 3; j >= 0; j--)
            if (ab[j] == amax_bits) {
                has = true;
                sign = (int)(__float_as_uint(v[j]) >> 31);
            }
        const int first = __builtin_ctzll(__ballot(has));   // amax is some element's |x|: has holds somewhere
        const float mx = __builtin_amdgcn_readlane(sign, first) ? -amax : amax;
        int qi[4] = {0, 0, 0, 0};
        float d = 0.0f;
        if (amax != 0.0f) {
            // correctly rounded f32 divisions (the compiler's IEEE division)
            const float iscale = -127.0f / mx;
            d = 1.0f / iscale;
            for (int j = 0; j < 4; j++) qi[j] = min((int)__builtin_rintf(iscale * v[j]), 127);
        }
        for (int j = 0; j < 4; j++) o[j] = f2h((float)qi[j]);
        if (mode == CONV_Q8_K_P4) {
            // elements 4L..4L+3 of a 64-group (L = lane % 16) go to slots 8(L%8) + 4(L/8) + {0,2,1,3}
            const int L = lane & 15;
            const uint16_t p[4] = {o[0], o[2], o[1], o[3]};
            const int64_t sl = b * 256 + 64 * (lane >> 4) + 8 * (L & 7) + 4 * (L >> 3);
            store_q4((uint16_t *)(act + Lay.q) + act_frag_off(m, sl, K), p);
        } else if (mode == CONV_Q8_K_P6) {
            // elements 4L..4L+3 (L = lane): half h = L/32, quarter q = (L/8)%4, l = 4(L%8);
            // slot 64g + 8(i + 4(q%2)) + 4(q/2) + {0,2,1,3} with g = l/16, i = (l%16)/4
            const int h = lane >> 5, q = (lane >> 3) & 3, l = 4 * (lane & 7), g = l >> 4, i = (l & 15) >> 2;
            const uint16_t p[4] = {o[0], o[2], o[1], o[3]};
            const int64_t sl = b * 256 + 128 * h + 64 * g + 8 * (i + 4 * (q & 1)) + 4 * (q >> 1);
            store_q4((uint16_t *)(act + Lay.q) + act_frag_off(m, sl, K), p);
        } else {
            store_q4(q, o);
        }
        if (Lay.i8) {   // natural-order int8 copy for the matrix-vector kernels
            const uint32_t w = (uint32_t)(qi[0] & 0xFF) | ((uint32_t)(qi[1] & 0xFF) << 8) |
                               ((uint32_t)(qi[2] & 0xFF) << 16) | ((uint32_t)(qi[3] & 0xFF) << 24);
            *(uint32_t *)(act + Lay.i8 + m * K + b * 256 + 4 * lane) = w;
        }
        int s = qi[0] + qi[1] + qi[2] + qi[3];
        s += dpp_i<DPP_QUAD_1032>(s);
        s += dpp_i<DPP_QUAD_2301>(s);
        if ((lane & 3) == 0) ((uint16_t *)(act + Lay.bs))[m * (K / 16) + b * 16 + (lane >> 2)] = f2h((float)s);
        if (lane == 0) ((float *)(act + Lay.d))[conv_is_frag(mode) ? b * Lay.mq + m : m * (K / 256) + b] = d;
    } else if (mode == CONV_Q8_0) {
        // GGML quantize_row_q8_0_ref over 32-element blocks (8 lanes each):
        // d = amax/127, q = roundf(x * (1/d)), stored d rounded to f16.
        float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
        // over the block's 8 lanes (a half row of 16): lane ^ 1, lane ^ 2, then the mirrored quad
        amax = fmaxf(amax, dpp_f<DPP_QUAD_1032>(amax));
        amax = fmaxf(amax, dpp_f<DPP_QUAD_2301>(amax));
        amax = fmaxf(amax, dpp_f<DPP_ROW_HALF_MIRROR>(amax));
        const float d = (float)((double)amax / 127.0);
        const float id = d != 0.0f ? (float)(1.0 / (double)d) : 0.0f;
        for (int j = 0; j < 4; j++) o[j] = f2h((float)(int)roundf(v[j] * id));
        store_q4(q, o);
        if ((lane & 7) == 0) ((float *)(act + Lay.d))[m * (K / 32) + b * 8 + (lane >> 3)] = h2f(f2h(d));
    } else {
        for (int j = 0; j < 4; j++) o[j] = f2h(v[j]);
        store_q4(q, o);
    }
}

// One wave per (row, 256-block); a workgroup's eight waves take eight consecutive rows of one
// block, so that in the matrix-core operand order (rows 16 bytes apart within an operand) the
// workgroup's stores fill whole 128-byte lines instead of 16 bytes of each.
#define AC_ROWS 8
__global__ void __launch_bounds__(64 * AC_ROWS) k_act_convert(int mode, const float * x, int64_t M, int64_t K,
                                                              uint8_t * act) {
    const int lane = threadIdx.x & 63;
    const int64_t n_rg = (M + AC_ROWS - 1) / AC_ROWS;
    const int64_t b = blockIdx.x / n_rg, m = AC_ROWS * (blockIdx.x - b * n_rg) + (threadIdx.x >> 6);
    if (m >= M) return;
    const act_layout Lay = act_layout_of(mode, M, K);
    const float4 t = *(const float4 *)(x + m * K + b * 256 + 4 * lane);
    const float v[4] = {t.x, t.y, t.z, t.w};
    convert_block256(v, lane, mode, act, Lay, m, K, b);
}

// RMSNorm + weight + conversion; one workgroup of up to 16 waves per row.  Wave wv
// owns the BPW consecutive 256-element blocks from wv*BPW; x and w are loaded once,
// before the row reduction, and kept in registers for the scaling pass (with 8 blocks per
// wave, rows above 16384, w is read in the scaling pass instead: 16 waves of 1024 threads
// leave 128 registers per lane, which x and w of 8 blocks together would overflow).
// GGML ggml_compute_forward_rms_norm_f32: sum += (double)(x*x); mean = (float)(sum/K);
// scale = 1.0f/sqrtf(mean + eps); y = x*scale; then ggml_mul by w.
// Output row m normalises input row r = xmap[m] (or m).  With n_part > 0 the row is first
// completed with a deferred split-K result, exactly as the GEMM's own reduction would:
// x[r] = ((0 + part[0][r]) + part[1][r] + ...) + x[r], written back to x.
template <int BPW>
__global__ void __launch_bounds__(1024) k_rmsnorm_convert(int mode, float * x, const int32_t * xmap,
                                                          const float * w, int64_t M, int64_t K, float eps,
                                                          uint8_t * act, const float * part, int n_part,
                                                          int64_t part_stride) {
#pragma clang fp contract(off)
    __shared__ double red[16];
    // Rows 64a + 8x .. 64a + 8x + 7 go to workgroups on XCD x (workgroup g runs on XCD g % 8):
    // the eight rows whose operand-order activations share 128-byte lines are written through
    // one L2 (a placement only: every row's arithmetic is its own).
    const int64_t wg = blockIdx.x, m = 64 * (wg >> 6) + 8 * (wg & 7) + ((wg >> 3) & 7);
    if (m >= M) return;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, nw = blockDim.x >> 6;
    const int nb = (int)(K >> 8);
    const int64_t r = xmap ? xmap[m] : m;
    float * xr = x + r * K;
    constexpr bool KEEP_W = BPW < 8;
    float4 t[BPW], g[KEEP_W ? BPW : 1];
#pragma unroll
    for (int j = 0; j < BPW; j++) {
        const int b = min(wv * BPW + j, nb - 1);   // clamped: the duplicate is not summed or stored
        t[j] = *(const float4 *)(xr + (int64_t)b * 256 + 4 * lane);
        if constexpr (KEEP_W) g[j] = *(const float4 *)(w + (int64_t)b * 256 + 4 * lane);
    }
    if (n_part > 0) {
        const float * pr = part + r * K + 4 * lane;
#pragma unroll
        for (int j = 0; j < BPW; j++) {
            const int b = min(wv * BPW + j, nb - 1);
            float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            // four slices in flight at a time, added in slice order.  Loads past the last
            // slice read the last slice again and add +0 instead: v starts at +0 and so is
            // never -0, and v + 0 = v for every other v.
            for (int s0 = 0; s0 < n_part; s0 += 4) {
                float4v p[4];
#pragma unroll
                for (int u = 0; u < 4; u++)
                    p[u] = *(const float4v *)(pr + min(s0 + u, n_part - 1) * part_stride + (int64_t)b * 256);
                const float4v z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const float4v q = s0 + u < n_part ? p[u] : z;
                    v.x = v.x + q.x;
                    v.y = v.y + q.y;
                    v.z = v.z + q.z;
                    v.w = v.w + q.w;
                }
            }
            t[j] = make_float4(v.x + t[j].x, v.y + t[j].y, v.z + t[j].z, v.w + t[j].w);
            if (wv * BPW + j < nb) *(float4 *)(xr + (int64_t)b * 256 + 4 * lane) = t[j];
        }
    }
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < BPW; j++) {
        if (wv * BPW + j < nb) {
            s += (double)(t[j].x * t[j].x);
            s += (double)(t[j].y * t[j].y);
            s += (double)(t[j].z * t[j].z);
            s += (double)(t[j].w * t[j].w);
        }
    }
    s = wave_sum_d(s);
    if (lane == 0) red[wv] = s;
    __syncthreads();
    double tot = 0.0;
    for (int i = 0; i < nw; i++) tot += red[i];
    const float mean = (float)(tot / (double)K);
    // correctly rounded f32 sqrt and division (the compiler's IEEE forms)
    const float root = sqrtf(mean + eps);
    const float scale = 1.0f / root;
    const act_layout Lay = act_layout_of(mode, M, K);
#pragma unroll
    for (int j = 0; j < BPW; j++) {
        const int b = wv * BPW + j;
        if (b < nb) {
            const float4 gw = KEEP_W ? g[KEEP_W ? j : 0] : *(const float4 *)(w + (int64_t)b * 256 + 4 * lane);
            const float v[4] = {(t[j].x * scale) * gw.x, (t[j].y * scale) * gw.y, (t[j].z * scale) * gw.z,
                                (t[j].w * scale) * gw.w};
            convert_block256(v, lane, mode, act, Lay, m, K, b);
        }
    }
}

// silu(gate) * up, then conversion.  gu row m = [gate F | up F]; one wave per (row, block).
// GGML ggml_silu_f32: x / (1 + exp(-x)).
__global__ void k_swiglu_convert(int mode, const float * gu, int64_t M, int64_t F, uint8_t * act) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t wid = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int64_t nb = F >> 8;
    if (wid >= M * nb) return;
    const int64_t m = wid / nb, b = wid - m * nb;
    const int64_t k = b * 256 + 4 * lane;
    const float4 g = *(const float4 *)(gu + m * 2 * F + k);
    const float4 u = *(const float4 *)(gu + m * 2 * F + F + k);
    const float v[4] = {silu_mul(g.x, u.x), silu_mul(g.y, u.y), silu_mul(g.z, u.z), silu_mul(g.w, u.w)};
    const act_layout Lay = act_layout_of(mode, M, F);
    convert_block256(v, lane, mode, act, Lay, m, F, b);
}

// ---------------------------------------------------------------------------
// C ABI launch wrappers
// ---------------------------------------------------------------------------
// Weight storage types the GEMMs read (activation conversion follows them).
static bool dev_type_ok(int t) {
    return t == DFX_TYPE_Q4_K || t == DFX_TYPE_Q6_K || t == DFX_TYPE_Q8_0 || t == DFX_TYPE_F16 || t == DFX_TYPE_F32;
}
static bool table_type_ok(int t) { return dev_type_ok(t); }

extern "C" int dfx_dequant(int type, const void * w, int64_t n_rows, int64_t n_cols, float * out, void * stream) {
    if (!table_type_ok(type) || n_cols <= 0 || n_rows <= 0 || (n_cols & 255)) {
        dfx_set_error("dfx_dequant: unsupported type %d or shape %lldx%lld", type, (long long)n_rows, (long long)n_cols);
        return DFX_ERR_UNSUPPORTED;
    }
    const int64_t total = n_rows * n_cols;
    const int64_t blocks = std::min<int64_t>((total + 255) / 256, 65536);
    hipLaunchKernelGGL(k_dequant, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, type,
                       (const uint8_t *)w, n_rows, n_cols, out);
    DFX_CHECK_LAUNCH("dfx_dequant");
    return DFX_OK;
}

extern "C" int dfx_embed(int type, const void * table, int64_t n_embd, const int32_t * tokens, int64_t M,
                         float * x, void * stream) {
    if (!table_type_ok(type) || n_embd <= 0 || (n_embd & 255) || M < 0) {
        dfx_set_error("dfx_embed: unsupported type %d or n_embd %lld", type, (long long)n_embd);
        return DFX_ERR_UNSUPPORTED;
    }
    if (M == 0) return DFX_OK;
    const int64_t total = M * n_embd;
    const int64_t blocks = std::min<int64_t>((total + 255) / 256, 65536);
    hipLaunchKernelGGL(k_embed, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, type,
                       (const uint8_t *)table, n_embd, tokens, M, x);
    DFX_CHECK_LAUNCH("dfx_embed");
    return DFX_OK;
}

extern "C" size_t dfx_act_bytes(int wtype, int64_t M, int64_t K) {
    return act_layout_of(conv_mode(wtype), M, K).bytes;
}

extern "C" int dfx_act_convert(int wtype, const float * x, int64_t M, int64_t K, void * act, void * stream) {
    if (!dev_type_ok(wtype) || K <= 0 || (K & 255) || M < 0) {
        dfx_set_error("dfx_act_convert: unsupported type %d or K %lld", wtype, (long long)K);
        return DFX_ERR_UNSUPPORTED;
    }
    if (M == 0) return DFX_OK;
    const int64_t groups = (K >> 8) * ((M + AC_ROWS - 1) / AC_ROWS);
    hipLaunchKernelGGL(k_act_convert, dim3((unsigned)groups), dim3(64 * AC_ROWS), 0, (hipStream_t)stream,
                       conv_mode(wtype), x, M, K, (uint8_t *)act);
    DFX_CHECK_LAUNCH("dfx_act_convert");
    return DFX_OK;
}

static int rmsnorm_launch(int wtype, float * x, const int32_t * xmap, const float * w, int64_t M, int64_t K,
                          float eps, void * act, const float * part, int n_part, int64_t part_stride, void * stream) {
    if (!dev_type_ok(wtype) || K <= 0 || (K & 255) || M < 0) {
        dfx_set_error("dfx_rmsnorm_convert: unsupported type %d or K %lld", wtype, (long long)K);
        return DFX_ERR_UNSUPPORTED;
    }
    const int64_t nb = K >> 8;
    if (nb > 128) {
        dfx_set_error("dfx_rmsnorm_convert: K %lld above 32768", (long long)K);
        return DFX_ERR_UNSUPPORTED;
    }
    if (M == 0) return DFX_OK;
    // blocks per wave: the fewest that keep the row within 16 waves
    const int bpw = nb <= 16 ? 1 : nb <= 32 ? 2 : nb <= 64 ? 4 : 8;
    const dim3 block((unsigned)(64 * ((nb + bpw - 1) / bpw)));
    auto kern = bpw == 1 ? k_rmsnorm_convert<1> : bpw == 2 ? k_rmsnorm_convert<2>
              : bpw == 4 ? k_rmsnorm_convert<4> : k_rmsnorm_convert<8>;
    hipLaunchKernelGGL(kern, dim3((unsigned)((M + 63) / 64 * 64)), block, 0, (hipStream_t)stream, conv_mode(wtype), x,
                       xmap, w, M, K, eps, (uint8_t *)act, part, n_part, part_stride);
    DFX_CHECK_LAUNCH("dfx_rmsnorm_convert");
    return DFX_OK;
}

int dfx_rmsnorm_convert_ex(int wtype, const float * x, const int32_t * xmap, const float * w, int64_t M, int64_t K,
                           float eps, void * act, void * stream) {
    // x is only read when no partial sums are added
    return rmsnorm_launch(wtype, const_cast<float *>(x), xmap, w, M, K, eps, act, nullptr, 0, 0, stream);
}

int dfx_rmsnorm_convert_add(int wtype, float * x, const int32_t * xmap, const float * part, int n_part,
                            int64_t part_rows, const float * w, int64_t M, int64_t K, float eps, void * act,
                            void * stream) {
    if (n_part < 0 || (n_part > 0 && (!part || part_rows < 1))) {
        dfx_set_error("dfx_rmsnorm_convert_add: bad partial sums (%d slices)", n_part);
        return DFX_ERR_ARG;
    }
    return rmsnorm_launch(wtype, x, xmap, w, M, K, eps, act, part, n_part, part_rows * K, stream);
}

extern "C" int dfx_rmsnorm_convert(int wtype, const float * x, const float * w, int64_t M, int64_t K, float eps,
                                   void * act, void * stream) {
    return dfx_rmsnorm_convert_ex(wtype, x, nullptr, w, M, K, eps, act, stream);
}

extern "C" int dfx_swiglu_convert(int wtype, const float * gu, int64_t M, int64_t F, void * act, void * stream) {
    if (!dev_type_ok(wtype) || F <= 0 || (F & 255) || M < 0) {
        dfx_set_error("dfx_swiglu_convert: unsupported type %d or F %lld", wtype, (long long)F);
        return DFX_ERR_UNSUPPORTED;
    }
    if (M == 0) return DFX_OK;
    const int64_t waves = M * (F >> 8);
    hipLaunchKernelGGL(k_swiglu_convert, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, (hipStream_t)stream,
                       conv_mode(wtype), gu, M, F, (uint8_t *)act);
    DFX_CHECK_LAUNCH("dfx_swiglu_convert");
    return DFX_OK;
}
