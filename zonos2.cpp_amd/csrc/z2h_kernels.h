// z2h_kernels.h — gfx950 kernels of one ragged continuous-batching decode step.
//
// Kernel map (reference op -> kernel; src/zonos2-graph.cpp line numbers):
//   k_resnorm        embedding sum (248-260) / emb_norm (300) / residual folds (332, 345, 353) /
//                    rms_w norms (92-95, 343, 347, 354), and the encoding of the normalised row in
//                    the next matmul's activation type (ggml's vec_dot_type conversion)
//   k_gemv_split     dense m16 matmuls with K split over a block's waves: fused QKV + gate
//                    (107-111), W_o (175), output head + softcap (357-362), dense FFN (179-185)
//   k_gemv_mfma      grouped expert matmuls on the m16 layout (mul_mat_id 223-231, routes grouped by
//                    expert from the top-k selection): gate/up + SwiGLU in one launch, down x route
//                    weight
//   k_gemv / k_gemv_rows   the same on the 64-row tiled layout (Q6_K, F16)
//   k_swiglu_encode / k_encode_rows   up * silu(gate) (183, 225) / fp32 rows encoded for the next matmul
//   k_attn_chunk     decode steps: QK-RMSNorm, |temp|, interleaved RoPE, f16 KV append (113-137) and
//                    ragged GQA decode attention over the slot's band in 64-row chunks (139-153)
//   k_attn_combine   chunk merge, per-head sigmoid gate (107, 173), encoding for W_o
//   k_attn_fa / k_attn_merge   (z2h_attn.h) wide passes: the same attention on MFMA over 128-key
//                    segments for tiles of rows of one slot, segments merged in order
//   k_attn_tile_f32  the per-slot prefill's in-prompt fp32 attention (155-169), with k_attn_combine
//   k_router_down    EDA router down-projection + state threading (199-203)
//   k_router_tail    router norm, erf-GELU MLP, softmax, bias, mask, top-k, weights (206-220)
//   k_kv_move / k_bias_add   KV row staging for host reads and writes / speaker-projection biases
//   k_kv_append      K/V rows of every token of a wide pass, before the pass's attention
//   k_sample         frame sampler (src/zonos2-sampler.cpp:16-77) on the step's logits
//
// Weight layouts in HBM: "m16" for Q4_K and Q8_0 (see k_gemv_mfma) and "row-tiled" (t64) for Q6_K
// and F16: a matrix of R rows x K columns is cut into 64-row tiles and 256-column units; the bytes
// of unit (row, u) are split into 16-byte chunks and chunk c of the 64 rows of a tile is stored
// contiguously, so every lane of a wave64 owns one row and each load instruction of the wave reads
// 1 KiB of contiguous HBM. Unit sizes equal the GGUF storage sizes: Q4_K 144 B = 9 chunks, Q8_0 8
// blocks = 17 chunks (16 of values, 1 of the 8 f16 scales), Q6_K 208 B = 13 chunks + an f16 d
// plane, F16 512 B = 32 chunks.
#pragma once
#include "z2h_common.h"
#include "z2h_stdorder.h"
#include <type_traits>

// Z2H_TEMPLATES_ONLY (defined by a second translation unit that only instantiates kernel templates):
// the non-template kernels below are left out there, so the library defines each of them once.

namespace z2d {

enum { WF_F16 = 1, WF_Q8_0 = 8, WF_Q4_K = 12, WF_Q6_K = 14 };
enum { ACT_NONE = -1, ACT_F16 = 1, ACT_Q8_0 = 8, ACT_Q8_K = 15 };

constexpr int NT = 16;          // tokens (or routes) per GEMV pass
constexpr int TILE = 64;        // rows per tile = lanes per wave
constexpr int ATT_CH = 64;      // attention rows per chunk (<= 64)

template <int WF> struct wfmt;
template <> struct wfmt<WF_Q4_K> { static constexpr int C = 9;  static constexpr int ACT = ACT_Q8_K; };
template <> struct wfmt<WF_Q6_K> { static constexpr int C = 13; static constexpr int ACT = ACT_Q8_K; };
template <> struct wfmt<WF_Q8_0> { static constexpr int C = 17; static constexpr int ACT = ACT_Q8_0; };
template <> struct wfmt<WF_F16>  { static constexpr int C = 32; static constexpr int ACT = ACT_F16; };

// Encoded activation rows [T][K] in global memory (planes used depend on the encoding).
struct ActBuf {
    int8_t * q;       // [T][K]     Q8_0 / Q8_K values
    float * d32;      // [T][K/32]  Q8_0 scale (f16-rounded)
    float * d256;     // [T][K/256] Q8_K scale
    int16_t * bs;     // [T][K/16]  Q8_K sums of 16
    uint16_t * h;     // [T][K]     f16
};

// ------------------------------------------------------------------ activation encoders
// Q8_K of one 256-block by one wave (4 elements per lane). The element of largest |x| (first
// occurrence) fixes iscale = -127/x; q = min(127, rint(iscale*x)); d = 1/iscale; sums of 16.
// q8k_quant_m: the block's values (qi, 4 per lane) and its scale d (the same in every lane), given
// the block's largest |x| (amax, from a wave max).
__device__ __forceinline__ float q8k_quant_m(const float (&v)[4], float amax, int (&qi)[4]) {
    if (amax == 0.0f) {
#pragma unroll
        for (int i = 0; i < 4; ++i) qi[i] = 0;
        return 0.0f;
    }
    // the first occurrence (lowest element index lane*4+i) of the largest |x| from ballots
    int best = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint64_t m = __ballot(fabsf(v[i]) == amax);
        if (m) best = min(best, (int) (__ffsll((unsigned long long) m) - 1) * 4 + i);
    }
    const int bi = best & 3;
    const float vb = bi == 0 ? v[0] : bi == 1 ? v[1] : bi == 2 ? v[2] : v[3];
    const float bval = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, vb), best >> 2));
    const float iscale = -127.0f / bval;
#pragma unroll
    for (int i = 0; i < 4; ++i) qi[i] = min(127, (int) rintf(iscale * v[i]));
    return 1.0f / iscale;
}
__device__ __forceinline__ float q8k_lmax(const float (&v)[4]) {
    return fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
}
__device__ __forceinline__ float q8k_quant(const float (&v)[4], int (&qi)[4]) {
    return q8k_quant_m(v, wave_max_f(q8k_lmax(v)), qi);
}
__device__ __forceinline__ void q8k_block_v(const float (&v)[4], int8_t * q, float * d, int16_t * bs, int lane) {
    int qi[4];
    const float dd = q8k_quant(v, qi);
    if (lane == 0) *d = dd;
    const uint32_t packed = (uint32_t) (qi[0] & 255) | ((uint32_t) (qi[1] & 255) << 8) |
                            ((uint32_t) (qi[2] & 255) << 16) | ((uint32_t) (qi[3] & 255) << 24);
    *(uint32_t *) (q + lane * 4) = packed;
    int s = qi[0] + qi[1] + qi[2] + qi[3];
    s += dpp_i<DPP_QUAD_XOR1>(s);                  // sum of the 4 lanes of a quad = 16 elements
    s += dpp_i<DPP_QUAD_XOR2>(s);
    if ((lane & 3) == 0) bs[lane >> 2] = (int16_t) s;
}

// Two independent 256-blocks by one wave: q8k_block_v on each, written as one straight-line
// sequence so the two max / ballot / scale chains interleave.
__device__ __forceinline__ void q8k_block_v2(const float (&va)[4], const float (&vb)[4], int8_t * qa, int8_t * qb,
                                             float * da, float * db, int16_t * bsa, int16_t * bsb, int lane) {
    int qia[4], qib[4];
    const float ma = wave_max_f(q8k_lmax(va)), mb = wave_max_f(q8k_lmax(vb));
    const float dda = q8k_quant_m(va, ma, qia), ddb = q8k_quant_m(vb, mb, qib);
    if (lane == 0) { *da = dda; *db = ddb; }
    *(uint32_t *) (qa + lane * 4) = (uint32_t) (qia[0] & 255) | ((uint32_t) (qia[1] & 255) << 8) | ((uint32_t) (qia[2] & 255) << 16) | ((uint32_t) (qia[3] & 255) << 24);
    *(uint32_t *) (qb + lane * 4) = (uint32_t) (qib[0] & 255) | ((uint32_t) (qib[1] & 255) << 8) | ((uint32_t) (qib[2] & 255) << 16) | ((uint32_t) (qib[3] & 255) << 24);
    int sa = qia[0] + qia[1] + qia[2] + qia[3], sb = qib[0] + qib[1] + qib[2] + qib[3];
    sa += dpp_i<DPP_QUAD_XOR1>(sa); sb += dpp_i<DPP_QUAD_XOR1>(sb);
    sa += dpp_i<DPP_QUAD_XOR2>(sa); sb += dpp_i<DPP_QUAD_XOR2>(sb);
    if ((lane & 3) == 0) { bsa[lane >> 2] = (int16_t) sa; bsb[lane >> 2] = (int16_t) sb; }
}

// Encode one row x[K] (any memory) by a 256-thread block into the given destination planes.
// x must hold Kp = round_up(K, 256) readable entries for Q8_K (callers keep K % 256 == 0 there);
// for Q8_0 / F16 the entries in [K, Kp) are encoded as zeros.
template <int AF>
__device__ __forceinline__ void encode_row(const float * x, int K, int8_t * q, float * d32, float * d256,
                                           int16_t * bs, uint16_t * h) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int Kp = (K + 255) & ~255;
    if constexpr (AF == ACT_Q8_K) {
        // two blocks per wave and pass (b and b + 4), so their reductions overlap
        const int nb = K / 256;
        for (int b = wave; b < nb; b += 8) {
            const float v0[4] = {x[256 * b + lane * 4], x[256 * b + lane * 4 + 1], x[256 * b + lane * 4 + 2], x[256 * b + lane * 4 + 3]};
            if (b + 4 < nb) {
                const int b1 = b + 4;
                const float v1[4] = {x[256 * b1 + lane * 4], x[256 * b1 + lane * 4 + 1], x[256 * b1 + lane * 4 + 2], x[256 * b1 + lane * 4 + 3]};
                q8k_block_v2(v0, v1, q + 256 * b, q + 256 * b1, d256 + b, d256 + b1, bs + 16 * b, bs + 16 * b1, lane);
            } else {
                q8k_block_v(v0, q + 256 * b, d256 + b, bs + 16 * b, lane);
            }
        }
    } else if constexpr (AF == ACT_Q8_0) {
        for (int i = tid; i < Kp; i += 256) {         // 64 lanes = two 32-blocks
            const float v = i < K ? x[i] : 0.0f;
            const float amax = max32_f(fabsf(v));
            const float dd = amax / 127.0f, id = amax != 0.0f ? 127.0f / amax : 0.0f;
            q[i] = (int8_t) (int) rintf(v * id);
            if ((i & 31) == 0) d32[i >> 5] = h2f(f2h(dd));
        }
    } else if constexpr (AF == ACT_F16) {
        for (int i = tid; i < Kp; i += 256) h[i] = i < K ? f2h(x[i]) : (uint16_t) 0;
    }
}

__host__ __device__ inline int kpad(int K) { return (K + 255) & ~255; }

// Row t of an ActBuf uses the padded length Kp as its stride.
__device__ __forceinline__ void encode_row_rt(int af, const float * x, int K, const ActBuf & a, int t) {
    const int Kp = kpad(K);
    if (af == ACT_Q8_K) encode_row<ACT_Q8_K>(x, K, a.q + (int64_t) t * Kp, nullptr, a.d256 + (int64_t) t * (Kp / 256), a.bs + (int64_t) t * (Kp / 16), nullptr);
    else if (af == ACT_Q8_0) encode_row<ACT_Q8_0>(x, K, a.q + (int64_t) t * Kp, a.d32 + (int64_t) t * (Kp / 32), nullptr, nullptr, nullptr);
    else if (af == ACT_F16) encode_row<ACT_F16>(x, K, nullptr, nullptr, nullptr, nullptr, a.h + (int64_t) t * Kp);
}

// Q8_K of a row that a 256-thread block holds in registers the norm kernels' way (thread tid owns
// elements 4 (tid + 256 j) .. + 3, so wave w holds 256-blocks w + 4j in q8k lane order): the blocks
// are encoded in place, in encode_row's pairs (w + 8m, w + 8m + 4), with no LDS round trip.
// Needs K % 1024 == 0 and K <= 1024 NV.
template <int NV>
__device__ __forceinline__ void encode_q8k_regs(const float4 (&xv)[NV], int K, const ActBuf & a, int t) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, Kp = kpad(K), nj = K / 1024;
    int8_t * q = a.q + (int64_t) t * Kp;
    float * d256 = a.d256 + (int64_t) t * (Kp / 256);
    int16_t * bs = a.bs + (int64_t) t * (Kp / 16);
#pragma unroll
    for (int j = 0; j < NV; j += 2) {
        if (j >= nj) break;
        const int b = wave + 4 * j;
        const float v0[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
        if (j + 1 < nj) {
            const int b1 = b + 4;
            const float v1[4] = {xv[j + 1].x, xv[j + 1].y, xv[j + 1].z, xv[j + 1].w};
            q8k_block_v2(v0, v1, q + 256 * b, q + 256 * b1, d256 + b, d256 + b1, bs + 16 * b, bs + 16 * b1, lane);
        } else {
            q8k_block_v(v0, q + 256 * b, d256 + b, bs + 16 * b, lane);
        }
    }
}

// Q8_0 of a row held in registers the norm kernels' way (thread tid owns elements 4 (tid + 256 j) ..
// + 3, so a 32-element block is 8 consecutive lanes): the block's largest |x| over those lanes by DPP
// (xor 1, xor 2 within quads, then the mirrored quad), then encode_row<ACT_Q8_0>'s arithmetic
// (d = amax / 127, q = rint(x * (127 / amax)), the scale stored as f16(d)). Needs K % 1024 == 0 and
// K <= 1024 NV.
template <int NV>
__device__ __forceinline__ void encode_q80_regs(const float4 (&xv)[NV], int K, const ActBuf & a, int t) {
    const int tid = threadIdx.x, Kp = kpad(K), nj = K / 1024;
    int8_t * q = a.q + (int64_t) t * Kp;
    float * d32 = a.d32 + (int64_t) t * (Kp / 32);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        if (j >= nj) break;
        const float4 v = xv[j];
        const float m = max8_f(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        const float dd = m / 127.0f, id = m != 0.0f ? 127.0f / m : 0.0f;
        const int e = tid + 256 * j;                                  // the thread's 4-element group
        const int q0 = (int) rintf(v.x * id), q1 = (int) rintf(v.y * id), q2 = (int) rintf(v.z * id), q3 = (int) rintf(v.w * id);
        *(uint32_t *) (q + 4 * e) = (uint32_t) (q0 & 255) | ((uint32_t) (q1 & 255) << 8) | ((uint32_t) (q2 & 255) << 16) |
                                    ((uint32_t) (q3 & 255) << 24);
        if ((tid & 7) == 0) d32[e >> 3] = h2f(f2h(dd));
    }
}

// Block-wide copy of n 16-byte items with all loads of a batch issued before its stores (a loop
// that loads and stores per iteration is not software-pipelined and pays one memory round trip per
// iteration). src(i) / dst(i) give the item addresses.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
template <int NTH, class Src, class Dst>
__device__ __forceinline__ void copy16(int n, Src src, Dst dst) {
    constexpr int B = 8;
    for (int base = 0; base < n; base += NTH * B) {
        u32x4 v0, v1, v2, v3, v4, v5, v6, v7;
        const int i0 = base + threadIdx.x;
#define C16_LD(J) if (i0 + NTH * J < n) v##J = *(const u32x4 *) src(i0 + NTH * J);
#define C16_ST(J) if (i0 + NTH * J < n) *(u32x4 *) dst(i0 + NTH * J) = v##J;
        C16_LD(0) C16_LD(1) C16_LD(2) C16_LD(3) C16_LD(4) C16_LD(5) C16_LD(6) C16_LD(7)
        C16_ST(0) C16_ST(1) C16_ST(2) C16_ST(3) C16_ST(4) C16_ST(5) C16_ST(6) C16_ST(7)
#undef C16_LD
#undef C16_ST
        static_assert(B == 8, "copy16 batch");
    }
}

// block-wide double sum (256 threads)
__device__ __forceinline__ double block_sum_d(double v, double * red) {
    v = wave_tree_d(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    lds_sync();                               // earlier readers of red are done
    if (lane == 0) red[wave] = v;
    lds_sync();
    return red[0] + red[1] + red[2] + red[3];
}

// y[i] = y[i] + b[i] (+ c[i]): the bias adds after the speaker projections (graph.cpp:272-278)
#ifndef Z2H_TEMPLATES_ONLY
__global__ void __launch_bounds__(256) k_bias_add(float * y, const float * b, const float * c, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float v = y[i] + b[i];
    if (c) v = v + c[i];
    y[i] = v;
}
#endif

// ------------------------------------------------------------------ dequantised table rows
__device__ __forceinline__ float table_elem(const uint8_t * row, int type, int i) {
    switch (type) {
        case 0: return ((const float *) row)[i];
        case 1: return h2f(((const uint16_t *) row)[i]);
        case 8: {
            const uint8_t * b = row + 34 * (i >> 5);
            return (float) (int8_t) b[2 + (i & 31)] * h2f(*(const uint16_t *) b);
        }
        case 12: {
            const uint8_t * b = row + 144 * (i >> 8);
            const int w = i & 255, j = w >> 5, p = j >> 1, l = w & 31;
            int s, m; q4k_sm(b + 4, j, s, m);
            const uint8_t qb = b[16 + 32 * p + l];
            const int qv = (j & 1) ? (qb >> 4) : (qb & 15);
            const float d = h2f(*(const uint16_t *) b), dmin = h2f(*(const uint16_t *) (b + 2));
            return (d * (float) s) * (float) qv - dmin * (float) m;
        }
        case 14: {
            const uint8_t * b = row + 210 * (i >> 8);
            const int w = i & 255, h = w >> 7, r = w & 127, m = r >> 5, l = r & 31;
            const uint8_t * ql = b + 64 * h, * qh = b + 128 + 32 * h;
            const int lo = (m & 1) ? ql[l + 32] : ql[l];
            const int nib = (m >= 2) ? (lo >> 4) : (lo & 15);
            const int q = (nib | (((qh[l] >> (2 * m)) & 3) << 4)) - 32;
            const float d = h2f(*(const uint16_t *) (b + 208));
            return d * (float) ((const int8_t *) (b + 192))[8 * h + l / 16 + 2 * m] * (float) q;
        }
    }
    return 0.0f;
}

__device__ __forceinline__ int64_t table_row_bytes(int type, int d) {
    switch (type) { case 0: return 4ll * d; case 1: return 2ll * d; case 8: return (int64_t) d / 32 * 34;
                    case 12: return (int64_t) d / 256 * 144; case 14: return (int64_t) d / 256 * 210; }
    return 0;
}

// ------------------------------------------------------------------ k_resnorm
enum { RN_EMBED = 0, RN_ACCUM = 1, RN_ADD = 2, RN_ENCODE = 3 };
constexpr int MAX_TABLES = 16;

struct ResNormArgs {
    int mode, d;
    const int32_t * ids; int W;
    const float * emb_in;              // injected rows: [T][d], or rows picked by emb_map
    const int32_t * emb_map;           // [T]: -1 = token t sums its ids, else its row of emb_in (NULL: row t)
    const uint8_t * tab[MAX_TABLES]; int tab_type[MAX_TABLES]; int64_t tab_rows[MAX_TABLES];
    const float * src; int k;         // ACCUM: [T*k][d] routes; ADD / ENCODE: [T][d]
    float * res;                       // [T][d] (ACCUM may pass null: no residual)
    const float * res_in;              // ACCUM / ADD: residual read from here instead of res (null: res)
    const float * norm_w; float eps;
    float * cur_out;                   // [T][d] fp32 normalised row (nullable)
    ActBuf act; int act_fmt;
    float * cap_x;                     // [T][d] folded FFN output (nullable)
    int * err;
};

// 4 consecutive elements of a dequantised table row (i0 % 4 == 0)
__device__ __forceinline__ float4 table_elem4(const uint8_t * row, int type, int i0) {
    switch (type) {
        case 0: return *(const float4 *) (row + 4 * (int64_t) i0);
        case 1: {
            const uint2 h = *(const uint2 *) (row + 2 * (int64_t) i0);
            return make_float4(h2f(h.x & 0xffffu), h2f(h.x >> 16), h2f(h.y & 0xffffu), h2f(h.y >> 16));
        }
        case 8: {
            const uint8_t * b = row + 34 * (i0 >> 5);
            const float dd = h2f(*(const uint16_t *) b);
            const uint8_t * qv = b + 2 + (i0 & 31);
            return make_float4((float) (int8_t) qv[0] * dd, (float) (int8_t) qv[1] * dd, (float) (int8_t) qv[2] * dd, (float) (int8_t) qv[3] * dd);
        }
    }
    return make_float4(table_elem(row, type, i0), table_elem(row, type, i0 + 1), table_elem(row, type, i0 + 2), table_elem(row, type, i0 + 3));
}

// table_elem4 for a table type known at compile time (F32 / F16 / Q8_0), with no type switch
template <int TT>
__device__ __forceinline__ float4 table_elem4_t(const uint8_t * row, int i0) {
    if constexpr (TT == 0) {
        return *(const float4 *) (row + 4 * (int64_t) i0);
    } else if constexpr (TT == 1) {
        const uint2 h = *(const uint2 *) (row + 2 * (int64_t) i0);
        return make_float4(h2f(h.x & 0xffffu), h2f(h.x >> 16), h2f(h.y & 0xffffu), h2f(h.y >> 16));
    } else {
        static_assert(TT == 8, "F32, F16 or Q8_0 tables");
        const uint8_t * b = row + 34 * (i0 >> 5);
        const float dd = h2f(*(const uint16_t *) b);
        const uint8_t * qv = b + 2 + (i0 & 31);
        return make_float4((float) (int8_t) qv[0] * dd, (float) (int8_t) qv[1] * dd, (float) (int8_t) qv[2] * dd, (float) (int8_t) qv[3] * dd);
    }
}

// One block per token; thread tid owns elements 4*(tid + 256*j) .. +3 (d % 4 == 0, d <= 4096). Every
// global read the block needs (norm weight, routes, residual, embedding rows) is issued before the
// first reduction and before the first store (a store between loads would order them: the
// compiler cannot tell the residual row from the sources), and every global store comes after the
// last barrier (a barrier waits for the block's outstanding stores). One instantiation per mode
// keeps each kernel's code to its own path. TT >= 0 (RN_EMBED): every table has GGUF type TT, and the
// token's table rows are read with no type switch: all tables' loads of an element group go out
// together (TW table slots, W <= TW; slots past W re-read the last table and are not added), the sum
// keeps the table order.
constexpr int RN_NV = 4;
template <int MODE, int TT = -1, int TW = MAX_TABLES>
__global__ void __launch_bounds__(256) k_resnorm(ResNormArgs a) {
    extern __shared__ float sm_rn[];
    float * xs = sm_rn;                // [d]
    __shared__ double red[4];
    const int t = blockIdx.x, d = a.d, tid = threadIdx.x;
    float * res = a.res ? a.res + (int64_t) t * d : nullptr;
    float4 nw[RN_NV], xv[RN_NV];
    float4 res_out[RN_NV], cap_out[RN_NV];          // stored at the end
    bool st_res = false, st_cap = false;
#pragma unroll
    for (int j = 0; j < RN_NV; ++j) {
        const int i0 = 4 * (tid + 256 * j);
        if (a.norm_w && i0 < d) nw[j] = *(const float4 *) (a.norm_w + i0);
    }
    auto add4 = [](float4 x, float4 y) { return make_float4(x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w); };
    if constexpr (MODE == RN_EMBED) {
        const int erow = a.emb_in ? (a.emb_map ? a.emb_map[t] : t) : -1;
        if (erow >= 0) {
            const float * er = a.emb_in + (int64_t) erow * d;
#pragma unroll
            for (int j = 0; j < RN_NV; ++j) {
                const int i0 = 4 * (tid + 256 * j);
                if (i0 < d) xv[j] = *(const float4 *) (er + i0);
            }
        } else if constexpr (TT >= 0) {
            const uint8_t * rows[TW];
            const int64_t rb = table_row_bytes(TT, d);
            int ids[TW];                                           // every id read before any flag write
#pragma unroll
            for (int kk = 0; kk < TW; ++kk) ids[kk] = a.ids[(int64_t) t * a.W + min(kk, a.W - 1)];
            bool bad = false;
#pragma unroll
            for (int kk = 0; kk < TW; ++kk) {
                const int kc = min(kk, a.W - 1);
                const bool ok = ids[kk] >= 0 && ids[kk] < a.tab_rows[kc];
                bad = bad || !ok;
                rows[kk] = a.tab[kc] + (int64_t) (ok ? ids[kk] : 0) * rb;
            }
            if (bad && tid == 0) atomicOr(a.err, 1);
#pragma unroll
            for (int j = 0; j < RN_NV; ++j) {
                if (1024 * j >= d) break;                          // (uniform) groups past the row
                const int i0 = min(4 * (tid + 256 * j), d - 4);
                float4 e[TW];
#pragma unroll
                for (int kk = 0; kk < TW; ++kk) e[kk] = table_elem4_t<TT>(rows[kk], i0);
                __builtin_amdgcn_sched_barrier(0);                 // every load of the group issues first
                float4 x = e[0];
#pragma unroll
                for (int kk = 1; kk < TW; ++kk) {
                    const float4 y = add4(x, e[kk]);
                    x = kk < a.W ? y : x;
                }
                xv[j] = x;
            }
        } else {
            // sum of the W tables' rows in column order (kk = 0, 1, ...), each row gathered whole
            const uint8_t * rows[MAX_TABLES];
            for (int kk = 0; kk < a.W; ++kk) {
                const int id = a.ids[(int64_t) t * a.W + kk];
                const bool ok = id >= 0 && id < a.tab_rows[kk];
                if (!ok && tid == 0) atomicOr(a.err, 1);
                rows[kk] = a.tab[kk] + (int64_t) (ok ? id : 0) * table_row_bytes(a.tab_type[kk], d);
            }
#pragma unroll
            for (int j = 0; j < RN_NV; ++j) {
                const int i0 = 4 * (tid + 256 * j);
                if (i0 >= d) continue;
                float4 e[MAX_TABLES];
#pragma unroll
                for (int kk = 0; kk < MAX_TABLES; ++kk) if (kk < a.W) e[kk] = table_elem4(rows[kk], a.tab_type[kk], i0);
                float4 x = e[0];
#pragma unroll
                for (int kk = 1; kk < MAX_TABLES; ++kk) if (kk < a.W) x = add4(x, e[kk]);
                xv[j] = x;
            }
        }
        // emb_norm (weightless); the normalised row seeds the residual stream
        double ss = 0.0;
#pragma unroll
        for (int j = 0; j < RN_NV; ++j)
            if (4 * (tid + 256 * j) < d) ss += (double) (xv[j].x * xv[j].x) + (double) (xv[j].y * xv[j].y) + (double) (xv[j].z * xv[j].z) + (double) (xv[j].w * xv[j].w);
        const double tot = block_sum_d(ss, red);
        const float scale = 1.0f / sqrtf((float) (tot / (double) d) + a.eps);
#pragma unroll
        for (int j = 0; j < RN_NV; ++j) {
            const int i0 = 4 * (tid + 256 * j);
            if (i0 >= d) continue;
            xv[j] = make_float4(xv[j].x * scale, xv[j].y * scale, xv[j].z * scale, xv[j].w * scale);
            res_out[j] = xv[j];
        }
        st_res = true;
    } else if constexpr (MODE == RN_ACCUM) {
        // sum of the token's k routes in route order, + residual
        const float * __restrict__ src = a.src + ((int64_t) t * a.k) * d;
        const float * rin = a.res_in ? a.res_in + (int64_t) t * d : res;
        float4 r[RN_NV][8], r0[RN_NV];
#pragma unroll
        for (int j = 0; j < RN_NV; ++j) {
            const int i0 = 4 * (tid + 256 * j);
            if (i0 >= d) continue;
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) if (jj < a.k) r[j][jj] = *(const float4 *) (src + (int64_t) jj * d + i0);
            r0[j] = res ? *(const float4 *) (rin + i0) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int j = 0; j < RN_NV; ++j) {
            const int i0 = 4 * (tid + 256 * j);
            if (i0 >= d) continue;
            float4 x = r[j][0];
#pragma unroll
            for (int jj = 1; jj < 8; ++jj) if (jj < a.k) x = add4(x, r[j][jj]);
            cap_out[j] = x;
            if (res) { x = add4(x, r0[j]); res_out[j] = x; }
            xv[j] = x;
        }
        st_cap = a.cap_x != nullptr;
        st_res = res != nullptr;
    } else if constexpr (MODE == RN_ADD) {
        // res = res_in (or res itself) + src
        const float * __restrict__ src = a.src + (int64_t) t * d;
        const float * rin = a.res_in ? a.res_in + (int64_t) t * d : res;
        float4 x[RN_NV], r0[RN_NV];
#pragma unroll
        for (int j = 0; j < RN_NV; ++j) {
            const int i0 = 4 * (tid + 256 * j);
            if (i0 < d) { x[j] = *(const float4 *) (src + i0); r0[j] = *(const float4 *) (rin + i0); }
        }
#pragma unroll
        for (int j = 0; j < RN_NV; ++j) {
            const int i0 = 4 * (tid + 256 * j);
            if (i0 >= d) continue;
            xv[j] = add4(x[j], r0[j]);
            res_out[j] = xv[j];
        }
        st_res = true;
    } else {
#pragma unroll
        for (int j = 0; j < RN_NV; ++j) {
            const int i0 = 4 * (tid + 256 * j);
            if (i0 < d) xv[j] = *(const float4 *) (a.src + (int64_t) t * d + i0);
        }
    }
    if (a.norm_w) {
        double ss = 0.0;
#pragma unroll
        for (int j = 0; j < RN_NV; ++j)
            if (4 * (tid + 256 * j) < d) ss += (double) (xv[j].x * xv[j].x) + (double) (xv[j].y * xv[j].y) + (double) (xv[j].z * xv[j].z) + (double) (xv[j].w * xv[j].w);
        const double tot = block_sum_d(ss, red);
        const float scale = 1.0f / sqrtf((float) (tot / (double) d) + a.eps);
#pragma unroll
        for (int j = 0; j < RN_NV; ++j) {
            const int i0 = 4 * (tid + 256 * j);
            if (i0 >= d) continue;
            xv[j] = make_float4((xv[j].x * scale) * nw[j].x, (xv[j].y * scale) * nw[j].y, (xv[j].z * scale) * nw[j].z, (xv[j].w * scale) * nw[j].w);
        }
    }
    if (a.act_fmt == ACT_Q8_K && d % 1024 == 0) {
        encode_q8k_regs(xv, d, a.act, t);            // each wave holds its blocks already
    } else if (a.act_fmt == ACT_Q8_0 && d % 1024 == 0) {
        encode_q80_regs(xv, d, a.act, t);            // each 8-lane group holds its block
    } else if (a.act_fmt != ACT_NONE) {
        // the encoders read the row from LDS (a 256-block spans the elements of 64 threads)
#pragma unroll
        for (int j = 0; j < RN_NV; ++j) {
            const int i0 = 4 * (tid + 256 * j);
            if (i0 < d) *(float4 *) (xs + i0) = xv[j];
        }
        lds_sync();
        encode_row_rt(a.act_fmt, xs, d, a.act, t);
    }
#pragma unroll
    for (int j = 0; j < RN_NV; ++j) {
        const int i0 = 4 * (tid + 256 * j);
        if (i0 >= d) continue;
        if (st_res) *(float4 *) (res + i0) = res_out[j];
        if (st_cap) *(float4 *) (a.cap_x + (int64_t) t * d + i0) = cap_out[j];
        if (a.norm_w && a.cur_out) *(float4 *) (a.cur_out + (int64_t) t * d + i0) = xv[j];
    }
}

// ------------------------------------------------------------------ k_gemv
enum { EPI_STORE = 0, EPI_SOFTCAP = 1, EPI_ROUTE_W = 2 };
enum { MM_PLAIN = 0, MM_SWIGLU = 1 };   // m16 kernel variants (host-side choice)

struct GemvArgs {
    const uint8_t * w[2];              // tiled weights (matrix m = blockIdx.z)
    const uint16_t * dpl[2];           // Q6_K f16 d plane
    int64_t mat_bytes, dpl_elems;      // per-expert strides
    int nsb, tiles, rows;              // padded K = nsb*256
    // token source
    int grouped;                       // 0: tokens [y*NT, ...) of n_tok; 1: routes with sel == blockIdx.y
    int n_tok;                         // dense token count / grouped: number of tokens T
    const int32_t * sel; int k;        // [T][k]
    ActBuf act;                        // ST_ACT source rows (indexed by token)
    int mode;                          // MM_* (m16 kernels)
    int act_by_route;                  // grouped: activation row = route (else token = route / k)
    int n_mats;                        // matrices in the launch (gate+up = 2)
    int tpb;                           // dense: tokens per block (<= NT)
    // output
    float * out[2]; int out_ld;        // out[m][row-index][rows]; row-index = token or route
    int epi; float cap; const float * route_w;
    int E;
    const int32_t * r_off;             // grouped: [E+1] route offsets by expert (k_route_sort)
    const int32_t * r_perm;            // grouped: [n_tok*k] flat route ids in expert order
    const float * xf; int xf_ld;       // k_gemv_split<..., XF>: fp32 source rows (stride xf_ld), encoded
                                       // to Q8_0 in the block's staging instead of act
};

// The grouping of mul_mat_id's routes by expert, as a stable counting sort of the flat top-k ids
// (route r = token * k + j): position of a route = offset of its expert + routes of that expert
// before it. One 1024-thread block; wave w owns the contiguous routes [w seg, (w + 1) seg) (whole
// 64-route rounds, the waves in flat order) and loads up to SORT_RPW rounds at once:
//   1. per wave and expert counts (LDS atomics);
//   2. expert offsets (a scan over the experts) and each wave's first position per expert;
//   3. each wave places its rounds in order with no block barrier: a lane's mask of the round's
//      lanes with the same expert comes from one ballot per bit of the expert id, its rank within
//      the expert from that mask, and the expert's lowest lane advances the wave's next position of
//      the expert (LDS; every lane reads it before that lane writes it).
// E <= SORT_EMAX.
constexpr int SORT_EMAX = 256;
constexpr int SORT_RPW = 16;
constexpr int LIST_MAX = 1024;   // routes a grouped matmul block lists in LDS itself (without k_route_sort)
#ifndef Z2H_TEMPLATES_ONLY
__global__ void __launch_bounds__(1024) k_route_sort(const int32_t * sel, int n_routes, int E, int32_t * off, int32_t * perm,
                                                     int32_t * cap_counts, int32_t * cap_off, int32_t * cap_perm) {
    __shared__ int s_wc[16][SORT_EMAX];              // per wave and expert: routes, then the wave's first position
    __shared__ int s_cnt[SORT_EMAX], s_off[SORT_EMAX + 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int seg = (n_routes + 1023) / 1024 * 64;
    const int lo = min(n_routes, wave * seg), hi = min(n_routes, lo + seg);
    // the wave's rounds b, b + 64, ... (up to SORT_RPW of them): route b + 64 j + lane in v[j]
    auto load_rounds = [&](int b, int (&v)[SORT_RPW]) {
#pragma unroll
        for (int j = 0; j < SORT_RPW; ++j) v[j] = sel[min(b + 64 * j + lane, hi - 1)];
    };
    for (int e = lane; e < E; e += 64) s_wc[wave][e] = 0;
    __syncthreads();
    for (int b = lo; b < hi; b += 64 * SORT_RPW) {
        int v[SORT_RPW];
        load_rounds(b, v);
#pragma unroll
        for (int j = 0; j < SORT_RPW; ++j)
            if (b + 64 * j + lane < hi) atomicAdd(&s_wc[wave][v[j]], 1);
    }
    __syncthreads();
    for (int e = tid; e < E; e += 1024) {
        int t = 0;
#pragma unroll
        for (int w = 0; w < 16; ++w) t += s_wc[w][e];
        s_cnt[e] = t;
    }
    __syncthreads();
    if (wave == 0) {                                 // exclusive offsets, experts 4 l .. 4 l + 3 in lane l
        int c[4], sum = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) { const int e = 4 * lane + i; c[i] = e < E ? s_cnt[e] : 0; sum += c[i]; }
        int incl = sum;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) { const int u = __shfl_up(incl, d, 64); if (lane >= d) incl += u; }
        int acc = incl - sum;
#pragma unroll
        for (int i = 0; i < 4; ++i) { const int e = 4 * lane + i; if (e < E) s_off[e] = acc; acc += c[i]; }
        if (lane == 63) s_off[E] = incl;
    }
    __syncthreads();
    for (int e = tid; e < E; e += 1024) {
        int c[16];
#pragma unroll
        for (int w = 0; w < 16; ++w) c[w] = s_wc[w][e];
        int acc = s_off[e];
#pragma unroll
        for (int w = 0; w < 16; ++w) { s_wc[w][e] = acc; acc += c[w]; }
    }
    __syncthreads();
    const int nbits = 32 - __builtin_clz(max(E - 1, 1));
    const uint64_t lt = (1ull << lane) - 1ull;
    for (int b = lo; b < hi; b += 64 * SORT_RPW) {
        int v[SORT_RPW];
        load_rounds(b, v);
#pragma unroll
        for (int j = 0; j < SORT_RPW; ++j) {
            const int r = b + 64 * j + lane;
            if (b + 64 * j >= hi) break;                 // wave-uniform
            const bool valid = r < hi;
            const int me = valid ? v[j] : 0;
            uint64_t same = __ballot(valid);
            for (int bit = 0; bit < nbits; ++bit) {
                const bool on = (me >> bit) & 1;
                const uint64_t bb = __ballot(on);
                same &= on ? bb : ~bb;
            }
            const int rank = __popcll(same & lt);
            const int first = s_wc[wave][me];
            if (valid) {
                perm[first + rank] = r;
                if (rank == 0) s_wc[wave][me] = first + __popcll(same);
            }
        }
    }
    for (int e = tid; e <= E; e += 1024) off[e] = s_off[e];
    if (cap_counts) {
        for (int e = tid; e < E; e += 1024) cap_counts[e] = s_cnt[e];
        for (int e = tid; e <= E; e += 1024) cap_off[e] = s_off[e];
        __syncthreads();
        for (int r = tid; r < n_routes; r += 1024) cap_perm[r] = perm[r];
    }
}
#endif

// Routes of expert e in ascending flat order (the stable counting sort of mul_mat_id's grouping).
__device__ __forceinline__ int build_route_list(const int32_t * sel, int n_routes, int e, int * list, int * wcount) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int total = 0;
    for (int base = 0; base < n_routes; base += 256) {
        const int r = base + tid;
        const bool hit = r < n_routes && sel[r] == e;
        const unsigned long long m = __ballot(hit);
        const int before = __popcll(m & ((1ull << lane) - 1ull));
        if (lane == 0) wcount[wave] = __popcll(m);
        lds_sync();
        int off = total;
        for (int w = 0; w < wave; ++w) off += wcount[w];
        if (hit) list[off + before] = r;
        const int add = wcount[0] + wcount[1] + wcount[2] + wcount[3];
        lds_sync();
        total += add;
    }
    return total;
}

// The routes of expert e for a grouped matmul block: from k_route_sort's table when given (r_perm),
// else listed in LDS by the block (lds, at most LIST_MAX routes). Same stable order either way.
__device__ __forceinline__ const int32_t * expert_routes(const GemvArgs & a, int e, int * lds, int * wcount, int & n_items) {
    if (a.r_perm) { n_items = a.r_off[e + 1] - a.r_off[e]; return a.r_perm + a.r_off[e]; }
    n_items = build_route_list(a.sel, a.n_tok * a.k, e, lds, wcount);
    return lds;
}

template <int WF>
__device__ __forceinline__ void load_unit(const uint4 * __restrict__ u, uint4 (&r)[wfmt<WF>::C]) {
#pragma unroll
    for (int c = 0; c < wfmt<WF>::C; ++c) r[c] = u[c * TILE];
}

// One 256-column unit of the lane's row against nt staged activation rows. The unit is decoded once
// (outside the token loop); each token's block value is added to the wave's LDS accumulator
// sacc[tt * TILE] (per lane), so the token loop carries no register arrays.
template <int WF>
__device__ __forceinline__ void gemv_unit(const uint4 (&u)[wfmt<WF>::C], const uint16_t * dp, int sb, int nsb, int K,
                                          const int8_t * sq, const float * sd32, const float * sd256,
                                          const int16_t * sbs, const uint16_t * sh, int nt, float * sacc) {
    if constexpr (WF == WF_Q4_K) {
        const uint4 hdr = u[0];
        const float d = h2f(hdr.x & 0xffffu), dmin = h2f(hdr.x >> 16);
        uint8_t scb[12];
        __builtin_memcpy(scb, &hdr.y, 4); __builtin_memcpy(scb + 4, &hdr.z, 4); __builtin_memcpy(scb + 8, &hdr.w, 4);
        int sc[8], mn[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) q4k_sm(scb, j, sc[j], mn[j]);
        // qs chunk c (1..8) holds bytes 16(c-1)..: pair p = (c-1)/2; low nibbles -> sub-block 2p,
        // high nibbles -> sub-block 2p+1, at element dword 16p + 4*((c-1)&1) (+8 for high) + m
        uint32_t lo[32], hi[32];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint4 v = u[c + 1];
            const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int m = 0; m < 4; ++m) { lo[4 * c + m] = w4[m] & 0x0f0f0f0fu; hi[4 * c + m] = (w4[m] >> 4) & 0x0f0f0f0fu; }
        }
        for (int tt = 0; tt < nt; ++tt) {
            const int * aq = (const int *) (sq + tt * K + sb * 256);
            int sumi = 0;
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                int il = 0, ih = 0;
#pragma unroll
                for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                    for (int m = 0; m < 4; ++m) {
                        il = sdot4((int) lo[8 * p + 4 * hf + m], aq[16 * p + 4 * hf + m], il);
                        ih = sdot4((int) hi[8 * p + 4 * hf + m], aq[16 * p + 8 + 4 * hf + m], ih);
                    }
                sumi += sc[2 * p] * il + sc[2 * p + 1] * ih;
            }
            const int16_t * bsr = sbs + tt * (K / 16) + sb * 16;
            int summ = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) summ += mn[j] * ((int) bsr[2 * j] + (int) bsr[2 * j + 1]);
            const float dx = sd256[tt * nsb + sb];
            sacc[tt * TILE] += (d * dx) * (float) sumi - (dmin * dx) * (float) summ;
        }
    } else if constexpr (WF == WF_Q6_K) {
        const uint4 scv = u[12];
        int8_t sc[16];
        __builtin_memcpy(sc, &scv, 16);
        const float d = h2f(*dp);
        // unsigned 6-bit values per element dword dw = 32h + 8grp + l4 (grp = element quarter of the half)
        uint32_t qv[64];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int l4 = 0; l4 < 8; ++l4) {
                const int a0 = 16 * h + l4, a1 = 16 * h + 8 + l4, ah = 8 * h + l4;
                const uint4 v0 = u[a0 >> 2], v1 = u[a1 >> 2], vh = u[8 + (ah >> 2)];
                const uint32_t L0 = (a0 & 3) == 0 ? v0.x : (a0 & 3) == 1 ? v0.y : (a0 & 3) == 2 ? v0.z : v0.w;
                const uint32_t L1 = (a1 & 3) == 0 ? v1.x : (a1 & 3) == 1 ? v1.y : (a1 & 3) == 2 ? v1.z : v1.w;
                const uint32_t H  = (ah & 3) == 0 ? vh.x : (ah & 3) == 1 ? vh.y : (ah & 3) == 2 ? vh.z : vh.w;
                qv[32 * h + l4]      = (L0 & 0x0f0f0f0fu) | ((H & 0x03030303u) << 4);
                qv[32 * h + 8 + l4]  = (L1 & 0x0f0f0f0fu) | (((H >> 2) & 0x03030303u) << 4);
                qv[32 * h + 16 + l4] = ((L0 >> 4) & 0x0f0f0f0fu) | (((H >> 4) & 0x03030303u) << 4);
                qv[32 * h + 24 + l4] = ((L1 >> 4) & 0x0f0f0f0fu) | (((H >> 6) & 0x03030303u) << 4);
            }
        for (int tt = 0; tt < nt; ++tt) {
            const int * aq = (const int *) (sq + tt * K + sb * 256);
            const int16_t * bsr = sbs + tt * (K / 16) + sb * 16;
            int sumi = 0;
#pragma unroll
            for (int g = 0; g < 16; ++g) {             // 16-element scale group = dwords 4g..4g+3
                int is = 0;
#pragma unroll
                for (int m = 0; m < 4; ++m) is = sdot4((int) qv[4 * g + m], aq[4 * g + m], is);
                sumi += (int) sc[g] * (is - 32 * (int) bsr[g]);
            }
            sacc[tt * TILE] += (d * sd256[tt * nsb + sb]) * (float) sumi;
        }
    } else if constexpr (WF == WF_Q8_0) {
        uint32_t qw[64];
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            const uint4 v = u[c];
            qw[4 * c] = v.x; qw[4 * c + 1] = v.y; qw[4 * c + 2] = v.z; qw[4 * c + 3] = v.w;
        }
        const uint4 dv = u[16];
        uint16_t dh[8];
        __builtin_memcpy(dh, &dv, 16);
        for (int tt = 0; tt < nt; ++tt) {
            const int * aq = (const int *) (sq + tt * K + sb * 256);
            const float * dx = sd32 + tt * (K / 32) + sb * 8;
            float a = sacc[tt * TILE];
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                int is = 0;
#pragma unroll
                for (int m = 0; m < 8; ++m) is = sdot4((int) qw[8 * b + m], aq[8 * b + m], is);
                a += (h2f(dh[b]) * dx[b]) * (float) is;
            }
            sacc[tt * TILE] = a;
        }
    } else {   // F16
        for (int tt = 0; tt < nt; ++tt) {
            const uint32_t * ah = (const uint32_t *) (sh + tt * K + sb * 256);
            float s = 0.0f;
#pragma unroll
            for (int c = 0; c < 32; ++c) {
                const uint4 v = u[c];
                s = fdot2(v.x, ah[4 * c], s); s = fdot2(v.y, ah[4 * c + 1], s);
                s = fdot2(v.z, ah[4 * c + 2], s); s = fdot2(v.w, ah[4 * c + 3], s);
            }
            sacc[tt * TILE] += s;
        }
    }
    (void) dp; (void) nsb; (void) sd32; (void) sd256; (void) sbs; (void) sh;
}

// Stage nt encoded activation rows (row tt = token tok(tt)) into the LDS planes of the row kernels.
template <int AF, class TokFn>
__device__ __forceinline__ void stage_acts(const GemvArgs & a, int nt, TokFn tok, int K, int8_t * sq, float * sd32,
                                           float * sd256, int16_t * sbs, uint16_t * sh) {
    const int tid = threadIdx.x;
    if constexpr (AF == ACT_Q8_K || AF == ACT_Q8_0) {
        const int per = K / 16;
        copy16<256>(nt * per, [&](int i) { return (const uint4 *) (a.act.q + (int64_t) tok(i / per) * K) + i % per; },
                    [&](int i) { return (uint4 *) (sq + (i / per) * K) + i % per; });
        if constexpr (AF == ACT_Q8_K) {
            for (int i = tid; i < nt * (K / 256); i += 256) sd256[i] = a.act.d256[(int64_t) tok(i / (K / 256)) * (K / 256) + i % (K / 256)];
            for (int i = tid; i < nt * (K / 16); i += 256) sbs[i] = a.act.bs[(int64_t) tok(i / (K / 16)) * (K / 16) + i % (K / 16)];
        } else {
            for (int i = tid; i < nt * (K / 32); i += 256) sd32[i] = a.act.d32[(int64_t) tok(i / (K / 32)) * (K / 32) + i % (K / 32)];
        }
    } else {
        const int per = K / 8;
        copy16<256>(nt * per, [&](int i) { return (const uint4 *) (a.act.h + (int64_t) tok(i / per) * K) + i % per; },
                    [&](int i) { return (uint4 *) (sh + (i / per) * K) + i % per; });
    }
}

// LDS budget of k_gemv for activations of K (padded) columns
__host__ __device__ inline size_t gemv_lds_bytes(int act, int K) {
    size_t b = (size_t) 4 * NT * TILE * 4;                         // reduction buffer
    if (act == ACT_Q8_K) b += (size_t) NT * K + (size_t) NT * (K / 256) * 4 + (size_t) NT * (K / 16) * 2;
    else if (act == ACT_Q8_0) b += (size_t) NT * K + (size_t) NT * (K / 32) * 4;
    else b += (size_t) NT * K * 2;
    return b + 64;
}

template <int WF>
__global__ void __launch_bounds__(256) k_gemv(GemvArgs a) {
    constexpr int AF = wfmt<WF>::ACT;
    constexpr int C = wfmt<WF>::C;
    extern __shared__ __attribute__((aligned(16))) char smem[];
    __shared__ int s_lds[LIST_MAX];
    __shared__ int s_wcnt[4];
    const int K = a.nsb * 256, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tile = blockIdx.x, m = blockIdx.z;
    // LDS carve-up
    float * s_red = (float *) smem;                                  // [4][NT][64]
    char * p = smem + 4 * NT * TILE * 4;
    int8_t * sq = nullptr; float * sd32 = nullptr; float * sd256 = nullptr; int16_t * sbs = nullptr; uint16_t * sh = nullptr;
    if constexpr (AF == ACT_Q8_K) {
        sq = (int8_t *) p; p += NT * K;
        sd256 = (float *) p; p += NT * (K / 256) * 4;
        sbs = (int16_t *) p; p += NT * (K / 16) * 2;
    } else if constexpr (AF == ACT_Q8_0) {
        sq = (int8_t *) p; p += NT * K;
        sd32 = (float *) p; p += NT * (K / 32) * 4;
    } else {
        sh = (uint16_t *) p; p += NT * K * 2;
    }

    // which rows (tokens / routes) this block serves
    int n_items, item0 = 0;
    int e = 0;
    const int32_t * s_list = nullptr;                                // grouped: the expert's routes
    if (a.grouped) {
        e = blockIdx.y;
        s_list = expert_routes(a, e, s_lds, s_wcnt, n_items);
        if (n_items == 0) return;
    } else {
        item0 = blockIdx.y * a.tpb;
        n_items = min(a.tpb, a.n_tok - item0);
        if (n_items <= 0) return;
    }
    const uint8_t * wbase = a.w[m] + (int64_t) e * a.mat_bytes;
    const uint16_t * dbase = WF == WF_Q6_K ? a.dpl[m] + (int64_t) e * a.dpl_elems : nullptr;
    const uint4 * wt = (const uint4 *) wbase + (size_t) tile * a.nsb * C * TILE + lane;
    // issue this wave's weight loads before the activations are staged (up to PF units stay in
    // registers for every token chunk; further units are loaded in the compute loop)
    constexpr int PF = 1;
    uint4 wr[PF][C];
#pragma unroll
    for (int j = 0; j < PF; ++j) {
        const int sb = wave + 4 * j;
        if (sb < a.nsb) load_unit<WF>(wt + (size_t) sb * C * TILE, wr[j]);
    }

    for (int c0 = 0; c0 < n_items; c0 += NT) {
        const int nt = min(NT, n_items - c0);
        lds_sync();
        // ---- stage the activation rows of this chunk into LDS
        stage_acts<AF>(a, nt, [&](int tt) { const int it = a.grouped ? s_list[c0 + tt] : item0 + c0 + tt;
                                             return a.grouped && !a.act_by_route ? it / a.k : it; },
                       K, sq, sd32, sd256, sbs, sh);
        lds_sync();
        // ---- each wave: its share of the 256-column units, lane = row of the tile; partial sums
        // accumulate in the wave's LDS slice s_red[wave][tt][lane] in unit order
        float * sacc = s_red + (wave * NT) * TILE + lane;
        for (int tt = 0; tt < nt; ++tt) sacc[tt * TILE] = 0.0f;
#pragma unroll
        for (int j = 0; j < PF; ++j) {
            const int sb = wave + 4 * j;
            if (sb < a.nsb) {
                const uint16_t * dp = WF == WF_Q6_K ? dbase + ((size_t) tile * a.nsb + sb) * TILE + lane : nullptr;
                gemv_unit<WF>(wr[j], dp, sb, a.nsb, K, sq, sd32, sd256, sbs, sh, nt, sacc);
            }
        }
        for (int sb = wave + 4 * PF; sb < a.nsb; sb += 4) {
            uint4 r[C];
            load_unit<WF>(wt + (size_t) sb * C * TILE, r);
            const uint16_t * dp = WF == WF_Q6_K ? dbase + ((size_t) tile * a.nsb + sb) * TILE + lane : nullptr;
            gemv_unit<WF>(r, dp, sb, a.nsb, K, sq, sd32, sd256, sbs, sh, nt, sacc);
        }
        lds_sync();
        // ---- reduce the 4 waves (in wave order) and store
        for (int o = tid; o < nt * TILE; o += 256) {
            const int tt = o / TILE, r = o % TILE;
            const float v = ((s_red[(0 * NT + tt) * TILE + r] + s_red[(1 * NT + tt) * TILE + r]) +
                              s_red[(2 * NT + tt) * TILE + r]) + s_red[(3 * NT + tt) * TILE + r];
            const int row = tile * TILE + r;
            if (row >= a.rows) continue;
            const int it = a.grouped ? s_list[c0 + tt] : item0 + c0 + tt;
            float y = v;
            if (a.epi == EPI_SOFTCAP) y = z_softcap(v, a.cap);
            else if (a.epi == EPI_ROUTE_W) y = v * a.route_w[it];
            a.out[m][(int64_t) it * a.out_ld + row] = y;
        }
    }
}

// Row-streaming variant for the grouped expert matmuls: each wave owns one 64-row tile over the
// full K (no cross-wave reduction), its 256-column units double-buffered in registers so one
// unit's loads are in flight while the previous one is decoded; the 4 waves of a block (4 tiles of
// the same expert matrix) share one activation staging of up to NTE routes.
constexpr int NTE = 8;

__host__ __device__ inline size_t gemv_rows_lds_bytes(int act, int K) {
    size_t b = (size_t) 4 * NTE * TILE * 4;                        // per-wave accumulators
    if (act == ACT_Q8_K) b += (size_t) NTE * K + (size_t) NTE * (K / 256) * 4 + (size_t) NTE * (K / 16) * 2;
    else if (act == ACT_Q8_0) b += (size_t) NTE * K + (size_t) NTE * (K / 32) * 4;
    else b += (size_t) NTE * K * 2;
    return b + 64;
}

template <int WF>
__global__ void __launch_bounds__(256) k_gemv_rows(GemvArgs a) {
    constexpr int AF = wfmt<WF>::ACT;
    constexpr int C = wfmt<WF>::C;
    extern __shared__ __attribute__((aligned(16))) char smem[];
    __shared__ int s_lds[LIST_MAX];
    __shared__ int s_wcnt[4];
    const int K = a.nsb * 256, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // grid z = matrix + n_mats * pass: pass p takes the expert's routes [p * NTE, p * NTE + NTE), so a
    // popular expert's routes spread over blocks instead of looping in one
    const int tile = blockIdx.x * 4 + wave, m = blockIdx.z % a.n_mats, pass = blockIdx.z / a.n_mats, e = blockIdx.y;
    float * s_acc = (float *) smem;                                  // [4][NTE][64]
    char * p = smem + 4 * NTE * TILE * 4;
    int8_t * sq = nullptr; float * sd32 = nullptr; float * sd256 = nullptr; int16_t * sbs = nullptr; uint16_t * sh = nullptr;
    if constexpr (AF == ACT_Q8_K) {
        sq = (int8_t *) p; p += NTE * K;
        sd256 = (float *) p; p += NTE * (K / 256) * 4;
        sbs = (int16_t *) p; p += NTE * (K / 16) * 2;
    } else if constexpr (AF == ACT_Q8_0) {
        sq = (int8_t *) p; p += NTE * K;
        sd32 = (float *) p; p += NTE * (K / 32) * 4;
    } else {
        sh = (uint16_t *) p; p += NTE * K * 2;
    }
    int n_items;
    const int32_t * s_list = expert_routes(a, e, s_lds, s_wcnt, n_items);
    if (n_items == 0) return;
    const bool has_tile = tile < a.tiles;
    const uint8_t * wbase = a.w[m] + (int64_t) e * a.mat_bytes;
    const uint16_t * dbase = WF == WF_Q6_K ? a.dpl[m] + (int64_t) e * a.dpl_elems : nullptr;
    const uint4 * wt = (const uint4 *) wbase + (size_t) (has_tile ? tile : 0) * a.nsb * C * TILE + lane;
    float * sacc = s_acc + (wave * NTE) * TILE + lane;

    {
        const int c0 = pass * NTE;
        if (c0 >= n_items) return;
        const int nt = min(NTE, n_items - c0);
        uint4 u0[C], u1[C];
        if (has_tile) {
            load_unit<WF>(wt, u0);
            if (a.nsb > 1) load_unit<WF>(wt + (size_t) C * TILE, u1);
        }
        lds_sync();
        stage_acts<AF>(a, nt, [&](int tt) { const int it = s_list[c0 + tt]; return a.act_by_route ? it : it / a.k; },
                       K, sq, sd32, sd256, sbs, sh);
        for (int tt = 0; tt < nt; ++tt) sacc[tt * TILE] = 0.0f;
        lds_sync();
        if (has_tile) {
            for (int sb = 0; sb < a.nsb; sb += 2) {
                const uint16_t * dp0 = WF == WF_Q6_K ? dbase + ((size_t) tile * a.nsb + sb) * TILE + lane : nullptr;
                gemv_unit<WF>(u0, dp0, sb, a.nsb, K, sq, sd32, sd256, sbs, sh, nt, sacc);
                if (sb + 2 < a.nsb) load_unit<WF>(wt + (size_t) (sb + 2) * C * TILE, u0);
                if (sb + 1 < a.nsb) {
                    const uint16_t * dp1 = WF == WF_Q6_K ? dbase + ((size_t) tile * a.nsb + sb + 1) * TILE + lane : nullptr;
                    gemv_unit<WF>(u1, dp1, sb + 1, a.nsb, K, sq, sd32, sd256, sbs, sh, nt, sacc);
                    if (sb + 3 < a.nsb) load_unit<WF>(wt + (size_t) (sb + 3) * C * TILE, u1);
                }
            }
            const int row = tile * TILE + lane;
            if (row < a.rows)
                for (int tt = 0; tt < nt; ++tt) {
                    const int it = s_list[c0 + tt];
                    float y = sacc[tt * TILE];
                    if (a.epi == EPI_ROUTE_W) y = y * a.route_w[it];
                    a.out[m][(int64_t) it * a.out_ld + row] = y;
                }
        }
    }
}

// MFMA variant for Q4_K and Q8_0 weights (v_mfma_i32_16x16x32_i8). The product is computed as
// C[token][row] = A[token][k] . B[k][row] with A = the encoded activations (from LDS) and B = the
// weights, so every lane ends with 4 tokens x 1 row and applies its own row's block scales. One
// wave owns a 16-row group over the full K and accumulates its row in block order, which is the
// CPU oracle's summation order. Layout "m16": per (16-row group, 256-column unit) the integer
// values are stored chunk-major for the lanes (lane l = (k-slice l/16, row l%16) owns 8 bytes of
// each 32-element sub-block), followed by the 16 rows' scale headers:
//   Q4_K 2304 B = 2 x 1 KiB nibble chunks + 16 x 16 B (d, dmin, scales)
//   Q8_0 4352 B = 4 x 1 KiB int8 chunks   + 16 x 16 B (eight f16 block scales)
typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef float v4f_t __attribute__((ext_vector_type(4)));
template <int WF> struct m16fmt;
// WPE: waves per SIMD of the PF = 1 kernels; GPF / GWPE: register-ring depth and waves per SIMD of
// the grouped (expert) launches
template <> struct m16fmt<WF_Q4_K> { static constexpr int QS = 2; static constexpr int BYTES = 2304; static constexpr int WPE = 5;
                                     static constexpr int GPF = 1; static constexpr int GWPE = 5; };
template <> struct m16fmt<WF_Q8_0> { static constexpr int QS = 4; static constexpr int BYTES = 4352; static constexpr int WPE = 4;
                                     static constexpr int GPF = 1; static constexpr int GWPE = 4; };
// Q6_K (8 or 16 token rows per pass): 3360 B = 2 x 1 KiB low-nibble chunks + 1 KiB of high
// bits + 16 x 16 B scales + 16 x f16 d; qs[3].x holds the d pair of the lane's row
template <> struct m16fmt<WF_Q6_K> { static constexpr int QS = 4; static constexpr int BYTES = 3360; static constexpr int WPE = 4;
                                     static constexpr int GPF = 1; static constexpr int GWPE = 4; };
constexpr int MT = 16;                  // tokens per MFMA pass

// token rows per pass of the m16 kernels: grouped expert launches stage up to MT_G routes (an
// expert serves ~2 at 16 requests), dense launches all MT tokens so each weight tile is read once
constexpr int MT_G = 8;
constexpr int M16_ZERO = 256;           // Q6_K: zero bytes ahead of the staged rows (the idle halves of the A operand)
__host__ __device__ inline size_t gemv_mfma_lds_bytes(int wf, int K, int rows) {
    const size_t KP = (size_t) K + 16;
    if (wf == WF_Q4_K) return rows * KP + (size_t) rows * (K / 32) * 4 + (size_t) rows * (K / 256) * 4 + 64;
    if (wf == WF_Q6_K) return M16_ZERO + rows * KP + (size_t) rows * (K / 16) * 4 + (size_t) rows * (K / 256) * 4 + 64;
    return rows * KP + (size_t) rows * (K / 32) * 4 + 64;
}

template <int WF>
__device__ __forceinline__ void m16_load(const uint4 * __restrict__ unit, int lane, uint4 (&qs)[m16fmt<WF>::QS], uint4 & hd) {
    if constexpr (WF == WF_Q6_K) {
        qs[0] = unit[lane]; qs[1] = unit[64 + lane]; qs[2] = unit[128 + lane];
        hd = unit[192 + (lane & 15)];                                    // the row's 16 scales
        qs[3].x = ((const uint32_t *) (unit + 208))[(lane & 15) >> 1];   // d of rows 2i, 2i + 1
        return;
    }
#pragma unroll
    for (int c = 0; c < m16fmt<WF>::QS; ++c) qs[c] = unit[c * 64 + lane];
    hd = unit[m16fmt<WF>::QS * 64 + (lane & 15)];
}

// One 256-column unit of a wave's 16 rows against the staged token rows. Token rows beyond the last
// valid one (ntm1) read that row instead (their results are discarded), so LDS holds only the valid
// rows. The unit's value x per (token, row) is folded into the row's sum by m16_fold: Q4_K x =
// fma(d, isum, -dmin * msum) and sum = fma(dx, x, sum) with the token's block scale dx (xd); Q8_0
// x = the unit's 8 scaled block products (xd = 1) and sum = sum + x. Every Q4_K matmul (the GEMVs
// here and k_gemm_q4k) folds the units of a row in superblock order with these operations, so a
// token's result does not depend on the batch it is in.
template <int WF>
__device__ __forceinline__ void m16_fold(float & acc, float x, float xd) {
    if constexpr (WF == WF_Q4_K) acc = __builtin_fmaf(xd, x, acc);
    else acc = acc + x;
}
template <int WF, int ROWS = 16>
__device__ __forceinline__ void m16_unit(const uint4 (&qs)[m16fmt<WF>::QS], const uint4 & hd, int sb, int K, int lane,
                                         const int8_t * sq, const int * sbs2, const float * sdx, int nsb, int ntm1, float (&acc)[4],
                                         float (&xd)[4]) {
    // every operand load and all MFMAs of the unit are issued before the scale arithmetic, so the 8
    // independent products pipeline instead of each waiting for its predecessor's scaling
    const int q = lane >> 4, r = min(lane & 15, ntm1), KP = K + 16;
    const int8_t * arow = sq + r * KP + sb * 256 + 8 * q;          // A: token r, k-slice q
    const v4i_t zero = {0, 0, 0, 0};
    long A[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) A[j] = *(const long *) (arow + 32 * j);
    v4i_t C[8];
    if constexpr (WF == WF_Q4_K) {
        const int * bsr = sbs2 + r * (K / 32) + sb * 8;              // token r (A operand row)
        const float a0 = (float) bsr[q], a1 = (float) bsr[q + 4];
        float dx[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) dx[i] = sdx[min(4 * q + i, ntm1) * nsb + sb];
        const uint32_t w[8] = {qs[0].x, qs[0].y, qs[0].z, qs[0].w, qs[1].x, qs[1].y, qs[1].z, qs[1].w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {                               // sub-block j = nibble half of pair j/2
            const int pr = j >> 1;
            const uint32_t b0 = (j & 1) ? (w[2 * pr] >> 4) & 0x0f0f0f0fu : w[2 * pr] & 0x0f0f0f0fu;
            const uint32_t b1 = (j & 1) ? (w[2 * pr + 1] >> 4) & 0x0f0f0f0fu : w[2 * pr + 1] & 0x0f0f0f0fu;
            C[j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[j], (long) (((uint64_t) b1 << 32) | b0), zero, 0, 0, 0);
        }
        // min correction sum_j m_j[row] * bsum_j[token] as an fp32 16x16x4 product (two k-halves):
        // integer products < 2^19 and sums < 2^23, so the fp32 result is exact
        // (6-bit scales / mins of sub-blocks 0-3 and 4-7, four per dword: GGUF K-quant packing)
        const uint32_t mn03 = hd.z & 0x3f3f3f3fu;
        const uint32_t mn47 = ((hd.w >> 4) & 0x0f0f0f0fu) | ((hd.z >> 2) & 0x30303030u);
        const float b0 = (float) ((mn03 >> (8 * q)) & 0xffu), b1 = (float) ((mn47 >> (8 * q)) & 0xffu);
        v4f_t S = {0.0f, 0.0f, 0.0f, 0.0f};
        S = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b0, S, 0, 0, 0);
        S = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b1, S, 0, 0, 0);
        const float d = h2f(hd.x & 0xffffu), dmin = h2f(hd.x >> 16);
        const uint32_t sc03 = hd.y & 0x3f3f3f3fu;
        const uint32_t sc47 = (hd.w & 0x0f0f0f0fu) | ((hd.y >> 2) & 0x30303030u);
        int sumi[4] = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int scj = (int) (((j < 4 ? sc03 : sc47) >> (8 * (j & 3))) & 0xffu);
#pragma unroll
            for (int i = 0; i < 4; ++i) sumi[i] += __mul24(scj, C[j][i]);   // |products| < 2^22
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc[i] = __builtin_fmaf(d, (float) sumi[i], -(dmin * S[i]));
            xd[i] = dx[i];
        }
    } else if constexpr (WF == WF_Q6_K) {
        // Token rows doubled, 8 per product: A slot s < 8 is token s over k-slots 0-15 of a 32-element
        // chunk (scale group 2m), slot s >= 8 token s - 8 over k-slots 16-31 (group 2m + 1); a lane
        // whose k-slice lies in the other half feeds zeros (M16_ZERO bytes ahead of the staged rows).
        // One MFMA then gives both groups' dots, lanes 0-31 group 2m and lanes 32-63 group 2m + 1
        // for the same tokens. ROWS = 16: a second product set (tokens 8-15) on the same weight
        // operands, its totals in lanes 32-63. The weights enter unsigned (0..63); the -32 offset is
        // subtracted as 32 * sum_g sc_g * bsum_g (bsum = the activation's sum over group g), an fp32
        // 16x16x4 product of integers (|sum| < 2^23: exact). The unit value is the Q6_K row
        // kernels': x = (d * dx) * (float) sum_g sc_g * (dot_g - 32 bsum_g).
        constexpr int NH = ROWS > 8 ? 2 : 1;
        const int q = lane >> 4, s = lane & 15, par = lane >> 5;
        const bool on = (s < 8) == (q < 2);
        long A[NH][8];
        float bs4[NH][4];
#pragma unroll
        for (int hh = 0; hh < NH; ++hh) {
            const int tok = min(8 * hh + (s & 7), ntm1);
            const int8_t * arow = on ? sq + tok * KP + sb * 256 + 8 * q : sq - M16_ZERO + 8 * q;
#pragma unroll
            for (int m = 0; m < 8; ++m) A[hh][m] = *(const long *) (arow + 32 * m);
            const float * bsf = (const float *) sbs2 + tok * (K / 16) + sb * 16 + q;   // group 4 kb + q
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) bs4[hh][kb] = bsf[4 * kb];
        }
        float dx[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) dx[i] = sdx[min((NH == 2 ? 4 * q : 4 * (q & 1)) + i, ntm1) * nsb + sb];
        const uint32_t L[8] = {qs[0].x, qs[0].y, qs[0].z, qs[0].w, qs[1].x, qs[1].y, qs[1].z, qs[1].w};
        const uint32_t H[4] = {qs[2].x, qs[2].y, qs[2].z, qs[2].w};
        const uint32_t scw[4] = {hd.x, hd.y, hd.z, hd.w};
        int sumi[NH][4];
#pragma unroll
        for (int hh = 0; hh < NH; ++hh)
#pragma unroll
            for (int i = 0; i < 4; ++i) sumi[hh][i] = 0;
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const uint32_t hb = H[m >> 1] >> (4 * (m & 1));
            const uint32_t b0 = (L[m] & 0x0f0f0f0fu) | ((hb << 4) & 0x30303030u);          // elements 0-3
            const uint32_t b1 = ((L[m] >> 4) & 0x0f0f0f0fu) | ((hb << 2) & 0x30303030u);   // elements 4-7
            const long B = (long) (((uint64_t) b1 << 32) | b0);
            const int scm = __builtin_amdgcn_sbfe(scw[m >> 1], 16 * (m & 1) + 8 * par, 8);
#pragma unroll
            for (int hh = 0; hh < NH; ++hh) {
                const v4i_t C = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[hh][m], B, zero, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) sumi[hh][i] += __mul24(scm, C[i]);   // |products| < 2^24
            }
        }
        // bias term: sum_g sc_g * bsum_g over the 16 groups as four k = 4 products
        v4f_t S[NH];
#pragma unroll
        for (int hh = 0; hh < NH; ++hh) S[hh] = (v4f_t) {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const float scg = (float) __builtin_amdgcn_sbfe(scw[kb], 8 * q, 8);
#pragma unroll
            for (int hh = 0; hh < NH; ++hh) S[hh] = __builtin_amdgcn_mfma_f32_16x16x4f32(bs4[hh][kb], scg, S[hh], 0, 0, 0);
        }
        const uint32_t dd = qs[3].x >> (16 * (s & 1));
        const float d = h2f(dd & 0xffffu);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int tot;
            float sb32;
            if constexpr (NH == 1) {
                tot = sumi[0][i] + up32_i(sumi[0][i]);                           // lanes 0-31
                sb32 = S[0][i];
            } else {
                // lanes 0-31: tokens 0-7 (own even groups + lane + 32's odd ones); lanes 32-63:
                // tokens 8-15 (own odd groups + lane - 32's even ones), one lane swap for both
                const auto sw = __builtin_amdgcn_permlane32_swap((unsigned) sumi[0][i], (unsigned) sumi[1][i], false, false);
                tot = par ? sumi[1][i] + (int) sw[0] : sumi[0][i] + (int) sw[1];
                sb32 = par ? S[1][i] : S[0][i];
            }
            tot -= 32 * (int) sb32;
            acc[i] = (d * dx[i]) * (float) tot;
            xd[i] = 1.0f;
        }
    } else {
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const uint4 v = qs[b >> 1];
            const uint32_t lo = (b & 1) ? v.z : v.x, hi = (b & 1) ? v.w : v.y;
            C[b] = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[b], (long) (((uint64_t) hi << 32) | lo), zero, 0, 0, 0);
        }
        uint16_t dh[8];
        __builtin_memcpy(dh, &hd, 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) xd[i] = 1.0f;
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const float dw = h2f(dh[b]);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] += (dw * sdx[min(4 * q + i, ntm1) * (K / 32) + sb * 8 + b]) * (float) C[b][i];
        }
    }
}

// Q4_K unit for blocks of at most 2 NP token rows. The A rows of token pair p are (token 2p + t,
// sub-block j) at row 8t + j (lane & 15): MFMA j takes a lane's A row only if the row's sub-block is
// j (zeros otherwise), so one accumulation chain over the unit's 8 sub-blocks leaves D[8t + j][row] =
// the sub-block j dot of token 2p + t with weight row `row` (lane & 15), with no products or scaling
// spent on idle token slots. Lane l (q = l >> 4) holds token 2p + (q >> 1)'s dots of sub-blocks
// 4 (q & 1) + v for the weight row whose scales it loaded; it forms sum_j sc_j dot_j and
// sum_j m_j bsum_j over them (integers) and the lane 16 above adds its half (up16_i): lanes with
// q = 0 and 2 end with the unit value of tokens 2p and 2p + 1 from the same integer sums and final
// operations as m16_unit (x = fma(d, isum, -(dmin * msum))), so the fold gives the same bits.
template <int NP>
__device__ __forceinline__ void m16_unit_q4k_pairs(const uint4 (&qs)[2], const uint4 & hd, int sb, int K, int lane,
                                                   const int8_t * sq, const int * sbs2, const float * sdx, int nsb,
                                                   int ntm1, float (&x)[NP], float (&xd)[NP]) {
    const int c = lane & 15, q = lane >> 4, h = q & 1, ja = c & 7, KP = K + 16;
    const v4i_t zero = {0, 0, 0, 0};
    long av[NP];
    int4 bq[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        const int ta = min(2 * p + (c >> 3), ntm1), to = min(2 * p + (q >> 1), ntm1);
        av[p] = *(const long *) (sq + ta * KP + sb * 256 + 32 * ja + 8 * q);
        bq[p] = *(const int4 *) (sbs2 + to * (K / 32) + sb * 8 + 4 * h);     // sums of 32, sub-blocks 4h..4h+3
        xd[p] = sdx[to * nsb + sb];
    }
    const uint32_t w[8] = {qs[0].x, qs[0].y, qs[0].z, qs[0].w, qs[1].x, qs[1].y, qs[1].z, qs[1].w};
    v4i_t C[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) C[p] = zero;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int pr = j >> 1;
        const uint32_t b0 = (j & 1) ? (w[2 * pr] >> 4) & 0x0f0f0f0fu : w[2 * pr] & 0x0f0f0f0fu;
        const uint32_t b1 = (j & 1) ? (w[2 * pr + 1] >> 4) & 0x0f0f0f0fu : w[2 * pr + 1] & 0x0f0f0f0fu;
        const long B = (long) (((uint64_t) b1 << 32) | b0);
#pragma unroll
        for (int p = 0; p < NP; ++p) C[p] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ja == j ? av[p] : 0L, B, C[p], 0, 0, 0);
    }
    // the 6-bit scales and mins of sub-blocks 4h .. 4h + 3 of the lane's weight row (GGUF K-quant
    // packing: sub-blocks 0-3 in the low 6 bits of bytes y / z, 4-7 from nibbles of w and the top 2
    // bits of y / z), selected by bit masks rather than a lane-divergent branch
    const uint32_t hm = 0u - (uint32_t) h, sh = 2 * h;
    const uint32_t sc = ((hd.y ^ ((hd.y ^ hd.w) & hm)) & 0x0f0f0f0fu) | ((hd.y >> sh) & 0x30303030u);
    const uint32_t mn = ((hd.z ^ ((hd.z ^ (hd.w >> 4)) & hm)) & 0x0f0f0f0fu) | ((hd.z >> sh) & 0x30303030u);
    const float d = h2f(hd.x & 0xffffu), dmin = h2f(hd.x >> 16);
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        const int bs[4] = {bq[p].x, bq[p].y, bq[p].z, bq[p].w};
        int is = 0, ms = 0;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            is += __mul24((int) ((sc >> (8 * v)) & 0xffu), C[p][v]);      // |products| < 2^22
            ms += __mul24((int) ((mn >> (8 * v)) & 0xffu), bs[v]);        // < 2^18
        }
        is += up16_i(is);
        ms += up16_i(ms);
        x[p] = __builtin_fmaf(d, (float) is, -(dmin * (float) ms));       // |ms| < 2^21: exact in fp32
    }
}

// Q8_0 unit for blocks of at most two token rows, in m16_unit_q4k_pairs' (token, sub-block) row layout:
// lane l (q = l >> 4) holds token q >> 1's dots of sub-blocks 4 (q & 1) + v with weight row l & 15.
// Each sub-block's value is m16_unit's x_b = (dw_b * dx_b) * dot_b; lanes with q = 0 and 2 take the
// other four from the lane 16 above and add the eight to 0 in sub-block order, m16_unit's order, so
// the unit value is the same bits.
__device__ __forceinline__ float m16_unit_q80_pairs(const uint4 (&qs)[4], const uint4 & hd, int sb, int K, int lane,
                                                    const int8_t * sq, const float * sdx, int ntm1) {
    const int c = lane & 15, q = lane >> 4, h = q & 1, ja = c & 7, KP = K + 16;
    const int ta = min(c >> 3, ntm1), to = min(q >> 1, ntm1);
    const long av = *(const long *) (sq + ta * KP + sb * 256 + 32 * ja + 8 * q);
    const float4 dx = *(const float4 *) (sdx + to * (K / 32) + sb * 8 + 4 * h);   // sub-blocks 4h .. 4h + 3
    v4i_t C = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint4 v = qs[j >> 1];
        const uint32_t lo = (j & 1) ? v.z : v.x, hi = (j & 1) ? v.w : v.y;
        C = __builtin_amdgcn_mfma_i32_16x16x32_i8(ja == j ? av : 0L, (long) (((uint64_t) hi << 32) | lo), C, 0, 0, 0);
    }
    // the row's f16 scales of sub-blocks 4h .. 4h + 3: two per dword of hd (selected by a bit mask; a
    // lane-dependent choice between the header's dwords would index a private copy of it)
    const uint32_t hm = 0u - (uint32_t) h;
    const uint32_t w0 = hd.x ^ ((hd.x ^ hd.z) & hm), w1 = hd.y ^ ((hd.y ^ hd.w) & hm);
    const float x0 = (h2f(w0 & 0xffffu) * dx.x) * (float) C[0], x1 = (h2f(w0 >> 16) * dx.y) * (float) C[1];
    const float x2 = (h2f(w1 & 0xffffu) * dx.z) * (float) C[2], x3 = (h2f(w1 >> 16) * dx.w) * (float) C[3];
    float t = 0.0f;
    t = t + x0; t = t + x1; t = t + x2; t = t + x3;
    t = t + up16_f(x0); t = t + up16_f(x1); t = t + up16_f(x2); t = t + up16_f(x3);
    return t;
}

// Stage the encoded activation rows of nt tokens (LDS row tt = token tok(tt)) for the m16 kernels:
// int8 values [rows][K+16], Q8_K sums of 32 [rows][K/32] and scales [rows][K/256], or Q8_0 scales
// [rows][K/32]. The block's 256 threads walk the nt x (K/16) 16-byte items in one flat sequence
// (thread tid takes items tid, tid + 256, ...; rows are not padded to the block width) with MAXJ
// items per thread in flight, so a chunk of nt * K/16 <= 256 * MAXJ items takes one round trip. Items
// past the chunk re-read its last row (every load issues without a branch) and are not stored. mid()
// runs once, after the first MAXJ items' loads are issued: the caller's weight loads go there, behind
// the staging loads, so the stores wait only for the staging data (loads complete in issue order).
// BS16 (Q6_K): the Q8_K sums of 16 as floats [rows][K/16] in place of the sums of 32.
template <int AF, int MAXJ, bool BS16 = false, class TokFn, class MidFn>
__device__ __forceinline__ void m16_stage_flat(const ActBuf & act, int nt, TokFn tok, int K, int8_t * sq, int * sbs2,
                                               float * sdx, MidFn mid) {
    const int tid = threadIdx.x, KP = K + 16;
    const int per = K / 16, ns = K / 32, nd = K / 256;
    const int dq = 256 / per, dr = 256 - dq * per;                   // item i -> i + 256: rows, columns
    int row = tid / per, c = tid - row * per;
    bool first = true;
    for (int base = 0; base < nt * per; base += 256 * MAXJ) {
        u32x4 v[MAXJ];
        uint32_t sv[MAXJ];
        float dv[MAXJ];
        int rj[MAXJ], cj[MAXJ];
#pragma unroll
        for (int j = 0; j < MAXJ; ++j) {
            rj[j] = row; cj[j] = c;
            const int tr = tok(min(row, nt - 1)), cs = min(c, ns - 1), cd = min(c, nd - 1);
            v[j] = *(const u32x4 *) (act.q + (int64_t) tr * K + c * 16);
            if constexpr (AF == ACT_Q8_K) {
                sv[j] = *(const uint32_t *) (act.bs + (int64_t) tr * (K / 16) + 2 * cs);
                dv[j] = act.d256[(int64_t) tr * nd + cd];
            } else {
                sv[j] = __builtin_bit_cast(uint32_t, act.d32[(int64_t) tr * ns + cs]);
            }
            row += dq; c += dr;
            if (c >= per) { c -= per; ++row; }
        }
        if (first) { mid(); first = false; }
#pragma unroll
        for (int j = 0; j < MAXJ; ++j) {
            const int r = rj[j], cc = cj[j];
            if (r >= nt) continue;
            *(u32x4 *) (sq + r * KP + cc * 16) = v[j];
            if (cc < ns) {
                if constexpr (BS16) {
                    float * f = (float *) sbs2 + r * (K / 16) + 2 * cc;
                    f[0] = (float) (int16_t) (sv[j] & 0xffffu);
                    f[1] = (float) (int16_t) (sv[j] >> 16);
                } else if constexpr (AF == ACT_Q8_K) {
                    sbs2[r * ns + cc] = (int) (int16_t) (sv[j] & 0xffffu) + (int) (int16_t) (sv[j] >> 16);
                } else {
                    sdx[r * ns + cc] = __builtin_bit_cast(float, sv[j]);
                }
            }
            if (AF == ACT_Q8_K && cc < nd) sdx[r * nd + cc] = dv[j];
        }
    }
}

// grid: x = 16-row group quads, y = expert (grouped) or token chunk of ROWS (dense), z = matrix +
// n_mats * route pass (grouped: routes [ROWS*pass, ROWS*pass+ROWS) of the expert, so hot experts
// spread over blocks). DUAL: each wave computes the same 16 rows of two matrices (w[0] = gate,
// w[1] = up) and stores up * silu(gate) (SwiGLU). The wave's weight units (the gate matrix's, then
// the up matrix's for DUAL) stream through a PF-deep register ring; the first PF are requested right
// behind the first activation staging loads. PF = 1 caps registers for 5 (Q4_K) / 4 (Q8_0) waves per
// SIMD; deeper rings (fewer waves per SIMD) keep more bytes in flight per wave where few blocks are
// resident (the expert matmuls: the touched experts x row-group quads come to under three blocks per
// CU).
// EARLY (a launch whose grid has one pass: every block's rows exist unless its expert is untouched):
// the wave's first PF weight units are requested unconditionally at entry, before the route listing,
// so the weight stream starts under it (an untouched expert's blocks, ~1 in 6 at 16 requests, read
// them for nothing). A conditional entry load would make the compiler wait for it at the branch's join.
template <int WF, bool DUAL, int ROWS, int PF, bool EARLY = false>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(PF > 1 ? m16fmt<WF>::GWPE : m16fmt<WF>::WPE,
                                                                          PF > 1 ? m16fmt<WF>::GWPE : m16fmt<WF>::WPE)))
k_gemv_mfma(GemvArgs a) {
    static_assert(WF != WF_Q6_K || ROWS == 8 || ROWS == 16, "Q6_K: one or two doubled 8-row product sets");
    constexpr int QS = m16fmt<WF>::QS, UB = m16fmt<WF>::BYTES;
    constexpr int AF = wfmt<WF>::ACT;
    extern __shared__ __attribute__((aligned(16))) char smem[];
    __shared__ int s_lds[LIST_MAX];
    __shared__ int s_wcnt[4];
    __shared__ int s_tok[ROWS];
    const int K = a.nsb * 256, KP = K + 16, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g16 = blockIdx.x * 4 + wave;
    const int nm = DUAL ? 1 : a.n_mats;
    const int m = blockIdx.z % nm, pass = blockIdx.z / nm;
    constexpr int ZB = WF == WF_Q6_K ? M16_ZERO : 0;                  // Q6_K: zero bytes, then the rows
    int8_t * sq = (int8_t *) smem + ZB;                              // [ROWS][K+16]
    int * sbs2 = (int *) (smem + ZB + ROWS * KP);                    // Q4_K: [ROWS][K/32] sums of 32; Q6_K: float [ROWS][K/16]
    float * sdx = AF == ACT_Q8_K ? (float *) (sbs2 + ROWS * (K / (WF == WF_Q6_K ? 16 : 32)))  // [ROWS][K/256]
                                 : (float *) (smem + ROWS * KP);     // Q8_0: [ROWS][K/32]
    if (WF == WF_Q6_K && tid < M16_ZERO / 16) ((uint4 *) smem)[tid] = make_uint4(0, 0, 0, 0);
    const int e = a.grouped ? (int) blockIdx.y : 0;
    const bool has = g16 < a.tiles;
    const int nsb = a.nsb, U = (DUAL ? 2 : 1) * nsb;
    const uint4 * ub0 = (const uint4 *) (a.w[DUAL ? 0 : m] + (int64_t) e * a.mat_bytes + (size_t) (has ? g16 : 0) * nsb * UB);
    const uint4 * ub1 = DUAL ? (const uint4 *) (a.w[1] + (int64_t) e * a.mat_bytes + (size_t) (has ? g16 : 0) * nsb * UB) : ub0;
    auto unit_ptr = [&](int u) { return u < nsb ? ub0 + (size_t) u * (UB / 16) : ub1 + (size_t) (u - nsb) * (UB / 16); };
    uint4 pq[PF][QS], ph[PF];
    if constexpr (EARLY) {
#pragma unroll
        for (int j = 0; j < PF; ++j) m16_load<WF>(unit_ptr(j), lane, pq[j], ph[j]);
    }
    int n_items, c0;
    const int32_t * s_list = nullptr;                                // grouped: the expert's routes
    if (a.grouped) {
        s_list = expert_routes(a, e, s_lds, s_wcnt, n_items);
        c0 = pass * ROWS;
    } else {
        n_items = a.n_tok;
        c0 = blockIdx.y * ROWS;
    }
    if (c0 >= n_items) return;
    const int nt = min(ROWS, n_items - c0);
    if (tid < ROWS) {
        int tok = 0;
        if (tid < nt) {
            const int it = a.grouped ? s_list[c0 + tid] : c0 + tid;
            tok = a.grouped && !a.act_by_route ? it / a.k : it;
        }
        s_tok[tid] = tok;
    }
    lds_sync();
    m16_stage_flat<AF, 2, WF == WF_Q6_K>(a.act, nt, [&](int tt) { return s_tok[tt]; }, K, sq, sbs2, sdx, [&]() {
#pragma unroll
        for (int j = 0; j < PF; ++j)
            if (!EARLY && has && j < U) m16_load<WF>(unit_ptr(j), lane, pq[j], ph[j]);
    });
    lds_sync();
    if (!has) return;
    const int q = lane >> 4, row = g16 * 16 + (lane & 15);
    auto store = [&](int t, float v0, float v1) {
        if (t >= nt) return;
        const int it = a.grouped ? s_list[c0 + t] : c0 + t;
        float y = v0;
        if (DUAL) y = v1 * z_silu(v0);
        else if (a.epi == EPI_SOFTCAP) y = z_softcap(y, a.cap);
        else if (a.epi == EPI_ROUTE_W) y = y * a.route_w[it];
        a.out[m][(int64_t) it * a.out_ld + row] = y;
    };
    if constexpr (WF == WF_Q4_K) {
        // at most two token rows (most expert blocks of a decode step): one token pair per product
        auto pairs = [&](auto np) {
            constexpr int NP = decltype(np)::value;
            float p0[NP], p1[NP];
#pragma unroll
            for (int p = 0; p < NP; ++p) p0[p] = p1[p] = 0.0f;
            for (int c = 0; c < U; c += PF) {
#pragma unroll
                for (int j = 0; j < PF; ++j) {
                    const int u = c + j;
                    if (u < U) {
                        float xv[NP], xd[NP];
                        m16_unit_q4k_pairs<NP>(pq[j], ph[j], u < nsb ? u : u - nsb, K, lane, sq, sbs2, sdx, nsb, nt - 1, xv, xd);
                        if (u + PF < U) m16_load<WF>(unit_ptr(u + PF), lane, pq[j], ph[j]);
#pragma unroll
                        for (int p = 0; p < NP; ++p) {
                            if (!DUAL || u < nsb) m16_fold<WF>(p0[p], xv[p], xd[p]);
                            else m16_fold<WF>(p1[p], xv[p], xd[p]);
                        }
                    }
                }
            }
            if (row < a.rows && (q & 1) == 0) {
#pragma unroll
                for (int p = 0; p < NP; ++p) store(2 * p + (q >> 1), p0[p], p1[p]);
            }
        };
        if (nt <= 2) { pairs(std::integral_constant<int, 1>{}); return; }
    }
    float acc0[4] = {0.0f, 0.0f, 0.0f, 0.0f}, acc1[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    // unit u (the gate matrix's units, then the up matrix's for DUAL) sits in ring slot u % PF
    for (int c = 0; c < U; c += PF) {
#pragma unroll
        for (int j = 0; j < PF; ++j) {
            const int u = c + j;
            if (u < U) {
                float t4[4] = {0.0f, 0.0f, 0.0f, 0.0f}, xd[4];
                m16_unit<WF, ROWS>(pq[j], ph[j], u < nsb ? u : u - nsb, K, lane, sq, sbs2, sdx, nsb, nt - 1, t4, xd);
                if (u + PF < U) m16_load<WF>(unit_ptr(u + PF), lane, pq[j], ph[j]);
                if (!DUAL || u < nsb) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) m16_fold<WF>(acc0[i], t4[i], xd[i]);
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) m16_fold<WF>(acc1[i], t4[i], xd[i]);
                }
            }
        }
    }
    if (row < a.rows) {
#pragma unroll
        for (int i = 0; i < 4; ++i) store(4 * q + i, acc0[i], acc1[i]);
    }
}

// Stage nt fp32 rows (LDS row tt = source row tok(tt) of x, stride ld) encoded to Q8_0 in the m16
// staging layout (int8 values [rows][K+16], block scales [rows][K/32]) with k_encode_rows' arithmetic:
// 8 lanes per 32-element block (4 values each), amax by xor lane swaps, d = amax / 127, q = rint(v *
// (127 / amax)), the scale stored as f16(d). At most XF_ITEMS float4 per thread (nt * K / 4 <= 256 *
// XF_ITEMS, host-checked); items past the rows re-read the last one and are not stored. mid() runs
// after the loads are issued.
constexpr int XF_ITEMS = 3;
template <class TokFn, class MidFn>
__device__ __forceinline__ void m16_stage_xf(const float * x, int ld, int nt, TokFn tok, int K, int8_t * sq, float * sdx, MidFn mid) {
    const int tid = threadIdx.x, KP = K + 16, per4 = K / 4, n = nt * per4;
    float4 v[XF_ITEMS];
#pragma unroll
    for (int j = 0; j < XF_ITEMS; ++j) {
        const int i = min(tid + 256 * j, n - 1), r = i / per4, c4 = i - r * per4;
        v[j] = *(const float4 *) (x + (int64_t) tok(r) * ld + 4 * c4);
    }
    mid();
#pragma unroll
    for (int j = 0; j < XF_ITEMS; ++j) {
        const int i = tid + 256 * j, ic = min(i, n - 1), r = ic / per4, c4 = ic - r * per4;
        const float amax = max8_f(fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
        const float dd = amax / 127.0f, id = amax != 0.0f ? 127.0f / amax : 0.0f;
        const int q0 = (int) rintf(v[j].x * id), q1 = (int) rintf(v[j].y * id), q2 = (int) rintf(v[j].z * id), q3 = (int) rintf(v[j].w * id);
        if (i < n) {
            *(uint32_t *) (sq + r * KP + 4 * c4) = (uint32_t) (q0 & 255) | ((uint32_t) (q1 & 255) << 8) |
                                                   ((uint32_t) (q2 & 255) << 16) | ((uint32_t) (q3 & 255) << 24);
            if ((c4 & 7) == 0) sdx[r * (K / 32) + (c4 >> 3)] = h2f(f2h(dd));
        }
    }
}

// m16 GEMV with the K units split over the block's 4 waves: one 16-row group per block (grid x), wave
// w takes units w, w+4, ... (all requested behind the first activation staging loads, so a wave has
// all its weight bytes in flight at once); every unit's values go to LDS and the 4 waves fold them (one token slot each) in superblock order (m16_fold), the
// order of every other Q4_K matmul. Dense: grid (groups, token chunks of ROWS, mats);
// grouped (expert matmuls): grid (groups, experts, passes of ROWS routes), the expert's routes listed
// first so blocks of untouched experts read no weights. Each 16-row group gives 4x more, shorter
// waves than a wave streaming the whole K, which keeps enough bytes in flight to cover HBM latency.
constexpr int SPLIT_UMAX = 4;          // units per wave (U <= 16)
// XF (Q8_0 weights, at most 256 * XF_ITEMS / (K / 4) rows): the activation rows are a.xf's fp32 rows,
// encoded in the staging (m16_stage_xf) rather than read from a.act.
// TP (Q4_K / Q8_0; the launch guarantees at most two token rows per block: at most two tokens): the
// token-pair units (m16_unit_q4k_pairs / m16_unit_q80_pairs) in place of the 16-slot unit.
template <int WF, bool DUAL, int ROWS, bool XF = false, bool TP = false>
__global__ void __launch_bounds__(256) k_gemv_split(GemvArgs a) {
    static_assert(!TP || WF == WF_Q4_K || WF == WF_Q8_0, "token-pair units: Q4_K and Q8_0");
    constexpr int QS = m16fmt<WF>::QS, UB = m16fmt<WF>::BYTES;
    constexpr int AF = wfmt<WF>::ACT;
    extern __shared__ __attribute__((aligned(16))) char smem[];
    __shared__ int s_lds[LIST_MAX];
    __shared__ int s_wcnt[4];
    __shared__ int s_tok[ROWS];
    __shared__ float s_x[4 * SPLIT_UMAX][4][64];                    // [unit][token of the lane][lane]
    static_assert(WF != WF_Q6_K || ROWS == 8 || ROWS == 16, "Q6_K: one or two doubled 8-row product sets");
    const int K = a.nsb * 256, KP = K + 16, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g16 = blockIdx.x;
    constexpr int ZB = WF == WF_Q6_K ? M16_ZERO : 0;                  // Q6_K: zero bytes, then the rows
    int8_t * sq = (int8_t *) smem + ZB;
    int * sbs2 = (int *) (smem + ZB + ROWS * KP);                    // Q4_K: sums of 32; Q6_K: float sums of 16
    float * sdx = AF == ACT_Q8_K ? (float *) (sbs2 + ROWS * (K / (WF == WF_Q6_K ? 16 : 32))) : (float *) (smem + ROWS * KP);
    if (WF == WF_Q6_K && tid < M16_ZERO / 16) ((uint4 *) smem)[tid] = make_uint4(0, 0, 0, 0);
    int e = 0, m = 0, n_items, c0;
    const int32_t * s_list = nullptr;                                // grouped: the expert's routes
    if (a.grouped) {
        e = blockIdx.y;
        s_list = expert_routes(a, e, s_lds, s_wcnt, n_items);
        c0 = blockIdx.z * ROWS;
    } else {
        m = DUAL ? 0 : blockIdx.z;
        n_items = a.n_tok;
        c0 = blockIdx.y * ROWS;
    }
    if (c0 >= n_items) return;
    const int nt = min(ROWS, n_items - c0);
    const int nsb = a.nsb, U = (DUAL ? 2 : 1) * nsb;
    const int64_t eoff = (int64_t) e * a.mat_bytes + (int64_t) g16 * nsb * UB;
    const uint4 * ub0 = (const uint4 *) (a.w[m] + eoff);
    const uint4 * ub1 = DUAL ? (const uint4 *) (a.w[1] + eoff) : ub0;
    auto unit_ptr = [&](int u) { return u < nsb ? ub0 + (size_t) u * (UB / 16) : ub1 + (size_t) (u - nsb) * (UB / 16); };
    uint4 pq[SPLIT_UMAX][QS], ph[SPLIT_UMAX];
    if (tid < ROWS) {
        const int tt = min(tid, nt - 1);
        int tok = c0 + tt;
        if (a.grouped) {
            const int it = s_list[c0 + tt];
            tok = a.act_by_route ? it : it / a.k;
        }
        s_tok[tid] = tok;
    }
    lds_sync();
    auto loads = [&]() {
#pragma unroll
        for (int j = 0; j < SPLIT_UMAX; ++j)
            if (wave + 4 * j < U) m16_load<WF>(unit_ptr(wave + 4 * j), lane, pq[j], ph[j]);
    };
    if constexpr (XF) {
        static_assert(WF == WF_Q8_0, "fp32 rows encoded to Q8_0");
        m16_stage_xf(a.xf, a.xf_ld, nt, [&](int tt) { return s_tok[tt]; }, K, sq, sdx, loads);
    } else {
        m16_stage_flat<AF, 8, WF == WF_Q6_K>(a.act, nt, [&](int tt) { return s_tok[tt]; }, K, sq, sbs2, sdx, loads);
    }
    lds_sync();
    // token pairs: the unit values (lanes with q = 0 and 2) go where the 16-slot unit leaves tokens 0
    // and 1 (slot i = t of lanes 0-15)
    if constexpr (TP) {
#pragma unroll
        for (int j = 0; j < SPLIT_UMAX; ++j) {
            const int u = wave + 4 * j;
            if (u < U) {
                float xv[1], xd[1];
                if constexpr (WF == WF_Q4_K) m16_unit_q4k_pairs<1>(pq[j], ph[j], u < nsb ? u : u - nsb, K, lane, sq, sbs2, sdx, nsb, nt - 1, xv, xd);
                else if constexpr (WF == WF_Q8_0) xv[0] = m16_unit_q80_pairs(pq[j], ph[j], u < nsb ? u : u - nsb, K, lane, sq, sdx, nt - 1);
                if (((lane >> 4) & 1) == 0) s_x[u][lane >> 5][lane & 15] = xv[0];
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < SPLIT_UMAX; ++j) {
            const int u = wave + 4 * j;
            if (u < U) {
                float t4[4] = {0.0f, 0.0f, 0.0f, 0.0f}, xd[4];
                m16_unit<WF, ROWS>(pq[j], ph[j], u < nsb ? u : u - nsb, K, lane, sq, sbs2, sdx, nsb, nt - 1, t4, xd);
#pragma unroll
                for (int i = 0; i < 4; ++i) s_x[u][i][lane] = t4[i];
            }
        }
    }
    lds_sync();
    // wave w folds token slot i = w of the MFMA layout (tokens 4q + w) for the group's 16 rows
    const int q = lane >> 4, row = g16 * 16 + (lane & 15), i = wave;
    if (row >= a.rows) return;
    {
        const int t = 4 * q + i;
        if (t >= nt) return;
        const int it = a.grouped ? s_list[c0 + t] : c0 + t;
        // the units in superblock order (the block scale of the token's superblock sb: Q8_K only)
        float g = 0.0f, up = 0.0f;
        for (int sb = 0; sb < nsb; ++sb) {
            const float xd = AF == ACT_Q8_K ? sdx[t * nsb + sb] : 1.0f;
            m16_fold<WF>(g, s_x[sb][i][lane], xd);
            if (DUAL) m16_fold<WF>(up, s_x[nsb + sb][i][lane], xd);
        }
        float y = g;
        if (DUAL) y = up * z_silu(g);
        else if (a.epi == EPI_SOFTCAP) y = z_softcap(y, a.cap);
        else if (a.epi == EPI_ROUTE_W) y = y * a.route_w[it];
        a.out[m][(int64_t) it * a.out_ld + row] = y;
    }
}

// Row rows[i] of an encoded activation buffer (row stride Kp) copied to row i of dst: the rows of a
// pass that get logits, gathered for the output head. One block per row.
#ifndef Z2H_TEMPLATES_ONLY
__global__ void __launch_bounds__(256) k_gather_act(ActBuf src, ActBuf dst, int Kp, int af, const int32_t * rows) {
    const int i = blockIdx.x, tid = threadIdx.x;
    const int64_t r = rows[i];
    if (af == ACT_F16) {
        for (int j = tid; j < Kp / 8; j += 256) ((uint4 *) (dst.h + (int64_t) i * Kp))[j] = ((const uint4 *) (src.h + r * Kp))[j];
        return;
    }
    for (int j = tid; j < Kp / 16; j += 256) ((uint4 *) (dst.q + (int64_t) i * Kp))[j] = ((const uint4 *) (src.q + r * Kp))[j];
    if (af == ACT_Q8_0) {
        for (int j = tid; j < Kp / 32; j += 256) dst.d32[(int64_t) i * (Kp / 32) + j] = src.d32[r * (Kp / 32) + j];
    } else {
        for (int j = tid; j < Kp / 256; j += 256) dst.d256[(int64_t) i * (Kp / 256) + j] = src.d256[r * (Kp / 256) + j];
        for (int j = tid; j < Kp / 16; j += 256) dst.bs[(int64_t) i * (Kp / 16) + j] = src.bs[r * (Kp / 16) + j];
    }
}
#endif

// Encode fp32 rows x[r][K] (row stride ld) in an activation type: one wave per (row, 256-block),
// same arithmetic as encode_row. Grid: ceil(n_rows * ceil(K/256) / 4) blocks of 256 threads.
struct EncodeArgs { const float * x; int ld, K, n_rows, act_fmt; ActBuf act; };
#ifndef Z2H_TEMPLATES_ONLY
__global__ void __launch_bounds__(256) k_encode_rows(EncodeArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int Kp = kpad(a.K), nb = Kp / 256;
    const int item = blockIdx.x * 4 + wave;
    if (item >= a.n_rows * nb) return;
    const int r = item / nb, b = item % nb;
    const float * x = a.x + (int64_t) r * a.ld + b * 256;
    float v[4];
    if (b * 256 + 256 <= a.K) {
        const float4 f = *(const float4 *) (x + lane * 4);
        v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = b * 256 + lane * 4 + e < a.K ? x[lane * 4 + e] : 0.0f;
    }
    if (a.act_fmt == ACT_Q8_K) {
        q8k_block_v(v, a.act.q + (int64_t) r * Kp + b * 256, a.act.d256 + (int64_t) r * nb + b, a.act.bs + (int64_t) r * (Kp / 16) + b * 16, lane);
    } else if (a.act_fmt == ACT_Q8_0) {
        const float amax = max8_f(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
        const float dd = amax / 127.0f, id = amax != 0.0f ? 127.0f / amax : 0.0f;
        int qi[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) qi[e] = (int) rintf(v[e] * id);
        const uint32_t packed = (uint32_t) (qi[0] & 255) | ((uint32_t) (qi[1] & 255) << 8) |
                                ((uint32_t) (qi[2] & 255) << 16) | ((uint32_t) (qi[3] & 255) << 24);
        *(uint32_t *) (a.act.q + (int64_t) r * Kp + b * 256 + lane * 4) = packed;
        if ((lane & 7) == 0) a.act.d32[(int64_t) r * (Kp / 32) + b * 8 + (lane >> 3)] = h2f(f2h(dd));
    } else {
        uint16_t * h = a.act.h + (int64_t) r * Kp + b * 256 + lane * 4;
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = f2h(v[e]);
    }
}
#endif

// ------------------------------------------------------------------ attention
struct AttnArgs {
    const float * qkvg;      // [T][R] fused projection output
    int R, nh, nkv, hd;
    const float * temp;      // [nh]
    float qk_eps, theta_scale, scale;
    const int32_t * slot_idx, * n_past;
    int T, S;
    uint16_t * kc, * vc;     // this layer's cache [slot][kvh][S][hd]
    float * cap_q, * cap_k, * cap_v, * cap_gate;   // fp32 captures (nullable)
    // partials
    float * part_o;          // [items][grp][hd]
    float * part_ml;         // [items][grp][2]
    float * o_out;           // [T][nh*hd] (combine: gated output, fp32)
    ActBuf act; int act_fmt; // encoding of o_out for W_o
    float * kf, * vf;        // per-slot prefill: this layer's fp32 prompt K/V [nkv][S][hd] (null: f16 cache only)
    int kf_split;            // kf / vf rows hold f16 hi / lo planes ([hd] hi halves, then [hd] lo halves)
    const int4 * tiles;      // k_attn_fa: wide-pass work items (null: decode items located from n_past)
    const float2 * rope;     // [S][hd/2] RoPE (cos, sin) by position and dim pair (k_rope_table)
};

// Wave-parallel item bookkeeping: lane u of each 64-token group loads n_past[u] (and slot_idx[u]) and
// an inclusive scan of the per-token chunk counts locates an item, so the cost is one load per 64
// tokens instead of a chain of dependent loads per token.
__device__ __forceinline__ int wave_scan_incl(int v, int lane) {
    // DPP only: row shifts right by 1, 2, 4, 8 (lanes without a source add 0), then lane 15 of each
    // row into the next row and lane 31 into the upper half
    (void) lane;
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);     // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);     // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);     // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);     // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);     // row_bcast:15 into rows 1, 3
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);     // row_bcast:31 into rows 2, 3
    return v;
}
__device__ __forceinline__ int lane_i(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
// item -> token t (with n_past np and slot), chunk c, kv head g; n_items = all items of the step
__device__ __forceinline__ bool attn_locate(const int32_t * n_past, const int32_t * slot_idx, int T, int nkv, int item,
                                            int & n_items, int & t, int & np, int & slot, int & c, int & g) {
    const int lane = threadIdx.x & 63, want = item / nkv;
    g = item % nkv;
    int base = 0;
    bool found = false;
    for (int t0 = 0; t0 < T; t0 += 64) {
        const int u = t0 + lane;
        const int npu = u < T ? n_past[u] : 0, su = u < T ? slot_idx[u] : 0;
        const int nc = u < T ? (npu + ATT_CH) / ATT_CH : 0;              // chunks of rows [0, n_past]
        const int incl = wave_scan_incl(nc, lane), excl = incl - nc;
        const uint64_t hit = __ballot(!found && want >= base + excl && want < base + incl);
        if (hit) {
            const int l = __ffsll((unsigned long long) hit) - 1;
            t = t0 + l;
            np = lane_i(npu, l);
            slot = lane_i(su, l);
            c = want - base - lane_i(excl, l);
            found = true;
        }
        base += lane_i(incl, 63);
    }
    n_items = base * nkv;
    return found;
}
// At most 64 tokens: lane u's token row (n_past, slot, chunk prefix) read once per block, and a
// persistent block's further items located from those registers (attn_locate's answer, no loads).
struct AttnTok { int npu, su, incl, excl, total; };
__device__ __forceinline__ AttnTok attn_tokens(const int32_t * n_past, const int32_t * slot_idx, int T) {
    const int lane = threadIdx.x & 63;
    AttnTok k;
    k.npu = lane < T ? n_past[lane] : 0;
    k.su = lane < T ? slot_idx[lane] : 0;
    const int nc = lane < T ? (k.npu + ATT_CH) / ATT_CH : 0;
    k.incl = wave_scan_incl(nc, lane);
    k.excl = k.incl - nc;
    k.total = lane_i(k.incl, 63);
    return k;
}
__device__ __forceinline__ bool attn_locate_t(const AttnTok & k, int nkv, int item, int & n_items, int & t, int & np,
                                              int & slot, int & c, int & g) {
    const int want = item / nkv;
    g = item % nkv;
    n_items = k.total * nkv;
    const uint64_t hit = __ballot(want >= k.excl && want < k.incl);
    if (!hit) return false;
    const int l = __ffsll((unsigned long long) hit) - 1;
    t = l;
    np = lane_i(k.npu, l);
    slot = lane_i(k.su, l);
    c = want - lane_i(k.excl, l);
    return true;
}
// chunks before token t (exclusive prefix) and token t's own chunk count
__device__ __forceinline__ void attn_chunks_of(const int32_t * n_past, int T, int t, int & before, int & nc_t) {
    const int lane = threadIdx.x & 63;
    int base = 0;
    before = 0; nc_t = 0;
    for (int t0 = 0; t0 < T && t0 <= t; t0 += 64) {
        const int u = t0 + lane;
        const int nc = u < T ? (n_past[u] + ATT_CH) / ATT_CH : 0;
        const int incl = wave_scan_incl(nc, lane);
        if (t < t0 + 64) {
            before = base + lane_i(incl - nc, t - t0);
            nc_t = lane_i(nc, t - t0);
        }
        base += lane_i(incl, 63);
    }
}

// RoPE angle of the lane's dim pair (lane < HD/2) at position pos: theta = pos * theta_scale^i by
// repeated fp32 multiplication, as the reference's rope_ext does; cs / sn its cosine and sine.
__device__ __forceinline__ void rope_cs(int pos, int pl, float theta_scale, float & cs, float & sn) {
    float th = (float) pos;
    for (int j = 0; j < pl; ++j) th = th * theta_scale;
    z_sincos(th, sn, cs);
}
// The table of rope_cs for every position < S and dim pair < np2 ([S][np2] (cos, sin)), formed once per
// context: the attention kernels read a lane's pair instead of walking its angle chain (up to np2 - 1
// dependent multiplies) per item.
#ifndef Z2H_TEMPLATES_ONLY
__global__ void __launch_bounds__(256) k_rope_table(float2 * out, int S, int np2, float theta_scale) {
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t) S * np2) return;
    float cs, sn;
    rope_cs((int) (i / np2), (int) (i % np2), theta_scale, cs, sn);
    out[i] = make_float2(cs, sn);
}
#endif
// (cos, sin) of dim pair pl at position pos from the table (positions clamped into [0, S))
__device__ __forceinline__ void rope_at(const AttnArgs & a, int pos, int pl, float & cs, float & sn) {
    const float2 v = a.rope[(int64_t) min(max(pos, 0), a.S - 1) * (a.hd / 2) + pl];
    cs = v.x; sn = v.y;
}
// Per-head RMSNorm (one wave, lane = dim pair (x0, x1); lanes past the head hold zeros) times mul,
// then RoPE with the lane's (cs, sn).
template <int HD>
__device__ __forceinline__ void norm_rope(float x0, float x1, float mul, float eps, float cs, float sn, float & y0, float & y1) {
    const double ss = wave_tree_d((double) (x0 * x0) + (double) (x1 * x1));
    const float sc = 1.0f / sqrtf((float) (ss / (double) HD) + eps);
    float z0 = x0 * sc, z1 = x1 * sc;
    if (mul != 1.0f) { z0 = z0 * mul; z1 = z1 * mul; }
    y0 = z0 * cs - z1 * sn;
    y1 = z0 * sn + z1 * cs;
}

// Decode attention with a block of 4 waves per item = (token, ATT_CH-row chunk of its band [0, n_past],
// KV head g). The block requests the chunk's K and V rows with coalesced 16-byte loads and, while
// they are in flight, forms the group's queries from the fused projection output (per-head RMSNorm,
// |temp|, interleaved RoPE with theta = pos * theta_scale^i by repeated fp32 multiplication, read from
// the context's per-position table and requested ahead of the chunk, f16);
// the chunk that holds the new row also forms k and v, puts them in the LDS copy and, with the
// partials after the last barrier (a barrier waits for earlier stores), in the f16 cache. Then every thread scores one (row, head) pair (f16 dot products, fp32 accumulation), one
// wave per head reduces the chunk's softmax partial (max, sum of exp; lane = row), and every thread accumulates
// one (head, dim pair) of the unnormalised P.V over the chunk's rows. k_attn_combine merges chunks.
// head_dim 128 in groups of 4 (the model family's shape) is held to five waves per SIMD (96 VGPRs):
// with K and V sharing the LDS tile (19 KB) that gives five resident blocks per compute unit.
template <int HD, int GRP>
__global__ void __launch_bounds__(256) k_attn_chunk(AttnArgs a) {
    constexpr int NP = HD / 2;                     // dim pairs (<= 64)
    constexpr int RW = HD / 8;                     // uint4 per K / V row
    constexpr int KST = HD + 8;                    // LDS row stride of K (halfs): breaks bank aliasing
    // the chunk's K rows, then (after the scores) its V rows in the same LDS: V waits in registers
    __shared__ __attribute__((aligned(16))) uint16_t s_k[ATT_CH * KST];
    uint16_t * const s_v = s_k;
    __shared__ __attribute__((aligned(16))) uint32_t s_q[GRP][NP];     // f16 pairs
    __shared__ __attribute__((aligned(16))) float s_p[GRP][ATT_CH];     // scores, then weights, by head
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nkv = a.nkv;
    int n_items, t, np, slot, c, g;
    const bool regs = a.T <= 64;                                     // (uniform) items from the token registers
    AttnTok tk{};
    if (regs) tk = attn_tokens(a.n_past, a.slot_idx, a.T);
    bool ok = regs ? attn_locate_t(tk, nkv, blockIdx.x, n_items, t, np, slot, c, g)
                   : attn_locate(a.n_past, a.slot_idx, a.T, nkv, blockIdx.x, n_items, t, np, slot, c, g);
    for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
        if (item != (int) blockIdx.x)
            ok = regs ? attn_locate_t(tk, nkv, item, n_items, t, np, slot, c, g)
                      : attn_locate(a.n_past, a.slot_idx, a.T, nkv, item, n_items, t, np, slot, c, g);
        if (!ok) break;
        const int L = np + 1, r0 = c * ATT_CH, nr = min(ATT_CH, L - r0);
        const bool last = r0 + nr == L;                              // the chunk holds the new row
        const int64_t band = (((int64_t) slot * nkv + g) * a.S + r0) * HD;
        // ---- the projection values this wave normalises (its query heads; wave 3 also the new k and
        // v), requested before the chunk so they arrive first
        const float * row = a.qkvg + (int64_t) t * a.R;
        constexpr int HPW = (GRP + 3) / 4;                           // query heads per wave
        float xq[HPW + 2][2];
#pragma unroll
        for (int j = 0; j < HPW; ++j) {
            const int h = wave + 4 * j;
            const float * src = row + (int64_t) (g * GRP + min(h, GRP - 1)) * HD;
            xq[j][0] = lane < NP ? src[2 * lane] : 0.0f;
            xq[j][1] = lane < NP ? src[2 * lane + 1] : 0.0f;
        }
        const bool mk = last && wave == 3;
        {
            const float * ksrc = row + (int64_t) (a.nh + g) * HD, * vsrc = row + (int64_t) (a.nh + nkv + g) * HD;
            xq[HPW][0] = mk && lane < NP ? ksrc[2 * lane] : 0.0f;
            xq[HPW][1] = mk && lane < NP ? ksrc[2 * lane + 1] : 0.0f;
            xq[HPW + 1][0] = mk && lane < NP ? vsrc[2 * lane] : 0.0f;
            xq[HPW + 1][1] = mk && lane < NP ? vsrc[2 * lane + 1] : 0.0f;
        }
        float cs, sn;                                                // the lane's RoPE pair at np
        rope_at(a, np, min(lane, NP - 1), cs, sn);
        // ---- K and V rows of the chunk, requested now and written to LDS after the query
        // arithmetic (rows past the chunk re-read its last row; the new row, still absent from the
        // cache, is overwritten below)
        constexpr int N4 = ATT_CH * RW;                              // uint4 per matrix
        static_assert(N4 <= 1024, "four 16-byte items per thread and matrix at most");
        // (named registers: an array here is not promoted out of scratch)
        uint4 k0, v0, k1 = {}, v1 = {}, k2 = {}, v2 = {}, k3 = {}, v3 = {};
        auto kv_at = [&](int i, uint4 & kk, uint4 & vv) {           // threads past N4 repeat the last item
            i = min(i, N4 - 1);
            const int r = min(i / RW, nr - 1), q4 = i % RW;
            kk = *(const uint4 *) (a.kc + band + (int64_t) r * HD + 8 * q4);
            vv = *(const uint4 *) (a.vc + band + (int64_t) r * HD + 8 * q4);
        };
        kv_at(tid, k0, v0);
        if constexpr (N4 > 256) kv_at(tid + 256, k1, v1);
        if constexpr (N4 > 512) { kv_at(tid + 512, k2, v2); kv_at(tid + 768, k3, v3); }
        // ---- queries of the group (one wave per head), and the new k / v row (wave 3)
        uint32_t nk = 0, nv = 0;
        {
#pragma unroll
            for (int j = 0; j < HPW; ++j) {
                const int h = wave + 4 * j;
                if (h >= GRP) break;
                const int qh = g * GRP + h;
                float y0, y1;
                norm_rope<HD>(xq[j][0], xq[j][1], a.temp[qh], a.qk_eps, cs, sn, y0, y1);
                if (lane < NP) {
                    s_q[h][lane] = (uint32_t) f2h(y0) | ((uint32_t) f2h(y1) << 16);
                    if (a.cap_q && c == 0) {
                        a.cap_q[((int64_t) t * a.nh + qh) * HD + 2 * lane] = y0;
                        a.cap_q[((int64_t) t * a.nh + qh) * HD + 2 * lane + 1] = y1;
                    }
                }
            }
            if (mk) {
                float k0, k1;
                norm_rope<HD>(xq[HPW][0], xq[HPW][1], 1.0f, a.qk_eps, cs, sn, k0, k1);
                if (lane < NP) {
                    const float v0 = xq[HPW + 1][0], v1 = xq[HPW + 1][1];
                    nk = (uint32_t) f2h(k0) | ((uint32_t) f2h(k1) << 16);
                    nv = (uint32_t) f2h(v0) | ((uint32_t) f2h(v1) << 16);
                    if (a.cap_k) {
                        a.cap_k[((int64_t) t * nkv + g) * HD + 2 * lane] = k0; a.cap_k[((int64_t) t * nkv + g) * HD + 2 * lane + 1] = k1;
                        a.cap_v[((int64_t) t * nkv + g) * HD + 2 * lane] = v0; a.cap_v[((int64_t) t * nkv + g) * HD + 2 * lane + 1] = v1;
                    }
                }
            }
        }
        // the chunk's rows into LDS; where the chunk holds the new row, its slot is written from nk
        // (nv) by wave 3 instead of the stale cache copy
        const int skip = last ? nr - 1 : -1;
        auto k_put = [&](int i, const uint4 & kk) { if (i < N4 && i / RW != skip) *(uint4 *) &s_k[(i / RW) * KST + 8 * (i % RW)] = kk; };
        auto v_put = [&](int i, const uint4 & vv) { if (i < N4 && i / RW != skip) *(uint4 *) &s_v[(i / RW) * HD + 8 * (i % RW)] = vv; };
        k_put(tid, k0);
        if constexpr (N4 > 256) k_put(tid + 256, k1);
        if constexpr (N4 > 512) { k_put(tid + 512, k2); k_put(tid + 768, k3); }
        if (mk && lane < NP) *(uint32_t *) &s_k[(nr - 1) * KST + 2 * lane] = nk;
        lds_sync();                                             // the chunk's K rows are in LDS
        // ---- scores: one (row, head) per thread, an fp32 fma chain over the head dims in order (the
        // f16 x f16 products are exact in fp32, so each step rounds once: one v_fma_mix_f32 each)
        for (int sidx = tid; sidx < ATT_CH * GRP; sidx += 256) {
            const int r = sidx / GRP, h = sidx % GRP;
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < RW; ++j) {
                const uint4 kk = *(const uint4 *) &s_k[r * KST + 8 * j];
                const uint4 qq = *(const uint4 *) &s_q[h][4 * j];
                acc = fma_f16x2(kk.x, qq.x, acc); acc = fma_f16x2(kk.y, qq.y, acc);
                acc = fma_f16x2(kk.z, qq.z, acc); acc = fma_f16x2(kk.w, qq.w, acc);
            }
            s_p[h][r] = r < nr ? acc * a.scale : -__builtin_inff();
        }
        lds_sync();
        // ---- per-head chunk softmax partial (lane = row); (max, sum) stored with the outputs
        float2 ml[(GRP + 3) / 4];
#pragma unroll
        for (int i = 0; i < (GRP + 3) / 4; ++i) {
            const int h = wave + 4 * i;
            if (h >= GRP) break;
            const float sv = lane < ATT_CH ? s_p[h][min(lane, ATT_CH - 1)] : -__builtin_inff();
            const float mx = wave_max_f(sv);
            const float pe = lane < nr ? z_expf(sv - mx) : 0.0f;
            ml[i] = make_float2(mx, wave_tree_f(pe));
            if (lane < ATT_CH) s_p[h][lane] = pe;
        }
        // ---- the chunk's V rows over its K rows (every wave has finished the scores)
        v_put(tid, v0);
        if constexpr (N4 > 256) v_put(tid + 256, v1);
        if constexpr (N4 > 512) { v_put(tid + 512, v2); v_put(tid + 768, v3); }
        if (mk && lane < NP) *(uint32_t *) &s_v[(nr - 1) * HD + 2 * lane] = nv;
        lds_sync();
        // ---- P.V: one (head, dim pair) per thread, rows in order (the weights of 4 rows per LDS read)
        static_assert(ATT_CH % 4 == 0, "weights read 4 rows at a time");
        for (int o = tid; o < GRP * NP; o += 256) {
            const int h = o / NP, dp = o % NP;
            float o0 = 0.0f, o1 = 0.0f;
#pragma unroll 4
            for (int r4 = 0; r4 < ATT_CH; r4 += 4) {
                const float4 p4 = *(const float4 *) &s_p[h][r4];
                const float pv[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t vv = *(const uint32_t *) &s_v[(r4 + j) * HD + 2 * dp];
                    o0 = __builtin_fmaf(pv[j], h2f(vv & 0xffffu), o0);
                    o1 = __builtin_fmaf(pv[j], h2f(vv >> 16), o1);
                }
            }
            *(float2 *) (a.part_o + ((int64_t) item * GRP + h) * HD + 2 * dp) = make_float2(o0, o1);
        }
        if (lane == 0) {
#pragma unroll
            for (int i = 0; i < (GRP + 3) / 4; ++i)
                if (wave + 4 * i < GRP) *(float2 *) (a.part_ml + ((int64_t) item * GRP + wave + 4 * i) * 2) = ml[i];
        }
        if (mk && lane < NP) {                                       // the new row into the cache
            *(uint32_t *) (a.kc + band + (int64_t) (nr - 1) * HD + 2 * lane) = nk;
            *(uint32_t *) (a.vc + band + (int64_t) (nr - 1) * HD + 2 * lane) = nv;
        }
        if (item + (int) gridDim.x < n_items) lds_sync();      // LDS reuse by the next item
    }
}

// Tiles of the per-slot prefill's fp32 attention (k_attn_tile_f32): up to ATT_TILE rows of one slot
// at consecutive positions per 64-row chunk.
constexpr int ATT_TILE = 16;

// K/V append for every token of a prefill chunk before its attention reads them: one wave per
// (token, KV head) forms the new k (per-head RMSNorm, RoPE at n_past) and v rows in f16 exactly as the
// attention kernel does for its new row, and stores them at row n_past of the slot's band.
template <int HD>
__global__ void __launch_bounds__(64) k_kv_append(AttnArgs a) {
    constexpr int NP = HD / 2;
    const int t = blockIdx.x, g = blockIdx.y, lane = threadIdx.x;
    const int np = a.n_past[t], slot = a.slot_idx[t], nkv = a.nkv;
    const float * row = a.qkvg + (int64_t) t * a.R;
    const float * ksrc = row + (int64_t) (a.nh + g) * HD, * vsrc = row + (int64_t) (a.nh + nkv + g) * HD;
    const float x0 = lane < NP ? ksrc[2 * lane] : 0.0f, x1 = lane < NP ? ksrc[2 * lane + 1] : 0.0f;
    const float v0 = lane < NP ? vsrc[2 * lane] : 0.0f, v1 = lane < NP ? vsrc[2 * lane + 1] : 0.0f;
    float cs, sn;
    rope_at(a, np, min(lane, NP - 1), cs, sn);
    float k0, k1;
    norm_rope<HD>(x0, x1, 1.0f, a.qk_eps, cs, sn, k0, k1);
    if (lane < NP) {
        const int64_t at = (((int64_t) slot * nkv + g) * a.S + np) * HD + 2 * lane;
        *(uint32_t *) (a.kc + at) = (uint32_t) f2h(k0) | ((uint32_t) f2h(k1) << 16);
        *(uint32_t *) (a.vc + at) = (uint32_t) f2h(v0) | ((uint32_t) f2h(v1) << 16);
        if (a.kf) {                                                  // the prompt's fp32 rows
            const int64_t af = ((int64_t) g * a.S + np) * HD;
            if (a.kf_split) {                                        // as f16 hi / lo planes in the row's bytes
                uint16_t * kr = (uint16_t *) (a.kf + af), * vr = (uint16_t *) (a.vf + af);
                uint32_t kl, vl;
                const uint32_t kh = f16_split2(k0, k1, kl), vh = f16_split2(v0, v1, vl);
                *(uint32_t *) (kr + 2 * lane) = kh;
                *(uint32_t *) (kr + HD + 2 * lane) = kl;
                *(uint32_t *) (vr + 2 * lane) = vh;
                *(uint32_t *) (vr + HD + 2 * lane) = vl;
            } else {
                *(float2 *) (a.kf + af + 2 * lane) = make_float2(k0, k1);
                *(float2 *) (a.vf + af + 2 * lane) = make_float2(v0, v1);
            }
        }
    }
}

// Per-slot prefill attention with the reference's in-prompt semantics (src/zonos2-graph.cpp:155-169:
// the prompt's K and V stay fp32 for its own causal attention, softmax(K^T q / sqrt(hd)) then V.P):
// k_attn_tile's tiling, item numbering and partial layout, with the chunk's K/V rows read from the
// fp32 prompt rows (a.kf / a.vf, [nkv][S][hd], written by k_kv_append) and fp32 queries; scores and
// P.V are fp32 fma chains over dims / rows in order. k_attn_combine merges the partials unchanged.
// LDS (dynamic): K [64][HD + 4], V [64][HD], per-wave queries [4][GRP][HD] and weights [4][64][GRP].
template <int HD, int GRP>
__global__ void __launch_bounds__(256) k_attn_tile_f32(AttnArgs a, const int4 * __restrict__ tiles) {
    constexpr int NP = HD / 2, KST = HD + 4, N4 = ATT_CH * HD / 4;
    extern __shared__ __attribute__((aligned(16))) float sm_at[];
    float * s_k = sm_at;                                             // [ATT_CH][KST]
    float * s_v = s_k + ATT_CH * KST;                                // [ATT_CH][HD]
    float * s_q = s_v + ATT_CH * HD;                                 // [4][GRP][HD]
    float * s_p = s_q + 4 * GRP * HD;                                // [4][ATT_CH][GRP]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nkv = a.nkv;
    const int4 e = tiles[blockIdx.x];
    const int t0 = e.x, m = e.y & 0xffff, g = e.y >> 16, c = e.z;
    const int p0 = a.n_past[t0];
    const int r0 = c * ATT_CH, nrmax = min(ATT_CH, p0 + m - r0);
    const float * kb = a.kf + ((int64_t) g * a.S + r0) * HD, * vb = a.vf + ((int64_t) g * a.S + r0) * HD;
    {
        // the chunk's rows once (rows past the tile's last one re-read it), every load before a store
        constexpr int PER = (N4 + 255) / 256;
        float4 kk[PER], vv[PER];
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int i = min(tid + 256 * j, N4 - 1), r = min(i / (HD / 4), nrmax - 1), d4 = i % (HD / 4);
            kk[j] = *(const float4 *) (kb + (int64_t) r * HD + 4 * d4);
            vv[j] = *(const float4 *) (vb + (int64_t) r * HD + 4 * d4);
        }
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int i = tid + 256 * j;
            if (i < N4) {
                *(float4 *) &s_k[(i / (HD / 4)) * KST + 4 * (i % (HD / 4))] = kk[j];
                *(float4 *) &s_v[(i / (HD / 4)) * HD + 4 * (i % (HD / 4))] = vv[j];
            }
        }
    }
    lds_sync();
    float * wq = s_q + wave * GRP * HD;
    float * wp = s_p + wave * ATT_CH * GRP;
    int before = e.w;
    for (int i = 0; i < m; ++i) {
        const int np = p0 + i, nc = (np + ATT_CH) / ATT_CH;
        const int64_t item = (int64_t) (before + c) * nkv + g;
        before += nc;
        if ((i & 3) != wave || c >= nc) continue;                    // row i is wave i % 4's; its band may end before c
        const int t = t0 + i, nr = min(ATT_CH, np + 1 - r0);
        {
            const float * row = a.qkvg + (int64_t) t * a.R;
            float cs, sn;
            rope_at(a, np, min(lane, NP - 1), cs, sn);
#pragma unroll
            for (int h = 0; h < GRP; ++h) {
                const int qh = g * GRP + h;
                const float * src = row + (int64_t) qh * HD;
                const float x0 = lane < NP ? src[2 * lane] : 0.0f, x1 = lane < NP ? src[2 * lane + 1] : 0.0f;
                float y0, y1;
                norm_rope<HD>(x0, x1, a.temp[qh], a.qk_eps, cs, sn, y0, y1);
                if (lane < NP) *(float2 *) &wq[h * HD + 2 * lane] = make_float2(y0, y1);
            }
        }
        // scores (lane = chunk row), then the chunk softmax of each head
#pragma unroll
        for (int h = 0; h < GRP; ++h) {
            float acc = 0.0f;
#pragma unroll 8
            for (int d4 = 0; d4 < HD / 4; ++d4) {
                const float4 kk = *(const float4 *) &s_k[lane * KST + 4 * d4];
                const float4 qq = *(const float4 *) &wq[h * HD + 4 * d4];
                acc = __builtin_fmaf(qq.x, kk.x, acc); acc = __builtin_fmaf(qq.y, kk.y, acc);
                acc = __builtin_fmaf(qq.z, kk.z, acc); acc = __builtin_fmaf(qq.w, kk.w, acc);
            }
            const float sv = lane < nr ? acc * a.scale : -__builtin_inff();
            const float mx = wave_max_f(sv);
            const float pe = lane < nr ? z_expf(sv - mx) : 0.0f;
            const float l = wave_tree_f(pe);
            wp[lane * GRP + h] = pe;
            if (lane == 0) *(float2 *) (a.part_ml + (item * GRP + h) * 2) = make_float2(mx, l);
        }
        // P.V: lane = dim pair, rows in order
#pragma unroll
        for (int h = 0; h < GRP; ++h) {
            if (lane >= NP) continue;
            float o0 = 0.0f, o1 = 0.0f;
#pragma unroll 16
            for (int r = 0; r < ATT_CH; ++r) {
                const float2 vv = *(const float2 *) &s_v[r * HD + 2 * lane];
                const float pp = wp[r * GRP + h];
                o0 = __builtin_fmaf(pp, vv.x, o0);
                o1 = __builtin_fmaf(pp, vv.y, o1);
            }
            *(float2 *) (a.part_o + (item * GRP + h) * HD + 2 * lane) = make_float2(o0, o1);
        }
    }
}
__host__ __device__ inline size_t attn_tile_f32_lds(int hd, int grp) {
    return (size_t) 4 * (ATT_CH * (hd + 4) + ATT_CH * hd + 4 * grp * hd + 4 * ATT_CH * grp);
}

// Merge the chunks of HPB query heads of one token and apply the per-head sigmoid gate. grid
// (nh / HPB, T), 8 waves: WPH = 8 / HPB waves per head. Every wave of a head forms the chunk weights
// exp(m_c - M) and the denominator sum_c w_c l_c over all of the token's chunks (lane = chunk); the
// head's first wave keeps the weights in LDS. Wave `part` of a head then sums w_c o_c over chunks
// c = part, part + WPH, ... (lane = dim pair) with 16 partial loads in flight per batch, and the
// WPH partial sums are added in wave order. When the block's HPB * hd outputs cover whole encoding
// blocks the block encodes them for W_o here, otherwise a separate encode pass follows
// (a.act_fmt == ACT_NONE).
constexpr int AM_B = 16;          // partial loads in flight per wave
// HD_ / HPB_ / GRP_: the head size, heads per block and group size known at compile time (0: the
// launch's values), so the index arithmetic of the model family's shape needs no integer divisions.
template <int HD_ = 0, int HPB_ = 0, int GRP_ = 0>
__global__ void __launch_bounds__(512) k_attn_combine(AttnArgs a, int hpb_rt, int ncs) {
    extern __shared__ float sm_ac[];
    const int hd = HD_ ? HD_ : a.hd, hpb = HPB_ ? HPB_ : hpb_rt, nh = a.nh, nkv = a.nkv, grp = GRP_ ? GRP_ : nh / nkv, t = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wph = 8 / hpb, hl = wave / wph, part = wave % wph;
    const int h0 = blockIdx.x * hpb, h = h0 + hl, g = h / grp, hh = h % grp;
    float * ob = sm_ac;                                              // [hpb * hd]
    float * pw = ob + hpb * hd;                                      // [8][hd] per-wave sums
    float * sw = pw + 8 * hd;                                        // [hpb][ncs] chunk weights
    float * sden = sw + hpb * ncs;                                   // [hpb]
    int item0, nc;
    // the gate logit of the thread's output head, requested before the chunk bookkeeping
    const float * gate = a.qkvg + (int64_t) t * a.R + (int64_t) (nh + 2 * nkv) * hd;
    const float gate_x = tid < hpb * hd ? gate[h0 + tid / hd] : 0.0f;
    attn_chunks_of(a.n_past, a.T, t, item0, nc);
    const float2 * __restrict__ ml2 = (const float2 *) a.part_ml;
    const float2 * __restrict__ po2 = (const float2 *) a.part_o;
    // partial (chunk c, this head) index: ((item0 + c) * nkv + g) * grp + hh
    const int64_t pbase = ((int64_t) item0 * nkv + g) * grp + hh, pstep = (int64_t) nkv * grp;
    float2 mr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int c = lane + 64 * j;
        mr[j] = c < nc ? ml2[pbase + c * pstep] : make_float2(-__builtin_inff(), 0.0f);
    }
    float m = fmaxf(fmaxf(mr[0].x, mr[1].x), fmaxf(mr[2].x, mr[3].x));
    for (int c = lane + 256; c < nc; c += 64) m = fmaxf(m, ml2[pbase + c * pstep].x);
    const float M = wave_max_f(m);
    float den = 0.0f;
    float * w = sw + hl * ncs;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int c = lane + 64 * j;
        if (c < nc) {
            const float e = z_expf(mr[j].x - M);
            den = __builtin_fmaf(e, mr[j].y, den);
            if (part == 0) w[c] = e;
        }
    }
    for (int c = lane + 256; c < nc; c += 64) {
        const float2 v = ml2[pbase + c * pstep];
        const float e = z_expf(v.x - M);
        den = __builtin_fmaf(e, v.y, den);
        if (part == 0) w[c] = e;
    }
    den = wave_tree_f(den);
    if (part == 0 && lane == 0) sden[hl] = den;
    lds_sync();
    const int np2 = hd / 2;
    for (int pi = lane; pi < np2; pi += 64) {
        float o0 = 0.0f, o1 = 0.0f;
        for (int c0 = part; c0 < nc; c0 += AM_B * wph) {
            float2 v[AM_B];
#pragma unroll
            for (int j = 0; j < AM_B; ++j) {
                const int c = min(c0 + j * wph, nc - 1);
                v[j] = po2[(pbase + c * pstep) * np2 + pi];
            }
#pragma unroll
            for (int j = 0; j < AM_B; ++j) {
                const int c = c0 + j * wph;
                const float ww = c < nc ? w[c] : 0.0f;
                o0 = __builtin_fmaf(ww, v[j].x, o0);
                o1 = __builtin_fmaf(ww, v[j].y, o1);
            }
        }
        pw[wave * hd + 2 * pi] = o0;
        pw[wave * hd + 2 * pi + 1] = o1;
    }
    lds_sync();
    for (int i = tid; i < hpb * hd; i += 512) {
        const int l = i / hd, dim = i - l * hd;
        float s = 0.0f;
        for (int p = 0; p < wph; ++p) s += pw[(l * wph + p) * hd + dim];
        const float gsig = z_sigmoid(i == tid ? gate_x : gate[h0 + l]);
        if (a.cap_gate && dim == 0) a.cap_gate[(int64_t) t * nh + h0 + l] = gsig;
        ob[i] = s * (gsig / sden[l]);
    }
    lds_sync();
    const int base = h0 * hd, span = hpb * hd;
    for (int i = tid; i < span; i += 512) a.o_out[(int64_t) t * nh * hd + base + i] = ob[i];
    if (a.act_fmt == ACT_NONE || tid >= 256) return;
    // the block's slice [base, base + span) of the token row, encoded in place of the row's blocks
    const int Kp = kpad(nh * hd);
    if (a.act_fmt == ACT_Q8_K)
        encode_row<ACT_Q8_K>(ob, span, a.act.q + (int64_t) t * Kp + base, nullptr,
                             a.act.d256 + (int64_t) t * (Kp / 256) + base / 256, a.act.bs + (int64_t) t * (Kp / 16) + base / 16, nullptr);
    else if (a.act_fmt == ACT_Q8_0)
        encode_row<ACT_Q8_0>(ob, span, a.act.q + (int64_t) t * Kp + base, a.act.d32 + (int64_t) t * (Kp / 32) + base / 32,
                             nullptr, nullptr, nullptr);
    else
        encode_row<ACT_F16>(ob, span, nullptr, nullptr, nullptr, nullptr, a.act.h + (int64_t) t * Kp + base);
}
__host__ __device__ inline size_t attn_combine_lds(int hpb, int hd, int ncs) {
    return (size_t) 4 * (hpb * hd + 8 * hd + hpb * ncs + 8);
}

// ------------------------------------------------------------------ router (exact contract)
struct RouterArgs {
    const float * x;          // [T][d] ffn_in
    int T, d, rd, E, k;
    const float * w_down;     // [rd][d]
    const float * b_down;     // [rd]
    const float * eda;        // [rd] or null
    const float * state_in;   // [T][rd] or null
    float * rh;               // [T][rd] (this layer's state)
    const float * norm_w;     // [rd]
    float eps;
    const float * w0t; const float * b0;   // [rd][rd+4] (rows padded), [rd]
    const float * w2t; const float * b2;
    const float * w4t;                      // [E][rd+4]
    const float * logit_bias;               // [E] or null
    const float * mask;                     // [E] additive 0/-inf or null
    const float * sc_bias;                  // router_bias [E]
    int32_t * sel; float * wsel;            // [T][k]
    float * cap_logits; float * cap_probs;  // [T][E] (nullable)
};

// rh[t][o] = lane-strided fma partials over d + xor butterfly, + bias (+ state * eda).
// grid (ceil(rd/4), T): wave = output row, blockIdx.y = token. All of a lane's loads are issued before
// its fma chain; the chain order (i = lane, lane+64, ... ascending) is the contract's. GUARD: d is
// not a multiple of 64 (lanes past the row's end keep a zero partial).
template <int NI, bool GUARD>   // NI = ceil(d / 64) elements per lane
__global__ void __launch_bounds__(256) k_router_down(RouterArgs a) {
    const int lane = threadIdx.x & 63, o = blockIdx.x * 4 + (threadIdx.x >> 6), t = blockIdx.y;
    if (o >= a.rd) return;
    const float * __restrict__ w = a.w_down + (int64_t) o * a.d + lane;
    const float * __restrict__ x = a.x + (int64_t) t * a.d + lane;
    float wv[NI], xv[NI];
#pragma unroll
    for (int j = 0; j < NI; ++j) {
        const bool in = !GUARD || lane + 64 * j < a.d;
        wv[j] = in ? w[64 * j] : 0.0f;
        xv[j] = in ? x[64 * j] : 0.0f;
    }
    const float b = a.b_down[o];
    const float st = a.eda && a.state_in ? a.state_in[(int64_t) t * a.rd + o] * a.eda[o] : 0.0f;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < NI; ++j)
        if (!GUARD || lane + 64 * j < a.d) acc = __builtin_fmaf(wv[j], xv[j], acc);
    float v = wave_tree_f(acc) + b;
    if (a.eda && a.state_in) v = v + st;
    if (lane == 0) a.rh[(int64_t) t * a.rd + o] = v;
}

// k_router_down for wide passes: the same per-(token, output) fma chain, wave tree, bias and state
// term. A block takes RD_T tokens, whose rows sit in LDS lane-major ([token][lane][j] = x[lane + 64 j],
// rows padded to NI + 4 floats so the lanes' 16-byte reads fall in distinct banks), and 32 outputs:
// wave w forms outputs 32 og + 8 w + [0, 8) in groups of OB, each group's weight rows held in
// registers across the RD_T tokens, so every LDS read of a token's row serves OB independent chains.
// Grid (rd / 32, ceil(T / RD_T)), 256 threads; tokens past T repeat the last row and are not stored.
constexpr int RD_T = 8;
__host__ __device__ inline size_t router_down_t_lds(int ni) { return (size_t) RD_T * 64 * (ni + 4) * 4; }
template <int NI, bool GUARD>
__global__ void __launch_bounds__(256) k_router_down_t(RouterArgs a) {
    static_assert(NI % 4 == 0, "16-byte LDS reads");
    constexpr int S = NI + 4, OB = NI >= 64 ? 2 : 4, PER = RD_T * (NI / 4) * 64 / 256;
    extern __shared__ __attribute__((aligned(16))) float xs_t[];     // [RD_T][64][S]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, t0 = blockIdx.y * RD_T;
    const int nt = min(RD_T, a.T - t0), d = GUARD ? a.d : 64 * NI;
    // staging item (tt, j4, ln): x[lane ln + 64 (4 j4 + c)], c < 4, as one 16-byte LDS store; every
    // load is issued before the first store
    {
        float4 v[PER];
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int idx = tid + 256 * u, ln = idx & 63, j4 = (idx >> 6) % (NI / 4), tt = (idx >> 6) / (NI / 4);
            const float * src = a.x + (int64_t) (t0 + min(tt, nt - 1)) * d + ln + 256 * j4;
            float e[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) e[c] = !GUARD || ln + 64 * (4 * j4 + c) < d ? src[64 * c] : 0.0f;
            v[u] = make_float4(e[0], e[1], e[2], e[3]);
        }
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int idx = tid + 256 * u, ln = idx & 63, j4 = (idx >> 6) % (NI / 4), tt = (idx >> 6) / (NI / 4);
            *(float4 *) (xs_t + (tt * 64 + ln) * S + 4 * j4) = v[u];
        }
    }
    lds_sync();
    const bool eda = a.eda && a.state_in;
#pragma unroll 1
    for (int g = 0; g < 8 / OB; ++g) {
        const int o0 = blockIdx.x * 32 + wave * 8 + g * OB;
        float wv[OB][NI], b[OB];
#pragma unroll
        for (int ob = 0; ob < OB; ++ob) {
            const float * __restrict__ w = a.w_down + (int64_t) (o0 + ob) * d + lane;
#pragma unroll
            for (int j = 0; j < NI; ++j) wv[ob][j] = !GUARD || lane + 64 * j < d ? w[64 * j] : 0.0f;
            b[ob] = a.b_down[o0 + ob];
        }
        // the state terms of the group's (token, output) pairs, lane tt * OB + ob, read back by readlane
        float st_l = 0.0f;
        if (eda && lane < RD_T * OB) {
            const int o = o0 + lane % OB;
            st_l = a.state_in[(int64_t) (t0 + min(lane / OB, nt - 1)) * a.rd + o] * a.eda[o];
        }
#pragma unroll 2
        for (int tt = 0; tt < RD_T; ++tt) {
            const int t = t0 + min(tt, nt - 1);
            const float * xr = xs_t + (tt * 64 + lane) * S;
            float acc[OB];
#pragma unroll
            for (int ob = 0; ob < OB; ++ob) acc[ob] = 0.0f;
#pragma unroll
            for (int j4 = 0; j4 < NI / 4; ++j4) {
                const float4 xv = *(const float4 *) (xr + 4 * j4);
                const float xx[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const int j = 4 * j4 + jj;
                    if (!GUARD || lane + 64 * j < d) {
#pragma unroll
                        for (int ob = 0; ob < OB; ++ob) acc[ob] = __builtin_fmaf(wv[ob][j], xx[jj], acc[ob]);
                    }
                }
            }
#pragma unroll
            for (int ob = 0; ob < OB; ++ob) {
                const float st = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, st_l), tt * OB + ob));
                float v = wave_tree_f(acc[ob]) + b[ob];
                if (eda) v = v + st;
                if (lane == 0 && tt < nt) a.rh[(int64_t) t * a.rd + o0 + ob] = v;
            }
        }
    }
}

// An MoE layer's FFN entry in one launch: residual add, ffn_norm, the activation encoding for the
// expert matmuls and the router down projection. Grid (ceil(rd/4), T), 256 threads. Every block of
// token t forms x = rms_w(res_in + src) with k_resnorm's RN_ADD arithmetic (same element ownership,
// double partial order and scale) into LDS. Wave w then forms router output o = 4 * blockIdx.x + w
// from the LDS row with k_router_down's fma chain, so rh is bit-identical to the two-kernel path; the
// blocks with blockIdx.x == 0 then store the new residual to res_out (never in place: the token's
// other blocks still read res_in), x to cur_out and its encoding, all after the block's only barrier
// (a barrier waits for the stores issued before it). The wave's router weights are requested
// before the row loads.
template <int NI, bool GUARD>
__global__ void __launch_bounds__(256) k_ffn_entry(ResNormArgs f, RouterArgs r) {
    extern __shared__ float xs[];      // [kpad(d)]
    __shared__ double red[4];
    const int t = blockIdx.y, d = f.d, tid = threadIdx.x, lane = tid & 63;
    const int o = blockIdx.x * 4 + (tid >> 6);
    const bool lead = blockIdx.x == 0, has_o = o < r.rd;
    const float * __restrict__ w = r.w_down + (int64_t) (has_o ? o : 0) * d + lane;
    float wv[NI];
#pragma unroll
    for (int j = 0; j < NI; ++j) wv[j] = !GUARD || lane + 64 * j < d ? w[64 * j] : 0.0f;
    const float b = has_o ? r.b_down[o] : 0.0f;
    const bool eda = r.eda && r.state_in;
    const float st = has_o && eda ? r.state_in[(int64_t) t * r.rd + o] * r.eda[o] : 0.0f;
    const float * __restrict__ src = f.src + (int64_t) t * d;
    const float * __restrict__ rin = f.res_in + (int64_t) t * d;
    float4 nw[RN_NV], xv[RN_NV];
#pragma unroll
    for (int j = 0; j < RN_NV; ++j) {
        const int i0 = 4 * (tid + 256 * j);
        if (i0 >= d) continue;
        nw[j] = *(const float4 *) (f.norm_w + i0);
        const float4 x = *(const float4 *) (src + i0), r0 = *(const float4 *) (rin + i0);
        xv[j] = make_float4(x.x + r0.x, x.y + r0.y, x.z + r0.z, x.w + r0.w);
    }
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < RN_NV; ++j)
        if (4 * (tid + 256 * j) < d) ss += (double) (xv[j].x * xv[j].x) + (double) (xv[j].y * xv[j].y) + (double) (xv[j].z * xv[j].z) + (double) (xv[j].w * xv[j].w);
    const double tot = block_sum_d(ss, red);
    const float scale = 1.0f / sqrtf((float) (tot / (double) d) + f.eps);
    float4 hv[RN_NV];                  // the new residual (stored after the barrier)
#pragma unroll
    for (int j = 0; j < RN_NV; ++j) {
        const int i0 = 4 * (tid + 256 * j);
        if (i0 >= d) continue;
        hv[j] = xv[j];
        xv[j] = make_float4((xv[j].x * scale) * nw[j].x, (xv[j].y * scale) * nw[j].y, (xv[j].z * scale) * nw[j].z, (xv[j].w * scale) * nw[j].w);
        *(float4 *) (xs + i0) = xv[j];
    }
    lds_sync();
    if (has_o) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < NI; ++j)
            if (!GUARD || lane + 64 * j < d) acc = __builtin_fmaf(wv[j], xs[lane + 64 * j], acc);
        float v = wave_tree_f(acc) + b;
        if (eda) v = v + st;
        if (lane == 0) r.rh[(int64_t) t * r.rd + o] = v;
    }
    if (!lead) return;
    if (f.act_fmt == ACT_Q8_K && d % 1024 == 0) encode_q8k_regs(xv, d, f.act, t);
    else if (f.act_fmt == ACT_Q8_0 && d % 1024 == 0) encode_q80_regs(xv, d, f.act, t);
    else if (f.act_fmt != ACT_NONE) encode_row_rt(f.act_fmt, xs, d, f.act, t);
#pragma unroll
    for (int j = 0; j < RN_NV; ++j) {
        const int i0 = 4 * (tid + 256 * j);
        if (i0 >= d) continue;
        *(float4 *) (f.res + (int64_t) t * d + i0) = hv[j];
        if (f.cur_out) *(float4 *) (f.cur_out + (int64_t) t * d + i0) = xv[j];
    }
}

// Router tail: RMS norm, the erf-GELU MLP (rd -> rd -> rd -> E), softmax, selection bias, top-k, one
// block per token. An MLP output is the dot of its weight row with the layer input as 8 fmaf partial
// chains over contiguous eighths of the row (partial p sums i = p*rd/8 ... (p+1)*rd/8 - 1 ascending)
// combined by a xor butterfly (4, 2, 1) across the 8 lanes of a lane group; the block's 128 groups
// take one output each (router_dim and E are at most 128), so a lane's chain is NM fmas and four waves
// per SIMD cover each other's latency. Each lane's weights (rows padded to rd + 4 floats) go straight
// from global memory to registers as float4s, all three matrices at entry, so the weight traffic
// overlaps the state load and the norm. The norm and softmax sums are wave trees; top-k ranks each expert
// against all others (score descending, ties to the lower index).
__host__ __device__ inline int pad4(int n) { return (n + 3) & ~3; }
__host__ __device__ inline size_t router_tail_lds(int rd, int E) {
    return (size_t) 4 * (2 * rd + (E <= 64 ? 64 : pad4(E)) + 64);
}

// Router tail blocks: RT_THREADS threads = RT_GROUPS lane groups of 8; lane group g takes outputs
// g + RT_GROUPS u of each MLP layer, lane p of the group the elements [p*NM, p*NM + NM) of each row.
constexpr int RT_THREADS = 1024, RT_GROUPS = RT_THREADS / 8;

// the lane's weights of outputs g + RT_GROUPS u (u < U) of a [n_out][ldw] matrix (rows beyond n_out
// clamp); a wave whose 8 groups all lie past n_out loads nothing (a wave-uniform test, no lane branch)
template <int NM, int U>
__device__ __forceinline__ void rt_load(const float * w, int ldw, int n_out, float4 (&wv)[U][NM / 4]) {
    const int tid = threadIdx.x, g = tid >> 3, p = tid & 7;
    const int g0 = __builtin_amdgcn_readfirstlane(tid >> 6) * 8;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        if (g0 + RT_GROUPS * u < n_out) {
            const float4 * wr = (const float4 *) (w + (int64_t) min(g + RT_GROUPS * u, n_out - 1) * ldw + p * NM);
#pragma unroll
            for (int m = 0; m < NM / 4; ++m) wv[u][m] = wr[m];
        } else {
#pragma unroll
            for (int m = 0; m < NM / 4; ++m) wv[u][m] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    }
}

// p[i] for i < n, else 0, with the load taken by every lane at a clamped index: a load under a lane
// or null-pointer condition becomes a branch, and the join after it waits for every load in flight,
// which would hold back the matrix loads issued after it
__device__ __forceinline__ float ld_or0(const float * p, int i, int n) {
    const float v = p[min(i, n - 1)];
    return i < n ? v : 0.0f;
}
// bias entries of the lane group's outputs g + RT_GROUPS u (u < U; rows beyond n_out clamp); a null b
// reads fb (>= n_out entries) and gives zeros
template <int U>
__device__ __forceinline__ void rt_bias(const float * b, const float * fb, int n_out, float (&bv)[U]) {
    const int g = threadIdx.x >> 3;
    const float * q = b ? b : fb;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const float v = q[min(g + RT_GROUPS * u, n_out - 1)];
        bv[u] = b ? v : 0.0f;
    }
}

// y[o] = post(dot(W[o], x)) for the lane group's outputs g + RT_GROUPS u, u < U (n_out <= RT_GROUPS U);
// MODE 0: gelu(dot + b1[u]); MODE 1: dot (+ b1[u] when has1: logit bias) (+ b2[u] when has2: mask)
// NT > 1: the same for NT token vectors x + n xs -> y + n ys on the same weight registers (each
// token's chain and sums as with NT = 1)
template <int MODE, int NM, int U, int NT = 1>
__device__ __forceinline__ void rt_layer(const float4 (&wv)[U][NM / 4], const float * x, int n_out, float * y,
                                         const float (&b1)[U], const float (&b2)[U], bool has1, bool has2,
                                         int xs = 0, int ys = 0) {
    const int tid = threadIdx.x, g = tid >> 3, p = tid & 7;
    float acc[NT][U];
#pragma unroll
    for (int n = 0; n < NT; ++n) {                 // one token's inputs in registers at a time
        float4 xr[NM / 4];
#pragma unroll
        for (int m = 0; m < NM / 4; ++m) xr[m] = *(const float4 *) (x + n * xs + p * NM + 4 * m);
#pragma unroll
        for (int u = 0; u < U; ++u) acc[n][u] = 0.0f;
#pragma unroll
        for (int m = 0; m < NM / 4; ++m)
#pragma unroll
            for (int u = 0; u < U; ++u) {
                acc[n][u] = __builtin_fmaf(wv[u][m].x, xr[m].x, acc[n][u]);
                acc[n][u] = __builtin_fmaf(wv[u][m].y, xr[m].y, acc[n][u]);
                acc[n][u] = __builtin_fmaf(wv[u][m].z, xr[m].z, acc[n][u]);
                acc[n][u] = __builtin_fmaf(wv[u][m].w, xr[m].w, acc[n][u]);
            }
        // lane p = 0 of the group ends with ((a0 + a4) + (a2 + a6)) + ((a1 + a5) + (a3 + a7)), the xor
        // butterfly's (4, 2, 1) sum, from DPP row shifts (lane i reads lane i + n of its 16-lane row)
#pragma unroll
        for (int u = 0; u < U; ++u) {
            acc[n][u] = acc[n][u] + dpp_f<DPP_ROW_SHL + 4>(acc[n][u]);
            acc[n][u] = acc[n][u] + dpp_f<DPP_ROW_SHL + 2>(acc[n][u]);
            acc[n][u] = acc[n][u] + dpp_f<DPP_ROW_SHL + 1>(acc[n][u]);
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int o = g + RT_GROUPS * u;
        if (o >= n_out) break;
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            float v = acc[n][u];                   // the group's sum (valid in lane p = 0)
            if (MODE == 0) v = z_gelu(v + b1[u]);
            else {
                if (has1) v = v + b1[u];
                if (has2) v = v + b2[u];
            }
            if (p == 0) y[n * ys + o] = v;
        }
    }
}

// softmax (own exp, double tree sum), selection scores and top-k of token t's logits s_l, in wave 0
// (s_y: >= 64 floats of scratch)
__device__ __forceinline__ void router_select(const RouterArgs & a, int t, int E, const float * s_l, float * s_y,
                                              const float (&sb)[4], const float (&mk)[4]) {
    const int lane = threadIdx.x & 63;
    float lg[4], pr[4], sc[4];
    float mx = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = lane + 64 * j;
        lg[j] = e < E ? s_l[e] : -__builtin_inff();
        mx = fmaxf(mx, lg[j]);
    }
    mx = wave_max_f(mx);
    float ex[4];
    double ps = 0.0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = lane + 64 * j;
        ex[j] = e < E ? z_expf(lg[j] - mx) : 0.0f;
        if (e < E) ps += (double) ex[j];
    }
    const float inv = (float) (1.0 / wave_tree_d(ps));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = lane + 64 * j;
        pr[j] = ex[j] * inv;
        sc[j] = pr[j] + sb[j];
        if (a.mask) sc[j] = sc[j] + mk[j];
        if (e < E) {
            if (a.cap_logits) a.cap_logits[(int64_t) t * E + e] = lg[j];
            if (a.cap_probs) a.cap_probs[(int64_t) t * E + e] = pr[j];
        }
    }
    // top-k: expert e's rank = #{e' : s[e'] > s[e] or (s[e'] == s[e] and e' < e)}. The scores go to
    // LDS (padded with -inf, which never outranks a real score) and every lane compares against all.
    float * s_s = s_y;                                                // [>= 64] (free after the MLP)
    const int En = E <= 64 ? 64 : ((E + 3) & ~3);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = lane + 64 * j;
        if (e < En) s_s[e] = e < E ? sc[j] : -__builtin_inff();
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    if (E <= 64) {
        const float me = sc[0];
        int rank = 0;
#pragma unroll
        for (int q4 = 0; q4 < 16; q4 += 4) {                         // 4 float4 of scores at a time
            float4 sv[4];
#pragma unroll
            for (int f = 0; f < 4; ++f) sv[f] = *(const float4 *) (s_s + 4 * (q4 + f));
#pragma unroll
            for (int f = 0; f < 4; ++f) {
                const int f4 = q4 + f;
                const float vv[4] = {sv[f].x, sv[f].y, sv[f].z, sv[f].w};
#pragma unroll
                for (int c = 0; c < 4; ++c) rank += (int) (vv[c] > me) | ((int) (vv[c] == me) & (int) (4 * f4 + c < lane));
            }
        }
        if (lane < E && rank < a.k) {
            a.sel[(int64_t) t * a.k + rank] = lane;
            a.wsel[(int64_t) t * a.k + rank] = pr[0];
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (64 * j >= E) break;
        const int e = lane + 64 * j;
        const float me = sc[j];
        int rank = 0;
        for (int f = 0; f < E; ++f) {
            const float v = s_s[f];
            rank += (int) (v > me) | ((int) (v == me) & (int) (f < e));
        }
        if (e < E && rank < a.k) {
            a.sel[(int64_t) t * a.k + rank] = e;
            a.wsel[(int64_t) t * a.k + rank] = pr[j];
        }
    }
}

// The router tail for router_dim = 8 * NM (<= 128 outputs per layer): token blockIdx.x (LOOP false:
// one block per token, decode steps; wide passes take router_tail_wide) or tokens blockIdx.x,
// blockIdx.x + gridDim.x, ... (LOOP: the three MLP matrices loaded once per block and kept in
// registers). Every global load of the block is issued at entry, the first state row first: the norm
// waits only for it, and the matrices, the biases and the mask arrive while it runs; with LOOP each
// further token's state row is requested a token ahead.
template <int NM, int UE, bool LOOP>
__device__ __forceinline__ void router_tail_body(const RouterArgs & a, float * sm_rt) {
    // per lane: one output of each layer (lane group g takes output g), J state elements (lane + 64j)
    // and JE expert entries (E <= 64 JE) for wave 0's norm and top-k; only these are loaded
    constexpr int UO = 1, J = (8 * NM + 63) / 64, JE = UE;
    const int rd = a.rd, E = a.E;
    float * s_x = sm_rt;                        // [rd]
    float * s_y = s_x + rd;                     // [rd] (then the top-k scores, >= 64 entries)
    float * s_l = s_y + max(rd, 64);            // [E]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float rh_n[J], nw[J], sb[4], mk[4];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int i = lane + 64 * j;
        rh_n[j] = ld_or0(a.rh + (int64_t) blockIdx.x * rd, i, rd);
        nw[j] = ld_or0(a.norm_w, i, rd);
    }
    // the small vectors before the three matrices: loads complete in issue order, so a layer that
    // needs its bias waits only for the loads issued before it (norm_w and sc_bias, never null,
    // stand in for absent rd- and E-sized vectors)
    float b0[UO], b2[UO], blg[UO], bmk[UO];
    rt_bias<UO>(a.b0, a.norm_w, rd, b0);
    rt_bias<UO>(a.b2, a.norm_w, rd, b2);
    rt_bias<UO>(a.logit_bias, a.sc_bias, E, blg);
    rt_bias<UO>(a.mask, a.sc_bias, E, bmk);
    const float * mask_or = a.mask ? a.mask : a.sc_bias;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (j < JE) {
            const int i = lane + 64 * j;
            sb[j] = ld_or0(a.sc_bias, i, E);
            const float m = ld_or0(mask_or, i, E);
            mk[j] = a.mask ? m : 0.0f;
        } else {
            sb[j] = 0.0f; mk[j] = 0.0f;
        }
    }
    const int ldw = rd + 4;
    float4 w0[UO][NM / 4], w2[UO][NM / 4], w4[UO][NM / 4];
    __builtin_amdgcn_sched_barrier(0);
    rt_load<NM, UO>(a.w0t, ldw, rd, w0);
    __builtin_amdgcn_sched_barrier(0);
    rt_load<NM, UO>(a.w2t, ldw, rd, w2);
    __builtin_amdgcn_sched_barrier(0);
    rt_load<NM, UO>(a.w4t, ldw, E, w4);
#pragma unroll 1
    for (int t = blockIdx.x; t < a.T; t += gridDim.x) {
        float rh[J];
#pragma unroll
        for (int j = 0; j < J; ++j) rh[j] = rh_n[j];
        const int tn = t + (int) gridDim.x;
        if (LOOP && tn < a.T) {
#pragma unroll
            for (int j = 0; j < J; ++j) rh_n[j] = ld_or0(a.rh + (int64_t) tn * rd, lane + 64 * j, rd);
        }
        if (LOOP && t != (int) blockIdx.x) lds_sync();  // the previous token's top-k has read s_y
        // router RMS norm: double lane partials (i = lane, lane + 64, ...) + wave tree
        if (wave == 0) {
            double part = 0.0;
#pragma unroll
            for (int j = 0; j < J; ++j) if (lane + 64 * j < rd) part += (double) (rh[j] * rh[j]);
            const double ss = wave_tree_d(part);
            const float scale = 1.0f / sqrtf((float) (ss / (double) rd) + a.eps);
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const int i = lane + 64 * j;
                if (i < rd) s_x[i] = (rh[j] * scale) * nw[j];
            }
        }
        lds_sync();                               // s_x holds the normalised state
        rt_layer<0, NM, UO>(w0, s_x, rd, s_y, b0, b0, false, false);
        lds_sync();
        rt_layer<0, NM, UO>(w2, s_y, rd, s_x, b2, b2, false, false);
        lds_sync();
        rt_layer<1, NM, UO>(w4, s_x, E, s_l, blg, bmk, a.logit_bias != nullptr, a.mask != nullptr);
        lds_sync();
        if (wave == 0) router_select(a, t, E, s_l, s_y, sb, mk);
        if (!LOOP) break;
    }
}

// grid: one block of RT_THREADS per token (decode steps) or up to one per CU with a token loop (LOOP,
// wide passes)
// The router tail for wide passes: tokens t + G n (n < RT_NTOK; G = gridDim.x, t = blockIdx.x +
// RT_NTOK G i) RT_NTOK at a time, the three MLP matrices loaded once per block and kept in registers.
// Each MLP layer forms every token's outputs on the same weight registers (rt_layer<..., RT_NTOK>);
// wave n normalises and selects token n. Every token's arithmetic is router_tail_body's. Dynamic LDS
// router_tail_wide_lds(rd, E).
constexpr int RT_NTOK = 4;
__host__ __device__ inline int rt_el(int E) { return E <= 64 ? 64 : pad4(E); }
__host__ __device__ inline size_t router_tail_wide_lds(int rd, int E) {
    const int sy = rd > rt_el(E) ? rd : rt_el(E);
    return (size_t) 4 * RT_NTOK * (rd + sy + rt_el(E));
}
template <int NM, int UE>
__device__ __forceinline__ void router_tail_wide(const RouterArgs & a, float * sm_rt) {
    constexpr int UO = 1, J = (8 * NM + 63) / 64, JE = UE, NT = RT_NTOK;
    const int rd = a.rd, E = a.E, G = gridDim.x, el = rt_el(E), sy = max(rd, el);
    float * s_x = sm_rt;                        // [NT][rd]
    float * s_y = s_x + NT * rd;                // [NT][sy] (then the top-k scores, el entries)
    float * s_l = s_y + NT * sy;                // [NT][el]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, t0 = blockIdx.x;
    // the state row of the wave's token (waves n < NT: token t + G n; tokens past T read row T - 1)
    const int wn = min(wave, NT - 1);
    float rn[J], nw[J], sb[4], mk[4];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int i = lane + 64 * j;
        rn[j] = ld_or0(a.rh + (int64_t) min(t0 + G * wn, a.T - 1) * rd, i, rd);
        nw[j] = ld_or0(a.norm_w, i, rd);
    }
    float b0[UO], b2[UO], blg[UO], bmk[UO];
    rt_bias<UO>(a.b0, a.norm_w, rd, b0);
    rt_bias<UO>(a.b2, a.norm_w, rd, b2);
    rt_bias<UO>(a.logit_bias, a.sc_bias, E, blg);
    rt_bias<UO>(a.mask, a.sc_bias, E, bmk);
    const float * mask_or = a.mask ? a.mask : a.sc_bias;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (j < JE) {
            const int i = lane + 64 * j;
            sb[j] = ld_or0(a.sc_bias, i, E);
            const float m = ld_or0(mask_or, i, E);
            mk[j] = a.mask ? m : 0.0f;
        } else {
            sb[j] = 0.0f; mk[j] = 0.0f;
        }
    }
    const int ldw = rd + 4;
    float4 w0[UO][NM / 4], w2[UO][NM / 4], w4[UO][NM / 4];
    __builtin_amdgcn_sched_barrier(0);
    rt_load<NM, UO>(a.w0t, ldw, rd, w0);
    __builtin_amdgcn_sched_barrier(0);
    rt_load<NM, UO>(a.w2t, ldw, rd, w2);
    __builtin_amdgcn_sched_barrier(0);
    rt_load<NM, UO>(a.w4t, ldw, E, w4);
#pragma unroll 1
    for (int t = t0; t < a.T; t += NT * G) {
        float rh[J];
#pragma unroll
        for (int j = 0; j < J; ++j) rh[j] = rn[j];
        const int tn = t + NT * G;              // the next group's row of the wave's token
        if (tn < a.T) {
#pragma unroll
            for (int j = 0; j < J; ++j) rn[j] = ld_or0(a.rh + (int64_t) min(tn + G * wn, a.T - 1) * rd, lane + 64 * j, rd);
        }
        if (t != t0) lds_sync();                // the previous group's top-k has read s_y / s_l
        // router RMS norm of the wave's token: double lane partials + wave tree
        if (wave < NT) {
            double part = 0.0;
#pragma unroll
            for (int j = 0; j < J; ++j) if (lane + 64 * j < rd) part += (double) (rh[j] * rh[j]);
            const double ss = wave_tree_d(part);
            const float scale = 1.0f / sqrtf((float) (ss / (double) rd) + a.eps);
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const int i = lane + 64 * j;
                if (i < rd) s_x[wave * rd + i] = (rh[j] * scale) * nw[j];
            }
        }
        lds_sync();
        rt_layer<0, NM, UO, NT>(w0, s_x, rd, s_y, b0, b0, false, false, rd, sy);
        lds_sync();
        rt_layer<0, NM, UO, NT>(w2, s_y, rd, s_x, b2, b2, false, false, sy, rd);
        lds_sync();
        rt_layer<1, NM, UO, NT>(w4, s_x, E, s_l, blg, bmk, a.logit_bias != nullptr, a.mask != nullptr, rd, el);
        lds_sync();
        const int tw = t + G * wave;            // (tokens past T: computed, not stored)
        if (wave < NT && tw < a.T) router_select(a, tw, E, s_l + wave * el, s_y + wave * sy, sb, mk);
    }
}

template <bool LOOP>
__global__ void __launch_bounds__(RT_THREADS) k_router_tail(RouterArgs a) {
    extern __shared__ __attribute__((aligned(16))) float sm_rt[];
    // router_dim in {32, 64, 128}, E <= 128 (host-checked)
#define RT_E(NM_) do { if (LOOP) { if (a.E <= 64) router_tail_wide<NM_, 1>(a, sm_rt); else router_tail_wide<NM_, 2>(a, sm_rt); } \
                       else { if (a.E <= 64) router_tail_body<NM_, 1, false>(a, sm_rt); else router_tail_body<NM_, 2, false>(a, sm_rt); } } while (0)
    switch (a.rd) {
        case 32:  RT_E(4); break;
        case 64:  RT_E(8); break;
        default:  RT_E(16); break;
    }
#undef RT_E
}

// ------------------------------------------------------------------ frame sampler
// Per-column sampling settings (the layout of z2h_sampling).
struct SampleParams { float temperature; int top_k; float top_p; float min_p; float rep_penalty; int rep_codebooks; int greedy; int pad; };
struct SampleArgs {
    const float * logits;             // [n][ncb][av]
    int ncb, av, np2;                 // np2 = power of two >= av (sort width)
    const SampleParams * sp;          // [n]
    const int32_t * hist; const int32_t * hlen; int hcap;   // [n][ncb][hcap] codes, [n][ncb] counts
    const double * u;                 // [n][ncb] canonical draws in [0, 1)
    int32_t * codes;                  // [n][ncb]
};
__host__ __device__ inline size_t sample_lds_bytes(int av, int np2) { return (size_t) np2 * 8 + (size_t) av * 8 + av + 64; }

// One block per (codebook, column), the steps of the reference's sampler (src/zonos2-sampler.cpp:16-77):
// greedy = first maximum of the raw logits; otherwise the repetition penalty (each history occurrence
// once, in order), temperature, candidates = the top_k ids by logit in descending order (or all ids in
// id order), p = exp(l - max) over a double sum, top-p along the probability order, min-p against the
// largest p, and the draw r = u * mass walked along the candidates (no draw is used where the kept
// mass is 0: the code is then the first id of the probability order). The ranking is a bitonic sort
// of (logit descending, id ascending) over np2 entries in LDS; the order-dependent sums (normaliser,
// kept mass, the walk) run in one thread in candidate order, as the reference's loops do. Where equal
// logits or probabilities could change the code, the decisions run again on the exact orders of
// std::partial_sort / std::sort (z2h_order), so the codes are the reference's with ties too.
#ifndef Z2H_TEMPLATES_ONLY
__global__ void __launch_bounds__(256) k_sample(SampleArgs a) {
    extern __shared__ __attribute__((aligned(16))) char sm_s[];
    float * s_key = (float *) sm_s;                              // [np2]
    int * s_idx = (int *) (s_key + a.np2);                       // [np2]
    float * s_lg = (float *) (s_idx + a.np2);                    // [av] penalised / tempered logits by id
    float * s_p = s_lg + a.av;                                   // [av] probabilities by candidate
    uint8_t * s_keep = (uint8_t *) (s_p + a.av);                 // [av]
    __shared__ float s_bv[4]; __shared__ int s_bi[4];
    const int cb = blockIdx.x, col = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int av = a.av, np2 = a.np2;
    const SampleParams sp = a.sp[col];
    const float * in = a.logits + ((size_t) col * a.ncb + cb) * av;
    int32_t * out = a.codes + (size_t) col * a.ncb + cb;
    if (sp.greedy) {                                             // first maximum
        float bv = -__builtin_inff(); int bi = 0x7fffffff;
        for (int j = tid; j < av; j += 256) { const float v = in[j]; if (bi == 0x7fffffff || v > bv) { bv = v; bi = j; } }
        for (int off = 32; off >= 1; off >>= 1) {
            const float ov = __shfl_xor(bv, off, 64); const int oi = __shfl_xor(bi, off, 64);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        if (lane == 0) { s_bv[wave] = bv; s_bi[wave] = bi; }
        __syncthreads();
        if (tid == 0) {
            for (int w = 1; w < 4; ++w) if (s_bv[w] > bv || (s_bv[w] == bv && s_bi[w] < bi)) { bv = s_bv[w]; bi = s_bi[w]; }
            *out = bi;
        }
        return;
    }
    for (int j = tid; j < av; j += 256) s_lg[j] = in[j];
    __syncthreads();
    if (tid == 0 && sp.rep_penalty != 1.0f && cb < sp.rep_codebooks) {
        const int32_t * h = a.hist + ((size_t) col * a.ncb + cb) * a.hcap;
        const int n = min(a.hlen[(size_t) col * a.ncb + cb], a.hcap);
        for (int i = 0; i < n; ++i) {
            const int t = h[i];
            if (t >= 0 && t < av) s_lg[t] = s_lg[t] > 0.0f ? s_lg[t] / sp.rep_penalty : s_lg[t] * sp.rep_penalty;
        }
    }
    __syncthreads();
    for (int j = tid; j < np2; j += 256) {
        float v = -__builtin_inff();
        if (j < av) {
            v = s_lg[j];
            if (sp.temperature > 0.0f) { v = v / sp.temperature; s_lg[j] = v; }
        }
        s_key[j] = v; s_idx[j] = j;
    }
    __syncthreads();
    // bitonic sort, descending by logit, ties to the lower id
    for (int size = 2; size <= np2; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = tid; i < np2 / 2; i += 256) {
                const int lo = 2 * i - (i & (stride - 1)), hi = lo + stride;
                const float kl = s_key[lo], kh = s_key[hi];
                const int il = s_idx[lo], ih = s_idx[hi];
                const bool hi_first = kh > kl || (kh == kl && ih < il);
                const bool desc = (lo & size) == 0;
                if (desc ? hi_first : !hi_first) { s_key[lo] = kh; s_key[hi] = kl; s_idx[lo] = ih; s_idx[hi] = il; }
            }
            __syncthreads();
        }
    const bool topk = sp.top_k > 0 && sp.top_k < av;
    const int n = topk ? sp.top_k : av;
    // candidate j: id s_idx[j] (top-k) or j (all ids); probability-rank r: candidate r (top-k: the
    // logit order is the probability order) or candidate s_idx[r]
    auto cand = [&](int j) { return topk ? s_idx[j] : j; };
    const float mx = s_key[0];
    for (int j = tid; j < n; j += 256) { s_p[j] = z_expf_cr(s_lg[cand(j)] - mx); s_keep[j] = 1; }
    __syncthreads();
    __shared__ double s_z;
    if (tid == 0) { double z = 0.0; for (int j = 0; j < n; ++j) z += (double) s_p[j]; s_z = z; }
    __syncthreads();
    const double z = s_z;
    for (int j = tid; j < n; j += 256) s_p[j] = (float) ((double) s_p[j] / z);
    __syncthreads();
    if (tid != 0) return;
    // The decisions run along two orders: the candidate order (the walk) and the probability order
    // (top-p, the min-p reference, the fallback). Where keys are distinct, the bitonic orders are the
    // reference's. Where equal keys make the reference's order depend on std::partial_sort /
    // std::sort, the position each decision lands on holds the same value in both orders, but it
    // can hold another id. So the first pass flags the cases where an equal-key neighbour could swap
    // the outcome: a top-p cut inside a run of equal probabilities, a fallback whose top probability
    // is shared, or a code whose logit is shared (top-k). Those cases run again on the library's
    // exact orders (z2h_order, one thread).
    const double top_p = sp.top_p > 0.0f && sp.top_p < 1.0f ? (double) sp.top_p : -1.0;
    auto decide = [&](auto cand_at, auto rank_at, bool flag_ties, bool & tie) -> int {
        tie = false;
        if (top_p > 0.0) {
            double c = 0.0; bool reached = false;
            for (int r = 0; r < n; ++r) {
                const int j = rank_at(r);
                if (reached) s_keep[j] = 0;
                c += (double) s_p[j];
                if (!reached && c >= top_p) {
                    reached = true;
                    if (flag_ties && r + 1 < n && s_p[rank_at(r + 1)] == s_p[j]) tie = true;
                }
            }
        }
        const int j0 = rank_at(0);
        if (sp.min_p > 0.0f) {
            const float floor_p = sp.min_p * s_p[j0];
            for (int j = 0; j < n; ++j) if (s_p[j] < floor_p) s_keep[j] = 0;
        }
        double mass = 0.0;
        for (int j = 0; j < n; ++j) mass += s_keep[j] ? (double) s_p[j] : 0.0;
        // equal logits around candidate position j (top-k: the candidate order is the logit order)
        auto shared_logit = [&](int j) {
            return topk && ((j > 0 && s_key[j - 1] == s_key[j]) || (j + 1 < av && s_key[j + 1] == s_key[j]));
        };
        if (mass > 0.0) {
            const double r = a.u[(size_t) col * a.ncb + cb] * (mass - 0.0) + 0.0;
            double acc = 0.0;
            for (int j = 0; j < n; ++j) {
                acc += s_keep[j] ? (double) s_p[j] : 0.0;
                if (acc >= r) {
                    if (flag_ties && shared_logit(j)) tie = true;
                    return cand_at(j);
                }
            }
        }
        if (flag_ties && ((n > 1 && s_p[rank_at(1)] == s_p[j0]) || shared_logit(j0))) tie = true;
        return cand_at(j0);
    };
    bool tie = false;
    int code = decide([&](int j) { return topk ? s_idx[j] : j; }, [&](int r) { return topk ? r : s_idx[r]; }, true, tie);
    if (tie) {
        // the library's orders: ids by logit (std::partial_sort over all ids, first top_k kept), then
        // candidate positions by probability (std::sort); s_key is free now and holds the id arrays
        int * ord = (int *) s_key;
        if (topk) {
            for (int i = 0; i < av; ++i) ord[i] = i;
            z2h_order::partial_order(ord, n, av, [&](int x, int y) { return s_lg[x] > s_lg[y]; });
            for (int j = 0; j < n; ++j) s_idx[j] = ord[j];
        }
        for (int j = 0; j < n; ++j) { ord[j] = j; s_keep[j] = 1; }
        z2h_order::sort_order(ord, n, [&](int x, int y) { return s_p[x] > s_p[y]; });
        code = decide([&](int j) { return topk ? s_idx[j] : j; }, [&](int r) { return ord[r]; }, false, tie);
    }
    *out = code;
}
#endif

// Device-resident step tables for the next step: column i's input frame = its sampled codes + the
// text pad id, and its row n_past + 1 (the slot indices stay).
#ifndef Z2H_TEMPLATES_ONLY
__global__ void __launch_bounds__(64) k_feed(const int32_t * codes, int ncb, int W, int text_pad, int32_t * ids, int32_t * n_past) {
    const int i = blockIdx.x, l = threadIdx.x;
    if (l < W) ids[(int64_t) i * W + l] = l < ncb ? codes[(int64_t) i * ncb + l] : text_pad;
    if (l == 0) n_past[i] = n_past[i] + 1;
}
#endif

// KV rows between the host layout [n][nkv][hd] (staged in device memory) and the cache layout
// [slot][kvh][S][hd]: dir 0 writes the cache, dir 1 reads it into the staging buffer.
#ifndef Z2H_TEMPLATES_ONLY
__global__ void __launch_bounds__(256) k_kv_move(uint4 * stage, uint16_t * cache, int n, int nkv, int hd, int S,
                                                 int row0, int slot, int dir) {
    const int cpr = hd / 8;                                        // 16-byte chunks per head row
    const int64_t total = (int64_t) n * nkv * cpr;
    for (int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t) gridDim.x * 256) {
        const int c = (int) (i % cpr), g = (int) ((i / cpr) % nkv), r = (int) (i / ((int64_t) cpr * nkv));
        uint4 * cp = (uint4 *) (cache + (((int64_t) slot * nkv + g) * S + row0 + r) * hd) + c;
        if (dir == 0) *cp = stage[i];
        else stage[i] = *cp;
    }
}
#endif

// y = up * silu(gate) of one route (or dense token) row, encoded for the down matmul.
struct SwigluArgs {
    const float * g; const float * u; int ff;
    ActBuf act; int act_fmt;
};

#ifndef Z2H_TEMPLATES_ONLY
__global__ void __launch_bounds__(256) k_swiglu_encode(SwigluArgs a) {
    extern __shared__ float sm_sw[];
    const int r = blockIdx.x, tid = threadIdx.x, Kp = kpad(a.ff);
    const float * __restrict__ g = a.g + (int64_t) r * a.ff;
    const float * __restrict__ u = a.u + (int64_t) r * a.ff;
    for (int i = tid; i < Kp; i += 256) sm_sw[i] = i < a.ff ? u[i] * z_silu(g[i]) : 0.0f;
    __syncthreads();
    encode_row_rt(a.act_fmt, sm_sw, a.ff, a.act, r);
}
#endif

} // namespace z2d
