// z2h_kernels.h — gfx950 kernels of one ragged continuous-batching decode step.
//
// Kernel map (reference op -> kernel; src/zonos2-graph.cpp line numbers):
//   k_resnorm        embedding sum (248-260) / emb_norm (300) / residual folds (332, 345, 353) /
//                    rms_w norms (92-95, 343, 347, 354), and the encoding of the normalised row in
//                    the next matmul's activation type (ggml's vec_dot_type conversion)
//   k_gemv<F, S>     every weight matmul: QKV+gate (107-111, fused into one matrix), W_o (175),
//                    expert gate/up and down (mul_mat_id 223-231, grouped by expert from the
//                    top-k selection), dense FFN (179-185), output head + softcap (357-362)
//   k_qkv_post       QK-RMSNorm, |temp|, interleaved RoPE, f16 KV append (113-137), sigmoid gate (107)
//   k_attn_partial   ragged GQA decode attention over the slot's band, split into 64-row chunks (139-153)
//   k_attn_combine   chunk merge, per-head sigmoid gate (173), encoding for W_o
//   k_router_down    EDA router down-projection + state threading (199-203)
//   k_router_tail    router norm, erf-GELU MLP, softmax, bias, top-k, weights (206-220)
//
// Weight layout in HBM ("row-tiled"): a matrix of R rows x K columns is cut into 64-row tiles and
// 256-column units. The bytes of unit (row, u) are split into 16-byte chunks; chunk c of the 64 rows
// of a tile are stored contiguously, so every lane of a wave64 owns one row and each load
// instruction of the wave reads 1 KiB of contiguous HBM. Unit sizes equal the GGUF storage sizes:
//   Q4_K 144 B = 9 chunks (chunk 0 = d,dmin,scales; 1..8 = qs), Q8_0 8 blocks = 17 chunks
//   (0..15 = qs, 16 = the 8 f16 scales), Q6_K 208 B = 13 chunks (ql, qh, scales) + an f16 d plane,
//   F16 512 B = 32 chunks.
#pragma once
#include "z2h_common.h"

namespace z2d {

enum { WF_F16 = 1, WF_Q8_0 = 8, WF_Q4_K = 12, WF_Q6_K = 14 };
enum { ACT_NONE = -1, ACT_F16 = 1, ACT_Q8_0 = 8, ACT_Q8_K = 15 };

constexpr int NT = 16;          // tokens (or routes) per GEMV pass
constexpr int TILE = 64;        // rows per tile = lanes per wave
constexpr int ATT_CH = 64;      // attention rows per chunk
constexpr int MAX_ROUTES = 1024; // top-k routes per step a grouped GEMV can list

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
__device__ __forceinline__ void q8k_block(const float * x, int8_t * q, float * d, int16_t * bs, int lane) {
    float v[4];
    float bax = -1.0f, bval = 0.0f;
    int bidx = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[i] = x[lane * 4 + i];
        const float ax = fabsf(v[i]);
        if (ax > bax) { bax = ax; bval = v[i]; bidx = lane * 4 + i; }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float oax = __shfl_xor(bax, off, WAVE), oval = __shfl_xor(bval, off, WAVE);
        const int oidx = __shfl_xor(bidx, off, WAVE);
        if (oax > bax || (oax == bax && oidx < bidx)) { bax = oax; bval = oval; bidx = oidx; }
    }
    int qi[4];
    if (bax == 0.0f) {
#pragma unroll
        for (int i = 0; i < 4; ++i) qi[i] = 0;
        if (lane == 0) *d = 0.0f;
    } else {
        const float iscale = -127.0f / bval;
#pragma unroll
        for (int i = 0; i < 4; ++i) qi[i] = min(127, (int) rintf(iscale * v[i]));
        if (lane == 0) *d = 1.0f / iscale;
    }
    const uint32_t packed = (uint32_t) (qi[0] & 255) | ((uint32_t) (qi[1] & 255) << 8) |
                            ((uint32_t) (qi[2] & 255) << 16) | ((uint32_t) (qi[3] & 255) << 24);
    *(uint32_t *) (q + lane * 4) = packed;
    int s = qi[0] + qi[1] + qi[2] + qi[3];
    s += __shfl_xor(s, 1, WAVE);
    s += __shfl_xor(s, 2, WAVE);
    if ((lane & 3) == 0) bs[lane >> 2] = (int16_t) s;
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
        for (int b = wave; b < K / 256; b += 4)
            q8k_block(x + 256 * b, q + 256 * b, d256 + b, bs + 16 * b, lane);
    } else if constexpr (AF == ACT_Q8_0) {
        for (int i = tid; i < Kp; i += 256) {         // 64 lanes = two 32-blocks
            const float v = i < K ? x[i] : 0.0f;
            float amax = fabsf(v);
#pragma unroll
            for (int off = 16; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, WAVE));
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

// block-wide double sum (256 threads)
__device__ __forceinline__ double block_sum_d(double v, double * red) {
    v = wave_tree_d(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

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
    const float * emb_in;
    const uint8_t * tab[MAX_TABLES]; int tab_type[MAX_TABLES]; int64_t tab_rows[MAX_TABLES];
    const float * src; int k;         // ACCUM: [T*k][d] routes; ADD / ENCODE: [T][d]
    float * res;                       // [T][d] (ACCUM may pass null: no residual)
    const float * norm_w; float eps;
    float * cur_out;                   // [T][d] fp32 normalised row (nullable)
    ActBuf act; int act_fmt;
    float * cap_x;                     // [T][d] folded FFN output (nullable)
    int * err;
};

__global__ void __launch_bounds__(256) k_resnorm(ResNormArgs a) {
    extern __shared__ float sm_rn[];
    float * xs = sm_rn;                // [d]
    __shared__ double red[4];
    const int t = blockIdx.x, d = a.d, tid = threadIdx.x;
    float * res = a.res ? a.res + (int64_t) t * d : nullptr;
    if (a.mode == RN_EMBED) {
        if (a.emb_in) {
            for (int i = tid; i < d; i += 256) xs[i] = a.emb_in[(int64_t) t * d + i];
        } else {
            for (int i = tid; i < d; i += 256) xs[i] = 0.0f;
            for (int kk = 0; kk < a.W; ++kk) {
                const int id = a.ids[(int64_t) t * a.W + kk];
                if (id < 0 || id >= a.tab_rows[kk]) { if (tid == 0) atomicOr(a.err, 1); continue; }
                const uint8_t * row = a.tab[kk] + (int64_t) id * table_row_bytes(a.tab_type[kk], d);
                for (int i = tid; i < d; i += 256) {
                    const float e = table_elem(row, a.tab_type[kk], i);
                    xs[i] = kk == 0 ? e : xs[i] + e;
                }
            }
        }
        double ss = 0.0;
        for (int i = tid; i < d; i += 256) ss += (double) (xs[i] * xs[i]);
        const double tot = block_sum_d(ss, red);
        const float scale = 1.0f / sqrtf((float) (tot / (double) d) + a.eps);
        for (int i = tid; i < d; i += 256) { const float v = xs[i] * scale; xs[i] = v; res[i] = v; }
    } else if (a.mode == RN_ACCUM) {
        for (int i = tid; i < d; i += 256) {
            const float * s = a.src + ((int64_t) t * a.k) * d + i;
            float x = s[0];
            for (int j = 1; j < a.k; ++j) x = x + s[(int64_t) j * d];
            if (a.cap_x) a.cap_x[(int64_t) t * d + i] = x;
            if (a.res) { const float r = x + res[i]; res[i] = r; xs[i] = r; }
            else xs[i] = x;
        }
    } else if (a.mode == RN_ADD) {
        for (int i = tid; i < d; i += 256) {
            const float r = a.src[(int64_t) t * d + i] + res[i];
            res[i] = r; xs[i] = r;
        }
    } else {
        for (int i = tid; i < d; i += 256) xs[i] = a.src[(int64_t) t * d + i];
    }
    __syncthreads();
    if (a.norm_w) {
        double ss = 0.0;
        for (int i = tid; i < d; i += 256) ss += (double) (xs[i] * xs[i]);
        const double tot = block_sum_d(ss, red);
        const float scale = 1.0f / sqrtf((float) (tot / (double) d) + a.eps);
        for (int i = tid; i < d; i += 256) {
            const float v = (xs[i] * scale) * a.norm_w[i];
            xs[i] = v;
            if (a.cur_out) a.cur_out[(int64_t) t * d + i] = v;
        }
        __syncthreads();
    }
    if (a.act_fmt != ACT_NONE) encode_row_rt(a.act_fmt, xs, d, a.act, t);
}

// ------------------------------------------------------------------ k_gemv
enum { ST_ACT = 0, ST_SWIGLU = 1 };
enum { EPI_STORE = 0, EPI_SOFTCAP = 1, EPI_ROUTE_W = 2 };

struct GemvArgs {
    const uint8_t * w[2];              // tiled weights (matrix m = blockIdx.z)
    const uint16_t * dpl[2];           // Q6_K f16 d plane
    int64_t mat_bytes, dpl_elems;      // per-expert strides
    int nsb, tiles, rows;              // padded K = nsb*256
    int K;                             // real K (SwiGLU staging encodes zeros beyond it)
    // token source
    int grouped;                       // 0: tokens [y*NT, ...) of n_tok; 1: routes with sel == blockIdx.y
    int n_tok;                         // dense token count / grouped: number of tokens T
    const int32_t * sel; int k;        // [T][k]
    ActBuf act;                        // ST_ACT source rows (indexed by token)
    const float * gu_g; const float * gu_u; int ff;   // ST_SWIGLU source rows (indexed by route / token)
    // output
    float * out[2]; int out_ld;        // out[m][row-index][rows]; row-index = token or route
    int epi; float cap; const float * route_w;
    int32_t * cap_counts; int32_t * cap_offsets; int32_t * cap_perm; int E;
};

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
        __syncthreads();
        int off = total;
        for (int w = 0; w < wave; ++w) off += wcount[w];
        if (hit) list[off + before] = r;
        const int add = wcount[0] + wcount[1] + wcount[2] + wcount[3];
        __syncthreads();
        total += add;
    }
    return total;
}

template <int WF>
__device__ __forceinline__ void gemv_unit(const uint4 * __restrict__ u, const uint16_t * dp, int sb, int nsb, int K,
                                          const int8_t * sq, const float * sd32, const float * sd256,
                                          const int16_t * sbs, const uint16_t * sh, int nt, float (&acc)[NT]) {
    constexpr int C = wfmt<WF>::C;
    if constexpr (WF == WF_Q4_K) {
        const uint4 hdr = u[0];
        uint32_t qw[32];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint4 v = u[(c + 1) * TILE];
            qw[4 * c] = v.x; qw[4 * c + 1] = v.y; qw[4 * c + 2] = v.z; qw[4 * c + 3] = v.w;
        }
        const float d = h2f(hdr.x & 0xffffu), dmin = h2f(hdr.x >> 16);
        uint8_t scb[12];
        __builtin_memcpy(scb, &hdr.y, 4); __builtin_memcpy(scb + 4, &hdr.z, 4); __builtin_memcpy(scb + 8, &hdr.w, 4);
        int sc[8], mn[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) q4k_sm(scb, j, sc[j], mn[j]);
        uint32_t lo[32], hi[32];
#pragma unroll
        for (int i = 0; i < 32; ++i) { lo[i] = qw[i] & 0x0f0f0f0fu; hi[i] = (qw[i] >> 4) & 0x0f0f0f0fu; }
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
            if (tt < nt) {
                const int * aq = (const int *) (sq + tt * K + sb * 256);
                int isum[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    const int p = c >> 1, hf = c & 1;
#pragma unroll
                    for (int m = 0; m < 4; ++m) {
                        isum[2 * p]     = sdot4((int) lo[4 * c + m], aq[16 * p + 4 * hf + m], isum[2 * p]);
                        isum[2 * p + 1] = sdot4((int) hi[4 * c + m], aq[16 * p + 8 + 4 * hf + m], isum[2 * p + 1]);
                    }
                }
                int sumi = 0, summ = 0;
                const int16_t * bsr = sbs + tt * (K / 16) + sb * 16;
#pragma unroll
                for (int j = 0; j < 8; ++j) { sumi += sc[j] * isum[j]; summ += mn[j] * ((int) bsr[2 * j] + (int) bsr[2 * j + 1]); }
                const float dx = sd256[tt * nsb + sb];
                acc[tt] += (d * dx) * (float) sumi - (dmin * dx) * (float) summ;
            }
        }
    } else if constexpr (WF == WF_Q6_K) {
        uint32_t ql[32], qh[16];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint4 v = u[c * TILE];
            ql[4 * c] = v.x; ql[4 * c + 1] = v.y; ql[4 * c + 2] = v.z; ql[4 * c + 3] = v.w;
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint4 v = u[(8 + c) * TILE];
            qh[4 * c] = v.x; qh[4 * c + 1] = v.y; qh[4 * c + 2] = v.z; qh[4 * c + 3] = v.w;
        }
        const uint4 scv = u[12 * TILE];
        int8_t sc[16];
        __builtin_memcpy(sc, &scv, 16);
        const float d = h2f(*dp);
        // unsigned 6-bit values of the 4 element groups per (half, l4)
        uint32_t qv[64];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int l4 = 0; l4 < 8; ++l4) {
                const uint32_t L0 = ql[16 * h + l4], L1 = ql[16 * h + 8 + l4], H = qh[8 * h + l4];
                qv[32 * h + l4]      = (L0 & 0x0f0f0f0fu) | ((H & 0x03030303u) << 4);
                qv[32 * h + 8 + l4]  = (L1 & 0x0f0f0f0fu) | (((H >> 2) & 0x03030303u) << 4);
                qv[32 * h + 16 + l4] = ((L0 >> 4) & 0x0f0f0f0fu) | (((H >> 4) & 0x03030303u) << 4);
                qv[32 * h + 24 + l4] = ((L1 >> 4) & 0x0f0f0f0fu) | (((H >> 6) & 0x03030303u) << 4);
            }
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
            if (tt < nt) {
                const int * aq = (const int *) (sq + tt * K + sb * 256);
                const int16_t * bsr = sbs + tt * (K / 16) + sb * 16;
                int sumi = 0;
#pragma unroll
                for (int g = 0; g < 16; ++g) {       // group g: elements 16g..16g+15 = dwords 4g..4g+3
                    int is = 0;
#pragma unroll
                    for (int m = 0; m < 4; ++m) {
                        const int dw = 4 * g + m;    // element dword index within the 256
                        const int h = dw >> 5, r = dw & 31, grp = r >> 3, l4 = r & 7;
                        is = sdot4((int) qv[32 * h + 8 * grp + l4], aq[dw], is);
                    }
                    sumi += (int) sc[g] * (is - 32 * (int) bsr[g]);
                }
                acc[tt] += (d * sd256[tt * nsb + sb]) * (float) sumi;
            }
        }
    } else if constexpr (WF == WF_Q8_0) {
        uint32_t qw[64];
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            const uint4 v = u[c * TILE];
            qw[4 * c] = v.x; qw[4 * c + 1] = v.y; qw[4 * c + 2] = v.z; qw[4 * c + 3] = v.w;
        }
        const uint4 dv = u[16 * TILE];
        uint16_t dh[8];
        __builtin_memcpy(dh, &dv, 16);
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
            if (tt < nt) {
                const int * aq = (const int *) (sq + tt * K + sb * 256);
                const float * dx = sd32 + tt * (K / 32) + sb * 8;
#pragma unroll
                for (int b = 0; b < 8; ++b) {
                    int is = 0;
#pragma unroll
                    for (int m = 0; m < 8; ++m) is = sdot4((int) qw[8 * b + m], aq[8 * b + m], is);
                    acc[tt] += (h2f(dh[b]) * dx[b]) * (float) is;
                }
            }
        }
    } else {   // F16
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
            if (tt < nt) {
                const uint32_t * ah = (const uint32_t *) (sh + tt * K + sb * 256);
                float s = 0.0f;
#pragma unroll 4
                for (int c = 0; c < 32; ++c) {
                    const uint4 v = u[c * TILE];
                    s = fdot2(v.x, ah[4 * c], s); s = fdot2(v.y, ah[4 * c + 1], s);
                    s = fdot2(v.z, ah[4 * c + 2], s); s = fdot2(v.w, ah[4 * c + 3], s);
                }
                acc[tt] += s;
            }
        }
    }
    (void) C; (void) dp; (void) nsb;
}

// LDS budget of k_gemv for activations of K columns (+ SwiGLU staging row)
__host__ __device__ inline size_t gemv_lds_bytes(int act, int K, int stage) {
    size_t b = (size_t) 4 * NT * TILE * 4;                         // reduction buffer
    if (act == ACT_Q8_K) b += (size_t) NT * K + (size_t) NT * (K / 256) * 4 + (size_t) NT * (K / 16) * 2;
    else if (act == ACT_Q8_0) b += (size_t) NT * K + (size_t) NT * (K / 32) * 4;
    else b += (size_t) NT * K * 2;
    if (stage == ST_SWIGLU) b += (size_t) K * 4;
    return b + 64;
}

template <int WF, int STAGE>
__global__ void __launch_bounds__(256) k_gemv(GemvArgs a) {
    constexpr int AF = wfmt<WF>::ACT;
    constexpr int C = wfmt<WF>::C;
    extern __shared__ __attribute__((aligned(16))) char smem[];
    __shared__ int s_list[MAX_ROUTES];
    __shared__ int s_wcnt[4];
    const int K = a.nsb * 256, Kr = a.K, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
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
    float * s_y = (float *) p;                                       // [K] SwiGLU staging

    // which rows (tokens / routes) this block serves
    int n_items, item0 = 0;
    int e = 0;
    if (a.grouped) {
        e = blockIdx.y;
        n_items = build_route_list(a.sel, a.n_tok * a.k, e, s_list, s_wcnt);
        if (a.cap_counts && tile == 0 && m == 0) {                   // grouping capture, one block per expert
            if (tid == 0) a.cap_counts[e] = n_items;
            for (int i = tid; i < n_items; i += 256) {
                int off = 0;
                for (int r = 0; r < a.n_tok * a.k; ++r) off += a.sel[r] < e;
                a.cap_perm[off + i] = s_list[i];
                if (i == 0) a.cap_offsets[e] = off;
            }
            if (n_items == 0 && tid == 0) {
                int off = 0;
                for (int r = 0; r < a.n_tok * a.k; ++r) off += a.sel[r] < e;
                a.cap_offsets[e] = off;
            }
            if (e == a.E - 1 && tid == 0) a.cap_offsets[a.E] = a.n_tok * a.k;
        }
        if (n_items == 0) return;
    } else {
        item0 = blockIdx.y * NT;
        n_items = min(NT, a.n_tok - item0);
        if (n_items <= 0) return;
    }
    const uint8_t * wbase = a.w[m] + (int64_t) e * a.mat_bytes;
    const uint16_t * dbase = WF == WF_Q6_K ? a.dpl[m] + (int64_t) e * a.dpl_elems : nullptr;
    const uint4 * wt = (const uint4 *) wbase + (size_t) tile * a.nsb * C * TILE + lane;

    for (int c0 = 0; c0 < n_items; c0 += NT) {
        const int nt = min(NT, n_items - c0);
        __syncthreads();
        // ---- stage the activation rows of this chunk into LDS
        for (int tt = 0; tt < nt; ++tt) {
            const int it = a.grouped ? s_list[c0 + tt] : item0 + c0 + tt;       // route or token
            if constexpr (STAGE == ST_ACT) {
                const int tok = a.grouped ? it / a.k : it;
                if constexpr (AF == ACT_Q8_K || AF == ACT_Q8_0) {
                    const uint4 * src = (const uint4 *) (a.act.q + (int64_t) tok * K);
                    uint4 * dst = (uint4 *) (sq + tt * K);
                    for (int i = tid; i < K / 16; i += 256) dst[i] = src[i];
                    if constexpr (AF == ACT_Q8_K) {
                        for (int i = tid; i < K / 256; i += 256) sd256[tt * (K / 256) + i] = a.act.d256[(int64_t) tok * (K / 256) + i];
                        for (int i = tid; i < K / 16; i += 256) sbs[tt * (K / 16) + i] = a.act.bs[(int64_t) tok * (K / 16) + i];
                    } else {
                        for (int i = tid; i < K / 32; i += 256) sd32[tt * (K / 32) + i] = a.act.d32[(int64_t) tok * (K / 32) + i];
                    }
                } else {
                    const uint4 * src = (const uint4 *) (a.act.h + (int64_t) tok * K);
                    uint4 * dst = (uint4 *) (sh + tt * K);
                    for (int i = tid; i < K / 8; i += 256) dst[i] = src[i];
                }
            } else {
                // y = up * silu(gate) of this route (graph.cpp:225), then encode for the down matmul
                const float * g = a.gu_g + (int64_t) it * a.ff;
                const float * uu = a.gu_u + (int64_t) it * a.ff;
                __syncthreads();
                for (int i = tid; i < Kr; i += 256) s_y[i] = uu[i] * z_silu(g[i]);
                __syncthreads();
                if constexpr (AF == ACT_Q8_K) encode_row<AF>(s_y, Kr, sq + tt * K, nullptr, sd256 + tt * (K / 256), sbs + tt * (K / 16), nullptr);
                else if constexpr (AF == ACT_Q8_0) encode_row<AF>(s_y, Kr, sq + tt * K, sd32 + tt * (K / 32), nullptr, nullptr, nullptr);
                else encode_row<AF>(s_y, Kr, nullptr, nullptr, nullptr, nullptr, sh + tt * K);
            }
        }
        __syncthreads();
        // ---- each wave: its share of the 256-column units, lane = row of the tile
        float acc[NT];
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) acc[tt] = 0.0f;
        for (int sb = wave; sb < a.nsb; sb += 4) {
            const uint16_t * dp = WF == WF_Q6_K ? dbase + ((size_t) tile * a.nsb + sb) * TILE + lane : nullptr;
            gemv_unit<WF>(wt + (size_t) sb * C * TILE, dp, sb, a.nsb, K, sq, sd32, sd256, sbs, sh, nt, acc);
        }
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) s_red[(wave * NT + tt) * TILE + lane] = acc[tt];
        __syncthreads();
        // ---- reduce the 4 waves (in wave order) and store
        for (int o = tid; o < nt * TILE; o += 256) {
            const int tt = o / TILE, r = o % TILE;
            const float v = ((s_red[(0 * NT + tt) * TILE + r] + s_red[(1 * NT + tt) * TILE + r]) +
                              s_red[(2 * NT + tt) * TILE + r]) + s_red[(3 * NT + tt) * TILE + r];
            const int row = tile * TILE + r;
            if (row >= a.rows) continue;
            const int it = a.grouped ? s_list[c0 + tt] : item0 + c0 + tt;
            float y = v;
            if (a.epi == EPI_SOFTCAP) y = tanhf(v * (1.0f / a.cap)) * a.cap;
            else if (a.epi == EPI_ROUTE_W) y = v * a.route_w[it];
            a.out[m][(int64_t) it * a.out_ld + row] = y;
        }
    }
}

// ------------------------------------------------------------------ attention
struct AttnArgs {
    const float * qkvg;      // [T][R] fused projection output
    int R, nh, nkv, hd;
    const float * temp;      // [nh]
    float qk_eps, theta_scale, scale;
    const int32_t * slot_idx, * n_past;
    int T, S;
    uint16_t * kc, * vc;     // this layer's cache [slot][kvh][S][hd]
    uint16_t * q16;          // [T][nh][hd]
    float * gate;            // [T][nh]
    float * cap_q, * cap_k, * cap_v;   // fp32 captures (nullable)
    // partials
    float * part_o;          // [items][grp][hd]
    float * part_ml;         // [items][grp][2]
    int n_items;             // sum over tokens of chunks, times nkv
    float * o_out;           // [T][nh*hd] (combine: gated output, fp32)
    ActBuf act; int act_fmt; // encoding of o_out for W_o
};

// QK-norm, |temp|, RoPE, KV append, sigmoid gate. One block per token, one wave per head.
__global__ void __launch_bounds__(256) k_qkv_post(AttnArgs a) {
    const int t = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int hd = a.hd, nh = a.nh, nkv = a.nkv;
    const float * row = a.qkvg + (int64_t) t * a.R;
    const int pos = a.n_past[t], slot = a.slot_idx[t];
    for (int h = wave; h < nh + 2 * nkv; h += 4) {
        const bool isq = h < nh, isk = h >= nh && h < nh + nkv;
        const float * src = row + (int64_t) h * hd;          // q heads, then k heads, then v heads
        if (!isq && !isk) {                                  // V: plain f16 store
            const int g = h - nh - nkv;
            uint16_t * dst = a.vc + (((int64_t) slot * nkv + g) * a.S + pos) * hd;
            for (int i = lane; i < hd; i += 64) {
                dst[i] = f2h(src[i]);
                if (a.cap_v) a.cap_v[((int64_t) t * nkv + g) * hd + i] = src[i];
            }
            continue;
        }
        double ss = 0.0;
        for (int i = lane; i < hd; i += 64) ss += (double) (src[i] * src[i]);
        ss = wave_tree_d(ss);
        const float sc = 1.0f / sqrtf((float) (ss / (double) hd) + a.qk_eps);
        const float tmp = isq ? a.temp[h] : 1.0f;
        for (int pi = lane; pi < hd / 2; pi += 64) {
            float x0 = src[2 * pi] * sc, x1 = src[2 * pi + 1] * sc;
            if (isq) { x0 = x0 * tmp; x1 = x1 * tmp; }
            float theta = (float) pos;
            for (int j = 0; j < pi; ++j) theta = theta * a.theta_scale;
            const float cs = cosf(theta), sn = sinf(theta);
            const float y0 = x0 * cs - x1 * sn, y1 = x0 * sn + x1 * cs;
            if (isq) {
                uint16_t * dq = a.q16 + ((int64_t) t * nh + h) * hd;
                dq[2 * pi] = f2h(y0); dq[2 * pi + 1] = f2h(y1);
                if (a.cap_q) { a.cap_q[((int64_t) t * nh + h) * hd + 2 * pi] = y0; a.cap_q[((int64_t) t * nh + h) * hd + 2 * pi + 1] = y1; }
            } else {
                const int g = h - nh;
                uint16_t * dk = a.kc + (((int64_t) slot * nkv + g) * a.S + pos) * hd;
                dk[2 * pi] = f2h(y0); dk[2 * pi + 1] = f2h(y1);
                if (a.cap_k) { a.cap_k[((int64_t) t * nkv + g) * hd + 2 * pi] = y0; a.cap_k[((int64_t) t * nkv + g) * hd + 2 * pi + 1] = y1; }
            }
        }
    }
    // gate = sigmoid(W_g x): the last nh columns of the fused projection
    for (int h = threadIdx.x; h < nh; h += 256)
        a.gate[(int64_t) t * nh + h] = z_sigmoid(row[(int64_t) (nh + 2 * nkv) * hd + h]);
}

// item i -> (token, chunk, kv head): tokens in order, chunks of ATT_CH rows, kv heads innermost
__device__ __forceinline__ bool attn_item(const int32_t * n_past, int T, int nkv, int i, int & t, int & c, int & g) {
    g = i % nkv;
    int rem = i / nkv;
    for (t = 0; t < T; ++t) {
        const int nc = (n_past[t] + 1 + ATT_CH - 1) / ATT_CH;
        if (rem < nc) { c = rem; return true; }
        rem -= nc;
    }
    return false;
}

// One 64-row chunk of one token's band for one KV head and its query-head group.
__global__ void __launch_bounds__(256) k_attn_partial(AttnArgs a) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int hd = a.hd, grp = a.nh / a.nkv, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ldk = hd + 8;                                          // padded f16 row stride
    uint16_t * sk = (uint16_t *) smem;                               // [ATT_CH][ldk]
    uint16_t * sv = sk + ATT_CH * ldk;                               // [ATT_CH][ldk]
    uint16_t * sq = sv + ATT_CH * ldk;                               // [grp][hd]
    float * sp = (float *) (sq + grp * hd + 8);                      // [grp][ATT_CH]
    for (int item = blockIdx.x; item < a.n_items; item += gridDim.x) {
        int t, c, g;
        if (!attn_item(a.n_past, a.T, a.nkv, item, t, c, g)) break;
        const int L = a.n_past[t] + 1, r0 = c * ATT_CH, nr = min(ATT_CH, L - r0);
        const int slot = a.slot_idx[t];
        const uint16_t * kb = a.kc + (((int64_t) slot * a.nkv + g) * a.S + r0) * hd;
        const uint16_t * vb = a.vc + (((int64_t) slot * a.nkv + g) * a.S + r0) * hd;
        __syncthreads();
        const int vpr = hd / 8;                                      // uint4 per row
        for (int i = tid; i < nr * vpr; i += 256) {
            const int r = i / vpr, cc = i % vpr;
            *(uint4 *) (sk + r * ldk + cc * 8) = ((const uint4 *) (kb + (int64_t) r * hd))[cc];
            *(uint4 *) (sv + r * ldk + cc * 8) = ((const uint4 *) (vb + (int64_t) r * hd))[cc];
        }
        for (int i = tid; i < grp * hd; i += 256) sq[i] = a.q16[((int64_t) t * a.nh + g * grp) * hd + i];
        __syncthreads();
        // scores: wave = head of the group (looped), lane = row
        for (int hh = wave; hh < grp; hh += 4) {
            float s = -__builtin_inff();
            if (lane < nr) {
                const uint32_t * kr = (const uint32_t *) (sk + lane * ldk);
                const uint32_t * qr = (const uint32_t *) (sq + hh * hd);
                float acc = 0.0f;
                for (int i = 0; i < hd / 2; ++i) acc = fdot2(kr[i], qr[i], acc);
                s = acc * a.scale;
            }
            const float mx = wave_max_f(s);
            const float pe = lane < nr ? z_expf(s - mx) : 0.0f;
            const float l = wave_tree_f(pe);
            sp[hh * ATT_CH + lane] = pe;
            if (lane == 0) {
                a.part_ml[((int64_t) item * grp + hh) * 2 + 0] = mx;
                a.part_ml[((int64_t) item * grp + hh) * 2 + 1] = l;
            }
        }
        __syncthreads();
        // P.V: wave = head (looped), lane = pair of head dims
        for (int hh = wave; hh < grp; hh += 4) {
            for (int pi = lane; pi < hd / 2; pi += 64) {
                float o0 = 0.0f, o1 = 0.0f;
                for (int r = 0; r < nr; ++r) {
                    const float pr = sp[hh * ATT_CH + r];
                    const uint32_t vv = *(const uint32_t *) (sv + r * ldk + 2 * pi);
                    o0 = __builtin_fmaf(pr, h2f(vv & 0xffffu), o0);
                    o1 = __builtin_fmaf(pr, h2f(vv >> 16), o1);
                }
                float * po = a.part_o + ((int64_t) item * grp + hh) * hd;
                po[2 * pi] = o0; po[2 * pi + 1] = o1;
            }
        }
    }
}

// Merge the chunks of every head of one token, apply the sigmoid gate, encode for W_o.
__global__ void __launch_bounds__(256) k_attn_combine(AttnArgs a) {
    extern __shared__ float sm_ac[];
    const int t = blockIdx.x, hd = a.hd, nh = a.nh, nkv = a.nkv, grp = nh / nkv, tid = threadIdx.x;
    int item0 = 0;
    for (int u = 0; u < t; ++u) item0 += (a.n_past[u] + 1 + ATT_CH - 1) / ATT_CH;
    const int nc = (a.n_past[t] + 1 + ATT_CH - 1) / ATT_CH;
    float * o = sm_ac;                                               // [nh*hd]
    for (int idx = tid; idx < nh * hd; idx += 256) {
        const int h = idx / hd, i = idx % hd, g = h / grp, hh = h % grp;
        float M = -__builtin_inff();
        for (int c = 0; c < nc; ++c) M = fmaxf(M, a.part_ml[((int64_t) ((item0 + c) * nkv + g) * grp + hh) * 2]);
        float den = 0.0f, num = 0.0f;
        for (int c = 0; c < nc; ++c) {
            const int64_t it = (int64_t) (item0 + c) * nkv + g;
            const float w = z_expf(a.part_ml[(it * grp + hh) * 2] - M);
            den = __builtin_fmaf(w, a.part_ml[(it * grp + hh) * 2 + 1], den);
            num = __builtin_fmaf(w, a.part_o[(it * grp + hh) * hd + i], num);
        }
        const float v = (num / den) * a.gate[(int64_t) t * nh + h];
        o[idx] = v;
        if (a.o_out) a.o_out[(int64_t) t * nh * hd + idx] = v;
    }
    __syncthreads();
    encode_row_rt(a.act_fmt, o, nh * hd, a.act, t);
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
    const float * w0t; const float * b0;   // [rd_in][rd_out] (transposed), [rd]
    const float * w2t; const float * b2;
    const float * w4t;                      // [rd][E]
    const float * logit_bias;               // [E] or null
    const float * mask;                     // [E] additive 0/-inf or null
    const float * sc_bias;                  // router_bias [E]
    int32_t * sel; float * wsel;            // [T][k]
    float * cap_logits; float * cap_probs;  // [T][E] (nullable)
};

// rh[t][o] = lane-strided fma partials over d + xor butterfly, + bias (+ state * eda).
__global__ void __launch_bounds__(256) k_router_down(RouterArgs a) {
    const int lane = threadIdx.x & 63, o = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (o >= a.rd) return;
    const float * w = a.w_down + (int64_t) o * a.d;
    for (int t = 0; t < a.T; ++t) {
        const float * x = a.x + (int64_t) t * a.d;
        float acc = 0.0f;
        for (int i = lane; i < a.d; i += 64) acc = __builtin_fmaf(w[i], x[i], acc);
        float v = wave_tree_f(acc) + a.b_down[o];
        if (a.eda && a.state_in) v = v + a.state_in[(int64_t) t * a.rd + o] * a.eda[o];
        if (lane == 0) a.rh[(int64_t) t * a.rd + o] = v;
    }
}

// One wave per token: norm, MLP, softmax, top-k (ties to the lower expert index).
__global__ void __launch_bounds__(64) k_router_tail(RouterArgs a) {
    __shared__ float s_a[512], s_b[512];
    const int t = blockIdx.x, lane = threadIdx.x, rd = a.rd, E = a.E;
    const float * rh = a.rh + (int64_t) t * rd;
    double part = 0.0;
    for (int i = lane; i < rd; i += 64) part += (double) (rh[i] * rh[i]);
    const double ss = wave_tree_d(part);
    const float scale = 1.0f / sqrtf((float) (ss / (double) rd) + a.eps);
    for (int i = lane; i < rd; i += 64) s_a[i] = (rh[i] * scale) * a.norm_w[i];
    __syncthreads();
    for (int o = lane; o < rd; o += 64) {
        float acc = 0.0f;
        for (int i = 0; i < rd; ++i) acc = __builtin_fmaf(a.w0t[(int64_t) i * rd + o], s_a[i], acc);
        s_b[o] = z_gelu(acc + a.b0[o]);
    }
    __syncthreads();
    for (int o = lane; o < rd; o += 64) {
        float acc = 0.0f;
        for (int i = 0; i < rd; ++i) acc = __builtin_fmaf(a.w2t[(int64_t) i * rd + o], s_b[i], acc);
        s_a[o] = z_gelu(acc + a.b2[o]);
    }
    __syncthreads();
    // logits: up to 4 experts per lane (E <= 256)
    float lg[4], ex[4], pr[4], sc[4];
    float mx = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = lane + 64 * j;
        lg[j] = -__builtin_inff();
        if (e < E) {
            float acc = 0.0f;
            for (int i = 0; i < rd; ++i) acc = __builtin_fmaf(a.w4t[(int64_t) i * E + e], s_a[i], acc);
            if (a.logit_bias) acc = acc + a.logit_bias[e];
            if (a.mask) acc = acc + a.mask[e];
            lg[j] = acc;
        }
        mx = fmaxf(mx, lg[j]);
    }
    mx = wave_max_f(mx);
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
        sc[j] = -__builtin_inff();
        if (e < E) {
            sc[j] = pr[j] + a.sc_bias[e];
            if (a.mask) sc[j] = sc[j] + a.mask[e];
            if (a.cap_logits) a.cap_logits[(int64_t) t * E + e] = lg[j];
            if (a.cap_probs) a.cap_probs[(int64_t) t * E + e] = pr[j];
        }
    }
    bool taken[4] = {false, false, false, false};
    for (int j = 0; j < a.k; ++j) {
        float bv = 0.0f; int bi = 0x7fffffff; float bp = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e = lane + 64 * q;
            if (e < E && !taken[q] && (bi == 0x7fffffff || sc[q] > bv)) { bv = sc[q]; bi = e; bp = pr[q]; }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float ov = __shfl_xor(bv, off, WAVE), op = __shfl_xor(bp, off, WAVE);
            const int oi = __shfl_xor(bi, off, WAVE);
            const bool better = oi != 0x7fffffff && (bi == 0x7fffffff || ov > bv || (ov == bv && oi < bi));
            if (better) { bv = ov; bi = oi; bp = op; }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) if (lane + 64 * q == bi) taken[q] = true;
        if (lane == 0) { a.sel[(int64_t) t * a.k + j] = bi; a.wsel[(int64_t) t * a.k + j] = bp; }
    }
}

} // namespace z2d
