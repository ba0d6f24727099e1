// z2h_gemm.h — MFMA GEMMs for the passes with many rows per weight tile: prefill chunks and mixed
// prefill + decode passes (mul_mat / mul_mat_id over a whole batch, src/zonos2-graph.cpp:107-111,
// 175, 179-185, 222-231). A block owns a tile of output rows x GM_T token (or route) rows and reads
// each weight byte of its rows once for all GM_T rows; the activations of the tile are staged in LDS
// one 256-column superblock at a time (double-buffered, the next superblock's loads in flight during
// the current one's products). Grouped launches (experts) take their tiles from the route grouping
// (k_route_sort's offsets and permutation): tile slots are numbered expert by expert, ceil(routes /
// GM_T) per expert, and blocks whose slot is past the last tile exit.
//
//   k_gemm_q4k   Q4_K weights (m16 layout) x Q8_K activations on int8 MFMA (v_mfma_i32_16x16x64_i8).
//                A Q4_K sub-block's 6-bit scale sc is split as 8 * (sc >> 3) + (sc & 7); the weights'
//                4-bit values times each part stay below 106, so two int8 products over the whole
//                superblock give sum_j sc_j * dot_j = 8 * hi + lo exactly, with no per-sub-block
//                scaling of MFMA results. The min term sum_j m_j * bsum_j (bsum = the activation's
//                sum over sub-block j) is one f16 MFMA on exact operands (bsum split as 64 * hi + lo),
//                exact in fp32. Per superblock: acc = fma(dx, fma(d, isum, -dmin * msum), acc), the
//                fold of the Q4_K GEMVs, so a row's result is the same bits at any batch width.
//   k_gemm_f16   F16 weights (t64 layout) x f16 activations on v_mfma_f32_16x16x32_f16, fp32
//                accumulation; the weight fragments stream straight from HBM into a register ring of
//                32-column steps. Every F16 matmul (decode widths too) runs on it.
#pragma once
#include "z2h_kernels.h"

namespace z2d {

constexpr int GM_T = 64;                 // token (route) rows per block tile
constexpr int GM_QP = 256 + 8;           // LDS pitch of a row's int8 superblock (bytes): 66 dwords, so the
                                         // 8-byte A reads of 16 rows fall in distinct banks
constexpr int GM_SP = 10;                // LDS pitch (dwords) of a row's 8 sub-block sum pairs (same reason)
constexpr int GM_HP = 256 + 8;           // LDS pitch of a row's f16 superblock (halves)

typedef _Float16 v4h_t __attribute__((ext_vector_type(4)));
typedef _Float16 v8h_t __attribute__((ext_vector_type(8)));
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

struct GemmArgs {
    const uint8_t * w[2];              // DUAL: gate, up (same layout); else w[0]
    int64_t mat_bytes;                 // per-expert stride of a matrix
    int nsb, rows, tiles;              // K = 256 * nsb; output rows; 16-row groups (m16) / 64-row tiles (t64)
    int grouped, n_tok, k, E, act_by_route;
    const int32_t * r_off, * r_perm;   // grouped: route offsets by expert [E+1], routes in expert order
    ActBuf act;
    float * out; int out_ld;           // out[row-index][rows]; row-index = token (dense) or route
    int epi; float cap; const float * route_w;
};

// Block tiles of GT rows in a launch (grid y): dense ceil(n_tok / GT); grouped at most
// ceil(routes / GT) + E.
__host__ __device__ inline int gemm_slots(int grouped, int n_tok, int k, int E, int GT) {
    return grouped ? (n_tok * k + GT - 1) / GT + E : (n_tok + GT - 1) / GT;
}

// The block's tile of up to GT rows: dense rows [c0, c0 + nt), or routes [c0, c0 + nt) of expert e
// in expert order. Every wave computes the same answer (no LDS); false for slots past the last tile.
template <int GT>
__device__ __forceinline__ bool gemm_tile(const GemmArgs & a, int slot, int & e, int & c0, int & nt) {
    e = 0;
    if (!a.grouped) {
        c0 = slot * GT;
        nt = min(GT, a.n_tok - c0);
        return nt > 0;
    }
    const int lane = threadIdx.x & 63;
    int base = 0;
    for (int e0 = 0; e0 < a.E; e0 += 64) {
        const int ee = e0 + lane;
        const int cnt = ee < a.E ? a.r_off[ee + 1] - a.r_off[ee] : 0;
        const int nte = (cnt + GT - 1) / GT;
        const int incl = wave_scan_incl(nte, lane);
        const int tot = __builtin_amdgcn_readlane(incl, 63);
        if (slot < base + tot) {
            const uint64_t hit = __ballot(slot < base + incl);
            const int l = (int) __ffsll((unsigned long long) hit) - 1;
            e = e0 + l;
            const int first = base + __builtin_amdgcn_readlane(incl, l) - __builtin_amdgcn_readlane(nte, l);
            c0 = (slot - first) * GT;
            nt = min(GT, __builtin_amdgcn_readlane(cnt, l) - c0);
            return true;
        }
        base += tot;
    }
    return false;
}

// Tile rows -> activation rows (s_row, the last valid row repeated past nt) and output row indices.
template <int GT>
__device__ __forceinline__ void gemm_rows(const GemmArgs & a, int e, int c0, int nt, int * s_row, int * s_out) {
    const int tid = threadIdx.x;
    if (tid < GT) {
        const int t = min(tid, nt - 1);
        const int it = a.grouped ? a.r_perm[a.r_off[e] + c0 + t] : c0 + t;
        s_out[tid] = it;
        s_row[tid] = a.grouped && !a.act_by_route ? it / a.k : it;
    }
}

__device__ __forceinline__ float gemm_epi(const GemmArgs & a, float y, int it) {
    if (a.epi == EPI_SOFTCAP) return z_softcap(y, a.cap);
    if (a.epi == EPI_ROUTE_W) return y * a.route_w[it];
    return y;
}

// ------------------------------------------------------------------ Q4_K x Q8_K
// One superblock of GM_T activation rows in registers (GM_T / 16 x 16 B of values, GM_T / 32 sub-block
// sum pairs and the block scale per thread), then in LDS: values [GM_T][GM_QP], sums as f16 pairs
// (hi, lo) with sum = 64 * hi + lo [GM_T][GM_SP], scales [GM_T].
struct GmQ8K { u32x4 v[GM_T / 16]; uint32_t s[GM_T / 32]; float dx; };

__device__ __forceinline__ void gm_load_q8k(GmQ8K & st, const ActBuf & act, int K, int sb, const int * s_row) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int j = 0; j < GM_T / 16; ++j) {
        const int i = tid + 256 * j, r = i >> 4, c = i & 15;
        st.v[j] = *(const u32x4 *) (act.q + (int64_t) s_row[r] * K + sb * 256 + c * 16);
    }
#pragma unroll
    for (int j = 0; j < GM_T / 32; ++j) {
        const int i = tid + 256 * j, r = i >> 3, jj = i & 7;
        st.s[j] = *(const uint32_t *) (act.bs + (int64_t) s_row[r] * (K / 16) + sb * 16 + 2 * jj);
    }
    st.dx = act.d256[(int64_t) s_row[tid & (GM_T - 1)] * (K / 256) + sb];
}

__device__ __forceinline__ void gm_store_q8k(const GmQ8K & st, int8_t * sq, uint32_t * ss, float * sdx) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int j = 0; j < GM_T / 16; ++j) {
        const int i = tid + 256 * j, r = i >> 4, c = i & 15;
        uint2 * dst = (uint2 *) (sq + r * GM_QP + c * 16);            // 8-byte aligned rows
        dst[0] = make_uint2(st.v[j].x, st.v[j].y);
        dst[1] = make_uint2(st.v[j].z, st.v[j].w);
    }
#pragma unroll
    for (int j = 0; j < GM_T / 32; ++j) {
        const int i = tid + 256 * j;
        const int s = (int) (int16_t) (st.s[j] & 0xffffu) + (int) (int16_t) (st.s[j] >> 16);   // |s| <= 32 * 128
        const _Float16 hi = (_Float16) (s >> 6), lo = (_Float16) (s & 63);
        ss[(i >> 3) * GM_SP + (i & 7)] = (uint32_t) __builtin_bit_cast(uint16_t, hi) | ((uint32_t) __builtin_bit_cast(uint16_t, lo) << 16);
    }
    if (tid < GM_T) sdx[tid] = st.dx;
}

// The B operands of one m16 unit (16 rows x 256 columns) for the lane's row and k-slice: for each
// pair of sub-blocks (2s, 2s+1) the 16 weight values times the high and the low part of their
// sub-block scales, the f16 operand of the min term, and the row's d / dmin.
struct GmQ4Unit { v4i_t bh[4], bl[4]; v4h_t bm; float d, dmin; };

__device__ __forceinline__ uint32_t gm_mul_bytes(uint32_t x, uint32_t s) {
    // four byte lanes (each <= 15) times s <= 7: two 16-bit products per half, no carry across bytes
    const u16x2_t r = __builtin_bit_cast(u16x2_t, x) * (u16x2_t) {(unsigned short) s, (unsigned short) s};
    return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ void gm_prep_q4k(const uint4 & q0, const uint4 & q1, const uint4 & hd, int lane, GmQ4Unit & u) {
    const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    // 6-bit scales / mins of sub-blocks 0-3 and 4-7 (GGUF K-quant packing)
    const uint32_t sc03 = hd.y & 0x3f3f3f3fu;
    const uint32_t sc47 = (hd.w & 0x0f0f0f0fu) | ((hd.y >> 2) & 0x30303030u);
    const uint32_t mn03 = hd.z & 0x3f3f3f3fu;
    const uint32_t mn47 = ((hd.w >> 4) & 0x0f0f0f0fu) | ((hd.z >> 2) & 0x30303030u);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const uint32_t sc = s < 2 ? sc03 : sc47;
        const int j0 = 2 * (s & 1);                                  // byte of sub-block 2s in sc
        const uint32_t h0 = (sc >> (8 * j0 + 3)) & 7u, l0 = (sc >> (8 * j0)) & 7u;
        const uint32_t h1 = (sc >> (8 * j0 + 11)) & 7u, l1 = (sc >> (8 * j0 + 8)) & 7u;
        const uint32_t a0 = w[2 * s] & 0x0f0f0f0fu, a1 = w[2 * s + 1] & 0x0f0f0f0fu;              // sub-block 2s
        const uint32_t b0 = (w[2 * s] >> 4) & 0x0f0f0f0fu, b1 = (w[2 * s + 1] >> 4) & 0x0f0f0f0fu;  // sub-block 2s+1
        u.bh[s] = (v4i_t) {(int) gm_mul_bytes(a0, h0), (int) gm_mul_bytes(a1, h0), (int) gm_mul_bytes(b0, h1), (int) gm_mul_bytes(b1, h1)};
        u.bl[s] = (v4i_t) {(int) gm_mul_bytes(a0, l0), (int) gm_mul_bytes(a1, l0), (int) gm_mul_bytes(b0, l1), (int) gm_mul_bytes(b1, l1)};
    }
    const int q = lane >> 4;
    const uint32_t mm = (q < 2 ? mn03 : mn47) >> (16 * (q & 1));
    const float ma = (float) (mm & 0xffu), mb = (float) ((mm >> 8) & 0xffu);
    u.bm = (v4h_t) {(_Float16) (64.0f * ma), (_Float16) ma, (_Float16) (64.0f * mb), (_Float16) mb};
    u.d = h2f(hd.x & 0xffffu);
    u.dmin = h2f(hd.x >> 16);
}

// grid: x = row blocks (DUAL: 4 16-row groups of gate and up, each wave one group of both; else 8
// groups, two per wave), y = tile slots. 256 threads; dynamic LDS gemm_q4k_lds().
__host__ __device__ inline size_t gemm_q4k_lds() { return 2 * (size_t) (GM_T * GM_QP + GM_T * GM_SP * 4 + GM_T * 4) + 2 * GM_T * 4; }

template <bool DUAL>
__global__ void __launch_bounds__(256, 2) k_gemm_q4k(GemmArgs a) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    constexpr int BUF = GM_T * GM_QP + GM_T * GM_SP * 4 + GM_T * 4;
    int * s_row = (int *) (smem + 2 * BUF), * s_out = s_row + GM_T;
    int e, c0, nt;
    if (!gemm_tile<GM_T>(a, blockIdx.y, e, c0, nt)) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, K = a.nsb * 256;
    gemm_rows<GM_T>(a, e, c0, nt, s_row, s_out);
    // the wave's two 16-row units
    const int gA = DUAL ? blockIdx.x * 4 + wave : (blockIdx.x * 4 + wave) * 2, gB = DUAL ? gA : gA + 1;
    const bool has = gA < a.tiles;
    const uint8_t * wA = a.w[0] + (int64_t) e * a.mat_bytes + (size_t) (has ? gA : 0) * a.nsb * 2304;
    const uint8_t * wB = (DUAL ? a.w[1] : a.w[0]) + (int64_t) e * a.mat_bytes + (size_t) (gB < a.tiles ? gB : 0) * a.nsb * 2304;
    uint4 raw[2][3];
    auto load_w = [&](int sb) {
        const uint4 * pa = (const uint4 *) (wA + (size_t) sb * 2304), * pb = (const uint4 *) (wB + (size_t) sb * 2304);
        raw[0][0] = pa[lane]; raw[0][1] = pa[64 + lane]; raw[0][2] = pa[128 + (lane & 15)];
        raw[1][0] = pb[lane]; raw[1][1] = pb[64 + lane]; raw[1][2] = pb[128 + (lane & 15)];
    };
    if (has) load_w(0);
    lds_sync();                                                      // s_row
    GmQ8K st;
    gm_load_q8k(st, a.act, K, 0, s_row);
    gm_store_q8k(st, (int8_t *) smem, (uint32_t *) (smem + GM_T * GM_QP), (float *) (smem + GM_T * GM_QP + GM_T * GM_SP * 4));
    lds_sync();
    float acc[2][GM_T / 16][4] = {};
    const v4i_t zi = {0, 0, 0, 0};
    const v4f_t zf = {0.0f, 0.0f, 0.0f, 0.0f};
    const int q = lane >> 4;
    for (int sb = 0; sb < a.nsb; ++sb) {
        char * buf = smem + (sb & 1) * BUF;
        const int8_t * sq = (const int8_t *) buf;
        const uint32_t * ss = (const uint32_t *) (buf + GM_T * GM_QP);
        const float * sdx = (const float *) (buf + GM_T * GM_QP + GM_T * GM_SP * 4);
        const bool more = sb + 1 < a.nsb;
        if (more) gm_load_q8k(st, a.act, K, sb + 1, s_row);
        if (has) {
            GmQ4Unit u[2];
            gm_prep_q4k(raw[0][0], raw[0][1], raw[0][2], lane, u[0]);
            gm_prep_q4k(raw[1][0], raw[1][1], raw[1][2], lane, u[1]);
            if (more) load_w(sb + 1);
#pragma unroll
            for (int ts = 0; ts < GM_T / 16; ++ts) {
                const int r = ts * 16 + (lane & 15);
                const int8_t * ap = sq + r * GM_QP + 8 * q;
                v4i_t A[4];
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const uint2 lo = *(const uint2 *) (ap + 64 * s), hi = *(const uint2 *) (ap + 64 * s + 32);
                    A[s] = (v4i_t) {(int) lo.x, (int) lo.y, (int) hi.x, (int) hi.y};
                }
                const v4h_t As = *(const v4h_t *) (ss + r * GM_SP + 2 * q);
                const v4f_t dx = *(const v4f_t *) (sdx + ts * 16 + 4 * q);
#pragma unroll
                for (int x = 0; x < 2; ++x) {
                    v4i_t ch = zi, cl = zi;
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        ch = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[s], u[x].bh[s], ch, 0, 0, 0);
                        cl = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[s], u[x].bl[s], cl, 0, 0, 0);
                    }
                    const v4f_t S = __builtin_amdgcn_mfma_f32_16x16x16f16(As, u[x].bm, zf, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        // the Q4_K unit value and fold of m16_unit / m16_fold (same operations)
                        const float f = (float) ((ch[i] << 3) + cl[i]);
                        acc[x][ts][i] = __builtin_fmaf(dx[i], __builtin_fmaf(u[x].d, f, -(u[x].dmin * S[i])), acc[x][ts][i]);
                    }
                }
            }
        }
        if (more) {
            char * nb = smem + ((sb + 1) & 1) * BUF;
            gm_store_q8k(st, (int8_t *) nb, (uint32_t *) (nb + GM_T * GM_QP), (float *) (nb + GM_T * GM_QP + GM_T * GM_SP * 4));
        }
        lds_sync();
    }
    if (!has) return;
    const int row = gA * 16 + (lane & 15), rowB = gB * 16 + (lane & 15);
#pragma unroll
    for (int ts = 0; ts < GM_T / 16; ++ts)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = ts * 16 + 4 * q + i;
            if (t >= nt) continue;
            const int it = s_out[t];
            float * o = a.out + (int64_t) it * a.out_ld;
            if (DUAL) {
                if (row < a.rows) o[row] = acc[1][ts][i] * z_silu(acc[0][ts][i]);
            } else {
                if (row < a.rows) o[row] = gemm_epi(a, acc[0][ts][i], it);
                if (rowB < a.rows) o[rowB] = gemm_epi(a, acc[1][ts][i], it);
            }
        }
}

// ------------------------------------------------------------------ F16 x f16
// Every F16 matmul runs on this kernel, in two shapes: wide (passes of more than 64 rows: tiles of 64
// token rows, each wave 64 output rows; DUAL 32 rows of gate and up) and narrow (decode widths: tiles
// of 16 token rows, each wave 16 output rows; DUAL 16 of gate and up). A row's output is the same
// chain of v_mfma_f32_16x16x32_f16 products over its 32-column steps in order in both shapes, so it
// does not depend on the width of the pass. grid: x = row blocks of 4 waves, y = tile slots; 256
// threads; dynamic LDS gemm_f16_lds(TS).
//   NG: 16-row sub-groups per wave (DUAL: NG / 2 of gate, then the same rows of up)
//   TS: 16-row token tiles per block tile (GT = 16 * TS token rows)
template <int TS>
struct GmF16 { u32x4 v[TS]; };                                       // half of one superblock's staging

// half h of one superblock of GT = 16 TS f16 activation rows: GT * 32 16-byte items, 256 TS per half
template <int TS>
__device__ __forceinline__ void gm_load_f16(GmF16<TS> & st, const ActBuf & act, int K, int sb, int h, const int * s_row) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int j = 0; j < TS; ++j) {
        const int i = 256 * TS * h + tid + 256 * j, r = i >> 5, c = i & 31;
        st.v[j] = *(const u32x4 *) (act.h + (int64_t) s_row[r] * K + sb * 256 + c * 8);
    }
}
template <int TS>
__device__ __forceinline__ void gm_store_f16(const GmF16<TS> & st, int h, uint16_t * sh) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int j = 0; j < TS; ++j) {
        const int i = 256 * TS * h + tid + 256 * j, r = i >> 5, c = i & 31;
        *(u32x4 *) (sh + r * GM_HP + c * 8) = st.v[j];
    }
}

__host__ __device__ inline size_t gemm_f16_lds(int ts) { return 2 * (size_t) (16 * ts) * GM_HP * 2 + 2 * (16 * ts) * 4; }

template <bool DUAL, int NG, int TS>
__global__ void __launch_bounds__(256, 2) k_gemm_f16(GemmArgs a) {
    constexpr int GT = 16 * TS, BUF = GT * GM_HP;                     // BUF in halves
    constexpr int RING = NG >= 4 ? 4 : 8;                            // 32-column weight steps in flight
    constexpr int RPW = DUAL ? 8 * NG : 16 * NG;                     // output rows per wave
    extern __shared__ __attribute__((aligned(16))) char smem[];
    uint16_t * sh0 = (uint16_t *) smem;
    int * s_row = (int *) (smem + 2 * BUF * 2), * s_out = s_row + GT;
    int e, c0, nt;
    if (!gemm_tile<GT>(a, blockIdx.y, e, c0, nt)) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, K = a.nsb * 256;
    gemm_rows<GT>(a, e, c0, nt, s_row, s_out);
    const int r0 = RPW * (blockIdx.x * 4 + wave);
    const bool has = r0 < a.rows;
    const int tile = has ? r0 / 64 : 0, sg0 = (r0 % 64) / 16;
    const uint8_t * base[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        // sub-group g: DUAL gate (g < NG / 2) or up rows r0 + 16 (g % (NG / 2)); else rows r0 + 16 g
        const uint8_t * wm = DUAL ? a.w[g / (NG / 2)] : a.w[0];
        const int sg = sg0 + (DUAL ? g % (NG / 2) : g);
        base[g] = wm + (int64_t) e * a.mat_bytes + ((size_t) tile * a.nsb * 32 * 64 + 16 * sg + (lane & 15)) * 16;
    }
    const int q = lane >> 4, nsteps = a.nsb * 8;
    // weight step kk (32 columns): chunk 4 * (kk % 8) + q of superblock kk / 8 (t64 layout)
    auto load_step = [&](int kk, u32x4 (&b)[NG]) {
        const size_t off = ((size_t) (kk >> 3) * 32 + 4 * (kk & 7) + q) * 64 * 16;
#pragma unroll
        for (int g = 0; g < NG; ++g) b[g] = *(const u32x4 *) (base[g] + off);
    };
    u32x4 ring[RING][NG];
#pragma unroll
    for (int j = 0; j < RING; ++j)
        if (has && j < nsteps) load_step(j, ring[j]);
    lds_sync();                                                      // s_row
    GmF16<TS> st;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        gm_load_f16<TS>(st, a.act, K, 0, h, s_row);
        gm_store_f16<TS>(st, h, sh0);
    }
    lds_sync();
    v4f_t acc[NG][TS];
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int ts = 0; ts < TS; ++ts) acc[g][ts] = (v4f_t) {0.0f, 0.0f, 0.0f, 0.0f};
    for (int sb = 0; sb < a.nsb; ++sb) {
        // the next superblock's rows go into the other buffer (free: every wave passed the barrier
        // after its last reads) in two halves, so only half of them occupy registers at a time
        const uint16_t * sh = sh0 + (sb & 1) * BUF;
        uint16_t * nb = sh0 + ((sb + 1) & 1) * BUF;
        const bool more = sb + 1 < a.nsb;
#pragma unroll
        for (int kb = 0; kb < 8; ++kb) {
            if (more && kb == 0) gm_load_f16<TS>(st, a.act, K, sb + 1, 0, s_row);
            if (more && kb == 3) { gm_store_f16<TS>(st, 0, nb); gm_load_f16<TS>(st, a.act, K, sb + 1, 1, s_row); }
            if (more && kb == 6) gm_store_f16<TS>(st, 1, nb);
            if (has) {
                const int kk = sb * 8 + kb;
                u32x4 (&b)[NG] = ring[kb % RING];                    // = kk % RING: RING divides 8
#pragma unroll
                for (int ts = 0; ts < TS; ++ts) {
                    const v8h_t A = *(const v8h_t *) (sh + (ts * 16 + (lane & 15)) * GM_HP + 32 * kb + 8 * q);
#pragma unroll
                    for (int g = 0; g < NG; ++g)
                        acc[g][ts] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, __builtin_bit_cast(v8h_t, b[g]), acc[g][ts], 0, 0, 0);
                }
                if (kk + RING < nsteps) load_step(kk + RING, b);
            }
        }
        lds_sync();
    }
    if (!has) return;
#pragma unroll
    for (int ts = 0; ts < TS; ++ts)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = ts * 16 + 4 * q + i;
            if (t >= nt) continue;
            const int it = s_out[t];
            float * o = a.out + (int64_t) it * a.out_ld;
            if (DUAL) {
#pragma unroll
                for (int g = 0; g < NG / 2; ++g) {
                    const int row = r0 + 16 * g + (lane & 15);
                    if (row < a.rows) o[row] = acc[g + NG / 2][ts][i] * z_silu(acc[g][ts][i]);
                }
            } else {
#pragma unroll
                for (int g = 0; g < NG; ++g) {
                    const int row = r0 + 16 * g + (lane & 15);
                    if (row < a.rows) o[row] = gemm_epi(a, acc[g][ts][i], it);
                }
            }
        }
}

} // namespace z2d
