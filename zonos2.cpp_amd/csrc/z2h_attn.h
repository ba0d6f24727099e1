// z2h_attn.h — ragged GQA attention on MFMA for wide passes (prefill chunks, mixed batches) and the
// per-slot prefill: src/zonos2-graph.cpp:113-175 (QK-norm, |temp|, interleaved RoPE, f16 KV append,
// softmax(K^T q / sqrt(hd)) V over the slot's band [0, n_past], sigmoid gate). Three kernels:
//   k_attn_flash16  wide passes with head_dim 128 and at most 4 query heads per KV head (the model
//                   family's shape): one block per tile walks the whole band over the f16 cache.
//   k_attn_flash32  the per-slot prefill's in-prompt attention over the prompt's fp32 K/V (same shapes).
//   k_attn_fa       every other shape, with k_attn_merge; described here first.
// (Decode steps attend through k_attn_chunk / k_attn_combine in z2h_kernels.h.)
//
// k_attn_fa: work item = (tile, KV head g, segment s): a tile is one row (decode) or a run of up to FA_ROWS rows
// of one slot at consecutive positions (wide passes); segment s is keys [128 s, 128 s + 128) of the
// band. The block loads the segment's K rows and V columns once for all rows of the tile, forms the
// rows' queries (one wave per row: per-head RMSNorm, |temp|, RoPE, f16) and computes, per row-head
// rh = row * GRP + head:
//   S^T = K Q^T            v_mfma_f32_16x16x32_f16 (M = 16 keys, N = 16 row-heads, K = 32 dims)
//   softmax over the segment's keys (causal mask per row), fp32, exp = z_expf
//   O^T = V^T P^T          the same MFMA with P split in two f16 parts (p = hi + lo, lo = p - hi)
// With S^T as the MFMA output, lane (rh, q) holds keys {16 mt + 4 q + i}, which is exactly the
// lane's share of the next product's P^T operand (the k-slot order only has to agree between the
// two operands); V is transposed on its way into LDS.
// A row whose band fits one segment is finished in the block (normalised, gated, encoded for W_o);
// the others leave one partial (max, sum, O) per segment, which k_attn_merge folds in order. A row's
// arithmetic does not depend on the tile it is in, so a row gives the same bits in any wide pass. A
// decode step attends through k_attn_chunk / k_attn_combine instead (64-row chunks, VALU arithmetic),
// so a row's attention output differs in its last bits between a decode step and a wide pass; the K/V
// rows it appends are the same bits either way.
#pragma once
#include "z2h_gemm.h"

namespace z2d {

constexpr int FA_SEG = 128;            // keys per segment
constexpr int FA_ROWS = 16;            // rows per wide tile (and rows * GRP <= 64)

__host__ __device__ inline int fa_nseg(int pos) { return (pos + FA_SEG) / FA_SEG; }   // segments of keys [0, pos]

// K rows [FA_SEG][hdp + 8], then V columns [hd][FA_SEG + 8] (the queries [64][hdp + 8] before them)
__host__ __device__ inline size_t attn_fa_lds(int hd) {
    const int hdp = hd < 32 ? 32 : hd;
    const size_t vt = (size_t) hd * (FA_SEG + 8), q = (size_t) 64 * (hdp + 8);
    return (size_t) FA_SEG * (hdp + 8) * 2 + (vt > q ? vt : q) * 2;
}

// decode items: item = (segment of token t, KV head g) over all tokens in order; sb = segments of the
// tokens before t
__device__ __forceinline__ bool fa_locate(const int32_t * n_past, const int32_t * slot_idx, int T, int nkv, int item,
                                          int & n_items, int & t, int & s, int & g, int & sb, int & np, int & slot) {
    const int lane = threadIdx.x & 63, want = item / nkv;
    g = item % nkv;
    int base = 0;
    bool found = false;
    for (int t0 = 0; t0 < T; t0 += 64) {
        const int u = t0 + lane;
        const int npu = u < T ? n_past[u] : 0, su = u < T ? slot_idx[u] : 0;
        const int ns = u < T ? fa_nseg(npu) : 0;
        const int incl = wave_scan_incl(ns, lane), excl = incl - ns;
        const uint64_t hit = __ballot(!found && want >= base + excl && want < base + incl);
        if (hit) {
            const int l = __ffsll((unsigned long long) hit) - 1;
            t = t0 + l;
            sb = base + lane_i(excl, l);
            s = want - sb;
            np = lane_i(npu, l);
            slot = lane_i(su, l);
            found = true;
        }
        base += lane_i(incl, 63);
    }
    n_items = base * nkv;
    return found;
}

// The block's output rows [m][GRP * HD] in s_out: stored to o_out (the group's slice of each row) and
// encoded for W_o (Q8_K per 256-block by one wave, as encode_row; Q8_0 / F16 through encode_row).
template <int HD, int GRP>
__device__ __forceinline__ void fa_store_rows(const AttnArgs & a, const float * s_out, int t0, int m, int g) {
    constexpr int SPAN = GRP * HD;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int base = g * SPAN, W = a.nh * HD;
    for (int i = tid; i < m * (SPAN / 4); i += 256) {
        const int r = i / (SPAN / 4), c = 4 * (i % (SPAN / 4));
        *(float4 *) (a.o_out + (int64_t) (t0 + r) * W + base + c) = *(const float4 *) (s_out + r * SPAN + c);
    }
    if (a.act_fmt == ACT_NONE) return;
    const int Kp = kpad(W);
    if (a.act_fmt == ACT_Q8_K) {
        // (the host encodes in the block only when the span covers whole 256-blocks)
        constexpr int NB = SPAN / 256 > 0 ? SPAN / 256 : 1;
        for (int b = wave; b < m * (SPAN / 256); b += 4) {
            const int r = b / NB, bb = b % NB, t = t0 + r;
            const float4 v4 = *(const float4 *) (s_out + r * SPAN + 256 * bb + 4 * lane);
            const float v[4] = {v4.x, v4.y, v4.z, v4.w};
            q8k_block_v(v, a.act.q + (int64_t) t * Kp + base + 256 * bb, a.act.d256 + (int64_t) t * (Kp / 256) + base / 256 + bb,
                        a.act.bs + (int64_t) t * (Kp / 16) + base / 16 + 16 * bb, lane);
        }
        return;
    }
    for (int r = 0; r < m; ++r) {
        const int t = t0 + r;
        if (a.act_fmt == ACT_Q8_0)
            encode_row<ACT_Q8_0>(s_out + r * SPAN, SPAN, a.act.q + (int64_t) t * Kp + base, a.act.d32 + (int64_t) t * (Kp / 32) + base / 32,
                                 nullptr, nullptr, nullptr);
        else
            encode_row<ACT_F16>(s_out + r * SPAN, SPAN, nullptr, nullptr, nullptr, nullptr, a.act.h + (int64_t) t * Kp + base);
    }
}

// grid: wide passes one block per item, a.tiles[2 item] = (first row t0, rows m | g << 16, segment,
// segments of all rows before t0) and a.tiles[2 item + 1] = (n_past of t0, its slot); decode steps a
// persistent grid over the items fa_locate finds.
// 256 threads; dynamic LDS attn_fa_lds(HD). Decode items form the new row's k / v (the last segment)
// and append them to the cache; wide passes have appended theirs (k_kv_append).
template <int HD, int GRP>
__global__ void __launch_bounds__(256, 2) k_attn_fa(AttnArgs a) {
    constexpr int HDP = HD < 32 ? 32 : HD;             // dims padded to the 32-wide k-steps of Q.K
    constexpr int KP = HDP + 8, VP = FA_SEG + 8;       // LDS pitches (halves)
    constexpr int NP = HD / 2;                         // dim pairs of a head (lane = pair)
    constexpr int DT = HD / 16;                        // 16-dim tiles of O
    constexpr int KS = HDP / 32;                       // k-steps of Q.K
    constexpr int MT = FA_SEG / 16;                    // 16-key tiles of a segment
    constexpr int PS = FA_SEG / 32;                    // 32-key steps of P.V
    constexpr int U4 = FA_SEG * HD / 8 / 256;          // 16-byte K (and V) items per thread
    static_assert(HD >= 16 && HD <= 128 && FA_SEG * HD / 8 % 256 == 0, "head size");
    extern __shared__ __attribute__((aligned(16))) char smem[];
    uint16_t * s_k = (uint16_t *) smem;                // [FA_SEG][KP]
    uint16_t * s_vt = s_k + FA_SEG * KP;               // [HD][VP]
    uint16_t * s_q = s_vt;                             // [64][KP] (before s_vt is filled)
    float * s_out = (float *) smem;                    // [rows][GRP * HD] (after the products)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, q4 = lane >> 4, c16 = lane & 15;
    const int nkv = a.nkv;
    const bool wide = a.tiles != nullptr;
    for (int item = blockIdx.x;; item += gridDim.x) {
        int t0, m, g, s, sb0, p0, slot;
        if (wide) {
            if (item >= (int) gridDim.x) break;
            const int4 e = a.tiles[2 * item], e2 = a.tiles[2 * item + 1];
            t0 = e.x; m = e.y & 0xffff; g = e.y >> 16; s = e.z; sb0 = e.w; p0 = e2.x; slot = e2.y;
        } else {
            int n_items;
            if (!fa_locate(a.n_past, a.slot_idx, a.T, nkv, item, n_items, t0, s, g, sb0, p0, slot)) break;
            m = 1;
        }
        const int plast = p0 + m - 1, nseg_t = fa_nseg(plast), k0 = s * FA_SEG;
        const int cmax = wide ? plast : p0 - 1;                       // last key row taken from the cache
        const int64_t band = ((int64_t) slot * nkv + g) * a.S * HD;
        const bool mk = !wide && s == nseg_t - 1;                     // decode: the segment holds the new row
        const int P = m * GRP, RT = P <= 16 ? 1 : P <= 32 ? 2 : 4;
        // ---- the wave's query inputs first, then the segment's K rows and V columns, so the query
        // arithmetic waits only for its own loads. Row-head slot k of the wave: with one row, rh =
        // wave + 4k (one wave per head); else row wave + 4 (k / GRP), head k % GRP (one wave per row).
        // (slots 8..15 only occur in wide tiles; their loads follow the K / V requests)
        constexpr int QK = 16, QK0 = 8;
        float qx0[QK], qx1[QK];
        auto q_load = [&](int k) {
            const int i = m == 1 ? (wave + 4 * k) / GRP : wave + 4 * (k / GRP), h = m == 1 ? (wave + 4 * k) % GRP : k % GRP;
            const bool ok = i < m && i * GRP + h < 16 * RT;
            const float * row = a.qkvg + (int64_t) (t0 + (ok ? i : 0)) * a.R + (int64_t) (g * GRP + h) * HD;
            qx0[k] = ok && lane < NP ? row[2 * lane] : 0.0f;
            qx1[k] = ok && lane < NP ? row[2 * lane + 1] : 0.0f;
        };
#pragma unroll
        for (int k = 0; k < QK0; ++k) q_load(k);
        float nx[4] = {0.0f, 0.0f, 0.0f, 0.0f};                     // the decode row's new k and v (wave 3)
        if (mk && wave == 3 && lane < NP) {
            const float * row = a.qkvg + (int64_t) t0 * a.R;
            nx[0] = row[(int64_t) (a.nh + g) * HD + 2 * lane]; nx[1] = row[(int64_t) (a.nh + g) * HD + 2 * lane + 1];
            nx[2] = row[(int64_t) (a.nh + nkv + g) * HD + 2 * lane]; nx[3] = row[(int64_t) (a.nh + nkv + g) * HD + 2 * lane + 1];
        }
        // K rows and V columns: every load issued (entries past cmax read the band's start and are
        // stored as zeros); K goes to LDS at once, V once the queries have left its region
        uint4 kr[U4], vr[U4];
#pragma unroll
        for (int j = 0; j < U4; ++j) {
            const int i = tid + 256 * j;
            const int r = i / (HD / 8), c = i % (HD / 8);             // K: key row r, dims 8c..
            kr[j] = *(const uint4 *) (a.kc + band + (k0 + r <= cmax ? (int64_t) (k0 + r) * HD + 8 * c : 0));
        }
#pragma unroll
        for (int j = 0; j < U4; ++j) {
            const int i = tid + 256 * j;
            const int r = i % FA_SEG, c = i / FA_SEG;                // V: key row r (lanes), dims 8c..
            vr[j] = *(const uint4 *) (a.vc + band + (k0 + r <= cmax ? (int64_t) (k0 + r) * HD + 8 * c : 0));
        }
#pragma unroll
        for (int k = QK0; k < QK; ++k) q_load(k);
        // K straight to LDS (its region is not shared with the queries)
#pragma unroll
        for (int j = 0; j < U4; ++j) {
            const int i = tid + 256 * j;
            const int r = i / (HD / 8), c = i % (HD / 8);
            *(uint4 *) &s_k[r * KP + 8 * c] = k0 + r <= cmax ? kr[j] : make_uint4(0, 0, 0, 0);
        }
        if constexpr (HD < HDP)                                       // zero dims [HD, HDP) of the K rows
            for (int i = tid; i < FA_SEG * (HDP - HD) / 8; i += 256) {
                const int r = i / ((HDP - HD) / 8), c = i % ((HDP - HD) / 8);
                *(uint4 *) &s_k[r * KP + HD + 8 * c] = make_uint4(0, 0, 0, 0);
            }
        // ---- queries of row-heads rh < 16 RT (past P: zeros), and the decode row's new k / v
        uint32_t nk = 0, nv = 0;
        {
            float cs = 1.0f, sn = 0.0f;
#pragma unroll
            for (int k = 0; k < QK; ++k) {
                const int i = m == 1 ? (wave + 4 * k) / GRP : wave + 4 * (k / GRP), h = m == 1 ? (wave + 4 * k) % GRP : k % GRP;
                const int rh = i * GRP + h;
                if (rh >= 16 * RT) continue;
                // one RoPE angle per row: the first row-head slot of each row (every slot with one row)
                if (i < m && (m == 1 ? k == 0 : h == 0)) rope_at(a, p0 + i, min(lane, NP - 1), cs, sn);
                uint32_t qv = 0;
                if (i < m) {
                    const int qh = g * GRP + h;
                    float y0, y1;
                    norm_rope<HD>(qx0[k], qx1[k], a.temp[qh], a.qk_eps, cs, sn, y0, y1);
                    if (lane < NP) {
                        qv = (uint32_t) f2h(y0) | ((uint32_t) f2h(y1) << 16);
                        if (a.cap_q && s == 0) {
                            a.cap_q[((int64_t) (t0 + i) * a.nh + qh) * HD + 2 * lane] = y0;
                            a.cap_q[((int64_t) (t0 + i) * a.nh + qh) * HD + 2 * lane + 1] = y1;
                        }
                    }
                }
                if (lane < HDP / 2) *(uint32_t *) &s_q[rh * KP + 2 * lane] = qv;
            }
        }
        if (mk && wave == 3) {
            float cs, sn, k0f, k1f;
            rope_at(a, p0, min(lane, NP - 1), cs, sn);
            norm_rope<HD>(nx[0], nx[1], 1.0f, a.qk_eps, cs, sn, k0f, k1f);
            if (lane < NP) {
                nk = (uint32_t) f2h(k0f) | ((uint32_t) f2h(k1f) << 16);
                nv = (uint32_t) f2h(nx[2]) | ((uint32_t) f2h(nx[3]) << 16);
                if (a.cap_k) {
                    a.cap_k[((int64_t) t0 * nkv + g) * HD + 2 * lane] = k0f; a.cap_k[((int64_t) t0 * nkv + g) * HD + 2 * lane + 1] = k1f;
                    a.cap_v[((int64_t) t0 * nkv + g) * HD + 2 * lane] = nx[2]; a.cap_v[((int64_t) t0 * nkv + g) * HD + 2 * lane + 1] = nx[3];
                }
            }
        }
        lds_sync();                                                   // queries and K rows in LDS
        const int rt = wave % RT, split = wave / RT, nsplit = 4 / RT;
        v8h_t qf[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) qf[ks] = *(const v8h_t *) &s_q[(16 * rt + c16) * KP + 32 * ks + 8 * q4];
        if (mk && wave == 3 && lane < NP) {
            // the new row (key p0) into the LDS copy of K and into the cache
            *(uint32_t *) &s_k[(p0 - k0) * KP + 2 * lane] = nk;
            *(uint32_t *) (a.kc + band + (int64_t) p0 * HD + 2 * lane) = nk;
            *(uint32_t *) (a.vc + band + (int64_t) p0 * HD + 2 * lane) = nv;
        }
        lds_sync();                                                   // s_q is free; s_k complete
        // ---- S^T = K Q^T for the wave's 16 row-heads, scaled and masked (key > the row's position)
        const int rh = 16 * rt + c16;
        const bool rh_ok = rh < P;
        const int prow = p0 + min(rh / GRP, m - 1);
        float sc[MT][4];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            v4f_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(*(const v8h_t *) &s_k[(16 * mt + c16) * KP + 32 * ks + 8 * q4], qf[ks], acc, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int kp = k0 + 16 * mt + 4 * q4 + i;
                sc[mt][i] = kp <= prow ? acc[i] * a.scale : -__builtin_inff();
            }
        }
        // ---- softmax over the segment (the rh's keys sit in lanes c16, c16 + 16, + 32, + 48)
        float mx = -__builtin_inff();
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sc[mt][i]);
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        float lsum = 0.0f;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float p = sc[mt][i] == -__builtin_inff() ? 0.0f : z_expf(sc[mt][i] - mx);
                sc[mt][i] = p;
                lsum = lsum + p;
            }
        lsum = lsum + __shfl_xor(lsum, 16);
        lsum = lsum + __shfl_xor(lsum, 32);
        v8h_t ph[PS], pl[PS];
#pragma unroll
        for (int ps = 0; ps < PS; ++ps)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float p = sc[2 * ps + (j >> 2)][j & 3];
                const _Float16 hi = (_Float16) p;
                ph[ps][j] = hi;
                pl[ps][j] = (_Float16) (p - (float) hi);
            }
        // ---- the V rows transposed into LDS (keys past cmax zeroed; the decode row's new v after them):
        // the lanes of a store are consecutive keys of one dim
#pragma unroll
        for (int j = 0; j < U4; ++j) {
            const int i = tid + 256 * j;
            const int r = i % FA_SEG, c = i / FA_SEG;
            const uint4 v = k0 + r <= cmax ? vr[j] : make_uint4(0, 0, 0, 0);
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) s_vt[(8 * c + e) * VP + r] = (uint16_t) (w[e >> 1] >> (16 * (e & 1)));
        }
        lds_sync();
        if (mk) {
            if (wave == 3 && lane < NP) {
                s_vt[(2 * lane) * VP + p0 - k0] = (uint16_t) (nv & 0xffffu);
                s_vt[(2 * lane + 1) * VP + p0 - k0] = (uint16_t) (nv >> 16);
            }
            lds_sync();
        }
        // ---- O^T = V^T P^T over the wave's dim tiles dt = split, split + nsplit, ... A row whose band
        // is one segment is finished here (normalised, gated, encoded); the others leave partials
        // (segment max, sum, unnormalised O) for k_attn_merge
        const int i_row = min(rh / GRP, m - 1), hh = rh % GRP, qh = g * GRP + hh, t_row = t0 + i_row;
        const int ns_row = fa_nseg(p0 + i_row);
        const bool fin = ns_row == 1;                                 // (then s == 0)
        float gsig = 0.0f;
        if (rh_ok && fin) gsig = z_sigmoid(a.qkvg[(int64_t) t_row * a.R + (int64_t) (a.nh + 2 * nkv) * HD + qh]);
        int sb_row = sb0;
        for (int j = 0; j < i_row; ++j) sb_row += fa_nseg(p0 + j);
        const bool has_seg = s < ns_row;
        const int64_t pidx = ((int64_t) (sb_row + s) * nkv + g) * GRP + hh;
        if (!fin && rh_ok && has_seg && q4 == 0 && split == 0) *(float2 *) (a.part_ml + pidx * 2) = make_float2(mx, lsum);
#pragma unroll
        for (int u = 0; u < DT; ++u) {
            const int dt = split + nsplit * u;
            if (dt >= DT) break;
            v4f_t o = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ps = 0; ps < PS; ++ps) {
                const uint16_t * vp = &s_vt[(16 * dt + c16) * VP + 32 * ps + 4 * q4];
                const uint2 lo = *(const uint2 *) vp, hi = *(const uint2 *) (vp + 16);
                const v8h_t vf = __builtin_bit_cast(v8h_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
                o = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, ph[ps], o, 0, 0, 0);
                o = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pl[ps], o, 0, 0, 0);
            }
            const int dim = 16 * dt + 4 * q4;
            if (!rh_ok) continue;
            if (fin) {
                const float f = gsig / lsum;
                *(float4 *) (s_out + i_row * (GRP * HD) + hh * HD + dim) = make_float4(o[0] * f, o[1] * f, o[2] * f, o[3] * f);
            } else if (has_seg) {
                *(float4 *) (a.part_o + pidx * HD + dim) = make_float4(o[0], o[1], o[2], o[3]);
            }
        }
        // rows [0, m1) of the tile are one-segment rows (positions below FA_SEG), finished by segment 0
        const int m1 = s == 0 ? max(0, min(m, FA_SEG - p0)) : 0;
        if (m1 > 0) {
            if (a.cap_gate && rh_ok && fin && q4 == 0 && split == 0) a.cap_gate[(int64_t) t_row * a.nh + qh] = gsig;
            lds_sync();                                               // s_out rows complete
            fa_store_rows<HD, GRP>(a, s_out, t0, m1, g);
        }
        lds_sync();                                                   // LDS reuse by the next item
    }
}

// The segments of rows whose band spans several: block (row t, KV head g), its GRP heads. Every
// partial of the row is requested at once into LDS, then each (head, 4 dims) folds the segments in
// order: M = max m_s, w_s = exp(m_s - M), L = sum w_s l_s, O = sum w_s O_s (fmaf chains), out =
// O * (sigmoid(gate) / L); the row's group slice is stored and encoded for W_o as k_attn_fa does.
// Dynamic LDS attn_merge_lds(hd, grp, max segments).
__host__ __device__ inline size_t attn_merge_lds(int hd, int grp, int nsmax) {
    return (size_t) 4 * ((size_t) nsmax * grp * (hd + 2) + (size_t) grp * hd);
}
template <int HD, int GRP>
__global__ void __launch_bounds__(256) k_attn_merge(AttnArgs a) {
    extern __shared__ __attribute__((aligned(16))) float sm_mg[];
    const int t = blockIdx.x / a.nkv, g = blockIdx.x % a.nkv, tid = threadIdx.x, nkv = a.nkv;
    const int lane = tid & 63;
    const int ns = fa_nseg(a.n_past[t]);
    if (ns == 1) return;                                              // finished by k_attn_fa
    // segments of the rows before t (every wave scans; lanes are rows)
    int sb = 0;
    for (int u0 = 0; u0 < t; u0 += 64) {
        const int u = u0 + lane;
        sb += lane_i(wave_scan_incl(u < t ? fa_nseg(a.n_past[u]) : 0, lane), 63);
    }
    float * s_o = sm_mg;                                              // [ns][GRP][HD]
    float * s_ml = s_o + (size_t) ns * GRP * HD;                      // [ns][GRP][2]
    float * s_out = s_ml + (size_t) ns * GRP * 2;                     // [GRP][HD]
    const int64_t pst = (int64_t) nkv * GRP, p_0 = ((int64_t) sb * nkv + g) * GRP;
    // partial (segment ss, head h) = p_0 + ss * pst + h; MB loads per thread in flight before their stores
    constexpr int MB = 8;
    for (int base = 0; base < ns * GRP * (HD / 4); base += 256 * MB) {
        float4 v[MB];
#pragma unroll
        for (int u = 0; u < MB; ++u) {
            const int i = min(base + tid + 256 * u, ns * GRP * (HD / 4) - 1);
            const int ss = i / (GRP * (HD / 4)), h = (i / (HD / 4)) % GRP, d4 = 4 * (i % (HD / 4));
            v[u] = *(const float4 *) (a.part_o + (p_0 + ss * pst + h) * HD + d4);
        }
#pragma unroll
        for (int u = 0; u < MB; ++u) {
            const int i = base + tid + 256 * u;
            if (i >= ns * GRP * (HD / 4)) break;
            const int ss = i / (GRP * (HD / 4)), h = (i / (HD / 4)) % GRP, d4 = 4 * (i % (HD / 4));
            *(float4 *) (s_o + (ss * GRP + h) * HD + d4) = v[u];
        }
    }
    for (int i = tid; i < ns * GRP; i += 256)
        *(float2 *) (s_ml + 2 * i) = *(const float2 *) (a.part_ml + (p_0 + (i / GRP) * pst + i % GRP) * 2);
    lds_sync();
    for (int u = tid; u < GRP * (HD / 4); u += 256) {
        const int h = u / (HD / 4), d4 = 4 * (u % (HD / 4)), qh = g * GRP + h;
        const float gs = z_sigmoid(a.qkvg[(int64_t) t * a.R + (int64_t) (a.nh + 2 * nkv) * HD + qh]);
        float M = -__builtin_inff();
        for (int ss = 0; ss < ns; ++ss) M = fmaxf(M, s_ml[(ss * GRP + h) * 2]);
        float L = 0.0f;
        float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int ss = 0; ss < ns; ++ss) {
            const float2 ml = *(const float2 *) (s_ml + (ss * GRP + h) * 2);
            const float w = ml.x == -__builtin_inff() ? 0.0f : z_expf(ml.x - M);
            const float4 po = *(const float4 *) (s_o + (ss * GRP + h) * HD + d4);
            L = __builtin_fmaf(w, ml.y, L);
            o = make_float4(__builtin_fmaf(w, po.x, o.x), __builtin_fmaf(w, po.y, o.y), __builtin_fmaf(w, po.z, o.z), __builtin_fmaf(w, po.w, o.w));
        }
        const float f = gs / L;
        if (a.cap_gate && d4 == 0) a.cap_gate[(int64_t) t * a.nh + qh] = gs;
        *(float4 *) (s_out + h * HD + d4) = make_float4(o.x * f, o.y * f, o.z * f, o.w * f);
    }
    lds_sync();
    fa_store_rows<HD, GRP>(a, s_out, t, 1, g);
}

// ------------------------------------------------------------------ wide passes, one flash pass per tile
// For head_dim 128 and at most 4 query heads per KV head, a wide pass's tiles (up to 16 rows of one slot
// at consecutive positions) take one block of 8 waves each instead of one item per segment: the block
// walks every 64-key segment of the band [0, last row] of the slot's f16 cache (the rows k_kv_append
// put there) with an online softmax, so no partials and no k_attn_merge:
//   S^T = K Q^T   one v_mfma_f32_16x16x32_f16 per 32 dims (f16 queries, as above)
//   O^T = V^T P^T P split in two f16 parts (p = hi + lo), two MFMAs per 32 keys
// Wave w takes row-heads [16 (w % 4), + 16) and keys [32 (w / 4), + 32) of every segment with its own
// running max m, sum l and O (m' = max(m, segment max), O = O exp(m - m') + V^T P^T, l = l exp(m - m') +
// sum P); at the end the two key halves merge (M = max(m0, m1), O = O0 exp(m0 - M) + O1 exp(m1 - M),
// likewise l) and O / l times the head's sigmoid gate is stored and encoded for W_o. The K / V segments
// are double-buffered in LDS: a segment's rows are stored while the one before is multiplied, with one
// barrier per segment. A row's arithmetic does not depend on the tile or the pass it is in (segments
// past its position multiply O and l by exactly 1 and add exact zeros).
// a.tiles[item] = (first row t0, rows m | g << 16, -, -); slot and positions from slot_idx / n_past.
constexpr int FH_SEG = 64;                                           // keys per segment
constexpr int FH_KP = 128 + 8;                                       // K row pitch (halves)
constexpr int FH_VP = FH_SEG + 4;                                    // V^T row pitch (halves, 34 dwords)
constexpr int FH_BUF = (FH_SEG * FH_KP + 128 * FH_VP) * 2;           // one buffer: K rows, then V^T (bytes)
__host__ __device__ inline size_t attn_flash16_lds() { return (size_t) 2 * FH_BUF; }

// max / sum of a value over the 4 lanes l, l ^ 16, l ^ 32, l ^ 48 (one MFMA column's k-slot lanes):
// v_permlane16_swap / v_permlane32_swap with both operands v hand each lane its partner's value and
// its own; every lane ends with the same bits (the lower row's value is the first operand). The two
// results are copied to scalars before the bit cast: __builtin_bit_cast of an element of the returned
// vector reads element 0 with this compiler.
__device__ __forceinline__ void fl_swap16(float v, float & lo, float & hi) {
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v), false, false);
    const unsigned r0 = r[0], r1 = r[1];
    lo = __builtin_bit_cast(float, r0);
    hi = __builtin_bit_cast(float, r1);
}
__device__ __forceinline__ void fl_swap32(float v, float & lo, float & hi) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v), false, false);
    const unsigned r0 = r[0], r1 = r[1];
    lo = __builtin_bit_cast(float, r0);
    hi = __builtin_bit_cast(float, r1);
}
__device__ __forceinline__ float fl_max4(float v) {
    float a, b;
    fl_swap16(v, a, b);
    fl_swap32(fmaxf(a, b), a, b);
    return fmaxf(a, b);
}
__device__ __forceinline__ float fl_sum4(float v) {
    float a, b;
    fl_swap16(v, a, b);
    fl_swap32(a + b, a, b);
    return a + b;
}
constexpr float FL_TAU = 8.0f;                                       // lazy rescale: P <= 2^8

template <int GRP>
__global__ void __launch_bounds__(512) k_attn_flash16(AttnArgs a) {
    constexpr int HD = 128, NP = HD / 2, DT = HD / 16, KS = HD / 32, RW = HD / 8;   // RW: uint4 per row
    static_assert(GRP <= 4, "at most 64 row-heads per tile");
    extern __shared__ __attribute__((aligned(16))) char sm_fh[];
    float * s_q = (float *) sm_fh;                                   // [64][HD + 4] queries (before the loop)
    float2 * s_cs = (float2 *) (sm_fh + 64 * (HD + 4) * 4);          // [16][NP] RoPE (cos, sin)
    float * s_th = (float *) (sm_fh + 64 * (HD + 4) * 4 + 16 * NP * 8);   // [16][NP] RoPE angles
    float * s_mrg = (float *) sm_fh;                                 // [4][34][64] key-half partials (after)
    float * s_out = (float *) (sm_fh + 4 * 34 * 64 * 4);             // [16][GRP * HD] output rows (after)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, q4 = lane >> 4, c16 = lane & 15;
    const int wq = wave & 3, kh = wave >> 2;
    const int nkv = a.nkv;
    const int4 e = a.tiles[blockIdx.x];
    const int t0 = e.x, m = e.y & 0xffff, g = e.y >> 16;
    const int p0 = a.n_past[t0], slot = a.slot_idx[t0], plast = p0 + m - 1, nseg = plast / FH_SEG + 1;
    const int P = m * GRP;
    const int64_t band = ((int64_t) slot * nkv + g) * a.S * HD;
    const uint4 * ksrc = (const uint4 *) (a.kc + band), * vsrc = (const uint4 *) (a.vc + band);
    // segment s into registers (rows past plast re-read plast; they are masked). K: item i = tid + 512 J
    // is row i / 16, 16-byte chunk i % 16 (coalesced rows). V: the key pair p = lane % 16 + 16 (wave / 4)
    // at chunk c = lane / 16 + 4 (wave % 4), both keys' chunk (named registers, not an array).
    uint4 ka0, ka1, vx, vy;
#define FH_LOAD(S_)                                                                                         \
    {                                                                                                       \
        const int r0_ = min(FH_SEG * (S_) + (tid >> 4), plast), r1_ = min(FH_SEG * (S_) + ((tid + 512) >> 4), plast); \
        ka0 = ksrc[(int64_t) r0_ * RW + (tid & 15)];                                                        \
        ka1 = ksrc[(int64_t) r1_ * RW + (tid & 15)];                                                        \
        const int p_ = (lane & 15) + 16 * (wave >> 2), c_ = (lane >> 4) + 4 * (wave & 3);                   \
        const int v0_ = min(FH_SEG * (S_) + 2 * p_, plast), v1_ = min(FH_SEG * (S_) + 2 * p_ + 1, plast);   \
        vx = vsrc[(int64_t) v0_ * RW + c_];                                                                 \
        vy = vsrc[(int64_t) v1_ * RW + c_];                                                                 \
    }
    // into buffer B_: K rows; V transposed (the key pair's two halves of dim d form one dword of row d;
    // a wave's 64 lanes write 64 distinct banks)
#define FH_STORE(B_)                                                                                        \
    {                                                                                                       \
        uint16_t * bk_ = (uint16_t *) (sm_fh + (B_) * FH_BUF), * bv_ = bk_ + FH_SEG * FH_KP;                \
        *(uint4 *) (bk_ + (tid >> 4) * FH_KP + 8 * (tid & 15)) = ka0;                                        \
        *(uint4 *) (bk_ + ((tid + 512) >> 4) * FH_KP + 8 * (tid & 15)) = ka1;                                \
        const int p_ = (lane & 15) + 16 * (wave >> 2), c_ = (lane >> 4) + 4 * (wave & 3);                   \
        uint16_t * pl_ = bv_ + 8 * c_ * FH_VP + 2 * p_;                                                     \
        const uint32_t x_[4] = {vx.x, vx.y, vx.z, vx.w}, y_[4] = {vy.x, vy.y, vy.z, vy.w};                 \
        _Pragma("unroll") for (int u_ = 0; u_ < 4; ++u_) {                                                  \
            *(uint32_t *) (pl_ + (2 * u_) * FH_VP) = (x_[u_] & 0xffffu) | (y_[u_] << 16);                   \
            *(uint32_t *) (pl_ + (2 * u_ + 1) * FH_VP) = (x_[u_] >> 16) | (y_[u_] & 0xffff0000u);           \
        }                                                                                                   \
    }
    FH_LOAD(0)
    // ---- RoPE angle chains (one thread per row), (cos, sin) per (row, dim pair), then the queries
    // (wave w: row-heads w, w + 8, ...; per-head RMSNorm, |temp|, RoPE; f16 for the products)
    if (tid < m) {
        float th = (float) (p0 + tid);
        for (int j = 0; j < NP; ++j) {
            s_th[tid * NP + j] = th;
            th = th * a.theta_scale;
        }
    }
    lds_sync();
    for (int i = tid; i < m * NP; i += 512) {
        float sn, cs;
        z_sincos(s_th[i], sn, cs);
        s_cs[i] = make_float2(cs, sn);
    }
    lds_sync();
    {
        constexpr int QW = 8;
        float2 xq[QW];
#pragma unroll
        for (int k = 0; k < QW; ++k) {
            const int rq = min(wave + 8 * k, P - 1), i = rq / GRP, qh = g * GRP + rq % GRP;
            xq[k] = *(const float2 *) (a.qkvg + (int64_t) (t0 + i) * a.R + (int64_t) qh * HD + 2 * lane);
        }
#pragma unroll
        for (int k = 0; k < QW; ++k) {
            const int rq = wave + 8 * k;
            if (rq < P) {                                            // (wave-uniform)
                const int i = rq / GRP, qh = g * GRP + rq % GRP;
                const float2 c = s_cs[i * NP + lane];
                float y0, y1;
                norm_rope<HD>(xq[k].x, xq[k].y, a.temp[qh], a.qk_eps, c.x, c.y, y0, y1);
                *(float2 *) &s_q[rq * (HD + 4) + 2 * lane] = make_float2(y0, y1);
                if (a.cap_q) *(float2 *) (a.cap_q + ((int64_t) (t0 + i) * a.nh + qh) * HD + 2 * lane) = make_float2(y0, y1);
            }
        }
    }
    lds_sync();
    const int rh = 16 * wq + c16;                                    // the lane's row-head (B columns)
    const bool rh_ok = rh < P;
    const int row = rh_ok ? rh / GRP : 0, pos = p0 + row;
    // f16(Q[rh][32 ks + 8 q4 .. + 7]) (the f16 query of the K / V products); the scores are taken to
    // log2 units in fp32 (times scale * log2(e)), so P = exp2(S - m)
    const float qscale = a.scale * 1.44269504088896341f;
    v8h_t qv[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
        for (int j = 0; j < 8; ++j) qv[ks][j] = rh_ok ? (_Float16) s_q[rh * (HD + 4) + 32 * ks + 8 * q4 + j] : (_Float16) 0.0f;
    }
    lds_sync();                                                      // queries read: LDS free for the K / V buffers
    FH_STORE(0)
    if (nseg > 1) { FH_LOAD(1) }
    lds_sync();
    const bool active = 16 * wq < P;                                 // the wave has row-heads
    // m_run: the row-head's reference max (log2 units), raised only when a segment's max exceeds it by
    // more than FL_TAU, so P <= 2^FL_TAU; l_part: this lane's share of the row-head's sum
    float m_run = -__builtin_inff(), l_part = 0.0f;
    v4f_t o[DT];
#pragma unroll
    for (int d = 0; d < DT; ++d) o[d] = (v4f_t) {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s = 0; s < nseg; ++s) {
        if (s + 1 < nseg) {                                          // the next segment into the other buffer
            FH_STORE((s + 1) & 1)
            if (s + 2 < nseg) { FH_LOAD(s + 2) }
        }
        if (active) {
            const uint16_t * bk = (const uint16_t *) (sm_fh + (s & 1) * FH_BUF), * bv = bk + FH_SEG * FH_KP;
            // S^T for the wave's 16 row-heads and its 32 keys of the segment; the causal mask only in
            // segments reaching past the tile's first row (block-uniform)
            const bool masked = FH_SEG * s + FH_SEG - 1 > p0;
            float sc[2][4];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                v4f_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
                const int kr = (32 * kh + 16 * mt + c16) * FH_KP + 8 * q4;
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(*(const v8h_t *) &bk[kr + 32 * ks], qv[ks], acc, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) sc[mt][i] = acc[i] * qscale;
                if (masked) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int key = FH_SEG * s + 32 * kh + 16 * mt + 4 * q4 + i;
                        if (!(rh_ok && key <= pos)) sc[mt][i] = -__builtin_inff();
                    }
                }
            }
            float mx = fmaxf(fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3])), fmaxf(fmaxf(sc[1][0], sc[1][1]), fmaxf(sc[1][2], sc[1][3])));
            mx = fl_max4(mx);
            const bool need = mx > m_run + FL_TAU;                   // (the first keys: m_run = -inf)
            if (__any(need)) {
                const float m_new = need ? mx : m_run;
                const float alpha = need ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;   // (0 from -inf)
#pragma unroll
                for (int d = 0; d < DT; ++d) o[d] = o[d] * alpha;
                l_part = l_part * alpha;
                m_run = m_new;
            }
            const float mref = m_run == -__builtin_inff() ? 0.0f : m_run;    // (all keys so far masked: weights 0)
            v8h_t ph, pl;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float p = __builtin_amdgcn_exp2f(sc[j >> 2][j & 3] - mref);
                l_part = l_part + p;
                const _Float16 hi = (_Float16) p;
                ph[j] = hi;
                pl[j] = (_Float16) (p - (float) hi);
            }
            // O^T += V^T P^T for the wave's row-heads, every dim tile
#pragma unroll
            for (int d = 0; d < DT; ++d) {
                const int off = (16 * d + c16) * FH_VP + 32 * kh + 4 * q4;
                const uint2 h0 = *(const uint2 *) &bv[off], h1 = *(const uint2 *) &bv[off + 16];
                const v8h_t vv = __builtin_bit_cast(v8h_t, make_uint4(h0.x, h0.y, h1.x, h1.y));
                v4f_t acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(vv, ph, o[d], 0, 0, 0);
                o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vv, pl, acc, 0, 0, 0);
            }
        }
        lds_sync();                                                  // segment s read, segment s + 1 stored
    }
    const float l_run = fl_sum4(l_part);
    float * mg = s_mrg + wq * (34 * 64);
    if (active && kh == 1) {
#pragma unroll
        for (int d = 0; d < DT; ++d)
#pragma unroll
            for (int i = 0; i < 4; ++i) mg[(4 * d + i) * 64 + lane] = o[d][i];
        mg[32 * 64 + lane] = m_run;
        mg[33 * 64 + lane] = l_run;
    }
    lds_sync();
    if (active && kh == 0 && rh_ok) {
        const float m1 = mg[32 * 64 + lane], l1 = mg[33 * 64 + lane];
        const float M = fmaxf(m_run, m1);                            // finite: key 0 is in every band
        const float a0 = __builtin_amdgcn_exp2f(m_run - M), a1 = __builtin_amdgcn_exp2f(m1 - M);
        const float l = __builtin_fmaf(l_run, a0, l1 * a1);
        const int h = rh % GRP, qhd = g * GRP + h, t = t0 + row;
        const float gsig = z_sigmoid(a.qkvg[(int64_t) t * a.R + (int64_t) (a.nh + 2 * nkv) * HD + qhd]);
        const float f = gsig / l;
        if (a.cap_gate && q4 == 0) a.cap_gate[(int64_t) t * a.nh + qhd] = gsig;
#pragma unroll
        for (int d = 0; d < DT; ++d) {
            float y[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) y[i] = __builtin_fmaf(o[d][i], a0, mg[(4 * d + i) * 64 + lane] * a1) * f;
            *(float4 *) (s_out + row * (GRP * HD) + h * HD + 16 * d + 4 * q4) = make_float4(y[0], y[1], y[2], y[3]);
        }
    }
    lds_sync();
    if (wave < 4) fa_store_rows<HD, GRP>(a, s_out, t0, m, g);        // (a 256-thread helper)
#undef FH_LOAD
#undef FH_STORE
}

// ------------------------------------------------------------------ per-slot prefill, fp32 K/V
// The prompt's rows attend to the prompt's own fp32 K/V (src/zonos2-graph.cpp:155-169, the reference's
// manual fp32 attention): one block per (tile of up to 16 rows of one slot at consecutive positions,
// KV head g) walks every 64-key segment of the band [0, last row] with an online softmax, so no
// partials leave the block. Every fp32 operand x is carried as two f16 parts, hi = f16(x) and
// lo = f16(x - hi) (x = hi + lo to about 2^-22 relative; k_kv_append stores the K / V rows split so),
// and each product a.b takes three v_mfma_f32_16x16x32_f16 (a_hi b_hi + a_lo b_hi + a_hi b_lo; the
// dropped a_lo b_lo is below 2^-22):
//   S^T = K Q^T   (M = 16 keys, N = 16 row-heads, k = 32 dims per step), then times scale * log2(e)
//   O^T = V^T P^T (M = 16 dims, N = 16 row-heads, k = 32 keys: slot j of the lane with k-slot group q
//                  is key 16 (j / 4) + 4 q + j % 4 of the 32, the S^T lanes' own values, so P stays put;
//                  V is transposed into LDS so the A operand reads those keys as two 8-byte loads)
// 8 waves: wave w takes row-heads [16 (w % 4), + 16) (rh = row * GRP + head) and keys [32 (w / 4), + 32)
// of every segment with its own reference max m (log2 units, raised only when a segment's max exceeds
// it by more than FL_TAU, so P = exp2(S - m) <= 2^FL_TAU), O and per-lane sums; at the end the two key
// halves merge (M = max(m0, m1), O = O0 2^(m0 - M) + O1 2^(m1 - M), likewise l), then O / l times the
// head's sigmoid gate is stored and encoded for W_o (fa_store_rows). The K / V segments are
// double-buffered in LDS: a segment's rows are stored while the one before is multiplied, one barrier
// per segment. A row's arithmetic does not depend on the tile it is in (segments past its position
// add exact zeros and rescale by exactly 1), so any prefill chunking gives the same bits.
// a.tiles[item] = (first row t0, rows m | g << 16, -, -); the rows' positions are n_past[t0 ..].
constexpr int FL_SEG = 64;                                           // keys per segment
constexpr int FL_KP = 128 + 8;                                       // K plane row pitch (halves)
constexpr int FL_VP = FL_SEG + 4;                                    // V^T plane row pitch (halves, 34 dwords)
constexpr int FL_BUF = 2 * (2 * FL_SEG * FL_KP + 2 * 128 * FL_VP);   // one buffer: K hi, K lo, V^T hi, V^T lo (bytes)
__host__ __device__ inline size_t attn_flash32_lds() { return (size_t) 2 * FL_BUF; }

template <int GRP>
__global__ void __launch_bounds__(512) k_attn_flash32(AttnArgs a) {
    constexpr int HD = 128, NP = HD / 2, DT = HD / 16, KS = HD / 32, RW = HD / 8;   // RW: 16-byte chunks per plane row
    static_assert(GRP <= 4, "at most 64 row-heads per tile");
    extern __shared__ __attribute__((aligned(16))) char sm_fl[];
    float * s_q = (float *) sm_fl;                                   // [64][HD + 4] queries (before the loop)
    float2 * s_cs = (float2 *) (sm_fl + 64 * (HD + 4) * 4);          // [16][NP] RoPE (cos, sin)
    float * s_th = (float *) (sm_fl + 64 * (HD + 4) * 4 + 16 * NP * 8);   // [16][NP] RoPE angles
    float * s_mrg = (float *) sm_fl;                                 // [4][34][64] key-half partials (after)
    float * s_out = (float *) (sm_fl + 4 * 34 * 64 * 4);             // [16][GRP * HD] output rows (after)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, q4 = lane >> 4, c16 = lane & 15;
    const int wq = wave & 3, kh = wave >> 2;
    const int nkv = a.nkv;
    const int4 e = a.tiles[blockIdx.x];
    const int t0 = e.x, m = e.y & 0xffff, g = e.y >> 16;
    const int p0 = a.n_past[t0], plast = p0 + m - 1, nseg = plast / FL_SEG + 1;
    const int P = m * GRP;
    // rows of 2 RW chunks (hi, then lo): 512 bytes, the fp32 row's
    const uint4 * ksrc = (const uint4 *) (a.kf + (int64_t) g * a.S * HD), * vsrc = (const uint4 *) (a.vf + (int64_t) g * a.S * HD);
    // segment s into registers (rows past plast re-read plast; they are masked). K: item i = tid + 512 J
    // is row i / 32, chunk i % 32 (coalesced rows). V: items (key pair p, chunk c) with p = lane % 16 +
    // 16 J, c = lane / 16 + 4 wave, both keys' chunk. Named registers: the compiler keeps an array
    // carried across the segment loop in scratch memory.
    uint4 ka0, ka1, ka2, ka3, vx0, vy0, vx1, vy1;
#define FL_LDK(J_, S_)                                                                                      \
    {                                                                                                       \
        const int i_ = tid + 512 * (J_), r_ = min(FL_SEG * (S_) + (i_ >> 5), plast);                        \
        ka##J_ = ksrc[(int64_t) r_ * (2 * RW) + (i_ & 31)];                                                 \
    }
#define FL_LDV(J_, S_)                                                                                      \
    {                                                                                                       \
        const int p_ = (lane & 15) + 16 * (J_), c_ = (lane >> 4) + 4 * wave;                                \
        const int r0_ = min(FL_SEG * (S_) + 2 * p_, plast), r1_ = min(FL_SEG * (S_) + 2 * p_ + 1, plast);   \
        vx##J_ = vsrc[(int64_t) r0_ * (2 * RW) + c_];                                                       \
        vy##J_ = vsrc[(int64_t) r1_ * (2 * RW) + c_];                                                       \
    }
#define FL_LOAD(S_) FL_LDK(0, S_) FL_LDK(1, S_) FL_LDK(2, S_) FL_LDK(3, S_) FL_LDV(0, S_) FL_LDV(1, S_)
    // into buffer B_: K rows into the hi / lo planes; V transposed (the key pair's two halves of dim d
    // form one dword of plane row d; a wave's 64 lanes write 64 distinct banks)
#define FL_STK(B_, J_)                                                                                      \
    {                                                                                                       \
        uint16_t * kh_ = (uint16_t *) (sm_fl + (B_) * FL_BUF), * kl_ = kh_ + FL_SEG * FL_KP;                \
        const int i_ = tid + 512 * (J_), r_ = i_ >> 5, c_ = i_ & 31;                                        \
        *(uint4 *) ((c_ < RW ? kh_ : kl_) + r_ * FL_KP + 8 * (c_ & (RW - 1))) = ka##J_;                     \
    }
#define FL_STV(B_, J_)                                                                                      \
    {                                                                                                       \
        uint16_t * vh_ = (uint16_t *) (sm_fl + (B_) * FL_BUF) + 2 * FL_SEG * FL_KP, * vl_ = vh_ + HD * FL_VP; \
        const int p_ = (lane & 15) + 16 * (J_), c_ = (lane >> 4) + 4 * wave;                                \
        uint16_t * pl_ = (c_ < RW ? vh_ : vl_) + 8 * (c_ & (RW - 1)) * FL_VP + 2 * p_;                      \
        const uint32_t x_[4] = {vx##J_.x, vx##J_.y, vx##J_.z, vx##J_.w}, y_[4] = {vy##J_.x, vy##J_.y, vy##J_.z, vy##J_.w}; \
        _Pragma("unroll") for (int u_ = 0; u_ < 4; ++u_) {                                                  \
            *(uint32_t *) (pl_ + (2 * u_) * FL_VP) = (x_[u_] & 0xffffu) | (y_[u_] << 16);                   \
            *(uint32_t *) (pl_ + (2 * u_ + 1) * FL_VP) = (x_[u_] >> 16) | (y_[u_] & 0xffff0000u);           \
        }                                                                                                   \
    }
#define FL_STORE(B_) FL_STK(B_, 0) FL_STK(B_, 1) FL_STK(B_, 2) FL_STK(B_, 3) FL_STV(B_, 0) FL_STV(B_, 1)
    FL_LOAD(0)
    // ---- RoPE: each row's angle chain theta_j = pos * theta_scale^j by repeated fp32 multiplication
    // (one thread per row), then (cos, sin) of every (row, dim pair)
    if (tid < m) {
        float th = (float) (p0 + tid);
        for (int j = 0; j < NP; ++j) {
            s_th[tid * NP + j] = th;
            th = th * a.theta_scale;
        }
    }
    lds_sync();
    for (int i = tid; i < m * NP; i += 512) {
        float sn, cs;
        z_sincos(s_th[i], sn, cs);
        s_cs[i] = make_float2(cs, sn);
    }
    lds_sync();
    // ---- queries: wave w forms row-heads w, w + 8, ... (lane = dim pair): per-head RMSNorm, |temp|,
    // RoPE; every input load of the wave is issued before the arithmetic
    {
        constexpr int QW = 8;                                        // row-heads per wave at most
        float2 xq[QW];
#pragma unroll
        for (int k = 0; k < QW; ++k) {
            const int rq = min(wave + 8 * k, P - 1), i = rq / GRP, qh = g * GRP + rq % GRP;
            xq[k] = *(const float2 *) (a.qkvg + (int64_t) (t0 + i) * a.R + (int64_t) qh * HD + 2 * lane);
        }
#pragma unroll
        for (int k = 0; k < QW; ++k) {
            const int rq = wave + 8 * k;
            if (rq < P) {                                            // (wave-uniform)
                const int i = rq / GRP, qh = g * GRP + rq % GRP;
                const float2 c = s_cs[i * NP + lane];
                float y0, y1;
                norm_rope<HD>(xq[k].x, xq[k].y, a.temp[qh], a.qk_eps, c.x, c.y, y0, y1);
                *(float2 *) &s_q[rq * (HD + 4) + 2 * lane] = make_float2(y0, y1);
            }
        }
    }
    lds_sync();
    const int rh = 16 * wq + c16;                                    // the lane's row-head (B columns)
    const bool rh_ok = rh < P;
    const int row = rh_ok ? rh / GRP : 0, pos = p0 + row;
    const float qscale = a.scale * 1.44269504088896341f;             // scores to log2 units
    v8h_t qh[KS], ql[KS];                                            // Q[rh][32 ks + 8 q4 .. + 7] hi / lo
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        uint32_t hh[4], ll[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float2 x = rh_ok ? *(const float2 *) &s_q[rh * (HD + 4) + 32 * ks + 8 * q4 + 2 * u] : make_float2(0.0f, 0.0f);
            hh[u] = f16_split2(x.x, x.y, ll[u]);
        }
        qh[ks] = __builtin_bit_cast(v8h_t, make_uint4(hh[0], hh[1], hh[2], hh[3]));
        ql[ks] = __builtin_bit_cast(v8h_t, make_uint4(ll[0], ll[1], ll[2], ll[3]));
    }
    lds_sync();                                                      // queries read: LDS free for the K / V buffers
    FL_STORE(0)
    if (nseg > 1) { FL_LOAD(1) }
    lds_sync();
    const bool active = 16 * wq < P;                                 // the wave has row-heads
    float m_run = -__builtin_inff(), l_part = 0.0f;
    v4f_t o[DT];
#pragma unroll
    for (int d = 0; d < DT; ++d) o[d] = (v4f_t) {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s = 0; s < nseg; ++s) {
        if (s + 1 < nseg) {                                          // the next segment into the other buffer
            FL_STORE((s + 1) & 1)
            if (s + 2 < nseg) { FL_LOAD(s + 2) }
        }
        if (active) {
            const uint16_t * bkh = (const uint16_t *) (sm_fl + (s & 1) * FL_BUF), * bkl = bkh + FL_SEG * FL_KP;
            const uint16_t * bvh = bkh + 2 * FL_SEG * FL_KP, * bvl = bvh + HD * FL_VP;
            // S^T for the wave's 16 row-heads and its 32 keys of the segment, in log2 units; the causal
            // mask only in segments reaching past the tile's first row (block-uniform)
            const bool masked = FL_SEG * s + FL_SEG - 1 > p0;
            float sc[2][4];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                v4f_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
                const int kr = (32 * kh + 16 * mt + c16) * FL_KP + 8 * q4;
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const v8h_t kh_ = *(const v8h_t *) &bkh[kr + 32 * ks];
                    const v8h_t kl_ = *(const v8h_t *) &bkl[kr + 32 * ks];
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh_, qh[ks], acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl_, qh[ks], acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh_, ql[ks], acc, 0, 0, 0);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) sc[mt][i] = acc[i] * qscale;
                if (masked) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int key = FL_SEG * s + 32 * kh + 16 * mt + 4 * q4 + i;
                        if (!(rh_ok && key <= pos)) sc[mt][i] = -__builtin_inff();
                    }
                }
            }
            float mx = fmaxf(fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3])), fmaxf(fmaxf(sc[1][0], sc[1][1]), fmaxf(sc[1][2], sc[1][3])));
            mx = fl_max4(mx);
            const bool need = mx > m_run + FL_TAU;                   // (the first keys: m_run = -inf)
            if (__any(need)) {
                const float m_new = need ? mx : m_run;
                const float alpha = need ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;   // (0 from -inf)
#pragma unroll
                for (int d = 0; d < DT; ++d) o[d] = o[d] * alpha;
                l_part = l_part * alpha;
                m_run = m_new;
            }
            const float mref = m_run == -__builtin_inff() ? 0.0f : m_run;    // (all keys so far masked: weights 0)
            v8h_t ph, pl;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float p = __builtin_amdgcn_exp2f(sc[j >> 2][j & 3] - mref);
                l_part = l_part + p;
                const _Float16 hi = (_Float16) p;
                ph[j] = hi;
                pl[j] = (_Float16) (p - (float) hi);
            }
            // O^T += V^T P^T for the wave's row-heads, every dim tile
#pragma unroll
            for (int d = 0; d < DT; ++d) {
                const int off = (16 * d + c16) * FL_VP + 32 * kh + 4 * q4;
                const uint2 h0 = *(const uint2 *) &bvh[off], h1 = *(const uint2 *) &bvh[off + 16];
                const uint2 l0 = *(const uint2 *) &bvl[off], l1 = *(const uint2 *) &bvl[off + 16];
                const v8h_t vh = __builtin_bit_cast(v8h_t, make_uint4(h0.x, h0.y, h1.x, h1.y));
                const v8h_t vl = __builtin_bit_cast(v8h_t, make_uint4(l0.x, l0.y, l1.x, l1.y));
                v4f_t acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, ph, o[d], 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(vl, ph, acc, 0, 0, 0);
                o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, pl, acc, 0, 0, 0);
            }
        }
        lds_sync();                                                  // segment s read, segment s + 1 stored
    }
    const float l_run = fl_sum4(l_part);
    float * mg = s_mrg + wq * (34 * 64);
    if (active && kh == 1) {
#pragma unroll
        for (int d = 0; d < DT; ++d)
#pragma unroll
            for (int i = 0; i < 4; ++i) mg[(4 * d + i) * 64 + lane] = o[d][i];
        mg[32 * 64 + lane] = m_run;
        mg[33 * 64 + lane] = l_run;
    }
    lds_sync();
    if (active && kh == 0 && rh_ok) {
        const float m1 = mg[32 * 64 + lane], l1 = mg[33 * 64 + lane];
        const float M = fmaxf(m_run, m1);                            // finite: key 0 is in every band
        const float a0 = __builtin_amdgcn_exp2f(m_run - M), a1 = __builtin_amdgcn_exp2f(m1 - M);
        const float l = __builtin_fmaf(l_run, a0, l1 * a1);
        const int h = rh % GRP, qhd = g * GRP + h, t = t0 + row;
        const float gsig = z_sigmoid(a.qkvg[(int64_t) t * a.R + (int64_t) (a.nh + 2 * nkv) * HD + qhd]);
        const float f = gsig / l;
        if (a.cap_gate && q4 == 0) a.cap_gate[(int64_t) t * a.nh + qhd] = gsig;
#pragma unroll
        for (int d = 0; d < DT; ++d) {
            float y[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) y[i] = __builtin_fmaf(o[d][i], a0, mg[(4 * d + i) * 64 + lane] * a1) * f;
            *(float4 *) (s_out + row * (GRP * HD) + h * HD + 16 * d + 4 * q4) = make_float4(y[0], y[1], y[2], y[3]);
        }
    }
    lds_sync();
    if (wave < 4) fa_store_rows<HD, GRP>(a, s_out, t0, m, g);        // (a 256-thread helper)
#undef FL_LOAD
#undef FL_LDK
#undef FL_LDV
#undef FL_STORE
#undef FL_STK
#undef FL_STV
}

} // namespace z2d
