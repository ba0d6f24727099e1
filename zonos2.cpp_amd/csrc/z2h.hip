// z2h.hip — context, weight repack/upload and step orchestration behind include/z2h.h.
//
// One HIP stream per context; every device buffer is allocated at create / finalize time, so a
// step performs no allocation. A step is a fixed sequence of kernels per layer (see z2h_kernels.h):
//   k_resnorm -> k_gemv(QKV+gate) -> k_attn_decode (QK-norm, RoPE, KV append, partials) -> k_attn_combine
//   -> k_gemv(W_o) -> k_resnorm(+attn, ffn_norm) -> [MoE] k_router_down -> k_router_tail
//   -> k_gemv(gate/up + SwiGLU, grouped) -> k_encode_rows -> k_gemv(down, grouped) | [dense] the same
//   FFN sequence ungrouped
// and after the last layer k_resnorm(output_norm) -> k_gemv(head, softcap).
#include "z2h.h"
#include "z2h_kernels.h"
#include "z2h_gemm.h"
#include "z2h_attn.h"
#include <hip/hip_ext.h>
#include "z2_formats.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <set>
#include <memory>
#include <string>
#include <thread>
#include <vector>

using namespace z2d;

// the token-pair K-split kernels, instantiated in z2h_tp.hip
namespace z2d {
extern template __global__ void k_gemv_split<WF_Q8_0, true, MT_G, false, true>(GemvArgs);
extern template __global__ void k_gemv_split<WF_Q8_0, false, MT_G, false, true>(GemvArgs);
extern template __global__ void k_gemv_split<WF_Q8_0, true, MT, false, true>(GemvArgs);
extern template __global__ void k_gemv_split<WF_Q8_0, false, MT, false, true>(GemvArgs);
extern template __global__ void k_gemv_split<WF_Q8_0, false, MT_G, true, true>(GemvArgs);
} // namespace z2d

namespace {

struct DevMat {
    int type = -1;
    bool m16 = false;                 // 16-row MFMA layout (Q4_K, Q8_0) instead of 64-row tiles
    int rows = 0, K = 0, nsb = 0, tiles = 0, n_mats = 1;
    uint8_t * w = nullptr;            // tiled bytes
    uint16_t * dpl = nullptr;         // Q6_K d plane
    int64_t mat_bytes = 0, dpl_elems = 0;
    bool ok() const { return w != nullptr; }
};

struct HostTensor { int type; int64_t ne[4]; std::vector<uint8_t> bytes; };

struct Layer {
    DevMat qkvg, wo, gate_exps, up_exps, down_exps, ffn_up, ffn_gate, ffn_down;
    float * attn_norm = nullptr, * ffn_norm = nullptr, * attn_temp = nullptr;
    bool moe = false;
    int k = 0, E = 0;
    float * r_down = nullptr, * r_down_b = nullptr, * r_m0t = nullptr, * r_m0_b = nullptr, * r_m2t = nullptr,
          * r_m2_b = nullptr, * r_m4t = nullptr, * r_norm = nullptr, * r_bias = nullptr, * r_eda = nullptr;
    float * logit_bias = nullptr, * mask = nullptr, * bias_buf = nullptr, * mask_buf = nullptr;
    std::map<std::string, HostTensor> stash;   // attn q/k/v/gate until all four are present
};

int act_of(int wtype) {
    switch (wtype) { case Z2H_Q4_K: case Z2H_Q6_K: return ACT_Q8_K; case Z2H_Q8_0: return ACT_Q8_0; case Z2H_F16: return ACT_F16; }
    return ACT_NONE;
}
int chunks_of(int wtype) {
    switch (wtype) { case Z2H_Q4_K: return 9; case Z2H_Q6_K: return 13; case Z2H_Q8_0: return 17; case Z2H_F16: return 32; }
    return 0;
}

} // namespace

// Weights of one model on one device, shared by every batch context created from it (refcounted:
// the creator's handle plus one reference per context).
struct z2h_model {
    z2h_hparams hp{};
    std::vector<int32_t> expert_used;
    int device = 0, W = 0, kmax = 1, rd = 0;
    std::string err;
    bool finalized = false;
    int refs = 1;
    int gen = 0;                      // bumped when a device pointer captured in step graphs changes
    std::vector<uint8_t> layer_skip;  // depth prune: nonzero = block bypassed (empty = none)
    int64_t bytes_w = 0;
    std::vector<void *> allocs;
    std::vector<uint8_t *> tab; std::vector<int> tab_type; std::vector<int64_t> tab_rows;
    DevMat head;
    float * output_norm = nullptr;
    DevMat spk_lda, spk_proj;
    float * spk_lda_b = nullptr, * spk_proj_b = nullptr;
    std::vector<Layer> layers;
    std::map<std::string, bool> seen;
};

struct z2h_ctx {
    z2h_model * m = nullptr;
    z2h_hparams hp{};                 // the model's (expert_used points into the model)
    int device = 0, n_slots = 0, S = 0, W = 0, kmax = 1, rd = 0;
    hipStream_t stream = nullptr;
    std::string err;
    bool finalized = false;
    int64_t bytes_kv = 0, bytes_scratch = 0;
    std::vector<void *> allocs;

    // KV cache [L][2][slot][kvh][S][hd]
    uint16_t * kv = nullptr;
    uint4 * kv_stage = nullptr;       // one slot's rows of one layer, host layout (kv_write / kv_read)

    // scratch (sized for n_slots tokens)
    int Tmax = 0, Kmax = 0, items_max = 0;   // Tmax: token rows of the scratch (steps and prefill chunks)
    int attn_slots = 2048;            // attention blocks resident at once (compute units x blocks per unit)
    int n_cu = 256;                   // compute units of the device
    int Tstep = 0;                    // columns a step may list (n_slots); captures are sized for it
    int pch = 0;                      // prefill chunk rows (<= Tmax)
    int max_rows = 0;                 // requested row capacity (z2h_create_batch_rows)
    int32_t * d_emb_map = nullptr;    // [Tmax] per-row embedding override
    int32_t * d_head_rows = nullptr;  // [Tmax] rows of a mixed pass that get logits
    int32_t * d_slot = nullptr, * d_npast = nullptr, * d_ids = nullptr; float * d_emb = nullptr;
    float * spk_io = nullptr;         // speaker projection: spk | lda out | proj out | delta
    float * res = nullptr, * res2 = nullptr, * cur = nullptr, * qkvg = nullptr, * wo_out = nullptr;
    float * part_o = nullptr, * part_ml = nullptr;
    float2 * rope = nullptr;          // [S][hd/2] RoPE (cos, sin) per position and dim pair
    float * pf_kv = nullptr;          // z2h_prefill: the prompt's fp32 K/V rows [L][2][nkv][S][hd] (one slot at a time)
    ActBuf act{}, act_y{};
    float * attn_o = nullptr;         // [T][nh*hd] gated attention output
    float * state = nullptr;          // [L][T][rd]
    float * state_ext = nullptr;      // [T][rd] external state for moe_forward
    float * state_one = nullptr;      // when set: the router state of the one layer run (no per-layer table)
    int32_t * sel = nullptr; float * wsel = nullptr;
    int32_t * r_off = nullptr, * r_perm = nullptr;   // routes grouped by expert ([E+1] offsets, [T*k] ids)
    float * gu_g = nullptr, * gu_u = nullptr, * eo = nullptr, * logits = nullptr, * tmp_x = nullptr;
    int * d_err = nullptr;
    int4 * d_tiles = nullptr;         // [items_max] attention tile entries of a kv_pre pass (k_attn_tile)
    int4 * h_tiles = nullptr;         // pinned staging for them
    int32_t * h_pin = nullptr;        // pinned staging for step inputs
    size_t h_pin_bytes = 0;

    // frame sampler: per-column settings, histories, draws and codes (device + pinned staging)
    SampleParams * d_sp = nullptr; int32_t * d_hist = nullptr, * d_hlen = nullptr, * d_codes = nullptr;
    double * d_u = nullptr;
    uint8_t * h_samp = nullptr;
    int resident_T = 0;               // columns whose next-step inputs z2h_sample_feed left in d_ids / d_npast
    int resident_last = 0;            // width of the last step whose inputs and logits are in d_* / logits
    std::vector<int32_t> last_np;     // host copy of the device table's n_past per column (last step, + 1 per feed)

    // HIP graphs of the whole step, one per (batch width, embedding-injection) pair
    bool use_graphs = true;
    std::map<std::pair<int, int>, hipGraphExec_t> graphs;
    int graph_gen = 0;                // the model generation the graphs were captured against

    // per-kernel event timing
    bool prof = false;
    std::vector<hipEvent_t> ev;
    std::vector<int> ev_fam;
    int ev_used = 0;
    int prof_fam = -1;                // family of the launches being issued (profiling windows)

    // capture
    bool capture = false;
    std::vector<uint8_t *> cap;       // per `what`: [L][Tmax][width]
    int cap_T = 0;
};

namespace {

int seterr(z2h_ctx * c, int code, const std::string & m) { if (c) c->err = m; return code; }
int seterr(z2h_model * c, int code, const std::string & m) { if (c) c->err = m; return code; }
int upload_mat_t64(z2h_model * mdl, int type, int64_t K, int64_t rows, int n_mats, const uint8_t * src, DevMat & dm);
int launch_attn_fa(z2h_ctx * ctx, const AttnArgs & a, int grid);
int launch_attn(z2h_ctx * ctx, const AttnArgs & a, int grid);
int launch_attn_tile(z2h_ctx * ctx, const AttnArgs & a, int n_tiles);
int launch_kv_append(z2h_ctx * ctx, const AttnArgs & a, int T);

constexpr int PROF_MAX = 16384;

// Profiling: while a window is open, every launch inside a prof_scope of family `fam` goes through
// hipExtLaunchKernelGGL with its own start / stop event pair, which the runtime timestamps at the
// kernel's own start and end (no extra packets between the launches of the step).
struct prof_scope {
    z2h_ctx * c; int keep;
    prof_scope(z2h_ctx * ctx, int fam) : c(ctx), keep(ctx->prof_fam) { c->prof_fam = fam; }
    ~prof_scope() { c->prof_fam = keep; }
};
// the event pair for the next launch, or nulls outside a window
inline void prof_pair(z2h_ctx * c, hipEvent_t & e0, hipEvent_t & e1) {
    e0 = e1 = nullptr;
    if (!c->prof || c->prof_fam < 0 || c->ev_used >= PROF_MAX) return;
    const int idx = c->ev_used++;
    c->ev_fam[idx] = c->prof_fam;
    e0 = c->ev[2 * idx]; e1 = c->ev[2 * idx + 1];
}
#define KL(K_, G_, B_, L_, S_, ...) do { hipEvent_t e0_, e1_; prof_pair(ctx, e0_, e1_); \
    if (e0_) hipExtLaunchKernelGGL(K_, G_, B_, L_, S_, e0_, e1_, 0, __VA_ARGS__); \
    else hipLaunchKernelGGL(K_, G_, B_, L_, S_, __VA_ARGS__); } while (0)

#define HIPX(expr) do { hipError_t e_ = (expr); if (e_ != hipSuccess) \
    return seterr(ctx, Z2H_EDEVICE, std::string(#expr) + ": " + hipGetErrorString(e_)); } while (0)
#define HIPM(expr) do { hipError_t e_ = (expr); if (e_ != hipSuccess) \
    return seterr(mdl, Z2H_EDEVICE, std::string(#expr) + ": " + hipGetErrorString(e_)); } while (0)

template <class O, class T>
int dalloc(O * owner, T ** p, size_t bytes, int64_t & counter) {
    void * v = nullptr;
    if (bytes == 0) bytes = 16;
    if (hipMalloc(&v, bytes) != hipSuccess) return seterr(owner, Z2H_ENOMEM, "hipMalloc failed (" + std::to_string(bytes) + " B)");
    owner->allocs.push_back(v);
    counter += (int64_t) bytes;
    *p = (T *) v;
    return Z2H_OK;
}

int upload_f32(z2h_model * mdl, const HostTensor & t, float ** out, int64_t n_expect) {
    const int64_t n = t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3];
    if (n_expect >= 0 && n != n_expect) return seterr(mdl, Z2H_EINVAL, "unexpected vector length");
    std::vector<float> f((size_t) n);
    const int64_t rows = n / t.ne[0];
    for (int64_t r = 0; r < rows; ++r) {
        const uint8_t * src = t.bytes.data() + r * z2::row_bytes(t.type, t.ne[0]);
        float * y = f.data() + r * t.ne[0];
        switch (t.type) {
            case Z2H_F32: std::memcpy(y, src, t.ne[0] * 4); break;
            case Z2H_F16: for (int64_t i = 0; i < t.ne[0]; ++i) { uint16_t h; std::memcpy(&h, src + 2 * i, 2); y[i] = z2::f16_to_f32(h); } break;
            case Z2H_Q8_0:
                for (int64_t b = 0; b < t.ne[0] / 32; ++b) {
                    uint16_t h; std::memcpy(&h, src + 34 * b, 2);
                    const float d = z2::f16_to_f32(h);
                    for (int j = 0; j < 32; ++j) y[32 * b + j] = (float) (int8_t) src[34 * b + 2 + j] * d;
                }
                break;
            default: return seterr(mdl, Z2H_ENOTSUP, "router/vector tensors must be F32, F16 or Q8_0");
        }
    }
    if (int rc = dalloc(mdl, out, f.size() * 4, mdl->bytes_w)) return rc;
    HIPM(hipMemcpy(*out, f.data(), f.size() * 4, hipMemcpyHostToDevice));
    return Z2H_OK;
}

// W [out][in] as fp32 rows padded to in + 4 floats (the router tail's LDS layout)
int upload_f32_rows_padded(z2h_model * mdl, const HostTensor & t, float ** out) {
    const int64_t in = t.ne[0], outn = t.ne[1], ld = in + 4;
    std::vector<float> rows((size_t) (ld * outn), 0.0f);
    for (int64_t r = 0; r < outn; ++r) {
        const uint8_t * src = t.bytes.data() + r * z2::row_bytes(t.type, in);
        for (int64_t i = 0; i < in; ++i) {
            float v = 0.0f;
            if (t.type == Z2H_F32) std::memcpy(&v, src + 4 * i, 4);
            else if (t.type == Z2H_F16) { uint16_t h; std::memcpy(&h, src + 2 * i, 2); v = z2::f16_to_f32(h); }
            else if (t.type == Z2H_Q8_0) { uint16_t h; std::memcpy(&h, src + 34 * (i / 32), 2); v = (float) (int8_t) src[34 * (i / 32) + 2 + i % 32] * z2::f16_to_f32(h); }
            else return seterr(mdl, Z2H_ENOTSUP, "router matrices must be F32, F16 or Q8_0");
            rows[r * ld + i] = v;
        }
    }
    if (int rc = dalloc(mdl, out, rows.size() * 4, mdl->bytes_w)) return rc;
    HIPM(hipMemcpy(*out, rows.data(), rows.size() * 4, hipMemcpyHostToDevice));
    return Z2H_OK;
}

// Repack into the 16-row MFMA layout (see k_gemv_mfma): per (group, unit) the lane-owned 8-byte
// k-slices of every 32-element sub-block, chunk-major for the 64 lanes, then the rows' scale headers.
int upload_mat_m16(z2h_model * mdl, int type, int64_t K, int64_t rows, int n_mats, const uint8_t * src, DevMat & dm) {
    const int UB = type == Z2H_Q4_K ? 2304 : 4352, QS = type == Z2H_Q4_K ? 2 : 4;
    dm.type = type; dm.m16 = true; dm.rows = (int) rows; dm.K = (int) K; dm.nsb = (int) ((K + 255) / 256);
    dm.tiles = (int) ((rows + 15) / 16); dm.n_mats = n_mats;
    dm.mat_bytes = (int64_t) dm.tiles * dm.nsb * UB;
    const int64_t rb = z2::row_bytes(type, K);
    std::vector<uint8_t> out((size_t) dm.mat_bytes * n_mats, 0);
    auto do_rows = [&](int64_t g0, int64_t g1) {          // global 16-row group range over all matrices
        for (int64_t gg = g0; gg < g1; ++gg) {
            const int e = (int) (gg / dm.tiles), g = (int) (gg % dm.tiles);
            uint8_t * mat = out.data() + (size_t) e * dm.mat_bytes;
            for (int r = 0; r < 16; ++r) {
                const int64_t row = (int64_t) g * 16 + r;
                if (row >= rows) break;
                const uint8_t * rp = src + ((int64_t) e * rows + row) * rb;
                for (int sb = 0; sb < dm.nsb; ++sb) {
                    uint8_t * unit = mat + ((size_t) g * dm.nsb + sb) * UB;
                    for (int q = 0; q < 4; ++q) {
                        const int lane = 16 * q + r;
                        for (int c = 0; c < QS; ++c) {
                            uint8_t * dst = unit + ((size_t) c * 64 + lane) * 16;
                            for (int h = 0; h < 2; ++h) {           // two sub-block slices per chunk
                                if (type == Z2H_Q4_K) {
                                    const int pr = 2 * c + h;        // qs pair
                                    std::memcpy(dst + 8 * h, rp + 144 * sb + 16 + 32 * pr + 8 * q, 8);
                                } else {
                                    const int64_t blk = (int64_t) sb * 8 + 2 * c + h;
                                    if (blk * 32 < K) std::memcpy(dst + 8 * h, rp + 34 * blk + 2 + 8 * q, 8);
                                }
                            }
                        }
                    }
                    uint8_t * hd = unit + (size_t) QS * 64 * 16 + (size_t) r * 16;
                    if (type == Z2H_Q4_K) std::memcpy(hd, rp + 144 * sb, 16);
                    else
                        for (int b = 0; b < 8; ++b) {
                            const int64_t blk = (int64_t) sb * 8 + b;
                            if (blk * 32 < K) std::memcpy(hd + 2 * b, rp + 34 * blk, 2);
                        }
                }
            }
        }
    };
    const int64_t total = (int64_t) n_mats * dm.tiles;
    const int nth = (int) std::max<int64_t>(1, std::min<int64_t>(16, total / 64));
    std::vector<std::thread> th;
    for (int i = 0; i < nth; ++i) th.emplace_back([&, i] { do_rows(total * i / nth, total * (i + 1) / nth); });
    for (auto & t : th) t.join();
    if (int rc = dalloc(mdl, &dm.w, out.size(), mdl->bytes_w)) return rc;
    HIPM(hipMemcpy(dm.w, out.data(), out.size(), hipMemcpyHostToDevice));
    return Z2H_OK;
}

// Q6_K matrices in the 16-row MFMA layout (k_gemv_mfma / k_gemv_split<WF_Q6_K>): per (16-row group, 256-column
// unit) 3360 B = two 1 KiB low-nibble chunks and one 1 KiB high-bit chunk (16 bytes per lane,
// lane-major), then the 16 rows' int8 scales (16 B each) and f16 d (2 B each). Lane l = (k-slice
// q = l/16, row r = l%16) owns elements 32m + 8q + j (j < 8) of each 32-element chunk m of the
// superblock, as 6-bit unsigned values v (the GGUF value + 32): low dword m byte j = (v_j & 15) |
// (v_{4+j} & 15) << 4; high dword m/2 byte j = h(v_j, m) | h(v_{4+j}, m) << 2 | h(v_j, m+1) << 4 |
// h(v_{4+j}, m+1) << 6 for even m, h = bits 4-5.
int upload_mat_m16q6(z2h_model * mdl, int64_t K, int64_t rows, int n_mats, const uint8_t * src, DevMat & dm) {
    constexpr int UB = 3360;
    if (K % 256) return seterr(mdl, Z2H_EINVAL, "K-quant row not a multiple of 256");
    dm.type = Z2H_Q6_K; dm.m16 = true; dm.rows = (int) rows; dm.K = (int) K; dm.nsb = (int) (K / 256);
    dm.tiles = (int) ((rows + 15) / 16); dm.n_mats = n_mats;
    dm.mat_bytes = (int64_t) dm.tiles * dm.nsb * UB;
    const int64_t rb = z2::row_bytes(Z2H_Q6_K, K);
    std::vector<uint8_t> out((size_t) dm.mat_bytes * n_mats, 0);
    auto do_groups = [&](int64_t g0, int64_t g1) {
        for (int64_t gg = g0; gg < g1; ++gg) {
            const int e = (int) (gg / dm.tiles), g = (int) (gg % dm.tiles);
            uint8_t * mat = out.data() + (size_t) e * dm.mat_bytes;
            for (int r = 0; r < 16; ++r) {
                const int64_t row = (int64_t) g * 16 + r;
                if (row >= rows) break;
                const uint8_t * rp = src + ((int64_t) e * rows + row) * rb;
                for (int sb = 0; sb < dm.nsb; ++sb) {
                    const uint8_t * blk = rp + 210 * sb;             // ql[128] qh[64] scales[16] d
                    uint8_t v[256];
                    for (int n = 0; n < 2; ++n) {
                        const uint8_t * ql = blk + 64 * n, * qh = blk + 128 + 32 * n;
                        for (int l = 0; l < 32; ++l) {
                            v[128 * n + l]      = (uint8_t) ((ql[l] & 15) | ((qh[l] & 3) << 4));
                            v[128 * n + l + 32] = (uint8_t) ((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4));
                            v[128 * n + l + 64] = (uint8_t) ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4));
                            v[128 * n + l + 96] = (uint8_t) ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4));
                        }
                    }
                    uint8_t * unit = mat + ((size_t) g * dm.nsb + sb) * UB;
                    for (int q = 0; q < 4; ++q) {
                        const int lane = 16 * q + r;
                        uint32_t lo[8] = {0}, hi[4] = {0};
                        for (int m = 0; m < 8; ++m)
                            for (int j = 0; j < 4; ++j) {
                                const uint32_t e0 = v[32 * m + 8 * q + j], e1 = v[32 * m + 8 * q + 4 + j];
                                lo[m] |= ((e0 & 15u) | ((e1 & 15u) << 4)) << (8 * j);
                                hi[m >> 1] |= (((e0 >> 4) & 3u) | (((e1 >> 4) & 3u) << 2)) << (8 * j + 4 * (m & 1));
                            }
                        std::memcpy(unit + (size_t) lane * 16, lo, 16);
                        std::memcpy(unit + (size_t) (64 + lane) * 16, lo + 4, 16);
                        std::memcpy(unit + (size_t) (128 + lane) * 16, hi, 16);
                    }
                    std::memcpy(unit + 3072 + 16 * r, blk + 192, 16);
                    std::memcpy(unit + 3328 + 2 * r, blk + 208, 2);
                }
            }
        }
    };
    const int64_t total = (int64_t) n_mats * dm.tiles;
    const int nth = (int) std::max<int64_t>(1, std::min<int64_t>(16, total / 64));
    std::vector<std::thread> th;
    for (int i = 0; i < nth; ++i) th.emplace_back([&, i] { do_groups(total * i / nth, total * (i + 1) / nth); });
    for (auto & t : th) t.join();
    if (int rc = dalloc(mdl, &dm.w, out.size(), mdl->bytes_w)) return rc;
    HIPM(hipMemcpy(dm.w, out.data(), out.size(), hipMemcpyHostToDevice));
    return Z2H_OK;
}

// Repack n_mats matrices of `rows` x K (GGUF rows, contiguous) into the device layout: the 16-row
// MFMA layouts for Q4_K / Q8_0 / Q6_K, the 64-row tiles for F16.
int upload_mat(z2h_model * mdl, int type, int64_t K, int64_t rows, int n_mats, const uint8_t * src, DevMat & dm) {
    if (type == Z2H_Q6_K) return upload_mat_m16q6(mdl, K, rows, n_mats, src, dm);
    if (type == Z2H_Q4_K || type == Z2H_Q8_0) {
        if (type == Z2H_Q4_K && K % 256) return seterr(mdl, Z2H_EINVAL, "K-quant row not a multiple of 256");
        if (type == Z2H_Q8_0 && K % 32) return seterr(mdl, Z2H_EINVAL, "Q8_0 row not a multiple of 32");
        return upload_mat_m16(mdl, type, K, rows, n_mats, src, dm);
    }
    return upload_mat_t64(mdl, type, K, rows, n_mats, src, dm);
}

// Repack n_mats matrices of `rows` x K (GGUF rows, contiguous) into the 64-row tiled layout.
int upload_mat_t64(z2h_model * mdl, int type, int64_t K, int64_t rows, int n_mats, const uint8_t * src, DevMat & dm) {
    const int C = chunks_of(type);
    if (!C) return seterr(mdl, Z2H_ENOTSUP, "matrix type not supported on the device (F16, Q8_0, Q4_K, Q6_K)");
    if ((type == Z2H_Q4_K || type == Z2H_Q6_K) && K % 256) return seterr(mdl, Z2H_EINVAL, "K-quant row not a multiple of 256");
    if (type == Z2H_Q8_0 && K % 32) return seterr(mdl, Z2H_EINVAL, "Q8_0 row not a multiple of 32");
    dm.type = type; dm.rows = (int) rows; dm.K = (int) K; dm.nsb = (int) ((K + 255) / 256);
    dm.tiles = (int) ((rows + TILE - 1) / TILE); dm.n_mats = n_mats;
    dm.mat_bytes = (int64_t) dm.tiles * dm.nsb * C * TILE * 16;
    dm.dpl_elems = type == Z2H_Q6_K ? (int64_t) dm.tiles * dm.nsb * TILE : 0;
    const int64_t rb = z2::row_bytes(type, K);
    std::vector<uint8_t> tiled((size_t) dm.mat_bytes * n_mats, 0);
    std::vector<uint16_t> dpl((size_t) dm.dpl_elems * n_mats, 0);
    auto repack_rows = [&](int e, int64_t r0, int64_t r1) {
        uint8_t * dst = tiled.data() + (size_t) e * dm.mat_bytes;
        for (int64_t r = r0; r < r1; ++r) {
            const uint8_t * row = src + ((int64_t) e * rows + r) * rb;
            const int64_t tile = r / TILE, lane = r % TILE;
            for (int sb = 0; sb < dm.nsb; ++sb) {
                uint8_t unit[512];
                std::memset(unit, 0, sizeof(unit));
                switch (type) {
                    case Z2H_Q4_K: std::memcpy(unit, row + 144 * sb, 144); break;
                    case Z2H_Q6_K:
                        std::memcpy(unit, row + 210 * sb, 208);
                        std::memcpy(&dpl[(size_t) e * dm.dpl_elems + ((size_t) tile * dm.nsb + sb) * TILE + lane], row + 210 * sb + 208, 2);
                        break;
                    case Z2H_Q8_0:
                        for (int b = 0; b < 8; ++b) {
                            const int64_t blk = (int64_t) sb * 8 + b;
                            if (blk * 32 >= K) break;
                            std::memcpy(unit + 32 * b, row + 34 * blk + 2, 32);
                            std::memcpy(unit + 256 + 2 * b, row + 34 * blk, 2);
                        }
                        break;
                    case Z2H_F16: {
                        const int64_t n = std::min<int64_t>(256, K - (int64_t) sb * 256);
                        std::memcpy(unit, row + (int64_t) sb * 512, (size_t) n * 2);
                        break;
                    }
                }
                for (int c = 0; c < C; ++c)
                    std::memcpy(dst + ((((size_t) tile * dm.nsb + sb) * C + c) * TILE + lane) * 16, unit + 16 * c, 16);
            }
        }
    };
    const int64_t total = (int64_t) n_mats * rows;
    const int nth = (int) std::max<int64_t>(1, std::min<int64_t>(16, total / 1024));
    std::vector<std::thread> th;
    for (int i = 0; i < nth; ++i)
        th.emplace_back([&, i] {
            for (int64_t g = total * i / nth; g < total * (i + 1) / nth; ) {
                const int e = (int) (g / rows);
                const int64_t r0 = g % rows, r1 = std::min<int64_t>(rows, r0 + (total * (i + 1) / nth - g));
                repack_rows(e, r0, r1);
                g += r1 - r0;
            }
        });
    for (auto & t : th) t.join();
    if (int rc = dalloc(mdl, &dm.w, tiled.size(), mdl->bytes_w)) return rc;
    HIPM(hipMemcpy(dm.w, tiled.data(), tiled.size(), hipMemcpyHostToDevice));
    if (type == Z2H_Q6_K) {
        if (int rc = dalloc(mdl, &dm.dpl, dpl.size() * 2, mdl->bytes_w)) return rc;
        HIPM(hipMemcpy(dm.dpl, dpl.data(), dpl.size() * 2, hipMemcpyHostToDevice));
    }
    return Z2H_OK;
}

bool parse_layer(const std::string & name, int & L, std::string & rest) {
    if (name.rfind("blk.", 0) != 0) return false;
    const size_t dot = name.find('.', 4);
    if (dot == std::string::npos) return false;
    L = std::atoi(name.substr(4, dot - 4).c_str());
    rest = name.substr(dot + 1);
    return true;
}

int fuse_qkvg(z2h_model * mdl, Layer & ly) {
    static const char * parts[4] = {"attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_gate.weight"};
    for (auto * p : parts) if (!ly.stash.count(p)) return Z2H_OK;   // not complete yet
    const int type = ly.stash["attn_q.weight"].type;
    const int64_t K = ly.stash["attn_q.weight"].ne[0];
    int64_t rows = 0;
    for (auto * p : parts) {
        const HostTensor & t = ly.stash[p];
        if (t.type != type || t.ne[0] != K) return seterr(mdl, Z2H_ENOTSUP, "attention projections must share type and input size");
        rows += t.ne[1];
    }
    std::vector<uint8_t> cat;
    for (auto * p : parts) cat.insert(cat.end(), ly.stash[p].bytes.begin(), ly.stash[p].bytes.end());
    ly.stash.clear();
    return upload_mat(mdl, type, K, rows, 1, cat.data(), ly.qkvg);
}

// pinned staging of one z2h_sample call: settings | histories | counts | draws | codes
size_t samp_stage_bytes(int T, int ncb) {
    return (size_t) T * sizeof(SampleParams) + (size_t) T * ncb * (Z2H_SAMPLE_HIST_MAX * 4 + 4 + 8 + 4) + 64;
}

int alloc_scratch(z2h_ctx * ctx) {
    const auto & hp = ctx->hp;
    // rows: a step's columns, or a pass of up to max(Z2H_PREFILL_CHUNK_MAX, max_rows) rows (a prefill
    // chunk or a mixed pass); a prompt is prefilled in passes of the whole row capacity by default
    const int pmax = Z2H_PREFILL_CHUNK_MAX;
    const int T = std::max({ctx->n_slots, pmax, ctx->max_rows}), d = hp.n_embd, nh = hp.n_head, nkv = hp.n_head_kv, hd = hp.head_dim;
    const int ff = hp.n_ff, K = ctx->kmax, E = std::max(1, hp.n_expert), rd = std::max(1, ctx->rd);
    ctx->Tmax = T;
    ctx->Tstep = ctx->n_slots;
    ctx->pch = T;
    ctx->Kmax = std::max({kpad(d), kpad(nh * hd), kpad(ff), kpad(std::max(1, hp.spk_dim)), kpad(std::max(1, hp.spk_lda_dim))});
    const int R = (nh + 2 * nkv) * hd + nh;
    const int grp = nh / nkv;
    ctx->items_max = T * ((ctx->S + ATT_CH - 1) / ATT_CH) * nkv;
    int64_t & b = ctx->bytes_scratch;
    int rc = 0;
    const int KM = ctx->Kmax;
    const int W = ctx->W;
    // act_y rows per token: the token's routes' FFN activations, or (the head's gathered rows) one
    // activation row of any matmul
    const size_t ypr = std::max((size_t) std::max(K, 1) * kpad(std::max(ff, 1)), (size_t) KM);
    if ((rc = dalloc(ctx, &ctx->d_slot, T * 4, b)) || (rc = dalloc(ctx, &ctx->d_npast, T * 4, b)) ||
        (rc = dalloc(ctx, &ctx->d_ids, (size_t) T * W * 4, b)) || (rc = dalloc(ctx, &ctx->d_emb, (size_t) T * d * 4, b)) ||
        (rc = dalloc(ctx, &ctx->res, (size_t) T * d * 4, b)) || (rc = dalloc(ctx, &ctx->res2, (size_t) T * d * 4, b)) ||
        (rc = dalloc(ctx, &ctx->cur, (size_t) T * d * 4, b)) ||
        (rc = dalloc(ctx, &ctx->tmp_x, (size_t) T * d * 4, b)) ||
        (rc = dalloc(ctx, &ctx->qkvg, (size_t) T * R * 4, b)) ||
        (rc = dalloc(ctx, &ctx->wo_out, (size_t) T * d * 4, b)) ||
        (rc = dalloc(ctx, &ctx->part_o, (size_t) ctx->items_max * grp * hd * 4, b)) ||
        (rc = dalloc(ctx, &ctx->part_ml, (size_t) ctx->items_max * grp * 2 * 4, b)) ||
        (rc = dalloc(ctx, &ctx->pf_kv, (size_t) hp.n_layer * 2 * nkv * ctx->S * hd * 4, b)) ||
        (rc = dalloc(ctx, &ctx->act.q, (size_t) T * KM, b)) || (rc = dalloc(ctx, &ctx->act.d32, (size_t) T * (KM / 32) * 4, b)) ||
        (rc = dalloc(ctx, &ctx->act.d256, (size_t) T * (KM / 256) * 4, b)) || (rc = dalloc(ctx, &ctx->act.bs, (size_t) T * (KM / 16) * 2, b)) ||
        (rc = dalloc(ctx, &ctx->act.h, (size_t) T * KM * 2, b)) ||
        (rc = dalloc(ctx, &ctx->act_y.q, (size_t) T * ypr, b)) ||
        (rc = dalloc(ctx, &ctx->act_y.d32, (size_t) T * (ypr / 32) * 4, b)) ||
        (rc = dalloc(ctx, &ctx->act_y.d256, (size_t) T * (ypr / 256) * 4, b)) ||
        (rc = dalloc(ctx, &ctx->act_y.bs, (size_t) T * (ypr / 16) * 2, b)) ||
        (rc = dalloc(ctx, &ctx->act_y.h, (size_t) T * ypr * 2, b)) ||
        (rc = dalloc(ctx, &ctx->d_head_rows, (size_t) T * 4, b)) ||
        (rc = dalloc(ctx, &ctx->attn_o, (size_t) T * nh * hd * 4, b)) ||
        (rc = dalloc(ctx, &ctx->state, (size_t) hp.n_layer * T * rd * 4, b)) || (rc = dalloc(ctx, &ctx->state_ext, (size_t) T * rd * 4, b)) ||
        (rc = dalloc(ctx, &ctx->sel, (size_t) T * K * 4, b)) || (rc = dalloc(ctx, &ctx->wsel, (size_t) T * K * 4, b)) ||
        (rc = dalloc(ctx, &ctx->r_off, (size_t) (E + 1) * 4, b)) || (rc = dalloc(ctx, &ctx->r_perm, (size_t) T * K * 4, b)) ||
        (rc = dalloc(ctx, &ctx->d_emb_map, (size_t) T * 4, b)) ||
        (rc = dalloc(ctx, &ctx->gu_g, (size_t) T * K * std::max(ff, 1) * 4, b)) || (rc = dalloc(ctx, &ctx->gu_u, (size_t) T * K * std::max(ff, 1) * 4, b)) ||
        (rc = dalloc(ctx, &ctx->eo, (size_t) T * K * d * 4, b)) ||
        (rc = dalloc(ctx, &ctx->logits, (size_t) T * hp.n_codebooks * hp.audio_vocab * 4, b)) ||
        (rc = dalloc(ctx, &ctx->d_err, 16, b)))
        return rc;
    if (hp.spk_dim > 0 && hp.spk_lda_dim > 0 &&
        (rc = dalloc(ctx, &ctx->spk_io, (size_t) Z2H_SPEAKER_MAX * (kpad(hp.spk_dim) + kpad(hp.spk_lda_dim) + 2 * kpad(d)) * 4, b)))
        return rc;
    (void) E;
    if ((rc = dalloc(ctx, &ctx->d_tiles, (size_t) 2 * ctx->items_max * sizeof(int4), b))) return rc;
    // RoPE (cos, sin) of every (position < S, dim pair), formed once by rope_cs's own arithmetic
    {
        const int np2 = hd / 2;
        if ((rc = dalloc(ctx, &ctx->rope, (size_t) ctx->S * np2 * sizeof(float2), b))) return rc;
        const int64_t n = (int64_t) ctx->S * np2;
        KL(k_rope_table, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, ctx->stream, ctx->rope, ctx->S, np2,
           std::pow(hp.rope_freq_base, -2.0f / (float) hd));
        HIPX(hipGetLastError());
        HIPX(hipStreamSynchronize(ctx->stream));
    }
    if (hipHostMalloc((void **) &ctx->h_tiles, (size_t) 2 * ctx->items_max * sizeof(int4), hipHostMallocDefault) != hipSuccess)
        return seterr(ctx, Z2H_ENOMEM, "hipHostMalloc failed");
    ctx->h_pin_bytes = (size_t) T * (4 + W) * 4;
    if (hipHostMalloc((void **) &ctx->h_pin, ctx->h_pin_bytes, hipHostMallocDefault) != hipSuccess)
        return seterr(ctx, Z2H_ENOMEM, "hipHostMalloc failed");
    const int ncb = std::max(1, (int) hp.n_codebooks);
    if ((rc = dalloc(ctx, &ctx->d_sp, (size_t) T * sizeof(SampleParams), b)) ||
        (rc = dalloc(ctx, &ctx->d_hist, (size_t) T * ncb * Z2H_SAMPLE_HIST_MAX * 4, b)) ||
        (rc = dalloc(ctx, &ctx->d_hlen, (size_t) T * ncb * 4, b)) || (rc = dalloc(ctx, &ctx->d_u, (size_t) T * ncb * 8, b)) ||
        (rc = dalloc(ctx, &ctx->d_codes, (size_t) T * ncb * 4, b)))
        return rc;
    if (hipHostMalloc((void **) &ctx->h_samp, samp_stage_bytes(T, ncb), hipHostMallocDefault) != hipSuccess)
        return seterr(ctx, Z2H_ENOMEM, "hipHostMalloc failed");
    return Z2H_OK;
}

// capture widths (elements per token, or per layer for grouping ids)
int64_t cap_width(const z2h_ctx * c, int what, int T) {
    const auto & hp = c->hp;
    const int d = hp.n_embd, nh = hp.n_head, nkv = hp.n_head_kv, hd = hp.head_dim;
    switch (what) {
        case Z2H_CAP_RES_IN: case Z2H_CAP_ATTN_IN: case Z2H_CAP_ATTN_OUT: case Z2H_CAP_FFN_IN:
        case Z2H_CAP_FFN_OUT: case Z2H_CAP_OUT_NORM: return (int64_t) T * d;
        case Z2H_CAP_Q: case Z2H_CAP_ATTN_O: return (int64_t) T * nh * hd;
        case Z2H_CAP_K: case Z2H_CAP_V: return (int64_t) T * nkv * hd;
        case Z2H_CAP_GATE: return (int64_t) T * nh;
        case Z2H_CAP_ROUTER_STATE: return (int64_t) T * std::max(1, c->rd);
        case Z2H_CAP_ROUTER_LOGITS: case Z2H_CAP_PROBS: return (int64_t) T * std::max(1, hp.n_expert);
        case Z2H_CAP_SEL: case Z2H_CAP_WEIGHTS: return (int64_t) T * c->kmax;
        case Z2H_CAP_COUNTS: return std::max(1, hp.n_expert);
        case Z2H_CAP_OFFSETS: return std::max(1, hp.n_expert) + 1;
        case Z2H_CAP_PERM: return (int64_t) T * c->kmax;
        case Z2H_CAP_EXPERT_OUT: return (int64_t) T * c->kmax * d;
    }
    return 0;
}

uint8_t * capp(z2h_ctx * c, int what, int L) {
    if (!c->capture) return nullptr;
    return c->cap[what] + (size_t) L * cap_width(c, what, c->Tstep) * 4;
}

int cap_copy(z2h_ctx * ctx, int what, int L, const void * src, int T) {
    if (!ctx->capture) return Z2H_OK;
    HIPX(hipMemcpyAsync(capp(ctx, what, L), src, (size_t) cap_width(ctx, what, T) * 4, hipMemcpyDeviceToDevice, ctx->stream));
    return Z2H_OK;
}

// ---------------------------------------------------------------- launch helpers
// Passes of more than 64 token rows (prefill chunks, mixed passes) run their Q4_K (m16) matmuls as
// GEMMs (k_gemm_q4k), decode steps the GEMVs: both fold a row's superblocks in the same order with
// the same operations. Every F16 (t64) matmul runs on k_gemm_f16, in its wide or narrow shape (same
// bits per row either way).
constexpr int GEMM_MIN_ROWS = 65;
bool use_gemm(const DevMat & m, int n_tok) {
    if (!m.m16 && m.type == Z2H_F16) return true;
    return n_tok >= GEMM_MIN_ROWS && m.m16 && m.type == Z2H_Q4_K;
}
// gate and up fused with SwiGLU in one GEMM launch: same type, layout and shape
bool gemm_dual_ok(const DevMat & g, const DevMat & u) {
    return g.type == u.type && g.m16 == u.m16 && g.nsb == u.nsb && g.tiles == u.tiles && g.rows == u.rows && g.mat_bytes == u.mat_bytes;
}

int launch_gemm(z2h_ctx * ctx, const DevMat & m0, const DevMat * m1, const GemvArgs & g, int fam) {
    const bool dual = g.mode == MM_SWIGLU;
    if (dual && (!m1 || !gemm_dual_ok(m0, *m1))) return seterr(ctx, Z2H_EINVAL, "gate/up layouts differ");
    if (!dual && m1) {
        // two matrices, two outputs: one launch each
        GemvArgs g0 = g, g1 = g;
        g1.out[0] = g.out[1];
        if (int rc = launch_gemm(ctx, m0, nullptr, g0, fam)) return rc;
        return launch_gemm(ctx, *m1, nullptr, g1, fam);
    }
    if (g.grouped && (!g.r_off || !g.r_perm)) return seterr(ctx, Z2H_EINVAL, "grouped GEMM without the route grouping");
    prof_scope ps(ctx, fam);
    GemmArgs a{};
    a.w[0] = m0.w; a.w[1] = dual ? m1->w : m0.w; a.mat_bytes = m0.mat_bytes;
    a.nsb = m0.nsb; a.rows = m0.rows; a.tiles = m0.tiles;
    a.grouped = g.grouped; a.n_tok = g.n_tok; a.k = g.k; a.E = g.E; a.act_by_route = g.act_by_route;
    a.r_off = g.r_off; a.r_perm = g.r_perm; a.act = g.act;
    a.out = g.out[0]; a.out_ld = g.out_ld; a.epi = g.epi; a.cap = g.cap; a.route_w = g.route_w;
    if (m0.type == Z2H_Q4_K) {
        const dim3 grid(dual ? (m0.tiles + 3) / 4 : (m0.tiles + 7) / 8, gemm_slots(a.grouped, a.n_tok, a.k, a.E, GM_T));
        if (dual) KL(k_gemm_q4k<true>, grid, dim3(256), gemm_q4k_lds(), ctx->stream, a);
        else KL(k_gemm_q4k<false>, grid, dim3(256), gemm_q4k_lds(), ctx->stream, a);
    } else {
        // wide tiles (64 token rows) for wide dense passes and experts averaging 32+ routes, else
        // narrow ones (16 token rows, 16 output rows per wave)
        const bool wide = a.grouped ? a.n_tok * a.k >= 32 * a.E : a.n_tok >= GEMM_MIN_ROWS;
        const int rpb = wide ? (dual ? 128 : 256) : 64;
        const dim3 grid((m0.rows + rpb - 1) / rpb, gemm_slots(a.grouped, a.n_tok, a.k, a.E, wide ? 64 : 16));
        const size_t lds = gemm_f16_lds(wide ? 4 : 1);
        if (wide) {
            if (dual) KL((k_gemm_f16<true, 4, 4>), grid, dim3(256), lds, ctx->stream, a);
            else KL((k_gemm_f16<false, 4, 4>), grid, dim3(256), lds, ctx->stream, a);
        } else {
            if (dual) KL((k_gemm_f16<true, 2, 1>), grid, dim3(256), lds, ctx->stream, a);
            else KL((k_gemm_f16<false, 1, 1>), grid, dim3(256), lds, ctx->stream, a);
        }
    }
    HIPX(hipGetLastError());
    return Z2H_OK;
}

// A down matmul whose fp32 input rows k_gemv_split encodes itself (no k_encode_rows launch): Q8_0
// weights in the m16 layout, one K-split block per 16-row group, at most XF_ITEMS float4 of rows per
// thread (one or two rows of the model's FFN width), grouped launches within the K-split's route limit.
bool xf_split_ok(const z2h_ctx * ctx, const DevMat & m, int rows, bool grouped) {
    return m.m16 && m.type == Z2H_Q8_0 && m.nsb <= 4 * SPLIT_UMAX && rows >= 1 &&
           (int64_t) rows * (m.nsb * 256 / 4) <= 256 * XF_ITEMS && (!grouped || (int64_t) rows * m.tiles <= 2 * ctx->n_cu);
}

int launch_gemv(z2h_ctx * ctx, const DevMat & m0, const DevMat * m1, const GemvArgs & base, int grid_y, int fam) {
    if (use_gemm(m0, base.n_tok) && (!m1 || gemm_dual_ok(m0, *m1)) && (!base.grouped || (base.r_off && base.r_perm)))
        return launch_gemm(ctx, m0, m1, base, fam);
    prof_scope ps(ctx, fam);
    GemvArgs a = base;
    a.w[0] = m0.w; a.w[1] = m1 ? m1->w : m0.w;
    a.dpl[0] = m0.dpl; a.dpl[1] = m1 ? m1->dpl : m0.dpl;
    a.mat_bytes = m0.mat_bytes; a.dpl_elems = m0.dpl_elems;
    a.nsb = m0.nsb; a.tiles = m0.tiles; a.rows = m0.rows;
    if (!a.grouped) {
        // spread the tokens over enough blocks to cover the chip (weights are re-read from L2/MALL)
        const int want = std::min(a.n_tok, std::max(1, (256 + m0.tiles - 1) / m0.tiles));
        const int chunks = std::max(want, (a.n_tok + NT - 1) / NT);
        a.tpb = (a.n_tok + chunks - 1) / chunks;
        grid_y = (a.n_tok + a.tpb - 1) / a.tpb;
    }
    const int af = act_of(m0.type);
    a.n_mats = m1 ? 2 : 1;
    if (m0.m16) {
        // grouped: ROWS = MT_G routes per pass (an expert serves at most n_tok routes); dense: all
        // MT tokens of a chunk per pass, so each weight tile is read once
        // grouped: 8-route passes for small batches (an expert serves ~2 routes at 16 requests), 16-route
        // passes from 128 routes (popular experts re-read their weights per pass; Q6_K keeps 8-route
        // passes there, its second product set costing more than the re-reads) and for the sorted
        // table; dense: 16-token passes
        // one pass of 16 routes covers every expert of a batch of at most 16 tokens (a token routes to an
        // expert once): those launches request each wave's first weight unit at entry (EARLY)
        const bool early = a.grouped && !a.r_perm && a.n_tok <= MT && m0.type == Z2H_Q4_K;
        const int rows = early ? MT : a.grouped && !a.r_perm && (a.n_tok * a.k < 128 || m0.type == Z2H_Q6_K) ? MT_G : MT;
        const size_t lds = gemv_mfma_lds_bytes(m0.type, m0.nsb * 256, rows);
        const int passes = a.grouped ? (a.n_tok + rows - 1) / rows : 1;
        if (!a.grouped) grid_y = (a.n_tok + rows - 1) / rows;
        const bool dual = a.mode == MM_SWIGLU;
        if (dual && (!m1 || m1->type != m0.type || m1->nsb != m0.nsb || m1->tiles != m0.tiles)) return seterr(ctx, Z2H_EINVAL, "gate/up layouts differ");
        // grouped launches whose routes, one block per (16-row group, route), stay within two blocks
        // per compute unit (one or two requests) take the K split too: a touched expert's weights
        // are then requested by four times as many waves as the row-group quads give it, each wave
        // with all of its units in flight
        const bool split_fits = (dual ? 2 : 1) * m0.nsb <= 4 * SPLIT_UMAX && (dual || a.n_mats == 1 || !a.grouped);
        const bool gsplit = a.grouped && (int64_t) a.n_tok * a.k * m0.tiles <= 2 * ctx->n_cu;
        if (a.xf) {
            // fp32 activation rows encoded in the staging (down matmuls of one or two tokens / routes)
            if (!xf_split_ok(ctx, m0, a.grouped ? a.n_tok * a.k : a.n_tok, a.grouped) || dual)
                return seterr(ctx, Z2H_EINVAL, "fp32-staged matmul outside its shapes");
            const size_t slds = gemv_mfma_lds_bytes(m0.type, m0.nsb * 256, MT_G);
            const int chunks = (a.n_tok + MT_G - 1) / MT_G;
            dim3 grid(m0.tiles, a.grouped ? grid_y : chunks, a.grouped ? chunks : 1), block(256);
            if (a.n_tok <= 2) KL((k_gemv_split<WF_Q8_0, false, MT_G, true, true>), grid, block, slds, ctx->stream, a);
            else KL((k_gemv_split<WF_Q8_0, false, MT_G, true>), grid, block, slds, ctx->stream, a);
            HIPX(hipGetLastError());
            return Z2H_OK;
        }
        if (split_fits && (!a.grouped || gsplit)) {
            // K split over the 4 waves of a block, one 16-row group per block; chunks of 8 tokens
            // where that still gives at most two blocks per compute unit (a weight tile is then read
            // by two blocks, which halves each block's staging and products). Grouped: grid (groups,
            // experts, passes of 8 routes)
            const bool half = a.grouped || (int64_t) m0.tiles * ((a.n_tok + MT_G - 1) / MT_G) <= 2 * ctx->n_cu;
            const int srows = half ? MT_G : MT;
            const size_t slds = gemv_mfma_lds_bytes(m0.type, m0.nsb * 256, srows);
            const int chunks = (a.n_tok + srows - 1) / srows;
            dim3 grid(m0.tiles, a.grouped ? grid_y : chunks, a.grouped ? chunks : dual ? 1 : a.n_mats), block(256);
            // at most two tokens (so at most two rows per block): Q8_0 takes the token-pair units
            const bool tp = a.n_tok <= 2;
#define SPL(W_, D_, R_) do { if (tp && W_ == WF_Q8_0) KL((k_gemv_split<W_, D_, R_, false, W_ == WF_Q8_0>), grid, block, slds, ctx->stream, a); \
                             else KL((k_gemv_split<W_, D_, R_>), grid, block, slds, ctx->stream, a); } while (0)
#define SPL_R(W_, D_) do { if (half) SPL(W_, D_, MT_G); else SPL(W_, D_, MT); } while (0)
            if (m0.type == Z2H_Q4_K) { if (dual) SPL_R(WF_Q4_K, true); else SPL_R(WF_Q4_K, false); }
            else if (m0.type == Z2H_Q6_K) { if (dual) SPL_R(WF_Q6_K, true); else SPL_R(WF_Q6_K, false); }
            else { if (dual) SPL_R(WF_Q8_0, true); else SPL_R(WF_Q8_0, false); }
#undef SPL_R
#undef SPL
            HIPX(hipGetLastError());
            return Z2H_OK;
        }
        dim3 grid((m0.tiles + 3) / 4, grid_y, (dual ? 1 : a.n_mats) * passes), block(256);
#define MM16(W_, D_, R_) KL((k_gemv_mfma<W_, D_, R_, R_ == MT_G ? m16fmt<W_>::GPF : 1>), grid, block, lds, ctx->stream, a)
        if (early) {
            if (dual) KL((k_gemv_mfma<WF_Q4_K, true, MT, 1, true>), grid, block, lds, ctx->stream, a);
            else KL((k_gemv_mfma<WF_Q4_K, false, MT, 1, true>), grid, block, lds, ctx->stream, a);
        } else if (m0.type == Z2H_Q4_K) {
            if (rows == MT_G) { if (dual) MM16(WF_Q4_K, true, MT_G); else MM16(WF_Q4_K, false, MT_G); }
            else { if (dual) MM16(WF_Q4_K, true, MT); else MM16(WF_Q4_K, false, MT); }
        } else if (m0.type == Z2H_Q6_K) {
            if (rows == MT_G) { if (dual) MM16(WF_Q6_K, true, MT_G); else MM16(WF_Q6_K, false, MT_G); }
            else { if (dual) MM16(WF_Q6_K, true, MT); else MM16(WF_Q6_K, false, MT); }
        } else {
            if (rows == MT_G) { if (dual) MM16(WF_Q8_0, true, MT_G); else MM16(WF_Q8_0, false, MT_G); }
            else { if (dual) MM16(WF_Q8_0, true, MT); else MM16(WF_Q8_0, false, MT); }
        }
#undef MM16
        HIPX(hipGetLastError());
        return Z2H_OK;
    }
    if (a.grouped) {
        // grouped expert matmuls: row-streaming kernel, 4 tiles per block, NTE routes per block
        const size_t lds = gemv_rows_lds_bytes(af, m0.nsb * 256);
        dim3 grid((m0.tiles + 3) / 4, grid_y, (m1 ? 2 : 1) * ((a.n_tok + NTE - 1) / NTE)), block(256);
        switch (m0.type) {
            case Z2H_Q4_K: KL(k_gemv_rows<WF_Q4_K>, grid, block, lds, ctx->stream, a); break;
            case Z2H_Q6_K: KL(k_gemv_rows<WF_Q6_K>, grid, block, lds, ctx->stream, a); break;
            case Z2H_Q8_0: KL(k_gemv_rows<WF_Q8_0>, grid, block, lds, ctx->stream, a); break;
            case Z2H_F16:  KL(k_gemv_rows<WF_F16>, grid, block, lds, ctx->stream, a); break;
            default: return seterr(ctx, Z2H_ENOTSUP, "gemv type");
        }
        HIPX(hipGetLastError());
        return Z2H_OK;
    }
    const size_t lds = gemv_lds_bytes(af, m0.nsb * 256);
    dim3 grid(m0.tiles, grid_y, m1 ? 2 : 1), block(256);
    switch (m0.type) {
        case Z2H_Q4_K: KL(k_gemv<WF_Q4_K>, grid, block, lds, ctx->stream, a); break;
        case Z2H_Q6_K: KL(k_gemv<WF_Q6_K>, grid, block, lds, ctx->stream, a); break;
        case Z2H_Q8_0: KL(k_gemv<WF_Q8_0>, grid, block, lds, ctx->stream, a); break;
        case Z2H_F16:  KL(k_gemv<WF_F16>, grid, block, lds, ctx->stream, a); break;
        default: return seterr(ctx, Z2H_ENOTSUP, "gemv type");
    }
    HIPX(hipGetLastError());
    return Z2H_OK;
}

// SwiGLU fused into the gate/up matmul: both in the 16-row MFMA layout with the same shape, or a
// pass of T rows that takes the GEMMs
bool fused_ffn(const DevMat & g, const DevMat & u, int T) {
    return (g.m16 && u.m16 && g.type == u.type && g.nsb == u.nsb && g.tiles == u.tiles) ||
           (use_gemm(g, T) && gemm_dual_ok(g, u));
}

int launch_encode(z2h_ctx * ctx, const float * x, int ld, int K, int n_rows, int act_fmt, const ActBuf & act) {
    prof_scope ps(ctx, Z2H_KF_SWIGLU);
    EncodeArgs e{x, ld, K, n_rows, act_fmt, act};
    const int items = n_rows * (kpad(K) / 256);
    KL(k_encode_rows, dim3((items + 3) / 4), dim3(256), 0, ctx->stream, e);
    HIPX(hipGetLastError());
    return Z2H_OK;
}

int launch_swiglu(z2h_ctx * ctx, int n_rows, int act_fmt) {
    prof_scope ps(ctx, Z2H_KF_SWIGLU);
    SwigluArgs w{};
    w.g = ctx->gu_g; w.u = ctx->gu_u; w.ff = ctx->hp.n_ff; w.act = ctx->act_y; w.act_fmt = act_fmt;
    KL(k_swiglu_encode, dim3(n_rows), dim3(256), (size_t) kpad(ctx->hp.n_ff) * 4, ctx->stream, w);
    HIPX(hipGetLastError());
    return Z2H_OK;
}

GemvArgs gemv_dense(z2h_ctx * ctx, int T, float * out, int out_ld, int epi) {
    GemvArgs a{};
    a.grouped = 0; a.n_tok = T; a.act = ctx->act;
    a.out[0] = out; a.out[1] = out; a.out_ld = out_ld; a.epi = epi; a.cap = ctx->hp.logit_softcap;
    return a;
}

int launch_resnorm(z2h_ctx * ctx, int T, ResNormArgs a) {
    prof_scope ps(ctx, Z2H_KF_RESNORM);
    if (!a.d) a.d = ctx->hp.n_embd;
    a.eps = ctx->hp.rms_eps; a.err = ctx->d_err;
    const size_t lds = (size_t) kpad(a.d) * 4;
    switch (a.mode) {
        case RN_EMBED: {
            // token ids over tables of one type (F32, F16, Q8_0): the switch-free gather
            int tt = a.W > 0 ? a.tab_type[0] : -1;
            for (int k = 1; k < a.W; ++k) if (a.tab_type[k] != tt) tt = -1;
            // (10 table slots cover the 9 codebooks + text of Zonos2 models with 10/16 of the loads)
            const bool w10 = a.W <= 10;
#define RNE(T_) do { if (w10) KL((k_resnorm<RN_EMBED, T_, 10>), dim3(T), dim3(256), lds, ctx->stream, a); \
                     else KL((k_resnorm<RN_EMBED, T_, MAX_TABLES>), dim3(T), dim3(256), lds, ctx->stream, a); } while (0)
            if (tt == 8) RNE(8);
            else if (tt == 1) RNE(1);
            else if (tt == 0) RNE(0);
            else KL(k_resnorm<RN_EMBED>, dim3(T), dim3(256), lds, ctx->stream, a);
#undef RNE
            break;
        }
        case RN_ACCUM: KL(k_resnorm<RN_ACCUM>, dim3(T), dim3(256), lds, ctx->stream, a); break;
        case RN_ADD: KL(k_resnorm<RN_ADD>, dim3(T), dim3(256), lds, ctx->stream, a); break;
        default: KL(k_resnorm<RN_ENCODE>, dim3(T), dim3(256), lds, ctx->stream, a); break;
    }
    HIPX(hipGetLastError());
    return Z2H_OK;
}

RouterArgs router_args(z2h_ctx * ctx, const Layer & ly, int L, int T, const float * state_in) {
    const auto & hp = ctx->hp;
    RouterArgs r{};
    r.x = ctx->cur; r.T = T; r.d = hp.n_embd; r.rd = ctx->rd; r.E = ly.E; r.k = ly.k;
    r.w_down = ly.r_down; r.b_down = ly.r_down_b; r.eda = ly.r_eda; r.state_in = state_in;
    r.rh = ctx->state_one ? ctx->state_one : ctx->state + (size_t) L * ctx->Tmax * ctx->rd;
    r.norm_w = ly.r_norm; r.eps = hp.rms_eps;
    r.w0t = ly.r_m0t; r.b0 = ly.r_m0_b; r.w2t = ly.r_m2t; r.b2 = ly.r_m2_b; r.w4t = ly.r_m4t;
    r.logit_bias = ly.logit_bias; r.mask = ly.mask; r.sc_bias = ly.r_bias;
    r.sel = ctx->sel; r.wsel = ctx->wsel;
    r.cap_logits = (float *) capp(ctx, Z2H_CAP_ROUTER_LOGITS, L);
    r.cap_probs = (float *) capp(ctx, Z2H_CAP_PROBS, L);
    return r;
}

// router-down elements per lane: the next power of two >= ceil(d / 64); unguarded when d fills every lane
int router_ni(int d) { return d <= 64 ? 1 : 1 << (32 - __builtin_clz((unsigned) ((d + 63) / 64 - 1))); }

// An MoE layer's FFN entry as one launch (k_ffn_entry): res_out = res_in + src, x = ffn_norm(res_out)
// into ctx->cur and the expert activations, router-down state of layer L.
int launch_ffn_entry(z2h_ctx * ctx, const Layer & ly, int L, int T, const float * state_in,
                     const float * src, const float * res_in, float * res_out) {
    prof_scope ps(ctx, Z2H_KF_ROUTER_DOWN);
    const auto & hp = ctx->hp;
    const RouterArgs r = router_args(ctx, ly, L, T, state_in);
    ResNormArgs f{};
    f.mode = RN_ADD; f.d = hp.n_embd; f.src = src; f.res_in = res_in; f.res = res_out; f.norm_w = ly.ffn_norm;
    f.eps = hp.rms_eps; f.cur_out = ctx->cur; f.act = ctx->act; f.act_fmt = act_of(ly.up_exps.type); f.err = ctx->d_err;
    const int ni = router_ni(hp.n_embd);
    const bool exact = hp.n_embd == 64 * ni;
    if (T >= GEMM_MIN_ROWS && ni % 4 == 0 && ctx->rd % 32 == 0) {
        // wide passes: the norm once per token (k_resnorm, the same arithmetic), then the router down
        // projection with each weight row reused across RD_T tokens
        f.res = res_out; f.res_in = res_in;
        if (int rc = launch_resnorm(ctx, T, f)) return rc;
        const dim3 g2(ctx->rd / 32, (T + RD_T - 1) / RD_T);
        const size_t l2 = router_down_t_lds(ni);
#define RDT(N_) do { if (exact) KL((k_router_down_t<N_, false>), g2, dim3(256), l2, ctx->stream, r); \
                     else KL((k_router_down_t<N_, true>), g2, dim3(256), l2, ctx->stream, r); } while (0)
        switch (ni) {
            case 4: RDT(4); break;
            case 8: RDT(8); break;
            case 16: RDT(16); break;
            case 32: RDT(32); break;
            default: RDT(64); break;
        }
#undef RDT
        HIPX(hipGetLastError());
        return Z2H_OK;
    }
    const dim3 grid((ctx->rd + 3) / 4, T);
    const size_t lds = (size_t) kpad(hp.n_embd) * 4;
#define FEN(N_) do { if (exact) KL((k_ffn_entry<N_, false>), grid, dim3(256), lds, ctx->stream, f, r); \
                     else KL((k_ffn_entry<N_, true>), grid, dim3(256), lds, ctx->stream, f, r); } while (0)
    switch (ni) {
        case 1: FEN(1); break;
        case 2: FEN(2); break;
        case 4: FEN(4); break;
        case 8: FEN(8); break;
        case 16: FEN(16); break;
        case 32: FEN(32); break;
        default: FEN(64); break;
    }
#undef FEN
    HIPX(hipGetLastError());
    return Z2H_OK;
}

// down_done: the router-down state of layer L is already in place (k_ffn_entry)
int expert_block(z2h_ctx * ctx, Layer & ly, int L, int T, const float * state_in, bool down_done = false) {
    const auto & hp = ctx->hp;
    int rc;
    // router (exact contract)
    const RouterArgs r = router_args(ctx, ly, L, T, state_in);
    if (!down_done) {
        prof_scope ps(ctx, Z2H_KF_ROUTER_DOWN);
        const dim3 grid((ctx->rd + 3) / 4, T);
        const int ni = router_ni(hp.n_embd);
        const bool exact = hp.n_embd == 64 * ni;
#define RDN(N_) do { if (exact) KL((k_router_down<N_, false>), grid, dim3(256), 0, ctx->stream, r); \
                     else KL((k_router_down<N_, true>), grid, dim3(256), 0, ctx->stream, r); } while (0)
        switch (ni) {
            case 1: RDN(1); break;
            case 2: RDN(2); break;
            case 4: RDN(4); break;
            case 8: RDN(8); break;
            case 16: RDN(16); break;
            case 32: RDN(32); break;
            default: RDN(64); break;
        }
#undef RDN
        HIPX(hipGetLastError());
    }
    {
        prof_scope ps(ctx, Z2H_KF_ROUTER_TAIL);
        // wide passes: up to one block per compute unit, each looping over its tokens with the MLP
        // matrices loaded once
        if (T >= GEMM_MIN_ROWS) KL(k_router_tail<true>, dim3(std::min((T + RT_NTOK - 1) / RT_NTOK, ctx->n_cu)), dim3(RT_THREADS), router_tail_wide_lds(ctx->rd, ly.E), ctx->stream, r);
        else KL(k_router_tail<false>, dim3(T), dim3(RT_THREADS), router_tail_lds(ctx->rd, ly.E), ctx->stream, r);
        HIPX(hipGetLastError());
    }
    // routes grouped by expert (mul_mat_id's grouping): the grouped matmul blocks list up to LIST_MAX
    // routes in LDS themselves; larger batches, and captures, take one sort kernel's table
    const bool sorted = ctx->capture || T * ly.k > LIST_MAX || use_gemm(ly.gate_exps, T) || use_gemm(ly.down_exps, T);
    if (sorted) {
        prof_scope ps(ctx, Z2H_KF_ROUTER_TAIL);
        int32_t * cc = ctx->capture ? (int32_t *) capp(ctx, Z2H_CAP_COUNTS, L) : nullptr;
        int32_t * co = ctx->capture ? (int32_t *) capp(ctx, Z2H_CAP_OFFSETS, L) : nullptr;
        int32_t * cp = ctx->capture ? (int32_t *) capp(ctx, Z2H_CAP_PERM, L) : nullptr;
        KL(k_route_sort, dim3(1), dim3(1024), 0, ctx->stream, (const int32_t *) ctx->sel, T * ly.k, ly.E, ctx->r_off, ctx->r_perm, cc, co, cp);
        HIPX(hipGetLastError());
    }
    if ((rc = cap_copy(ctx, Z2H_CAP_ROUTER_STATE, L, r.rh, T))) return rc;
    if ((rc = cap_copy(ctx, Z2H_CAP_SEL, L, ctx->sel, T))) return rc;
    if ((rc = cap_copy(ctx, Z2H_CAP_WEIGHTS, L, ctx->wsel, T))) return rc;
    if (fused_ffn(ly.gate_exps, ly.up_exps, T)) {
        // gate + up + SwiGLU in one grouped launch -> y [route][ff] fp32, encoded once for down
        GemvArgs g{};
        g.grouped = 1; g.n_tok = T; g.sel = ctx->sel; g.k = ly.k; g.act = ctx->act; g.E = ly.E; g.mode = MM_SWIGLU;
        g.out[0] = ctx->gu_g; g.out[1] = ctx->gu_g; g.out_ld = hp.n_ff; g.epi = EPI_STORE;
        g.r_off = sorted ? ctx->r_off : nullptr; g.r_perm = sorted ? ctx->r_perm : nullptr;
        if ((rc = launch_gemv(ctx, ly.gate_exps, &ly.up_exps, g, ly.E, Z2H_KF_GEMV_GATEUP))) return rc;
        // one or two routes over Q8_0 experts: the down matmul encodes the fp32 rows itself
        const bool xf = !sorted && xf_split_ok(ctx, ly.down_exps, T * ly.k, true);
        if (!xf && (rc = launch_encode(ctx, ctx->gu_g, hp.n_ff, hp.n_ff, T * ly.k, act_of(ly.down_exps.type), ctx->act_y))) return rc;
        GemvArgs dn{};
        dn.grouped = 1; dn.n_tok = T; dn.sel = ctx->sel; dn.k = ly.k; dn.E = ly.E;
        dn.act = ctx->act_y; dn.act_by_route = 1;
        if (xf) { dn.xf = ctx->gu_g; dn.xf_ld = hp.n_ff; }

        dn.out[0] = ctx->eo; dn.out[1] = ctx->eo; dn.out_ld = hp.n_embd; dn.epi = EPI_ROUTE_W; dn.route_w = ctx->wsel;
        dn.r_off = sorted ? ctx->r_off : nullptr; dn.r_perm = sorted ? ctx->r_perm : nullptr;
        if ((rc = launch_gemv(ctx, ly.down_exps, nullptr, dn, ly.E, Z2H_KF_GEMV_DOWN))) return rc;
        return cap_copy(ctx, Z2H_CAP_EXPERT_OUT, L, ctx->eo, T);
    }
    // gate + up (grouped by expert)
    GemvArgs g{};
    g.grouped = 1; g.n_tok = T; g.sel = ctx->sel; g.k = ly.k; g.act = ctx->act; g.E = ly.E;
    g.out[0] = ctx->gu_g; g.out[1] = ctx->gu_u; g.out_ld = hp.n_ff; g.epi = EPI_STORE;
    g.r_off = sorted ? ctx->r_off : nullptr; g.r_perm = sorted ? ctx->r_perm : nullptr;
    if ((rc = launch_gemv(ctx, ly.gate_exps, &ly.up_exps, g, ly.E, Z2H_KF_GEMV_GATEUP))) return rc;
    // y = up * silu(gate) per route, encoded once for the down matmul
    if ((rc = launch_swiglu(ctx, T * ly.k, act_of(ly.down_exps.type)))) return rc;
    // down, route weight
    GemvArgs dn{};
    dn.grouped = 1; dn.n_tok = T; dn.sel = ctx->sel; dn.k = ly.k; dn.E = ly.E;
    dn.act = ctx->act_y; dn.act_by_route = 1;
    dn.out[0] = ctx->eo; dn.out[1] = ctx->eo; dn.out_ld = hp.n_embd; dn.epi = EPI_ROUTE_W; dn.route_w = ctx->wsel;
    dn.r_off = sorted ? ctx->r_off : nullptr; dn.r_perm = sorted ? ctx->r_perm : nullptr;
    if ((rc = launch_gemv(ctx, ly.down_exps, nullptr, dn, ly.E, Z2H_KF_GEMV_DOWN))) return rc;
    if ((rc = cap_copy(ctx, Z2H_CAP_EXPERT_OUT, L, ctx->eo, T))) return rc;
    return Z2H_OK;
}

int dense_block(z2h_ctx * ctx, Layer & ly, int T) {
    const auto & hp = ctx->hp;
    int rc;
    if (fused_ffn(ly.ffn_gate, ly.ffn_up, T)) {
        GemvArgs g = gemv_dense(ctx, T, ctx->gu_g, hp.n_ff, EPI_STORE);
        g.mode = MM_SWIGLU;
        if ((rc = launch_gemv(ctx, ly.ffn_gate, &ly.ffn_up, g, 1, Z2H_KF_GEMV_DENSE))) return rc;
        const bool xf = xf_split_ok(ctx, ly.ffn_down, T, false) && !use_gemm(ly.ffn_down, T);
        if (!xf && (rc = launch_encode(ctx, ctx->gu_g, hp.n_ff, hp.n_ff, T, act_of(ly.ffn_down.type), ctx->act_y))) return rc;
        GemvArgs dn = gemv_dense(ctx, T, ctx->eo, hp.n_embd, EPI_STORE);
        dn.act = ctx->act_y;
        if (xf) { dn.xf = ctx->gu_g; dn.xf_ld = hp.n_ff; }
        return launch_gemv(ctx, ly.ffn_down, nullptr, dn, 1, Z2H_KF_GEMV_DENSE);
    }
    GemvArgs g = gemv_dense(ctx, T, ctx->gu_g, hp.n_ff, EPI_STORE);
    g.out[0] = ctx->gu_g; g.out[1] = ctx->gu_u;
    if ((rc = launch_gemv(ctx, ly.ffn_gate, &ly.ffn_up, g, 1, Z2H_KF_GEMV_DENSE))) return rc;
    if ((rc = launch_swiglu(ctx, T, act_of(ly.ffn_down.type)))) return rc;
    GemvArgs dn = gemv_dense(ctx, T, ctx->eo, hp.n_embd, EPI_STORE);
    dn.act = ctx->act_y;
    return launch_gemv(ctx, ly.ffn_down, nullptr, dn, 1, Z2H_KF_GEMV_DENSE);
}

// The whole decode step on device-resident inputs in ctx->d_* (T tokens, host copy of n_past).
// kv_pre: append every token's K/V row before the attention (prefill chunks and mixed batches, whose
// rows of one slot attend to each other); d_emb_map: per token -1 (sum of its ids) or its row of d_emb.
// f32_prompt (per-slot prefill): the rows also keep their fp32 K/V in ctx->pf_kv and attend over those
// (the reference's in-prompt attention, src/zonos2-graph.cpp:155-169) instead of the f16 cache rows.
// head_rows: which rows get logits (rows [0, n_head) of d_logits): every row, none, the last row, or
// the n_head rows listed in d_head_rows.
enum { HEAD_ALL = 0, HEAD_NONE = 1, HEAD_LAST = 2, HEAD_ROWS = 3 };
int run_step(z2h_ctx * ctx, int T, const int32_t * h_npast, const int32_t * d_slot, const int32_t * d_npast,
             const int32_t * d_ids, const float * d_emb, float * d_logits, bool kv_pre = false,
             const int32_t * d_emb_map = nullptr, const int32_t * h_slot = nullptr, bool f32_prompt = false,
             int head_rows = HEAD_ALL, const int32_t * d_head_rows = nullptr, int n_head = 0) {
    const auto & hp = ctx->hp;
    const int d = hp.n_embd, nh = hp.n_head, nkv = hp.n_head_kv, hd = hp.head_dim;
    int rc;
    ctx->cap_T = T;
    // the blocks that run (depth prune: a skipped block passes the residual through unchanged)
    std::vector<int> run;
    for (int L = 0; L < hp.n_layer; ++L)
        if (L >= (int) ctx->m->layer_skip.size() || !ctx->m->layer_skip[L]) run.push_back(L);
    const int n_run = (int) run.size();
    // embeddings + emb_norm + the first block's attn_norm (output_norm when every block is skipped)
    ResNormArgs e{};
    e.mode = RN_EMBED; e.ids = d_ids; e.W = ctx->W; e.emb_in = d_emb; e.emb_map = d_emb_map;
    for (int k = 0; k < ctx->W; ++k) { e.tab[k] = ctx->m->tab[k]; e.tab_type[k] = ctx->m->tab_type[k]; e.tab_rows[k] = ctx->m->tab_rows[k]; }
    e.res = ctx->res;
    if (n_run) {
        e.norm_w = ctx->m->layers[run[0]].attn_norm; e.cur_out = (float *) capp(ctx, Z2H_CAP_ATTN_IN, run[0]);
        e.act_fmt = act_of(ctx->m->layers[run[0]].qkvg.type);
    } else {
        e.norm_w = ctx->m->output_norm; e.cur_out = (float *) capp(ctx, Z2H_CAP_OUT_NORM, 0);
        e.act_fmt = act_of(ctx->m->head.type);
    }
    e.act = ctx->act;
    if ((rc = launch_resnorm(ctx, T, e))) return rc;
    if (n_run && (rc = cap_copy(ctx, Z2H_CAP_RES_IN, run[0], ctx->res, T))) return rc;
    (void) h_npast;
    // decode steps: a persistent attention grid (the item count comes from the device n_past table),
    // as many blocks as fit on the chip at once; blocks loop over the items beyond it
    const int grp = nh / nkv;
    const int attn_grid = std::min(ctx->items_max, ctx->attn_slots);
    // wide passes (host copies of the rows' slots and positions at hand): work items (tile, KV head,
    // segment), a tile being up to FA_ROWS rows of one slot at consecutive positions (k_attn_fa)
    int n_fa = 0;
    // head_dim 128 and at most 4 query heads per KV head: one block per (tile, KV head) walks the whole
    // band with an online softmax (k_attn_flash16: no partials, no merge pass)
    const bool flash16 = kv_pre && !f32_prompt && hd == 128 && grp <= 4;
    if (flash16 && h_slot && h_npast) {
        for (int t = 0; t < T;) {
            int m = 1;
            while (t + m < T && m < FA_ROWS && h_slot[t + m] == h_slot[t] && h_npast[t + m] == h_npast[t] + m) ++m;
            for (int g = 0; g < nkv; ++g) {
                if (n_fa >= ctx->items_max) return seterr(ctx, Z2H_EINVAL, "attention tile table overflow");
                ctx->h_tiles[n_fa++] = make_int4(t, m | (g << 16), 0, 0);
            }
            t += m;
        }
        // longest bands first: blocks start in grid order, so a grid larger than the chip's resident
        // blocks ends with short tiles instead of a late long one (each tile's arithmetic is its own)
        std::stable_sort(ctx->h_tiles, ctx->h_tiles + n_fa, [&](const int4 & x, const int4 & y) {
            return h_npast[x.x] + (x.y & 0xffff) > h_npast[y.x] + (y.y & 0xffff);
        });
        HIPX(hipMemcpyAsync(ctx->d_tiles, ctx->h_tiles, (size_t) n_fa * sizeof(int4), hipMemcpyHostToDevice, ctx->stream));
    } else if (kv_pre && !f32_prompt && h_slot && h_npast) {
        const int rows_max = std::max(1, std::min(FA_ROWS, 64 / grp));
        int segs = 0;
        for (int t = 0; t < T;) {
            int m = 1;
            while (t + m < T && m < rows_max && h_slot[t + m] == h_slot[t] && h_npast[t + m] == h_npast[t] + m) ++m;
            const int ns = fa_nseg(h_npast[t] + m - 1);
            for (int s = 0; s < ns; ++s)
                for (int g = 0; g < nkv; ++g) {
                    if (n_fa >= ctx->items_max) return seterr(ctx, Z2H_EINVAL, "attention tile table overflow");
                    ctx->h_tiles[2 * n_fa] = make_int4(t, m | (g << 16), s, segs);
                    ctx->h_tiles[2 * n_fa + 1] = make_int4(h_npast[t], h_slot[t], 0, 0);
                    ++n_fa;
                }
            for (int j = 0; j < m; ++j) segs += fa_nseg(h_npast[t + j]);
            t += m;
        }
        HIPX(hipMemcpyAsync(ctx->d_tiles, ctx->h_tiles, (size_t) 2 * n_fa * sizeof(int4), hipMemcpyHostToDevice, ctx->stream));
    }
    // per-slot prefill (f32_prompt): tiles of up to ATT_TILE rows of one slot at consecutive positions
    // share each 64-row chunk of the prompt's fp32 K/V (k_attn_tile_f32, then k_attn_combine)
    int n_tiles = 0;
    // head_dim 128 and at most 4 query heads per KV head: one block per (tile, KV head) walks the whole
    // band with an online softmax (k_attn_flash32: no partials, no merge pass)
    const bool flash32 = kv_pre && f32_prompt && hd == 128 && nh / nkv <= 4;
    if (flash32 && h_slot && h_npast) {
        for (int t = 0; t < T;) {
            int m = 1;
            while (t + m < T && m < ATT_TILE && h_slot[t + m] == h_slot[t] && h_npast[t + m] == h_npast[t] + m) ++m;
            for (int g = 0; g < nkv; ++g) {
                if (n_tiles >= ctx->items_max) return seterr(ctx, Z2H_EINVAL, "attention tile table overflow");
                ctx->h_tiles[n_tiles++] = make_int4(t, m | (g << 16), 0, 0);
            }
            t += m;
        }
        std::stable_sort(ctx->h_tiles, ctx->h_tiles + n_tiles, [&](const int4 & x, const int4 & y) {   // longest bands first
            return h_npast[x.x] + (x.y & 0xffff) > h_npast[y.x] + (y.y & 0xffff);
        });
        HIPX(hipMemcpyAsync(ctx->d_tiles, ctx->h_tiles, (size_t) n_tiles * sizeof(int4), hipMemcpyHostToDevice, ctx->stream));
    } else if (kv_pre && f32_prompt && h_slot && h_npast) {
        int before = 0;
        for (int t = 0; t < T;) {
            int m = 1;
            while (t + m < T && m < ATT_TILE && h_slot[t + m] == h_slot[t] && h_npast[t + m] == h_npast[t] + m) ++m;
            const int nc_last = (h_npast[t + m - 1] + ATT_CH) / ATT_CH;
            for (int c = 0; c < nc_last; ++c)
                for (int g = 0; g < nkv; ++g) {
                    if (n_tiles >= ctx->items_max) return seterr(ctx, Z2H_EINVAL, "attention tile table overflow");
                    ctx->h_tiles[n_tiles++] = make_int4(t, m | (g << 16), c, before);
                }
            for (int j = 0; j < m; ++j) before += (h_npast[t + j] + ATT_CH) / ATT_CH;
            t += m;
        }
        HIPX(hipMemcpyAsync(ctx->d_tiles, ctx->h_tiles, (size_t) n_tiles * sizeof(int4), hipMemcpyHostToDevice, ctx->stream));
    }
    const int R = (nh + 2 * nkv) * hd + nh;
    int prev_moe = -1;
    for (int i = 0; i < n_run; ++i) {
        const int L = run[i];
        Layer & ly = ctx->m->layers[L];
        // fused QKV + gate projection
        if ((rc = launch_gemv(ctx, ly.qkvg, nullptr, gemv_dense(ctx, T, ctx->qkvg, R, EPI_STORE), 1, Z2H_KF_GEMV_QKV))) return rc;
        AttnArgs a{};
        a.qkvg = ctx->qkvg; a.R = R; a.nh = nh; a.nkv = nkv; a.hd = hd; a.temp = ly.attn_temp;
        a.qk_eps = hp.qk_norm_eps; a.theta_scale = std::pow(hp.rope_freq_base, -2.0f / (float) hd); a.rope = ctx->rope;
        a.scale = 1.0f / std::sqrt((float) hd);
        a.slot_idx = d_slot; a.n_past = d_npast; a.T = T; a.S = ctx->S;
        const size_t lsz = (size_t) ctx->n_slots * nkv * ctx->S * hd;
        a.kc = ctx->kv + (size_t) (2 * L) * lsz; a.vc = ctx->kv + (size_t) (2 * L + 1) * lsz;
        a.cap_q = (float *) capp(ctx, Z2H_CAP_Q, L); a.cap_k = (float *) capp(ctx, Z2H_CAP_K, L); a.cap_v = (float *) capp(ctx, Z2H_CAP_V, L);
        a.cap_gate = (float *) capp(ctx, Z2H_CAP_GATE, L);
        a.part_o = ctx->part_o; a.part_ml = ctx->part_ml;
        a.o_out = ctx->attn_o;
        if (f32_prompt) {
            a.kf = ctx->pf_kv + (size_t) (2 * L) * nkv * ctx->S * hd;
            a.vf = a.kf + (size_t) nkv * ctx->S * hd;
            a.kf_split = flash32;                                    // k_attn_flash32 reads f16 hi / lo planes
        }
        a.act = ctx->act;
        const int wo_act = act_of(ly.wo.type);
        bool in_block;
        if (flash32) {
            in_block = (grp * hd) % 256 == 0;
            a.act_fmt = in_block ? wo_act : ACT_NONE;
            a.tiles = (const int4 *) ctx->d_tiles;
            prof_scope ps(ctx, Z2H_KF_ATTN);
            if ((rc = launch_kv_append(ctx, a, T))) return rc;
            const size_t lds = attn_flash32_lds();
            switch (grp) {
                case 1: KL(k_attn_flash32<1>, dim3(n_tiles), dim3(512), lds, ctx->stream, a); break;
                case 2: KL(k_attn_flash32<2>, dim3(n_tiles), dim3(512), lds, ctx->stream, a); break;
                default: KL(k_attn_flash32<4>, dim3(n_tiles), dim3(512), lds, ctx->stream, a); break;
            }
            HIPX(hipGetLastError());
        } else if (!kv_pre || f32_prompt) {
            // heads per combine block: the fewest (1, 2, 4 or 8, dividing the group) whose outputs
            // cover whole encoding blocks, so the block encodes its slice for W_o; else a separate
            // encode pass
            int hpb = 0;
            for (int h = 1; h <= 8 && !hpb; h *= 2)
                if (grp % h == 0 && (h * hd) % 256 == 0) hpb = h;
            in_block = hpb != 0;
            if (!hpb) hpb = 1;
            a.act_fmt = in_block ? wo_act : ACT_NONE;
            {
                // decode steps: QK-norm / RoPE / KV append fused in, items from the device n_past table;
                // per-slot prefill: the appended fp32 prompt rows
                prof_scope ps(ctx, Z2H_KF_ATTN);
                if (kv_pre) {
                    if ((rc = launch_kv_append(ctx, a, T))) return rc;
                    if ((rc = launch_attn_tile(ctx, a, n_tiles))) return rc;
                } else if ((rc = launch_attn(ctx, a, attn_grid))) return rc;
            }
            prof_scope ps(ctx, Z2H_KF_ATTN_COMBINE);
            const int nc_max = (ctx->S + ATT_CH - 1) / ATT_CH;
            if (hd == 128 && hpb == 2 && grp == 4)
                KL((k_attn_combine<128, 2, 4>), dim3(nh / hpb, T), dim3(512), attn_combine_lds(hpb, hd, nc_max), ctx->stream, a, hpb, nc_max);
            else
                KL(k_attn_combine<>, dim3(nh / hpb, T), dim3(512), attn_combine_lds(hpb, hd, nc_max), ctx->stream, a, hpb, nc_max);
            HIPX(hipGetLastError());
        } else {
            // wide passes: k_attn_fa / k_attn_merge finish (and encode) a KV group's heads of a row in
            // one block
            in_block = (grp * hd) % 256 == 0;
            a.act_fmt = in_block ? wo_act : ACT_NONE;
            prof_scope ps(ctx, Z2H_KF_ATTN);
            if ((rc = launch_kv_append(ctx, a, T))) return rc;
            a.tiles = (const int4 *) ctx->d_tiles;
            if (flash16 && n_fa > 0) {
                const size_t lds = attn_flash16_lds();
                switch (grp) {
                    case 1: KL(k_attn_flash16<1>, dim3(n_fa), dim3(512), lds, ctx->stream, a); break;
                    case 2: KL(k_attn_flash16<2>, dim3(n_fa), dim3(512), lds, ctx->stream, a); break;
                    default: KL(k_attn_flash16<4>, dim3(n_fa), dim3(512), lds, ctx->stream, a); break;
                }
                HIPX(hipGetLastError());
            } else if (n_fa > 0 && (rc = launch_attn_fa(ctx, a, n_fa))) return rc;
        }
        if (!in_block) {
            ResNormArgs en{};
            en.mode = RN_ENCODE; en.d = nh * hd; en.src = ctx->attn_o; en.act = ctx->act; en.act_fmt = wo_act;
            if ((rc = launch_resnorm(ctx, T, en))) return rc;
        }
        if ((rc = cap_copy(ctx, Z2H_CAP_ATTN_O, L, ctx->attn_o, T))) return rc;
        // W_o
        if ((rc = launch_gemv(ctx, ly.wo, nullptr, gemv_dense(ctx, T, ctx->wo_out, d, EPI_STORE), 1, Z2H_KF_GEMV_WO))) return rc;
        if ((rc = cap_copy(ctx, Z2H_CAP_ATTN_OUT, L, ctx->wo_out, T))) return rc;
        // res += attn; ffn_norm; encode for the FFN (MoE layers: with the router down projection, the
        // new residual in res2 until the FFN output folds it back into res)
        if (ly.moe) {
            const float * st = prev_moe >= 0 ? ctx->state + (size_t) prev_moe * ctx->Tmax * ctx->rd : nullptr;
            if ((rc = launch_ffn_entry(ctx, ly, L, T, st, ctx->wo_out, ctx->res, ctx->res2))) return rc;
            if ((rc = cap_copy(ctx, Z2H_CAP_FFN_IN, L, ctx->cur, T))) return rc;
            if ((rc = expert_block(ctx, ly, L, T, st, true))) return rc;
            prev_moe = L;
        } else {
            ResNormArgs f{};
            f.mode = RN_ADD; f.src = ctx->wo_out; f.res = ctx->res; f.norm_w = ly.ffn_norm; f.cur_out = ctx->cur;
            f.act = ctx->act; f.act_fmt = act_of(ly.ffn_up.type);
            if ((rc = launch_resnorm(ctx, T, f))) return rc;
            if ((rc = cap_copy(ctx, Z2H_CAP_FFN_IN, L, ctx->cur, T))) return rc;
            if ((rc = dense_block(ctx, ly, T))) return rc;
        }
        // fold the FFN output into the residual; next layer's attn_norm (or output_norm)
        ResNormArgs n{};
        n.mode = RN_ACCUM; n.src = ctx->eo; n.k = ly.moe ? ly.k : 1; n.res = ctx->res;
        n.res_in = ly.moe ? ctx->res2 : nullptr;
        n.cap_x = (float *) capp(ctx, Z2H_CAP_FFN_OUT, L);
        const bool last = i + 1 == n_run;
        const int nx = last ? -1 : run[i + 1];
        n.norm_w = last ? ctx->m->output_norm : ctx->m->layers[nx].attn_norm;
        n.cur_out = last ? (float *) capp(ctx, Z2H_CAP_OUT_NORM, 0) : (float *) capp(ctx, Z2H_CAP_ATTN_IN, nx);
        n.act = ctx->act; n.act_fmt = act_of(last ? ctx->m->head.type : ctx->m->layers[nx].qkvg.type);
        if ((rc = launch_resnorm(ctx, T, n))) return rc;
        if (!last && (rc = cap_copy(ctx, Z2H_CAP_RES_IN, nx, ctx->res, T))) return rc;
    }
    // output head + softcap on the rows that want logits
    if (head_rows == HEAD_NONE) return Z2H_OK;
    const int nout = hp.n_codebooks * hp.audio_vocab;
    GemvArgs h = gemv_dense(ctx, T, d_logits, nout, hp.logit_softcap > 0.0f ? EPI_SOFTCAP : EPI_STORE);
    const int haf = act_of(ctx->m->head.type), Kp = kpad(d);
    if (head_rows == HEAD_LAST) {
        // the encoded row T - 1 as a one-row buffer
        const int64_t r = T - 1;
        h.n_tok = 1;
        h.act.q = ctx->act.q + r * Kp; h.act.d32 = ctx->act.d32 + r * (Kp / 32); h.act.d256 = ctx->act.d256 + r * (Kp / 256);
        h.act.bs = ctx->act.bs + r * (Kp / 16); h.act.h = ctx->act.h + r * Kp;
    } else if (head_rows == HEAD_ROWS) {
        if (n_head <= 0) return Z2H_OK;
        prof_scope ps(ctx, Z2H_KF_GEMV_HEAD);
        KL(k_gather_act, dim3(n_head), dim3(256), 0, ctx->stream, ctx->act, ctx->act_y, Kp, haf, d_head_rows);
        HIPX(hipGetLastError());
        h.n_tok = n_head;
        h.act = ctx->act_y;
    }
    return launch_gemv(ctx, ctx->m->head, nullptr, h, 1, Z2H_KF_GEMV_HEAD);
}

// Raise a kernel's dynamic-LDS limit to what gfx950's 160 KiB leaves beside its static LDS.
int allow_lds(const void * fn, std::string & err) {
    hipFuncAttributes fa{};
    hipError_t e = hipFuncGetAttributes(&fa, fn);
    if (e == hipSuccess) e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 - (int) fa.sharedSizeBytes);
    if (e != hipSuccess) { err = std::string("hipFuncSetAttribute: ") + hipGetErrorString(e); return Z2H_EDEVICE; }
    return Z2H_OK;
}

// every kernel with a dynamic LDS carve-up may use the rest of the 160 KiB beside its static LDS
int set_lds_limits(std::string & err) {
#define LDS_ATTR(K_) if (int rc_ = allow_lds((const void *) &(K_), err)) return rc_;
    LDS_ATTR(k_gemv<WF_Q4_K>) LDS_ATTR(k_gemv<WF_Q6_K>) LDS_ATTR(k_gemv<WF_Q8_0>) LDS_ATTR(k_gemv<WF_F16>)
    LDS_ATTR(k_gemv_rows<WF_Q4_K>) LDS_ATTR(k_gemv_rows<WF_Q6_K>) LDS_ATTR(k_gemv_rows<WF_Q8_0>) LDS_ATTR(k_gemv_rows<WF_F16>)
    LDS_ATTR((k_gemv_split<WF_Q4_K, false, MT>)) LDS_ATTR((k_gemv_split<WF_Q8_0, false, MT>))
    LDS_ATTR((k_gemv_split<WF_Q4_K, true, MT>)) LDS_ATTR((k_gemv_split<WF_Q8_0, true, MT>))
    LDS_ATTR((k_gemv_split<WF_Q8_0, false, MT, false, true>)) LDS_ATTR((k_gemv_split<WF_Q8_0, true, MT, false, true>))
    LDS_ATTR((k_gemv_mfma<WF_Q4_K, false, MT, 1>)) LDS_ATTR((k_gemv_mfma<WF_Q8_0, false, MT, 1>))
    LDS_ATTR((k_gemv_mfma<WF_Q4_K, false, MT, 1, true>)) LDS_ATTR((k_gemv_mfma<WF_Q4_K, true, MT, 1, true>))
    LDS_ATTR((k_gemv_mfma<WF_Q4_K, true, MT, 1>)) LDS_ATTR((k_gemv_mfma<WF_Q8_0, true, MT, 1>))
    LDS_ATTR((k_gemv_mfma<WF_Q4_K, false, MT_G, m16fmt<WF_Q4_K>::GPF>)) LDS_ATTR((k_gemv_mfma<WF_Q8_0, false, MT_G, m16fmt<WF_Q8_0>::GPF>))
    LDS_ATTR((k_gemv_mfma<WF_Q4_K, true, MT_G, m16fmt<WF_Q4_K>::GPF>)) LDS_ATTR((k_gemv_mfma<WF_Q8_0, true, MT_G, m16fmt<WF_Q8_0>::GPF>))
    LDS_ATTR((k_gemv_mfma<WF_Q6_K, false, MT_G, m16fmt<WF_Q6_K>::GPF>)) LDS_ATTR((k_gemv_mfma<WF_Q6_K, true, MT_G, m16fmt<WF_Q6_K>::GPF>))
    LDS_ATTR((k_gemv_mfma<WF_Q6_K, false, MT, 1>)) LDS_ATTR((k_gemv_mfma<WF_Q6_K, true, MT, 1>))
    LDS_ATTR((k_gemv_split<WF_Q6_K, false, MT>)) LDS_ATTR((k_gemv_split<WF_Q6_K, true, MT>))
    LDS_ATTR((k_gemv_split<WF_Q6_K, false, MT_G>)) LDS_ATTR((k_gemv_split<WF_Q6_K, true, MT_G>))
    LDS_ATTR((k_router_down_t<4, false>)) LDS_ATTR((k_router_down_t<8, false>)) LDS_ATTR((k_router_down_t<16, false>))
    LDS_ATTR((k_router_down_t<32, false>)) LDS_ATTR((k_router_down_t<64, false>))
    LDS_ATTR((k_router_down_t<4, true>)) LDS_ATTR((k_router_down_t<8, true>)) LDS_ATTR((k_router_down_t<16, true>))
    LDS_ATTR((k_router_down_t<32, true>)) LDS_ATTR((k_router_down_t<64, true>))
    LDS_ATTR(k_gemm_q4k<true>) LDS_ATTR(k_gemm_q4k<false>)
    LDS_ATTR(k_attn_flash32<1>) LDS_ATTR(k_attn_flash32<2>) LDS_ATTR(k_attn_flash32<4>)
    LDS_ATTR(k_attn_flash16<1>) LDS_ATTR(k_attn_flash16<2>) LDS_ATTR(k_attn_flash16<4>)
    LDS_ATTR((k_gemm_f16<true, 4, 4>)) LDS_ATTR((k_gemm_f16<false, 4, 4>)) LDS_ATTR((k_gemm_f16<true, 2, 1>)) LDS_ATTR((k_gemm_f16<false, 1, 1>))
#define LDS_TF(H_) LDS_ATTR((k_attn_tile_f32<H_, 1>)) LDS_ATTR((k_attn_tile_f32<H_, 2>)) LDS_ATTR((k_attn_tile_f32<H_, 4>)) LDS_ATTR((k_attn_tile_f32<H_, 8>)) \
                   LDS_ATTR((k_attn_fa<H_, 1>)) LDS_ATTR((k_attn_fa<H_, 2>)) LDS_ATTR((k_attn_fa<H_, 4>)) LDS_ATTR((k_attn_fa<H_, 8>)) \
                   LDS_ATTR((k_attn_merge<H_, 1>)) LDS_ATTR((k_attn_merge<H_, 2>)) LDS_ATTR((k_attn_merge<H_, 4>)) LDS_ATTR((k_attn_merge<H_, 8>))
    LDS_TF(16) LDS_TF(32) LDS_TF(64) LDS_TF(128)
#undef LDS_TF
    LDS_ATTR(k_router_tail<false>) LDS_ATTR(k_router_tail<true>) LDS_ATTR(k_attn_combine<>) LDS_ATTR((k_attn_combine<128, 2, 4>)) LDS_ATTR(k_resnorm<RN_EMBED>) LDS_ATTR((k_resnorm<RN_EMBED, 8>)) LDS_ATTR((k_resnorm<RN_EMBED, 1>)) LDS_ATTR((k_resnorm<RN_EMBED, 0>)) LDS_ATTR((k_resnorm<RN_EMBED, 8, 10>)) LDS_ATTR((k_resnorm<RN_EMBED, 1, 10>)) LDS_ATTR((k_resnorm<RN_EMBED, 0, 10>)) LDS_ATTR(k_resnorm<RN_ACCUM>) LDS_ATTR(k_resnorm<RN_ADD>) LDS_ATTR(k_resnorm<RN_ENCODE>) LDS_ATTR(k_swiglu_encode)
#undef LDS_ATTR
    return Z2H_OK;
}

// one wave per (token, 64-row chunk, KV head) item, instantiated per head size and group size
int launch_kv_append(z2h_ctx * ctx, const AttnArgs & a, int T) {
    const dim3 grid(T, a.nkv);
    switch (a.hd) {
        case 16: KL(k_kv_append<16>, grid, dim3(64), 0, ctx->stream, a); break;
        case 32: KL(k_kv_append<32>, grid, dim3(64), 0, ctx->stream, a); break;
        case 64: KL(k_kv_append<64>, grid, dim3(64), 0, ctx->stream, a); break;
        default: KL(k_kv_append<128>, grid, dim3(64), 0, ctx->stream, a); break;
    }
    HIPX(hipGetLastError());
    return Z2H_OK;
}

int launch_attn_tile(z2h_ctx * ctx, const AttnArgs & a, int n_tiles) {
    const int grp = a.nh / a.nkv;
    if (a.kf) {
        const size_t lds = attn_tile_f32_lds(a.hd, grp);
#define ATF(H_, G_) KL((k_attn_tile_f32<H_, G_>), dim3(n_tiles), dim3(256), lds, ctx->stream, a, (const int4 *) ctx->d_tiles)
#define ATF_G(H_) switch (grp) { case 1: ATF(H_, 1); break; case 2: ATF(H_, 2); break; case 4: ATF(H_, 4); break; default: ATF(H_, 8); }
        switch (a.hd) {
            case 16: ATF_G(16) break;
            case 32: ATF_G(32) break;
            case 64: ATF_G(64) break;
            default: ATF_G(128) break;
        }
#undef ATF_G
#undef ATF
        HIPX(hipGetLastError());
        return Z2H_OK;
    }
    return seterr(ctx, Z2H_EINVAL, "chunk tiles without the prompt's fp32 K/V");
}

int launch_attn(z2h_ctx * ctx, const AttnArgs & a, int grid) {
    const int grp = a.nh / a.nkv;
#define ATT(H_, G_) KL((k_attn_chunk<H_, G_>), dim3(grid), dim3(256), 0, ctx->stream, a)
#define ATT_G(H_) switch (grp) { case 1: ATT(H_, 1); break; case 2: ATT(H_, 2); break; case 4: ATT(H_, 4); break; default: ATT(H_, 8); }
    switch (a.hd) {
        case 16: ATT_G(16) break;
        case 32: ATT_G(32) break;
        case 64: ATT_G(64) break;
        default: ATT_G(128) break;
    }
#undef ATT_G
#undef ATT
    HIPX(hipGetLastError());
    return Z2H_OK;
}

// k_attn_fa on `grid` blocks, then k_attn_merge over (row, KV head) for the rows of several segments
int launch_attn_fa(z2h_ctx * ctx, const AttnArgs & a, int grid) {
    const int grp = a.nh / a.nkv;
    const size_t lds = attn_fa_lds(a.hd);
    const size_t mlds = attn_merge_lds(a.hd, grp, (ctx->S + FA_SEG - 1) / FA_SEG);
#define ATT(H_, G_) do { KL((k_attn_fa<H_, G_>), dim3(grid), dim3(256), lds, ctx->stream, a); \
                         KL((k_attn_merge<H_, G_>), dim3(a.T * a.nkv), dim3(256), mlds, ctx->stream, a); } while (0)
#define ATT_G(H_) switch (grp) { case 1: ATT(H_, 1); break; case 2: ATT(H_, 2); break; case 4: ATT(H_, 4); break; default: ATT(H_, 8); }
    switch (a.hd) {
        case 16: ATT_G(16) break;
        case 32: ATT_G(32) break;
        case 64: ATT_G(64) break;
        default: ATT_G(128) break;
    }
#undef ATT_G
#undef ATT
    HIPX(hipGetLastError());
    return Z2H_OK;
}

int check_err_flag(z2h_ctx * ctx) {
    int h = 0;
    HIPX(hipMemcpy(&h, ctx->d_err, 4, hipMemcpyDeviceToHost));
    if (h) {
        HIPX(hipMemset(ctx->d_err, 0, 4));
        return seterr(ctx, Z2H_EINVAL, "token id out of range");
    }
    return Z2H_OK;
}

int validate_step(z2h_ctx * ctx, int T, const int32_t * slot_idx, const int32_t * n_past) {
    if (!ctx->finalized) return seterr(ctx, Z2H_ESTATE, "z2h_finalize not called");
    if (T <= 0 || T > ctx->Tstep) return seterr(ctx, Z2H_EINVAL, "n_active out of range");
    for (int t = 0; t < T; ++t) {
        if (slot_idx && (slot_idx[t] < 0 || slot_idx[t] >= ctx->n_slots)) return seterr(ctx, Z2H_EINVAL, "slot index out of range");
        if (n_past[t] < 0 || n_past[t] >= ctx->S) return seterr(ctx, Z2H_EINVAL, "n_past out of range (slot full)");
        if (slot_idx) for (int u = 0; u < t; ++u) if (slot_idx[u] == slot_idx[t]) return seterr(ctx, Z2H_EINVAL, "duplicate slot in step");
    }
    return Z2H_OK;
}

// Step on the context's input buffers (d_slot, d_npast, d_ids | d_emb) into ctx->logits: replayed
// from a captured HIP graph when graphs are on and neither capture nor profiling is active.
int step_internal(z2h_ctx * ctx, int T, const int32_t * h_npast, bool use_ids) {
    const int32_t * ids = use_ids ? ctx->d_ids : nullptr;
    const float * emb = use_ids ? nullptr : ctx->d_emb;
    if (!ctx->use_graphs || ctx->capture || ctx->prof)
        return run_step(ctx, T, h_npast, ctx->d_slot, ctx->d_npast, ids, emb, ctx->logits);
    if (ctx->graph_gen != ctx->m->gen) {             // a mask or bias buffer changed under the captured graphs
        for (auto & g : ctx->graphs) (void) hipGraphExecDestroy(g.second);
        ctx->graphs.clear();
        ctx->graph_gen = ctx->m->gen;
    }
    const auto key = std::make_pair(T, use_ids ? 1 : 0);
    auto it = ctx->graphs.find(key);
    if (it == ctx->graphs.end()) {
        hipGraph_t g = nullptr;
        HIPX(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
        const int rc = run_step(ctx, T, h_npast, ctx->d_slot, ctx->d_npast, ids, emb, ctx->logits);
        const hipError_t ec = hipStreamEndCapture(ctx->stream, &g);
        if (rc) { if (g) (void) hipGraphDestroy(g); return rc; }
        if (ec != hipSuccess) return seterr(ctx, Z2H_EDEVICE, std::string("graph capture: ") + hipGetErrorString(ec));
        hipGraphExec_t ex = nullptr;
        const hipError_t ei = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
        (void) hipGraphDestroy(g);
        if (ei != hipSuccess) return seterr(ctx, Z2H_EDEVICE, std::string("graph instantiate: ") + hipGetErrorString(ei));
        it = ctx->graphs.emplace(key, ex).first;
    }
    HIPX(hipGraphLaunch(it->second, ctx->stream));
    return Z2H_OK;
}

} // namespace

// ---------------------------------------------------------------- the no-allocation MoE layer's scratch
// z2h_model_moe_forward_noalloc carves every intermediate buffer of one MoE layer from this array
// instead of a context's allocations. Each GPU the library runs on holds its own copy for the life of
// the process; host code never names it (its name is a host-side stand-in): it uses the per-device
// address that hipGetSymbolAddress returns, taken once per device with that device current.
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t) 16 << 20;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void * g_scratch_ptr[NOALLOC_MAX_DEVICES] = {};
int g_scratch_cus[NOALLOC_MAX_DEVICES] = {};

// the device address of `scratch` on `device` and the device's compute-unit count (both looked up on
// the first call for that device, with that device current; the caller's current device is kept)
int scratch_address(int device, void ** out, int * n_cu, std::string & err) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (device < 0 || device >= NOALLOC_MAX_DEVICES) { err = "device index out of range"; return Z2H_EINVAL; }
    if (!g_scratch_ptr[device]) {
        int keep = 0;
        if (hipGetDevice(&keep) != hipSuccess) { err = "hipGetDevice failed"; return Z2H_EDEVICE; }
        if (hipSetDevice(device) != hipSuccess) { err = "hipSetDevice failed"; return Z2H_EDEVICE; }
        void * p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        int cus = 0;
        const hipError_t e2 = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
        (void) hipSetDevice(keep);
        if (e != hipSuccess || !p) { err = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e); return Z2H_EDEVICE; }
        if (e2 != hipSuccess || cus <= 0) { err = "compute-unit count query failed"; return Z2H_EDEVICE; }
        g_scratch_ptr[device] = p;
        g_scratch_cus[device] = cus;
    }
    *out = g_scratch_ptr[device];
    *n_cu = g_scratch_cus[device];
    return Z2H_OK;
}

// makes `device` current for a scope and restores the caller's current device on every exit path
struct DeviceScope {
    int prev = -1;
    bool ok = false;
    explicit DeviceScope(int device) {
        if (hipGetDevice(&prev) != hipSuccess) return;
        ok = prev == device || hipSetDevice(device) == hipSuccess;
    }
    ~DeviceScope() { if (ok && prev >= 0) (void) hipSetDevice(prev); }
};
} // namespace

// ====================================================================== C ABI
extern "C" {

int z2h_model_create(const z2h_hparams * hp, int device, z2h_model ** out) {
    if (!out) return Z2H_EINVAL;
    *out = nullptr;
    if (!hp || !hp->expert_used || hp->n_layer <= 0) return Z2H_EINVAL;
    if (hp->n_head <= 0 || hp->n_head_kv <= 0 || hp->n_head % hp->n_head_kv) return Z2H_EINVAL;
    {   // decode attention instantiations: head_dim 16/32/64/128, query heads per KV head 1/2/4/8
        const int hd = hp->head_dim, grp = hp->n_head / hp->n_head_kv;
        if ((hd != 16 && hd != 32 && hd != 64 && hd != 128) || (grp != 1 && grp != 2 && grp != 4 && grp != 8)) return Z2H_ENOTSUP;
    }
    if (hp->n_codebooks + 1 > MAX_TABLES) return Z2H_ENOTSUP;
    if (hp->n_embd % 4 || hp->n_embd > 4 * 256 * RN_NV) return Z2H_ENOTSUP;   // k_resnorm row layout
    if (hipSetDevice(device) != hipSuccess) return Z2H_EDEVICE;
    auto mdl = std::make_unique<z2h_model>();
    mdl->hp = *hp;
    mdl->expert_used.assign(hp->expert_used, hp->expert_used + hp->n_layer);
    mdl->hp.expert_used = mdl->expert_used.data();
    mdl->device = device;
    mdl->W = hp->n_codebooks + 1;
    mdl->rd = hp->router_dim;
    for (int L = 0; L < hp->n_layer; ++L) mdl->kmax = std::max(mdl->kmax, hp->expert_used[L]);
    mdl->layers.resize(hp->n_layer);
    mdl->tab.assign(mdl->W, nullptr); mdl->tab_type.assign(mdl->W, -1); mdl->tab_rows.assign(mdl->W, 0);
    *out = mdl.release();
    return Z2H_OK;
}

int z2h_model_upload_tensor(z2h_model * mdl, const char * name_c, int type, const int64_t ne_in[4], const void * data, size_t nbytes) {
    if (!mdl || !name_c || !ne_in || !data) return Z2H_EINVAL;
    if (mdl->finalized) return seterr(mdl, Z2H_ESTATE, "model already finalized");
    if (!z2::type_known(type)) return seterr(mdl, Z2H_ENOTSUP, std::string("unsupported tensor type for ") + name_c);
    HostTensor t; t.type = type;
    for (int i = 0; i < 4; ++i) t.ne[i] = ne_in[i] > 0 ? ne_in[i] : 1;
    if (t.ne[0] % z2::type_block(type)) return seterr(mdl, Z2H_EINVAL, std::string("row not block aligned: ") + name_c);
    const int64_t expect = z2::row_bytes(type, t.ne[0]) * t.ne[1] * t.ne[2] * t.ne[3];
    if ((int64_t) nbytes != expect) return seterr(mdl, Z2H_EINVAL, std::string("byte size mismatch for ") + name_c);
    if (hipSetDevice(mdl->device) != hipSuccess) return Z2H_EDEVICE;
    const std::string name(name_c);
    const auto & hp = mdl->hp;
    const uint8_t * src = (const uint8_t *) data;
    auto copy_host = [&]() { t.bytes.assign(src, src + nbytes); };
    mdl->seen[name] = true;
    int L; std::string rest;
    if (parse_layer(name, L, rest)) {
        if (L < 0 || L >= hp.n_layer) return seterr(mdl, Z2H_EINVAL, "layer index out of range: " + name);
        Layer & ly = mdl->layers[L];
        if (rest == "attn_q.weight" || rest == "attn_k.weight" || rest == "attn_v.weight" || rest == "attn_gate.weight") {
            copy_host();
            ly.stash[rest] = std::move(t);
            return fuse_qkvg(mdl, ly);
        }
        if (rest == "attn_output.weight") return upload_mat(mdl, type, t.ne[0], t.ne[1], 1, src, ly.wo);
        if (rest == "ffn_up.weight") return upload_mat(mdl, type, t.ne[0], t.ne[1], 1, src, ly.ffn_up);
        if (rest == "ffn_gate.weight") return upload_mat(mdl, type, t.ne[0], t.ne[1], 1, src, ly.ffn_gate);
        if (rest == "ffn_down.weight") return upload_mat(mdl, type, t.ne[0], t.ne[1], 1, src, ly.ffn_down);
        if (rest == "ffn_gate_exps.weight") return upload_mat(mdl, type, t.ne[0], t.ne[1], (int) t.ne[2], src, ly.gate_exps);
        if (rest == "ffn_up_exps.weight") { ly.E = (int) t.ne[2]; return upload_mat(mdl, type, t.ne[0], t.ne[1], (int) t.ne[2], src, ly.up_exps); }
        if (rest == "ffn_down_exps.weight") return upload_mat(mdl, type, t.ne[0], t.ne[1], (int) t.ne[2], src, ly.down_exps);
        copy_host();
        if (rest == "attn_norm.weight") return upload_f32(mdl, t, &ly.attn_norm, hp.n_embd);
        if (rest == "ffn_norm.weight") return upload_f32(mdl, t, &ly.ffn_norm, hp.n_embd);
        if (rest == "attn_temp") return upload_f32(mdl, t, &ly.attn_temp, hp.n_head);
        if (rest == "router_down.weight") {
            if (t.ne[1] != mdl->rd) return seterr(mdl, Z2H_EINVAL, "router_dim mismatch: " + name);
            return upload_f32(mdl, t, &ly.r_down, -1);
        }
        if (rest == "router_down.bias") return upload_f32(mdl, t, &ly.r_down_b, mdl->rd);
        if (rest == "router_mlp0.weight") return upload_f32_rows_padded(mdl, t, &ly.r_m0t);
        if (rest == "router_mlp0.bias") return upload_f32(mdl, t, &ly.r_m0_b, mdl->rd);
        if (rest == "router_mlp2.weight") return upload_f32_rows_padded(mdl, t, &ly.r_m2t);
        if (rest == "router_mlp2.bias") return upload_f32(mdl, t, &ly.r_m2_b, mdl->rd);
        if (rest == "router_mlp4.weight") return upload_f32_rows_padded(mdl, t, &ly.r_m4t);
        if (rest == "router_norm.weight") return upload_f32(mdl, t, &ly.r_norm, mdl->rd);
        if (rest == "router_bias") return upload_f32(mdl, t, &ly.r_bias, -1);
        if (rest == "router_eda_scale") return upload_f32(mdl, t, &ly.r_eda, mdl->rd);
        return seterr(mdl, Z2H_EINVAL, "unknown tensor " + name);
    }
    if (name.rfind("audio_embd.", 0) == 0 || name == "text_embd.weight") {
        const int k = name == "text_embd.weight" ? hp.n_codebooks : std::atoi(name.c_str() + 11);
        if (k < 0 || k > hp.n_codebooks || t.ne[0] != hp.n_embd) return seterr(mdl, Z2H_EINVAL, "bad embedding table " + name);
        if (type != Z2H_F32 && type != Z2H_F16 && type != Z2H_Q8_0 && type != Z2H_Q4_K && type != Z2H_Q6_K)
            return seterr(mdl, Z2H_ENOTSUP, "embedding type");
        uint8_t * p = nullptr;
        if (int rc = dalloc(mdl, &p, nbytes, mdl->bytes_w)) return rc;
        HIPM(hipMemcpy(p, data, nbytes, hipMemcpyHostToDevice));
        mdl->tab[k] = p; mdl->tab_type[k] = type; mdl->tab_rows[k] = t.ne[1];
        return Z2H_OK;
    }
    if (name == "output.weight") return upload_mat(mdl, type, t.ne[0], t.ne[1], 1, src, mdl->head);
    if (name == "spk_lda.weight") return upload_mat(mdl, type, t.ne[0], t.ne[1], 1, src, mdl->spk_lda);
    if (name == "spk_proj.weight") return upload_mat(mdl, type, t.ne[0], t.ne[1], 1, src, mdl->spk_proj);
    copy_host();
    if (name == "output_norm.weight") return upload_f32(mdl, t, &mdl->output_norm, hp.n_embd);
    if (name == "spk_lda.bias") return upload_f32(mdl, t, &mdl->spk_lda_b, -1);
    if (name == "spk_proj.bias") return upload_f32(mdl, t, &mdl->spk_proj_b, hp.n_embd);
    return seterr(mdl, Z2H_EINVAL, "unknown tensor " + name);
}

int z2h_model_finalize(z2h_model * mdl) {
    if (!mdl) return Z2H_EINVAL;
    if (mdl->finalized) return Z2H_OK;
    const auto & hp = mdl->hp;
    std::string missing;
    for (int k = 0; k < mdl->W; ++k) if (!mdl->tab[k]) missing += (k < hp.n_codebooks ? "audio_embd." + std::to_string(k) : std::string("text_embd")) + " ";
    if (!mdl->head.ok()) missing += "output.weight ";
    if (!mdl->output_norm) missing += "output_norm.weight ";
    for (int L = 0; L < hp.n_layer; ++L) {
        Layer & ly = mdl->layers[L];
        const std::string b = "blk." + std::to_string(L) + ".";
        ly.k = hp.expert_used[L]; ly.moe = ly.k > 0;
        if (!ly.qkvg.ok()) missing += b + "attn_{q,k,v,gate} ";
        if (!ly.wo.ok()) missing += b + "attn_output ";
        if (!ly.attn_norm) missing += b + "attn_norm ";
        if (!ly.ffn_norm) missing += b + "ffn_norm ";
        if (!ly.attn_temp) missing += b + "attn_temp ";
        if (ly.moe) {
            if (!ly.gate_exps.ok() || !ly.up_exps.ok() || !ly.down_exps.ok()) missing += b + "ffn_*_exps ";
            if (!ly.r_down || !ly.r_down_b || !ly.r_m0t || !ly.r_m0_b || !ly.r_m2t || !ly.r_m2_b || !ly.r_m4t || !ly.r_norm || !ly.r_bias)
                missing += b + "router_* ";
            if (ly.up_exps.ok() && ly.k > ly.E) return seterr(mdl, Z2H_EINVAL, b + "top-k exceeds the expert count");
            if (ly.up_exps.ok() && ly.E > 128) return seterr(mdl, Z2H_ENOTSUP, "more than 128 experts");
            if (ly.up_exps.ok() && (ly.up_exps.rows != hp.n_ff || ly.down_exps.K != hp.n_ff)) return seterr(mdl, Z2H_EINVAL, b + "expert shape mismatch");
        } else if (!ly.ffn_up.ok() || !ly.ffn_gate.ok() || !ly.ffn_down.ok()) missing += b + "ffn_{up,gate,down} ";
    }
    if (!missing.empty()) return seterr(mdl, Z2H_EINVAL, "missing tensors: " + missing);
    {
        std::string err;
        if (hipSetDevice(mdl->device) != hipSuccess) return seterr(mdl, Z2H_EDEVICE, "hipSetDevice failed");
        if (int rc = set_lds_limits(err)) return seterr(mdl, rc, err);
    }
    if (mdl->rd > 0) {
        if (mdl->rd != 32 && mdl->rd != 64 && mdl->rd != 128) return seterr(mdl, Z2H_ENOTSUP, "router_dim must be 32, 64 or 128");
        if (mdl->kmax > 8) return seterr(mdl, Z2H_ENOTSUP, "top-k above 8");
    }
    mdl->finalized = true;
    return Z2H_OK;
}

const char * z2h_model_last_error(const z2h_model * mdl) { return mdl ? mdl->err.c_str() : "null model"; }

void z2h_model_release(z2h_model * mdl) {
    if (!mdl || --mdl->refs > 0) return;
    (void) hipSetDevice(mdl->device);
    for (void * p : mdl->allocs) (void) hipFree(p);
    delete mdl;
}

int z2h_create_batch(z2h_model * mdl, int n_slots, int slot_cap_frames, z2h_ctx ** out) {
    return z2h_create_batch_rows(mdl, n_slots, slot_cap_frames, 0, out);
}

int z2h_create_batch_rows(z2h_model * mdl, int n_slots, int slot_cap_frames, int max_rows, z2h_ctx ** out) {
    if (!out) return Z2H_EINVAL;
    *out = nullptr;
    if (!mdl || n_slots <= 0 || slot_cap_frames <= 0) return Z2H_EINVAL;
    if (hipSetDevice(mdl->device) != hipSuccess) return Z2H_EDEVICE;
    auto ctx = std::make_unique<z2h_ctx>();
    z2h_ctx * c = ctx.get();
    c->m = mdl; ++mdl->refs;
    c->hp = mdl->hp;
    c->device = mdl->device; c->n_slots = n_slots;
    c->max_rows = std::max(0, max_rows);
    c->S = ((slot_cap_frames + 255) / 256) * 256;
    c->W = mdl->W; c->rd = mdl->rd; c->kmax = mdl->kmax;
    const auto & hp = c->hp;
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) { z2h_destroy(ctx.release()); return Z2H_EDEVICE; }
    const size_t kv_elems = (size_t) hp.n_layer * 2 * n_slots * hp.n_head_kv * c->S * hp.head_dim;
    if (dalloc(c, &c->kv, kv_elems * 2, c->bytes_kv) ||
        dalloc(c, &c->kv_stage, (size_t) c->S * hp.n_head_kv * hp.head_dim * 2, c->bytes_scratch)) { z2h_destroy(ctx.release()); return Z2H_ENOMEM; }
    if (hipMemset(c->kv, 0, kv_elems * 2) != hipSuccess) { z2h_destroy(ctx.release()); return Z2H_EDEVICE; }
    if (mdl->finalized) {
        if (int rc = z2h_finalize(c)) { z2h_destroy(ctx.release()); return rc; }
    }
    *out = ctx.release();
    return Z2H_OK;
}

int z2h_create(const z2h_hparams * hp, int n_slots, int slot_cap_frames, int device, z2h_ctx ** out) {
    if (!out) return Z2H_EINVAL;
    *out = nullptr;
    if (n_slots <= 0 || slot_cap_frames <= 0) return Z2H_EINVAL;
    z2h_model * mdl = nullptr;
    if (int rc = z2h_model_create(hp, device, &mdl)) return rc;
    const int rc = z2h_create_batch(mdl, n_slots, slot_cap_frames, out);
    z2h_model_release(mdl);                          // the context holds the only reference now
    return rc;
}

int z2h_slot_cap(const z2h_ctx * ctx) { return ctx ? ctx->S : 0; }

int z2h_upload_tensor(z2h_ctx * ctx, const char * name, int type, const int64_t ne[4], const void * data, size_t nbytes) {
    if (!ctx) return Z2H_EINVAL;
    if (ctx->finalized) return seterr(ctx, Z2H_ESTATE, "context already finalized");
    const int rc = z2h_model_upload_tensor(ctx->m, name, type, ne, data, nbytes);
    if (rc) ctx->err = ctx->m->err;
    return rc;
}

int z2h_finalize(z2h_ctx * ctx) {
    if (!ctx) return Z2H_EINVAL;
    if (ctx->finalized) return Z2H_OK;
    if (int rc = z2h_model_finalize(ctx->m)) { ctx->err = ctx->m->err; return rc; }
    const auto & hp = ctx->hp;
    if (hp.n_expert > SORT_EMAX) return seterr(ctx, Z2H_ENOTSUP, "more experts than the route sort handles (256)");
    if (int rc = alloc_scratch(ctx)) return rc;
    HIPX(hipMemset(ctx->d_err, 0, 16));
    {
        std::string err;
        if (int rc = set_lds_limits(err)) return seterr(ctx, rc, err);
    }
    {
        int n_cu = 0, per_cu = 0;
        HIPX(hipSetDevice(ctx->device));
        HIPX(hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, ctx->device));
        const void * fn = nullptr;
        const int grp = hp.n_head / std::max(1, hp.n_head_kv);
#define ATT_FN(H_) fn = grp == 1 ? (const void *) &k_attn_chunk<H_, 1> : grp == 2 ? (const void *) &k_attn_chunk<H_, 2> : \
                        grp == 4 ? (const void *) &k_attn_chunk<H_, 4> : (const void *) &k_attn_chunk<H_, 8>
        switch (hp.head_dim) {
            case 16: ATT_FN(16); break;
            case 32: ATT_FN(32); break;
            case 64: ATT_FN(64); break;
            default: ATT_FN(128); break;
        }
#undef ATT_FN
        HIPX(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 256, 0));
        if (n_cu > 0 && per_cu > 0) ctx->attn_slots = n_cu * per_cu;
        if (n_cu > 0) ctx->n_cu = n_cu;
    }
    (void) hp;
    ctx->graph_gen = ctx->m->gen;
    ctx->finalized = true;
    return Z2H_OK;
}

int z2h_kv_write(z2h_ctx * ctx, int layer, int slot, int row0, int n, const uint16_t * k, const uint16_t * v) {
    if (!ctx) return Z2H_EINVAL;
    const auto & hp = ctx->hp;
    if (layer < 0 || layer >= hp.n_layer || slot < 0 || slot >= ctx->n_slots || row0 < 0 || n < 0 || row0 + n > ctx->S)
        return seterr(ctx, Z2H_EINVAL, "kv_write out of range");
    if (n == 0) return Z2H_OK;
    HIPX(hipSetDevice(ctx->device));
    const int nkv = hp.n_head_kv, hd = hp.head_dim;
    const size_t lsz = (size_t) ctx->n_slots * nkv * ctx->S * hd;
    const int grid = (int) std::min<int64_t>(1024, ((int64_t) n * nkv * (hd / 8) + 255) / 256);
    for (int which = 0; which < 2; ++which) {
        const uint16_t * src = which ? v : k;
        if (!src) continue;
        HIPX(hipMemcpyAsync(ctx->kv_stage, src, (size_t) n * nkv * hd * 2, hipMemcpyHostToDevice, ctx->stream));
        KL(k_kv_move, dim3(grid), dim3(256), 0, ctx->stream, ctx->kv_stage,
                           ctx->kv + (size_t) (2 * layer + which) * lsz, n, nkv, hd, ctx->S, row0, slot, 0);
        HIPX(hipGetLastError());
        HIPX(hipStreamSynchronize(ctx->stream));      // the staging buffer is reused by the next copy
    }
    return Z2H_OK;
}

int z2h_kv_read(z2h_ctx * ctx, int layer, int slot, int row0, int n, uint16_t * k, uint16_t * v) {
    if (!ctx) return Z2H_EINVAL;
    const auto & hp = ctx->hp;
    if (layer < 0 || layer >= hp.n_layer || slot < 0 || slot >= ctx->n_slots || row0 < 0 || n < 0 || row0 + n > ctx->S)
        return seterr(ctx, Z2H_EINVAL, "kv_read out of range");
    if (n == 0) return Z2H_OK;
    HIPX(hipSetDevice(ctx->device));
    const int nkv = hp.n_head_kv, hd = hp.head_dim;
    const size_t lsz = (size_t) ctx->n_slots * nkv * ctx->S * hd;
    const int grid = (int) std::min<int64_t>(1024, ((int64_t) n * nkv * (hd / 8) + 255) / 256);
    for (int which = 0; which < 2; ++which) {
        uint16_t * dst = which ? v : k;
        if (!dst) continue;
        KL(k_kv_move, dim3(grid), dim3(256), 0, ctx->stream, ctx->kv_stage,
                           ctx->kv + (size_t) (2 * layer + which) * lsz, n, nkv, hd, ctx->S, row0, slot, 1);
        HIPX(hipGetLastError());
        HIPX(hipMemcpyAsync(dst, ctx->kv_stage, (size_t) n * nkv * hd * 2, hipMemcpyDeviceToHost, ctx->stream));
        HIPX(hipStreamSynchronize(ctx->stream));
    }
    return Z2H_OK;
}

int z2h_step(z2h_ctx * ctx, int T, const int32_t * slot_idx, const int32_t * n_past, const int32_t * ids,
             const float * emb, float * out_logits) {
    if (!ctx || !slot_idx || !n_past || (!ids && !emb)) return ctx ? seterr(ctx, Z2H_EINVAL, "null argument") : Z2H_EINVAL;
    if (int rc = validate_step(ctx, T, slot_idx, n_past)) return rc;
    if (ids) {
        for (int t = 0; t < T; ++t)
            for (int k = 0; k < ctx->W; ++k) {
                const int id = ids[(size_t) t * ctx->W + k];
                if (id < 0 || id >= ctx->m->tab_rows[k]) return seterr(ctx, Z2H_EINVAL, "token id out of range");
            }
    }
    HIPX(hipSetDevice(ctx->device));
    int32_t * hp_ = ctx->h_pin;
    std::memcpy(hp_, slot_idx, (size_t) T * 4);
    std::memcpy(hp_ + T, n_past, (size_t) T * 4);
    if (ids) std::memcpy(hp_ + 2 * T, ids, (size_t) T * ctx->W * 4);
    HIPX(hipMemcpyAsync(ctx->d_slot, hp_, (size_t) T * 4, hipMemcpyHostToDevice, ctx->stream));
    HIPX(hipMemcpyAsync(ctx->d_npast, hp_ + T, (size_t) T * 4, hipMemcpyHostToDevice, ctx->stream));
    if (ids) HIPX(hipMemcpyAsync(ctx->d_ids, hp_ + 2 * T, (size_t) T * ctx->W * 4, hipMemcpyHostToDevice, ctx->stream));
    if (emb) HIPX(hipMemcpyAsync(ctx->d_emb, emb, (size_t) T * ctx->hp.n_embd * 4, hipMemcpyHostToDevice, ctx->stream));
    ctx->resident_T = ctx->resident_last = 0;
    ctx->last_np.assign(n_past, n_past + T);
    if (int rc = step_internal(ctx, T, n_past, ids != nullptr)) return rc;
    const size_t nout = (size_t) T * ctx->hp.n_codebooks * ctx->hp.audio_vocab;
    if (out_logits) HIPX(hipMemcpyAsync(out_logits, ctx->logits, nout * 4, hipMemcpyDeviceToHost, ctx->stream));
    HIPX(hipStreamSynchronize(ctx->stream));
    if (int rc = check_err_flag(ctx)) return rc;
    ctx->resident_last = T;
    return Z2H_OK;
}

int z2h_step_device(z2h_ctx * ctx, int T, const int32_t * d_slot, const int32_t * d_npast, const int32_t * h_npast,
                    const int32_t * d_ids, const float * d_emb, float * d_logits, void * stream) {
    if (!ctx || !d_slot || !d_npast || !h_npast || (!d_ids && !d_emb) || !d_logits) return ctx ? seterr(ctx, Z2H_EINVAL, "null argument") : Z2H_EINVAL;
    if (int rc = validate_step(ctx, T, nullptr, h_npast)) return rc;
    hipStream_t keep = ctx->stream;
    if (stream) ctx->stream = (hipStream_t) stream;
    int rc = Z2H_OK;
    ctx->resident_T = ctx->resident_last = 0;
    ctx->last_np.assign(h_npast, h_npast + T);
    if (ctx->use_graphs && !ctx->capture && !ctx->prof) {
        // inputs into the context's fixed buffers, replay, logits out
        const size_t nout = (size_t) T * ctx->hp.n_codebooks * ctx->hp.audio_vocab;
        auto cp = [&](void * dst, const void * src, size_t n) {
            return hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, ctx->stream) == hipSuccess;
        };
        if (!cp(ctx->d_slot, d_slot, (size_t) T * 4) || !cp(ctx->d_npast, d_npast, (size_t) T * 4) ||
            (d_ids && !cp(ctx->d_ids, d_ids, (size_t) T * ctx->W * 4)) ||
            (d_emb && !cp(ctx->d_emb, d_emb, (size_t) T * ctx->hp.n_embd * 4)))
            rc = seterr(ctx, Z2H_EDEVICE, "input copy failed");
        if (!rc) rc = step_internal(ctx, T, h_npast, d_ids != nullptr);
        if (!rc && !cp(d_logits, ctx->logits, nout * 4)) rc = seterr(ctx, Z2H_EDEVICE, "logits copy failed");
        if (!rc && d_ids) ctx->resident_last = T;
    } else {
        rc = run_step(ctx, T, h_npast, d_slot, d_npast, d_ids, d_emb, d_logits);
    }
    ctx->stream = keep;
    return rc;
}

// Speaker rows (graph.cpp:262-297): sp = W_proj (W_lda spk + b_lda) + b_proj (+ delta), for n <=
// Z2H_SPEAKER_MAX speaker vectors at once (each GEMV takes the n rows as one batch) -> host [n][n_embd]
static int speaker_rows(z2h_ctx * ctx, int n, const float * spk, const float * delta, float * out) {
    z2h_model * m = ctx->m;
    const auto & hp = ctx->hp;
    if (!m->spk_lda.ok() || !m->spk_proj.ok() || !m->spk_lda_b || !m->spk_proj_b || !ctx->spk_io)
        return seterr(ctx, Z2H_ESTATE, "speaker tensors (spk_lda / spk_proj) not uploaded");
    if (n <= 0 || n > Z2H_SPEAKER_MAX) return seterr(ctx, Z2H_EINVAL, "speaker rows out of range (1 .. Z2H_SPEAKER_MAX)");
    const int sd = hp.spk_dim, ld = hp.spk_lda_dim, d = hp.n_embd;
    if (m->spk_lda.K != sd || m->spk_lda.rows != ld || m->spk_proj.K != ld || m->spk_proj.rows != d)
        return seterr(ctx, Z2H_EINVAL, "speaker tensor shapes do not match spk_dim / spk_lda_dim");
    float * x = ctx->spk_io, * sl = x + (size_t) n * kpad(sd), * sp = sl + (size_t) n * kpad(ld), * dl = sp + (size_t) n * kpad(d);
    int rc;
    HIPX(hipMemcpyAsync(x, spk, (size_t) n * sd * 4, hipMemcpyHostToDevice, ctx->stream));
    if (delta) HIPX(hipMemcpyAsync(dl, delta, (size_t) n * d * 4, hipMemcpyHostToDevice, ctx->stream));
    if ((rc = launch_encode(ctx, x, sd, sd, n, act_of(m->spk_lda.type), ctx->act))) return rc;
    if ((rc = launch_gemv(ctx, m->spk_lda, nullptr, gemv_dense(ctx, n, sl, ld, EPI_STORE), 1, Z2H_KF_GEMV_DENSE))) return rc;
    for (int r = 0; r < n; ++r) {
        KL(k_bias_add, dim3((ld + 255) / 256), dim3(256), 0, ctx->stream, sl + (size_t) r * ld, (const float *) m->spk_lda_b, (const float *) nullptr, ld);
        HIPX(hipGetLastError());
    }
    if ((rc = launch_encode(ctx, sl, ld, ld, n, act_of(m->spk_proj.type), ctx->act))) return rc;
    if ((rc = launch_gemv(ctx, m->spk_proj, nullptr, gemv_dense(ctx, n, sp, d, EPI_STORE), 1, Z2H_KF_GEMV_DENSE))) return rc;
    for (int r = 0; r < n; ++r) {
        KL(k_bias_add, dim3((d + 255) / 256), dim3(256), 0, ctx->stream, sp + (size_t) r * d, (const float *) m->spk_proj_b,
           (const float *) (delta ? dl + (size_t) r * d : nullptr), d);
        HIPX(hipGetLastError());
    }
    HIPX(hipMemcpyAsync(out, sp, (size_t) n * d * 4, hipMemcpyDeviceToHost, ctx->stream));
    HIPX(hipStreamSynchronize(ctx->stream));
    return Z2H_OK;
}

int z2h_prefill(z2h_ctx * ctx, int slot, const int32_t * ids, int n0, const float * spk, int spk_pos,
                const float * delta, float * last_logits) {
    if (!ctx || !ids || !last_logits) return Z2H_EINVAL;
    if (!ctx->finalized) return seterr(ctx, Z2H_ESTATE, "z2h_finalize not called");
    if (slot < 0 || slot >= ctx->n_slots) return seterr(ctx, Z2H_EINVAL, "slot out of range");
    if (n0 <= 0 || n0 > ctx->S) return seterr(ctx, Z2H_EINVAL, "prefill n0 exceeds slot_cap");
    if (spk && (spk_pos < 0 || spk_pos >= n0)) return seterr(ctx, Z2H_EINVAL, "spk_pos outside the prompt");
    const int W = ctx->W;
    for (int64_t i = 0; i < (int64_t) n0 * W; ++i) {
        const int k = (int) (i % W);
        if ((!spk || i / W != spk_pos) && (ids[i] < 0 || ids[i] >= ctx->m->tab_rows[k])) return seterr(ctx, Z2H_EINVAL, "token id out of range");
    }
    HIPX(hipSetDevice(ctx->device));
    ctx->resident_T = ctx->resident_last = 0;
    std::vector<float> sp;
    if (spk) {
        sp.resize(ctx->hp.n_embd);
        if (int rc = speaker_rows(ctx, 1, spk, delta, sp.data())) return rc;
    }
    // causal prefill in chunks of rows [r0, r0 + T): every row of a chunk appends its K/V (f16 into the
    // cache, fp32 into the prompt rows) before the chunk's attention, then row r attends the prompt's
    // fp32 rows [0, r], as the reference's one-graph prefill attends its fp32 K/V (graph.cpp:155-169).
    // A row's arithmetic does not depend on the chunk it is in, so any chunk size gives the same bits.
    // With capture on, chunks stay within the step width the capture buffers hold.
    const int chunk = std::max(1, std::min(ctx->pch, ctx->capture ? ctx->Tstep : ctx->Tmax));
    const size_t row = (size_t) ctx->hp.n_codebooks * ctx->hp.audio_vocab;
    for (int r0 = 0; r0 < n0; r0 += chunk) {
        const int T = std::min(chunk, n0 - r0);
        const bool last = r0 + T == n0;
        int32_t * hp_ = ctx->h_pin;
        for (int t = 0; t < T; ++t) { hp_[t] = slot; hp_[T + t] = r0 + t; }
        std::memcpy(hp_ + 2 * T, ids + (size_t) r0 * W, (size_t) T * W * 4);
        const int er = spk && spk_pos >= r0 && spk_pos < r0 + T ? spk_pos - r0 : -1;
        if (er >= 0) for (int k = 0; k < W; ++k) hp_[2 * T + er * W + k] = 0;      // the row's ids are unused
        int32_t * map = hp_ + 2 * T + T * W;                         // -1 but for the speaker row
        for (int t = 0; t < T; ++t) map[t] = t == er ? 0 : -1;
        HIPX(hipMemcpyAsync(ctx->d_slot, hp_, (size_t) T * 4, hipMemcpyHostToDevice, ctx->stream));
        HIPX(hipMemcpyAsync(ctx->d_npast, hp_ + T, (size_t) T * 4, hipMemcpyHostToDevice, ctx->stream));
        HIPX(hipMemcpyAsync(ctx->d_ids, hp_ + 2 * T, (size_t) T * W * 4, hipMemcpyHostToDevice, ctx->stream));
        if (er >= 0) {
            HIPX(hipMemcpyAsync(ctx->d_emb, sp.data(), (size_t) ctx->hp.n_embd * 4, hipMemcpyHostToDevice, ctx->stream));
            HIPX(hipMemcpyAsync(ctx->d_emb_map, map, (size_t) T * 4, hipMemcpyHostToDevice, ctx->stream));
        }
        if (int rc = run_step(ctx, T, hp_ + T, ctx->d_slot, ctx->d_npast, ctx->d_ids, er >= 0 ? ctx->d_emb : nullptr,
                              ctx->logits, /*kv_pre=*/true, er >= 0 ? ctx->d_emb_map : nullptr, hp_, /*f32_prompt=*/true,
                              last ? HEAD_LAST : HEAD_NONE)) return rc;
        if (last) HIPX(hipMemcpyAsync(last_logits, ctx->logits, row * 4, hipMemcpyDeviceToHost, ctx->stream));
        HIPX(hipStreamSynchronize(ctx->stream));               // the pinned inputs are reused by the next chunk
    }
    return check_err_flag(ctx);
}

int z2h_speaker_embed(z2h_ctx * ctx, int n, const float * spk, const float * delta, float * out) {
    if (!ctx || !spk || !out) return ctx ? seterr(ctx, Z2H_EINVAL, "null argument") : Z2H_EINVAL;
    if (!ctx->finalized) return seterr(ctx, Z2H_ESTATE, "z2h_finalize not called");
    HIPX(hipSetDevice(ctx->device));
    return speaker_rows(ctx, n, spk, delta, out);
}

int z2h_step_mixed(z2h_ctx * ctx, int n_rows, const int32_t * slot_idx, const int32_t * n_past, const int32_t * ids,
                   const int32_t * emb_map, const float * emb, int n_emb, int n_out, const int32_t * out_rows, float * out_logits) {
    if (!ctx || !slot_idx || !n_past || !ids || (n_out > 0 && (!out_rows || !out_logits)))
        return ctx ? seterr(ctx, Z2H_EINVAL, "null argument") : Z2H_EINVAL;
    if (!ctx->finalized) return seterr(ctx, Z2H_ESTATE, "z2h_finalize not called");
    if (n_rows <= 0 || n_rows > ctx->Tmax || (ctx->capture && n_rows > ctx->Tstep)) return seterr(ctx, Z2H_EINVAL, "n_rows out of range");
    if (emb_map && (!emb || n_emb <= 0)) return seterr(ctx, Z2H_EINVAL, "emb_map without embedding rows");
    const int W = ctx->W;
    std::set<std::pair<int, int>> seen;
    for (int t = 0; t < n_rows; ++t) {
        if (slot_idx[t] < 0 || slot_idx[t] >= ctx->n_slots) return seterr(ctx, Z2H_EINVAL, "slot index out of range");
        if (n_past[t] < 0 || n_past[t] >= ctx->S) return seterr(ctx, Z2H_EINVAL, "n_past out of range");
        if (!seen.insert({slot_idx[t], n_past[t]}).second) return seterr(ctx, Z2H_EINVAL, "two rows write the same cache row");
        const int em = emb_map ? emb_map[t] : -1;
        if (em < -1 || em >= n_emb) return seterr(ctx, Z2H_EINVAL, "emb_map entry out of range");
        if (em < 0)
            for (int k = 0; k < W; ++k) {
                const int id = ids[(size_t) t * W + k];
                if (id < 0 || id >= ctx->m->tab_rows[k]) return seterr(ctx, Z2H_EINVAL, "token id out of range");
            }
    }
    if (n_out < 0 || n_out > ctx->Tmax) return seterr(ctx, Z2H_EINVAL, "n_out out of range");
    for (int i = 0; i < n_out; ++i)
        if (out_rows[i] < 0 || out_rows[i] >= n_rows) return seterr(ctx, Z2H_EINVAL, "out_rows entry out of range");
    if (emb_map && (size_t) n_emb * ctx->hp.n_embd > (size_t) ctx->Tmax * ctx->hp.n_embd) return seterr(ctx, Z2H_EINVAL, "too many embedding rows");
    HIPX(hipSetDevice(ctx->device));
    ctx->resident_T = ctx->resident_last = 0;
    int32_t * hp_ = ctx->h_pin;
    std::memcpy(hp_, slot_idx, (size_t) n_rows * 4);
    std::memcpy(hp_ + n_rows, n_past, (size_t) n_rows * 4);
    int32_t * hid = hp_ + 2 * n_rows;
    std::memcpy(hid, ids, (size_t) n_rows * W * 4);
    int32_t * map = hid + (size_t) n_rows * W;
    for (int t = 0; t < n_rows; ++t) {
        map[t] = emb_map ? emb_map[t] : -1;
        if (map[t] >= 0) for (int k = 0; k < W; ++k) hid[(size_t) t * W + k] = 0;     // unused ids
    }
    HIPX(hipMemcpyAsync(ctx->d_slot, hp_, (size_t) n_rows * 4, hipMemcpyHostToDevice, ctx->stream));
    HIPX(hipMemcpyAsync(ctx->d_npast, hp_ + n_rows, (size_t) n_rows * 4, hipMemcpyHostToDevice, ctx->stream));
    HIPX(hipMemcpyAsync(ctx->d_ids, hid, (size_t) n_rows * W * 4, hipMemcpyHostToDevice, ctx->stream));
    if (emb_map) {
        HIPX(hipMemcpyAsync(ctx->d_emb_map, map, (size_t) n_rows * 4, hipMemcpyHostToDevice, ctx->stream));
        HIPX(hipMemcpyAsync(ctx->d_emb, emb, (size_t) n_emb * ctx->hp.n_embd * 4, hipMemcpyHostToDevice, ctx->stream));
    }
    // the requested rows' indices (pinned, after the ids and the embedding map)
    int32_t * hrows = map + n_rows;
    std::memcpy(hrows, out_rows, (size_t) n_out * 4);
    if (n_out > 0) HIPX(hipMemcpyAsync(ctx->d_head_rows, hrows, (size_t) n_out * 4, hipMemcpyHostToDevice, ctx->stream));
    // every row appends its K/V before the attention; a slot's rows attend causally to each other; the
    // head runs on the requested rows only
    if (int rc = run_step(ctx, n_rows, hp_ + n_rows, ctx->d_slot, ctx->d_npast, ctx->d_ids, emb_map ? ctx->d_emb : nullptr,
                          ctx->logits, /*kv_pre=*/true, emb_map ? ctx->d_emb_map : nullptr, hp_, false,
                          HEAD_ROWS, ctx->d_head_rows, n_out)) return rc;
    const size_t row = (size_t) ctx->hp.n_codebooks * ctx->hp.audio_vocab;
    if (n_out > 0) HIPX(hipMemcpyAsync(out_logits, ctx->logits, (size_t) n_out * row * 4, hipMemcpyDeviceToHost, ctx->stream));
    HIPX(hipStreamSynchronize(ctx->stream));
    return check_err_flag(ctx);
}

int z2h_set_prefill_chunk(z2h_ctx * ctx, int rows) {
    if (!ctx) return Z2H_EINVAL;
    if (!ctx->finalized) return seterr(ctx, Z2H_ESTATE, "z2h_finalize not called");
    if (rows <= 0 || rows > ctx->Tmax) return seterr(ctx, Z2H_EINVAL, "prefill chunk out of range (1 .. the context's row capacity)");
    ctx->pch = rows;
    return Z2H_OK;
}

int z2h_moe_forward_device(z2h_ctx * ctx, int layer, int T, const float * d_x, const float * d_state_in, float * d_out, void * stream) {
    if (!ctx || !d_x || !d_out) return Z2H_EINVAL;
    if (!ctx->finalized) return seterr(ctx, Z2H_ESTATE, "z2h_finalize not called");
    if (layer < 0 || layer >= ctx->hp.n_layer || !ctx->m->layers[layer].moe) return seterr(ctx, Z2H_EINVAL, "layer is not MoE");
    if (T <= 0 || T > ctx->Tmax || (ctx->capture && T > ctx->Tstep)) return seterr(ctx, Z2H_EINVAL, "n_tokens out of range");
    hipStream_t keep = ctx->stream;
    if (stream) ctx->stream = (hipStream_t) stream;
    ctx->cap_T = T;
    Layer & ly = ctx->m->layers[layer];
    int rc;
    HIPX(hipMemcpyAsync(ctx->cur, d_x, (size_t) T * ctx->hp.n_embd * 4, hipMemcpyDeviceToDevice, ctx->stream));
    ResNormArgs e{};
    e.mode = RN_ENCODE; e.src = ctx->cur; e.act = ctx->act; e.act_fmt = act_of(ly.up_exps.type);
    if ((rc = launch_resnorm(ctx, T, e))) { ctx->stream = keep; return rc; }
    if ((rc = expert_block(ctx, ly, layer, T, d_state_in))) { ctx->stream = keep; return rc; }
    ResNormArgs n{};
    n.mode = RN_ACCUM; n.src = ctx->eo; n.k = ly.k; n.res = nullptr; n.cap_x = d_out; n.act_fmt = ACT_NONE;
    rc = launch_resnorm(ctx, T, n);
    if (!rc) rc = cap_copy(ctx, Z2H_CAP_FFN_OUT, layer, d_out, T);
    ctx->stream = keep;
    return rc;
}

int z2h_moe_forward(z2h_ctx * ctx, int layer, int T, const float * x, const float * state_in, float * out) {
    if (!ctx || !x || !out) return Z2H_EINVAL;
    if (!ctx->finalized) return seterr(ctx, Z2H_ESTATE, "z2h_finalize not called");
    if (T <= 0 || T > ctx->Tmax) return seterr(ctx, Z2H_EINVAL, "n_tokens out of range");
    HIPX(hipSetDevice(ctx->device));
    HIPX(hipMemcpyAsync(ctx->tmp_x, x, (size_t) T * ctx->hp.n_embd * 4, hipMemcpyHostToDevice, ctx->stream));
    if (state_in) HIPX(hipMemcpyAsync(ctx->state_ext, state_in, (size_t) T * ctx->rd * 4, hipMemcpyHostToDevice, ctx->stream));
    if (int rc = z2h_moe_forward_device(ctx, layer, T, ctx->tmp_x, state_in ? ctx->state_ext : nullptr, ctx->wo_out, nullptr)) return rc;
    HIPX(hipMemcpyAsync(out, ctx->wo_out, (size_t) T * ctx->hp.n_embd * 4, hipMemcpyDeviceToHost, ctx->stream));
    HIPX(hipStreamSynchronize(ctx->stream));
    return Z2H_OK;
}

int z2h_model_moe_forward_noalloc(z2h_model * mdl, int layer, int T, const float * d_x, const float * d_state_in,
                                  float * d_state_out, float * d_out, void * stream) {
    if (!mdl || !d_x || !d_out) return mdl ? seterr(mdl, Z2H_EINVAL, "null argument") : Z2H_EINVAL;
    if (!mdl->finalized) return seterr(mdl, Z2H_ESTATE, "model not finalized");
    const auto & hp = mdl->hp;
    if (layer < 0 || layer >= hp.n_layer || !mdl->layers[layer].moe) return seterr(mdl, Z2H_EINVAL, "layer is not MoE");
    Layer & ly = mdl->layers[layer];
    if (T <= 0 || T * ly.k > LIST_MAX) return seterr(mdl, Z2H_EINVAL, "n_tokens out of range (1 .. 1024 / top-k)");
    // the buffers z2h_moe_forward_device takes from a context, carved 256-byte aligned from `scratch`
    const int d = hp.n_embd, ff = hp.n_ff, K = ly.k, E = std::max(1, ly.E), rd = std::max(1, mdl->rd);
    const int Kd = kpad(d), Kf = kpad(std::max(ff, 1)), R = T * K;
    struct Piece { void ** at; size_t bytes; };
    z2h_ctx c;
    std::vector<Piece> plan;                          // (host vector: no device allocation)
    plan.reserve(20);
    auto want = [&](auto ** p, size_t n) { plan.push_back({(void **) p, n}); };
    want(&c.act.q, (size_t) T * Kd); want(&c.act.d32, (size_t) T * (Kd / 32) * 4); want(&c.act.d256, (size_t) T * (Kd / 256) * 4);
    want(&c.act.bs, (size_t) T * (Kd / 16) * 2); want(&c.act.h, (size_t) T * Kd * 2);
    want(&c.act_y.q, (size_t) R * Kf); want(&c.act_y.d32, (size_t) R * (Kf / 32) * 4); want(&c.act_y.d256, (size_t) R * (Kf / 256) * 4);
    want(&c.act_y.bs, (size_t) R * (Kf / 16) * 2); want(&c.act_y.h, (size_t) R * Kf * 2);
    want(&c.sel, (size_t) R * 4); want(&c.wsel, (size_t) R * 4);
    want(&c.r_off, (size_t) (E + 1) * 4); want(&c.r_perm, (size_t) R * 4);
    want(&c.gu_g, (size_t) R * ff * 4); want(&c.gu_u, (size_t) R * ff * 4); want(&c.eo, (size_t) R * d * 4);
    if (!d_state_out) want(&c.state_one, (size_t) T * rd * 4);
    size_t total = 0;
    for (const Piece & pc : plan) total += (pc.bytes + 255) & ~(size_t) 255;
    if (total > NOALLOC_SCRATCH_BYTES)
        return seterr(mdl, Z2H_EINVAL, "z2h_model_moe_forward_noalloc: " + std::to_string(T) + " tokens need " + std::to_string(total) +
                                       " bytes of scratch; the static scratch holds " + std::to_string(NOALLOC_SCRATCH_BYTES));
    void * base = nullptr;
    int n_cu = 0;
    std::string err;
    if (int rc = scratch_address(mdl->device, &base, &n_cu, err)) return seterr(mdl, rc, err);
    DeviceScope on(mdl->device);                      // the caller's current device comes back on return
    if (!on.ok) return seterr(mdl, Z2H_EDEVICE, "hipSetDevice failed");
    size_t off = 0;
    for (const Piece & pc : plan) { *pc.at = (uint8_t *) base + off; off += (pc.bytes + 255) & ~(size_t) 255; }
    if (d_state_out) c.state_one = d_state_out;
    c.m = mdl; c.hp = hp; c.device = mdl->device; c.stream = (hipStream_t) stream; c.n_cu = n_cu;
    c.W = mdl->W; c.rd = mdl->rd; c.kmax = mdl->kmax; c.Tmax = c.Tstep = T; c.finalized = true;
    c.cur = const_cast<float *>(d_x);                 // read only: the router input and the encoder's source
    // the kernels of z2h_moe_forward_device: encode, router + grouped experts, k-sum (no memset, no copy)
    int rc;
    ResNormArgs e{};
    e.mode = RN_ENCODE; e.src = c.cur; e.act = c.act; e.act_fmt = act_of(ly.up_exps.type);
    if (!(rc = launch_resnorm(&c, T, e)) && !(rc = expert_block(&c, ly, layer, T, d_state_in))) {
        ResNormArgs n{};
        n.mode = RN_ACCUM; n.src = c.eo; n.k = ly.k; n.res = nullptr; n.cap_x = d_out; n.act_fmt = ACT_NONE;
        rc = launch_resnorm(&c, T, n);
    }
    if (rc) return seterr(mdl, rc, c.err);
    return Z2H_OK;
}

int z2h_model_set_expert_mask(z2h_model * mdl, int layer, const uint8_t * keep) {
    if (!mdl) return Z2H_EINVAL;
    if (layer < 0 || layer >= mdl->hp.n_layer || !mdl->layers[layer].up_exps.ok()) return seterr(mdl, Z2H_EINVAL, "layer is not MoE");
    if (hipSetDevice(mdl->device) != hipSuccess) return Z2H_EDEVICE;
    Layer & ly = mdl->layers[layer];
    ++mdl->gen;                                      // captured graphs bake the mask pointer in
    if (!keep) { ly.mask = nullptr; return Z2H_OK; }
    std::vector<float> m(ly.E);
    for (int e = 0; e < ly.E; ++e) m[e] = keep[e] ? 0.0f : -INFINITY;
    if (!ly.mask_buf) if (int rc = dalloc(mdl, &ly.mask_buf, (size_t) ly.E * 4, mdl->bytes_w)) return rc;
    HIPM(hipMemcpy(ly.mask_buf, m.data(), m.size() * 4, hipMemcpyHostToDevice));
    ly.mask = ly.mask_buf;
    return Z2H_OK;
}

int z2h_model_set_logit_bias(z2h_model * mdl, int layer, const float * bias) {
    if (!mdl) return Z2H_EINVAL;
    if (layer < 0 || layer >= mdl->hp.n_layer || !mdl->layers[layer].up_exps.ok()) return seterr(mdl, Z2H_EINVAL, "layer is not MoE");
    if (hipSetDevice(mdl->device) != hipSuccess) return Z2H_EDEVICE;
    Layer & ly = mdl->layers[layer];
    ++mdl->gen;
    if (!bias) { ly.logit_bias = nullptr; return Z2H_OK; }
    if (!ly.bias_buf) if (int rc = dalloc(mdl, &ly.bias_buf, (size_t) ly.E * 4, mdl->bytes_w)) return rc;
    HIPM(hipMemcpy(ly.bias_buf, bias, (size_t) ly.E * 4, hipMemcpyHostToDevice));
    ly.logit_bias = ly.bias_buf;
    return Z2H_OK;
}

int z2h_model_set_layer_skip(z2h_model * mdl, const uint8_t * skip) {
    if (!mdl) return Z2H_EINVAL;
    std::vector<uint8_t> v;
    if (skip) for (int L = 0; L < mdl->hp.n_layer; ++L) v.push_back(skip[L] ? 1 : 0);
    if (std::find(v.begin(), v.end(), 1) == v.end()) v.clear();
    if (v != mdl->layer_skip) { mdl->layer_skip = v; ++mdl->gen; }   // captured graphs bake the block list in
    return Z2H_OK;
}

int z2h_set_layer_skip(z2h_ctx * ctx, const uint8_t * skip) {
    if (!ctx) return Z2H_EINVAL;
    if (ctx->stream) (void) hipStreamSynchronize(ctx->stream);
    return z2h_model_set_layer_skip(ctx->m, skip);
}

int z2h_set_expert_mask(z2h_ctx * ctx, int layer, const uint8_t * keep) {
    if (!ctx) return Z2H_EINVAL;
    if (ctx->stream) (void) hipStreamSynchronize(ctx->stream);
    const int rc = z2h_model_set_expert_mask(ctx->m, layer, keep);
    if (rc) ctx->err = ctx->m->err;
    return rc;
}

int z2h_set_logit_bias(z2h_ctx * ctx, int layer, const float * bias) {
    if (!ctx) return Z2H_EINVAL;
    if (ctx->stream) (void) hipStreamSynchronize(ctx->stream);
    const int rc = z2h_model_set_logit_bias(ctx->m, layer, bias);
    if (rc) ctx->err = ctx->m->err;
    return rc;
}

int z2h_set_capture(z2h_ctx * ctx, int enable) {
    if (!ctx) return Z2H_EINVAL;
    if (!ctx->finalized) return seterr(ctx, Z2H_ESTATE, "z2h_finalize not called");
    if (enable && ctx->cap.empty()) {
        ctx->cap.assign(Z2H_CAP_COUNT_, nullptr);
        for (int w = 0; w < Z2H_CAP_COUNT_; ++w) {
            const size_t n = (size_t) cap_width(ctx, w, ctx->Tstep) * 4 * ctx->hp.n_layer;
            if (int rc = dalloc(ctx, &ctx->cap[w], n, ctx->bytes_scratch)) return rc;
            HIPX(hipMemset(ctx->cap[w], 0, n));
        }
    }
    ctx->capture = enable != 0;
    return Z2H_OK;
}

int64_t z2h_capture_bytes(z2h_ctx * ctx, int what, int n_tokens) {
    if (!ctx || what < 0 || what >= Z2H_CAP_COUNT_) return -1;
    return cap_width(ctx, what, n_tokens) * 4;
}

int z2h_read_capture(z2h_ctx * ctx, int layer, int what, void * host, size_t nbytes) {
    if (!ctx || !host) return Z2H_EINVAL;
    if (ctx->cap.empty()) return seterr(ctx, Z2H_ESTATE, "capture was never enabled");
    if (what < 0 || what >= Z2H_CAP_COUNT_ || layer < 0 || layer >= ctx->hp.n_layer) return seterr(ctx, Z2H_EINVAL, "bad capture id");
    const size_t n = (size_t) cap_width(ctx, what, ctx->cap_T) * 4;
    if (nbytes < n) return seterr(ctx, Z2H_EINVAL, "capture buffer too small");
    HIPX(hipStreamSynchronize(ctx->stream));
    const int L = what == Z2H_CAP_OUT_NORM ? 0 : layer;
    HIPX(hipMemcpy(host, ctx->cap[what] + (size_t) L * cap_width(ctx, what, ctx->Tstep) * 4, n, hipMemcpyDeviceToHost));
    return Z2H_OK;
}

int z2h_set_graphs(z2h_ctx * ctx, int enable) {
    if (!ctx) return Z2H_EINVAL;
    ctx->use_graphs = enable != 0;
    return Z2H_OK;
}

int z2h_profile_begin(z2h_ctx * ctx) {
    if (!ctx) return Z2H_EINVAL;
    if (ctx->ev.empty()) {
        ctx->ev.resize(2 * PROF_MAX);
        ctx->ev_fam.resize(PROF_MAX);
        for (auto & e : ctx->ev) HIPX(hipEventCreate(&e));
    }
    HIPX(hipStreamSynchronize(ctx->stream));
    ctx->ev_used = 0;
    ctx->prof = true;
    return Z2H_OK;
}

int z2h_profile_end(z2h_ctx * ctx, double * ms, int32_t * launches) {
    if (!ctx || !ms || !launches) return Z2H_EINVAL;
    if (!ctx->prof) return seterr(ctx, Z2H_ESTATE, "profile window not open");
    ctx->prof = false;
    // launches may have gone to a caller's stream (z2h_step_device): wait on the events themselves
    for (int f = 0; f < Z2H_KF_COUNT_; ++f) { ms[f] = 0.0; launches[f] = 0; }
    for (int i = 0; i < ctx->ev_used; ++i) {
        float t = 0.0f;
        HIPX(hipEventSynchronize(ctx->ev[2 * i + 1]));
        HIPX(hipEventElapsedTime(&t, ctx->ev[2 * i], ctx->ev[2 * i + 1]));
        ms[ctx->ev_fam[i]] += t;
        launches[ctx->ev_fam[i]] += 1;
    }
    if (ctx->ev_used >= PROF_MAX) return seterr(ctx, Z2H_EINVAL, "profile window overflowed");
    return Z2H_OK;
}

int64_t z2h_device_bytes(const z2h_ctx * ctx, int what) {
    if (!ctx) return -1;
    return what == 0 ? ctx->m->bytes_w : what == 1 ? ctx->bytes_kv : ctx->bytes_scratch;
}

const char * z2h_last_error(const z2h_ctx * ctx) { return ctx ? ctx->err.c_str() : "null context"; }

static int sample_impl(z2h_ctx * ctx, int n_active, const float * d_logits, const z2h_sampling * sp, const int32_t * hist,
                       const int32_t * hist_len, int hist_cap, const double * u, int32_t * codes, bool feed) {
    static_assert(sizeof(z2h_sampling) == sizeof(SampleParams), "z2h_sampling layout");
    if (!ctx || !sp || !u || !codes) return ctx ? seterr(ctx, Z2H_EINVAL, "null argument") : Z2H_EINVAL;
    if (!ctx->finalized) return seterr(ctx, Z2H_ESTATE, "z2h_finalize not called");
    if (n_active <= 0 || n_active > ctx->Tstep) return seterr(ctx, Z2H_EINVAL, "n_active out of range");
    if (hist && (hist_cap < 0 || hist_cap > Z2H_SAMPLE_HIST_MAX || !hist_len))
        return seterr(ctx, Z2H_EINVAL, "history capacity out of range (at most Z2H_SAMPLE_HIST_MAX)");
    const int ncb = ctx->hp.n_codebooks, av = ctx->hp.audio_vocab;
    int np2 = 1;
    while (np2 < av) np2 <<= 1;
    if (ncb <= 0 || av <= 0 || np2 > 4096) return seterr(ctx, Z2H_ENOTSUP, "audio vocabulary too large for the sampler");
    const int hc = hist ? hist_cap : 0;
    for (int i = 0; i < n_active * ncb; ++i)
        if (hist && (hist_len[i] < 0 || hist_len[i] > hc)) return seterr(ctx, Z2H_EINVAL, "history length out of range");
    HIPX(hipSetDevice(ctx->device));
    // stage the inputs in pinned memory, then one copy each
    uint8_t * h = ctx->h_samp;
    SampleParams * hsp = (SampleParams *) h;
    int32_t * hh = (int32_t *) (hsp + n_active);
    int32_t * hl = hh + (size_t) n_active * ncb * std::max(hc, 1);
    double * hu = (double *) (((uintptr_t) (hl + (size_t) n_active * ncb) + 7) & ~(uintptr_t) 7);
    std::memcpy(hsp, sp, (size_t) n_active * sizeof(SampleParams));
    if (hc) std::memcpy(hh, hist, (size_t) n_active * ncb * hc * 4);
    if (hist) std::memcpy(hl, hist_len, (size_t) n_active * ncb * 4);
    else std::memset(hl, 0, (size_t) n_active * ncb * 4);
    std::memcpy(hu, u, (size_t) n_active * ncb * 8);
    HIPX(hipMemcpyAsync(ctx->d_sp, hsp, (size_t) n_active * sizeof(SampleParams), hipMemcpyHostToDevice, ctx->stream));
    if (hc) HIPX(hipMemcpyAsync(ctx->d_hist, hh, (size_t) n_active * ncb * hc * 4, hipMemcpyHostToDevice, ctx->stream));
    HIPX(hipMemcpyAsync(ctx->d_hlen, hl, (size_t) n_active * ncb * 4, hipMemcpyHostToDevice, ctx->stream));
    HIPX(hipMemcpyAsync(ctx->d_u, hu, (size_t) n_active * ncb * 8, hipMemcpyHostToDevice, ctx->stream));
    SampleArgs a{};
    a.logits = d_logits ? d_logits : ctx->logits;
    a.ncb = ncb; a.av = av; a.np2 = np2;
    a.sp = ctx->d_sp; a.hist = ctx->d_hist; a.hlen = ctx->d_hlen; a.hcap = std::max(hc, 1);
    a.u = ctx->d_u; a.codes = ctx->d_codes;
    KL(k_sample, dim3(ncb, n_active), dim3(256), sample_lds_bytes(av, np2), ctx->stream, a);
    HIPX(hipGetLastError());
    ctx->resident_T = 0;
    if (feed) {
        ctx->resident_last = 0;                      // the tables now hold the next step's inputs
        KL(k_feed, dim3(n_active), dim3(64), 0, ctx->stream, ctx->d_codes, ncb, ctx->W, (int) ctx->hp.text_vocab,
           ctx->d_ids, ctx->d_npast);
        HIPX(hipGetLastError());
    }
    int32_t * hc_out = (int32_t *) (hu + (size_t) n_active * ncb);
    HIPX(hipMemcpyAsync(hc_out, ctx->d_codes, (size_t) n_active * ncb * 4, hipMemcpyDeviceToHost, ctx->stream));
    HIPX(hipStreamSynchronize(ctx->stream));
    std::memcpy(codes, hc_out, (size_t) n_active * ncb * 4);
    if (feed) {
        ctx->resident_T = n_active;
        for (int i = 0; i < n_active; ++i) ctx->last_np[i] += 1;     // what k_feed wrote
    }
    return Z2H_OK;
}

int z2h_sample(z2h_ctx * ctx, int n_active, const float * d_logits, const z2h_sampling * sp, const int32_t * hist,
               const int32_t * hist_len, int hist_cap, const double * u, int32_t * codes) {
    return sample_impl(ctx, n_active, d_logits, sp, hist, hist_len, hist_cap, u, codes, false);
}

int z2h_sample_feed(z2h_ctx * ctx, int n_active, const z2h_sampling * sp, const int32_t * hist, const int32_t * hist_len,
                    int hist_cap, const double * u, int32_t * codes) {
    if (ctx && (ctx->resident_last != n_active || (int) ctx->last_np.size() != n_active))
        return seterr(ctx, Z2H_ESTATE, "z2h_sample_feed: the last step had another width or no device tables");
    return sample_impl(ctx, n_active, nullptr, sp, hist, hist_len, hist_cap, u, codes, true);
}

int z2h_step_resident(z2h_ctx * ctx, int n_active) {
    if (!ctx) return Z2H_EINVAL;
    if (!ctx->finalized) return seterr(ctx, Z2H_ESTATE, "z2h_finalize not called");
    if (n_active <= 0 || n_active != ctx->resident_T)
        return seterr(ctx, Z2H_ESTATE, "z2h_step_resident: no fed device tables of this width (z2h_sample_feed)");
    // the fed rows must fit the slots' bands, as z2h_step checks (a full slot refuses the step before
    // any launch; the device tables keep the refused n_past, so only a new z2h_step resumes)
    for (int i = 0; i < n_active; ++i)
        if ((int) ctx->last_np.size() != n_active || ctx->last_np[i] < 0 || ctx->last_np[i] >= ctx->S) {
            ctx->resident_T = 0;
            return seterr(ctx, Z2H_EINVAL, "z2h_step_resident: n_past out of range (slot full)");
        }
    HIPX(hipSetDevice(ctx->device));
    ctx->resident_T = 0;
    if (int rc = step_internal(ctx, n_active, nullptr, true)) return rc;
    ctx->resident_last = n_active;
    return Z2H_OK;
}

void z2h_destroy(z2h_ctx * ctx) {
    if (!ctx) return;
    (void) hipSetDevice(ctx->device);
    if (ctx->stream) (void) hipStreamSynchronize(ctx->stream);
    for (auto & g : ctx->graphs) (void) hipGraphExecDestroy(g.second);
    for (auto & e : ctx->ev) (void) hipEventDestroy(e);
    for (void * p : ctx->allocs) (void) hipFree(p);
    if (ctx->h_pin) (void) hipHostFree(ctx->h_pin);
    if (ctx->h_tiles) (void) hipHostFree(ctx->h_tiles);
    if (ctx->h_samp) (void) hipHostFree(ctx->h_samp);
    if (ctx->stream) (void) hipStreamDestroy(ctx->stream);
    z2h_model * mdl = ctx->m;
    delete ctx;
    z2h_model_release(mdl);
}

} // extern "C"
