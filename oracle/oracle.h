// oracle.h — CPU restatement of the reference's ggml CPU decode path (TEST INFRASTRUCTURE ONLY).
//
// This library is the parity checker and the timed CPU baseline. Only tests/, the smoke check and
// bench.py's cpu_baseline leg may load it; the product never links or calls it.
//
// It restates, op for op, what src/zonos2-graph.cpp composes from ggml ops for one continuous-
// batching decode step (build_graph 242-366, build_attention 101-176, build_moe 191-239,
// build_dense_ffn 179-185, zonos2_batch_step 762-837) and for the per-slot prefill
// (zonos2_batch_slot_prefill 703-760, manual causal attention 155-169). ggml itself is not
// available, so ggml's op semantics are restated from its public definitions (see oracle.cpp for
// the per-function notes, including which parts are "parity unpinned").
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct orc_hparams {
    int32_t n_layer, n_embd, head_dim, n_head, n_head_kv, n_ff, n_expert, n_ctx_train;
    float   rope_freq_base, rms_eps, qk_norm_eps, logit_softcap;
    int32_t n_codebooks, codebook_size, audio_vocab, eoa_id, audio_pad_id, text_vocab;
    int32_t spk_dim, spk_lda_dim;
    int32_t router_dim;            // router_down.ne1 (0 if the model has no MoE layer)
    const int32_t * expert_used;   // [n_layer]; 0 = dense FFN, else MoE top-k
} orc_hparams;

// Activation encodings a weight type is dotted against (ggml "vec_dot_type").
enum { ORC_ACT_F32 = 0, ORC_ACT_F16 = 1, ORC_ACT_Q8_0 = 8, ORC_ACT_Q8_K = 15 };

typedef struct orc_model orc_model;
typedef struct orc_kv    orc_kv;

// Per-layer capture arrays (any may be NULL). Layer-major, strides use T = tokens of the call,
// K = max top-k over layers, E = n_expert, rd = router_dim.
typedef struct orc_capture {
    float   * res_in;        // [L][T][d]    residual stream entering layer L
    float   * attn_in;       // [L][T][d]    rms_w(res, attn_norm)
    float   * q;             // [L][T][nh*hd]  after QK-norm, |temp| and RoPE (fp32)
    float   * k;             // [L][T][nkv*hd] after QK-norm and RoPE (fp32, before f16 store)
    float   * v;             // [L][T][nkv*hd]
    float   * gate;          // [L][T][nh]   sigmoid(W_g x)
    float   * attn_o;        // [L][T][nh*hd] gated attention output (input of W_o)
    float   * attn_out;      // [L][T][d]    W_o output
    float   * ffn_in;        // [L][T][d]    rms_w(layer_res, ffn_norm)
    float   * router_state;  // [L][T][rd]
    float   * router_logits; // [L][T][E]
    float   * probs;         // [L][T][E]
    int32_t * sel;           // [L][T][K]
    float   * weights;       // [L][T][K]
    float   * ffn_out;       // [L][T][d]
    float   * out_norm;      // [T][d]
} orc_capture;

int  orc_set_threads(int n);

orc_model * orc_model_create(const orc_hparams * hp);
// Borrow `data` (caller keeps it alive). ne[] is ggml order (ne0 fastest), unused dims = 1.
int  orc_model_set(orc_model * m, const char * name, int type, const int64_t ne[4], const void * data);
int  orc_model_finalize(orc_model * m);
// Harness-only additive pre-softmax router-logit bias for layer L (NULL clears). Not a reference
// input; used to impose a skewed expert popularity.
int  orc_model_set_logit_bias(orc_model * m, int layer, const float * bias);
// Runtime expert mask of layer L (zonos2_set_expert_mask, src/zonos2.cpp:203-239): keep[e] == 0 adds
// -inf to expert e's router logit before the softmax and to its selection score (graph.cpp:212, 218);
// NULL clears.
int  orc_model_set_expert_mask(orc_model * m, int layer, const uint8_t * keep);
// Depth prune (zonos2_model::layer_skip, src/zonos2.h:116-121; graph.cpp:334-341): skip[L] != 0
// bypasses block L (the residual passes through unchanged); NULL clears. skip has n_layer entries.
int  orc_model_set_layer_skip(orc_model * m, const uint8_t * skip);
void orc_model_free(orc_model * m);
const char * orc_last_error(void);

orc_kv * orc_kv_create(const orc_model * m, int n_slots, int slot_cap_frames);
int  orc_kv_slot_cap(const orc_kv * kv);
// rows [row0, row0+n) of `slot` in layer L; host layout [n][n_head_kv][head_dim] f16 bits.
int  orc_kv_write(orc_kv * kv, int layer, int slot, int row0, int n, const uint16_t * k, const uint16_t * v);
int  orc_kv_read(const orc_kv * kv, int layer, int slot, int row0, int n, uint16_t * k, uint16_t * v);
void orc_kv_free(orc_kv * kv);

// One decode step over T active columns (one new row each). ids: [T][n_codebooks+1] or NULL when
// emb ([T][d], injected in place of the summed embedding, before emb_norm) is given.
int orc_step(orc_model * m, orc_kv * kv, int T, const int32_t * slot_idx, const int32_t * n_past,
             const int32_t * ids, const float * emb, float * logits, orc_capture * cap);

// Per-slot prefill of n0 prompt rows (ids [n0][W]); writes K/V rows [0,n0) of `slot` and the
// last row's logits. spk (optional [spk_dim]) replaces row spk_pos's embedding by
// spk_proj(spk_lda(spk)) (+ delta [d] if given).
// Rows from any slots in one pass (several rows of a slot at distinct n_past attend to each other
// causally: every row's K/V is appended before the attention); emb_map [T] (or NULL): -1 = the row
// sums its ids, e >= 0 = the row takes emb[e]. logits [T][ncb*av].
int orc_step_mixed(orc_model * m, orc_kv * kv, int T, const int32_t * slot_idx, const int32_t * n_past,
                   const int32_t * ids, const int32_t * emb_map, const float * emb, float * logits);
int orc_prefill(orc_model * m, orc_kv * kv, int slot, const int32_t * ids, int n0,
                const float * spk, int spk_pos, const float * delta, float * last_logits);

// ---- layer-local entry points (teacher forcing: the caller supplies the layer input) ----
int orc_router(orc_model * m, int layer, int T, const float * ffn_in, const float * state_in,
               float * rh, float * logits, float * probs, int32_t * sel, float * w);
int orc_group(int T, int k, int E, const int32_t * sel, int32_t * counts, int32_t * offsets, int32_t * perm);
// One frame code for one (column, codebook): the reference sampler's steps (src/zonos2-sampler.cpp:16-77)
// with the uniform draw given as the canonical double u (r = u * kept mass). exp_mode 0: the terms are
// std::exp(float) as in the reference; 1: exp in double (orc_exp_d) rounded to float.
int orc_sample(const float * logits, int vocab, float temperature, int top_k, float top_p, float min_p,
               float rep_penalty, int rep_codebooks, int greedy, int cb, const int32_t * hist, int hist_len,
               double u, int exp_mode);
double orc_exp_d(double x);
int orc_experts(orc_model * m, int layer, int T, const float * ffn_in, const int32_t * sel,
                const float * w, float * expert_out, float * out);
int orc_dense_ffn(orc_model * m, int layer, int T, const float * ffn_in, float * out);
int orc_attention(orc_model * m, orc_kv * kv, int layer, int T, const int32_t * slot_idx,
                  const int32_t * n_past, const float * attn_in, float * attn_o, float * attn_out);

// ---- primitives (for known-answer tests) ----
int   orc_dequant(int type, const void * src, float * dst, int64_t n);
int   orc_matmul(int type, const void * w, int64_t n_in, int64_t n_out, int T, const float * x, float * y);
int   orc_quant_act(int act, const float * x, int64_t n, int8_t * q, float * d, int16_t * bsum, uint16_t * h);
float orc_expf(float x);
void  orc_sincos(float x, float * s, float * c);   // RoPE angle sin / cos (z_sincos)
float orc_softcap(float x, float cap);             // cap * tanh(x / cap) (z_softcap)
float orc_erff(float x);
float orc_gelu_erf(float x);
float orc_silu(float x);
int   orc_rope(float * x, int n_heads, int hd, int pos, float base);
uint16_t orc_f32_to_f16(float x);
float    orc_f16_to_f32(uint16_t h);

#ifdef __cplusplus
}
#endif
