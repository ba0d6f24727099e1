/* z2h.h — C ABI of libzonos2_hip.so, the MI355X (gfx950) ragged continuous-batching decode step of
 * the ZONOS2 MoE backbone.
 *
 * Every entry point is extern "C", takes plain pointers and sizes, and returns an int status
 * (Z2H_OK == 0). The per-context message of the last failure is available from z2h_last_error().
 * No C++ exception crosses this boundary. A context is not reentrant: one thread drives it, as in
 * the reference (src/server.cpp:905-911, docs/INTERNALS.md:200).
 *
 * Weights live in a reference-counted z2h_model (the reference's zonos2_model, loaded once); each
 * z2h_ctx (the reference's zonos2_batch_ctx: KV cache, scratch, step graphs) holds one reference, so
 * several batch contexts can share one model. z2h_create is the one-call form: model and context.
 *
 * Reference interfaces replaced (file:line in Zyphra/zonos2.cpp):
 *   z2h_model_create      zonos2_model_load hparams    src/zonos2.cpp:15-97, src/zonos2.h:124
 *   z2h_model_upload_tensor zonos2_model_load tensors  src/zonos2.cpp:100-119, name map 137-183
 *   z2h_model_finalize    zonos2_model_load field map  src/zonos2.cpp:126-185
 *   z2h_model_release     zonos2_model_free            src/zonos2.h:125, src/zonos2.cpp:188-195
 *   z2h_create_batch      zonos2_batch_init            src/zonos2-graph.cpp:639-690 (KV alloc, S rounding)
 *   z2h_create            zonos2_model_load + zonos2_batch_init in one call
 *   z2h_upload_tensor     as z2h_model_upload_tensor on the context's model
 *   z2h_finalize          as z2h_model_finalize, then the context's scratch
 *   z2h_step              zonos2_batch_step            src/zonos2-graph.cpp:762-837 (+ slot_logits 839-841)
 *   z2h_prefill           zonos2_batch_slot_prefill    src/zonos2-graph.cpp:703-760
 *   z2h_speaker_embed     the speaker column of build_graph, src/zonos2-graph.cpp:262-297
 *   z2h_moe_forward       build_moe                    src/zonos2-graph.cpp:191-239 (one MoE layer)
 *   z2h_set_expert_mask   zonos2_set_expert_mask       src/zonos2.cpp:203-239, src/zonos2.h:136
 *   z2h_destroy           zonos2_batch_free            src/zonos2-graph.cpp:692-701 (+ drops the model reference)
 */
#ifndef Z2H_H
#define Z2H_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    Z2H_OK = 0,
    Z2H_EINVAL = 1,     /* bad argument (shape, range, missing tensor) */
    Z2H_ENOMEM = 2,     /* device or host allocation failed */
    Z2H_EDEVICE = 3,    /* HIP runtime error */
    Z2H_ESTATE = 4,     /* call not valid in the context's current state */
    Z2H_ENOTSUP = 5     /* unsupported tensor type / layout */
};

/* GGUF tensor type ids accepted by z2h_upload_tensor */
enum { Z2H_F32 = 0, Z2H_F16 = 1, Z2H_Q8_0 = 8, Z2H_Q4_K = 12, Z2H_Q6_K = 14 };

/* Mirrors zonos2_hparams (src/zonos2.h:14-50); router_dim = router_down.ne1 (src/zonos2.cpp:241-246). */
typedef struct z2h_hparams {
    int32_t n_layer, n_embd, head_dim, n_head, n_head_kv, n_ff, n_expert, n_ctx_train;
    float   rope_freq_base, rms_eps, qk_norm_eps, logit_softcap;
    int32_t n_codebooks, codebook_size, audio_vocab, eoa_id, audio_pad_id, text_vocab;
    int32_t spk_dim, spk_lda_dim;
    int32_t router_dim;
    const int32_t * expert_used;   /* [n_layer]: 0 = dense FFN, else MoE top-k */
} z2h_hparams;

typedef struct z2h_model z2h_model;
typedef struct z2h_ctx z2h_ctx;

/* Weights only, on HIP device `device`; refcount 1. Upload every tensor, then finalize. */
int z2h_model_create(const z2h_hparams * hp, int device, z2h_model ** out);
/* Tensor hand-over as for z2h_upload_tensor below. */
int z2h_model_upload_tensor(z2h_model * m, const char * name, int type, const int64_t ne[4],
                            const void * data, size_t nbytes);
/* Checks that every tensor the forward pass needs is present; no uploads afterwards. */
int z2h_model_finalize(z2h_model * m);
/* Expert mask / router-logit bias (see z2h_set_expert_mask / z2h_set_logit_bias) on the model: every
 * context sharing it sees the change at its next step. No step may be in flight on any of them. */
int z2h_model_set_expert_mask(z2h_model * m, int layer, const uint8_t * keep);
int z2h_model_set_logit_bias(z2h_model * m, int layer, const float * bias);
/* Depth prune (zonos2_model::layer_skip, src/zonos2.h:116-121; src/zonos2-graph.cpp:334-341):
 * skip[L] != 0 bypasses block L in every following step and prefill (attention, KV append and FFN are
 * not run; the residual passes through unchanged; the router state threads past it). skip has
 * n_layer entries; NULL clears. */
int z2h_model_set_layer_skip(z2h_model * m, const uint8_t * skip);
const char * z2h_model_last_error(const z2h_model * m);
/* Drops one reference; the weights are freed with the last one (contexts hold one each). */
void z2h_model_release(z2h_model * m);

/* A batch context over a model (takes a reference; the model may be finalized before or after, through
 * z2h_finalize). n_slots decode slots of slot_cap_frames rows each (rounded up to a multiple of 256,
 * as the reference does); the KV cache is zero-filled. */
int z2h_create_batch(z2h_model * m, int n_slots, int slot_cap_frames, z2h_ctx ** out);
/* The same with room for max_rows rows per pass (z2h_step_mixed, z2h_moe_forward; at least n_slots
 * and Z2H_PREFILL_CHUNK_MAX); the step scratch grows with it (about 0.2 MB per row at d_model 2048,
 * plus attention partials for max_rows x slot_cap / 32 chunks). No reference counterpart. */
int z2h_create_batch_rows(z2h_model * m, int n_slots, int slot_cap_frames, int max_rows, z2h_ctx ** out);

/* A new model on HIP device `device` and a batch context over it (which then holds the model's only
 * reference) in one call. */
int z2h_create(const z2h_hparams * hp, int n_slots, int slot_cap_frames, int device, z2h_ctx ** out);

/* Hand over one GGUF tensor: name as in the reference GGUF, ggml ne order (ne0 fastest, unused = 1),
 * host bytes in GGUF block layout. The bytes are copied (repacked for the device) before return. */
int z2h_upload_tensor(z2h_ctx * ctx, const char * name, int type, const int64_t ne[4],
                      const void * data, size_t nbytes);

/* After all uploads: finalizes the context's model (if not yet) and allocates the step scratch. */
int z2h_finalize(z2h_ctx * ctx);

/* Slot rows per slot after rounding (the reference's slot_cap). */
int z2h_slot_cap(const z2h_ctx * ctx);

/* Write / read KV rows [row0, row0+n_rows) of `slot` in layer `layer`. Host layout
 * [n_rows][n_head_kv][head_dim] of f16 bits; either pointer may be NULL. */
int z2h_kv_write(z2h_ctx * ctx, int layer, int slot, int row0, int n_rows, const uint16_t * k, const uint16_t * v);
int z2h_kv_read(z2h_ctx * ctx, int layer, int slot, int row0, int n_rows, uint16_t * k, uint16_t * v);

/* One batched decode step over n_active columns. slot_idx[i] selects the KV band, n_past[i] is the
 * row the new K/V are written at (the row count already in the cache), ids is [n_active][n_codebooks+1]
 * (audio codes then the text id), or NULL when emb ([n_active][n_embd] fp32, injected in place of the
 * summed embedding before emb_norm) is given. out_logits receives [n_active][n_codebooks][audio_vocab]
 * post-softcap logits, or stays on the device only (out_logits NULL) for z2h_sample. Unlike the
 * reference, idle slots are simply not listed (no padded columns). */
int z2h_step(z2h_ctx * ctx, int n_active, const int32_t * slot_idx, const int32_t * n_past,
             const int32_t * ids, const float * emb, float * out_logits);

/* Same step with device-resident inputs/outputs, enqueued on `stream` (a hipStream_t, NULL = the
 * context's stream) without synchronizing. d_slot_idx/d_n_past: [n_active] int32; d_ids or d_emb as
 * above; d_logits [n_active][n_codebooks*audio_vocab]. h_n_past must hold the same n_past values on
 * the host (grid sizing for the ragged attention). */
int z2h_step_device(z2h_ctx * ctx, int n_active, const int32_t * d_slot_idx, const int32_t * d_n_past,
                    const int32_t * h_n_past, const int32_t * d_ids, const float * d_emb,
                    float * d_logits, void * stream);

/* Prefill n0 prompt rows into `slot` (rows [0, n0)), causal within the prompt as in the reference's
 * per-slot prefill: the rows attend each other's fp32 K/V (src/zonos2-graph.cpp:155-169) while their
 * f16 rows are written to the slot's cache for the decode steps; ids [n0][n_codebooks+1]. spk
 * (optional, [spk_dim]) replaces row spk_pos's embedding by spk_proj(spk_lda(spk)) (+ delta [n_embd]
 * if non-NULL). last_logits receives the final row's [n_codebooks][audio_vocab] logits. */
int z2h_prefill(z2h_ctx * ctx, int slot, const int32_t * ids, int n0, const float * spk, int spk_pos,
                const float * delta, float * last_logits);

/* The speaker rows of n speaker vectors (spk [n][spk_dim]; n <= Z2H_SPEAKER_MAX): spk_proj(spk_lda(spk)
 * + b_lda) + b_proj (+ delta [n][n_embd] if non-NULL), into out [n][n_embd] (host memory) - the
 * column the reference writes over a prompt row before emb_norm (src/zonos2-graph.cpp:262-297), for
 * callers that place speaker rows in a mixed pass themselves (emb_map / emb of z2h_step_mixed);
 * z2h_prefill computes its speaker row the same way. Synchronizes the context's stream. */
#define Z2H_SPEAKER_MAX 64
int z2h_speaker_embed(z2h_ctx * ctx, int n, const float * spk, const float * delta, float * out);

/* One pass over n_rows rows from any slots, decode columns and prefill-chunk rows mixed (the
 * reference has no mixed pass; it is its zonos2_batch_step and zonos2_batch_slot_prefill graphs in
 * one, src/zonos2-graph.cpp:703-837). Row t writes slot_idx[t]'s cache row n_past[t] and attends to
 * that slot's rows [0, n_past[t]], including rows of this pass: every row's K/V is appended before
 * the attention. No two rows may share (slot, n_past). ids [n_rows][n_codebooks+1]; emb_map (NULL, or
 * [n_rows]: -1 = the row sums its ids, e >= 0 = the row takes emb[e], e.g. a speaker prefix row) with
 * emb [n_emb][n_embd]. out_logits [n_out][n_codebooks][audio_vocab] receives the logits of rows
 * out_rows[0 .. n_out) (the output head runs on those rows only). n_rows and n_out are limited by
 * the context's row capacity (z2h_create_batch_rows). */
int z2h_step_mixed(z2h_ctx * ctx, int n_rows, const int32_t * slot_idx, const int32_t * n_past, const int32_t * ids,
                   const int32_t * emb_map, const float * emb, int n_emb, int n_out, const int32_t * out_rows, float * out_logits);

/* Rows per prefill chunk (1 .. the context's row capacity, max(n_slots, Z2H_PREFILL_CHUNK_MAX, max_rows);
 * default the capacity, so a prompt that fits is one pass and streams each layer's weights once).
 * A chunk's rows go through each layer together (the projections and expert matmuls see them as one
 * batch; every row appends its K/V before the chunk's attention), so a prompt of n0 rows takes
 * ceil(n0 / rows) passes instead of n0 single-row steps. Any chunk size gives the same results. No
 * reference counterpart: the reference builds one graph over the whole prompt. */
#define Z2H_PREFILL_CHUNK_MAX 256
int z2h_set_prefill_chunk(z2h_ctx * ctx, int rows);

/* One MoE layer (build_moe) on n_tokens host rows x [n_tokens][n_embd] (the layer's ffn_in); state_in
 * ([n_tokens][router_dim], may be NULL) is the previous MoE layer's router state. out [n_tokens][n_embd]. */
int z2h_moe_forward(z2h_ctx * ctx, int layer, int n_tokens, const float * x, const float * state_in, float * out);
/* Device-pointer variant, enqueued on `stream` without synchronizing. */
int z2h_moe_forward_device(z2h_ctx * ctx, int layer, int n_tokens, const float * d_x, const float * d_state_in,
                           float * d_out, void * stream);

/* One MoE layer (as z2h_moe_forward_device) on a model alone, allocating nothing: no context, and no
 * hipMalloc / hipFree or other allocating call. No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid it). Every intermediate buffer (activation encodings, routing, route lists, SwiGLU
 * rows, per-route outputs, the router state unless d_state_out is given) is carved from a static
 * device array of 16 MiB per GPU, held until the process ends; a call whose buffers would not fit
 * (n_tokens x top-k routes at the model's widths) is refused with Z2H_EINVAL before any launch, as
 * is n_tokens * top-k > 1024. Calls on one GPU share that array: calls that overlap on one GPU (two
 * streams, two threads) race and must be serialized by the caller. Enqueued on `stream` (NULL: the
 * null stream) without synchronizing. d_x [n_tokens][n_embd] (the layer's ffn_in), d_state_in
 * ([n_tokens][router_dim] or NULL), d_state_out (NULL, or [n_tokens][router_dim] receiving this
 * layer's router state), d_out [n_tokens][n_embd]. Results are bit-identical to z2h_moe_forward_device.
 * The caller's current HIP device is the same on return. Errors: z2h_model_last_error. */
int z2h_model_moe_forward_noalloc(z2h_model * m, int layer, int n_tokens, const float * d_x, const float * d_state_in,
                                  float * d_state_out, float * d_out, void * stream);

/* Runtime expert mask for one MoE layer: keep[e] != 0 keeps expert e routable (logits and selection
 * scores of the others get -inf); keep == NULL clears the layer's mask. */
int z2h_set_expert_mask(z2h_ctx * ctx, int layer, const uint8_t * keep);

/* Depth prune on the context's model (see z2h_model_set_layer_skip). */
int z2h_set_layer_skip(z2h_ctx * ctx, const uint8_t * skip);

/* Additive pre-softmax router-logit bias for one MoE layer ([n_expert] fp32, NULL clears). Not a
 * reference input: a benchmark hook to impose a skewed expert popularity. */
int z2h_set_logit_bias(z2h_ctx * ctx, int layer, const float * bias);

/* Frame sampling on the device, for callers that keep the logits in HBM. It follows the reference's
 * per-codebook sampler (src/zonos2-sampler.cpp:16-77, called per slot by zonos2_slot_sample,
 * src/zonos2-graph.cpp:843-870) with the random generator left on the host: column i, codebook cb
 * applies the repetition penalty over hist, temperature, top-k (logit descending), softmax (float
 * exp terms over a double sum), top-p, min-p and draws at u * kept mass along the candidates, with
 * equal logits and probabilities in the orders that the reference's std::partial_sort / std::sort
 * (GCC 11 libstdc++) give them. u[i][cb] is the canonical double in [0, 1) that the host sampler's
 * std::uniform_real_distribution would take from its mt19937 (std::generate_canonical<double, 53>);
 * it is not used where the kept mass is 0 (for finite logits: min_p > 1), where the host sampler
 * takes no draw.
 * The exp terms are exp(x) computed in double and rounded to float, so a draw can differ from the
 * host sampler's (glibc expf) only where the two roundings differ by an ulp and u falls between the
 * two cumulative sums.
 *   d_logits  [n_active][n_codebooks][audio_vocab] on the device, NULL = the last z2h_step's logits
 *   sp        [n_active] settings (greedy takes the first maximum of the raw logits)
 *   hist      [n_active][n_codebooks][hist_cap] recent codes, oldest first (NULL: no penalty);
 *             hist_len [n_active][n_codebooks] entries used; hist_cap <= Z2H_SAMPLE_HIST_MAX
 *   u         [n_active][n_codebooks];  codes out [n_active][n_codebooks] (host memory)
 * Synchronizes the context's stream. */
#define Z2H_SAMPLE_HIST_MAX 256
typedef struct z2h_sampling {
    float   temperature;
    int32_t top_k;            /* 0 or >= audio_vocab: every id is a candidate */
    float   top_p;            /* 0 disables */
    float   min_p;            /* 0 disables */
    float   rep_penalty;
    int32_t rep_codebooks;    /* codebooks cb < rep_codebooks get the penalty */
    int32_t greedy;
    int32_t reserved;
} z2h_sampling;
int z2h_sample(z2h_ctx * ctx, int n_active, const float * d_logits, const z2h_sampling * sp, const int32_t * hist,
               const int32_t * hist_len, int hist_cap, const double * u, int32_t * codes);

/* Device-resident step tables (no reference counterpart; the reference repacks ids, positions and its
 * mask on the host every step, src/zonos2-graph.cpp:773-813). z2h_sample_feed is z2h_sample on the
 * last step's logits (which must come from z2h_step, z2h_step_resident or the graph path of
 * z2h_step_device with ids) that also writes each column's next input frame (its codes + the text pad
 * id text_vocab) and n_past + 1 into the context's step tables; z2h_step_resident(ctx, n) then runs
 * the next step of the same n columns from those tables without any host upload, leaving the logits
 * on the device (enqueued, not synchronized). Any other step, prefill or sample clears the tables. */
int z2h_sample_feed(z2h_ctx * ctx, int n_active, const z2h_sampling * sp, const int32_t * hist, const int32_t * hist_len,
                    int hist_cap, const double * u, int32_t * codes);
int z2h_step_resident(z2h_ctx * ctx, int n_active);

/* Debug capture of per-layer intermediates of the following steps (off by default). */
enum {
    Z2H_CAP_RES_IN = 0, Z2H_CAP_ATTN_IN, Z2H_CAP_Q, Z2H_CAP_K, Z2H_CAP_V, Z2H_CAP_GATE, Z2H_CAP_ATTN_O,
    Z2H_CAP_ATTN_OUT, Z2H_CAP_FFN_IN, Z2H_CAP_ROUTER_STATE, Z2H_CAP_ROUTER_LOGITS, Z2H_CAP_PROBS,
    Z2H_CAP_SEL, Z2H_CAP_WEIGHTS, Z2H_CAP_FFN_OUT, Z2H_CAP_OUT_NORM, Z2H_CAP_COUNTS, Z2H_CAP_OFFSETS,
    Z2H_CAP_PERM, Z2H_CAP_EXPERT_OUT, Z2H_CAP_COUNT_
};
int z2h_set_capture(z2h_ctx * ctx, int enable);
/* Copy capture `what` of `layer` (ignored for OUT_NORM) from the last step / moe_forward into host.
 * Sizes: see z2h_capture_bytes. SEL and WEIGHTS hold the layer's [n_tokens][top_k of that layer]
 * rows at the start of a buffer sized for the model's largest top-k. */
int64_t z2h_capture_bytes(z2h_ctx * ctx, int what, int n_tokens);
int z2h_read_capture(z2h_ctx * ctx, int layer, int what, void * host, size_t nbytes);

/* Replay each step from a HIP graph captured once per (batch width, id/embedding input) pair
 * (default on; the counterpart of the reference's CUDA-graph replay of its decode-graph ladder,
 * CMakeLists.txt:34, src/zonos2-graph.cpp:670-680). Steps with capture or profiling run eagerly. */
int z2h_set_graphs(z2h_ctx * ctx, int enable);

/* Per-kernel-family timing with HIP events recorded around every launch on the context's stream
 * (the reference's only equivalent is the ZONOS2_PROFILE_STEP phase split, src/zonos2-graph.cpp:768,
 * 815-829). Between begin and end every launch is bracketed by an event pair; end synchronizes and
 * writes the summed milliseconds and launch counts per family. Up to 16384 launches per window. */
enum {
    Z2H_KF_RESNORM = 0, Z2H_KF_GEMV_QKV, Z2H_KF_QKV_POST, Z2H_KF_ATTN, Z2H_KF_ATTN_COMBINE, Z2H_KF_GEMV_WO,
    Z2H_KF_ROUTER_DOWN, Z2H_KF_ROUTER_TAIL, Z2H_KF_GEMV_GATEUP, Z2H_KF_GEMV_DOWN, Z2H_KF_GEMV_DENSE,
    Z2H_KF_GEMV_HEAD, Z2H_KF_SWIGLU, Z2H_KF_COUNT_
};
int z2h_profile_begin(z2h_ctx * ctx);
int z2h_profile_end(z2h_ctx * ctx, double * ms, int32_t * launches);

/* Device memory held by weights (the shared model), KV cache and scratch (bytes). */
int64_t z2h_device_bytes(const z2h_ctx * ctx, int what /* 0 weights, 1 kv, 2 scratch */);

/* Message of the context's last failure. */
const char * z2h_last_error(const z2h_ctx * ctx);
void z2h_destroy(z2h_ctx * ctx);

#ifdef __cplusplus
}
#endif
#endif /* Z2H_H */
