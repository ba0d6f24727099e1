// zonos2.h — the ZONOS2 continuous-batching decode API on the MI355X HIP library (include/z2h.h).
//
// Source-compatible with the batched-decode subset of the reference's src/zonos2.h: the same type
// and function names, argument meaning, ownership and bool/stderr error behaviour, so a caller of
// the reference (its server worker loop, --batch-test / --decode-bench) compiles against this
// header unchanged for these entry points. The ggml objects of the reference's structs are
// replaced by opaque device handles; nothing here includes ggml.
//
// Reference interfaces mirrored (file:line in Zyphra/zonos2.cpp):
//   zonos2_hparams              src/zonos2.h:14-50
//   zonos2_model (+ layer_skip) src/zonos2.h:89-121
//   zonos2_model_load / free    src/zonos2.h:124-125, src/zonos2.cpp:15-195
//   zonos2_router_dim           src/zonos2.h:128, src/zonos2.cpp:241-246
//   zonos2_set_expert_mask      src/zonos2.h:130-136, src/zonos2.cpp:203-239
//   zonos2_prompt_options       src/zonos2.h:178-188 (+ zonos2_build_prompt 190-194, defined by the reference's
//                               src/zonos2-prompt.cpp compiled against this header)
//   zonos2_backend_name         stands for ggml_backend_name(model.backend), src/server.cpp:1601
//   zonos2_sampling / sampler   src/zonos2.h:197-210, src/zonos2-sampler.h
//   zonos2_frame_cb             src/zonos2.h:212-215
//   zonos2_batch_ctx / slot     src/zonos2.h:217-274
//   zonos2_batch_init / free    src/zonos2.h:276-280, src/zonos2-graph.cpp:639-701
//   zonos2_batch_slot_prefill   src/zonos2.h:282-289, src/zonos2-graph.cpp:703-760
//   zonos2_batch_step           src/zonos2.h:291-294, src/zonos2-graph.cpp:762-837
//   zonos2_batch_slot_logits    src/zonos2.h:296-298, src/zonos2-graph.cpp:839-841
//   zonos2_slot_sample          src/zonos2.h:300-306, src/zonos2-graph.cpp:843-870
//   zonos2_generate             src/zonos2.h:308-325, src/zonos2-graph.cpp:515-605 (recompute), 877-981 (KV)
#pragma once

#include "z2h.h"

#include <cstdint>
#include <functional>
#include <map>
#include <string>
#include <vector>

struct zonos2_hparams {
    uint32_t n_layer      = 0;
    uint32_t n_embd       = 0;
    uint32_t head_dim     = 0;
    uint32_t n_head       = 0;
    uint32_t n_head_kv    = 0;
    uint32_t n_ff         = 0;
    uint32_t n_expert     = 0;
    uint32_t n_ctx_train  = 0;

    float rope_freq_base  = 10000.0f;
    float rms_eps         = 1e-5f;
    float qk_norm_eps     = 1e-6f;
    float logit_softcap   = 15.0f;

    uint32_t n_codebooks  = 0;
    uint32_t codebook_size= 0;
    uint32_t audio_vocab  = 0;
    uint32_t eoa_id       = 0;
    uint32_t audio_pad_id = 0;
    uint32_t text_vocab   = 0;

    uint32_t spk_dim      = 0;
    uint32_t spk_lda_dim  = 0;

    // prompt-building conditioning layout (carried for source compatibility; the decode step does
    // not read it)
    uint32_t             cond_speaking_rate_buckets   = 8;
    std::vector<int32_t> cond_quality_bucket_counts   = {12, 12, 12, 8, 8, 8};
    uint32_t             cond_speaker_bg_buckets      = 2;
    uint32_t             cond_accurate_buckets        = 1;
    int32_t              cond_default_quality_feature = 5;
    int32_t              cond_default_quality_bucket  = 3;

    std::vector<int32_t> expert_used;   // per layer: 0 => dense FFN, else MoE with this top-k
};

// A model whose weights live on one MI355X (device 0). The caller owns the struct; the device
// weights are reference counted, so batch contexts created from it stay valid until freed.
struct zonos2_model {
    zonos2_hparams hp;
    z2h_model * dev = nullptr;                       // device weights (see include/z2h.h)
    bool is_gpu = false;
    int router_dim = 0;                              // router_down ne1 (0 when no MoE layer)
    std::map<std::string, std::vector<int64_t>> tensors;   // loaded tensor name -> ne (ggml order)

    // depth prune: layer_skip[L] != 0 bypasses block L in every following prefill / step (the
    // residual passes through unchanged). Set directly on the model, as in the reference.
    std::vector<char> layer_skip;
};

// Load a zonos2 GGUF onto the GPU. use_gpu = false is refused (this build has no CPU backend).
// Returns false (with a message on stderr) on a missing key / tensor, an unsupported tensor type
// or a device failure.
bool zonos2_model_load(zonos2_model & model, const char * path, bool use_gpu);
void zonos2_model_free(zonos2_model & model);

// Hyperparameters, router_dim and the tensor table of a zonos2 GGUF, without touching the device
// (no counterpart in the reference: the first half of zonos2_model_load, for loader checks and
// tools that only inspect a file).
bool zonos2_model_read_meta(zonos2_model & model, const char * path);

// router hidden dimension, derived from the router_down weight (ne1)
int zonos2_router_dim(const zonos2_model & model);

// Runtime expert mask: for each MoE layer id in `keep` only the listed experts stay routable (the
// others get -inf router logits and selection scores); layers absent from `keep` are unmasked and
// {} clears every mask. Applies to every batch context of the model from its next step.
bool zonos2_set_expert_mask(zonos2_model & model, const std::map<int, std::vector<int>> & keep);

// Options of the text prompt builder (src/zonos2.h:178-188, same fields and defaults). The builder
// itself, zonos2_build_prompt (src/zonos2-prompt.cpp), reads only model.hp (its cond_* layout,
// n_codebooks, text_vocab, audio_pad_id) and is not part of this library: a caller that builds
// prompts compiles the reference's src/zonos2-prompt.cpp against this header.
struct zonos2_prompt_options {
    bool             prepend_silence        = true;  // append 17 sheared-silence frames
    int              speaking_rate_bucket   = -1;    // -1 = no speaking-rate row
    std::vector<int> quality_buckets;                // per-feature bucket (-1 = skip); empty => default
    bool             add_speaker_slot        = false; // prepend a speaker slot (+ markers) for cloning
    bool             clean_speaker_background = true;
    bool             accurate_mode           = true;
};

// Row-major input_ids [n_rows][n_codebooks + 1] of `text` (src/zonos2.h:190-194); spk_pos is the
// speaker slot's row when one was prepended, else -1. Defined by src/zonos2-prompt.cpp.
std::vector<int32_t> zonos2_build_prompt(const zonos2_model & model, const std::string & text,
                                         const zonos2_prompt_options & opt, int & n_rows, int & spk_pos);

// Name of the device the model's weights live on, for the messages and placement choices a caller
// made from ggml_backend_name(model.backend) (src/server.cpp:1601); "" before a successful load.
const char * zonos2_backend_name(const zonos2_model & model);

struct zonos2_sampling {
    float    temperature   = 1.15f;
    int      top_k         = 106;
    float    top_p         = 0.0f;   // 0 disables
    float    min_p         = 0.18f;
    float    rep_penalty   = 1.2f;
    int      rep_window    = 50;
    int      rep_codebooks = 8;
    uint32_t seed          = 0;
    bool     greedy        = false;
    float    emotion_cfg_scale = 1.0f;
};

struct zonos2_sampler;   // zonos2-sampler.h

using zonos2_frame_cb = std::function<bool(int frame_idx, const int32_t * codes, int ncb)>;

// A fixed set of n_slots decode sequences over one model. Slot s owns KV rows [0, slot_cap) of its
// own band; a step runs only the listed active slots (no padded idle columns).
struct zonos2_batch_ctx {
    const zonos2_model * model = nullptr;
    int n_slots  = 0;
    int slot_cap = 0;                 // rows per slot (a multiple of 256)
    int W = 0, ncb = 0, av = 0;       // n_codebooks+1, n_codebooks, audio_vocab

    // Widths a server warms up (the reference's decode-graph ladder {1,2,4,...,n_slots}); here the
    // device captures one HIP graph per active-column count on first use, so warming these widths
    // captures those graphs ahead of traffic.
    struct dec_graph { int width = 0; };
    std::vector<dec_graph> dec_ladder;

    z2h_ctx * dev = nullptr;          // device KV cache, scratch and step graphs

    // host scratch (reused each step)
    std::vector<int32_t> h_slot, h_npast, h_ids;
    std::vector<float>   h_logits;    // [n_slots][ncb][av], by slot index
    std::vector<float>   h_compact;   // [n_active][ncb][av] when the active slots are not 0..n-1
    int last_n = 0;                   // columns of the last step (their slot indices: h_slot[0, last_n))
    bool device_sampling = false;     // steps keep the logits on the GPU for zonos2_batch_sample
    // device-resident tables: zonos2_batch_sample left the next step's inputs of the last step's
    // columns on the GPU (fed_ids [last_n][W]); a step over the same slots with those next_ids runs
    // from them without host packing
    bool resident = false;
    std::vector<int32_t> fed_ids;
    std::vector<int32_t> h_slot_prev, h_npast_prev;   // the last step's columns and rows
};

// Per-slot decode state (graph-facing only; the sampler and output codes live with the caller).
struct zonos2_slot {
    int  index = -1;        // cache slot / decode column
    bool active = false;
    bool done   = false;
    int  n_past = 0;        // logical position where the next frame is written
    int  step   = 0;        // frames sampled so far
    int  eos_frame = -1;
    int  countdown = -1;
    std::vector<int32_t> next_ids; // [W] next input frame (audio codes + text pad)
};

// Allocate the KV cache (zero-filled) and step scratch; slot_cap_frames is rounded up to a multiple
// of 256. Returns false on allocation failure (after freeing partial state).
bool zonos2_batch_init(zonos2_batch_ctx & bc, const zonos2_model & model, int n_slots, int slot_cap_frames);
void zonos2_batch_free(zonos2_batch_ctx & bc);

// Prefill one sequence into `slot` (rows [0, n0) of its band). prompt_ids: row-major [n0][W] floats
// (rounded to the nearest integer id); out_logits receives the last prompt row's logits
// [n_codebooks][audio_vocab]. spk ([spk_dim], optional) replaces row spk_pos's embedding by
// spk_proj(spk_lda(spk)) (+ spk_emotion_delta [n_embd]). Returns false if n0 is not in [1, slot_cap]
// or on a device failure.
bool zonos2_batch_slot_prefill(zonos2_batch_ctx & bc, int slot, const float * prompt_ids, int n0,
                               const float * spk, int spk_pos, float * out_logits,
                               const float * spk_emotion_delta = nullptr);

// One batched decode step over the slots in `active` that are non-null, active and not done: each
// writes next_ids at its n_past, the step runs, each such slot's n_past advances by one. On a
// device failure a message goes to stderr and no n_past advances.
void zonos2_batch_step(zonos2_batch_ctx & bc, const std::vector<zonos2_slot *> & active);

// Slot `index`'s logits from the last step: [n_codebooks][audio_vocab], valid until the next step
// (not filled while bc.device_sampling is set: the logits then stay on the GPU).
const float * zonos2_batch_slot_logits(const zonos2_batch_ctx & bc, int index);

// Device sampling (no counterpart in the reference, whose sampler runs on the host per slot): draws
// the frame of every column of the last zonos2_batch_step on the GPU (include/z2h.h z2h_sample) with
// slot i's sampler smps[i] (settings, repetition history, and its mt19937 for the draws), then does
// zonos2_slot_sample's bookkeeping for each slot (history, eos / countdown, next_ids, step, done) and
// appends its codes to *out_codes[i]. `slots` must be exactly the slots the last step ran. With
// bc.device_sampling set, the step leaves the logits on the GPU (no host copy). Returns false (message
// on stderr) on a mismatch or a device failure; keep[i] receives on_frame's verdict per slot.
bool zonos2_batch_sample(zonos2_batch_ctx & bc, const std::vector<zonos2_slot *> & slots,
                         const std::vector<zonos2_sampler *> & smps, const std::vector<std::vector<int32_t> *> & out_codes,
                         int max_frames, const zonos2_frame_cb & on_frame, std::vector<char> * keep = nullptr);

// Sample one frame for `slot` from `logits` with `smp`, append its codes to out_codes, advance the
// slot's eos / countdown / step state and prepare next_ids; sets slot.done when finished (eos
// countdown elapsed, max_frames reached, or on_frame returned false). Returns on_frame's verdict.
bool zonos2_slot_sample(const zonos2_model & model, zonos2_slot & slot, zonos2_sampler & smp,
                        const float * logits, std::vector<int32_t> & out_codes,
                        int max_frames, const zonos2_frame_cb & on_frame);

// Autoregressive generation of one sequence. use_kv = true: one prefill, then one decode step per
// frame against the KV cache (the batch runtime at one slot; with spk, spk_emotion_delta and
// sp.emotion_cfg_scale != 1 a second slot is prefilled without the delta and every frame is drawn
// from uncond + scale * (cond - uncond)). use_kv = false: every frame recomputes a full prefill of
// the prompt and the frames so far (O(n^2)). prompt_ids: row-major [n0][n_codebooks + 1] floats.
// Appends the codes to out_codes ([n_frames][n_codebooks]), sets eos_frame (-1 if none), returns
// the frame count (0 on a failed start). spk ([spk_dim]) replaces row spk_pos's embedding during the
// prefill by spk_proj(spk_lda(spk)) (+ spk_emotion_delta [n_embd]). out_full_ids (optional) receives
// the consumed sequence [n0 + n_frames][n_codebooks + 1]: the prompt rows, then each frame's codes and
// the text pad. on_frame streams frames; returning false stops.
int zonos2_generate(const zonos2_model & model, const float * prompt_ids, int n0,
                    int max_frames, const zonos2_sampling & sp,
                    std::vector<int32_t> & out_codes, int & eos_frame, bool use_kv = true,
                    const float * spk = nullptr, int spk_pos = 0,
                    std::vector<int32_t> * out_full_ids = nullptr,
                    const zonos2_frame_cb & on_frame = {},
                    const float * spk_emotion_delta = nullptr);
