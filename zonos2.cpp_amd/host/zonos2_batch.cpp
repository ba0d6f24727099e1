// zonos2.h on the MI355X HIP library: GGUF model load, expert mask and the continuous-batching
// entry points (init / free / slot prefill / step / slot logits).
//
// The loader reads the same GGUF keys and tensor names as the reference (src/zonos2.cpp:15-186)
// and hands every tensor the device path uses to z2h_model_upload_tensor, which repacks it into the
// device layouts. The batch entry points translate the reference's slot lists into the flat arrays
// of z2h_step / z2h_prefill (src/zonos2-graph.cpp:639-841).
#include "zonos2.h"
#include "gguf.h"
#include "zonos2-sampler.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <limits>
#include <random>

namespace {

bool fail(const std::string & msg) {
    fprintf(stderr, "zonos2: %s\n", msg.c_str());
    return false;
}

// tensors the device path consumes; anything else in the file is listed in model.tensors only
bool used_tensor(const std::string & n) {
    if (n == "text_embd.weight" || n == "output.weight" || n == "output_norm.weight") return true;
    if (n.rfind("audio_embd.", 0) == 0 || n.rfind("spk_lda.", 0) == 0 || n.rfind("spk_proj.", 0) == 0) return true;
    return n.rfind("blk.", 0) == 0;
}

z2h_hparams to_z2h(const zonos2_hparams & hp, int router_dim) {
    z2h_hparams h{};
    h.n_layer = (int32_t) hp.n_layer; h.n_embd = (int32_t) hp.n_embd; h.head_dim = (int32_t) hp.head_dim;
    h.n_head = (int32_t) hp.n_head; h.n_head_kv = (int32_t) hp.n_head_kv; h.n_ff = (int32_t) hp.n_ff;
    h.n_expert = (int32_t) hp.n_expert; h.n_ctx_train = (int32_t) hp.n_ctx_train;
    h.rope_freq_base = hp.rope_freq_base; h.rms_eps = hp.rms_eps; h.qk_norm_eps = hp.qk_norm_eps;
    h.logit_softcap = hp.logit_softcap;
    h.n_codebooks = (int32_t) hp.n_codebooks; h.codebook_size = (int32_t) hp.codebook_size;
    h.audio_vocab = (int32_t) hp.audio_vocab; h.eoa_id = (int32_t) hp.eoa_id; h.audio_pad_id = (int32_t) hp.audio_pad_id;
    h.text_vocab = (int32_t) hp.text_vocab; h.spk_dim = (int32_t) hp.spk_dim; h.spk_lda_dim = (int32_t) hp.spk_lda_dim;
    h.router_dim = router_dim;
    h.expert_used = hp.expert_used.data();
    return h;
}

// push the caller-set depth prune to the device before a prefill / step
bool sync_layer_skip(const zonos2_model & m) {
    const int nl = (int) m.hp.n_layer;
    std::vector<uint8_t> skip(nl, 0);
    bool any = false;
    for (int L = 0; L < nl && L < (int) m.layer_skip.size(); ++L) if (m.layer_skip[L]) { skip[L] = 1; any = true; }
    return z2h_model_set_layer_skip(m.dev, any ? skip.data() : nullptr) == Z2H_OK;
}

} // namespace

// Header, hyperparameters and tensor table of a zonos2 GGUF, without touching the device.
bool zonos2_model_read_meta(zonos2_model & m, const char * path) {
    m = zonos2_model();
    z2::gguf_file f;
    std::string err;
    if (!path || !z2::gguf_read_header(path, f, err)) return fail(std::string("failed to open gguf '") + (path ? path : "") + "': " + err);
    auto & hp = m.hp;
    bool ok = true;
    auto u32 = [&](const char * key, uint32_t & dst) {
        const z2::gguf_value * v = f.find(key);
        if (!v || v->type == z2::GV_STR || v->type == z2::GV_ARR) { fail(std::string("missing kv '") + key + "'"); ok = false; return; }
        dst = (uint32_t) v->as_i64();
    };
    auto f32 = [&](const char * key, float & dst) {
        const z2::gguf_value * v = f.find(key);
        if (!v || v->type == z2::GV_STR || v->type == z2::GV_ARR) { fail(std::string("missing kv '") + key + "'"); ok = false; return; }
        dst = (float) v->as_f64();
    };
    u32("zonos2.block_count", hp.n_layer);
    u32("zonos2.embedding_length", hp.n_embd);
    u32("zonos2.head_dim", hp.head_dim);
    u32("zonos2.attention.head_count", hp.n_head);
    u32("zonos2.attention.head_count_kv", hp.n_head_kv);
    u32("zonos2.feed_forward_length", hp.n_ff);
    u32("zonos2.expert_count", hp.n_expert);
    u32("zonos2.context_length", hp.n_ctx_train);
    f32("zonos2.rope.freq_base", hp.rope_freq_base);
    f32("zonos2.attention.layer_norm_rms_epsilon", hp.rms_eps);
    f32("zonos2.attention.qk_norm_epsilon", hp.qk_norm_eps);
    f32("zonos2.logit_softcap", hp.logit_softcap);
    u32("zonos2.n_codebooks", hp.n_codebooks);
    u32("zonos2.codebook_size", hp.codebook_size);
    u32("zonos2.audio_vocab", hp.audio_vocab);
    u32("zonos2.eoa_id", hp.eoa_id);
    u32("zonos2.audio_pad_id", hp.audio_pad_id);
    u32("zonos2.text_vocab", hp.text_vocab);
    u32("zonos2.speaker.embedding_dim", hp.spk_dim);
    u32("zonos2.speaker.lda_dim", hp.spk_lda_dim);
    const z2::gguf_value * eu = f.find("zonos2.expert_used_count_per_layer");
    if (!eu || eu->type != z2::GV_ARR || eu->arr_type != z2::GV_I32) {
        ok = fail("missing/!int32 expert_used_count_per_layer");
    } else {
        hp.expert_used.resize(eu->n);
        std::memcpy(hp.expert_used.data(), eu->raw.data(), eu->n * 4);
        if (eu->n != hp.n_layer) ok = fail("expert_used n=" + std::to_string(eu->n) + " != n_layer=" + std::to_string(hp.n_layer));
    }
    if (!ok) return false;
    for (const auto & t : f.tensors) m.tensors[t.name] = t.ne;
    // router_dim = router_down ne1 of the first MoE layer (src/zonos2.cpp:241-246)
    for (uint32_t L = 0; L < hp.n_layer; ++L) {
        auto it = m.tensors.find("blk." + std::to_string(L) + ".router_down.weight");
        if (it != m.tensors.end() && it->second.size() >= 2) { m.router_dim = (int) it->second[1]; break; }
    }
    return true;
}

bool zonos2_model_load(zonos2_model & m, const char * path, bool use_gpu) {
    if (!use_gpu) return fail("this build runs the model on the MI355X only; use_gpu=false has no CPU backend");
    if (!zonos2_model_read_meta(m, path)) return false;
    z2::gguf_file f;
    std::string err;
    if (!z2::gguf_read_header(path, f, err)) return fail(err);
    // required tensors, as the reference's loader demands them (src/zonos2.cpp:137-183)
    const auto & hp = m.hp;
    std::vector<std::string> req = {"text_embd.weight", "spk_lda.weight", "spk_lda.bias", "spk_proj.weight",
                                    "spk_proj.bias", "output_norm.weight", "output.weight"};
    for (uint32_t i = 0; i < hp.n_codebooks; ++i) req.push_back("audio_embd." + std::to_string(i) + ".weight");
    for (uint32_t L = 0; L < hp.n_layer; ++L) {
        const std::string b = "blk." + std::to_string(L) + ".";
        for (const char * n : {"attn_norm.weight", "ffn_norm.weight", "attn_q.weight", "attn_k.weight", "attn_v.weight",
                               "attn_output.weight", "attn_temp", "attn_gate.weight"}) req.push_back(b + n);
        if (hp.expert_used[L] > 0) {
            for (const char * n : {"ffn_gate_exps.weight", "ffn_up_exps.weight", "ffn_down_exps.weight", "router_down.weight",
                                   "router_down.bias", "router_mlp0.weight", "router_mlp0.bias", "router_mlp2.weight",
                                   "router_mlp2.bias", "router_mlp4.weight", "router_norm.weight", "router_bias"}) req.push_back(b + n);
        } else {
            for (const char * n : {"ffn_up.weight", "ffn_gate.weight", "ffn_down.weight"}) req.push_back(b + n);
        }
    }
    bool ok = true;
    for (const auto & n : req) if (!m.tensors.count(n)) ok = fail("required tensor '" + n + "' not found");
    if (!ok) return false;

    const z2h_hparams h = to_z2h(hp, m.router_dim);
    if (int rc = z2h_model_create(&h, 0, &m.dev)) {
        m.dev = nullptr;
        return fail("device model create failed (status " + std::to_string(rc) + "): unsupported shape or no GPU");
    }
    m.is_gpu = true;
    std::vector<uint8_t> buf;
    size_t total = 0;
    int n_up = 0;
    for (const auto & t : f.tensors) {
        if (!used_tensor(t.name)) continue;
        if (!z2::gguf_read_tensor(path, f, t, buf, err)) { zonos2_model_free(m); return fail(err); }
        int64_t ne[4] = {1, 1, 1, 1};
        for (size_t i = 0; i < t.ne.size() && i < 4; ++i) ne[i] = t.ne[i];
        if (int rc = z2h_model_upload_tensor(m.dev, t.name.c_str(), t.type, ne, buf.data(), buf.size())) {
            const std::string msg = std::string(z2h_model_last_error(m.dev)) + " (status " + std::to_string(rc) + ")";
            zonos2_model_free(m);
            return fail("tensor '" + t.name + "': " + msg);
        }
        total += buf.size();
        ++n_up;
    }
    if (int rc = z2h_model_finalize(m.dev)) {
        const std::string msg = z2h_model_last_error(m.dev);
        zonos2_model_free(m);
        return fail("model check failed (status " + std::to_string(rc) + "): " + msg);
    }
    fprintf(stderr, "zonos2: loaded %d tensors, %.2f GiB onto the MI355X\n", n_up, total / (1024.0 * 1024.0 * 1024.0));
    return true;
}

void zonos2_model_free(zonos2_model & m) {
    if (m.dev) z2h_model_release(m.dev);
    m = zonos2_model();
}

int zonos2_router_dim(const zonos2_model & m) { return m.router_dim; }

bool zonos2_set_expert_mask(zonos2_model & m, const std::map<int, std::vector<int>> & keep) {
    if (!m.dev) return fail("expert mask: model not loaded");
    const int nl = (int) m.hp.n_layer;
    for (int L = 0; L < nl; ++L)                    // clear every previous mask
        if (m.hp.expert_used[L] > 0 && z2h_model_set_expert_mask(m.dev, L, nullptr) != Z2H_OK)
            return fail(std::string("expert mask: ") + z2h_model_last_error(m.dev));
    int n_layers = 0, dropped = 0;
    for (const auto & kv : keep) {
        const int L = kv.first;
        if (L < 0 || L >= nl || m.hp.expert_used[L] <= 0) continue;
        auto it = m.tensors.find("blk." + std::to_string(L) + ".ffn_up_exps.weight");
        const int ne = it != m.tensors.end() && it->second.size() >= 3 ? (int) it->second[2] : (int) m.hp.n_expert;
        std::vector<uint8_t> k(ne, 0);
        for (const int e : kv.second) if (e >= 0 && e < ne) k[e] = 1;
        for (const uint8_t v : k) dropped += v ? 0 : 1;
        if (z2h_model_set_expert_mask(m.dev, L, k.data()) != Z2H_OK)
            return fail(std::string("expert mask: ") + z2h_model_last_error(m.dev));
        ++n_layers;
    }
    if (n_layers) fprintf(stderr, "zonos2: expert mask on %d MoE layers, %d experts dropped\n", n_layers, dropped);
    return true;
}

bool zonos2_batch_init(zonos2_batch_ctx & bc, const zonos2_model & m, int n_slots, int slot_cap_frames) {
    zonos2_batch_free(bc);
    if (!m.dev) return fail("batch init: model not loaded");
    if (n_slots <= 0 || slot_cap_frames <= 0) return fail("batch init: n_slots and slot_cap_frames must be positive");
    if (int rc = z2h_create_batch(m.dev, n_slots, slot_cap_frames, &bc.dev)) {
        bc.dev = nullptr;
        return fail("batch KV alloc failed (" + std::to_string(n_slots) + " slots x " + std::to_string(slot_cap_frames) +
                    " rows, status " + std::to_string(rc) + "): " + z2h_model_last_error(m.dev));
    }
    bc.model = &m;
    bc.n_slots = n_slots;
    bc.slot_cap = z2h_slot_cap(bc.dev);
    bc.W = (int) m.hp.n_codebooks + 1;
    bc.ncb = (int) m.hp.n_codebooks;
    bc.av = (int) m.hp.audio_vocab;
    for (int w = 1; w < n_slots; w *= 2) bc.dec_ladder.push_back({w});
    bc.dec_ladder.push_back({n_slots});
    bc.h_slot.assign(n_slots, 0);
    bc.h_npast.assign(n_slots, 0);
    bc.h_ids.assign((size_t) n_slots * bc.W, 0);
    bc.h_logits.assign((size_t) n_slots * bc.ncb * bc.av, 0.0f);
    return true;
}

void zonos2_batch_free(zonos2_batch_ctx & bc) {
    if (bc.dev) z2h_destroy(bc.dev);
    bc = zonos2_batch_ctx();
}

bool zonos2_batch_slot_prefill(zonos2_batch_ctx & bc, int slot, const float * prompt_ids, int n0,
                               const float * spk, int spk_pos, float * out_logits,
                               const float * spk_emotion_delta) {
    if (!bc.dev || !bc.model) return fail("prefill: batch context not initialised");
    if (n0 <= 0 || n0 > bc.slot_cap) return fail("prefill n0=" + std::to_string(n0) + " exceeds slot_cap=" + std::to_string(bc.slot_cap));
    if (slot < 0 || slot >= bc.n_slots) return fail("prefill: slot " + std::to_string(slot) + " out of range");
    if (!prompt_ids || !out_logits) return fail("prefill: null prompt or output");
    if (!sync_layer_skip(*bc.model)) return fail("prefill: layer skip");
    std::vector<int32_t> ids((size_t) n0 * bc.W);
    for (size_t i = 0; i < ids.size(); ++i) ids[i] = (int32_t) lroundf(prompt_ids[i]);
    if (int rc = z2h_prefill(bc.dev, slot, ids.data(), n0, spk, spk ? spk_pos : -1, spk ? spk_emotion_delta : nullptr, out_logits))
        return fail("prefill failed (status " + std::to_string(rc) + "): " + z2h_last_error(bc.dev));
    return true;
}

void zonos2_batch_step(zonos2_batch_ctx & bc, const std::vector<zonos2_slot *> & active) {
    if (!bc.dev || !bc.model) { fail("step: batch context not initialised"); return; }
    std::vector<zonos2_slot *> run;
    for (zonos2_slot * sp : active)
        if (sp && sp->active && !sp->done) run.push_back(sp);
    if (run.empty()) return;
    // ascending slot index, so the usual low-first allocation writes the logits in place
    std::stable_sort(run.begin(), run.end(), [](const zonos2_slot * a, const zonos2_slot * b) { return a->index < b->index; });
    const int n = (int) run.size(), W = bc.W;
    bool dense = true;
    for (int i = 0; i < n; ++i) {
        zonos2_slot & s = *run[i];
        if (s.index < 0 || s.index >= bc.n_slots || (int) s.next_ids.size() < W) {
            fail("step: slot " + std::to_string(s.index) + " has no valid index / next_ids");
            return;
        }
        bc.h_slot[i] = s.index;
        bc.h_npast[i] = s.n_past;
        std::memcpy(&bc.h_ids[(size_t) i * W], s.next_ids.data(), (size_t) W * 4);
        dense = dense && s.index == i;
    }
    const size_t row = (size_t) bc.ncb * bc.av;
    if (!dense) bc.h_compact.resize((size_t) n * row);
    float * out = dense ? bc.h_logits.data() : bc.h_compact.data();
    if (!sync_layer_skip(*bc.model)) { fail("step: layer skip"); return; }
    // the same columns as the last step, each one row further, fed by the device sampler: run from
    // the device-resident tables
    bool resident = bc.resident && bc.device_sampling && n == bc.last_n && (int) bc.fed_ids.size() == n * W;
    // (a slot whose band is full takes the host path, which refuses the step before any launch)
    for (int i = 0; resident && i < n; ++i)
        resident = run[i]->index == bc.h_slot_prev[i] && run[i]->n_past == bc.h_npast_prev[i] + 1 &&
                   run[i]->n_past < bc.slot_cap &&
                   std::equal(run[i]->next_ids.begin(), run[i]->next_ids.begin() + W, bc.fed_ids.begin() + (size_t) i * W);
    bc.resident = false;
    if (resident) {
        if (int rc = z2h_step_resident(bc.dev, n)) {
            fail("step failed (status " + std::to_string(rc) + "): " + z2h_last_error(bc.dev));
            return;
        }
        for (int i = 0; i < n; ++i) { bc.h_slot_prev[i] = run[i]->index; bc.h_npast_prev[i] = run[i]->n_past; }
        bc.last_n = n;
        for (zonos2_slot * sp : run) sp->n_past += 1;
        return;
    }
    bc.last_n = 0;
    if (int rc = z2h_step(bc.dev, n, bc.h_slot.data(), bc.h_npast.data(), bc.h_ids.data(), nullptr,
                          bc.device_sampling ? nullptr : out)) {
        fail("step failed (status " + std::to_string(rc) + "): " + z2h_last_error(bc.dev));
        return;
    }
    bc.last_n = n;
    bc.h_slot_prev.assign(bc.h_slot.begin(), bc.h_slot.begin() + n);
    bc.h_npast_prev.assign(bc.h_npast.begin(), bc.h_npast.begin() + n);
    if (!dense && !bc.device_sampling)
        for (int i = 0; i < n; ++i)
            std::memcpy(&bc.h_logits[(size_t) run[i]->index * row], &out[(size_t) i * row], row * 4);
    for (zonos2_slot * sp : run) sp->n_past += 1;
}

const char * zonos2_backend_name(const zonos2_model & model) {
    return model.is_gpu && model.dev ? "ROCm HIP (MI355X, gfx950)" : "";
}

const float * zonos2_batch_slot_logits(const zonos2_batch_ctx & bc, int index) {
    return bc.h_logits.data() + (size_t) index * bc.av * bc.ncb;
}

bool zonos2_batch_sample(zonos2_batch_ctx & bc, const std::vector<zonos2_slot *> & slots,
                         const std::vector<zonos2_sampler *> & smps, const std::vector<std::vector<int32_t> *> & out_codes,
                         int max_frames, const zonos2_frame_cb & on_frame, std::vector<char> * keep) {
    if (!bc.dev || !bc.model) return fail("sample: batch context not initialised");
    const int n = bc.last_n, ncb = bc.ncb;
    if (n <= 0) return fail("sample: no step to sample from");
    if ((int) slots.size() != n || smps.size() != slots.size() || out_codes.size() != slots.size())
        return fail("sample: slots / samplers / outputs must list exactly the last step's slots");
    // column of each slot in the last step, the per-column settings, histories and draws
    std::vector<int> col(n, -1);
    for (int i = 0; i < n; ++i) {
        if (!slots[i] || !smps[i] || !out_codes[i]) return fail("sample: null slot / sampler / output");
        for (int c = 0; c < n; ++c) if (bc.h_slot[c] == slots[i]->index) col[i] = c;
        if (col[i] < 0) return fail("sample: slot " + std::to_string(slots[i]->index) + " was not in the last step");
    }
    int cap = 1;
    for (int i = 0; i < n; ++i)
        for (const auto & h : smps[i]->hist) cap = std::max(cap, (int) h.size());
    if (cap > Z2H_SAMPLE_HIST_MAX) return fail("sample: repetition window above Z2H_SAMPLE_HIST_MAX");
    std::vector<z2h_sampling> sp(n);
    std::vector<int32_t> hist((size_t) n * ncb * cap, 0), hlen((size_t) n * ncb, 0), codes((size_t) n * ncb);
    std::vector<double> u((size_t) n * ncb, 0.0);
    for (int i = 0; i < n; ++i) {
        const int c = col[i];
        zonos2_sampler & smp = *smps[i];
        if (smp.n_cb != ncb || smp.vocab != bc.av) return fail("sample: sampler shape differs from the model's");
        z2h_sampling & s = sp[c];
        s.temperature = smp.sp.temperature; s.top_k = smp.sp.top_k; s.top_p = smp.sp.top_p; s.min_p = smp.sp.min_p;
        s.rep_penalty = smp.sp.rep_penalty; s.rep_codebooks = smp.sp.rep_codebooks; s.greedy = smp.sp.greedy ? 1 : 0;
        s.reserved = 0;
        for (int cb = 0; cb < ncb; ++cb) {
            const auto & h = smp.hist[cb];
            int j = 0;
            for (const int t : h) hist[((size_t) c * ncb + cb) * cap + j++] = t;
            hlen[(size_t) c * ncb + cb] = j;
            // the host sampler's draw: uniform_real_distribution<double>(0, mass) on its mt19937 is
            // generate_canonical<double, 53> times the mass, taken once per codebook in order. It
            // takes none where the kept mass is 0 (src/zonos2-sampler.cpp:70); with finite logits the
            // largest probability is > 0 and survives top-p, so that happens exactly when min-p
            // drops it too, min_p > 1 (min_p * p_max rounds above p_max for any float min_p > 1)
            if (!smp.sp.greedy && !(smp.sp.min_p > 1.0f))
                u[(size_t) c * ncb + cb] = std::generate_canonical<double, std::numeric_limits<double>::digits>(smp.rng);
        }
    }
    if (int rc = z2h_sample_feed(bc.dev, n, sp.data(), hist.data(), hlen.data(), cap, u.data(), codes.data()))
        return fail("sample failed (status " + std::to_string(rc) + "): " + z2h_last_error(bc.dev));
    // the next step's inputs now wait on the GPU, by column
    bc.fed_ids.assign((size_t) n * bc.W, (int32_t) bc.model->hp.text_vocab);
    for (int c = 0; c < n; ++c)
        for (int cb = 0; cb < ncb; ++cb) bc.fed_ids[(size_t) c * bc.W + cb] = codes[(size_t) c * ncb + cb];
    bc.resident = true;
    if (keep) keep->assign(n, 1);
    for (int i = 0; i < n; ++i) {
        const std::vector<int> frame(codes.begin() + (size_t) col[i] * ncb, codes.begin() + (size_t) (col[i] + 1) * ncb);
        const bool k = zonos2_slot_finish_frame(*bc.model, *slots[i], *smps[i], frame, *out_codes[i], max_frames, on_frame);
        if (keep) (*keep)[i] = k;
    }
    return true;
}
