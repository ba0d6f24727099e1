// zonos2_generate (src/zonos2.h:308-325) on the batch API.
//
// use_kv = true is the reference's real-time path (src/zonos2-graph.cpp:877-951): one prefill, then
// one decode step per frame against the slot's KV band, i.e. the batch runtime at one slot, or two
// when emotion guidance is on: the second slot is prefilled without the emotion delta and steps in
// lockstep, and each frame is sampled from uncond + scale * (cond - uncond).
// use_kv = false is the reference's O(n^2) path (src/zonos2-graph.cpp:515-605): every frame runs a
// full causal prefill of the prompt plus the frames generated so far and samples from its last row.
// Both sample on the host with zonos2_sampler, so a seed gives the reference's draws for the same
// logits, and both rebuild the consumed input sequence for out_full_ids (graph.cpp:966-979).
#include "zonos2.h"
#include "zonos2-sampler.h"

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>

namespace {

// frees the batch context on every exit path
struct BatchScope {
    zonos2_batch_ctx bc;
    ~BatchScope() { zonos2_batch_free(bc); }
};

// One audio frame at 44.1 kHz spans 512 samples; frames/s above 44100 / 512 is faster than real time.
constexpr double FRAME_SECONDS = 512.0 / 44100.0;

int generate_cached(const zonos2_model & m, const float * prompt_ids, int n0, int max_frames,
                    const zonos2_sampling & sp, std::vector<int32_t> & out_codes, int & eos_frame,
                    const float * spk, int spk_pos, const zonos2_frame_cb & on_frame, const float * delta) {
    const int ncb = (int) m.hp.n_codebooks, av = (int) m.hp.audio_vocab;
    const size_t n_logits = (size_t) ncb * av;
    eos_frame = -1;
    const bool guided = spk && delta && sp.emotion_cfg_scale != 1.0f;

    BatchScope b;
    if (!zonos2_batch_init(b.bc, m, guided ? 2 : 1, n0 + max_frames + 8)) return 0;
    zonos2_sampler smp(sp, ncb, av);

    // slot 0 carries the emotion delta; slot 1 (guided only) is the unconditioned twin
    zonos2_slot cond, twin;
    cond.index = 0; cond.active = true; cond.n_past = n0;
    twin.index = 1; twin.active = guided; twin.n_past = n0;
    std::vector<float> lc(n_logits), lu(guided ? n_logits : 0), mix(guided ? n_logits : 0);
    if (!zonos2_batch_slot_prefill(b.bc, 0, prompt_ids, n0, spk, spk_pos, lc.data(), delta)) return 0;
    if (guided && !zonos2_batch_slot_prefill(b.bc, 1, prompt_ids, n0, spk, spk_pos, lu.data(), nullptr)) return 0;

    std::vector<zonos2_slot *> active{&cond};
    if (guided) active.push_back(&twin);
    int frames = 0, steps = 0;
    const auto t0 = std::chrono::steady_clock::now();
    for (;;) {
        const float * draw_from = lc.data();
        if (guided) {
            const float s = sp.emotion_cfg_scale;
            for (size_t i = 0; i < n_logits; ++i) mix[i] = lu[i] + s * (lc[i] - lu[i]);
            draw_from = mix.data();
        }
        zonos2_slot_sample(m, cond, smp, draw_from, out_codes, max_frames, on_frame);
        ++frames;
        if (guided) {                      // the twin consumes the same frame and stops with slot 0
            twin.next_ids = cond.next_ids;
            twin.step = cond.step;
            twin.eos_frame = cond.eos_frame;
            twin.countdown = cond.countdown;
            twin.done = cond.done;
        }
        if (cond.done) break;
        zonos2_batch_step(b.bc, active);
        std::memcpy(lc.data(), zonos2_batch_slot_logits(b.bc, 0), n_logits * sizeof(float));
        if (guided) std::memcpy(lu.data(), zonos2_batch_slot_logits(b.bc, 1), n_logits * sizeof(float));
        ++steps;
    }
    eos_frame = cond.eos_frame;
    if (steps > 0) {
        const double dt = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        fprintf(stderr, "generate(kv): %d decode steps in %.3fs = %.1f frames/s (real-time = %.1f), RTF=%.2f\n",
                steps, dt, steps / dt, 1.0 / FRAME_SECONDS, (dt / steps) / FRAME_SECONDS);
    }
    return frames;
}

int generate_recompute(const zonos2_model & m, const float * prompt_ids, int n0, int max_frames,
                       const zonos2_sampling & sp, std::vector<int32_t> & out_codes, int & eos_frame,
                       const float * spk, int spk_pos, const zonos2_frame_cb & on_frame, const float * delta) {
    const int ncb = (int) m.hp.n_codebooks, av = (int) m.hp.audio_vocab, W = ncb + 1;
    eos_frame = -1;
    if (max_frames <= 0) return 0;
    // the sequence as consumed: prompt ids rounded to integers, then each frame + the text pad
    std::vector<float> seq((size_t) n0 * W);
    for (size_t i = 0; i < seq.size(); ++i) seq[i] = (float) lroundf(prompt_ids[i]);

    BatchScope b;
    if (!zonos2_batch_init(b.bc, m, 1, n0 + max_frames)) return 0;
    zonos2_sampler smp(sp, ncb, av);
    std::vector<float> lo((size_t) ncb * av);
    std::vector<int> frame(ncb);
    int countdown = -1, frames = 0;
    for (int step = 0; step < max_frames; ++step) {
        const int n = (int) (seq.size() / W);
        if (!zonos2_batch_slot_prefill(b.bc, 0, seq.data(), n, spk, spk ? spk_pos : -1, lo.data(), spk ? delta : nullptr)) {
            fprintf(stderr, "generate: compute failed at step %d\n", step);
            break;
        }
        for (int cb = 0; cb < ncb; ++cb) frame[cb] = smp.sample(lo.data() + (size_t) cb * av, cb);
        smp.accept(frame);
        out_codes.insert(out_codes.end(), frame.begin(), frame.end());
        ++frames;
        if (on_frame) {
            const std::vector<int32_t> fc(frame.begin(), frame.end());
            if (!on_frame(frames - 1, fc.data(), ncb)) break;
        }
        for (int cb = 0; cb < ncb; ++cb) seq.push_back((float) frame[cb]);
        seq.push_back((float) m.hp.text_vocab);
        // end of audio: the first eoa code in any codebook fixes the aligned frame, then n_codebooks + 1
        // more frames are drawn
        int last_eoa = -1;
        for (int cb = 0; cb < ncb; ++cb) if (frame[cb] == (int) m.hp.eoa_id) last_eoa = cb;
        if (eos_frame < 0 && last_eoa >= 0) {
            eos_frame = step - last_eoa > 0 ? step - last_eoa : 0;
            countdown = ncb + 1;
        }
        if (countdown > 0 && --countdown == 0) break;
    }
    return frames;
}

} // namespace

int zonos2_generate(const zonos2_model & model, const float * prompt_ids, int n0, int max_frames,
                    const zonos2_sampling & sp, std::vector<int32_t> & out_codes, int & eos_frame, bool use_kv,
                    const float * spk, int spk_pos, std::vector<int32_t> * out_full_ids,
                    const zonos2_frame_cb & on_frame, const float * spk_emotion_delta) {
    const size_t first = out_codes.size();
    const int nf = use_kv
        ? generate_cached(model, prompt_ids, n0, max_frames, sp, out_codes, eos_frame, spk, spk_pos, on_frame, spk_emotion_delta)
        : generate_recompute(model, prompt_ids, n0, max_frames, sp, out_codes, eos_frame, spk, spk_pos, on_frame, spk_emotion_delta);
    if (out_full_ids) {
        const int ncb = (int) model.hp.n_codebooks, W = ncb + 1;
        out_full_ids->clear();
        out_full_ids->reserve((size_t) (n0 + nf) * W);
        for (int i = 0; i < n0 * W; ++i) out_full_ids->push_back((int32_t) lroundf(prompt_ids[i]));
        for (int f = 0; f < nf; ++f) {
            const int32_t * fr = out_codes.data() + first + (size_t) f * ncb;
            out_full_ids->insert(out_full_ids->end(), fr, fr + ncb);
            out_full_ids->push_back((int32_t) model.hp.text_vocab);
        }
    }
    return nf;
}
