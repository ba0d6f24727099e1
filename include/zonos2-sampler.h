// zonos2-sampler.h — per-codebook frame sampler on the host: repetition penalty, temperature,
// top-k, top-p, min-p and a multinomial draw (the reference's src/zonos2-sampler.h, same members
// and behaviour; restated in host/zonos2_sampler.cpp).
#pragma once

#include "zonos2.h"

#include <deque>
#include <random>
#include <vector>

struct zonos2_sampler {
    zonos2_sampling sp;
    std::mt19937 rng;
    int n_cb;
    int vocab;
    std::vector<std::deque<int>> hist;   // recent codes per codebook (repetition penalty window)

    zonos2_sampler(const zonos2_sampling & s, int n_codebooks, int vocab_);
    int  sample(const float * logits, int cb);        // logits: [vocab]
    void accept(const std::vector<int> & frame);      // push a sampled frame into the history
};

// The part of zonos2_slot_sample after the draws (history, eos / countdown, next_ids, step, done), for
// a frame sampled elsewhere (zonos2_batch_sample). Returns on_frame's verdict.
bool zonos2_slot_finish_frame(const zonos2_model & m, zonos2_slot & s, zonos2_sampler & smp, const std::vector<int> & frame,
                              std::vector<int32_t> & out_codes, int max_frames, const zonos2_frame_cb & on_frame);
