// Host frame sampler and per-slot frame bookkeeping.
//
// zonos2_sampler follows the reference's src/zonos2-sampler.cpp:5-77 step for step, because a
// caller that switches libraries must draw the same codes from the same logits and seed: the
// candidate set is chosen with std::partial_sort and ranked with std::sort on the same comparators
// over the same index sequences (so equal logits break the same way under the same C++ library),
// probabilities are float exp over a double sum, and the draw is one
// std::uniform_real_distribution<double> value from a std::mt19937 seeded with sp.seed.
// zonos2_slot_sample follows src/zonos2-graph.cpp:843-870.
#include "zonos2-sampler.h"

#include <algorithm>
#include <cmath>

zonos2_sampler::zonos2_sampler(const zonos2_sampling & s, int n_codebooks, int vocab_)
    : sp(s), rng(s.seed), n_cb(n_codebooks), vocab(vocab_), hist(n_codebooks) {}

void zonos2_sampler::accept(const std::vector<int> & frame) {
    const int n = std::min(n_cb, (int) frame.size());
    for (int cb = 0; cb < n; ++cb) {
        std::deque<int> & h = hist[cb];
        h.push_back(frame[cb]);
        while ((int) h.size() > sp.rep_window) h.pop_front();
    }
}

int zonos2_sampler::sample(const float * in, int cb) {
    if (sp.greedy) {                                 // first maximum
        int best = 0;
        for (int i = 1; i < vocab; ++i) if (in[i] > in[best]) best = i;
        return best;
    }
    std::vector<float> lg(in, in + vocab);
    // repetition penalty: every occurrence in the codebook's window applies once
    if (sp.rep_penalty != 1.0f && cb < sp.rep_codebooks)
        for (const int t : hist[cb])
            if (t >= 0 && t < vocab) lg[t] = lg[t] > 0.0f ? lg[t] / sp.rep_penalty : lg[t] * sp.rep_penalty;
    if (sp.temperature > 0.0f)
        for (float & v : lg) v /= sp.temperature;

    // candidates: all ids, or the top_k by logit
    std::vector<int> cand(vocab);
    for (int i = 0; i < vocab; ++i) cand[i] = i;
    const int k = sp.top_k > 0 && sp.top_k < vocab ? sp.top_k : vocab;
    const auto by_logit = [&lg](int a, int b) { return lg[a] > lg[b]; };
    if (k < vocab) {
        std::partial_sort(cand.begin(), cand.begin() + k, cand.end(), by_logit);
        cand.resize(k);
    }
    const size_t n = cand.size();

    // softmax over the candidates (float terms, double normaliser)
    float mx = -1e30f;
    for (const int i : cand) mx = std::max(mx, lg[i]);
    std::vector<float> p(n);
    double z = 0.0;
    for (size_t j = 0; j < n; ++j) { p[j] = std::exp(lg[cand[j]] - mx); z += p[j]; }
    for (float & v : p) v = (float) (v / z);

    // rank by probability (top-p walks it; min-p compares with its head)
    std::vector<int> rank(n);
    for (size_t j = 0; j < n; ++j) rank[j] = (int) j;
    std::sort(rank.begin(), rank.end(), [&p](int a, int b) { return p[a] > p[b]; });

    std::vector<char> keep(n, 1);
    if (sp.top_p > 0.0f && sp.top_p < 1.0f) {
        double c = 0.0;
        bool reached = false;
        for (const int r : rank) {
            if (reached) keep[r] = 0;
            c += p[r];
            if (c >= sp.top_p) reached = true;
        }
    }
    if (sp.min_p > 0.0f) {
        const float floor_p = sp.min_p * p[rank[0]];
        for (size_t j = 0; j < n; ++j) if (p[j] < floor_p) keep[j] = 0;
    }
    double mass = 0.0;
    for (size_t j = 0; j < n; ++j) { if (!keep[j]) p[j] = 0.0f; mass += p[j]; }
    if (mass <= 0.0) return cand[rank[0]];

    std::uniform_real_distribution<double> draw(0.0, mass);
    const double r = draw(rng);
    double acc = 0.0;
    for (size_t j = 0; j < n; ++j) {
        acc += p[j];
        if (acc >= r) return cand[j];
    }
    return cand[rank[0]];
}

bool zonos2_slot_sample(const zonos2_model & m, zonos2_slot & s, zonos2_sampler & smp,
                        const float * logits, std::vector<int32_t> & out_codes,
                        int max_frames, const zonos2_frame_cb & on_frame) {
    const int ncb = (int) m.hp.n_codebooks, av = (int) m.hp.audio_vocab;
    std::vector<int> frame(ncb);
    for (int cb = 0; cb < ncb; ++cb) frame[cb] = smp.sample(logits + (size_t) cb * av, cb);
    return zonos2_slot_finish_frame(m, s, smp, frame, out_codes, max_frames, on_frame);
}

bool zonos2_slot_finish_frame(const zonos2_model & m, zonos2_slot & s, zonos2_sampler & smp, const std::vector<int> & frame,
                              std::vector<int32_t> & out_codes, int max_frames, const zonos2_frame_cb & on_frame) {
    const int ncb = (int) m.hp.n_codebooks;
    smp.accept(frame);
    out_codes.insert(out_codes.end(), frame.begin(), frame.end());

    const int frame_idx = s.step;
    bool keep = true;
    if (on_frame) {
        const std::vector<int32_t> codes(frame.begin(), frame.end());
        keep = on_frame(frame_idx, codes.data(), ncb);
    }
    // end of audio: the highest codebook that emitted eoa dates the end (codebooks are sheared by
    // one frame each), and the slot runs ncb + 1 more frames so every codebook can finish
    int last_eoa = -1;
    for (int cb = 0; cb < ncb; ++cb) if (frame[cb] == (int) m.hp.eoa_id) last_eoa = cb;
    if (s.eos_frame < 0 && last_eoa >= 0) {
        s.eos_frame = std::max(0, frame_idx - last_eoa);
        s.countdown = ncb + 1;
    }
    const bool finished = s.countdown > 0 && --s.countdown == 0;

    s.next_ids.assign(frame.begin(), frame.end());
    s.next_ids.push_back((int32_t) m.hp.text_vocab);
    s.step += 1;
    if (!keep || finished || s.step >= max_frames) s.done = true;
    return keep;
}
