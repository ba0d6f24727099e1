// zonos2_generate against loops written directly on the batch API, on a GGUF model (argv[1]).
//
// The KV path must be the one-slot batch runtime: prefill, then sample / step per frame
// (src/zonos2-graph.cpp:877-951); with emotion guidance a second slot prefilled without the delta
// steps in lockstep and each frame is drawn from uncond + scale * (cond - uncond). The recompute path
// must be a full prefill of the growing sequence per frame (graph.cpp:515-605). Codes, eos_frame,
// frame counts, out_full_ids and on_frame's early stop are compared; exit status 0 when all agree.
#include "zonos2.h"
#include "zonos2-sampler.h"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

namespace {

int g_fail = 0;
void expect(bool ok, const char * what) {
    printf("%s: %s\n", ok ? "ok  " : "FAIL", what);
    if (!ok) ++g_fail;
}

std::vector<float> prompt_rows(const zonos2_model & m, int n0, uint32_t seed) {
    const int ncb = (int) m.hp.n_codebooks, W = ncb + 1;
    std::mt19937 rng(seed);
    std::vector<float> ids((size_t) n0 * W);
    for (int t = 0; t < n0; ++t) {
        for (int k = 0; k < ncb; ++k) ids[(size_t) t * W + k] = (float) (rng() % m.hp.codebook_size);
        ids[(size_t) t * W + ncb] = (float) (rng() % (m.hp.text_vocab + 1));
    }
    return ids;
}

std::vector<float> normal_vec(size_t n, uint32_t seed, float scale) {
    std::mt19937 rng(seed);
    std::normal_distribution<float> nd(0.0f, scale);
    std::vector<float> v(n);
    for (float & x : v) x = nd(rng);
    return v;
}

// the KV path by hand: one slot (two with guidance), host sampler
int hand_kv(const zonos2_model & m, const std::vector<float> & prompt, int n0, int max_frames, const zonos2_sampling & sp,
            const float * spk, int spk_pos, const float * delta, std::vector<int32_t> & codes, int & eos) {
    const int ncb = (int) m.hp.n_codebooks, av = (int) m.hp.audio_vocab;
    const bool guided = spk && delta && sp.emotion_cfg_scale != 1.0f;
    zonos2_batch_ctx bc;
    if (!zonos2_batch_init(bc, m, guided ? 2 : 1, n0 + max_frames + 8)) return -1;
    zonos2_sampler smp(sp, ncb, av);
    std::vector<float> c((size_t) ncb * av), u(c.size()), g(c.size());
    zonos2_slot a, b;
    a.index = 0; a.active = true; a.n_past = n0;
    b.index = 1; b.active = true; b.n_past = n0;
    if (!zonos2_batch_slot_prefill(bc, 0, prompt.data(), n0, spk, spk_pos, c.data(), delta)) return -1;
    if (guided && !zonos2_batch_slot_prefill(bc, 1, prompt.data(), n0, spk, spk_pos, u.data(), nullptr)) return -1;
    int n = 0;
    while (true) {
        if (guided)
            for (size_t i = 0; i < g.size(); ++i) g[i] = u[i] + sp.emotion_cfg_scale * (c[i] - u[i]);
        zonos2_slot_sample(m, a, smp, guided ? g.data() : c.data(), codes, max_frames, {});
        ++n;
        if (a.done) break;
        b.next_ids = a.next_ids;
        std::vector<zonos2_slot *> act{&a};
        if (guided) act.push_back(&b);
        zonos2_batch_step(bc, act);
        std::memcpy(c.data(), zonos2_batch_slot_logits(bc, 0), c.size() * 4);
        if (guided) std::memcpy(u.data(), zonos2_batch_slot_logits(bc, 1), u.size() * 4);
    }
    eos = a.eos_frame;
    zonos2_batch_free(bc);
    return n;
}

// the recompute path by hand: a prefill of prompt + frames so far for every frame
int hand_recompute(const zonos2_model & m, const std::vector<float> & prompt, int n0, int max_frames,
                   const zonos2_sampling & sp, std::vector<int32_t> & codes, int & eos) {
    const int ncb = (int) m.hp.n_codebooks, av = (int) m.hp.audio_vocab;
    zonos2_batch_ctx bc;
    if (!zonos2_batch_init(bc, m, 1, n0 + max_frames)) return -1;
    zonos2_sampler smp(sp, ncb, av);
    std::vector<float> seq = prompt, lo((size_t) ncb * av);
    eos = -1;
    int countdown = -1, n = 0;
    for (int f = 0; f < max_frames; ++f) {
        if (!zonos2_batch_slot_prefill(bc, 0, seq.data(), n0 + f, nullptr, -1, lo.data())) return -1;
        std::vector<int> fr(ncb);
        for (int cb = 0; cb < ncb; ++cb) fr[cb] = smp.sample(lo.data() + (size_t) cb * av, cb);
        smp.accept(fr);
        codes.insert(codes.end(), fr.begin(), fr.end());
        ++n;
        for (int cb = 0; cb < ncb; ++cb) seq.push_back((float) fr[cb]);
        seq.push_back((float) m.hp.text_vocab);
        int last = -1;
        for (int cb = 0; cb < ncb; ++cb) if (fr[cb] == (int) m.hp.eoa_id) last = cb;
        if (eos < 0 && last >= 0) { eos = f - last > 0 ? f - last : 0; countdown = ncb + 1; }
        if (countdown > 0 && --countdown == 0) break;
    }
    zonos2_batch_free(bc);
    return n;
}

} // namespace

int main(int argc, char ** argv) {
    if (argc < 2) { fprintf(stderr, "usage: generate_kat model.gguf\n"); return 2; }
    zonos2_model m;
    if (!zonos2_model_load(m, argv[1], true)) return 1;
    const int ncb = (int) m.hp.n_codebooks, W = ncb + 1, n0 = 12, max_frames = 24;
    const std::vector<float> prompt = prompt_rows(m, n0, 3);
    const std::vector<float> spk = normal_vec(m.hp.spk_dim, 4, 1.0f), delta = normal_vec(m.hp.n_embd, 5, 0.5f);

    for (int greedy = 1; greedy >= 0; --greedy) {
        zonos2_sampling sp;
        sp.greedy = greedy != 0;
        sp.seed = 17;
        const char * mode = greedy ? "greedy" : "sampled";
        // KV path, no speaker
        std::vector<int32_t> c1, c2, full;
        int e1 = -2, e2 = -2;
        const int n1 = zonos2_generate(m, prompt.data(), n0, max_frames, sp, c1, e1, true, nullptr, 0, &full);
        const int n2 = hand_kv(m, prompt, n0, max_frames, sp, nullptr, 0, nullptr, c2, e2);
        printf("[%s] kv: %d frames, eos_frame %d\n", mode, n1, e1);
        expect(n1 > 0 && n1 == n2 && c1 == c2 && e1 == e2, "kv path == one-slot batch loop");
        bool ids_ok = (int) full.size() == (n0 + n1) * W;
        for (int i = 0; ids_ok && i < n0 * W; ++i) ids_ok = full[i] == (int32_t) lroundf(prompt[i]);
        for (int f = 0; ids_ok && f < n1; ++f) {
            for (int cb = 0; cb < ncb; ++cb) ids_ok = ids_ok && full[(size_t) (n0 + f) * W + cb] == c1[(size_t) f * ncb + cb];
            ids_ok = ids_ok && full[(size_t) (n0 + f) * W + ncb] == (int32_t) m.hp.text_vocab;
        }
        expect(ids_ok, "out_full_ids = prompt rows + frames + text pad");
        // guided: speaker + emotion delta + cfg scale
        sp.emotion_cfg_scale = 2.5f;
        std::vector<int32_t> g1, g2, d1;
        int ge1 = -2, ge2 = -2, de1 = -2;
        const int gn1 = zonos2_generate(m, prompt.data(), n0, max_frames, sp, g1, ge1, true, spk.data(), 0, nullptr, {}, delta.data());
        const int gn2 = hand_kv(m, prompt, n0, max_frames, sp, spk.data(), 0, delta.data(), g2, ge2);
        expect(gn1 > 0 && gn1 == gn2 && g1 == g2 && ge1 == ge2, "emotion-guided kv path == two-slot batch loop");
        // scale 1: no twin, the delta rides on the single slot
        sp.emotion_cfg_scale = 1.0f;
        const int dn1 = zonos2_generate(m, prompt.data(), n0, max_frames, sp, d1, de1, true, spk.data(), 0, nullptr, {}, delta.data());
        std::vector<int32_t> d2;
        int de2 = -2;
        const int dn2 = hand_kv(m, prompt, n0, max_frames, sp, spk.data(), 0, delta.data(), d2, de2);
        expect(dn1 > 0 && dn1 == dn2 && d1 == d2 && de1 == de2, "cfg scale 1: one slot with the delta");
        // recompute path
        std::vector<int32_t> r1, r2;
        int re1 = -2, re2 = -2;
        const int rn1 = zonos2_generate(m, prompt.data(), n0, max_frames, sp, r1, re1, false);
        const int rn2 = hand_recompute(m, prompt, n0, max_frames, sp, r2, re2);
        printf("[%s] recompute: %d frames, eos_frame %d\n", mode, rn1, re1);
        expect(rn1 > 0 && rn1 == rn2 && r1 == r2 && re1 == re2, "recompute path == prefill of the growing sequence");
        expect(std::vector<int32_t>(r1.begin(), r1.begin() + ncb) == std::vector<int32_t>(c1.begin(), c1.begin() + ncb),
               "first frame: recompute == kv (both from the prompt's prefill)");
        // on_frame stops the KV path after frame 3
        std::vector<int32_t> s1;
        int se = -2, seen = 0;
        const int sn = zonos2_generate(m, prompt.data(), n0, max_frames, sp, s1, se, true, nullptr, 0, nullptr,
                                       [&](int idx, const int32_t *, int) { seen = idx + 1; return idx < 3; });
        expect(sn == 4 && seen == 4 && std::vector<int32_t>(c1.begin(), c1.begin() + 4 * ncb) == s1, "on_frame false stops the stream");
    }
    zonos2_model_free(m);
    printf("generate KAT: %s\n", g_fail ? "FAILED" : "OK");
    return g_fail ? 1 : 0;
}
