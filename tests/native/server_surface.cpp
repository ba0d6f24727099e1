// A caller shaped like the reference server's decode worker (src/server.cpp:1015-1195, 1216-1218,
// 1601): the same zonos2.h calls, struct fields and hparams, written against this repository's
// include/zonos2.h. The test compiles and links it (no device use at run time is required: the
// binary only runs when given a model path).
#include "zonos2.h"
#include "zonos2-sampler.h"

#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

namespace {

struct Request {
    std::vector<float> ids;
    int n0 = 0, spk_pos = 0;
    std::unique_ptr<zonos2_sampler> smp;
    zonos2_slot slot;
    std::vector<float> logits;
    std::vector<int32_t> codes;
};

// warm-up over the decode-width ladder, as a server does before taking traffic
void warm(zonos2_batch_ctx & bc, const zonos2_model & m) {
    std::vector<float> prompt((size_t) 16 * bc.W, 0.0f), lo((size_t) bc.av * bc.ncb);
    for (const auto & g : bc.dec_ladder) {
        zonos2_slot s;
        s.index = g.width - 1; s.active = true; s.n_past = 16;
        s.next_ids.assign(bc.W, 0);
        if (!zonos2_batch_slot_prefill(bc, s.index, prompt.data(), 16, nullptr, 0, lo.data())) return;
        std::vector<zonos2_slot *> one{&s};
        zonos2_batch_step(bc, one);
    }
    (void) m;
}

int serve(const char * path, const std::string & text) {
    zonos2_model m;
    if (!zonos2_model_load(m, path, true)) return 1;
    std::printf("backend: %s\n", zonos2_backend_name(m));
    const zonos2_hparams & hp = m.hp;
    std::printf("spk_dim %u n_embd %u ncb %u av %u rate buckets %u quality features %zu\n", hp.spk_dim, hp.n_embd,
                hp.n_codebooks, hp.audio_vocab, hp.cond_speaking_rate_buckets, hp.cond_quality_bucket_counts.size());
    zonos2_batch_ctx bc;
    if (!zonos2_batch_init(bc, m, 4, 512)) return 1;
    warm(bc, m);
    zonos2_prompt_options opt;
    opt.add_speaker_slot = true;
    opt.quality_buckets.assign(hp.cond_quality_bucket_counts.size(), -1);
    Request r;
    int n_rows = 0, spk_pos = -1;
    const std::vector<int32_t> ids = zonos2_build_prompt(m, text, opt, n_rows, spk_pos);
    r.ids.assign(ids.begin(), ids.end());
    r.n0 = n_rows;
    r.spk_pos = spk_pos >= 0 ? spk_pos : 0;
    zonos2_sampling sp;
    sp.seed = 7;
    r.smp = std::make_unique<zonos2_sampler>(sp, (int) hp.n_codebooks, (int) hp.audio_vocab);
    r.slot.index = 0; r.slot.active = true; r.slot.n_past = r.n0;
    r.logits.resize((size_t) bc.av * bc.ncb);
    std::vector<float> spk(hp.spk_dim, 0.0f), delta(hp.n_embd, 0.0f);
    if (!zonos2_batch_slot_prefill(bc, 0, r.ids.data(), r.n0, spk.data(), r.spk_pos, r.logits.data(), delta.data())) return 1;
    zonos2_slot_sample(m, r.slot, *r.smp, r.logits.data(), r.codes, 64, {});
    while (!r.slot.done) {
        std::vector<zonos2_slot *> active{&r.slot};
        zonos2_batch_step(bc, active);
        std::memcpy(r.logits.data(), zonos2_batch_slot_logits(bc, 0), r.logits.size() * sizeof(float));
        zonos2_slot_sample(m, r.slot, *r.smp, r.logits.data(), r.codes, 64,
                           [](int, const int32_t *, int) { return true; });
    }
    zonos2_batch_free(bc);
    zonos2_model_free(m);
    return 0;
}

} // namespace

int main(int argc, char ** argv) {
    if (argc < 2) { std::printf("usage: server_surface model.gguf [text]\n"); return 0; }
    return serve(argv[1], argc > 2 ? argv[2] : "hello");
}
