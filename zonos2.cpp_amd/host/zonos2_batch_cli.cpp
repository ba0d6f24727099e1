// zonos2-batch — command-line harness of the batched decode API (include/zonos2.h).
//
//   --info           print the GGUF's hyperparameters and tensor table as JSON (no device use)
//   --decode-bench   the reference's decode-throughput probe (src/main.cpp:107-156): prefill n_slots
//                    identical prompts, 8 warm-up steps, then time --steps batched steps with greedy
//                    feedback; prints aggregate frames/s
//   --batch-test     the reference's batched-decode validation (src/main.cpp:158-285): every request
//                    is decoded alone (a one-slot context: the reference's single-sequence KV path is
//                    its batch runtime at one slot) and inside one shared batch with idle slots; the
//                    codes are compared per frame. F.1 (one slot, greedy) must be exact; F.2 (identical
//                    prompts in two slots) must match.
// Prompts are seeded random id rows of --prompt-len frames (the text prompt builder is not part of
// this library); --requests R gives R prompts, request i reusing prompt i % 2 when --dup is set.
// --gpu-sample samples the batched run's frames on the GPU from the step's logits
// (zonos2_batch_sample) instead of the host sampler; --sampled makes --decode-bench use the default
// sampling settings instead of greedy feedback.
#include "zonos2.h"
#include "zonos2-sampler.h"

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <random>
#include <string>
#include <vector>

namespace {

struct Args {
    std::string model;
    bool info = false, bench = false, test = false, greedy = false, dup = false;
    bool gpu_sample = false;          // sample on the GPU from the step's logits (zonos2_batch_sample)
    bool sampled = false;             // decode-bench: default sampling settings instead of greedy
    int slots = 0, steps = 64, max_frames = 48, prompt_len = 32, requests = 3;
    uint32_t seed = 1;
};

int usage() {
    fprintf(stderr, "usage: zonos2-batch --model F.gguf (--info | --decode-bench | --batch-test)\n"
                    "       [--slots N] [--steps K] [--max-frames M] [--prompt-len N0] [--requests R]\n"
                    "       [--greedy] [--dup] [--seed S] [--gpu-sample] [--sampled]\n");
    return 2;
}

std::vector<float> make_prompt(const zonos2_model & m, int n0, uint32_t seed) {
    const int ncb = (int) m.hp.n_codebooks, W = ncb + 1;
    std::mt19937 rng(seed);
    std::vector<float> ids((size_t) n0 * W);
    for (int t = 0; t < n0; ++t) {
        for (int k = 0; k < ncb; ++k) ids[(size_t) t * W + k] = (float) (rng() % m.hp.codebook_size);
        ids[(size_t) t * W + ncb] = (float) (rng() % (m.hp.text_vocab + 1));
    }
    return ids;
}

int run_info(const Args & a) {
    zonos2_model m;
    if (!zonos2_model_read_meta(m, a.model.c_str())) return 1;
    const auto & h = m.hp;
    printf("{\"hparams\": {\"n_layer\": %u, \"n_embd\": %u, \"head_dim\": %u, \"n_head\": %u, \"n_head_kv\": %u, "
           "\"n_ff\": %u, \"n_expert\": %u, \"n_ctx_train\": %u, \"rope_freq_base\": %.9g, \"rms_eps\": %.9g, "
           "\"qk_norm_eps\": %.9g, \"logit_softcap\": %.9g, \"n_codebooks\": %u, \"codebook_size\": %u, "
           "\"audio_vocab\": %u, \"eoa_id\": %u, \"audio_pad_id\": %u, \"text_vocab\": %u, \"spk_dim\": %u, "
           "\"spk_lda_dim\": %u, \"expert_used\": [",
           h.n_layer, h.n_embd, h.head_dim, h.n_head, h.n_head_kv, h.n_ff, h.n_expert, h.n_ctx_train,
           h.rope_freq_base, h.rms_eps, h.qk_norm_eps, h.logit_softcap, h.n_codebooks, h.codebook_size,
           h.audio_vocab, h.eoa_id, h.audio_pad_id, h.text_vocab, h.spk_dim, h.spk_lda_dim);
    for (size_t i = 0; i < h.expert_used.size(); ++i) printf("%s%d", i ? ", " : "", h.expert_used[i]);
    printf("]}, \"router_dim\": %d, \"tensors\": {", m.router_dim);
    bool first = true;
    for (const auto & t : m.tensors) {
        printf("%s\"%s\": [", first ? "" : ", ", t.first.c_str());
        for (size_t i = 0; i < t.second.size(); ++i) printf("%s%lld", i ? ", " : "", (long long) t.second[i]);
        printf("]");
        first = false;
    }
    printf("}}\n");
    return 0;
}

int run_decode_bench(zonos2_model & m, const Args & a) {
    const int ncb = (int) m.hp.n_codebooks, av = (int) m.hp.audio_vocab;
    const int n_slots = std::max(1, a.slots), n_steps = a.steps, n0 = a.prompt_len;
    const std::vector<float> idf = make_prompt(m, n0, a.seed);
    zonos2_batch_ctx bc;
    if (!zonos2_batch_init(bc, m, n_slots, n0 + n_steps + 16)) { fprintf(stderr, "decode-bench: batch init failed\n"); return 1; }
    zonos2_sampling sp; sp.greedy = !a.sampled; sp.seed = a.seed;
    std::vector<zonos2_sampler> smp(n_slots, zonos2_sampler(sp, ncb, av));
    std::vector<zonos2_slot> slots(n_slots);
    std::vector<std::vector<float>> lo(n_slots, std::vector<float>((size_t) av * ncb));
    std::vector<int32_t> sink;
    std::vector<zonos2_slot *> active(n_slots);
    for (int i = 0; i < n_slots; ++i) {
        slots[i] = zonos2_slot{}; slots[i].index = i; slots[i].active = true; slots[i].n_past = n0;
        if (!zonos2_batch_slot_prefill(bc, i, idf.data(), n0, nullptr, 0, lo[i].data())) {
            fprintf(stderr, "decode-bench: prefill slot %d failed\n", i); zonos2_batch_free(bc); return 1;
        }
        active[i] = &slots[i];
    }
    // a frame = sampling (host: from the copied logits; --gpu-sample: on the GPU from the step's
    // logits) + one batched step
    std::vector<zonos2_sampler *> smp_p(n_slots);
    std::vector<std::vector<int32_t> *> sink_p(n_slots, &sink);
    for (int i = 0; i < n_slots; ++i) smp_p[i] = &smp[i];
    for (int i = 0; i < n_slots; ++i) zonos2_slot_sample(m, slots[i], smp[i], lo[i].data(), sink, n_steps + n0 + 32, {});
    bc.device_sampling = a.gpu_sample;
    bool ok = true;
    auto step_once = [&]() {
        for (int i = 0; i < n_slots; ++i) slots[i].done = false;
        zonos2_batch_step(bc, active);
        if (a.gpu_sample) {
            ok = ok && zonos2_batch_sample(bc, active, smp_p, sink_p, n_steps + n0 + 32, {});
        } else {
            for (int i = 0; i < n_slots; ++i) {
                std::memcpy(lo[i].data(), zonos2_batch_slot_logits(bc, i), (size_t) av * ncb * sizeof(float));
                zonos2_slot_sample(m, slots[i], smp[i], lo[i].data(), sink, n_steps + n0 + 32, {});
            }
        }
        sink.clear();
    };
    for (int w = 0; w < 8; ++w) step_once();
    const auto t0 = std::chrono::steady_clock::now();
    for (int s = 0; s < n_steps; ++s) step_once();
    const double dt = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    const double fps = (double) n_slots * n_steps / dt;
    if (!ok) { zonos2_batch_free(bc); return 1; }
    printf("decode-bench: slots=%d steps=%d  %.3fs  %.0f frames/s  %.1fx real-time  (%.1f frames/s/slot)  [%s, sampling on the %s]\n",
           n_slots, n_steps, dt, fps, fps / (44100.0 / 512.0), fps / n_slots, sp.greedy ? "greedy" : "sampled",
           a.gpu_sample ? "GPU" : "host");
    zonos2_batch_free(bc);
    return 0;
}

// one request decoded in a context of its own (the single-sequence path)
std::vector<int32_t> decode_alone(zonos2_model & m, const std::vector<float> & idf, int n0, int max_frames,
                                  const zonos2_sampling & sp, int & eos) {
    const int ncb = (int) m.hp.n_codebooks, av = (int) m.hp.audio_vocab;
    std::vector<int32_t> codes;
    zonos2_batch_ctx bc;
    if (!zonos2_batch_init(bc, m, 1, n0 + max_frames)) return codes;
    zonos2_sampler smp(sp, ncb, av);
    zonos2_slot s; s.index = 0; s.active = true; s.n_past = n0;
    std::vector<float> lo((size_t) av * ncb);
    if (!zonos2_batch_slot_prefill(bc, 0, idf.data(), n0, nullptr, 0, lo.data())) { zonos2_batch_free(bc); return codes; }
    std::vector<zonos2_slot *> one{&s};
    for (;;) {
        zonos2_slot_sample(m, s, smp, lo.data(), codes, max_frames, {});
        if (s.done) break;
        zonos2_batch_step(bc, one);
        std::memcpy(lo.data(), zonos2_batch_slot_logits(bc, 0), lo.size() * sizeof(float));
    }
    eos = s.eos_frame;
    zonos2_batch_free(bc);
    return codes;
}

int run_batch_test(zonos2_model & m, const Args & a) {
    const int ncb = (int) m.hp.n_codebooks, av = (int) m.hp.audio_vocab;
    const int n_req = std::max(1, a.requests), n_slots = std::max(n_req, a.slots);
    zonos2_sampling sp;
    sp.greedy = a.greedy;
    sp.seed = a.seed;
    struct Job {
        std::vector<float> idf;
        int n0 = 0, prompt_id = 0, eos_frame = -1;
        std::unique_ptr<zonos2_sampler> smp;
        zonos2_slot slot;
        std::vector<float> logits;
        std::vector<int32_t> codes;
    };
    std::vector<Job> jobs(n_req);
    int max_n0 = 0;
    for (int i = 0; i < n_req; ++i) {
        jobs[i].prompt_id = a.dup ? i % 2 : i;
        jobs[i].n0 = a.prompt_len + (a.dup ? 0 : 3 * i);            // ragged unless duplicated
        jobs[i].idf = make_prompt(m, jobs[i].n0, a.seed + 101u * (uint32_t) jobs[i].prompt_id);
        max_n0 = std::max(max_n0, jobs[i].n0);
    }
    std::vector<std::vector<int32_t>> ref(n_req);
    std::vector<int> ref_eos(n_req, -1);
    for (int i = 0; i < n_req; ++i) ref[i] = decode_alone(m, jobs[i].idf, jobs[i].n0, a.max_frames, sp, ref_eos[i]);

    zonos2_batch_ctx bc;
    if (!zonos2_batch_init(bc, m, n_slots, max_n0 + a.max_frames)) { fprintf(stderr, "batch-test: batch init failed\n"); return 1; }
    for (int i = 0; i < n_req; ++i) {
        Job & j = jobs[i];
        j.smp = std::make_unique<zonos2_sampler>(sp, ncb, av);
        j.slot = zonos2_slot{}; j.slot.index = i; j.slot.active = true; j.slot.n_past = j.n0;
        j.logits.assign((size_t) av * ncb, 0.0f);
        if (!zonos2_batch_slot_prefill(bc, i, j.idf.data(), j.n0, nullptr, 0, j.logits.data())) {
            j.slot.done = true;
            fprintf(stderr, "batch-test: prefill slot %d failed\n", i);
        }
    }
    // the first frame comes from the prefill logits on the host; later frames are sampled on the host
    // from the step's logits, or on the GPU (--gpu-sample) straight after the step
    bc.device_sampling = a.gpu_sample;
    for (Job & j : jobs) {
        if (!j.slot.active || j.slot.done) continue;
        zonos2_slot_sample(m, j.slot, *j.smp, j.logits.data(), j.codes, a.max_frames, {});
        j.eos_frame = j.slot.eos_frame;
    }
    for (;;) {
        std::vector<zonos2_slot *> list;
        for (Job & j : jobs) if (j.slot.active && !j.slot.done) list.push_back(&j.slot);
        if (list.empty()) break;
        zonos2_batch_step(bc, list);
        if (a.gpu_sample) {
            std::vector<zonos2_sampler *> smps;
            std::vector<std::vector<int32_t> *> outs;
            for (zonos2_slot * s : list) { smps.push_back(jobs[s->index].smp.get()); outs.push_back(&jobs[s->index].codes); }
            if (!zonos2_batch_sample(bc, list, smps, outs, a.max_frames, {})) { zonos2_batch_free(bc); return 1; }
        } else {
            for (zonos2_slot * s : list) {
                Job & j = jobs[s->index];
                std::memcpy(j.logits.data(), zonos2_batch_slot_logits(bc, s->index), (size_t) av * ncb * sizeof(float));
                zonos2_slot_sample(m, j.slot, *j.smp, j.logits.data(), j.codes, a.max_frames, {});
            }
        }
        for (zonos2_slot * s : list) jobs[s->index].eos_frame = s->eos_frame;
    }
    printf("\n=== batch-test: %d requests in %d slots, %s%s, max=%d ===\n", n_req, n_slots, sp.greedy ? "greedy" : "sampling",
           a.gpu_sample ? " on the GPU" : "", a.max_frames);
    int fails = 0, exact_all = 1;
    for (int i = 0; i < n_req; ++i) {
        const auto & b = jobs[i].codes;
        const auto & r = ref[i];
        const int nb = (int) b.size() / ncb, nr = (int) r.size() / ncb, cmp = std::min(nb, nr);
        int first_div = -1, agree = 0;
        for (int f = 0; f < cmp; ++f) {
            bool eq = true;
            for (int cb = 0; cb < ncb; ++cb) if (b[(size_t) f * ncb + cb] != r[(size_t) f * ncb + cb]) { eq = false; break; }
            if (eq) ++agree; else if (first_div < 0) first_div = f;
        }
        const bool exact = nb == nr && agree == cmp && nr > 0;
        exact_all &= exact ? 1 : 0;
        printf("  req %d (prompt %d, n0=%d): batch=%d(eos=%d) ref=%d(eos=%d)  agree=%d/%d first_div=%d %s\n",
               i, jobs[i].prompt_id, jobs[i].n0, nb, jobs[i].eos_frame, nr, ref_eos[i], agree, cmp, first_div, exact ? "EXACT" : "");
        if (n_slots == 1 && sp.greedy && !exact) ++fails;            // F.1
    }
    for (int i = 0; i < n_req; ++i)
        for (int k = i + 1; k < n_req; ++k)
            if (jobs[i].prompt_id == jobs[k].prompt_id && jobs[i].n0 == jobs[k].n0) {
                const bool same = jobs[i].codes == jobs[k].codes;
                printf("  F.2 slots %d,%d identical prompt -> %s\n", i, k, same ? "MATCH" : "MISMATCH");
                if (!same) ++fails;
            }
    printf("  batch == alone for every request: %s\n", exact_all ? "yes" : "no");
    zonos2_batch_free(bc);
    printf("batch-test: %s\n", fails ? "FAIL" : "OK");
    return fails ? 1 : 0;
}

} // namespace

int main(int argc, char ** argv) {
    Args a;
    for (int i = 1; i < argc; ++i) {
        const std::string s = argv[i];
        auto next = [&]() -> const char * { return i + 1 < argc ? argv[++i] : nullptr; };
        const char * v = nullptr;
        if (s == "--model" && (v = next())) a.model = v;
        else if (s == "--info") a.info = true;
        else if (s == "--decode-bench") a.bench = true;
        else if (s == "--batch-test") a.test = true;
        else if (s == "--greedy") a.greedy = true;
        else if (s == "--dup") a.dup = true;
        else if (s == "--gpu-sample") a.gpu_sample = true;
        else if (s == "--sampled") a.sampled = true;
        else if (s == "--slots" && (v = next())) a.slots = std::atoi(v);
        else if (s == "--steps" && (v = next())) a.steps = std::atoi(v);
        else if (s == "--max-frames" && (v = next())) a.max_frames = std::atoi(v);
        else if (s == "--prompt-len" && (v = next())) a.prompt_len = std::atoi(v);
        else if (s == "--requests" && (v = next())) a.requests = std::atoi(v);
        else if (s == "--seed" && (v = next())) a.seed = (uint32_t) std::strtoul(v, nullptr, 10);
        else return usage();
    }
    if (a.model.empty() || (a.info + a.bench + a.test) != 1) return usage();
    if (a.info) return run_info(a);
    zonos2_model m;
    if (!zonos2_model_load(m, a.model.c_str(), true)) return 1;
    const int rc = a.bench ? run_decode_bench(m, a) : run_batch_test(m, a);
    zonos2_model_free(m);
    return rc;
}
