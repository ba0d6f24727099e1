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
//   --generate       zonos2_generate on one prompt (src/main.cpp:545-578): KV path, or --no-kv for the
//                    recompute path; --cfg S adds a seeded speaker vector and emotion delta with
//                    emotion_cfg_scale S; prints the reference's "generate:" report lines
// Prompts are seeded random id rows of --prompt-len frames (the text prompt builder is not part of
// this library); --requests R gives R prompts, request i reusing prompt i % 2 when --dup is set.
// --gpu-sample samples the batched run's frames on the GPU from the step's logits
// (zonos2_batch_sample) instead of the host sampler; --sampled makes --decode-bench use the default
// sampling settings instead of greedy feedback. --slot-cap N gives the batch-test's shared context
// slots of N frames, so requests that outgrow it must have their next step refused (exit status 3,
// "batch-test: step refused: ..."), the no-write behaviour of a full band.
#include "zonos2.h"
#include "zonos2-sampler.h"

#include <algorithm>
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
    bool generate = false, no_kv = false;
    float cfg = 1.0f;                 // generate: emotion_cfg_scale (with a seeded speaker + delta when != 1)
    int slots = 0, steps = 64, max_frames = 48, prompt_len = 32, requests = 3;
    int slot_cap = 0;                 // batch-test: slot capacity of the shared context (0: fits every request)
    uint32_t seed = 1;
};

int usage() {
    fprintf(stderr, "usage: zonos2-batch --model F.gguf (--info | --decode-bench | --batch-test | --generate)\n"
                    "       [--slots N] [--steps K] [--max-frames M] [--prompt-len N0] [--requests R]\n"
                    "       [--greedy] [--dup] [--seed S] [--gpu-sample] [--sampled] [--slot-cap N]\n"
                    "       [--no-kv] [--cfg S]\n");
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

// One request of a harness run: its prompt, sampler, slot record and the frames it produced.
struct Request {
    std::vector<float> prompt;        // [n0][W] ids as floats (the prefill API's form)
    int n0 = 0, prompt_id = 0;
    std::unique_ptr<zonos2_sampler> smp;
    zonos2_slot slot;
    std::vector<float> logits;        // [ncb][av]: the prefill's, then (host sampling) the last step's
    std::vector<int32_t> codes;
};

// A batch context and the requests living in it. Frames are produced by advance(): one batched step
// over the listed requests, then one frame each, sampled on the host from the step's logits or on the
// GPU (zonos2_batch_sample). A slot whose step is refused (its band is full) stops the run.
struct Harness {
    zonos2_model & m;
    zonos2_batch_ctx bc;
    bool gpu = false, ready = false;
    int frame_cap = 0;                // frames after which a request is cut (sampler max_frames)
    std::string refused;              // why a step was refused, if one was
    Harness(zonos2_model & model, int n_slots, int slot_cap, bool gpu_sampling, int frames) : m(model), gpu(gpu_sampling), frame_cap(frames) {
        ready = zonos2_batch_init(bc, m, n_slots, slot_cap);
        bc.device_sampling = gpu;
    }
    ~Harness() { if (ready) zonos2_batch_free(bc); }
    int ncb() const { return (int) m.hp.n_codebooks; }
    int av() const { return (int) m.hp.audio_vocab; }

    // prefill the request into slot `index` and take its first frame from the prefill logits
    bool admit(Request & r, int index, const zonos2_sampling & sp) {
        r.smp = std::make_unique<zonos2_sampler>(sp, ncb(), av());
        r.slot = zonos2_slot{};
        r.slot.index = index; r.slot.active = true; r.slot.n_past = r.n0;
        r.logits.assign((size_t) av() * ncb(), 0.0f);
        if (!zonos2_batch_slot_prefill(bc, index, r.prompt.data(), r.n0, nullptr, 0, r.logits.data())) return false;
        zonos2_slot_sample(m, r.slot, *r.smp, r.logits.data(), r.codes, frame_cap, {});
        return true;
    }

    // one step over `reqs` (their slots' done flags as the caller left them) and one frame each
    bool advance(const std::vector<Request *> & reqs) {
        std::vector<zonos2_slot *> cols;
        std::vector<int> before;
        for (Request * r : reqs) { cols.push_back(&r->slot); before.push_back(r->slot.n_past); }
        zonos2_batch_step(bc, cols);
        for (size_t i = 0; i < reqs.size(); ++i)
            if (reqs[i]->slot.n_past == before[i]) {
                refused = "slot " + std::to_string(reqs[i]->slot.index) + " at n_past " + std::to_string(before[i]) +
                          " (slot capacity " + std::to_string(bc.slot_cap) + ")";
                return false;
            }
        if (gpu) {
            std::vector<zonos2_sampler *> smps;
            std::vector<std::vector<int32_t> *> outs;
            for (Request * r : reqs) { smps.push_back(r->smp.get()); outs.push_back(&r->codes); }
            return zonos2_batch_sample(bc, cols, smps, outs, frame_cap, {});
        }
        for (Request * r : reqs) {
            const float * src = zonos2_batch_slot_logits(bc, r->slot.index);
            r->logits.assign(src, src + (size_t) av() * ncb());
            zonos2_slot_sample(m, r->slot, *r->smp, r->logits.data(), r->codes, frame_cap, {});
        }
        return true;
    }

    // frames until every request is done (or a step is refused)
    bool drain(std::vector<Request *> reqs) {
        for (;;) {
            std::vector<Request *> live;
            for (Request * r : reqs) if (r->slot.active && !r->slot.done) live.push_back(r);
            if (live.empty()) return true;
            if (!advance(live)) return false;
        }
    }
};

// decode-bench: n_slots copies of one prompt, 8 untimed frames, then --steps timed frames with the
// done flags cleared every frame (EOS is ignored, as in the reference's probe)
int run_decode_bench(zonos2_model & m, const Args & a) {
    const int n_slots = std::max(1, a.slots), n0 = a.prompt_len;
    Harness h(m, n_slots, n0 + a.steps + 16, a.gpu_sample, a.steps + n0 + 32);
    if (!h.ready) { fprintf(stderr, "decode-bench: batch init failed\n"); return 1; }
    zonos2_sampling sp; sp.greedy = !a.sampled; sp.seed = a.seed;
    std::vector<Request> reqs(n_slots);
    std::vector<Request *> all;
    for (int i = 0; i < n_slots; ++i) {
        reqs[i].n0 = n0;
        reqs[i].prompt = make_prompt(m, n0, a.seed);
        if (!h.admit(reqs[i], i, sp)) { fprintf(stderr, "decode-bench: prefill slot %d failed\n", i); return 1; }
        all.push_back(&reqs[i]);
    }
    auto frames = [&](int n) {
        for (int f = 0; f < n; ++f) {
            for (Request * r : all) { r->slot.done = false; r->codes.clear(); }
            if (!h.advance(all)) return false;
        }
        return true;
    };
    if (!frames(8)) return 1;
    const auto t0 = std::chrono::steady_clock::now();
    if (!frames(a.steps)) return 1;
    const double dt = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    const double fps = (double) n_slots * a.steps / dt;
    printf("decode-bench: slots=%d steps=%d  %.3fs  %.0f frames/s  %.1fx real-time  (%.1f frames/s/slot)  [%s, sampling on the %s]\n",
           n_slots, a.steps, dt, fps, fps / (44100.0 / 512.0), fps / n_slots, sp.greedy ? "greedy" : "sampled",
           a.gpu_sample ? "GPU" : "host");
    return 0;
}

// batch-test: every request decoded alone in a one-slot context (host sampling), then all of them in
// one shared context of max(--slots, requests) slots (idle slots stay unlisted); frames compared.
int run_batch_test(zonos2_model & m, const Args & a) {
    const int ncb = (int) m.hp.n_codebooks;
    const int n_req = std::max(1, a.requests), n_slots = std::max(n_req, a.slots);
    zonos2_sampling sp; sp.greedy = a.greedy; sp.seed = a.seed;
    auto make = [&](std::vector<Request> & v) {
        v.resize(n_req);
        for (int i = 0; i < n_req; ++i) {
            v[i].prompt_id = a.dup ? i % 2 : i;
            v[i].n0 = a.prompt_len + (a.dup ? 0 : 3 * i);              // ragged unless duplicated
            v[i].prompt = make_prompt(m, v[i].n0, a.seed + 101u * (uint32_t) v[i].prompt_id);
        }
    };
    std::vector<Request> alone, batched;
    make(alone);
    make(batched);
    int max_n0 = 0;
    for (const Request & r : batched) max_n0 = std::max(max_n0, r.n0);
    if (a.slot_cap <= 0)
        for (Request & r : alone) {
            Harness one(m, 1, r.n0 + a.max_frames, false, a.max_frames);
            if (!one.ready || !one.admit(r, 0, sp) || !one.drain({&r})) r.codes.clear();
        }
    Harness h(m, n_slots, a.slot_cap > 0 ? a.slot_cap : max_n0 + a.max_frames, a.gpu_sample, a.max_frames);
    if (!h.ready) { fprintf(stderr, "batch-test: batch init failed\n"); return 1; }
    std::vector<Request *> live;
    for (int i = 0; i < n_req; ++i) {
        if (h.admit(batched[i], i, sp)) live.push_back(&batched[i]);
        else fprintf(stderr, "batch-test: prefill slot %d failed\n", i);
    }
    if (!h.drain(live)) {
        if (!h.refused.empty()) {
            printf("batch-test: step refused: %s\n", h.refused.c_str());
            return 3;
        }
        fprintf(stderr, "batch-test: batched run failed\n");
        return 1;
    }
    if (a.slot_cap > 0) { printf("batch-test: no slot reached its capacity\n"); return 0; }
    printf("\n=== batch-test: %d requests in %d slots, %s%s, max=%d ===\n", n_req, n_slots, sp.greedy ? "greedy" : "sampling",
           a.gpu_sample ? " on the GPU" : "", a.max_frames);
    auto frame_eq = [&](const std::vector<int32_t> & x, const std::vector<int32_t> & y, int f) {
        return std::equal(x.begin() + (size_t) f * ncb, x.begin() + (size_t) (f + 1) * ncb, y.begin() + (size_t) f * ncb);
    };
    int fails = 0;
    bool all_exact = true;
    for (int i = 0; i < n_req; ++i) {
        const Request & b = batched[i], & r = alone[i];
        const int nb = (int) b.codes.size() / ncb, nr = (int) r.codes.size() / ncb, common = std::min(nb, nr);
        int same = 0, diverge = -1;
        for (int f = 0; f < common; ++f) {
            if (frame_eq(b.codes, r.codes, f)) ++same;
            else if (diverge < 0) diverge = f;
        }
        const bool exact = nr > 0 && nb == nr && same == common;
        all_exact = all_exact && exact;
        printf("  req %d (prompt %d, n0=%d): batch=%d(eos=%d) ref=%d(eos=%d)  agree=%d/%d first_div=%d %s\n",
               i, b.prompt_id, b.n0, nb, b.slot.eos_frame, nr, r.slot.eos_frame, same, common, diverge, exact ? "EXACT" : "");
        if (n_slots == 1 && sp.greedy && !exact) ++fails;             // one slot, greedy: must be exact
    }
    for (int i = 0; i < n_req; ++i)
        for (int k = i + 1; k < n_req; ++k) {
            if (batched[i].prompt_id != batched[k].prompt_id || batched[i].n0 != batched[k].n0) continue;
            const bool match = batched[i].codes == batched[k].codes;  // identical prompts: identical frames
            printf("  F.2 slots %d,%d identical prompt -> %s\n", i, k, match ? "MATCH" : "MISMATCH");
            fails += match ? 0 : 1;
        }
    printf("  batch == alone for every request: %s\n", all_exact ? "yes" : "no");
    printf("batch-test: %s\n", fails ? "FAIL" : "OK");
    return fails ? 1 : 0;
}

// generate: one request through zonos2_generate, with the reference CLI's report lines
int run_generate(zonos2_model & m, const Args & a) {
    const int ncb = (int) m.hp.n_codebooks, n0 = a.prompt_len;
    zonos2_sampling sp; sp.greedy = a.greedy; sp.seed = a.seed; sp.emotion_cfg_scale = a.cfg;
    const std::vector<float> ids = make_prompt(m, n0, a.seed);
    std::vector<float> spk, delta;
    if (a.cfg != 1.0f) {                                  // a seeded speaker vector and emotion delta
        std::mt19937 rng(a.seed + 1);
        std::normal_distribution<float> nd(0.0f, 1.0f);
        spk.resize(m.hp.spk_dim); delta.resize(m.hp.n_embd);
        for (float & x : spk) x = nd(rng);
        for (float & x : delta) x = 0.5f * nd(rng);
    }
    printf("generate: prompt [%d, %d], max=%d, %s, seed=%u, %s\n", n0, ncb + 1, a.max_frames,
           sp.greedy ? "greedy" : "sampling", sp.seed, a.no_kv ? "recompute" : "kv-cache");
    std::vector<int32_t> codes;
    int eos_frame = -1;
    const int n = zonos2_generate(m, ids.data(), n0, a.max_frames, sp, codes, eos_frame, !a.no_kv,
                                  spk.empty() ? nullptr : spk.data(), 0, nullptr, {},
                                  delta.empty() ? nullptr : delta.data());
    printf("generate: %d frames, eos_frame=%d\n", n, eos_frame);
    if (n > 0) {
        printf("  frame0:");
        for (int cb = 0; cb < ncb; ++cb) printf(" %d", codes[cb]);
        printf("\n");
    }
    return n > 0 ? 0 : 1;
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
        else if (s == "--slot-cap" && (v = next())) a.slot_cap = std::atoi(v);
        else if (s == "--generate") a.generate = true;
        else if (s == "--no-kv") a.no_kv = true;
        else if (s == "--cfg" && (v = next())) a.cfg = (float) std::atof(v);
        else return usage();
    }
    if (a.model.empty() || (a.info + a.bench + a.test + a.generate) != 1) return usage();
    if (a.info) return run_info(a);
    zonos2_model m;
    if (!zonos2_model_load(m, a.model.c_str(), true)) return 1;
    const int rc = a.bench ? run_decode_bench(m, a) : a.generate ? run_generate(m, a) : run_batch_test(m, a);
    zonos2_model_free(m);
    return rc;
}
