// Drives zonos2_sampler over a logits file: argv = path steps ncb vocab seed greedy temperature
// top_k top_p min_p rep_penalty rep_window rep_codebooks. Prints one line of ncb codes per step
// (each frame is accepted into the history before the next step).
#include "zonos2-sampler.h"

#include <cstdio>
#include <cstdlib>
#include <vector>

int main(int argc, char ** argv) {
    if (argc != 14) return 2;
    const int steps = std::atoi(argv[2]), ncb = std::atoi(argv[3]), vocab = std::atoi(argv[4]);
    zonos2_sampling sp;
    sp.seed = (uint32_t) std::strtoul(argv[5], nullptr, 10);
    sp.greedy = std::atoi(argv[6]) != 0;
    sp.temperature = std::strtof(argv[7], nullptr);
    sp.top_k = std::atoi(argv[8]);
    sp.top_p = std::strtof(argv[9], nullptr);
    sp.min_p = std::strtof(argv[10], nullptr);
    sp.rep_penalty = std::strtof(argv[11], nullptr);
    sp.rep_window = std::atoi(argv[12]);
    sp.rep_codebooks = std::atoi(argv[13]);
    std::vector<float> lg((size_t) steps * ncb * vocab);
    FILE * f = std::fopen(argv[1], "rb");
    if (!f || std::fread(lg.data(), 4, lg.size(), f) != lg.size()) return 3;
    std::fclose(f);
    zonos2_sampler smp(sp, ncb, vocab);
    for (int s = 0; s < steps; ++s) {
        std::vector<int> frame(ncb);
        for (int cb = 0; cb < ncb; ++cb) frame[cb] = smp.sample(&lg[((size_t) s * ncb + cb) * vocab], cb);
        smp.accept(frame);
        for (int cb = 0; cb < ncb; ++cb) std::printf("%d%c", frame[cb], cb + 1 < ncb ? ' ' : '\n');
    }
    return 0;
}
