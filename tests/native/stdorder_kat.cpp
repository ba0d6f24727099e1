// Checks z2h_order (csrc/z2h_stdorder.h) against this toolchain's std::partial_sort and std::sort, the
// calls of the reference's frame sampler, on keys with many equal values: for each case the id
// permutations must be identical. argv[1] = number of random cases. Inputs built by McIlroy's
// quicksort adversary ("A Killer Adversary for Quicksort", 1999) against std::sort itself drive the
// introsort into its depth limit, so the heap-sort fallback and the limit's value are compared too.
// Prints "ok <cases>" or the first differing case.
#include "../../zonos2.cpp_amd/csrc/z2h_stdorder.h"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

int main(int argc, char ** argv) {
    const int cases = argc > 1 ? std::atoi(argv[1]) : 2000;
    std::mt19937 rng(12345);
    for (int c = 0; c < cases; ++c) {
        // sizes from 0 to 1100 (the sampler sorts up to the audio vocabulary), key alphabets from 1
        // value (every key equal) to all distinct, and sorted / reversed runs that stress the pivots
        const int n = c < 40 ? c : (int) (rng() % 1101);
        const int alphabet = 1 + (int) (rng() % (c % 3 == 0 ? 4 : c % 3 == 1 ? 64 : 100000));
        std::vector<float> key(n);
        for (int i = 0; i < n; ++i) key[i] = (float) (rng() % alphabet) * 0.25f;
        if (c % 7 == 3) std::sort(key.begin(), key.end());
        if (c % 7 == 4) std::sort(key.begin(), key.end(), [](float a, float b) { return a > b; });
        auto before = [&key](int a, int b) { return key[a] > key[b]; };
        std::vector<int> want(n), got(n);
        for (int i = 0; i < n; ++i) want[i] = got[i] = i;
        std::sort(want.begin(), want.end(), before);
        z2h_order::sort_order(got.data(), n, before);
        if (want != got) { printf("sort differs: case %d n %d alphabet %d\n", c, n, alphabet); return 1; }
        const int k = n ? 1 + (int) (rng() % n) : 0;
        for (int i = 0; i < n; ++i) want[i] = got[i] = i;
        std::partial_sort(want.begin(), want.begin() + k, want.end(), before);
        z2h_order::partial_order(got.data(), k, n, before);
        if (want != got) { printf("partial_sort differs: case %d n %d k %d alphabet %d\n", c, n, k, alphabet); return 1; }
    }
    for (int n = 17; n <= 1100; n += (n < 200 ? 1 : 37)) {
        // the adversary freezes a "gas" key the first time two gas keys meet, keeping the pivot
        // candidate gas, so every partition peels off a constant number of keys
        const int gas = n;
        std::vector<int> val(n, gas), ids(n);
        int solid = 0, candidate = 0;
        for (int i = 0; i < n; ++i) ids[i] = i;
        auto adversary = [&](int x, int y) {
            if (val[x] == gas && val[y] == gas) val[x == candidate ? x : y] = solid++;
            if (val[x] == gas) candidate = x;
            else if (val[y] == gas) candidate = y;
            return val[x] < val[y];
        };
        std::sort(ids.begin(), ids.end(), adversary);
        // distinct keys sort to one permutation whatever the algorithm; pairs and quadruples of equal
        // keys (the adversary's keys halved / quartered) keep the bad pivots and expose the order
        for (int sh = 1; sh <= 2; ++sh) {
            auto before = [&val, sh](int a, int b) { return (val[a] >> sh) < (val[b] >> sh); };
            std::vector<int> want(n), got(n);
            for (int i = 0; i < n; ++i) want[i] = got[i] = i;
            std::sort(want.begin(), want.end(), before);
            z2h_order::sort_order(got.data(), n, before);
            if (want != got) { printf("sort differs on the adversary's input: n %d shift %d\n", n, sh); return 1; }
        }
    }
    printf("ok %d\n", cases);
    return 0;
}
