"""The oracle's frame sampler (orc_sample) and its double exp, on the CPU.

orc_exp_d is pinned against the C library's double exp (math.exp) to a few double ulps, and its
float rounding against numpy's float32(exp(x)). orc_sample is pinned draw for draw against the
independent Python restatement of the reference sampler in test_sampler.py (itself checked against
the host sampler zonos2_sampler), with the uniform draw fed in: exp_mode 1 (double exp rounded to
float, the device sampler's arithmetic) must agree on every draw; exp_mode 0 (std::exp on floats,
the reference's arithmetic) on almost every draw, since glibc's expf differs from the rounded double
exp by an ulp for about one input in ten thousand."""
import math

import numpy as np
import pytest

import oracle_py as O
from test_sampler import CASES, PySampler


def test_exp_d_against_libm():
    rng = np.random.default_rng(3)
    # normal double results (below -708.39 they are subnormal and lose relative precision)
    xs = np.concatenate([rng.uniform(-708.0, 0.0, 20000), rng.uniform(-104.0, 0.0, 20000),
                         rng.uniform(-1.0, 0.0, 20000), [0.0, -0.0, -1e-300, -0.34657359027997264, -708.39]])
    worst = 0.0
    for x in xs:
        want = math.exp(float(x))
        got = O.exp_d(float(x))
        if want == 0.0:
            assert got == 0.0
            continue
        worst = max(worst, abs(got / want - 1.0))
    assert worst < 4 * 2.0 ** -52, worst
    assert O.exp_d(-746.0) == 0.0 and O.exp_d(-float("inf")) == 0.0


def test_exp_d_rounds_to_the_float_exp():
    rng = np.random.default_rng(4)
    xs = rng.uniform(-104.0, 0.0, 50000).astype(np.float32)
    bad = sum(np.float32(O.exp_d(float(x))) != np.float32(np.exp(np.float64(x))) for x in xs)
    assert bad == 0


class FedSampler(PySampler):
    """PySampler whose draw is the given canonical u."""
    def __init__(self, sp, ncb, vocab):
        super().__init__(sp, ncb, vocab)
        self.u = None

    def uniform(self, hi):
        return self.u * (hi - 0.0) + 0.0


@pytest.mark.parametrize("case", range(len(CASES)))
def test_orc_sample_matches_restatement(case):
    sp = CASES[case]
    steps, ncb, vocab = 10, 9, 1025
    rng = np.random.default_rng(500 + case)
    lg = (rng.standard_normal((steps, ncb, vocab)) * 2.5).astype(np.float32)
    lg[:, :, 7] += 3.0
    u = rng.random((steps, ncb))
    ref = FedSampler(sp, ncb, vocab)
    agree0 = total = 0
    for s in range(steps):
        frame = []
        for cb in range(ncb):
            ref.u = float(u[s, cb])
            want = ref.sample(lg[s, cb], cb)
            hist = list(ref.hist[cb])
            got1 = O.sample(lg[s, cb], sp, cb, u[s, cb], hist, exp_mode=1)
            got0 = O.sample(lg[s, cb], sp, cb, u[s, cb], hist, exp_mode=0)
            assert got1 == want, (s, cb)
            agree0 += got0 == want
            total += 1
            frame.append(want)
        ref.accept(frame)
    assert agree0 >= total - 1


def test_orc_sample_edge_settings():
    rng = np.random.default_rng(9)
    lg = rng.standard_normal(1025).astype(np.float32)
    base = dict(temperature=1.0, top_k=0, top_p=0.0, min_p=0.0, rep_penalty=1.0, rep_codebooks=8, greedy=0)
    # u -> 0 takes the first candidate with mass; top_k = 1 is greedy on the tempered logits
    assert O.sample(lg, dict(base, top_k=1), 0, 0.999) == int(np.argmax(lg))
    assert O.sample(lg, dict(base, greedy=1), 0, 0.5) == int(np.argmax(lg))
    # min_p = 1 keeps only the most probable candidate
    assert O.sample(lg, dict(base, min_p=1.0), 0, 0.7) == int(np.argmax(lg))
    # a huge penalty on the arg-max's history pushes it out of a top-1 pick
    am = int(np.argmax(lg))
    lg2 = lg.copy(); lg2[am] = abs(lg2[am]) + 0.5
    pick = O.sample(lg2, dict(base, top_k=1, rep_penalty=1e6), 0, 0.5, hist=[am])
    assert pick != am
