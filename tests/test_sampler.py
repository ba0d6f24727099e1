"""Host frame sampler (zonos2_sampler, the reference's src/zonos2-sampler.cpp:5-77) against an
independent Python restatement of its published steps, draw for draw: numpy's MT19937 with the
legacy (init_genrand) seeding is std::mt19937, and std::uniform_real_distribution<double> is
(x1 + x2 * 2^32) / 2^64 scaled by the kept mass (generate_canonical with two 32-bit draws). Logits are
distinct random values, so the candidate and probability orders have no ties."""
import subprocess
from collections import deque
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def kat_bin(tmp_path_factory):
    out = tmp_path_factory.mktemp("sampler") / "sampler_kat"
    cmd = ["g++", "-O2", "-std=c++17", "-ffp-contract=off", f"-I{ROOT / 'include'}",
           str(ROOT / "tests" / "native" / "sampler_kat.cpp"), str(ROOT / "zonos2.cpp_amd" / "host" / "zonos2_sampler.cpp"),
           "-o", str(out)]
    subprocess.run(cmd, check=True)
    return out


class PySampler:
    def __init__(self, sp, ncb, vocab):
        self.sp, self.ncb, self.vocab = sp, ncb, vocab
        self.bg = np.random.MT19937()
        self.bg._legacy_seeding(sp["seed"])
        self.hist = [deque() for _ in range(ncb)]

    def uniform(self, hi):
        x1, x2 = (int(v) for v in self.bg.random_raw(2))
        ret = (float(x1) + float(x2) * 4294967296.0) / 18446744073709551616.0
        if ret >= 1.0:
            ret = np.nextafter(1.0, 0.0)
        return ret * (hi - 0.0) + 0.0

    def accept(self, frame):
        for cb in range(self.ncb):
            self.hist[cb].append(frame[cb])
            while len(self.hist[cb]) > self.sp["rep_window"]:
                self.hist[cb].popleft()

    def sample(self, logits, cb):
        sp, V = self.sp, self.vocab
        f32 = np.float32
        if sp["greedy"]:
            return int(np.argmax(logits))
        lg = logits.astype(f32).copy()
        rp = f32(sp["rep_penalty"])
        if rp != f32(1.0) and cb < sp["rep_codebooks"]:
            for t in self.hist[cb]:
                lg[t] = lg[t] / rp if lg[t] > 0 else lg[t] * rp
        if sp["temperature"] > 0:
            lg = (lg / f32(sp["temperature"])).astype(f32)
        k = sp["top_k"] if 0 < sp["top_k"] < V else V
        cand = list(np.argsort(-lg, kind="stable")[:k]) if k < V else list(range(V))
        mx = max(float(lg[i]) for i in cand)
        p = np.array([np.exp(np.float64(f32(lg[i] - f32(mx)))) for i in cand]).astype(f32)
        z = float(np.sum(p.astype(np.float64)))
        p = (p.astype(np.float64) / z).astype(f32)
        rank = sorted(range(len(cand)), key=lambda j: -float(p[j]))
        keep = np.ones(len(cand), bool)
        if 0 < sp["top_p"] < 1:
            c, reached = 0.0, False
            for r in rank:
                if reached:
                    keep[r] = False
                c += float(p[r])
                if c >= float(f32(sp["top_p"])):
                    reached = True
        if sp["min_p"] > 0:
            floor_p = f32(sp["min_p"]) * p[rank[0]]
            keep &= ~(p < floor_p)
        p[~keep] = 0
        mass = 0.0
        for v in p:
            mass += float(v)
        if mass <= 0:
            return int(cand[rank[0]])
        r = self.uniform(mass)
        acc = 0.0
        for j in range(len(cand)):
            acc += float(p[j])
            if acc >= r:
                return int(cand[j])
        return int(cand[rank[0]])


CASES = [
    dict(seed=0, greedy=0, temperature=1.15, top_k=106, top_p=0.0, min_p=0.18, rep_penalty=1.2, rep_window=50, rep_codebooks=8),
    dict(seed=7, greedy=0, temperature=0.8, top_k=0, top_p=0.9, min_p=0.0, rep_penalty=1.0, rep_window=50, rep_codebooks=8),
    dict(seed=123, greedy=0, temperature=1.0, top_k=20, top_p=0.7, min_p=0.05, rep_penalty=1.5, rep_window=4, rep_codebooks=3),
    dict(seed=5, greedy=1, temperature=1.0, top_k=0, top_p=0.0, min_p=0.0, rep_penalty=1.2, rep_window=50, rep_codebooks=8),
    dict(seed=9, greedy=0, temperature=1.0, top_k=40, top_p=0.8, min_p=1.5, rep_penalty=1.2, rep_window=50, rep_codebooks=8),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_sampler_draws_match_restatement(kat_bin, tmp_path, case):
    sp = CASES[case]
    steps, ncb, vocab = 12, 9, 300
    rng = np.random.default_rng(100 + case)
    lg = (rng.standard_normal((steps, ncb, vocab)) * 2.0).astype(np.float32)
    lg[:, :, 5] += 3.0                      # a popular code, so the repetition penalty has work to do
    path = tmp_path / "logits.bin"
    lg.tofile(path)
    args = [str(kat_bin), str(path), str(steps), str(ncb), str(vocab)] + [str(sp[k]) for k in
            ("seed", "greedy", "temperature", "top_k", "top_p", "min_p", "rep_penalty", "rep_window", "rep_codebooks")]
    out = subprocess.run(args, check=True, capture_output=True, text=True).stdout.split("\n")
    got = [list(map(int, line.split())) for line in out if line.strip()]
    ps = PySampler(sp, ncb, vocab)
    want = []
    for s in range(steps):
        frame = [ps.sample(lg[s, cb], cb) for cb in range(ncb)]
        ps.accept(frame)
        want.append(frame)
    assert got == want
    if sp["greedy"]:
        assert want[0] == [int(np.argmax(lg[0, cb])) for cb in range(ncb)]


@pytest.mark.parametrize("min_p", [1.0, np.nextafter(np.float32(1.0), np.float32(2.0)), 1.5, 7.0])
def test_kept_mass_is_zero_exactly_above_min_p_one(min_p):
    """The sampler takes no draw where the kept mass is 0. For finite logits the most probable
    candidate survives top-p, and min-p drops it exactly when min_p > 1 (min_p * p_max rounds above
    p_max for every float above 1): the rule the device sampling glue uses to skip a draw."""
    rng = np.random.default_rng(3)
    sp = dict(seed=4, greedy=0, temperature=0.9, top_k=0, top_p=0.6, min_p=float(np.float32(min_p)),
              rep_penalty=1.0, rep_window=8, rep_codebooks=0)
    for trial in range(40):
        ps = PySampler(sp, 1, 257)
        lg = (rng.standard_normal(257) * (0.01 if trial % 2 else 4.0)).astype(np.float32)
        before = ps.bg.state["state"]["pos"]
        code = ps.sample(lg, 0)
        drew = ps.bg.state["state"]["pos"] != before
        assert drew == (not np.float32(min_p) > 1), (trial, min_p)
        if not drew:
            assert code == int(np.argmax(lg))


def test_library_orders_match_std_sorts(tmp_path):
    """The device sampler's exact orders for equal keys (csrc/z2h_stdorder.h) against this
    toolchain's std::partial_sort and std::sort, the calls of the reference sampler
    (src/zonos2-sampler.cpp:40-58): identical permutations on keys with many equal values and on
    McIlroy-adversary inputs that drive the introsort into its heap-sort fallback."""
    out = tmp_path / "stdorder_kat"
    subprocess.run(["g++", "-O2", "-std=c++17", str(ROOT / "tests" / "native" / "stdorder_kat.cpp"), "-o", str(out)],
                   check=True)
    r = subprocess.run([str(out), "4000"], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.startswith("ok"), r.stdout
