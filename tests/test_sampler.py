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
