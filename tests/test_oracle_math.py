"""Pins the oracle's elementwise functions, RoPE and attention against the mathematics.

exp/erf are this project's own (Cody-Waite + Taylor; Abramowitz & Stegun 7.1.26); they are
checked against the correctly rounded double-precision functions. RoPE is checked through its
defining properties (norm preservation, identity at position 0, relative-position invariance of
q.k) and attention through a float64 softmax restatement on tiny cases plus invariants.
"""
import ctypes as C
import math

import numpy as np
import pytest

import oracle_py as O
from zonos2_amd import configs, synth

L = O.lib()


def ulp_dist(a, b):
    ia = np.float32(a).view(np.int32).astype(np.int64)
    ib = np.float32(b).view(np.int32).astype(np.int64)
    return abs(int(ia) - int(ib))


def test_expf_within_2ulp():
    xs = np.concatenate([np.linspace(-87, 88, 20001), np.linspace(-1, 1, 2001), [0.0, -0.0, 1e-30, -1e-30]])
    worst = 0
    for x in xs.astype(np.float32):
        got = L.orc_expf(float(x))
        want = np.float32(math.exp(float(x)))
        worst = max(worst, ulp_dist(got, want))
    assert worst <= 2
    assert L.orc_expf(100.0) == math.inf and L.orc_expf(-110.0) == 0.0


def test_erf_abs_error():
    xs = np.linspace(-6, 6, 24001).astype(np.float32)
    err = max(abs(L.orc_erff(float(x)) - math.erf(float(x))) for x in xs)
    # A&S 7.1.26 is within 1.5e-7 in exact arithmetic; fp32 evaluation of 1 - p*exp(-x^2) near
    # |erf| = 1 adds up to ~2 ulp(1) = 2.4e-7
    assert err <= 4e-7
    assert L.orc_erff(0.0) == 0.0 and L.orc_erff(-1.0) == -L.orc_erff(1.0)


def _sincos(x):
    s, c = C.c_float(), C.c_float()
    L.orc_sincos(float(x), C.byref(s), C.byref(c))
    return s.value, c.value


def test_rope_sincos_against_double():
    # RoPE angles pos * base^(-2i/hd): every quadrant, multiples of pi/2 (the reduction's edges) and
    # large positions; the reduction is in double, the polynomials in fp32 (< 4e-9), so the error is
    # the fp32 rounding of the reduced angle and of the result: < 1.5e-7
    rng = np.random.default_rng(5)
    xs = np.concatenate([rng.uniform(0, 8192, 20000), np.arange(0, 40) * (math.pi / 4), [0.0, 1e-30, 2 ** 23]])
    worst = 0.0
    for x in xs.astype(np.float32):
        s, c = _sincos(x)
        worst = max(worst, abs(s - math.sin(float(x))), abs(c - math.cos(float(x))))
    assert worst < 1.5e-7, worst
    assert _sincos(0.0) == (0.0, 1.0)


def test_softcap_against_double_tanh():
    # cap * tanh(x / cap) for cap 15: within 2 fp32 ulps of the result over the logit range, odd,
    # exact at 0, saturating at +-cap; the small-|y| Taylor branch and the exp branch meet at 2^-10
    cap = 15.0
    xs = np.concatenate([np.linspace(-200, 200, 40001), 15 * 2.0 ** -10 * np.linspace(0.9, 1.1, 2001),
                         [1e-30, 1e-8, 3e-4]]).astype(np.float32)
    worst = 0
    for x in xs:
        got = L.orc_softcap(float(x), cap)
        want = np.float32(cap * math.tanh(float(np.float32(float(x) * np.float32(1.0 / cap)))))
        worst = max(worst, ulp_dist(got, want))
        assert L.orc_softcap(-float(x), cap) == -got
    assert worst <= 2, worst
    assert L.orc_softcap(0.0, cap) == 0.0 and L.orc_softcap(1e6, cap) == cap


def test_gelu_silu():
    for x in np.linspace(-8, 8, 1601).astype(np.float32):
        g = 0.5 * float(x) * (1 + math.erf(float(x) / math.sqrt(2)))
        assert abs(L.orc_gelu_erf(float(x)) - g) <= 3e-7 * max(1.0, abs(float(x)))
        s = float(x) / (1 + math.exp(-float(x)))
        assert abs(L.orc_silu(float(x)) - s) <= 3e-7 * max(1.0, abs(float(x)))


def _rope(x, pos, base=10000.0):
    y = np.ascontiguousarray(x, np.float32).copy()
    nh, hd = y.shape
    O.check(L.orc_rope(O.ptr(y), nh, hd, pos, base))
    return y


def test_rope_properties():
    rng = np.random.default_rng(0)
    q = rng.standard_normal((4, 128)).astype(np.float32)
    k = rng.standard_normal((4, 128)).astype(np.float32)
    assert np.array_equal(_rope(q, 0), q)                             # identity at position 0
    for p in (1, 17, 1000):
        r = _rope(q, p)
        assert np.allclose(np.linalg.norm(r, axis=1), np.linalg.norm(q, axis=1), rtol=1e-5)
    # q(p1).k(p2) depends only on p1 - p2
    d1 = (_rope(q, 40) * _rope(k, 10)).sum(1)
    d2 = (_rope(q, 130) * _rope(k, 100)).sum(1)
    assert np.allclose(d1, d2, rtol=2e-4, atol=2e-4)
    # pair (0,1) rotates by pos radians, the last pair by pos * base^(-(hd-2)/hd)
    e = np.zeros((1, 128), np.float32); e[0, 0] = 1.0
    r = _rope(e, 3)
    assert abs(r[0, 0] - math.cos(3)) < 1e-6 and abs(r[0, 1] - math.sin(3)) < 1e-6
    e = np.zeros((1, 128), np.float32); e[0, 126] = 1.0
    r = _rope(e, 3)
    th = 3 * 10000.0 ** (-126 / 128)
    assert abs(r[0, 126] - math.cos(th)) < 1e-6 and abs(r[0, 127] - math.sin(th)) < 1e-6


def _attn_model():
    cfg = configs.ModelConfig("attn-kat", n_layer=1, n_embd=256, n_head=4, n_head_kv=2, head_dim=64,
                              n_expert=4, top_k=1, n_ff=256, bulk=configs.Q8_0, router_dim=64)
    model = synth.generate_model(cfg, 3)
    return cfg, model


def test_attention_vs_float64_restatement():
    """Decode attention over ragged bands vs a float64 softmax(q.K^T / sqrt(hd)) V on the same
    f16 cache, from the step's own q (rounded to f16, as the F16-cache path does) and gate."""
    cfg, model = _attn_model()
    om = O.OracleModel(cfg.hparams(), model)
    kv = O.OracleKV(om, 2, 64)
    n_past = [5, 37]
    for s, n in enumerate(n_past):
        k, v = synth.kv_rows(cfg, 0, s, n, 11)
        kv.write(0, s, 0, k, v)
    x = np.random.default_rng(5).standard_normal((2, cfg.n_embd)).astype(np.float32)
    si = np.array([0, 1], np.int32)
    _, cap = O.step(om, kv, si, np.array(n_past, np.int32), emb=x, capture=True)
    hd, nh, grp = cfg.head_dim, cfg.n_head, cfg.n_head // cfg.n_head_kv
    for t, s in enumerate(si):
        n = n_past[t] + 1                                   # the band includes the new row
        kk, vv = kv.read(0, s, 0, n)
        kk = kk.view(np.float16).astype(np.float64)
        vv = vv.view(np.float16).astype(np.float64)
        for h in range(nh):
            g = h // grp
            q = cap["q"][0, t, h * hd:(h + 1) * hd].astype(np.float16).astype(np.float64)
            sc = kk[:, g, :] @ q / math.sqrt(hd)
            p = np.exp(sc - sc.max())
            o = (p / p.sum()) @ vv[:, g, :] * cap["gate"][0, t, h]
            got = cap["attn_o"][0, t, h * hd:(h + 1) * hd]
            assert np.allclose(got, o, rtol=1e-5, atol=1e-6), (t, h)


def test_attention_single_row_is_value():
    """With one visible row the softmax is 1: output = gate * V[0] (f16 value)."""
    cfg, model = _attn_model()
    om = O.OracleModel(cfg.hparams(), model)
    kv = O.OracleKV(om, 1, 16)
    x = np.random.default_rng(6).standard_normal((1, cfg.n_embd)).astype(np.float32)
    wl = configs.Workload("one", 1, [0], 16, inject_embeddings=True)
    _, cap = O.step(om, kv, np.array([0], np.int32), np.array([0], np.int32), emb=x, capture=True)
    vrow = kv.read(0, 0, 0, 1)[1].view(np.float16).astype(np.float32)[0]
    gate = cap["gate"][0, 0]
    for h in range(cfg.n_head):
        g = h // (cfg.n_head // cfg.n_head_kv)
        assert np.allclose(cap["attn_o"][0, 0, h * cfg.head_dim:(h + 1) * cfg.head_dim], vrow[g] * gate[h], rtol=1e-6, atol=1e-7)
