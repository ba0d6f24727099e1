"""Device frame sampler (z2h_sample) against the oracle's restatement of the reference sampler.

With the same logits, settings, histories and canonical draws u, the device codes equal orc_sample's
with exp_mode 1 (exp in double rounded to float, the device's arithmetic) on every draw; against
exp_mode 0 (std::exp on floats, the reference's arithmetic) they agree on all but a rare draw that
falls between the two roundings' cumulative sums. Logits are distinct random values, except in the
tied-logits test (equal keys in the orders of std::partial_sort / std::sort on both sides); min_p > 1
keeps no mass, so the code is the most probable candidate whatever u is."""
import numpy as np
import pytest

import oracle_py as O
from zonos2_amd import configs, synth
from zonos2_amd.z2h import Context, Z2HError, lib

pytestmark = pytest.mark.gpu

SETTINGS = [
    dict(temperature=1.15, top_k=106, top_p=0.0, min_p=0.18, rep_penalty=1.2, rep_codebooks=8, greedy=0),
    dict(temperature=0.8, top_k=0, top_p=0.9, min_p=0.0, rep_penalty=1.0, rep_codebooks=8, greedy=0),
    dict(temperature=1.0, top_k=20, top_p=0.7, min_p=0.05, rep_penalty=1.5, rep_codebooks=3, greedy=0),
    dict(temperature=0.0, top_k=50, top_p=0.0, min_p=0.0, rep_penalty=1.3, rep_codebooks=9, greedy=0),
    dict(temperature=1.0, top_k=0, top_p=0.0, min_p=0.0, rep_penalty=1.2, rep_codebooks=8, greedy=1),
    dict(temperature=1.3, top_k=1025, top_p=0.95, min_p=0.02, rep_penalty=1.1, rep_codebooks=9, greedy=0),
    dict(temperature=1.0, top_k=40, top_p=0.8, min_p=1.5, rep_penalty=1.2, rep_codebooks=8, greedy=0),   # kept mass 0
]


@pytest.fixture(scope="module")
def ctx():
    cfg, wl = configs.C1()
    c = Context(cfg.hparams(), wl.n_slots, wl.slot_cap)
    c.upload(synth.generate_model(cfg, 42))
    yield cfg, wl, c
    c.close()


def _oracle_codes(lg, sp, u, hist, hlen, exp_mode):
    n, ncb = u.shape
    return np.array([[O.sample(lg[i, cb], sp[i], cb, u[i, cb], hist[i, cb, :hlen[i, cb]], exp_mode)
                      for cb in range(ncb)] for i in range(n)], np.int32)


def test_device_sampler_matches_oracle(ctx):
    import torch
    cfg, wl, c = ctx
    n, ncb, av = wl.n_slots, cfg.n_codebooks, cfg.audio_vocab
    rng = np.random.default_rng(11)
    agree0 = total = 0
    for trial in range(24):
        print(f"trial {trial}", flush=True)
        lg = (rng.standard_normal((n, ncb, av)) * 2.5).astype(np.float32)
        lg[..., 7] += 3.0
        sp = [SETTINGS[(trial + i) % len(SETTINGS)] for i in range(n)]
        hist = rng.integers(0, av, (n, ncb, 64)).astype(np.int32)
        hist[..., ::5] = 7                                            # repeated codes: penalties stack
        hlen = rng.integers(0, 65, (n, ncb)).astype(np.int32)
        u = rng.random((n, ncb))
        d = torch.from_numpy(lg).cuda()
        torch.cuda.synchronize()
        got = c.sample(sp, u, hist, hlen, d_logits=d.data_ptr())
        want = _oracle_codes(lg, sp, u, hist, hlen, 1)
        np.testing.assert_array_equal(got, want)
        agree0 += int((got == _oracle_codes(lg, sp, u, hist, hlen, 0)).sum())
        total += got.size
    assert agree0 >= total - 2


def test_device_sampler_tied_logits_and_zero_mass(ctx):
    """Equal keys: logits on a coarse grid (runs of equal logits, so equal probabilities, at the top-k
    cut, at the top and inside the walk) and logits one ulp apart (distinct logits whose exp terms
    round to equal probabilities). The reference orders such keys as std::partial_sort / std::sort
    leave them, and so does orc_sample (it calls them): device == oracle on every code. With
    min_p > 1 (no kept mass) the code is the first id of the probability order for any u."""
    import torch
    cfg, wl, c = ctx
    n, ncb, av = wl.n_slots, cfg.n_codebooks, cfg.audio_vocab
    rng = np.random.default_rng(13)
    no_hist = np.zeros((n, ncb, 1), np.int32), np.zeros((n, ncb), np.int32)
    tied = SETTINGS + [dict(temperature=1.0, top_k=1, top_p=0.0, min_p=0.0, rep_penalty=1.0, rep_codebooks=0, greedy=0),
                       dict(temperature=1.0, top_k=3, top_p=0.5, min_p=0.0, rep_penalty=1.0, rep_codebooks=0, greedy=0)]
    for trial in range(12):
        print(f"tied trial {trial}", flush=True)
        if trial % 2 == 0:
            lg = (np.round(rng.standard_normal((n, ncb, av)) * 2.0) * 0.5).astype(np.float32)
        else:
            lg = (rng.standard_normal((n, ncb, av)) * 0.3).astype(np.float32)
            src = rng.integers(0, av, (n, ncb, av // 2))
            dst = rng.integers(0, av, (n, ncb, av // 2))
            for i in range(n):
                for cb in range(ncb):
                    lg[i, cb, dst[i, cb]] = np.nextafter(lg[i, cb, src[i, cb]], np.float32(np.inf))
        sp = [tied[(trial + i) % len(tied)] for i in range(n)]
        u = rng.random((n, ncb))
        d = torch.from_numpy(lg).cuda()
        torch.cuda.synchronize()
        got = c.sample(sp, u, d_logits=d.data_ptr())
        np.testing.assert_array_equal(got, _oracle_codes(lg, sp, u, *no_hist, 1))
    zero = SETTINGS[-1]
    assert zero["min_p"] > 1
    lg = (rng.standard_normal((n, ncb, av)) * 2.5).astype(np.float32)
    d = torch.from_numpy(lg).cuda()
    torch.cuda.synchronize()
    a = c.sample([zero] * n, rng.random((n, ncb)), d_logits=d.data_ptr())
    b = c.sample([zero] * n, rng.random((n, ncb)), d_logits=d.data_ptr())
    np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(a, lg.argmax(axis=2))                 # temperature 1, no history


def test_device_sampler_on_step_logits(ctx):
    cfg, wl, c = ctx
    n = wl.n_slots
    rng = np.random.default_rng(12)
    emb = rng.standard_normal((n, cfg.n_embd)).astype(np.float32)
    logits = c.step(np.arange(n), np.array(wl.kv_lens[:n]), emb=emb).reshape(n, cfg.n_codebooks, cfg.audio_vocab)
    sp = [SETTINGS[0]] * n
    u = rng.random((n, cfg.n_codebooks))
    got = c.sample(sp, u)                                             # the last step's logits, no history
    hist = np.zeros((n, cfg.n_codebooks, 1), np.int32)
    hlen = np.zeros((n, cfg.n_codebooks), np.int32)
    np.testing.assert_array_equal(got, _oracle_codes(logits, sp, u, hist, hlen, 1))
    greedy = c.sample([SETTINGS[4]] * n, u)
    np.testing.assert_array_equal(greedy, logits.argmax(axis=2))


def test_resident_decode_loop_matches_host_loop():
    """Device-resident tables: z2h_sample_feed + z2h_step_resident for 12 frames gives the same codes
    (and K/V rows) as host steps fed with the same codes (next ids = codes + the text pad, n_past + 1)
    and z2h_sample on their logits, with the same draws."""
    cfg, wl = configs.C1()
    model = synth.generate_model(cfg, 43)
    n, ncb, W = wl.n_slots, cfg.n_codebooks, cfg.n_codebooks + 1
    a = Context(cfg.hparams(), wl.n_slots, wl.slot_cap); a.upload(model)
    b = Context(cfg.hparams(), wl.n_slots, wl.slot_cap); b.upload(model)
    rng = np.random.default_rng(21)
    slots = np.arange(n)
    npast = np.array([3, 17, 40, 9], np.int32)[:n]
    ids = np.concatenate([rng.integers(0, cfg.audio_vocab, (n, ncb)), np.full((n, 1), cfg.text_vocab)], axis=1).astype(np.int32)
    sp = [SETTINGS[i % 4] for i in range(n)]
    a.step(slots, npast, ids=ids)
    b.step(slots, npast, ids=ids)
    for f in range(12):
        print(f"frame {f}", flush=True)
        u = rng.random((n, ncb))
        ca = a.sample_feed(sp, u)
        cb_ = b.sample(sp, u)
        np.testing.assert_array_equal(ca, cb_)
        npast = npast + 1
        a.step_resident(n)
        b.step(slots, npast, ids=np.concatenate([cb_, np.full((n, 1), cfg.text_vocab, np.int32)], axis=1))
    u = rng.random((n, ncb))
    np.testing.assert_array_equal(a.sample(sp, u), b.sample(sp, u))
    for L in range(cfg.n_layer):
        for s in range(n):
            ka, va = a.kv_read(L, s, 0, int(npast[s]) + 1)
            kb, vb = b.kv_read(L, s, 0, int(npast[s]) + 1)
            np.testing.assert_array_equal(ka, kb)
            np.testing.assert_array_equal(va, vb)
    with pytest.raises(Exception):
        a.step_resident(n)                                           # the tables were consumed
    a.close(); b.close()


def test_resident_steps_stop_at_slot_capacity():
    """The device-resident loop (z2h_sample_feed advances n_past on the GPU) must refuse a step whose
    fed row would be the slot's row S (past its band, i.e. row 0 of the next KV head's band or past the
    cache), before any launch, as z2h_step refuses it: the last valid row S - 1 steps, row S raises,
    and no band's row 0 changes."""
    cfg, wl = configs.C1()
    model = synth.generate_model(cfg, 46)
    n, ncb = wl.n_slots, cfg.n_codebooks
    c = Context(cfg.hparams(), n, wl.slot_cap)
    c.upload(model)
    S = lib().z2h_slot_cap(c.ctx)
    rng = np.random.default_rng(5)
    for L in range(cfg.n_layer):
        for s in range(n):
            k, v = synth.kv_rows(cfg, L, s, S - 3, 9)
            c.kv_write(L, s, 0, k, v)
    row0 = [[c.kv_read(L, s, 0, 1) for s in range(n)] for L in range(cfg.n_layer)]
    slots = np.arange(n, dtype=np.int32)
    npast = np.full(n, S - 3, np.int32)
    ids = np.concatenate([rng.integers(0, cfg.audio_vocab, (n, ncb)), np.full((n, 1), cfg.text_vocab)], axis=1).astype(np.int32)
    sp = [SETTINGS[i % 4] for i in range(n)]
    c.step(slots, npast, ids=ids)                                  # row S - 3
    for f in range(2):                                             # rows S - 2, S - 1
        c.sample_feed(sp, rng.random((n, ncb)))
        c.step_resident(n)
    c.sample_feed(sp, rng.random((n, ncb)))                        # the tables now hold row S
    with pytest.raises(Z2HError) as e:
        c.step_resident(n)
    assert "slot full" in str(e.value)
    for L in range(cfg.n_layer):
        for s in range(n):
            k0, v0 = c.kv_read(L, s, 0, 1)
            assert np.array_equal(k0, row0[L][s][0]) and np.array_equal(v0, row0[L][s][1]), f"row 0 of layer {L} slot {s} changed"
    # the context stays usable: a host step at valid rows runs
    c.step(slots, np.full(n, 5, np.int32), ids=ids)
    c.close()
