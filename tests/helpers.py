"""Shared test helpers: build the same synthetic model / KV / inputs for the device and the oracle."""
from __future__ import annotations

import numpy as np

import oracle_py as O
from zonos2_amd import configs, synth

# parity bar of the floating-point path: per-layer hidden states and logits reach cosine >= 0.9999
# and max |difference| <= 1e-2 against the oracle
COS_MIN = 0.9999
MAXABS = 1e-2


def cos(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / np.sqrt((a @ a) * (b @ b) + 1e-300))


def assert_close(name, got, want, cos_min=COS_MIN, maxabs=MAXABS):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (name, got.shape, want.shape)
    c, m = cos(got, want), float(np.abs(got - want).max())
    assert c >= cos_min and m <= maxabs, f"{name}: cos={c:.7f} maxabs={m:.3e}"
    return c, m


def fill_kv(cfg, wl, writers, seed=7):
    """N(0,1) f16 rows [0, n_past) of every active slot, identical for every writer."""
    for L in range(cfg.n_layer):
        for s, n in enumerate(wl.kv_lens):
            if n == 0:
                continue
            k, v = synth.kv_rows(cfg, L, s, n, seed)
            for w in writers:
                w(L, s, 0, k, v)


def oracle_pair(cfg, model, wl, logit_bias=None):
    om = O.OracleModel(cfg.hparams(), model, logit_bias=logit_bias)
    okv = O.OracleKV(om, wl.n_slots, wl.slot_cap)
    return om, okv


def min_topk_margin(probs, bias, k):
    """Smallest gap between the k-th and (k+1)-th selection score over tokens."""
    sc = probs + bias[None, :]
    s = -np.sort(-sc, axis=1)
    return float((s[:, k - 1] - s[:, k]).min()) if sc.shape[1] > k else float("inf")
