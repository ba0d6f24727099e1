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


def router_bias(model, layer):
    """router_bias of an MoE layer (added to the probabilities for the selection, graph.cpp:215-218)."""
    return model[f"blk.{layer}.router_bias"].data.view(np.float32).astype(np.float32)


def min_topk_margin(probs, bias, k):
    """Smallest gap between the k-th and (k+1)-th selection score (probs + router_bias) over tokens."""
    sc = probs + bias[None, :]
    s = -np.sort(-sc, axis=1)
    return float((s[:, k - 1] - s[:, k]).min()) if sc.shape[1] > k else float("inf")


def explain_topk_flips(om, model, cfg, T, gpu_cap, orc_cap, label=""):
    """End-to-end runs of the device and of the oracle route some tokens differently once their
    hidden states drift apart (different summation orders in every matmul). For every MoE layer
    where the two runs' top-k ids differ, take the first differing token and the expert pair that
    swapped (one selected only by the device, one only by the oracle, or the first position where the
    orders differ) and report the oracle's selection-score margin between them, on the oracle's own
    layer input. The bound it must sit under comes from the measured hidden-state error of that layer:
    the largest selection-score movement that replacing the oracle's layer input (ffn_in and the
    threaded router state) by the device's causes, over all tokens and experts of the layer, times
    two (a pair's margin closes by at most the sum of the two movements). A flip at a margin above it
    would not be a near-tie but a routing error. gpu_cap / orc_cap: per-layer dicts of the "ffn_in"
    rows ([T][d]) and, for the device, its "sel" ([T][k]); each run's router state is threaded by
    re-running the oracle router on its own inputs, and the device's sel is checked to be the oracle
    router's on the device's input (the teacher-forced bit-exact contract). Returns the rows reported."""
    import oracle_py as O
    rows = []
    prev_g = prev_o = None
    E = cfg.n_expert
    for L in range(cfg.n_layer):
        k = cfg.expert_used[L]
        if k == 0:
            continue
        rg = O.router(om, L, gpu_cap[L]["ffn_in"], prev_g)
        ro = O.router(om, L, orc_cap[L]["ffn_in"], prev_o)
        assert np.array_equal(rg["sel"], gpu_cap[L]["sel"]), f"{label} L{L}: device routing differs from the oracle router on its input"
        bias = router_bias(model, L)
        sg, so = rg["probs"] + bias[None, :], ro["probs"] + bias[None, :]
        move = float(np.abs(sg.astype(np.float64) - so).max())
        hid = float(np.abs(gpu_cap[L]["ffn_in"].astype(np.float64) - orc_cap[L]["ffn_in"]).max())
        diff = np.flatnonzero((rg["sel"] != ro["sel"]).any(axis=1))
        if diff.size:
            t = int(diff[0])
            only_g = [e for e in rg["sel"][t] if e not in ro["sel"][t]]
            only_o = [e for e in ro["sel"][t] if e not in rg["sel"][t]]
            if only_g:
                a, b = int(only_o[0]), int(only_g[0])
            else:
                j = int(np.flatnonzero(rg["sel"][t] != ro["sel"][t])[0])
                a, b = int(ro["sel"][t][j]), int(rg["sel"][t][j])
            margin = float(so[t, a]) - float(so[t, b])
            gaps = np.diff(-np.sort(-so, axis=1), axis=1)
            rows.append((L, t, a, b, margin, 2 * move, hid, float(np.median(-gaps))))
            print(f"{label} L{L}: {diff.size} tokens route differently; first t={t}: oracle prefers {a} over {b} by "
                  f"{margin:.3e} (bound {2 * move:.3e} from max|d ffn_in| {hid:.3e}; median adjacent score gap "
                  f"{float(np.median(-gaps)):.3e})")
            assert 0.0 <= margin <= 2 * move, f"{label} L{L}: top-k flip at margin {margin:.3e} > bound {2 * move:.3e}"
        prev_g, prev_o = rg["rh"], ro["rh"]
    return rows


def check_layers_teacher_forced(ctx, om, okv, model, cfg, T, slot_idx, n_past, got, label=""):
    """Per-layer parity of a captured step: every layer's attention from the device's attn_in (the
    oracle appends its own K/V rows to okv), the router bit-exact from ffn_in, the dense FFN or the
    experts on the device's routing from ffn_in, the residual folds bit-exact, and the head from
    out_norm, each held to the full bar. Returns the worst per-layer cosine."""
    d, E = cfg.n_embd, cfg.n_expert
    rd = lambda L, n: ctx.read_capture(L, n, T)
    si, npast = np.ascontiguousarray(slot_idx, np.int32), np.ascontiguousarray(n_past, np.int32)
    prev, worst = None, 1.0
    for L in range(cfg.n_layer):
        res_in, attn_in = rd(L, "res_in").reshape(T, d), rd(L, "attn_in").reshape(T, d)
        ffn_in, attn_out, ffn_out = rd(L, "ffn_in").reshape(T, d), rd(L, "attn_out").reshape(T, d), rd(L, "ffn_out").reshape(T, d)
        ao = np.empty((T, cfg.n_head * cfg.head_dim), np.float32)
        oo = np.empty((T, d), np.float32)
        O.check(O.lib().orc_attention(om.m, okv.kv, L, T, O.ptr(si), O.ptr(npast), O.ptr(attn_in), O.ptr(ao), O.ptr(oo)))
        worst = min(worst, assert_close(f"{label} L{L} attn_out", attn_out, oo)[0])
        k = cfg.expert_used[L]
        if k:
            r = O.router(om, L, ffn_in, prev)
            sel = rd(L, "sel").ravel()[:T * k].reshape(T, k)
            assert np.array_equal(sel, r["sel"]), f"{label} L{L} top-k ids"
            assert np.array_equal(rd(L, "probs").reshape(T, E).view(np.uint32), r["probs"].view(np.uint32)), f"{label} L{L} probs"
            w = rd(L, "weights").ravel()[:T * k].reshape(T, k)
            _, out = O.experts(om, L, ffn_in, sel, w)
            prev = r["rh"]
        else:
            out = np.empty((T, d), np.float32)
            O.check(O.lib().orc_dense_ffn(om.m, L, T, O.ptr(np.ascontiguousarray(ffn_in)), O.ptr(out)))
        worst = min(worst, assert_close(f"{label} L{L} ffn_out", ffn_out, out)[0])
        if L + 1 < cfg.n_layer:
            assert np.array_equal(rd(L + 1, "res_in").reshape(T, d), ffn_out + (attn_out + res_in)), f"{label} L{L} residual fold"
    hn = ctx.read_capture(0, "out_norm", T).reshape(T, d)
    hw = model["output.weight"]
    mout = O.matmul(hw.type, hw.data, hw.ne[0], hw.ne[1], hn).astype(np.float64)
    assert_close(f"{label} head + softcap", got, cfg.logit_softcap * np.tanh(mout / cfg.logit_softcap))
    return worst
