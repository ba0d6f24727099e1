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


# stages of a captured decode step, in the order the step forms them
STAGES = ("res_in", "attn_in", "q", "k", "v", "gate", "attn_o", "attn_out", "ffn_in", "router_state",
          "router_logits", "probs", "sel", "weights", "ffn_out")


def end_to_end_stages(ctx, ocap, cfg, T):
    """Compare a captured device step with the oracle's end-to-end capture of the same step, stage by
    stage and layer by layer, bit for bit. Returns [(layer, stage, n_differing, max_abs_diff)] for every
    (layer, stage) whose bits differ (empty when the two runs are bit-identical), plus the out_norm row.
    Dense layers have no router stages; per-layer top-k widths may differ (the capture is [T][K])."""
    rows = []
    K = max(max(cfg.expert_used), 1)
    for L in range(cfg.n_layer):
        k = cfg.expert_used[L]
        for st in STAGES:
            if k == 0 and st in ("router_state", "router_logits", "probs", "sel", "weights"):
                continue
            g = ctx.read_capture(L, st, T)
            o = np.asarray(ocap[st][L])
            if st in ("sel", "weights"):                      # device [T][k_L], oracle [T][K]
                g, o = g.ravel()[:T * k].reshape(T, k), o.reshape(T, K)[:, :k]
            elif st in ("router_logits", "probs"):           # device [T][E_L], oracle [T][E]
                E = cfg.n_exp(L)
                g, o = g.ravel()[:T * E].reshape(T, E), o.reshape(T, -1)[:, :E]
            g, o = g.reshape(T, -1), o.reshape(T, -1)
            if g.dtype == np.float32:
                neq = g.view(np.uint32) != o.view(np.uint32)
            else:
                neq = g != o
            if neq.any():
                rows.append((L, st, int(neq.sum()), float(np.abs(g.astype(np.float64) - o).max())))
    g = ctx.read_capture(0, "out_norm", T).reshape(T, -1)
    neq = g.view(np.uint32) != np.asarray(ocap["out_norm"]).reshape(T, -1).view(np.uint32)
    if neq.any():
        rows.append((cfg.n_layer, "out_norm", int(neq.sum()), float(np.abs(g.astype(np.float64) - ocap["out_norm"].reshape(T, -1)).max())))
    return rows


def report_stages(label, rows, got, want):
    print(f"{label}: end to end, {len(rows)} (layer, stage) pairs differ from the oracle; logits "
          f"cos {cos(got, want):.7f} maxabs {np.abs(np.asarray(got, np.float64) - want).max():.3e} "
          f"bit-identical {np.array_equal(np.asarray(got).view(np.uint32), np.asarray(want).view(np.uint32))}")
    for r in rows[:12]:
        print(f"  L{r[0]} {r[1]}: {r[2]} elements differ, max |diff| {r[3]:.3e}")


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
