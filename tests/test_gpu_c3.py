"""Full-size 24-layer Q4_K decode step (16 ragged requests) on the device vs the oracle.

Every layer is checked with the device's own layer inputs (teacher forcing), so the bar holds per
layer rather than after 24 layers of drift: attention from attn_in, the router from ffn_in
(bit-exact), the experts from ffn_in with the device's routing, the residual folds exactly, and the
head from the device's out_norm. End to end (the oracle's own step from the same ids and cache),
every stage, the routing and the logits are bit-identical.
"""
import numpy as np
import pytest

import oracle_py as O
from helpers import assert_close, end_to_end_stages, fill_kv, oracle_pair, report_stages
from zonos2_amd import configs, synth
from zonos2_amd.z2h import Context

pytestmark = [pytest.mark.gpu, pytest.mark.slow]


@pytest.fixture(scope="module")
def c3():
    cfg, wl = configs.C3()
    model = synth.generate_model(cfg, 42)
    ctx = Context(cfg.hparams(), wl.n_slots, wl.slot_cap)
    ctx.upload(model)
    om0, okv = oracle_pair(cfg, model, wl)
    fill_kv(cfg, wl, [ctx.kv_write, okv.write])
    bias = synth.router_biases(ctx, cfg, wl)         # load-balanced routing, also given to the oracle
    om = O.OracleModel(cfg.hparams(), model, logit_bias=bias)
    okv.model = om
    return cfg, wl, model, ctx, om, okv


def test_c3_layers_teacher_forced(c3):
    cfg, wl, model, ctx, om, okv = c3
    T, d, E, k = len(wl.kv_lens), cfg.n_embd, cfg.n_expert, cfg.top_k
    inp = synth.step_inputs(cfg, wl)
    ctx.set_capture(True)
    got = ctx.step(inp.slot_idx, inp.n_past, ids=inp.ids)
    rd = lambda L, n: ctx.read_capture(L, n, T)
    prev = None
    worst = 1.0
    for L in range(cfg.n_layer):
        res_in = rd(L, "res_in").reshape(T, d)
        attn_in = rd(L, "attn_in").reshape(T, d)
        ffn_in = rd(L, "ffn_in").reshape(T, d)
        attn_out = rd(L, "attn_out").reshape(T, d)
        ffn_out = rd(L, "ffn_out").reshape(T, d)
        # attention from the device's attn_in (the oracle appends its own new K/V row)
        ao = np.empty((T, cfg.n_head * cfg.head_dim), np.float32)
        oo = np.empty((T, d), np.float32)
        O.check(O.lib().orc_attention(om.m, okv.kv, L, T, O.ptr(inp.slot_idx), O.ptr(inp.n_past), O.ptr(attn_in),
                                      O.ptr(ao), O.ptr(oo)))
        c, _ = assert_close(f"L{L} attn_out", attn_out, oo)
        worst = min(worst, c)
        assert_close(f"L{L} attn_o", rd(L, "attn_o").reshape(T, -1), ao)
        # router bit-exact on identical input
        r = O.router(om, L, ffn_in, prev)
        sel = rd(L, "sel").reshape(T, k)
        assert np.array_equal(sel, r["sel"]), f"L{L} top-k ids"
        assert np.array_equal(rd(L, "probs").reshape(T, E).view(np.uint32), r["probs"].view(np.uint32)), f"L{L} probs"
        assert np.array_equal(rd(L, "router_state").reshape(T, -1).view(np.uint32), r["rh"].view(np.uint32)), f"L{L} rh"
        counts, offsets, perm = O.group(sel, E)
        assert np.array_equal(rd(L, "perm"), perm) and np.array_equal(rd(L, "offsets"), offsets)
        # experts with the device's routing
        w = rd(L, "weights").reshape(T, k)
        _, out = O.experts(om, L, ffn_in, sel, w)
        c, _ = assert_close(f"L{L} ffn_out", ffn_out, out)
        worst = min(worst, c)
        # residual folds are plain fp32 adds: bit-exact
        layer_res = attn_out + res_in
        if L + 1 < cfg.n_layer:
            assert np.array_equal(rd(L + 1, "res_in").reshape(T, d), ffn_out + layer_res), f"L{L} residual fold"
        prev = r["rh"]
    # output head on the device's final normalised row (teacher-forced, like every layer)
    hn = ctx.read_capture(0, "out_norm", T).reshape(T, d)
    hw = model["output.weight"]
    mout = O.matmul(hw.type, hw.data, hw.ne[0], hw.ne[1], hn).astype(np.float64)
    cap_ = cfg.logit_softcap
    assert_close("head + softcap", got, cap_ * np.tanh(mout / cap_))
    print(f"worst per-layer cos {worst:.7f}")


def test_c3_end_to_end_bit_identical(c3):
    """The whole 24-layer step, not teacher-forced: the oracle runs its own step from the same token
    ids and KV cache. Every quantized matmul, norm, RoPE, attention split and merge, router and head
    follows one fixed operation order on both sides, so every stage of every layer, the routing and
    the logits are the same bits. The captured step's logits equal the uncaptured step's."""
    cfg, wl, model, ctx, om, okv = c3
    T = len(wl.kv_lens)
    # (the oracle's step rewrites row n_past of every slot in each layer before that layer's
    # attention, so rows appended by other tests do not leak in)
    inp = synth.step_inputs(cfg, wl)
    ctx.set_capture(False)
    plain = ctx.step(inp.slot_idx, inp.n_past, ids=inp.ids)
    ctx.set_capture(True)
    got = ctx.step(inp.slot_idx, inp.n_past, ids=inp.ids)
    assert np.array_equal(plain.view(np.uint32), got.view(np.uint32)), "capture changed the step"
    want, ocap = O.step(om, okv, inp.slot_idx, inp.n_past, ids=inp.ids, capture=True)
    rows = end_to_end_stages(ctx, ocap, cfg, T)
    report_stages("C3", rows, got, want)
    for L in range(cfg.n_layer):
        assert np.array_equal(ctx.read_capture(L, "sel", T).reshape(T, -1), ocap["sel"][L]), f"L{L}: routing differs"
    assert not rows, f"first differing stage: L{rows[0][0]} {rows[0][1]}"
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), "logits differ"


def test_c3_step_deterministic_and_slot_independent(c3):
    cfg, wl, model, ctx, om, okv = c3
    inp = synth.step_inputs(cfg, wl)
    ctx.set_capture(False)
    a = ctx.step(inp.slot_idx, inp.n_past, ids=inp.ids)
    b = ctx.step(inp.slot_idx, inp.n_past, ids=inp.ids)
    assert np.array_equal(a, b)
    # a subset of the columns gives bit-identical rows (no cross-request coupling)
    sub = [3, 7, 11]
    c = ctx.step(inp.slot_idx[sub], inp.n_past[sub], ids=inp.ids[sub])
    assert np.array_equal(c, a[sub])
