"""The 64-request configuration at full depth (the 24-layer model, KV lengths log-uniform in [16, 4096],
Zipf(1.2) expert popularity as a pre-softmax router-logit bias mirrored in the oracle, router logits
load-balanced on a calibration batch) with Q6_K and Q8_0 weights: every layer teacher-forced against
the oracle, the router bit-exact, and end to end (the oracle's own step) every stage and the routing
bit-identical; the logits too, except behind the Q8_0 model's F16 head (matrix-core order: full bar)."""

import numpy as np
import pytest

import oracle_py as O
from helpers import assert_close, end_to_end_stages, fill_kv, report_stages
from zonos2_amd import configs, synth
from zonos2_amd.z2h import Context

pytestmark = [pytest.mark.gpu, pytest.mark.slow]


@pytest.mark.parametrize("bulk", [configs.Q6_K, configs.Q8_0], ids=["q6_k", "q8_0"])
def test_c4_layers_teacher_forced(bulk):
    cfg, wl = configs.C4(bulk)
    assert cfg.n_layer == 24 and len(wl.kv_lens) == 64
    model = synth.generate_model(cfg, 7)
    ctx = Context(cfg.hparams(), wl.n_slots, wl.slot_cap)
    ctx.upload(model)
    om0 = O.OracleModel(cfg.hparams(), model)
    okv = O.OracleKV(om0, wl.n_slots, wl.slot_cap)
    fill_kv(cfg, wl, [ctx.kv_write, okv.write])
    bias = synth.router_biases(ctx, cfg, wl)         # balanced + Zipf, also given to the oracle
    om = O.OracleModel(cfg.hparams(), model, logit_bias=bias)
    okv.model = om
    T, d, E, k = len(wl.kv_lens), cfg.n_embd, cfg.n_expert, cfg.top_k
    inp = synth.step_inputs(cfg, wl)
    ctx.set_capture(True)
    got = ctx.step(inp.slot_idx, inp.n_past, ids=inp.ids)
    rd = lambda L, n: ctx.read_capture(L, n, T)
    prev = None
    for L in range(cfg.n_layer):
        res_in = rd(L, "res_in").reshape(T, d)
        attn_in = rd(L, "attn_in").reshape(T, d)
        ffn_in = rd(L, "ffn_in").reshape(T, d)
        attn_out = rd(L, "attn_out").reshape(T, d)
        ffn_out = rd(L, "ffn_out").reshape(T, d)
        ao = np.empty((T, cfg.n_head * cfg.head_dim), np.float32)
        oo = np.empty((T, d), np.float32)
        O.check(O.lib().orc_attention(om.m, okv.kv, L, T, O.ptr(inp.slot_idx), O.ptr(inp.n_past), O.ptr(attn_in),
                                      O.ptr(ao), O.ptr(oo)))
        assert_close(f"L{L} attn_out", attn_out, oo)
        r = O.router(om, L, ffn_in, prev)
        sel = rd(L, "sel").reshape(T, k)
        assert np.array_equal(sel, r["sel"]), f"L{L} top-k ids"
        assert np.array_equal(rd(L, "probs").reshape(T, E).view(np.uint32), r["probs"].view(np.uint32)), f"L{L} probs"
        counts, offsets, perm = O.group(sel, E)
        assert np.array_equal(rd(L, "counts"), counts) and np.array_equal(rd(L, "perm"), perm)
        w = rd(L, "weights").reshape(T, k)
        _, out = O.experts(om, L, ffn_in, sel, w)
        assert_close(f"L{L} ffn_out", ffn_out, out)
        if L + 1 < cfg.n_layer:
            assert np.array_equal(rd(L + 1, "res_in").reshape(T, d), ffn_out + (attn_out + res_in)), f"L{L} residual fold"
        prev = r["rh"]
        print(f"L{L}: {len(set(sel.ravel().tolist()))} experts touched, max routes {counts.max()}")
    hn = ctx.read_capture(0, "out_norm", T).reshape(T, d)
    hw = model["output.weight"]
    mout = O.matmul(hw.type, hw.data, hw.ne[0], hw.ne[1], hn).astype(np.float64)
    assert_close("head + softcap", got, cfg.logit_softcap * np.tanh(mout / cfg.logit_softcap))
    # end to end: the oracle's own step from the same ids (its step rewrites row n_past of every slot
    # in each layer before that layer's attention, so the rows appended above do not leak in)
    want, ocap = O.step(om, okv, inp.slot_idx, inp.n_past, ids=inp.ids, capture=True)
    rows = end_to_end_stages(ctx, ocap, cfg, T)
    report_stages(f"C4 {configs.TYPE_NAMES[bulk]}", rows, got, want)
    for L in range(cfg.n_layer):
        assert np.array_equal(rd(L, "sel").reshape(T, k), ocap["sel"][L]), f"L{L}: routing differs"
    assert not rows, f"first differing stage: L{rows[0][0]} {rows[0][1]}"
    if model["output.weight"].type == configs.F16:
        # the F16 head runs on the matrix cores (their internal summation order): the full bar
        assert_close("end-to-end logits", got, want)
    else:
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), "logits differ"
    ctx.close()
