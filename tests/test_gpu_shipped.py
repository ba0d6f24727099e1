"""The released model's topology at full size (docs/INTERNALS.md:252-259): 28 layers with dense SwiGLU
FFNs on layers 0, 1, 2 and 27 between 24 MoE layers of 16 experts, top-1 routing with top-2 on layer
26, router_dim 128, 9 x 1026 logits, and two layers pruned to 12 and 14 experts (the per-layer counts of
a pruned GGUF, src/zonos2-graph.cpp:194-197), stepped for 16 ragged requests. End to end against the
oracle's own step: every stage of every layer, the routing and the logits bit-identical."""
import numpy as np
import pytest

import oracle_py as O
from helpers import end_to_end_stages, fill_kv, oracle_pair, report_stages
from zonos2_amd import configs, synth
from zonos2_amd.z2h import Context

pytestmark = [pytest.mark.gpu, pytest.mark.slow]


def test_shipped_topology_end_to_end_bit_identical():
    cfg, wl = configs.shipped(configs.Q4_K)
    assert cfg.expert_used[26] == 2 and cfg.expert_used[0] == cfg.expert_used[27] == 0 and cfg.n_exp(9) == 12
    model = synth.generate_model(cfg, 21)
    ctx = Context(cfg.hparams(), wl.n_slots, wl.slot_cap)
    ctx.upload(model)
    om0, okv = oracle_pair(cfg, model, wl)
    fill_kv(cfg, wl, [ctx.kv_write, okv.write])
    bias = synth.router_biases(ctx, cfg, wl)
    om = O.OracleModel(cfg.hparams(), model, logit_bias=bias)
    okv.model = om
    T = len(wl.kv_lens)
    inp = synth.step_inputs(cfg, wl)
    ctx.set_capture(False)
    plain = ctx.step(inp.slot_idx, inp.n_past, ids=inp.ids)
    ctx.set_capture(True)
    got = ctx.step(inp.slot_idx, inp.n_past, ids=inp.ids)
    assert np.array_equal(plain.view(np.uint32), got.view(np.uint32)), "capture changed the step"
    want, ocap = O.step(om, okv, inp.slot_idx, inp.n_past, ids=inp.ids, capture=True)
    rows = end_to_end_stages(ctx, ocap, cfg, T)
    report_stages("shipped topology", rows, got, want)
    touched = []
    for L in range(cfg.n_layer):
        k = cfg.expert_used[L]
        if not k:
            continue
        sel = ctx.read_capture(L, "sel", T)[:T * k].reshape(T, k)
        assert np.array_equal(sel, ocap["sel"][L][:, :k]), f"L{L}: routing differs"
        assert sel.max() < cfg.n_exp(L)
        touched.append(len(set(sel.ravel().tolist())))
    print(f"experts touched per MoE layer: {touched}")
    assert not rows, f"first differing stage: L{rows[0][0]} {rows[0][1]}"
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), "logits differ"
    # a subset of the requests gives bit-identical rows
    sub = [0, 5, 15]
    ctx.set_capture(False)
    part = ctx.step(inp.slot_idx[sub], inp.n_past[sub], ids=inp.ids[sub])
    assert np.array_equal(part, got[sub])
    ctx.close()
