"""The released model's topology at full size (docs/INTERNALS.md:252-259): 28 layers with dense SwiGLU
FFNs on layers 0, 1, 2 and 27 between 24 MoE layers of 16 experts, top-1 routing with top-2 on layer
26, router_dim 128, 9 x 1026 logits, and two layers pruned to 12 and 14 experts (the per-layer counts of
a pruned GGUF, src/zonos2-graph.cpp:194-197), stepped for 16 ragged requests. End to end against the
oracle's own step: every stage of every layer, the routing and the logits bit-identical."""
import dataclasses

import numpy as np
import pytest

import oracle_py as O
from helpers import assert_close, end_to_end_stages, fill_kv, oracle_pair, report_stages
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


@pytest.mark.parametrize("bulk", [configs.Q8_0, configs.Q6_K, configs.Q4_K])
def test_one_and_two_request_steps_bit_identical(bulk):
    """Steps of one and two requests on a 4-layer cut of the released topology (dense, top-1 MoE,
    top-2 MoE pruned to 12 experts, dense) at d 2048: the expert matmuls of so few routes take the
    K-split GEMV (one block per 16-row group and route), every stage and the logits bit-identical to
    the oracle's step (the logits behind the Q8_0 model's F16 head at the full bar), and each request's
    logits the same bits alone and in the pair."""
    base, _ = configs.shipped(bulk)
    cfg = dataclasses.replace(base, name=f"{base.name}-cut4", n_layer=4, expert_used=[0, 1, 2, 0],
                              layer_experts={2: 12})
    wl = configs.Workload("two-requests", n_slots=2, kv_lens=[300, 77], slot_cap=512)
    model = synth.generate_model(cfg, 31)
    ctx = Context(cfg.hparams(), wl.n_slots, wl.slot_cap)
    ctx.upload(model)
    om, okv = oracle_pair(cfg, model, wl)
    fill_kv(cfg, wl, [ctx.kv_write, okv.write])
    inp = synth.step_inputs(cfg, wl)
    alone = {}
    for sub in ([0], [1], [1, 0]):
        T = len(sub)
        print(f"{cfg.name}: step of requests {sub}", flush=True)
        # uncaptured steps take the launches of the graph-replayed path (for Q8_0 experts the down
        # matmul encodes its fp32 rows itself); captured ones the sorted route table
        ctx.set_capture(False)
        plain = ctx.step(inp.slot_idx[sub], inp.n_past[sub], ids=inp.ids[sub])
        ctx.set_capture(True)
        got = ctx.step(inp.slot_idx[sub], inp.n_past[sub], ids=inp.ids[sub])
        assert np.array_equal(plain.view(np.uint32), got.view(np.uint32)), "capture changed the step"
        want, ocap = O.step(om, okv, inp.slot_idx[sub], inp.n_past[sub], ids=inp.ids[sub], capture=True)
        rows = end_to_end_stages(ctx, ocap, cfg, T)
        report_stages(f"{cfg.name} requests {sub}", rows, got, want)
        assert not rows, f"first differing stage: L{rows[0][0]} {rows[0][1]}"
        if model["output.weight"].type == configs.F16:
            # the Q8_0 model's F16 head runs on the matrix cores (their internal summation order)
            assert_close("logits", got, want)
        else:
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), "logits differ"
        if T == 1:
            alone[sub[0]] = got[0]
        else:
            for i, s in enumerate(sub):
                assert np.array_equal(got[i].view(np.uint32), alone[s].view(np.uint32))
    ctx.close()
