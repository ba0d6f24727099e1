"""Pins the oracle's routing: top-k order and ties, the grouping permutation, and the router
against an independent float64 restatement of build_moe's router (src/zonos2-graph.cpp:199-220)."""
import math

import numpy as np
import pytest

import oracle_py as O
from zonos2_amd import configs, synth


def _router_cfg(E=16, k=4, d=256, rd=64):
    return configs.ModelConfig("router-kat", n_layer=2, n_embd=d, n_head=2, n_head_kv=1, head_dim=128,
                               n_expert=E, top_k=k, n_ff=256, bulk=configs.Q8_0, router_dim=rd)


def _f32(model, name):
    t = model[name]
    return t.data.view(np.float32).reshape(tuple(reversed(t.ne))).astype(np.float64)


def _ref_router(model, L, x, state):
    """float64 restatement: down(+bias)(+state*eda) -> rms_w -> gelu MLP -> softmax -> +bias -> top-k."""
    b = f"blk.{L}."
    rh = x @ _f32(model, b + "router_down.weight").T + _f32(model, b + "router_down.bias")
    if state is not None and (b + "router_eda_scale") in model:
        rh = rh + state * _f32(model, b + "router_eda_scale")
    rn = rh / np.sqrt((rh * rh).mean(1, keepdims=True) + 1e-5) * _f32(model, b + "router_norm.weight")
    gelu = np.vectorize(lambda v: 0.5 * v * (1 + math.erf(v / math.sqrt(2))))
    h = gelu(rn @ _f32(model, b + "router_mlp0.weight").T + _f32(model, b + "router_mlp0.bias"))
    h = gelu(h @ _f32(model, b + "router_mlp2.weight").T + _f32(model, b + "router_mlp2.bias"))
    lg = h @ _f32(model, b + "router_mlp4.weight").T
    p = np.exp(lg - lg.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    sc = p + _f32(model, b + "router_bias")
    return rh, lg, p, sc


def test_router_vs_float64():
    cfg = _router_cfg()
    model = synth.generate_model(cfg, 9)
    om = O.OracleModel(cfg.hparams(), model)
    x = synth.gen_normal_f32((32, cfg.n_embd), 1, "x")
    r0 = O.router(om, 0, x, None)
    rh, lg, p, sc = _ref_router(model, 0, x.astype(np.float64), None)
    assert np.allclose(r0["rh"], rh, rtol=1e-5, atol=1e-6)
    assert np.allclose(r0["logits"], lg, rtol=1e-4, atol=1e-6)
    assert np.allclose(r0["probs"], p, rtol=1e-5, atol=1e-8)
    # selection: wherever the float64 margin is clear of rounding, ids must agree in order
    k = cfg.top_k
    order = np.argsort(-sc, axis=1, kind="stable")[:, :k]
    s = -np.sort(-sc, axis=1)
    clear = np.all(np.diff(s[:, :k + 1], axis=1) < -1e-6, axis=1)
    assert clear.sum() > 20
    assert np.array_equal(r0["sel"][clear], order[clear])
    assert np.allclose(r0["w"], np.take_along_axis(r0["probs"], r0["sel"], 1))
    # EDA state threading on the second MoE layer
    r1 = O.router(om, 1, x, r0["rh"])
    rh1, *_ = _ref_router(model, 1, x.astype(np.float64), r0["rh"].astype(np.float64))
    assert np.allclose(r1["rh"], rh1, rtol=1e-5, atol=1e-6)


def test_topk_ties_go_to_lower_index():
    """Equal selection scores: the lower expert index wins (bias makes whole groups tie)."""
    cfg = _router_cfg(E=8, k=3)
    model = synth.generate_model(cfg, 10)
    # zero router_mlp4 -> uniform probs; router_bias with ties decides the order
    name = "blk.0.router_mlp4.weight"
    model[name].data[:] = 0
    bias = np.array([0.0, 0.5, 0.5, 0.1, 0.5, 0.1, 0.0, 0.2], np.float32)
    model["blk.0.router_bias"].data[:] = np.frombuffer(bias.tobytes(), np.uint8)
    om = O.OracleModel(cfg.hparams(), model)
    x = synth.gen_normal_f32((4, cfg.n_embd), 2, "x")
    r = O.router(om, 0, x, None)
    assert np.all(r["sel"] == np.array([1, 2, 4]))
    assert np.allclose(r["w"], 1.0 / 8)


def test_expert_mask_renormalizes_and_never_routes_dropped():
    """zonos2_set_expert_mask (src/zonos2.cpp:203-239; graph.cpp:212, 218): the survivors' probabilities
    are the softmax over the survivors alone (as in a pruned model), a dropped expert gets probability 0
    and is never selected even when its router_bias is the largest."""
    cfg = _router_cfg(E=16, k=4)
    model = synth.generate_model(cfg, 11)
    bias = np.zeros(16, np.float32)
    bias[3] = 10.0                                  # would always win the selection if not masked
    model["blk.0.router_bias"].data[:] = np.frombuffer(bias.tobytes(), np.uint8)
    om = O.OracleModel(cfg.hparams(), model)
    x = synth.gen_normal_f32((24, cfg.n_embd), 3, "x")
    r_open = O.router(om, 0, x, None)
    assert np.all(r_open["sel"][:, 0] == 3)
    keep = np.ones(16, np.uint8)
    keep[[3, 5, 6, 11]] = 0
    om.set_expert_mask(0, keep)
    r = O.router(om, 0, x, None)
    kept = keep.astype(bool)
    assert np.all(r["probs"][:, ~kept] == 0.0)
    assert not np.isin(r["sel"], np.flatnonzero(~kept)).any()
    # float64: softmax over the kept logits only
    _, lg, _, _ = _ref_router(model, 0, x.astype(np.float64), None)
    lk = lg[:, kept]
    pk = np.exp(lk - lk.max(1, keepdims=True))
    pk /= pk.sum(1, keepdims=True)
    assert np.allclose(r["probs"][:, kept], pk, rtol=1e-4, atol=1e-7)
    assert np.array_equal(r["rh"].view(np.uint32), r_open["rh"].view(np.uint32))
    om.set_expert_mask(0, None)
    r2 = O.router(om, 0, x, None)
    assert np.array_equal(r2["probs"].view(np.uint32), r_open["probs"].view(np.uint32))


@pytest.mark.parametrize("T,k,E", [(1, 1, 4), (16, 4, 32), (64, 4, 32), (7, 2, 8)])
def test_grouping_is_stable_counting_sort(T, k, E):
    rng = np.random.default_rng(T * 100 + E)
    sel = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    counts, offsets, perm = O.group(sel, E)
    flat = sel.ravel()
    assert np.array_equal(counts, np.bincount(flat, minlength=E))
    assert np.array_equal(offsets, np.concatenate([[0], np.cumsum(counts)]))
    assert np.array_equal(perm, np.argsort(flat, kind="stable"))


def test_grouping_rejects_bad_ids():
    with pytest.raises(RuntimeError):
        O.group(np.array([[0, 9]], np.int32), 4)
