"""Pins the oracle's whole decode step and prefill against a float64 restatement of build_graph.

Every connection of the step is checked teacher-forced, stage by stage, from the oracle's own
captures: emb_norm -> attn_norm -> QKV + gate projections -> QK-norm, |temp|, interleaved RoPE ->
f16 KV append -> GQA softmax attention over the slot's band -> gate -> W_o -> residual -> ffn_norm ->
experts (on the oracle's routing, which test_oracle_router pins) or the dense SwiGLU FFN -> residual
-> output_norm -> head -> softcap (src/zonos2-graph.cpp:92-185, 248-366). The float64 side uses
the dequantized weights (block decoding is pinned by test_oracle_formats) and no activation
quantization, so the matmul stages agree to the activation-quantization error and the rest to
float32 rounding. A dropped term, a wrong residual, a transposed weight or a wrong RoPE position
fails one of the stages.

Depth prune (zonos2_model::layer_skip, graph.cpp:334-341) is pinned by its definition: skipping
block 0 of a two-block model equals the one-block model made of block 1 alone.
"""
import math

import numpy as np
import pytest

import oracle_py as O
from helpers import cos
from zonos2_amd import configs, synth


def _mat(model, name):
    t = model[name]
    n = int(np.prod(t.ne))
    return O.dequant(t.type, t.data, n).astype(np.float64).reshape(tuple(reversed(t.ne)))


def _vec(model, name):
    return model[name].data.view(np.float32).astype(np.float64)


def _rms(x, w=None, eps=1e-5):
    y = x / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    return y * w if w is not None else y


def _rope(x, pos, base):
    """interleaved pairs (2i, 2i+1) rotated by pos * base^(-2i/hd)"""
    hd = x.shape[-1]
    th = pos * base ** (-2.0 * np.arange(hd // 2) / hd)
    c, s = np.cos(th), np.sin(th)
    y = x.copy()
    y[..., 0::2] = x[..., 0::2] * c - x[..., 1::2] * s
    y[..., 1::2] = x[..., 0::2] * s + x[..., 1::2] * c
    return y


def _silu(x):
    return x / (1.0 + np.exp(-x))


def _sig(x):
    return 1.0 / (1.0 + np.exp(-x))


def _close(name, got, want, c_min, rel):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    c = cos(got, want)
    m = float(np.abs(got - want).max()) / max(float(np.abs(want).max()), 1e-30)
    assert c >= c_min and m <= rel, f"{name}: cos={c:.8f} rel maxabs={m:.3e}"


MM = (0.9999, 3e-2)      # one activation-quantized matmul (Q8_0) against float64
F32 = (0.9999999, 1e-5)  # float32 elementwise / reduction against float64


def _cfg(expert_used):
    m = configs.ModelConfig("step-kat", n_layer=len(expert_used), n_embd=256, n_head=8, n_head_kv=2, head_dim=32,
                            n_expert=8, top_k=2, n_ff=512, bulk=configs.Q8_0, router_bias_std=1e-4,
                            expert_used=list(expert_used))
    w = configs.Workload("step-kat", n_slots=4, kv_lens=[3, 17, 64, 130], slot_cap=131, inject_embeddings=True)
    return m, w


def _check_step(cfg, wl, model, om, okv, inp, logits, cap):
    hp = cfg.hparams()
    d, nh, nkv, hd = cfg.n_embd, cfg.n_head, cfg.n_head_kv, cfg.head_dim
    eps, base = hp["rms_eps"], hp["rope_freq_base"]
    T = len(inp.slot_idx)
    x0 = _rms(inp.emb.astype(np.float64), eps=eps)
    _close("emb_norm -> res_in[0]", cap["res_in"][0], x0, *F32)
    for L in range(cfg.n_layer):
        b = f"blk.{L}."
        res = cap["res_in"][L].astype(np.float64)
        if L > 0:  # fold of the previous block: res = res_prev + attn_out_prev + ffn_out_prev
            want = cap["res_in"][L - 1].astype(np.float64) + cap["attn_out"][L - 1] + cap["ffn_out"][L - 1]
            _close(f"L{L} residual fold", res, want, *F32)
        cur = _rms(res, _vec(model, b + "attn_norm.weight"), eps)
        _close(f"L{L} attn_norm", cap["attn_in"][L], cur, *F32)
        xin = cap["attn_in"][L].astype(np.float64)
        q = (xin @ _mat(model, b + "attn_q.weight").T).reshape(T, nh, hd)
        k = (xin @ _mat(model, b + "attn_k.weight").T).reshape(T, nkv, hd)
        v = (xin @ _mat(model, b + "attn_v.weight").T).reshape(T, nkv, hd)
        g = _sig(xin @ _mat(model, b + "attn_gate.weight").T)
        q = _rms(q, eps=hp["qk_norm_eps"]) * _vec(model, b + "attn_temp")[None, :, None]
        k = _rms(k, eps=hp["qk_norm_eps"])
        for t in range(T):
            q[t] = _rope(q[t], inp.n_past[t], base)
            k[t] = _rope(k[t], inp.n_past[t], base)
        _close(f"L{L} q", cap["q"][L], q.reshape(T, -1), *MM)
        _close(f"L{L} k", cap["k"][L], k.reshape(T, -1), *MM)
        _close(f"L{L} v", cap["v"][L], v.reshape(T, -1), *MM)
        _close(f"L{L} gate", cap["gate"][L], g, *MM)
        # attention on the oracle's q / gate and its f16 cache (new row appended at n_past)
        qo = cap["q"][L].astype(np.float64).reshape(T, nh, hd)
        go = cap["gate"][L].astype(np.float64)
        o = np.zeros((T, nh, hd))
        for t in range(T):
            n = inp.n_past[t] + 1
            kr, vr = okv.read(L, inp.slot_idx[t], 0, n)
            kr = kr.view(np.float16).astype(np.float64)
            vr = vr.view(np.float16).astype(np.float64)
            newk = cap["k"][L][t].reshape(nkv, hd).astype(np.float16).astype(np.float64)
            assert np.array_equal(kr[n - 1], newk), f"L{L} KV append row (token {t})"
            for h in range(nh):
                gk = h // (nh // nkv)
                s = kr[:, gk, :] @ qo[t, h] / math.sqrt(hd)
                p = np.exp(s - s.max())
                o[t, h] = (p / p.sum()) @ vr[:, gk, :] * go[t, h]
        _close(f"L{L} attention", cap["attn_o"][L], o.reshape(T, -1), 0.99999, 5e-3)
        ao = cap["attn_out"][L]
        _close(f"L{L} W_o", ao, cap["attn_o"][L].astype(np.float64) @ _mat(model, b + "attn_output.weight").T, *MM)
        res2 = res + ao
        _close(f"L{L} ffn_norm", cap["ffn_in"][L], _rms(res2, _vec(model, b + "ffn_norm.weight"), eps), *F32)
        fi = cap["ffn_in"][L].astype(np.float64)
        if cfg.expert_used[L]:
            kL = cfg.expert_used[L]
            sel, w = cap["sel"][L][:, :kL], cap["weights"][L][:, :kL]
            assert np.allclose(w, np.take_along_axis(cap["probs"][L], sel, 1), rtol=0, atol=0)
            G = _mat(model, b + "ffn_gate_exps.weight")
            U = _mat(model, b + "ffn_up_exps.weight")
            D = _mat(model, b + "ffn_down_exps.weight")
            out = np.zeros((T, d))
            for t in range(T):
                for j in range(kL):
                    e = sel[t, j]
                    y = (U[e] @ fi[t]) * _silu(G[e] @ fi[t])
                    out[t] += w[t, j] * (D[e] @ y)
        else:
            y = (fi @ _mat(model, b + "ffn_up.weight").T) * _silu(fi @ _mat(model, b + "ffn_gate.weight").T)
            out = y @ _mat(model, b + "ffn_down.weight").T
        _close(f"L{L} ffn_out", cap["ffn_out"][L], out, 0.9998, 5e-2)
    last = cfg.n_layer - 1
    resf = cap["res_in"][last].astype(np.float64) + cap["attn_out"][last] + cap["ffn_out"][last]
    hn = _rms(resf, _vec(model, "output_norm.weight"), eps)
    _close("output_norm", cap["out_norm"], hn, *F32)
    mout = cap["out_norm"].astype(np.float64) @ _mat(model, "output.weight").T
    cap_ = hp["logit_softcap"]
    _close("head + softcap", logits, cap_ * np.tanh(mout / cap_), *MM)


@pytest.mark.parametrize("expert_used", [(2, 2), (0, 2)], ids=["moe-moe", "dense-moe"])
def test_step_vs_float64_restatement(expert_used):
    cfg, wl = _cfg(expert_used)
    model = synth.generate_model(cfg, 31)
    om = O.OracleModel(cfg.hparams(), model)
    okv = O.OracleKV(om, wl.n_slots, wl.slot_cap)
    for L in range(cfg.n_layer):
        for s, n in enumerate(wl.kv_lens):
            k, v = synth.kv_rows(cfg, L, s, n, 7)
            okv.write(L, s, 0, k, v)
    inp = synth.step_inputs(cfg, wl)
    logits, cap = O.step(om, okv, inp.slot_idx, inp.n_past, emb=inp.emb, capture=True)
    _check_step(cfg, wl, model, om, okv, inp, logits, cap)


def test_token_ids_sum_the_embedding_rows():
    """ids path: emb = sum of the W table rows in column order (graph.cpp:248-260), then emb_norm."""
    cfg, wl = _cfg((2, 2))
    model = synth.generate_model(cfg, 32)
    om = O.OracleModel(cfg.hparams(), model)
    okv = O.OracleKV(om, wl.n_slots, wl.slot_cap)
    inp = synth.step_inputs(cfg, wl)
    ids = inp.ids
    W = cfg.n_codebooks + 1
    emb = np.zeros((len(ids), cfg.n_embd), np.float32)
    for kk in range(W):
        name = f"audio_embd.{kk}.weight" if kk < cfg.n_codebooks else "text_embd.weight"
        tab = _mat(model, name).astype(np.float32)
        for t in range(len(ids)):
            emb[t] = emb[t] + tab[ids[t, kk]] if kk else tab[ids[t, kk]]
    okv2 = O.OracleKV(om, wl.n_slots, wl.slot_cap)
    a = O.step(om, okv, inp.slot_idx, inp.n_past, ids=ids)
    b = O.step(om, okv2, inp.slot_idx, inp.n_past, emb=emb)
    assert np.array_equal(a, b)


def test_layer_skip_is_block_removal():
    cfg, wl = _cfg((2, 2))
    model = synth.generate_model(cfg, 33)
    om = O.OracleModel(cfg.hparams(), model)
    om.set_layer_skip([1, 0])
    # the one-block model made of block 1 (its router_eda_scale has no earlier MoE state to read)
    cfg1, _ = _cfg((2,))
    m1 = {}
    for name, t in model.items():
        if name.startswith("blk.0."):
            continue
        nn = name.replace("blk.1.", "blk.0.")
        m1[nn] = synth.Tensor(nn, t.type, t.ne, t.data)
    om1 = O.OracleModel(cfg1.hparams(), m1)
    kv2 = O.OracleKV(om, wl.n_slots, wl.slot_cap)
    kv1 = O.OracleKV(om1, wl.n_slots, wl.slot_cap)
    for s, n in enumerate(wl.kv_lens):
        k, v = synth.kv_rows(cfg, 1, s, n, 7)
        kv2.write(1, s, 0, k, v)
        kv1.write(0, s, 0, k, v)
    inp = synth.step_inputs(cfg, wl)
    a = O.step(om, kv2, inp.slot_idx, inp.n_past, emb=inp.emb)
    b = O.step(om1, kv1, inp.slot_idx, inp.n_past, emb=inp.emb)
    assert np.array_equal(a, b)
    # and the prefill path
    ids = np.stack([inp.ids[0]] * 5)
    assert np.array_equal(O.prefill(om, kv2, 0, ids), O.prefill(om1, kv1, 0, ids))
    om.set_layer_skip(None)
    c = O.step(om, kv2, inp.slot_idx, inp.n_past, emb=inp.emb)
    assert not np.array_equal(a, c)


def _stepwise(om, kv, slot, ids, emb_rows=None):
    """n0 single-row decode steps (row t at position t); emb_rows {t: row} replaces row t's embedding"""
    out = None
    for t in range(ids.shape[0]):
        if emb_rows and t in emb_rows:
            out = O.step(om, kv, [slot], [t], emb=emb_rows[t][None, :])
        else:
            out = O.step(om, kv, [slot], [t], ids=ids[t:t + 1])
    return out[0]


def test_prefill_equals_stepwise_decode():
    """KV decode == recompute (graph.cpp:515-604): the causal prefill (fp32 K/V within the prompt,
    graph.cpp:155-169) and n0 single-row decode steps over the f16 cache agree to f16 rounding, and
    write the same cache rows."""
    cfg, wl = _cfg((0, 2))
    model = synth.generate_model(cfg, 34)
    om = O.OracleModel(cfg.hparams(), model)
    rng = np.random.default_rng(5)
    n0 = 23
    ids = np.concatenate([rng.integers(0, cfg.audio_vocab, (n0, cfg.n_codebooks)),
                          rng.integers(0, cfg.text_vocab + 1, (n0, 1))], axis=1).astype(np.int32)
    kv_a = O.OracleKV(om, 2, 64)
    kv_b = O.OracleKV(om, 2, 64)
    a = O.prefill(om, kv_a, 1, ids)
    b = _stepwise(om, kv_b, 1, ids)
    _close("prefill vs steps", a, b, 0.99999, 2e-2)
    for L in range(cfg.n_layer):
        ka, va = kv_a.read(L, 1, 0, n0)
        kb, vb = kv_b.read(L, 1, 0, n0)
        _close(f"L{L} K rows", ka.view(np.float16), kb.view(np.float16), 0.99999, 2e-2)
        _close(f"L{L} V rows", va.view(np.float16), vb.view(np.float16), 0.99999, 2e-2)


def test_speaker_splice_replaces_the_row():
    """spk: row spk_pos's embedding is REPLACED by spk_proj(spk_lda(spk)) (+ delta), before emb_norm
    (graph.cpp:262-297). Checked against steps that inject the float64 speaker row there."""
    cfg, wl = _cfg((2, 2))
    model = synth.generate_model(cfg, 35)
    om = O.OracleModel(cfg.hparams(), model)
    rng = np.random.default_rng(6)
    n0, pos = 9, 3
    ids = np.concatenate([rng.integers(0, cfg.audio_vocab, (n0, cfg.n_codebooks)),
                          rng.integers(0, cfg.text_vocab + 1, (n0, 1))], axis=1).astype(np.int32)
    spk = synth.gen_normal_f32((cfg.spk_dim,), 3, "spk")
    delta = synth.gen_normal_f32((cfg.n_embd,), 4, "delta") * 0.1
    sl = _mat(model, "spk_lda.weight") @ spk.astype(np.float64) + _vec(model, "spk_lda.bias")
    sp = _mat(model, "spk_proj.weight") @ sl + _vec(model, "spk_proj.bias") + delta
    a = O.prefill(om, O.OracleKV(om, 1, 16), 0, ids, spk=spk, spk_pos=pos, delta=delta)
    b = _stepwise(om, O.OracleKV(om, 1, 16), 0, ids, {pos: sp.astype(np.float32)})
    _close("speaker prefill vs injected steps", a, b, 0.99999, 2e-2)
    plain = O.prefill(om, O.OracleKV(om, 1, 16), 0, ids)
    d_ab, d_ap = float(np.abs(a - b).max()), float(np.abs(a - plain).max())
    assert d_ap > 5 * d_ab, f"the speaker row changed too little ({d_ap:.3e} vs {d_ab:.3e})"
