"""Device decode step vs the CPU oracle (C ABI via ctypes), on the tiny config and one MoE layer.

Bars: routing (router state, logits, probabilities, top-k ids, weights) and the grouping (counts,
offsets, permutation) bit-exact on identical router inputs; hidden states and logits cos >= 0.9999
and max-abs <= 1e-2 per layer.
"""
import numpy as np
import pytest

import oracle_py as O
from helpers import COS_MIN, MAXABS, assert_close, fill_kv, oracle_pair, min_topk_margin, router_bias
from zonos2_amd import configs, synth
from zonos2_amd.z2h import Context, Model

pytestmark = pytest.mark.gpu


def _build(cfg, wl, seed=42):
    model = synth.generate_model(cfg, seed)
    ctx = Context(cfg.hparams(), wl.n_slots, wl.slot_cap)
    ctx.upload(model)
    om, okv = oracle_pair(cfg, model, wl)
    fill_kv(cfg, wl, [ctx.kv_write, okv.write])
    return model, ctx, om, okv


def _check_routing(cfg, ctx, om, T, model=None):
    """Teacher-forced: the oracle router on the device's router input must match bit for bit."""
    prev = None
    E, rd = cfg.n_expert, cfg.router_dim
    for L in range(cfg.n_layer):
        k = cfg.expert_used[L]
        if k == 0:
            continue
        x = ctx.read_capture(L, "ffn_in", T).reshape(T, cfg.n_embd)
        ref = O.router(om, L, x, prev)
        rh = ctx.read_capture(L, "router_state", T).reshape(T, rd)
        lg = ctx.read_capture(L, "router_logits", T).reshape(T, E)
        pr = ctx.read_capture(L, "probs", T).reshape(T, E)
        sel = ctx.read_capture(L, "sel", T).ravel()[:T * k].reshape(T, k)
        w = ctx.read_capture(L, "weights", T).ravel()[:T * k].reshape(T, k)
        for name, a, b in (("rh", rh, ref["rh"]), ("logits", lg, ref["logits"]), ("probs", pr, ref["probs"]),
                           ("w", w, ref["w"])):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"layer {L} {name} not bit-exact"
        assert np.array_equal(sel, ref["sel"]), f"layer {L} top-k ids differ"
        counts, offsets, perm = O.group(sel, E)
        assert np.array_equal(ctx.read_capture(L, "counts", T), counts)
        assert np.array_equal(ctx.read_capture(L, "offsets", T), offsets)
        assert np.array_equal(ctx.read_capture(L, "perm", T)[:T * k], perm)
        # experts on the same routing: weighted per-route outputs and the k-sum
        eo, out = O.experts(om, L, x, sel, w)
        geo = ctx.read_capture(L, "expert_out", T).reshape(-1, cfg.n_embd)[:T * k]
        assert_close(f"layer {L} expert_out", geo, eo)
        rb = router_bias(model, L) if model is not None else np.zeros(E, np.float32)
        print(f"layer {L}: routing bit-exact, min top-k margin (probs + router_bias) {min_topk_margin(ref['probs'], rb, k):.3e}")
        prev = rh


def test_c1_step_vs_oracle():
    cfg, wl = configs.C1()
    model, ctx, om, okv = _build(cfg, wl)
    inp = synth.step_inputs(cfg, wl)
    T = len(wl.kv_lens)
    ctx.set_capture(True)
    got = ctx.step(inp.slot_idx, inp.n_past, emb=inp.emb)
    want, cap = O.step(om, okv, inp.slot_idx, inp.n_past, emb=inp.emb, capture=True)
    for L in range(cfg.n_layer):
        for name in ("res_in", "attn_in", "q", "k", "v", "attn_o", "attn_out", "ffn_in", "ffn_out"):
            g = ctx.read_capture(L, name, T).reshape(cap[name][L].shape)
            assert_close(f"layer {L} {name}", g, cap[name][L])
    assert_close("out_norm", ctx.read_capture(0, "out_norm", T).reshape(T, -1), cap["out_norm"])
    assert_close("logits", got, want)
    _check_routing(cfg, ctx, om, T, model)
    # the new K/V rows written by the step
    for L in range(cfg.n_layer):
        for s, n in enumerate(wl.kv_lens):
            gk, gv = ctx.kv_read(L, s, n, 1)
            ok, ov = okv.read(L, s, n, 1)
            assert_close(f"kv {L}/{s}", gk.view(np.float16).astype(np.float32), ok.view(np.float16).astype(np.float32))
            assert_close(f"kv {L}/{s}", gv.view(np.float16).astype(np.float32), ov.view(np.float16).astype(np.float32))


def test_c1_step_with_token_ids():
    cfg, wl = configs.C1()
    model, ctx, om, okv = _build(cfg, wl, seed=43)
    inp = synth.step_inputs(cfg, wl)
    got = ctx.step(inp.slot_idx, inp.n_past, ids=inp.ids)
    want = O.step(om, okv, inp.slot_idx, inp.n_past, ids=inp.ids)
    assert_close("logits(ids)", got, want)


def test_device_resident_step_equals_host_step():
    """z2h_step_device (inputs and logits in device memory, enqueued on the caller's stream; the
    entry the decode benchmark times) against z2h_step (host buffers): the same logits bit for bit,
    with token ids and with injected embeddings. A step writes its K/V row at n_past, so repeating
    it with the same inputs rewrites the same values."""
    import torch
    cfg, wl = configs.C1()
    model, ctx, om, okv = _build(cfg, wl, seed=47)
    inp = synth.step_inputs(cfg, wl)
    T = len(wl.kv_lens)
    dev = torch.device("cuda:0")
    d_slot = torch.from_numpy(inp.slot_idx).to(dev)
    d_npast = torch.from_numpy(inp.n_past).to(dev)
    d_ids = torch.from_numpy(inp.ids).to(dev)
    d_emb = torch.from_numpy(inp.emb).to(dev)
    d_out = torch.empty((T, cfg.n_codebooks * cfg.audio_vocab), dtype=torch.float32, device=dev)
    stream = torch.cuda.Stream(device=dev)
    for kind in ("ids", "emb"):
        want = ctx.step(inp.slot_idx, inp.n_past, **({"ids": inp.ids} if kind == "ids" else {"emb": inp.emb}))
        d_out.fill_(float("nan"))
        torch.cuda.synchronize()
        ctx.step_device(T, d_slot.data_ptr(), d_npast.data_ptr(), inp.n_past,
                        d_ids.data_ptr() if kind == "ids" else 0, d_emb.data_ptr() if kind == "emb" else 0,
                        d_out.data_ptr(), stream=stream.cuda_stream)
        stream.synchronize()
        np.testing.assert_array_equal(d_out.cpu().numpy(), want, err_msg=kind)
    ctx.close()


def test_c1_batch_invariance():
    """A column's result does not depend on the other columns (reference --batch-test F.1/F.2)."""
    cfg, wl = configs.C1()
    model, ctx, om, okv = _build(cfg, wl, seed=44)
    inp = synth.step_inputs(cfg, wl)
    full = ctx.step(inp.slot_idx, inp.n_past, emb=inp.emb)
    for t in range(len(wl.kv_lens)):
        one = ctx.step(inp.slot_idx[t:t + 1], inp.n_past[t:t + 1], emb=inp.emb[t:t + 1])
        assert np.array_equal(one[0], full[t]), f"column {t} differs when stepped alone"


def test_c2_moe_layer_vs_oracle():
    cfg, wl = configs.C2()
    model = synth.generate_model(cfg, 42)
    ctx = Context(cfg.hparams(), wl.n_slots, wl.slot_cap)
    ctx.upload(model)
    om = O.OracleModel(cfg.hparams(), model)
    T = wl.n_slots
    x = synth.gen_normal_f32((T, cfg.n_embd), wl.seed, "inputs.moe")
    ctx.set_capture(True)
    got = ctx.moe_forward(0, x)
    ref = O.router(om, 0, x, None)
    sel = ctx.read_capture(0, "sel", T).reshape(T, ctx.kmax)[:, :cfg.top_k]
    assert np.array_equal(sel, ref["sel"])
    for name in ("router_state", "router_logits", "probs"):
        key = {"router_state": "rh", "router_logits": "logits", "probs": "probs"}[name]
        assert np.array_equal(ctx.read_capture(0, name, T).reshape(ref[key].shape).view(np.uint32), ref[key].view(np.uint32)), name
    counts, offsets, perm = O.group(ref["sel"], cfg.n_expert)
    assert np.array_equal(ctx.read_capture(0, "counts", T), counts)
    assert np.array_equal(ctx.read_capture(0, "offsets", T), offsets)
    assert np.array_equal(ctx.read_capture(0, "perm", T), perm)
    eo, out = O.experts(om, 0, x, ref["sel"], ref["w"])
    assert_close("moe out", got, out)


@pytest.mark.parametrize("T", [4, 100], ids=["per-token-router", "wide-router"])
def test_router_ties_go_to_the_lower_expert_index(T):
    """Exact ties in the selection scores through the device router: with router_mlp4 zero every
    router logit is 0, so the softmax gives exactly 1/E (1/7 under a one-expert mask) to every kept
    expert, and router_bias decides the order with tied values. north_star's contract: scores
    descending, ties to the lower expert index. The device's top-k ids, weights and grouping must be
    the oracle's, and the ids the closed-form answer. 4 tokens take the per-token router tail
    (k_router_tail<false>), 100 the wide passes' (k_router_down_t + k_router_tail<true>, from 65 rows)."""
    cfg, wl = configs.C1()
    model = synth.generate_model(cfg, 45)
    E, k, d = cfg.n_expert, cfg.top_k, cfg.n_embd
    bias = np.array([0.0, 0.5, 0.5, 0.0, 0.5, 0.0, 0.25, 0.5], np.float32)
    for L in range(cfg.n_layer):
        if cfg.expert_used[L] == 0:
            continue
        model[f"blk.{L}.router_mlp4.weight"].data[...] = 0
        model[f"blk.{L}.router_bias"].data[...] = bias.view(model[f"blk.{L}.router_bias"].data.dtype)
    ctx = Context(cfg.hparams(), max(T, wl.n_slots), wl.slot_cap, max_rows=T)
    ctx.upload(model)
    om = O.OracleModel(cfg.hparams(), model)
    x = synth.gen_normal_f32((T, d), 3, "inputs.ties")
    L = next(L for L in range(cfg.n_layer) if cfg.expert_used[L])
    ctx.set_capture(True)
    for keep, want_sel in ((None, [1, 2]), (np.array([1, 0, 1, 1, 1, 1, 1, 1], np.uint8), [2, 4])):
        ctx.set_expert_mask(L, keep)
        om.set_expert_mask(L, keep)
        got = ctx.moe_forward(L, x)
        sel = ctx.read_capture(L, "sel", T).reshape(T, ctx.kmax)[:, :k]
        w = ctx.read_capture(L, "weights", T).reshape(T, ctx.kmax)[:, :k]
        ref = O.router(om, L, x, None)
        p = np.float32(1.0) / np.float32(E if keep is None else int(keep.sum()))
        kept = ref["probs"][:, keep.astype(bool)] if keep is not None else ref["probs"]
        assert np.all(kept == kept[0, 0]), "probabilities not tied"
        assert np.array_equal(sel, np.tile(np.array(want_sel, np.int32), (T, 1))), f"device top-k {sel[0]} != {want_sel}"
        assert np.array_equal(sel, ref["sel"])
        assert np.array_equal(w.view(np.uint32), ref["w"].view(np.uint32))
        assert abs(float(ref["probs"][0, want_sel[0]]) - float(p)) < 1e-6
        counts, offsets, perm = O.group(sel, E)
        assert np.array_equal(ctx.read_capture(L, "perm", T)[:T * k], perm)
        eo, out = O.experts(om, L, x, sel, w)
        assert_close("tied-route moe out", got, out)
    ctx.close()


def test_graph_replay_matches_eager():
    """Whole-step HIP-graph replays equal the eager launch sequence bit for bit, replay after replay,
    with eager work and other batch widths interleaved."""
    cfg, wl = configs.C1()
    model, ctx, om, okv = _build(cfg, wl, seed=45)
    inp = synth.step_inputs(cfg, wl)
    ctx.set_graphs(False)
    ref = ctx.step(inp.slot_idx, inp.n_past, emb=inp.emb)
    ref2 = ctx.step(inp.slot_idx[:2], inp.n_past[:2], emb=inp.emb[:2])
    ctx.set_graphs(True)
    x = synth.gen_normal_f32((4, cfg.n_embd), 3, "x")
    for rep in range(4):
        got = ctx.step(inp.slot_idx, inp.n_past, emb=inp.emb)
        assert np.array_equal(got, ref), f"replay {rep}"
        got2 = ctx.step(inp.slot_idx[:2], inp.n_past[:2], emb=inp.emb[:2])
        assert np.array_equal(got2, ref2), f"replay {rep} (width 2)"
        ctx.moe_forward(0, x)                      # eager work between replays


def test_shared_model_contexts_and_mask_invalidation():
    """Two batch contexts over one device model (zonos2_model loaded once, several zonos2_batch_ctx)
    step exactly like a context with its own copy of the weights; a model-level expert mask reaches
    every context, including through its already-captured step graphs."""
    cfg, wl = configs.C1()
    model = synth.generate_model(cfg, 46)
    shared = Model(cfg.hparams(), model)
    a = Context(None, wl.n_slots, wl.slot_cap, model=shared)
    b = Context(None, wl.n_slots, wl.slot_cap, model=shared)
    shared.close()                                  # the contexts keep the weights alive
    own = Context(cfg.hparams(), wl.n_slots, wl.slot_cap)
    own.upload(model)
    om, okv = oracle_pair(cfg, model, wl)
    fill_kv(cfg, wl, [a.kv_write, b.kv_write, own.kv_write])
    inp = synth.step_inputs(cfg, wl)
    want = own.step(inp.slot_idx, inp.n_past, emb=inp.emb)
    assert np.array_equal(a.step(inp.slot_idx, inp.n_past, emb=inp.emb), want)
    assert np.array_equal(b.step(inp.slot_idx, inp.n_past, emb=inp.emb), want)
    assert a.device_bytes(0) == b.device_bytes(0) == own.device_bytes(0)
    # drop half the experts of the first MoE layer on the shared model only
    L = next(i for i, k in enumerate(cfg.expert_used) if k > 0)
    keep = np.zeros(cfg.n_expert, np.uint8)
    keep[::2] = 1
    a.set_expert_mask(L, keep)
    own.set_expert_mask(L, keep)
    own.set_graphs(False)
    want_m = own.step(inp.slot_idx, inp.n_past, emb=inp.emb)
    assert not np.array_equal(want_m, want)
    assert np.array_equal(b.step(inp.slot_idx, inp.n_past, emb=inp.emb), want_m)
    a.set_capture(True)
    a.step(inp.slot_idx, inp.n_past, emb=inp.emb)
    T = len(inp.slot_idx)
    sel = a.read_capture(L, "sel", T).reshape(T, a.kmax)[:, :cfg.expert_used[L]]
    assert np.all(sel % 2 == 0), "a masked expert was routed"
    om.set_expert_mask(L, keep)
    _check_routing(cfg, a, om, T, model)            # masked routing bit-exact against the oracle
    a.set_capture(False)
    a.set_expert_mask(L, None)
    assert np.array_equal(b.step(inp.slot_idx, inp.n_past, emb=inp.emb), want)
    for c in (a, b, own):
        c.close()


def _prompt(cfg, n0, seed):
    rng = np.random.default_rng(seed)
    return np.concatenate([rng.integers(0, cfg.audio_vocab, (n0, cfg.n_codebooks)),
                           rng.integers(0, cfg.text_vocab + 1, (n0, 1))], axis=1).astype(np.int32)


def test_prefill_with_speaker_vs_oracle():
    """zonos2_batch_slot_prefill with a speaker row (graph.cpp:262-297, 703-760): the device prefill
    (speaker projections on the device, the prompt's own rows attended with fp32 K/V as the
    reference's one-graph prefill does, graph.cpp:155-169) against the oracle's prefill at the full
    bar: last-row logits and the f16 K/V rows left in the cache."""
    cfg, wl = configs.C1()
    model = synth.generate_model(cfg, 47)
    ctx = Context(cfg.hparams(), wl.n_slots, wl.slot_cap)
    ctx.upload(model)
    om = O.OracleModel(cfg.hparams(), model)
    n0, pos, slot = 12, 2, 1
    ids = _prompt(cfg, n0, 8)
    spk = synth.gen_normal_f32((cfg.spk_dim,), 3, "spk")
    delta = synth.gen_normal_f32((cfg.n_embd,), 4, "delta") * 0.1
    got = ctx.prefill(slot, ids, spk=spk, spk_pos=pos, delta=delta)
    okv = O.OracleKV(om, wl.n_slots, wl.slot_cap)
    want = O.prefill(om, okv, slot, ids, spk=spk, spk_pos=pos, delta=delta)
    assert_close("prefill(spk) vs oracle prefill", got, want)
    for L in range(cfg.n_layer):
        gk, gv = ctx.kv_read(L, slot, 0, n0)
        ok, ov = okv.read(L, slot, 0, n0)
        assert_close(f"prefill K rows L{L}", gk.view(np.float16).astype(np.float32), ok.view(np.float16).astype(np.float32))
        assert_close(f"prefill V rows L{L}", gv.view(np.float16).astype(np.float32), ov.view(np.float16).astype(np.float32))
    # the same prompt as row-by-row decode steps attends the f16 cache instead (the reference's decode
    # path): close, but not the prefill's numbers
    kv2 = O.OracleKV(om, wl.n_slots, wl.slot_cap)
    for t in range(n0):
        if t == pos:
            dec = O.step(om, kv2, [slot], [t], emb=_speaker_row_f32(model, spk, delta)[None, :])
        else:
            dec = O.step(om, kv2, [slot], [t], ids=ids[t:t + 1])
    assert_close("oracle prefill vs oracle steps", want, dec[0], cos_min=0.999, maxabs=1e-1)
    ctx.close()


def _speaker_row_f32(model, spk, delta):
    """spk_proj(spk_lda(spk) + b_lda) + b_proj + delta with the oracle's quantized matmuls"""
    lw, pw = model["spk_lda.weight"], model["spk_proj.weight"]
    sl = O.matmul(lw.type, lw.data, lw.ne[0], lw.ne[1], spk[None, :])[0] + model["spk_lda.bias"].data.view(np.float32)
    sp = O.matmul(pw.type, pw.data, pw.ne[0], pw.ne[1], sl[None, :])[0] + model["spk_proj.bias"].data.view(np.float32)
    return (sp + delta).astype(np.float32)


def test_layer_skip_vs_oracle():
    """Depth prune (zonos2_model::layer_skip): block 0 bypassed, through captured graphs too."""
    cfg, wl = configs.C1()
    model, ctx, om, okv = _build(cfg, wl, seed=48)
    inp = synth.step_inputs(cfg, wl)
    full = ctx.step(inp.slot_idx, inp.n_past, emb=inp.emb)        # captures the graph
    ctx.set_layer_skip([1, 0])
    om.set_layer_skip([1, 0])
    got = ctx.step(inp.slot_idx, inp.n_past, emb=inp.emb)
    want = O.step(om, okv, inp.slot_idx, inp.n_past, emb=inp.emb)
    assert_close("logits (block 0 skipped)", got, want)
    assert not np.array_equal(got, full)
    ctx.set_layer_skip(None)
    assert np.array_equal(ctx.step(inp.slot_idx, inp.n_past, emb=inp.emb), full)
    ctx.close()


def test_tiled_attention_equals_decode_steps():
    """Mixed passes append every row's K/V (k_kv_append) and attend through tiles of up to 16 rows of
    one slot at consecutive positions on MFMA (k_attn_fa, 128-key segments); decode steps append and
    attend in k_attn_chunk. A 100-row run of one slot in one mixed pass (tiles of 16 and a ragged 4)
    and the same rows stepped one by one leave bit-identical K/V rows (the same per-head norm, RoPE
    and f16 rounding) and logits within the parity bar (the two attention kernels sum in different
    orders)."""
    cfg, wl = configs.C1()
    model = synth.generate_model(cfg, 52)
    n0, slot = 100, 1
    ids = _prompt(cfg, n0, 13)
    m = Model(cfg.hparams(), model)
    a = Context(None, wl.n_slots, wl.slot_cap, model=m, max_rows=n0)
    print("one mixed pass of 100 rows", flush=True)
    rows = np.arange(n0, dtype=np.int32)
    got = a.step_mixed(np.full(n0, slot, np.int32), rows, ids, rows)
    b = Context(None, wl.n_slots, wl.slot_cap, model=m)
    print("100 decode steps", flush=True)
    for t in range(n0):
        lg = b.step([slot], [t], ids=ids[t:t + 1])
        assert_close(f"row {t} logits (mixed pass vs decode step)", got[t], lg[0])
    for L in range(cfg.n_layer):
        ka, va = a.kv_read(L, slot, 0, n0)
        kb, vb = b.kv_read(L, slot, 0, n0)
        np.testing.assert_array_equal(ka, kb)
        np.testing.assert_array_equal(va, vb)
    a.close(); b.close(); m.close()


def test_chunked_prefill_is_chunk_size_independent():
    """Chunked prefill (every row of a chunk appends its K/V before the chunk's attention, which reads
    the prompt's fp32 rows) gives the same bits for any chunk size: one row at a time, 7-row chunks
    (ragged last chunk, the speaker row inside a chunk) and the whole prompt in one chunk; the last-row
    logits also match the oracle's one-graph prefill (full bar)."""
    cfg, wl = configs.C1()
    model = synth.generate_model(cfg, 48)
    om = O.OracleModel(cfg.hparams(), model)
    n0, pos, slot = 61, 23, 2
    ids = _prompt(cfg, n0, 9)
    spk = synth.gen_normal_f32((cfg.spk_dim,), 5, "spk")
    outs, kvs = [], []
    for chunk in (1, 7, 256):
        ctx = Context(cfg.hparams(), wl.n_slots, wl.slot_cap)
        ctx.upload(model)
        ctx.set_prefill_chunk(chunk)
        print(f"prefill chunk {chunk}", flush=True)
        outs.append(ctx.prefill(slot, ids, spk=spk, spk_pos=pos))
        kvs.append([ctx.kv_read(L, slot, 0, n0) for L in range(cfg.n_layer)])
        ctx.close()
    for i in (1, 2):
        np.testing.assert_array_equal(outs[i], outs[0])
        for L in range(cfg.n_layer):
            np.testing.assert_array_equal(kvs[i][L][0], kvs[0][L][0])
            np.testing.assert_array_equal(kvs[i][L][1], kvs[0][L][1])
    okv = O.OracleKV(om, wl.n_slots, wl.slot_cap)
    want = O.prefill(om, okv, slot, ids, spk=spk, spk_pos=pos)
    assert_close("chunked prefill vs oracle prefill", outs[2], want)


def test_route_lists_in_lds_match_the_sorted_table():
    """Grouped matmuls list an expert's routes in LDS (small batches) or read k_route_sort's table
    (large batches, and whenever captures are on): both are the same stable grouping, so the step's
    logits are identical with capture on and off."""
    cfg, wl = configs.C2()
    model = synth.generate_model(cfg, 44)
    ctx = Context(cfg.hparams(), wl.n_slots, wl.slot_cap)
    ctx.upload(model)
    rng = np.random.default_rng(8)
    emb = rng.standard_normal((wl.n_slots, cfg.n_embd)).astype(np.float32)
    slots, npast = np.arange(wl.n_slots), np.zeros(wl.n_slots, np.int32)
    ctx.set_capture(True)
    a = ctx.step(slots, npast, emb=emb)
    ctx.set_capture(False)
    b = ctx.step(slots, npast, emb=emb)
    np.testing.assert_array_equal(a, b)
    ctx.close()


@pytest.mark.parametrize("E,k,T", [(64, 8, 2100), (48, 3, 300), (128, 4, 200), (128, 6, 40)])
def test_route_table_over_many_routes_and_experts(E, k, T):
    """The route grouping (mul_mat_id, src/zonos2-graph.cpp:222-231) of a wide MoE pass: 2100 tokens x
    top-8 of 64 experts is 16800 routes, more than one 1024 x 16-route chunk of the sort kernel; 48
    experts (not a power of two) x top-3; 128 experts (the most a model may have: two expert entries
    per lane in the router's top-k) through the wide (200 tokens) and the per-token (40) router. Router
    outputs and the counts, offsets and permutation are bit-exact against the oracle, the layer output
    within the bar, and the same pass without captures (experts listing their routes in LDS up to
    1024 routes) gives the same bits."""
    cfg = configs.ModelConfig("wide-route-sort", n_layer=1, n_embd=256, n_head=8, n_head_kv=2, head_dim=32,
                              n_expert=E, top_k=k, n_ff=256, bulk=configs.Q8_0, router_bias_std=1e-4)
    model = synth.generate_model(cfg, 46)
    ctx = Context(cfg.hparams(), T, 4)
    ctx.upload(model)
    om = O.OracleModel(cfg.hparams(), model)
    x = synth.gen_normal_f32((T, cfg.n_embd), 47, "inputs.moe")
    ctx.set_capture(True)
    got = ctx.moe_forward(0, x)
    ref = O.router(om, 0, x, None)
    sel = ctx.read_capture(0, "sel", T).reshape(T, ctx.kmax)[:, :k]
    assert np.array_equal(sel, ref["sel"])
    assert np.array_equal(ctx.read_capture(0, "probs", T).reshape(ref["probs"].shape).view(np.uint32),
                          ref["probs"].view(np.uint32))
    counts, offsets, perm = O.group(ref["sel"], E)
    assert np.array_equal(ctx.read_capture(0, "counts", T), counts)
    assert np.array_equal(ctx.read_capture(0, "offsets", T), offsets)
    assert np.array_equal(ctx.read_capture(0, "perm", T)[:T * k], perm)
    eo, out = O.experts(om, 0, x, ref["sel"], ref["w"])
    assert_close("moe out", got, out)
    ctx.set_capture(False)
    np.testing.assert_array_equal(ctx.moe_forward(0, x), got)
    ctx.close()
