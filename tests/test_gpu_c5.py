"""The mixed chunked-prefill + decode pass at the 24-layer model's shapes (d_model 2048, 16 / 4 heads,
head_dim 128, 32 experts top-4, SwiGLU 1536, 9 x 1025 logits) on a two-layer depth cut, with Q4_K and
with F16 weights: two 256-row prompt chunks, each after a speaker row (a 2048-d N(0,1) speaker vector
through spk_lda -> spk_proj on the device, z2h_speaker_embed), at 256-aligned offsets inside their
prompts (the earlier rows pre-filled in the cache), plus decode columns, all in one z2h_step_mixed
pass. Every layer is checked with the device's own layer inputs against the oracle (the mixed
pass's per-layer arithmetic is the decode step's, which orc_step_mixed / orc_attention restate,
pinned on orc_step in test_oracle_mixed.py): attention from attn_in for every row (K/V appended
before the attention, a slot's rows causal), the router bit-exact from ffn_in, the experts on the
device's routing, the residual folds bit-exact, the head from out_norm, and the K/V rows the pass
wrote. The speaker rows are checked against the oracle's projection. End to end, the requested rows'
logits against orc_step_mixed."""
import dataclasses

import numpy as np
import pytest

import oracle_py as O
from helpers import assert_close, cos
from zonos2_amd import configs, synth
from zonos2_amd.z2h import Context, Model

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

CHUNK, N_DEC = 256, 8


def _speaker_rows_oracle(model, spk):
    lw, pw = model["spk_lda.weight"], model["spk_proj.weight"]
    sl = O.matmul(lw.type, lw.data, lw.ne[0], lw.ne[1], spk) + model["spk_lda.bias"].data.view(np.float32)[None, :]
    return O.matmul(pw.type, pw.data, pw.ne[0], pw.ne[1], sl) + model["spk_proj.bias"].data.view(np.float32)[None, :]


@pytest.mark.parametrize("bulk", [configs.Q4_K, configs.F16], ids=["q4_k", "f16"])
def test_c5_mixed_pass_layers_teacher_forced(bulk):
    cfg = dataclasses.replace(configs.zonos2_24l(bulk), n_layer=2, expert_used=[4, 4])
    model = synth.generate_model(cfg, 5)
    rng = np.random.default_rng(17)
    # two prompts: a chunk of CHUNK rows at a 256-aligned offset, after a speaker row
    r0 = [256, 512]
    dec_lens = [int(x) for x in rng.integers(32, 700, N_DEC)]
    slots, npast, emap = [], [], []
    for i, r in enumerate(r0):
        for j in range(CHUNK + 1):                   # the speaker row, then the chunk's prompt rows
            slots.append(i); npast.append(r + j); emap.append(i if j == 0 else -1)
    for i, n in enumerate(dec_lens):
        slots.append(2 + i); npast.append(n); emap.append(-1)
    slots, npast, emap = np.array(slots, np.int32), np.array(npast, np.int32), np.array(emap, np.int32)
    T, d, E, k = len(slots), cfg.n_embd, cfg.n_expert, cfg.top_k
    ids = np.concatenate([rng.integers(0, cfg.audio_vocab, (T, cfg.n_codebooks)),
                          rng.integers(0, cfg.text_vocab + 1, (T, 1))], axis=1).astype(np.int32)
    cap = max(r + CHUNK + 1 for r in r0) + 1
    m = Model(cfg.hparams(), model)
    # capture buffers hold n_slots rows: one slot per row of the pass (only 10 are written)
    ctx = Context(None, T, cap, model=m, max_rows=T)
    om = O.OracleModel(cfg.hparams(), model)
    okv = O.OracleKV(om, T, cap)
    for L in range(cfg.n_layer):
        for i, r in enumerate(r0):
            kk, vv = synth.kv_rows(cfg, L, i, r, 21)
            ctx.kv_write(L, i, 0, kk, vv); okv.write(L, i, 0, kk, vv)
        for i, n in enumerate(dec_lens):
            kk, vv = synth.kv_rows(cfg, L, 2 + i, n, 21)
            ctx.kv_write(L, 2 + i, 0, kk, vv); okv.write(L, 2 + i, 0, kk, vv)
    # speaker rows on the device, checked against the oracle's projection
    spk = rng.standard_normal((len(r0), cfg.spk_dim)).astype(np.float32)
    emb = ctx.speaker_embed(spk)
    assert_close("speaker rows", emb, _speaker_rows_oracle(model, spk))
    out_rows = np.array([CHUNK, 2 * CHUNK + 1] + list(range(2 * (CHUNK + 1), T)), np.int32)
    ctx.set_capture(True)
    print(f"{cfg.name}: {T} rows in one mixed pass", flush=True)
    got = ctx.step_mixed(slots, npast, ids, out_rows, emb_map=emap, emb=emb)
    rd = lambda L, n: ctx.read_capture(L, n, T)
    prev = None
    gcap, worst = {}, 1.0
    for L in range(cfg.n_layer):
        res_in = rd(L, "res_in").reshape(T, d)
        attn_in = rd(L, "attn_in").reshape(T, d)
        ffn_in = rd(L, "ffn_in").reshape(T, d)
        attn_out = rd(L, "attn_out").reshape(T, d)
        ffn_out = rd(L, "ffn_out").reshape(T, d)
        ao = np.empty((T, cfg.n_head * cfg.head_dim), np.float32)
        oo = np.empty((T, d), np.float32)
        O.check(O.lib().orc_attention(om.m, okv.kv, L, T, O.ptr(slots), O.ptr(npast), O.ptr(attn_in), O.ptr(ao), O.ptr(oo)))
        c, _ = assert_close(f"L{L} attn_out", attn_out, oo)
        worst = min(worst, c)
        assert_close(f"L{L} attn_o", rd(L, "attn_o").reshape(T, -1), ao)
        for s_, n_ in [(0, r0[0]), (1, r0[1])] + [(2 + i, n) for i, n in enumerate(dec_lens)]:
            rows = CHUNK + 1 if s_ < 2 else 1
            gk, gv = ctx.kv_read(L, s_, n_, rows)
            ok_, ov = okv.read(L, s_, n_, rows)
            assert_close(f"L{L} K rows slot {s_}", gk.view(np.float16).astype(np.float32), ok_.view(np.float16).astype(np.float32))
            assert_close(f"L{L} V rows slot {s_}", gv.view(np.float16).astype(np.float32), ov.view(np.float16).astype(np.float32))
        r = O.router(om, L, ffn_in, prev)
        sel = rd(L, "sel").reshape(T, k)
        assert np.array_equal(sel, r["sel"]), f"L{L} top-k ids"
        assert np.array_equal(rd(L, "probs").reshape(T, E).view(np.uint32), r["probs"].view(np.uint32)), f"L{L} probs"
        counts, offsets, perm = O.group(sel, E)
        assert np.array_equal(rd(L, "perm"), perm) and np.array_equal(rd(L, "offsets"), offsets)
        w = rd(L, "weights").reshape(T, k)
        _, out = O.experts(om, L, ffn_in, sel, w)
        c, _ = assert_close(f"L{L} ffn_out", ffn_out, out)
        worst = min(worst, c)
        if L + 1 < cfg.n_layer:
            assert np.array_equal(rd(L + 1, "res_in").reshape(T, d), ffn_out + (attn_out + res_in)), f"L{L} residual fold"
        prev = r["rh"]
        gcap[L] = {"ffn_in": ffn_in, "sel": sel}
        print(f"L{L}: {counts.max()} routes on the busiest expert, {int((counts > 0).sum())} experts touched", flush=True)
    hn = ctx.read_capture(0, "out_norm", T).reshape(T, d)
    hw = model["output.weight"]
    mout = O.matmul(hw.type, hw.data, hw.ne[0], hw.ne[1], hn[out_rows]).astype(np.float64)
    assert_close("head + softcap", got, cfg.logit_softcap * np.tanh(mout / cfg.logit_softcap))
    # end to end against the oracle's mixed pass on a fresh copy of the pre-filled cache
    okv2 = O.OracleKV(om, T, cap)
    for L in range(cfg.n_layer):
        for i, r in enumerate(r0):
            kk, vv = synth.kv_rows(cfg, L, i, r, 21)
            okv2.write(L, i, 0, kk, vv)
        for i, n in enumerate(dec_lens):
            kk, vv = synth.kv_rows(cfg, L, 2 + i, n, 21)
            okv2.write(L, 2 + i, 0, kk, vv)
    want = O.step_mixed(om, okv2, slots, npast, ids, emb_map=emap, emb=emb)[out_rows]
    c_e2e = cos(got, want)
    print(f"{cfg.name}: worst per-layer cos {worst:.7f}; end-to-end logits cos {c_e2e:.7f} maxabs {np.abs(got - want).max():.3e}")
    assert c_e2e >= 0.999                             # two layers: routing feedback barely moves the logits
    ctx.close()
    m.close()
