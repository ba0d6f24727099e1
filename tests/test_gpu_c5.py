"""The mixed chunked-prefill + decode pass at the 24-layer model's shapes (d_model 2048, 16 / 4 heads,
head_dim 128, 32 experts top-4, SwiGLU 1536, 9 x 1025 logits) on a two-layer depth cut, with Q4_K and
with F16 weights, on two layouts: bench.py's timed pass (8 chunks + 32 decode columns, 2088 rows) and a
small one (2 chunks + 8 decode columns). The prompt chunks are 256 rows, each after a speaker row (a 2048-d N(0,1) speaker vector
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


@pytest.mark.parametrize("layout", ["two-chunks", "timed"])
@pytest.mark.parametrize("bulk", [configs.Q4_K, configs.F16], ids=["q4_k", "f16"])
def test_c5_mixed_pass_layers_teacher_forced(bulk, layout):
    cfg = dataclasses.replace(configs.zonos2_24l(bulk), n_layer=2, expert_used=[4, 4])
    model = synth.generate_model(cfg, 5)
    # "timed": bench.py's pass (seed 55: 8 chunks of 256 rows after speaker rows + 32 decode columns =
    # 2088 rows, ~261 routes per expert, several 64-route GEMM tiles per expert); "two-chunks": 2 chunks
    # + 8 decode columns
    lay = configs.mixed_layout(cfg) if layout == "timed" else configs.mixed_layout(cfg, seed=17, n_pre=2, n_dec=N_DEC)
    slots, npast, emap, ids, out_rows = lay.slots, lay.npast, lay.emap, lay.ids, lay.out_rows
    n_pre = len(lay.r0)
    T, d, E, k = len(slots), cfg.n_embd, cfg.n_expert, cfg.top_k
    cap = lay.cap
    n_slots = n_pre + len(lay.dlen)
    m = Model(cfg.hparams(), model)
    # captures are sized for n_slots columns: one slot per row of the pass (only n_slots are used)
    ctx = Context(None, T, cap, model=m, max_rows=T)
    om = O.OracleModel(cfg.hparams(), model)

    def prefilled_kv(writers):
        for L in range(cfg.n_layer):
            for s_, n in list(enumerate(lay.r0)) + [(n_pre + i, n) for i, n in enumerate(lay.dlen)]:
                if n:
                    kk, vv = synth.kv_rows(cfg, L, s_, n, 21)
                    for w in writers:
                        w(L, s_, 0, kk, vv)

    okv = O.OracleKV(om, n_slots, cap)
    prefilled_kv([ctx.kv_write, okv.write])
    # speaker rows on the device, checked against the oracle's projection
    spk = lay.spk
    emb = ctx.speaker_embed(spk)
    assert_close("speaker rows", emb, _speaker_rows_oracle(model, spk))
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
        c_o, m_o = assert_close(f"L{L} attn_o", rd(L, "attn_o").reshape(T, -1), ao)
        print(f"L{L}: attention output vs the oracle: cos {c_o:.8f} max |d| {m_o:.3e}", flush=True)
        for s_, n_ in list(enumerate(lay.r0)) + [(n_pre + i, n) for i, n in enumerate(lay.dlen)]:
            rows = CHUNK + 1 if s_ < n_pre else 1
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
        exact = np.array_equal(ffn_out.view(np.uint32), out.view(np.uint32))
        if L + 1 < cfg.n_layer:
            assert np.array_equal(rd(L + 1, "res_in").reshape(T, d), ffn_out + (attn_out + res_in)), f"L{L} residual fold"
        prev = r["rh"]
        gcap[L] = {"ffn_in": ffn_in, "sel": sel}
        print(f"L{L}: {counts.max()} routes on the busiest expert, {int((counts > 0).sum())} experts touched; "
              f"experts' output bit-identical to the oracle's: {exact}", flush=True)
    hn = ctx.read_capture(0, "out_norm", T).reshape(T, d)
    hw = model["output.weight"]
    mout = O.matmul(hw.type, hw.data, hw.ne[0], hw.ne[1], hn[out_rows]).astype(np.float64)
    assert_close("head + softcap", got, cfg.logit_softcap * np.tanh(mout / cfg.logit_softcap))
    # end to end against the oracle's mixed pass on a fresh copy of the pre-filled cache
    okv2 = O.OracleKV(om, n_slots, cap)
    prefilled_kv([okv2.write])
    want = O.step_mixed(om, okv2, slots, npast, ids, emb_map=emap, emb=emb)[out_rows]
    c_e2e = cos(got, want)
    print(f"{cfg.name}: worst per-layer cos {worst:.7f}; end-to-end logits cos {c_e2e:.7f} maxabs {np.abs(got - want).max():.3e}")
    assert c_e2e >= 0.999                             # two layers: routing feedback barely moves the logits
    ctx.close()
    m.close()
