"""The flash attention kernels at every query-head group they are built for (head_dim 128 with 1, 2 or
4 query heads per KV head), on one-layer Q8_0 models: a per-slot prefill of a 150-row prompt (three
64-key segments; the prompt's rows attend to their fp32 K/V through k_attn_flash32) against the
oracle's prefill, and a mixed pass of two prefill chunks and two decode columns (bands up to 201
keys, k_attn_flash16 over the f16 cache) against the oracle's mixed step, both at the full bar, the
mixed pass also bit for bit against the same rows run as separate passes."""
import numpy as np
import pytest

import oracle_py as O
from helpers import assert_close
from test_gpu_mixed import _batch, _fill
from zonos2_amd import configs, synth
from zonos2_amd.z2h import Context, Model

pytestmark = pytest.mark.gpu


def _cfg(grp):
    return configs.ModelConfig(f"hd128-grp{grp}", n_layer=1, n_embd=256, n_head=2 * grp, n_head_kv=2, head_dim=128,
                               n_expert=8, top_k=2, n_ff=256, bulk=configs.Q8_0)


@pytest.mark.parametrize("grp", [1, 2, 4])
def test_flash_prefill_vs_oracle(grp):
    cfg = _cfg(grp)
    model = synth.generate_model(cfg, 80 + grp)
    ctx = Context(cfg.hparams(), 2, 256, max_rows=256)
    ctx.upload(model)
    om = O.OracleModel(cfg.hparams(), model)
    rng = np.random.default_rng(90 + grp)
    n0, slot = 150, 1
    ids = np.concatenate([rng.integers(0, cfg.audio_vocab, (n0, cfg.n_codebooks)),
                          rng.integers(0, cfg.text_vocab + 1, (n0, 1))], axis=1).astype(np.int32)
    print(f"{cfg.name}: {n0}-row prefill", flush=True)
    got = ctx.prefill(slot, ids)
    okv = O.OracleKV(om, 2, 256)
    want = O.prefill(om, okv, slot, ids)
    c, m = assert_close(f"{cfg.name} prefill logits", got, want)
    print(f"{cfg.name}: prefill logits cos {c:.8f} max |d| {m:.3e}", flush=True)
    gk, gv = ctx.kv_read(0, slot, 0, n0)
    ok, ov = okv.read(0, slot, 0, n0)
    assert_close("K rows", gk.view(np.float16).astype(np.float32), ok.view(np.float16).astype(np.float32))
    assert_close("V rows", gv.view(np.float16).astype(np.float32), ov.view(np.float16).astype(np.float32))
    ctx.close()


@pytest.mark.parametrize("grp", [1, 2, 4])
def test_flash_mixed_pass_vs_oracle_and_separate_passes(grp):
    cfg = _cfg(grp)
    model = synth.generate_model(cfg, 70 + grp)
    m = Model(cfg.hparams(), model)
    rng = np.random.default_rng(60 + grp)
    cap = 256
    chunks, decodes = [(0, 0, 40, False), (1, 150, 36, False)], [(2, 130), (3, 200)]
    pre = {1: 150, 2: 130, 3: 200}
    slots, npast, ids, emap, emb, groups = _batch(cfg, rng, chunks, decodes)
    out_rows = np.array([g[-1] for g in groups] + [5, groups[1][3]], np.int32)
    print(f"{cfg.name}: {len(slots)} rows in one mixed pass", flush=True)
    ctx = Context(None, 4, cap, model=m)
    om = O.OracleModel(cfg.hparams(), model)
    okv = O.OracleKV(om, 4, cap)
    for s, n in pre.items():
        _fill(cfg, [ctx.kv_write, okv.write], s, n, 70 + s)
    got = ctx.step_mixed(slots, npast, ids, out_rows, emb_map=emap, emb=emb)
    want = O.step_mixed(om, okv, slots, npast, ids, emb_map=emap, emb=emb)[out_rows]
    worst = 1.0
    for i, r in enumerate(out_rows):
        c, _ = assert_close(f"mixed row {r}", got[i], want[i])
        worst = min(worst, c)
    print(f"{cfg.name}: worst row cos {worst:.8f}", flush=True)
    ctx2 = Context(None, 4, cap, model=m)
    for s, n in pre.items():
        _fill(cfg, [ctx2.kv_write], s, n, 70 + s)
    sep = {}
    for g in groups:
        gi = np.array(g)
        lo = ctx2.step_mixed(slots[gi], npast[gi], ids[gi], np.arange(len(g)), emb_map=emap[gi], emb=emb)
        for j, r in enumerate(g):
            sep[r] = lo[j]
    for i, r in enumerate(out_rows):
        np.testing.assert_array_equal(got[i], sep[int(r)])
    ctx.close(); ctx2.close(); m.close()
