"""Passes wider than 64 rows (prefill chunks, mixed passes, wide decode batches) run their Q4_K and F16
matmuls as MFMA GEMMs (k_gemm_q4k, k_gemm_f16); narrower ones run the decode GEMVs. The model is a
two-layer cut of the 24-layer shapes (d_model 2048, 16 / 4 heads, head_dim 128, SwiGLU 1536) with a
dense FFN block (dense gate/up/down GEMMs) and an MoE block (32 experts top-4, grouped GEMMs).

Q4_K: every Q4_K matmul folds a row's superblocks in order with the same operations
(fma(dx, fma(d, isum, -dmin * msum), acc)); F16: every F16 matmul runs on k_gemm_f16 (wide or narrow
tiles), the same chain of f16 MFMA products per row. Q6_K: every Q6_K matmul runs on the 16-row MFMA
GEMV at every width (experts in 8- or 16-route passes, dense projections in 16-token passes), each
row adding its superblocks' (d * dx) * sum in order. So a row's logits and K/V are the same bits in a
96-column step and in 16-column steps, and a prompt prefilled in 200-row chunks equals one prefilled
in 16-row chunks. The wide step is held to the oracle layer by layer (teacher-forced, full bar)."""
import dataclasses

import numpy as np
import pytest

import oracle_py as O
from helpers import assert_close, check_layers_teacher_forced, cos
from zonos2_amd import configs, synth
from zonos2_amd.z2h import Context, Model

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

N_SLOTS = 96


def _cut(bulk, seed):
    cfg = dataclasses.replace(configs.zonos2_24l(bulk), n_layer=2, expert_used=[0, 4])
    return cfg, synth.generate_model(cfg, seed)


def _ctx(cfg, model, lens, cap):
    m = Model(cfg.hparams(), model)
    ctx = Context(None, N_SLOTS, cap, model=m)
    om = O.OracleModel(cfg.hparams(), model)
    okv = O.OracleKV(om, N_SLOTS, cap)
    for L in range(cfg.n_layer):
        for s, n in enumerate(lens):
            k, v = synth.kv_rows(cfg, L, s, n, 31)
            ctx.kv_write(L, s, 0, k, v)
            okv.write(L, s, 0, k, v)
    return m, ctx, om, okv


@pytest.mark.parametrize("bulk", [configs.Q4_K, configs.F16, configs.Q6_K], ids=["q4_k", "f16", "q6_k"])
def test_wide_step_gemm_equals_narrow_steps_and_oracle(bulk):
    cfg, model = _cut(bulk, 61)
    rng = np.random.default_rng(62)
    lens = [int(x) for x in rng.integers(1, 500, N_SLOTS)]
    m, ctx, om, okv = _ctx(cfg, model, lens, 512)
    slots = np.arange(N_SLOTS, dtype=np.int32)
    npast = np.array(lens, np.int32)
    ids = np.concatenate([rng.integers(0, cfg.audio_vocab, (N_SLOTS, cfg.n_codebooks)),
                          rng.integers(0, cfg.text_vocab + 1, (N_SLOTS, 1))], axis=1).astype(np.int32)
    print(f"{cfg.name}: {N_SLOTS}-column step (GEMM path)", flush=True)
    ctx.set_capture(True)
    wide = ctx.step(slots, npast, ids=ids)
    worst = check_layers_teacher_forced(ctx, om, okv, model, cfg, N_SLOTS, slots, npast, wide, cfg.name)
    ctx.set_capture(False)
    wide_kv = [ctx.kv_read(L, s, lens[s], 1) for L in range(cfg.n_layer) for s in (0, 47, 95)]
    narrow = np.concatenate([ctx.step(slots[i:i + 16], npast[i:i + 16], ids=ids[i:i + 16]) for i in range(0, N_SLOTS, 16)])
    narrow_kv = [ctx.kv_read(L, s, lens[s], 1) for L in range(cfg.n_layer) for s in (0, 47, 95)]
    print(f"{cfg.name}: worst per-layer cos {worst:.7f}; wide vs narrow max |d| {np.abs(wide - narrow).max():.3e}", flush=True)
    np.testing.assert_array_equal(wide, narrow)
    for a, b in zip(wide_kv, narrow_kv):
        np.testing.assert_array_equal(a[0], b[0])
        np.testing.assert_array_equal(a[1], b[1])
    ctx.close()
    m.close()


def test_q4k_prefill_chunks_across_the_gemm_width():
    """A 200-row prompt prefilled in one 200-row chunk (GEMMs) and in 16-row chunks (GEMVs): same
    last-row logits and K/V bits; both against the oracle's one-graph prefill."""
    cfg, model = _cut(configs.Q4_K, 63)
    rng = np.random.default_rng(64)
    n0, pos, slot = 200, 37, 5
    ids = np.concatenate([rng.integers(0, cfg.audio_vocab, (n0, cfg.n_codebooks)),
                          rng.integers(0, cfg.text_vocab + 1, (n0, 1))], axis=1).astype(np.int32)
    spk = rng.standard_normal(cfg.spk_dim).astype(np.float32)
    outs, kvs = [], []
    m = Model(cfg.hparams(), model)
    for chunk in (200, 16):
        ctx = Context(None, 8, 256, model=m)
        ctx.set_prefill_chunk(chunk)
        print(f"prefill chunk {chunk}", flush=True)
        outs.append(ctx.prefill(slot, ids, spk=spk, spk_pos=pos))
        kvs.append([ctx.kv_read(L, slot, 0, n0) for L in range(cfg.n_layer)])
        ctx.close()
    np.testing.assert_array_equal(outs[0], outs[1])
    for L in range(cfg.n_layer):
        np.testing.assert_array_equal(kvs[0][L][0], kvs[1][L][0])
        np.testing.assert_array_equal(kvs[0][L][1], kvs[1][L][1])
    # end to end through both layers (the MoE layer's routing of the last row can round the other way
    # on a near-tie); the per-layer bar is held by the teacher-forced wide-step test above
    om = O.OracleModel(cfg.hparams(), model)
    want = O.prefill(om, O.OracleKV(om, 8, 256), slot, ids, spk=spk, spk_pos=pos)
    c = cos(outs[0], want)
    print(f"200-row prefill vs oracle prefill: cos {c:.7f} max |d| {np.abs(outs[0] - want).max():.3e}", flush=True)
    assert c >= 0.9999
    m.close()
