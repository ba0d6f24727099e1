"""Token-id embeddings on the device: the step's first kernel sums the W table rows of each token's
ids in column order (src/zonos2-graph.cpp:248-260) and applies emb_norm (graph.cpp:300). When all
tables share one type (F32, F16 or Q8_0) it reads them without a per-table type switch; otherwise
it takes the generic gather. Each variant's layer-0 residual (the normalised embedding) equals the
oracle's bit for bit: the same dequantised values, the same fp32 additions in table order and the
same emb_norm arithmetic. The step's logits are held to the usual bar."""
import dataclasses

import numpy as np
import pytest

import oracle_py as O
from helpers import assert_close, fill_kv
from zonos2_amd import configs, synth
from zonos2_amd.z2h import Context

pytestmark = pytest.mark.gpu

VARIANTS = {
    "f32": lambda kk, ncb: configs.F32,
    "f16": lambda kk, ncb: configs.F16,
    "q8_0": lambda kk, ncb: configs.Q8_0,
    "mixed": lambda kk, ncb: configs.Q8_0 if kk < ncb else configs.F32,
}


def _model(variant):
    cfg, wl = configs.C1()
    wl = dataclasses.replace(wl, inject_embeddings=False)
    model = synth.generate_model(cfg, 71)
    ncb = cfg.n_codebooks
    for n, t, ne, init in cfg.tensors():
        kk = int(n.split(".")[1]) if n.startswith("audio_embd.") else ncb if n == "text_embd.weight" else None
        if kk is not None:
            model[n] = synth.generate_tensor(n, VARIANTS[variant](kk, ncb), ne, init, 71)
    return cfg, wl, model


@pytest.mark.parametrize("variant", list(VARIANTS))
def test_token_id_embeddings_vs_oracle(variant):
    cfg, wl, model = _model(variant)
    ctx = Context(cfg.hparams(), wl.n_slots, wl.slot_cap)
    ctx.upload(model)
    om = O.OracleModel(cfg.hparams(), model)
    okv = O.OracleKV(om, wl.n_slots, wl.slot_cap)
    fill_kv(cfg, wl, [ctx.kv_write, okv.write])
    inp = synth.step_inputs(cfg, wl)
    T = len(inp.slot_idx)
    print(f"{variant}: {T}-token step from ids", flush=True)
    ctx.set_capture(True)
    got = ctx.step(inp.slot_idx, inp.n_past, ids=inp.ids)
    res0 = ctx.read_capture(0, "res_in", T).reshape(T, cfg.n_embd)
    ctx.set_capture(False)
    want, cap = O.step(om, okv, inp.slot_idx, inp.n_past, ids=inp.ids, capture=True)
    ref0 = cap["res_in"][0]
    print(f"{variant}: layer-0 residual max |d| {np.abs(res0.astype(np.float64) - ref0).max():.3e}", flush=True)
    np.testing.assert_array_equal(res0, ref0, err_msg=f"{variant} layer-0 residual")
    assert_close(f"{variant} logits", got, want)
    ctx.close()
