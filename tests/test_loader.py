"""GGUF loader conformance on the reference's own fixture, tests/golden/dummy-zonos2.gguf (copied
from the reference's tests/fixtures/): the library's loader (zonos2_model_read_meta, the host half
of zonos2_model_load) reads every key and tensor the reference's loader reads
(src/zonos2.cpp:34-71, 137-183), router_dim from router_down ne1 (src/zonos2.cpp:241-246), and agrees
with an independent Python reading of the same file."""
import json
import subprocess

import numpy as np

import oracle_py as O
from gguf_read import hparams, read
from zonos2_amd.lib import BUILD

FIXTURE = "tests/golden/dummy-zonos2.gguf"


def _info(root):
    out = subprocess.run([str(BUILD / "zonos2-batch"), "--model", str(root / FIXTURE), "--info"],
                         check=True, capture_output=True, text=True).stdout
    return json.loads(out)


def test_loader_reads_every_key_and_tensor(root):
    info = _info(root)
    version, kv, tensors = read(root / FIXTURE)
    hp = hparams(kv, tensors)
    for k, v in info["hparams"].items():
        want = hp[k]
        if isinstance(v, float):
            assert np.float32(v) == np.float32(want), k
        else:
            assert v == want, k
    assert info["router_dim"] == hp["router_dim"] == 32
    assert {n: list(t.ne) for n, t in tensors.items()} == info["tensors"]
    # the reference's required set (src/zonos2.cpp:137-183)
    names = set(info["tensors"])
    req = {"text_embd.weight", "spk_lda.weight", "spk_lda.bias", "spk_proj.weight", "spk_proj.bias",
           "output_norm.weight", "output.weight"} | {f"audio_embd.{i}.weight" for i in range(hp["n_codebooks"])}
    for L, k in enumerate(hp["expert_used"]):
        b = f"blk.{L}."
        req |= {b + n for n in ("attn_norm.weight", "ffn_norm.weight", "attn_q.weight", "attn_k.weight",
                                "attn_v.weight", "attn_output.weight", "attn_temp", "attn_gate.weight")}
        if k:
            req |= {b + n for n in ("ffn_gate_exps.weight", "ffn_up_exps.weight", "ffn_down_exps.weight",
                                    "router_down.weight", "router_down.bias", "router_mlp0.weight", "router_mlp0.bias",
                                    "router_mlp2.weight", "router_mlp2.bias", "router_mlp4.weight", "router_norm.weight",
                                    "router_bias")}
        else:
            req |= {b + n for n in ("ffn_up.weight", "ffn_gate.weight", "ffn_down.weight")}
    assert req <= names
    # shapes the graph relies on (ggml ne order)
    d, av, ncb = hp["n_embd"], hp["audio_vocab"], hp["n_codebooks"]
    assert info["tensors"]["text_embd.weight"] == [d, hp["text_vocab"] + 1]
    assert info["tensors"]["output.weight"] == [d, ncb * av]
    assert info["tensors"]["blk.1.ffn_up_exps.weight"] == [d, hp["n_ff"], hp["n_expert"]]
    assert "blk.1.router_eda_scale" not in names and "blk.2.router_eda_scale" in names   # first MoE layer has none


def test_fixture_runs_through_the_oracle(root):
    """The fixture is a complete model: the oracle decodes a step on it (dense layers 0 and 3, MoE
    1 and 2 with top-1 and top-2 of 4 experts, F16 weights)."""
    _, kv, tensors = read(root / FIXTURE)
    hp = hparams(kv, tensors)
    om = O.OracleModel(hp, tensors)
    okv = O.OracleKV(om, 2, 16)
    ids = np.array([[1, 2, 3, 4, 5, 6, 7, 8, 9, 10], [1024, 1025, 0, 0, 0, 0, 0, 0, 0, 519]], np.int32)
    logits = O.step(om, okv, [0, 1], [0, 0], ids=ids)
    assert logits.shape == (2, hp["n_codebooks"] * hp["audio_vocab"])
    assert np.isfinite(logits).all() and np.abs(logits).max() <= hp["logit_softcap"]
