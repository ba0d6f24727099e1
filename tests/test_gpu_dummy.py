"""The reference's own fixture model (tests/golden/dummy-zonos2.gguf: 4 blocks, dense 0 and 3, MoE 1
and 2 with top-1 / top-2 of 4 experts, router_dim 32, head_dim 16, F16 weights) through the device
library: steps and a speaker prefill against the oracle on the same file, and the zonos2.h API's
--batch-test / --decode-bench harness (F.1 / F.2 of src/main.cpp:158-285)."""
import subprocess

import numpy as np
import pytest

import oracle_py as O
from gguf_read import hparams, read
from helpers import assert_close
from zonos2_amd.lib import BUILD
from zonos2_amd.z2h import Context

pytestmark = pytest.mark.gpu
FIXTURE = "tests/golden/dummy-zonos2.gguf"


@pytest.fixture(scope="module")
def dummy(root):
    _, kv, tensors = read(root / FIXTURE)
    return hparams(kv, tensors), tensors


def _ids(hp, T, seed):
    rng = np.random.default_rng(seed)
    return np.concatenate([rng.integers(0, hp["audio_vocab"], (T, hp["n_codebooks"])),
                           rng.integers(0, hp["text_vocab"] + 1, (T, 1))], axis=1).astype(np.int32)


def test_dummy_model_steps_vs_oracle(dummy):
    hp, tensors = dummy
    n_slots, cap = 4, 40
    ctx = Context(hp, n_slots, cap)
    ctx.upload(tensors)
    om = O.OracleModel(hp, tensors)
    okv = O.OracleKV(om, n_slots, cap)
    # prefill ragged prompts row by row on both sides, then decode a few batched steps
    lens = [3, 9, 1, 14]
    for s, n in enumerate(lens):
        ids = _ids(hp, n, 10 + s)
        for t in range(n):
            ctx.step([s], [t], ids=ids[t:t + 1])
            O.step(om, okv, [s], [t], ids=ids[t:t + 1])
    ctx.set_capture(True)
    npast = list(lens)
    for it in range(3):
        ids = _ids(hp, n_slots, 50 + it)
        got = ctx.step(list(range(n_slots)), npast, ids=ids)
        want, cap_o = O.step(om, okv, list(range(n_slots)), npast, ids=ids, capture=True)
        assert_close(f"dummy logits step {it}", got, want)
        for L, k in enumerate(hp["expert_used"]):
            if not k:
                continue
            # the layer's own top-k rows [T][k] lead the T * kmax capture buffer
            sel = ctx.read_capture(L, "sel", n_slots).ravel()[:n_slots * k].reshape(n_slots, k)
            assert np.array_equal(sel, cap_o["sel"][L][:, :k]), f"layer {L} routing"
        npast = [n + 1 for n in npast]
    ctx.close()


def test_dummy_model_speaker_prefill_vs_oracle(dummy):
    hp, tensors = dummy
    ctx = Context(hp, 2, 32)
    ctx.upload(tensors)
    om = O.OracleModel(hp, tensors)
    ids = _ids(hp, 7, 3)
    rng = np.random.default_rng(4)
    spk = rng.standard_normal(hp["spk_dim"]).astype(np.float32)
    delta = (0.1 * rng.standard_normal(hp["n_embd"])).astype(np.float32)
    got = ctx.prefill(1, ids, spk=spk, spk_pos=0, delta=delta)
    want = O.prefill(om, O.OracleKV(om, 2, 32), 1, ids, spk=spk, spk_pos=0, delta=delta)
    assert_close("dummy prefill(spk)", got, want)
    ctx.close()


def _cli(*args):
    r = subprocess.run([str(BUILD / "zonos2-batch"), *args], capture_output=True, text=True, timeout=300)
    print(r.stdout[-3000:], r.stderr[-2000:])
    return r


def test_batch_test_harness_on_fixture(root):
    r = _cli("--model", str(root / FIXTURE), "--batch-test", "--greedy", "--slots", "5", "--requests", "4",
             "--dup", "--max-frames", "24", "--prompt-len", "12")
    assert r.returncode == 0 and "batch-test: OK" in r.stdout
    assert "batch == alone for every request: yes" in r.stdout
    r = _cli("--model", str(root / FIXTURE), "--batch-test", "--slots", "3", "--requests", "3",
             "--max-frames", "16", "--prompt-len", "10", "--seed", "9")
    assert r.returncode == 0 and "batch == alone for every request: yes" in r.stdout


def test_decode_bench_harness_on_fixture(root):
    r = _cli("--model", str(root / FIXTURE), "--decode-bench", "--slots", "4", "--steps", "16", "--prompt-len", "8")
    assert r.returncode == 0 and "decode-bench: slots=4 steps=16" in r.stdout


def test_batch_test_harness_with_gpu_sampling(root):
    """The batched run samples on the GPU (zonos2_batch_sample), the per-request reference runs on
    the host sampler: greedy codes must agree exactly (F.1 / F.2 as in the reference's harness); with
    sampling, identical prompts in two slots must still draw identical codes (F.2)."""
    r = _cli("--model", str(root / FIXTURE), "--batch-test", "--greedy", "--gpu-sample", "--slots", "5", "--requests", "4",
             "--dup", "--max-frames", "24", "--prompt-len", "12")
    assert r.returncode == 0 and "batch-test: OK" in r.stdout, r.stdout + r.stderr
    assert "batch == alone for every request: yes" in r.stdout
    r = _cli("--model", str(root / FIXTURE), "--batch-test", "--gpu-sample", "--slots", "4", "--requests", "4", "--dup",
             "--max-frames", "20", "--prompt-len", "10", "--seed", "9")
    assert r.returncode == 0 and "batch-test: OK" in r.stdout, r.stdout + r.stderr
    assert "MISMATCH" not in r.stdout


def test_decode_bench_harness_with_gpu_sampling(root):
    for extra in (["--gpu-sample"], ["--gpu-sample", "--sampled"], ["--sampled"]):
        r = _cli("--model", str(root / FIXTURE), "--decode-bench", "--slots", "4", "--steps", "16", "--prompt-len", "8", *extra)
        assert r.returncode == 0 and "decode-bench: slots=4 steps=16" in r.stdout, r.stdout + r.stderr


def test_batch_api_refuses_a_step_past_slot_capacity(root):
    """zonos2_batch_step with device sampling (zonos2_batch_sample feeding the device-resident
    tables): requests whose 250-row prompt + frames outgrow a 256-row slot (six resident steps fill
    rows 250..255) must have the step at row 256
    refused before any launch (the batch API falls back to z2h_step, which rejects the full slot)
    instead of writing past the band. The harness reports the refusal and exits with status 3."""
    r = _cli("--model", str(root / FIXTURE), "--batch-test", "--greedy", "--gpu-sample", "--slots", "3", "--requests", "3",
             "--dup", "--max-frames", "64", "--prompt-len", "250", "--slot-cap", "256")
    assert r.returncode == 3, r.stdout + r.stderr
    assert "batch-test: step refused: slot" in r.stdout and "at n_past 256 (slot capacity 256)" in r.stdout


def test_generate_matches_batch_api_loops(root):
    """zonos2_generate (src/zonos2.h:308-325) on the reference's fixture: the KV path equals a
    one-slot batch loop, the emotion-guided KV path a two-slot loop mixing uncond + scale *
    (cond - uncond), the recompute path a prefill of the growing sequence per frame; greedy and
    sampled, with out_full_ids and on_frame's early stop (tests/native/generate_kat.cpp)."""
    kat = BUILD / "generate_kat"
    assert kat.exists(), "generate_kat not built (python __graft_entry__.py)"
    r = subprocess.run([str(kat), str(root / FIXTURE)], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0 and "generate KAT: OK" in r.stdout, r.stdout + r.stderr


def test_generate_cli_reports_frames(root):
    r = _cli("--model", str(root / FIXTURE), "--generate", "--greedy", "--max-frames", "16", "--prompt-len", "10")
    assert r.returncode == 0, r.stdout + r.stderr
    assert "generate: prompt [10, " in r.stdout and "kv-cache" in r.stdout
    assert "generate: " in r.stdout and "frames, eos_frame=" in r.stdout and "  frame0:" in r.stdout
    r2 = _cli("--model", str(root / FIXTURE), "--generate", "--greedy", "--max-frames", "16", "--prompt-len", "10", "--no-kv")
    assert r2.returncode == 0 and "recompute" in r2.stdout, r2.stdout + r2.stderr
    # the first frame comes from the prompt's prefill on both paths
    f0 = [l for l in r.stdout.splitlines() if l.startswith("  frame0:")]
    f0r = [l for l in r2.stdout.splitlines() if l.startswith("  frame0:")]
    assert f0 == f0r
