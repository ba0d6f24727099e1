"""Pins the oracle's mixed pass (orc_step_mixed, the checker of z2h_step_mixed) on the oracle's decode
step (orc_step, pinned stage by stage in test_oracle_step.py).

A mixed pass takes rows from several slots at once: prefill-chunk rows of a slot at consecutive
positions (each appends its K/V before the pass's attention, so a slot's rows attend to each other
causally) and decode columns. Its defining property: every row equals the decode step of that row
alone, run after the rows of its slot at lower positions (src/zonos2-graph.cpp:762-837 for one column;
the reference's KV-cache invariant that decoding row by row equals processing the prompt, graph.cpp:
515-604). Replaying the pass as one single-row orc_step per row, in position order within each slot,
must therefore give the same logits and the same K/V cache bit for bit. The batch mixes speaker rows
(emb_map entries taking an injected embedding), two chunks starting at non-zero offsets over
pre-filled cache rows, a chunk at offset 0 and decode columns.
"""
import numpy as np
import pytest

import oracle_py as O
from zonos2_amd import configs, synth


def _ids(cfg, n, rng):
    return np.concatenate([rng.integers(0, cfg.audio_vocab, (n, cfg.n_codebooks)),
                           rng.integers(0, cfg.text_vocab + 1, (n, 1))], axis=1).astype(np.int32)


@pytest.fixture(scope="module")
def c1():
    cfg, _ = configs.C1()
    return cfg, synth.generate_model(cfg, 49)


def _batch(cfg, rng):
    # (slot, first row, rows, speaker row at the chunk's first row?) then decode columns (slot, n_past)
    chunks = [(0, 0, 24, True), (1, 64, 20, False), (2, 32, 17, True)]
    decodes = [(3, 17), (4, 100)]
    pre = {1: 64, 2: 32, 3: 17, 4: 100}
    slots, npast, emap, emb = [], [], [], []
    ids = []
    for slot, r0, n, spk in chunks:
        for i in range(n):
            slots.append(slot); npast.append(r0 + i)
            if spk and i == 0:
                emap.append(len(emb)); emb.append(rng.standard_normal(cfg.n_embd).astype(np.float32))
            else:
                emap.append(-1)
        ids.append(_ids(cfg, n, rng))
    for slot, p in decodes:
        slots.append(slot); npast.append(p); emap.append(-1)
        ids.append(_ids(cfg, 1, rng))
    return (np.array(slots, np.int32), np.array(npast, np.int32), np.concatenate(ids), np.array(emap, np.int32),
            np.stack(emb), pre)


def _kv_pair(cfg, om, pre, cap):
    kvs = [O.OracleKV(om, 5, cap), O.OracleKV(om, 5, cap)]
    for s, n in pre.items():
        for L in range(cfg.n_layer):
            k, v = synth.kv_rows(cfg, L, s, n, 80 + s)
            for kv in kvs:
                kv.write(L, s, 0, k, v)
    return kvs


def test_mixed_pass_equals_single_row_steps(c1):
    cfg, model = c1
    rng = np.random.default_rng(7)
    slots, npast, ids, emap, emb, pre = _batch(cfg, rng)
    om = O.OracleModel(cfg.hparams(), model)
    cap = 131
    kv_mixed, kv_seq = _kv_pair(cfg, om, pre, cap)
    # rows in a shuffled order: the pass's result may not depend on where a row sits in the batch
    order = rng.permutation(len(slots))
    got = O.step_mixed(om, kv_mixed, slots[order], npast[order], ids[order], emb_map=emap[order], emb=emb)
    got = got[np.argsort(order)]
    # replay: one single-row decode step per row, lower positions of a slot first
    want = np.empty_like(got)
    for r in np.lexsort((slots, npast)):
        if emap[r] >= 0:
            want[r] = O.step(om, kv_seq, slots[r:r + 1], npast[r:r + 1], emb=emb[emap[r]][None, :])[0]
        else:
            want[r] = O.step(om, kv_seq, slots[r:r + 1], npast[r:r + 1], ids=ids[r:r + 1])[0]
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    for s in range(5):
        for L in range(cfg.n_layer):
            a, b = kv_mixed.read(L, s, 0, cap), kv_seq.read(L, s, 0, cap)
            np.testing.assert_array_equal(a[0], b[0])
            np.testing.assert_array_equal(a[1], b[1])


def test_mixed_pass_rows_attend_within_their_slot(c1):
    """A planted mistake must fail the replay: attending only to the pre-filled rows (dropping the
    pass's own earlier rows of the slot) is what a mixed pass without the K/V pre-append computes,
    and it differs from the single-row replay."""
    cfg, model = c1
    rng = np.random.default_rng(8)
    slots, npast, ids, emap, emb, pre = _batch(cfg, rng)
    om = O.OracleModel(cfg.hparams(), model)
    kv_a, kv_b = _kv_pair(cfg, om, pre, 131)
    mixed = O.step_mixed(om, kv_a, slots, npast, ids, emb_map=emap, emb=emb)
    # each chunk row as an independent column whose band holds only the pre-filled rows (+ itself)
    r = int(np.flatnonzero((slots == 1) & (npast == 70))[0])
    alone = O.step(om, kv_b, slots[r:r + 1], npast[r:r + 1], ids=ids[r:r + 1])[0]
    assert not np.array_equal(mixed[r], alone)
