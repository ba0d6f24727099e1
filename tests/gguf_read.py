"""Minimal GGUF reader for the tests (public container format: magic, version, counts, typed KV
pairs, tensor infos, aligned data). Returns the key/value map and synth.Tensor objects, so a file's
weights can be handed to the device library and to the oracle alike."""
import struct

import numpy as np

from zonos2_amd import synth

_SCALAR = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}
_BLOCK = {0: (1, 4), 1: (1, 2), 8: (32, 34), 12: (256, 144), 14: (256, 210)}


def read(path):
    b = open(path, "rb").read()
    assert b[:4] == b"GGUF"
    off = 4

    def rd(fmt):
        nonlocal off
        v = struct.unpack_from("<" + fmt, b, off)
        off += struct.calcsize("<" + fmt)
        return v[0] if len(v) == 1 else v

    def rs():
        nonlocal off
        n = rd("Q")
        s = b[off:off + n].decode()
        off += n
        return s

    def val(t):
        if t == 8:
            return rs()
        if t == 9:
            at, n = rd("I"), rd("Q")
            return [val(at) for _ in range(n)]
        return rd(_SCALAR[t])

    version, nt, nkv = rd("I"), rd("Q"), rd("Q")
    kv = {}
    for _ in range(nkv):
        k = rs()
        kv[k] = val(rd("I"))
    infos = []
    for _ in range(nt):
        name = rs()
        nd = rd("I")
        ne = tuple(rd("Q") for _ in range(nd))
        infos.append((name, ne, rd("I"), rd("Q")))
    align = kv.get("general.alignment", 32)
    data0 = (off + align - 1) // align * align
    tensors = {}
    for name, ne, ttype, toff in infos:
        blk, size = _BLOCK[ttype]
        nbytes = int(np.prod(ne)) // blk * size
        raw = np.frombuffer(b, np.uint8, nbytes, data0 + toff).copy()
        tensors[name] = synth.Tensor(name, ttype, ne, raw)
    return version, kv, tensors


def hparams(kv, tensors):
    """z2h / oracle hparams dict from the zonos2.* keys (router_dim = router_down ne1)."""
    g = lambda k: kv["zonos2." + k]
    rd = next((t.ne[1] for n, t in tensors.items() if n.endswith(".router_down.weight")), 0)
    return dict(n_layer=g("block_count"), n_embd=g("embedding_length"), head_dim=g("head_dim"),
                n_head=g("attention.head_count"), n_head_kv=g("attention.head_count_kv"),
                n_ff=g("feed_forward_length"), n_expert=g("expert_count"), n_ctx_train=g("context_length"),
                rope_freq_base=g("rope.freq_base"), rms_eps=g("attention.layer_norm_rms_epsilon"),
                qk_norm_eps=g("attention.qk_norm_epsilon"), logit_softcap=g("logit_softcap"),
                n_codebooks=g("n_codebooks"), codebook_size=g("codebook_size"), audio_vocab=g("audio_vocab"),
                eoa_id=g("eoa_id"), audio_pad_id=g("audio_pad_id"), text_vocab=g("text_vocab"),
                spk_dim=g("speaker.embedding_dim"), spk_lda_dim=g("speaker.lda_dim"), router_dim=rd,
                expert_used=list(g("expert_used_count_per_layer")))
