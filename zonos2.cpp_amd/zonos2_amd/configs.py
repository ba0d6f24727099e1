"""Synthetic model / workload configurations of the decode-step benchmarks.

Tensor names and shapes follow the reference's GGUF layout (src/zonos2.cpp:137-183,
scripts/make-dummy-model.py:95-136); ne is ggml order (ne0 fastest). Per-tensor storage types follow
the reference's quantize policy (src/quantize.cpp:49-131, pick_qtype non-experts-only mode): 1-D
tensors F32; the high-precision set (output head, text/audio embeddings, speaker projections) one
tier above the bulk type (F16 over Q8_0, Q8_0 over K-quants); every other matrix the bulk type. The
routers are kept F32 because the decode step's router is specified as fp32.

Init: matrices N(0, 0.02); norm weights 1; attn_temp |N(0,1)| (the checkpoint stores |temp|,
models/convert-zonos2-to-gguf.py:207); other 1-D biases N(0, 0.02). router_bias is N(0, router_bias_std)
with std 0 by default. The 24-layer configurations use a wider router MLP init (see zonos2_24l) and
a load-balancing pre-softmax logit bias calibrated on the device (synth.router_biases), so routing
spreads over the experts as a trained router's does; the 64-request configuration adds Zipf(1.2)
log-popularity on top.
"""
from __future__ import annotations

from dataclasses import dataclass, field

F32, F16, Q8_0, Q4_K, Q6_K = 0, 1, 8, 12, 14
TYPE_NAMES = {F32: "F32", F16: "F16", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K"}
BLOCK = {F32: (1, 4), F16: (1, 2), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}


def row_bytes(t: int, n: int) -> int:
    be, bb = BLOCK[t]
    assert n % be == 0, (t, n)
    return n // be * bb


@dataclass
class ModelConfig:
    name: str
    n_layer: int
    n_embd: int
    n_head: int
    n_head_kv: int
    head_dim: int
    n_expert: int
    top_k: int
    n_ff: int
    bulk: int
    router_dim: int = 128
    n_codebooks: int = 9
    audio_vocab: int = 1025
    text_vocab: int = 519
    spk_dim: int = 64
    spk_lda_dim: int = 32
    n_ctx_train: int = 4096
    rope_freq_base: float = 10000.0
    rms_eps: float = 1e-5
    qk_norm_eps: float = 1e-6
    logit_softcap: float = 15.0
    expert_used: list[int] | None = None     # per layer; default all MoE with top_k
    router_bias_std: float = 0.0
    router_mlp_std: float = 0.02               # router MLP matrices mlp0 / mlp2 N(0, std)
    router_out_std: float = 0.02               # router output matrix mlp4 N(0, std)
    layer_experts: dict | None = None          # pruned layers: {layer: expert count} (ne[2] of the stacks)

    def __post_init__(self):
        if self.expert_used is None:
            self.expert_used = [self.top_k] * self.n_layer

    def n_exp(self, layer: int) -> int:
        """Experts of an MoE layer: the stacks' ne[2], fewer than n_expert in a pruned layer."""
        return (self.layer_experts or {}).get(layer, self.n_expert)

    @property
    def codebook_size(self) -> int:
        return self.audio_vocab - 2

    def hparams(self) -> dict:
        return dict(
            n_layer=self.n_layer, n_embd=self.n_embd, head_dim=self.head_dim, n_head=self.n_head,
            n_head_kv=self.n_head_kv, n_ff=self.n_ff, n_expert=self.n_expert,
            n_ctx_train=self.n_ctx_train, rope_freq_base=self.rope_freq_base, rms_eps=self.rms_eps,
            qk_norm_eps=self.qk_norm_eps, logit_softcap=self.logit_softcap,
            n_codebooks=self.n_codebooks, codebook_size=self.codebook_size,
            audio_vocab=self.audio_vocab, eoa_id=self.codebook_size, audio_pad_id=self.codebook_size + 1,
            text_vocab=self.text_vocab, spk_dim=self.spk_dim, spk_lda_dim=self.spk_lda_dim,
            router_dim=self.router_dim if any(self.expert_used) else 0,
            expert_used=list(self.expert_used))

    def high_tier(self) -> int:
        if self.bulk in (Q8_0, F16):
            return F16
        return Q8_0

    def tensors(self) -> list[tuple[str, int, tuple[int, ...], tuple]]:
        """[(name, type, ne, init)] with init = (kind, a, b): 0 normal(a,b), 1 b*|N(0,1)|, 2 const a."""
        d, hd, nh, nkv, ff, rd = self.n_embd, self.head_dim, self.n_head, self.n_head_kv, self.n_ff, self.router_dim
        W, hi = (0, 0.0, 0.02), self.high_tier()
        RW = (0, 0.0, self.router_mlp_std)
        out: list = []
        for i in range(self.n_codebooks):
            out.append((f"audio_embd.{i}.weight", hi, (d, self.audio_vocab), W))
        out.append(("text_embd.weight", hi, (d, self.text_vocab + 1), W))
        out.append(("spk_lda.weight", hi, (self.spk_dim, self.spk_lda_dim), W))
        out.append(("spk_lda.bias", F32, (self.spk_lda_dim,), W))
        out.append(("spk_proj.weight", hi, (self.spk_lda_dim, d), W))
        out.append(("spk_proj.bias", F32, (d,), W))
        out.append(("output_norm.weight", F32, (d,), (2, 1.0, 0.0)))
        out.append(("output.weight", hi, (d, self.n_codebooks * self.audio_vocab), W))
        seen_moe = False
        for L in range(self.n_layer):
            b = f"blk.{L}."
            bt = self.bulk
            out += [
                (b + "attn_norm.weight", F32, (d,), (2, 1.0, 0.0)),
                (b + "ffn_norm.weight", F32, (d,), (2, 1.0, 0.0)),
                (b + "attn_q.weight", bt, (d, nh * hd), W),
                (b + "attn_k.weight", bt, (d, nkv * hd), W),
                (b + "attn_v.weight", bt, (d, nkv * hd), W),
                (b + "attn_output.weight", bt, (nh * hd, d), W),
                (b + "attn_temp", F32, (nh,), (1, 0.0, 1.0)),
                (b + "attn_gate.weight", bt, (d, nh), W),
            ]
            if self.expert_used[L] == 0:
                out += [
                    (b + "ffn_up.weight", bt, (d, ff), W),
                    (b + "ffn_gate.weight", bt, (d, ff), W),
                    (b + "ffn_down.weight", bt, (ff, d), W),
                ]
                continue
            E = self.n_exp(L)
            out += [
                (b + "ffn_gate_exps.weight", bt, (d, ff, E), W),
                (b + "ffn_up_exps.weight", bt, (d, ff, E), W),
                (b + "ffn_down_exps.weight", bt, (ff, d, E), W),
                (b + "router_down.weight", F32, (d, rd), W),
                (b + "router_down.bias", F32, (rd,), W),
                (b + "router_mlp0.weight", F32, (rd, rd), RW),
                (b + "router_mlp0.bias", F32, (rd,), W),
                (b + "router_mlp2.weight", F32, (rd, rd), RW),
                (b + "router_mlp2.bias", F32, (rd,), W),
                (b + "router_mlp4.weight", F32, (rd, E), (0, 0.0, self.router_out_std)),
                (b + "router_norm.weight", F32, (rd,), (2, 1.0, 0.0)),
                (b + "router_bias", F32, (E,), (0, 0.0, self.router_bias_std) if self.router_bias_std > 0 else (2, 0.0, 0.0)),
            ]
            if seen_moe:
                out.append((b + "router_eda_scale", F32, (rd,), W))
            seen_moe = True
        return out


@dataclass
class Workload:
    name: str
    n_slots: int
    kv_lens: list[int]                  # n_past per active request (rows already in the cache)
    slot_cap: int                       # frames per slot (rounded up to 256 by the runtime)
    inject_embeddings: bool = False     # feed N(0,1) embeddings instead of token ids
    zipf: float | None = None           # pre-softmax Zipf(s) expert-popularity bias
    seed: int = 1234
    extra: dict = field(default_factory=dict)


def C1() -> tuple[ModelConfig, Workload]:
    m = ModelConfig("tiny-moe-q8_0", n_layer=2, n_embd=256, n_head=8, n_head_kv=2, head_dim=32,
                    n_expert=8, top_k=2, n_ff=512, bulk=Q8_0, router_bias_std=1e-4)
    w = Workload("c1-4req", n_slots=4, kv_lens=[3, 17, 64, 130], slot_cap=131, inject_embeddings=True)
    return m, w


def C2() -> tuple[ModelConfig, Workload]:
    m = ModelConfig("moe-layer-q4_k", n_layer=1, n_embd=2048, n_head=16, n_head_kv=4, head_dim=128,
                    n_expert=32, top_k=4, n_ff=1536, bulk=Q4_K, spk_dim=2048, spk_lda_dim=1024)
    w = Workload("c2-16tok", n_slots=16, kv_lens=[0] * 16, slot_cap=256, inject_embeddings=True)
    return m, w


def zonos2_24l(bulk: int) -> ModelConfig:
    # router MLP: hidden matrices N(0, 1/sqrt(router_dim)) keep unit-variance pre-activations through
    # the erf-GELU layers, and the output matrix N(0, 0.3) gives per-token logit spreads of about 1,
    # as in a trained router (with N(0, 0.02) throughout they vary by ~1e-3 between tokens)
    return ModelConfig(f"zonos2-24l-{TYPE_NAMES[bulk].lower()}", n_layer=24, n_embd=2048, n_head=16,
                       n_head_kv=4, head_dim=128, n_expert=32, top_k=4, n_ff=1536, bulk=bulk,
                       spk_dim=2048, spk_lda_dim=1024, router_mlp_std=128 ** -0.5, router_out_std=0.3)


def _rng(seed):
    import numpy as np
    return np.random.default_rng(seed)


def C3() -> tuple[ModelConfig, Workload]:
    rng = _rng(3)
    lens = [int(x) for x in rng.integers(32, 2049, size=16)]
    return zonos2_24l(Q4_K), Workload("c3-16req-ragged", n_slots=16, kv_lens=lens, slot_cap=2049,
                                      extra={"balance": True})


def C4(bulk: int) -> tuple[ModelConfig, Workload]:
    import numpy as np
    rng = _rng(4)
    lens = [int(x) for x in np.exp(rng.uniform(np.log(16), np.log(4096), size=64))]
    return zonos2_24l(bulk), Workload("c4-64req-zipf", n_slots=64, kv_lens=lens, slot_cap=4097, zipf=1.2,
                                      extra={"balance": True})


def shipped(bulk: int = Q4_K) -> tuple[ModelConfig, Workload]:
    """The released model's topology (docs/INTERNALS.md:252-259): 28 layers, dense SwiGLU FFN on layers
    0, 1, 2 and 27, MoE on 3-26 with 16 experts top-1 (top-2 on layer 26), router_dim 128, 9 x 1026
    logits (eoa 1024, pad 1025). Layers 9 and 20 are pruned to 12 and 14 experts, the per-layer counts
    a pruned GGUF carries in the stacks' ne[2] (src/zonos2-graph.cpp:194-197). The FFN hidden size
    1536 stands in for the checkpoint's. Workload: C3's 16 ragged requests."""
    eu = [0, 0, 0] + [1] * 23 + [2] + [0]
    m = ModelConfig(f"zonos2-shipped-{TYPE_NAMES[bulk].lower()}", n_layer=28, n_embd=2048, n_head=16, n_head_kv=4,
                    head_dim=128, n_expert=16, top_k=1, n_ff=1536, bulk=bulk, audio_vocab=1026, spk_dim=2048,
                    spk_lda_dim=1024, router_mlp_std=128 ** -0.5, router_out_std=0.3, expert_used=eu,
                    layer_experts={9: 12, 20: 14})
    _, w3 = C3()
    return m, Workload("shipped-16req-ragged", n_slots=16, kv_lens=w3.kv_lens, slot_cap=2049, extra={"balance": True})


def zipf_bias(n_expert: int, s: float, layer: int, seed: int = 99):
    """Additive log-popularity bias log(p_e) for p_e ~ 1/rank^s, rank permuted per layer."""
    import numpy as np
    rng = np.random.default_rng(seed + layer)
    ranks = rng.permutation(n_expert) + 1
    p = 1.0 / ranks.astype(np.float64) ** s
    p /= p.sum()
    return np.log(p).astype(np.float32)


@dataclass
class MixedLayout:
    """Rows of one mixed pass: prefill chunks of several prompts (each after a speaker row) and decode
    columns, in pass order."""
    slots: "np.ndarray"      # int32 [R] slot of each row
    npast: "np.ndarray"      # int32 [R] position (row of the slot's band) of each row
    emap: "np.ndarray"       # int32 [R] -1: the row sums its ids; e >= 0: the row takes speaker row e
    ids: "np.ndarray"        # int32 [R][n_codebooks + 1]
    spk: "np.ndarray"        # float32 [n_pre][spk_dim] speaker vectors (through spk_lda -> spk_proj)
    r0: list                 # chunk start inside each prompt (256-aligned; earlier rows pre-filled)
    dlen: list               # KV length of each decode column
    out_rows: "np.ndarray"   # int32 rows whose logits are read: each chunk's last row, every decode row
    cap: int                 # slot capacity the layout needs


def mixed_layout(cfg: ModelConfig, seed: int = 55, n_pre: int = 8, n_dec: int = 32, chunk: int = 256) -> MixedLayout:
    """The mixed chunked-prefill + decode batch of the C5 workload: n_pre chunks of `chunk` prompt rows,
    each after a speaker row, at a 256-aligned offset inside a prompt of U[300, 1200] rows, plus n_dec
    decode columns with KV lengths U[32, 1200]. With the defaults: 8 x (256 + 1) + 32 = 2088 rows."""
    import numpy as np
    rng = np.random.default_rng(seed)
    plen = rng.integers(300, 1201, n_pre)
    r0 = [int(rng.integers(0, (int(p) - chunk) // 256 + 1)) * 256 for p in plen]
    dlen = [int(x) for x in rng.integers(32, 1201, n_dec)]
    cap = max(max(r + chunk + 1 for r in r0), max(dlen) + 1)
    slots, npast, emap, last = [], [], [], []
    for i, r in enumerate(r0):
        for j in range(chunk + 1):                 # the speaker row, then the chunk's prompt rows
            slots.append(i); npast.append(r + j); emap.append(i if j == 0 else -1)
        last.append(len(slots) - 1)
    for i, n in enumerate(dlen):
        slots.append(n_pre + i); npast.append(n); emap.append(-1); last.append(len(slots) - 1)
    R = len(slots)
    ids = np.concatenate([rng.integers(0, cfg.audio_vocab, (R, cfg.n_codebooks)),
                          rng.integers(0, cfg.text_vocab + 1, (R, 1))], axis=1).astype(np.int32)
    spk = rng.standard_normal((n_pre, cfg.spk_dim)).astype(np.float32)
    return MixedLayout(np.array(slots, np.int32), np.array(npast, np.int32), np.array(emap, np.int32), ids, spk,
                       r0, dlen, np.array(last, np.int32), cap)
