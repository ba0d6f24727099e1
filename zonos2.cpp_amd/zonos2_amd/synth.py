"""Synthetic model weights, KV caches and step inputs (host memory, numpy).

Every value is a pure function of (seed, tensor name, element index) computed by
libzonos2_host.so (splitmix64 counter + inverse normal CDF, then the GGUF-format quantizers), so the CPU
oracle and the device see identical bytes and any config can be regenerated on any host.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

from .configs import BLOCK, F16, ModelConfig, Workload, row_bytes
from .lib import host_lib


@dataclass
class Tensor:
    name: str
    type: int
    ne: tuple
    data: np.ndarray        # uint8 bytes

    @property
    def ne4(self):
        return tuple(self.ne) + (1,) * (4 - len(self.ne))


def _threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def generate_tensor(name: str, ttype: int, ne: tuple, init: tuple, seed: int) -> Tensor:
    lib = host_lib()
    n_per_row = ne[0]
    nrows = int(np.prod(ne[1:])) if len(ne) > 1 else 1
    nb = row_bytes(ttype, n_per_row) * nrows
    buf = np.empty(nb, dtype=np.uint8)
    kind, a, b = init
    rc = lib.z2s_generate(C.c_uint64(seed), C.c_uint64(lib.z2s_stream_id(name.encode())), kind,
                          C.c_float(a), C.c_float(b), ttype, C.c_int64(nrows), C.c_int64(n_per_row),
                          buf.ctypes.data_as(C.c_void_p), _threads())
    if rc != 0:
        raise RuntimeError(f"generate failed for {name}")
    return Tensor(name, ttype, tuple(ne), buf)


def generate_model(cfg: ModelConfig, seed: int = 42) -> dict[str, Tensor]:
    return {n: generate_tensor(n, t, ne, init, seed) for n, t, ne, init in cfg.tensors()}


def gen_normal_f16(n: int, seed: int, stream: str) -> np.ndarray:
    lib = host_lib()
    out = np.empty(n, dtype=np.uint16)
    rc = lib.z2s_generate(C.c_uint64(seed), C.c_uint64(lib.z2s_stream_id(stream.encode())), 0,
                          C.c_float(0.0), C.c_float(1.0), F16, C.c_int64(1), C.c_int64(n),
                          out.ctypes.data_as(C.c_void_p), _threads())
    assert rc == 0
    return out


def gen_normal_f32(shape, seed: int, stream: str) -> np.ndarray:
    lib = host_lib()
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    rc = lib.z2s_generate(C.c_uint64(seed), C.c_uint64(lib.z2s_stream_id(stream.encode())), 0,
                          C.c_float(0.0), C.c_float(1.0), 0, C.c_int64(1), C.c_int64(n),
                          out.ctypes.data_as(C.c_void_p), _threads())
    assert rc == 0
    return out.reshape(shape)


def kv_rows(cfg: ModelConfig, layer: int, slot: int, n_rows: int, seed: int):
    """N(0,1) f16 K and V rows [n_rows][n_head_kv][head_dim] for one slot of one layer."""
    n = n_rows * cfg.n_head_kv * cfg.head_dim
    k = gen_normal_f16(n, seed, f"kv.k.{layer}.{slot}").reshape(n_rows, cfg.n_head_kv, cfg.head_dim)
    v = gen_normal_f16(n, seed, f"kv.v.{layer}.{slot}").reshape(n_rows, cfg.n_head_kv, cfg.head_dim)
    return k, v


@dataclass
class StepInputs:
    slot_idx: np.ndarray    # int32 [T]
    n_past: np.ndarray      # int32 [T]
    ids: np.ndarray         # int32 [T][W]
    emb: np.ndarray | None  # float32 [T][d]


def step_inputs(cfg: ModelConfig, wl: Workload) -> StepInputs:
    T = len(wl.kv_lens)
    rng = np.random.default_rng(wl.seed)
    W = cfg.n_codebooks + 1
    ids = np.empty((T, W), dtype=np.int32)
    ids[:, :cfg.n_codebooks] = rng.integers(0, cfg.audio_vocab, size=(T, cfg.n_codebooks))
    ids[:, cfg.n_codebooks] = rng.integers(0, cfg.text_vocab + 1, size=T)
    emb = gen_normal_f32((T, cfg.n_embd), wl.seed, "inputs.emb") if wl.inject_embeddings else None
    return StepInputs(np.arange(T, dtype=np.int32), np.array(wl.kv_lens, dtype=np.int32), ids, emb)


def router_biases(ctx, cfg: ModelConfig, wl: Workload) -> dict | None:
    """Pre-softmax router-logit biases of a workload, set on the device context and returned (so the
    oracle can be given the same ones).

    A random-init router gives every token nearly the same mean logit per expert, so a few experts
    win every selection. A trained router is load-balanced, which we emulate by subtracting each
    expert's mean logit over a calibration batch (different ids, same positions) run on the device
    without biases. Workloads with a Zipf(s) popularity add log-popularity on top. Layers without
    MoE get none. Only the 24-layer configurations ask for balancing (wl.extra["balance"])."""
    if not wl.extra.get("balance") and not wl.zipf:
        return None
    T = len(wl.kv_lens)
    moe = [L for L in range(cfg.n_layer) if cfg.expert_used[L] > 0]
    bias = {L: np.zeros(cfg.n_exp(L), np.float32) for L in moe}
    if wl.extra.get("balance"):
        inp = step_inputs(cfg, wl)
        rng = np.random.default_rng(wl.seed + 17)
        ids = inp.ids.copy()
        ids[:, :cfg.n_codebooks] = rng.integers(0, cfg.audio_vocab, size=(T, cfg.n_codebooks))
        for L in moe:
            ctx.set_logit_bias(L, None)
        ctx.set_capture(True)
        ctx.step(inp.slot_idx, inp.n_past, ids=ids)
        for L in moe:
            E = cfg.n_exp(L)                                 # the capture holds [T][E] of the layer
            lg = ctx.read_capture(L, "router_logits", T)[:T * E].reshape(T, E)
            bias[L] = (-lg.astype(np.float64).mean(0)).astype(np.float32)
        ctx.set_capture(False)
    if wl.zipf:
        from .configs import zipf_bias
        for L in moe:
            bias[L] = (bias[L] + zipf_bias(cfg.n_exp(L), wl.zipf, L)).astype(np.float32)
    for L in moe:
        ctx.set_logit_bias(L, bias[L])
    return bias
