"""ctypes binding of the CPU oracle (TEST INFRASTRUCTURE ONLY: tests/, smoke() and bench.py's
cpu_baseline leg). The product never imports this module."""
from __future__ import annotations

import ctypes as C
from functools import lru_cache
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
F32P = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")


class Hparams(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("n_layer", "n_embd", "head_dim", "n_head", "n_head_kv", "n_ff",
                                          "n_expert", "n_ctx_train")] + \
               [(n, C.c_float) for n in ("rope_freq_base", "rms_eps", "qk_norm_eps", "logit_softcap")] + \
               [(n, C.c_int32) for n in ("n_codebooks", "codebook_size", "audio_vocab", "eoa_id",
                                          "audio_pad_id", "text_vocab", "spk_dim", "spk_lda_dim",
                                          "router_dim")] + \
               [("expert_used", C.POINTER(C.c_int32))]


class Capture(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("res_in", "attn_in", "q", "k", "v", "gate", "attn_o", "attn_out",
                                          "ffn_in", "router_state", "router_logits", "probs", "sel", "weights",
                                          "ffn_out", "out_norm")]


@lru_cache(None)
def lib() -> C.CDLL:
    p = HERE / "build" / "liboracle.so"
    if not p.exists():
        raise RuntimeError(f"{p} not built (make -C oracle)")
    L = C.CDLL(str(p))
    vp, i32, i64, f32 = C.c_void_p, C.c_int, C.c_int64, C.c_float
    sig = {
        "orc_set_threads": (i32, [i32]),
        "orc_model_create": (vp, [C.POINTER(Hparams)]),
        "orc_model_set": (i32, [vp, C.c_char_p, i32, C.POINTER(C.c_int64), vp]),
        "orc_model_finalize": (i32, [vp]),
        "orc_model_set_logit_bias": (i32, [vp, i32, vp]),
        "orc_model_set_expert_mask": (i32, [vp, i32, vp]),
        "orc_model_set_layer_skip": (i32, [vp, vp]),
        "orc_model_free": (None, [vp]),
        "orc_last_error": (C.c_char_p, []),
        "orc_kv_create": (vp, [vp, i32, i32]),
        "orc_kv_slot_cap": (i32, [vp]),
        "orc_kv_write": (i32, [vp, i32, i32, i32, i32, vp, vp]),
        "orc_kv_read": (i32, [vp, i32, i32, i32, i32, vp, vp]),
        "orc_kv_free": (None, [vp]),
        "orc_step": (i32, [vp, vp, i32, vp, vp, vp, vp, vp, vp]),
        "orc_prefill": (i32, [vp, vp, i32, vp, i32, vp, i32, vp, vp]),
        "orc_router": (i32, [vp, i32, i32, vp, vp, vp, vp, vp, vp, vp]),
        "orc_group": (i32, [i32, i32, i32, vp, vp, vp, vp]),
        "orc_experts": (i32, [vp, i32, i32, vp, vp, vp, vp, vp]),
        "orc_dense_ffn": (i32, [vp, i32, i32, vp, vp]),
        "orc_attention": (i32, [vp, vp, i32, i32, vp, vp, vp, vp, vp]),
        "orc_dequant": (i32, [i32, vp, vp, i64]),
        "orc_matmul": (i32, [i32, vp, i64, i64, i32, vp, vp]),
        "orc_quant_act": (i32, [i32, vp, i64, vp, vp, vp, vp]),
        "orc_expf": (f32, [f32]), "orc_erff": (f32, [f32]), "orc_gelu_erf": (f32, [f32]),
        "orc_silu": (f32, [f32]),
        "orc_sincos": (None, [f32, C.POINTER(f32), C.POINTER(f32)]),
        "orc_softcap": (f32, [f32, f32]),
        "orc_rope": (i32, [vp, i32, i32, i32, f32]),
        "orc_f32_to_f16": (C.c_uint16, [f32]), "orc_f16_to_f32": (f32, [C.c_uint16]),
        "orc_sample": (i32, [vp, i32, f32, i32, f32, f32, f32, i32, i32, i32, vp, i32, C.c_double, i32]),
        "orc_exp_d": (C.c_double, [C.c_double]),
        "orc_step_mixed": (i32, [vp, vp, i32, vp, vp, vp, vp, vp, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype, fn.argtypes = res, args
    return L


def ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def check(rc):
    if rc != 0:
        raise RuntimeError("oracle: " + lib().orc_last_error().decode())


def make_hparams(hp: dict):
    eu = (C.c_int32 * len(hp["expert_used"]))(*hp["expert_used"])
    h = Hparams(**{k: v for k, v in hp.items() if k != "expert_used"})
    h.expert_used = C.cast(eu, C.POINTER(C.c_int32))
    return h, eu


class OracleModel:
    """The oracle's view of a model: borrows the numpy tensor bytes (kept alive here)."""

    def __init__(self, hp: dict, tensors: dict, logit_bias: dict | None = None):
        self.hp = hp
        self._h, self._eu = make_hparams(hp)
        self.m = lib().orc_model_create(C.byref(self._h))
        if not self.m:
            check(1)
        self._keep = []
        for t in tensors.values():
            ne = (C.c_int64 * 4)(*t.ne4)
            self._keep.append(t.data)
            check(lib().orc_model_set(self.m, t.name.encode(), t.type, ne, ptr(t.data)))
        check(lib().orc_model_finalize(self.m))
        for L, b in (logit_bias or {}).items():
            b = np.ascontiguousarray(b, dtype=np.float32)
            self._keep.append(b)
            check(lib().orc_model_set_logit_bias(self.m, L, ptr(b)))
        self.kmax = max([k for k in hp["expert_used"]] + [1])

    def set_expert_mask(self, layer, keep):
        k = None if keep is None else np.ascontiguousarray(keep, dtype=np.uint8)
        check(lib().orc_model_set_expert_mask(self.m, layer, ptr(k)))

    def set_layer_skip(self, skip):
        self._skip = None if skip is None else np.ascontiguousarray(skip, dtype=np.uint8)
        check(lib().orc_model_set_layer_skip(self.m, ptr(self._skip)))

    def __del__(self):
        if getattr(self, "m", None):
            lib().orc_model_free(self.m)
            self.m = None


class OracleKV:
    def __init__(self, model: OracleModel, n_slots: int, slot_cap: int):
        self.model = model
        self.kv = lib().orc_kv_create(model.m, n_slots, slot_cap)
        if not self.kv:
            check(1)
        self.S = lib().orc_kv_slot_cap(self.kv)

    def write(self, layer, slot, row0, k, v):
        k = np.ascontiguousarray(k, dtype=np.uint16)
        v = np.ascontiguousarray(v, dtype=np.uint16)
        check(lib().orc_kv_write(self.kv, layer, slot, row0, k.shape[0], ptr(k), ptr(v)))

    def read(self, layer, slot, row0, n):
        hp = self.model.hp
        k = np.empty((n, hp["n_head_kv"], hp["head_dim"]), np.uint16)
        v = np.empty_like(k)
        check(lib().orc_kv_read(self.kv, layer, slot, row0, n, ptr(k), ptr(v)))
        return k, v

    def __del__(self):
        if getattr(self, "kv", None):
            lib().orc_kv_free(self.kv)
            self.kv = None


CAPTURE_FIELDS = ("res_in", "attn_in", "q", "k", "v", "gate", "attn_o", "attn_out", "ffn_in", "router_state",
                  "router_logits", "probs", "sel", "weights", "ffn_out", "out_norm")


def step(model: OracleModel, kv: OracleKV, slot_idx, n_past, ids=None, emb=None, capture=False):
    hp = model.hp
    T = len(slot_idx)
    si = np.ascontiguousarray(slot_idx, np.int32)
    npast = np.ascontiguousarray(n_past, np.int32)
    ids = None if ids is None else np.ascontiguousarray(ids, np.int32)
    emb = None if emb is None else np.ascontiguousarray(emb, np.float32)
    nout = hp["n_codebooks"] * hp["audio_vocab"]
    logits = np.empty((T, nout), np.float32)
    cap = None
    capd = {}
    if capture:
        L, d, nh, nkv, hd = hp["n_layer"], hp["n_embd"], hp["n_head"], hp["n_head_kv"], hp["head_dim"]
        K, E, rd = model.kmax, max(1, hp["n_expert"]), max(1, hp["router_dim"])
        shapes = dict(res_in=(L, T, d), attn_in=(L, T, d), q=(L, T, nh * hd), k=(L, T, nkv * hd),
                      v=(L, T, nkv * hd), gate=(L, T, nh), attn_o=(L, T, nh * hd), attn_out=(L, T, d),
                      ffn_in=(L, T, d), router_state=(L, T, rd), router_logits=(L, T, E), probs=(L, T, E),
                      sel=(L, T, K), weights=(L, T, K), ffn_out=(L, T, d), out_norm=(T, d))
        for n, s in shapes.items():
            capd[n] = np.zeros(s, np.int32 if n == "sel" else np.float32)
        cap = Capture(**{n: capd[n].ctypes.data for n in CAPTURE_FIELDS})
    check(lib().orc_step(model.m, kv.kv, T, ptr(si), ptr(npast), ptr(ids), ptr(emb), ptr(logits),
                         C.byref(cap) if cap is not None else None))
    return (logits, capd) if capture else logits


def router(model: OracleModel, layer, ffn_in, state_in=None):
    hp = model.hp
    x = np.ascontiguousarray(ffn_in, np.float32)
    T = x.shape[0]
    k, E, rd = hp["expert_used"][layer], hp["n_expert"], hp["router_dim"]
    st = None if state_in is None else np.ascontiguousarray(state_in, np.float32)
    rh = np.empty((T, rd), np.float32)
    lg = np.empty((T, E), np.float32)
    pr = np.empty((T, E), np.float32)
    sel = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    check(lib().orc_router(model.m, layer, T, ptr(x), ptr(st), ptr(rh), ptr(lg), ptr(pr), ptr(sel), ptr(w)))
    return dict(rh=rh, logits=lg, probs=pr, sel=sel, w=w)


def group(sel, E):
    sel = np.ascontiguousarray(sel, np.int32)
    T, k = sel.shape
    counts = np.empty(E, np.int32)
    offsets = np.empty(E + 1, np.int32)
    perm = np.empty(T * k, np.int32)
    check(lib().orc_group(T, k, E, ptr(sel), ptr(counts), ptr(offsets), ptr(perm)))
    return counts, offsets, perm


def experts(model: OracleModel, layer, ffn_in, sel, w):
    x = np.ascontiguousarray(ffn_in, np.float32)
    sel = np.ascontiguousarray(sel, np.int32)
    w = np.ascontiguousarray(w, np.float32)
    T, k = sel.shape
    d = model.hp["n_embd"]
    eo = np.empty((T * k, d), np.float32)
    out = np.empty((T, d), np.float32)
    check(lib().orc_experts(model.m, layer, T, ptr(x), ptr(sel), ptr(w), ptr(eo), ptr(out)))
    return eo, out


def matmul(wtype, wbytes, n_in, n_out, x):
    x = np.ascontiguousarray(x, np.float32)
    T = x.shape[0]
    y = np.empty((T, n_out), np.float32)
    check(lib().orc_matmul(wtype, ptr(wbytes), n_in, n_out, T, ptr(x), ptr(y)))
    return y


def dequant(wtype, wbytes, n):
    y = np.empty(n, np.float32)
    check(lib().orc_dequant(wtype, ptr(np.ascontiguousarray(wbytes)), ptr(y), n))
    return y


def prefill(model: OracleModel, kv: OracleKV, slot, ids, spk=None, spk_pos=0, delta=None):
    """Causal prefill of ids [n0][W] into `slot`; returns the last row's logits [ncb * av]."""
    hp = model.hp
    ids = np.ascontiguousarray(ids, np.int32)
    spk = None if spk is None else np.ascontiguousarray(spk, np.float32)
    delta = None if delta is None else np.ascontiguousarray(delta, np.float32)
    out = np.empty(hp["n_codebooks"] * hp["audio_vocab"], np.float32)
    check(lib().orc_prefill(model.m, kv.kv, slot, ptr(ids), ids.shape[0], ptr(spk), spk_pos, ptr(delta), ptr(out)))
    return out


def sample(logits, sp: dict, cb: int, u: float, hist=None, exp_mode: int = 1) -> int:
    """One frame code for one codebook (orc_sample); sp holds the z2h_sampling fields, hist the
    codebook's recent codes (oldest first)."""
    lg = np.ascontiguousarray(logits, np.float32)
    h = np.ascontiguousarray(hist if hist is not None else [], np.int32)
    return int(lib().orc_sample(ptr(lg), lg.size, sp["temperature"], sp["top_k"], sp["top_p"], sp["min_p"],
                                sp["rep_penalty"], sp["rep_codebooks"], sp["greedy"], cb, ptr(h) if h.size else None,
                                int(h.size), float(u), exp_mode))


def exp_d(x: float) -> float:
    return float(lib().orc_exp_d(float(x)))


def step_mixed(model: "OracleModel", kv: "OracleKV", slot_idx, n_past, ids, emb_map=None, emb=None):
    """orc_step_mixed: logits [T][ncb*av] of rows from any slots (a slot's rows causal in the pass)."""
    si = np.ascontiguousarray(slot_idx, np.int32)
    npast = np.ascontiguousarray(n_past, np.int32)
    ids = np.ascontiguousarray(ids, np.int32)
    em = None if emb_map is None else np.ascontiguousarray(emb_map, np.int32)
    e = None if emb is None else np.ascontiguousarray(emb, np.float32)
    hp = model.hp
    out = np.empty((len(si), hp["n_codebooks"] * hp["audio_vocab"]), np.float32)
    check(lib().orc_step_mixed(model.m, kv.kv, len(si), ptr(si), ptr(npast), ptr(ids), ptr(em), ptr(e), ptr(out)))
    return out
