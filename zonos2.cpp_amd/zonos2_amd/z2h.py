"""ctypes binding of include/z2h.h (libzonos2_hip.so). Loading fails loudly when the library is not
built; there is no fallback path."""
from __future__ import annotations

import ctypes as C
from functools import lru_cache

import numpy as np

from .lib import _load

OK, EINVAL, ENOMEM, EDEVICE, ESTATE, ENOTSUP = range(6)
CAP = {n: i for i, n in enumerate(
    ("res_in", "attn_in", "q", "k", "v", "gate", "attn_o", "attn_out", "ffn_in", "router_state", "router_logits",
     "probs", "sel", "weights", "ffn_out", "out_norm", "counts", "offsets", "perm", "expert_out"))}
INT_CAPS = {"sel", "counts", "offsets", "perm"}


class Hparams(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("n_layer", "n_embd", "head_dim", "n_head", "n_head_kv", "n_ff",
                                          "n_expert", "n_ctx_train")] + \
               [(n, C.c_float) for n in ("rope_freq_base", "rms_eps", "qk_norm_eps", "logit_softcap")] + \
               [(n, C.c_int32) for n in ("n_codebooks", "codebook_size", "audio_vocab", "eoa_id",
                                          "audio_pad_id", "text_vocab", "spk_dim", "spk_lda_dim",
                                          "router_dim")] + \
               [("expert_used", C.POINTER(C.c_int32))]


@lru_cache(None)
def lib() -> C.CDLL:
    L = _load("libzonos2_hip.so")
    vp, i32, i64 = C.c_void_p, C.c_int, C.c_int64
    sig = {
        "z2h_model_create": (i32, [C.POINTER(Hparams), i32, C.POINTER(vp)]),
        "z2h_model_upload_tensor": (i32, [vp, C.c_char_p, i32, C.POINTER(C.c_int64), vp, C.c_size_t]),
        "z2h_model_finalize": (i32, [vp]),
        "z2h_model_set_expert_mask": (i32, [vp, i32, vp]),
        "z2h_model_set_logit_bias": (i32, [vp, i32, vp]),
        "z2h_model_set_layer_skip": (i32, [vp, vp]),
        "z2h_set_layer_skip": (i32, [vp, vp]),
        "z2h_model_last_error": (C.c_char_p, [vp]),
        "z2h_model_release": (None, [vp]),
        "z2h_create_batch": (i32, [vp, i32, i32, C.POINTER(vp)]),
        "z2h_create_batch_rows": (i32, [vp, i32, i32, i32, C.POINTER(vp)]),
        "z2h_step_mixed": (i32, [vp, i32, vp, vp, vp, vp, vp, i32, i32, vp, vp]),
        "z2h_create": (i32, [C.POINTER(Hparams), i32, i32, i32, C.POINTER(vp)]),
        "z2h_upload_tensor": (i32, [vp, C.c_char_p, i32, C.POINTER(C.c_int64), vp, C.c_size_t]),
        "z2h_finalize": (i32, [vp]),
        "z2h_slot_cap": (i32, [vp]),
        "z2h_kv_write": (i32, [vp, i32, i32, i32, i32, vp, vp]),
        "z2h_kv_read": (i32, [vp, i32, i32, i32, i32, vp, vp]),
        "z2h_step": (i32, [vp, i32, vp, vp, vp, vp, vp]),
        "z2h_step_device": (i32, [vp, i32, vp, vp, vp, vp, vp, vp, vp]),
        "z2h_prefill": (i32, [vp, i32, vp, i32, vp, i32, vp, vp]),
        "z2h_speaker_embed": (i32, [vp, i32, vp, vp, vp]),
        "z2h_moe_forward": (i32, [vp, i32, i32, vp, vp, vp]),
        "z2h_moe_forward_device": (i32, [vp, i32, i32, vp, vp, vp, vp]),
        "z2h_model_moe_forward_noalloc": (i32, [vp, i32, i32, vp, vp, vp, vp, vp]),
        "z2h_set_expert_mask": (i32, [vp, i32, vp]),
        "z2h_set_logit_bias": (i32, [vp, i32, vp]),
        "z2h_set_capture": (i32, [vp, i32]),
        "z2h_capture_bytes": (i64, [vp, i32, i32]),
        "z2h_read_capture": (i32, [vp, i32, i32, vp, C.c_size_t]),
        "z2h_device_bytes": (i64, [vp, i32]),
        "z2h_set_graphs": (i32, [vp, i32]),
        "z2h_profile_begin": (i32, [vp]),
        "z2h_profile_end": (i32, [vp, vp, vp]),
        "z2h_sample": (i32, [vp, i32, vp, vp, vp, vp, i32, vp, vp]),
        "z2h_set_prefill_chunk": (i32, [vp, i32]),
        "z2h_sample_feed": (i32, [vp, i32, vp, vp, vp, i32, vp, vp]),
        "z2h_step_resident": (i32, [vp, i32]),
        "z2h_last_error": (C.c_char_p, [vp]),
        "z2h_destroy": (None, [vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype, fn.argtypes = res, args
    return L


EXPORTS = ("z2h_model_create", "z2h_model_upload_tensor", "z2h_model_finalize", "z2h_model_set_expert_mask",
           "z2h_model_set_logit_bias", "z2h_model_set_layer_skip", "z2h_set_layer_skip", "z2h_model_last_error", "z2h_model_release", "z2h_create_batch",
           "z2h_create", "z2h_upload_tensor", "z2h_finalize", "z2h_slot_cap", "z2h_kv_write", "z2h_kv_read",
           "z2h_step", "z2h_step_device", "z2h_prefill", "z2h_moe_forward", "z2h_moe_forward_device",
           "z2h_model_moe_forward_noalloc", "z2h_speaker_embed",
           "z2h_set_expert_mask", "z2h_set_logit_bias", "z2h_set_capture", "z2h_capture_bytes",
           "z2h_read_capture", "z2h_device_bytes", "z2h_set_graphs", "z2h_profile_begin", "z2h_profile_end", "z2h_sample", "z2h_set_prefill_chunk",
           "z2h_sample_feed", "z2h_step_resident", "z2h_create_batch_rows", "z2h_step_mixed",
           "z2h_last_error", "z2h_destroy")
KERNEL_FAMILIES = ("resnorm", "gemv_qkv", "qkv_post", "attn", "attn_combine", "gemv_wo", "router_down", "router_tail",
                   "gemv_gateup", "gemv_down", "gemv_dense", "gemv_head", "swiglu")


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class Sampling(C.Structure):
    """z2h_sampling (include/z2h.h)."""
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int32), ("top_p", C.c_float), ("min_p", C.c_float),
                ("rep_penalty", C.c_float), ("rep_codebooks", C.c_int32), ("greedy", C.c_int32), ("reserved", C.c_int32)]


class Z2HError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"z2h error {code}: {msg}")
        self.code = code


def _hparams(hp: dict):
    eu = (C.c_int32 * hp["n_layer"])(*hp["expert_used"])
    h = Hparams(**{k: v for k, v in hp.items() if k != "expert_used"})
    h.expert_used = C.cast(eu, C.POINTER(C.c_int32))
    return h, eu


class Model:
    """Device weights shared by any number of contexts (mirrors zonos2_model)."""

    def __init__(self, hp: dict, tensors: dict | None = None, device: int = 0):
        self.hp = dict(hp)
        h, _eu = _hparams(hp)
        out = C.c_void_p()
        rc = lib().z2h_model_create(C.byref(h), device, C.byref(out))
        if rc != OK:
            raise Z2HError(rc, "z2h_model_create failed")
        self.m = out
        if tensors is not None:
            self.upload(tensors)

    def check(self, rc):
        if rc != OK:
            raise Z2HError(rc, lib().z2h_model_last_error(self.m).decode())

    def upload(self, tensors: dict):
        for t in tensors.values():
            ne = (C.c_int64 * 4)(*t.ne4)
            self.check(lib().z2h_model_upload_tensor(self.m, t.name.encode(), t.type, ne, _p(t.data), t.data.nbytes))
        self.check(lib().z2h_model_finalize(self.m))

    def set_expert_mask(self, layer, keep):
        k = None if keep is None else np.ascontiguousarray(keep, dtype=np.uint8)
        self.check(lib().z2h_model_set_expert_mask(self.m, layer, _p(k)))

    def moe_forward_noalloc(self, layer, n_tokens, d_x, d_state_in, d_state_out, d_out, stream=None):
        """z2h_model_moe_forward_noalloc on device pointers (ints), enqueued on `stream`."""
        self.check(lib().z2h_model_moe_forward_noalloc(self.m, layer, n_tokens, d_x, d_state_in or None,
                                                       d_state_out or None, d_out, stream))

    def close(self):
        if getattr(self, "m", None):
            lib().z2h_model_release(self.m)
            self.m = None

    def __del__(self):
        self.close()


class Context:
    """One decode-step context on a device (mirrors zonos2_batch_ctx). Built either from hparams (a
    private model, weights uploaded through upload()) or over a shared Model."""

    def __init__(self, hp: dict | None, n_slots: int, slot_cap: int, device: int = 0, model: Model | None = None,
                 max_rows: int = 0):
        out = C.c_void_p()
        if model is not None:
            self.hp = dict(model.hp)
            rc = lib().z2h_create_batch_rows(model.m, n_slots, slot_cap, max_rows, C.byref(out))
            if rc != OK:
                raise Z2HError(rc, lib().z2h_model_last_error(model.m).decode())
        else:
            self.hp = dict(hp)
            h, _eu = _hparams(hp)
            rc = lib().z2h_create(C.byref(h), n_slots, slot_cap, device, C.byref(out))
            if rc != OK:
                raise Z2HError(rc, "z2h_create failed")
        hp = self.hp
        self.ctx = out
        self.n_slots = n_slots
        self.S = lib().z2h_slot_cap(self.ctx)
        self.kmax = max([k for k in hp["expert_used"]] + [1])

    def check(self, rc):
        if rc != OK:
            raise Z2HError(rc, lib().z2h_last_error(self.ctx).decode())

    def upload(self, tensors: dict):
        for t in tensors.values():
            ne = (C.c_int64 * 4)(*t.ne4)
            self.check(lib().z2h_upload_tensor(self.ctx, t.name.encode(), t.type, ne, _p(t.data), t.data.nbytes))
        self.check(lib().z2h_finalize(self.ctx))

    def kv_write(self, layer, slot, row0, k, v):
        k = np.ascontiguousarray(k, np.uint16)
        v = np.ascontiguousarray(v, np.uint16)
        self.check(lib().z2h_kv_write(self.ctx, layer, slot, row0, k.shape[0], _p(k), _p(v)))

    def kv_read(self, layer, slot, row0, n):
        k = np.empty((n, self.hp["n_head_kv"], self.hp["head_dim"]), np.uint16)
        v = np.empty_like(k)
        self.check(lib().z2h_kv_read(self.ctx, layer, slot, row0, n, _p(k), _p(v)))
        return k, v

    def step(self, slot_idx, n_past, ids=None, emb=None):
        si = np.ascontiguousarray(slot_idx, np.int32)
        npast = np.ascontiguousarray(n_past, np.int32)
        ids = None if ids is None else np.ascontiguousarray(ids, np.int32)
        emb = None if emb is None else np.ascontiguousarray(emb, np.float32)
        T = len(si)
        out = np.empty((T, self.hp["n_codebooks"] * self.hp["audio_vocab"]), np.float32)
        self.check(lib().z2h_step(self.ctx, T, _p(si), _p(npast), _p(ids), _p(emb), _p(out)))
        return out

    def prefill(self, slot, ids, spk=None, spk_pos=-1, delta=None):
        ids = np.ascontiguousarray(ids, np.int32)
        spk = None if spk is None else np.ascontiguousarray(spk, np.float32)
        delta = None if delta is None else np.ascontiguousarray(delta, np.float32)
        out = np.empty(self.hp["n_codebooks"] * self.hp["audio_vocab"], np.float32)
        self.check(lib().z2h_prefill(self.ctx, slot, _p(ids), ids.shape[0], _p(spk), spk_pos, _p(delta), _p(out)))
        return out

    def sample_feed(self, sp, u, hist=None, hist_len=None):
        """z2h_sample_feed: sample the last step's columns and leave their next inputs on the device."""
        n = len(sp)
        arr = (Sampling * n)(*[Sampling(**d) for d in sp])
        u = np.ascontiguousarray(u, np.float64)
        codes = np.empty((n, self.hp["n_codebooks"]), np.int32)
        cap = 0
        if hist is not None:
            hist = np.ascontiguousarray(hist, np.int32)
            hist_len = np.ascontiguousarray(hist_len, np.int32)
            cap = hist.shape[-1]
        self.check(lib().z2h_sample_feed(self.ctx, n, C.cast(arr, C.c_void_p), _p(hist), _p(hist_len), cap, _p(u), _p(codes)))
        return codes

    def step_resident(self, n: int):
        self.check(lib().z2h_step_resident(self.ctx, n))

    def speaker_embed(self, spk, delta=None):
        """z2h_speaker_embed: speaker rows [n][n_embd] of speaker vectors spk [n][spk_dim]."""
        spk = np.ascontiguousarray(np.atleast_2d(spk), np.float32)
        d = None if delta is None else np.ascontiguousarray(np.atleast_2d(delta), np.float32)
        out = np.empty((spk.shape[0], self.hp["n_embd"]), np.float32)
        self.check(lib().z2h_speaker_embed(self.ctx, spk.shape[0], _p(spk), _p(d), _p(out)))
        return out

    def step_mixed(self, slot_idx, n_past, ids, out_rows, emb_map=None, emb=None):
        """z2h_step_mixed: rows from any slots (prefill chunks and decode columns); returns the logits
        of out_rows [n_out][n_codebooks * audio_vocab]."""
        si = np.ascontiguousarray(slot_idx, np.int32)
        npast = np.ascontiguousarray(n_past, np.int32)
        ids = np.ascontiguousarray(ids, np.int32)
        orow = np.ascontiguousarray(out_rows, np.int32)
        em = None if emb_map is None else np.ascontiguousarray(emb_map, np.int32)
        e = None if emb is None else np.ascontiguousarray(emb, np.float32)
        out = np.empty((len(orow), self.hp["n_codebooks"] * self.hp["audio_vocab"]), np.float32)
        self.check(lib().z2h_step_mixed(self.ctx, len(si), _p(si), _p(npast), _p(ids), _p(em), _p(e),
                                        0 if e is None else e.shape[0], len(orow), _p(orow), _p(out)))
        return out

    def set_prefill_chunk(self, rows: int):
        self.check(lib().z2h_set_prefill_chunk(self.ctx, rows))

    def moe_forward(self, layer, x, state_in=None):
        x = np.ascontiguousarray(x, np.float32)
        st = None if state_in is None else np.ascontiguousarray(state_in, np.float32)
        out = np.empty_like(x)
        self.check(lib().z2h_moe_forward(self.ctx, layer, x.shape[0], _p(x), _p(st), _p(out)))
        return out

    def set_logit_bias(self, layer, bias):
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        self.check(lib().z2h_set_logit_bias(self.ctx, layer, _p(b)))

    def set_expert_mask(self, layer, keep):
        k = None if keep is None else np.ascontiguousarray(keep, np.uint8)
        self.check(lib().z2h_set_expert_mask(self.ctx, layer, _p(k)))

    def set_layer_skip(self, skip):
        k = None if skip is None else np.ascontiguousarray(skip, np.uint8)
        self.check(lib().z2h_set_layer_skip(self.ctx, _p(k)))

    def set_capture(self, on: bool):
        self.check(lib().z2h_set_capture(self.ctx, 1 if on else 0))

    def read_capture(self, layer, what: str, n_tokens: int):
        w = CAP[what]
        nb = lib().z2h_capture_bytes(self.ctx, w, n_tokens)
        out = np.empty(nb // 4, np.int32 if what in INT_CAPS else np.float32)
        self.check(lib().z2h_read_capture(self.ctx, layer, w, _p(out), nb))
        return out

    def set_graphs(self, on: bool):
        self.check(lib().z2h_set_graphs(self.ctx, 1 if on else 0))

    def profile_begin(self):
        self.check(lib().z2h_profile_begin(self.ctx))

    def profile_end(self):
        ms = np.zeros(len(KERNEL_FAMILIES), np.float64)
        n = np.zeros(len(KERNEL_FAMILIES), np.int32)
        self.check(lib().z2h_profile_end(self.ctx, _p(ms), _p(n)))
        return {k: (float(ms[i]), int(n[i])) for i, k in enumerate(KERNEL_FAMILIES)}

    def step_device(self, T, d_slot, d_npast, h_npast, d_ids, d_emb, d_logits, stream=None):
        """Device pointers (ints) as produced by torch's data_ptr(); stream is a hipStream_t handle."""
        h = np.ascontiguousarray(h_npast, np.int32)
        self.check(lib().z2h_step_device(self.ctx, T, C.c_void_p(d_slot), C.c_void_p(d_npast), _p(h),
                                         C.c_void_p(d_ids) if d_ids else None, C.c_void_p(d_emb) if d_emb else None,
                                         C.c_void_p(d_logits), C.c_void_p(stream) if stream else None))

    def moe_forward_device(self, layer, T, d_x, d_state, d_out, stream=None):
        self.check(lib().z2h_moe_forward_device(self.ctx, layer, T, C.c_void_p(d_x), C.c_void_p(d_state) if d_state else None,
                                                C.c_void_p(d_out), C.c_void_p(stream) if stream else None))

    def sample(self, sp, u, hist=None, hist_len=None, d_logits=None):
        """Device frame sampling: sp = list of dicts (one per column) with z2h_sampling fields, u
        [n][ncb] canonical draws, hist [n][ncb][cap] / hist_len [n][ncb] (or None); d_logits a device
        pointer (int) or None for the last step's logits. Returns codes [n][ncb]."""
        n = len(sp)
        arr = (Sampling * n)(*[Sampling(**d) for d in sp])
        u = np.ascontiguousarray(u, np.float64)
        ncb = self.hp["n_codebooks"]
        codes = np.empty((n, ncb), np.int32)
        cap = 0
        if hist is not None:
            hist = np.ascontiguousarray(hist, np.int32)
            hist_len = np.ascontiguousarray(hist_len, np.int32)
            cap = hist.shape[-1]
        self.check(lib().z2h_sample(self.ctx, n, C.c_void_p(d_logits) if d_logits else None, C.cast(arr, C.c_void_p),
                                    _p(hist), _p(hist_len), cap, _p(u), _p(codes)))
        return codes

    def device_bytes(self, what: int) -> int:
        return int(lib().z2h_device_bytes(self.ctx, what))

    def close(self):
        if getattr(self, "ctx", None):
            lib().z2h_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        self.close()
