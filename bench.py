#!/usr/bin/env python3
"""Decode-step benchmark on one MI355X.

Workload (default): the full 24-layer ZONOS2-scale MoE backbone (d_model 2048, 16/4 heads, head_dim
128, 32 experts top-4, SwiGLU 1536, 9 x 1025 logits, Q4_K weights, fp32 routers), one continuous-
batching decode step for 16 ragged requests with KV lengths uniform in [32, 2048]. Random-init
weights and N(0,1) f16 KV caches (synthetic data, no checkpoint). Inputs stay resident in HBM over the
timed region; a step is one call of z2h_step_device (all 24 layers + head, logits left on the device).

Prints one JSON line: tok/s (= active requests / step time), the roofline of the dominant kernel
(grouped expert gate/up GEMV) from HIP events recorded around its launches, the whole-step fraction
of HBM peak, and the CPU oracle timed on a bounded sample of the same step on the host cores.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "zonos2.cpp_amd", ROOT / "oracle"):
    sys.path.insert(0, str(_p))

HBM_PEAK_GBPS = 8000.0


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def profiled_traffic(config: str):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE passes (profiles/gemv_gateup_c3_traffic.md, copy-calibrated), or None."""
    p = ROOT / "profiles" / "gemv_gateup_c3_traffic.md"
    if config != "c3" or not p.exists():
        return None
    m = re.search(r"^gemv_gateup_traffic_bytes: (\d+)", p.read_text(), re.M)
    return int(m.group(1)) if m else None


def model_bytes(model, names):
    return sum(model[n].data.nbytes for n in names if n in model)


def step_bytes(cfg, model, wl, used_experts):
    """Algorithmic HBM bytes of one decode step: touched experts, attention + router + norm
    tensors, the KV band read (n_past + 1 rows) and the new rows written, head, gathered embedding
    rows and the logits."""
    T = len(wl.kv_lens)
    kvrow = cfg.n_head_kv * cfg.head_dim * 2
    B = 0
    per_expert = {}
    for L in range(cfg.n_layer):
        b = f"blk.{L}."
        ex = 0
        for nm in ("ffn_gate_exps.weight", "ffn_up_exps.weight", "ffn_down_exps.weight"):
            if b + nm in model:                      # MoE layers: only the experts the step routed to
                t = model[b + nm]
                ex += t.data.nbytes // t.ne[2] * len(used_experts[L])
        per_expert[L] = ex
        rest = [n for n in model if n.startswith(b) and "_exps" not in n]
        B += ex + model_bytes(model, rest)
        B += sum((n + 1) * kvrow * 2 for n in wl.kv_lens) + T * kvrow * 2
    B += model_bytes(model, ["output.weight", "output_norm.weight"])
    from zonos2_amd.configs import row_bytes
    for k in range(cfg.n_codebooks):
        t = model[f"audio_embd.{k}.weight"]
        B += T * row_bytes(t.type, cfg.n_embd)
    B += T * row_bytes(model["text_embd.weight"].type, cfg.n_embd)
    B += T * cfg.n_codebooks * cfg.audio_vocab * 4
    return B, per_expert


def decode_leg(np, torch, cfg, wl, steps, warmup, cpu_steps, label, keep=False):
    """One configuration's decode step: generate and upload the model, fill the KV cache, calibrate
    the routing biases, time `steps` graph-replayed z2h_step_device calls on a torch stream (inputs
    resident in HBM), time the host-buffer boundary, take per-kernel HIP-event times, and (cpu_steps >
    0) time the oracle on the host cores and compare its logits and routing with the device's."""
    from zonos2_amd import synth
    from zonos2_amd.z2h import Context, Model
    T = len(wl.kv_lens)
    t0 = time.time()
    model = synth.generate_model(cfg, seed=42)
    log(f"[{label}] generated {cfg.name}: {sum(t.data.nbytes for t in model.values()) / 1e9:.2f} GB in {time.time() - t0:.1f}s")
    t0 = time.time()
    mdl = Model(cfg.hparams(), model)              # device weights, shared with the mixed-pass context
    ctx = Context(None, wl.n_slots, wl.slot_cap, model=mdl)
    kv_cache = {}
    for L in range(cfg.n_layer):
        for s_, n in enumerate(wl.kv_lens):
            k, v = synth.kv_rows(cfg, L, s_, n, 7)
            ctx.kv_write(L, s_, 0, k, v)
            kv_cache[(L, s_)] = (k, v)
    # load-balanced routing (+ Zipf popularity for the 64-request configuration), calibrated on the device
    bias = synth.router_biases(ctx, cfg, wl)
    log(f"[{label}] uploaded + KV filled in {time.time() - t0:.1f}s; weights {ctx.device_bytes(0) / 1e9:.2f} GB, "
        f"KV {ctx.device_bytes(1) / 1e9:.2f} GB")
    inp = synth.step_inputs(cfg, wl)
    # one capture step: routing (touched experts per layer) and logits for the parity check
    ctx.set_capture(True)
    logits_gpu = ctx.step(inp.slot_idx, inp.n_past, ids=inp.ids)
    used, sel_gpu = {}, {}
    for L in range(cfg.n_layer):
        k = cfg.expert_used[L]
        if k:
            sel_gpu[L] = ctx.read_capture(L, "sel", T)[:T * k].reshape(T, k)
            used[L] = sorted(set(sel_gpu[L].ravel().tolist()))
    ctx.set_capture(False)

    dev = torch.device("cuda:0")
    d_slot = torch.from_numpy(inp.slot_idx).to(dev)
    d_npast = torch.from_numpy(inp.n_past).to(dev)
    d_ids = torch.from_numpy(inp.ids).to(dev)
    d_logits = torch.empty((T, cfg.n_codebooks * cfg.audio_vocab), dtype=torch.float32, device=dev)
    stream = torch.cuda.Stream(device=dev)
    sh = stream.cuda_stream

    def one():
        ctx.step_device(T, d_slot.data_ptr(), d_npast.data_ptr(), inp.n_past, d_ids.data_ptr(), 0,
                        d_logits.data_ptr(), stream=sh)

    for _ in range(warmup):
        one()
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    ev0.record(stream)
    for i in range(steps):
        evs[i].record(stream)
        one()
    evs[steps].record(stream)
    ev1.record(stream)
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / steps
    med_ms = float(np.median([evs[i].elapsed_time(evs[i + 1]) for i in range(steps)]))
    log(f"[{label}] step: {ms:.3f} ms mean over {steps} steps (median {med_ms:.3f} ms)")
    got = d_logits.cpu().numpy()
    assert np.array_equal(got, logits_gpu), "device-resident step differs from the host-API step"

    # the host-buffer boundary (z2h_step: slot ids, n_past and token ids uploaded, logits copied back
    # and waited for), wall clock per call; reported beside `value`, never as it
    host_ms = []
    for i in range(warmup + steps):
        t0 = time.perf_counter()
        ctx.step(inp.slot_idx, inp.n_past, ids=inp.ids)
        if i >= warmup:
            host_ms.append((time.perf_counter() - t0) * 1000.0)
    host_med = float(np.median(host_ms))
    log(f"[{label}] host-API step (PCIe both ways, synchronous): {host_med:.3f} ms median over {steps} calls")

    # per-kernel HIP-event window (separate pass over the same steps, eager launches): every launch
    # carries a start / stop event pair timestamped at the kernel's own start and end
    ctx.profile_begin()
    for _ in range(steps):
        one()
    prof = ctx.profile_end()
    for k, (t, n) in prof.items():
        if n:
            log(f"  {k:14s} {t / steps * 1000:9.1f} us/step  {n // steps:4d} launches/step  {t / n * 1000:8.2f} us/launch")

    B, _ = step_bytes(cfg, model, wl, used)
    moe = [L for L in range(cfg.n_layer) if cfg.expert_used[L]]
    # dominant kernel: grouped expert gate/up GEMV; per launch = touched experts x (gate + up bytes)
    # + the encoded activations read + the fp32 gate/up rows written
    gu_w = sum(model[f"blk.{L}.ffn_gate_exps.weight"].data.nbytes // cfg.n_exp(L) * 2 * len(used[L]) for L in moe)
    act_b = len(moe) * T * (cfg.n_embd + cfg.n_embd // 256 * 4 + cfg.n_embd // 16 * 2)
    gu_out = sum(T * cfg.expert_used[L] * cfg.n_ff * 4 for L in moe)   # one fp32 SwiGLU row per route
    gu_ms, gu_n = prof["gemv_gateup"]
    dom_gbps = (gu_w + act_b + gu_out) * steps / (gu_ms / 1000.0) / 1e9 if gu_ms > 0 else 0.0
    step_gbps = B / (ms / 1000.0) / 1e9
    out = {
        "cfg": cfg, "wl": wl, "T": T, "ms": ms, "med_ms": med_ms, "host_med": host_med, "prof": prof, "B": B,
        "step_gbps": step_gbps, "dom_gbps": dom_gbps, "gu_ms": gu_ms, "gu_n": gu_n,
        "gu_bytes": int((gu_w + act_b + gu_out) / max(1, len(moe))),
        "roofline": {"kernel": gateup_kernel_of(cfg.bulk), "bound": "hbm", "achieved": round(dom_gbps, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(dom_gbps / HBM_PEAK_GBPS, 4),
                     "avg_launch_us": round(gu_ms / max(1, gu_n) * 1000.0, 2),
                     "bytes_per_launch": int((gu_w + act_b + gu_out) / max(1, len(moe)))},
        "step_hbm": {"bytes": B, "achieved": round(step_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(step_gbps / HBM_PEAK_GBPS, 4)},
        "cpu": None, "parity": None,
    }
    if cpu_steps > 0:
        import oracle_py as O
        threads, nproc, cpu_model = cpu_share()
        O.lib().orc_set_threads(threads)
        om = O.OracleModel(cfg.hparams(), model, logit_bias=bias)
        okv = O.OracleKV(om, wl.n_slots, wl.slot_cap)
        for (L, s_), (k, v) in kv_cache.items():
            okv.write(L, s_, 0, k, v)
        t0 = time.time()
        ref, cap = O.step(om, okv, inp.slot_idx, inp.n_past, ids=inp.ids, capture=True)   # warm-up 1 (+ parity capture)
        t_first = time.time() - t0
        O.step(om, okv, inp.slot_idx, inp.n_past, ids=inp.ids)                             # warm-up 2
        times = []
        for _ in range(cpu_steps):
            t0 = time.time()
            O.step(om, okv, inp.slot_idx, inp.n_past, ids=inp.ids)
            times.append(time.time() - t0)
        t_cpu = float(np.median(times))
        a, b = got.astype(np.float64).ravel(), ref.astype(np.float64).ravel()
        cosv = float(a @ b / np.sqrt((a @ a) * (b @ b)))
        mism = sum(int(not np.array_equal(sel_gpu[L], cap["sel"][L][:, :cfg.expert_used[L]])) for L in moe)
        bit = bool(np.array_equal(got.view(np.uint32), ref.view(np.uint32)))
        log(f"[{label}] oracle: {t_cpu:.2f}s/step on {threads} threads (first {t_first:.2f}s); logits cos {cosv:.7f}, "
            f"max|d| {np.abs(a - b).max():.2e}, bit-identical {bit}; layers whose top-k ids differ end to end: {mism}/{len(moe)}")
        out["cpu"] = {"value": round(T / t_cpu, 3), "unit": "tok/s", "cores": threads, "kind": "port",
                      "sample": f"{2 + cpu_steps} full decode steps of the same workload (median of {cpu_steps} "
                                f"after 2 warm-ups), C++ restatement of the ggml CPU path",
                      "nproc": nproc, "cpu_model": cpu_model, "threads": threads}
        out["parity"] = {"logits_cos": round(cosv, 7), "logits_max_abs": float(np.abs(a - b).max()),
                         "logits_bit_identical": bit, "layers_routing_differs": mism}
        del om, okv
    if keep:
        out.update(model=model, mdl=mdl, ctx=ctx, inp=inp, d_logits=d_logits, stream=stream)
    else:
        ctx.close()
        mdl.close()
    return out


def single_stream(np, torch, steps, warmup):
    """One request on the released topology with Q8_0 weights (the model of the reference's published
    single-stream rate): 28 layers, dense 0/1/2/27, 16 experts top-1 (top-2 on layer 26), KV length
    512. The graph-replayed device-resident step, and a greedy generation loop over the host API (ids
    up, 9 x 1026 logits down, argmax on the host per frame), the shape of the reference's generate(kv)."""
    from zonos2_amd import configs, synth
    from zonos2_amd.z2h import Context, Model
    cfg, _ = configs.shipped(configs.Q8_0)
    n_past = 512
    model = synth.generate_model(cfg, seed=42)
    mdl = Model(cfg.hparams(), model)
    ctx = Context(None, 1, n_past + warmup + 2 * steps + 16, model=mdl)
    for L in range(cfg.n_layer):
        k, v = synth.kv_rows(cfg, L, 0, n_past, 7)
        ctx.kv_write(L, 0, 0, k, v)
    rng = np.random.default_rng(9)
    ids = np.concatenate([rng.integers(0, cfg.audio_vocab, (1, cfg.n_codebooks)), [[cfg.text_vocab]]], axis=1).astype(np.int32)
    dev = torch.device("cuda:0")
    d_slot = torch.zeros(1, dtype=torch.int32, device=dev)
    d_npast = torch.full((1,), n_past, dtype=torch.int32, device=dev)
    d_ids = torch.from_numpy(ids).to(dev)
    d_logits = torch.empty((1, cfg.n_codebooks * cfg.audio_vocab), dtype=torch.float32, device=dev)
    stream = torch.cuda.Stream(device=dev)
    h_np = np.array([n_past], np.int32)

    def one():
        ctx.step_device(1, d_slot.data_ptr(), d_npast.data_ptr(), h_np, d_ids.data_ptr(), 0, d_logits.data_ptr(),
                        stream=stream.cuda_stream)

    for _ in range(warmup):
        one()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        one()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    # greedy generation over the host API: each frame's step writes row n_past, its argmax codes feed the
    # next frame
    slot = np.zeros(1, np.int32)
    cur = ids.copy()
    pos = n_past
    for _ in range(warmup):
        lg = ctx.step(slot, np.array([pos], np.int32), ids=cur).reshape(cfg.n_codebooks, cfg.audio_vocab)
        cur[0, :cfg.n_codebooks] = lg.argmax(1)
        pos += 1
    t0 = time.perf_counter()
    for _ in range(steps):
        lg = ctx.step(slot, np.array([pos], np.int32), ids=cur).reshape(cfg.n_codebooks, cfg.audio_vocab)
        cur[0, :cfg.n_codebooks] = lg.argmax(1)
        pos += 1
    loop_ms = (time.perf_counter() - t0) * 1000.0 / steps
    ctx.close()
    mdl.close()
    frame_s = 512.0 / 44100.0
    log(f"single stream ({cfg.name}, KV {n_past}): step {ms:.3f} ms ({1000.0 / ms:.0f} frames/s); host-API greedy loop "
        f"{loop_ms:.3f} ms per frame ({1000.0 / loop_ms:.0f} frames/s, RTF {loop_ms / 1000.0 / frame_s:.3f})")
    return {"model": f"{cfg.name}: 28 layers, dense FFN on 0/1/2/27, 16 experts top-1 (top-2 on layer 26), 9 x 1026 logits",
            "kv_len": n_past, "requests": 1,
            "step_ms": round(ms, 4), "step_frames_per_s": round(1000.0 / ms, 1),
            "loop_ms_per_frame": round(loop_ms, 4), "loop_frames_per_s": round(1000.0 / loop_ms, 1),
            "rtf": round(loop_ms / 1000.0 / frame_s, 4),
            "note": "step: device-resident graph replay; loop: host API per frame (ids up, logits down, host argmax), "
                    "the reference's generate(kv) shape; its published rate is ~300 frames/s greedy on one H100"}


def cpu_small(np, cpu_steps):
    """The oracle on the two configurations too small for a GPU leg: C1 (one decode step of the tiny
    2-layer model, 4 ragged requests) and C2 (one MoE layer, 16 tokens: router + grouped experts).
    Median of cpu_steps after 2 warm-ups."""
    import oracle_py as O
    from zonos2_amd import configs, synth
    threads, nproc, cpu_model = cpu_share()
    O.lib().orc_set_threads(threads)
    res = {}
    cfg, wl = configs.C1()
    model = synth.generate_model(cfg, 42)
    om = O.OracleModel(cfg.hparams(), model)
    okv = O.OracleKV(om, wl.n_slots, wl.slot_cap)
    for L in range(cfg.n_layer):
        for s_, n in enumerate(wl.kv_lens):
            k, v = synth.kv_rows(cfg, L, s_, n, 7)
            okv.write(L, s_, 0, k, v)
    inp = synth.step_inputs(cfg, wl)
    ts = []
    for i in range(2 + cpu_steps):
        t0 = time.perf_counter()
        O.step(om, okv, inp.slot_idx, inp.n_past, emb=inp.emb)
        if i >= 2:
            ts.append(time.perf_counter() - t0)
    t = float(np.median(ts))
    res["c1"] = {"value": round(len(wl.kv_lens) / t, 1), "unit": "tok/s", "ms_per_step": round(t * 1000.0, 3)}
    cfg, wl = configs.C2()
    model = synth.generate_model(cfg, 42)
    om = O.OracleModel(cfg.hparams(), model)
    x = synth.gen_normal_f32((16, cfg.n_embd), 11, "inputs.c2")
    ts = []
    for i in range(2 + cpu_steps):
        t0 = time.perf_counter()
        r = O.router(om, 0, x, None)
        O.experts(om, 0, x, r["sel"], r["w"])
        if i >= 2:
            ts.append(time.perf_counter() - t0)
    t = float(np.median(ts))
    res["c2"] = {"value": round(16 / t, 1), "unit": "tok/s", "ms_per_layer": round(t * 1000.0, 3)}
    for k in res:
        res[k].update(cores=threads, kind="port", nproc=nproc, cpu_model=cpu_model,
                      sample=f"median of {cpu_steps} after 2 warm-ups, C++ restatement of the ggml CPU path")
    log(f"oracle C1 {res['c1']['ms_per_step']} ms/step, C2 {res['c2']['ms_per_layer']} ms/layer on {threads} threads")
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c3", choices=["c3", "c4-q6_k", "c4-q8_0"],
                    help="the configuration of the main line (value, roofline)")
    ap.add_argument("--legs", default="all", choices=["all", "main", "single"],
                    help="all: also the C4 Q6_K / Q8_0 legs, the single-stream leg and the C1 / C2 CPU baselines "
                         "beside the C3 line; main: the main configuration only; single: the single-stream leg "
                         "alone (its JSON on one line, for profiling)")
    ap.add_argument("--cpu-steps", type=int, default=5, help="timed oracle steps for the CPU baselines after 2 warm-ups (0: skip)")
    ap.add_argument("--no-mixed-f16", dest="mixed_f16", action="store_false",
                    help="skip the mixed pass on the F16-weight model")
    ap.add_argument("--calib-copy", action="store_true",
                    help="after the timed region, copy 256 MiB device to device once (a kernel of known traffic "
                         "for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU only (no multi-GPU path); use --gpus 1", file=sys.stderr)
        return 2

    import numpy as np
    import torch
    from zonos2_amd import configs, synth
    from zonos2_amd.z2h import Context, Model

    if args.legs == "single":
        print(json.dumps({"single_stream": single_stream(np, torch, args.steps * 5, args.warmup)}), flush=True)
        return 0
    if args.config == "c3":
        cfg, wl = configs.C3()
    elif args.config == "c4-q6_k":
        cfg, wl = configs.C4(configs.Q6_K)
    else:
        cfg, wl = configs.C4(configs.Q8_0)
    main_leg = decode_leg(np, torch, cfg, wl, args.steps, args.warmup, args.cpu_steps, args.config, keep=True)
    T, ms = main_leg["T"], main_leg["ms"]
    ctx, mdl, model, d_logits = main_leg["ctx"], main_leg["mdl"], main_leg["model"], main_leg["d_logits"]

    # the next rows of the path, outside the decode step: prefill of one 1024-row prompt in one pass
    # (a context whose row capacity holds the prompt) and device sampling of the step's columns with the
    # default settings
    rng_p = np.random.default_rng(5)
    n_pf = 1024
    pids = np.concatenate([rng_p.integers(0, cfg.audio_vocab, (n_pf, cfg.n_codebooks)),
                           rng_p.integers(0, cfg.text_vocab + 1, (n_pf, 1))], axis=1).astype(np.int32)
    pctx = Context(None, 1, n_pf, model=mdl, max_rows=n_pf)
    pctx.prefill(0, pids[:16])
    pf = []
    for _ in range(3):
        t0 = time.perf_counter()
        pctx.prefill(0, pids)
        pf.append(time.perf_counter() - t0)
    pctx.close()
    pf_ms = float(np.median(pf)) * 1000.0
    log(f"prefill: {n_pf} rows in one pass, {pf_ms:.1f} ms ({n_pf / pf_ms * 1000.0:.0f} rows/s)")
    sp_def = dict(temperature=1.15, top_k=106, top_p=0.0, min_p=0.18, rep_penalty=1.2, rep_codebooks=8, greedy=0)
    hist = rng_p.integers(0, cfg.audio_vocab, (T, cfg.n_codebooks, 50)).astype(np.int32)
    hlen = np.full((T, cfg.n_codebooks), 50, np.int32)
    uu = rng_p.random((T, cfg.n_codebooks))
    ctx.sample([sp_def] * T, uu, hist, hlen, d_logits=d_logits.data_ptr())
    t0 = time.perf_counter()
    for _ in range(20):
        ctx.sample([sp_def] * T, uu, hist, hlen, d_logits=d_logits.data_ptr())
    samp_us = (time.perf_counter() - t0) / 20 * 1e6
    log(f"device sampling: {samp_us:.1f} us per frame of {T} columns (host round trip included)")

    mixed = mixed_pass(np, Context, synth, cfg, mdl) if args.config == "c3" else None
    ctx.close()
    mdl.close()
    del model
    main_leg.pop("model"); main_leg.pop("mdl"); main_leg.pop("ctx")
    mixed_f16 = None
    if args.config == "c3" and args.mixed_f16:
        # the same mixed pass on the 24-layer model with F16 weights (about 15 GB)
        fcfg = configs.zonos2_24l(configs.F16)
        t0 = time.time()
        fmodel = synth.generate_model(fcfg, seed=43)
        fmdl = Model(fcfg.hparams(), fmodel)
        del fmodel
        log(f"F16 model generated + uploaded in {time.time() - t0:.1f}s")
        mixed_f16 = mixed_pass(np, Context, synth, fcfg, fmdl)
        fmdl.close()

    c4, single, cpu_more = None, None, None
    if args.config == "c3" and args.legs == "all":
        c4 = {}
        for bulk, key in ((configs.Q6_K, "q6_k"), (configs.Q8_0, "q8_0")):
            c4cfg, c4wl = configs.C4(bulk)
            leg = decode_leg(np, torch, c4cfg, c4wl, args.steps, args.warmup, args.cpu_steps, f"c4-{key}")
            c4[key] = {"value": round(leg["T"] / (leg["ms"] / 1000.0), 1), "unit": "tok/s",
                       "ms_per_step": round(leg["ms"], 4), "median_ms_per_step": round(leg["med_ms"], 4),
                       "dtype": dtype_of(bulk), "requests": leg["T"], "kv_lens": "log-uniform [16, 4096]",
                       "routing": "Zipf(1.2) expert popularity on load-balanced router logits",
                       "step_hbm": leg["step_hbm"], "roofline": leg["roofline"], "cpu_baseline": leg["cpu"],
                       "parity": leg["parity"],
                       "kernels_us_per_step": {k: round(t / args.steps * 1000.0, 1) for k, (t, n) in leg["prof"].items() if n}}
        single = single_stream(np, torch, args.steps * 5, args.warmup)
        if args.cpu_steps > 0:
            cpu_more = cpu_small(np, args.cpu_steps)

    line = {
        "metric": "batched-decode tok/s (Q4_K MoE step, 16 ragged reqs); % of HBM peak GB/s",
        "value": round(T / (ms / 1000.0), 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "median_ms_per_step": round(main_leg["med_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype_of(cfg.bulk),
        "data": "synthetic (random-init weights, N(0,1) f16 KV, uniform token ids)",
        "config": {"workload": f"{cfg.name}: {cfg.n_layer}-layer MoE backbone decode step, {T} ragged requests "
                               f"(KV {min(wl.kv_lens)}..{max(wl.kv_lens)}), d_model {cfg.n_embd}, "
                               f"{cfg.n_expert} experts top-{cfg.top_k}",
                   "requests": T, "kv_lens": wl.kv_lens, "parallelism": "single GPU"},
        "host_api": {"ms_per_step": round(main_leg["host_med"], 4), "tok_per_s": round(T / (main_leg["host_med"] / 1000.0), 1),
                     "note": "z2h_step with host buffers: inputs uploaded, logits read back, synchronous"},
        "step_hbm": main_leg["step_hbm"],
        "roofline": dict(main_leg["roofline"], traffic=profiled_traffic(args.config)),
        "kernels_us_per_step": {k: round(t / args.steps * 1000.0, 1) for k, (t, n) in main_leg["prof"].items() if n},
        "cpu_baseline": main_leg["cpu"],
        "parity": main_leg["parity"],
        "prefill": {"rows": n_pf, "passes": 1, "ms": round(pf_ms, 2), "rows_per_s": round(n_pf / pf_ms * 1000.0, 1)},
        "sampler": {"columns": T, "settings": "temperature 1.15, top-k 106, min-p 0.18, repetition 1.2 over 50",
                    "us_per_frame_step": round(samp_us, 1)},
        "mixed": mixed,
        "mixed_f16": mixed_f16,
        "c4": c4,
        "single_stream": single,
        "cpu_baselines": None if cpu_more is None else dict(cpu_more, c3=main_leg["cpu"],
                                                            c4_q6_k=c4["q6_k"]["cpu_baseline"], c4_q8_0=c4["q8_0"]["cpu_baseline"]),
    }
    if args.config != "c3":
        line["metric"] = "batched-decode tok/s (MoE step); % of HBM peak GB/s"
    print(json.dumps(line), flush=True)
    if args.calib_copy:
        dev = torch.device("cuda:0")
        src = torch.empty(64 << 20, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log("calibration copy: 256 MiB read + 256 MiB written")
    return 0


def cpu_share():
    """Threads for the CPU baseline: the cores this process may run on, capped by OMP_NUM_THREADS
    when it is set (the machine's share for one GPU); also nproc and the CPU model, for the record."""
    nproc = os.cpu_count() or 1
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = nproc
    cap = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    threads = max(1, min(avail, cap) if cap > 0 else avail)
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return threads, nproc, model


INT8_MFMA_PEAK_TOPS = 5000.0
F16_MFMA_PEAK_TFLOPS = 2500.0


def configs_f16():
    from zonos2_amd.configs import F16
    return F16


def dtype_of(bulk):
    """The arithmetic of the expert and projection matmuls for a weight type."""
    from zonos2_amd.configs import TYPE_NAMES
    w = TYPE_NAMES[bulk].lower()
    if w in ("q4_k", "q8_0"):
        act = "q8_k" if w == "q4_k" else "q8_0"
        return f"{w} weights x {act} activations (int8 MFMA dot, fp32 accumulate); f16 KV; fp32 router"
    if w == "q6_k":
        return "q6_k weights x q8_k activations (int8 MFMA dot, fp32 accumulate); f16 KV; fp32 router"
    return f"{w} weights x f16 activations (fp32 accumulate); f16 KV; fp32 router"


def type_name(t):
    from zonos2_amd.configs import TYPE_NAMES
    return TYPE_NAMES[t]


def gateup_kernel_of(bulk):
    from zonos2_amd.configs import TYPE_NAMES
    w = TYPE_NAMES[bulk]
    if w in ("Q4_K", "Q8_0", "Q6_K"):
        return f"k_gemv_mfma<{w}, DUAL> grouped expert gate/up + SwiGLU"
    return f"k_gemm_f16<DUAL> grouped expert gate/up + SwiGLU"



def mixed_pass(np, Context, synth, cfg, mdl):
    """One mixed pass of chunked prefill and decode rows on the same weights: 8 prefill chunks of
    256 prompt rows, each after a speaker row (a 2048-d N(0,1) embedding row in place of the summed
    token embeddings), at a 256-aligned offset inside a prompt of U[300, 1200] rows whose earlier rows
    are pre-filled N(0,1) in the KV cache, plus 32 decode columns with KV lengths U[32, 1200]:
    2088 rows through every layer in one z2h_step_mixed call (host API: ids up, 40 logit rows down).
    Median of 3 after one warm-up; algorithmic FLOPs count the expert, projection and attention-score
    products (2 per multiply-add)."""
    from zonos2_amd.configs import mixed_layout
    lay = mixed_layout(cfg)                        # seed 55: 8 x (256 + 1) + 32 = 2088 rows
    n_pre, n_dec, chunk = len(lay.r0), len(lay.dlen), 256
    r0, dlen, cap, spk = lay.r0, lay.dlen, lay.cap, lay.spk
    R = len(lay.slots)
    mctx = Context(None, n_pre + n_dec, cap, model=mdl, max_rows=R)
    for L in range(cfg.n_layer):
        for i, r in enumerate(r0):
            if r:
                k, v = synth.kv_rows(cfg, L, i, r, 11)
                mctx.kv_write(L, i, 0, k, v)
        for i, n in enumerate(dlen):
            k, v = synth.kv_rows(cfg, L, n_pre + i, n, 11)
            mctx.kv_write(L, n_pre + i, 0, k, v)
    args = (lay.slots, lay.npast, lay.ids, lay.out_rows)
    emap_a = lay.emap
    npast = lay.npast

    def one_pass():
        emb = mctx.speaker_embed(spk)                  # spk_lda -> spk_proj on the device (graph.cpp:262-297)
        return mctx.step_mixed(*args, emb_map=emap_a, emb=emb)

    one_pass()
    ts = []
    for _ in range(3):
        t0 = time.perf_counter()
        one_pass()
        ts.append(time.perf_counter() - t0)
    ms = float(np.median(ts)) * 1000.0
    mctx.close()
    d, ff, k = cfg.n_embd, cfg.n_ff, cfg.top_k
    R_qkvg = (cfg.n_head + 2 * cfg.n_head_kv) * cfg.head_dim + cfg.n_head
    per_row = 2 * (k * 3 * ff * d + R_qkvg * d + d * cfg.n_head * cfg.head_dim)
    ctx_rows = int(sum(int(n) + 1 for n in npast))
    flops = cfg.n_layer * (R * per_row + 2 * 2 * ctx_rows * cfg.n_head * cfg.head_dim)
    tops = flops / (ms / 1000.0) / 1e12
    f16 = cfg.bulk == configs_f16()
    peak, peak_unit = (F16_MFMA_PEAK_TFLOPS, "TFLOP/s (fp16)") if f16 else (INT8_MFMA_PEAK_TOPS, "TOP/s (int8)")
    log(f"mixed pass ({type_name(cfg.bulk)}): {R} rows ({n_pre} prefill chunks + {n_dec} decode) in {ms:.1f} ms, "
        f"{R / ms * 1000.0:.0f} rows/s, {tops:.1f} {peak_unit} algorithmic ({tops / peak:.2%} of the MFMA peak)")
    return {"rows": R, "prefill_chunks": n_pre, "chunk_rows": chunk, "decode_rows": n_dec, "ms": round(ms, 2),
            "rows_per_s": round(R / ms * 1000.0, 1),
            "roofline": {"bound": "mfma", "achieved": round(tops, 2), "peak": peak, "unit": peak_unit,
                         "frac": round(tops / peak, 5)},
            "weights": type_name(cfg.bulk).lower(), "speaker_rows": "2048-d N(0,1) speaker vectors through spk_lda -> spk_proj on the device (z2h_speaker_embed), in the timed pass"}


if __name__ == "__main__":
    sys.exit(main())
