"""Decode benchmark: Llama-3.2-3B-architecture Q8_0, batch 1, one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config llama-3.2-3b] [--no-cpu-baseline]
    python bench.py --config qwen3-8b | mistral-7b-v0.3 | tinyllama-1.1b   (the other decode configs)
    python bench.py --sweep                                             (the Q8_0 kernel sweep)
    python bench.py --sweep-kquant                                      (the K-quant prefill projections)

Workload: seeded synthetic N(0, 0.02) weights quantized to
Q8_0, a 512-token random prompt prefilled (n-1 tokens, as the reference seam does), then
greedy decode.  A "step" is one decode token through the resident engine's device-side
loop (embedding gather -> 28 layers -> lm_head -> argmax fed back on the device).  The
timed region is exactly K steps, bracketed by device synchronisation; weights, KV cache
and the token live in HBM throughout.

Prints one JSON line with the metric, the live roofline of the dominant kernel (the Q8_0
GEMV, HIP events on the engine's stream over a second pass of the same K steps) and the
CPU baseline (the C++ restatement of Camelid's CPU forward, timed on this host).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, AMD published peak
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 matrix-core peak, AMD published
HEADLINE = "llama-3.2-3b"
ARCH = {"llama-3.2-3b": "Llama-3.2-3B-arch Q8_0", "tinyllama-1.1b": "TinyLlama-1.1B-arch Q8_0",
        "mistral-7b-v0.3": "Mistral-7B-v0.3-arch Q8_0 (8K context)", "qwen3-8b": "Qwen3-8B-arch Q4_K_M"}
# MI355X peak engine clock (AMD published), for the VALU ceiling of the prefill GEMM's fold
PEAK_CLOCK_HZ = 2.4e9
# Measured HBM bytes per launch of the dominant kernel class, not measured by this script:
# rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes over `bench.py --probe-traffic`, each
# scaled by what the same counter reads for a device copy of known size, averaged over the
# GEMV launches of one C3 step (profiles/traffic_gemv_llama-3.2-3b_q8_0.md).
TRAFFIC: dict = {"llama-3.2-3b": 37285133}
TRAFFIC_SOURCE = ("profiles/traffic_gemv_llama-3.2-3b_q8_0.md: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE "
                  "passes, scaled by a copy kernel's reading; a recorded figure, not measured in this run")
# Q8_0 [N, K] shapes, weights N(0, 0.02) and activations N(0, 1), seed 2
SWEEP_SHAPES = [(2048, 2048), (5632, 2048), (2048, 5632), (32000, 2048), (128256, 3072)]


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def host_cpu() -> dict:
    """The host's CPU as lscpu reports it, and the CPUs this process may run on."""
    info = {"model": None, "nproc": os.cpu_count(), "physical_cores": None,
            "allowed_cpus": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None}
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        kv = dict(line.split(":", 1) for line in out.splitlines() if ":" in line)
        kv = {k.strip(): v.strip() for k, v in kv.items()}
        info["model"] = kv.get("Model name")
        if kv.get("Core(s) per socket") and kv.get("Socket(s)"):
            info["physical_cores"] = int(kv["Core(s) per socket"]) * int(kv["Socket(s)"])
    except (OSError, ValueError):
        pass
    return info


def cpu_baseline(model, cfg, prompt_len: int, n_steps: int, thread_counts: list) -> dict:
    """Oracle (C++ restatement of Camelid's CPU path) decode steps at the benchmark's
    positions: KV for the prompt is seeded with f16-rounded random rows, then `n_steps`
    greedy steps run from position prompt_len-1, once per thread count (OpenMP threads over
    output rows; the first count is the reported value)."""
    from oracle.oracle import OracleModel, set_threads
    orc = OracleModel(model, prompt_len + n_steps + 1)
    rng = np.random.default_rng(0)
    n = prompt_len - 1
    for layer in range(cfg.n_layers):
        k = rng.normal(0, 1, (cfg.n_kv_heads, n, cfg.head_dim)).astype(np.float32)
        v = rng.normal(0, 1, (cfg.n_kv_heads, n, cfg.head_dim)).astype(np.float32)
        orc.seed_kv(layer, k, v)
    runs = []
    for threads in thread_counts:
        set_threads(threads)
        tok = 1
        t0 = time.perf_counter()
        for i in range(n_steps):
            tok, _, _ = orc.forward(tok, n + i)
        dt = time.perf_counter() - t0
        runs.append({"threads": threads, "tok_s": round(n_steps / dt, 3), "s": round(dt, 2)})
        log(f"CPU baseline, {threads} threads: {n_steps / dt:.2f} tok/s")
    orc.close()
    return {"value": runs[0]["tok_s"], "unit": "tok/s", "cores": runs[0]["threads"], "kind": "port",
            "sample": f"{n_steps} greedy decode steps of the same {ARCH[cfg.name]} model at positions "
                      f"{n}..{n + n_steps - 1} (KV history seeded), oracle/camelid_oracle.cpp, "
                      f"{runs[0]['threads']} OpenMP threads over output rows",
            "runs": runs, "host": host_cpu()}


def hbm_bandwidth(bytes_per_array: int = 1 << 30, reps: int = 10) -> dict:
    """Measured HBM bandwidth of this device: STREAM triad and a read-only pass over arrays of
    1 GiB (well beyond the 256 MB last-level cache), best of `reps` passes."""
    import ctypes as C
    from camelid_amd import _native as N
    t, r = C.c_double(), C.c_double()
    N.check(N.lib().camelid_hip_hbm_bandwidth(bytes_per_array, reps, C.byref(t), C.byref(r)))
    return {"triad_GBps": round(t.value, 1), "read_GBps": round(r.value, 1), "spec_GBps": HBM_PEAK_GBS,
            "bytes_per_array": bytes_per_array, "passes": reps}


def run_sweep(iters_min: int = 200) -> dict:
    """each [N, K] Q8_0 matrix as a batch-1 GEMV (GB/s against HBM peak) and as the
    512-token prefill GEMM (int8 TOP/s against the matrix-core peak).  Weight copies rotate
    over more than 1 GB so that no launch finds its matrix in L2 or MALL; the activations are
    quantized on the device."""
    import ctypes as C
    from camelid_amd import _native as N
    from camelid_amd.engine import DeviceBuffer
    from camelid_amd.model import synth_f32, synth_q8_0
    L = N.lib()
    T = 512
    out = []
    for rows, k in SWEEP_SHAPES:
        wire = synth_q8_0(f"sweep.{rows}x{k}.weight", 2, rows, k)
        q = np.empty(rows * k, np.int8)
        d = np.empty(rows * k // 32, np.uint16)
        N.check(L.camelid_q8_0_repack(N.ptr(wire, C.c_uint8), rows, k, 34, N.ptr(q, C.c_int8), N.ptr(d, C.c_uint16)))
        wbytes = rows * k * 34 / 32
        copies = int(min(48, max(2, np.ceil(1.2e9 / wbytes))))
        qb = [DeviceBuffer.from_array(q) for _ in range(copies)]
        db = [DeviceBuffer.from_array(d) for _ in range(copies)]
        x = DeviceBuffer.from_array(synth_f32(f"sweep.{rows}x{k}.x", 2, T * k, 1.0))
        xq, xs = DeviceBuffer(T * k), DeviceBuffer(T * k // 32 * 4)
        N.check(L.camelid_hip_quantize_q8_0(x.ptr, T * k, xq.ptr, xs.ptr, None))
        y = DeviceBuffer(T * rows * 4)
        qp = (N.vp * copies)(*[b.ptr for b in qb])
        dp = (N.vp * copies)(*[b.ptr for b in db])
        ms = C.c_float(0)
        it = max(iters_min, 4 * copies)
        N.check(L.camelid_hip_time_q8_0(0, qp, dp, copies, rows, k, xq.ptr, xs.ptr, 1, y.ptr, it, C.byref(ms)))
        gemv_us = ms.value * 1e3 / it
        gbytes = wbytes + k * 34 / 32 + rows * 4
        itg = max(10, 2 * copies)
        N.check(L.camelid_hip_time_q8_0(1, qp, dp, copies, rows, k, xq.ptr, xs.ptr, T, y.ptr, itg, C.byref(ms)))
        gemm_us = ms.value * 1e3 / itg
        ops = 2.0 * rows * k * T
        out.append({"shape": [rows, k], "gemv_us": round(gemv_us, 2),
                    "gemv_gbs": round(gbytes / gemv_us / 1e3, 1), "gemv_hbm_frac": round(gbytes / gemv_us / 1e3 / HBM_PEAK_GBS, 4),
                    "gemm_tokens": T, "gemm_us": round(gemm_us, 1), "gemm_tops": round(ops / gemm_us / 1e6, 1),
                    "gemm_mfma_frac": round(ops / gemm_us / 1e6 / INT8_PEAK_TOPS, 4), "weight_copies": copies})
        log(f"sweep {rows}x{k}: GEMV {gemv_us:.2f} us {out[-1]['gemv_gbs']} GB/s; "
            f"GEMM(T={T}) {gemm_us:.1f} us {out[-1]['gemm_tops']} TOP/s")
        del qb, db, x, xq, xs, y
    return {"metric": "Q8_0 GEMV GB/s and prefill GEMM int8 TOP/s, isolated kernel sweep, 1 MI355X",
            "config": {"workload": "BASELINE configs[1]: Q8_0 [N,K] weights N(0,0.02) seed 2, activations N(0,1) "
                                   "quantized on device; GEMV batch 1, GEMM batch 512"},
            "peaks": {"hbm_gbs": HBM_PEAK_GBS, "int8_tops": INT8_PEAK_TOPS}, "shapes": out}


KQUANT_SWEEP_SHAPES = [(1, 4096, 4096), (1, 5120, 4096), (1, 24576, 4096), (1, 4096, 12288), (2, 1024, 4096)]


def run_sweep_kquant(tokens: int = 512, iters: int = 20) -> dict:
    """The K-quant prefill projections of configs[4] (Qwen3-8B Q4_K_M: q, q|k, gate|up, down as
    Q4_K; v as Q6_K) over a 512-token chunk: k_gemm_q4k / k_gemm_q6k2 on the int8 matrix cores,
    `iters` back-to-back launches after one warm-up timed with HIP events on the launching stream
    (Q6_K's class-major weight planes built once beforehand, as at model upload).  int8 TOP/s =
    2 N K T / time, against the matrix-core peak."""
    import ctypes as C
    from camelid_amd import _native as N
    from camelid_amd.engine import DeviceBuffer
    from camelid_amd.model import synth_f32, synth_kquant
    L = N.lib()
    T = tokens
    out = []
    for quant, rows, k in KQUANT_SWEEP_SHAPES:
        wire = synth_kquant(f"ksweep.{rows}x{k}.weight", 2, rows, k, quant)
        nsb = k // 256
        a = np.empty(rows * k // 2, np.uint8)
        b = np.empty(rows * nsb * (16 if quant == 1 else 64), np.uint8)
        sc = np.empty(max(rows * nsb * 16, 1), np.int8)
        d = np.empty(max(rows * nsb, 1), np.uint16)
        N.check(L.camelid_kquant_repack(quant, N.ptr(wire, C.c_uint8), rows, k, N.ptr(a, C.c_uint8),
                                        N.ptr(b, C.c_uint8), N.ptr(sc, C.c_int8), N.ptr(d, C.c_uint16)))
        da, db, dsc, dd = (DeviceBuffer.from_array(v) for v in (a, b, sc, d))
        x = DeviceBuffer.from_array(synth_f32(f"ksweep.{rows}x{k}.x", 2, T * k, 1.0))
        yd, yq, ybs = DeviceBuffer(T * nsb * 4), DeviceBuffer(T * k), DeviceBuffer(T * k // 32 * 4)
        N.check(L.camelid_hip_quantize_q8_k(x.ptr, T * k, yd.ptr, yq.ptr, ybs.ptr, None))
        y = DeviceBuffer(T * rows * 4)

        ms = C.c_float(0.0)
        N.check(L.camelid_hip_time_kquant(quant, da.ptr, db.ptr, dsc.ptr, dd.ptr, rows, k, T, yd.ptr, yq.ptr,
                                          y.ptr, iters, C.byref(ms)))
        us = ms.value / iters * 1e3
        ops = 2.0 * rows * k * T
        q6 = "k_gemm_q6k" if os.environ.get("CAMELID_HIP_Q6K_GEMM2") == "0" else "k_gemm_q6k2"
        name = "k_gemm_q4k" if quant == 1 else (q6 if T > 8 else "k_gemv_q6k_multi")
        out.append({"quant": "Q4_K" if quant == 1 else "Q6_K", "kernel": name, "shape": [rows, k], "tokens": T,
                    "us": round(us, 1), "tops": round(ops / us / 1e6, 1),
                    "mfma_frac": round(ops / us / 1e6 / INT8_PEAK_TOPS, 4)})
        log(f"kquant sweep {out[-1]['quant']} {rows}x{k} T={T}: {name} {us:.1f} us, {out[-1]['tops']} TOP/s")
        del da, db, dsc, dd, x, yd, yq, ybs, y
    return {"metric": "K-quant prefill projection int8 TOP/s over a 512-token chunk, 1 MI355X",
            "config": {"workload": "configs[4] Qwen3-8B Q4_K_M projection shapes, weights N(0,0.02) seed 2, "
                                   "activations N(0,1) quantized to Q8_K on device"},
            "peaks": {"int8_tops": INT8_PEAK_TOPS}, "shapes": out}


ATT_PHASES = ("qkv_rope_kvstore", "scores_max", "exp", "denominator", "output_sums", "quantize_store")


def kquant_norm_phases(cfg, gs) -> dict:
    """The norm-fused K-quant launches of the last layer (k_norm_qk4_v6: kind 0, k_norm_gemv_q4k:
    kind 1), from the measurement build's stamps: workgroup 0 (the RMSNorm + Q8_K row) in slot
    0 -- 0 start, 6 squares stored, 8..11 after the one-pass sum's f64 scan, segmented scan,
    special-step entries and replay, 12 the special-step count, 7 sum done, 2 y, 3 block maxima,
    4 quants, 5 stores completed, 1 published; every ceil(grid / 256)-th other workgroup in slot
    blockIdx / that -- 0 start, 3 flag seen and activation staged, 5 end.  Times in us from
    workgroup 0's start."""
    res = {}
    hd, nq, nkv = cfg.head_dim, cfg.n_heads, cfg.n_kv_heads
    gu_r = 16 if 2 * cfg.ffn_dim >= 16384 else 8  # (rows per gate|up workgroup, as the engine launches it)
    wgs = {0: ((nq + nkv) * hd + 7) // 8 + (nkv * hd + 7) // 8, 1: (2 * cfg.ffn_dim + gu_r - 1) // gu_r}
    for kind, name in enumerate(("norm_qk4_v6", "norm_gemv_q4k_gate_up")):
        g = gs[kind]
        w0 = g[0]
        if w0[0] <= 0:
            continue
        t0 = w0[0]
        us = lambda v: round(float(v - t0) * 0.01, 3)
        ph = {"squares_stored": us(w0[6]), "sum_f64_scan": us(w0[8]), "sum_seg_scan": us(w0[9]),
              "sum_specials": us(w0[10]), "sum_replay": us(w0[11]), "special_steps": int(w0[12]),
              "sum_done": us(w0[7]), "y": us(w0[2]), "block_maxima": us(w0[3]), "quants": us(w0[4]),
              "stores_completed": us(w0[5]), "published": us(w0[1])}
        every = (1 + wgs[kind] + 255) // 256
        ws = g[1:]
        ok = (ws[:, 0] > 0) & (ws[:, 3] > 0) & (ws[:, 5] > 0)
        ws = ws[ok]
        if len(ws):
            ph.update({"waiters_sampled": int(len(ws)), "waiters_every": every,
                       "waiter_start_mean": us(ws[:, 0].mean()), "waiter_start_max": us(ws[:, 0].max()),
                       "staged_mean": us(ws[:, 3].mean()), "staged_min": us(ws[:, 3].min()),
                       "end_mean": us(ws[:, 5].mean()), "end_max": us(ws[:, 5].max())})
        res[name] = ph
        log(f"{name} phases (us from workgroup 0's start): " + ", ".join(f"{k} {v}" for k, v in ph.items()))
    return res


def fused_attention_phases(st) -> dict:
    """The single-workgroup attention's phases from its stamps st[layer][head][9]."""
    d = np.diff(st[:, :, :7], axis=2) * 0.01  # 100 MHz ticks -> us
    res = {name: round(float(d[:, :, i].mean()), 3) for i, name in enumerate(ATT_PHASES)}
    # inside the score phase (from its start): thread 0's K-row loads issued, wave 0's scores done
    for i, name in ((7, "k_rows_issued"), (8, "wave0_scores_done")):
        v = (st[:, :, i] - st[:, :, 1]) * 0.01
        res[name] = round(float(v[st[:, :, i] > 0].mean()), 3) if (st[:, :, i] > 0).any() else None
    res["workgroup_total"] = round(float((st[:, :, 6] - st[:, :, 0]).mean() * 0.01), 3)
    res["start_spread"] = round(float((st[:, :, 0].max(1) - st[:, :, 0].min(1)).mean() * 0.01), 3)
    res["launch_span"] = round(float((st[:, :, 6].max(1) - st[:, :, 0].min(1)).mean() * 0.01), 3)
    log("attention phases (us, mean over layers and heads): " + ", ".join(f"{k} {v}" for k, v in res.items()))
    return res


def attention_phases(cfg) -> dict:
    """Per-phase times of the decode attention in the last timed step, from the measurement
    build's in-kernel timestamps (100 MHz counter, thread 0 of every head's workgroup): the
    mean over layers and heads of each phase, the workgroups' start spread within a launch
    and the launch span (first start to last end), in microseconds."""
    import ctypes as C
    from camelid_amd import _native as N
    na, ng, nsp, nao = 64 * 64 * 9, 2 * 256 * 13, 2 * 1024 * 8, 64 * 2 * 4
    buf = (C.c_uint64 * (na + ng + nsp + nao))()
    got = C.c_size_t(0)
    N.check(N.lib().camelid_hip_phase_stamps(buf, na + ng + nsp + nao, C.byref(got)))
    allst = np.frombuffer(buf, np.uint64).astype(np.int64)
    st = allst[:na].reshape(64, 64, 9)[:cfg.n_layers, :cfg.n_heads]
    res = {}
    if (st[:, :, 0] > 0).all():  # (the single-workgroup attention ran; else the split one did)
        res.update(fused_attention_phases(st))
        # the output projection's workgroups of the same launches (first and last workgroup),
        # from the attention workgroups' first start and last end of each layer
        ao = allst[na + ng + nsp:].reshape(64, 2, 4)[:cfg.n_layers]
        if (ao[:, :, 0] > 0).all():
            a0, a1 = st[:, :, 0].min(1)[:, None], st[:, :, 6].max(1)[:, None]
            ph = {"start_from_attention_start": float((ao[:, :, 0] - a0).mean() * 0.01),
                  "tag_seen_from_attention_end": float((ao[:, :, 1] - a1).mean() * 0.01),
                  "staged_from_attention_end": float((ao[:, :, 2] - a1).mean() * 0.01),
                  "end_from_attention_end": float((ao[:, :, 3] - a1).mean() * 0.01),
                  "last_end_from_attention_start": float((ao[:, :, 3].max(1)[:, None] - a0).mean() * 0.01)}
            res["output_projection"] = {k: round(v, 3) for k, v in ph.items()}
            log("output projection workgroups (us): " + ", ".join(f"{k} {v:.3f}" for k, v in ph.items()))
    # the norm-fused GEMVs of the last layer (mean over the workgroups that recorded)
    gs = allst[na:na + ng].reshape(2, 256, 13)
    kquant = cfg.quant_scheme != "q8_0"
    if kquant:
        res.update(kquant_norm_phases(cfg, gs))
    for kind, name in enumerate(() if kquant else ("qkv_norm_gemv", "gate_up_norm_gemv")):
        g = gs[kind]
        g = g[g[:, 0] > 0]
        if not len(g):
            continue
        t0 = g[:, 0]
        ph = {"norm_inputs_arrived": float((g[:, 6] - t0).mean() * 0.01),
              "sum_of_squares_done": float((g[:, 7] - t0).mean() * 0.01),
              "sum_f64_scan": float((g[:, 8] - t0).mean() * 0.01) if (g[:, 8] > 0).all() else None,
              "sum_seg_scan": float((g[:, 9] - t0).mean() * 0.01) if (g[:, 9] > 0).all() else None,
              "sum_specials": float((g[:, 10] - t0).mean() * 0.01) if (g[:, 10] > 0).all() else None,
              "sum_replay": float((g[:, 11] - t0).mean() * 0.01) if (g[:, 11] > 0).all() else None,
              "special_steps_mean": float(g[:, 12].mean()), "special_steps_max": float(g[:, 12].max()),
              "norm_done": float((g[:, 1] - t0).mean() * 0.01),
              "weight_loads_issued": float((g[:, 2] - t0).mean() * 0.01),
              "past_norm_barrier": float((g[:, 3] - t0).mean() * 0.01),
              "dots_done": float((g[:, 4] - t0).mean() * 0.01),
              "end": float((g[:, 5] - t0).mean() * 0.01),
              "start_spread": float((t0.max() - t0.min()) * 0.01),
              "launch_span": float((g[:, 5].max() - t0.min()) * 0.01),
              "workgroups": int(len(g))}
        res[name] = {k: (round(v, 3) if v is not None else None) for k, v in ph.items()}
        log(f"{name} phases (us from each workgroup's start): " +
            ", ".join(f"{k} {v:.3f}" for k, v in ph.items() if v is not None))
    # the split attention (when it ran in the last layer)
    sp = allst[na + ng:na + ng + nsp].reshape(2, 1024, 8)
    for kind, name, labels in ((0, "att_scores_split", ("q_built", "scores_done", "end")),
                               (1, "att_out_split", ("scores_max", "exp", "denominator", "output_sums", "end"))):
        g = sp[kind]
        g = g[(g[:, 0] > 0) & (g[:, len(labels)] > 0)]
        if not len(g):
            continue
        t0 = g[:, 0]
        ph = {lab: float((g[:, i + 1] - t0).mean() * 0.01) for i, lab in enumerate(labels)}
        if kind == 1 and (g[:, 6] > 0).any():  # the output chain's time in its adds / at barriers
            ph["chain_adds"] = float(g[:, 6].mean() * 0.01)
            ph["chain_barrier_wait"] = float(g[:, 7].mean() * 0.01)
        ph["start_spread"] = float((t0.max() - t0.min()) * 0.01)
        ph["launch_span"] = float((g[:, len(labels)].max() - t0.min()) * 0.01)
        ph["workgroups"] = int(len(g))
        res[name] = {k: round(v, 3) for k, v in ph.items()}
        log(f"{name} phases (us from each workgroup's start): " + ", ".join(f"{k} {v:.3f}" for k, v in ph.items()))
    # the output projection's workgroups of the last split launch (first and last workgroup:
    # the Q4_K ones of k_att_fused or the Q8_0 ones of k_att_out), from the split output
    # workgroups' first start and last end
    ao = allst[na + ng + nsp:].reshape(64, 2, 4)[cfg.n_layers - 1]
    g = sp[1]
    g = g[(g[:, 0] > 0) & (g[:, 5] > 0)]
    if (ao[:, 0] > 0).all() and (ao[:, 3] > 0).all() and len(g) and "output_projection" not in res:
        a0, a1 = g[:, 0].min(), g[:, 5].max()
        ph = {"start_from_output_start": float((ao[:, 0] - a0).mean() * 0.01),
              "tag_seen_from_output_end": float((ao[:, 1] - a1).mean() * 0.01),
              "staged_from_output_end": float((ao[:, 2] - a1).mean() * 0.01),
              "end_from_output_end": float((ao[:, 3] - a1).mean() * 0.01),
              "last_end_from_output_start": float((ao[:, 3].max() - a0) * 0.01)}
        res["output_projection_split"] = {k: round(v, 3) for k, v in ph.items()}
        log("output projection workgroups of the split launch, last layer (us): " +
            ", ".join(f"{k} {v:.3f}" for k, v in ph.items()))
    return res


def probe_traffic() -> int:
    """The workload of the traffic counter passes: a 256 MiB device-to-device copy (the
    counters' scale reference), then three C3 decode steps launched without graphs on a
    seeded 511-position KV history."""
    import ctypes as C
    os.environ["CAMELID_HIP_GRAPHS"] = "0"
    from camelid_amd.engine import DeviceBuffer
    from camelid_amd.model import CONFIGS, ResidentSession, SyntheticModel
    hip = C.CDLL("libamdhip64.so")
    n = 256 << 20
    a, b = DeviceBuffer(n), DeviceBuffer(n)
    for _ in range(3):
        if hip.hipMemcpy(b.ptr, a.ptr, C.c_size_t(n), 3) != 0:
            raise RuntimeError("device copy failed")
    cfg = CONFIGS[HEADLINE]
    model = SyntheticModel.generate(cfg)
    P = cfg.prompt_len
    sess = ResidentSession(model, P + 16, device_loop=True)
    eng = sess.engine
    rng = np.random.default_rng(0)
    for layer in range(cfg.n_layers):
        k = rng.normal(0, 1, (cfg.n_kv_heads, P - 1, cfg.head_dim)).astype(np.float32)
        v = rng.normal(0, 1, (cfg.n_kv_heads, P - 1, cfg.head_dim)).astype(np.float32)
        eng.seed_layer(layer, k, v, P - 1)
    eng.set_filled(P - 1)
    log(f"probe: 3 copies of 256 MiB, then decode tokens {list(eng.generate(1, P - 1, 3, cfg.scale()))}")
    sess.close()
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--config", default="llama-3.2-3b")
    ap.add_argument("--prompt", type=int, default=None, help="prompt length (default: the config's)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-steps", type=int, default=16)
    ap.add_argument("--no-profile", action="store_true")
    ap.add_argument("--no-hbm-probe", action="store_true", help="skip the HBM triad/read bandwidth probe")
    ap.add_argument("--sweep", action="store_true", help="run the isolated Q8_0 GEMV/GEMM sweep (configs[1])")
    ap.add_argument("--sweep-kquant", action="store_true",
                    help="time the K-quant prefill projections (Q4_K GEMM, Q6_K multi-token GEMV) of configs[4]")
    ap.add_argument("--probe-traffic", action="store_true",
                    help="the workload of the rocprofv3 FETCH_SIZE/WRITE_SIZE passes (no JSON line)")
    ap.add_argument("--phase-stamps", action="store_true",
                    help="load the measurement build (libcamelid_hip_stamps.so, built by `python -m "
                         "camelid_amd.build --stamps`) and report the decode attention's per-phase times "
                         "from in-kernel timestamps of the last timed step")
    ap.add_argument("--seed-kv", action="store_true",
                    help="seed the prompt's KV rows with random f16 values instead of running the prefill "
                         "(kernel profiling of the decode steps alone; skips the parity check)")
    args = ap.parse_args()

    if args.phase_stamps:  # (before the library is loaded)
        os.environ["CAMELID_HIP_LIB"] = "libcamelid_hip_stamps.so"
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the resident decode path runs on a single MI355X with no "
              "sharding or collectives (multi-GPU sharding is a design note, not a measured path).",
              file=sys.stderr)
        return 2

    from camelid_amd.engine import device_info
    from camelid_amd.model import CONFIGS, ResidentSession, SyntheticModel, prompt_tokens, rope_tables

    if args.probe_traffic:
        return probe_traffic()
    if args.sweep:
        dev_name, n_cu = device_info()
        log(f"device {dev_name}, {n_cu} CUs; Q8_0 kernel sweep")
        res = run_sweep()
        res["config"]["device"] = dev_name
        print(json.dumps(res), flush=True)
        return 0

    if args.sweep_kquant:
        dev_name, n_cu = device_info()
        log(f"device {dev_name}, {n_cu} CUs; K-quant prefill projection sweep")
        res = run_sweep_kquant()
        res["config"]["device"] = dev_name
        print(json.dumps(res), flush=True)
        return 0

    cfg = CONFIGS[args.config]
    P = args.prompt or cfg.prompt_len
    K, W = args.steps, args.warmup
    dev_name, n_cu = device_info()
    log(f"device {dev_name}, {n_cu} CUs; config {cfg.name}: prompt {P}, warmup {W}, steps {K}")

    t0 = time.perf_counter()
    model = SyntheticModel.generate(cfg)
    log(f"generated synthetic {ARCH[cfg.name]} weights in {time.perf_counter() - t0:.1f}s")
    prompt = prompt_tokens(cfg, P)
    max_pos = P + W + K
    t0 = time.perf_counter()
    sess = ResidentSession(model, max_pos, device_loop=True)
    eng = sess.engine
    log(f"uploaded weights in {time.perf_counter() - t0:.1f}s")

    # prefill of the first P-1 prompt tokens (inference.rs:4411), timed separately
    t0 = time.perf_counter()
    if args.seed_kv:
        rng = np.random.default_rng(0)
        for layer in range(cfg.n_layers):
            k = rng.normal(0, 1, (cfg.n_kv_heads, P - 1, cfg.head_dim)).astype(np.float32)
            v = rng.normal(0, 1, (cfg.n_kv_heads, P - 1, cfg.head_dim)).astype(np.float32)
            eng.seed_layer(layer, k, v, P - 1)
        eng.set_filled(P - 1)
        prefill_s = None
        log(f"seeded KV for {P - 1} positions")
    else:
        sess.prefill(prompt[:-1])
        prefill_s = time.perf_counter() - t0
        log(f"prefill {P - 1} tokens: {prefill_s:.3f}s")

    pos0 = P - 1
    warm = eng.generate(int(prompt[-1]), pos0, W, cfg.scale()) if W else np.array([prompt[-1]], np.uint32)
    last = int(warm[-1]) if W else int(prompt[-1])
    start_pos = pos0 + W
    from camelid_amd import _native as N
    N.check(N.lib().camelid_hip_synchronize())
    t0 = time.perf_counter()
    toks = eng.generate(last, start_pos, K, cfg.scale())
    N.check(N.lib().camelid_hip_synchronize())
    dt = time.perf_counter() - t0
    tok_s = K / dt
    log(f"decode {K} steps: {dt * 1e3:.1f} ms -> {tok_s:.1f} tok/s")

    # algorithmic bytes of the timed steps (positions start_pos .. start_pos+K-1)
    total_bytes = sum(cfg.decode_bytes(p) for p in range(start_pos, start_pos + K))
    hbm_frac = total_bytes / dt / (HBM_PEAK_GBS * 1e9)

    # parity: the stream must equal the oracle's golden stream when one exists
    stream = [int(t) for t in (list(warm) if W else [])] + [int(t) for t in toks]
    parity = None
    # the longest committed stream for this prompt length (a shorter one is a prefix check)
    golds = sorted((ROOT / "tests" / "golden").glob(f"{cfg.name}_p{P}_d*.json"),
                   key=lambda f: int(f.stem.rsplit("_d", 1)[1]))
    gold = golds[-1] if golds else None
    if gold is not None and not args.seed_kv:
        g = json.loads(gold.read_text())
        n = min(len(stream), len(g["tokens"]))
        parity = {"golden": gold.name, "compared": n, "identical": stream[:n] == g["tokens"][:n]}
        log(f"token parity vs golden: {parity}")

    phases = attention_phases(cfg) if args.phase_stamps else None

    roofline = None
    roofline_attention = None
    prof = None
    if not args.no_profile:
        eng.set_filled(start_pos)
        eng.profile_begin()
        toks2 = eng.generate(last, start_pos, K, cfg.scale())
        prof = eng.profile_end()
        assert [int(t) for t in toks2] == [int(t) for t in toks], "profiled pass diverged"
        g = prof["gemv"]
        achieved = g["bytes"] / (g["ms"] * 1e-3) / 1e9
        kname = ("Q8_0 GEMV: k_gemv_norm (RMSNorm + qkv) + k_gemv_k (down + residual) + k_gemv_gu_silu "
                 "(RMSNorm + gate/up + SwiGLU + Q8_0) + k_gemv_argmax (lm_head); the o projection runs inside the "
                 "attention launch (k_attention / k_att_fused) and is counted with it" if cfg.quant_scheme == "q8_0"
                 else "K-quant GEMV: k_gemv_q4k + k_gemv_q6k (incl. lm_head); from the split attention's first "
                 "position on, the Q4_K o projection runs inside that launch (k_att_fused) and is counted with it")
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": TRAFFIC.get(cfg.name),
                    "traffic_source": TRAFFIC_SOURCE if cfg.name in TRAFFIC else None,
                    "kernel": kname + ", all launches of K steps (algorithmic bytes / summed dispatch durations)",
                    "avg_launch_us": round(g["ms"] * 1e3 / max(g["launches"], 1), 3),
                    "launches": g["launches"]}
        # the costliest single launch per step: the decode attention (with the o projection's
        # workgroups where they ride in it), reported against the same HBM peak; its time is set by
        # the CPU-order serial f32 chains (scores, softmax denominator, output sums), not by bytes
        a = prof["attention"]
        if a["launches"]:
            att_achieved = a["bytes"] / (a["ms"] * 1e-3) / 1e9
            roofline_attention = {
                "bound": "hbm", "achieved": round(att_achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(att_achieved / HBM_PEAK_GBS, 4),
                "kernel": ("decode attention + o projection (k_attention / k_att_fused with the W_o workgroups)"
                           if cfg.quant_scheme == "q8_0" else
                           "decode attention (k_attention; k_att_fused with the Q4_K W_o workgroups)")
                + ": K/V read and written, q/k/v in, output and (where its workgroups ride in the launch) W_o + "
                  "residual bytes / summed dispatch durations",
                "avg_launch_us": round(a["ms"] * 1e3 / a["launches"], 3), "launches": a["launches"],
                "share_of_step": round(a["ms"] / (sum(v["ms"] for v in prof.values()) or 1.0), 4),
                "note": "latency-bound: the in-order f32 chains the CPU reference fixes, not HBM bytes"}
        log("per-kernel (profiled pass): " + ", ".join(
            f"{k} {v['ms']:.2f}ms/{v['launches']}" for k, v in prof.items()))

    # speculative verify (verify_batch): the first 8 timed steps' inputs in one batched
    # forward; its tokens must be the decode loop's.  Host call incl. input staging.
    verify = None
    if K >= 8 and not args.seed_kv:
        inputs = [last] + [int(t) for t in toks[:7]]
        vcos, vsin = rope_tables(cfg, start_pos, 8)
        embs = model.embed(inputs)
        eng.set_filled(start_pos)
        pred = eng.verify_batch(embs, vcos, vsin, start_pos, cfg.scale())
        t0 = time.perf_counter()
        for _ in range(5):
            pred = eng.verify_batch(embs, vcos, vsin, start_pos, cfg.scale())
        vdt = (time.perf_counter() - t0) / 5
        verify = {"k": 8, "ms": round(vdt * 1e3, 3), "tokens_identical": [int(t) for t in pred] == [int(t) for t in toks[:8]],
                  "tok_s_if_all_accepted": round(8 / vdt, 1)}
        log(f"verify k=8: {vdt * 1e3:.2f} ms, tokens identical to the decode loop: {verify['tokens_identical']}")

    # prefill projections under the profiler: a second prefill of the same prompt from
    # position 0 (rewrites the same KV rows), for the matrix-core utilisation
    prefill_mm = None
    if not args.no_profile and not args.seed_kv:
        eng.set_filled(0)
        eng.profile_begin()
        sess.prefill(prompt[:-1])
        pprof = eng.profile_end()
        g = pprof["prefill_gemm"]
        tops = g["bytes"] / (g["ms"] * 1e-3) / 1e12 if g["ms"] else 0.0
        # the bit-exact fold costs 3 unpacked VALU ops per output row, token and 32-wide block
        # (64 int8 ops): float(dot) * w_scale as one mixed FMA on the dot offset by 1.5 * 2^23,
        # the product with the activation scale, the add; a ceiling of 64 lanes x clock / 3 x 64
        # ops per CU (the plain form's 4 ops, for matrices with an infinite weight scale, only
        # lowers it)
        fold_ceiling = n_cu * 64 * PEAK_CLOCK_HZ / 3 * 64 / 1e12
        # (the same rate over the ceiling of the 4-operation fold -- convert, x w_scale, x x_scale,
        # add -- which the GEMM used before the offset accumulator: the figure earlier builds reported)
        fold4_ceiling = fold_ceiling * 3 / 4
        prefill_mm = {"tokens": P - 1, "gemm_tops": round(tops, 1), "gemm_ms": round(g["ms"], 3),
                      "gemm_launches": g["launches"], "int8_peak_tops": INT8_PEAK_TOPS,
                      "mfma_frac": round(tops / INT8_PEAK_TOPS, 4),
                      "valu_fold_ceiling_tops": round(fold_ceiling, 1),
                      "frac_of_fold_ceiling": round(tops / fold_ceiling, 4), "fold_valu_ops": 3,
                      "frac_of_4op_fold_ceiling": round(tops / fold4_ceiling, 4),
                      "all_kernels_ms": round(sum(v["ms"] for v in pprof.values()), 3)}
        log(f"prefill projections: {tops:.1f} TOP/s over {g['launches']} launches "
            f"({tops / INT8_PEAK_TOPS:.3f} of the int8 peak, {tops / fold_ceiling:.3f} of the fold ceiling)")

    hbm = None
    if not args.no_hbm_probe:
        hbm = hbm_bandwidth()
        hbm["decode_frac_of_triad"] = round(total_bytes / dt / 1e9 / hbm["triad_GBps"], 4)
        hbm["decode_frac_of_read"] = round(total_bytes / dt / 1e9 / hbm["read_GBps"], 4)
        if roofline:
            roofline["frac_of_measured_read"] = round(roofline["achieved"] / hbm["read_GBps"], 4)
        log(f"HBM measured: triad {hbm['triad_GBps']} GB/s, read {hbm['read_GBps']} GB/s (spec {HBM_PEAK_GBS})")

    cpu = None
    if not args.no_cpu_baseline:
        share = int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))
        share = min(share, len(os.sched_getaffinity(0)))
        counts = [share] + ([1] if share > 1 else [])
        log(f"CPU baseline: {args.cpu_steps} oracle decode steps at {counts} threads")
        cpu = cpu_baseline(model, cfg, P, args.cpu_steps, counts)

    out = {
        "metric": f"decode tok/s & % of HBM roofline, {ARCH[cfg.name]}, batch 1, 1 MI355X",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(dt * 1e3 / K, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("int8xint8->int32, f32 accumulate (Q8_0)" if cfg.quant_scheme == "q8_0" else
                  "Q4_K/Q6_K x Q8_K -> int32, f32 accumulate"),
        "data": f"synthetic: seeded N(0,0.02) weights quantized to {cfg.quant_scheme.upper()}, random prompt ids",
        "config": {"workload": f"{ARCH[cfg.name]} greedy decode, batch 1, {P}-token prompt, "
                               f"steps at positions {start_pos}..{start_pos + K - 1}",
                   "prompt_len": P, "decode_steps": K, "device": dev_name},
        "hbm_roofline_frac": round(hbm_frac, 4),
        "bytes_per_token": round(total_bytes / K),
        "prefill_tok_s": round((P - 1) / prefill_s, 2) if prefill_s else None,
        "prefill_matrix_cores": prefill_mm,
        "hbm_measured": hbm,
        "parity": parity,
        "roofline": roofline,
        "roofline_attention": roofline_attention,
        "cpu_baseline": cpu,
        "verify": verify,
    }
    if prof:
        out["kernels_ms"] = {k: round(v["ms"], 3) for k, v in prof.items()}
    if phases:
        out["attention_phases_us"] = phases
    print(json.dumps(out), flush=True)
    sess.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
