#!/usr/bin/env python3
"""Decode hot-path benchmark on one MI355X.

Workload: one Qwen3-8B decoder layer of single-token
decode through the hot path -- attn_q/attn_k Q4_K, attn_v Q6_K, GQA attention
(32 query / 8 kv heads, head_dim 128) over an fp16 KV cache of 8192
positions, attn_o Q4_K, ffn_gate/ffn_up Q4_K 12288x4096, ffn_down Q6_K
4096x12288.  A step is one such layer, launched as QwenModel::forward_token
launches it: attn_q/k/v as one grouped GEMV launch, attention (split and
merge), attn_o, ffn_gate/ffn_up with SwiGLU in one launch, ffn_down (the
norms, RoPE and residual adds between them are not part of the step).
Steps rotate over LAYERS distinct
copies of weights and caches (>= 512 MB in total) so every byte comes from
HBM, not the 256 MB Infinity Cache.  Inputs are synthetic (seeded random
quant blocks with d, dmin in [1e-3, 1e-2]; N(0,1) fp16 activations/caches)
and are resident in HBM before timing starts.

value = algorithmic bytes per step / time per step (GB/s, all kernels of the
step; HIP events on the launch stream around the K timed steps).  roofline:
the kernel with the largest share of step time, its algorithmic bytes per
launch over its average launch duration over a second pass of the same K
steps, from HIP events that each of its kernels' dispatches stamps
(hipExtLaunchKernel; for attention, the split and merge kernels' durations
added, as rocprofv3 counts them), every launch of that pass run with the
queue drained before and after it (a stamped dispatch's events otherwise
also count the wait for the kernel before it and the launches queued
behind it).
rocprof_step: the same steps re-run in a child process under rocprofv3
--kernel-trace, each op's mean kernel duration as the trace records it (the
figures of the committed profiles/ summaries; roofline.rocprof is the
dominant kernel's roofline from them); configs 1 and 2 likewise re-run
under rocprofv3 (their kernel_us; kernel_us_stamped is the dispatch-stamped
figure).  cpu_baseline: the
oracle's restatement of the reference's host arithmetic (dequant to fp16 with
the host rule, fp32 dot; fp32 attention) on a bounded sample of the same
layer, on this machine's host cores.  attention_cfg4
(16 sequences in one batched attention launch).  decode_cfg5: BASELINE
config 5 (the whole synthetic Qwen3-8B, greedy decode tok/s) from
bin/decode_qwen3, its weights written to a GGUF file in the temp directory
and loaded by QwenModel::load(GgufFile) (load time and GB/s reported);
decode_cfg5_fp16: the same file loaded with DequantizeToFp16 (fp16 weights,
the fp16 GEMVs), 64-token prompt then 128 greedy steps.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "citlali-llm-engine_amd"))

HBM_PEAK_GBPS = 8000.0
LAYERS = 4
COPY_HALVES = 1 << 29   # 1 GiB read + 1 GiB written by the calibration copy
HIDDEN, FFN, HEADS, KV_HEADS, HEAD_DIM, CTX = 4096, 12288, 32, 8, 128, 8192

# (name, kind, rows=out_features, cols=in_features, input, output)
GEMVS = [
    ("attn_q", "q4k", HEADS * HEAD_DIM, HIDDEN, "x", "q"),
    ("attn_k", "q4k", KV_HEADS * HEAD_DIM, HIDDEN, "x", "k"),
    ("attn_v", "q6k", KV_HEADS * HEAD_DIM, HIDDEN, "x", "v"),
    ("attn_o", "q4k", HIDDEN, HEADS * HEAD_DIM, "att", "o"),
    ("ffn_gate", "q4k", FFN, HIDDEN, "x", "gate"),
    ("ffn_up", "q4k", FFN, HIDDEN, "x", "up"),
    ("ffn_down", "q6k", HIDDEN, FFN, "up", "down"),
]
# the step's launches, as QwenModel::forward_token issues them for one layer
ORDER = ["attn_qkv", "attention", "attn_o", "ffn_gate_up", "ffn_down"]
SB_BYTES = {"q4k": 144, "q6k": 210}


def weight_bytes(kind, rows, cols):
    return rows * (cols // 256) * SB_BYTES[kind]


def attention_bytes(L):
    return 2 * L * KV_HEADS * HEAD_DIM * 2 + 2 * HEADS * HEAD_DIM * 2


def kernel_bytes():
    """Algorithmic bytes per launch: every weight byte once, the shared input
    once, each output once (fp16)."""
    spec = {n: (k, r, c) for n, k, r, c, _, _ in GEMVS}
    wb = {n: weight_bytes(*spec[n]) for n in spec}
    return {
        "attn_qkv": wb["attn_q"] + wb["attn_k"] + wb["attn_v"] + HIDDEN * 2 + (HEADS + 2 * KV_HEADS) * HEAD_DIM * 2,
        "attention": attention_bytes(CTX),
        "attn_o": wb["attn_o"] + HEADS * HEAD_DIM * 2 + HIDDEN * 2,
        "ffn_gate_up": wb["ffn_gate"] + wb["ffn_up"] + HIDDEN * 2 + FFN * 2,
        "ffn_down": wb["ffn_down"] + FFN * 2 + HIDDEN * 2,
    }


class Layer:
    def __init__(self, hip, host):
        self.w = {n: hip.DeviceArray.from_numpy(host[n]) for n, *_ in GEMVS}
        self.kc = hip.DeviceArray.from_numpy(host["k_cache"])
        self.vc = hip.DeviceArray.from_numpy(host["v_cache"])


def make_host_layer(hip):
    rng = hip.synth.Rng(0)
    host = {n: hip.synth.quant_matrix(k, rng, r, c) for n, k, r, c, _, _ in GEMVS}
    host["k_cache"] = hip.synth.normal_f16(rng, CTX * KV_HEADS * HEAD_DIM)
    host["v_cache"] = hip.synth.normal_f16(rng, CTX * KV_HEADS * HEAD_DIM)
    host["x"] = hip.synth.normal_f16(rng, HIDDEN)
    return host


def run_gpu(args):
    import pycitlali as hip
    lib = hip.load()
    hip.check(lib.citlali_hip_init(0))
    host = make_host_layer(hip)
    layers = [Layer(hip, host) for _ in range(LAYERS)]
    act = {"x": hip.DeviceArray.from_numpy(host["x"])}
    for name, size in (("q", HEADS * HEAD_DIM), ("k", KV_HEADS * HEAD_DIM), ("v", KV_HEADS * HEAD_DIM),
                       ("att", HEADS * HEAD_DIM), ("o", HIDDEN), ("up", FFN), ("down", HIDDEN)):
        act[name] = hip.DeviceArray(size * 2)
    scores = hip.DeviceArray(HEADS * CTX * 4)
    spec = {n: (k, r, c, i, o) for n, k, r, c, i, o in GEMVS}
    qkv = ["attn_q", "attn_k", "attn_v"]

    def launch(name, layer):
        if name == "attn_qkv":
            hip.device.matvec_group([spec[n][0] for n in qkv], [layer.w[n] for n in qkv], act["x"],
                                    [act[spec[n][4]] for n in qkv], [spec[n][1] for n in qkv], HIDDEN)
        elif name == "attention":
            hip.device.attention(act["q"], layer.kc, layer.vc, scores, act["att"], CTX - 1, CTX, HEADS, KV_HEADS,
                                 HEAD_DIM)
        elif name == "ffn_gate_up":
            # gate and up GEMVs with SwiGLU; the activation feeds ffn_down
            hip.device.matvec_gate_up_swiglu("q4k", layer.w["ffn_gate"], layer.w["ffn_up"], act["x"], act["up"],
                                             HIDDEN, FFN)
        else:
            k, r, c, i, o = spec[name]
            hip.device.matvec(k, layer.w[name], act[i], act[o], c, r)

    def step(s, timed=None):
        """One layer; `timed` maps kernel names to DispatchTimers (HIP events
        stamped by each kernel's own dispatch on the launch stream)."""
        layer = layers[s % LAYERS]
        for name in ORDER:
            if timed and name in timed:
                # the queue drained before and after: a stamped dispatch's
                # events would otherwise also count the wait for the kernel
                # before it and the launches queued behind it
                hip.synchronize()
                with timed[name]:
                    launch(name, layer)
                hip.synchronize()
            else:
                launch(name, layer)

    # warmup, and a per-kernel pass to find the kernel with the largest share
    for s in range(args.warmup):
        step(s)
    hip.synchronize()
    if args.trace_child:
        # under the parent's rocprofv3 kernel trace: the K steps, nothing else
        for s in range(args.steps):
            step(s)
        hip.synchronize()
        return None
    cal = max(8, 2 * LAYERS)
    cal_timers = [{n: hip.device.DispatchTimer() for n in ORDER} for _ in range(cal)]
    for s in range(cal):
        step(s, cal_timers[s])
    hip.synchronize()
    per = {n: sum(t[n].ms() for t in cal_timers) / cal for n in ORDER}
    dominant = max(per, key=per.get)

    # timed region: K steps, nothing armed (value, ms_per_step)
    hip.synchronize()
    t0, t1 = hip.Event(), hip.Event()
    t0.record()
    for s in range(args.steps):
        step(s)
    t1.record()
    t1.synchronize()
    hip.synchronize()
    total_ms = t0.elapsed_ms(t1)
    # the same K steps again with every launch timed, each kernel by its own
    # dispatch and each launch with the queue drained before and after it
    # (so this pass is kept out of `value`); the dominant kernel's figure
    # is the mean of its K launches
    all_timers = [{n: hip.device.DispatchTimer() for n in ORDER} for _ in range(args.steps)]
    for s in range(args.steps):
        step(s, all_timers[s])
    dom_timers = [t[dominant] for t in all_timers]
    hip.synchronize()
    dom_ms = sum(t.ms() for t in dom_timers) / args.steps

    # measured HBM read ceiling: 2 GiB streamed once per launch
    big = hip.DeviceArray(2 << 30)
    sink = hip.DeviceArray(16)
    e0, e1 = hip.Event(), hip.Event()
    hip.check(lib.citlali_hip_stream_read(big.vp, big.nbytes, sink.vp))
    e0.record()
    for _ in range(5):
        hip.check(lib.citlali_hip_stream_read(big.vp, big.nbytes, sink.vp))
    e1.record()
    e1.synchronize()
    stream_gbps = 5 * big.nbytes / (e0.elapsed_ms(e1) * 1e-3) / 1e9
    # plain copy kernel of known size (COPY_HALVES fp16 read + written): the
    # calibration launch for rocprofv3 FETCH_SIZE / WRITE_SIZE counters
    dst = hip.DeviceArray(COPY_HALVES * 2)
    hip.check(lib.citlali_hip_copy(big.vp, dst.vp, COPY_HALVES))
    e0.record()
    hip.check(lib.citlali_hip_copy(big.vp, dst.vp, COPY_HALVES))
    e1.record()
    e1.synchronize()
    copy_gbps = 2 * COPY_HALVES * 2 / (e0.elapsed_ms(e1) * 1e-3) / 1e9
    dst.close()
    big.close()
    return total_ms, dominant, dom_ms, per, (stream_gbps, copy_gbps), host


ROTATE_BYTES = 512 << 20   # configs 1 and 2 cycle through this much of independent copies


def _rotated_copies(hip, host_bytes, unit_bytes):
    """ceil(ROTATE_BYTES / unit_bytes) device copies of `host_bytes` (uint8)
    in one allocation, each slot 256-byte aligned; returns (buffer, slot, n)."""
    slot = -(-unit_bytes // 256) * 256
    n = -(-ROTATE_BYTES // unit_bytes)
    buf = hip.DeviceArray(slot * n)
    buf.upload(host_bytes, 0)
    for i in range(1, n):
        hip.check(hip.load().citlali_hip_memcpy_d2d(buf.at(i * slot), buf.vp, host_bytes.nbytes))
    return buf, slot, n


CONFIG_REPS = 10   # timed passes over the rotated copies, configs 1 and 2


def _time_rotated(hip, launch, n, reps, stamped=True):
    """Mean launch time (us) over reps passes of n back-to-back launches
    (launch(i) uses copy i): HIP events around all of them, and the kernels'
    own dispatch-stamped time (each kernel's duration, added per launch) of
    one more pass (stamped=False: that pass is left out, for the rocprofv3
    child, whose trace then holds one untimed pass and the reps timed
    ones)."""
    for i in range(n):
        launch(i)
    e0, e1 = hip.Event(), hip.Event()
    e0.record()
    for _ in range(reps):
        for i in range(n):
            launch(i)
    e1.record()
    e1.synchronize()
    wall_us = e0.elapsed_ms(e1) / (reps * n) * 1e3
    if not stamped:
        return wall_us, None
    # each kernel stamped by its own dispatch, the queue drained around each
    # launch (as in the step's roofline pass)
    timers = [hip.device.DispatchTimer() for _ in range(n)]
    for i in range(n):
        hip.synchronize()
        with timers[i]:
            launch(i)
        hip.synchronize()
    kern_us = sum(t.ms() for t in timers) / n * 1e3
    return wall_us, kern_us


def matvec_cfg1(stamped=True):
    """Q4_K GEMV of a 3072 x 1024 matrix (4 super-blocks
    per row, seed 0), x N(0,1) fp16, y fp32 (citlali_hip_matvec_q4k_to_float);
    also the same bytes read as 1024 rows of 12 super-blocks (K = 3072).
    Rotated over >= 512 MB of copies so the weights come from HBM."""
    import pycitlali as hip
    rng = hip.synth.Rng(0)
    w = hip.synth.quant_matrix("q4k", rng, 3072, 1024)
    x = hip.synth.normal_f16(rng, 3072)
    buf, slot, n = _rotated_copies(hip, w, w.nbytes)
    dx = hip.DeviceArray.from_numpy(x)
    dy = hip.DeviceArray(3072 * 4)
    out = {}
    for name, rows, cols in (("3072x1024", 3072, 1024), ("1024x3072", 1024, 3072)):
        wall, kern = _time_rotated(hip, lambda i: hip.device.matvec("q4k", buf.at(i * slot), dx, dy, cols, rows,
                                                                   f32_out=True), n, CONFIG_REPS, stamped)
        alg = w.nbytes + cols * 2 + rows * 4
        out[name] = {"bytes_per_launch": alg, "copies_rotated": n, "us_per_launch": round(wall, 3),
                     "GBps": round(alg / (wall * 1e-6) / 1e9, 1), "frac_of_8TBps": round(alg / (wall * 1e-6) / 8e12, 4)}
        if kern is not None:
            out[name].update({"kernel_us_stamped": round(kern, 3),
                              "kernel_GBps_stamped": round(alg / (kern * 1e-6) / 1e9, 1)})
    for a in (buf, dx, dy):
        a.close()
    return {"workload": "BASELINE config 1: Q4_K GEMV 3072 rows x 1024 cols (4 super-blocks/row), fp32 y; "
                        "also read as 1024 x 3072 (12 super-blocks/row)", **out}


def attention_cfg2(stamped=True):
    """Qwen3-0.6B decode attention, 16 query / 8 kv heads,
    head_dim 128, 1024 cached positions (position 1023), q/K/V N(0,1) fp16
    (seed 0), fp16 output; rotated over >= 512 MB of K/V copies."""
    import pycitlali as hip
    heads, kv, hd, L = 16, 8, 128, 1024
    rng = hip.synth.Rng(0)
    q = hip.synth.normal_f16(rng, heads * hd)
    k = hip.synth.normal_f16(rng, L * kv * hd)
    v = hip.synth.normal_f16(rng, L * kv * hd)
    kv_bytes = k.nbytes
    kb, slot, n = _rotated_copies(hip, np.concatenate([k, v]).view(np.uint8), 2 * kv_bytes)   # slot: K then V
    dq = hip.DeviceArray.from_numpy(q)
    scores = hip.DeviceArray(heads * L * 4)
    do = hip.DeviceArray(heads * hd * 2)
    wall, kern = _time_rotated(hip, lambda i: hip.device.attention(dq, kb.at(i * slot), kb.at(i * slot + kv_bytes),
                                                                  scores, do, L - 1, L, heads, kv, hd), n, CONFIG_REPS,
                               stamped)
    alg = 2 * kv_bytes + 2 * heads * hd * 2
    for a in (kb, dq, scores, do):
        a.close()
    out = {"workload": "BASELINE config 2: Qwen3-0.6B decode attention, 16/8 heads, head_dim 128, L=1024",
           "bytes_per_launch": alg, "copies_rotated": n, "us_per_launch": round(wall, 3),
           "GBps": round(alg / (wall * 1e-6) / 1e9, 1), "frac_of_8TBps": round(alg / (wall * 1e-6) / 8e12, 4)}
    if kern is not None:
        out.update({"kernel_us_stamped": round(kern, 3), "kernel_GBps_stamped": round(alg / (kern * 1e-6) / 1e9, 1)})
    return out


def attention_cfg4():
    """BASELINE config 4 beside the headline: 16 independent sequences at the
    Qwen3-8B head shape (32 / 8 heads, head_dim 128) in one batched attention
    launch, KV lengths uniform in [4096, 32768] from seed 4, caches of
    ~2.1 GB (far beyond the Infinity Cache).  GB/s = K and V bytes read per
    launch (sum of the lengths x 8 kv heads x 128 x 2 B x 2) over the mean
    launch time of 20 launches (HIP events, split + merge)."""
    import pycitlali as hip
    nseq, max_len = 16, 32768
    rng = np.random.default_rng(4)
    lens = rng.integers(4096, max_len + 1, nseq)
    stride = max_len * KV_HEADS * HEAD_DIM
    kc, vc = hip.DeviceArray(nseq * stride * 2), hip.DeviceArray(nseq * stride * 2)
    block = rng.standard_normal(32 << 20, dtype=np.float32).astype(np.float16)   # 64 MB, tiled
    for buf in (kc, vc):
        for off in range(0, buf.nbytes, block.nbytes):
            n = min(block.nbytes, buf.nbytes - off)
            buf.upload(block[: n // 2], off)
    q = hip.DeviceArray.from_numpy(rng.standard_normal(nseq * HEADS * HEAD_DIM).astype(np.float16))
    pos = hip.DeviceArray.from_numpy((lens - 1).astype(np.int32))
    ws_bytes = hip.device.attention_workspace_bytes(max_len, nseq, HEADS, KV_HEADS, HEAD_DIM)
    ws = hip.DeviceArray(max(ws_bytes, 16))
    out = hip.DeviceArray(nseq * HEADS * HEAD_DIM * 2)

    def launch():
        hip.device.attention_batched(q, kc, vc, stride, pos, max_len, nseq, HEADS, KV_HEADS, HEAD_DIM, ws, ws_bytes,
                                     out)
    for _ in range(3):
        launch()
    reps = 20
    e0, e1 = hip.Event(), hip.Event()
    e0.record()
    for _ in range(reps):
        launch()
    e1.record()
    e1.synchronize()
    us = e0.elapsed_ms(e1) / reps * 1e3
    kv_bytes = int(lens.sum()) * KV_HEADS * HEAD_DIM * 2 * 2
    for a in (kc, vc, q, pos, ws, out):
        a.close()
    return {"workload": "BASELINE config 4: 16 sequences, 32/8 heads, head_dim 128, KV lengths uniform in "
                        "[4096, 32768] (seed 4), one batched launch",
            "positions": int(lens.sum()), "kv_bytes": kv_bytes, "us_per_launch": round(us, 2),
            "GBps": round(kv_bytes / (us * 1e-6) / 1e9, 1), "frac_of_8TBps": round(kv_bytes / (us * 1e-6) / 8e12, 4)}


def cpu_baseline(host, budget_s):
    """BASELINE's CPU path on this machine's host cores, in the same run: the
    reference's own host dequant (weight_loader.cpp:147-323, compiled from
    its sources into oracle/_ref by oracle/Makefile; the oracle's pinned
    restatement of it where that build is absent) of each weight row to fp16,
    then an fp32 dot -- variant (i), per call, the CPU analogue of the fused
    GPU kernel -- or the fp32 dot over rows dequantised beforehand (variant
    (ii)); attention in fp32 (the oracle's, kernels.cu:545-649's arithmetic:
    the reference has no CPU attention).  Every config at 1 thread and at
    all cores, on bounded samples (each said in `sample`), ~budget_s per
    measurement.  Returns (headline, entries): the headline is config 3,
    variant (i), all cores."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle_binding import Oracle, RefLib
    import pycitlali as hip
    orc = Oracle()
    ref = RefLib.try_load()
    cores = int(orc.lib.orc_num_threads())
    kind = "reference" if ref else "port"
    code = ("reference dequant (oracle/_ref) + fp32 dot" if ref else
            "oracle restatement of the reference dequant + fp32 dot")

    def mv_i(k, w, x, cin, rows, th):
        if ref:
            return ref.matvec_dequant_dot(k, w, x, cin, rows, th)
        return orc.matvec_f16dot(k, w, x, cin, rows, th)

    def mv_ii(wf16, x, cin, rows, th):
        if ref:
            return ref.matvec_f16_dot(wf16, x, cin, rows, th)
        y = np.empty(rows, np.float32)
        orc.lib.orc_matvec_f16(wf16.ctypes.data, x.ctypes.data, y.ctypes.data, cin, rows, th)
        return y

    def dequant(k, w, count):
        if ref:
            return ref.dequant(k, w, count)
        out = np.empty(count, np.uint16)
        getattr(orc.lib, f"orc_dequant_{k}_f16")(w.ctypes.data, count, out.ctypes.data)
        return out

    def rate(fn, budget):
        """calls per second: at least one call, then until `budget` seconds"""
        n, t0 = 0, time.perf_counter()
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if el >= budget:
                return n / el, n, el

    entries = []

    def add(config, variant, th, value, unit, sample):
        entries.append({"config": config, "variant": variant, "threads": th, "value": round(value, 4),
                        "unit": unit, "kind": kind, "sample": sample})

    spec = {n: (k, r, c, i) for n, k, r, c, i, _ in GEMVS}
    x = host["x"]
    ins = {"x": x, "att": np.ascontiguousarray(x[: HEADS * HEAD_DIM]), "up": np.ascontiguousarray(np.resize(x, FFN))}
    f16 = {n: dequant(k, host[n], r * c) for n, (k, r, c, _) in spec.items()}
    kb = kernel_bytes()
    layer_bytes = sum(kb.values())

    # config 1: Q4_K 3072 x 1024, fp32 y
    rng = hip.synth.Rng(0)
    w1 = hip.synth.quant_matrix("q4k", rng, 3072, 1024)
    x1 = hip.synth.normal_f16(rng, 1024)
    w1f = dequant("q4k", w1, 3072 * 1024)
    b1 = w1.nbytes + 1024 * 2 + 3072 * 4
    for th in (1, cores):
        r, n, el = rate(lambda: mv_i("q4k", w1, x1, 1024, 3072, th), budget_s)
        add(1, "i", th, b1 * r / 1e9, "GB/s", f"{n} calls in {el:.1f} s ({code}; {1e6 / r:.0f} us/call)")
        r, n, el = rate(lambda: mv_ii(w1f, x1, 1024, 3072, th), budget_s)
        add(1, "ii", th, b1 * r / 1e9, "GB/s", f"{n} calls in {el:.1f} s (fp32 dot over pre-dequantised fp16; "
                                                f"{1e6 / r:.0f} us/call)")

    # config 2: attention 16/8/128 at L = 1024
    rng = hip.synth.Rng(0)
    q2 = hip.synth.normal_f16(rng, 16 * 128)
    k2 = hip.synth.normal_f16(rng, 1024 * 8 * 128)
    v2 = hip.synth.normal_f16(rng, 1024 * 8 * 128)
    b2 = 2 * k2.nbytes + 2 * 16 * 128 * 2
    for th in (1, cores):
        r, n, el = rate(lambda: orc.attention_f32(q2, k2, v2, 1023, 16, 8, 128, th), budget_s)
        add(2, "fp32", th, b2 * r / 1e9, "GB/s", f"{n} calls in {el:.1f} s ({1e6 / r:.0f} us/call)")

    # config 3: one Qwen3-8B layer step (7 GEMVs + attention at L = 8192)
    q = ins["att"]

    def layer_step(th, variant, L=CTX):
        for n, (k, r, c, i) in spec.items():
            if variant == "i":
                mv_i(k, host[n], ins[i], c, r, th)
            else:
                mv_ii(f16[n], ins[i], c, r, th)
        orc.attention_f32(q, host["k_cache"], host["v_cache"], L - 1, HEADS, KV_HEADS, HEAD_DIM, th)

    headline = None
    for th in (1, cores):
        for variant in ("i", "ii"):
            r, n, el = rate(lambda: layer_step(th, variant), budget_s)
            add(3, variant, th, layer_bytes * r / 1e9, "GB/s",
                f"{n} full Qwen3-8B layer step(s) (7 GEMVs, "
                f"{code if variant == 'i' else 'fp32 dot over pre-dequantised fp16'}; fp32 attention at "
                f"L={CTX}) in {el:.1f} s")
            if th == cores and variant == "i":
                headline = dict(entries[-1])

    # config 4: 16 sequences, lengths from default_rng(4) in [4096, 32768]:
    # timed on the first sequences of the set, scaled per K/V byte
    lens = np.random.default_rng(4).integers(4096, 32768 + 1, 16)
    gen = np.random.default_rng(44)
    kv_s = [gen.standard_normal(int(L) * KV_HEADS * HEAD_DIM, dtype=np.float32).astype(np.float16).view(np.uint16)
            for L in lens[:2]]
    vv_s = [gen.standard_normal(int(L) * KV_HEADS * HEAD_DIM, dtype=np.float32).astype(np.float16).view(np.uint16)
            for L in lens[:2]]
    q4 = gen.standard_normal(HEADS * HEAD_DIM, dtype=np.float32).astype(np.float16).view(np.uint16)
    for th, nseq in ((1, 1), (cores, 2)):
        def seqs():
            for j in range(nseq):
                orc.attention_f32(q4, kv_s[j], vv_s[j], int(lens[j]) - 1, HEADS, KV_HEADS, HEAD_DIM, th)
        r, n, el = rate(seqs, budget_s)
        bytes_ = int(sum(lens[:nseq])) * KV_HEADS * HEAD_DIM * 4
        add(4, "fp32", th, bytes_ * r / 1e9, "GB/s",
            f"sequence(s) 0..{nseq - 1} of the 16 (L={','.join(str(int(v)) for v in lens[:nseq])}), "
            f"{n} pass(es) in {el:.1f} s; the full set is {int(lens.sum())} positions")

    # config 5: tok/s of the whole decode = 36 layer steps (attention at the
    # mean decode length 640) + the Q6_K output GEMV (151936 x 4096), from one
    # layer step and 1/16 of the output rows
    rows_part = 151936 // 16
    wo = hip.synth.quant_matrix("q6k", hip.synth.Rng(5), rows_part, HIDDEN)
    for th in (1, cores):
        t_layer = 1.0 / rate(lambda: layer_step(th, "i", L=640), budget_s / 2)[0]
        t_out = 1.0 / rate(lambda: mv_i("q6k", wo, x, HIDDEN, rows_part, th), budget_s / 2)[0]
        tok_s = 1.0 / (36 * t_layer + 16 * t_out)
        add(5, "i", th, tok_s, "tok/s", f"1 layer step at L=640 ({t_layer * 1e3:.0f} ms) x 36 + 1/16 of the output "
                                        f"GEMV rows ({t_out * 1e3:.0f} ms) x 16 ({code})")
    cpu = {"value": headline["value"], "unit": headline["unit"], "cores": cores, "kind": kind,
           "sample": headline["sample"]}
    return cpu, entries


PMC_SUMMARY = os.path.join(ROOT, "profiles", "cfg3_layer_hbm_traffic_pmc.md")


DECODE_BIN = os.path.join(ROOT, "citlali-llm-engine_amd", "bin", "decode_qwen3")


def decode_cfg5(fp16=False):
    """BASELINE config 5 beside the headline: the synthetic Qwen3-8B greedy
    decode through QwenModel (bin/decode_qwen3, a child process; every one of
    the 36 layers has its own weights), loaded from a GGUF file of its
    weights (written to /dev/shm or the temp directory, removed after
    loading), 512-token prompt then 256 greedy steps; decode tok/s.  fp16:
    loaded with DequantizeToFp16, 64-token prompt then 128 steps."""
    import subprocess
    import tempfile
    if not os.path.exists(DECODE_BIN):
        return {"error": "citlali-llm-engine_amd/bin/decode_qwen3 is not built"}
    import shutil
    # ~5.4 GB with every layer's own weights: a RAM-backed directory when it
    # has room (the load then reads page-cache pages), else the temp directory
    base = tempfile.gettempdir()
    if os.path.isdir("/dev/shm") and shutil.disk_usage("/dev/shm").free > (12 << 30):
        base = "/dev/shm"
    path = os.path.join(base, f"citlali_cfg5_{os.getpid()}.gguf")
    cmd = [DECODE_BIN, "--gguf", path] + (["--fp16", "--prompt", "64", "--steps", "128"] if fp16 else [])
    try:
        p = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    finally:
        if os.path.exists(path):
            os.remove(path)
    if p.returncode != 0:
        return {"error": (p.stderr or p.stdout)[-300:]}
    return json.loads(p.stdout.strip().splitlines()[-1])


# the dispatches of one step, in launch order, and the step op each belongs to
STEP_DISPATCHES = [("matvec_group_kernel", "attn_qkv"), ("attn_mfma_kernel", "attention"),
                   ("attn_merge_kernel", "attention"), ("matvec_stream_kernel", "attn_o"),
                   ("matvec_gate_up_kernel", "ffn_gate_up"), ("matvec_stream_kernel", "ffn_down")]


def _rocprof_rows(child_args):
    """This script with `child_args` in a child process under `rocprofv3
    --kernel-trace`: (the trace's dispatches sorted by start, the child's
    stdout); (None, None) without rocprofv3, ({"error": ...}, None) when the
    run or its trace is unusable."""
    import csv
    import glob
    import shutil
    import subprocess
    import tempfile
    exe = shutil.which("rocprofv3")
    if exe is None:
        return None, None
    with tempfile.TemporaryDirectory(dir="/tmp" if os.path.isdir("/tmp") else None) as d:
        cmd = [exe, "--kernel-trace", "--output-format", "csv", "-d", d, "-o", "trace", "--", sys.executable,
               os.path.abspath(__file__), *child_args]
        env = dict(os.environ, TMPDIR=d)
        try:
            p = subprocess.run(cmd, capture_output=True, text=True, timeout=300, cwd=d, env=env)
        except subprocess.TimeoutExpired:
            return {"error": "rocprofv3 pass timed out"}, None
        files = glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True)
        if not files:
            return {"error": f"no kernel trace (rocprofv3 exit {p.returncode}): {(p.stderr or p.stdout)[-200:]}"}, None
        rows = []
        for f in files:
            rows += list(csv.DictReader(open(f)))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    return rows, p.stdout


def _dur_us(r):
    return (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3


def rocprof_config_kernels():
    """Kernel durations of configs 1 and 2 as rocprofv3 measures them: the
    same rotated launches (one untimed pass, CONFIG_REPS timed passes, no
    dispatch-stamped pass) run by this script in --trace-configs mode under
    `rocprofv3 --kernel-trace`.  Config 1: the mean duration of the GEMV
    dispatches of the timed passes, per shape; config 2: the mean split and
    merge durations and their sum per launch.  {} without rocprofv3."""
    rows, out = _rocprof_rows(["--trace-configs"])
    if rows is None:
        return {}
    if isinstance(rows, dict):
        return {"error": rows["error"]}
    try:
        copies = json.loads([ln for ln in out.splitlines() if ln.startswith("{")][-1])
    except (IndexError, ValueError):
        return {"error": "the --trace-configs child printed no launch counts"}
    res = {}
    mv = [r for r in rows if "matvec" in r["Kernel_Name"]]
    shapes = list(copies["cfg1"].items())
    if len(mv) != sum(n * (1 + CONFIG_REPS) for _, n in shapes):
        return {"error": f"{len(mv)} GEMV dispatches traced for config 1"}
    at = 0
    for name, n in shapes:
        timed = mv[at + n: at + n * (1 + CONFIG_REPS)]
        at += n * (1 + CONFIG_REPS)
        res[name] = round(sum(_dur_us(r) for r in timed) / len(timed), 3)
    n2 = copies["cfg2"] * CONFIG_REPS
    split = [r for r in rows if "attn_" in r["Kernel_Name"] and "merge" not in r["Kernel_Name"]][-n2:]
    merge = [r for r in rows if "attn_merge" in r["Kernel_Name"]][-n2:]
    if len(split) != n2 or len(merge) not in (0, n2):
        return {"error": f"{len(split)} split / {len(merge)} merge dispatches traced for config 2, {n2} timed"}
    s_us = sum(_dur_us(r) for r in split) / n2
    m_us = sum(_dur_us(r) for r in merge) / n2 if merge else 0.0
    res["cfg2"] = {"split_us": round(s_us, 3), "merge_us": round(m_us, 3), "kernel_us": round(s_us + m_us, 3)}
    return res


def rocprof_step_kernels(args):
    """Kernel durations of the config-3 step as rocprofv3 measures them:
    this script in --trace-child mode (the same warmup and K steps, nothing
    else) under `rocprofv3 --kernel-trace`, a child process.  The last 6 K
    dispatches of the trace are the K steps (q/k/v, attention split,
    attention merge, attn_o, gate/up, ffn_down); per op, the mean of its
    kernels' end - start over the K steps (attention: split + merge, the gap
    between them excluded).  These are the figures the committed rocprofv3
    summaries report; the event-stamped kernels_us include each dispatch's
    event overhead.  None when rocprofv3 is absent, an error entry when its
    trace is unusable."""
    rows, _ = _rocprof_rows(["--trace-child", "--steps", str(args.steps), "--warmup", str(args.warmup)])
    if rows is None or isinstance(rows, dict):
        return rows
    n = len(STEP_DISPATCHES) * args.steps
    if len(rows) < n:
        return {"error": f"{len(rows)} dispatches traced, {n} expected"}
    rows = rows[-n:]
    sums = {op: 0.0 for op in ORDER}
    split = merge = 0.0
    for i, r in enumerate(rows):
        want, op = STEP_DISPATCHES[i % len(STEP_DISPATCHES)]
        if want not in r["Kernel_Name"]:
            return {"error": f"dispatch {i} of the timed steps is {r['Kernel_Name'][:80]}, expected {want}"}
        us = _dur_us(r)
        sums[op] += us
        if want == "attn_mfma_kernel":
            split += us
        elif want == "attn_merge_kernel":
            merge += us
    k = args.steps
    return {"kernels_us": {op: round(v / k, 3) for op, v in sums.items()},
            "attention_split_us": round(split / k, 3), "attention_merge_us": round(merge / k, 3),
            "step_kernel_us": round(sum(sums.values()) / k, 3)}


def read_traffic(kernel):
    """HBM bytes per launch of `kernel` (a step-kernel name) from the
    committed rocprofv3 PMC summary: the line 'traffic_bytes_per_launch
    <kernel>: N' (FETCH_SIZE + WRITE_SIZE, scaled by the copy calibration)."""
    if not os.path.exists(PMC_SUMMARY):
        return None
    key = f"traffic_bytes_per_launch {kernel}:"
    for line in open(PMC_SUMMARY):
        if line.startswith(key):
            return int(float(line.split(":", 1)[1]))
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=2.0, help="per CPU-baseline measurement")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true", help="skip the config-5 whole-model decode run")
    ap.add_argument("--no-rocprof", action="store_true", help="skip the rocprofv3 kernel-trace pass")
    ap.add_argument("--trace-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--trace-configs", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the decode hot path here is a single-GPU build "
              "(multi-GPU sharding is a design note, not a measured mode)", file=sys.stderr)
        sys.exit(2)

    if args.trace_child:
        run_gpu(args)
        return
    if args.trace_configs:
        # under the parent's rocprofv3 kernel trace: configs 1 and 2, unstamped
        c1, c2 = matvec_cfg1(stamped=False), attention_cfg2(stamped=False)
        print(json.dumps({"cfg1": {k: v["copies_rotated"] for k, v in c1.items() if isinstance(v, dict)},
                          "cfg2": c2["copies_rotated"]}), flush=True)
        return
    total_ms, dominant, dom_ms, per, (stream_gbps, copy_gbps), host = run_gpu(args)
    kb = kernel_bytes()
    step_bytes = sum(kb.values())
    ms_step = total_ms / args.steps
    value = step_bytes / (ms_step * 1e-3) / 1e9
    achieved = kb[dominant] / (dom_ms * 1e-3) / 1e9
    line = {
        "metric": "achieved HBM GB/s (decode attn, Q4_K/Q6_K matvec); Qwen3-8B decode tok/s",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "BASELINE config 3: Qwen3-8B one-layer decode (7 Q4_K/Q6_K fused-dequant GEMVs in "
                               "4 launches -- q/k/v grouped, gate/up with SwiGLU -- + 32/8-head attention, "
                               "head_dim 128, L=8192)",
                   "layers_rotated": LAYERS, "bytes_per_step": step_bytes,
                   "layer_tok_per_s_equiv": round(1000.0 / ms_step, 1)},
        "roofline": {"bound": "hbm", "kernel": dominant, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "bytes_per_launch": kb[dominant], "us_per_launch": round(dom_ms * 1e3, 3),
                     "traffic": read_traffic(dominant)},
        "kernels_us": {n: round(per[n] * 1e3, 2) for n in ORDER},
        "kernels_GBps": {n: round(kb[n] / (per[n] * 1e-3) / 1e9, 1) for n in ORDER},
        "stream_read_GBps": round(stream_gbps, 1),
        "copy_GBps": round(copy_gbps, 1),
        "cpu_baseline": None,
    }
    rp = None if args.no_rocprof else rocprof_step_kernels(args)
    if rp and "kernels_us" in rp:
        ku = rp["kernels_us"]
        rp["kernels_GBps"] = {n: round(kb[n] / (ku[n] * 1e-6) / 1e9, 1) for n in ORDER}
        a = kb[dominant] / (ku[dominant] * 1e-6) / 1e9
        line["roofline"]["rocprof"] = {"us_per_launch": ku[dominant], "achieved": round(a, 1),
                                       "frac": round(a / HBM_PEAK_GBPS, 4)}
    line["rocprof_step"] = rp
    line["matvec_cfg1"] = matvec_cfg1()
    line["attention_cfg2"] = attention_cfg2()
    rc = {} if args.no_rocprof else rocprof_config_kernels()
    if "error" in rc:
        line["matvec_cfg1"]["rocprof"] = line["attention_cfg2"]["rocprof"] = rc
    for shape, us in rc.items():
        if shape in line["matvec_cfg1"]:
            c = line["matvec_cfg1"][shape]
            c.update({"kernel_us": us, "kernel_GBps": round(c["bytes_per_launch"] / (us * 1e-6) / 1e9, 1)})
    if "cfg2" in rc:
        c = line["attention_cfg2"]
        c.update({"kernel_us": rc["cfg2"]["kernel_us"], "split_us": rc["cfg2"]["split_us"],
                  "merge_us": rc["cfg2"]["merge_us"],
                  "kernel_GBps": round(c["bytes_per_launch"] / (rc["cfg2"]["kernel_us"] * 1e-6) / 1e9, 1)})
    line["attention_cfg4"] = attention_cfg4()
    if not args.no_cpu:
        line["cpu_baseline"], line["cpu_baseline_configs"] = cpu_baseline(host, args.cpu_seconds)
    line["decode_cfg5"] = None if args.no_decode else decode_cfg5()
    line["decode_cfg5_fp16"] = None if args.no_decode else decode_cfg5(fp16=True)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
