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
steps, from HIP events that the kernel's own dispatches stamp
(hipExtLaunchKernel; for attention, split start to merge end).  cpu_baseline: the
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
        """One layer; `timed` maps kernel names to KernelTimers (HIP events
        stamped by the kernels' own dispatches on the launch stream)."""
        layer = layers[s % LAYERS]
        for name in ORDER:
            if timed and name in timed:
                with timed[name]:
                    launch(name, layer)
            else:
                launch(name, layer)

    # warmup, and a per-kernel pass to find the kernel with the largest share
    for s in range(args.warmup):
        step(s)
    hip.synchronize()
    cal = max(8, 2 * LAYERS)
    cal_timers = [{n: hip.device.KernelTimer() for n in ORDER} for _ in range(cal)]
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
    # the same K steps again with the dominant kernel's launches timed (a
    # dispatch that stamps events is scheduled slightly differently, so this
    # pass is kept out of `value`)
    dom_timers = [hip.device.KernelTimer() for _ in range(args.steps)]
    for s in range(args.steps):
        step(s, {dominant: dom_timers[s]})
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
    """The oracle (restated reference arithmetic) on the host cores: one
    layer step -- every GEMV as repo dequant to fp16 + fp32 dot, attention in
    fp32 -- repeated until ~budget_s seconds have passed."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle_binding import Oracle
    orc = Oracle()
    threads = int(orc.lib.orc_num_threads())
    x = host["x"]
    q = np.ascontiguousarray(host["x"][: HEADS * HEAD_DIM])
    up = np.ascontiguousarray(np.resize(host["x"], FFN))
    ins = {"x": x, "att": q, "up": up}
    runs, t_start = 0, time.perf_counter()
    while True:
        for n, k, r, c, i, _ in GEMVS:
            orc.matvec_f16dot(k, host[n], ins[i], c, r, threads)
        orc.attention_f32(q, host["k_cache"], host["v_cache"], CTX - 1, HEADS, KV_HEADS, HEAD_DIM, threads)
        runs += 1
        el = time.perf_counter() - t_start
        if el >= budget_s:
            break
    step_bytes = sum(kernel_bytes().values())
    return {"value": round(step_bytes * runs / el / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{runs} full Qwen3-8B layer step(s) (7 GEMVs dequant->fp16->fp32 dot + fp32 attention "
                      f"at L={CTX}) in {el:.1f} s"}


PMC_SUMMARY = os.path.join(ROOT, "profiles", "cfg3_layer_hbm_traffic_pmc.md")


DECODE_BIN = os.path.join(ROOT, "citlali-llm-engine_amd", "bin", "decode_qwen3")


def decode_cfg5(fp16=False):
    """BASELINE config 5 beside the headline: the synthetic Qwen3-8B greedy
    decode through QwenModel (bin/decode_qwen3, a child process), loaded from
    a GGUF file of its weights (written to the temp directory, removed after
    loading), 512-token prompt then 256 greedy steps; decode tok/s.  fp16:
    loaded with DequantizeToFp16, 64-token prompt then 128 steps."""
    import subprocess
    import tempfile
    if not os.path.exists(DECODE_BIN):
        return {"error": "citlali-llm-engine_amd/bin/decode_qwen3 is not built"}
    path = os.path.join(tempfile.gettempdir(), f"citlali_cfg5_{os.getpid()}.gguf")
    cmd = [DECODE_BIN, "--gguf", path] + (["--fp16", "--prompt", "64", "--steps", "128"] if fp16 else [])
    try:
        p = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    finally:
        if os.path.exists(path):
            os.remove(path)
    if p.returncode != 0:
        return {"error": (p.stderr or p.stdout)[-300:]}
    return json.loads(p.stdout.strip().splitlines()[-1])


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
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true", help="skip the config-5 whole-model decode run")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the decode hot path here is a single-GPU build "
              "(multi-GPU sharding is a design note, not a measured mode)", file=sys.stderr)
        sys.exit(2)

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
    line["attention_cfg4"] = attention_cfg4()
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(host, args.cpu_seconds)
    line["decode_cfg5"] = None if args.no_decode else decode_cfg5()
    line["decode_cfg5_fp16"] = None if args.no_decode else decode_cfg5(fp16=True)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
