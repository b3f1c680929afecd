"""Benchmark of the MI355X read path: step 0 of one sparse layer at the headline shape.

Workload: packed int4 k4v4 cache, prefix 32768 tokens, batch
1, 28 query / 4 KV heads, head_dim 128, mask block of 32 queries (all 32 are selection
rows), read budget 2048 per KV head.  One step = split-K attention over [prefix | block]
with prefix statistics, the value-aware score pass, the read-set top-k and the gather of
the selected K/V into the compact bf16 buffer -- everything step 0 of the reference's
fast path does for a sparse layer (session.py:1403-1454).  Inputs are synthetic (seeded
N(0,1), LogNormal key channels, 4 sink keys x8) and resident in HBM before timing.

The step is captured once in a HIP graph and replayed; the dominant kernel (split-K
pass 1) is also timed alone from its own graph.  Prints ONE JSON line.

    python bench.py [--steps K] [--warmup W] [--split-tokens S] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--split-tokens", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-reps", type=int, default=3)
    ap.add_argument("--eager", action="store_true", help="also time the step without the HIP graph")
    return ap.parse_args()


def algorithmic(sh):
    """Bytes and flops of one step 0 of config 2 (formulas of the benchmark definition)."""
    n, h, d, k = sh.n, sh.hkv, sh.d, sh.read_k
    r = (sh.hq // sh.hkv) * sh.t
    bkv = 64 + 16                      # int4 codes + f16 scale/zero per token per K or V
    pass1 = n * 2 * bkv * h
    pass2 = n * 2 * bkv * h            # value-aware: K and V again
    scores = n * h * 4 + k * h * 8
    gather = k * h * 2 * bkv + k * h * 2 * d * 2
    flops1 = 4 * r * n * d * h
    flops2 = 2 * r * n * d * h
    return dict(bytes=pass1 + pass2 + scores + gather, flops=flops1 + flops2, pass1_bytes=pass1, pass1_flops=flops1)


def time_graph(fn, steps, warmup):
    """Capture fn() in a HIP graph, then replay it `warmup` times untimed and `steps`
    times between two events, all on the current stream (the replay stream).  Every
    kernel launched by fn uses torch's current stream, which is the capture stream
    during capture.  Returns ms per replay."""
    side = torch.cuda.Stream()                 # default priority
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()                                   # allocate / load the kernels outside capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    cur = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(cur)
    for _ in range(steps):
        g.replay()
    e1.record(cur)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps, g


def cpu_baseline(sh, q, kd, vd, kc, vc, reps):
    """The reference's CPU torch path for the same step (oracle restatement, float32)."""
    from oracle import attention as OA

    torch.set_num_threads(os.cpu_count() or 1)
    args = (q.float(), kd.float(), vd.float(), kc.float(), vc.float())
    t0 = time.perf_counter()
    OA.reference_cpu_step(*args, query_indices=range(sh.t), topk=sh.read_k)        # warm-up
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        OA.reference_cpu_step(*args, query_indices=range(sh.t), topk=sh.read_k)
        times.append(time.perf_counter() - t0)
    return statistics.median(times), torch.get_num_threads()


def main():
    a = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: the read/keep path shards per (sequence, KV head) with no "
              "exchange and this build has no multi-GPU leg; run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)

    from maskahead_amd import _native as N
    from maskahead_amd.kernels import (gather_packed_kv, prefix_scores, quantize_key_groups_into,
                                       quantize_values_into, splitk_attention, topk_ascending)
    from maskahead_amd.kernels.splitk import Prefix
    from maskahead_amd.workloads import CONFIGS, layer_inputs, packed_layout

    sh = CONFIGS["c2"]
    dev = torch.device("cuda:0")
    q, k, v, kc, vc = layer_inputs(sh, dtype=torch.bfloat16)
    lay = packed_layout(sh.b, sh.hkv, sh.n, sh.d, device=dev)
    quantize_key_groups_into(k.to(dev), lay["kq"], lay["ks"], lay["kz"], bits=4, token_group=32)
    quantize_values_into(v.to(dev), lay["vq"], lay["vs"], lay["vz"], bits=4, channel_group=32)
    prefix = Prefix(kq=lay["kq"], ks=lay["ks"], kz=lay["kz"], vq=lay["vq"], vs=lay["vs"], vz=lay["vz"],
                    nq=sh.n, kb=4, vb=4)
    qg, kcg, vcg = q.to(dev), kc.to(dev), vc.to(dev)
    rows = torch.arange(sh.t, dtype=torch.int32, device=dev)
    compact_k = torch.empty((sh.b, sh.hkv, sh.read_k + sh.t, sh.d), dtype=torch.bfloat16, device=dev)
    compact_v = torch.empty_like(compact_k)

    class View:
        k_bits = v_bits = 4
        length = quantized_length = sh.n
        residual_length = 0
        key_token_group = value_channel_group = 32
        k_q, k_scale, k_zero = lay["kq"], lay["ks"], lay["kz"]
        v_q, v_scale, v_zero = lay["vq"], lay["vs"], lay["vz"]
        k_fp = v_fp = k_residual = v_residual = None
        head_dim = sh.d
        key_mode = "channel"

    view = View()
    result = {}

    def step():
        out, stats = splitk_attention(qg, prefix, kcg, vcg, want_prefix=True, split_tokens=a.split_tokens)
        mass, score = prefix_scores(qg, prefix, stats, rows, value=True)
        idx = topk_ascending(score, sh.read_k)
        gather_packed_kv(view, idx, out_key=compact_k[:, :, :sh.read_k], out_value=compact_v[:, :, :sh.read_k])
        result["out"], result["idx"] = out, idx

    ms_step, _ = time_graph(step, a.steps, a.warmup)

    # the dominant kernel alone: split-K pass 1 (same arguments, its own graph)
    lib = N.load()
    hq, t, d, hkv = sh.hq, sh.t, sh.d, sh.hkv
    ws_bytes = int(lib.ma_splitk_workspace_bytes(sh.b, hkv, hq, t, d, sh.n, 0, a.split_tokens))
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
    pre_native = prefix.native()
    qt, kct, vct = N.t4(qg), N.t4(kcg), N.t4(vcg)

    def partial():
        N.check(lib.ma_splitk_partial(qt, sh.b, hq, t, d, pre_native, hkv, kct, vct, t, 0, 0, 0, d ** -0.5,
                                      a.split_tokens, ws.data_ptr(), ws_bytes,
                                      torch.cuda.current_stream().cuda_stream), "ma_splitk_partial")

    ms_partial, _ = time_graph(partial, a.steps, a.warmup)

    def scores_only():
        _, stats = result["stats_holder"]
        prefix_scores(qg, prefix, stats, rows, value=True)

    out0, stats0 = splitk_attention(qg, prefix, kcg, vcg, want_prefix=True, split_tokens=a.split_tokens)
    result["stats_holder"] = (out0, stats0)
    ms_scores, _ = time_graph(scores_only, a.steps, a.warmup)

    ms_eager = None
    if a.eager:
        for _ in range(a.warmup):
            step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(a.steps):
            step()
        e1.record()
        torch.cuda.synchronize()
        ms_eager = e0.elapsed_time(e1) / a.steps

    alg = algorithmic(sh)
    t_step = ms_step * 1e-3
    gbs = alg["bytes"] / t_step / 1e9
    t1 = ms_partial * 1e-3
    p1_tflops = alg["pass1_flops"] / t1 / 1e12
    p1_gbs = alg["pass1_bytes"] / t1 / 1e9
    line = {
        "metric": "µs per layer block-step + achieved HBM GB/s (% roofline), 32k prefix, int4 KV",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "us_per_layer_step": round(ms_step * 1e3, 3),
        "hbm_roofline_frac": round(gbs / HBM_PEAK_GBS, 4),
        "mfma_frac": round(alg["flops"] / t_step / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 mfma / int4 kv",
        "data": "synthetic (seed 1234: N(0,1) Q/K/V, LogNormal(0,0.5) key channels, 4 sink keys x8)",
        "config": {"workload": f"{sh.name}: step 0 (split-K attention + value-aware scores + read-set top-k "
                               f"+ gather), B{sh.b} Hq{sh.hq} Hkv{sh.hkv} D{sh.d} T{sh.t} read {sh.read_k}",
                   "prefix": sh.n, "kv": "int4 k4v4 (KG 32, VG 32, f16 scale/zero)",
                   "split_tokens": a.split_tokens or "auto", "graph": True,
                   "algorithmic_bytes": alg["bytes"], "algorithmic_flops": alg["flops"]},
        "stages_us": {"splitk_partial": round(ms_partial * 1e3, 3), "scores": round(ms_scores * 1e3, 3)},
        "roofline": {"kernel": "splitk_fwd_kernel<128> (pass 1)", "bound": "mfma",
                     "achieved": round(p1_tflops, 2), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(p1_tflops / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None,
                     "hbm_gbs": round(p1_gbs, 1), "hbm_frac": round(p1_gbs / HBM_PEAK_GBS, 4)},
    }
    if ms_eager is not None:
        line["eager_us_per_step"] = round(ms_eager * 1e3, 3)
    if not a.no_cpu:
        from oracle import attention as OA

        kd = OA.dequantize_keys(lay["kq"].cpu(), lay["ks"].cpu(), lay["kz"].cpu()).to(torch.bfloat16)
        vd = OA.dequantize_values(lay["vq"].cpu(), lay["vs"].cpu(), lay["vz"].cpu()).to(torch.bfloat16)
        sec, cores = cpu_baseline(sh, q, kd, vd, kc, vc, a.cpu_reps)
        line["cpu_baseline"] = {"value": round(alg["bytes"] / sec / 1e9, 3), "unit": "GB/s",
                                "us_per_layer_step": round(sec * 1e6, 1), "cores": cores, "kind": "port",
                                "sample": f"one full config-2 layer step 0 (prefix {sh.n}, dequantized bf16 K/V, "
                                          f"float32 torch ops), median of {a.cpu_reps} after 1 warm-up",
                                "cpu": platform.processor() or platform.machine()}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
