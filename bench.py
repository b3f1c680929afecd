"""Benchmark of the MI355X read path: step 0 of a sparse layer at the headline shape.

Workload: packed int4 k4v4 cache, prefix 32768 tokens, batch
1, 28 query / 4 KV heads, head_dim 128, mask block of 32 queries (all 32 are selection
rows), read budget 2048 per KV head.  One layer step = split-K attention over
[prefix | block] with prefix statistics, the value-aware score pass, the read-set top-k
and the gather of the selected K/V into the layer's compact bf16 buffer -- everything
step 0 of the reference's fast path does for a sparse layer (session.py:1403-1454).

One timed step is that layer step for each of --layers layers (28: the layer count of the
7B-class model of configs 1 and 4), each layer with its own packed cache (the tokens of
one seeded cache rolled by a per-layer offset), so no layer reads K/V left warm by the
previous one; the reported per-layer time is the step time / layers.  Inputs are
synthetic (seeded N(0,1), LogNormal key channels, 4 sink keys x8) and resident in HBM
before timing.  The step is captured once in a HIP graph and replayed; the dominant
kernel (split-K pass 1) is also timed alone from its own graph.  Prints ONE JSON line.

    python bench.py [--steps K] [--warmup W] [--layers L] [--split-tokens S] [--no-cpu]

--workload evict measures instead the packed lazy eviction of every layer (the rebuild
that follows a keep-set selection); its JSON line names its own metric.
"""

from __future__ import annotations

import argparse
import json
import math
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
PASS1_KERNEL = "splitk_fwd_kernel<128, 0, true>"  # packed-source split-K pass 1, whole tiles (carries the current block)
SCORE_KERNEL = "score_kernel<128, 0, 1, 1024, false, true>"  # value-aware score pass over packed K/V


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--split-tokens", type=int, default=0)
    ap.add_argument("--layers", type=int, default=28, help="layers per timed step, each with its own cache")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="wall-clock budget of the CPU baseline sample (repeated whole steps)")
    ap.add_argument("--eager-steps", type=int, default=3,
                    help="steps of the same workload timed without the HIP graph (0: skip)")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the extra workloads of the default line (config 1 block step, config 3 keep "
                         "step, 28-layer packed eviction)")
    ap.add_argument("--workload", choices=("step0", "evict", "substep"), default="step0",
                    help="step0: the headline read step (default); evict: the packed lazy eviction of all "
                         "28 layers (state compaction, rebuild plan, rebuild); substep: the denoising "
                         "sub-step attention over [2048 selected | block] of 28 layers")
    ap.add_argument("--block", type=int, default=32, help="substep: queries per block (32, or 8 for the "
                                                          "Fast-dLLM block cache)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="launch a plain 512 MiB device copy three times first, as the calibration "
                         "kernel of a FETCH_SIZE / WRITE_SIZE counter run")
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
    return dict(bytes=pass1 + pass2 + scores + gather, flops=flops1 + flops2, pass1_bytes=pass1, pass1_flops=flops1,
                pass2_bytes=pass2 + n * h * 4 * 2, pass2_flops=flops2)


def time_graph(fn, steps, warmup, inner=1):
    """Capture `inner` calls of fn() in one HIP graph, then replay it `warmup` times
    untimed and `steps` times between two events, all on the current stream (the replay
    stream).  Every kernel launched by fn uses torch's current stream, which is the
    capture stream during capture, so the events bracket exactly the replayed kernels.
    Returns ms per call of fn."""
    side = torch.cuda.Stream()                 # default priority
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()                                   # allocate / load the kernels outside capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    # captured on the warm-up stream, so that what fn() keeps per stream (the select
    # state) already exists: nothing is allocated or zero-filled during capture
    with torch.cuda.graph(g, stream=side):
        for _ in range(inner):
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
    return e0.elapsed_time(e1) / (steps * inner), g


def load_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed counter summary
    (profiles/traffic_c2_k4v4_n32768.md): the fenced JSON block holds, per kernel,
    FETCH_SIZE and WRITE_SIZE in KiB per dispatch and the copy-kernel calibration
    factor of each counter.  None when the summary or the kernel is absent."""
    f = ROOT / "profiles" / "traffic_c2_k4v4_n32768.md"
    if not f.exists():
        return None
    txt = f.read_text()
    try:
        blob = json.loads(txt.split("```json", 1)[1].split("```", 1)[0])
    except (IndexError, ValueError):
        return None
    k = blob.get("kernels", {}).get(kernel)
    if k is None:
        return None
    return int(round(k["fetch_kib"] * 1024 * blob["fetch_factor"] + k["write_kib"] * 1024 * blob["write_factor"]))


def cpu_baseline(sh, q, kd, vd, kc, vc, budget_s):
    """The reference's CPU torch path for the same step (oracle restatement, float32),
    repeated on whole steps until `budget_s` seconds have passed (at least 3 timed steps,
    after one warm-up).  Returns (median seconds per step, threads, steps timed)."""
    from oracle import attention as OA

    torch.set_num_threads(os.cpu_count() or 1)
    args = (q.float(), kd.float(), vd.float(), kc.float(), vc.float())
    OA.reference_cpu_step(*args, query_indices=range(sh.t), topk=sh.read_k)        # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or time.perf_counter() - t_start < budget_s:
        t0 = time.perf_counter()
        OA.reference_cpu_step(*args, query_indices=range(sh.t), topk=sh.read_k)
        times.append(time.perf_counter() - t0)
    return statistics.median(times), torch.get_num_threads(), len(times)


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

    if a.workload == "evict":
        bench_evict(a)
        return
    if a.workload == "substep":
        bench_substep(a)
        return
    from maskahead_amd import _native as N
    from maskahead_amd.kernels import (Step0Buffers, prefix_scores, quantize_key_groups_into, quantize_values_into,
                                       splitk_attention, step0_select)
    from maskahead_amd.kernels.splitk import Prefix
    from maskahead_amd.workloads import CONFIGS, layer_inputs, packed_layout

    sh = CONFIGS["c2"]
    dev = torch.device("cuda:0")
    if a.copy_probe:
        # calibration kernel for the HBM byte counters: a plain copy of 512 MiB
        # (536 870 912 B read + 536 870 912 B written per launch)
        src = torch.ones((512 << 20,), dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    q, k, v, kc, vc = layer_inputs(sh, dtype=torch.bfloat16)
    qg, kcg, vcg = q.to(dev), kc.to(dev), vc.to(dev)
    kdev, vdev = k.to(dev), v.to(dev)
    rows = list(range(sh.t))          # the whole block in order (mode "all"), as the session passes it

    layers = []
    for li in range(a.layers):
        lay = packed_layout(sh.b, sh.hkv, sh.n, sh.d, device=dev)
        shift = (li * 977) % sh.n
        quantize_key_groups_into(torch.roll(kdev, shift, dims=2), lay["kq"], lay["ks"], lay["kz"], bits=4,
                                 token_group=32)
        quantize_values_into(torch.roll(vdev, shift, dims=2), lay["vq"], lay["vs"], lay["vz"], bits=4,
                             channel_group=32)
        prefix = Prefix(kq=lay["kq"], ks=lay["ks"], kz=lay["kz"], vq=lay["vq"], vs=lay["vs"], vz=lay["vz"],
                        nq=sh.n, kb=4, vb=4)
        compact_k = torch.empty((sh.b, sh.hkv, sh.read_k + sh.t, sh.d), dtype=torch.bfloat16, device=dev)
        layers.append(dict(prefix=prefix, lay=lay, ck=compact_k, cv=torch.empty_like(compact_k), bufs=Step0Buffers()))
    del kdev, vdev
    prefix, lay = layers[0]["prefix"], layers[0]["lay"]
    result = {}

    step_ws = Step0Buffers()                 # one scratch workspace, shared by the layers

    def layer_step(L):
        # the session's step 0 (FastLayerPath.step0): one library call into the layer's own
        # reused buffers -- split-K attention, value-aware scores building the select's first
        # histogram level, the read-set top-k and the gather
        out, _, mass, score, idx = step0_select(L["bufs"], qg, L["prefix"], kcg, vcg, rows, sh.read_k, value=True,
                                                out_key=L["ck"][:, :, :sh.read_k],
                                                out_value=L["cv"][:, :, :sh.read_k], workspace=step_ws)
        result["out"], result["idx"] = out, idx

    def step():
        for L in layers:
            layer_step(L)

    ms_step, _ = time_graph(step, a.steps, a.warmup)
    ms_layer = ms_step / a.layers

    # The two large kernels of the step, each alone in a graph that launches it once per
    # layer on that layer's own cache (as cold as in the step: the layers' caches together
    # exceed the 256 MB Infinity Cache): split-K pass 1 and the value-aware score pass.
    lib = N.load()
    hq, t, d, hkv = sh.hq, sh.t, sh.d, sh.hkv
    ws_bytes = int(lib.ma_splitk_workspace_bytes(sh.b, hkv, hq, t, d, sh.n, 0, a.split_tokens))
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
    natives = [L["prefix"].native() for L in layers]
    qt, kct, vct = N.t4(qg), N.t4(kcg), N.t4(vcg)

    def partial_all():
        st = torch.cuda.current_stream().cuda_stream
        for pn in natives:
            N.check(lib.ma_splitk_partial(qt, sh.b, hq, t, d, pn, hkv, kct, vct, t, 0, 0, 0, d ** -0.5,
                                          a.split_tokens, ws.data_ptr(), ws_bytes, st), "ma_splitk_partial")

    stats_all = [splitk_attention(qg, L["prefix"], kcg, vcg, want_prefix=True, split_tokens=a.split_tokens)[1]
                 for L in layers]

    def scores_all(q_rows=rows):
        for L, stl in zip(layers, stats_all):
            prefix_scores(qg, L["prefix"], stl, q_rows, value=True)

    ms_partial = time_graph(partial_all, a.steps, a.warmup)[0] / a.layers
    ms_scores = time_graph(scores_all, a.steps, a.warmup)[0] / a.layers
    # the score pass with one and two selection positions (7 and 14 rows per KV head): the
    # GQA-reduced VALU variant and the padded 32-row MFMA variant, each forced
    variants = {}
    for pos in ([sh.t - 1], [sh.t - 2, sh.t - 1]):
        pos_dev = torch.tensor(pos, dtype=torch.int32, device=dev)   # a device row table, made before capture
        for name, mode in (("valu", 2), ("mfma", 1)):
            prev_path = lib.ma_prefix_scores_path(mode)
            try:
                variants[(len(pos), name)] = time_graph(lambda: scores_all(pos_dev), a.steps, a.warmup)[0] / a.layers
            finally:
                lib.ma_prefix_scores_path(prev_path)
    del stats_all

    ms_eager = None
    if a.eager_steps > 0:
        step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(a.eager_steps):
            step()
        e1.record()
        torch.cuda.synchronize()
        ms_eager = e0.elapsed_time(e1) / a.eager_steps / a.layers

    alg = algorithmic(sh)
    t_step = ms_layer * 1e-3
    gbs = alg["bytes"] / t_step / 1e9
    kernels = {
        "splitk_partial": dict(kernel=PASS1_KERNEL, ms=ms_partial, flops=alg["pass1_flops"], bytes=alg["pass1_bytes"]),
        "scores": dict(kernel=SCORE_KERNEL, ms=ms_scores, flops=alg["pass2_flops"], bytes=alg["pass2_bytes"]),
    }
    dom_name = max(kernels, key=lambda kk: kernels[kk]["ms"])
    dom = kernels[dom_name]
    t_dom = dom["ms"] * 1e-3
    f_mfma = dom["flops"] / t_dom / 1e12 / MFMA_BF16_PEAK_TFLOPS
    f_hbm = dom["bytes"] / t_dom / 1e9 / HBM_PEAK_GBS
    t_mfma_floor = dom["flops"] / (MFMA_BF16_PEAK_TFLOPS * 1e12)
    t_hbm_floor = dom["bytes"] / (HBM_PEAK_GBS * 1e9)
    if t_mfma_floor >= t_hbm_floor:
        roof = {"bound": "mfma", "achieved": round(dom["flops"] / t_dom / 1e12, 2), "peak": MFMA_BF16_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(f_mfma, 4)}
    else:
        roof = {"bound": "hbm", "achieved": round(dom["bytes"] / t_dom / 1e9, 2), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(f_hbm, 4)}
    roof["traffic"] = load_traffic(dom["kernel"])
    roof.update({"kernel": dom["kernel"], "avg_launch_us": round(dom["ms"] * 1e3, 3),
                 "algorithmic_bytes": dom["bytes"], "algorithmic_flops": dom["flops"],
                 "hbm_frac": round(f_hbm, 4), "mfma_frac": round(f_mfma, 4)})
    line = {
        "metric": "\u00b5s per layer block-step + achieved HBM GB/s (% roofline), 32k prefix, int4 KV",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "us_per_layer_step": round(ms_layer * 1e3, 3),
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
                               f"+ gather), B{sh.b} Hq{sh.hq} Hkv{sh.hkv} D{sh.d} T{sh.t} read {sh.read_k}; "
                               f"one step = {a.layers} layers, each with its own cache",
                   "layers": a.layers,
                   "prefix": sh.n, "kv": "int4 k4v4 (KG 32, VG 32, f16 scale/zero)",
                   "split_tokens": a.split_tokens or "auto", "graph": True,
                   "algorithmic_bytes": alg["bytes"], "algorithmic_flops": alg["flops"]},
        "stages_us": {kk: round(v["ms"] * 1e3, 3) for kk, v in kernels.items()},
        "roofline": roof,
    }
    g = sh.hq // sh.hkv
    line["score_variants"] = {
        f"r2_{npos * g}": {"rows": f"{npos} selection position(s) x {g} query heads per KV head",
                           "valu_us": round(variants[(npos, "valu")] * 1e3, 3),
                           "mfma_padded_us": round(variants[(npos, "mfma")] * 1e3, 3),
                           "valu_hbm_frac": round(alg["pass2_bytes"] / (variants[(npos, "valu")] * 1e-3) / 1e9
                                                  / HBM_PEAK_GBS, 4)}
        for npos in (1, 2)}
    if ms_eager is not None:
        # the same layer step launched op by op from Python (ctypes argument packing and
        # torch allocations on every call), as a session without graph capture runs it
        line["eager_us_per_step"] = round(ms_eager * 1e3, 3)
        line["eager_hbm_frac"] = round(alg["bytes"] / (ms_eager * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    if not a.no_extras:
        del layers, result
        torch.cuda.empty_cache()
        line["extras"] = {"c1_block_step": extra_c1_block(a), "c3_keep_step": extra_c3_keep(a),
                          "c4_block_step": extra_c4_block(a), "evict_28_layers": extra_evict(a)}
    if not a.no_cpu:
        from oracle import attention as OA

        kd = OA.dequantize_keys(lay["kq"].cpu(), lay["ks"].cpu(), lay["kz"].cpu()).to(torch.bfloat16)
        vd = OA.dequantize_values(lay["vq"].cpu(), lay["vs"].cpu(), lay["vz"].cpu()).to(torch.bfloat16)
        sec, cores, reps = cpu_baseline(sh, q, kd, vd, kc, vc, a.cpu_seconds)
        line["cpu_baseline"] = {"value": round(alg["bytes"] / sec / 1e9, 3), "unit": "GB/s",
                                "us_per_layer_step": round(sec * 1e6, 1), "cores": cores, "kind": "port",
                                "sample": f"{reps} whole config-2 step-0 layer steps (prefix {sh.n}, dequantized "
                                          f"bf16 K/V, float32 torch ops) in ~{a.cpu_seconds:g} s after 1 warm-up; "
                                          f"median step",
                                "cpu": platform.processor() or platform.machine(),
                                "os_cpu_count": os.cpu_count()}
    print(json.dumps(line), flush=True)


def bench_substep(a):
    """A denoising sub-step of every layer (session.py:1286-1336; sdpa_compact,
    reference.py:403-426): softmax attention of the block's queries over [the 2 048
    entries selected at step 0 | the block's own K/V], per layer from that layer's compact
    bf16 buffer, as runtime.fastpath.compact_attention runs it (split-K pass 1 + merge, no
    copy of the block into the buffer).  28 layers per timed step in one HIP graph."""
    from maskahead_amd.kernels import splitk_attention
    from maskahead_amd.kernels.splitk import Prefix

    dev = torch.device("cuda:0")
    B, HQ, H, D, K, T = 1, 28, 4, 128, 2048, a.block
    g = torch.Generator(device="cuda").manual_seed(1234)
    layers = []
    for _ in range(a.layers):
        ck = torch.randn((B, H, K + 32, D), device=dev, generator=g).to(torch.bfloat16)
        cv = torch.randn((B, H, K + 32, D), device=dev, generator=g).to(torch.bfloat16)
        layers.append(Prefix.dense(ck[:, :, :K], cv[:, :, :K]))
    q = torch.randn((B, HQ, T, D), device=dev, generator=g).to(torch.bfloat16)
    kc = torch.randn((B, H, T, D), device=dev, generator=g).to(torch.bfloat16)
    vc = torch.randn((B, H, T, D), device=dev, generator=g).to(torch.bfloat16)
    scale = D ** -0.5

    def step():
        for pre in layers:
            splitk_attention(q, pre, kc, vc, scaling=scale, split_tokens=a.split_tokens)

    ms_step, _ = time_graph(step, a.steps, a.warmup)
    us = ms_step * 1e3 / a.layers
    R = (HQ // H) * T
    nbytes = H * (K + T) * D * 2 * 2 + 2 * B * HQ * T * D * 2      # K, V read; Q read, out written
    flops = 4 * R * (K + T) * D * H
    t = us * 1e-6
    f_hbm = nbytes / t / 1e9 / HBM_PEAK_GBS
    f_mfma = flops / t / 1e12 / MFMA_BF16_PEAK_TFLOPS
    line = {
        "metric": f"\u00b5s per layer sub-step (attention over [2048 selected | {T}-token block], bf16 compact)",
        "value": round(us, 3), "unit": "us", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms_step, 5), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (seed 1234: N(0,1) compact K/V, queries, block K/V)",
        "config": {"workload": f"substep_k2048_t{T}: B{B} Hq{HQ} Hkv{H} D{D}, {a.layers} layers per graph replay",
                   "split_tokens": a.split_tokens or "auto", "algorithmic_bytes": nbytes, "algorithmic_flops": flops},
        "roofline": {"bound": "hbm" if nbytes / HBM_PEAK_GBS / 1e9 >= flops / MFMA_BF16_PEAK_TFLOPS / 1e12 else "mfma",
                     "achieved": round(nbytes / t / 1e9, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(f_hbm, 4), "traffic": None, "kernel": "splitk_fwd_kernel<128, 2> + "
                     "splitk_combine_kernel<128> (whole sub-step)", "avg_launch_us": round(us, 3),
                     "mfma_frac": round(f_mfma, 4)},
    }
    if not a.no_cpu:
        from oracle import attention as OA

        # the reference's CPU sub-step (sdpa_compact, reference.py:403-426, restated in
        # oracle.attention.dense_attention) on the first layer's compact buffer, repeated
        pre0 = layers[0]
        args = (q.cpu(), pre0.kf.cpu(), pre0.vf.cpu(), kc.cpu(), vc.cpu())
        torch.set_num_threads(os.cpu_count() or 1)
        OA.dense_attention(*args)
        ctimes = []
        t_start = time.perf_counter()
        while len(ctimes) < 3 or time.perf_counter() - t_start < min(a.cpu_seconds, 10.0):
            t0 = time.perf_counter()
            OA.dense_attention(*args)
            ctimes.append(time.perf_counter() - t0)
        sec = statistics.median(ctimes)
        line["cpu_baseline"] = {"value": round(sec * 1e6, 1), "unit": "us", "cores": torch.get_num_threads(),
                                "kind": "port",
                                "sample": f"{len(ctimes)} layer sub-steps (oracle dense_attention over [2048 | {T}], "
                                          "float64 torch ops) after 1 warm-up; median",
                                "cpu": platform.processor() or platform.machine(), "os_cpu_count": os.cpu_count()}
    print(json.dumps(line), flush=True)


def bench_evict(a):
    print(json.dumps(measure_evict(a, with_cpu=not a.no_cpu)), flush=True)


def measure_evict(a, with_cpu):
    """The packed lazy eviction of every layer (session.py:270-361 + cache.py:236-335):
    28 layers x 4 KV heads of a 32 768-token int4 prefix + 32 bf16 residual tokens,
    keep 4 096 per lane (a 128-token recency window + a clustered seeded score), repack
    threshold 0.5.  A step = the eviction state's compaction, the rebuild plan and the
    rebuild, with the decode loop's check=False (one host synchronisation, the plan's
    counts; the rebuild's error status is read after the timed region), timed one eviction
    at a time from a restored cache.  The rebuild launch is also timed alone with
    events over repeated launches on fixed lists (the roofline kernel)."""
    from maskahead_amd import _native as N
    from maskahead_amd.cache import PackedKVCache
    from maskahead_amd.config import QuantizationConfig
    from maskahead_amd.eviction import EvictionConfig, EvictionState
    from maskahead_amd.kernels.rebuild import rebuild_packed, rebuild_plan
    from maskahead_amd.kernels.splitk import Prefix
    from maskahead_amd.runtime.session import evict_to

    dev = torch.device("cuda:0")
    L, B, H, D, N0, R, C, W, repack = a.layers, 1, 4, 128, 32768, 32, 4096, 128, 0.5
    cache = PackedKVCache(num_layers=L, batch_size=B, num_kv_heads=H, head_dim=D, max_tokens=1 << 20,
                          quant=QuantizationConfig(residual_tokens=R), device=dev)
    g = torch.Generator(device="cuda").manual_seed(1234)
    cache.begin_append(N0 + R)
    for li in range(L):
        k = torch.randn((B, H, N0 + R, D), device=dev, generator=g).to(torch.bfloat16)
        v = torch.randn((B, H, N0 + R, D), device=dev, generator=g).to(torch.bfloat16)
        cache.stage_layer(li, k, v)
    cache.commit_append()
    n = cache.length
    st = EvictionState(num_layers=L, batch_size=B, num_kv_heads=H, capacity=n, device=dev)
    st.append(range(n))
    gc = torch.Generator().manual_seed(1234)
    score = torch.rand((L, B, H, n), generator=gc)
    grp = torch.arange(n) // 32
    for lane in range(L * B * H):
        dense = torch.randperm(n // 32, generator=gc)[:20]
        score[lane // (B * H), (lane // H) % B, lane % H] += 2.0 * torch.isin(grp, dense)
    score[..., n - W:] = 1e9
    keep = score.topk(C, dim=-1).indices.sort(dim=-1).values.to(dev)
    names = ("k_q", "k_scale", "k_zero", "v_q", "v_scale", "v_zero", "k_residual", "v_residual")
    saved = {x: getattr(cache, x) for x in names}
    meta = ("length", "quantized_length", "residual_length", "dropped")   # capacities follow the planes
    saved_meta = {x: getattr(cache, x) for x in meta}
    pos0, phys0 = st.pos.clone(), st.phys.clone()
    cfg = EvictionConfig(policy="recent", recent_window=W, capacity_floor=W, compaction="lazy", repack_below=repack)

    def restore():
        for x in names:
            setattr(cache, x, saved[x])
        for x in meta:
            setattr(cache, x, saved_meta[x])
        st.pos.copy_(pos0)
        st.phys.copy_(phys0)
        st.live = n

    times = []
    for i in range(a.warmup + a.steps):
        restore()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        # the decode loop's hot path: the plan's count read-back is the one host
        # synchronisation; the rebuild's error status is read after the timed region
        evict_to(cache, st, keep, cfg, next_position=n, check=False)
        torch.cuda.synchronize()
        if i >= a.warmup:
            times.append(time.perf_counter() - t0)
        cache.check_rebuild()
    us = statistics.median(times) * 1e6
    new_lens = (cache.length, cache.quantized_length, cache.residual_length)

    # the rebuild alone: the lists of this eviction, fixed storage, repeated launches
    restore()
    st.compact(keep)
    need = max(1, math.ceil(repack * 32))
    gb, enc, stg = rebuild_plan(st.phys, st.pos, C, quantized_length=cache.quantized_length, need=need,
                                tail_groups=0, window=min(W, C))
    ga = torch.empty((L, B, H, 0), dtype=torch.int64, device=dev)
    g1, m, nst = gb.shape[-1], enc.shape[-1], stg.shape[-1]
    g2 = -(-m // 32)
    ql = (g1 + g2) * 32
    f = lambda t: t.flatten(0, 1)  # noqa: E731
    kq = torch.empty((L, B, H, ql // 32, D, 16), dtype=torch.uint8, device=dev)
    ks, kz = (torch.empty((L, B, H, ql // 32, D), dtype=torch.float16, device=dev) for _ in range(2))
    vq = torch.empty((L, B, H, ql, D // 32, 16), dtype=torch.uint8, device=dev)
    vs, vz = (torch.empty((L, B, H, ql, D // 32), dtype=torch.float16, device=dev) for _ in range(2))
    kr, vr = (torch.empty((L, B, H, max(nst, 1), D), dtype=torch.bfloat16, device=dev) for _ in range(2))
    old = Prefix(kq=f(cache.k_q), ks=f(cache.k_scale), kz=f(cache.k_zero), vq=f(cache.v_q), vs=f(cache.v_scale),
                 vz=f(cache.v_zero), kf=f(cache.k_residual), vf=f(cache.v_residual), nq=cache.quantized_length,
                 nf=cache.residual_length, kb=4, vb=4)
    new = Prefix(kq=f(kq), ks=f(ks), kz=f(kz), vq=f(vq), vs=f(vs), vz=f(vz), kf=f(kr), vf=f(vr), nq=ql, nf=nst,
                 kb=4, vb=4)
    remap = torch.empty((L, B, H, n), dtype=torch.int64, device=dev)

    def rebuild():
        rebuild_packed(old, new, B=L * B, H=H, D=D, groups_before=gb, encode=enc, groups_after=ga, stage=stg,
                       remap=remap)

    for _ in range(3):
        rebuild()
    torch.cuda.synchronize()
    inner = 20
    cur = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    lib = N.load()
    on, nn = old.native(), new.native()
    status = torch.empty((L * B * H,), dtype=torch.int32, device=dev)
    import ctypes

    gb2, enc2, stg2 = (t.reshape(L * B * H, t.shape[-1]) for t in (gb, enc, stg))
    args = (ctypes.byref(on), L * B, H, D, ctypes.byref(nn), gb2.data_ptr(), gb2.stride(0), g1, enc2.data_ptr(),
            enc2.stride(0), m, None, 0, 0, stg2.data_ptr(), stg2.stride(0), nst, remap.data_ptr(), n, None, 0, 0,
            status.data_ptr(), cur.cuda_stream)
    e0.record(cur)
    for _ in range(inner):
        N.check(lib.ma_rebuild_packed(*args), "ma_rebuild_packed")
    e1.record(cur)
    torch.cuda.synchronize()
    us_rebuild = e0.elapsed_time(e1) * 1e3 / inner

    # algorithmic bytes of the rebuild launches (per lane, summed): kept groups read +
    # written (5 120 B per group: K and V codes 2 x 2 048 B, scale / zero 2 x 512 B);
    # encoded and staged entries read from the packed part (160 B: 64 B K codes + 64 B V
    # codes + 16 + 16 B of scale / zero) or the bf16 residual (512 B); encoded entries
    # written packed (160 B), staged ones bf16 (512 B); the remap written (8 B per old slot)
    lanes = L * B * H
    src = torch.cat([enc, stg], -1)
    n_packed = int(((src >= 0) & (src < cache.quantized_length)).sum())
    n_res = int((src >= cache.quantized_length).sum())
    n_enc, n_stg = int((enc >= 0).sum()), int((stg >= 0).sum())
    n_grp = int((gb >= 0).sum())
    rb_bytes = (n_grp * 5120 * 2 + n_packed * 160 + n_res * 512 + n_enc * 160 + n_stg * 512 + lanes * n * 8
                + lanes * (g1 * 32 + m + nst) * 8)
    achieved = rb_bytes / (us_rebuild * 1e-6) / 1e9
    line = {
        "metric": "\u00b5s per packed lazy eviction of 28 layers (keep 4096 of 32800 per KV head, int4 KV)",
        "value": round(us, 1),
        "unit": "us",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(us / 1e3, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 codes / bf16 requantization",
        "data": "synthetic (seed 1234: N(0,1) K/V; clustered seeded keep score, 128-token window)",
        "config": {"workload": f"evict_c4_k4v4_n32768: state compaction + rebuild plan + packed rebuild of "
                               f"{L} layers x {H} KV heads, prefix {N0} int4 + {R} bf16, keep {C}, window {W}, "
                               f"repack_below {repack}",
                   "layers": L, "new_lengths": new_lens, "kept_groups": n_grp, "encoded": n_enc,
                   "staged": n_stg},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "rebuild_kernel", "avg_launch_us": round(us_rebuild, 2),
                     "algorithmic_bytes": rb_bytes},
    }
    if with_cpu:
        from oracle import rebuild as OR

        # bounded sample: 2 of the layers, the same lists, on the host
        Ls = 2
        store = {"kq": cache.k_q[:Ls].cpu(), "ks": cache.k_scale[:Ls].cpu(), "kz": cache.k_zero[:Ls].cpu(),
                 "vq": cache.v_q[:Ls].cpu(), "vs": cache.v_scale[:Ls].cpu(), "vz": cache.v_zero[:Ls].cpu(),
                 "kr": cache.k_residual[:Ls].cpu(), "vr": cache.v_residual[:Ls].cpu()}
        lens = (cache.length, cache.quantized_length, cache.residual_length, cache.dropped)
        pos, phys = pos0[:Ls, ..., :n].cpu().to(torch.int64), phys0[:Ls, ..., :n].cpu().to(torch.int64)
        torch.set_num_threads(os.cpu_count() or 1)
        ctimes = []
        t_start = time.perf_counter()
        while len(ctimes) < 2 or time.perf_counter() - t_start < min(a.cpu_seconds, 30.0):
            t0 = time.perf_counter()
            OR.evict(store, lens, pos, phys, keep[:Ls].cpu(), next_position=n, stage_mode=False, mode="lazy",
                     repack_below=repack, recent_window=W)
            ctimes.append(time.perf_counter() - t0)
        per_evict = statistics.median(ctimes) * L / Ls
        line["cpu_baseline"] = {"value": round(per_evict * 1e6, 1), "unit": "us", "cores": torch.get_num_threads(),
                                "kind": "port",
                                "sample": f"{len(ctimes)} evictions of {Ls} of the {L} layers (oracle/rebuild.py, "
                                          f"torch CPU ops), median x {L // Ls}",
                                "cpu": platform.processor() or platform.machine(), "os_cpu_count": os.cpu_count()}
    return line


def _roof(nbytes, flops, seconds):
    """The roofline of a whole workload: HBM and MFMA fractions, bound = the larger floor."""
    f_hbm = nbytes / seconds / 1e9 / HBM_PEAK_GBS
    f_mfma = flops / seconds / 1e12 / MFMA_BF16_PEAK_TFLOPS
    hbm_bound = nbytes / HBM_PEAK_GBS / 1e9 >= flops / MFMA_BF16_PEAK_TFLOPS / 1e12
    return {"bound": "hbm" if hbm_bound else "mfma",
            "achieved": round(nbytes / seconds / 1e9, 2) if hbm_bound else round(flops / seconds / 1e12, 2),
            "unit": "GB/s" if hbm_bound else "TFLOP/s", "frac": round(f_hbm if hbm_bound else f_mfma, 4),
            "hbm_frac": round(f_hbm, 4), "mfma_frac": round(f_mfma, 4), "algorithmic_bytes": nbytes,
            "algorithmic_flops": flops}


def extra_c1_block(a):
    """BASELINE config 1, one block step of every layer: step 0 over a bf16 prefix of
    32 768 tokens (split-K attention with prefix statistics, value-aware scores, read-set
    top-k of 2 048, gather into the compact buffer) and the block's 3 further denoising
    sub-steps over [2 048 selected | block] (session.py:1403-1454, 1286-1336).  28 layers,
    each with its own cache, in one HIP graph."""
    from maskahead_amd.kernels import gather_packed_kv, prefix_scores_topk, splitk_attention
    from maskahead_amd.kernels.splitk import Prefix
    from maskahead_amd.workloads import CONFIGS, layer_inputs

    sh, dev, subs = CONFIGS["c1"], torch.device("cuda:0"), 3
    q, k, v, kc, vc = layer_inputs(sh, dtype=torch.bfloat16)
    qg, kcg, vcg = q.to(dev), kc.to(dev), vc.to(dev)
    kdev, vdev = k.to(dev), v.to(dev)
    rows = list(range(sh.t))

    class View:
        """a bf16 cache layer, as the gather reads it"""
        k_bits = v_bits = 16
        quantized_length = residual_length = 0
        key_token_group = value_channel_group = 32
        k_q = k_scale = k_zero = v_q = v_scale = v_zero = k_residual = v_residual = None
        head_dim = sh.d
        key_mode = "channel"

        def __init__(self, kf, vf):
            self.k_fp, self.v_fp, self.length = kf, vf, kf.shape[2]

    layers = []
    for li in range(a.layers):
        shift = (li * 977) % sh.n
        kf = torch.roll(kdev, shift, dims=2).contiguous()
        vf = torch.roll(vdev, shift, dims=2).contiguous()
        ck = torch.empty((sh.b, sh.hkv, sh.read_k, sh.d), dtype=torch.bfloat16, device=dev)
        layers.append((Prefix.dense(kf, vf), View(kf, vf), ck, torch.empty_like(ck)))
    del kdev, vdev

    def step():
        for pre, view, ck, cv in layers:
            _, stats = splitk_attention(qg, pre, kcg, vcg, want_prefix=True)
            _, score, idx = prefix_scores_topk(qg, pre, stats, rows, sh.read_k, value=True, rank="score")
            gather_packed_kv(view, idx, out_key=ck, out_value=cv)
            sel = Prefix.dense(ck, cv)
            for _ in range(subs):
                splitk_attention(qg, sel, kcg, vcg)

    ms = time_graph(step, max(5, a.steps // 5), 2)[0] / a.layers
    r = (sh.hq // sh.hkv) * sh.t
    kv = sh.n * sh.d * 2 * 2 * sh.hkv                       # bf16 K + V of the prefix
    sel_kv = (sh.read_k + sh.t) * sh.d * 2 * 2 * sh.hkv
    nbytes = (2 * kv + sh.n * sh.hkv * 8 + 2 * sh.read_k * sh.d * 2 * 2 * sh.hkv + subs * sel_kv)
    flops = 4 * r * sh.n * sh.d * sh.hkv + 2 * r * sh.n * sh.d * sh.hkv + subs * 4 * r * (sh.read_k + sh.t) * sh.d * sh.hkv
    del layers
    torch.cuda.empty_cache()
    return {"workload": f"{sh.name}: step 0 + {subs} sub-steps, bf16 prefix {sh.n}, read {sh.read_k}, "
                        f"{a.layers} layers each with its own cache, one HIP graph",
            "us_per_layer_block_step": round(ms * 1e3, 3), "roofline": _roof(nbytes, flops, ms * 1e-3)}


def extra_c3_keep(a, layers=4, reps=5):
    """BASELINE config 3, the look-ahead keep/evict step: per layer the probe forward of 96
    queries (the block + 2 look-ahead blocks, block-causal) over a bf16 prefix of 65 536
    tokens with their prefix mass, the keep score (value_score) and the keep set of 8 192
    per KV head (128-token window, 4 sinks); then the in-place compaction of every layer
    and the append of the finalized 32-token block (session.py:1985-2034, 2289-2297;
    eviction.py:325-418; cache.py:342-367).  Launched op by op from Python, as the session
    runs it; median of `reps` steps of `layers` layers, each from a restored cache."""
    from maskahead_amd.cache import PackedKVCache
    from maskahead_amd.config import QuantizationConfig
    from maskahead_amd.kernels.keep import keep_select, value_score
    from maskahead_amd.runtime.fastpath import FastLayerPath
    from maskahead_amd.workloads import CONFIGS, layer_inputs

    sh, dev = CONFIGS["c3"], torch.device("cuda:0")
    q, k, v, kc, vc = layer_inputs(sh, dtype=torch.bfloat16)
    qg, kcg, vcg = q.to(dev), kc.to(dev), vc.to(dev)
    cache = PackedKVCache(num_layers=layers, batch_size=sh.b, num_kv_heads=sh.hkv, head_dim=sh.d,
                          max_tokens=sh.n + 64, quant=QuantizationConfig(k_bits=16, v_bits=16), device=dev)
    cache.begin_append(sh.n)
    kdev, vdev = k.to(dev), v.to(dev)
    for li in range(layers):
        shift = (li * 977) % sh.n
        cache.stage_layer(li, torch.roll(kdev, shift, dims=2), torch.roll(vdev, shift, dims=2))
    cache.commit_append()
    del kdev, vdev
    saved = (cache.k_fp.clone(), cache.v_fp.clone())
    meta = ("length", "quantized_length", "residual_length", "dropped")
    saved_meta = {x: getattr(cache, x) for x in meta}
    pos = torch.arange(sh.n, dtype=torch.int32, device=dev).expand(sh.b, sh.hkv, sh.n).contiguous()
    fp = FastLayerPath(cache=cache, block_size=32, query_indices=list(range(32)))
    blk_k, blk_v = kcg[:, :, :32].contiguous(), vcg[:, :, :32].contiguous()

    def step():
        keeps = []
        for li in range(layers):
            _, mass = fp.attend(li, qg, kcg, vcg, causal=32, q_pos0=sh.n, mass_rows=list(range(sh.t)))
            score = value_score(mass, cache.layer_view(li).v_fp)
            keeps.append(keep_select(pos, score, sh.keep_k, 128, sink_tokens=4, check=False))
        cache.compact(torch.stack(keeps))
        cache.begin_append(32)
        for li in range(layers):
            cache.stage_layer(li, blk_k, blk_v)
        cache.commit_append()

    times = []
    for i in range(reps + 1):
        cache.k_fp, cache.v_fp = saved[0].clone(), saved[1].clone()   # the step shrinks the planes
        for x in meta:
            setattr(cache, x, saved_meta[x])
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        step()
        torch.cuda.synchronize()
        if i:
            times.append(time.perf_counter() - t0)
    sec = statistics.median(times) / layers
    r = (sh.hq // sh.hkv) * sh.t
    kv = sh.n * sh.d * 2 * sh.hkv                           # one bf16 plane (K or V) of the prefix
    nbytes = (2 * kv + kv + kv + sh.n * sh.hkv * 4 * 3 + 2 * sh.keep_k * sh.d * 2 * 2 * sh.hkv
              + 32 * sh.d * 2 * 2 * sh.hkv)
    flops = 4 * r * sh.n * sh.d * sh.hkv + 2 * r * sh.n * sh.d * sh.hkv
    del cache, saved
    torch.cuda.empty_cache()
    return {"workload": f"{sh.name}: probe of {sh.t} queries (block-causal) + prefix mass + value_score + keep "
                        f"{sh.keep_k} of {sh.n} per KV head, compaction in place + append of 32 tokens; "
                        f"{layers} layers, eager, median of {reps}",
            "us_per_layer_keep_step": round(sec * 1e6, 1), "roofline": _roof(nbytes, flops, sec)}


def extra_c4_block(a, L=28, dense=2):
    """BASELINE config 4, the ragged multi-sequence full-model block step: 8 sequences with
    prefix lengths uniform in [8 192, 131 072] (seed 1234), 28 layers of the config-1 head
    shape (the first 2 dense), packed int4 KV (every whole group quantized), read 2 048 /
    keep 4 096 per KV head.  One block of the batch, from freshly built caches (one per
    sequence): step 0 of every layer (fast-path routing: split-K attention, value-aware
    scores with the fused read-set select, gather), the lookahead eviction (keep score,
    keep set, packed lazy rebuild), 3 denoising sub-steps and the block's finalize (its KV
    appended) (session.py:1403-1454, 1985-2034, 270-361, 1286-1336, 2289-2297).  Launched
    op by op from Python, phase by phase as a batched forward does (BatchFastPath: each
    layer's step 0 per sequence over its own prefix, its sub-steps as one call over the
    batch's shared compact buffer), so the host's launches of one sequence overlap the GPU
    work of the others; the evictions of the batch read their plans' counts back in one
    synchronisation (lookahead_evict_batch).  Algorithmic bytes per sequence of prefix n (P = n x 4 KV heads x 160 B of int4 K and V with their
    scales): step 0 streams the prefix twice in a sparse layer (attention, scores) and once
    in a dense one; the eviction reads V once per layer (keep score) and reads and writes
    the 4 096 kept entries; the sub-steps read the 2 048-entry bf16 compact buffers of the
    sparse layers and the 4 096 kept entries of the dense ones."""
    from maskahead_amd.cache import PackedKVCache
    from maskahead_amd.config import QuantizationConfig
    from maskahead_amd.eviction import EvictionConfig, EvictionState
    from maskahead_amd.runtime.batch import BatchFastPath
    from maskahead_amd.runtime.fastpath import BlockContext
    from maskahead_amd.runtime.session import admit_new_entries, live_slot_masks, lookahead_evict_batch

    dev = torch.device("cuda:0")
    hq, hkv, d, t, read_k, keep_k, W = 28, 4, 128, 32, 2048, 4096, 64
    lens = torch.randint(8192, 131073, (8,), generator=torch.Generator().manual_seed(1234)).tolist()
    cfg = EvictionConfig(policy="lookahead", recent_window=W, capacity_floor=512, compaction="lazy",
                         repack_below=1.0, sink_tokens=4)

    class Seq:
        """One sequence of the batch: its cache, eviction state and block inputs."""

        def __init__(self, n, seed):
            g = torch.Generator(device=dev).manual_seed(seed)
            chan = torch.empty((1, hkv, 1, d), device=dev).log_normal_(0.0, 0.5, generator=g)
            k = torch.randn((1, hkv, n, d), device=dev, generator=g) * chan
            k[:, :, :4] *= 8.0
            k = k.to(torch.bfloat16)
            v = torch.randn((1, hkv, n, d), device=dev, generator=g).to(torch.bfloat16)
            self.blocks = [tuple(x.to(torch.bfloat16) for x in (
                torch.randn((1, hq, t, d), device=dev, generator=g),
                torch.randn((1, hkv, t, d), device=dev, generator=g) * chan,
                torch.randn((1, hkv, t, d), device=dev, generator=g))) for _ in range(L)]
            self.cache = PackedKVCache(num_layers=L, batch_size=1, num_kv_heads=hkv, head_dim=d,
                                       max_tokens=n + 4 * t, quant=QuantizationConfig(residual_tokens=0), device=dev)
            self.cache.begin_append(n)
            for layer in range(L):
                self.cache.stage_layer(layer, torch.roll(k, 977 * layer, dims=2), v)
            self.cache.commit_append()
            del k, v
            self.st = EvictionState(num_layers=L, batch_size=1, num_kv_heads=hkv, capacity=n + 4 * t, device=dev)
            self.st.append(range(n))
            self.n = n

    class Batch:
        """The batch as a batched forward hands it over: every layer's block queries and K/V
        as [8, H, 32, D] tensors, and one BatchFastPath over the 8 caches (one compact
        buffer [8, Hkv, 2048 + 32, D] per layer, as the reference's batched session keeps)."""

        def __init__(self, seqs):
            self.seqs = seqs
            self.blocks = [tuple(torch.cat([s.blocks[layer][j] for s in seqs]) for j in range(3)) for layer in range(L)]
            for s in seqs:
                del s.blocks
            self.bp = BatchFastPath([s.cache for s in seqs], block_size=t, query_indices=list(range(t)),
                                    dense_prefix_layers=dense)

    def block_step(batch):
        """One block of the batch, phase by phase as a batched forward runs it: step 0 of
        every layer (each sequence over its own prefix), the lookahead eviction of every
        sequence, 3 sub-steps (one call per sparse layer over the batch's compact buffer),
        the finalize.  Returns the seconds it took."""
        seqs, bp, blocks = batch.seqs, batch.bp, batch.blocks
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        # step 0 keeps each layer's mass per physical slot; the eviction puts all layers' in
        # live order at once (lookahead_scores, per_slot)
        ctxs = [BlockContext(step_index=0, old_cache_len=s.n, topk=read_k, evicting=True, live_len=s.st.live,
                             want_mass=True) for s in seqs]
        for layer in range(L):
            bp.route(layer, *blocks[layer], ctxs)
        lookahead_evict_batch([(s.cache, s.st, p.last_mass, None, s.n) for s, p in zip(seqs, bp.paths)], cfg, keep_k,
                              per_slot=True)
        for s, p in zip(seqs, bp.paths):
            p.slot_masks = live_slot_masks(s.cache, s.st)
        for step in (1, 2, 3):
            for ctx in ctxs:
                ctx.step_index = step
            for layer in range(L):
                bp.route(layer, *blocks[layer], ctxs)
        for i, s in enumerate(seqs):
            s.cache.begin_append(t)
            for layer in range(L):
                s.cache.stage_layer(layer, blocks[layer][1][i:i + 1], blocks[layer][2][i:i + 1])
            s.cache.commit_append()
            admit_new_entries(s.cache, s.st, s.n)
        torch.cuda.synchronize()
        sec = time.perf_counter() - t0
        for s in seqs:
            s.cache.check_rebuild()                      # the eviction's deferred error status
        return sec

    # warm-up: the same batch once (kernels loaded, and torch's caching allocator grown to
    # the batch's footprint, so the timed block reuses its blocks as a serving process does:
    # a cold allocator's device allocations synchronize the host); then fresh caches
    batch = Batch([Seq(n, 1234 + i) for i, n in enumerate(lens)])
    block_step(batch)
    del batch
    batch = Batch([Seq(n, 1234 + i) for i, n in enumerate(lens)])
    sec = block_step(batch)
    del batch
    torch.cuda.empty_cache()
    r = (hq // hkv) * t
    nbytes = flops = 0
    for n in lens:
        P = n * hkv * 160
        nbytes += (L - dense) * 2 * P + dense * P                                     # step 0
        nbytes += L * n * hkv * 80 + 2 * L * keep_k * hkv * 160                       # eviction
        nbytes += 3 * ((L - dense) * read_k * hkv * d * 2 * 2 + dense * keep_k * hkv * 160)   # sub-steps
        flops += (L - dense) * 6 * r * n * d * hkv + dense * 4 * r * n * d * hkv
        flops += 3 * ((L - dense) * 4 * r * read_k * d * hkv + dense * 4 * r * keep_k * d * hkv)
    return {"workload": f"c4: 8 sequences, prefixes {sorted(lens)}, 28 layers ({dense} dense), packed int4, "
                        f"read {read_k} / keep {keep_k}: one block of the batch -- step 0 of every layer, the "
                        f"lookahead eviction, 3 sub-steps, the finalize -- eager, phase by phase; sub-steps batched "
                        f"over the sequences (BatchFastPath)",
            "us_per_block_step": round(sec * 1e6, 1), "roofline": _roof(nbytes, flops, sec)}


def extra_evict(a):
    """The 28-layer packed lazy eviction (measure_evict), in short."""
    import copy

    b = copy.copy(a)
    b.steps, b.warmup = min(a.steps, 10), 2
    line = measure_evict(b, with_cpu=False)
    torch.cuda.empty_cache()
    return {"workload": line["config"]["workload"], "us_per_eviction": line["value"], "roofline": line["roofline"]}


if __name__ == "__main__":
    main()
