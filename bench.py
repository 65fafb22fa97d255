"""Benchmark of the gfx950 Qwen3 attention hot path (one GPU).

Default workload (the headline metric's configs[1]): Qwen3-4B-shape decode attention, batch 1,
32 query heads / 8 KV heads / head_dim 128, 36 layers each with its own fp32 KV cache of
4096 positions.  One step = one new token through all 36 layers: per layer one fused
launch (QK-norm + RoPE of Q and K, KV append at position 4095, split-K attention over
keys 0..4095), the 36 launches replayed as one HIP graph.  `value` = algorithmic bytes
(K+V of 4096 positions + q + out per layer) / step time, inputs resident in HBM.

Also reported: causal prefill (configs[2]: 2048 tokens, 36 layers, fused prologue +
fp32-MFMA attention) TFLOP/s, the dominant kernels' per-launch durations from HIP events
(on the launch stream) with their roofline fractions, and the reference CPU attention loop
(the oracle restatement of src/model.cpp:191-214, OpenMP over heads) timed on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
# HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, each scaled by
# the factor a plain 256 MiB copy needs (FETCH x2.000, WRITE x1.000); profiles/*_hbm_traffic.md
# and profiles/prefill_configs2_kernel_trace.md hold the runs.
TRAFFIC_DECODE_PER_LAYER = (16539 + 303.5) * 2.0 * 1024 + (528 + 16) * 1024  # k_decode + k_combine
TRAFFIC_PREFILL = 24704 * 2.0 * 1024 + 32773 * 1024                          # k_prefill
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix
D = 128


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser(description="One JSON line: configs[1] decode (headline) + configs[2] prefill.")
    ap.add_argument("--gpus", type=int, default=1, help="GPUs (this build measures one)")
    ap.add_argument("--steps", type=int, default=256, help="timed decode steps (one token through 36 layers each)")
    ap.add_argument("--warmup", type=int, default=20, help="untimed decode steps before the timed ones")
    ap.add_argument("--prefill-steps", type=int, default=5, help="timed 36-layer prefill steps of 2048 tokens")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-graph", action="store_true", help="launch the per-layer kernels eagerly")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the parity-case shapes reported beside the headline (configs[3], configs[4] contiguous "
                         "and paged, configs[2] in 512-token chunks)")
    ap.add_argument("--only", choices=["decode", "decode-groups", "prefill", "prefill-chunked", "prefill-groups",
                                       "longctx", "batched", "batched-paged"], default=None,
                    help="run one workload and print its result (decode: the headline line without prefill and extras; "
                         "decode-groups / prefill-groups: the dense Qwen3 GQA group sizes)")
    ap.add_argument("--calib-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB (counter calibration) and exit")
    return ap.parse_args()


# ---------------------------------------------------------------- helpers
class Timer:
    """HIP events on the stream the kernels are launched on (torch's current stream)."""

    def __init__(self, torch):
        self.torch = torch
        self.a = torch.cuda.Event(enable_timing=True)
        self.b = torch.cuda.Event(enable_timing=True)

    def start(self):
        self.a.record()

    def stop_ms(self) -> float:
        self.b.record()
        self.b.synchronize()
        return self.a.elapsed_time(self.b)


def graph_ms(torch, fn, reps: int = 20, warm: int = 3) -> float:
    """Average time of fn() replayed as one HIP graph, measured with events on the stream
    the graph runs on (the launches inside fn go to torch's current stream)."""
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # first launches load code objects outside the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(warm):
        g.replay()
    t = Timer(torch)
    t.start()
    for _ in range(reps):
        g.replay()
    return t.stop_ms() / reps


# ---------------------------------------------------------------- decode
def bench_decode(torch, A, H, HKV, n_layer, ctx, steps, warmup, use_graph, spike_every=0, seed=1000):
    shape = A.AttnShape(H, HKV)
    dev = "cuda"
    kd = HKV * D
    kc = torch.empty((n_layer, ctx, kd), dtype=torch.float32, device=dev)
    vc = torch.empty_like(kc)
    for l in range(n_layer):
        A.synth_fill(kc[l], seed + 2 * l, row_len=kd, spike_every=spike_every, spike_mult=4.0)
        A.synth_fill(vc[l], seed + 2 * l + 1)
    qkv = A.synth_fill(torch.empty((n_layer, 1, shape.qkv), dtype=torch.float32, device=dev), seed + 999)
    gam = torch.empty((n_layer, 2, D), dtype=torch.float32, device=dev)
    A.synth_fill(gam, seed + 777)
    gam.mul_(0.1).add_(1.0)
    cs = A.rope_table(ctx, device=dev)
    pos_dev = torch.tensor([ctx - 1], dtype=torch.int32, device=dev)
    out = torch.empty((n_layer, 1, H, D), dtype=torch.float32, device=dev)
    ws = [A.DecodeWorkspace(1, H, HKV, ctx, device=dev) for _ in range(n_layer)]

    def layer(l):
        A.decode_step(qkv[l], kc[l], vc[l], shape, gam[l, 0], gam[l, 1], cs, ws[l], pos_dev=pos_dev, out=out[l])

    def step():
        for l in range(n_layer):
            layer(l)

    torch.cuda.synchronize()
    graph = None
    if use_graph:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()  # warm: first launches load code objects outside the capture
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        torch.cuda.synchronize()

    run = graph.replay if graph is not None else step
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    t = Timer(torch)
    t.start()
    for _ in range(steps):
        run()
    ms = t.stop_ms() / steps
    kern_ms = ms / n_layer  # the step is n_layer back-to-back launches of the one kernel
    bytes_layer = A.decode_bytes(ctx, H, HKV)
    return {
        "ms_per_step": ms,
        "bytes_per_step": bytes_layer * n_layer,
        "gbs": bytes_layer * n_layer / (ms * 1e-3) / 1e9,
        "kernel_ms": kern_ms,
        "kernel_gbs": bytes_layer / (kern_ms * 1e-3) / 1e9,
        "bytes_per_launch": bytes_layer,
        "graph": graph is not None,
    }


def bench_batched(torch, A, steps, warmup, use_graph, seed=3000, block_size=0):
    """1.7B shape, 64 sequences with kv_len ~ U[256, 8192], 28 layers.  block_size > 0: the same
    sequences in a paged pool (shuffled blocks of block_size rows, fused paged step)."""
    import numpy as np
    H, HKV, n_layer, nseq = 16, 8, 28, 64
    shape = A.AttnShape(H, HKV)
    rng = np.random.default_rng(seed)
    lens = rng.integers(256, 8193, nseq).astype(np.int32)
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
    rows = int(lens.sum())
    kd = HKV * D
    dev = "cuda"
    if block_size:
        rows = sum(-(-int(n) // block_size) for n in lens) * block_size
    kc = torch.empty((n_layer, rows, kd), dtype=torch.float32, device=dev)
    vc = torch.empty_like(kc)
    for l in range(n_layer):
        A.synth_fill(kc[l], seed + 2 * l)
        A.synth_fill(vc[l], seed + 2 * l + 1)
    qkv = A.synth_fill(torch.empty((n_layer, nseq, shape.qkv), dtype=torch.float32, device=dev), seed + 99)
    gam = torch.ones((2, D), dtype=torch.float32, device=dev)
    cs = A.rope_table(int(lens.max()), device=dev)
    off_d = torch.from_numpy(offs).to(dev)
    len_d = torch.from_numpy(lens).to(dev)
    table_d = None
    if block_size:
        # each sequence's rows in whole blocks; the blocks of all sequences shuffled over the pool
        nblk = [-(-int(n) // block_size) for n in lens]
        perm = rng.permutation(sum(nblk)).astype(np.int32)
        table = np.zeros((nseq, max(nblk)), np.int32)
        k = 0
        for si in range(nseq):
            table[si, :nblk[si]] = perm[k:k + nblk[si]]
            k += nblk[si]
        table_d = torch.from_numpy(table).to(dev)
    out = torch.empty((n_layer, nseq, H, D), dtype=torch.float32, device=dev)
    ws = [A.DecodeWorkspace(nseq, H, HKV, int(lens.max()), device=dev) for _ in range(n_layer)]

    def layer(l):
        if table_d is not None:
            A.decode_step_paged(qkv[l], kc[l], vc[l], table_d, block_size, len_d, shape, gam[0], gam[1], cs, ws[l],
                                out=out[l])
        else:
            A.decode_step(qkv[l], kc[l], vc[l], shape, gam[0], gam[1], cs, ws[l], kv_offset=off_d, kv_len=len_d,
                          out=out[l])

    def step():
        for l in range(n_layer):
            layer(l)

    torch.cuda.synchronize()
    graph = None
    if use_graph:
        step()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
    run = graph.replay if graph is not None else step
    for _ in range(warmup):
        run()
    t = Timer(torch)
    t.start()
    for _ in range(steps):
        run()
    ms = t.stop_ms() / steps
    bytes_layer = sum(A.decode_bytes(int(x), H, HKV) for x in lens)
    kern_ms = ms / n_layer
    return {"ms_per_step": ms, "gbs": bytes_layer * n_layer / (ms * 1e-3) / 1e9, "kernel_ms": kern_ms,
            "kernel_gbs": bytes_layer / (kern_ms * 1e-3) / 1e9, "bytes_per_launch": bytes_layer,
            "sum_kv_len": int(lens.sum()), "block_size": block_size}


# ---------------------------------------------------------------- prefill
def bench_prefill(torch, A, H, HKV, n_layer, T, steps, warmup, seed=2000):
    shape = A.AttnShape(H, HKV)
    dev = "cuda"
    kd = HKV * D
    qkv_src = A.synth_fill(torch.empty((n_layer, T, shape.qkv), dtype=torch.float32, device=dev), seed)
    qkv = torch.empty_like(qkv_src)
    kc = torch.empty((n_layer, T, kd), dtype=torch.float32, device=dev)
    vc = torch.empty_like(kc)
    gam = torch.empty((n_layer, 2, D), dtype=torch.float32, device=dev)
    A.synth_fill(gam, seed + 1)
    gam.mul_(0.1).add_(1.0)
    cs = A.rope_table(T, device=dev)
    pos_dev = torch.zeros(1, dtype=torch.int32, device=dev)
    out = torch.empty((n_layer, T, H, D), dtype=torch.float32, device=dev)
    ws = A.PrefillWorkspace(T, H, HKV, T)

    def attn(l):  # the attention kernel alone, on rows the prologue has normed
        A.attn_prefill(qkv[l], kc[l], vc[l], pos_dev, shape, B=T, out=out[l])

    def step():  # per layer: key prologue (norm + RoPE + append), attention with q normed in-kernel
        for l in range(n_layer):
            A.prefill_step(qkv[l], kc[l], vc[l], shape, gam[l, 0], gam[l, 1], cs, pos_dev, ws, B=T, out=out[l])

    qkv.copy_(qkv_src)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t = Timer(torch)
    tot = 0.0
    for _ in range(steps):
        qkv.copy_(qkv_src)  # the prologue normalises in place: restore raw projections (untimed)
        t.start()
        step()
        tot += t.stop_ms()
    ms = tot / steps
    flops_layer = A.flops_causal(T, 0, H)
    # the dominant kernel alone: n_layer attention launches in one graph, on q rows normed by
    # the full prologue (the same contraction the fused step runs; it also norms q as it stages it)
    qkv.copy_(qkv_src)
    for l in range(n_layer):
        A.qkv_prepare(qkv[l], shape, gam[l, 0], gam[l, 1], cs, pos_dev, kc[l], vc[l])
    kern_ms = graph_ms(torch, lambda: [attn(l) for l in range(n_layer)], reps=5, warm=1) / n_layer
    return {"ms_per_step": ms, "tflops": flops_layer * n_layer / (ms * 1e-3) / 1e12, "kernel_ms": kern_ms,
            "kernel_tflops": flops_layer / (kern_ms * 1e-3) / 1e12, "flops_per_launch": flops_layer}


def bench_prefill_chunked(torch, A, H, HKV, n_layer, T, chunk, split=True, seed=2100, step=False):
    """configs[2]'s prompt as the reference engine feeds it: chunks of `chunk` tokens at pos0 = 0, chunk, ...
    (src/cuda/model_cuda.cu:1912 caps a prefill chunk at 512).  Attention launches only, one graph; with
    step=True the engine's whole chunk path instead (ei_prefill_step: key prologue + attention with q normed
    in-kernel; replays re-norm the K heads in place, which keeps them bounded)."""
    shape = A.AttnShape(H, HKV)
    dev = "cuda"
    kd = HKV * D
    q = A.synth_fill(torch.empty((n_layer, T, shape.qkv), dtype=torch.float32, device=dev), seed)
    kc = A.synth_fill(torch.empty((n_layer, T, kd), dtype=torch.float32, device=dev), seed + 1)
    vc = A.synth_fill(torch.empty((n_layer, T, kd), dtype=torch.float32, device=dev), seed + 2)
    out = torch.empty((n_layer, T, H, D), dtype=torch.float32, device=dev)
    starts = list(range(0, T, chunk))
    pos = [torch.tensor([s], dtype=torch.int32, device=dev) for s in starts]
    ws = A.PrefillWorkspace(chunk, H, HKV, T) if split else None  # the engine's path: key split for short chunks
    gam = torch.ones((2, D), dtype=torch.float32, device=dev)
    cs = A.rope_table(T, device=dev) if step else None

    def run():
        for l in range(n_layer):
            for s, p in zip(starts, pos):
                n = min(chunk, T - s)
                if step:
                    A.prefill_step(q[l, s:s + n], kc[l], vc[l], shape, gam[0], gam[1], cs, p, ws, B=n,
                                   out=out[l, s:s + n])
                else:
                    A.attn_prefill(q[l, s:s + n], kc[l], vc[l], p, shape, B=n, out=out[l, s:s + n], ws=ws)

    ms = graph_ms(torch, run, reps=5, warm=1) / n_layer
    flops = A.flops_causal(T, 0, H)
    key = "step_ms_per_layer" if step else "kernel_ms_per_layer"
    return {"chunk": chunk, "key_split": split, key: ms, key.replace("ms_per_layer", "tflops"): flops / (ms * 1e-3) / 1e12}


# ---------------------------------------------------------------- CPU baseline
def cpu_baseline(budget_s: float = 12.0):
    """Reference CPU attention loop (oracle restatement of src/model.cpp:191-214, OpenMP over
    heads) on configs[1]'s shape: decode layers with ctx 4096 until the time budget is spent."""
    import numpy as np
    from oracle import oracle as O
    cores = min(int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1), 64)
    O.set_threads(cores)
    H, HKV, T = 32, 8, 4096
    k = O.normal((T, HKV, D), 1)
    v = O.normal((T, HKV, D), 2)
    q = O.normal((H, D), 3)
    O.attn_decode(q, k, v, T, H, HKV, D)  # warm
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s or n < 3:
        O.attn_decode(q, k, v, T, H, HKV, D)
        n += 1
    dt = (time.perf_counter() - t0) / n
    gbs = (4.0 * (2 * T * HKV * D + 2 * H * D)) / dt / 1e9
    _ = np
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"{n} single-layer decode steps at configs[1] shape (H32/HKV8, ctx 4096), "
                      f"{dt * 1e3:.2f} ms per layer, {dt * 36 * 1e3:.1f} ms per 36-layer token"}


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the attention path has no multi-GPU leg in this build "
              "(one process per GPU would shard decode by KV head and prefill by head); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    from exactinfer_amd import build as B
    B.ensure_built()  # builds only when nothing is built
    from exactinfer_amd import attention as A
    if not torch.cuda.is_available():
        sys.exit("bench.py needs a GPU")
    if args.calib_copy:
        n = args.calib_copy * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calib_copy_bytes": n * 4}))
        return
    use_graph = not args.no_graph
    res = {}
    if args.only in (None, "decode"):
        log("decode configs[1] ...")
        res["decode"] = bench_decode(torch, A, 32, 8, 36, 4096, args.steps, args.warmup, use_graph)
        log(json.dumps(res["decode"]))
    if args.only in (None, "prefill"):
        log("prefill configs[2] ...")
        res["prefill"] = bench_prefill(torch, A, 32, 8, 36, 2048, args.prefill_steps, 1)
        log(json.dumps(res["prefill"]))
    extra = args.only is None and not args.no_extra
    if extra or args.only == "prefill-chunked":
        log("prefill configs[2] in 512-token chunks ...")
        res["prefill_chunked"] = bench_prefill_chunked(torch, A, 32, 8, 36, 2048, 512)
        res["prefill_chunked"].update(bench_prefill_chunked(torch, A, 32, 8, 36, 2048, 512, step=True))
        log(json.dumps(res["prefill_chunked"]))
        log(json.dumps(bench_prefill_chunked(torch, A, 32, 8, 36, 2048, 512, split=False)))
    if args.only == "decode-groups":  # configs[1]'s decode at the other dense Qwen3 group sizes
        res["decode_groups"] = {}
        for H, HKV in ((16, 8), (32, 8), (40, 8), (64, 8)):
            r = bench_decode(torch, A, H, HKV, 36, 4096, args.steps, args.warmup, use_graph, seed=5000 + H)
            res["decode_groups"][f"H{H}/HKV{HKV}"] = r
            log(f"H{H}/HKV{HKV}: " + json.dumps(r))
    if args.only == "prefill-groups":  # GQA group sizes of the dense Qwen3 family, T = 2048 in one chunk
        res["prefill_groups"] = {}
        for H, HKV in ((16, 8), (32, 8), (40, 8), (64, 8), (8, 8)):
            r = bench_prefill_chunked(torch, A, H, HKV, 8, 2048, 2048, seed=2200 + H)
            res["prefill_groups"][f"H{H}/HKV{HKV}"] = r
            log(f"H{H}/HKV{HKV}: " + json.dumps(r))
    if extra or args.only == "longctx":
        log("long-context decode configs[3] ...")
        res["longctx"] = bench_decode(torch, A, 16, 8, 28, 32768, max(8, args.steps // 8), 3, use_graph,
                                      spike_every=512, seed=4000)
        log(json.dumps(res["longctx"]))
    if extra or args.only == "batched":
        log("batched ragged decode configs[4] ...")
        res["batched"] = bench_batched(torch, A, 128 if args.steps >= 128 else args.steps, 3, use_graph)
        log(json.dumps(res["batched"]))
    if extra or args.only == "batched-paged":
        log("batched ragged decode configs[4], paged KV (64-row blocks, shuffled) ...")
        res["batched_paged"] = bench_batched(torch, A, 128 if args.steps >= 128 else args.steps, 3, use_graph,
                                             block_size=64)
        log(json.dumps(res["batched_paged"]))
    if args.only not in (None, "decode"):
        print(json.dumps(res))
        return
    cpu = None if args.no_cpu else cpu_baseline()
    dec, pre = res["decode"], res.get("prefill")
    line = {
        "metric": "attn decode GB/s (% of HBM peak) @4B ctx4096; causal prefill attn TFLOP/s",
        "value": round(dec["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded counter-based N(0,1) Q/K/V and KV caches, gamma = 1 + 0.1 N(0,1))",
        "config": {"workload": "configs[1]: Qwen3-4B-shape decode attention, batch 1, H32/HKV8/D128, 36 layers, "
                               "ctx 4096 per layer, fused QK-norm+RoPE+append+split-K attention per layer, "
                               "36 launches per step in one HIP graph" if dec["graph"] else "eager launches",
                   "pct_hbm_peak": round(100 * dec["gbs"] / HBM_PEAK_GBS, 2)},
        "roofline": {"bound": "hbm", "achieved": round(dec["kernel_gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dec["kernel_gbs"] / HBM_PEAK_GBS, 4), "traffic": TRAFFIC_DECODE_PER_LAYER,
                     "kernel": "k_decode<4,true,8> + k_combine<4> (one layer)", "kernel_us": round(dec["kernel_ms"] * 1e3, 3),
                     "bytes_per_launch": dec["bytes_per_launch"]},
        "cpu_baseline": cpu,
    }
    if pre is not None:
        line["prefill"] = {"workload": "configs[2]: Qwen3-4B-shape causal prefill, T=2048, 36 layers, per layer "
                                       "ei_prefill_step: key prologue (QK-norm + RoPE + append) + k_prefill "
                                       "(fp32 MFMA; q QK-norm + RoPE in-kernel)",
                           "tflops": round(pre["tflops"], 3), "ms_per_step": round(pre["ms_per_step"], 4),
                           "roofline": {"bound": "mfma", "achieved": round(pre["kernel_tflops"], 3),
                                        "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                                        "frac": round(pre["kernel_tflops"] / FP32_MFMA_PEAK_TFLOPS, 4),
                                        "traffic": TRAFFIC_PREFILL, "kernel": "k_prefill<false> (q normed beforehand)",
                                        "kernel_us": round(pre["kernel_ms"] * 1e3, 2),
                                        "flops_per_launch": pre["flops_per_launch"]}}
    # the other configs (parity-test shapes), measured beside the headline for context
    ex = {}
    for k in ("longctx", "batched", "batched_paged", "prefill_chunked"):
        if k in res:
            ex[k] = {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in res[k].items()}
            if "gbs" in res[k]:
                ex[k]["pct_hbm_peak"] = round(100 * res[k]["gbs"] / HBM_PEAK_GBS, 2)
    if ex:
        line["extra"] = ex
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
