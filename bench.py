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
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix
D = 128
PROFILES = ROOT / "profiles"


def profile_traffic(name: str):
    """HBM bytes per launch recorded in a committed rocprofv3 summary (profiles/<name>): the line
    `traffic_bytes_per_launch: N` holds FETCH_SIZE and WRITE_SIZE per dispatch, each scaled by
    the factor a plain copy of known size needs.  None when the summary or the line is absent."""
    import re
    f = PROFILES / name
    if not f.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.]+)", f.read_text())
    return float(m.group(1)) if m else None


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
                                       "longctx", "batched", "batched-paged", "stream-ceiling", "read-ceiling", "configs0",
                                       "project"],
                    default=None,
                    help="run one workload and print its result (decode: the headline line without prefill and extras; "
                         "decode-groups / prefill-groups: the dense Qwen3 GQA group sizes)")
    ap.add_argument("--read-ceiling-sizes", action="store_true",
                    help="with --only read-ceiling: also the per-launch sizes of the projection and prefill kernels")
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


def bench_stream_ceiling(torch, A, H, HKV, n_layer, ctx, reps=50, seed=1000):
    """The decode plan's memory traffic alone (ei_stream_ceiling): n_layer launches over separate
    caches of ctx positions in one graph, the same grid and DMA pattern as the decode."""
    from exactinfer_amd import _capi
    dev = "cuda"
    kd = HKV * D
    kc = torch.empty((n_layer, ctx, kd), dtype=torch.float32, device=dev)
    vc = torch.empty_like(kc)
    for l in range(n_layer):
        A.synth_fill(kc[l], seed + 2 * l)
        A.synth_fill(vc[l], seed + 2 * l + 1)
    sink = torch.empty((HKV * 256,), dtype=torch.float32, device=dev)

    def run():
        for l in range(n_layer):
            _capi.call("ei_stream_ceiling", A._stream(), kc[l].data_ptr(), vc[l].data_ptr(), HKV, ctx, sink.data_ptr())

    ms = graph_ms(torch, run, reps=reps, warm=5) / n_layer
    kv_bytes = 2.0 * ctx * kd * 4
    return {"kernel_ms": ms, "kv_bytes_per_launch": kv_bytes, "gbs": kv_bytes / (ms * 1e-3) / 1e9,
            "decode_bytes_per_launch": A.decode_bytes(ctx, H, HKV)}


def bench_read_ceiling(torch, A, nbytes=2 * 4096 * 8 * D * 4, n_layer=36, reps=50, seed=1000):
    """The read ceiling of one decode launch's bytes (ei_read_ceiling): n_layer launches, each a plain
    non-temporal streaming read of its own nbytes buffer (configs[1]'s K+V per layer by default: no
    launch finds its bytes in a cache), replayed as one graph, for 128, 256, 512 and 1024 workgroups
    of 256 threads (2048 or 4096 where 1024 would need over 64 loads per thread), each with the loads
    interleaved with their uses by the compiler and with every load issued first.  Returns each
    variant's time per launch and the best."""
    from exactinfer_amd import _capi
    dev = "cuda"
    buf = torch.empty((n_layer, nbytes // 4), dtype=torch.float32, device=dev)
    for l in range(n_layer):
        A.synth_fill(buf[l], seed + l)
    sink = torch.empty((4096 * 4,), dtype=torch.float32, device=dev)
    res = {"bytes_per_launch": nbytes, "launches_per_graph": n_layer}
    best = None
    for n_wg in (128, 256, 512, 1024, 2048, 4096):
        per_thread = -(-nbytes // (n_wg * 256 * 16))  # 16-byte loads per thread
        if n_wg > 1024 and nbytes <= 1024 * 256 * 64 * 16:
            break
        if per_thread > 64:
            continue
        for all_in_flight in (0, 1):  # loads interleaved with their uses by the compiler, or all issued first
            if all_in_flight and per_thread > 32 and n_wg != 128:
                continue

            def run():
                for l in range(n_layer):
                    _capi.call("ei_read_ceiling", A._stream(), buf[l].data_ptr(), nbytes, n_wg, all_in_flight,
                               sink.data_ptr())

            ms = graph_ms(torch, run, reps=reps, warm=5) / n_layer
            gbs = nbytes / (ms * 1e-3) / 1e9
            res[f"wg{n_wg}" + ("_all" if all_in_flight else "")] = {"kernel_us": round(ms * 1e3, 3),
                                                                   "gbs": round(gbs, 1)}
            if best is None or gbs > best[1]:
                best = (f"{n_wg}" + (" all loads in flight" if all_in_flight else ""), gbs, ms)
    res.update({"best_grid": best[0], "kernel_us": round(best[2] * 1e3, 3), "gbs": best[1]})
    del buf
    return res


def bench_project(torch, A, E=2560, H=32, HKV=8, n_layer=36, seed=7000):
    """The decode step's QKV projection at Qwen3-4B shape (ei_qkv_project: attention RMSNorm + the
    fused [Wq|Wk|Wv] GEMV, one token): n_layer launches over separate weights in one graph, for fp32
    and fp16 weights and Q8_0 / Q4_K / Q6_K blocks; GB/s of the weight stream + x + out.  Then the whole decode layer from the
    residual (projection + fused decode step, ctx 4096) per layer."""
    import numpy as np
    from exactinfer_amd import _capi
    dev = "cuda"
    shape = A.AttnShape(H, HKV)
    n_out = shape.qkv
    x = A.synth_fill(torch.empty((n_layer, 1, E), dtype=torch.float32, device=dev), seed)
    gam = torch.ones((E,), dtype=torch.float32, device=dev)
    qkv = torch.empty((n_layer, 1, n_out), dtype=torch.float32, device=dev)
    res = {"workload": f"Qwen3-4B shape: E {E}, {n_out} output rows, one token, {n_layer} layers in one graph"}
    for wtype, name, esize in ((0, "f32", 4), (1, "f16", 2)):
        w = torch.empty((n_layer, n_out, E), dtype=torch.float32, device=dev)
        A.synth_fill(w, seed + 1 + wtype)
        w.mul_(0.05)
        if wtype == 1:
            w = w.to(torch.float16)

        def run():
            for l in range(n_layer):
                _capi.call("ei_qkv_project", A._stream(), x[l].data_ptr(), E, 1, E, gam.data_ptr(), 1e-6,
                           w[l].data_ptr(), wtype, n_out, qkv[l].data_ptr(), n_out)

        ms = graph_ms(torch, run, reps=20, warm=3) / n_layer
        nbytes = n_out * E * esize + 4.0 * (E + n_out)
        res[name] = {"kernel_us": round(ms * 1e3, 3), "bytes_per_launch": nbytes,
                     "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                     "pct_hbm_peak": round(100 * nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2)}
        if wtype == 1:  # the decode layer from the residual: projection + fused decode step at ctx 4096
            ctx = 4096
            kc = torch.empty((n_layer, ctx, HKV * D), dtype=torch.float32, device=dev)
            vc = torch.empty_like(kc)
            for l in range(n_layer):
                A.synth_fill(kc[l], seed + 10 + 2 * l)
                A.synth_fill(vc[l], seed + 11 + 2 * l)
            g2 = torch.ones((2, D), dtype=torch.float32, device=dev)
            cs = A.rope_table(ctx)
            pos = torch.tensor([ctx - 1], dtype=torch.int32, device=dev)
            out = torch.empty((n_layer, 1, H, D), dtype=torch.float32, device=dev)
            ws = [A.DecodeWorkspace(1, H, HKV, ctx) for _ in range(n_layer)]

            def layer_run():
                for l in range(n_layer):
                    _capi.call("ei_qkv_project", A._stream(), x[l].data_ptr(), E, 1, E, gam.data_ptr(), 1e-6,
                               w[l].data_ptr(), wtype, n_out, qkv[l].data_ptr(), n_out)
                    A.decode_step(qkv[l], kc[l], vc[l], shape, g2[0], g2[1], cs, ws[l], pos_dev=pos, out=out[l])

            ms2 = graph_ms(torch, layer_run, reps=20, warm=3) / n_layer
            tot = nbytes + A.decode_bytes(ctx, H, HKV)
            res["decode_layer_from_residual_f16"] = {"us_per_layer": round(ms2 * 1e3, 3), "bytes": tot,
                                                     "gbs": round(tot / (ms2 * 1e-3) / 1e9, 1)}
        del w
    # quantised rows in their GGUF block layout: random bytes, block scales set to small finite values
    qfmt = {8: ("q8_0", 32, 34, (0,)), 12: ("q4_k", 256, 144, (0, 2)), 14: ("q6_k", 256, 210, (208,))}
    dbytes = torch.tensor(list(np.array([0.01], np.float16).view(np.uint8)), dtype=torch.uint8, device=dev)
    for wtype, (name, vals, bb, d_offs) in qfmt.items():
        rb = E // vals * bb
        g = torch.Generator(device=dev)
        g.manual_seed(seed + wtype)
        w = torch.randint(0, 256, (n_layer, n_out * rb), dtype=torch.uint8, device=dev, generator=g)
        blk = w.view(-1, bb)
        for off in d_offs:
            blk[:, off:off + 2] = dbytes

        def run_q():
            for l in range(n_layer):
                _capi.call("ei_qkv_project", A._stream(), x[l].data_ptr(), E, 1, E, gam.data_ptr(), 1e-6,
                           w[l].data_ptr(), wtype, n_out, qkv[l].data_ptr(), n_out)

        ms = graph_ms(torch, run_q, reps=20, warm=3) / n_layer
        nbytes = n_out * rb + 4.0 * (E + n_out)
        res[name] = {"kernel_us": round(ms * 1e3, 3), "bytes_per_launch": nbytes,
                     "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                     "pct_hbm_peak": round(100 * nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2)}
        del w, blk
    return res


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
        qkv.copy_(qkv_src)  # the prologue normalises the K heads in place: restore raw projections (untimed)
        t.start()
        step()
        tot += t.stop_ms()
    ms = tot / steps
    flops_layer = A.flops_causal(T, 0, H)
    # the step's two kernels per layer (key prologue + k_prefill<true>) replayed as one graph of
    # n_layer steps; replays re-norm the already normed K heads in place, which keeps them bounded
    # and runs the same arithmetic
    qkv.copy_(qkv_src)
    step_layer_ms = graph_ms(torch, step, reps=max(steps, 3), warm=1) / n_layer
    # the attention kernel without the q norm (k_prefill<false>), on q rows the full prologue normed
    qkv.copy_(qkv_src)
    for l in range(n_layer):
        A.qkv_prepare(qkv[l], shape, gam[l, 0], gam[l, 1], cs, pos_dev, kc[l], vc[l])
    plain_ms = graph_ms(torch, lambda: [attn(l) for l in range(n_layer)], reps=5, warm=1) / n_layer
    return {"ms_per_step": ms, "tflops": flops_layer * n_layer / (ms * 1e-3) / 1e12,
            "step_layer_ms": step_layer_ms, "step_layer_tflops": flops_layer / (step_layer_ms * 1e-3) / 1e12,
            "plain_kernel_ms": plain_ms, "plain_kernel_tflops": flops_layer / (plain_ms * 1e-3) / 1e12,
            "flops_per_launch": flops_layer}


def bench_prefill_chunked(torch, A, H, HKV, n_layer, T, chunk, split=True, seed=2100, step=False, block_size=0):
    """configs[2]'s prompt as the reference engine feeds it: chunks of `chunk` tokens at pos0 = 0, chunk, ...
    (src/cuda/model_cuda.cu:1912 caps a prefill chunk at 512).  Attention launches only, one graph; with
    step=True the engine's whole chunk path instead (ei_prefill_step: key prologue + attention with q normed
    in-kernel; replays re-norm the K heads in place, which keeps them bounded).  block_size > 0: the
    step over a paged pool (each layer's cache rows in shuffled blocks of block_size rows,
    ei_prefill_step_paged)."""
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
    tables = None
    if block_size:
        import numpy as np
        rng = np.random.default_rng(seed + 7)
        tables = [torch.from_numpy(rng.permutation(T // block_size).astype(np.int32)).to(dev) for _ in range(n_layer)]

    def run():
        for l in range(n_layer):
            for s, p in zip(starts, pos):
                n = min(chunk, T - s)
                if step:
                    A.prefill_step(q[l, s:s + n], kc[l], vc[l], shape, gam[0], gam[1], cs, p, ws, B=n,
                                   out=out[l, s:s + n], block_table=None if tables is None else tables[l],
                                   block_size=block_size)
                else:
                    A.attn_prefill(q[l, s:s + n], kc[l], vc[l], p, shape, B=n, out=out[l, s:s + n], ws=ws)

    ms = graph_ms(torch, run, reps=5, warm=1) / n_layer
    flops = A.flops_causal(T, 0, H)
    key = ("paged_step_ms_per_layer" if block_size else "step_ms_per_layer") if step else "kernel_ms_per_layer"
    return {"chunk": chunk, "key_split": split, key: ms, key.replace("ms_per_layer", "tflops"): flops / (ms * 1e-3) / 1e12}


# ---------------------------------------------------------------- CPU baseline
def cpu_info():
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return model, os.cpu_count() or 1


def cpu_baseline(budget_s: float = 10.0):
    """The reference CPU attention (the oracle's restatement of src/model.cpp:191-214, one token at
    a time as src/model.cpp:138-140 runs it, OpenMP over query heads) on this host:
    - the headline value: decode layers at configs[1]'s shape (H32/HKV8, ctx 4096) for ~budget_s;
    - one 0.6B-shape layer (H16/HKV8), 512 prompt tokens then 128 decode steps;
    - configs[2]'s prefill (H32/HKV8, 2048 tokens), timed on every 16th row and scaled by FLOPs."""
    import numpy as np
    from exactinfer_amd import attention as A
    from oracle import oracle as O
    cores = min(int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1), 64)
    O.set_threads(cores)
    model, nproc = cpu_info()
    # configs[1] decode
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
    gbs = A.decode_bytes(T, H, HKV) / dt / 1e9
    # prompt of 512 tokens then 128 decode steps, one token at a time
    H0, HKV0, P, G0 = 16, 8, 512, 128
    k0 = O.normal((P + G0, HKV0, D), 11)
    v0 = O.normal((P + G0, HKV0, D), 12)
    q0 = O.normal((P + G0, H0, D), 13)
    t0 = time.perf_counter()
    for t in range(P):
        O.attn_decode(q0[t], k0, v0, t + 1, H0, HKV0, D)
    t_pre = time.perf_counter() - t0
    t0 = time.perf_counter()
    for t in range(P, P + G0):
        O.attn_decode(q0[t], k0, v0, t + 1, H0, HKV0, D)
    t_dec = time.perf_counter() - t0
    dec_bytes0 = sum(A.decode_bytes(t + 1, H0, HKV0) for t in range(P, P + G0))
    # configs[2] prefill on a row sample, scaled by the FLOPs of the rows timed
    H2, HKV2, T2, stride = 32, 8, 2048, 16
    k2 = O.normal((T2, HKV2, D), 21)
    v2 = O.normal((T2, HKV2, D), 22)
    q2 = O.normal((T2 // stride, H2, D), 23)
    rows = list(range(stride - 1, T2, stride))
    t0 = time.perf_counter()
    for i, b in enumerate(rows):
        O.attn_decode(q2[i], k2, v2, b + 1, H2, HKV2, D)
    t_rows = time.perf_counter() - t0
    flops_rows = sum(4.0 * D * (b + 1) * H2 for b in rows)
    pre_tflops = flops_rows / t_rows / 1e12
    _ = np
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "cpu_model": model, "nproc": nproc,
            "sample": f"{n} single-layer decode steps at configs[1] shape (H32/HKV8, ctx 4096), "
                      f"{dt * 1e3:.2f} ms per layer, {dt * 36 * 1e3:.1f} ms per 36-layer token",
            "configs0": {"workload": "Qwen3-0.6B shape H16/HKV8, one layer: 512 prompt tokens then 128 decode steps, "
                                     "one token at a time (src/model.cpp:138-140)",
                         "prefill_ms": round(t_pre * 1e3, 2), "prefill_tok_s": round(P / t_pre, 1),
                         "prefill_tflops": round(A.flops_causal(P, 0, H0) / t_pre / 1e12, 5),
                         "decode_ms": round(t_dec * 1e3, 2), "decode_tok_s": round(G0 / t_dec, 1),
                         "decode_gbs": round(dec_bytes0 / t_dec / 1e9, 3)},
            "prefill_configs2": {"workload": "H32/HKV8, 2048-token causal prefill, one token at a time; every 16th "
                                             "row timed and scaled by the FLOPs of the rows timed",
                                 "tflops": round(pre_tflops, 5),
                                 "ms_per_layer_scaled": round(A.flops_causal(T2, 0, H2) / (pre_tflops * 1e12) * 1e3,
                                                              1)}}


def bench_configs0_gpu(torch, A):
    """configs[0] on the GPU path: one 0.6B-shape layer, the 512-token prompt as one fused prefill
    step, then 128 fused decode steps (each appends one row), timed with HIP events."""
    H, HKV, P, G = 16, 8, 512, 128
    shape = A.AttnShape(H, HKV)
    dev = "cuda"
    n_ctx = P + G
    qkv = A.synth_fill(torch.empty((n_ctx, shape.qkv), dtype=torch.float32, device=dev), 600)
    kc = torch.zeros((n_ctx, HKV * D), dtype=torch.float32, device=dev)
    vc = torch.zeros_like(kc)
    gam = torch.ones((2, D), dtype=torch.float32, device=dev)
    cs = A.rope_table(n_ctx)
    pws = A.PrefillWorkspace(P, H, HKV, n_ctx)
    dws = A.DecodeWorkspace(1, H, HKV, n_ctx)
    pos0 = torch.zeros(1, dtype=torch.int32, device=dev)
    poss = [torch.tensor([t], dtype=torch.int32, device=dev) for t in range(P, n_ctx)]
    src = qkv.clone()

    def run():
        A.prefill_step(qkv[:P], kc, vc, shape, gam[0], gam[1], cs, pos0, pws, B=P)
        for i, t in enumerate(range(P, n_ctx)):
            A.decode_step(qkv[t:t + 1], kc, vc, shape, gam[0], gam[1], cs, dws, pos_dev=poss[i])

    run()
    torch.cuda.synchronize()
    qkv.copy_(src)
    tm = Timer(torch)
    tm.start()
    A.prefill_step(qkv[:P], kc, vc, shape, gam[0], gam[1], cs, pos0, pws, B=P)
    pre_ms = tm.stop_ms()
    tm.start()
    for i, t in enumerate(range(P, n_ctx)):
        A.decode_step(qkv[t:t + 1], kc, vc, shape, gam[0], gam[1], cs, dws, pos_dev=poss[i])
    dec_ms = tm.stop_ms()

    # the same work as HIP graphs, the way an engine replays its steps: the prompt's prefill step as
    # one graph, the 128 decode steps (one fused launch + split merge each, own position word) as another
    def prefill_only():
        A.prefill_step(qkv[:P], kc, vc, shape, gam[0], gam[1], cs, pos0, pws, B=P)

    def decode_all():
        for i, t in enumerate(range(P, n_ctx)):
            A.decode_step(qkv[t:t + 1], kc, vc, shape, gam[0], gam[1], cs, dws, pos_dev=poss[i])

    qkv.copy_(src)
    pre_g = graph_ms(torch, prefill_only, reps=20, warm=2)
    dec_g = graph_ms(torch, decode_all, reps=20, warm=2)
    dec_bytes = sum(A.decode_bytes(t + 1, H, HKV) for t in range(P, n_ctx))
    return {"prefill_ms": pre_ms, "decode_ms_128_steps": dec_ms, "decode_us_per_step": dec_ms * 1e3 / G,
            "note": "eager launches, one layer: launch-latency bound at this size",
            "graph": True, "graph_prefill_ms": pre_g,
            "graph_prefill_tflops": A.flops_causal(P, 0, H) / (pre_g * 1e-3) / 1e12,
            "graph_decode_ms_128_steps": dec_g, "graph_decode_us_per_step": dec_g * 1e3 / G,
            "graph_decode_gbs": dec_bytes / (dec_g * 1e-3) / 1e9}


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the attention path has no multi-GPU leg in this build "
              "(one process per GPU would shard decode by KV head and prefill by head); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    from exactinfer_amd import build as B
    B.ensure_built()  # builds only when nothing is built or a source is newer than the library
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
        res["prefill_chunked"].update(bench_prefill_chunked(torch, A, 32, 8, 36, 2048, 512, step=True, block_size=64))
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
    if extra or args.only == "stream-ceiling":
        log("stream ceiling of the configs[1] decode plan ...")
        res["stream_ceiling"] = bench_stream_ceiling(torch, A, 32, 8, 36, 4096)
        lc = bench_stream_ceiling(torch, A, 16, 8, 28, 32768, reps=10)  # configs[3]'s plan (1024-key chunks)
        res["stream_ceiling"]["longctx"] = {"kernel_ms": round(lc["kernel_ms"], 4), "gbs": round(lc["gbs"], 1),
                                            "pct_hbm_peak": round(100 * lc["gbs"] / HBM_PEAK_GBS, 2)}
        log(json.dumps(res["stream_ceiling"]))
    if args.only in (None, "decode", "read-ceiling"):
        log("read ceiling of configs[1]'s per-layer bytes ...")
        res["read_ceiling"] = bench_read_ceiling(torch, A)
        log(json.dumps(res["read_ceiling"]))
    if args.only == "read-ceiling" and args.read_ceiling_sizes:  # the per-launch sizes of the other kernels
        res["read_ceiling"]["by_size"] = {}
        for mb in (4, 8.9, 12.9, 16.7, 31.5, 67, 134, 268):
            nb = int(mb * 1e6) // 4096 * 4096
            r = bench_read_ceiling(torch, A, nbytes=nb, n_layer=max(4, min(36, int(1.2e9 // nb))), reps=20)
            res["read_ceiling"]["by_size"][f"{nb / 1e6:.1f}MB"] = {k: r[k] for k in ("best_grid", "kernel_us",
                                                                                     "gbs")}
            log(f"{nb / 1e6:.1f} MB: " + json.dumps(r))
    if extra or args.only == "project":
        log("QKV projection at Qwen3-4B shape ...")
        res["project"] = bench_project(torch, A)
        log(json.dumps(res["project"]))
    if extra or args.only == "configs0":
        log("configs[0] on the GPU path ...")
        res["configs0"] = bench_configs0_gpu(torch, A)
        log(json.dumps(res["configs0"]))
    if args.only not in (None, "decode"):
        print(json.dumps(res))
        return
    cpu = None if args.no_cpu else cpu_baseline()
    dec, pre, rc = res["decode"], res.get("prefill"), res["read_ceiling"]
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
                     "frac": round(dec["kernel_gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": profile_traffic("decode_configs1_hbm_traffic.md"),
                     "kernel": "k_decode<4,true,8> + k_combine<4> (one layer, graph-timed)",
                     "kernel_us": round(dec["kernel_ms"] * 1e3, 3), "bytes_per_launch": dec["bytes_per_launch"],
                     # what a plain streaming read of the same K+V bytes per launch reaches (36 launches
                     # in one graph, best of 256/512/1024 workgroups), and this kernel's fraction of it
                     "ceiling_gbs": round(rc["gbs"], 1), "ceiling_us": rc["kernel_us"],
                     "ceiling_frac": round(dec["kernel_gbs"] / rc["gbs"], 4),
                     "ceiling_pct_hbm_peak": round(100 * rc["gbs"] / HBM_PEAK_GBS, 2)},
        "cpu_baseline": cpu,
    }
    if pre is not None:
        line["prefill"] = {"workload": "configs[2]: Qwen3-4B-shape causal prefill, T=2048, 36 layers, per layer "
                                       "ei_prefill_step: key prologue (QK-norm + RoPE + append) + k_prefill "
                                       "(fp32 MFMA; q QK-norm + RoPE in-kernel)",
                           "tflops": round(pre["tflops"], 3), "ms_per_step": round(pre["ms_per_step"], 4),
                           "roofline": {"bound": "mfma", "achieved": round(pre["step_layer_tflops"], 3),
                                        "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                                        "frac": round(pre["step_layer_tflops"] / FP32_MFMA_PEAK_TFLOPS, 4),
                                        "traffic": profile_traffic("prefill_configs2_hbm_traffic.md"),
                                        "kernel": "k_qkv_prepare (key heads) + k_prefill<true> (one layer of the "
                                                  "step, graph-timed)",
                                        "kernel_us": round(pre["step_layer_ms"] * 1e3, 2),
                                        "flops_per_launch": pre["flops_per_launch"],
                                        "plain_kernel": {"kernel": "k_prefill<false> (q normed beforehand)",
                                                         "kernel_us": round(pre["plain_kernel_ms"] * 1e3, 2),
                                                         "tflops": round(pre["plain_kernel_tflops"], 3)}}}
    # the other configs (parity-test shapes), measured beside the headline for context
    ex = {}
    for k in ("longctx", "batched", "batched_paged", "prefill_chunked", "stream_ceiling", "read_ceiling", "configs0",
              "project"):
        if k in res:
            ex[k] = {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in res[k].items()}
            if "gbs" in res[k]:
                ex[k]["pct_hbm_peak"] = round(100 * res[k]["gbs"] / HBM_PEAK_GBS, 2)
    if ex:
        line["extra"] = ex
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
