#!/usr/bin/env python3
"""Benchmark of the expert dequant-matmul path on one MI355X.

Headline (value): routed-expert decode matvec, IQ3_S, 256 experts top-8 of Zipf(1.1) routing, gate/up 1536 x 4096
and down 4096 x 1536 with the SwiGLU between them, float16 activations, batch 1. A step is one decode pass of the
batch through 16 distinct routed-expert layers (about 1 GB of expert bytes, four times the 256 MB MALL), each a
BlockSwitchGLU call as the engine makes it (the gate+up+SwiGLU launch, then the down launch), captured once as a HIP
graph and replayed. value = algorithmic bytes / time: the distinct experts' packed bytes plus activations in and out
(x, h written and read, y). one_launch: the same layers as one launch each (gate, up, SwiGLU and down:
strata_expert_layer).

Beside it, on the same line, the other workloads of the path:
  decode_t4      the same at 4 tokens (two launches a layer)
  speculate      the same layer in Q2_0, 5 rows (1 + 4 draft tokens), 16 layers
  q4k_matvec     one Q4_K 4096 x 4096 matrix, float32 x, batch 1 (graphs of 64 distinct copies), and its CPU path
  prompt         512-token prompt chunk, IQ3_XXS, 256 experts top-8, bfloat16: tiles on the GPU, the fused
                 gate/up/SwiGLU and scatter-down MFMA kernels; TFLOPS over the real pairs' 2 * pairs * 3 * H * F
  prompt_q2_0    the same chunk in Q2_0 blocks
  dense_decode   the dense half of a mixed-model decode token: q, k, v 4096 x 4096 Q6_K fused into one launch, o
                 Q8_0, the shared expert's Q4_K gate and up 1536 x 4096 with the SwiGLU in one launch and its
                 down 4096 x 1536, lm_head 151936 x 4096 Q6_K, one float16 token each (graphs over copies, at least
                 1 GB and 8 copies a graph, so that a replay's start spreads over 8 launches or more);
                 shared_in_routed: the shared expert's gate and up taken by the headline layers' routed gate+up
                 launches instead (its marginal time over those launches alone);
                 shared_down_in_routed: its down taken by the layers' routed down launches the same way
  moe_block      one decode token through whole MoE blocks (fused.RoutedMoE: router, top-8, routed experts, the
                 shared expert riding in the routed launches, its gate, the combine): us a block and GB/s
  prefill        a 2048-token prefill of the mixed model, bfloat16: the routed IQ3_S experts through the tiles and
                 the dense layers dequantized for the chunk and multiplied by the library product, TFLOPS
  roofline       the dominant kernel (the gate+up+SwiGLU launch): algorithmic bytes per launch / its mean duration
                 (HIP events around a graph of those launches only, on the stream they run on), against 8 TB/s
  cpu_baseline   the oracle's numpy decode of the touched experts (one thread) + float32 matvecs (BLAS on the
                 host's cores) on a few layers of the headline workload; q4k_matvec carries its own

--dense prints only dense_decode as its own line; --only NAME one other sub-workload (prompt, prompt_q2_0, prefill
with two IQ3_S layers, q4k); --prefill-tokens N the prefill's prompt length (2048; at 4096 and more, eight tiles
an expert or more, the experts' full chunks of 16 tiles take the wide form).
"""

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

E, H, F, K = 256, 4096, 1536, 8
VOCAB = 151936
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=16)
    ap.add_argument("--tokens", type=int, default=1)
    ap.add_argument("--prefill-tokens", type=int, default=2048)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prompt", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="only the headline, decode_t4, roofline and prompt")
    ap.add_argument("--dense", action="store_true", help="only the dense half of a mixed-model decode token")
    ap.add_argument("--only", choices=("prompt", "prompt_q2_0", "prefill", "q4k", "moe"),
                    help="only this sub-workload, printed as its own line (for profiling one kernel family)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also copy 512 MiB with torch's copy kernel three times: the known-size reference that "
                         "scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters to bytes")
    return ap.parse_args()


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "routed_glu_iq3s_traffic.md")


def measured_traffic():
    """HBM bytes per gate+up launch as rocprofv3's counters gave them (the committed summary), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch"):
                    return int(line.split("=")[1].strip())
    except (OSError, ValueError, IndexError):
        pass
    return None


def time_graph(graph, steps, warmup):
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3  # seconds


def decode_layers(B, synth, dev, layers, kind="IQ3_S", seed=0):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    out = []
    for _ in range(layers):
        mats = [synth.random_stack(kind, E * r * c, dev, g) for r, c in ((F, H), (F, H), (H, F))]
        out.append((B.BlockSwitchLinear(mats[0], kind, (E, F, H)), B.BlockSwitchLinear(mats[1], kind, (E, F, H)),
                    B.BlockSwitchLinear(mats[2], kind, (E, H, F))))
    return out


def decode_bench(B, synth, dev, lins, tokens, steps, warmup, rng):
    """A step: every layer of `lins` called as the engine calls it (BlockSwitchGLU: the gate/up/SwiGLU launch, then
    down). Returns (GB/s, ms per step, bytes per step, (mean bytes of a gate/up launch, its mean seconds in a graph
    of those launches alone), routes, GB/s of the same layers as one launch each (strata_expert_layer; None above
    one token))."""
    routes = [synth.zipf_routing(tokens, E, K, rng)[0] for _ in lins]
    idx = [torch.from_numpy(r).to(torch.int32).to(dev) for r in routes]
    x = (torch.randn((tokens, H), device=dev)).half()
    mat_bytes = lins[0][0].blocks.numel() // E
    glus = [B.BlockSwitchGLU(gate, up, down) for gate, up, down in lins]

    def layered():
        for glu, ix in zip(glus, idx):
            glu(x, ix)

    def one_launch():
        for (gate, up, down), ix in zip(lins, idx):
            B.expert_layer(gate, up, down, x, ix.reshape(-1))

    def gate_up_only():
        for (gate, up, down), ix in zip(lins, idx):
            B.gate_up_swiglu(gate, up, x, ix.reshape(-1), K)

    one = tokens == 1
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graphs = {}
    with torch.cuda.stream(stream):  # one eager pass first: the library's lazy state, torch's allocator
        for name, run in (("layer", layered), ("gu", gate_up_only), ("one", one_launch))[:3 if one else 2]:
            run()
            torch.cuda.synchronize()
            graphs[name] = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graphs[name], stream=stream):
                run()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    step_bytes, gu_bytes = 0, 0
    for r in routes:
        d = len(np.unique(r))
        # the distinct experts' gate, up and down; x in, h between the halves (written and read), y out
        step_bytes += d * 3 * mat_bytes + tokens * H * 2 + 2 * tokens * K * F * 2 + tokens * K * H * 2
        gu_bytes += d * 2 * mat_bytes + tokens * H * 2 + tokens * K * F * 2  # gate/up launch: x in, h out
    t = time_graph(graphs["layer"], steps, warmup)
    t_gu = time_graph(graphs["gu"], steps, warmup)
    gbs_one = None
    if one:
        gbs_one = step_bytes * steps / time_graph(graphs["one"], steps, warmup) / 1e9
        if B.layer_status(dev):
            raise RuntimeError("a wait of the one-launch layer gave up")
    gate_up = (gu_bytes / len(lins), t_gu / steps / len(lins))
    return step_bytes * steps / t / 1e9, t / steps * 1e3, step_bytes, gate_up, routes, gbs_one


def prompt_bench(B, synth, dev, steps, warmup, rng, layers=4, tokens=512, kind="IQ3_XXS"):
    """A 512-token prompt chunk of `layers` distinct expert layers in `kind` (256 experts top-8 of Zipf routing,
    bfloat16 tokens) through switch_glu's tiles. TFLOPS over the real pairs' 2 * pairs * 3 * H * F, against the
    dense MFMA peak and against the HBM ceiling of reading every expert's weights once."""
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    lins = []
    for _ in range(layers):
        mats = [synth.random_stack(kind, E * r * c, dev, g) for r, c in ((F, H), (F, H), (H, F))]
        lins.append((B.BlockSwitchLinear(mats[0], kind, (E, F, H)), B.BlockSwitchLinear(mats[1], kind, (E, F, H)),
                     B.BlockSwitchLinear(mats[2], kind, (E, H, F))))
    idx = [torch.from_numpy(synth.zipf_routing(tokens, E, K, rng)[0]).to(torch.int32).to(dev) for _ in lins]
    x = torch.randn((tokens, H), device=dev).to(torch.bfloat16)
    for (gate, up, down), ix in zip(lins, idx):
        B._tiled_glu(x, ix, up, gate, down)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for (gate, up, down), ix in zip(lins, idx):
            B._tiled_glu(x, ix, up, gate, down)
    t = time_graph(graph, steps, warmup)
    flops = 2.0 * tokens * K * 3 * H * F * layers
    tflops = flops * steps / t / 1e12
    per, bb = synth.BLOCK[kind]
    ceiling = 2.0 * tokens * K * 3 * H * F / (3 * E * F * H / per * bb) * HBM_PEAK_GBS / 1e3
    del lins
    torch.cuda.empty_cache()
    return {"workload": f"prompt chunk {tokens} tokens, {kind}, 256 experts top-8, bf16", "tflops": round(tflops, 2),
            "ms_per_layer": round(t / steps / layers * 1e3, 4), "mfma_peak_frac": round(tflops / BF16_PEAK_TFLOPS, 4),
            "hbm_bound_tflops": round(ceiling, 1), "hbm_bound_frac": round(tflops / ceiling, 4)}


# The dense layers of a mixed-model decode token, as an engine runs them: q, k and v fused into one 12288-row
# layer (dense.FusedLinear), the shared expert's gate and up with the SwiGLU in one launch (dense.gate_up_swiglu).
DENSE = [("qkv", "Q6_K", 3 * 4096, 4096, "matvec"), ("o", "Q8_0", 4096, 4096, "matvec"),
         ("shared_gate_up", "Q4_K", 2 * 1536, 4096, "glu"), ("shared_down", "Q4_K", 4096, 1536, "matvec"),
         ("lm_head", "Q6_K", 151936, 4096, "matvec")]


def dense_bench(B, synth, dev, steps, warmup):
    """Each dense launch of a decode token at one token: mean time over a graph of distinct copies."""
    from strata_mlx_amd import dense as D
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    out, total_bytes, total_s = {}, 0, 0.0
    for name, kind, rows, cols, how in DENSE:
        per, bb = synth.DENSE.get(kind) or synth.BLOCK[kind]
        nbytes = rows * cols // per * bb
        copies = max(8, -(-(1 << 30) // nbytes))
        mats = [synth.random_stack(kind, rows * cols, dev, g) for _ in range(copies)]
        x = (torch.randn((1, cols), device=dev) / 8).half()
        if how == "glu":  # gate: the first half of the rows, up: the second
            half = rows // 2 * (cols // per * bb)
            layers = [(D.BlockLinear(m[:half], kind, (rows // 2, cols)), D.BlockLinear(m[half:], kind, (rows // 2, cols)))
                      for m in mats]

            def run(i):
                D.gate_up_swiglu(layers[i][0], layers[i][1], x)
        else:
            def run(i):
                B.window_matvec(mats[i], kind, rows, cols, x)
        graph = torch.cuda.CUDAGraph()
        run(0)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph):
            for i in range(copies):
                run(i)
        t = time_graph(graph, steps, warmup) / steps / copies
        out[name] = {"kind": kind, "rows": rows, "cols": cols, "us": round(t * 1e6, 2),
                     "gbs": round(nbytes / t / 1e9, 1), "hbm_frac": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4)}
        total_bytes += nbytes
        total_s += t
        del mats
        torch.cuda.empty_cache()
    return {"metric": "dense decode matvec GB/s (mixed model, one token)", "value": round(total_bytes / total_s / 1e9, 1),
            "unit": "GB/s", "us_per_token": round(total_s * 1e6, 1), "bytes_per_token": total_bytes,
            "hbm_frac": round(total_bytes / total_s / 1e9 / HBM_PEAK_GBS, 4), "dtype": "f16",
            "data": "synthetic (random blocks)", "layers": out}


def shared_fused_bench(B, D, synth, dev, lins, steps, warmup, rng):
    """One decode token's routed gate/up/SwiGLU (the layers' IQ3_S stacks, 256 experts top-8) with a shared expert's
    Q4_K gate and up (1536 x 4096 each) in the same launch (blocks.gate_up_swiglu_shared), against the routed launch
    alone and the two launches apart: the shared expert's marginal time a layer and its bytes' rate over it."""
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    routes = [synth.zipf_routing(1, E, K, rng)[0] for _ in lins]
    idx = [torch.from_numpy(r).to(torch.int32).to(dev).reshape(-1) for r in routes]
    x = (torch.randn((1, H), device=dev) / 8).half()
    shared = [tuple(D.BlockLinear(synth.random_stack("Q4_K", F * H, dev, g), "Q4_K", (F, H)) for _ in range(2))
              for _ in lins]

    def alone():
        for (gate, up, _), ix in zip(lins, idx):
            B.gate_up_swiglu(gate, up, x, ix, K)

    def apart():
        for (gate, up, _), ix, (sg, su) in zip(lins, idx, shared):
            B.gate_up_swiglu(gate, up, x, ix, K)
            D.gate_up_swiglu(sg, su, x)

    def fused():
        for (gate, up, _), ix, (sg, su) in zip(lins, idx, shared):
            if B.gate_up_swiglu_shared(gate, up, x, ix, sg, su) is None:
                raise RuntimeError("the routed launch did not take the shared expert")

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):  # one eager pass of each first: the library's lazy state, torch's allocator
        for run in (alone, apart, fused):
            run()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graphs = {}
    for name, run in (("alone", alone), ("apart", apart), ("fused", fused)):
        graphs[name] = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graphs[name]):
            run()
    us = {name: time_graph(gr, steps, warmup) / steps / len(lins) * 1e6 for name, gr in graphs.items()}
    mat_bytes = lins[0][0].blocks.numel() // E
    routed_bytes = sum(len(np.unique(r)) * 2 * mat_bytes for r in routes) / len(lins) + H * 2 + K * F * 2
    shared_bytes = 2 * shared[0][0].blocks.numel() + F * 2  # gate and up in, h out (x counted with the routed)
    marginal = us["fused"] - us["alone"]
    return {"workload": f"one decode token's gate/up/SwiGLU, {len(lins)} layers: routed IQ3_S 256 experts top-8 + "
                        f"shared expert Q4_K {F} x {H} gate and up",
            "routed_us": round(us["alone"], 3), "apart_us": round(us["apart"], 3), "fused_us": round(us["fused"], 3),
            "shared_bytes": int(shared_bytes), "shared_marginal_us": round(marginal, 3),
            "shared_hbm_frac": round(shared_bytes / (marginal * 1e-6) / 1e9 / HBM_PEAK_GBS, 4) if marginal > 0 else None,
            "fused_hbm_frac": round((routed_bytes + shared_bytes) / (us["fused"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def shared_down_bench(B, D, synth, dev, lins, steps, warmup, rng):
    """One decode token's routed down (the layers' IQ3_S stacks, 4096 x 1536, 256 experts top-8) with a shared
    expert's Q4_K down (4096 x 1536) in the same launch (blocks.expert_matvec_shared), against the routed launch
    alone and the two launches apart: the shared down's marginal time a layer and its bytes' rate over it."""
    g = torch.Generator(device=dev)
    g.manual_seed(6)
    routes = [synth.zipf_routing(1, E, K, rng)[0] for _ in lins]
    idx = [torch.from_numpy(r).to(torch.int32).to(dev).reshape(-1) for r in routes]
    h = (torch.randn((K, F), device=dev) / 8).half()
    sx = (torch.randn((1, F), device=dev) / 8).half()
    shared = [D.BlockLinear(synth.random_stack("Q4_K", H * F, dev, g), "Q4_K", (H, F)) for _ in lins]
    calls = [B.expert_matvec_shared(down, ix, sd) for (_, _, down), ix, sd in zip(lins, idx, shared)]

    def alone():
        for (_, _, down), ix in zip(lins, idx):
            B.expert_matvec(down, ix, h)

    def apart():
        for (_, _, down), ix, sd in zip(lins, idx, shared):
            B.expert_matvec(down, ix, h)
            B.window_matvec(sd.blocks, "Q4_K", H, F, sx)

    def fused():
        for call in calls:
            if call(h, sx) is None:
                raise RuntimeError("the routed down launch did not take the shared expert")

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):  # one eager pass of each first: the library's lazy state, torch's allocator
        for run in (alone, apart, fused):
            run()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graphs = {}
    for name, run in (("alone", alone), ("apart", apart), ("fused", fused)):
        graphs[name] = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graphs[name]):
            run()
    us = {name: time_graph(gr, steps, warmup) / steps / len(lins) * 1e6 for name, gr in graphs.items()}
    mat_bytes = lins[0][2].blocks.numel() // E
    routed_bytes = sum(len(np.unique(r)) * mat_bytes for r in routes) / len(lins) + K * F * 2 + K * H * 2
    shared_bytes = shared[0].blocks.numel() + F * 2 + H * 2  # its rows and token in, its rows' sums out
    marginal = us["fused"] - us["alone"]
    return {"workload": f"one decode token's down, {len(lins)} layers: routed IQ3_S 256 experts top-8 {H} x {F} + "
                        f"shared expert Q4_K {H} x {F}",
            "routed_us": round(us["alone"], 3), "apart_us": round(us["apart"], 3), "fused_us": round(us["fused"], 3),
            "shared_bytes": int(shared_bytes), "shared_marginal_us": round(marginal, 3),
            "shared_hbm_frac": round(shared_bytes / (marginal * 1e-6) / 1e9 / HBM_PEAK_GBS, 4) if marginal > 0 else None,
            "fused_hbm_frac": round((routed_bytes + shared_bytes) / (us["fused"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def moe_block_bench(B, D, FU, synth, dev, lins, steps, warmup):
    """One decode token through the layers' whole MoE blocks (fused.RoutedMoE: the router (256 x 4096 float16) and
    the shared expert's gate in one launch, the top-8 and softmax in the routed gate/up launch, the routed IQ3_S
    experts, a Q4_K shared expert riding in the routed launches, its sigmoid gate, the combine), each block's routing
    made by its own router from the same token: microseconds a block and the block's bytes (the distinct experts'
    rows, the shared expert, the router and gate weights) over that time."""
    g = torch.Generator(device=dev)
    g.manual_seed(8)
    x = (torch.randn((1, H), device=dev) / 64).half()
    blocks, mats = [], []
    for gate, up, down in lins:
        router = FU.WindowLinear((torch.randn((E, H), device=dev, generator=g) / 64).half())
        shared = [D.BlockLinear(synth.random_stack("Q4_K", r * c, dev, g), "Q4_K", (r, c)) for r, c in
                  ((F, H), (F, H), (H, F))]
        sgate = FU.WindowLinear((torch.randn((1, H), device=dev, generator=g) / 64).half())
        blocks.append(FU.RoutedMoE(router, B.BlockSwitchGLU(gate, up, down), *shared, sgate, K))
        mats.append((router, shared))

    def run():
        for moe in blocks:
            moe(x)

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        run()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    paths = sorted({moe.last_path for moe in blocks})
    if paths != ["choice in the launch"]:
        raise RuntimeError(f"the choice and the shared expert were not in the routed launches: {paths}")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    us = time_graph(graph, steps, warmup) / steps / len(blocks) * 1e6
    distinct = []
    for moe in blocks:  # each block's experts, as its router chose them for this token
        idx, _ = FU.route(moe.router, x, K)
        distinct.append(len(torch.unique(idx)))
    row = lins[0][0].blocks.numel() // E  # one expert's gate (or up, or down) bytes
    routed = sum(distinct) / len(distinct) * 3 * row
    shared_bytes = sum(lay.blocks.numel() for lay in mats[0][1])
    total = routed + shared_bytes + E * H * 2 + H * 2 + K * F * 2 + H * 2
    return {"workload": f"one decode token through {len(blocks)} MoE blocks: router 256 x 4096 float16, top-8, "
                        f"routed IQ3_S {F} x {H} / {H} x {F} choosing its experts in the gate/up launch, shared expert "
                        f"Q4_K riding in the routed launches, "
                        f"its gate, the combine", "us_per_block": round(us, 2),
            "bytes_per_block": int(total), "gbs": round(total / (us * 1e-6) / 1e9, 1),
            "hbm_frac": round(total / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def host_cpu():
    """(the host's cores as this process sees them, the threads BLAS is given, the CPU model)."""
    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    threads = int(os.environ.get("OMP_NUM_THREADS", cores) or cores)
    threads = max(1, min(threads, cores))
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return cores, threads, model


def cpu_baseline(lins, routes, tokens, budget_s=15.0, max_layers=4):
    """The reference's CPU path restated (the oracle): numpy decode of the touched experts (one thread, as numpy
    decodes) and their float32 matvecs (BLAS on the host's cores), layer by layer until about budget_s of CPU work.
    The experts' bytes are copied to the host first, untimed: the CPU path reads them from memory. Returns (layers,
    algorithmic bytes, seconds, BLAS threads)."""
    from threadpoolctl import threadpool_limits

    from oracle import blocks as O

    mat_bytes = F * H // 256 * 110
    done, secs, layers = 0, 0.0, 0
    x = np.random.default_rng(5).standard_normal((tokens, H)).astype(np.float16)
    _, threads, _ = host_cpu()
    with threadpool_limits(limits=threads):
        for (gate, up, down), r in zip(lins, routes):
            used = [int(e) for e in np.unique(r)]
            host = {n: {e: lin.blocks[e * mat_bytes:(e + 1) * mat_bytes].cpu().numpy() for e in used}
                    for n, lin in (("gate", gate), ("up", up), ("down", down))}
            t0 = time.perf_counter()
            w = {n: {e: O.dequantize(b, "IQ3_S", (H, F) if n == "down" else (F, H)) for e, b in host[n].items()}
                 for n in host}
            flat = r.reshape(-1)
            g = np.stack([w["gate"][int(e)] @ x[p // K].astype(np.float32) for p, e in enumerate(flat)])
            u = np.stack([w["up"][int(e)] @ x[p // K].astype(np.float32) for p, e in enumerate(flat)])
            with np.errstate(over="ignore"):  # a product past float16's range rounds to inf, as on the device
                h = O.swiglu_rounded(g.astype(np.float16), u.astype(np.float16), np.float16)
            np.stack([w["down"][int(e)] @ h[p].astype(np.float32) for p, e in enumerate(flat)])
            secs += time.perf_counter() - t0
            layers += 1
            done += len(used) * 3 * mat_bytes + x.nbytes + 2 * len(flat) * F * 2 + len(flat) * H * 2
            if secs > budget_s or layers >= max_layers:
                break
    return layers, done, secs, threads


def q4k_bench(B, synth, dev, steps, warmup, copies=64):
    """One Q4_K 4096 x 4096 matrix times float32 x, batch 1: graphs over `copies` distinct matrices (604 MB, past
    the MALL). Returns the sub-object, with the CPU path (the oracle's to_affine-style decode, then x @ W.T) timed on
    the host beside it."""
    from threadpoolctl import threadpool_limits

    from oracle import blocks as O

    rows = cols = 4096
    nbytes = rows * cols // 256 * 144
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    mats = [synth.random_stack("Q4_K", rows * cols, dev, g) for _ in range(copies)]
    x = torch.randn((1, cols), device=dev)
    B.window_matvec(mats[0], "Q4_K", rows, cols, x)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for m in mats:
            B.window_matvec(m, "Q4_K", rows, cols, x)
    t = time_graph(graph, steps, warmup) / steps / copies
    moved = nbytes + cols * 4 + rows * 4
    host = mats[0].cpu().numpy()
    xh = x.cpu().numpy()
    cores, threads, model = host_cpu()
    reps, secs = 0, 0.0
    with threadpool_limits(limits=threads):
        while secs < 5.0 and reps < 50:
            t0 = time.perf_counter()
            w = O.dequantize(host, "Q4_K", (rows, cols))
            xh @ w.T
            secs += time.perf_counter() - t0
            reps += 1
    del mats
    torch.cuda.empty_cache()
    return {"workload": "Q4_K 4096x4096 matvec, float32 x, batch 1", "us_per_matvec": round(t * 1e6, 2),
            "gbs": round(moved / t / 1e9, 1), "hbm_frac": round(moved / t / 1e9 / HBM_PEAK_GBS, 4),
            "cpu": {"us_per_matvec": round(secs / reps * 1e6, 1), "gbs": round(moved * reps / secs / 1e9, 4),
                    "cores": threads, "kind": "port",
                    "sample": f"{reps} matvecs: numpy decode (one thread) + x @ W.T (BLAS, {threads} threads)"}}


def prefill_bench(B, D, synth, dev, lins, steps, warmup, rng, tokens=2048):
    """A prefill of `tokens` tokens (2048 by default) of the mixed model, bfloat16: the routed IQ3_S experts of `lins`
    (Zipf top-8) through the tiles, and the dense layers (q, k, v Q6_K fused, o Q8_0, the shared expert's Q4_K gate
    and up fused, down) as the reference multiplies a prompt chunk: each dequantized for the chunk, then the library product. Returns
    TFLOPS over the real products' flops, each part and all."""
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    mk = lambda kind, r, c: D.BlockLinear(synth.random_stack(kind, r * c, dev, g), kind, (r, c))
    # q, k, v as one layer and the shared expert's gate and up as one, as the decode runs them
    dense = [D.FusedLinear([mk("Q6_K", H, H) for _ in range(3)]), mk("Q8_0", H, H),
             D.FusedLinear([mk("Q4_K", F, H) for _ in range(2)]), mk("Q4_K", H, F)]
    idx = [torch.from_numpy(synth.zipf_routing(tokens, E, K, rng)[0]).to(torch.int32).to(dev) for _ in lins]
    x = torch.randn((tokens, H), device=dev).to(torch.bfloat16)
    xf = torch.randn((tokens, F), device=dev).to(torch.bfloat16)

    def routed():
        for (gate, up, down), ix in zip(lins, idx):
            B._tiled_glu(x, ix, up, gate, down)

    def dense_all():
        for lin in dense:
            lin(xf if lin.input_dims == F else x)

    out = {}
    for name, fn, flops in (("routed", routed, 2.0 * tokens * K * 3 * H * F * len(lins)),
                            ("dense", dense_all, sum(2.0 * tokens * lin.output_dims * lin.input_dims for lin in dense))):
        fn()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn()
        t = time_graph(graph, steps, warmup) / steps
        out[name] = {"tflops": round(flops / t / 1e12, 2), "ms": round(t * 1e3, 4),
                     "layers": len(lins) if name == "routed" else len(dense)}
        out[name]["_flops"] = flops
    fl = out["routed"]["_flops"] / len(lins) + out["dense"]["_flops"]
    ms = out["routed"]["ms"] / len(lins) + out["dense"]["ms"]
    for v in out.values():
        v.pop("_flops")
    out.update({"workload": f"{tokens}-token prefill, bf16: routed IQ3_S 256 experts top-8 (one layer) + dense q/k/v "
                            "Q6_K, o Q8_0, shared expert Q4_K", "tflops": round(fl / ms / 1e9, 2),
                "ms_per_layer": round(ms, 4), "mfma_peak_frac": round(fl / ms / 1e9 / BF16_PEAK_TFLOPS, 4)})
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: the path has no multi-GPU form (asked for {args.gpus} GPUs); "
              "it measures one GPU's share", file=sys.stderr)
        sys.exit(2)
    from strata_mlx_amd import blocks as B
    from strata_mlx_amd import synth

    dev = torch.device("cuda:0")
    rng = np.random.default_rng(0)

    def note(msg):
        print(f"[bench] {msg}", file=sys.stderr, flush=True)

    if args.copy_probe:
        src = torch.ones(512 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.dense:
        note("dense half of a mixed-model decode token")
        print(json.dumps(dense_bench(B, synth, dev, max(2, args.steps // 5), 2)))
        return

    if args.only:
        note(f"only {args.only}")
        steps = max(2, args.steps // 10)
        if args.only in ("prompt", "prompt_q2_0"):
            out = prompt_bench(B, synth, dev, steps, 2, rng, kind="Q2_0" if args.only == "prompt_q2_0" else "IQ3_XXS")
        elif args.only == "q4k":
            out = q4k_bench(B, synth, dev, max(2, args.steps // 5), 2)
        elif args.only == "moe":
            from strata_mlx_amd import dense as D
            from strata_mlx_amd import fused as FU
            out = moe_block_bench(B, D, FU, synth, dev, decode_layers(B, synth, dev, args.layers), args.steps,
                                  args.warmup)
        else:
            from strata_mlx_amd import dense as D
            out = prefill_bench(B, D, synth, dev, decode_layers(B, synth, dev, 2), steps, 2, rng,
                                tokens=args.prefill_tokens)
        print(json.dumps({args.only: out}))
        return
    note(f"making {args.layers} IQ3_S layers of 256 experts")
    lins = decode_layers(B, synth, dev, args.layers)
    note("decode, batch {}".format(args.tokens))
    gbs, ms, step_bytes, (gu_bytes, gu_s), routes, gbs_one = decode_bench(B, synth, dev, lins, args.tokens,
                                                                           args.steps, args.warmup, rng)
    note(f"decode: {gbs:.1f} GB/s (one launch a layer: {gbs_one}); batch 4")
    gbs4, ms4, _, _, _, _ = decode_bench(B, synth, dev, lins, 4, args.steps, args.warmup, rng)
    achieved = gu_bytes / gu_s / 1e9
    result = {
        "metric": "expert decode matvec GB/s (% HBM peak) + prompt dequant-GEMM TFLOPS",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: random IQ3_S blocks (d=|N(0,1)|*0.01), Zipf(1.1) top-8 routing, x ~ N(0,1) float16 as the "
                "workload names it; on these random blocks the float16 SwiGLU and down overflow to inf in part, which "
                "no launch's timing depends on (the parity tests run the same launches at x ~ N(0,1)/64)",
        "config": {"workload": f"routed-expert decode, IQ3_S, 256 experts top-8, gate/up 1536x4096, down 4096x1536, "
                               f"SwiGLU, batch {args.tokens}; a step = {args.layers} distinct layers, each one "
                               f"BlockSwitchGLU call (gate/up/SwiGLU, then down)",
                   "tokens": args.tokens, "experts": E, "top_k": K, "hidden": H, "ffn": F, "layers": args.layers,
                   "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)},
        "one_launch": None if gbs_one is None else {
            "gbs": round(gbs_one, 1), "hbm_frac": round(gbs_one / HBM_PEAK_GBS, 4),
            "note": "the same layers as one launch each (routed_layer_kernel: gate, up, SwiGLU and down, the pair's "
                    "h handed over in memory; strata_expert_layer)"},
        "decode_t4": {"gbs": round(gbs4, 1), "ms_per_step": round(ms4, 4), "hbm_frac": round(gbs4 / HBM_PEAK_GBS, 4),
                      "note": "gate/up/SwiGLU then down, two launches a layer"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "kernel": "routed_glu_kernel IQ3_S gate+up+SwiGLU (strata_expert_gate_up_swiglu)",
                     "bytes_per_launch": int(gu_bytes), "mean_launch_us": round(gu_s * 1e6, 3)},
    }
    if not args.no_extra:
        note("speculative verify, Q2_0, 5 rows")
        q2 = decode_layers(B, synth, dev, args.layers, "Q2_0", seed=7)
        gq, msq, _, _, _, _ = decode_bench(B, synth, dev, q2, 5, args.steps, args.warmup, rng)
        result["speculate"] = {"workload": "Q2_0 routed decode, 256 experts top-8, 5 rows (1 + 4 draft), 16 layers",
                               "gbs": round(gq, 1), "ms_per_step": round(msq, 4), "hbm_frac": round(gq / HBM_PEAK_GBS, 4)}
        del q2
        torch.cuda.empty_cache()
        note("Q4_K 4096 x 4096, float32 x")
        result["q4k_matvec"] = q4k_bench(B, synth, dev, max(2, args.steps // 5), 2)
    if not args.no_prompt:
        note("prompt chunk")
        result["prompt"] = prompt_bench(B, synth, dev, max(2, args.steps // 10), 2, rng)
        note("prompt chunk, Q2_0")
        result["prompt_q2_0"] = prompt_bench(B, synth, dev, max(2, args.steps // 10), 2, rng, kind="Q2_0")
    if not args.no_extra:
        note("dense half of a decode token")
        dd = dense_bench(B, synth, dev, max(2, args.steps // 5), 2)
        result["dense_decode"] = {k: dd[k] for k in ("value", "unit", "us_per_token", "bytes_per_token", "hbm_frac")}
        result["dense_decode"]["layers"] = {n: {k: v[k] for k in ("kind", "us", "hbm_frac")} for n, v in dd["layers"].items()}
        from strata_mlx_amd import dense as D
        note("shared expert's gate and up in the routed launch")
        result["dense_decode"]["shared_in_routed"] = shared_fused_bench(B, D, synth, dev, lins, args.steps, args.warmup,
                                                                        rng)
        note("shared expert's down in the routed down launch")
        result["dense_decode"]["shared_down_in_routed"] = shared_down_bench(B, D, synth, dev, lins, args.steps,
                                                                            args.warmup, rng)
        # the same token with the shared expert's launches replaced by their marginal cost in the routed launches
        lay, sg, sd = dd["layers"], result["dense_decode"]["shared_in_routed"], result["dense_decode"]["shared_down_in_routed"]
        riding_us = sum(lay[n]["us"] for n in ("qkv", "o", "lm_head")) + max(0.0, sg["shared_marginal_us"]) + \
            max(0.0, sd["shared_marginal_us"])
        result["dense_decode"]["shared_riding"] = {
            "us_per_token": round(riding_us, 1), "gbs": round(dd["bytes_per_token"] / riding_us / 1e3, 1),
            "hbm_frac": round(dd["bytes_per_token"] / riding_us / 1e3 / HBM_PEAK_GBS, 4),
            "note": "q/k/v, o and lm_head as above; the shared expert's gate/up and down at their marginal time in "
                    "the routed launches (the same bytes a token)"}
        note("whole MoE blocks at one token")
        from strata_mlx_amd import fused as FU
        result["moe_block"] = moe_block_bench(B, D, FU, synth, dev, lins, args.steps, args.warmup)
        note("2048-token prefill")
        result["prefill"] = prefill_bench(B, D, synth, dev, lins[:2], max(2, args.steps // 10), 2, rng,
                                          tokens=args.prefill_tokens)
    if not args.no_cpu_baseline:
        note("cpu baseline")
        layers, done, secs, threads = cpu_baseline(lins, routes, args.tokens)
        cores, _, model = host_cpu()
        result["cpu_baseline"] = {"value": round(done / secs / 1e9, 4), "unit": "GB/s", "cores": threads,
                                  "kind": "port",
                                  "sample": f"{layers} layers of the headline workload at batch {args.tokens}: numpy "
                                            f"decode of the touched experts (one thread) + float32 matvecs (BLAS, "
                                            f"{threads} threads) + SwiGLU (oracle/blocks.py)",
                                  "seconds": round(secs, 2), "host_cores": cores, "cpu_model": model}
    print(json.dumps(result))


if __name__ == "__main__":
    main()
