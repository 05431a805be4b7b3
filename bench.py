#!/usr/bin/env python3
"""Benchmark of the LATENT fused low-rank expert FFN on one MI355X.

Workload (DeepSeek-V3-shaped LATENT MoE layer): 256 experts, d=7168,
ff=2048, uniform rank 256, NF4 group 32 + fp16 scales, top-8 softmax routing,
bf16 activations.  A step is one `latent_moe_ffn_forward` call (token->expert
grouping + the fused factor chain + router-weighted combine) on one batch;
inputs are resident in HBM before the timed region.

Cache honesty: the 256 MB MALL would hold a small batch's experts, so the
timed loop rotates over `--layers` independently generated layers (1 GB of
packed factors each) and several routings; consecutive steps never touch the
same layer.

Timing of the decode points: W eager warmup steps, then exactly K steps
captured in one HIP graph (torch.cuda.CUDAGraph) that is replayed once
untimed and once timed, HIP events around the timed replay: the seven
kernels of a step run back to back as in a graph-launched decode loop (the
way the reference's llama.cpp backend launches decode).  The same K steps
issued eagerly are timed too and reported as `eager_ms_per_step`
(`--timing eager` makes them the figure).

The headline `value` is tokens/s at batch 64; batches 1, 2, 4, 8, 16 and 32, the
4096-token prefill, the heterogeneous-rank layer (ranks 64..512, 10% INT8
groups, drop below 0.05, batches 16 and 256) and the 58-layer graph-captured
stack are reported under "sweep", "prefill", "hetero" and "stack".  HBM GB/s
counts the packed factor bytes of the distinct experts each step routes to
(at each expert's true rank; the heterogeneous layer also reports the bytes
padded to max_rank).

Prefill routing: the stated skew (popularity proportional to rank^-1.1,
about 0 to 400 tokens per expert) is not reachable with a Zipf logit bias at
4096 tokens x top-8 over 256 experts (gamma 0.11 gives about 77..374 tokens
per expert, gamma 0.4 about 18..1980), so the default bias falls linearly with
the popularity rank (beta 1.5: about 6..436, some 20 experts below 16); the
Zipf form is --zipf-gamma.  The tokens-per-expert histogram is reported.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

METRIC = "MoE-layer tokens/sec + HBM GB/s (% roofline), decode b=1..64 & prefill 4096"
HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
E, D, FF, R, K = 256, 7168, 2048, 256, 8
EXPERT_BYTES = (2 * D * R + 2 * R * FF + FF * R + R * D) // 2 + (2 * D * R + 2 * R * FF + FF * R + R * D) // 32 * 2
PAIR_FLOPS = 2 * (2 * D * R + 2 * R * FF + FF * R + R * D)


def parse():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--batch", type=int, default=64, help="headline decode batch")
    p.add_argument("--sweep", type=str, default="1,2,4,8,16,32", help="other decode batches ('' to skip)")
    p.add_argument("--prefill", type=int, default=4096, help="prefill tokens (0 to skip)")
    p.add_argument("--prefill-steps", type=int, default=5)
    p.add_argument("--layers", type=int, default=4, help="distinct layers rotated in the timed loop")
    p.add_argument("--routings", type=int, default=16, help="distinct routings per batch size")
    p.add_argument("--timing", choices=("graph", "eager"), default="graph",
                   help="decode points: K steps replayed from one HIP graph (default) or issued eagerly")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--copy-probe-mb", type=int, default=0,
                   help="run one device-to-device copy of this many MiB first (counter calibration)")
    p.add_argument("--stack", type=int, default=58,
                   help="layers of the graph-captured stacked decode (0 to skip)")
    p.add_argument("--stack-batch", type=int, default=32)
    p.add_argument("--stack-steps", type=int, default=10)
    p.add_argument("--zipf-gamma", type=float, default=0.0,
                   help="prefill router Zipf skew gamma * (-1.1 ln rank) (0: off)")
    p.add_argument("--rank-beta", type=float, default=1.5,
                   help="prefill router skew falling linearly with the popularity rank (about 6..436 at 1.5)")
    p.add_argument("--hetero", type=str, default="16,256",
                   help="batches of the heterogeneous-rank layer ('' to skip)")
    p.add_argument("--cpu-steps", type=int, default=5, help="CPU-baseline steps per setting (median)")
    return p.parse_args()


def realized_bytes(ids_list):
    """Packed factor bytes of the distinct experts each routing touches."""
    out = []
    for ids in ids_list:
        v = ids[(ids >= 0) & (ids < E)]
        out.append(np.unique(v).size * EXPERT_BYTES)
    return out


def time_loop(fn, n_steps, warmup, torch):
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(n_steps):
        fn(i)
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / n_steps  # ms per step


def graph_time(torch, fn, n_steps):
    """ms per step of exactly `n_steps` steps captured once in a HIP graph
    (torch.cuda.CUDAGraph): one untimed replay, then one timed replay."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn(0)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n_steps):
            fn(i)
    ms = time_loop(lambda i: g.replay(), 1, 1, torch)
    del g
    return ms / n_steps


def decode_point(torch, latent, gsynth, layers, batch, steps, warmup, n_routings, timing="graph"):
    routes = [gsynth.route(seed=10_000 + 97 * batch + r, n_tokens=batch, n_expert=E, k=K) for r in range(n_routings)]
    xs = [gsynth.bf16_input(seed=20_000 + 89 * batch + r, n_tokens=batch, d=D) for r in range(n_routings)]
    outs = [torch.empty((batch, D), dtype=torch.float32, device="cuda") for _ in range(n_routings)]
    for L in layers:
        L.workspace(batch, K)
    ws = layers[0].workspace(batch, K)

    def step(i):
        r = i % n_routings
        ids, w = routes[r]
        latent.moe_forward(xs[r], ids, w, layers[i % len(layers)], out=outs[r], workspace=ws)

    eager = time_loop(step, steps, warmup, torch)
    gms = graph_time(torch, step, steps) if timing == "graph" else None
    ms = gms if gms is not None else eager
    ids_host = [routes[i % n_routings][0].cpu().numpy() for i in range(steps)]
    bytes_per_step = float(np.mean(realized_bytes(ids_host)))
    gbps = bytes_per_step / (ms * 1e-3) / 1e9
    return {
        "batch": batch,
        "path": latent.moe_path(layers[0], xs[0], K),
        "launch": latent.moe.stream_launch(layers[0], xs[0], K),
        "ms_per_step": ms,
        "timing": timing,
        "eager_ms_per_step": eager,
        "tokens_per_s": batch / (ms * 1e-3),
        "hbm_gbps": gbps,
        "roofline_frac": gbps / HBM_PEAK_GBPS,
        "bytes_per_step": bytes_per_step,
        "distinct_experts_mean": bytes_per_step / EXPERT_BYTES,
    }, routes, xs


def histogram(counts):
    """Tokens per expert: order statistics and the tail below 16."""
    c = np.sort(counts)
    q = lambda f: int(c[min(len(c) - 1, int(f * (len(c) - 1)))])
    return {"min": int(c[0]), "p10": q(0.1), "p25": q(0.25), "median": q(0.5), "p75": q(0.75), "p90": q(0.9),
            "max": int(c[-1]), "experts_below_16": int((c < 16).sum()), "experts_empty": int((c == 0).sum())}


def prefill_point(torch, latent, gsynth, layers, tokens, steps, zipf_gamma, rank_beta):
    ids, w = gsynth.route(seed=30_000, n_tokens=tokens, n_expert=E, k=K, zipf_gamma=zipf_gamma, rank_beta=rank_beta)
    x = gsynth.bf16_input(seed=30_001, n_tokens=tokens, d=D)
    out = torch.empty((tokens, D), dtype=torch.float32, device="cuda")
    ws = layers[0].workspace(tokens, K)

    def step(i):
        latent.moe_forward(x, ids, w, layers[i % len(layers)], out=out, workspace=ws)

    ms = time_loop(step, steps, 1, torch)
    counts = np.bincount(ids.cpu().numpy().reshape(-1), minlength=E)
    flops = float(PAIR_FLOPS) * int((ids >= 0).sum().item())
    tflops = flops / (ms * 1e-3) / 1e12
    return {
        "tokens": tokens,
        "ms_per_step": ms,
        "tokens_per_s": tokens / (ms * 1e-3),
        "tflops": tflops,
        "mfma_frac_bf16_peak": tflops / MFMA_BF16_PEAK_TFLOPS,
        "tokens_per_expert": histogram(counts),
        "path": latent.moe_path(layers[0], x, K),
        "zipf_gamma": zipf_gamma,
        "rank_beta": rank_beta,
    }, (ids, w, x)


def stack_point(torch, latent, gsynth, n_layers, batch, steps):
    """n_layers DeepSeek-V3-shaped LATENT MoE layers, each with its own seeded
    router (W_r ~ N(0, 1/d), fp32) and a residual add, decoded as one HIP graph."""
    t0 = time.time()
    torch.cuda.synchronize()
    alloc0 = torch.cuda.memory_allocated()
    layers = [gsynth.make_layer(seed=500_000 + 7919 * l, n_expert=E, d=D, ff=FF, max_rank=R) for l in range(n_layers)]
    torch.cuda.synchronize()
    resident_alloc = torch.cuda.memory_allocated() - alloc0  # what the process holds for the layers
    routers = []
    for l in range(n_layers):
        g = torch.Generator(device="cuda")
        g.manual_seed(900_000 + l)
        w = torch.randn((D, E), generator=g, device="cuda") / np.sqrt(D)
        routers.append(latent.Router(w, K))
    torch.cuda.synchronize()
    gen_s = time.time() - t0
    stack = latent.DecodeStack(layers, routers, batch)
    x0 = gsynth.bf16_input(seed=777, n_tokens=batch, d=D).float()
    stack.load(x0)
    # Eager (one host call per kernel) for comparison, then the captured graph.
    eager_ms = time_loop(lambda i: stack.forward(), 3, 1, torch)
    eager_out = stack.forward().clone()
    stack.capture()
    ms = time_loop(lambda i: stack.replay(), steps, 2, torch)
    stack.load(x0)
    replay_out = stack.replay().clone()
    torch.cuda.synchronize()
    replay_equal = bool(torch.equal(replay_out, eager_out))
    replay_maxdiff = float((replay_out - eager_out).abs().max().item())
    ids = [t.cpu().numpy() for t in stack.layer_ids()]
    step_bytes = float(sum(realized_bytes(ids)))
    resident = stack.resident_bytes()
    dense_bf16 = n_layers * E * 2 * (3 * D * FF)
    gbps = step_bytes / (ms * 1e-3) / 1e9
    out = {
        "layers": n_layers,
        "batch": batch,
        "graph": "torch.cuda.CUDAGraph (HIP graph): per layer 2 router kernels + expert FFN + residual add",
        "ms_per_step": ms,
        "us_per_layer": ms * 1e3 / n_layers,
        "tokens_per_s": batch / (ms * 1e-3),
        "layer_tokens_per_s": batch * n_layers / (ms * 1e-3),
        "eager_ms_per_step": eager_ms,
        "bytes_per_step": step_bytes,
        "hbm_gbps": gbps,
        "roofline_frac": gbps / HBM_PEAK_GBPS,
        "router_bytes_per_step": stack.router_bytes(),
        "resident_bytes": resident,
        "resident_allocated_bytes": resident_alloc,
        "dense_bf16_bytes": dense_bf16,
        "compression_vs_dense_bf16": dense_bf16 / resident_alloc,
        "replay_equals_eager": replay_equal,
        "replay_max_abs_diff_vs_eager": replay_maxdiff,
        "generate_s": gen_s,
    }
    del stack, layers, routers
    torch.cuda.empty_cache()
    return out


def _host_subset(torch, layer, ids, ref):
    """The routed experts of one step as an oracle layer (copied out of the
    timed region), and the ids renumbered to it."""
    experts = np.unique(ids[(ids >= 0) & (ids < E)])
    lut = -np.ones(E, np.int64)
    lut[experts] = np.arange(experts.size)
    local = np.where(ids >= 0, lut[np.clip(ids, 0, E - 1)], -1).astype(np.int32)
    facs = {}
    for name in layer.factors():
        f = layer.factor_rows(name, experts)  # the routed experts, back in the row layout
        facs[name] = ref.StackedFactor(f.codes.cpu().numpy(), f.scales.cpu().numpy().view(np.float16))
    return ref.StackedLayer(factors=facs, d=D, ff=FF, max_rank=R), local, experts.size


def cpu_baseline(torch, layer, routes, xs, batch, steps, prefill_inputs, prefill_tokens):
    """The oracle (numpy restatement of loader/latent_runtime.py, each routed
    expert dequantized once per step) on the same workloads, timed on the
    host: decode steps at `batch` with all host threads the GPU box grants
    (OMP_NUM_THREADS) and with one, median of `steps` steps each; and one
    prefill step on the first `prefill_tokens` tokens of the prefill batch
    (all threads)."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from threadpoolctl import threadpool_limits

    from oracle import latent_ref as ref

    threads_all = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or os.cpu_count()
    decode = {}
    experts_seen = 0
    for threads in (threads_all, 1):
        times = []
        for s in range(steps):
            ids = routes[s % len(routes)][0].cpu().numpy()
            w = routes[s % len(routes)][1].cpu().numpy()
            x = xs[s % len(xs)].float().cpu().numpy()
            host, local, n_exp = _host_subset(torch, layer, ids, ref)
            experts_seen += n_exp
            with threadpool_limits(limits=threads):
                t0 = time.perf_counter()
                ref.moe_forward(x, local, w, host)
                times.append(time.perf_counter() - t0)
        decode[threads] = float(np.median(times))
    prefill = None
    if prefill_inputs is not None and prefill_tokens:
        ids_p, w_p, x_p = prefill_inputs
        ids = ids_p[:prefill_tokens].cpu().numpy()
        w = w_p[:prefill_tokens].cpu().numpy()
        x = x_p[:prefill_tokens].float().cpu().numpy()
        host, local, n_exp = _host_subset(torch, layer, ids, ref)
        with threadpool_limits(limits=threads_all):
            t0 = time.perf_counter()
            ref.moe_forward(x, local, w, host)
            dt = time.perf_counter() - t0
        prefill = {"value": prefill_tokens / dt, "unit": "tokens/s", "cores": threads_all, "kind": "port",
                   "sample": f"one prefill step on the first {prefill_tokens} of the prefill batch's tokens "
                             f"({n_exp} distinct experts, each dequantized once; numpy fp32), {dt:.1f} s"}
    per_step = experts_seen / (2 * steps)
    return {
        "value": batch / decode[threads_all],
        "unit": "tokens/s",
        "cores": threads_all,
        "kind": "port",
        "sample": f"median of {steps} decode steps at batch {batch} ({per_step:.0f} distinct experts per step, "
                  f"each dequantized once; numpy fp32 with {threads_all} BLAS threads; {os.cpu_count()} host cores "
                  f"visible); data generation and host copies excluded",
        "single_thread": {"value": batch / decode[1], "unit": "tokens/s", "cores": 1,
                          "sample": f"the same {steps} steps, median, 1 BLAS thread"},
        "prefill": prefill,
    }


def expert_bytes(torch, layer):
    """Packed bytes of each expert's six factors, at its true rank and padded
    to max_rank: NF4 codes and fp16 scales, plus the INT8 side bytes of its
    flagged groups (32 per group, in place of the group's 16 code bytes) and
    the per-row bitmap words and offsets a kernel reads for a factor that has
    them.  Returns two float64 arrays [E]."""
    ranks = layer.ranks[:, 0].to(torch.int64)
    true_b = torch.zeros(layer.n_expert, dtype=torch.float64, device=ranks.device)
    pad_b = torch.zeros_like(true_b)
    for name, f in layer.factors().items():
        rows, cols = f.rows, f.cols
        if name.endswith("_a"):  # [n_in, R]: the rank is the column count
            t_elems = rows * torch.clamp(ranks, max=cols)
        else:  # [R, n_out]: the rank is the row count
            t_elems = torch.clamp(ranks, max=rows) * cols
        true_b += t_elems.double() / 2 + t_elems.double() / 32 * 2
        pad_b += rows * cols / 2 + rows * cols / 32 * 2
        if f.has_int8:
            v = f.int8_bitmap.to(torch.int64) & 0xFFFFFFFF
            bits = torch.zeros_like(v)
            for _ in range(32):
                bits += v & 1
                v >>= 1
            per_e = bits.reshape(layer.n_expert, -1).sum(1).double()
            extra = 16 * per_e + rows * (f.int8_bitmap.shape[-1] * 4 + 4)
            true_b += extra
            pad_b += extra
    return true_b.cpu().numpy(), pad_b.cpu().numpy()


R_H = 512  # heterogeneous layer: max_rank


def hetero_point(torch, latent, gsynth, batches, steps, warmup):
    """Heterogeneous compression at the decode shapes: ranks drawn from
    {64, 128, 256, 512} per expert, padded to max_rank 512, 10% of the groups
    INT8, routed slots with renormalised weight below 0.05 dropped."""
    rng = np.random.default_rng(40_000)
    ranks = [int(v) for v in rng.choice([64, 128, 256, 512], size=E)]
    t0 = time.time()
    layers = [gsynth.make_layer(seed=41_000 + 13 * i, n_expert=E, d=D, ff=FF, max_rank=R_H, ranks=ranks,
                                int8_fraction=0.1) for i in range(2)]
    torch.cuda.synchronize()
    gen_s = time.time() - t0
    true_b, pad_b = expert_bytes(torch, layers[0])
    out = []
    for batch in batches:
        routes = [gsynth.route(seed=42_000 + 31 * batch + r, n_tokens=batch, n_expert=E, k=K, drop_below=0.05)
                  for r in range(4)]
        xs = [gsynth.bf16_input(seed=43_000 + 37 * batch + r, n_tokens=batch, d=D) for r in range(4)]
        y = torch.empty((batch, D), dtype=torch.float32, device="cuda")
        ws = layers[0].workspace(batch, K)
        for L in layers:
            L.workspace(batch, K)

        def step(i):
            ids, w = routes[i % 4]
            latent.moe_forward(xs[i % 4], ids, w, layers[i % 2], out=y, workspace=ws)

        ms = time_loop(step, steps, warmup, torch)
        tb, pb, dropped = [], [], 0
        for ids, _ in routes:
            h = ids.cpu().numpy()
            ex = np.unique(h[(h >= 0) & (h < E)])
            tb.append(float(true_b[ex].sum()))
            pb.append(float(pad_b[ex].sum()))
            dropped += int((h < 0).sum())
        tbytes, pbytes = float(np.mean(tb)), float(np.mean(pb))
        out.append({
            "batch": batch,
            "path": latent.moe_path(layers[0], xs[0], K),
            "ms_per_step": ms,
            "tokens_per_s": batch / (ms * 1e-3),
            "bytes_per_step_true_rank": tbytes,
            "bytes_per_step_padded": pbytes,
            "hbm_gbps_true_rank": tbytes / (ms * 1e-3) / 1e9,
            "hbm_gbps_padded": pbytes / (ms * 1e-3) / 1e9,
            "roofline_frac_true_rank": tbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
            "dropped_slots_frac": dropped / (4 * batch * K),
        })
    mean_rank = float(np.mean(ranks))
    del layers
    torch.cuda.empty_cache()
    return {"ranks_mean": mean_rank, "int8_fraction": 0.1, "max_rank": R_H, "generate_s": gen_s, "points": out}


PROFILES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")
TRAFFIC_PROFILE = {
    "stream": ("streaming_decode_b64_hbm_traffic.md", "traffic_bytes_per_step:"),
}


def measured_traffic(path):
    """HBM bytes per batch-64 step of `path` from the committed counter summary
    (two rocprofv3 --pmc passes, FETCH_SIZE and WRITE_SIZE, scaled by a 1 GiB
    copy), or None when there is none."""
    name, key = TRAFFIC_PROFILE.get(path, (None, None))
    if name is None:
        return None
    try:
        with open(os.path.join(PROFILES, name)) as f:
            for line in f:
                if line.startswith(key):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the expert-parallel "
              "multi-GPU path is not built", file=sys.stderr)
        sys.exit(2)
    import torch

    import latent_amd as latent
    from latent_amd import synth as gsynth

    if args.copy_probe_mb:
        src = torch.empty(args.copy_probe_mb << 20, dtype=torch.uint8, device="cuda")
        torch.empty_like(src).copy_(src)
        torch.cuda.synchronize()
        del src
    t0 = time.time()
    layers = [gsynth.make_layer(seed=1 + 1000 * i, n_expert=E, d=D, ff=FF, max_rank=R) for i in range(args.layers)]
    torch.cuda.synchronize()
    print(f"# generated {args.layers} layers ({layers[0].nbytes() / 1e9:.3f} GB packed each) in {time.time() - t0:.1f} s",
          file=sys.stderr, flush=True)

    def show(pt):
        return (f"# decode B={pt['batch']}: {pt['ms_per_step'] * 1e3:.1f} us/step ({pt['timing']}), "
                f"{pt['hbm_gbps']:.0f} GB/s; eager {pt['eager_ms_per_step'] * 1e3:.1f} us/step")

    head, routes, xs = decode_point(torch, latent, gsynth, layers, args.batch, args.steps, args.warmup, args.routings,
                                    args.timing)
    print(show(head), file=sys.stderr, flush=True)
    sweep = []
    for b in [int(v) for v in args.sweep.split(",") if v.strip()]:
        pt, _, _ = decode_point(torch, latent, gsynth, layers, b, args.steps, args.warmup, args.routings,
                                args.timing)
        sweep.append(pt)
        print(show(pt), file=sys.stderr, flush=True)
    prefill, prefill_inputs = None, None
    if args.prefill:
        prefill, prefill_inputs = prefill_point(torch, latent, gsynth, layers, args.prefill, args.prefill_steps,
                                                args.zipf_gamma, args.rank_beta)
        print(f"# prefill T={args.prefill}: {prefill['ms_per_step']:.2f} ms/step, tokens per expert "
              f"{prefill['tokens_per_expert']}", file=sys.stderr, flush=True)
    hetero = None
    if args.hetero:
        hetero = hetero_point(torch, latent, gsynth, [int(v) for v in args.hetero.split(",") if v.strip()],
                              max(10, args.steps // 4), 3)
        for pt in hetero["points"]:
            print(f"# hetero B={pt['batch']} ({pt['path']}): {pt['ms_per_step'] * 1e3:.1f} us/step, "
                  f"{pt['hbm_gbps_true_rank']:.0f} GB/s at true rank ({pt['hbm_gbps_padded']:.0f} padded)",
                  file=sys.stderr, flush=True)
    stack = None
    if args.stack:
        stack = stack_point(torch, latent, gsynth, args.stack, args.stack_batch, args.stack_steps)
        print(f"# stack {args.stack} layers B={args.stack_batch}: {stack['ms_per_step']:.2f} ms/step "
              f"({stack['us_per_layer']:.1f} us/layer, {stack['hbm_gbps']:.0f} GB/s; eager "
              f"{stack['eager_ms_per_step']:.2f} ms; generated in {stack['generate_s']:.1f} s; "
              f"{stack['resident_allocated_bytes'] / 1e9:.2f} GB allocated; replay == eager: "
              f"{stack['replay_equals_eager']})", file=sys.stderr, flush=True)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(torch, layers[0], routes, xs, args.batch, args.cpu_steps,
                           prefill_inputs if args.prefill else None, min(args.prefill, 1024))
        print(f"# cpu baseline: {cpu['value']:.2f} tokens/s ({cpu['cores']} threads), "
              f"{cpu['single_thread']['value']:.2f} (1 thread); prefill "
              f"{cpu['prefill']['value'] if cpu['prefill'] else 0:.1f} tokens/s", file=sys.stderr, flush=True)

    result = {
        "metric": METRIC,
        "value": head["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "timing": head["timing"],
        "eager_ms_per_step": head["eager_ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16" if head["path"] in ("stream", "prefill") else "f32",  # fp16 MFMA operands, fp32 accumulation
        "data": "synthetic (seeded closed-form low-rank factors packed NF4 g32 on the GPU; bf16 N(0,1) tokens; "
                "softmax top-8 routing)",
        "config": {
            "workload": "deepseek-v3-shaped LATENT MoE layer decode",
            "n_expert": E, "n_embd": D, "n_ff": FF, "rank": R, "top_k": K, "batch": args.batch,
            "layers_rotated": args.layers, "routings": args.routings,
        },
        "hbm_gbps": head["hbm_gbps"],
        "roofline": {
            "bound": "hbm",
            "achieved": head["hbm_gbps"],
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": head["roofline_frac"],
            "traffic": measured_traffic(head["path"]) if args.batch == 64 else None,
            "traffic_source": "profiles/%s (rocprofv3 --pmc)" % TRAFFIC_PROFILE.get(head["path"], ("none",))[0],
            "kernel": {
                "stream": "latent_moe_ffn_forward, streaming MFMA path: prep + 3 item kernels (A, B+C, D) + 2 "
                          "reductions + combine (7 launches per step; the step is the unit)",
            }.get(head["path"], "latent_moe_ffn_forward (prep + 3 phase kernels per step)"),
            "bytes_per_launch": head["bytes_per_step"],
        },
        "cpu_baseline": cpu,
        "sweep": sweep,
        "prefill": prefill,
        "hetero": hetero,
        "stack": stack,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
