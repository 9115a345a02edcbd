"""Benchmark of the routed-expert MoE layer on one MI355X.

Default workload (the headline config): int8 experts, decode M = 1 row, hidden 2048, expert FFN 768, 128 experts,
top-8 softmax routing from N(0, 1) router logits, per-row int8 activations, bf16 output; 48 distinct layer tables
(29 GB, far beyond the 256 MB Infinity Cache), the layers chained as a decode step chains them (each layer's output
is the next one's input). A step is one token through the 48 layers; four HIP graphs hold four tokens with their own
routing and are replayed in turn. The fused layer kernel (d3_moe_a8) runs each layer in one launch.

Other workloads of the same layer shape:
    --format w4a8 --rows 4                      W4A8 experts, 4 decode lines batched (uniform routing)
    --format w6a8 --routing zipf                W6A8 over 48 layers, experts per layer drawn from Zipf(1.1)
    --mode prefill                              FP8 experts, 256 rows at once, Zipf(1.1) routing: the grouped
                                                MFMA path (d3_moe_a8_prefill), 16 layers chained
    --mode resident --format fp8                the reference's own layouts and float activations (kernels.route +
                                                offload.resident_decode), the drop-in path for converted files
    --mode resident --rows 256 --routing zipf   its prompt path (offload.resident_prefill: grouped bf16 MFMA products)
    --mode gemv                                 one FP8 expert weight [1536, 2048] with a bf16 scale per output row
                                                against one bf16 row, dequantize-then-matmul semantics
                                                (kernels.fp8_linear): 128 distinct weights, one launch each

    --shape model                               the reference model's own layer: 256 experts of FFN 512

    python bench.py [--steps K] [--warmup W] [--mode decode|prefill|resident|block] [--format int8|w4a8|w6a8|fp8]
                    [--rows M] [--layers L] [--routing normal|zipf] [--shape config|model] [--no-cpu-baseline]
                    [--calibrate-copy]

Prints one JSON line: metric (expert-weight GB/s), tokens/s, the roofline of the layer (algorithmic bytes per launch
/ average launch time from HIP events on the replay stream, against 8 TB/s HBM) and the reference's CPU path timed on
a bounded sample of the same workload on this host. The default run (int8, one row) also times the other formats'
one-row layers (W4A8 and FP8 with normal routing, W6A8 with Zipf routing) under config.other_formats, and the other
workloads of the same layer under config.other_workloads: the single FP8 GEMV, W4A8 with 4 and 16 batched lines,
the 256-row FP8 prefill, the reference-format resident decode and 256-row prompt in the four formats and the int8
block (as their own modes run them, without the CPU leg).
"""
import argparse
import ctypes
import json
import math
import os
import pathlib
import sys
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "comfyui-drama3_amd"))

import torch  # noqa: E402

from drama3 import formats, moe  # noqa: E402

METRIC = "MoE-layer expert-weight HBM GB/s (% of peak) at M=1; decode tokens/s"
# HBM bytes per launch of the fused kernel, from rocprofv3 FETCH_SIZE / WRITE_SIZE passes scaled by the same counters
# on a plain copy kernel of known size (`--calibrate-copy`); keyed by (mode, format, rows)
TRAFFIC_PROFILES = {("decode", "int8", 1): ROOT / "profiles" / "moe_a8_int8_m1.md",
                    ("decode", "w4a8", 1): ROOT / "profiles" / "moe_a8_w4a8_m1.md",
                    ("decode", "fp8", 1): ROOT / "profiles" / "moe_a8_fp8_m1.md",
                    ("decode", "w6a8", 1): ROOT / "profiles" / "moe_a8_w6a8_m1_zipf.md",
                    ("decode", "w4a8", 4): ROOT / "profiles" / "moe_a8_w4a8_m4.md",
                    ("prefill", "fp8", 256): ROOT / "profiles" / "moe_a8_prefill_fp8_t256.md"}
PEAK_GBS = 8000.0
PEAK_FP8_TFLOPS = 5000.0
FORMATS = {"int8": formats.FMT_I8, "w4a8": formats.FMT_W4, "w6a8": formats.FMT_W6, "fp8": formats.FMT_F8}
DTYPES = {"int8": "int8", "w4a8": "int4xint8", "w6a8": "int6xint8", "fp8": "fp8e4m3"}
H, I, E, TOPK = 2048, 768, 128, 8
GRAPH_TOKENS = 4
ZIPF_S = 1.1


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def make_layers(fmt, layers, device, seed=0, experts=None):
    experts = E if experts is None else experts
    gen = torch.Generator(device=device).manual_seed(seed)
    banks = []
    for _ in range(layers):
        gu = torch.randn((experts, 2 * I, H), generator=gen, device=device) * 0.02
        gate_up = formats.quantize(gu, fmt)
        del gu
        dn = torch.randn((experts, H, I), generator=gen, device=device) * 0.02
        down = formats.quantize(dn, fmt)
        del dn
        banks.append((gate_up, down))
    return banks


def make_logits(routing, tokens, layers, rows, device, seed=1):
    """Router logits [tokens, layers, rows, E] bf16. normal: N(0, 1). zipf: log p(rank) + Gumbel noise with
    p(rank) ~ rank^-1.1 over a per-layer permutation of the experts, so the top-8 is a draw of 8 distinct experts
    without replacement from Zipf(1.1) (Gumbel-top-k)."""
    gen = torch.Generator(device=device).manual_seed(seed)
    if routing == "normal":
        return torch.randn((tokens, layers, rows, E), generator=gen, device=device).to(torch.bfloat16)
    ranks = torch.arange(1, E + 1, device=device, dtype=torch.float32)
    logp = -ZIPF_S * torch.log(ranks)
    out = torch.empty((tokens, layers, rows, E), device=device)
    for layer in range(layers):
        perm = torch.randperm(E, generator=gen, device=device)
        base = torch.empty(E, device=device)
        base[perm] = logp
        u = torch.rand((tokens, rows, E), generator=gen, device=device).clamp_(1e-12, 1 - 1e-7)
        out[:, layer] = base - torch.log(-torch.log(u))
    return out.to(torch.bfloat16)


def expert_bytes(gate_up, down):
    return gate_up.expert_bytes() + down.expert_bytes()


def cpu_threads():
    """Threads for the CPU path: every core this process may run on, within the CPU share the job is given (the
    OMP_NUM_THREADS the environment sets for it, when it sets one)."""
    affinity = len(os.sched_getaffinity(0))
    share = os.environ.get("OMP_NUM_THREADS")
    return min(affinity, int(share)) if share and share.isdigit() and int(share) > 0 else affinity


def cpu_baseline(banks, fmt, logits, x, grouped=False, budget_s=12.0, passes=None):
    """The reference's CPU path (oracle/cpu_path.py) on this host: bf16 matmuls from the quantized banks per routed
    expert, over a sample of the same layers and routing; GB/s over the same algorithmic bytes (each routed expert's
    weights once per layer pass). The sample rotates over `passes` (token, layer) pairs of distinct layers, each with
    its own routed experts copied to host memory, so that the working set (32 x 8 experts, 1.2 GB at int8) is far
    larger than the host's last-level cache and every pass reads its experts from DRAM, as the reference's does."""
    from oracle import cpu_path
    threads = cpu_threads()
    torch.set_num_threads(threads)
    passes = passes or (4 if grouped else 32)  # a prefill pass already reads ~126 experts (600 MB)
    per_expert = expert_bytes(*banks[0])
    lg = logits.cpu()
    xs = x.cpu()
    tokens, layers = lg.shape[0], len(banks)
    sample = []  # (token, layer, ids, weights, host banks of the routed experts only, ids renumbered)
    for i in range(min(passes, tokens * layers)):
        t, layer = i % tokens, (i * 7) % layers
        w, ids = torch.softmax(lg[t, layer].float(), -1).topk(TOPK, dim=-1)
        w = (w / w.sum(-1, keepdim=True)).to(torch.bfloat16)
        used = torch.unique(ids)
        local = torch.searchsorted(used, ids)
        host = []
        for b in banks[layer]:
            rows = b.weight.view(b.experts, b.rows, -1)[used.to(b.weight.device)].reshape(-1, b.weight.shape[1])
            scale = b.scale.view(b.experts, b.rows, *b.scale.shape[1:])[used.to(b.scale.device)]
            host.append((rows.cpu(), scale.reshape(-1, *b.scale.shape[1:]).cpu()))
        sample.append((t, local, w, host, len(used)))
    done, moved, started = 0, 0, time.perf_counter()
    while time.perf_counter() - started < budget_s:
        t, ids, w, host, n_used = sample[done % len(sample)]
        if grouped:
            cpu_path.grouped_layer(xs[t], ids, w, host[0], host[1], fmt, H, I)
            moved += n_used * per_expert + xs[t].shape[0] * (2 * H * 2 + E * 2)
        else:
            cpu_path.layer(xs[t, :1], ids[0], w[0], host[0], host[1], fmt, H, I)
            moved += TOPK * per_expert + 2 * H * 2 + E * 2
        done += 1
    elapsed = time.perf_counter() - started
    rows = xs.shape[1] if grouped else 1
    what = "cpu_path.grouped_layer" if grouped else "cpu_path.layer"
    return {"value": round(moved / elapsed / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "tokens_per_s": round(done * rows / elapsed / layers, 3),
            "sample": f"{done} layer passes ({rows} rows, top-8) rotating over {len(sample)} (token, layer) pairs of "
                      f"{len({(i * 7) % layers for i in range(len(sample))})} layers ({len(sample)} x their routed "
                      f"experts in host memory), {elapsed:.1f} s, torch {threads} threads of "
                      f"{len(os.sched_getaffinity(0))} in the affinity mask, {what}: _weight_int8pack_mm / "
                      f"dequantize-then-linear per expert"}


def measured_traffic(mode, fmt_name, rows):
    """HBM bytes per launch recorded in the workload's profile summary (line `traffic_bytes_per_launch: N`), or
    None."""
    path = TRAFFIC_PROFILES.get((mode, fmt_name, rows))
    if path is None or not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.strip().startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1].strip())
    return None


def calibrate_copy(device):
    """A plain elementwise kernel of known traffic for scaling the PMC byte counters: three launches that each read
    and write 256 MiB (float32 x * 1.0)."""
    a = torch.ones(64 << 20, dtype=torch.float32, device=device)
    b = torch.empty_like(a)
    for _ in range(3):
        torch.mul(a, 1.0, out=b)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "elementwise mul", "launches": 3, "read_bytes": a.numel() * 4,
                      "write_bytes": b.numel() * 4}), flush=True)


def timed_replays(graphs, stream, steps, warmup):
    for i in range(warmup):
        graphs[i % len(graphs)].replay()
    stream.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(steps):
        graphs[i % len(graphs)].replay()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end)


def run_decode(args, fmt, device):
    M, L = args.rows, args.layers
    log(f"building {L} layers of {args.format} experts")
    banks = make_layers(fmt, L, device)
    logits = make_logits(args.routing, GRAPH_TOKENS, L, M, device)
    gen = torch.Generator(device=device).manual_seed(2)
    x0 = torch.randn((GRAPH_TOKENS, M, H), generator=gen, device=device).to(torch.bfloat16)

    # routing of every (token, layer), for the exact count of experts each launch reads
    unique = []
    for t in range(GRAPH_TOKENS):
        x = x0[t]
        for layer, (gate_up, down) in enumerate(banks):
            x, ids, _ = moe.moe_layer(x, logits[t, layer], gate_up, down, TOPK, routing=True)
            unique.append(len(torch.unique(ids)))
    torch.cuda.synchronize()
    per_expert = expert_bytes(*banks[0])
    act_bytes = M * (2 * H * 2 + E * 2)
    bytes_per_token = [sum(unique[t * L:(t + 1) * L]) * per_expert + L * act_bytes for t in range(GRAPH_TOKENS)]

    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    graphs = []
    with torch.cuda.stream(stream):
        moe.prepare(device, H, I, stream)
        bufs = [x0[t].clone() for t in range(GRAPH_TOKENS)]
        for t in range(GRAPH_TOKENS):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                x = bufs[t]
                for layer, (gate_up, down) in enumerate(banks):
                    x = moe.moe_layer(x, logits[t, layer], gate_up, down, TOPK)
            graphs.append(g)
        ms = timed_replays(graphs, stream, args.steps, args.warmup)
    torch.cuda.synchronize()
    status = moe.status(device, H, I, stream)
    if status & moe.STATUS_INVALID:
        raise RuntimeError(f"fused layer reported status {status}")
    total_bytes = sum(bytes_per_token[i % GRAPH_TOKENS] for i in range(args.steps))
    launches = args.steps * L
    cpu = None
    if not args.no_cpu_baseline:
        log("timing the reference's CPU path")
        cpu = cpu_baseline(banks, fmt, logits[:, :, :1], x0[:, :1])
    config = {"workload": f"routed-expert MoE layer, {args.format} experts, decode M={M}, hidden {H}, FFN {I}, "
                          f"{E} experts top-{TOPK} ({args.routing} routing), {L} layers chained per token",
              "rows": M, "layers": L, "unique_experts_per_launch": round(sum(unique) / len(unique), 2),
              "waits_recomputed": bool(status & moe.STATUS_RECOMPUTED)}
    # the grouped path routes, quantizes and groups up to 16 rows in one launch
    kernel = "d3::moe_a8_one_row_kernel" if M == 1 else "d3::moe_a8_kernel" if M < moe.grouped_from_rows(fmt) else \
        f"d3_moe_a8_prefill ({5 if M <= 16 else 6} launches)"
    return ms, total_bytes, launches, args.steps * M, config, kernel, cpu


def run_block(args, fmt, device):
    """SparseMoeBlock.forward for M decode rows (moe.moe_block; one row in one launch, more in four): the router's
    logits from its bf16 weights [E, H], the routed experts, and a shared expert of the layer's format and shape with
    its gate, per layer. Algorithmic bytes: the routed experts read (once for all rows), the shared expert, the router
    and gate rows, x and out."""
    L, M = args.layers, args.rows
    log(f"building {L} layers of {args.format} experts, routers and shared experts")
    banks = make_layers(fmt, L, device)
    shared = make_layers(fmt, L, device, seed=5, experts=1)
    gen = torch.Generator(device=device).manual_seed(4)
    routers = [(torch.randn((E, H), generator=gen, device=device) * 0.02).to(torch.bfloat16) for _ in range(L)]
    gates = [(torch.randn((H,), generator=gen, device=device) * 0.05).to(torch.bfloat16) for _ in range(L)]
    x0 = torch.randn((GRAPH_TOKENS, M, H), generator=gen, device=device).to(torch.bfloat16)
    unique = []
    for t in range(GRAPH_TOKENS):
        x = x0[t]
        for layer, (gate_up, down) in enumerate(banks):
            x, ids, _ = moe.moe_block(x, gate_up, down, TOPK, router=routers[layer], shared=shared[layer],
                                      shared_gate=gates[layer], routing=True)
            unique.append(len(torch.unique(ids)))
    torch.cuda.synchronize()
    per_expert = expert_bytes(*banks[0])
    fixed = expert_bytes(*shared[0]) + E * H * 2 + H * 2 + M * 2 * H * 2
    bytes_per_token = [sum(unique[t * L:(t + 1) * L]) * per_expert + L * fixed for t in range(GRAPH_TOKENS)]
    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    graphs = []
    with torch.cuda.stream(stream):
        moe.prepare(device, H, I, stream)
        bufs = [x0[t].clone() for t in range(GRAPH_TOKENS)]
        for t in range(GRAPH_TOKENS):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                x = bufs[t]
                for layer, (gate_up, down) in enumerate(banks):
                    x = moe.moe_block(x, gate_up, down, TOPK, router=routers[layer], shared=shared[layer],
                                      shared_gate=gates[layer])
            graphs.append(g)
        ms = timed_replays(graphs, stream, args.steps, args.warmup)
    torch.cuda.synchronize()
    status = moe.status(device, H, I, stream)
    if status & moe.STATUS_INVALID:
        raise RuntimeError(f"fused layer reported status {status}")
    total_bytes = sum(bytes_per_token[i % GRAPH_TOKENS] for i in range(args.steps))
    config = {"workload": f"MoE block (router {E}x{H} bf16, routed {args.format} experts top-{TOPK}, shared expert "
                          f"of FFN {I} with its gate), decode M={M}, hidden {H}, FFN {I}, {L} layers chained per token",
              "rows": M, "layers": L, "unique_experts_per_launch": round(sum(unique) / len(unique), 2),
              "waits_recomputed": bool(status & moe.STATUS_RECOMPUTED)}
    kernel = ("d3::moe_a8_one_row_kernel (block)" if M == 1 else
              "router_logits_kernel, d3_moe_a8 (routed, one expert for the shared), block_combine_kernel")
    return ms, total_bytes, args.steps * L, args.steps * M, config, kernel, None


def run_prefill(args, fmt, device):
    T, L = args.rows, args.layers
    log(f"building {L} layers of {args.format} experts")
    banks = make_layers(fmt, L, device)
    logits = make_logits(args.routing, 1, L, T, device)[0]
    gen = torch.Generator(device=device).manual_seed(2)
    x0 = torch.randn((T, H), generator=gen, device=device).to(torch.bfloat16)
    unique = []
    x = x0
    for layer, (gate_up, down) in enumerate(banks):
        x, ids, _ = moe.moe_prefill(x, gate_up, down, TOPK, logits=logits[layer], routing=True)
        unique.append(len(torch.unique(ids)))
    torch.cuda.synchronize()
    per_expert = expert_bytes(*banks[0])
    step_bytes = sum(unique) * per_expert + L * T * (2 * H * 2 + E * 2)
    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(stream):
        buf = x0.clone()
        moe.moe_prefill(buf, *banks[0], TOPK, logits=logits[0])  # warm the allocator on this stream
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            x = buf
            for layer, (gate_up, down) in enumerate(banks):
                x = moe.moe_prefill(x, gate_up, down, TOPK, logits=logits[layer])
        ms = timed_replays([g], stream, args.steps, args.warmup)
    torch.cuda.synchronize()
    cpu = None
    if not args.no_cpu_baseline:
        log("timing the reference's CPU path")
        sample = min(T, 32)
        cpu = cpu_baseline(banks, fmt, logits[None, :, :sample], x0[None, :sample], grouped=True)
    flops = 2 * TOPK * T * (2 * I * H + H * I)
    config = {"workload": f"routed-expert MoE layer, {args.format} experts, {T} rows at once (prefill), hidden {H}, "
                          f"FFN {I}, {E} experts top-{TOPK} ({args.routing} routing), {L} layers chained",
              "rows": T, "layers": L, "unique_experts_per_launch": round(sum(unique) / len(unique), 2),
              "mfma_tflops": round(flops * L * args.steps / (ms * 1e-3) / 1e12, 2),
              "mfma_frac_fp8_peak": round(flops * L * args.steps / (ms * 1e-3) / 1e12 / PEAK_FP8_TFLOPS, 5)}
    return (ms, step_bytes * args.steps, args.steps * L, args.steps * T, config,
            f"d3_moe_a8_prefill ({5 if T <= 16 else 6} launches)", cpu)


def run_gemv(args, fmt, device):
    """One FP8 expert weight [1536, 2048] with a bf16 scale per output row (absmax / 448) against one bf16 row,
    dequantize-then-matmul semantics (kernels.fp8_linear, d3_gemv_fp8_rows): x ~ N(0, 1), weights ~ N(0, 0.02), seed
    0. `layers` distinct weights (128: 400 MB, beyond the Infinity Cache), one launch each, in one graph; also the same
    weights as one stacked matrix in one launch (how experts_decode's gate_up multiplies k experts at once). The CPU
    leg times the reference's path, dequantize to bf16 then torch's bf16 linear, on the host."""
    from drama3 import kernels
    N, K, count = 2 * I, H, args.layers
    gen = torch.Generator(device=device).manual_seed(0)
    x = torch.randn((1, K), generator=gen, device=device).to(torch.bfloat16)
    weights = torch.empty((count * N, K), dtype=torch.uint8, device=device)
    scales = torch.empty((count * N,), dtype=torch.bfloat16, device=device)
    for m in range(count):
        bank = formats.quantize(torch.randn((1, N, K), generator=gen, device=device) * 0.02, formats.FMT_F8)
        weights[m * N:(m + 1) * N] = bank.weight
        scales[m * N:(m + 1) * N] = bank.scale
    mats = [(weights[m * N:(m + 1) * N], scales[m * N:(m + 1) * N]) for m in range(count)]
    bytes_per_call = N * K + N * 2 + K * 2 + N * 2  # weight bytes, row scales, x in, y out
    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(stream):
        outs = [kernels.fp8_linear(x, w, sc) for w, sc in mats]
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            outs = [kernels.fp8_linear(x, w, sc) for w, sc in mats]
        ms = timed_replays([g], stream, args.steps, args.warmup)
        kernels.fp8_linear(x, weights, scales)
        gs = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gs, stream=stream):
            stacked = kernels.fp8_linear(x, weights, scales)
        ms_stacked = timed_replays([gs], stream, args.steps, args.warmup)
    torch.cuda.synchronize()
    if not torch.equal(stacked[0, :N], outs[0][0]):
        raise RuntimeError("stacked and single launches differ")
    launches = args.steps * count
    stacked_gbs = (bytes_per_call - K * 2) * count * args.steps / (ms_stacked * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu_baseline:
        log("timing the reference's CPU path")
        from oracle import cpu_path
        threads = cpu_threads()
        torch.set_num_threads(threads)
        host = [(w.cpu().view(torch.float8_e4m3fn), sc.cpu()) for w, sc in mats[:32]]  # 100 MB, beyond the LLC
        xc = x.cpu()
        done, started = 0, time.perf_counter()
        while time.perf_counter() - started < 10.0:
            w, sc = host[done % len(host)]
            cpu_path.fp8_rows_linear(xc, w, sc)
            done += 1
        elapsed = time.perf_counter() - started
        cpu = {"value": round(done * bytes_per_call / elapsed / 1e9, 3), "unit": "GB/s", "cores": threads,
               "kind": "port", "us_per_call": round(elapsed / done * 1e6, 2),
               "sample": f"{done} calls rotating over {len(host)} distinct weights in host memory, {elapsed:.1f} s, "
                         f"torch {threads} threads of {len(os.sched_getaffinity(0))} in the affinity mask, "
                         f"cpu_path.fp8_rows_linear: dequantize to bf16, then torch's bf16 linear"}
    config = {"workload": f"FP8 expert weight [{N}, {K}] with a bf16 scale per output row, one bf16 row, dequantize "
                          f"then matmul (fp8_linear), {count} distinct weights, one launch each",
              "rows": 1, "weights": count, "us_per_call": round(ms * 1e3 / launches, 3),
              "stacked_one_launch_gbs": round(stacked_gbs, 1),
              "stacked_one_launch_us": round(ms_stacked * 1e3 / args.steps, 2)}
    return ms, bytes_per_call * launches, launches, launches, config, "d3::gemv_fp8_rows_kernel", cpu


STREAM_BYTES = 2 << 30            # the streaming-read buffer: 2 GiB, far beyond the 256 MB Infinity Cache
STREAM_GRIDS = (2048, 8192, 16384, 32768, 65536)
ONE_SHOT_BYTES = {"w4a8 layer (19.5 MB)": 8 * 2_433_024, "int8 layer (37.8 MB)": 8 * 4_725_760}
EMPTY_GRID = 768                  # the one-row layer's grid


def measure_ceiling(device, layers=48, steps=50, warmup=5):
    """What the device allows a layer, measured with the library's probe kernels (d3_stream_read, d3_empty_launch):
    - stream_read_gbs: one 2 GiB buffer read once per launch, the best of a few grids, 10 launches timed;
    - one_shot: `layers` distinct buffers of a layer's bytes, one read launch each, chained in a graph as the layers
      are: us per launch (the gap between graph nodes included) and GB/s, at grids of one, four and eight 16-byte
      loads per thread;
    - empty_launch_us: `layers` empty launches of the one-row layer's grid in a graph, us per node."""
    from drama3 import _lib
    lib = _lib.lib()
    sink = torch.zeros(4, dtype=torch.int32, device=device)
    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    handle = ctypes.c_void_p(stream.cuda_stream)
    out = {}
    with torch.cuda.stream(stream):
        big = torch.ones(STREAM_BYTES // 4, dtype=torch.int32, device=device)
        best = None
        per_grid = {}
        for grid in STREAM_GRIDS:
            for _ in range(3):
                _lib.check(lib.d3_stream_read(big.data_ptr(), STREAM_BYTES, sink.data_ptr(), grid, handle), "read")
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(stream)
            for _ in range(10):
                _lib.check(lib.d3_stream_read(big.data_ptr(), STREAM_BYTES, sink.data_ptr(), grid, handle), "read")
            end.record(stream)
            end.synchronize()
            gbs = 10 * STREAM_BYTES / (start.elapsed_time(end) * 1e-3) / 1e9
            per_grid[grid] = round(gbs, 1)
            best = gbs if best is None else max(best, gbs)
        del big
        out["stream_read_gbs"] = round(best, 1)
        out["stream_read_gbs_by_grid"] = per_grid
        one_shot = {}
        for name, nbytes in ONE_SHOT_BYTES.items():
            nbytes -= nbytes % 16
            bufs = [torch.ones(nbytes // 4, dtype=torch.int32, device=device) for _ in range(layers)]
            runs = {}
            for loads in (1, 4, 8):
                grid = -(-nbytes // (16 * 256 * loads))
                for b in bufs:  # outside capture first, as the graph will run it
                    _lib.check(lib.d3_stream_read(b.data_ptr(), nbytes, sink.data_ptr(), grid, handle), "read")
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=stream):
                    for b in bufs:
                        _lib.check(lib.d3_stream_read(b.data_ptr(), nbytes, sink.data_ptr(), grid, handle), "read")
                ms = timed_replays([g], stream, steps, warmup)
                us = ms * 1e3 / (steps * layers)
                runs[f"grid {grid}"] = {"us_per_launch": round(us, 3), "gbs": round(nbytes / (us * 1e-6) / 1e9, 1)}
                del g
            del bufs
            torch.cuda.empty_cache()
            one_shot[name] = runs
        out["one_shot"] = one_shot
        _lib.check(lib.d3_empty_launch(EMPTY_GRID, handle), "empty")
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for _ in range(layers):
                _lib.check(lib.d3_empty_launch(EMPTY_GRID, handle), "empty")
        ms = timed_replays([g], stream, steps, warmup)
        out["empty_launch_us"] = round(ms * 1e3 / (steps * layers), 3)
        out["empty_launch_grid"] = EMPTY_GRID
    torch.cuda.synchronize()
    return out


def run_ceiling(args, fmt, device):
    """--mode ceiling: measure_ceiling alone, one JSON line."""
    ceiling = measure_ceiling(device, layers=args.layers, steps=args.steps, warmup=args.warmup)
    print(json.dumps({"metric": "device ceiling: streaming HBM read, one-shot layer reads, empty launches",
                      "value": ceiling["stream_read_gbs"], "unit": "GB/s", "n_gpus": 1, "higher_is_better": True,
                      "peak": PEAK_GBS, "data": "synthetic", "config": {"workload": "probe kernels", **ceiling}}),
          flush=True)


def decode_summary(args, fmt_name, routing, device):
    """One-row decode of another format (same shape, 48 layers), as run_decode measures it: a dict for
    config.other_formats."""
    sub = argparse.Namespace(**vars(args))
    sub.format, sub.routing, sub.rows, sub.no_cpu_baseline = fmt_name, routing, 1, True
    ms, total_bytes, launches, tokens, config, kernel, _ = run_decode(sub, FORMATS[fmt_name], device)
    torch.cuda.empty_cache()
    launch_us = ms * 1e3 / launches
    gbs = total_bytes / launches / (launch_us * 1e-6) / 1e9
    return {"format": fmt_name, "routing": routing, "us_per_layer": round(launch_us, 3), "gbs": round(gbs, 1),
            "frac_of_peak": round(gbs / PEAK_GBS, 4), "tokens_per_s": round(tokens / (ms * 1e-3), 2),
            "bytes_per_launch": int(total_bytes / launches),
            "unique_experts_per_launch": config["unique_experts_per_launch"],
            "traffic": measured_traffic("decode", fmt_name, 1)}


def workload_summary(args, device, mode, fmt_name, rows, routing, layers, steps, warmup):
    """Another workload of the layer, run as its own mode runs it by default (layers, steps, warmup): a dict for
    config.other_workloads."""
    sub = argparse.Namespace(**vars(args))
    sub.mode, sub.format, sub.rows, sub.routing = mode, fmt_name, rows, routing
    sub.layers, sub.steps, sub.warmup, sub.no_cpu_baseline = layers, steps, warmup, True
    sub.routed, sub.launches = True, 2  # resident: the routing in the gate_up launch, as `--routed`
    run = {"prefill": run_prefill, "gemv": run_gemv, "resident": run_resident, "block": run_block}.get(mode, run_decode)
    ms, total_bytes, launches, tokens, config, kernel, _ = run(sub, FORMATS[fmt_name], device)
    torch.cuda.empty_cache()
    launch_us = ms * 1e3 / launches
    gbs = total_bytes / launches / (launch_us * 1e-6) / 1e9
    return {"workload": config["workload"], "mode": mode, "format": fmt_name, "rows": rows, "routing": routing,
            "us_per_launch": round(launch_us, 3), "gbs": round(gbs, 1), "frac_of_peak": round(gbs / PEAK_GBS, 4),
            "calls_per_s" if mode == "gemv" else "rows_per_s": round(tokens / (ms * 1e-3), 2),
            "bytes_per_launch": int(total_bytes / launches), "kernel": kernel,
            "traffic": measured_traffic(mode, fmt_name, rows)}


def make_reference_banks(fmt_name, layers, device, seed=3):
    """Banks in the reference's own layouts (offload.py:72-90, 264-273) with random codes and scales of the right
    shapes and ranges: int8 rows with float32 row scales, FP8 rows with 128 x 128 float32 block scales, W4A8 / W6A8
    code rows with e4m3 group-16 scales, float32 channel scales and a codebook at 4 bits."""
    gen = torch.Generator(device=device).manual_seed(seed)
    kind = {"int8": "int8", "fp8": "fp8", "w4a8": "w4", "w6a8": "w6"}[fmt_name]
    out = []
    for _ in range(layers):
        banks = []
        for n, k in ((2 * I, H), (H, I)):
            if kind == "int8":
                f = {"_qdata": torch.randint(-127, 128, (E * n, k), generator=gen, device=device, dtype=torch.int8),
                     "scale": torch.rand((E * n,), generator=gen, device=device) * 1e-3}
            elif kind == "fp8":
                w = torch.randint(0, 0x7E, (E * n, k), generator=gen, device=device, dtype=torch.uint8)
                w |= torch.randint(0, 2, (E * n, k), generator=gen, device=device, dtype=torch.uint8) << 7
                f = {"weight": w, "scale": torch.rand((E * n // 128, k // 128), generator=gen, device=device) * 1e-2}
            else:
                bits = int(kind[1])
                f = {"_qdata": torch.randint(0, 256, (E * n, k * bits // 8), generator=gen, device=device,
                                             dtype=torch.uint8),
                     "scale": torch.randint(0x28, 0x38, (E * n, k // 16), generator=gen, device=device,
                                            dtype=torch.uint8),
                     "s_channel": torch.rand((E * n,), generator=gen, device=device) * 1e-3}
            banks.append(f)
        cb = (torch.linspace(-8, 7, 16, device=device),) * 2 if kind == "w4" else (None, None)
        out.append((kind, tuple(banks), cb))
    return out


def bank_bytes(fields):
    return sum(t.numel() * t.element_size() for t in fields.values()) // E


def run_resident_prompt(args, fmt, device):
    """The reference-format prompt path (kernels.route + offload.resident_prefill: the pairs grouped by expert, the
    rows gathered, rotated and split into bf16 planes, the grouped products on the matrix cores per bank, the SwiGLU
    between them, the weighted sum) over args.rows rows, L layers in one HIP graph, each layer over the same rows."""
    from drama3 import kernels, offload
    T, L = args.rows, args.layers
    log(f"building {L} layers of {args.format} experts in the reference's layouts")
    layers = make_reference_banks(args.format, L, device)
    logits = make_logits(args.routing, 1, L, T, device)[0]
    gen = torch.Generator(device=device).manual_seed(2)
    x0 = torch.randn((T, H), generator=gen, device=device).to(torch.bfloat16)
    rows = (2 * I, H)

    def layer_step(x, layer):
        kind, banks, cbs = layers[layer]
        ids, w = kernels.route(logits[layer], TOPK)
        return offload.resident_prefill(x, ids, w, banks, rows, kind, cbs, E)

    unique = [len(torch.unique(kernels.route(logits[layer], TOPK)[0])) for layer in range(L)]
    per_expert = sum(bank_bytes(f) for f in layers[0][1])
    step_bytes = sum(unique) * per_expert + L * T * (2 * H * 2 + E * 2)
    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(stream):
        for layer in range(L):  # constants and allocator pools before capture
            layer_step(x0, layer)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for layer in range(L):
                layer_step(x0, layer)
        ms = timed_replays([g], stream, args.steps, args.warmup)
    torch.cuda.synchronize()
    # the matrix-core products as issued: three planes of both banks' rows (int8 planes on the int8 cores for int8 and
    # the codes; bf16 planes for fp8, one for its gate_up, whose rows are bf16 already)
    flops = 2 * TOPK * T * ((1 if args.format == "fp8" else 3) * 2 * I * H + 3 * H * I)
    config = {"workload": f"routed-expert MoE layer in the reference's {args.format} layout (float activations, "
                          f"route + resident_prefill), {T} rows at once (prefill), hidden {H}, FFN {I}, {E} experts "
                          f"top-{TOPK} ({args.routing} routing), {L} layers", "rows": T, "layers": L,
              "unique_experts_per_launch": round(sum(unique) / len(unique), 2),
              "us_per_layer": round(ms * 1e3 / (args.steps * L), 2),
              "mfma_ops_per_s_e12": round(flops * L * args.steps / (ms * 1e-3) / 1e12, 2),
              "mfma_type": "bf16" if args.format == "fp8" else "int8"}
    return (ms, step_bytes * args.steps, args.steps * L, args.steps * T, config,
            "route + resident_prefill (d3::grouped_i8_kernel / grouped_fp8_kernel per bank, 7 launches)", None)


def run_resident(args, fmt, device):
    """The reference-format decode path (kernels.route + offload.resident_decode: rotate, gemv, rotate(SwiGLU),
    gemv, weighted sum; FP8 without the rotations), one row, layers chained in HIP graphs; with more rows, the prompt
    path (run_resident_prompt)."""
    from drama3 import kernels, offload
    if args.rows > 1:
        return run_resident_prompt(args, fmt, device)
    L = args.layers
    offload.RESIDENT_LAUNCHES = args.launches
    log(f"building {L} layers of {args.format} experts in the reference's layouts")
    layers = make_reference_banks(args.format, L, device)
    logits = make_logits(args.routing, GRAPH_TOKENS, L, 1, device)
    gen = torch.Generator(device=device).manual_seed(2)
    x0 = torch.randn((GRAPH_TOKENS, 1, H), generator=gen, device=device).to(torch.bfloat16)
    rows = (2 * I, H)

    def layer_step(x, lg, layer):
        kind, banks, cbs = layers[layer]
        if args.routed:  # the routing in the gate_up launch's prologue
            return offload.routed_decode(x, lg, TOPK, banks, rows, kind, cbs)[0]
        ids, w = kernels.route(lg, TOPK)
        return offload.resident_decode(x, ids[0], w[0], banks, rows, kind, cbs)

    per_expert = sum(bank_bytes(f) for f in layers[0][1])
    layer_bytes = TOPK * per_expert + 2 * H * 2 + E * 2
    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    graphs = []
    with torch.cuda.stream(stream):
        x = x0[0]
        for layer in range(L):  # constants and allocator pools before capture
            x = layer_step(x, logits[0, layer], layer)
        bufs = [x0[t].clone() for t in range(GRAPH_TOKENS)]
        for t in range(GRAPH_TOKENS):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                x = bufs[t]
                for layer in range(L):
                    x = layer_step(x, logits[t, layer], layer)
            graphs.append(g)
        ms = timed_replays(graphs, stream, args.steps, args.warmup)
    torch.cuda.synchronize()
    if args.launches == 1:
        what = ("routed_decode (1 launch: the routing, gate_up, down)" if args.routed else
                "route + resident_decode (2 launches: route, then gate_up and down)")
    else:
        what = ("routed_decode (2 launches: gate_up with the routing, down)" if args.routed else
                "route + resident_decode (3 launches: route, gate_up, down)")
    config = {"workload": f"routed-expert MoE layer in the reference's {args.format} layout (float activations, "
                          f"{'routed_decode' if args.routed else 'route + resident_decode'}), decode M=1, hidden {H}, "
                          f"FFN {I}, {E} experts top-{TOPK}, {L} layers chained per token", "rows": 1, "layers": L,
              "unique_experts_per_launch": TOPK}
    return ms, layer_bytes * L * args.steps, args.steps * L, args.steps, config, what, None


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=None)
    p.add_argument("--warmup", type=int, default=None)
    p.add_argument("--mode", default="decode", choices=["decode", "prefill", "resident", "block", "gemv", "ceiling"])
    p.add_argument("--routed", action="store_true", help="--mode resident: route inside the gate_up launch")
    p.add_argument("--launches", type=int, default=2, choices=[1, 2],
                   help="--mode resident: the two-launch decode (default) or the one-launch one")
    p.add_argument("--format", default=None, choices=sorted(FORMATS))
    p.add_argument("--rows", type=int, default=None)
    p.add_argument("--layers", type=int, default=None)
    p.add_argument("--routing", default=None, choices=["normal", "zipf"])
    p.add_argument("--shape", default="config", choices=["config", "model"],
                   help="config: 128 experts of FFN 768 (the headline layer); model: 256 experts of FFN 512, the "
                        "reference model's own layer (drama3/fish/config.json)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--calibrate-copy", action="store_true", help="only run the copy kernel that scales PMC counters")
    p.add_argument("--headline-only", action="store_true", help="the default run without the other formats' lines")
    args = p.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the routed-expert path runs on one MI355X, each GPU holding every expert "
              "of every layer (decode lines split across GPUs need no exchange); run it with --gpus 1",
              file=sys.stderr)
        sys.exit(2)
    prefill = args.mode == "prefill"
    default_run = args.mode == "decode" and args.format is None and args.rows is None and args.routing is None
    args.format = args.format or ("fp8" if prefill or args.mode == "gemv" else "int8")
    args.rows = args.rows or (256 if prefill else 1)
    prompt = prefill or (args.mode == "resident" and args.rows > 1)
    args.layers = args.layers or (16 if prefill else 8 if prompt else 128 if args.mode == "gemv" else 48)
    args.routing = args.routing or ("zipf" if prompt else "normal")
    args.steps = args.steps or (20 if prefill else 10 if prompt else 100)
    args.warmup = args.warmup if args.warmup is not None else (3 if prefill else 8)
    fmt = FORMATS[args.format]
    global E, I
    if args.shape == "model":
        E, I = 256, 512
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    if args.calibrate_copy:
        calibrate_copy(device)
        return
    if args.mode == "ceiling":
        run_ceiling(args, fmt, device)
        return

    run = {"prefill": run_prefill, "resident": run_resident, "block": run_block, "gemv": run_gemv}.get(args.mode,
                                                                                                     run_decode)
    ms, total_bytes, launches, tokens, config, kernel, cpu = run(args, fmt, device)
    ceiling = None
    if default_run and args.shape == "config":
        log("measuring the device's ceiling (streaming read, one-shot layer reads, empty launches)")
        ceiling = measure_ceiling(device, steps=20, warmup=3)
        config["ceiling"] = ceiling
    if default_run and args.shape == "config" and not args.headline_only:
        # the north star's target formats at one row, and the 48-layer Zipf sweep of W6A8
        config["other_formats"] = []
        for fmt_name, routing in (("w4a8", "normal"), ("fp8", "normal"), ("w6a8", "zipf")):
            log(f"timing {fmt_name} one-row decode ({routing} routing)")
            config["other_formats"].append(decode_summary(args, fmt_name, routing, device))
        # the other workloads of the layer: the single FP8 GEMV, W4A8 batched lines, the FP8 prefill; and the drop-in
        # paths around it: the reference-format resident decode (routing in the gate_up launch) in every format, and
        # the block with the router and the shared expert
        config["other_workloads"] = []
        for mode, fmt_name, rows, routing, layers, steps, warmup in (("gemv", "fp8", 1, "normal", 128, 100, 8),
                                                                     ("decode", "w4a8", 4, "normal", 48, 100, 8),
                                                                     ("decode", "w4a8", 16, "normal", 48, 100, 8),
                                                                     ("prefill", "fp8", 256, "zipf", 16, 20, 3),
                                                                     ("resident", "int8", 1, "normal", 48, 100, 8),
                                                                     ("resident", "fp8", 1, "normal", 48, 100, 8),
                                                                     ("resident", "w4a8", 1, "normal", 48, 100, 8),
                                                                     ("resident", "w6a8", 1, "normal", 48, 100, 8),
                                                                     ("resident", "int8", 256, "zipf", 8, 10, 2),
                                                                     ("resident", "fp8", 256, "zipf", 8, 10, 2),
                                                                     ("resident", "w4a8", 256, "zipf", 8, 10, 2),
                                                                     ("resident", "w6a8", 256, "zipf", 8, 10, 2),
                                                                     ("block", "int8", 1, "normal", 48, 100, 8),
                                                                     ("block", "int8", 4, "normal", 48, 100, 8)):
            log(f"timing {mode} {fmt_name}, {rows} rows")
            config["other_workloads"].append(workload_summary(args, device, mode, fmt_name, rows, routing, layers,
                                                              steps, warmup))
    gbs = total_bytes / (ms * 1e-3) / 1e9
    launch_us = ms * 1e3 / launches
    bytes_per_launch = total_bytes / launches
    config.update({"tokens_per_s": round(tokens / (ms * 1e-3), 2), "pct_of_peak_hbm": round(100 * gbs / PEAK_GBS, 2),
                   "bytes_per_launch": int(bytes_per_launch)})
    achieved = bytes_per_launch / (launch_us * 1e-6) / 1e9
    line = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms / args.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": DTYPES[args.format],
        "data": f"synthetic: weights N(0, 0.02) quantized, activations N(0, 1), router logits "
                f"{'N(0, 1)' if args.routing == 'normal' else 'Zipf(1.1) Gumbel-top-k'}, seeded",
        "config": config,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_GBS, 4), "traffic": measured_traffic(args.mode, args.format, args.rows)
                     if args.shape == "config" else None,
                     "kernel": kernel, "launch_us": round(launch_us, 3),
                     "measured_peak": None if ceiling is None else ceiling["stream_read_gbs"],
                     "frac_of_measured_peak": None if ceiling is None else
                     round(achieved / ceiling["stream_read_gbs"], 4)},
        "cpu_baseline": cpu,
    }
    if not math.isfinite(gbs):
        raise RuntimeError("no time measured")
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
