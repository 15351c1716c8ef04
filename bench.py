"""Benchmark of the paged-KV decode hot path on one MI355X.

Default workload: config C2 of BASELINE.json -- one Llama-3-8B-shaped attention
layer over int8 (G64) paged KV, B=32 sequences with context lengths drawn from
U[1024, 8192] (seed 1).  One step = append-quantize one new K/V token per
sequence + paged attention of the new query over all L_b + 1 tokens.

Steps rotate over ``--layers`` independent layer pools (default 4, ~1.3 GB of
KV) so that a step never finds its KV in the 256 MB Infinity Cache, the same
access pattern a 32-layer model has.  Inputs are synthetic and resident in HBM
before timing.  The timed steps are captured as one HIP graph and replayed
once untimed, then once timed for the step time (``--eager`` launches them
from the host instead); ``roofline.achieved`` divides the algorithmic bytes
(or flops) of a launch by its average duration: HIP events around a graph
replay of the timed steps' attention launches, over the launch count, with
the stream held by a spin kernel while the host submits the graph, so that
the span holds GPU work only (``roofline.kernel_timing``; beside it: the
launch inside the step, step graph time minus an append-only graph's, and
events around each launch of a host-launched pass, which add their own
overhead).  For the HBM-bound
decode workloads ``roofline.read_probe`` times ``pkv_read_probe`` -- a kernel
that only reads every byte of the pages the step's sequences hold, at the
same wave count -- the same way, and ``roofline.frac_of_read_probe`` compares
the launch with it.  Prints one JSON line (rank 0).

    python bench.py [--gpus 1] [--steps 100] [--warmup 20] [--workload c2]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "mlx-one_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBS = 8000.0  # MI355X published HBM3E bandwidth
MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense fp16/bf16 MFMA (no sparsity)
# GPU clock cycles the stream is held per step of the event pass (~100 us of
# host enqueue time per step at ~2.4 GHz)
SLEEP_CYCLES_PER_STEP = 240_000
# GPU clock cycles the stream is held before a timed graph replay (~1 ms): the
# host submits the graph's launches meanwhile, so the first one starts right
# after the opening event and the span holds GPU work only
GRAPH_HOLD_CYCLES = 2_400_000


def held_replay(graph, device):
    """Replay ``graph`` between two HIP events, the stream held by a bounded
    spin kernel while the host submits it; returns the span in ms."""
    import torch

    stream = torch.cuda.current_stream(device)
    span = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
    torch.cuda._sleep(GRAPH_HOLD_CYCLES)
    span[0].record(stream)
    graph.replay()
    span[1].record(stream)
    torch.cuda.synchronize()
    return span[0].elapsed_time(span[1])


def measured_traffic(workload):
    """HBM bytes per attention launch measured with rocprofv3 PMC counters
    (FETCH_SIZE + WRITE_SIZE, calibrated on a copy kernel), as recorded in
    profiles/pkv_attention_<workload>_traffic.md; None when not profiled."""
    path = ROOT / "profiles" / f"pkv_attention_{workload}_traffic.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1])
    return None


def kv_bytes_per_token(w):
    """K+V bytes of one cached token: 2*HK*(D*bits/8 + (D/G)*4), or 2*HK*D*2 for bf16."""
    if w.bits == 16:
        return 2 * w.kv_heads * w.head_dim * 2
    return 2 * w.kv_heads * (w.head_dim * w.bits // 8 + (w.head_dim // w.group_size) * 4)


def algorithmic_bytes(w, lengths):
    """Algorithmic bytes of the attention launch and of the whole step.

    ``lengths`` are the tokens attended per sequence (after the append).
    Attention: every cached token's K/V once, queries and outputs (bf16), one
    4-byte block-table entry per page.  Step (the C2 formula):
    attention + the new bf16 K/V rows the append reads.
    """
    tokens = float(sum(lengths))
    kv = kv_bytes_per_token(w) * tokens
    qo = w.batch * w.heads * w.num_queries * w.head_dim * 2 * 2
    table = 4 * sum(math.ceil(x / w.page_tokens) for x in lengths)
    attention = kv + qo + table
    new_rows = float(w.step_appends().sum()) * 2 * w.kv_heads * w.head_dim * 2
    return attention, attention + new_rows


def is_prefill(w):
    """Query blocks past 32 rows per KV head run on the MFMA prefill kernel."""
    return w.num_queries * (w.heads // w.kv_heads) > 32


def attention_flops(w, lengths, widths=None):
    """Causal-exact flops of one attention launch: 4*D per (query row, visible
    token) for QK^T and PV.  Query q of a chunk of Q sits at L - Q + q and sees
    L - Q + q + 1 tokens, so a sequence costs 4*D*H*(Q*(L - Q) + Q*(Q + 1)/2)
    (Q = the sequence's width in a mixed batch)."""
    widths = [w.num_queries] * len(lengths) if widths is None else widths
    pairs = sum(q * (int(x) - q) + q * (q + 1) // 2 for x, q in zip(lengths, widths))
    return 4.0 * w.head_dim * w.heads * pairs


def mixed_roofline(w, lengths):
    """A mixed batch's two bounds: the decode rows' algorithmic bytes (KV, Q/O,
    block table) at the HBM peak and the prefill rows' flops at the MFMA peak;
    ``ideal_ms`` is their sum, a lower bound for the launch."""
    widths = [int(x) for x in w.step_widths()]
    small = [i for i, q in enumerate(widths) if q * (w.heads // w.kv_heads) <= 32]
    large = [i for i in range(len(widths)) if i not in small]
    dec_bytes = kv_bytes_per_token(w) * sum(float(lengths[i]) for i in small) + len(small) * (
        w.heads * w.head_dim * 2 * 2) + 4 * sum(math.ceil(lengths[i] / w.page_tokens)
                                                for i in small)
    flops = attention_flops(w, [lengths[i] for i in large], [widths[i] for i in large])
    ideal_ms = (dec_bytes / (HBM_PEAK_GBS * 1e9) + flops / (MFMA_PEAK_TFLOPS * 1e12)) * 1e3
    return dec_bytes, flops, ideal_ms


class Layer:
    """One layer's page pool, filled with the workload's context tokens."""

    def __init__(self, w, inst, index, fmt, device):
        import numpy as np
        import torch

        from pkv import ops

        self.fmt = fmt
        self.pool = ops.allocate_pool(fmt, inst.num_pages, device)
        self.table = torch.from_numpy(inst.table).to(device)
        gen = torch.Generator(device=device)
        gen.manual_seed(1000 * w.seed + index)
        rng = np.random.default_rng([w.seed, index, 7])
        channels = w.kv_heads * w.head_dim
        picks = []
        for _ in range(2):
            count = max(1, int(round(w.outlier_fraction * channels))) if w.outlier_fraction else 0
            pick = rng.choice(channels, count, replace=False) if count else np.zeros(0, np.int64)
            picks.append(np.divmod(pick, w.head_dim))
        lengths = inst.context.astype(np.int64)
        chunk = 256
        for start in range(0, int(lengths.max()), chunk):
            width = np.clip(lengths - start, 0, chunk).astype(np.int32)
            kv = []
            for side in range(2):
                x = torch.randn((w.batch, w.kv_heads, chunk, w.head_dim), generator=gen,
                                device=device, dtype=torch.float32)
                hk, d = picks[side]
                if len(hk):
                    x[:, torch.from_numpy(hk).to(device), :, torch.from_numpy(d).to(device)] *= (
                        w.outlier_scale)
                kv.append(x.to(fmt.dtype))
            ops.append_quantize(fmt, self.pool, kv[0], kv[1], self.table,
                                torch.full((w.batch,), start, dtype=torch.int32, device=device),
                                torch.from_numpy(width).to(device))
        self.new_k = torch.randn((w.batch, w.kv_heads, w.append_tokens, w.head_dim),
                                 generator=gen, device=device).to(fmt.dtype)
        self.new_v = torch.randn((w.batch, w.kv_heads, w.append_tokens, w.head_dim),
                                 generator=gen, device=device).to(fmt.dtype)
        self.queries = torch.from_numpy(inst.queries).to(device=device, dtype=fmt.dtype)
        self.out = torch.empty_like(self.queries)
        self.widths = (torch.from_numpy(w.step_widths().astype(np.int32)).to(device)
                       if w.widths else None)


def cpu_baseline(w, inst, layer, device, budget_s):
    """Time the oracle's C restatement of the reference algorithm on this host.

    Runs the whole step for as many sequences as fit the time budget (all of
    them for C2) on reference-format pages copied out of the GPU pool, with
    every host core.  Also returns the max/mean abs difference between the GPU
    output of the same step and the oracle's on the sampled sequences.
    """
    import numpy as np
    import torch

    from oracle import cport
    from pkv import ops

    fmt = layer.fmt
    cores = len(os.sched_getaffinity(0))
    used = sorted({int(p) for p in inst.table.ravel() if p >= 0})
    pages = ops.gather_pages(fmt, layer.pool, used)
    torch.cuda.synchronize()
    num = inst.num_pages
    host = []
    for t in pages:
        a = t.view(torch.int16).cpu().numpy().view(np.uint16) if t.element_size() == 2 else t.cpu().numpy()
        full = np.zeros((num,) + a.shape[1:], a.dtype)
        full[used] = a
        host.append(full)
    lengths = inst.total_lengths
    positions = inst.positions
    widths = inst.widths
    q = layer.queries.float().cpu().numpy()
    scale = 1.0 / math.sqrt(w.head_dim)

    new = np.random.default_rng(0).standard_normal(
        (w.batch * w.kv_heads * 2 * max(w.append_tokens, 1), w.head_dim)).astype(np.float32)

    def run(rows):
        sub = slice(0, rows)
        if w.bits != 16 and w.append_tokens:
            cport.quantize_rows(new[:rows * w.kv_heads * 2 * w.append_tokens], w.bits, w.group_size)
        if w.bits == 16:                      # float pages: (K, V) bits in the page dtype
            return cport.paged_attention(q[sub], inst.table[sub], lengths[sub], positions[sub],
                                         widths[sub], heads_kv=w.kv_heads,
                                         page_tokens=w.page_tokens, bits=0, float_pages=host,
                                         float_f16=fmt.dtype == torch.float16, scale=scale,
                                         threads=cores)
        return cport.paged_attention(q[sub], inst.table[sub], lengths[sub], positions[sub],
                                     widths[sub], heads_kv=w.kv_heads, page_tokens=w.page_tokens,
                                     bits=w.bits, group_size=w.group_size, pages=host,
                                     scale=scale, threads=cores)

    if is_prefill(w) and not w.widths:
        # a bounded sample: the first sequence's whole chunk
        rows = 1
        started = time.perf_counter()
        want = run(rows)
        first = time.perf_counter() - started
    else:
        started = time.perf_counter()
        want = run(w.batch)                   # warm-up and a full-step reference
        first = time.perf_counter() - started
        rows = w.batch
    reps = max(1, min(5, int(budget_s / max(first, 1e-3))))
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run(rows)
        times.append(time.perf_counter() - t0)
    step_s = float(np.median(times))
    if w.widths:
        return {"value": float(widths[:rows].sum()) / step_s, "unit": "tok/s", "cores": cores,
                "cpu_model": cpu_model(), "kind": "port",
                "sample": f"full {w.name} step ({rows} sequences of widths "
                          f"{sorted(set(int(x) for x in widths))}: quantize the new K/V rows + "
                          f"causal attention over {int(lengths.sum())} tokens), median of {reps}, "
                          f"OpenMP C restatement (oracle/pkv_oracle.c) on reference-format pages",
                "ms_per_step": step_s * 1e3}, want
    if is_prefill(w):
        return {"value": rows * w.num_queries / step_s, "unit": "tok/s", "cores": cores,
                "cpu_model": cpu_model(), "kind": "port",
                "sample": f"{w.name} step of {rows} of {w.batch} sequences (quantize its "
                          f"{w.append_tokens} new K/V rows + causal attention of its "
                          f"{w.num_queries}-token chunk over {int(lengths[0])} tokens), median "
                          f"of {reps}, OpenMP C restatement (oracle/pkv_oracle.c) on "
                          f"reference-format pages",
                "ms_per_step": step_s * 1e3}, want
    return {"value": rows / step_s, "unit": "seqs*tok/s", "cores": cores,
            "cpu_model": cpu_model(), "kind": "port",
            "sample": f"full {w.name} step ({rows} sequences, 1 layer: quantize the new K/V "
                      f"rows + attention over {int(lengths.sum())} cached tokens), median of "
                      f"{reps}, OpenMP C restatement (oracle/pkv_oracle.c) on "
                      f"reference-format pages",
            "ms_per_step": step_s * 1e3}, want


def cpu_model():
    """The host CPU's model name (``lscpu``'s "Model name", from /proc/cpuinfo)."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def copy_probe():
    """Three device-to-device copies of 256 MiB: 256 MiB read + 256 MiB written each."""
    import torch

    n = 256 << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_read": n, "copy_probe_bytes_written": n, "copies": 3}))
    return 0


def workload_waves(w, lengths):
    """Waves for a workload that fixes its partition size (C3: 512-token
    partitions): one wave per partition of every (sequence, KV head).  0 when
    the workload leaves it to the device's capacity."""
    if not w.split_tokens:
        return 0
    tiles = sum(max(1, -(-int(x) // 16)) for x in lengths) * w.kv_heads
    return max(1, -(-tiles * 16 // w.split_tokens))


def layer_bench(args):
    """End to end through ``PagedRunner.execute``: decode steps of one Llama-3-8B
    attention layer (q/k/v projections, RoPE, append + paged attention in
    libpkv, output projection) for C2's batch and context lengths, q8_0 KV
    (f16 activations, as the reference's CacheManager pairs q8_0 with f16).
    Contexts are prefilled through the runner in 1,024-token chunks before
    timing; each timed step is one runner call (host bookkeeping included).
    This is ``--workload layer --arena host``; the default is the device
    arena (``layer_device_bench``)."""
    import numpy as np
    import torch

    from pkv import _native, workloads
    from pkv.cache_manager import CacheConfig, CacheManager
    from pkv.layer import AttentionStack, ModelSpec
    from pkv.runner import ForwardRequest, PagedRunner

    _native.load()
    device = torch.device("cuda:0")
    w = workloads.get("c2")
    inst = workloads.generate(w, kv=False)
    spec = ModelSpec(hidden=4096, query_heads=w.heads, kv_heads=w.kv_heads, head_dim=w.head_dim,
                     num_layers=1, dtype="float16")
    model = AttentionStack(spec, device=device, seed=w.seed)
    cm = CacheManager(model, CacheConfig(block_size_tokens=w.page_tokens, key_type="q8_0",
                                         value_type="q8_0", group_size=w.group_size,
                                         memory_budget_bytes=64 << 30), device=device)
    handles = [cm.create_handle(f"seq{b}", key_type="q8_0", value_type="q8_0")
               for b in range(w.batch)]
    runner = PagedRunner(model)
    gen = torch.Generator(device=device)
    gen.manual_seed(w.seed)
    context = [int(x) for x in inst.context]

    def step(widths, phase, hidden=None):
        if hidden is None:
            hidden = [torch.randn((n, spec.hidden), generator=gen, device=device,
                                  dtype=torch.float16) for n in widths]
        reqs = [ForwardRequest(None, (), h.bundle.entries, phase=phase, runtime=cm,
                               handle=h, request_id=h.request_id, hidden=x)
                for h, n, x in zip(handles, widths, hidden) if n > 0]
        return runner.execute(reqs)

    chunk = 1024
    while True:
        left = [c - h.token_count for c, h in zip(context, handles)]
        if max(left) <= 0:
            break
        # rows with nothing left to prefill sit the chunk out
        step([min(chunk, max(n, 0)) for n in left], "prefill")
    # decode inputs are generated before timing: [step][row] -> [1, hidden]
    decode_in = torch.randn((args.warmup + args.steps, w.batch, 1, spec.hidden), generator=gen,
                            device=device, dtype=torch.float16).unbind(0)
    decode_in = [x.unbind(0) for x in decode_in]
    torch.cuda.synchronize()
    for i in range(args.warmup):
        step([1] * w.batch, "decode", decode_in[i])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step([1] * w.batch, "decode", decode_in[args.warmup + i])
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / args.steps * 1e3
    trace = runner.last_trace
    result = {
        "metric": "e2e attention-layer decode tok/s (PagedRunner, Llama-3-8B layer, q8_0 KV)",
        "value": round(w.batch / (ms / 1e3), 1), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "layer", "batch": w.batch, "hidden": spec.hidden,
                   "heads": spec.query_heads, "kv_heads": spec.kv_heads,
                   "head_dim": spec.head_dim, "kv": "q8_0", "group_size": w.group_size,
                   "page_tokens": w.page_tokens,
                   "mean_context": float(np.mean([h.token_count for h in handles]))},
        "host_dispatch_ms_last_step": round(trace.get("synchronized_kernel_dispatch_ms", 0.0), 4),
    }
    print(json.dumps(result))
    return 0


def layer_device_bench(args):
    """The same layer decode steps through the same reference-named calls
    (``CacheManager.create_handle`` + ``PagedRunner.execute``) with the page
    bookkeeping on the device: ``CacheConfig(page_arena="device")`` gives each
    handle a ``DevicePageArena`` slot, so a step is one reservation kernel
    instead of per-sequence host page tables.  Unless ``--eager``, the runner
    replays repeated decode steps of the same sequences as captured HIP graphs
    (reservation, then QKV GEMM, RoPE, append, attention, merge, output GEMM),
    reading the reservation's error bits between the two.  ``--arena host``
    runs the same steps with host page tables (``layer_bench``)."""
    import numpy as np
    import torch

    from pkv import _native, workloads
    from pkv.cache_manager import CacheConfig, CacheManager
    from pkv.layer import AttentionStack, ModelSpec
    from pkv.ops import PageFormat
    from pkv.runner import ForwardRequest, PagedRunner

    _native.load()
    device = torch.device("cuda:0")
    w = workloads.get("c2")
    inst = workloads.generate(w, kv=False)
    spec = ModelSpec(hidden=4096, query_heads=w.heads, kv_heads=w.kv_heads, head_dim=w.head_dim,
                     num_layers=1, dtype="float16")
    model = AttentionStack(spec, device=device, seed=w.seed)
    fmt = PageFormat(w.kv_heads, w.head_dim, w.page_tokens, 8, w.group_size, torch.float16)
    context = [int(x) for x in inst.context]
    extra = args.warmup + args.steps + 2
    pages = sum(-(-(c + extra) // w.page_tokens) for c in context) + w.batch
    cm = CacheManager(model, CacheConfig(block_size_tokens=w.page_tokens, key_type="q8_0",
                                         value_type="q8_0", group_size=w.group_size,
                                         memory_budget_bytes=64 << 30, device_pages=pages,
                                         page_arena="device", max_sequences=w.batch,
                                         max_sequence_tokens=max(context) + extra),
                      device=device)
    handles = [cm.create_handle(f"seq{b}", key_type="q8_0", value_type="q8_0")
               for b in range(w.batch)]
    runner = PagedRunner(model, graphs=not args.eager)
    gen = torch.Generator(device=device)
    gen.manual_seed(w.seed)

    def requests(rows, hidden, phase):
        return [ForwardRequest(None, (), handles[b].bundle.entries, phase=phase,
                               runtime=cm, handle=handles[b], request_id=handles[b].request_id,
                               hidden=x) for b, x in zip(rows, hidden)]

    chunk = 1024
    while True:
        left = [c - h.token_count for c, h in zip(context, handles)]
        rows = [b for b in range(w.batch) if left[b] > 0]
        if not rows:
            break
        hidden = [torch.randn((min(chunk, left[b]), spec.hidden), generator=gen, device=device,
                              dtype=torch.float16) for b in rows]
        runner.execute(requests(rows, hidden, "prefill"))
    decode_in = torch.randn((args.warmup + args.steps, w.batch, 1, spec.hidden), generator=gen,
                            device=device, dtype=torch.float16)
    decode_in = [x.unbind(0) for x in decode_in.unbind(0)]
    every = list(range(w.batch))
    for i in range(args.warmup):
        runner.execute(requests(every, decode_in[i], "decode"))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        runner.execute(requests(every, decode_in[args.warmup + i], "decode"))
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / args.steps * 1e3
    arena = handles[0].bundle.entries[0].arena
    mirror = list(arena.lengths)
    arena.sync_lengths()
    assert arena.lengths == mirror, "host length mirror differs from the device"
    arena.check()
    result = {
        "metric": "e2e attention-layer decode tok/s (CacheManager + PagedRunner on the device "
                  "page arena, Llama-3-8B layer, q8_0 KV)",
        "value": round(w.batch / (ms / 1e3), 1), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "layer", "arena": "device", "graph": not args.eager,
                   "batch": w.batch, "hidden": spec.hidden, "heads": spec.query_heads,
                   "kv_heads": spec.kv_heads, "head_dim": spec.head_dim, "kv": "q8_0",
                   "group_size": w.group_size, "page_tokens": w.page_tokens,
                   "mean_context": float(np.mean([h.token_count for h in handles]))},
        "trace": {k: runner.last_trace.get(k) for k in ("page_arena", "graph_replay",
                                                        "batch_size")},
    }
    print(json.dumps(result))
    return 0


def read_probe(lib, fmt, layers, table, lengths, waves, steps, device):
    """Time ``pkv_read_probe`` over the pages the step's sequences hold (every
    KV head, block-table order) at the decode launch's wave count, rotating
    over the layer pools like the timed steps: one captured graph of ``steps``
    launches between two HIP events.  Returns ``(ms per launch, bytes per
    launch, pages)``."""
    import numpy as np
    import torch

    from pkv import _native

    pages = [table[b, :-(-int(n) // fmt.page_tokens)] for b, n in enumerate(lengths)]
    ids = torch.from_numpy(np.concatenate(pages).astype(np.int32)).to(device)
    out = torch.empty(waves * 64, dtype=torch.int32, device=device)
    layout = fmt.c_layout

    def launch(i):
        pool = layers[i % len(layers)].pool
        code = lib.pkv_read_probe(_native.stream_handle(device), layout, pool.data_ptr(),
                                  pool.shape[0], ids.data_ptr(), ids.numel(), waves,
                                  out.data_ptr())
        if code:
            _native.check(code, "read probe")

    for i in range(len(layers)):
        launch(i)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(steps):
            launch(i)
    graph.replay()
    torch.cuda.synchronize()
    ms = held_replay(graph, device) / steps
    return ms, int(ids.numel()) * fmt.page_bytes, int(ids.numel())


def main(argv=None):
    parser = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--workload", default="c2")
    parser.add_argument("--layers", type=int, default=4)
    parser.add_argument("--waves", type=int, default=0,
                        help="attention work waves (0: the workload's partition size, else the "
                             "library default for the shape and batch)")
    parser.add_argument("--no-fuse", action="store_true",
                        help="single-token steps: launch the append and the attention "
                             "separately instead of the fused pkv_append_paged_attention")
    parser.add_argument("--decode-kernel", choices=("mfma", "valu"), default="mfma",
                        help="kernel for decode rows (<= 4 query rows per KV head, quantized "
                             "pages): the MFMA form (default) or the vector-ALU form")
    parser.add_argument("--graph", action="store_true",
                        help="kept for older command lines: graph replay is the default "
                             "(--eager turns it off)")
    parser.add_argument("--eager", action="store_true",
                        help="launch each timed step from the host instead of replaying "
                             "captured HIP graphs (attention workloads: the timed steps as one "
                             "graph; layer workload on the device arena: each decode step)")
    parser.add_argument("--cpu-budget", type=float, default=15.0,
                        help="seconds of CPU baseline timing (0 disables)")
    parser.add_argument("--arena", choices=("host", "device"), default="device",
                        help="layer workload: page bookkeeping on the device (CacheManager with "
                             "page_arena=\"device\", the default) or on the host (host page "
                             "tables per sequence)")
    parser.add_argument("--copy-probe", action="store_true",
                        help="only run three 256 MiB device copies (calibrates rocprofv3 "
                             "FETCH_SIZE / WRITE_SIZE against a kernel of known traffic)")
    args = parser.parse_args(argv)
    if args.copy_probe:
        return copy_probe()
    if args.workload == "layer":
        if args.gpus != 1:
            print(json.dumps({"error": "this build measures one GPU only; run with --gpus 1"}))
            return 2
        return layer_device_bench(args) if args.arena == "device" else layer_bench(args)
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only: the paged decode path "
                          "shards by sequence with no exchange; run with --gpus 1"}))
        return 2

    import numpy as np
    import torch

    from pkv import _native, ops, workloads

    _native.load()
    ops.select_decode_kernel(args.decode_kernel)
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    w = workloads.get(args.workload)
    total_steps = args.warmup + args.steps
    growth = 0 if w.fixed_chunk else math.ceil(total_steps / args.layers) * w.append_tokens
    inst = workloads.generate(w, extra_tokens=growth, kv=False)
    fmt = ops.PageFormat(w.kv_heads, w.head_dim, w.page_tokens, w.bits, w.group_size,
                         torch.bfloat16)
    layers = [Layer(w, inst, i, fmt, device) for i in range(args.layers)]
    torch.cuda.synchronize()

    context = inst.context.astype(np.int64)
    scale = 1.0 / math.sqrt(w.head_dim)
    appends = w.step_appends()
    waves = args.waves or workload_waves(w, context + appends) or ops.default_waves(
        fmt, w.heads, ops.decode_queries(fmt, w.heads, w.num_queries) or w.num_queries, w.batch)
    # per-step device arrays (no host->device copies inside the timed loop)
    plans = []
    for s in range(total_steps):
        li = s % args.layers
        start = context + (0 if w.fixed_chunk else (s // args.layers) * appends)
        lens = start + appends
        plans.append((li, torch.from_numpy(start.astype(np.int32)).to(device),
                      torch.from_numpy(lens.astype(np.int32)).to(device),
                      [int(x) for x in lens]))
    workspace = torch.empty(ops.workspace_bytes(fmt, w.heads, w.num_queries, waves),
                            dtype=torch.uint8, device=device)

    lib = _native.load()
    layout = fmt.c_layout

    # single-token steps append and attend in one call (pkv_append_paged_attention)
    fused = (not args.no_fuse and w.append_tokens == 1 and w.num_queries == 1 and not w.widths
             and args.decode_kernel == "mfma")

    def step(s, ev=None, append=True, attend=True):
        li, start, lens, _ = plans[s]
        layer = layers[li]
        h = _native.stream_handle(device)
        if fused and append and attend:
            if ev is not None:
                ev[0].record(torch.cuda.current_stream(device))
            code = lib.pkv_append_paged_attention(
                h, layout, layer.pool.data_ptr(), layer.pool.shape[0], layer.new_k.data_ptr(),
                layer.new_v.data_ptr(), layer.queries.data_ptr(), w.batch, w.heads,
                layer.table.data_ptr(), layer.table.shape[1], lens.data_ptr(), scale, waves,
                workspace.data_ptr(), workspace.numel(), layer.out.data_ptr())
            if ev is not None:
                ev[1].record(torch.cuda.current_stream(device))
            if code:
                _native.check(code, "append + attention")
            return
        if w.append_tokens and append:
            code = lib.pkv_append_quantize(h, layout, layer.pool.data_ptr(), layer.pool.shape[0],
                                           layer.new_k.data_ptr(), layer.new_v.data_ptr(), w.batch,
                                           w.append_tokens, layer.table.data_ptr(),
                                           layer.table.shape[1], start.data_ptr(),
                                           _native.ptr(layer.widths), None)
            if code:
                _native.check(code, "append")
        if not attend:
            return
        if ev is not None:
            ev[0].record(torch.cuda.current_stream(device))
        code = lib.pkv_paged_attention(h, layout, layer.pool.data_ptr(), layer.pool.shape[0],
                                       layer.queries.data_ptr(), w.batch, w.heads, w.num_queries,
                                       layer.table.data_ptr(), layer.table.shape[1],
                                       lens.data_ptr(), None, _native.ptr(layer.widths), scale,
                                       waves,
                                       workspace.data_ptr(), workspace.numel(),
                                       layer.out.data_ptr())
        if ev is not None:
            ev[1].record(torch.cuda.current_stream(device))
        if code:
            _native.check(code, "attention")

    # first step checked against the oracle below (before warm-up mutates the pools)
    check_step = None
    if args.cpu_budget > 0:
        step(0)
        torch.cuda.synchronize()
        check_step = layers[0].out.float().cpu().numpy()
        # undo nothing: the appended token is re-written identically by later steps
    for s in range(args.warmup):
        step(s)
    torch.cuda.synchronize()

    # The timed steps are captured as one HIP graph and replayed (no host
    # launch gaps): that replay gives the step time.  The attention launches
    # of the same steps are captured as a second graph (no appends), replayed
    # between two HIP events on the stream: that span over the launches gives
    # the average launch duration for the roofline (kernel, merge and the gaps
    # between them, as a graph-replayed decode loop runs them).  Events
    # recorded around each launch of a host-launched pass are reported beside
    # it; each such event adds its own few microseconds.  Re-running a step
    # re-appends the same token at the same position (idempotent).
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(args.steps)]
    graph = attn_graph = append_graph = None
    if not args.eager:
        try:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for i in range(args.steps):
                    step(args.warmup + i)
            graph.replay()          # untimed: the first replay uploads the graph
            attn_graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(attn_graph):
                for i in range(args.steps):
                    step(args.warmup + i, append=fused)   # fused: the step's one launch
            attn_graph.replay()
            if w.append_tokens and not fused:
                append_graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(append_graph):
                    for i in range(args.steps):
                        step(args.warmup + i, attend=False)
                append_graph.replay()
            torch.cuda.synchronize()
        except RuntimeError as exc:
            print(f"bench: graph capture unavailable ({exc}); timing host launches",
                  file=sys.stderr)
            graph = attn_graph = append_graph = None
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    if graph is not None:
        graph.replay()
    else:
        for i in range(args.steps):
            step(args.warmup + i, events[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    span_ms = append_ms = None
    if graph is not None:
        span_ms = held_replay(attn_graph, device) / args.steps
        if append_graph is not None:
            append_ms = held_replay(append_graph, device) / args.steps
            step_graph_ms = held_replay(graph, device) / args.steps
        # Hold the stream with a bounded spin kernel while the host enqueues
        # the per-launch pass, so that its events bracket GPU work only.
        torch.cuda._sleep(int(args.steps * SLEEP_CYCLES_PER_STEP))
        for i in range(args.steps):
            step(args.warmup + i, events[i])
        torch.cuda.synchronize()
    per_launch_ms = float(np.mean([a.elapsed_time(b) for a, b in events]))
    attn_ms = span_ms if span_ms is not None else per_launch_ms
    ms_per_step = wall / args.steps * 1e3
    timing = ("HIP events around a graph replay of the timed steps' attention launches "
              "(stream held while the host submits it), divided by the launch count"
              if span_ms is not None else
              "HIP events per launch in the timed host-launched steps")
    timed = plans[args.warmup:]
    mean_lens = np.mean([p[3] for p in timed], axis=0)
    attn_bytes, step_bytes = algorithmic_bytes(w, mean_lens)
    prefill = is_prefill(w)
    value = float(w.step_widths().sum() if prefill else w.batch) / (ms_per_step / 1e3)
    roofline = None
    if attn_ms and w.widths:
        # decode rows on the HBM roofline, prefill rows on the MFMA one
        dec_bytes, flops, ideal_ms = mixed_roofline(w, mean_lens)
        roofline = {"bound": "hbm+mfma", "achieved": round(ideal_ms / attn_ms, 4), "peak": 1.0,
                    "unit": "ideal time / launch time", "frac": round(ideal_ms / attn_ms, 4),
                    "traffic": measured_traffic(w.name),
                    "kernel": "pkv_paged_attention (prefill_kernel + attn_kernel + merge_kernel)",
                    "kernel_timing": timing, "kernel_ms": round(attn_ms, 5),
                    "ideal_ms": round(ideal_ms, 5), "decode_bytes": int(dec_bytes),
                    "prefill_flops": int(flops)}
    elif attn_ms and prefill:
        flops = attention_flops(w, mean_lens)
        achieved = flops / (attn_ms / 1e3) / 1e12
        roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": MFMA_PEAK_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(achieved / MFMA_PEAK_TFLOPS, 4),
                    "traffic": measured_traffic(w.name),
                    "kernel": "pkv_paged_attention (prefill_kernel)",
                    "kernel_timing": timing,
                    "kernel_ms": round(attn_ms, 5), "flops_per_launch": int(flops),
                    "bytes_per_launch": int(attn_bytes),
                    "hbm_gbs": round(attn_bytes / (attn_ms / 1e3) / 1e9, 1)}
    elif attn_ms:
        if fused:   # the launch also reads the new K/V rows
            attn_bytes = step_bytes
        rows = w.num_queries * w.heads // w.kv_heads
        valu = args.decode_kernel == "valu" and w.bits != 16 and rows <= 4 and not fused
        achieved = attn_bytes / (attn_ms / 1e3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                    "traffic": measured_traffic(w.name),
                    "kernel": ("pkv_append_paged_attention (attn_kernel with the fused "
                               "append + merge_kernel)" if fused else
                               "pkv_paged_attention ({} + merge_kernel)".format(
                                   "valu_kernel" if valu else "attn_kernel")),
                    "kernel_timing": timing,
                    "kernel_ms": round(attn_ms, 5), "bytes_per_launch": int(attn_bytes)}
    if roofline is not None and roofline["bound"] == "hbm" and graph is not None:
        # the same pages read by a kernel that does nothing else
        probe_ms, probe_bytes, probe_pages = read_probe(
            lib, fmt, layers, inst.table, plans[args.warmup][3], waves, args.steps, device)
        probe_gbs = probe_bytes / (probe_ms / 1e3) / 1e9
        roofline["read_probe"] = {
            "kernel_ms": round(probe_ms, 5), "achieved": round(probe_gbs, 1), "unit": "GB/s",
            "frac": round(probe_gbs / HBM_PEAK_GBS, 4), "bytes_per_launch": probe_bytes,
            "pages": probe_pages, "waves": waves,
            "what": "pkv_read_probe: every byte of the pages the step's sequences hold "
                    "(all KV heads), block-table order, equal runs over the attention's "
                    "wave count, loads only; graph replay between HIP events"}
        roofline["frac_of_read_probe"] = round(roofline["achieved"] / probe_gbs, 4)
    if roofline is not None:
        roofline["kernel_ms_events_per_launch"] = round(per_launch_ms, 5)
        if append_ms is not None:
            # the launch inside the step (after its append): step graph time
            # minus an append-only graph's
            roofline["kernel_ms_in_step"] = round(step_graph_ms - append_ms, 5)
    kv = {8: "int8", 4: "4-bit", 16: "bf16"}[w.bits]
    shape = ("Llama-3-8B shape, " if (w.heads, w.kv_heads, w.head_dim) == (32, 8, 128) else "")
    if w.widths:
        metric = f"mixed decode + prefill attention query tok/s ({kv} paged KV, 1 layer)"
        unit = "tok/s"
    elif prefill:
        metric = f"chunked-prefill attention query tok/s ({kv} paged KV, 1 layer)"
        unit = "tok/s"
    else:
        kind = "decode-attn" if w.num_queries == 1 else f"verify-attn ({w.num_queries} drafts)"
        metric = f"{kind} seqs*tok/s ({kv} paged KV, {shape}1 layer)"
        unit = "seqs*tok/s"
    result = {
        "metric": metric,
        "value": round(value, 1), "unit": unit, "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": {8: "int8", 4: "u4", 16: "bf16"}[w.bits],
        "data": "synthetic",
        "config": {"workload": w.name, "batch": w.batch, "heads": w.heads,
                   "kv_heads": w.kv_heads, "head_dim": w.head_dim, "page_tokens": w.page_tokens,
                   "bits": w.bits, "group_size": w.group_size, "num_queries": w.num_queries,
                   "mean_context": float(mean_lens.mean()),
                   "waves": waves, "layers_rotated": args.layers, "graph": graph is not None,
                   "decode_kernel": args.decode_kernel, "fused_append": fused},
        "step_hbm_gbs": round(step_bytes / (ms_per_step / 1e3) / 1e9, 1),
        "roofline": roofline,
    }
    if args.cpu_budget > 0:
        base, want = cpu_baseline(w, inst, layers[0], device, args.cpu_budget)
        got = check_step[:want.shape[0]]
        # The oracle reads the pool after all steps; later steps only wrote
        # positions past step 0's lengths (or, for a fixed chunk, the same
        # chunk again), which leaves what the oracle reads unchanged.
        err = np.abs(got - workloads.bf16_round(want.reshape(got.shape)))
        base["check_vs_gpu"] = {"max_abs": float(err.max()), "mean_abs": float(err.mean())}
        result["cpu_baseline"] = base
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
