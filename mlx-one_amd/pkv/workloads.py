"""Benchmark and parity workloads C1-C5 (synthetic, seeded).

Each config is a one-layer paged-attention step on synthetic N(0, 1) data.
Draw order from ``numpy.random.default_rng(seed)``: sequence lengths, block
table permutation, queries, keys, values, then outlier channels.  Float data
is rounded to the page dtype (bf16) on the host; the same arrays feed the GPU
path and the CPU oracle.
"""

from __future__ import annotations

from dataclasses import dataclass, field, replace

import numpy as np


@dataclass(frozen=True)
class Workload:
    name: str
    batch: int
    heads: int
    kv_heads: int
    head_dim: int
    page_tokens: int
    bits: int                      # 4, 8, or 16 (float pages)
    group_size: int = 64
    num_queries: int = 1           # 1 decode, 1 + drafts for verify
    append_tokens: int = 0         # new tokens appended by the step
    lengths: tuple = ()            # cached tokens before the step (fixed lengths)
    length_range: tuple = ()       # (lo, hi) inclusive, drawn per sequence
    split_tokens: int = 0          # 0 = planner default
    shared_prefix_pages: int = 0
    outlier_fraction: float = 0.0
    outlier_scale: float = 8.0
    arena_pages: int = 0           # 0 = exactly the pages needed (+ spare)
    fixed_chunk: bool = False      # every step re-appends the same chunk (fixed shape)
    seed: int = 0
    description: str = ""
    widths: tuple = ()             # per-sequence query rows (mixed batches); () = num_queries
    tail_lengths: tuple = ()       # fixed lengths of the last sequences after the drawn ones

    def step_widths(self):
        """Query rows of each sequence in one step (its last tokens)."""
        if self.widths:
            return np.asarray(self.widths, np.int64)
        return np.full(self.batch, self.num_queries, np.int64)

    def step_appends(self):
        """Tokens each sequence appends in one step (a mixed batch appends its
        query rows)."""
        if self.widths:
            return np.asarray(self.widths, np.int64)
        return np.full(self.batch, self.append_tokens, np.int64)


CONFIGS = {
    "c1": Workload("c1", batch=4, heads=8, kv_heads=2, head_dim=64, page_tokens=16, bits=16,
                   lengths=(128, 256, 384, 512), arena_pages=128, seed=0,
                   description="bf16 paged decode, B4 H8/HK2 D64 P16, L in {128,256,384,512}"),
    "c2": Workload("c2", batch=32, heads=32, kv_heads=8, head_dim=128, page_tokens=16, bits=8,
                   group_size=64, append_tokens=1, length_range=(1024, 8192),
                   outlier_fraction=0.01, seed=1,
                   description="int8 G64 paged decode + append, Llama-3-8B shape, B32, "
                               "L~U[1024,8192]"),
    "c3": Workload("c3", batch=8, heads=32, kv_heads=4, head_dim=128, page_tokens=32, bits=4,
                   group_size=64, lengths=(32768,) * 8, split_tokens=512, seed=2,
                   description="4-bit G64 long-context decode, B8 H32/HK4 P32 L=32768, "
                               "split 512"),
    "c4": Workload("c4", batch=16, heads=32, kv_heads=8, head_dim=128, page_tokens=16, bits=8,
                   group_size=64, num_queries=5, append_tokens=5, length_range=(512, 4096),
                   shared_prefix_pages=16, seed=3,
                   description="int8 speculative verify, B16 Q5 causal drafts, 256-token "
                               "shared prefix"),
    "c5": Workload("c5", batch=4, heads=32, kv_heads=8, head_dim=128, page_tokens=16, bits=8,
                   group_size=64, num_queries=512, append_tokens=512, lengths=(4096,) * 4,
                   fixed_chunk=True, seed=4,
                   description="int8 G64 chunked prefill: 512-token causal query chunk per "
                               "sequence over a 4096-token paged prefix plus the chunk, B4 "
                               "H32/HK8 D128 P16"),
    # C2's decode rows and C5's prefill chunks in one padded batch (the
    # reference pads mixed widths into one forward, engine/paged.py:345-346)
    "mixed": Workload("mixed", batch=36, heads=32, kv_heads=8, head_dim=128, page_tokens=16,
                      bits=8, group_size=64, num_queries=512, append_tokens=512,
                      length_range=(1024, 8192), tail_lengths=(4096,) * 4,
                      widths=(1,) * 32 + (512,) * 4, outlier_fraction=0.01, fixed_chunk=True,
                      seed=5,
                      description="mixed batch, int8 G64: 32 decode rows (L~U[1024,8192]) and "
                                  "4 prefill chunks of 512 over 4096 cached tokens, one call"),
}


def get(name, **overrides):
    return replace(CONFIGS[name], **overrides)


def bf16_round(x):
    """float32 -> bfloat16 values (round to nearest even), kept as float32.

    32-bit integer arithmetic: the largest finite pattern plus the rounding
    increment stays below 2**32; NaNs stay NaN."""
    x = np.ascontiguousarray(x, np.float32)
    bits = x.view(np.uint32)
    out = bits + np.uint32(0x7FFF)
    out += (bits >> np.uint32(16)) & np.uint32(1)
    out &= np.uint32(0xFFFF0000)
    out = out.view(np.float32)
    nan = np.isnan(x)
    if nan.any():
        out[nan] = np.float32("nan")
    return out


@dataclass
class Instance:
    """Host arrays of one generated workload."""

    workload: Workload
    context: np.ndarray            # [B] cached tokens before the step
    table: np.ndarray              # [B, max_pages] int32 page ids
    queries: np.ndarray            # [B, H, Q, D] float32 (bf16 values)
    keys: list = field(default_factory=list)    # per sequence [HK, L_b + append, D]
    values: list = field(default_factory=list)
    num_pages: int = 0

    @property
    def widths(self):
        return self.workload.step_widths().astype(np.int32)

    @property
    def total_lengths(self):
        return self.context + self.workload.step_appends()

    @property
    def positions(self):
        """Logical positions of the query rows: a sequence's ``width`` rows are
        its last tokens, padding rows continue after them."""
        w = self.workload
        return np.stack([np.arange(n - q, n - q + w.num_queries)
                         for n, q in zip(self.total_lengths, w.step_widths())]).astype(np.int32)


def generate(w: Workload, *, extra_tokens=0, layer=0, kv=True):
    """Draw one instance; ``extra_tokens`` reserves pages for later decode steps.

    ``kv=False`` stops after the queries (lengths, table and queries only), for
    callers that draw K/V on the device.
    """
    rng = np.random.default_rng(w.seed if layer == 0 else [w.seed, layer])
    if w.lengths:
        context = np.asarray(w.lengths, np.int64)
    else:
        lo, hi = w.length_range
        drawn = rng.integers(lo, hi, size=w.batch - len(w.tail_lengths), endpoint=True)
        context = np.concatenate([drawn, np.asarray(w.tail_lengths, np.int64)]).astype(np.int64)
    total = context + w.step_appends()
    capacity = total + extra_tokens
    pages_per = (capacity + w.page_tokens - 1) // w.page_tokens
    # a shared prefix cannot be longer than the shortest sequence's full pages
    shared = min(w.shared_prefix_pages, int(total.min()) // w.page_tokens)
    distinct = int(pages_per.sum()) - shared * (w.batch - 1) if shared else int(pages_per.sum())
    arena = max(w.arena_pages, distinct)
    perm = rng.permutation(arena).astype(np.int32)
    max_pages = int(pages_per.max())
    table = np.full((w.batch, max_pages), -1, np.int32)
    cursor = 0
    prefix = perm[:shared]
    if shared:
        cursor = shared
    for b in range(w.batch):
        n = int(pages_per[b])
        own = n - shared if shared else n
        ids = np.concatenate([prefix, perm[cursor:cursor + own]]) if shared else perm[cursor:cursor + n]
        cursor += own
        table[b, :n] = ids
    queries = bf16_round(rng.standard_normal((w.batch, w.heads, w.num_queries, w.head_dim),
                                             dtype=np.float32))
    if not kv:
        return Instance(w, context.astype(np.int32), table, queries, [], [], arena)
    keys = [rng.standard_normal((w.kv_heads, int(n), w.head_dim), dtype=np.float32) for n in total]
    values = [rng.standard_normal((w.kv_heads, int(n), w.head_dim), dtype=np.float32)
              for n in total]
    if shared:
        # identical leading pages carry identical tokens
        span = shared * w.page_tokens
        for b in range(1, w.batch):
            keys[b][:, :span] = keys[0][:, :span]
            values[b][:, :span] = values[0][:, :span]
    if w.outlier_fraction:
        channels = w.kv_heads * w.head_dim
        count = max(1, int(round(w.outlier_fraction * channels)))
        for arrays in (keys, values):
            pick = rng.choice(channels, count, replace=False)
            hk, d = np.divmod(pick, w.head_dim)
            for a in arrays:
                a[hk, :, d] *= w.outlier_scale
    keys = [bf16_round(k) for k in keys]
    values = [bf16_round(v) for v in values]
    return Instance(w, context.astype(np.int32), table, queries, keys, values, arena)
