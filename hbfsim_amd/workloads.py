"""Deterministic synthetic access streams for the benchmark configurations.

Every random draw is a counter-based SplitMix64 output, so a stream is a pure
function of (seed, stream id, index) and the same on every machine and on the
GPU.  Exponential inter-arrival gaps use a fixed inverse-CDF table in
picoseconds with integer interpolation; the table is built once on the host
from `math.log` and its checksum is pinned in the tests.

Record layout: uint64 [n, 4] = addr, bytes, issue_ps, flags (0 read, 1 write).
"""
from __future__ import annotations

import dataclasses
import math
import pathlib

import numpy as np

PROFILES = pathlib.Path(__file__).resolve().parent / "profiles"
GOLDEN = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)
EXP_TABLE_BITS = 12
EXP_TABLE_CAP = 20.0  # the last bucket ends at 20 x mean instead of infinity


def splitmix(v: np.ndarray) -> np.ndarray:
    """SplitMix64 finaliser with its increment (uint64 arrays, wrapping)."""
    with np.errstate(over="ignore"):
        z = (v + GOLDEN).astype(np.uint64)
        z = (z ^ (z >> np.uint64(30))) * M1
        z = (z ^ (z >> np.uint64(27))) * M2
        return z ^ (z >> np.uint64(31))


def stream_key(seed: int, stream: int) -> np.uint64:
    x = np.array([(seed * 0x100000001B3 + stream * 0xD1B54A32D192ED03) & (2**64 - 1)],
                 dtype=np.uint64)
    return splitmix(x)[0]


def draws(seed: int, stream: int, start: int, count: int) -> np.ndarray:
    """Outputs start..start+count-1 of the SplitMix64 sequence keyed by (seed, stream)."""
    idx = np.arange(start, start + count, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return splitmix(stream_key(seed, stream) + idx * GOLDEN)


def exp_table(mean_ps: int) -> np.ndarray:
    """T[k] = round(mean * -ln(1 - k / 2^bits)), k = 0..2^bits, last capped."""
    size = 1 << EXP_TABLE_BITS
    t = np.zeros(size + 1, dtype=np.uint64)
    for k in range(size):
        t[k] = int(round(mean_ps * -math.log1p(-k / size)))
    t[size] = int(round(mean_ps * EXP_TABLE_CAP))
    return t


def exp_gaps(u: np.ndarray, table: np.ndarray) -> np.ndarray:
    """Integer inverse-CDF sample: top bits pick the bucket, the next 20 bits
    interpolate linearly inside it."""
    hi = (u >> np.uint64(64 - EXP_TABLE_BITS)).astype(np.int64)
    lo = ((u >> np.uint64(64 - EXP_TABLE_BITS - 20)) & np.uint64(0xFFFFF))
    a = table[hi]
    b = table[hi + 1]
    return a + (((b - a) * lo) >> np.uint64(20))


@dataclasses.dataclass
class Stream:
    """A workload: ranges to register and the records to time."""
    profile: pathlib.Path
    ranges: list[tuple[int, int, int]]  # (base, length, permissions)
    records: np.ndarray                  # uint64 [n, 4]
    name: str = ""


RANGE_BASE = 0x7F00_0000_0000  # where synthetic ranges start (any address works)


def config0(n: int = 1 << 20, seed: int = 0, mean_gap_ps: int = 2000,
            range_bytes: int = 1 << 30, line: int = 128,
            write_fraction_per_mille: int = 0) -> Stream:
    """Config 0: uniform random 128-B lines in one 1 GiB range, Poisson issue
    with mean gap 2 ns, all reads (writes optional for wider tests)."""
    lines = range_bytes // line
    u_addr = draws(seed, 1, 0, n)
    idx = (u_addr % np.uint64(lines)).astype(np.uint64)
    gaps = exp_gaps(draws(seed, 2, 0, n), exp_table(mean_gap_ps))
    issue = np.cumsum(gaps, dtype=np.uint64)
    rec = np.zeros((n, 4), dtype=np.uint64)
    rec[:, 0] = np.uint64(RANGE_BASE) + idx * np.uint64(line)
    rec[:, 1] = line
    rec[:, 2] = issue
    if write_fraction_per_mille:
        w = (draws(seed, 3, 0, n) % np.uint64(1000)) < np.uint64(write_fraction_per_mille)
        rec[:, 3] = w.astype(np.uint64)
    return Stream(PROFILES / "c0.json", [(RANGE_BASE, range_bytes, 3)], rec, "config0")


# ---------------------------------------------------------------------------
# Config 2: Qwen3-30B-A3B-shaped MoE decode


@dataclasses.dataclass(frozen=True)
class MoeShape:
    layers: int = 48
    experts: int = 128
    top_k: int = 8
    hidden: int = 2048
    intermediate: int = 768
    tokens: int = 32
    zipf_s: float = 1.1
    seed: int = 1
    line: int = 128
    issuers: int = 256        # concurrent wavefronts issuing lines
    gap_ps: int = 64_000      # each issues one line every 64 ns
    base: int = 0x5000_0000_0000

    @property
    def expert_bytes(self) -> int:
        return 3 * self.hidden * self.intermediate * 2  # gate, up, down in bf16

    @property
    def lines_per_expert(self) -> int:
        return self.expert_bytes // self.line

    def expert_base(self, layer: int, expert: int) -> int:
        return self.base + (layer * self.experts + expert) * self.expert_bytes


QWEN3_30B_A3B = MoeShape()

# Config 4: OLMoE-shaped trace (16 layers x 64 experts, top-8 of 32 tokens,
# intermediate 1024) under the thermal-coupled model.
OLMOE = MoeShape(layers=16, experts=64, intermediate=1024, seed=3, base=0x6000_0000_0000)
C4_ACCESSES = 100_000_000

# The 64 x 64 x 8 EQ3 grid of config 4: one layer per die of an 11 mm x
# 11 mm stack of 8 dies thinned to 50 um (cell 172 um x 172 um x 50 um of
# silicon, 1.66e6 J/(m^3 K), 150 W/(m K) laterally; 4.3e-3 W/K per cell
# through a 10-um bond layer between dies; 2 W/K from the top die to a
# 45 C ambient), stepped every 1 us.
C4_GRID = dict(nx=64, ny=64, nz=8, sweeps=4, capacity_j_per_k=2.46e-6, gx_w_per_k=7.5e-3,
               gy_w_per_k=7.5e-3, gz_w_per_k=4.3e-3, top_g_w_per_k=4.9e-4, ambient_k=318.15,
               dt_s=1e-6)
# Reliability inputs (the reference leaves them null: reliability.json): Ea
# 1.04 eV at 85 C (test_system_models.py:12), a retention period of 50 us at
# 85 C (time-compressed so refresh shows within a 25-ms trace), 20 nJ per
# 128-B access, 10 uJ per refresh, 0.1 W static per die; throttle at 55 /
# 60 / 70 C with 1 K hysteresis, 2-us action delay, 10-us dwell, and one
# admission per ns while light.  Channel c occupies block (c % 4, c / 4) of
# the x-y plane.
C4_RELIABILITY = dict(policy=1, regions_x=4, regions_y=2, window_ps=1_000_000,
                      static_power_w=2e-4, access_energy_j=20e-9, refresh_energy_j=10e-6,
                      activation_energy_ev=1.04, reference_k=358.15, retention_ps=50_000_000,
                      light_k=328.15, severe_k=333.15, shutdown_k=343.15, hysteresis_k=1.0,
                      action_delay_ps=2_000_000, min_dwell_ps=10_000_000, light_gap_ps=1000)


def staggered_ages(dies: int, retention_ps: int) -> np.ndarray:
    """Initial equivalent ages: die d last refreshed d/dies of a period ago."""
    return np.array([d * retention_ps // dies for d in range(dies)], np.uint64)


def c4_segments(shape: MoeShape = OLMOE, steps: int = 2) -> np.ndarray:
    """Expert bases of `steps` decode steps streamed back to back."""
    sel = moe_selection(shape, steps)
    return np.concatenate([moe_segments(shape, s) for s in sel])


def zipf_alias(n: int, s: float) -> tuple[np.ndarray, np.ndarray]:
    """Walker/Vose alias table for P(k) ~ 1/(k+1)^s, k = 0..n-1, with
    integer acceptance thresholds out of 2^32 so sampling is exact integer
    arithmetic on the host and on the GPU."""
    one = 1 << 32
    w = [1.0 / math.pow(k + 1, s) for k in range(n)]
    total = math.fsum(w)
    q = [int(round(x / total * n * one)) for x in w]
    q[0] += n * one - sum(q)
    prob = [0] * n
    alias = list(range(n))
    small = [i for i in range(n) if q[i] < one]
    large = [i for i in range(n) if q[i] >= one]
    while small and large:
        lo = small.pop()
        hi = large.pop()
        prob[lo] = q[lo]
        alias[lo] = hi
        q[hi] -= one - q[lo]
        (small if q[hi] < one else large).append(hi)
    for i in large + small:
        prob[i] = one
    return np.array(prob, np.uint64), np.array(alias, np.uint64)


def alias_sample(u: np.ndarray, prob: np.ndarray, alias: np.ndarray) -> np.ndarray:
    n = np.uint64(len(prob))
    col = ((u >> np.uint64(32)) * n) >> np.uint64(32)
    frac = u & np.uint64(0xFFFFFFFF)
    return np.where(frac < prob[col], col, alias[col])


def moe_selection(shape: MoeShape, steps: int, first_step: int = 0) -> list[list[np.ndarray]]:
    """sel[s][l]: sorted union over the step's tokens of each token's top-k
    experts, drawn without replacement from Zipf(s) (up to 64 draws per
    token, duplicates skipped; the rare shortfall is filled by the lowest
    unused expert ids)."""
    prob, alias = zipf_alias(shape.experts, shape.zipf_s)
    attempts = 64
    out = []
    per_step = shape.layers * shape.tokens * attempts
    for s in range(first_step, first_step + steps):
        u = draws(shape.seed, 100, s * per_step, per_step)
        e = alias_sample(u, prob, alias).reshape(shape.layers, shape.tokens, attempts)
        layers = []
        for l_ in range(shape.layers):
            chosen = np.zeros(shape.experts, bool)
            for t in range(shape.tokens):
                seen = []
                for x in e[l_, t]:
                    if x not in seen:
                        seen.append(int(x))
                        if len(seen) == shape.top_k:
                            break
                k = 0
                while len(seen) < shape.top_k:
                    if k not in seen:
                        seen.append(k)
                    k += 1
                chosen[seen] = True
            layers.append(np.nonzero(chosen)[0].astype(np.int64))
        out.append(layers)
    return out


def moe_segments(shape: MoeShape, selection: list[np.ndarray]) -> np.ndarray:
    """Expert base addresses read in one decode step, in issue order."""
    bases = [shape.expert_base(l_, int(e)) for l_, sel in enumerate(selection) for e in sel]
    return np.array(bases, np.uint64)


def moe_ranges(shape: MoeShape) -> list[tuple[int, int, int]]:
    """Every expert registered as its own read-only HBF range."""
    return [(shape.expert_base(l_, e), shape.expert_bytes, 1)
            for l_ in range(shape.layers) for e in range(shape.experts)]


def segment_records(seg_base: np.ndarray, lines: int, line: int, gap_ps: int, issuers: int,
                    start: int = 0, count: int | None = None, flags: int = 0) -> np.ndarray:
    """Host mirror of the GPU workload compiler (hbfsim_amd_gen_segment_lines)."""
    total = len(seg_base) * lines
    count = total - start if count is None else count
    j = np.arange(start, start + count, dtype=np.uint64)
    rec = np.zeros((count, 4), np.uint64)
    rec[:, 0] = seg_base[(j // np.uint64(lines)).astype(np.int64)] + \
        (j % np.uint64(lines)) * np.uint64(line)
    rec[:, 1] = line
    rec[:, 2] = (j // np.uint64(issuers)) * np.uint64(gap_ps)
    rec[:, 3] = flags
    return rec


def gpu_segment_records(seg_base: np.ndarray, lines: int, line: int, gap_ps: int, issuers: int,
                        flags: int = 0, out=None, stream=None):
    """Compiles one step's records on the GPU; returns an int64 [n, 4] tensor."""
    import ctypes

    import torch

    from . import _native as nat
    lib = nat.load()
    n = len(seg_base) * lines
    if out is None:
        out = torch.empty((n, 4), dtype=torch.int64, device="cuda")
    bases = torch.from_numpy(seg_base.view(np.int64)).cuda()
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    nat.check(lib.hbfsim_amd_gen_segment_lines(
        out.data_ptr(), out.shape[0], bases.data_ptr(), len(seg_base), lines, line, gap_ps,
        issuers, flags, ctypes.c_void_p(stream)), "generate records")
    torch.cuda.current_stream().synchronize()
    return out[:n]


# ---------------------------------------------------------------------------
# Spans: runs of consecutive lines, each with its own length and operation
# (the GPU compiler is hbfsim_amd_gen_spans).


def span_records(base: np.ndarray, first: np.ndarray, op: np.ndarray, line: int, gap_ps: int,
                 issuers: int, start: int = 0, count: int | None = None) -> np.ndarray:
    """Host mirror of the GPU span compiler: records [start, start + count)."""
    total = int(first[-1])
    count = total - start if count is None else count
    j = np.arange(start, start + count, dtype=np.uint64)
    s = np.searchsorted(first[:-1].astype(np.uint64), j, side="right") - 1
    rec = np.zeros((count, 4), np.uint64)
    rec[:, 0] = base[s] + (j - first[s].astype(np.uint64)) * np.uint64(line)
    rec[:, 1] = line
    rec[:, 2] = (j // np.uint64(issuers)) * np.uint64(gap_ps)
    rec[:, 3] = op[s].astype(np.uint64)
    return rec


def gpu_span_records(base: np.ndarray, first: np.ndarray, op: np.ndarray, line: int,
                     gap_ps: int, issuers: int, out=None, stream=None):
    """Compiles spans' records on the GPU; returns an int64 [n, 4] tensor."""
    import ctypes

    import torch

    from . import _native as nat
    lib = nat.load()
    n = int(first[-1])
    if out is None:
        out = torch.empty((max(n, 1), 4), dtype=torch.int64, device="cuda")
    d_base = torch.from_numpy(np.ascontiguousarray(base, np.uint64).view(np.int64)).cuda()
    d_first = torch.from_numpy(np.ascontiguousarray(first, np.uint64).view(np.int64)).cuda()
    d_op = torch.from_numpy(np.ascontiguousarray(op, np.uint32).view(np.int32)).cuda()
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    nat.check(lib.hbfsim_amd_gen_spans(
        out.data_ptr(), out.shape[0], d_base.data_ptr(), d_first.data_ptr(), d_op.data_ptr(),
        len(base), n, line, gap_ps, issuers, ctypes.c_void_p(stream)), "generate span records")
    torch.cuda.current_stream().synchronize()
    return out[:n]


def _spans(parts: list[tuple[int, int, int]]) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(base, lines, op) triples -> (base, first, op) arrays."""
    base = np.array([p[0] for p in parts], np.uint64)
    lines = np.array([p[1] for p in parts], np.uint64)
    op = np.array([p[2] for p in parts], np.uint32)
    first = np.zeros(len(parts) + 1, np.uint64)
    np.cumsum(lines, out=first[1:])
    return base, first, op


# ---------------------------------------------------------------------------
# Config 1: TinyLlama-1.1B-shaped decode weight streaming.  Every step reads
# every weight tensor front to back in 128-B lines, 256 wavefronts issuing a
# line each every 64 ns; each tensor is its own read-only range.  Profile c0.


@dataclasses.dataclass(frozen=True)
class DenseShape:
    layers: int = 22
    hidden: int = 2048
    intermediate: int = 5632
    heads: int = 32
    kv_heads: int = 4
    vocab: int = 32000
    dtype_bytes: int = 2
    line: int = 128
    issuers: int = 256
    gap_ps: int = 64_000
    page: int = 16384
    base: int = 0x4000_0000_0000

    def tensors(self) -> list[tuple[str, int]]:
        """(name, bytes) in the order a decode step reads them."""
        h, i, d = self.hidden, self.intermediate, self.dtype_bytes
        kv = self.kv_heads * (h // self.heads)
        out = [("embed_tokens", self.vocab * h * d)]
        for l_ in range(self.layers):
            out += [(f"{l_}.input_layernorm", h * d), (f"{l_}.q_proj", h * h * d),
                    (f"{l_}.k_proj", kv * h * d), (f"{l_}.v_proj", kv * h * d),
                    (f"{l_}.o_proj", h * h * d), (f"{l_}.post_attention_layernorm", h * d),
                    (f"{l_}.gate_proj", i * h * d), (f"{l_}.up_proj", i * h * d),
                    (f"{l_}.down_proj", h * i * d)]
        out += [("norm", h * d), ("lm_head", self.vocab * h * d)]
        return out

    def layout(self) -> list[tuple[int, int]]:
        """(base, bytes) per tensor, packed on page boundaries."""
        out, at = [], self.base
        for _, nbytes in self.tensors():
            out.append((at, nbytes))
            at += -(-nbytes // self.page) * self.page
        return out


TINYLLAMA = DenseShape()


def dense_ranges(shape: DenseShape) -> list[tuple[int, int, int]]:
    return [(b, n, 1) for b, n in shape.layout()]


def dense_spans(shape: DenseShape) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """One decode step's spans: every tensor, whole lines."""
    return _spans([(b, -(-n // shape.line), 0) for b, n in shape.layout()])


# ---------------------------------------------------------------------------
# Config 3: paged KV cache.  K and V of every layer live in pools of 16-token
# blocks (kv_heads * head_dim values per token, bf16); each sequence's blocks
# are scattered over its pools by a seeded permutation, with room for the
# steps' appends.  A decode step, layer by layer: every sequence appends its
# new token (K, then V: token_bytes of writes each, which end on a 16-KiB page
# boundary every 8 tokens and then program), then every sequence's K and V
# blocks are read up to the current length.  Profile c3 (256 GiB).


@dataclasses.dataclass(frozen=True)
class PagedKvShape:
    layers: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    dtype_bytes: int = 2
    block_tokens: int = 16
    seqs: int = 64
    min_len: int = 1024
    max_len: int = 32768
    seed: int = 2
    steps: int = 32
    line: int = 128
    issuers: int = 256
    gap_ps: int = 64_000
    page: int = 16384
    base: int = 0x3000_0000_0000

    @property
    def token_bytes(self) -> int:
        return self.kv_heads * self.head_dim * self.dtype_bytes

    @property
    def block_bytes(self) -> int:
        return self.block_tokens * self.token_bytes

    def lengths(self) -> np.ndarray:
        rng = np.random.default_rng(self.seed)
        return rng.integers(self.min_len, self.max_len + 1, self.seqs).astype(np.int64)

    def blocks_per_seq(self) -> np.ndarray:
        return -(-(self.lengths() + self.steps) // self.block_tokens)

    def pool_bytes(self) -> int:
        return int(self.blocks_per_seq().sum()) * self.block_bytes

    def pool_base(self, layer: int, kind: int) -> int:
        span = -(-self.pool_bytes() // self.page) * self.page
        return self.base + (2 * layer + kind) * span

    def tables(self) -> list[list[np.ndarray]]:
        """tables[layer][kind] -> physical block of (seq, logical block), flattened
        by sequence (offsets from blocks_per_seq)."""
        rng = np.random.default_rng(self.seed + 1)
        nblk = int(self.blocks_per_seq().sum())
        return [[rng.permutation(nblk) for _ in range(2)] for _ in range(self.layers)]


PAGED_KV = PagedKvShape()


def kv_ranges(shape: PagedKvShape) -> list[tuple[int, int, int]]:
    return [(shape.pool_base(l_, k), shape.pool_bytes(), 3)
            for l_ in range(shape.layers) for k in range(2)]


def kv_spans(shape: PagedKvShape, step: int,
             tables=None) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Decode step `step` (0-based) of the paged-KV configuration."""
    tables = shape.tables() if tables is None else tables
    lens = shape.lengths() + step                  # tokens before this step's append
    bps = shape.blocks_per_seq()
    off = np.concatenate([[0], np.cumsum(bps)[:-1]])
    tb, bt, line = shape.token_bytes, shape.block_bytes, shape.line
    wlines = tb // line
    nread = -(-(lens + 1) // shape.block_tokens)   # blocks read, the new token included
    seq_of = np.repeat(np.arange(shape.seqs), nread)
    blk_of = np.arange(int(nread.sum())) - np.repeat(np.cumsum(nread) - nread, nread)
    valid = np.minimum(shape.block_tokens, lens[seq_of] + 1 - blk_of * shape.block_tokens)
    rlines = (valid * tb // line).astype(np.uint64)
    bases, lines, ops = [], [], []
    for l_ in range(shape.layers):
        pk, pv = shape.pool_base(l_, 0), shape.pool_base(l_, 1)
        tk, tv = tables[l_]
        # appends: K then V of every sequence
        blk = off + lens // shape.block_tokens
        at = (lens % shape.block_tokens) * tb
        wb = np.empty(2 * shape.seqs, np.uint64)
        wb[0::2] = np.uint64(pk) + tk[blk].astype(np.uint64) * np.uint64(bt) + at.astype(np.uint64)
        wb[1::2] = np.uint64(pv) + tv[blk].astype(np.uint64) * np.uint64(bt) + at.astype(np.uint64)
        bases.append(wb)
        lines.append(np.full(2 * shape.seqs, wlines, np.uint64))
        ops.append(np.ones(2 * shape.seqs, np.uint32))
        # reads: every sequence's K blocks, then its V blocks
        phys = off[seq_of] + blk_of
        kb = np.uint64(pk) + tk[phys].astype(np.uint64) * np.uint64(bt)
        vb = np.uint64(pv) + tv[phys].astype(np.uint64) * np.uint64(bt)
        starts = np.concatenate([[0], np.cumsum(nread)[:-1]])
        order_b, order_l = [], []
        for s in range(shape.seqs):
            a, z = starts[s], starts[s] + nread[s]
            order_b += [kb[a:z], vb[a:z]]
            order_l += [rlines[a:z], rlines[a:z]]
        bases.append(np.concatenate(order_b))
        lines.append(np.concatenate(order_l))
        ops.append(np.zeros(sum(len(x) for x in order_b), np.uint32))
    base = np.concatenate(bases)
    nl = np.concatenate(lines)
    first = np.zeros(len(base) + 1, np.uint64)
    np.cumsum(nl, out=first[1:])
    return base, first, np.concatenate(ops)


# ---------------------------------------------------------------------------
# Routed-expert trace events (adapters/vllm_capacity/trace_schema.json,
# written by trace_collector.py:163-199) compiled into record streams.  An
# event is one (token, layer) of a request: its top-k experts and the
# compact list of their tensor accesses, each a byte range
# [source_offset_begin, source_offset_end) of a checkpoint shard with the
# pages it touches and a stream-wide access_order_sequence.  Each tensor
# access becomes one span of line reads at the shard's base address, in
# access order.


def _event_int(event: dict, key: str) -> int:
    value = event[key]
    if isinstance(value, bool) or not isinstance(value, int) or value < 0:
        raise ValueError(f"trace event field {key} must be a non-negative integer")
    return value


def trace_event_spans(events, shard_base: dict[str, int], page_bytes: int, line_bytes: int,
                      whole_pages: bool = False) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Spans (base, first, op) for the tensor accesses of schema-1 trace
    events, in access order.  A span reads the lines covering the tensor's
    byte range (with whole_pages, its pages [page_begin, page_end)) at
    shard_base[source_shard] + offset.  Raises ValueError where the
    reference's readers reject an event (trace_replay.py:100-108 and
    trace_collector.py:154-160: schema version, empty or repeated top-k ids)
    and where an event disagrees with how the collector wrote it (page
    bounds from the offsets, access sequences consecutive from one event to
    the next, an expert tensor of an expert outside the top-k)."""
    if page_bytes <= 0 or line_bytes <= 0 or page_bytes % line_bytes:
        raise ValueError("page_bytes must be a positive multiple of line_bytes")
    parts: list[tuple[int, int, int]] = []
    next_seq = None
    for event in events:
        if isinstance(event, (str, bytes)):
            import json
            event = json.loads(event)
        if event.get("schema_version") != 1:
            raise ValueError("unsupported trace schema")
        ids = [int(v) for v in event["topk_expert_ids"]]
        if not ids or len(set(ids)) != len(ids) or min(ids) < 0:
            raise ValueError("invalid top-k expert list")
        begin = _event_int(event, "access_order_sequence_begin")
        end = _event_int(event, "access_order_sequence_end")
        if next_seq is not None and begin != next_seq:
            raise ValueError("access order sequences are not consecutive across events")
        tensors = sorted(event["expert_tensors"], key=lambda t: _event_int(t, "access_order_sequence"))
        if [int(t["access_order_sequence"]) for t in tensors] != list(range(begin, end)):
            raise ValueError("tensor access sequences do not fill the event's range")
        next_seq = end
        for t in tensors:
            if int(t["expert_id"]) not in ids:
                raise ValueError("tensor access of an expert outside the top-k")
            lo = _event_int(t, "source_offset_begin")
            hi = _event_int(t, "source_offset_end")
            if hi <= lo:
                raise ValueError("empty tensor byte range")
            pb, pe = _event_int(t, "page_begin"), _event_int(t, "page_end")
            if pb != lo // page_bytes or pe != (hi + page_bytes - 1) // page_bytes:
                raise ValueError("page bounds differ from the byte range")
            shard = t["source_shard"]
            if shard not in shard_base:
                raise ValueError(f"no base address for shard {shard!r}")
            if int(shard_base[shard]) % line_bytes:
                raise ValueError("shard base addresses must be line-aligned")
            if whole_pages:
                lo, hi = pb * page_bytes, pe * page_bytes
            first_line = lo // line_bytes
            lines = (hi + line_bytes - 1) // line_bytes - first_line
            parts.append((int(shard_base[shard]) + first_line * line_bytes, lines, 0))
    if not parts:
        raise ValueError("trace contains no expert accesses")
    return _spans(parts)
