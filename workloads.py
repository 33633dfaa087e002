"""Synthetic workloads for bench.py and the tests: seeded KV pools, block selections, a model-free runner
and the multi-agent pressure driver.

Shapes follow the pool layout [2, L, NB, BS, H, hd] (nanovllm/engine/model_runner.py:120).
Values are generated on the pool's device, one (K/V, layer) plane at a time,
with a torch.Generator seeded per plane so any plane can be regenerated.
"""

import time
from dataclasses import dataclass

import numpy as np
import torch


@dataclass(frozen=True)
class PoolShape:
    layers: int
    num_blocks: int
    block_size: int = 256
    kv_heads: int = 8
    head_dim: int = 128

    @property
    def shape(self) -> tuple[int, ...]:
        return (2, self.layers, self.num_blocks, self.block_size, self.kv_heads, self.head_dim)

    @property
    def block_elems(self) -> int:
        return 2 * self.layers * self.block_size * self.kv_heads * self.head_dim

    @property
    def block_bytes_bf16(self) -> int:
        return 2 * self.block_elems

    @property
    def rows_per_block(self) -> int:
        return 2 * self.layers * self.block_size * self.kv_heads


# Qwen3 KV geometry (8 KV heads, head_dim 128, 256-token blocks).
QWEN3_8B = PoolShape(layers=36, num_blocks=320)
QWEN3_0_6B = PoolShape(layers=28, num_blocks=512)


def _plane_generator(device, seed: int, kv: int, layer: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed((seed * 1_000_003 + kv * 4099 + layer) & 0x7FFFFFFFFFFFFFFF)
    return g


def fill_normal(pool: torch.Tensor, seed: int = 0):
    """pool <- bf16(N(0, 1)), plane by plane."""
    for kv in range(2):
        for layer in range(pool.shape[1]):
            g = _plane_generator(pool.device, seed, kv, layer)
            plane = pool[kv, layer]
            plane.copy_(torch.randn(plane.shape, generator=g, device=pool.device, dtype=torch.float32))
    return pool


def fill_student_t(pool: torch.Tensor, seed: int = 0, df: int = 4, scale: float = 0.5,
                   outlier_channels: int = 4, outlier_gain: float = 20.0):
    """pool <- bf16(scale * t_df) with `outlier_channels` seeded channels per (K/V, layer, head) x gain.

    t_df = z / sqrt(chi2_df / df) with chi2_df a sum of df squared normals.
    """
    heads, hd = pool.shape[4], pool.shape[5]
    for kv in range(2):
        for layer in range(pool.shape[1]):
            g = _plane_generator(pool.device, seed, kv, layer)
            plane = pool[kv, layer]
            z = torch.randn(plane.shape, generator=g, device=pool.device, dtype=torch.float32)
            chi2 = torch.zeros_like(z)
            for _ in range(df):
                chi2.add_(torch.randn(plane.shape, generator=g, device=pool.device, dtype=torch.float32).square_())
            t = z.div_(chi2.div_(df).sqrt_()).mul_(scale)
            del chi2
            gain = torch.ones((heads, hd), device=pool.device, dtype=torch.float32)
            for h in range(heads):
                channels = torch.randperm(hd, generator=g, device=pool.device)[:outlier_channels]
                gain[h, channels] = outlier_gain
            plane.copy_(t.mul_(gain))
    return pool


def block_selection(num_blocks: int, count: int, seed: int, exclude=()) -> list[int]:
    """`count` distinct seeded block ids from [0, num_blocks) minus `exclude`."""
    g = torch.Generator().manual_seed(seed)
    excluded = set(exclude)
    order = [b for b in torch.randperm(num_blocks, generator=g).tolist() if b not in excluded]
    if count > len(order):
        raise ValueError(f"cannot pick {count} of {len(order)} blocks")
    return order[:count]


# ---------------------------------------------------------------------------
# Model-free engine runs

def synthetic_kv(tokens: torch.Tensor, positions: torch.Tensor, layers: int, heads: int, head_dim: int,
                 dtype=torch.bfloat16) -> torch.Tensor:
    """Deterministic K and V rows [2, layers, n, heads, head_dim] for tokens at positions.

    A stand-in for a model's projections: any block's expected contents can be
    recomputed from its tokens and positions alone. All layers come from one
    broadcast expression per K/V half, so a run costs a few launches per step.
    """
    dev = tokens.device
    t = tokens.to(torch.float32)[:, None, None]
    p = positions.to(torch.float32)[:, None, None]
    h = torch.arange(heads, device=dev, dtype=torch.float32)[None, :, None]
    d = torch.arange(head_dim, device=dev, dtype=torch.float32)[None, None, :]
    base = 0.37 * t + 0.0113 * p + 0.71 * h + 0.173 * d  # [n, heads, head_dim]
    layer = torch.arange(layers, device=dev)
    # Outlier channels: amplitude 5 where (7d + 3h + layer) % 29 == 0.
    hit = (d.to(torch.int64) * 7 + h.to(torch.int64) * 3 + layer[:, None, None, None]) % 29 == 0
    amp = 1.0 + 4.0 * hit.to(torch.float32)  # [layers, 1, heads, head_dim]
    out = torch.empty((2, layers, tokens.numel(), heads, head_dim), dtype=dtype, device=dev)
    for kv in range(2):
        offset = (1.31 * layer.to(torch.float64) + 2.9 * kv).to(torch.float32)[:, None, None, None]
        out[kv] = (torch.sin(base[None] + offset) * amp).to(dtype)
    return out


class SyntheticKVRunner:
    """Runner for kvx.engine.llm_engine.LLMEngine that writes every scheduled token's K/V.

    call("run", seqs, is_prefill) computes the slot mapping the way
    nanovllm's ModelRunner does (model_runner.py:156-166, 186) and uploads
    it, the token ids and the positions through pinned memory without
    blocking the host (:169-173, 187-190), writes synthetic_kv rows for all
    layers through kvx.ops.store_kvcache on the current stream, then
    "samples" `next_token` for each sequence on the device and reads the
    tokens back, which blocks the host until the step's GPU work is done, as
    the reference's sampler readback does (:223). `blocked_s` adds up the
    host time spent in those readbacks.
    """

    def __init__(self, pool: torch.Tensor, next_token: int = 1):
        self.kv_cache = pool
        self.world_size = 1
        self.block_size = pool.shape[3]
        self.next_token = next_token
        self.tokens_written = 0
        self.blocked_s = 0.0

    def call(self, method, *args):
        if method == "exit":
            return None
        from kvx import ops
        from kvx.engine.slot_mapping import decode_slot_mapping, prefill_slot_mapping, upload

        seqs, is_prefill = args
        bs = self.block_size
        if is_prefill:
            slots = prefill_slot_mapping(seqs, bs)
            toks, pos = [], []
            for seq in seqs:
                start = seq.num_cached_tokens
                toks += seq.token_ids[start:start + seq.num_scheduled_tokens]
                pos.append(np.arange(start, start + seq.num_scheduled_tokens, dtype=np.int64))
            pos = np.concatenate(pos) if pos else np.empty(0, dtype=np.int64)
        else:
            slots = decode_slot_mapping(seqs, bs)
            toks = [seq.last_token for seq in seqs]
            pos = np.array([len(seq) - 1 for seq in seqs], dtype=np.int64)
        if len(slots):
            pool = self.kv_cache
            dev = pool.device
            t = upload(np.asarray(toks, dtype=np.int64), dev)
            p = upload(pos, dev)
            mapping = upload(slots, dev)
            kv = synthetic_kv(t, p, pool.shape[1], pool.shape[4], pool.shape[5], pool.dtype)
            for layer in range(pool.shape[1]):
                ops.store_kvcache(kv[0, layer], kv[1, layer], pool[0, layer], pool[1, layer], mapping)
            self.tokens_written += len(slots)
        sampled = torch.full((len(seqs),), self.next_token, dtype=torch.int64, device=self.kv_cache.device)
        t0 = time.perf_counter()
        tokens = sampled.tolist()
        self.blocked_s += time.perf_counter() - t0
        return tokens


def expected_block(pool: torch.Tensor, token_ids, start_position: int) -> torch.Tensor:
    """[2, L, BS, H, hd] contents SyntheticKVRunner writes for one full block of tokens."""
    dev = pool.device
    t = torch.tensor(list(token_ids), device=dev)
    p = torch.arange(start_position, start_position + len(token_ids), device=dev)
    return synthetic_kv(t, p, pool.shape[1], pool.shape[4], pool.shape[5], pool.dtype)


@dataclass
class AgentPressureResult:
    turns: int
    wall_s: float
    saved_blocks: int
    restored_blocks: int
    prefetched_blocks: int
    budget_skips: int
    d2h_bytes: int
    h2d_bytes: int
    blocks_checked: int
    blocks_fp8_round_trip: int
    host_blocked_s: float = 0.0  # in the runner's token readbacks
    drain_s: float = 0.0         # after the last step, waiting for the copy streams and the GPU

    @property
    def link_gbs(self) -> float:
        return (self.d2h_bytes + self.h2d_bytes) / self.wall_s / 1e9


def run_agent_pressure(engine, agents: int = 4, context: int = 32768, turns: int = 12, append: int = 2048,
                       seed: int = 0, verify: bool = True, verify_stride: int = 1,
                       hints: str | None = "deferred") -> AgentPressureResult:
    """Multi-turn agents sharing one pool: each turn an agent returns with its whole context plus `append`
    new tokens, evicting others' blocks (saved to the CPU tier) and restoring or prefetching its own.

    With verify=True every `verify_stride`-th full block (and the last) of each finished request must hold
    either the exact synthetic KV (GPU hit or recomputed) or its FP8 round trip (restored from an FP8 entry) --
    a block restored from the wrong slot, or read before its restore finished, matches neither.

    `hints` says when the next agent's prefix is hinted with prefetch_prefix:
    - "deferred": right after the current request is added, with defer=True. The engine starts the hint in
      the step that admits the current request, after its admission and before the model runs, so the next
      agent's restores (H2D) overlap the current request's compute and the saves (D2H) of the blocks they
      evict;
    - "after_first_step": after the request's first step (or, if that step finished it, once it is checked),
      as a client without deferred hints has to: the restores then start after that step's compute;
    - None: no hints.
    A hint started before the current request's admission would let the prefetch evict the current agent's
    own cached blocks (the least recently used ones), which its admission would then restore again.
    """
    if hints not in ("deferred", "after_first_step", None):
        raise ValueError(f"unknown hint mode {hints!r}")
    from kvx import ops
    from kvx.engine.sequence import SamplingParams, Sequence

    g = torch.Generator().manual_seed(seed)
    histories = [torch.randint(2, 50000, (context,), generator=g).tolist() for _ in range(agents)]
    pool = engine.model_runner.kv_cache
    cache = engine._cpu_prefix_cache
    bs = pool.shape[3]
    params = SamplingParams(temperature=0, max_tokens=1, ignore_eos=True)
    checked = fp8_hits = 0
    blocked_before = getattr(engine.model_runner, "blocked_s", 0.0)
    t0 = time.perf_counter()
    for turn in range(turns):
        for a in range(agents):
            histories[a] += torch.randint(2, 50000, (append,), generator=g).tolist()
            engine.add_request(histories[a], params)
            nxt = Sequence(histories[(a + 1) % agents]) if hints and agents > 1 else None
            if nxt is not None and hints == "deferred":
                engine.prefetch_prefix(nxt, defer=True)
                nxt = None
            while not engine.is_finished():
                engine.step()
                if nxt is not None and not engine.is_finished():
                    # After this request's admission, so the prefetch takes other agents' blocks, not its own.
                    engine.prefetch_prefix(nxt)
                    nxt = None
            histories[a] += [engine.model_runner.next_token]
            if verify:
                # The request's full blocks are now idle GPU hits: check a sample of them.
                manager = engine.scheduler.block_manager
                h = -1
                full_blocks = (len(histories[a]) - 1) // bs
                for i in range(full_blocks):
                    tokens = histories[a][i * bs:(i + 1) * bs]
                    h = manager.compute_hash(tokens, h)
                    block_id = manager.hash_to_block_id.get(h)
                    if block_id is None:
                        break
                    if i % verify_stride and i != full_blocks - 1:
                        continue
                    if cache is not None:
                        cache.before_block_use(block_id)
                    expect = expected_block(pool, tokens, i * bs)
                    got = pool[:, :, block_id]
                    if torch.equal(got.view(torch.int16), expect.view(torch.int16)):
                        checked += 1
                        continue
                    payload = torch.empty(expect.shape, dtype=torch.float8_e4m3fn, device=pool.device)
                    scale = torch.empty((*expect.shape[:-1], 1), dtype=cache._scale_dtype, device=pool.device)
                    ops.fp8_quantize(expect, payload, scale)
                    round_trip = torch.empty_like(expect)
                    ops.fp8_dequantize(payload, scale, round_trip)
                    if not torch.equal(got.view(torch.int16), round_trip.view(torch.int16)):
                        raise AssertionError(f"turn {turn} agent {a}: block {i} (GPU block {block_id}) holds "
                                             "neither its KV nor the FP8 round trip of it")
                    checked += 1
                    fp8_hits += 1
            if nxt is not None:
                # The request finished in one step: hint once it is checked (the prefetch may recycle its blocks).
                engine.prefetch_prefix(nxt)
    t_drain = time.perf_counter()
    if cache is not None:
        cache.synchronize()
    torch.cuda.synchronize(pool.device)
    wall = time.perf_counter() - t0
    drain = time.perf_counter() - t_drain
    stats = cache.stats if cache is not None else {"saved_blocks": 0, "restored_blocks": 0, "budget_skips": 0}
    entry = cache.block_bytes if cache is not None else 0
    blocked = getattr(engine.model_runner, "blocked_s", 0.0) - blocked_before
    return AgentPressureResult(turns * agents, wall, stats["saved_blocks"], stats["restored_blocks"],
                               cache.prefetched_blocks if cache is not None else 0, stats["budget_skips"],
                               stats["saved_blocks"] * entry, stats["restored_blocks"] * entry, checked, fp8_hits,
                               blocked, drain)

