"""KV pool, step execution and the two HIP-graph modes of the engine harness.

A step is a list of (sequence, tokens to compute). `ModelRunner.execute` lays the tokens out
as one flat batch, builds the attention metadata (on the device from resident block tables,
or on the host as the reference does) and runs the model one of three ways, chosen per step
as kvserve's ModelRunner chooses (src/kvserve/model_runner.py:130-143):

  decode_graph  every sequence computes one token and the batch fits a captured bucket: the
                whole forward pass replays from one HIP graph over static buffers, the batch
                padded with rows that write the pool's scratch block;
  piecewise     any other step of at most `max_piecewise_tokens` tokens: the model's row-wise
                stages replay from HIP graphs captured per token-count bucket, and the
                attention steps run eagerly in between on the real tokens (the boundary of
                src/kvserve/cuda_graph.py:140-241);
  eager         larger steps, or graphs disabled.

`Batcher` forms the steps (no scheduler here): sequences in flight first, then arrivals, under
a token budget, so prefill chunks and decodes share steps as they do under kvserve's
scheduler.
"""

from __future__ import annotations

from collections import Counter
from dataclasses import dataclass, field

import numpy as np
import torch

from kvserve_amd.attention import AttentionMetadata, build_metadata
from kvserve_amd.engine.model import PagedLlama, StageOut
from kvserve_amd.metadata import DeviceMetadata, MetaBuffers


def decode_buckets(max_batch: int) -> list[int]:
    """Padded batch sizes with a captured decode graph: 1, 2, 4, 8, every 8 up to 64 (where the
    small-batch projections' cost follows the row count closely), every 32 beyond; the
    largest is max_batch itself."""
    sizes = [s for s in (1, 2, 4, 8) if s < max_batch]
    sizes += [s for s in range(16, min(max_batch, 64) + 1, 8) if s < max_batch]
    sizes += list(range(96, max_batch, 32))
    return sizes + [max_batch]


def token_buckets(max_tokens: int) -> list[int]:
    """Token counts with captured piecewise stages: 1, 2, 4, 8, 16, 32, 48 (launch-bound steps,
    where padding is nearly free), then from 64 on steps of 1/4 of the bucket: every 16 up to
    128, every 32 up to 256, every 64 up to 512, every 128 up to 1024, every 256 beyond, so
    padding never adds more than a quarter of the row-wise work; the largest is max_tokens."""
    sizes = [1, 2, 4, 8, 16, 32, 48]
    sizes += list(range(64, 129, 16)) + list(range(160, 257, 32)) + list(range(320, 513, 64))
    sizes += list(range(640, 1025, 128)) + list(range(1280, max_tokens, 256))
    return sorted({s for s in sizes if s < max_tokens} | {max_tokens})


def _bucket(sizes: list[int], n: int) -> int | None:
    for s in sizes:
        if s >= n:
            return s
    return None


# -- KV pool -----------------------------------------------------------------------------------


class KVPool:
    """The paged KV cache of every layer, [L, 2, num_blocks + 1, BS, Hkv, D], and its free list.
    Block `num_blocks` is scratch for graph padding rows and is never handed out."""

    def __init__(self, model: PagedLlama, num_blocks: int, block_size: int, dtype: torch.dtype):
        cfg = model.cfg
        shape = (cfg.num_layers, 2, num_blocks + 1, block_size, cfg.num_kv_heads, cfg.head_dim)
        if dtype == torch.float8_e4m3fn:  # zero bytes viewed as E4M3 (+0)
            self.tensor = torch.zeros(shape, dtype=torch.uint8, device=model.device).view(dtype)
        else:
            self.tensor = torch.zeros(shape, dtype=dtype, device=model.device)
        self.num_blocks, self.block_size = num_blocks, block_size
        self.scratch_block = num_blocks
        self._free = list(range(num_blocks))[::-1]  # a stack: low ids first

    @staticmethod
    def blocks_in(model: PagedLlama, gib: float, block_size: int, dtype: torch.dtype) -> int:
        """Blocks that fit `gib` GiB: K and V of every layer for `block_size` tokens each
        (the reference's sizing, model_runner.py:94-98)."""
        cfg = model.cfg
        per_block = 2 * cfg.num_layers * block_size * cfg.num_kv_heads * cfg.head_dim * dtype.itemsize
        return max(1, int(gib * 2**30) // per_block)

    @property
    def free_blocks(self) -> int:
        return len(self._free)

    def take(self, n: int) -> list[int]:
        if n > len(self._free):
            raise RuntimeError(f"KV pool exhausted: {n} blocks wanted, {len(self._free)} free")
        got = self._free[len(self._free) - n :][::-1]
        del self._free[len(self._free) - n :]
        return got

    def give_back(self, blocks: list[int]) -> None:
        self._free.extend(reversed(blocks))


@dataclass(eq=False)
class Sequence:
    tokens: list[int]  # prompt, then generated tokens
    max_new_tokens: int = 1 << 30
    table: list[int] = field(default_factory=list)  # physical block ids
    computed: int = 0  # tokens whose K/V are in the pool
    prompt_len: int = -1

    def __post_init__(self) -> None:
        if self.prompt_len < 0:
            self.prompt_len = len(self.tokens)

    @property
    def pending(self) -> int:
        return len(self.tokens) - self.computed

    @property
    def generated(self) -> list[int]:
        return self.tokens[self.prompt_len :]

    @property
    def finished(self) -> bool:
        return len(self.tokens) - self.prompt_len >= self.max_new_tokens


# -- graphs --------------------------------------------------------------------------------------


class _GraphCapture:
    """Captures Python callables as HIP graphs on one shared memory pool (the first capture
    creates it), after warm-up runs on a side stream so that lazy initialisation inside
    libraries and allocator growth happen outside the capture."""

    def __init__(self) -> None:
        self.pool = None
        self.side = torch.cuda.Stream()

    def __call__(self, fn, warmups: int = 2):
        main = torch.cuda.current_stream()
        self.side.wait_stream(main)
        with torch.cuda.stream(self.side):
            for _ in range(warmups):
                fn()
        main.wait_stream(self.side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=self.pool):
            out = fn()
        if self.pool is None:
            self.pool = graph.pool()
        return graph, out


class DecodeGraphRunner:
    """Whole-forward HIP graphs for uniform decode steps, one per bucket of decode_buckets.

    Static inputs (ids, positions, slots, tables, lengths) live in a MetaBuffers; a batch of n
    replays the smallest bucket >= n, its rows n.. padded with token 0 at position 0, one key,
    the scratch block's first slot and a table row of the scratch block, so they never touch
    blocks a sequence owns. A refresh writes only the first `width` table columns (the longest
    table of the batch): the kernels read ceil(seq_len / BS) columns, never max_seq_len."""

    def __init__(self, model: PagedLlama, pool: KVPool, max_batch: int, max_blocks_per_seq: int):
        self.model, self.pool = model, pool
        self.sizes = decode_buckets(max_batch)
        self.scratch_slot = pool.scratch_block * pool.block_size
        self.buf = MetaBuffers(model.device, self.sizes[-1], self.sizes[-1], max_blocks_per_seq,
                               slot_fill=self.scratch_slot, table_fill=pool.scratch_block)  # fmt: skip
        self.graphs: dict[int, tuple[torch.cuda.CUDAGraph, torch.Tensor]] = {}

    @property
    def max_batch(self) -> int:
        return self.sizes[-1]

    def _meta(self, n: int) -> AttentionMetadata:
        b = self.buf
        return AttentionMetadata(b.slot_mapping[:n], b.block_tables[:n], b.seq_lens[:n], b.query_lens[:n],
                                 b.query_start_loc[: n + 1], max_seq_len=1, max_query_len=1)  # fmt: skip

    @torch.inference_mode()
    def capture(self, cap: _GraphCapture) -> None:
        """Largest bucket first, so the smaller graphs reuse its pool memory."""
        b = self.buf
        for n in sorted(self.sizes, reverse=True):
            meta = self._meta(n)
            self.graphs[n] = cap(lambda n=n, meta=meta: self.model(b.input_ids[:n], b.positions[:n],
                                                                   self.pool.tensor, meta))  # fmt: skip

    @torch.inference_mode()
    def replay_host(self, ids: list[int], positions: list[int], slots: list[int], tables: list[list[int]],
                    seq_lens: list[int]) -> torch.Tensor:  # fmt: skip
        """Refresh the static buffers from host lists (the reference's path) and replay."""
        n = len(ids)
        size = _bucket(self.sizes, n)
        width = max(len(t) for t in tables)
        vec = np.empty((4, size), dtype=np.int64)
        vec[0, :n], vec[0, n:] = ids, 0
        vec[1, :n], vec[1, n:] = positions, 0
        vec[2, :n], vec[2, n:] = slots, self.scratch_slot
        vec[3, :n], vec[3, n:] = seq_lens, 1
        rows = np.full((size, width), self.pool.scratch_block, dtype=np.int64)
        for r, t in enumerate(tables):
            rows[r, : len(t)] = t
        dev = self.buf.input_ids.device
        v = torch.from_numpy(vec).to(dev, non_blocking=True)
        b = self.buf
        for dst, row in ((b.input_ids, 0), (b.positions, 1), (b.slot_mapping, 2), (b.seq_lens, 3)):
            dst[:size].copy_(v[row])
        b.block_tables[:size, :width].copy_(torch.from_numpy(rows).to(dev, non_blocking=True))
        graph, out = self.graphs[size]
        graph.replay()
        return out[:n]

    @torch.inference_mode()
    def replay_device(self, dm: DeviceMetadata, keyed: list[tuple[object, list[int]]], starts: list[int],
                      ids: list[int]) -> torch.Tensor:  # fmt: skip
        """Refresh the static buffers on the device from the resident tables, then replay."""
        n = len(ids)
        size = _bucket(self.sizes, n)
        width = max(len(t) for _, t in keyed)
        dm.build(keyed, starts, [1] * n, ids, buffers=self.buf, pad_seqs=size - n, pad_slot=self.scratch_slot,
                 table_pad=self.pool.scratch_block, width=width)  # fmt: skip
        graph, out = self.graphs[size]
        graph.replay()
        return out[:n]


class PiecewiseGraphRunner:
    """HIP graphs of the model's row-wise stages, one per (stage, token bucket); the attention
    steps run eagerly between the replays on the real rows (src/kvserve/cuda_graph.py:140-241).

    Stages read and write static buffers: token ids, the residual stream, the fused QKV
    projection and the attention output. Rows past the step's token count hold stale but
    finite values from earlier steps; they are computed and dropped, and never reach attention
    or the cache."""

    def __init__(self, model: PagedLlama, max_tokens: int, ids: torch.Tensor | None = None):
        self.model = model
        self.sizes = token_buckets(max_tokens)
        t, cfg, dev, dt = self.sizes[-1], model.cfg, model.device, model.dtype
        self.ids = ids[:t] if ids is not None else torch.zeros(t, dtype=torch.long, device=dev)
        if self.ids.shape[0] < t:
            raise ValueError("the shared token-id buffer is shorter than the largest bucket")
        self.resid = torch.zeros(t, cfg.hidden_size, dtype=dt, device=dev)
        self.qkv = torch.zeros(t, (cfg.num_heads + 2 * cfg.num_kv_heads) * cfg.head_dim, dtype=dt, device=dev)
        self.attn = torch.zeros(t, cfg.num_heads, cfg.head_dim, dtype=dt, device=dev)
        self.q = torch.zeros(t, cfg.num_heads, cfg.head_dim, dtype=dt, device=dev)  # rotated queries
        self.graphs: dict[tuple[int, int], torch.cuda.CUDAGraph] = {}

    @property
    def max_tokens(self) -> int:
        return self.sizes[-1]

    def _stage(self, i: int, n: int) -> None:
        s = self.model.stage(i, self.ids[:n], self.resid[:n], self.attn[:n], defer=False)
        self.resid[:n].copy_(s.resid)  # after the last stage: the final hidden states
        if s.qkv is not None:
            self.qkv[:n].copy_(s.qkv)

    @torch.inference_mode()
    def capture(self, cap: _GraphCapture) -> None:
        for n in sorted(self.sizes, reverse=True):
            for i in range(self.model.num_layers + 1):
                self.graphs[(i, n)], _ = cap(lambda i=i, n=n: self._stage(i, n))

    @torch.inference_mode()
    def run(self, n: int, positions: torch.Tensor, kv_caches: torch.Tensor, meta: AttentionMetadata) -> torch.Tensor:
        """Final hidden states [n, hidden] of a step whose token ids are in `self.ids[:n]`."""
        size = _bucket(self.sizes, n)
        L = self.model.num_layers
        for i in range(L + 1):
            self.graphs[(i, size)].replay()
            if i < L:
                s = StageOut(self.resid[:n], self.qkv[:n], None)
                self.model.attention(i, s, positions, kv_caches[i], meta, out=self.attn[:n], q_out=self.q[:n])
        return self.resid[:n]


# -- steps ---------------------------------------------------------------------------------------


class ModelRunner:
    """Owns the model's KV pool and runs steps of (sequence, tokens) with greedy sampling.

    Pool size: `num_blocks`, or as many blocks as `kv_cache_gib` GiB hold. The graph modes
    default to on for a graph-capturable backend on the GPU (the capability the reference
    checks as `backend is TritonAttention`, model_runner.py:47) and off otherwise;
    `device_metadata` (default on the GPU when the backend reads the packed layout) builds step
    inputs with kvh_prepare_metadata from resident block tables."""

    def __init__(self, model: PagedLlama, *, num_blocks: int | None = None, kv_cache_gib: float | None = None,
                 block_size: int = 16, max_model_len: int = 4096, decode_graphs: bool | None = None,
                 piecewise_graphs: bool | None = None, max_graph_batch: int = 128, max_piecewise_tokens: int = 512,
                 token_budget: int = 2048, device_metadata: bool | None = None, max_seqs: int = 1024,
                 kv_cache_dtype: torch.dtype | None = None):  # fmt: skip
        if max_model_len > model.max_positions:
            # positions past the RoPE tables would be clamped (fused kernel) or index out of range
            raise ValueError(f"max_model_len {max_model_len} exceeds the model's {model.max_positions} RoPE positions")
        self.model = model
        self.device = model.device
        self.block_size, self.max_model_len = block_size, max_model_len
        self.token_budget = token_budget
        kv_dtype = model.dtype if kv_cache_dtype is None else kv_cache_dtype
        if num_blocks is None:
            if kv_cache_gib is None:
                raise ValueError("give num_blocks or kv_cache_gib")
            num_blocks = KVPool.blocks_in(model, kv_cache_gib, block_size, kv_dtype)
        self.pool = KVPool(model, num_blocks, block_size, kv_dtype)
        self.width = -(-max_model_len // block_size)
        backend = model.backend
        capturable = self.device.type == "cuda" and getattr(backend, "graph_capturable", False)
        decode_graphs = capturable if decode_graphs is None else decode_graphs
        piecewise_graphs = capturable if piecewise_graphs is None else piecewise_graphs
        self.padded_layout = getattr(backend, "needs_padded_layout", True)
        if device_metadata is None:
            device_metadata = self.device.type == "cuda" and not self.padded_layout
        if device_metadata and self.padded_layout:
            raise ValueError("device metadata does not build the torch backend's padded layout")
        self.dm = None
        if device_metadata:
            tokens = max(token_budget, max_graph_batch, max_piecewise_tokens if piecewise_graphs else 1)
            self.dm = DeviceMetadata(self.device, max_seqs, self.width, block_size, tokens)
        self.paths: Counter[str] = Counter()
        self.decode_runner: DecodeGraphRunner | None = None
        self.piecewise: PiecewiseGraphRunner | None = None
        if decode_graphs or piecewise_graphs:
            if not getattr(backend, "graph_capturable", False):
                raise ValueError(f"backend {getattr(backend, 'name', backend)} cannot be captured in a graph")
            cap = _GraphCapture()
            if piecewise_graphs:
                ids = self.dm.buffers.input_ids if self.dm is not None else None
                self.piecewise = PiecewiseGraphRunner(model, min(max_piecewise_tokens, token_budget), ids)
                self.piecewise.capture(cap)
            if decode_graphs:
                self.decode_runner = DecodeGraphRunner(model, self.pool, max_graph_batch, self.width)
                self.decode_runner.capture(cap)

    @property
    def kv_caches(self) -> torch.Tensor:
        return self.pool.tensor

    def release(self, seq: Sequence) -> None:
        self.pool.give_back(seq.table)
        seq.table = []
        if self.dm is not None:
            self.dm.release(id(seq))

    def _route(self, query_lens: list[int], num_tokens: int, eager: bool) -> str:
        if not eager:
            d = self.decode_runner
            if d is not None and max(query_lens) == 1 and len(query_lens) <= d.max_batch:
                return "decode_graph"
            if self.piecewise is not None and num_tokens <= self.piecewise.max_tokens:
                return "piecewise"
        return "eager"

    @torch.inference_mode()
    def execute(self, scheduled: list[tuple[Sequence, int]], eager: bool = False) -> dict[Sequence, int]:
        """One forward over `scheduled`; every sequence whose whole context is computed after it
        gets its greedy next token appended. Returns {sequence: token} for those."""
        bs = self.block_size
        ids: list[int] = []
        starts, qlens, last_rows, sampled = [], [], [], []
        for seq, n in scheduled:
            start = seq.computed
            if n < 1 or start + n > len(seq.tokens):
                raise ValueError(f"cannot compute {n} tokens of a sequence with {seq.pending} pending")
            if start + n > self.max_model_len:
                raise ValueError(f"sequence of {start + n} tokens exceeds max_model_len={self.max_model_len}")
            need = -(-(start + n) // bs) - len(seq.table)
            if need > 0:
                seq.table += self.pool.take(need)
            ids += seq.tokens[start : start + n]
            starts.append(start)
            qlens.append(n)
            if start + n == len(seq.tokens):
                last_rows.append(len(ids) - 1)
                sampled.append(seq)
        T = len(ids)
        path = self._route(qlens, T, eager)
        if self.dm is not None:
            keyed = [(id(seq), seq.table) for seq, _ in scheduled]
            if path == "decode_graph":
                hidden = self.decode_runner.replay_device(self.dm, keyed, starts, ids)
            else:
                meta, ids_t, pos_t = self.dm.build(keyed, starts, qlens, ids)
                if path == "piecewise":  # the stages read the shared id buffer dm.build filled
                    hidden = self.piecewise.run(T, pos_t, self.pool.tensor, meta)
                else:
                    hidden = self.model(ids_t, pos_t, self.pool.tensor, meta)
        else:
            # the reference's host path (model_runner.py:114-125, 165-197)
            pos, slots, seq_lens = [], [], []
            for (seq, n), start in zip(scheduled, starts):
                pos += range(start, start + n)
                slots += [seq.table[p // bs] * bs + p % bs for p in range(start, start + n)]
                seq_lens.append(start + n)
            tables = [seq.table for seq, _ in scheduled]
            if path == "decode_graph":
                hidden = self.decode_runner.replay_host(ids, pos, slots, tables, seq_lens)
            else:
                meta = build_metadata(self.device, tables, slots, seq_lens, qlens, padded_layout=self.padded_layout)
                pos_t = torch.tensor(pos, dtype=torch.long, device=self.device)
                if path == "piecewise":
                    self.piecewise.ids[:T].copy_(torch.tensor(ids, dtype=torch.long), non_blocking=True)
                    hidden = self.piecewise.run(T, pos_t, self.pool.tensor, meta)
                else:
                    ids_t = torch.tensor(ids, dtype=torch.long, device=self.device)
                    hidden = self.model(ids_t, pos_t, self.pool.tensor, meta)
        self.paths[path] += 1
        for seq, n in scheduled:
            seq.computed += n
        if not sampled:
            return {}
        rows = torch.tensor(last_rows, dtype=torch.long, device=self.device)
        tokens = self.model.logits(hidden.index_select(0, rows)).argmax(dim=-1).tolist()
        for seq, tok in zip(sampled, tokens):
            seq.tokens.append(tok)
        return dict(zip(sampled, tokens))

    # convenience for benchmarks: whole batches in lockstep
    def prefill(self, seqs: list[Sequence]) -> None:
        """Compute the rest of every sequence's prompt, chunked to the token budget per step; the
        step that completes a prompt samples its first token."""
        while any(s.computed < s.prompt_len for s in seqs):
            room, step = self.token_budget, []
            for s in seqs:
                n = min(s.prompt_len - s.computed, room)
                if n > 0:
                    step.append((s, n))
                    room -= n
                if room == 0:
                    break
            self.execute(step)

    def decode(self, seqs: list[Sequence], eager: bool = False) -> list[int]:
        """One token for each sequence (each has exactly one token pending)."""
        got = self.execute([(s, 1) for s in seqs], eager=eager)
        return [got[s] for s in seqs]


class Batcher:
    """Scheduler-free continuous batching: every step spends at most `token_budget` tokens,
    first on the sequences already admitted (a decode token, or the next chunk of a prompt
    still being computed), oldest first, then on newly submitted prompts in arrival order,
    chunked to what the budget leaves. Finished sequences release their blocks."""

    def __init__(self, runner: ModelRunner, token_budget: int | None = None, max_seqs: int = 256):
        self.runner = runner
        self.budget = token_budget or runner.token_budget
        self.max_seqs = max_seqs
        self.admitted: list[Sequence] = []
        self.queue: list[Sequence] = []

    def submit(self, prompt: list[int], max_new_tokens: int) -> Sequence:
        seq = Sequence(list(prompt), max_new_tokens)
        self.queue.append(seq)
        return seq

    @property
    def busy(self) -> bool:
        return bool(self.admitted or self.queue)

    def step(self, eager: bool = False) -> list[Sequence]:
        """Run one step; returns the sequences it finished."""
        room, plan = self.budget, []
        for seq in self.admitted:
            if room == 0:
                break
            n = min(seq.pending, room)
            plan.append((seq, n))
            room -= n
        while self.queue and room > 0 and len(self.admitted) < self.max_seqs:
            seq = self.queue.pop(0)
            self.admitted.append(seq)
            n = min(seq.pending, room)
            plan.append((seq, n))
            room -= n
        if not plan:
            return []
        self.runner.execute(plan, eager=eager)
        done = [s for s in self.admitted if s.finished]
        for s in done:
            self.admitted.remove(s)
            self.runner.release(s)
        return done

    def drain(self, eager: bool = False) -> None:
        while self.busy:
            self.step(eager)


def generate(runner: ModelRunner, prompts: list[list[int]], max_new_tokens: int, eager: bool = False,
             token_budget: int | None = None) -> list[list[int]]:  # fmt: skip
    """Greedy generation of all prompts together through a Batcher; the generated tokens."""
    b = Batcher(runner, token_budget)
    seqs = [b.submit(p, max_new_tokens) for p in prompts]
    b.drain(eager)
    return [s.generated for s in seqs]
