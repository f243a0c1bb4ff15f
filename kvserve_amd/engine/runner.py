"""KV pool, step execution and HIP-graph decode replay for the engine harness.

Follows the reference's ModelRunner (src/kvserve/model_runner.py:19-156) and
DecodeGraphRunner (src/kvserve/cuda_graph.py:28-137), without its scheduler: the caller
hands in sequences and the runner lays out the flat token batch, the slots
(kv_cache.py:155-169) and the metadata (model_runner.py:165-197), runs the model and
picks greedy tokens.

The pool is [layers, 2, num_blocks + 1, block_size, kv_heads, head_dim]; the extra block
is scratch space for graph padding rows, outside what sequences are given.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from kvserve_amd.attention import AttentionMetadata, build_metadata
from kvserve_amd.metadata import DeviceMetadata, MetaBuffers


@dataclass
class Sequence:
    token_ids: list[int]
    block_table: list[int] = field(default_factory=list)
    num_computed: int = 0  # tokens whose K/V are in the pool
    prompt_len: int = -1  # set from token_ids when left at -1

    def __post_init__(self) -> None:
        if self.prompt_len < 0:
            self.prompt_len = len(self.token_ids)

    @property
    def num_tokens(self) -> int:
        return len(self.token_ids)


def capture_sizes(max_batch: int) -> list[int]:
    """Decode-graph buckets: 1, 2, 4, 8, then every 16 (cuda_graph.py:28-33)."""
    sizes = [s for s in (1, 2, 4, 8) if s <= max_batch]
    sizes += list(range(16, max_batch + 1, 16))
    if sizes[-1] != max_batch:
        sizes.append(max_batch)
    return sizes


class DecodeGraphRunner:
    """One HIP graph per padded decode batch size, replayed on static input buffers.

    Padding rows write their K/V to the scratch block's first slot, read a one-token
    context from the scratch block and are dropped from the output. The attention call
    inside the graph never reads max_seq_len (the graph's metadata carries 1), and only the
    first ceil(seq_len / block_size) table columns of a row are refreshed per step
    (cuda_graph.py:111-137).
    """

    def __init__(self, model, kv_caches: torch.Tensor, scratch_block: int, block_size: int, max_batch: int,
                 max_blocks_per_seq: int):  # fmt: skip
        self.model = model
        self.kv_caches = kv_caches
        self.scratch_block = scratch_block
        self.scratch_slot = scratch_block * block_size
        self.sizes = capture_sizes(max_batch)
        self.max_batch = self.sizes[-1]
        b = self.max_batch
        # static inputs, filled as cuda_graph.py:54-62 fills them
        self.buf = MetaBuffers(kv_caches.device, b, b, max_blocks_per_seq, slot_fill=self.scratch_slot,
                               table_fill=scratch_block)  # fmt: skip
        self.input_ids, self.positions = self.buf.input_ids, self.buf.positions
        self.slot_mapping, self.block_tables = self.buf.slot_mapping, self.buf.block_tables
        self.seq_lens, self.query_lens = self.buf.seq_lens, self.buf.query_lens
        self.query_start_loc = self.buf.query_start_loc
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self.outputs: dict[int, torch.Tensor] = {}

    def _metadata(self, n: int) -> AttentionMetadata:
        return AttentionMetadata(
            slot_mapping=self.slot_mapping[:n],
            block_tables=self.block_tables[:n],
            seq_lens=self.seq_lens[:n],
            query_lens=self.query_lens[:n],
            query_start_loc=self.query_start_loc[: n + 1],
            max_seq_len=1,  # not read by the HIP backend
            max_query_len=1,
        )

    @torch.inference_mode()
    def capture(self) -> None:
        """All buckets, largest first, sharing one memory pool; warm-up runs on a side stream
        touch only the scratch block."""
        pool = None
        side = torch.cuda.Stream()
        for n in reversed(self.sizes):
            args = (self.input_ids[:n], self.positions[:n], self.kv_caches, self._metadata(n))
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(2):
                    self.model(*args)
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=pool):
                self.outputs[n] = self.model(*args)
            pool = g.pool()
            self.graphs[n] = g
        torch.cuda.synchronize()

    def bucket(self, n: int) -> int | None:
        return next((s for s in self.sizes if s >= n), None)

    @torch.inference_mode()
    def run(self, input_ids: list[int], positions: list[int], slots: list[int], block_tables: list[list[int]],
            seq_lens: list[int]) -> torch.Tensor:  # fmt: skip
        """Replay for a uniform decode batch; hidden states [n, hidden]."""
        n = len(input_ids)
        size = self.bucket(n)
        if size is None:
            raise ValueError(f"decode batch {n} exceeds the largest captured graph ({self.max_batch})")
        pad = size - n
        self.input_ids[:size].copy_(torch.tensor(input_ids + [0] * pad), non_blocking=True)
        self.positions[:size].copy_(torch.tensor(positions + [0] * pad), non_blocking=True)
        self.slot_mapping[:size].copy_(torch.tensor(slots + [self.scratch_slot] * pad), non_blocking=True)
        self.seq_lens[:size].copy_(torch.tensor(seq_lens + [1] * pad), non_blocking=True)
        width = max(len(t) for t in block_tables)
        rows = [t + [self.scratch_block] * (width - len(t)) for t in block_tables]
        rows += [[self.scratch_block] * width] * pad
        self.block_tables[:size, :width].copy_(torch.tensor(rows), non_blocking=True)
        self.graphs[size].replay()
        return self.outputs[size][:n]

    @torch.inference_mode()
    def run_device(self, dm: DeviceMetadata, seqs: list[tuple[object, list[int]]], starts: list[int],
                   input_ids: list[int]) -> torch.Tensor:  # fmt: skip
        """`run` with the static buffers refreshed on the device from resident block tables
        (same contents: scratch padding, the first `width` table columns)."""
        n = len(input_ids)
        size = self.bucket(n)
        if size is None:
            raise ValueError(f"decode batch {n} exceeds the largest captured graph ({self.max_batch})")
        width = max(len(t) for _, t in seqs)
        dm.build(seqs, starts, [1] * n, input_ids, buffers=self.buf, pad_seqs=size - n, pad_slot=self.scratch_slot,
                 table_pad=self.scratch_block, width=width)  # fmt: skip
        self.graphs[size].replay()
        return self.outputs[size][:n]


class ModelRunner:
    """Owns the model and the paged KV pool; runs prefill and decode steps with greedy
    sampling. `use_graphs` replays decode steps from HIP graphs (the backend must be
    graph-capturable)."""

    def __init__(self, model, num_blocks: int, block_size: int = 16, max_model_len: int = 4096,
                 use_graphs: bool = True, max_graph_batch: int = 128, prefill_token_budget: int = 2048,
                 device_metadata: bool | None = None, max_seqs: int = 1024,
                 kv_cache_dtype: torch.dtype | None = None):  # fmt: skip
        cfg = model.cfg
        p = next(model.parameters())
        self.model = model
        self.device, self.dtype = p.device, p.dtype
        self.block_size = block_size
        self.max_model_len = max_model_len
        self.num_blocks = num_blocks
        self.scratch_block = num_blocks
        # kv_cache_dtype: the model's dtype, or torch.float8_e4m3fn (E4M3 with each layer's
        # k_scale / v_scale; HIP backend only)
        self.kv_dtype = self.dtype if kv_cache_dtype is None else kv_cache_dtype
        shape = (cfg.num_layers, 2, num_blocks + 1, block_size, cfg.num_kv_heads, cfg.head_dim)
        if self.kv_dtype == torch.float8_e4m3fn:  # zero bytes, viewed as E4M3 (+0)
            self.kv_caches = torch.zeros(shape, dtype=torch.uint8, device=self.device).view(self.kv_dtype)
        else:
            self.kv_caches = torch.zeros(shape, dtype=self.kv_dtype, device=self.device)
        self.free_blocks = list(range(num_blocks - 1, -1, -1))
        self.prefill_token_budget = prefill_token_budget
        backend = model.layers[0].self_attn.backend
        self.padded_layout = getattr(backend, "needs_padded_layout", True)
        # step inputs from block tables kept on the device (kvh_prepare_metadata) unless the
        # backend needs the torch reference's padded layout, which only the host builds
        if device_metadata is None:
            device_metadata = not self.padded_layout and self.device.type == "cuda"
        if device_metadata and self.padded_layout:
            raise ValueError("device metadata does not build the padded layout")
        self.dm = None
        if device_metadata:
            self.dm = DeviceMetadata(self.device, max_seqs, -(-max_model_len // block_size), block_size,
                                     max(prefill_token_budget, max_graph_batch))  # fmt: skip
        self.graphs: DecodeGraphRunner | None = None
        if use_graphs:
            if not getattr(backend, "graph_capturable", False):
                raise ValueError(f"backend {getattr(backend, 'name', backend)} cannot be captured in a graph")
            self.graphs = DecodeGraphRunner(model, self.kv_caches, self.scratch_block, block_size, max_graph_batch,
                                            -(-max_model_len // block_size))  # fmt: skip
            self.graphs.capture()
        self.steps = {"decode_graph": 0, "eager": 0}

    # -- pool ----------------------------------------------------------------------------------
    def _reserve(self, seq: Sequence, length: int) -> None:
        need = -(-length // self.block_size) - len(seq.block_table)
        if need > len(self.free_blocks):
            raise RuntimeError("KV pool exhausted")
        for _ in range(max(0, need)):
            seq.block_table.append(self.free_blocks.pop())

    def release(self, seq: Sequence) -> None:
        self.free_blocks.extend(reversed(seq.block_table))
        seq.block_table = []
        if self.dm is not None:
            self.dm.release(id(seq))

    def slots(self, seq: Sequence, start: int, n: int) -> list[int]:
        """Slots of positions start .. start + n - 1 (kv_cache.py:155-169)."""
        bs, t = self.block_size, seq.block_table
        return [t[pos // bs] * bs + pos % bs for pos in range(start, start + n)]

    # -- steps -----------------------------------------------------------------------------------
    @torch.inference_mode()
    def step(self, scheduled: list[tuple[Sequence, int]], force_eager: bool = False) -> dict[int, int]:
        """One forward over `scheduled` (sequence, tokens to compute). Sequences whose context is
        complete after the step get a greedy token, appended to them; returns {index: token}."""
        ids, starts, query_lens, tables, rows, done = [], [], [], [], [], []
        for k, (seq, n) in enumerate(scheduled):
            start = seq.num_computed
            if start + n > self.max_model_len:
                raise ValueError("sequence exceeds max_model_len")
            self._reserve(seq, start + n)
            ids += seq.token_ids[start : start + n]
            starts.append(start)
            query_lens.append(n)
            tables.append(seq.block_table)
            if start + n == seq.num_tokens:
                rows.append(len(ids) - 1)
                done.append(k)
        decode = max(query_lens) == 1
        use_graph = self.graphs is not None and decode and not force_eager and len(ids) <= self.graphs.max_batch
        if self.dm is not None:
            keyed = [(id(seq), seq.block_table) for seq, _ in scheduled]
            if use_graph:
                hidden = self.graphs.run_device(self.dm, keyed, starts, ids)
            else:
                meta, ids_t, pos_t = self.dm.build(keyed, starts, query_lens, ids)
                hidden = self.model(ids_t, pos_t, self.kv_caches, meta)
        else:
            # the reference's host path (model_runner.py:114-125, 165-197; cuda_graph.py:111-134)
            pos, slots, seq_lens = [], [], []
            for (seq, n), start in zip(scheduled, starts):
                pos += range(start, start + n)
                slots += self.slots(seq, start, n)
                seq_lens.append(start + n)
            if use_graph:
                hidden = self.graphs.run(ids, pos, slots, tables, seq_lens)
            else:
                meta = build_metadata(self.device, tables, slots, seq_lens, query_lens,
                                      padded_layout=self.padded_layout)  # fmt: skip
                hidden = self.model(torch.tensor(ids, device=self.device), torch.tensor(pos, device=self.device),
                                    self.kv_caches, meta)  # fmt: skip
        self.steps["decode_graph" if use_graph else "eager"] += 1
        for seq, n in scheduled:
            seq.num_computed += n
        if not rows:
            return {}
        logits = self.model.compute_logits(hidden[torch.tensor(rows, device=self.device)])
        tokens = logits.argmax(dim=-1).tolist()
        out = {}
        for k, tok in zip(done, tokens):
            scheduled[k][0].token_ids.append(tok)
            out[k] = tok
        return out

    def prefill(self, seqs: list[Sequence]) -> None:
        """Compute every prompt in chunks of at most the token budget per step (chunked
        prefill); the last chunk of each prompt yields its first generated token."""
        while True:
            budget, sched = self.prefill_token_budget, []
            for seq in seqs:
                n = min(seq.prompt_len - seq.num_computed, budget)
                if n > 0:
                    sched.append((seq, n))
                    budget -= n
                if budget == 0:
                    break
            if not sched:
                return
            self.step(sched)

    def decode(self, seqs: list[Sequence], force_eager: bool = False) -> list[int]:
        """One token for every sequence (each has exactly one uncomputed token)."""
        res = self.step([(s, 1) for s in seqs], force_eager=force_eager)
        return [res[k] for k in range(len(seqs))]

    def generate(self, prompts: list[list[int]], max_new_tokens: int, force_eager: bool = False) -> list[list[int]]:
        """Greedy generation; returns the generated tokens of each prompt."""
        seqs = [Sequence(list(p)) for p in prompts]
        self.prefill(seqs)
        for _ in range(max_new_tokens - 1):
            self.decode(seqs, force_eager=force_eager)
        out = [s.token_ids[len(p):] for s, p in zip(seqs, prompts)]
        for s in seqs:
            self.release(s)
        return out
