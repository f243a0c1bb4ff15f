"""Restatement of the reference's per-step attention inputs. TEST INFRASTRUCTURE ONLY.

The checker for kvh_prepare_metadata / kvserve_amd.metadata.DeviceMetadata. Plain Python
lists, following the reference step by step:
  slot / slots     KVCacheManager.slot and .slots               (src/kvserve/kv_cache.py:155-169)
  step_inputs      ModelRunner.execute's per-sequence loop      (src/kvserve/model_runner.py:114-125)
  build_metadata   build_metadata, Triton layout (no padding)    (src/kvserve/model_runner.py:165-189)
  graph_refresh    DecodeGraphRunner.__init__ buffers and .run   (src/kvserve/cuda_graph.py:54-62, 111-134)
"""

from __future__ import annotations


def slot(table: list[int], position: int, block_size: int) -> int:
    """kv_cache.py:155-157."""
    return table[position // block_size] * block_size + position % block_size


def slots(table: list[int], start: int, n: int, block_size: int) -> list[int]:
    """kv_cache.py:159-169: one run per block instead of per token."""
    out: list[int] = []
    pos, end = start, start + n
    while pos < end:
        block_end = min(end, (pos // block_size + 1) * block_size)
        base = table[pos // block_size] * block_size - (pos // block_size) * block_size
        out.extend(range(base + pos, base + block_end))
        pos = block_end
    return out


def step_inputs(batch: list[tuple[list[int], list[int], int, int]], block_size: int) -> dict[str, list]:
    """model_runner.py:114-125 for a batch of (token_ids, block_table, start, n)."""
    input_ids, positions, slot_mapping, seq_lens, query_lens = [], [], [], [], []
    for tokens, table, start, n in batch:
        input_ids += tokens[start : start + n]
        positions += range(start, start + n)
        slot_mapping += slots(table, start, n, block_size)
        seq_lens.append(start + n)
        query_lens.append(n)
    return dict(input_ids=input_ids, positions=positions, slots=slot_mapping, seq_lens=seq_lens,
                query_lens=query_lens)  # fmt: skip


def build_metadata(tables: list[list[int]], slot_mapping: list[int], seq_lens: list[int],
                   query_lens: list[int]) -> dict[str, object]:  # fmt: skip
    """model_runner.py:165-189 (the layout the Triton backend gets: no q_gather / q_valid)."""
    max_blocks = max(len(t) for t in tables)
    padded = [t + [0] * (max_blocks - len(t)) for t in tables]
    query_start_loc = [0]
    for n in query_lens:
        query_start_loc.append(query_start_loc[-1] + n)
    return dict(slot_mapping=list(slot_mapping), block_tables=padded, seq_lens=list(seq_lens),
                query_lens=list(query_lens), query_start_loc=query_start_loc, max_seq_len=max(seq_lens),
                max_query_len=max(query_lens))  # fmt: skip


def graph_buffers(max_batch: int, max_blocks_per_seq: int, scratch_block: int, block_size: int) -> dict[str, list]:
    """The static buffers as DecodeGraphRunner.__init__ fills them (cuda_graph.py:54-62)."""
    return dict(
        input_ids=[0] * max_batch,
        positions=[0] * max_batch,
        slot_mapping=[scratch_block * block_size] * max_batch,
        block_tables=[[scratch_block] * max_blocks_per_seq for _ in range(max_batch)],
        seq_lens=[1] * max_batch,
        query_lens=[1] * max_batch,
        query_start_loc=list(range(max_batch + 1)),
    )


def graph_refresh(buf: dict[str, list], size: int, input_ids: list[int], positions: list[int],
                  slot_mapping: list[int], tables: list[list[int]], seq_lens: list[int], scratch_block: int,
                  block_size: int) -> None:  # fmt: skip
    """DecodeGraphRunner.run's copies into the static buffers for padded batch `size`
    (cuda_graph.py:124-134), in place: pad rows get token 0, position 0, the scratch slot,
    seq_len 1; table rows are refreshed only in their first `width` columns."""
    pad = size - len(input_ids)
    scratch_slot = scratch_block * block_size
    buf["input_ids"][:size] = input_ids + [0] * pad
    buf["positions"][:size] = positions + [0] * pad
    buf["slot_mapping"][:size] = slot_mapping + [scratch_slot] * pad
    buf["seq_lens"][:size] = seq_lens + [1] * pad
    width = max(len(t) for t in tables)
    rows = [t + [scratch_block] * (width - len(t)) for t in tables]
    rows += [[scratch_block] * width] * pad
    for r, row in enumerate(rows):
        buf["block_tables"][r][:width] = row
