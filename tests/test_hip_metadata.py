"""kvh_prepare_metadata (kvserve_amd.metadata.DeviceMetadata) against the metadata oracle
(oracle/metadata.py): bit-exact int64 tensors over simulated engine runs.

A small engine loop draws blocks from a seeded shuffled pool, runs chunked prefill and decode
steps, shares prefix blocks between sequences (kv_cache.py:109-134), releases sequences and
reuses their pool rows, and replaces a live sequence's table (a preemption). Every step's
device metadata must equal the reference's build_metadata (model_runner.py:165-189) of the
same step, and in graph mode the whole static buffers must equal DecodeGraphRunner.run's
(cuda_graph.py:111-134), including the stale table columns it does not refresh.
"""

from __future__ import annotations

import random

import pytest
import torch

from kvserve_amd import _lib
from kvserve_amd.metadata import DeviceMetadata, MetaBuffers
from oracle import metadata as om

pytestmark = pytest.mark.gpu

BS = 16


class _Seq:
    def __init__(self, tokens: list[int]):
        self.tokens = tokens
        self.table: list[int] = []
        self.done = 0  # tokens computed


class _Engine:
    def __init__(self, seed: int, num_blocks: int = 6000):
        self.rng = random.Random(seed)
        self.free = list(range(num_blocks))
        self.rng.shuffle(self.free)

    def new_seq(self, prompt_len: int, share_from: _Seq | None = None) -> _Seq:
        s = _Seq([self.rng.randrange(128_000) for _ in range(prompt_len)])
        k = 0
        if share_from is not None and len(share_from.table) > 1:
            k = self.rng.randint(1, len(share_from.table) - 1)
            k = min(k, share_from.done // BS, (prompt_len - 1) // BS)
        if k > 0:
            s.table = share_from.table[:k]  # shared physical blocks, already computed
            s.tokens[: k * BS] = share_from.tokens[: k * BS]
            s.done = k * BS
        return s

    def reserve(self, s: _Seq, length: int, spare: int = 0) -> None:
        need = -(-length // BS) + spare - len(s.table)
        for _ in range(max(0, need)):
            s.table.append(self.free.pop())

    def release(self, s: _Seq) -> None:
        self.free.extend(s.table)
        s.table = []


def _expect(batch):
    inp = om.step_inputs([(s.tokens, s.table, start, n) for s, start, n in batch], BS)
    meta = om.build_metadata([s.table for s, _, _ in batch], inp["slots"], inp["seq_lens"], inp["query_lens"])
    return inp, meta


def _check_eager(dm: DeviceMetadata, batch) -> None:
    inp, want = _expect(batch)
    meta, ids, pos = dm.build([(id(s), s.table) for s, _, _ in batch], [b[1] for b in batch],
                              [b[2] for b in batch], inp["input_ids"])  # fmt: skip
    assert meta.slot_mapping.tolist() == want["slot_mapping"]
    assert meta.block_tables.tolist() == want["block_tables"]
    assert meta.seq_lens.tolist() == want["seq_lens"]
    assert meta.query_lens.tolist() == want["query_lens"]
    assert meta.query_start_loc.tolist() == want["query_start_loc"]
    assert (meta.max_seq_len, meta.max_query_len) == (want["max_seq_len"], want["max_query_len"])
    assert pos.tolist() == inp["positions"]
    assert ids.tolist() == inp["input_ids"]


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_engine_run_matches_build_metadata(hip_device, seed):
    eng = _Engine(seed)
    rng = eng.rng
    dm = DeviceMetadata(hip_device, max_seqs=64, max_blocks_per_seq=300, block_size=BS, max_tokens=4096)
    live: list[_Seq] = []
    for step in range(40):
        # admit new sequences (some sharing a prefix with a live one)
        for _ in range(rng.randint(0, 3)):
            if len(live) < 40:
                src = rng.choice(live) if live and rng.random() < 0.4 else None
                live.append(eng.new_seq(rng.randint(1, 1500), share_from=src))
        budget, batch = 2048, []
        for s in live:
            if budget == 0:
                break
            left = len(s.tokens) - s.done
            if left == 0:  # decode: one new token
                s.tokens.append(rng.randrange(128_000))
                left = 1
            n = min(left, budget, rng.choice([1, 7, 64, 512]))
            eng.reserve(s, s.done + n, spare=rng.choice([0, 0, 1]))
            batch.append((s, s.done, n))
            budget -= n
        if not batch:
            continue
        _check_eager(dm, batch)
        for s, start, n in batch:
            s.done = start + n
        # finish some sequences; preempt one (its table is replaced, the key kept)
        for s in list(live):
            if s.done >= len(s.tokens) and rng.random() < 0.15:
                dm.release(id(s))
                eng.release(s)
                live.remove(s)
        if live and step % 9 == 5:
            victim = rng.choice(live)
            eng.release(victim)
            victim.done = 0
    torch.cuda.synchronize()


def test_graph_refresh_matches_decode_graph_runner(hip_device):
    eng = _Engine(7)
    rng = eng.rng
    max_batch, W, scratch = 24, 64, 6000
    dm = DeviceMetadata(hip_device, max_seqs=64, max_blocks_per_seq=W, block_size=BS, max_tokens=256)
    gb = MetaBuffers(hip_device, max_batch, max_batch, W, slot_fill=scratch * BS, table_fill=scratch)
    want = om.graph_buffers(max_batch, W, scratch, BS)
    sizes = [1, 2, 4, 8, 16, 24]
    seqs = [eng.new_seq(rng.randint(1, 600)) for _ in range(max_batch)]
    for s in seqs:
        s.done = len(s.tokens)
    for step in range(30):
        n = rng.randint(1, max_batch)
        batch = []
        for s in rng.sample(seqs, n):
            s.tokens.append(rng.randrange(128_000))
            eng.reserve(s, len(s.tokens))
            batch.append((s, len(s.tokens) - 1, 1))
        size = next(z for z in sizes if z >= n)
        inp = om.step_inputs([(s.tokens, s.table, st, q) for s, st, q in batch], BS)
        width = max(len(s.table) for s, _, _ in batch)
        dm.build([(id(s), s.table) for s, _, _ in batch], [b[1] for b in batch], [1] * n, inp["input_ids"],
                 buffers=gb, pad_seqs=size - n, pad_slot=scratch * BS, table_pad=scratch, width=width)  # fmt: skip
        om.graph_refresh(want, size, inp["input_ids"], inp["positions"], inp["slots"],
                         [s.table for s, _, _ in batch], inp["seq_lens"], scratch, BS)  # fmt: skip
        for s, st, _ in batch:
            s.done = st + 1
        for name in ("input_ids", "positions", "slot_mapping", "seq_lens", "query_lens", "query_start_loc",
                     "block_tables"):  # fmt: skip
            assert getattr(gb, name).tolist() == want[name], (step, name)


def test_single_token_batch_and_resent_table(hip_device):
    dm = DeviceMetadata(hip_device, max_seqs=2, max_blocks_per_seq=4, block_size=BS, max_tokens=8)
    table = [3]
    meta, ids, pos = dm.build([("a", table)], [0], [1], [42])
    assert meta.slot_mapping.tolist() == [48] and ids.tolist() == [42] and pos.tolist() == [0]
    table.append(9)  # appended in place: only column 1 is sent
    meta, _, _ = dm.build([("a", table)], [16], [1])
    assert meta.slot_mapping.tolist() == [144] and meta.block_tables.tolist() == [[3, 9]]
    new_table = [5, 6]  # replaced (a preemption): sent whole
    meta, _, _ = dm.build([("a", new_table)], [17], [1])
    assert meta.slot_mapping.tolist() == [97] and meta.block_tables.tolist() == [[5, 6]]
    dm.release("a")
    meta, _, _ = dm.build([("b", [1]), ("c", [2, 0])], [0, 20], [3, 2], None)  # rows reused
    assert meta.slot_mapping.tolist() == [16, 17, 18, 4, 5]
    assert meta.block_tables.tolist() == [[1, 0], [2, 0]]
    assert meta.query_start_loc.tolist() == [0, 3, 5]
    with pytest.raises(RuntimeError, match="live sequences"):
        dm.build([("d", [1])], [0], [1])
    with pytest.raises(ValueError, match="outside"):
        dm.build([("b", [1])], [10], [7])


def test_device_side_bounds_on_raw_packed_data(hip_device):
    """Packed data the host wrapper would reject: updates outside the pool are skipped and a
    position past a sequence's table gets slot -1; nothing is written out of bounds."""
    dev = hip_device
    lib = _lib.load()
    pool = torch.full((2, 4), 7, dtype=torch.long, device=dev)
    guard = torch.full((64,), -5, dtype=torch.long, device=dev)  # outputs live inside a guarded arena
    slots, posn, sl, qsl = guard[0:8], guard[16:24], guard[32:36], guard[40:44]
    bt = torch.full((3, 4), -9, dtype=torch.long, device=dev)
    packed = torch.tensor([0, 30, 4, 2,  # row 0, positions 30..33, 2 blocks: 32 and 33 are past the table
                           5, 0, 1, 1,  # row 5 does not exist: no table, slot -1
                           0, 1, 11,  # update (0, 1) = 11
                           2, 0, 99, 0, 9, 99, 1, -1, 99],  # updates outside the pool, skipped
                          dtype=torch.int32, device=dev)  # fmt: skip
    st = lib.kvh_prepare_metadata(packed.data_ptr(), 2, 1, 4, 5, pool.data_ptr(), 2, 4, 4, bt.data_ptr(), 4, 3, 0,
                                  slots.data_ptr(), posn.data_ptr(), None, sl.data_ptr(), None, qsl.data_ptr(),
                                  777, BS, torch.cuda.current_stream().cuda_stream)  # fmt: skip
    _lib.check(st, "kvh_prepare_metadata")
    torch.cuda.synchronize()
    assert pool.tolist() == [[7, 11, 7, 7], [7, 7, 7, 7]]
    assert slots.tolist()[:6] == [11 * BS + 14, 11 * BS + 15, -1, -1, -1, 777]
    assert posn.tolist()[:6] == [30, 31, 32, 33, 0, 0]
    assert sl.tolist()[:3] == [34, 1, 1] and qsl.tolist()[:4] == [0, 4, 5, 6]
    assert bt.tolist() == [[7, 11, 0, -9], [0, 0, 0, -9], [0, 0, 0, -9]]
    g = guard.tolist()
    assert g[6:16] == [-5] * 10 and g[24:32] == [-5] * 8 and g[36:40] == [-5] * 4 and g[44:] == [-5] * 20
