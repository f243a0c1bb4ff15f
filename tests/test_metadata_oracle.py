"""The metadata oracle (oracle/metadata.py) pinned on the CPU, and the argument checks of
kvh_prepare_metadata (they return before any HIP call, so they run without a GPU).

Pins: the reference's own known answers for the slot formula (tests/test_kv_cache.py:50-63:
per-token slots of a two-block table, and `slots` == per-token `slot` on a reversed table at
its seven (start, n) cases); the decomposition slot = (table[p // BS], p % BS) on random tables;
query_start_loc as prefix sums and the 0 / scratch padding rules of build_metadata
(model_runner.py:175-180) and DecodeGraphRunner.run (cuda_graph.py:124-134), including the
stale columns the graph refresh leaves past `width`.
"""

from __future__ import annotations

import random

import pytest

from kvserve_amd import _lib
from oracle import metadata as om

E_NULL, E_SHAPE, E_ALIGN = -1, -2, -4


def test_slot_known_answer():
    # kv_cache.py:155-157 on a 6-token sequence over two blocks of 4 (test_kv_cache.py:50-55)
    b0, b1 = 5, 2
    assert [om.slot([b0, b1], p, 4) for p in range(6)] == [20, 21, 22, 23, 8, 9]


@pytest.mark.parametrize(("start", "n"), [(0, 1), (0, 4), (3, 1), (3, 6), (2, 13), (8, 4), (5, 0)])
def test_slots_matches_per_token_slot_on_reversed_table(start, n):
    table = list(range(5))[::-1]  # 20 tokens in 5 blocks of 4, reversed (test_kv_cache.py:57-63)
    assert om.slots(table, start, n, 4) == [om.slot(table, p, 4) for p in range(start, start + n)]


def test_slot_decomposes_into_block_and_offset():
    rng = random.Random(0)
    for bs in (1, 4, 16, 32):
        table = rng.sample(range(10_000), 40)
        got = om.slots(table, 3, 40 * bs - 3, bs)
        assert len(set(got)) == len(got)  # distinct blocks give distinct slots
        for i, s in enumerate(got):
            p = 3 + i
            assert divmod(s, bs) == (table[p // bs], p % bs)


def test_step_inputs_and_build_metadata_layout():
    rng = random.Random(1)
    batch = []
    for _ in range(9):
        n_tok = rng.randint(1, 200)
        start = rng.randint(0, n_tok - 1)
        n = rng.randint(1, n_tok - start)
        table = rng.sample(range(1000), -(-n_tok // 16) + rng.randint(0, 2))  # may hold spare blocks
        batch.append((list(range(n_tok)), table, start, n))
    inp = om.step_inputs(batch, 16)
    meta = om.build_metadata([b[1] for b in batch], inp["slots"], inp["seq_lens"], inp["query_lens"])
    qsl = meta["query_start_loc"]
    assert qsl[0] == 0 and len(qsl) == len(batch) + 1
    width = max(len(b[1]) for b in batch)
    for i, (tokens, table, start, n) in enumerate(batch):
        assert qsl[i + 1] - qsl[i] == n
        assert meta["block_tables"][i] == table + [0] * (width - len(table))
        assert meta["seq_lens"][i] == start + n
        assert inp["positions"][qsl[i] : qsl[i + 1]] == list(range(start, start + n))
        assert inp["input_ids"][qsl[i] : qsl[i + 1]] == tokens[start : start + n]
    assert meta["max_seq_len"] == max(b[2] + b[3] for b in batch)
    assert meta["max_query_len"] == max(b[3] for b in batch)


def test_graph_refresh_pads_and_keeps_stale_columns():
    buf = om.graph_buffers(8, 6, scratch_block=99, block_size=4)
    om.graph_refresh(buf, 4, [7, 8], [5, 9], [41, 13], [[10, 11], [3, 2, 1, 0, 4, 6]], [6, 10], 99, 4)
    assert buf["input_ids"][:4] == [7, 8, 0, 0] and buf["positions"][:4] == [5, 9, 0, 0]
    assert buf["slot_mapping"] == [41, 13, 396, 396] + [396] * 4
    assert buf["seq_lens"][:4] == [6, 10, 1, 1]
    assert buf["block_tables"][0] == [10, 11, 99, 99, 99, 99]
    assert buf["block_tables"][2] == [99] * 6
    # a narrower refresh leaves the columns past its width as they were
    om.graph_refresh(buf, 2, [1], [0], [40], [[10]], [1], 99, 4)
    assert buf["block_tables"][1] == [99, 2, 1, 0, 4, 6]
    assert buf["query_start_loc"] == list(range(9)) and buf["query_lens"] == [1] * 8


# -- kvh_prepare_metadata argument checks (no HIP call is made) ----------------------------------
@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def _meta_args(**over):
    a = dict(packed=0x1000, B=4, P=0, U=0, T=4, pool=0x2000, pool_rows=16, pool_rs=64, pool_w=64, bt=0x3000,
             bt_rs=64, bt_w=8, bt_pad=0, slots=0x4000, pos=0x5000, ids=None, sl=0x6000, ql=0x7000, qsl=0x8000,
             pad_slot=-1, BS=16, stream=None)  # fmt: skip
    a.update(over)
    return a


def _call_meta(lib, a):
    return lib.kvh_prepare_metadata(
        a["packed"], a["B"], a["P"], a["U"], a["T"], a["pool"], a["pool_rows"], a["pool_rs"], a["pool_w"], a["bt"],
        a["bt_rs"], a["bt_w"], a["bt_pad"], a["slots"], a["pos"], a["ids"], a["sl"], a["ql"], a["qsl"],
        a["pad_slot"], a["BS"], a["stream"],
    )  # fmt: skip


@pytest.mark.parametrize(
    "over,status",
    [
        (dict(B=0, P=0), E_SHAPE),
        (dict(B=-1), E_SHAPE),
        (dict(U=-1), E_SHAPE),
        (dict(T=-1), E_SHAPE),
        (dict(T=2**31), E_SHAPE),
        (dict(pool_rows=0), E_SHAPE),
        (dict(pool_rs=32), E_SHAPE),  # row stride below the width
        (dict(BS=0), E_SHAPE),
        (dict(bt_rs=4), E_SHAPE),  # row stride below bt_width
        (dict(bt=None), E_NULL),
        (dict(pool=None), E_NULL),
        (dict(slots=None), E_NULL),
        (dict(sl=None), E_NULL),
        (dict(qsl=None), E_NULL),
        (dict(packed=None), E_NULL),
        (dict(packed=0x1002), E_ALIGN),
        (dict(slots=0x4004), E_ALIGN),
    ],
)  # fmt: skip
def test_prepare_metadata_rejects_bad_arguments(lib, over, status):
    assert _call_meta(lib, _meta_args(**over)) == status


def test_prepare_metadata_optional_outputs_do_not_excuse_required_ones(lib):
    # a pad-only batch needs no packed data and positions / ids / query_lens may be null, but
    # slot_mapping may not
    assert _call_meta(lib, _meta_args(bt=None, bt_w=0, B=0, P=1, T=0, packed=None, ql=None, pos=None, ids=None,
                                      slots=None)) == E_NULL  # fmt: skip
