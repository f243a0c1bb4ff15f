"""Cascade decode over a shared table prefix (prefix caching: several sequences' block tables
start with the same physical blocks, configs[3] of BASELINE.json): the shared keys are computed
once per group of sequences and merged with each sequence's own keys. The output must match
the oracle as for any other batch (TorchAttention reads every sequence's table on its own,
src/kvserve/attention.py:31-82); the cases vary the group shape (when the batch has more than
16 rows, SG = 64 / (q_len G) sequences per 64-row group over 16-bit caches and 32 / (q_len G)
per 32-row group over E4M3 caches, else 16 / (q_len G) per 16-row group: over 16-bit caches
one group of 16 in g4_b16, two in g4_b23_ragged, one at D = 64 in d64_bs16_b9, 16-row groups
in g1_b5_sg16 and d64_bs32_b2, 4 and 5 members of 16 and 12 rows in g8_q2_sg1 and
g4_q3_rs12, 5 members in g4_b5_partial; over E4M3 caches two 32-row groups in g4_b16, three in
g4_b23_ragged, one of 5 members in g4_b5_partial), where the
sharing stops (a diverging table, the shortest member context), members that do not join
(padding rows, short contexts), E4M3 caches and graph replays whose metadata switches the
cascade on and off.
"""

from __future__ import annotations

import math
import random

import pytest
import torch

from kvserve_amd import HipAttention, last_launch_kernels, workloads
from oracle import fp8, torch_reference
from tests import paged_check as pc

pytestmark = pytest.mark.gpu


def shared_workload(q_lens, ctx_lens, heads, D, BS, shared_blocks, width, seed, diverge=None):
    """Tables = the same `shared_blocks` physical blocks, then unique shuffled blocks. A
    sequence whose table is shorter than the shared run takes only its first blocks of it.
    diverge = (seq, block): that sequence's table holds a private copy's id from that column on."""
    rng = random.Random(seed)
    seq_lens = [q + c for q, c in zip(q_lens, ctx_lens)]
    need = [math.ceil(s / BS) for s in seq_lens]
    pool = shared_blocks + sum(max(0, n - shared_blocks) for n in need) + shared_blocks + 8
    ids = list(range(pool))
    rng.shuffle(ids)
    shared = ids[:shared_blocks]
    i = shared_blocks
    tables = []
    for n in need:
        own = max(0, n - shared_blocks)
        tables.append(shared[: min(n, shared_blocks)] + ids[i : i + own])
        i += own
    if diverge is not None:
        s, col = diverge
        spare = ids[i : i + shared_blocks]
        for j in range(col, min(shared_blocks, len(tables[s]))):
            tables[s][j] = spare[j]
    H, Hkv = heads
    return workloads.Workload("shared", list(q_lens), seq_lens, tables, pool, H, Hkv, D, BS, width=width)


def _check(b, out, tol=pc.TOL_16BIT):
    seqs = [s for s, q in enumerate(b.workload.query_lens) if q > 0]
    err = pc.max_err_vs_oracle(b, out, seqs)
    assert err <= tol, err
    return err


CASES = {
    # name: (q_lens, ctx_lens, heads, D, BS, shared_blocks, width)
    "g4_b16": ([1] * 16, [random.Random(1).randint(1700, 3000) for _ in range(16)], (32, 8), 128, 16, 100, 600),
    "g1_b5_sg16": ([1] * 5, [900, 1200, 2000, 1100, 5000], (16, 16), 128, 16, 50, 600),
    "d64_bs32_b2": ([1, 1], [700, 1500], (32, 8), 64, 32, 20, 300),
    "d64_bs16_b9": ([1] * 9, [600 + 173 * i for i in range(9)], (32, 8), 64, 16, 36, 600),
    "g8_q2_sg1": ([2, 1, 2, 2, 1, 2, 1, 1, 2], [1000 + 97 * i for i in range(9)], (32, 4), 128, 16, 40, 600),
    "g4_q3_rs12": ([3, 1, 2, 3, 3, 1], [800, 1900, 600, 1500, 1000, 3000], (32, 8), 128, 16, 30, 600),
    "g4_b23_ragged": ([1] * 23, [300 + 211 * i for i in range(23)], (32, 8), 128, 16, 18, 800),
    "g4_b5_partial": ([1] * 5, [900, 1700, 2500, 1200, 3100], (32, 8), 128, 16, 40, 600),
}


@pytest.mark.parametrize("name", list(CASES))
def test_shared_prefix_matches_oracle(hip_device, name):
    q, c, heads, D, BS, shared, width = CASES[name]
    w = shared_workload(q, c, heads, D, BS, shared, width, seed=7)
    b = workloads.materialize(w, torch.bfloat16, hip_device, seed=7)
    out = pc.attend(b)
    kinds = last_launch_kernels()
    assert kinds[0] == "share", kinds
    err = _check(b, out)
    print(f"{name}: {kinds} err {err:.3e}")


@pytest.mark.parametrize("name", ["g4_b16", "g1_b5_sg16", "g4_b23_ragged", "d64_bs16_b9"])
def test_shared_prefix_fp16(hip_device, name):
    """The fp16 instances of the cascade paths: one and two 64-row groups, 16-row groups, and
    64-row groups at D = 64."""
    q, c, heads, D, BS, shared, width = CASES[name]
    w = shared_workload(q, c, heads, D, BS, shared, width, seed=9)
    b = workloads.materialize(w, torch.float16, hip_device, seed=9)
    out = pc.attend(b)
    assert last_launch_kernels()[0] == "share", last_launch_kernels()
    _check(b, out)


def test_members_numbered_across_scan_windows(hip_device):
    """150 sequences (three 64-sequence scan windows of the decode kernel, several sequences
    per thread in the share kernel), non-members spread over all windows: each member's group
    and row in the prefix tiles come from its number among the members, counted across windows."""
    rng = random.Random(21)
    q = [1] * 150
    ctx = [rng.randint(300, 2500) if i % 7 else rng.randint(20, 250) for i in range(150)]
    w = shared_workload(q, ctx, (32, 8), 128, 16, 18, 600, seed=21)
    b = workloads.materialize(w, torch.bfloat16, hip_device, seed=21)
    out = pc.attend(b)
    assert last_launch_kernels()[0] == "share"
    seqs = list(range(0, 150, 3)) + [149]
    err = pc.max_err_vs_oracle(b, out, seqs)
    assert err <= pc.TOL_16BIT, err


def test_padding_rows_and_short_contexts_stay_out(hip_device):
    """Graph padding rows (seq_len 1, tables of one scratch block) and sequences with under
    256 context tokens are not members; the members still share their prefix."""
    q = [1] * 10
    ctx = [2000, 0, 1500, 100, 1800, 0, 2500, 255, 256, 3000]
    w = shared_workload(q, ctx, (32, 8), 128, 16, 16, 600, seed=3)
    used = {x for t in w.tables for x in t}
    scratch = next(x for x in range(w.num_blocks) if x not in used)
    for s in (1, 5):  # padding rows: one token in the scratch block
        w.tables[s] = [scratch]
    b = workloads.materialize(w, torch.bfloat16, hip_device, seed=3)
    out = pc.attend(b)
    assert last_launch_kernels()[0] == "share"
    _check(b, out)


@pytest.mark.parametrize("col", [3, 40])
def test_diverging_table(hip_device, col):
    """One member's table leaves the shared run at column col: the shared length stops
    there (col 3: below 256 tokens, so no prefix segments at all)."""
    q = [1] * 8
    ctx = [1000 + 300 * i for i in range(8)]
    w = shared_workload(q, ctx, (32, 8), 128, 16, 60, 600, seed=col, diverge=(5, col))
    b = workloads.materialize(w, torch.bfloat16, hip_device, seed=col)
    out = pc.attend(b)
    _check(b, out)


def test_shortest_member_limits_the_shared_length(hip_device):
    """A member whose whole table lies inside the shared run (its new token lands in a shared
    block, read by every other sequence as part of its context)."""
    q = [1] * 6
    ctx = [3000, 700, 2600, 4000, 1200, 2200]  # 700 < 100 blocks x 16
    w = shared_workload(q, ctx, (32, 8), 128, 16, 100, 600, seed=11)
    b = workloads.materialize(w, torch.bfloat16, hip_device, seed=11)
    out = pc.attend(b)
    _check(b, out)


@pytest.mark.parametrize("k_scale,v_scale", [(1.0, 1.0), (0.5, 2.0)])
def test_shared_prefix_fp8(hip_device, k_scale, v_scale):
    _fp8_case(hip_device, "g4_b16", k_scale, v_scale, seed=5)


@pytest.mark.parametrize(
    "name", ["g4_b23_ragged", "g4_q3_rs12", "g8_q2_sg1", "d64_bs16_b9", "g4_b5_partial", "g1_b5_sg16", "d64_bs32_b2"]
)
def test_shared_prefix_fp8_groups(hip_device, name):
    """E4M3 caches stack a batch of more than 16 rows into 32-row prefix groups (two tiles per
    wave): three groups of 8 members with a ragged last one, 2 members of 12 rows, 2 of 16
    rows with padding rows between mixed query lengths, D = 64, one group of 5 members (20 of
    its 32 rows); batches of at most 16 rows keep one 16-row group."""
    _fp8_case(hip_device, name, 0.5, 2.0, seed=13)


def _fp8_case(hip_device, name, k_scale, v_scale, seed):
    q, c, heads, D, BS, shared, width = CASES[name]
    w = shared_workload(q, c, heads, D, BS, shared, width, seed=seed)
    b = workloads.materialize(w, torch.bfloat16, hip_device, seed=seed)
    kc = fp8.quantize(b.k_cache, k_scale).to(hip_device)
    vc = fp8.quantize(b.v_cache, v_scale).to(hip_device)
    HipAttention.write_kv(kc, vc, b.k_new, b.v_new, b.meta.slot_mapping, k_scale=k_scale, v_scale=v_scale)
    out = HipAttention.forward(b.q, kc, vc, b.meta, w.scale, k_scale=k_scale, v_scale=v_scale)
    assert last_launch_kernels()[0] == "share"
    m = b.meta
    ref = torch_reference.forward(
        b.q.float().cpu(), fp8.dequantize(kc.cpu(), k_scale), fp8.dequantize(vc.cpu(), v_scale),
        m.block_tables.cpu(), m.seq_lens.cpu(), m.query_lens.cpu(), w.scale,
    )  # fmt: skip
    err = (out.float().cpu() - ref).abs().max().item()
    assert err <= pc.TOL_16BIT, err


@pytest.mark.parametrize("fp8_cache", [False, True], ids=["bf16", "e4m3"])
def test_graph_replays_switch_the_cascade(hip_device, fp8_cache):
    """One captured forward replayed over metadata edited in place: shared tables (prefix
    segments: one 64-row group over bf16 caches, two 32-row groups over E4M3 caches), then one
    table diverging at column 0 (no sharing, plain records), then shared again with other
    lengths; every replay equals the eager call on the same metadata."""
    q, c, heads, D, BS, shared, width = CASES["g4_b16"]
    w = shared_workload(q, c, heads, D, BS, shared, width, seed=9)
    b = workloads.materialize(w, torch.bfloat16, hip_device, seed=9)
    kw = {"k_scale": 0.5, "v_scale": 2.0} if fp8_cache else {}
    if fp8_cache:
        b.k_cache = fp8.quantize(b.k_cache, kw["k_scale"]).to(hip_device)
        b.v_cache = fp8.quantize(b.v_cache, kw["v_scale"]).to(hip_device)
    HipAttention.write_kv(b.k_cache, b.v_cache, b.k_new, b.v_new, b.meta.slot_mapping, **kw)
    m = b.meta
    out = torch.empty_like(b.q)

    def fwd(**extra):
        return HipAttention.forward(b.q, b.k_cache, b.v_cache, m, w.scale, **kw, **extra)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fwd(out=out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fwd(out=out)

    bt0 = m.block_tables.clone()
    sl0 = m.seq_lens.clone()
    edits = [
        lambda: None,
        lambda: m.block_tables[3, 0].copy_(bt0[3, shared + 1]),  # seq 3 diverges at column 0
        lambda: (m.block_tables.copy_(bt0), m.seq_lens.copy_(sl0 - torch.arange(16, device=sl0.device) * 7)),
    ]
    for i, edit in enumerate(edits):
        edit()
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        torch.randn(1 << 20, device=hip_device).sum()  # eager work between replays
        eager = fwd()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), eager.view(torch.int16)), i
    # the last state against the oracle (seq_lens shortened: fresh workload view of it)
    w.seq_lens = m.seq_lens.tolist()
    if not fp8_cache:
        _check(b, got)
        return
    ref = torch_reference.forward(
        b.q.float().cpu(), fp8.dequantize(b.k_cache.cpu(), kw["k_scale"]), fp8.dequantize(b.v_cache.cpu(), kw["v_scale"]),
        m.block_tables.cpu(), m.seq_lens.cpu(), m.query_lens.cpu(), w.scale,
    )  # fmt: skip
    assert (got.float().cpu() - ref).abs().max().item() <= pc.TOL_16BIT
