"""HIP-graph capture of the backend, as the reference's DecodeGraphRunner uses it (GPU).

Static buffers, scratch block and padding follow src/kvserve/cuda_graph.py:54-76 and
:111-137: one graph per bucket captures write_kv + forward with max_seq_len = 1, the
batch is padded with the scratch slot / seq_len 1 / scratch block, and only the first
`width` table columns are refreshed before each replay. Every replay is checked against
an eager call on the same inputs (bitwise) and against the fp64 oracle, with eager work
and synchronisations between replays.
"""

import random

import pytest
import torch

from kvserve_amd import HipAttention
from kvserve_amd.attention import AttentionMetadata
from kvserve_amd.workloads import PagedBatch, Workload
from tests import paged_check as pc

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
def test_decode_graph_replays_match_eager(hip_device, dtype):
    dev = hip_device
    H, Hkv, D, BS = 32, 8, 128, 16
    NB, bucket, max_blocks = 1500, 8, 256  # pool + 1 scratch block, width = max_model_len / BS
    scratch_block = NB
    scratch_slot = scratch_block * BS
    gen = torch.Generator(device=dev).manual_seed(0)
    k_cache = torch.randn(NB + 1, BS, Hkv, D, generator=gen, device=dev).to(dtype)
    v_cache = torch.randn(NB + 1, BS, Hkv, D, generator=gen, device=dev).to(dtype)

    q = torch.zeros(bucket, H, D, device=dev, dtype=dtype)
    k = torch.zeros(bucket, Hkv, D, device=dev, dtype=dtype)
    v = torch.zeros(bucket, Hkv, D, device=dev, dtype=dtype)
    slot_mapping = torch.full((bucket,), scratch_slot, dtype=torch.long, device=dev)
    block_tables = torch.full((bucket, max_blocks), scratch_block, dtype=torch.long, device=dev)
    seq_lens = torch.ones(bucket, dtype=torch.long, device=dev)
    meta = AttentionMetadata(
        slot_mapping=slot_mapping,
        block_tables=block_tables,
        seq_lens=seq_lens,
        query_lens=torch.ones(bucket, dtype=torch.long, device=dev),
        query_start_loc=torch.arange(bucket + 1, dtype=torch.long, device=dev),
        max_seq_len=1,  # unused by the backend, as in the reference's decode graph
        max_query_len=1,
    )
    scale = D**-0.5

    def step():
        HipAttention.write_kv(k_cache, v_cache, k, v, meta.slot_mapping)
        return HipAttention.forward(q, k_cache, v_cache, meta, scale)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()

    rng = random.Random(1)
    ids = list(range(NB))
    for it in range(4):
        n = rng.choice([3, 5, 8])  # real rows; the rest of the bucket is padding
        lens = [rng.randint(1, 2048) for _ in range(n)]
        rng.shuffle(ids)
        tables, i = [], 0
        for L in lens:
            nb = -(-L // BS)
            tables.append(ids[i : i + nb])
            i += nb
        width = max(len(t) for t in tables)
        rows = [t + [scratch_block] * (width - len(t)) for t in tables] + [[scratch_block] * width] * (bucket - n)
        slots = [t[(L - 1) // BS] * BS + (L - 1) % BS for t, L in zip(tables, lens)]
        q.copy_(torch.randn(bucket, H, D, generator=gen, device=dev).to(dtype))
        k.copy_(torch.randn(bucket, Hkv, D, generator=gen, device=dev).to(dtype))
        v.copy_(torch.randn(bucket, Hkv, D, generator=gen, device=dev).to(dtype))
        slot_mapping.copy_(torch.tensor(slots + [scratch_slot] * (bucket - n)), non_blocking=True)
        seq_lens.copy_(torch.tensor(lens + [1] * (bucket - n)), non_blocking=True)
        block_tables[:, :width].copy_(torch.tensor(rows), non_blocking=True)

        graph.replay()
        replayed = out.clone()
        _ = torch.randn(512, 512, device=dev) @ torch.randn(512, 512, device=dev)  # unrelated eager work
        torch.cuda.synchronize()
        eager = HipAttention.forward(q, k_cache, v_cache, meta, scale)
        torch.cuda.synchronize()
        assert torch.equal(replayed.view(torch.int16 if dtype != torch.float32 else torch.int32),
                           eager.view(torch.int16 if dtype != torch.float32 else torch.int32)), f"replay {it}"  # fmt: skip

        wl = Workload("graph", [1] * n, lens, tables, NB + 1, H, Hkv, D, BS)
        batch = PagedBatch(wl, q[:n], k[:n], v[:n], k_cache, v_cache, meta)
        tol = pc.TOL_F32 if dtype == torch.float32 else pc.TOL_16BIT
        assert pc.max_err_vs_oracle(batch, replayed[:n], list(range(n))) <= tol, f"replay {it}"
        assert pc.written_rows_match(PagedBatch(wl, q[:n], k[:n], v[:n], k_cache, v_cache,
                                                AttentionMetadata(slot_mapping[:n], *[None] * 4, 0, 0)))  # fmt: skip
