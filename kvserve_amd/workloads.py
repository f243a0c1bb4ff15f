"""Seeded synthetic paged batches: the reference's parity CASES and the five BASELINE configs.

Layout follows the reference's own generator (tests/test_triton_attention.py:13-52):
`random.Random(seed)` draws lengths and shuffles the physical block pool, each sequence
takes ceil(seq_len / block_size) distinct blocks, rows are 0-padded to the longest, and
q / K / V are N(0, 1). Block ids and slots use kvserve's slot formula
(src/kvserve/kv_cache.py:155-169): slot = table[pos // BS] * BS + pos % BS.

A `Workload` is host-only (lengths, tables); `materialize` puts values on a device.
"""

from __future__ import annotations

import math
import random
from dataclasses import dataclass, field

import torch

from kvserve_amd.attention import AttentionMetadata

# tests/test_triton_attention.py:55-61: (query_lens, context_lens)
REFERENCE_CASES: dict[str, tuple[list[int], list[int]]] = {
    "decode": ([1] * 8, [5, 17, 64, 100, 1, 300, 16, 33]),
    "prefill": ([7, 64, 130], [0, 0, 0]),
    "chunked_prefill": ([50, 16, 3], [100, 16, 250]),
    "mixed": ([1, 1, 200, 1, 37], [40, 511, 0, 2, 70]),
    "long_decode": ([1, 1], [4000, 2047]),
}


def slots_for(table: list[int], block_size: int, start: int, n: int) -> list[int]:
    """Flat KV slots of positions [start, start + n) of a sequence with this block table."""
    return [table[p // block_size] * block_size + p % block_size for p in range(start, start + n)]


@dataclass
class Workload:
    name: str
    query_lens: list[int]
    seq_lens: list[int]  # context INCLUDING this step's query tokens
    tables: list[list[int]]  # physical block ids per sequence (unpadded)
    num_blocks: int  # pool size (block ids are < num_blocks)
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    width: int = 0  # block-table row width W (0: longest table)
    notes: dict = field(default_factory=dict)

    @property
    def scale(self) -> float:
        return self.head_dim**-0.5

    @property
    def num_tokens(self) -> int:
        return sum(self.query_lens)

    @property
    def context_lens(self) -> list[int]:
        return [s - q for s, q in zip(self.seq_lens, self.query_lens)]

    def table_width(self) -> int:
        return max(self.width, max(len(t) for t in self.tables))

    def slot_mapping(self) -> list[int]:
        out: list[int] = []
        for t, s, q in zip(self.tables, self.seq_lens, self.query_lens):
            out += slots_for(t, self.block_size, s - q, q)
        return out

    def unique_tokens(self) -> int:
        """Tokens held by the distinct physical blocks the step reads (a shared block counts once)."""
        seen: dict[int, int] = {}
        bs = self.block_size
        for t, s in zip(self.tables, self.seq_lens):
            for i in range(math.ceil(s / bs)):
                used = min(bs, s - i * bs)
                seen[t[i]] = max(seen.get(t[i], 0), used)
        return sum(seen.values())

    def kv_bytes(self, elem_bytes: int, unique: bool = True) -> int:
        n = self.unique_tokens() if unique else sum(self.seq_lens)
        return 2 * self.num_kv_heads * self.head_dim * elem_bytes * n

    def algorithmic_bytes(self, elem_bytes: int, unique: bool = True, kv_elem_bytes: int | None = None) -> int:
        """K/V read once + Q read + O written + block-table and length metadata (K/V elements
        of kv_elem_bytes, 1 for an E4M3 cache; default elem_bytes)."""
        qo = 2 * self.num_tokens * self.num_heads * self.head_dim * elem_bytes
        bt = 8 * sum(math.ceil(s / self.block_size) for s in self.seq_lens)
        md = 8 * (3 * len(self.seq_lens) + 1)
        kv = self.kv_bytes(elem_bytes if kv_elem_bytes is None else kv_elem_bytes, unique)
        return kv + qo + bt + md

    def flops(self) -> int:
        """4 * H * D per visible (query row, key) pair: QK^T and PV, multiply-add = 2."""
        tot = 0
        for s, q in zip(self.seq_lens, self.query_lens):
            c = s - q
            tot += q * c + q * (q + 1) // 2
        return 4 * self.num_heads * self.head_dim * tot


def _disjoint_tables(rng: random.Random, seq_lens: list[int], bs: int, pool: int) -> list[list[int]]:
    need = [math.ceil(s / bs) for s in seq_lens]
    if sum(need) > pool:
        raise ValueError(f"pool of {pool} blocks cannot hold {sum(need)}")
    ids = list(range(pool))
    rng.shuffle(ids)
    tables, i = [], 0
    for n in need:
        tables.append(ids[i : i + n])
        i += n
    return tables


def reference_case(
    name: str, num_heads: int, num_kv_heads: int, head_dim: int = 64, block_size: int = 16, seed: int = 0
) -> Workload:
    """One of the reference's CASES with its generator's pool: sum of blocks + 8 spare, shuffled."""
    q, c = REFERENCE_CASES[name]
    return custom(name, q, c, num_heads, num_kv_heads, head_dim, block_size, seed)


def custom(
    name: str,
    query_lens: list[int],
    context_lens: list[int],
    num_heads: int,
    num_kv_heads: int,
    head_dim: int,
    block_size: int,
    seed: int = 0,
    spare_blocks: int = 8,
) -> Workload:
    rng = random.Random(seed)
    seq_lens = [c + q for q, c in zip(query_lens, context_lens)]
    pool = sum(math.ceil(s / block_size) for s in seq_lens) + spare_blocks
    tables = _disjoint_tables(rng, seq_lens, block_size, pool)
    return Workload(name, list(query_lens), seq_lens, tables, pool, num_heads, num_kv_heads, head_dim, block_size)


def baseline_config(idx: int, seed: int = 0) -> Workload:
    """BASELINE.json configs[idx - 1] (1-based, as C1..C5)."""
    rng = random.Random(seed)
    bs = 16
    if idx == 1:  # Llama-3.2-1B decode: B=8, ctx U[64,512], 512-block pool
        seq = [rng.randint(64, 512) for _ in range(8)]
        tables = _disjoint_tables(rng, seq, bs, 512)
        return Workload("c1_1b_decode", [1] * 8, seq, tables, 512, 32, 8, 64, bs, width=32)
    if idx == 2:  # Llama-3.1-8B decode: B=64, ctx U[1024,8192], 40k-block pool
        seq = [rng.randint(1024, 8192) for _ in range(64)]
        tables = _disjoint_tables(rng, seq, bs, 40_000)
        return Workload("c2_8b_decode", [1] * 64, seq, tables, 40_000, 32, 8, 128, bs, width=512)
    if idx == 3:  # mixed chunked-prefill step, decodes first as the scheduler orders them
        dec = [rng.randint(256, 4096) for _ in range(512)]
        pre_ctx = [rng.randint(0, 4096) for _ in range(4)]
        seq = dec + [c + 384 for c in pre_ctx]
        ql = [1] * 512 + [384] * 4
        need = sum(math.ceil(s / bs) for s in seq)
        pool = int(need * 1.1)
        tables = _disjoint_tables(rng, seq, bs, pool)
        return Workload("c3_mixed_prefill", ql, seq, tables, pool, 32, 8, 128, bs, width=280)
    if idx == 4:  # long context, 750-block shared prefix in every table
        seq = [rng.randint(16_000, 32_000) for _ in range(16)]
        shared_blocks = 750
        ids = list(range(40_000))
        rng.shuffle(ids)
        shared = ids[:shared_blocks]
        i = shared_blocks
        tables = []
        for s in seq:
            n = math.ceil(s / bs) - shared_blocks
            tables.append(shared + ids[i : i + n])
            i += n
        w = Workload("c4_long_prefix_shared", [1] * 16, seq, tables, 40_000, 32, 8, 128, bs, width=2000)
        w.notes["shared_prefix_blocks"] = shared_blocks
        return w
    if idx == 5:  # speculative verify: 5 draft tokens over ctx U[2048,4096]
        ctx = [rng.randint(2048, 4096) for _ in range(32)]
        seq = [c + 5 for c in ctx]
        tables = _disjoint_tables(rng, seq, bs, 40_000)
        return Workload("c5_spec_verify", [5] * 32, seq, tables, 40_000, 32, 8, 128, bs, width=257)
    raise ValueError(f"no config {idx}")


@dataclass
class PagedBatch:
    """Device tensors of a workload: the step's q/k/v and a pool holding the cached context."""

    workload: Workload
    q: torch.Tensor  # [T, H, D]
    k_new: torch.Tensor  # [T, Hkv, D] this step's keys (written by write_kv)
    v_new: torch.Tensor
    k_cache: torch.Tensor  # [num_blocks, BS, Hkv, D]
    v_cache: torch.Tensor
    meta: AttentionMetadata


def materialize(
    w: Workload, dtype: torch.dtype, device: str | torch.device, seed: int = 0, fill: str = "randn"
) -> PagedBatch:
    """Values N(0, 1) from a generator seeded with `seed` on `device` (fill="randn"), or an
    uninitialised pool (fill="empty") for bandwidth runs where content does not matter."""
    device = torch.device(device)
    gen = torch.Generator(device=device).manual_seed(seed)
    T, H, Hkv, D = w.num_tokens, w.num_heads, w.num_kv_heads, w.head_dim
    shape = (w.num_blocks, w.block_size, Hkv, D)

    def randn(*s: int) -> torch.Tensor:
        return torch.randn(*s, generator=gen, device=device, dtype=torch.float32).to(dtype)

    q = randn(T, H, D)
    k_new, v_new = randn(T, Hkv, D), randn(T, Hkv, D)
    if fill == "randn":
        k_cache = torch.empty(shape, dtype=dtype, device=device)
        v_cache = torch.empty(shape, dtype=dtype, device=device)
        for c in (k_cache, v_cache):  # block by block keeps the fp32 staging small
            step = max(1, (1 << 26) // (w.block_size * Hkv * D))
            for b0 in range(0, w.num_blocks, step):
                b1 = min(w.num_blocks, b0 + step)
                c[b0:b1] = randn(b1 - b0, w.block_size, Hkv, D)
    else:
        k_cache = torch.empty(shape, dtype=dtype, device=device)
        v_cache = torch.empty(shape, dtype=dtype, device=device)
    width = w.table_width()
    rows = [t + [0] * (width - len(t)) for t in w.tables]
    qsl = [0]
    for n in w.query_lens:
        qsl.append(qsl[-1] + n)
    meta = AttentionMetadata(
        slot_mapping=torch.tensor(w.slot_mapping(), dtype=torch.long, device=device),
        block_tables=torch.tensor(rows, dtype=torch.long, device=device),
        seq_lens=torch.tensor(w.seq_lens, dtype=torch.long, device=device),
        query_lens=torch.tensor(w.query_lens, dtype=torch.long, device=device),
        query_start_loc=torch.tensor(qsl, dtype=torch.long, device=device),
        max_seq_len=max(w.seq_lens),
        max_query_len=max(w.query_lens),
    )
    return PagedBatch(w, q, k_new, v_new, k_cache, v_cache, meta)
