"""Device-side attention metadata: block tables resident in HBM, one upload per step.

The reference rebuilds a step's metadata on the host every step: `build_metadata`
(src/kvserve/model_runner.py:165-197) pads every scheduled sequence's whole block table and
uploads five tensors, and `DecodeGraphRunner.run` (src/kvserve/cuda_graph.py:111-134) does
the same into static buffers (scratch-padded, only the first `width` table columns). Both are
O(B x W) Python per step; the reference's own profile names this input preparation as the
cost that dominates at large batch.

`DeviceMetadata` keeps each live sequence's block table in a device pool row, appends only
the entries added since the previous step, and uploads one packed int32 buffer per step
(per-sequence row/start/q_len/n_blocks, the new table entries, the token ids) through a
pinned staging ring; `kvh_prepare_metadata` expands it on the device into the same tensors
the reference builds (`slot_mapping`, `block_tables`, `seq_lens`, `query_lens`,
`query_start_loc`, plus `positions` and `input_ids`). Host work per step is O(B + new
blocks + T).

Block tables must be append-only between releases, as the reference's KVCacheManager keeps
them (kv_cache.py:118-153: blocks are appended, and `free` replaces the list with a new
empty one). A sequence whose table list object changes, or shrinks, is re-sent from column 0.
"""

from __future__ import annotations

from collections.abc import Hashable, Sequence

import numpy as np
import torch

from kvserve_amd import _lib
from kvserve_amd.attention import AttentionMetadata


class MetaBuffers:
    """Device outputs of `DeviceMetadata.build`, sized for `max_tokens` tokens and `max_seqs`
    sequences; rebuilt in place by every build that targets them. The initial contents are
    the graph runner's static-buffer defaults (cuda_graph.py:54-62): slots `slot_fill`,
    tables `table_fill`, seq_len 1, query_len 1, query_start_loc = arange."""

    def __init__(self, device: torch.device | str, max_tokens: int, max_seqs: int, width: int, slot_fill: int = 0,
                 table_fill: int = 0):  # fmt: skip
        i64 = dict(dtype=torch.long, device=device)
        self.max_tokens, self.max_seqs, self.width = max_tokens, max_seqs, width
        self.slot_mapping = torch.full((max_tokens,), slot_fill, **i64)
        self.positions = torch.zeros(max_tokens, **i64)
        self.input_ids = torch.zeros(max_tokens, **i64)
        self.block_tables = torch.full((max_seqs, width), table_fill, **i64)
        self.seq_lens = torch.ones(max_seqs, **i64)
        self.query_lens = torch.ones(max_seqs, **i64)
        self.query_start_loc = torch.arange(max_seqs + 1, **i64)


class _Staging:
    """One pinned host buffer and its device twin; `ready` orders reuse after the upload."""

    def __init__(self, device: torch.device, cap: int):
        self.cap = cap
        self.host = torch.empty(cap, dtype=torch.int32, pin_memory=True)
        self.view = self.host.numpy()
        self.dev = torch.empty(cap, dtype=torch.int32, device=device)
        self.ready = torch.cuda.Event()
        self.used = False


class DeviceMetadata:
    """Resident block tables for up to `max_seqs` live sequences of at most
    `max_blocks_per_seq` blocks, and a default `MetaBuffers` for `max_tokens` tokens."""

    RING = 2

    def __init__(self, device: torch.device | str, max_seqs: int, max_blocks_per_seq: int, block_size: int,
                 max_tokens: int):  # fmt: skip
        if max_seqs <= 0 or max_blocks_per_seq <= 0 or block_size <= 0 or max_tokens <= 0:
            raise ValueError("DeviceMetadata sizes must be positive")
        if max_seqs >= 2**31 or max_blocks_per_seq >= 2**31:
            raise ValueError("DeviceMetadata sizes must fit int32")
        self.device = torch.device(device)
        self.block_size = block_size
        self.max_seqs = max_seqs
        self.width = max_blocks_per_seq
        self.pool = torch.zeros(max_seqs, max_blocks_per_seq, dtype=torch.long, device=self.device)
        self.buffers = MetaBuffers(self.device, max_tokens, max_seqs, max_blocks_per_seq)
        # key -> [row, the table list last seen, entries already in the pool]
        self._rows: dict[Hashable, list] = {}
        self._free = list(range(max_seqs - 1, -1, -1))
        self._ring = [_Staging(self.device, 4096) for _ in range(self.RING)]
        self._next = 0
        self._lib = _lib.load()

    # -- rows ------------------------------------------------------------------------------------
    def release(self, key: Hashable) -> None:
        """Forget a sequence (its pool row is reused by the next new one)."""
        ent = self._rows.pop(key, None)
        if ent is not None:
            self._free.append(ent[0])

    def _entry(self, key: Hashable, table: list[int]) -> list:
        ent = self._rows.get(key)
        if ent is None:
            if not self._free:
                raise RuntimeError(f"DeviceMetadata: more than {self.max_seqs} live sequences")
            ent = [self._free.pop(), table, 0]
            self._rows[key] = ent
        elif ent[1] is not table or len(table) < ent[2]:
            ent[1], ent[2] = table, 0  # a new table for this sequence: send it whole
        return ent

    def _staging(self, n: int) -> _Staging:
        st = self._ring[self._next]
        self._next = (self._next + 1) % self.RING
        if st.used:
            st.ready.synchronize()  # its previous upload has been read
        if n > st.cap:
            cap = max(n, 2 * st.cap)
            st.host = torch.empty(cap, dtype=torch.int32, pin_memory=True)
            st.view = st.host.numpy()
            st.dev = torch.empty(cap, dtype=torch.int32, device=self.device)
            st.cap = cap
        return st

    # -- build -----------------------------------------------------------------------------------
    def build(
        self,
        seqs: Sequence[tuple[Hashable, list[int]]],
        starts: Sequence[int],
        query_lens: Sequence[int],
        input_ids: Sequence[int] | None = None,
        *,
        buffers: MetaBuffers | None = None,
        pad_seqs: int = 0,
        pad_slot: int = -1,
        table_pad: int = 0,
        width: int | None = None,
    ) -> tuple[AttentionMetadata, torch.Tensor, torch.Tensor]:
        """Metadata of one step: sequence b is `seqs[b] = (key, block_table)` and computes
        `query_lens[b]` tokens from position `starts[b]`. Returns the metadata and the
        `input_ids` / `positions` tensors (views of `buffers`, valid until the next build that
        targets them).

        Defaults follow build_metadata (model_runner.py:165-197): tables 0-padded to the
        longest. The graph runner's refresh (cuda_graph.py:111-134) is `pad_seqs` one-token
        rows with `pad_slot`, `table_pad` = the scratch block and `width` columns written.
        """
        buf = self.buffers if buffers is None else buffers
        B = len(seqs)
        if len(starts) != B or len(query_lens) != B:
            raise ValueError("seqs, starts and query_lens differ in length")
        if B + pad_seqs < 1:
            raise ValueError("empty batch")
        bs = self.block_size
        rec = np.empty((B, 4), dtype=np.int64)
        upd: list[int] = []
        sent: list[tuple[list, int]] = []  # pool rows extended by this call, committed after launch
        max_nb = 0
        for b, (key, table) in enumerate(seqs):
            ent = self._entry(key, table)
            n = len(table)
            if n > self.width:
                raise ValueError(f"block table of {n} entries exceeds max_blocks_per_seq={self.width}")
            s, q = int(starts[b]), int(query_lens[b])
            if s < 0 or q < 0 or s + q > n * bs:
                raise ValueError(f"sequence {b}: positions [{s}, {s + q}) outside its {n} blocks")
            if n > ent[2]:
                row = ent[0]
                for c in range(ent[2], n):
                    upd += (row, c, table[c])
                sent.append((ent, n))
            rec[b] = (ent[0], s, q, n)
            max_nb = max(max_nb, n)
        T = int(rec[:, 2].sum()) if B else 0
        if input_ids is not None and len(input_ids) != T:
            raise ValueError(f"{len(input_ids)} input ids for {T} tokens")
        if T + pad_seqs > buf.max_tokens or B + pad_seqs > buf.max_seqs:
            raise ValueError(f"batch of {T + pad_seqs} tokens / {B + pad_seqs} sequences exceeds the buffers")
        w = max_nb if width is None else width
        if w < max_nb or w > buf.width:
            raise ValueError(f"table width {w} must lie in [{max_nb}, {buf.width}]")
        U = len(upd) // 3
        if U and not 0 <= min(upd[2::3]) <= max(upd[2::3]) < 2**31:
            raise ValueError("block ids must lie in [0, 2**31)")
        n_ids = T if input_ids is not None else 0
        total = 4 * B + 3 * U + n_ids
        st = self._staging(max(total, 1))
        v = st.view
        v[: 4 * B] = rec.reshape(-1)
        if U:
            v[4 * B : 4 * B + 3 * U] = upd
        if n_ids:
            v[4 * B + 3 * U : total] = input_ids
        if total:
            st.dev[:total].copy_(st.host[:total], non_blocking=True)
        st.ready.record()
        st.used = True
        lib = self._lib
        status = lib.kvh_prepare_metadata(
            st.dev.data_ptr(), B, pad_seqs, U, T,
            self.pool.data_ptr(), self.max_seqs, self.pool.stride(0), self.width,
            buf.block_tables.data_ptr(), buf.block_tables.stride(0), w, table_pad,
            buf.slot_mapping.data_ptr(), buf.positions.data_ptr(),
            buf.input_ids.data_ptr() if input_ids is not None else None,
            buf.seq_lens.data_ptr(), buf.query_lens.data_ptr(), buf.query_start_loc.data_ptr(),
            pad_slot, bs, torch.cuda.current_stream(self.device).cuda_stream,
        )  # fmt: skip
        _lib.check(status, "kvh_prepare_metadata")
        for ent, n in sent:
            ent[2] = n
        rows, toks = B + pad_seqs, T + pad_seqs
        seq_max = int((rec[:, 1] + rec[:, 2]).max()) if B else 1
        q_max = int(rec[:, 2].max()) if B else 1
        meta = AttentionMetadata(
            slot_mapping=buf.slot_mapping[:toks],
            block_tables=buf.block_tables[:rows, :w],
            seq_lens=buf.seq_lens[:rows],
            query_lens=buf.query_lens[:rows],
            query_start_loc=buf.query_start_loc[: rows + 1],
            max_seq_len=max(seq_max, 1 if pad_seqs else 0),
            max_query_len=max(q_max, 1 if pad_seqs else 0),
        )
        return meta, buf.input_ids[:toks], buf.positions[:toks]
