"""Helpers shared by the GPU parity tests: run the HIP path, check it against the oracle.

The oracle side (oracle/, CPU) is only ever the checker here.
"""

from __future__ import annotations

import numpy as np
import torch

import oracle
from oracle import torch_reference
from kvserve_amd import HipAttention
from kvserve_amd.workloads import PagedBatch

# Parity bar for 16-bit storage with fp32 accumulation: max |hip - oracle| over all checked
# elements, against the oracle evaluated on the same 16-bit-rounded inputs.
TOL_16BIT = 2e-2
# exact-fp32 path vs the fp64 oracle
TOL_F32 = 1e-4


def attend(batch: PagedBatch, write: bool = True, out: torch.Tensor | None = None) -> torch.Tensor:
    """The backend's two calls as Attention.attend makes them (src/kvserve/model.py:106-108)."""
    if write:
        HipAttention.write_kv(batch.k_cache, batch.v_cache, batch.k_new, batch.v_new, batch.meta.slot_mapping)
    return HipAttention.forward(batch.q, batch.k_cache, batch.v_cache, batch.meta, batch.workload.scale, out=out)


def torch_oracle_full(batch: PagedBatch) -> torch.Tensor:
    """The torch restatement on CPU in fp32 over the whole (small) batch."""
    w, m = batch.workload, batch.meta
    return torch_reference.forward(
        batch.q.float().cpu(), batch.k_cache.float().cpu(), batch.v_cache.float().cpu(), m.block_tables.cpu(),
        m.seq_lens.cpu(), m.query_lens.cpu(), w.scale,
    )  # fmt: skip


def oracle_rows(batch: PagedBatch, seq: int, rows: list[int] | None = None) -> tuple[np.ndarray, list[int]]:
    """fp64 C oracle for some query rows of one sequence, reading the (device) cache as it is.

    Row i of a sequence sees keys 0 .. ctx + i, so it is evaluated as a one-query sequence of
    length ctx + i + 1 over the same pages. Returns ([len(rows), H, D], flat token ids)."""
    w = batch.workload
    table = w.tables[seq]
    dev = batch.k_cache.device
    idx = torch.tensor(table, dtype=torch.long, device=dev)
    kc = batch.k_cache.index_select(0, idx).to(torch.float64).cpu().numpy()
    vc = batch.v_cache.index_select(0, idx).to(torch.float64).cpu().numpy()
    q0 = sum(w.query_lens[:seq])
    ql = w.query_lens[seq]
    ctx = w.seq_lens[seq] - ql
    rows = list(range(ql)) if rows is None else rows
    toks = [q0 + i for i in rows]
    q = batch.q[torch.tensor(toks, device=dev)].to(torch.float64).cpu().numpy()
    n = len(rows)
    bt = np.tile(np.arange(len(table), dtype=np.int64), (n, 1))
    sl = np.asarray([ctx + i + 1 for i in rows], dtype=np.int64)
    qsl = np.arange(n + 1, dtype=np.int64)
    return oracle.paged_attention_f64(q, kc, vc, bt, sl, qsl, w.scale), toks


def max_err_vs_oracle(batch: PagedBatch, out: torch.Tensor, seqs: list[int], rows_per_seq: int | None = None) -> float:
    """Max abs error of `out` against the fp64 oracle over the chosen sequences; long
    queries are sampled at rows_per_seq evenly spaced rows (first and last included)."""
    worst = 0.0
    for s in seqs:
        ql = batch.workload.query_lens[s]
        rows = None
        if rows_per_seq is not None and ql > rows_per_seq:
            rows = sorted(set(np.linspace(0, ql - 1, rows_per_seq).round().astype(int).tolist()))
        ref, toks = oracle_rows(batch, s, rows)
        got = out[torch.tensor(toks, device=out.device)].to(torch.float64).cpu().numpy()
        worst = max(worst, float(np.max(np.abs(got - ref))) if got.size else 0.0)
    return worst


def written_rows_match(batch: PagedBatch) -> bool:
    """Every slot of slot_mapping holds this step's k/v row, bit for bit."""
    bs = batch.workload.block_size
    s = batch.meta.slot_mapping
    kc = batch.k_cache.view(-1, *batch.k_cache.shape[2:])
    vc = batch.v_cache.view(-1, *batch.v_cache.shape[2:])
    eq = lambda a, b: torch.equal(a.view(torch.int16) if a.element_size() == 2 else a.view(torch.int32),  # noqa: E731
                                  b.view(torch.int16) if b.element_size() == 2 else b.view(torch.int32))
    del bs
    return eq(kc[s], batch.k_new) and eq(vc[s], batch.v_new)
