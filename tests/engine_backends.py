"""Torch attention backend for the engine tests: the reference's TorchAttention
(src/kvserve/attention.py:31-82) restated in oracle/torch_reference.py, behind the same
static-method interface as HipAttention. Test infrastructure only."""

from __future__ import annotations

import torch

from oracle import torch_reference


class TorchRefAttention:
    name = "torch"
    graph_capturable = False  # derives shapes from per-step host values (cuda_graph.py:17-18)
    needs_padded_layout = True

    @staticmethod
    def write_kv(k_cache, v_cache, k, v, slots) -> None:
        torch_reference.write_kv(k_cache, v_cache, k, v, slots)

    @staticmethod
    def forward(q, k_cache, v_cache, meta, scale, out=None) -> torch.Tensor:
        res = torch_reference.forward(q, k_cache, v_cache, meta.block_tables, meta.seq_lens, meta.query_lens, scale,
                                      meta.q_gather, meta.q_valid).to(q.dtype)  # fmt: skip
        if out is not None:
            out.copy_(res)
            return out
        return res
