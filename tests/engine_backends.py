"""Torch attention backend for the engine tests: the reference's TorchAttention
(src/kvserve/attention.py:31-82) restated in oracle/torch_reference.py, behind the same
static-method interface as HipAttention. Test infrastructure only."""

from __future__ import annotations

from types import SimpleNamespace

import torch

from kvserve_amd.engine.model import rope_tables
from oracle import fp8, torch_reference


def rope(cfg, max_positions: int, device=None) -> SimpleNamespace:
    """The model's fp32 cos / sin tables as `.cos` / `.sin` [max_positions, head_dim]."""
    cos, sin = rope_tables(cfg, max_positions, device)
    return SimpleNamespace(cos=cos, sin=sin)


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


class TorchRefFP8Attention(TorchRefAttention):
    """The same over an E4M3 cache: write_kv stores the oracle's quantization
    (x / scale).clamp(-448, 448).to(float8_e4m3fn), forward attends in fp32 over the
    dequantized caches (e4m3 * scale)."""

    name = "torch-fp8"

    @staticmethod
    def write_kv(k_cache, v_cache, k, v, slots, k_scale=1.0, v_scale=1.0) -> None:
        kq = fp8.quantize(k, k_scale).to(k_cache.device).view(torch.uint8)
        vq = fp8.quantize(v, v_scale).to(v_cache.device).view(torch.uint8)
        torch_reference.write_kv(k_cache.view(torch.uint8), v_cache.view(torch.uint8), kq, vq, slots)

    @staticmethod
    def forward(q, k_cache, v_cache, meta, scale, out=None, k_scale=1.0, v_scale=1.0) -> torch.Tensor:
        kd, vd = fp8.dequantize(k_cache, k_scale), fp8.dequantize(v_cache, v_scale)
        res = torch_reference.forward(q.float(), kd, vd, meta.block_tables, meta.seq_lens, meta.query_lens, scale,
                                      meta.q_gather, meta.q_valid).to(q.dtype)  # fmt: skip
        if out is not None:
            out.copy_(res)
            return out
        return res
