"""Restatement of the reference's torch attention path. TEST INFRASTRUCTURE ONLY.

The checker for large parity cases and the CPU baseline of bench.py. It follows
TorchAttention (src/kvserve/attention.py:39-82) step by step:
  write_kv: cache.view(-1, Hkv, D)[slots] = k                            (:39-45)
  forward:  gather ceil(max_seq_len / BS) pages per sequence -> [B, S, Hkv, D],
            repeat_interleave(H / Hkv) for GQA, gather padded queries with q_gather,
            mask k_pos <= (seq_len - query_len) + i, scaled_dot_product_attention,
            un-pad with q_valid                                          (:47-82)
and the padded-layout metadata of build_metadata (src/kvserve/model_runner.py:190-196),
plus the RoPE of Attention.project (src/kvserve/model.py:55-70, 84-94) that precedes it.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def rope(x: torch.Tensor, cos_table: torch.Tensor, sin_table: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
    """RotaryEmbedding.forward on one of q / k (src/kvserve/model.py:55-70): the fp32 tables
    gathered at the positions and cast to x's dtype, then x * cos + rotate_half(x) * sin in
    x's dtype, rotate_half(x) = cat(-x2, x1)."""
    cos = cos_table[positions].to(x.dtype)[:, None]
    sin = sin_table[positions].to(x.dtype)[:, None]
    x1, x2 = x.chunk(2, dim=-1)
    return x * cos + torch.cat([-x2, x1], dim=-1) * sin


def write_kv(k_cache: torch.Tensor, v_cache: torch.Tensor, k: torch.Tensor, v: torch.Tensor, slots: torch.Tensor):
    k_cache.view(-1, *k_cache.shape[2:])[slots] = k
    v_cache.view(-1, *v_cache.shape[2:])[slots] = v


def padded_layout(query_lens: list[int], device="cpu") -> tuple[torch.Tensor, torch.Tensor]:
    """q_gather [B, max_q] (0-padded flat indices) and q_valid [B, max_q]."""
    max_q = max(query_lens)
    q_gather, q_valid, off = [], [], 0
    for n in query_lens:
        q_gather.append(list(range(off, off + n)) + [0] * (max_q - n))
        q_valid.append([True] * n + [False] * (max_q - n))
        off += n
    return (
        torch.tensor(q_gather, dtype=torch.long, device=device),
        torch.tensor(q_valid, dtype=torch.bool, device=device),
    )


def forward(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    query_lens: torch.Tensor,
    scale: float,
    q_gather: torch.Tensor | None = None,
    q_valid: torch.Tensor | None = None,
) -> torch.Tensor:
    """TorchAttention.forward on explicit tensors; returns [T, H, D] in flat token order."""
    num_tokens, num_heads, _ = q.shape
    block_size, num_kv_heads = k_cache.shape[1], k_cache.shape[2]
    ql = [int(x) for x in query_lens.tolist()]
    if q_gather is None or q_valid is None:
        q_gather, q_valid = padded_layout(ql, q.device)
    max_seq_len = int(seq_lens.max())
    max_query_len = max(ql)
    num_blocks = -(-max_seq_len // block_size)
    tables = block_tables[:, :num_blocks]
    k = k_cache[tables].flatten(1, 2)[:, :max_seq_len].transpose(1, 2)
    v = v_cache[tables].flatten(1, 2)[:, :max_seq_len].transpose(1, 2)
    if num_kv_heads != num_heads:
        k = k.repeat_interleave(num_heads // num_kv_heads, dim=1)
        v = v.repeat_interleave(num_heads // num_kv_heads, dim=1)
    qp = q[q_gather].transpose(1, 2)  # [B, H, max_q, D]
    device = q.device
    q_pos = (seq_lens - query_lens)[:, None] + torch.arange(max_query_len, device=device)
    k_pos = torch.arange(max_seq_len, device=device)
    mask = k_pos[None, None, :] <= q_pos[:, :, None]
    res = F.scaled_dot_product_attention(qp, k, v, attn_mask=mask[:, None], scale=scale)
    res = res.transpose(1, 2)[q_valid]
    assert res.shape[0] == num_tokens
    return res

