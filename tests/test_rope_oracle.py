"""The oracle's RoPE (oracle/torch_reference.rope) pinned against Hugging Face transformers'
own apply_rotary_pos_emb with its Llama 3 rotary tables, bit for bit in fp32 and bf16."""

from __future__ import annotations

import dataclasses

import pytest
import torch

from kvserve_amd.engine import LLAMA_3_2_1B
from tests.engine_backends import rope as rope_table
from oracle import torch_reference

transformers = pytest.importorskip("transformers")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rope_matches_transformers(dtype):
    from transformers.models.llama import modeling_llama as hf

    cfg = LLAMA_3_2_1B
    hf_cfg = transformers.LlamaConfig(**{k: v for k, v in cfg.to_hf_dict().items() if k not in ("model_type", "architectures")})
    rot = hf.LlamaRotaryEmbedding(hf_cfg)
    g = torch.Generator().manual_seed(0)
    T = 37
    positions = torch.randint(0, 4096, (T,), generator=g)
    q = torch.randn(T, cfg.num_heads, cfg.head_dim, generator=g).to(dtype)
    # HF computes cos/sin in fp32 for the positions and casts them to the activation dtype
    cos_hf, sin_hf = rot(q.transpose(0, 1)[None], positions[None])
    want = hf.apply_rotary_pos_emb(q.transpose(0, 1)[None], q.transpose(0, 1)[None], cos_hf, sin_hf)[0][0]
    want = want.transpose(0, 1)
    # the oracle, fed with fp32 tables of the same frequencies
    table = rope_table(cfg, 4096)
    got = torch_reference.rope(q, table.cos, table.sin, positions)
    assert torch.equal(got, want)


def test_planted_mistake_is_caught():
    """The oracle is a rotation (norms kept, position 0 the identity), and a rotate_half with
    the halves' signs swapped (a plausible slip) gives different values."""
    g = torch.Generator().manual_seed(1)
    x = torch.randn(5, 2, 8, generator=g)
    table = rope_table(dataclasses.replace(LLAMA_3_2_1B, head_dim=8), 64)
    pos = torch.tensor([0, 1, 7, 30, 63])
    r = torch_reference.rope(x, table.cos, table.sin, pos)
    torch.testing.assert_close(r.norm(dim=-1), x.norm(dim=-1))
    x1, x2 = x.chunk(2, dim=-1)
    cos = table.cos[pos][:, None]
    sin = table.sin[pos][:, None]
    wrong = x * cos + torch.cat([x2, -x1], dim=-1) * sin
    assert not torch.allclose(wrong[1:], r[1:])
    torch.testing.assert_close(r[0], x[0])  # position 0 is the identity
