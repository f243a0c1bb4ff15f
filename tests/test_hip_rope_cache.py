"""kvh_rope_and_cache (HipAttention.rope_and_cache) against the reference's torch steps it
replaces: RoPE of q and k (src/kvserve/model.py:55-70, 84-94) and write_kv
(src/kvserve/attention.py:39-45), bit for bit in bf16, fp16 and fp32."""

from __future__ import annotations

import dataclasses

import pytest
import torch

from kvserve_amd import HipAttention
from kvserve_amd.engine import LLAMA_3_2_1B
from kvserve_amd.engine.model import RotaryEmbedding
from oracle import torch_reference

pytestmark = pytest.mark.gpu


def _case(dtype, H, Hkv, D, T, num_blocks=64, BS=16, max_pos=4096, extra=0, seed=0):
    dev = "cuda:0"
    g = torch.Generator(device=dev).manual_seed(seed)
    width = (H + 2 * Hkv) * D
    buf = torch.randn(T, width + extra, generator=g, device=dev).to(dtype)
    qkv = buf[:, :width]  # a strided view when extra > 0
    rope = RotaryEmbedding(dataclasses.replace(LLAMA_3_2_1B, head_dim=D), max_pos, device=dev)
    positions = torch.randint(0, max_pos, (T,), generator=g, device=dev)
    slots = torch.randperm(num_blocks * BS, generator=g, device=dev)[:T]
    kc = torch.randn(num_blocks, BS, Hkv, D, generator=g, device=dev).to(dtype)
    vc = torch.randn(num_blocks, BS, Hkv, D, generator=g, device=dev).to(dtype)
    return qkv, rope, positions, slots, kc, vc


def _reference(qkv, rope, positions, slots, kc, vc, H, Hkv, D):
    q, k, v = qkv.split([H * D, Hkv * D, Hkv * D], dim=-1)
    q = q.reshape(-1, H, D)
    k = k.reshape(-1, Hkv, D)
    v = v.reshape(-1, Hkv, D)
    q = torch_reference.rope(q, rope.cos, rope.sin, positions)
    k = torch_reference.rope(k, rope.cos, rope.sin, positions)
    kc, vc = kc.clone(), vc.clone()
    torch_reference.write_kv(kc, vc, k, v, slots)
    return q, kc, vc


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("H,Hkv,D,T", [(32, 8, 64, 17), (32, 8, 128, 300), (8, 2, 64, 1), (16, 16, 128, 5)])
def test_bit_exact_against_torch_steps(hip_device, dtype, H, Hkv, D, T):
    qkv, rope, pos, slots, kc, vc = _case(dtype, H, Hkv, D, T, extra=16 if T > 1 else 0)
    want_q, want_k, want_v = _reference(qkv, rope, pos, slots, kc, vc, H, Hkv, D)
    got_q = HipAttention.rope_and_cache(qkv, pos, rope.cos, rope.sin, kc, vc, slots, H)
    torch.cuda.synchronize()
    assert torch.equal(got_q, want_q)
    assert torch.equal(kc, want_k)
    assert torch.equal(vc, want_v)


def test_out_of_pool_slots_and_clamped_positions(hip_device):
    H, Hkv, D, T = 32, 8, 128, 8
    qkv, rope, pos, slots, kc, vc = _case(torch.bfloat16, H, Hkv, D, T)
    slots[2] = -1
    slots[5] = kc.shape[0] * kc.shape[1]  # one past the pool
    kc0, vc0 = kc.clone(), vc.clone()
    got_q = HipAttention.rope_and_cache(qkv, pos, rope.cos, rope.sin, kc, vc, slots, H)
    keep = torch.tensor([i not in (2, 5) for i in range(T)], device=kc.device)
    want_q, want_k, want_v = _reference(qkv[keep], rope, pos[keep], slots[keep], kc0, vc0, H, Hkv, D)
    assert torch.equal(got_q[keep], want_q)
    assert torch.equal(kc, want_k) and torch.equal(vc, want_v)
    # a position past the table reads its last row
    pos2 = pos.clone()
    pos2[0] = 10**9
    q2 = HipAttention.rope_and_cache(qkv, pos2, rope.cos, rope.sin, kc.clone(), vc.clone(), slots, H)
    pos3 = pos.clone()
    pos3[0] = rope.cos.shape[0] - 1
    q3 = HipAttention.rope_and_cache(qkv, pos3, rope.cos, rope.sin, kc.clone(), vc.clone(), slots, H)
    assert torch.equal(q2, q3)


def test_argument_errors(hip_device):
    qkv, rope, pos, slots, kc, vc = _case(torch.bfloat16, 8, 2, 64, 4)
    with pytest.raises(ValueError):
        HipAttention.rope_and_cache(qkv[:, :-64], pos, rope.cos, rope.sin, kc, vc, slots, 8)
    with pytest.raises(ValueError):
        HipAttention.rope_and_cache(qkv, pos, rope.cos.half(), rope.sin.half(), kc, vc, slots, 8)
    with pytest.raises(ValueError):
        HipAttention.rope_and_cache(qkv, pos[:2], rope.cos, rope.sin, kc, vc, slots, 8)
