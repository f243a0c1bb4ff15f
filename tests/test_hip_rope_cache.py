"""kvh_rope_and_cache (HipAttention.rope_and_cache) against the reference's torch steps it
replaces: RoPE of q and k (src/kvserve/model.py:55-70, 84-94) and write_kv
(src/kvserve/attention.py:39-45), bit for bit in bf16, fp16 and fp32."""

from __future__ import annotations

import dataclasses

import pytest
import torch

from kvserve_amd import HipAttention, _lib
from kvserve_amd.engine import LLAMA_3_2_1B
from tests.engine_backends import rope as rope_table
from oracle import torch_reference

pytestmark = pytest.mark.gpu


def _case(dtype, H, Hkv, D, T, num_blocks=64, BS=16, max_pos=4096, extra=0, seed=0):
    dev = "cuda:0"
    g = torch.Generator(device=dev).manual_seed(seed)
    width = (H + 2 * Hkv) * D
    buf = torch.randn(T, width + extra, generator=g, device=dev).to(dtype)
    qkv = buf[:, :width]  # a strided view when extra > 0
    rope = rope_table(dataclasses.replace(LLAMA_3_2_1B, head_dim=D), max_pos, device=dev)
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


# -- the QKV projection fused with RoPE + cache write (kvh_gemv_rope_and_cache) ----------------
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 17, 33, 64])
@pytest.mark.parametrize("H,Hkv,D,k", [(32, 8, 128, 4096), (32, 8, 64, 2048), (8, 2, 64, 136)])
@pytest.mark.parametrize("fp8", [False, True], ids=["cache16", "e4m3"])
def test_gemv_rope_and_cache_is_gemv_then_rope_and_cache(hip_device, dtype, m, H, Hkv, D, k, fp8):
    """The fused kernel gives the bits of the projection on kvh_gemv (m <= 4) or kvh_gemm_skinny
    (m > 4) followed by rope_and_cache: the same q, the same cache bytes (16-bit or E4M3 with
    scales), slots outside the pool skipped; k = 136 runs the GEMV's tail loop. Past 4 rows with
    k % 1024 != 0 (no MFMA form) the library rejects the call before any launch and the caches
    stay untouched."""
    from kvserve_amd.engine import ops
    from oracle import fp8 as fp8_oracle

    g = torch.Generator(device=hip_device).manual_seed(m * D + k + fp8)
    x = torch.randn(m, k, generator=g, device=hip_device).to(dtype)
    w = (torch.randn((H + 2 * Hkv) * D, k, generator=g, device=hip_device) * 0.05).to(dtype)
    rope = rope_table(dataclasses.replace(LLAMA_3_2_1B, head_dim=D), 4096, device=hip_device)
    pos = torch.randint(0, 4096, (m,), generator=g, device=hip_device)
    NB, BS = 32, 16
    slots = torch.randperm(NB * BS, generator=g, device=hip_device)[:m]
    if m > 1:
        slots[1] = NB * BS + 5  # outside the pool: no cache write
    sc = dict(k_scale=0.5, v_scale=1.5) if fp8 else {}
    kc = torch.randn(NB, BS, Hkv, D, generator=g, device=hip_device).to(dtype)
    vc = torch.randn(NB, BS, Hkv, D, generator=g, device=hip_device).to(dtype)
    if fp8:
        kc, vc = fp8_oracle.quantize(kc, 1.0).to(hip_device), fp8_oracle.quantize(vc, 1.0).to(hip_device)
    kc2, vc2 = kc.clone(), vc.clone()
    if m > 4 and k % 1024:
        with pytest.raises(_lib.KvhError) as err:
            HipAttention.gemv_rope_and_cache(x, w, pos, rope.cos, rope.sin, kc, vc, slots, H, **sc)
        assert err.value.status == -5  # KVH_E_UNSUPPORTED
        torch.cuda.synchronize()
        assert torch.equal(kc.view(torch.uint8), kc2.view(torch.uint8))
        assert torch.equal(vc.view(torch.uint8), vc2.view(torch.uint8))
        return
    got = HipAttention.gemv_rope_and_cache(x, w, pos, rope.cos, rope.sin, kc, vc, slots, H, **sc)
    proj = ops.gemv(x, w) if m <= 4 else ops.gemm_skinny(x, w)
    want = HipAttention.rope_and_cache(proj, pos, rope.cos, rope.sin, kc2, vc2, slots, H, **sc)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert torch.equal(kc.view(torch.uint8), kc2.view(torch.uint8))
    assert torch.equal(vc.view(torch.uint8), vc2.view(torch.uint8))
