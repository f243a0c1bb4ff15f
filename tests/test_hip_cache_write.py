"""reshape_and_cache on the GPU vs the oracle, bit for bit (GPU).

Semantics: TorchAttention.write_kv (src/kvserve/attention.py:39-45). Bar: bit-exact.
"""

import numpy as np
import pytest
import torch

import oracle
from kvserve_amd import HipAttention

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.contiguous().cpu()
    return t.view(torch.int16 if t.element_size() == 2 else torch.int32).numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=str)
@pytest.mark.parametrize("shape", [(2048, 8, 128, 16), (37, 8, 64, 16), (5, 2, 12, 4), (9, 3, 5, 4)], ids=str)
def test_write_matches_oracle(hip_device, dtype, shape):
    T, Hkv, D, BS = shape
    NB = T // BS + 11
    g = torch.Generator(device=hip_device).manual_seed(T)
    kc = torch.randn(NB, BS, Hkv, D, generator=g, device=hip_device).to(dtype)
    vc = torch.randn(NB, BS, Hkv, D, generator=g, device=hip_device).to(dtype)
    # v as a strided view of a fused projection output, like model.py:89-92
    fused = torch.randn(T, 3, Hkv, D, generator=g, device=hip_device).to(dtype)
    k, v = fused[:, 0], fused[:, 2]
    slots = torch.randperm(NB * BS, generator=torch.Generator().manual_seed(T))[:T].to(hip_device)
    kc_ref, vc_ref = _bits(kc).copy(), _bits(vc).copy()
    HipAttention.write_kv(kc, vc, k, v, slots)
    oracle.reshape_and_cache(_bits(k), _bits(v), slots.cpu().numpy(), kc_ref, vc_ref)
    assert np.array_equal(_bits(kc), kc_ref)
    assert np.array_equal(_bits(vc), vc_ref)


def test_duplicate_and_out_of_range_slots(hip_device):
    """Graph padding rows all write one scratch slot (cuda_graph.py:57,127): the slot ends up
    holding, chunk by chunk, the data of the duplicates. Slots outside the pool are skipped."""
    T, Hkv, D, BS, NB = 12, 8, 128, 16, 6
    kc = torch.zeros(NB, BS, Hkv, D, device=hip_device, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    k = torch.randn(T, Hkv, D, device=hip_device).to(torch.bfloat16)
    v = torch.randn(T, Hkv, D, device=hip_device).to(torch.bfloat16)
    scratch = (NB - 1) * BS
    slots = torch.tensor([3, 17, scratch, scratch, scratch, -1, NB * BS, 40, scratch, 2, 50, 1 << 40],
                         device=hip_device)  # fmt: skip
    HipAttention.write_kv(kc, vc, k, v, slots)
    flat_k, flat_v = kc.view(-1, Hkv, D), vc.view(-1, Hkv, D)
    for t, s in enumerate(slots.tolist()):
        if 0 <= s < NB * BS and s != scratch:
            assert torch.equal(flat_k[s].view(torch.int16), k[t].view(torch.int16))
            assert torch.equal(flat_v[s].view(torch.int16), v[t].view(torch.int16))
    # concurrent writes of one slot race; each 16-byte vector store is whole, so every
    # 8-element chunk of the slot is that chunk of one of the duplicates
    dup = [t for t, s in enumerate(slots.tolist()) if s == scratch]
    for cache, src in ((flat_k, k), (flat_v, v)):
        got = cache[scratch].view(torch.int16).reshape(-1, 8)
        cands = torch.stack([src[t].view(torch.int16).reshape(-1, 8) for t in dup])  # [dups, chunks, 8]
        assert (cands == got).all(dim=-1).any(dim=0).all()
    written = {s for s in slots.tolist() if 0 <= s < NB * BS}
    untouched = [i for i in range(NB * BS) if i not in written]
    assert torch.count_nonzero(flat_k[untouched].float()) == 0
    assert torch.count_nonzero(flat_v[untouched].float()) == 0
