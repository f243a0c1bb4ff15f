"""kvh_paged_attention_static (the entry point that allocates nothing) against kvh_paged_attention.

Both entry points run the same kernels on the same inputs; the static one takes its split-K
workspace from the library's device-resident scratch instead of a caller's buffer, so the
outputs must be equal bit for bit. Two calls in a row, the second on a smaller batch, check
that nothing a call leaves in the shared scratch leaks into the next one; a graph-free decode
batch, a speculative-verify batch (two 16-row tiles per kv head), a shared-prefix cascade
batch and a mixed prefill + decode batch cover every workspace region. The oversized case is
rejected before any GPU work.
"""

import ctypes
import random

import pytest
import torch

from kvserve_amd import HipAttention, _lib, last_launch_kernels, workloads
from tests import paged_check as pc
from tests.test_hip_cascade import shared_workload

pytestmark = pytest.mark.gpu

E_SCRATCH = -7


def _static_call(b, out: torch.Tensor) -> int:
    """kvh_paged_attention_static through the C ABI on the batch's current stream."""
    w, m = b.workload, b.meta
    kc, vc, q = b.k_cache, b.v_cache, b.q
    return _lib.load().kvh_paged_attention_static(
        q.data_ptr(), q.stride(0), q.stride(1),
        kc.data_ptr(), _lib.i64x3(kc.stride()[:3]), vc.data_ptr(), _lib.i64x3(vc.stride()[:3]), kc.shape[0],
        out.data_ptr(), out.stride(0), out.stride(1),
        m.block_tables.data_ptr(), m.block_tables.stride(0), m.block_tables.shape[1],
        m.seq_lens.data_ptr(), m.query_start_loc.data_ptr(),
        q.shape[0], m.block_tables.shape[0], w.num_heads, w.num_kv_heads, w.head_dim, w.block_size,
        int(m.max_query_len), float(w.scale), _lib.KVH_DTYPE[q.dtype],
        torch.cuda.current_stream().cuda_stream,
    )  # fmt: skip


def _both(b) -> tuple[torch.Tensor, torch.Tensor, list[str]]:
    HipAttention.write_kv(b.k_cache, b.v_cache, b.k_new, b.v_new, b.meta.slot_mapping)
    ref = HipAttention.forward(b.q, b.k_cache, b.v_cache, b.meta, b.workload.scale)
    kinds = last_launch_kernels()
    out = torch.full_like(b.q, float("nan"))
    st = _static_call(b, out)
    assert st == 0, _lib.strerror(st)
    torch.cuda.synchronize()
    return ref, out, kinds


def _pair(large, small, dtype, device, expect_kind=None):
    for seed, w in enumerate((large, small)):
        print(f"no-alloc: {w.name} seqs={len(w.query_lens)} tokens={w.num_tokens} dtype={dtype}", flush=True)
        b = workloads.materialize(w, dtype, device, seed=seed)
        ref, out, kinds = _both(b)
        if expect_kind is not None:
            assert expect_kind in kinds, kinds
        assert torch.equal(ref.view(torch.int16), out.view(torch.int16)), f"{w.name}: static != workspace call"
        # and both meet the oracle bar (sampled rows)
        seqs = list(range(0, len(w.query_lens), max(1, len(w.query_lens) // 8)))
        err = pc.max_err_vs_oracle(b, out, seqs, rows_per_seq=16)
        assert err <= pc.TOL_16BIT, f"{w.name}: {err}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
def test_static_decode_then_smaller(hip_device, dtype):
    rng = random.Random(3)
    big = workloads.custom("dec64", [1] * 64, [rng.randint(200, 3000) for _ in range(64)], 32, 8, 128, 16, seed=3)
    small = workloads.custom("dec5", [1] * 5, [17, 900, 1, 64, 2500], 32, 8, 128, 16, seed=4)
    _pair(big, small, dtype, hip_device, expect_kind="decode")


def test_static_verify_then_smaller(hip_device):
    big = workloads.custom("verify32", [5] * 32, [2048 + 61 * i for i in range(32)], 32, 8, 128, 16, seed=5)
    small = workloads.custom("verify3", [5, 2, 5], [700, 40, 5], 32, 8, 128, 16, seed=6)
    _pair(big, small, torch.bfloat16, hip_device)


def test_static_cascade_then_smaller(hip_device):
    """Shared table prefixes on long tables: the share kernel and the prefix partials."""
    rng = random.Random(7)
    big = shared_workload([1] * 16, [rng.randint(1700, 3000) for _ in range(16)], (32, 8), 128, 16, 100, 600, seed=7)
    small = shared_workload([1] * 4, [900, 1500, 2000, 1300], (32, 8), 128, 16, 50, 600, seed=8)
    _pair(big, small, torch.bfloat16, hip_device, expect_kind="share")


def test_static_mixed_then_smaller(hip_device):
    """Prefill-class and decode sequences in one batch: prefill partials and the plan (at the
    size of the 2048-token mixed step: 512 decodes and 4 prefill chunks of 384)."""
    big = workloads.baseline_config(3, seed=0)
    small = workloads.custom("mixed_small", [1, 80], [20, 500], 32, 8, 128, 16, seed=10)
    _pair(big, small, torch.bfloat16, hip_device, expect_kind="prefill")


def test_static_entry_captured_in_a_graph(hip_device):
    """kvh_paged_attention_static captured in a HIP graph and replayed over fresh queries and
    edited sequence lengths: every replay equals the workspace call on the same inputs bit for
    bit, with eager work and synchronisations between replays. One eager call on the device
    comes first (it resolves the scratch's device address and the occupancy the launches are
    sized by, neither of which is a stream operation to record)."""
    w = workloads.custom("graph_mixed", [1, 1, 80, 5, 1], [300, 2000, 500, 900, 17], 32, 8, 128, 16, seed=31)
    b = workloads.materialize(w, torch.bfloat16, hip_device, seed=31)
    HipAttention.write_kv(b.k_cache, b.v_cache, b.k_new, b.v_new, b.meta.slot_mapping)
    out = torch.full_like(b.q, float("nan"))
    assert _static_call(b, out) == 0
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        st = _static_call(b, out)
    assert st == 0, _lib.strerror(st)
    gen = torch.Generator(device=hip_device).manual_seed(5)
    base_len = b.meta.seq_lens.clone()
    for rep in (1, 2, 3, 0):  # the last replay with the workload's own lengths, for the oracle
        print(f"no-alloc graph replay {rep}", flush=True)
        b.q.copy_(torch.randn(b.q.shape, generator=gen, device=hip_device).to(b.q.dtype))
        b.meta.seq_lens.copy_(base_len)
        b.meta.seq_lens[1] -= 400 * rep  # the long decode sequence sees fewer keys
        out.fill_(float("nan"))
        graph.replay()
        ref = HipAttention.forward(b.q, b.k_cache, b.v_cache, b.meta, w.scale)
        torch.cuda.synchronize()
        assert torch.equal(ref.view(torch.int16), out.view(torch.int16)), f"replay {rep}"
    err = pc.max_err_vs_oracle(b, out, list(range(len(w.query_lens))), rows_per_seq=16)
    assert err <= pc.TOL_16BIT, err


def test_static_rejects_oversized_launch(hip_device):
    """A launch whose workspace exceeds the static scratch (256 MiB) is rejected with
    KVH_E_SCRATCH before any GPU work: a mixed step of 2000 decode sequences and 4 prefills."""
    lib = _lib.load()
    ws = lib.kvh_paged_attention_workspace_size(2500, 2004, 32, 8, 128, 280, 16, 384, 2)
    assert ws > (256 << 20)
    assert lib.kvh_paged_attention_workspace_size(2048, 516, 32, 8, 128, 280, 16, 384, 2) <= (256 << 20)
    dummy = ctypes.c_void_p(0x1000)
    st = lib.kvh_paged_attention_static(
        dummy, 4096, 128, dummy, _lib.i64x3((16384, 1024, 128)), dummy, _lib.i64x3((16384, 1024, 128)), 70_000,
        dummy, 4096, 128, dummy, 280, 280, dummy, dummy, 2500, 2004, 32, 8, 128, 16, 384, 128**-0.5, 2, None,
    )  # fmt: skip
    assert st == E_SCRATCH
    assert "static scratch" in _lib.strerror(st)
