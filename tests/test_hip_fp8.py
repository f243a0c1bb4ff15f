"""E4M3 KV cache on the GPU (the *_fp8 entry points through HipAttention) against the FP8
oracle (oracle/fp8.py):
  * the cache writes (write_kv, rope_and_cache) store PyTorch's
    (x.float() / scale).clamp(-448, 448).to(float8_e4m3fn) bit for bit;
  * attention over E4M3 caches matches the torch restatement of TorchAttention.forward run on
    the dequantized caches (e4m3 * scale, fp32) within the 16-bit bar (max-abs 2e-2), over the
    reference's parity cases, D = 128 mixed batches (the prefill kernel's E4M3 stages) and
    split decode segments;
  * every E4M3 byte reaches the output exactly (one-key sequences return V exactly).
"""

from __future__ import annotations

import dataclasses
import random

import pytest
import torch

from kvserve_amd import HipAttention, last_launch_kernels, workloads
from kvserve_amd.attention import AttentionMetadata
from kvserve_amd.engine import LLAMA_3_2_1B
from tests.engine_backends import rope as rope_table
from oracle import fp8, torch_reference
from tests import paged_check as pc

pytestmark = pytest.mark.gpu

FP8 = fp8.FP8


def _fp8_caches(b: workloads.PagedBatch, k_scale: float, v_scale: float):
    """The batch's random caches quantized (oracle, CPU) into E4M3 device tensors."""
    kc = fp8.quantize(b.k_cache, k_scale).to(b.k_cache.device)
    vc = fp8.quantize(b.v_cache, v_scale).to(b.v_cache.device)
    return kc, vc


def _oracle(b: workloads.PagedBatch, kc, vc, k_scale, v_scale):
    m = b.meta
    return torch_reference.forward(
        b.q.float().cpu(), fp8.dequantize(kc.cpu(), k_scale), fp8.dequantize(vc.cpu(), v_scale),
        m.block_tables.cpu(), m.seq_lens.cpu(), m.query_lens.cpu(), b.workload.scale,
    )  # fmt: skip


def _attend_fp8(b, kc, vc, k_scale, v_scale):
    HipAttention.write_kv(kc, vc, b.k_new, b.v_new, b.meta.slot_mapping, k_scale=k_scale, v_scale=v_scale)
    return HipAttention.forward(b.q, kc, vc, b.meta, b.workload.scale, k_scale=k_scale, v_scale=v_scale)


# -- cache writes ---------------------------------------------------------------------------------
def _special_values(n: int, dtype, gen) -> torch.Tensor:
    """Wide-range values: N(0, 1) x 10^U(-3, 3), exact E4M3 midpoints, signed zeros, values
    beyond the saturation bound."""
    x = torch.randn(n, generator=gen, device="cuda:0") * 10 ** (torch.rand(n, generator=gen, device="cuda:0") * 6 - 3)
    mids = torch.tensor([1.0625, 1.1875, 3 * 2.0**-11, 2.0**-10, 240.0, 432.0, -17.0, 464.0, 1e5, -0.0],
                        device="cuda:0")  # fmt: skip
    x[: mids.numel()] = mids
    return x.to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=str)
@pytest.mark.parametrize("k_scale,v_scale", [(1.0, 1.0), (0.37, 2.5)])
def test_write_kv_fp8_bit_exact(hip_device, dtype, k_scale, v_scale):
    gen = torch.Generator(device=hip_device).manual_seed(3)
    T, Hkv, D, NB, BS = 37, 8, 128, 64, 16
    k = _special_values(T * Hkv * D, dtype, gen).view(T, Hkv, D)
    wide = _special_values(T * (Hkv * D + 64), dtype, gen).view(T, Hkv * D + 64)
    v = wide[:, 64:].view(T, Hkv, D)  # a strided view, like the fused QKV output
    slots = torch.randperm(NB * BS, generator=gen, device=hip_device)[:T]
    slots[5] = NB * BS + 3  # outside the pool: skipped
    kc = torch.randint(0, 256, (NB, BS, Hkv, D), generator=gen, device=hip_device, dtype=torch.uint8).view(FP8)
    vc = torch.randint(0, 256, (NB, BS, Hkv, D), generator=gen, device=hip_device, dtype=torch.uint8).view(FP8)
    want_k, want_v = kc.view(torch.uint8).cpu().clone(), vc.view(torch.uint8).cpu().clone()
    ok = slots < NB * BS
    s_ok = slots[ok].cpu()
    want_k.view(-1, Hkv, D)[s_ok] = fp8.quantize(k[ok], k_scale).view(torch.uint8)
    want_v.view(-1, Hkv, D)[s_ok] = fp8.quantize(v[ok], v_scale).view(torch.uint8)
    HipAttention.write_kv(kc, vc, k, v, slots, k_scale=k_scale, v_scale=v_scale)
    torch.cuda.synchronize()
    assert torch.equal(kc.view(torch.uint8).cpu(), want_k)
    assert torch.equal(vc.view(torch.uint8).cpu(), want_v)


def test_write_kv_fp8_nan_stays_nan(hip_device):
    k = torch.full((1, 1, 16), float("nan"), device=hip_device, dtype=torch.bfloat16)
    kc = torch.zeros((1, 16, 1, 16), dtype=torch.uint8, device=hip_device).view(FP8)
    vc = torch.zeros_like(kc)
    HipAttention.write_kv(kc, vc, k, k, torch.zeros(1, dtype=torch.long, device=hip_device), k_scale=2.0)
    torch.cuda.synchronize()
    assert set(kc.view(torch.uint8)[0, 0, 0].tolist()) <= {0x7F, 0xFF}  # a NaN code (its sign is not specified)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=str)
def test_rope_and_cache_fp8_bit_exact(hip_device, dtype):
    H, Hkv, D, T, NB, BS = 32, 8, 128, 45, 64, 16
    k_scale, v_scale = 0.75, 1.5
    gen = torch.Generator(device=hip_device).manual_seed(11)
    qkv = (torch.randn(T, (H + 2 * Hkv) * D, generator=gen, device=hip_device) * 40).to(dtype)
    rope = rope_table(dataclasses.replace(LLAMA_3_2_1B, head_dim=D), 4096, device=hip_device)
    pos = torch.randint(0, 4096, (T,), generator=gen, device=hip_device)
    slots = torch.randperm(NB * BS, generator=gen, device=hip_device)[:T]
    kc = torch.zeros((NB, BS, Hkv, D), dtype=torch.uint8, device=hip_device).view(FP8)
    vc = torch.zeros_like(kc)
    q, k, v = qkv.split([H * D, Hkv * D, Hkv * D], dim=-1)
    want_q = torch_reference.rope(q.reshape(T, H, D), rope.cos, rope.sin, pos)
    k_rot = torch_reference.rope(k.reshape(T, Hkv, D), rope.cos, rope.sin, pos)
    want_k = torch.zeros((NB * BS, Hkv, D), dtype=torch.uint8)
    want_v = torch.zeros_like(want_k)
    want_k[slots.cpu()] = fp8.quantize(k_rot, k_scale).view(torch.uint8)
    want_v[slots.cpu()] = fp8.quantize(v.reshape(T, Hkv, D), v_scale).view(torch.uint8)
    got_q = HipAttention.rope_and_cache(qkv, pos, rope.cos, rope.sin, kc, vc, slots, H, k_scale=k_scale,
                                        v_scale=v_scale)  # fmt: skip
    torch.cuda.synchronize()
    assert torch.equal(got_q, want_q)
    assert torch.equal(kc.view(torch.uint8).cpu().view(-1, Hkv, D), want_k)
    assert torch.equal(vc.view(torch.uint8).cpu().view(-1, Hkv, D), want_v)


# -- attention ------------------------------------------------------------------------------------
@pytest.mark.parametrize("case", list(workloads.REFERENCE_CASES))
@pytest.mark.parametrize("heads", [(32, 8), (16, 16)], ids=lambda h: f"{h[0]}q{h[1]}kv")
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
def test_reference_cases_fp8(hip_device, case, heads, dtype):
    w = workloads.reference_case(case, *heads, head_dim=64, block_size=16, seed=0)
    b = workloads.materialize(w, dtype, hip_device, seed=0)
    k_scale, v_scale = 0.5, 0.25
    kc, vc = _fp8_caches(b, k_scale, v_scale)
    out = _attend_fp8(b, kc, vc, k_scale, v_scale)
    ref = _oracle(b, kc, vc, k_scale, v_scale)
    err = (out.float().cpu() - ref).abs().max().item()
    assert err <= pc.TOL_16BIT, f"{case} {heads} {dtype}: max abs err {err}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
def test_d128_mixed_batch_uses_the_prefill_kernel(hip_device, dtype):
    """Prefill-class sequences (q_len > 4 at G = 4) with cached context next to decode rows."""
    w = workloads.custom("fp8_mixed", [200, 1, 70, 1, 1, 33], [300, 900, 0, 2000, 17, 4000], 32, 8, 128, 16, seed=4)
    b = workloads.materialize(w, dtype, hip_device, seed=4)
    kc, vc = _fp8_caches(b, 1.0, 0.5)
    out = _attend_fp8(b, kc, vc, 1.0, 0.5)
    assert "prefill" in last_launch_kernels()
    err = (out.float().cpu() - _oracle(b, kc, vc, 1.0, 0.5)).abs().max().item()
    assert err <= pc.TOL_16BIT, err


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("draft", [5, 12, 16], ids=["2_tiles", "3_tiles", "4_tiles"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
def test_verify_tiles_fp8(hip_device, head_dim, draft, dtype):
    """Decode-class verify batches over E4M3 caches: two, three and four 16-row tiles per wave
    at both MFMA head sizes and both 16-bit query types."""
    w = workloads.custom("fp8_verify", [draft] * 6, [40, 700, 1900, 3, 1200, 260], 32, 8, head_dim, 16, seed=draft)
    b = workloads.materialize(w, dtype, hip_device, seed=draft)
    kc, vc = _fp8_caches(b, 0.5, 2.0)
    out = _attend_fp8(b, kc, vc, 0.5, 2.0)
    assert last_launch_kernels() == ["decode", "reduce"], last_launch_kernels()
    err = (out.float().cpu() - _oracle(b, kc, vc, 0.5, 2.0)).abs().max().item()
    assert err <= pc.TOL_16BIT, f"D {head_dim} draft {draft} {dtype}: {err}"


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
def test_short_tables_fp8(hip_device, head_dim, dtype):
    """Decode over tables of at most 1024 keys takes the single-launch short decode over E4M3
    caches too."""
    w = workloads.custom("fp8_short", [1] * 7, [0, 15, 200, 511, 999, 64, 700], 32, 8, head_dim, 16, seed=6)
    b = workloads.materialize(w, dtype, hip_device, seed=6)
    kc, vc = _fp8_caches(b, 1.0, 0.5)
    out = _attend_fp8(b, kc, vc, 1.0, 0.5)
    assert last_launch_kernels() == ["decode"], last_launch_kernels()
    err = (out.float().cpu() - _oracle(b, kc, vc, 1.0, 0.5)).abs().max().item()
    assert err <= pc.TOL_16BIT, f"D {head_dim} {dtype}: {err}"


def test_split_decode_segments(hip_device):
    """Long contexts next to a short one: the stream-K units split the long segments, whose
    pieces the merge kernel combines (and scales by v_scale); q_len 5 takes 2 row tiles."""
    w = workloads.custom("fp8_long", [1] * 3 + [5], [12000, 9000, 300, 7000], 32, 8, 128, 16, seed=5)
    b = workloads.materialize(w, torch.bfloat16, hip_device, seed=5)
    kc, vc = _fp8_caches(b, 2.0, 0.125)
    out = _attend_fp8(b, kc, vc, 2.0, 0.125)
    err = (out.float().cpu() - _oracle(b, kc, vc, 2.0, 0.125)).abs().max().item()
    assert err <= pc.TOL_16BIT, err


@pytest.mark.parametrize("idx", [2, 4, 5])
def test_baseline_configs_fp8(hip_device, idx):
    """BASELINE configs 2, 4 and 5 at full size over E4M3 caches: the single-tile decode with
    two dispatch rounds, the 32-row cascade groups, and the two-tile verify rows whose split
    pieces keep their partials in tile blocks. Any E4M3 content will do (the caches are cast on
    the device); the fp64 oracle reads the dequantized caches after the step's write, over
    sampled sequences."""
    w = workloads.baseline_config(idx, seed=0)
    b = workloads.materialize(w, torch.bfloat16, hip_device, seed=idx)
    ks, vs = 0.5, 2.0
    kc = (b.k_cache.float() / ks).clamp(-fp8.FP8_MAX, fp8.FP8_MAX).to(torch.float8_e4m3fn)
    vc = (b.v_cache.float() / vs).clamp(-fp8.FP8_MAX, fp8.FP8_MAX).to(torch.float8_e4m3fn)
    out = _attend_fp8(b, kc, vc, ks, vs)
    kinds = last_launch_kernels()
    torch.cuda.synchronize()
    assert kinds == (["share", "decode", "reduce"] if idx == 4 else ["decode", "reduce"]), kinds
    assert torch.isfinite(out.float()).all()
    deq = dataclasses.replace(b, k_cache=fp8.dequantize(kc, ks), v_cache=fp8.dequantize(vc, vs))
    seqs = list(range(0, len(w.query_lens), 4 if idx == 2 else 1))
    err = pc.max_err_vs_oracle(deq, out, seqs)
    print(f"config {idx} over E4M3: max abs err vs fp64 oracle {err:.3e}")
    assert err <= pc.TOL_16BIT, err


def test_partial_second_dispatch_round(hip_device):
    """Tables 4096 keys wide over contexts of 120-260 tokens: the decode launch is sized from
    the tables for two workgroups per CU (256 units, the first 128 in the first dispatch round),
    but the chunks give only ~210 units work, so part of the second round is active. Its units
    take the head halves the other way round and 3/4 of a first-round unit's share of the split;
    every chunk must still reach exactly one unit and every head its own rows."""
    rng = random.Random(17)
    ctx = [rng.randint(120, 260) for _ in range(64)]
    seq = [c + 1 for c in ctx]
    pool = 20_000
    tables = workloads._disjoint_tables(rng, seq, 16, pool)
    w = workloads.Workload("fp8_round2", [1] * 64, seq, tables, pool, 32, 8, 128, 16, width=256)
    b = workloads.materialize(w, torch.bfloat16, hip_device, seed=17)
    kc, vc = _fp8_caches(b, 0.5, 1.0)
    out = _attend_fp8(b, kc, vc, 0.5, 1.0)
    assert last_launch_kernels() == ["decode", "reduce"], last_launch_kernels()
    err = (out.float().cpu() - _oracle(b, kc, vc, 0.5, 1.0)).abs().max().item()
    assert err <= pc.TOL_16BIT, err


@pytest.mark.parametrize("D", [64, 128])
def test_every_code_reaches_the_output_exactly(hip_device, D):
    """Sequences of one key: the output is that key's V, e4m3 * v_scale, exact in bf16 for a
    power-of-two scale. The V rows hold all 254 finite codes."""
    Hkv, H, B, BS = 8, 8, 4, 16
    codes = torch.tensor([c for c in range(256) if c not in (0x7F, 0xFF)] + [0, 0x38], dtype=torch.uint8)
    vals = codes.repeat(-(-B * Hkv * D // codes.numel()))[: B * Hkv * D].view(B, Hkv, D)
    kc = torch.zeros((B, BS, Hkv, D), dtype=torch.uint8)
    vc = torch.zeros((B, BS, Hkv, D), dtype=torch.uint8)
    vc[:, 0] = vals
    kc[:, 0] = torch.randint(0, 0x70, (B, Hkv, D), dtype=torch.uint8)  # finite keys
    kc, vc = kc.to(hip_device).view(FP8), vc.to(hip_device).view(FP8)
    dev = hip_device
    meta = AttentionMetadata(
        slot_mapping=torch.empty(0, dtype=torch.long, device=dev),
        block_tables=torch.arange(B, device=dev).view(B, 1),
        seq_lens=torch.ones(B, dtype=torch.long, device=dev),
        query_lens=torch.ones(B, dtype=torch.long, device=dev),
        query_start_loc=torch.arange(B + 1, device=dev),
        max_seq_len=1,
        max_query_len=1,
    )
    q = torch.randn(B, H, D, device=dev).to(torch.bfloat16)
    out = HipAttention.forward(q, kc, vc, meta, D**-0.5, k_scale=0.5, v_scale=4.0)
    want = fp8.dequantize(vals.view(FP8), 4.0)  # [B, Hkv, D]; G = 1
    assert torch.equal(out.float().cpu(), want)


@pytest.mark.parametrize("D,BS", [(128, 32), (64, 64)])
def test_other_block_sizes(hip_device, D, BS):
    w = workloads.custom("fp8_bs", [1, 40, 1, 9], [100, 70, 3000, 0], 32, 8, D, BS, seed=6)
    b = workloads.materialize(w, torch.bfloat16, hip_device, seed=6)
    kc, vc = _fp8_caches(b, 0.75, 1.25)
    out = _attend_fp8(b, kc, vc, 0.75, 1.25)
    err = (out.float().cpu() - _oracle(b, kc, vc, 0.75, 1.25)).abs().max().item()
    assert err <= pc.TOL_16BIT, err


def test_decode_graph_replays_match_eager(hip_device):
    """write_kv + forward over E4M3 caches captured once (the decode graph's static buffers,
    cuda_graph.py:54-76) and replayed with new inputs: each replay equals an eager call bit
    for bit and the dequantized oracle within the 16-bit bar."""
    import random

    dev = hip_device
    H, Hkv, D, BS, NB, bucket, width_max = 32, 8, 128, 16, 900, 8, 128
    k_scale, v_scale = 0.5, 0.75
    gen = torch.Generator(device=dev).manual_seed(9)
    kc = fp8.quantize(torch.randn(NB + 1, BS, Hkv, D, generator=gen, device=dev), k_scale).to(dev)
    vc = fp8.quantize(torch.randn(NB + 1, BS, Hkv, D, generator=gen, device=dev), v_scale).to(dev)
    q = torch.zeros(bucket, H, D, device=dev, dtype=torch.bfloat16)
    k = torch.zeros(bucket, Hkv, D, device=dev, dtype=torch.bfloat16)
    v = torch.zeros(bucket, Hkv, D, device=dev, dtype=torch.bfloat16)
    meta = AttentionMetadata(
        slot_mapping=torch.full((bucket,), NB * BS, dtype=torch.long, device=dev),
        block_tables=torch.full((bucket, width_max), NB, dtype=torch.long, device=dev),
        seq_lens=torch.ones(bucket, dtype=torch.long, device=dev),
        query_lens=torch.ones(bucket, dtype=torch.long, device=dev),
        query_start_loc=torch.arange(bucket + 1, dtype=torch.long, device=dev),
        max_seq_len=1,
        max_query_len=1,
    )

    def step():
        HipAttention.write_kv(kc, vc, k, v, meta.slot_mapping, k_scale=k_scale, v_scale=v_scale)
        return HipAttention.forward(q, kc, vc, meta, D**-0.5, k_scale=k_scale, v_scale=v_scale)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()
    rng = random.Random(2)
    ids = list(range(NB))
    for it in range(4):
        n = rng.choice([2, 5, 8])
        lens = [rng.randint(1, 2000) for _ in range(n)]
        rng.shuffle(ids)
        tables, i = [], 0
        for L in lens:
            tables.append(ids[i : i + -(-L // BS)])
            i += len(tables[-1])
        width = max(len(t) for t in tables)
        rows = [t + [NB] * (width - len(t)) for t in tables] + [[NB] * width] * (bucket - n)
        slots = [t[(L - 1) // BS] * BS + (L - 1) % BS for t, L in zip(tables, lens)]
        q.copy_(torch.randn(bucket, H, D, generator=gen, device=dev).to(torch.bfloat16))
        k.copy_(torch.randn(bucket, Hkv, D, generator=gen, device=dev).to(torch.bfloat16))
        v.copy_(torch.randn(bucket, Hkv, D, generator=gen, device=dev).to(torch.bfloat16))
        meta.slot_mapping.copy_(torch.tensor(slots + [NB * BS] * (bucket - n)))
        meta.seq_lens.copy_(torch.tensor(lens + [1] * (bucket - n)))
        meta.block_tables[:, :width].copy_(torch.tensor(rows))
        graph.replay()
        replayed = out.clone()
        torch.cuda.synchronize()
        eager = HipAttention.forward(q, kc, vc, meta, D**-0.5, k_scale=k_scale, v_scale=v_scale)
        torch.cuda.synchronize()
        assert torch.equal(replayed.view(torch.int16), eager.view(torch.int16)), it
        ref = torch_reference.forward(
            q[:n].float().cpu(), fp8.dequantize(kc.cpu(), k_scale), fp8.dequantize(vc.cpu(), v_scale),
            meta.block_tables[:n].cpu(), meta.seq_lens[:n].cpu(), torch.ones(n, dtype=torch.long), D**-0.5,
        )  # fmt: skip
        assert (replayed[:n].float().cpu() - ref).abs().max().item() <= pc.TOL_16BIT, it
