"""HIP paged attention vs the oracle (GPU). Calls go through the C ABI via HipAttention.

Mirrors the reference's parity suite (tests/test_triton_attention.py:55-86: CASES x heads x
dtype at D=64/BS=16, plus D=128/BS=32) and adds the five BASELINE configs at full size,
the committed golden fixtures, the exact-fp32 path and the edge cases of the contract.
Tolerance: max-abs <= 2e-2 for bf16/fp16 storage against the oracle on the same rounded
inputs (stricter than the reference's atol=rtol=2e-2), 1e-4 for the fp32 path.
"""

import random

import numpy as np
import pytest
import torch

from kvserve_amd import HipAttention, last_launch_kernels, workloads
from kvserve_amd.attention import AttentionMetadata
from tests import paged_check as pc
from tests.golden.make_golden import load_fixtures

pytestmark = pytest.mark.gpu

HEADS = [(32, 8), (16, 16), (32, 4)]
DTYPES = [torch.bfloat16, torch.float16]


@pytest.mark.parametrize("case", list(workloads.REFERENCE_CASES))
@pytest.mark.parametrize("heads", HEADS, ids=lambda h: f"{h[0]}q{h[1]}kv")
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_reference_cases(hip_device, case, heads, dtype):
    w = workloads.reference_case(case, *heads, head_dim=64, block_size=16, seed=0)
    b = workloads.materialize(w, dtype, hip_device, seed=0)
    out = pc.attend(b)
    assert pc.written_rows_match(b)
    ref = pc.torch_oracle_full(b)
    err = (out.float().cpu() - ref).abs().max().item()
    assert err <= pc.TOL_16BIT, f"{case} {heads} {dtype}: max abs err {err}"


@pytest.mark.parametrize("draft", [12, 16], ids=["48_rows", "64_rows"])
def test_long_verify_keeps_every_wave(hip_device, draft):
    """Speculative verify of 12 and 16 draft tokens (48 / 64 query rows per kv head: the
    three- and four-tile decode kernels, which fit one wave per SIMD, so the launch keeps
    every resident wave) at C5's size: 32 sequences over 2048-4096 cached tokens, against the
    fp64 oracle on every sequence."""
    rng = random.Random(draft)
    ctx = [rng.randint(2048, 4096) for _ in range(32)]
    w = workloads.custom(f"verify{draft}", [draft] * 32, ctx, 32, 8, 128, 16, seed=draft)
    b = workloads.materialize(w, torch.bfloat16, hip_device, seed=draft)
    out = pc.attend(b)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    assert last_launch_kernels() == ["decode", "reduce"], last_launch_kernels()
    err = pc.max_err_vs_oracle(b, out, list(range(32)))
    assert err <= pc.TOL_16BIT, err


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("draft", [5, 12, 16], ids=["2_tiles", "3_tiles", "4_tiles"])
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_verify_tiles_each_head_size(hip_device, head_dim, draft, dtype):
    """Decode-class verify batches (draft x G = 4 rows per kv head: two, three and four 16-row
    tiles per wave) at both MFMA head sizes and both 16-bit types, against the torch oracle."""
    w = workloads.custom("verify_d", [draft] * 6, [40, 700, 1900, 3, 1200, 260], 32, 8, head_dim, 16, seed=draft)
    b = workloads.materialize(w, dtype, hip_device, seed=draft)
    out = pc.attend(b)
    assert last_launch_kernels() == ["decode", "reduce"], last_launch_kernels()
    err = (out.float().cpu() - pc.torch_oracle_full(b)).abs().max().item()
    assert err <= pc.TOL_16BIT, f"D {head_dim} draft {draft} {dtype}: {err}"


def test_head_dim_128_and_block_32(hip_device):
    w = workloads.custom("d128_bs32", [1, 9, 1], [80, 40, 1000], 32, 8, 128, 32, seed=0)
    b = workloads.materialize(w, torch.bfloat16, hip_device)
    out = pc.attend(b)
    err = (out.float().cpu() - pc.torch_oracle_full(b)).abs().max().item()
    assert err <= pc.TOL_16BIT, err


def test_golden_fixtures(hip_device):
    for name, fx in load_fixtures().items():
        q = torch.from_numpy(fx["q_bits"].view(np.int16)).view(torch.bfloat16).to(hip_device)
        kc = torch.from_numpy(fx["k_bits"].view(np.int16)).view(torch.bfloat16).to(hip_device)
        vc = torch.from_numpy(fx["v_bits"].view(np.int16)).view(torch.bfloat16).to(hip_device)
        qsl = torch.from_numpy(fx["query_start_loc"]).to(hip_device)
        meta = AttentionMetadata(
            slot_mapping=torch.empty(0, dtype=torch.long, device=hip_device),
            block_tables=torch.from_numpy(fx["block_tables"]).to(hip_device),
            seq_lens=torch.from_numpy(fx["seq_lens"]).to(hip_device),
            query_lens=(qsl[1:] - qsl[:-1]),
            query_start_loc=qsl,
            max_seq_len=int(fx["seq_lens"].max()),
            max_query_len=int(np.diff(fx["query_start_loc"]).max()),
        )
        out = HipAttention.forward(q, kc, vc, meta, float(fx["scale"]))
        err = np.abs(out.double().cpu().numpy() - fx["out"]).max()
        assert err <= pc.TOL_16BIT, f"{name}: {err}"


@pytest.mark.parametrize("case", list(workloads.REFERENCE_CASES))
def test_fp32_path(hip_device, case):
    w = workloads.reference_case(case, 32, 8, head_dim=64, block_size=16, seed=1)
    b = workloads.materialize(w, torch.float32, hip_device, seed=1)
    out = pc.attend(b)
    assert last_launch_kernels() == ["f32"]
    err = pc.max_err_vs_oracle(b, out, list(range(len(w.query_lens))))
    assert err <= pc.TOL_F32, err


@pytest.mark.parametrize("head_dim", [160, 256])
def test_fp32_head_dims_above_128(hip_device, head_dim):
    """The exact-fp32 path at head sizes past 128 (four elements per lane)."""
    w = workloads.reference_case("mixed", 32, 8, head_dim=head_dim, block_size=16, seed=5)
    b = workloads.materialize(w, torch.float32, hip_device, seed=5)
    out = pc.attend(b)
    assert last_launch_kernels() == ["f32"]
    err = pc.max_err_vs_oracle(b, out, list(range(len(w.query_lens))))
    assert err <= pc.TOL_F32, err


def test_fp32_any_block_size(hip_device):
    """The exact-fp32 path serves the reference's CPU-only block sizes too (e.g. 4)."""
    w = workloads.custom("bs4", [3, 1, 7], [9, 30, 0], 8, 2, 64, 4, seed=2)
    b = workloads.materialize(w, torch.float32, hip_device, seed=2)
    out = pc.attend(b)
    assert pc.max_err_vs_oracle(b, out, [0, 1, 2]) <= pc.TOL_F32


@pytest.mark.parametrize("kind", ["q_x8", "outlier_channels"])
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_sharp_softmax_large_scores(hip_device, kind, dtype):
    """Large scores (a sharp softmax, as attention sinks and outlier channels give real models):
    q scaled by 8 (scores up to ~50 in log2 units), or four channels of q and of every key
    scaled by 16 and 4. Decode, verify and prefill rows (the stream-K decode and the prefill
    kernel) against the fp64 oracle at the 16-bit tolerance: the softmax scale is applied in
    fp32, never rounded into a 16-bit operand."""
    w = workloads.custom("sharp", [1, 5, 384, 200, 1], [2000, 1500, 1000, 0, 3000], 32, 8, 128, 16, seed=21)
    b = workloads.materialize(w, dtype, hip_device, seed=21)
    if kind == "q_x8":
        b.q.mul_(8)
    else:
        b.q[..., :4] *= 16
        b.k_new[..., :4] *= 4
        b.k_cache[..., :4] *= 4
    out = pc.attend(b)
    assert "prefill" in last_launch_kernels()
    err = pc.max_err_vs_oracle(b, out, list(range(len(w.query_lens))), rows_per_seq=64)
    assert err <= pc.TOL_16BIT, f"{kind} {dtype}: max abs err {err}"


@pytest.mark.parametrize("case", list(workloads.REFERENCE_CASES))
@pytest.mark.parametrize("head_dim", [32, 80, 96, 256])
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_head_sizes_outside_the_mfma_tiles(hip_device, case, head_dim, dtype):
    """Head sizes other than 64 and 128 (the reference pads any head size to a power of two and
    masks it, kernels/paged_attention.py:64-67,154) run on the vector-ALU kernel: the
    reference's CASES against the torch oracle at the 16-bit tolerance."""
    w = workloads.reference_case(case, 32, 8, head_dim=head_dim, block_size=16, seed=3)
    b = workloads.materialize(w, dtype, hip_device, seed=3)
    out = pc.attend(b)
    assert last_launch_kernels() == ["valu16"]
    assert pc.written_rows_match(b)
    err = (out.float().cpu() - pc.torch_oracle_full(b)).abs().max().item()
    assert err <= pc.TOL_16BIT, f"{case} D={head_dim} {dtype}: max abs err {err}"


@pytest.mark.parametrize(
    "heads,block_size",
    [((32, 8), 8), ((32, 8), 24), ((128, 1), 16)],
    ids=["bs8", "bs24", "g128"],
)
def test_pages_and_groups_outside_the_mfma_tiles(hip_device, heads, block_size):
    """Pages that are not whole 16-token tiles, and GQA groups above 64 query heads, run on the
    vector-ALU kernel at D = 128: decode, verify and prefill rows against the torch oracle."""
    w = workloads.custom("odd_pages", [1, 5, 37, 1], [300, 64, 100, 0], *heads, 128, block_size, seed=4)
    b = workloads.materialize(w, torch.bfloat16, hip_device, seed=4)
    out = pc.attend(b)
    assert last_launch_kernels() == ["valu16"]
    err = (out.float().cpu() - pc.torch_oracle_full(b)).abs().max().item()
    assert err <= pc.TOL_16BIT, f"{heads} BS={block_size}: {err}"


@pytest.mark.parametrize("idx", [1, 2, 3, 4, 5])
def test_baseline_configs(hip_device, idx):
    """BASELINE configs at full size: write + attend, then the fp64 oracle on sampled
    sequences/rows, plus size-independent properties (finite output, written rows exact)."""
    w = workloads.baseline_config(idx, seed=0)
    b = workloads.materialize(w, torch.bfloat16, hip_device, seed=idx)
    out = pc.attend(b)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    assert pc.written_rows_match(b)
    nseq = len(w.query_lens)
    if idx == 3:  # 512 decodes then 4 prefills: sample decodes, all prefills at 24 rows
        seqs = list(range(0, 512, 16)) + [511, 512, 513, 514, 515]
        err = pc.max_err_vs_oracle(b, out, seqs, rows_per_seq=24)
    else:
        seqs = list(range(nseq)) if nseq <= 64 else list(range(0, nseq, 4))
        err = pc.max_err_vs_oracle(b, out, seqs)
    print(f"config {idx}: max abs err vs fp64 oracle {err:.3e}; kernels {last_launch_kernels()}")
    assert err <= pc.TOL_16BIT, err
    if idx == 4:  # the 750 shared blocks go through the cascade's prefix segments
        assert last_launch_kernels()[0] == "share"


def test_out_argument_and_strided_inputs(hip_device):
    """out= a slice of a larger static buffer (piecewise mode, cuda_graph.py:240); q and v
    strided views of a fused QKV output (model.py:89-92)."""
    H, Hkv, D = 32, 8, 128
    w = workloads.custom("strided", [1, 5, 1, 30], [100, 60, 7, 0], H, Hkv, D, 16, seed=3)
    b = workloads.materialize(w, torch.bfloat16, hip_device, seed=3)
    T = w.num_tokens
    qkv = torch.randn(T, (H + 2 * Hkv) * D, device=hip_device, dtype=torch.bfloat16)
    q, k, v = qkv.split([H * D, Hkv * D, Hkv * D], dim=-1)
    q, k, v = q.view(T, H, D), k.view(T, Hkv, D), v.view(T, Hkv, D)
    assert not q.is_contiguous() and not v.is_contiguous()
    kc2, vc2 = b.k_cache.clone(), b.v_cache.clone()
    HipAttention.write_kv(b.k_cache, b.v_cache, k, v, b.meta.slot_mapping)
    HipAttention.write_kv(kc2, vc2, k.contiguous(), v.contiguous(), b.meta.slot_mapping)
    assert torch.equal(b.k_cache.view(torch.int16), kc2.view(torch.int16))
    assert torch.equal(b.v_cache.view(torch.int16), vc2.view(torch.int16))
    static = torch.full((T + 7, H, D), float("nan"), device=hip_device, dtype=torch.bfloat16)
    dst = static[:T]
    ret = HipAttention.forward(q, b.k_cache, b.v_cache, b.meta, w.scale, out=dst)
    assert ret is dst
    ref = HipAttention.forward(q.contiguous(), b.k_cache, b.v_cache, b.meta, w.scale)
    assert torch.equal(dst.view(torch.int16), ref.view(torch.int16))
    assert torch.isnan(static[T:].float()).all()  # nothing written past the real rows
    b.q = q
    assert pc.max_err_vs_oracle(b, dst, [0, 1, 2, 3]) <= pc.TOL_16BIT


def test_stale_slots_and_columns_never_read(hip_device):
    """Slots past seq_len hold NaN, and table columns past ceil(seq_len / BS) point at
    all-NaN blocks (stale graph rows, cuda_graph.py:129-134): the output stays exact."""
    H, Hkv, D, BS = 32, 8, 128, 16
    w = workloads.custom("stale", [1, 1, 3, 1], [40, 511, 77, 4000], H, Hkv, D, BS, seed=4, spare_blocks=16)
    b = workloads.materialize(w, torch.bfloat16, hip_device, seed=4)
    used = set()
    for t, s in zip(w.tables, w.seq_lens):
        nblk = -(-s // BS)
        used.update(t[:nblk])
        last = t[nblk - 1]
        tail = s - (nblk - 1) * BS
        b.k_cache[last, tail:] = float("nan")
        b.v_cache[last, tail:] = float("nan")
    spare = [i for i in range(w.num_blocks) if i not in used]
    b.k_cache[spare] = float("nan")
    b.v_cache[spare] = float("nan")
    width = w.table_width() + 64
    bt = torch.tensor(spare[:1], device=hip_device).repeat(len(w.tables), width)
    for i, t in enumerate(w.tables):
        bt[i, : len(t)] = torch.tensor(t)
    b.meta.block_tables = bt
    out = pc.attend(b)
    assert torch.isfinite(out.float()).all()
    assert pc.max_err_vs_oracle(b, out, [0, 1, 2, 3]) <= pc.TOL_16BIT


@pytest.mark.parametrize("heads", [(32, 8), (16, 16), (32, 2), (64, 4)], ids=lambda h: f"{h[0]}q{h[1]}kv")
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_short_tables_take_the_single_launch_decode(hip_device, heads, head_dim, dtype):
    """Decode batches over block tables of at most 1024 keys (the 1B decode config's shape) run
    one launch: a workgroup per (sequence, kv head) whose 4 waves split the chunks and combine
    their partials in LDS. Contexts from 0 to the table's end, so some waves see no chunk.
    Against the torch oracle, and against the stream-K kernels + merge on the same batch seen
    through a table 4x wider (within accumulation rounding)."""
    ctx = [0, 1, 31, 32, 33, 95, 96, 200, 511, 1023]
    w = workloads.custom("short", [1] * len(ctx), ctx, *heads, head_dim, 16, seed=13)
    b = workloads.materialize(w, dtype, hip_device, seed=13)
    assert b.meta.block_tables.shape[1] == 64
    out = pc.attend(b)
    assert last_launch_kernels() == ["decode"]
    err = (out.float().cpu() - pc.torch_oracle_full(b)).abs().max().item()
    assert err <= pc.TOL_16BIT, f"{heads} D={head_dim}: {err}"
    bt = torch.zeros(len(ctx), 256, dtype=torch.long, device=hip_device)
    bt[:, :64] = b.meta.block_tables
    b.meta.block_tables = bt
    wide = HipAttention.forward(b.q, b.k_cache, b.v_cache, b.meta, w.scale)
    assert "reduce" in last_launch_kernels()
    assert (out.float() - wide.float()).abs().max().item() <= 1e-2


def test_split_k_matches_single_pass(hip_device):
    """The same batch with a wide table (split-K partitions + log-sum-exp reduce) and a
    narrow one (one partition per sequence) agree within accumulation rounding."""
    w = workloads.custom("split", [1] * 8, [4000, 17, 900, 2047, 3, 1500, 64, 3999], 32, 8, 128, 16, seed=5)
    b = workloads.materialize(w, torch.bfloat16, hip_device, seed=5)
    HipAttention.write_kv(b.k_cache, b.v_cache, b.k_new, b.v_new, b.meta.slot_mapping)
    narrow = HipAttention.forward(b.q, b.k_cache, b.v_cache, b.meta, w.scale)
    k_narrow = last_launch_kernels()
    bt = torch.zeros(8, 8192, dtype=torch.long, device=hip_device)
    bt[:, : b.meta.block_tables.shape[1]] = b.meta.block_tables
    b.meta.block_tables = bt
    wide = HipAttention.forward(b.q, b.k_cache, b.v_cache, b.meta, w.scale)
    k_wide = last_launch_kernels()
    assert "reduce" in k_wide, k_wide
    assert (narrow.float() - wide.float()).abs().max().item() <= 1e-2
    assert pc.max_err_vs_oracle(b, wide, list(range(8))) <= pc.TOL_16BIT
    print("narrow:", k_narrow, "wide:", k_wide)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_partial_second_dispatch_round(hip_device, dtype):
    """D = 64, 16-bit caches: the decode kernel fits two workgroups per CU, so a launch sized
    from 4096-key tables holds two dispatch rounds of units; contexts of 120-260 tokens give
    only part of the second round work. Second-round units take the two halves of the 8-head
    group the other way round from first-round units; every head must still get its own rows
    (TorchAttention reads each sequence on its own, src/kvserve/attention.py:31-82)."""
    rng = random.Random(23)
    seq = [rng.randint(120, 260) + 1 for _ in range(64)]
    pool = 20_000
    tables = workloads._disjoint_tables(rng, seq, 16, pool)
    w = workloads.Workload("round2", [1] * 64, seq, tables, pool, 32, 8, 64, 16, width=256)
    b = workloads.materialize(w, dtype, hip_device, seed=23)
    out = pc.attend(b)
    assert last_launch_kernels() == ["decode", "reduce"], last_launch_kernels()
    assert pc.max_err_vs_oracle(b, out, list(range(64))) <= pc.TOL_16BIT


def test_mixed_batch_dispatch(hip_device):
    """Decode-class rows take the stream-K decode kernel and longer queries the prefill
    kernel (whose work plan the decode launch lays out), all launched over the same
    metadata with no host synchronisation."""
    w = workloads.reference_case("mixed", 32, 8, head_dim=128, block_size=16)
    b = workloads.materialize(w, torch.bfloat16, hip_device)
    out = pc.attend(b)
    kinds = last_launch_kernels()
    assert kinds == ["decode", "prefill", "reduce"], kinds
    assert pc.max_err_vs_oracle(b, out, list(range(5))) <= pc.TOL_16BIT
    dec = workloads.reference_case("decode", 32, 8, head_dim=128, block_size=16)
    bd = workloads.materialize(dec, torch.bfloat16, hip_device)
    pc.attend(bd)
    assert "prefill" not in last_launch_kernels()


@pytest.mark.parametrize(
    ("heads", "q_lens", "ctx_lens"),
    [
        ((32, 8), [1, 130, 3, 700, 33, 1], [50, 0, 4000, 1000, 3000, 9]),  # G=4, ragged tiles
        ((16, 16), [65, 1, 200], [0, 300, 2500]),  # G=1: prefill from 17 queries per sequence
        ((32, 2), [8, 1], [30_000, 70]),  # G=16: one tile per kv head, split over ~256 units
        ((32, 4), [4096], [0]),  # one long prompt, causal from key 0
    ],
    ids=["g4_ragged", "g1", "g16_long_ctx", "g8_long_prompt"],
)
def test_prefill_stream_k(hip_device, heads, q_lens, ctx_lens):
    """Prefill-class sequences go through the stream-K prefill kernel: tiles cut between
    work units (including tiles merged from more than 16 pieces) match the oracle."""
    H, Hkv = heads
    w = workloads.custom("pre_sk", q_lens, ctx_lens, H, Hkv, 128, 16, seed=7)
    b = workloads.materialize(w, torch.bfloat16, hip_device, seed=7)
    out = pc.attend(b)
    kinds = last_launch_kernels()
    assert "prefill" in kinds and "reduce" in kinds, kinds
    assert torch.isfinite(out.float()).all()
    err = pc.max_err_vs_oracle(b, out, list(range(len(q_lens))), rows_per_seq=16)
    assert err <= pc.TOL_16BIT, err


def test_prefill_is_deterministic(hip_device):
    """Two calls on the same inputs give bit-identical outputs (fixed unit ranges and merge
    order; no atomics)."""
    w = workloads.custom("pre_det", [300, 1, 77], [2000, 500, 0], 32, 8, 128, 16, seed=8)
    b = workloads.materialize(w, torch.bfloat16, hip_device, seed=8)
    o1 = pc.attend(b)
    o2 = HipAttention.forward(b.q, b.k_cache, b.v_cache, b.meta, w.scale)
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))


def test_rows_without_keys_write_zeros(hip_device):
    """seq_len < q_len leaves early rows with no visible key: they come out as zeros (the
    reference divides by l = 0 -> 1, kernels/paged_attention.py:113)."""
    w = workloads.custom("nokeys", [4], [0], 32, 8, 128, 16, seed=6)
    b = workloads.materialize(w, torch.bfloat16, hip_device, seed=6)
    b.meta.seq_lens = torch.tensor([2], dtype=torch.long, device=hip_device)  # ctx = -2
    out = HipAttention.forward(b.q, b.k_cache, b.v_cache, b.meta, w.scale)
    assert torch.count_nonzero(out[:2].float()) == 0
    assert torch.isfinite(out.float()).all()


def test_empty_batch(hip_device):
    q = torch.empty(0, 32, 128, device=hip_device, dtype=torch.bfloat16)
    kc = torch.zeros(4, 16, 8, 128, device=hip_device, dtype=torch.bfloat16)
    meta = AttentionMetadata(
        slot_mapping=torch.empty(0, dtype=torch.long, device=hip_device),
        block_tables=torch.zeros(0, 1, dtype=torch.long, device=hip_device),
        seq_lens=torch.zeros(0, dtype=torch.long, device=hip_device),
        query_lens=torch.zeros(0, dtype=torch.long, device=hip_device),
        query_start_loc=torch.zeros(1, dtype=torch.long, device=hip_device),
        max_seq_len=0,
        max_query_len=0,
    )
    out = HipAttention.forward(q, kc, kc, meta, 0.1)
    assert out.shape == (0, 32, 128)
    HipAttention.write_kv(kc, kc, q[:, :8], q[:, :8], meta.slot_mapping)


def test_argument_errors_raise(hip_device):
    w = workloads.reference_case("decode", 32, 8, head_dim=128)
    b = workloads.materialize(w, torch.bfloat16, hip_device)
    with pytest.raises(ValueError):
        HipAttention.forward(b.q.float(), b.k_cache, b.v_cache, b.meta, w.scale)
    for d in (100, 264):  # head sizes no kernel computes: not whole 16-byte rows, past 256
        bad = torch.empty(b.k_cache.shape[:3] + (d,), dtype=torch.bfloat16, device=hip_device)
        q = torch.empty(b.q.shape[:2] + (d,), dtype=torch.bfloat16, device=hip_device)
        with pytest.raises((ValueError, RuntimeError)):
            HipAttention.forward(q, bad, bad, b.meta, w.scale)


@pytest.mark.parametrize("block_size", [32, 64])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_prefill_class_large_blocks(hip_device, block_size, head_dim, dtype):
    """Prefill-class queries (q_len * G > 64) over 16-bit caches with 32- and 64-token pages:
    the prefill kernel's chunks cross page boundaries inside a page, next to decode rows."""
    w = workloads.custom(f"pre_bs{block_size}", [40, 1, 100, 17, 1], [70, 500, 0, 1000, 33], 32, 8, head_dim,
                         block_size, seed=11)  # fmt: skip
    b = workloads.materialize(w, dtype, hip_device, seed=11)
    out = pc.attend(b)
    kinds = last_launch_kernels()
    assert "prefill" in kinds, kinds
    assert pc.written_rows_match(b)
    err = (out.float().cpu() - pc.torch_oracle_full(b)).abs().max().item()
    assert err <= pc.TOL_16BIT, f"BS {block_size} D {head_dim} {dtype}: {err}"


@pytest.mark.parametrize(
    ("heads", "q_lens", "ctx_lens"),
    [
        ((32, 1), [1] * 6, [5, 300, 17, 1000, 64, 2]),  # G=32 decode: two 16-row tiles per kv head
        ((32, 1), [2, 1, 2], [400, 90, 3]),  # G=32 verify: 64 rows, four tiles, decode class
        ((32, 1), [1, 40, 1, 9], [700, 30, 2, 0]),  # G=32 mixed: prefill tiles of 4 tokens
        ((64, 1), [1] * 4, [33, 800, 1, 250]),  # G=64 decode: four tiles per kv head
        ((64, 2), [1, 20, 1], [500, 60, 7]),  # G=64 mixed: prefill tiles of 2 tokens
    ],
    ids=["g32_decode", "g32_verify", "g32_mixed", "g64_decode", "g64_mixed"],
)
@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_wide_gqa_groups(hip_device, heads, q_lens, ctx_lens, dtype):
    """GQA groups of 32 and 64 query heads per kv head (the largest the C ABI accepts)."""
    H, Hkv = heads
    w = workloads.custom("wide_g", q_lens, ctx_lens, H, Hkv, 128, 16, seed=12)
    b = workloads.materialize(w, dtype, hip_device, seed=12)
    out = pc.attend(b)
    assert torch.isfinite(out.float()).all()
    err = (out.float().cpu() - pc.torch_oracle_full(b)).abs().max().item()
    assert err <= pc.TOL_16BIT, f"{heads} {q_lens}: {err} ({last_launch_kernels()})"


def test_auto_selector_on_the_device(hip_device):
    """The selector on a real gfx950 device, nothing patched: "auto" gives HipAttention for
    block sizes the 16-token tiles divide and the caller's fallback otherwise (the reference's
    contract, src/kvserve/attention.py:113-124); "hip" raises for a block size it cannot tile."""
    from kvserve_amd import get_backend, hip_eligible

    fallback = object()
    for bs in (16, 32, 64):
        assert hip_eligible(hip_device, bs)
        assert get_backend("auto", hip_device, bs, fallback) is HipAttention
        assert get_backend("hip", hip_device, bs) is HipAttention
    for bs in (8, 24):
        assert get_backend("auto", hip_device, bs, fallback) is fallback
        with pytest.raises(ValueError):
            get_backend("hip", hip_device, bs)
    assert get_backend("auto", "cpu", 16, fallback) is fallback
    assert get_backend("auto", hip_device, 8) is None
    # a head size the MFMA kernels do not take keeps the caller's choice under "auto"
    assert get_backend("auto", hip_device, 16, fallback, head_dim=96) is fallback
    assert get_backend("auto", hip_device, 16, fallback, head_dim=128) is HipAttention
    assert get_backend("hip", hip_device, 16, head_dim=96) is HipAttention


@pytest.mark.parametrize("layout", ["padded_rows", "head_major"])
@pytest.mark.parametrize("fp8", [False, True], ids=["bf16", "e4m3"])
def test_strided_cache_layouts(hip_device, layout, fp8):
    """Caches as views with non-packed strides -- rows padded past head_dim (NaN in the
    padding), or a head-major pool [blocks, heads, slots, D] seen as [blocks, slots, heads, D]
    -- through write_kv and a forward with decode rows and prefill tiles: the same bits as the
    same calls on packed caches (the launch plan depends on shapes only), and the packed run
    within tolerance of the fp64 oracle."""
    H, Hkv, D, BS = 32, 8, 128, 16
    w = workloads.custom("strided_cache", [1, 1, 3, 70], [300, 40, 100, 33], H, Hkv, D, BS, seed=5)
    b = workloads.materialize(w, torch.bfloat16, hip_device, seed=5)
    NB = b.k_cache.shape[0]
    kw = {}
    kc, vc = b.k_cache, b.v_cache
    if fp8:
        kw = {"k_scale": 0.5, "v_scale": 0.25}
        kc = (kc.float() / 0.5).clamp(-448, 448).to(torch.float8_e4m3fn)
        vc = (vc.float() / 0.25).clamp(-448, 448).to(torch.float8_e4m3fn)

    def strided_copy(c):
        if layout == "padded_rows":
            big = torch.empty((NB, BS, Hkv, D + 64), dtype=c.dtype, device=c.device)
            big.view(torch.uint8).fill_(0x7F if fp8 else 0xFF)  # NaN in E4M3 / bf16
            view = big[..., :D]
        else:
            view = torch.empty((NB, Hkv, BS, D), dtype=c.dtype, device=c.device).permute(0, 2, 1, 3)
        view.copy_(c)
        assert not view.is_contiguous() and view.shape == c.shape
        return view

    ks, vs = strided_copy(kc), strided_copy(vc)
    bits = torch.uint8 if fp8 else torch.int16
    for k_cache, v_cache in ((kc, vc), (ks, vs)):
        HipAttention.write_kv(k_cache, v_cache, b.k_new, b.v_new, b.meta.slot_mapping, **kw)
    assert torch.equal(ks.contiguous().view(bits), kc.view(bits))
    assert torch.equal(vs.contiguous().view(bits), vc.view(bits))
    ref = HipAttention.forward(b.q, kc, vc, b.meta, w.scale, **kw)
    got = HipAttention.forward(b.q, ks, vs, b.meta, w.scale, **kw)
    torch.cuda.synchronize()
    assert "prefill" in last_launch_kernels()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    if not fp8:  # E4M3 attention against the oracle: tests/test_hip_fp8.py
        assert pc.max_err_vs_oracle(b, ref, list(range(len(w.query_lens)))) <= pc.TOL_16BIT


@pytest.mark.parametrize("fp8", [False, True], ids=["bf16", "e4m3"])
def test_prefill_page_outside_the_pool_after_the_first_window(hip_device, fp8):
    """A block-table entry outside the pool is a missing page: its 16 keys take no part in
    the softmax (the prefill kernel reads block 0 for it and masks the keys). Placed past the
    first 64 chunks of long stream-K pieces (8 x 2048 queries over 2048 cached tokens), it
    also pins that a page-window refresh extends the unmasked run only up to such a page, in
    the 16-bit tile and in the E4M3 tile (scales 0.5 / 0.25). Expected rows are computed here
    in fp64 from the (dequantized) cache without those keys."""
    from oracle import fp8 as fp8_oracle

    H, Hkv, D, BS = 32, 8, 128, 16
    w = workloads.custom("missing_page", [2048] * 8, [2048] * 8, H, Hkv, D, BS, seed=11)
    b = workloads.materialize(w, torch.bfloat16, hip_device, seed=11)
    seq, page = 3, 200  # tokens 3200 .. 3215 of sequence 3
    b.meta.block_tables[seq, page] = w.num_blocks + 7
    if fp8:
        ks, vs = 0.5, 0.25
        kc8 = fp8_oracle.quantize(b.k_cache, ks).to(hip_device)
        vc8 = fp8_oracle.quantize(b.v_cache, vs).to(hip_device)
        HipAttention.write_kv(kc8, vc8, b.k_new, b.v_new, b.meta.slot_mapping, k_scale=ks, v_scale=vs)
        out = HipAttention.forward(b.q, kc8, vc8, b.meta, w.scale, k_scale=ks, v_scale=vs)
    else:
        out = pc.attend(b)
    assert "prefill" in last_launch_kernels()
    G, ctx, q0 = H // Hkv, w.seq_lens[seq] - w.query_lens[seq], sum(w.query_lens[:seq])
    table = torch.tensor(w.tables[seq], dtype=torch.long, device=hip_device)
    if fp8:
        kc = fp8_oracle.dequantize(kc8.index_select(0, table).cpu(), ks).to(torch.float64)
        vc = fp8_oracle.dequantize(vc8.index_select(0, table).cpu(), vs).to(torch.float64)
        kc, vc = kc.reshape(-1, Hkv, D).numpy(), vc.reshape(-1, Hkv, D).numpy()
    else:
        kc = b.k_cache.index_select(0, table).to(torch.float64).cpu().reshape(-1, Hkv, D).numpy()
        vc = b.v_cache.index_select(0, table).to(torch.float64).cpu().reshape(-1, Hkv, D).numpy()
    keep = np.ones(kc.shape[0], dtype=bool)
    keep[page * BS : (page + 1) * BS] = False
    err = 0.0
    for i in (100, 1151, 1152, 1500, 2047):  # rows before, at and past the missing page
        lim = ctx + i + 1
        sel = np.nonzero(keep[:lim])[0]
        q = b.q[q0 + i].to(torch.float64).cpu().numpy()
        for h in (0, 5, 13, 31):
            s = kc[sel, h // G] @ q[h] * w.scale
            p = np.exp(s - s.max())
            ref = p @ vc[sel, h // G] / p.sum()
            err = max(err, float(np.abs(ref - out[q0 + i, h].float().cpu().numpy()).max()))
    assert err <= pc.TOL_16BIT, err
