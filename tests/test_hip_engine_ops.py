"""libkvhip's engine-harness kernels (kvh_add_rmsnorm, kvh_silu_mul, kvh_gemv,
kvh_gemv_silu_mul) against the
PyTorch operations they replace in the Llama layer (src/kvserve/model.py:22-32 and its MLP),
in bf16 and fp16. The residual sum is bit-exact (one rounding, as PyTorch's add). The norm's
fp32 statistics differ in summation order and rsqrt, and its output is rounded twice (x * r to
the storage type, then times the weight), so it agrees to two units in the last place; SiLU
(exp implementations differ) to one. The GEMV is checked against an fp32 product, and the
fused gate_up + SiLU * up GEMV bit for bit against the GEMV followed by kvh_silu_mul."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from kvserve_amd import HipAttention
from kvserve_amd.engine import LLAMA_3_2_1B, ops
from kvserve_amd.engine.model import PagedLlama, random_weights
from kvserve_amd.engine.runner import ModelRunner, Sequence

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16]


def _ulp_close(got: torch.Tensor, want: torch.Tensor, ulps: int = 1) -> None:
    assert got.dtype == want.dtype and got.shape == want.shape
    g, w = got.float(), want.float()
    eps = torch.finfo(want.dtype).eps
    tol = ulps * eps * torch.maximum(g.abs(), w.abs()) + torch.finfo(want.dtype).tiny
    bad = (g - w).abs() > tol
    assert not bad.any(), f"{int(bad.sum())} elements beyond {ulps} ulp; worst {((g - w).abs() / tol).max():.2f}"


def _rmsnorm(x, w, eps):  # model.py RMSNorm
    x32 = x.float()
    return w * (x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("T,hd", [(1, 2048), (7, 4096), (300, 8192), (2, 136)])
def test_add_rmsnorm(hip_device, dtype, T, hd):
    g = torch.Generator(device=hip_device).manual_seed(T + hd)
    x = torch.randn(T, hd, generator=g, device=hip_device).to(dtype)
    d = (torch.randn(T, hd, generator=g, device=hip_device) * 3).to(dtype)
    w = (torch.rand(hd, generator=g, device=hip_device) + 0.5).to(dtype)
    xo, h = ops.add_rmsnorm(x, d, w, 1e-5)
    assert torch.equal(xo, x + d)
    _ulp_close(h, _rmsnorm(x + d, w, 1e-5), ulps=2)
    x2, h2 = ops.add_rmsnorm(x, None, w, 1e-6)
    assert x2 is x
    _ulp_close(h2, _rmsnorm(x, w, 1e-6), ulps=2)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("T,inter", [(1, 8192), (5, 14336), (513, 64)])
def test_silu_mul(hip_device, dtype, T, inter):
    g = torch.Generator(device=hip_device).manual_seed(inter)
    gu = (torch.randn(T, 2 * inter, generator=g, device=hip_device) * 4).to(dtype)
    gate, up = gu.chunk(2, dim=-1)
    _ulp_close(ops.silu_mul(gu), F.silu(gate) * up)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("m", [1, 2, 3, 8])
@pytest.mark.parametrize("n,k", [(6144, 4096), (4096, 14336), (1003, 1032), (28672, 2048), (5, 8)])
def test_gemv_against_fp32(hip_device, dtype, m, n, k):
    g = torch.Generator(device=hip_device).manual_seed(m * n + k)
    x = torch.randn(m, k, generator=g, device=hip_device).to(dtype)
    w = (torch.randn(n, k, generator=g, device=hip_device) * 0.05).to(dtype)
    got = ops.gemv(x, w)
    ref = x.float() @ w.float().t()
    # fp32 accumulation in a different order, then one rounding to dtype
    tol = 2 * torch.finfo(dtype).eps * ref.abs() + 1e-3 * ref.abs().max()
    assert ((got.float() - ref).abs() <= tol).all()


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("m", [1, 2, 3, 4])
@pytest.mark.parametrize("inter,k", [(14336, 4096), (8192, 2048), (1003, 1032), (3, 8)])
def test_gemv_silu_mul_is_gemv_then_silu_mul(hip_device, dtype, m, inter, k):
    """The fused gate_up projection + silu_mul gives the bits of the two kernels in sequence
    (the sums are rounded to dtype before the activation, as the projection's output is); odd
    inter covers a wave whose second (gate, up) pair is past the end."""
    g = torch.Generator(device=hip_device).manual_seed(m * inter + k)
    x = torch.randn(m, k, generator=g, device=hip_device).to(dtype)
    w = (torch.randn(2 * inter, k, generator=g, device=hip_device) * 0.08).to(dtype)
    fused = ops.mlp_act(x, w)
    assert fused.shape == (m, inter)
    gu = ops.gemv(x, w)
    pad = -(-inter // 8) * 8  # kvh_silu_mul takes inter % 8 == 0: halves placed in a padded row
    gu_pad = torch.zeros(m, 2 * pad, dtype=dtype, device=hip_device)
    gu_pad[:, :inter], gu_pad[:, pad : pad + inter] = gu[:, :inter], gu[:, inter:]
    want = ops.silu_mul(gu_pad)[:, :inter]
    assert torch.equal(fused.view(torch.int16), want.view(torch.int16))
    if inter % 8 == 0:  # more rows: the two-step fallback (kvh_silu_mul takes inter % 8 == 0)
        big = torch.randn(ops.GEMV_MAX_ROWS + 1, k, generator=g, device=hip_device).to(dtype)
        assert torch.equal(ops.mlp_act(big, w), ops.silu_mul(ops.linear(big, w)))


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("m", [5, 16, 17, 33, 64])
@pytest.mark.parametrize("n,k", [(6144, 4096), (2048, 8192), (16, 1024)])
def test_gemm_skinny_against_fp32(hip_device, dtype, m, n, k):
    """The skinny MFMA GEMM (5 .. 64 rows; partial row tiles of 16) against an fp32 product,
    the same bar as the GEMV, and deterministic across calls."""
    g = torch.Generator(device=hip_device).manual_seed(m * n + k)
    x = torch.randn(m, k, generator=g, device=hip_device).to(dtype)
    w = (torch.randn(n, k, generator=g, device=hip_device) * 0.05).to(dtype)
    got = ops.gemm_skinny(x, w)
    ref = x.float() @ w.float().t()
    tol = 2 * torch.finfo(dtype).eps * ref.abs() + 1e-3 * ref.abs().max()
    assert ((got.float() - ref).abs() <= tol).all()
    assert torch.equal(got.view(torch.int16), ops.gemm_skinny(x, w).view(torch.int16))


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("m", [5, 8, 17, 64])
@pytest.mark.parametrize("inter,k", [(8192, 2048), (16, 1024)])
def test_gemm_skinny_silu_mul_is_skinny_then_silu_mul(hip_device, dtype, m, inter, k):
    """kvh_gemm_skinny_silu_mul (8 gate + 8 up rows per workgroup, silu_mul in the epilogue)
    gives the bits of kvh_gemm_skinny followed by kvh_silu_mul."""
    from kvserve_amd import _lib

    g = torch.Generator(device=hip_device).manual_seed(m * inter + k)
    x = torch.randn(m, k, generator=g, device=hip_device).to(dtype)
    w = (torch.randn(2 * inter, k, generator=g, device=hip_device) * 0.05).to(dtype)
    y = torch.empty(m, inter, dtype=dtype, device=hip_device)
    st = _lib.load().kvh_gemm_skinny_silu_mul(x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), y.data_ptr(),
                                              y.stride(0), m, inter, k, _lib.KVH_DTYPE[dtype],
                                              torch.cuda.current_stream().cuda_stream)  # fmt: skip
    assert st == 0
    want = ops.silu_mul(ops.gemm_skinny(x, w))
    assert torch.equal(y.view(torch.int16), want.view(torch.int16))


def test_gemv_strided_rows_and_large_batches_fall_back(hip_device):
    x = torch.randn(3, 4096 + 64, device=hip_device).to(torch.bfloat16)[:, :4096]
    w = torch.randn(512, 4096, device=hip_device).to(torch.bfloat16)
    ref = x.float() @ w.float().t()
    assert (ops.linear(x, w).float() - ref).abs().max() <= 0.05 * ref.abs().max()
    big = torch.randn(65, 4096, device=hip_device).to(torch.bfloat16)  # past the skinny GEMM: hipBLASLt
    assert torch.equal(ops.linear(big, w), F.linear(big, w))


def test_fused_model_matches_the_unfused_model(hip_device):
    """The same bf16 weights with and without libkvhip's layer kernels, through whole steps over a
    KV pool (cache write + paged attention in every layer): a prefill of T prompts, then a decode
    step of T rows -- T = 1 and 4 (GEMV; projection + RoPE + cache write in one kernel), 5, 48 and
    64 (skinny MFMA projections; the fused QKV + RoPE + cache write) and 80 (hipBLASLt). Logits
    of both steps agree within bf16 accuracy."""
    cfg = LLAMA_3_2_1B.with_layers(2)
    w = random_weights(cfg, hip_device, torch.bfloat16, seed=7, std=0.03)
    models = [PagedLlama(cfg, w, HipAttention, 512, fused_ops=f) for f in (True, False)]
    assert models[0].fused_ops and not models[1].fused_ops
    assert models[0].defers_projection(48) and not models[1].defers_projection(48)
    for T in (1, 4, 5, 48, 64, 80):
        logits = []
        for mdl in models:
            r = ModelRunner(mdl, num_blocks=T * 2 + 4, max_model_len=512, decode_graphs=False, piecewise_graphs=False)
            seqs = [Sequence([(131 * i + 7 * j) % cfg.vocab_size for j in range(11)]) for i in range(T)]
            got = []
            orig = mdl.logits
            mdl.logits = lambda h, _o=orig, _g=got: _g.append(_o(h)) or _g[-1]
            try:
                r.prefill(seqs)
                r.decode(seqs)
            finally:
                mdl.logits = orig
            logits.append(torch.cat(got))
        scale = logits[1].abs().max().item()
        assert (logits[0] - logits[1]).abs().max().item() <= 0.03 * scale, T
