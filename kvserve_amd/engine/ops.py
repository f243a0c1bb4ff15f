"""libkvhip's engine-harness kernels (kvh_add_rmsnorm, kvh_silu_mul, kvh_gemv,
kvh_gemv_silu_mul) for fp16 / bf16 tensors on the GPU: the elementwise steps of a Llama layer
in single passes and a weight-streaming GEMV for decode-sized batches (for the gate_up
projection with SiLU * up in its epilogue). The model uses them on the GPU with 16-bit
weights and keeps the PyTorch operations elsewhere (the CPU path the Hugging Face checks run).
"""

from __future__ import annotations

import torch

from kvserve_amd import _lib

# Rows up to which the model takes kvh_gemv (its limit is 8): measured on MI355X at the 8B
# shapes, the GEMV beats hipBLASLt up to 4 rows (QKV 9.6 vs 19.0 us, o_proj 9.5 vs 18.9,
# down 17.5 vs 19.3; gate_up 36.6 vs 34.9) and loses at 8 (gate_up 58 vs 36).
GEMV_MAX_ROWS = 4


def enabled(x: torch.Tensor) -> bool:
    return x.is_cuda and x.dtype in (torch.bfloat16, torch.float16)


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _same_gpu(*tensors: torch.Tensor) -> None:
    """All arguments on one GPU: a host tensor's address in a kernel would fault the GPU."""
    dev = tensors[0].get_device()
    if dev < 0 or any(t.get_device() != dev for t in tensors):
        raise ValueError(f"libkvhip kernels need every tensor on one GPU (got {[str(t.device) for t in tensors]})")


def add_rmsnorm(x: torch.Tensor, delta: torch.Tensor | None, weight: torch.Tensor,
                eps: float) -> tuple[torch.Tensor, torch.Tensor]:  # fmt: skip
    """(x + delta, RMSNorm(x + delta)) for [T, hidden] rows; with delta None, (x, RMSNorm(x))."""
    _same_gpu(x, weight, *([delta] if delta is not None else []))
    T, hd = x.shape
    h = torch.empty_like(x)
    xo = torch.empty_like(x) if delta is not None else x
    st = _lib.load().kvh_add_rmsnorm(
        x.data_ptr(), x.stride(0), delta.data_ptr() if delta is not None else None,
        delta.stride(0) if delta is not None else 0, weight.data_ptr(), xo.data_ptr(), xo.stride(0), h.data_ptr(),
        h.stride(0), T, hd, float(eps), _lib.KVH_DTYPE[x.dtype], _stream(x),
    )  # fmt: skip
    _lib.check(st, "kvh_add_rmsnorm")
    return xo, h


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    _same_gpu(gate_up)
    T, two_i = gate_up.shape
    out = torch.empty((T, two_i // 2), dtype=gate_up.dtype, device=gate_up.device)
    st = _lib.load().kvh_silu_mul(gate_up.data_ptr(), gate_up.stride(0), out.data_ptr(), out.stride(0), T, two_i // 2,
                                  _lib.KVH_DTYPE[gate_up.dtype], _stream(gate_up))  # fmt: skip
    _lib.check(st, "kvh_silu_mul")
    return out


def skinny_wins(m: int, n: int, k: int) -> bool:
    """Where kvh_gemm_skinny beats hipBLASLt inside the decode graph (measured on MI355X at the
    1B / 8B shapes; the skinny kernel re-reads x per 16 weight rows, so its edge shrinks with m
    and the weight size): up to 8 rows for weights up to 80 MB (8B o_proj 9.7 vs 19.3 us
    alone; decode at batch 8: 8B +3%, 1B +7%), up to 32 rows for weights up to 13 MB (the 1B
    QKV and o_proj; 1B at batch 32 +4%). Larger weights at 16 rows, everything at 64 rows and
    the 8B o_proj at 32 won alone but not inside the model."""
    if n % 16 or k % 1024:
        return False
    w_bytes = 2 * n * k
    if m <= 8:
        return w_bytes <= 80e6
    return m <= 32 and w_bytes <= 13e6


def qkv_rope_fused(m: int, n: int, k: int) -> bool:
    """Whether the QKV projection of m rows runs fused with RoPE + cache write
    (gemv_rope_and_cache; the GEMV up to 4 rows, the skinny MFMA form above). The fusion saves
    the separate rope_and_cache launch and the qkv round trip, so it pays past skinny_wins's
    limits (measured inside the decode graph): up to 64 rows for weights up to 13 MB (1B QKV:
    batch 48 +4-7%, batch 64 +2-3% against hipBLASLt + rope_and_cache) and up to 16 rows for
    weights up to 80 MB (8B QKV; at 32 rows -3%, at 64 rows -9%)."""
    if 0 < m <= GEMV_MAX_ROWS:
        return True
    if m > 64 or n % 16 or k % 1024:
        return False
    w_bytes = 2 * n * k
    return w_bytes <= 13e6 or (m <= 16 and w_bytes <= 80e6)


def linear(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """x @ weight.T: kvh_gemv for at most GEMV_MAX_ROWS rows, kvh_gemm_skinny where it beats
    hipBLASLt (skinny_wins), else PyTorch (hipBLASLt)."""
    m = x.shape[0]
    if m == 0 or x.stride(-1) != 1 or not weight.is_contiguous():
        return torch.nn.functional.linear(x, weight)
    if m <= GEMV_MAX_ROWS:
        return gemv(x, weight)
    if skinny_wins(m, *weight.shape):
        return gemm_skinny(x, weight)
    return torch.nn.functional.linear(x, weight)


def gemm_skinny(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """x @ weight.T on kvh_gemm_skinny (x: at most 64 rows; n % 16 == 0, k % 1024 == 0)."""
    _same_gpu(x, weight)
    m = x.shape[0]
    n, k = weight.shape
    y = torch.empty((m, n), dtype=x.dtype, device=x.device)
    st = _lib.load().kvh_gemm_skinny(x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0), y.data_ptr(),
                                     y.stride(0), m, n, k, _lib.KVH_DTYPE[x.dtype], _stream(x))  # fmt: skip
    _lib.check(st, "kvh_gemm_skinny")
    return y


def mlp_act(x: torch.Tensor, gate_up_weight: torch.Tensor) -> torch.Tensor:
    """silu_mul(linear(x, gate_up_weight)): for at most GEMV_MAX_ROWS rows one kvh_gemv_silu_mul
    (the activation in the projection's epilogue, the same bits), else the two steps."""
    m = x.shape[0]
    if m == 0 or x.stride(-1) != 1 or not gate_up_weight.is_contiguous():
        return silu_mul(linear(x, gate_up_weight))
    _same_gpu(x, gate_up_weight)
    if m > GEMV_MAX_ROWS:
        two_i, k = gate_up_weight.shape
        if two_i % 16 or not skinny_wins(m, two_i, k):
            return silu_mul(linear(x, gate_up_weight))
        y = torch.empty((m, two_i // 2), dtype=x.dtype, device=x.device)
        st = _lib.load().kvh_gemm_skinny_silu_mul(x.data_ptr(), x.stride(0), gate_up_weight.data_ptr(),
                                                  gate_up_weight.stride(0), y.data_ptr(), y.stride(0), m, two_i // 2, k,
                                                  _lib.KVH_DTYPE[x.dtype], _stream(x))  # fmt: skip
        _lib.check(st, "kvh_gemm_skinny_silu_mul")
        return y
    two_i, k = gate_up_weight.shape
    y = torch.empty((m, two_i // 2), dtype=x.dtype, device=x.device)
    st = _lib.load().kvh_gemv_silu_mul(x.data_ptr(), x.stride(0), gate_up_weight.data_ptr(), gate_up_weight.stride(0),
                                       y.data_ptr(), y.stride(0), m, two_i // 2, k, _lib.KVH_DTYPE[x.dtype],
                                       _stream(x))  # fmt: skip
    _lib.check(st, "kvh_gemv_silu_mul")
    return y


def gemv(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """x @ weight.T on kvh_gemv (x: at most 8 rows, unit stride in k; weight contiguous)."""
    _same_gpu(x, weight)
    m = x.shape[0]
    n, k = weight.shape
    y = torch.empty((m, n), dtype=x.dtype, device=x.device)
    st = _lib.load().kvh_gemv(x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0), y.data_ptr(), y.stride(0),
                              m, n, k, _lib.KVH_DTYPE[x.dtype], _stream(x))  # fmt: skip
    _lib.check(st, "kvh_gemv")
    return y
