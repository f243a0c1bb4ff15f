"""kvserve's attention-backend interface, served by the gfx950 HIP kernels.

Mirrors src/kvserve/attention.py of the reference:
  * `AttentionMetadata` has the same fields and meaning (attention.py:17-28);
  * `HipAttention` is a class used as a namespace of static methods with the exact
    `write_kv` / `forward` signatures of the reference's backends (attention.py:39-82,
    :88-102), so `Attention.attend` (model.py:96-108) calls it unchanged;
  * `get_backend(name, device, block_size, fallback, head_dim)` keeps the reference's selector contract
    (attention.py:113-124) for the names this package serves ("hip", and "auto", which
    falls back instead of raising).

Both methods run on `torch.cuda.current_stream()`, allocate only through torch's caching
allocator (the output when `out is None`, and the split-K workspace), never synchronise
and never read `meta.max_seq_len`, so they can be captured in a HIP graph (the decode
graph of cuda_graph.py:79-102) and called between piecewise-graph replays
(cuda_graph.py:234-240).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from kvserve_amd import _lib


@dataclass
class AttentionMetadata:
    """Same fields as the reference's AttentionMetadata (src/kvserve/attention.py:17-28)."""

    slot_mapping: torch.Tensor  # [T] flat KV slot for each new token
    block_tables: torch.Tensor  # [B, max_blocks] physical block ids, 0-padded
    seq_lens: torch.Tensor  # [B] context length including this step's tokens
    query_lens: torch.Tensor  # [B] tokens computed this step
    query_start_loc: torch.Tensor  # [B + 1] offset of each sequence's first token in the flat batch
    max_seq_len: int
    max_query_len: int
    # Padded layout, needed only by the reference's torch backend; never read here.
    q_gather: torch.Tensor | None = None
    q_valid: torch.Tensor | None = None


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_handle(device: torch.device) -> int:
    if _RAW_STREAM is not None and device.index is not None:
        return _RAW_STREAM(device.index)  # the current stream's handle without a Stream object
    return torch.cuda.current_stream(device).cuda_stream


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _dtype_code(*tensors: torch.Tensor) -> int:
    dt = tensors[0].dtype
    _require(all(t.dtype == dt for t in tensors), f"dtype mismatch: {[t.dtype for t in tensors]}")
    _require(dt in _lib.KVH_DTYPE, f"unsupported dtype {dt} (float32, float16, bfloat16)")
    return _lib.KVH_DTYPE[dt]


def _check_cache(k_cache: torch.Tensor, v_cache: torch.Tensor) -> None:
    _require(k_cache.dim() == 4 and k_cache.shape == v_cache.shape, "caches must be [num_blocks, block_size, kv_heads, D]")
    _require(k_cache.stride(-1) == 1 and v_cache.stride(-1) == 1, "cache last dim must be contiguous")
    _require(k_cache.is_cuda and v_cache.is_cuda, "caches must be on a HIP device")


# Per-call host work matters at decode sizes (tens of microseconds against kernels of the same
# order), so what depends only on the cache tensors' layout is checked once per layout and
# kept: (num_blocks, block_size, kv_heads, head_dim, k strides, v strides, device index).
_CACHE_LAYOUTS: dict = {}
_WS_SIZES: dict = {}


def _cache_layout(k_cache: torch.Tensor, v_cache: torch.Tensor) -> tuple:
    """(num_blocks, block_size, kv_heads, head_dim, k strides, v strides, device index)."""
    ks, vs = k_cache.stride(), v_cache.stride()
    key = (k_cache.data_ptr(), v_cache.data_ptr(), k_cache.get_device(), v_cache.get_device(), k_cache.dtype,
           v_cache.dtype, k_cache.shape, v_cache.shape, ks, vs)  # fmt: skip
    hit = _CACHE_LAYOUTS.get(key)
    if hit is None:
        _check_cache(k_cache, v_cache)
        _require(k_cache.get_device() == v_cache.get_device(), "k_cache and v_cache are on different devices")
        if len(_CACHE_LAYOUTS) > 256:
            _CACHE_LAYOUTS.clear()
        hit = (*k_cache.shape, tuple(ks[:3]), tuple(vs[:3]), k_cache.get_device())
        _CACHE_LAYOUTS[key] = hit
    return hit


def _on_device(dev: int, **tensors: torch.Tensor) -> None:
    """Every tensor argument lives on the caches' device: a host tensor's address handed to a
    kernel would be a GPU memory fault, not an error."""
    for name, t in tensors.items():
        if t.get_device() != dev:
            raise ValueError(f"{name} must be on the caches' device cuda:{dev} (got {t.device})")


def _workspace_size(lib, *shape) -> int:
    n = _WS_SIZES.get(shape)
    if n is None:
        n = lib.kvh_paged_attention_workspace_size(*shape)
        if len(_WS_SIZES) > 256:
            _WS_SIZES.clear()
        _WS_SIZES[shape] = n
    return n


# E4M3 KV caches (the *_fp8 entry points): float8_e4m3fn tensors with one scale per tensor.
FP8 = torch.float8_e4m3fn


def _kv_format(k_cache: torch.Tensor, v_cache: torch.Tensor, k_scale: float, v_scale: float) -> bool:
    """True for E4M3 caches (scales positive and finite); 16-bit / fp32 caches take no scales."""
    fp8 = k_cache.dtype == FP8
    _require(v_cache.dtype == k_cache.dtype, f"k/v cache dtypes differ: {k_cache.dtype}, {v_cache.dtype}")
    if fp8:
        _require(all(0.0 < float(x) < float("inf") for x in (k_scale, v_scale)), "FP8 scales must be positive, finite")
    else:
        _require(k_scale == 1.0 and v_scale == 1.0, "k_scale / v_scale apply to float8_e4m3fn caches only")
    return fp8


def _check_index(t: torch.Tensor, name: str, dim: int) -> None:
    _require(t.dtype == torch.int64, f"{name} must be int64 (got {t.dtype})")
    _require(t.dim() == dim and t.stride(-1) == 1, f"{name} must be {dim}-d with a contiguous last dim")


class HipAttention:
    """Paged attention on hand-written gfx950 kernels (decode split-K + reduce, MFMA prefill).

    Drop-in for the reference's TritonAttention (src/kvserve/attention.py:85-102): same
    static methods, same arguments, same return value.
    """

    name = "hip"
    # Capabilities the reference's ModelRunner expresses as `backend is TritonAttention`
    # identity checks (model_runner.py:45,47,190).
    graph_capturable = True  # decode and piecewise graphs may capture it
    needs_padded_layout = False  # never reads meta.q_gather / meta.q_valid
    needs_warmup = False  # ahead-of-time compiled: nothing to JIT (model_runner.py:62-89)

    @staticmethod
    def write_kv(
        k_cache: torch.Tensor,
        v_cache: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        slots: torch.Tensor,
        k_scale: float = 1.0,
        v_scale: float = 1.0,
    ) -> None:
        """reshape_and_cache: cache.view(-1, Hkv, D)[slots] = k (and v), bit for bit.

        caches: [num_blocks, block_size, kv_heads, head_dim]; k, v: [T, kv_heads, head_dim],
        any token/head stride (v is typically a strided view of the fused QKV output).
        Slots outside the pool are skipped instead of raising. float8_e4m3fn caches store
        (x / scale).clamp(-448, 448).to(float8_e4m3fn) with the given scales, bit for bit.
        """
        num_blocks, block_size, num_kv_heads, head_dim, kcs, vcs, dev = _cache_layout(k_cache, v_cache)
        fp8 = _kv_format(k_cache, v_cache, k_scale, v_scale)
        _on_device(dev, k=k, v=v, slot_mapping=slots)
        _require(k.dim() == 3 and k.shape == v.shape, "k and v must be [T, kv_heads, head_dim]")
        _require(k.shape[1:] == (num_kv_heads, head_dim), f"k/v rows {tuple(k.shape[1:])} != cache rows")
        _require(k.stride(-1) == 1 and v.stride(-1) == 1, "k/v last dim must be contiguous")
        _check_index(slots, "slot_mapping", 1)
        _require(slots.shape[0] == k.shape[0], "one slot per token")
        fast = _lib.fast()
        if fp8:
            dtype = _dtype_code(k, v)
            st = fast.reshape_and_cache_fp8(
                k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1),
                k_cache.data_ptr(), *kcs, v_cache.data_ptr(), *vcs, slots.data_ptr(), k.shape[0], num_blocks,
                num_kv_heads, head_dim, block_size, dtype, float(k_scale), float(v_scale),
                _stream_handle(k_cache.device),
            )  # fmt: skip
            _lib.check(st, "kvh_reshape_and_cache_fp8")
            return
        dtype = _dtype_code(k_cache, v_cache, k, v)
        st = fast.reshape_and_cache(
            k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1),
            k_cache.data_ptr(), *kcs, v_cache.data_ptr(), *vcs,
            slots.data_ptr(), k.shape[0], num_blocks, num_kv_heads, head_dim, block_size, dtype,
            _stream_handle(k_cache.device),
        )  # fmt: skip
        _lib.check(st, "kvh_reshape_and_cache")

    # Extension beyond the reference's interface: RoPE + QKV split + write_kv in one kernel.
    fused_rope_cache = True

    @staticmethod
    def rope_and_cache(
        qkv: torch.Tensor,
        positions: torch.Tensor,
        cos: torch.Tensor,
        sin: torch.Tensor,
        k_cache: torch.Tensor,
        v_cache: torch.Tensor,
        slots: torch.Tensor,
        num_heads: int,
        out: torch.Tensor | None = None,
        k_scale: float = 1.0,
        v_scale: float = 1.0,
    ) -> torch.Tensor:
        """The step before forward() in one kernel (kvh_rope_and_cache; float8_e4m3fn caches:
        kvh_rope_and_cache_fp8, the keys and values stored as write_kv stores them).

        qkv: [T, (num_heads + 2 kv_heads) head_dim], the fused projection (model.py:84-94);
        positions: int64 [T]; cos, sin: fp32 [max_positions, head_dim] (RotaryEmbedding's
        tables). Writes RoPE(k) and v into the caches at `slots` (as write_kv) and returns
        RoPE(q) as [T, num_heads, head_dim] (in `out` if given), bit-identical to the
        reference's bf16/fp16/fp32 torch operations.
        """
        num_blocks, block_size, num_kv_heads, head_dim, kcs, vcs, dev = _cache_layout(k_cache, v_cache)
        fp8 = _kv_format(k_cache, v_cache, k_scale, v_scale)
        _on_device(dev, qkv=qkv, positions=positions, cos=cos, sin=sin, slot_mapping=slots)
        _require(qkv.dim() == 2 and qkv.stride(-1) == 1, "qkv must be [T, (H + 2 Hkv) D] with a contiguous last dim")
        _require(qkv.shape[1] == (num_heads + 2 * num_kv_heads) * head_dim, "qkv width != (H + 2 Hkv) D")
        _require(cos.dtype == torch.float32 and sin.dtype == torch.float32, "cos/sin tables must be fp32")
        _require(cos.dim() == 2 and cos.shape == sin.shape and cos.shape[1] == head_dim, "cos/sin must be [P, D]")
        _require(cos.is_contiguous() and sin.is_contiguous(), "cos/sin tables must be contiguous")
        _check_index(positions, "positions", 1)
        _check_index(slots, "slot_mapping", 1)
        num_tokens = qkv.shape[0]
        _require(positions.shape[0] == num_tokens and slots.shape[0] == num_tokens, "one position and slot per token")
        if out is None:
            out = torch.empty((num_tokens, num_heads, head_dim), dtype=qkv.dtype, device=qkv.device)
        _on_device(dev, out=out)
        _require(out.shape == (num_tokens, num_heads, head_dim) and out.stride(-1) == 1, "out must be [T, H, D]")
        dtype = _dtype_code(qkv, out) if fp8 else _dtype_code(qkv, k_cache, v_cache, out)
        if num_tokens == 0:
            return out
        st = _lib.fast().rope_and_cache(
            qkv.data_ptr(), qkv.stride(0), positions.data_ptr(), cos.data_ptr(), sin.data_ptr(), cos.shape[0],
            out.data_ptr(), out.stride(0), out.stride(1),
            k_cache.data_ptr(), *kcs, v_cache.data_ptr(), *vcs,
            slots.data_ptr(), num_tokens, num_blocks, num_heads, num_kv_heads, head_dim, block_size, dtype,
            int(fp8), float(k_scale), float(v_scale), _stream_handle(qkv.device),
        )  # fmt: skip
        _lib.check(st, "kvh_rope_and_cache_fp8" if fp8 else "kvh_rope_and_cache")
        return out

    # rows up to which gemv_rope_and_cache applies (up to 4 on the GEMV, then on the MFMA units)
    GEMV_ROPE_MAX_ROWS = 64

    @staticmethod
    def gemv_rope_and_cache(
        x: torch.Tensor,
        w_qkv: torch.Tensor,
        positions: torch.Tensor,
        cos: torch.Tensor,
        sin: torch.Tensor,
        k_cache: torch.Tensor,
        v_cache: torch.Tensor,
        slots: torch.Tensor,
        num_heads: int,
        out: torch.Tensor | None = None,
        k_scale: float = 1.0,
        v_scale: float = 1.0,
    ) -> torch.Tensor:
        """rope_and_cache(x @ w_qkv.T, ...) in one kernel (kvh_gemv_rope_and_cache) for at most
        GEMV_ROPE_MAX_ROWS rows of 16-bit x: the same bits as the projection on kvh_gemv (up to 4
        rows) or kvh_gemm_skinny (more; hidden % 1024 == 0, head_dim % 16 == 0) followed by
        rope_and_cache. x: [T, hidden]; w_qkv: [(H + 2 Hkv) D, hidden], contiguous."""
        num_blocks, block_size, num_kv_heads, head_dim, kcs, vcs, dev = _cache_layout(k_cache, v_cache)
        fp8 = _kv_format(k_cache, v_cache, k_scale, v_scale)
        _on_device(dev, x=x, w_qkv=w_qkv, positions=positions, cos=cos, sin=sin, slot_mapping=slots)
        _require(x.dim() == 2, "x must be [T, hidden]")
        num_tokens, hidden = x.shape
        _require(0 < num_tokens <= HipAttention.GEMV_ROPE_MAX_ROWS, "gemv_rope_and_cache takes 1 .. 64 rows")
        _require(x.stride(-1) == 1 and w_qkv.is_contiguous(), "x needs a contiguous last dim, w_qkv contiguous")
        _require(w_qkv.shape == ((num_heads + 2 * num_kv_heads) * head_dim, hidden), "w_qkv must be [(H + 2 Hkv) D, k]")
        _require(cos.dtype == torch.float32 and sin.dtype == torch.float32, "cos/sin tables must be fp32")
        _require(cos.dim() == 2 and cos.shape == sin.shape and cos.shape[1] == head_dim, "cos/sin must be [P, D]")
        _require(cos.is_contiguous() and sin.is_contiguous(), "cos/sin tables must be contiguous")
        _check_index(positions, "positions", 1)
        _check_index(slots, "slot_mapping", 1)
        _require(positions.shape[0] == num_tokens and slots.shape[0] == num_tokens, "one position and slot per token")
        if out is None:
            out = torch.empty((num_tokens, num_heads, head_dim), dtype=x.dtype, device=x.device)
        _on_device(dev, out=out)
        _require(out.shape == (num_tokens, num_heads, head_dim) and out.stride(-1) == 1, "out must be [T, H, D]")
        dtype = _dtype_code(x, w_qkv, out) if fp8 else _dtype_code(x, w_qkv, k_cache, v_cache, out)
        st = _lib.load().kvh_gemv_rope_and_cache(
            x.data_ptr(), x.stride(0), w_qkv.data_ptr(), w_qkv.stride(0), num_tokens, hidden,
            positions.data_ptr(), cos.data_ptr(), sin.data_ptr(), cos.shape[0],
            out.data_ptr(), out.stride(0), out.stride(1),
            k_cache.data_ptr(), _lib.i64x3(kcs), v_cache.data_ptr(), _lib.i64x3(vcs),
            slots.data_ptr(), num_blocks, num_heads, num_kv_heads, head_dim, block_size, dtype, int(fp8),
            float(k_scale), float(v_scale), _stream_handle(x.device),
        )  # fmt: skip
        _lib.check(st, "kvh_gemv_rope_and_cache")
        return out

    @staticmethod
    def forward(
        q: torch.Tensor,
        k_cache: torch.Tensor,
        v_cache: torch.Tensor,
        meta: AttentionMetadata,
        scale: float,
        out: torch.Tensor | None = None,
        k_scale: float = 1.0,
        v_scale: float = 1.0,
    ) -> torch.Tensor:
        """q: [T, H, D]; caches: [num_blocks, block_size, H_kv, D]. Returns [T, H, D] (in `out` if given).
        float8_e4m3fn caches hold keys / values as e4m3 * k_scale / v_scale (q and out bf16 or fp16)."""
        num_blocks, block_size, num_kv_heads, head_dim, kcs, vcs, dev = _cache_layout(k_cache, v_cache)
        fp8 = _kv_format(k_cache, v_cache, k_scale, v_scale)
        tables, seq_lens, qsl = meta.block_tables, meta.seq_lens, meta.query_start_loc
        _on_device(dev, q=q, block_tables=tables, seq_lens=seq_lens, query_start_loc=qsl)
        _require(q.dim() == 3 and q.shape[2] == head_dim, "q must be [T, H, head_dim]")
        _require(q.stride(-1) == 1, "q last dim must be contiguous")
        num_tokens, num_heads, _ = q.shape
        _require(num_heads % num_kv_heads == 0, "num_heads must be a multiple of num_kv_heads")
        _check_index(tables, "block_tables", 2)
        _check_index(seq_lens, "seq_lens", 1)
        _check_index(qsl, "query_start_loc", 1)
        num_seqs = tables.shape[0]
        _require(seq_lens.shape[0] == num_seqs and qsl.shape[0] == num_seqs + 1, "metadata sizes disagree")
        if out is None:
            out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        _on_device(dev, out=out)
        _require(out.shape == q.shape and out.stride(-1) == 1, "out must match q with a contiguous last dim")
        dtype = _dtype_code(q, out) if fp8 else _dtype_code(q, k_cache, v_cache, out)
        _require(not fp8 or q.dtype != torch.float32, "float8_e4m3fn caches need bf16 or fp16 queries")
        if num_tokens == 0 or num_seqs == 0:
            return out
        lib = _lib.load()
        width = tables.shape[1]
        max_q = int(meta.max_query_len)
        ws_bytes = _workspace_size(lib, num_tokens, num_seqs, num_heads, num_kv_heads, head_dim, width, block_size, max_q,
                                   dtype)  # fmt: skip
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
        fast = _lib.fast()
        ws_ptr = ws.data_ptr() if ws is not None else None
        if fp8:
            st = fast.paged_attention_fp8(
                q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), *kcs, v_cache.data_ptr(), *vcs,
                num_blocks, out.data_ptr(), out.stride(0), out.stride(1), tables.data_ptr(), tables.stride(0), width,
                seq_lens.data_ptr(), qsl.data_ptr(), num_tokens, num_seqs, num_heads, num_kv_heads, head_dim,
                block_size, max_q, float(scale), float(k_scale), float(v_scale), dtype, ws_ptr, ws_bytes,
                _stream_handle(q.device),
            )  # fmt: skip
            _lib.check(st, "kvh_paged_attention_fp8")
        else:
            st = fast.paged_attention(
                q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), *kcs, v_cache.data_ptr(), *vcs,
                num_blocks, out.data_ptr(), out.stride(0), out.stride(1), tables.data_ptr(), tables.stride(0), width,
                seq_lens.data_ptr(), qsl.data_ptr(), num_tokens, num_seqs, num_heads, num_kv_heads, head_dim,
                block_size, max_q, float(scale), dtype, ws_ptr, ws_bytes, _stream_handle(q.device),
            )  # fmt: skip
            _lib.check(st, "kvh_paged_attention")
        return out


def last_launch_kernels() -> list[str]:
    """Kernel kinds launched by the last forward() on this thread, in order."""
    buf = (ctypes.c_int32 * 8)()
    n = _lib.load().kvh_last_launch_kernels(buf, 8)
    return [_lib.KERNEL_KINDS.get(buf[i], "?") for i in range(min(n, 8))]


def hip_available() -> bool:
    """True when a ROCm build of torch sees a GPU and libkvhip loads."""
    if torch.version.hip is None or not torch.cuda.is_available():
        return False
    try:
        _lib.load()
    except (RuntimeError, OSError):
        return False
    return True


# Head sizes the MFMA kernels take; the vector-ALU kernel serves any other head size of whole
# 16-byte rows up to 256 (correct, at a fraction of the bandwidth).
MFMA_HEAD_DIMS = (64, 128)


def head_dim_supported(head_dim: int) -> bool:
    """A head size HipAttention computes at all (bf16 / fp16: a multiple of 8 up to 256)."""
    return 0 < head_dim <= 256 and head_dim % 8 == 0


def hip_eligible(device: str, block_size: int, head_dim: int | None = None) -> bool:
    """True when the HIP backend serves this engine at speed: a ROCm device, libkvhip loaded, a
    block size the 16-token MFMA tiles divide and (when the caller passes it) a head size the
    MFMA kernels take (64 or 128)."""
    if head_dim is not None and head_dim not in MFMA_HEAD_DIMS:
        return False
    return str(device).startswith("cuda") and block_size >= 16 and block_size % 16 == 0 and hip_available()


def get_backend(name: str, device: str, block_size: int, fallback=None, head_dim: int | None = None):
    """Selector with the reference's contract (src/kvserve/attention.py:113-124).

    "auto" never raises, as in the reference: it resolves to HipAttention when the backend can
    run here at speed (`hip_eligible`; pass `head_dim` so that a model whose heads the MFMA
    kernels do not take -- anything but 64 and 128 -- keeps the caller's choice), otherwise to
    `fallback` -- the backend the caller's own "auto" would pick (kvserve passes its torch /
    triton choice; None when not given). "hip" raises RuntimeError when the backend cannot run
    and ValueError for a block size the kernels do not tile or a head size they cannot compute
    (not a multiple of 8, or above 256), like the reference's "triton"; other head sizes run on
    the vector-ALU kernel. The reference's "torch" and "triton" names stay with its own classes:
    this package ships no CPU path.
    """
    if name == "auto":
        return HipAttention if hip_eligible(device, block_size, head_dim) else fallback
    if name == "hip":
        if not hip_available():
            raise RuntimeError("hip backend needs a ROCm GPU and a built kvserve_amd/lib/libkvhip.so")
        if block_size < 16 or block_size % 16 != 0:
            raise ValueError("hip backend needs block_size a multiple of 16 (16-token MFMA tiles)")
        if head_dim is not None and not head_dim_supported(head_dim):
            raise ValueError(f"hip backend computes head sizes that are multiples of 8 up to 256, not {head_dim}")
        return HipAttention
    if name in ("torch", "triton"):
        raise ValueError(f"backend {name!r} belongs to kvserve.attention; kvserve_amd serves 'hip' and 'auto'")
    raise ValueError(f"unknown attention backend {name!r}")


def build_metadata(
    device: torch.device | str,
    block_tables: list[list[int]],
    slots: list[int],
    seq_lens: list[int],
    query_lens: list[int],
    padded_layout: bool = False,
) -> AttentionMetadata:
    """Metadata for a flat batch where sequence i contributes query_lens[i] tokens.

    Same layout and dtypes as the reference's build_metadata (src/kvserve/model_runner.py:165-197):
    int64 tensors, block tables 0-padded to the longest row, query_start_loc prefix sums.
    The padded q_gather / q_valid tensors are built only when `padded_layout` is set
    (the reference keys this on `backend is not TritonAttention`, :190).
    """
    max_blocks = max(len(t) for t in block_tables)
    tables = [t + [0] * (max_blocks - len(t)) for t in block_tables]
    max_q = max(query_lens)
    query_start_loc = [0]
    for n in query_lens:
        query_start_loc.append(query_start_loc[-1] + n)
    meta = AttentionMetadata(
        slot_mapping=torch.tensor(slots, dtype=torch.long, device=device),
        block_tables=torch.tensor(tables, dtype=torch.long, device=device),
        seq_lens=torch.tensor(seq_lens, dtype=torch.long, device=device),
        query_lens=torch.tensor(query_lens, dtype=torch.long, device=device),
        query_start_loc=torch.tensor(query_start_loc, dtype=torch.long, device=device),
        max_seq_len=max(seq_lens),
        max_query_len=max_q,
    )
    if padded_layout:
        q_gather, q_valid = [], []
        for start, n in zip(query_start_loc, query_lens):
            q_gather.append(list(range(start, start + n)) + [0] * (max_q - n))
            q_valid.append([True] * n + [False] * (max_q - n))
        meta.q_gather = torch.tensor(q_gather, dtype=torch.long, device=device)
        meta.q_valid = torch.tensor(q_valid, dtype=torch.bool, device=device)
    return meta
