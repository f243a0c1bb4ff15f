"""ctypes binding of libkvhip.so (the C ABI declared in include/kvhip.h).

torch is imported first on purpose: torch ships its own HIP runtime (libamdhip64.so.7),
and loading it before libkvhip makes the library bind to that same runtime instance,
so the hipStream_t handles torch hands out are valid inside the library.

There is no fallback: if the library is missing or fails to load, every entry point
raises. Build it with `python -m kvserve_amd.build`.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (see module docstring: must precede the CDLL load)

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libkvhip.so"

ABI_VERSION = 1

KVH_DTYPE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

KERNEL_KINDS = {1: "decode", 2: "prefill", 3: "reduce", 4: "f32", 5: "share", 6: "valu16"}

_i32, _i64, _f32, _vp, _sz = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t
_i64p = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes), in the order of include/kvhip.h
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "kvh_abi_version": (ctypes.c_int, []),
    "kvh_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "kvh_reshape_and_cache": (
        ctypes.c_int,
        [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64p, _vp, _i64p, _vp, _i64, _i64, _i32, _i32, _i32, _i32, _vp],
    ),
    "kvh_reshape_and_cache_fp8": (
        ctypes.c_int,
        [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64p, _vp, _i64p, _vp, _i64, _i64, _i32, _i32, _i32, _i32, _f32, _f32,
         _vp],
    ),
    "kvh_rope_and_cache": (
        ctypes.c_int,
        [
            _vp, _i64, _vp, _vp, _vp, _i64,  # qkv, positions, cos/sin tables
            _vp, _i64, _i64,  # q_out
            _vp, _i64p, _vp, _i64p,  # caches
            _vp, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _vp,  # slots, sizes, dtype, stream
        ],  # fmt: skip
    ),
    "kvh_rope_and_cache_fp8": (
        ctypes.c_int,
        [
            _vp, _i64, _vp, _vp, _vp, _i64,  # qkv, positions, cos/sin tables
            _vp, _i64, _i64,  # q_out
            _vp, _i64p, _vp, _i64p,  # caches
            _vp, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _f32, _f32, _vp,  # slots, sizes, dtype, scales, stream
        ],  # fmt: skip
    ),
    "kvh_gemv_rope_and_cache": (
        ctypes.c_int,
        [
            _vp, _i64, _vp, _i64, _i32, _i32,  # x, w_qkv, m, k
            _vp, _vp, _vp, _i64,  # positions, cos/sin tables
            _vp, _i64, _i64,  # q_out
            _vp, _i64p, _vp, _i64p,  # caches
            _vp, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _f32, _vp,  # slots, sizes, dtype, fp8, scales
        ],  # fmt: skip
    ),
    "kvh_prepare_metadata": (
        ctypes.c_int,
        [
            _vp, _i32, _i32, _i32, _i64,  # packed, num_seqs, num_pad_seqs, num_updates, num_tokens
            _vp, _i32, _i64, _i32,  # table pool
            _vp, _i64, _i32, _i64,  # block tables, row stride, width, pad
            _vp, _vp, _vp, _vp, _vp, _vp,  # slots, positions, input_ids, seq_lens, query_lens, qsl
            _i64, _i32, _vp,  # pad_slot, block_size, stream
        ],  # fmt: skip
    ),
    "kvh_paged_attention_workspace_size": (_sz, [_i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "kvh_paged_attention": (
        ctypes.c_int,
        [
            _vp, _i64, _i64,  # q
            _vp, _i64p, _vp, _i64p, _i64,  # caches, num_blocks
            _vp, _i64, _i64,  # out
            _vp, _i64, _i32,  # block tables
            _vp, _vp,  # seq_lens, query_start_loc
            _i64, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _i32,  # sizes, scale, dtype
            _vp, _sz, _vp,  # workspace, stream
        ],  # fmt: skip
    ),
    "kvh_paged_attention_static": (
        ctypes.c_int,
        [
            _vp, _i64, _i64,  # q
            _vp, _i64p, _vp, _i64p, _i64,  # caches, num_blocks
            _vp, _i64, _i64,  # out
            _vp, _i64, _i32,  # block tables
            _vp, _vp,  # seq_lens, query_start_loc
            _i64, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _i32,  # sizes, scale, dtype
            _vp,  # stream
        ],  # fmt: skip
    ),
    "kvh_paged_attention_fp8": (
        ctypes.c_int,
        [
            _vp, _i64, _i64,  # q
            _vp, _i64p, _vp, _i64p, _i64,  # caches, num_blocks
            _vp, _i64, _i64,  # out
            _vp, _i64, _i32,  # block tables
            _vp, _vp,  # seq_lens, query_start_loc
            _i64, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _f32, _f32, _i32,  # sizes, scales, dtype
            _vp, _sz, _vp,  # workspace, stream
        ],  # fmt: skip
    ),
    "kvh_add_rmsnorm": (
        ctypes.c_int,
        [_vp, _i64, _vp, _i64, _vp, _vp, _i64, _vp, _i64, _i64, _i32, _f32, _i32, _vp],
    ),
    "kvh_silu_mul": (ctypes.c_int, [_vp, _i64, _vp, _i64, _i64, _i32, _i32, _vp]),
    "kvh_gemv": (ctypes.c_int, [_vp, _i64, _vp, _i64, _vp, _i64, _i32, _i32, _i32, _i32, _vp]),
    "kvh_gemm_skinny": (ctypes.c_int, [_vp, _i64, _vp, _i64, _vp, _i64, _i32, _i32, _i32, _i32, _vp]),
    "kvh_gemm_skinny_silu_mul": (ctypes.c_int, [_vp, _i64, _vp, _i64, _vp, _i64, _i32, _i32, _i32, _i32, _vp]),
    "kvh_gemv_silu_mul": (ctypes.c_int, [_vp, _i64, _vp, _i64, _vp, _i64, _i32, _i32, _i32, _i32, _vp]),
    "kvh_profile_arm": (ctypes.c_int, [ctypes.POINTER(ctypes.c_void_p), _i32]),
    "kvh_last_launch_kernels": (ctypes.c_int, [ctypes.POINTER(ctypes.c_int32), _i32]),
    "kvh_probe": (ctypes.c_int, [_i32, _vp, _vp, _i64, _i32, _i32, _vp]),
}

_lib: ctypes.CDLL | None = None
_fast = None
_lock = threading.Lock()


class KvhError(RuntimeError):
    """A nonzero status from libkvhip (argument error or failed HIP launch)."""

    def __init__(self, status: int, where: str):
        self.status = status
        super().__init__(f"{where}: {strerror(status)} (status {status})")


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raises RuntimeError when it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: the HIP backend has no fallback. Build it with `python -m kvserve_amd.build`."
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        version = lib.kvh_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"libkvhip ABI {version} does not match the Python binding ({ABI_VERSION})")
        global _fast
        try:
            from kvserve_amd import _kvhfast
        except ImportError as e:
            raise RuntimeError(
                f"kvserve_amd/_kvhfast is not built ({e}): build it with `python -m kvserve_amd.build`."
            ) from e
        _kvhfast.bind(lib._handle)
        _fast = _kvhfast
        _lib = lib
    return _lib


def fast():
    """The METH_FASTCALL binding of the per-step entry points, bound to the loaded library."""
    if _fast is None:
        load()
    return _fast


def strerror(status: int) -> str:
    return load().kvh_strerror(status).decode()


def check(status: int, where: str) -> None:
    if status != 0:
        raise KvhError(status, where)


def i64x3(values) -> ctypes.Array:
    return (ctypes.c_int64 * 3)(*[int(v) for v in values])
