"""CPU oracle for kvserve's attention hot path. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this package,
and only as the checker / the CPU baseline; the product (kvserve_amd) never does.

Two independent restatements of the reference's semantics:
  * `paged_attention_f64` - plain-C fp64 brute force over the closed form
    (paged_attention_oracle.c), one query row at a time;
  * `oracle.torch_reference` - the reference's own algorithm, TorchAttention.forward
    (src/kvserve/attention.py:47-82): gather pages, repeat_interleave for GQA, masked SDPA.

Pinning (tests/test_oracle.py): the two agree with each other; both satisfy known answers
(seq_len = 1 -> v0, constant V -> V, q = 0 -> mean of visible V, shift invariance,
block-permutation and padding-width invariance, GQA G = 1 equals per-head MHA); the slot
formula matches the reference's per-token slot on reversed tables (tests/test_kv_cache.py:57-63
of the reference); and each planted mistake (KVO_MUT_*) is rejected by at least one check.
The reference ships no golden vectors for this path.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

MUT_GQA_MODULO = 1
MUT_CAUSAL_OFF = 2
MUT_NO_SCALE = 4
MUT_PAGE_INDEX = 8
MUT_CTX_ZERO = 16
MUT_NO_MAXSHIFT = 32
MUTANTS = {
    "gqa_modulo": MUT_GQA_MODULO,
    "causal_off_by_one": MUT_CAUSAL_OFF,
    "no_scale": MUT_NO_SCALE,
    "page_index": MUT_PAGE_INDEX,
    "ctx_zero": MUT_CTX_ZERO,
    "no_max_shift": MUT_NO_MAXSHIFT,
}

_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            from oracle.build import build

            build()
        lib = ctypes.CDLL(str(LIB_PATH))
        vp, i64, i32, f64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_double
        lib.kvo_paged_attention.restype = ctypes.c_int
        lib.kvo_paged_attention.argtypes = [vp, i64, i32, i32, vp, vp, i64, i32, i32, vp, i32, vp, vp, i32, f64, i32, vp]
        lib.kvo_reshape_and_cache.restype = None
        lib.kvo_reshape_and_cache.argtypes = [vp, vp, i64, i32, i32, i32, vp, vp, vp, i64, i32]
        lib.kvo_slots.restype = ctypes.c_int64
        lib.kvo_slots.argtypes = [vp, i32, i64, i64, vp]
        _lib = lib
    return _lib


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def paged_attention_f64(
    q: np.ndarray,
    k_cache: np.ndarray,
    v_cache: np.ndarray,
    block_tables: np.ndarray,
    seq_lens: np.ndarray,
    query_start_loc: np.ndarray,
    scale: float,
    flags: int = 0,
) -> np.ndarray:
    """q [T, H, D]; caches [NB, BS, Hkv, D]; returns out [T, H, D] float64."""
    q = _c(q, np.float64)
    kc, vc = _c(k_cache, np.float64), _c(v_cache, np.float64)
    bt = _c(block_tables, np.int64)
    sl, qsl = _c(seq_lens, np.int64), _c(query_start_loc, np.int64)
    T, H, D = q.shape
    NB, BS, Hkv, _ = kc.shape
    out = np.zeros((T, H, D), dtype=np.float64)
    st = load().kvo_paged_attention(
        _ptr(q), T, H, D, _ptr(kc), _ptr(vc), NB, BS, Hkv, _ptr(bt), bt.shape[1], _ptr(sl), _ptr(qsl), bt.shape[0],
        float(scale), int(flags), _ptr(out),
    )  # fmt: skip
    if st != 0:
        raise ValueError("oracle: inconsistent metadata or block id outside the pool")
    return out


def reshape_and_cache(
    k: np.ndarray, v: np.ndarray, slots: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray
) -> None:
    """In place on contiguous caches [NB, BS, Hkv, D]; k, v [T, Hkv, D] of the caches' dtype."""
    assert k_cache.flags.c_contiguous and v_cache.flags.c_contiguous
    k, v = np.ascontiguousarray(k), np.ascontiguousarray(v)
    assert k.dtype == v.dtype == k_cache.dtype == v_cache.dtype
    s = _c(slots, np.int64)
    T, Hkv, D = k.shape
    NB, BS = k_cache.shape[:2]
    load().kvo_reshape_and_cache(_ptr(k), _ptr(v), T, Hkv, D, k.itemsize, _ptr(s), _ptr(k_cache), _ptr(v_cache), NB, BS)


def slots(table: list[int], block_size: int, start: int, n: int) -> list[int]:
    """Per-block-run slot formula of KVCacheManager.slots (src/kvserve/kv_cache.py:159-169)."""
    t = _c(np.asarray(table if table else [0]), np.int64)
    out = np.zeros(max(n, 1), dtype=np.int64)
    k = load().kvo_slots(_ptr(t), block_size, start, n, _ptr(out))
    return out[:k].tolist()
