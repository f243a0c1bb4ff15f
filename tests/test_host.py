"""Host-side checks that need no GPU: the C ABI library, the plan, the Python boundary."""

import ctypes
import math
import random
import re
from pathlib import Path

import pytest
import torch

from kvserve_amd import _lib, attention, workloads

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "kvhip.h"

E_NULL, E_SHAPE, E_DTYPE, E_ALIGN, E_UNSUPPORTED, E_WORKSPACE, E_SCRATCH = -1, -2, -3, -4, -5, -6, -7


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    return re.findall(r"KVH_API\s+[\w\s\*]+?\b(kvh_\w+)\s*\(", text)


def test_header_declares_the_abi():
    names = declared_symbols()
    assert set(names) == set(_lib.SIGNATURES), names


def test_library_exports_every_declared_symbol(lib):
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert lib.kvh_abi_version() == _lib.ABI_VERSION


def test_strerror_covers_every_status(lib):
    for code in (0, E_NULL, E_SHAPE, E_DTYPE, E_ALIGN, E_UNSUPPORTED, E_WORKSPACE, E_SCRATCH):
        msg = lib.kvh_strerror(code).decode()
        assert msg and (code == 0 or "kvhip" in msg)
    assert lib.kvh_strerror(-99).decode() == "kvhip: unknown status"


def _attn_args(**over):
    """Arguments of kvh_paged_attention for a C2-like shape with fake (never dereferenced)
    16-byte-aligned pointers; every call below fails validation before any HIP call."""
    a = dict(
        q=0x1000, q_ts=32 * 128, q_hs=128, kc=0x2000, kcs=(16 * 8 * 128, 8 * 128, 128), vc=0x3000,
        vcs=(16 * 8 * 128, 8 * 128, 128), nb=40_000, out=0x4000, o_ts=32 * 128, o_hs=128, bt=0x5000,
        bt_rs=512, W=512, sl=0x6000, qsl=0x7000, T=64, B=64, H=32, Hkv=8, D=128, BS=16, max_q=1,
        scale=128**-0.5, dtype=2, ws=0, ws_bytes=0, stream=None,
    )  # fmt: skip
    a.update(over)
    return a


def _call(lib, a):
    return lib.kvh_paged_attention(
        a["q"], a["q_ts"], a["q_hs"], a["kc"], _lib.i64x3(a["kcs"]), a["vc"], _lib.i64x3(a["vcs"]), a["nb"],
        a["out"], a["o_ts"], a["o_hs"], a["bt"], a["bt_rs"], a["W"], a["sl"], a["qsl"], a["T"], a["B"], a["H"],
        a["Hkv"], a["D"], a["BS"], a["max_q"], a["scale"], a["dtype"], a["ws"], a["ws_bytes"], a["stream"],
    )  # fmt: skip


@pytest.mark.parametrize(
    ("over", "status"),
    [
        (dict(dtype=7), E_DTYPE),
        (dict(H=30), E_SHAPE),
        (dict(D=100), E_UNSUPPORTED),  # 16-bit rows of whole 16-byte vectors only
        (dict(D=264), E_UNSUPPORTED),  # the vector-ALU kernel's query row holds 256
        (dict(Hkv=0), E_SHAPE),
        (dict(W=0), E_SHAPE),
        (dict(q=0), E_NULL),
        (dict(bt_rs=100), E_SHAPE),
        (dict(q=0x1008), E_ALIGN),
        (dict(q_hs=132), E_ALIGN),
        (dict(ws=0, ws_bytes=0), E_WORKSPACE),  # C2 needs split-K scratch
        (dict(dtype=0, D=102), E_UNSUPPORTED),
        (dict(B=70_000), E_UNSUPPORTED),
        (dict(T=600_000_000), E_UNSUPPORTED),  # query rows T * G past 2^31
    ],
)
def test_attention_validation(lib, over, status):
    assert _call(lib, _attn_args(**over)) == status
    assert _call_fast(_attn_args(**over)) == status


def _call_fast(a):
    """The same call through the METH_FASTCALL binding the backend uses per step."""
    return _lib.fast().paged_attention(
        a["q"], a["q_ts"], a["q_hs"], a["kc"], *a["kcs"], a["vc"], *a["vcs"], a["nb"],
        a["out"], a["o_ts"], a["o_hs"], a["bt"], a["bt_rs"], a["W"], a["sl"], a["qsl"], a["T"], a["B"], a["H"],
        a["Hkv"], a["D"], a["BS"], a["max_q"], a["scale"], a["dtype"], a["ws"] or None, a["ws_bytes"], a["stream"],
    )  # fmt: skip


def test_fast_binding_is_bound_to_the_loaded_library(lib):
    """_kvhfast resolves its entry points in the library ctypes opened; argument count and
    type errors are Python exceptions, statuses come back unchanged."""
    fast = _lib.fast()
    with pytest.raises(TypeError, match="32 arguments"):
        fast.paged_attention(1, 2)
    with pytest.raises(TypeError):
        fast.paged_attention(*(["x"] * 32))
    strides = (16 * 8 * 128, 8 * 128, 128)
    args = [0x1000, 8 * 128, 128, 0x2000, 8 * 128, 128, 0x3000, *strides, 0x4000, *strides, 0x5000, 10, 100, 8, 128, 16]
    assert fast.reshape_and_cache(*args, 9, None) == E_DTYPE
    assert fast.reshape_and_cache_fp8(*args, 2, 0.0, 1.0, None) == E_SHAPE  # scale must be positive
    rope = [0x1000, 48 * 128, 0x2000, 0x3000, 0x3800, 64, 0x4000, 32 * 128, 128, 0x5000, *strides, 0x6000, *strides,
            0x7000, 10, 100, 32, 8, 128, 16]  # fmt: skip
    assert fast.rope_and_cache(*rope, 9, 0, 1.0, 1.0, None) == E_DTYPE
    assert fast.rope_and_cache(*rope, 2, 1, -1.0, 1.0, None) == E_SHAPE


def test_empty_batch_is_a_no_op(lib):
    assert _call(lib, _attn_args(T=0, q=0, out=0)) == 0
    assert _call(lib, _attn_args(B=0)) == 0


def test_cache_write_validation(lib):
    f = lib.kvh_reshape_and_cache
    strides = _lib.i64x3((16 * 8 * 128, 8 * 128, 128))
    args = [0x1000, 8 * 128, 128, 0x2000, 8 * 128, 128, 0x3000, strides, 0x4000, strides, 0x5000, 10, 100, 8, 128, 16]
    assert f(*args, 9, None) == E_DTYPE
    assert f(*args[:11], 0, *args[12:], 2, None) == 0  # no tokens: nothing to launch
    bad = list(args)
    bad[0] = 0
    assert f(*bad, 2, None) == E_NULL
    bad = list(args)
    bad[0] = 0x1001
    assert f(*bad, 2, None) == E_ALIGN


def test_static_entry_rejects_oversized_launch_on_the_host(lib):
    """kvh_paged_attention_static checks its workspace need against the static scratch
    (256 MiB) before touching the device: no GPU is needed to see the rejection."""
    a = _attn_args(T=2500, B=2004, W=280, bt_rs=280, max_q=384)
    f = lib.kvh_paged_attention_static
    args = (a["q"], a["q_ts"], a["q_hs"], a["kc"], _lib.i64x3(a["kcs"]), a["vc"], _lib.i64x3(a["vcs"]), a["nb"],
            a["out"], a["o_ts"], a["o_hs"], a["bt"], a["bt_rs"], a["W"], a["sl"], a["qsl"], a["T"], a["B"], a["H"],
            a["Hkv"], a["D"], a["BS"], a["max_q"], a["scale"], a["dtype"], None)  # fmt: skip
    assert lib.kvh_paged_attention_workspace_size(2500, 2004, 32, 8, 128, 280, 16, 384, 2) > 256 << 20
    assert f(*args) == E_SCRATCH
    bad = list(args)
    bad[18] = 30  # H % Hkv != 0: the shape check comes first
    assert f(*bad) == E_SHAPE
    bad = list(args)
    bad[16] = 0  # no tokens: nothing to launch
    assert f(*bad) == 0


def test_workspace_follows_the_plan(lib):
    """Decode partial slots: one per (sequence, head group) plus one per possible decode work
    unit (8192 waves / 8 heads per unit when Hkv % 8 == 0), each holding RS = QS * G rows; merge-job records
    (16 int32) for 8192 decode units, plus 768 prefill units, their two 128-row partial
    slots each and the prefill plan (sequence list, flat starts, one 64-byte record per prefill
    workgroup) when the batch has prefill-class queries."""
    ws = lib.kvh_paged_attention_workspace_size

    def want(B, Hkv, G, QS, D, hgw=8, prefill=False):
        slots = B * Hkv // hgw + 8192 // hgw
        rows = slots * hgw * QS * G
        up = lambda x: -(-x // 256) * 256  # noqa: E731
        jobs = 8192 + (768 if prefill else 0)
        prows = 2 * 768 * 128 if prefill else 0
        plan = up(32) + up(B * 4) + up((B + 1) * 8) + up(768 * 64) if prefill else 0
        return up(rows * D * 4) + up(rows * 2 * 4) + up(jobs * 16 * 4) + up(prows * D * 4) + up(prows * 2 * 4) + plan

    # C1: tables of at most 1024 keys take the short decode (one workgroup per sequence and kv
    # head, partials combined in LDS): no workspace
    assert ws(8, 8, 32, 8, 64, 32, 16, 1, 2) == 0
    assert ws(8, 8, 32, 8, 64, 64, 16, 1, 2) == 0
    assert ws(8, 8, 32, 8, 64, 65, 16, 1, 2) == want(8, 8, 4, 1, 64)
    assert ws(8, 8, 32, 8, 64, 32, 16, 5, 2) == want(8, 8, 4, 5, 64)  # verify rows: two tiles, stream-K
    assert ws(64, 64, 32, 8, 128, 512, 16, 1, 2) == want(64, 8, 4, 1, 128)  # C2
    assert ws(160, 32, 32, 8, 128, 257, 16, 5, 2) == want(32, 8, 4, 5, 128)  # C5: verify rows
    assert ws(2048, 516, 32, 8, 128, 280, 16, 384, 2) == want(516, 8, 4, 4, 128, prefill=True)  # C3
    assert ws(8, 8, 16, 2, 64, 128, 16, 1, 2) == want(8, 2, 8, 1, 64, hgw=2)  # two kv heads

    def cascade(B, Hkv, RS, D, hgw=8):
        # share header, decode list, prefix partials for 64-row groups (16-bit caches, when
        # the batch has more than 16 rows) or 16-row groups (E4M3 caches), whichever is
        # larger: (groups x head groups + 2048 / hgw unit slots) x hgw x group rows, and one
        # merge record per (sequence, head group)
        up = lambda x: -(-x // 256) * 256  # noqa: E731
        nhg = Hkv // hgw

        def rows(nx):
            sg = 1 if RS >= 16 * nx else 16 * nx // RS
            return (-(-B // sg) * nhg + 2048 // hgw) * hgw * 16 * nx

        xr = max(rows(4 if B * RS > 16 else 1), rows(1))
        return up(8 * 8) + up(B * 4) + up(xr * D * 4) + up(xr * 2 * 4) + up(B * nhg * 16 * 4)

    # C4: tables over 8192 keys plan the cascade over a shared prefix
    assert ws(16, 16, 32, 8, 128, 2000, 16, 1, 2) == want(16, 8, 4, 1, 128) + cascade(16, 8, 4, 128)
    assert ws(5, 5, 16, 16, 128, 600, 16, 1, 2) == want(5, 16, 1, 1, 128) + cascade(5, 16, 1, 128)
    assert ws(64, 64, 32, 8, 128, 512, 16, 1, 0) == 0  # fp32 path: no split
    assert ws(64, 64, 30, 8, 128, 512, 16, 1, 2) == 0  # invalid shape


@pytest.mark.parametrize(
    ("args", "status"),
    [
        ((7, 0x1000, 0x2000, 1 << 20, 256, 0), E_SHAPE),  # unknown probe
        ((6, 0x1000, 0x2000, (1 << 20) + 16, 256, 0), E_SHAPE),  # page gather: not whole pages
        ((6, 0x1000, 0x2000, 3 * 4096, 256, 0), E_SHAPE),  # page gather: 3 pages, not a power of two
        ((5, 0x1000, None, 1 << 20, 256, 0), E_NULL),  # non-temporal stream read: a read probe
        ((4, None, 0x2000, 5, 256, 10), E_SHAPE),  # interleave: at most 4 FMAs per MFMA
        ((4, None, 0x2000, 2, 256, 0), E_SHAPE),
        ((3, None, 0x2000, 0, 256, 0), E_SHAPE),  # co-issue with both wave kinds idle
        ((0, 0x1000, 0x2000, 1 << 20, 0, 0), E_SHAPE),  # no workgroups
        ((0, 0x1000, 0x2000, 1 << 20, 70_000, 0), E_SHAPE),
        ((0, 0x1000, None, 1 << 20, 256, 0), E_NULL),
        ((1, None, 0x2000, 1 << 20, 256, 0), E_NULL),
        ((0, 0x1000, 0x2000, 1000, 256, 0), E_SHAPE),  # not whole 16-byte vectors
        ((1, 0x1008, 0x2000, 1 << 20, 256, 0), E_ALIGN),
        ((2, None, 0x2000, 0, 256, 0), E_SHAPE),  # MFMA probe without iterations
        ((2, None, 0x2004, 0, 256, 10), E_ALIGN),
    ],
)
def test_probe_rejects_bad_arguments(lib, args, status):
    """The measurement probes (kvh_probe) validate before any launch."""
    assert lib.kvh_probe(*args, None) == status


def test_get_backend_contract(monkeypatch):
    """The reference's selector (attention.py:113-124): "auto" never raises -- it falls back
    when the backend cannot run or the block size does not tile; "hip" raises RuntimeError /
    ValueError like "triton"; unknown names raise ValueError."""
    fallback = object()
    with pytest.raises(ValueError):
        attention.get_backend("torch", "cuda", 16)
    with pytest.raises(ValueError):
        attention.get_backend("nope", "cuda", 16)
    assert attention.get_backend("auto", "cpu", 16, fallback=fallback) is fallback
    assert attention.get_backend("auto", "cpu", 16) is None
    if not attention.hip_available():
        with pytest.raises(RuntimeError):
            attention.get_backend("hip", "cuda", 16)
        assert attention.get_backend("auto", "cuda", 16, fallback=fallback) is fallback
    monkeypatch.setattr(attention, "hip_available", lambda: True)
    assert attention.get_backend("hip", "cuda", 16) is attention.HipAttention
    assert attention.get_backend("auto", "cuda", 32) is attention.HipAttention
    assert attention.get_backend("auto", "cuda:0", 16, fallback=fallback) is attention.HipAttention
    for bs in (8, 24, 4):  # blocks the 16-token tiles do not divide
        assert attention.get_backend("auto", "cuda", bs, fallback=fallback) is fallback
        with pytest.raises(ValueError):
            attention.get_backend("hip", "cuda", bs)
    assert attention.get_backend("auto", "cpu", 16, fallback=fallback) is fallback
    # head sizes: "auto" keeps the caller's choice unless the MFMA kernels take the heads;
    # "hip" computes any multiple of 8 up to 256 and rejects the rest
    for d in (64, 128):
        assert attention.get_backend("auto", "cuda", 16, fallback=fallback, head_dim=d) is attention.HipAttention
        assert attention.get_backend("hip", "cuda", 16, head_dim=d) is attention.HipAttention
    for d in (32, 80, 96, 256):
        assert attention.get_backend("auto", "cuda", 16, fallback=fallback, head_dim=d) is fallback
        assert attention.get_backend("hip", "cuda", 16, head_dim=d) is attention.HipAttention
    for d in (100, 264, 0):
        assert attention.get_backend("auto", "cuda", 16, fallback=fallback, head_dim=d) is fallback
        with pytest.raises(ValueError):
            attention.get_backend("hip", "cuda", 16, head_dim=d)
    cls = attention.HipAttention
    assert cls.graph_capturable and not cls.needs_padded_layout


class _NoLib:
    """Stands in for the loaded library: any attribute access is a failure."""

    def __getattr__(self, name):
        raise AssertionError(f"{name} reached the library with a host tensor argument")


def test_host_tensors_are_rejected_before_the_library(monkeypatch):
    """A CPU tensor's address must never reach a kernel: every tensor argument is checked
    against the caches' device before any library call (a GPU memory fault otherwise)."""
    monkeypatch.setattr(attention._lib, "load", lambda: _NoLib())
    monkeypatch.setattr(attention._lib, "fast", lambda: _NoLib())
    monkeypatch.setattr(attention, "_workspace_size", lambda *a: 0)
    T, H, Hkv, D, BS, NB = 4, 8, 2, 64, 16, 8
    layout = (NB, BS, Hkv, D, (BS * Hkv * D, Hkv * D, D), (BS * Hkv * D, Hkv * D, D), 0)
    monkeypatch.setattr(attention, "_cache_layout", lambda kc, vc: layout)
    kc = torch.zeros(NB, BS, Hkv, D, dtype=torch.bfloat16)
    q = torch.zeros(T, H, D, dtype=torch.bfloat16)
    k = torch.zeros(T, Hkv, D, dtype=torch.bfloat16)
    slots = torch.arange(T)
    meta = attention.build_metadata("cpu", [[0]], slots.tolist(), [T], [T])
    with pytest.raises(ValueError, match="device"):
        attention.HipAttention.forward(q, kc, kc, meta, 0.125)
    with pytest.raises(ValueError, match="device"):
        attention.HipAttention.write_kv(kc, kc, k, k, slots)
    qkv = torch.zeros(T, (H + 2 * Hkv) * D, dtype=torch.bfloat16)
    cos = torch.zeros(64, D)
    with pytest.raises(ValueError, match="device"):
        attention.HipAttention.rope_and_cache(qkv, slots, cos, cos, kc, kc, slots, H)
    x = torch.zeros(T, 256, dtype=torch.bfloat16)
    w = torch.zeros((H + 2 * Hkv) * D, 256, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="device"):
        attention.HipAttention.gemv_rope_and_cache(x, w, slots, cos, cos, kc, kc, slots, H)


def test_build_metadata_layout():
    tables = [[5, 2], [7], [1, 3, 4]]
    m = attention.build_metadata("cpu", tables, [81, 112, 50, 51], [20, 1, 40], [2, 1, 1], padded_layout=True)
    assert m.block_tables.tolist() == [[5, 2, 0], [7, 0, 0], [1, 3, 4]]  # 0-padded
    assert m.query_start_loc.tolist() == [0, 2, 3, 4]
    assert m.max_seq_len == 40 and m.max_query_len == 2
    for t in (m.slot_mapping, m.block_tables, m.seq_lens, m.query_lens, m.query_start_loc):
        assert t.dtype == torch.int64
    assert m.q_gather.tolist() == [[0, 1], [2, 0], [3, 0]]
    assert m.q_valid.tolist() == [[True, True], [True, False], [True, False]]
    assert attention.build_metadata("cpu", tables, [1, 2, 3, 4], [20, 1, 40], [2, 1, 1]).q_gather is None


def test_baseline_config_shapes():
    c1, c2, c3, c4, c5 = (workloads.baseline_config(i) for i in range(1, 6))
    assert (len(c1.seq_lens), c1.num_heads, c1.num_kv_heads, c1.head_dim) == (8, 32, 8, 64)
    assert all(64 <= s <= 512 for s in c1.seq_lens) and c1.num_blocks == 512
    assert (len(c2.seq_lens), c2.head_dim) == (64, 128) and all(1024 <= s <= 8192 for s in c2.seq_lens)
    assert c3.num_tokens == 2048 and c3.query_lens.count(384) == 4 and c3.query_lens.count(1) == 512
    assert all(0 <= c <= 4096 for c in c3.context_lens[512:])
    assert all(256 <= s <= 4096 for s in c3.seq_lens[:512])
    assert all(t[:750] == c4.tables[0][:750] for t in c4.tables)
    assert all(16_000 <= s <= 32_000 for s in c4.seq_lens) and c4.table_width() == 2000
    assert c5.query_lens == [5] * 32 and all(2048 <= c <= 4096 for c in c5.context_lens)
    for w in (c1, c2, c3, c5):  # disjoint physical blocks
        used = [b for t in w.tables for b in t]
        assert len(used) == len(set(used)) and max(used) < w.num_blocks


def test_byte_and_flop_formulas():
    w = workloads.custom("tiny", [1, 3], [20, 4], 4, 2, 64, 16)
    # seq_lens 21 and 7; keys bytes = 2 * Hkv * D * e * tokens
    assert w.kv_bytes(2) == 2 * 2 * 64 * 2 * 28
    assert w.algorithmic_bytes(2) == w.kv_bytes(2) + 2 * 4 * 4 * 64 * 2 + 8 * (2 + 1) + 8 * 7
    # visible (row, key) pairs: 21 + (5 + 6 + 7) = 39
    assert w.flops() == 4 * 4 * 64 * 39
    c4 = workloads.baseline_config(4)
    shared = 750 * 16
    assert c4.unique_tokens() == shared + sum(s - shared for s in c4.seq_lens)


def test_product_never_imports_the_oracle():
    pkg = ROOT / "kvserve_amd"
    for f in list(pkg.rglob("*.py")) + list(pkg.rglob("*.hip")) + list(pkg.rglob("*.h")):
        text = f.read_text()
        assert not re.search(r"^\s*(from|import)\s+oracle\b", text, re.M), f
        assert "liboracle" not in text, f


def test_load_fails_loudly_without_library(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libkvhip.so")
    with pytest.raises(RuntimeError, match="no fallback"):
        _lib.load()


def test_ctypes_signatures_match_header():
    text = HEADER.read_text()
    for name, (_, args) in _lib.SIGNATURES.items():
        m = re.search(r"KVH_API[^;(]*?\b" + name + r"\s*\(([^;]*?)\)\s*;", text, re.S)
        assert m, name
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(args), (name, len(params), len(args))
    assert ctypes.sizeof(ctypes.c_size_t) == 8


# -- argument checks of the fused engine GEMVs (they return before any HIP call) ------------------
def _glu(lib, **over):
    a = dict(x=0x1000, xs=4096, w=0x2000, ws=4096, y=0x3000, ys=14336, m=1, inter=14336, k=4096, dtype=2)
    a.update(over)
    return lib.kvh_gemv_silu_mul(a["x"], a["xs"], a["w"], a["ws"], a["y"], a["ys"], a["m"], a["inter"], a["k"],
                                 a["dtype"], None)  # fmt: skip


@pytest.mark.parametrize(
    "over,status",
    [
        (dict(dtype=0), E_DTYPE),  # 16-bit only
        (dict(m=5), E_UNSUPPORTED),
        (dict(k=4095), E_UNSUPPORTED),
        (dict(m=-1), E_SHAPE),
        (dict(x=None), E_NULL),
        (dict(ys=100), E_SHAPE),
        (dict(x=0x1008), E_ALIGN),
        (dict(m=0), 0),
    ],
)  # fmt: skip
def test_gemv_silu_mul_validation(lib, over, status):
    assert _glu(lib, **over) == status


def _gr(lib, **over):
    a = dict(x=0x1000, xs=2048, w=0x2000, ws=2048, m=1, k=2048, pos=0x3000, cos=0x4000, sin=0x5000, q=0x6000,
             kc=0x7000, kcs=(16 * 512, 512, 64), vc=0x8000, vcs=(16 * 512, 512, 64), slots=0x9000, H=32, Hkv=8,
             D=64, dtype=2, fp8=0, ks=1.0, vs=1.0)  # fmt: skip
    a.update(over)
    return lib.kvh_gemv_rope_and_cache(
        a["x"], a["xs"], a["w"], a["ws"], a["m"], a["k"], a["pos"], a["cos"], a["sin"], 4096, a["q"], 32 * 64, 64,
        a["kc"], _lib.i64x3(a["kcs"]), a["vc"], _lib.i64x3(a["vcs"]), a["slots"], 64, a["H"], a["Hkv"], a["D"], 16,
        a["dtype"], a["fp8"], a["ks"], a["vs"], None,
    )  # fmt: skip


@pytest.mark.parametrize(
    "over,status",
    [
        (dict(dtype=0), E_DTYPE),
        (dict(fp8=1, ks=0.0), E_SHAPE),
        (dict(m=65), E_UNSUPPORTED),
        (dict(m=5, k=1032, xs=1032, ws=1032), E_UNSUPPORTED),
        (dict(D=63), E_UNSUPPORTED),
        (dict(k=100), E_UNSUPPORTED),
        (dict(slots=None), E_NULL),
        (dict(kcs=(16 * 512, 512, -64)), E_SHAPE),
        (dict(xs=1024), E_SHAPE),
        (dict(w=0x2004), E_ALIGN),
        (dict(q=0x6001), E_ALIGN),
        (dict(m=0), 0),
    ],
)  # fmt: skip
def test_gemv_rope_and_cache_validation(lib, over, status):
    assert _gr(lib, **over) == status


def _sk(lib, **over):
    a = dict(x=0x1000, xs=4096, w=0x2000, ws=4096, y=0x3000, ys=6144, m=8, n=6144, k=4096, dtype=2)
    a.update(over)
    return lib.kvh_gemm_skinny(a["x"], a["xs"], a["w"], a["ws"], a["y"], a["ys"], a["m"], a["n"], a["k"], a["dtype"],
                               None)  # fmt: skip


@pytest.mark.parametrize(
    "over,status",
    [
        (dict(dtype=0), E_DTYPE),
        (dict(m=65), E_UNSUPPORTED),
        (dict(n=6150), E_UNSUPPORTED),
        (dict(k=4000), E_UNSUPPORTED),
        (dict(w=None), E_NULL),
        (dict(xs=1024), E_SHAPE),
        (dict(x=0x1004), E_ALIGN),
        (dict(m=0), 0),
    ],
)  # fmt: skip
def test_gemm_skinny_validation(lib, over, status):
    assert _sk(lib, **over) == status


@pytest.mark.parametrize(
    "over,status",
    [
        (dict(dtype=0), E_DTYPE),
        (dict(m=65), E_UNSUPPORTED),
        (dict(n=6148), E_UNSUPPORTED),  # inter % 8
        (dict(k=4000), E_UNSUPPORTED),
        (dict(y=None), E_NULL),
        (dict(m=0), 0),
    ],
)  # fmt: skip
def test_gemm_skinny_silu_mul_validation(lib, over, status):
    a = dict(x=0x1000, xs=4096, w=0x2000, ws=4096, y=0x3000, ys=6144, m=8, n=6144, k=4096, dtype=2)
    a.update(over)
    st = lib.kvh_gemm_skinny_silu_mul(a["x"], a["xs"], a["w"], a["ws"], a["y"], a["ys"], a["m"], a["n"], a["k"],
                                      a["dtype"], None)  # fmt: skip
    assert st == status


def test_bench_refuses_more_than_one_gpu_and_a_missing_gpu():
    """bench.py measures one GPU: --gpus 2 exits with status 2 and says so; without a GPU it
    exits with status 1 instead of measuring anything on the host."""
    import subprocess
    import sys

    bench = str(ROOT / "bench.py")
    r = subprocess.run([sys.executable, bench, "--gpus", "2"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 2 and "one GPU" in r.stderr and not r.stdout.strip()
    if not torch.cuda.is_available():
        r = subprocess.run([sys.executable, bench, "--only", "1"], capture_output=True, text=True, timeout=300)
        assert r.returncode == 1 and "needs a ROCm GPU" in r.stderr and not r.stdout.strip()


# A kernel shaped like the page-table load of the prefill kernel: a divergent load, then the
# join. SPILL marks where the register allocator put the spill store of a live-everywhere pair.
_ISA_TEMPLATE = """_ZN3kvh4testEv:
; %bb.0:
\tv_cmp_gt_i32_e32 vcc, s5, v0
\ts_and_saveexec_b64 s[8:9], vcc
\ts_cbranch_execz .LBB0_2
; %bb.1:
\tglobal_load_dwordx2 v[4:5], v[4:5], off
{inside}
.LBB0_2:
{before}
\ts_or_b64 exec, exec, s[8:9]
{after}
\ts_cmp_lt_i32 s6, 2
\ts_cbranch_scc1 .LBB0_4
; %bb.3:
\ts_mov_b64 s[2:3], exec
\ts_and_b64 exec, exec, s[10:11]
{masked}
\ts_mov_b64 exec, s[2:3]
.LBB0_4:
{end}
\ts_endpgm
.Lfunc_end0:
"""


def _isa(**kw):
    slots = {k: "" for k in ("inside", "before", "after", "masked", "end")}
    slots.update(kw)
    return _ISA_TEMPLATE.format(**slots)


SPILL = "\tscratch_store_dwordx2 off, v[42:43], off offset:20"
RELOAD = "\tscratch_load_dwordx2 v[42:43], off, off offset:20"


def test_isa_check_finds_spill_stores_under_a_partial_exec_mask():
    from kvserve_amd import isa_check

    assert isa_check.check(_isa(after=SPILL, end=SPILL + "\n" + RELOAD)) == []
    # the faulting shape: the store in the join block ahead of the exec restore
    (hit,) = isa_check.check(_isa(before=SPILL, end=RELOAD))
    assert "scratch_store_dwordx2" in hit and "partial EXEC" in hit
    assert len(isa_check.check(_isa(inside=SPILL))) == 1
    assert len(isa_check.check(_isa(masked=SPILL))) == 1
    # reloads inside a divergent region refill the lanes that use them: not reported
    assert isa_check.check(_isa(inside=RELOAD, masked=RELOAD)) == []


def test_isa_check_joins_take_the_weaker_state():
    from kvserve_amd import isa_check

    # one predecessor of the join restores EXEC, the other arrives with the narrowed mask
    asm = _isa(end=SPILL).replace("\ts_mov_b64 exec, s[2:3]\n", "\ts_cbranch_vccz .LBB0_4\n\ts_mov_b64 exec, s[2:3]\n")
    assert len(isa_check.check(asm)) == 1
    assert isa_check.check(_isa(end=SPILL)) == []


def test_built_kernels_have_no_partial_exec_spills():
    from kvserve_amd import isa_check

    # the device assembly each object was assembled from (kept by the build's -save-temps)
    asms = sorted((Path(__file__).resolve().parents[1] / "kvserve_amd" / "_build").glob("*-hip-amdgcn-amd-amdhsa-gfx950.s"))
    if not asms:
        pytest.skip("no device assembly: run python -m kvserve_amd.build")
    assert [hit for a in asms for hit in isa_check.check(a.read_text())] == []


def test_prefill_priority_change_points_match_the_per_chunk_level():
    """The prefill kernel sets a wave's priority level only at a tile's first chunk and at
    the chunks its `next_drop` names; the level it holds must equal the per-chunk level
    min(3, K left / (total + 1)) at every chunk. Both expressions are taken from the source."""
    src = (Path(__file__).resolve().parent.parent / "kvserve_amd/csrc/paged_attention.hip").read_text()
    steps = int(re.search(r"constexpr int kPrioSteps = (\d+);", src).group(1))
    lvl_src = re.search(r"const int lvl = (min\(3, .*?\));", src).group(1)
    drop_src = re.search(r"next_drop = lvl > 0 \? (.*?) : INT32_MAX;", src).group(1)

    def py(expr):  # the expressions are non-negative integer arithmetic: C / is floor division
        return expr.replace("kPrioSteps", str(steps)).replace("/", "//")

    lvl_of = eval("lambda i, n, rest, total: " + py(lvl_src))  # noqa: S307 (source text of this repo)
    drop_of = eval("lambda lvl, n, rest, total: " + py(drop_src))  # noqa: S307
    big = 1 << 31
    for total in range(1, 90):
        for n in range(1, min(total, 30) + 1):
            for rest in range(0, total - n + 1):
                lvl = lvl_of(0, n, rest, total)
                nxt = drop_of(lvl, n, rest, total) if lvl > 0 else big
                for i in range(n):
                    if i >= nxt:
                        lvl = lvl_of(i, n, rest, total)
                        nxt = drop_of(lvl, n, rest, total) if lvl > 0 else big
                    assert lvl == lvl_of(i, n, rest, total), (total, n, rest, i)


def test_partial_tile_block_layout():
    """The tile-block layout of split-piece partials (multi-tile rows over E4M3 caches):
    `part_ofs`, which the merge reads by, must place a head group's cap rows x D floats as a
    permutation of [0, cap D) in whole float4s, and the writer's store address (lane (j, n) of
    tile t, float4 k of its accumulator row: lp + k 16 m) must be part_ofs of that lane's row
    and column, for every cap a launch uses (RS = q_len G rows) at both MFMA head sizes. The
    expressions are taken from the source."""
    src = (Path(__file__).resolve().parent.parent / "kvserve_amd/csrc/paged_attention.hip").read_text()
    body = re.search(r"int part_ofs\(int r, int c4, int cap\) \{(.*?)\n\}", src, re.S).group(1)
    tnm = re.search(r"const int t = (.*?), n = (.*?), m = (.*?);", body)
    ret = re.search(r"return (.*?);", body).group(1)
    lp = re.search(r"float\* lp = ws_acc \+ (.*?);", src).group(1)
    st = re.search(r"\*\(f32x4\*\)\(lp \+ (.*?)\) =", src).group(1)

    def cdiv(e):  # C integer expressions on non-negative ints -> Python (>>, &, min carry over)
        return e.replace("/", "//")

    def part_ofs(r, c4, cap, D):
        VW = D // 16
        env = {"r": r, "c4": c4, "cap": cap, "D": D, "VW": VW, "min": min}
        env["t"] = eval(cdiv(tnm.group(1)), env)  # noqa: S307 (source text of this repo)
        env["n"] = eval(cdiv(tnm.group(2)), env)  # noqa: S307
        env["m"] = eval(cdiv(tnm.group(3)), env)  # noqa: S307
        return eval(cdiv(ret), env)  # noqa: S307

    for D in (64, 128):
        VW = D // 16
        for cap in (16, 20, 24, 32, 48, 64, 12, 4):
            offs = {part_ofs(r, c4, cap, D) for r in range(cap) for c4 in range(D // 4)}
            assert len(offs) == cap * D // 4 and offs == set(range(0, cap * D, 4)), (D, cap)
            for t in range((cap + 15) // 16):
                m = min(16, cap - 16 * t)
                for j in range(4):
                    for n in range(m):
                        env = {"row_base": 0, "t": t, "D": D, "j": j, "m": m, "n": n, "VW": VW}
                        base = eval(cdiv(lp), env)  # noqa: S307
                        for e in range(4):
                            for i in range(0, VW, 4):
                                env.update(e=e, i=i)
                                got = base + eval(cdiv(st), env)  # noqa: S307
                                # lane (j, n) holds d = VW (4 j + e) + i .. + 3 of row 16 t + n
                                c4 = (VW * (4 * j + e) + i) // 4
                                assert got == part_ofs(16 * t + n, c4, cap, D), (D, cap, t, j, n, e, i)


def test_decode_cost_split_partitions_the_positions():
    """The decode kernel's stream-K split (`CostSplit`: the first P positions cost wp, the others
    wr; the first R1 units take K1 parts of the total cost, the others K2) must give every
    position of [0, C) to exactly one unit, units in order, and `unit_of` must name the unit
    whose range holds each position (the merge records list a segment's pieces by it). Costs
    and shares 1 must give the plain split [u C / NUa, (u + 1) C / NUa). The expressions are
    taken from the source and checked against a walk over every position."""
    src = (Path(__file__).resolve().parent.parent / "kvserve_amd/csrc/paged_attention.hip").read_text()
    body = re.search(r"struct CostSplit \{(.*?)\n\};", src, re.S).group(1)

    def expr(fn):  # the returned expression of a one-line member function
        e = re.search(rf"int64_t {fn}\(int64_t \w+\) const \{{ return (.*?); \}}", body).group(1)
        if " ? " in e:  # c ? a : b (one conditional, at the top level)
            cond, rest = e.split(" ? ", 1)
            a, b = rest.split(" : ", 1)
            e = f"({a}) if ({cond}) else ({b})"
        return e.replace("/", "//")

    fns = [(name, expr(name), arg) for name, arg in
           (("cost", "x"), ("first", "c"), ("cum", "u"), ("begin", "u"), ("unit_at", "m"), ("unit_of", "x"))]
    consts = dict(re.findall(r"constexpr int64_t (kPrefix64Cost|kChunkCost|kRound1Share|kRound2Share) = (\d+)", src))
    consts.update(re.findall(r", (kChunkCost|kRound2Share) = (\d+);", src))
    w64 = (int(consts["kPrefix64Cost"]), int(consts["kChunkCost"]))
    weights = [(1, 1), w64, (10, 8)]
    rounds = (int(consts["kRound1Share"]), int(consts["kRound2Share"]))
    shares = [(1, 1), rounds, (5, 4)]
    # (weights, shares) as the kernel combines them: 64-row prefix groups (16-bit caches: no
    # round shares), E4M3 caches (shares, even costs); and weights with shares together
    used = {((1, 1), (1, 1)), (w64, (1, 1)), ((1, 1), rounds), (w64, rounds), ((10, 8), rounds)}

    def split(P, C, NUa, wp, wr, R1, K1, K2):
        env = {"P": P, "C": C, "NUa": NUa, "wp": wp, "wr": wr, "T": wp * P + wr * (C - P)}
        R1 = min(R1, NUa)
        env.update({"R1": R1, "K1": K1, "K2": K2, "Q": K1 * R1 + K2 * (NUa - R1)})
        for name, e, arg in fns:  # each may call the ones before it
            env[name] = eval(f"lambda {arg}: {e}", env)  # noqa: S307 (source text of this repo)
        return env["begin"], env["unit_of"]

    # the kernel's active units: at most ceil(C / kMinUnitChunks) (active_units)
    internal = (Path(__file__).resolve().parent.parent / "kvserve_amd/csrc/kvh_internal.h").read_text()
    min_chunks = int(re.search(r"kMinUnitChunks = (\d+);", internal + src).group(1))

    rng = random.Random(5)
    cases = [(0, 1, 1), (3, 3, 2), (375, 6375, 128)] + [
        (rng.randint(0, c), c, rng.randint(1, 300)) for c in (rng.randint(1, 4000) for _ in range(300))
    ]
    # every small shape at the kernel's unit counts (NUa <= ceil(C / kMinUnitChunks))
    cases += [(P, C, NUa) for C in range(1, 19) for P in range(C + 1) for NUa in range(1, -(-C // min_chunks) + 1)]
    for P, C, NUa in cases:
        R1 = rng.choice([NUa, NUa // 2, rng.randint(0, NUa)])
        active = NUa <= -(-C // min_chunks)
        for wp, wr in weights:
            for K1, K2 in shares:
                begin, unit_of = split(P, C, NUa, wp, wr, R1, K1, K2)
                assert begin(0) == 0 and begin(NUa) == C, (P, C, NUa, wp, wr, R1, K1, K2)
                for u in range(NUa):
                    a, b = begin(u), begin(u + 1)
                    assert a <= b
                    if wp == wr == K1 == K2 == 1:
                        assert a == u * C // NUa
                    # a segment's pieces sit on consecutive units, one each, and the merge reads
                    # every one: at the kernel's unit counts and the source's weights and shares
                    # (in the combinations the kernel uses) no unit may be empty
                    if active and ((wp, wr), (K1, K2)) in used:
                        assert a < b, ("empty unit", P, C, NUa, wp, wr, R1, K1, K2, u)
                    for x in range(a, b):
                        assert unit_of(x) == u, (P, C, NUa, wp, wr, R1, K1, K2, u, x)
