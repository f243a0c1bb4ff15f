"""The E4M3 oracle (oracle/fp8.py) pinned on the CPU against the format's definition.

PyTorch's float8_e4m3fn conversion is the quantizer the GPU write kernels are checked
against; here it is pinned by the closed form of E4M3 (bias 7, 3 mantissa bits, subnormals,
0x7f / 0xff NaN, largest 448): every byte decodes to its closed-form value, every finite value
encodes back to its byte, midpoints between neighbours round to the even byte, values beyond
448 saturate (through the clamp) and the scale divides. Also the argument checks of the
*_fp8 C entry points, which return before any HIP call.
"""

from __future__ import annotations

import math

import pytest
import torch

from kvserve_amd import _lib
from oracle import fp8

E_NULL, E_SHAPE, E_DTYPE, E_ALIGN, E_UNSUPPORTED = -1, -2, -3, -4, -5


def test_every_code_decodes_to_the_closed_form():
    codes = torch.arange(256, dtype=torch.uint8)
    got = codes.view(fp8.FP8).float().tolist()
    for c in range(256):
        want = fp8.e4m3_value(c)
        if math.isnan(want):
            assert math.isnan(got[c]) and c in (0x7F, 0xFF)
        else:
            assert got[c] == want and math.copysign(1.0, got[c]) == math.copysign(1.0, want), c
    assert fp8.e4m3_value(0x7E) == 448.0 and fp8.e4m3_value(0x01) == 2.0**-9 and fp8.e4m3_value(0x38) == 1.0


def test_every_finite_value_encodes_back_to_its_code():
    finite = [c for c in range(256) if not math.isnan(fp8.e4m3_value(c))]
    vals = torch.tensor([fp8.e4m3_value(c) for c in finite])
    assert fp8.quantize(vals, 1.0).view(torch.uint8).tolist() == finite


def test_midpoints_round_to_even_and_neighbours_to_nearest():
    pos = sorted((fp8.e4m3_value(c), c) for c in range(0x00, 0x7F))
    mids, want, want_b, want_a = [], [], [], []
    for (v0, c0), (v1, c1) in zip(pos, pos[1:]):
        mids.append((v0 + v1) / 2)  # exact in fp32: 5 significant bits at most
        want.append(c0 if c0 % 2 == 0 else c1)
        want_b.append(c0)
        want_a.append(c1)
    m32 = torch.tensor(mids, dtype=torch.float64).float()
    assert m32.double().tolist() == mids
    assert fp8.quantize(m32, 1.0).view(torch.uint8).tolist() == want
    # the fp32 neighbours of each midpoint round to the nearer code
    lo = torch.nextafter(m32, torch.tensor(-math.inf))
    hi = torch.nextafter(m32, torch.tensor(math.inf))
    assert fp8.quantize(lo, 1.0).view(torch.uint8).tolist() == want_b
    assert fp8.quantize(hi, 1.0).view(torch.uint8).tolist() == want_a
    # negatives mirror with the sign bit
    assert fp8.quantize(-m32, 1.0).view(torch.uint8).tolist() == [c | 0x80 for c in want]


def test_saturation_nan_signed_zero_and_scale():
    x = torch.tensor([448.0, 449.0, 464.0, 1e6, math.inf, -1e6, -math.inf, -1e-30, 0.0, math.nan])
    got = fp8.quantize(x, 1.0).view(torch.uint8).tolist()
    assert got[:8] == [0x7E, 0x7E, 0x7E, 0x7E, 0x7E, 0xFE, 0xFE, 0x80] and got[8] == 0x00
    assert got[9] in (0x7F, 0xFF)
    # the scale divides: 3 / 3 = 1.0 exactly, 0.75 / 0.5 = 1.5
    assert fp8.quantize(torch.tensor([3.0, 0.75]), torch.tensor(3.0).item()).view(torch.uint8).tolist()[0] == 0x38
    assert fp8.quantize(torch.tensor([0.75]), 0.5).view(torch.uint8).tolist() == [0x3C]
    c = torch.tensor([0x3C, 0xBC], dtype=torch.uint8).view(fp8.FP8)
    assert fp8.dequantize(c, 0.5).tolist() == [0.75, -0.75]


# -- argument checks of the *_fp8 entry points ---------------------------------------------------
@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def _rac8(lib, **over):
    a = dict(k=0x1000, kts=1024, khs=128, v=0x2000, vts=1024, vhs=128, kc=0x3000, kcs=(16 * 1024, 1024, 128),
             vc=0x4000, vcs=(16 * 1024, 1024, 128), slots=0x5000, T=4, nb=64, Hkv=8, D=128, BS=16, dtype=2,
             ks=1.0, vs=1.0)  # fmt: skip
    a.update(over)
    return lib.kvh_reshape_and_cache_fp8(
        a["k"], a["kts"], a["khs"], a["v"], a["vts"], a["vhs"], a["kc"], _lib.i64x3(a["kcs"]), a["vc"],
        _lib.i64x3(a["vcs"]), a["slots"], a["T"], a["nb"], a["Hkv"], a["D"], a["BS"], a["dtype"], a["ks"], a["vs"],
        None,
    )  # fmt: skip


@pytest.mark.parametrize(
    "over,status",
    [
        (dict(dtype=3), E_DTYPE),
        (dict(ks=0.0), E_SHAPE),
        (dict(vs=-1.0), E_SHAPE),
        (dict(ks=math.inf), E_SHAPE),
        (dict(vs=math.nan), E_SHAPE),
        (dict(D=12), E_UNSUPPORTED),
        (dict(k=None), E_NULL),
        (dict(k=0x1008), E_ALIGN),  # source rows need 16-byte alignment
        (dict(kc=0x3004), E_ALIGN),  # cache rows need 8-byte alignment
        (dict(kcs=(16 * 1024, 1024, 4)), E_ALIGN),
        (dict(kts=1020), E_ALIGN),
    ],
)  # fmt: skip
def test_reshape_and_cache_fp8_rejects_bad_arguments(lib, over, status):
    assert _rac8(lib, **over) == status


def _pa8(lib, **over):
    a = dict(q=0x1000, kcs=(16 * 1024, 1024, 128), vcs=(16 * 1024, 1024, 128), ks=1.0, vs=1.0, dtype=2, ws=0,
             ws_bytes=0, D=128, BS=16)  # fmt: skip
    a.update(over)
    return lib.kvh_paged_attention_fp8(
        a["q"], 32 * 128, 128, 0x2000, _lib.i64x3(a["kcs"]), 0x3000, _lib.i64x3(a["vcs"]), 64, 0x4000, 32 * 128, 128,
        0x5000, 128, 128, 0x6000, 0x7000, 8, 8, 32, 8, a["D"], a["BS"], 1, 128**-0.5, a["ks"], a["vs"], a["dtype"],
        a["ws"], a["ws_bytes"], None,
    )  # fmt: skip


@pytest.mark.parametrize(
    "over,status",
    [
        (dict(dtype=0), E_UNSUPPORTED),  # fp32 queries have no E4M3 path
        (dict(D=96), E_UNSUPPORTED),  # E4M3 caches feed the MFMA kernels only: D 64 / 128,
        (dict(BS=8), E_UNSUPPORTED),  # pages of whole 16-token tiles
        (dict(ks=0.0), E_SHAPE),
        (dict(vs=math.inf), E_SHAPE),
        (dict(kcs=(16 * 1024, 1024, 8)), E_ALIGN),  # E4M3 rows are read 16 bytes at a time
        (dict(ws=0, ws_bytes=0), -6),  # a workspace is required
    ],
)  # fmt: skip
def test_paged_attention_fp8_rejects_bad_arguments(lib, over, status):
    assert _pa8(lib, **over) == status
