"""The measurement probes behind `bench.py --probes` (kvh_probe) compute what they claim, so
the ceilings they report are measurements of real work (GPU): the stream read and the page
gather fold every dword of their buffer into their sink (the XOR of the sink equals the XOR of
the buffer: the gather's scattered order visits every page once), the copy copies exactly, and
the MFMA, co-issue and interleave probes run to finite sums. Small sizes; no timing."""

import numpy as np
import pytest
import torch

from kvserve_amd import _lib

pytestmark = pytest.mark.gpu


def _probe(lib, kind, src, dst, nbytes, blocks, iters):
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(lib.kvh_probe(kind, src, dst, nbytes, blocks, iters, stream), "kvh_probe")
    torch.cuda.synchronize()


@pytest.mark.parametrize("kind", [0, 5], ids=["ordinary", "non_temporal"])
@pytest.mark.parametrize("nbytes,blocks", [(1 << 20, 4), (3 * (1 << 20) + 4096, 7)])
def test_stream_read_reads_every_dword(hip_device, kind, nbytes, blocks):
    """Buffers the grid does not divide evenly (the tail loop) included; ordinary and
    non-temporal loads."""
    lib = _lib.load()
    g = torch.Generator(device=hip_device).manual_seed(nbytes)
    src = torch.randint(-(1 << 31), (1 << 31) - 1, (nbytes // 4,), generator=g, dtype=torch.int32, device=hip_device)
    sink = torch.zeros(blocks * 256, dtype=torch.int32, device=hip_device)
    _probe(lib, kind, src.data_ptr(), sink.data_ptr(), nbytes, blocks, 0)
    want = np.bitwise_xor.reduce(src.cpu().numpy().view(np.uint32))
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    assert got == want


@pytest.mark.parametrize("pages,blocks", [(256, 4), (64, 3), (1, 1)])
def test_page_gather_reads_every_page(hip_device, pages, blocks):
    """16 pages per wave (whole groups of 4 in flight), runs of 5-6 pages (the tail loop), and
    waves with no page at all."""
    lib = _lib.load()
    nbytes = pages * 4096
    g = torch.Generator(device=hip_device).manual_seed(pages)
    src = torch.randint(-(1 << 31), (1 << 31) - 1, (nbytes // 4,), generator=g, dtype=torch.int32, device=hip_device)
    sink = torch.zeros(blocks * 256, dtype=torch.int32, device=hip_device)
    _probe(lib, 6, src.data_ptr(), sink.data_ptr(), nbytes, blocks, 0)
    want = np.bitwise_xor.reduce(src.cpu().numpy().view(np.uint32))
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    assert got == want


def test_copy_is_exact(hip_device):
    lib = _lib.load()
    n = (5 << 20) + 1024
    src = torch.randint(-(1 << 31), (1 << 31) - 1, (n // 4,), dtype=torch.int32, device=hip_device)
    dst = torch.zeros_like(src)
    _probe(lib, 1, src.data_ptr(), dst.data_ptr(), n, 9, 0)
    assert torch.equal(src, dst)


@pytest.mark.parametrize(
    ("kind", "nbytes", "iters", "threads"),
    [(2, 0, 100, 256), (3, 50, 100, 512), (3, 0, 100, 512), (3, 50, 0, 512)]
    + [(4, nv, 50, 256) for nv in range(5)],
    ids=["mfma", "coissue_both", "coissue_mfma", "coissue_valu"] + [f"interleave_{nv}" for nv in range(5)],
)
def test_compute_probes_run_to_finite_sums(hip_device, kind, nbytes, iters, threads):
    lib = _lib.load()
    blocks = 8
    sink = torch.full((blocks * threads,), float("nan"), dtype=torch.float32, device=hip_device)
    _probe(lib, kind, None, sink.data_ptr(), nbytes, blocks, iters)
    assert torch.isfinite(sink).all()
