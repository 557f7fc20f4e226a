"""The read-only ceiling kernel (nc_debug_read_pages) reads exactly the pages it is given: the XOR of its checksum
words equals the XOR of every dword of those pages, computed on the host, for page order, a random order, an order
with repeats and out-of-range entries (read as page 0), odd page counts and grids with idle waves."""
import numpy as np
import pytest
import torch

from nanochat_amd.native import pointer, stream

pytestmark = pytest.mark.gpu


def expected(src_np, order, n):
    """XOR of every dword of the pages read: page order[i] (page 0 when outside the buffer), or page i."""
    pages = src_np.view(np.uint32).reshape(-1, 512)
    idx = np.arange(n) if order is None else np.where((order >= 0) & (order < len(pages)), order, 0)
    return int(np.bitwise_xor.reduce(pages[idx].ravel())) if n else 0


@pytest.mark.parametrize("pages,n,grid,kind", [(300, 300, 4, "page"), (300, 300, 7, "random"), (97, 211, 3, "repeats"),
                                               (64, 5, 16, "page"), (64, 0, 2, "page"), (33, 40, 1, "bad")])
def test_checksum_covers_exactly_the_pages(lib, device, pages, n, grid, kind):
    rng = np.random.default_rng(pages * 1000 + n)
    src_np = rng.integers(0, 256, pages * 2048, dtype=np.uint8)
    if kind == "page":
        order = None
    elif kind == "random":
        order = rng.permutation(pages).astype(np.int32)
    elif kind == "repeats":
        order = rng.integers(0, pages, n).astype(np.int32)
    else:
        order = rng.integers(-5, pages + 5, n).astype(np.int32)
    src = torch.from_numpy(src_np).to(device)
    ord_t = None if order is None else torch.from_numpy(order).to(device)
    sink = torch.full((grid * 256,), 0x5A5A5A5A, dtype=torch.int32, device=device)
    rc = lib.nc_debug_read_pages(pointer(src), src.numel(), None if ord_t is None else pointer(ord_t), n, grid,
                                 pointer(sink), stream())
    assert rc == 0
    torch.cuda.synchronize()
    got = int(np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32)))
    assert got == expected(src_np, order, n)
