"""fsp_index_stats on the GPU (csrc/index_stats.hip): bounds of two index arrays and the number
of descents of the first, against torch's reductions on the same arrays, for both index
widths, the edge lengths of the grid (0, 1, partial and capped grids) and values beyond the
int32 range."""

import pytest
import torch

from flagsparse_amd._index_stats import index_stats

pytestmark = pytest.mark.gpu


def _want(a, b):
    if a.numel() == 0:
        return [2**63 - 1, -2**63, 2**63 - 1, -2**63, 0]
    desc = int((a[1:] < a[:-1]).sum()) if a.numel() > 1 else 0
    return [int(a.min()), int(a.max()), int(b.min()), int(b.max()), desc]


@pytest.mark.parametrize("n", [0, 1, 2, 255, 4097, 1 << 20, (1 << 22) + 3, 50_000_000])
@pytest.mark.parametrize("dt_a,dt_b", [(torch.int32, torch.int32), (torch.int64, torch.int32),
                                       (torch.int32, torch.int64), (torch.int64, torch.int64)])
def test_index_stats(dev, n, dt_a, dt_b):
    print(f"index_stats n={n} {dt_a} {dt_b}", flush=True)
    g = torch.Generator(device=dev).manual_seed(n)
    a = torch.randint(-1000, 1 << 30, (n,), generator=g, device=dev, dtype=torch.int64)
    if dt_a == torch.int64 and n:
        a[n // 2] = (1 << 40) + 7  # beyond int32
    b = torch.randint(0, 1 << 31, (n,), generator=g, device=dev, dtype=torch.int64)
    if dt_b == torch.int64 and n:
        b[-1] = -(1 << 35)
    a, b = a.to(dt_a), b.to(dt_b)
    assert index_stats(a, b) == _want(a, b)
    if n > 1:  # views one element in: not 16-byte aligned, the element-wise path
        assert index_stats(a[1:], b[1:]) == _want(a[1:], b[1:])
    s = torch.sort(a).values  # in order: no descents
    assert index_stats(s, b) == _want(s, b)
    assert index_stats(s, b)[4] == 0


def test_index_stats_row_order_cases(dev):
    rows = torch.tensor([0, 0, 1, 3, 3, 2, 5, 5, 4], dtype=torch.int32, device=dev)
    cols = torch.tensor([9, 1, 2, 3, 4, 5, 6, 7, 8], dtype=torch.int32, device=dev)
    assert index_stats(rows, cols) == [0, 5, 1, 9, 2]
    eq = torch.full((10000,), 7, dtype=torch.int32, device=dev)  # equal rows are in order
    assert index_stats(eq, eq)[4] == 0
