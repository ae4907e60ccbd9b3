"""Launch-shape rules that need no GPU: the automatic column tiles of SpMM (spmm_csr._auto_tile_cols)
and the lanes per entry of SDDMM (sddmm_csr._sddmm_lane_shape), on CPU tensors of the shapes
they are measured on."""

import pytest
import torch

from flagsparse_amd import sddmm_csr, spmm_csr


@pytest.mark.parametrize("rows,n,dtype,want", [
    (1 << 20, 64, torch.float32, None),   # 256 MiB: untiled
    (1 << 20, 32, torch.float64, None),   # 256 MiB
    (1 << 20, 64, torch.float64, 32),     # 512 MiB: half-width tiles
    (1 << 20, 128, torch.float32, 64),
    (1 << 20, 256, torch.float32, 128),   # 1 GiB: 512 MiB slices
    (1 << 20, 256, torch.float64, 64),    # 2 GiB
    (1 << 20, 100, torch.float32, 64),    # not a power of two: tiles of 64 and 36
    (1000, 16, torch.float32, None),
])
def test_spmm_auto_tile_cols(rows, n, dtype, want):
    B = torch.empty(rows, n, dtype=dtype)
    t = spmm_csr._auto_tile_cols(B)
    assert t == want
    if t is not None:  # a tile is narrower than B and its slice fits the byte limit
        assert t < n and rows * t * B.element_size() <= spmm_csr.SPMM_B_TILE_BYTES


@pytest.mark.parametrize("K,dtype,want", [
    (1, torch.float32, (1, 1)), (8, torch.float32, (2, 4)), (32, torch.float32, (8, 4)),
    (64, torch.float32, (16, 4)), (128, torch.float32, (16, 4)), (256, torch.float32, (16, 4)),
    (512, torch.float32, (32, 4)),       # 16 lanes would not hold K in four steps
    (33, torch.float64, (16, 1)), (64, torch.float64, (16, 2)), (128, torch.float64, (16, 2)),
])
def test_sddmm_lane_shape(K, dtype, want):
    x = torch.empty(16, K, dtype=dtype)
    y = torch.empty(16, K, dtype=dtype)
    lanes, vec = sddmm_csr._sddmm_lane_shape(K, x, y)
    assert (lanes, vec) == want
    assert lanes <= 16 or K > 4 * (lanes // 2) * vec
