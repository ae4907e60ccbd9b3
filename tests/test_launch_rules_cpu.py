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
    B = torch.empty(rows, n, dtype=dtype, device="meta")  # the rule reads shape and dtype only
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


class _Ptr:
    """Stands in for B / C in _spmm_lane_shape, which reads only data_ptr()."""

    def __init__(self, addr):
        self.addr = addr

    def data_ptr(self):
        return self.addr


@pytest.mark.parametrize("n,dtype,tile,aligned,want", [
    (256, torch.float32, 128, True, (32, 4)),   # tile 128 = 32 lanes x 4: as chosen
    (256, torch.float64, 64, True, (32, 2)),
    (64, torch.float64, 32, True, (16, 2)),
    (128, torch.float32, 64, True, (16, 4)),
    (255, torch.float32, 128, True, (64, 1)),   # odd N: 4-byte lanes, a launched tile of 64
    (256, torch.float32, 128, False, (64, 1)),  # unaligned B or C: the same
    (100, torch.float32, 64, True, (16, 4)),
    (64, torch.float32, None, True, (16, 4)),   # untiled: the group covers all of N
])
def test_spmm_launched_tile_width(n, dtype, tile, aligned, want):
    # the kernel's tile is lanes * vec columns (lanes <= 64): the rule's tile when 16-byte
    # lanes cover it, else narrower (64 * vec) - more tiles, each re-reading A
    base = 4096 if aligned else 4100
    lanes, vec = spmm_csr._spmm_lane_shape(n, dtype, _Ptr(base), _Ptr(base), tile)
    assert (lanes, vec) == want
    width = n if tile is None else min(n, tile)
    assert lanes * vec == width or (lanes == 64 and lanes * vec < width)
