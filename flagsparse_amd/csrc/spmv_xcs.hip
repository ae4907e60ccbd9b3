// CSR / COO-run SpMV for gfx950 with the columns split into one panel per XCD ("XCS" layout).
//
// Why: a CSR SpMV whose columns are spread over an x larger than one XCD's 4 MiB L2 pays a
// full 128-byte line from the fabric for almost every 4-byte x gather.  Here the columns are
// cut into eight panels of about equal nnz and every workgroup that gathers from panel p runs
// on XCD p, so each XCD's L2 holds only its eighth of x.
//
// Layout (built by the host prepare step, flagsparse_amd/_spmv_layouts.py):
//   tiles   contiguous row ranges [r0, r0 + R), R <= kXcsRowsCap (a long row is a tile alone)
//   items   the entries of one tile that fall in one panel, cut into pieces of <= kXcsItemCap
//           entries; each item's entries are contiguous in (vals, pidx), start on a multiple
//           of 4, and are ordered by row (original order inside a row)
//   pidx    (local row << col_bits) | (column - panel_base[panel])
//   rows    "direct" when all of a row's entries lie in one item: that item writes y;
//           "split" otherwise: every item of the tile writes one partial per split row (zero
//           when it holds none of that row) and a second launch (split_row_combine_kernel)
//           adds the tile's partials in item order - a fixed order, so the result does not
//           depend on timing; "empty" rows are written as 0 by the tile's first item.
//           No workgroup waits for or signals another: a device-scope fence would write back
//           and invalidate the XCD's L2, which holds the x panel this layout exists to keep.
//
// Reference behaviour followed (src/flagsparse/sparse_operations/): spmv_csr.py:94-120 (row
// sums; fp32 summed in fp64 on the default path, :498-536) and :161-279 (opt path, native
// accumulation); spmv_coo.py:51-108 (one output per row run).
#include "fsp_device.hpp"
#include "fsp_internal.hpp"

namespace fsp {
namespace {

constexpr int kItemCap = (int)kXcsItemCap;
constexpr int kRowsCap = (int)kXcsRowsCap;
constexpr int kItemUPT = kItemCap / (4 * kBlock);  // quads of entries per thread
static_assert(kItemUPT * 4 * kBlock == kItemCap, "item capacity must be whole quads per thread");
static_assert(kRowsCap % 32 == 0 && kRowsCap <= 65535, "row ids are kept as 16-bit values");

__device__ __forceinline__ bool mask_bit(const uint32_t* m, int r) {
  return (m[r >> 5] >> (r & 31)) & 1u;
}

template <typename T, typename A, bool NT>
__global__ __launch_bounds__(kBlock) void spmv_xcs_kernel(
    const T* __restrict__ vals, const uint32_t* __restrict__ pidx,
    const int* __restrict__ panel_base, int col_bits, const T* __restrict__ x,
    T* __restrict__ y, const int* __restrict__ row_map, const i32x4* __restrict__ items,
    int n_slots, const i32x4* __restrict__ tiles, const int64_t* __restrict__ tile_part_base,
    const uint32_t* __restrict__ masks, A* __restrict__ partials) {
  __shared__ A s_prod[kItemCap];
  __shared__ uint16_t s_row[kItemCap];
  __shared__ int16_t s_start[kRowsCap];  // first entry of each local row in this item, -1: none
  __shared__ int16_t s_end[kRowsCap];    // one past its last entry
  __shared__ uint32_t s_split[kRowsCap / 32];
  __shared__ uint32_t s_empty[kRowsCap / 32];
  __shared__ int s_rank[kRowsCap / 32];

  const int tid = threadIdx.x;
  const int slot = xcd_logical_block(blockIdx.x, n_slots);
  const i32x4 d0 = items[2 * slot];
  const i32x4 d1 = items[2 * slot + 1];
  const int tile = d0.z;
  if (tile < 0) return;  // padding slot
  const int e0 = d0.x, len = d0.y, k = d0.w;
  const int r0 = d1.x, R = d1.y, panel = d1.z;
  if (R <= 0 || R > kRowsCap || len < 0 || len > kItemCap) return;  // not a planner item
  const i32x4 td = tiles[tile];
  const int mask_off = td.x, S = td.y;
  const int W = (R + 31) >> 5;

  for (int w = tid; w < W; w += kBlock) {
    s_split[w] = masks[mask_off + w];
    s_empty[w] = masks[mask_off + W + w];
  }
  for (int r = tid; r < R; r += kBlock) s_start[r] = -1;

  // Entries -> products and local rows in LDS.
  const int cbase = panel_base[panel];
  const uint32_t cmask = (1u << col_bits) - 1u;
  T v[kItemUPT][4];
  uint32_t c[kItemUPT][4];
#pragma unroll
  for (int u = 0; u < kItemUPT; ++u) {
    const int i = 4 * (tid + u * kBlock);
    if (i < len) {
      if constexpr (sizeof(T) == 4) {
        const f32x4 vv = ld_stream<NT>(reinterpret_cast<const f32x4*>(vals + e0 + i));
        v[u][0] = vv.x; v[u][1] = vv.y; v[u][2] = vv.z; v[u][3] = vv.w;
      } else {
        const f64x2 a = ld_stream<NT>(reinterpret_cast<const f64x2*>(vals + e0 + i));
        const f64x2 b = ld_stream<NT>(reinterpret_cast<const f64x2*>(vals + e0 + i + 2));
        v[u][0] = a.x; v[u][1] = a.y; v[u][2] = b.x; v[u][3] = b.y;
      }
      const i32x4 cc = ld_stream<NT>(reinterpret_cast<const i32x4*>(pidx + e0 + i));
      c[u][0] = (uint32_t)cc.x; c[u][1] = (uint32_t)cc.y;
      c[u][2] = (uint32_t)cc.z; c[u][3] = (uint32_t)cc.w;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) { v[u][j] = T(0); c[u][j] = 0u; }
    }
  }
  T xv[kItemUPT][4];
#pragma unroll
  for (int u = 0; u < kItemUPT; ++u)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = 4 * (tid + u * kBlock) + j;
      xv[u][j] = i < len ? x[cbase + (int)(c[u][j] & cmask)] : T(0);
    }
#pragma unroll
  for (int u = 0; u < kItemUPT; ++u)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = 4 * (tid + u * kBlock) + j;
      if (i < len) {
        s_prod[i] = A(v[u][j]) * A(xv[u][j]);
        s_row[i] = (uint16_t)(c[u][j] >> col_bits);
      }
    }
  __syncthreads();
  // Row runs: entries are ordered by local row, so each present row is one run [start, end).
  for (int i = tid; i < len; i += kBlock) {
    const int r = s_row[i];
    if (i == 0 || s_row[i - 1] != r) s_start[r] = (int16_t)i;
    if (i == len - 1 || s_row[i + 1] != r) s_end[r] = (int16_t)(i + 1);
  }

  // Split-row ranks: s_rank[w] = split rows in words [0, w).
  if (tid < 64) {
    int carry = 0;
    for (int w0 = 0; w0 < W; w0 += 64) {
      const int w = w0 + tid;
      const int cnt = w < W ? __popc(s_split[w]) : 0;
      int incl = cnt;
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const int t = __shfl_up(incl, off, kWave);
        if (tid >= off) incl += t;
      }
      if (w < W) s_rank[w] = carry + incl - cnt;
      carry += __shfl(incl, kWave - 1, kWave);
    }
  }
  __syncthreads();

  const int64_t pbase = tile_part_base[tile];
  // Lanes per row: the largest power of two G <= 64 with G * next_pow2(R) <= 256.
  int lg = 0;
  if (R < kBlock) {
    int p2 = 1, lp = 0;
    while (p2 < R) { p2 <<= 1; ++lp; }
    lg = 8 - lp;
    if (lg > 6) lg = 6;
  }
  const int G = 1 << lg;
  const int ngrp = kBlock >> lg;
  const int grp = tid >> lg, lane = tid & (G - 1);
  for (int r = grp; r < R; r += ngrp) {
    if (mask_bit(s_empty, r)) {
      if (k == 0 && lane == 0) {
        const int row = r0 + r;
        y[row_map ? row_map[row] : row] = T(0);
      }
      continue;
    }
    const bool split = mask_bit(s_split, r);
    const int lo = s_start[r];
    if (!split && lo < 0) continue;  // a direct row written by another item
    const int hi = lo < 0 ? lo : s_end[r];
    A acc = A(0);
    for (int i = lo + lane; i < hi; i += G) acc += s_prod[i];
    if (G > 1) acc = group_sum(acc, G);
    if (lane == 0) {
      if (split) {
        const int s = s_rank[r >> 5] + __popc(s_split[r >> 5] & ((1u << (r & 31)) - 1u));
        partials[pbase + (int64_t)k * S + s] = acc;
      } else {
        const int row = r0 + r;
        y[row_map ? row_map[row] : row] = T(acc);
      }
    }
  }
}

template <typename T, typename A>
int launch_xcs(const void* vals, const uint32_t* pidx, const int32_t* panel_base, int col_bits,
               const void* x, void* y, const int32_t* row_map, const int32_t* items,
               int64_t n_slots, const int32_t* tiles, const int64_t* tile_part_base,
               const uint32_t* masks, void* partials, const int32_t* groups,
               const int64_t* group_base, const int32_t* split_rows, int64_t n_groups,
               hipStream_t st) {
  hipLaunchKernelGGL((spmv_xcs_kernel<T, A, true>), dim3((unsigned)n_slots), dim3(kBlock), 0, st,
                     static_cast<const T*>(vals), pidx, panel_base, col_bits,
                     static_cast<const T*>(x), static_cast<T*>(y), row_map,
                     reinterpret_cast<const i32x4*>(items), (int)n_slots,
                     reinterpret_cast<const i32x4*>(tiles), tile_part_base, masks,
                     static_cast<A*>(partials));
  int rc = check_hip(hipGetLastError(), "spmv_xcs_kernel launch");
  if (rc || n_groups == 0) return rc;
  hipLaunchKernelGGL((split_row_combine_kernel<T, A>), dim3((unsigned)n_groups), dim3(kBlock), 0,
                     st, reinterpret_cast<const i32x4*>(groups), group_base, split_rows,
                     static_cast<const A*>(partials), static_cast<T*>(y), row_map);
  return check_hip(hipGetLastError(), "split_row_combine_kernel launch");
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace fsp

using namespace fsp;

extern "C" int fsp_spmv_xcs(int dtype, int acc_f64, const void* vals, const uint32_t* pidx,
                            int64_t n_entries, const int32_t* panel_base, int col_bits,
                            const void* x, void* y, const int32_t* row_map, int64_t n_out,
                            const int32_t* items, int64_t n_slots, const int32_t* tiles,
                            const int64_t* tile_part_base, const uint32_t* masks,
                            void* partials, const int32_t* groups, const int64_t* group_base,
                            const int32_t* split_rows, int64_t n_groups, void* stream) {
  if (dtype != FSP_F32 && dtype != FSP_F64) return set_error(FSP_ENOTSUP, "fsp_spmv_xcs: dtype");
  if (n_entries < 0 || n_slots < 0 || n_out < 0 || n_groups < 0)
    return set_error(FSP_EINVAL, "fsp_spmv_xcs: negative size");
  if (n_entries > 0x7fffffffLL - kXcsItemCap || n_slots > 0x3fffffffLL ||
      n_groups > 0x7fffffffLL)
    return set_error(FSP_EINVAL, "fsp_spmv_xcs: too many entries, slots or groups");
  if (col_bits < 1 || col_bits > 24)
    return set_error(FSP_EINVAL, "fsp_spmv_xcs: col_bits outside [1, 24]");
  if (n_slots > 0 && (!vals || !pidx || !panel_base || !x || !y || !items || !tiles ||
                      !tile_part_base || !masks))
    return set_error(FSP_EINVAL, "fsp_spmv_xcs: null pointer");
  if (n_groups > 0 && (!groups || !group_base || !split_rows || !partials))
    return set_error(FSP_EINVAL, "fsp_spmv_xcs: null split-row pointer");
  if (!aligned16(vals) || !aligned16(pidx) || !aligned16(items) || !aligned16(tiles) ||
      !aligned16(groups))
    return set_error(FSP_EINVAL,
                     "fsp_spmv_xcs: vals, pidx, items, tiles and groups must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (row_map && n_out > 0) {
    int rc = (dtype == FSP_F32) ? fill_zero<float>(static_cast<float*>(y), n_out, st)
                                : fill_zero<double>(static_cast<double*>(y), n_out, st);
    if (rc) return rc;
  }
  if (n_slots == 0) return FSP_OK;
  if (dtype == FSP_F32) {
    if (acc_f64)
      return launch_xcs<float, double>(vals, pidx, panel_base, col_bits, x, y, row_map, items,
                                       n_slots, tiles, tile_part_base, masks, partials, groups,
                                       group_base, split_rows, n_groups, st);
    return launch_xcs<float, float>(vals, pidx, panel_base, col_bits, x, y, row_map, items,
                                    n_slots, tiles, tile_part_base, masks, partials, groups,
                                    group_base, split_rows, n_groups, st);
  }
  return launch_xcs<double, double>(vals, pidx, panel_base, col_bits, x, y, row_map, items,
                                    n_slots, tiles, tile_part_base, masks, partials, groups,
                                    group_base, split_rows, n_groups, st);
}
