// Row-block plans built on the device, for the paths that plan on every call (CSR SpMM
// without a prepared object, COO SpMM) and for the SpMM prepare step: no copy of the row
// pointers to the host and no host loop over rows.
//
// The rows are cut into windows of window_rows rows.  One thread plans its window with the
// rules of the host planner fsp_plan_row_blocks (abi.cpp): a block takes at most rows_cap
// consecutive rows of at most long_threshold entries while their entries fit nnz_cap; a row
// longer than long_threshold becomes ceil(len / chunk) chunk descriptors, and when that is
// more than one it gets a run of partial slots and a combine group.  The one difference is
// that no block crosses a window boundary.  Pass 1 counts each window's descriptors, partial
// slots and split rows (three rows of n_win counters); the caller turns each row into
// exclusive offsets (a prefix sum) and allocates the tables; pass 2 runs the same code and
// writes at those offsets.
//
// When long_threshold == nnz_cap every row that fits a block is short, so a block's end is
// the last row boundary within nnz_cap entries of its start: a binary search over the row
// pointers (about log2(rows_cap) loads per block instead of one per row).  That lets a thread
// plan a wide window quickly, and wide windows cut few blocks short.
//
// Reference behaviour replaced: the bucket planning of spmm_csr.py:417-477
// (_build_spmm_opt_split_metadata's host Python loop over long rows, _build_spmm_opt_buckets).
#include "fsp_device.hpp"
#include "fsp_internal.hpp"

namespace fsp {
namespace {

template <typename P>
__global__ __launch_bounds__(kBlock) void plan_windows_kernel(
    const P* __restrict__ rowptr, int64_t n_rows, int64_t n_win, int64_t window,
    int64_t nnz_cap, int64_t rows_cap, int64_t long_threshold, int64_t chunk,
    int64_t* __restrict__ counts,
    const int64_t* __restrict__ offsets, i32x4* __restrict__ desc, int64_t* __restrict__ ranges,
    i32x4* __restrict__ groups, int64_t* __restrict__ group_base,
    int32_t* __restrict__ split_rows) {
  const int64_t w = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (w >= n_win) return;
  const bool emit = offsets != nullptr;
  int64_t nd = emit ? offsets[w] : 0;
  int64_t np = emit ? offsets[n_win + w] : 0;
  int64_t ns = emit ? offsets[2 * n_win + w] : 0;
  int64_t i = w * window;
  const int64_t end = (i + window < n_rows) ? i + window : n_rows;
  const bool bisect = long_threshold >= nnz_cap;
  while (i < end) {
    const int64_t a = (int64_t)rowptr[i];
    const int64_t len = (int64_t)rowptr[i + 1] - a;
    if (len > long_threshold) {
      const int64_t nch = (len + chunk - 1) / chunk;
      const int64_t base = nch > 1 ? np : -1;
      if (emit) {
        for (int64_t k = 0; k < nch; ++k) {
          i32x4 d;
          d.x = (int)i; d.y = (int)k; d.z = (int)nch; d.w = (int)base;
          desc[nd + k] = d;
          if (ranges) {
            const int64_t lo = a + k * chunk;
            ranges[2 * (nd + k)] = lo;
            ranges[2 * (nd + k) + 1] = (lo + chunk < a + len) ? lo + chunk : a + len;
          }
        }
        if (nch > 1) {
          i32x4 g;
          g.x = (int)ns; g.y = 1; g.z = (int)nch; g.w = 0;
          groups[ns] = g;
          group_base[ns] = base;
          split_rows[ns] = (int32_t)i;
        }
      }
      nd += nch;
      if (nch > 1) {
        np += nch;
        ++ns;
      }
      ++i;
      continue;
    }
    // Row i is short (len <= long_threshold <= nnz_cap), so it always starts a block.
    const int64_t jmax = (i + rows_cap < end) ? i + rows_cap : end;
    int64_t j = i + 1, acc = len;
    if (bisect) {
      // largest j in [i + 1, jmax] with rowptr[j] - a <= nnz_cap (true at j = i + 1)
      int64_t hi = jmax;
      while (j < hi) {
        const int64_t mid = j + (hi - j + 1) / 2;
        if ((int64_t)rowptr[mid] - a <= nnz_cap) j = mid;
        else hi = mid - 1;
      }
      acc = (int64_t)rowptr[j] - a;
    } else {
      while (j < jmax) {
        const int64_t l = (int64_t)rowptr[j + 1] - (int64_t)rowptr[j];
        if (l > long_threshold || acc + l > nnz_cap) break;
        acc += l;
        ++j;
      }
    }
    if (emit) {
      i32x4 d;
      d.x = (int)i; d.y = (int)j; d.z = 0; d.w = 0;
      desc[nd] = d;
      if (ranges) {
        ranges[2 * nd] = a;
        ranges[2 * nd + 1] = a + acc;
      }
    }
    ++nd;
    i = j;
  }
  if (!emit) {
    counts[w] = nd;
    counts[n_win + w] = np;
    counts[2 * n_win + w] = ns;
  }
}

int check_plan_args(int rowptr_bits, int64_t n_rows, int64_t window, int64_t nnz_cap,
                    int64_t rows_cap, int64_t long_threshold, int64_t chunk, const void* rowptr,
                    const char* who) {
  if (rowptr_bits != 32 && rowptr_bits != 64)
    return set_error(FSP_EINVAL, std::string(who) + ": rowptr_bits must be 32 or 64");
  if (n_rows < 0 || n_rows >= 0x7fffffffLL)
    return set_error(FSP_EINVAL, std::string(who) + ": n_rows must be in [0, 2^31-1)");
  if (n_rows > 0 && !rowptr) return set_error(FSP_EINVAL, std::string(who) + ": null rowptr");
  if (nnz_cap < 1 || rows_cap < 1 || chunk < 1 || long_threshold < 1 ||
      long_threshold > nnz_cap || window < 1)
    return set_error(FSP_EINVAL, std::string(who) +
                                     ": need 1 <= long_threshold <= nnz_cap, rows_cap >= 1, "
                                     "chunk >= 1, window_rows >= 1");
  return FSP_OK;
}

template <typename P>
int launch_plan(const void* rowptr, int64_t n_rows, int64_t window, int64_t nnz_cap,
                int64_t rows_cap, int64_t long_threshold, int64_t chunk, int64_t* counts,
                const int64_t* offsets, int32_t* desc, int64_t* ranges, int32_t* groups,
                int64_t* group_base, int32_t* split_rows, hipStream_t st) {
  const int64_t n_win = (n_rows + window - 1) / window;
  if (n_win == 0) return FSP_OK;
  const int64_t blocks = (n_win + kBlock - 1) / kBlock;
  hipLaunchKernelGGL((plan_windows_kernel<P>), dim3((unsigned)blocks), dim3(kBlock), 0, st,
                     static_cast<const P*>(rowptr), n_rows, n_win, window, nnz_cap, rows_cap,
                     long_threshold, chunk, counts, offsets, reinterpret_cast<i32x4*>(desc),
                     ranges, reinterpret_cast<i32x4*>(groups), group_base, split_rows);
  return check_hip(hipGetLastError(), "plan_windows_kernel launch");
}

// The chunk plan of the panel layout on the device, one wave per panel: the greedy rule of
// fsp_plan_panel_chunks (abi.cpp) over the panel's runs in order - a run starts where the
// previous one ended, unless the open chunk already holds runs_cap runs (the rest of the
// chunk is padding); a run longer than the chunk's free space continues in the next chunks
// (each piece counts as a run of the chunk it lies in); the panel's last chunk is padded.
// Writes each run's first position relative to its panel, and each panel's padded length.
// The wave loads 64 run lengths at a time (one coalesced load), then steps through them with
// the chunk state (position, entries and runs of the open chunk) the same in every lane; a
// run's pieces are taken in closed form: the rest of the open chunk, whole chunks, a tail.
constexpr int kPanelPlanBlock = kWave;

__device__ __forceinline__ int64_t readlane64(int64_t v, int lane) {
  const int lo = __builtin_amdgcn_readlane((int)(v & 0xffffffff), lane);
  const int hi = __builtin_amdgcn_readlane((int)(v >> 32), lane);
  return ((int64_t)hi << 32) | (uint32_t)lo;
}

__global__ __launch_bounds__(kPanelPlanBlock) void plan_panel_chunks_kernel(
    const int64_t* __restrict__ panel_runs, const int64_t* __restrict__ run_len, int64_t chunk,
    int64_t runs_cap, int64_t* __restrict__ run_pos, int64_t* __restrict__ panel_len) {
  const int64_t p = blockIdx.x;
  const int lane = threadIdx.x;
  const int64_t r0 = panel_runs[p], r1 = panel_runs[p + 1];
  int64_t pos = 0, used = 0, runs = 0;  // the open chunk's entries and runs (wave-uniform)
  for (int64_t rb = r0; rb < r1; rb += kWave) {
    const int n = r1 - rb < kWave ? (int)(r1 - rb) : kWave;
    const int64_t mine = lane < n ? run_len[rb + lane] : 0;
    int64_t my_pos = 0;
    for (int j = 0; j < n; ++j) {
      int64_t len = readlane64(mine, j);
      if (len < 1) len = 1;  // runs are never empty (checked by the caller)
      if (runs == runs_cap) {  // close the chunk: the rest is padding
        pos += chunk - used;
        used = runs = 0;
      }
      if (lane == j) my_pos = pos;
      const int64_t space = chunk - used;
      pos += len;
      if (len < space) {
        used += len;
        ++runs;
      } else {  // fills the open chunk, then whole chunks, then a tail (a piece of its own)
        const int64_t tail = (len - space) % chunk;
        used = tail;
        runs = tail ? 1 : 0;
      }
    }
    if (lane < n) run_pos[rb + lane] = my_pos;
  }
  if (used > 0) pos += chunk - used;  // the panel's last chunk
  if (lane == 0) panel_len[p] = pos;
}

}  // namespace
}  // namespace fsp

using namespace fsp;

extern "C" int fsp_plan_panel_chunks_device(const int64_t* panel_runs, int64_t n_panels,
                                            const int64_t* run_len, int64_t chunk,
                                            int64_t runs_cap, int64_t* run_pos,
                                            int64_t* panel_len, void* stream) {
  if (n_panels < 0 || chunk < 1 || runs_cap < 1)
    return set_error(FSP_EINVAL, "fsp_plan_panel_chunks_device: need n_panels >= 0, chunk >= 1, "
                                 "runs_cap >= 1");
  if (n_panels == 0) return FSP_OK;
  if (!panel_runs || !panel_len || !run_len || !run_pos)
    return set_error(FSP_EINVAL, "fsp_plan_panel_chunks_device: null pointer");
  if (n_panels > 0x7fffffffLL)
    return set_error(FSP_EINVAL, "fsp_plan_panel_chunks_device: too many panels");
  hipLaunchKernelGGL(plan_panel_chunks_kernel, dim3((unsigned)n_panels), dim3(kPanelPlanBlock), 0,
                     static_cast<hipStream_t>(stream), panel_runs, run_len, chunk, runs_cap,
                     run_pos, panel_len);
  return check_hip(hipGetLastError(), "plan_panel_chunks_kernel launch");
}

extern "C" int fsp_plan_windows_count(const void* rowptr, int rowptr_bits, int64_t n_rows,
                                      int64_t window_rows, int64_t nnz_cap, int64_t rows_cap,
                                      int64_t long_threshold, int64_t chunk, int64_t* counts,
                                      void* stream) {
  int rc = check_plan_args(rowptr_bits, n_rows, window_rows, nnz_cap, rows_cap, long_threshold,
                           chunk, rowptr, "fsp_plan_windows_count");
  if (rc) return rc;
  if (n_rows > 0 && !counts) return set_error(FSP_EINVAL, "fsp_plan_windows_count: null counts");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (rowptr_bits == 32)
    return launch_plan<int>(rowptr, n_rows, window_rows, nnz_cap, rows_cap, long_threshold, chunk,
                            counts, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, st);
  return launch_plan<int64_t>(rowptr, n_rows, window_rows, nnz_cap, rows_cap, long_threshold,
                              chunk, counts, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                              st);
}

extern "C" int fsp_plan_windows_emit(const void* rowptr, int rowptr_bits, int64_t n_rows,
                                     int64_t window_rows, int64_t nnz_cap, int64_t rows_cap,
                                     int64_t long_threshold, int64_t chunk,
                                     const int64_t* offsets, int32_t* desc, int64_t* ranges,
                                     int32_t* groups, int64_t* group_base, int32_t* split_rows,
                                     void* stream) {
  int rc = check_plan_args(rowptr_bits, n_rows, window_rows, nnz_cap, rows_cap, long_threshold,
                           chunk, rowptr, "fsp_plan_windows_emit");
  if (rc) return rc;
  if (n_rows > 0 && (!offsets || !desc))
    return set_error(FSP_EINVAL, "fsp_plan_windows_emit: null offsets or desc");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (rowptr_bits == 32)
    return launch_plan<int>(rowptr, n_rows, window_rows, nnz_cap, rows_cap, long_threshold, chunk,
                            nullptr, offsets, desc, ranges, groups, group_base, split_rows, st);
  return launch_plan<int64_t>(rowptr, n_rows, window_rows, nnz_cap, rows_cap, long_threshold,
                              chunk, nullptr, offsets, desc, ranges, groups, group_base,
                              split_rows, st);
}
