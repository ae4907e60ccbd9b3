// C-ABI housekeeping and the host-side row-block planner.
//
// The planner replaces the reference's per-bucket row lists (spmv_csr.py:281-327,
// spmm_csr.py:444-477) and its host Python loop over long rows (spmm_csr.py:417-441) with one
// O(n_rows) greedy pass that emits a descriptor per workgroup.
#include <string>

#include "fsp_internal.hpp"

namespace fsp {

static thread_local std::string g_last_error;

int set_error(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return FSP_OK;
  return set_error(FSP_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

}  // namespace fsp

using namespace fsp;

extern "C" const char* fsp_last_error(void) { return g_last_error.c_str(); }

extern "C" int fsp_abi_version(void) { return 17; }

extern "C" int64_t fsp_spmv_stream_nnz_cap(void) { return kSpmvStreamNnzCap; }
extern "C" int64_t fsp_spmv_stream_rows_cap(void) { return kSpmvStreamRowsCap; }
extern "C" int64_t fsp_spmv_chunk_nnz_cap(void) { return kSpmvChunkCap; }
extern "C" int64_t fsp_spmm_block_nnz_cap(void) { return kSpmmNnzCap; }
extern "C" int64_t fsp_xcs_item_cap(void) { return kXcsItemCap; }
extern "C" int64_t fsp_xcs_rows_cap(void) { return kXcsRowsCap; }
extern "C" int64_t fsp_stage_window_cap(void) { return kStageWinCap; }
extern "C" int64_t fsp_stage_window_rows_cap(void) { return kStageWinRows; }
extern "C" int64_t fsp_stage_chunk(void) { return kStageChunkEntries; }
extern "C" int64_t fsp_xcs_window_slots_cap(void) { return kXcsWinSlotsCap; }
extern "C" int64_t fsp_xcs_window_rows_cap(void) { return kXcsWinRowsCap; }
extern "C" int64_t fsp_xcs_item_runs_cap(void) { return kXcsItemRunsCap; }
extern "C" int64_t fsp_xcs_sorted_item_cap(void) { return kXcsSortedItemCap; }
extern "C" int64_t fsp_xcs_sorted_col_bits(void) { return kXcsSortedColBits; }
extern "C" int64_t fsp_panel_bytes_cap(void) { return kPanelBytes; }
extern "C" int64_t fsp_panel_chunk(void) { return kPanelChunk; }
extern "C" int64_t fsp_panel_chunk_runs_cap(void) { return kPanelChunkRunsCap; }

extern "C" int fsp_plan_row_blocks(const int64_t* rowptr, int64_t n_rows, int64_t nnz_cap,
                                   int64_t rows_cap, int64_t long_threshold, int64_t chunk,
                                   int32_t* desc_out, int64_t* n_desc, int64_t* n_parts,
                                   int64_t* n_split_rows) {
  if (!n_desc || !n_parts || !n_split_rows) return set_error(FSP_EINVAL, "plan: null output");
  if (n_rows < 0) return set_error(FSP_EINVAL, "plan: negative n_rows");
  if (n_rows > 0 && !rowptr) return set_error(FSP_EINVAL, "plan: null rowptr");
  if (n_rows >= 0x7fffffffLL) return set_error(FSP_EINVAL, "plan: n_rows must be < 2^31-1");
  if (nnz_cap < 1 || rows_cap < 1 || chunk < 1 || long_threshold < 1 || long_threshold > nnz_cap)
    return set_error(FSP_EINVAL, "plan: need 1 <= long_threshold <= nnz_cap, rows_cap >= 1, chunk >= 1");
  int64_t nd = 0, np = 0, ns = 0;
  auto emit = [&](int64_t a, int64_t b, int64_t c, int64_t d) {
    if (desc_out) {
      int32_t* o = desc_out + 4 * nd;
      o[0] = (int32_t)a;
      o[1] = (int32_t)b;
      o[2] = (int32_t)c;
      o[3] = (int32_t)d;
    }
    ++nd;
  };
  int64_t i = 0;
  while (i < n_rows) {
    const int64_t len = rowptr[i + 1] - rowptr[i];
    if (len < 0) return set_error(FSP_EINVAL, "plan: rowptr must be non-decreasing");
    if (len > long_threshold) {
      const int64_t nch = (len + chunk - 1) / chunk;
      if (nch > 0x7fffffffLL || np + nch > 0x7fffffffLL)
        return set_error(FSP_EINVAL, "plan: too many chunks");
      const int64_t base = nch > 1 ? np : -1;
      for (int64_t k = 0; k < nch; ++k) emit(i, k, nch, base);
      if (nch > 1) {
        np += nch;
        ++ns;
      }
      ++i;
      continue;
    }
    int64_t j = i, acc = 0;
    while (j < n_rows && j - i < rows_cap) {
      const int64_t l = rowptr[j + 1] - rowptr[j];
      if (l < 0) return set_error(FSP_EINVAL, "plan: rowptr must be non-decreasing");
      if (l > long_threshold || acc + l > nnz_cap) break;
      acc += l;
      ++j;
    }
    emit(i, j, 0, 0);
    i = j;
  }
  if (nd > 0x7fffffffLL) return set_error(FSP_EINVAL, "plan: more than 2^31-1 descriptors");
  *n_desc = nd;
  *n_parts = np;
  *n_split_rows = ns;
  return FSP_OK;
}

// Chunks of the panel layout, greedily: each panel's runs (a row's entries in that panel) are
// laid out one after the other; a chunk (chunk entries) closes when it is full, or after the
// runs_cap-th run that starts or continues in it, in which case the rest of it is padding.  A
// run longer than what is left of a chunk continues in the next one (and counts there too).
extern "C" int fsp_plan_panel_chunks(const int64_t* panel_runs, int64_t n_panels,
                                     const int64_t* run_len, int64_t chunk, int64_t runs_cap,
                                     int64_t* run_pos, int64_t* panel_end) {
  if (n_panels < 0 || chunk < 1 || runs_cap < 1)
    return set_error(FSP_EINVAL, "fsp_plan_panel_chunks: need n_panels >= 0, chunk >= 1, "
                                 "runs_cap >= 1");
  if (n_panels > 0 && (!panel_runs || !panel_end))
    return set_error(FSP_EINVAL, "fsp_plan_panel_chunks: null pointer");
  if (n_panels > 0 && panel_runs[0] != 0)
    return set_error(FSP_EINVAL, "fsp_plan_panel_chunks: panel_runs[0] must be 0");
  int64_t pos = 0;
  for (int64_t p = 0; p < n_panels; ++p) {
    const int64_t r0 = panel_runs[p], r1 = panel_runs[p + 1];
    if (r1 < r0) return set_error(FSP_EINVAL, "fsp_plan_panel_chunks: panel_runs decreasing");
    if (r1 > r0 && (!run_len || !run_pos))
      return set_error(FSP_EINVAL, "fsp_plan_panel_chunks: null run arrays");
    int64_t used = 0, runs = 0;  // entries and runs of the open chunk
    for (int64_t r = r0; r < r1; ++r) {
      int64_t left = run_len[r];
      if (left < 1) return set_error(FSP_EINVAL, "fsp_plan_panel_chunks: empty run");
      if (runs == runs_cap) {  // close the chunk: the rest is padding
        pos += chunk - used;
        used = runs = 0;
      }
      run_pos[r] = pos;
      while (left > 0) {
        const int64_t piece = left < chunk - used ? left : chunk - used;
        ++runs;
        used += piece;
        pos += piece;
        left -= piece;
        if (used == chunk) used = runs = 0;
      }
    }
    if (used > 0) pos += chunk - used;  // the panel's last chunk
    panel_end[p] = pos;
  }
  return FSP_OK;
}
