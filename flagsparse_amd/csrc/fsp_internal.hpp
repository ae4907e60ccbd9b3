// Host-side helpers shared by the C-ABI translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "flagsparse_hip.h"

namespace fsp {

// Kernel capacities (see the kernels for why each value is what it is).
constexpr int64_t kSpmvStreamSlots = 1024;               // LDS product slots per short-row block
constexpr int64_t kSpmvStreamNnzCap = kSpmvStreamSlots - 3;
constexpr int64_t kSpmvStreamRowsCap = 1024;
constexpr int64_t kSpmvChunkUnitsPerThread = 4;
constexpr int64_t kSpmvChunkCap = kSpmvChunkUnitsPerThread * 4 * 256 - 3;
constexpr int64_t kSpmmSlots = 2048;                     // LDS (col, val) slots per SpMM block
constexpr int64_t kSpmmNnzCap = kSpmmSlots - 3;
constexpr int64_t kIndexStatsBlocks = 1024;             // first-pass workgroups of fsp_index_stats
constexpr int64_t kXcsItemCap = 2048;                    // entries of one XCS item
constexpr int64_t kXcsRowsCap = 8192;                    // rows of one XCS tile
constexpr int64_t kXcsWinSlotsCap = 4096;                // partial slots of one combine window
constexpr int64_t kXcsWinRowsCap = 2048;                 // rows of one combine window
constexpr int64_t kXcsItemRunsCap = 64;                  // stored runs (windows) of one XCS item
constexpr int64_t kXcsSortedItemCap = 4096;              // entries of one sorted-gather XCS item
constexpr int64_t kXcsSortedColBits = 19;                // column bits of a sorted-gather entry
constexpr int64_t kPanelBytes = 131072;                  // x panel copied to LDS (panel SpMV)
constexpr int64_t kPanelChunk = 512;                     // entries per wave chunk (panel SpMV)
constexpr int64_t kPanelChunkRunsCap = 64;               // runs (rows) of one chunk, at most
constexpr int64_t kStageWinCap = 8192;                   // entries of one staged-x window
constexpr int64_t kStageWinRows = 4096;                  // rows of one staged-x window
constexpr int64_t kStageChunkEntries = 512;             // staged entries per wave chunk

// Zero y[0, n) on stream st (used before row-mapped launches that leave rows untouched).
int fill_zero_f32(float* y, int64_t n, hipStream_t st);
int fill_zero_f64(double* y, int64_t n, hipStream_t st);
template <typename T> int fill_zero(T* y, int64_t n, hipStream_t st);
template <> inline int fill_zero<float>(float* y, int64_t n, hipStream_t st) {
  return fill_zero_f32(y, n, st);
}
template <> inline int fill_zero<double>(double* y, int64_t n, hipStream_t st) {
  return fill_zero_f64(y, n, st);
}

int set_error(int code, const std::string& msg);
int check_hip(hipError_t e, const char* what);

}  // namespace fsp
