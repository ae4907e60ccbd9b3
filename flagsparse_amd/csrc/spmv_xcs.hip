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
//           entries, ordered by row (original order inside a row); an item's Q = ceil(len/4)
//           quads of entries start on a multiple of 4 and are stored thread-major: with
//           qp = ceil(Q/256) quads per thread and nt = ceil(Q/qp) threads, logical quad
//           qp*t + u is at memory quad t + nt*u (coalesced loads, contiguous rows per thread)
//   pidx    (local row << col_bits) | (column - the panel's first column)
//   slots   one item descriptor per workgroup in launch order, 12 int32:
//           {entry start, count, rank k in tile, first stored run, r0, rows R, panel first
//            column, stored runs, 0, 0, tile (-1: empty slot), 0}
//   rows    every item computes the sum of each row run it holds (in row order) and stores
//           them by combine window: the sums of its rows in window w go to a run of slots of
//           their own inside w's range (item_runs: {first slot, first sum, sums, stored
//           length}, a run starting on a line and padded with zeros to whole lines); a second
//           launch
//           (xcs_window_combine_kernel) gives every row the sum of its slots in item order - a
//           fixed order, so the result does not depend on timing - and writes y in row order.
//           Items never write y themselves: a y line would then be written piecewise by items
//           on several XCDs, and those partial-line writes cost more than the extra slots
//           (measured on MI355X: cfg3's short rows 323 -> 243 us without them).
//           No workgroup waits for or signals another: a device-scope fence would write back
//           and invalidate the XCD's L2, which holds the x panel this layout exists to keep.
//
// Long rows of power-law matrices also have a second layout, "panels" (spmv_panel_kernel):
// x is cut into panels of 2^col_bits columns, at most 128 KiB each, and a row with many entries
// per panel gets them gathered from an LDS copy of the panel instead of from L2:
//   entries  the long rows' entries ordered by (panel, row), each panel's run padded with
//            zero entries of its last row to a multiple of kPanelChunk.  An entry is its value
//            and 16 bits, pcol = column in the panel | 0x8000 when it starts a run (its row
//            differs from the previous entry's, or it opens a chunk): the kernel needs row
//            changes only, never row numbers, since a chunk's runs take consecutive slots.
//            Values: inside a chunk, logical quad 2L + h (lane L's h-th quad) is stored at
//            quad h * 64 + L, so each 16-byte load of a wave reads one contiguous kilobyte;
//            pcol in logical order (lane L's 8 entries are the 16 bytes at 16 L)
//   chunks   kPanelChunk consecutive entries, one wave's unit of work; chunk_info[c] = {the
//            first partial slot of chunk c, which has one slot per run (row) it holds; the
//            number of its entries in use - a chunk closed early, and each panel's last one,
//            end in padding}
//   jobs     workgroup j copies panel job_panel[j] into LDS and its waves take the chunks
//            [jobs[j], jobs[j+1]) in turn; no barrier after the copy
// Each long row's slots are then added by panel_combine_kernel (one wave per row, fixed order).
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
constexpr int kItemRuns = (int)kXcsItemRunsCap;
static_assert(kItemRuns <= kBlock, "an item's runs are loaded one per thread");

// DPP move with bound_ctrl: the value of the lane that CTRL selects, 0 where that lane lies
// outside the control's range or ROW_MASK leaves the lane's row out.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_bc(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xF, true);
}
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ double dpp_bc(double v) {
  const int64_t b = __double_as_longlong(v);
  const int lo = dpp_bc<CTRL, ROW_MASK>((int)(b & 0xffffffff));
  const int hi = dpp_bc<CTRL, ROW_MASK>((int)(b >> 32));
  return __longlong_as_double(((int64_t)hi << 32) | (uint32_t)lo);
}
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_bc(float v) {
  return __int_as_float(dpp_bc<CTRL, ROW_MASK>(__float_as_int(v)));
}

// Lane l's value of v (l wave-uniform).
__device__ __forceinline__ float lane_value(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ double lane_value(double v, int l) {
  const int64_t b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_readlane((int)(b & 0xffffffff), l);
  const int hi = __builtin_amdgcn_readlane((int)(b >> 32), l);
  return __longlong_as_double(((int64_t)hi << 32) | (uint32_t)lo);
}

// One step of the wave scans of the XCS and panel kernels: (h, v) a segmented inclusive scan
// (h: a run starts in this lane's part; combine(a, b) = (a.h | b.h, b.h ? b.v : a.v + b.v)), c
// a plain one, with the source lane that the DPP control CTRL selects.  Lanes without a source
// read 0, the identity of all three parts (no start, +0.0, 0), and the sum is selected rather
// than branched to (a branch per step cost the panel kernel a third of its scan instructions).
template <int CTRL, int ROW_MASK, typename A>
__device__ __forceinline__ void seg_scan_step(int& h, A& v, int& c) {
  const int ho = dpp_bc<CTRL, ROW_MASK>(h);
  const A vo = dpp_bc<CTRL, ROW_MASK>(v);
  const int co = dpp_bc<CTRL, ROW_MASK>(c);
  const A sum = vo + v;
  v = h ? v : sum;
  h |= ho;
  c += co;
}

// Inclusive scans over the wave (seg_scan_step): shifts by 1, 2, 4 and 8 inside each 16-lane
// row, then each row's last lane to the rows after it - a fixed order of additions.
template <typename A>
__device__ __forceinline__ void wave_seg_scan(int& h, A& v, int& c) {
  seg_scan_step<kDppRowShr1, 0xF>(h, v, c);
  seg_scan_step<kDppRowShr1 + 1, 0xF>(h, v, c);
  seg_scan_step<kDppRowShr1 + 3, 0xF>(h, v, c);
  seg_scan_step<kDppRowShr1 + 7, 0xF>(h, v, c);
  seg_scan_step<kDppRowBcast15, 0xA>(h, v, c);
  seg_scan_step<kDppRowBcast31, 0xC>(h, v, c);
}

// Occupancy cap.  The kernel needs about 17 KiB of LDS (its partial-sum buffer, 16 KiB, and
// the run table) and 50 VGPRs, so up to 8 workgroups would share a CU; more waves only queue
// more x requests at the XCD's L2.  Measured on MI355X, cfg3's XCS kernel with 2 / 3 / 4 / 5 /
// 6 / 7 / 8 workgroups per CU: 157.9 / 137.6 / 126.8 / 128.3 / 132.0 / 134.5 / 134.8 us (the
// whole call 264.0 us at 4, 265.2 at 5).  The launch adds unused dynamic LDS up to this many
// bytes per workgroup (with the static arrays, 39 KiB), so that four fit the CU's 160 KiB.
constexpr unsigned kXcsLdsPerWorkgroup = 38u * 1024u;
template <typename A>
constexpr unsigned xcs_lds_reserve() {
  return kXcsLdsPerWorkgroup - (unsigned)(kItemCap * sizeof(A));
}

// Segmented sums over an item: thread t owns a contiguous run of the item's entries, which
// holds whole runs (rows) and pieces of runs that continue from or into its neighbours.  A
// workgroup-wide segmented scan over (has a run start, sum of the last run piece) - combine(a,
// b) = (a.h | b.h, b.h ? b.v : a.v + b.v), evaluated in a fixed pattern - gives each thread
// the sum of the run piece that ends just before its chunk.  No LDS round trip of products.
template <typename T, typename A, bool NT>
__global__ __launch_bounds__(kBlock) void spmv_xcs_kernel(
    const T* __restrict__ vals, const uint32_t* __restrict__ pidx, int col_bits,
    const T* __restrict__ x, const i32x4* __restrict__ items, int n_slots,
    const i32x4* __restrict__ item_runs, A* __restrict__ partials) {
  constexpr int kPer = kItemCap / kBlock;  // entries per thread at most
  constexpr int kQuads = kPer / 4;
  static_assert(kQuads * 4 == kPer, "whole quads of entries per thread");
  __shared__ int s_first_row[kWavesPerBlock];
  __shared__ int s_last_row[kWavesPerBlock];
  __shared__ int s_wh[kWavesPerBlock];
  __shared__ int s_wc[kWavesPerBlock];
  __shared__ A s_wv[kWavesPerBlock];
  // The item's run sums, written out together at the end in whole lines (stored one by one
  // from the threads, partial lines could leave L2 before they filled).
  __shared__ A s_part[kItemCap];
  // Where the sums go: one stored run per combine window the item's rows reach.
  __shared__ i32x4 s_runs[kItemRuns];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1), wid = tid / kWave;
  const int slot = xcd_logical_block(blockIdx.x, n_slots);
  const i32x4 d0 = items[3 * slot];
  const i32x4 d1 = items[3 * slot + 1];
  const i32x4 d2 = items[3 * slot + 2];
  if (d2.z < 0) return;  // empty slot
  const int e0 = d0.x, len = d0.y, run0 = d0.w;
  const int R = d1.y, cbase = d1.z, n_ir = d1.w;
  if (R <= 0 || R > kRowsCap || len < 0 || len > kItemCap || n_ir < 0 || n_ir > kItemRuns)
    return;  // not a planner item
  // Issued first; stored to LDS once the entry loads are in flight.
  i32x4 my_run = {0, 0, 0, 0};
  if (tid < n_ir) my_run = item_runs[run0 + tid];

  // Entries [i0, i0 + nm) of this thread (thread-major storage, see the file comment).
  const int q_tot = (len + 3) >> 2;
  const int qp = q_tot > 0 ? (q_tot + kBlock - 1) / kBlock : 1;
  const int nt = (q_tot + qp - 1) / qp;
  const int i0 = 4 * qp * tid;
  const int nm = len - i0 < 0 ? 0 : (len - i0 > 4 * qp ? 4 * qp : len - i0);
  T v[kPer];
  uint32_t c[kPer];
#pragma unroll
  for (int h = 0; h < kQuads; ++h) {
    if (h < qp && 4 * h < nm) {
      const int m = 4 * (tid + nt * h);  // memory position of logical quad qp*tid + h
      if constexpr (sizeof(T) == 4) {
        const f32x4 vv = ld_stream<NT>(reinterpret_cast<const f32x4*>(vals + e0 + m));
        v[4 * h] = vv.x; v[4 * h + 1] = vv.y; v[4 * h + 2] = vv.z; v[4 * h + 3] = vv.w;
      } else {
        const f64x2 a = ld_stream<NT>(reinterpret_cast<const f64x2*>(vals + e0 + m));
        const f64x2 b = ld_stream<NT>(reinterpret_cast<const f64x2*>(vals + e0 + m + 2));
        v[4 * h] = a.x; v[4 * h + 1] = a.y; v[4 * h + 2] = b.x; v[4 * h + 3] = b.y;
      }
      const i32x4 cc = ld_stream<NT>(reinterpret_cast<const i32x4*>(pidx + e0 + m));
      c[4 * h] = (uint32_t)cc.x; c[4 * h + 1] = (uint32_t)cc.y;
      c[4 * h + 2] = (uint32_t)cc.z; c[4 * h + 3] = (uint32_t)cc.w;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) { v[4 * h + j] = T(0); c[4 * h + j] = 0u; }
    }
  }
  const uint32_t cmask = (1u << col_bits) - 1u;
  // Every gather is issued, also for the positions past this thread's entries (which read the
  // panel's first column, present in any item), and the value is dropped afterwards: a load
  // under a per-lane condition is an exec-masked region of its own, and with the fp64
  // conversion inside it the compiler waits for each gather before issuing the next.
  T xv[kPer];
#pragma unroll
  for (int q = 0; q < kPer; ++q) xv[q] = x[cbase + (q < nm ? (int)(c[q] & cmask) : 0)];
  A prod[kPer];
  int row[kPer];
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    prod[q] = q < nm ? A(v[q]) * A(xv[q]) : A(0);
    row[q] = (int)(c[q] >> col_bits);
  }

  // Rows of the entries just before and just after this thread's chunk (-1: none).
  const int my_first = nm > 0 ? row[0] : -1;
  int my_last = row[0];
#pragma unroll
  for (int q = 1; q < kPer; ++q)
    if (q < nm) my_last = row[q];
  if (lane == 0) s_first_row[wid] = my_first;
  if (lane == kWave - 1) s_last_row[wid] = my_last;
  if (tid < n_ir) s_runs[tid] = my_run;
  __syncthreads();
  int prev_row = __shfl_up(my_last, 1, kWave);
  if (lane == 0) prev_row = wid > 0 ? s_last_row[wid - 1] : -1;
  if (tid == 0) prev_row = -1;
  int next_row = __shfl_down(my_first, 1, kWave);
  if (lane == kWave - 1) next_row = wid + 1 < kWavesPerBlock ? s_first_row[wid + 1] : -1;
  if (i0 + nm >= len) next_row = -1;  // my chunk ends the item

  // Every run (row) whose last entry lies in this chunk is emitted by this thread: at an
  // internal row change, or at the chunk's last entry when the next entry belongs to another
  // row.  The chunk's first run, when it continues from before (cont), gets the carry - the
  // sum of its entries before this chunk - from the scan below.
  //
  // Pass 1 (before the scan): whether a run starts here, the sum of the last run piece (the
  // scan's input) and how many runs end here (each takes one partial slot).  Pass 2 (after
  // it) sums the runs again and emits them.  Nothing but prod and row stays
  // live across the scan, which keeps the register count, and with it the number of waves in
  // flight per SIMD, up.
  const bool cont = nm > 0 && my_first == prev_row;
  const bool last_ends = nm > 0 && next_row != my_last;
  int has_head = (nm > 0 && !cont) ? 1 : 0;
  int n_end = last_ends ? 1 : 0;
  A piece = A(0);
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    if (q < nm) {
      if (q > 0 && row[q] != row[q - 1]) {
        has_head = 1;
        ++n_end;
        piece = A(0);
      }
      piece += prod[q];
    }
  }

  // Workgroup scans, one barrier: segmented scan of (has_head, last piece) gives the carry,
  // and a plain scan of n_end gives this thread's first slot.
  int h_in = has_head;
  A v_in = piece;
  int c_in = n_end;
  wave_seg_scan(h_in, v_in, c_in);
  if (lane == kWave - 1) {
    s_wh[wid] = h_in;
    s_wv[wid] = v_in;
    s_wc[wid] = c_in;
  }
  const int h_ex = dpp_mov<kDppWaveShr1>(0, h_in);  // lane 0: (0, 0, 0)
  const A v_ex = dpp_mov<kDppWaveShr1>(A(0), v_in);
  const int c_ex = dpp_mov<kDppWaveShr1>(0, c_in);
  __syncthreads();
  A pv = A(0);
  int pc = 0;
  for (int j = 0; j < kWavesPerBlock; ++j) {
    if (j < wid) {  // waves before this one, in order
      const A wv = s_wv[j];
      if (!s_wh[j]) pv = pv + wv; else pv = wv;
      pc += s_wc[j];
    }
  }
  const A carry = h_ex ? v_ex : pv + v_ex;

  // Pass 2, in row order: each run to the item's next slot.
  A* out = s_part + pc + c_ex;
  bool first = true;
  A run = A(0);
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    if (q < nm) {
      if (q > 0 && row[q] != row[q - 1]) {
        *out++ = (first && cont) ? carry + run : run;
        first = false;
        run = A(0);
      }
      run += prod[q];
    }
  }
  if (last_ends) *out = (first && cont) ? carry + run : run;
  __syncthreads();
  // Out in whole lines: run j holds the item's sums [r.y, r.y + r.z) at stored slots from r.x,
  // padded with zeros to r.w slots (a run starts on a line, so no line has two writers).
  for (int j = 0; j < n_ir; ++j) {
    const i32x4 r = s_runs[j];
    for (int l = tid; l < r.w; l += kBlock) partials[r.x + l] = l < r.z ? s_part[r.y + l] : A(0);
  }
}

// Sorted-gather items (item format 1).  The rate of random 4-byte gathers from L2 depends on
// how close together the 64 lanes of one gather instruction reach: measured on MI355X with
// groups of 2048 gathers in a 2 MiB range, 137 us in random order and 131 us sorted and laid
// out lane-major; with the lanes about one line apart (2048 gathers in 256 KiB) 98 us.  An
// item here holds up to 4096 entries (a workgroup of 512 threads), and its gather entries are
// stored in column order, lane-major: gather k of thread t is entry (t/64)*512 + 64k + t%64 of
// the column order.  Each gather entry carries the entry's position in row order and whether
// it starts a row run there, so the gathered x values go to LDS in row order, and after one
// barrier every thread reads back its 8 consecutive row-order positions - the layout of the
// thread-major kernel above, whose segmented scan and emission follow unchanged (run starts
// from the flags instead of row comparisons).
//   vals   row order: position 8t + e of thread t at quad (e/4) * P/8 + t, element e % 4
//   gidx   column order, the same quads: (row-order position << 20) | run start << 19 | column
//          in the panel (19 bits); P = the item's length rounded up to 512
constexpr int kSortedBlock = 512;
constexpr int kSortedWaves = kSortedBlock / kWave;
constexpr int kSortedCap = (int)kXcsSortedItemCap;
constexpr int kSortedPer = kSortedCap / kSortedBlock;
static_assert(kSortedPer == 8, "eight entries per thread");
constexpr int kSortedWaveEntries = kWave * kSortedPer;  // 512: a wave's share of an item
constexpr unsigned kSortedColBits = (unsigned)kXcsSortedColBits;
constexpr unsigned kSortedColMask = (1u << kSortedColBits) - 1u;
constexpr unsigned kSortedPosShift = kSortedColBits + 1u;
static_assert(kSortedPosShift + 12 <= 32, "a position below 4096 fits the word");

// LDS of the sorted-gather kernel: the item's x values and run-start flags in row order, then
// (the same bytes, after the scan's barrier) its run sums.
template <typename T, typename A>
constexpr int sorted_lds_bytes() {
  constexpr int stage = kSortedCap * ((int)sizeof(T) + 1);
  constexpr int part = kSortedCap * (int)sizeof(A);
  return stage > part ? stage : part;
}
// Workgroups per CU of the sorted-gather kernel, set by the LDS each one claims.
constexpr unsigned kXcsSortedLdsPerWorkgroup = 40u * 1024u;

template <typename T, typename A>
__global__ __launch_bounds__(kSortedBlock) void spmv_xcs_sorted_kernel(
    const T* __restrict__ vals, const uint32_t* __restrict__ gidx, const T* __restrict__ x,
    const i32x4* __restrict__ items, int n_slots, const i32x4* __restrict__ item_runs,
    A* __restrict__ partials) {
  constexpr int kPer = kSortedPer;
  __shared__ __align__(16) unsigned char s_buf[sorted_lds_bytes<T, A>()];
  T* const s_x = reinterpret_cast<T*>(s_buf);
  unsigned char* const s_fl = s_buf + kSortedCap * sizeof(T);
  A* const s_part = reinterpret_cast<A*>(s_buf);
  __shared__ int s_wh[kSortedWaves];
  __shared__ int s_wc[kSortedWaves];
  __shared__ A s_wv[kSortedWaves];
  __shared__ i32x4 s_runs[kItemRuns];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1), wid = tid / kWave;
  const int slot = xcd_logical_block(blockIdx.x, n_slots);
  const i32x4 d0 = items[3 * slot];
  const i32x4 d1 = items[3 * slot + 1];
  const i32x4 d2 = items[3 * slot + 2];
  if (d2.z < 0) return;  // empty slot
  const int e0 = d0.x, len = d0.y, run0 = d0.w;
  const int cbase = d1.z, n_ir = d1.w;
  if (len <= 0 || len > kSortedCap || n_ir < 0 || n_ir > kItemRuns) return;  // no planner item
  i32x4 my_run = {0, 0, 0, 0};
  if (tid < n_ir) my_run = item_runs[run0 + tid];

  // Threads [0, P/8) hold entries; the others re-read thread 0's quads and drop them.
  const int n_thr = (len + kSortedWaveEntries - 1) / kSortedWaveEntries * kWave;
  const int tt = tid < n_thr ? tid : 0;
  T v[kPer];
  uint32_t g[kPer];
#pragma unroll
  for (int u = 0; u < kPer / 4; ++u) {
    const int m = e0 + 4 * (u * n_thr + tt);
    if constexpr (sizeof(T) == 4) {
      const f32x4 vv = ld_stream<true>(reinterpret_cast<const f32x4*>(vals + m));
      v[4 * u] = vv.x; v[4 * u + 1] = vv.y; v[4 * u + 2] = vv.z; v[4 * u + 3] = vv.w;
    } else {
      const f64x2 a = ld_stream<true>(reinterpret_cast<const f64x2*>(vals + m));
      const f64x2 b = ld_stream<true>(reinterpret_cast<const f64x2*>(vals + m + 2));
      v[4 * u] = a.x; v[4 * u + 1] = a.y; v[4 * u + 2] = b.x; v[4 * u + 3] = b.y;
    }
    const i32x4 gg = ld_stream<true>(reinterpret_cast<const i32x4*>(gidx + m));
    g[4 * u] = (uint32_t)gg.x; g[4 * u + 1] = (uint32_t)gg.y;
    g[4 * u + 2] = (uint32_t)gg.z; g[4 * u + 3] = (uint32_t)gg.w;
  }
  // Gathers in column order, all issued (positions past the item read the panel's first
  // value), then each value stored at its row-order position.
  T xv[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const bool ok = tid < n_thr && wid * kSortedWaveEntries + k * kWave + lane < len;
    xv[k] = x[cbase + (ok ? (int)(g[k] & kSortedColMask) : 0)];
  }
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    if (tid < n_thr && wid * kSortedWaveEntries + k * kWave + lane < len) {
      const int p = (int)(g[k] >> kSortedPosShift);
      s_x[p] = xv[k];
      s_fl[p] = (unsigned char)((g[k] >> kSortedColBits) & 1u);
    }
  }
  if (tid < n_ir) s_runs[tid] = my_run;
  __syncthreads();

  // Row order: this thread's positions [i0, i0 + nm).
  const int i0 = kPer * tid;
  const int nm = len - i0 < 0 ? 0 : (len - i0 > kPer ? kPer : len - i0);
  A prod[kPer];
  bool st[kPer];
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const bool in = q < nm;
    prod[q] = in ? A(v[q]) * A(s_x[in ? i0 + q : 0]) : A(0);
    st[q] = in && s_fl[i0 + q] != 0;
  }
  const bool next_starts = i0 + kPer < len ? s_fl[i0 + kPer] != 0 : true;

  // As spmv_xcs_kernel: pass 1 (run starts, the last run piece, runs ending here), the
  // workgroup scans, pass 2 (each run to the item's next slot), the stored runs written out.
  const bool cont = nm > 0 && !st[0];
  const bool last_ends = nm > 0 && next_starts;
  int has_head = (nm > 0 && !cont) ? 1 : 0;
  int n_end = last_ends ? 1 : 0;
  A piece = A(0);
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    if (q < nm) {
      if (q > 0 && st[q]) {
        has_head = 1;
        ++n_end;
        piece = A(0);
      }
      piece += prod[q];
    }
  }
  int h_in = has_head;
  A v_in = piece;
  int c_in = n_end;
  wave_seg_scan(h_in, v_in, c_in);
  if (lane == kWave - 1) {
    s_wh[wid] = h_in;
    s_wv[wid] = v_in;
    s_wc[wid] = c_in;
  }
  const int h_ex = dpp_mov<kDppWaveShr1>(0, h_in);  // lane 0: (0, 0, 0)
  const A v_ex = dpp_mov<kDppWaveShr1>(A(0), v_in);
  const int c_ex = dpp_mov<kDppWaveShr1>(0, c_in);
  __syncthreads();  // also: every row-order read of s_x / s_fl is done before s_part reuses them
  A pv = A(0);
  int pc = 0;
  for (int j = 0; j < kSortedWaves; ++j) {
    if (j < wid) {
      const A wv = s_wv[j];
      if (!s_wh[j]) pv = pv + wv; else pv = wv;
      pc += s_wc[j];
    }
  }
  const A carry = h_ex ? v_ex : pv + v_ex;
  A* out = s_part + pc + c_ex;
  bool first = true;
  A run = A(0);
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    if (q < nm) {
      if (q > 0 && st[q]) {
        *out++ = (first && cont) ? carry + run : run;
        first = false;
        run = A(0);
      }
      run += prod[q];
    }
  }
  if (last_ends) *out = (first && cont) ? carry + run : run;
  __syncthreads();
  for (int j = 0; j < n_ir; ++j) {
    const i32x4 r = s_runs[j];
    for (int l = tid; l < r.w; l += kSortedBlock)
      partials[r.x + l] = l < r.z ? s_part[r.y + l] : A(0);
  }
}

// Second pass: row r gets y = the sum of its partial sums in item order (a fixed order, so the
// result does not depend on timing), 0 without any.  Rows are grouped into windows of
// consecutive rows whose sums fit LDS (<= kXcsWinSlotsCap sums, <= kXcsWinRowsCap rows), and
// the partials buffer holds the windows one after the other (inside a window one run per item,
// each starting on a cache line, see spmv_xcs_kernel).  A workgroup per window:
//   1. streams the window's stored range with every load of a thread issued before the first
//      is used, and scatters each sum to LDS position dest[slot] - the window's sums in
//      (row, item) order; padding slots (dest -1) are dropped;
//   2. takes each row's number of sums (row_count, one byte per row; a row with more than 255
//      sums is a window of its own) and their exclusive scan over the window - the row's first
//      LDS position; thread t holds rows t, t + NB, ..., scanned block by block (a wave scan
//      each), the wave totals of every block exchanged at the barrier of step 1;
//   3. gives row r the sum of its positions, in order, and writes y.  Rows of at most kInline
//      sums are summed by the thread that holds them; rows with more are listed in LDS and
//      shared out among all the threads (measured on MI355X, cfg3: 42.5 -> 40.8 us; each wave
//      had run its row loops as long as its longest row).
// A window of one row with more sums than a window takes ({row, -1, ...}) is summed by the
// whole workgroup - thread t takes its slots t, t + NB, ... in order, then the fixed workgroup
// tree.
// A separate launch: the kernel boundary makes the first pass's partials visible on every
// XCD, so neither pass needs a device-scope fence.
// Loads per thread and round of the stream step: a whole 4096-slot window in one round
// (measured on MI355X with 256 threads: cfg3 49.1 us at 16 per thread, 50.8 at 8, 53.0 at 4;
// cfg4 14.7 / 14.4 / 13.8).
// Threads per combine workgroup.  A window's LDS (its 4096 sums, 32 KiB, and the row list)
// allows 4 workgroups per CU: with 512 threads that is every wave slot of the CU.  Measured on
// MI355X, cfg3: 41.1 us with 256 threads, 36.7 us with 512, 38.1 us with 1024 (then with 3
// workgroups per CU, the row list taking more LDS than it can need).
constexpr int kCombBlock = 512;
// Sums of a row added by the thread that holds it (rows with more go to the shared list).
// Measured on MI355X, whole call: cfg3 268.1 / 268.3 / 269.1 us with 2 / 3 / 4; the combine of
// cfg4 (rows of about four sums) 18.2 / 18.3 / 17.4 us.
constexpr int kInline = 2;

// Inclusive scan of c over the wave (DPP, as the count part of wave_seg_scan).
__device__ __forceinline__ int wave_incl_scan(int c) {
  c += dpp_mov<kDppRowShr1, 0xF>(0, c);
  c += dpp_mov<kDppRowShr1 + 1, 0xF>(0, c);
  c += dpp_mov<kDppRowShr1 + 3, 0xF>(0, c);
  c += dpp_mov<kDppRowShr1 + 7, 0xF>(0, c);
  c += dpp_mov<kDppRowBcast15, 0xA>(0, c);
  c += dpp_mov<kDppRowBcast31, 0xC>(0, c);
  return c;
}

// A row count that marks a row the window leaves alone (no sums here, and y written by the
// panel rows of the same launch: the long rows of the hybrid).
constexpr int kRowSkip = 255;

// Window wi of the combine (the body of xcs_window_combine_kernel, NB threads).
template <typename T, typename A, int NB>
__device__ __forceinline__ void combine_window(
    int wi, const i32x4* __restrict__ windows, const int16_t* __restrict__ dest,
    const uint8_t* __restrict__ row_count, const A* __restrict__ partials, T* __restrict__ y,
    const int* __restrict__ row_map, int win_cap) {
  constexpr int kWaves = NB / kWave;
  constexpr int kPer = (int)kXcsWinSlotsCap / NB;  // loads per thread: a whole window at once
  constexpr int kRound = kPer * NB;
  constexpr int kRowsPer = (int)kXcsWinRowsCap / NB;  // rows per thread
  // win_cap sums of LDS (the layout's window size): smaller windows leave room for more
  // workgroups per CU, whose stream and sum phases then overlap.
  extern __shared__ __align__(16) unsigned char s_dyn[];
  A* const s_val = reinterpret_cast<A*>(s_dyn);
  __shared__ A s_red[kWaves];
  __shared__ int s_wtot[kRowsPer][kWaves];
  // Rows with more than kInline sums, listed for a second pass: (row in the window << 20) |
  // (first position << 8) | sums.  A window holds at most kXcsWinSlotsCap sums, so at most
  // kXcsWinSlotsCap / (kInline + 1) such rows; sized so, the list leaves the LDS of four
  // workgroups per CU (a list of kXcsWinRowsCap entries put 40.2 KiB in each and allowed three:
  // measured on MI355X, cfg3's combine 41.6 -> 40.8 us, the whole call 267.5 -> 265.4 us).
  constexpr int kLongCap = (int)kXcsWinSlotsCap / (kInline + 1);
  __shared__ int s_nlong;
  __shared__ int s_long[kLongCap];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1), wid = tid / kWave;
  if (tid == 0) s_nlong = 0;  // read after the barrier below
  const i32x4 w0 = windows[2 * wi];
  const int total = windows[2 * wi + 1].x;
  const int row0 = w0.x, nr = w0.y, base = w0.z, len = w0.w;

  if (nr < 0) {  // one row with more sums than a window takes: a workgroup sum in fixed order
    A acc = A(0);
    for (int l = tid; l < len; l += NB) acc += partials[base + l];
    acc = wave_sum(acc);
    if (lane == 0) s_red[wid] = acc;
    __syncthreads();
    acc = s_red[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) acc += s_red[w];
    if (tid == 0) y[row_map ? row_map[row0] : row0] = T(acc);
    return;
  }
  if (nr > (int)kXcsWinRowsCap || total > win_cap) return;  // not a layout window (uniform)

  // The sums of this thread's rows tid + m * NB, requested first (they do not depend on LDS).
  // With rows strided so, every store of y covers consecutive rows (measured on MI355X, cfg3:
  // 35.4 us, against 37.3 us with 4 consecutive rows per thread and one scan).
  auto row_of = [&](int m) { return tid + m * NB; };
  int cnt[kRowsPer];
  bool skip[kRowsPer];
#pragma unroll
  for (int m = 0; m < kRowsPer; ++m) {
    const int c = row_of(m) < nr ? (int)row_count[row0 + row_of(m)] : 0;
    skip[m] = c == kRowSkip;
    cnt[m] = skip[m] ? 0 : c;
  }

  // Every load of a thread is issued before the first is used.  (Measured on MI355X, cfg3:
  // reading 4 slots per load - 16-byte sums, 8-byte dest words - was slower, 52.1 / 53.0 us
  // with 2 / 4 groups per thread against 50.6 us at 8 single loads: more registers, fewer
  // workgroups per CU.)
  for (int c0 = 0; c0 < len; c0 += kRound) {  // uniform
    A v[kPer];
    int d[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int j = c0 + tid + k * NB;
      const int jj = j < len ? j : 0;  // past the end: reload the first slot, dropped below
      v[k] = partials[base + jj];
      d[k] = (int)dest[base + jj];
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k)
      if (c0 + tid + k * NB < len && (unsigned)d[k] < (unsigned)win_cap) s_val[d[k]] = v[k];
  }
  // First positions: the exclusive scan of the row counts over the window, in row order.
  int rs[kRowsPer];
  int incl[kRowsPer];
#pragma unroll
  for (int m = 0; m < kRowsPer; ++m) {
    incl[m] = wave_incl_scan(cnt[m]);
    if (lane == kWave - 1) s_wtot[m][wid] = incl[m];
  }
  __syncthreads();
  int before = 0;  // rows of the blocks before block m, then of the waves before this one
#pragma unroll
  for (int m = 0; m < kRowsPer; ++m) {
    int mine = 0, blk = 0;
    for (int j = 0; j < kWaves; ++j) {
      const int t = s_wtot[m][j];
      blk += t;
      if (j < wid) mine += t;
    }
    rs[m] = before + mine + incl[m] - cnt[m];
    before += blk;
  }

  // The first kInline sums of all the thread's rows are requested together (most rows have
  // fewer); rows with more are listed and summed afterwards by all threads, in order.
  A acc[kRowsPer];
#pragma unroll
  for (int m = 0; m < kRowsPer; ++m) {
    A t[kInline];
#pragma unroll
    for (int u = 0; u < kInline; ++u) t[u] = cnt[m] > u ? s_val[rs[m] + u] : A(0);
    acc[m] = A(0);
#pragma unroll
    for (int u = 0; u < kInline; ++u)
      if (cnt[m] > u) acc[m] += t[u];
  }
#pragma unroll
  for (int m = 0; m < kRowsPer; ++m) {
    const int i = row_of(m);
    if (i < nr && !skip[m]) {
      if (cnt[m] > kInline) {
        const int at = atomicAdd(&s_nlong, 1);
        if (at < kLongCap) s_long[at] = (i << 20) | (rs[m] << 8) | cnt[m];  // always, in a layout
      } else {
        const int row = row0 + i;
        y[row_map ? row_map[row] : row] = T(acc[m]);
      }
    }
  }
  __syncthreads();
  const int n_long = s_nlong < kLongCap ? s_nlong : kLongCap;
  for (int j = tid; j < n_long; j += NB) {
    const int e = s_long[j];
    const int i = e >> 20, a = (e >> 8) & 0xfff, b = a + (e & 0xff);
    A r = A(0);  // the same order as above: 0 + s[a] + s[a + 1] + ...
    for (int k = a; k < b; k += 4) {
      A t[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) t[u] = k + u < b ? s_val[k + u] : A(0);
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (k + u < b) r += t[u];
    }
    const int row = row0 + i;
    y[row_map ? row_map[row] : row] = T(r);
  }
}

template <typename T, typename A, int NB>
__global__ __launch_bounds__(NB) void xcs_window_combine_kernel(
    const i32x4* __restrict__ windows, const int16_t* __restrict__ dest,
    const uint8_t* __restrict__ row_count, const A* __restrict__ partials, T* __restrict__ y,
    const int* __restrict__ row_map, int win_cap) {
  combine_window<T, A, NB>((int)blockIdx.x, windows, dest, row_count, partials, y, row_map,
                           win_cap);
}

// Panel layout (see the file comment): one workgroup per job, waves independent after the
// panel copy.  A wave's chunk: lane L holds entries [8L, 8L + 8), their rows non-decreasing;
// the runs that end in a lane are emitted by it, the first one with the carry from the lanes
// before (a segmented wave scan), into consecutive slots from chunk_info[c].x in entry order;
// the chunk's entries past its first chunk_info[c].y are padding and add exactly 0 (a product
// 0 * x would be NaN where x holds an infinity or a NaN).
// One workgroup of 16 waves per CU, holding a 128 KiB panel (measured on MI355X, cfg3 whole
// path: 0.315 ms with 64 KiB panels and 2 workgroups of 512 per CU, 0.290 ms with 128 KiB
// panels and 1024 threads, 0.300 ms with 128 KiB and 512 threads; the wider panels also
// carry more rows - those with 4 entries per panel - at the same partial count).
constexpr int kPanelBlock = 1024;
// Word 3 of a raw buffer resource on gfx9-family GPUs (gfx950): 32-bit data format, no swizzle.
constexpr int kBufferRsrcWord3 = 0x00020000;
// A byte offset no buffer here reaches: a store there is dropped by the range check.
constexpr unsigned kDropOffset = 0xFFFFFFF0u;

// Orders the LDS accesses of one wave across its lanes (wavefront-scope fences around the
// wave barrier): what a lane wrote before is visible to every lane after.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <typename A>
__device__ __forceinline__ void store_partial(__amdgpu_buffer_rsrc_t r, unsigned off, A v) {
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
  if constexpr (sizeof(A) == 8) {
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, off, 0, 0);
  } else {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, off, 0, 0);
  }
}
constexpr int kPanelPerLane = (int)kPanelChunk / kWave;
// Chunk buffers per wave of spmv_panel_kernel (registers: 8 values + 4 words of 16-bit entries
// + a slot each).  Measured on MI355X, cfg3: 3, 4, 5 and 6 buffers within 0.2 us of each other.
constexpr int kPanelBuffers = 3;
static_assert(kPanelPerLane == 8, "eight entries per lane");
static_assert(kPanelChunkRunsCap == kWave, "a chunk's runs are staged one per lane");

constexpr uint32_t kRunStart = 0x8000u;  // pcol: the entry starts a run

// The staged-x pass of a job (see the file comment): chunks [c0, c1) of kStageChunk staged
// entries, one wave per chunk, lane l taking entries 64k + l, so that each load of columns
// and each store of staged values covers 64 consecutive entries.  Entry e of chunk c (in use:
// below info.y) stores x[its column] at xs[e + sdelta[s]], s its segment: info.x for the
// chunk's first entry, one more at every later entry whose column has the segment bit (a
// layout rule: a chunk holds at most kWave segments).  The chunk's segment offsets are loaded
// a lane each and handed round with ds_bpermute.  A chunk's columns are requested two chunks
// ahead and its offsets one chunk ahead, so no wait of the loop is for a load issued in the
// same round; every store is issued (entries not in use store past the buffer's range, which
// the hardware drops), so the compiler keeps its count of the operations in flight.
constexpr int kStageChunk = (int)kStageChunkEntries;
// Chunk buffers of the staging loop (columns two chunks ahead).  Measured on MI355X: 3 / 4 / 6
// buffers, cfg3's panel pass 128.4 / 129.4 / 131.8 us, cfg4's 59.2 / 62.4 / 64.5 us.
constexpr int kStageBuffers = 3;
static_assert(kStageBuffers >= 3, "a chunk's offsets are loaded a round after its columns");
constexpr uint32_t kSegStart = 0x8000u;  // scol: the entry opens a segment

template <typename T>
__device__ __forceinline__ void store_staged(__amdgpu_buffer_rsrc_t r, unsigned off, T v) {
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
  if constexpr (sizeof(T) == 8) {
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, off, 0, 0);
  } else {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, off, 0, 0);
  }
}

template <typename T>
__device__ __forceinline__ void stage_panel_chunks(const T* sx, uint32_t cmask,
                                                   const uint16_t* __restrict__ scol,
                                                   const i32x2* __restrict__ sinfo,
                                                   const int* __restrict__ sdelta, int c0,
                                                   int c1, __amdgpu_buffer_rsrc_t xs) {
  constexpr int kPer = kStageChunk / kWave;
  constexpr int kStride = kPanelBlock / kWave;
  const int lane = (int)threadIdx.x & (kWave - 1);
  const int wid = (int)threadIdx.x / kWave;
  struct Chunk {
    uint32_t col[kPer];
    i32x2 info;
    int dl;
  };
  // past the job's last chunk: its last chunk again (loads only; never processed)
  auto load_cols = [&](int c, Chunk& k) {
    const int cc = c < c1 ? c : c1 - 1;
    const int e0 = cc * kStageChunk;
#pragma unroll
    for (int q = 0; q < kPer; ++q) k.col[q] = __builtin_nontemporal_load(scol + e0 + q * kWave + lane);
    k.info = sinfo[cc];
  };
  auto load_dl = [&](Chunk& k) { k.dl = sdelta[k.info.x + lane]; };
  auto process = [&](const Chunk& cur, int cc) {
    const unsigned base = (unsigned)(cc * kStageChunk + lane);
    int seen = 0;  // segment starts after the chunk's first entry, in the rounds before
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const uint32_t w = cur.col[q];
      const bool start = (w & kSegStart) != 0 && (q > 0 || lane > 0);
      const uint64_t bal = __builtin_amdgcn_ballot_w64(start);
      const int below = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                  __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
      const int off = seen + below + (start ? 1 : 0);
      seen += __builtin_popcountll(bal);
      const int delta = __builtin_amdgcn_ds_bpermute(off << 2, cur.dl);
      const T xv = sx[w & cmask];
      const unsigned e = base + (unsigned)(q * kWave);
      store_staged<T>(xs, q * kWave + lane < cur.info.y ? (e + (unsigned)delta) * (unsigned)sizeof(T)
                                                        : kDropOffset, xv);
    }
  };
  int c = c0 + wid;
  if (c >= c1) return;  // the whole wave
  // kStageBuffers chunk buffers: buffer b of a round holds the chunk b strides on; before one
  // is processed, the next one's offsets and the columns of the chunk kStageBuffers - 1
  // strides ahead are requested.
  constexpr int kSB = kStageBuffers;
  Chunk buf[kSB];
#pragma unroll
  for (int b = 0; b + 1 < kSB; ++b) load_cols(c + b * kStride, buf[b]);
  load_dl(buf[0]);
  for (; c < c1; c += kSB * kStride) {
#pragma unroll
    for (int b = 0; b < kSB; ++b) {
      const int cur = c + b * kStride;
      if (cur >= c1) break;
      load_dl(buf[(b + 1) % kSB]);
      load_cols(cur + (kSB - 1) * kStride, buf[(b + kSB - 1) % kSB]);
      process(buf[b], cur);
    }
  }
}

template <typename T, typename A>
__global__ __launch_bounds__(kPanelBlock) void spmv_panel_kernel(
    const T* __restrict__ vals, const uint16_t* __restrict__ pcol, int col_bits,
    const T* __restrict__ x, int64_t x_len, const int* __restrict__ jobs,
    const int* __restrict__ job_panel, const i32x2* __restrict__ chunk_info,
    A* __restrict__ partials, int64_t n_partials, const uint16_t* __restrict__ scol,
    const int* __restrict__ stage_jobs, const i32x2* __restrict__ sinfo,
    const int* __restrict__ sdelta, T* __restrict__ xs, int64_t n_xs) {
  extern __shared__ __align__(16) unsigned char s_dyn[];
  // Each wave's run sums of its current chunk in slot order (at most kWave: a layout rule),
  // then one slot per lane for the stores of lanes where no run ends.
  __shared__ A s_stage[kPanelBlock / kWave][2 * kWave];
  // The partial sums as a buffer resource of n_partials slots (< 2^32 bytes, checked by the
  // host): stores beyond it are dropped by the hardware.
  const __amdgpu_buffer_rsrc_t out_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      partials, 0, (int)(n_partials * (int64_t)sizeof(A)), kBufferRsrcWord3);
  T* const sx = reinterpret_cast<T*>(s_dyn);
  const int job = blockIdx.x;
  const int64_t pbase = (int64_t)job_panel[job] << col_bits;
  const int64_t rest = x_len - pbase;
  const int width = rest < ((int64_t)1 << col_bits) ? (int)rest : (1 << col_bits);
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  const uint32_t cmask = (1u << col_bits) - 1u;
  const int c_hi = jobs[job + 1];
  // The entries are streamed once with non-temporal loads, and the next chunks' loads are
  // issued before the current chunk is reduced, so a wave keeps chunks in flight.  The
  // chunk's first slot is loaded with its entries: loaded on its own after the next chunk's
  // loads, waiting for it (loads complete in order) also waited for the whole next chunk.
  auto load_chunk = [&](int chunk, T (&v)[kPanelPerLane], i32x4& c, i32x2& info) {
    const int64_t e0 = (int64_t)chunk * kPanelChunk;
#pragma unroll
    for (int h = 0; h < kPanelPerLane / 4; ++h) {
      const int64_t m = e0 + 4 * (h * kWave + lane);  // logical quad 2 * lane + h
      if constexpr (sizeof(T) == 4) {
        const f32x4 vv = ld_stream<true>(reinterpret_cast<const f32x4*>(vals + m));
        v[4 * h] = vv.x; v[4 * h + 1] = vv.y; v[4 * h + 2] = vv.z; v[4 * h + 3] = vv.w;
      } else {
        const f64x2 a = ld_stream<true>(reinterpret_cast<const f64x2*>(vals + m));
        const f64x2 b = ld_stream<true>(reinterpret_cast<const f64x2*>(vals + m + 2));
        v[4 * h] = a.x; v[4 * h + 1] = a.y; v[4 * h + 2] = b.x; v[4 * h + 3] = b.y;
      }
    }
    c = ld_stream<true>(reinterpret_cast<const i32x4*>(pcol + e0) + lane);
    info = chunk_info[chunk];
  };
  // One chunk's reduction: products from the LDS panel, then the runs (rows) that end in each
  // lane are emitted, the first one with the carry from the lanes before (a segmented wave
  // scan), into consecutive slots from the chunk's first (info.x); entries from info.y on are
  // padding, whose products are 0 whatever x holds.
  auto reduce_chunk = [&](const T (&v)[kPanelPerLane], const i32x4& cq, const i32x2& info) {
    const int slot0 = info.x, used = info.y;
    bool start[kPanelPerLane];
    T xg[kPanelPerLane];
    const uint32_t cw[4] = {(uint32_t)cq.x, (uint32_t)cq.y, (uint32_t)cq.z, (uint32_t)cq.w};
#pragma unroll
    for (int q = 0; q < kPanelPerLane; ++q) {
      const uint32_t e = (q & 1) ? cw[q >> 1] >> 16 : cw[q >> 1] & 0xffffu;
      xg[q] = sx[e & cmask];
      start[q] = (e & kRunStart) != 0;
    }
    // Padding (value 0) takes x = 0 too, so that it adds exactly 0 whatever x holds.  Only a
    // panel's last chunk and a chunk closed early have any (the same in all lanes), so the
    // others skip this; with a select on every product the kernel took 1.8 us longer (cfg3).
    if (used < (int)kPanelChunk) {
      const int lim = used - kPanelPerLane * lane;
#pragma unroll
      for (int q = 0; q < kPanelPerLane; ++q)
        if (q >= lim) xg[q] = T(0);
    }
    constexpr int kLast = kPanelPerLane - 1;
    // a chunk starts a run whatever its first entry says, and ends one (lane 63 reads 1)
    const bool cont = lane > 0 && !start[0];
    const bool end_last = dpp_mov<kDppWaveShl1>(1, (int)start[0]) != 0;
    // Running sums of the runs inside the lane (restarted where a run starts).  With float32
    // entries and fp64 sums a product is exact, so fma(v, x, s) is the sum s + v * x rounded
    // once, as an add of the product would be.
    int has_head = cont ? 0 : 1;
    int n_end = end_last ? 1 : 0;
    A run[kPanelPerLane];
    run[0] = A(v[0]) * A(xg[0]);
#pragma unroll
    for (int q = 1; q < kPanelPerLane; ++q) {
      if constexpr (sizeof(T) == 4 && sizeof(A) == 8) {
        run[q] = __builtin_fma(A(v[q]), A(xg[q]), start[q] ? A(0) : run[q - 1]);
      } else {
        const A p = A(v[q]) * A(xg[q]);
        run[q] = start[q] ? p : run[q - 1] + p;
      }
      has_head |= (int)start[q];
      n_end += (int)start[q];
    }
    // Segmented scan of (has_head, last piece) and a plain scan of n_end over the wave, all
    // through DPP; then each lane takes the scans of the lane before it: the carry into its
    // first run and its first slot.  (Branch-free steps, fma products and the stores below
    // took this kernel from 107 to 84 VGPRs and 878 to 729 VALU instructions; measured on
    // MI355X, cfg3: 94.2 -> 93.1 us, the whole call 263.6 -> 262.0 us.)
    int h_in = has_head;
    A v_in = run[kLast];
    int c_in = n_end;
    wave_seg_scan(h_in, v_in, c_in);
    const A carry = dpp_bc<kDppWaveShr1, 0xF>(v_in);   // lane 0: 0
    const int slot = dpp_bc<kDppWaveShr1, 0xF>(c_in);
    const int n_runs = __builtin_amdgcn_readlane(c_in, kWave - 1);
    // The chunk's runs go to this wave's LDS row in slot order, and one store of 64
    // consecutive slots writes them in whole lines (stored from the lanes where the runs end,
    // eight stores per lane pieced the lines together: 90 against 80 us on cfg3; and any
    // store that only some paths issue makes the compiler wait for every load in flight).
    // Every lane writes each of its eight run sums: to the run's slot where a run ends there,
    // else to a slot of its own past the chunk's.  Then the lane's first run, when it
    // continues from the lanes before, gets the carry.
    A* const st = s_stage[wid];
    int j = slot;
#pragma unroll
    for (int q = 0; q < kPanelPerLane; ++q) {
      const bool ends = q < kLast ? start[q + 1] : end_last;
      st[(ends && j < kWave) ? j : kWave + lane] = run[q];
      j += (int)ends;
    }
    {
      const bool fix = cont && j > slot && slot < kWave;
      const int at = fix ? slot : kWave + lane;
      st[at] = st[at] + (fix ? carry : A(0));
    }
    wave_sync();  // the row is written and read by this wave only
    const A staged = st[lane];
    store_partial(out_rsrc, lane < n_runs ? (unsigned)(slot0 + lane) * (unsigned)sizeof(A)
                                          : kDropOffset, staged);
    wave_sync();  // read before the next chunk writes the row again
  };

  // kNB chunk buffers per wave: while one chunk is reduced, the next kNB - 1 are in flight
  // (with two buffers the next chunk was requested only one reduction before it was needed,
  // and the waves waited on memory: 5.2 TB/s on cfg3's long rows).
  constexpr int kStride = kPanelBlock / kWave;
  constexpr int kNB = kPanelBuffers;
  T v[kNB][kPanelPerLane];
  i32x4 c[kNB];
  i32x2 sl[kNB];
#pragma unroll
  for (int b = 0; b < kNB; ++b) {
    c[b] = i32x4{0, 0, 0, 0};
    sl[b] = i32x2{0, 0};
  }
  int ch = jobs[job] + wid;
  // The first chunks' entries are requested before the panel copy, so the two overlap.
#pragma unroll
  for (int b = 0; b + 1 < kNB; ++b)
    if (ch + b * kStride < c_hi) load_chunk(ch + b * kStride, v[b], c[b], sl[b]);

  // Panel copy: every thread issues all its 16-byte loads before its first LDS store (one
  // memory round trip; as a load-store loop the copy waited for each load in turn).  A panel
  // starts at a multiple of 2^col_bits values; the vector part needs x 16-byte aligned there.
  {
    constexpr int kVec = 16 / (int)sizeof(T);
    constexpr int kCopy = (int)(kPanelBytes / 16 / kPanelBlock);  // vectors per thread, at most
    const T* src = x + pbase;
    const bool vec_ok = (reinterpret_cast<uintptr_t>(src) & 15u) == 0;
    const int n_vec = vec_ok ? width / kVec : 0;
    i32x4 buf[kCopy];
#pragma unroll
    for (int k = 0; k < kCopy; ++k) {
      const int i = (int)threadIdx.x + k * kPanelBlock;
      if (i < n_vec) buf[k] = *reinterpret_cast<const i32x4*>(src + (int64_t)i * kVec);
    }
#pragma unroll
    for (int k = 0; k < kCopy; ++k) {
      const int i = (int)threadIdx.x + k * kPanelBlock;
      if (i < n_vec) *reinterpret_cast<i32x4*>(sx + i * kVec) = buf[k];
    }
    for (int i = n_vec * kVec + (int)threadIdx.x; i < width; i += kPanelBlock) sx[i] = src[i];
  }
  __syncthreads();

  // Buffer b holds the chunks ch + b * kStride of each round; before reducing one, the chunk
  // kNB - 1 strides ahead is requested into the buffer reduced last.
  for (; ch < c_hi; ch += kNB * kStride) {
#pragma unroll
    for (int b = 0; b < kNB; ++b) {
      const int cur = ch + b * kStride;
      if (cur >= c_hi) break;
      const int ahead = cur + (kNB - 1) * kStride;
      if (ahead < c_hi) load_chunk(ahead, v[(b + kNB - 1) % kNB], c[(b + kNB - 1) % kNB],
                                   sl[(b + kNB - 1) % kNB]);
      reduce_chunk(v[b], c[b], sl[b]);
    }
  }
  // the staged-x entries of the job, from the same LDS panel
  if (scol != nullptr) {
    const __amdgpu_buffer_rsrc_t xs_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        xs, 0, (int)(n_xs * (int64_t)sizeof(T)), kBufferRsrcWord3);
    stage_panel_chunks<T>(sx, cmask, scol, sinfo, sdelta, stage_jobs[job], stage_jobs[job + 1],
                          xs_rsrc);
  }
}

template <typename T, typename A>
constexpr unsigned xcs_sorted_lds_reserve() {
  constexpr unsigned used = (unsigned)sorted_lds_bytes<T, A>() +
                            (unsigned)(kSortedWaves * (2 * sizeof(int) + sizeof(A))) +
                            (unsigned)(kItemRuns * sizeof(i32x4));
  return used < kXcsSortedLdsPerWorkgroup ? kXcsSortedLdsPerWorkgroup - used : 0u;
}

template <typename T, typename A>
int launch_xcs(int item_format, const void* vals, const uint32_t* pidx, int col_bits,
               const void* x, void* y, const int32_t* row_map, const int32_t* items,
               int64_t n_slots, const int32_t* item_runs, void* partials,
               const int32_t* windows, int64_t n_windows, int64_t window_slots,
               const int16_t* dest, const uint8_t* row_count, hipStream_t st) {
  if (n_slots > 0 && item_format == 1) {
    hipLaunchKernelGGL((spmv_xcs_sorted_kernel<T, A>), dim3((unsigned)n_slots),
                       dim3(kSortedBlock), (xcs_sorted_lds_reserve<T, A>()), st,
                       static_cast<const T*>(vals), pidx, static_cast<const T*>(x),
                       reinterpret_cast<const i32x4*>(items), (int)n_slots,
                       reinterpret_cast<const i32x4*>(item_runs), static_cast<A*>(partials));
    int rc = check_hip(hipGetLastError(), "spmv_xcs_sorted_kernel launch");
    if (rc) return rc;
  } else if (n_slots > 0) {
    hipLaunchKernelGGL((spmv_xcs_kernel<T, A, true>), dim3((unsigned)n_slots), dim3(kBlock),
                       xcs_lds_reserve<A>(), st, static_cast<const T*>(vals), pidx, col_bits,
                       static_cast<const T*>(x), reinterpret_cast<const i32x4*>(items),
                       (int)n_slots, reinterpret_cast<const i32x4*>(item_runs),
                       static_cast<A*>(partials));
    int rc = check_hip(hipGetLastError(), "spmv_xcs_kernel launch");
    if (rc) return rc;
  }
  if (n_windows == 0) return FSP_OK;
  hipLaunchKernelGGL((xcs_window_combine_kernel<T, A, kCombBlock>), dim3((unsigned)n_windows),
                     dim3(kCombBlock), (size_t)window_slots * sizeof(A), st,
                     reinterpret_cast<const i32x4*>(windows), dest, row_count,
                     static_cast<const A*>(partials), static_cast<T*>(y), row_map,
                     (int)window_slots);
  return check_hip(hipGetLastError(), "xcs_window_combine_kernel launch");
}

// Second pass of the panel layout: its rows have hundreds of slots each, so one wave adds a
// row's slots - lane l the slots k = l, l + 64, ... in order, then a fixed wave tree.  A chunk
// gives consecutive rows consecutive slots, so a line of partials serves 16 neighbouring rows:
// workgroups are remapped so that each XCD takes one contiguous range of rows and fetches such
// a line into its L2 once.
// Panel row i by the calling wave (the body of panel_combine_kernel).
template <typename T, typename A>
__device__ __forceinline__ void combine_panel_row(
    int i, const int* __restrict__ rows, const int* __restrict__ row_ptr,
    const int* __restrict__ slots, const A* __restrict__ partials, T* __restrict__ y,
    const int* __restrict__ row_map) {
  const int lane = threadIdx.x & (kWave - 1);
  const int a = row_ptr[i], b = row_ptr[i + 1];
  A acc = A(0);
  // slot indices, then partials, requested kU at a time (measured on MI355X, cfg3: 12.6 us
  // in hardware order, 9.3 us remapped, 8.6 us with 8 instead of 4 at a time)
  constexpr int kU = 8;
  for (int k0 = a + lane; k0 < b; k0 += kU * kWave) {
    int sl[kU];
    A pv[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) sl[u] = k0 + u * kWave < b ? slots[k0 + u * kWave] : -1;
#pragma unroll
    for (int u = 0; u < kU; ++u) pv[u] = sl[u] >= 0 ? partials[sl[u]] : A(0);
#pragma unroll
    for (int u = 0; u < kU; ++u) acc += pv[u];
  }
  acc = wave_sum(acc);
  if (lane == 0) {
    const int row = rows[i];
    y[row_map ? row_map[row] : row] = T(acc);
  }
}

template <typename T, typename A>
__global__ __launch_bounds__(kBlock) void panel_combine_kernel(
    const int* __restrict__ rows, const int* __restrict__ row_ptr, const int* __restrict__ slots,
    const A* __restrict__ partials, T* __restrict__ y, const int* __restrict__ row_map,
    int n_rows) {
  const int blk = xcd_logical_block((int)blockIdx.x, (int)gridDim.x);
  const int i = blk * kWavesPerBlock + (int)(threadIdx.x / kWave);
  if (i >= n_rows) return;  // whole waves leave together
  combine_panel_row<T, A>(i, rows, row_ptr, slots, partials, y, row_map);
}

// The second pass of the XCS + panel hybrid in one launch: workgroups [0, n_pblocks) take the
// panel part's rows (a wave each, NB / 64 rows per workgroup, remapped so that each XCD takes
// one contiguous range of rows), the rest the XCS part's combine windows, whose rows counted
// kRowSkip (the long rows) are left to the panel rows.  The panel rows' loads are latency
// bound (a slot index, then the partial it names); beside the windows' streams they cost
// little.
template <typename T, typename A, int NB>
__global__ __launch_bounds__(NB) void hybrid_combine_kernel(
    const i32x4* __restrict__ windows, const int16_t* __restrict__ dest,
    const uint8_t* __restrict__ row_count, const A* __restrict__ xcs_partials,
    int win_cap, const int* __restrict__ rows, const int* __restrict__ row_ptr,
    const int* __restrict__ slots, const A* __restrict__ panel_partials, int n_rows,
    int n_pblocks, T* __restrict__ y, const int* __restrict__ row_map) {
  const int b = (int)blockIdx.x;
  if (b < n_pblocks) {  // uniform
    const int i = xcd_logical_block(b, n_pblocks) * (NB / kWave) + (int)(threadIdx.x / kWave);
    if (i < n_rows)  // whole waves
      combine_panel_row<T, A>(i, rows, row_ptr, slots, panel_partials, y, row_map);
    return;
  }
  combine_window<T, A, NB>(b - n_pblocks, windows, dest, row_count, xcs_partials, y, row_map,
                           win_cap);
}

// N consecutive values from p (16-byte aligned) by 16-byte loads.
template <int N, typename T>
__device__ __forceinline__ void load16x(const T* __restrict__ p, T (&out)[N]) {
  constexpr int kPerLoad = 16 / sizeof(T);
  static_assert(N % kPerLoad == 0, "whole 16-byte loads");
  const i32x4* q = reinterpret_cast<const i32x4*>(p);
#pragma unroll
  for (int j = 0; j < N / kPerLoad; ++j) {
    const i32x4 w = q[j];
    __builtin_memcpy(&out[j * kPerLoad], &w, 16);
  }
}

// Staged-x windows (see the file comment).
constexpr uint32_t kStageSkip = 0x8000u;  // row_end: a row the window leaves alone

// Window w of the staged-x layout, NB threads: the window's entries f < L (its segments, one
// per panel with entries of the window's rows) are at first + f in vals, dest and xs (the
// staged x values, written there by the panel jobs), first a multiple of 8 and the arrays
// readable up to the next multiple of 8 past first + L.  Products go to LDS position dest (the
// entry's rank in (row, panel) order); a segmented scan over the positions (thread t:
// positions 8t .. 8t + 7 in order, marked where a row starts by the bits of heads[w * NB + t],
// then the threads and the waves in fixed DPP trees) leaves each row's sum at its
// last position, and row r of the window, positions [row_end[r - 1], row_end[r]) (0 for the
// first row), writes it to y.
template <typename T, typename A, int NB>
__device__ __forceinline__ void stage_combine_window(
    int w, const i32x4* __restrict__ windows, const T* __restrict__ vals,
    const int16_t* __restrict__ dest, const T* __restrict__ xs,
    const uint16_t* __restrict__ row_end, const uint8_t* __restrict__ heads,
    T* __restrict__ y, const int* __restrict__ row_map) {
  constexpr int kWaves = NB / kWave;
  constexpr int kPer = 8;                  // entries per thread
  constexpr int kCap = kPer * NB;          // entries of a window
  constexpr int kRowsPer = 4;              // rows per thread
  static_assert(kCap <= (int)kStageWinCap && kRowsPer * NB <= (int)kStageWinRows, "caps");
  static_assert(kPer == 8, "a thread scans one byte of row starts");
  // The products, position p at slot p + p / 8 (a thread's 8 positions then start 9 slots
  // after the previous thread's: its scan's LDS accesses do not all fall on the same banks).
  __shared__ A s_val[kCap + kCap / kPer];
  auto slot = [](int p) { return p + (p >> 3); };
  __shared__ int s_wh[kWaves];
  __shared__ A s_wv[kWaves];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wid = tid / kWave;
  const i32x4 win = windows[w];
  const int row0 = win.x, nr = win.y, L = win.z, first = win.w;
  if (nr > kRowsPer * NB || L > kCap || (first & (kPer - 1))) return;  // not a layout window
  // values, positions and staged x values: window-major, entries f0 .. f0 + 7 of the window
  // by 16-byte loads (the window starts at a multiple of 8 entries, the arrays are padded to
  // the next window); a thread past the end loads the first entries again, dropped below
  const int f0 = kPer * tid;
  const int64_t g = first + (f0 < L ? f0 : 0);
  T v[kPer], xv[kPer];
  int d[kPer];
  load16x<kPer>(vals + g, v);
  load16x<kPer>(xs + g, xv);
  {
    const i32x4 dw = *reinterpret_cast<const i32x4*>(dest + g);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      d[2 * j] = (int)(int16_t)(dw[j] & 0xFFFF);
      d[2 * j + 1] = dw[j] >> 16;
    }
  }
  const unsigned hb = heads[(int64_t)w * NB + tid];
  // the rows' positions: [start, end) (both 0 past the window's rows)
  int start[kRowsPer], end[kRowsPer];
  bool skip[kRowsPer];
#pragma unroll
  for (int m = 0; m < kRowsPer; ++m) {
    const int r = tid + m * NB;
    const unsigned e = r < nr ? row_end[row0 + r] : 0u;
    const unsigned e0 = (r > 0 && r < nr) ? row_end[row0 + r - 1] : 0u;
    skip[m] = (e & kStageSkip) != 0;
    end[m] = (int)(e & (kStageSkip - 1u));
    start[m] = (int)(e0 & (kStageSkip - 1u));
  }
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    if (f0 + k < L && (unsigned)d[k] < (unsigned)kCap) s_val[slot(d[k])] = A(v[k]) * A(xv[k]);
  }
  __syncthreads();  // the products in place
  // the segmented scan: positions past L start rows of their own (and add nothing).  Each
  // thread scans its positions in place; only the last position before its first row start
  // (k0) then needs what the threads before carry in - a row that ends later has its sum
  // complete from its own start.
  const int p0 = kPer * tid;
  const unsigned hv = hb | (p0 + kPer > L ? ~0u << (L > p0 ? L - p0 : 0) : 0u);
  const int k0 = hv ? __builtin_ctz(hv) : kPer;
  A run = A(0), pre = A(0);
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    if (p0 + q < L) {
      const A vq = s_val[slot(p0) + q];
      run = ((hv >> q) & 1u) ? vq : run + vq;
      if (q + 1 == k0) pre = run;
      s_val[slot(p0) + q] = run;
    }
  }
  int h_in = hv ? 1 : 0, dummy = 0;
  A v_in = run;
  wave_seg_scan(h_in, v_in, dummy);
  if (lane == kWave - 1) {
    s_wh[wid] = h_in;
    s_wv[wid] = v_in;
  }
  const A lane_c = dpp_bc<kDppWaveShr1, 0xF>(v_in);  // lane 0: 0
  const int lane_h = dpp_bc<kDppWaveShr1, 0xF>(h_in);
  __syncthreads();
  // What the waves before carry into this one: lane j takes wave j's (start, carry-out), a
  // segmented scan over lanes 0 .. kWaves - 1 (a fixed tree inside one 16-lane row), read at
  // lane wid - 1 (a loop over the waves before, one LDS read after another, measured slower).
  static_assert(kWaves <= 16, "the waves' carries are scanned inside one DPP row");
  int hw = lane < kWaves ? s_wh[lane] : 0, cw = 0;
  A vw = lane < kWaves ? s_wv[lane] : A(0);
  seg_scan_step<kDppRowShr1, 0xF>(hw, vw, cw);
  seg_scan_step<kDppRowShr1 + 1, 0xF>(hw, vw, cw);
  seg_scan_step<kDppRowShr1 + 3, 0xF>(hw, vw, cw);
  seg_scan_step<kDppRowShr1 + 7, 0xF>(hw, vw, cw);
  const A wave_c = wid > 0 ? lane_value(vw, wid - 1) : A(0);
  const A cin = lane_h ? lane_c : wave_c + lane_c;
  if (k0 > 0 && p0 + k0 - 1 < L) s_val[slot(p0) + k0 - 1] = cin + pre;
  __syncthreads();  // every row's sum at its last position
#pragma unroll
  for (int m = 0; m < kRowsPer; ++m) {
    const int i = tid + m * NB;
    if (i >= nr || skip[m]) continue;
    const int row = row0 + i;
    const bool any = end[m] > start[m] && end[m] <= L;
    y[row_map ? row_map[row] : row] = any ? T(s_val[slot(end[m] - 1)]) : T(0);
  }
}

// The second pass of the staged-x layout: workgroups [0, n_pblocks) take the panel part's
// long rows (as in hybrid_combine_kernel), the rest the windows.
template <typename T, typename A, int NB>
__global__ __launch_bounds__(NB) void stage_combine_kernel(
    const i32x4* __restrict__ windows, const T* __restrict__ vals,
    const int16_t* __restrict__ dest, const T* __restrict__ xs,
    const uint16_t* __restrict__ row_end, const uint8_t* __restrict__ heads,
    const int* __restrict__ rows,
    const int* __restrict__ row_ptr, const int* __restrict__ slots,
    const A* __restrict__ panel_partials, int n_rows, int n_pblocks, T* __restrict__ y,
    const int* __restrict__ row_map) {
  const int b = (int)blockIdx.x;
  if (b < n_pblocks) {  // uniform
    const int i = xcd_logical_block(b, n_pblocks) * (NB / kWave) + (int)(threadIdx.x / kWave);
    if (i < n_rows)  // whole waves
      combine_panel_row<T, A>(i, rows, row_ptr, slots, panel_partials, y, row_map);
    return;
  }
  // Windows in hardware order (consecutive windows on different XCDs, all of them reading near
  // the same addresses at a time), last first: the panel jobs stage the last windows' x values
  // last, so those are the likeliest still in the MALL.  Measured on MI355X (combine alone /
  // whole call): cfg3 69.9 / 195.4 us against 72.6 / 198.1 us with each XCD taking a
  // contiguous range of windows, 69.5 / 196.1 us first window first; cfg4 74.6 / 131.0 against
  // 78.4 / 134.9 us.
  const int nw = (int)gridDim.x - n_pblocks;
  stage_combine_window<T, A, NB>(nw - 1 - (b - n_pblocks), windows, vals, dest, xs, row_end,
                                 heads, y, row_map);
}

template <typename T, typename A>
int launch_panels(const void* vals, const uint16_t* pcol, int col_bits, const void* x,
                  int64_t x_len, void* y, const int32_t* row_map, const int32_t* jobs,
                  const int32_t* job_panel, int64_t n_jobs, const int32_t* chunk_info,
                  void* partials, int64_t n_partials, const int32_t* rows,
                  const int32_t* row_ptr, const int32_t* slots, int64_t n_rows,
                  const uint16_t* scol, const int32_t* stage_jobs, const int32_t* sinfo,
                  const int32_t* sdelta, void* xs, int64_t n_xs, hipStream_t st) {
  if (n_jobs > 0) {
    hipLaunchKernelGGL((spmv_panel_kernel<T, A>), dim3((unsigned)n_jobs), dim3(kPanelBlock),
                       ((size_t)1 << col_bits) * sizeof(T), st, static_cast<const T*>(vals),
                       pcol, col_bits, static_cast<const T*>(x), x_len, jobs, job_panel,
                       reinterpret_cast<const i32x2*>(chunk_info), static_cast<A*>(partials),
                       n_partials, scol, stage_jobs, reinterpret_cast<const i32x2*>(sinfo),
                       sdelta, static_cast<T*>(xs), n_xs);
    int rc = check_hip(hipGetLastError(), "spmv_panel_kernel launch");
    if (rc) return rc;
  }
  if (n_rows == 0) return FSP_OK;
  const int64_t blocks = (n_rows + kWavesPerBlock - 1) / kWavesPerBlock;
  hipLaunchKernelGGL((panel_combine_kernel<T, A>), dim3((unsigned)blocks), dim3(kBlock), 0, st,
                     rows, row_ptr, slots, static_cast<const A*>(partials), static_cast<T*>(y),
                     row_map, (int)n_rows);
  return check_hip(hipGetLastError(), "panel_combine_kernel launch");
}

template <typename T, typename A>
int launch_hybrid_combine(void* y, const int32_t* row_map, const void* xcs_partials,
                          const int32_t* windows, int64_t n_windows, int64_t window_slots,
                          const int16_t* dest, const uint8_t* row_count,
                          const void* panel_partials, const int32_t* rows,
                          const int32_t* row_ptr, const int32_t* slots, int64_t n_rows,
                          hipStream_t st) {
  constexpr int kRowsPerBlock = kCombBlock / kWave;
  const int64_t n_pblocks = (n_rows + kRowsPerBlock - 1) / kRowsPerBlock;
  const int64_t grid = n_pblocks + n_windows;
  if (grid == 0) return FSP_OK;
  hipLaunchKernelGGL((hybrid_combine_kernel<T, A, kCombBlock>), dim3((unsigned)grid),
                     dim3(kCombBlock), (size_t)window_slots * sizeof(A), st,
                     reinterpret_cast<const i32x4*>(windows), dest, row_count,
                     static_cast<const A*>(xcs_partials), (int)window_slots, rows, row_ptr,
                     slots, static_cast<const A*>(panel_partials), (int)n_rows, (int)n_pblocks,
                     static_cast<T*>(y), row_map);
  return check_hip(hipGetLastError(), "hybrid_combine_kernel launch");
}

// The staged-x combine's workgroup: 512 threads for windows of up to 4096 entries and 2048
// rows (four workgroups per CU), 1024 for twice that (two per CU).
template <typename T, typename A, int NB>
int launch_stage_combine_nb(void* y, const int32_t* row_map, const int32_t* windows,
                            int64_t n_windows, const void* vals, const int16_t* dest,
                            const void* xs, const uint16_t* row_end, const uint8_t* heads,
                            const void* panel_partials, const int32_t* rows,
                            const int32_t* row_ptr, const int32_t* slots, int64_t n_rows,
                            hipStream_t st) {
  constexpr int kRowsPerBlock = NB / kWave;
  const int64_t n_pblocks = (n_rows + kRowsPerBlock - 1) / kRowsPerBlock;
  const int64_t grid = n_pblocks + n_windows;
  if (grid == 0) return FSP_OK;
  hipLaunchKernelGGL((stage_combine_kernel<T, A, NB>), dim3((unsigned)grid), dim3(NB), 0, st,
                     reinterpret_cast<const i32x4*>(windows), static_cast<const T*>(vals), dest,
                     static_cast<const T*>(xs), row_end, heads, rows, row_ptr, slots,
                     static_cast<const A*>(panel_partials), (int)n_rows, (int)n_pblocks,
                     static_cast<T*>(y), row_map);
  return check_hip(hipGetLastError(), "stage_combine_kernel launch");
}

template <typename T, typename A>
int launch_stage_combine(void* y, const int32_t* row_map, const int32_t* windows,
                         int64_t n_windows, int64_t window_cap, const void* vals,
                         const int16_t* dest, const void* xs, const uint16_t* row_end,
                         const uint8_t* heads, const void* panel_partials, const int32_t* rows,
                         const int32_t* row_ptr, const int32_t* slots, int64_t n_rows,
                         hipStream_t st) {
  if (window_cap <= kStageWinCap / 2)
    return launch_stage_combine_nb<T, A, 512>(y, row_map, windows, n_windows, vals, dest, xs,
                                              row_end, heads, panel_partials, rows, row_ptr,
                                              slots, n_rows, st);
  return launch_stage_combine_nb<T, A, 1024>(y, row_map, windows, n_windows, vals, dest, xs,
                                             row_end, heads, panel_partials, rows, row_ptr,
                                             slots, n_rows, st);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace fsp

using namespace fsp;

extern "C" int fsp_spmv_xcs(int dtype, int acc_f64, const void* vals, const uint32_t* pidx,
                            int64_t n_entries, int col_bits, const void* x, void* y,
                            const int32_t* row_map, int64_t n_out, const int32_t* items,
                            int64_t n_slots, const int32_t* item_runs, void* partials,
                            const int32_t* windows, int64_t n_windows, int64_t window_slots,
                            const int16_t* dest, const uint8_t* row_count, int item_format,
                            void* stream) {
  if (dtype != FSP_F32 && dtype != FSP_F64) return set_error(FSP_ENOTSUP, "fsp_spmv_xcs: dtype");
  if (item_format != 0 && item_format != 1)
    return set_error(FSP_EINVAL, "fsp_spmv_xcs: item_format must be 0 or 1");
  if (item_format == 1 && col_bits > (int)kXcsSortedColBits)
    return set_error(FSP_EINVAL, "fsp_spmv_xcs: sorted-gather items take col_bits <= " +
                                     std::to_string(kXcsSortedColBits));
  if (n_entries < 0 || n_slots < 0 || n_out < 0 || n_windows < 0)
    return set_error(FSP_EINVAL, "fsp_spmv_xcs: negative size");
  if (n_entries > 0x7fffffffLL - kXcsSortedItemCap || n_slots > 0x3fffffffLL ||
      n_windows > 0x3fffffffLL)
    return set_error(FSP_EINVAL, "fsp_spmv_xcs: too many entries, slots or windows");
  if (col_bits < 1 || col_bits > 24)
    return set_error(FSP_EINVAL, "fsp_spmv_xcs: col_bits outside [1, 24]");
  if (n_windows > 0 && (window_slots < 1 || window_slots > kXcsWinSlotsCap))
    return set_error(FSP_EINVAL, "fsp_spmv_xcs: window_slots outside [1, " +
                                     std::to_string(kXcsWinSlotsCap) + "]");
  if (n_slots > 0 && (!vals || !pidx || !x || !items || !item_runs || !partials))
    return set_error(FSP_EINVAL, "fsp_spmv_xcs: null pointer");
  if (n_windows > 0 && (!y || !windows || !dest || !row_count || !partials))
    return set_error(FSP_EINVAL, "fsp_spmv_xcs: null combine-table pointer");
  if (!aligned16(vals) || !aligned16(pidx) || !aligned16(items) || !aligned16(item_runs) ||
      !aligned16(windows))
    return set_error(FSP_EINVAL,
                     "fsp_spmv_xcs: vals, pidx, items, item_runs and windows must be 16-byte "
                     "aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (row_map && n_out > 0) {
    int rc = (dtype == FSP_F32) ? fill_zero<float>(static_cast<float*>(y), n_out, st)
                                : fill_zero<double>(static_cast<double*>(y), n_out, st);
    if (rc) return rc;
  }
#define FSP_XCS_ARGS item_format, vals, pidx, col_bits, x, y, row_map, items, n_slots, item_runs, \
                     partials, windows, n_windows, window_slots, dest, row_count, st
  if (dtype == FSP_F32) {
    if (acc_f64) return launch_xcs<float, double>(FSP_XCS_ARGS);
    return launch_xcs<float, float>(FSP_XCS_ARGS);
  }
  return launch_xcs<double, double>(FSP_XCS_ARGS);
#undef FSP_XCS_ARGS
}

extern "C" int fsp_spmv_panels(int dtype, int acc_f64, const void* vals, const uint16_t* pcol,
                               int64_t n_entries, int col_bits, const void* x, int64_t x_len,
                               void* y, const int32_t* row_map, const int32_t* jobs,
                               const int32_t* job_panel, int64_t n_jobs,
                               const int32_t* chunk_info, void* partials, int64_t n_partials,
                               const int32_t* rows, const int32_t* row_ptr,
                               const int32_t* slots, int64_t n_rows, const uint16_t* scol,
                               int64_t n_staged, const int32_t* stage_jobs,
                               const int32_t* stage_info, const int32_t* seg_delta, void* xs,
                               int64_t n_xs, void* stream) {
  if (dtype != FSP_F32 && dtype != FSP_F64)
    return set_error(FSP_ENOTSUP, "fsp_spmv_panels: dtype");
  const int64_t vsize = dtype == FSP_F32 ? 4 : 8;
  if (n_entries < 0 || n_jobs < 0 || n_rows < 0 || x_len < 0 || n_partials < 0 ||
      n_staged < 0 || n_xs < 0)
    return set_error(FSP_EINVAL, "fsp_spmv_panels: negative size");
  if (n_partials * 8 > 0x7fffffffLL)
    return set_error(FSP_EINVAL, "fsp_spmv_panels: more partial slots than 2^31 bytes hold");
  if (n_entries % kPanelChunk != 0 || n_entries / kPanelChunk > 0x7fffffffLL ||
      n_jobs > 0x7fffffffLL || n_rows > 0x7fffffffLL - kBlock)
    return set_error(FSP_EINVAL, "fsp_spmv_panels: n_entries must be a multiple of " +
                                     std::to_string(kPanelChunk) + " and sizes within int32");
  if (n_staged % kStageChunk != 0 || n_staged > 0x3fffffffLL)
    return set_error(FSP_EINVAL, "fsp_spmv_panels: n_staged must be a multiple of " +
                                     std::to_string(kStageChunk) + " below 2^30");
  if (n_xs * vsize > 0x7fffffffLL)
    return set_error(FSP_EINVAL, "fsp_spmv_panels: staged values beyond 2^31 bytes");
  if (col_bits < 1 || col_bits > 15 || (vsize << col_bits) > kPanelBytes)
    return set_error(FSP_EINVAL, "fsp_spmv_panels: col_bits must be <= 15 and a panel of "
                                 "2^col_bits values must fit " +
                                     std::to_string(kPanelBytes) + " bytes of LDS");
  if (n_jobs > 0 && (!x || !jobs || !job_panel))
    return set_error(FSP_EINVAL, "fsp_spmv_panels: null pointer");
  if (n_jobs > 0 && n_entries > 0 && (!vals || !pcol || !chunk_info || !partials))
    return set_error(FSP_EINVAL, "fsp_spmv_panels: null entry pointer");
  if (n_jobs > 0 && n_staged > 0 && (!scol || !stage_jobs || !stage_info || !seg_delta || !xs))
    return set_error(FSP_EINVAL, "fsp_spmv_panels: null staging pointer");
  if ((reinterpret_cast<uintptr_t>(chunk_info) & 7u) != 0 ||
      (reinterpret_cast<uintptr_t>(stage_info) & 7u) != 0)
    return set_error(FSP_EINVAL,
                     "fsp_spmv_panels: chunk_info and stage_info must be 8-byte aligned");
  if (n_rows > 0 && (!y || !rows || !row_ptr || !slots || !partials))
    return set_error(FSP_EINVAL, "fsp_spmv_panels: null row pointer");
  if (!aligned16(vals) || !aligned16(pcol))
    return set_error(FSP_EINVAL, "fsp_spmv_panels: vals and pcol must be 16-byte aligned");
  if (n_jobs == 0 && n_rows == 0) return FSP_OK;
  if (n_staged == 0) scol = nullptr;  // the kernel stages nothing
  hipStream_t st = static_cast<hipStream_t>(stream);
#define FSP_PANEL_ARGS vals, pcol, col_bits, x, x_len, y, row_map, jobs, job_panel, n_jobs, \
                       chunk_info, partials, n_partials, rows, row_ptr, slots, n_rows, scol, \
                       stage_jobs, stage_info, seg_delta, xs, n_xs, st
  if (dtype == FSP_F32) {
    if (acc_f64) return launch_panels<float, double>(FSP_PANEL_ARGS);
    return launch_panels<float, float>(FSP_PANEL_ARGS);
  }
  return launch_panels<double, double>(FSP_PANEL_ARGS);
#undef FSP_PANEL_ARGS
}

extern "C" int fsp_spmv_stage_combine(int dtype, int acc_f64, void* y, const int32_t* row_map,
                                      int64_t n_out, const int32_t* windows, int64_t n_windows,
                                      int64_t window_cap, const void* vals,
                                      const int16_t* dest, const void* xs,
                                      int64_t n_entries, const uint16_t* row_end,
                                      const uint8_t* heads, const void* panel_partials,
                                      const int32_t* rows,
                                      const int32_t* row_ptr, const int32_t* slots,
                                      int64_t n_rows, void* stream) {
  if (dtype != FSP_F32 && dtype != FSP_F64)
    return set_error(FSP_ENOTSUP, "fsp_spmv_stage_combine: dtype");
  if (n_windows < 0 || n_rows < 0 || n_entries < 0 || n_out < 0)
    return set_error(FSP_EINVAL, "fsp_spmv_stage_combine: negative size");
  if (n_windows > 0x3fffffffLL || n_rows > 0x3fffffffLL || n_entries > 0x7fffffffLL)
    return set_error(FSP_EINVAL, "fsp_spmv_stage_combine: sizes beyond int32");
  if (n_windows > 0 && (!y || !windows || !vals || !dest || !xs || !row_end || !heads))
    return set_error(FSP_EINVAL, "fsp_spmv_stage_combine: null window-table pointer");
  if (n_windows > 0 && window_cap != kStageWinCap / 2 && window_cap != kStageWinCap)
    return set_error(FSP_EINVAL, "fsp_spmv_stage_combine: window_cap must be " +
                                     std::to_string(kStageWinCap / 2) + " or " +
                                     std::to_string(kStageWinCap));
  if (n_rows > 0 && (!y || !rows || !row_ptr || !slots || !panel_partials))
    return set_error(FSP_EINVAL, "fsp_spmv_stage_combine: null panel-row pointer");
  if (!aligned16(windows))
    return set_error(FSP_EINVAL, "fsp_spmv_stage_combine: windows must be 16-byte aligned");
  if (n_windows > 0 && (!aligned16(vals) || !aligned16(dest) || !aligned16(xs)))
    return set_error(FSP_EINVAL, "fsp_spmv_stage_combine: vals, dest and xs must be 16-byte "
                                 "aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (row_map && n_out > 0) {
    int rc = (dtype == FSP_F32) ? fill_zero<float>(static_cast<float*>(y), n_out, st)
                                : fill_zero<double>(static_cast<double*>(y), n_out, st);
    if (rc) return rc;
  }
#define FSP_STAGE_ARGS y, row_map, windows, n_windows, window_cap, vals, dest, xs, row_end, heads, \
                       panel_partials, rows, row_ptr, slots, n_rows, st
  if (dtype == FSP_F32) {
    if (acc_f64) return launch_stage_combine<float, double>(FSP_STAGE_ARGS);
    return launch_stage_combine<float, float>(FSP_STAGE_ARGS);
  }
  return launch_stage_combine<double, double>(FSP_STAGE_ARGS);
#undef FSP_STAGE_ARGS
}

extern "C" int fsp_spmv_hybrid_combine(int dtype, int acc_f64, void* y, const int32_t* row_map,
                                       const void* xcs_partials, const int32_t* windows,
                                       int64_t n_windows, int64_t window_slots,
                                       const int16_t* dest, const uint8_t* row_count,
                                       const void* panel_partials, const int32_t* rows,
                                       const int32_t* row_ptr, const int32_t* slots,
                                       int64_t n_rows, void* stream) {
  if (dtype != FSP_F32 && dtype != FSP_F64)
    return set_error(FSP_ENOTSUP, "fsp_spmv_hybrid_combine: dtype");
  if (n_windows < 0 || n_rows < 0)
    return set_error(FSP_EINVAL, "fsp_spmv_hybrid_combine: negative size");
  if (n_windows > 0x3fffffffLL || n_rows > 0x3fffffffLL)
    return set_error(FSP_EINVAL, "fsp_spmv_hybrid_combine: too many windows or rows");
  if (n_windows > 0 && (window_slots < 1 || window_slots > kXcsWinSlotsCap))
    return set_error(FSP_EINVAL, "fsp_spmv_hybrid_combine: window_slots outside [1, " +
                                     std::to_string(kXcsWinSlotsCap) + "]");
  if (n_windows > 0 && (!y || !windows || !dest || !row_count || !xcs_partials))
    return set_error(FSP_EINVAL, "fsp_spmv_hybrid_combine: null combine-table pointer");
  if (n_rows > 0 && (!y || !rows || !row_ptr || !slots || !panel_partials))
    return set_error(FSP_EINVAL, "fsp_spmv_hybrid_combine: null panel-row pointer");
  if (!aligned16(windows))
    return set_error(FSP_EINVAL, "fsp_spmv_hybrid_combine: windows must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t slots_lds = n_windows > 0 ? window_slots : 1;
#define FSP_HYB_ARGS y, row_map, xcs_partials, windows, n_windows, slots_lds, dest, row_count, \
                     panel_partials, rows, row_ptr, slots, n_rows, st
  if (dtype == FSP_F32) {
    if (acc_f64) return launch_hybrid_combine<float, double>(FSP_HYB_ARGS);
    return launch_hybrid_combine<float, float>(FSP_HYB_ARGS);
  }
  return launch_hybrid_combine<double, double>(FSP_HYB_ARGS);
#undef FSP_HYB_ARGS
}
