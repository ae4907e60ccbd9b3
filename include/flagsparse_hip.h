/*
 * flagsparse_hip.h - C ABI of the MI355X (gfx950) sparse-product library: CSR/COO SpMV,
 * CSR/COO SpMM, CSR SDDMM, and a Matrix Market reader.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t passed as void*.
 * Nothing here allocates device memory: workspaces (partial sums, descriptor tables) are
 * owned by the caller, which sizes them from the plan functions below.
 * Every function returns 0 on success or a negative fsp_status; fsp_last_error() then
 * holds a message for the calling thread.  No C++ exception crosses this boundary.
 *
 * Reference interfaces replaced (paths relative to the FlagSparse source tree,
 * src/flagsparse/sparse_operations/):
 *   fsp_plan_row_blocks  - bucket/split planning of spmv_csr.py:281-327 (_build_spmv_opt_buckets)
 *                          and spmm_csr.py:417-477 (_build_spmm_opt_split_metadata,
 *                          _build_spmm_opt_buckets); one descriptor table replaces the
 *                          per-bucket row lists.
 *   fsp_plan_windows_count / fsp_plan_windows_emit
 *                        - the same planning on the device (spmm_csr.py:417-477, the host
 *                          Python loop over long rows included), for per-call plans.
 *   fsp_spmv_csr         - the Triton launches of spmv_csr.py:329-376
 *                          (_triton_spmv_csr_impl_opt_prepared, use_opt=True) and
 *                          spmv_csr.py:510-536 (_triton_spmv_csr_impl_prepared, default
 *                          path, fp32 accumulated in fp64); with row_map != NULL it also
 *                          replaces the row-run launch of spmv_coo.py:254-268 (_spmv_coo_seg_*).
 *   fsp_spmv_xcs         - the same launches as fsp_spmv_csr (spmv_csr.py:329-376, :510-536,
 *                          spmv_coo.py:254-268) for matrices whose x does not fit one XCD's L2:
 *                          columns split into one panel per XCD (layout built by the prepare
 *                          step, flagsparse_amd/_spmv_layouts.py).
 *   fsp_spmv_panels      - the same launches, for the long rows of power-law matrices (x panels
 *                          copied to LDS), which also stage x for the short rows of the
 *                          staged-x layout; used with fsp_spmv_xcs or fsp_spmv_stage_combine.
 *   fsp_spmv_hybrid_combine
 *                        - the second pass of fsp_spmv_xcs and fsp_spmv_panels in one launch
 *                          (same reference launches: the row sums of spmv_csr.py:329-376 and
 *                          :510-536).
 *   fsp_spmv_stage_combine
 *                        - the second pass of the staged-x layout (its row sums) with that of
 *                          fsp_spmv_panels, in one launch (the same reference launches).
 *   fsp_spmv_coo_atomic  - spmv_coo.py:269-280 (_spmv_coo_atomic_*, sort_by_row=False).
 *   fsp_spmm_csr         - spmm_csr.py:525-574 (_triton_spmm_csr_impl, base path) and
 *                          spmm_csr.py:922-1055 (bucketed opt path incl. the two-pass
 *                          long-row split); for row-sorted COO also the row-run launch of
 *                          spmm_coo.py:394-461 (_triton_spmm_coo_rowrun_impl).
 *   fsp_spmm_coo_atomic  - spmm_coo.py:464-523 (_triton_spmm_coo_atomic_impl).
 *   fsp_sddmm_csr        - sddmm_csr.py:107-151 (_sddmm_csr_real_kernel) and its launch in
 *                          _run_sddmm_prepared (:271-347).
 *   fsp_index_stats      - the per-call index checks of spmm_coo.py:312-371 (min/max of row
 *                          and col) and the row-order test of the row-run route (:394-461).
 *   fsp_mtx_read         - the .mtx parsing of the reference's test loaders
 *                          (tests/test_spmv.py:29-103 and its copies).
 */
#ifndef FLAGSPARSE_HIP_H
#define FLAGSPARSE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Value type of data / x / y / B / C. */
enum fsp_dtype { FSP_F32 = 0, FSP_F64 = 1 };

enum fsp_status {
  FSP_OK = 0,
  FSP_EINVAL = -1,   /* bad argument (sizes, null pointers, alignment, unsupported combo) */
  FSP_EHIP = -2,     /* a HIP runtime call failed */
  FSP_ENOTSUP = -3   /* dtype / index width not built */
};

/* Message for the last failing call made by this thread ("" if none). */
const char* fsp_last_error(void);

/* ABI revision of this header (bumped on any signature change). */
int fsp_abi_version(void);

/* Kernel capacities the planner must respect (fixed at build time). */
int64_t fsp_spmv_stream_nnz_cap(void);   /* max nnz of one short-row block            */
int64_t fsp_spmv_stream_rows_cap(void);  /* max rows of one short-row block           */
int64_t fsp_spmv_chunk_nnz_cap(void);    /* max nnz of one long-row chunk             */
int64_t fsp_spmm_block_nnz_cap(void);    /* max nnz of one SpMM row block / row part  */
int64_t fsp_xcs_item_cap(void);          /* max entries of one XCS item               */
int64_t fsp_xcs_rows_cap(void);          /* max rows of one XCS tile                  */
int64_t fsp_xcs_window_slots_cap(void);  /* max partial slots of one XCS combine window */
int64_t fsp_xcs_window_rows_cap(void);   /* max rows of one XCS combine window        */
int64_t fsp_xcs_item_runs_cap(void);     /* max stored runs (windows) of one XCS item */
int64_t fsp_xcs_sorted_item_cap(void);   /* max entries of a sorted-gather XCS item     */
int64_t fsp_xcs_sorted_col_bits(void);   /* max col_bits of sorted-gather XCS items     */
int64_t fsp_panel_bytes_cap(void);       /* max bytes of one x panel (panel SpMV)     */
int64_t fsp_panel_chunk(void);           /* entries per chunk (panel SpMV)            */
int64_t fsp_panel_chunk_runs_cap(void);  /* runs (rows) per chunk, at most (panel SpMV) */
int64_t fsp_stage_window_cap(void);      /* max entries of one staged-x window          */
int64_t fsp_stage_window_rows_cap(void); /* max rows of one staged-x window             */
int64_t fsp_stage_chunk(void);           /* staged entries per chunk (staged-x layout)  */

/*
 * Host-side planner.  rowptr: host array of n_rows+1 int64 offsets (CSR indptr, or the
 * COO run offsets).  Rows are packed greedily, in row order, into descriptors of 4 int32:
 *   short-row block : {row_begin, row_end, 0, 0}      rows with len <= long_threshold,
 *                                                      block nnz <= nnz_cap, rows <= rows_cap
 *   long-row chunk  : {row, k, nchunks, part_base}    row split into ceil(len/chunk) chunks;
 *                                                      part_base = -1 when nchunks == 1
 * Pass desc_out == NULL to only count.  Outputs: number of descriptors, number of partial
 * slots (sum of nchunks over rows with nchunks > 1) and number of split rows.
 * Requires 1 <= long_threshold <= nnz_cap, rows_cap >= 1, chunk >= 1.
 */
int fsp_plan_row_blocks(const int64_t* rowptr, int64_t n_rows, int64_t nnz_cap,
                        int64_t rows_cap, int64_t long_threshold, int64_t chunk,
                        int32_t* desc_out, int64_t* n_desc, int64_t* n_parts,
                        int64_t* n_split_rows);

/*
 * Chunk plan of the panel layout (fsp_spmv_panels), on the host: panel p's runs - the entries
 * of one row inside the panel, run_len[r] >= 1 of them, r in [panel_runs[p], panel_runs[p+1])
 * - are laid out one after the other from where panel p - 1 ended; a chunk of `chunk` entries
 * closes when it is full or after the runs_cap-th run starting or continuing in it (its rest
 * is then padding), and each panel ends on a chunk boundary.  Out: run_pos[r], the storage
 * position of run r's first entry, and panel_end[p], the position after panel p.  No
 * reference counterpart: it keeps every chunk within the run count fsp_spmv_panels stages
 * (fsp_panel_chunk_runs_cap()); the reference has no panel layout.
 */
int fsp_plan_panel_chunks(const int64_t* panel_runs, int64_t n_panels, const int64_t* run_len,
                          int64_t chunk, int64_t runs_cap, int64_t* run_pos, int64_t* panel_end);

/*
 * The same chunk plan on the device (no host copy, no host loop), one wave per panel; the
 * prepare step takes it when a prefix sum of the run lengths does not already give the plan
 * (a chunk of more than runs_cap runs).  panel_runs, run_len: device int64 as above (every
 * run of at least one entry, not checked here); outputs, device int64: run_pos[r] = the
 * position of run r's first entry counted from its panel's first position, panel_len[p] =
 * panel p's padded length (a multiple of chunk), so that panel_end is their prefix sum.  Like
 * fsp_plan_panel_chunks it has no reference counterpart (the reference has no panel layout);
 * it keeps the prepare step on the device, as the planners below do for the reference's host
 * loops (spmm_csr.py:417-441).
 */
int fsp_plan_panel_chunks_device(const int64_t* panel_runs, int64_t n_panels,
                                 const int64_t* run_len, int64_t chunk, int64_t runs_cap,
                                 int64_t* run_pos, int64_t* panel_len, void* stream);

/*
 * The same plan built on the device in two passes (no host copy of rowptr, no host loop):
 * the rows are cut into windows of window_rows rows and each window is planned with the rules
 * of fsp_plan_row_blocks, except that no block crosses a window boundary.  Replaces the host
 * loop of spmm_csr.py:417-441 (_build_spmm_opt_split_metadata), the bucket lists of :444-477
 * and spmv_csr.py:281-327 (_build_spmv_opt_buckets).  One thread plans a window; with
 * long_threshold == nnz_cap it finds each block's end by binary search, so wide windows
 * (e.g. 16 * rows_cap rows) stay cheap.
 *   rowptr         device row pointers, int32 (rowptr_bits 32) or int64 (64), n_rows + 1
 *   window_rows    rows per window (>= 1)
 *   counts         pass 1 output, device int64 [3][n_win], n_win = ceil(n_rows / window_rows):
 *                  per window the number of descriptors, partial slots and split rows
 *   offsets        pass 2 input: the exclusive prefix sum of each of the three rows of counts
 *   desc           [n_desc] int32 quadruples, as fsp_plan_row_blocks writes them
 *   ranges         optional [n_desc][2] int64 entry ranges {lo, hi} (as fsp_spmv_csr takes)
 *   groups, group_base, split_rows
 *                  one combine group per split row, {s, 1, nch, 0} / first part / row (the
 *                  fsp_spmv_csr / fsp_spmm_csr group format); sized by pass 1's totals
 * Both passes are asynchronous on stream; the caller reads the totals (one small copy) between
 * them to size the tables.
 */
int fsp_plan_windows_count(const void* rowptr, int rowptr_bits, int64_t n_rows,
                           int64_t window_rows, int64_t nnz_cap, int64_t rows_cap,
                           int64_t long_threshold, int64_t chunk, int64_t* counts, void* stream);
int fsp_plan_windows_emit(const void* rowptr, int rowptr_bits, int64_t n_rows,
                          int64_t window_rows, int64_t nnz_cap, int64_t rows_cap,
                          int64_t long_threshold, int64_t chunk, const int64_t* offsets,
                          int32_t* desc, int64_t* ranges, int32_t* groups, int64_t* group_base,
                          int32_t* split_rows, void* stream);

/*
 * y = A @ x for CSR A (or COO row runs when row_map != NULL).
 *   dtype      FSP_F32 / FSP_F64 (vals, x, y)
 *   acc_f64    1: accumulate in fp64 (reference default path for fp32), 0: native type
 *   vals,cols  nnz entries; cols int32; both 16-byte aligned
 *   rowptr     n_rows+1 offsets, int32 (rowptr_bits=32) or int64 (64)
 *   row_map    NULL: output row r is y[r]; else y[row_map[r]] and y[0..n_out) is zeroed first
 *   desc       n_desc descriptors from fsp_plan_row_blocks with the caps above
 *   ranges     n_desc pairs of int64 {lo, hi}: the entry range of each descriptor (a short
 *              block's rowptr[r0] .. rowptr[r1], or chunk k of a row: lo = rowptr[row] +
 *              k*chunk, hi = min(lo + chunk, rowptr[row+1])), so the kernel's entry loads do
 *              not wait for the row pointers
 *   chunk      the chunk size the plan was built with (<= fsp_spmv_chunk_nnz_cap())
 *   partials   >= n_parts slots of 8 bytes (chunk sums of split rows)
 *   groups     n_groups split-row groups, 4 int32 each {first, S, n, 0}: rows
 *              split_rows[first .. first+S) get sum over j < n of
 *              partials[group_base[g] + j*S + s] (a second launch on the same stream).  For
 *              this layout every split row is its own group {g, 1, nch, 0} with base = part.
 *              Calls sharing partials must not overlap.
 *   xcd_remap  1: place consecutive descriptors on the same XCD (L2 locality of x); 0: hardware
 *              order (workgroup i on XCD i % 8), the faster choice measured for this kernel
 */
int fsp_spmv_csr(int dtype, int acc_f64, const void* vals, const int32_t* cols,
                 const void* rowptr, int rowptr_bits, int64_t n_rows, int64_t nnz,
                 const void* x, void* y, const int32_t* row_map, int64_t n_out,
                 const int32_t* desc, const int64_t* ranges, int64_t n_desc, int64_t chunk,
                 void* partials, const int32_t* groups, const int64_t* group_base,
                 const int32_t* split_rows, int64_t n_groups, int xcd_remap, void* stream);

/*
 * fsp_spmv_csr without a caller workspace, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  It has
 * no counterpart in the reference: it is fsp_spmv_csr with `partials` replaced by a static
 * device array of fsp_spmv_scratch_slots() 8-byte slots (1 MiB) that every GPU holds for the
 * life of the process.
 *   n_parts   the plan's partial slots (fsp_plan_row_blocks' n_parts, or the device planner's
 *             total); a plan needing more than fsp_spmv_scratch_slots() is rejected with
 *             FSP_EINVAL (use fsp_spmv_csr with a workspace of that size instead)
 * Nothing is allocated: the array's device address is resolved once per device
 * (hipGetSymbolAddress) on the first call made with that device current.  Every call on one
 * GPU shares the array: calls that overlap on one GPU (two streams, two threads) race and give
 * wrong sums.  The array keeps the last call's contents; a call writes every slot it reads
 * first, so nothing needs clearing.
 */
int64_t fsp_spmv_scratch_slots(void);
int fsp_spmv_csr_static(int dtype, int acc_f64, const void* vals, const int32_t* cols,
                        const void* rowptr, int rowptr_bits, int64_t n_rows, int64_t nnz,
                        const void* x, void* y, const int32_t* row_map, int64_t n_out,
                        const int32_t* desc, const int64_t* ranges, int64_t n_desc, int64_t chunk,
                        int64_t n_parts, const int32_t* groups, const int64_t* group_base,
                        const int32_t* split_rows, int64_t n_groups, int xcd_remap, void* stream);

/*
 * y = A @ x in the XCD column-split layout (fp32/fp64 values, fp64 or native accumulation).
 *   vals, pidx   n_entries padded entries (16-byte aligned), by item_format:
 *                0: items of <= fsp_xcs_item_cap() entries in row order, pidx = (local row <<
 *                   col_bits) | (column - the panel's first column), every item starting on a
 *                   multiple of 4 and stored thread-major (256 threads);
 *                1: items of <= fsp_xcs_sorted_item_cap() entries padded to a multiple of 512,
 *                   one workgroup of 512 threads; vals in row order, position 8t + e at quad
 *                   (e / 4) * P/8 + t (P the padded length), element e % 4; pidx in column
 *                   order in the same quads, entry (t/64)*512 + 64k + t%64 of the column order
 *                   as element k of thread t, each = (its row-order position << (B + 1)) |
 *                   (1 << B when it starts a row run there) | (column - the panel's first
 *                   column), B = fsp_xcs_sorted_col_bits()
 *   col_bits     in [1, 24] (format 1: <= fsp_xcs_sorted_col_bits())
 *   row_map      NULL: layout row r is y[r]; else y[row_map[r]] and y[0..n_out) is zeroed first
 *   items        n_slots slots of 12 int32 in launch order (slot j runs on XCD j / (n_slots/8)
 *                when n_slots is a multiple of 8): {entry start, count, rank k in tile, first
 *                stored run, r0, rows, panel first column, stored runs (<=
 *                fsp_xcs_item_runs_cap()), 0, 0, tile (-1 marks an empty slot), 0}
 *   item_runs    int32 quadruples {first slot, first sum, sums, stored length}: an item's row
 *                run sums (in row order) [first sum, first sum + sums) go to partials[first
 *                slot ...], followed by zeros up to the stored length
 *   partials     the stored slots (8 bytes each with fp64 accumulation, else the value size)
 *   windows, dest, row_count
 *                the second launch (y written in row order), one workgroup per window:
 *                windows[w] = 8 int32 {row0, rows, first slot, stored length, sums, 0, 0, 0}:
 *                rows [row0, row0 + rows) (<= fsp_xcs_window_rows_cap()) take their sums from
 *                partials[first slot .. + stored length): slot s goes to position dest[s] of the
 *                window (its rank in (row, item) order; -1: padding, dropped; at most
 *                window_slots <= fsp_xcs_window_slots_cap() sums, the LDS each workgroup
 *                takes) and row r gets the sum, in that order, of its row_count[r] positions
 *                (one byte per row, at most 254; a row's first position is the sum of the
 *                counts of the window's rows before it; a count of 255 marks a row without
 *                sums that the window leaves alone - y written by fsp_spmv_hybrid_combine's
 *                panel rows).  rows = -1: one row given the sum of all the window's slots (a
 *                row with more sums than a window takes, or more than 254).  Calls sharing
 *                partials must not overlap.
 */
int fsp_spmv_xcs(int dtype, int acc_f64, const void* vals, const uint32_t* pidx,
                 int64_t n_entries, int col_bits, const void* x, void* y,
                 const int32_t* row_map, int64_t n_out, const int32_t* items, int64_t n_slots,
                 const int32_t* item_runs, void* partials, const int32_t* windows,
                 int64_t n_windows, int64_t window_slots, const int16_t* dest,
                 const uint8_t* row_count, int item_format, void* stream);

/*
 * y[rows[i]] (y[row_map[rows[i]]] when row_map != NULL) = row i of A @ x for the long rows of
 * a matrix in the panel layout: x is cut into panels of 2^col_bits columns, copied one at a
 * time into LDS, and the gathers read LDS.  Same reference launches as fsp_spmv_csr; used
 * beside fsp_spmv_xcs for power-law matrices, whose long rows put many entries in every panel.
 *   vals, pcol   n_entries entries (a multiple of fsp_panel_chunk(), both 16-byte aligned)
 *                in (panel, row) order, each panel's run padded with val 0 entries of its
 *                last row (padding only at the end of a chunk).  pcol (16 bits) = column - panel * 2^col_bits, | 0x8000 when the
 *                entry starts a run: its row differs from the previous entry's (the first
 *                entry of a chunk always starts one).  vals: inside each chunk the quad (4
 *                entries) at logical position 2L + h is stored at quad position 64h + L
 *                (L < 64, h < 2); pcol in logical order
 *   col_bits     <= 15, and 2^col_bits values must fit fsp_panel_bytes_cap() bytes
 *   jobs         n_jobs + 1 increasing chunk indices: workgroup j copies panel job_panel[j] of
 *                x (x_len values in all) into LDS and runs chunks [jobs[j], jobs[j+1])
 *   chunk_info   per chunk two int32 (8-byte aligned): its first partial slot (8 bytes each)
 *                and the number of its entries in use, the rest being padding that adds
 *                exactly 0 whatever x holds; a chunk writes one slot per run it holds, in
 *                entry order, and holds at most fsp_panel_chunk_runs_cap() runs (the sums of
 *                runs past that many are not written)
 *   n_partials   slots in partials (n_partials * 8 < 2^31: the kernel stores through a buffer
 *                resource of that size)
 *   rows, row_ptr, slots
 *                n_rows long rows; rows[i] gets the sum of partials[slots[k]], k in
 *                [row_ptr[i], row_ptr[i+1]) (a second launch, one wave per row: lane l adds
 *                k = l, l + 64, ... in order, then a fixed tree).  Calls sharing partials must
 *                not overlap.  Other rows of y are not written.
 */
int fsp_spmv_panels(int dtype, int acc_f64, const void* vals, const uint16_t* pcol,
                    int64_t n_entries, int col_bits, const void* x, int64_t x_len, void* y,
                    const int32_t* row_map, const int32_t* jobs, const int32_t* job_panel,
                    int64_t n_jobs, const int32_t* chunk_info, void* partials,
                    int64_t n_partials, const int32_t* rows, const int32_t* row_ptr,
                    const int32_t* slots, int64_t n_rows, const uint16_t* scol,
                    int64_t n_staged, const int32_t* stage_jobs, const int32_t* stage_info,
                    const int32_t* seg_delta, void* xs, int64_t n_xs, void* stream);

/*
 * The staged-x layout (the short rows of matrices whose columns are spread over an x larger
 * than an L2).  Its first pass is fsp_spmv_panels' jobs: job j, beside its chunks of long
 * rows, stages x for chunks [stage_jobs[j], stage_jobs[j+1]) of fsp_stage_chunk() entries of
 * its panel: scol (16 bits each, n_staged of them, a multiple of the chunk) = column -
 * panel * 2^col_bits, | 0x8000 where the entry opens a segment (the entries of one panel for
 * one window of rows); stage_info per chunk two int32 (8-byte aligned) {the segment of its
 * first entry, its entries in use (the rest padding)}, a chunk holding at most 64 segments
 * (counting the one its first entry continues); seg_delta per segment an int32 (and 64 more,
 * any value, readable after the last): entry e of segment s stores its x value at xs[e +
 * seg_delta[s]], inside xs[0 .. n_xs) (n_xs values of 2^31 bytes at most; a store outside is
 * dropped).  n_staged = 0 stages nothing.
 * fsp_spmv_stage_combine is the second pass: one workgroup per window of rows, beside the
 * panel part's long rows (rows .. n_rows, over panel_partials, as fsp_spmv_panels' second
 * pass; n_rows may be 0).  Same reference launches as fsp_spmv_csr.
 *   windows      n_windows int32 quadruples {row0, rows, entries L, first}: rows [row0, row0 +
 *                rows) (<= window_cap / 2), L <= window_cap entries at [first, first + L) of
 *                vals, dest and xs, first a multiple of 8 (a window otherwise is skipped);
 *                the arrays (n_entries long, 16-byte aligned) readable up to the next
 *                multiple of 8 past first + L
 *   window_cap   fsp_stage_window_cap() or half of it: workgroups of 1024 or 512 threads
 *   dest         int16 per entry: its rank in the window's (row, panel) order; the product
 *                vals[i] * xs[i] (in the accumulation type) goes to that position
 *   row_end      uint16 per row: the end of the row's positions in its window (it starts
 *                where the window's previous row ends, the first at 0), | 0x8000 for a row
 *                the window leaves alone (y written by the panel rows); row r gets the sum of
 *                its positions (a segmented scan over the window's positions: 8 consecutive
 *                positions per thread in order, then the threads and the waves in fixed
 *                trees)
 *   heads        window_cap / 8 bytes per window: bit q of byte t set where position 8t + q
 *                starts a row (a row of the window with entries)
 *   row_map      NULL: layout row r is y[r]; else y[row_map[r]], and y[0..n_out) is zeroed
 *                first
 * Calls sharing xs or panel_partials must not overlap.
 */
int fsp_spmv_stage_combine(int dtype, int acc_f64, void* y, const int32_t* row_map,
                           int64_t n_out, const int32_t* windows, int64_t n_windows,
                           int64_t window_cap, const void* vals, const int16_t* dest,
                           const void* xs,
                           int64_t n_entries, const uint16_t* row_end, const uint8_t* heads,
                           const void* panel_partials, const int32_t* rows,
                           const int32_t* row_ptr, const int32_t* slots, int64_t n_rows,
                           void* stream);

/*
 * The second passes of fsp_spmv_xcs (the combine windows: windows .. row_count, over
 * xcs_partials) and of fsp_spmv_panels (its long rows: rows, row_ptr, slots, over
 * panel_partials) in one launch, after both first passes (called with n_windows = 0 and
 * n_rows = 0 respectively), on the same stream.  The windows' rows counted 255 are the long
 * rows, whose y the panel rows write.  Same tables and semantics as the two calls' second
 * passes; the panel rows' latency-bound loads run beside the windows' streams.
 */
int fsp_spmv_hybrid_combine(int dtype, int acc_f64, void* y, const int32_t* row_map,
                            const void* xcs_partials, const int32_t* windows, int64_t n_windows,
                            int64_t window_slots, const int16_t* dest, const uint8_t* row_count,
                            const void* panel_partials, const int32_t* rows,
                            const int32_t* row_ptr, const int32_t* slots, int64_t n_rows,
                            void* stream);

/*
 * y = A @ x for unsorted COO with atomics (reference sort_by_row=False route); y[0..n_rows)
 * is zeroed first.  Accumulation order, and so the last bits of y, are not deterministic.
 * nnz_per_block: entries per 256-thread workgroup (reference block_size knob).
 */
int fsp_spmv_coo_atomic(int dtype, const void* vals, const int32_t* rows, const int32_t* cols,
                        int64_t nnz, const void* x, void* y, int64_t n_rows,
                        int64_t nnz_per_block, void* stream);

/*
 * C[n_rows, N] = A @ B for CSR A and row-major B[n_cols, ldb] (N columns used).
 *   lanes_per_row  G in {1,2,4,...,64}: lanes sharing one B row; the plan must have been
 *                  built with rows_cap <= 256/G and nnz_cap <= fsp_spmm_block_nnz_cap()
 *   vec            elements per lane per load: 4 (fp32) / 2 (fp64) for 16-byte loads, or 1;
 *                  vec > 1 requires ldb, ldc, N multiples of vec and 16-byte aligned B, C
 *   partials       >= n_parts * N slots of 8 bytes (part sums of rows cut into parts)
 *   groups         one per row cut into parts, {g, 1, nch, 0}: C[split_rows[g], :] = sum over
 *                  k < nch of partials[(group_base[g] + k) * N + :] (a second launch on the
 *                  same stream).  Calls sharing partials must not overlap.
 */
int fsp_spmm_csr(int dtype, int acc_f64, const void* vals, const int32_t* cols,
                 const void* rowptr, int rowptr_bits, int64_t n_rows, int64_t nnz,
                 const void* B, int64_t ldb, int64_t N, void* C, int64_t ldc,
                 const int32_t* desc, int64_t n_desc, int64_t chunk, int lanes_per_row,
                 int vec, void* partials, const int32_t* groups, const int64_t* group_base,
                 const int32_t* split_rows, int64_t n_groups, int xcd_remap, void* stream);

/*
 * COO SpMM with atomics: C_acc[rows[e], n] += vals[e] * B[cols[e], n] for every entry e and
 * n < N.  Replaces the reference's atomic route, spmm_coo.py:244-271 (_spmm_coo_atomic_real_
 * kernel) and :464-523 (_triton_spmm_coo_atomic_impl).  C_acc[0 .. n_rows*ldc) is zeroed first;
 * it holds fp64 when dtype is FSP_F64 or acc_f64 != 0 (the reference computes fp32 inputs in
 * fp64), else fp32, and the caller rounds it to the output dtype.  The addition order, and so
 * the last bits of C_acc, are not deterministic.  The row-run route (flagsparse_spmm_coo's
 * default) needs no entry point of its own: row-ordered entries with their row pointer are CSR,
 * and go through fsp_spmm_csr.
 */
int fsp_spmm_coo_atomic(int dtype, int acc_f64, const void* vals, const int32_t* rows,
                        const int32_t* cols, int64_t nnz, const void* B, int64_t ldb, int64_t N,
                        void* C_acc, int64_t ldc, int64_t n_rows, void* stream);

/*
 * Index checks in one pass: out[0..5) = {min a, max a, min b, max b, number of i in [1, n) with
 * a[i] < a[i-1]} over n entries of two index arrays (a_bits / b_bits 32 or 64, int32 / int64).
 * partial is device scratch of fsp_index_stats_partial_len() int64 values; out is 5 int64 on
 * the device.  Two launches on the stream, no host synchronisation.  n == 0 gives
 * {INT64_MAX, INT64_MIN, INT64_MAX, INT64_MIN, 0}.
 */
int fsp_index_stats(const void* a, int a_bits, const void* b, int b_bits, int64_t n,
                    int64_t* partial, int64_t* out, void* stream);
int64_t fsp_index_stats_partial_len(void);

/*
 * CSR SDDMM: out[p] = alpha * dot(x[row(p), 0..K), y[cols[p], 0..K)) + beta * data_in[p]
 * for p < nnz (the data_in term only when data_in != NULL), x [.][ldx] and y [.][ldy] row-major.
 *   dtype            FSP_F32 / FSP_F64 (x, y, data_in)
 *   acc_f64          fp32 inputs: accumulate in fp64 (the reference's "acc64" variant)
 *   out_f64          fp32 inputs: out holds fp64 (the "acc64_out64" variant), else the input type
 *   lanes_per_entry  G in {1,2,4,...,64} lanes share one entry
 *   vec              elements per lane per load: 4 (fp32) / 2 (fp64) for 16-byte loads, or 1;
 *                    vec > 1 requires K, ldx, ldy multiples of vec and 16-byte aligned x, y
 * Two schedules:
 *   n_desc > 0       a row-block plan (fsp_plan_windows_* or fsp_plan_row_blocks with
 *                    rows_cap <= 256/G, nnz_cap and chunk <= fsp_spmm_block_nnz_cap()): desc,
 *                    ranges and the CSR rowptr (int32 or int64, rowptr_bits) of the pattern;
 *                    needs K <= 4*G*vec and 16-byte aligned cols; row_ids is not read
 *   n_desc == 0      one lane group per entry; row_ids gives each entry's row
 * Deterministic: a fixed reduction order per entry.
 */
int fsp_sddmm_csr(int dtype, int acc_f64, int out_f64, const int32_t* cols,
                  const int32_t* row_ids, const void* rowptr, int rowptr_bits, int64_t nnz,
                  const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t K,
                  const void* data_in, double alpha, double beta, void* out,
                  const int32_t* desc, const int64_t* ranges, int64_t n_desc,
                  int lanes_per_entry, int vec, void* stream);

/*
 * Matrix Market coordinate file reader (host only, no GPU): the format of the reference's
 * SuiteSparse test drivers (tests/test_spmv.py:29-103, tests/test_spmm_coo.py:156-249,
 * tests/test_spmv_coo.py:257-305).  info[0..7) receives n_rows, n_cols, the header nnz, the
 * field (0 real / integer, 1 pattern, 2 complex), the symmetry (0 general, 1 symmetric,
 * 2 skew-symmetric, 3 hermitian), the number of entries read and how many lacked a value.
 * With rows == NULL only the header is read; otherwise up to min(nnz, capacity) entry lines
 * are returned as 0-based rows / cols and vals (two doubles per entry for complex files), in
 * file order; lines with fewer than two tokens are skipped.  Expansion of symmetric storage
 * and duplicate summation are left to the caller.
 */
int fsp_mtx_read(const char* path, int64_t* info, int64_t* rows, int64_t* cols, double* vals,
                 int64_t capacity);

/*
 * Measurement probes (bench.py): no counterpart in the reference and not on the product path.
 * They time, alone, the access patterns the kernels above are bound by.  Each workgroup writes
 * the sum of what it loaded to out[workgroup] (fsp_probe_*_blocks(n) values).
 *   fsp_probe_gather  n (a multiple of 4) random 4-byte gathers x[idx[i]] from fp32 x[x_len],
 *                     16 per thread in flight (idx int32, 16-byte aligned; clamped into x)
 *   fsp_probe_rows    n random gathers of whole 256-byte rows b[rows[i]][0..64) from a
 *                     row-major fp32 b[n_rows][64], 16 lanes per row, 4 rows per lane in
 *                     flight (row indices clamped into b)
 *   fsp_probe_stream  a read of n16 consecutive 16-byte vectors from src (16-byte aligned),
 *                     non-temporal loads, 8 per thread in flight (the value written is a parity
 *                     bit count, only there so that no load can be dropped)
 */
int64_t fsp_probe_gather_blocks(int64_t n);
int fsp_probe_gather(const float* x, int64_t x_len, const int32_t* idx, int64_t n, float* out,
                     void* stream);
int64_t fsp_probe_rows_blocks(int64_t n);
int fsp_probe_rows(const float* b, int64_t n_rows, int64_t row_floats, const int32_t* rows,
                   int64_t n, float* out, void* stream);
int64_t fsp_probe_stream_blocks(int64_t n16);
int fsp_probe_stream(const void* src, int64_t n16, float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FLAGSPARSE_HIP_H */
