/*
 * fsp_oracle.c - CPU oracle for the flagsparse_amd hot path.
 *
 * TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may call this code, and only as the checker.  The product path (flagsparse_amd) never
 * links, loads or calls it.
 *
 * What "correct" means for the reference (src/flagsparse/...): every test of the path
 * compares against an fp64 accumulation of the same products -
 *   tests/test_spmv.py:143-174      fp64 torch.sparse.mm for CSR SpMV, cast back
 *   tests/test_spmv_coo.py:56-71    fp64 coalesced COO mm for COO SpMV
 *   tests/test_spmm.py:270-311      fp64 torch.sparse.mm for CSR SpMM
 * and the reference's default SpMV path itself sums fp32 inputs in fp64
 * (sparse_operations/spmv_csr.py:498-536).  These functions restate that sum plainly:
 * one row at a time, entries in storage order, every product and sum in fp64.
 */
#include <stddef.h>
#include <stdint.h>

/*
 * y[r] = sum of vals[i] * x[cols[i]] for i in [rowptr[r], rowptr[r] + cap_r), where
 * cap_r = rowptr[r+1] - rowptr[r], or min(that, row_cap[r]) when row_cap != NULL.
 * Follows spmv_csr.py:94-120 (_spmv_csr_real_kernel): the row's entries are summed and
 * entries beyond MAX_SEGMENTS * BLOCK_NNZ are not visited (row_cap carries that limit).
 */
void oracle_spmv_csr_f64(int64_t n_rows, const int64_t* rowptr, const int64_t* cols,
                         const double* vals, const double* x, const int64_t* row_cap,
                         double* y) {
  for (int64_t r = 0; r < n_rows; ++r) {
    int64_t b = rowptr[r], e = rowptr[r + 1];
    if (row_cap && e - b > row_cap[r]) e = b + row_cap[r];
    double acc = 0.0;
    for (int64_t i = b; i < e; ++i) acc += vals[i] * x[cols[i]];
    y[r] = acc;
  }
}

/*
 * y = A @ x for COO entries in the given order: y[0..n_rows) = 0, then y[rows[i]] +=
 * vals[i] * x[cols[i]].  Follows spmv_coo.py:51-108 (row-run kernel: one sum per run, rows
 * without entries stay 0 from y = zeros at spmv_coo.py:250) and the coalesced fp64 reference
 * of tests/test_spmv_coo.py:56-71 (duplicates are summed).
 */
void oracle_spmv_coo_f64(int64_t nnz, const int64_t* rows, const int64_t* cols,
                         const double* vals, const double* x, int64_t n_rows, double* y) {
  for (int64_t r = 0; r < n_rows; ++r) y[r] = 0.0;
  for (int64_t i = 0; i < nnz; ++i) y[rows[i]] += vals[i] * x[cols[i]];
}

/*
 * C[r, n] = sum over the row's entries of vals[i] * B[cols[i], n], fp64, for n < N.
 * Follows spmm_csr.py:92-134 (_spmm_csr_real_kernel with ACC_DTYPE fp64 for fp32 inputs,
 * spmm_csr.py:548-555) and tests/test_spmm.py:270-311.
 */
void oracle_spmm_csr_f64(int64_t n_rows, const int64_t* rowptr, const int64_t* cols,
                         const double* vals, const double* B, int64_t ldb, int64_t N,
                         double* C, int64_t ldc) {
  for (int64_t r = 0; r < n_rows; ++r) {
    double* c = C + r * ldc;
    for (int64_t n = 0; n < N; ++n) c[n] = 0.0;
    for (int64_t i = rowptr[r]; i < rowptr[r + 1]; ++i) {
      const double a = vals[i];
      const double* b = B + cols[i] * ldb;
      for (int64_t n = 0; n < N; ++n) c[n] += a * b[n];
    }
  }
}

/*
 * C = A @ B for COO entries in the given order, row-major B[., ldb] and C[n_rows, ldc]:
 * C[0..n_rows) = 0, then C[rows[i], n] += vals[i] * B[cols[i], n] for n < N, fp64.  Follows
 * spmm_coo.py:136-180 (row-run kernel over the lexicographically sorted, coalesced entries;
 * rows without a run keep 0 from C = zeros at spmm_coo.py:414) and its fp64 torch.sparse
 * reference (spmm_coo.py:697-713): duplicates of one (row, col) are summed.
 */
void oracle_spmm_coo_f64(int64_t nnz, const int64_t* rows, const int64_t* cols,
                         const double* vals, const double* B, int64_t ldb, int64_t N,
                         int64_t n_rows, double* C, int64_t ldc) {
  for (int64_t r = 0; r < n_rows; ++r)
    for (int64_t n = 0; n < N; ++n) C[r * ldc + n] = 0.0;
  for (int64_t i = 0; i < nnz; ++i) {
    double* c = C + rows[i] * ldc;
    const double* b = B + cols[i] * ldb;
    for (int64_t n = 0; n < N; ++n) c[n] += vals[i] * b[n];
  }
}

/*
 * SDDMM on a CSR pattern: out[p] = alpha * sum_k x[r, k] * y[cols[p], k] + beta * data[p] for
 * the entries p of row r, fp64, k in increasing order (the data term only when data != NULL).
 * Follows sddmm_csr.py:107-151 (_sddmm_csr_real_kernel) and its torch reference
 * sddmm_csr.py:425-437; x [n_rows][ldx], y [.][ldy] row-major.
 */
void oracle_sddmm_csr_f64(int64_t n_rows, const int64_t* rowptr, const int64_t* cols,
                          const double* x, int64_t ldx, const double* y, int64_t ldy, int64_t K,
                          const double* data, double alpha, double beta, double* out) {
  for (int64_t r = 0; r < n_rows; ++r) {
    const double* xr = x + r * ldx;
    for (int64_t p = rowptr[r]; p < rowptr[r + 1]; ++p) {
      const double* yc = y + cols[p] * ldy;
      double acc = 0.0;
      for (int64_t k = 0; k < K; ++k) acc += xr[k] * yc[k];
      out[p] = alpha * acc + (data ? beta * data[p] : 0.0);
    }
  }
}
