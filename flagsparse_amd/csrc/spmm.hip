// CSR SpMM C = A @ B for gfx950 (row-major B and C), one launch over a descriptor table.
//
// Reference behaviour followed (src/flagsparse/sparse_operations/):
//   spmm_csr.py:92-134     base kernel, C[row, n] = sum_k a_k * B[col_k, n]; fp32 inputs are
//                          computed in fp64 (spmm_csr.py:544-573)
//   spmm_csr.py:602-775    opt batched / vector row kernels (native precision)
//   spmm_csr.py:778-919    opt long-row split: per-part sums, then parts added in index order
//
// Mapping (a gather-bound contraction, so no MFMA):
//   * G lanes share one B row; each lane owns VW consecutive columns (16-byte loads for
//     VW = 4 fp32 / 2 fp64), so a group covers a tile of W = G*VW columns; blockIdx.y
//     selects the tile.
//   * short-row block {r0, r1, 0, 0}: the block's (col, val) entries are staged into LDS with
//     16-byte loads; group g computes row r0+g alone (no cross-lane reduction), 4 B rows in
//     flight per lane.
//   * row part {row, k, nch, part}: the 256/G groups stride over the part's entries, then a
//     fixed-order LDS reduction over groups; with nch > 1 the part's sums go to partials and
//     a second launch (spmm_split_combine_kernel) adds a row's parts in index order.
#include "fsp_device.hpp"
#include "fsp_internal.hpp"

namespace fsp {
namespace {

constexpr int kSlots = (int)kSpmmSlots;
// B rows requested together per lane of a short row.  Measured on MI355X, cfg5 (fp32 N=64):
// 663.5 / 663.0 / 661.9 us with 4 / 6 / 8 (N=16: 324.7 / 325.3 / 326.0; fp64 N=16: 367.2 /
// 368.4 / 366.5): the kernel is bound by the rate at which L2 misses are filled, not by the
// loads a lane keeps in flight.
constexpr int kRowsInFlight = 4;
constexpr int kStageUPT = kSlots / (4 * kBlock);
static_assert(kStageUPT * 4 * kBlock == kSlots, "staging slots must be whole quads per thread");

template <typename T, int VW> struct VecOf;
template <> struct VecOf<float, 4> { typedef f32x4 type; };
template <> struct VecOf<float, 2> { typedef f32x2 type; };
template <> struct VecOf<float, 1> { typedef float type; };
template <> struct VecOf<double, 2> { typedef f64x2 type; };
template <> struct VecOf<double, 1> { typedef double type; };

template <typename T, int VW>
__device__ __forceinline__ void load_vec(const T* p, T (&out)[VW]) {
  typedef typename VecOf<T, VW>::type V;
  const V v = *reinterpret_cast<const V*>(p);
  if constexpr (VW == 1) {
    out[0] = v;
  } else {
#pragma unroll
    for (int j = 0; j < VW; ++j) out[j] = v[j];
  }
}

template <typename T, typename A, int VW>
__device__ __forceinline__ void store_vec(T* p, const A (&acc)[VW]) {
  typedef typename VecOf<T, VW>::type V;
  V v;
  if constexpr (VW == 1) {
    v = T(acc[0]);
  } else {
#pragma unroll
    for (int j = 0; j < VW; ++j) v[j] = T(acc[j]);
  }
  *reinterpret_cast<V*>(p) = v;
}

struct SplitGroups {
  const int32_t* groups;
  const int64_t* base;
  const int32_t* rows;
  int64_t n;
};

template <typename T, typename A, int VW>
constexpr int spmm_scratch_bytes() {
  return (kSlots * (int)sizeof(T) > kBlock * VW * (int)sizeof(A)) ? kSlots * (int)sizeof(T)
                                                                   : kBlock * VW * (int)sizeof(A);
}

template <typename T, typename A, typename P, int VW, bool NT>
__global__ __launch_bounds__(kBlock) void spmm_rowblock_kernel(
    const T* __restrict__ vals, const int* __restrict__ cols, const P* __restrict__ rowptr,
    P nnz_total, const T* __restrict__ B, int64_t ldb, int N, T* __restrict__ C, int64_t ldc,
    const i32x4* __restrict__ desc, int n_desc, P chunk, int lg, A* __restrict__ partials,
    int xcd_remap) {
  __shared__ int s_col[kSlots];
  __shared__ __attribute__((aligned(16))) unsigned char s_raw[spmm_scratch_bytes<T, A, VW>()];
  __shared__ P s_ptr[kBlock + 1];
  T* s_val = reinterpret_cast<T*>(s_raw);
  A* s_red = reinterpret_cast<A*>(s_raw);  // reused after the entries are consumed

  const int tid = threadIdx.x;
  int b = blockIdx.x;
  if (xcd_remap) b = xcd_logical_block(b, n_desc);
  const int tile = blockIdx.y;
  const int G = 1 << lg, ngrp = kBlock >> lg;
  const int grp = tid >> lg, lane = tid & (G - 1);
  const int W = G * VW;
  const int ncol = tile * W + lane * VW;
  const bool col_ok = ncol < N;  // VW > 1 implies N % VW == 0: the whole vector is in range
  const i32x4 d = desc[b];

  P lo, hi;
  int R = 0;
  if (d.z == 0) {
    R = d.y - d.x;
    if (R <= 0 || R > ngrp) return;  // not a planner descriptor; uniform per block
    for (int i = tid; i <= R; i += kBlock) s_ptr[i] = rowptr[d.x + i];
    __syncthreads();
    lo = s_ptr[0];
    hi = s_ptr[R];
  } else {
    const P rs = rowptr[d.x], re = rowptr[d.x + 1];
    lo = rs + P(d.y) * chunk;
    hi = (lo + chunk < re) ? lo + chunk : re;
  }
  if (hi - lo > P(kSpmmNnzCap)) return;  // uniform per block

  // Stage the (col, val) entries [lo, hi) into LDS with 16-byte loads.
  {
    const P s0 = lo & ~P(3);
    T v[kStageUPT][4];
    int c[kStageUPT][4];
#pragma unroll
    for (int u = 0; u < kStageUPT; ++u) {
      const P base = s0 + P(4) * (tid + u * kBlock);
      if (base < hi) {
        QuadLoader<NT, T>::load(vals, cols, base, lo, hi, nnz_total, v[u], c[u]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) { v[u][j] = T(0); c[u][j] = -1; }
      }
    }
#pragma unroll
    for (int u = 0; u < kStageUPT; ++u) {
      const P base = s0 + P(4) * (tid + u * kBlock);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (c[u][j] >= 0) {
          const int o = (int)(base + j - lo);
          s_col[o] = c[u][j];
          s_val[o] = v[u][j];
        }
    }
  }
  __syncthreads();

  A acc[VW];
#pragma unroll
  for (int j = 0; j < VW; ++j) acc[j] = A(0);

  if (d.z == 0) {
    // ---------------- short rows: group grp owns row d.x + grp ----------------
    if (grp < R && col_ok) {
      const int a = (int)(s_ptr[grp] - lo), e = (int)(s_ptr[grp + 1] - lo);
      const T* Bc = B + ncol;
      int i = a;
      for (; i + kRowsInFlight <= e; i += kRowsInFlight) {
        T bv[kRowsInFlight][VW];
#pragma unroll
        for (int q = 0; q < kRowsInFlight; ++q)
          load_vec<T, VW>(Bc + (int64_t)s_col[i + q] * ldb, bv[q]);
#pragma unroll
        for (int q = 0; q < kRowsInFlight; ++q) {
          const A av = A(s_val[i + q]);
#pragma unroll
          for (int j = 0; j < VW; ++j) acc[j] += av * A(bv[q][j]);
        }
      }
      for (; i < e; ++i) {
        T bv[VW];
        load_vec<T, VW>(Bc + (int64_t)s_col[i] * ldb, bv);
        const A av = A(s_val[i]);
#pragma unroll
        for (int j = 0; j < VW; ++j) acc[j] += av * A(bv[j]);
      }
      store_vec<T, A, VW>(C + (int64_t)(d.x + grp) * ldc + ncol, acc);
    }
    return;
  }

  // ---------------- one part of a long row ----------------
  const int row = d.x, k = d.y, nch = d.z, part = d.w;
  const int len = (int)(hi - lo);
  if (col_ok) {
    const T* Bc = B + ncol;
    int i = grp;
    for (; i + 3 * ngrp < len; i += 4 * ngrp) {
      T bv[4][VW];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        load_vec<T, VW>(Bc + (int64_t)s_col[i + q * ngrp] * ldb, bv[q]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const A av = A(s_val[i + q * ngrp]);
#pragma unroll
        for (int j = 0; j < VW; ++j) acc[j] += av * A(bv[q][j]);
      }
    }
    for (; i < len; i += ngrp) {
      T bv[VW];
      load_vec<T, VW>(Bc + (int64_t)s_col[i] * ldb, bv);
      const A av = A(s_val[i]);
#pragma unroll
      for (int j = 0; j < VW; ++j) acc[j] += av * A(bv[j]);
    }
  }
  __syncthreads();  // every group is done with s_val before s_red (same bytes) is written
#pragma unroll
  for (int j = 0; j < VW; ++j) s_red[grp * W + lane * VW + j] = acc[j];
  __syncthreads();
  const int col = tile * W + tid;
  const bool mine = tid < W && col < N;
  A sum = A(0);
  if (mine)
    for (int g = 0; g < ngrp; ++g) sum += s_red[g * W + tid];

  if (!mine) return;
  if (nch == 1) C[(int64_t)row * ldc + col] = T(sum);
  else partials[(int64_t)(part + k) * N + col] = sum;
}

// Second pass for rows cut into parts: C[row, :] = sum over k < nch of the part sums, k in
// increasing order.  One workgroup per split row (group {g, 1, nch, 0}, first part
// group_base[g]); a separate launch, so the first pass needs no device-scope fence.
template <typename T, typename A>
__global__ __launch_bounds__(kBlock) void spmm_split_combine_kernel(
    const i32x4* __restrict__ groups, const int64_t* __restrict__ group_base,
    const int* __restrict__ split_rows, const A* __restrict__ partials, int N,
    T* __restrict__ C, int64_t ldc) {
  const i32x4 g = groups[blockIdx.x];
  const int nch = g.z;
  const int64_t part = group_base[blockIdx.x];
  const int row = split_rows[g.x];
  for (int col = threadIdx.x; col < N; col += kBlock) {
    A acc = A(0);
    for (int k = 0; k < nch; ++k) acc += partials[(part + k) * N + col];
    C[(int64_t)row * ldc + col] = T(acc);
  }
}

// COO SpMM with atomics (the reference's "atomic" route, spmm_coo.py:244-271, 464-523):
// C_acc[rows[e], n] += vals[e] * B[cols[e], n] for every entry e and column n < N, in the
// accumulation type A (fp64 for fp32 inputs, as the reference's canonical fp64 compute).
// Thread i of the flattened (entry, column) range handles entry i / N, column i % N, so the
// lanes of a wave walk one B row and one C row contiguously.  The order of the additions, and
// so the last bits of C_acc, are not deterministic (as in the reference).
template <typename T, typename A>
__global__ __launch_bounds__(kBlock) void spmm_coo_atomic_kernel(
    const T* __restrict__ vals, const int* __restrict__ rows, const int* __restrict__ cols,
    int64_t total, int N, const T* __restrict__ B, int64_t ldb, A* __restrict__ C,
    int64_t ldc) {
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < total; i += stride) {
    const int64_t e = i / N;
    const int n = (int)(i - e * N);
    const A prod = A(vals[e]) * A(B[(int64_t)cols[e] * ldb + n]);
    atomicAdd(&C[(int64_t)rows[e] * ldc + n], prod);
  }
}

template <typename T, typename A, typename P, int VW>
int launch_spmm(const void* vals, const int32_t* cols, const void* rowptr, int64_t nnz,
                const void* B, int64_t ldb, int64_t N, void* C, int64_t ldc, const int32_t* desc,
                int64_t n_desc, int64_t chunk, int lg, void* partials, const SplitGroups& sg,
                int64_t n_tiles, int xcd_remap, hipStream_t st) {
  hipLaunchKernelGGL((spmm_rowblock_kernel<T, A, P, VW, true>),
                     dim3((unsigned)n_desc, (unsigned)n_tiles), dim3(kBlock), 0, st,
                     static_cast<const T*>(vals), cols, static_cast<const P*>(rowptr), (P)nnz,
                     static_cast<const T*>(B), ldb, (int)N, static_cast<T*>(C), ldc,
                     reinterpret_cast<const i32x4*>(desc), (int)n_desc, (P)chunk, lg,
                     static_cast<A*>(partials), xcd_remap);
  int rc = check_hip(hipGetLastError(), "spmm_rowblock_kernel launch");
  if (rc || sg.n == 0) return rc;
  hipLaunchKernelGGL((spmm_split_combine_kernel<T, A>), dim3((unsigned)sg.n), dim3(kBlock), 0, st,
                     reinterpret_cast<const i32x4*>(sg.groups), sg.base, sg.rows,
                     static_cast<const A*>(partials), (int)N, static_cast<T*>(C), ldc);
  return check_hip(hipGetLastError(), "spmm_split_combine_kernel launch");
}

template <typename T, typename A, typename P>
int dispatch_vec(int vec, const void* vals, const int32_t* cols, const void* rowptr, int64_t nnz,
                 const void* B, int64_t ldb, int64_t N, void* C, int64_t ldc,
                 const int32_t* desc, int64_t n_desc, int64_t chunk, int lg, void* partials,
                 const SplitGroups& sg, int64_t n_tiles, int xcd_remap, hipStream_t st) {
  if constexpr (sizeof(T) == 4) {
    if (vec == 4)
      return launch_spmm<T, A, P, 4>(vals, cols, rowptr, nnz, B, ldb, N, C, ldc, desc, n_desc,
                                     chunk, lg, partials, sg, n_tiles, xcd_remap, st);
  }
  if (vec == 2)
    return launch_spmm<T, A, P, 2>(vals, cols, rowptr, nnz, B, ldb, N, C, ldc, desc, n_desc,
                                   chunk, lg, partials, sg, n_tiles, xcd_remap, st);
  return launch_spmm<T, A, P, 1>(vals, cols, rowptr, nnz, B, ldb, N, C, ldc, desc, n_desc, chunk,
                                 lg, partials, sg, n_tiles, xcd_remap, st);
}

template <typename T, typename A>
int dispatch_ptr(int rowptr_bits, int vec, const void* vals, const int32_t* cols,
                 const void* rowptr, int64_t nnz, const void* B, int64_t ldb, int64_t N, void* C,
                 int64_t ldc, const int32_t* desc, int64_t n_desc, int64_t chunk, int lg,
                 void* partials, const SplitGroups& sg, int64_t n_tiles, int xcd_remap,
                 hipStream_t st) {
  if (rowptr_bits == 32)
    return dispatch_vec<T, A, int>(vec, vals, cols, rowptr, nnz, B, ldb, N, C, ldc, desc, n_desc,
                                   chunk, lg, partials, sg, n_tiles, xcd_remap, st);
  return dispatch_vec<T, A, int64_t>(vec, vals, cols, rowptr, nnz, B, ldb, N, C, ldc, desc,
                                     n_desc, chunk, lg, partials, sg, n_tiles, xcd_remap, st);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace fsp

using namespace fsp;

extern "C" int fsp_spmm_csr(int dtype, int acc_f64, const void* vals, const int32_t* cols,
                            const void* rowptr, int rowptr_bits, int64_t n_rows, int64_t nnz,
                            const void* B, int64_t ldb, int64_t N, void* C, int64_t ldc,
                            const int32_t* desc, int64_t n_desc, int64_t chunk, int lanes_per_row,
                            int vec, void* partials, const int32_t* groups,
                            const int64_t* group_base, const int32_t* split_rows,
                            int64_t n_groups, int xcd_remap, void* stream) {
  if (dtype != FSP_F32 && dtype != FSP_F64) return set_error(FSP_ENOTSUP, "fsp_spmm_csr: dtype");
  if (rowptr_bits != 32 && rowptr_bits != 64)
    return set_error(FSP_EINVAL, "fsp_spmm_csr: rowptr_bits must be 32 or 64");
  if (n_rows < 0 || nnz < 0 || N < 0 || n_desc < 0 || n_groups < 0)
    return set_error(FSP_EINVAL, "fsp_spmm_csr: negative size");
  if (n_groups > 0x7fffffffLL) return set_error(FSP_EINVAL, "fsp_spmm_csr: too many groups");
  if (n_groups > 0 && (!groups || !group_base || !split_rows || !partials))
    return set_error(FSP_EINVAL, "fsp_spmm_csr: null split-row pointer");
  if (n_desc > 0x7fffffffLL || n_rows > 0x7fffffffLL || N > 0x7fffffffLL)
    return set_error(FSP_EINVAL, "fsp_spmm_csr: size exceeds 2^31-1");
  if (rowptr_bits == 32 && nnz > 0x7fffffffLL)
    return set_error(FSP_EINVAL, "fsp_spmm_csr: nnz exceeds int32 rowptr range");
  int lg = -1;
  for (int g = 0; g <= 6; ++g)
    if (lanes_per_row == (1 << g)) lg = g;
  if (lg < 0) return set_error(FSP_EINVAL, "fsp_spmm_csr: lanes_per_row must be 1,2,4,...,64");
  const int max_vec = (dtype == FSP_F32) ? 4 : 2;
  if (vec != 1 && vec != 2 && vec != max_vec)
    return set_error(FSP_EINVAL, "fsp_spmm_csr: vec must be 1, 2 or 4 (fp32) / 1, 2 (fp64)");
  if (chunk < 1 || chunk > kSpmmNnzCap)
    return set_error(FSP_EINVAL, "fsp_spmm_csr: chunk outside [1, fsp_spmm_block_nnz_cap()]");
  if (N == 0 || n_desc == 0) return FSP_OK;
  if (vec > 1 && (N % vec || ldb % vec || ldc % vec || !aligned16(B) || !aligned16(C)))
    return set_error(FSP_EINVAL, "fsp_spmm_csr: vec > 1 needs N, ldb, ldc multiples of vec and "
                                 "16-byte aligned B, C");
  if (ldb < N || ldc < N) return set_error(FSP_EINVAL, "fsp_spmm_csr: ldb/ldc smaller than N");
  if (!rowptr || !C || !desc) return set_error(FSP_EINVAL, "fsp_spmm_csr: null pointer");
  if (nnz > 0 && (!vals || !cols || !B)) return set_error(FSP_EINVAL, "fsp_spmm_csr: null pointer");
  if (!aligned16(vals) || !aligned16(cols) || !aligned16(desc))
    return set_error(FSP_EINVAL, "fsp_spmm_csr: vals, cols and desc must be 16-byte aligned");
  const int64_t W = (int64_t)lanes_per_row * vec;
  const int64_t n_tiles = (N + W - 1) / W;
  if (n_tiles > 65535) return set_error(FSP_EINVAL, "fsp_spmm_csr: too many column tiles");
  if (!aligned16(groups)) return set_error(FSP_EINVAL, "fsp_spmm_csr: groups must be 16-byte aligned");
  const SplitGroups sg{groups, group_base, split_rows, n_groups};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == FSP_F32) {
    if (acc_f64)
      return dispatch_ptr<float, double>(rowptr_bits, vec, vals, cols, rowptr, nnz, B, ldb, N, C,
                                         ldc, desc, n_desc, chunk, lg, partials, sg, n_tiles,
                                         xcd_remap, st);
    return dispatch_ptr<float, float>(rowptr_bits, vec, vals, cols, rowptr, nnz, B, ldb, N, C, ldc,
                                      desc, n_desc, chunk, lg, partials, sg, n_tiles,
                                      xcd_remap, st);
  }
  return dispatch_ptr<double, double>(rowptr_bits, vec, vals, cols, rowptr, nnz, B, ldb, N, C,
                                      ldc, desc, n_desc, chunk, lg, partials, sg, n_tiles,
                                      xcd_remap, st);
}

extern "C" int fsp_spmm_coo_atomic(int dtype, int acc_f64, const void* vals, const int32_t* rows,
                                   const int32_t* cols, int64_t nnz, const void* B, int64_t ldb,
                                   int64_t N, void* C_acc, int64_t ldc, int64_t n_rows,
                                   void* stream) {
  if (dtype != FSP_F32 && dtype != FSP_F64)
    return set_error(FSP_ENOTSUP, "fsp_spmm_coo_atomic: dtype");
  if (nnz < 0 || N < 0 || n_rows < 0) return set_error(FSP_EINVAL, "fsp_spmm_coo_atomic: negative size");
  if (N > 0x7fffffffLL || nnz > 0x7fffffffLL)
    return set_error(FSP_EINVAL, "fsp_spmm_coo_atomic: size exceeds 2^31-1");
  if (ldc < N || ldb < N) return set_error(FSP_EINVAL, "fsp_spmm_coo_atomic: ldb/ldc smaller than N");
  if (n_rows > 0 && ldc > 0 && !C_acc) return set_error(FSP_EINVAL, "fsp_spmm_coo_atomic: null C");
  if (nnz > 0 && N > 0 && (!vals || !rows || !cols || !B))
    return set_error(FSP_EINVAL, "fsp_spmm_coo_atomic: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool wide = dtype == FSP_F64 || acc_f64;
  // C_acc[0 .. n_rows*ldc) = 0, then the atomic pass.
  int rc = wide ? fill_zero<double>(static_cast<double*>(C_acc), n_rows * ldc, st)
                : fill_zero<float>(static_cast<float*>(C_acc), n_rows * ldc, st);
  if (rc) return rc;
  const int64_t total = nnz * N;
  if (total == 0) return FSP_OK;
  int64_t blocks = (total + kBlock - 1) / kBlock;
  if (blocks > 65536) blocks = 65536;  // grid-stride loop covers the rest
  if (dtype == FSP_F32 && acc_f64)
    hipLaunchKernelGGL((spmm_coo_atomic_kernel<float, double>), dim3((unsigned)blocks),
                       dim3(kBlock), 0, st, static_cast<const float*>(vals), rows, cols, total,
                       (int)N, static_cast<const float*>(B), ldb, static_cast<double*>(C_acc), ldc);
  else if (dtype == FSP_F32)
    hipLaunchKernelGGL((spmm_coo_atomic_kernel<float, float>), dim3((unsigned)blocks),
                       dim3(kBlock), 0, st, static_cast<const float*>(vals), rows, cols, total,
                       (int)N, static_cast<const float*>(B), ldb, static_cast<float*>(C_acc), ldc);
  else
    hipLaunchKernelGGL((spmm_coo_atomic_kernel<double, double>), dim3((unsigned)blocks),
                       dim3(kBlock), 0, st, static_cast<const double*>(vals), rows, cols, total,
                       (int)N, static_cast<const double*>(B), ldb, static_cast<double*>(C_acc),
                       ldc);
  return check_hip(hipGetLastError(), "spmm_coo_atomic_kernel launch");
}
