// CSR / COO-run SpMV for gfx950: one fused launch over a row-block descriptor table.
//
// Reference behaviour followed (src/flagsparse/sparse_operations/):
//   spmv_csr.py:94-120    base kernel: y[row] = sum over the row's nnz, fp32 summed in fp64
//                         (spmv_csr.py:498-536 casts to fp64 and back)
//   spmv_csr.py:161-279   opt kernels: native-precision accumulation (use_opt=True)
//   spmv_coo.py:51-108    row-run kernel: one output row per run, rows without a run are 0
//   spmv_coo.py:111-150   atomic kernel for unsorted COO
//
// Work decomposition (MI355X-first, not the reference's bucket launches):
//   * short-row block  {r0, r1, 0, 0}: the block's contiguous nnz range (<= 1021 entries) is
//     read with 16-byte loads, one quad of entries per thread and step; products go to LDS;
//     then each row is summed by a group of G lanes (G = 256 / next_pow2(rows), <= 64) with a
//     butterfly shuffle reduction.
//   * long-row chunk   {row, k, nch, part}: 256 threads sum <= 4093 entries of one row in
//     registers, reduce across the workgroup; with nch > 1 the chunk sum goes to
//     partials[part + k] and a second launch (split_row_combine_kernel) adds
//     partials[part .. part+nch) in index order, so the result does not depend on timing.
#include <atomic>
#include <mutex>
#include <string>

#include "fsp_device.hpp"
#include "fsp_internal.hpp"

namespace fsp {
namespace {

constexpr int kStreamSlots = (int)kSpmvStreamSlots;
constexpr int kStreamRows = (int)kSpmvStreamRowsCap;
constexpr int kStreamUPT = kStreamSlots / (4 * kBlock);  // quads per thread in a short-row block
constexpr int kChunkUPT = (int)kSpmvChunkUnitsPerThread;
static_assert(kStreamUPT * 4 * kBlock == kStreamSlots, "stream slots must be whole quads per thread");

// x[c] for the entries a thread holds (c >= 0), 0 for the empty positions (c < 0), with all
// of a thread's gathers in flight together.  When the value is widened to the accumulator
// type (fp32 x summed in fp64), a load under a per-lane condition became an exec-masked region
// with the conversion inside, and the compiler waited for each gather before issuing the next;
// those gathers are therefore issued for every position - an empty one reads x[0], which
// exists whenever the descriptor has an entry (any), the only case in which it runs - and the
// value dropped afterwards.  Without a conversion the conditional form keeps its loads
// together and needs fewer registers (fp64 row blocks: 72 against 84 VGPRs, 7 against 5 waves
// per SIMD).
template <int U, typename A, typename T>
__device__ __forceinline__ void gather_x(const T* __restrict__ x, const int (&c)[U][4], bool any,
                                         T (&xv)[U][4]) {
  if constexpr (sizeof(A) == sizeof(T)) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) xv[u][j] = c[u][j] >= 0 ? x[c[u][j]] : T(0);
  } else {
    if (!any) {  // uniform per workgroup
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int j = 0; j < 4; ++j) xv[u][j] = T(0);
      return;
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) xv[u][j] = x[c[u][j] >= 0 ? c[u][j] : 0];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (c[u][j] < 0) xv[u][j] = T(0);
  }
}

template <typename T, typename A, typename P, bool NT>
__global__ __launch_bounds__(kBlock) void spmv_rowblock_kernel(
    const T* __restrict__ vals, const int* __restrict__ cols, const P* __restrict__ rowptr,
    P nnz_total, const T* __restrict__ x, T* __restrict__ y, const int* __restrict__ row_map,
    const i32x4* __restrict__ desc, const int64_t* __restrict__ ranges, int n_desc, P chunk,
    A* __restrict__ partials, int64_t partials_cap, int xcd_remap) {
  __shared__ A s_prod[kStreamSlots];
  __shared__ P s_ptr[kStreamRows + 1];
  __shared__ A s_red[kWavesPerBlock];

  const int tid = threadIdx.x;
  int b = blockIdx.x;
  if (xcd_remap) b = xcd_logical_block(b, n_desc);
  const i32x4 d = desc[b];
  // The descriptor's entry range [lo, hi) comes from the plan, so the entry loads do not
  // wait for the row pointers.
  const P lo = (P)ranges[2 * b], hi = (P)ranges[2 * b + 1];

  if (d.z == 0) {
    // ---------------- short-row block: rows [r0, r0 + R) ----------------
    const int r0 = d.x, R = d.y - d.x;
    if (R <= 0 || R > kStreamRows || hi - lo > P(kSpmvStreamNnzCap) || hi < lo)
      return;  // not a planner descriptor; uniform per block
    const P s0 = lo & ~P(3);

    T v[kStreamUPT][4];
    int c[kStreamUPT][4];
#pragma unroll
    for (int u = 0; u < kStreamUPT; ++u) {
      const P base = s0 + P(4) * (tid + u * kBlock);
      if (base < hi) {
        QuadLoader<NT, T>::load(vals, cols, base, lo, hi, nnz_total, v[u], c[u]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) { v[u][j] = T(0); c[u][j] = -1; }
      }
    }
    constexpr int kPtrPT = (kStreamRows + kBlock) / kBlock;  // row pointers per thread
    P rp[kPtrPT];
#pragma unroll
    for (int u = 0; u < kPtrPT; ++u) {
      const int i = tid + u * kBlock;
      rp[u] = i <= R ? rowptr[r0 + i] : P(0);
    }
    T xv[kStreamUPT][4];
    gather_x<kStreamUPT, A>(x, c, hi > lo, xv);
#pragma unroll
    for (int u = 0; u < kStreamUPT; ++u) {
      const P base = s0 + P(4) * (tid + u * kBlock);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (c[u][j] >= 0) s_prod[(int)(base + j - lo)] = A(v[u][j]) * A(xv[u][j]);
    }
#pragma unroll
    for (int u = 0; u < kPtrPT; ++u) {
      const int i = tid + u * kBlock;
      if (i <= R) s_ptr[i] = rp[u];
    }
    __syncthreads();

    // Lanes per row: the largest power of two G <= 64 with G * next_pow2(R) <= 256.
    int lg = 0;
    if (R < kBlock) {
      int p2 = 1, lp = 0;
      while (p2 < R) { p2 <<= 1; ++lp; }
      lg = 8 - lp;  // log2(256 / p2)
      if (lg > 6) lg = 6;
    }
    const int G = 1 << lg;
    const int ngrp = kBlock >> lg;
    const int grp = tid >> lg, lane = tid & (G - 1);
    // With G > 1, ngrp >= R, so each group runs at most one iteration and its lanes stay
    // converged for the shuffles.
    for (int r = grp; r < R; r += ngrp) {
      const int a = (int)(s_ptr[r] - lo), e = (int)(s_ptr[r + 1] - lo);
      A acc = A(0);
      for (int i = a + lane; i < e; i += G) acc += s_prod[i];
      if (G > 1) acc = group_sum(acc, G);
      if (lane == 0) {
        const int row = r0 + r;
        y[row_map ? row_map[row] : row] = T(acc);
      }
    }
    return;
  }

  // ---------------- long-row chunk ----------------
  const int row = d.x, k = d.y, nch = d.z, part = d.w;
  if (hi - lo > chunk || hi < lo) return;  // not a planner descriptor; uniform per block
  const P s0 = lo & ~P(3);

  T v[kChunkUPT][4];
  int c[kChunkUPT][4];
#pragma unroll
  for (int u = 0; u < kChunkUPT; ++u) {
    const P base = s0 + P(4) * (tid + u * kBlock);
    if (base < hi) {
      QuadLoader<NT, T>::load(vals, cols, base, lo, hi, nnz_total, v[u], c[u]);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) { v[u][j] = T(0); c[u][j] = -1; }
    }
  }
  T xv[kChunkUPT][4];
  gather_x<kChunkUPT, A>(x, c, hi > lo, xv);
  A acc = A(0);
#pragma unroll
  for (int u = 0; u < kChunkUPT; ++u)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc += A(v[u][j]) * A(xv[u][j]);

  const A total = block_sum(acc, s_red);
  if (tid == 0) {
    if (nch == 1) y[row_map ? row_map[row] : row] = T(total);
    else if ((int64_t)part + k < partials_cap) partials[part + k] = total;
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void spmv_coo_atomic_kernel(
    const T* __restrict__ vals, const int* __restrict__ rows, const int* __restrict__ cols,
    int64_t nnz, const T* __restrict__ x, T* __restrict__ y, int64_t per_block) {
  const int64_t begin = (int64_t)blockIdx.x * per_block;
  int64_t end = begin + per_block;
  if (end > nnz) end = nnz;
  for (int64_t i = begin + threadIdx.x; i < end; i += kBlock)
    atomicAdd(&y[rows[i]], vals[i] * x[cols[i]]);
}

template <typename T, typename A, typename P>
int launch_spmv(const void* vals, const int32_t* cols, const void* rowptr, int64_t nnz,
                const void* x, void* y, const int32_t* row_map, int64_t n_out,
                const int32_t* desc, const int64_t* ranges, int64_t n_desc, int64_t chunk,
                void* partials, int64_t partials_cap, const int32_t* groups,
                const int64_t* group_base, const int32_t* split_rows, int64_t n_groups,
                int xcd_remap, hipStream_t st) {
  if (row_map) {
    int rc = fill_zero<T>(static_cast<T*>(y), n_out, st);
    if (rc) return rc;
  }
  if (n_desc == 0) return FSP_OK;
  // Plain (temporal) loads for the entries: measured on MI355X they stream faster here than
  // non-temporal ones when the kernel also writes y (cfg2: 60.5 vs 63.9 us), and this
  // layout's x reuse is local enough not to need protection in L2.
  hipLaunchKernelGGL((spmv_rowblock_kernel<T, A, P, false>), dim3((unsigned)n_desc), dim3(kBlock),
                     0, st, static_cast<const T*>(vals), cols, static_cast<const P*>(rowptr),
                     (P)nnz, static_cast<const T*>(x), static_cast<T*>(y), row_map,
                     reinterpret_cast<const i32x4*>(desc), ranges, (int)n_desc, (P)chunk,
                     static_cast<A*>(partials), partials_cap, xcd_remap);
  int rc = check_hip(hipGetLastError(), "spmv_rowblock_kernel launch");
  if (rc || n_groups == 0) return rc;
  hipLaunchKernelGGL((split_row_combine_kernel<T, A>), dim3((unsigned)n_groups), dim3(kBlock), 0,
                     st, reinterpret_cast<const i32x4*>(groups), group_base, split_rows,
                     static_cast<A*>(partials), partials_cap, static_cast<T*>(y), row_map, 0);
  return check_hip(hipGetLastError(), "split_row_combine_kernel launch");
}

template <typename T, typename A>
int dispatch_ptr(int rowptr_bits, const void* vals, const int32_t* cols, const void* rowptr,
                 int64_t nnz, const void* x, void* y, const int32_t* row_map, int64_t n_out,
                 const int32_t* desc, const int64_t* ranges, int64_t n_desc, int64_t chunk,
                 void* partials, int64_t partials_cap, const int32_t* groups,
                 const int64_t* group_base, const int32_t* split_rows, int64_t n_groups,
                 int xcd_remap, hipStream_t st) {
  if (rowptr_bits == 32)
    return launch_spmv<T, A, int>(vals, cols, rowptr, nnz, x, y, row_map, n_out, desc, ranges,
                                  n_desc, chunk, partials, partials_cap, groups, group_base,
                                  split_rows, n_groups, xcd_remap, st);
  return launch_spmv<T, A, int64_t>(vals, cols, rowptr, nnz, x, y, row_map, n_out, desc, ranges,
                                    n_desc, chunk, partials, partials_cap, groups, group_base,
                                    split_rows, n_groups, xcd_remap, st);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <typename T>
__global__ __launch_bounds__(kBlock) void fill_zero_kernel(T* __restrict__ y, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) y[i] = T(0);
}

template <typename T>
int launch_fill(T* y, int64_t n, hipStream_t st) {
  if (n <= 0) return FSP_OK;
  int64_t blocks = (n + kBlock - 1) / kBlock;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(fill_zero_kernel<T>, dim3((unsigned)blocks), dim3(kBlock), 0, st, y, n);
  return check_hip(hipGetLastError(), "fill_zero_kernel launch");
}

}  // namespace

int fill_zero_f32(float* y, int64_t n, hipStream_t st) { return launch_fill<float>(y, n, st); }
int fill_zero_f64(double* y, int64_t n, hipStream_t st) { return launch_fill<double>(y, n, st); }

}  // namespace fsp

using namespace fsp;

namespace {

// The checks and launches of fsp_spmv_csr; partials holds partials_cap slots (INT64_MAX when
// the caller sized it; the kernels then never compare).
int spmv_csr_checked(const char* who, int dtype, int acc_f64, const void* vals,
                     const int32_t* cols, const void* rowptr, int rowptr_bits, int64_t n_rows,
                     int64_t nnz, const void* x, void* y, const int32_t* row_map, int64_t n_out,
                     const int32_t* desc, const int64_t* ranges, int64_t n_desc, int64_t chunk,
                     void* partials, int64_t partials_cap, const int32_t* groups,
                     const int64_t* group_base, const int32_t* split_rows, int64_t n_groups,
                     int xcd_remap, void* stream) {
  const std::string w(who);
  if (dtype != FSP_F32 && dtype != FSP_F64) return set_error(FSP_ENOTSUP, w + ": dtype");
  if (rowptr_bits != 32 && rowptr_bits != 64)
    return set_error(FSP_EINVAL, w + ": rowptr_bits must be 32 or 64");
  if (n_rows < 0 || nnz < 0 || n_desc < 0 || n_out < 0 || n_groups < 0)
    return set_error(FSP_EINVAL, w + ": negative size");
  if (n_desc > 0x7fffffffLL || n_rows > 0x7fffffffLL || n_groups > 0x7fffffffLL)
    return set_error(FSP_EINVAL, w + ": more than 2^31-1 rows, descriptors or groups");
  if (rowptr_bits == 32 && nnz > 0x7fffffffLL)
    return set_error(FSP_EINVAL, w + ": nnz exceeds int32 rowptr range");
  if (chunk < 1 || chunk > kSpmvChunkCap)
    return set_error(FSP_EINVAL, w + ": chunk outside [1, fsp_spmv_chunk_nnz_cap()]");
  if (n_desc > 0 && (!rowptr || !y || !desc || !ranges))
    return set_error(FSP_EINVAL, w + ": null pointer");
  if (nnz > 0 && (!vals || !cols || !x)) return set_error(FSP_EINVAL, w + ": null pointer");
  if (n_groups > 0 && (!groups || !group_base || !split_rows || !partials))
    return set_error(FSP_EINVAL, w + ": null split-row pointer");
  if (!aligned16(vals) || !aligned16(cols) || !aligned16(desc) || !aligned16(groups))
    return set_error(FSP_EINVAL, w + ": vals, cols, desc and groups must be 16-byte aligned");
  if (row_map && !y) return set_error(FSP_EINVAL, w + ": null y");
  hipStream_t st = static_cast<hipStream_t>(stream);
#define FSP_SPMV_ARGS rowptr_bits, vals, cols, rowptr, nnz, x, y, row_map, n_out, desc, ranges, \
                      n_desc, chunk, partials, partials_cap, groups, group_base, split_rows, \
                      n_groups, xcd_remap, st
  if (dtype == FSP_F32) {
    if (acc_f64) return dispatch_ptr<float, double>(FSP_SPMV_ARGS);
    return dispatch_ptr<float, float>(FSP_SPMV_ARGS);
  }
  return dispatch_ptr<double, double>(FSP_SPMV_ARGS);
#undef FSP_SPMV_ARGS
}

// The partial-sum workspace of fsp_spmv_csr_static: one array per GPU for the life of the
// process.  Its name is a host-side handle only; kernels get the device address that
// hipGetSymbolAddress returns for the current device, resolved once per device.
constexpr int64_t kSpmvScratchSlots = 1 << 17;  // 8-byte slots: 1 MiB per GPU
__device__ __align__(256) double scratch[kSpmvScratchSlots];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mutex;

int scratch_for_current_device(void** out) {
  int dev = -1;
  int rc = check_hip(hipGetDevice(&dev), "fsp_spmv_csr_static: hipGetDevice");
  if (rc) return rc;
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(FSP_EINVAL, "fsp_spmv_csr_static: device index beyond " +
                                     std::to_string(kMaxDevices));
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      rc = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                     "fsp_spmv_csr_static: hipGetSymbolAddress");
      if (rc) return rc;
      if (!p) return set_error(FSP_EHIP, "fsp_spmv_csr_static: null scratch address");
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return FSP_OK;
}

}  // namespace

extern "C" int fsp_spmv_csr(int dtype, int acc_f64, const void* vals, const int32_t* cols,
                            const void* rowptr, int rowptr_bits, int64_t n_rows, int64_t nnz,
                            const void* x, void* y, const int32_t* row_map, int64_t n_out,
                            const int32_t* desc, const int64_t* ranges, int64_t n_desc,
                            int64_t chunk, void* partials, const int32_t* groups,
                            const int64_t* group_base, const int32_t* split_rows,
                            int64_t n_groups, int xcd_remap, void* stream) {
  return spmv_csr_checked("fsp_spmv_csr", dtype, acc_f64, vals, cols, rowptr, rowptr_bits, n_rows,
                          nnz, x, y, row_map, n_out, desc, ranges, n_desc, chunk, partials,
                          INT64_MAX, groups, group_base, split_rows, n_groups, xcd_remap,
                          stream);
}

extern "C" int64_t fsp_spmv_scratch_slots(void) { return kSpmvScratchSlots; }

extern "C" int fsp_spmv_csr_static(int dtype, int acc_f64, const void* vals,
                                   const int32_t* cols, const void* rowptr, int rowptr_bits,
                                   int64_t n_rows, int64_t nnz, const void* x, void* y,
                                   const int32_t* row_map, int64_t n_out, const int32_t* desc,
                                   const int64_t* ranges, int64_t n_desc, int64_t chunk,
                                   int64_t n_parts, const int32_t* groups,
                                   const int64_t* group_base, const int32_t* split_rows,
                                   int64_t n_groups, int xcd_remap, void* stream) {
  if (n_parts < 0 || n_parts > kSpmvScratchSlots)
    return set_error(FSP_EINVAL, "fsp_spmv_csr_static: the plan needs " + std::to_string(n_parts) +
                                     " partial slots; the static workspace holds " +
                                     std::to_string(kSpmvScratchSlots) +
                                     " (use fsp_spmv_csr with a workspace of that size)");
  void* ptr = nullptr;
  int rc = scratch_for_current_device(&ptr);
  if (rc) return rc;
  return spmv_csr_checked("fsp_spmv_csr_static", dtype, acc_f64, vals, cols, rowptr, rowptr_bits,
                          n_rows, nnz, x, y, row_map, n_out, desc, ranges, n_desc, chunk, ptr,
                          kSpmvScratchSlots, groups, group_base, split_rows, n_groups, xcd_remap,
                          stream);
}

extern "C" int fsp_spmv_coo_atomic(int dtype, const void* vals, const int32_t* rows,
                                   const int32_t* cols, int64_t nnz, const void* x, void* y,
                                   int64_t n_rows, int64_t nnz_per_block, void* stream) {
  if (dtype != FSP_F32 && dtype != FSP_F64)
    return set_error(FSP_ENOTSUP, "fsp_spmv_coo_atomic: dtype");
  if (nnz < 0 || n_rows < 0 || nnz_per_block < 1)
    return set_error(FSP_EINVAL, "fsp_spmv_coo_atomic: bad size");
  if (n_rows > 0 && !y) return set_error(FSP_EINVAL, "fsp_spmv_coo_atomic: null y");
  if (nnz > 0 && (!vals || !rows || !cols || !x))
    return set_error(FSP_EINVAL, "fsp_spmv_coo_atomic: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t blocks = (nnz + nnz_per_block - 1) / nnz_per_block;
  if (blocks > 0x7fffffffLL) return set_error(FSP_EINVAL, "fsp_spmv_coo_atomic: grid too large");
  if (dtype == FSP_F32) {
    int rc = fill_zero<float>(static_cast<float*>(y), n_rows, st);
    if (rc || nnz == 0) return rc;
    hipLaunchKernelGGL(spmv_coo_atomic_kernel<float>, dim3((unsigned)blocks), dim3(kBlock), 0, st,
                       static_cast<const float*>(vals), rows, cols, nnz,
                       static_cast<const float*>(x), static_cast<float*>(y), nnz_per_block);
  } else {
    int rc = fill_zero<double>(static_cast<double*>(y), n_rows, st);
    if (rc || nnz == 0) return rc;
    hipLaunchKernelGGL(spmv_coo_atomic_kernel<double>, dim3((unsigned)blocks), dim3(kBlock), 0, st,
                       static_cast<const double*>(vals), rows, cols, nnz,
                       static_cast<const double*>(x), static_cast<double*>(y), nnz_per_block);
  }
  return check_hip(hipGetLastError(), "spmv_coo_atomic_kernel launch");
}
