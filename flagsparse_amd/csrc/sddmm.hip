// CSR SDDMM for gfx950: out[p] = alpha * dot(x[row(p)], y[col(p)]) + beta * in[p] for every
// stored entry p of a CSR pattern (x [n_rows, K], y [n_cols, K], both row-major).
//
// Reference behaviour followed (src/flagsparse/sparse_operations/sddmm_csr.py):
//   :107-151  _sddmm_csr_real_kernel: one value per entry, accumulated in the input type
//             (float64 for the "acc64" diagnostic variants, :253-268), then alpha / beta
//   :271-347  launch: row ids per entry from the prepare step (:82-90)
//
// Mapping: a gather-bound contraction (one K-long dot per entry, y rows at random), so no MFMA.
// G lanes share one entry, each holding VW consecutive elements (16-byte loads for VW = 4 fp32
// / 2 fp64) of the x row and the y row, so a group covers G*VW elements of K per step.
//
// sddmm_rowblock_kernel (K <= 4*G*VW): one launch over a row-block plan.  A workgroup stages
// its entries' columns into LDS with 16-byte loads; in a short-row block each lane group owns
// one row, keeps that row of x in registers (loaded once) and walks the row's entries four at
// a time (four y rows in flight per lane); a long row is cut into chunks that all groups of a
// workgroup share.  Entries are independent, so chunks need no second pass.
// sddmm_flat_kernel (any K): a group per entry, x and y rows both loaded per entry.
// Each dot ends with a sum over the G lanes (group_sum: DPP row permutes, no LDS round trip)
// in a fixed order, so results are deterministic.
#include "fsp_device.hpp"
#include "fsp_internal.hpp"

namespace fsp {
namespace {

template <typename T, int VW> struct SVec;
template <> struct SVec<float, 4> { typedef f32x4 type; };
template <> struct SVec<float, 2> { typedef f32x2 type; };
template <> struct SVec<float, 1> { typedef float type; };
template <> struct SVec<double, 2> { typedef f64x2 type; };
template <> struct SVec<double, 1> { typedef double type; };

template <typename T, int VW>
__device__ __forceinline__ void sload(const T* p, T (&o)[VW]) {
  typedef typename SVec<T, VW>::type V;
  const V v = *reinterpret_cast<const V*>(p);
  if constexpr (VW == 1) {
    o[0] = v;
  } else {
#pragma unroll
    for (int j = 0; j < VW; ++j) o[j] = v[j];
  }
}

constexpr int kSdSlots = (int)kSpmmSlots;  // staged columns per workgroup
constexpr int kSdStageUPT = kSdSlots / (4 * kBlock);

// One row-block descriptor per workgroup (the plan of fsp_plan_windows_*: short-row blocks
// {r0, r1, 0, 0} with <= 256/G rows, chunks {row, k, nch, part} of long rows; ranges [lo, hi)).
template <typename T, typename A, typename O, typename P, int VW, int KC>
__global__ __launch_bounds__(kBlock) void sddmm_rowblock_kernel(
    const int* __restrict__ cols, const P* __restrict__ rowptr, int64_t nnz_total,
    const T* __restrict__ x, int64_t ldx, const T* __restrict__ y, int64_t ldy, int K,
    const T* __restrict__ in, double alpha, double beta, O* __restrict__ out,
    const i32x4* __restrict__ desc, const int64_t* __restrict__ ranges, int n_desc, int lg,
    int xcd_remap) {
  __shared__ int s_col[kSdSlots];
  __shared__ P s_ptr[kBlock + 1];
  // Results are collected in LDS and written out together at the end, in whole lines: written
  // straight from the groups, 16 bytes at a time, partial lines were evicted by the y gathers
  // before they filled (cfg5 pattern, K = 64: 935 -> 789 us without those stores).  A 4-byte
  // result takes the slot of the column it came from; wider ones get their own array.
  __shared__ O s_out_wide[sizeof(O) == sizeof(int) ? 1 : kSdSlots];
  O* const s_out = sizeof(O) == sizeof(int) ? reinterpret_cast<O*>(s_col) : s_out_wide;
  const int tid = threadIdx.x;
  int b = blockIdx.x;
  if (xcd_remap) b = xcd_logical_block(b, n_desc);
  const int G = 1 << lg, ngrp = kBlock >> lg;
  const int grp = tid >> lg, lane = tid & (G - 1);
  const i32x4 d = desc[b];
  const int64_t lo = ranges[2 * b], hi = ranges[2 * b + 1];
  if (hi - lo > kSpmmNnzCap || hi < lo) return;  // not a planner descriptor; uniform per block
  const int R = d.z == 0 ? d.y - d.x : 0;
  if (d.z == 0 && (R <= 0 || R > ngrp)) return;  // uniform per block
  // Stage the columns of [lo, hi) with 16-byte loads.
  {
    const int64_t s0 = lo & ~int64_t(3);
#pragma unroll
    for (int u = 0; u < kSdStageUPT; ++u) {
      const int64_t base = s0 + 4 * (int64_t)(tid + u * kBlock);
      if (base < hi) {
        int cc[4];
        if (base + 4 <= nnz_total) {
          const i32x4 v = *reinterpret_cast<const i32x4*>(cols + base);
          cc[0] = v.x; cc[1] = v.y; cc[2] = v.z; cc[3] = v.w;
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) cc[j] = base + j < nnz_total ? cols[base + j] : 0;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (base + j >= lo && base + j < hi) s_col[(int)(base + j - lo)] = cc[j];
      }
    }
  }
  for (int i = tid; i <= R; i += kBlock) s_ptr[i] = rowptr[d.x + i];
  __syncthreads();

  // This group's row and entry range (relative to lo), entries visited with stride `step`;
  // groups without a row get an empty range (no early exit: the block meets a barrier below).
  int row = d.x, a = 0, e = 0, step = 4;
  if (d.z == 0) {
    if (grp < R) {
      row = d.x + grp;
      a = (int)(s_ptr[grp] - lo);
      e = (int)(s_ptr[grp + 1] - lo);
    }
  } else {
    a = 4 * grp;
    e = (int)(hi - lo);
    step = 4 * ngrp;
  }
  // The row of x, in registers: lane holds elements lane*VW + c*G*VW (+ j) for c < KC.
  // Loaded without a per-lane condition (row is a row of the block for every group; a lane
  // past K reads element 0 and zeroes it), so the KC loads are in flight together.  K == 0
  // (x and y may then be absent) skips every load; the condition is uniform.
  const bool any_k = K > 0;
  T xr[KC][VW];
  const T* xp = x + (int64_t)row * ldx;
#pragma unroll
  for (int c = 0; c < KC; ++c) {
    const int k = (lane + c * G) * VW;
    if (any_k) {
      sload<T, VW>(xp + (k < K ? k : 0), xr[c]);
    } else {
#pragma unroll
      for (int j = 0; j < VW; ++j) xr[c][j] = T(0);
    }
  }
#pragma unroll
  for (int c = 0; c < KC; ++c)
#pragma unroll
    for (int j = 0; j < VW; ++j)
      if ((lane + c * G) * VW >= K) xr[c][j] = T(0);
  const A a_alpha = A(alpha), a_beta = A(beta);
  for (int i = a; i < e; i += step) {
    // Four entries i .. i+3 of this group (fewer at the end of the range).  All their y loads
    // are issued before the first is used: a position past the range reads entry i's row and
    // a lane past K reads element 0, and both are dropped below.  (A load under a per-lane
    // condition is an exec-masked region of its own; with the products inside it the
    // compiler waited for each load before issuing the next.)
    T yv[4][KC][VW];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const T* yp = y + (int64_t)s_col[i + q < e ? i + q : i] * ldy;
#pragma unroll
      for (int c = 0; c < KC; ++c) {
        const int k = (lane + c * G) * VW;
        if (any_k) {
          sload<T, VW>(yp + (k < K ? k : 0), yv[q][c]);
        } else {
#pragma unroll
          for (int j = 0; j < VW; ++j) yv[q][c][j] = T(0);
        }
      }
    }
    A acc[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc[q] = A(0);
#pragma unroll
      for (int c = 0; c < KC; ++c) {
        const bool use = i + q < e && (lane + c * G) * VW < K;
#pragma unroll
        for (int j = 0; j < VW; ++j) acc[q] += use ? A(xr[c][j]) * A(yv[q][c][j]) : A(0);
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] = group_sum(acc[q], G);
    // Every lane of the group holds the four sums.  With G >= 4, lanes 0..3 keep them; with
    // narrower groups lane q mod G keeps result q.  A slot's column was read above by this
    // group only, so its result may take the slot (the group's lanes run in lockstep).
    if (G >= 4) {
      if (lane < 4 && i + lane < e) {
        A v = lane == 0 ? acc[0] : lane == 1 ? acc[1] : lane == 2 ? acc[2] : acc[3];
        v *= a_alpha;
        if (in) v += A(in[lo + i + lane]) * a_beta;
        s_out[i + lane] = O(v);
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if ((q & (G - 1)) == lane && i + q < e) {
          A v = acc[q] * a_alpha;
          if (in) v += A(in[lo + i + q]) * a_beta;
          s_out[i + q] = O(v);
        }
      }
    }
  }
  __syncthreads();
  for (int i = tid; i < (int)(hi - lo); i += kBlock) out[lo + i] = s_out[i];
}

template <typename T, typename A, typename O, int VW>
__global__ __launch_bounds__(kBlock) void sddmm_flat_kernel(
    const int* __restrict__ cols, const int* __restrict__ row_ids, int64_t nnz,
    const T* __restrict__ x, int64_t ldx, const T* __restrict__ y, int64_t ldy, int K,
    const T* __restrict__ in, double alpha, double beta, O* __restrict__ out, int lg) {
  constexpr int kU = 4;  // entries per group and step: 2*kU vector loads in flight per lane
  const int G = 1 << lg;
  const int groups = kBlock >> lg;
  const int grp = threadIdx.x >> lg, lane = threadIdx.x & (G - 1);
  const A a_alpha = A(alpha), a_beta = A(beta);
  // A workgroup step covers kU * groups consecutive entries; entry u of group g is
  // base + u * groups + g, so the groups of a wave store neighbouring results together.
  // XCD k runs one contiguous range of steps (xcd_logical_block), so the y rows that
  // neighbouring rows share (banded patterns) are fetched into one L2, not eight.
  const int64_t span = (int64_t)kU * groups;
  const int64_t first = xcd_logical_block((int)blockIdx.x, (int)gridDim.x);
  for (int64_t base = first * span; base < nnz; base += (int64_t)gridDim.x * span) {
    int64_t r[kU], c[kU];
    bool ok[kU];
    // Loads are issued for every position, past the end too (entry nnz - 1 again), and the
    // results dropped there, so that all of a lane's loads are in flight together (a load under
    // a per-lane condition is an exec-masked region that the compiler may wait on by itself).
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t p = base + u * groups + grp;
      ok[u] = p < nnz;
      const int64_t pc = ok[u] ? p : nnz - 1;
      r[u] = row_ids[pc];
      c[u] = cols[pc];
    }
    A acc[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) acc[u] = A(0);
    for (int k = lane * VW; k < K; k += G * VW) {
      T xv[kU][VW], yv[kU][VW];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        sload<T, VW>(x + r[u] * ldx + k, xv[u]);
        sload<T, VW>(y + c[u] * ldy + k, yv[u]);
      }
#pragma unroll
      for (int u = 0; u < kU; ++u)
#pragma unroll
        for (int j = 0; j < VW; ++j) acc[u] += ok[u] ? A(xv[u][j]) * A(yv[u][j]) : A(0);
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      acc[u] = group_sum(acc[u], G);
      if (lane == 0 && ok[u]) {
        const int64_t p = base + u * groups + grp;
        A v = acc[u] * a_alpha;
        if (in) v += A(in[p]) * a_beta;
        out[p] = O(v);
      }
    }
  }
}

template <typename T, typename A, typename O>
int launch_sddmm(int vec, const int32_t* cols, const int32_t* row_ids, int64_t nnz, const void* x,
                 int64_t ldx, const void* y, int64_t ldy, int64_t K, const void* in, double alpha,
                 double beta, void* out, int lg, hipStream_t st) {
  const int64_t per_step = 4 * (kBlock >> lg);  // entries per workgroup step (kU = 4)
  int64_t blocks = (nnz + per_step - 1) / per_step;
  if (blocks > (1 << 20)) blocks = 1 << 20;  // grid-stride loop covers the rest
  const T* xt = static_cast<const T*>(x);
  const T* yt = static_cast<const T*>(y);
  const T* it = static_cast<const T*>(in);
  O* ot = static_cast<O*>(out);
  if constexpr (sizeof(T) == 4) {
    if (vec == 4) {
      hipLaunchKernelGGL((sddmm_flat_kernel<T, A, O, 4>), dim3((unsigned)blocks), dim3(kBlock), 0,
                         st, cols, row_ids, nnz, xt, ldx, yt, ldy, (int)K, it, alpha, beta, ot, lg);
      return check_hip(hipGetLastError(), "sddmm_flat_kernel launch");
    }
  }
  if (vec == 2)
    hipLaunchKernelGGL((sddmm_flat_kernel<T, A, O, 2>), dim3((unsigned)blocks), dim3(kBlock), 0, st,
                       cols, row_ids, nnz, xt, ldx, yt, ldy, (int)K, it, alpha, beta, ot, lg);
  else
    hipLaunchKernelGGL((sddmm_flat_kernel<T, A, O, 1>), dim3((unsigned)blocks), dim3(kBlock), 0, st,
                       cols, row_ids, nnz, xt, ldx, yt, ldy, (int)K, it, alpha, beta, ot, lg);
  return check_hip(hipGetLastError(), "sddmm_flat_kernel launch");
}

template <typename T, typename A, typename O, typename P, int VW>
int launch_rows_kc(int kc, const int32_t* cols, const void* rowptr, int64_t nnz, const void* x,
                   int64_t ldx, const void* y, int64_t ldy, int64_t K, const void* in,
                   double alpha, double beta, void* out, const int32_t* desc,
                   const int64_t* ranges, int64_t n_desc, int lg, hipStream_t st) {
#define FSP_SD_ROWS(KCV)                                                                      \
  hipLaunchKernelGGL((sddmm_rowblock_kernel<T, A, O, P, VW, KCV>), dim3((unsigned)n_desc),    \
                     dim3(kBlock), 0, st, cols, static_cast<const P*>(rowptr), nnz,            \
                     static_cast<const T*>(x), ldx, static_cast<const T*>(y), ldy, (int)K,     \
                     static_cast<const T*>(in), alpha, beta, static_cast<O*>(out),             \
                     reinterpret_cast<const i32x4*>(desc), ranges, (int)n_desc, lg, 1)
  if (kc == 1) FSP_SD_ROWS(1);
  else if (kc == 2) FSP_SD_ROWS(2);
  else FSP_SD_ROWS(4);
#undef FSP_SD_ROWS
  return check_hip(hipGetLastError(), "sddmm_rowblock_kernel launch");
}

template <typename T, typename A, typename O>
int launch_rows(int vec, int rowptr_bits, const int32_t* cols, const void* rowptr, int64_t nnz,
                const void* x, int64_t ldx, const void* y, int64_t ldy, int64_t K,
                const void* in, double alpha, double beta, void* out, const int32_t* desc,
                const int64_t* ranges, int64_t n_desc, int lg, hipStream_t st) {
  const int64_t per_step = (int64_t)vec << lg;
  const int kc = (int)((K + per_step - 1) / per_step);  // 1, 2 or 4 (checked by the caller)
  const int kcp = kc <= 1 ? 1 : kc <= 2 ? 2 : 4;
#define FSP_SD_ARGS cols, rowptr, nnz, x, ldx, y, ldy, K, in, alpha, beta, out, desc, ranges, n_desc, lg, st
  if (rowptr_bits == 32) {
    if constexpr (sizeof(T) == 4) {
      if (vec == 4) return launch_rows_kc<T, A, O, int, 4>(kcp, FSP_SD_ARGS);
    }
    if (vec == 2) return launch_rows_kc<T, A, O, int, 2>(kcp, FSP_SD_ARGS);
    return launch_rows_kc<T, A, O, int, 1>(kcp, FSP_SD_ARGS);
  }
  if constexpr (sizeof(T) == 4) {
    if (vec == 4) return launch_rows_kc<T, A, O, int64_t, 4>(kcp, FSP_SD_ARGS);
  }
  if (vec == 2) return launch_rows_kc<T, A, O, int64_t, 2>(kcp, FSP_SD_ARGS);
  return launch_rows_kc<T, A, O, int64_t, 1>(kcp, FSP_SD_ARGS);
#undef FSP_SD_ARGS
}

template <typename T, typename A, typename O>
int launch_any(int vec, int rowptr_bits, const int32_t* cols, const int32_t* row_ids,
               const void* rowptr, int64_t nnz, const void* x, int64_t ldx, const void* y,
               int64_t ldy, int64_t K, const void* in, double alpha, double beta, void* out,
               const int32_t* desc, const int64_t* ranges, int64_t n_desc, int lg,
               hipStream_t st) {
  if (n_desc > 0)
    return launch_rows<T, A, O>(vec, rowptr_bits, cols, rowptr, nnz, x, ldx, y, ldy, K, in,
                                alpha, beta, out, desc, ranges, n_desc, lg, st);
  return launch_sddmm<T, A, O>(vec, cols, row_ids, nnz, x, ldx, y, ldy, K, in, alpha, beta, out,
                               lg, st);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace fsp

using namespace fsp;

extern "C" int fsp_sddmm_csr(int dtype, int acc_f64, int out_f64, const int32_t* cols,
                             const int32_t* row_ids, const void* rowptr, int rowptr_bits,
                             int64_t nnz, const void* x, int64_t ldx, const void* y, int64_t ldy,
                             int64_t K, const void* data_in, double alpha, double beta, void* out,
                             const int32_t* desc, const int64_t* ranges, int64_t n_desc,
                             int lanes_per_entry, int vec, void* stream) {
  if (dtype != FSP_F32 && dtype != FSP_F64) return set_error(FSP_ENOTSUP, "fsp_sddmm_csr: dtype");
  if (nnz < 0 || K < 0) return set_error(FSP_EINVAL, "fsp_sddmm_csr: negative size");
  if (K > 0x7fffffffLL) return set_error(FSP_EINVAL, "fsp_sddmm_csr: K exceeds 2^31-1");
  int lg = -1;
  for (int g = 0; g <= 6; ++g)
    if (lanes_per_entry == (1 << g)) lg = g;
  if (lg < 0) return set_error(FSP_EINVAL, "fsp_sddmm_csr: lanes_per_entry must be 1,2,4,...,64");
  const int max_vec = (dtype == FSP_F32) ? 4 : 2;
  if (vec != 1 && vec != 2 && vec != max_vec)
    return set_error(FSP_EINVAL, "fsp_sddmm_csr: vec must be 1, 2 or 4 (fp32) / 1, 2 (fp64)");
  if (nnz == 0) return FSP_OK;
  if (!cols || !out) return set_error(FSP_EINVAL, "fsp_sddmm_csr: null pointer");
  if (K > 0 && (!x || !y)) return set_error(FSP_EINVAL, "fsp_sddmm_csr: null x or y");
  if (ldx < K || ldy < K) return set_error(FSP_EINVAL, "fsp_sddmm_csr: ldx/ldy smaller than K");
  if (vec > 1 && (K % vec || ldx % vec || ldy % vec || !aligned16(x) || !aligned16(y)))
    return set_error(FSP_EINVAL, "fsp_sddmm_csr: vec > 1 needs K, ldx, ldy multiples of vec and "
                                 "16-byte aligned x, y");
  if (out_f64 && dtype != FSP_F32)
    return set_error(FSP_EINVAL, "fsp_sddmm_csr: out_f64 applies to fp32 inputs only");
  if (n_desc < 0 || n_desc > 0x7fffffffLL)
    return set_error(FSP_EINVAL, "fsp_sddmm_csr: n_desc outside [0, 2^31-1]");
  if (n_desc > 0) {
    if (!desc || !ranges || !rowptr)
      return set_error(FSP_EINVAL, "fsp_sddmm_csr: row-block plan without desc/ranges/rowptr");
    if (rowptr_bits != 32 && rowptr_bits != 64)
      return set_error(FSP_EINVAL, "fsp_sddmm_csr: rowptr_bits must be 32 or 64");
    if (K > 4 * ((int64_t)vec << lg))
      return set_error(FSP_EINVAL, "fsp_sddmm_csr: a row-block plan needs K <= 4 * lanes * vec");
    if (!aligned16(cols)) return set_error(FSP_EINVAL, "fsp_sddmm_csr: cols must be 16-byte aligned");
  } else if (!row_ids) {
    return set_error(FSP_EINVAL, "fsp_sddmm_csr: null row_ids");
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
#define FSP_SD_CALL vec, rowptr_bits, cols, row_ids, rowptr, nnz, x, ldx, y, ldy, K, data_in, \
                    alpha, beta, out, desc, ranges, n_desc, lg, st
  if (dtype == FSP_F64) return launch_any<double, double, double>(FSP_SD_CALL);
  if (out_f64) return launch_any<float, double, double>(FSP_SD_CALL);
  if (acc_f64) return launch_any<float, double, float>(FSP_SD_CALL);
  return launch_any<float, float, float>(FSP_SD_CALL);
#undef FSP_SD_CALL
}
