// One pass over two index arrays of the same length (COO rows and columns): the minimum and
// maximum of each and the number of places where the first one decreases.  The validation of
// a COO call needs exactly these (indices in range, int32-representable, rows already in
// order); as separate torch reductions they were four passes plus a fifth for the order, each
// reading the arrays again (cfg5-shape COO SpMM: 226 us of a 1.2 ms call).
//
// Reference behaviour replaced: the per-call checks of spmm_coo.py:312-371
// (_prepare_spmm_coo_inputs: min/max of row and col) and the sortedness test that decides
// whether the entries must be sorted (spmm_coo.py:394-461, _coo_is_sorted_lex).
//
// Two launches, no atomics: up to kIndexStatsBlocks workgroups each reduce a grid-strided share into five
// partials (registers, then a wave reduction and one LDS step), then one workgroup reduces the
// partials in a fixed order.
#include <climits>
#include <limits>

#include "fsp_device.hpp"
#include "fsp_internal.hpp"

namespace fsp {
namespace {

constexpr int kStats = 5;  // min a, max a, min b, max b, descents of a

__device__ __forceinline__ int64_t wave_min64(int64_t v) {
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int64_t o = __shfl_xor(v, off, kWave);
    v = o < v ? o : v;
  }
  return v;
}

__device__ __forceinline__ int64_t wave_max64(int64_t v) {
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int64_t o = __shfl_xor(v, off, kWave);
    v = o > v ? o : v;
  }
  return v;
}

__device__ __forceinline__ int64_t wave_add64(int64_t v) {
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Reduce the five values of every thread of the workgroup; thread 0 returns the result in s.
__device__ __forceinline__ void block_stats(int64_t (&s)[kStats], int64_t (*lds)[kStats]) {
  s[0] = wave_min64(s[0]);
  s[1] = wave_max64(s[1]);
  s[2] = wave_min64(s[2]);
  s[3] = wave_max64(s[3]);
  s[4] = wave_add64(s[4]);
  const int wid = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  if (lane == 0) {
#pragma unroll
    for (int k = 0; k < kStats; ++k) lds[wid][k] = s[k];
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kWavesPerBlock; ++w) {
      s[0] = lds[w][0] < s[0] ? lds[w][0] : s[0];
      s[1] = lds[w][1] > s[1] ? lds[w][1] : s[1];
      s[2] = lds[w][2] < s[2] ? lds[w][2] : s[2];
      s[3] = lds[w][3] > s[3] ? lds[w][3] : s[3];
      s[4] += lds[w][4];
    }
  }
}

typedef int64_t i64x2 __attribute__((ext_vector_type(2)));

// Four consecutive elements from 16-byte-aligned storage.
template <typename T>
__device__ __forceinline__ void load_quad(const T* p, T (&v)[4]) {
  if constexpr (sizeof(T) == 4) {
    const i32x4 q = *reinterpret_cast<const i32x4*>(p);
    v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
  } else {
    const i64x2 q0 = reinterpret_cast<const i64x2*>(p)[0];
    const i64x2 q1 = reinterpret_cast<const i64x2*>(p)[1];
    v[0] = q0.x; v[1] = q0.y; v[2] = q1.x; v[3] = q1.y;
  }
}

// Grid-strided over quads of four elements (16-byte loads; VEC requires a and b 16-byte
// aligned), min / max kept in the index type; the element before a lane's quad comes from the
// lane below (lane 0 reads it).  Without VEC, one element per step.
template <typename IA, typename IB, bool VEC>
__global__ __launch_bounds__(kBlock) void index_stats_kernel(const IA* __restrict__ a,
                                                             const IB* __restrict__ b, int64_t n,
                                                             int64_t* __restrict__ partial) {
  __shared__ int64_t lds[kWavesPerBlock][kStats];
  IA mina = std::numeric_limits<IA>::max(), maxa = std::numeric_limits<IA>::min();
  IB minb = std::numeric_limits<IB>::max(), maxb = std::numeric_limits<IB>::min();
  int64_t desc = 0;
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  if constexpr (VEC) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t nq = n / 4;
    // the loop runs the same number of times in every lane of a wave (the shuffle needs them)
    const int64_t first = (int64_t)blockIdx.x * kBlock + threadIdx.x - lane;
    for (int64_t q0 = first; q0 < nq; q0 += stride) {
      const int64_t q = q0 + lane;
      const bool ok = q < nq;
      IA va[4] = {0, 0, 0, 0};
      IB vb[4] = {0, 0, 0, 0};
      if (ok) {
        load_quad<IA>(a + 4 * q, va);
        load_quad<IB>(b + 4 * q, vb);
      }
      IA prev = __shfl_up(va[3], 1, kWave);
      if (lane == 0 && ok && q > 0) prev = a[4 * q - 1];
      if (ok) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          mina = va[j] < mina ? va[j] : mina;
          maxa = va[j] > maxa ? va[j] : maxa;
          minb = vb[j] < minb ? vb[j] : minb;
          maxb = vb[j] > maxb ? vb[j] : maxb;
        }
        desc += (q > 0 && va[0] < prev) + (va[1] < va[0]) + (va[2] < va[1]) + (va[3] < va[2]);
      }
    }
    // the n % 4 tail
    for (int64_t i = 4 * nq + (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
      const IA x = a[i];
      const IB y = b[i];
      mina = x < mina ? x : mina;
      maxa = x > maxa ? x : maxa;
      minb = y < minb ? y : minb;
      maxb = y > maxb ? y : maxb;
      if (i > 0 && x < a[i - 1]) ++desc;
    }
  } else {
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
      const IA x = a[i];
      const IB y = b[i];
      mina = x < mina ? x : mina;
      maxa = x > maxa ? x : maxa;
      minb = y < minb ? y : minb;
      maxb = y > maxb ? y : maxb;
      if (i > 0 && x < a[i - 1]) ++desc;
    }
  }
  int64_t s[kStats] = {(int64_t)mina, (int64_t)maxa, (int64_t)minb, (int64_t)maxb, desc};
  if (n == 0) {
    s[0] = LLONG_MAX; s[1] = LLONG_MIN; s[2] = LLONG_MAX; s[3] = LLONG_MIN;
  }
  // A thread that saw no element holds its type's extremes: neutral for min / max over values
  // of that type.
  block_stats(s, lds);
  if (threadIdx.x == 0) {
#pragma unroll
    for (int k = 0; k < kStats; ++k) partial[(int64_t)blockIdx.x * kStats + k] = s[k];
  }
}

__global__ __launch_bounds__(kBlock) void index_stats_final_kernel(
    const int64_t* __restrict__ partial, int n_partial, int64_t* __restrict__ out) {
  __shared__ int64_t lds[kWavesPerBlock][kStats];
  int64_t s[kStats] = {LLONG_MAX, LLONG_MIN, LLONG_MAX, LLONG_MIN, 0};
  for (int p = threadIdx.x; p < n_partial; p += kBlock) {
    const int64_t* q = partial + (int64_t)p * kStats;
    s[0] = q[0] < s[0] ? q[0] : s[0];
    s[1] = q[1] > s[1] ? q[1] : s[1];
    s[2] = q[2] < s[2] ? q[2] : s[2];
    s[3] = q[3] > s[3] ? q[3] : s[3];
    s[4] += q[4];
  }
  block_stats(s, lds);
  if (threadIdx.x == 0) {
#pragma unroll
    for (int k = 0; k < kStats; ++k) out[k] = s[k];
  }
}

template <typename IA, typename IB>
int launch_stats(const void* a, const void* b, int64_t n, int64_t* partial, int64_t* out,
                 hipStream_t st) {
  int64_t blocks = (n + (int64_t)kBlock * 16 - 1) / ((int64_t)kBlock * 16);
  if (blocks < 1) blocks = 1;
  if (blocks > kIndexStatsBlocks) blocks = kIndexStatsBlocks;
  const bool vec = ((uintptr_t)a % 16 == 0) && ((uintptr_t)b % 16 == 0);
  if (vec)
    hipLaunchKernelGGL((index_stats_kernel<IA, IB, true>), dim3((unsigned)blocks), dim3(kBlock), 0,
                       st, static_cast<const IA*>(a), static_cast<const IB*>(b), n, partial);
  else
    hipLaunchKernelGGL((index_stats_kernel<IA, IB, false>), dim3((unsigned)blocks), dim3(kBlock),
                       0, st, static_cast<const IA*>(a), static_cast<const IB*>(b), n, partial);
  int rc = check_hip(hipGetLastError(), "index_stats_kernel launch");
  if (rc) return rc;
  hipLaunchKernelGGL(index_stats_final_kernel, dim3(1), dim3(kBlock), 0, st, partial,
                     (int)blocks, out);
  return check_hip(hipGetLastError(), "index_stats_final_kernel launch");
}

}  // namespace
}  // namespace fsp

using namespace fsp;

extern "C" int fsp_index_stats(const void* a, int a_bits, const void* b, int b_bits, int64_t n,
                               int64_t* partial, int64_t* out, void* stream) {
  if ((a_bits != 32 && a_bits != 64) || (b_bits != 32 && b_bits != 64))
    return set_error(FSP_EINVAL, "fsp_index_stats: index widths must be 32 or 64");
  if (n < 0) return set_error(FSP_EINVAL, "fsp_index_stats: n must be >= 0");
  if (!partial || !out)
    return set_error(FSP_EINVAL, "fsp_index_stats: null partial or out");
  if (n > 0 && (!a || !b)) return set_error(FSP_EINVAL, "fsp_index_stats: null index array");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (a_bits == 32 && b_bits == 32) return launch_stats<int32_t, int32_t>(a, b, n, partial, out, st);
  if (a_bits == 32) return launch_stats<int32_t, int64_t>(a, b, n, partial, out, st);
  if (b_bits == 32) return launch_stats<int64_t, int32_t>(a, b, n, partial, out, st);
  return launch_stats<int64_t, int64_t>(a, b, n, partial, out, st);
}

extern "C" int64_t fsp_index_stats_partial_len(void) { return kIndexStatsBlocks * 5; }
