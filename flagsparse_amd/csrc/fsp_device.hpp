// Device-side building blocks shared by the SpMV / SpMM kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fsp {

constexpr int kWave = 64;
constexpr int kBlock = 256;               // threads per workgroup (4 waves)
constexpr int kWavesPerBlock = kBlock / kWave;

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef double f64x2 __attribute__((ext_vector_type(2)));

// Streaming loads: the matrix arrays are read exactly once per call; with NT they are fetched
// with the non-temporal hint and do not displace x / B lines from L2 and the MALL (used where
// x or B is held in L2 on purpose: the XCS SpMV and the SpMM kernels).
template <bool NT, typename V>
__device__ __forceinline__ V ld_stream(const V* p) {
  if constexpr (NT) {
    return __builtin_nontemporal_load(p);
  } else {
    return *p;
  }
}

// Four consecutive matrix entries ("a quad"): values converted to the accumulator type.
// base is a multiple of 4, so the 16-byte vector loads are aligned when the array base is.
// Entries outside [lo, hi) are returned with val = 0 and col = -1.
template <bool NT, typename T>
struct QuadLoader;

template <bool NT>
struct QuadLoader<NT, float> {
  template <typename P>
  __device__ __forceinline__ static void load(const float* __restrict__ vals,
                                              const int* __restrict__ cols, P base, P lo,
                                              P hi, P nnz_total, float (&v)[4], int (&c)[4]) {
    if (base + 4 <= nnz_total) {
      f32x4 vv = ld_stream<NT>(reinterpret_cast<const f32x4*>(vals + base));
      i32x4 cc = ld_stream<NT>(reinterpret_cast<const i32x4*>(cols + base));
      v[0] = vv.x; v[1] = vv.y; v[2] = vv.z; v[3] = vv.w;
      c[0] = cc.x; c[1] = cc.y; c[2] = cc.z; c[3] = cc.w;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool ok = base + j < nnz_total;
        v[j] = ok ? vals[base + j] : 0.0f;
        c[j] = ok ? cols[base + j] : -1;
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool in = (base + j >= lo) && (base + j < hi);
      if (!in) { v[j] = 0.0f; c[j] = -1; }
    }
  }
};

template <bool NT>
struct QuadLoader<NT, double> {
  template <typename P>
  __device__ __forceinline__ static void load(const double* __restrict__ vals,
                                              const int* __restrict__ cols, P base, P lo,
                                              P hi, P nnz_total, double (&v)[4], int (&c)[4]) {
    if (base + 4 <= nnz_total) {
      f64x2 v01 = ld_stream<NT>(reinterpret_cast<const f64x2*>(vals + base));
      f64x2 v23 = ld_stream<NT>(reinterpret_cast<const f64x2*>(vals + base + 2));
      i32x4 cc = ld_stream<NT>(reinterpret_cast<const i32x4*>(cols + base));
      v[0] = v01.x; v[1] = v01.y; v[2] = v23.x; v[3] = v23.y;
      c[0] = cc.x; c[1] = cc.y; c[2] = cc.z; c[3] = cc.w;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool ok = base + j < nnz_total;
        v[j] = ok ? vals[base + j] : 0.0;
        c[j] = ok ? cols[base + j] : -1;
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool in = (base + j >= lo) && (base + j < hi);
      if (!in) { v[j] = 0.0; c[j] = -1; }
    }
  }
};

// Lane permutes through DPP (a VALU modifier, no LDS round trip).  dpp_add<CTRL>(v) adds the
// value of the lane that the DPP control word CTRL selects; all sources used here lie inside
// the lane's 16-lane row, so every lane reads a valid source.
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF,
                                                        false));
}

template <int CTRL>
__device__ __forceinline__ double dpp_add(double v) {
  const int64_t b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(b & 0xffffffff), CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(b >> 32), CTRL, 0xF, 0xF, false);
  return v + __longlong_as_double(((int64_t)hi << 32) | (uint32_t)lo);
}

// DPP move: the value of the lane that CTRL selects, or `old` where that lane lies outside the
// control's range or ROW_MASK leaves the lane's row out (bound_ctrl off).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ int dpp_mov(int old, int v) {
  return __builtin_amdgcn_update_dpp(old, v, CTRL, ROW_MASK, 0xF, false);
}

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_mov(float old, float v) {
  return __int_as_float(dpp_mov<CTRL, ROW_MASK>(__float_as_int(old), __float_as_int(v)));
}

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ double dpp_mov(double old, double v) {
  const int64_t b = __double_as_longlong(v), o = __double_as_longlong(old);
  const int lo = dpp_mov<CTRL, ROW_MASK>((int)(o & 0xffffffff), (int)(b & 0xffffffff));
  const int hi = dpp_mov<CTRL, ROW_MASK>((int)(o >> 32), (int)(b >> 32));
  return __longlong_as_double(((int64_t)hi << 32) | (uint32_t)lo);
}

// DPP controls of the GFX9 family used for wave-wide scans.
constexpr int kDppRowShr1 = 0x111;  // row_shr:n = 0x110 + n (inside a 16-lane row)
constexpr int kDppRowBcast15 = 0x142;  // lane 15 of each row to the next row
constexpr int kDppRowBcast31 = 0x143;  // lane 31 to rows 2 and 3
constexpr int kDppWaveShl1 = 0x130;  // lane i takes lane i + 1
constexpr int kDppWaveShr1 = 0x138;  // lane i takes lane i - 1

// Sum over aligned groups of g lanes (g a power of two, g <= 64); every lane of the group ends
// with the total.  Inside a 16-lane row: quad permutes [1,0,3,2] and [2,3,0,1], then the
// half-row mirror and the row mirror (DPP); across rows, lane exchanges (ds_bpermute).  The
// order of the additions is fixed, so the result is deterministic.  All lanes of a group must
// be active.
template <typename A>
__device__ __forceinline__ A group_sum(A v, int g) {
  if (g >= 2) v = dpp_add<0xB1>(v);   // quad_perm [1,0,3,2]
  if (g >= 4) v = dpp_add<0x4E>(v);   // quad_perm [2,3,0,1]
  if (g >= 8) v = dpp_add<0x141>(v);  // row_half_mirror
  if (g >= 16) v = dpp_add<0x140>(v); // row_mirror
  if (g >= 32) v += __shfl_xor(v, 16, kWave);
  if (g >= 64) v += __shfl_xor(v, 32, kWave);
  return v;
}

template <typename A>
__device__ __forceinline__ A wave_sum(A v) {
  return group_sum(v, kWave);
}

// Workgroup sum in a fixed order: group_sum inside each wave, then waves 0..3 in order.
// Result valid in every thread.  red must hold kWavesPerBlock entries.
template <typename A>
__device__ __forceinline__ A block_sum(A v, A* red) {
  v = wave_sum(v);
  const int tid = threadIdx.x;
  __syncthreads();  // red may still be read by a previous call
  if ((tid & (kWave - 1)) == 0) red[tid / kWave] = v;
  __syncthreads();
  A t = red[0];
#pragma unroll
  for (int w = 1; w < kWavesPerBlock; ++w) t += red[w];
  return t;
}

// Workgroups are dispatched round-robin over the 8 XCDs (workgroup i runs on XCD i % 8).
// Remap so that XCD k processes one contiguous range of logical blocks: neighbouring rows
// (which share x / B lines) then meet in the same L2.  Bijective for any n.
__device__ __forceinline__ int xcd_logical_block(int i, int n) {
  constexpr int kXcd = 8;
  const int q = n / kXcd, r = n % kXcd;
  const int x = i % kXcd, j = i / kXcd;
  return (x < r) ? x * (q + 1) + j : r * (q + 1) + (x - r) * q + j;
}

// Second pass of every split-row SpMV: rows whose entries were summed by several workgroups
// get y[row] = sum over j < n of partials[base + j*S + s], in a fixed order (j increasing for
// S > 1; for S == 1 a fixed workgroup tree), so the result does not depend on which workgroup
// finished first.  Group g covers S rows split_rows[first .. first + S), its partials start at
// group_base[g] and are laid out [n][S].  It runs as a separate launch on the same stream: the
// kernel boundary makes the first pass's partials visible on every XCD, so neither pass needs
// a device-scope fence.  With reset != 0 every slot read is set back to 0, for first passes
// that write only the slots of rows they hold.  Slots at or beyond partials_cap (the
// workspace's size) are neither read nor written.
template <typename T, typename A>
__global__ __launch_bounds__(kBlock) void split_row_combine_kernel(
    const i32x4* __restrict__ groups, const int64_t* __restrict__ group_base,
    const int* __restrict__ split_rows, A* __restrict__ partials, int64_t partials_cap,
    T* __restrict__ y, const int* __restrict__ row_map, int reset) {
  __shared__ A red[kWavesPerBlock];
  const i32x4 g = groups[blockIdx.x];
  const int first = g.x, S = g.y, n = g.z;
  const int64_t base = group_base[blockIdx.x];
  if (S == 1) {
    // One row: the workgroup sums its n partials (thread t takes t, t + 256, ... in order,
    // then the fixed-order workgroup sum), so a row cut into many chunks is not summed by a
    // single thread.
    A acc = A(0);
    for (int j = threadIdx.x; j < n; j += kBlock) {
      if (base + j >= partials_cap) break;  // a plan larger than the workspace
      A* p = &partials[base + j];
      acc += *p;
      if (reset) *p = A(0);
    }
    acc = block_sum(acc, red);
    if (threadIdx.x == 0) {
      const int row = split_rows[first];
      y[row_map ? row_map[row] : row] = T(acc);
    }
    return;
  }
  for (int s = threadIdx.x; s < S; s += kBlock) {
    A acc = A(0);
    for (int j = 0; j < n; ++j) {
      if (base + (int64_t)j * S + s >= partials_cap) break;  // a plan larger than the workspace
      A* p = &partials[base + (int64_t)j * S + s];
      acc += *p;
      if (reset) *p = A(0);
    }
    const int row = split_rows[first + s];
    y[row_map ? row_map[row] : row] = T(acc);
  }
}

}  // namespace fsp
