// Measurement probes for bench.py: the rates at which gfx950 serves the two access patterns
// the SpMV / SpMM kernels are bound by, measured alone, so that the kernels' times can be read
// against them (no counterpart in the reference; nothing on the product path calls these).
//
//   probe_gather_kernel  random 4-byte gathers x[idx[i]]: each thread takes 16 consecutive
//                        indices (four 16-byte loads) and issues its 16 gathers together - the
//                        pattern of the SpMV x gathers (spmv_xcs_kernel issues 8 per thread)
//   probe_rows_kernel    random row gathers from a row-major matrix: 16 lanes share one row of
//                        row_bytes (16 bytes each), each lane has four rows in flight - the
//                        pattern of the SpMM B-row gathers (spmm_rowblock_kernel, N = 64 fp32)
//   probe_stream_kernel  a plain read of a contiguous range with non-temporal 16-byte loads,
//                        eight in flight per thread - the entry stream of the panel kernel
//                        (spmv_panel_kernel) without its LDS gathers, sums and stores
//
// Every workgroup writes the sum of what it loaded to out[blockIdx.x] (a fixed-order reduction),
// so no load can be dropped by the compiler and the write traffic is one value per workgroup.
#include "fsp_device.hpp"
#include "fsp_internal.hpp"

namespace fsp {
namespace {

constexpr int kGatherPer = 16;  // gathers per thread
constexpr int kRowLanes = 16;   // lanes per row (16 bytes each)
constexpr int kRowsInFlight = 4;

__global__ __launch_bounds__(kBlock) void probe_gather_kernel(const float* __restrict__ x,
                                                              unsigned x_last,
                                                              const i32x4* __restrict__ idx,
                                                              int64_t n4,
                                                              float* __restrict__ out) {
  __shared__ float red[kWavesPerBlock];
  const int64_t q0 = ((int64_t)blockIdx.x * kBlock + threadIdx.x) * (kGatherPer / 4);
  i32x4 c[kGatherPer / 4];
#pragma unroll
  for (int u = 0; u < kGatherPer / 4; ++u) {
    const int64_t q = q0 + u < n4 ? q0 + u : n4 - 1;  // the tail reloads the last quad
    c[u] = __builtin_nontemporal_load(&idx[q]);
  }
  // indices are clamped into x (an unsigned min per gather), so no input can read outside it
  float v[kGatherPer];
#pragma unroll
  for (int u = 0; u < kGatherPer / 4; ++u) {
    v[4 * u] = x[min((unsigned)c[u].x, x_last)];
    v[4 * u + 1] = x[min((unsigned)c[u].y, x_last)];
    v[4 * u + 2] = x[min((unsigned)c[u].z, x_last)];
    v[4 * u + 3] = x[min((unsigned)c[u].w, x_last)];
  }
  float acc = 0.0f;
#pragma unroll
  for (int u = 0; u < kGatherPer / 4; ++u)
    if (q0 + u < n4) acc += (v[4 * u] + v[4 * u + 1]) + (v[4 * u + 2] + v[4 * u + 3]);
  acc = block_sum(acc, red);
  if (threadIdx.x == 0) out[blockIdx.x] = acc;
}

__global__ __launch_bounds__(kBlock) void probe_rows_kernel(const float* __restrict__ b,
                                                            unsigned row_last, int64_t row_floats,
                                                            const int* __restrict__ rows,
                                                            int64_t n, float* __restrict__ out) {
  __shared__ float red[kWavesPerBlock];
  const int lane = threadIdx.x & (kRowLanes - 1);
  const int64_t grp = ((int64_t)blockIdx.x * kBlock + threadIdx.x) / kRowLanes;
  const int64_t groups = (int64_t)gridDim.x * (kBlock / kRowLanes);
  int r[kRowsInFlight];
#pragma unroll
  for (int u = 0; u < kRowsInFlight; ++u) {
    const int64_t i = grp + u * groups;
    r[u] = (int)min((unsigned)rows[i < n ? i : n - 1], row_last);  // clamped into b
  }
  f32x4 v[kRowsInFlight];
#pragma unroll
  for (int u = 0; u < kRowsInFlight; ++u)
    v[u] = *reinterpret_cast<const f32x4*>(b + (int64_t)r[u] * row_floats + 4 * lane);
  float acc = 0.0f;
#pragma unroll
  for (int u = 0; u < kRowsInFlight; ++u)
    if (grp + u * groups < n) acc += (v[u].x + v[u].y) + (v[u].z + v[u].w);
  acc = block_sum(acc, red);
  if (threadIdx.x == 0) out[blockIdx.x] = acc;
}

constexpr int kStreamPer = 8;  // 16-byte loads per thread

__global__ __launch_bounds__(kBlock) void probe_stream_kernel(const i32x4* __restrict__ src,
                                                              int64_t n16,
                                                              float* __restrict__ out) {
  __shared__ float red[kWavesPerBlock];
  const int64_t v0 = (int64_t)blockIdx.x * kBlock * kStreamPer + threadIdx.x;
  i32x4 v[kStreamPer];
#pragma unroll
  for (int u = 0; u < kStreamPer; ++u) {
    const int64_t i = v0 + (int64_t)u * kBlock;
    v[u] = ld_stream<true>(src + (i < n16 ? i : n16 - 1));  // the tail reloads the last one
  }
  int acc = 0;
#pragma unroll
  for (int u = 0; u < kStreamPer; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  float f = (float)(acc & 1);
  f = block_sum(f, red);
  if (threadIdx.x == 0) out[blockIdx.x] = f;
}

}  // namespace
}  // namespace fsp

using namespace fsp;

extern "C" int64_t fsp_probe_gather_blocks(int64_t n) {
  return n <= 0 ? 0 : (n + (int64_t)kBlock * kGatherPer - 1) / ((int64_t)kBlock * kGatherPer);
}

extern "C" int fsp_probe_gather(const float* x, int64_t x_len, const int32_t* idx, int64_t n,
                                float* out, void* stream) {
  if (n < 0 || x_len < 0) return set_error(FSP_EINVAL, "fsp_probe_gather: negative size");
  if (n % 4) return set_error(FSP_EINVAL, "fsp_probe_gather: n must be a multiple of 4");
  if (n == 0) return FSP_OK;
  if (!x || !idx || !out || x_len == 0) return set_error(FSP_EINVAL, "fsp_probe_gather: null");
  if (x_len > 0x7fffffffLL) return set_error(FSP_EINVAL, "fsp_probe_gather: x beyond 2^31");
  if ((reinterpret_cast<uintptr_t>(idx) & 15u) != 0)
    return set_error(FSP_EINVAL, "fsp_probe_gather: idx must be 16-byte aligned");
  const int64_t blocks = fsp_probe_gather_blocks(n);
  if (blocks > 0x7fffffffLL) return set_error(FSP_EINVAL, "fsp_probe_gather: n too large");
  hipLaunchKernelGGL(probe_gather_kernel, dim3((unsigned)blocks), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), x, (unsigned)(x_len - 1),
                     reinterpret_cast<const i32x4*>(idx), n / 4, out);
  return check_hip(hipGetLastError(), "probe_gather_kernel launch");
}

extern "C" int64_t fsp_probe_rows_blocks(int64_t n) {
  const int64_t per_block = (int64_t)(kBlock / kRowLanes) * kRowsInFlight;
  return n <= 0 ? 0 : (n + per_block - 1) / per_block;
}

extern "C" int fsp_probe_rows(const float* b, int64_t n_rows, int64_t row_floats,
                              const int32_t* rows, int64_t n, float* out, void* stream) {
  if (n < 0 || n_rows < 0) return set_error(FSP_EINVAL, "fsp_probe_rows: negative size");
  if (row_floats != 4 * kRowLanes)
    return set_error(FSP_EINVAL, "fsp_probe_rows: rows of 64 floats (256 bytes) only");
  if (n == 0) return FSP_OK;
  if (!b || !rows || !out || n_rows == 0) return set_error(FSP_EINVAL, "fsp_probe_rows: null");
  if (n_rows > 0x7fffffffLL) return set_error(FSP_EINVAL, "fsp_probe_rows: n_rows beyond 2^31");
  if ((reinterpret_cast<uintptr_t>(b) & 15u) != 0)
    return set_error(FSP_EINVAL, "fsp_probe_rows: b must be 16-byte aligned");
  const int64_t blocks = fsp_probe_rows_blocks(n);
  if (blocks > 0x7fffffffLL) return set_error(FSP_EINVAL, "fsp_probe_rows: n too large");
  hipLaunchKernelGGL(probe_rows_kernel, dim3((unsigned)blocks), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), b, (unsigned)(n_rows - 1), row_floats, rows,
                     n, out);
  return check_hip(hipGetLastError(), "probe_rows_kernel launch");
}

extern "C" int64_t fsp_probe_stream_blocks(int64_t n16) {
  const int64_t per_block = (int64_t)kBlock * kStreamPer;
  return n16 <= 0 ? 0 : (n16 + per_block - 1) / per_block;
}

extern "C" int fsp_probe_stream(const void* src, int64_t n16, float* out, void* stream) {
  if (n16 < 0) return set_error(FSP_EINVAL, "fsp_probe_stream: negative size");
  if (n16 == 0) return FSP_OK;
  if (!src || !out) return set_error(FSP_EINVAL, "fsp_probe_stream: null");
  if ((reinterpret_cast<uintptr_t>(src) & 15u) != 0)
    return set_error(FSP_EINVAL, "fsp_probe_stream: src must be 16-byte aligned");
  const int64_t blocks = fsp_probe_stream_blocks(n16);
  if (blocks > 0x7fffffffLL) return set_error(FSP_EINVAL, "fsp_probe_stream: n16 too large");
  hipLaunchKernelGGL(probe_stream_kernel, dim3((unsigned)blocks), dim3(kBlock), 0,
                     static_cast<hipStream_t>(stream), static_cast<const i32x4*>(src), n16, out);
  return check_hip(hipGetLastError(), "probe_stream_kernel launch");
}
