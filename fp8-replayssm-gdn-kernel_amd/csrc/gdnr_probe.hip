// gdnr_probe.hip -- the HBM floor of the decode path's traffic, for the
// benchmark: a coalesced stream over one buffer (a checkpoint's codes), read
// only (the replay's dominant traffic) or read and written back in place (the
// flush's), with plain or non-temporal loads. Each lane moves 16 bytes per
// access; consecutive lanes touch
// consecutive 16-byte pieces; a grid of 8 workgroups of 256 threads per
// compute unit strides over the buffer, four accesses in flight per lane.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gdnr_internal.h"

namespace gdnr {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

template <bool WRITE, bool NT>
__global__ __launch_bounds__(256) void stream_probe_kernel(u32x4_t* buf, int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (int64_t i = i0; i < n16; i += 4 * stride) {
    u32x4_t x[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (i + k * stride < n16) {
        // (non-temporal: as the decode kernels read the checkpoint codes)
        if constexpr (NT) x[k] = __builtin_nontemporal_load(buf + i + k * stride);
        else x[k] = buf[i + k * stride];
      }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (i + k * stride >= n16) continue;
      if constexpr (WRITE) {
        asm volatile("" : "+v"(x[k]));  // stored back as it was read, but not as a known copy
        buf[i + k * stride] = x[k];
      } else {
        asm volatile("" ::"v"(x[k]));  // the piece is consumed: the load stays
      }
    }
  }
}

// The decode kernel's access order: 8 waves per workgroup, one workgroup
// per compute unit, every wave reading its own contiguous chunk of
// chunk16 pieces in 16 loads in flight per lane (the decode's row wave: its
// value head's 16 KiB, all requested at once), chunks in wave order.
// TILED: within its chunk (128-byte rows) a wave reads as the decode
// kernel's row wave reads its value head: load 2 i + h of lane (nn, q4)
// takes bytes [32 q4 + 16 h, +16) of row 32 (i >> 1) + 2 nn + (i & 1), so
// every load covers half of each of 16 rows; otherwise 1 KiB contiguous.
template <bool NT, bool TILED>
__global__ __launch_bounds__(512) void chunk_probe_kernel(const u32x4_t* buf, int64_t n16, int64_t chunk16) {
  const int64_t wave = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int nn = lane & 15, q4 = lane >> 4;
  for (int64_t base = wave * chunk16; base < n16; base += (int64_t)gridDim.x * 8 * chunk16) {
    u32x4_t x[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int t = k >> 1, h = k & 1;
      const int piece = TILED ? 8 * (32 * (t >> 1) + 2 * nn + (t & 1)) + 2 * q4 + h : 64 * k + lane;
      const int64_t i = base + piece;
      if (piece < chunk16 && i < n16) {
        if constexpr (NT) x[k] = __builtin_nontemporal_load(buf + i);
        else x[k] = buf[i];
      }
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) asm volatile("" ::"v"(x[k]));
  }
}

}  // namespace

int launch_stream_probe(void* buf, int64_t bytes, bool write, bool nt, bool chunked, bool tiled, void* stream) {
  if (chunked) {
    hipStream_t s = (hipStream_t)stream;
    const int64_t n16 = bytes / 16;
    const unsigned grid = (unsigned)device_cus();
    const int64_t chunk16 = 1024;  // 16 KiB per wave per pass
    const u32x4_t* b = (const u32x4_t*)buf;
    if (nt && tiled) hipLaunchKernelGGL((chunk_probe_kernel<true, true>), dim3(grid), dim3(512), 0, s, b, n16, chunk16);
    else if (nt) hipLaunchKernelGGL((chunk_probe_kernel<true, false>), dim3(grid), dim3(512), 0, s, b, n16, chunk16);
    else if (tiled) hipLaunchKernelGGL((chunk_probe_kernel<false, true>), dim3(grid), dim3(512), 0, s, b, n16, chunk16);
    else hipLaunchKernelGGL((chunk_probe_kernel<false, false>), dim3(grid), dim3(512), 0, s, b, n16, chunk16);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : (int)e;
  }
  hipStream_t s = (hipStream_t)stream;
  const int64_t n16 = bytes / 16;
  const unsigned grid = (unsigned)(8 * device_cus());
  u32x4_t* b = (u32x4_t*)buf;
  if (write && nt) hipLaunchKernelGGL((stream_probe_kernel<true, true>), dim3(grid), dim3(256), 0, s, b, n16);
  else if (write) hipLaunchKernelGGL((stream_probe_kernel<true, false>), dim3(grid), dim3(256), 0, s, b, n16);
  else if (nt) hipLaunchKernelGGL((stream_probe_kernel<false, true>), dim3(grid), dim3(256), 0, s, b, n16);
  else hipLaunchKernelGGL((stream_probe_kernel<false, false>), dim3(grid), dim3(256), 0, s, b, n16);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : (int)e;
}

}  // namespace gdnr
