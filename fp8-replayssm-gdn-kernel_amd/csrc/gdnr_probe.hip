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

}  // namespace

int launch_stream_probe(void* buf, int64_t bytes, bool write, bool nt, void* stream) {
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
