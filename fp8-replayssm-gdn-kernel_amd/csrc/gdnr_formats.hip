// gdnr_formats.hip -- every checkpoint format of the reference's quantiser on
// gfx950: head, row, tile and vblock granularity, fp8 e4m3fn or int8 codes
// (prototype/gdn_replay_fp8_reference.py:36-37,40-106 quantise, :109-134
// dequantise), for a per-layer choice of format. The decode path itself
// reads vblock/32 fp8 (gdnr_kernels.hip has the fast vblock32 quantiser);
// these kernels build and read the other formats.
//
// A scale group is the set of state elements that share one scale:
//   head    rows [0, V)           x columns [0, K)
//   row     row r                 x columns [0, K)
//   tile    rows [i t, (i+1) t)   x columns [j t, (j+1) t)
//   vblock  rows [i t, (i+1) t)   x columns [0, K)
// Quantise: amax = max |x| over the group (NaN propagates), s = amax / qmax
// (qmax 448, or 127 for int8), 1 when amax is not > 0; the stored scale is
// fp16(s). The codes divide by the UNROUNDED s for tile and vblock and by the
// fp16-rounded scale for head and row, as the reference does (ref:83-94).
// fp8: clamp to +-448 keeping NaN, round to nearest even, NaN -> 0x7F|sign.
// int8: round half to even, clamp to +-127, NaN -> 0.
// Dequantise: code * float(stored scale).
//
// Not on the decode path: one workgroup per scale group, two passes over its
// elements (amax, then codes), byte stores.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gdnr_device.h"
#include "gdnr_internal.h"

namespace gdnr {
namespace {

struct Group {
  int r0, c0, R, C;  // rows [r0, r0 + R) x columns [c0, c0 + C) of the head
  int gi, gj;        // index of the group's scale along the scale's last two dims
};

__device__ __forceinline__ Group group_of(const FormatArgs& a, int g) {
  Group q;
  switch (a.gran) {
    case kGranHead: q = {0, 0, a.V, a.K, 0, 0}; break;
    case kGranRow: q = {g, 0, 1, a.K, g, 0}; break;
    case kGranTile: {
      const int nc = a.K / a.tile, i = g / nc, j = g - i * nc;
      q = {i * a.tile, j * a.tile, a.tile, a.tile, i, j};
      break;
    }
    default: q = {g * a.tile, 0, a.tile, a.K, g, 0}; break;  // vblock
  }
  return q;
}

__device__ __forceinline__ int groups_per_head(const FormatArgs& a) {
  switch (a.gran) {
    case kGranHead: return 1;
    case kGranRow: return a.V;
    case kGranTile: return (a.V / a.tile) * (a.K / a.tile);
    default: return a.V / a.tile;
  }
}

__global__ __launch_bounds__(256) void format_quantize_kernel(const FormatArgs a) {
  __shared__ uint32_t red[4];
  __shared__ int red_sat[4];
  const int gph = groups_per_head(a);
  const int64_t item = blockIdx.x;  // (b, hv, group)
  const int g = (int)(item % gph);
  const int hv = (int)((item / gph) % a.HV);
  const int b = (int)(item / ((int64_t)gph * a.HV));
  const Group q = group_of(a, g);
  const float* src = a.state + (int64_t)b * a.st_b + (int64_t)hv * a.st_h;
  const int n = q.R * q.C;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // pass 1: max |x| as bits (NaN above every finite value)
  uint32_t am = 0;
  for (int e = threadIdx.x; e < n; e += 256) {
    const int r = e / q.C, c = e - r * q.C;
    am = max(am, __float_as_uint(src[(int64_t)(q.r0 + r) * a.st_v + q.c0 + c]) & 0x7FFFFFFFu);
  }
  am = wave_max_u32(am);
  if (lane == 0) red[wave] = am;
  __syncthreads();
  am = max(max(red[0], red[1]), max(red[2], red[3]));
  const float qmax = a.int8 ? 127.0f : 448.0f;
  const float amax = __uint_as_float(am);
  const float s32 = (amax > 0.0f) ? amax / qmax : 1.0f;
  const float s16 = (float)(_Float16)s32;
  const float div = (a.gran == kGranHead || a.gran == kGranRow) ? s16 : s32;
  // pass 2: codes
  int sat = 0;
  uint8_t* dst = (uint8_t*)a.payload + (int64_t)b * a.pl_b + (int64_t)hv * a.pl_h;
  for (int e = threadIdx.x; e < n; e += 256) {
    const int r = e / q.C, c = e - r * q.C;
    const int64_t row = q.r0 + r;
    const float y = src[row * a.st_v + q.c0 + c] / div;
    sat += fabsf(y) > qmax ? 1 : 0;
    uint8_t code;
    if (a.int8) {
      const float t = rintf(y);
      code = (uint8_t)(int8_t)(int)((t != t) ? 0.0f : fminf(fmaxf(t, -127.0f), 127.0f));
    } else {
      code = (uint8_t)(f32x4_to_fp8_ref(y, 0.0f, 0.0f, 0.0f) & 0xFFu);
    }
    dst[row * a.pl_v + q.c0 + c] = code;
  }
  sat = wave_sum_i32(sat);
  if (lane == 0) red_sat[wave] = sat;
  __syncthreads();
  if (threadIdx.x == 0) {
    const int64_t so = (int64_t)b * a.sc_b + (int64_t)hv * a.sc_h + (int64_t)q.gi * a.sc_r + (int64_t)q.gj * a.sc_c;
    if (a.scale_dt == DT_F32) ((float*)a.scale)[so] = s16;
    else ((_Float16*)a.scale)[so] = (_Float16)s32;
    if (a.saturated)
      a.saturated[(int64_t)b * a.sa_b + (int64_t)hv * a.sa_h + (int64_t)q.gi * a.sa_r + (int64_t)q.gj * a.sa_c] =
          red_sat[0] + red_sat[1] + red_sat[2] + red_sat[3];
  }
}

__global__ __launch_bounds__(256) void format_dequantize_kernel(const FormatArgs a) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)a.B * a.HV * a.V * a.K;
  if (e >= total) return;
  const int c = (int)(e % a.K);
  const int r = (int)((e / a.K) % a.V);
  const int hv = (int)((e / ((int64_t)a.K * a.V)) % a.HV);
  const int b = (int)(e / ((int64_t)a.K * a.V * a.HV));
  int64_t so;
  switch (a.gran) {
    case kGranHead: so = 0; break;
    case kGranRow: so = (int64_t)r * a.sc_r; break;
    case kGranTile: so = (int64_t)(r / a.tile) * a.sc_r + (int64_t)(c / a.tile) * a.sc_c; break;
    default: so = (int64_t)(r / a.tile) * a.sc_r; break;
  }
  so += (int64_t)b * a.sc_b + (int64_t)hv * a.sc_h;
  const float sc = a.scale_dt == DT_F32 ? ((const float*)a.scale)[so] : (float)((const _Float16*)a.scale)[so];
  const uint8_t code = ((const uint8_t*)a.payload)[(int64_t)b * a.pl_b + (int64_t)hv * a.pl_h + (int64_t)r * a.pl_v + c];
  float x;
  if (a.int8) {
    x = (float)(int8_t)code;
  } else {
    float f[4];
    fp8x4_to_f32((uint32_t)code, f);
    x = f[0];
  }
  ((float*)a.state)[(int64_t)b * a.st_b + (int64_t)hv * a.st_h + (int64_t)r * a.st_v + c] = x * sc;
}

}  // namespace

int launch_format_quantize(const FormatArgs& a, void* stream) {
  int gph;
  switch (a.gran) {
    case kGranHead: gph = 1; break;
    case kGranRow: gph = a.V; break;
    case kGranTile: gph = (a.V / a.tile) * (a.K / a.tile); break;
    default: gph = a.V / a.tile; break;
  }
  const int64_t groups = (int64_t)a.B * a.HV * gph;
  hipLaunchKernelGGL(format_quantize_kernel, dim3((unsigned)groups), dim3(256), 0, (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

int launch_format_dequantize(const FormatArgs& a, void* stream) {
  const int64_t total = (int64_t)a.B * a.HV * a.V * a.K;
  hipLaunchKernelGGL(format_dequantize_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

}  // namespace gdnr
