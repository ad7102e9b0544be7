// gdnr_device.h -- gfx950 device helpers: storage formats, fp8 conversion,
// DPP cross-lane reductions, explicit s_waitcnt.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gdnr_internal.h"

namespace gdnr {

typedef __attribute__((address_space(3))) void lds_void_t;

// ---------------------------------------------------------------- formats
__device__ __forceinline__ float bf16_to_f32(uint32_t bits) { return __uint_as_float(bits << 16); }

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// float pair -> packed bfloat16 bits (lo in bits 0-15): one gfx950
// v_cvt_pk_bf16_f32, round-to-nearest-even, NaN quietened -- torch's rule.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
// float -> bfloat16 bits (same conversion, one value).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}

// Storage traits of the activation dtype (q, k/v rings, out, mixed_qkv).
// Raw-bit access (``Bits``/``Pair``): loads that stay unconverted until the
// value is needed (see replay_kernel's step 2).
struct ActBF16 {
  static constexpr int kBytes = 2;
  using Bits = uint16_t;
  using Pair = uint32_t;
  __device__ static Bits ld_bits(const void* p, int64_t i) { return ((const uint16_t*)p)[i]; }
  __device__ static float from_bits(uint32_t b) { return bf16_to_f32(b & 0xFFFFu); }
  __device__ static Pair ld_pair_bits(const void* p) { return *(const uint32_t*)p; }
  __device__ static float2 from_pair(Pair w) { return make_float2(bf16_to_f32(w & 0xFFFFu), bf16_to_f32(w >> 16)); }
  __device__ static float ld(const void* p, int64_t i) { return bf16_to_f32(((const uint16_t*)p)[i]); }
  __device__ static void st(void* p, int64_t i, float x) { ((uint16_t*)p)[i] = (uint16_t)f32_to_bf16(x); }
  __device__ static float round(float x) { return bf16_to_f32(f32_to_bf16(x)); }
  // two consecutive elements starting at byte address p (4-byte aligned)
  __device__ static float2 ld2(const void* p) {
    uint32_t w = *(const uint32_t*)p;
    return make_float2(bf16_to_f32(w & 0xFFFFu), bf16_to_f32(w >> 16));
  }
  __device__ static void st2(void* p, float x, float y) { *(uint32_t*)p = pack_bf16x2(x, y); }
  // 16 consecutive elements at byte address p (16-byte aligned)
  __device__ static void ld16(const void* p, float* f) {
    const uint4* q = (const uint4*)p;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      uint4 w = q[i];
      uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f[8 * i + 2 * j] = bf16_to_f32(ws[j] & 0xFFFFu);
        f[8 * i + 2 * j + 1] = bf16_to_f32(ws[j] >> 16);
      }
    }
  }
};

struct ActF16 {
  static constexpr int kBytes = 2;
  using Bits = uint16_t;
  using Pair = uint32_t;
  __device__ static Bits ld_bits(const void* p, int64_t i) { return ((const uint16_t*)p)[i]; }
  __device__ static float from_bits(uint32_t b) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(b & 0xFFFFu)); }
  __device__ static Pair ld_pair_bits(const void* p) { return *(const uint32_t*)p; }
  __device__ static float2 from_pair(Pair w) { return make_float2(from_bits(w), from_bits(w >> 16)); }
  __device__ static float ld(const void* p, int64_t i) { return (float)((const _Float16*)p)[i]; }
  __device__ static void st(void* p, int64_t i, float x) { ((_Float16*)p)[i] = (_Float16)x; }
  __device__ static float round(float x) { return (float)(_Float16)x; }
  __device__ static float2 ld2(const void* p) {
    const _Float16* h = (const _Float16*)p;
    return make_float2((float)h[0], (float)h[1]);
  }
  __device__ static void st2(void* p, float x, float y) {
    _Float16* h = (_Float16*)p;
    h[0] = (_Float16)x;
    h[1] = (_Float16)y;
  }
  __device__ static void ld16(const void* p, float* f) {
    const _Float16* h = (const _Float16*)p;
#pragma unroll
    for (int i = 0; i < 16; ++i) f[i] = (float)h[i];
  }
};

struct ActF32 {
  static constexpr int kBytes = 4;
  using Bits = uint32_t;
  using Pair = uint2;
  __device__ static Bits ld_bits(const void* p, int64_t i) { return ((const uint32_t*)p)[i]; }
  __device__ static float from_bits(uint32_t b) { return __uint_as_float(b); }
  __device__ static Pair ld_pair_bits(const void* p) { return *(const uint2*)p; }
  __device__ static float2 from_pair(Pair w) { return make_float2(__uint_as_float(w.x), __uint_as_float(w.y)); }
  __device__ static float ld(const void* p, int64_t i) { return ((const float*)p)[i]; }
  __device__ static void st(void* p, int64_t i, float x) { ((float*)p)[i] = x; }
  __device__ static float round(float x) { return x; }
  __device__ static float2 ld2(const void* p) { return *(const float2*)p; }
  __device__ static void st2(void* p, float x, float y) { *(float2*)p = make_float2(x, y); }
  __device__ static void ld16(const void* p, float* f) {
    const float4* q = (const float4*)p;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float4 w = q[i];
      f[4 * i] = w.x;
      f[4 * i + 1] = w.y;
      f[4 * i + 2] = w.z;
      f[4 * i + 3] = w.w;
    }
  }
};

// Runtime-typed scalar access (gating scalars, a/b, A_log, dt_bias, scales).
__device__ __forceinline__ float ld_dt(const void* p, int64_t i, int dt) {
  if (dt == DT_BF16) return bf16_to_f32(((const uint16_t*)p)[i]);
  if (dt == DT_F16) return (float)((const _Float16*)p)[i];
  return ((const float*)p)[i];
}
__device__ __forceinline__ void st_dt(void* p, int64_t i, int dt, float x) {
  if (dt == DT_BF16) ((uint16_t*)p)[i] = (uint16_t)f32_to_bf16(x);
  else if (dt == DT_F16) ((_Float16*)p)[i] = (_Float16)x;
  else ((float*)p)[i] = x;
}
__device__ __forceinline__ float round_dt(float x, int dt) {
  if (dt == DT_BF16) return bf16_to_f32(f32_to_bf16(x));
  if (dt == DT_F16) return (float)(_Float16)x;
  return x;
}
__device__ __forceinline__ int64_t ld_int(const void* p, int64_t i, int dt) {
  if (dt == DT_I64) return ((const int64_t*)p)[i];
  if (dt == DT_I32) return ((const int32_t*)p)[i];
  return ((const uint8_t*)p)[i];  // bool / u8
}

// ---------------------------------------------------------------- fp8 (OCP e4m3fn on gfx950)
// 4 packed codes -> 4 floats (byte 0 first).
__device__ __forceinline__ void fp8x4_to_f32(uint32_t w, float* f) {
  auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  f[0] = lo[0];
  f[1] = lo[1];
  f[2] = hi[0];
  f[3] = hi[1];
}
// 4 e4m3 codes -> 4 bf16 values, packed in pairs (codes 0, 1 | codes 2, 3):
// every e4m3 value, subnormals included, is exact in bf16; scale 1.0 makes
// the scaled convert a plain one.
__device__ __forceinline__ uint2 fp8x4_to_bf16x4(uint32_t w) {
  return make_uint2(__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false)),
                    __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true)));
}
// the same for f16 (every e4m3 value is exact in f16)
__device__ __forceinline__ uint2 fp8x4_to_f16x4(uint32_t w) {
  return make_uint2(__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false)),
                    __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true)));
}
// 4 floats -> 4 packed codes, round-to-nearest-even (inputs already clamped).
__device__ __forceinline__ uint32_t f32x4_to_fp8(float a, float b, float c, float d) {
  // (the first convert writes bytes 0-1 and keeps the word's other half,
  // which the second overwrites: a's bits as that half spare a register copy)
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, __float_as_int(a), false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}
// clamp to the e4m3fn range, keeping NaN (torch.clamp propagates NaN).
__device__ __forceinline__ float clamp448(float x) {
  return (x != x) ? x : fminf(fmaxf(x, -448.0f), 448.0f);
}
// 4 floats -> 4 codes exactly as the reference's clamp + e4m3fn cast writes
// them, for any input: clamp to +-448 keeping NaN, round to nearest even, NaN
// -> 0x7F | sign (the convert instruction writes 0xFF for every NaN).
__device__ __forceinline__ uint32_t f32x4_to_fp8_ref(float a, float b, float c, float d) {
  uint32_t w = f32x4_to_fp8(clamp448(a), clamp448(b), clamp448(c), clamp448(d));
  const float v[4] = {a, b, c, d};
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (v[e] != v[e]) w = (w & ~(0xFFu << (8 * e))) | ((__float_as_uint(v[e]) >> 31 ? 0xFFu : 0x7Fu) << (8 * e));
  return w;
}

// Quantiser quotient: the correctly rounded x / s (what IEEE division gives)
// from r = RN(1/s), in 5 VALU operations instead of the division sequence.
// q0 = RN(x r) is within 1.5 ulp of x / s; a correction with the residual
// x - s q (exact by FMA) brings it within 1 ulp, and a second correction is
// correctly rounded (Markstein's theorem: r within 1/2 ulp of 1/s, q within
// 1 ulp of x / s, no underflow or overflow). Callers use it only when the
// block's amax is finite and s >= 2^-64, so |x / s| <= 448 (1 + 2^-23) and
// every quotient the fp8 code depends on (|x / s| >= 2^-10) is a normal
// number. The residual is formed negated, d = s q - x: a zero quotient then
// keeps the sign of x (q - d r with d = +0 is q itself), as IEEE division
// keeps it, with no separate sign fix.
__device__ __forceinline__ float quotient_rn(float x, float s, float r) {
  float q = x * r;
  q = fmaf(-fmaf(q, s, -x), r, q);
  q = fmaf(-fmaf(q, s, -x), r, q);
  return q;
}
// The same correctly rounded x / s from one double product, r64 = RN64(1 / s):
// q = RN32(RN64(x r64)). The double product is within 2^-52 (relative) of
// x / s. Where x / s is a normal float it is a quotient of two 24-bit
// significands, which is never an f32 rounding midpoint and lies at least
// 2^-50 (relative) from every one (|x - s m| >= 2^(a - 26) for x = X 2^a and
// any midpoint m within a factor 2 of x / s), so the product rounds to the
// same float. Smaller quotients (|x / s| < 2^-126) round to +-0 in e4m3 either
// way, with the sign of x. Used under the same conditions as quotient_rn.
__device__ __forceinline__ float quotient_f64(float x, double r64) { return (float)((double)x * r64); }
// Whether a block with this amax (bits of |x| max) and scale takes quotient_rn:
// amax finite and s >= 2^-64.
__device__ __forceinline__ bool quotient_fast(uint32_t amax_bits, float s) {
  return amax_bits < 0x7F800000u && s >= 0x1p-64f;
}

// ---------------------------------------------------------------- cross-lane (DPP, wave64)
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, ROW_MASK, 0xF, false));
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_u(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, ROW_MASK, 0xF, false);
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7-i within 8
constexpr int kDppMirror = 0x140;     // lane i <-> 15-i within 16
constexpr int kDppBcast15 = 0x142;
constexpr int kDppBcast31 = 0x143;

// every lane of each aligned 8-lane group receives the group sum
__device__ __forceinline__ float sum8(float x) {
  x += dpp_f<kDppXor1>(x);
  x += dpp_f<kDppXor2>(x);
  x += dpp_f<kDppHalfMirror>(x);
  return x;
}
__device__ __forceinline__ float readlane_f(float x, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
}
// wave-uniform sum of all 64 lanes
__device__ __forceinline__ float wave_sum(float x) {
  x = sum8(x);
  x += dpp_f<kDppMirror>(x);
  x += dpp_f<kDppBcast15, 0xA>(x);
  x += dpp_f<kDppBcast31, 0xC>(x);
  return readlane_f(x, 63);
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
  x = max(x, dpp_u<kDppXor1>(x));
  x = max(x, dpp_u<kDppXor2>(x));
  x = max(x, dpp_u<kDppHalfMirror>(x));
  x = max(x, dpp_u<kDppMirror>(x));
  x = max(x, dpp_u<kDppBcast15, 0xA>(x));
  x = max(x, dpp_u<kDppBcast31, 0xC>(x));
  return (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
}
__device__ __forceinline__ int wave_sum_i32(int x) {
  x += (int)dpp_u<kDppXor1>((uint32_t)x);
  x += (int)dpp_u<kDppXor2>((uint32_t)x);
  x += (int)dpp_u<kDppHalfMirror>((uint32_t)x);
  x += (int)dpp_u<kDppMirror>((uint32_t)x);
  x += (int)dpp_u<kDppBcast15, 0xA>((uint32_t)x);
  x += (int)dpp_u<kDppBcast31, 0xC>((uint32_t)x);
  return __builtin_amdgcn_readlane(x, 63);
}

// ---------------------------------------------------------------- LDS flags
// Acquire-load of an LDS flag, made wave-uniform: every lane reads the same
// word, and a uniform loop exit keeps the polling loops out of the CFG
// structurizer (which would otherwise merge the code after them).
__device__ __forceinline__ bool flag_set(int* f) {
  return __builtin_amdgcn_readfirstlane(__hip_atomic_load(f, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP)) != 0;
}
// bounded wait for an LDS flag, at most `polls` polls (kWaitPolls unless
// the host set another budget: gdnr_set_wait_polls); a wait that gives up
// is counted in the device status word (gdnr_wait_timeouts) and reported to
// the caller, which then skips its in-place checkpoint stores
__device__ __forceinline__ bool wait_flag(int* f, uint32_t* status, uint32_t polls) {
  for (uint32_t it = 0; it < polls; ++it) {
    if (flag_set(f)) return true;
    __builtin_amdgcn_s_sleep(1);
  }
  if ((threadIdx.x & 63) == 0 && status) atomicAdd(status, 1u);
  return false;
}

// bounded wait for an LDS counter to reach `target` (counted like wait_flag)
__device__ __forceinline__ bool wait_count(int* f, int target, uint32_t* status, uint32_t polls) {
  for (uint32_t it = 0; it < polls; ++it) {
    if (__builtin_amdgcn_readfirstlane(__hip_atomic_load(f, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP)) >= target)
      return true;
    __builtin_amdgcn_s_sleep(1);
  }
  if ((threadIdx.x & 63) == 0 && status) atomicAdd(status, 1u);
  return false;
}

// ---------------------------------------------------------------- waits
// s_waitcnt immediate (gfx9): vmcnt[3:0] + vmcnt_hi[15:14], expcnt[6:4], lgkmcnt[11:8].
#define GDNR_WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt((((n) & 0xF) | ((((n) >> 4) & 0x3) << 14) | (0x7 << 4) | (0xF << 8)))
#define GDNR_WAIT_LGKM0() __builtin_amdgcn_s_waitcnt((0xF) | (0x3 << 14) | (0x7 << 4) | (0x0 << 8))
// Scheduling barrier (no memory semantics): keeps instruction order across it.
#define GDNR_COMPILER_FENCE() __builtin_amdgcn_sched_barrier(0)


}  // namespace gdnr
