// gdnr_step.hip -- one ReplaySSM decode step on gfx950 (MI355X) for rings of
// up to 16 tokens: replay or flush per sequence, optionally fused with the
// full-contract preparation of the new token.
//
// Grid: x = V-tile + n_vt * (value-head group within the key head), y = key
// head h, z = sequence b (no integer division on the way to the first load).
// Workgroup = gw value heads sharing key head h, block_v V-rows of each, and
// two waves per head:
//   lead j (wave j): loads its share of the k ring (all L slots split over
//     the leads by direct-to-LDS DMA; slots beyond the fill are read and
//     ignored), q and the gates; prepares the new token (fused), forms the
//     Gram matrix and the coefficient chain of head j (c_t and T0 of a
//     replay, the rebuild factors of a flush) and publishes them through an
//     LDS flag. It loads no checkpoint row: a wave whose loads back up in the
//     memory pipeline cannot issue anything else, and the checkpoint stream
//     would stall the chain.
//   streamer j (wave gw + j): waits until the whole k ring has landed, then
//     requests the v rows of head j and its block_v checkpoint rows -- vblock
//     scales and NCH = block_v / 8 loads of 16 bytes a lane in the MFMA
//     operand layout (lane (l16, q4) of 16-row block i holds row l16, bytes
//     [16 q4, +16) and [64 + 16 q4, +16)), which serves both the replay
//     matvec and the flush rebuild. It stages the v rows in LDS, waits for the
//     coefficients, folds w = sum_t c_t v_t, emits its rows and appends the
//     new token. A flush splits the head's vblocks between the streamer and
//     the lead once both have published.
//
// Replay, the adjoint of the reference's reverse chain
// (prototype/gdn_replayssm_fp8_kernel.py:121-173), in Gram form:
//   dq_t = k_t.q, G_tu = k_t.k_u                   (MFMA Gram matrix of [K; q])
//   s_t  = beta_t (dq_t - sum_{u>t} G_tu s_u)       (t descending)
//   c_t  = s_t prod_{u>t} gamma_u,  T0 = prod_u gamma_u (q - sum_t s_t k_t)
//   o    = ((scale * codes) . T0 + sum_t c_t v_t) K^-1/2
// Flush: the forward rebuild in matrix form on MFMA (section 7), o from the
// rebuilt state, requantisation in place.
//
// LDS: the k ring is stored with an XOR swizzle of 16-byte chunks (chunk c of
// token t at position c ^ (t & 15)) so that operand reads of 16 different
// tokens at one column hit 16 different bank groups. The new token's k lives
// in a row of its own: the ring DMA of its slot may land after it is written.
//
// Compiled once per activation dtype (GDNR_ACT = 0 bf16, 1 f16, 2 f32).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "gdnr_device.h"
#include "gdnr_internal.h"

#ifndef GDNR_ACT
#error "compile with -DGDNR_ACT=0|1|2"
#endif

namespace gdnr {
namespace {

constexpr int K = kKeyDim;
constexpr int LP = kStepRing;  // ring capacity of this kernel: one 16-token block

typedef short bf16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));  // 16-byte chunk as a native vector (no memcpy)

__device__ __forceinline__ float readlane_fv(float x, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
// Opaque copy: values derived from the result are recomputed inside the loop
// that makes the copy instead of being hoisted out of it (and spilled).
__device__ __forceinline__ uint32_t opaque(uint32_t x) {
  asm volatile("" : "+v"(x));
  return x;
}
// Loads at wave-uniform addresses of data the kernel does not write before
// reading it, through the scalar cache (constant address space): they count
// in lgkmcnt, so waiting for them never waits for the vector loads.
typedef __attribute__((address_space(4))) const uint32_t const_u32;
__device__ __forceinline__ uint32_t ld_u32_uniform(const void* p) { return *(const_u32*)p; }
// 16-bit value: the aligned dword holding it (allocations are at least 4-byte granular)
__device__ __forceinline__ uint32_t ld_u16_uniform(const uint16_t* p) {
  const uintptr_t ad = (uintptr_t)p;
  return (ld_u32_uniform((const void*)(ad & ~(uintptr_t)3)) >> (8u * (uint32_t)(ad & 2))) & 0xFFFFu;
}
// DPP move within a 16-lane row; lanes whose source is outside the row get `fill`.
template <int CTRL>
__device__ __forceinline__ float dpp_row(float x, float fill) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, fill), __builtin_bit_cast(int, x),
                                                               CTRL, 0xF, 0xF, false));
}
// inclusive prefix / suffix products over the lanes of each 16-lane row
__device__ __forceinline__ float row_prefix_prod(float x) {
  x *= dpp_row<0x111>(x, 1.f);  // row_shr:1
  x *= dpp_row<0x112>(x, 1.f);  // row_shr:2
  x *= dpp_row<0x114>(x, 1.f);  // row_shr:4
  x *= dpp_row<0x118>(x, 1.f);  // row_shr:8
  return x;
}
__device__ __forceinline__ float row_suffix_prod(float x) {
  x *= dpp_row<0x101>(x, 1.f);  // row_shl:1
  x *= dpp_row<0x102>(x, 1.f);  // row_shl:2
  x *= dpp_row<0x104>(x, 1.f);  // row_shl:4
  x *= dpp_row<0x108>(x, 1.f);  // row_shl:8
  return x;
}

// the workgroup's dynamic LDS (layout in StepArgs: lds_* byte offsets)
extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

// byte offset of byte `by` of token t's row in the swizzled k ring (ROWB = K * ES)
template <int ROWB>
__device__ __forceinline__ int kr_off(int t, int by) {
  return t * ROWB + ((((by >> 4) ^ (t & 15))) << 4) + (by & 15);
}

// Rows of X = [k_0 .. k_{n-1}, q]: LDS byte address of byte `by` of row x
// (x < n: the ring, or the new token's own row at x == pos; x >= n: q).
// Rows beyond n are zeroed by the callers.
struct XRows {
  int lds_k, lds_knew, lds_q, n, pos;
  template <int ROWB>
  __device__ __forceinline__ int off(int x, int by) const {
    return x < n ? (x == pos ? lds_knew + by : lds_k + kr_off<ROWB>(x, by)) : lds_q + by;
  }
};

template <int ROWB>
__device__ __forceinline__ int xr_off_row(int lds_k, int lds_knew, int lds_q, int x, int n, int pos, int by) {
  return x < n ? (x == pos ? lds_knew + by : lds_k + kr_off<ROWB>(x, by)) : lds_q + by;
}

// raw bits of a gating input (f32, or the activation dtype) and their value
template <bool GATE_F32, class Act>
__device__ __forceinline__ uint32_t ld_gate_bits(const uint8_t* p) {
  if constexpr (GATE_F32) return *(const uint32_t*)p;
  else return (uint32_t)Act::ld_bits(p, 0);
}
template <bool GATE_F32, class Act>
__device__ __forceinline__ float gate_value(uint32_t bits) {
  if constexpr (GATE_F32) return __uint_as_float(bits);
  else return Act::from_bits(bits);
}

// ---- flush (section 7), out of line: the rebuild's register pressure stays
// out of the replay path's allocation. Every operand is wave-uniform; the
// call passes them one by one in VGPRs (a struct would go through the stack),
// so they are made uniform again on entry.
struct FlushArgs {
  uint8_t* ck_rows;   // the head's checkpoint rows (block_v rows of ck_v bytes)
  uint8_t* scale_hv;  // the head's vblock scales
  uint8_t* out_rows;  // the head's output rows
  uint32_t ck_v, sc_v;  // row / vblock byte strides
  int32_t sc_row0;      // first vblock of the rows
  float out_scale;
  int32_t lds_k, lds_knew, lds_q, lds_r, lds_fac, lds_lam, lds_kt, vbuf;
  int32_t lds_xam;  // amax exchange of the head: [block][vblock] words
  int32_t j_head, n, pos, mm, nvb;  // head, ring fill, new slot, 16-row block of each vblock, vblocks
};

__device__ __forceinline__ int32_t uni(int32_t x) { return __builtin_amdgcn_readfirstlane(x); }
// global-memory view of a pointer passed as a generic one (the callee would
// otherwise access it with flat instructions, which count in both wait counters)
template <class T>
__device__ __forceinline__ __attribute__((address_space(1))) T* gptr(const void* p) {
  return (__attribute__((address_space(1))) T*)p;
}
__device__ __forceinline__ uint8_t* uni(uint8_t* p) {
  const uint64_t v = (uint64_t)p;
  return (uint8_t*)(((uint64_t)(uint32_t)uni((int32_t)(v >> 32)) << 32) | (uint32_t)uni((int32_t)v));
}

// The two waves of a head rebuild one 16-row block each (mm = 0 streamer,
// mm = 1 lead) of every vblock of the head, and exchange the block amax per
// vblock through LDS: a word per (block, vblock), cleared at kernel start,
// written once as amax bits | 2^31 (amax bits are below 2^31).
template <class Act, int NCH>
__device__ __attribute__((noinline)) void flush_vblocks(
    uint8_t* f_ck_rows, uint8_t* f_scale_hv, uint8_t* f_out_rows, uint32_t f_ck_v, uint32_t f_sc_v, int32_t f_sc_row0,
    float f_out_scale, int32_t f_lds_k, int32_t f_lds_knew, int32_t f_lds_q, int32_t f_lds_r, int32_t f_lds_fac,
    int32_t f_lds_lam, int32_t f_lds_kt, int32_t f_vbuf, int32_t f_lds_xam, int32_t f_j_head, int32_t f_n,
    int32_t f_pos, int32_t f_mm, int32_t f_nvb, uint32_t* f_status, uint32_t f_polls, bool f_ok) {
  FlushArgs f{f_ck_rows, f_scale_hv, f_out_rows, f_ck_v,  f_sc_v,    f_sc_row0, f_out_scale, f_lds_k,
              f_lds_knew, f_lds_q,   f_lds_r,  f_lds_fac, f_lds_lam, f_lds_kt,  f_vbuf,      f_lds_xam,
              f_j_head,   f_n,       f_pos,    f_mm,      f_nvb};
  constexpr int ES = Act::kBytes;
  constexpr int ROWB = K * ES;
  constexpr int RPW = 8 * NCH;
  constexpr bool BF16 = std::is_same<Act, ActBF16>::value;
  constexpr bool F16 = std::is_same<Act, ActF16>::value;
  const int lane = threadIdx.x & 63;
  const int q4 = lane >> 4, l16 = lane & 15;
  const int j_head = uni(f.j_head), n = uni(f.n), pos = uni(f.pos), mm = uni(f.mm), nvb = uni(f.nvb);
  const uint32_t ck_v = (uint32_t)uni((int32_t)f.ck_v), sc_v = (uint32_t)uni((int32_t)f.sc_v);
  f.sc_row0 = uni(f.sc_row0), f.lds_k = uni(f.lds_k), f.lds_knew = uni(f.lds_knew), f.lds_q = uni(f.lds_q);
  f.lds_r = uni(f.lds_r), f.lds_fac = uni(f.lds_fac), f.lds_lam = uni(f.lds_lam), f.lds_kt = uni(f.lds_kt);
  f.lds_xam = uni(f.lds_xam);
  f.out_scale = __builtin_bit_cast(float, uni(__builtin_bit_cast(int32_t, f.out_scale)));
  uint8_t* ck_rows = uni(f.ck_rows);
  uint8_t* scale_hv = uni(f.scale_hv);
  uint8_t* out_rows = uni(f.out_rows);
  const uint8_t* vbuf = lds + uni(f.vbuf);
  const uint32_t ck_lo = (uint32_t)l16 * ck_v + 16 * q4;
  const XRows xr{f.lds_k, f.lds_knew, f.lds_q, n, pos};
  int* xam_mine = (int*)(lds + f.lds_xam) + mm * kMaxVBlocks;
  int* xam_other = (int*)(lds + f.lds_xam) + (1 - mm) * kMaxVBlocks;
  // Per vblock p, block mm (rows 32 p + 16 mm + [0, 16)): lane l owns row
  // l % 16; the contraction walks the columns in the order of ck, so every
  // checkpoint operand comes straight from those registers and the
  // requantised codes go back as the same two 16-byte words.
  //   A.  P^T = [K; q] S_0^T          (tokens x rows; the q row gives S_0 q)
  //       W^T = v - pre . P^T
  //   B.  U^T = R W^T,  U~^T = post . U^T,  o = lam_all S_0 q + sum_t U~^T[t] (k_t . q)
  //   C.  S_n^T = lam_all S_0^T + K^T U~^T
  // The accumulator of each step is, lane for lane, the B operand of the next
  // (lane (l16, q4) holds tokens 4 q4 + e of row l16), so W^T and U~^T stay
  // in registers. Then the vblock amax (this block's and the other wave's)
  // and the requantisation of this block.
  {
    const float* Rj = (const float*)(lds + f.lds_r) + j_head * LP * LP;
    const float4* fac = (const float4*)(lds + f.lds_fac) + j_head * LP;
    const float lam_all = ((const float*)(lds + f.lds_lam))[j_head];
    // codes of this block of vblock p: cf[hh] (the layout of ck); the next
    // vblock's are requested into the same registers as soon as the rebuild
    // has consumed them. The row pointer is laundered: the compiler must not
    // fold these loads into the replay's ck registers (that would keep all of
    // ck live through the rebuild).
    uint4 cf[2];
    const uint8_t* ck_rows_f = ck_rows;
    asm volatile("" : "+s"(ck_rows_f));
    auto load_blk = [&](int p) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const u32x4_t w = *gptr<const u32x4_t>(ck_rows_f + ((32 * p + 16 * mm) * ck_v + 64 * hh + ck_lo));
        cf[hh] = make_uint4(w[0], w[1], w[2], w[3]);
      }
    };
    load_blk(0);
    // the first codes are waited for here, outside the loop: a load pending
    // on entry to the loop would make its header wait for every store of the
    // previous vblock as well
    GDNR_WAIT_VMCNT(0);
#pragma unroll 1
    for (int p = 0; p < nvb; ++p) {
      const float sc = f16_bits_to_f32((uint16_t)ld_u16_uniform((const uint16_t*)(scale_hv + (f.sc_row0 + p) * sc_v)));
      const int rl = 32 * p + 16 * mm + l16;  // row within the head's rows
      const uint32_t cw[8] = {cf[0].x, cf[0].y, cf[0].z, cf[0].w, cf[1].x, cf[1].y, cf[1].z, cf[1].w};
      float o_part = 0.f;
      // the codes of the block as 16-bit MFMA B operands, once for A and C
      // (e4m3 values are exact in bf16 and f16): k-step m holds columns
      // 64 (m / 2) + 16 q4 + 8 (m % 2) + [0, 8), words 2m, 2m + 1
      uint4 bvs[4];
      if constexpr (BF16 || F16) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const uint2 b0 = BF16 ? fp8x4_to_bf16x4(cw[2 * m]) : fp8x4_to_f16x4(cw[2 * m]);
          const uint2 b1 = BF16 ? fp8x4_to_bf16x4(cw[2 * m + 1]) : fp8x4_to_f16x4(cw[2 * m + 1]);
          bvs[m] = make_uint4(b0.x, b0.y, b1.x, b1.y);
        }
        if (p + 1 < nvb) load_blk(p + 1);  // the codes of vblock p are consumed
      }
      // A: P^T of the token block (rows x >= n read the q row: row n is S_0 q,
      // the rows past it are never used) and W^T
      auto x_times_s0 = [&](auto row_off) {  // row_off(by): LDS offset of this lane's X row at byte by
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
        if constexpr (BF16 || F16) {
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            const uint4 av = *(const uint4*)(lds + row_off((64 * (m >> 1) + 16 * q4 + 8 * (m & 1)) * 2));
            if constexpr (BF16)
              acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av),
                                                            __builtin_bit_cast(bf16x8_t, bvs[m]), acc, 0, 0, 0);
            else
              acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, av),
                                                           __builtin_bit_cast(f16x8_t, bvs[m]), acc, 0, 0, 0);
          }
        } else {
#pragma unroll
          for (int kc = 0; kc < 8; ++kc) {
            const int col = 64 * (kc >> 2) + 16 * q4 + 4 * (kc & 3);
            float fa[4];
            fp8x4_to_f32(opaque(cw[kc]), fa);
#pragma unroll
            for (int e = 0; e < 4; ++e)
              acc = __builtin_amdgcn_mfma_f32_16x16x4f32(*(const float*)(lds + row_off((col + e) * 4)), fa[e], acc, 0,
                                                         0, 0);
          }
        }
        return acc;
      };
      float wv[4];
      {
        const f32x4_t acc = x_times_s0([&](int by) { return xr.off<ROWB>(l16, by); });
        // branch-free: every lane reads a valid token's v and factors
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int t = 4 * q4 + e;
          const bool tok = t < n;
          const int tc = tok ? t : 0;
          const float pv = acc[e] * sc;
          const float w = Act::ld(vbuf, tc * RPW + rl) - fac[tc].x * pv;
          wv[e] = tok ? w : 0.f;
          o_part = (t == n) ? fmaf(lam_all, pv, o_part) : o_part;
        }
      }
      if (n >= LP) {
        // a full ring: the q row is a block of its own (every row of it is S_0 q)
        const f32x4_t acc = x_times_s0([&](int by) { return f.lds_q + by; });
        if (q4 == 0) o_part = fmaf(lam_all, acc[0] * sc, o_part);
      }
      // B: U^T = R W^T (fp32 MFMA, contraction index q4 <-> token 4 q4 + e)
      uint4 packed;
      {
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
        const float* rrow = Rj + l16 * LP + 4 * q4;
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(rrow[0], wv[0], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(rrow[1], wv[1], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(rrow[2], wv[2], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(rrow[3], wv[3], acc, 0, 0, 0);
        float ut[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float4 fc = fac[4 * q4 + e];
          ut[e] = acc[e] * fc.y;
          o_part = fmaf(ut[e], fc.z, o_part);
        }
        if constexpr (BF16) {
          // hi/lo split: U~ = hi + lo to ~16 bits, both halves bf16 MFMA operands
          const uint32_t h01 = pack_bf16x2(ut[0], ut[1]), h23 = pack_bf16x2(ut[2], ut[3]);
          const uint32_t l01 =
              pack_bf16x2(ut[0] - __uint_as_float(h01 << 16), ut[1] - __uint_as_float(h01 & 0xFFFF0000u));
          const uint32_t l23 =
              pack_bf16x2(ut[2] - __uint_as_float(h23 << 16), ut[3] - __uint_as_float(h23 & 0xFFFF0000u));
          packed = make_uint4(h01, h23, l01, l23);
        } else {
          packed = make_uint4(__float_as_uint(ut[0]), __float_as_uint(ut[1]), __float_as_uint(ut[2]),
                              __float_as_uint(ut[3]));
        }
      }
      o_part += __shfl_xor(o_part, 16);
      o_part += __shfl_xor(o_part, 32);
      if (q4 == 0) {
        const float o = o_part * f.out_scale;
        if constexpr (ES == 4) *gptr<float>(out_rows + 4 * rl) = o;
        else if constexpr (BF16) *gptr<uint16_t>(out_rows + 2 * rl) = (uint16_t)f32_to_bf16(o);
        else *gptr<_Float16>(out_rows + 2 * rl) = (_Float16)o;
      }
      // C: S_n^T tiles sn[ct] (ct = 4 hh + w): D row 4 q4 + e of tile ct is
      // column 64 hh + 16 q4 + 4 w + e, and row l16 of K^T tile ct (the A
      // operand of lane l) holds that column ordering already.
      // bf16: lam_all scale S_0^T enters through the MFMA as (ls I) S_0^T with
      // ls = lam_all * scale split into bf16 hi + lo (relative error 2^-18).
      // Each hi/lo pair is one 16x16x32 MFMA: lane (l16, q4) supplies k-slots
      // 8 q4 + j, j < 4 the hi part and j >= 4 the lo part of token / column
      // 4 q4 + (j & 3) -- (ls_hi I | ls_lo I) against the codes twice, then
      // (K^T | K^T) against (U~_hi ; U~_lo)
      f32x4_t sn[8];
      if constexpr (BF16) {
        const float ls = lam_all * sc;
        const uint32_t hb = f32_to_bf16(ls);
        const uint32_t lb = f32_to_bf16(ls - __uint_as_float(hb << 16));
        short h4[4], l4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool diag = l16 == 4 * q4 + e;
          h4[e] = (short)(diag ? hb : 0u);
          l4[e] = (short)(diag ? lb : 0u);
        }
        const bf16x8_t a_ls = __builtin_bit_cast(
            bf16x8_t, (short __attribute__((ext_vector_type(8)))){h4[0], h4[1], h4[2], h4[3], l4[0], l4[1], l4[2], l4[3]});
#pragma unroll
        for (int ct = 0; ct < 8; ++ct) {
          const uint4 bv = bvs[ct >> 1];
          const uint2 c2 = (ct & 1) ? make_uint2(bv.z, bv.w) : make_uint2(bv.x, bv.y);
          const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
          sn[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              a_ls, __builtin_bit_cast(bf16x8_t, make_uint4(c2.x, c2.y, c2.x, c2.y)), z, 0, 0, 0);
        }
      } else {
#pragma unroll
        for (int ct = 0; ct < 8; ++ct) {
          float fc[4];
          fp8x4_to_f32(cw[ct], fc);
#pragma unroll
          for (int e = 0; e < 4; ++e) sn[ct][e] = lam_all * (fc[e] * sc);
        }
      }
      if constexpr (!(BF16 || F16))
        if (p + 1 < nvb) load_blk(p + 1);  // the codes of vblock p are consumed
      const uint8_t* kt_lane = lds + f.lds_kt + l16 * 16 * ES + 4 * q4 * ES;  // tokens 4 q4 + e
#pragma unroll
      for (int ct = 0; ct < 8; ++ct) {
        const uint8_t* ktrow = kt_lane + ct * 256 * ES;
        if constexpr (BF16) {
          const uint2 k2 = *(const uint2*)ktrow;
          sn[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, make_uint4(k2.x, k2.y, k2.x, k2.y)),
                                                           __builtin_bit_cast(bf16x8_t, packed), sn[ct], 0, 0, 0);
        } else {
          const float uf[4] = {__uint_as_float(packed.x), __uint_as_float(packed.y), __uint_as_float(packed.z),
                               __uint_as_float(packed.w)};
#pragma unroll
          for (int e = 0; e < 4; ++e)
            sn[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(Act::ld(ktrow, e), uf[e], sn[ct], 0, 0, 0);
        }
      }
      // |x| max of the block: one v_maximum3 per two values (IEEE maximum: NaN
      // propagates, like torch.amax); |x| bits order like the values, NaN
      // above every finite value
      float am = 0.f;
#pragma unroll
      for (int ct = 0; ct < 8; ++ct)
#pragma unroll
        for (int e = 0; e < 4; e += 2)
          am = __builtin_elementwise_maximum(__builtin_elementwise_maximum(am, __builtin_fabsf(sn[ct][e])),
                                             __builtin_fabsf(sn[ct][e + 1]));
      uint32_t amb = wave_max_u32(__float_as_uint(am));
      // the vblock amax: this block's and the other wave's (bounded wait: the
      // other wave posts every vblock before it waits for this one)
      __hip_atomic_store(xam_mine + p, (int)(amb | 0x80000000u), __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
      uint32_t other = 0;
      uint32_t it = 0;
      for (; it < f_polls; ++it) {
        other = (uint32_t)__builtin_amdgcn_readfirstlane(
            __hip_atomic_load(xam_other + p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP));
        if (other >> 31) break;
        __builtin_amdgcn_s_sleep(1);
      }
      if (it == f_polls) {
        if (lane == 0 && f_status) atomicAdd(f_status, 1u);
        f_ok = false;
      }
      amb = max(amb, other & 0x7FFFFFFFu);
      // requantisation (the reference quantiser, ref:36-37,83-99: s = amax/448,
      // 1 when amax is not > 0; codes = e4m3fn(clamp(x / s, +-448)) with the
      // unrounded fp32 s; the quotient by quotient_rn when the block is finite)
      const float amax = __uint_as_float(amb);
      const float s32 = (amax > 0.0f) ? amax / 448.0f : 1.0f;
      const bool fast = quotient_fast(amb, s32);
      const float rcp = 1.0f / s32;
      uint8_t* rp = ck_rows + ((32 * p + 16 * mm + l16) * ck_v + 16 * q4);
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        uint32_t wd[4];
        if (fast) {
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const f32x4_t& v = sn[4 * hh + w];
            wd[w] = f32x4_to_fp8(quotient_rn(v[0], s32, rcp), quotient_rn(v[1], s32, rcp),
                                 quotient_rn(v[2], s32, rcp), quotient_rn(v[3], s32, rcp));
          }
        } else {
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const f32x4_t& v = sn[4 * hh + w];
            wd[w] = f32x4_to_fp8_ref(v[0] / s32, v[1] / s32, v[2] / s32, v[3] / s32);
          }
        }
        if (f_ok) *gptr<u32x4_t>(rp + 64 * hh) = u32x4_t{wd[0], wd[1], wd[2], wd[3]};
      }
      if (f_ok && mm == 0 && lane == 0)
        *gptr<uint16_t>(scale_hv + (f.sc_row0 + p) * sc_v) = __builtin_bit_cast(uint16_t, (_Float16)s32);
    }
  }
}

template <class Act, int NCH, bool FUSED, bool GATE_F32, bool SLOTS>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void step_kernel(const StepArgs a) {
  constexpr int ES = Act::kBytes;
  constexpr int ROWB = K * ES;          // bytes of one k-ring row
  constexpr int RPW = 8 * NCH;          // V-rows per streamer (= block_v)
  constexpr int NBLK = NCH / 2;         // 16-row blocks per wave
  constexpr int NVB = NCH / 4;          // 32-row vblocks per wave
  constexpr int CPT_K = ROWB / 16;      // 16-byte chunks per key row
  constexpr int CPT_V = RPW * ES / 16;  // 16-byte chunks of one token's slice of this wave's v rows
  constexpr int NV = LP * CPT_V / 64;   // 16-byte v-row chunks per lead lane, all LP slots
  constexpr int EPC = 16 / ES;          // elements per chunk
  constexpr bool BF16 = std::is_same<Act, ActBF16>::value;
  constexpr bool F16 = std::is_same<Act, ActF16>::value;

  const int lane = threadIdx.x & 63;
  const int q4 = lane >> 4, l16 = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = a.sw;
  int vt = 0, sub = blockIdx.x;
  if (a.n_vt > 1) {
    sub = blockIdx.x / a.n_vt;
    vt = blockIdx.x - sub * a.n_vt;
  }
  const int h = blockIdx.y, b = blockIdx.z;
  // the slot holding sequence b's checkpoint and rings (vLLM's
  // ssm_state_indices; its load completes at the barrier B0 below)
  uint32_t slot_raw = 0;
  if constexpr (SLOTS) slot_raw = ld_u32_uniform(a.slot + b * a.sl_s);
  const int hv0 = h * a.G + sub * a.gw;
  const bool head_lead = wave < a.gw;                  // waves [0, gw): coefficient chains
  const int j_head = head_lead ? wave : wave - a.gw;  // waves [gw, 2 gw): the rows of head j
  constexpr int r0 = 0;
  const int hv = hv0 + j_head;
  const int v0 = vt * a.block_v;
  const int L = a.L;

  // ---- 0. the head leads publish their coefficients through LDS flags -------------
  // flags[j]: head j's coefficients are in LDS; flags[gw + j]: lead j's
  // share of the k ring has landed; flags[2 gw + j]: streamer j's copy of
  // the v rows is in LDS; then the new token's (gamma, beta) per head, then
  // the flush's amax exchange words (2 kMaxVBlocks per head)
  int* flags = (int*)(lds + a.lds_flag);
  float* newgates = (float*)(flags + 3 * a.gw);
  if (wave == 0 && lane < 3 * a.gw) flags[lane] = 0;
  if (wave == 0 && lane < 2 * kMaxVBlocks * a.gw) flags[5 * a.gw + lane] = 0;  // flush amax exchange
  GDNR_WAIT_LGKM0();
  __builtin_amdgcn_s_barrier();  // B0, the only workgroup barrier
  int bs = b;  // index of the sequence's checkpoint / ring rows
  if constexpr (SLOTS) {
    const int sl = (int)__builtin_amdgcn_readfirstlane((int)slot_raw);
    bs = (sl >= 0 && sl < a.n_slots) ? sl : 0;  // out of range: the null slot
  }

  // ---- 1. metadata (scalar), requested by each wave once its first loads are
  // out: the lead after its ring requests, the streamer before it waits for
  // the ring. (Requested before them, a spill of the loaded value into a VGPR
  // lane would wait for this load ahead of the ring requests.)
  int n_raw = 0, pos_raw = -1;
  uint32_t flush_word = 0, flush_shift = 0;
  auto request_meta = [&]() {
    n_raw = (int)ld_u32_uniform(a.valid_len + b * a.vl_s);
    if constexpr (FUSED) pos_raw = (int)ld_u32_uniform(a.pos + b * a.pos_s);
    // flush flag: the aligned dword holding the byte
    if (a.flush) {
      const uintptr_t fa = (uintptr_t)(a.flush + b * a.fl_s);
      flush_word = ld_u32_uniform((const void*)(fa & ~(uintptr_t)3));
      flush_shift = 8u * (uint32_t)(fa & 3);
    }
  };
  // per-sequence metadata, read once the wave needs it
  int n = 0, pos = -1;
  bool do_flush = false;
  auto read_meta = [&]() {
    GDNR_WAIT_LGKM0();
    n = __builtin_amdgcn_readfirstlane(n_raw);
    n = n < 0 ? 0 : (n > L ? L : n);
    if constexpr (FUSED) {
      const int p = __builtin_amdgcn_readfirstlane(pos_raw);
      pos = (p >= 0 && p < L) ? p : -1;
    }
    do_flush = __builtin_amdgcn_readfirstlane((flush_word >> flush_shift) & 0xFFu) != 0;
  };

  // ---- 2-4. lead of head j: ring, new token, Gram, chain, publish ------------------
  // The lead first requests what the chain needs -- its share of the k ring
  // (the 16-byte chunks of all L slots split over the gw leads by
  // direct-to-LDS DMA; slots beyond the fill are read and ignored), q (lead
  // 0; fused: q and k of the new token in every lead), the gates of its head
  // -- right after the workgroup barrier B0; the streamers request nothing until
  // every share has landed, so the ring requests of the grid reach memory
  // ahead of the checkpoint stream. It raises flags[gw + j] when its share
  // has landed and waits for the other leads' shares.
  uint8_t* vbuf = lds + a.lds_v + j_head * LP * RPW * ES;
  float* c_head = (float*)(lds + a.lds_c) + j_head * RPW;  // c_t of head j (replay)
  // checkpoint rows (replay): ck[hh * NBLK + i] = row 16 i + l16, bytes
  // [64 hh + 16 q4, +16); word w of it holds columns 64 hh + 16 q4 + 4 w + e,
  // at a uniform base per 16-row block + one 32-bit lane offset
  uint8_t* scale_hv = a.scale + (bs * a.sc_b + hv * a.sc_h);
  uint8_t* ck_rows = a.ckpt + (bs * a.ck_b + hv * a.ck_h + (v0 + r0) * a.ck_v);
  const uint32_t ck_lo = (uint32_t)l16 * a.ck_v + 16 * q4;
  uint8_t* out_rows = a.out + (b * a.o_b + hv * a.o_h + (v0 + r0) * ES);
  // wait for this head's lead (bounded: the lead always publishes)
  bool waits_ok = true;
  auto await_coefficients = [&]() { waits_ok = wait_flag(flags + j_head, a.status, a.wait_polls) && waits_ok; };
  // Ring append of the new token (full contract): its v rows from this
  // wave's LDS copy, its gates, and (streamer 0 of the key head's first
  // workgroup) q (output) and k from what the lead left in LDS. Issued after
  // every load of the wave.
  auto append_token = [&]() {
    if constexpr (FUSED) {
      if (pos >= 0) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          const int c = 64 * i + lane;
          if (c / CPT_V == pos)
            *(u32x4_t*)(a.v + (bs * a.v_b + pos * a.v_t + hv * a.v_h + v0 * ES + 16 * (c % CPT_V))) =
                *(const u32x4_t*)(vbuf + 16 * c);
        }
        if (vt == 0 && lane == 0) {
          Act::st(a.g + (bs * a.g_b + pos * a.g_t + hv * a.g_h), 0, newgates[2 * j_head]);
          Act::st(a.beta + (bs * a.be_b + pos * a.be_t + hv * a.be_h), 0, newgates[2 * j_head + 1]);
        }
      }
      if (j_head == 0 && vt == 0 && sub == 0) {
        const float2 q2 = Act::ld2(lds + a.lds_q + 2 * lane * ES);
        Act::st2(a.q_out + (b * a.qo_b + h * a.qo_h + 2 * lane * ES), q2.x, q2.y);
        if (pos >= 0) {
          const float2 k2 = Act::ld2(lds + a.lds_knew + 2 * lane * ES);
          Act::st2(a.k + (bs * a.k_b + pos * a.k_t + h * a.k_h + 2 * lane * ES), k2.x, k2.y);
        }
      }
    }
  };

  if (__builtin_amdgcn_readfirstlane((int)head_lead) != 0) {
    const int j = j_head;
    typename Act::Pair q_bits{}, k_bits{};
    uint32_t a_raw = 0, b_raw = 0;
    float alog_raw = 0.f, dtb_raw = 0.f;
    typename Act::Bits g_bits = 0, b_bits = 0;
    {
      const uint8_t* kbase = a.k + (bs * a.k_b + h * a.k_h);
      const uint32_t kt_bytes = a.k_t;
      const int nch = L * CPT_K;
      const int share = ((nch + a.gw - 1) / a.gw + 63) / 64 * 64;  // whole DMA instructions
      const int c_end = min(nch, (j + 1) * share);
      // destination chunk p of token t holds source chunk p ^ (t & 15)
      for (int c0 = j * share; c0 < c_end; c0 += 64) {
        const int c = c0 + lane;
        const int t = c / CPT_K, ch = c % CPT_K;
        if (c < c_end)
          __builtin_amdgcn_global_load_lds(kbase + (uint32_t)(t * kt_bytes + 16 * (ch ^ (t & 15))),
                                           (lds_void_t*)(lds + a.lds_k + c0 * 16), 16, 0, 0);
      }
    }
    if constexpr (!FUSED) {
      if (j == 0 && lane < CPT_K) {
        const uint8_t* qrow = a.q + (b * a.q_b + h * a.q_h);
        __builtin_amdgcn_global_load_lds(qrow + 16 * lane, (lds_void_t*)(lds + a.lds_q), 16, 0, 0);
      }
    } else {
      // (every load below is unconditional -- lanes past the data read a valid
      // element and drop it -- so that no branch join forces an early wait)
      const uint8_t* row = a.mixed + b * a.mx_b;
      q_bits = Act::ld_pair_bits(row + (h * K + 2 * lane) * ES);
      k_bits = Act::ld_pair_bits(row + (a.H * K + h * K + 2 * lane) * ES);
      a_raw = ld_gate_bits<GATE_F32, Act>(a.a + (b * a.a_b + hv * a.a_h));
      b_raw = ld_gate_bits<GATE_F32, Act>(a.bgate + (b * a.bg_b + hv * a.bg_h));
      alog_raw = *(const float*)(a.a_log + hv * a.al_s);
      dtb_raw = *(const float*)(a.dt_bias + hv * a.db_s);
    }
    {
      const int tl = lane < L ? lane : 0;
      g_bits = Act::ld_bits(a.g + (bs * a.g_b + tl * a.g_t + hv * a.g_h), 0);
      b_bits = Act::ld_bits(a.beta + (bs * a.be_b + tl * a.be_t + hv * a.be_h), 0);
    }
    request_meta();
    float q0 = 0.f, q1 = 0.f, k0 = 0.f, k1 = 0.f, gate_new = 0.f, beta_new = 0.f;
    GDNR_WAIT_VMCNT(0);  // this lead's share of the k ring and its small operands landed
    // (this flag also starts the streamers: the checkpoint stream begins once
    // the chain's operands are in, and the lead issues no load after it)
    __hip_atomic_store(flags + a.gw + j, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    read_meta();
    if constexpr (FUSED) {
      // full-contract preparation of the new token's q and k (reference
      // kernel:504-533); every lead writes the same values
      const float2 qr = Act::from_pair(q_bits), kr = Act::from_pair(k_bits);
      const float qd = sqrtf(wave_sum(fmaf(qr.y, qr.y, qr.x * qr.x)) + 1e-6f);
      const float kd = sqrtf(wave_sum(fmaf(kr.y, kr.y, kr.x * kr.x)) + 1e-6f);
      q0 = Act::round(qr.x / qd);
      q1 = Act::round(qr.y / qd);
      k0 = Act::round(kr.x / kd);
      k1 = Act::round(kr.y / kd);
      Act::st2(lds + a.lds_q + 2 * lane * ES, q0, q1);
      Act::st2(lds + a.lds_knew + 2 * lane * ES, k0, k1);
    }
    // gates (gamma = e^g, beta) of the tokens
    const bool on = lane < n;
    float2 gb = make_float2(1.f, 0.f);
    if (on) gb = make_float2(expf(Act::from_bits(g_bits)), Act::from_bits(b_bits));
    if constexpr (FUSED) {
      // gates of the new token (reference kernel:534-562)
      // (same inputs in every lane)
      const float x = gate_value<GATE_F32, Act>(a_raw) + dtb_raw;
      const float sp = x <= 20.0f ? logf(1.0f + expf(x)) : x;  // kernel:560, as written there
      gate_new = readlane_fv(Act::round(-expf(alog_raw) * sp), 0);
      beta_new = readlane_fv(Act::round(1.0f / (1.0f + expf(-gate_value<GATE_F32, Act>(b_raw)))), 0);
      if (on && lane == pos) gb = make_float2(expf(gate_new), beta_new);
    }
    // the other leads' shares of the k ring (bounded waits: every lead raises its flag)
    for (int jj = 0; jj < a.gw; ++jj) waits_ok = wait_flag(flags + a.gw + jj, a.status, a.wait_polls) && waits_ok;

    // Gram of the slot rows Y = [slots 0..15, q, new k]: D00 = slots x slots,
    // D01 = slots x [q, new k], D11 = [q, new k] x [q, new k], from one read of
    // each operand row; G [18][20] (row r, column c) with q at 16, new k at 17.
    float* G = (float*)(lds + a.lds_g) + j * 18 * 20;
    {
      const int n_extra = FUSED ? 2 : 1;
      const bool zs = l16 >= L, ze = l16 >= n_extra;
      const int erow = l16 == 1 ? a.lds_knew : a.lds_q;
      f32x4_t d00 = {0.f, 0.f, 0.f, 0.f}, d01 = d00, d11 = d00;
      if constexpr (std::is_same<Act, ActF32>::value) {
#pragma unroll 4
        for (int kc = 0; kc < K / 4; ++kc) {
          float ka = *(const float*)(lds + a.lds_k + kr_off<ROWB>(l16, (kc * 4 + q4) * 4));
          float ea = *(const float*)(lds + erow + (kc * 4 + q4) * 4);
          ka = zs ? 0.f : ka;
          ea = ze ? 0.f : ea;
          d00 = __builtin_amdgcn_mfma_f32_16x16x4f32(ka, ka, d00, 0, 0, 0);
          d01 = __builtin_amdgcn_mfma_f32_16x16x4f32(ka, ea, d01, 0, 0, 0);
          d11 = __builtin_amdgcn_mfma_f32_16x16x4f32(ea, ea, d11, 0, 0, 0);
        }
      } else {
        uint4 ka[4], ea[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          ka[m] = *(const uint4*)(lds + a.lds_k + kr_off<ROWB>(l16, (4 * m + q4) * 16));
          ea[m] = *(const uint4*)(lds + erow + (4 * m + q4) * 16);
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          if (zs) ka[m] = make_uint4(0u, 0u, 0u, 0u);
          if (ze) ea[m] = make_uint4(0u, 0u, 0u, 0u);
          if constexpr (std::is_same<Act, ActBF16>::value) {
            const bf16x8_t ak = __builtin_bit_cast(bf16x8_t, ka[m]), ae = __builtin_bit_cast(bf16x8_t, ea[m]);
            d00 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak, ak, d00, 0, 0, 0);
            d01 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak, ae, d01, 0, 0, 0);
            d11 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ae, ae, d11, 0, 0, 0);
          } else {
            const f16x8_t ak = __builtin_bit_cast(f16x8_t, ka[m]), ae = __builtin_bit_cast(f16x8_t, ea[m]);
            d00 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ak, ak, d00, 0, 0, 0);
            d01 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ak, ae, d01, 0, 0, 0);
            d11 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ae, ae, d11, 0, 0, 0);
          }
        }
      }
      // D[4 q4 + e][l16]: D00 is symmetric, so lane l writes row l16, columns 4 q4 .. + 3
      *(float4*)(G + l16 * 20 + 4 * q4) = make_float4(d00[0], d00[1], d00[2], d00[3]);
      if (l16 < 2) {
        // column 16 + l16 of rows 4 q4 + e, and its mirror (row 16 + l16)
        *(float4*)(G + (16 + l16) * 20 + 4 * q4) = make_float4(d01[0], d01[1], d01[2], d01[3]);
#pragma unroll
        for (int e = 0; e < 4; ++e) G[(4 * q4 + e) * 20 + 16 + l16] = d01[e];
        if (q4 == 0) {
          G[16 * 20 + 16 + l16] = d11[0];
          G[17 * 20 + 16 + l16] = d11[1];
        }
      }
    }
    // lane t < 16: row of token t (the new k's row at t == pos); columns by token
    float grow[20];
    {
      const float4* gr = (const float4*)(G + (lane == pos ? 17 : l16) * 20);
#pragma unroll
      for (int i = 0; i < 5; ++i) {
        const float4 v4 = gr[i];
        grow[4 * i] = v4.x;
        grow[4 * i + 1] = v4.y;
        grow[4 * i + 2] = v4.z;
        grow[4 * i + 3] = v4.w;
      }
    }
    float gcol[LP];  // G[token lane][token t], zero for t >= n
#pragma unroll
    for (int t = 0; t < LP; ++t) gcol[t] = t < n ? (t == pos ? grow[17] : grow[t]) : 0.f;
    const float dq = on ? grow[16] : 0.f;
    // prod_{x >= t} gamma_x (inclusive suffix) and prod_{x > t} gamma_x
    const float suf_in = row_suffix_prod(gb.x);
    const float suf_ex = dpp_row<0x101>(suf_in, 1.f);
    const float lam_all = readlane_fv(suf_in, 0);
    // (the branch conditions are re-made wave-uniform: the divergence
    // analysis loses track of values set inside read_meta, and a branch it
    // takes for divergent is structurised into one path through both tails)
    if (__builtin_amdgcn_readfirstlane((int)do_flush) == 0) {
      // s_t, t descending: acc_l = sum_{u > t} G[l][u] s_u (s_t = 0 for t >= n: beta = 0)
      float acc = 0.f, s_mine = 0.f;
      const float beta = gb.y;
#pragma unroll
      for (int t = LP - 1; t >= 0; --t) {
        const float sv = readlane_fv(beta * (dq - acc), t);
        s_mine = lane == t ? sv : s_mine;
        acc = fmaf(gcol[t], sv, acc);
      }
      const float c_mine = on ? s_mine * suf_ex : 0.f;
      // s and c to LDS (this head's T0 area, overwritten below) and back as
      // VGPR broadcasts: no SGPRs held across the loop
      float* sc_lds = (float*)(lds + a.lds_t) + j * K;
      if (lane < LP) {
        sc_lds[lane] = s_mine;
        sc_lds[LP + lane] = c_mine;
      }
      float sb[LP], cb[LP];
#pragma unroll
      for (int i = 0; i < LP / 4; ++i) {
        const float4 s4 = ((const float4*)sc_lds)[i], c4 = ((const float4*)(sc_lds + LP))[i];
        sb[4 * i] = s4.x, sb[4 * i + 1] = s4.y, sb[4 * i + 2] = s4.z, sb[4 * i + 3] = s4.w;
        cb[4 * i] = c4.x, cb[4 * i + 1] = c4.y, cb[4 * i + 2] = c4.z, cb[4 * i + 3] = c4.w;
      }
      // c for the streamer's w = sum_t c_t v_t (this head's c area)
      if (lane < LP) c_head[lane] = c_mine;
      // T0 = lam_all (q - sum_t s_t k_t), lane owns columns 2 lane, 2 lane + 1
      // (all 16 operand pairs are read first, then the FMAs)
      float2 kk[LP];
#pragma unroll
      for (int t = 0; t < LP; ++t)
        kk[t] = Act::ld2(lds + xr_off_row<ROWB>(a.lds_k, a.lds_knew, a.lds_q, t, n, pos, 2 * lane * ES));
      float2 U = Act::ld2(lds + a.lds_q + 2 * lane * ES);
#pragma unroll
      for (int t = 0; t < LP; ++t) {
        const float st = sb[t];
        U.x = fmaf(-st, kk[t].x, U.x);
        U.y = fmaf(-st, kk[t].y, U.y);
      }
      *(float2*)(lds + a.lds_t + (j * K + 2 * lane) * 4) = make_float2(lam_all * U.x, lam_all * U.y);
    } else {
      const XRows xr{a.lds_k, a.lds_knew, a.lds_q, n, pos};
      // K^T as MFMA A-operand tiles of 16 K-columns x 16 tokens, tile ct at
      // ct * 256 * ES bytes; row r of tile ct is K column
      // 64 (ct / 4) + 16 (r / 4) + 4 (ct % 4) + r % 4, the column order of the
      // checkpoint operand in section 7. Raw ring bits, zero for tokens t >= n;
      // every lead writes the same tiles.
#pragma unroll
      for (int cc = 0; cc < K / 64; ++cc) {
        const int c = cc * 64 + lane;
        const int ct = 4 * (c >> 6) + ((c >> 2) & 3);
        const int row = 4 * ((c >> 4) & 3) + (c & 3);
        uint32_t wd[4 * ES];  // 16 tokens x ES bytes
        if constexpr (ES == 2) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int t0 = 2 * i, t1 = t0 + 1;
            const uint32_t lo = *(const uint16_t*)(lds + xr.off<ROWB>(t0, c * 2));
            const uint32_t hi = *(const uint16_t*)(lds + xr.off<ROWB>(t1, c * 2));
            wd[i] = (t0 < n ? lo : 0u) | (t1 < n ? hi << 16 : 0u);
          }
        } else {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const uint32_t x = *(const uint32_t*)(lds + xr.off<ROWB>(i, c * 4));
            wd[i] = i < n ? x : 0u;
          }
        }
        uint4* dst = (uint4*)(lds + a.lds_kt + ct * 256 * ES + row * 16 * ES);
#pragma unroll
        for (int i = 0; i < ES; ++i) dst[i] = make_uint4(wd[4 * i], wd[4 * i + 1], wd[4 * i + 2], wd[4 * i + 3]);
      }
      // flush factors of head j:
      //   pre_t  = prod_{x<=t} gamma_x        post_t = beta_t prod_{x>t} gamma_x
      //   M[t][s] = beta_s prod_{s<x<=t} gamma_x (k_s . k_t)   (s < t)
      // so that the forward residuals u_t = v_t - (gamma_t S_t) k_t obey
      //   u_t = (v_t - pre_t S_0 k_t) - sum_{s<t} M[t][s] u_s,  i.e.  u = R w, R = (I + M)^-1.
      const float pre = row_prefix_prod(gb.x);
      const float post = gb.y * suf_ex;
      if (lane < LP)
        ((float4*)(lds + a.lds_fac))[j * LP + lane] = make_float4(on ? pre : 0.f, on ? post : 0.f, dq, 0.f);
      if (lane == 0) ((float*)(lds + a.lds_lam))[j] = lam_all;
      // M[t][s] = beta_s prod_{s<x<=t} gamma_x G[s][t] (s < t < n), built with
      // lane = column s, then R = (I + M)^-1 by forward substitution with lane =
      // column c. Broadcast operands (gamma, rows of M) go through LDS (this
      // head's U~ area, unused until the rebuild) into VGPRs.
      float* bc = (float*)(lds + a.lds_u + j * LP * 192);  // [gamma (16) | M (16 x 16)]
      if (lane < LP) bc[lane] = gb.x;
      float gam[LP];
#pragma unroll
      for (int i = 0; i < LP / 4; ++i) {
        const float4 g4 = ((const float4*)bc)[i];
        gam[4 * i] = g4.x, gam[4 * i + 1] = g4.y, gam[4 * i + 2] = g4.z, gam[4 * i + 3] = g4.w;
      }
      float* Mm = bc + LP;
      float run = 1.f;
#pragma unroll
      for (int t = 0; t < LP; ++t) {
        if (t > lane) run *= gam[t];
        if (lane < LP) Mm[t * LP + lane] = (lane < t && t < n) ? gb.y * run * gcol[t] : 0.f;
      }
      float r[LP];
#pragma unroll
      for (int t = 0; t < LP; ++t) {
        float mrow[LP];
#pragma unroll
        for (int i = 0; i < LP / 4; ++i) {
          const float4 m4 = ((const float4*)(Mm + t * LP))[i];
          mrow[4 * i] = m4.x, mrow[4 * i + 1] = m4.y, mrow[4 * i + 2] = m4.z, mrow[4 * i + 3] = m4.w;
        }
        float x = (t == lane) ? 1.f : 0.f;
#pragma unroll
        for (int s2 = 0; s2 < t; ++s2) x = fmaf(-mrow[s2], r[s2], x);
        r[t] = x;
      }
      if (lane < LP) {
        float* Rj = (float*)(lds + a.lds_r) + j * LP * LP;
#pragma unroll
        for (int t = 0; t < LP; ++t) Rj[t * LP + lane] = (t < n && on) ? r[t] : 0.f;
      }
    }
    // the new token's gates, for the streamer's ring append
    if (FUSED && lane == 0) {
      newgates[2 * j] = gate_new;
      newgates[2 * j + 1] = beta_new;
    }
    // publish: this head's coefficients (or flush factors), new gates and
    // the shared q / new k / K^T are in LDS
    __hip_atomic_store(flags + j, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (__builtin_amdgcn_readfirstlane((int)do_flush) == 0) return;
    // a flush splits every vblock of the head between the two waves of the
    // head: the lead takes the upper 16 rows once the streamer's copy of the
    // v rows is in LDS (bounded wait: the streamer always raises the flag)
    waits_ok = wait_flag(flags + 2 * a.gw + j, a.status, a.wait_polls) && waits_ok;
  }

  // ---- streamer of head j_head ---------------------------------------------------
  if (__builtin_amdgcn_readfirstlane((int)head_lead) == 0) {
    // Stream once the k ring has landed (bounded waits: every lead raises its
    // flag): the ring requests of the grid reach memory ahead of the checkpoint
    // stream. A replay holds its checkpoint rows in registers; a flush reads
    // them one vblock at a time in section 7 (its registers go to the rebuild).
    request_meta();
    for (int jj = 0; jj < a.gw; ++jj) waits_ok = wait_flag(flags + a.gw + jj, a.status, a.wait_polls) && waits_ok;
    read_meta();
    // v rows of head j first (a replay folds them into w before its matvec):
    // chunk c = 64 i + lane holds rows
    // EPC (c % CPT_V) + [0, EPC) of token c / CPT_V. Tokens at or past the fill
    // re-read slot 0 (a cache hit; dropped below); the new token's slot reads
    // the new v from mixed_qkv. Every lane loads: the instruction count is static.
    u32x4_t vch[NV];
    {
      const uint8_t* vring = a.v + (bs * a.v_b + hv * a.v_h + v0 * ES);
      const uint32_t vt_bytes = a.v_t;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int c = 64 * i + lane;
        const int t = c / CPT_V, rc = c % CPT_V;
        const uint8_t* src = vring + ((uint32_t)(t < n ? t : 0) * vt_bytes + 16u * (uint32_t)rc);
        if constexpr (FUSED)
          if (t == pos) src = a.mixed + (b * a.mx_b + (2 * a.H * K + hv * a.V + v0) * ES + 16 * rc);
        vch[i] = *(const u32x4_t*)src;
      }
    }
    if (__builtin_amdgcn_readfirstlane((int)do_flush) == 0) {
      // ---- replay: o = (scale * codes) . T0 + w -----------------------------------
      uint32_t sc_bits[NVB];  // scalar
#pragma unroll
      for (int p = 0; p < NVB; ++p) sc_bits[p] = ld_u16_uniform((const uint16_t*)(scale_hv + ((v0 + r0) / kVBlock + p) * a.sc_v));
      // checkpoint rows, row-contiguous: load i covers rows 8 i + [0, 8) of
      // the wave's rows (1 KB when they are 128 bytes apart); lane l holds row
      // 8 i + r8 at columns 16 c8 + [0, 16), r8 = l / 8, c8 = l % 8
      const int r8 = lane >> 3, c8 = lane & 7;
      uint4 ck[NCH];
      GDNR_COMPILER_FENCE();
      {
        const uint32_t lo = (uint32_t)r8 * (uint32_t)a.ck_v + 16u * (uint32_t)c8;
        const uint32_t rstep = 8u * (uint32_t)a.ck_v;
#pragma unroll
        for (int i = 0; i < NCH; ++i) ck[i] = *(const uint4*)(ck_rows + (lo + (uint32_t)i * rstep));
      }
      GDNR_COMPILER_FENCE();
      // the v rows land ahead of the checkpoint rows: copy them to LDS in
      // token-major order (chunk c at byte 16 c) and free their registers
      GDNR_WAIT_VMCNT(NCH);
#pragma unroll
      for (int i = 0; i < NV; ++i) *(u32x4_t*)(vbuf + 16 * (64 * i + lane)) = vch[i];
      __hip_atomic_store(flags + 2 * a.gw + j_head, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
      await_coefficients();
      // The 8 lanes of a row group reduce their NCH partial dots by halving
      // (partners l ^ 7, l ^ 2, l ^ 1 select on bits 2, 1, 0 of c8): value m
      // of a lane ends as the total of chunk index ibase + m, row
      // 8 (ibase + m) + r8. With NCH = 4 the last step is a plain sum and the
      // lanes with c8 odd emit nothing.
      constexpr int NFIN = NCH >= 8 ? NCH / 8 : 1;
      const int b0 = c8 & 1, b1 = (c8 >> 1) & 1, b2 = (c8 >> 2) & 1;
      const int ibase = b2 * (NCH / 2) + b1 * (NCH / 4) + (NCH >= 8 ? b0 * (NCH / 8) : 0);
      // w = sum_t c_t v_t of each row this lane emits, tokens in order (the
      // sum does not depend on block_v)
      float wrow[NFIN];
#pragma unroll
      for (int m = 0; m < NFIN; ++m) {
        const int row = 8 * (ibase + m) + r8;
        float w = 0.f;
#pragma unroll
        for (int t = 0; t < LP; ++t) {
          // slots at or past the fill hold stale data: selected away, never summed
          const float wt = fmaf(c_head[t], Act::ld(vbuf, t * RPW + row), w);
          w = t < n ? wt : w;
        }
        wrow[m] = w;
      }
      // partial dots of the lane's 16 columns with T0
      float Tv[16];
      {
        const float4* tp = (const float4*)(lds + a.lds_t + (j_head * K + 16 * c8) * 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float4 w = tp[i];
          Tv[4 * i] = w.x;
          Tv[4 * i + 1] = w.y;
          Tv[4 * i + 2] = w.z;
          Tv[4 * i + 3] = w.w;
        }
      }
      float P[NCH];
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        const uint4 c = ck[i];
        const uint32_t w4[4] = {c.x, c.y, c.z, c.w};
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          float f[4];
          fp8x4_to_f32(w4[w], f);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc = fmaf(f[e], Tv[4 * w + e], acc);
        }
        P[i] = acc;
      }
      // halving steps: keep one half, add the partner's copy of it
#pragma unroll
      for (int m = 0; m < NCH / 2; ++m) {
        const float send = b2 ? P[m] : P[m + NCH / 2];
        const float keep = b2 ? P[m + NCH / 2] : P[m];
        P[m] = keep + dpp_f<kDppHalfMirror>(send);
      }
#pragma unroll
      for (int m = 0; m < NCH / 4; ++m) {
        const float send = b1 ? P[m] : P[m + NCH / 4];
        const float keep = b1 ? P[m + NCH / 4] : P[m];
        P[m] = keep + dpp_f<kDppXor2>(send);
      }
      if constexpr (NCH >= 8) {
#pragma unroll
        for (int m = 0; m < NCH / 8; ++m) {
          const float send = b0 ? P[m] : P[m + NCH / 8];
          const float keep = b0 ? P[m + NCH / 8] : P[m];
          P[m] = keep + dpp_f<kDppXor1>(send);
        }
      } else {
        P[0] += dpp_f<kDppXor1>(P[0]);
      }
      if (NCH >= 8 || b0 == 0) {
#pragma unroll
        for (int m = 0; m < NFIN; ++m) {
          const int row = 8 * (ibase + m) + r8;
          // scale of the row's vblock (row / 32 = (ibase + m) / 4), by bit-selects
          // (a select of lane-indexed entries would become a private-array load)
          const int pv = (ibase + m) >> 2;
          uint32_t sb = sc_bits[0];
#pragma unroll
          for (int q = 1; q < NVB; ++q) sb ^= (sb ^ sc_bits[q]) & (0u - (uint32_t)(pv == q));
          const float sc = f16_bits_to_f32((uint16_t)sb);
          Act::st(out_rows, row, fmaf(P[m], sc, wrow[m]) * a.out_scale);
        }
      }
      append_token();
      return;
    }
    // flush: no checkpoint rows in registers (section 7 reads them per vblock)
    GDNR_WAIT_VMCNT(0);
#pragma unroll
    for (int i = 0; i < NV; ++i) *(u32x4_t*)(vbuf + 16 * (64 * i + lane)) = vch[i];
    __hip_atomic_store(flags + 2 * a.gw + j_head, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    await_coefficients();
  }

  // ---- 7. flush: MFMA rebuild of block 1 (lead) or 0 (streamer) of every
  // vblock of the head, out of line
  flush_vblocks<Act, NCH>(ck_rows, scale_hv, out_rows, a.ck_v, a.sc_v, (v0 + r0) / kVBlock, a.out_scale, a.lds_k,
                          a.lds_knew, a.lds_q, a.lds_r, a.lds_fac, a.lds_lam, a.lds_kt, (int32_t)(vbuf - lds),
                          a.lds_flag + 4 * (5 * a.gw + 2 * kMaxVBlocks * j_head), j_head, n, pos,
                          head_lead ? 1 : 0, NVB, a.status, a.wait_polls, waits_ok);
  if (__builtin_amdgcn_readfirstlane((int)head_lead) == 0) append_token();
}

#if GDNR_ACT == 0
using Act = ActBF16;
#define GDNR_SUFFIX(name) name##_bf16
#elif GDNR_ACT == 1
using Act = ActF16;
#define GDNR_SUFFIX(name) name##_f16
#else
using Act = ActF32;
#define GDNR_SUFFIX(name) name##_f32
#endif

template <int NCH, bool FUSED, bool GATE_F32, bool SLOTS = false>
void launch_step_variant(const StepArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)(a.n_vt * (a.G / a.gw)), (unsigned)a.H, (unsigned)a.B), block((unsigned)(64 * a.sw));
  auto kernel = step_kernel<Act, NCH, FUSED, GATE_F32, SLOTS>;
  if (a.lds_bytes > 64 * 1024) {
    // gfx950 has 160 KiB of LDS per workgroup; dynamic allocations above
    // 64 KiB must be enabled per kernel (idempotent, cheap)
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, a.lds_bytes);
    if (e != hipSuccess) return;  // the launch below reports the error
  }
  hipLaunchKernelGGL(kernel, grid, block, a.lds_bytes, s, a);
}

template <int NCH>
void launch_step_nch(const StepArgs& a, bool fused, bool gate_f32, hipStream_t s) {
  if (!fused) launch_step_variant<NCH, false, false>(a, s);
  else if (a.slot && gate_f32) launch_step_variant<NCH, true, true, true>(a, s);
  else if (a.slot) launch_step_variant<NCH, true, false, true>(a, s);
  else if (gate_f32) launch_step_variant<NCH, true, true>(a, s);
  else launch_step_variant<NCH, true, false>(a, s);
}

}  // namespace

int GDNR_SUFFIX(launch_step)(const StepArgs& a, bool fused, bool gate_f32, void* stream) {
  hipStream_t s = (hipStream_t)stream;
  if (a.rpw == 128) launch_step_nch<16>(a, fused, gate_f32, s);
  else if (a.rpw == 64) launch_step_nch<8>(a, fused, gate_f32, s);
  else launch_step_nch<4>(a, fused, gate_f32, s);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : (int)e;
}

}  // namespace gdnr
