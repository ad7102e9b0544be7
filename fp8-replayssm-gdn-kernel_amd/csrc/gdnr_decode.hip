// gdnr_decode.hip -- the ReplaySSM decode step on gfx950 (MI355X) for rings of
// up to 16 tokens with 16-bit activations (bf16 or f16): replay or flush per
// sequence, optionally fused with the full-contract preparation of the new
// token. (f32 activations take the step kernel of gdnr_step.hip.)
//
// The checkpoint stream starts at the first instruction of every wave. The
// coefficient chain of a head does not stand between the stream and the
// output: every wave projects its checkpoint rows on all ring keys and the
// query with bf16/f16 MFMAs,
//   P = X S_0^T,   X = [k_0 .. k_{n-1}, q, 0 ..]   (16 x 128, tokens x K),
// and the chain only supplies the weights that combine those projections.
// Replay, the adjoint of the reference's reverse chain
// (prototype/gdn_replayssm_fp8_kernel.py:121-173) in Gram form:
//   s_t = beta_t (dq_t - sum_{u>t} G_tu s_u),  G = K K^T,  dq = K q
//   c_t = s_t prod_{u>t} gamma_u,  lam = prod_u gamma_u
//   o   = (scale (lam P_q - sum_t lam s_t P_t) + sum_t c_t v_t) K^-1/2
// (scale * codes is the dequantised checkpoint, so S_0 T_0 with the
// reference's T_0 = lam (q - sum_t s_t k_t) is sum_t alpha_t P_t.)
// Flush, the forward rebuild of kernel:177-242 in matrix form (W = V - pre P,
// U = (I + M)^-1 W, S_n = lam S_0 + K^T (post U)), o from the rebuilt state,
// requantisation in place with the reference quantiser (ref:36-37,83-99).
//
// Grid: x = group of gw value heads within the key head, y = key head h,
// z = sequence b. Workgroup: gw value heads x nwh waves, wave (j, part)
// owning V-rows [64 part, +64) of value head j. One wave per head (the
// chain wave, part == (b + h) % nwh) also forms the head's Gram matrix and
// coefficient chain (or flush factors) and publishes them through LDS; the
// others wait for its flag only after their own projections are done.
//
// Operand layouts (16x16x32 MFMA; lane = 16 q4 + l16; k-step m = 0..3 of a
// lane covers columns 32 q4 + 8 m + 0..7):
//   X (A operand): lane (t = l16, q4) holds X[t][32 q4 + 8 m + 0..7]: the
//     64 bytes at 64 q4 of the row (elements 32 q4 .. 32 q4 + 31).
//   codes (B operand) of tile i (16 rows): lane (nn = l16, q4) holds row
//     r(i, nn) = 32 (i >> 1) + 2 nn + (i & 1) of the wave's rows, bytes
//     [32 q4, +32) (the codes of the same columns). Tiles 2p, 2p + 1 are
//     vblock p of the wave, and a lane's rows of a token's v sit in two
//     4-byte pairs.
//   P (accumulator): lane (nn, q4) holds P[token 4 q4 + e][row r(i, nn)].
//
// Compiled once per 16-bit activation dtype (GDNR_ACT = 0 bf16, 1 f16).
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <type_traits>

#include "gdnr_device.h"
#include "gdnr_internal.h"

#ifndef GDNR_ACT
#error "compile with -DGDNR_ACT=0|1|2"
#endif

#if GDNR_ACT != 2

namespace gdnr {
namespace {

constexpr int K = kKeyDim;
constexpr int NT = kStepRing;  // token rows of the operands (ring capacity <= 16)

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

#if GDNR_ACT == 0
using Act = ActBF16;
#define GDNR_SUFFIX(name) name##_bf16
#else
using Act = ActF16;
#define GDNR_SUFFIX(name) name##_f16
#endif
constexpr bool kBF16 = std::is_same<Act, ActBF16>::value;

__device__ __forceinline__ f32x4_t mfma16(u32x4_t a, u32x4_t b, f32x4_t c) {
  if constexpr (kBF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
}
// 4 e4m3 codes -> 4 values of the activation type (exact), packed in pairs
__device__ __forceinline__ uint2 codes4(uint32_t w) { return kBF16 ? fp8x4_to_bf16x4(w) : fp8x4_to_f16x4(w); }
// the 8 codes of k-step m of a lane's 32 bytes of a row (c[0]: bytes
// [32 q4, +16), c[1]: [32 q4 + 16, +16); k-step m: bytes 32 q4 + 8 m + 0..7)
__device__ __forceinline__ u32x4_t codes8(const u32x4_t* c, int m) {
  const u32x4_t w = c[m >> 1];
  const uint32_t w0 = (m & 1) ? w[2] : w[0], w1 = (m & 1) ? w[3] : w[1];
  const uint2 lo = codes4(w0);
  const uint2 hi = codes4(w1);
  return u32x4_t{lo.x, lo.y, hi.x, hi.y};
}
// f32x4_to_fp8_ref with its constants formed where it runs (through empty
// asm statements, which stay in place): the flush's rare division path uses
// it, and constants hoisted out of the flush loop would hold registers for
// the whole loop
__device__ __forceinline__ uint32_t f32x4_to_fp8_ref_cold(float a, float b, float c, float d) {
  float lim = 448.0f;
  uint32_t k7f = 0x7Fu, kff = 0xFFu;
  asm volatile("" : "+v"(lim), "+v"(k7f), "+v"(kff));
  const float v[4] = {a, b, c, d};
  float cl[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) cl[e] = (v[e] != v[e]) ? v[e] : fminf(fmaxf(v[e], -lim), lim);
  uint32_t w = f32x4_to_fp8(cl[0], cl[1], cl[2], cl[3]);
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (v[e] != v[e]) w = (w & ~(kff << (8 * e))) | ((__float_as_uint(v[e]) >> 31 ? kff : k7f) << (8 * e));
  return w;
}
// activation value from 16 bits
__device__ __forceinline__ float act_val(uint32_t bits16) { return Act::from_bits(bits16 & 0xFFFFu); }
__device__ __forceinline__ uint32_t act_bits(float x) {
  if constexpr (kBF16) return f32_to_bf16(x);
  else return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
}

__device__ __forceinline__ float rdl(float x, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
}
__device__ __forceinline__ int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }
// a uniform value the compiler cannot see through: work derived from it
// stays after this point (is not hoisted into code shared by the roles,
// where it would wait for the argument block)
__device__ __forceinline__ int opaque_s(int x) {
  asm volatile("" : "+s"(x));
  return x;
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

// uniform loads through the scalar cache of data this kernel does not write
// before reading it (constant address space; they count in lgkmcnt)
typedef __attribute__((address_space(4))) const uint32_t const_u32;
__device__ __forceinline__ uint32_t ld_u32_uniform(const void* p) { return *(const_u32*)p; }
__device__ __forceinline__ uint32_t ld_u16_uniform(const uint8_t* p) {
  const uintptr_t ad = (uintptr_t)p;
  return (ld_u32_uniform((const void*)(ad & ~(uintptr_t)3)) >> (8u * (uint32_t)(ad & 2))) & 0xFFFFu;
}
__device__ __forceinline__ u32x4_t ld16(const uint8_t* p) { return *(const u32x4_t*)p; }
typedef __attribute__((address_space(1))) const u32x4_t g_u32x4;
typedef __attribute__((address_space(1))) u32x4_t g_u32x4_w;
// The kernel's arguments as laid out in the kernarg segment (parameters in
// order, naturally aligned), to reach the argument block by address.
struct DecodeKernArgs {
  uint8_t* ckpt;
  uint8_t* kring;
  uint32_t ck_b, ck_h, ck_v, k_b, k_t, k_h;
  int32_t L, G, shape;
  StepArgs a;
};
// The argument block through a pointer the compiler cannot see through:
// its scalar loads issue after this point (they are not hoisted above the
// checkpoint loads, whose address registers they could otherwise tie up).
typedef __attribute__((address_space(4))) const StepArgs c_args;
typedef __attribute__((address_space(4))) const uint8_t c_u8;
__device__ __forceinline__ const StepArgs& opaque_args() {
  uint64_t v = (uint64_t)((c_u8*)__builtin_amdgcn_kernarg_segment_ptr() + offsetof(DecodeKernArgs, a));
  uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
  asm volatile("" : "+s"(lo), "+s"(hi));
  return *(const StepArgs*)(c_args*)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ uint32_t ld32(const uint8_t* p) { return *(const uint32_t*)p; }
// A sequence's (slot's) base in a tensor, in 64 bits: the tensors of a slot
// cache may span more than 4 GiB; offsets inside one sequence stay 32-bit.
__device__ __forceinline__ uint8_t* sbase(const uint8_t* p, int seq, uint32_t stride) {
  return (uint8_t*)p + (uint64_t)(uint32_t)seq * stride;
}
// x + y for two 32-bit products, kept as two multiplies and an add: the fused
// form (v_mad_u64_u32, whose unused upper addend half the allocator may give
// a register an outstanding load is filling) makes the wave wait for every
// load issued before it
__device__ __forceinline__ uint32_t off_sum(uint32_t x, uint32_t y) {
  asm volatile("" : "+v"(x), "+v"(y));
  return x + y;
}
// Direct global -> LDS copy of 16 bytes per lane (global_load_lds_dwordx4):
// lane l's 16 bytes land at LDS address lds_addr + 16 l (lds_addr wave-uniform,
// through M0, which is restored). Written as inline assembly so that the
// compiler does not order every later LDS read after it: the caller waits for
// it (vmcnt) before reading the destination, and the compiler's own vmcnt
// waits, which do not count it, can only wait longer than they need.
__device__ __forceinline__ void dma16(const uint8_t* src, uint32_t lds_addr) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %2, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds_addr), "v"(src)
      : "memory");
}

// DPP move within a 16-lane row; lanes whose source is outside the row get `fill`
template <int CTRL>
__device__ __forceinline__ float dpp_row(float x, float fill) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, fill), __builtin_bit_cast(int, x),
                                                               CTRL, 0xF, 0xF, false));
}
// every lane of each 16-lane row gets lane n of its row (DPP row_newbcast)
template <int N>
__device__ __forceinline__ float row_bcast(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x150 + N, 0xF, 0xF, false));
}
__device__ __forceinline__ float row_bcast_n(float x, int n) {
  switch (n) {
    case 0: return row_bcast<0>(x);   case 1: return row_bcast<1>(x);   case 2: return row_bcast<2>(x);
    case 3: return row_bcast<3>(x);   case 4: return row_bcast<4>(x);   case 5: return row_bcast<5>(x);
    case 6: return row_bcast<6>(x);   case 7: return row_bcast<7>(x);   case 8: return row_bcast<8>(x);
    case 9: return row_bcast<9>(x);   case 10: return row_bcast<10>(x); case 11: return row_bcast<11>(x);
    case 12: return row_bcast<12>(x); case 13: return row_bcast<13>(x); case 14: return row_bcast<14>(x);
    default: return row_bcast<15>(x);
  }
}
__device__ __forceinline__ float row_prefix_prod(float x) {
  x *= dpp_row<0x111>(x, 1.f);
  x *= dpp_row<0x112>(x, 1.f);
  x *= dpp_row<0x114>(x, 1.f);
  x *= dpp_row<0x118>(x, 1.f);
  return x;
}
__device__ __forceinline__ float row_suffix_prod(float x) {
  x *= dpp_row<0x101>(x, 1.f);
  x *= dpp_row<0x102>(x, 1.f);
  x *= dpp_row<0x104>(x, 1.f);
  x *= dpp_row<0x108>(x, 1.f);
  return x;
}

// Sum over the four 16-lane rows of per-tile partials: p[i] is lane (nn, q4)'s
// partial of tile i; on return lane (nn, q4) holds the total of tile q4
// (v_permlane32_swap then v_permlane16_swap: a reduce-scatter in 3 swaps).
__device__ __forceinline__ float rows_reduce_scatter(float p0, float p1, float p2, float p3) {
  const auto r0 = __builtin_amdgcn_permlane32_swap(__float_as_uint(p0), __float_as_uint(p2), false, false);
  const auto r1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(p1), __float_as_uint(p3), false, false);
  const float u0 = __uint_as_float(r0[0]) + __uint_as_float(r0[1]);
  const float u1 = __uint_as_float(r1[0]) + __uint_as_float(r1[1]);
  const auto r2 = __builtin_amdgcn_permlane16_swap(__float_as_uint(u0), __float_as_uint(u1), false, false);
  return __uint_as_float(r2[0]) + __uint_as_float(r2[1]);
}

// The U~ operand of a flush's K^T U~ MFMA (16x16x32, k-slot 8 q4 + j) from
// this lane's 16-bit hi and lo words of tokens 4 q4 .. 4 q4 + 3 (h01 = hi
// of tokens 4 q4 and 4 q4 + 1, ...). One half-wave swap per word pair gives
// lanes q4 < 2 the hi words of tokens 4 q4 .. +3 and 4 q4 + 8 .. +3, lanes
// q4 >= 2 the lo words of tokens 4 q4 - 8 .. -5 and 4 q4 .. +3: k-slots
// 8 q4 .. 8 q4 + 7 hold positions 8 (q4 & 1) .. + 7 of kt_pos's token order.
__device__ __forceinline__ u32x4_t utilde_operand(uint32_t h01, uint32_t h23, uint32_t l01, uint32_t l23) {
  const auto s01 = __builtin_amdgcn_permlane32_swap(h01, l01, false, false);
  const auto s23 = __builtin_amdgcn_permlane32_swap(h23, l23, false, false);
  return u32x4_t{s01[0], s23[0], s01[1], s23[1]};
}
// max(m, |a|, |b|), NaN propagating (one v_maximum3_f32)
__device__ __forceinline__ float max3_abs(float m, float a, float b) {
  return __builtin_elementwise_maximum(__builtin_elementwise_maximum(m, __builtin_fabsf(a)), __builtin_fabsf(b));
}
// Position of token t in a row of the flush's K^T tiles (bits 2 and 3
// swapped: positions 0..7 hold tokens 0..3 and 8..11, positions 8..15
// tokens 4..7 and 12..15), so that lane (nn, q4) reads its 8 16-bit operand
// values as one 16-byte read at position 8 (q4 & 1).
__device__ __forceinline__ int kt_pos(int t) { return (t & 3) | ((t & 4) << 1) | ((t & 8) >> 1); }

extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

// LDS of a workgroup (bytes). A unit's chain wave writes its blocks before
// it sets the unit's flag; the unit's row waves only read them after.
constexpr int kXStride = 272;                  // X row stride (256 + 16: conflict-free operand reads)
constexpr int kLX = 0;                         // X rows [16][kXStride], the A operand in row form
constexpr int kLQK = kLX + 16 * kXStride;      // the prepared q and k rows [2][256] (pair layout = row form)
constexpr int kLKT = kLQK + 512;               // K^T operand tiles [8][16][16] act (flush)
constexpr int kLG = kLKT + 8 * 16 * 16 * 2;    // Gram rows f32 [16][16]
constexpr int kLDq = kLG + 1024;               // k_t . q of a full ring f32 [16]
constexpr int kLFlag = kLDq + 64;              // int [16]: the unit's flags (kFlag* below)
constexpr int kLHeads = kLFlag + 64;           // per value head blocks
constexpr int kFlagReady = 0;                  // the chain wave's LDS blocks are complete
constexpr int kFlagXRows = 1;                  // (NCH > 1 replay) the X rows and the query row are in LDS
constexpr int kFlagGram = 2;                   // (NCH > 1 replay) row waves done with their Gram groups (count)
constexpr int kChainGroups = 2;                // (NCH > 1 replay) Gram groups c < 2 the chain wave forms
constexpr int kGfStride = 68;                  // (NCH > 1 replay) floats per row of the ring's Gram matrix
constexpr int kFlagVStaged = 4;                // + w: row wave w's v rows are in LDS (flush)
constexpr int kFlagHelped = 8;                 // + w: vblocks of row wave w rebuilt by helpers (flush)
// per value head (offsets from the head's block)
constexpr int kHCoef = 0;                      // f32 [16]: c_t (replay)
constexpr int kHLam = kHCoef + 64;             // f32 [4]: lam, the scale of the T_0 rows
constexpr int kHFac = kHLam + 16;              // float4 [16]: (pre, post, dq, 0) (flush)
constexpr int kHT0 = kHFac + 256;              // (replay) f32 [16]: the X rows' weights alpha (one chunk);
                                               // act [3][128]: T_0 as hi, mid and lo rows (NCH > 1 chunks)
constexpr int kHM = kHT0;                      // f32 [16][16]: M (chain scratch; flush, so T_0's bytes;
                                               // then the helpers' o partials, [kPartials][64] float2)
constexpr int kHR = kHM + 1024;                // f32 [16][16]: R = (I + M)^-1 (flush)
constexpr int kHeadLds = kHR + 1024;
constexpr int kPartials = 2;                   // helper o partials per value head (512 bytes each, in M's area)
static_assert(kPartials * 512 <= kHR - kHM, "the helpers' o partials must fit M's area");

constexpr int kMaxDecodeHeads = 2;            // value heads per unit (gw)
constexpr int kUnitBase = kLHeads + kMaxDecodeHeads * kHeadLds;  // LDS of one unit before its v rows
// The layout above is that of a ring of NT tokens (one chunk). A ring of NCH
// chunks of NT tokens (L <= 16 NCH; NCH > 1 takes one value head per unit)
// scales every per-token block: NCH NT X rows (keys only: the query of
// NCH > 1 stays in kLQK), K^T tiles, Gram blocks and k.q per chunk; per
// head, NCH NT coefficients, flush factors, M and R blocks, and the chunk
// decays lam_c (kHLam: [0] lam, [1] the T_0 rows' scale, [2 + c] lam_c).
template <int NCH>
struct Lay {
  static constexpr int kLX = 0;
  static constexpr int kLQK = kLX + NT * NCH * kXStride;
  static constexpr int kLKT = kLQK + 512;
  static constexpr int kLG = kLKT + NCH * 8 * 16 * 16 * 2;
  static constexpr int kLDq = kLG + NCH * 1024;
  static constexpr int kLFlag = kLDq + NCH * 64;
  static constexpr int kLHeads = kLFlag + 64;
  static constexpr int kHCoef = 0;
  static constexpr int kHLam = kHCoef + NCH * 64;
  static constexpr int kHFac = kHLam + (NCH == 1 ? 16 : 64);
  static constexpr int kHT0 = kHFac + NCH * 256;
  static constexpr int kHM = kHT0;
  static constexpr int kHR = kHM + NCH * 1024;
  static constexpr int kHeadLds = kHR + NCH * 1024;
  static constexpr int kHeads = NCH == 1 ? kMaxDecodeHeads : 1;
  static constexpr int kUnitBase = kLHeads + kHeads * kHeadLds;
};
static_assert(Lay<1>::kUnitBase == kUnitBase && Lay<1>::kHR == kHR && Lay<1>::kHFac == kHFac,
              "a one-chunk ring keeps the layout above");
// then per row wave: its v rows, token-major ([16 nch][64 vb + 16] bytes),
// and two buffers of one vblock's codes for the flush (4 blocks of 64 x 16
// bytes): the row wave's prefetch, and a helper's (a ring of nch > 1 chunks
// takes no helpers: the prefetch buffer only, so that two workgroups of
// its largest units share a compute unit; a wave of one vblock, 32 rows,
// needs neither)
constexpr int kVblockBytes = 4 * 64 * 16;
__host__ __device__ constexpr int row_wave_lds(int nch, int vb) {
  return NT * nch * (64 * vb + 16) + (vb > 1 ? (nch == 1 ? 2 : 1) : 0) * kVblockBytes;
}
// Vblocks of each row wave of a flushing unit that helpers rebuild (the
// last ones), given nhelp helper waves: the smallest longest chain
// max(vb - k, ceil(rpu k / nhelp)), at most one per helper (each helper job
// needs a buffer: the helped row wave's, or the partner unit's second), and
// at most kPartials / nwh per row wave (a value head's nwh row waves share
// its kPartials o-partial slots). nhelp is 0 when the partner unit flushes
// too: the workgroup's SIMDs are then busy with row waves, and a helper only
// lengthens the launch.
__device__ __forceinline__ int helper_vblocks(int vb, int rpu, int nhelp, int nwh) {
  int best = vb, kb = 0;
  for (int k = 1; k < vb && k <= nhelp && k * nwh <= kPartials; ++k) {
    const int crit = max(vb - k, (rpu * k + nhelp - 1) / nhelp);
    if (crit < best) {
      best = crit;
      kb = k;
    }
  }
  return kb;
}
__host__ __device__ constexpr int unit_lds(int nch, int rpu, int vb) {
  return (nch == 1 ? Lay<1>::kUnitBase : nch == 2 ? Lay<2>::kUnitBase : Lay<4>::kUnitBase) + rpu * row_wave_lds(nch, vb);
}

// raw bits of a gating input (f32, or the activation dtype) and their value
template <bool GATE_F32>
__device__ __forceinline__ uint32_t gate_bits(const uint8_t* p) {
  if constexpr (GATE_F32) return ld32(p);
  else return *(const uint16_t*)p;
}
template <bool GATE_F32>
__device__ __forceinline__ float gate_value(uint32_t bits) {
  if constexpr (GATE_F32) return __uint_as_float(bits);
  else return act_val(bits);
}

// Workgroup roles: wave 0 is the chain wave of the workgroup's key head (it
// streams no checkpoint rows: a wave whose loads back up in the memory
// pipeline cannot issue anything else, and the chain would wait behind
// them); waves 1 + NWH j + part own V-rows [64 part, +64) of value head j.
// The first kernel arguments (the key ring and checkpoint addressing, the
// ring length and the head grouping) are preloaded into SGPRs at wave launch
// (gfx950 kernarg preload, the build's -amdgpu-kernarg-preload-count): the
// first requests of every wave issue before any scalar load returns.
// Everything else comes from the StepArgs block.
template <int TPW, int NWH, int NCH, bool FUSED, bool GATE_F32, bool SLOTS>
__global__ __launch_bounds__(768) __attribute__((amdgpu_waves_per_eu(3))) void decode_kernel(
    uint8_t* ckpt, uint8_t* kring, uint32_t ck_b, uint32_t ck_h, uint32_t ck_v, uint32_t k_b, uint32_t k_t,
    uint32_t k_h, int32_t L, int32_t G, int32_t shape, const StepArgs a) {
  constexpr int ES = 2;
  // the LDS layout of an NCH-chunk ring (these shadow the one-chunk names)
  using LY = Lay<NCH>;
  constexpr int kLX = LY::kLX, kLQK = LY::kLQK, kLKT = LY::kLKT, kLG = LY::kLG, kLDq = LY::kLDq;
  constexpr int kLFlag = LY::kLFlag, kLHeads = LY::kLHeads, kHCoef = LY::kHCoef, kHLam = LY::kHLam;
  constexpr int kHFac = LY::kHFac, kHT0 = LY::kHT0, kHM = LY::kHM, kHR = LY::kHR, kHeadLds = LY::kHeadLds;
  constexpr int kUnitBase = LY::kUnitBase;
  // (row waves) stage their v rows, convert their codes and read back their
  // v words before the chain's flag, rather than after it: a ring of chunks,
  // and the small-batch shapes (waves of 32 or 64 rows), whose launches wait
  // on their chain; the headline shape (waves of 128 rows) waits on its stream
  constexpr bool kEarly = NCH > 1 || TPW <= 4;
  constexpr int RPW = 16 * TPW;           // V-rows per row wave
  constexpr int VB = TPW / 2;             // vblocks (32 rows) per row wave
  constexpr int VSTRIDE = RPW * ES + 16;  // LDS bytes per token of a row wave's v rows
  const int lane = threadIdx.x & 63;
  const int q4 = lane >> 4, l16 = lane & 15;
  const int w = uni(threadIdx.x >> 6);
  const int gw = shape & 0xFF, U = (shape >> 8) & 0xFF;  // value heads per unit, units per workgroup
  // workgroups numbered sequence-fastest (grid x = sequences) or head-fastest
  const bool seq_major = (shape >> 16) != 0;
  const int bx = (int)(seq_major ? blockIdx.y : blockIdx.x), by = (int)(seq_major ? blockIdx.x : blockIdx.y);
  const int rpu = gw * NWH;                     // row waves per unit
  const bool chain = w < U;                     // waves [0, U): the chain waves
  // (uniform indices: the divisions are VALU code, readfirstlane keeps the
  // results and every address built from them in SGPRs)
  const int u = uni(chain ? w : (w - U) / rpu);  // the wave's unit
  // the U units of a workgroup: SP consecutive sequences x HP consecutive
  // (key head, value-head group) pairs; a flushing sequence's heads spread
  // over several workgroups, a workgroup's codes over few rows of memory
  const int HP = U == 4 ? 2 : 1, SP = U == 4 ? 2 : U;
  const int uh = HP == 2 ? (u & 1) : 0, us = HP == 2 ? (u >> 1) : u;
  const int r = uni(bx * HP + uh);  // the unit's (key head, value-head group)
  const int n_grp = uni(G / gw);
  const int h = uni(r / n_grp), grp = r - h * n_grp, b0 = uni(by * SP + us);
  const int hv0 = h * G + grp * gw;              // first value head of the unit
  uint8_t* const ul = lds + u * unit_lds(NCH, rpu, TPW / 2);  // the unit's LDS block

  int bs = b0;
  if constexpr (SLOTS) {
    const int sl = (int)uni((int)ld_u32_uniform(a.slot + b0 * a.sl_s));
    bs = (sl >= 0 && sl < a.n_slots) ? sl : 0;
  }
  // per-sequence metadata (scalar; needed by every wave): the loads issue
  // early, the values are decoded where they are first needed
  struct MetaRaw {
    int n_raw, pos_raw;
    uint32_t flush_word, flush_shift;
  };
  auto load_meta = [&](const StepArgs& A, int bq) {
    MetaRaw m{(int)ld_u32_uniform(A.valid_len + bq * A.vl_s), -1, 0u, 0u};
    if constexpr (FUSED) m.pos_raw = (int)ld_u32_uniform(A.pos + bq * A.pos_s);
    if (A.flush) {
      const uintptr_t fa = (uintptr_t)(A.flush + bq * A.fl_s);
      m.flush_word = ld_u32_uniform((const void*)(fa & ~(uintptr_t)3));
      m.flush_shift = 8u * (uint32_t)(fa & 3);
    }
    return m;
  };
  auto decode_meta = [&](const MetaRaw& m, int& n, int& pos, bool& do_flush) {
    n = min(max(uni(m.n_raw), 0), L);
    pos = -1;
    if constexpr (FUSED) {
      const int p = uni(m.pos_raw);
      pos = (p >= 0 && p < L) ? p : -1;
    }
    do_flush = uni((int)((m.flush_word >> m.flush_shift) & 0xFFu)) != 0;
  };
  auto read_meta = [&](const StepArgs& A, int& n, int& pos, bool& do_flush) {
    decode_meta(load_meta(A, opaque_s(b0)), n, pos, do_flush);
  };

  // ---- the flush's rebuild of one vblock: 32 V-rows (tiles ii = 0, 1: rows
  // 32 p + 2 nn + ii of a row wave's block) on every ring token: P = X S_0^T,
  // W = v - pre P, U = R W, U~ = post U, then S_n = lam S_0 + K^T U~ by 16 x 4
  // column groups kept in registers; the vblock amax and o = S_n q as the
  // groups complete, then the requantisation in place. A row wave rebuilds
  // its own vblocks with it, and a chain wave whose chain is published
  // rebuilds the last ones of a flushing unit's row waves (the helpers
  // below). uu: the unit's LDS block, hb: the head's, vr: the row wave's v
  // rows, nf: the ring fill, c: the vblock's codes (cur layout), scp: its
  // scale, rows: the row wave's checkpoint rows, st: false when a wait the
  // rebuild depends on gave up (the codes are then not stored, the checkpoint
  // stays as it was). Returns the new scale and
  // this lane's shares op[ii] of o for the two tiles; after_pass1() runs once
  // the codes are no longer needed.
  //
  // S_n column group ct of tile ii: lane (nn, q4) gets
  // S_n[row r(ii, nn)][32 q4 + 4 ct + e], code byte 4 ct + e of its 32. The
  // update K^T U~ is one 16x16x32 MFMA per group with U~ split into hi + lo
  // halves (k-slots in utilde_operand's token order); its accumulator input
  // is lam S_0, or the codes alone when lam scale is folded out (below).
  auto flush_vblock = [&](const uint8_t* uu, const uint8_t* hb, const uint8_t* vr, int nf, const u32x4_t (&c)[2][2],
                          float scp, uint8_t* rows, int p, bool st, float* op, auto&& after_pass1) -> float {
    // (lam of the whole ring; of chunk 0 for a ring of NCH > 1 chunks)
    const float lamv = ((const float*)(hb + kHLam))[NCH == 1 ? 0 : 2];
    // One chunk, bf16 operands: ls = lam scale is folded out of the state.
    // The MFMA accumulates A = code + K^T (U~ / ls) (the codes enter
    // unscaled), the amax is ls max|A| (rounding is monotone, so it equals
    // the max of the rounded products), and the quotient multiplies A by
    // RN64(ls / s): for a state ls A that is a float this is within 2^-52 of
    // x / s, the bound quotient_f64 needs. That saves one multiply per
    // element. Taken while 1 / ls and U~ / ls stay in range.
    const float ls = lamv * scp;
    const bool fold = NCH == 1 && kBF16 && uni((int)(ls >= 0x1p-64f && ls <= 0x1p64f)) != 0;
    const float rls = fold ? __builtin_amdgcn_rcpf(ls) : 1.0f;  // (1 ulp: U~ / ls is an operand, not a result)
    u32x4_t packed[2];
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
      // P on the ring tokens, and on the query as a block of its own (every
      // A row is q; output row 0 is the one used)
      f32x4_t pr = {0.f, 0.f, 0.f, 0.f}, pq = pr;
      int xo = kLX + l16 * kXStride + 64 * q4, qo = kLQK + 64 * q4;
      asm volatile("" : "+v"(xo), "+v"(qo));  // read in the loop, not held across it
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const u32x4_t x = *(const u32x4_t*)(uu + xo + 16 * m);
        const u32x4_t qx = *(const u32x4_t*)(uu + qo + 16 * m);
        const u32x4_t bv = codes8(c[ii], m);
        pr = mfma16(x, bv, pr);
        pq = mfma16(qx, bv, pq);
      }
      float wv[4], post[4], dqt[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int t = 4 * q4 + e;
        const float4 fc = *(const float4*)(hb + kHFac + 16 * t);
        post[e] = fc.y;
        dqt[e] = fc.z;
        // v of token t for tile ii (zero at or past the fill)
        const uint32_t vw = *(const uint32_t*)(vr + t * VSTRIDE + (32 * p + 2 * l16) * ES);
        const float vv = act_val(ii ? (vw >> 16) : vw);
        wv[e] = t < nf ? vv - fc.x * (pr[e] * scp) : 0.f;
      }
      const float4 rr = *(const float4*)(hb + kHR + 4 * (l16 * NT + 4 * q4));
      const float rrv[4] = {rr.x, rr.y, rr.z, rr.w};
      f32x4_t uv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 4; ++e) uv = __builtin_amdgcn_mfma_f32_16x16x4f32(rrv[e], wv[e], uv, 0, 0, 0);
      // o = S_n q = lam (S_0 q) + sum_t U~_t (k_t . q): this lane's share
      float ut[4];
      // (pq[0] is S_0 q at every q4: counted at q4 == 0 only)
      float o = (q4 == 0 ? lamv * scp : 0.f) * pq[0];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ut[e] = uv[e] * post[e];
        o = fmaf(ut[e], dqt[e], o);
      }
      op[ii] = o;
      if constexpr (kBF16) {
        // hi/lo split: U~ (/ ls when folded) = hi + lo to ~16 bits, both
        // halves bf16 operands
        const float u0 = ut[0] * rls, u1 = ut[1] * rls, u2 = ut[2] * rls, u3 = ut[3] * rls;
        const uint32_t h01 = pack_bf16x2(u0, u1), h23 = pack_bf16x2(u2, u3);
        const uint32_t l01 = pack_bf16x2(u0 - __uint_as_float(h01 << 16), u1 - __uint_as_float(h01 & 0xFFFF0000u));
        const uint32_t l23 = pack_bf16x2(u2 - __uint_as_float(h23 << 16), u3 - __uint_as_float(h23 & 0xFFFF0000u));
        packed[ii] = utilde_operand(h01, h23, l01, l23);
      } else {
        _Float16 hh[4], ll[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          hh[e] = (_Float16)ut[e];
          ll[e] = (_Float16)(ut[e] - (float)hh[e]);
        }
        auto pk = [](_Float16 x, _Float16 y) {
          return (uint32_t)__builtin_bit_cast(uint16_t, x) | ((uint32_t)__builtin_bit_cast(uint16_t, y) << 16);
        };
        packed[ii] = utilde_operand(pk(hh[0], hh[1]), pk(hh[2], hh[3]), pk(ll[0], ll[1]), pk(ll[2], ll[3]));
      }
    }
    // pass 1: S_n of the vblock's 2 x 8 column groups (kept) and the vblock
    // amax (|x| max, NaN propagating like torch.amax). lam scale S_0 is the
    // MFMA's accumulator input: lane (nn, q4)'s four outputs of group ct are
    // the columns of its own code bytes 4 ct .. 4 ct + 3, so each lane forms
    // them from its codes (one f32 rounding of lam scale x code).
    f32x4_t sv[2][8];
    float am = 0.f;
    {
      auto pass1 = [&](auto folded) {
#pragma unroll
        for (int ct = 0; ct < 8; ++ct) {
#pragma unroll
          for (int ii = 0; ii < 2; ++ii) {
            const uint32_t cw4 = c[ii][ct >> 2][ct & 3];
            const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)cw4, false);
            const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)cw4, true);
            const f32x4_t s0 = decltype(folded)::value ? f32x4_t{lo[0], lo[1], hi[0], hi[1]}
                                                       : f32x4_t{ls * lo[0], ls * lo[1], ls * hi[0], ls * hi[1]};
            const u32x4_t k8 = *(const u32x4_t*)(uu + kLKT + 32 * (ct * 16 + l16) + 16 * (q4 & 1));
            sv[ii][ct] = mfma16(k8, packed[ii], s0);
          }
        }
      };
      if (fold)
        pass1(std::true_type{});
      else
        pass1(std::false_type{});
      if constexpr (NCH > 1) {
        // (the codes are not needed past chunk 0)
        after_pass1();
        // chunks 1.. in turn, from the state so far (sv, f32), the one-chunk
        // rebuild with S for lam scale S_0: P = X_c S^T with S as 16-bit
        // hi + lo operands (two MFMAs per k-step), W = v - pre P,
        // U = R_c W, U~ = post U, S <- lam_c S + K_c^T U~ (lam_c S the
        // MFMA's accumulator input), o <- lam_c o + sum_t U~_t (k_t . q)
#pragma unroll 1
        for (int cc = 1; cc < NCH; ++cc) {
          if (NT * cc >= nf) break;
          const float lc = ((const float*)(hb + kHLam))[2 + cc];
          u32x4_t pk2[2];
#pragma unroll
          for (int ii = 0; ii < 2; ++ii) {
            f32x4_t pr = {0.f, 0.f, 0.f, 0.f};
            int xo = kLX + (NT * cc + l16) * kXStride + 64 * q4;
            asm volatile("" : "+v"(xo));
#pragma unroll
            for (int m = 0; m < 4; ++m) {
              const u32x4_t x = *(const u32x4_t*)(uu + xo + 16 * m);
              const f32x4_t a0 = sv[ii][2 * m], a1 = sv[ii][2 * m + 1];
              const float v8[8] = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
              uint32_t hi[4], lo[4];
#pragma unroll
              for (int w2 = 0; w2 < 4; ++w2) {
                const uint32_t hb2 = act_bits(v8[2 * w2]) | (act_bits(v8[2 * w2 + 1]) << 16);
                const float2 hv = Act::from_pair(hb2);
                hi[w2] = hb2;
                lo[w2] = act_bits(v8[2 * w2] - hv.x) | (act_bits(v8[2 * w2 + 1] - hv.y) << 16);
              }
              pr = mfma16(x, u32x4_t{hi[0], hi[1], hi[2], hi[3]}, pr);
              pr = mfma16(x, u32x4_t{lo[0], lo[1], lo[2], lo[3]}, pr);
            }
            float wv[4], post[4], dqt[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int t = NT * cc + 4 * q4 + e;
              const float4 fc = *(const float4*)(hb + kHFac + 16 * t);
              post[e] = fc.y;
              dqt[e] = fc.z;
              const uint32_t vw = *(const uint32_t*)(vr + t * VSTRIDE + (32 * p + 2 * l16) * ES);
              const float vv = act_val(ii ? (vw >> 16) : vw);
              wv[e] = t < nf ? vv - fc.x * pr[e] : 0.f;
            }
            const float4 rr = *(const float4*)(hb + kHR + 1024 * cc + 4 * (l16 * NT + 4 * q4));
            const float rrv[4] = {rr.x, rr.y, rr.z, rr.w};
            f32x4_t uv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int e = 0; e < 4; ++e) uv = __builtin_amdgcn_mfma_f32_16x16x4f32(rrv[e], wv[e], uv, 0, 0, 0);
            float ut[4];
            float o = lc * op[ii];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              ut[e] = uv[e] * post[e];
              o = fmaf(ut[e], dqt[e], o);
            }
            op[ii] = o;
            uint32_t h2[2], l2[2];
#pragma unroll
            for (int w2 = 0; w2 < 2; ++w2) {
              h2[w2] = act_bits(ut[2 * w2]) | (act_bits(ut[2 * w2 + 1]) << 16);
              const float2 hv = Act::from_pair(h2[w2]);
              l2[w2] = act_bits(ut[2 * w2] - hv.x) | (act_bits(ut[2 * w2 + 1] - hv.y) << 16);
            }
            pk2[ii] = utilde_operand(h2[0], h2[1], l2[0], l2[1]);
          }
#pragma unroll
          for (int ct = 0; ct < 8; ++ct) {
#pragma unroll
            for (int ii = 0; ii < 2; ++ii) {
              const u32x4_t k8 = *(const u32x4_t*)(uu + kLKT + cc * (8 * 16 * 16 * 2) + 32 * (ct * 16 + l16) +
                                                   16 * (q4 & 1));
              const f32x4_t acc = sv[ii][ct] * lc;
              sv[ii][ct] = mfma16(k8, pk2[ii], acc);
            }
          }
        }
      }
      // (two running maxima, each taking two elements per instruction)
      float am1 = 0.f;
#pragma unroll
      for (int ct = 0; ct < 8; ++ct) {
#pragma unroll
        for (int ii = 0; ii < 2; ++ii) {
          const f32x4_t sg = sv[ii][ct];
          am = max3_abs(am, sg[0], sg[1]);
          am1 = max3_abs(am1, sg[2], sg[3]);
        }
      }
      am = __builtin_elementwise_maximum(am, am1);
    }
    if constexpr (NCH == 1) after_pass1();
    // the reference quantiser (ref:36-37,83-99): s = amax / 448 (1 when amax
    // is not > 0); codes = e4m3fn(clamp(x / s, +-448)) with the unrounded s;
    // the quotient by quotient_f64 when the block is finite (x = xs A)
    const float xs = fold ? ls : 1.0f;
    const float amax = xs * __uint_as_float(wave_max_u32(__float_as_uint(am)));
    const float s32 = (amax > 0.0f) ? amax / 448.0f : 1.0f;
    const bool fast = quotient_fast(__float_as_uint(amax), s32);
    const double r64 = (double)xs / (double)s32;
    // pass 2: the kept column groups requantised and stored (the division
    // path of non-finite or tiny-scale blocks is a loop of its own)
    auto pass2 = [&](auto quant) {
#pragma unroll
      for (int ii = 0; ii < 2; ++ii) {
        const uint32_t ro = (uint32_t)(32 * p + 2 * l16 + ii) * ck_v + 32 * q4;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          uint32_t wd[4];
#pragma unroll
          for (int w4 = 0; w4 < 4; ++w4) wd[w4] = quant(sv[ii][4 * hh + w4]);
          if (st) *(g_u32x4_w*)(rows + ro + 16 * hh) = u32x4_t{wd[0], wd[1], wd[2], wd[3]};
        }
      }
    };
    if (uni((int)fast) != 0) {
      pass2([&](const f32x4_t& v) {
        return f32x4_to_fp8(quotient_f64(v[0], r64), quotient_f64(v[1], r64), quotient_f64(v[2], r64),
                            quotient_f64(v[3], r64));
      });
    } else {
      // (one quotient at a time: this path is rare and should hold few registers)
      pass2([&](const f32x4_t& v) {
        __builtin_amdgcn_sched_barrier(0);
        float qv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          qv[e] = (xs * v[e]) / s32;
          __builtin_amdgcn_sched_barrier(0);
        }
        const uint32_t wd = f32x4_to_fp8_ref_cold(qv[0], qv[1], qv[2], qv[3]);
        __builtin_amdgcn_sched_barrier(0);
        return wd;
      });
    }
    return s32;
  };
  // DMA of one vblock's codes (rows 32 pv + 2 nn + ii of `rows`) into a
  // buffer in the cur layout: block k = 2 ii + hh, lane (nn, q4) gets bytes
  // [32 q4 + 16 hh, +16) of its row
  auto dma_vblock = [&](const uint8_t* rows, int pv, const uint8_t* buf) {
    const uint32_t ba = (uint32_t)uni((int)(uint32_t)(uintptr_t)buf);
#pragma unroll
    for (int k = 0; k < 4; ++k)
      dma16(rows + (uint32_t)(32 * pv + 2 * l16 + (k >> 1)) * ck_v + 32 * q4 + 16 * (k & 1), ba + 1024 * k);
  };
  // the partner unit: the same (key head, value-head group) in the
  // workgroup's other sequence (b0 ^ 1); while it does not flush, its chain
  // wave and buffers help a flushing unit
  const bool has_partner = U >= 2;
  const int up = U == 4 ? (u ^ 2) : (u ^ 1);
  auto partner_flushes = [&](const StepArgs& A) {
    int pn, ppos;
    bool pfl;
    decode_meta(load_meta(A, opaque_s(b0 ^ 1)), pn, ppos, pfl);
    return pfl;
  };

  if (chain) {
    // ================= chain wave =================================================
    // (the sequence index through opaque_s: addresses from the argument block
    // are formed here, not in code shared with the row waves)
    const int b = opaque_s(b0);
    // the unit's flags start clear; the row waves read them only after barrier 1
    if (lane < 16) ((volatile int*)(ul + kLFlag))[lane] = 0;
    GDNR_WAIT_LGKM0();
    // Lane (t = l16, row q4). For the gates, the coefficient chain and the
    // flush factors, row j holds value head hv0 + j of the unit (rows at or
    // past gw repeat the last head and publish nothing): the heads advance in
    // the same instructions.
    const int jr = q4 < gw ? q4 : gw - 1;
    const bool pub = q4 < gw;
    const int hvr = hv0 + jr;
    // ---- loads: the key ring in the X layout (all 16 rows; rows at or past
    // the fill are zeroed below), the metadata, the query / new-token rows,
    // the gates (lane (t, j): token t of head j). A ring of NCH > 1 chunks
    // loads NCH blocks of 16 rows (chunk c row t: slot 16 c + t), and its
    // one value head's gates by token: lane (t, q4) holds token 16 q4 + t.
    const int tl = l16 < L ? l16 : 0;
    const uint8_t* krow = sbase(kring, bs, k_b) + (h * k_h + (uint32_t)tl * k_t) + 64 * q4;
    u32x4_t xr[NCH][4];
#pragma unroll
    for (int m = 0; m < 4; ++m) xr[0][m] = ld16(krow + 16 * m);
#pragma unroll
    for (int c = 1; c < NCH; ++c) {
      const int tc = NT * c + l16;
      const uint8_t* kc = sbase(kring, bs, k_b) + (h * k_h + (uint32_t)(tc < L ? tc : 0) * k_t) + 64 * q4;
#pragma unroll
      for (int m = 0; m < 4; ++m) xr[c][m] = ld16(kc + 16 * m);
    }
    const int tk = NT * q4 + l16;           // (NCH > 1) the token of this lane's gates and chain
    const int tg = NCH == 1 ? tl : (tk < L ? tk : 0);
    GDNR_COMPILER_FENCE();
    const MetaRaw meta = load_meta(a, b);
    MetaRaw pmeta{};
    if (has_partner) pmeta = load_meta(a, b ^ 1);
    uint32_t qbits, kbits = 0;
    if constexpr (FUSED) {
      const uint8_t* row = a.mixed + b * a.mx_b;
      qbits = ld32(row + (h * K + 2 * lane) * ES);
      kbits = ld32(row + (a.H * K + h * K + 2 * lane) * ES);
    } else {
      qbits = ld32(a.q + (b * a.q_b + h * a.q_h) + 4 * lane);
    }
    const uint32_t g_raw = *(const uint16_t*)(sbase(a.g, bs, a.g_b) + off_sum((uint32_t)tg * a.g_t, hvr * a.g_h));
    const uint32_t be_raw =
        *(const uint16_t*)(sbase(a.beta, bs, a.be_b) + off_sum((uint32_t)tg * a.be_t, hvr * a.be_h));
    uint32_t ab0 = 0, ab1 = 0;
    float alog = 0.f, dtb = 0.f;
    if constexpr (FUSED) {
      ab0 = gate_bits<GATE_F32>(a.a + off_sum(b * a.a_b, hvr * a.a_h));
      ab1 = gate_bits<GATE_F32>(a.bgate + off_sum(b * a.bg_b, hvr * a.bg_h));
      alog = *(const float*)(a.a_log + hvr * a.al_s);
      dtb = *(const float*)(a.dt_bias + hvr * a.db_s);
    }
    // (barrier 1: the chain requests of the workgroup enter the memory
    // pipeline before any checkpoint row; the row waves wait here)
    GDNR_COMPILER_FENCE();
    __builtin_amdgcn_s_barrier();
    GDNR_COMPILER_FENCE();
    int n, pos;
    bool do_flush;
    decode_meta(meta, n, pos, do_flush);
    const bool full = n >= NT;
    // every load above is needed next; waiting for them here keeps later
    // waits from covering the ring-append stores
    GDNR_WAIT_VMCNT(0);

    // ---- flush helper, set-up: this wave rebuilds vblocks of a flushing unit
    // v, its own (helper 0) or, while its own unit replays, the partner unit
    // (helper 1): the last nh vblocks of each of v's row waves, jobs
    // g = kk rpu + w (vblock VB - nh + kk of row wave w) split evenly between
    // v's helpers. Job (kk, w) reads its codes into row wave w's second
    // buffer, of v for kk = 0 and of v's partner for kk = 1 (a replaying
    // unit's are unused). The DMAs and the rebuilds follow the chain's
    // publication (issued earlier, the DMAs would sit in the memory pipeline
    // ahead of what the chain and the row waves wait for).
    int hv_unit = -1, h_nh = 0, h_g0 = 0, h_g1 = 0, h_nf = n, h_bs = bs;
    {
      int pn = 0, ppos;
      bool pfl = false;
      if (has_partner) decode_meta(pmeta, pn, ppos, pfl);
      int hidx = 0, nhelp = NCH == 1 ? 1 : 0;
      if (do_flush) {
        hv_unit = u;
        if constexpr (NCH == 1) nhelp = has_partner ? (pfl ? 0 : 2) : 1;
      } else if (NCH == 1 && has_partner && pfl) {
        hv_unit = up;
        hidx = 1;
        nhelp = 2;
        h_nf = pn;
        h_bs = b ^ 1;
        if constexpr (SLOTS) {
          const int sl = (int)uni((int)ld_u32_uniform(a.slot + (b ^ 1) * a.sl_s));
          h_bs = (sl >= 0 && sl < a.n_slots) ? sl : 0;
        }
      }
      hv_unit = uni(hv_unit);
      if (hv_unit >= 0 && nhelp > 0) {
        h_nh = uni(helper_vblocks(VB, rpu, nhelp, NWH));
        const int jobs = h_nh * rpu, per = (jobs + nhelp - 1) / nhelp;
        h_g0 = uni(hidx * per);
        h_g1 = uni(min(jobs, h_g0 + per));
      }
    }
    auto job_rows = [&](int wv) {
      return sbase(ckpt, h_bs, ck_b) + ((hv0 + wv / NWH) * ck_h + RPW * (wv % NWH) * ck_v);
    };
    auto job_buf = [&](int kk, int wv) {
      const int bu = kk == 0 ? hv_unit : (hv_unit == u ? up : u);
      return lds + bu * unit_lds(NCH, rpu, VB) + kUnitBase + wv * row_wave_lds(NCH, VB) + NT * NCH * VSTRIDE +
             kVblockBytes;
    };

    // ---- the query (and new key) rows: normalised as the preparation does
    // (x / sqrt(sum x^2 + 1e-6), lane pairs, rounded to the ring dtype); the
    // pair layout is the row form: element c at byte 2 c
    {
      const float2 qr = Act::from_pair(qbits);
      uint32_t qw, kw = 0;
      if constexpr (FUSED) {
        const float2 kr = Act::from_pair(kbits);
        const float qd = sqrtf(wave_sum(fmaf(qr.y, qr.y, qr.x * qr.x)) + 1e-6f);
        const float kd = sqrtf(wave_sum(fmaf(kr.y, kr.y, kr.x * kr.x)) + 1e-6f);
        qw = act_bits(Act::round(qr.x / qd)) | (act_bits(Act::round(qr.y / qd)) << 16);
        kw = act_bits(Act::round(kr.x / kd)) | (act_bits(Act::round(kr.y / kd)) << 16);
        // q_out and the ring append of the new key (one unit per key head)
        if (grp == 0) {
          *(uint32_t*)(a.q_out + (b * a.qo_b + h * a.qo_h) + 4 * lane) = qw;
          if (pos >= 0) *(uint32_t*)(sbase(kring, bs, k_b) + ((uint32_t)pos * k_t + h * k_h) + 4 * lane) = kw;
        }
      } else {
        qw = qbits;
      }
      *(uint32_t*)(ul + kLQK + 4 * lane) = qw;
      *(uint32_t*)(ul + kLQK + 256 + 4 * lane) = kw;
    }
    if constexpr (NCH == 1) {
    // ---- X rows: t < n the ring (the new token's own row at t == pos), t == n
    // the query, the rest zero (a full ring, n == 16, takes the query as a
    // block of its own: the q row of kLQK); written to LDS in row form
    u32x4_t xa[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int off = 64 * q4 + 16 * m;
      const u32x4_t z = {0u, 0u, 0u, 0u};
      const u32x4_t qv = *(const u32x4_t*)(ul + kLQK + off);
      u32x4_t x = l16 < n ? xr[0][m] : (l16 == n ? qv : z);
      if constexpr (FUSED) {
        const u32x4_t kv = *(const u32x4_t*)(ul + kLQK + 256 + off);
        x = (l16 == pos && l16 < n) ? kv : x;
      }
      xa[m] = x;
      *(u32x4_t*)(ul + kLX + l16 * kXStride + off) = x;
    }
    // (a replay's row waves take the X rows as their product operands: they
    // start on them now, not at the flag that publishes the weights)
    if (!do_flush) {
      GDNR_WAIT_LGKM0();
      if (lane == 0)
        __hip_atomic_store((int*)(ul + kLFlag) + kFlagXRows, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    // ---- Gram matrix G = X X^T (rows t < n; the query row n gives k_t . q)
    f32x4_t gacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 4; ++m) gacc = mfma16(xa[m], xa[m], gacc);
    float* Gs = (float*)(ul + kLG);
    float* Dq = (float*)(ul + kLDq);
    // G[4 q4 + e][u] at lane (u, q4) is row u, columns 4 q4 + e (symmetric)
    *(float4*)(Gs + l16 * 16 + 4 * q4) = make_float4(gacc[0], gacc[1], gacc[2], gacc[3]);
    if (full) {
      f32x4_t dacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int off = 64 * q4 + 16 * m;
        const u32x4_t qv = *(const u32x4_t*)(ul + kLQK + off);
        dacc = mfma16(xa[m], l16 == 0 ? qv : u32x4_t{0u, 0u, 0u, 0u}, dacc);
      }
      if (l16 == 0) *(float4*)(Dq + 4 * q4) = make_float4(dacc[0], dacc[1], dacc[2], dacc[3]);
    }
    const bool on = l16 < n;
    float gcol[NT];  // G[lane token][t], zero for t >= n
    {
      const float4* gr = (const float4*)(Gs + l16 * 16);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 v4 = gr[i];
        gcol[4 * i] = v4.x, gcol[4 * i + 1] = v4.y, gcol[4 * i + 2] = v4.z, gcol[4 * i + 3] = v4.w;
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) gcol[t] = t < n ? gcol[t] : 0.f;
    }
    const float dq = on ? (full ? Dq[l16] : Gs[l16 * 16 + (full ? 0 : n)]) : 0.f;
    if (do_flush) {
      // K^T operand tiles [ct][M][position] (flush): element (t, col) of X
      // with col = 32 q4 + 8 m + j8 goes to tile ct = 2 m + j8 / 4, row
      // M = 4 q4 + j8 % 4 (tile ct, row M: column 32 (M >> 2) + 4 ct + (M & 3)),
      // position kt_pos(t); tokens t >= n are zero
      uint16_t* kt = (uint16_t*)(ul + kLKT);
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const u32x4_t x = on ? xa[m] : u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
        for (int j8 = 0; j8 < 8; ++j8) {
          const uint16_t e16 = (uint16_t)((x[j8 >> 1] >> (16 * (j8 & 1))) & 0xFFFFu);
          kt[((2 * m + (j8 >> 2)) * 16 + 4 * q4 + (j8 & 3)) * 16 + kt_pos(l16)] = e16;
        }
      }
    }

    // ---- per row (value head): gates, then the coefficient chain or the flush factors
    uint8_t* hl = ul + kLHeads + jr * kHeadLds;
    float gg = act_val(g_raw);
    float bb = act_val(be_raw);
    if constexpr (FUSED) {
      // the new token's gates from the preparation formulas (kernel:534-562)
      const float a_in = gate_value<GATE_F32>(ab0), b_in = gate_value<GATE_F32>(ab1);
      const float x = a_in + dtb;
      const float sp = x <= 20.0f ? logf(1.0f + expf(x)) : x;  // kernel:560, as written there
      const float gate_new = Act::round(-expf(alog) * sp);
      const float beta_new = Act::round(1.0f / (1.0f + expf(-b_in)));
      if (pos >= 0 && l16 == 0 && pub) {
        *(uint16_t*)(sbase(a.g, bs, a.g_b) + ((uint32_t)pos * a.g_t + hvr * a.g_h)) = (uint16_t)act_bits(gate_new);
        *(uint16_t*)(sbase(a.beta, bs, a.be_b) + ((uint32_t)pos * a.be_t + hvr * a.be_h)) = (uint16_t)act_bits(beta_new);
      }
      gg = l16 == pos ? gate_new : gg;
      bb = l16 == pos ? beta_new : bb;
    }
    const float gam = on ? expf(gg) : 1.f;
    const float bet = on ? bb : 0.f;
    const float suf_in = row_suffix_prod(gam);
    const float suf_ex = dpp_row<0x101>(suf_in, 1.f);
    const float lam = row_bcast<0>(suf_in);
    if (l16 == 0 && pub) ((float*)(hl + kHLam))[0] = lam;
    if (!do_flush) {
      // s_t, t descending: acc_l = sum_{u > t} G[l][u] s_u
      float acc = 0.f, s_mine = 0.f;
#pragma unroll
      for (int t = NT - 1; t >= 0; --t) {
        const float sv = row_bcast_n(bet * (dq - acc), t);
        s_mine = l16 == t ? sv : s_mine;
        acc = fmaf(gcol[t], sv, acc);
      }
      const float c = on ? s_mine * suf_ex : 0.f;
      // the weights alpha of the X rows: T_0 = sum_t alpha_t X_t (+ lam q for a
      // full ring) = lam (q - sum_t s_t k_t), the reference's transformed
      // query; the row waves weight their products S_0 X_t^T with them
      const float al = on ? -lam * s_mine : (l16 == n ? lam : 0.f);
      if (pub) {
        ((float*)(hl + kHCoef))[l16] = c;
        ((float*)(hl + kHT0))[l16] = al;
      }
    } else {
      // flush factors (kernel:177-242 in matrix form):
      //   pre_t = prod_{x<=t} gamma_x,  post_t = beta_t prod_{x>t} gamma_x,
      //   M[t][s] = beta_s prod_{s<x<=t} gamma_x G[s][t] (s < t < n), R = (I + M)^-1
      const float pre = row_prefix_prod(gam);
      const float post = bet * suf_ex;
      if (pub) ((float4*)(hl + kHFac))[l16] = make_float4(on ? pre : 0.f, on ? post : 0.f, dq, 0.f);
      // M (lane = column s; the gammas of the row by row broadcast)
      float* Mm = (float*)(hl + kHM);
      {
        float run = 1.f;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const float gt = row_bcast_n(gam, t);
          run = t > l16 ? run * gt : run;
          if (pub) Mm[t * NT + l16] = (l16 < t && t < n) ? bet * run * gcol[t] : 0.f;
        }
      }
      // R by forward substitution, lane = column c:
      // R[t][c] = delta_tc - sum_{s<t} M[t][s] R[s][c]
      float r[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        float x = (t == l16) ? 1.f : 0.f;
#pragma unroll
        for (int s4 = 0; s4 < t; s4 += 4) {
          const float4 m4 = *(const float4*)(Mm + t * NT + s4);
          x = fmaf(-m4.x, r[s4], x);
          if (s4 + 1 < t) x = fmaf(-m4.y, r[s4 + 1], x);
          if (s4 + 2 < t) x = fmaf(-m4.z, r[s4 + 2], x);
          if (s4 + 3 < t) x = fmaf(-m4.w, r[s4 + 3], x);
        }
        r[t] = x;
      }
      if (pub) {
        float* Rj = (float*)(hl + kHR);
#pragma unroll
        for (int t = 0; t < NT; ++t) Rj[t * NT + l16] = (t < n && on) ? r[t] : 0.f;
      }
    }
    } else {
    // ---- a ring of NCH chunks, one value head (hv0). X rows: the keys only
    // (tokens at or past the fill zero, the new token's own row at pos),
    // row form in LDS and the A operand in registers, per chunk. Chunks past
    // the fill are not formed (nothing reads them), and only the chunk that
    // holds the fill, or the new token, needs a select.
    u32x4_t xa[NCH][4];
    const int pc = (FUSED && pos >= 0 && pos < n) ? pos / NT : -1;  // chunk of the new token's row
    // (the new key's row in operand form, read once: a read inside the
    // chunk's branch would wait for it there)
    u32x4_t kv[4];
#pragma unroll
    for (int m = 0; m < 4; ++m)
      kv[m] = FUSED ? *(const u32x4_t*)(ul + kLQK + 256 + 64 * q4 + 16 * m) : u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
    for (int m = 0; m < 4; ++m) asm volatile("" : "+v"(kv[m]));
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
#pragma unroll
      for (int m = 0; m < 4; ++m) xa[c][m] = xr[c][m];  // (a chunk past the fill: its Gram is not used)
      if (NT * c >= n) continue;
      const int t = NT * c + l16;
      const bool keep = t < n, isnew = c == pc && t == pos;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int off = 64 * q4 + 16 * m;
        u32x4_t x = isnew ? kv[m] : xr[c][m];
        x = keep ? x : u32x4_t{0u, 0u, 0u, 0u};
        xa[c][m] = x;
        *(u32x4_t*)(ul + kLX + t * kXStride + off) = x;
      }
    }
    float* Gs = (float*)(ul + kLG);
    float* Dq = (float*)(ul + kLDq);
    // (replay) the ring's whole Gram matrix, row t at float kGfStride t: the
    // K^T tiles' area, which only a flush uses
    static_assert(NT * NCH * kGfStride * 4 <= kLDq - kLKT, "the full Gram must fit the K^T and Gram blocks");
    float* Gf = (float*)(ul + kLKT);
    if (do_flush) {
      // Gram block of each chunk, G_c = X_c X_c^T (the chunks' products
      // interleaved: four independent accumulations), k_t . q of every
      // token, and the chunks' K^T operand tiles (as for one chunk)
      f32x4_t gacc[NCH], dacc[NCH];
#pragma unroll
      for (int c = 0; c < NCH; ++c) gacc[c] = dacc[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const u32x4_t qv = *(const u32x4_t*)(ul + kLQK + 64 * q4 + 16 * m);
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
          gacc[c] = mfma16(xa[c][m], xa[c][m], gacc[c]);
          dacc[c] = mfma16(xa[c][m], l16 == 0 ? qv : u32x4_t{0u, 0u, 0u, 0u}, dacc[c]);
        }
      }
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        if (NT * c >= n) continue;
        *(float4*)(Gs + c * 256 + l16 * 16 + 4 * q4) = make_float4(gacc[c][0], gacc[c][1], gacc[c][2], gacc[c][3]);
        if (l16 == 0) *(float4*)(Dq + NT * c + 4 * q4) = make_float4(dacc[c][0], dacc[c][1], dacc[c][2], dacc[c][3]);
        uint16_t* kt = (uint16_t*)(ul + kLKT) + c * (8 * 16 * 16);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const u32x4_t x = xa[c][m];
#pragma unroll
          for (int j8 = 0; j8 < 8; ++j8) {
            const uint16_t e16 = (uint16_t)((x[j8 >> 1] >> (16 * (j8 & 1))) & 0xFFFFu);
            kt[((2 * m + (j8 >> 2)) * 16 + 4 * q4 + (j8 & 3)) * 16 + kt_pos(l16)] = e16;
          }
        }
      }
    } else {
      // the upper tiles of the ring's Gram matrix, G[16 r + i][16 c + j]
      // for r <= c, and k_t . q of every token: for each chunk c in the ring
      // (group c) the products X_c X_r^T (r <= c) and X_c q interleaved.
      // Lane (j, q4) of the tile X_c X_r^T holds G[16 c + 4 q4 + e][16 r + j],
      // which is G[16 r + j][16 c + 4 q4 + e]: one float4 of row 16 r + j.
      // Groups c >= kChainGroups are the row waves' (they read the X rows
      // from LDS once the flag is up), the first ones this wave's.
      GDNR_WAIT_LGKM0();
      if (lane == 0)
        __hip_atomic_store((int*)(ul + kLFlag) + kFlagXRows, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
      u32x4_t qb[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const u32x4_t qv = *(const u32x4_t*)(ul + kLQK + 64 * q4 + 16 * m);
        qb[m] = l16 == 0 ? qv : u32x4_t{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int c = 0; c < (NCH < kChainGroups ? NCH : kChainGroups); ++c) {
        if (NT * c >= n) continue;
        f32x4_t tacc[NCH], dacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int r = 0; r <= c; ++r) tacc[r] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < 4; ++m) {
#pragma unroll
          for (int r = 0; r <= c; ++r) tacc[r] = mfma16(xa[c][m], xa[r][m], tacc[r]);
          dacc = mfma16(xa[c][m], qb[m], dacc);
        }
#pragma unroll
        for (int r = 0; r <= c; ++r) {
          f32x4_t g = tacc[r];
          if (r == c) {
            // (the diagonal tile keeps its strict upper part only: u > t)
#pragma unroll
            for (int e = 0; e < 4; ++e) g[e] = 4 * q4 + e > l16 ? g[e] : 0.f;
          }
          *(float4*)(Gf + (NT * r + l16) * kGfStride + NT * c + 4 * q4) = make_float4(g[0], g[1], g[2], g[3]);
        }
        if (l16 == 0) *(float4*)(Dq + NT * c + 4 * q4) = make_float4(dacc[0], dacc[1], dacc[2], dacc[3]);
      }
    }
    // lane (t, q4): token tk = 16 q4 + t, of chunk q4; its gates
    const bool on = tk < n;
    uint8_t* hl = ul + kLHeads;
    float gg = act_val(g_raw);
    float bb = act_val(be_raw);
    if constexpr (FUSED) {
      const float a_in = gate_value<GATE_F32>(ab0), b_in = gate_value<GATE_F32>(ab1);
      const float x = a_in + dtb;
      const float sp = x <= 20.0f ? logf(1.0f + expf(x)) : x;  // kernel:560, as written there
      const float gate_new = Act::round(-expf(alog) * sp);
      const float beta_new = Act::round(1.0f / (1.0f + expf(-b_in)));
      if (pos >= 0 && lane == 0) {
        *(uint16_t*)(sbase(a.g, bs, a.g_b) + ((uint32_t)pos * a.g_t + hvr * a.g_h)) = (uint16_t)act_bits(gate_new);
        *(uint16_t*)(sbase(a.beta, bs, a.be_b) + ((uint32_t)pos * a.be_t + hvr * a.be_h)) = (uint16_t)act_bits(beta_new);
      }
      gg = tk == pos ? gate_new : gg;
      bb = tk == pos ? beta_new : bb;
    }
    const float gam = on ? expf(gg) : 1.f;
    const float bet = on ? bb : 0.f;
    const float suf_in = row_suffix_prod(gam);    // within the chunk (a 16-lane row)
    const float suf_ex = dpp_row<0x101>(suf_in, 1.f);
    const float lamc = row_bcast<0>(suf_in);      // lam_c of the lane's chunk
    if (!do_flush) {
      // Replay: the one-chunk recurrence over the whole ring,
      // s_t = beta_t (k_t . q - sum_{u > t} G_tu s_u) (tokens from the last
      // to the first, kernel:121-173 read as in the one-chunk chain), with
      // c_t = s_t prod_{u > t} gamma_u and T_0 = lam (q - sum_t s_t k_t).
      // Lane tk holds row tk of G from the later chunks' tiles and the strict
      // upper part of its own chunk's (so that its sum stops at its own
      // token within the chunk; it takes its s at the chunk's end); s_t of
      // each step is read from its lane (uniform) and T_0's sum accumulated
      // with it.
      (void)wait_count((int*)(ul + kLFlag) + kFlagGram, rpu, a.status, a.wait_polls);  // (the row waves' groups)
      float gb[NCH][NT];
      {
        float4 g4[NCH][4];
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            g4[c][i] = NT * c < n ? *(const float4*)(Gf + tk * kGfStride + NT * c + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            gb[c][4 * i] = g4[c][i].x, gb[c][4 * i + 1] = g4[c][i].y;
            gb[c][4 * i + 2] = g4[c][i].z, gb[c][4 * i + 3] = g4[c][i].w;
          }
      }
      const float bd = on ? bet * Dq[tk] : 0.f;
      float acc = 0.f, ax = 0.f, ay = 0.f, s_mine = 0.f;
#pragma unroll
      for (int c = NCH - 1; c >= 0; --c) {
        if (NT * c >= n) continue;
        // (the chunk's 16 key words of this lane's columns, read at once: one
        // wait for them all rather than one every step)
        uint32_t xw[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) xw[t] = *(const uint32_t*)(ul + kLX + (NT * c + t) * kXStride + 4 * lane);
#pragma unroll
        for (int t = 0; t < NT; ++t) asm volatile("" : "+v"(xw[t]));
#pragma unroll
        for (int t = NT - 1; t >= 0; --t) {
          const float st = rdl(fmaf(-bet, acc, bd), NT * c + t);
          acc = fmaf(gb[c][t], st, acc);
          const float2 xv = Act::from_pair(xw[t]);
          ax = fmaf(st, xv.x, ax);
          ay = fmaf(st, xv.y, ay);
        }
        s_mine = q4 == c ? fmaf(-bet, acc, bd) : s_mine;
      }
      // prod_{u > t} gamma_u over the ring: within the lane's chunk, then the
      // later chunks' lam_c
      const float l1 = rdl(lamc, NT), l2 = NCH > 2 ? rdl(lamc, 2 * NT) : 1.f, l3 = NCH > 3 ? rdl(lamc, 3 * NT) : 1.f;
      const float later = (q4 < 1 ? l1 : 1.f) * (q4 < 2 ? l2 : 1.f) * (q4 < 3 ? l3 : 1.f);
      const float lam_all = rdl(lamc, 0) * l1 * l2 * l3;
      ((float*)(hl + kHCoef))[tk] = on ? s_mine * (suf_ex * later) : 0.f;
      const float2 qv = Act::from_pair(*(const uint32_t*)(ul + kLQK + 4 * lane));
      const float2 T = make_float2(lam_all * (qv.x - ax), lam_all * (qv.y - ay));
      // T_0 = T: three 16-bit rows (f16 rows scaled by a power of two)
      float tx = T.x, ty = T.y, t0s = 1.f;
      if constexpr (!kBF16) {
        const float mx = __uint_as_float(wave_max_u32(max(__float_as_uint(fabsf(tx)), __float_as_uint(fabsf(ty)))));
        if (mx > 0.f && mx < __builtin_inff()) {
          int ex;
          (void)frexpf(mx, &ex);
          ex = uni(ex);
          tx = ldexpf(tx, -ex);
          ty = ldexpf(ty, -ex);
          t0s = ldexpf(1.f, ex);
        }
      }
      const uint32_t hw = act_bits(tx) | (act_bits(ty) << 16);
      const float2 hv2 = Act::from_pair(hw);
      const float rx = tx - hv2.x, ry = ty - hv2.y;
      const uint32_t mw = act_bits(rx) | (act_bits(ry) << 16);
      const float2 mv2 = Act::from_pair(mw);
      const uint32_t lw = act_bits(rx - mv2.x) | (act_bits(ry - mv2.y) << 16);
      *(uint32_t*)(hl + kHT0 + 4 * lane) = hw;
      *(uint32_t*)(hl + kHT0 + 256 + 4 * lane) = mw;
      *(uint32_t*)(hl + kHT0 + 512 + 4 * lane) = lw;
      if (lane == 0) {
        ((float*)(hl + kHLam))[0] = lam_all;
        ((float*)(hl + kHLam))[1] = t0s;
      }
    } else {
      // flush factors of every chunk at once (row q4 = chunk q4), each the
      // one-chunk factors within its chunk: pre_t, post_t, k_t . q, lam_c,
      // M_c and R_c = (I + M_c)^-1; the rebuild takes the chunks in turn
      const float pre = row_prefix_prod(gam);
      const float post = bet * suf_ex;
      ((float4*)(hl + kHFac))[tk] = make_float4(on ? pre : 0.f, on ? post : 0.f, on ? Dq[tk] : 0.f, 0.f);
      // the lane's Gram row within its chunk (tokens at or past the fill zero)
      const int nc = min(max(n - NT * q4, 0), NT);
      float gcol[NT];
      {
        const float4* gr = (const float4*)(Gs + q4 * 256 + l16 * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float4 v4 = gr[i];
          gcol[4 * i] = v4.x, gcol[4 * i + 1] = v4.y, gcol[4 * i + 2] = v4.z, gcol[4 * i + 3] = v4.w;
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) gcol[t] = t < nc ? gcol[t] : 0.f;
      }
      if (l16 == 0) ((float*)(hl + kHLam))[2 + q4] = lamc;
      float* Mm = (float*)(hl + kHM) + q4 * 256;
      {
        float run = 1.f;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const float gt = row_bcast_n(gam, t);
          run = t > l16 ? run * gt : run;
          Mm[t * NT + l16] = (l16 < t && t < nc) ? bet * run * gcol[t] : 0.f;
        }
      }
      float r[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        float x = (t == l16) ? 1.f : 0.f;
#pragma unroll
        for (int s4 = 0; s4 < t; s4 += 4) {
          const float4 m4 = *(const float4*)(Mm + t * NT + s4);
          x = fmaf(-m4.x, r[s4], x);
          if (s4 + 1 < t) x = fmaf(-m4.y, r[s4 + 1], x);
          if (s4 + 2 < t) x = fmaf(-m4.z, r[s4 + 2], x);
          if (s4 + 3 < t) x = fmaf(-m4.w, r[s4 + 3], x);
        }
        r[t] = x;
      }
      float* Rj = (float*)(hl + kHR) + q4 * 256;
#pragma unroll
      for (int t = 0; t < NT; ++t) Rj[t * NT + l16] = (t < nc && on) ? r[t] : 0.f;
    }
    }
    // everything is in LDS before the flag
    GDNR_WAIT_LGKM0();
    if (lane == 0)
      __hip_atomic_store((int*)(ul + kLFlag) + kFlagReady, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);

    // ---- flush helper, the rebuilds (each issues exactly 4 stores: with two
    // jobs "4 outstanding" means the job's DMA has landed, with one "none")
    if (h_g0 >= h_g1) return;
    {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
      const int g = h_g0 + jj;
      if (g < h_g1) dma_vblock(job_rows(g % rpu), VB - h_nh + g / rpu, job_buf(g / rpu, g % rpu));
    }

      uint8_t* const uv = lds + hv_unit * unit_lds(NCH, rpu, VB);
      int* const vflags = (int*)(uv + kLFlag);
      // (a wait that gives up leaves the checkpoint alone: the job's codes
      // and scale are not stored, its flags still raised)
      bool h_ok = hv_unit == u || wait_flag(vflags + kFlagReady, a.status, a.wait_polls);
      uint32_t nsc = 0;
      uint8_t* sc_addr = nullptr;
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int g = h_g0 + jj;
        if (g >= h_g1) break;
        const int kk = g / rpu, wv = g % rpu, pv = VB - h_nh + kk;
        if (h_g1 - h_g0 == 2) GDNR_WAIT_VMCNT(4);
        else GDNR_WAIT_VMCNT(0);
        h_ok = wait_flag(vflags + kFlagVStaged + wv, a.status, a.wait_polls) && h_ok;
        const uint8_t* buf = job_buf(kk, wv);
        u32x4_t c[2][2];
#pragma unroll
        for (int k = 0; k < 4; ++k) c[k >> 1][k & 1] = *(const u32x4_t*)(buf + 1024 * k + 16 * lane);
        const int hvj = hv0 + wv / NWH, partj = wv % NWH;
        uint8_t* const sc_j =
            sbase(a.scale, h_bs, a.sc_b) + (hvj * a.sc_h + (RPW * partj / kVBlock + pv) * a.sc_v);
        const float scp = f16_bits_to_f32(ld_u16_uniform(sc_j));
        const uint8_t* hbv = uv + kLHeads + (wv / NWH) * kHeadLds;
        float op[2];
        const float s32 =
            flush_vblock(uv, hbv, uv + kUnitBase + wv * row_wave_lds(NCH, VB), h_nf, c, scp, job_rows(wv), pv, h_ok, op,
                         []() {});
        *(float2*)(hbv + kHM + 512 * (partj * h_nh + kk) + 8 * lane) = make_float2(op[0], op[1]);
        GDNR_WAIT_LGKM0();
        if (lane == 0)
          __hip_atomic_fetch_add(vflags + kFlagHelped + wv, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        nsc = lane == jj ? (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)s32) : nsc;
        sc_addr = lane == jj ? sc_j : sc_addr;
      }
      if (h_ok && lane < h_g1 - h_g0) *(uint16_t*)sc_addr = (uint16_t)nsc;
      // (a job whose wait gave up stored nothing, so the count-based waits
      // above may have under-counted its DMA: drain it before the wave ends)
      if (!h_ok) GDNR_WAIT_VMCNT(0);
    }
    return;
  }

  // ================= row waves ====================================================
  const int b = opaque_s(b0);
  const int wr = (w - U) - u * rpu;
  const int j = uni(wr / NWH), part = wr - j * NWH;  // value head in the unit, row block of it
  // (barrier 1: every chain wave's requests go first)
  GDNR_COMPILER_FENCE();
  __builtin_amdgcn_s_barrier();
  GDNR_COMPILER_FENCE();
  const int hv = hv0 + j;
  const int R0 = RPW * part;
  const uint8_t* hl = ul + kLHeads + j * kHeadLds;
  // ---- checkpoint rows of the wave's tiles (preloaded arguments only):
  // vblock 0 (both branches start with it), then the sequence's metadata;
  // the other tiles only for the replay (the flush reads each vblock in turn,
  // and a wave with fewer loads in the memory pipeline gets to its first
  // vblock sooner)
  uint8_t* ck_rows = sbase(ckpt, bs, ck_b) + (hv * ck_h + R0 * ck_v);
  u32x4_t cw[TPW][2];
  // (non-temporal: the codes are read once per step and not again before the
  // next step's, which a decode batch of any size finds evicted; the hint
  // keeps them from displacing the rings and the step's other data in L2
  // and the Infinity Cache. Measured 11.44 vs 11.96 us/step at B=64, L=16.)
  auto load_tile = [&](int i) {
    const uint32_t off = (uint32_t)(32 * (i >> 1) + 2 * l16 + (i & 1)) * ck_v + 32 * q4;
    cw[i][0] = __builtin_nontemporal_load((g_u32x4*)(ck_rows + off));
    cw[i][1] = __builtin_nontemporal_load((g_u32x4*)(ck_rows + off + 16));
  };
  load_tile(0);
  load_tile(1);
  GDNR_COMPILER_FENCE();
  const StepArgs& A = opaque_args();
  int n, pos;
  bool do_flush;
  read_meta(A, n, pos, do_flush);
  // (the flush: how many of its vblocks helpers take)
  uint8_t* const vl = ul + kUnitBase + wr * row_wave_lds(NCH, VB);
  uint8_t* const pf = vl + NT * NCH * VSTRIDE;
  int nh = 0;
  if (!do_flush) {
#pragma unroll
    for (int i = 2; i < TPW; ++i) load_tile(i);
  } else {
    const int nhelp = NCH > 1 ? 0 : has_partner ? (partner_flushes(A) ? 0 : 2) : 1;
    nh = uni(helper_vblocks(VB, rpu, nhelp, NWH));
  }
  uint8_t* scale_hv = sbase(A.scale, bs, A.sc_b) + (hv * A.sc_h);
  const int vb0 = R0 / kVBlock;
  float sct[VB];  // the vblock scales
#pragma unroll
  for (int p = 0; p < VB; ++p) sct[p] = f16_bits_to_f32(ld_u16_uniform(scale_hv + (vb0 + p) * A.sc_v));
  // v rows of the filled slots in 16-byte pieces (CPT per token): load k of
  // lane l is token vtok(k) = k TPL + l / CPT, bytes [16 (l % CPT), +16) of
  // the wave's row block; the new token's from mixed_qkv; slots at or past
  // the fill re-read slot 0 (dropped when used). A ring of NCH chunks:
  // load k of chunk c is token 16 c + vtok(k).
  constexpr int CPT = RPW * ES / 16;  // pieces per token row block
  constexpr int TPL = 64 / CPT;       // tokens per load
  constexpr int NVL = NT / TPL;       // loads per lane and chunk
  const int vpiece = lane % CPT;
  auto vtok = [&](int k) { return k * TPL + lane / CPT; };
  u32x4_t vq[NCH][NVL];
  {
    const uint8_t* vbase = sbase(A.v, bs, A.v_b) + (hv * A.v_h + R0 * ES) + 16 * vpiece;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int k = 0; k < NVL; ++k) {
        const int t = NT * c + vtok(k);
        const uint8_t* src = vbase + (uint32_t)(t < n ? t : 0) * A.v_t;
        if constexpr (FUSED)
          if (t == pos) src = A.mixed + (b * A.mx_b + (2 * A.H * K + hv * A.V + R0) * ES) + 16 * vpiece;
        vq[c][k] = *(g_u32x4*)src;
      }
  }
  GDNR_COMPILER_FENCE();
  // the chain wave's LDS blocks are complete once its flag is set (a flag,
  // not a workgroup barrier: the waves of a flushing unit need not wait for
  // the other units' row waves to get their loads issued)
  // (a wait that gives up: the step's output is meaningless, and a flush
  // stores no codes or scales.) A replay of a one-chunk ring in a workgroup
  // of fewer than 4 units, or of 32- or 64-row waves, waits for it after its
  // products (which take the X rows only): there the chain's time to the
  // flag is what the step waits for. With 4 units of 128-row waves the
  // flag comes well before the codes (the stream is the step), and it is
  // taken first, as in a flush. A ring of NCH > 1 chunks, whose chain takes
  // longer, first stages its v rows (and a replay converts its codes). (The
  // waits sit in each branch, so that the flush's early request of its next
  // codes is on the flush's path only: a path joining the replay's after it
  // would make the compiler's waits for the v rows cover it.)
  const bool flag_first = !kEarly && U == 4;
  bool ready_ok = true;
  // the v rows go to LDS token-major ([16][VS] bytes; the replay once its
  // products are issued, the flush first): lane (nn, q4) then reads the two
  // rows of tiles (2p, 2p + 1) of token 4 q4 + e as one word
  auto stage_v = [&]() {
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int k = 0; k < NVL; ++k) *(u32x4_t*)(vl + (NT * c + vtok(k)) * VSTRIDE + 16 * vpiece) = vq[c][k];
  };
  // v of token 16 c + 4 q4 + e for tile i (zero at or past the fill)
  auto vval = [&](int i, int e, int c = 0) {
    const int t = NT * c + 4 * q4 + e;
    const uint32_t wv = *(const uint32_t*)(vl + t * VSTRIDE + (32 * (i >> 1) + 2 * l16) * ES);
    const float x = act_val((i & 1) ? (wv >> 16) : wv);
    return t < n ? x : 0.f;
  };
  uint8_t* out_rows = A.out + (b * A.o_b + hv * A.o_h + R0 * ES);
  // o of tiles 4 g .. 4 g + 3 from per-tile partials: lane (l16, q4) stores
  // the row of tile 4 g + q4
  auto store_out = [&](int g, float p0, float p1, float p2, float p3, bool keep = true) {
    float o = rows_reduce_scatter(p0, p1, p2, p3);
    asm volatile("" : "+v"(o));  // (no tail shared between the branches)
    if (keep) Act::st(out_rows, 64 * g + 32 * (q4 >> 1) + 2 * l16 + (q4 & 1), o * A.out_scale);
  };
  // o of every tile from its partials; a wave of 32 rows (2 tiles) stores
  // from lanes q4 < 2, whose sums take tiles 0 and 1 only (the same sums as
  // those rows get in a wider wave)
  auto store_parts = [&](const float* pp) {
    if constexpr (TPW >= 4) {
#pragma unroll
      for (int g = 0; g < TPW / 4; ++g) store_out(g, pp[4 * g], pp[4 * g + 1], pp[4 * g + 2], pp[4 * g + 3]);
    } else {
      store_out(0, pp[0], pp[1], 0.f, 0.f, q4 < 2);
    }
  };

  if (!do_flush) {
    // ---- replay: o = (scale S_0 T_0 + sum_t c_t v_t) K^-1/2 ---------------------------
    if constexpr (!kEarly)
      if (flag_first) ready_ok = wait_flag((int*)(ul + kLFlag) + kFlagReady, A.status, A.wait_polls);
    // ring append of the new token's v rows (full contract; this wave's
    // rows, which no other wave reads): the lanes that loaded token pos. (The
    // flush appends from LDS after its loop: no store is outstanding when the
    // loop starts, so its waits for each vblock's codes never cover a store.)
    if constexpr (FUSED) {
      if (pos >= 0) {
        uint8_t* vw = sbase(A.v, bs, A.v_b) + ((uint32_t)pos * A.v_t + hv * A.v_h + R0 * ES) + 16 * vpiece;
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
          for (int k = 0; k < NVL; ++k)
            if (NT * c + vtok(k) == pos) *(u32x4_t*)vw = vq[c][k];
      }
    }
    // One-chunk ring: T_0 = sum_t alpha_t X_t (+ lam q for a full ring), so
    // S_0 T_0 = sum_t alpha_t S_0 X_t: the X rows are the A operand (lane
    // (row, q4) gets S_0 X_t for t = 4 q4 + e) and each lane weights its four
    // outputs by alpha; the products need only the X rows, the weights come
    // with the chain's flag. A ring of NCH > 1 chunks (64 X rows): T_0 enters
    // as the A operand rows 0 (hi), 1 (mid) and 2 (lo), the other rows zero:
    // lanes q4 == 0 get (S_0 T_0)[row] as the sum of their first three outputs
    u32x4_t cb[kEarly ? TPW : 1][4];  // (kEarly) the codes as B operands
    constexpr int kVH = TPW >= 4 ? 2 : 1;  // (waves of 32 rows: tiles 0 and 1 only)
    uint32_t vwd[NCH][kVH][4];        // (kEarly) the v words of tiles (2 h, 2 h + 1), token 16 c + 4 q4 + e
    if constexpr (kEarly) {
      if constexpr (NCH > 1) {
      // the chain's Gram groups c >= kChainGroups, round robin over the row
      // waves (as the chain forms its own: X rows from LDS as operands);
      // first, while the codes and v rows are on their way
      int* const gflags = (int*)(ul + kLFlag);
      bool mine = false;
#pragma unroll
      for (int c = kChainGroups; c < NCH; ++c) mine = mine || ((NCH - 1 - c) % rpu == wr && NT * c < n);
      if (mine && wait_flag(gflags + kFlagXRows, A.status, A.wait_polls)) {
        float* Gf = (float*)(ul + kLKT);
        float* Dq = (float*)(ul + kLDq);
#pragma unroll
        for (int c = kChainGroups; c < NCH; ++c) {
          if ((NCH - 1 - c) % rpu != wr || NT * c >= n) continue;
          f32x4_t tacc[NCH], dacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int r = 0; r <= c; ++r) tacc[r] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            const int off = 64 * q4 + 16 * m;
            u32x4_t xo[NCH];
#pragma unroll
            for (int r = 0; r <= c; ++r) xo[r] = *(const u32x4_t*)(ul + kLX + (NT * r + l16) * kXStride + off);
            const u32x4_t qv = *(const u32x4_t*)(ul + kLQK + off);
#pragma unroll
            for (int r = 0; r <= c; ++r) tacc[r] = mfma16(xo[c], xo[r], tacc[r]);
            dacc = mfma16(xo[c], l16 == 0 ? qv : u32x4_t{0u, 0u, 0u, 0u}, dacc);
          }
#pragma unroll
          for (int r = 0; r <= c; ++r) {
            f32x4_t g = tacc[r];
            if (r == c) {
#pragma unroll
              for (int e = 0; e < 4; ++e) g[e] = 4 * q4 + e > l16 ? g[e] : 0.f;
            }
            *(float4*)(Gf + (NT * r + l16) * kGfStride + NT * c + 4 * q4) = make_float4(g[0], g[1], g[2], g[3]);
          }
          if (l16 == 0) *(float4*)(Dq + NT * c + 4 * q4) = make_float4(dacc[0], dacc[1], dacc[2], dacc[3]);
        }
      }
      GDNR_WAIT_LGKM0();
      if (lane == 0) __hip_atomic_fetch_add(gflags + kFlagGram, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
      stage_v();
#pragma unroll
      for (int i = 0; i < TPW; ++i)
#pragma unroll
        for (int m = 0; m < 4; ++m) cb[i][m] = codes8(cw[i], m);
      // (the v words the sums below take, read back now: one wait here
      // rather than one a token after the chain's flag)
#pragma unroll
      for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int h = 0; h < kVH; ++h)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            vwd[c][h][e] = NT * c < n ? *(const uint32_t*)(vl + (NT * c + 4 * q4 + e) * VSTRIDE + (32 * h + 2 * l16) * ES) : 0u;
#pragma unroll
      for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int h = 0; h < kVH; ++h)
#pragma unroll
          for (int e = 0; e < 4; ++e) asm volatile("" : "+v"(vwd[c][h][e]));
      if constexpr (NCH > 1) (void)wait_flag((int*)(ul + kLFlag) + kFlagReady, A.status, A.wait_polls);
    }
    // (the codes taken afresh: no conversion here is shared with the flush
    // branch, so none is hoisted above the branch)
#pragma unroll
    for (int i = 0; i < TPW; ++i) asm volatile("" : "+v"(cw[i][0]), "+v"(cw[i][1]));
    // the products tile by tile as the codes land, then the v terms
    float pt[TPW];
    if constexpr (NCH == 1) {
      const bool full = n >= NT;  // (the query not among the X rows)
      if (!flag_first) (void)wait_flag((int*)(ul + kLFlag) + kFlagXRows, A.status, A.wait_polls);
      u32x4_t xa[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) xa[m] = *(const u32x4_t*)(ul + kLX + l16 * kXStride + 64 * q4 + 16 * m);
      f32x4_t pc[TPW];
      float pq[TPW];  // (a full ring) S_0 q at lanes q4 == 0: every A row the query
      // (the full-ring case as a loop of its own: a branch per MFMA would keep
      // the tiles' MFMA chains from interleaving)
      auto products = [&](auto with_q) {
#pragma unroll
        for (int i = 0; i < TPW; ++i) {
          f32x4_t c = {0.f, 0.f, 0.f, 0.f}, cq = c;
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            u32x4_t bv;
            if constexpr (kEarly) bv = cb[i][m];
            else bv = codes8(cw[i], m);
            c = mfma16(xa[m], bv, c);
            if constexpr (decltype(with_q)::value) cq = mfma16(*(const u32x4_t*)(ul + kLQK + 64 * q4 + 16 * m), bv, cq);
          }
          pc[i] = c;
          pq[i] = cq[0];
        }
      };
      if (full) products(std::true_type{});
      else products(std::false_type{});
      if (!flag_first) (void)wait_flag((int*)(ul + kLFlag) + kFlagReady, A.status, A.wait_polls);
      const float4 al = *(const float4*)(hl + kHT0 + 16 * q4);
      const float lq = (full && q4 == 0) ? ((const float*)(hl + kHLam))[0] : 0.f;
#pragma unroll
      for (int i = 0; i < TPW; ++i) {
        float x = al.x * pc[i][0];
        x = fmaf(al.y, pc[i][1], x);
        x = fmaf(al.z, pc[i][2], x);
        x = fmaf(al.w, pc[i][3], x);
        x = fmaf(lq, pq[i], x);
        pt[i] = x * sct[i >> 1];
      }
    } else {
      const uint8_t* arow = hl + kHT0 + 256 * (l16 < 3 ? l16 : 0) + 64 * q4;
      const float t0s = ((const float*)(hl + kHLam))[1];
#pragma unroll
      for (int i = 0; i < TPW; ++i) {
        f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const u32x4_t x = *(const u32x4_t*)(arow + 16 * m);
          c = mfma16(l16 < 3 ? x : u32x4_t{0u, 0u, 0u, 0u}, cb[i][m], c);
        }
        pt[i] = (c[0] + (c[1] + c[2])) * (sct[i >> 1] * t0s);
      }
    }
    const float4 cc = *(const float4*)(hl + kHCoef + 16 * q4);
    float part_[TPW];
    if constexpr (!kEarly) {
      stage_v();
#pragma unroll
      for (int i = 0; i < TPW; ++i) {
        float wsum = cc.x * vval(i, 0);
        wsum = fmaf(cc.y, vval(i, 1), wsum);
        wsum = fmaf(cc.z, vval(i, 2), wsum);
        wsum = fmaf(cc.w, vval(i, 3), wsum);
        part_[i] = pt[i] + wsum;
      }
    } else {
      // every chunk's tokens: coefficients c_t of token 16 c + 4 q4 + e
      // (zero at or past the fill), v from the words read before the flag;
      // summed as the branch above sums them (chunk 0 always, pt + its sum
      // the only use of pt, so that the compiler contracts it the same way):
      // either kind of launch gives the same bits
      auto vw_val = [&](int c, int i, int e) {
        const uint32_t w = vwd[c][i >> 1][e];
        const float x = act_val((i & 1) ? (w >> 16) : w);
        return NT * c + 4 * q4 + e < n ? x : 0.f;
      };
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        if (c > 0 && NT * c >= n) break;
        const float4 cq = *(const float4*)(hl + kHCoef + 4 * (NT * c + 4 * q4));
#pragma unroll
        for (int i = 0; i < TPW; ++i) {
          float wsum = cq.x * vw_val(c, i, 0);
          wsum = fmaf(cq.y, vw_val(c, i, 1), wsum);
          wsum = fmaf(cq.z, vw_val(c, i, 2), wsum);
          wsum = fmaf(cq.w, vw_val(c, i, 3), wsum);
          part_[i] = c == 0 ? pt[i] + wsum : part_[i] + wsum;
        }
      }
    }
    store_parts(part_);
    return;
  }

  // ---- flush: the wave's vblocks in turn (flush_vblock); the last nh of
  // them rebuilt by helper waves, whose o shares come back through LDS.
  // The v rows go to LDS first; then vblock 1's codes go to the prefetch
  // buffer, long before vblock 0 is rebuilt, and only then does the wave
  // wait for the chain's flag. (Staged after that request, the v rows would
  // wait for it: the compiler's waits before the LDS writes cover the DMA.)
  stage_v();
  int* const flags = (int*)(ul + kLFlag);
  if (lane == 0) __hip_atomic_store(flags + kFlagVStaged + wr, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  const int own = VB - nh;
  if (own > 1) dma_vblock(ck_rows, 1, pf);
  ready_ok = wait_flag((int*)(ul + kLFlag) + kFlagReady, A.status, A.wait_polls);
  u32x4_t cur[2][2] = {{cw[0][0], cw[0][1]}, {cw[1][0], cw[1][1]}};
  // The codes of vblock p + 1 come from the wave's prefetch buffer, which
  // direct DMA fills while vblock p - 1 is finished and p is rebuilt. Each
  // iteration issues its DMA and then exactly 4 stores, so "4 outstanding"
  // means the DMA of the iteration before has landed (the first iteration's
  // wait takes everything: vblock 1's DMA, issued after the v rows, is then
  // the only request outstanding). (Not with vblock 0's rows: ahead of the v
  // rows it would delay the first vblock.)
  // (a loop, not unrolled: one vblock's registers at a time; the indices
  // that depend on p are formed by selects, not by indexing registers)
  float opart_all[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i) opart_all[i] = 0.f;
  // the new vblock scales, lane p holding vblock p's: stored after the loop,
  // so that the loop's only memory requests are the codes it reads and
  // writes (its waits for the next vblock's codes then never cover a store)
  uint32_t new_scale = 0;
#pragma unroll 1
  for (int p = 0; p < own; ++p) {
    float scp = sct[0];
#pragma unroll
    for (int q = 1; q < VB; ++q) scp = p == q ? sct[q] : scp;
    float op[2];
    const float s32 = flush_vblock(ul, hl, vl, n, cur, scp, ck_rows, p, ready_ok, op, [&]() {
      // the next vblock's codes from the prefetch buffer (into the same
      // registers), then the buffer refilled with the one after
      if (p + 1 < own) {
        if (p == 0) GDNR_WAIT_VMCNT(0);
        else GDNR_WAIT_VMCNT(4);
#pragma unroll
        for (int k = 0; k < 4; ++k) cur[k >> 1][k & 1] = *(const u32x4_t*)(pf + 1024 * k + 16 * lane);
        GDNR_WAIT_LGKM0();
        if (p + 2 < own) dma_vblock(ck_rows, p + 2, pf);
      }
    });
#pragma unroll
    for (int k = 0; k < TPW; ++k) opart_all[k] = k == 2 * p ? op[0] : (k == 2 * p + 1 ? op[1] : opart_all[k]);
    new_scale = lane == p ? (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)s32) : new_scale;
  }
  if (nh > 0) {
    (void)wait_count(flags + kFlagHelped + wr, nh, A.status, A.wait_polls);  // (the helpers gate their own stores)
    for (int kk = 0; kk < nh; ++kk) {
      const int p = own + kk;
      const float2 o2 = *(const float2*)(hl + kHM + 512 * (part * nh + kk) + 8 * lane);
#pragma unroll
      for (int k = 0; k < TPW; ++k) opart_all[k] = k == 2 * p ? o2.x : (k == 2 * p + 1 ? o2.y : opart_all[k]);
    }
  }
  store_parts(opart_all);
  if (ready_ok && lane < own) *(uint16_t*)(scale_hv + (vb0 + lane) * A.sc_v) = (uint16_t)new_scale;
  // (with no code stores the loop's count-based DMA waits may have
  // under-counted: drain the last prefetch before the wave ends)
  if (!ready_ok) GDNR_WAIT_VMCNT(0);
  if constexpr (FUSED) {
    if (pos >= 0 && lane < CPT) {
      uint8_t* vw = sbase(A.v, bs, A.v_b) + ((uint32_t)pos * A.v_t + hv * A.v_h + R0 * ES) + 16 * lane;
      *(u32x4_t*)vw = *(const u32x4_t*)(vl + pos * VSTRIDE + 16 * lane);
    }
  }
}

template <int TPW, int NWH, int NCH, bool FUSED, bool GATE_F32, bool SLOTS>
int launch_variant(const StepArgs& a, hipStream_t s) {
  const int hp = a.units == 4 ? 2 : 1, sp = a.units / hp;  // as in the kernel
  const unsigned gh = (unsigned)(a.H * (a.G / a.gw) / hp), gs = (unsigned)(a.B / sp);
  const dim3 grid(a.seq_major ? gs : gh, a.seq_major ? gh : gs),
      block((unsigned)(64 * a.units * (1 + a.gw * NWH)));
  auto kernel = decode_kernel<TPW, NWH, NCH, FUSED, GATE_F32, SLOTS>;
  if (a.lds_bytes > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, a.lds_bytes);
    if (e != hipSuccess) return (int)e;
  }
  hipLaunchKernelGGL(kernel, grid, block, a.lds_bytes, s, a.ckpt, a.k, a.ck_b, a.ck_h, a.ck_v, a.k_b, a.k_t, a.k_h,
                     a.L, a.G, a.gw | (a.units << 8) | (a.seq_major << 16), a);
  return 0;
}

template <int TPW, int NWH, int NCH = 1>
int launch_shape(const StepArgs& a, bool fused, bool gate_f32, hipStream_t s) {
  if (!fused) return launch_variant<TPW, NWH, NCH, false, false, false>(a, s);
  if (a.slot && gate_f32) return launch_variant<TPW, NWH, NCH, true, true, true>(a, s);
  if (a.slot) return launch_variant<TPW, NWH, NCH, true, false, true>(a, s);
  if (gate_f32) return launch_variant<TPW, NWH, NCH, true, true, false>(a, s);
  return launch_variant<TPW, NWH, NCH, true, false, false>(a, s);
}

}  // namespace

#if GDNR_ACT == 0
// LDS bytes of the decode kernel for gw value heads (of nwh row waves each;
// the layout is the same for both activation dtypes)
int32_t decode_lds_bytes(int32_t units, int32_t row_waves, int32_t vblocks, int32_t chunks) {
  return units * unit_lds(chunks, row_waves, vblocks);
}
#endif

int GDNR_SUFFIX(launch_decode)(const StepArgs& a, bool fused, bool gate_f32, void* stream) {
  hipStream_t s = (hipStream_t)stream;
  int rc;
  // V = 64 a.sw: one wave of 64 rows per value head; 128: one of 128 rows,
  // or four of 32 (small batches); 256: two of 128
  // (a ring longer than one chunk: waves of 32 rows, one per 32 of V, while
  // a workgroup has a compute unit to itself; else of 64 rows)
  if (a.L > kStepRing && a.V / a.nwh == 32)
    rc = a.sw == 1 ? launch_shape<2, 2, kDecodeChunks>(a, fused, gate_f32, s)
                   : launch_shape<2, 4, kDecodeChunks>(a, fused, gate_f32, s);
  else if (a.L > kStepRing)
    rc = a.sw == 1 ? launch_shape<4, 1, kDecodeChunks>(a, fused, gate_f32, s)
                   : launch_shape<4, 2, kDecodeChunks>(a, fused, gate_f32, s);
  else if (a.sw == 1) rc = launch_shape<4, 1>(a, fused, gate_f32, s);
  else if (a.sw == 2 && a.nwh == 4) rc = launch_shape<2, 4>(a, fused, gate_f32, s);
  else if (a.sw == 2) rc = launch_shape<8, 1>(a, fused, gate_f32, s);
  else rc = launch_shape<8, 2>(a, fused, gate_f32, s);
  if (rc) return rc;
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : (int)e;
}

}  // namespace gdnr

#endif  // GDNR_ACT != 2
