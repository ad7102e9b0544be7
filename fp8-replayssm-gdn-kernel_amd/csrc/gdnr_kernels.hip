// gdnr_kernels.hip -- gfx950 (MI355X) kernels of the ReplaySSM GDN decode path.
//
// Workgroup = (sequence b, gw value heads that share one key head, V-tile).
// One wave64 per value head. Per workgroup:
//   1. the ring (q, k, v) staged into LDS by direct-to-LDS DMA
//      (global_load_lds_dwordx4): no VGPR round trip, runtime ring length;
//   2. per-lane loads of small operands (gating scalars, fused-prep inputs);
//   3. the fp8 checkpoint tile streamed into VGPRs with coalesced 128-bit
//      loads (each load instruction of a wave reads 8 contiguous 128-byte rows);
//   4. s_waitcnt vmcnt(NCH): everything except the checkpoint tile has landed
//      (vector-memory loads retire in issue order), so the latency-bound
//      adjoint chain runs while the checkpoint is still in flight;
//   5. the checkpoint matvec o = (codes . T) * scale on the VALU (no MFMA:
//      one FMA per byte), rows reduced across 8 lanes with DPP.
// The order of steps 2-3 is pinned with compiler fences.
// These kernels serve rings longer than 16 tokens, the split path, the
// standalone prep and the quantiser; rings of up to 16 tokens go through the
// decode kernel (gdnr_decode.hip, 16-bit activations) or the step kernel
// (gdnr_step.hip, f32 activations).
//
// This file is compiled once per activation dtype: GDNR_ACT=0 (bf16, also
// holds the dtype-free quantiser kernels), 1 (f16), 2 (f32).
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

// Reduce NCH per-lane partial row sums across the 8 lanes of a row group
// (lanes 8m..8m+7 hold the 8 K-chunks of the same rows). Transposing
// butterfly: each step halves the live partials. Afterwards lane i of the
// group holds, in P[0 .. NCH/8), the totals of rows j = (NCH/8)*i + r; for
// NCH == 4, P[0] holds the total of row j = i >> 1 (pairs of lanes agree).
template <int NCH>
__device__ __forceinline__ void butterfly8(float* P, int gi) {
  {
    const bool hi = (gi & 4) != 0;
#pragma unroll
    for (int a = 0; a < NCH / 2; ++a) {
      float send = hi ? P[a] : P[a + NCH / 2];
      float keep = hi ? P[a + NCH / 2] : P[a];
      P[a] = keep + dpp_f<kDppHalfMirror>(send);
    }
  }
  {
    const bool hi = (gi & 2) != 0;
#pragma unroll
    for (int a = 0; a < NCH / 4; ++a) {
      float send = hi ? P[a] : P[a + NCH / 4];
      float keep = hi ? P[a + NCH / 4] : P[a];
      P[a] = keep + dpp_f<kDppXor2>(send);
    }
  }
  if constexpr (NCH >= 8) {
    const bool hi = (gi & 1) != 0;
#pragma unroll
    for (int a = 0; a < NCH / 8; ++a) {
      float send = hi ? P[a] : P[a + NCH / 8];
      float keep = hi ? P[a + NCH / 8] : P[a];
      P[a] = keep + dpp_f<kDppXor1>(send);
    }
  } else {
    P[0] += dpp_f<kDppXor1>(P[0]);
  }
}

// rows (within the V-tile) whose totals lane group-index gi holds after butterfly8
template <int NCH>
__device__ __forceinline__ int out_row(int gi, int gm, int r) {
  if constexpr (NCH >= 8) return 8 * ((NCH / 8) * gi + r) + gm;
  else return 8 * (gi >> 1) + gm;
}
// Stage n_chunks 16-byte chunks into LDS at `lds_off` + 16*c with direct
// DMA issued by ONE wave; src(c) returns the global address of chunk c or
// nullptr to skip it. The LDS destination of a DMA instruction is
// wave-uniform (M0): lane l writes 16 bytes at dst + 16*l. The sequence is
// fully unrolled to a compile-time bound with wave-uniform skips, so the
// number of vector-memory instructions on every path is static (the
// compiler's wait counting stays exact across it).
template <int MAX_INSTR, class SrcFn>
__device__ __forceinline__ void dma_stage(uint8_t* lds, int lds_off, int n_chunks, int lane, SrcFn src) {
#pragma unroll
  for (int it = 0; it < MAX_INSTR; ++it) {
    const int base = it * 64;
    if (base < n_chunks) {
      const int c = base + lane;
      const void* p = (c < n_chunks) ? src(c) : nullptr;
      if (p) __builtin_amdgcn_global_load_lds(p, (lds_void_t*)(lds + lds_off + base * 16), 16, 0, 0);
    }
  }
}

// wave-uniform loads of per-sequence metadata (scalar memory path)
__device__ __forceinline__ int32_t uniform_i32(const int32_t* p) { return __builtin_amdgcn_readfirstlane(*p); }
__device__ __forceinline__ uint32_t uniform_u8(const uint8_t* p) {
  const uintptr_t addr = (uintptr_t)p;
  const uint32_t w = *(const uint32_t*)(addr & ~(uintptr_t)3);  // aligned word holding the byte
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)((w >> (8 * (addr & 3))) & 0xFFu));
}
template <bool GATE_F32, class Act>
__device__ __forceinline__ float ld_gate(const void* p, int64_t i) {
  if constexpr (GATE_F32) return ((const float*)p)[i];
  else return Act::ld(p, i);
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f32_to_f16_bits(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }

template <class Act, int NCH, int MODE, bool GATE_F32>
__global__ __launch_bounds__(256) void replay_kernel(const ReplayArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr bool APPLY = MODE == kModeApply;
  constexpr bool FUSED = MODE == kModeFused;
  constexpr int ES = Act::kBytes;
  constexpr int BV = NCH * 8;            // V rows of the tile
  constexpr int CPT_K = K * ES / 16;     // 16-byte chunks per key row
  constexpr int CPT_V = BV * ES / 16;    // 16-byte chunks per value-row slice
  constexpr int NR = NCH >= 8 ? NCH / 8 : 1;
  constexpr int NVB = NCH / 4;           // vblocks in the tile

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gw = a.gw;
  int wg = blockIdx.x;
  const int vt = wg % a.n_vt;
  wg /= a.n_vt;
  const int groups = a.HV / gw;
  const int hv0 = (wg % groups) * gw;
  const int b = wg / groups;
  // the sequence's state (checkpoint, scales, rings) sits in slot slot[b] of
  // a slot-indexed cache when a.slot is set (fused step only; clamped to
  // [0, n_slots), slot 0 being the null slot), otherwise in row b; the
  // metadata, the step inputs, q_out and out stay per batch entry b
  int bs = b;
  if constexpr (FUSED) {
    if (a.slot) {
      const int sl = uniform_i32(a.slot + (int64_t)b * a.sl_s);
      bs = (sl >= 0 && sl < a.n_slots) ? sl : 0;
    }
  }
  const int h = hv0 / a.G;
  const int hv = hv0 + wave;
  const int v0 = vt * BV;
  const int gi = lane & 7;   // K-chunk (16 columns) of this lane in the tile layout
  const int gm = lane >> 3;  // row within an 8-row group

  // ---- 0. per-sequence metadata (one scalar-memory round trip) ----------
  int n = uniform_i32(a.valid_len + (int64_t)b * a.vl_s);
  n = n < 0 ? 0 : (n > a.L ? a.L : n);
  bool do_flush = false;
  if constexpr (!APPLY) {
    if (a.flush) do_flush = uniform_u8(a.flush + (int64_t)b * a.fl_s) != 0;
  }
  int pos = -1;
  if constexpr (FUSED) {
    const int p = uniform_i32(a.pos + (int64_t)b * a.pos_s);
    pos = (p >= 0 && p < a.L) ? p : -1;
  }

  // ---- 1. ring -> LDS (direct DMA) --------------------------------------
  // wave 0 stages q and the key ring; every wave stages its own value head's
  // rows of the tile. LDS: k [t][K], v [j][t][BV] (j = value head in the WG).
  constexpr int MAXI_K = (kMaxRing * CPT_K + 63) / 64;
  constexpr int MAXI_V = (kMaxRing * CPT_V + 63) / 64;
  if constexpr (!APPLY) {
    if (wave == 0) {
      if constexpr (!FUSED) {
        const uint8_t* qrow = (const uint8_t*)a.q + ((int64_t)b * a.q_b + (int64_t)h * a.q_h) * ES;
        dma_stage<(CPT_K + 63) / 64>(lds, a.lds_q, CPT_K, lane, [&](int c) -> const void* { return qrow + 16 * c; });
      }
      const uint8_t* kbase = (const uint8_t*)a.k + ((int64_t)bs * a.k_b + (int64_t)h * a.k_h) * ES;
      dma_stage<MAXI_K>(lds, a.lds_k, n * CPT_K, lane, [&](int c) -> const void* {
        const int t = c / CPT_K;
        if (t == pos) return nullptr;
        return kbase + (int64_t)t * a.k_t * ES + 16 * (c % CPT_K);
      });
    }
  } else {
    // transformed query T_0 of this wave's value head (f32, 32 chunks)
    const uint8_t* tqrow = (const uint8_t*)(a.tq + (int64_t)b * a.tq_b + (int64_t)hv * a.tq_h);
    dma_stage<1>(lds, a.lds_t + wave * K * 4, K * 4 / 16, lane, [&](int c) -> const void* { return tqrow + 16 * c; });
  }
  {
    const uint8_t* vbase = (const uint8_t*)a.v + ((int64_t)bs * a.v_b + (int64_t)hv * a.v_h + v0) * ES;
    dma_stage<MAXI_V>(lds, a.lds_v + wave * a.L * BV * ES, n * CPT_V, lane, [&](int c) -> const void* {
      const int t = c / CPT_V;
      if (t == pos) return nullptr;
      return vbase + (int64_t)t * a.v_t * ES + 16 * (c % CPT_V);
    });
  }

  // ---- 2. small per-lane operands (raw bits; converted after step 4) ----
  // Issued after the DMA and right before the checkpoint tile: only the NCH
  // straight-line tile loads separate them from their first use, so the
  // compiler's own wait there is vmcnt(NCH) as well.
  // gating of token t for value head j of the workgroup: thread -> (t, j)
  const int gb_t = (int)threadIdx.x / gw;
  const int gb_j = (int)threadIdx.x % gw;
  const bool gb_live = !APPLY && gb_t < n && gb_t != pos;
  // Unconditional loads from always-valid slots: a guarded load would join a
  // phi whose extension the compiler schedules (and waits for) right away.
  const int gb_slot = gb_t < a.L ? gb_t : a.L - 1;
  typename Act::Bits g_bits = 0, beta_bits = 0;
  if constexpr (!APPLY) {
    g_bits = Act::ld_bits(a.g, (int64_t)bs * a.g_b + (int64_t)gb_slot * a.g_t + (int64_t)(hv0 + gb_j) * a.g_h);
    beta_bits = Act::ld_bits(a.beta, (int64_t)bs * a.be_b + (int64_t)gb_slot * a.be_t + (int64_t)(hv0 + gb_j) * a.be_h);
  }
  float cval = 0.f;  // APPLY: lane t holds c_t (lanes >= n are ignored)
  if constexpr (APPLY) {
    const int slot = lane < a.L ? lane : a.L - 1;
    cval = a.coef[(int64_t)b * a.co_b + (int64_t)hv * a.co_h + (int64_t)slot * a.co_t];
  }
  typename Act::Pair q_bits{}, k_bits{};
  constexpr int NVR = (BV + 63) / 64;
  typename Act::Bits v_bits[NVR];
  using GateBits = typename std::conditional<GATE_F32, uint32_t, typename Act::Bits>::type;
  GateBits a_bits = 0, b_bits = 0;
  uint32_t alog_bits = 0, dtb_bits = 0;
  if constexpr (FUSED) {
    const uint8_t* row = (const uint8_t*)a.mixed + (int64_t)b * a.mx_b * ES;
    q_bits = Act::ld_pair_bits(row + (int64_t)(h * K + 2 * lane) * ES);
    k_bits = Act::ld_pair_bits(row + (int64_t)(a.H * K + h * K + 2 * lane) * ES);
#pragma unroll
    for (int r = 0; r < NVR; ++r) {
      const int e = lane + 64 * r < BV ? lane + 64 * r : BV - 1;
      v_bits[r] = Act::ld_bits(row, (int64_t)2 * a.H * K + (int64_t)hv * a.V + v0 + e);
    }
    if constexpr (GATE_F32) {
      a_bits = ((const uint32_t*)a.a)[(int64_t)b * a.a_b + (int64_t)hv * a.a_h];
      b_bits = ((const uint32_t*)a.bgate)[(int64_t)b * a.bg_b + (int64_t)hv * a.bg_h];
    } else {
      a_bits = Act::ld_bits(a.a, (int64_t)b * a.a_b + (int64_t)hv * a.a_h);
      b_bits = Act::ld_bits(a.bgate, (int64_t)b * a.bg_b + (int64_t)hv * a.bg_h);
    }
    alog_bits = ((const uint32_t*)a.a_log)[(int64_t)hv * a.al_s];
    dtb_bits = ((const uint32_t*)a.dt_bias)[(int64_t)hv * a.db_s];
  }

  // ---- 3. checkpoint tile -> VGPRs (non-temporal: read once per step) ------
  GDNR_COMPILER_FENCE();
  uint4 ck[NCH];
  uint8_t* ckp = a.ckpt + (int64_t)bs * a.ck_b + (int64_t)hv * a.ck_h + (int64_t)(v0 + gm) * a.ck_v + 16 * gi;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    typedef uint32_t u32x4_nt __attribute__((ext_vector_type(4)));
    const u32x4_nt v = __builtin_nontemporal_load((const u32x4_nt*)(ckp + (int64_t)(8 * j) * a.ck_v));
    ck[j] = make_uint4(v[0], v[1], v[2], v[3]);
  }
  GDNR_COMPILER_FENCE();
  // ---- 4. all but the checkpoint tile has landed --------------------------
  GDNR_WAIT_VMCNT(NCH);
  // (no register barriers on the small operands: an inline-asm use of a
  // pending load makes the compiler fall back to vmcnt(0); their loads sit
  // in the same block as the tile loads, so its own wait is vmcnt(NCH).)
  if (gb_live) {
    *(float2*)(lds + a.lds_gb + (gb_t * gw + gb_j) * 8) = make_float2(expf(Act::from_bits(g_bits)), Act::from_bits(beta_bits));
  }
  if constexpr (FUSED) {
    // full-contract preparation of the new token (reference kernel:504-576)
    const float2 q_raw = Act::from_pair(q_bits), k_raw = Act::from_pair(k_bits);
    float v_raw[NVR];
#pragma unroll
    for (int r = 0; r < NVR; ++r) v_raw[r] = Act::from_bits(v_bits[r]);
    const float a_raw = GATE_F32 ? __uint_as_float(a_bits) : Act::from_bits(a_bits);
    const float b_raw = GATE_F32 ? __uint_as_float(b_bits) : Act::from_bits(b_bits);
    const float alog_raw = __uint_as_float(alog_bits), dtb_raw = __uint_as_float(dtb_bits);
    const float sq = wave_sum(fmaf(q_raw.y, q_raw.y, q_raw.x * q_raw.x));
    const float sk = wave_sum(fmaf(k_raw.y, k_raw.y, k_raw.x * k_raw.x));
    const float qd = sqrtf(sq + 1e-6f), kd = sqrtf(sk + 1e-6f);
    const float q0 = Act::round(q_raw.x / qd), q1 = Act::round(q_raw.y / qd);
    const float k0 = Act::round(k_raw.x / kd), k1 = Act::round(k_raw.y / kd);
    const float xg = a_raw + dtb_raw;
    const float sp = xg <= 20.0f ? logf(1.0f + expf(xg)) : xg;  // kernel:560, as written there
    const float gate = Act::round(-expf(alog_raw) * sp);
    const float bet = Act::round(1.0f / (1.0f + expf(-b_raw)));
    if (wave == 0) Act::st2(lds + a.lds_q + 2 * lane * ES, q0, q1);
    if (pos >= 0) {
      if (wave == 0) Act::st2(lds + a.lds_k + (pos * K + 2 * lane) * ES, k0, k1);
      if (lane == 0) *(float2*)(lds + a.lds_gb + (pos * gw + wave) * 8) = make_float2(expf(gate), bet);
#pragma unroll
      for (int r = 0; r < NVR; ++r) {
        const int e = lane + 64 * r;
        if (e < BV) Act::st(lds + a.lds_v, (int64_t)(wave * a.L + pos) * BV + e, v_raw[r]);
      }
      // append to the global ring (each V-tile writes its own v rows)
      if (vt == 0) {
        if (wave == 0) {
          uint8_t* kr = (uint8_t*)a.k + ((int64_t)bs * a.k_b + (int64_t)pos * a.k_t + (int64_t)h * a.k_h) * ES;
          Act::st2(kr + 2 * lane * ES, k0, k1);
        }
        if (lane == 0) {
          Act::st(a.g, (int64_t)bs * a.g_b + (int64_t)pos * a.g_t + (int64_t)hv * a.g_h, gate);
          Act::st(a.beta, (int64_t)bs * a.be_b + (int64_t)pos * a.be_t + (int64_t)hv * a.be_h, bet);
        }
      }
#pragma unroll
      for (int r = 0; r < NVR; ++r) {
        const int e = lane + 64 * r;
        if (e < BV)
          Act::st(a.v, (int64_t)bs * a.v_b + (int64_t)pos * a.v_t + (int64_t)hv * a.v_h + v0 + e, v_raw[r]);
      }
    }
    if (vt == 0 && wave == 0) {
      uint8_t* qo = (uint8_t*)a.q_out + ((int64_t)b * a.qo_b + (int64_t)h * a.qo_h) * ES;
      Act::st2(qo + 2 * lane * ES, q0, q1);
    }
  }
  GDNR_WAIT_LGKM0();
  __builtin_amdgcn_s_barrier();

  float* out_tq = (float*)(lds + a.lds_t) + wave * K;
  const uint16_t* scale_hv = a.scale + (int64_t)bs * a.sc_b + (int64_t)hv * a.sc_h;
  if (!do_flush) {
    // scale of this lane's output rows: loaded now, converted after the matvec
    uint32_t sc_bits = scale_hv[(int64_t)((v0 + out_row<NCH>(gi, gm, 0)) / kVBlock) * a.sc_v];
    // ---- 5. adjoint chain: T <- exp(g)(T - c k), c = beta (k . T), o += c v
    float acc[NR];
    int rows[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      acc[r] = 0.f;
      rows[r] = out_row<NCH>(gi, gm, r);
    }
    const uint8_t* vl = lds + a.lds_v + (int64_t)wave * a.L * BV * ES;
    if constexpr (!APPLY) {
      // T = lam * U: U carries the undecayed query, lam the decay product
      float2 U = Act::ld2(lds + a.lds_q + 2 * lane * ES);
      float lam = 1.0f;
      for (int t = n - 1; t >= 0; --t) {
        const float2 kk = Act::ld2(lds + a.lds_k + (t * K + 2 * lane) * ES);
        const float2 gbv = *(const float2*)(lds + a.lds_gb + (t * gw + wave) * 8);
        const float d = wave_sum(fmaf(kk.y, U.y, kk.x * U.x));
        const float s = gbv.y * d;
        const float c = s * lam;
        U.x = fmaf(-s, kk.x, U.x);
        U.y = fmaf(-s, kk.y, U.y);
        lam *= gbv.x;
        const uint8_t* vt_row = vl + (int64_t)t * BV * ES;
#pragma unroll
        for (int r = 0; r < NR; ++r) acc[r] = fmaf(c, Act::ld(vt_row, rows[r]), acc[r]);
      }
      *(float2*)(out_tq + 2 * lane) = make_float2(lam * U.x, lam * U.y);
    } else {
      for (int t = 0; t < n; ++t) {
        const float c = readlane_f(cval, t);
        const uint8_t* vt_row = vl + (int64_t)t * BV * ES;
#pragma unroll
        for (int r = 0; r < NR; ++r) acc[r] = fmaf(c, Act::ld(vt_row, rows[r]), acc[r]);
      }
    }
    // ---- 6. checkpoint matvec ---------------------------------------------
    float T16[16];
    {
      const float4* tp = (const float4*)(out_tq + 16 * gi);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 w = tp[i];
        T16[4 * i] = w.x;
        T16[4 * i + 1] = w.y;
        T16[4 * i + 2] = w.z;
        T16[4 * i + 3] = w.w;
      }
    }
    float P[NCH];
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const uint32_t w[4] = {ck[j].x, ck[j].y, ck[j].z, ck[j].w};
      float p = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float f[4];
        fp8x4_to_f32(w[i], f);
        p = fmaf(f[0], T16[4 * i], p);
        p = fmaf(f[1], T16[4 * i + 1], p);
        p = fmaf(f[2], T16[4 * i + 2], p);
        p = fmaf(f[3], T16[4 * i + 3], p);
      }
      P[j] = p;
    }
    butterfly8<NCH>(P, gi);
    const float sc = f16_bits_to_f32((uint16_t)sc_bits);
    if (NCH >= 8 || (gi & 1) == 0) {
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const float o = fmaf(P[r], sc, acc[r]) * a.out_scale;
        Act::st(a.out, (int64_t)b * a.o_b + (int64_t)hv * a.o_h + v0 + rows[r], o);
      }
    }
  } else {
    // ---- flush: forward rebuild, emit, requantise in place (32 rows a pass)
    uint32_t sc_bits[NVB];
#pragma unroll
    for (int p = 0; p < NVB; ++p) sc_bits[p] = scale_hv[(int64_t)(v0 / kVBlock + p) * a.sc_v];
    float q16[16];
    Act::ld16(lds + a.lds_q + 16 * gi * ES, q16);
    const uint8_t* vl = lds + a.lds_v + (int64_t)wave * a.L * BV * ES;
#pragma unroll
    for (int p = 0; p < NVB; ++p) {
      float s[4][16];
      const float sc = f16_bits_to_f32((uint16_t)sc_bits[p]);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const uint32_t w[4] = {ck[4 * p + jj].x, ck[4 * p + jj].y, ck[4 * p + jj].z, ck[4 * p + jj].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          fp8x4_to_f32(w[i], &s[jj][4 * i]);
#pragma unroll
          for (int e = 0; e < 4; ++e) s[jj][4 * i + e] *= sc;
        }
      }
      for (int t = 0; t < n; ++t) {
        float kk[16];
        Act::ld16(lds + a.lds_k + (t * K + 16 * gi) * ES, kk);
        const float2 gbv = *(const float2*)(lds + a.lds_gb + (t * gw + wave) * 8);
        const uint8_t* vt_row = vl + (int64_t)t * BV * ES;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          float r = 0.f;
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            s[jj][e] *= gbv.x;
            r = fmaf(s[jj][e], kk[e], r);
          }
          r = sum8(r);
          const float u = (Act::ld(vt_row, 32 * p + 8 * jj + gm) - r) * gbv.y;
#pragma unroll
          for (int e = 0; e < 16; ++e) s[jj][e] = fmaf(u, kk[e], s[jj][e]);
        }
      }
      // o = (S q) K^-1/2 from the rebuilt fp32 rows
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        float o = 0.f;
#pragma unroll
        for (int e = 0; e < 16; ++e) o = fmaf(s[jj][e], q16[e], o);
        o = sum8(o);
        if (gi == 0) Act::st(a.out, (int64_t)b * a.o_b + (int64_t)hv * a.o_h + v0 + 32 * p + 8 * jj + gm, o * a.out_scale);
      }
      // requantise this vblock (reference quantiser, ref:36-37,83-99)
      uint32_t am = 0;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int e = 0; e < 16; ++e) am = max(am, __float_as_uint(s[jj][e]) & 0x7FFFFFFFu);
      am = wave_max_u32(am);
      const float amax = __uint_as_float(am);
      const float s32 = (amax > 0.0f) ? amax / 448.0f : 1.0f;
      const _Float16 s16 = (_Float16)s32;
      const bool fast = quotient_fast(am, s32);
      const float r = 1.0f / s32;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        uint32_t wq[4];
        if (fast) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            wq[i] = f32x4_to_fp8(quotient_rn(s[jj][4 * i], s32, r), quotient_rn(s[jj][4 * i + 1], s32, r),
                                 quotient_rn(s[jj][4 * i + 2], s32, r), quotient_rn(s[jj][4 * i + 3], s32, r));
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            wq[i] = f32x4_to_fp8_ref(s[jj][4 * i] / s32, s[jj][4 * i + 1] / s32, s[jj][4 * i + 2] / s32,
                                     s[jj][4 * i + 3] / s32);
        }
        *(uint4*)(ckp + (int64_t)(8 * (4 * p + jj)) * a.ck_v) = make_uint4(wq[0], wq[1], wq[2], wq[3]);
      }
      if (lane == 0)
        a.scale[(int64_t)bs * a.sc_b + (int64_t)hv * a.sc_h + (int64_t)(v0 / kVBlock + p) * a.sc_v] =
            __builtin_bit_cast(uint16_t, s16);
    }
  }
}

// Split precompute (reference kernel:798-896 / :1021-1126): the adjoint chain
// only, writing T_0 and c_t. One wave per value head, gw heads per workgroup
// sharing the staged key ring.
template <class Act>
__global__ __launch_bounds__(256) void precompute_kernel(const ReplayArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int ES = Act::kBytes;
  constexpr int CPT_K = K * ES / 16;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gw = a.gw;
  const int groups = a.HV / gw;
  const int hv0 = (blockIdx.x % groups) * gw;
  const int b = blockIdx.x / groups;
  const int h = hv0 / a.G;
  const int hv = hv0 + wave;
  int n = uniform_i32(a.valid_len + (int64_t)b * a.vl_s);
  n = n < 0 ? 0 : (n > a.L ? a.L : n);

  const int gb_t = (int)threadIdx.x / gw;
  const int gb_j = (int)threadIdx.x % gw;
  const bool gb_live = gb_t < n;
  float g_raw = 0.f, beta_raw = 0.f;
  if (gb_live) {
    g_raw = Act::ld(a.g, (int64_t)b * a.g_b + (int64_t)gb_t * a.g_t + (int64_t)(hv0 + gb_j) * a.g_h);
    beta_raw = Act::ld(a.beta, (int64_t)b * a.be_b + (int64_t)gb_t * a.be_t + (int64_t)(hv0 + gb_j) * a.be_h);
  }
  if (wave == 0) {
    const uint8_t* qrow = (const uint8_t*)a.q + ((int64_t)b * a.q_b + (int64_t)h * a.q_h) * ES;
    dma_stage<(CPT_K + 63) / 64>(lds, a.lds_q, CPT_K, lane, [&](int c) -> const void* { return qrow + 16 * c; });
    const uint8_t* kbase = (const uint8_t*)a.k + ((int64_t)b * a.k_b + (int64_t)h * a.k_h) * ES;
    dma_stage<(kMaxRing * CPT_K + 63) / 64>(lds, a.lds_k, n * CPT_K, lane, [&](int c) -> const void* {
      return kbase + (int64_t)(c / CPT_K) * a.k_t * ES + 16 * (c % CPT_K);
    });
  }
  GDNR_WAIT_VMCNT(0);
  if (gb_live) *(float2*)(lds + a.lds_gb + (gb_t * gw + gb_j) * 8) = make_float2(expf(g_raw), beta_raw);
  GDNR_WAIT_LGKM0();
  __builtin_amdgcn_s_barrier();

  float2 U = Act::ld2(lds + a.lds_q + 2 * lane * ES);
  float lam = 1.0f;
  float* coef = a.coef + (int64_t)b * a.co_b + (int64_t)hv * a.co_h;
  for (int t = n - 1; t >= 0; --t) {
    const float2 kk = Act::ld2(lds + a.lds_k + (t * K + 2 * lane) * ES);
    const float2 gbv = *(const float2*)(lds + a.lds_gb + (t * gw + wave) * 8);
    const float d = wave_sum(fmaf(kk.y, U.y, kk.x * U.x));
    const float s = gbv.y * d;
    if (lane == 0) coef[(int64_t)t * a.co_t] = s * lam;
    U.x = fmaf(-s, kk.x, U.x);
    U.y = fmaf(-s, kk.y, U.y);
    lam *= gbv.x;
  }
  float* tq = a.tq + (int64_t)b * a.tq_b + (int64_t)hv * a.tq_h;
  *(float2*)(tq + 2 * lane) = make_float2(lam * U.x, lam * U.y);
}

// Standalone full-contract preparation (reference kernel:453-576): one wave
// per (sequence, key head); four per workgroup.
template <class Act, bool GATE_F32>
__global__ __launch_bounds__(256) void prep_kernel(const PrepArgs a) {
  constexpr int ES = Act::kBytes;
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (item >= a.B * a.H) return;
  const int b = item / a.H;
  const int h = item % a.H;
  const int p32 = a.pos[(int64_t)b * a.pos_s];
  const int pos = (p32 >= 0 && p32 < a.L) ? p32 : -1;
  const uint8_t* row = (const uint8_t*)a.mixed + (int64_t)b * a.mx_b * ES;
  const float2 qr = Act::ld2(row + (int64_t)(h * K + 2 * lane) * ES);
  const float2 kr = Act::ld2(row + (int64_t)(a.H * K + h * K + 2 * lane) * ES);
  const float qd = sqrtf(wave_sum(fmaf(qr.y, qr.y, qr.x * qr.x)) + 1e-6f);
  const float kd = sqrtf(wave_sum(fmaf(kr.y, kr.y, kr.x * kr.x)) + 1e-6f);
  uint8_t* qo = (uint8_t*)a.q_out + ((int64_t)b * a.qo_b + (int64_t)h * a.qo_h) * ES;
  Act::st2(qo + 2 * lane * ES, qr.x / qd, qr.y / qd);
  if (pos < 0) return;
  uint8_t* kw = (uint8_t*)a.k + ((int64_t)b * a.k_b + (int64_t)pos * a.k_t + (int64_t)h * a.k_h) * ES;
  Act::st2(kw + 2 * lane * ES, kr.x / kd, kr.y / kd);
  for (int j = 0; j < a.G; ++j) {
    const int hv = h * a.G + j;
    for (int e = 2 * lane; e < a.V; e += 128) {
      const float2 vv = Act::ld2(row + ((int64_t)2 * a.H * K + (int64_t)hv * a.V + e) * ES);
      uint8_t* vw = (uint8_t*)a.v + ((int64_t)b * a.v_b + (int64_t)pos * a.v_t + (int64_t)hv * a.v_h + e) * ES;
      Act::st2(vw, vv.x, vv.y);
    }
    if (lane == 0) {
      const float x = ld_gate<GATE_F32, Act>(a.a, (int64_t)b * a.a_b + (int64_t)hv * a.a_h) + a.dt_bias[(int64_t)hv * a.db_s];
      const float sp = x <= 20.0f ? logf(1.0f + expf(x)) : x;  // kernel:560, as written there
      const float gate = -expf(a.a_log[(int64_t)hv * a.al_s]) * sp;
      const float bet = 1.0f / (1.0f + expf(-ld_gate<GATE_F32, Act>(a.bgate, (int64_t)b * a.bg_b + (int64_t)hv * a.bg_h)));
      Act::st(a.g, (int64_t)b * a.g_b + (int64_t)pos * a.g_t + (int64_t)hv * a.g_h, gate);
      Act::st(a.beta, (int64_t)b * a.be_b + (int64_t)pos * a.be_t + (int64_t)hv * a.be_h, bet);
    }
  }
}

#if GDNR_ACT == 0
// vblock32 quantiser (reference ref:36-37,71-99): one wave per 32 x 128 block.
__global__ __launch_bounds__(256) void quantize_kernel(const QuantArgs a) {
  const int lane = threadIdx.x & 63;
  const int nvb = a.V / kVBlock;
  const int item = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (item >= a.B * a.HV * nvb) return;
  const int vb = item % nvb;
  const int hv = (item / nvb) % a.HV;
  const int b = item / (nvb * a.HV);
  const int gi = lane & 7, gm = lane >> 3;
  const float* src = a.state + (int64_t)b * a.st_b + (int64_t)hv * a.st_h + (int64_t)(vb * kVBlock + gm) * a.st_v + 16 * gi;
  float x[4][16];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float4* p = (const float4*)(src + (int64_t)(8 * j) * a.st_v);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 w = p[i];
      x[j][4 * i] = w.x;
      x[j][4 * i + 1] = w.y;
      x[j][4 * i + 2] = w.z;
      x[j][4 * i + 3] = w.w;
    }
  }
  uint32_t am = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) am = max(am, __float_as_uint(x[j][e]) & 0x7FFFFFFFu);
  am = wave_max_u32(am);
  const float amax = __uint_as_float(am);
  const float s32 = (amax > 0.0f) ? amax / 448.0f : 1.0f;
  int sat = 0;
  uint8_t* dst = a.codes + (int64_t)b * a.ck_b + (int64_t)hv * a.ck_h + (int64_t)(vb * kVBlock + gm) * a.ck_v + 16 * gi;
  // quotients x / s32 as IEEE division rounds them: quotient_rn when the
  // block is finite (|x / s32| <= 448 (1 + 2^-23): no clamp needed), else
  // the division with the reference's clamp and NaN encoding
  const bool fast = quotient_fast(am, s32);
  const float r = 1.0f / s32;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float y[16];
    uint4 w;
    if (fast) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        y[e] = quotient_rn(x[j][e], s32, r);
        sat += fabsf(y[e]) > 448.0f ? 1 : 0;
      }
      w.x = f32x4_to_fp8(y[0], y[1], y[2], y[3]);
      w.y = f32x4_to_fp8(y[4], y[5], y[6], y[7]);
      w.z = f32x4_to_fp8(y[8], y[9], y[10], y[11]);
      w.w = f32x4_to_fp8(y[12], y[13], y[14], y[15]);
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        y[e] = x[j][e] / s32;
        sat += fabsf(y[e]) > 448.0f ? 1 : 0;
      }
      w.x = f32x4_to_fp8_ref(y[0], y[1], y[2], y[3]);
      w.y = f32x4_to_fp8_ref(y[4], y[5], y[6], y[7]);
      w.z = f32x4_to_fp8_ref(y[8], y[9], y[10], y[11]);
      w.w = f32x4_to_fp8_ref(y[12], y[13], y[14], y[15]);
    }
    *(uint4*)(dst + (int64_t)(8 * j) * a.ck_v) = w;
  }
  sat = wave_sum_i32(sat);
  if (lane == 0) {
    st_dt(a.scale, (int64_t)b * a.sc_b + (int64_t)hv * a.sc_h + (int64_t)vb * a.sc_v, a.scale_dt, (float)(_Float16)s32);
    if (a.saturated) a.saturated[(int64_t)b * a.sa_b + (int64_t)hv * a.sa_h + (int64_t)vb * a.sa_v] = sat;
  }
}

// state = float(code) * float(scale) (reference ref:109-134).
__global__ __launch_bounds__(256) void dequantize_kernel(const QuantArgs a) {
  const int lane = threadIdx.x & 63;
  const int nvb = a.V / kVBlock;
  const int item = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (item >= a.B * a.HV * nvb) return;
  const int vb = item % nvb;
  const int hv = (item / nvb) % a.HV;
  const int b = item / (nvb * a.HV);
  const int gi = lane & 7, gm = lane >> 3;
  const float sc = ld_dt(a.scale, (int64_t)b * a.sc_b + (int64_t)hv * a.sc_h + (int64_t)vb * a.sc_v, a.scale_dt);
  const uint8_t* src = a.codes + (int64_t)b * a.ck_b + (int64_t)hv * a.ck_h + (int64_t)(vb * kVBlock + gm) * a.ck_v + 16 * gi;
  float* dst = (float*)a.state + (int64_t)b * a.st_b + (int64_t)hv * a.st_h + (int64_t)(vb * kVBlock + gm) * a.st_v + 16 * gi;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint4 w = *(const uint4*)(src + (int64_t)(8 * j) * a.ck_v);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    float4* d = (float4*)(dst + (int64_t)(8 * j) * a.st_v);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float f[4];
      fp8x4_to_f32(ws[i], f);
      d[i] = make_float4(f[0] * sc, f[1] * sc, f[2] * sc, f[3] * sc);
    }
  }
}

#endif  // GDNR_ACT == 0

// ------------------------------------------------------------------ launch
int finish_launch() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : (int)e;
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

template <int NCH, int MODE, bool GATE_F32>
void launch_replay_variant(const ReplayArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)(a.B * (a.HV / a.gw) * a.n_vt)), block((unsigned)(64 * a.gw));
  hipLaunchKernelGGL((replay_kernel<Act, NCH, MODE, GATE_F32>), grid, block, a.lds_bytes, s, a);
}

template <int NCH>
void launch_replay_nch(const ReplayArgs& a, int mode, bool gate_f32, hipStream_t s) {
  if (mode == kModeApply) launch_replay_variant<NCH, kModeApply, false>(a, s);
  else if (mode == kModeFused && gate_f32) launch_replay_variant<NCH, kModeFused, true>(a, s);
  else if (mode == kModeFused) launch_replay_variant<NCH, kModeFused, false>(a, s);
  else launch_replay_variant<NCH, kModeReplay, false>(a, s);
}

}  // namespace

int GDNR_SUFFIX(launch_replay)(const ReplayArgs& a, int mode, bool gate_f32, void* stream) {
  hipStream_t s = (hipStream_t)stream;
  switch (a.block_v) {
    case 32: launch_replay_nch<4>(a, mode, gate_f32, s); break;
    case 64: launch_replay_nch<8>(a, mode, gate_f32, s); break;
    default: launch_replay_nch<16>(a, mode, gate_f32, s); break;
  }
  return finish_launch();
}

int GDNR_SUFFIX(launch_precompute)(const ReplayArgs& a, void* stream) {
  const dim3 grid((unsigned)(a.B * (a.HV / a.gw))), block((unsigned)(64 * a.gw));
  hipLaunchKernelGGL(precompute_kernel<Act>, grid, block, a.lds_bytes, (hipStream_t)stream, a);
  return finish_launch();
}

int GDNR_SUFFIX(launch_prep)(const PrepArgs& a, bool gate_f32, void* stream) {
  const dim3 grid((unsigned)((a.B * a.H + 3) / 4)), block(256);
  if (gate_f32) hipLaunchKernelGGL((prep_kernel<Act, true>), grid, block, 0, (hipStream_t)stream, a);
  else hipLaunchKernelGGL((prep_kernel<Act, false>), grid, block, 0, (hipStream_t)stream, a);
  return finish_launch();
}

#if GDNR_ACT == 0
int launch_quantize(const QuantArgs& a, void* stream) {
  const int items = a.B * a.HV * (a.V / kVBlock);
  hipLaunchKernelGGL(quantize_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, (hipStream_t)stream, a);
  return finish_launch();
}

int launch_dequantize(const QuantArgs& a, void* stream) {
  const int items = a.B * a.HV * (a.V / kVBlock);
  hipLaunchKernelGGL(dequantize_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, (hipStream_t)stream, a);
  return finish_launch();
}

const char* hip_error_string(int code) { return hipGetErrorString((hipError_t)code); }
#endif

}  // namespace gdnr
