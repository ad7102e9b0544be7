// gdnr_rmw.hip -- the full-state read-modify-write decode step on gfx950:
// the comparator of the ReplaySSM path. One gated delta-rule token per
// sequence is applied to a state held in full ([B,HV,V,K], bf16/f16/f32),
// which is read and written back:
//   S <- e^g S;  r = S k;  S <- S + beta (v - r) k^T;  o = (S q) K^-1/2
// (the reference's _gdn_bf16_step_kernel, prototype/gdn_replayssm_fp8_kernel.py:245-341,
// host wrapper gdn_bf16_step :408-450; fp32 arithmetic, the state stored
// back in its own dtype with round-to-nearest-even, o in the activation dtype).
//
// The packed form takes the production operator's contract instead: the raw
// mixed_qkv row, q/k L2 norm and the gates in the kernel, a slot-indexed
// state and out [B, 1, HV, V] (findings.md:35-45) -- the comparator of the
// full-contract ReplaySSM step.
//
// The state update keeps the reference's order and roundings (S' = e^g S
// elementwise, r = S' k, S = S' + c k with c = (v - r) beta); the output uses
// S q = S' q + c (k . q), so its two row sums (S' k and S' q) are reduced
// together -- equal to the reference's sum of (S q) up to fp32 rounding.
//
// HBM-bound: every state byte is read once and written once; nothing else is
// larger than a row. A wave owns 32 V-rows of one value head; a lane owns one
// 16-byte chunk of a row (8 elements of a 2-byte state, 4 of an f32 one), so
// a row spans 16 or 32 lanes and each wave instruction moves 4 or 2 whole
// rows. All of a wave's chunk loads are issued before the first is used; each
// row's store follows its compute while later rows are still arriving. The
// row sums reduce across the row's lanes with DPP (plus one swizzle for
// 32-lane rows). Measured on MI355X at the C1 shape: within 15% of an in-place
// load/store kernel with the same access pattern and no arithmetic.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gdnr_device.h"
#include "gdnr_internal.h"

namespace gdnr {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// sum over the aligned group of LANES lanes (16 or 32), in every lane of it
template <int LANES>
__device__ __forceinline__ float row_sum(float x) {
  x = sum8(x);
  x += dpp_f<kDppMirror>(x);
  if constexpr (LANES == 32) x += __shfl_xor(x, 16);
  return x;
}

// 16-byte chunk <-> EPC floats in the state dtype
template <class S>
__device__ __forceinline__ void chunk_to_f32(const u32x4_t c, float* f) {
  const uint32_t w[4] = {c[0], c[1], c[2], c[3]};
  if constexpr (S::kBytes == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = __uint_as_float(w[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float2 p = S::from_pair(w[i]);
      f[2 * i] = p.x;
      f[2 * i + 1] = p.y;
    }
  }
}
template <class S>
__device__ __forceinline__ u32x4_t f32_to_chunk(const float* f) {
  if constexpr (S::kBytes == 4) {
    return u32x4_t{__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3])};
  } else {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t pair;
      S::st2(&pair, f[2 * i], f[2 * i + 1]);
      w[i] = pair;
    }
    return u32x4_t{w[0], w[1], w[2], w[3]};
  }
}

// RPW V-rows of one value head per wave, four waves per workgroup over
// consecutive rows of a sequence's [HV, V] row space. PACKED: the production
// contract -- q, k, v from the raw mixed_qkv row, q and k L2-normalised and
// the gates formed in fp32 here (the formulas of the full-contract prep,
// kernel:504-562), the state of slot slot[b].
template <class S, class Act, int RPW, bool PACKED = false, bool GATE_F32 = false>
__global__ __launch_bounds__(256) void rmw_step_kernel(const RmwArgs a) {
  constexpr int ES = S::kBytes;
  constexpr int EPC = 16 / ES;              // state elements per lane chunk
  constexpr int LPR = kKeyDim / EPC;        // lanes per row: 16 or 32
  constexpr int RPI = 64 / LPR;             // rows per wave instruction: 4 or 2
  constexpr int NI = RPW / RPI;             // chunk loads per lane
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = blockIdx.y;
  const int flat = (blockIdx.x * 4 + wave) * RPW;  // first row in the sequence's [HV, V] rows
  if (flat >= a.HV * a.V) return;                  // wave-uniform
  const int hv = flat / a.V, row0 = flat - hv * a.V;
  const int h = hv / a.G;
  const int cl = lane % LPR, rsub = lane / LPR;
  int bs = b;  // the state's row of this sequence
  if constexpr (PACKED) {
    const int sl = (int)__builtin_amdgcn_readfirstlane((int)*(const uint32_t*)(a.slot + b * a.sl_s));
    bs = (sl >= 0 && sl < a.n_slots) ? sl : 0;  // out of range: the null slot
  }

  uint8_t* sbase = (uint8_t*)a.state + (bs * a.st_b + hv * a.st_h + (int64_t)row0 * a.st_v) * ES;
  const uint32_t row_bytes = (uint32_t)(a.st_v * ES);
  const uint32_t lane_off = (uint32_t)rsub * row_bytes + 16u * (uint32_t)cl;
  u32x4_t ch[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) ch[i] = *(const u32x4_t*)(sbase + (lane_off + (uint32_t)(i * RPI) * row_bytes));

  // k and q of the key head at this lane's columns, the head's gate and
  // beta, and the v element of each row this lane touches
  float kf[EPC], qf[EPC], gamma, beta;
  const uint8_t* vp;
  if constexpr (PACKED) {
    const uint8_t* row = (const uint8_t*)a.mixed + (int64_t)b * a.mx_b * Act::kBytes;
    const uint8_t* qp = row + (h * kKeyDim + EPC * cl) * Act::kBytes;
    const uint8_t* kp = row + ((a.H + h) * kKeyDim + EPC * cl) * Act::kBytes;
    float qs = 0.f, ks = 0.f;
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      qf[e] = Act::ld(qp, e);
      kf[e] = Act::ld(kp, e);
      qs = fmaf(qf[e], qf[e], qs);
      ks = fmaf(kf[e], kf[e], ks);
    }
    const float qd = sqrtf(row_sum<LPR>(qs) + 1e-6f), kd = sqrtf(row_sum<LPR>(ks) + 1e-6f);
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      qf[e] = qf[e] / qd;
      kf[e] = kf[e] / kd;
    }
    const float araw = GATE_F32 ? ((const float*)a.a)[b * a.a_b + hv * a.a_h] : Act::ld(a.a, b * a.a_b + hv * a.a_h);
    const float braw = GATE_F32 ? ((const float*)a.bgate)[b * a.bg_b + hv * a.bg_h]
                                : Act::ld(a.bgate, b * a.bg_b + hv * a.bg_h);
    const float x = araw + a.dt_bias[hv * a.db_s];
    const float sp = x <= 20.0f ? logf(1.0f + expf(x)) : x;
    gamma = expf(-expf(a.a_log[hv * a.al_s]) * sp);
    beta = 1.0f / (1.0f + expf(-braw));
    vp = row + (2 * a.H * kKeyDim + hv * a.V + row0 + rsub) * Act::kBytes;
  } else {
    const uint8_t* kp = (const uint8_t*)a.k + (b * a.k_b + h * a.k_h + EPC * cl) * Act::kBytes;
    const uint8_t* qp = (const uint8_t*)a.q + (b * a.q_b + h * a.q_h + EPC * cl) * Act::kBytes;
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      kf[e] = Act::ld(kp, e);
      qf[e] = Act::ld(qp, e);
    }
    gamma = expf(Act::ld(a.g, b * a.g_b + hv * a.g_h));
    beta = Act::ld(a.beta, b * a.be_b + hv * a.be_h);
    vp = (const uint8_t*)a.v + (b * a.v_b + hv * a.v_h + row0 + rsub) * Act::kBytes;
  }
  uint8_t* op = (uint8_t*)a.out + (b * a.o_b + hv * a.o_h + row0 + rsub) * Act::kBytes;

  float kq = 0.f;
#pragma unroll
  for (int e = 0; e < EPC; ++e) kq = fmaf(kf[e], qf[e], kq);
  kq = row_sum<LPR>(kq);
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    float s[EPC];
    chunk_to_f32<S>(ch[i], s);
    float r = 0.f, sq = 0.f;
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      s[e] *= gamma;
      r = fmaf(s[e], kf[e], r);
      sq = fmaf(s[e], qf[e], sq);
    }
    r = row_sum<LPR>(r);
    sq = row_sum<LPR>(sq);
    const float c = (Act::ld(vp, i * RPI) - r) * beta;
#pragma unroll
    for (int e = 0; e < EPC; ++e) s[e] = fmaf(c, kf[e], s[e]);
    const float o = fmaf(c, kq, sq);
    *(u32x4_t*)(sbase + (lane_off + (uint32_t)(i * RPI) * row_bytes)) = f32_to_chunk<S>(s);
    if (cl == 0) Act::st(op, i * RPI, o * a.out_scale);
  }
}

template <class S, class Act, bool PACKED = false, bool GATE_F32 = false>
void launch_rows(const RmwArgs& a, hipStream_t s) {
  const int rows = a.HV * a.V;  // V % 32 == 0: a wave's rows stay in one head
  const dim3 grid((rows + 4 * 32 - 1) / (4 * 32), a.B);
  hipLaunchKernelGGL((rmw_step_kernel<S, Act, 32, PACKED, GATE_F32>), grid, dim3(256), 0, s, a);
}

template <class S>
int launch_for_state(const RmwArgs& a, int act, hipStream_t s) {
  switch (act) {
    case DT_BF16: launch_rows<S, ActBF16>(a, s); break;
    case DT_F16: launch_rows<S, ActF16>(a, s); break;
    case DT_F32: launch_rows<S, ActF32>(a, s); break;
    default: return (int)hipErrorInvalidValue;
  }
  return (int)hipGetLastError();
}

template <class S>
int launch_packed_for_state(const RmwArgs& a, int act, bool gate_f32, hipStream_t s) {
  switch (act) {
    case DT_BF16: gate_f32 ? launch_rows<S, ActBF16, true, true>(a, s) : launch_rows<S, ActBF16, true, false>(a, s); break;
    case DT_F16: gate_f32 ? launch_rows<S, ActF16, true, true>(a, s) : launch_rows<S, ActF16, true, false>(a, s); break;
    case DT_F32: launch_rows<S, ActF32, true, true>(a, s); break;
    default: return (int)hipErrorInvalidValue;
  }
  return (int)hipGetLastError();
}

}  // namespace

int launch_rmw_packed(const RmwArgs& a, int state_dt, int act_dt, bool gate_f32, void* stream) {
  const hipStream_t s = (hipStream_t)stream;
  switch (state_dt) {
    case DT_BF16: return launch_packed_for_state<ActBF16>(a, act_dt, gate_f32, s);
    case DT_F16: return launch_packed_for_state<ActF16>(a, act_dt, gate_f32, s);
    case DT_F32: return launch_packed_for_state<ActF32>(a, act_dt, gate_f32, s);
    default: return (int)hipErrorInvalidValue;
  }
}

int launch_rmw_step(const RmwArgs& a, int state_dt, int act_dt, void* stream) {
  const hipStream_t s = (hipStream_t)stream;
  switch (state_dt) {
    case DT_BF16: return launch_for_state<ActBF16>(a, act_dt, s);
    case DT_F16: return launch_for_state<ActF16>(a, act_dt, s);
    case DT_F32: return launch_for_state<ActF32>(a, act_dt, s);
    default: return (int)hipErrorInvalidValue;
  }
}

}  // namespace gdnr
