// gdnr_internal.h -- kernel argument blocks shared by the C-ABI layer
// (gdnr_abi.cpp, host validation) and the HIP kernels (gdnr_kernels.hip).
// All strides are in elements of the tensor they index.
#pragma once

#include <stdint.h>

namespace gdnr {

enum DType : int32_t {
  DT_BF16 = 0, DT_F16 = 1, DT_F32 = 2, DT_FP8 = 3, DT_U8 = 4, DT_I32 = 5, DT_I64 = 6, DT_BOOL = 7
};

constexpr int kKeyDim = 128;      // K: the only head_k_dim built (Qwen3.5 / Qwen3-Next GDN)
constexpr int kVBlock = 32;       // V-rows per checkpoint scale
constexpr int kMaxVBlocks = 4;    // vblocks per step-kernel V-tile (block_v <= 128)
constexpr int kMaxRing = 64;      // ring capacity bound (one VGPR lane per token)
constexpr int kMaxWavesPerWG = 4; // value heads per workgroup (one wave each)

// Replay / flush / split-apply / fused prep+replay: one workgroup per
// (sequence b, group of gw value heads sharing key head h, V-tile vt).
//
// Hot-path dtypes are compile-time: q, k/v/g/beta rings, out and mixed_qkv
// share the activation dtype (template), the checkpoint scale is fp16,
// valid_len/pos are int32, flush is one byte per sequence, a/b are the
// activation dtype or f32 (template), A_log/dt_bias are f32.
struct ReplayArgs {
  uint8_t* ckpt; int64_t ck_b, ck_h, ck_v;
  uint16_t* scale; int64_t sc_b, sc_h, sc_v;      // fp16 bits
  const void* q; int64_t q_b, q_h;
  void* k; int64_t k_b, k_t, k_h;
  void* v; int64_t v_b, v_t, v_h;
  void* g; int64_t g_b, g_t, g_h;
  void* beta; int64_t be_b, be_t, be_h;
  const int32_t* valid_len; int64_t vl_s;
  const uint8_t* flush; int64_t fl_s;              // nullptr: never flush
  void* out; int64_t o_b, o_h;
  // split buffers: precompute writes them, apply reads them
  float* tq; int64_t tq_b, tq_h;
  float* coef; int64_t co_b, co_h, co_t;
  // fused preparation (prep_replay)
  const void* mixed; int64_t mx_b;
  const void* a; int64_t a_b, a_h;
  const void* bgate; int64_t bg_b, bg_h;
  const float* a_log; int64_t al_s;
  const float* dt_bias; int64_t db_s;
  const int32_t* pos; int64_t pos_s;
  void* q_out; int64_t qo_b, qo_h;
  // geometry
  int32_t B, H, HV, G, V, L;   // L = ring capacity (tensor dim 1)
  int32_t gw;                  // value heads (waves) per workgroup, divides G
  int32_t block_v, n_vt;       // V rows per workgroup, V / block_v
  float out_scale;             // K^-1/2
  // LDS byte offsets (computed on the host)
  int32_t lds_q, lds_k, lds_v, lds_gb, lds_t, lds_bytes;
  // step kernel (gdnr_step.hip, rings of up to kStepRing tokens): waves per
  // workgroup, V-rows per wave, the new token's k row, per-head publish
  // flags, coefficients and [17 x 17] Gram matrices
  int32_t sw, rpw, lds_knew, lds_flag, lds_c, lds_g;
  int32_t units;  // decode kernel: (key head, value-head group) units per workgroup
  int32_t nwh;    // decode kernel: row waves per value head
  int32_t seq_major;  // decode kernel: workgroups numbered sequence-fastest (grid x = sequences)
  // flush (MFMA rebuild), per head: R = (I + M)^-1 [16 x 16] f32, per-token
  // factors (pre, post, dq, -) f32, lam_all f32; K^T operand tiles [K x 16]
  // in the ring dtype; per-head scratch (3 KiB)
  int32_t lds_r, lds_fac, lds_kt, lds_lam, lds_u;
  // slot indirection of the fused step (see StepArgs); slot == nullptr: none
  const int32_t* slot; int64_t sl_s; int32_t n_slots;
};

constexpr int32_t kMaxStepLds = 160 * 1024;  // gfx950 LDS per workgroup
constexpr int kStepRing = 16;                // ring capacity handled by the step kernel
constexpr int kDecodeChunks = 4;             // chunks of kStepRing tokens of the decode kernel's longest ring
constexpr uint32_t kWaitPolls = 1u << 22;     // default poll budget of a bounded LDS wait

// Argument block of the step kernel (gdnr_step.hip), built on the host from a
// validated ReplayArgs: byte pointers and 32-bit BYTE strides (the host checks
// that every tensor's byte extent fits), so that address arithmetic is 32-bit
// scalar work and the block stays small enough to live in SGPRs.
struct StepArgs {
  uint8_t* ckpt; uint8_t* scale;  // scale: fp16 bits
  const uint8_t* q; uint8_t* k; uint8_t* v; uint8_t* g; uint8_t* beta; uint8_t* out;
  const uint8_t* valid_len; const uint8_t* flush; const uint8_t* pos;  // flush: nullptr = never
  const uint8_t* mixed; const uint8_t* a; const uint8_t* bgate; const uint8_t* a_log; const uint8_t* dt_bias;
  uint8_t* q_out;
  uint32_t ck_b, ck_h, ck_v, sc_b, sc_h, sc_v, q_b, q_h, k_b, k_t, k_h, v_b, v_t, v_h;
  uint32_t g_b, g_t, g_h, be_b, be_t, be_h, vl_s, fl_s, pos_s, o_b, o_h, mx_b;
  uint32_t a_b, a_h, bg_b, bg_h, al_s, db_s, qo_b, qo_h;
  int32_t B, H, G, V, L, gw, block_v, n_vt, sw, rpw, units, nwh, seq_major;
  float out_scale;
  int32_t lds_q, lds_knew, lds_k, lds_flag, lds_c, lds_t, lds_g, lds_v, lds_r, lds_fac, lds_kt, lds_lam, lds_u, lds_bytes;
  // slot indirection (fused step only): sequence b's checkpoint, scale and
  // ring rows are those of slot slot[b] (int32, clamped to [0, n_slots));
  // nullptr: slot b
  const uint8_t* slot; uint32_t sl_s; int32_t n_slots;
  // device word counting bounded waits that gave up (status_word()), and
  // the poll budget of every bounded wait (wait_polls())
  uint32_t* status;
  uint32_t wait_polls;
};

struct PrepArgs {
  const void* mixed; int64_t mx_b;
  const void* a; int64_t a_b, a_h;
  const void* bgate; int64_t bg_b, bg_h;
  const float* a_log; int64_t al_s;
  const float* dt_bias; int64_t db_s;
  const int32_t* pos; int64_t pos_s;
  void* q_out; int64_t qo_b, qo_h;
  void* k; int64_t k_b, k_t, k_h;
  void* v; int64_t v_b, v_t, v_h;
  void* g; int64_t g_b, g_t, g_h;
  void* beta; int64_t be_b, be_t, be_h;
  int32_t B, H, HV, G, V, L;
};

struct QuantArgs {
  const float* state; int64_t st_b, st_h, st_v;   // quantise reads, dequantise writes (as float*)
  uint8_t* codes; int64_t ck_b, ck_h, ck_v;
  void* scale; int64_t sc_b, sc_h, sc_v; int32_t scale_dt;
  int32_t* saturated; int64_t sa_b, sa_h, sa_v;   // may be null
  int32_t B, HV, V;
};

// Checkpoint formats of the reference quantiser (gdnr_formats.hip): scale
// group granularity, tile size (tile / vblock), fp8 or int8 codes. Strides
// in elements; the scale and saturated tensors are indexed [b, hv, i, j]
// (unused trailing strides are 0).
enum Granularity : int32_t { kGranHead = 0, kGranRow = 1, kGranTile = 2, kGranVblock = 3 };
struct FormatArgs {
  float* state; int64_t st_b, st_h, st_v;  // quantise reads it, dequantise writes it
  void* payload; int64_t pl_b, pl_h, pl_v;
  void* scale; int64_t sc_b, sc_h, sc_r, sc_c; int32_t scale_dt;
  int32_t* saturated; int64_t sa_b, sa_h, sa_r, sa_c;  // may be null
  int32_t B, HV, V, K, gran, tile, int8;
};

// Full-state read-modify-write decode step (gdnr_rmw.hip). The state
// strides are in state elements, the others in activation elements.
struct RmwArgs {
  void* state; int64_t st_b, st_h, st_v;
  const void* q; int64_t q_b, q_h;
  const void* k; int64_t k_b, k_h;
  const void* v; int64_t v_b, v_h;
  const void* g; int64_t g_b, g_h;
  const void* beta; int64_t be_b, be_h;
  void* out; int64_t o_b, o_h;
  int32_t B, HV, V, G;
  float out_scale;
  // production contract (packed decode): q, k, v from the raw mixed_qkv row,
  // q/k L2 norm and the gates computed in the kernel, the state addressed by
  // slot[b] (clamped to [0, n_slots)); q, k, v, g, beta above are unused
  const void* mixed; int64_t mx_b;
  const void* a; int64_t a_b, a_h;
  const void* bgate; int64_t bg_b, bg_h;
  const float* a_log; int64_t al_s;
  const float* dt_bias; int64_t db_s;
  const int32_t* slot; int64_t sl_s; int32_t n_slots, H;
};

// Launch modes of the replay kernel.
enum ReplayMode : int { kModeReplay = 0, kModeApply = 1, kModeFused = 2 };

// Launchers: one set per activation dtype, each in its own translation unit
// (gdnr_kernels.hip compiled with GDNR_ACT=0/1/2). Return 0 or a hipError_t.
#define GDNR_DECLARE_LAUNCHERS(SUFFIX)                                                      \
  int launch_replay_##SUFFIX(const ReplayArgs& a, int mode, bool gate_f32, void* stream); \
  int launch_precompute_##SUFFIX(const ReplayArgs& a, void* stream);                      \
  int launch_prep_##SUFFIX(const PrepArgs& a, bool gate_f32, void* stream);                \
  int launch_step_##SUFFIX(const StepArgs& a, bool fused, bool gate_f32, void* stream);
GDNR_DECLARE_LAUNCHERS(bf16)
GDNR_DECLARE_LAUNCHERS(f16)
GDNR_DECLARE_LAUNCHERS(f32)
#undef GDNR_DECLARE_LAUNCHERS
// decode kernel (gdnr_decode.hip): 16-bit activations, rings of <= 16 tokens,
// V % 64 == 0; StepArgs.gw value heads per workgroup, StepArgs.sw = V / 64
// waves per value head
int launch_decode_bf16(const StepArgs& a, bool fused, bool gate_f32, void* stream);
int launch_decode_f16(const StepArgs& a, bool fused, bool gate_f32, void* stream);
int32_t decode_lds_bytes(int32_t units, int32_t row_waves, int32_t vblocks, int32_t chunks);
// the device word of the current device that counts bounded waits which gave
// up (nullptr if the symbol cannot be resolved), and its host read-out
uint32_t* status_word();
int read_status(uint32_t* count, bool reset);
// poll budget of the kernels' bounded waits (kWaitPolls until the host sets
// another with gdnr_set_wait_polls; process-wide)
uint32_t wait_polls();
uint32_t set_wait_polls(uint32_t polls);
int device_cus();
// The split replay's device array for gdnr_replay_fp8_split_noalloc (T_0 and
// the coefficients, packed; 3 MiB per GPU: B*HV <= 4096 at K = 128 with a
// ring of up to 64), and its address on the current device (nullptr if the
// symbol cannot be resolved).
constexpr int64_t kSplitScratchBytes = 3 << 20;
uint8_t* split_scratch();
int launch_quantize(const QuantArgs& a, void* stream);
int launch_rmw_step(const RmwArgs& a, int state_dt, int act_dt, void* stream);
int launch_rmw_packed(const RmwArgs& a, int state_dt, int act_dt, bool gate_f32, void* stream);
int launch_format_quantize(const FormatArgs& a, void* stream);
int launch_format_dequantize(const FormatArgs& a, void* stream);
int launch_dequantize(const QuantArgs& a, void* stream);
// coalesced stream over bytes (a multiple of 16) at buf: read only, or read
// and written back in place; plain or non-temporal loads; chunked: read only,
// in the decode kernel's order (a 16 KiB chunk per wave, 16 loads in flight),
// tiled: with the decode row wave's load pattern inside each chunk
int launch_stream_probe(void* buf, int64_t bytes, bool write, bool nt, bool chunked, bool tiled, void* stream);
const char* hip_error_string(int code);

}  // namespace gdnr
