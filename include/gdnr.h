/*
 * gdnr.h -- C ABI of libgdnreplay.so: the ReplaySSM decode path of gated
 * delta-rule (GDN) layers, written for AMD Instinct MI355X (gfx950).
 *
 * The path keeps each sequence's recurrent state S [HV, V, K] as an
 * FP8-E4M3FN checkpoint with one fp16 scale per 32 V-rows x K ("vblock32"),
 * plus a ring of the last L tokens' (k, v, g, beta). A decode step replays
 * the ring against the dequantised checkpoint and emits o = S q * K^-1/2
 * without materialising S; when the ring fills, the state is rebuilt and
 * requantised in place ("flush").
 *
 * Conventions shared by every entry point:
 *  - Tensors are passed as gdnr_tensor: a device pointer, a dtype code,
 *    the logical shape and per-dimension strides counted in ELEMENTS.
 *    Outer strides are arbitrary; the innermost (K or V) stride must be 1.
 *  - `stream` is a hipStream_t (NULL = the default stream). Kernels are
 *    enqueued asynchronously; no entry point synchronises the device.
 *  - The library allocates no device memory: every buffer is caller-owned.
 *  - No C++ exception crosses the ABI. A nonzero return code means nothing
 *    was launched; gdnr_last_error() (thread-local) says why.
 *  - Arguments are validated on the host before any HIP call, so a bad
 *    shape, dtype, stride or alignment is an error, never a silent
 *    out-of-bounds access. Per-sequence device metadata (valid_len, pos) is
 *    clamped in the kernels: valid_len to [0, ring length]; a pos outside
 *    [0, ring length) appends nothing.
 */
#ifndef GDNR_H
#define GDNR_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GDNR_ABI_VERSION 1
#define GDNR_MAX_DIMS 4

typedef enum gdnr_dtype {
  GDNR_DTYPE_BF16 = 0,
  GDNR_DTYPE_F16 = 1,
  GDNR_DTYPE_F32 = 2,
  GDNR_DTYPE_FP8E4M3FN = 3, /* OCP e4m3fn: bias 7, max 448, no inf, 0x7F/0xFF NaN */
  GDNR_DTYPE_U8 = 4,        /* accepted wherever fp8 codes are: raw bytes */
  GDNR_DTYPE_I32 = 5,
  GDNR_DTYPE_I64 = 6,
  GDNR_DTYPE_BOOL = 7,
  GDNR_DTYPE_I8 = 8         /* int8 checkpoint codes (the *_int8 formats) */
} gdnr_dtype;

/* scale-group granularity of a checkpoint format (gdnr_quantize_checkpoint) */
typedef enum gdnr_granularity {
  GDNR_GRANULARITY_HEAD = 0,   /* one scale per value head [V, K] */
  GDNR_GRANULARITY_ROW = 1,    /* one scale per V-row */
  GDNR_GRANULARITY_TILE = 2,   /* one scale per tile_size x tile_size tile */
  GDNR_GRANULARITY_VBLOCK = 3  /* one scale per tile_size V-rows x K */
} gdnr_granularity;

typedef struct gdnr_tensor {
  void* data;                       /* device pointer */
  int32_t dtype;                    /* gdnr_dtype */
  int32_t ndim;                     /* 1..GDNR_MAX_DIMS */
  int64_t shape[GDNR_MAX_DIMS];
  int64_t strides[GDNR_MAX_DIMS];   /* in elements */
} gdnr_tensor;

enum {
  GDNR_OK = 0,
  GDNR_ERR_INVALID_ARGUMENT = 1, /* shape / dtype / stride / alignment misuse */
  GDNR_ERR_UNSUPPORTED = 2,      /* legal for the reference, not built here (e.g. K != 128) */
  GDNR_ERR_HIP = 3               /* a HIP runtime call failed */
};

/* Thread-local description of the last failure on this thread ("" if none). */
const char* gdnr_last_error(void);

/* GDNR_ABI_VERSION of the loaded library. */
int gdnr_abi_version(void);

/*
 * Diagnostics of the decode kernels' bounded waits. Inside a workgroup the
 * waves hand the coefficient chain, the flush factors and the flush's
 * helper results to each other through LDS flags, and every such wait is
 * bounded (2^22 polls by default). A wait that gives up adds 1 to a
 * per-device status word; the wave then goes on with whatever the LDS holds,
 * so the step's outputs are meaningless, but it skips its in-place
 * checkpoint code and scale stores (decode and step kernels alike): a step
 * whose waits gave up leaves the checkpoint as it was. Ring appends, which
 * depend on no wait, are still made.
 * *count receives the current device's word; reset != 0 clears it. This
 * call synchronises the device (it copies the word to the host).
 * No counterpart in the reference (its Triton kernels have no inter-wave waits).
 */
int gdnr_wait_timeouts(uint32_t* count, int32_t reset);

/*
 * Sets the poll budget of every bounded wait of later launches (process-wide;
 * 4194304 = 2^22 is the default) and returns the previous budget. A budget of
 * 0 makes every wait give up at once: a test of the give-up path, whose
 * kernels still run to their end. No counterpart in the reference.
 */
uint32_t gdnr_set_wait_polls(uint32_t polls);

/*
 * The decode kernel's launch plan for a shape (the plan gdnr_replay_fp8,
 * gdnr_prep_replay_fp8 and the slot entry use with 16-bit activations: rings
 * of <= 16 tokens with V = 64, 128 or 256, and rings of <= 64 tokens, as
 * 16-token chunks, with V = 64 or 128 while batch * value_heads is at most
 * twice the device's compute units): plan[0] = V-rows per row wave,
 * plan[1] = row waves per value head, plan[2] = value heads per unit (gw),
 * plan[3] = units per workgroup, plan[4] = LDS bytes per workgroup.
 * GDNR_ERR_UNSUPPORTED when the shape takes another kernel. Host-only (it reads the current device's
 * compute-unit count); tests use it to name the instantiation they cover.
 * No counterpart in the reference (its tiling is the block_v argument).
 */
int gdnr_decode_plan(int32_t batch, int32_t heads, int32_t value_heads, int32_t value_dim, int32_t ring_len,
                     int32_t act_dtype, int32_t* plan);

/*
 * Measurement probe: one coalesced pass over `buffer` (any dtype,
 * C-contiguous, 16-byte aligned, a whole number of 16-byte pieces), reading
 * it, or (flags bit 0) reading it and writing every piece back unchanged in
 * place; flags bit 1 makes the loads non-temporal, as the decode kernels'
 * checkpoint loads are; flags bit 2 (reads only) reads in the decode
 * kernel's order instead of a grid-strided sweep: one workgroup of 8 waves
 * per compute unit, each wave a contiguous 16 KiB chunk with 16 loads in
 * flight per lane; with bit 3 as well, each chunk is read in the decode row
 * wave's pattern (every load takes half of each of 16 rows of 128 bytes). Timed by the benchmark as the HBM floor of the decode
 * step's checkpoint traffic (the replay reads the codes once, the flush
 * reads and rewrites them) and swept over buffer sizes for the per-launch
 * fixed cost and the plateau. The buffer's contents are left unchanged.
 * No counterpart in the reference (its byte counts are formulas:
 * prototype/bench_gdn_replayssm.py:45-87; its bandwidth probes are
 * prototype/bench_kernel_diag.py:39-148).
 */
int gdnr_stream_probe(const gdnr_tensor* buffer, int32_t flags, void* stream);

/*
 * One decode step of the replay, per sequence b:
 *   flush[b] == 0: adjoint replay of ring tokens [0, valid_len[b]) against the
 *                  dequantised checkpoint; writes out[b] only.
 *   flush[b] != 0: forward rebuild of the state over the same tokens, writes
 *                  out[b] from the rebuilt fp32 state, then requantises it to
 *                  vblock32 IN PLACE (checkpoint[b], checkpoint_scale[b]).
 * Shapes: checkpoint [B,HV,V,K] fp8/u8; checkpoint_scale [B,HV,V/32] f16;
 *   q [B,H,K]; k_cache [B,L,H,K]; v_cache [B,L,HV,V]; g_cache, beta_cache
 *   [B,L,HV]; valid_len [B] i32; flush [B] bool|u8; out [B,HV,V].
 *   q, k_cache, v_cache, g_cache, beta_cache and out share one dtype
 *   (bf16|f16|f32). K == 128, V % 32 == 0, HV % H == 0, 1 <= L <= 64.
 * block_v (32|64|128, dividing V) is the number of V-rows one workgroup
 *   streams; unlike the reference it does not constrain the flush.
 * Replaces gdn_replay_fp8, prototype/gdn_replayssm_fp8_kernel.py:344-405
 * (device work: _gdn_replay_fp8_kernel, same file :20-242).
 */
int gdnr_replay_fp8(const gdnr_tensor* checkpoint, const gdnr_tensor* checkpoint_scale,
                    const gdnr_tensor* q, const gdnr_tensor* k_cache,
                    const gdnr_tensor* v_cache, const gdnr_tensor* g_cache,
                    const gdnr_tensor* beta_cache, const gdnr_tensor* valid_len,
                    const gdnr_tensor* flush, const gdnr_tensor* out,
                    int32_t block_v, void* stream);

/*
 * Non-flush replay as two launches: a precompute that writes the
 * transformed query T_0 into transformed_query [B,HV,K] f32 and the
 * per-token coefficients c_t = beta_t (k_t . T_t) into coefficient
 * [B,HV,Lc] f32 (Lc >= ring length; only t < valid_len[b] is written), then
 * an apply that streams the checkpoint: out = (scale*codes) T_0 + sum_t c_t v_t.
 * precompute_grouped selects one precompute workgroup per key head (k read
 * once for the GQA group) instead of one per value head; results are equal.
 * block_kc is accepted for signature parity and must be 128 or K.
 * Replaces gdn_replay_fp8_split, prototype/gdn_replayssm_fp8_kernel.py:1129-1235
 * (device work: same file :798-1126).
 */
int gdnr_replay_fp8_split(const gdnr_tensor* checkpoint, const gdnr_tensor* checkpoint_scale,
                          const gdnr_tensor* q, const gdnr_tensor* k_cache,
                          const gdnr_tensor* v_cache, const gdnr_tensor* g_cache,
                          const gdnr_tensor* beta_cache, const gdnr_tensor* valid_len,
                          const gdnr_tensor* transformed_query,
                          const gdnr_tensor* coefficient, const gdnr_tensor* out,
                          int32_t block_v, int32_t block_kc, int32_t precompute_grouped,
                          void* stream);

/*
 * gdnr_replay_fp8_split without the two buffers: T_0 and the coefficients
 * live in a device array of the library (3 MiB per GPU, held until the
 * process ends), so the call allocates nothing. No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Limit:
 * B*HV*(K + ring length)*4 bytes <= 3 MiB (B*HV <= 4096 at K = 128 with a
 * ring of up to 64); larger calls return GDNR_ERR_UNSUPPORTED. Every call on
 * a GPU shares that GPU's array: calls that overlap on one GPU (concurrent
 * streams, or graphs replayed concurrently) race. Arguments and results are
 * otherwise those of gdnr_replay_fp8_split.
 */
int gdnr_replay_fp8_split_noalloc(const gdnr_tensor* checkpoint, const gdnr_tensor* checkpoint_scale,
                                  const gdnr_tensor* q, const gdnr_tensor* k_cache,
                                  const gdnr_tensor* v_cache, const gdnr_tensor* g_cache,
                                  const gdnr_tensor* beta_cache, const gdnr_tensor* valid_len,
                                  const gdnr_tensor* out, int32_t block_v, int32_t block_kc,
                                  int32_t precompute_grouped, void* stream);

/*
 * Full-contract preparation of one token per sequence:
 *   q,k <- x / sqrt(sum(x^2) + 1e-6) (per key head), q -> q_out[b],
 *   k -> k_ring[b, pos[b]], v (copied) -> v_ring[b, pos[b]],
 *   g = -exp(A_log) * softplus_20(a + dt_bias) -> g_ring[b, pos[b]],
 *   beta = sigmoid(b) -> beta_ring[b, pos[b]].
 * Shapes: mixed_qkv [B, 2*H*K + HV*V] (row stride free, unit inner stride);
 *   a, b [B,HV] f32 or the ring dtype; a_log, dt_bias [HV] f32; pos [B]
 *   i32; q_out [B,H,K]; k_ring [B,L,H,K]; v_ring [B,L,HV,V];
 *   g_ring, beta_ring [B,L,HV]. mixed_qkv, q_out, k_ring, v_ring share a dtype.
 * `fused` is accepted for signature parity (0 and 1 run the same kernel).
 * beta_ring is addressed with its own strides (the reference reuses
 * g_ring's, kernel:570-575; identical whenever the two rings match).
 * Replaces gdn_prep_ring, prototype/gdn_replayssm_fp8_kernel.py:710-795
 * (device work: same file :453-707).
 */
int gdnr_prep_ring(const gdnr_tensor* mixed_qkv, const gdnr_tensor* a, const gdnr_tensor* b,
                   const gdnr_tensor* a_log, const gdnr_tensor* dt_bias,
                   const gdnr_tensor* pos, const gdnr_tensor* q_out,
                   const gdnr_tensor* k_ring, const gdnr_tensor* v_ring,
                   const gdnr_tensor* g_ring, const gdnr_tensor* beta_ring,
                   int32_t fused, void* stream);

/*
 * The whole full-contract decode step in ONE launch: gdnr_prep_ring followed
 * by gdnr_replay_fp8 on the same buffers, with results identical to that
 * pair (the freshly appended token is taken from registers, rounded to the
 * ring dtype exactly as the ring stores it).
 * Composes prep_step + gdn_replay_fp8 as sequenced by
 * prototype/bench_gdn_full_contract.py:138-154,246-297.
 */
int gdnr_prep_replay_fp8(const gdnr_tensor* mixed_qkv, const gdnr_tensor* a,
                         const gdnr_tensor* b, const gdnr_tensor* a_log,
                         const gdnr_tensor* dt_bias, const gdnr_tensor* pos,
                         const gdnr_tensor* checkpoint, const gdnr_tensor* checkpoint_scale,
                         const gdnr_tensor* q_out, const gdnr_tensor* k_ring,
                         const gdnr_tensor* v_ring, const gdnr_tensor* g_ring,
                         const gdnr_tensor* beta_ring, const gdnr_tensor* valid_len,
                         const gdnr_tensor* flush, const gdnr_tensor* out,
                         int32_t block_v, void* stream);

/*
 * gdnr_prep_replay_fp8 over a slot-indexed cache (vLLM's layout): sequence
 * b's checkpoint, scale and ring rows are those of slot state_indices[b].
 * checkpoint [S,HV,V,K], checkpoint_scale [S,HV,V/32], k_ring [S,L,H,K],
 * v_ring [S,L,HV,V], g_ring, beta_ring [S,L,HV] hold S >= 1 slots; slot 0 is
 * the null slot, which padded batch entries point at (their writes land
 * there and their outputs are meaningless). state_indices [B] i32 (clamped
 * on the device to [0, S), out of range -> 0); mixed_qkv, a, b, pos, q_out,
 * valid_len, flush and out are per batch entry as in gdnr_prep_replay_fp8.
 * Two batch entries must not name the same non-null slot. 1 <= L <= 64, as
 * for gdnr_prep_replay_fp8; caches of any size (slot bases and offsets are
 * formed in 64 bits).
 * No counterpart in the reference's kernels: the slot contract is the
 * production op's (initial_state = kv_cache[1] [slots,HV,V,K],
 * ssm_state_indices with slot 0 the null block), findings.md:35-45, applied
 * to the full-contract step of prototype/bench_gdn_full_contract.py:113-154.
 */
int gdnr_prep_replay_fp8_slots(const gdnr_tensor* mixed_qkv, const gdnr_tensor* a,
                               const gdnr_tensor* b, const gdnr_tensor* a_log,
                               const gdnr_tensor* dt_bias, const gdnr_tensor* pos,
                               const gdnr_tensor* state_indices,
                               const gdnr_tensor* checkpoint, const gdnr_tensor* checkpoint_scale,
                               const gdnr_tensor* q_out, const gdnr_tensor* k_ring,
                               const gdnr_tensor* v_ring, const gdnr_tensor* g_ring,
                               const gdnr_tensor* beta_ring, const gdnr_tensor* valid_len,
                               const gdnr_tensor* flush, const gdnr_tensor* out,
                               int32_t block_v, void* stream);

/*
 * vblock32 quantiser, bit-exact with the reference's
 *   s = amax/448 (f32) if amax > 0 else 1;  codes = e4m3fn(clamp(x/s, +-448));
 *   stored scale = fp16(s)
 * (the codes divide by the unrounded f32 s, as the reference does before it
 * stores the scale in fp16: ref:83-99).
 * state [B,HV,V,K] f32 -> payload [B,HV,V,K] fp8|u8, scale [B,HV,V/32] f16|f32.
 * saturated (optional, may be NULL) [B,HV,V/32] i32 receives the per-vblock
 * count of |x/scale| > 448.
 * Replaces quantize_checkpoint(state, "vblock", 32),
 * prototype/gdn_replay_fp8_reference.py:40-106 (vblock branch :71-87, :91-99).
 */
int gdnr_quantize_vblock32(const gdnr_tensor* state, const gdnr_tensor* payload,
                           const gdnr_tensor* scale, const gdnr_tensor* saturated,
                           void* stream);

/*
 * state = float(payload) * float(scale) per vblock32.
 * Replaces dequantize_checkpoint, prototype/gdn_replay_fp8_reference.py:109-134.
 */
int gdnr_dequantize_vblock32(const gdnr_tensor* payload, const gdnr_tensor* scale,
                             const gdnr_tensor* state, void* stream);

/*
 * The comparator of the ReplaySSM path: one gated delta-rule token per
 * sequence applied to a state held in full, read and written back in place:
 *   S <- exp(g) S;  r = S k;  S <- S + beta (v - r) k^T;  out = (S q) K^-1/2
 * (fp32 arithmetic; S stored back in its own dtype, round-to-nearest-even).
 * Shapes: state [B,HV,V,K] bf16|f16|f32 (16-byte aligned rows); q, k [B,H,K];
 *   v [B,HV,V]; g, beta [B,HV]; out [B,HV,V]. q, k, v, g, beta and out share
 *   one dtype (bf16|f16|f32). K == 128, V % 32 == 0, HV % H == 0, B <= 65535.
 * Replaces gdn_bf16_step, prototype/gdn_replayssm_fp8_kernel.py:408-450
 * (device work: _gdn_bf16_step_kernel, same file :245-341).
 */
int gdnr_bf16_step(const gdnr_tensor* state, const gdnr_tensor* q, const gdnr_tensor* k,
                   const gdnr_tensor* v, const gdnr_tensor* g, const gdnr_tensor* beta,
                   const gdnr_tensor* out, void* stream);

/*
 * The comparator in the production operator's contract (vLLM's packed GDN
 * decode): per batch entry b, q, k, v from the raw mixed_qkv row
 * [q heads | k heads | v heads], q and k L2-normalised (x / sqrt(sum x^2 +
 * 1e-6)), g = -exp(A_log) softplus_20(a + dt_bias), beta = sigmoid(b), all
 * in fp32; then the step of gdnr_bf16_step on the state of slot
 * state_indices[b] (slot 0 the null slot; clamped on the device).
 * Shapes: mixed_qkv [B, 2*H*K + HV*V]; a, b [B,HV] (f32 or the mixed_qkv
 * dtype); a_log, dt_bias [HV] f32; state [S,HV,V,K] bf16|f16|f32;
 * state_indices [B] i32; out [B,1,HV,V] in the mixed_qkv dtype; scale
 * multiplies o = S q (the production op's scale argument, head_k_dim^-1/2
 * in vLLM's call; it must be finite). A non-null slot may appear once per
 * batch (entries sharing one race, as in the production op); padding
 * entries all write the null slot, in an unspecified order.
 * The production op's contract is findings.md:35-45; the reference times its
 * full-contract step against it (prototype/bench_gdn_full_contract.py).
 */
int gdnr_bf16_step_packed(const gdnr_tensor* mixed_qkv, const gdnr_tensor* a, const gdnr_tensor* b,
                          const gdnr_tensor* a_log, const gdnr_tensor* dt_bias,
                          const gdnr_tensor* state, const gdnr_tensor* state_indices,
                          const gdnr_tensor* out, float scale, void* stream);

/*
 * Every checkpoint format of the reference's quantiser: granularity head,
 * row, tile or vblock (tile_size for the last two), codes fp8 e4m3fn
 * (payload fp8|u8) or int8 (payload i8, the "*_int8" formats). Per scale
 * group: s = amax/qmax (qmax 448 or 127), 1 when amax is not > 0; stored
 * scale fp16(s); codes = clamp(x / s) with the unrounded s for tile and
 * vblock and the fp16-rounded scale for head and row; fp8 rounds to nearest
 * even (NaN -> 0x7F|sign), int8 rounds half to even (NaN -> 0).
 * Shapes: state [B,HV,V,K] f32; payload [B,HV,V,K]; scale f16|f32 (f32 holds
 * the fp16 values) [B,HV,1,1] head, [B,HV,V,1] row, [B,HV,V/t,K/t] tile,
 * [B,HV,V/t] vblock; saturated (optional, may be NULL) i32 of the scale's
 * shape: per group, the count of |x/s| > qmax.
 * Replaces quantize_checkpoint(state, granularity, tile_size),
 * prototype/gdn_replay_fp8_reference.py:40-106.
 */
int gdnr_quantize_checkpoint(const gdnr_tensor* state, const gdnr_tensor* payload,
                             const gdnr_tensor* scale, const gdnr_tensor* saturated,
                             int32_t granularity, int32_t tile_size, void* stream);

/*
 * state = float(code) * float(scale) for any format of gdnr_quantize_checkpoint.
 * Replaces dequantize_checkpoint, prototype/gdn_replay_fp8_reference.py:109-134.
 */
int gdnr_dequantize_checkpoint(const gdnr_tensor* payload, const gdnr_tensor* scale,
                               const gdnr_tensor* state, int32_t granularity, int32_t tile_size,
                               void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GDNR_H */
