// gdnr_abi.cpp -- the extern "C" boundary of libgdnreplay.so (include/gdnr.h).
//
// Each entry point validates shapes, dtypes, strides and alignment on the
// host, fills a kernel argument block and enqueues the kernels on the
// caller's stream. Nothing here allocates device memory or synchronises.
// The reference wrappers validate nothing (prototype/gdn_replayssm_fp8_kernel.py
// :344-405, :710-795, :1129-1235); misuse there corrupts memory silently,
// here it is an error code plus a message.
#include <stdarg.h>
#include <stdio.h>

#include <initializer_list>
#include <string>

#include "gdnr.h"
#include "gdnr_internal.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

#define GDNR_TRY(expr)          \
  do {                          \
    const int rc_ = (expr);     \
    if (rc_ != GDNR_OK) return rc_; \
  } while (0)

int elem_size(int dt) {
  switch (dt) {
    case GDNR_DTYPE_BF16:
    case GDNR_DTYPE_F16: return 2;
    case GDNR_DTYPE_F32:
    case GDNR_DTYPE_I32: return 4;
    case GDNR_DTYPE_I64: return 8;
    case GDNR_DTYPE_FP8E4M3FN:
    case GDNR_DTYPE_U8:
    case GDNR_DTYPE_I8:
    case GDNR_DTYPE_BOOL: return 1;
    default: return 0;
  }
}

const char* dtype_name(int dt) {
  switch (dt) {
    case GDNR_DTYPE_BF16: return "bf16";
    case GDNR_DTYPE_F16: return "f16";
    case GDNR_DTYPE_F32: return "f32";
    case GDNR_DTYPE_FP8E4M3FN: return "fp8e4m3fn";
    case GDNR_DTYPE_U8: return "u8";
    case GDNR_DTYPE_I8: return "i8";
    case GDNR_DTYPE_I32: return "i32";
    case GDNR_DTYPE_I64: return "i64";
    case GDNR_DTYPE_BOOL: return "bool";
    default: return "?";
  }
}

int check_desc(const gdnr_tensor* t, const char* name, int ndim) {
  if (!t) return fail(GDNR_ERR_INVALID_ARGUMENT, "%s: null tensor descriptor", name);
  if (t->ndim != ndim) return fail(GDNR_ERR_INVALID_ARGUMENT, "%s: expected %d dims, got %d", name, ndim, t->ndim);
  if (elem_size(t->dtype) == 0) return fail(GDNR_ERR_INVALID_ARGUMENT, "%s: unknown dtype code %d", name, t->dtype);
  int64_t numel = 1;
  for (int d = 0; d < ndim; ++d) {
    if (t->shape[d] < 0) return fail(GDNR_ERR_INVALID_ARGUMENT, "%s: negative extent in dim %d", name, d);
    if (t->strides[d] < 0) return fail(GDNR_ERR_INVALID_ARGUMENT, "%s: negative stride in dim %d", name, d);
    numel *= t->shape[d];
  }
  if (numel > 0 && t->data == nullptr) return fail(GDNR_ERR_INVALID_ARGUMENT, "%s: null data pointer", name);
  return GDNR_OK;
}

int check_dtype(const gdnr_tensor* t, const char* name, std::initializer_list<int> allowed) {
  for (int d : allowed)
    if (t->dtype == d) return GDNR_OK;
  std::string list;
  for (int d : allowed) {
    if (!list.empty()) list += "|";
    list += dtype_name(d);
  }
  return fail(GDNR_ERR_INVALID_ARGUMENT, "%s: dtype %s not accepted (expected %s)", name, dtype_name(t->dtype),
              list.c_str());
}

int check_shape(const gdnr_tensor* t, const char* name, std::initializer_list<int64_t> shape) {
  int d = 0;
  for (int64_t s : shape) {
    if (t->shape[d] != s)
      return fail(GDNR_ERR_INVALID_ARGUMENT, "%s: dim %d is %lld, expected %lld", name, d, (long long)t->shape[d],
                  (long long)s);
    ++d;
  }
  return GDNR_OK;
}

int check_inner_unit(const gdnr_tensor* t, const char* name) {
  const int last = t->ndim - 1;
  if (t->shape[last] > 1 && t->strides[last] != 1)
    return fail(GDNR_ERR_INVALID_ARGUMENT, "%s: innermost stride must be 1 (got %lld)", name,
                (long long)t->strides[last]);
  return GDNR_OK;
}

// base pointer and every outer stride (in bytes) must be multiples of `align`
int check_align(const gdnr_tensor* t, const char* name, int align) {
  const int es = elem_size(t->dtype);
  if (((uintptr_t)t->data) % align)
    return fail(GDNR_ERR_INVALID_ARGUMENT, "%s: data pointer must be %d-byte aligned", name, align);
  for (int d = 0; d + 1 < t->ndim; ++d)
    if (t->shape[d] > 1 && (t->strides[d] * es) % align)
      return fail(GDNR_ERR_INVALID_ARGUMENT, "%s: stride of dim %d (%lld bytes) must be a multiple of %d", name, d,
                  (long long)(t->strides[d] * es), align);
  return GDNR_OK;
}

bool is_act(int dt) { return dt == GDNR_DTYPE_BF16 || dt == GDNR_DTYPE_F16 || dt == GDNR_DTYPE_F32; }

int check_scalar_vec(const gdnr_tensor* t, const char* name, int ndim, std::initializer_list<int64_t> shape) {
  GDNR_TRY(check_desc(t, name, ndim));
  GDNR_TRY(check_dtype(t, name, {GDNR_DTYPE_BF16, GDNR_DTYPE_F16, GDNR_DTYPE_F32}));
  return check_shape(t, name, shape);
}

// valid_len / pos: int32; flush: one byte (bool | u8) per sequence
int check_index_vec(const gdnr_tensor* t, const char* name, int64_t batch, bool is_flag) {
  GDNR_TRY(check_desc(t, name, 1));
  if (is_flag)
    GDNR_TRY(check_dtype(t, name, {GDNR_DTYPE_BOOL, GDNR_DTYPE_U8}));
  else
    GDNR_TRY(check_dtype(t, name, {GDNR_DTYPE_I32}));
  return check_shape(t, name, {batch});
}

struct Geometry {
  int64_t B, L, H, K, HV, V;
  int act;
};

// q [B,H,K] (optional), k_cache [B,L,H,K], v_cache [B,L,HV,V], g/beta [B,L,HV]
int check_ring(const gdnr_tensor* k_cache, const gdnr_tensor* v_cache, const gdnr_tensor* g_cache,
               const gdnr_tensor* beta_cache, Geometry* geo, int ring_align) {
  GDNR_TRY(check_desc(k_cache, "k_cache", 4));
  GDNR_TRY(check_desc(v_cache, "v_cache", 4));
  if (!is_act(k_cache->dtype))
    return fail(GDNR_ERR_INVALID_ARGUMENT, "k_cache: dtype %s not accepted (expected bf16|f16|f32)",
                dtype_name(k_cache->dtype));
  geo->act = k_cache->dtype;
  geo->B = k_cache->shape[0];
  geo->L = k_cache->shape[1];
  geo->H = k_cache->shape[2];
  geo->K = k_cache->shape[3];
  geo->HV = v_cache->shape[2];
  geo->V = v_cache->shape[3];
  if (v_cache->dtype != geo->act)
    return fail(GDNR_ERR_INVALID_ARGUMENT, "v_cache: dtype %s differs from k_cache's %s", dtype_name(v_cache->dtype),
                dtype_name(geo->act));
  GDNR_TRY(check_shape(v_cache, "v_cache", {geo->B, geo->L}));
  GDNR_TRY(check_scalar_vec(g_cache, "g_cache", 3, {geo->B, geo->L, geo->HV}));
  GDNR_TRY(check_scalar_vec(beta_cache, "beta_cache", 3, {geo->B, geo->L, geo->HV}));
  if (g_cache->dtype != geo->act || beta_cache->dtype != geo->act)
    return fail(GDNR_ERR_UNSUPPORTED, "g_cache/beta_cache dtypes (%s/%s) must equal the k/v ring dtype %s",
                dtype_name(g_cache->dtype), dtype_name(beta_cache->dtype), dtype_name(geo->act));
  GDNR_TRY(check_inner_unit(k_cache, "k_cache"));
  GDNR_TRY(check_inner_unit(v_cache, "v_cache"));
  GDNR_TRY(check_align(k_cache, "k_cache", ring_align));
  GDNR_TRY(check_align(v_cache, "v_cache", ring_align));
  if (geo->K != gdnr::kKeyDim)
    return fail(GDNR_ERR_UNSUPPORTED, "key head dim K=%lld: only K=%d is built", (long long)geo->K, gdnr::kKeyDim);
  if (geo->H <= 0 || geo->HV <= 0 || geo->HV % geo->H)
    return fail(GDNR_ERR_INVALID_ARGUMENT, "value heads (%lld) must be a positive multiple of key heads (%lld)",
                (long long)geo->HV, (long long)geo->H);
  if (geo->V <= 0 || geo->V % gdnr::kVBlock)
    return fail(GDNR_ERR_INVALID_ARGUMENT, "value head dim V=%lld must be a positive multiple of %d",
                (long long)geo->V, gdnr::kVBlock);
  if (geo->L < 1 || geo->L > gdnr::kMaxRing)
    return fail(GDNR_ERR_UNSUPPORTED, "ring length %lld outside [1, %d]", (long long)geo->L, gdnr::kMaxRing);
  return GDNR_OK;
}

int largest_group(int64_t G) {
  for (int gw = gdnr::kMaxWavesPerWG; gw > 1; --gw)
    if (G % gw == 0) return gw;
  return 1;
}

int32_t align16(int64_t x) { return (int32_t)((x + 15) / 16 * 16); }

// LDS layout of the replay workgroup; returns total bytes.
int32_t layout_lds(gdnr::ReplayArgs* a, int es, bool stage_k, bool stage_v) {
  const int64_t K = gdnr::kKeyDim;
  int64_t off = 0;
  a->lds_q = 0;
  off = align16(K * es);
  a->lds_k = (int32_t)off;
  if (stage_k) off = align16(off + (int64_t)a->L * K * es);
  a->lds_v = (int32_t)off;
  if (stage_v) off = align16(off + (int64_t)a->L * a->gw * a->block_v * es);
  a->lds_gb = (int32_t)off;
  off = align16(off + (int64_t)a->L * a->gw * 8);
  a->lds_t = (int32_t)off;
  off = align16(off + (int64_t)a->gw * K * 4);
  a->lds_bytes = (int32_t)off;
  return a->lds_bytes;
}

constexpr int32_t kMaxLds = 64 * 1024;

// The replay kernel (rings longer than kStepRing) runs one wave per value
// head and V-tile, so the tile height sets how many waves the launch has.
// Starting from the requested block_v, halve it while the launch would have
// fewer than two waves per compute unit (results do not depend on the tile:
// every row's replay, rebuild and vblock requantisation is the same). At
// B=8, HV=32, L=64: 10.47 us per step with 64-row tiles, 12.21 with 128.
void fit_replay_tile(gdnr::ReplayArgs* a) {
  const int64_t cus = gdnr::device_cus();
  while (a->block_v > 32 && a->V % (a->block_v / 2) == 0 &&
         (int64_t)a->B * a->HV * (a->V / a->block_v) < 2 * cus)
    a->block_v /= 2;
  a->n_vt = a->V / a->block_v;
}

// pick the value heads per workgroup so the LDS layout fits
int fit_lds(gdnr::ReplayArgs* a, int es, bool stage_k, bool stage_v) {
  for (int gw = largest_group(a->G); gw >= 1; --gw) {
    if (a->G % gw) continue;
    a->gw = gw;
    if (layout_lds(a, es, stage_k, stage_v) <= kMaxLds) return GDNR_OK;
  }
  return fail(GDNR_ERR_UNSUPPORTED, "ring length %d with block_v=%d needs %d bytes of LDS (> %d); use a smaller block_v",
              a->L, a->block_v, a->lds_bytes, kMaxLds);
}

// LDS plan of the step kernel (gdnr_step.hip, L <= kStepRing) for the
// current gw / block_v: q | new k | k ring | flags | c | T0 | slot Gram per head |
// v rows | flush: R | factors | K^T tiles | lam_all | per-head scratch (w partials of a
// replay, decays and M of the flush factors).
int32_t layout_step(gdnr::ReplayArgs* a, int es) {
  const int64_t K = gdnr::kKeyDim, LP = gdnr::kStepRing;
  a->rpw = a->block_v;  // one streamer wave per head owns the head's block_v rows
  a->sw = 2 * a->gw;     // plus one coefficient-chain wave per head
  int64_t off = 0;
  auto region = [&off](int32_t* field, int64_t bytes) {
    *field = (int32_t)off;
    off = align16(off + bytes);
  };
  region(&a->lds_q, K * es);
  region(&a->lds_knew, K * es);
  region(&a->lds_k, (int64_t)a->L * K * es);
  // per head: 3 flags, the new (gamma, beta), the flush amax exchange words
  region(&a->lds_flag, (int64_t)a->gw * 4 * (5 + 2 * gdnr::kMaxVBlocks));
  region(&a->lds_c, (int64_t)a->gw * a->block_v * 4);  // c_t per head (replay)
  region(&a->lds_t, (int64_t)a->gw * K * 4);
  region(&a->lds_g, (int64_t)a->gw * (LP + 2) * 20 * 4);  // [slots, q, new k]^2, row stride 20
  region(&a->lds_v, (int64_t)a->gw * LP * a->rpw * es);
  region(&a->lds_r, (int64_t)a->gw * LP * LP * 4);
  region(&a->lds_fac, (int64_t)a->gw * LP * 16);
  region(&a->lds_kt, K * LP * es);
  region(&a->lds_lam, (int64_t)a->gw * 4);
  region(&a->lds_u, (int64_t)a->gw * LP * 192);  // per-head scratch
  a->lds_bytes = (int32_t)off;
  return a->lds_bytes;
}

// value heads per workgroup and V-tile height for the step kernel: the
// largest that fit in LDS with at most 8 waves, starting from the requested
// block_v (results do not depend on either).
int fit_step(gdnr::ReplayArgs* a, int es) {
  const int32_t requested = a->block_v;
  for (int bv = requested; bv >= 32; bv /= 2) {
    if (a->V % bv) continue;
    for (int gw = largest_group(a->G); gw >= 1; --gw) {
      if (a->G % gw) continue;
      a->gw = gw;
      a->block_v = bv;
      a->n_vt = a->V / bv;
      if (layout_step(a, es) <= gdnr::kMaxStepLds && a->sw <= 8) return GDNR_OK;
    }
  }
  return fail(GDNR_ERR_UNSUPPORTED, "no step-kernel tiling fits (V=%d, G=%d)", a->V, a->G);
}

// The step kernel moves v-ring rows (and the new token's v) in pairs of
// elements and forms every address as a 32-bit byte offset from a tensor's
// base pointer: it takes tensors whose byte extent (largest reachable offset)
// is below 2^31.
bool step_offsets_fit(const gdnr::ReplayArgs& a, int es) {
  const bool pairs = a.v_b % 2 == 0 && a.v_t % 2 == 0 && a.v_h % 2 == 0 && (a.mixed == nullptr || a.mx_b % 2 == 0);
  if (!pairs) return false;
  const int64_t lim = (int64_t)1 << 31;
  const int64_t B = a.B, L = a.L, HV = a.HV, H = a.H, V = a.V, K = gdnr::kKeyDim;
  const int64_t S = a.slot ? a.n_slots : B;  // rows of the checkpoint, scale and rings
  auto fits = [lim](int64_t extent_bytes) { return extent_bytes >= 0 && extent_bytes < lim; };
  bool ok = fits(((S - 1) * a.ck_b + (HV - 1) * a.ck_h + (V - 1) * a.ck_v + K)) &&
            fits(2 * ((S - 1) * a.sc_b + (HV - 1) * a.sc_h + (V / gdnr::kVBlock - 1) * a.sc_v + 1)) &&
            fits(es * ((S - 1) * a.k_b + (L - 1) * a.k_t + (H - 1) * a.k_h + K)) &&
            fits(es * ((S - 1) * a.v_b + (L - 1) * a.v_t + (HV - 1) * a.v_h + V)) &&
            fits(es * ((S - 1) * a.g_b + (L - 1) * a.g_t + (HV - 1) * a.g_h + 1)) &&
            fits(es * ((S - 1) * a.be_b + (L - 1) * a.be_t + (HV - 1) * a.be_h + 1)) &&
            (!a.slot || fits(4 * ((B - 1) * a.sl_s + 1))) &&
            fits(es * ((B - 1) * a.o_b + (HV - 1) * a.o_h + V)) && fits(4 * ((B - 1) * a.vl_s + 1)) &&
            fits((B - 1) * a.fl_s + 4);
  if (a.mixed) {
    ok = ok && fits(es * ((B - 1) * a.mx_b + 2 * H * K + HV * V)) && fits(4 * ((B - 1) * a.pos_s + 1)) &&
         fits(es * ((B - 1) * a.qo_b + (H - 1) * a.qo_h + K)) && fits(4 * ((B - 1) * a.a_b + (HV - 1) * a.a_h + 1)) &&
         fits(4 * ((B - 1) * a.bg_b + (HV - 1) * a.bg_h + 1)) && fits(4 * ((HV - 1) * a.al_s + 1)) &&
         fits(4 * ((HV - 1) * a.db_s + 1));
  } else {
    ok = ok && fits(es * ((B - 1) * a.q_b + (H - 1) * a.q_h + K));
  }
  return ok;
}

// The decode kernel forms each sequence's (slot's) base address in 64 bits
// and every offset inside one sequence, or inside the per-batch tensors, in
// 32 bits: it takes checkpoints and rings of any total size whose sequence
// strides fit 32 bits and whose per-sequence extent is below 2^31 bytes.
bool decode_offsets_fit(const gdnr::ReplayArgs& a, int es) {
  const int64_t lim = (int64_t)1 << 31, ulim = (int64_t)1 << 32;
  const int64_t B = a.B, L = a.L, HV = a.HV, H = a.H, V = a.V, K = gdnr::kKeyDim;
  auto fits = [lim](int64_t extent_bytes) { return extent_bytes >= 0 && extent_bytes < lim; };
  auto stride_fits = [ulim](int64_t stride_bytes) { return stride_bytes >= 0 && stride_bytes < ulim; };
  bool ok = stride_fits(a.ck_b) && stride_fits(2 * a.sc_b) && stride_fits(es * a.k_b) && stride_fits(es * a.v_b) &&
            stride_fits(es * a.g_b) && stride_fits(es * a.be_b) &&
            fits((HV - 1) * a.ck_h + (V - 1) * a.ck_v + K) &&
            fits(2 * ((HV - 1) * a.sc_h + (V / gdnr::kVBlock - 1) * a.sc_v + 1)) &&
            fits(es * ((L - 1) * a.k_t + (H - 1) * a.k_h + K)) && fits(es * ((L - 1) * a.v_t + (HV - 1) * a.v_h + V)) &&
            fits(es * ((L - 1) * a.g_t + (HV - 1) * a.g_h + 1)) && fits(es * ((L - 1) * a.be_t + (HV - 1) * a.be_h + 1)) &&
            (!a.slot || fits(4 * ((B - 1) * a.sl_s + 1))) &&
            fits(es * ((B - 1) * a.o_b + (HV - 1) * a.o_h + V)) && fits(4 * ((B - 1) * a.vl_s + 1)) &&
            fits((B - 1) * a.fl_s + 4);
  if (a.mixed) {
    ok = ok && fits(es * ((B - 1) * a.mx_b + 2 * H * K + HV * V)) && fits(4 * ((B - 1) * a.pos_s + 1)) &&
         fits(es * ((B - 1) * a.qo_b + (H - 1) * a.qo_h + K)) && fits(4 * ((B - 1) * a.a_b + (HV - 1) * a.a_h + 1)) &&
         fits(4 * ((B - 1) * a.bg_b + (HV - 1) * a.bg_h + 1)) && fits(4 * ((HV - 1) * a.al_s + 1)) &&
         fits(4 * ((HV - 1) * a.db_s + 1));
  } else {
    ok = ok && fits(es * ((B - 1) * a.q_b + (H - 1) * a.q_h + K));
  }
  return ok;
}

// StepArgs from a validated, fitted ReplayArgs (element strides -> byte strides).
gdnr::StepArgs make_step_args(const gdnr::ReplayArgs& r, int es, int gate_es) {
  gdnr::StepArgs s = {};
  s.ckpt = r.ckpt;
  s.scale = (uint8_t*)r.scale;
  s.q = (const uint8_t*)r.q;
  s.k = (uint8_t*)r.k;
  s.v = (uint8_t*)r.v;
  s.g = (uint8_t*)r.g;
  s.beta = (uint8_t*)r.beta;
  s.out = (uint8_t*)r.out;
  s.valid_len = (const uint8_t*)r.valid_len;
  s.flush = r.flush;
  s.pos = (const uint8_t*)r.pos;
  s.mixed = (const uint8_t*)r.mixed;
  s.a = (const uint8_t*)r.a;
  s.bgate = (const uint8_t*)r.bgate;
  s.a_log = (const uint8_t*)r.a_log;
  s.dt_bias = (const uint8_t*)r.dt_bias;
  s.q_out = (uint8_t*)r.q_out;
  auto u32 = [](int64_t x) { return (uint32_t)x; };
  s.ck_b = u32(r.ck_b), s.ck_h = u32(r.ck_h), s.ck_v = u32(r.ck_v);
  s.sc_b = u32(2 * r.sc_b), s.sc_h = u32(2 * r.sc_h), s.sc_v = u32(2 * r.sc_v);
  s.q_b = u32(es * r.q_b), s.q_h = u32(es * r.q_h);
  s.k_b = u32(es * r.k_b), s.k_t = u32(es * r.k_t), s.k_h = u32(es * r.k_h);
  s.v_b = u32(es * r.v_b), s.v_t = u32(es * r.v_t), s.v_h = u32(es * r.v_h);
  s.g_b = u32(es * r.g_b), s.g_t = u32(es * r.g_t), s.g_h = u32(es * r.g_h);
  s.be_b = u32(es * r.be_b), s.be_t = u32(es * r.be_t), s.be_h = u32(es * r.be_h);
  s.vl_s = u32(4 * r.vl_s), s.fl_s = u32(r.fl_s), s.pos_s = u32(4 * r.pos_s);
  s.o_b = u32(es * r.o_b), s.o_h = u32(es * r.o_h), s.mx_b = u32(es * r.mx_b);
  s.a_b = u32(gate_es * r.a_b), s.a_h = u32(gate_es * r.a_h), s.bg_b = u32(gate_es * r.bg_b),
  s.bg_h = u32(gate_es * r.bg_h);
  s.al_s = u32(4 * r.al_s), s.db_s = u32(4 * r.db_s);
  s.qo_b = u32(es * r.qo_b), s.qo_h = u32(es * r.qo_h);
  s.B = r.B, s.H = r.H, s.G = r.G, s.V = r.V, s.L = r.L, s.gw = r.gw, s.block_v = r.block_v, s.n_vt = r.n_vt;
  s.sw = r.sw, s.rpw = r.rpw, s.units = r.units, s.nwh = r.nwh, s.seq_major = r.seq_major;
  s.out_scale = r.out_scale;
  s.lds_q = r.lds_q, s.lds_knew = r.lds_knew, s.lds_k = r.lds_k, s.lds_flag = r.lds_flag, s.lds_c = r.lds_c;
  s.lds_t = r.lds_t, s.lds_g = r.lds_g, s.lds_v = r.lds_v, s.lds_r = r.lds_r, s.lds_fac = r.lds_fac;
  s.lds_kt = r.lds_kt, s.lds_lam = r.lds_lam, s.lds_u = r.lds_u, s.lds_bytes = r.lds_bytes;
  s.slot = (const uint8_t*)r.slot, s.sl_s = u32(4 * r.sl_s), s.n_slots = r.n_slots;
  return s;
}

int check_checkpoint(const gdnr_tensor* checkpoint, const gdnr_tensor* scale, const Geometry& g) {
  GDNR_TRY(check_desc(checkpoint, "checkpoint", 4));
  GDNR_TRY(check_dtype(checkpoint, "checkpoint", {GDNR_DTYPE_FP8E4M3FN, GDNR_DTYPE_U8}));
  GDNR_TRY(check_shape(checkpoint, "checkpoint", {g.B, g.HV, g.V, g.K}));
  GDNR_TRY(check_inner_unit(checkpoint, "checkpoint"));
  GDNR_TRY(check_align(checkpoint, "checkpoint", 16));
  GDNR_TRY(check_desc(scale, "checkpoint_scale", 3));
  GDNR_TRY(check_dtype(scale, "checkpoint_scale", {GDNR_DTYPE_F16}));
  return check_shape(scale, "checkpoint_scale", {g.B, g.HV, g.V / gdnr::kVBlock});
}

int check_act_tensor(const gdnr_tensor* t, const char* name, int ndim, std::initializer_list<int64_t> shape, int act,
                     int align) {
  GDNR_TRY(check_desc(t, name, ndim));
  if (t->dtype != act)
    return fail(GDNR_ERR_INVALID_ARGUMENT, "%s: dtype %s differs from the ring dtype %s", name, dtype_name(t->dtype),
                dtype_name(act));
  GDNR_TRY(check_shape(t, name, shape));
  GDNR_TRY(check_inner_unit(t, name));
  return check_align(t, name, align);
}

int check_block_v(int32_t block_v, const Geometry& g) {
  if (block_v != 32 && block_v != 64 && block_v != 128)
    return fail(GDNR_ERR_INVALID_ARGUMENT, "block_v=%d: expected 32, 64 or 128", block_v);
  if (g.V % block_v) return fail(GDNR_ERR_INVALID_ARGUMENT, "block_v=%d does not divide V=%lld", block_v, (long long)g.V);
  return GDNR_OK;
}

void fill_common(gdnr::ReplayArgs* a, const Geometry& g, int32_t block_v) {
  a->B = (int32_t)g.B;
  a->H = (int32_t)g.H;
  a->HV = (int32_t)g.HV;
  a->G = (int32_t)(g.HV / g.H);
  a->V = (int32_t)g.V;
  a->L = (int32_t)g.L;
  a->block_v = block_v;
  a->n_vt = (int32_t)(g.V / block_v);
  a->out_scale = 1.0f / __builtin_sqrtf((float)g.K);
}

void fill_ckpt(gdnr::ReplayArgs* a, const gdnr_tensor* c, const gdnr_tensor* s) {
  a->ckpt = (uint8_t*)c->data;
  a->ck_b = c->strides[0];
  a->ck_h = c->strides[1];
  a->ck_v = c->strides[2];
  a->scale = (uint16_t*)s->data;
  a->sc_b = s->strides[0];
  a->sc_h = s->strides[1];
  a->sc_v = s->strides[2];
}

void fill_ring(gdnr::ReplayArgs* a, const gdnr_tensor* k, const gdnr_tensor* v, const gdnr_tensor* g,
               const gdnr_tensor* be) {
  a->k = k->data;
  a->k_b = k->strides[0];
  a->k_t = k->strides[1];
  a->k_h = k->strides[2];
  a->v = v->data;
  a->v_b = v->strides[0];
  a->v_t = v->strides[1];
  a->v_h = v->strides[2];
  a->g = g->data;
  a->g_b = g->strides[0];
  a->g_t = g->strides[1];
  a->g_h = g->strides[2];
  a->beta = be->data;
  a->be_b = be->strides[0];
  a->be_t = be->strides[1];
  a->be_h = be->strides[2];
}

template <class T>
void fill_index(const gdnr_tensor* t, const T** p, int64_t* s) {
  *p = (const T*)t->data;
  *s = t->strides[0];
}

// The decode kernel (gdnr_decode.hip) takes 16-bit activations, rings of up
// to kStepRing tokens and V = 64, 128 or 256 (one wave of 64 or 128 rows per
// value head, four of 32 rows for V = 128 at small batches, two of 128 rows
// for V = 256); gw value heads per workgroup beside its chain wave. Rings
// of up to kDecodeChunks kStepRing tokens run as chunks of kStepRing on
// V = 64 or 128 (one value head per unit, waves of 32 or 64 rows). sw
// carries V / 64 to the launcher.
bool decode_eligible(const gdnr::ReplayArgs& a, int act) {
  if (act != GDNR_DTYPE_BF16 && act != GDNR_DTYPE_F16) return false;
  if (a.L <= gdnr::kStepRing) return a.V == 64 || a.V == 128 || a.V == 256;
  // (a ring of chunks: while its workgroups, two per compute unit, run in
  // one round; larger batches run faster on the long-ring kernel)
  return a.L <= gdnr::kDecodeChunks * gdnr::kStepRing && (a.V == 64 || a.V == 128) &&
         (int64_t)a.B * a.H * a.G <= 2 * (int64_t)gdnr::device_cus();
}
void fit_decode(gdnr::ReplayArgs* a) {
  const int32_t cus = gdnr::device_cus();
  if (a->L > gdnr::kStepRing) {
    // a ring of chunks: one value head per unit and workgroup. Waves of 32
    // rows (one vblock each) while the workgroups do not outnumber the
    // compute units; else waves of 64 rows, so that two workgroups share a
    // compute unit (with 32-row waves, 5 waves each, their chains wait on
    // the SIMDs: B=16, L=64 11.19 against 9.25 us per step, where B=8 takes
    // 6.71 against 6.98)
    a->gw = 1;
    const bool narrow = (int64_t)a->B * a->H * a->G <= cus;
    a->nwh = a->V / (narrow ? 32 : 64);
    a->sw = a->V / 64;
    a->units = 1;
    // (numbered sequence-fastest while narrow, as the one-chunk small-batch
    // plan below)
    a->seq_major = narrow ? 1 : 0;
    a->lds_bytes = gdnr::decode_lds_bytes(1, a->nwh, narrow ? 1 : 2, gdnr::kDecodeChunks);
    return;
  }
  a->nwh = a->V == 256 ? 2 : 1;  // row waves per value head
  a->gw = a->G % 2 == 0 ? 2 : 1;  // value heads per unit (at most 2; they share the unit's chain wave)
  // small batches: one value head per unit (twice the units), and for V = 128
  // four row waves of 32 rows per head while the units do not outnumber the
  // compute units: the launch spreads over the whole chip, and every wave's
  // share of the stream and of a flush (one vblock) is short. B=8, L=4:
  // 5.18 us per step against 5.72 with two waves of 64 rows; L=16 4.56
  // against 4.76; B=16, L=16 5.34 against 5.52.
  if (a->gw == 2 && (int64_t)a->B * a->H * (a->G / 2) < cus) a->gw = 1;
  if (a->V == 128 && (int64_t)a->B * a->H * (a->G / a->gw) <= cus) a->nwh = 4;
  // The small-batch plan numbers its workgroups sequence-fastest: the
  // dispatcher spreads consecutive workgroups over the XCDs, so each XCD then
  // holds all the head groups of its sequences, whose per-sequence rows
  // (metadata, mixed_qkv, gates) its L2 serves to every head (B=8, L=16:
  // 4.18 against 4.56 us per step; L=4 4.88 against 5.17; B=8, L=64 on the
  // chunked path 6.43 against 6.73; B=16, L=16 5.20 against 5.34). Larger
  // launches keep head-fastest numbering (B=64 unchanged, B=512 81.1
  // against 77.3 the other way).
  a->seq_major = a->nwh == 4 ? 1 : 0;
  a->sw = a->V / 64;
  // units per workgroup: as many as fit one CU (12 waves) while the grid
  // still covers every CU; the kernel takes a workgroup's units as SP
  // sequences x HP head groups (4 = 2 x 2, 2 = 2 x 1), which must divide B
  // and the head groups of a sequence
  const int32_t per_seq = a->H * (a->G / a->gw), waves = 1 + a->gw * a->nwh;
  a->units = 1;
  // Large launches (at least 16 units per compute unit) keep one unit per
  // workgroup: four small workgroups share a compute unit, and one's start
  // (its chain's ring round trip) overlaps the others' streams. At B=512,
  // L=8: 80.1 us per step against 86.3 with 4-unit workgroups (one per
  // compute unit, run one after another); at B=128 4 units win, 21.5 us
  // against 22.8.
  const bool large = (int64_t)a->B * per_seq >= 16 * (int64_t)cus;
  for (int32_t u : {4, 2}) {
    if (large) break;
    const int32_t hp = u == 4 ? 2 : 1, sp = u / hp;
    if (a->B % sp == 0 && per_seq % hp == 0 && u * waves <= 12 && (int64_t)a->B * per_seq / u >= cus) {
      a->units = u;
      break;
    }
  }
  // vblocks per row wave: V / 32 / nwh
  a->lds_bytes = gdnr::decode_lds_bytes(a->units, a->gw * a->nwh, a->V / 32 / a->nwh, 1);
}
int launch_decode(const gdnr::ReplayArgs& r, int act, bool fused, bool gate_f32, void* stream) {
  gdnr::StepArgs a = make_step_args(r, elem_size(act), gate_f32 ? 4 : elem_size(act));
  a.status = gdnr::status_word();
  a.wait_polls = gdnr::wait_polls();
  if (act == GDNR_DTYPE_BF16) return gdnr::launch_decode_bf16(a, fused, gate_f32, stream);
  return gdnr::launch_decode_f16(a, fused, gate_f32, stream);
}

int launch_replay(const gdnr::ReplayArgs& a, int act, int mode, bool gate_f32, void* stream) {
  if (act == GDNR_DTYPE_BF16) return gdnr::launch_replay_bf16(a, mode, gate_f32, stream);
  if (act == GDNR_DTYPE_F16) return gdnr::launch_replay_f16(a, mode, gate_f32, stream);
  return gdnr::launch_replay_f32(a, mode, gate_f32, stream);
}
int launch_step(const gdnr::ReplayArgs& r, int act, bool fused, bool gate_f32, void* stream) {
  gdnr::StepArgs a = make_step_args(r, elem_size(act), gate_f32 ? 4 : elem_size(act));
  a.status = gdnr::status_word();
  a.wait_polls = gdnr::wait_polls();
  if (act == GDNR_DTYPE_BF16) return gdnr::launch_step_bf16(a, fused, gate_f32, stream);
  if (act == GDNR_DTYPE_F16) return gdnr::launch_step_f16(a, fused, gate_f32, stream);
  return gdnr::launch_step_f32(a, fused, gate_f32, stream);
}
int launch_precompute(const gdnr::ReplayArgs& a, int act, void* stream) {
  if (act == GDNR_DTYPE_BF16) return gdnr::launch_precompute_bf16(a, stream);
  if (act == GDNR_DTYPE_F16) return gdnr::launch_precompute_f16(a, stream);
  return gdnr::launch_precompute_f32(a, stream);
}
int launch_prep(const gdnr::PrepArgs& a, int act, bool gate_f32, void* stream) {
  if (act == GDNR_DTYPE_BF16) return gdnr::launch_prep_bf16(a, gate_f32, stream);
  if (act == GDNR_DTYPE_F16) return gdnr::launch_prep_f16(a, gate_f32, stream);
  return gdnr::launch_prep_f32(a, gate_f32, stream);
}

int hip_status(int rc) {
  if (rc == 0) return GDNR_OK;
  return fail(GDNR_ERR_HIP, "kernel launch failed: %s", gdnr::hip_error_string(rc));
}

int check_prep_inputs(const gdnr_tensor* mixed_qkv, const gdnr_tensor* a, const gdnr_tensor* b,
                      const gdnr_tensor* a_log, const gdnr_tensor* dt_bias, const gdnr_tensor* pos, const Geometry& g) {
  GDNR_TRY(check_desc(mixed_qkv, "mixed_qkv", 2));
  if (mixed_qkv->dtype != g.act)
    return fail(GDNR_ERR_INVALID_ARGUMENT, "mixed_qkv: dtype %s differs from the ring dtype %s",
                dtype_name(mixed_qkv->dtype), dtype_name(g.act));
  // rows of at least 2 H K + HV V elements: the preparation reads the first
  // 2 H K + HV V of each row (q heads | k heads | v heads, kernel:500-550) and
  // steps between rows by the row stride, so a wider row buffer is accepted
  // as the reference accepts it
  const int64_t width = 2 * g.H * g.K + g.HV * g.V;
  if (mixed_qkv->shape[0] != g.B || mixed_qkv->shape[1] < width)
    return fail(GDNR_ERR_INVALID_ARGUMENT,
                "mixed_qkv: shape [%lld, %lld], expected [%lld, >= %lld] (2 H K + HV V)",
                (long long)mixed_qkv->shape[0], (long long)mixed_qkv->shape[1], (long long)g.B, (long long)width);
  GDNR_TRY(check_inner_unit(mixed_qkv, "mixed_qkv"));
  GDNR_TRY(check_align(mixed_qkv, "mixed_qkv", 2 * elem_size(g.act)));
  GDNR_TRY(check_scalar_vec(a, "a", 2, {g.B, g.HV}));
  GDNR_TRY(check_scalar_vec(b, "b", 2, {g.B, g.HV}));
  if (a->dtype != b->dtype || (a->dtype != g.act && a->dtype != GDNR_DTYPE_F32))
    return fail(GDNR_ERR_UNSUPPORTED, "a/b dtypes (%s/%s) must match each other and be f32 or the ring dtype %s",
                dtype_name(a->dtype), dtype_name(b->dtype), dtype_name(g.act));
  GDNR_TRY(check_desc(a_log, "a_log", 1));
  GDNR_TRY(check_dtype(a_log, "a_log", {GDNR_DTYPE_F32}));
  GDNR_TRY(check_shape(a_log, "a_log", {g.HV}));
  GDNR_TRY(check_desc(dt_bias, "dt_bias", 1));
  GDNR_TRY(check_dtype(dt_bias, "dt_bias", {GDNR_DTYPE_F32}));
  GDNR_TRY(check_shape(dt_bias, "dt_bias", {g.HV}));
  return check_index_vec(pos, "pos", g.B, false);
}

void fill_prep_inputs(gdnr::ReplayArgs* r, const gdnr_tensor* mixed_qkv, const gdnr_tensor* a, const gdnr_tensor* b,
                      const gdnr_tensor* a_log, const gdnr_tensor* dt_bias, const gdnr_tensor* pos,
                      const gdnr_tensor* q_out) {
  r->mixed = mixed_qkv->data;
  r->mx_b = mixed_qkv->strides[0];
  r->a = a->data;
  r->a_b = a->strides[0];
  r->a_h = a->strides[1];
  r->bgate = b->data;
  r->bg_b = b->strides[0];
  r->bg_h = b->strides[1];
  r->a_log = (const float*)a_log->data;
  r->al_s = a_log->strides[0];
  r->dt_bias = (const float*)dt_bias->data;
  r->db_s = dt_bias->strides[0];
  fill_index(pos, &r->pos, &r->pos_s);
  r->q_out = q_out->data;
  r->qo_b = q_out->strides[0];
  r->qo_h = q_out->strides[1];
}

int check_quant(const gdnr_tensor* state, const gdnr_tensor* payload, const gdnr_tensor* scale, int64_t* B,
                int64_t* HV, int64_t* V) {
  GDNR_TRY(check_desc(state, "state", 4));
  GDNR_TRY(check_dtype(state, "state", {GDNR_DTYPE_F32}));
  *B = state->shape[0];
  *HV = state->shape[1];
  *V = state->shape[2];
  if (state->shape[3] != gdnr::kKeyDim)
    return fail(GDNR_ERR_UNSUPPORTED, "key head dim K=%lld: only K=%d is built", (long long)state->shape[3],
                gdnr::kKeyDim);
  if (*V % gdnr::kVBlock)
    return fail(GDNR_ERR_INVALID_ARGUMENT, "value head dim V=%lld must be a multiple of %d", (long long)*V,
                gdnr::kVBlock);
  GDNR_TRY(check_inner_unit(state, "state"));
  GDNR_TRY(check_align(state, "state", 16));
  GDNR_TRY(check_desc(payload, "payload", 4));
  GDNR_TRY(check_dtype(payload, "payload", {GDNR_DTYPE_FP8E4M3FN, GDNR_DTYPE_U8}));
  GDNR_TRY(check_shape(payload, "payload", {*B, *HV, *V, (int64_t)gdnr::kKeyDim}));
  GDNR_TRY(check_inner_unit(payload, "payload"));
  GDNR_TRY(check_align(payload, "payload", 16));
  GDNR_TRY(check_desc(scale, "scale", 3));
  GDNR_TRY(check_dtype(scale, "scale", {GDNR_DTYPE_F16, GDNR_DTYPE_F32}));
  return check_shape(scale, "scale", {*B, *HV, *V / gdnr::kVBlock});
}

void fill_quant(gdnr::QuantArgs* q, const gdnr_tensor* state, const gdnr_tensor* payload, const gdnr_tensor* scale,
                int64_t B, int64_t HV, int64_t V) {
  q->state = (const float*)state->data;
  q->st_b = state->strides[0];
  q->st_h = state->strides[1];
  q->st_v = state->strides[2];
  q->codes = (uint8_t*)payload->data;
  q->ck_b = payload->strides[0];
  q->ck_h = payload->strides[1];
  q->ck_v = payload->strides[2];
  q->scale = scale->data;
  q->sc_b = scale->strides[0];
  q->sc_h = scale->strides[1];
  q->sc_v = scale->strides[2];
  q->scale_dt = scale->dtype;
  q->saturated = nullptr;
  q->B = (int32_t)B;
  q->HV = (int32_t)HV;
  q->V = (int32_t)V;
}

}  // namespace

extern "C" {

const char* gdnr_last_error(void) { return g_last_error.c_str(); }

int gdnr_abi_version(void) { return GDNR_ABI_VERSION; }

int gdnr_wait_timeouts(uint32_t* count, int32_t reset) {
  g_last_error.clear();
  if (!count) return fail(GDNR_ERR_INVALID_ARGUMENT, "count is NULL");
  const int rc = gdnr::read_status(count, reset != 0);
  if (rc) return fail(GDNR_ERR_HIP, "reading the wait status word failed: %s", gdnr::hip_error_string(rc));
  return GDNR_OK;
}

uint32_t gdnr_set_wait_polls(uint32_t polls) { return gdnr::set_wait_polls(polls); }

int gdnr_decode_plan(int32_t batch, int32_t heads, int32_t value_heads, int32_t value_dim, int32_t ring_len,
                     int32_t act_dtype, int32_t* plan) {
  g_last_error.clear();
  if (!plan) return fail(GDNR_ERR_INVALID_ARGUMENT, "plan is NULL");
  if (batch <= 0 || heads <= 0 || value_heads <= 0 || value_heads % heads != 0 || ring_len <= 0)
    return fail(GDNR_ERR_INVALID_ARGUMENT, "batch, heads, value_heads (a multiple of heads) and ring_len must be > 0");
  gdnr::ReplayArgs a = {};
  a.B = batch, a.H = heads, a.HV = value_heads, a.G = value_heads / heads, a.V = value_dim, a.L = ring_len;
  if (!decode_eligible(a, act_dtype))
    return fail(GDNR_ERR_UNSUPPORTED,
                "no decode-kernel plan: 16-bit activations, and L <= %d with V in {64, 128, 256} or L <= %d with "
                "V in {64, 128}",
                gdnr::kStepRing, gdnr::kDecodeChunks * gdnr::kStepRing);
  fit_decode(&a);
  plan[0] = a.V / a.nwh;
  plan[1] = a.nwh;
  plan[2] = a.gw;
  plan[3] = a.units;
  plan[4] = a.lds_bytes;
  return GDNR_OK;
}

int gdnr_replay_fp8(const gdnr_tensor* checkpoint, const gdnr_tensor* checkpoint_scale, const gdnr_tensor* q,
                    const gdnr_tensor* k_cache, const gdnr_tensor* v_cache, const gdnr_tensor* g_cache,
                    const gdnr_tensor* beta_cache, const gdnr_tensor* valid_len, const gdnr_tensor* flush,
                    const gdnr_tensor* out, int32_t block_v, void* stream) {
  g_last_error.clear();
  Geometry g;
  GDNR_TRY(check_ring(k_cache, v_cache, g_cache, beta_cache, &g, 16));
  GDNR_TRY(check_checkpoint(checkpoint, checkpoint_scale, g));
  GDNR_TRY(check_act_tensor(q, "q", 3, {g.B, g.H, g.K}, g.act, 16));
  GDNR_TRY(check_index_vec(valid_len, "valid_len", g.B, false));
  GDNR_TRY(check_index_vec(flush, "flush", g.B, true));
  GDNR_TRY(check_act_tensor(out, "out", 3, {g.B, g.HV, g.V}, g.act, 2));
  GDNR_TRY(check_block_v(block_v, g));
  if (g.B == 0) return GDNR_OK;
  gdnr::ReplayArgs a = {};
  fill_common(&a, g, block_v);
  fill_ckpt(&a, checkpoint, checkpoint_scale);
  fill_ring(&a, k_cache, v_cache, g_cache, beta_cache);
  a.q = q->data;
  a.q_b = q->strides[0];
  a.q_h = q->strides[1];
  fill_index(valid_len, &a.valid_len, &a.vl_s);
  fill_index(flush, &a.flush, &a.fl_s);
  a.out = out->data;
  a.o_b = out->strides[0];
  a.o_h = out->strides[1];
  if (decode_eligible(a, g.act) && decode_offsets_fit(a, elem_size(g.act))) {
    fit_decode(&a);
    return hip_status(launch_decode(a, g.act, false, false, stream));
  }
  if (a.L <= gdnr::kStepRing && step_offsets_fit(a, elem_size(g.act))) {
    GDNR_TRY(fit_step(&a, elem_size(g.act)));
    return hip_status(launch_step(a, g.act, false, false, stream));
  }
  fit_replay_tile(&a);
  GDNR_TRY(fit_lds(&a, elem_size(g.act), true, true));
  return hip_status(launch_replay(a, g.act, gdnr::kModeReplay, false, stream));
}

namespace {
// The two launches of the split replay (precompute, then apply) once the
// arguments are validated; tq [B,HV,K] and coef [B,HV,>=L] f32 with element
// strides.
int split_launch(const Geometry& g, const gdnr_tensor* checkpoint, const gdnr_tensor* checkpoint_scale,
                 const gdnr_tensor* q, const gdnr_tensor* k_cache, const gdnr_tensor* v_cache,
                 const gdnr_tensor* g_cache, const gdnr_tensor* beta_cache, const gdnr_tensor* valid_len,
                 float* tq, int64_t tq_b, int64_t tq_h, float* coef, int64_t co_b, int64_t co_h, int64_t co_t,
                 const gdnr_tensor* out, int32_t block_v, int32_t precompute_grouped, void* stream) {
  gdnr::ReplayArgs a = {};
  fill_common(&a, g, block_v);
  fill_ckpt(&a, checkpoint, checkpoint_scale);
  fill_ring(&a, k_cache, v_cache, g_cache, beta_cache);
  a.q = q->data;
  a.q_b = q->strides[0];
  a.q_h = q->strides[1];
  fill_index(valid_len, &a.valid_len, &a.vl_s);
  a.flush = nullptr;
  a.tq = tq;
  a.tq_b = tq_b;
  a.tq_h = tq_h;
  a.coef = coef;
  a.co_b = co_b;
  a.co_h = co_h;
  a.co_t = co_t;
  a.out = out->data;
  a.o_b = out->strides[0];
  a.o_h = out->strides[1];

  // precompute: one workgroup per key head (grouped) or per value head
  gdnr::ReplayArgs pre = a;
  pre.block_v = 32;
  pre.n_vt = 1;
  if (precompute_grouped) {
    GDNR_TRY(fit_lds(&pre, elem_size(g.act), true, false));
  } else {
    pre.gw = 1;
    layout_lds(&pre, elem_size(g.act), true, false);
  }
  GDNR_TRY(hip_status(launch_precompute(pre, g.act, stream)));
  GDNR_TRY(fit_lds(&a, elem_size(g.act), false, true));
  return hip_status(launch_replay(a, g.act, gdnr::kModeApply, false, stream));
}

// argument checks shared by the two split entry points (all but the buffers)
int check_split(const gdnr_tensor* checkpoint, const gdnr_tensor* checkpoint_scale, const gdnr_tensor* q,
                const gdnr_tensor* k_cache, const gdnr_tensor* v_cache, const gdnr_tensor* g_cache,
                const gdnr_tensor* beta_cache, const gdnr_tensor* valid_len, const gdnr_tensor* out,
                int32_t block_v, int32_t block_kc, Geometry* g) {
  GDNR_TRY(check_ring(k_cache, v_cache, g_cache, beta_cache, g, 16));
  GDNR_TRY(check_checkpoint(checkpoint, checkpoint_scale, *g));
  GDNR_TRY(check_act_tensor(q, "q", 3, {g->B, g->H, g->K}, g->act, 16));
  GDNR_TRY(check_index_vec(valid_len, "valid_len", g->B, false));
  GDNR_TRY(check_act_tensor(out, "out", 3, {g->B, g->HV, g->V}, g->act, 2));
  GDNR_TRY(check_block_v(block_v, *g));
  if (block_kc != 128 && block_kc != g->K)
    return fail(GDNR_ERR_UNSUPPORTED, "block_kc=%d: the checkpoint is streamed in whole 128-column rows", block_kc);
  return GDNR_OK;
}
}  // namespace

int gdnr_replay_fp8_split(const gdnr_tensor* checkpoint, const gdnr_tensor* checkpoint_scale, const gdnr_tensor* q,
                          const gdnr_tensor* k_cache, const gdnr_tensor* v_cache, const gdnr_tensor* g_cache,
                          const gdnr_tensor* beta_cache, const gdnr_tensor* valid_len,
                          const gdnr_tensor* transformed_query, const gdnr_tensor* coefficient,
                          const gdnr_tensor* out, int32_t block_v, int32_t block_kc, int32_t precompute_grouped,
                          void* stream) {
  g_last_error.clear();
  Geometry g;
  GDNR_TRY(check_split(checkpoint, checkpoint_scale, q, k_cache, v_cache, g_cache, beta_cache, valid_len, out,
                       block_v, block_kc, &g));
  GDNR_TRY(check_desc(transformed_query, "transformed_query_buffer", 3));
  GDNR_TRY(check_dtype(transformed_query, "transformed_query_buffer", {GDNR_DTYPE_F32}));
  GDNR_TRY(check_shape(transformed_query, "transformed_query_buffer", {g.B, g.HV, g.K}));
  GDNR_TRY(check_inner_unit(transformed_query, "transformed_query_buffer"));
  GDNR_TRY(check_align(transformed_query, "transformed_query_buffer", 16));
  GDNR_TRY(check_desc(coefficient, "coefficient_buffer", 3));
  GDNR_TRY(check_dtype(coefficient, "coefficient_buffer", {GDNR_DTYPE_F32}));
  GDNR_TRY(check_shape(coefficient, "coefficient_buffer", {g.B, g.HV}));
  if (coefficient->shape[2] < g.L)
    return fail(GDNR_ERR_INVALID_ARGUMENT, "coefficient_buffer: last dim %lld is shorter than the ring (%lld)",
                (long long)coefficient->shape[2], (long long)g.L);
  if (g.B == 0) return GDNR_OK;
  return split_launch(g, checkpoint, checkpoint_scale, q, k_cache, v_cache, g_cache, beta_cache, valid_len,
                      (float*)transformed_query->data, transformed_query->strides[0], transformed_query->strides[1],
                      (float*)coefficient->data, coefficient->strides[0], coefficient->strides[1],
                      coefficient->strides[2], out, block_v, precompute_grouped, stream);
}

int gdnr_replay_fp8_split_noalloc(const gdnr_tensor* checkpoint, const gdnr_tensor* checkpoint_scale,
                                  const gdnr_tensor* q, const gdnr_tensor* k_cache, const gdnr_tensor* v_cache,
                                  const gdnr_tensor* g_cache, const gdnr_tensor* beta_cache,
                                  const gdnr_tensor* valid_len, const gdnr_tensor* out, int32_t block_v,
                                  int32_t block_kc, int32_t precompute_grouped, void* stream) {
  g_last_error.clear();
  Geometry g;
  GDNR_TRY(check_split(checkpoint, checkpoint_scale, q, k_cache, v_cache, g_cache, beta_cache, valid_len, out,
                       block_v, block_kc, &g));
  // T_0 [B,HV,K] then the coefficients [B,HV,L], packed, in the device array
  const int64_t heads = (int64_t)g.B * g.HV;
  const int64_t tq_bytes = heads * g.K * 4, bytes = tq_bytes + heads * g.L * 4;
  if (bytes > (int64_t)gdnr::kSplitScratchBytes)
    return fail(GDNR_ERR_UNSUPPORTED,
                "split scratch: B*HV=%lld with K=%lld and ring length %lld needs %lld bytes, more than the %lld "
                "this entry point holds per GPU (use gdnr_replay_fp8_split with caller buffers)",
                (long long)heads, (long long)g.K, (long long)g.L, (long long)bytes,
                (long long)gdnr::kSplitScratchBytes);
  if (g.B == 0) return GDNR_OK;
  uint8_t* scratch = gdnr::split_scratch();
  if (!scratch) return fail(GDNR_ERR_HIP, "split scratch: hipGetSymbolAddress failed on the current device");
  return split_launch(g, checkpoint, checkpoint_scale, q, k_cache, v_cache, g_cache, beta_cache, valid_len,
                      (float*)scratch, (int64_t)g.HV * g.K, g.K, (float*)(scratch + tq_bytes), (int64_t)g.HV * g.L,
                      g.L, 1, out, block_v, precompute_grouped, stream);
}

int gdnr_prep_ring(const gdnr_tensor* mixed_qkv, const gdnr_tensor* a, const gdnr_tensor* b,
                   const gdnr_tensor* a_log, const gdnr_tensor* dt_bias, const gdnr_tensor* pos,
                   const gdnr_tensor* q_out, const gdnr_tensor* k_ring, const gdnr_tensor* v_ring,
                   const gdnr_tensor* g_ring, const gdnr_tensor* beta_ring, int32_t fused, void* stream) {
  (void)fused;
  g_last_error.clear();
  Geometry g;
  GDNR_TRY(check_ring(k_ring, v_ring, g_ring, beta_ring, &g, 4));
  GDNR_TRY(check_act_tensor(q_out, "q_out", 3, {g.B, g.H, g.K}, g.act, 2 * elem_size(g.act)));
  GDNR_TRY(check_prep_inputs(mixed_qkv, a, b, a_log, dt_bias, pos, g));
  if (g.B == 0) return GDNR_OK;
  gdnr::ReplayArgs r = {};
  fill_prep_inputs(&r, mixed_qkv, a, b, a_log, dt_bias, pos, q_out);
  gdnr::PrepArgs p = {};
  p.mixed = r.mixed;
  p.mx_b = r.mx_b;
  p.a = r.a;
  p.a_b = r.a_b;
  p.a_h = r.a_h;
  p.bgate = r.bgate;
  p.bg_b = r.bg_b;
  p.bg_h = r.bg_h;
  p.a_log = r.a_log;
  p.al_s = r.al_s;
  p.dt_bias = r.dt_bias;
  p.db_s = r.db_s;
  p.pos = r.pos;
  p.pos_s = r.pos_s;
  p.q_out = r.q_out;
  p.qo_b = r.qo_b;
  p.qo_h = r.qo_h;
  p.k = k_ring->data;
  p.k_b = k_ring->strides[0];
  p.k_t = k_ring->strides[1];
  p.k_h = k_ring->strides[2];
  p.v = v_ring->data;
  p.v_b = v_ring->strides[0];
  p.v_t = v_ring->strides[1];
  p.v_h = v_ring->strides[2];
  p.g = g_ring->data;
  p.g_b = g_ring->strides[0];
  p.g_t = g_ring->strides[1];
  p.g_h = g_ring->strides[2];
  p.beta = beta_ring->data;
  p.be_b = beta_ring->strides[0];
  p.be_t = beta_ring->strides[1];
  p.be_h = beta_ring->strides[2];
  p.B = (int32_t)g.B;
  p.H = (int32_t)g.H;
  p.HV = (int32_t)g.HV;
  p.G = (int32_t)(g.HV / g.H);
  p.V = (int32_t)g.V;
  p.L = (int32_t)g.L;
  return hip_status(launch_prep(p, g.act, a->dtype == GDNR_DTYPE_F32, stream));
}

int gdnr_prep_replay_fp8(const gdnr_tensor* mixed_qkv, const gdnr_tensor* a, const gdnr_tensor* b,
                         const gdnr_tensor* a_log, const gdnr_tensor* dt_bias, const gdnr_tensor* pos,
                         const gdnr_tensor* checkpoint, const gdnr_tensor* checkpoint_scale,
                         const gdnr_tensor* q_out, const gdnr_tensor* k_ring, const gdnr_tensor* v_ring,
                         const gdnr_tensor* g_ring, const gdnr_tensor* beta_ring, const gdnr_tensor* valid_len,
                         const gdnr_tensor* flush, const gdnr_tensor* out, int32_t block_v, void* stream) {
  g_last_error.clear();
  Geometry g;
  GDNR_TRY(check_ring(k_ring, v_ring, g_ring, beta_ring, &g, 16));
  GDNR_TRY(check_checkpoint(checkpoint, checkpoint_scale, g));
  GDNR_TRY(check_act_tensor(q_out, "q_out", 3, {g.B, g.H, g.K}, g.act, 2 * elem_size(g.act)));
  GDNR_TRY(check_prep_inputs(mixed_qkv, a, b, a_log, dt_bias, pos, g));
  GDNR_TRY(check_index_vec(valid_len, "valid_len", g.B, false));
  GDNR_TRY(check_index_vec(flush, "flush", g.B, true));
  GDNR_TRY(check_act_tensor(out, "out", 3, {g.B, g.HV, g.V}, g.act, 2));
  GDNR_TRY(check_block_v(block_v, g));
  if (g.B == 0) return GDNR_OK;
  gdnr::ReplayArgs r = {};
  fill_common(&r, g, block_v);
  fill_ckpt(&r, checkpoint, checkpoint_scale);
  fill_ring(&r, k_ring, v_ring, g_ring, beta_ring);
  fill_prep_inputs(&r, mixed_qkv, a, b, a_log, dt_bias, pos, q_out);
  r.q = q_out->data;
  r.q_b = q_out->strides[0];
  r.q_h = q_out->strides[1];
  fill_index(valid_len, &r.valid_len, &r.vl_s);
  fill_index(flush, &r.flush, &r.fl_s);
  r.out = out->data;
  r.o_b = out->strides[0];
  r.o_h = out->strides[1];
  if (decode_eligible(r, g.act) && decode_offsets_fit(r, elem_size(g.act))) {
    fit_decode(&r);
    return hip_status(launch_decode(r, g.act, true, a->dtype == GDNR_DTYPE_F32, stream));
  }
  if (r.L <= gdnr::kStepRing && step_offsets_fit(r, elem_size(g.act))) {
    GDNR_TRY(fit_step(&r, elem_size(g.act)));
    return hip_status(launch_step(r, g.act, true, a->dtype == GDNR_DTYPE_F32, stream));
  }
  fit_replay_tile(&r);
  GDNR_TRY(fit_lds(&r, elem_size(g.act), true, true));
  return hip_status(launch_replay(r, g.act, gdnr::kModeFused, a->dtype == GDNR_DTYPE_F32, stream));
}

int gdnr_prep_replay_fp8_slots(const gdnr_tensor* mixed_qkv, const gdnr_tensor* a, const gdnr_tensor* b,
                               const gdnr_tensor* a_log, const gdnr_tensor* dt_bias, const gdnr_tensor* pos,
                               const gdnr_tensor* state_indices, const gdnr_tensor* checkpoint,
                               const gdnr_tensor* checkpoint_scale, const gdnr_tensor* q_out,
                               const gdnr_tensor* k_ring, const gdnr_tensor* v_ring, const gdnr_tensor* g_ring,
                               const gdnr_tensor* beta_ring, const gdnr_tensor* valid_len, const gdnr_tensor* flush,
                               const gdnr_tensor* out, int32_t block_v, void* stream) {
  g_last_error.clear();
  Geometry slots;  // the slot-indexed tensors: rows = slots
  GDNR_TRY(check_ring(k_ring, v_ring, g_ring, beta_ring, &slots, 16));
  GDNR_TRY(check_checkpoint(checkpoint, checkpoint_scale, slots));
  GDNR_TRY(check_desc(state_indices, "state_indices", 1));
  GDNR_TRY(check_dtype(state_indices, "state_indices", {GDNR_DTYPE_I32}));
  if (slots.B < 1) return fail(GDNR_ERR_INVALID_ARGUMENT, "the slot tensors hold no slot (slot 0 is the null slot)");
  if (slots.B > INT32_MAX) return fail(GDNR_ERR_UNSUPPORTED, "more than 2^31 slots");
  Geometry g = slots;  // the per-sequence tensors: rows = batch
  g.B = state_indices->shape[0];
  GDNR_TRY(check_act_tensor(q_out, "q_out", 3, {g.B, g.H, g.K}, g.act, 2 * elem_size(g.act)));
  GDNR_TRY(check_prep_inputs(mixed_qkv, a, b, a_log, dt_bias, pos, g));
  GDNR_TRY(check_index_vec(valid_len, "valid_len", g.B, false));
  GDNR_TRY(check_index_vec(flush, "flush", g.B, true));
  GDNR_TRY(check_act_tensor(out, "out", 3, {g.B, g.HV, g.V}, g.act, 2));
  GDNR_TRY(check_block_v(block_v, g));
  if (g.B == 0) return GDNR_OK;
  gdnr::ReplayArgs r = {};
  fill_common(&r, g, block_v);
  fill_ckpt(&r, checkpoint, checkpoint_scale);
  fill_ring(&r, k_ring, v_ring, g_ring, beta_ring);
  fill_prep_inputs(&r, mixed_qkv, a, b, a_log, dt_bias, pos, q_out);
  r.q = q_out->data;
  r.q_b = q_out->strides[0];
  r.q_h = q_out->strides[1];
  fill_index(valid_len, &r.valid_len, &r.vl_s);
  fill_index(flush, &r.flush, &r.fl_s);
  fill_index(state_indices, &r.slot, &r.sl_s);
  r.n_slots = (int32_t)slots.B;
  r.out = out->data;
  r.o_b = out->strides[0];
  r.o_h = out->strides[1];
  // the decode kernel (16-bit activations, rings of <= 16 tokens, or of
  // <= 64 with V <= 128; 64-bit slot bases, 32-bit offsets inside a slot),
  // else the step kernel (rings of <= 16 tokens, tensors under 2 GiB), else
  // the long-ring kernel (rings of up to 64 tokens, every address in 64 bits)
  if (decode_eligible(r, g.act) && decode_offsets_fit(r, elem_size(g.act))) {
    fit_decode(&r);
    return hip_status(launch_decode(r, g.act, true, a->dtype == GDNR_DTYPE_F32, stream));
  }
  if (r.L <= gdnr::kStepRing && step_offsets_fit(r, elem_size(g.act))) {
    GDNR_TRY(fit_step(&r, elem_size(g.act)));
    return hip_status(launch_step(r, g.act, true, a->dtype == GDNR_DTYPE_F32, stream));
  }
  fit_replay_tile(&r);
  GDNR_TRY(fit_lds(&r, elem_size(g.act), true, true));
  return hip_status(launch_replay(r, g.act, gdnr::kModeFused, a->dtype == GDNR_DTYPE_F32, stream));
}

int gdnr_quantize_vblock32(const gdnr_tensor* state, const gdnr_tensor* payload, const gdnr_tensor* scale,
                           const gdnr_tensor* saturated, void* stream) {
  g_last_error.clear();
  int64_t B, HV, V;
  GDNR_TRY(check_quant(state, payload, scale, &B, &HV, &V));
  if (saturated) {
    GDNR_TRY(check_desc(saturated, "saturated", 3));
    GDNR_TRY(check_dtype(saturated, "saturated", {GDNR_DTYPE_I32}));
    GDNR_TRY(check_shape(saturated, "saturated", {B, HV, V / gdnr::kVBlock}));
  }
  if (B * HV * V == 0) return GDNR_OK;
  gdnr::QuantArgs q = {};
  fill_quant(&q, state, payload, scale, B, HV, V);
  if (saturated) {
    q.saturated = (int32_t*)saturated->data;
    q.sa_b = saturated->strides[0];
    q.sa_h = saturated->strides[1];
    q.sa_v = saturated->strides[2];
  }
  return hip_status(gdnr::launch_quantize(q, stream));
}

int gdnr_dequantize_vblock32(const gdnr_tensor* payload, const gdnr_tensor* scale, const gdnr_tensor* state,
                             void* stream) {
  g_last_error.clear();
  int64_t B, HV, V;
  GDNR_TRY(check_quant(state, payload, scale, &B, &HV, &V));
  if (B * HV * V == 0) return GDNR_OK;
  gdnr::QuantArgs q = {};
  fill_quant(&q, state, payload, scale, B, HV, V);
  return hip_status(gdnr::launch_dequantize(q, stream));
}

int gdnr_stream_probe(const gdnr_tensor* buffer, int32_t flags, void* stream) {
  g_last_error.clear();
  if (!buffer) return fail(GDNR_ERR_INVALID_ARGUMENT, "buffer: null tensor descriptor");
  if (buffer->ndim < 1 || buffer->ndim > GDNR_MAX_DIMS)
    return fail(GDNR_ERR_INVALID_ARGUMENT, "buffer: %d dims", buffer->ndim);
  GDNR_TRY(check_desc(buffer, "buffer", buffer->ndim));
  // C-contiguous, whole 16-byte pieces
  int64_t numel = 1;
  for (int d = buffer->ndim - 1; d >= 0; --d) {
    if (buffer->shape[d] > 1 && buffer->strides[d] != numel)
      return fail(GDNR_ERR_INVALID_ARGUMENT, "buffer: not contiguous (dim %d)", d);
    numel *= buffer->shape[d];
  }
  const int64_t bytes = numel * elem_size(buffer->dtype);
  if (bytes % 16) return fail(GDNR_ERR_INVALID_ARGUMENT, "buffer: %lld bytes is not a multiple of 16", (long long)bytes);
  GDNR_TRY(check_align(buffer, "buffer", 16));
  if (bytes == 0) return GDNR_OK;
  if ((flags & ~15) || ((flags & 4) && (flags & 1)) || ((flags & 8) && !(flags & 4)))
    return fail(GDNR_ERR_INVALID_ARGUMENT,
                "flags: %d (bit 0 write-back, bit 1 non-temporal, bit 2 chunked read, bit 3 tiled chunks; "
                "chunked reads only)", flags);
  return hip_status(gdnr::launch_stream_probe(buffer->data, bytes, (flags & 1) != 0, (flags & 2) != 0,
                                              (flags & 4) != 0, (flags & 8) != 0, stream));
}

int gdnr_bf16_step(const gdnr_tensor* state, const gdnr_tensor* q, const gdnr_tensor* k, const gdnr_tensor* v,
                   const gdnr_tensor* g, const gdnr_tensor* beta, const gdnr_tensor* out, void* stream) {
  g_last_error.clear();
  GDNR_TRY(check_desc(state, "state", 4));
  GDNR_TRY(check_dtype(state, "state", {GDNR_DTYPE_BF16, GDNR_DTYPE_F16, GDNR_DTYPE_F32}));
  const int64_t B = state->shape[0], HV = state->shape[1], V = state->shape[2], K = state->shape[3];
  if (K != gdnr::kKeyDim)
    return fail(GDNR_ERR_UNSUPPORTED, "state: K=%lld (only K=%d is built)", (long long)K, gdnr::kKeyDim);
  if (V % gdnr::kVBlock)
    return fail(GDNR_ERR_UNSUPPORTED, "state: V=%lld is not a multiple of %d", (long long)V, gdnr::kVBlock);
  GDNR_TRY(check_inner_unit(state, "state"));
  GDNR_TRY(check_align(state, "state", 16));
  const int ses = elem_size(state->dtype);
  if (state->strides[2] * ses * 32 >= ((int64_t)1 << 31))
    return fail(GDNR_ERR_UNSUPPORTED, "state: row stride of %lld bytes is too large", (long long)(state->strides[2] * ses));
  GDNR_TRY(check_desc(k, "k", 3));
  const int act = k->dtype;
  if (!is_act(act)) return fail(GDNR_ERR_INVALID_ARGUMENT, "k: dtype %s is not bf16|f16|f32", dtype_name(act));
  const int64_t H = k->shape[1];
  if (H <= 0 || HV % H)
    return fail(GDNR_ERR_INVALID_ARGUMENT, "k: %lld key heads do not divide %lld value heads", (long long)H,
                (long long)HV);
  const int es = elem_size(act);
  GDNR_TRY(check_act_tensor(k, "k", 3, {B, H, K}, act, es));
  GDNR_TRY(check_act_tensor(q, "q", 3, {B, H, K}, act, es));
  GDNR_TRY(check_act_tensor(v, "v", 3, {B, HV, V}, act, es));
  GDNR_TRY(check_act_tensor(g, "g", 2, {B, HV}, act, es));
  GDNR_TRY(check_act_tensor(beta, "beta", 2, {B, HV}, act, es));
  GDNR_TRY(check_act_tensor(out, "out", 3, {B, HV, V}, act, es));
  if (B > 65535) return fail(GDNR_ERR_UNSUPPORTED, "batch %lld exceeds 65535", (long long)B);
  if (B * HV * V == 0) return GDNR_OK;
  gdnr::RmwArgs a = {};
  a.state = state->data, a.st_b = state->strides[0], a.st_h = state->strides[1], a.st_v = state->strides[2];
  a.q = q->data, a.q_b = q->strides[0], a.q_h = q->strides[1];
  a.k = k->data, a.k_b = k->strides[0], a.k_h = k->strides[1];
  a.v = v->data, a.v_b = v->strides[0], a.v_h = v->strides[1];
  a.g = g->data, a.g_b = g->strides[0], a.g_h = g->strides[1];
  a.beta = beta->data, a.be_b = beta->strides[0], a.be_h = beta->strides[1];
  a.out = out->data, a.o_b = out->strides[0], a.o_h = out->strides[1];
  a.B = (int32_t)B, a.HV = (int32_t)HV, a.V = (int32_t)V, a.G = (int32_t)(HV / H);
  a.out_scale = 1.0f / __builtin_sqrtf((float)K);
  return hip_status(gdnr::launch_rmw_step(a, state->dtype, act, stream));
}

int gdnr_bf16_step_packed(const gdnr_tensor* mixed_qkv, const gdnr_tensor* a, const gdnr_tensor* b,
                          const gdnr_tensor* a_log, const gdnr_tensor* dt_bias, const gdnr_tensor* state,
                          const gdnr_tensor* state_indices, const gdnr_tensor* out, float scale, void* stream) {
  g_last_error.clear();
  if (!(scale - scale == 0.0f)) return fail(GDNR_ERR_INVALID_ARGUMENT, "scale: %g is not finite", (double)scale);
  GDNR_TRY(check_desc(state, "state", 4));
  GDNR_TRY(check_dtype(state, "state", {GDNR_DTYPE_BF16, GDNR_DTYPE_F16, GDNR_DTYPE_F32}));
  const int64_t S = state->shape[0], HV = state->shape[1], V = state->shape[2], K = state->shape[3];
  if (K != gdnr::kKeyDim)
    return fail(GDNR_ERR_UNSUPPORTED, "state: K=%lld (only K=%d is built)", (long long)K, gdnr::kKeyDim);
  if (V % gdnr::kVBlock)
    return fail(GDNR_ERR_UNSUPPORTED, "state: V=%lld is not a multiple of %d", (long long)V, gdnr::kVBlock);
  if (S < 1) return fail(GDNR_ERR_INVALID_ARGUMENT, "state holds no slot (slot 0 is the null slot)");
  GDNR_TRY(check_inner_unit(state, "state"));
  GDNR_TRY(check_align(state, "state", 16));
  const int ses = elem_size(state->dtype);
  if (state->strides[2] * ses * 32 >= ((int64_t)1 << 31))
    return fail(GDNR_ERR_UNSUPPORTED, "state: row stride of %lld bytes is too large", (long long)(state->strides[2] * ses));
  GDNR_TRY(check_desc(mixed_qkv, "mixed_qkv", 2));
  const int act = mixed_qkv->dtype;
  if (!is_act(act)) return fail(GDNR_ERR_INVALID_ARGUMENT, "mixed_qkv: dtype %s is not bf16|f16|f32", dtype_name(act));
  const int64_t B = mixed_qkv->shape[0], width = mixed_qkv->shape[1];
  const int64_t hk2 = width - HV * V;
  if (hk2 <= 0 || hk2 % (2 * K))
    return fail(GDNR_ERR_INVALID_ARGUMENT, "mixed_qkv: width %lld is not 2 H K + HV V (HV=%lld, V=%lld, K=%lld)",
                (long long)width, (long long)HV, (long long)V, (long long)K);
  const int64_t H = hk2 / (2 * K);
  if (HV % H)
    return fail(GDNR_ERR_INVALID_ARGUMENT, "%lld key heads do not divide %lld value heads", (long long)H, (long long)HV);
  GDNR_TRY(check_inner_unit(mixed_qkv, "mixed_qkv"));
  GDNR_TRY(check_desc(a, "a", 2));
  GDNR_TRY(check_desc(b, "b", 2));
  if (a->dtype != b->dtype || (a->dtype != act && a->dtype != GDNR_DTYPE_F32))
    return fail(GDNR_ERR_INVALID_ARGUMENT, "a/b: dtypes %s/%s (expected both f32 or both %s)", dtype_name(a->dtype),
                dtype_name(b->dtype), dtype_name(act));
  GDNR_TRY(check_shape(a, "a", {B, HV}));
  GDNR_TRY(check_shape(b, "b", {B, HV}));
  GDNR_TRY(check_desc(a_log, "a_log", 1));
  GDNR_TRY(check_desc(dt_bias, "dt_bias", 1));
  GDNR_TRY(check_dtype(a_log, "a_log", {GDNR_DTYPE_F32}));
  GDNR_TRY(check_dtype(dt_bias, "dt_bias", {GDNR_DTYPE_F32}));
  GDNR_TRY(check_shape(a_log, "a_log", {HV}));
  GDNR_TRY(check_shape(dt_bias, "dt_bias", {HV}));
  GDNR_TRY(check_index_vec(state_indices, "state_indices", B, false));
  GDNR_TRY(check_act_tensor(out, "out", 4, {B, 1, HV, V}, act, elem_size(act)));
  if (B > 65535) return fail(GDNR_ERR_UNSUPPORTED, "batch %lld exceeds 65535", (long long)B);
  if (B * HV * V == 0) return GDNR_OK;
  gdnr::RmwArgs r = {};
  r.state = state->data, r.st_b = state->strides[0], r.st_h = state->strides[1], r.st_v = state->strides[2];
  r.mixed = mixed_qkv->data, r.mx_b = mixed_qkv->strides[0];
  r.a = a->data, r.a_b = a->strides[0], r.a_h = a->strides[1];
  r.bgate = b->data, r.bg_b = b->strides[0], r.bg_h = b->strides[1];
  r.a_log = (const float*)a_log->data, r.al_s = a_log->strides[0];
  r.dt_bias = (const float*)dt_bias->data, r.db_s = dt_bias->strides[0];
  r.slot = (const int32_t*)state_indices->data, r.sl_s = state_indices->strides[0];
  r.out = out->data, r.o_b = out->strides[0], r.o_h = out->strides[2];
  r.B = (int32_t)B, r.HV = (int32_t)HV, r.V = (int32_t)V, r.G = (int32_t)(HV / H), r.H = (int32_t)H;
  r.n_slots = (int32_t)S;
  r.out_scale = scale;
  return hip_status(gdnr::launch_rmw_packed(r, state->dtype, act, a->dtype == GDNR_DTYPE_F32, stream));
}

namespace {
// the scale (or saturated) tensor of a format: shape per granularity, and its
// [b, hv, i, j] strides
int check_format_scale(const gdnr_tensor* t, const char* name, int gran, int64_t B, int64_t HV, int64_t V, int64_t K,
                       int64_t tile, std::initializer_list<int> dtypes, int64_t st[4]) {
  const bool vb = gran == GDNR_GRANULARITY_VBLOCK;
  GDNR_TRY(check_desc(t, name, vb ? 3 : 4));
  GDNR_TRY(check_dtype(t, name, dtypes));
  if (gran == GDNR_GRANULARITY_HEAD) GDNR_TRY(check_shape(t, name, {B, HV, 1, 1}));
  else if (gran == GDNR_GRANULARITY_ROW) GDNR_TRY(check_shape(t, name, {B, HV, V, 1}));
  else if (gran == GDNR_GRANULARITY_TILE) GDNR_TRY(check_shape(t, name, {B, HV, V / tile, K / tile}));
  else GDNR_TRY(check_shape(t, name, {B, HV, V / tile}));
  st[0] = t->strides[0], st[1] = t->strides[1], st[2] = t->strides[2], st[3] = vb ? 0 : t->strides[3];
  return GDNR_OK;
}

int check_format(const gdnr_tensor* state, const gdnr_tensor* payload, const gdnr_tensor* scale,
                 const gdnr_tensor* saturated, int32_t gran, int32_t tile, gdnr::FormatArgs* f) {
  GDNR_TRY(check_desc(state, "state", 4));
  GDNR_TRY(check_dtype(state, "state", {GDNR_DTYPE_F32}));
  const int64_t B = state->shape[0], HV = state->shape[1], V = state->shape[2], K = state->shape[3];
  GDNR_TRY(check_desc(payload, "payload", 4));
  GDNR_TRY(check_dtype(payload, "payload", {GDNR_DTYPE_FP8E4M3FN, GDNR_DTYPE_U8, GDNR_DTYPE_I8}));
  GDNR_TRY(check_shape(payload, "payload", {B, HV, V, K}));
  GDNR_TRY(check_inner_unit(state, "state"));
  GDNR_TRY(check_inner_unit(payload, "payload"));
  if (gran < GDNR_GRANULARITY_HEAD || gran > GDNR_GRANULARITY_VBLOCK)
    return fail(GDNR_ERR_INVALID_ARGUMENT, "granularity %d: expected 0 (head), 1 (row), 2 (tile) or 3 (vblock)",
                gran);
  const bool tiled = gran == GDNR_GRANULARITY_TILE || gran == GDNR_GRANULARITY_VBLOCK;
  if (tiled && (tile < 1 || V % tile || (gran == GDNR_GRANULARITY_TILE && K % tile)))
    return fail(GDNR_ERR_INVALID_ARGUMENT, "tile_size=%d must divide V=%lld%s", tile, (long long)V,
                gran == GDNR_GRANULARITY_TILE ? " and K" : "");
  if (B * HV > INT32_MAX || V > INT32_MAX || K > INT32_MAX)
    return fail(GDNR_ERR_UNSUPPORTED, "state extents too large");
  int64_t sc[4], sa[4] = {0, 0, 0, 0};
  GDNR_TRY(check_format_scale(scale, "scale", gran, B, HV, V, K, tiled ? tile : 1,
                              {GDNR_DTYPE_F16, GDNR_DTYPE_F32}, sc));
  if (saturated)
    GDNR_TRY(check_format_scale(saturated, "saturated", gran, B, HV, V, K, tiled ? tile : 1, {GDNR_DTYPE_I32}, sa));
  *f = {};
  f->state = (float*)state->data, f->st_b = state->strides[0], f->st_h = state->strides[1], f->st_v = state->strides[2];
  f->payload = payload->data, f->pl_b = payload->strides[0], f->pl_h = payload->strides[1];
  f->pl_v = payload->strides[2];
  f->scale = scale->data, f->sc_b = sc[0], f->sc_h = sc[1], f->sc_r = sc[2], f->sc_c = sc[3];
  f->scale_dt = scale->dtype == GDNR_DTYPE_F32 ? gdnr::DT_F32 : gdnr::DT_F16;
  f->saturated = saturated ? (int32_t*)saturated->data : nullptr;
  f->sa_b = sa[0], f->sa_h = sa[1], f->sa_r = sa[2], f->sa_c = sa[3];
  f->B = (int32_t)B, f->HV = (int32_t)HV, f->V = (int32_t)V, f->K = (int32_t)K;
  f->gran = gran, f->tile = tiled ? tile : 1, f->int8 = payload->dtype == GDNR_DTYPE_I8;
  return GDNR_OK;
}
}  // namespace

int gdnr_quantize_checkpoint(const gdnr_tensor* state, const gdnr_tensor* payload, const gdnr_tensor* scale,
                             const gdnr_tensor* saturated, int32_t granularity, int32_t tile_size, void* stream) {
  g_last_error.clear();
  gdnr::FormatArgs f;
  GDNR_TRY(check_format(state, payload, scale, saturated, granularity, tile_size, &f));
  if ((int64_t)f.B * f.HV * f.V * f.K == 0) return GDNR_OK;
  return hip_status(gdnr::launch_format_quantize(f, stream));
}

int gdnr_dequantize_checkpoint(const gdnr_tensor* payload, const gdnr_tensor* scale, const gdnr_tensor* state,
                               int32_t granularity, int32_t tile_size, void* stream) {
  g_last_error.clear();
  gdnr::FormatArgs f;
  GDNR_TRY(check_format(state, payload, scale, nullptr, granularity, tile_size, &f));
  if ((int64_t)f.B * f.HV * f.V * f.K == 0) return GDNR_OK;
  return hip_status(gdnr::launch_format_dequantize(f, stream));
}

}  // extern "C"
