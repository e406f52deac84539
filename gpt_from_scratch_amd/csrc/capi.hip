// capi.hip — the extern "C" surface declared in include/mi_attn.h.
//
// Validates every argument before anything is enqueued, picks the kernel
// family (bf16/f16 MFMA when the shape and alignment allow it, exact-fp32
// VALU otherwise) and reports failures as status codes plus a per-thread
// message.  No allocation and no synchronisation.  Global mutable state: the
// thread-local error text, and the forward's per-device cache of the compute
// unit count (atomic entries, written once per device with the same value).
#include <atomic>
#include <cmath>
#include <initializer_list>
#include <utility>
#include <dlfcn.h>
#include <limits.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include <string>

#include "../../include/mi_attn.h"
#include "mi_kernels.h"

namespace {

thread_local std::string g_last_error;

mi_status fail(mi_status st, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
mi_status fail(mi_status st, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return st;
}

mi_status ok() {
  g_last_error.clear();
  return MI_OK;
}

// One build of this library per process.  Two builds loaded side by side
// register kernels of the same names with the HIP runtime, and a process that
// held four builds at once saw every build's outputs change from call to call
// (cause not traced; each build alone is bitwise deterministic).  The first
// copy loaded records "<pid>:<path>" in MI_ATTN_LIBRARY (the pid keeps a child
// process from inheriting the claim); a copy from another path that finds its
// own pid there refuses every entry point that launches work.
char g_first_copy[PATH_MAX + 32];  // set when another copy claimed the process first

__attribute__((constructor)) void claim_process() {
  Dl_info info;
  char self[PATH_MAX];
  if (!dladdr((void*)&claim_process, &info) || !info.dli_fname || !realpath(info.dli_fname, self))
    return;
  char mine[PATH_MAX + 32];
  snprintf(mine, sizeof(mine), "%ld:%s", (long)getpid(), self);
  const char* prev = getenv("MI_ATTN_LIBRARY");
  char pid[32];
  const int np = snprintf(pid, sizeof(pid), "%ld:", (long)getpid());
  if (prev && strncmp(prev, pid, np) == 0) {
    if (strcmp(prev, mine) != 0) snprintf(g_first_copy, sizeof(g_first_copy), "%s", prev + np);
    return;
  }
  setenv("MI_ATTN_LIBRARY", mine, 1);
}

#define MI_SOLE_COPY()                                                                      \
  do {                                                                                      \
    if (g_first_copy[0])                                                                    \
      return fail(MI_ERR_UNSUPPORTED,                                                       \
                  "another build of libmi_attn (%s) is loaded in this process; one build "  \
                  "per process",                                                            \
                  g_first_copy);                                                            \
  } while (0)

int elem_size(int dt) { return dt == MI_F32 ? 4 : 2; }

bool dtype_ok(int dt) { return dt == MI_F32 || dt == MI_F16 || dt == MI_BF16; }

// Tensor [B,H,S,D] with strides {sb, sh, ss, sd}: require sd == 1 and a non-null pointer.
mi_status check_attn_tensor(const char* name, const void* p, const int64_t* st) {
  if (p == nullptr) return fail(MI_ERR_INVALID_ARGUMENT, "%s: null pointer", name);
  if (st == nullptr) return fail(MI_ERR_INVALID_ARGUMENT, "%s: null strides", name);
  if (st[3] != 1)
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: dim stride must be 1 (got %lld)", name,
                (long long)st[3]);
  for (int i = 0; i < 3; ++i)
    if (st[i] < 0) return fail(MI_ERR_INVALID_ARGUMENT, "%s: negative stride", name);
  return MI_OK;
}

// The matrix-core kernels' operand tensors: 16-byte aligned base and strides
// that keep every row 16-byte aligned, and a row stride small enough that the
// byte offset of any row inside a 256-row tile fits the 32-bit offsets of
// their buffer loads.
bool aligned16(const void* p, const int64_t* st, int esz) {
  if (((uintptr_t)p) % 16) return false;
  for (int i = 0; i < 3; ++i)
    if ((st[i] * esz) % 16) return false;
  return st[2] * esz * 256 < (int64_t(1) << 31);
}

mi::TensorArg targ(const void* p, const int64_t* st) {
  mi::TensorArg t;
  t.ptr = p;
  t.sb = st[0];
  t.sh = st[1];
  t.ss = st[2];
  return t;
}

mi_status check_shape(int dtype, int B, int H, int S, int D, float scale) {
  if (!dtype_ok(dtype)) return fail(MI_ERR_INVALID_ARGUMENT, "unknown dtype %d", dtype);
  if (B <= 0 || H <= 0 || S <= 0 || D <= 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "sizes must be positive (B=%d H=%d S=%d D=%d)", B, H, S, D);
  if ((int64_t)B * H * S >= (1ll << 31))
    return fail(MI_ERR_UNSUPPORTED, "B*H*S = %lld rows exceeds 2^31", (long long)B * H * S);
  if (!(scale > 0.f) || scale != scale)
    return fail(MI_ERR_INVALID_ARGUMENT, "scale must be a positive finite number");
  return MI_OK;
}

mi_status launched(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(MI_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

// Inputs shared by the dK/dV and dQ stages.
mi_status check_grad_inputs(int dtype, int D, int S, const void* q, const int64_t* qs,
                            const void* k, const int64_t* ks, const void* v, const int64_t* vs,
                            const void* dout, const int64_t* dos, const float* lse,
                            const float* ws) {
  mi_status st;
  if ((st = check_attn_tensor("q", q, qs)) != MI_OK) return st;
  if ((st = check_attn_tensor("k", k, ks)) != MI_OK) return st;
  if ((st = check_attn_tensor("v", v, vs)) != MI_OK) return st;
  if ((st = check_attn_tensor("dout", dout, dos)) != MI_OK) return st;
  if (lse == nullptr || ws == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "lse / workspace: null pointer");
  if (!mi::valu_supports(D) && !mi::mfma_supports(dtype, D, S))
    return fail(MI_ERR_UNSUPPORTED, "head dim %d not supported (16, 32, 64, 128)", D);
  return MI_OK;
}

mi::AttnArgs grad_args(int B, int H, int S, int D, int causal, float scale, const void* q,
                       const int64_t* qs, const void* k, const int64_t* ks, const void* v,
                       const int64_t* vs, const void* dout, const int64_t* dos,
                       const float* lse, const float* ws) {
  mi::AttnArgs a = {};
  a.q = targ(q, qs);
  a.k = targ(k, ks);
  a.v = targ(v, vs);
  a.dout = targ(dout, dos);
  a.lse = const_cast<float*>(lse);
  a.delta = const_cast<float*>(ws);                 // ws[0 .. B*H*S): delta
  a.lse2 = ws + (int64_t)B * H * S;                 // ws[B*H*S ..): lse * log2(e)
  a.B = B; a.H = H; a.S = S; a.D = D;
  a.scale = scale;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.causal = causal ? 1 : 0;
  return a;
}

}  // namespace

extern "C" {

int mi_version(void) { return (2 << 16) | 5; }

const char* mi_status_str(mi_status s) {
  switch (s) {
    case MI_OK: return "ok";
    case MI_ERR_INVALID_ARGUMENT: return "invalid argument";
    case MI_ERR_UNSUPPORTED: return "unsupported";
    case MI_ERR_LAUNCH: return "launch failed";
  }
  return "unknown status";
}

const char* mi_last_error(void) { return g_last_error.c_str(); }

mi_status mi_attn_fwd(mi_dtype dtype, int B, int H, int S, int D, int causal, float scale,
                      const void* q, const int64_t q_strides[4], const void* k,
                      const int64_t k_strides[4], const void* v, const int64_t v_strides[4],
                      void* o, const int64_t o_strides[4], float* lse, void* stream) {
  MI_SOLE_COPY();
  mi_status st;
  if ((st = check_shape(dtype, B, H, S, D, scale)) != MI_OK) return st;
  if ((st = check_attn_tensor("q", q, q_strides)) != MI_OK) return st;
  if ((st = check_attn_tensor("k", k, k_strides)) != MI_OK) return st;
  if ((st = check_attn_tensor("v", v, v_strides)) != MI_OK) return st;
  if ((st = check_attn_tensor("o", o, o_strides)) != MI_OK) return st;
  if (lse == nullptr) return fail(MI_ERR_INVALID_ARGUMENT, "lse: null pointer");
  if (((uintptr_t)lse) % 4) return fail(MI_ERR_INVALID_ARGUMENT, "lse: misaligned");

  mi::AttnArgs a = {};
  a.q = targ(q, q_strides);
  a.k = targ(k, k_strides);
  a.v = targ(v, v_strides);
  a.o = targ(o, o_strides);
  a.lse = lse;
  a.B = B; a.H = H; a.S = S; a.D = D;
  a.scale = scale;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.causal = causal ? 1 : 0;

  const int esz = elem_size(dtype);
  const bool al = aligned16(q, q_strides, esz) && aligned16(k, k_strides, esz) &&
                  aligned16(v, v_strides, esz) && aligned16(o, o_strides, esz);
  if (al && mi::mfma_supports(dtype, D, S))
    return launched(mi::launch_attn_fwd_mfma(dtype, a, (hipStream_t)stream), "attn_fwd_mfma");
  if (!mi::valu_supports(D))
    return fail(MI_ERR_UNSUPPORTED, "head dim %d not supported (16, 32, 64, 128)", D);
  return launched(mi::launch_attn_fwd_valu(dtype, a, (hipStream_t)stream), "attn_fwd_valu");
}

static mi_status grads_impl(mi_dtype dtype, int B, int H, int S, int D, int causal, float scale,
                            const void* q, const int64_t q_strides[4], const void* k,
                            const int64_t k_strides[4], const void* v,
                            const int64_t v_strides[4], const void* dout,
                            const int64_t dout_strides[4], const float* lse, const float* ws,
                            void* dq, const int64_t dq_strides[4], void* dk,
                            const int64_t dk_strides[4], void* dv, const int64_t dv_strides[4],
                            const mi::RopeTab* rope, void* stream);

mi_status mi_attn_bwd(mi_dtype dtype, int B, int H, int S, int D, int causal, float scale,
                      const void* q, const int64_t q_strides[4], const void* k,
                      const int64_t k_strides[4], const void* v, const int64_t v_strides[4],
                      const void* o, const int64_t o_strides[4], const void* dout,
                      const int64_t dout_strides[4], const float* lse, float* ws, void* dq,
                      const int64_t dq_strides[4], void* dk, const int64_t dk_strides[4],
                      void* dv, const int64_t dv_strides[4], void* stream) {
  MI_SOLE_COPY();
  // Validate everything up front so that nothing is enqueued on a bad call.
  mi_status st;
  if ((st = check_shape(dtype, B, H, S, D, scale)) != MI_OK) return st;
  if ((st = check_attn_tensor("o", o, o_strides)) != MI_OK) return st;
  if ((st = check_attn_tensor("dq", dq, dq_strides)) != MI_OK) return st;
  if ((st = check_grad_inputs(dtype, D, S, q, q_strides, k, k_strides, v, v_strides, dout,
                              dout_strides, lse, ws)) != MI_OK)
    return st;
  if ((st = check_attn_tensor("dk", dk, dk_strides)) != MI_OK) return st;
  if ((st = check_attn_tensor("dv", dv, dv_strides)) != MI_OK) return st;
  if ((st = mi_attn_bwd_preprocess(dtype, B, H, S, D, o, o_strides, dout, dout_strides, lse, ws,
                                   stream)) != MI_OK)
    return st;
  return mi_attn_bwd_grads(dtype, B, H, S, D, causal, scale, q, q_strides, k, k_strides, v,
                           v_strides, dout, dout_strides, lse, ws, dq, dq_strides, dk,
                           dk_strides, dv, dv_strides, stream);
}

mi_status mi_attn_bwd_grads(mi_dtype dtype, int B, int H, int S, int D, int causal, float scale,
                            const void* q, const int64_t q_strides[4], const void* k,
                            const int64_t k_strides[4], const void* v,
                            const int64_t v_strides[4], const void* dout,
                            const int64_t dout_strides[4], const float* lse, const float* ws,
                            void* dq, const int64_t dq_strides[4], void* dk,
                            const int64_t dk_strides[4], void* dv, const int64_t dv_strides[4],
                            void* stream) {
  MI_SOLE_COPY();
  return grads_impl(dtype, B, H, S, D, causal, scale, q, q_strides, k, k_strides, v, v_strides,
                    dout, dout_strides, lse, ws, dq, dq_strides, dk, dk_strides, dv, dv_strides,
                    nullptr, stream);
}

static mi_status rope_common(mi_dtype x_dtype, mi_dtype tab_dtype, int S, int B, int H, int D,
                             int inverse, int nt, const void* const* ins,
                             const int64_t* const* in_st, void* const* outs,
                             const int64_t* const* out_st, const void* cos_tab,
                             const int64_t cos_strides[2], const void* sin_tab,
                             const int64_t sin_strides[2], void* stream);

// Whether the gradients run on the matrix-core kernels: bf16/f16 at their
// head dims and sequence multiple, every row 16-byte aligned.
static bool bwd_mfma_path(mi_dtype dtype, int D, int S, const void* q, const int64_t* qs,
                          const void* k, const int64_t* ks, const void* v, const int64_t* vs,
                          const void* dout, const int64_t* dos, const void* dq,
                          const int64_t* dqs, const void* dk, const int64_t* dks, const void* dv,
                          const int64_t* dvs) {
  const int esz = elem_size(dtype);
  return mi::mfma_supports(dtype, D, S) && aligned16(q, qs, esz) && aligned16(k, ks, esz) &&
         aligned16(v, vs, esz) && aligned16(dout, dos, esz) && aligned16(dq, dqs, esz) &&
         aligned16(dk, dks, esz) && aligned16(dv, dvs, esz);
}

// Whether the matrix-core kernels can rotate dQ and dK as they store them:
// their stores read four 16-bit angles per table with one vector load, so the
// tables must be 16-bit, with contiguous angles and every row start aligned to
// four of them; head dims 16 and 32 (run in the D = 64 layout) have no
// rotating stores.  Otherwise the host runs the inverse RoPE as a separate
// pass.
static bool rope_fusable(const mi::RopeTab& r, int D) {
  const int tsz = elem_size((mi_dtype)r.tdt);
  return D >= 64 && r.tdt != MI_F32 && r.cs_i == 1 && r.ss_i == 1 && r.cs_s % 4 == 0 && r.ss_s % 4 == 0 &&
         ((uintptr_t)r.cos) % (4 * tsz) == 0 && ((uintptr_t)r.sin) % (4 * tsz) == 0;
}

// `rope` != nullptr: dQ and dK leave inverse-rotated (mi_attn_bwd_rope).
static mi_status grads_impl(mi_dtype dtype, int B, int H, int S, int D, int causal, float scale,
                            const void* q, const int64_t q_strides[4], const void* k,
                            const int64_t k_strides[4], const void* v,
                            const int64_t v_strides[4], const void* dout,
                            const int64_t dout_strides[4], const float* lse, const float* ws,
                            void* dq, const int64_t dq_strides[4], void* dk,
                            const int64_t dk_strides[4], void* dv, const int64_t dv_strides[4],
                            const mi::RopeTab* rope, void* stream) {
  mi_status st;
  if ((st = check_shape(dtype, B, H, S, D, scale)) != MI_OK) return st;
  if ((st = check_grad_inputs(dtype, D, S, q, q_strides, k, k_strides, v, v_strides, dout,
                              dout_strides, lse, ws)) != MI_OK)
    return st;
  if ((st = check_attn_tensor("dq", dq, dq_strides)) != MI_OK) return st;
  if ((st = check_attn_tensor("dk", dk, dk_strides)) != MI_OK) return st;
  if ((st = check_attn_tensor("dv", dv, dv_strides)) != MI_OK) return st;
  if (bwd_mfma_path(dtype, D, S, q, q_strides, k, k_strides, v, v_strides, dout, dout_strides,
                    dq, dq_strides, dk, dk_strides, dv, dv_strides)) {
    mi::AttnArgs a = grad_args(B, H, S, D, causal, scale, q, q_strides, k, k_strides, v,
                               v_strides, dout, dout_strides, lse, ws);
    a.dq = targ(dq, dq_strides);
    a.dk = targ(dk, dk_strides);
    a.dv = targ(dv, dv_strides);
    const bool fuse_rope = rope && rope_fusable(*rope, D);
    if (fuse_rope) a.rope = *rope;
    if ((st = launched(mi::launch_attn_bwd_mfma(dtype, a, (hipStream_t)stream),
                       "attn_bwd_mfma")) != MI_OK || !rope || fuse_rope)
      return st;
  } else {
    if ((st = mi_attn_bwd_dkdv(dtype, B, H, S, D, causal, scale, q, q_strides, k, k_strides, v,
                               v_strides, dout, dout_strides, lse, ws, dk, dk_strides, dv,
                               dv_strides, stream)) != MI_OK)
      return st;
    if ((st = mi_attn_bwd_dq(dtype, B, H, S, D, causal, scale, q, q_strides, k, k_strides, v,
                             v_strides, dout, dout_strides, lse, ws, dq, dq_strides,
                             stream)) != MI_OK)
      return st;
    if (!rope) return MI_OK;
  }
  // kernels or tables without the fused rotation: the inverse RoPE pass over
  // dQ and dK in place ([B, H, S, D] strides reordered to the RoPE kernel's
  // [S, B, H, D])
  const int64_t qs[4] = {dq_strides[2], dq_strides[0], dq_strides[1], dq_strides[3]};
  const int64_t ks[4] = {dk_strides[2], dk_strides[0], dk_strides[1], dk_strides[3]};
  const int64_t cst[2] = {rope->cs_s, rope->cs_i}, sst[2] = {rope->ss_s, rope->ss_i};
  const void* ins[2] = {dq, dk};
  const int64_t* ist[2] = {qs, ks};
  void* outs[2] = {dq, dk};
  return rope_common(dtype, (mi_dtype)rope->tdt, S, B, H, D, 1, 2, ins, ist, outs, ist,
                     rope->cos, cst, rope->sin, sst, stream);
}

mi_status mi_attn_bwd_rope(mi_dtype dtype, int B, int H, int S, int D, int causal, float scale,
                           const void* q, const int64_t q_strides[4], const void* k,
                           const int64_t k_strides[4], const void* v, const int64_t v_strides[4],
                           const void* o, const int64_t o_strides[4], const void* dout,
                           const int64_t dout_strides[4], const float* lse, float* ws, void* dq,
                           const int64_t dq_strides[4], void* dk, const int64_t dk_strides[4],
                           void* dv, const int64_t dv_strides[4], mi_dtype tab_dtype,
                           const void* cos_tab, const int64_t cos_strides[2],
                           const void* sin_tab, const int64_t sin_strides[2], void* stream) {
  MI_SOLE_COPY();
  mi_status st;
  if ((st = check_shape(dtype, B, H, S, D, scale)) != MI_OK) return st;
  if ((st = check_attn_tensor("o", o, o_strides)) != MI_OK) return st;
  if ((st = check_attn_tensor("dq", dq, dq_strides)) != MI_OK) return st;
  if ((st = check_grad_inputs(dtype, D, S, q, q_strides, k, k_strides, v, v_strides, dout,
                              dout_strides, lse, ws)) != MI_OK)
    return st;
  if ((st = check_attn_tensor("dk", dk, dk_strides)) != MI_OK) return st;
  if ((st = check_attn_tensor("dv", dv, dv_strides)) != MI_OK) return st;
  if (!dtype_ok(tab_dtype)) return fail(MI_ERR_INVALID_ARGUMENT, "unknown table dtype %d", tab_dtype);
  if (D % 2) return fail(MI_ERR_INVALID_ARGUMENT, "HEAD_DIM must be even (got %d)", D);
  if (!cos_tab || !sin_tab || !cos_strides || !sin_strides)
    return fail(MI_ERR_INVALID_ARGUMENT, "cos/sin: null pointer");
  if (((uintptr_t)cos_tab) % elem_size(tab_dtype) || ((uintptr_t)sin_tab) % elem_size(tab_dtype))
    return fail(MI_ERR_INVALID_ARGUMENT, "cos/sin: misaligned");
  mi::RopeTab rope;
  rope.cos = cos_tab;
  rope.sin = sin_tab;
  rope.cs_s = cos_strides[0];
  rope.cs_i = cos_strides[1];
  rope.ss_s = sin_strides[0];
  rope.ss_i = sin_strides[1];
  rope.tdt = tab_dtype;
  // The separate inverse-RoPE pass (taken when the kernels cannot rotate as
  // they store) has its own launch limit: refuse before anything is enqueued.
  const bool fused = bwd_mfma_path(dtype, D, S, q, q_strides, k, k_strides, v, v_strides, dout,
                                   dout_strides, dq, dq_strides, dk, dk_strides, dv,
                                   dv_strides) &&
                     rope_fusable(rope, D);
  if (!fused && (uint64_t)2 * S * B * H * (D / 2) >= (1ull << 31))
    return fail(MI_ERR_UNSUPPORTED, "tensor too large for one launch");
  if ((st = mi_attn_bwd_preprocess(dtype, B, H, S, D, o, o_strides, dout, dout_strides, lse, ws,
                                   stream)) != MI_OK)
    return st;
  return grads_impl(dtype, B, H, S, D, causal, scale, q, q_strides, k, k_strides, v, v_strides,
                    dout, dout_strides, lse, ws, dq, dq_strides, dk, dk_strides, dv, dv_strides,
                    &rope, stream);
}

mi_status mi_attn_bwd_preprocess(mi_dtype dtype, int B, int H, int S, int D, const void* o,
                                 const int64_t o_strides[4], const void* dout,
                                 const int64_t dout_strides[4], const float* lse, float* ws,
                                 void* stream) {
  MI_SOLE_COPY();
  mi_status st;
  if ((st = check_shape(dtype, B, H, S, D, 1.f)) != MI_OK) return st;
  if ((st = check_attn_tensor("o", o, o_strides)) != MI_OK) return st;
  if ((st = check_attn_tensor("dout", dout, dout_strides)) != MI_OK) return st;
  if (lse == nullptr || ws == nullptr)
    return fail(MI_ERR_INVALID_ARGUMENT, "lse / workspace: null pointer");
  mi::AttnArgs a = {};
  a.o = targ(o, o_strides);
  a.dout = targ(dout, dout_strides);
  a.lse = const_cast<float*>(lse);
  a.delta = ws;
  a.B = B; a.H = H; a.S = S; a.D = D;
  return launched(mi::launch_attn_delta(dtype, a, (hipStream_t)stream), "attn_delta");
}

mi_status mi_attn_bwd_dkdv(mi_dtype dtype, int B, int H, int S, int D, int causal, float scale,
                           const void* q, const int64_t q_strides[4], const void* k,
                           const int64_t k_strides[4], const void* v, const int64_t v_strides[4],
                           const void* dout, const int64_t dout_strides[4], const float* lse,
                           const float* ws, void* dk, const int64_t dk_strides[4], void* dv,
                           const int64_t dv_strides[4], void* stream) {
  MI_SOLE_COPY();
  mi_status st;
  if ((st = check_shape(dtype, B, H, S, D, scale)) != MI_OK) return st;
  if ((st = check_grad_inputs(dtype, D, S, q, q_strides, k, k_strides, v, v_strides, dout,
                              dout_strides, lse, ws)) != MI_OK)
    return st;
  if ((st = check_attn_tensor("dk", dk, dk_strides)) != MI_OK) return st;
  if ((st = check_attn_tensor("dv", dv, dv_strides)) != MI_OK) return st;
  mi::AttnArgs a = grad_args(B, H, S, D, causal, scale, q, q_strides, k, k_strides, v, v_strides,
                             dout, dout_strides, lse, ws);
  a.dk = targ(dk, dk_strides);
  a.dv = targ(dv, dv_strides);
  const int esz = elem_size(dtype);
  const bool al = aligned16(q, q_strides, esz) && aligned16(k, k_strides, esz) &&
                  aligned16(v, v_strides, esz) && aligned16(dout, dout_strides, esz) &&
                  aligned16(dk, dk_strides, esz) && aligned16(dv, dv_strides, esz);
  hipStream_t s = (hipStream_t)stream;
  if (al && mi::mfma_supports(dtype, D, S))
    return launched(mi::launch_attn_bwd_dkdv_mfma(dtype, a, s), "attn_bwd_dkdv_mfma");
  return launched(mi::launch_attn_bwd_dkdv_valu(dtype, a, s), "attn_bwd_dkdv_valu");
}

mi_status mi_attn_bwd_dq(mi_dtype dtype, int B, int H, int S, int D, int causal, float scale,
                         const void* q, const int64_t q_strides[4], const void* k,
                         const int64_t k_strides[4], const void* v, const int64_t v_strides[4],
                         const void* dout, const int64_t dout_strides[4], const float* lse,
                         const float* ws, void* dq, const int64_t dq_strides[4],
                         void* stream) {
  MI_SOLE_COPY();
  mi_status st;
  if ((st = check_shape(dtype, B, H, S, D, scale)) != MI_OK) return st;
  if ((st = check_grad_inputs(dtype, D, S, q, q_strides, k, k_strides, v, v_strides, dout,
                              dout_strides, lse, ws)) != MI_OK)
    return st;
  if ((st = check_attn_tensor("dq", dq, dq_strides)) != MI_OK) return st;
  mi::AttnArgs a = grad_args(B, H, S, D, causal, scale, q, q_strides, k, k_strides, v, v_strides,
                             dout, dout_strides, lse, ws);
  a.dq = targ(dq, dq_strides);
  const int esz = elem_size(dtype);
  const bool al = aligned16(q, q_strides, esz) && aligned16(k, k_strides, esz) &&
                  aligned16(v, v_strides, esz) && aligned16(dout, dout_strides, esz) &&
                  aligned16(dq, dq_strides, esz);
  hipStream_t s = (hipStream_t)stream;
  if (al && mi::mfma_supports(dtype, D, S))
    return launched(mi::launch_attn_bwd_dq_mfma(dtype, a, s), "attn_bwd_dq_mfma");
  return launched(mi::launch_attn_bwd_dq_valu(dtype, a, s), "attn_bwd_dq_valu");
}

static mi_status rope_common(mi_dtype x_dtype, mi_dtype tab_dtype, int S, int B, int H, int D,
                             int inverse, int nt, const void* const* ins,
                             const int64_t* const* in_st, void* const* outs,
                             const int64_t* const* out_st, const void* cos_tab,
                             const int64_t cos_strides[2], const void* sin_tab,
                             const int64_t sin_strides[2], void* stream) {
  if (!dtype_ok(x_dtype) || !dtype_ok(tab_dtype))
    return fail(MI_ERR_INVALID_ARGUMENT, "unknown dtype");
  if (S <= 0 || B <= 0 || H <= 0 || D <= 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "sizes must be positive (S=%d B=%d H=%d D=%d)", S, B, H, D);
  if (D % 2) return fail(MI_ERR_INVALID_ARGUMENT, "HEAD_DIM must be even (got %d)", D);
  if ((uint64_t)nt * S * B * H * (D / 2) >= (1ull << 31))
    return fail(MI_ERR_UNSUPPORTED, "tensor too large for one launch");
  if (!cos_tab || !sin_tab || !cos_strides || !sin_strides)
    return fail(MI_ERR_INVALID_ARGUMENT, "cos/sin: null pointer");
  mi::RopeArgs a = {};
  a.ntensors = nt;
  a.cos_tab = cos_tab;
  a.sin_tab = sin_tab;
  a.cs_s = cos_strides[0];
  a.cs_i = cos_strides[1];
  a.ss_s = sin_strides[0];
  a.ss_i = sin_strides[1];
  a.S = S; a.B = B; a.H = H; a.D = D;
  a.inverse = inverse ? 1 : 0;
  const int esz = elem_size(x_dtype);
  const int vecn = 16 / esz;
  // the vector path also reads vecn/2 consecutive angles of a table row with
  // one aligned load
  const int np = vecn / 2;
  const int abytes = np * elem_size(tab_dtype);
  bool vec = (D % vecn == 0) && a.cs_i == 1 && a.ss_i == 1 && a.cs_s % np == 0 &&
             a.ss_s % np == 0 && ((uintptr_t)cos_tab) % abytes == 0 &&
             ((uintptr_t)sin_tab) % abytes == 0;
  for (int t = 0; t < nt; ++t) {
    if (!ins[t] || !outs[t] || !in_st[t] || !out_st[t])
      return fail(MI_ERR_INVALID_ARGUMENT, "rope tensor %d: null pointer", t);
    mi::RopeTensor& T = a.t[t];
    T.in = ins[t];
    T.out = outs[t];
    T.is_s = in_st[t][0]; T.is_b = in_st[t][1]; T.is_h = in_st[t][2]; T.is_d = in_st[t][3];
    T.os_s = out_st[t][0]; T.os_b = out_st[t][1]; T.os_h = out_st[t][2]; T.os_d = out_st[t][3];
    if (T.is_d != 1 || T.os_d != 1) vec = false;
    if (((uintptr_t)T.in) % 16 || ((uintptr_t)T.out) % 16) vec = false;
    for (int i = 0; i < 3; ++i)
      if ((in_st[t][i] * esz) % 16 || (out_st[t][i] * esz) % 16) vec = false;
  }
  return launched(mi::launch_rope(x_dtype, tab_dtype, a, vec, (hipStream_t)stream), "rope");
}

mi_status mi_rope(mi_dtype x_dtype, mi_dtype tab_dtype, int S, int B, int H, int D, int inverse,
                  const void* x, const int64_t x_strides[4], const void* cos_tab,
                  const int64_t cos_strides[2], const void* sin_tab, const int64_t sin_strides[2],
                  void* out, const int64_t out_strides[4], void* stream) {
  MI_SOLE_COPY();
  const void* ins[1] = {x};
  const int64_t* ist[1] = {x_strides};
  void* outs[1] = {out};
  const int64_t* ost[1] = {out_strides};
  return rope_common(x_dtype, tab_dtype, S, B, H, D, inverse, 1, ins, ist, outs, ost, cos_tab,
                     cos_strides, sin_tab, sin_strides, stream);
}

mi_status mi_rope_qk(mi_dtype x_dtype, mi_dtype tab_dtype, int S, int B, int H, int D,
                     int inverse, const void* q, const int64_t q_strides[4], const void* k,
                     const int64_t k_strides[4], const void* cos_tab, const int64_t cos_strides[2],
                     const void* sin_tab, const int64_t sin_strides[2], void* q_out,
                     const int64_t q_out_strides[4], void* k_out, const int64_t k_out_strides[4],
                     void* stream) {
  MI_SOLE_COPY();
  const void* ins[2] = {q, k};
  const int64_t* ist[2] = {q_strides, k_strides};
  void* outs[2] = {q_out, k_out};
  const int64_t* ost[2] = {q_out_strides, k_out_strides};
  return rope_common(x_dtype, tab_dtype, S, B, H, D, inverse, 2, ins, ist, outs, ost, cos_tab,
                     cos_strides, sin_tab, sin_strides, stream);
}

mi_status mi_copy_qk(mi_dtype dtype, int S, int B, int H, int D, const void* q,
                     const int64_t q_strides[4], const void* k, const int64_t k_strides[4],
                     void* q_out, const int64_t q_out_strides[4], void* k_out,
                     const int64_t k_out_strides[4], void* stream) {
  MI_SOLE_COPY();
  if (!dtype_ok(dtype)) return fail(MI_ERR_INVALID_ARGUMENT, "unknown dtype %d", dtype);
  if (S <= 0 || B <= 0 || H <= 0 || D <= 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "sizes must be positive (S=%d B=%d H=%d D=%d)", S, B, H, D);
  const int esz = elem_size(dtype);
  if ((D * esz) % 16) return fail(MI_ERR_UNSUPPORTED, "D * element size must be a multiple of 16");
  if ((uint64_t)S * B * H * (D * esz / 16) >= (1ull << 31))
    return fail(MI_ERR_UNSUPPORTED, "tensor too large for one launch");
  const void* ins[2] = {q, k};
  const int64_t* ist[2] = {q_strides, k_strides};
  void* outs[2] = {q_out, k_out};
  const int64_t* ost[2] = {q_out_strides, k_out_strides};
  mi::RopeArgs a = {};
  a.ntensors = 2;
  a.S = S; a.B = B; a.H = H; a.D = D;
  for (int t = 0; t < 2; ++t) {
    if (!ins[t] || !outs[t] || !ist[t] || !ost[t])
      return fail(MI_ERR_INVALID_ARGUMENT, "copy tensor %d: null pointer", t);
    if (ist[t][3] != 1 || ost[t][3] != 1)
      return fail(MI_ERR_UNSUPPORTED, "copy tensor %d: dim stride must be 1", t);
    if (((uintptr_t)ins[t]) % 16 || ((uintptr_t)outs[t]) % 16)
      return fail(MI_ERR_UNSUPPORTED, "copy tensor %d: base not 16-byte aligned", t);
    for (int i = 0; i < 3; ++i)
      if (ist[t][i] < 0 || ost[t][i] < 0 || (ist[t][i] * esz) % 16 || (ost[t][i] * esz) % 16)
        return fail(MI_ERR_UNSUPPORTED, "copy tensor %d: strides must be 16-byte multiples", t);
    mi::RopeTensor& T = a.t[t];
    T.in = ins[t];
    T.out = outs[t];
    T.is_s = ist[t][0]; T.is_b = ist[t][1]; T.is_h = ist[t][2]; T.is_d = 1;
    T.os_s = ost[t][0]; T.os_b = ost[t][1]; T.os_h = ost[t][2]; T.os_d = 1;
  }
  return launched(mi::launch_copy_qk(dtype, a, (hipStream_t)stream), "copy_qk");
}

static mi_status xent_common(mi_dtype dtype, int64_t rows, int64_t vocab, const void* logits,
                             int64_t row_stride, const int64_t* target, mi::XentArgs& a) {
  if (!dtype_ok(dtype)) return fail(MI_ERR_INVALID_ARGUMENT, "unknown dtype %d", dtype);
  if (rows <= 0 || vocab <= 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "sizes must be positive (rows=%lld vocab=%lld)",
                (long long)rows, (long long)vocab);
  if (rows >= (1ll << 31)) return fail(MI_ERR_UNSUPPORTED, "rows = %lld exceeds 2^31", (long long)rows);
  if (row_stride < vocab)
    return fail(MI_ERR_INVALID_ARGUMENT, "row_stride %lld < vocab %lld", (long long)row_stride,
                (long long)vocab);
  if (!logits || !target) return fail(MI_ERR_INVALID_ARGUMENT, "logits / target: null pointer");
  if (((uintptr_t)logits) % elem_size(dtype) || ((uintptr_t)target) % 8)
    return fail(MI_ERR_INVALID_ARGUMENT, "logits / target: misaligned");
  a = {};
  a.logits = logits;
  a.rows = rows;
  a.vocab = vocab;
  a.row_stride = row_stride;
  a.target = target;
  return MI_OK;
}

mi_status mi_xent_fwd(mi_dtype dtype, int64_t rows, int64_t vocab, const void* logits,
                      int64_t row_stride, const int64_t* target, void* loss, float* lse,
                      void* stream) {
  MI_SOLE_COPY();
  mi::XentArgs a;
  if (mi_status st = xent_common(dtype, rows, vocab, logits, row_stride, target, a)) return st;
  if (!loss || !lse) return fail(MI_ERR_INVALID_ARGUMENT, "loss / lse: null pointer");
  if (((uintptr_t)loss) % elem_size(dtype) || ((uintptr_t)lse) % 4)
    return fail(MI_ERR_INVALID_ARGUMENT, "loss / lse: misaligned");
  a.loss = loss;
  a.lse = lse;
  return launched(mi::launch_xent_fwd(dtype, a, (hipStream_t)stream), "xent_fwd");
}

mi_status mi_xent_bwd(mi_dtype dtype, int64_t rows, int64_t vocab, const void* logits,
                      int64_t row_stride, const int64_t* target, const float* lse,
                      const void* grad_loss, void* grad_logits, int64_t grad_row_stride,
                      void* stream) {
  MI_SOLE_COPY();
  mi::XentArgs a;
  if (mi_status st = xent_common(dtype, rows, vocab, logits, row_stride, target, a)) return st;
  if (!lse || !grad_loss || !grad_logits)
    return fail(MI_ERR_INVALID_ARGUMENT, "lse / grad_loss / grad_logits: null pointer");
  if (((uintptr_t)lse) % 4 || ((uintptr_t)grad_loss) % elem_size(dtype) ||
      ((uintptr_t)grad_logits) % elem_size(dtype))
    return fail(MI_ERR_INVALID_ARGUMENT, "lse / grad_loss / grad_logits: misaligned");
  if (grad_row_stride < vocab)
    return fail(MI_ERR_INVALID_ARGUMENT, "grad_row_stride %lld < vocab %lld",
                (long long)grad_row_stride, (long long)vocab);
  if (grad_logits == logits && grad_row_stride != row_stride)
    return fail(MI_ERR_INVALID_ARGUMENT, "in-place backward needs grad_row_stride == row_stride");
  a.lse = (float*)lse;
  a.grad_loss = grad_loss;
  a.grad = grad_logits;
  a.grad_row_stride = grad_row_stride;
  return launched(mi::launch_xent_bwd(dtype, a, (hipStream_t)stream), "xent_bwd");
}

static bool rms_dtypes_ok(int x_dtype, int w_dtype) {
  return dtype_ok(x_dtype) && (w_dtype == x_dtype || w_dtype == MI_F32);
}

static mi_status rms_common(mi_dtype x_dtype, mi_dtype w_dtype, int64_t rows, int64_t hidden,
                            const void* x, int64_t x_row_stride, const void* weight,
                            mi::RmsArgs& a) {
  if (!rms_dtypes_ok(x_dtype, w_dtype))
    return fail(MI_ERR_INVALID_ARGUMENT,
                "dtypes (x %d, weight %d): weight must have x's dtype or be fp32", x_dtype,
                w_dtype);
  if (rows <= 0 || hidden <= 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "sizes must be positive (rows=%lld hidden=%lld)",
                (long long)rows, (long long)hidden);
  if ((rows + 3) / 4 >= (1ll << 31))
    return fail(MI_ERR_UNSUPPORTED, "rows = %lld too many for one launch", (long long)rows);
  if (x_row_stride < hidden)
    return fail(MI_ERR_INVALID_ARGUMENT, "x row stride %lld < hidden %lld",
                (long long)x_row_stride, (long long)hidden);
  if (!x || !weight) return fail(MI_ERR_INVALID_ARGUMENT, "x / weight: null pointer");
  if (((uintptr_t)x) % elem_size(x_dtype) || ((uintptr_t)weight) % elem_size(w_dtype))
    return fail(MI_ERR_INVALID_ARGUMENT, "x / weight: misaligned");
  a = {};
  a.rows = rows;
  a.hidden = hidden;
  a.x = x;
  a.x_stride = x_row_stride;
  a.w = weight;
  return MI_OK;
}

// 4-element vectors: every row of every tensor starts on a 4-element boundary.
static bool rms_vec_ok(int64_t hidden, std::initializer_list<std::pair<const void*, int64_t>> rows,
                       std::initializer_list<std::pair<const void*, int>> bases) {
  if (hidden % 4) return false;
  for (auto& b : bases)
    if (((uintptr_t)b.first) % (4 * b.second)) return false;
  for (auto& r : rows)
    if (r.second % 4) return false;
  return true;
}

// A fused residual add's extra operand: `rows` rows of `hidden` x_dtype
// elements, `stride` apart.
static mi_status rms_add_operand(const char* name, mi_dtype x_dtype, int64_t hidden,
                                 const void* p, int64_t stride) {
  if (!p) return fail(MI_ERR_INVALID_ARGUMENT, "%s: null pointer", name);
  if (stride < hidden)
    return fail(MI_ERR_INVALID_ARGUMENT, "%s row stride %lld < hidden %lld", name,
                (long long)stride, (long long)hidden);
  if (((uintptr_t)p) % elem_size(x_dtype))
    return fail(MI_ERR_INVALID_ARGUMENT, "%s: misaligned", name);
  return MI_OK;
}

static mi_status rms_fwd(mi_dtype x_dtype, mi_dtype w_dtype, int64_t rows, int64_t hidden,
                         float eps, const void* x, int64_t x_row_stride, const void* res,
                         int64_t res_row_stride, const void* weight, void* sum,
                         int64_t sum_row_stride, void* y, int64_t y_row_stride, float* rstd,
                         void* stream) {
  mi::RmsArgs a;
  if (mi_status st = rms_common(x_dtype, w_dtype, rows, hidden, x, x_row_stride, weight, a))
    return st;
  const bool add = res != nullptr || sum != nullptr;
  if (add) {
    if (mi_status st = rms_add_operand("residual", x_dtype, hidden, res, res_row_stride)) return st;
    if (mi_status st = rms_add_operand("sum", x_dtype, hidden, sum, sum_row_stride)) return st;
    a.res = res;
    a.res_stride = res_row_stride;
    a.sum = sum;
    a.sum_stride = sum_row_stride;
  }
  if (!(eps >= 0.f) || !std::isfinite(eps))
    return fail(MI_ERR_INVALID_ARGUMENT, "eps must be a finite number >= 0");
  const int y_dtype = w_dtype == MI_F32 ? MI_F32 : x_dtype;
  if (!y || !rstd) return fail(MI_ERR_INVALID_ARGUMENT, "y / rstd: null pointer");
  if (y_row_stride < hidden)
    return fail(MI_ERR_INVALID_ARGUMENT, "y row stride %lld < hidden %lld",
                (long long)y_row_stride, (long long)hidden);
  if (((uintptr_t)y) % elem_size(y_dtype) || ((uintptr_t)rstd) % 4)
    return fail(MI_ERR_INVALID_ARGUMENT, "y / rstd: misaligned");
  a.eps = eps;
  a.y = y;
  a.y_stride = y_row_stride;
  a.rstd = rstd;
  bool vec = rms_vec_ok(hidden, {{x, x_row_stride}, {y, y_row_stride}},
                        {{x, elem_size(x_dtype)}, {y, elem_size(y_dtype)},
                         {weight, elem_size(w_dtype)}});
  if (add)
    vec = vec && rms_vec_ok(hidden, {{res, res_row_stride}, {sum, sum_row_stride}},
                            {{res, elem_size(x_dtype)}, {sum, elem_size(x_dtype)}});
  // 16-byte accesses: bf16 x, every row of every operand 8-element aligned
  if (vec && x_dtype == MI_BF16 && hidden % 8 == 0) {
    bool v16 = x_row_stride % 8 == 0 && y_row_stride % 8 == 0 && ((uintptr_t)x) % 16 == 0 &&
               ((uintptr_t)y) % 16 == 0 && ((uintptr_t)weight) % 16 == 0;
    if (add)
      v16 = v16 && res_row_stride % 8 == 0 && sum_row_stride % 8 == 0 &&
            ((uintptr_t)res) % 16 == 0 && ((uintptr_t)sum) % 16 == 0;
    a.vec16 = v16;
  }
  return launched(mi::launch_rmsnorm_fwd(x_dtype, w_dtype, a, vec, (hipStream_t)stream),
                  add ? "rmsnorm_add_fwd" : "rmsnorm_fwd");
}

mi_status mi_rmsnorm_fwd(mi_dtype x_dtype, mi_dtype w_dtype, int64_t rows, int64_t hidden,
                         float eps, const void* x, int64_t x_row_stride, const void* weight,
                         void* y, int64_t y_row_stride, float* rstd, void* stream) {
  MI_SOLE_COPY();
  return rms_fwd(x_dtype, w_dtype, rows, hidden, eps, x, x_row_stride, nullptr, 0, weight,
                 nullptr, 0, y, y_row_stride, rstd, stream);
}

mi_status mi_rmsnorm_add_fwd(mi_dtype x_dtype, mi_dtype w_dtype, int64_t rows, int64_t hidden,
                             float eps, const void* x, int64_t x_row_stride, const void* res,
                             int64_t res_row_stride, const void* weight, void* sum,
                             int64_t sum_row_stride, void* y, int64_t y_row_stride, float* rstd,
                             void* stream) {
  MI_SOLE_COPY();
  if (!res || !sum) return fail(MI_ERR_INVALID_ARGUMENT, "residual / sum: null pointer");
  return rms_fwd(x_dtype, w_dtype, rows, hidden, eps, x, x_row_stride, res, res_row_stride,
                 weight, sum, sum_row_stride, y, y_row_stride, rstd, stream);
}

int64_t mi_rmsnorm_bwd_workspace(int64_t rows, int64_t hidden) {
  if (rows <= 0 || hidden <= 0) return 0;
  return mi::rmsnorm_parts(rows) * hidden;
}

static mi_status rms_bwd(mi_dtype x_dtype, mi_dtype w_dtype, int64_t rows, int64_t hidden,
                         const void* x, int64_t x_row_stride, const void* weight,
                         const float* rstd, const void* dy, int64_t dy_row_stride,
                         const void* dsum, int64_t dsum_row_stride, void* dx,
                         int64_t dx_row_stride, void* dweight, float* workspace,
                         int64_t workspace_elems, void* stream, bool dw_acc = false) {
  mi::RmsArgs a;
  if (mi_status st = rms_common(x_dtype, w_dtype, rows, hidden, x, x_row_stride, weight, a))
    return st;
  if (dsum) {
    if (mi_status st = rms_add_operand("dsum", x_dtype, hidden, dsum, dsum_row_stride)) return st;
    a.dsum = dsum;
    a.dsum_stride = dsum_row_stride;
  }
  const int y_dtype = w_dtype == MI_F32 ? MI_F32 : x_dtype;
  if (!rstd || !dy || !dx || !dweight || !workspace)
    return fail(MI_ERR_INVALID_ARGUMENT, "rstd / dy / dx / dweight / workspace: null pointer");
  if (dy_row_stride < hidden || dx_row_stride < hidden)
    return fail(MI_ERR_INVALID_ARGUMENT, "dy / dx row stride < hidden %lld", (long long)hidden);
  if (((uintptr_t)rstd) % 4 || ((uintptr_t)workspace) % 4 ||
      ((uintptr_t)dy) % elem_size(y_dtype) || ((uintptr_t)dx) % elem_size(x_dtype) ||
      ((uintptr_t)dweight) % elem_size(w_dtype))
    return fail(MI_ERR_INVALID_ARGUMENT, "rstd / dy / dx / dweight / workspace: misaligned");
  const int64_t need = mi_rmsnorm_bwd_workspace(rows, hidden);
  if (workspace_elems < need)
    return fail(MI_ERR_INVALID_ARGUMENT, "workspace holds %lld floats, %lld needed",
                (long long)workspace_elems, (long long)need);
  a.rstd = (float*)rstd;
  a.dy = dy;
  a.dy_stride = dy_row_stride;
  a.dx = dx;
  a.dx_stride = dx_row_stride;
  a.dw = dweight;
  a.dw_acc = dw_acc ? 1 : 0;
  a.partial = workspace;
  a.parts = (int)mi::rmsnorm_parts(rows);
  bool vec = rms_vec_ok(hidden, {{x, x_row_stride}, {dy, dy_row_stride}, {dx, dx_row_stride}},
                        {{x, elem_size(x_dtype)}, {dy, elem_size(y_dtype)},
                         {dx, elem_size(x_dtype)}, {weight, elem_size(w_dtype)}});
  if (dsum)
    vec = vec && rms_vec_ok(hidden, {{dsum, dsum_row_stride}}, {{dsum, elem_size(x_dtype)}});
  return launched(mi::launch_rmsnorm_bwd(x_dtype, w_dtype, a, vec, (hipStream_t)stream),
                  dsum ? "rmsnorm_add_bwd" : "rmsnorm_bwd");
}

mi_status mi_rmsnorm_bwd(mi_dtype x_dtype, mi_dtype w_dtype, int64_t rows, int64_t hidden,
                         const void* x, int64_t x_row_stride, const void* weight,
                         const float* rstd, const void* dy, int64_t dy_row_stride, void* dx,
                         int64_t dx_row_stride, void* dweight, float* workspace,
                         int64_t workspace_elems, void* stream) {
  MI_SOLE_COPY();
  return rms_bwd(x_dtype, w_dtype, rows, hidden, x, x_row_stride, weight, rstd, dy,
                 dy_row_stride, nullptr, 0, dx, dx_row_stride, dweight, workspace,
                 workspace_elems, stream);
}

mi_status mi_rmsnorm_add_bwd(mi_dtype x_dtype, mi_dtype w_dtype, int64_t rows, int64_t hidden,
                             const void* sum, int64_t sum_row_stride, const void* weight,
                             const float* rstd, const void* dy, int64_t dy_row_stride,
                             const void* dsum, int64_t dsum_row_stride, void* dx,
                             int64_t dx_row_stride, void* dweight, float* workspace,
                             int64_t workspace_elems, void* stream) {
  MI_SOLE_COPY();
  if (!dsum) return fail(MI_ERR_INVALID_ARGUMENT, "dsum: null pointer");
  return rms_bwd(x_dtype, w_dtype, rows, hidden, sum, sum_row_stride, weight, rstd, dy,
                 dy_row_stride, dsum, dsum_row_stride, dx, dx_row_stride, dweight, workspace,
                 workspace_elems, stream);
}

mi_status mi_rmsnorm_bwd_acc(mi_dtype x_dtype, mi_dtype w_dtype, int64_t rows, int64_t hidden,
                             const void* x, int64_t x_row_stride, const void* weight,
                             const float* rstd, const void* dy, int64_t dy_row_stride, void* dx,
                             int64_t dx_row_stride, void* dweight, float* workspace,
                             int64_t workspace_elems, void* stream) {
  MI_SOLE_COPY();
  return rms_bwd(x_dtype, w_dtype, rows, hidden, x, x_row_stride, weight, rstd, dy,
                 dy_row_stride, nullptr, 0, dx, dx_row_stride, dweight, workspace,
                 workspace_elems, stream, true);
}

mi_status mi_rmsnorm_add_bwd_acc(mi_dtype x_dtype, mi_dtype w_dtype, int64_t rows,
                                 int64_t hidden, const void* sum, int64_t sum_row_stride,
                                 const void* weight, const float* rstd, const void* dy,
                                 int64_t dy_row_stride, const void* dsum, int64_t dsum_row_stride,
                                 void* dx, int64_t dx_row_stride, void* dweight, float* workspace,
                                 int64_t workspace_elems, void* stream) {
  MI_SOLE_COPY();
  if (!dsum) return fail(MI_ERR_INVALID_ARGUMENT, "dsum: null pointer");
  return rms_bwd(x_dtype, w_dtype, rows, hidden, sum, sum_row_stride, weight, rstd, dy,
                 dy_row_stride, dsum, dsum_row_stride, dx, dx_row_stride, dweight, workspace,
                 workspace_elems, stream, true);
}

static mi_status swiglu_common(mi_dtype dtype, int64_t rows, int64_t inter, const void* gu,
                               int64_t gu_stride, void* out, int64_t out_stride,
                               int64_t out_min_stride) {
  if (!dtype_ok(dtype)) return fail(MI_ERR_INVALID_ARGUMENT, "unknown dtype %d", dtype);
  if (rows <= 0 || inter <= 0)
    return fail(MI_ERR_INVALID_ARGUMENT, "sizes must be positive (rows=%lld inter=%lld)",
                (long long)rows, (long long)inter);
  if (gu_stride < 2 * inter || out_stride < out_min_stride)
    return fail(MI_ERR_INVALID_ARGUMENT, "row strides (%lld, %lld) shorter than the rows",
                (long long)gu_stride, (long long)out_stride);
  if ((inter + 127) / 128 >= (1ll << 31))
    return fail(MI_ERR_UNSUPPORTED, "inter = %lld too large", (long long)inter);
  if (!gu || !out) return fail(MI_ERR_INVALID_ARGUMENT, "gate_up / out: null pointer");
  if (((uintptr_t)gu) % elem_size(dtype) || ((uintptr_t)out) % elem_size(dtype))
    return fail(MI_ERR_INVALID_ARGUMENT, "gate_up / out: misaligned");
  return MI_OK;
}

// 8-element vectors: every row of every tensor starts on a 16-byte boundary
// for 16-bit types (32 bytes for fp32, loaded as two 16-byte halves).
static bool swiglu_vec_ok(int dtype, int64_t inter, std::initializer_list<const void*> ptrs,
                          std::initializer_list<int64_t> strides) {
  const int esz = elem_size(dtype);
  if (inter % 8) return false;
  for (const void* p : ptrs)
    if (((uintptr_t)p) % (4 * esz) || (((uintptr_t)p) % 16 && esz == 2)) return false;
  for (int64_t s : strides)
    if (s % 8) return false;
  return true;
}

mi_status mi_swiglu_fwd(mi_dtype dtype, int64_t rows, int64_t inter, const void* gate_up,
                        int64_t gate_up_row_stride, void* out, int64_t out_row_stride,
                        void* stream) {
  MI_SOLE_COPY();
  if (mi_status st = swiglu_common(dtype, rows, inter, gate_up, gate_up_row_stride, out,
                                   out_row_stride, inter))
    return st;
  const bool vec = swiglu_vec_ok(dtype, inter, {gate_up, out},
                                 {gate_up_row_stride, out_row_stride});
  return launched(mi::launch_swiglu(false, dtype, rows, inter, gate_up, gate_up_row_stride,
                                    nullptr, 0, out, out_row_stride, vec, (hipStream_t)stream),
                  "swiglu_fwd");
}

mi_status mi_swiglu_bwd(mi_dtype dtype, int64_t rows, int64_t inter, const void* gate_up,
                        int64_t gate_up_row_stride, const void* dout, int64_t dout_row_stride,
                        void* dgate_up, int64_t dgate_up_row_stride, void* stream) {
  MI_SOLE_COPY();
  if (mi_status st = swiglu_common(dtype, rows, inter, gate_up, gate_up_row_stride, dgate_up,
                                   dgate_up_row_stride, 2 * inter))
    return st;
  if (!dout) return fail(MI_ERR_INVALID_ARGUMENT, "dout: null pointer");
  if (dout_row_stride < inter)
    return fail(MI_ERR_INVALID_ARGUMENT, "dout row stride %lld < inter %lld",
                (long long)dout_row_stride, (long long)inter);
  if (((uintptr_t)dout) % elem_size(dtype))
    return fail(MI_ERR_INVALID_ARGUMENT, "dout: misaligned");
  const bool vec = swiglu_vec_ok(dtype, inter, {gate_up, dout, dgate_up},
                                 {gate_up_row_stride, dout_row_stride, dgate_up_row_stride});
  return launched(mi::launch_swiglu(true, dtype, rows, inter, gate_up, gate_up_row_stride, dout,
                                    dout_row_stride, dgate_up, dgate_up_row_stride, vec,
                                    (hipStream_t)stream),
                  "swiglu_bwd");
}

int64_t mi_adamw_workspace(void) { return 1 + mi::adam_parts(); }

mi_status mi_grad_sumsq(mi_dtype grad_dtype, int64_t n, const void* grad, float* workspace,
                        int64_t workspace_elems, void* stream) {
  MI_SOLE_COPY();
  if (!dtype_ok(grad_dtype)) return fail(MI_ERR_INVALID_ARGUMENT, "unknown dtype %d", grad_dtype);
  if (n <= 0) return fail(MI_ERR_INVALID_ARGUMENT, "n must be positive (got %lld)", (long long)n);
  if (!grad || !workspace) return fail(MI_ERR_INVALID_ARGUMENT, "grad / workspace: null pointer");
  if (((uintptr_t)grad) % elem_size(grad_dtype) || ((uintptr_t)workspace) % 4)
    return fail(MI_ERR_INVALID_ARGUMENT, "grad / workspace: misaligned");
  if (workspace_elems < mi_adamw_workspace())
    return fail(MI_ERR_INVALID_ARGUMENT, "workspace holds %lld floats, %lld needed",
                (long long)workspace_elems, (long long)mi_adamw_workspace());
  const bool vec = ((uintptr_t)grad) % 16 == 0;
  return launched(mi::launch_grad_sumsq(grad_dtype, n, grad, vec, workspace, workspace + 1,
                                        (hipStream_t)stream),
                  "grad_sumsq");
}

mi_status mi_adamw_step(mi_dtype grad_dtype, mi_dtype param_dtype, int64_t n, const void* grad,
                        float* master, float* exp_avg, float* exp_avg_sq, void* param,
                        float weight_decay_factor, float lerp_weight, float beta2,
                        float one_minus_beta2, float step_size, float bias_correction2_sqrt,
                        float eps, float clip, const float* grad_sumsq, void* stream) {
  MI_SOLE_COPY();
  if (!dtype_ok(grad_dtype) || !dtype_ok(param_dtype))
    return fail(MI_ERR_INVALID_ARGUMENT, "unknown dtype (grad %d, param %d)", grad_dtype,
                param_dtype);
  if (n <= 0) return fail(MI_ERR_INVALID_ARGUMENT, "n must be positive (got %lld)", (long long)n);
  if (!grad || !master || !exp_avg || !exp_avg_sq)
    return fail(MI_ERR_INVALID_ARGUMENT, "grad / master / exp_avg / exp_avg_sq: null pointer");
  if (((uintptr_t)grad) % elem_size(grad_dtype) || ((uintptr_t)master) % 4 ||
      ((uintptr_t)exp_avg) % 4 || ((uintptr_t)exp_avg_sq) % 4 ||
      ((uintptr_t)param) % elem_size(param_dtype))
    return fail(MI_ERR_INVALID_ARGUMENT, "a buffer is misaligned");
  const float hp[8] = {weight_decay_factor, lerp_weight, beta2, one_minus_beta2, step_size,
                       bias_correction2_sqrt, eps, clip};
  for (float x : hp)
    if (!std::isfinite(x)) return fail(MI_ERR_INVALID_ARGUMENT, "hyperparameters must be finite");
  if (!(bias_correction2_sqrt > 0.f))
    return fail(MI_ERR_INVALID_ARGUMENT, "bias_correction2_sqrt must be positive");
  if (clip > 0.f && !grad_sumsq)
    return fail(MI_ERR_INVALID_ARGUMENT, "clip > 0 needs grad_sumsq (from mi_grad_sumsq)");
  const uintptr_t al = 16;
  const bool vec = ((uintptr_t)grad) % (4 * elem_size(grad_dtype)) == 0 &&
                   ((uintptr_t)master) % al == 0 && ((uintptr_t)exp_avg) % al == 0 &&
                   ((uintptr_t)exp_avg_sq) % al == 0 &&
                   ((uintptr_t)param) % (4 * elem_size(param_dtype)) == 0;
  return launched(mi::launch_adamw_step(grad_dtype, param_dtype, n, grad, master, exp_avg,
                                        exp_avg_sq, param, hp, grad_sumsq, vec,
                                        (hipStream_t)stream),
                  "adamw_step");
}

}  // extern "C"

// ---------------------------------------------------------------------------
// mi_attn_bwd_noalloc: the workspace of mi_attn_bwd taken from a static
// device array instead of the caller.  `scratch` names a host-side stand-in
// for the array in host code, so host code only ever uses the per-device
// address that hipGetSymbolAddress returns (kept in g_scratch).
// ---------------------------------------------------------------------------
namespace {

__device__ __attribute__((aligned(256))) float scratch[2 * MI_ATTN_NOALLOC_MAX_ROWS];

constexpr int kMaxDevices = 64;
std::atomic<float*> g_scratch[kMaxDevices];

// Device address of `scratch` on the device `stream` belongs to, looked up
// once per device with that device current (threads that race here store the
// same address).
mi_status scratch_on(void* stream, float** out) {
  int dev = -1;
  hipError_t e = hipStreamGetDevice((hipStream_t)stream, &dev);
  if (e != hipSuccess) return fail(MI_ERR_LAUNCH, "hipStreamGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(MI_ERR_UNSUPPORTED, "device %d: at most %d devices", dev, kMaxDevices);
  float* p = g_scratch[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    int cur = -1;
    if ((e = hipGetDevice(&cur)) != hipSuccess)
      return fail(MI_ERR_LAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess)
      return fail(MI_ERR_LAUNCH, "hipSetDevice(%d): %s", dev, hipGetErrorString(e));
    void* addr = nullptr;
    const hipError_t es = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (cur != dev && (e = hipSetDevice(cur)) != hipSuccess)
      return fail(MI_ERR_LAUNCH, "hipSetDevice(%d): %s", cur, hipGetErrorString(e));
    if (es != hipSuccess || addr == nullptr)
      return fail(MI_ERR_LAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                  hipGetErrorString(es));
    p = (float*)addr;
    g_scratch[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return MI_OK;
}

}  // namespace

extern "C" mi_status mi_attn_bwd_noalloc(
    mi_dtype dtype, int B, int H, int S, int D, int causal, float scale, const void* q,
    const int64_t q_strides[4], const void* k, const int64_t k_strides[4], const void* v,
    const int64_t v_strides[4], const void* o, const int64_t o_strides[4], const void* dout,
    const int64_t dout_strides[4], const float* lse, void* dq, const int64_t dq_strides[4],
    void* dk, const int64_t dk_strides[4], void* dv, const int64_t dv_strides[4], void* stream) {
  MI_SOLE_COPY();
  mi_status st;
  if ((st = check_shape(dtype, B, H, S, D, scale)) != MI_OK) return st;
  const int64_t rows = (int64_t)B * H * S;
  if (rows > MI_ATTN_NOALLOC_MAX_ROWS)
    return fail(MI_ERR_INVALID_ARGUMENT,
                "B*H*S = %lld exceeds MI_ATTN_NOALLOC_MAX_ROWS = %d (the static workspace)",
                (long long)rows, MI_ATTN_NOALLOC_MAX_ROWS);
  float* ws = nullptr;
  if ((st = scratch_on(stream, &ws)) != MI_OK) return st;
  // mi_attn_bwd validates every other argument before it enqueues anything;
  // the preprocess overwrites ws[0, 2 * rows) before the gradient launch reads it.
  return mi_attn_bwd(dtype, B, H, S, D, causal, scale, q, q_strides, k, k_strides, v, v_strides,
                     o, o_strides, dout, dout_strides, lse, ws, dq, dq_strides, dk, dk_strides,
                     dv, dv_strides, stream);
}
