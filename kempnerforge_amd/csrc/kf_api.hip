// C ABI entry points (declared in include/kf_attn.h).  Host-side argument
// checks happen here, before any launch, so that every kernel only ever sees
// shapes its grid and indexing were written for.
#include <stdarg.h>
#include <stdio.h>

#include "kf_common.h"
#include "kf_internal.h"

#include <atomic>

namespace kf {

static thread_local char g_err[512] = "";

int device_cu_count() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

static int check_common(int B, int Sq, int Sk, int Hq, int Hkv, int D, int dtype) {
  KF_CHECK_ARG(B > 0 && Sq > 0 && Sk > 0, "B, Sq, Sk must be positive (got %d, %d, %d)", B, Sq,
               Sk);
  KF_CHECK_ARG(Hq > 0 && Hkv > 0 && Hq % Hkv == 0,
               "n_heads (%d) must be a positive multiple of n_kv_heads (%d)", Hq, Hkv);
  KF_CHECK_ARG(D > 0 && D % 2 == 0 && D <= 256, "head_dim must be even and <= 256 (got %d)", D);
  KF_CHECK_ARG(dtype == F32 || dtype == BF16 || dtype == F16, "unsupported dtype code %d", dtype);
  return KF_OK;
}

static FwdArgs make_fwd(const void* q, const void* k, const void* v, const float* cos,
                        const float* sin, void* out, float* lse, int B, int Sq, int Sk, int Hq,
                        int Hkv, int D, int64_t ksb, int64_t kss, int64_t ksh, int64_t vsb,
                        int64_t vss, int64_t vsh, int k_rotated, int causal,
                        const int32_t* doc, const int32_t* kvalid, int dtype, void* stream) {
  FwdArgs a;
  a.q = q; a.k = k; a.v = v; a.cos = cos; a.sin = sin; a.out = out; a.lse = lse;
  a.B = B; a.Sq = Sq; a.Sk = Sk; a.Hq = Hq; a.Hkv = Hkv; a.D = D;
  a.ksb = ksb; a.kss = kss; a.ksh = ksh; a.vsb = vsb; a.vss = vss; a.vsh = vsh;
  a.k_rotated = k_rotated; a.causal = causal; a.doc = doc; a.kvalid = kvalid; a.dtype = dtype;
  a.scale = 1.0f / sqrtf((float)D);
  a.stream = (hipStream_t)stream;
  return a;
}

// Explicit masks: the reference builds causal & same-document & valid-key
// masks only for full-sequence self-attention (kempnerforge/model/
// attention.py:204-227, kempnerforge/model/mot.py:188-198).
static int check_masks(const int32_t* doc, const int32_t* kvalid, int causal, int Sq, int Sk,
                       int k_rotated) {
  if (!doc && !kvalid) return KF_OK;
  KF_CHECK_ARG(causal && Sq == Sk && !k_rotated,
               "doc_ids / key_valid need causal self-attention over un-rotated keys (Sq == Sk)");
  return KF_OK;
}

static size_t fwd_ws(const FwdArgs& a) {
  if (fwd_mfma_supported(a)) return fwd_mfma_workspace(a.B, a.Sk, a.Hkv, a.D);
  if (fwd_f32_supported(a)) return a.k_rotated ? 0 : fwd_f32_workspace(a.B, a.Sk, a.Hkv, a.D);
  return 0;
}

static size_t bwd_ws(const BwdArgs& a) {
  if (bwd_mfma_supported(a)) return bwd_mfma_workspace(a.B, a.S, a.Hq, a.Hkv, a.D);
  if (bwd_f32_supported(a)) return bwd_f32_workspace(a.B, a.S, a.Hq, a.Hkv, a.D);
  return bwd_generic_workspace(a.B, a.S, a.Hq);
}

}  // namespace kf

using namespace kf;

extern "C" {

int kf_version(void) { return 100; }

const char* kf_last_error(void) { return g_err; }

int kf_attn_fwd_workspace_size(int B, int Sq, int Sk, int Hq, int Hkv, int D, int dtype,
                               size_t* bytes) {
  int rc = check_common(B, Sq, Sk, Hq, Hkv, D, dtype);
  if (rc) return rc;
  KF_CHECK_ARG(bytes != nullptr, "bytes is null");
  // Contiguous BSHD strides and aligned pointers are assumed for the estimate;
  // a call that falls back to the generic kernels needs no workspace.
  FwdArgs a = make_fwd((void*)16, (void*)16, (void*)16, (float*)16, (float*)16, (void*)16,
                       nullptr, B, Sq, Sk, Hq, Hkv, D, (int64_t)Sk * Hkv * D, (int64_t)Hkv * D, D,
                       (int64_t)Sk * Hkv * D, (int64_t)Hkv * D, D, 0, 1, nullptr, nullptr, dtype,
                       nullptr);
  *bytes = fwd_ws(a);
  return KF_OK;
}

int kf_attn_fwd(const void* q, const void* k, const void* v, const float* rope_cos,
                const float* rope_sin, void* out, float* lse, void* workspace,
                size_t workspace_bytes, int B, int Sq, int Sk, int Hq, int Hkv, int D,
                int64_t ksb, int64_t kss, int64_t ksh, int64_t vsb, int64_t vss, int64_t vsh,
                int k_rotated, int causal, const int32_t* doc_ids, const int32_t* key_valid,
                int dtype, void* stream) {
  int rc = check_common(B, Sq, Sk, Hq, Hkv, D, dtype);
  if (rc) return rc;
  KF_CHECK_ARG(q && k && v && rope_cos && rope_sin && out, "null tensor pointer");
  KF_CHECK_ARG(k_rotated || Sk == Sq, "un-rotated keys need Sk == Sq (got %d, %d)", Sk, Sq);
  rc = check_masks(doc_ids, key_valid, causal, Sq, Sk, k_rotated);
  if (rc) return rc;
  FwdArgs a = make_fwd(q, k, v, rope_cos, rope_sin, out, lse, B, Sq, Sk, Hq, Hkv, D, ksb, kss,
                       ksh, vsb, vss, vsh, k_rotated, causal, doc_ids, key_valid, dtype, stream);
  if (fwd_mfma_supported(a)) {
    const size_t need = fwd_mfma_workspace(B, Sk, Hkv, D);
    if (workspace_bytes < need || (need && !workspace)) {
      set_error("workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
      return KF_ERR_WORKSPACE;
    }
    return fwd_mfma(a, workspace);
  }
  if (fwd_f32_supported(a)) {
    const size_t need = fwd_ws(a);
    if (workspace_bytes < need || (need && !workspace)) {
      set_error("workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
      return KF_ERR_WORKSPACE;
    }
    return fwd_f32(a, workspace);
  }
  return fwd_generic(a);
}

}  // extern "C"

namespace {
// Sizing stand-in for a backward call: aligned non-null pointers, no masks.
kf::BwdArgs sizing_args(int B, int S, int Hq, int Hkv, int D, int dtype, int causal) {
  kf::BwdArgs a{};
  a.B = B; a.S = S; a.Hq = Hq; a.Hkv = Hkv; a.D = D; a.dtype = dtype; a.causal = causal;
  a.q = a.k = a.v = a.out = a.dout = (void*)16;
  a.dq = a.dk = a.dv = (void*)16;
  a.cos = a.sin = (float*)16;
  return a;
}
}  // namespace

extern "C" {

int kf_attn_bwd_workspace_size(int B, int S, int Hq, int Hkv, int D, int dtype, size_t* bytes) {
  int rc = check_common(B, S, S, Hq, Hkv, D, dtype);
  if (rc) return rc;
  KF_CHECK_ARG(bytes != nullptr, "bytes is null");
  const BwdArgs a = sizing_args(B, S, Hq, Hkv, D, dtype, 1);
  *bytes = bwd_ws(a);
  return KF_OK;
}

int kf_attn_bwd_workspace_size_ds(int B, int S, int Hq, int Hkv, int D, int dtype, int causal,
                                  size_t* bytes) {
  int rc = check_common(B, S, S, Hq, Hkv, D, dtype);
  if (rc) return rc;
  KF_CHECK_ARG(bytes != nullptr, "bytes is null");
  const BwdArgs a = sizing_args(B, S, Hq, Hkv, D, dtype, causal);
  *bytes = bwd_mfma_supported(a)  ? bwd_mfma_workspace_ds(a)
           : bwd_f32_supported(a) ? bwd_f32_workspace_ds(B, S, Hq, Hkv, D, causal)
                                  : bwd_ws(a);
  return KF_OK;
}

int kf_attn_bwd(const void* q, const void* k, const void* v, const float* rope_cos,
                const float* rope_sin, const void* out, const float* lse, const void* dout,
                void* dq, void* dk, void* dv, void* workspace, size_t workspace_bytes, int B,
                int S, int Hq, int Hkv, int D, int causal, const int32_t* doc_ids,
                const int32_t* key_valid, int dtype, void* stream) {
  int rc = check_common(B, S, S, Hq, Hkv, D, dtype);
  if (rc) return rc;
  KF_CHECK_ARG(q && k && v && rope_cos && rope_sin && out && lse && dout && dq && dk && dv,
               "null tensor pointer");
  rc = check_masks(doc_ids, key_valid, causal, S, S, 0);
  if (rc) return rc;
  BwdArgs a;
  a.q = q; a.k = k; a.v = v; a.cos = rope_cos; a.sin = rope_sin; a.out = out; a.lse = lse;
  a.dout = dout; a.dq = dq; a.dk = dk; a.dv = dv;
  a.B = B; a.S = S; a.Hq = Hq; a.Hkv = Hkv; a.D = D; a.causal = causal; a.dtype = dtype;
  a.doc = doc_ids;
  a.kvalid = key_valid;
  a.scale = 1.0f / sqrtf((float)D);
  a.stream = (hipStream_t)stream;
  if (bwd_mfma_supported(a)) {
    const size_t need = bwd_mfma_workspace(B, S, Hq, Hkv, D);
    if (workspace_bytes < need || !workspace) {
      set_error("workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
      return KF_ERR_WORKSPACE;
    }
    return bwd_mfma(a, workspace, workspace_bytes);
  }
  const size_t need = bwd_ws(a);
  if (workspace_bytes < need || !workspace) {
    set_error("workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
    return KF_ERR_WORKSPACE;
  }
  if (bwd_f32_supported(a)) return bwd_f32(a, workspace, workspace_bytes);
  return bwd_generic(a, workspace);
}

// Whether the rotated-operand pair (kf_attn_fwd_rot / kf_attn_bwd_rot) takes
// these sizes, dtype and mask kinds: both MFMA paths, pointer alignment aside.
static bool rot_supported(int B, int S, int Hq, int Hkv, int D, int dtype, int has_doc,
                          int has_key_valid) {
  FwdArgs f = make_fwd((void*)16, (void*)16, (void*)16, (float*)16, (float*)16, (void*)16,
                       (float*)16, B, S, S, Hq, Hkv, D, (int64_t)S * Hkv * D, (int64_t)Hkv * D,
                       D, (int64_t)S * Hkv * D, (int64_t)Hkv * D, D, 0, 1,
                       has_doc ? (const int32_t*)16 : nullptr,
                       has_key_valid ? (const int32_t*)16 : nullptr, dtype, nullptr);
  BwdArgs b = sizing_args(B, S, Hq, Hkv, D, dtype, 1);
  b.doc = f.doc;
  b.kvalid = f.kvalid;
  return fwd_mfma_supported(f) && bwd_mfma_supported(b);
}

int kf_attn_rot_size(int B, int S, int Hq, int Hkv, int D, int dtype, int has_doc,
                     int has_key_valid, size_t* bytes) {
  int rc = check_common(B, S, S, Hq, Hkv, D, dtype);
  if (rc) return rc;
  KF_CHECK_ARG(bytes != nullptr, "bytes is null");
  if (!rot_supported(B, S, Hq, Hkv, D, dtype, has_doc, has_key_valid)) {
    set_error(
        "the rotated-operand path needs bf16 or fp16, head_dim 64 or 128 and one mask kind at most");
    return KF_ERR_UNSUPPORTED;
  }
  *bytes = rot_bytes(B, S, Hq, Hkv, D);
  return KF_OK;
}

int kf_attn_fwd_rot(const void* q, const void* k, const void* v, const float* rope_cos,
                    const float* rope_sin, void* out, float* lse, void* rot, void* workspace,
                    size_t workspace_bytes, int B, int S, int Hq, int Hkv, int D, int causal,
                    const int32_t* doc_ids, const int32_t* key_valid, int dtype, void* stream) {
  int rc = check_common(B, S, S, Hq, Hkv, D, dtype);
  if (rc) return rc;
  KF_CHECK_ARG(q && k && v && rope_cos && rope_sin && out && lse && rot, "null tensor pointer");
  rc = check_masks(doc_ids, key_valid, causal, S, S, 0);
  if (rc) return rc;
  FwdArgs a = make_fwd(q, k, v, rope_cos, rope_sin, out, lse, B, S, S, Hq, Hkv, D,
                       (int64_t)S * Hkv * D, (int64_t)Hkv * D, D, (int64_t)S * Hkv * D,
                       (int64_t)Hkv * D, D, 0, causal, doc_ids, key_valid, dtype, stream);
  if (!rot_supported(B, S, Hq, Hkv, D, dtype, doc_ids != nullptr, key_valid != nullptr) ||
      !fwd_mfma_supported(a) || ((uintptr_t)rot & 15) != 0) {
    set_error("kf_attn_fwd_rot needs the MFMA path (sizes as kf_attn_rot_size accepts, "
              "16-byte aligned pointers)");
    return KF_ERR_UNSUPPORTED;
  }
  a.rot = rot;
  const size_t need = fwd_mfma_workspace(B, S, Hkv, D);
  if (workspace_bytes < need || !workspace) {
    set_error("workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
    return KF_ERR_WORKSPACE;
  }
  return fwd_mfma(a, workspace);
}

int kf_attn_bwd_rot_workspace_size(int B, int S, int Hq, int Hkv, int D, int dtype, int causal,
                                   int with_ds, size_t* bytes) {
  int rc = check_common(B, S, S, Hq, Hkv, D, dtype);
  if (rc) return rc;
  KF_CHECK_ARG(bytes != nullptr, "bytes is null");
  if (!rot_supported(B, S, Hq, Hkv, D, dtype, 0, 0)) {
    set_error("the rotated-operand path needs bf16 or fp16 and head_dim 64 or 128");
    return KF_ERR_UNSUPPORTED;
  }
  BwdArgs a = sizing_args(B, S, Hq, Hkv, D, dtype, causal);
  a.rot = (const void*)16;
  *bytes = with_ds ? bwd_mfma_workspace_ds(a) : bwd_mfma_workspace(B, S, Hq, Hkv, D, true);
  return KF_OK;
}

int kf_attn_bwd_rot(const void* rot, const void* v, const float* rope_cos, const float* rope_sin,
                    const void* out, const float* lse, const void* dout, void* dq, void* dk,
                    void* dv, void* workspace, size_t workspace_bytes, int B, int S, int Hq,
                    int Hkv, int D, int causal, const int32_t* doc_ids, const int32_t* key_valid,
                    int dtype, void* stream) {
  int rc = check_common(B, S, S, Hq, Hkv, D, dtype);
  if (rc) return rc;
  KF_CHECK_ARG(rot && v && rope_cos && rope_sin && out && lse && dout && dq && dk && dv,
               "null tensor pointer");
  rc = check_masks(doc_ids, key_valid, causal, S, S, 0);
  if (rc) return rc;
  BwdArgs a;
  a.q = nullptr; a.k = nullptr; a.rot = rot;
  a.v = v; a.cos = rope_cos; a.sin = rope_sin; a.out = out; a.lse = lse;
  a.dout = dout; a.dq = dq; a.dk = dk; a.dv = dv;
  a.B = B; a.S = S; a.Hq = Hq; a.Hkv = Hkv; a.D = D; a.causal = causal; a.dtype = dtype;
  a.doc = doc_ids;
  a.kvalid = key_valid;
  a.scale = 1.0f / sqrtf((float)D);
  a.stream = (hipStream_t)stream;
  if (!rot_supported(B, S, Hq, Hkv, D, dtype, doc_ids != nullptr, key_valid != nullptr) ||
      !bwd_mfma_supported(a) || ((uintptr_t)rot & 15) != 0) {
    set_error("kf_attn_bwd_rot needs the MFMA path (sizes as kf_attn_rot_size accepts, "
              "16-byte aligned pointers)");
    return KF_ERR_UNSUPPORTED;
  }
  const size_t need = bwd_mfma_workspace(B, S, Hq, Hkv, D, true);
  if (workspace_bytes < need || !workspace) {
    set_error("workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
    return KF_ERR_WORKSPACE;
  }
  return bwd_mfma(a, workspace, workspace_bytes);
}

int kf_attn_decode_workspace_size(int B, int Hq, int Hkv, int D, int max_len, int dtype,
                                  size_t* bytes) {
  int rc = check_common(B, 1, max_len, Hq, Hkv, D, dtype);
  if (rc) return rc;
  KF_CHECK_ARG(bytes != nullptr, "bytes is null");
  *bytes = decode_workspace(B, Hq, Hkv, D, max_len);
  return KF_OK;
}

}  // extern "C"

namespace {
// Checks shared by both decode entry points; fills *a.
int decode_args(kf::DecodeArgs* a, const void* q_new, const void* k_new, const void* v_new,
                void* k_cache, void* v_cache, const int32_t* lens, const float* rope_cos,
                const float* rope_sin, int64_t rope_row_offset, int64_t rope_rows, void* out,
                int B, int Smax, int Hq, int Hkv, int D, int max_len,
                const float* q_norm_weight, const float* k_norm_weight, float norm_eps,
                int dtype, void* stream) {
  int rc = check_common(B, 1, max_len, Hq, Hkv, D, dtype);
  if (rc) return rc;
  KF_CHECK_ARG(q_new && k_new && v_new && k_cache && v_cache && lens && rope_cos && rope_sin &&
                   out,
               "null tensor pointer");
  KF_CHECK_ARG(!q_norm_weight == !k_norm_weight,
               "QK-norm needs both q_norm_weight and k_norm_weight (or neither)");
  KF_CHECK_ARG(max_len <= Smax, "max_len (%d) exceeds the cache length (%d)", max_len, Smax);
  KF_CHECK_ARG(rope_rows > 0, "rope tables must have at least one row");
  a->q_new = q_new; a->k_new = k_new; a->v_new = v_new; a->k_cache = k_cache;
  a->v_cache = v_cache;
  a->lens = lens; a->cos = rope_cos; a->sin = rope_sin; a->rope_row_offset = rope_row_offset;
  a->rope_rows = rope_rows;
  a->out = out; a->B = B; a->Smax = Smax; a->Hq = Hq; a->Hkv = Hkv; a->D = D;
  a->max_len = max_len;
  a->q_norm_w = q_norm_weight; a->k_norm_w = k_norm_weight; a->norm_eps = norm_eps;
  a->dtype = dtype; a->scale = 1.0f / sqrtf((float)D); a->stream = (hipStream_t)stream;
  return KF_OK;
}
}  // namespace

extern "C" {

int kf_attn_decode(const void* q_new, const void* k_new, const void* v_new, void* k_cache,
                   void* v_cache, const int32_t* lens, const float* rope_cos,
                   const float* rope_sin, int64_t rope_row_offset, int64_t rope_rows, void* out,
                   void* workspace,
                   size_t workspace_bytes, int B, int Smax, int Hq, int Hkv, int D, int max_len,
                   const float* q_norm_weight, const float* k_norm_weight, float norm_eps,
                   int dtype, void* stream) {
  DecodeArgs a;
  int rc = decode_args(&a, q_new, k_new, v_new, k_cache, v_cache, lens, rope_cos, rope_sin,
                       rope_row_offset, rope_rows, out, B, Smax, Hq, Hkv, D, max_len,
                       q_norm_weight, k_norm_weight, norm_eps, dtype, stream);
  if (rc) return rc;
  const size_t need = decode_workspace(B, Hq, Hkv, D, max_len);
  if (workspace_bytes < need || !workspace) {
    set_error("workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
    return KF_ERR_WORKSPACE;
  }
  return decode(a, workspace);
}

int kf_attn_decode_noalloc(const void* q_new, const void* k_new, const void* v_new,
                           void* k_cache, void* v_cache, const int32_t* lens,
                           const float* rope_cos, const float* rope_sin,
                           int64_t rope_row_offset, int64_t rope_rows, void* out, int B,
                           int Smax, int Hq, int Hkv, int D, int max_len,
                           const float* q_norm_weight, const float* k_norm_weight,
                           float norm_eps, int dtype, void* stream) {
  DecodeArgs a;
  int rc = decode_args(&a, q_new, k_new, v_new, k_cache, v_cache, lens, rope_cos, rope_sin,
                       rope_row_offset, rope_rows, out, B, Smax, Hq, Hkv, D, max_len,
                       q_norm_weight, k_norm_weight, norm_eps, dtype, stream);
  if (rc) return rc;
  const size_t need = decode_workspace(B, Hq, Hkv, D, max_len);
  if (need > DECODE_SCRATCH_BYTES) {
    set_error("decode needs %zu bytes of partials, more than the %zu-byte static scratch of "
              "kf_attn_decode_noalloc; use kf_attn_decode with a workspace",
              need, (size_t)DECODE_SCRATCH_BYTES);
    return KF_ERR_WORKSPACE;
  }
  void* ptr = nullptr;
  rc = decode_scratch(&ptr);
  if (rc) return rc;
  return decode(a, ptr);
}

int kf_kv_cache_append(const void* k_new, const void* v_new, const float* rope_cos,
                       const float* rope_sin, void* k_cache, void* v_cache, int start, int B,
                       int Snew, int Hkv, int Smax, int D, int dtype, void* stream) {
  int rc = check_common(B, Snew, Smax, Hkv, Hkv, D, dtype);
  if (rc) return rc;
  KF_CHECK_ARG(k_new && v_new && rope_cos && rope_sin && k_cache && v_cache,
               "null tensor pointer");
  KF_CHECK_ARG(start >= 0 && start + Snew <= Smax,
               "cache overflow: start %d + %d new tokens > capacity %d", start, Snew, Smax);
  return cache_append(k_new, v_new, rope_cos, rope_sin, k_cache, v_cache, start, B, Snew, Hkv,
                      Smax, D, dtype, (hipStream_t)stream);
}

int kf_attn_capture_workspace_size(int B, int Sq, int Sk, int Hq, int Hkv, int D, int dtype,
                                   size_t* bytes) {
  return kf_attn_fwd_workspace_size(B, Sq, Sk, Hq, Hkv, D, dtype, bytes);
}

int kf_attn_capture(const void* q, const void* k, const void* v, const float* rope_cos,
                    const float* rope_sin, float* probs, void* out, float* lse, void* workspace,
                    size_t workspace_bytes, int B, int Sq, int Sk, int Hq, int Hkv, int D,
                    int64_t ksb, int64_t kss, int64_t ksh, int64_t vsb, int64_t vss,
                    int64_t vsh, int k_rotated, int causal, const int32_t* doc_ids,
                    const int32_t* key_valid, int dtype, void* stream) {
  int rc = check_common(B, Sq, Sk, Hq, Hkv, D, dtype);
  if (rc) return rc;
  KF_CHECK_ARG(q && k && v && rope_cos && rope_sin && out && probs && lse, "null tensor pointer");
  KF_CHECK_ARG(k_rotated || Sk == Sq, "un-rotated keys need Sk == Sq (got %d, %d)", Sk, Sq);
  rc = check_masks(doc_ids, key_valid, causal, Sq, Sk, k_rotated);
  if (rc) return rc;
  FwdArgs a = make_fwd(q, k, v, rope_cos, rope_sin, out, lse, B, Sq, Sk, Hq, Hkv, D, ksb, kss,
                       ksh, vsb, vss, vsh, k_rotated, causal, doc_ids, key_valid, dtype, stream);
  if (fwd_mfma_supported(a) && ((uintptr_t)probs & 15) == 0) {
    const size_t need = fwd_mfma_workspace(B, Sk, Hkv, D);
    if (workspace_bytes < need || !workspace) {
      set_error("workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
      return KF_ERR_WORKSPACE;
    }
    return capture_probs_mfma(a, probs, workspace);
  }
  if (fwd_f32_supported(a)) {
    const size_t need = fwd_ws(a);
    if (workspace_bytes < need || (need && !workspace)) {
      set_error("workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
      return KF_ERR_WORKSPACE;
    }
    return capture_f32(a, probs, workspace);
  }
  rc = fwd_generic(a);
  if (rc) return rc;
  return capture_probs_generic(a, lse, probs);
}

}  // extern "C"
