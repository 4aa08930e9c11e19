// Internal (non-exported) argument bundles and launcher declarations shared by
// the kernel translation units and the C-ABI layer in kf_api.hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "kf_attn.h"

namespace kf {

struct FwdArgs {
  const void* q;      // [B, Sq, Hq, D] contiguous, pre-RoPE
  const void* k;      // element (b, s, h, d) at b*ksb + s*kss + h*ksh + d
  const void* v;      // element (b, s, h, d) at b*vsb + s*vss + h*vsh + d
  const float* cos;   // [Sq, D/2] float32 rows for query (and key) positions
  const float* sin;
  void* out;          // [B, Sq, Hq, D] contiguous
  float* lse;         // [B, Hq, Sq] float32 (may be null for the generic path)
  int B, Sq, Sk, Hq, Hkv, D;
  int64_t ksb, kss, ksh, vsb, vss, vsh;
  int k_rotated;      // 1: k already holds post-RoPE keys (KV-cache contents)
  int causal;         // 1: top-left causal mask (query i sees keys j <= i)
  const int32_t* doc; // [B, S] document id per position (packed sequences) or null;
                      // query i then also needs doc[i] == doc[j] (requires Sq == Sk)
  const int32_t* kvalid;  // [B, S] 1 = valid key (key padding mask) or null; query i
                          // then needs kvalid[j], and a query that sees no key at
                          // all attends every key (requires Sq == Sk)
  int dtype;
  float scale;        // softmax scale, D^-1/2
  hipStream_t stream;
  void* rot = nullptr;  // null, or the backward's rotated operands written by fwd_mfma (self-
                        // attention): K [B*Hkv][P][D] then Q [B*Hq][P][D] bf16 after
                        // RoPE, P = S rounded up to 128, rows past S zero
};

struct BwdArgs {
  const void *q, *k, *v;  // [B, S, H, D] contiguous, pre-RoPE
  const float *cos, *sin; // [S, D/2]
  const void* out;        // forward output [B, S, Hq, D]
  const float* lse;       // [B, Hq, S]
  const void* dout;       // [B, S, Hq, D]
  void *dq, *dk, *dv;     // pre-RoPE gradients, same layouts as q, k, v
  int B, S, Hq, Hkv, D;
  int causal, dtype;
  const int32_t* doc;     // [B, S] document ids or null (see FwdArgs::doc)
  const int32_t* kvalid;  // [B, S] key validity or null (see FwdArgs::kvalid)
  float scale;
  hipStream_t stream;
  const void* rot = nullptr;  // FwdArgs::rot of the forward call; q and k are then unused
};

// generic kernels (kf_generic.hip)
int fwd_generic(const FwdArgs& a);
// workspace: delta [B*Hq*S] float32, then one guard flag per (b, position)
size_t bwd_generic_workspace(int B, int S, int Hq);
int bwd_generic(const BwdArgs& a, void* workspace);
int capture_probs_generic(const FwdArgs& a, const float* lse, float* probs);

// float32 MFMA kernels (kf_f32.hip): no explicit masks, head_dim 64 or 128.
// Workspaces: the forward's rotated K (unused when a.k_rotated); the
// backward's rotated Q and K and per-row softmax statistics.
bool fwd_f32_supported(const FwdArgs& a);
size_t fwd_f32_workspace(int B, int Sk, int Hkv, int D);
int fwd_f32(const FwdArgs& a, void* workspace);
// out, lse (a.lse must be set) and the probabilities, float32 [B, Hq, Sq, Sk];
// the workspace is fwd_f32's
int capture_f32(const FwdArgs& a, float* probs, void* workspace);
bool bwd_f32_supported(const BwdArgs& a);
size_t bwd_f32_workspace(int B, int S, int Hq, int Hkv, int D);
// with the dS records (used without an explicit mask when workspace_bytes
// reaches it: dQ then multiplies them by K instead of recomputing S and dP)
size_t bwd_f32_workspace_ds(int B, int S, int Hq, int Hkv, int D, int causal);
int bwd_f32(const BwdArgs& a, void* workspace, size_t workspace_bytes);

// bf16 MFMA kernels (kf_fwd.hip, kf_bwd.hip, kf_capture.hip)
bool fwd_mfma_supported(const FwdArgs& a);
// Rotated K [B*Hkv][Skp][D] bf16 (Skp a multiple of 64, rows past Sk zero) and,
// by v_mode: KV_V_ROWS zero-padded V [B*Hkv][Skp][D]; KV_V_TRANSPOSED V^T
// [B*Hkv][D][Skp], keys of each 16 in the P^T fragment order 0-3, 8-11, 4-7,
// 12-15 (what the forward kernel reads); KV_V_NONE no V (vn unused).  With
// a.doc also the [min, max] document id of each 64-key tile, [B][Skp/64]
// (a.kvalid: valid count and first valid key).
enum { KV_V_ROWS = 0, KV_V_TRANSPOSED = 1, KV_V_NONE = 2 };
// Compute units of the current device (cached per device), to size persistent grids.
int device_cu_count();
// krot holds krows >= Skp rows per KV head (null: only the tile records); qpad,
// if set, is the rotated-Q buffer of FwdArgs::rot, whose rows past Sq it zeroes.
int launch_kv_prep(const FwdArgs& a, void* krot, int krows, void* vn, int Skp, int2* ranges,
                   int v_mode, void* qpad = nullptr);
// Packed documents: B*nblk blocks of `rows` positions ordered by how many
// 64-position tiles each lists, most first (order[r] = block index; counts is
// scratch of the same size).  key_side: key blocks listing query tiles from
// their diagonal on; else query blocks listing key tiles up to theirs.
int launch_doc_order(const int32_t* doc, const int2* ranges, int S, int rstride, int rows, int B,
                     int nblk, int key_side, int* counts, int* order, hipStream_t stream);
// Key padding: flags[b] = 1 when every key of batch row b is valid (ranges:
// kv_prep's tile records, rstride per batch row), else 0.
int launch_kpm_row_flags(const int2* ranges, int rstride, int S, int B, int* flags,
                         hipStream_t stream);
// bytes of FwdArgs::rot
size_t rot_bytes(int B, int S, int Hq, int Hkv, int D);
size_t fwd_mfma_workspace(int B, int Sk, int Hkv, int D);
int fwd_mfma(const FwdArgs& a, void* workspace);
// LSE (a.lse), probabilities and out (a.out) of the capture path in one launch
// after kv_prep; the workspace is fwd_mfma's.
int capture_probs_mfma(const FwdArgs& a, float* probs, void* workspace);

// dS record tile of the backward (dK/dV kernels write, dQ reads): DS_REC_Q
// query positions x DS_REC_K keys of one query head, 4 KB of bf16.
constexpr int DS_REC_Q = 64, DS_REC_K = 32;

bool bwd_mfma_supported(const BwdArgs& a);
size_t bwd_mfma_workspace(int B, int S, int Hq, int Hkv, int D, bool rot = false);
// Workspace with which bwd_mfma stores the dS tiles once for dQ instead of
// recomputing S and dP (unmasked launches up to a size cap); otherwise
// bwd_mfma_workspace.  bwd_mfma takes that path when workspace_bytes allows.
size_t bwd_mfma_workspace_ds(const BwdArgs& a);
int bwd_mfma(const BwdArgs& a, void* workspace, size_t workspace_bytes);

// decode (kf_decode.hip)
struct DecodeArgs {
  const void *q_new, *k_new, *v_new;  // [B,1,Hq,D], [B,1,Hkv,D], [B,1,Hkv,D] contiguous
  void *k_cache, *v_cache;            // [B, Hkv, Smax, D] contiguous
  const int32_t* lens;                // [B] cached tokens per sequence = new token position
  const float *cos, *sin;             // table; row = lens[b] - rope_row_offset
  int64_t rope_row_offset;
  int64_t rope_rows;                  // rows in the tables
  void* out;                          // [B, 1, Hq, D]
  int B, Smax, Hq, Hkv, D, max_len;   // max_len >= lens[b] + 1 for every b
  const float *q_norm_w, *k_norm_w;   // [D] float32 QK-norm weights, or both null
  float norm_eps;
  int dtype;
  float scale;
  hipStream_t stream;
};
size_t decode_workspace(int B, int Hq, int Hkv, int D, int max_len);
// float32 decode on the fp32 matrix cores (kf_f32.hip), after the caller's
// append of the new token: split-K over at most `slots` partials of the
// decode workspace's layout
bool decode_f32_supported(const DecodeArgs& a);
int decode_f32(const DecodeArgs& a, void* workspace, size_t slots);
int decode(const DecodeArgs& a, void* workspace);
// Allocation-free decode: the current device's copy of a static device array
// of DECODE_SCRATCH_BYTES stands in for the workspace.
constexpr size_t DECODE_SCRATCH_BYTES = (size_t)32 << 20;
int decode_scratch(void** ptr);

// cache append (kf_decode.hip)
int cache_append(const void* k_new, const void* v_new, const float* cos, const float* sin,
                 void* k_cache, void* v_cache, int start, int B, int Snew, int Hkv, int Smax,
                 int D, int dtype, hipStream_t stream);

}  // namespace kf
