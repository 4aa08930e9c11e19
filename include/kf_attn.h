/* kf_attn.h — C ABI of the MI355X (gfx950) attention path for KempnerForge.
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream, and
 * launches asynchronously on that stream.  No entry point allocates, frees or
 * synchronises: the caller (PyTorch's caching allocator on the Python side)
 * owns every buffer, workspace included.  Pointers are borrowed for the call.
 *
 * Layout conventions (element strides, head dim contiguous):
 *   BSHD  = [batch, seq, heads, head_dim]  — what q_proj(x).view(B,S,H,D) gives
 *           (kempnerforge/model/attention.py:150-152)
 *   cache = [batch, kv_heads, max_seq, head_dim]
 *           (kempnerforge/model/attention.py:46-51)
 * RoPE tables are the reference's float32 [rows, head_dim/2] cos/sin tables
 * (kempnerforge/model/position.py:12-40); the kernels cast them to the input
 * dtype exactly as apply_rope does (kempnerforge/model/position.py:65-68).
 *
 * dtype codes: 0 = float32, 1 = bfloat16, 2 = float16.
 * Return value: KF_OK (0) or an error code; kf_last_error() then holds a
 * thread-local message.  Inputs holding NaN/Inf propagate to the outputs.
 */
#ifndef KF_ATTN_H
#define KF_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KF_OK 0
#define KF_ERR_INVALID_ARGUMENT 1
#define KF_ERR_UNSUPPORTED 2
#define KF_ERR_HIP 3
#define KF_ERR_WORKSPACE 4

#define KF_DTYPE_F32 0
#define KF_DTYPE_BF16 1
#define KF_DTYPE_F16 2

/* Library version (major*10000 + minor*100 + patch). */
int kf_version(void);

/* Message describing the last error returned on this thread ("" if none). */
const char* kf_last_error(void);

/* Workspace bytes kf_attn_fwd needs for these sizes (0 is possible). */
int kf_attn_fwd_workspace_size(int B, int Sq, int Sk, int Hq, int Hkv, int D, int dtype,
                               size_t* bytes);

/* Causal (or full) GQA attention forward with RoPE fused.
 *
 * Replaces, inside Attention.forward, apply_rope on q and k
 * (kempnerforge/model/attention.py:165-166), the repeat_interleave GQA
 * expansion (:173-175) and F.scaled_dot_product_attention(q, k, v,
 * is_causal=...) (:228-231), plus the transpose back to BSHD (:234).
 *
 *   q    [B, Sq, Hq, D] BSHD contiguous, before RoPE
 *   k, v element (b,s,h,d) at k + b*ksb + s*kss + h*ksh + d (likewise v);
 *        k is before RoPE (k_rotated = 0, requires Sk == Sq) or already
 *        rotated, e.g. KV-cache contents (k_rotated = 1)
 *   rope_cos, rope_sin  [Sq, D/2] float32: row i is query (and key) i's angle
 *   out  [B, Sq, Hq, D] BSHD contiguous, dtype of q
 *   lse  [B, Hq, Sq] float32 natural-log softmax denominators (may be NULL)
 *   causal: 1 = top-left causal mask (query i sees keys j <= i), which is what
 *   SDPA's is_causal=True does; 0 = no mask.
 *   doc_ids  [B, S] int32 document id of each position of packed sequences, or
 *   NULL.  Given, query i sees key j only if j <= i and doc_ids[b][i] ==
 *   doc_ids[b][j]: the explicit mask of the reference's packed-sequence branch
 *   (kempnerforge/model/attention.py:204-227, doc_ids from
 *   kempnerforge/data/dataset.py:27-65).  Needs causal = 1, k_rotated = 0.
 *   key_valid  [B, S] int32, 1 = the key may be attended (key_padding_mask),
 *   or NULL.  Given, query i also needs key_valid[b][j] != 0; a query that
 *   sees no key at all is unmasked entirely and attends every key, the NaN
 *   guard of the reference's explicit-mask branches (kempnerforge/model/
 *   attention.py:214-225, kempnerforge/model/mot.py:188-198).  Needs
 *   causal = 1, k_rotated = 0; combines with doc_ids.
 * Query head h reads KV head h / (Hq / Hkv).  Scale is D^-1/2.
 */
int kf_attn_fwd(const void* q, const void* k, const void* v, const float* rope_cos,
                const float* rope_sin, void* out, float* lse, void* workspace,
                size_t workspace_bytes, int B, int Sq, int Sk, int Hq, int Hkv, int D,
                int64_t ksb, int64_t kss, int64_t ksh, int64_t vsb, int64_t vss, int64_t vsh,
                int k_rotated, int causal, const int32_t* doc_ids, const int32_t* key_valid,
                int dtype, void* stream);

/* Workspace bytes kf_attn_bwd needs. */
int kf_attn_bwd_workspace_size(int B, int S, int Hq, int Hkv, int D, int dtype, size_t* bytes);

/* Workspace bytes with which kf_attn_bwd keeps the dS tiles (bf16 or fp16, the
 * input's type) of the dK/dV
 * pass for dQ instead of recomputing S and dP (one fewer pass over the
 * attention matrix; B*Hq*P*(P+64) bytes extra for causal, 2*B*Hq*P*P for full
 * attention, P = S rounded up to 128).  Applies to the bf16 / fp16 kernels up to
 * 32 GiB of tiles (and S <= 65536 with doc_ids or key_valid; with doc_ids the
 * tiles are written only where documents meet; with key_valid only causal
 * launches keep them, and only for the batch rows whose key 0 is valid, which
 * have no rows attending past the diagonal: the others recompute, decided on
 * the device).  float32 (head_dim 64 or 128, no doc_ids or key_valid) keeps
 * float32 [32][64] dS blocks, (t/2 + 1) per 32-position tile t when causal,
 * S/32 * ceil(S/64) for full attention, per query head, up to 32 GiB.
 * Otherwise this equals kf_attn_bwd_workspace_size.  kf_attn_bwd takes the faster path whenever
 * workspace_bytes reaches this size.  No counterpart in the reference (its
 * SDPA backward manages its own memory). */
int kf_attn_bwd_workspace_size_ds(int B, int S, int Hq, int Hkv, int D, int dtype, int causal,
                                  size_t* bytes);

/* Backward of kf_attn_fwd (k_rotated = 0, Sq == Sk == S, contiguous BSHD).
 *
 * Replaces the autograd backward the reference gets from
 * scaled_loss.backward() (scripts/train.py:850) through SDPA
 * (kempnerforge/model/attention.py:231), repeat_interleave (:173-175) and
 * apply_rope (:165-166; kempnerforge/model/position.py:71).
 *   out, lse  what kf_attn_fwd returned for these inputs
 *   dout      [B, S, Hq, D] gradient of out
 *   dq        [B, S, Hq, D]  gradient w.r.t. q before RoPE
 *   dk, dv    [B, S, Hkv, D] gradients w.r.t. k (before RoPE) and v, summed
 *             over the Hq/Hkv query heads of each KV group
 *   doc_ids, key_valid  as for kf_attn_fwd (NULL or what the forward used)
 */
int kf_attn_bwd(const void* q, const void* k, const void* v, const float* rope_cos,
                const float* rope_sin, const void* out, const float* lse, const void* dout,
                void* dq, void* dk, void* dv, void* workspace, size_t workspace_bytes, int B,
                int S, int Hq, int Hkv, int D, int causal, const int32_t* doc_ids,
                const int32_t* key_valid, int dtype, void* stream);

/* Rotated operands kept from the forward for the backward ("rot"): q and k
 * after RoPE as the backward's kernels read them, K [B*Hkv][P][D] then Q
 * [B*Hq][P][D] in the input's type, P = S rounded up to 128, rows past S zero.  The pair
 * below replaces kf_attn_fwd / kf_attn_bwd for self-attention (k_rotated = 0,
 * contiguous BSHD k and v): the forward writes rot next to out and lse, and
 * the backward reads it instead of q and k, skipping their rotation (one fewer
 * pass over q and k).  A caller that keeps rot for the backward need not keep
 * q and k, which is what the reference's autograd saves for SDPA's backward
 * (kempnerforge/model/attention.py:165-166,231).  Results are bit-identical
 * to kf_attn_fwd / kf_attn_bwd.  No counterpart in the reference's interface.
 *
 * kf_attn_rot_size: bytes of rot, or KF_ERR_UNSUPPORTED when the pair does
 * not take these sizes, dtype (bf16 or fp16) or mask kinds (has_doc,
 * has_key_valid: whether doc_ids / key_valid will be passed). */
int kf_attn_rot_size(int B, int S, int Hq, int Hkv, int D, int dtype, int has_doc,
                     int has_key_valid, size_t* bytes);

/* kf_attn_fwd (same arguments; Sq == Sk == S, contiguous BSHD k and v) that
 * also fills rot.  Workspace: kf_attn_fwd_workspace_size.  KF_ERR_UNSUPPORTED
 * when kf_attn_rot_size rejects the sizes or a pointer is not 16-byte aligned;
 * then call kf_attn_fwd / kf_attn_bwd instead. */
int kf_attn_fwd_rot(const void* q, const void* k, const void* v, const float* rope_cos,
                    const float* rope_sin, void* out, float* lse, void* rot, void* workspace,
                    size_t workspace_bytes, int B, int S, int Hq, int Hkv, int D, int causal,
                    const int32_t* doc_ids, const int32_t* key_valid, int dtype, void* stream);

/* Workspace bytes of kf_attn_bwd_rot: with_ds = 0 the minimum, 1 with the dS
 * records kept (as kf_attn_bwd_workspace_size_ds; equal to the minimum where
 * records do not apply).  Smaller than
 * kf_attn_bwd's by the size of rot. */
int kf_attn_bwd_rot_workspace_size(int B, int S, int Hq, int Hkv, int D, int dtype, int causal,
                                   int with_ds, size_t* bytes);

/* kf_attn_bwd reading the rotated q and k from rot (kf_attn_fwd_rot of the
 * same q, k, cos, sin and masks) instead of q and k. */
int kf_attn_bwd_rot(const void* rot, const void* v, const float* rope_cos, const float* rope_sin,
                    const void* out, const float* lse, const void* dout, void* dq, void* dk,
                    void* dv, void* workspace, size_t workspace_bytes, int B, int S, int Hq,
                    int Hkv, int D, int causal, const int32_t* doc_ids, const int32_t* key_valid,
                    int dtype, void* stream);

/* Workspace bytes kf_attn_decode needs; max_len bounds lens[b] + 1. */
int kf_attn_decode_workspace_size(int B, int Hq, int Hkv, int D, int max_len, int dtype,
                                  size_t* bytes);

/* One KV-cache decode step (one new token per sequence).
 *
 * Replaces, for seq_len == 1 with a cache: apply_rope at start_pos
 * (kempnerforge/model/transformer.py:418-425; attention.py:165-166),
 * KVCache.update (kempnerforge/model/attention.py:54-70), the whole-cache
 * repeat_interleave (:173-175) and SDPA with is_causal=False (:229-231).
 *   q_new [B,1,Hq,D], k_new/v_new [B,1,Hkv,D] contiguous, before RoPE
 *   k_cache, v_cache [B, Hkv, Smax, D] contiguous; on return position lens[b]
 *       of sequence b holds the rotated k_new and v_new
 *   lens  [B] int32 on the device: tokens already cached for each sequence,
 *       i.e. the new token's position (the reference keeps one scalar
 *       KVCache.seq_len for the batch; equal entries reproduce it)
 *   rope_cos/sin [rope_rows, D/2]: sequence b uses row lens[b] - rope_row_offset
 *   out  [B, 1, Hq, D]
 *   max_len  an upper bound on lens[b] + 1 (<= Smax)
 *   q_norm_weight, k_norm_weight  [D] float32 per-head RMSNorm weights, or
 *       both NULL: given, q_new and k_new are normalised first, as the
 *       reference's q_norm / k_norm do before RoPE (kempnerforge/model/
 *       attention.py:155-157; norm.py:22-27, eps = norm_eps), inside the
 *       decode launches instead of separate ones
 * lens is not modified.  Attention covers keys 0..lens[b] with no mask.
 * lens may differ per sequence (a ragged batch): each sequence attends its
 * own prefix at its own RoPE position.
 * lens lives on the device, so it cannot be validated before the launch: a
 * sequence whose lens[b] + 1 exceeds max_len, or whose table row falls outside
 * [0, rope_rows), gets NaN outputs and no cache write instead of a fault.
 */
int kf_attn_decode(const void* q_new, const void* k_new, const void* v_new, void* k_cache,
                   void* v_cache, const int32_t* lens, const float* rope_cos,
                   const float* rope_sin, int64_t rope_row_offset, int64_t rope_rows, void* out,
                   void* workspace,
                   size_t workspace_bytes, int B, int Smax, int Hq, int Hkv, int D, int max_len,
                   const float* q_norm_weight, const float* k_norm_weight, float norm_eps,
                   int dtype, void* stream);

/* kf_attn_decode without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation).  No counterpart in the reference.
 *
 * Same arguments and results as kf_attn_decode.  The split-K partial results
 * live in one static device array of 32 MiB per GPU, held from the library's
 * load until the process ends; a call whose workspace would not fit
 * (kf_attn_decode_workspace_size > 32 MiB, e.g. B * Hkv beyond about 6000 at
 * 8 query heads per KV head and head_dim 128) returns KF_ERR_WORKSPACE.  Each
 * call writes the partials it reads, so nothing needs clearing between calls.
 * Every call on one GPU uses the same array: calls that overlap on one GPU
 * (concurrent streams) race and must be serialised by the caller.  Allocates
 * nothing, synchronises nothing. */
int kf_attn_decode_noalloc(const void* q_new, const void* k_new, const void* v_new,
                           void* k_cache, void* v_cache, const int32_t* lens,
                           const float* rope_cos, const float* rope_sin,
                           int64_t rope_row_offset, int64_t rope_rows, void* out, int B,
                           int Smax, int Hq, int Hkv, int D, int max_len,
                           const float* q_norm_weight, const float* k_norm_weight,
                           float norm_eps, int dtype, void* stream);

/* Append Snew tokens to a KV cache at positions start .. start+Snew-1.
 *
 * Replaces apply_rope on k (kempnerforge/model/attention.py:166) followed by
 * KVCache.update's slice assignment (kempnerforge/model/attention.py:65-68).
 *   k_new, v_new [B, Snew, Hkv, D] contiguous, before RoPE
 *   rope_cos/sin [Snew, D/2]: row i rotates token start + i
 */
int kf_kv_cache_append(const void* k_new, const void* v_new, const float* rope_cos,
                       const float* rope_sin, void* k_cache, void* v_cache, int start, int B,
                       int Snew, int Hkv, int Smax, int D, int dtype, void* stream);

/* Workspace bytes kf_attn_capture needs. */
int kf_attn_capture_workspace_size(int B, int Sq, int Sk, int Hq, int Hkv, int D, int dtype,
                                   size_t* bytes);

/* Attention with materialised probabilities (interpretability capture).
 *
 * Replaces Attention._attention_with_weights
 * (kempnerforge/model/attention.py:238-280): softmax(Q K^T * D^-1/2 + mask)
 * written as float32 probs [B, Hq, Sq, Sk] (0 where masked) and out = P V in
 * BSHD.  Arguments as for kf_attn_fwd; lse [B, Hq, Sq] is required here.
 */
int kf_attn_capture(const void* q, const void* k, const void* v, const float* rope_cos,
                    const float* rope_sin, float* probs, void* out, float* lse, void* workspace,
                    size_t workspace_bytes, int B, int Sq, int Sk, int Hq, int Hkv, int D,
                    int64_t ksb, int64_t kss, int64_t ksh, int64_t vsb, int64_t vss,
                    int64_t vsh, int k_rotated, int causal, const int32_t* doc_ids,
                    const int32_t* key_valid, int dtype, void* stream);

/* ---- Measurement hooks.  No counterpart in the reference: they exist so a
 * benchmark can time each kernel of the library on the stream it runs on. */

/* on != 0: bracket every kernel launch of the library with two HIP events
 * recorded on the launch stream (adds two event records per launch). */
int kf_prof_enable(int on);

/* Wait for the recorded events, aggregate by kernel name and clear the record.
 * Writes up to cap entries: names[64*i] (NUL-terminated), total_ms[i],
 * counts[i] (any of the arrays may be NULL).  Returns the number of distinct
 * kernel names recorded. */
int kf_prof_collect(char* names, float* total_ms, int* counts, int cap);

#ifdef __cplusplus
}
#endif

#endif /* KF_ATTN_H */
