// KV-cache decode (one new token per sequence) and cache append.
//
// decode = three launches on the caller's stream:
//  1. append   rotate k_new at position lens[b] (eager RoPE rounding) and write
//              it and v_new into the caches (the reference's KVCache.update).
//  2. split    split-K attention: workgroup (split, b, kv head) streams CH keys
//              of one KV head once and serves all n_rep query heads of the
//              group from that single read (the reference expands the cache
//              n_rep times first).  D/8 threads share a key row, each loading
//              16 contiguous bytes, so a pass reads whole rows coalesced.
//              Writes partial (o, m, l) per (b, hq, split) in float32.
//  3. merge    one workgroup per (b, hq) rescales and sums the partials.
// Shapes outside the fast path (dtype other than bf16, D not in {64, 128}, or
// n_rep not in {1, 2, 4, 8}) use decode_generic: one wavefront per (b, hq).
#include "kf_common.h"
#include "kf_internal.h"

namespace kf {

namespace {

constexpr int CH = 256;  // keys per split

// A device-side cache length is usable when the new token's position fits the
// grid (len + 1 <= max_len <= Smax) and its RoPE row lies inside the table.
// Anything else yields NaN outputs and no cache write, never an access outside
// the buffers.
__device__ __forceinline__ bool decode_len_ok(int len, int max_len, int64_t row_offset,
                                              int64_t rope_rows) {
  const int64_t trow = (int64_t)len - row_offset;
  return len >= 0 && len < max_len && trow >= 0 && trow < rope_rows;
}

// Append rotated k / plain v for `Snew` tokens per sequence.  Token i of
// sequence b goes to position pos_b + i where pos_b = lens ? lens[b] : start,
// and is rotated with table row (pos_b + i - row_offset).  With `lens`, a
// sequence failing decode_len_ok(lens[b], max_len, ...) is skipped.
template <typename T>
__global__ __launch_bounds__(256) void append_kernel(const T* __restrict__ k_new,
                                                     const T* __restrict__ v_new,
                                                     const float* __restrict__ cos,
                                                     const float* __restrict__ sin,
                                                     T* __restrict__ kc, T* __restrict__ vc,
                                                     const int32_t* __restrict__ lens, int start,
                                                     int64_t row_offset, int64_t rope_rows,
                                                     int max_len, int B, int Snew, int Hkv,
                                                     int Smax, int D) {
  const int half = D / 2;
  const int64_t n = (int64_t)B * Snew * Hkv * half;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= n) return;
  const int d = (int)(idx % half);
  const int g = (int)((idx / half) % Hkv);
  const int i = (int)((idx / ((int64_t)half * Hkv)) % Snew);
  const int b = (int)(idx / ((int64_t)half * Hkv * Snew));
  if (lens && !decode_len_ok(lens[b], max_len, row_offset, rope_rows)) return;
  const int pos = (lens ? lens[b] : start) + i;
  if (pos < 0 || pos >= Smax || pos - row_offset >= rope_rows) return;
  const int64_t src = (((int64_t)b * Snew + i) * Hkv + g) * D;
  const int64_t dst = (((int64_t)b * Hkv + g) * Smax + pos) * D;
  const int64_t trow = pos - row_offset;
  float r1, r2;
  rope_pair<T>(to_f32(k_new[src + d]), to_f32(k_new[src + d + half]), cos[trow * half + d],
               sin[trow * half + d], r1, r2);
  kc[dst + d] = from_f32<T>(r1);
  kc[dst + d + half] = from_f32<T>(r2);
  vc[dst + d] = v_new[src + d];
  vc[dst + d + half] = v_new[src + d + half];
}

template <int D, int NREP>
__global__ __launch_bounds__(256) void decode_split_kernel(
    const bf16* __restrict__ q_new, const float* __restrict__ cos, const float* __restrict__ sin,
    int64_t row_offset, int64_t rope_rows, int max_len, const bf16* __restrict__ kc,
    const bf16* __restrict__ vc, const int32_t* __restrict__ lens, float* __restrict__ opart,
    float* __restrict__ mpart, float* __restrict__ lpart, int Hq, int Hkv, int Smax, int nsplit,
    float scale_log2) {
  constexpr int TPR = D / 8;        // threads per key row (16 bytes each)
  constexpr int RPP = 256 / TPR;    // rows per pass
  constexpr int NP = CH / RPP;      // passes per split
  constexpr int HALF = D / 2;
  __shared__ float sq[NREP][D];
  __shared__ float sp[NREP][CH];
  __shared__ float so[4][NREP * D];  // per-wavefront partial o
  __shared__ float sm[NREP], sl[NREP];

  const int sp_idx = blockIdx.x;
  const int bg = blockIdx.y;
  const int b = bg / Hkv, g = bg % Hkv;
  if (!decode_len_ok(lens[b], max_len, row_offset, rope_rows)) return;
  const int L = lens[b] + 1;
  const int k0 = sp_idx * CH;
  if (k0 >= L) return;
  const int k1 = min(k0 + CH, L);
  const int tid = threadIdx.x;
  const int c = tid % TPR, rg = tid / TPR;
  const int w = tid >> 6, lane = tid & 63;

  const bf16* kb = kc + ((int64_t)b * Hkv + g) * Smax * D;
  const bf16* vb = vc + ((int64_t)b * Hkv + g) * Smax * D;
  // issue the whole split's K reads first (NP x 16 bytes per thread in flight)
  u32x4 kr[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int row = k0 + p * RPP + rg;
    kr[p] = row < k1 ? *(const u32x4*)(kb + (int64_t)row * D + 8 * c) : u32x4{0u, 0u, 0u, 0u};
  }

  // rotated queries of the group, float32 in LDS
  const int64_t trow = (int64_t)(L - 1) - row_offset;
  for (int it = tid; it < NREP * HALF; it += 256) {
    const int hr = it / HALF, d = it % HALF;
    const bf16* qr = q_new + ((int64_t)b * Hq + g * NREP + hr) * D;
    float r1, r2;
    rope_pair<bf16>((float)qr[d], (float)qr[d + HALF], cos[trow * HALF + d],
                    sin[trow * HALF + d], r1, r2);
    sq[hr][d] = r1;
    sq[hr][d + HALF] = r2;
  }
  __syncthreads();
  float qreg[NREP][8];
#pragma unroll
  for (int hr = 0; hr < NREP; ++hr)
#pragma unroll
    for (int e = 0; e < 8; ++e) qreg[hr][e] = sq[hr][8 * c + e];

#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int row = k0 + p * RPP + rg;
    float kf[8];
    unpack8(kr[p], kf);
    float part[NREP];
#pragma unroll
    for (int hr = 0; hr < NREP; ++hr) {
      float s = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) s += qreg[hr][e] * kf[e];
      part[hr] = s;
    }
#pragma unroll
    for (int o = 1; o < TPR; o <<= 1)
#pragma unroll
      for (int hr = 0; hr < NREP; ++hr) part[hr] += __shfl_xor(part[hr], o, 64);
    if (c == 0 && row < k1) {
#pragma unroll
      for (int hr = 0; hr < NREP; ++hr) sp[hr][row - k0] = part[hr] * scale_log2;
    }
  }
  // V reads overlap the softmax below
  u32x4 vr[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int row = k0 + p * RPP + rg;
    vr[p] = row < k1 ? *(const u32x4*)(vb + (int64_t)row * D + 8 * c) : u32x4{0u, 0u, 0u, 0u};
  }
  __syncthreads();
  // softmax over this split, one wavefront per query head
  for (int hr = w; hr < NREP; hr += 4) {
    float mx = -INFINITY;
    for (int j = lane; j < k1 - k0; j += 64) mx = fmaxf(mx, sp[hr][j]);
    mx = wave_max(mx);
    float sum = 0.f;
    for (int j = lane; j < CH; j += 64) {
      const float p = j < k1 - k0 ? fast_exp2(sp[hr][j] - mx) : 0.f;
      sp[hr][j] = p;
      sum += p;
    }
    sum = wave_sum(sum);
    if (lane == 0) {
      sm[hr] = mx;
      sl[hr] = sum;
    }
  }
  __syncthreads();
  float acc[NREP][8];
#pragma unroll
  for (int hr = 0; hr < NREP; ++hr)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[hr][e] = 0.f;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int j = p * RPP + rg;  // rows past k1 hold zeros and p = 0
    float vf[8];
    unpack8(vr[p], vf);
#pragma unroll
    for (int hr = 0; hr < NREP; ++hr) {
      const float pr = sp[hr][j];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[hr][e] += pr * vf[e];
    }
  }
  // reduce over the row groups: first inside the wavefront, then across the 4
#pragma unroll
  for (int o = TPR; o < 64; o <<= 1)
#pragma unroll
    for (int hr = 0; hr < NREP; ++hr)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[hr][e] += __shfl_xor(acc[hr][e], o, 64);
  if (lane < TPR) {
#pragma unroll
    for (int hr = 0; hr < NREP; ++hr)
#pragma unroll
      for (int e = 0; e < 8; ++e) so[w][hr * D + 8 * c + e] = acc[hr][e];
  }
  __syncthreads();
  for (int it = tid; it < NREP * D; it += 256) {
    const int hr = it / D, d = it % D;
    const float s = so[0][it] + so[1][it] + so[2][it] + so[3][it];
    const int64_t ph = ((int64_t)b * Hq + g * NREP + hr) * nsplit + sp_idx;
    opart[ph * D + d] = s;
    if (d == 0) {
      mpart[ph] = sm[hr];
      lpart[ph] = sl[hr];
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void decode_merge_kernel(const float* __restrict__ opart,
                                                           const float* __restrict__ mpart,
                                                           const float* __restrict__ lpart,
                                                           const int32_t* __restrict__ lens,
                                                           T* __restrict__ out, int Hq, int D,
                                                           int nsplit, int max_len,
                                                           int64_t row_offset,
                                                           int64_t rope_rows) {
  const int bh = blockIdx.x;
  const int b = bh / Hq;
  if (!decode_len_ok(lens[b], max_len, row_offset, rope_rows)) {
    for (int d = threadIdx.x; d < D; d += 256) out[(int64_t)bh * D + d] = from_f32<T>(NAN);
    return;
  }
  const int ns = (lens[b] + 1 + CH - 1) / CH;  // <= nsplit because lens[b] < max_len
  const int64_t base = (int64_t)bh * nsplit;
  float M = -INFINITY;
  for (int s = 0; s < ns; ++s) M = fmaxf(M, mpart[base + s]);
  float lt = 0.f;
  for (int s = 0; s < ns; ++s) lt += lpart[base + s] * fast_exp2(mpart[base + s] - M);
  const float inv = 1.f / lt;
  for (int d = threadIdx.x; d < D; d += 256) {
    float o = 0.f;
    for (int s = 0; s < ns; ++s) o += opart[(base + s) * D + d] * fast_exp2(mpart[base + s] - M);
    out[(int64_t)bh * D + d] = from_f32<T>(o * inv);
  }
}

// One wavefront per (b, hq); keys 0..lens[b] read from the (already appended)
// cache.  Any D <= 256.
template <typename T>
__global__ __launch_bounds__(256) void decode_generic_kernel(
    const T* __restrict__ q_new, const float* __restrict__ cos, const float* __restrict__ sin,
    int64_t row_offset, int64_t rope_rows, int max_len, const T* __restrict__ kc,
    const T* __restrict__ vc, const int32_t* __restrict__ lens, T* __restrict__ out, int B,
    int Hq, int Hkv, int Smax, int D, float scale) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= B * Hq) return;
  const int b = row / Hq, hq = row % Hq, g = hq / (Hq / Hkv);
  if (!decode_len_ok(lens[b], max_len, row_offset, rope_rows)) {
    for (int d = lane; d < D; d += 64) out[(int64_t)row * D + d] = from_f32<T>(NAN);
    return;
  }
  const int L = lens[b] + 1;
  const int half = D / 2;
  const int64_t trow = (int64_t)(L - 1) - row_offset;
  const T* qr = q_new + (int64_t)row * D;
  float qv[4], acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = lane + 64 * i;
    qv[i] = 0.f;
    if (d < D) {
      const int j = d < half ? d : d - half;
      float r1, r2;
      rope_pair<T>(to_f32(qr[j]), to_f32(qr[j + half]), cos[trow * half + j],
                   sin[trow * half + j], r1, r2);
      qv[i] = d < half ? r1 : r2;
    }
  }
  const T* kb = kc + ((int64_t)b * Hkv + g) * Smax * D;
  const T* vb = vc + ((int64_t)b * Hkv + g) * Smax * D;
  float m = -INFINITY, l = 0.f;
  for (int j = 0; j < L; ++j) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = lane + 64 * i;
      if (d < D) s += qv[i] * to_f32(kb[(int64_t)j * D + d]);
    }
    s = wave_sum(s) * scale;
    const float mn = fmaxf(m, s);
    const float alpha = expf(m - mn), p = expf(s - mn);
    l = l * alpha + p;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = lane + 64 * i;
      acc[i] = acc[i] * alpha + (d < D ? p * to_f32(vb[(int64_t)j * D + d]) : 0.f);
    }
    m = mn;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = lane + 64 * i;
    if (d < D) out[(int64_t)row * D + d] = from_f32<T>(acc[i] / l);
  }
}

template <typename T>
int launch_append(const T* k_new, const T* v_new, const float* cos, const float* sin, T* kc,
                  T* vc, const int32_t* lens, int start, int64_t row_offset, int64_t rope_rows,
                  int max_len, int B, int Snew, int Hkv, int Smax, int D, hipStream_t stream) {
  const int64_t n = (int64_t)B * Snew * Hkv * (D / 2);
  if (n == 0) return KF_OK;
  KF_LAUNCH("kv_append", append_kernel<T>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                     k_new, v_new, cos, sin, kc, vc, lens, start, row_offset, rope_rows, max_len,
                     B, Snew, Hkv, Smax, D);
  KF_CHECK_LAUNCH();
  return KF_OK;
}

template <int D, int NREP>
int launch_split(const DecodeArgs& a, float* opart, float* mpart, float* lpart, int nsplit) {
  KF_LAUNCH("decode_split", (decode_split_kernel<D, NREP>), dim3(nsplit, a.B * a.Hkv), dim3(256), 0,
                     a.stream, (const bf16*)a.q_new, a.cos, a.sin, a.rope_row_offset,
                     a.rope_rows, a.max_len, (const bf16*)a.k_cache, (const bf16*)a.v_cache,
                     a.lens, opart, mpart, lpart, a.Hq, a.Hkv, a.Smax, nsplit,
                     a.scale * kLog2e);
  KF_CHECK_LAUNCH();
  return KF_OK;
}

template <int D>
int dispatch_nrep(const DecodeArgs& a, float* opart, float* mpart, float* lpart, int nsplit) {
  switch (a.Hq / a.Hkv) {
    case 1: return launch_split<D, 1>(a, opart, mpart, lpart, nsplit);
    case 2: return launch_split<D, 2>(a, opart, mpart, lpart, nsplit);
    case 4: return launch_split<D, 4>(a, opart, mpart, lpart, nsplit);
    case 8: return launch_split<D, 8>(a, opart, mpart, lpart, nsplit);
  }
  return KF_ERR_UNSUPPORTED;
}

template <typename T>
int decode_typed(const DecodeArgs& a, void* workspace) {
  int rc = launch_append<T>((const T*)a.k_new, (const T*)a.v_new, a.cos, a.sin, (T*)a.k_cache,
                            (T*)a.v_cache, a.lens, 0, a.rope_row_offset, a.rope_rows, a.max_len,
                            a.B, 1, a.Hkv, a.Smax, a.D, a.stream);
  if (rc) return rc;
  const int n_rep = a.Hq / a.Hkv;
  const bool fast = __is_same(T, bf16) && (a.D == 64 || a.D == 128) &&
                    (n_rep == 1 || n_rep == 2 || n_rep == 4 || n_rep == 8);
  if (fast) {
    const int nsplit = (a.max_len + CH - 1) / CH;
    float* opart = (float*)workspace;
    float* mpart = opart + (size_t)a.B * a.Hq * nsplit * a.D;
    float* lpart = mpart + (size_t)a.B * a.Hq * nsplit;
    rc = a.D == 128 ? dispatch_nrep<128>(a, opart, mpart, lpart, nsplit)
                    : dispatch_nrep<64>(a, opart, mpart, lpart, nsplit);
    if (rc) return rc;
    KF_LAUNCH("decode_merge", decode_merge_kernel<T>, dim3(a.B * a.Hq), dim3(256), 0, a.stream, opart,
                       mpart, lpart, a.lens, (T*)a.out, a.Hq, a.D, nsplit, a.max_len,
                       a.rope_row_offset, a.rope_rows);
    KF_CHECK_LAUNCH();
    return KF_OK;
  }
  KF_LAUNCH("decode_generic", decode_generic_kernel<T>, dim3((a.B * a.Hq + 3) / 4), dim3(256), 0,
                     a.stream, (const T*)a.q_new, a.cos, a.sin, a.rope_row_offset, a.rope_rows,
                     a.max_len, (const T*)a.k_cache, (const T*)a.v_cache, a.lens, (T*)a.out, a.B,
                     a.Hq, a.Hkv, a.Smax, a.D, a.scale);
  KF_CHECK_LAUNCH();
  return KF_OK;
}

}  // namespace

size_t decode_workspace(int B, int Hq, int D, int max_len) {
  const size_t nsplit = (size_t)((max_len + CH - 1) / CH);
  return (size_t)B * Hq * nsplit * (D + 2) * sizeof(float);
}

int decode(const DecodeArgs& a, void* workspace) {
  switch (a.dtype) {
    case F32: return decode_typed<float>(a, workspace);
    case BF16: return decode_typed<bf16>(a, workspace);
    case F16: return decode_typed<_Float16>(a, workspace);
  }
  set_error("unsupported dtype %d", a.dtype);
  return KF_ERR_UNSUPPORTED;
}

int cache_append(const void* k_new, const void* v_new, const float* cos, const float* sin,
                 void* k_cache, void* v_cache, int start, int B, int Snew, int Hkv, int Smax,
                 int D, int dtype, hipStream_t stream) {
  // token i uses table row i (row_offset = start); the caller's table has Snew rows
  switch (dtype) {
    case F32:
      return launch_append<float>((const float*)k_new, (const float*)v_new, cos, sin,
                                  (float*)k_cache, (float*)v_cache, nullptr, start, start, Snew,
                                  Smax, B, Snew, Hkv, Smax, D, stream);
    case BF16:
      return launch_append<bf16>((const bf16*)k_new, (const bf16*)v_new, cos, sin,
                                 (bf16*)k_cache, (bf16*)v_cache, nullptr, start, start, Snew,
                                 Smax, B, Snew, Hkv, Smax, D, stream);
    case F16:
      return launch_append<_Float16>((const _Float16*)k_new, (const _Float16*)v_new, cos, sin,
                                     (_Float16*)k_cache, (_Float16*)v_cache, nullptr, start,
                                     start, Snew, Smax, B, Snew, Hkv, Smax, D, stream);
  }
  set_error("unsupported dtype %d", dtype);
  return KF_ERR_UNSUPPORTED;
}

}  // namespace kf
