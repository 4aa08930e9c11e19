// Generic attention kernels: any head_dim (even, <= 256) and dtype f32/bf16/f16.
//
// These carry the float32 path (the debug configuration is checked at 1e-5)
// and every shape the MFMA kernels do not cover.  One wavefront owns one query
// row (forward, dQ) or one key row (dK/dV); lane `l` owns head-dim elements
// l, l+64, l+128, l+192.  Dot products are wavefront reductions.  RoPE is
// applied at load from the float32 tables with the reference's eager rounding.
#include "kf_common.h"
#include "kf_internal.h"

namespace kf {

namespace {

constexpr int kMaxPer = 4;  // head_dim <= 256 = 4 * 64 lanes

// Load row `x` (head_dim D, stride 1) rotated by table row `trow`.
// `rot`=false loads it unchanged.  Lane owns d = lane + 64*i.
template <typename T>
__device__ __forceinline__ void load_row(const T* __restrict__ x, const float* __restrict__ cos,
                                         const float* __restrict__ sin, int64_t trow, int D,
                                         bool rot, int lane, float* out) {
  const int half = D / 2;
#pragma unroll
  for (int i = 0; i < kMaxPer; ++i) {
    const int d = lane + 64 * i;
    float r = 0.f;
    if (d < D) {
      const float xd = to_f32(x[d]);
      if (rot) {
        const int j = d < half ? d : d - half;
        const float x1 = d < half ? xd : to_f32(x[d - half]);
        const float x2 = d < half ? to_f32(x[d + half]) : xd;
        float r1, r2;
        rope_pair<T>(x1, x2, cos[trow * half + j], sin[trow * half + j], r1, r2);
        r = d < half ? r1 : r2;
      } else {
        r = xd;
      }
    }
    out[i] = r;
  }
}

__device__ __forceinline__ float wdot(const float* a, const float* b) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kMaxPer; ++i) s += a[i] * b[i];
  return wave_sum(s);
}

// Apply the RoPE backward to a wavefront-distributed fp32 row and store it.
template <typename T>
__device__ __forceinline__ void store_row_rope_bwd(float* __restrict__ lds_row, const float* g,
                                                   const float* __restrict__ cos,
                                                   const float* __restrict__ sin, int64_t trow,
                                                   int D, int lane, T* __restrict__ dst) {
  const int half = D / 2;
#pragma unroll
  for (int i = 0; i < kMaxPer; ++i) {
    const int d = lane + 64 * i;
    if (d < D) lds_row[d] = g[i];
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
#pragma unroll
  for (int i = 0; i < kMaxPer; ++i) {
    const int d = lane + 64 * i;
    if (d < D) {
      const int j = d < half ? d : d - half;
      const float g1 = lds_row[j], g2 = lds_row[j + half];
      float d1, d2;
      rope_pair_bwd<T>(g1, g2, cos[trow * half + j], sin[trow * half + j], d1, d2);
      dst[d] = from_f32<T>(d < half ? d1 : d2);
    }
  }
}

// Explicit masks (doc ids, key validity; each may be null) for query i, key j
// of the batch row whose ids start at roff; di = doc[i].
__device__ __forceinline__ bool sees(const int32_t* __restrict__ doc,
                                     const int32_t* __restrict__ kv, int64_t roff, int i, int j,
                                     int causal, int di) {
  return (!causal || j <= i) && (!doc || doc[roff + j] == di) && (!kv || kv[roff + j] != 0);
}

// Whether query i sees any key at all (wavefront-uniform).  Only a key
// validity mask can leave a row empty; such a row attends every key instead
// (the reference's NaN guard, mask | ~mask.any(-1)).
__device__ __forceinline__ bool sees_any(const int32_t* __restrict__ doc,
                                         const int32_t* __restrict__ kv, int64_t roff, int i,
                                         int Sk, int causal, int di, int lane) {
  if (!kv) return true;
  const int end = causal ? min(Sk, i + 1) : Sk;
  for (int j0 = 0; j0 < end; j0 += 64) {
    const int j = j0 + lane;
    if (__builtin_amdgcn_ballot_w64(j < end && sees(doc, kv, roff, i, j, causal, di)) != 0)
      return true;
  }
  return false;
}

}  // namespace

// ------------------------------------------------------------------ forward
// grid.x = ceil(B*Hq*Sq / 4), block = 256 (4 waves, one query row each).
template <typename T>
__global__ __launch_bounds__(256) void fwd_generic_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const float* __restrict__ cos, const float* __restrict__ sin, T* __restrict__ out,
    float* __restrict__ lse, int B, int Sq, int Sk, int Hq, int Hkv, int D, int64_t ksb,
    int64_t kss, int64_t ksh, int64_t vsb, int64_t vss, int64_t vsh, int k_rotated, int causal,
    const int32_t* __restrict__ doc, const int32_t* __restrict__ kv, float scale) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= (int64_t)B * Hq * Sq) return;
  const int i = (int)(row % Sq);
  const int hq = (int)((row / Sq) % Hq);
  const int b = (int)(row / ((int64_t)Sq * Hq));
  const int g = hq / (Hq / Hkv);

  float qr[kMaxPer];
  load_row<T>(q + (((int64_t)b * Sq + i) * Hq + hq) * D, cos, sin, i, D, true, lane, qr);

  float acc[kMaxPer] = {0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  const int64_t roff = (int64_t)b * Sk;
  const int di = doc ? doc[roff + i] : 0;
  const bool guard = !sees_any(doc, kv, roff, i, Sk, causal, di, lane);
  const int kend = causal && !guard ? min(Sk, i + 1) : Sk;
  for (int j = 0; j < kend; ++j) {
    if (!guard && !sees(doc, kv, roff, i, j, causal, di)) continue;  // masked key
    float kr[kMaxPer], vv[kMaxPer];
    load_row<T>(k + b * ksb + j * kss + g * ksh, cos, sin, j, D, !k_rotated, lane, kr);
    load_row<T>(v + b * vsb + j * vss + g * vsh, cos, sin, 0, D, false, lane, vv);
    const float s = wdot(qr, kr) * scale;
    const float mn = fmaxf(m, s);
    const float alpha = expf(m - mn);
    const float p = expf(s - mn);
    l = l * alpha + p;
#pragma unroll
    for (int t = 0; t < kMaxPer; ++t) acc[t] = acc[t] * alpha + p * vv[t];
    m = mn;
  }
  const float inv = 1.f / l;
  T* o = out + (((int64_t)b * Sq + i) * Hq + hq) * D;
#pragma unroll
  for (int t = 0; t < kMaxPer; ++t) {
    const int d = lane + 64 * t;
    if (d < D) o[d] = from_f32<T>(acc[t] * inv);
  }
  if (lse != nullptr && lane == 0) lse[((int64_t)b * Hq + hq) * Sq + i] = m + logf(l);
}

// ------------------------------------------------------------------ backward
// delta[b,h,i] = sum_d dO[b,i,h,d] * O[b,i,h,d]
// With explicit masks it also writes guard[b, i] (1: row i sees no key and
// attends every key), once per (b, i).
template <typename T>
__global__ __launch_bounds__(256) void bwd_delta_kernel(const T* __restrict__ o,
                                                        const T* __restrict__ dout,
                                                        float* __restrict__ delta,
                                                        int32_t* __restrict__ guard, int B, int S,
                                                        int Hq, int D, int causal,
                                                        const int32_t* __restrict__ doc,
                                                        const int32_t* __restrict__ kv) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= (int64_t)B * S * Hq) return;  // row enumerates (b, i, h) in BSHD order
  const int64_t base = row * D;
  float s = 0.f;
  for (int d = lane; d < D; d += 64) s += to_f32(o[base + d]) * to_f32(dout[base + d]);
  s = wave_sum(s);
  const int h = (int)(row % Hq);
  const int i = (int)((row / Hq) % S);
  const int b = (int)(row / ((int64_t)Hq * S));
  if (lane == 0) delta[((int64_t)b * Hq + h) * S + i] = s;
  if (h == 0) {
    const int64_t roff = (int64_t)b * S;
    const int di = doc ? doc[roff + i] : 0;
    const bool g = !sees_any(doc, kv, roff, i, S, causal, di, lane);
    if (lane == 0) guard[roff + i] = g;
  }
}

// dQ: one wave per (b, hq, i); iterates keys j <= i.
template <typename T>
__global__ __launch_bounds__(256) void bwd_dq_generic_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const float* __restrict__ cos, const float* __restrict__ sin, const T* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ delta, T* __restrict__ dq, int B,
    int S, int Hq, int Hkv, int D, int causal, const int32_t* __restrict__ doc,
    const int32_t* __restrict__ kv, const int32_t* __restrict__ guard, float scale) {
  __shared__ float lds[4][256];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t row = (int64_t)blockIdx.x * 4 + w;
  if (row >= (int64_t)B * Hq * S) return;
  const int i = (int)(row % S);
  const int hq = (int)((row / S) % Hq);
  const int b = (int)(row / ((int64_t)S * Hq));
  const int g = hq / (Hq / Hkv);
  const int64_t qoff = (((int64_t)b * S + i) * Hq + hq) * D;
  float qr[kMaxPer], dor[kMaxPer];
  load_row<T>(q + qoff, cos, sin, i, D, true, lane, qr);
  load_row<T>(dout + qoff, cos, sin, 0, D, false, lane, dor);
  const float L = lse[((int64_t)b * Hq + hq) * S + i];
  const float Di = delta[((int64_t)b * Hq + hq) * S + i];
  float acc[kMaxPer] = {0.f, 0.f, 0.f, 0.f};
  const int64_t roff = (int64_t)b * S;
  const int di = doc ? doc[roff + i] : 0;
  const bool grd = guard[roff + i] != 0;
  const int kend = causal && !grd ? i + 1 : S;
  for (int j = 0; j < kend; ++j) {
    if (!grd && !sees(doc, kv, roff, i, j, causal, di)) continue;
    const int64_t koff = (((int64_t)b * S + j) * Hkv + g) * D;
    float kr[kMaxPer], vv[kMaxPer];
    load_row<T>(k + koff, cos, sin, j, D, true, lane, kr);
    load_row<T>(v + koff, cos, sin, 0, D, false, lane, vv);
    const float s = wdot(qr, kr) * scale;
    const float p = expf(s - L);
    const float dp = wdot(dor, vv);
    const float ds = p * (dp - Di);
#pragma unroll
    for (int t = 0; t < kMaxPer; ++t) acc[t] += ds * kr[t];
  }
#pragma unroll
  for (int t = 0; t < kMaxPer; ++t) acc[t] *= scale;
  store_row_rope_bwd<T>(lds[w], acc, cos, sin, i, D, lane, dq + qoff);
}

// dK, dV: one wave per (b, g, j); iterates the group's query heads and i >= j.
template <typename T>
__global__ __launch_bounds__(256) void bwd_dkdv_generic_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const float* __restrict__ cos, const float* __restrict__ sin, const T* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ delta, T* __restrict__ dk,
    T* __restrict__ dv, int B, int S, int Hq, int Hkv, int D, int causal,
    const int32_t* __restrict__ doc, const int32_t* __restrict__ kv,
    const int32_t* __restrict__ guard, float scale) {
  __shared__ float lds[4][256];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t row = (int64_t)blockIdx.x * 4 + w;
  if (row >= (int64_t)B * Hkv * S) return;
  const int j = (int)(row % S);
  const int g = (int)((row / S) % Hkv);
  const int b = (int)(row / ((int64_t)S * Hkv));
  const int n_rep = Hq / Hkv;
  const int64_t koff = (((int64_t)b * S + j) * Hkv + g) * D;
  float kr[kMaxPer], vv[kMaxPer];
  load_row<T>(k + koff, cos, sin, j, D, true, lane, kr);
  load_row<T>(v + koff, cos, sin, 0, D, false, lane, vv);
  float adk[kMaxPer] = {0.f, 0.f, 0.f, 0.f}, adv[kMaxPer] = {0.f, 0.f, 0.f, 0.f};
  const int64_t roff = (int64_t)b * S;
  for (int hl = 0; hl < n_rep; ++hl) {
    const int hq = g * n_rep + hl;
    // a guarded row (with a validity mask) may sit before j
    for (int i = causal && !kv ? j : 0; i < S; ++i) {
      const int di = doc ? doc[roff + i] : 0;
      if (!guard[roff + i] && !sees(doc, kv, roff, i, j, causal, di)) continue;
      const int64_t qoff = (((int64_t)b * S + i) * Hq + hq) * D;
      float qr[kMaxPer], dor[kMaxPer];
      load_row<T>(q + qoff, cos, sin, i, D, true, lane, qr);
      load_row<T>(dout + qoff, cos, sin, 0, D, false, lane, dor);
      const float L = lse[((int64_t)b * Hq + hq) * S + i];
      const float Di = delta[((int64_t)b * Hq + hq) * S + i];
      const float s = wdot(qr, kr) * scale;
      const float p = expf(s - L);
      const float dp = wdot(dor, vv);
      const float ds = p * (dp - Di);
#pragma unroll
      for (int t = 0; t < kMaxPer; ++t) {
        adv[t] += p * dor[t];
        adk[t] += ds * qr[t];
      }
    }
  }
#pragma unroll
  for (int t = 0; t < kMaxPer; ++t) {
    adk[t] *= scale;
    const int d = lane + 64 * t;
    if (d < D) dv[koff + d] = from_f32<T>(adv[t]);
  }
  store_row_rope_bwd<T>(lds[w], adk, cos, sin, j, D, lane, dk + koff);
}

// ------------------------------------------------------------------ capture
// P[b,h,i,j] = exp(s_ij - lse_i) (0 where masked), float32.  One wave per row;
// lane-strided over keys so each store instruction writes 64 consecutive floats.
template <typename T>
__global__ __launch_bounds__(256) void capture_probs_generic_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const float* __restrict__ cos,
    const float* __restrict__ sin, const float* __restrict__ lse, float* __restrict__ probs,
    int B, int Sq, int Sk, int Hq, int Hkv, int D, int64_t ksb, int64_t kss, int64_t ksh,
    int k_rotated, int causal, const int32_t* __restrict__ doc, const int32_t* __restrict__ kv,
    float scale) {
  __shared__ float lds[4][256];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t row = (int64_t)blockIdx.x * 4 + w;
  if (row >= (int64_t)B * Hq * Sq) return;
  const int i = (int)(row % Sq);
  const int hq = (int)((row / Sq) % Hq);
  const int b = (int)(row / ((int64_t)Sq * Hq));
  const int g = hq / (Hq / Hkv);
  float qr[kMaxPer];
  load_row<T>(q + (((int64_t)b * Sq + i) * Hq + hq) * D, cos, sin, i, D, true, lane, qr);
  // stash the rotated query row in LDS so each lane can run its own dot products
#pragma unroll
  for (int t = 0; t < kMaxPer; ++t) {
    const int d = lane + 64 * t;
    if (d < D) lds[w][d] = qr[t];
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  const float L = lse[((int64_t)b * Hq + hq) * Sq + i];
  float* prow = probs + row * Sk;
  const int half = D / 2;
  const int64_t roff = (int64_t)b * Sk;
  const int di = doc ? doc[roff + i] : 0;
  const bool guard = !sees_any(doc, kv, roff, i, Sk, causal, di, lane);
  for (int j = lane; j < Sk; j += 64) {
    float p = 0.f;
    if (guard || sees(doc, kv, roff, i, j, causal, di)) {
      const T* kr = k + b * ksb + j * kss + g * ksh;
      float s = 0.f;
      for (int d = 0; d < half; ++d) {
        float k1 = to_f32(kr[d]), k2 = to_f32(kr[d + half]);
        if (!k_rotated) {
          float r1, r2;
          rope_pair<T>(k1, k2, cos[(int64_t)j * half + d], sin[(int64_t)j * half + d], r1, r2);
          k1 = r1;
          k2 = r2;
        }
        s += lds[w][d] * k1 + lds[w][d + half] * k2;
      }
      p = expf(s * scale - L);
    }
    prow[j] = p;
  }
}

// ------------------------------------------------------------------ launchers
template <typename T>
int launch_fwd_generic(const FwdArgs& a) {
  const int64_t rows = (int64_t)a.B * a.Hq * a.Sq;
  dim3 grid((unsigned)((rows + 3) / 4));
  KF_LAUNCH("fwd_generic", (fwd_generic_kernel<T>), grid, dim3(256), 0, a.stream, (const T*)a.q,
                     (const T*)a.k, (const T*)a.v, a.cos, a.sin, (T*)a.out, a.lse, a.B, a.Sq,
                     a.Sk, a.Hq, a.Hkv, a.D, a.ksb, a.kss, a.ksh, a.vsb, a.vss, a.vsh,
                     a.k_rotated, a.causal, a.doc, a.kvalid, a.scale);
  KF_CHECK_LAUNCH();
  return KF_OK;
}

template <typename T>
int launch_bwd_generic(const BwdArgs& a, void* workspace) {
  float* delta = (float*)workspace;
  int32_t* guard = (int32_t*)(delta + (size_t)a.B * a.Hq * a.S);
  const int64_t qrows = (int64_t)a.B * a.Hq * a.S;
  const int64_t krows = (int64_t)a.B * a.Hkv * a.S;
  KF_LAUNCH("bwd_delta_generic", (bwd_delta_kernel<T>), dim3((unsigned)((qrows + 3) / 4)), dim3(256), 0,
                     a.stream, (const T*)a.out, (const T*)a.dout, delta, guard, a.B, a.S, a.Hq,
                     a.D, a.causal, a.doc, a.kvalid);
  KF_CHECK_LAUNCH();
  KF_LAUNCH("bwd_dq_generic", (bwd_dq_generic_kernel<T>), dim3((unsigned)((qrows + 3) / 4)), dim3(256), 0,
                     a.stream, (const T*)a.q, (const T*)a.k, (const T*)a.v, a.cos, a.sin,
                     (const T*)a.dout, a.lse, delta, (T*)a.dq, a.B, a.S, a.Hq, a.Hkv, a.D,
                     a.causal, a.doc, a.kvalid, guard, a.scale);
  KF_CHECK_LAUNCH();
  KF_LAUNCH("bwd_dkdv_generic", (bwd_dkdv_generic_kernel<T>), dim3((unsigned)((krows + 3) / 4)), dim3(256),
                     0, a.stream, (const T*)a.q, (const T*)a.k, (const T*)a.v, a.cos, a.sin,
                     (const T*)a.dout, a.lse, delta, (T*)a.dk, (T*)a.dv, a.B, a.S, a.Hq, a.Hkv,
                     a.D, a.causal, a.doc, a.kvalid, guard, a.scale);
  KF_CHECK_LAUNCH();
  return KF_OK;
}

template <typename T>
int launch_capture_probs_generic(const FwdArgs& a, const float* lse, float* probs) {
  const int64_t rows = (int64_t)a.B * a.Hq * a.Sq;
  KF_LAUNCH("capture_probs_generic", (capture_probs_generic_kernel<T>), dim3((unsigned)((rows + 3) / 4)),
                     dim3(256), 0, a.stream, (const T*)a.q, (const T*)a.k, a.cos, a.sin, lse,
                     probs, a.B, a.Sq, a.Sk, a.Hq, a.Hkv, a.D, a.ksb, a.kss, a.ksh, a.k_rotated,
                     a.causal, a.doc, a.kvalid, a.scale);
  KF_CHECK_LAUNCH();
  return KF_OK;
}

int fwd_generic(const FwdArgs& a) {
  switch (a.dtype) {
    case F32: return launch_fwd_generic<float>(a);
    case BF16: return launch_fwd_generic<bf16>(a);
    case F16: return launch_fwd_generic<_Float16>(a);
  }
  set_error("unsupported dtype %d", a.dtype);
  return KF_ERR_UNSUPPORTED;
}

size_t bwd_generic_workspace(int B, int S, int Hq) {
  return (size_t)B * Hq * S * sizeof(float) + (size_t)B * S * sizeof(int32_t);
}

int bwd_generic(const BwdArgs& a, void* workspace) {
  switch (a.dtype) {
    case F32: return launch_bwd_generic<float>(a, workspace);
    case BF16: return launch_bwd_generic<bf16>(a, workspace);
    case F16: return launch_bwd_generic<_Float16>(a, workspace);
  }
  set_error("unsupported dtype %d", a.dtype);
  return KF_ERR_UNSUPPORTED;
}

int capture_probs_generic(const FwdArgs& a, const float* lse, float* probs) {
  switch (a.dtype) {
    case F32: return launch_capture_probs_generic<float>(a, lse, probs);
    case BF16: return launch_capture_probs_generic<bf16>(a, lse, probs);
    case F16: return launch_capture_probs_generic<_Float16>(a, lse, probs);
  }
  set_error("unsupported dtype %d", a.dtype);
  return KF_ERR_UNSUPPORTED;
}

}  // namespace kf
