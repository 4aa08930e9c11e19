// KV-cache decode (one new token per sequence) and cache append.
//
// decode = two launches on the caller's stream:
//  1. split    split-K attention: workgroup (split, b, kv head) streams CH keys
//              of one KV head once and serves all n_rep query heads of the
//              group from that single read (the reference expands the cache
//              n_rep times first).  D/8 threads share a key row, each loading
//              16 contiguous bytes, so a pass reads whole rows coalesced.
//              Writes partial (o, m, l) per (b, hq, split) in float32.  The
//              split holding position lens[b] rotates k_new (eager RoPE
//              rounding) and writes it and v_new into the caches (the
//              reference's KVCache.update) instead of reading that row.
//  2. merge    one wavefront per (b, hq) rescales and sums the partials.
// With QK-norm weights the per-head RMSNorm of q_new and k_new (the
// reference's q_norm / k_norm, applied before RoPE) happens where the rows
// are loaded, instead of in separate launches.
// Shapes outside the fast path (dtype other than bf16, D not in {64, 128}, or
// n_rep > 32) use decode_generic: one wavefront per (b, hq).
#include "kf_common.h"
#include "kf_internal.h"
#include "kf_mfma.h"

namespace kf {

namespace {

constexpr int CH = 1024;  // keys per split

// RMSNorm of one element given its row's sum of squares, as the reference's
// RMSNorm computes it (kempnerforge/model/norm.py:22-27): float32
// x * rsqrt(mean(x^2) + eps), times the weight, rounded to the storage type.
template <typename T>
__device__ __forceinline__ float rms_scale(float x, float ss, int D, float eps, float w) {
  const float r = rsqrtf(ss / (float)D + eps);
  return round_to<T>((x * r) * w);
}

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
                                                     int Smax, int D,
                                                     const float* __restrict__ knw, float eps) {
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
  float x1 = to_f32(k_new[src + d]), x2 = to_f32(k_new[src + d + half]);
  if (knw != nullptr) {  // QK-norm of the key row (the whole row's sum of squares)
    float ss = 0.f;
    for (int e = 0; e < D; ++e) {
      const float x = to_f32(k_new[src + e]);
      ss += x * x;
    }
    x1 = rms_scale<T>(x1, ss, D, eps, knw[d]);
    x2 = rms_scale<T>(x2, ss, D, eps, knw[d + half]);
  }
  float r1, r2;
  rope_pair<T>(x1, x2, cos[trow * half + d], sin[trow * half + d], r1, r2);
  kc[dst + d] = from_f32<T>(r1);
  kc[dst + d + half] = from_f32<T>(r2);
  vc[dst + d] = v_new[src + d];
  vc[dst + d + half] = v_new[src + d + half];
}

// Split-K decode on MFMA.  Workgroup = (split of CH keys, b, KV head), 4
// independent wavefronts of NCH chunks x KC keys each.  Per chunk:
//   S^T = K q^T   v_mfma_f32_32x32x16_bf16, the KV group's n_rep query heads
//                 as the B-operand columns (zero-padded to 32), so a lane owns
//                 one head and the online softmax is lane-local; K rows go
//                 from HBM straight into A-operand registers.
//   O^T += V^T P^T  V rows staged in LDS by direct global->LDS loads and read
//                 transposed (ds_read_b64_tr_b16).
// Loads run one chunk ahead (K registers and V LDS buffers double-buffered),
// so every wavefront keeps a chunk in flight while it computes the previous.
// Chunks past the split's end load a clamped row (L2 hits) and are not
// computed, which keeps the memory-counter accounting static.  The
// wavefronts' (m, l, o) are merged in LDS into one partial per
// (b, head, split).  The wavefront owning position lens[b] rotates k_new,
// writes k and v into the caches and uses them in place of that row.
// 16-byte global load issued from inline asm, so that the compiler's
// memory-counter bookkeeping does not see it: the caller waits with
// wait_vm<N>() and passes the destination through it before any use.  (Its
// own count would be off by the untracked direct-to-LDS loads in between.)
template <int OFF>
__device__ __forceinline__ void gload16(u32x4& r, uint32_t voff, const void* base) {
  asm volatile(KF_VMEM_ASM_NOPS "global_load_dwordx4 %0, %1, %2 offset:%3"
               : "=v"(r)
               : "v"(voff), "s"(base), "n"(OFF)
               : "memory");
}
template <int N, int I = 0>
__device__ __forceinline__ void gload16_row(u32x4* r, uint32_t voff, const void* base) {
  if constexpr (I < N) {
    gload16<32 * I>(r[I], voff, base);
    gload16_row<N, I + 1>(r, voff, base);
  }
}
// s_waitcnt vmcnt(N), then the registers in r[0..n) count as written here
template <int N, int n>
__device__ __forceinline__ void wait_vm(u32x4* r) {
  asm volatile("s_waitcnt vmcnt(%1)" : "+v"(r[0]) : "n"(N) : "memory");
#pragma unroll
  for (int i = 1; i < n; ++i) asm volatile("" : "+v"(r[i])::"memory");
}

// Longest-processing-time-first order of the split grid.  A full split of CH
// keys takes ~40 us of one workgroup slot's share of HBM at C4's size, and the
// grid runs in 2-3 rounds of slots, so a round that ends on full splits idles
// half the machine for tens of microseconds.  Flat block id f maps to: first
// every full split (b, g, k < len_b / CH), then each sequence's partial split
// (len_b % CH keys) ordered by size, largest first, so the last workgroups
// dispatched are the shortest.  One wavefront computes it (lane = batch row,
// B <= 64) and leaves {split, b, g} in job[], split = -1 for no work.
__device__ __forceinline__ void decode_job(const int32_t* __restrict__ lens, int B, int Hkv,
                                           int max_len, int64_t row_offset, int64_t rope_rows,
                                           int f, int lane, int* job) {
  int Lb = 0;
  if (lane < B) {
    const int len = lens[lane];
    Lb = decode_len_ok(len, max_len, row_offset, rope_rows) ? len + 1 : 0;
  }
  const int nf = Lb / CH, r = Lb % CH;
  int incl = nf * Hkv;  // inclusive prefix of full splits over the batch rows
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o, 64);
    if (lane >= o) incl += y;
  }
  const int F = __shfl(incl, 63, 64);
  int sp = -1, bb = 0, gg = 0;
  if (f < F) {
    const uint64_t m = __builtin_amdgcn_ballot_w64(incl - nf * Hkv <= f && f < incl);
    bb = (int)__builtin_ctzll(m);
    const int nfb = __shfl(nf, bb, 64);
    const int within = f - (__shfl(incl, bb, 64) - nfb * Hkv);
    sp = within % nfb;
    gg = within / nfb;
  } else {
    const int p = (f - F) / Hkv;
    gg = (f - F) % Hkv;
    // rank of this row's partial split: larger first, ties by row
    int rank = 0;
    for (int j = 0; j < B; ++j) {
      const int rj = __shfl(r, j, 64);
      rank += (rj > r) || (rj == r && j < lane);
    }
    const uint64_t m = __builtin_amdgcn_ballot_w64(r > 0 && rank == p);
    if (m) {
      bb = (int)__builtin_ctzll(m);
      sp = __shfl(nf, bb, 64);
    }
  }
  if (lane == 0) {
    job[0] = sp;
    job[1] = bb;
    job[2] = gg;
  }
}

constexpr int DEC_WAVES = 4;
constexpr int KC = 32;                    // keys per chunk
constexpr int NCH = CH / (DEC_WAVES * KC);  // chunks per wavefront

template <int D, bool QKN>
__global__ __launch_bounds__(256, 2) void decode_split_kernel(
    const bf16* __restrict__ q_new, const bf16* __restrict__ k_new,
    const bf16* __restrict__ v_new, const float* __restrict__ cos, const float* __restrict__ sin,
    int64_t row_offset, int64_t rope_rows, int max_len, bf16* kc, bf16* vc,
    const int32_t* __restrict__ lens, float* __restrict__ opart, float* __restrict__ mpart,
    float* __restrict__ lpart, int Hq, int Hkv, int Smax, int nsplit, int n_rep,
    float scale_log2, const float* __restrict__ qnw, const float* __restrict__ knw, float eps) {
  using namespace mfma;
  constexpr int KS = D / 16, DT = D / 32, KR = D / 8, HALF = D / 2;
  constexpr int WKEYS = NCH * KC;      // keys per wavefront
  constexpr int VI = KC * KR / 64;     // LDS copies per V chunk
  constexpr int PER_CHUNK = KS + VI;   // vector-memory instructions per chunk
  static_assert(PER_CHUNK < 64, "vmcnt range");
  __shared__ __attribute__((aligned(16))) bf16 sV[DEC_WAVES][2][KC * D];
  __shared__ __attribute__((aligned(16))) bf16 sNew[2][D];
  __shared__ float sML[DEC_WAVES][2][32];
  static_assert(sizeof(sV) >= DEC_WAVES * 32 * D * sizeof(float), "merge buffer");

  // which split this workgroup computes: longest first (see decode_job)
  __shared__ int sJob[3];
  const int B = gridDim.y / Hkv;
  if (B <= 64) {
    if (threadIdx.x < 64)
      decode_job(lens, B, Hkv, max_len, row_offset, rope_rows,
                 blockIdx.y * gridDim.x + blockIdx.x, threadIdx.x, sJob);
  } else if (threadIdx.x == 0) {
    sJob[0] = blockIdx.x;
    sJob[1] = blockIdx.y / Hkv;
    sJob[2] = blockIdx.y % Hkv;
  }
  __syncthreads();
  const int sp_idx = sJob[0];
  if (sp_idx < 0) return;
  const int b = sJob[1], g = sJob[2];
  if (!decode_len_ok(lens[b], max_len, row_offset, rope_rows)) return;
  const int L = lens[b] + 1;
  const int newrow = L - 1;  // the token being decoded
  const int k0 = sp_idx * CH;
  if (k0 >= L) return;
  const int k1 = min(k0 + CH, L);
  const int w = wave_id(), lane = threadIdx.x & 63, hh = lane >> 5, c32 = lane & 31;
  const int64_t trow = (int64_t)newrow - row_offset;
  const int kw0 = k0 + w * WKEYS;                                   // first key of the wavefront
  const int nvc = min(max((k1 - kw0 + KC - 1) / KC, 0), NCH);       // chunks holding keys
  const bool own_new = newrow >= kw0 && newrow < kw0 + WKEYS;

  bf16* kb = kc + ((int64_t)b * Hkv + g) * Smax * D;
  bf16* vb = vc + ((int64_t)b * Hkv + g) * Smax * D;
  const float* cr = cos + trow * HALF;
  const float* sr = sin + trow * HALF;

  // the new token: rotated k and v into the caches and into sNew
  if (own_new) {
    const bf16* kn = k_new + ((int64_t)b * Hkv + g) * D;
    const bf16* vn = v_new + ((int64_t)b * Hkv + g) * D;
    // lanes 0 .. HALF/8-1 hold elements d0..d0+7 and d0+HALF..+7 of the key
    const bool kl = lane < HALF / 8;
    const int d0 = kl ? 8 * lane : 0;
    float x1[8], x2[8];
    if (kl) {
      unpack8(*(const u32x4*)(kn + d0), x1);
      unpack8(*(const u32x4*)(kn + d0 + HALF), x2);
    }
    if constexpr (QKN) {
      float ss = 0.f;
      if (kl)
#pragma unroll
        for (int j = 0; j < 8; ++j) ss += x1[j] * x1[j] + x2[j] * x2[j];
#pragma unroll
      for (int o = 1; o < HALF / 8; o <<= 1) ss += __shfl_xor(ss, o, 64);
      if (kl)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          x1[j] = rms_scale<bf16>(x1[j], ss, D, eps, knw[d0 + j]);
          x2[j] = rms_scale<bf16>(x2[j], ss, D, eps, knw[d0 + HALF + j]);
        }
    }
    if (kl) {
      float r1[8], r2[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) rope_pair<bf16>(x1[j], x2[j], cr[d0 + j], sr[d0 + j], r1[j], r2[j]);
      const u32x4 a1 = pack8(r1), a2 = pack8(r2);
      *(u32x4*)(sNew[0] + d0) = a1;
      *(u32x4*)(sNew[0] + d0 + HALF) = a2;
      *(u32x4*)(kb + (int64_t)newrow * D + d0) = a1;
      *(u32x4*)(kb + (int64_t)newrow * D + d0 + HALF) = a2;
    } else if (lane >= 32 && lane < 32 + KR) {
      const int d0 = 8 * (lane - 32);
      const u32x4 x = *(const u32x4*)(vn + d0);
      *(u32x4*)(sNew[1] + d0) = x;
      *(u32x4*)(vb + (int64_t)newrow * D + d0) = x;
    }
  }
  // query fragment (B operand): column = head of the group, slots = d
  u32x4 qf[KS];
  if constexpr (QKN) {
    // lanes l and l ^ 32 hold the two halves of one query row: both load,
    // one exchange completes the row's sum of squares
    const bool ql = c32 < n_rep;
    const bf16* qr = q_new + ((int64_t)b * Hq + g * n_rep + (ql ? c32 : 0)) * D;
    u32x4 ra[KS / 2], rb[KS / 2];
    float ss = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS / 2; ++ks) {
      const int d0 = 16 * ks + 8 * hh;
      ra[ks] = *(const u32x4*)(qr + d0);
      rb[ks] = *(const u32x4*)(qr + d0 + HALF);
      float x1[8], x2[8];
      unpack8(ra[ks], x1);
      unpack8(rb[ks], x2);
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += x1[j] * x1[j] + x2[j] * x2[j];
    }
    ss = pair_sum32(ss);
#pragma unroll
    for (int ks = 0; ks < KS / 2; ++ks) {
      const int d0 = 16 * ks + 8 * hh;
      float x1[8], x2[8], r1[8], r2[8];
      unpack8(ra[ks], x1);
      unpack8(rb[ks], x2);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        x1[j] = rms_scale<bf16>(x1[j], ss, D, eps, qnw[d0 + j]);
        x2[j] = rms_scale<bf16>(x2[j], ss, D, eps, qnw[d0 + HALF + j]);
        rope_pair<bf16>(x1[j], x2[j], cr[d0 + j], sr[d0 + j], r1[j], r2[j]);
      }
      const u32x4 z = {0u, 0u, 0u, 0u};
      qf[ks] = ql ? pack8(r1) : z;
      qf[ks + KS / 2] = ql ? pack8(r2) : z;
    }
  } else if (c32 < n_rep) {
    const bf16* qr = q_new + ((int64_t)b * Hq + g * n_rep + c32) * D;
#pragma unroll
    for (int ks = 0; ks < KS / 2; ++ks) {
      const int d0 = 16 * ks + 8 * hh;
      float x1[8], x2[8], r1[8], r2[8];
      unpack8(*(const u32x4*)(qr + d0), x1);
      unpack8(*(const u32x4*)(qr + d0 + HALF), x2);
#pragma unroll
      for (int j = 0; j < 8; ++j) rope_pair<bf16>(x1[j], x2[j], cr[d0 + j], sr[d0 + j], r1[j], r2[j]);
      qf[ks] = pack8(r1);
      qf[ks + KS / 2] = pack8(r2);
    }
  } else {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = u32x4{0u, 0u, 0u, 0u};
  }
  // finish every tracked load's consumer before the first direct-to-LDS load
  // is issued (see gload16)
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(qf[ks])::"memory");

  // chunk loads: K rows into registers, V rows into this wavefront's LDS buffer
  u32x4 kreg[2][KS];
  auto issue = [&](int c, u32x4 (&kr)[KS], bf16* tV) {
    const int r0 = kw0 + c * KC;
    const int key = min(r0 + c32, k1 - 1);
    gload16_row<KS>(kr, (uint32_t)(key * D + 8 * hh) * 2u, kb);
    const uint32_t tva = lds_addr(tV);
#pragma unroll
    for (int j = 0; j < VI; ++j) {
      const int Lc = j * 64 + lane;
      const int row = Lc / KR, pc = Lc % KR;
      const int lc = pc ^ swz<KR>(row);
      const uint32_t grow = (uint32_t)min(r0 + row, k1 - 1);
      dma16(tva + j * 1024, (grow * D + (uint32_t)lc * 8u) * 2u, vb);
    }
  };

  const TrOffsets<D> tro = tr_offsets<D>(lane);
  float m = -INFINITY, lsum = 0.f;
  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[dt][i] = 0.f;

  issue(0, kreg[0], sV[w][0]);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (c + 1 < NCH) issue(c + 1, kreg[(c + 1) & 1], sV[w][(c + 1) & 1]);
    // K of chunk c has landed once only V(c) and the next chunk are pending;
    // waited on every path, so the registers stay owned until they land
    if (c + 1 < NCH)
      wait_vm<VI + PER_CHUNK, KS>(kreg[c & 1]);
    else
      wait_vm<VI, KS>(kreg[c & 1]);
    if (c < nvc) {
      const int r0 = kw0 + c * KC;
      bf16* tV = sV[w][c & 1];
      const bool has_new = own_new && newrow >= r0 && newrow < r0 + KC;
      // the new row's lane takes k from sNew (a select, so that no load
      // target is overwritten under divergence, which would force a full
      // memory-counter wait)
      u32x4 nk[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) nk[ks] = u32x4{0u, 0u, 0u, 0u};
      if (has_new) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) nk[ks] = *(const u32x4*)(sNew[0] + 16 * ks + 8 * hh);
      }
      const bool is_new = has_new && c32 == newrow - r0;
      bf16x8 kf[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kf[ks] = as_bf16x8(is_new ? nk[ks] : kreg[c & 1][ks]);
      f32x16 sc;
#pragma unroll
      for (int i = 0; i < 16; ++i) sc[i] = 0.f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks], as_bf16x8(qf[ks]), sc, 0, 0, 0);
      const int lim = k1 - 1 - r0;  // last valid key of the chunk, local
      float tmax = -INFINITY;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int local = 8 * (i >> 2) + 4 * hh + (i & 3);
        sc[i] = local > lim ? -INFINITY : sc[i] * scale_log2;
        tmax = fmaxf(tmax, sc[i]);
      }
      tmax = pair_max32(tmax);
      const float mnew = fmaxf(m, tmax);  // finite: key r0 is valid
      const float alpha = fast_exp2(m - mnew);
      float psum = 0.f;
      u32x4 pk[2];
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        const float p0 = fast_exp2(sc[i] - mnew), p1 = fast_exp2(sc[i + 1] - mnew);
        psum += p0 + p1;
        pk[i >> 3][(i & 7) >> 1] = pack2(p0, p1);
      }
      lsum = lsum * alpha + psum;
      m = mnew;
      // V of chunk c has landed once only the next chunk's loads are pending
      if (c + 1 < NCH)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PER_CHUNK) : "memory");
      else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      if (lim < KC - 1) {
        // rows past the split's end hold clamped copies of a row that may be
        // stale (the slot being written): zero them so 0 * V stays 0
        for (int Lc = (lim + 1) * KR + lane; Lc < KC * KR; Lc += 64)
          *(u32x4*)(tV + Lc * 8) = u32x4{0u, 0u, 0u, 0u};
      }
      if (has_new && lane < KR) {
        const int row = newrow - r0;
        *(u32x4*)(tV + (row * KR + (lane ^ swz<KR>(row))) * 8) = *(const u32x4*)(sNew[1] + 8 * lane);
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[dt][i] *= alpha;
#pragma unroll
      for (int cc = 0; cc < 2; ++cc)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const bf16x8 a = lds_frag_t<D>(tV, tro, cc, dt);
          acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, as_bf16x8(pk[cc]), acc[dt], 0, 0, 0);
        }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  const float ltot = pair_sum32(lsum);
  // merge the wavefronts: (m, l) per head, then o through LDS (reuses sV)
  if (hh == 0) {
    sML[w][0][c32] = m;
    sML[w][1][c32] = ltot;
  }
  __syncthreads();
  // [wave][D][32 heads], head index XOR-swizzled by d so that both the column
  // writes below and the row reads after are conflict-free
  float* so = (float*)&sV[0][0][0];
  auto so_at = [&](int ww, int d, int h) { return ((ww * D + d) << 5) + (h ^ ((d >> 1) & 31)); };
  float M = -INFINITY;
#pragma unroll
  for (int ww = 0; ww < DEC_WAVES; ++ww) M = fmaxf(M, sML[ww][0][c32]);
  const float wgt = m == -INFINITY ? 0.f : fast_exp2(m - M);
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int d = 32 * dt + 8 * (i >> 2) + 4 * hh + (i & 3);
      so[so_at(w, d, c32)] = acc[dt][i] * wgt;
    }
  __syncthreads();
  for (int it = threadIdx.x; it < n_rep * D; it += 256) {
    const int hr = it / D, d = it % D;
    float o = 0.f;
#pragma unroll
    for (int ww = 0; ww < DEC_WAVES; ++ww) o += so[so_at(ww, d, hr)];
    const int64_t ph = ((int64_t)b * Hq + g * n_rep + hr) * nsplit + sp_idx;
    opart[ph * D + d] = o;
    if (d == 0) {
      float Mh = -INFINITY;
#pragma unroll
      for (int ww = 0; ww < DEC_WAVES; ++ww) Mh = fmaxf(Mh, sML[ww][0][hr]);
      float lh = 0.f;
#pragma unroll
      for (int ww = 0; ww < DEC_WAVES; ++ww)
        lh += sML[ww][0][hr] == -INFINITY ? 0.f : sML[ww][1][hr] * fast_exp2(sML[ww][0][hr] - Mh);
      mpart[ph] = Mh;
      lpart[ph] = lh;
    }
  }
}

// One workgroup of D threads per (b, hq): every thread rescales and sums its
// output element over the splits (independent loads, unrolled).
template <typename T>
__global__ __launch_bounds__(256) void decode_merge_kernel(const float* __restrict__ opart,
                                                           const float* __restrict__ mpart,
                                                           const float* __restrict__ lpart,
                                                           const int32_t* __restrict__ lens,
                                                           T* __restrict__ out, int Hq, int D,
                                                           int nsplit, int max_len,
                                                           int64_t row_offset,
                                                           int64_t rope_rows) {
  __shared__ float sw[1024];
  __shared__ float sinv;
  const int bh = blockIdx.x;
  const int b = bh / Hq;
  const int d = threadIdx.x;
  if (!decode_len_ok(lens[b], max_len, row_offset, rope_rows)) {
    if (d < D) out[(int64_t)bh * D + d] = from_f32<T>(NAN);
    return;
  }
  const int ns = min((lens[b] + 1 + CH - 1) / CH, 1024);  // <= nsplit (lens[b] < max_len)
  const int64_t base = (int64_t)bh * nsplit;
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    float M = -INFINITY;
    for (int s0 = lane; s0 < ns; s0 += 64) M = fmaxf(M, mpart[base + s0]);
    M = wave_max(M);
    float lt = 0.f;
    for (int s0 = lane; s0 < ns; s0 += 64) {
      const float wgt = fast_exp2(mpart[base + s0] - M);
      sw[s0] = wgt;
      lt += lpart[base + s0] * wgt;
    }
    lt = wave_sum(lt);
    if (lane == 0) sinv = 1.f / lt;
  }
  __syncthreads();
  if (d >= D) return;
  float o = 0.f;
  int s = 0;
  for (; s + 4 <= ns; s += 4) {
    const float a0 = opart[(base + s) * D + d], a1 = opart[(base + s + 1) * D + d];
    const float a2 = opart[(base + s + 2) * D + d], a3 = opart[(base + s + 3) * D + d];
    o += a0 * sw[s] + a1 * sw[s + 1] + a2 * sw[s + 2] + a3 * sw[s + 3];
  }
  for (; s < ns; ++s) o += opart[(base + s) * D + d] * sw[s];
  out[(int64_t)bh * D + d] = from_f32<T>(o * sinv);
}

// One wavefront per (b, hq); keys 0..lens[b] read from the (already appended)
// cache.  Any D <= 256.
template <typename T>
__global__ __launch_bounds__(256) void decode_generic_kernel(
    const T* __restrict__ q_new, const float* __restrict__ cos, const float* __restrict__ sin,
    int64_t row_offset, int64_t rope_rows, int max_len, const T* __restrict__ kc,
    const T* __restrict__ vc, const int32_t* __restrict__ lens, T* __restrict__ out, int B,
    int Hq, int Hkv, int Smax, int D, float scale, const float* __restrict__ qnw, float eps) {
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
  float ss = 0.f;  // QK-norm: the query row's sum of squares
  if (qnw != nullptr) {
    for (int d = lane; d < D; d += 64) ss += to_f32(qr[d]) * to_f32(qr[d]);
    ss = wave_sum(ss);
  }
  float qv[4], acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = lane + 64 * i;
    qv[i] = 0.f;
    if (d < D) {
      const int j = d < half ? d : d - half;
      float x1 = to_f32(qr[j]), x2 = to_f32(qr[j + half]);
      if (qnw != nullptr) {
        x1 = rms_scale<T>(x1, ss, D, eps, qnw[j]);
        x2 = rms_scale<T>(x2, ss, D, eps, qnw[j + half]);
      }
      float r1, r2;
      rope_pair<T>(x1, x2, cos[trow * half + j], sin[trow * half + j], r1, r2);
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
                  int max_len, int B, int Snew, int Hkv, int Smax, int D, hipStream_t stream,
                  const float* knw = nullptr, float eps = 0.f) {
  const int64_t n = (int64_t)B * Snew * Hkv * (D / 2);
  if (n == 0) return KF_OK;
  KF_LAUNCH("kv_append", append_kernel<T>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                     k_new, v_new, cos, sin, kc, vc, lens, start, row_offset, rope_rows, max_len,
                     B, Snew, Hkv, Smax, D, knw, eps);
  KF_CHECK_LAUNCH();
  return KF_OK;
}

template <int D>
int launch_split(const DecodeArgs& a, float* opart, float* mpart, float* lpart, int nsplit) {
  const bool qkn = a.q_norm_w != nullptr;
  KF_LAUNCH("decode_split", (qkn ? decode_split_kernel<D, true> : decode_split_kernel<D, false>),
            dim3(nsplit, a.B * a.Hkv), dim3(256), 0,
            a.stream, (const bf16*)a.q_new, (const bf16*)a.k_new, (const bf16*)a.v_new, a.cos,
            a.sin, a.rope_row_offset, a.rope_rows, a.max_len, (bf16*)a.k_cache, (bf16*)a.v_cache,
            a.lens, opart, mpart, lpart, a.Hq, a.Hkv, a.Smax, nsplit, a.Hq / a.Hkv,
            a.scale * kLog2e, a.q_norm_w, a.k_norm_w, a.norm_eps);
  KF_CHECK_LAUNCH();
  return KF_OK;
}

template <typename T>
int decode_typed(const DecodeArgs& a, void* workspace) {
  int rc = KF_OK;
  const int n_rep = a.Hq / a.Hkv;
  const bool fast = __is_same(T, bf16) && (a.D == 64 || a.D == 128) && n_rep <= 32 &&
                    (a.max_len + CH - 1) / CH <= 1024 &&
                    ((uintptr_t)a.q_new | (uintptr_t)a.k_new | (uintptr_t)a.v_new |
                     (uintptr_t)a.k_cache | (uintptr_t)a.v_cache) % 16 == 0;
  if (fast) {
    const int nsplit = (a.max_len + CH - 1) / CH;
    float* opart = (float*)workspace;
    float* mpart = opart + (size_t)a.B * a.Hq * nsplit * a.D;
    float* lpart = mpart + (size_t)a.B * a.Hq * nsplit;
    rc = a.D == 128 ? launch_split<128>(a, opart, mpart, lpart, nsplit)
                    : launch_split<64>(a, opart, mpart, lpart, nsplit);
    if (rc) return rc;
    KF_LAUNCH("decode_merge", decode_merge_kernel<T>, dim3(a.B * a.Hq), dim3(a.D), 0, a.stream,
              opart, mpart, lpart, a.lens, (T*)a.out, a.Hq, a.D, nsplit, a.max_len,
              a.rope_row_offset, a.rope_rows);
    KF_CHECK_LAUNCH();
    return KF_OK;
  }
  rc = launch_append<T>((const T*)a.k_new, (const T*)a.v_new, a.cos, a.sin, (T*)a.k_cache,
                        (T*)a.v_cache, a.lens, 0, a.rope_row_offset, a.rope_rows, a.max_len, a.B,
                        1, a.Hkv, a.Smax, a.D, a.stream, a.k_norm_w, a.norm_eps);
  if (rc) return rc;
  KF_LAUNCH("decode_generic", decode_generic_kernel<T>, dim3((a.B * a.Hq + 3) / 4), dim3(256), 0,
                     a.stream, (const T*)a.q_new, a.cos, a.sin, a.rope_row_offset, a.rope_rows,
                     a.max_len, (const T*)a.k_cache, (const T*)a.v_cache, a.lens, (T*)a.out, a.B,
                     a.Hq, a.Hkv, a.Smax, a.D, a.scale, a.q_norm_w, a.norm_eps);
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
