// KV-cache decode (one new token per sequence) and cache append.
//
// decode = two launches on the caller's stream:
//  1. stream   persistent split-K attention: the key chunks of every
//              (sequence, KV head) pair form one list that the grid's
//              wavefronts split into equal contiguous ranges; each wavefront
//              streams its range once, serving all n_rep query heads of a
//              pair from that single read (the reference expands the cache
//              n_rep times first), and writes one partial (o, m, l) per pair
//              it touches, in float32.  The wavefront holding position
//              lens[b] rotates k_new (eager RoPE rounding) and writes it and
//              v_new into the caches (the reference's KVCache.update) instead
//              of reading that row.
//  2. merge    one workgroup per (b, hq) rescales and sums the partials.
// With QK-norm weights the per-head RMSNorm of q_new and k_new (the
// reference's q_norm / k_norm, applied before RoPE) happens where the rows
// are loaded, instead of in separate launches.
// float32 with D in {64, 128} and n_rep <= 16 appends here and decodes on the
// fp32 matrix cores (decode_f32, kf_f32.hip); other shapes (D not in {64, 128},
// or n_rep > 16) use decode_generic: one wavefront per (b, hq).
#include "kf_common.h"
#include "kf_internal.h"
#include "kf_mfma.h"

#include <algorithm>
#include <atomic>
#include <climits>
#include <mutex>
#include <type_traits>

namespace kf {

namespace {

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

// ---- streaming schedule -----------------------------------------------------
// Every (sequence b, KV head g) pair p = b * Hkv + g holds nck(b) = ceil((lens[b]
// + 1) / KC) chunks of KC keys (0 when the length is unusable).  The chunks of
// all pairs, in (b, g, key) order, form one list of C chunks, and wavefront w
// of the NW in the grid streams the contiguous range [w C / NW, (w + 1) C / NW):
// every wavefront reads the same number of bytes (to one chunk), whatever the
// lengths, and keeps its loads in flight across pair boundaries.  A wavefront
// writes one partial (o, m, l) per pair it touches, in slot w + p: the pairs a
// wavefront touches are consecutive and the wavefronts touching a pair are
// consecutive, so (w, p) -> w + p is one-to-one; NW + B * Hkv slots suffice.
constexpr int KC = 32;          // keys per chunk
constexpr int DEC_WAVES = 4;    // independent wavefronts per workgroup
constexpr int DEC_GRID_MAX = 512;

struct DecodeSched {
  const int32_t* lens;
  int B, Hkv, max_len;
  int64_t row_offset, rope_rows;
  __device__ __forceinline__ int nck(int b) const {
    const int len = lens[b];
    return decode_len_ok(len, max_len, row_offset, rope_rows) ? (len + KC) / KC : 0;
  }
};

__device__ __forceinline__ int wave_sum_int(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return __builtin_amdgcn_readfirstlane(v);
}

// Total chunks C over all pairs (wavefront-uniform).
__device__ __forceinline__ int total_chunks(const DecodeSched& s, int lane) {
  int tot = 0;
  for (int b0 = 0; b0 < s.B; b0 += 64) tot += wave_sum_int(b0 + lane < s.B ? s.nck(b0 + lane) : 0);
  return tot * s.Hkv;
}

// Sequence holding global chunk c (0 <= c < C) and the index of its first
// chunk, Hkv * (chunks of the sequences before it).  Wavefront-uniform.
__device__ __forceinline__ void locate_chunk(const DecodeSched& s, int c, int lane, int& b_out,
                                             int& base_out) {
  int run = 0;
  b_out = 0;
  base_out = 0;
  for (int b0 = 0; b0 < s.B; b0 += 64) {
    const int b = b0 + lane;
    const int n = (b < s.B ? s.nck(b) : 0) * s.Hkv;
    int incl = n;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(incl, o, 64);
      if (lane >= o) incl += y;
    }
    const uint64_t m = __builtin_amdgcn_ballot_w64(n > 0 && run + incl - n <= c && c < run + incl);
    if (m) {
      const int l = (int)__builtin_ctzll(m);
      b_out = b0 + l;
      base_out = run + __shfl(incl - n, l, 64);
      b_out = __builtin_amdgcn_readfirstlane(b_out);
      base_out = __builtin_amdgcn_readfirstlane(base_out);
      return;
    }
    run += __builtin_amdgcn_readfirstlane(__shfl(incl, 63, 64));
  }
}

// floor(x / d) for 0 <= x < 2^53 and 0 < d < 2^31: the double quotient is
// within one of the exact one (its relative error is below 2^-52 and x / d <
// 2^53), so one correction step either way makes it exact, in far fewer
// instructions than a 64-bit integer division.
__device__ __forceinline__ int64_t floor_div(int64_t x, int64_t d) {
  int64_t q = (int64_t)((double)x / (double)d);
  if (q * d > x)
    --q;
  else if ((q + 1) * d <= x)
    ++q;
  return q;
}

// First chunk of wavefront w's range, floor(w C / NW).
__device__ __forceinline__ int range_start(int w, int C, int NW) {
  return (int)floor_div((int64_t)w * C, NW);
}

// The wavefront whose range holds chunk c: the largest w with w C / NW <= c.
__device__ __forceinline__ int chunk_owner(int c, int C, int NW) {
  return (int)floor_div(((int64_t)c + 1) * NW - 1, C);
}

// Position in the chunk list: pair (b, g), local chunk lc of nck, new-token
// position len (keys 0 .. len are attended).
struct Cursor {
  int b, g, lc, nck, len;
};

__device__ __forceinline__ Cursor cursor_at(const DecodeSched& s, int c, int lane) {
  Cursor cur;
  int base;
  locate_chunk(s, c, lane, cur.b, base);
  cur.nck = max(s.nck(cur.b), 1);  // >= 1 for any c < C
  cur.len = s.lens[cur.b];
  const int rem = c - base;
  cur.g = rem / cur.nck;
  cur.lc = rem % cur.nck;
  return cur;
}

__device__ __forceinline__ void cursor_next(Cursor& cur, const DecodeSched& s) {
  if (++cur.lc < cur.nck) return;
  cur.lc = 0;
  if (++cur.g < s.Hkv) return;
  cur.g = 0;
  for (++cur.b; cur.b < s.B; ++cur.b) {
    cur.nck = s.nck(cur.b);
    if (cur.nck > 0) break;
  }
  if (cur.b < s.B) cur.len = s.lens[cur.b];
}

// Streaming split-K decode on MFMA.  Each wavefront walks its chunk range
// independently (no workgroup barriers).  Per chunk of KC = 32 keys of pair
// (b, g), with v_mfma_f32_16x16x32_bf16 / _f16 (operand layout below):
//   S^T = K q^T   two 16-key blocks; the pair's n_rep <= 16 query heads are the
//                 B-operand columns (zero-padded to 16), so one read of the KV
//                 head serves every head of the group
//   O^T += V^T P^T  V rows go to the wavefront's LDS tile and come back
//                 transposed (ds_read_b64_tr_b16) as the A operand; P^T is the
//                 B operand straight from the S registers
// Every global load is an ordinary compiler-tracked load into registers: the
// next chunk's K rows, V rows and, at a pair's first chunk, its q rows and
// RoPE table row (at the chunk holding position lens[b], the new token's k and
// v) are loaded while the current chunk is computed, and the compiler's own
// memory-counter waits cover them exactly.  A pair's start turns the q rows
// into the rotated q operand (RMS-normalised first with QK-norm weights); the
// chunk holding the new token rotates k_new, writes the new k / v rows into
// the caches (the reference's KVCache.update) and uses them in place of that
// row.  Rows past the pair's last key are loaded clamped and zeroed on the way
// into LDS (a clamped copy of a stale row times a zero probability stays 0).
//
// MFMA 16x16x32 operand layout (lane l, q4 = l / 16, j = 0..7):
//   A[m][k]: m = l % 16, k = 8 q4 + j     B[k][n]: n = l % 16, k = 8 q4 + j
//   C[m][n]: n = l % 16, register i holds m = 4 q4 + i
// S^T: m = key, n = head, k = head dim (32 ks + 8 q4 + j); the lane's C
// registers hold keys 4 q4 + i of each 16-key block, which, read as slots
// j < 4 (block 0) and j >= 4 (block 1), are the B operand of O^T += V^T P^T
// with k slot j <-> key (j < 4 ? 4 q4 + j : 16 + 4 q4 + j - 4).
typedef float f32x4v __attribute__((ext_vector_type(4)));

template <typename T, int D, bool QKN>
__global__ __launch_bounds__(256, 2) void decode_stream_kernel(
    const T* __restrict__ q_new, const T* __restrict__ k_new,
    const T* __restrict__ v_new, const float* __restrict__ cos, const float* __restrict__ sin,
    int64_t row_offset, int64_t rope_rows, int max_len, T* kc, T* vc,
    const int32_t* __restrict__ lens, float* __restrict__ opart, float* __restrict__ mlpart,
    int B, int Hq, int Hkv, int Smax, int n_rep, float scale_log2,
    const float* __restrict__ qnw, const float* __restrict__ knw, float eps) {
  using namespace mfma;
  constexpr int KT = D / 32;          // 32-dim k-steps of S
  constexpr int DB = D / 16;          // 16-dim output blocks
  constexpr int KR = D / 8;           // 16-byte chunks per row
  constexpr int HALF = D / 2;
  constexpr int VL = KC * KR / 64;    // 16-byte V loads per lane and chunk
  static_assert(KC == 32, "two 16-key blocks per chunk");
  struct WaveLds {
    T v[KC * D];   // the chunk's V rows, 16-byte chunks swizzled by row
    float cs[2][64];  // cos, sin row of the pair's new position
    T nw[D];       // rotated k_new
  };
  __shared__ __attribute__((aligned(16))) WaveLds lds_all[DEC_WAVES];

  const int w = wave_id(), lane = threadIdx.x & 63, q4 = lane >> 4, c16 = lane & 15;
  WaveLds& L = lds_all[w];
  const DecodeSched s{lens, B, Hkv, max_len, row_offset, rope_rows};
  const int NW = gridDim.x * DEC_WAVES, gw = blockIdx.x * DEC_WAVES + w;
  const int C = total_chunks(s, lane);
  const int c_lo = range_start(gw, C, NW), c_hi = range_start(gw + 1, C, NW);
  if (c_lo >= c_hi) return;

  // the chunk's rows, loaded one step ahead: each set is reloaded for the next
  // chunk as soon as this chunk's products have read it, so one register set
  // per operand keeps a chunk in flight
  u32x4 kreg[2][KT];  // key 16 kb + c16 of the chunk, dims 32 ks + 8 q4 .. + 7
  u32x4 vreg[VL];     // V row (64 j + lane) / KR, chunk (64 j + lane) % KR
  struct Stash {
    u32x4 q[KT];     // q row of head c16 (0 for c16 >= n_rep), dims 32 ks + 8 q4 .. + 7
    float cs[2];     // cos / sin of the new position, dim lane (< HALF)
    uint32_t kv[2];  // k_new / v_new, dims 2 lane, 2 lane + 1 (lane < D / 2)
  };
  // The cache is streamed once per step and at serving sizes does not fit the
  // MALL: non-temporal loads (~15% more HBM read rate than cached ones).
  auto load_k = [&](const Cursor& cur) {
    const int last = cur.len;  // keys 0 .. len
    const int64_t base = ((int64_t)cur.b * Hkv + cur.g) * Smax * D;
    const int r0 = cur.lc * KC;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int key = min(r0 + 16 * kb + c16, last);
#pragma unroll
      for (int ks = 0; ks < KT; ++ks)
        kreg[kb][ks] = __builtin_nontemporal_load((const u32x4*)(kc + base + (int64_t)key * D + 32 * ks + 8 * q4));
    }
  };
  auto load_v = [&](const Cursor& cur) {
    const int last = cur.len;
    const int64_t base = ((int64_t)cur.b * Hkv + cur.g) * Smax * D;
    const int r0 = cur.lc * KC;
#pragma unroll
    for (int j = 0; j < VL; ++j) {
      const int li = 64 * j + lane, row = li / KR, pc = li % KR;
      const int key = min(r0 + row, last);
      vreg[j] = __builtin_nontemporal_load((const u32x4*)(vc + base + (int64_t)key * D + 8 * pc));
    }
  };
  auto load_stash = [&](const Cursor& cur, Stash& st, bool pair_start, bool new_tok) {
    if (pair_start) {
      const int h = c16 < n_rep ? c16 : 0;
      const T* qr = q_new + ((int64_t)cur.b * Hq + (int64_t)cur.g * n_rep + h) * D;
#pragma unroll
      for (int ks = 0; ks < KT; ++ks) st.q[ks] = *(const u32x4*)(qr + 32 * ks + 8 * q4);
      const int64_t trow = (int64_t)cur.len - row_offset;
      const int e = lane < HALF ? lane : 0;
      st.cs[0] = cos[trow * HALF + e];
      st.cs[1] = sin[trow * HALF + e];
    }
    if (new_tok) {
      const int64_t row = ((int64_t)cur.b * Hkv + cur.g) * D;
      const int e = lane < D / 2 ? lane : 0;
      st.kv[0] = ((const uint32_t*)(k_new + row))[e];
      st.kv[1] = ((const uint32_t*)(v_new + row))[e];
    }
  };

  // transposed-read byte offsets of this lane in the V tile, per 16-dim block:
  // address lane a = c16 of group q4 reads row 4 q4 + a / 4, dims 16 blk +
  // 4 (a % 4) .. + 3 (the second read: row + 16, the same swizzle)
  // chunk (2 blk + x) of the row lands at (2 blk + x) ^ sw = 2 (blk ^ (sw >> 1)) +
  // (x ^ (sw & 1)): one xor per block
  const int tr_row = 4 * q4 + (c16 >> 2), tr_sw = swz<KR>(tr_row);
  const uint32_t tr_base = (uint32_t)((tr_row * KR + (((c16 & 3) >> 1) ^ (tr_sw & 1))) * 16 +
                                      (4 * (c16 & 1)) * 2);
  const int tr_hs = tr_sw >> 1;

  Stash st;
  u32x4 qf[KT];
  f32x4v acc[DB];
  float m = -INFINITY, lsum = 0.f;
  Cursor cc = cursor_at(s, c_lo, lane);  // chunk being computed
  Cursor ic = cc;                        // chunk being loaded
  load_stash(ic, st, true, ic.lc == ic.nck - 1);
  load_k(ic);
  load_v(ic);

  for (int i = c_lo; i < c_hi; ++i) {
    const bool seg_start = i == c_lo || cc.lc == 0;
    const bool has_new = cc.lc == cc.nck - 1;
    const int newrow = cc.len;
    const int r0 = cc.lc * KC;
    const int lim = newrow - r0;  // last valid key of the chunk, local
    const T* kvrow_k = nullptr;
    if (seg_start) {
      // the pair's cos / sin row into LDS, then the rotated q operand
      if (lane < HALF) {
        L.cs[0][lane] = st.cs[0];
        L.cs[1][lane] = st.cs[1];
      }
      float ss = 0.f;
      if constexpr (QKN) {
#pragma unroll
        for (int ks = 0; ks < KT; ++ks) {
          float x[8];
          unpack8<T>(st.q[ks], x);
#pragma unroll
          for (int j = 0; j < 8; ++j) ss += x[j] * x[j];
        }
        // the four lanes of one head (q4 = 0..3) hold its whole row
        ss += __shfl_xor(ss, 16, 64);
        ss += __shfl_xor(ss, 32, 64);
      }
#pragma unroll
      for (int ks = 0; ks < KT / 2; ++ks) {
        const int d0 = 32 * ks + 8 * q4;  // < HALF; its partner is d0 + HALF (ks + KT / 2)
        float x1[8], x2[8], r1[8], r2[8];
        unpack8<T>(st.q[ks], x1);
        unpack8<T>(st.q[ks + KT / 2], x2);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if constexpr (QKN) {
            x1[j] = rms_scale<T>(x1[j], ss, D, eps, qnw[d0 + j]);
            x2[j] = rms_scale<T>(x2[j], ss, D, eps, qnw[d0 + HALF + j]);
          }
          rope_pair<T>(x1[j], x2[j], L.cs[0][d0 + j], L.cs[1][d0 + j], r1[j], r2[j]);
        }
        const u32x4 z = {0u, 0u, 0u, 0u};
        qf[ks] = c16 < n_rep ? pack8<T>(r1) : z;
        qf[ks + KT / 2] = c16 < n_rep ? pack8<T>(r2) : z;
      }
      m = -INFINITY;
      lsum = 0.f;
#pragma unroll
      for (int blk = 0; blk < DB; ++blk) acc[blk] = f32x4v{0.f, 0.f, 0.f, 0.f};
    }
    uint32_t vnew = 0u;
    if (has_new) {
      // the new token: lane e < D / 2 holds dims 2e, 2e + 1; the RoPE partner
      // dims (+ HALF) sit in lane e ^ (HALF / 2)
      const int e = lane;
      const bool act = e < D / 2;
      const bool first = (e & (HALF / 2)) == 0;  // dims < HALF
      const uint32_t own = st.kv[0];
      const uint32_t par = (uint32_t)__shfl_xor((int)own, HALF / 2, 64);
      float x[2], y[2];
      unpack2<T>(own, x[0], x[1]);
      unpack2<T>(par, y[0], y[1]);
      const int dd = (2 * e) % HALF;  // table index of the pair
      if constexpr (QKN) {
        float ss = act ? x[0] * x[0] + x[1] * x[1] : 0.f;
        ss = wave_sum(ss);
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int d = act ? 2 * e + t : 0;
          const int dp = d ^ HALF;  // the partner dim
          x[t] = rms_scale<T>(x[t], ss, D, eps, knw[d]);
          y[t] = rms_scale<T>(y[t], ss, D, eps, knw[dp]);
        }
      }
      float r[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        float r1, r2;
        const float c = L.cs[0][dd + t], sn = L.cs[1][dd + t];
        if (first)
          rope_pair<T>(x[t], y[t], c, sn, r1, r2);
        else
          rope_pair<T>(y[t], x[t], c, sn, r1, r2);
        r[t] = first ? r1 : r2;
      }
      const uint32_t rk = pack2<T>(r[0], r[1]);
      const int64_t crow = (((int64_t)cc.b * Hkv + cc.g) * Smax + newrow) * D;
      if (act) {
        ((uint32_t*)L.nw)[e] = rk;
        ((uint32_t*)(kc + crow))[e] = rk;
        ((uint32_t*)(vc + crow))[e] = st.kv[1];
      }
      vnew = st.kv[1];
      kvrow_k = L.nw;
    }
    // the next chunk (possibly of the next pair): its pair data now, its K
    // rows once this chunk's S products have read kreg, its V rows once this
    // chunk's V rows are in LDS
    const bool more = i + 1 < c_hi;
    if (more) {
      cursor_next(ic, s);
      load_stash(ic, st, ic.lc == 0, ic.lc == ic.nck - 1);
    }
    if (has_new) {
      // the lane of the new row takes its key from L.nw
      const int loc = newrow - r0;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const bool is_new = 16 * kb + c16 == loc;
#pragma unroll
        for (int ks = 0; ks < KT; ++ks) {
          const u32x4 nk = *(const u32x4*)(kvrow_k + 32 * ks + 8 * q4);
          kreg[kb][ks] = is_new ? nk : kreg[kb][ks];
        }
      }
    }
    // S^T and the online softmax (per head: lanes c16, c16 + 16, + 32, + 48)
    f32x4v sc[2];
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      sc[kb] = f32x4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KT; ++ks)
        sc[kb] = mfma16<T>(as_bf16x8(kreg[kb][ks]), as_bf16x8(qf[ks]), sc[kb]);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int local = 16 * kb + 4 * q4 + t;
        sc[kb][t] = local > lim ? -INFINITY : sc[kb][t] * scale_log2;
        tmax = fmaxf(tmax, sc[kb][t]);
      }
    }
    if (more) load_k(ic);
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float mnew = fmaxf(m, tmax);  // finite: key r0 is valid
    const float alpha = fast_exp2(m - mnew);
    float p[8];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      p[t] = fast_exp2(sc[0][t] - mnew);
      p[4 + t] = fast_exp2(sc[1][t] - mnew);
    }
    float psum = 0.f;
#pragma unroll
    for (int t = 0; t < 8; ++t) psum += p[t];
    lsum = lsum * alpha + psum;
    m = mnew;
    const u32x4 pb = {pack2<T>(p[0], p[1]), pack2<T>(p[2], p[3]), pack2<T>(p[4], p[5]), pack2<T>(p[6], p[7])};
    // V rows into the tile (rows past the last key as zeros, the new row from v_new)
#pragma unroll
    for (int j = 0; j < VL; ++j) {
      const int li = 64 * j + lane, row = li / KR, pc = li % KR;
      const u32x4 z = {0u, 0u, 0u, 0u};
      *(u32x4*)(L.v + (row * KR + (pc ^ swz<KR>(row))) * 8) = row > lim ? z : vreg[j];
    }
    // the V registers are free: the next chunk's rows (loaded one step ahead,
    // like its K rows, which were issued at the top of this step)
    if (more) load_v(ic);
    if (has_new && lane < D / 2) {
      const int row = newrow - r0, el = 2 * lane, pc = el >> 3;
      *(uint32_t*)(L.v + (row * KR + (pc ^ swz<KR>(row))) * 8 + (el & 7)) = vnew;
    }
#pragma unroll
    for (int blk = 0; blk < DB; ++blk) acc[blk] *= alpha;
#pragma unroll
    for (int blk = 0; blk < DB; ++blk) {
      const char* base = (const char*)L.v + tr_base + (uint32_t)((blk ^ tr_hs) * 32);
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)base);
      const s16x4 hi =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(base + 16 * KR * 16));
      typedef short s16x8 __attribute__((ext_vector_type(8)));
      const s16x8 vt = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      acc[blk] = mfma16<T>(__builtin_bit_cast(bf16x8, vt), as_bf16x8(pb), acc[blk]);
    }
    if (!more || has_new) {
      // the pair's part of this wavefront ends: partial (o, m, l) to slot gw + p
      float ltot = lsum + __shfl_xor(lsum, 16, 64);
      ltot += __shfl_xor(ltot, 32, 64);
      if (c16 < n_rep) {
        const int64_t slot = (int64_t)gw + (int64_t)cc.b * Hkv + cc.g;
        float* orow = opart + (slot * n_rep + c16) * D;
#pragma unroll
        for (int blk = 0; blk < DB; ++blk) *(f32x4v*)(orow + 16 * blk + 4 * q4) = acc[blk];
        if (q4 == 0) *(float2*)(mlpart + (slot * n_rep + c16) * 2) = make_float2(m, ltot);
      }
    }
    cursor_next(cc, s);
  }
}

// One wavefront per (b, hq), four per workgroup: the partials of the
// wavefronts whose ranges met pair (b, g) are rescaled to a common maximum and
// summed.  The slot range comes from one pass over lens; the partial outputs
// of the first MERGE_PRE slots are then loaded together with the (m, l)
// values, so a merge costs two dependent memory round trips.
constexpr int MERGE_PRE = 16;

template <typename T, int D>
__global__ __launch_bounds__(256) void decode_merge_kernel(
    const float* __restrict__ opart, const float* __restrict__ mlpart,
    const int32_t* __restrict__ lens, T* __restrict__ out, int B, int Hq, int Hkv, int NW,
    int max_len, int64_t row_offset, int64_t rope_rows) {
  constexpr int PER = D / 64;
  const int lane = threadIdx.x & 63;
  const int bh = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (bh >= B * Hq) return;
  const int b = bh / Hq, hq = bh % Hq, n_rep = Hq / Hkv, g = hq / n_rep, h = hq % n_rep;
  const DecodeSched s{lens, B, Hkv, max_len, row_offset, rope_rows};
  // C, Hkv * (chunks of the sequences before b) and b's chunks, from one
  // load of lens per lane
  int tot = 0, pre = 0, n = 0;
  for (int b0 = 0; b0 < B; b0 += 64) {
    const int nb = b0 + lane < B ? s.nck(b0 + lane) : 0;
    tot += wave_sum_int(nb);
    pre += wave_sum_int(b0 + lane < b ? nb : 0);
    if (b >= b0 && b < b0 + 64) n = __shfl(nb, b - b0, 64);
  }
  const int C = tot * Hkv;
  T* orow = out + (int64_t)bh * D + lane;
  if (n == 0) {  // unusable length: NaN output, no cache write happened
#pragma unroll
    for (int k = 0; k < PER; ++k) orow[64 * k] = from_f32<T>(NAN);
    return;
  }
  const int c0 = pre * Hkv + g * n;
  const int w0 = chunk_owner(c0, C, NW), ns = chunk_owner(c0 + n - 1, C, NW) - w0 + 1;
  const int64_t first = ((int64_t)w0 + (int64_t)b * Hkv + g) * n_rep + h;  // slot w0 + p's row
  const float* ob = opart + first * D + lane;
  const float* mb = mlpart + first * 2;
  const int64_t ost = (int64_t)n_rep * D, mst = (int64_t)n_rep * 2;  // per slot
  // wavefronts with an empty range (C < NW) between w0 and w1 wrote nothing:
  // their slots hold stale data, get weight 0 and are never added
  auto live = [&](int j) {
    return j < ns && range_start(w0 + j, C, NW) != range_start(w0 + j + 1, C, NW);
  };
  float po[MERGE_PRE][PER];
#pragma unroll
  for (int j = 0; j < MERGE_PRE; ++j)
#pragma unroll
    for (int k = 0; k < PER; ++k) po[j][k] = j < ns ? ob[j * ost + 64 * k] : 0.f;
  const bool live0 = live(lane);
  float2 ml0 = make_float2(-INFINITY, 0.f);
  if (live0) ml0 = *(const float2*)(mb + lane * mst);
  float M = ml0.x;
  for (int j = 64 + lane; j < ns; j += 64)
    if (live(j)) M = fmaxf(M, mb[j * mst]);
  M = wave_max(M);
  const float wgt0 = live0 ? fast_exp2(ml0.x - M) : 0.f;
  float lt = live0 ? ml0.y * wgt0 : 0.f;
  for (int j = 64 + lane; j < ns; j += 64)
    if (live(j)) lt += mb[j * mst + 1] * fast_exp2(mb[j * mst] - M);
  lt = wave_sum(lt);
  float o[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) o[k] = 0.f;
#pragma unroll
  for (int j = 0; j < MERGE_PRE; ++j) {
    const float wj = __shfl(wgt0, j, 64);
    if (wj != 0.f)
#pragma unroll
      for (int k = 0; k < PER; ++k) o[k] += po[j][k] * wj;
  }
  for (int j = MERGE_PRE; j < ns; ++j) {
    const float wj = j < 64 ? __shfl(wgt0, j, 64)
                            : (live(j) ? fast_exp2(mb[j * mst] - M) : 0.f);
    if (wj != 0.f)
#pragma unroll
      for (int k = 0; k < PER; ++k) o[k] += ob[j * ost + 64 * k] * wj;
  }
  const float inv = 1.f / lt;
#pragma unroll
  for (int k = 0; k < PER; ++k) orow[64 * k] = from_f32<T>(o[k] * inv);
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

// Grid of the stream kernel: two workgroups per CU, at most DEC_GRID_MAX.
int decode_grid() { return std::max(1, std::min(DEC_GRID_MAX, 2 * device_cu_count())); }

template <typename T, int D>
int launch_stream(const DecodeArgs& a, float* opart, float* mlpart, int grid) {
  const bool qkn = a.q_norm_w != nullptr;
  KF_LAUNCH("decode_stream",
            (qkn ? decode_stream_kernel<T, D, true> : decode_stream_kernel<T, D, false>),
            dim3(grid), dim3(64 * DEC_WAVES), 0, a.stream, (const T*)a.q_new,
            (const T*)a.k_new, (const T*)a.v_new, a.cos, a.sin, a.rope_row_offset,
            a.rope_rows, a.max_len, (T*)a.k_cache, (T*)a.v_cache, a.lens, opart, mlpart,
            a.B, a.Hq, a.Hkv, a.Smax, a.Hq / a.Hkv, a.scale * kLog2e, a.q_norm_w, a.k_norm_w,
            a.norm_eps);
  KF_CHECK_LAUNCH();
  return KF_OK;
}

// Partial slots of the stream kernel: one per (wavefront, pair it touches),
// at most the grid's wavefronts plus the pairs.
size_t decode_slots(int B, int Hkv) { return (size_t)DEC_GRID_MAX * DEC_WAVES + (size_t)B * Hkv; }

template <typename T>
int decode_typed(const DecodeArgs& a, void* workspace) {
  int rc = KF_OK;
  const int n_rep = a.Hq / a.Hkv;
  const bool fast = (__is_same(T, bf16) || __is_same(T, f16)) && (a.D == 64 || a.D == 128) &&
                    n_rep <= 16 &&
                    (int64_t)a.B * a.Hkv * ((a.max_len + KC - 1) / KC) < INT_MAX &&
                    ((uintptr_t)a.q_new | (uintptr_t)a.k_new | (uintptr_t)a.v_new |
                     (uintptr_t)a.k_cache | (uintptr_t)a.v_cache) % 16 == 0;
  if (fast) {
    const size_t slots = decode_slots(a.B, a.Hkv);
    float* opart = (float*)workspace;
    float* mlpart = opart + slots * n_rep * a.D;
    const int grid = decode_grid();
    if constexpr (__is_same(T, bf16) || __is_same(T, f16)) {
      rc = a.D == 128 ? launch_stream<T, 128>(a, opart, mlpart, grid)
                      : launch_stream<T, 64>(a, opart, mlpart, grid);
      if (rc) return rc;
      KF_LAUNCH("decode_merge",
                (a.D == 128 ? decode_merge_kernel<T, 128> : decode_merge_kernel<T, 64>),
                dim3((a.B * a.Hq + 3) / 4), dim3(256), 0, a.stream, opart, mlpart, a.lens,
                (T*)a.out, a.B, a.Hq, a.Hkv, grid * DEC_WAVES, a.max_len, a.rope_row_offset,
                a.rope_rows);
      KF_CHECK_LAUNCH();
      return KF_OK;
    }
  }
  rc = launch_append<T>((const T*)a.k_new, (const T*)a.v_new, a.cos, a.sin, (T*)a.k_cache,
                        (T*)a.v_cache, a.lens, 0, a.rope_row_offset, a.rope_rows, a.max_len, a.B,
                        1, a.Hkv, a.Smax, a.D, a.stream, a.k_norm_w, a.norm_eps);
  if (rc) return rc;
  if (__is_same(T, float) && decode_f32_supported(a))
    return decode_f32(a, workspace, decode_slots(a.B, a.Hkv));
  KF_LAUNCH("decode_generic", decode_generic_kernel<T>, dim3((a.B * a.Hq + 3) / 4), dim3(256), 0,
                     a.stream, (const T*)a.q_new, a.cos, a.sin, a.rope_row_offset, a.rope_rows,
                     a.max_len, (const T*)a.k_cache, (const T*)a.v_cache, a.lens, (T*)a.out, a.B,
                     a.Hq, a.Hkv, a.Smax, a.D, a.scale, a.q_norm_w, a.norm_eps);
  KF_CHECK_LAUNCH();
  return KF_OK;
}

}  // namespace

size_t decode_workspace(int B, int Hq, int Hkv, int D, int max_len) {
  (void)max_len;
  const size_t n_rep = (size_t)(Hq / Hkv);
  return decode_slots(B, Hkv) * n_rep * (size_t)(D + 2) * sizeof(float);
}

// ---- allocation-free decode ---------------------------------------------------
// The decode's partials for callers that cannot allocate: one array in device
// memory for the life of the process, a copy per device the library runs on.
// In host code `scratch` only names the symbol; the device address of the
// current device's copy comes from hipGetSymbolAddress, looked up once per
// device and kept.  Nothing in it needs clearing: a call reads only the
// partial slots it wrote itself.
static __device__ __align__(256) unsigned char scratch[DECODE_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;
}  // namespace

int decode_scratch(void** ptr) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("decode scratch: no usable current device (%s)", hipGetErrorString(e));
    return KF_ERR_HIP;
  }
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || p == nullptr) {
        set_error("decode scratch: hipGetSymbolAddress failed (%s)", hipGetErrorString(e));
        return KF_ERR_HIP;
      }
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *ptr = p;
  return KF_OK;
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
