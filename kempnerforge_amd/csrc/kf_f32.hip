// float32 attention on the fp32 matrix cores (v_mfma_f32_16x16x4_f32): the
// forward, dQ and dK/dV, the KV-cache decode and the probability capture of
// the reference's mixed_precision = "fp32" (kempnerforge/config/training.py:31;
// attention at kempnerforge/model/attention.py:228-231 then runs SDPA in
// float32), causal or full attention, with packed documents or key padding
// (one kind at a time), head_dim 64 or 128.  Nothing is rounded below float32:
// the products are exact and the sums accumulate in float32, as the
// reference's float32 SDPA does (other head sizes and both masks at once stay
// on the generic kernels).
//
// One MFMA multiplies a 16x4 A by a 4x16 B into a 16x16 C: lane l holds
// A[l % 16][l / 16], B[l / 16][l % 16] and C[4 (l / 16) + r][l % 16] in its
// register r = 0..3.  Each kernel orients its score tiles so that l % 16 runs
// over the rows the kernel owns (query rows in the forward and dQ, key rows in
// dK/dV): row statistics and accumulators stay in the lane, and a score tile's
// C registers are the B operand of the next product as they are — MFMA kk of
// that product contracts, in lane group g = l / 16, over row
// 16 (kk / 4) + 4 g + kk % 4 of the C tile, which lane (g, l % 16) holds in
// register kk % 4 of block kk / 4.
//
// The head dimension of a contraction over D is split over the four lane
// groups so that a lane holds both halves of each RoPE pair: group g holds the
// 16-byte chunks (D/32) g + j of the first half and the same chunks of the
// second half (chunk_of), so the rows a lane loads itself rotate in registers.
//
// LDS tiles are [32 rows][D] floats with 16-byte chunk c of row r at position
// c ^ (r % 16): the chunk reads (16 consecutive rows, one chunk per pass) and
// the element reads (rows 4 apart, 16 consecutive floats each) both meet 64
// distinct banks.  Tiles reach LDS by direct global->LDS loads one tile ahead,
// into the other of two buffers, one barrier per tile; the tiles that need
// RoPE (K, and Q in dK/dV) come from a prepass that writes the rotated rows.
#include "kf_internal.h"
#include "kf_mfma.h"

namespace kf {

namespace {

using mfma::row_info;
using mfma::RowInfo;
using mfma::wave_id;
using mfma::xcd_logical_id;

constexpr int F_ROWS = 64;  // query rows per workgroup (forward, dQ): 4 wavefronts x 16
constexpr int F_BN = 32;    // keys per tile (forward, dQ), query positions per tile (dK/dV)
constexpr int F_BK = 64;    // keys per workgroup (dK/dV): 4 wavefronts x 16

__device__ __forceinline__ f32x4 mma(float a, float b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// j-th 16-byte chunk (j < D/16) of lane group g's share of a D-float row
template <int D>
__device__ __forceinline__ int chunk_of(int j, int g) {
  constexpr int H = D / 32;
  return j < H ? H * g + j : D / 8 + H * g + (j - H);
}
// float index of chunk c of row r of an LDS tile
template <int D>
__device__ __forceinline__ int tix(int r, int c) {
  return (r * (D / 4) + (c ^ (r & 15))) * 4;
}
// element (r, d) of an LDS tile
template <int D>
__device__ __forceinline__ float tel(const float* t, int r, int d) {
  return t[tix<D>(r, d >> 2) + (d & 3)];
}

// over the four lanes l % 16 + 16 g of one row
__device__ __forceinline__ float quad_max(float x) {
  x = fmaxf(x, __shfl_xor(x, 16, 64));
  return fmaxf(x, __shfl_xor(x, 32, 64));
}
__device__ __forceinline__ float quad_sum(float x) {
  x += __shfl_xor(x, 16, 64);
  return x + __shfl_xor(x, 32, 64);
}

__device__ __forceinline__ void rope4(f32x4& x1, f32x4& x2, const f32x4& c, const f32x4& s) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float r1, r2;
    rope_pair<float>(x1[e], x2[e], c[e], s[e], r1, r2);
    x1[e] = r1;
    x2[e] = r2;
  }
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

typedef double f64x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f64x4 to_f64(const f32x4& x) {
  return f64x4{(double)x[0], (double)x[1], (double)x[2], (double)x[3]};
}
__device__ __forceinline__ f32x4 to_f32x4(const f64x4& x) {
  return f32x4{(float)x[0], (float)x[1], (float)x[2], (float)x[3]};
}

// [32 rows][D] floats, rows `ld` floats apart from the wavefront-uniform base
// g, into a swizzled LDS tile by direct global->LDS loads: each instruction
// moves 64 lanes x 16 bytes into 1 KB of contiguous LDS, so a lane loads the
// chunk that belongs at its LDS position; the 4 wavefronts split the
// instructions.  Rows at or past rows_valid repeat row rows_valid - 1 (finite
// values, which the callers' masks multiply by zero).  Completion: the
// caller's lds_copy_wait and barrier.
template <int D, int ROWS = F_BN>
__device__ __forceinline__ void tile_dma(const float* g, uint32_t ld, float* lds, int w, int lane,
                                         int rows_valid) {
  constexpr int R = D / 4, PER = ROWS * R / 64 / 4;
  asm volatile("" : "+v"(lane));  // offsets recomputed per call, not kept live across the loop
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int L = (w * PER + j) * 64 + lane, row = L / R, pc = L % R;
    const uint32_t off =
        ((uint32_t)min(row, rows_valid - 1) * ld + (uint32_t)(pc ^ (row & 15)) * 4u) * 4u;
    mfma::dma16(mfma::lds_addr(lds + (w * PER + j) * 256), off, g);
  }
}

// A row's D/16 chunks of lane group g (chunk_of order), RoPE'd at table row
// `pos` when rot; zero when !valid.
template <int D>
__device__ __forceinline__ void load_row_share(const float* __restrict__ row,
                                               const float* __restrict__ cos,
                                               const float* __restrict__ sin, int pos, int g,
                                               bool valid, bool rot, f32x4* x) {
  constexpr int NJ = D / 16;
#pragma unroll
  for (int j = 0; j < NJ; ++j) x[j] = valid ? *(const f32x4*)(row + 4 * chunk_of<D>(j, g)) : zero4();
  if (valid && rot) {
#pragma unroll
    for (int j = 0; j < NJ / 2; ++j) {
      const int64_t o = (int64_t)pos * (D / 2) + 4 * chunk_of<D>(j, g);
      rope4(x[j], x[j + NJ / 2], *(const f32x4*)(cos + o), *(const f32x4*)(sin + o));
    }
  }
}

// C[16 x 16] (+)= tile rows r0..r0+15 (A, chunk reads) times the lane's row
// share x (B): the transposed score tile of one 16-row block.
template <int D>
__device__ __forceinline__ void scores2(const float* tile, const f32x4* x, int c16, int g,
                                        f32x4& s0, f32x4& s1) {
  constexpr int NJ = D / 16;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int c = chunk_of<D>(j, g);
    const f32x4 a0 = *(const f32x4*)(tile + tix<D>(c16, c));
    const f32x4 a1 = *(const f32x4*)(tile + tix<D>(16 + c16, c));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      s0 = mma(a0[e], x[j][e], s0);
      s1 = mma(a1[e], x[j][e], s1);
    }
  }
}

// acc[db] = alpha acc[db] + tile^T p: the [D x 16] product of a tile's
// columns with a 32 x 16 score tile held as p0 (rows 0-15) and p1 (rows
// 16-31), in the C tile's contraction order.  Each 16-column block's 8
// products go into a fresh accumulator that is added once, so a running sum
// is rounded once per tile rather than once per MFMA (its float32 error over
// thousands of positions stays at the reference's own order); two blocks
// interleave so that consecutive MFMAs are independent.
template <int D>
__device__ __forceinline__ void accum_t(const float* tile, const f32x4& p0, const f32x4& p1,
                                        int c16, int g, f32x4* acc, float alpha = 1.f) {
  constexpr int NB = D / 16;
#pragma unroll
  for (int db = 0; db < NB; db += 2) {
    f32x4 f0 = zero4(), f1 = zero4();
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const int row = 16 * (kk >> 2) + 4 * g + (kk & 3);
      const float b = kk < 4 ? p0[kk & 3] : p1[kk & 3];
      f0 = mma(tel<D>(tile, row, 16 * db + c16), b, f0);
      f1 = mma(tel<D>(tile, row, 16 * (db + 1) + c16), b, f1);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      acc[db][r] = __builtin_fmaf(acc[db][r], alpha, f0[r]);
      acc[db + 1][r] = __builtin_fmaf(acc[db + 1][r], alpha, f1[r]);
    }
  }
}

// accum_t of two products at once, ta^T pa into a and tb^T pb into b (the
// dK/dV kernel's dV and dK), their chains interleaved.
template <int D>
__device__ __forceinline__ void accum_t2(const float* ta, const f32x4& pa0, const f32x4& pa1,
                                         f32x4* a, const float* tb, const f32x4& pb0,
                                         const f32x4& pb1, f32x4* b, int c16, int g) {
  constexpr int NB = D / 16;
#pragma unroll
  for (int db = 0; db < NB; ++db) {
    f32x4 fa = zero4(), fb = zero4();
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const int row = 16 * (kk >> 2) + 4 * g + (kk & 3);
      fa = mma(tel<D>(ta, row, 16 * db + c16), kk < 4 ? pa0[kk & 3] : pa1[kk & 3], fa);
      fb = mma(tel<D>(tb, row, 16 * db + c16), kk < 4 ? pb0[kk & 3] : pb1[kk & 3], fb);
    }
    a[db] += fa;
    b[db] += fb;
    __builtin_amdgcn_sched_barrier(0);  // the next block's reads stay behind this block's products
  }
}

// ------------------------------------------------------------------ prepass
// dst[(b H + h) Sp + s][D] = src[b, s, h, :] after RoPE at table row s (rot)
// or as is; rows s in [S, Sp) zero.  One thread per chunk pair.
template <int D>
__global__ __launch_bounds__(256) void rows_f32_kernel(const float* __restrict__ src, int64_t sb,
                                                       int64_t ss, int64_t sh,
                                                       const float* __restrict__ cos,
                                                       const float* __restrict__ sin,
                                                       float* __restrict__ dst, int S, int Sp,
                                                       int H, int rot, int64_t pairs) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p >= pairs) return;
  const int c = (int)(p % (D / 8));
  const int64_t rowi = p / (D / 8);
  const int s = (int)(rowi % Sp);
  const int64_t bh = rowi / Sp;
  const int h = (int)(bh % H);
  const int64_t b = bh / H;
  f32x4 x1 = zero4(), x2 = zero4();
  if (s < S) {
    const float* row = src + b * sb + (int64_t)s * ss + (int64_t)h * sh;
    x1 = *(const f32x4*)(row + 4 * c);
    x2 = *(const f32x4*)(row + D / 2 + 4 * c);
    if (rot) {
      const int64_t o = (int64_t)s * (D / 2) + 4 * c;
      rope4(x1, x2, *(const f32x4*)(cos + o), *(const f32x4*)(sin + o));
    }
  }
  *(f32x4*)(dst + rowi * D + 4 * c) = x1;
  *(f32x4*)(dst + rowi * D + D / 2 + 4 * c) = x2;
}

// Per query row (b, h, i), i < Sp: -lse log2(e) and Delta = sum_d dO O, in
// 64-float groups per 32 positions ([B Hq][Sp/32][nl x 32, Delta x 32]);
// rows past S get -inf and 0 (probability zero).  16 lanes per row.
template <int D>
__global__ __launch_bounds__(256) void stats_f32_kernel(const float* __restrict__ o,
                                                        const float* __restrict__ dout,
                                                        const float* __restrict__ lse,
                                                        float* __restrict__ stats, int S, int Sp,
                                                        int Hq, int64_t rows) {
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);  // (b Hq + h) Sp + i
  const int l = threadIdx.x & 15;
  const int i = (int)(row % Sp);
  const int64_t bh = row / Sp;
  const bool valid = row < rows && i < S;
  float s = 0.f;
  if (valid) {
    const int64_t off = ((bh / Hq * S + i) * Hq + bh % Hq) * D;
#pragma unroll
    for (int c = l; c < D / 4; c += 16) {
      const f32x4 a = *(const f32x4*)(o + off + 4 * c);
      const f32x4 b = *(const f32x4*)(dout + off + 4 * c);
      s += a[0] * b[0] + a[1] * b[1] + a[2] * b[2] + a[3] * b[3];
    }
  }
#pragma unroll
  for (int x = 8; x >= 1; x >>= 1) s += __shfl_xor(s, x, 16);
  if (row < rows && l == 0) {
    float* grp = stats + (bh * (Sp / F_BN) + i / F_BN) * (2 * F_BN) + i % F_BN;
    grp[0] = valid ? -lse[bh * S + i] * kLog2e : -INFINITY;
    grp[F_BN] = valid ? s : 0.f;
  }
}

// ------------------------------------------------------------------ masks
// Explicit masks, one kind at a time, on causal self-attention (Sq == Sk):
// MASK_DOC, a query sees only keys of its own document, and the walks skip
// the 32-position tiles whose [min, max] document id misses the workgroup's
// (exact for any id pattern); MASK_KPM, a query sees only valid keys, and the
// rows before the batch row's first valid key, which would see none, attend
// every key instead (the reference's NaN guard, mask | ~mask.any(-1)).
using mfma::MASK_DOC;
using mfma::MASK_KPM;
using mfma::MASK_NONE;
constexpr int F_MAX_TILES = 4096;  // 32-position tiles of a batch row (S <= 131072)

// Per batch row: MASK_DOC the [min, max] id of each 32-position tile;
// MASK_KPM the first valid key (INT_MAX when none; -1 when every key is valid,
// which the kernels then treat as plain causal attention).  One workgroup per
// row.
__global__ __launch_bounds__(256) void mask_prep_f32_kernel(const int32_t* __restrict__ mask,
                                                            int mode, int S, int nt,
                                                            int2* __restrict__ ranges,
                                                            int* __restrict__ first_valid) {
  __shared__ int sf;
  const int32_t* mrow = mask + (int64_t)blockIdx.x * S;
  if (mode == MASK_DOC) {
    for (int t = threadIdx.x; t < nt; t += 256) {
      int lo = INT_MAX, hi = INT_MIN;
      for (int j = t * F_BN; j < min(S, t * F_BN + F_BN); ++j) {
        lo = min(lo, mrow[j]);
        hi = max(hi, mrow[j]);
      }
      ranges[(int64_t)blockIdx.x * nt + t] = make_int2(lo, hi);
    }
  } else {
    __shared__ int sn;
    if (threadIdx.x == 0) {
      sf = INT_MAX;
      sn = 0;
    }
    __syncthreads();
    int f = INT_MAX, n = 0;
    for (int j = threadIdx.x; j < S; j += 256)
      if (mrow[j] != 0) {
        f = min(f, j);
        ++n;
      }
    atomicMin(&sf, f);
    atomicAdd(&sn, n);
    __syncthreads();
    if (threadIdx.x == 0) first_valid[blockIdx.x] = sn == S ? -1 : sf;
  }
}

// [min, max] document id of positions [p_begin, p_end), at most 64 of them;
// wavefront-uniform.
__device__ __forceinline__ int2 doc_range64(const int32_t* __restrict__ mrow, int p_begin,
                                            int p_end, int lane) {
  const int p = p_begin + lane;
  const int d = p < p_end ? mrow[p] : 0;
  const int lo = mfma::wave_min_i(p < p_end ? d : INT_MAX);
  const int hi = mfma::wave_max_i(p < p_end ? d : INT_MIN);
  return make_int2(__builtin_amdgcn_readfirstlane(lo), __builtin_amdgcn_readfirstlane(hi));
}

// Lists, ascending, the tiles t in [t_begin, t_end) whose document range meets
// [lo, hi]; returns the count.  One wavefront; the caller publishes the count
// and synchronises before the list is read.
__device__ __forceinline__ int list_doc_tiles(const int2* __restrict__ rng, int t_begin, int t_end,
                                              int lo, int hi, uint16_t* list, int lane) {
  int n = 0;
  for (int base = t_begin; base < t_end; base += 64) {
    const int t = base + lane;
    bool vis = false;
    if (t < t_end) {
      const int2 r = rng[t];
      vis = r.x <= hi && r.y >= lo;
    }
    const uint64_t m = __builtin_amdgcn_ballot_w64(vis);
    const int below = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
    if (vis) list[n + below] = (uint16_t)t;
    n += __builtin_popcountll(m);
  }
  return n;
}

// The key tiles a query-row workgroup (forward, dQ) walks: the causal range up
// to its last row (every key when one of its rows is a guarded one), under
// MASK_DOC only the listed tiles.  Returns the count; tiles: tile_at.
template <int MODE>
struct KeyWalk {
  const int32_t* mrow;  // the batch row's mask (doc ids or key validity)
  int n, fv, di;        // tiles; first valid key (MASK_KPM); this lane's row's document
  bool guarded;         // this lane's row attends every key (MASK_KPM)
  bool plain;           // MASK_KPM with every key valid: plain causal attention
};
template <int MODE>
__device__ __forceinline__ KeyWalk<MODE> key_walk(const RowInfo& ri, int kend_causal, int S,
                                                  int bm_pos, const int32_t* mask,
                                                  const int2* ranges, const int* first_valid,
                                                  int nt32, uint16_t* list, int* count, int w,
                                                  int lane) {
  KeyWalk<MODE> k{nullptr, (kend_causal + F_BN - 1) / F_BN, 0, 0, false, MODE == MASK_NONE};
  if (MODE == MASK_NONE) return k;
  k.mrow = mask + (int64_t)ri.b * S;
  if (MODE == MASK_KPM) {
    const int fv = first_valid[ri.b];
    k.plain = fv < 0;
    k.fv = max(fv, 0);
    k.guarded = ri.pos < k.fv;
    if (ri.p0 < k.fv) k.n = (S + F_BN - 1) / F_BN;
  } else {
    k.di = ri.q_valid ? k.mrow[ri.pos] : 0;
    const int2 dr = doc_range64(k.mrow, ri.p0, min(ri.p0 + bm_pos, S), lane);
    if (w == 0) {
      const int n = list_doc_tiles(ranges + (int64_t)ri.b * nt32, 0, k.n, dr.x, dr.y, list, lane);
      if (lane == 0) *count = n;
    }
    __syncthreads();
    k.n = __builtin_amdgcn_readfirstlane(*count);
  }
  return k;
}

// Whether this lane's row (query position pos, causal limit lim = pos - k0)
// sees key k0 + j.
template <int MODE>
__device__ __forceinline__ bool row_sees(const KeyWalk<MODE>& k, int k0, int j, int lim, int S) {
  const int key = k0 + j;
  if (MODE == MASK_DOC) return j <= lim && k.mrow[min(key, S - 1)] == k.di;
  return k.guarded ? key < S : j <= lim && k.mrow[min(key, S - 1)] != 0;
}

// ------------------------------------------------------------------ forward
// Workgroup: 4 wavefronts x 16 (head, position) rows of one KV group (the
// rows of all its query heads share each K/V tile); S^T = K·Q^T per 32-key
// tile, online softmax in the lane, O^T += V^T·P^T.  K comes rotated: element
// (b, g, key, d) at kt + b kb_b + g kb_h + key kld + d (the prepass's rows or
// a rotated cache).
template <int D, int MODE>
__global__ __launch_bounds__(256, 2) void fwd_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ cos, const float* __restrict__ sin,
    const float* kt, int64_t kb_b, int64_t kb_h, int kld, const float* v, int64_t vsb,
    int64_t vsh, int vss, float* __restrict__ out, float* __restrict__ lse, int Sq, int Sk,
    int Hq, int Hkv, int n_rep, int bm_pos, int nqb, int causal, float scale_log2,
    const int32_t* __restrict__ mask, const int2* __restrict__ ranges,
    const int* __restrict__ first_valid, int nt32) {
  constexpr int NJ = D / 16, NB = D / 16;
  __shared__ __attribute__((aligned(16))) float sK[2][F_BN * D];
  __shared__ __attribute__((aligned(16))) float sV[2][F_BN * D];
  __shared__ uint16_t sList[MODE == MASK_DOC ? F_MAX_TILES : 1];
  __shared__ int sCount;

  const int lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15, w = wave_id();
  const int logical = xcd_logical_id(blockIdx.x, gridDim.x, nqb);
  const RowInfo ri = row_info(logical, nqb, Hkv, n_rep, bm_pos, Sq, w * 16 + c16);
  const KeyWalk<MODE> kw =
      key_walk<MODE>(ri, causal ? min(Sk, min(ri.p0 + bm_pos, Sq)) : Sk, Sk, bm_pos, mask,
                     ranges, first_valid, nt32, sList, &sCount, w, lane);
  auto tile_at = [&](int i) {
    return MODE == MASK_DOC ? __builtin_amdgcn_readfirstlane((int)sList[i]) : i;
  };
  const float* kb = kt + (int64_t)ri.b * kb_b + (int64_t)ri.g * kb_h;
  const float* vb = v + (int64_t)ri.b * vsb + (int64_t)ri.g * vsh;
  auto stage = [&](int t, int buf) {
    const int k0 = t * F_BN;
    tile_dma<D>(kb + (int64_t)k0 * kld, (uint32_t)kld, sK[buf], w, lane, Sk - k0);
    tile_dma<D>(vb + (int64_t)k0 * vss, (uint32_t)vss, sV[buf], w, lane, Sk - k0);
  };
  if (kw.n > 0) stage(tile_at(0), 0);

  f32x4 qr[NJ];
  load_row_share<D>(q + (((int64_t)ri.b * Sq + ri.pos) * Hq + ri.hq) * D, cos, sin, ri.pos, g,
                    ri.q_valid, true, qr);

  float m = -INFINITY, l = 0.f;
  f32x4 o[NB];
#pragma unroll
  for (int db = 0; db < NB; ++db) o[db] = zero4();
  mfma::lds_copy_wait();
  __syncthreads();

  for (int i = 0; i < kw.n; ++i) {
    const int buf = i & 1, t = tile_at(i);
    if (i + 1 < kw.n) stage(tile_at(i + 1), buf ^ 1);
    const float* tK = sK[buf];
    const float* tV = sV[buf];
    f32x4 s0 = zero4(), s1 = zero4();
    scores2<D>(tK, qr, c16, g, s0, s1);

    const int k0 = t * F_BN;
    if (kw.plain) {
      if ((causal && k0 + F_BN - 1 > ri.p0) || k0 + F_BN > Sk) {
        const int lim = (causal ? min(ri.pos, Sk - 1) : Sk - 1) - k0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          s0[r] = 4 * g + r > lim ? -INFINITY : s0[r];
          s1[r] = 16 + 4 * g + r > lim ? -INFINITY : s1[r];
        }
      }
    } else {
      const int lim = min(ri.pos, Sk - 1) - k0;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s0[r] = row_sees<MODE>(kw, k0, 4 * g + r, lim, Sk) ? s0[r] : -INFINITY;
        s1[r] = row_sees<MODE>(kw, k0, 16 + 4 * g + r, lim, Sk) ? s1[r] : -INFINITY;
      }
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) tmax = fmaxf(tmax, fmaxf(s0[r], s1[r]));
    tmax = quad_max(tmax) * scale_log2;
    const float mnew = fmaxf(m, tmax);
    // with an explicit mask a row may have seen no key yet (max still -inf)
    const float mref = MODE == MASK_NONE || mnew != -INFINITY ? mnew : 0.f;
    const float alpha = fast_exp2(m - mref);
    m = mnew;
    l *= alpha;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s0[r] = fast_exp2(__builtin_fmaf(s0[r], scale_log2, -mref));
      s1[r] = fast_exp2(__builtin_fmaf(s1[r], scale_log2, -mref));
      l += s0[r] + s1[r];
    }
    accum_t<D>(tV, s0, s1, c16, g, o, alpha);
    mfma::lds_copy_wait();
    __syncthreads();
  }

  const float lt = quad_sum(l);
  if (ri.q_valid) {
    const float inv = 1.f / lt;
    float* orow = out + (((int64_t)ri.b * Sq + ri.pos) * Hq + ri.hq) * D;
#pragma unroll
    for (int db = 0; db < NB; ++db) *(f32x4*)(orow + 16 * db + 4 * g) = o[db] * inv;
    if (lse != nullptr && g == 0)
      lse[((int64_t)ri.b * Hq + ri.hq) * Sq + ri.pos] = (m + log2f(lt)) * kLn2;
  }
}

// ------------------------------------------------------------------ capture
// The probabilities P = exp(s - lse) as float32 [B, Hq, Sq, Sk] after the
// forward has written out and lse: the forward's rows and key walk recompute
// S^T = K·Q^T per 32-key tile (K tiles only) and store each lane's row
// segment; every tile the walk skips (right of the causal frontier, or whose
// documents miss the rows') is written as zeros.  The stores are write-back:
// the two 64-byte halves of a row's 128-byte segment come from two store
// instructions, and L2 joins them into whole lines (non-temporal stores ran
// the C5-cap slice about 20% slower).
template <int D, int MODE>
__global__ __launch_bounds__(256, 2) void capture_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ cos, const float* __restrict__ sin,
    const float* kt, int64_t kb_b, int64_t kb_h, int kld, const float* __restrict__ lse,
    float* __restrict__ probs, int Sq, int Sk, int Hq, int Hkv, int n_rep, int bm_pos, int nqb,
    int causal, float scale_log2, const int32_t* __restrict__ mask,
    const int2* __restrict__ ranges, const int* __restrict__ first_valid, int nt32) {
  constexpr int NJ = D / 16;
  __shared__ __attribute__((aligned(16))) float sK[2][F_BN * D];
  __shared__ uint16_t sList[MODE == MASK_DOC ? F_MAX_TILES : 1];
  __shared__ int sCount;

  const int lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15, w = wave_id();
  const int logical = xcd_logical_id(blockIdx.x, gridDim.x, nqb);
  const RowInfo ri = row_info(logical, nqb, Hkv, n_rep, bm_pos, Sq, w * 16 + c16);
  const KeyWalk<MODE> kw =
      key_walk<MODE>(ri, causal ? min(Sk, min(ri.p0 + bm_pos, Sq)) : Sk, Sk, bm_pos, mask,
                     ranges, first_valid, nt32, sList, &sCount, w, lane);
  auto tile_at = [&](int i) {
    return MODE == MASK_DOC ? __builtin_amdgcn_readfirstlane((int)sList[i]) : i;
  };
  const float* kb = kt + (int64_t)ri.b * kb_b + (int64_t)ri.g * kb_h;
  auto stage = [&](int t, int buf) {
    const int k0 = t * F_BN;
    tile_dma<D>(kb + (int64_t)k0 * kld, (uint32_t)kld, sK[buf], w, lane, Sk - k0);
  };
  if (kw.n > 0) stage(tile_at(0), 0);

  f32x4 qr[NJ];
  load_row_share<D>(q + (((int64_t)ri.b * Sq + ri.pos) * Hq + ri.hq) * D, cos, sin, ri.pos, g,
                    ri.q_valid, true, qr);
  const float nl = ri.q_valid ? -lse[((int64_t)ri.b * Hq + ri.hq) * Sq + ri.pos] * kLog2e : 0.f;
  float* prow = probs + (((int64_t)ri.b * Hq + ri.hq) * Sq + ri.pos) * Sk;
  const bool vec = (Sk & 3) == 0 && ((uintptr_t)probs & 15) == 0;  // rows 16-byte aligned
  // four probabilities (or zeros) at keys key0.. of this lane's row
  auto put4 = [&](int key0, const f32x4& x) {
    if (!ri.q_valid) return;
    if (vec && key0 + 3 < Sk) {
      *(f32x4*)(prow + key0) = x;
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (key0 + r < Sk) prow[key0 + r] = x[r];
    }
  };
  mfma::lds_copy_wait();
  __syncthreads();

  for (int i = 0; i < kw.n; ++i) {
    const int buf = i & 1, t = tile_at(i);
    if (i + 1 < kw.n) stage(tile_at(i + 1), buf ^ 1);
    f32x4 s0 = zero4(), s1 = zero4();
    scores2<D>(sK[buf], qr, c16, g, s0, s1);
    const int k0 = t * F_BN;
    const int lim = (causal ? min(ri.pos, Sk - 1) : Sk - 1) - k0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      bool v0, v1;
      if (kw.plain) {
        v0 = 4 * g + r <= lim;
        v1 = 16 + 4 * g + r <= lim;
      } else {
        v0 = row_sees<MODE>(kw, k0, 4 * g + r, lim, Sk);
        v1 = row_sees<MODE>(kw, k0, 16 + 4 * g + r, lim, Sk);
      }
      s0[r] = v0 ? fast_exp2(__builtin_fmaf(s0[r], scale_log2, nl)) : 0.f;
      s1[r] = v1 ? fast_exp2(__builtin_fmaf(s1[r], scale_log2, nl)) : 0.f;
    }
    put4(k0 + 4 * g, s0);
    put4(k0 + 16 + 4 * g, s1);
    mfma::lds_copy_wait();
    __syncthreads();
  }
  // zeros in the tiles the walk left out (the list is ascending)
  const int ntot = (Sk + F_BN - 1) / F_BN;
  int li = 0;
  for (int t = 0; t < ntot; ++t) {
    if (MODE == MASK_DOC) {
      if (li < kw.n && tile_at(li) == t) {
        ++li;
        continue;
      }
    } else if (t < kw.n) {
      continue;
    }
    put4(t * F_BN + 8 * g, zero4());
    put4(t * F_BN + 8 * g + 4, zero4());
  }
}

// ---- dS records (float32 backward without an explicit mask) --------------
// The dK/dV pass stores each tile's dS as a record block [32 positions][64
// keys] per (query head, 32-position tile t, 64-key block kb); the dQ pass
// multiplies them by K instead of recomputing S and dP.  Causal: the blocks
// kb <= t / 2 only, numbered tile by tile (rec_off); full attention: nkb
// blocks per tile.
__host__ __device__ __forceinline__ int nkb_of(int S) { return (S + F_BK - 1) / F_BK; }
__host__ __device__ __forceinline__ int64_t rec_off(int t, int kb, int causal, int nkb) {
  if (!causal) return (int64_t)t * nkb + kb;
  const int64_t h = t / 2;
  return ((t & 1) ? (h + 1) * (h + 1) : h * (h + 1)) + kb;  // sum over t' < t of t'/2 + 1
}
// record blocks per query head
__host__ __device__ __forceinline__ int64_t rec_blocks(int S, int causal) {
  const int nt = (S + F_BN - 1) / F_BN;
  return rec_off(nt, 0, causal, nkb_of(S));
}

// ------------------------------------------------------------------ backward
// Store a lane's share (d = 16 db + 4 g + r) of scale * G^T after the RoPE
// backward at table row pos (the pair of d < D/2 is d + D/2, in block db + NB/2).
template <int D>
__device__ __forceinline__ void store_grad_rope(float* __restrict__ row, const f32x4* acc,
                                                const float* __restrict__ cos,
                                                const float* __restrict__ sin, int pos, int g,
                                                float scale) {
  constexpr int NB = D / 16;
#pragma unroll
  for (int db = 0; db < NB / 2; ++db) {
    const int d = 16 * db + 4 * g;
    const f32x4 c = *(const f32x4*)(cos + (int64_t)pos * (D / 2) + d);
    const f32x4 s = *(const f32x4*)(sin + (int64_t)pos * (D / 2) + d);
    f32x4 lo, hi;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float d1, d2;
      rope_pair_bwd<float>(acc[db][r] * scale, acc[db + NB / 2][r] * scale, c[r], s[r], d1, d2);
      lo[r] = d1;
      hi[r] = d2;
    }
    *(f32x4*)(row + d) = lo;
    *(f32x4*)(row + D / 2 + d) = hi;
  }
}

// dQ: the forward's rows and tiles; per 32-key tile S^T = K·Q^T and
// dP^T = V·dO^T, dS^T = P^T (dP^T - Delta), dQ^T += K^T·dS^T.  qr / kr: the
// prepass's rotated rows, Sp per head.
template <int D, int MODE>
__global__ __launch_bounds__(256, 2) void bwd_dq_f32_kernel(
    const float* __restrict__ qr_rows, const float* kr_rows, const float* v,
    const float* __restrict__ cos, const float* __restrict__ sin, const float* __restrict__ dout,
    const float* __restrict__ stats, float* __restrict__ dq, int S, int Sp, int Hq, int Hkv,
    int n_rep, int bm_pos, int nqb, int causal, float scale, float scale_log2,
    const int32_t* __restrict__ mask, const int2* __restrict__ ranges,
    const int* __restrict__ first_valid, int nt32) {
  constexpr int NJ = D / 16, NB = D / 16;
  __shared__ __attribute__((aligned(16))) float sK[2][F_BN * D];
  __shared__ __attribute__((aligned(16))) float sV[2][F_BN * D];
  __shared__ uint16_t sList[MODE == MASK_DOC ? F_MAX_TILES : 1];
  __shared__ int sCount;

  const int lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15, w = wave_id();
  const int logical = xcd_logical_id(blockIdx.x, gridDim.x, nqb);
  const RowInfo ri = row_info(logical, nqb, Hkv, n_rep, bm_pos, S, w * 16 + c16);
  const KeyWalk<MODE> kw = key_walk<MODE>(ri, causal ? min(S, ri.p0 + bm_pos) : S, S, bm_pos,
                                          mask, ranges, first_valid, nt32, sList, &sCount, w,
                                          lane);
  auto tile_at = [&](int i) {
    return MODE == MASK_DOC ? __builtin_amdgcn_readfirstlane((int)sList[i]) : i;
  };
  const float* kb = kr_rows + ((int64_t)ri.b * Hkv + ri.g) * Sp * D;
  const float* vb = v + ((int64_t)ri.b * S * Hkv + ri.g) * D;
  const int vss = Hkv * D;
  auto stage = [&](int t, int buf) {
    const int k0 = t * F_BN;
    tile_dma<D>(kb + (int64_t)k0 * D, (uint32_t)D, sK[buf], w, lane, S - k0);
    tile_dma<D>(vb + (int64_t)k0 * vss, (uint32_t)vss, sV[buf], w, lane, S - k0);
  };
  if (kw.n > 0) stage(tile_at(0), 0);

  const int64_t hrow = (int64_t)ri.b * Hq + ri.hq;
  const int64_t roff = ((int64_t)ri.b * S + ri.pos) * Hq + ri.hq;
  f32x4 qr[NJ], dr[NJ];
  load_row_share<D>(qr_rows + (hrow * Sp + ri.pos) * D, cos, sin, ri.pos, g, ri.q_valid, false, qr);
  load_row_share<D>(dout + roff * D, cos, sin, ri.pos, g, ri.q_valid, false, dr);
  const float* st = stats + (hrow * (Sp / F_BN) + ri.pos / F_BN) * (2 * F_BN) + ri.pos % F_BN;
  const float nl = ri.q_valid ? st[0] : 0.f;
  const float dl = ri.q_valid ? st[F_BN] : 0.f;

  f32x4 acc[NB];
#pragma unroll
  for (int db = 0; db < NB; ++db) acc[db] = zero4();
  mfma::lds_copy_wait();
  __syncthreads();

  for (int i = 0; i < kw.n; ++i) {
    const int buf = i & 1, t = tile_at(i);
    if (i + 1 < kw.n) stage(tile_at(i + 1), buf ^ 1);
    const float* tK = sK[buf];
    const float* tV = sV[buf];
    f32x4 s0 = zero4(), s1 = zero4(), d0 = zero4(), d1 = zero4();
    scores2<D>(tK, qr, c16, g, s0, s1);
    scores2<D>(tV, dr, c16, g, d0, d1);
    const int k0 = t * F_BN;
    const bool edge = !kw.plain || (causal && k0 + F_BN - 1 > ri.p0) || k0 + F_BN > S;
    const int lim = (causal ? min(ri.pos, S - 1) : S - 1) - k0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float p0 = fast_exp2(__builtin_fmaf(s0[r], scale_log2, nl));
      float p1 = fast_exp2(__builtin_fmaf(s1[r], scale_log2, nl));
      if (edge) {
        if (kw.plain) {
          p0 = 4 * g + r > lim ? 0.f : p0;
          p1 = 16 + 4 * g + r > lim ? 0.f : p1;
        } else {
          p0 = row_sees<MODE>(kw, k0, 4 * g + r, lim, S) ? p0 : 0.f;
          p1 = row_sees<MODE>(kw, k0, 16 + 4 * g + r, lim, S) ? p1 : 0.f;
        }
      }
      s0[r] = p0 * (d0[r] - dl);
      s1[r] = p1 * (d1[r] - dl);
    }
    accum_t<D>(tK, s0, s1, c16, g, acc);
    mfma::lds_copy_wait();
    __syncthreads();
  }
  if (ri.q_valid) store_grad_rope<D>(dq + roff * D, acc, cos, sin, ri.pos, g, scale);
}

// dQ from the dS records: the forward's rows and key tiles, dQ^T += K^T·dS^T
// with each lane's record row segments as the B operand (two 16-byte loads
// per tile); blocks right of a row's causal record range contribute zero.
template <int D>
__global__ __launch_bounds__(256, 2) void bwd_dq_rec_f32_kernel(
    const float* kr_rows, const float* __restrict__ rec, const float* __restrict__ cos,
    const float* __restrict__ sin, float* __restrict__ dq, int S, int Sp, int Hq, int Hkv,
    int n_rep, int bm_pos, int nqb, int causal, float scale, int64_t rec_nt) {
  constexpr int NB = D / 16;
  __shared__ __attribute__((aligned(16))) float sK[2][F_BN * D];

  const int lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15, w = wave_id();
  const int logical = xcd_logical_id(blockIdx.x, gridDim.x, nqb);
  const RowInfo ri = row_info(logical, nqb, Hkv, n_rep, bm_pos, S, w * 16 + c16);
  const int kend = causal ? min(S, ri.p0 + bm_pos) : S;
  const int ntiles = (kend + F_BN - 1) / F_BN;
  const float* kb = kr_rows + ((int64_t)ri.b * Hkv + ri.g) * Sp * D;
  auto stage = [&](int t, int buf) {
    const int k0 = t * F_BN;
    tile_dma<D>(kb + (int64_t)k0 * D, (uint32_t)D, sK[buf], w, lane, S - k0);
  };
  if (ntiles > 0) stage(0, 0);
  const int tq = ri.pos / F_BN;  // this row's query tile
  const float* rrow = rec + (((int64_t)ri.b * Hq + ri.hq) * rec_nt + rec_off(tq, 0, causal, nkb_of(S))) *
                                (F_BN * F_BK) + (ri.pos % F_BN) * F_BK;
  f32x4 acc[NB];
#pragma unroll
  for (int db = 0; db < NB; ++db) acc[db] = zero4();
  mfma::lds_copy_wait();
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < ntiles) stage(t + 1, buf ^ 1);
    const int kbk = t / 2;
    f32x4 r0 = zero4(), r1 = zero4();
    if (ri.q_valid && (!causal || kbk <= tq / 2)) {
      const float* p = rrow + (int64_t)kbk * (F_BN * F_BK) + F_BN * (t & 1) + 4 * g;
      r0 = __builtin_nontemporal_load((const f32x4*)p);
      r1 = __builtin_nontemporal_load((const f32x4*)(p + 16));
    }
    accum_t<D>(sK[buf], r0, r1, c16, g, acc);
    mfma::lds_copy_wait();
    __syncthreads();
  }
  if (ri.q_valid)
    store_grad_rope<D>(dq + (((int64_t)ri.b * S + ri.pos) * Hq + ri.hq) * D, acc, cos, sin,
                       ri.pos, g, scale);
}

// dK/dV: a workgroup owns 64 keys of one KV head (16 per wavefront, one per
// lane column), their rotated K and V rows in registers, and walks every
// query head of the group over the query tiles from the keys' diagonal on
// (under MASK_DOC only the listed ones; under MASK_KPM also the guarded rows'
// tiles below it): S = Q·K^T and dP = dO·V^T per 32-position tile, then
// dV^T += dO^T·P and dK^T += Q^T·dS.  Key blocks are numbered longest first.
template <int D, int MODE, bool REC = false>
__global__ __launch_bounds__(256, 2) void bwd_dkdv_f32_kernel(
    const float* qr_rows, const float* __restrict__ kr_rows, const float* __restrict__ v,
    const float* __restrict__ cos, const float* __restrict__ sin, const float* dout,
    const float* stats, double* __restrict__ sum64, float* __restrict__ dk,
    float* __restrict__ dv, int S, int Sp, int Hq, int Hkv, int n_rep, int causal, float scale,
    float scale_log2, const int32_t* __restrict__ mask, const int2* __restrict__ ranges,
    const int* __restrict__ first_valid, int nt32, float* __restrict__ rec, int64_t rec_nt) {
  constexpr int NJ = D / 16, NB = D / 16;
  __shared__ __attribute__((aligned(16))) float sQ[2][F_BN * D];
  __shared__ __attribute__((aligned(16))) float sO[2][F_BN * D];
  __shared__ __attribute__((aligned(16))) float sS[2][2 * F_BN];  // -lse log2(e), Delta
  __shared__ uint16_t sList[MODE == MASK_DOC ? F_MAX_TILES : 1];
  __shared__ __attribute__((aligned(16))) int32_t sDoc[MODE == MASK_DOC ? 2 : 1][64];
  __shared__ int sCount;

  const int lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15, w = wave_id();
  const int BH = gridDim.x / ((S + F_BK - 1) / F_BK);
  const int kblk = blockIdx.x / BH, bh = blockIdx.x % BH;
  const int b = bh / Hkv, hk = bh % Hkv;
  const int k0 = kblk * F_BK;
  const int key = k0 + 16 * w + c16;
  const bool kvalid = key < S;

  const int nt = (S + F_BN - 1) / F_BN, t0 = causal ? k0 / F_BN : 0;
  // the query tiles walked per head: tile_of(0 .. per-1)
  const int32_t* mrow = MODE != MASK_NONE ? mask + (int64_t)b * S : nullptr;
  int per = nt - t0, ng = 0, kdoc = 0;
  // MASK_KPM: query rows below fvk (the guarded ones, for a key inside the
  // sequence) see this key, and so do rows from kkey on (INT_MAX: padding key)
  int fvk = 0, kkey = INT_MAX;
  if (MODE == MASK_KPM) {
    const int fv = max(first_valid[b], 0);  // (-1: every key valid)
    ng = fv >= S ? t0 : min((fv + F_BN - 1) / F_BN, t0);  // guarded rows' tiles below t0
    per += ng;
    fvk = kvalid ? fv : 0;
    kkey = kvalid && mrow[key] != 0 ? key : INT_MAX;
  } else if (MODE == MASK_DOC) {
    kdoc = kvalid ? mrow[key] : 0;
    const int2 dr = doc_range64(mrow, k0, min(k0 + F_BK, S), lane);
    if (w == 0) {
      const int n = list_doc_tiles(ranges + (int64_t)b * nt32, t0, nt, dr.x, dr.y, sList, lane);
      if (lane == 0) sCount = n;
    }
    __syncthreads();
    per = __builtin_amdgcn_readfirstlane(sCount);
  }
  auto tile_of = [&](int u) {
    return MODE == MASK_DOC ? __builtin_amdgcn_readfirstlane((int)sList[u])
                            : MODE == MASK_KPM && u < ng ? u : t0 + u - ng;
  };
  const int total = per * n_rep;
  const int oss = Hq * D;
  auto stage = [&](int it, int buf) {
    const int hq = hk * n_rep + it / per, q0 = tile_of(it % per) * F_BN;
    const int64_t hrow = (int64_t)b * Hq + hq;
    tile_dma<D>(qr_rows + (hrow * Sp + q0) * D, (uint32_t)D, sQ[buf], w, lane, F_BN);
    tile_dma<D>(dout + (((int64_t)b * S + q0) * Hq + hq) * D, (uint32_t)oss, sO[buf], w, lane,
                S - q0);
    if (w == 0) mfma::row_to_lds(stats + (hrow * (Sp / F_BN) + q0 / F_BN) * (2 * F_BN), sS[buf], lane);
    if (MODE == MASK_DOC && w == 1)  // the tile's document ids (positions past S repeat S - 1)
      mfma::dma4(mfma::lds_addr(sDoc[buf]), 4u * (uint32_t)min(lane, S - 1 - q0), mrow + q0);
  };
  if (total > 0) stage(0, 0);

  const int64_t koff = ((int64_t)b * S + key) * Hkv + hk;
  f32x4 kr[NJ], vr[NJ];
  load_row_share<D>(kr_rows + (((int64_t)b * Hkv + hk) * Sp + key) * D, cos, sin, key, g, kvalid,
                    false, kr);
  load_row_share<D>(v + koff * D, cos, sin, key, g, kvalid, false, vr);

  f32x4 adk[NB], adv[NB];
#pragma unroll
  for (int db = 0; db < NB; ++db) adk[db] = adv[db] = zero4();
  mfma::lds_copy_wait();
  __syncthreads();

  for (int it = 0; it < total; ++it) {
    const int buf = it & 1;
    if (it + 1 < total) stage(it + 1, buf ^ 1);
    const float* tQ = sQ[buf];
    const float* tO = sO[buf];
    // MASK_DOC: bit r (4 + r) set when query offset 4g + r (16 + 4g + r) is in
    // this key's document (formed before the products, whose registers it
    // would otherwise share)
    int same = 0;
    if (MODE == MASK_DOC) {
      const mfma::i32x4 dq0 = *(const mfma::i32x4*)(sDoc[buf] + 4 * g);
      const mfma::i32x4 dq1 = *(const mfma::i32x4*)(sDoc[buf] + 16 + 4 * g);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        same |= (dq0[r] == kdoc ? 1 : 0) << r | (dq1[r] == kdoc ? 16 : 0) << r;
      asm volatile("" : "+v"(same));
    }
    f32x4 s0 = zero4(), s1 = zero4(), d0 = zero4(), d1 = zero4();
    scores2<D>(tQ, kr, c16, g, s0, s1);
    scores2<D>(tO, vr, c16, g, d0, d1);
    const int q0 = tile_of(it % per) * F_BN;
    const bool edge = MODE != MASK_NONE || (causal && q0 < k0 + F_BK - 1);
    const int lim = key - q0;  // position offsets below lim are masked (causal)
    const int klim = kkey - q0;  // MASK_KPM: offsets from klim on see this (valid) key
    {
      const f32x4 nl0 = *(const f32x4*)(sS[buf] + 4 * g);
      const f32x4 nl1 = *(const f32x4*)(sS[buf] + 16 + 4 * g);

#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p0 = fast_exp2(__builtin_fmaf(s0[r], scale_log2, nl0[r]));
        const float p1 = fast_exp2(__builtin_fmaf(s1[r], scale_log2, nl1[r]));
        bool v0 = true, v1 = true;
        if (edge) {
          const int o0 = 4 * g + r, o1 = 16 + 4 * g + r;
          if (MODE == MASK_NONE) {
            v0 = o0 >= lim;
            v1 = o1 >= lim;
          } else if (MODE == MASK_DOC) {
            v0 = o0 >= lim && ((same >> r) & 1);
            v1 = o1 >= lim && ((same >> (4 + r)) & 1);
          } else {  // guarded rows (below fvk) see every key, the others valid keys up to theirs
            v0 = q0 + o0 < fvk || o0 >= klim;
            v1 = q0 + o1 < fvk || o1 >= klim;
          }
        }
        s0[r] = v0 ? p0 : 0.f;
        s1[r] = v1 ? p1 : 0.f;
      }
    }
    {
      const f32x4 dl0 = *(const f32x4*)(sS[buf] + F_BN + 4 * g);
      const f32x4 dl1 = *(const f32x4*)(sS[buf] + F_BN + 16 + 4 * g);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        d0[r] = s0[r] * (d0[r] - dl0[r]);
        d1[r] = s1[r] * (d1[r] - dl1[r]);
      }
    }
    accum_t2<D>(tO, s0, s1, adv, tQ, d0, d1, adk, c16, g);
    if (it % per == per - 1 && it + 1 < total) {
      // a query head done: its sums (unscaled, before the RoPE backward) join
      // the group's in float64, in this lane's own elements of sum64 (per key
      // row, D dK then D dV values), so the group sum adds no float32
      // rounding per head: the float32 error stays that of one head's sum
      const int h = it / per;
      if (kvalid) {
        // (the row offset recomputed from a laundered key: not kept live across the loop)
        int kl = key;
        asm volatile("" : "+v"(kl));
        const int64_t ro = 2 * ((((int64_t)b * S + kl) * Hkv + hk) * D) + 4 * g;
#pragma unroll
        for (int db = 0; db < NB; ++db) {
          f64x4* pk = (f64x4*)(sum64 + ro + 16 * db);
          f64x4* pv = (f64x4*)(sum64 + ro + D + 16 * db);
          const f64x4 ak = to_f64(adk[db]), av = to_f64(adv[db]);
          *pk = h == 0 ? ak : *pk + ak;
          *pv = h == 0 ? av : *pv + av;
          __builtin_amdgcn_sched_barrier(0);  // one block's loads in flight at a time
        }
      }
#pragma unroll
      for (int db = 0; db < NB; ++db) adk[db] = adv[db] = zero4();
    }
    mfma::lds_copy_wait();
    __syncthreads();
    if (REC) {
      // this tile's dS (unscaled; zero for keys past S) into its record block
      // [32 positions][64 keys] for the dQ pass, after the end-of-tile wait
      // (vmcnt counts stores with the staging loads: a store issued inside
      // the tile would hold that wait until it is written)
      const int t = q0 / F_BN, hq = hk * n_rep + it / per;
      float* blk = rec + (((int64_t)b * Hq + hq) * rec_nt + rec_off(t, kblk, causal, nkb_of(S))) *
                             (F_BN * F_BK) + 16 * w + c16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        __builtin_nontemporal_store(kvalid ? d0[r] : 0.f, blk + (4 * g + r) * F_BK);
        __builtin_nontemporal_store(kvalid ? d1[r] : 0.f, blk + (16 + 4 * g + r) * F_BK);
      }
    }
  }
  if (kvalid) {
    int kl = key;
    asm volatile("" : "+v"(kl));
    const int64_t ko = (((int64_t)b * S + kl) * Hkv + hk) * D;
    if (n_rep > 1 && per > 0) {
#pragma unroll
      for (int db = 0; db < NB; ++db) {
        const double* pk = sum64 + 2 * ko + 16 * db + 4 * g;
        adk[db] = to_f32x4(*(const f64x4*)pk + to_f64(adk[db]));
        adv[db] = to_f32x4(*(const f64x4*)(pk + D) + to_f64(adv[db]));
      }
    }
    store_grad_rope<D>(dk + ko, adk, cos, sin, kl, g, scale);
    float* vrow = dv + ko;
#pragma unroll
    for (int db = 0; db < NB; ++db) *(f32x4*)(vrow + 16 * db + 4 * g) = adv[db];
  }
}

// QK-norm of one element: x / rms(row) * w, the row's sum of squares ss
// (RMSNorm in float32, kempnerforge/model/norm.py)
__device__ __forceinline__ float rms_scale_f32(float x, float ss, int D, float eps, float w) {
  const float r = rsqrtf(ss / (float)D + eps);
  return (x * r) * w;
}

// ------------------------------------------------------------------ decode
// One new token per sequence against the KV cache (after kv_append has
// written the rotated new key and value at position lens[b]): split-K over
// the cache rows.  Workgroup = one (sequence, KV head, split) item, the
// group's n_rep <= 16 query heads as the 16 columns of S^T = K·q^T; per step
// 64 keys, 16 per wavefront: the lane's K row chunks straight from HBM (one
// step ahead, in registers) as the A operand, V rows by direct loads into LDS
// (double-buffered) for O^T += V^T·P^T.  The wavefronts' states combine
// through LDS into one partial (unnormalised o, max, sum) per item;
// decode_merge_f32 combines an item's splits.
constexpr int DEC_KEYS = 64;  // keys per step (4 wavefronts x 16)

template <int D, bool QKN>
__global__ __launch_bounds__(256, 2) void decode_f32_kernel(
    const float* __restrict__ q_new, const float* __restrict__ cos, const float* __restrict__ sin,
    int64_t row_offset, int64_t rope_rows, int max_len, const float* kc, const float* vc,
    const int32_t* __restrict__ lens, float* __restrict__ opart, float* __restrict__ mlpart,
    int Hq, int Hkv, int Smax, int n_rep, int nsplit, float scale_log2,
    const float* __restrict__ qnw, float eps) {
  constexpr int NJ = D / 16, NB = D / 16;
  __shared__ __attribute__((aligned(16))) float sV[2][DEC_KEYS * D];
  __shared__ float sM[4][16], sL[4][16];

  const int lane = threadIdx.x & 63, g = lane >> 4, c16 = lane & 15, w = wave_id();
  const int item = blockIdx.x, pair = item / nsplit, split = item % nsplit;
  const int b = pair / Hkv, hk = pair % Hkv;
  const int len = lens[b];
  const int64_t trow = (int64_t)len - row_offset;
  const bool ok = len >= 0 && len < max_len && trow >= 0 && trow < rope_rows;
  const int L = ok ? len + 1 : 0;
  const int per = (L + nsplit - 1) / nsplit;
  const int chunk = (per + DEC_KEYS - 1) / DEC_KEYS * DEC_KEYS;
  const int lo = split * chunk, hi = min(L, lo + chunk);
  float* op = opart + (int64_t)item * n_rep * D;
  float* mp = mlpart + (int64_t)item * n_rep * 2;
  if (lo >= hi) {  // nothing in this split: an empty partial
    if (threadIdx.x < n_rep) {
      mp[2 * threadIdx.x] = -INFINITY;
      mp[2 * threadIdx.x + 1] = 0.f;
    }
    return;
  }
  const int nsteps = (hi - lo + DEC_KEYS - 1) / DEC_KEYS;
  const float* kb = kc + ((int64_t)b * Hkv + hk) * Smax * D;
  const float* vb = vc + ((int64_t)b * Hkv + hk) * Smax * D;
  auto stage_v = [&](int i, int buf) {
    const int k0 = lo + i * DEC_KEYS;
    tile_dma<D, DEC_KEYS>(vb + (int64_t)k0 * D, (uint32_t)D, sV[buf], w, lane, hi - k0);
  };
  // this lane's K row chunks for step i (rows past hi repeat hi - 1)
  auto load_k = [&](int i, f32x4* x) {
    const int key = min(lo + i * DEC_KEYS + 16 * w + c16, hi - 1);
#pragma unroll
    for (int j = 0; j < NJ; ++j) x[j] = *(const f32x4*)(kb + (int64_t)key * D + 4 * chunk_of<D>(j, g));
  };
  stage_v(0, 0);
  f32x4 kx[NJ];
  load_k(0, kx);

  // the query column c16 (head hk n_rep + c16): QK-norm, then RoPE at trow
  f32x4 qx[NJ];
  {
    const bool hv = c16 < n_rep;
    load_row_share<D>(q_new + ((int64_t)b * Hq + hk * n_rep + min(c16, n_rep - 1)) * D, cos, sin,
                      0, g, hv, false, qx);
    if (QKN) {
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) ss += qx[j][e] * qx[j][e];
      ss = quad_sum(ss);
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          qx[j][e] = rms_scale_f32(qx[j][e], ss, D, eps, qnw[4 * chunk_of<D>(j, g) + e]);
    }
    if (hv) {
#pragma unroll
      for (int j = 0; j < NJ / 2; ++j) {
        const int64_t o = trow * (D / 2) + 4 * chunk_of<D>(j, g);
        rope4(qx[j], qx[j + NJ / 2], *(const f32x4*)(cos + o), *(const f32x4*)(sin + o));
      }
    }
  }

  float m = -INFINITY, l = 0.f;
  f32x4 o[NB];
#pragma unroll
  for (int db = 0; db < NB; ++db) o[db] = zero4();
  mfma::lds_copy_wait();
  __syncthreads();

  for (int i = 0; i < nsteps; ++i) {
    const int buf = i & 1;
    f32x4 kn[NJ];
    if (i + 1 < nsteps) {
      stage_v(i + 1, buf ^ 1);
      load_k(i + 1, kn);
    }
    // S^T for this wavefront's 16 keys: C[key 4g + r][head c16]
    f32x4 s = zero4();
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) s = mma(kx[j][e], qx[j][e], s);
    // (the A operand is K[key c16][d]: the lane's own row chunks)
    const int kbase = lo + i * DEC_KEYS + 16 * w;
    float tmax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s[r] = kbase + 4 * g + r < hi ? s[r] : -INFINITY;
      tmax = fmaxf(tmax, s[r]);
    }
    tmax = quad_max(tmax) * scale_log2;
    const float mnew = fmaxf(m, tmax);
    const float mref = mnew == -INFINITY ? 0.f : mnew;  // a wavefront's keys may all lie past hi
    const float alpha = fast_exp2(m - mref);
    m = mnew;
    l *= alpha;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s[r] = fast_exp2(__builtin_fmaf(s[r], scale_log2, -mref));
      l += s[r];
    }
    // O^T += V^T P^T over the 16 keys: MFMA kk contracts key 16w + 4g + kk
    const float* tV = sV[buf];
#pragma unroll
    for (int db = 0; db < NB; ++db) {
      f32x4 f = zero4();
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        f = mma(tel<D>(tV, 16 * w + 4 * g + kk, 16 * db + c16), s[kk], f);
#pragma unroll
      for (int r = 0; r < 4; ++r) o[db][r] = __builtin_fmaf(o[db][r], alpha, f[r]);
    }
    if (i + 1 < nsteps) {
#pragma unroll
      for (int j = 0; j < NJ; ++j) kx[j] = kn[j];
    }
    mfma::lds_copy_wait();
    __syncthreads();
  }

  // combine the 4 wavefronts: O^T slices through the (now free) V buffers
  l = quad_sum(l);
  float* sO = sV[0];  // [4][D][16]
#pragma unroll
  for (int db = 0; db < NB; ++db)
#pragma unroll
    for (int r = 0; r < 4; ++r) sO[(w * D + 16 * db + 4 * g + r) * 16 + c16] = o[db][r];
  if (g == 0) {
    sM[w][c16] = m;
    sL[w][c16] = l;
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < n_rep * D; idx += 256) {
    const int h = idx / D, d = idx % D;
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < 4; ++v) mx = fmaxf(mx, sM[v][h]);
    float acc = 0.f, lt = 0.f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float wgt = sM[v][h] == -INFINITY ? 0.f : fast_exp2(sM[v][h] - mx);
      acc += wgt * sO[(v * D + d) * 16 + h];
      lt += wgt * sL[v][h];
    }
    op[h * D + d] = acc;
    if (d == 0) {
      mp[2 * h] = mx;
      mp[2 * h + 1] = lt;
    }
  }
}

// out[b, hq] = the splits' partials combined (max and sums in log2 units);
// NaN for a sequence whose length fails the checks.  One wavefront per row.
template <int D>
__global__ __launch_bounds__(256) void decode_merge_f32_kernel(
    const float* __restrict__ opart, const float* __restrict__ mlpart,
    const int32_t* __restrict__ lens, float* __restrict__ out, int B, int Hq, int Hkv,
    int nsplit, int max_len, int64_t row_offset, int64_t rope_rows) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= B * Hq) return;
  const int b = row / Hq, hq = row % Hq, n_rep = Hq / Hkv, hk = hq / n_rep, h = hq % n_rep;
  const int len = lens[b];
  const int64_t trow = (int64_t)len - row_offset;
  float* orow = out + (int64_t)row * D;
  if (!(len >= 0 && len < max_len && trow >= 0 && trow < rope_rows)) {
    for (int d = lane; d < D; d += 64) orow[d] = NAN;
    return;
  }
  const int64_t item0 = ((int64_t)b * Hkv + hk) * nsplit;
  float mx = -INFINITY;
  for (int s = 0; s < nsplit; ++s) mx = fmaxf(mx, mlpart[((item0 + s) * n_rep + h) * 2]);
  float acc[D / 64] = {}, lt = 0.f;
  for (int s = 0; s < nsplit; ++s) {
    const float* ml = mlpart + ((item0 + s) * n_rep + h) * 2;
    if (ml[1] == 0.f) continue;
    const float wgt = fast_exp2(ml[0] - mx);
    lt += wgt * ml[1];
    const float* o = opart + ((item0 + s) * n_rep + h) * D;
#pragma unroll
    for (int k = 0; k < D / 64; ++k) acc[k] += wgt * o[64 * k + lane];
  }
  const float inv = 1.f / lt;
#pragma unroll
  for (int k = 0; k < D / 64; ++k) orow[64 * k + lane] = acc[k] * inv;
}

template <int D>
int launch_rows(const float* src, int64_t sb, int64_t ss, int64_t sh, const float* cos,
                const float* sin, float* dst, int B, int S, int Sp, int H, int rot,
                hipStream_t stream) {
  const int64_t pairs = (int64_t)B * H * Sp * (D / 8);
  KF_CHECK_ARG((pairs + 255) / 256 < (1LL << 31), "grid too large");
  KF_LAUNCH("rows_f32", (rows_f32_kernel<D>), dim3((unsigned)((pairs + 255) / 256)), dim3(256),
            0, stream, src, sb, ss, sh, cos, sin, dst, S, Sp, H, rot, pairs);
  KF_CHECK_LAUNCH();
  return KF_OK;
}

size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

int mask_mode_of(const int32_t* doc, const int32_t* kvalid) {
  return doc ? MASK_DOC : kvalid ? MASK_KPM : MASK_NONE;
}

// the mask records (mask_prep_f32) at the end of a workspace of `base` bytes
struct MaskRec {
  int2* ranges;
  int* first_valid;
  int nt32;
};
MaskRec mask_rec(void* workspace, size_t base, int B, int S) {
  MaskRec m;
  m.nt32 = (S + F_BN - 1) / F_BN;
  m.ranges = (int2*)((char*)workspace + al256(base));
  m.first_valid = (int*)(m.ranges + (size_t)B * m.nt32);
  return m;
}
size_t mask_rec_bytes(int B, int S) {
  return (size_t)B * ((S + F_BN - 1) / F_BN) * sizeof(int2) + (size_t)B * sizeof(int);
}
int launch_mask_prep(const int32_t* mask, int mode, int B, int S, const MaskRec& m,
                     hipStream_t stream) {
  KF_LAUNCH("mask_prep_f32", mask_prep_f32_kernel, dim3(B), dim3(256), 0, stream, mask, mode, S,
            m.nt32, m.ranges, m.first_valid);
  KF_CHECK_LAUNCH();
  return KF_OK;
}

size_t fwd_krot_bytes(int B, int Sk, int Hkv, int D) {
  return (size_t)B * Hkv * ((Sk + F_BK - 1) / F_BK * F_BK) * D * sizeof(float);
}

template <int D, int MODE>
void launch_fwd_f32(const FwdArgs& a, const float* kt, int64_t kb_b, int64_t kb_h, int kld,
                    int n_rep, int bm_pos, int nqb, unsigned nblk, const MaskRec& mr) {
  KF_LAUNCH("fwd_f32", (fwd_f32_kernel<D, MODE>), dim3(nblk), dim3(256), 0, a.stream,
            (const float*)a.q, a.cos, a.sin, kt, kb_b, kb_h, kld, (const float*)a.v, a.vsb, a.vsh,
            (int)a.vss, (float*)a.out, a.lse, a.Sq, a.Sk, a.Hq, a.Hkv, n_rep, bm_pos, nqb,
            a.causal, a.scale * kLog2e, a.doc ? a.doc : a.kvalid, mr.ranges, mr.first_valid,
            mr.nt32);
}

template <int D>
int fwd_f32_t(const FwdArgs& a, void* workspace) {
  const int n_rep = a.Hq / a.Hkv, bm_pos = F_ROWS / n_rep;
  const int nqb = (a.Sq + bm_pos - 1) / bm_pos;
  const int64_t nblk = (int64_t)nqb * a.B * a.Hkv;
  KF_CHECK_ARG(nblk < (1LL << 31), "grid too large");
  const float* kt = (const float*)a.k;
  int64_t kb_b = a.ksb, kb_h = a.ksh, kld = a.kss;
  if (!a.k_rotated) {
    const int Skp = (a.Sk + F_BK - 1) / F_BK * F_BK;
    float* krot = (float*)workspace;
    const int rc = launch_rows<D>((const float*)a.k, a.ksb, a.kss, a.ksh, a.cos, a.sin, krot, a.B,
                                  a.Sk, Skp, a.Hkv, 1, a.stream);
    if (rc) return rc;
    kt = krot;
    kb_h = (int64_t)Skp * D;
    kb_b = a.Hkv * kb_h;
    kld = D;
  }
  const int mode = mask_mode_of(a.doc, a.kvalid);
  MaskRec mr{nullptr, nullptr, 0};
  if (mode != MASK_NONE) {
    mr = mask_rec(workspace, fwd_krot_bytes(a.B, a.Sk, a.Hkv, D), a.B, a.Sk);
    const int rc = launch_mask_prep(a.doc ? a.doc : a.kvalid, mode, a.B, a.Sk, mr, a.stream);
    if (rc) return rc;
  }
  if (mode == MASK_DOC)
    launch_fwd_f32<D, MASK_DOC>(a, kt, kb_b, kb_h, (int)kld, n_rep, bm_pos, nqb, (unsigned)nblk, mr);
  else if (mode == MASK_KPM)
    launch_fwd_f32<D, MASK_KPM>(a, kt, kb_b, kb_h, (int)kld, n_rep, bm_pos, nqb, (unsigned)nblk, mr);
  else
    launch_fwd_f32<D, MASK_NONE>(a, kt, kb_b, kb_h, (int)kld, n_rep, bm_pos, nqb, (unsigned)nblk,
                                 mr);
  KF_CHECK_LAUNCH();
  return KF_OK;
}

// backward workspace: rotated Q, rotated K, row statistics, then (n_rep > 1)
// the float64 group sums, then the mask records
size_t bwd_base_bytes(int B, int S, int Hq, int Hkv, int D, size_t* sum_off) {
  const size_t Sp = (size_t)(S + F_BK - 1) / F_BK * F_BK;
  const size_t f = ((size_t)B * Hq * Sp * D + (size_t)B * Hkv * Sp * D + (size_t)B * Hq * Sp * 2) *
                   sizeof(float);
  *sum_off = al256(f);
  return *sum_off + (Hq > Hkv ? (size_t)B * S * Hkv * D * 2 * sizeof(double) : 0);
}

template <int D, int MODE>
void launch_bwd_kernels(const BwdArgs& a, float* qrot, float* krot, float* stats, double* sum64,
                        int Sp, int n_rep, int bm_pos, int nqb, unsigned nqblk, unsigned nkblk,
                        const MaskRec& mr, float* rec) {
  const int32_t* mask = a.doc ? a.doc : a.kvalid;
  if constexpr (MODE == MASK_NONE) {
   if (rec != nullptr) {
    // dK/dV first, keeping dS; then dQ from the records
    const int64_t rnt = rec_blocks(a.S, a.causal);
    KF_LAUNCH("bwd_dkdv_f32", (bwd_dkdv_f32_kernel<D, MODE, true>), dim3(nkblk), dim3(256), 0,
              a.stream, qrot, krot, (const float*)a.v, a.cos, a.sin, (const float*)a.dout,
              stats, sum64, (float*)a.dk, (float*)a.dv, a.S, Sp, a.Hq, a.Hkv, n_rep, a.causal,
              a.scale, a.scale * kLog2e, mask, mr.ranges, mr.first_valid, mr.nt32, rec, rnt);
    KF_LAUNCH("bwd_dq_rec_f32", (bwd_dq_rec_f32_kernel<D>), dim3(nqblk), dim3(256), 0, a.stream,
              krot, rec, a.cos, a.sin, (float*)a.dq, a.S, Sp, a.Hq, a.Hkv, n_rep, bm_pos, nqb,
              a.causal, a.scale, rnt);
    return;
   }
  }
  KF_LAUNCH("bwd_dq_f32", (bwd_dq_f32_kernel<D, MODE>), dim3(nqblk), dim3(256), 0, a.stream,
            qrot, krot, (const float*)a.v, a.cos, a.sin, (const float*)a.dout, stats,
            (float*)a.dq, a.S, Sp, a.Hq, a.Hkv, n_rep, bm_pos, nqb, a.causal, a.scale,
            a.scale * kLog2e, mask, mr.ranges, mr.first_valid, mr.nt32);
  KF_LAUNCH("bwd_dkdv_f32", (bwd_dkdv_f32_kernel<D, MODE>), dim3(nkblk), dim3(256), 0, a.stream,
            qrot, krot, (const float*)a.v, a.cos, a.sin, (const float*)a.dout, stats, sum64,
            (float*)a.dk, (float*)a.dv, a.S, Sp, a.Hq, a.Hkv, n_rep, a.causal, a.scale,
            a.scale * kLog2e, mask, mr.ranges, mr.first_valid, mr.nt32, nullptr, 0);
}

// bytes of the dS records, or 0 past the cap (dQ then recomputes S and dP)
constexpr size_t F_REC_MAX = (size_t)32 << 30;
size_t rec_bytes(int B, int S, int Hq, int causal) {
  const size_t n = (size_t)B * Hq * (size_t)rec_blocks(S, causal) * (F_BN * F_BK) * sizeof(float);
  return n <= F_REC_MAX ? n : 0;
}

template <int D>
int bwd_f32_t(const BwdArgs& a, void* workspace, float* rec) {
  const int n_rep = a.Hq / a.Hkv, bm_pos = F_ROWS / n_rep;
  const int nqb = (a.S + bm_pos - 1) / bm_pos;
  const int Sp = (a.S + F_BK - 1) / F_BK * F_BK;
  const int64_t nqblk = (int64_t)nqb * a.B * a.Hkv;
  const int64_t nkblk = (int64_t)(Sp / F_BK) * a.B * a.Hkv;
  KF_CHECK_ARG(nqblk < (1LL << 31) && nkblk < (1LL << 31), "grid too large");
  size_t sum_off = 0;
  const size_t base = bwd_base_bytes(a.B, a.S, a.Hq, a.Hkv, D, &sum_off);
  float* qrot = (float*)workspace;
  float* krot = qrot + (size_t)a.B * a.Hq * Sp * D;
  float* stats = krot + (size_t)a.B * a.Hkv * Sp * D;
  double* sum64 = (double*)((char*)workspace + sum_off);
  const int64_t qss = (int64_t)a.Hq * D, kss = (int64_t)a.Hkv * D;
  int rc = launch_rows<D>((const float*)a.q, a.S * qss, qss, D, a.cos, a.sin, qrot, a.B, a.S, Sp,
                          a.Hq, 1, a.stream);
  if (rc) return rc;
  rc = launch_rows<D>((const float*)a.k, a.S * kss, kss, D, a.cos, a.sin, krot, a.B, a.S, Sp,
                      a.Hkv, 1, a.stream);
  if (rc) return rc;
  const int64_t rows = (int64_t)a.B * a.Hq * Sp;
  KF_LAUNCH("stats_f32", (stats_f32_kernel<D>), dim3((unsigned)((rows + 15) / 16)), dim3(256), 0,
            a.stream, (const float*)a.out, (const float*)a.dout, a.lse, stats, a.S, Sp, a.Hq,
            rows);
  const int mode = mask_mode_of(a.doc, a.kvalid);
  MaskRec mr{nullptr, nullptr, 0};
  if (mode != MASK_NONE) {
    mr = mask_rec(workspace, base, a.B, a.S);
    rc = launch_mask_prep(a.doc ? a.doc : a.kvalid, mode, a.B, a.S, mr, a.stream);
    if (rc) return rc;
  }
  if (mode == MASK_DOC)
    launch_bwd_kernels<D, MASK_DOC>(a, qrot, krot, stats, sum64, Sp, n_rep, bm_pos, nqb,
                                    (unsigned)nqblk, (unsigned)nkblk, mr, rec);
  else if (mode == MASK_KPM)
    launch_bwd_kernels<D, MASK_KPM>(a, qrot, krot, stats, sum64, Sp, n_rep, bm_pos, nqb,
                                    (unsigned)nqblk, (unsigned)nkblk, mr, rec);
  else
    launch_bwd_kernels<D, MASK_NONE>(a, qrot, krot, stats, sum64, Sp, n_rep, bm_pos, nqb,
                                     (unsigned)nqblk, (unsigned)nkblk, mr, rec);
  KF_CHECK_LAUNCH();
  return KF_OK;
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

bool fwd_f32_supported(const FwdArgs& a) {
  if (a.dtype != F32 || (a.D != 64 && a.D != 128)) return false;
  if (a.rot || (a.doc && a.kvalid)) return false;
  if (a.Sq < 1 || a.Sk < 1 || a.Hkv < 1 || a.Hq % a.Hkv) return false;
  if (a.Hq / a.Hkv > F_ROWS) return false;
  // an explicit mask: causal self-attention (as the C ABI checks), within the tile list
  if ((a.doc || a.kvalid) &&
      (!a.causal || a.Sq != a.Sk || a.k_rotated || (a.Sk + F_BN - 1) / F_BN > F_MAX_TILES))
    return false;
  if (!al16(a.q) || !al16(a.k) || !al16(a.v) || !al16(a.out) || !al16(a.cos) || !al16(a.sin))
    return false;
  if ((a.ksb | a.kss | a.ksh | a.vsb | a.vss | a.vsh) & 3) return false;
  // row strides of the direct tile loads (32-bit offsets)
  if (a.kss > (1 << 24) || a.vss > (1 << 24)) return false;
  return true;
}

size_t fwd_f32_workspace(int B, int Sk, int Hkv, int D) {
  return al256(fwd_krot_bytes(B, Sk, Hkv, D)) + mask_rec_bytes(B, Sk);
}

int fwd_f32(const FwdArgs& a, void* workspace) {
  return a.D == 128 ? fwd_f32_t<128>(a, workspace) : fwd_f32_t<64>(a, workspace);
}

int capture_f32(const FwdArgs& a, float* probs, void* workspace) {
  int rc = fwd_f32(a, workspace);  // out, lse, and the rotated K / mask records it leaves
  if (rc) return rc;
  const int n_rep = a.Hq / a.Hkv, bm_pos = F_ROWS / n_rep;
  const int nqb = (a.Sq + bm_pos - 1) / bm_pos;
  const unsigned nblk = (unsigned)((int64_t)nqb * a.B * a.Hkv);
  const float* kt = (const float*)a.k;
  int64_t kb_b = a.ksb, kb_h = a.ksh, kld = a.kss;
  if (!a.k_rotated) {
    const int Skp = (a.Sk + F_BK - 1) / F_BK * F_BK;
    kt = (const float*)workspace;
    kb_h = (int64_t)Skp * a.D;
    kb_b = a.Hkv * kb_h;
    kld = a.D;
  }
  const int mode = mask_mode_of(a.doc, a.kvalid);
  MaskRec mr{nullptr, nullptr, 0};
  if (mode != MASK_NONE) mr = mask_rec(workspace, fwd_krot_bytes(a.B, a.Sk, a.Hkv, a.D), a.B, a.Sk);
  const int32_t* mask = a.doc ? a.doc : a.kvalid;
#define KF_CAP_F32(DD, M)                                                                        KF_LAUNCH("capture_f32", (capture_f32_kernel<DD, M>), dim3(nblk), dim3(256), 0, a.stream,                (const float*)a.q, a.cos, a.sin, kt, kb_b, kb_h, (int)kld, a.lse, probs, a.Sq,                  a.Sk, a.Hq, a.Hkv, n_rep, bm_pos, nqb, a.causal, a.scale * kLog2e, mask,                       mr.ranges, mr.first_valid, mr.nt32)
  if (a.D == 128) {
    if (mode == MASK_DOC) KF_CAP_F32(128, MASK_DOC);
    else if (mode == MASK_KPM) KF_CAP_F32(128, MASK_KPM);
    else KF_CAP_F32(128, MASK_NONE);
  } else {
    if (mode == MASK_DOC) KF_CAP_F32(64, MASK_DOC);
    else if (mode == MASK_KPM) KF_CAP_F32(64, MASK_KPM);
    else KF_CAP_F32(64, MASK_NONE);
  }
#undef KF_CAP_F32
  KF_CHECK_LAUNCH();
  return KF_OK;
}

bool bwd_f32_supported(const BwdArgs& a) {
  if (a.dtype != F32 || (a.D != 64 && a.D != 128)) return false;
  if (a.rot || (a.doc && a.kvalid)) return false;
  if (a.S < 1 || a.Hkv < 1 || a.Hq % a.Hkv) return false;
  if (a.Hq / a.Hkv > F_ROWS || (int64_t)a.Hq * a.D > (1 << 24)) return false;
  if ((a.doc || a.kvalid) && (!a.causal || (a.S + F_BN - 1) / F_BN > F_MAX_TILES)) return false;
  return al16(a.q) && al16(a.k) && al16(a.v) && al16(a.cos) && al16(a.sin) && al16(a.out) &&
         al16(a.dout) && al16(a.dq) && al16(a.dk) && al16(a.dv);
}

size_t bwd_f32_workspace(int B, int S, int Hq, int Hkv, int D) {
  size_t sum_off = 0;
  return al256(bwd_base_bytes(B, S, Hq, Hkv, D, &sum_off)) + mask_rec_bytes(B, S);
}

size_t bwd_f32_workspace_ds(int B, int S, int Hq, int Hkv, int D, int causal) {
  const size_t rb = rec_bytes(B, S, Hq, causal);
  return rb ? al256(bwd_f32_workspace(B, S, Hq, Hkv, D)) + rb : bwd_f32_workspace(B, S, Hq, Hkv, D);
}

int bwd_f32(const BwdArgs& a, void* workspace, size_t workspace_bytes) {
  // the dS records when there is no explicit mask and the workspace holds them
  float* rec = nullptr;
  if (!a.doc && !a.kvalid && rec_bytes(a.B, a.S, a.Hq, a.causal) != 0 &&
      workspace_bytes >= bwd_f32_workspace_ds(a.B, a.S, a.Hq, a.Hkv, a.D, a.causal))
    rec = (float*)((char*)workspace + al256(bwd_f32_workspace(a.B, a.S, a.Hq, a.Hkv, a.D)));
  return a.D == 128 ? bwd_f32_t<128>(a, workspace, rec) : bwd_f32_t<64>(a, workspace, rec);
}


bool decode_f32_supported(const DecodeArgs& a) {
  if (a.dtype != F32 || (a.D != 64 && a.D != 128) || a.Hkv < 1 || a.Hq % a.Hkv) return false;
  if (a.Hq / a.Hkv > 16) return false;
  return al16(a.q_new) && al16(a.k_cache) && al16(a.v_cache) && al16(a.cos) && al16(a.sin) &&
         al16(a.out);
}

int decode_f32(const DecodeArgs& a, void* workspace, size_t slots) {
  const int n_rep = a.Hq / a.Hkv;
  const int64_t pairs = (int64_t)a.B * a.Hkv;
  const int nsplit = (int)(1 + (int64_t)(slots - pairs) / pairs);  // items fit the slots
  const int64_t items = pairs * nsplit;
  KF_CHECK_ARG(items < (1LL << 31) && (size_t)items <= slots, "decode grid too large");
  float* opart = (float*)workspace;
  float* mlpart = opart + slots * n_rep * a.D;
  const bool qkn = a.q_norm_w != nullptr;
  const float sl = a.scale * kLog2e;
#define KF_DEC_F32(DD, Q)                                                                      \
  KF_LAUNCH("decode_f32", (decode_f32_kernel<DD, Q>), dim3((unsigned)items), dim3(256), 0,    \
            a.stream, (const float*)a.q_new, a.cos, a.sin, a.rope_row_offset, a.rope_rows,     \
            a.max_len, (const float*)a.k_cache, (const float*)a.v_cache, a.lens, opart, mlpart, \
            a.Hq, a.Hkv, a.Smax, n_rep, nsplit, sl, a.q_norm_w, a.norm_eps)
  if (a.D == 128) {
    if (qkn) KF_DEC_F32(128, true);
    else KF_DEC_F32(128, false);
  } else {
    if (qkn) KF_DEC_F32(64, true);
    else KF_DEC_F32(64, false);
  }
#undef KF_DEC_F32
  KF_LAUNCH("decode_merge_f32",
            (a.D == 128 ? decode_merge_f32_kernel<128> : decode_merge_f32_kernel<64>),
            dim3((a.B * a.Hq + 3) / 4), dim3(256), 0, a.stream, opart, mlpart, a.lens,
            (float*)a.out, a.B, a.Hq, a.Hkv, nsplit, a.max_len, a.rope_row_offset, a.rope_rows);
  KF_CHECK_LAUNCH();
  return KF_OK;
}

}  // namespace kf
