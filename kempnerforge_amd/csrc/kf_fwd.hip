// bf16 / fp16 MFMA forward attention for gfx950 (head_dim 64 or 128).
//
// Two kernels:
//  kv_prep   stages one KV head's keys and values in the layout the MFMA loop
//            reads: K rotated by RoPE (eager rounding in the input dtype)
//            [bh][Skp][D], and V either as V^T [bh][D][Skp] in P^T fragment
//            key order (forward) or
//            row-major [bh][Skp][D] (backward); keys >= Sk zeroed.
//            With document ids it also records each 64-key tile's id range,
//            with a key-validity mask its valid-key count and first valid key.
//  fwd_mfma  flash forward.  One workgroup = 4 wavefronts = 128 "rows", where
//            a row is (query head of the KV group, position): every K/V tile in
//            LDS is shared by all n_rep query heads of the group.  Each wave
//            owns 32 rows and computes S^T = K·Q^T with
//            v_mfma_f32_32x32x16_bf16 (_f16), so a lane holds one query's 32 scores of
//            a 64-key tile: the online-softmax max/sum is lane-local plus one
//            exchange with lane^32.  O^T = V^T·P^T accumulates in 16 fp32
//            registers per 32-d tile; its V^T operand is one ds_read_b128 of
//            the staged V^T tile.  RoPE of q happens at the Q load.
//
// MFMA 32x32x16 operand layout used (lane l, h = l/32, slot j = 0..7):
//   A[m][k]: m = l%32, k = 8h + j     B[k][n]: n = l%32, k = 8h + j
//   C[m][n]: n = l%32, register i holds m = 8*(i/4) + 4h + (i%4)
// Only the A/B k-assignment has to agree between the two operands; both
// operands are always built with the same (h, j) -> k map.
#include "kf_common.h"
#include "kf_internal.h"
#include "kf_mfma.h"

#include <type_traits>

namespace kf {

namespace {

using namespace mfma;

// how far (log2 units) a row's max may outgrow the forward's exponent base
// before the running output is rescaled
constexpr float RESCALE_SLACK = 8.f;
// LDS fragment reads in flight ahead of the forward's MFMAs (depth 3: 1% faster than
// the compiler's order; 5 and 8 measured no better)
constexpr int FWD_PF = 3;

template <typename T, int D>
__global__ __launch_bounds__(256) void kv_prep_kernel(
    const T* __restrict__ k, const T* __restrict__ v, const float* __restrict__ cos,
    const float* __restrict__ sin, T* __restrict__ krot, int krows, T* __restrict__ vn,
    int Sk, int Skp, int Hkv, int64_t ksb, int64_t kss, int64_t ksh, int64_t vsb, int64_t vss,
    int64_t vsh, int k_rotated, const int32_t* __restrict__ doc, const int32_t* __restrict__ kvalid,
    int2* __restrict__ ranges, int v_mode, T* __restrict__ qpad, int Hq) {
  constexpr int HALF = D / 2;
  __shared__ __attribute__((aligned(16))) T sVt[D * BN];  // KV_V_TRANSPOSED: [d][key slot]
  constexpr int CP = HALF / 8;
  const int s0 = blockIdx.x * BN;
  const int bh = blockIdx.y;
  const int b = bh / Hkv, g = bh % Hkv;
  const int tid = threadIdx.x;
  // tiles below Skp carry V and the tile records; the ones up to krows only K rows
  const int nvb = Skp / BN;
  const bool vtile = (int)blockIdx.x < nvb;

  if (vtile && doc != nullptr && g == 0 && tid < 64) {
    // document-id range of this tile (empty: min > max, when all keys >= Sk)
    const int s = s0 + tid;
    const int d = s < Sk ? doc[(int64_t)b * Sk + s] : 0;
    const int lo = wave_min_i(s < Sk ? d : INT_MAX), hi = wave_max_i(s < Sk ? d : INT_MIN);
    if (tid == 0) ranges[(int64_t)b * nvb + blockIdx.x] = make_int2(lo, hi);
  } else if (vtile && kvalid != nullptr && g == 0 && tid < 64) {
    // number of valid keys in this tile and the first one's position
    const int s = s0 + tid;
    const bool ok = s < Sk && kvalid[(int64_t)b * Sk + s] != 0;
    const uint64_t m = __builtin_amdgcn_ballot_w64(ok);
    if (tid == 0)
      ranges[(int64_t)b * nvb + blockIdx.x] =
          make_int2(__builtin_popcountll(m), m ? s0 + __builtin_ctzll(m) : INT_MAX);
  }

  for (int it = tid; krot != nullptr && it < BN * CP; it += 256) {
    const int key = it / CP, c = it % CP;
    const int s = s0 + key;
    u32x4 o1 = {0u, 0u, 0u, 0u}, o2 = {0u, 0u, 0u, 0u};
    if (s < Sk) {
      const T* src = k + b * ksb + (int64_t)s * kss + g * ksh;
      const u32x4 a = *(const u32x4*)(src + 8 * c);
      const u32x4 bb = *(const u32x4*)(src + 8 * c + HALF);
      if (k_rotated) {
        o1 = a;
        o2 = bb;
      } else {
        float x1[8], x2[8];
        unpack8<T>(a, x1);
        unpack8<T>(bb, x2);
        rope8<T>(x1, x2, cos + (int64_t)s * HALF + 8 * c, sin + (int64_t)s * HALF + 8 * c, o1,
                   o2);
      }
    }
    T* dst = krot + ((int64_t)bh * krows + s) * D;
    *(u32x4*)(dst + 8 * c) = o1;
    *(u32x4*)(dst + 8 * c + HALF) = o2;
  }
  if (qpad != nullptr && s0 + BN > Sk) {
    // rotated-Q rows past the sequence, for the group's query heads
    const int n_rep = Hq / Hkv;
    for (int it = tid; it < n_rep * BN * (D / 8); it += 256) {
      const int hl = it / (BN * (D / 8)), r = (it / (D / 8)) % BN, c = it % (D / 8);
      const int s = s0 + r;
      if (s >= Sk && s < krows)
        *(u32x4*)(qpad + (((int64_t)b * Hq + g * n_rep + hl) * krows + s) * D + 8 * c) =
            u32x4{0u, 0u, 0u, 0u};
    }
  }
  if (!vtile || v_mode == KV_V_NONE) return;
  if (v_mode == KV_V_ROWS) {
    for (int it = tid; it < BN * (D / 8); it += 256) {
      const int key = it / (D / 8), c = it % (D / 8);
      const int s = s0 + key;
      u32x4 a = {0u, 0u, 0u, 0u};
      if (s < Sk) a = *(const u32x4*)(v + b * vsb + (int64_t)s * vss + g * vsh + 8 * c);
      *(u32x4*)(vn + ((int64_t)bh * Skp + s) * D + 8 * c) = a;
    }
    return;
  }
  // V^T: [bh][D][Skp], keys of each 16-key group stored in the order
  // 0-3, 8-11, 4-7, 12-15 (bits 2 and 3 of the key index swapped).  That is the
  // key order of a P^T fragment built from the 32x32 C layout (lane half h holds
  // keys 4h..4h+3 and 8+4h..8+4h+3 of each 16), so one 16-byte read of a V^T row
  // is a complete A fragment of O^T += V^T P^T.
  //
  // The transpose goes through LDS as [d][key slot] rows of 128 bytes.  A lane
  // takes two adjacent keys (adjacent slots) of one 16-byte d chunk c and
  // writes 8 packed dwords, rows 8c..8c+7; a wavefront covers 16 key pairs x
  // 4 chunks.  Odd chunks walk their rows in pair-swapped order (row 8c + (jj ^
  // 1) at step jj), so each store has both row parities in flight (the two
  // 128-byte halves of a 256-byte bank window), and rows 16..31 of every 32
  // hold their 16-byte slot chunks at index ^ 4: the 64 lanes of a store meet
  // 64 distinct banks.  The 16-byte reads undo the chunk swizzle.
  constexpr int CH = D / 32;  // 4-chunk groups of a key row
  for (int it = tid; it < (BN / 2) * (D / 8); it += 256) {
    const int rest = it >> 6;
    const int c = 4 * (rest % CH) + (it & 3);
    const int kp = 16 * (rest / CH) + ((it >> 2) & 15);
    const int s = s0 + 2 * kp;
    const T* src = v + b * vsb + (int64_t)s * vss + g * vsh + 8 * c;
    u32x4 a = {0u, 0u, 0u, 0u}, a2 = {0u, 0u, 0u, 0u};
    if (s < Sk) a = *(const u32x4*)src;
    if (s + 1 < Sk) a2 = *(const u32x4*)(src + vss);
    uint32_t wd[8];  // (key 2kp, key 2kp + 1) of d = 8c + j
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      wd[2 * i] = (a[i] & 0xffffu) | (a2[i] << 16);
      wd[2 * i + 1] = (a[i] >> 16) | (a2[i] & 0xffff0000u);
    }
    const int key = 2 * kp;
    const int slot = (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1);
    const int col = slot ^ (32 * ((c >> 1) & 1));
    const int flip = c & 1;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj)
      *(uint32_t*)&sVt[(8 * c + (jj ^ flip)) * BN + col] = flip ? wd[jj ^ 1] : wd[jj];
  }
  __syncthreads();
  for (int it = tid; it < D * (BN / 8); it += 256) {
    const int d = it / (BN / 8), c = it % (BN / 8);
    const int pc = c ^ (4 * ((d >> 4) & 1));
    *(u32x4*)(vn + ((int64_t)bh * D + d) * Skp + s0 + 8 * c) = *(const u32x4*)&sVt[d * BN + 8 * pc];
  }
}

// Load this lane's rotated Q fragment: slots ks cover d = 16ks + 8h + 0..7.
template <typename T, int D>
__device__ __forceinline__ void load_q_frag(const T* __restrict__ q,
                                            const float* __restrict__ cos,
                                            const float* __restrict__ sin, const RowInfo& ri,
                                            int Sq, int Hq, int hh, bf16x8* qf) {
  constexpr int KS = D / 16, HALF = D / 2;
  if (!ri.q_valid) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = as_bf16x8(u32x4{0u, 0u, 0u, 0u});
    return;
  }
  const T* qrow = q + (((int64_t)ri.b * Sq + ri.pos) * Hq + ri.hq) * D;
  const float* cr = cos + (int64_t)ri.pos * HALF;
  const float* sr = sin + (int64_t)ri.pos * HALF;
#pragma unroll
  for (int ks = 0; ks < KS / 2; ++ks) {
    const int d0 = 16 * ks + 8 * hh;
    float x1[8], x2[8];
    unpack8<T>(*(const u32x4*)(qrow + d0), x1);
    unpack8<T>(*(const u32x4*)(qrow + d0 + HALF), x2);
    u32x4 o1, o2;
    rope8<T>(x1, x2, cr + d0, sr + d0, o1, o2);
    qf[ks] = as_bf16x8(o1);
    qf[ks + KS / 2] = as_bf16x8(o2);
  }
}

// MODE selects the explicit mask (causal self-attention, Sq == Sk):
//  MASK_DOC  packed documents (aux = document ids).  The workgroup walks only
//            the key tiles listed by doc_tile_list, last to first; listed tiles
//            carrying the mask flag get the element test doc[key] == doc[query]
//            next to the causal one.
//  MASK_KPM  key padding (aux = 1 for a valid key).  Tiles without a valid key
//            are skipped; tiles with some padded keys get the element test.
//            Rows before the first valid key (the guarded prefix) attend every
//            key, so a workgroup holding one walks all tiles.
// The running max starts at -1e30 instead of -inf in both, because a row can
// see no key at all in a listed tile (exp2 of -inf - -inf would be NaN); every
// row sees some key in some tile, so the final max is a real score.
template <typename T, int D, int MODE>
__global__ __launch_bounds__(256, 2) void fwd_mfma_kernel(
    const T* __restrict__ q, const float* __restrict__ cos, const float* __restrict__ sin,
    const T* __restrict__ krot, const T* __restrict__ vn, T* __restrict__ out,
    float* __restrict__ lse, int Sq, int Sk, int Skp, int krows, int Hq, int Hkv, int n_rep,
    int bm_pos, int nqb, float scale_log2, int causal, const int32_t* __restrict__ aux,
    const int2* __restrict__ ranges, T* __restrict__ qrot, const int* __restrict__ order,
    const int* __restrict__ kpm_flags) {
  constexpr bool DOC = MODE == MASK_DOC, KPM = MODE == MASK_KPM, LIST = DOC || KPM;
  constexpr int KS = D / 16, DT = D / 32;
  constexpr int KR = D / 8;  // 16-byte chunks per K / V row
  __shared__ __attribute__((aligned(16))) T sK[2][BN * D];
  __shared__ __attribute__((aligned(16))) T sV[2][BN * D];
  __shared__ __attribute__((aligned(16))) int32_t sKD[2][BN];  // LIST: per-key aux values
  __shared__ uint16_t sList[DOC_MAX_TILES];                     // LIST: listed key tiles
  __shared__ int sCount, sFirst;

  const int tid = threadIdx.x, w = wave_id(), lane = tid & 63, hh = lane >> 5, c32 = lane & 31;
  int logical = xcd_logical_id(blockIdx.x, gridDim.x, nqb);
  if (order != nullptr) {
    // DOC: the workgroup of rank r takes the (batch row, query block) of the
    // r-th most listed key tiles, its KV heads adjacent (longest first, each
    // XCD every 8th)
    const int bq = order[blockIdx.x / Hkv];
    logical = ((bq / nqb) * Hkv + (int)blockIdx.x % Hkv) * nqb + (nqb - 1 - bq % nqb);
  }
  const RowInfo ri = row_info(logical, nqb, Hkv, n_rep, bm_pos, Sq, w * 32 + c32);
  const int bh = ri.b * Hkv + ri.g;

  const int kend = causal ? min(Sk, min(ri.p0 + bm_pos, Sq)) : Sk;
  int ntiles = (kend + BN - 1) / BN;
  const int32_t* arow = LIST ? aux + (int64_t)ri.b * Sk : nullptr;
  const int2* rec = ranges + (int64_t)ri.b * (Skp / BN);
  // kpm_flags (per batch row, 1 = every key valid): those rows are fwd32_kernel's
  if (KPM && kpm_flags != nullptr && kpm_flags[ri.b] != 0) return;
  const T* kbase = krot + (int64_t)bh * krows * D;
  const T* vbase = vn + (int64_t)bh * D * Skp;  // V^T, keys in fragment order
  auto stage = [&](int t, int buf) {
    tile_to_lds<BN, KR>(kbase + (int64_t)t * BN * D, D, sK[buf], w, lane);
    tile_to_lds<D, BN / 8>(vbase + (int64_t)t * BN, Skp, sV[buf], w, lane);
    if (LIST && w == 0) dma4(lds_addr(sKD[buf]), (uint32_t)min(t * BN + lane, Sk - 1) * 4u, arow);
  };
  int di = 0;       // DOC: this row's document
  bool grd = false;  // KPM: this row is in the guarded prefix
  if constexpr (DOC) {
    // The list is walked backwards.  Its last tile, the one holding the
    // block's last position, is always listed: it loads while the list is built.
    if (ntiles > 0) stage(ntiles - 1, 0);
    di = arow[min(ri.pos, Sq - 1)];
    if (w == 0) {
      const int n = doc_tile_list(arow, ri.p0, min(ri.p0 + bm_pos, Sq), rec, 0, ntiles, sList,
                                  lane);
      if (lane == 0) sCount = n;
    }
    __syncthreads();
    ntiles = __builtin_amdgcn_readfirstlane(sCount);
  } else if constexpr (KPM) {
    const int nall = Skp / BN;
    if (w == 0) {
      const int fv = kpm_first_valid(rec, nall, lane);
      // a guarded row attends every key: list (and test) every tile
      const bool guard_block = ri.p0 < fv;
      const int n = kpm_tile_list(rec, 0, guard_block ? nall : ntiles,
                                  [&](int, int2 r) { return guard_block ? 2 : r.x == 0 ? 0 : r.x < BN ? 2 : 1; },
                                  sList, lane);
      if (lane == 0) {
        sCount = n;
        sFirst = fv;
      }
    }
    __syncthreads();
    ntiles = __builtin_amdgcn_readfirstlane(sCount);
    grd = ri.pos < sFirst;
  } else {
    if (ntiles > 0) stage(0, 0);
  }
  // iteration -> entry (tile | DOC_MASK_FLAG when it needs the element test)
  auto entry = [&](int it) -> int {
    return DOC ? __builtin_amdgcn_readfirstlane((int)sList[ntiles - 1 - it])
               : KPM ? __builtin_amdgcn_readfirstlane((int)sList[it]) : it;
  };
  auto tile_of = [](int e) -> int { return LIST ? e & ~DOC_MASK_FLAG : e; };
  if (KPM && ntiles > 0) stage(tile_of(entry(0)), 0);

  bf16x8 qf[KS];
  load_q_frag<T, D>(q, cos, sin, ri, Sq, Hq, hh, qf);

  float m = LIST ? -1e30f : -INFINITY, lsum = 0.f;
  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[dt][i] = 0.f;

  lds_copy_wait();
  __syncthreads();
  // the tile loop unrolled by two, so that each copy's LDS buffer is a
  // compile-time constant: fragment addresses are then loop-invariant per lane
  // (the buffer only changes the instruction's immediate offset)
  auto tile_body = [&](int it, auto bufc) {
    constexpr int buf = decltype(bufc)::value;
    const int e = entry(it);
    const int t = tile_of(e);
    if (it + 1 < ntiles) stage(tile_of(entry(it + 1)), buf ^ 1);
    const T* tK = sK[buf];
    const T* tV = sV[buf];

    f32x16 s[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) s[mt][i] = 0.f;
    // fragment reads three MFMAs ahead of their use (the order fenced against
    // the scheduler, which otherwise issues each read right before its MFMA)
    {
      constexpr int NQ = 2 * KS;
      auto kfrag = [&](int j) { return lds_frag<KR>(tK, 32 * (j & 1) + c32, 2 * (j >> 1) + hh); };
      bf16x8 fa[NQ];
#pragma unroll
      for (int j = 0; j < FWD_PF; ++j) fa[j] = kfrag(j);
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        __builtin_amdgcn_sched_barrier(0);
        if (j + FWD_PF < NQ) fa[j + FWD_PF] = kfrag(j + FWD_PF);
        s[j & 1] = mfma32<T>(fa[j], qf[j >> 1], s[j & 1]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }

    const int k0 = t * BN;
    const bool need_mask = (causal && k0 + BN - 1 > ri.p0) || (k0 + BN > Sk);
    if (LIST && (e & DOC_MASK_FLAG)) {
      // DOC: causal and same document; KPM: causal and valid, or anything
      // below Sk for a guarded row
      const int lim = (grd ? Sk - 1 : min(ri.pos, Sk - 1)) - k0;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const i32x4 kd = *(const i32x4*)&sKD[buf][32 * mt + 8 * g4 + 4 * hh];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int local = 32 * mt + 8 * g4 + 4 * hh + j;
            const int i = 4 * g4 + j;
            const bool other = DOC ? kd[j] != di : (!grd && kd[j] == 0);
            s[mt][i] = (local > lim || other) ? -INFINITY : s[mt][i];
          }
        }
    } else if (need_mask) {
      // last visible key of this lane's row, relative to k0 (branch-free select)
      const int lim = (causal ? min(ri.pos, Sk - 1) : Sk - 1) - k0;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int local = 32 * mt + 8 * (i >> 2) + 4 * hh + (i & 3);
          s[mt][i] = local > lim ? -INFINITY : s[mt][i];
        }
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) tmax = fmaxf(tmax, s[mt][i]);
    tmax = pair_max32(tmax) * scale_log2;
    // Rescale the running output only when some row's max grew by more than
    // RESCALE_SLACK (log2 units): until then the exponent base m lags the
    // row's max by at most that much, so p <= 2^RESCALE_SLACK, well inside
    // bf16, fp16 and fp32 range with their precision unchanged (O / l and the LSE
    // m + log2(l) are exact for any base).  Rows whose max did not move keep
    // alpha = 1.  The branch is wavefront-uniform.
    if (__builtin_amdgcn_ballot_w64(tmax > m + RESCALE_SLACK) != 0) {
      const float mnew = fmaxf(m, tmax);
      const float alpha = fast_exp2(m - mnew);
      lsum *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[dt][i] *= alpha;
      m = mnew;
    }
    float psum = 0.f;
    u32x4 pk[4];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        const float p0 = fast_exp2(__builtin_fmaf(s[mt][i], scale_log2, -m));
        const float p1 = fast_exp2(__builtin_fmaf(s[mt][i + 1], scale_log2, -m));
        psum += p0 + p1;
        pk[2 * mt + (i >> 3)][(i & 7) >> 1] = pack2<T>(p0, p1);
      }
    lsum += psum;
    {
      constexpr int NV = 4 * DT;
      auto vfrag = [&](int j) {
        return lds_frag<BN / 8>(tV, 32 * (j % DT) + c32, 2 * (j / DT) + hh);
      };
      bf16x8 fb[NV];
#pragma unroll
      for (int j = 0; j < FWD_PF; ++j) fb[j] = vfrag(j);
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        __builtin_amdgcn_sched_barrier(0);
        if (j + FWD_PF < NV) fb[j + FWD_PF] = vfrag(j + FWD_PF);
        acc[j % DT] = mfma32<T>(fb[j], as_bf16x8(pk[j / DT]), acc[j % DT]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    lds_copy_wait();
    __syncthreads();
  };
  for (int it = 0; it < ntiles; it += 2) {
    tile_body(it, std::integral_constant<int, 0>{});
    if (it + 1 < ntiles) tile_body(it + 1, std::integral_constant<int, 1>{});
  }

  const float ltot = pair_sum32(lsum);
  const float inv = 1.f / ltot;
  // The output leaves through LDS (the tile buffers are free after the loop's
  // last barrier): each wavefront writes its 32 rows into its own 32 x D slice,
  // 16-byte chunks XOR-swizzled by row, then stores whole 16-byte chunks, each
  // row by KR consecutive lanes, so a store instruction covers 64 / KR whole
  // rows instead of 16 bytes of each of 32 rows.
  T* slice = &sK[0][0] + w * 32 * D;  // 32 rows x D (sK holds 2 x 64 rows)
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
      const int ch = 4 * dt + gi;  // 16-byte chunk of columns 32 dt + 8 gi ..
      u32x2 pk2;
      pk2[0] = pack2<T>(acc[dt][4 * gi] * inv, acc[dt][4 * gi + 1] * inv);
      pk2[1] = pack2<T>(acc[dt][4 * gi + 2] * inv, acc[dt][4 * gi + 3] * inv);
      *(u32x2*)(slice + (c32 * KR + (ch ^ (c32 & (KR - 1)))) * 8 + 4 * hh) = pk2;
    }
  __syncthreads();
#pragma unroll
  for (int i2 = 0; i2 < 32 * KR / 64; ++i2) {
    const int L = 64 * i2 + lane, row = L / KR, ch = L % KR;
    const u32x4 v = *(const u32x4*)(slice + (row * KR + (ch ^ (row & (KR - 1)))) * 8);
    const RowInfo rj = row_info(logical, nqb, Hkv, n_rep, bm_pos, Sq, w * 32 + row);
    if (rj.q_valid) *(u32x4*)(out + (((int64_t)rj.b * Sq + rj.pos) * Hq + rj.hq) * D + 8 * ch) = v;
  }
  if (qrot != nullptr) {
    // the rotated q rows for the backward, the same way (read there long after:
    // streaming stores); fragment ks holds the row's 16-byte chunk c below
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int c = ks < KS / 2 ? 2 * ks + hh : KR / 2 + 2 * (ks - KS / 2) + hh;
      *(u32x4*)(slice + (c32 * KR + (c ^ (c32 & (KR - 1)))) * 8) = __builtin_bit_cast(u32x4, qf[ks]);
    }
    __syncthreads();
#pragma unroll
    for (int i2 = 0; i2 < 32 * KR / 64; ++i2) {
      const int L = 64 * i2 + lane, row = L / KR, ch = L % KR;
      const u32x4 v = *(const u32x4*)(slice + (row * KR + (ch ^ (row & (KR - 1)))) * 8);
      const RowInfo rj = row_info(logical, nqb, Hkv, n_rep, bm_pos, Sq, w * 32 + row);
      if (rj.q_valid)
        __builtin_nontemporal_store(
            v, (u32x4*)(qrot + (((int64_t)rj.b * Hq + rj.hq) * krows + rj.pos) * D + 8 * ch));
    }
  }
  if (ri.q_valid && lse != nullptr && hh == 0)
    lse[((int64_t)ri.b * Hq + ri.hq) * Sq + ri.pos] = (m + log2f(ltot)) * kLn2;
}

// Forward without an explicit mask on 32-key tiles: half the LDS (32 KB per
// workgroup, K and V^T double-buffered) and half the score registers of
// fwd_mfma_kernel, so that three workgroups share a CU (three wavefronts per
// SIMD to hide each one's MFMA -> softmax -> MFMA dependencies; measured on
// the loop's skeleton: 1779 against 1444 TFLOP/s for two workgroups of
// 64-key tiles).  Same rows per workgroup and the same per-key arithmetic as
// fwd_mfma_kernel; the running max is taken per 32-key tile, so the points
// where the output is rescaled (and with them the last bits) can differ.
constexpr int FBN = 32;  // keys per tile of fwd32_kernel
template <typename T, int D>
__global__ __launch_bounds__(256, 3) void fwd32_kernel(
    const T* __restrict__ q, const float* __restrict__ cos, const float* __restrict__ sin,
    const T* __restrict__ krot, const T* __restrict__ vn, T* __restrict__ out,
    float* __restrict__ lse, int Sq, int Sk, int Skp, int krows, int Hq, int Hkv, int n_rep,
    int bm_pos, int nqb, float scale_log2, int causal, T* __restrict__ qrot,
    const int* __restrict__ kpm_flags) {
  constexpr int KS = D / 16, DT = D / 32;
  constexpr int KR = D / 8;  // 16-byte chunks per K row
  __shared__ __attribute__((aligned(16))) T sK[2][FBN * D];
  __shared__ __attribute__((aligned(16))) T sV[2][D * FBN];

  const int tid = threadIdx.x, w = wave_id(), lane = tid & 63, hh = lane >> 5, c32 = lane & 31;
  const int logical = xcd_logical_id(blockIdx.x, gridDim.x, nqb);
  const RowInfo ri = row_info(logical, nqb, Hkv, n_rep, bm_pos, Sq, w * 32 + c32);
  // key padding (kpm_flags per batch row, 1 = every key valid): only the rows
  // without padding (plain causal attention); fwd_mfma_kernel takes the others
  if (kpm_flags != nullptr && kpm_flags[ri.b] == 0) return;
  const int bh = ri.b * Hkv + ri.g;
  const int kend = causal ? min(Sk, min(ri.p0 + bm_pos, Sq)) : Sk;
  const int ntiles = (kend + FBN - 1) / FBN;
  const T* kbase = krot + (int64_t)bh * krows * D;
  const T* vbase = vn + (int64_t)bh * D * Skp;  // V^T, keys in fragment order
  auto stage = [&](int t, int buf) {
    tile_to_lds<FBN, KR>(kbase + (int64_t)t * FBN * D, D, sK[buf], w, lane);
    tile_to_lds<D, FBN / 8>(vbase + (int64_t)t * FBN, Skp, sV[buf], w, lane);
  };
  if (ntiles > 0) stage(0, 0);

  bf16x8 qf[KS];
  load_q_frag<T, D>(q, cos, sin, ri, Sq, Hq, hh, qf);

  float m = -INFINITY, lsum = 0.f;
  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[dt][i] = 0.f;

  lds_copy_wait();
  __syncthreads();
  auto tile_body = [&](int it, auto bufc) {
    constexpr int buf = decltype(bufc)::value;
    if (it + 1 < ntiles) stage(it + 1, buf ^ 1);
    const T* tK = sK[buf];
    const T* tV = sV[buf];

    // S^T of the tile's 32 keys x this wavefront's 32 rows
    f32x16 s;
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = 0.f;
    {
      auto kfrag = [&](int j) { return lds_frag<KR>(tK, c32, 2 * j + hh); };
      bf16x8 fa[KS];
#pragma unroll
      for (int j = 0; j < FWD_PF; ++j) fa[j] = kfrag(j);
#pragma unroll
      for (int j = 0; j < KS; ++j) {
        __builtin_amdgcn_sched_barrier(0);
        if (j + FWD_PF < KS) fa[j + FWD_PF] = kfrag(j + FWD_PF);
        s = mfma32<T>(fa[j], qf[j], s);
      }
      __builtin_amdgcn_sched_barrier(0);
    }

    const int k0 = it * FBN;
    if ((causal && k0 + FBN - 1 > ri.p0) || (k0 + FBN > Sk)) {
      // last visible key of this lane's row, relative to k0 (branch-free select)
      const int lim = (causal ? min(ri.pos, Sk - 1) : Sk - 1) - k0;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int local = 8 * (i >> 2) + 4 * hh + (i & 3);
        s[i] = local > lim ? -INFINITY : s[i];
      }
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) tmax = fmaxf(tmax, s[i]);
    tmax = pair_max32(tmax) * scale_log2;
    if (__builtin_amdgcn_ballot_w64(tmax > m + RESCALE_SLACK) != 0) {
      const float mnew = fmaxf(m, tmax);
      const float alpha = fast_exp2(m - mnew);
      lsum *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[dt][i] *= alpha;
      m = mnew;
    }
    float psum = 0.f;
    u32x4 pk[2];
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      const float p0 = fast_exp2(__builtin_fmaf(s[i], scale_log2, -m));
      const float p1 = fast_exp2(__builtin_fmaf(s[i + 1], scale_log2, -m));
      psum += p0 + p1;
      pk[i >> 3][(i & 7) >> 1] = pack2<T>(p0, p1);
    }
    lsum += psum;
    {
      constexpr int NV = 2 * DT;
      auto vfrag = [&](int j) {
        return lds_frag<FBN / 8>(tV, 32 * (j % DT) + c32, 2 * (j / DT) + hh);
      };
      bf16x8 fb[NV];
#pragma unroll
      for (int j = 0; j < FWD_PF; ++j) fb[j] = vfrag(j);
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        __builtin_amdgcn_sched_barrier(0);
        if (j + FWD_PF < NV) fb[j + FWD_PF] = vfrag(j + FWD_PF);
        acc[j % DT] = mfma32<T>(fb[j], as_bf16x8(pk[j / DT]), acc[j % DT]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    lds_copy_wait();
    __syncthreads();
  };
  for (int it = 0; it < ntiles; it += 2) {
    tile_body(it, std::integral_constant<int, 0>{});
    if (it + 1 < ntiles) tile_body(it + 1, std::integral_constant<int, 1>{});
  }

  const float ltot = pair_sum32(lsum);
  const float inv = 1.f / ltot;
  // The output leaves through LDS (the tile buffers are free after the loop's
  // last barrier): each wavefront writes its 32 rows into its own 32 x D slice,
  // 16-byte chunks XOR-swizzled by row, then stores whole 16-byte chunks, each
  // row by KR consecutive lanes, so a store instruction covers 64 / KR whole
  // rows instead of 16 bytes of each of 32 rows.
  T* slice = w < 2 ? sK[w] : sV[w - 2];  // FBN x D elements = 32 rows x D
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
      const int ch = 4 * dt + gi;  // 16-byte chunk of columns 32 dt + 8 gi ..
      u32x2 pk2;
      pk2[0] = pack2<T>(acc[dt][4 * gi] * inv, acc[dt][4 * gi + 1] * inv);
      pk2[1] = pack2<T>(acc[dt][4 * gi + 2] * inv, acc[dt][4 * gi + 3] * inv);
      *(u32x2*)(slice + (c32 * KR + (ch ^ (c32 & (KR - 1)))) * 8 + 4 * hh) = pk2;
    }
  __syncthreads();
#pragma unroll
  for (int i2 = 0; i2 < 32 * KR / 64; ++i2) {
    const int L = 64 * i2 + lane, row = L / KR, ch = L % KR;
    const u32x4 v = *(const u32x4*)(slice + (row * KR + (ch ^ (row & (KR - 1)))) * 8);
    const RowInfo rj = row_info(logical, nqb, Hkv, n_rep, bm_pos, Sq, w * 32 + row);
    if (rj.q_valid) *(u32x4*)(out + (((int64_t)rj.b * Sq + rj.pos) * Hq + rj.hq) * D + 8 * ch) = v;
  }
  if (qrot != nullptr) {
    // the rotated q rows for the backward, the same way (read there long after:
    // streaming stores); fragment ks holds the row's 16-byte chunk c below
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int c = ks < KS / 2 ? 2 * ks + hh : KR / 2 + 2 * (ks - KS / 2) + hh;
      *(u32x4*)(slice + (c32 * KR + (c ^ (c32 & (KR - 1)))) * 8) = __builtin_bit_cast(u32x4, qf[ks]);
    }
    __syncthreads();
#pragma unroll
    for (int i2 = 0; i2 < 32 * KR / 64; ++i2) {
      const int L = 64 * i2 + lane, row = L / KR, ch = L % KR;
      const u32x4 v = *(const u32x4*)(slice + (row * KR + (ch ^ (row & (KR - 1)))) * 8);
      const RowInfo rj = row_info(logical, nqb, Hkv, n_rep, bm_pos, Sq, w * 32 + row);
      if (rj.q_valid)
        __builtin_nontemporal_store(
            v, (u32x4*)(qrot + (((int64_t)rj.b * Hq + rj.hq) * krows + rj.pos) * D + 8 * ch));
    }
  }
  // this row's LSE: its index recomputed here from a laundered row number, so
  // the prologue's 64-bit value is not kept live (in scratch) across the loop
  int r_l = w * 32 + c32;
  asm volatile("" : "+v"(r_l));
  const RowInfo rl = row_info(logical, nqb, Hkv, n_rep, bm_pos, Sq, r_l);
  if (rl.q_valid && lse != nullptr && hh == 0)
    lse[((int64_t)rl.b * Hq + rl.hq) * Sq + rl.pos] = (m + log2f(ltot)) * kLn2;
}

// Capture: LSE, the probabilities P = exp(s - lse) as float32 [B, Hq, Sq, Sk]
// and out = P·V in one launch; a workgroup takes the query blocks r and
// nqb-1-r of one KV head, one after the other.  The workgroup walks a block's
// key tiles twice in the forward's S^T = K·Q^T layout (a lane holds one query
// row's 32 scores of a 64-key tile): the first walk forms each row's running
// max and sum only (no P·V), with the four tile buffers as a ring of K tiles
// staged three ahead; the second forms the normalised P, stores it, and
// accumulates O^T = V^T·P^T from P rounded to T, so O needs no final
// division.  P leaves through an LDS slice per wavefront (see store_p) as
// whole 128-byte line segments.  The stores of tile t issue in tile t+1,
// after its tile loads and zero rows: the end-of-tile wait (vmcnt counts loads
// and stores together, in issue order) can then leave them in flight through
// tile t+2.  Key tiles right of the causal frontier are zero without
// computing; their rows are spread over the tile iterations.  Stores are
// non-temporal: nothing reads P back, and cached it would evict the K and V
// tiles the other workgroups of the KV head re-read.  Pairing a long query
// block with a short one gives every workgroup about the same work, so the
// grid runs as one even wave; one block per workgroup (long and short blocks
// alternating) left the CUs of the long blocks busy long after the others had
// drained.  Explicit masks as in the
// forward (MASK_DOC: other documents get P = 0; MASK_KPM: padded keys get 0,
// except in guarded rows before the first valid key, which attend every key
// below Sk, so a workgroup holding one walks every tile); with an explicit
// mask every tile takes the element test.
template <typename T, int D, int MODE>
__global__ __launch_bounds__(256, 2) void capture_probs_mfma_kernel(
    const T* __restrict__ q, const float* __restrict__ cos, const float* __restrict__ sin,
    const T* __restrict__ krot, const T* __restrict__ vn, T* __restrict__ out,
    float* __restrict__ lse, float* __restrict__ probs, int Sq, int Sk, int Skp, int Hq, int Hkv,
    int n_rep, int bm_pos, int nqb, float scale_log2, int causal,
    const int32_t* __restrict__ aux, const int2* __restrict__ ranges) {
  constexpr bool DOC = MODE == MASK_DOC, KPM = MODE == MASK_KPM, LIST = DOC || KPM;
  constexpr int KS = D / 16, DT = D / 32;
  constexpr int KR = D / 8;
  __shared__ __attribute__((aligned(16))) T sK[2][BN * D];
  __shared__ __attribute__((aligned(16))) T sV[2][BN * D];
  __shared__ __attribute__((aligned(16))) int32_t sKD[4][BN];  // LIST: per-key aux values
  __shared__ __attribute__((aligned(16))) float sP[4][32 * 32];  // per wave: 32 rows x 32 keys

  // workgroup = query blocks r and nqb-1-r of one (batch row, KV head): every
  // workgroup gets about the same number of key tiles, so the grid runs in one
  // even wave (one block per workgroup leaves the long blocks' CUs busy long
  // after the short ones' have drained)
  const int npair = (nqb + 1) / 2;
  const int pl = xcd_logical_id(blockIdx.x, gridDim.x, npair);
  const int bhq = pl / npair, pr = pl % npair;
  const int nb = 2 * pr + 1 == nqb ? 1 : 2;
  for (int kb = 0; kb < nb; ++kb) {
    // length rank of this block (0 = longest): even workgroups take the long
    // one first, odd ones the short one
    const int zq = (kb ^ (pl & 1)) == 0 ? pr : nqb - 1 - pr;
    if (kb > 0) __syncthreads();  // the previous block's LDS reads are done
    // the lane's values are formed anew per block (laundered): held across
    // the block loop, the addresses derived from them spill
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int w = wave_id(), lane = tid & 63, hh = lane >> 5, c32 = lane & 31;
    // row_info maps logical index bh*nqb + j to query block nqb-1-j
    const RowInfo ri = row_info(bhq * nqb + zq, nqb, Hkv, n_rep, bm_pos, Sq, w * 32 + c32);
    const int bh = ri.b * Hkv + ri.g;
    const int32_t* arow = LIST ? aux + (int64_t)ri.b * Sk : nullptr;
    const int nrows = n_rep * bm_pos;  // rows of the block in use

    const int qmax = min(ri.p0 + bm_pos, Sq) - 1;  // largest position in the block
    const int ntiles_all = (Sk + BN - 1) / BN;
    // KPM: first valid key of the batch row; rows before it are guarded
    const int fv = KPM ? kpm_first_valid(ranges + (int64_t)ri.b * (Skp / BN), Skp / BN, lane) : 0;
    const int ntiles = causal && !(KPM && ri.p0 < fv) ? min(ntiles_all, (qmax + BN) / BN)
                                                        : ntiles_all;
    const int di = DOC ? arow[min(ri.pos, Sq - 1)] : 0;  // DOC: this row's document
    const bool grd = KPM && ri.pos < fv;                  // KPM: guarded row
    const T* kbase = krot + (int64_t)bh * Skp * D;
    const T* vbase = vn + (int64_t)bh * D * Skp;  // V^T, keys in fragment order
    auto stage_k = [&](int t, int buf) {
      tile_to_lds<BN, KR>(kbase + (int64_t)t * BN * D, D, sK[buf], w, lane);
      if (LIST && w == 0) dma4(lds_addr(sKD[buf]), (uint32_t)min(t * BN + lane, Sk - 1) * 4u, arow);
    };
    auto stage_v = [&](int t, int buf) {
      tile_to_lds<D, BN / 8>(vbase + (int64_t)t * BN, Skp, sV[buf], w, lane);
    };
    // Walk 1 reads only K tiles: all four tile buffers form its ring, staged
    // three tiles ahead (slot s: sK[0], sK[1], sV[0], sV[1]; aux values in sKD[s])
    T* const ring[4] = {sK[0], sK[1], sV[0], sV[1]};
    auto stage_kr = [&](int t, int slot) {
      tile_to_lds<BN, KR>(kbase + (int64_t)t * BN * D, D, ring[slot], w, lane);
      if (LIST && w == 0)
        dma4(lds_addr(sKD[slot]), (uint32_t)min(t * BN + lane, Sk - 1) * 4u, arow);
    };
#pragma unroll
    for (int t = 0; t < 3; ++t)
      if (t < ntiles) stage_kr(t, t);

    bf16x8 qf[KS];
    load_q_frag<T, D>(q, cos, sin, ri, Sq, Hq, hh, qf);

    // S^T of tile t with masked scores set to -inf
    auto scores = [&](int t, const T* tK, const int32_t* kdl, f32x16 (&s)[2]) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) s[mt][i] = 0.f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const bf16x8 a = lds_frag<KR>(tK, 32 * mt + c32, 2 * ks + hh);
          s[mt] = mfma32<T>(a, qf[ks], s[mt]);
        }
      }
      const int k0 = t * BN;
      if constexpr (LIST) {
        // explicit masks come with causal self-attention
        const int lim = (grd ? Sk - 1 : min(ri.pos, Sk - 1)) - k0;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            const i32x4 kd = *(const i32x4*)&kdl[32 * mt + 8 * g4 + 4 * hh];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int local = 32 * mt + 8 * g4 + 4 * hh + j;
              const bool other = DOC ? kd[j] != di : (!grd && kd[j] == 0);
              s[mt][4 * g4 + j] = (local > lim || other) ? -INFINITY : s[mt][4 * g4 + j];
            }
          }
      } else if ((causal && k0 + BN - 1 > ri.p0) || k0 + BN > Sk) {
        const int lim = (causal ? min(ri.pos, Sk - 1) : Sk - 1) - k0;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int local = 32 * mt + 8 * (i >> 2) + 4 * hh + (i & 3);
            s[mt][i] = local > lim ? -INFINITY : s[mt][i];
          }
      }
    };

    // Key tiles right of the causal frontier are zero.  Their rows are written
    // in 2*ntiles pieces, one at the start of each tile iteration of the two
    // walks (ahead of that iteration's tile loads), so the zeros stream out
    // while the block computes instead of after it.
    const bool vec4 = (Sk & 3) == 0;  // 16-byte aligned rows
    const int zstart = ntiles * BN;
    const int zper = causal && zstart < Sk ? (nrows + 2 * ntiles - 1) / (2 * ntiles) : 0;
    auto zero_rows = [&](int z) {
      const int r1 = min(z * zper + zper, nrows);
      for (int r = z * zper; r < r1; ++r) {
        const int pos = ri.p0 + r % bm_pos;
        if (pos >= Sq) continue;
        float* zrow =
            probs + (((int64_t)ri.b * Hq + (int64_t)ri.g * n_rep + r / bm_pos) * Sq + pos) * Sk;
        for (int key = zstart + tid * 4; key < Sk; key += 256 * 4) {
          if (vec4) {
            __builtin_nontemporal_store(f32x4{0.f, 0.f, 0.f, 0.f}, (f32x4*)(zrow + key));
          } else {
            for (int e = key; e < min(key + 4, Sk); ++e) zrow[e] = 0.f;
          }
        }
      }
    };

    lds_copy_wait();
    __syncthreads();
    // Walk 1: running max m and sum (log2 domain).  Starting m at -1e30 keeps
    // exp2(m - mnew) finite for a row that sees no key in a tile.  Its last
    // iteration stages tile 0 of walk 2 (K and V) into the buffer pair whose
    // slots it is not reading (pair 1 when ntiles is odd).  Walk 1 is unrolled
    // by four and walk 2 by two so that each copy's LDS buffer is a
    // compile-time constant.
    float m = -1e30f, lsum = 0.f;
    constexpr int NK = BN * KR / 64 / 4;  // direct loads per lane of one K tile
    auto body1 = [&](int it, auto slotc) {
      constexpr int slot = decltype(slotc)::value;
      zero_rows(it);
      if (it + 3 < ntiles) {
        stage_kr(it + 3, (slot + 3) & 3);
      } else if (it + 1 == ntiles) {
        stage_k(0, (slot & 1) ^ 1);
        stage_v(0, (slot & 1) ^ 1);
      }
      f32x16 s[2];
      scores(it, ring[slot], sKD[slot], s);
      float tmax = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) tmax = fmaxf(tmax, s[mt][i]);
      const float mnew = fmaxf(m, pair_max32(tmax) * scale_log2);
      float psum = 0.f;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) psum += fast_exp2(__builtin_fmaf(s[mt][i], scale_log2, -mnew));
      lsum = lsum * fast_exp2(m - mnew) + psum;
      m = mnew;
      // tile it + 1 in LDS; tiles it + 2 and it + 3 (NK loads per lane each,
      // issued after it) may stay in flight
      if (it + 3 < ntiles)
        vm_wait<2 * NK>();
      else if (it + 2 < ntiles)
        vm_wait<NK>();
      else
        lds_copy_wait();
      __syncthreads();
    };
    for (int it = 0; it < ntiles; it += 4) {
      body1(it, std::integral_constant<int, 0>{});
      if (it + 1 < ntiles) body1(it + 1, std::integral_constant<int, 1>{});
      if (it + 2 < ntiles) body1(it + 2, std::integral_constant<int, 2>{});
      if (it + 3 < ntiles) body1(it + 3, std::integral_constant<int, 3>{});
    }
    const float L = m + log2f(pair_sum32(lsum));  // log2-domain LSE of this row
    if (ri.q_valid && hh == 0) lse[((int64_t)ri.b * Hq + ri.hq) * Sq + ri.pos] = L * kLn2;

    // Walk 2: P, its stores, and O^T += V^T P^T
    f32x16 acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[dt][i] = 0.f;
    // P leaves through the wave's LDS slice, 32 rows x 32 keys at a time: the C
    // layout is written as 16-byte chunks (chunk c of row r at c ^ (r & 7), so
    // neither the writes nor the reads conflict) and read back so that 8 lanes
    // cover a row's 128 bytes: every store instruction writes 8 whole 128-byte
    // line segments.  Lane l stores rows 8j + l/8 (j = 0..3) of the wave.
    float* prs[4];
    int pvalid = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = w * 32 + 8 * j + (lane >> 3);
      const int pos = ri.p0 + r % bm_pos;
      const bool ok = r < nrows && pos < Sq;
      pvalid |= (int)ok << j;
      prs[j] = probs + (((int64_t)ri.b * Hq + (int64_t)ri.g * n_rep + (ok ? r / bm_pos : 0)) * Sq +
                        (ok ? pos : 0)) * Sk;
    }
    float* stg = sP[w];
    f32x16 held[2];  // P of the previous tile, stored by the next
    // true when every lane of store_p(t)'s 8 store instructions is active, so
    // that exactly 8 vector-memory instructions issue
    auto full_p = [&](int t) { return pvalid == 15 && vec4 && (t + 1) * BN <= Sk; };
    auto store_p = [&](int t) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4)
          *(f32x4*)&stg[c32 * 32 + (((2 * g4 + hh) ^ (c32 & 7)) * 4)] =
              f32x4{held[mt][4 * g4], held[mt][4 * g4 + 1], held[mt][4 * g4 + 2],
                    held[mt][4 * g4 + 3]};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int rr = 8 * j + (lane >> 3), cl = lane & 7;
          const f32x4 v4 = *(const f32x4*)&stg[rr * 32 + ((cl ^ (rr & 7)) * 4)];
          const int key = t * BN + 32 * mt + 4 * cl;
          if (!((pvalid >> j) & 1)) continue;
          if (vec4) {
            if (key < Sk) __builtin_nontemporal_store(v4, (f32x4*)(prs[j] + key));
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (key + e < Sk) prs[j][key + e] = v4[e];
          }
        }
      }
    };
    auto body2 = [&](int it, auto bufc) {
      constexpr int buf = decltype(bufc)::value;
      // the tile loads, the zero rows, then P of tile it - 1: the 8 P stores
      // are the last vector-memory instructions of the tile, so the end-of-tile
      // wait can leave them in flight through the next tile
      if (it + 1 < ntiles) {
        stage_k(it + 1, buf ^ 1);
        stage_v(it + 1, buf ^ 1);
      }
      zero_rows(ntiles + it);
      const bool full = it > 0 && __builtin_amdgcn_ballot_w64(!full_p(it - 1)) == 0;
      if (it > 0) store_p(it - 1);
      f32x16 s[2];
      scores(it, sK[buf], sKD[buf], s);
      u32x4 pk[4];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
          const float p0 = fast_exp2(__builtin_fmaf(s[mt][i], scale_log2, -L));
          const float p1 = fast_exp2(__builtin_fmaf(s[mt][i + 1], scale_log2, -L));
          held[mt][i] = p0;
          held[mt][i + 1] = p1;
          pk[2 * mt + (i >> 3)][(i & 7) >> 1] = pack2<T>(p0, p1);
        }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const bf16x8 pb = as_bf16x8(pk[c]);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const bf16x8 a = lds_frag<BN / 8>(sV[buf], 32 * dt + c32, 2 * c + hh);
          acc[dt] = mfma32<T>(a, pb, acc[dt]);
        }
      }
      if (full)
        vm_wait<8>();
      else
        lds_copy_wait();
      __syncthreads();
    };
    // walk 2 starts in the buffer walk 1's last iteration filled: buffer 1 when
    // ntiles is odd (that first tile is peeled), else 0
    int it2 = 0;
    if (ntiles & 1) {
      body2(0, std::integral_constant<int, 1>{});
      it2 = 1;
    }
    for (; it2 < ntiles; it2 += 2) {
      body2(it2, std::integral_constant<int, 0>{});
      if (it2 + 1 < ntiles) body2(it2 + 1, std::integral_constant<int, 1>{});
    }
    if (ntiles > 0) store_p(ntiles - 1);

    if (ri.q_valid) {
      T* orow = out + (((int64_t)ri.b * Sq + ri.pos) * Hq + ri.hq) * D;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          const int d = 32 * dt + 8 * gi + 4 * hh;
          u32x2 pk2;
          pk2[0] = pack2<T>(acc[dt][4 * gi], acc[dt][4 * gi + 1]);
          pk2[1] = pack2<T>(acc[dt][4 * gi + 2], acc[dt][4 * gi + 3]);
          *(u32x2*)(orow + d) = pk2;
        }
    }
  }
}

int pick_bm_pos(int n_rep) { return n_rep <= ROWS ? ROWS / n_rep : 0; }

}  // namespace

bool fwd_mfma_supported(const FwdArgs& a) {
  if ((a.dtype != BF16 && a.dtype != F16) || (a.D != 64 && a.D != 128)) return false;
  // one explicit mask kind at a time, with a tile list that fits
  if (a.doc && a.kvalid) return false;
  if ((a.doc || a.kvalid) && (a.Sk + BN - 1) / BN > DOC_MAX_TILES) return false;
  const int n_rep = a.Hq / a.Hkv;
  if (n_rep < 1 || n_rep > ROWS) return false;
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  if (!al16(a.q) || !al16(a.k) || !al16(a.v) || !al16(a.out) || !al16(a.cos) || !al16(a.sin))
    return false;
  if ((a.ksb | a.kss | a.ksh | a.vsb | a.vss | a.vsh) & 7) return false;
  return true;
}

// krot ([B*Hkv][Skp][D]) and V^T ([B*Hkv][D][Skp]), 16-bit elements, then the per-tile
// records ([B][Skp/64] int2, written only with an explicit mask), then the
// query blocks' listed-tile counts and order (packed documents; at most Sk
// blocks of one position per batch row).
size_t fwd_mfma_workspace(int B, int Sk, int Hkv, int D) {
  const size_t Skp = (size_t)((Sk + BN - 1) / BN) * BN;
  return 2 * (size_t)B * Hkv * Skp * D * sizeof(uint16_t) + (size_t)B * (Skp / BN) * sizeof(int2) +
         2 * (size_t)B * Skp * sizeof(int);
}

namespace {
template <typename T, int D>
void launch_kv_prep_t(const FwdArgs& a, void* krot, int krows, void* vn, int Skp, int2* ranges,
                      int v_mode, void* qpad) {
  dim3 grid((krot ? krows : Skp) / BN, a.B * a.Hkv);
  KF_LAUNCH("kv_prep", (kv_prep_kernel<T, D>), grid, dim3(256), 0, a.stream, (const T*)a.k,
            (const T*)a.v, a.cos, a.sin, (T*)krot, krows, (T*)vn, a.Sk, Skp, a.Hkv, a.ksb, a.kss,
            a.ksh, a.vsb, a.vss, a.vsh, a.k_rotated, a.doc, a.kvalid, ranges, v_mode, (T*)qpad,
            a.Hq);
}
}  // namespace

int launch_kv_prep(const FwdArgs& a, void* krot, int krows, void* vn, int Skp, int2* ranges,
                   int v_mode, void* qpad) {
  const bool h = a.dtype == F16;
  if (a.D == 128) {
    if (h) launch_kv_prep_t<f16, 128>(a, krot, krows, vn, Skp, ranges, v_mode, qpad);
    else launch_kv_prep_t<bf16, 128>(a, krot, krows, vn, Skp, ranges, v_mode, qpad);
  } else {
    if (h) launch_kv_prep_t<f16, 64>(a, krot, krows, vn, Skp, ranges, v_mode, qpad);
    else launch_kv_prep_t<bf16, 64>(a, krot, krows, vn, Skp, ranges, v_mode, qpad);
  }
  KF_CHECK_LAUNCH();
  return KF_OK;
}

namespace {
// flags[b] = 1 when every key of batch row b is valid (from its tile records),
// else 0: one wavefront per batch row
__global__ __launch_bounds__(64) void kpm_row_flags_kernel(const int2* __restrict__ ranges,
                                                           int rstride, int S,
                                                           int* __restrict__ flags) {
  const bool all = kpm_all_valid(ranges + (int64_t)blockIdx.x * rstride, S, threadIdx.x);
  if (threadIdx.x == 0) flags[blockIdx.x] = all ? 1 : 0;
}
}  // namespace

int launch_kpm_row_flags(const int2* ranges, int rstride, int S, int B, int* flags,
                         hipStream_t stream) {
  KF_LAUNCH("kpm_row_flags", kpm_row_flags_kernel, dim3(B), dim3(64), 0, stream, ranges, rstride,
            S, flags);
  KF_CHECK_LAUNCH();
  return KF_OK;
}

size_t rot_bytes(int B, int S, int Hq, int Hkv, int D) {
  return ((size_t)B * Hkv + (size_t)B * Hq) * (size_t)((S + 127) / 128 * 128) * D *
         sizeof(uint16_t);
}

namespace {

struct FwdWs {
  uint16_t *krot, *vn;  // 16-bit elements of the call's dtype
  int2* ranges;
  int *counts, *order;  // [B][Skp] each (packed documents)
  int krows;       // rows of krot per KV head
  uint16_t* qrot;  // a.rot's rotated Q, or null
};

// With a.rot the rotated K goes there (P rows per KV head, as the backward
// reads it) instead of the workspace's krot region, and the forward also
// writes the rotated Q after it.
FwdWs carve_fwd(const FwdArgs& a, void* workspace, int Skp) {
  FwdWs w;
  w.krot = (uint16_t*)workspace;
  w.vn = w.krot + (size_t)a.B * a.Hkv * Skp * a.D;
  w.ranges = (int2*)(w.vn + (size_t)a.B * a.Hkv * Skp * a.D);
  w.counts = (int*)(w.ranges + (size_t)a.B * (Skp / BN));
  w.order = w.counts + (size_t)a.B * Skp;
  w.krows = Skp;
  w.qrot = nullptr;
  if (a.rot != nullptr) {
    w.krows = (a.Sk + 127) / 128 * 128;
    w.krot = (uint16_t*)a.rot;
    w.qrot = w.krot + (size_t)a.B * a.Hkv * w.krows * a.D;
  }
  return w;
}

int mask_mode(const FwdArgs& a) { return a.doc ? MASK_DOC : a.kvalid ? MASK_KPM : MASK_NONE; }

template <typename T, int D, int MODE>
void launch_fwd_kernel(const FwdArgs& a, const FwdWs& w, int Skp, int n_rep, int bm_pos, int nqb,
                       unsigned nblk, const int* order, const int* kpm_flags = nullptr) {
  KF_LAUNCH("fwd_mfma", (fwd_mfma_kernel<T, D, MODE>), dim3(nblk), dim3(256), 0, a.stream,
            (const T*)a.q, a.cos, a.sin, (const T*)w.krot, (const T*)w.vn, (T*)a.out, a.lse, a.Sq,
            a.Sk, Skp, w.krows, a.Hq, a.Hkv, n_rep, bm_pos, nqb, a.scale * kLog2e, a.causal,
            a.doc ? a.doc : a.kvalid, w.ranges, (T*)w.qrot, order, kpm_flags);
}

template <typename T, int D>
void launch_fwd32(const FwdArgs& a, const FwdWs& w, int Skp, int n_rep, int bm_pos, int nqb,
                  unsigned nblk, const int* kpm_flags) {
  KF_LAUNCH("fwd_mfma", (fwd32_kernel<T, D>), dim3(nblk), dim3(256), 0, a.stream, (const T*)a.q,
            a.cos, a.sin, (const T*)w.krot, (const T*)w.vn, (T*)a.out, a.lse, a.Sq, a.Sk, Skp,
            w.krows, a.Hq, a.Hkv, n_rep, bm_pos, nqb, a.scale * kLog2e, a.causal, (T*)w.qrot,
            kpm_flags);
}

template <typename T, int D>
void launch_fwd_mode(const FwdArgs& a, const FwdWs& w, int Skp, int n_rep, int bm_pos, int nqb,
                     unsigned nblk) {
  switch (mask_mode(a)) {
    case MASK_DOC:
      launch_fwd_kernel<T, D, MASK_DOC>(a, w, Skp, n_rep, bm_pos, nqb, nblk, w.order);
      break;
    case MASK_KPM:
      // causal self-attention: batch rows without padding run the unmasked
      // kernel, the others the masked one (each launch skips the other's rows)
    {
      // (w.counts holds the per-row flags: launch_kpm_row_flags in fwd_mfma)
      const int* flags = a.causal && a.Sq == a.Sk ? w.counts : nullptr;
      if (flags) launch_fwd32<T, D>(a, w, Skp, n_rep, bm_pos, nqb, nblk, flags);
      launch_fwd_kernel<T, D, MASK_KPM>(a, w, Skp, n_rep, bm_pos, nqb, nblk, nullptr, flags);
      break;
    }
    default: launch_fwd32<T, D>(a, w, Skp, n_rep, bm_pos, nqb, nblk, nullptr);
  }
}

template <typename T, int D, int MODE>
void launch_capture_kernel(const FwdArgs& a, const FwdWs& w, float* probs, int Skp, int n_rep,
                           int bm_pos, int nqb, unsigned nblk) {
  KF_LAUNCH("capture_probs_mfma", (capture_probs_mfma_kernel<T, D, MODE>), dim3(nblk), dim3(256),
            0, a.stream, (const T*)a.q, a.cos, a.sin, (const T*)w.krot, (const T*)w.vn,
            (T*)a.out, a.lse, probs, a.Sq, a.Sk, Skp, a.Hq, a.Hkv, n_rep, bm_pos, nqb,
            a.scale * kLog2e, a.causal, a.doc ? a.doc : a.kvalid, w.ranges);
}

template <typename T, int D>
void launch_capture_mode(const FwdArgs& a, const FwdWs& w, float* probs, int Skp, int n_rep,
                         int bm_pos, int nqb, unsigned nblk) {
  switch (mask_mode(a)) {
    case MASK_DOC:
      launch_capture_kernel<T, D, MASK_DOC>(a, w, probs, Skp, n_rep, bm_pos, nqb, nblk);
      break;
    case MASK_KPM:
      launch_capture_kernel<T, D, MASK_KPM>(a, w, probs, Skp, n_rep, bm_pos, nqb, nblk);
      break;
    default: launch_capture_kernel<T, D, MASK_NONE>(a, w, probs, Skp, n_rep, bm_pos, nqb, nblk);
  }
}

}  // namespace

int fwd_mfma(const FwdArgs& a, void* workspace) {
  const int Skp = (a.Sk + BN - 1) / BN * BN;
  const FwdWs w = carve_fwd(a, workspace, Skp);
  int rc = launch_kv_prep(a, w.krot, w.krows, w.vn, Skp, w.ranges, KV_V_TRANSPOSED, w.qrot);
  if (rc) return rc;
  const int n_rep = a.Hq / a.Hkv;
  const int bm_pos = pick_bm_pos(n_rep);
  const int nqb = (a.Sq + bm_pos - 1) / bm_pos;
  const int64_t nblk = (int64_t)nqb * a.B * a.Hkv;
  KF_CHECK_ARG(nblk < (1LL << 31), "grid too large");
  if (a.doc) {
    // the query blocks by their listed key tiles, most first
    rc = launch_doc_order(a.doc, w.ranges, a.Sq, Skp / BN, bm_pos, a.B, nqb, 0, w.counts,
                          w.order, a.stream);
    if (rc) return rc;
  }
  if (a.kvalid && a.causal && a.Sq == a.Sk) {
    rc = launch_kpm_row_flags(w.ranges, Skp / BN, a.Sk, a.B, w.counts, a.stream);
    if (rc) return rc;
  }
  const bool h = a.dtype == F16;
  if (a.D == 128) {
    if (h) launch_fwd_mode<f16, 128>(a, w, Skp, n_rep, bm_pos, nqb, (unsigned)nblk);
    else launch_fwd_mode<bf16, 128>(a, w, Skp, n_rep, bm_pos, nqb, (unsigned)nblk);
  } else {
    if (h) launch_fwd_mode<f16, 64>(a, w, Skp, n_rep, bm_pos, nqb, (unsigned)nblk);
    else launch_fwd_mode<bf16, 64>(a, w, Skp, n_rep, bm_pos, nqb, (unsigned)nblk);
  }
  KF_CHECK_LAUNCH();
  return KF_OK;
}

int capture_probs_mfma(const FwdArgs& a, float* probs, void* workspace) {
  const int Skp = (a.Sk + BN - 1) / BN * BN;
  const FwdWs w = carve_fwd(a, workspace, Skp);
  int rc = launch_kv_prep(a, w.krot, Skp, w.vn, Skp, w.ranges, KV_V_TRANSPOSED);
  if (rc) return rc;
  const int n_rep = a.Hq / a.Hkv;
  const int bm_pos = pick_bm_pos(n_rep);
  const int nqb = (a.Sq + bm_pos - 1) / bm_pos;
  // one workgroup per pair of query blocks
  const int64_t nblk = (int64_t)((nqb + 1) / 2) * a.B * a.Hkv;
  KF_CHECK_ARG(nblk < (1LL << 31), "grid too large");
  const bool h = a.dtype == F16;
  if (a.D == 128) {
    if (h) launch_capture_mode<f16, 128>(a, w, probs, Skp, n_rep, bm_pos, nqb, (unsigned)nblk);
    else launch_capture_mode<bf16, 128>(a, w, probs, Skp, n_rep, bm_pos, nqb, (unsigned)nblk);
  } else {
    if (h) launch_capture_mode<f16, 64>(a, w, probs, Skp, n_rep, bm_pos, nqb, (unsigned)nblk);
    else launch_capture_mode<bf16, 64>(a, w, probs, Skp, n_rep, bm_pos, nqb, (unsigned)nblk);
  }
  KF_CHECK_LAUNCH();
  return KF_OK;
}

}  // namespace kf
